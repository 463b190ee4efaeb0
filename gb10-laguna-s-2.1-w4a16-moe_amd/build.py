"""Build the gfx950 HIP library ``libw4a16moe.so`` in-tree with hipcc.

Every HIP source under ``csrc/`` goes into one shared library exposing the C
ABI declared in ``include/w4a16_moe.h``.  The library is written next to this
file so it travels with the source tree; the Python shim loads it from here.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libw4a16moe.so"
LIB_PATH = PKG_DIR / LIB_NAME
OFFLOAD_ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # Packed fp32 VALU forms stay off: hand-written and compiler-made
    # v_pk_{add,mul,fma}_f32 are excluded from every kernel here.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP library)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    if verbose and proc.stderr.strip():
        noise = "is not a recognized feature for this target"
        lines = [ln for ln in proc.stderr.splitlines() if noise not in ln]
        if lines:
            print("\n".join(lines), file=sys.stderr, flush=True)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source to an object (in parallel), link them into
    LIB_PATH (atomic replace)."""
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    cc = hipcc()
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with tempfile.TemporaryDirectory(dir=PKG_DIR) as tmp:
        objs = [Path(tmp) / (src.stem + ".o") for src in srcs]
        with ThreadPoolExecutor(max_workers=jobs) as ex:
            for f in [ex.submit(_run, [cc, *HIPCC_FLAGS, "-c", "-o", str(o), str(src)], verbose)
                      for src, o in zip(srcs, objs)]:
                f.result()
        tmp_lib = Path(tmp) / LIB_NAME
        _run([cc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(tmp_lib),
              *map(str, objs)], verbose)
        os.replace(tmp_lib, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
