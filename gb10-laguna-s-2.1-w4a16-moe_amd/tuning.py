"""Per-M dispatch tables: the tile selector of the W4A16 MoE call.

The reference's stock path reads tuned kernel configurations from a JSON file
per (E, N, device, dtype) whose top-level keys are token counts M
(configs/E=256,N=1024,device_name=NVIDIA_GB10,dtype=int4_w4a16.json, written
by bench/tune_configs.py); a call uses the entry whose M is nearest to its
own.  Here the same file shape holds, per M, the dispatch choices of struct
w4a16_moe_tuning (include/w4a16_moe.h): which experts run on the GEMV and
which on the MFMA kernels, and how many token rows a GEMV pass serves.  The
kernels' tile shapes themselves are fixed at build time.

Files live in ``configs/`` next to this module (or in $W4A16_MOE_CONFIG_DIR)
and are written by ``tune.py``.  Without a file for the shape and device the
library's built-in choices apply.  W4A16_MOE_TUNING=default ignores the files.
"""

from __future__ import annotations

import functools
import json
import os
from dataclasses import asdict, dataclass
from pathlib import Path

from . import _lib

CONFIG_DIR = Path(__file__).resolve().parent / "configs"
# gemv_only_max_m that means "every M in this bucket runs GEMV-only"
ALWAYS = 1 << 30


@dataclass(frozen=True)
class Tuning:
    gemv_only_max_m: int = 24
    gemv_max_tokens: int = 4
    gemv_tokens_per_pass: int = 0
    mfma_tile_m: int = 0
    gemv_units_per_wg: int = 0
    gemv_lanes_per_row: int = 0
    w2_fused_max_m: int = 0
    mfma_row_tiles: int = 0

    def to_struct(self) -> _lib.TuningStruct:
        t = _lib.TuningStruct()
        t.gemv_only_max_m = int(self.gemv_only_max_m)
        t.gemv_max_tokens = int(self.gemv_max_tokens)
        t.gemv_tokens_per_pass = int(self.gemv_tokens_per_pass)
        t.mfma_tile_m = int(self.mfma_tile_m)
        t.gemv_units_per_wg = int(self.gemv_units_per_wg)
        t.gemv_lanes_per_row = int(self.gemv_lanes_per_row)
        t.w2_fused_max_m = int(self.w2_fused_max_m)
        t.mfma_row_tiles = int(self.mfma_row_tiles)
        return t

    @classmethod
    def from_struct(cls, t: _lib.TuningStruct) -> "Tuning":
        return cls(**{k: int(getattr(t, k)) for k in cls.__dataclass_fields__})

    @classmethod
    def from_dict(cls, d: dict) -> "Tuning":
        unknown = set(d) - set(cls.__dataclass_fields__)
        if unknown:
            raise ValueError(f"unknown tuning fields {sorted(unknown)}")
        return cls(**{k: int(v) for k, v in d.items()})

    def to_dict(self) -> dict:
        return asdict(self)


def device_name(device=None) -> str:
    """The device part of a table's file name (see _device_name)."""
    import torch

    idx = torch.cuda.current_device() if device is None else torch.device(device).index
    return _device_name(0 if idx is None else idx)


@functools.lru_cache(maxsize=16)
def _device_name(index: int) -> str:
    """gfx architecture and compute-unit count, e.g. "gfx950_cu256".  (The
    marketing name depends on the host's libdrm id table and can read as a
    generic "AMD Radeon Graphics".)"""
    import torch

    props = torch.cuda.get_device_properties(index)
    arch = (getattr(props, "gcnArchName", "") or "").split(":")[0]
    if not arch:
        arch = props.name.replace(" ", "_")
    return f"{arch}_cu{props.multi_processor_count}"


def config_name(E: int, N: int, K: int, group: int, dev_name: str) -> str:
    return f"E={E},N={N},K={K},group={group},device_name={dev_name},dtype=int4_w4a16.json"


def _config_dir() -> Path:
    d = os.environ.get("W4A16_MOE_CONFIG_DIR")
    return Path(d) if d else CONFIG_DIR


def parse_table(text: str) -> dict[int, Tuning]:
    raw = json.loads(text)
    if not isinstance(raw, dict) or not raw:
        raise ValueError("a tuning table is a non-empty JSON object keyed by M")
    return {int(m): Tuning.from_dict(v) for m, v in raw.items()}


def dump_table(table: dict[int, Tuning]) -> str:
    return json.dumps({str(m): table[m].to_dict() for m in sorted(table)}, indent=2) + "\n"


@functools.lru_cache(maxsize=64)
def _load(path: str) -> dict[int, Tuning] | None:
    p = Path(path)
    if not p.exists():
        return None
    return parse_table(p.read_text())


def load_table(E: int, N: int, K: int, group: int, dev_name: str,
               directory: Path | None = None) -> dict[int, Tuning] | None:
    d = directory if directory is not None else _config_dir()
    return _load(str(d / config_name(E, N, K, group, dev_name)))


def nearest(table: dict[int, Tuning], M: int) -> Tuning:
    """The entry for the key nearest to M (ties to the smaller key)."""
    key = min(table, key=lambda m: (abs(m - M), m))
    return table[key]


def select(M: int, E: int, N: int, K: int, group: int, device=None) -> Tuning | None:
    """Tuning for one call, or None for the library's built-in choices."""
    if os.environ.get("W4A16_MOE_TUNING", "") == "default":
        return None
    table = load_table(E, N, K, group, device_name(device))
    return None if table is None else nearest(table, M)
