"""ctypes binding of ``libw4a16moe.so`` (the C ABI in include/w4a16_moe.h).

torch must be imported before the library is loaded: torch ships its own HIP
runtime under the soname ``libamdhip64.so.7`` and the dynamic linker then binds
this library to that same runtime, so device pointers and streams from torch
are valid here.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (loads torch's HIP runtime first, see above)

LIB_PATH = Path(__file__).resolve().parent / "libw4a16moe.so"

W4A16_OK = 0
W4A16_ERR_NULL_POINTER = 1
W4A16_ERR_INVALID_SHAPE = 2
W4A16_ERR_UNSUPPORTED_GROUP = 3
W4A16_ERR_WORKSPACE_TOO_SMALL = 4
W4A16_ERR_MISALIGNED = 5
W4A16_ERR_INVALID_BLOCK = 6
W4A16_ERR_HIP = 7
W4A16_ERR_UNSUPPORTED_DTYPE = 8
W4A16_ERR_INVALID_TUNING = 9
W4A16_ERR_SCRATCH_TOO_SMALL = 10
W4A16_ERR_WRONG_DEVICE = 11
NOALLOC_SCRATCH_BYTES = 64 << 20

LOGITS_F32 = 0
LOGITS_BF16 = 1
ROUTER_MAX_TOPK = 64

WS_SORTED_IDS = 0
WS_EXPERT_IDS = 1
WS_HEADER = 2
WS_OFFSETS = 3
WS_INTER = 4
WS_PARTIAL = 5
WS_TILES = 6
WS_GEMV_BLOCKS = 7
WS_NFIELDS = 8

FUSED_BLOCK_M = 16
GEMV_MAX_TOKENS = 4
GEMV_ONLY_MAX_M = 24

EXPORTED_SYMBOLS = (
    "w4a16_moe_align_sizes",
    "w4a16_moe_align_block_size",
    "w4a16_moe_workspace_size",
    "w4a16_moe_workspace_layout",
    "w4a16_moe_fused_experts",
    "w4a16_moe_fused_experts_profiled",
    "w4a16_moe_run_stage",
    "w4a16_moe_dropped_pairs",
    "w4a16_moe_capture_id",
    "w4a16_moe_router_topk_softmax",
    "w4a16_moe_default_tuning",
    "w4a16_moe_workspace_size_ex",
    "w4a16_moe_fused_experts_ex",
    "w4a16_moe_run_stage_ex",
    "w4a16_moe_workspace_layout_ex",
    "w4a16_moe_stage_launches",
    "w4a16_moe_fused_experts_noalloc",
    "w4a16_moe_strerror",
    "w4a16_moe_abi_version",
)

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class LibraryNotBuilt(RuntimeError):
    pass


class TuningStruct(ctypes.Structure):
    """struct w4a16_moe_tuning (include/w4a16_moe.h)."""

    _fields_ = [("gemv_only_max_m", ctypes.c_int32), ("gemv_max_tokens", ctypes.c_int32),
                ("gemv_tokens_per_pass", ctypes.c_int32), ("mfma_tile_m", ctypes.c_int32),
                ("gemv_units_per_wg", ctypes.c_int32), ("gemv_lanes_per_row", ctypes.c_int32),
                ("w2_fused_max_m", ctypes.c_int32), ("mfma_row_tiles", ctypes.c_int32)]


def _declare(lib: ctypes.CDLL) -> None:
    lib.w4a16_moe_abi_version.restype = ctypes.c_int
    lib.w4a16_moe_abi_version.argtypes = []
    lib.w4a16_moe_strerror.restype = ctypes.c_char_p
    lib.w4a16_moe_strerror.argtypes = [ctypes.c_int]
    lib.w4a16_moe_align_sizes.restype = ctypes.c_int
    lib.w4a16_moe_align_sizes.argtypes = [
        _i64, _i64, _i64, _i64, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]
    lib.w4a16_moe_align_block_size.restype = ctypes.c_int
    lib.w4a16_moe_align_block_size.argtypes = [
        _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp]
    lib.w4a16_moe_workspace_size.restype = ctypes.c_int
    lib.w4a16_moe_workspace_size.argtypes = [
        _i64, _i64, _i64, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_size_t)]
    lib.w4a16_moe_workspace_layout.restype = ctypes.c_int
    lib.w4a16_moe_workspace_layout.argtypes = [
        _i64, _i64, _i64, _i64, _i64, _i64, ctypes.POINTER(ctypes.c_size_t)]
    fused = [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp,
             _i64, _i64, _i64, _i64, _i64, _i64, _vp, _i64, _vp, ctypes.c_size_t, _vp]
    lib.w4a16_moe_fused_experts.restype = ctypes.c_int
    lib.w4a16_moe_fused_experts.argtypes = fused
    lib.w4a16_moe_fused_experts_profiled.restype = ctypes.c_int
    lib.w4a16_moe_fused_experts_profiled.argtypes = fused + [ctypes.POINTER(ctypes.c_float)]
    lib.w4a16_moe_run_stage.restype = ctypes.c_int
    lib.w4a16_moe_run_stage.argtypes = [ctypes.c_int] + fused
    lib.w4a16_moe_dropped_pairs.restype = ctypes.c_int
    lib.w4a16_moe_dropped_pairs.argtypes = [_vp, ctypes.POINTER(ctypes.c_int32), _vp]
    lib.w4a16_moe_capture_id.restype = ctypes.c_int
    lib.w4a16_moe_capture_id.argtypes = [_vp, ctypes.POINTER(ctypes.c_uint64)]
    tp = ctypes.POINTER(TuningStruct)
    lib.w4a16_moe_default_tuning.restype = ctypes.c_int
    lib.w4a16_moe_default_tuning.argtypes = [_i64] * 6 + [tp]
    lib.w4a16_moe_workspace_size_ex.restype = ctypes.c_int
    lib.w4a16_moe_workspace_size_ex.argtypes = [_i64] * 6 + [tp, ctypes.POINTER(ctypes.c_size_t)]
    lib.w4a16_moe_fused_experts_ex.restype = ctypes.c_int
    lib.w4a16_moe_fused_experts_ex.argtypes = fused + [tp]
    lib.w4a16_moe_run_stage_ex.restype = ctypes.c_int
    lib.w4a16_moe_run_stage_ex.argtypes = [ctypes.c_int] + fused + [tp]
    lib.w4a16_moe_workspace_layout_ex.restype = ctypes.c_int
    lib.w4a16_moe_workspace_layout_ex.argtypes = [_i64] * 6 + [tp, ctypes.POINTER(ctypes.c_size_t)]
    lib.w4a16_moe_stage_launches.restype = ctypes.c_int
    lib.w4a16_moe_stage_launches.argtypes = [_i64] * 6 + [tp, ctypes.POINTER(ctypes.c_int32)]
    lib.w4a16_moe_fused_experts_noalloc.restype = ctypes.c_int
    lib.w4a16_moe_fused_experts_noalloc.argtypes = fused[:16] + [_vp, tp]
    lib.w4a16_moe_router_topk_softmax.restype = ctypes.c_int
    lib.w4a16_moe_router_topk_softmax.argtypes = [
        _vp, ctypes.c_int, _i64, _i64, _i64, _i64, ctypes.c_int, _vp, _vp, _vp]


def lib() -> ctypes.CDLL:
    """Load the HIP library; raises LibraryNotBuilt if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise LibraryNotBuilt(
                    f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                    "(hipcc --offload-arch=gfx950)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            _declare(handle)
            if handle.w4a16_moe_abi_version() != 1:
                raise RuntimeError("libw4a16moe.so ABI version mismatch")
            _lib = handle
    return _lib


def strerror(status: int) -> str:
    return lib().w4a16_moe_strerror(status).decode()


def align_sizes(M: int, topk: int, num_experts: int, block_size: int) -> tuple[int, int]:
    em, nb = _i64(), _i64()
    st = lib().w4a16_moe_align_sizes(M, topk, num_experts, block_size,
                                     ctypes.byref(em), ctypes.byref(nb))
    check(st)
    return em.value, nb.value


def workspace_size(M: int, topk: int, E: int, N: int, K: int, group: int) -> int:
    out = ctypes.c_size_t()
    check(lib().w4a16_moe_workspace_size(M, topk, E, N, K, group, ctypes.byref(out)))
    return out.value


def workspace_size_ex(M: int, topk: int, E: int, N: int, K: int, group: int,
                      tuning: "TuningStruct | None") -> int:
    out = ctypes.c_size_t()
    ptr = ctypes.byref(tuning) if tuning is not None else None
    check(lib().w4a16_moe_workspace_size_ex(M, topk, E, N, K, group, ptr, ctypes.byref(out)))
    return out.value


def default_tuning(M: int, topk: int, E: int, N: int, K: int, group: int) -> TuningStruct:
    t = TuningStruct()
    check(lib().w4a16_moe_default_tuning(M, topk, E, N, K, group, ctypes.byref(t)))
    return t


def workspace_layout(M: int, topk: int, E: int, N: int, K: int, group: int) -> list[int]:
    arr = (ctypes.c_size_t * WS_NFIELDS)()
    check(lib().w4a16_moe_workspace_layout(M, topk, E, N, K, group, arr))
    return list(arr)


def workspace_layout_ex(M: int, topk: int, E: int, N: int, K: int, group: int,
                        tuning: "TuningStruct | None") -> list[int]:
    arr = (ctypes.c_size_t * WS_NFIELDS)()
    ptr = ctypes.byref(tuning) if tuning is not None else None
    check(lib().w4a16_moe_workspace_layout_ex(M, topk, E, N, K, group, ptr, arr))
    return list(arr)


def stage_launches(M: int, topk: int, E: int, N: int, K: int, group: int,
                   tuning: "TuningStruct | None") -> list[int]:
    """Kernel launches of each stage (sort, w13, w2, combine) of such a call."""
    arr = (ctypes.c_int32 * 4)()
    ptr = ctypes.byref(tuning) if tuning is not None else None
    check(lib().w4a16_moe_stage_launches(M, topk, E, N, K, group, ptr, arr))
    return list(arr)


class W4A16Error(AssertionError, ValueError):
    """Argument rejected by the library.

    An AssertionError, as the reference's own checks are asserts, and a
    ValueError for callers that expect one.
    """


class W4A16RuntimeError(RuntimeError):
    """The HIP runtime reported a failure."""


def capture_id(stream: int) -> int:
    """0 when `stream` is not being captured into a HIP graph, else the id of
    the capture in progress."""
    out = ctypes.c_uint64()
    check(lib().w4a16_moe_capture_id(stream, ctypes.byref(out)))
    return int(out.value)


def check(status: int) -> None:
    if status == W4A16_OK:
        return
    msg = f"w4a16_moe: {strerror(status)} (status {status})"
    if status == W4A16_ERR_HIP:
        raise W4A16RuntimeError(msg)
    raise W4A16Error(msg)
