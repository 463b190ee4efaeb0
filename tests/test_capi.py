"""The C ABI library loads, exports what the header declares, and rejects bad
arguments on the host (CPU only: no call here reaches the GPU)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

HEADER = Path(__file__).resolve().parents[1] / "include" / "w4a16_moe.h"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(w4a16_moe_\w+)\s*\(", text)))


def test_header_declares_expected_api():
    names = _declared_functions()
    assert "w4a16_moe_fused_experts" in names
    assert "w4a16_moe_align_block_size" in names
    assert len(names) >= 9


def test_library_exports_every_declared_symbol(lib, pkg):
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} not exported"
    assert set(_declared_functions()) == set(pkg._lib.EXPORTED_SYMBOLS)


def test_abi_version_and_strerror(lib, pkg):
    assert lib.w4a16_moe_abi_version() == 1
    for code in range(9):
        assert pkg._lib.strerror(code)
    assert pkg._lib.strerror(99) == "unknown status"


@pytest.mark.parametrize("M,topk,E,B", [(1, 10, 256, 16), (16, 10, 256, 16), (64, 10, 256, 16),
                                        (1024, 10, 256, 16), (4096, 10, 256, 16),
                                        (0, 10, 256, 16), (7, 3, 5, 1), (3, 2, 9, 128)])
def test_align_sizes_match_reference_formula(pkg, orc, M, topk, E, B):
    em, nb = pkg._lib.align_sizes(M, topk, E, B)
    assert (em, nb) == orc.align_sizes(M * topk, E, B)


def test_align_sizes_known_values(pkg):
    # EM per config at block 16 (E=256, topk=10)
    want = {1: 3856, 16: 4000, 64: 4480, 1024: 14080, 4096: 44800}
    for M, em in want.items():
        assert pkg._lib.align_sizes(M, 10, 256, 16) == (em, em // 16)


def test_align_sizes_rejects(pkg):
    with pytest.raises(AssertionError):
        pkg._lib.align_sizes(4, 2, 8, 0)
    with pytest.raises(ValueError):
        pkg._lib.align_sizes(-1, 2, 8, 16)
    with pytest.raises(ValueError):
        pkg._lib.align_sizes(4, 2, 2000, 16)  # E > 1024


def test_workspace_layout(pkg):
    L = pkg._lib
    M, topk, E, N, K, G = 16, 10, 256, 1024, 3072, 32
    size = L.workspace_size(M, topk, E, N, K, G)
    off = L.workspace_layout(M, topk, E, N, K, G)
    assert off[L.WS_HEADER] == 0  # dropped counter is read from the workspace base
    assert all(o % 256 == 0 for o in off)
    n_tok = M * topk
    ends = {
        L.WS_SORTED_IDS: off[L.WS_SORTED_IDS] + 4000 * 4,
        L.WS_EXPERT_IDS: off[L.WS_EXPERT_IDS] + 250 * 4,
        L.WS_OFFSETS: off[L.WS_OFFSETS] + (E + 1) * 4,
        L.WS_INTER: off[L.WS_INTER] + n_tok * N * 2,
        L.WS_PARTIAL: off[L.WS_PARTIAL] + n_tok * K * 2,  # bf16 rows above M=4
    }
    spans = sorted((off[f], end) for f, end in ends.items())
    for (a0, a1), (b0, _) in zip(spans, spans[1:]):
        assert a1 <= b0
    assert max(ends.values()) <= size


@pytest.mark.parametrize("M,elt", [(1, 4), (4, 4), (5, 2), (64, 2)])
def test_workspace_partial_dtype(pkg, M, elt):
    # The weighted w2 rows are fp32 up to M=4 and bf16 above, the reference's
    # two rounding points (kernels/w4a16_moe.py:311 and :763); the tile list
    # follows the partial rows directly.
    L = pkg._lib
    topk, E, N, K, G = 10, 256, 1024, 3072, 32
    off = L.workspace_layout(M, topk, E, N, K, G)
    span = off[L.WS_TILES] - off[L.WS_PARTIAL]
    need = M * topk * K * elt
    assert need <= span < need + 256


_FUSED_ARGTYPES = 19


def _fused(lib, **kw):
    """Call w4a16_moe_fused_experts with fake (never dereferenced) pointers."""
    P = 1 << 20  # 16-byte aligned fake address
    a = dict(hidden=P, ld_hidden=3072, w13=P, w2=P, s13=P, s2=P, tw=P, ids=P,
             M=16, topk=10, E=256, N=1024, K=3072, group=32, out=P, ld_out=3072,
             ws=P, ws_bytes=0, stream=None)
    a.update(kw)
    return lib.w4a16_moe_fused_experts(
        a["hidden"], a["ld_hidden"], a["w13"], a["w2"], a["s13"], a["s2"], a["tw"],
        a["ids"], a["M"], a["topk"], a["E"], a["N"], a["K"], a["group"], a["out"],
        a["ld_out"], a["ws"], a["ws_bytes"], a["stream"])


def test_fused_validation_codes(lib, pkg):
    L = pkg._lib
    # workspace size 0 -> too small (every other argument valid)
    assert _fused(lib) == L.W4A16_ERR_WORKSPACE_TOO_SMALL
    big = L.workspace_size(16, 10, 256, 1024, 3072, 32)
    assert _fused(lib, hidden=None, ws_bytes=big) == L.W4A16_ERR_NULL_POINTER
    assert _fused(lib, ws=None, ws_bytes=big) == L.W4A16_ERR_NULL_POINTER
    assert _fused(lib, group=16, ws_bytes=big) == L.W4A16_ERR_UNSUPPORTED_GROUP
    assert _fused(lib, group=48, ws_bytes=big) == L.W4A16_ERR_UNSUPPORTED_GROUP
    assert _fused(lib, K=3000, ld_hidden=3000, ld_out=3000, ws_bytes=big) \
        == L.W4A16_ERR_UNSUPPORTED_GROUP
    assert _fused(lib, topk=0, ws_bytes=big) == L.W4A16_ERR_INVALID_SHAPE
    assert _fused(lib, E=0, ws_bytes=big) == L.W4A16_ERR_INVALID_SHAPE
    assert _fused(lib, E=1025, ws_bytes=big) == L.W4A16_ERR_INVALID_SHAPE
    assert _fused(lib, M=-1, ws_bytes=big) == L.W4A16_ERR_INVALID_SHAPE
    assert _fused(lib, ld_hidden=100, ws_bytes=big) == L.W4A16_ERR_INVALID_SHAPE
    assert _fused(lib, hidden=(1 << 20) + 2, ws_bytes=big) == L.W4A16_ERR_MISALIGNED
    assert _fused(lib, ld_hidden=3076, ws_bytes=big) == L.W4A16_ERR_MISALIGNED
    assert _fused(lib, w13=(1 << 20) + 4, ws_bytes=big) == L.W4A16_ERR_MISALIGNED
    assert _fused(lib, ws=(1 << 20) + 16, ws_bytes=big) == L.W4A16_ERR_MISALIGNED
    # M = 0 is a valid no-op that touches nothing
    assert _fused(lib, M=0, ws_bytes=0) == L.W4A16_OK


def test_align_validation_codes(lib, pkg):
    L = pkg._lib
    P = 1 << 20
    f = lib.w4a16_moe_align_block_size
    assert f(P, 4, 2, 8, 0, P, P, P, None, None, None) == L.W4A16_ERR_INVALID_BLOCK
    assert f(None, 4, 2, 8, 16, P, P, P, None, None, None) == L.W4A16_ERR_NULL_POINTER
    assert f(P, 4, 2, 8, 16, None, P, P, None, None, None) == L.W4A16_ERR_NULL_POINTER
    assert f(P, 4, 0, 8, 16, P, P, P, None, None, None) == L.W4A16_ERR_INVALID_SHAPE


def test_null_output_pointers(lib, pkg):
    L = pkg._lib
    assert lib.w4a16_moe_workspace_size(1, 1, 1, 32, 32, 32, None) == L.W4A16_ERR_NULL_POINTER
    assert lib.w4a16_moe_align_sizes(1, 1, 1, 1, None, None) == L.W4A16_ERR_NULL_POINTER
    assert lib.w4a16_moe_dropped_pairs(None, ctypes.byref(ctypes.c_int32()), None) \
        == L.W4A16_ERR_NULL_POINTER


def test_python_shim_rejects_without_gpu_work(pkg):
    import torch

    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    w = torch.zeros(4, 64, 32, dtype=torch.uint8)
    s = torch.zeros(4, 64, 2, dtype=torch.bfloat16)
    ids = torch.zeros(2, 2, dtype=torch.int32)
    tw = torch.zeros(2, 2)
    with pytest.raises(AssertionError):  # CPU tensors are refused, like the reference
        pkg.fused_experts_w4a16(x, w, w, s, s, tw, ids, 32)
    with pytest.raises(AssertionError):
        pkg.moe_align_block_size(ids, 16, 4)
    w4 = torch.zeros(4, 1, 32, 64, dtype=torch.uint8)
    assert pkg.is_repacked(w4) and not pkg.is_repacked(w)
    a, b = pkg.repack_weights(w, s)
    assert a is w and b is s
