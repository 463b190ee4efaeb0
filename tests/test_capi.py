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
    for code in range(12):
        assert pkg._lib.strerror(code) != "unknown status", code
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


def test_mfma_activation_offset_limit_is_a_shape_error(lib, pkg):
    """Calls that run the MFMA kernels address activation rows with 32-bit
    byte offsets; a hidden buffer past that bound is refused on the host
    (before any GPU work) instead of failing at the kernel launch."""
    L = pkg._lib
    M, ld = 2048, 1 << 20  # M * ld * 2 bytes = 4 GiB
    big = L.workspace_size(M, 10, 256, 1024, 3072, 32)
    assert _fused(lib, M=M, ld_hidden=ld, ws_bytes=big) == L.W4A16_ERR_INVALID_SHAPE
    # the GEMV-only path (M at most the GEMV-only bound) has 64-bit row
    # offsets: the same stride passes the shape checks (and stops at the
    # workspace check, still before any GPU work)
    assert _fused(lib, M=16, ld_hidden=ld, ws_bytes=0) == L.W4A16_ERR_WORKSPACE_TOO_SMALL
    # the w2 partial rows (M * topk * K * 2 bytes) are an output of the MFMA
    # kernels, addressed the same way: 69,904 tokens fit, 69,905 do not
    for M, want in ((69904, L.W4A16_ERR_WORKSPACE_TOO_SMALL),
                    (69905, L.W4A16_ERR_INVALID_SHAPE)):
        assert _fused(lib, M=M, ld_hidden=3072, ws_bytes=0) == want


@pytest.mark.parametrize("M,want", [(0, [0, 0, 0, 0]), (1, [0, 1, 1, 0]), (4, [0, 1, 1, 0]),
                                    (16, [0, 1, 1, 1]), (64, [1, 1, 1, 1]),
                                    (1024, [2, 1, 1, 1]), (4096, [2, 1, 1, 1])])
def test_stage_launches(pkg, M, want):
    """Kernels per stage: no sort for self-routed calls (M <= 24), w2 fused
    with the top-k sum for M <= 4, one mixed GEMV + MFMA launch per GEMM for
    the split dispatch, MFMA only once experts average 32+ pairs, the
    two-launch sort from 8192 pairs."""
    assert pkg._lib.stage_launches(M, 10, 256, 1024, 3072, 32, None) == want


def test_stage_launches_follow_tuning(pkg):
    L = pkg._lib
    t = pkg.Tuning(gemv_only_max_m=0, gemv_max_tokens=0).to_struct()
    assert L.stage_launches(16, 10, 256, 1024, 3072, 32, t) == [1, 1, 1, 1]
    t = pkg.Tuning(w2_fused_max_m=8).to_struct()
    assert L.stage_launches(8, 10, 256, 1024, 3072, 32, t) == [0, 1, 1, 0]


def test_workspace_layout_ex_follows_tuning(pkg):
    L = pkg._lib
    args = (1024, 10, 256, 1024, 3072, 32)
    assert L.workspace_layout_ex(*args, None) == L.workspace_layout(*args)
    t128 = pkg.Tuning(gemv_only_max_m=24, gemv_max_tokens=4, mfma_tile_m=128).to_struct()
    t192 = pkg.Tuning(gemv_only_max_m=24, gemv_max_tokens=4, mfma_tile_m=192).to_struct()
    a, b = L.workspace_layout_ex(*args, t128), L.workspace_layout_ex(*args, t192)
    # a taller MFMA tile means fewer tiles: the GEMV block list moves down
    assert a[L.WS_TILES] == b[L.WS_TILES]
    assert a[L.WS_GEMV_BLOCKS] > b[L.WS_GEMV_BLOCKS]
    for off in (a, b):
        assert all(o % 256 == 0 for o in off)
    for t, off in ((t128, a), (t192, b)):
        assert L.workspace_size_ex(*args, t) > max(off)


def test_workspace_pool_holds_one_buffer_of_the_largest_need(pkg):
    """Fifty distinct M values on one stream keep one buffer, of the largest
    call's size; another stream gets its own; each graph capture gets a
    buffer of its own (never the stream's eager one, never another
    capture's), and a capture buffer outgrown within its capture is kept
    (retired) until the captures are released."""
    import random

    import torch

    L = pkg._lib
    pool = pkg.w4a16_moe.WorkspacePool(
        alloc=lambda n, d: torch.empty(n, dtype=torch.uint8, device="cpu"))
    Ms = random.Random(0).sample(range(1, 5000), 50)
    size = {M: L.workspace_size(M, 10, 256, 1024, 3072, 32) for M in Ms}
    for M in Ms:
        buf = pool.get("cuda:0", 7, size[M])
        assert buf.numel() >= size[M]
    assert pool.cached_bytes() == max(size.values())
    assert pool.retired_bytes() == 0
    pool.get("cuda:0", 9, size[Ms[0]])
    assert pool.cached_bytes() == max(size.values()) + size[Ms[0]]
    eager = pool.get("cuda:0", 11, 4000)
    # two captures on the same stream: distinct buffers, not the eager one
    cap_a = pool.get("cuda:0", 11, 1000, capture_id=5)
    cap_b = pool.get("cuda:0", 11, 1000, capture_id=6)
    ptrs = {eager.data_ptr(), cap_a.data_ptr(), cap_b.data_ptr()}
    assert len(ptrs) == 3
    # calls of one capture share its buffer; the eager stream keeps its own
    assert pool.get("cuda:0", 11, 800, capture_id=5).data_ptr() == cap_a.data_ptr()
    assert pool.get("cuda:0", 11, 100).data_ptr() == eager.data_ptr()
    # a capture buffer outgrown within its capture stays alive
    grown = pool.get("cuda:0", 11, 5000, capture_id=5)
    assert grown.data_ptr() not in ptrs
    assert pool.retired_bytes() == cap_a.numel() == 1000
    assert pool.capture_bytes() == 1000 + 5000 + 1000
    live = pool.cached_bytes()
    pool.release_captures()
    assert pool.retired_bytes() == 0 and pool.capture_bytes() == 0
    assert pool.cached_bytes() == live - 6000
    assert pool.get("cuda:0", 11, 100).data_ptr() == eager.data_ptr()
    pool.clear()
    assert pool.cached_bytes() == 0 and pool.retired_bytes() == 0


@pytest.mark.gpu
def test_capture_id_tells_captures_apart(pkg):
    """0 outside capture; during capture a nonzero id, different for two
    captures of the same stream."""
    import torch

    L = pkg._lib
    s = torch.cuda.Stream()
    assert L.capture_id(s.cuda_stream) == 0
    ids = []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            ids.append(L.capture_id(s.cuda_stream))
            torch.zeros(4, device="cuda").add_(1)
        del g
    assert ids[0] != 0 and ids[1] != 0 and ids[0] != ids[1]
    assert L.capture_id(s.cuda_stream) == 0
