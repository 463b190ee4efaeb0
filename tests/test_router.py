"""Router step: logits -> top-k experts + softmax weights.

CPU tests pin the oracle (oracle.moe_oracle.router_topk_softmax) against the
library routines the reference calls (torch.topk, torch.softmax --
bench/bench_moe.py:225-230) and against the stable torch.sort where torch.topk
leaves the order of equal logits open.  GPU tests compare the HIP kernel, called
through the C ABI, with the oracle (ids bit-exact, weights to a few fp32 ulp)
and with torch's own topk + softmax on the GPU.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

# fp32 softmax weights: exp, a sum of at most E terms and one division -- a few
# ulp of the float64 value.
W_RTOL = 2e-6


def _tie_free_logits(M, E, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((M, E), generator=g, dtype=torch.float32)
    for m in range(M):  # redraw the (rare) rows holding equal values
        while torch.unique(x[m]).numel() != E:
            x[m] = torch.randn((E,), generator=g)
    return x


def _tied_logits(M, E, seed, levels=4):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, levels, (M, E), generator=g).to(torch.float32)


def _stable_desc(x, k):
    return torch.sort(x, dim=-1, descending=True, stable=True).indices[:, :k]


# ---------------------------------------------------------------------------
# oracle pins (CPU)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("E,k", [(256, 10), (64, 1), (100, 64), (1024, 8)])
def test_oracle_matches_torch_topk_softmax_tie_free(orc, E, k):
    x = _tie_free_logits(64, E, seed=E + k)
    vals, ids = torch.topk(x, k, dim=-1)
    w, oid = orc.router_topk_softmax(x.numpy(), k)
    np.testing.assert_array_equal(oid, ids.numpy())
    np.testing.assert_allclose(w, torch.softmax(vals, dim=-1).numpy(), rtol=W_RTOL, atol=0)
    w_all, oid_all = orc.router_topk_softmax(x.numpy(), k, renormalize=False)
    np.testing.assert_array_equal(oid_all, ids.numpy())
    p = torch.softmax(x, dim=-1).gather(1, ids)
    np.testing.assert_allclose(w_all, p.numpy(), rtol=W_RTOL, atol=1e-30)


def test_oracle_ties_follow_stable_sort(orc):
    x = _tied_logits(128, 256, seed=3)
    k = 10
    _, oid = orc.router_topk_softmax(x.numpy(), k)
    np.testing.assert_array_equal(oid, _stable_desc(x, k).numpy())
    # same selected values as torch.topk, whose order among equals is its own
    tv = torch.topk(x, k, dim=-1).values.numpy()
    np.testing.assert_array_equal(np.take_along_axis(x.numpy(), oid, 1), tv)


def test_oracle_special_values_match_torch_topk(orc):
    nan, inf = float("nan"), float("inf")
    rows = [[1.0, nan, inf, -inf, 2.0, nan, -0.0, 0.0],
            [-inf, -inf, -inf, -inf, -inf, -inf, -inf, -1.0],
            [0.0, -0.0, 0.0, -0.0, -1.0, 3.0, inf, -2.0]]
    x = torch.tensor(rows, dtype=torch.float32)
    for k in (1, 3, 5, 8):
        tv = torch.topk(x, k, dim=-1).values.numpy()
        w, oid = orc.router_topk_softmax(x.numpy(), k)
        ov = np.take_along_axis(x.numpy(), oid, 1)
        np.testing.assert_array_equal(ov, tv)  # NaN == NaN here; -0.0 == +0.0
    # torch.topk does not rank +0.0 above -0.0: it returns a -0.0 ahead of +0.0
    z = torch.topk(torch.tensor([[-0.0, 0.0, -0.0, 0.0]]), 4).values[0]
    signs = [np.signbit(v) for v in z.numpy()]
    assert signs.index(True) < len(signs) - 1 - signs[::-1].index(False)


def test_oracle_softmax_closed_forms(orc):
    w, _ = orc.router_topk_softmax(np.full((3, 32), 0.25, np.float32), 8)
    np.testing.assert_array_equal(w, np.full((3, 8), 1 / 8))
    a, b = 1.5, -0.75
    w, ids = orc.router_topk_softmax(np.array([[b, a, -9.0]], np.float32), 2)
    assert list(ids[0]) == [1, 0]
    assert w[0, 0] == pytest.approx(1 / (1 + np.exp(b - a)), rel=1e-15)
    assert w[0, 1] == pytest.approx(1 / (1 + np.exp(a - b)), rel=1e-15)


def test_planted_tie_order_fails_stable_sort_pin(orc):
    # ties to the HIGHER index: the stable-sort pin must reject it
    x = _tied_logits(32, 256, seed=5)
    _, rid = orc.router_topk_softmax(x.numpy()[:, ::-1].copy(), 10)
    planted = 255 - rid
    assert not np.array_equal(planted, _stable_desc(x, 10).numpy())


def test_planted_full_softmax_fails_renormalized_pin(orc):
    x = _tie_free_logits(16, 256, seed=9)
    vals, _ = torch.topk(x, 10, dim=-1)
    w_planted, _ = orc.router_topk_softmax(x.numpy(), 10, renormalize=False)
    ref = torch.softmax(vals, dim=-1).numpy()
    assert not np.allclose(w_planted, ref, rtol=W_RTOL, atol=0)


# ---------------------------------------------------------------------------
# C ABI argument checks (host only, no GPU work)
# ---------------------------------------------------------------------------


def _router(lib, **kw):
    P = 1 << 20
    a = dict(logits=P, dtype=0, ld=256, M=16, E=256, k=10, renorm=1, w=P, ids=P, stream=None)
    a.update(kw)
    return lib.w4a16_moe_router_topk_softmax(a["logits"], a["dtype"], a["ld"], a["M"], a["E"],
                                             a["k"], a["renorm"], a["w"], a["ids"], a["stream"])


def test_router_validation_codes(lib, pkg):
    L = pkg._lib
    assert _router(lib, M=0) == L.W4A16_OK  # nothing to launch
    assert _router(lib, M=0, logits=None, w=None, ids=None) == L.W4A16_OK
    assert _router(lib, dtype=2) == L.W4A16_ERR_UNSUPPORTED_DTYPE
    assert _router(lib, k=0) == L.W4A16_ERR_INVALID_SHAPE
    assert _router(lib, k=65, E=512, ld=512) == L.W4A16_ERR_INVALID_SHAPE
    assert _router(lib, k=9, E=8, ld=8) == L.W4A16_ERR_INVALID_SHAPE
    assert _router(lib, E=0) == L.W4A16_ERR_INVALID_SHAPE
    assert _router(lib, E=1025, ld=1025) == L.W4A16_ERR_INVALID_SHAPE
    assert _router(lib, renorm=2) == L.W4A16_ERR_INVALID_SHAPE
    assert _router(lib, ld=255) == L.W4A16_ERR_INVALID_SHAPE
    assert _router(lib, M=-1) == L.W4A16_ERR_INVALID_SHAPE
    assert _router(lib, logits=None) == L.W4A16_ERR_NULL_POINTER
    assert _router(lib, ids=None) == L.W4A16_ERR_NULL_POINTER
    assert _router(lib, logits=(1 << 20) + 2) == L.W4A16_ERR_MISALIGNED
    assert _router(lib, w=(1 << 20) + 2) == L.W4A16_ERR_MISALIGNED
    assert L.strerror(L.W4A16_ERR_UNSUPPORTED_DTYPE) == "unsupported logits dtype"


def test_router_wrapper_rejects_cpu_and_bad_dtype(pkg):
    with pytest.raises(pkg._lib.W4A16Error):
        pkg.router_topk_softmax(torch.zeros(4, 8), 2)  # CPU tensor
    with pytest.raises(pkg._lib.W4A16Error):
        pkg.router_topk_softmax(torch.zeros(4, 8, dtype=torch.float16), 2)


# ---------------------------------------------------------------------------
# GPU parity (through the C ABI)
# ---------------------------------------------------------------------------


def _check_against_oracle(orc, x_gpu, w, ids, k, renormalize):
    x32 = x_gpu.float().cpu().numpy()
    ow, oid = orc.router_topk_softmax(x32, k, renormalize=renormalize)
    np.testing.assert_array_equal(ids.cpu().numpy(), oid)
    np.testing.assert_allclose(w.cpu().numpy(), ow, rtol=W_RTOL, atol=1e-30)


@pytest.mark.gpu
@pytest.mark.parametrize("E,k", [(256, 10), (256, 1), (8, 8), (100, 64), (512, 16),
                                 (1024, 10), (64, 64), (200, 33)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("renormalize", [True, False])
def test_router_matches_oracle(pkg, orc, dev, E, k, dtype, renormalize):
    M = 77
    print(f"router E={E} k={k} {dtype} renorm={renormalize}", flush=True)
    # bf16 rounding creates ties, which the oracle orders like the kernel
    x = _tie_free_logits(M, E, seed=E * 7 + k).to(dtype)
    xg = x.to(dev)
    w, ids = pkg.router_topk_softmax(xg, k, renormalize)
    torch.cuda.synchronize()
    assert w.dtype == torch.float32 and ids.dtype == torch.int32
    _check_against_oracle(orc, xg, w, ids, k, renormalize)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 16, 64, 1024, 4096])
def test_router_full_size_matches_torch_on_gpu(pkg, dev, M):
    """The reference's own routing code (torch.topk + softmax) on this GPU."""
    print(f"router full size M={M}", flush=True)
    x = _tie_free_logits(M, 256, seed=M).to(dev)
    w, ids = pkg.router_topk_softmax(x, 10)
    vals, tids = torch.topk(x, 10, dim=-1)
    tw = torch.softmax(vals, dim=-1)
    torch.cuda.synchronize()
    assert torch.equal(ids, tids.to(torch.int32))
    torch.testing.assert_close(w, tw, rtol=W_RTOL, atol=0)


@pytest.mark.gpu
def test_router_ties_and_special_values(pkg, orc, dev):
    x = _tied_logits(300, 256, seed=11)
    nan, inf = float("nan"), float("inf")
    x[0, 5] = nan
    x[0, 9] = nan
    x[1, :] = -inf
    x[1, 200] = inf
    x[2, :] = 0.0
    x[2, ::3] = -0.0
    x[3, 17] = -inf
    xg = x.to(dev)
    for k in (1, 10, 64):
        print(f"router ties k={k}", flush=True)
        w, ids = pkg.router_topk_softmax(xg, k)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ids[4:].cpu().numpy(), _stable_desc(x[4:], k).numpy())
        _, oid = orc.router_topk_softmax(x.numpy(), k)
        np.testing.assert_array_equal(ids.cpu().numpy(), oid)
        ow, _ = orc.router_topk_softmax(x[3:].numpy(), k)
        np.testing.assert_allclose(w[3:].cpu().numpy(), ow, rtol=W_RTOL, atol=1e-30)
        assert torch.isnan(w[0]).all()  # a selected NaN makes the softmax NaN, as in torch


@pytest.mark.gpu
def test_router_strided_and_out(pkg, orc, dev):
    big = _tie_free_logits(40, 300, seed=2).to(dev)
    x = big[:, 20:276]  # ld 300, E 256
    w = torch.full((40, 10), -1.0, device=dev)
    ids = torch.full((40, 10), -1, dtype=torch.int32, device=dev)
    rw, rids = pkg.router_topk_softmax(x, 10, out=(w, ids))
    torch.cuda.synchronize()
    assert rw.data_ptr() == w.data_ptr() and rids.data_ptr() == ids.data_ptr()
    _check_against_oracle(orc, x, w, ids, 10, True)
    e = torch.empty((0, 256), device=dev)
    w0, i0 = pkg.router_topk_softmax(e, 10)
    assert w0.shape == (0, 10) and i0.shape == (0, 10)


@pytest.mark.gpu
def test_router_graph_replay(pkg, orc, dev):
    sets = [_tie_free_logits(16, 256, seed=100 + i) for i in range(3)]
    static = sets[0].to(dev)
    pkg.router_topk_softmax(static, 10)  # warm the library before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        w, ids = pkg.router_topk_softmax(static, 10)
    for rep in range(2):
        for s in sets:
            static.copy_(s.to(dev))
            g.replay()
            torch.cuda.synchronize()
            _check_against_oracle(orc, static, w, ids, 10, True)


@pytest.mark.gpu
def test_router_feeds_fused_experts(pkg, synth, dev):
    """Router output drives the MoE call exactly like torch.topk routing."""
    shape = synth.LayerShape(E=16, topk=4, K=256, N=128, group=32)
    w13, w2, s13, s2 = synth.make_weights(shape, dev, seed=4)
    x = synth.make_hidden(12, shape.K, dev, seed=4)
    logits = _tie_free_logits(12, shape.E, seed=4).to(dev)
    w, ids = pkg.router_topk_softmax(logits, shape.topk)
    vals, tids = torch.topk(logits, shape.topk, dim=-1)
    tw = torch.softmax(vals, dim=-1)
    out = pkg.fused_experts_w4a16(x, w13, w2, s13, s2, w, ids, shape.group)
    ref = pkg.fused_experts_w4a16(x, w13, w2, s13, s2, tw, tids.to(torch.int32), shape.group)
    torch.cuda.synchronize()
    assert torch.equal(ids, tids.to(torch.int32))
    torch.testing.assert_close(out.float(), ref.float(), rtol=0, atol=2e-2 * ref.abs().max().item())


def test_router_symbol_is_declared(lib):
    assert isinstance(lib.w4a16_moe_router_topk_softmax, ctypes._CFuncPtr)
