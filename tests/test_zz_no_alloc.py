"""The allocation-free entry point (w4a16_moe_fused_experts_noalloc) against
the workspace entry point (w4a16_moe_fused_experts_ex), through the C ABI.

Both run the same kernels in the same order, so the outputs must be equal
bit for bit.  Two calls in a row, the second with a smaller input: the
static scratch keeps the first call's contents, which the second must not
depend on.  No counterpart in the reference (it has no allocation-free
variant)."""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _args(x, w, tw, ti, shape, out):
    w13, w2, s13, s2 = w
    return (x.data_ptr(), x.stride(0), w13.data_ptr(), w2.data_ptr(), s13.data_ptr(),
            s2.data_ptr(), tw.data_ptr(), ti.data_ptr(), x.shape[0], shape.topk, shape.E,
            shape.N, shape.K, shape.group, out.data_ptr(), out.stride(0))


def _pair(pkg, lib, synth, shape, w, M, seed, skewed=False):
    """(no-alloc output, workspace output) for one seeded input."""
    L = pkg._lib
    dev = w[0].device
    x = synth.make_hidden(M, shape.K, dev, seed=seed)
    tw, ti = synth.make_routing(M, shape.E, shape.topk, dev, seed=seed, skewed=skewed)
    stream = torch.cuda.current_stream(dev).cuda_stream
    a = torch.full((M, shape.K), float("nan"), dtype=torch.bfloat16, device=dev)
    b = torch.full((M, shape.K), float("nan"), dtype=torch.bfloat16, device=dev)
    print(f"no-alloc M={M} E={shape.E} K={shape.K} N={shape.N} seed={seed}", flush=True)
    st = lib.w4a16_moe_fused_experts_noalloc(*_args(x, w, tw, ti, shape, a), stream, None)
    L.check(st)
    nbytes = L.workspace_size(M, shape.topk, shape.E, shape.N, shape.K, shape.group)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    st = lib.w4a16_moe_fused_experts_ex(*_args(x, w, tw, ti, shape, b), ws.data_ptr(), nbytes,
                                        stream, None)
    L.check(st)
    torch.cuda.synchronize()
    return a, b


@pytest.mark.parametrize("E,topk,K,N,Ms", [
    # full-size layer: an MFMA + GEMV split call, then a self-routed decode call
    (256, 10, 3072, 1024, (200, 16)),
    # a prefill-sized call (two-launch sort, all experts on MFMA), then one token
    (16, 4, 512, 256, (4096, 1)),
])
def test_noalloc_matches_workspace_entry(pkg, lib, synth, dev, E, topk, K, N, Ms):
    shape = synth.LayerShape(E=E, topk=topk, K=K, N=N, group=32)
    w = synth.make_weights(shape, dev, seed=7)
    for i, M in enumerate(Ms):
        a, b = _pair(pkg, lib, synth, shape, w, M, seed=100 + i, skewed=(i == 0))
        assert not torch.isnan(a.float()).any()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"M={M}"


def test_noalloc_rejects_calls_beyond_the_scratch(pkg, lib):
    """Host-side refusal before any GPU work (fake, never-read pointers)."""
    L = pkg._lib
    P = 1 << 20
    M = 4096  # workspace 336 MB > 64 MiB
    assert L.workspace_size(M, 10, 256, 1024, 3072, 32) > L.NOALLOC_SCRATCH_BYTES
    st = lib.w4a16_moe_fused_experts_noalloc(P, 3072, P, P, P, P, P, P, M, 10, 256, 1024,
                                             3072, 32, P, 3072, None, None)
    assert st == L.W4A16_ERR_SCRATCH_TOO_SMALL
    assert "static scratch" in L.strerror(st)
    # the largest fitting M of the benchmark shape (the header states it)
    assert L.workspace_size(818, 10, 256, 1024, 3072, 32) <= L.NOALLOC_SCRATCH_BYTES
    # M = 0 is a no-op that touches nothing
    assert lib.w4a16_moe_fused_experts_noalloc(P, 3072, P, P, P, P, P, P, 0, 10, 256, 1024,
                                               3072, 32, P, 3072, None, None) == L.W4A16_OK
    # scales that are not 16-byte aligned (every expert then runs on the GEMV
    # kernels, a layout of its own): the size check uses that layout and
    # still answers with the scratch's own error, before any pointer check
    for s13, s2 in ((P + 2, P), (P, P + 6)):
        st = lib.w4a16_moe_fused_experts_noalloc(P, 3072, P, P, s13, s2, P, P, M, 10, 256,
                                                 1024, 3072, 32, P, 3072, None, None)
        assert st == L.W4A16_ERR_SCRATCH_TOO_SMALL, st
    assert "device" in L.strerror(L.W4A16_ERR_WRONG_DEVICE)


def test_noalloc_graph_replay(pkg, lib, synth, dev):
    """One eager call (it resolves the scratch's address), then two calls of
    different M captured into one HIP graph and replayed three times with
    eager work between the replays; every replay's outputs equal the
    workspace entry point's bit for bit."""
    L = pkg._lib
    shape = synth.LayerShape(E=32, topk=4, K=512, N=256, group=32)
    w = synth.make_weights(shape, dev, seed=11)
    Ms = (300, 7)
    ins = []
    for i, M in enumerate(Ms):
        x = synth.make_hidden(M, shape.K, dev, seed=40 + i)
        tw, ti = synth.make_routing(M, shape.E, shape.topk, dev, seed=40 + i, skewed=(i == 0))
        ins.append((x, tw, ti))
    expect = []
    for (x, tw, ti), M in zip(ins, Ms):
        b = torch.empty((M, shape.K), dtype=torch.bfloat16, device=dev)
        nbytes = L.workspace_size(M, shape.topk, shape.E, shape.N, shape.K, shape.group)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        L.check(lib.w4a16_moe_fused_experts_ex(*_args(x, w, tw, ti, shape, b), ws.data_ptr(),
                                                nbytes, torch.cuda.current_stream().cuda_stream,
                                                None))
        expect.append(b)
    outs = [torch.empty((M, shape.K), dtype=torch.bfloat16, device=dev) for M in Ms]
    # the eager call before capture resolves the scratch address on this device
    x, tw, ti = ins[1]
    L.check(lib.w4a16_moe_fused_experts_noalloc(*_args(x, w, tw, ti, shape, outs[1]),
                                                torch.cuda.current_stream().cuda_stream, None))
    torch.cuda.synchronize()
    print("no-alloc graph: capture", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = torch.cuda.current_stream().cuda_stream
        for (x, tw, ti), o in zip(ins, outs):
            L.check(lib.w4a16_moe_fused_experts_noalloc(*_args(x, w, tw, ti, shape, o), s, None))
    for r in range(3):
        for o in outs:
            o.fill_(float("nan"))
        # eager work between replays: the scratch keeps this call's contents
        x, tw, ti = ins[0]
        junk = torch.empty_like(outs[0])
        L.check(lib.w4a16_moe_fused_experts_noalloc(
            *_args(synth.make_hidden(Ms[0], shape.K, dev, seed=90 + r), w, tw, ti, shape, junk),
            torch.cuda.current_stream().cuda_stream, None))
        torch.cuda.synchronize()
        print(f"no-alloc graph: replay {r}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        for o, e, M in zip(outs, expect, Ms):
            assert torch.equal(o.view(torch.int16), e.view(torch.int16)), f"replay {r} M={M}"
