"""HIP moe_align_block_size vs the oracle: bit-exact over the whole buffers."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _run(pkg, ids_np, block, E, dev):
    ids = torch.from_numpy(np.ascontiguousarray(ids_np, dtype=np.int32)).to(dev)
    s, e, n, off, drop = pkg.moe_align_block_size_full(ids, block, E)
    torch.cuda.synchronize()
    return s.cpu().numpy(), e.cpu().numpy(), n.cpu().numpy(), off.cpu().numpy(), \
        int(drop.cpu()[0])


def _assert_exact(got, want, tag):
    names = ("sorted_token_ids", "expert_ids", "num_tokens_post_padded", "offsets")
    for name, g, w in zip(names, got[:4], want[:4]):
        assert g.shape == w.shape, f"{tag}: {name} shape {g.shape} vs {w.shape}"
        if not np.array_equal(g, w):
            bad = np.nonzero(g != w)[0][:8]
            raise AssertionError(f"{tag}: {name} differs at {bad.tolist()}: "
                                 f"{g[bad].tolist()} vs {w[bad].tolist()}")
    assert got[4] == want[4], f"{tag}: dropped {got[4]} vs {want[4]}"


@pytest.mark.parametrize("cfg_index", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("block", [16, 64])
def test_align_configs(pkg, orc, synth, dev, cfg_index, block):
    cfg = synth.CONFIGS[cfg_index]
    print(f"align config {cfg_index} M={cfg.M} block={block}", flush=True)
    tw, ti = synth.make_routing(cfg.M, 256, 10, "cpu", seed=0, skewed=cfg.skewed)
    got = _run(pkg, ti.numpy(), block, 256, dev)
    _assert_exact(got, orc.moe_align_block_size(ti.numpy(), block, 256), f"cfg{cfg_index}")


@pytest.mark.parametrize("block", [1, 2, 8, 32, 128])
def test_align_blocks(pkg, orc, dev, block):
    rng = np.random.default_rng(block)
    for M in (0, 1, 3, 64, 700):
        ids = rng.integers(0, 256, size=(M, 10)).astype(np.int32)
        print(f"align block={block} M={M}", flush=True)
        _assert_exact(_run(pkg, ids, block, 256, dev),
                      orc.moe_align_block_size(ids, block, 256), f"B{block} M{M}")


@pytest.mark.parametrize("E", [1, 3, 64, 300, 512, 513, 1024])
def test_align_expert_counts(pkg, orc, dev, E):
    rng = np.random.default_rng(E)
    for M, topk in ((1, 1), (5, 4), (257, 8), (3000, 2)):
        ids = rng.integers(0, E, size=(M, topk)).astype(np.int32)
        print(f"align E={E} M={M} topk={topk}", flush=True)
        _assert_exact(_run(pkg, ids, 16, E, dev), orc.moe_align_block_size(ids, 16, E),
                      f"E{E} M{M}")


def test_align_matches_c_oracle_random(pkg, orc, dev):
    rng = np.random.default_rng(7)
    for i in range(40):
        E = int(rng.integers(1, 300))
        M = int(rng.integers(0, 500))
        topk = int(rng.integers(1, 12))
        block = int(rng.choice([1, 4, 16, 64]))
        ids = rng.integers(0, E, size=(M, topk)).astype(np.int32)
        _assert_exact(_run(pkg, ids, block, E, dev),
                      orc.moe_align_block_size_c(ids, block, E), f"random {i}")


def test_align_all_to_one_expert(pkg, orc, dev):
    ids = np.full((4096, 10), 5, np.int32)
    _assert_exact(_run(pkg, ids, 16, 256, dev), orc.moe_align_block_size(ids, 16, 256),
                  "one expert")


def test_align_out_of_range_ids_are_dropped(pkg, orc, dev):
    rng = np.random.default_rng(11)
    ids = rng.integers(0, 32, size=(50, 4)).astype(np.int32)
    ids[3, 1] = -1
    ids[10, 0] = 32
    ids[20, 3] = 10**6
    got = _run(pkg, ids, 16, 32, dev)
    want = orc.moe_align_block_size(ids, 16, 32)
    assert want[4] == 3
    _assert_exact(got, want, "dropped")


def test_align_int64_ids_and_plain_api(pkg, orc, dev):
    rng = np.random.default_rng(12)
    ids = rng.integers(0, 256, size=(16, 10))
    t = torch.from_numpy(ids).to(dev)  # int64, cast like kernels/w4a16_moe.py:239-241
    s, e, n = pkg.moe_align_block_size(t, 16, 256)
    want = orc.moe_align_block_size(ids.astype(np.int32), 16, 256)
    assert np.array_equal(s.cpu().numpy(), want[0])
    assert np.array_equal(e.cpu().numpy(), want[1])
    assert np.array_equal(n.cpu().numpy(), want[2])
