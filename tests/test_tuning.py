"""Per-M dispatch tuning: the C struct's validation, the JSON table and its
nearest-M selection (CPU), and on the GPU that every tuning the autotuner can
choose computes the same layer (against the oracle) and really changes the
dispatch (the MFMA tile count the align kernel writes)."""

from __future__ import annotations

import ctypes
import importlib
import json

import numpy as np
import pytest
import torch


def _fused_ex(lib, tuning, **kw):
    P = 1 << 20
    a = dict(hidden=P, ld_hidden=3072, w13=P, w2=P, s13=P, s2=P, tw=P, ids=P,
             M=16, topk=10, E=256, N=1024, K=3072, group=32, out=P, ld_out=3072,
             ws=P, ws_bytes=1 << 40, stream=None)
    a.update(kw)
    ptr = None if tuning is None else ctypes.byref(tuning)
    return lib.w4a16_moe_fused_experts_ex(
        a["hidden"], a["ld_hidden"], a["w13"], a["w2"], a["s13"], a["s2"], a["tw"],
        a["ids"], a["M"], a["topk"], a["E"], a["N"], a["K"], a["group"], a["out"],
        a["ld_out"], a["ws"], a["ws_bytes"], a["stream"], ptr)


@pytest.mark.parametrize("field,value", [
    ("gemv_only_max_m", -1), ("gemv_max_tokens", -1), ("gemv_max_tokens", 16),
    ("gemv_tokens_per_pass", 3), ("gemv_tokens_per_pass", 8), ("mfma_tile_m", 96),
    ("mfma_tile_m", 256), ("gemv_units_per_wg", 3), ("gemv_units_per_wg", 8),
    ("gemv_lanes_per_row", 16), ("gemv_lanes_per_row", 4), ("w2_fused_max_m", -1),
    ("mfma_row_tiles", -1), ("mfma_row_tiles", 17)])
def test_invalid_tuning_rejected_on_host(lib, pkg, field, value):
    t = pkg.Tuning().to_struct()
    setattr(t, field, value)
    assert _fused_ex(lib, t) == pkg._lib.W4A16_ERR_INVALID_TUNING
    assert pkg._lib.strerror(pkg._lib.W4A16_ERR_INVALID_TUNING) == "invalid tuning value"


def test_default_tuning_and_workspace_sizes(pkg):
    L = pkg._lib
    d = L.default_tuning(16, 10, 256, 1024, 3072, 32)
    assert (d.gemv_only_max_m, d.gemv_max_tokens, d.gemv_tokens_per_pass, d.mfma_tile_m,
            d.gemv_units_per_wg, d.gemv_lanes_per_row, d.w2_fused_max_m) == \
        (24, 4, 0, 64, 0, 0, 4)
    assert d.mfma_row_tiles == 0
    # built-in MFMA tile height: 64 slots below 24 pairs per expert, 128 below
    # 64, then 192
    assert L.default_tuning(614, 10, 256, 1024, 3072, 32).mfma_tile_m == 64
    assert L.default_tuning(615, 10, 256, 1024, 3072, 32).mfma_tile_m == 128
    assert L.default_tuning(1024, 10, 256, 1024, 3072, 32).mfma_tile_m == 128
    assert L.default_tuning(1638, 10, 256, 1024, 3072, 32).mfma_tile_m == 128
    assert L.default_tuning(1639, 10, 256, 1024, 3072, 32).mfma_tile_m == 192
    assert L.default_tuning(4096, 10, 256, 1024, 3072, 32).mfma_tile_m == 192
    for M in (1, 16, 64, 4096):
        base = L.workspace_size(M, 10, 256, 1024, 3072, 32)
        assert L.workspace_size_ex(M, 10, 256, 1024, 3072, 32, None) == base
        assert L.workspace_size_ex(M, 10, 256, 1024, 3072, 32, pkg.Tuning().to_struct()) == base
    # every expert on MFMA tiles needs a longer tile list than the default split
    all_mfma = pkg.Tuning(gemv_only_max_m=0, gemv_max_tokens=0).to_struct()
    assert L.workspace_size_ex(64, 10, 256, 1024, 3072, 32, all_mfma) > \
        L.workspace_size(64, 10, 256, 1024, 3072, 32)
    # GEMV-only drops the tile list but lists every sorted block for the GEMV
    gemv_only = pkg.Tuning(gemv_only_max_m=pkg.tuning.ALWAYS).to_struct()
    assert L.workspace_size_ex(4096, 10, 256, 1024, 3072, 32, gemv_only) != \
        L.workspace_size(4096, 10, 256, 1024, 3072, 32)


def test_table_roundtrip_and_nearest(pkg, tmp_path):
    T = pkg.tuning
    table = {1: T.Tuning(T.ALWAYS, 4, 1, 0), 16: T.Tuning(T.ALWAYS, 4, 2, 0),
             64: T.Tuning(0, 8, 4, 0), 4096: T.Tuning(0, 2, 0, 0)}
    text = T.dump_table(table)
    assert list(json.loads(text)) == ["1", "16", "64", "4096"]  # M keys only, like vLLM's
    assert T.parse_table(text) == table
    assert T.nearest(table, 1) == table[1]
    assert T.nearest(table, 8) == table[1]       # |8-1| = 7 < |8-16| = 8
    assert T.nearest(table, 40) == table[16]     # tie 24/24 -> smaller key
    assert T.nearest(table, 100) == table[64]
    assert T.nearest(table, 10**6) == table[4096]
    name = T.config_name(256, 1024, 3072, 32, "AMD_Test_GPU")
    assert name == "E=256,N=1024,K=3072,group=32,device_name=AMD_Test_GPU,dtype=int4_w4a16.json"
    (tmp_path / name).write_text(text)
    assert T.load_table(256, 1024, 3072, 32, "AMD_Test_GPU", tmp_path) == table
    assert T.load_table(256, 1024, 3072, 64, "AMD_Test_GPU", tmp_path) is None
    with pytest.raises(ValueError):
        T.parse_table('{"1": {"gemv_only_max_m": 1, "block_m": 16}}')
    with pytest.raises(ValueError):
        T.parse_table("{}")


def test_committed_tables_are_valid(pkg):
    T = pkg.tuning
    for f in sorted(T.CONFIG_DIR.glob("*.json")):
        table = T.parse_table(f.read_text())
        for t in table.values():
            assert _valid(pkg, t), (f.name, t)


def _valid(pkg, t):
    L = pkg._lib
    try:
        L.workspace_size_ex(16, 10, 256, 1024, 3072, 32, t.to_struct())
    except L.W4A16Error:
        return False
    return True


def _tune_module(pkg):
    return importlib.import_module(pkg.__name__ + ".tune")


def test_builtin_as_explicit_tuning(pkg):
    """Tuning.from_struct of the library's built-in choice for M reproduces it:
    the same workspace, and the all-MFMA split from 32 pairs per expert."""
    L = pkg._lib
    for M in (1, 16, 64, 1024, 4096):
        t = pkg.Tuning.from_struct(L.default_tuning(M, 10, 256, 1024, 3072, 32))
        assert t.to_struct().gemv_max_tokens == t.gemv_max_tokens
        assert L.workspace_size_ex(M, 10, 256, 1024, 3072, 32, t.to_struct()) == \
            L.workspace_size(M, 10, 256, 1024, 3072, 32)
        assert (t.gemv_max_tokens == 0) == (M * 10 >= 32 * 256)
    tune = _tune_module(pkg)
    base = pkg.Tuning.from_struct(L.default_tuning(4096, 10, 256, 1024, 3072, 32))
    cands = tune.candidates(4096, 1024, 3072, pkg.Tuning, pkg.tuning.ALWAYS, base)
    assert cands[0] == base and any(c.mfma_tile_m == 128 for c in cands)
    assert any(c.mfma_tile_m == 64 for c in cands)


def test_candidates_are_valid(pkg):
    tune = _tune_module(pkg)
    for M in (1, 4, 16, 64, 4096):
        cands = tune.candidates(M, 1024, 3072, pkg.Tuning, pkg.tuning.ALWAYS)
        assert len(set(cands)) == len(cands) and cands[0] == pkg.Tuning()
        assert all(_valid(pkg, c) for c in cands)
        assert any(c.gemv_only_max_m == pkg.tuning.ALWAYS for c in cands)
        assert any(c.gemv_only_max_m == 0 for c in cands) == (M > 1)


# ---------------------------------------------------------------------------
# GPU
# ---------------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("M", [3, 40, 300])
def test_every_candidate_matches_oracle(pkg, orc, synth, dev, M):
    shape = synth.LayerShape(E=16, topk=4, K=512, N=256, group=32)
    w13, w2, s13, s2 = synth.make_weights(shape, dev, seed=M)
    x = synth.make_hidden(M, shape.K, dev, seed=M)
    tw, ti = synth.make_routing(M, shape.E, shape.topk, dev, seed=M)
    ref = orc.moe_reference(x, w13, w2, s13, s2, tw, ti, shape.group, out_dtype=None)
    for cand in _tune_module(pkg).candidates(M, shape.N, shape.K, pkg.Tuning, pkg.tuning.ALWAYS):
        print(f"tuning M={M} {cand}", flush=True)
        out = pkg.fused_experts_w4a16(x, w13, w2, s13, s2, tw, ti, shape.group, tuning=cand)
        torch.cuda.synchronize()
        o = out.float().cpu()
        assert orc.rel_l2(o, ref) <= 5e-3, cand
        assert orc.max_abs(o, ref) <= 2e-2 * ref.abs().max().item(), cand


@pytest.mark.gpu
def test_tuning_changes_dispatch(pkg, synth, dev):
    """gemv_max_tokens decides which experts get MFMA tiles (header[2])."""
    shape = synth.LayerShape(E=16, topk=4, K=512, N=256, group=32)
    w13, w2, s13, s2 = synth.make_weights(shape, dev, seed=1)
    M = 40
    x = synth.make_hidden(M, shape.K, dev, seed=1)
    tw, ti = synth.make_routing(M, shape.E, shape.topk, dev, seed=1)
    counts = np.bincount(ti.cpu().numpy().reshape(-1), minlength=shape.E)
    for thr in (0, 4, 8, 15):
        t = pkg.Tuning(gemv_only_max_m=0, gemv_max_tokens=thr)
        pkg.fused_experts_w4a16(x, w13, w2, s13, s2, tw, ti, shape.group, tuning=t)
        ws, off = pkg.workspace_tensor(x, ti, w13, w2, shape.group, tuning=t)
        hdr = ws[off[pkg._lib.WS_HEADER]:off[pkg._lib.WS_HEADER] + 16].view(torch.int32).cpu()
        want_tiles = int(sum((c + 191) // 192 for c in counts if c > thr))
        want_gemv = int(sum(1 for c in counts if 0 < c <= thr))
        assert int(hdr[2]) == want_tiles, thr
        assert int(hdr[3]) == want_gemv, thr


@pytest.mark.gpu
def test_table_file_is_used(pkg, synth, dev, tmp_path, monkeypatch):
    T = pkg.tuning
    shape = synth.LayerShape(E=16, topk=4, K=512, N=256, group=32)
    w13, w2, s13, s2 = synth.make_weights(shape, dev, seed=2)
    M = 40
    x = synth.make_hidden(M, shape.K, dev, seed=2)
    tw, ti = synth.make_routing(M, shape.E, shape.topk, dev, seed=2)
    table = {8: T.Tuning(T.ALWAYS, 4, 2, 0), 64: T.Tuning(0, 0, 0, 0)}
    (tmp_path / T.config_name(16, 256, 512, 32, T.device_name(dev))).write_text(
        T.dump_table(table))
    monkeypatch.setenv("W4A16_MOE_CONFIG_DIR", str(tmp_path))
    monkeypatch.delenv("W4A16_MOE_TUNING", raising=False)
    assert T.select(M, 16, 256, 512, 32, dev) == table[64]
    out = pkg.fused_experts_w4a16(x, w13, w2, s13, s2, tw, ti, shape.group)
    ws, off = pkg.workspace_tensor(x, ti, w13, w2, shape.group)
    hdr = ws[off[pkg._lib.WS_HEADER]:off[pkg._lib.WS_HEADER] + 16].view(torch.int32).cpu()
    counts = np.bincount(ti.cpu().numpy().reshape(-1), minlength=shape.E)
    assert int(hdr[2]) == int(sum((c + 127) // 128 for c in counts if c > 0))  # all MFMA
    monkeypatch.setenv("W4A16_MOE_TUNING", "default")
    assert T.select(M, 16, 256, 512, 32, dev) is None
    ref = pkg.fused_experts_w4a16(x, w13, w2, s13, s2, tw, ti, shape.group)
    torch.cuda.synchronize()
    rel = (out.float() - ref.float()).norm() / ref.float().norm()
    assert rel.item() <= 5e-3
