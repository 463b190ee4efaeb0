"""Pins the CPU oracle (CPU only).

Each oracle function is checked against something other than itself: known
answers worked out by hand from the reference's stated formulas, an
independent formulation (the C counting sort), brute force from the
definition, invariants, and special cases.  The planted-mistake tests at the
end show these checks reject plausible errors.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st


# ---------------------------------------------------------------------------
# pack / unpack  (bench/bench_moe.py:41-53, :87-99; integration/apply.py:29-42)
# ---------------------------------------------------------------------------


def test_pack_known_answer(orc):
    codes = np.arange(16, dtype=np.uint8)[None, :]
    packed = orc.pack_int4(codes)
    # packed[k//2] = q[2k+1]*16 + q[2k]
    assert packed.tolist() == [[0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE]]
    # int32 view: element 8j+i is nibble i of word j
    words = packed.view(np.uint32)
    assert [hex(w) for w in words[0]] == ["0x76543210", "0xfedcba98"]
    assert (orc.unpack_int4(packed) == codes).all()


def test_pack_roundtrip_random(orc):
    rng = np.random.default_rng(1)
    codes = rng.integers(0, 16, size=(3, 5, 64), dtype=np.uint8)
    assert (orc.unpack_int4(orc.pack_int4(codes)) == codes).all()


def test_as_bytes_int32_view(orc):
    rng = np.random.default_rng(2)
    b = rng.integers(0, 256, size=(2, 3, 16), dtype=np.uint8)
    w32 = torch.from_numpy(b.copy()).view(torch.int32)
    assert w32.shape == (2, 3, 4)
    assert (orc.as_bytes(w32) == b).all()


# ---------------------------------------------------------------------------
# dequant  (bench/bench_moe.py:102-119)
# ---------------------------------------------------------------------------


def _bits(x: float) -> int:
    return int(np.float32(x).view(np.uint32) >> 16)


def test_dequant_unit_scale_is_integer(orc):
    codes = np.arange(16, dtype=np.uint8)[None, :]
    codes = np.tile(codes, (1, 2))  # 32 = one group
    packed = orc.pack_int4(codes)
    scale = np.array([[_bits(1.0)]], dtype=np.uint16)
    w = orc.dequant(packed, scale, 32)
    assert w.tolist() == [list(range(-8, 8)) * 2]


def test_dequant_power_of_two_scale_exact(orc):
    rng = np.random.default_rng(3)
    codes = rng.integers(0, 16, size=(4, 64), dtype=np.uint8)
    scales = np.array([[_bits(0.5), _bits(2.0**-7)]] * 4, dtype=np.uint16)
    w = orc.dequant(orc.pack_int4(codes), scales, 32)
    s = np.repeat(np.array([0.5, 2.0**-7], np.float32)[None, :], 4, 0)
    assert (w == (codes.astype(np.float32) - 8) * np.repeat(s, 32, axis=1)).all()


def test_dequant_rounds_to_bf16_nearest_even(orc):
    # scale 1 + 2^-7 (bf16 0x3F81): 7*s = 7.0546875 -> 7.0625 (round up),
    # 3*s = 3.0234375 is a tie between 3.015625 and 3.03125 -> even -> 3.03125,
    # -8*s = -8.0625 is exact, 1*s exact.
    codes = np.full((1, 32), 8, dtype=np.uint8)
    codes[0, :4] = [15, 11, 0, 9]
    scale = np.array([[0x3F81]], dtype=np.uint16)
    w = orc.dequant(orc.pack_int4(codes), scale, 32)
    assert w[0, :4].tolist() == [7.0625, 3.03125, -8.0625, 1.0078125]
    assert (w[0, 4:] == 0).all()


def test_bf16_rounding_helper(orc):
    vals = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0234375], np.float32)
    # 1+2^-8 is a tie -> 1.0 (even); 1+3*2^-8 tie -> 1+2^-6 (even)
    assert orc.bf16_round(vals).tolist() == [1.0, 1.0, 1.015625, -2.5, 3.03125]


# ---------------------------------------------------------------------------
# moe_align_block_size  (kernels/w4a16_moe.py:187-290)
# ---------------------------------------------------------------------------


def _check_same(a, b):
    for x, y in zip(a[:3], b[:3]):
        assert np.array_equal(np.asarray(x), np.asarray(y))


def test_align_known_answer(orc):
    ids = np.array([[2, 0], [2, 1]], np.int32)  # flat f: 0->2, 1->0, 2->2, 3->1
    s, e, n, off, drop = orc.moe_align_block_size(ids, 4, 4)
    assert s.tolist() == [1, 4, 4, 4, 3, 4, 4, 4, 0, 2, 4, 4, 4, 4, 4, 4]
    assert e.tolist() == [0, 1, 2, -1]
    assert n.tolist() == [12]
    assert off.tolist() == [0, 4, 8, 12, 12]
    assert drop == 0
    _check_same(orc.moe_align_block_size_c(ids, 4, 4), (s, e, n))
    _check_same(orc.align_bruteforce(ids, 4, 4), (s, e, n))


def test_align_empty(orc):
    ids = np.zeros((0, 10), np.int32)
    s, e, n, _, _ = orc.moe_align_block_size(ids, 16, 256)
    em = 256 * 15
    assert s.shape == (em,) and (s == 0).all()
    assert e.shape == (em // 16,) and (e == -1).all()
    assert n.tolist() == [0]
    _check_same(orc.moe_align_block_size_c(ids, 16, 256), (s, e, n))


def test_align_block1_is_stable_argsort(orc):
    rng = np.random.default_rng(4)
    ids = rng.integers(0, 7, size=(50, 3)).astype(np.int32)
    s, e, n, _, _ = orc.moe_align_block_size(ids, 1, 7)
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind="stable")
    assert (s[: flat.size] == order).all()
    assert (e[: flat.size] == flat[order]).all()
    assert n[0] == flat.size


def test_align_single_expert(orc):
    ids = np.full((9, 2), 3, np.int32)
    s, e, n, _, _ = orc.moe_align_block_size(ids, 8, 5)
    assert s[:18].tolist() == list(range(18))
    assert s[18:24].tolist() == [18] * 6
    assert n[0] == 24
    assert e[:3].tolist() == [3, 3, 3] and (e[3:] == -1).all()


def _invariants(ids, block, E, out):
    s, e, n = (np.asarray(v) for v in out[:3])
    flat = np.asarray(ids).reshape(-1)
    n_tok = flat.size
    valid = (flat >= 0) & (flat < E)
    em = (n_tok + E * (block - 1) + block - 1) // block * block
    assert s.shape == (em,) and e.shape == (em // block,)
    real = s[s < n_tok]
    assert sorted(real.tolist()) == sorted(np.nonzero(valid)[0].tolist())
    npost = int(n[0])
    assert npost % block == 0 and (s[npost:] == n_tok).all()
    assert (e[npost // block:] == -1).all()
    for b in range(npost // block):
        seg = s[b * block:(b + 1) * block]
        vals = seg[seg < n_tok]
        assert (flat[vals] == e[b]).all()
        assert (np.diff(vals) > 0).all()
        # padding only at the end of a block
        k = vals.size
        assert (seg[k:] == n_tok).all()
    assert (np.diff(e[: npost // block]) >= 0).all()


@settings(max_examples=60, deadline=None, suppress_health_check=[HealthCheck.too_slow])
@given(M=st.integers(0, 40), topk=st.integers(1, 6), E=st.integers(1, 40),
       block=st.sampled_from([1, 2, 3, 8, 16, 64]), seed=st.integers(0, 10**6),
       bad=st.booleans())
def test_align_three_ways_agree(orc, M, topk, E, block, seed, bad):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, E, size=(M, topk)).astype(np.int32)
    if bad and ids.size:
        ids.reshape(-1)[rng.integers(0, ids.size)] = E + 3
    a = orc.moe_align_block_size(ids, block, E)
    b = orc.moe_align_block_size_c(ids, block, E)
    _check_same(a, b)
    assert np.array_equal(a[3], b[3]) and a[4] == b[4]
    if not bad:
        _check_same(a, orc.align_bruteforce(ids, block, E))
        _invariants(ids, block, E, a)


def test_align_full_size_configs(orc, synth):
    for cfg in synth.CONFIGS[:3]:
        tw, ti = synth.make_routing(cfg.M, 256, 10, "cpu", seed=0, skewed=cfg.skewed)
        a = orc.moe_align_block_size(ti.numpy(), 16, 256)
        _check_same(a, orc.moe_align_block_size_c(ti.numpy(), 16, 256))
        _invariants(ti.numpy(), 16, 256, a)


# ---------------------------------------------------------------------------
# moe_reference  (bench/bench_moe.py:271-303)
# ---------------------------------------------------------------------------


def _tiny(synth, seed=0, M=3, E=4, K=64, N=32, topk=2, group=32):
    shape = synth.LayerShape(E=E, topk=topk, K=K, N=N, group=group)
    w13, w2, s13, s2 = synth.make_weights(shape, "cpu", seed=seed)
    x = synth.make_hidden(M, K, "cpu", seed=seed)
    tw, ti = synth.make_routing(M, E, topk, "cpu", seed=seed)
    return shape, x, w13, w2, s13, s2, tw, ti


@pytest.mark.parametrize("exact", [False, True])
def test_moe_reference_matches_f64_bruteforce(orc, synth, exact):
    shape, x, w13, w2, s13, s2, tw, ti = _tiny(synth)
    got = orc.moe_reference(x, w13, w2, s13, s2, tw, ti, 32, exact_weights=exact,
                            out_dtype=None)
    deq = orc.dequant_exact if exact else orc.dequant
    W13 = deq(w13, orc._scale_bits(s13), 32)
    W2 = deq(w2, orc._scale_bits(s2), 32)
    want = orc.moe_bruteforce_f64(x.float().numpy(), W13, W2, tw.numpy(), ti.numpy())
    assert orc.rel_l2(got, torch.from_numpy(want)) < 2e-6


def test_moe_reference_zero_weight_routing(orc, synth):
    shape, x, w13, w2, s13, s2, tw, ti = _tiny(synth)
    out = orc.moe_reference(x, w13, w2, s13, s2, torch.zeros_like(tw), ti, 32,
                            out_dtype=None)
    assert (out == 0).all()


def test_moe_reference_linear_in_routing_weights(orc, synth):
    shape, x, w13, w2, s13, s2, tw, ti = _tiny(synth, M=4)
    a = orc.moe_reference(x, w13, w2, s13, s2, tw, ti, 32, out_dtype=None)
    b = orc.moe_reference(x, w13, w2, s13, s2, 2 * tw, ti, 32, out_dtype=None)
    assert orc.rel_l2(b, 2 * a) < 1e-6


# ---------------------------------------------------------------------------
# planted mistakes: the checks above must reject them
# ---------------------------------------------------------------------------


def test_planted_swapped_nibbles_fails_kat(orc):
    def bad_pack(codes):
        return (codes[..., 0::2].astype(np.uint16) * 16 + codes[..., 1::2]).astype(np.uint8)

    codes = np.arange(16, dtype=np.uint8)[None, :]
    assert bad_pack(codes).tolist() != [[0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE]]


def test_planted_unstable_sort_fails_bruteforce(orc):
    ids = np.array([[1, 0, 1, 1, 0, 1, 1, 1, 0, 1, 1, 0, 1, 1, 1, 1, 1]] * 3, np.int32)
    flat = ids.reshape(-1)
    want = orc.align_bruteforce(ids, 1, 2)[0]
    unstable = np.argsort(flat[::-1], kind="stable")[::-1]
    unstable = flat.size - 1 - unstable  # equal keys in descending index order
    assert not np.array_equal(unstable, want[: flat.size])


def test_planted_missing_offset_fails_dequant_kat(orc):
    codes = np.tile(np.arange(16, dtype=np.uint8), 2)[None, :]
    bad = orc.unpack_int4(orc.pack_int4(codes)).astype(np.float32)  # forgot -8
    assert bad.tolist() != [list(range(-8, 8)) * 2]


def test_planted_no_silu_fails_bruteforce(orc, synth):
    shape, x, w13, w2, s13, s2, tw, ti = _tiny(synth)
    W13 = orc.dequant(w13, orc._scale_bits(s13), 32).astype(np.float64)
    W2 = orc.dequant(w2, orc._scale_bits(s2), 32).astype(np.float64)
    want = orc.moe_bruteforce_f64(x.float().numpy(), W13, W2, tw.numpy(), ti.numpy())
    xf = x.float().numpy().astype(np.float64)
    bad = np.zeros_like(want)
    for m in range(xf.shape[0]):
        for t in range(ti.shape[1]):
            e = int(ti[m, t])
            y = W13[e] @ xf[m]
            bad[m] += float(tw[m, t]) * (W2[e] @ (y[:32] * y[32:]))  # gate not SiLU'd
    assert orc.rel_l2(torch.from_numpy(bad), torch.from_numpy(want)) > 1e-2


@pytest.mark.parametrize("group", [32, 64, 128])
def test_torch_dequant_equals_numpy_dequant(orc, group):
    rng = np.random.default_rng(5)
    packed = rng.integers(0, 256, size=(6, 128), dtype=np.uint8)
    scales = orc.f32_to_bf16_bits(rng.uniform(0.001, 3.0, size=(6, 256 // group)))
    s_t = torch.from_numpy(scales.view(np.int16)).view(torch.bfloat16)
    got = orc.dequant_t(torch.from_numpy(packed), s_t, group).numpy()
    assert np.array_equal(got, orc.dequant(packed, scales, group))
    got_x = orc.dequant_t(torch.from_numpy(packed), s_t, group, exact=True).numpy()
    assert np.array_equal(got_x.astype(np.float64), orc.dequant_exact(packed, scales, group))


# ---------------------------------------------------------------------------
# the reference kernel's bf16 rounding points (kernels/w4a16_moe.py:489, :311)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("inter,partial", [(True, False), (False, True), (True, True)])
def test_moe_reference_rounding_points_match_bruteforce(orc, synth, inter, partial):
    # Independent scalar float64 loops round at the same points; leaving a
    # rounding out (or putting it elsewhere) differs by bf16 ulps, far above
    # the fp32-vs-float64 noise of 1e-6.
    shape, x, w13, w2, s13, s2, tw, ti = _tiny(synth, M=4, topk=3)
    W13 = orc.dequant(w13, orc._scale_bits(s13), 32)
    W2 = orc.dequant(w2, orc._scale_bits(s2), 32)
    xf, twn, tin = x.float().numpy(), tw.numpy(), ti.numpy()
    got = orc.moe_reference(x, w13, w2, s13, s2, tw, ti, 32, round_inter=inter,
                            round_partial=partial, out_dtype=None)
    want = orc.moe_bruteforce_f64(xf, W13, W2, twn, tin, round_inter=inter,
                                  round_partial=partial)
    plain = orc.moe_bruteforce_f64(xf, W13, W2, twn, tin)
    other = orc.moe_bruteforce_f64(xf, W13, W2, twn, tin, round_inter=not inter,
                                   round_partial=partial)
    assert orc.rel_l2(got, torch.from_numpy(want)) < 2e-6
    assert orc.rel_l2(torch.from_numpy(plain), torch.from_numpy(want)) > 1e-4
    assert orc.rel_l2(torch.from_numpy(other), torch.from_numpy(want)) > 1e-4


def test_moe_reference_round_partial_skips_invalid_slots(orc, synth):
    # A slot routed outside [0, E) contributes nothing: the same as routing it
    # with weight 0 (whose bf16 partial is +0.0).
    shape, x, w13, w2, s13, s2, tw, ti = _tiny(synth, M=4, topk=3)
    bad = ti.clone()
    bad[1, 2] = -1
    bad[3, 0] = shape.E
    zw = tw.clone()
    zw[1, 2] = 0.0
    zw[3, 0] = 0.0
    a = orc.moe_reference(x, w13, w2, s13, s2, tw, bad, 32, round_partial=True,
                          out_dtype=None)
    b = orc.moe_reference(x, w13, w2, s13, s2, zw, ti, 32, round_partial=True,
                          out_dtype=None)
    assert torch.equal(a, b)
