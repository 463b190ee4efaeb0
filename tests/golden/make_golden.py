"""Writes the golden fixtures under tests/golden/ (run once; outputs are committed).

The reference has no tests and ships no vectors for this path, so these
fixtures are worked out here from the reference's stated definitions, with
code that shares nothing with ``oracle/``:

* ``align_cases.json`` -- moe_align_block_size (kernels/w4a16_moe.py:187-290)
  from its definition: for experts in ascending order, the flat indices
  f = m*topk + k routed to that expert in ascending order, padded with the
  sentinel M*topk to a multiple of the block size; the tail of the
  fixed-size buffer of round_up(M*topk + E*(block-1), block) slots
  (kernels/w4a16_moe.py:153-157) is sentinel too;
  expert_ids[b] is the expert whose padded segment holds position b*block,
  -1 past num_post.  Two cases carry expected values written by hand.
* ``dequant_cases.json`` -- (code - 8) * fp32(scale) rounded to bf16
  (bench/bench_moe.py:102-119) for hand-picked words and scales, rounded by
  torch's bf16 cast.
* ``moe_*.npz`` -- whole-layer cases (bench/bench_moe.py:271-303): inputs and
  the float64 output from bf16-rounded dequantized weights, computed with
  float64 numpy matrix products.  ``moe_gemv`` routes at most 4 pairs to each
  expert; ``moe_mfma`` (M = 24 > 16) routes more (the matrix-core path).

Usage:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


# ---------------------------------------------------------------------------
# align
# ---------------------------------------------------------------------------


def align_from_definition(ids: list[list[int]], num_experts: int, block: int):
    flat = [e for row in ids for e in row]
    n_tok = len(flat)
    em = (n_tok + num_experts * (block - 1) + block - 1) // block * block
    n_blocks = em // block
    sorted_ids: list[int] = []
    seg_start = []
    for e in range(num_experts):
        seg_start.append(len(sorted_ids))
        mine = [f for f in range(n_tok) if flat[f] == e]
        sorted_ids += mine
        while len(sorted_ids) % block:
            sorted_ids.append(n_tok)
    num_post = len(sorted_ids)
    seg_start.append(num_post)
    sorted_ids += [n_tok] * (em - num_post)
    expert_ids = []
    for b in range(n_blocks):
        pos = b * block
        owner = -1
        for e in range(num_experts):
            if seg_start[e] <= pos < seg_start[e + 1]:
                owner = e
        expert_ids.append(owner)
    dropped = sum(1 for e in flat if not 0 <= e < num_experts)
    return dict(sorted_ids=sorted_ids, expert_ids=expert_ids, num_post=num_post,
                offsets=seg_start, dropped=dropped)


HAND_ALIGN = [
    # ids [[1,0],[1,2]], E=3, block=2: flat 0..3 -> experts 1,0,1,2
    # expert 0: [1, pad]; expert 1: [0, 2]; expert 2: [3, pad];
    # buffer: 4 + 3*1 = 7 rounded up to 8 slots, 4 blocks
    dict(ids=[[1, 0], [1, 2]], num_experts=3, block=2,
         sorted_ids=[1, 4, 0, 2, 3, 4, 4, 4], expert_ids=[0, 1, 2, -1], num_post=6),
    # ids [[2],[2],[0]], E=4, block=4: expert 0: [2,pad,pad,pad]; 2: [0,1,pad,pad]
    # buffer: 3 + 4*3 = 15 rounded up to 16 slots, 4 blocks
    dict(ids=[[2], [2], [0]], num_experts=4, block=4,
         sorted_ids=[2, 3, 3, 3, 0, 1, 3, 3, 3, 3, 3, 3, 3, 3, 3, 3],
         expert_ids=[0, 2, -1, -1], num_post=8),
]


def align_cases() -> list[dict]:
    cases = []
    for hand in HAND_ALIGN:
        got = align_from_definition(hand["ids"], hand["num_experts"], hand["block"])
        for k in ("sorted_ids", "expert_ids", "num_post"):
            assert got[k] == hand[k], (k, got[k], hand[k])
        cases.append(dict(ids=hand["ids"], num_experts=hand["num_experts"],
                          block=hand["block"], source="hand", **got))
    rng = np.random.default_rng(20261201)
    shapes = [(0, 10, 256, 16), (1, 10, 256, 16), (5, 3, 7, 4), (16, 10, 256, 16),
              (9, 4, 8, 1), (33, 2, 5, 8), (7, 6, 64, 32), (12, 8, 1024, 16)]
    for M, topk, E, block in shapes:
        ids = np.stack([rng.choice(E, size=topk, replace=False) for _ in range(M)]) \
            if M else np.zeros((0, topk), dtype=np.int64)
        ids = ids.astype(int).tolist()
        cases.append(dict(ids=ids, num_experts=E, block=block, source="definition",
                          **align_from_definition(ids, E, block)))
    # skewed: every pair to one expert; and duplicate ids inside one row
    ids = [[3, 3, 3]] * 6
    cases.append(dict(ids=ids, num_experts=4, block=4, source="definition",
                      **align_from_definition(ids, 4, 4)))
    # ids outside [0, E): skipped and counted (the library's rule; the
    # reference does not validate ids)
    ids = [[0, -1], [5, 1], [1, 0], [4, 2]]
    cases.append(dict(ids=ids, num_experts=4, block=2, source="definition",
                      **align_from_definition(ids, 4, 2)))
    return cases


# ---------------------------------------------------------------------------
# dequant
# ---------------------------------------------------------------------------


def bf16_bits(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().astype(np.uint16)


def bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


def dequant_row(words: list[int], scale_bits: list[int], group: int) -> list[int]:
    codes = [(w >> (4 * i)) & 0xF for w in words for i in range(8)]
    scales = bits_to_f32(np.array(scale_bits, dtype=np.uint16))
    vals = np.array([np.float32(c - 8) * scales[k // group] for k, c in enumerate(codes)],
                    dtype=np.float32)
    return bf16_bits(vals).tolist()


def dequant_cases() -> list[dict]:
    cases = []
    one = int(bf16_bits(np.array([1.0]))[0])
    # scale 1: the codes 0..15 give the integers -8..7
    cases.append(dict(words=[0x76543210, 0xFEDCBA98, 0x76543210, 0xFEDCBA98],
                      scale_bits=[one], group=32))
    # a scale whose products need rounding: 0.0123 in bf16 times 3 and 7
    s = int(bf16_bits(np.array([0.0123]))[0])
    cases.append(dict(words=[0xB8F0A7C1, 0x0123CDEF, 0x89ABCDEF, 0x55AA55AA],
                      scale_bits=[s], group=32))
    # group 64 with two scales (second group uses a negative scale)
    s1 = int(bf16_bits(np.array([0.0171]))[0])
    s2 = int(bf16_bits(np.array([-0.006]))[0])
    cases.append(dict(words=[0x12345678, 0x9ABCDEF0] * 8, scale_bits=[s1, s2], group=64))
    for c in cases:
        c["expected_bits"] = dequant_row(c["words"], c["scale_bits"], c["group"])
    # the hand-checked answer of the first case: -8..7, twice
    ints = [float(v) for v in range(-8, 8)] * 2
    assert cases[0]["expected_bits"] == bf16_bits(np.array(ints)).tolist()
    return cases


# ---------------------------------------------------------------------------
# whole layer
# ---------------------------------------------------------------------------


def unpack_codes(packed_u8: np.ndarray) -> np.ndarray:
    lo = packed_u8 & 0xF
    hi = packed_u8 >> 4
    return np.stack([lo, hi], axis=-1).reshape(*packed_u8.shape[:-1], -1)


def dequant_bf16(packed_u8: np.ndarray, scale_bits: np.ndarray, group: int) -> np.ndarray:
    codes = unpack_codes(packed_u8).astype(np.float32) - 8.0
    scale = bits_to_f32(scale_bits)
    vals = codes * np.repeat(scale, group, axis=-1)
    return bits_to_f32(bf16_bits(vals)).astype(np.float64)


def moe_case(name: str, *, M, E, topk, K, N, group, seed, heavy: bool):
    rng = np.random.default_rng(seed)
    w13 = rng.integers(0, 256, size=(E, 2 * N, K // 2), dtype=np.uint8)
    w2 = rng.integers(0, 256, size=(E, K, N // 2), dtype=np.uint8)
    s13 = bf16_bits(rng.uniform(0.005, 0.02, size=(E, 2 * N, K // group)))
    s2 = bf16_bits(rng.uniform(0.005, 0.02, size=(E, K, N // group)))
    x = bf16_bits(rng.standard_normal((M, K)))
    if heavy:
        ids = np.stack([rng.choice(E, size=topk, replace=False) for _ in range(M)])
    else:
        # at most 4 pairs per expert
        pool = np.repeat(np.arange(E), 4)
        while True:  # distinct experts per row, as top-k gives
            ids = rng.permutation(pool)[: M * topk].reshape(M, topk)
            if all(len(set(row)) == topk for row in ids):
                break
    logits = rng.standard_normal((M, topk)).astype(np.float32)
    tw = (np.exp(logits) / np.exp(logits).sum(1, keepdims=True)).astype(np.float32)

    W13 = dequant_bf16(w13, s13, group)
    W2 = dequant_bf16(w2, s2, group)
    xf = bits_to_f32(x).astype(np.float64)
    out = np.zeros((M, K))
    inter = np.zeros((M, topk, N))
    for m in range(M):
        for t in range(topk):
            e = ids[m, t]
            y = W13[e] @ xf[m]
            g, u = y[:N], y[N:]
            a = g / (1.0 + np.exp(-g)) * u
            inter[m, t] = a
            out[m] += float(tw[m, t]) * (W2[e] @ a)
    np.savez_compressed(
        HERE / f"{name}.npz",
        w13=w13, w2=w2, w13_scale_bits=s13, w2_scale_bits=s2, hidden_bits=x,
        topk_ids=ids.astype(np.int32), topk_weights=tw,
        group=np.int32(group), expected_out=out, expected_inter=inter)


def main() -> None:
    (HERE / "align_cases.json").write_text(json.dumps(align_cases(), separators=(",", ":")))
    (HERE / "dequant_cases.json").write_text(json.dumps(dequant_cases(), indent=1))
    moe_case("moe_gemv", M=6, E=8, topk=4, K=256, N=64, group=32, seed=11, heavy=False)
    moe_case("moe_mfma", M=24, E=2, topk=2, K=256, N=256, group=64, seed=12, heavy=True)


if __name__ == "__main__":
    main()
