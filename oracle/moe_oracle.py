"""CPU oracle for the W4A16 grouped-expert MoE path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg may import this module, and only as the
checker (or the timed CPU baseline).  The product path never calls it and has
no CPU fallback.

Every function restates the reference's algorithm from its source text; the
reference itself is never imported or executed.  Citations are
``file:line`` into vladimir-voinea/gb10-laguna-s-2.1-w4a16-moe.

Contents and what pins each one (the checks live in tests/test_oracle.py):

* ``pack_int4`` / ``unpack_int4`` -- bench/bench_moe.py:87-99.  Pinned by the
  known-answer bytes of the formula ``packed[k//2] = q[2k+1]*16 + q[2k]``
  (bench_moe.py:47) and by the int32 view of compressed-tensors
  (element 8j+i in bits 4i of word j, integration/apply.py:29-42).
* ``dequant`` -- bench/bench_moe.py:102-119, ``(code-8) * fp32(scale)`` rounded
  to bf16.  Pinned by closed forms (scale 1 gives the integers -8..7; scales
  that are powers of two are exact) and a hand-rounded RNE case.
* ``moe_align_block_size`` -- kernels/w4a16_moe.py:187-290, restated op by op
  (histogram, padded cumsum, stable sort, amin rank, searchsorted).  Pinned by
  the independent C counting sort in align_ref.c, by brute force from the
  definition on small inputs, by its invariants, and by special cases
  (no pairs, one expert, block 1 = a textbook stable argsort).
* ``moe_reference`` -- bench/bench_moe.py:271-303 (per-expert fp32 GEMMs,
  SiLU(gate)*up, top-k-weighted index_add_, bf16 cast), with the dequant done
  inside (it is the timed CPU baseline).  Pinned by a float64 brute force
  (``moe_bruteforce_f64``) on tiny shapes and by linearity/zero-routing cases.
  ``moe_partials`` returns the same loop's per-(token, slot) rows before the
  sum (pinned through moe_reference, which sums them).  Its options for the reference kernel's two bf16 rounding points
  (``round_inter``: SiLU(gate)*up, kernels/w4a16_moe.py:489; ``round_partial``:
  the top-k-weighted w2 rows, :311, summed in slot order by :638-668) are
  pinned by the brute force's own scalar rounding at the same points, on
  inputs where leaving a rounding out moves the result far beyond the
  fp32-vs-float64 noise.

* ``router_topk_softmax`` -- bench/bench_moe.py:225-230 (``torch.topk`` then
  ``torch.softmax`` over the selected logits), equal logits in ascending
  expert index.  Pinned by torch.topk itself on tie-free rows, by the stable
  ``torch.sort`` on rows full of ties (torch.topk's own order among equal
  values is unspecified and differs), by torch.topk's placement of NaN, +-inf
  and signed zeros, by ``torch.softmax`` and by closed forms (equal logits
  give 1/k, two logits give the logistic function).

Synthetic inputs are built by the product's own generator; the oracle only
consumes tensors.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

ORACLE_DIR = Path(__file__).resolve().parent
_C_LIB_PATH = ORACLE_DIR / "liboracle_align.so"

# ---------------------------------------------------------------------------
# bf16 helpers (numpy has no bf16 dtype; bf16 values travel as uint16 bits)
# ---------------------------------------------------------------------------


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16); NaN stays NaN."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    nan = np.isnan(a)
    rounded = np.where(nan, (u >> 16).astype(np.uint32) | 0x40, rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(a: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


# ---------------------------------------------------------------------------
# pack-quantized int4 (bench/bench_moe.py:41-119)
# ---------------------------------------------------------------------------


def pack_int4(codes: np.ndarray) -> np.ndarray:
    """Codes 0..15 [..., k] -> bytes [..., k/2]; low nibble = even k.

    Restates pack_int4_nibbles, bench/bench_moe.py:87-92.
    """
    codes = np.asarray(codes)
    assert codes.shape[-1] % 2 == 0
    assert codes.min(initial=0) >= 0 and codes.max(initial=0) <= 15
    low = codes[..., 0::2].astype(np.uint16)
    high = codes[..., 1::2].astype(np.uint16)
    return (high * 16 + low).astype(np.uint8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """Bytes [..., k/2] -> codes [..., k]; restates bench/bench_moe.py:95-99."""
    packed = np.asarray(packed, dtype=np.uint8)
    low = packed & 0x0F
    high = (packed >> 4) & 0x0F
    return np.stack([low, high], axis=-1).reshape(*packed.shape[:-1], -1)


def as_bytes(w) -> np.ndarray:
    """uint8 view of packed weights given as uint8 [..., k/2] or int32 [..., k/8]."""
    if isinstance(w, torch.Tensor):
        w = w.detach().cpu()
        if w.dtype == torch.int32:
            w = w.view(torch.uint8)
        w = w.numpy()
    w = np.ascontiguousarray(w)
    if w.dtype in (np.int32, np.uint32):
        w = w.view(np.uint8)
    assert w.dtype == np.uint8
    return w


def dequant(packed, scale_bits, group: int) -> np.ndarray:
    """(code - 8) * fp32(bf16 scale), rounded to bf16, returned as float32.

    Restates dequant_int4_w4a16, bench/bench_moe.py:102-119, fed with the
    stored bf16 scales.
    """
    codes = unpack_int4(as_bytes(packed)).astype(np.int16) - 8
    s = bf16_bits_to_f32(np.asarray(scale_bits, dtype=np.uint16))
    k = codes.shape[-1]
    assert k % group == 0 and s.shape[-1] == k // group
    s_full = np.repeat(s, group, axis=-1)
    return bf16_round(codes.astype(np.float32) * s_full)


def dequant_exact(packed, scale_bits, group: int) -> np.ndarray:
    """(code - 8) * scale in float64, no rounding (for tight checks)."""
    codes = unpack_int4(as_bytes(packed)).astype(np.float64) - 8.0
    s = bf16_bits_to_f32(np.asarray(scale_bits, dtype=np.uint16)).astype(np.float64)
    return codes * np.repeat(s, group, axis=-1)


# ---------------------------------------------------------------------------
# moe_align_block_size (kernels/w4a16_moe.py:141-290)
# ---------------------------------------------------------------------------


def align_sizes(n_tok: int, num_experts: int, block: int) -> tuple[int, int]:
    """EM and block count; kernels/w4a16_moe.py:153-157."""
    em = n_tok + num_experts * (block - 1)
    em = (em + block - 1) // block * block
    return em, em // block


def moe_align_block_size(topk_ids, block_size: int, num_experts: int):
    """Numpy restatement of kernels/w4a16_moe.py:187-290, op by op.

    Returns (sorted_token_ids int32[EM], expert_ids int32[EM/B],
    num_tokens_post_padded int32[1], offsets int32[E+1], dropped int).
    Ids outside [0, E) are skipped (and counted), as the product does.
    """
    ids = np.asarray(topk_ids).reshape(-1).astype(np.int64)  # :238-241
    n_tok = ids.size
    em, nb = align_sizes(n_tok, num_experts, block_size)
    sorted_ids = np.full(em, n_tok, dtype=np.int32)  # :230
    expert_ids = np.full(nb, -1, dtype=np.int32)  # :231
    offsets = np.zeros(num_experts + 1, dtype=np.int64)
    valid = (ids >= 0) & (ids < num_experts)
    dropped = int((~valid).sum())
    if n_tok == 0:  # :233-235
        return sorted_ids, expert_ids, np.zeros(1, np.int32), offsets.astype(np.int32), 0
    flat = np.arange(n_tok, dtype=np.int64)[valid]
    experts = ids[valid]
    counts = np.zeros(num_experts, dtype=np.int64)
    np.add.at(counts, experts, 1)  # scatter_add_ histogram, :249
    blocks_per = (counts + (block_size - 1)) // block_size  # :251
    tokens_pad_per = blocks_per * block_size  # :252
    offsets[1:] = np.cumsum(tokens_pad_per)  # :258-259
    num_post = np.array([offsets[-1]], dtype=np.int32)  # :261
    order = np.argsort(experts, kind="stable")  # torch.sort(stable=True), :263
    sorted_expert = experts[order]
    arange = np.arange(sorted_expert.size, dtype=np.int64)
    exp_first = np.full(num_experts, sorted_expert.size, dtype=np.int64)  # :271
    np.minimum.at(exp_first, sorted_expert, arange)  # scatter_reduce amin, :272-274
    rank = arange - exp_first[sorted_expert]  # :275
    dest = offsets[sorted_expert] + rank  # :276
    sorted_ids[dest] = flat[order].astype(np.int32)  # :278
    block_tok0 = np.arange(nb, dtype=np.int64) * block_size
    e_for_block = np.searchsorted(offsets[1:], block_tok0, side="right")  # :283
    e_for_block = np.where(block_tok0 < offsets[-1], e_for_block, -1)  # :286-288
    expert_ids[:] = e_for_block.astype(np.int32)
    return sorted_ids, expert_ids, num_post, offsets.astype(np.int32), dropped


def moe_align_block_size_c(topk_ids, block_size: int, num_experts: int):
    """Same outputs from the C counting-sort oracle (align_ref.c)."""
    lib = _c_lib()
    ids = np.ascontiguousarray(np.asarray(topk_ids).reshape(-1), dtype=np.int32)
    n_tok = ids.size
    em, nb = align_sizes(n_tok, num_experts, block_size)
    sorted_ids = np.empty(em, dtype=np.int32)
    expert_ids = np.empty(nb, dtype=np.int32)
    num_post = np.zeros(1, dtype=np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    dropped = np.zeros(1, dtype=np.int32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    st = lib.oracle_align_block_size(
        p(ids), n_tok, num_experts, block_size, p(sorted_ids), em, p(expert_ids), nb,
        p(num_post), p(offsets), p(dropped))
    if st != 0:
        raise RuntimeError(f"oracle_align_block_size failed: {st}")
    return sorted_ids, expert_ids, num_post, offsets, int(dropped[0])


def align_bruteforce(topk_ids, block_size: int, num_experts: int):
    """The definition, in plain Python loops (small inputs only)."""
    ids = [int(v) for v in np.asarray(topk_ids).reshape(-1)]
    n_tok = len(ids)
    em, nb = align_sizes(n_tok, num_experts, block_size)
    out, eids = [], []
    for e in range(num_experts):
        mine = [f for f, v in enumerate(ids) if v == e]
        if not mine:
            continue
        pad = -len(mine) % block_size
        seg = mine + [n_tok] * pad
        out += seg
        eids += [e] * (len(seg) // block_size)
    num_post = len(out)
    out += [n_tok] * (em - len(out))
    eids += [-1] * (nb - len(eids))
    return (np.array(out, np.int32), np.array(eids, np.int32),
            np.array([num_post], np.int32))


_c_handle = None


def _c_lib():
    global _c_handle
    if _c_handle is None:
        if not _C_LIB_PATH.exists():
            build_c_oracle()
        lib = ctypes.CDLL(str(_C_LIB_PATH))
        i64, vp = ctypes.c_int64, ctypes.c_void_p
        lib.oracle_align_block_size.restype = ctypes.c_int
        lib.oracle_align_block_size.argtypes = [
            vp, i64, i64, i64, vp, i64, vp, i64, vp, vp, vp]
        _c_handle = lib
    return _c_handle


def build_c_oracle() -> Path:
    import subprocess

    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return _C_LIB_PATH


# ---------------------------------------------------------------------------
# The dequant MoE reference (bench/bench_moe.py:271-303)
# ---------------------------------------------------------------------------


def _scale_bits(s) -> np.ndarray:
    if isinstance(s, torch.Tensor):
        s = s.detach().cpu()
        assert s.dtype == torch.bfloat16
        return s.view(torch.int16).numpy().view(np.uint16)
    return np.asarray(s, dtype=np.uint16)


def dequant_t(packed: torch.Tensor, scale: torch.Tensor, group: int,
              exact: bool = False) -> torch.Tensor:
    """Torch (CPU) version of ``dequant``: same values, vectorized.

    packed: uint8 [..., k/2] (or int32 [..., k/8]); scale: bf16 [..., k/group].
    exact=False rounds (code-8)*scale to bf16 like bench/bench_moe.py:119;
    exact=True keeps the fp32 product (exact: <= 12 significant bits).
    """
    if packed.dtype == torch.int32:
        packed = packed.view(torch.uint8)
    lo = (packed & 0x0F).to(torch.int16)
    hi = (packed >> 4).to(torch.int16)
    codes = torch.stack([lo, hi], dim=-1).reshape(*packed.shape[:-1], -1)
    vals = (codes - 8).to(torch.float32)
    s = scale.to(torch.float32).repeat_interleave(group, dim=-1)
    w = vals * s
    return w if exact else w.to(torch.bfloat16).to(torch.float32)


def _dequant_torch(packed_e, scale_e, group: int, exact: bool) -> torch.Tensor:
    """Dequantize one expert's rows to an fp32 tensor (bf16-rounded unless exact)."""
    return dequant_t(packed_e, scale_e, group, exact)


def _as_u8_tensor(w) -> torch.Tensor:
    if not isinstance(w, torch.Tensor):
        w = torch.from_numpy(as_bytes(w))
    w = w.detach().cpu()
    if w.dtype == torch.int32:
        w = w.view(torch.uint8)
    assert w.dtype == torch.uint8
    return w


def _expert_rows(hidden: torch.Tensor, w13, w2, w13_scale, w2_scale,
                 topk_weights: torch.Tensor, topk_ids: torch.Tensor, group: int,
                 exact_weights: bool, round_inter: bool, bf16_weight_experts):
    """Yield (token_idx, slot_idx, fp32 top-k-weighted w2 rows) per routed expert.

    The per-expert body of run_reference (bench/bench_moe.py:277-303): fp32
    ``F.linear`` against the dequantized w13, SiLU(gate)*up (silu_and_mul,
    :271-274), fp32 ``F.linear`` against w2, times the routing weight.
    """
    hidden = hidden.detach().cpu()
    w13b = _as_u8_tensor(w13)
    w2b = _as_u8_tensor(w2)
    s13 = w13_scale.detach().cpu()
    s2 = w2_scale.detach().cpu()
    assert s13.dtype == torch.bfloat16 and s2.dtype == torch.bfloat16
    E = w13b.shape[0]
    N = w13b.shape[1] // 2
    h = hidden.to(torch.float32)
    tw = topk_weights.detach().cpu().to(torch.float32)
    ids = topk_ids.detach().cpu().to(torch.int64)
    for e in range(E):
        mask = ids == e
        if not bool(mask.any()):
            continue
        token_idx, slot_idx = mask.nonzero(as_tuple=True)
        exact = exact_weights and e not in bf16_weight_experts
        W13 = _dequant_torch(w13b[e], s13[e], group, exact)  # [2N, K]
        W2 = _dequant_torch(w2b[e], s2[e], group, exact)  # [K, N]
        y = F.linear(h[token_idx], W13)
        a = F.silu(y[:, :N]) * y[:, N:]
        if round_inter:
            a = a.to(torch.bfloat16).to(torch.float32)
        yield token_idx, slot_idx, F.linear(a, W2) * tw[token_idx, slot_idx].unsqueeze(-1)


def moe_partials(hidden: torch.Tensor, w13, w2, w13_scale, w2_scale,
                 topk_weights: torch.Tensor, topk_ids: torch.Tensor, group: int = 32,
                 *, exact_weights: bool = False, round_inter: bool = False,
                 bf16_weight_experts=()):
    """(partial fp32 [M, topk, K], valid bool [M, topk]): the top-k-weighted
    w2 row of every (token, slot) pair before any rounding, zero where the
    slot's id is outside [0, E) -- the rows the reference kernel stores in its
    partial buffer (kernels/w4a16_moe.py:311, :851-888).  Options as in
    moe_reference."""
    M, K = hidden.shape
    topk = topk_ids.shape[1]
    part = torch.zeros((M, topk, K), dtype=torch.float32)
    valid = torch.zeros((M, topk), dtype=torch.bool)
    for token_idx, slot_idx, z in _expert_rows(hidden, w13, w2, w13_scale, w2_scale,
                                               topk_weights, topk_ids, group, exact_weights,
                                               round_inter, bf16_weight_experts):
        part[token_idx, slot_idx] = z
        valid[token_idx, slot_idx] = True
    return part, valid


def moe_reference(hidden: torch.Tensor, w13, w2, w13_scale, w2_scale,
                  topk_weights: torch.Tensor, topk_ids: torch.Tensor, group: int = 32,
                  *, exact_weights: bool = False, round_inter: bool = False,
                  round_partial: bool = False, bf16_weight_experts=(),
                  out_dtype=torch.bfloat16) -> torch.Tensor:
    """PyTorch CPU dequant reference for one MoE layer.

    Restates run_reference (bench/bench_moe.py:277-303): for every expert with
    routed pairs, fp32 ``F.linear`` against the dequantized w13, SiLU(gate)*up
    (silu_and_mul, :271-274), fp32 ``F.linear`` against w2, then
    ``index_add_`` of the top-k-weighted rows in expert order and a final cast.
    The dequantization runs inside (from the unchanged packed tensors).

    exact_weights: use (code-8)*scale without the bf16 rounding of the dequant.
    bf16_weight_experts: experts that keep the bf16 rounding even when
    exact_weights is set (a per-expert mix of both rounding points).
    round_inter: round SiLU(gate)*up to bf16 like the reference kernel does
    (kernels/w4a16_moe.py:489).
    round_partial: round each top-k-weighted w2 row to bf16 and sum the rows
    of a token in fp32 in slot order from +0.0, leaving out slots whose id is
    outside [0, E) -- the reference kernel's bf16 partial buffer
    (kernels/w4a16_moe.py:311) and _moe_sum_kernel (:638-668).
    """
    M, K = hidden.shape
    out = torch.zeros((M, K), dtype=torch.float32)
    args = (hidden, w13, w2, w13_scale, w2_scale, topk_weights, topk_ids, group)
    if round_partial:
        part, valid = moe_partials(*args, exact_weights=exact_weights,
                                   round_inter=round_inter,
                                   bf16_weight_experts=bf16_weight_experts)
        part = part.to(torch.bfloat16).to(torch.float32)
        for t in range(part.shape[1]):
            rows = valid[:, t]
            out[rows] += part[rows, t]
    else:
        for token_idx, _, z in _expert_rows(*args, exact_weights, round_inter,
                                            bf16_weight_experts):
            out.index_add_(0, token_idx, z)
    return out if out_dtype is None else out.to(out_dtype)


def moe_bruteforce_f64(hidden_f32: np.ndarray, w13_deq: np.ndarray, w2_deq: np.ndarray,
                       topk_weights: np.ndarray, topk_ids: np.ndarray, *,
                       round_inter: bool = False, round_partial: bool = False) -> np.ndarray:
    """Float64 scalar loops straight from the definition (tiny shapes only).

    out[m,k] = sum_t w[m,t] * sum_n W2[e,k,n] * silu(g_n) * u_n,
    g_n = sum_j W13[e,n,j] x[m,j],  u_n = sum_j W13[e,N+n,j] x[m,j].
    round_inter rounds each silu(g_n) * u_n to bf16, round_partial each
    w[m,t] * sum_n (...) term (the reference kernel's rounding points,
    kernels/w4a16_moe.py:489 and :311); the terms are summed in slot order.
    """
    x = np.asarray(hidden_f32, dtype=np.float64)
    M, K = x.shape
    N = w13_deq.shape[1] // 2
    out = np.zeros((M, K), dtype=np.float64)
    for m in range(M):
        for t in range(topk_ids.shape[1]):
            e = int(topk_ids[m, t])
            if e < 0 or e >= w13_deq.shape[0]:
                continue
            a = np.zeros(N)
            for n in range(N):
                g = sum(float(w13_deq[e, n, j]) * x[m, j] for j in range(K))
                u = sum(float(w13_deq[e, N + n, j]) * x[m, j] for j in range(K))
                a[n] = g / (1.0 + np.exp(-g)) * u
                if round_inter:
                    a[n] = float(bf16_round(np.array([a[n]], dtype=np.float32))[0])
            for k in range(K):
                p = float(topk_weights[m, t]) * sum(
                    float(w2_deq[e, k, n]) * a[n] for n in range(N))
                if round_partial:
                    p = float(bf16_round(np.array([p], dtype=np.float32))[0])
                out[m, k] += p
    return out


# ---------------------------------------------------------------------------
# router step (bench/bench_moe.py:225-230)
# ---------------------------------------------------------------------------


def router_topk_softmax(logits, topk: int, renormalize: bool = True):
    """(weights float64 [M, topk], ids int64 [M, topk]) from fp32 logits [M, E].

    Selection: ``torch.topk(logits, topk)`` (bench_moe.py:227) -- descending
    value, NaN first, -0.0 equal to +0.0; equal values in ascending index.
    Weights: ``torch.softmax(vals)`` over the selected logits
    (bench_moe.py:231), evaluated in float64; renormalize=False gives the
    softmax over all E logits read at the selected experts instead.
    """
    x = np.asarray(logits, dtype=np.float32)
    M, E = x.shape
    if M == 0:
        return np.zeros((0, topk)), np.zeros((0, topk), dtype=np.int64)
    xd = x.astype(np.float64)
    nan = np.isnan(xd)
    # rank key: NaN above everything, then by value (-0.0 == +0.0 in float compare)
    rank = np.where(nan, np.inf, xd)
    ids = np.empty((M, topk), dtype=np.int64)
    for m in range(M):
        order = sorted(range(E), key=lambda j: (not nan[m, j], -rank[m, j], j))
        ids[m] = order[:topk]
    vals = np.take_along_axis(xd, ids, axis=1)
    mx = vals[:, :1]
    with np.errstate(invalid="ignore"):  # inf - inf and NaN rows give NaN, as in torch
        ex = np.exp(vals - mx)
        if renormalize:
            den = ex.sum(axis=1, keepdims=True)
        else:
            den = np.exp(xd - mx).sum(axis=1, keepdims=True)
        return ex / den, ids


# ---------------------------------------------------------------------------
# error metrics (bench/bench_moe.py:520-527)
# ---------------------------------------------------------------------------


def rel_l2(a, b) -> float:
    a = torch.as_tensor(a).double()
    b = torch.as_tensor(b).double()
    return float((a - b).norm() / (b.norm() + 1e-30))


def max_abs(a, b) -> float:
    return float((torch.as_tensor(a).double() - torch.as_tensor(b).double()).abs().max())
