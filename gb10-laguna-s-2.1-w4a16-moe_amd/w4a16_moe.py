"""W4A16 grouped-expert MoE for MI355X -- the reference's Python interface.

Mirrors ``kernels/w4a16_moe.py`` of vladimir-voinea/gb10-laguna-s-2.1-w4a16-moe
(same function names, positional arguments and argument meaning) on top of the
HIP library ``libw4a16moe.so`` (C ABI: include/w4a16_moe.h).  PyTorch supplies
device memory and the current stream only; all arithmetic runs in the HIP
kernels.  There is no CPU fallback: a missing library raises.

Differences from the reference, all deliberate:
  * weights are consumed in the stock pack-quantized layout; ``repack_weights``
    is the identity and 4-D repacked tensors are refused;
  * the top-k combine is deterministic (slot order) for every M, where the
    reference uses fp32 atomics for M <= 4;
  * ``moe_align_block_size`` returns fresh tensors instead of buffers aliased
    across calls;
  * expert ids outside [0, E) are skipped (and counted) instead of indexing
    out of bounds.
"""

from __future__ import annotations

import ctypes
import threading

import torch

from . import _lib
from . import tuning as _tuning

_GROUP_SIZE_DEFAULT = 32
# Accepted for signature compatibility with the reference; the HIP kernels
# choose their own tiling.
BLOCK_M = 16
BLOCK_N = 64
BLOCK_K = 64



class WorkspacePool:
    """Workspaces of the fused call, kept for reuse.

    Eager calls: one buffer per (device, stream), grown to the largest size a
    call has needed and reused by every smaller call.  Calls on one stream run
    in order, so they can share one buffer; calls on different streams get
    different buffers (the C ABI's rule: calls sharing a workspace must not
    overlap).

    Calls under HIP graph capture: one buffer per (device, stream, capture),
    shared only by the calls of that capture (which the graph runs in order).
    A graph runs on whatever stream it is replayed on, so graphs captured on
    one stream may later run concurrently; giving each capture its own buffer
    keeps them apart.  Capture buffers are never reused by later calls, and a
    capture buffer outgrown within its capture stays alive (the graph's
    kernels keep its address): both are held until ``release_captures()``
    (or ``clear()``), which callers make once the graphs are destroyed.

    The reference pools its scratch per (device, M, ...) shape
    (kernels/w4a16_moe.py:293-316), which keeps one buffer per distinct M for
    the life of the process.
    """

    def __init__(self, alloc=None):
        self._alloc = alloc or (lambda nbytes, device: torch.empty(
            nbytes, dtype=torch.uint8, device=device))
        self._bufs: dict[tuple, torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []  # capture buffers outgrown in their capture
        self._lock = threading.Lock()

    def get(self, device, stream: int, nbytes: int, capture_id: int = 0) -> torch.Tensor:
        """A workspace of at least `nbytes` for a call on `stream`, under the
        graph capture `capture_id` (0: not capturing)."""
        key = (str(device), int(stream), int(capture_id))
        need = max(int(nbytes), 256)
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < need:
                if buf is not None and capture_id:
                    self._retired.append(buf)
                buf = self._alloc(need, device)
                self._bufs[key] = buf
            return buf

    def cached_bytes(self) -> int:
        """Bytes held by the live buffers (eager and capture ones)."""
        return sum(b.numel() for b in self._bufs.values())

    def capture_bytes(self) -> int:
        """Bytes held for graph captures (live and outgrown)."""
        return (sum(b.numel() for k, b in self._bufs.items() if k[2])
                + sum(b.numel() for b in self._retired))

    def retired_bytes(self) -> int:
        """Bytes of capture buffers outgrown within their capture (held until
        ``release_captures()``)."""
        return sum(b.numel() for b in self._retired)

    def release_captures(self) -> None:
        """Drop every capture buffer; only once the graphs that captured them
        are destroyed.  The eager buffers stay."""
        with self._lock:
            self._bufs = {k: b for k, b in self._bufs.items() if not k[2]}
            self._retired.clear()

    def clear(self) -> None:
        """Drop every buffer; only for callers whose graphs are all gone."""
        with self._lock:
            self._bufs.clear()
            self._retired.clear()


_WS_POOL = WorkspacePool()


def release_graph_workspaces() -> None:
    """Free the workspaces held for HIP-graph captures of fused_experts_w4a16.

    Each captured graph keeps its own workspace (graphs captured on one stream
    may be replayed concurrently); call this once those graphs are destroyed.
    Eager calls' workspaces are kept.  No counterpart in the reference, whose
    per-shape scratch is never freed (kernels/w4a16_moe.py:293-316).
    """
    _WS_POOL.release_captures()


def _fail(msg: str) -> None:
    raise _lib.W4A16Error(msg)


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------
# Load-side layout helpers (reference: kernels/w4a16_moe.py:63-121)
# ---------------------------------------------------------------------------


def repack_weights(w_q: torch.Tensor, scales: torch.Tensor, block_n: int = BLOCK_N):
    """Identity: the HIP kernels read the stock layout directly.

    Reference: repack_weights, kernels/w4a16_moe.py:63-116, which permutes
    ``(E, N_out, K/2)`` into an N-tile-major 4-D layout.  Keeping this entry
    point lets the reference's load hook (integration/apply.py:99-112) run
    unchanged; it binds the same tensors and frees nothing extra.
    """
    if w_q.ndim != 3 or scales.ndim != 3:
        _fail("repack_weights expects 3-D (E, N_out, K_packed) weights and scales")
    return w_q, scales


def is_repacked(w_q: torch.Tensor) -> bool:
    """True for the reference's 4-D N-tile layout (kernels/w4a16_moe.py:119-121)."""
    return w_q.ndim == 4


# ---------------------------------------------------------------------------
# Routing: expert-sorted block assignment (kernels/w4a16_moe.py:187-290)
# ---------------------------------------------------------------------------


def _ids_i32(topk_ids: torch.Tensor) -> torch.Tensor:
    if topk_ids.dtype != torch.int32:
        topk_ids = topk_ids.to(torch.int32)
    return topk_ids.contiguous()


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int, num_experts: int):
    """Sort token-slots by expert and pad each expert to a multiple of block_size.

    Returns (sorted_token_ids int32[EM], expert_ids int32[EM/B],
    num_tokens_post_padded int32[1]) with EM = round_up(M*topk + E*(B-1), B),
    bit-identical to kernels/w4a16_moe.py:187-290.  One HIP launch on the
    current stream, no host synchronisation.
    """
    if not topk_ids.is_cuda:
        _fail("topk_ids must be on the GPU")
    if topk_ids.ndim != 2:
        _fail("topk_ids must be [M, topk]")
    M, topk = topk_ids.shape
    em, nb = _lib.align_sizes(M, topk, num_experts, block_size)
    dev = topk_ids.device
    ids = _ids_i32(topk_ids)
    sorted_ids = torch.empty(em, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(nb, dtype=torch.int32, device=dev)
    num_post = torch.empty(1, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        st = _lib.lib().w4a16_moe_align_block_size(
            ids.data_ptr(), M, topk, num_experts, block_size, sorted_ids.data_ptr(),
            expert_ids.data_ptr(), num_post.data_ptr(), None, None, _stream_ptr(dev))
    _lib.check(st)
    return sorted_ids, expert_ids, num_post


def moe_align_block_size_full(topk_ids: torch.Tensor, block_size: int, num_experts: int):
    """moe_align_block_size plus expert_offsets int32[E+1] and the dropped count."""
    if not topk_ids.is_cuda or topk_ids.ndim != 2:
        _fail("topk_ids must be a [M, topk] GPU tensor")
    M, topk = topk_ids.shape
    em, nb = _lib.align_sizes(M, topk, num_experts, block_size)
    dev = topk_ids.device
    ids = _ids_i32(topk_ids)
    sorted_ids = torch.empty(em, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(nb, dtype=torch.int32, device=dev)
    num_post = torch.empty(1, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    dropped = torch.empty(1, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        st = _lib.lib().w4a16_moe_align_block_size(
            ids.data_ptr(), M, topk, num_experts, block_size, sorted_ids.data_ptr(),
            expert_ids.data_ptr(), num_post.data_ptr(), offsets.data_ptr(),
            dropped.data_ptr(), _stream_ptr(dev))
    _lib.check(st)
    return sorted_ids, expert_ids, num_post, offsets, dropped


# ---------------------------------------------------------------------------
# Fused experts (kernels/w4a16_moe.py:678-909)
# ---------------------------------------------------------------------------


def _packed_cols(w: torch.Tensor) -> int:
    """Input elements per row of a packed weight (uint8: 2/byte, int32: 8/word)."""
    if w.dtype == torch.uint8 or w.dtype == torch.int8:
        return w.shape[-1] * 2
    if w.dtype == torch.int32:
        return w.shape[-1] * 8
    _fail(f"packed weights must be uint8 or int32, got {w.dtype}")
    return 0


def _workspace(device: torch.device, M: int, topk: int, E: int, N: int, K: int,
               group: int, tuning: "_tuning.Tuning | None" = None) -> torch.Tensor:
    """The pool's workspace for the current stream, at least this call's size."""
    ts = None if tuning is None else tuning.to_struct()
    nbytes = _lib.workspace_size_ex(M, topk, E, N, K, group, ts)
    stream = _stream_ptr(device)
    cap = _lib.capture_id(stream) if torch.cuda.is_current_stream_capturing() else 0
    return _WS_POOL.get(device, stream, nbytes, capture_id=cap)


class _Prepared:
    __slots__ = ("hidden", "w1_q", "w2_q", "w1_scale", "w2_scale", "topk_weights",
                 "topk_ids", "M", "K", "N", "E", "topk", "group", "device", "tuning")


def _prepare(hidden, w1_q, w2_q, w1_scale, w2_scale, topk_weights, topk_ids,
             group_size) -> _Prepared:
    """The reference's argument checks (kernels/w4a16_moe.py:716-750)."""
    if not (hidden.is_cuda and hidden.ndim == 2):
        _fail("hidden must be a 2-D GPU tensor")
    if not (topk_ids.is_cuda and topk_weights.is_cuda):
        _fail("topk_ids and topk_weights must be on the GPU")
    if topk_ids.shape != topk_weights.shape or topk_ids.ndim != 2:
        _fail("topk_ids and topk_weights must both be [M, topk]")
    if hidden.dtype != torch.bfloat16:
        _fail("bf16 activations required")
    if is_repacked(w1_q) or is_repacked(w2_q):
        _fail("4-D repacked weights are not accepted; pass the stock "
              "(E, N_out, K_packed) pack-quantized tensors")
    if w1_q.ndim != 3 or w2_q.ndim != 3 or w1_scale.ndim != 3 or w2_scale.ndim != 3:
        _fail("weights and scales must be 3-D")
    for t in (w1_q, w2_q, w1_scale, w2_scale):
        if not t.is_cuda or t.device != hidden.device:
            _fail("weights must be on the same GPU as hidden")
        if not t.is_contiguous():
            _fail("weights and scales must be contiguous")
    if w1_scale.dtype != torch.bfloat16 or w2_scale.dtype != torch.bfloat16:
        _fail("scales must be bf16")
    p = _Prepared()
    p.M, p.K = hidden.shape
    p.topk = int(topk_ids.shape[1])
    p.E = int(w1_q.shape[0])
    twoN = int(w1_q.shape[1])
    if twoN % 2:
        _fail("w13 must have an even number of rows (gate then up)")
    p.N = twoN // 2
    if _packed_cols(w1_q) != p.K:
        _fail(f"K mismatch: packed {_packed_cols(w1_q)} vs hidden {p.K}")
    if tuple(w2_q.shape[:2]) != (p.E, p.K) or _packed_cols(w2_q) != p.N:
        _fail("w2 must be (E, K, N packed)")
    g = int(group_size)
    if g <= 0 or p.K % g or p.N % g:
        _fail("group_size must divide K and N")
    if tuple(w1_scale.shape) != (p.E, twoN, p.K // g):
        _fail("w13 scale must be (E, 2N, K/group)")
    if tuple(w2_scale.shape) != (p.E, p.K, p.N // g):
        _fail("w2 scale must be (E, K, N/group)")
    p.group = g
    p.device = hidden.device
    if hidden.stride(1) != 1 or hidden.stride(0) % 8 or hidden.data_ptr() % 16:
        hidden = hidden.contiguous()
    p.hidden = hidden
    p.w1_q, p.w2_q, p.w1_scale, p.w2_scale = w1_q, w2_q, w1_scale, w2_scale
    tw = topk_weights
    if tw.dtype != torch.float32:
        tw = tw.to(torch.float32)
    p.topk_weights = tw.contiguous()
    p.topk_ids = _ids_i32(topk_ids)
    p.tuning = None
    return p


def _tuning_for(p: _Prepared, tuning) -> None:
    """Explicit tuning, else the device table's entry for M, else built-in."""
    if tuning is None:
        tuning = _tuning.select(p.M, p.E, p.N, p.K, p.group, p.device)
    elif not isinstance(tuning, _tuning.Tuning):
        _fail("tuning must be a tuning.Tuning")
    p.tuning = tuning


def _tuning_ptr(p: _Prepared):
    return None if p.tuning is None else ctypes.byref(p.tuning.to_struct())


def _fused_args(p: _Prepared, out: torch.Tensor, ws: torch.Tensor):
    return (p.hidden.data_ptr(), p.hidden.stride(0), p.w1_q.data_ptr(), p.w2_q.data_ptr(),
            p.w1_scale.data_ptr(), p.w2_scale.data_ptr(), p.topk_weights.data_ptr(),
            p.topk_ids.data_ptr(), p.M, p.topk, p.E, p.N, p.K, p.group,
            out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(),
            _stream_ptr(p.device))


def fused_experts_w4a16(
    hidden: torch.Tensor,
    w1_q: torch.Tensor,
    w2_q: torch.Tensor,
    w1_scale: torch.Tensor,
    w2_scale: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    group_size: int = _GROUP_SIZE_DEFAULT,
    *,
    block_m: int = BLOCK_M,
    block_n: int = BLOCK_N,
    block_k: int = BLOCK_K,
    tuning: "_tuning.Tuning | None" = None,
) -> torch.Tensor:
    """Fused W4A16 grouped-MoE experts (w13 + SiLU-mul + w2 + top-k sum).

    Reference: fused_experts_w4a16, kernels/w4a16_moe.py:678-909, same
    positional arguments:

    hidden        [M, K] bf16 activations.
    w1_q, w1_scale  (E, 2N, K/2) uint8 or (E, 2N, K/8) int32 pack-quantized
                    w13 (rows 0..N-1 gate, N..2N-1 up) and (E, 2N, K/group) bf16.
    w2_q, w2_scale  (E, K, N/2) uint8 or (E, K, N/8) int32, (E, K, N/group) bf16.
    topk_weights  [M, topk] routing weights (fp32; other float dtypes are cast).
    topk_ids      [M, topk] expert ids (int32; int64 is cast).
    group_size    symmetric int4 group size along the reduction axis (32/64/128).
    block_m, block_n, block_k: accepted for compatibility, not used.
    tuning        dispatch choices (tuning.Tuning); default: the device's tuned
                  table entry nearest to M if a table exists, else the
                  library's built-in choices.

    Returns a new [M, K] bf16 tensor.  All work is enqueued on the current
    stream with no host synchronisation (HIP-graph capturable once the
    per-shape workspace exists).
    """
    del block_m, block_n, block_k
    p = _prepare(hidden, w1_q, w2_q, w1_scale, w2_scale, topk_weights, topk_ids,
                 group_size)
    out = torch.empty((p.M, p.K), dtype=torch.bfloat16, device=p.device)
    if p.M == 0:
        return out
    _tuning_for(p, tuning)
    ws = _workspace(p.device, p.M, p.topk, p.E, p.N, p.K, p.group, p.tuning)
    with torch.cuda.device(p.device):
        st = _lib.lib().w4a16_moe_fused_experts_ex(*_fused_args(p, out, ws), _tuning_ptr(p))
    _lib.check(st)
    return out


def fused_experts_w4a16_profiled(hidden, w1_q, w2_q, w1_scale, w2_scale, topk_weights,
                                 topk_ids, group_size: int = _GROUP_SIZE_DEFAULT):
    """Run once with HIP events between stages (synchronises).

    Returns (out, {"align": ms, "w13": ms, "w2": ms, "combine": ms}).
    Measurement helper; no counterpart in the reference.
    """
    p = _prepare(hidden, w1_q, w2_q, w1_scale, w2_scale, topk_weights, topk_ids,
                 group_size)
    out = torch.empty((p.M, p.K), dtype=torch.bfloat16, device=p.device)
    ms = (ctypes.c_float * 4)()
    if p.M == 0:
        return out, dict.fromkeys(("align", "w13", "w2", "combine"), 0.0)
    ws = _workspace(p.device, p.M, p.topk, p.E, p.N, p.K, p.group)
    with torch.cuda.device(p.device):
        st = _lib.lib().w4a16_moe_fused_experts_profiled(*_fused_args(p, out, ws), ms)
    _lib.check(st)
    return out, {"align": ms[0], "w13": ms[1], "w2": ms[2], "combine": ms[3]}


def workspace_tensor(hidden: torch.Tensor, topk_ids: torch.Tensor, w1_q: torch.Tensor,
                     w2_q: torch.Tensor, group_size: int = _GROUP_SIZE_DEFAULT,
                     tuning: "_tuning.Tuning | None" = None):
    """The workspace fused_experts_w4a16 uses for this shape on the current
    stream (and tuning, chosen as that call chooses it), with the field
    offsets of that call's layout."""
    M, K = hidden.shape
    topk = topk_ids.shape[1]
    E = w1_q.shape[0]
    N = w1_q.shape[1] // 2
    if tuning is None:
        tuning = _tuning.select(M, E, N, K, group_size, hidden.device)
    ws = _workspace(hidden.device, M, topk, E, N, K, group_size, tuning)
    ts = None if tuning is None else tuning.to_struct()
    return ws, _lib.workspace_layout_ex(M, topk, E, N, K, group_size, ts)


def dropped_pairs(hidden: torch.Tensor, topk_ids: torch.Tensor, w1_q: torch.Tensor,
                  w2_q: torch.Tensor, group_size: int = _GROUP_SIZE_DEFAULT) -> int:
    """Out-of-range pairs skipped by the last fused call of this shape (syncs)."""
    ws, _ = workspace_tensor(hidden, topk_ids, w1_q, w2_q, group_size)
    cnt = ctypes.c_int32()
    with torch.cuda.device(hidden.device):
        st = _lib.lib().w4a16_moe_dropped_pairs(ws.data_ptr(), ctypes.byref(cnt),
                                                _stream_ptr(hidden.device))
    _lib.check(st)
    return cnt.value
