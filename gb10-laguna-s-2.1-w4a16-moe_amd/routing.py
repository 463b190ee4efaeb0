"""Router step in front of the MoE layer: logits -> (topk_weights, topk_ids).

The reference computes routing as ``torch.topk`` then ``torch.softmax`` over
the selected logits (make_routing, bench/bench_moe.py:225-230); vLLM hands the
result to the MoE layer's ``apply()`` (integration/apply.py:149-166).  Here
the same step is one HIP launch (C entry ``w4a16_moe_router_topk_softmax``)
whose outputs feed ``fused_experts_w4a16`` directly: fp32 weights and int32
ids, both contiguous ``[M, topk]``.
"""

from __future__ import annotations

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.LOGITS_F32, torch.bfloat16: _lib.LOGITS_BF16}


def router_topk_softmax(router_logits: torch.Tensor, topk: int, renormalize: bool = True,
                        *, out: tuple[torch.Tensor, torch.Tensor] | None = None):
    """Select each row's ``topk`` experts and their weights.

    router_logits  [M, E] fp32 or bf16 on the GPU (unit stride along E).
    topk           1 <= topk <= min(64, E).
    renormalize    True: softmax over the selected logits (the reference's
                   ``torch.softmax(vals)``); False: the softmax over all E
                   logits, read at the selected experts.
    out            optional preallocated (weights fp32, ids int32) [M, topk].

    Returns ``(topk_weights fp32 [M, topk], topk_ids int32 [M, topk])``; ids
    are ordered by descending logit, equal logits by ascending expert index.
    """
    if router_logits.dim() != 2:
        raise _lib.W4A16Error("router_logits must be [M, E]")
    if router_logits.dtype not in _DTYPES:
        raise _lib.W4A16Error(f"router_logits dtype {router_logits.dtype} not fp32/bf16")
    if not router_logits.is_cuda:
        raise _lib.W4A16Error("router_logits must be a GPU tensor")
    x = router_logits
    if x.stride(1) != 1:
        x = x.contiguous()
    M, E = x.shape
    k = int(topk)
    if out is None:
        weights = torch.empty((M, k), dtype=torch.float32, device=x.device)
        ids = torch.empty((M, k), dtype=torch.int32, device=x.device)
    else:
        weights, ids = out
        if (weights.shape != (M, k) or ids.shape != (M, k) or weights.dtype != torch.float32
                or ids.dtype != torch.int32 or not weights.is_contiguous()
                or not ids.is_contiguous()):
            raise _lib.W4A16Error("out must be contiguous (fp32, int32) tensors of [M, topk]")
    ld = x.stride(0) if M > 1 else E
    _lib.check(_lib.lib().w4a16_moe_router_topk_softmax(
        x.data_ptr(), _DTYPES[x.dtype], ld, M, E, k, 1 if renormalize else 0,
        weights.data_ptr(), ids.data_ptr(), torch.cuda.current_stream(x.device).cuda_stream))
    return weights, ids
