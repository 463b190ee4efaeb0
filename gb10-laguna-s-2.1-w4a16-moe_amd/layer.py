"""One MoE layer outside vLLM: router step + fused W4A16 experts.

The two launches the reference's serving path makes per MoE layer -- routing
(torch.topk + softmax, bench/bench_moe.py:225-230) and fused_experts_w4a16
(kernels/w4a16_moe.py:678-909) -- over weights read by the checkpoint adapter.
"""

from __future__ import annotations

import torch

from .checkpoint import GATE_UP_DOWN, MoELayerWeights, load_moe_layer
from .routing import router_topk_softmax
from .w4a16_moe import fused_experts_w4a16


class W4A16MoELayer:
    def __init__(self, weights: MoELayerWeights, topk: int, renormalize: bool = True):
        self.weights = weights
        self.topk = int(topk)
        self.renormalize = bool(renormalize)

    @classmethod
    def from_checkpoint(cls, source, prefix: str, topk: int, renormalize: bool = True,
                        device="cuda", names=GATE_UP_DOWN) -> "W4A16MoELayer":
        return cls(load_moe_layer(source, prefix, device=device, names=names), topk,
                   renormalize)

    def route(self, router_logits: torch.Tensor):
        return router_topk_softmax(router_logits, self.topk, self.renormalize)

    def __call__(self, hidden: torch.Tensor, router_logits: torch.Tensor) -> torch.Tensor:
        w = self.weights
        topk_weights, topk_ids = self.route(router_logits)
        return fused_experts_w4a16(hidden, w.w13, w.w2, w.s13, w.s2, topk_weights, topk_ids,
                                   w.group_size)
