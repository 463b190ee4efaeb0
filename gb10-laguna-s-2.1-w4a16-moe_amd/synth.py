"""Seeded synthetic inputs for the benchmark configurations.

Distributions (one MoE layer of the Laguna-S-2.1 shape by default):
  * int4 codes uniform in [0, 15] (value = code - 8), i.e. uniform packed bytes;
  * bf16 scales uniform in [0.005, 0.02], one per 32 input elements;
  * hidden states bf16 N(0, 1);
  * router logits fp32 N(0, 1) [M, E], plus, for skewed routing, a per-expert
    bias drawn once from N(0, 1.5**2); topk_ids = top-k indices (int32),
    topk_weights = softmax over the k selected logits (fp32), as in
    bench/bench_moe.py:210-231.

Sub-seeds follow the reference's scheme (bench/bench_moe.py:179, :223, :241):
weights ``seed``, hidden ``seed + 1000 + M``, routing ``seed + 17000 + M``,
skew bias ``seed + 29000``.  Tensors are generated with a torch.Generator on
the target device, so CPU and GPU draws differ; every check compares outputs
computed from the same tensors.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

E_DEFAULT = 256
TOPK_DEFAULT = 10
K_DEFAULT = 3072  # hidden size
N_DEFAULT = 1024  # intermediate size
GROUP_DEFAULT = 32
SKEW_STD = 1.5


@dataclass(frozen=True)
class LayerShape:
    E: int = E_DEFAULT
    topk: int = TOPK_DEFAULT
    K: int = K_DEFAULT
    N: int = N_DEFAULT
    group: int = GROUP_DEFAULT

    @property
    def bytes_per_expert(self) -> int:
        """Packed weight + scale bytes of one expert (w13 + s13 + w2 + s2)."""
        w13 = 2 * self.N * self.K // 2
        w2 = self.K * self.N // 2
        s13 = 2 * self.N * (self.K // self.group) * 2
        s2 = self.K * (self.N // self.group) * 2
        return w13 + w2 + s13 + s2

    @property
    def w13_bytes_per_expert(self) -> int:
        return 2 * self.N * self.K // 2 + 2 * self.N * (self.K // self.group) * 2

    @property
    def w2_bytes_per_expert(self) -> int:
        return self.K * self.N // 2 + self.K * (self.N // self.group) * 2

    def flops(self, M: int) -> int:
        """2*M*topk*(2*N*K + K*N): the algorithmic FLOPs of one call."""
        return 2 * M * self.topk * (2 * self.N * self.K + self.K * self.N)


@dataclass(frozen=True)
class BenchConfig:
    index: int
    M: int
    skewed: bool
    description: str


# The five configurations of the benchmark (BASELINE.json "configs").
CONFIGS = (
    BenchConfig(0, 1, False, "M=1 decode, uniform routing"),
    BenchConfig(1, 16, False, "M=16 decode, uniform routing"),
    BenchConfig(2, 64, True, "M=64, skewed routing (per-expert bias std 1.5)"),
    BenchConfig(3, 1024, False, "M=1024 chunked prefill, uniform routing"),
    BenchConfig(4, 4096, False, "M=4096 prefill, uniform routing"),
)


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=torch.device(device))
    g.manual_seed(seed)
    return g


def make_weights(shape: LayerShape, device, seed: int = 0, dtype_packed=torch.int32):
    """Packed pack-quantized weights and bf16 scales.

    Returns (w13 [E, 2N, K/8] int32, w2 [E, K, N/8] int32,
             s13 [E, 2N, K/G] bf16, s2 [E, K, N/G] bf16).
    With dtype_packed=torch.uint8 the packed tensors are [E, rows, cols/2].
    """
    E, K, N, G = shape.E, shape.K, shape.N, shape.group
    g = _gen(device, seed)
    w13 = torch.randint(0, 256, (E, 2 * N, K // 2), generator=g, device=device,
                        dtype=torch.uint8)
    w2 = torch.randint(0, 256, (E, K, N // 2), generator=g, device=device,
                       dtype=torch.uint8)
    s13 = (torch.rand((E, 2 * N, K // G), generator=g, device=device) * 0.015 + 0.005
           ).to(torch.bfloat16)
    s2 = (torch.rand((E, K, N // G), generator=g, device=device) * 0.015 + 0.005
          ).to(torch.bfloat16)
    if dtype_packed == torch.int32:
        w13 = w13.view(torch.int32)
        w2 = w2.view(torch.int32)
    return w13, w2, s13, s2


def make_hidden(M: int, K: int, device, seed: int = 0, scale: float = 1.0) -> torch.Tensor:
    g = _gen(device, seed + 1000 + M)
    return (torch.randn((M, K), generator=g, device=device) * scale).to(torch.bfloat16)


def make_routing(M: int, E: int, topk: int, device, seed: int = 0, skewed: bool = False,
                 bias_seed: int | None = None):
    """(topk_weights fp32 [M, topk], topk_ids int32 [M, topk]).

    bias_seed fixes the skew bias independently of the logits' seed (default:
    the same seed).
    """
    g = _gen(device, seed + 17000 + M)
    logits = torch.randn((M, E), generator=g, device=device, dtype=torch.float32)
    if skewed:
        gb = _gen(device, (seed if bias_seed is None else bias_seed) + 29000)
        bias = torch.randn((E,), generator=gb, device=device, dtype=torch.float32) * SKEW_STD
        logits = logits + bias
    vals, ids = torch.topk(logits, k=topk, dim=-1)
    weights = torch.softmax(vals, dim=-1)
    return weights.contiguous(), ids.to(torch.int32).contiguous()


def touched_experts(topk_ids: torch.Tensor, E: int) -> int:
    ids = topk_ids.reshape(-1)
    ids = ids[(ids >= 0) & (ids < E)]
    return int(torch.unique(ids).numel())
