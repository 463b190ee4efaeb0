"""Checkpoint adapter: compressed-tensors ``pack-quantized`` MoE experts ->
the tensors ``fused_experts_w4a16`` consumes, unchanged.

A compressed-tensors W4A16 checkpoint stores every routed expert projection as
three tensors (integration/apply.py:29-42, tasks/TASK-01-microbench.md:8-14):

    {prefix}.experts.{e}.{proj}.weight_packed  int32 [out, in/8]
        element k of a row is nibble k % 8 of word k / 8, value = code - 8
    {prefix}.experts.{e}.{proj}.weight_scale   bf16  [out, in/group]
    {prefix}.experts.{e}.{proj}.weight_shape   int   [2] = (out, in)

with proj = gate_proj and up_proj (out = N, in = K) and down_proj (out = K,
in = N).  vLLM stores them transposed at load and transposes them back after
loading, ending at exactly the stacked per-expert layout (E, out, in/8)
(integration/apply.py:29-42); this adapter builds that layout straight from
the files:

    w13 [E, 2N, K/8] int32   rows 0..N-1 gate, N..2N-1 up
                             (the split of kernels/w4a16_moe.py:430-431)
    s13 [E, 2N, K/group] bf16
    w2  [E, K, N/8] int32,   s2 [E, K, N/group] bf16

No value is changed on the way: the packed words and the scale bits are
copied as stored.  ``save_moe_layer`` writes the same format (for exports and
tests).

``W4A16MoELayer`` is one MoE layer over such weights outside vLLM: the two
launches the reference's serving path makes per layer -- routing (torch.topk
+ softmax, bench/bench_moe.py:225-230) and fused_experts_w4a16
(kernels/w4a16_moe.py:678-909).
"""

from __future__ import annotations

import json
import re
from dataclasses import dataclass
from pathlib import Path

import torch

from . import _lib
from .routing import router_topk_softmax
from .w4a16_moe import fused_experts_w4a16

GATE_UP_DOWN = ("gate_proj", "up_proj", "down_proj")  # HF / vLLM default names
W1_W3_W2 = ("w1", "w3", "w2")                          # Mixtral-style names
SUPPORTED_GROUPS = (32, 64, 128)


class CheckpointError(_lib.W4A16Error):
    """The checkpoint is not a W4A16 pack-quantized MoE this path accepts."""


@dataclass
class MoELayerWeights:
    """One MoE layer's routed experts in the layout fused_experts_w4a16 reads."""

    w13: torch.Tensor
    w2: torch.Tensor
    s13: torch.Tensor
    s2: torch.Tensor
    group_size: int

    @property
    def num_experts(self) -> int:
        return self.w13.shape[0]

    @property
    def intermediate_size(self) -> int:  # N
        return self.w13.shape[1] // 2

    @property
    def hidden_size(self) -> int:  # K
        return self.w2.shape[1]


# ---------------------------------------------------------------------------
# quantization_config (config.json)
# ---------------------------------------------------------------------------


def quantization_config(group_size: int = 32) -> dict:
    """The compressed-tensors ``quantization_config`` block of a W4A16 group
    checkpoint (symmetric int4, group along the input axis, pack-quantized)."""
    return {
        "quant_method": "compressed-tensors",
        "format": "pack-quantized",
        "config_groups": {
            "group_0": {
                "targets": ["Linear"],
                "weights": {"num_bits": 4, "type": "int", "symmetric": True,
                            "strategy": "group", "group_size": int(group_size),
                            "actorder": None, "dynamic": False},
                "input_activations": None,
                "output_activations": None,
                "format": "pack-quantized",
            }
        },
    }


def check_quantization_config(qc: dict) -> int:
    """Validate a compressed-tensors quantization_config; return its group size.

    Accepts only what the kernels compute: 4-bit symmetric integer weights,
    one scale per group along the input axis, pack-quantized storage, no
    activation reordering and no quantized activations.
    """
    if qc.get("quant_method", "compressed-tensors") != "compressed-tensors":
        raise CheckpointError(f"quant_method {qc.get('quant_method')!r} is not compressed-tensors")
    groups = qc.get("config_groups") or {}
    if not groups:
        raise CheckpointError("quantization_config has no config_groups")
    sizes = set()
    for name, grp in groups.items():
        fmt = grp.get("format", qc.get("format"))
        if fmt != "pack-quantized":
            raise CheckpointError(f"{name}: format {fmt!r}, need pack-quantized")
        w = grp.get("weights") or {}
        if w.get("num_bits") != 4 or w.get("type", "int") != "int":
            raise CheckpointError(f"{name}: weights must be 4-bit int")
        if not w.get("symmetric", False):
            raise CheckpointError(f"{name}: asymmetric (zero-point) weights are not supported")
        if w.get("strategy") != "group":
            raise CheckpointError(f"{name}: strategy {w.get('strategy')!r}, need group")
        if w.get("actorder") not in (None, False, "none"):
            raise CheckpointError(f"{name}: activation reordering is not supported")
        if grp.get("input_activations"):
            raise CheckpointError(f"{name}: quantized activations are not W4A16")
        sizes.add(int(w.get("group_size", 0)))
    if len(sizes) != 1 or next(iter(sizes)) not in SUPPORTED_GROUPS:
        raise CheckpointError(f"group sizes {sorted(sizes)} not one of {SUPPORTED_GROUPS}")
    return next(iter(sizes))


# ---------------------------------------------------------------------------
# tensor index over one or more .safetensors files
# ---------------------------------------------------------------------------


class _Index:
    """name -> file over a checkpoint directory or file list; opens lazily."""

    def __init__(self, source):
        from safetensors import safe_open

        self._safe_open = safe_open
        paths: list[Path]
        src = Path(source) if isinstance(source, (str, Path)) else None
        self.config: dict | None = None
        if src is not None and src.is_dir():
            cfg = src / "config.json"
            if cfg.exists():
                self.config = json.loads(cfg.read_text())
            idx = src / "model.safetensors.index.json"
            if idx.exists():
                wm = json.loads(idx.read_text())["weight_map"]
                self.where = {k: src / v for k, v in wm.items()}
                self._handles: dict[Path, object] = {}
                return
            paths = sorted(src.glob("*.safetensors"))
        elif src is not None:
            paths = [src]
        else:
            paths = [Path(p) for p in source]
        if not paths:
            raise CheckpointError(f"no .safetensors files in {source}")
        self.where = {}
        self._handles = {}
        for p in paths:
            h = self._open(p)
            for k in h.keys():
                self.where[k] = p

    def _open(self, p: Path):
        h = self._handles.get(p)
        if h is None:
            h = self._safe_open(str(p), framework="pt", device="cpu")
            self._handles[p] = h
        return h

    def __contains__(self, name: str) -> bool:
        return name in self.where

    def get(self, name: str) -> torch.Tensor:
        p = self.where.get(name)
        if p is None:
            raise CheckpointError(f"tensor {name} not found in the checkpoint")
        return self._open(p).get_tensor(name)


def list_moe_layers(source, names=GATE_UP_DOWN) -> list[str]:
    """Prefixes of every layer holding routed experts in pack-quantized form."""
    idx = _Index(source)
    pat = re.compile(r"^(.*)\.experts\.0\." + re.escape(names[0]) + r"\.weight_packed$")
    found = [m.group(1) for k in idx.where if (m := pat.match(k))]

    def order(p):
        nums = [int(t) for t in re.findall(r"\d+", p)]
        return (nums, p)

    return sorted(found, key=order)


def _count_experts(idx: _Index, prefix: str, proj: str) -> int:
    pat = re.compile(r"^" + re.escape(prefix) + r"\.experts\.(\d+)\." + re.escape(proj)
                     + r"\.weight_packed$")
    ids = {int(m.group(1)) for k in idx.where if (m := pat.match(k))}
    if not ids:
        raise CheckpointError(f"no experts under {prefix}")
    E = max(ids) + 1
    missing = sorted(set(range(E)) - ids)
    if missing:
        raise CheckpointError(f"{prefix}: experts {missing[:8]} missing")
    return E


def _proj(idx: _Index, prefix: str, e: int, proj: str, group: int | None):
    base = f"{prefix}.experts.{e}.{proj}"
    if f"{base}.weight_zero_point" in idx:
        raise CheckpointError(f"{base}: zero points present (asymmetric); not supported")
    if f"{base}.weight_g_idx" in idx:
        raise CheckpointError(f"{base}: activation-order g_idx present; not supported")
    packed = idx.get(f"{base}.weight_packed")
    scale = idx.get(f"{base}.weight_scale")
    if packed.dtype != torch.int32 or packed.dim() != 2:
        raise CheckpointError(f"{base}.weight_packed must be a 2-D int32 tensor")
    out_f, words = packed.shape
    in_f = words * 8
    if f"{base}.weight_shape" in idx:
        shp = [int(v) for v in idx.get(f"{base}.weight_shape").reshape(-1).tolist()]
        if shp != [out_f, in_f]:
            raise CheckpointError(f"{base}: weight_shape {shp} != packed {[out_f, in_f]}")
    if scale.dim() != 2 or scale.shape[0] != out_f or scale.shape[1] == 0:
        raise CheckpointError(f"{base}.weight_scale shape {tuple(scale.shape)} does not match")
    g = in_f // scale.shape[1]
    if g * scale.shape[1] != in_f or (group is not None and g != group):
        raise CheckpointError(f"{base}: scale columns {scale.shape[1]} do not give group "
                              f"{group if group is not None else '32/64/128'}")
    if scale.dtype != torch.bfloat16:
        raise CheckpointError(f"{base}.weight_scale is {scale.dtype}, need bfloat16")
    return packed, scale, g


def load_moe_layer(source, prefix: str, *, device="cuda", names=GATE_UP_DOWN,
                   group_size: int | None = None) -> MoELayerWeights:
    """Read one layer's routed experts from a compressed-tensors checkpoint.

    source      a checkpoint directory (config.json + *.safetensors, sharded
                or not), one .safetensors file, or a list of files.
    prefix      the layer's module path, e.g. "model.layers.3.mlp".
    names       the (gate, up, down) projection names of the checkpoint.
    group_size  expected group; default: config.json's, else the scales'.
    """
    idx = _Index(source)
    if idx.config is not None and "quantization_config" in idx.config:
        cfg_group = check_quantization_config(idx.config["quantization_config"])
        if group_size is not None and group_size != cfg_group:
            raise CheckpointError(f"group_size {group_size} != config.json's {cfg_group}")
        group_size = cfg_group
    gate, up, down = names
    E = _count_experts(idx, prefix, gate)
    for p in (up, down):
        if _count_experts(idx, prefix, p) != E:
            raise CheckpointError(f"{prefix}: {p} has a different expert count than {gate}")

    g0, s0, grp = _proj(idx, prefix, 0, gate, group_size)
    if grp not in SUPPORTED_GROUPS:
        raise CheckpointError(f"group {grp} not one of {SUPPORTED_GROUPS}")
    N, K = g0.shape[0], g0.shape[1] * 8
    w13 = torch.empty((E, 2 * N, K // 8), dtype=torch.int32)
    s13 = torch.empty((E, 2 * N, K // grp), dtype=torch.bfloat16)
    w2 = torch.empty((E, K, N // 8), dtype=torch.int32)
    s2 = torch.empty((E, K, N // grp), dtype=torch.bfloat16)
    for e in range(E):
        for proj, rows in ((gate, slice(0, N)), (up, slice(N, 2 * N))):
            pk, sc, _ = _proj(idx, prefix, e, proj, grp)
            if tuple(pk.shape) != (N, K // 8):
                raise CheckpointError(f"{prefix}.experts.{e}.{proj}: shape {tuple(pk.shape)}, "
                                      f"expected {(N, K // 8)}")
            w13[e, rows] = pk
            s13[e, rows] = sc
        pk, sc, _ = _proj(idx, prefix, e, down, grp)
        if tuple(pk.shape) != (K, N // 8):
            raise CheckpointError(f"{prefix}.experts.{e}.{down}: shape {tuple(pk.shape)}, "
                                  f"expected {(K, N // 8)}")
        w2[e] = pk
        s2[e] = sc
    dev = torch.device(device)
    if dev.type != "cpu":
        w13, w2, s13, s2 = (t.to(dev, non_blocking=False) for t in (w13, w2, s13, s2))
    return MoELayerWeights(w13=w13, w2=w2, s13=s13, s2=s2, group_size=grp)


def save_moe_layer(path, prefix: str, w13: torch.Tensor, w2: torch.Tensor,
                   s13: torch.Tensor, s2: torch.Tensor, *, names=GATE_UP_DOWN,
                   extra: dict[str, torch.Tensor] | None = None) -> Path:
    """Write one layer's experts as compressed-tensors pack-quantized tensors
    (the inverse of load_moe_layer).  Packed weights may be int32 [E, rows,
    cols/8] or uint8 [E, rows, cols/2]."""
    from safetensors.torch import save_file

    w13 = w13.detach().cpu().contiguous()
    w2 = w2.detach().cpu().contiguous()
    if w13.dtype == torch.uint8:
        w13 = w13.view(torch.int32)
    if w2.dtype == torch.uint8:
        w2 = w2.view(torch.int32)
    s13 = s13.detach().cpu().contiguous()
    s2 = s2.detach().cpu().contiguous()
    E, twoN, kw = w13.shape
    N, K = twoN // 2, kw * 8
    gate, up, down = names
    out: dict[str, torch.Tensor] = dict(extra or {})
    for e in range(E):
        for proj, rows, shp in ((gate, slice(0, N), (N, K)), (up, slice(N, twoN), (N, K))):
            base = f"{prefix}.experts.{e}.{proj}"
            out[f"{base}.weight_packed"] = w13[e, rows].clone()
            out[f"{base}.weight_scale"] = s13[e, rows].clone()
            out[f"{base}.weight_shape"] = torch.tensor(shp, dtype=torch.int64)
        base = f"{prefix}.experts.{e}.{down}"
        out[f"{base}.weight_packed"] = w2[e].clone()
        out[f"{base}.weight_scale"] = s2[e].clone()
        out[f"{base}.weight_shape"] = torch.tensor((K, N), dtype=torch.int64)
    p = Path(path)
    save_file(out, str(p))
    return p


class W4A16MoELayer:
    """Router step + fused W4A16 experts over one layer's weights."""

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
