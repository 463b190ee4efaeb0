"""vLLM-style integration: bind the W4A16 path into a compressed-tensors WNA16
MoE method and route its ``apply()`` here.

The reference patches vLLM's source files on disk (integration/apply.py):
after loading, ``process_weights_after_loading`` binds repacked weights and
``fused_experts_w4a16`` onto the layer (:91-141); ``apply()`` then calls it with
the top-k tensors it already has when the environment variable
``GB10_W4A16_CUSTOM`` is "1", and falls through to the stock kernel otherwise
(:149-169).  Here the same two hooks are installed in-process by wrapping the
method class, and removed again by ``uninstall``:

* the weights stay in the stock pack-quantized layout, so binding is a
  reference to the tensors vLLM already holds -- nothing is repacked and
  nothing needs freeing;
* the environment variable, the bound attribute names and the fall-through
  rule are the reference's, so an operator's configuration carries over.
"""

from __future__ import annotations

import functools
import inspect
import os

from . import _lib
from .w4a16_moe import fused_experts_w4a16, repack_weights

ENV_FLAG = "GB10_W4A16_CUSTOM"
_MARK = "_w4a16_amd_original_methods"


def custom_enabled() -> bool:
    """The reference's switch: env GB10_W4A16_CUSTOM == "1"
    (integration/apply.py:98, :155)."""
    return os.environ.get(ENV_FLAG) == "1"


def bind_layer(layer, group_size: int) -> None:
    """Bind the fused entry and its weights on ``layer``.

    Reference: the process_weights_after_loading insert,
    integration/apply.py:91-141.  ``layer`` carries vLLM's post-load tensors
    ``w13_weight_packed`` (E, 2N, K/2) uint8 (or (E, 2N, K/8) int32),
    ``w13_weight_scale`` (E, 2N, K/group) and the w2 pair; they are bound as
    they are (repack_weights is the identity for this path).
    """
    w1q, w1s = repack_weights(layer.w13_weight_packed.data, layer.w13_weight_scale.data)
    w2q, w2s = repack_weights(layer.w2_weight_packed.data, layer.w2_weight_scale.data)
    g = int(group_size)
    if g not in (32, 64, 128):
        raise _lib.W4A16Error(f"group_size {g} not supported (32, 64 or 128)")
    layer._gb10_w1_q = w1q
    layer._gb10_w1_scale = w1s
    layer._gb10_w2_q = w2q
    layer._gb10_w2_scale = w2s
    layer._gb10_group_size = g
    layer._gb10_fused = fused_experts_w4a16


def apply(layer, x, topk_weights, topk_ids, stock=None, *stock_args, **stock_kwargs):
    """The apply() insert, integration/apply.py:149-169.

    With the flag set and the layer bound, returns
    ``fused_experts_w4a16(x, w1_q, w2_q, w1_scale, w2_scale, topk_weights,
    topk_ids, group_size=...)``; otherwise calls ``stock(*stock_args,
    **stock_kwargs)`` (the stock fused_experts path).
    """
    fn = getattr(layer, "_gb10_fused", None)
    if fn is not None and custom_enabled():
        return fn(x, layer._gb10_w1_q, layer._gb10_w2_q, layer._gb10_w1_scale,
                  layer._gb10_w2_scale, topk_weights, topk_ids,
                  group_size=layer._gb10_group_size)
    if stock is None:
        raise RuntimeError("W4A16 path not bound (or disabled) and no stock path given")
    return stock(*stock_args, **stock_kwargs)


def install(method_cls) -> None:
    """Wrap ``method_cls.process_weights_after_loading`` and ``.apply``.

    ``method_cls`` is a vLLM-style MoE quantization method (the reference
    targets CompressedTensorsWNA16MoEMethod): ``process_weights_after_loading
    (self, layer)`` and an ``apply`` whose parameters include ``layer``, ``x``,
    ``topk_weights`` and ``topk_ids`` (bound by name, so positional and
    keyword callers both work).  ``self.group_size`` gives the group, as in the
    reference (:114).  Installing twice is a no-op.
    """
    if _MARK in method_cls.__dict__:
        return
    orig_process = method_cls.process_weights_after_loading
    orig_apply = method_cls.apply
    sig = inspect.signature(orig_apply)
    for need in ("layer", "x", "topk_weights", "topk_ids"):
        if need not in sig.parameters:
            raise TypeError(f"{method_cls.__name__}.apply has no parameter {need!r}")

    @functools.wraps(orig_process)
    def process_weights_after_loading(self, layer, *a, **kw):
        r = orig_process(self, layer, *a, **kw)
        if custom_enabled():
            bind_layer(layer, self.group_size)
        return r

    @functools.wraps(orig_apply)
    def apply_wrapped(self, *a, **kw):
        b = sig.bind(self, *a, **kw)
        layer = b.arguments["layer"]
        fn = getattr(layer, "_gb10_fused", None)
        if fn is not None and custom_enabled():
            return fn(b.arguments["x"], layer._gb10_w1_q, layer._gb10_w2_q,
                      layer._gb10_w1_scale, layer._gb10_w2_scale,
                      b.arguments["topk_weights"], b.arguments["topk_ids"],
                      group_size=layer._gb10_group_size)
        return orig_apply(self, *a, **kw)

    setattr(method_cls, _MARK, (orig_process, orig_apply))
    method_cls.process_weights_after_loading = process_weights_after_loading
    method_cls.apply = apply_wrapped


def uninstall(method_cls) -> None:
    """Restore the methods ``install`` wrapped (the reference's --revert)."""
    orig = method_cls.__dict__.get(_MARK)
    if orig is None:
        return
    method_cls.process_weights_after_loading, method_cls.apply = orig
    delattr(method_cls, _MARK)


_VLLM_MODULES = (  # where the reference finds the class (integration/apply.py:199-210)
    "vllm.model_executor.layers.quantization.compressed_tensors."
    "compressed_tensors_moe.compressed_tensors_moe_wna16",
    "vllm.model_executor.layers.quantization.compressed_tensors.compressed_tensors_moe_wna16",
    "vllm.model_executor.layers.quantization.compressed_tensors.compressed_tensors_moe",
)


def install_into_vllm():
    """Install into the running vLLM's CompressedTensorsWNA16MoEMethod and
    return the class.  Raises ImportError when vLLM or the class is absent."""
    import importlib

    for name in _VLLM_MODULES:
        try:
            mod = importlib.import_module(name)
        except ImportError:
            continue
        cls = getattr(mod, "CompressedTensorsWNA16MoEMethod", None)
        if cls is not None:
            install(cls)
            return cls
    raise ImportError("vLLM's CompressedTensorsWNA16MoEMethod is not importable here")
