"""Checkpoint adapter (compressed-tensors pack-quantized experts) and the
vLLM-style apply() shim.

The layout pin builds checkpoint tensors from int4 codes with the
compressed-tensors word formula (element 8j+i of a row in bits 4i of word j,
integration/apply.py:29-42) -- independent of the adapter's writer -- and checks
that the loaded tensors dequantize (oracle) to (code - 8) * scale with gate
rows before up rows (kernels/w4a16_moe.py:430-431).
"""

from __future__ import annotations

import json
import types

import numpy as np
import pytest
import torch
from safetensors.torch import save_file


def _words(codes: np.ndarray) -> torch.Tensor:
    """int4 codes [out, in] -> int32 words [out, in/8], element 8j+i in bits 4i."""
    out, inn = codes.shape
    c = codes.reshape(out, inn // 8, 8).astype(np.uint64)
    w = np.zeros((out, inn // 8), dtype=np.uint64)
    for i in range(8):
        w |= c[:, :, i] << np.uint64(4 * i)
    return torch.from_numpy(w.astype(np.uint32).view(np.int32))


def _scales(rng, out, inn, group):
    s = torch.from_numpy(rng.uniform(0.005, 0.02, (out, inn // group)).astype(np.float32))
    return s.to(torch.bfloat16)


def _write_ckpt(path, prefix, E, K, N, group, seed=0, names=("gate_proj", "up_proj", "down_proj"),
                skip=None, extra=None):
    rng = np.random.default_rng(seed)
    tensors, codes = {}, {}
    for e in range(E):
        for proj, (out, inn) in zip(names, ((N, K), (N, K), (K, N))):
            if skip == (e, proj):
                continue
            c = rng.integers(0, 16, (out, inn))
            codes[(e, proj)] = c
            base = f"{prefix}.experts.{e}.{proj}"
            tensors[f"{base}.weight_packed"] = _words(c)
            tensors[f"{base}.weight_scale"] = _scales(rng, out, inn, group)
            tensors[f"{base}.weight_shape"] = torch.tensor([out, inn])
    if extra:
        tensors.update(extra)
    save_file(tensors, str(path))
    return tensors, codes


def test_loaded_layout_dequantizes_to_codes(pkg, orc, tmp_path):
    E, K, N, G = 3, 256, 64, 32
    f = tmp_path / "layer.safetensors"
    t, codes = _write_ckpt(f, "model.layers.0.mlp", E, K, N, G)
    w = pkg.load_moe_layer(f, "model.layers.0.mlp", device="cpu")
    assert w.w13.shape == (E, 2 * N, K // 8) and w.w13.dtype == torch.int32
    assert w.w2.shape == (E, K, N // 8) and w.s2.shape == (E, K, N // G)
    assert w.group_size == G and w.num_experts == E
    assert (w.intermediate_size, w.hidden_size) == (N, K)
    for e in range(E):
        deq13 = orc.dequant(w.w13[e].numpy(), orc._scale_bits(w.s13[e]), G)
        for proj, rows in (("gate_proj", slice(0, N)), ("up_proj", slice(N, 2 * N))):
            sc = t[f"model.layers.0.mlp.experts.{e}.{proj}.weight_scale"].float().numpy()
            want = orc.bf16_round((codes[(e, proj)] - 8) * np.repeat(sc, G, axis=1))
            np.testing.assert_array_equal(deq13[rows], want)
        deq2 = orc.dequant(w.w2[e].numpy(), orc._scale_bits(w.s2[e]), G)
        sc = t[f"model.layers.0.mlp.experts.{e}.down_proj.weight_scale"].float().numpy()
        np.testing.assert_array_equal(
            deq2, orc.bf16_round((codes[(e, "down_proj")] - 8) * np.repeat(sc, G, axis=1)))


def test_word_formula_known_answer():
    # codes 0..7 in one word: nibble i holds i -> 0x76543210
    assert int(_words(np.arange(8)[None, :])[0, 0]) == 0x76543210
    # code 15 in the top nibble is the sign bit of the int32 word
    c = np.zeros((1, 8), dtype=np.int64)
    c[0, 7] = 15
    assert int(_words(c)[0, 0]) == np.int32(np.uint32(0xF0000000).view(np.int32))


def test_save_load_roundtrip(pkg, synth, tmp_path):
    shape = synth.LayerShape(E=4, topk=2, K=256, N=128, group=64)
    w13, w2, s13, s2 = synth.make_weights(shape, "cpu", seed=3)
    f = pkg.save_moe_layer(tmp_path / "x.safetensors", "blk.7.moe", w13, w2, s13, s2)
    w = pkg.load_moe_layer(f, "blk.7.moe", device="cpu")
    for a, b in ((w.w13, w13), (w.w2, w2), (w.s13, s13), (w.s2, s2)):
        assert a.dtype == b.dtype and torch.equal(a, b)
    assert w.group_size == 64
    # uint8 packed input writes the same words
    w13u, w2u, _, _ = synth.make_weights(shape, "cpu", seed=3, dtype_packed=torch.uint8)
    f2 = pkg.save_moe_layer(tmp_path / "y.safetensors", "blk.7.moe", w13u, w2u, s13, s2)
    assert torch.equal(pkg.load_moe_layer(f2, "blk.7.moe", device="cpu").w13, w13)


def test_sharded_directory_with_config(pkg, tmp_path):
    E, K, N, G = 2, 128, 64, 32
    d = tmp_path / "ckpt"
    d.mkdir()
    weight_map = {}
    for li in (10, 2):  # numeric layer order, not lexical
        fname = f"model-{li:05d}.safetensors"
        t, _ = _write_ckpt(d / fname, f"model.layers.{li}.mlp", E, K, N, G, seed=li)
        weight_map.update({k: fname for k in t})
    (d / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    (d / "config.json").write_text(json.dumps(
        {"quantization_config": pkg.checkpoint.quantization_config(G)}))
    assert pkg.list_moe_layers(d) == ["model.layers.2.mlp", "model.layers.10.mlp"]
    w = pkg.load_moe_layer(d, "model.layers.10.mlp", device="cpu")
    assert w.w13.shape == (E, 2 * N, K // 8)
    with pytest.raises(pkg.CheckpointError):
        pkg.load_moe_layer(d, "model.layers.10.mlp", device="cpu", group_size=64)


def test_mixtral_names(pkg, tmp_path):
    f = tmp_path / "m.safetensors"
    _write_ckpt(f, "layers.0.block_sparse_moe", 2, 128, 64, 32, names=("w1", "w3", "w2"))
    w = pkg.load_moe_layer(f, "layers.0.block_sparse_moe", device="cpu",
                           names=pkg.checkpoint.W1_W3_W2)
    assert w.w2.shape == (2, 128, 8)


@pytest.mark.parametrize("change,match", [
    ({"num_bits": 8}, "4-bit"),
    ({"symmetric": False}, "asymmetric"),
    ({"strategy": "channel"}, "strategy"),
    ({"group_size": 16}, "group sizes"),
    ({"actorder": "group"}, "reordering"),
])
def test_quantization_config_rejects(pkg, change, match):
    qc = pkg.checkpoint.quantization_config(32)
    qc["config_groups"]["group_0"]["weights"].update(change)
    with pytest.raises(pkg.CheckpointError, match=match):
        pkg.checkpoint.check_quantization_config(qc)


def test_quantization_config_rejects_format_and_activations(pkg):
    qc = pkg.checkpoint.quantization_config(32)
    qc["config_groups"]["group_0"]["format"] = "float-quantized"
    with pytest.raises(pkg.CheckpointError, match="pack-quantized"):
        pkg.checkpoint.check_quantization_config(qc)
    qc = pkg.checkpoint.quantization_config(32)
    qc["config_groups"]["group_0"]["input_activations"] = {"num_bits": 8}
    with pytest.raises(pkg.CheckpointError, match="W4A16"):
        pkg.checkpoint.check_quantization_config(qc)
    assert pkg.checkpoint.check_quantization_config(pkg.checkpoint.quantization_config(128)) == 128


def test_checkpoint_errors(pkg, tmp_path):
    p = "m"
    f = tmp_path / "a.safetensors"
    _write_ckpt(f, p, 3, 128, 64, 32, skip=(1, "up_proj"))
    with pytest.raises(pkg.CheckpointError, match="missing|different expert count"):
        pkg.load_moe_layer(f, p, device="cpu")
    f = tmp_path / "b.safetensors"
    _write_ckpt(f, p, 3, 128, 64, 32, skip=(1, "gate_proj"))
    with pytest.raises(pkg.CheckpointError, match="missing"):
        pkg.load_moe_layer(f, p, device="cpu")
    f = tmp_path / "c.safetensors"
    _write_ckpt(f, p, 1, 128, 64, 32,
                extra={f"{p}.experts.0.gate_proj.weight_zero_point": torch.zeros(64, 4)})
    with pytest.raises(pkg.CheckpointError, match="zero points"):
        pkg.load_moe_layer(f, p, device="cpu")
    f = tmp_path / "d.safetensors"
    _write_ckpt(f, p, 1, 128, 64, 32,
                extra={f"{p}.experts.0.up_proj.weight_g_idx": torch.zeros(128, dtype=torch.int32)})
    with pytest.raises(pkg.CheckpointError, match="g_idx"):
        pkg.load_moe_layer(f, p, device="cpu")
    f = tmp_path / "e.safetensors"
    _write_ckpt(f, p, 1, 128, 64, 32,
                extra={f"{p}.experts.0.down_proj.weight_shape": torch.tensor([128, 72])})
    with pytest.raises(pkg.CheckpointError, match="weight_shape"):
        pkg.load_moe_layer(f, p, device="cpu")
    f = tmp_path / "g.safetensors"
    _write_ckpt(f, p, 1, 128, 64, 32,
                extra={f"{p}.experts.0.down_proj.weight_scale": torch.ones(128, 3).bfloat16()})
    with pytest.raises(pkg.CheckpointError, match="scale columns"):
        pkg.load_moe_layer(f, p, device="cpu")
    with pytest.raises(pkg.CheckpointError, match="no experts"):
        pkg.load_moe_layer(f, "other", device="cpu")


# ---------------------------------------------------------------------------
# apply() shim (integration/apply.py:91-169), against a vLLM-shaped stand-in
# ---------------------------------------------------------------------------


class _FakeMethod:
    """The two methods the reference patches, with vLLM's parameter names."""

    def __init__(self, group_size=32):
        self.group_size = group_size
        self.processed = 0

    def process_weights_after_loading(self, layer):
        self.processed += 1

    def apply(self, layer, x, topk_weights, topk_ids, activation="silu"):
        return ("stock", x, activation)


def _fake_layer(synth, device="cpu"):
    shape = synth.LayerShape(E=4, topk=2, K=128, N=64, group=32)
    w13, w2, s13, s2 = synth.make_weights(shape, device, seed=1, dtype_packed=torch.uint8)
    return types.SimpleNamespace(w13_weight_packed=w13, w2_weight_packed=w2,
                                 w13_weight_scale=s13, w2_weight_scale=s2), shape


@pytest.fixture
def fake_cls():
    cls = type("FakeWNA16", (_FakeMethod,), {})
    yield cls


def test_shim_env_off_keeps_stock(pkg, synth, fake_cls, monkeypatch):
    monkeypatch.delenv(pkg.integration.ENV_FLAG, raising=False)
    pkg.integration.install(fake_cls)
    m, (layer, _) = fake_cls(), _fake_layer(synth)
    m.process_weights_after_loading(layer)
    assert m.processed == 1 and not hasattr(layer, "_gb10_fused")
    assert m.apply(layer, "X", None, None)[0] == "stock"
    pkg.integration.uninstall(fake_cls)
    assert fake_cls.apply is _FakeMethod.apply


def test_shim_env_on_binds_and_routes(pkg, synth, fake_cls, monkeypatch):
    calls = []

    def recorder(*a, **kw):
        calls.append((a, kw))
        return "custom"

    monkeypatch.setenv(pkg.integration.ENV_FLAG, "1")
    monkeypatch.setattr(pkg.integration, "fused_experts_w4a16", recorder)
    pkg.integration.install(fake_cls)
    pkg.integration.install(fake_cls)  # idempotent
    m, (layer, _) = fake_cls(group_size=32), _fake_layer(synth)
    m.process_weights_after_loading(layer)
    assert m.processed == 1
    # bound tensors are the stock tensors themselves (no repack, nothing freed)
    same = lambda a, b: a.data_ptr() == b.data_ptr() and a.shape == b.shape  # noqa: E731
    assert same(layer._gb10_w1_q, layer.w13_weight_packed)
    assert same(layer._gb10_w2_scale, layer.w2_weight_scale)
    assert layer._gb10_group_size == 32
    tw, ti = torch.ones(3, 2), torch.zeros(3, 2, dtype=torch.int32)
    assert m.apply(layer, "X", tw, ti) == "custom"
    assert m.apply(layer=layer, x="Y", topk_weights=tw, topk_ids=ti) == "custom"
    a, kw = calls[0]
    assert a[0] == "X" and same(a[1], layer.w13_weight_packed)
    assert same(a[2], layer.w2_weight_packed)
    assert same(a[3], layer.w13_weight_scale) and same(a[4], layer.w2_weight_scale)
    assert a[5] is tw and a[6] is ti and kw == {"group_size": 32}
    assert calls[1][0][0] == "Y"
    # flag cleared at run time: fall through to stock, as the reference does
    monkeypatch.delenv(pkg.integration.ENV_FLAG)
    assert m.apply(layer, "Z", tw, ti) == ("stock", "Z", "silu")
    pkg.integration.uninstall(fake_cls)


def test_shim_function_form_and_errors(pkg, synth, monkeypatch):
    layer, _ = _fake_layer(synth)
    monkeypatch.setenv(pkg.integration.ENV_FLAG, "1")
    assert pkg.integration.apply(layer, "x", None, None, lambda v: ("stock", v), 5) == ("stock", 5)
    with pytest.raises(RuntimeError):
        pkg.integration.apply(layer, "x", None, None)
    with pytest.raises(pkg._lib.W4A16Error):
        pkg.integration.bind_layer(layer, 16)

    class NoIds:
        def process_weights_after_loading(self, layer):
            pass

        def apply(self, layer, x, router_logits):
            pass

    with pytest.raises(TypeError):
        pkg.integration.install(NoIds)
    with pytest.raises(ImportError):
        pkg.integration.install_into_vllm()


# ---------------------------------------------------------------------------
# GPU: checkpoint -> router -> fused experts
# ---------------------------------------------------------------------------


@pytest.mark.gpu
def test_checkpoint_layer_matches_oracle(pkg, orc, synth, dev, tmp_path):
    E, K, N, G, topk, M = 8, 256, 128, 32, 3, 20
    print("checkpoint layer E=8 K=256 N=128", flush=True)
    f = tmp_path / "l.safetensors"
    _write_ckpt(f, "model.layers.0.mlp", E, K, N, G, seed=7)
    layer = pkg.W4A16MoELayer.from_checkpoint(f, "model.layers.0.mlp", topk, device=dev)
    x = synth.make_hidden(M, K, dev, seed=7)
    g = torch.Generator().manual_seed(7)
    logits = torch.randn((M, E), generator=g).to(dev)
    out = layer(x, logits)
    vals, ids = torch.topk(logits, topk, dim=-1)
    tw = torch.softmax(vals, dim=-1)
    w = layer.weights
    ref = orc.moe_reference(x.cpu(), w.w13.cpu(), w.w2.cpu(), w.s13.cpu(), w.s2.cpu(),
                            tw.cpu(), ids.to(torch.int32).cpu(), G)
    torch.cuda.synchronize()
    o, r = out.float().cpu(), ref.float()
    assert orc.rel_l2(o, r) <= 5e-3
    assert orc.max_abs(o, r) <= 2e-2 * r.abs().max().item()


@pytest.mark.gpu
def test_shim_on_gpu_equals_direct_call(pkg, synth, dev, monkeypatch):
    monkeypatch.setenv(pkg.integration.ENV_FLAG, "1")
    cls = type("FakeWNA16Gpu", (_FakeMethod,), {})
    pkg.integration.install(cls)
    try:
        layer, shape = _fake_layer(synth, dev)
        m = cls(group_size=shape.group)
        m.process_weights_after_loading(layer)
        x = synth.make_hidden(9, shape.K, dev, seed=2)
        tw, ti = synth.make_routing(9, shape.E, shape.topk, dev, seed=2)
        got = m.apply(layer, x, tw, ti)
        want = pkg.fused_experts_w4a16(x, layer.w13_weight_packed, layer.w2_weight_packed,
                                       layer.w13_weight_scale, layer.w2_weight_scale, tw, ti,
                                       group_size=shape.group)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    finally:
        pkg.integration.uninstall(cls)
