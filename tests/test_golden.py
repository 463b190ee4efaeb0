"""The committed golden fixtures (tests/golden/) against the oracle and the HIP path.

The fixtures are worked out from the reference's definitions by
tests/golden/make_golden.py, which shares no code with ``oracle/``:
align cases (kernels/w4a16_moe.py:187-290) are bit-exact targets; dequant
cases (bench/bench_moe.py:102-119) are bit-exact bf16 patterns; the
whole-layer cases (bench/bench_moe.py:271-303) hold the float64 output from
bf16-rounded dequantized weights.  Tolerances for those:
  * oracle (fp32, same weight rounding): rel-L2 <= 1e-5;
  * HIP path: rel-L2 <= 5e-3 and max-abs <= 2e-2 * max|out|.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
MOE_CASES = ["moe_gemv", "moe_mfma"]


def _align_cases():
    return json.loads((GOLDEN / "align_cases.json").read_text())


def _dequant_cases():
    return json.loads((GOLDEN / "dequant_cases.json").read_text())


def _ids(case):
    topk = len(case["ids"][0]) if case["ids"] else 10
    return np.array(case["ids"], dtype=np.int32).reshape(-1, topk)


def _moe(name):
    with np.load(GOLDEN / f"{name}.npz") as z:
        return {k: z[k] for k in z.files}


def _bits_to_bf16(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(b.astype(np.int16)).view(torch.bfloat16)


def _moe_tensors(c, device):
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    return dict(
        hidden=_bits_to_bf16(c["hidden_bits"]).to(device),
        w13=to(c["w13"]), w2=to(c["w2"]),
        w13_scale=_bits_to_bf16(c["w13_scale_bits"]).to(device),
        w2_scale=_bits_to_bf16(c["w2_scale_bits"]).to(device),
        topk_weights=to(c["topk_weights"]), topk_ids=to(c["topk_ids"]),
        group=int(c["group"]))


# ---------------------------------------------------------------------------
# oracle (CPU)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("i", range(len(_align_cases())))
def test_oracle_align_golden(orc, i):
    case = _align_cases()[i]
    ids = _ids(case)
    for fn in (orc.moe_align_block_size, orc.moe_align_block_size_c):
        s, e, n = fn(ids, case["block"], case["num_experts"])[:3]
        assert np.asarray(s).tolist() == case["sorted_ids"], fn.__name__
        assert np.asarray(e).tolist() == case["expert_ids"], fn.__name__
        assert int(np.asarray(n).reshape(-1)[0]) == case["num_post"], fn.__name__


@pytest.mark.parametrize("i", range(len(_dequant_cases())))
def test_oracle_dequant_golden(orc, i):
    case = _dequant_cases()[i]
    words = np.array(case["words"], dtype=np.uint32)[None, :]
    scales = np.array(case["scale_bits"], dtype=np.uint16)[None, :]
    got = orc.dequant(words.view(np.uint8), scales, case["group"])
    assert orc.f32_to_bf16_bits(got).reshape(-1).tolist() == case["expected_bits"]


@pytest.mark.parametrize("name", MOE_CASES)
def test_oracle_moe_golden(orc, name):
    c = _moe(name)
    t = _moe_tensors(c, "cpu")
    got = orc.moe_reference(t["hidden"], t["w13"], t["w2"], t["w13_scale"], t["w2_scale"],
                            t["topk_weights"], t["topk_ids"], t["group"], out_dtype=None)
    want = torch.from_numpy(c["expected_out"])
    assert orc.rel_l2(got, want) <= 1e-5


# ---------------------------------------------------------------------------
# HIP path (GPU)
# ---------------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(len(_align_cases())))
def test_gpu_align_golden(pkg, dev, i):
    case = _align_cases()[i]
    ids = torch.from_numpy(_ids(case)).to(dev)
    s, e, n, off, drop = pkg.moe_align_block_size_full(ids, case["block"],
                                                       case["num_experts"])
    torch.cuda.synchronize()
    assert off.cpu().tolist() == case["offsets"]
    assert int(drop.cpu()[0]) == case["dropped"]
    assert s.cpu().tolist() == case["sorted_ids"]
    assert e.cpu().tolist() == case["expert_ids"]
    assert int(n.cpu().reshape(-1)[0]) == case["num_post"]


@pytest.mark.gpu
@pytest.mark.parametrize("name", MOE_CASES)
def test_gpu_moe_golden(pkg, orc, dev, name):
    c = _moe(name)
    t = _moe_tensors(c, dev)
    out = pkg.fused_experts_w4a16(t["hidden"], t["w13"], t["w2"], t["w13_scale"],
                                  t["w2_scale"], t["topk_weights"], t["topk_ids"],
                                  group_size=t["group"])
    torch.cuda.synchronize()
    want = torch.from_numpy(c["expected_out"])
    got = out.float().cpu()
    rl2 = orc.rel_l2(got, want)
    mab = orc.max_abs(got, want)
    scale = float(want.abs().max())
    print(f"{name}: rel_l2={rl2:.3e} max_abs={mab:.3e} max|out|={scale:.3e}", flush=True)
    assert rl2 <= 5e-3
    assert mab <= 2e-2 * scale
