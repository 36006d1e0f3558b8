"""GPU results against the golden fixtures written by apus's own CPU kernels.
Bars as in test_gpu_parity.py / test_gpu_moe.py: activation codes and scales
bit-exact; raw GEMMs max|d|/max|ref| <= 1e-3; BF16 linears within one BF16 ulp
plus 1e-4*max|ref| of the reference's unrounded GEMM; routed MoE 2^-7."""
import numpy as np
import pytest

from helpers import bf16_linear_ok, max_rel
from test_golden import bits, load, moe_experts

pytestmark = pytest.mark.gpu


def test_act_quant_golden_gpu(hip):
    d = load("act.npz")
    c, s = hip.act_quant(d["x"])
    assert np.array_equal(c, d["codes"]) and np.array_equal(bits(s), bits(d["scales"]))


@pytest.mark.parametrize("kind", ["fp4", "fp8"])
def test_gemm_golden_gpu(hip, kind):
    d = load(f"{kind}.npz")
    got = getattr(hip, f"{kind}_gemm")(d["w"], d["ws"], d["codes"], d["scales"])
    assert max_rel(got, d["gemm"]) <= 1e-3
    lin = getattr(hip, f"{kind}_linear")(d["w"], d["ws"], d["x"])
    ok = bf16_linear_ok(lin, d["gemm"], 1e-4 * np.abs(d["gemm"]).max())
    assert ok.all()


def test_moe_golden_gpu(hip):
    d = load("moe.npz")
    y = hip.moe_routed(moe_experts(d), d["x"], d["idx"], d["wgt"], float(d["limit"]),
                       layer_id=4242)
    assert max_rel(y, d["y"]) <= 2.0 ** -7
