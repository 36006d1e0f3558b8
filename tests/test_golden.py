"""The oracle reproduces the golden fixtures written by apus's own compiled CPU
kernels (tests/golden/make_golden.py), bit for bit. Runs anywhere (the
fixtures are committed; the apus sources are not needed)."""
import hashlib
import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def test_fixture_checksums():
    for line in open(os.path.join(HERE, "SHA256SUMS")):
        digest, name = line.split()
        assert hashlib.sha256(open(os.path.join(HERE, name), "rb").read()).hexdigest() == digest


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_act_quant_golden(oracle):
    d = load("act.npz")
    c, s = oracle.act_quant(d["x"])
    assert np.array_equal(c, d["codes"]) and np.array_equal(bits(s), bits(d["scales"]))


@pytest.mark.parametrize("kind", ["fp4", "fp8"])
def test_gemm_golden(oracle, kind):
    d = load(f"{kind}.npz")
    c, s = oracle.act_quant(d["x"])
    assert np.array_equal(c, d["codes"]) and np.array_equal(bits(s), bits(d["scales"]))
    gemm = getattr(oracle, f"{kind}_gemm")(d["w"], d["ws"], c, s)
    lin = getattr(oracle, f"{kind}_linear")(d["w"], d["ws"], d["x"])
    assert np.array_equal(bits(gemm), bits(d["gemm"]))
    assert np.array_equal(bits(lin), bits(d["linear"]))


def moe_experts(d):
    E = max(int(k[1:k.index("_")]) for k in d.files if k.startswith("e")) + 1
    return [tuple(d[f"e{e}_{n}"] for n in ("w1", "w1s", "w2", "w2s", "w3", "w3s"))
            for e in range(E)]


def test_moe_golden(oracle):
    d = load("moe.npz")
    y = oracle.moe_routed(moe_experts(d), d["x"], d["idx"], d["wgt"], float(d["limit"]))
    assert np.array_equal(bits(y), bits(d["y"]))
