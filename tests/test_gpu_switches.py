"""Every environment-selected schedule runs and gives the default's results.

The backend reads its schedule switches once per process, so each case runs
tests/switch_probe.py in a child process with one switch set (one process on
the GPU at a time: the child runs while this one waits) and compares its
outputs with a child run without switches:

* APUS_HIP_PRE_LDS=0 / 2 (many-row w1/w3 work items on the resident-
  activation schedule instead of the LDS one / the w2 ones on the LDS
  schedule too), with APUS_HIP_PRE_RA=0 /
  APUS_HIP_PRE_RA13=0 as well (many-row w2 / w1-w3 on the double-buffered
  prefill schedule),
  APUS_HIP_PAIR13_WIDE=0 / 1 (narrow or wide one-token w1/w3 workgroups),
  APUS_HIP_MOE_PAIRS=0 / 64 (always sort by expert / per-pair kernels up to
  64 pairs), APUS_HIP_MOE_SIDE=0 (the shared expert on the caller's stream),
  APUS_HIP_LAYER1=0 (two launches per one-token layer): the routed dispatch
  keeps one accumulation order in every schedule, so y and the h codes must
  be bit-identical, and so must the sublayer's outputs;
* APUS_HIP_LDS_TILE=0 (dense FP8 GEMMs with more than 8 rows on the
  register-ring tile schedule instead of the LDS one): both form one chain
  per output over the 128-groups in order, so the dense outputs must be
  bit-identical too; APUS_HIP_NARROW=0 (9..64-row dense FP8 GEMMs on the
  tile schedule instead of the narrow one, which splits K in four): those
  outputs held to the oracle's bars; APUS_HIP_SPLIT=0 (FP8 and MXFP4
  launches of at most 8 rows on tiled weights on the few-row schedule
  instead of the split-K GEMV, another K split): those outputs held to the oracle's bars;
  APUS_HIP_GRP=0 (grouped launches of few-row entries on tiled weights on
  the few-row schedule instead of the grouped GEMV): the grouped MXFP4
  outputs held to the oracle's bars;
* APUS_HIP_DEC_KS=1 / 2 / 4 (waves splitting K in the few-row schedule):
  dense outputs change only in fp32 summation order, so they are held to
  the oracle's bars (max-rel 1e-3, err/esc 1e-4); routed outputs stay
  bit-identical (the routed launches fix their own chains). The sublayer's
  FP8 shared expert is a chain of dense few-row linears, so its output (and
  the final bf16(routed + shared)) may move by BF16 roundings: held to the
  sublayer bars against the default run (max |d| / max |ref| <= 2^-6,
  mean |d| / mean |ref| <= 2^-9).
"""
import os
import subprocess
import sys

import numpy as np
import pytest

from helpers import bf16_linear_ok, err_esc, max_rel

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
PROBE = os.path.join(HERE, "switch_probe.py")
SWITCHES = ["APUS_HIP_PRE_LDS", "APUS_HIP_PRE_RA", "APUS_HIP_PRE_RA13", "APUS_HIP_DEC_KS",
            "APUS_HIP_PAIR13_WIDE", "APUS_HIP_MOE_PAIRS", "APUS_HIP_MOE_SIDE", "APUS_HIP_LAYER1",
            "APUS_HIP_LDS_TILE", "APUS_HIP_NARROW", "APUS_HIP_SPLIT", "APUS_HIP_GRP"]


def _probe(tmp_path, name, env_set):
    env = {k: v for k, v in os.environ.items() if k not in SWITCHES}
    env.update(env_set)
    out = tmp_path / f"{name}.npz"
    print(f"switch probe {name} {env_set}", flush=True)
    r = subprocess.run([sys.executable, "-u", PROBE, str(out)], env=env, timeout=300,
                       capture_output=True, text=True)
    assert r.returncode == 0, f"{name}: rc {r.returncode}\n{r.stdout[-2000:]}\n{r.stderr[-3000:]}"
    return dict(np.load(out))


@pytest.fixture(scope="module")
def default_run(tmp_path_factory):
    return _probe(tmp_path_factory.mktemp("switch"), "default", {})


ROUTED = [k for s in (1, 2, 4, 64) for k in (f"y{s}", f"hc{s}", f"he{s}")] + \
    ["fwd_out", "fwd_routed", "fwd_shared", "fwd_idx"]


def _same(a, b):
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


CASES = [{"APUS_HIP_PRE_LDS": "0"}, {"APUS_HIP_PRE_LDS": "2"},
         {"APUS_HIP_PRE_LDS": "0", "APUS_HIP_PRE_RA": "0"},
         {"APUS_HIP_PRE_LDS": "0", "APUS_HIP_PRE_RA13": "0"},
         {"APUS_HIP_PAIR13_WIDE": "0"}, {"APUS_HIP_PAIR13_WIDE": "1"},
         {"APUS_HIP_MOE_PAIRS": "0"}, {"APUS_HIP_MOE_PAIRS": "64"},
         {"APUS_HIP_MOE_SIDE": "0"}, {"APUS_HIP_LAYER1": "0"},
         {"APUS_HIP_DEC_KS": "1"}, {"APUS_HIP_DEC_KS": "2"}, {"APUS_HIP_DEC_KS": "4"},
         {"APUS_HIP_LDS_TILE": "0"}, {"APUS_HIP_NARROW": "0"}, {"APUS_HIP_SPLIT": "0"},
         {"APUS_HIP_GRP": "0"}]


@pytest.mark.parametrize("env", CASES, ids=lambda e: ",".join(f"{k[9:]}={v}" for k, v in e.items()))
def test_switch(oracle, tmp_path, default_run, env):
    var = "APUS_HIP_DEC_KS" if "APUS_HIP_DEC_KS" in env else next(iter(env))
    val = env[var]
    got = _probe(tmp_path, "_".join(f"{k}_{v}" for k, v in env.items()), env)
    base = default_run
    dense_chain = {"fwd_shared", "fwd_out"} if var == "APUS_HIP_DEC_KS" else set()
    for k in ROUTED:
        assert np.isfinite(got[k]).all() if got[k].dtype == np.float32 else True, k
        if k in dense_chain:
            d = np.abs(got[k] - base[k])
            assert d.max() <= 2.0 ** -6 * np.abs(base[k]).max(), k
            assert d.mean() <= 2.0 ** -9 * np.abs(base[k]).mean(), k
            continue
        assert _same(got[k], base[k]), f"{var}={val}: {k} differs from the default schedule"
    # dense launches: bitwise unless the K split was changed (a forced few-row
    # split also turns the split-K GEMV off)
    split = var in ("APUS_HIP_SPLIT", "APUS_HIP_DEC_KS")
    keys = ([] if var == "APUS_HIP_GRP" else [f"fp4_y{i}" for i in range(12)]) + \
        ([] if split else ["fp8_y"])
    if var != "APUS_HIP_DEC_KS":
        for k in keys:
            assert _same(got[k], base[k]), k
    for name in ("t1", "t2", "t3", "t4", "t5", "t6", "t7", "l1", "f1", "l2"):
        if var == "APUS_HIP_NARROW" and name in ("t3", "t4", "t5"):
            continue    # another K split: held to the oracle's bars below
        if split and name in ("t6", "t7", "l1", "f1", "l2"):
            continue
        y = got[f"{name}_y"]
        assert _same(y, base[f"{name}_y"]), f"{var}={val}: {name} differs from the default schedule"
    want = oracle.fp8_linear(got["l1_w"], got["l1_ws"], got["l1_x"])
    c, s = oracle.act_quant(got["l1_x"])
    unrounded = oracle.fp8_gemm(got["l1_w"], got["l1_ws"], c, s)
    assert bf16_linear_ok(got["l1_y"], unrounded, 1e-4 * np.abs(unrounded).max()).all()
    assert max_rel(got["l1_y"], want) <= 2.0 ** -6
    for name in ("t1", "t2", "t3", "t4", "t5", "t6", "t7"):
        y = got[f"{name}_y"]
        args = (got[f"{name}_w"], got[f"{name}_ws"], got[f"{name}_c"], got[f"{name}_s"])
        truth, esc = oracle.fp8_truth(*args)
        assert max_rel(y, oracle.fp8_gemm(*args)) <= 1e-3 and err_esc(y, truth, esc) <= 1e-4, name
    args = (got["f1_w"], got["f1_ws"], got["f1_c"], got["f1_s"])
    truth, esc = oracle.fp4_truth(*args)
    assert max_rel(got["f1_y"], oracle.fp4_gemm(*args)) <= 1e-3 and err_esc(got["f1_y"], truth, esc) <= 1e-4
    c, s = oracle.act_quant(got["l2_x"])
    unrounded = oracle.fp4_gemm(got["l2_w"], got["l2_ws"], c, s)
    assert bf16_linear_ok(got["l2_y"], unrounded, 1e-4 * np.abs(unrounded).max()).all()
    want = oracle.fp8_gemm(got["fp8_w"], got["fp8_ws"], got["fp8_c"], got["fp8_s"])
    truth, esc = oracle.fp8_truth(got["fp8_w"], got["fp8_ws"], got["fp8_c"], got["fp8_s"])
    assert max_rel(got["fp8_y"], want) <= 1e-3
    assert err_esc(got["fp8_y"], truth, esc) <= 1e-4
    for i in range(12):
        w, ws = got[f"fp4_w{i}"], got[f"fp4_ws{i}"]
        want = oracle.fp4_gemm(w, ws, got["fp4_c"], got["fp4_s"])
        truth, esc = oracle.fp4_truth(w, ws, got["fp4_c"], got["fp4_s"])
        assert max_rel(got[f"fp4_y{i}"], want) <= 1e-3, i
        assert err_esc(got[f"fp4_y{i}"], truth, esc) <= 1e-4, i
