"""Dense FP8 schedules on tiled weights, swept over their instances.

The host FP8 entry points keep weights MFMA-tiled in the dense cache when K
is 1024, 2048, 4096 or 8192 and O % 128 == 0, so these calls reach:

* the split-K GEMV (at most 8 rows; one workgroup per 16-row weight tile,
  16 waves or 8 at K = 1024 splitting K): codes through apus_hip_fp8_gemm,
  fp32 rows quantised in the kernel through apus_hip_fp8_linear;
* the narrow schedule (9..64 rows; 1, 2 or 4 token tiles, 4 waves splitting
  K in quarters).

Every (rows, K) instance is held to the oracle's GEMM bar (max-rel 1e-3,
err/esc 1e-4 against the exact value) or, for the BF16 linear, to one BF16
ulp of the oracle's unrounded value plus 1e-4 of the largest.
"""
import numpy as np
import pytest

from helpers import acts, bf16_linear_ok, err_esc, fp8_weights, max_rel

pytestmark = pytest.mark.gpu

KS = (1024, 2048, 4096, 8192)


@pytest.mark.parametrize("K", KS)
@pytest.mark.parametrize("M", (9, 16, 17, 32, 33, 64))
def test_narrow_instances(hip, oracle, rng, M, K):
    O = 256
    w, ws = fp8_weights(rng, O, K)
    c, s = oracle.act_quant(acts(rng, M, K, 2.0))
    got = hip.fp8_gemm(w, ws, c, s)
    truth, esc = oracle.fp8_truth(w, ws, c, s)
    assert max_rel(got, oracle.fp8_gemm(w, ws, c, s)) <= 1e-3
    assert err_esc(got, truth, esc) <= 1e-4


@pytest.mark.parametrize("K", KS)
@pytest.mark.parametrize("M", (1, 2, 5, 8))
def test_split_instances(hip, oracle, rng, M, K):
    O = 384
    w, ws = fp8_weights(rng, O, K)
    x = acts(rng, M, K, 2.0)
    c, s = oracle.act_quant(x)
    got = hip.fp8_gemm(w, ws, c, s)
    unrounded = oracle.fp8_gemm(w, ws, c, s)
    truth, esc = oracle.fp8_truth(w, ws, c, s)
    assert max_rel(got, unrounded) <= 1e-3
    assert err_esc(got, truth, esc) <= 1e-4
    lin = hip.fp8_linear(w, ws, x)
    assert bf16_linear_ok(lin, unrounded, 1e-4 * np.abs(unrounded).max()).all()
