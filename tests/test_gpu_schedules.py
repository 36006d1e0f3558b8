"""Dense FP8 schedules on tiled weights, swept over their instances.

The host FP8 and MXFP4 entry points keep weights MFMA-tiled in the dense cache when K
is 1024, 2048, 4096 or 8192 and O % 128 == 0, so these calls reach:

* the split-K GEMV (at most 8 rows; one workgroup per 16-row weight tile,
  16 waves or 8 at K = 1024 splitting K), FP8 and MXFP4 weights: codes
  through apus_hip_fp8_gemm / apus_hip_fp4_gemm, fp32 rows quantised in the
  kernel through apus_hip_fp8_linear / apus_hip_fp4_linear;
* the narrow schedule (9..64 rows; 1, 2 or 4 token tiles, 4 waves splitting
  K in quarters).

Every (rows, K) instance is held to the oracle's GEMM bar (max-rel 1e-3,
err/esc 1e-4 against the exact value) or, for the BF16 linear, to one BF16
ulp of the oracle's unrounded value plus 1e-4 of the largest. These
schedules and the grouped GEMV also run captured in a HIP graph, replayed
with eager work between the replays, bit for bit as eagerly.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import acts, bf16_linear_ok, err_esc, fp4_weights, fp8_weights, max_rel

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
def test_split_instances_fp4(hip, oracle, rng, M, K):
    """MXFP4 weights on the split-K GEMV: codes and fp32 rows."""
    O = 384
    w, ws = fp4_weights(rng, O, K)
    x = acts(rng, M, K, 2.0)
    c, s = oracle.act_quant(x)
    got = hip.fp4_gemm(w, ws, c, s)
    unrounded = oracle.fp4_gemm(w, ws, c, s)
    truth, esc = oracle.fp4_truth(w, ws, c, s)
    assert max_rel(got, unrounded) <= 1e-3
    assert err_esc(got, truth, esc) <= 1e-4
    lin = hip.fp4_linear(w, ws, x)
    assert bf16_linear_ok(lin, unrounded, 1e-4 * np.abs(unrounded).max()).all()


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


def test_dense_schedules_graph_replays(hip, oracle, rng):
    """The split-K GEMV (codes and fp32 rows), the narrow schedule and the
    grouped GEMV captured in one graph and replayed three times with eager
    work between the replays: every replay equals the eager run bit for
    bit."""
    import ctypes as C
    L = hip.lib()
    K, O = 4096, 1024
    w, ws = fp8_weights(rng, O, K)
    dw, dws = hip.DevBuf.from_array(w), hip.DevBuf.from_array(ws)
    tw = hip.DevBuf(O * K)
    hip._check(L.apus_hip_pack_weights_dev(1, dw.ptr, None, tw.ptr, None, O, K), "pack")
    x = acts(rng, 40, K)
    dx = hip.DevBuf.from_array(x)
    dc, ds = hip.DevBuf(40 * K), hip.DevBuf(40 * (K // 128) * 4)
    hip._check(L.apus_hip_act_quant_dev(dx.ptr, 40, K, dc.ptr, ds.ptr), "act_quant")
    wsp = hip.DevBuf(L.apus_hip_linear_workspace(3, K))
    y_lin, y_m1, y_m40 = hip.DevBuf(3 * O * 4), hip.DevBuf(O * 4), hip.DevBuf(40 * O * 4)
    # grouped: 6 one-row MXFP4 entries on tiled weights
    w4, ws4 = fp4_weights(rng, 2048, K)
    d4, ds4 = hip.DevBuf.from_array(w4), hip.DevBuf.from_array(ws4)
    t4, ts4 = hip.DevBuf(2048 * K // 2), hip.DevBuf(2048 * K // 32)
    hip._check(L.apus_hip_pack_weights_dev(0, d4.ptr, ds4.ptr, t4.ptr, ts4.ptr, 2048, K), "pack fp4")
    y_g = hip.DevBuf(6 * 2048 * 4)
    ents = (hip.ApusHipGemmEnt * 6)()
    for i in range(6):
        ents[i] = hip.ApusHipGemmEnt(t4.ptr, ts4.ptr, y_g.ptr, None, None, i, i, 1, 0)
    de = hip.DevBuf(C.sizeof(ents))
    hip._check(L.apus_hip_h2d(de.ptr, C.addressof(ents), C.sizeof(ents)), "h2d")

    def run():
        hip._check(L.apus_hip_linear_dev(1 | hip.W_TILED, tw.ptr, dws.ptr, dx.ptr, y_lin.ptr, 3, K, O,
                                         wsp.ptr), "linear")
        hip._check(L.apus_hip_fp8_gemm_dev(tw.ptr, dws.ptr, dc.ptr, ds.ptr, y_m1.ptr, 1, O, K, hip.W_TILED),
                   "gemm M=1")
        hip._check(L.apus_hip_fp8_gemm_dev(tw.ptr, dws.ptr, dc.ptr, ds.ptr, y_m40.ptr, 40, O, K,
                                           hip.W_TILED), "gemm M=40")
        hip._check(L.apus_hip_gemm_grouped_dev(0 | hip.W_TILED, de.ptr, 6, dc.ptr, ds.ptr, 2048, K, 2048,
                                               0, 1), "grouped")

    outs = ((y_lin, (3, O)), (y_m1, (1, O)), (y_m40, (40, O)), (y_g, (6, 2048)))
    run()
    hip._check(L.apus_hip_synchronize(), "sync")
    eager = [b.to_array(np.float32, shp).copy() for b, shp in outs]
    hip._check(L.apus_hip_graph_begin(), "graph_begin")
    run()
    hip._check(L.apus_hip_graph_end(), "graph_end")
    for rep in range(3):
        for b, shp in outs:
            hip._check(L.apus_hip_memset(b.ptr, 0, int(np.prod(shp)) * 4), "memset")
        hip._check(L.apus_hip_graph_replay(1), "replay")
        hip._check(L.apus_hip_synchronize(), "sync")
        for (b, shp), e in zip(outs, eager):
            assert np.array_equal(b.to_array(np.float32, shp).view(np.uint32), e.view(np.uint32)), rep
        run()                                        # eager launches between replays
        hip._check(L.apus_hip_synchronize(), "sync")
    c6, s6 = oracle.act_quant(x[:6])
    assert max_rel(eager[3], oracle.fp4_gemm(w4, ws4, c6, s6)) <= 1e-3
