"""Edge cases of the element rules on the GPU.

* The SwiGLU element (c/moe.h:113-126) on its own, apus_hip_swiglu_dev,
  over a grid that includes g and u at and beyond +-limit, |g| past 88
  (expf over- and underflow), zeros, subnormals, infinities and NaN, with
  limit 10 and without a limit: equal to the oracle (glibc expf) bit for
  bit, except where the exact value lies within 2^-19 (relative) of a BF16
  rounding boundary, where either neighbour is allowed; and within one
  BF16 ulp of the float64 value wherever the fp32 steps stay in range.
* E8M0 weight scale bytes 251..254 decode as 2^(b-127) inside the GEMM
  (bit-exact against the oracle with an activation scale of 2^-8, so the
  products stay finite); byte 255 (+inf in the reference, NaN on the
  matrix cores) is refused by the host-pointer entry points.
* Non-finite activations: refused by the host-pointer entry points; on the
  device entry points a group holding an infinity gets the reference's scale
  (+inf) and signed-zero codes for its finite elements, and its GEMM row
  comes out NaN while the other rows are unaffected.
* apus_hip_memset refuses to run while a graph capture is open.
* The split-K GEMV's in-kernel quantisation of fp32 rows (FP8 linears of up
  to 8 rows on tiled weights) equals act-quant followed by the same GEMV on
  codes, bit for bit, with NaN-only, infinite, zero, subnormal and large
  groups.
"""
import ctypes as C

import numpy as np
import pytest

from helpers import acts, bf16, fp4_weights, fp8_weights

pytestmark = pytest.mark.gpu


def swiglu_gpu(hip, g, u, limit):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    dg, du = hip.DevBuf.from_array(g), hip.DevBuf.from_array(u)
    dh = hip.DevBuf(g.nbytes)
    hip._check(hip.lib().apus_hip_swiglu_dev(dg.ptr, du.ptr, g.size, limit, dh.ptr), "swiglu")
    return dh.to_array(np.float32, g.shape)


def swiglu_grid(rng):
    special = np.array([0.0, -0.0, 1e-40, -1e-40, 1e-30, 0.5, -0.5, 1.0, -1.0, -1.2784645,
                        9.999999, 10.0, 10.000001, 11.0, -10.0, -10.000001, -11.0, 20.0, -20.0,
                        87.0, 88.5, 89.0, 100.0, -87.0, -88.5, -89.0, -100.0, -104.0, 3e38,
                        -3e38, np.inf, -np.inf, np.nan], np.float32)
    g1, u1 = np.meshgrid(special, special)
    g2 = (rng.standard_normal(200000) * 4).astype(np.float32)
    u2 = (rng.standard_normal(200000) * 4).astype(np.float32)
    g3 = rng.uniform(-120, 120, 50000).astype(np.float32)
    u3 = rng.uniform(-12, 12, 50000).astype(np.float32)
    return (np.concatenate([g1.ravel(), bf16(g2), g3]),
            np.concatenate([u1.ravel(), bf16(u2), u3]))


def swiglu_f64(g, u, limit):
    g = g.astype(np.float64)
    u = u.astype(np.float64)
    if limit > 0:
        u = np.where(u > limit, limit, np.where(u < -limit, -limit, u))
        g = np.where(g > limit, limit, g)
    with np.errstate(over="ignore", invalid="ignore"):
        return (g * (1.0 / (1.0 + np.exp(-g)))) * u


@pytest.mark.parametrize("limit", [10.0, 0.0])
def test_swiglu_element(hip, oracle, limit):
    rng = np.random.default_rng(77)
    g, u = swiglu_grid(rng)
    got = swiglu_gpu(hip, g, u, limit)
    want = oracle.swiglu(g, u, limit)
    exact = swiglu_f64(g, u, limit)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    same = got.view(np.uint32) == want.view(np.uint32)
    # where they differ, the exact value must be within 2^-19 of a BF16
    # rounding boundary: both neighbours are then correct roundings of an
    # fp32 evaluation with a different (correctly bounded) expf
    with np.errstate(invalid="ignore", over="ignore"):
        lo = bf16((exact * (1 - 2.0 ** -19)).astype(np.float32))
        hi = bf16((exact * (1 + 2.0 ** -19)).astype(np.float32))
    cand = (got == lo) | (got == hi) | same
    bad = np.nonzero(~cand & ~nan)[0]
    assert bad.size == 0, f"limit {limit}: g {g[bad[:5]]} u {u[bad[:5]]}: gpu {got[bad[:5]]} cpu {want[bad[:5]]}"
    # and within one BF16 ulp of the float64 value wherever the fp32 steps
    # neither overflow (expf(-g) for g < -88) nor leave the normal range
    gc = np.minimum(g, limit) if limit > 0 else g
    with np.errstate(invalid="ignore"):
        fin = (np.isfinite(exact) & np.isfinite(got) & (np.abs(gc) <= 80) &
               ((np.abs(exact) >= 2.0 ** -100) | (exact == 0)))
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(exact[fin]), 2.0 ** -100))) - 7)
    assert np.all(np.abs(got[fin].astype(np.float64) - exact[fin]) <= ulp)
    assert np.all(np.abs(want[fin].astype(np.float64) - exact[fin]) <= ulp)
    flips = int((~same & ~nan).sum())
    print(f"limit {limit}: {g.size} elements, {flips} one-ulp differences from glibc expf")
    assert flips <= g.size // 1000
    if limit > 0:
        # clamps: g above the limit and u beyond +-limit give the clamped value exactly
        m = (g > limit) & np.isfinite(u)
        assert np.array_equal(got[m], oracle.swiglu(np.full(m.sum(), limit, np.float32), u[m], limit))


def test_e8m0_high_bytes(hip, oracle):
    """Scale bytes 251..254 in FP4 and FP8 weights, one-hot activations with
    scale 2^-8: the GEMM returns 2^-8 times the decoded weight, bit-exact."""
    K, O = 256, 128
    rng = np.random.default_rng(3)
    w, ws = fp4_weights(rng, O, K)
    ws[:, :] = 251 + (np.arange(O)[:, None] + np.arange(K // 32)[None, :]) % 4
    codes = np.zeros((8, K), np.uint8)
    for i in range(8):
        codes[i, 17 * i + 3] = 0x38                     # 1.0
    scales = np.full((8, K // 128), 2.0 ** -8, np.float32)
    got = hip.fp4_gemm(w, ws, codes, scales)
    want = oracle.fp4_gemm(w, ws, codes, scales)
    assert np.isfinite(want).all()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    w8, ws8 = fp8_weights(rng, O, K)
    ws8[:, :] = np.array([[251, 254]], np.uint8)
    got8 = hip.fp8_gemm(w8, ws8, codes, scales)
    want8 = oracle.fp8_gemm(w8, ws8, codes, scales)
    assert np.isfinite(want8).all()
    assert np.array_equal(got8.view(np.uint32), want8.view(np.uint32))


def test_e8m0_255_refused(hip, oracle):
    K, O = 256, 128
    rng = np.random.default_rng(4)
    w, ws = fp4_weights(rng, O, K)
    ws[5, 2] = 255
    c, s = oracle.act_quant(acts(rng, 2, K))
    with pytest.raises(hip.ApusHipError, match="255"):
        hip.fp4_gemm(w, ws, c, s)
    with pytest.raises(hip.ApusHipError, match="255"):
        hip.fp4_linear(w, ws, acts(rng, 1, K))
    w8, ws8 = fp8_weights(rng, O, K)
    ws8[0, 1] = 255
    with pytest.raises(hip.ApusHipError, match="255"):
        hip.fp8_gemm(w8, ws8, c, s)
    w8[0, 0] = 0x7F
    ws8[0, 1] = 120
    with pytest.raises(hip.ApusHipError, match="0x7f"):
        hip.fp8_gemm(w8, ws8, c, s)


@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_nonfinite_activation_refused(hip, bad):
    K, O = 256, 128
    rng = np.random.default_rng(5)
    w, ws = fp4_weights(rng, O, K)
    x = acts(rng, 2, K)
    x[1, 100] = bad
    with pytest.raises(hip.ApusHipError, match="non-finite"):
        hip.fp4_linear(w, ws, x)
    with pytest.raises(hip.ApusHipError, match="non-finite"):
        hip.act_quant(x)


def test_nonfinite_activation_dev(hip, oracle):
    K, O = 256, 128
    rng = np.random.default_rng(6)
    x = acts(rng, 2, K)
    x[0, 5] = np.inf
    dx = hip.DevBuf.from_array(x)
    dc, ds = hip.DevBuf(2 * K), hip.DevBuf(2 * (K // 128) * 4)
    hip._check(hip.lib().apus_hip_act_quant_dev(dx.ptr, 2, K, dc.ptr, ds.ptr), "act_quant_dev")
    codes = dc.to_array(np.uint8, (2, K))
    scales = ds.to_array(np.float32, (2, K // 128))
    assert scales[0, 0] == np.inf                        # the reference's scale for the group
    fin = np.arange(128) != 5
    want0 = np.where(x[0, :128] < 0, 0x80, 0x00)[fin]    # x / inf: signed zeros
    assert np.array_equal(codes[0, :128][fin], want0)
    rc, rs = oracle.act_quant(bf16(x[:, :]).copy())
    assert np.array_equal(codes[0, 128:], rc[0, 128:]) and np.array_equal(codes[1], rc[1])
    assert np.array_equal(scales[0, 1:], rs[0, 1:]) and np.array_equal(scales[1], rs[1])
    w, ws = fp4_weights(rng, O, K)
    dw, dws = hip.DevBuf.from_array(w), hip.DevBuf.from_array(ws)
    dout = hip.DevBuf(2 * O * 4)
    hip._check(hip.lib().apus_hip_fp4_gemm_dev(dw.ptr, dws.ptr, dc.ptr, ds.ptr, dout.ptr, 2, O, K, 0),
               "fp4_gemm_dev")
    out = dout.to_array(np.float32, (2, O))
    assert np.isnan(out[0]).all()
    want1 = oracle.fp4_gemm(w, ws, rc[1:].copy(), rs[1:].copy())
    assert np.abs(out[1] - want1[0]).max() <= 1e-3 * np.abs(want1).max()


def test_memset_refused_under_capture(hip):
    L = hip.lib()
    buf = hip.DevBuf(4096)
    hip._check(L.apus_hip_memset(buf.ptr, 0, 4096), "memset")
    hip._check(L.apus_hip_graph_begin(), "graph_begin")
    rc = L.apus_hip_memset(buf.ptr, 1, 4096)
    msg = L.apus_hip_last_error().decode()
    hip._check(L.apus_hip_graph_end(), "graph_end")
    assert rc != 0 and "capture" in msg
    hip._check(L.apus_hip_memset(buf.ptr, 7, 4096), "memset after capture")
    assert (buf.to_array(np.uint8, (4096,)) == 7).all()


def test_act_quant_dev_unaligned(hip, oracle):
    """x rows that are not 16-byte aligned take the one-wave-per-group
    kernel; codes and scales equal the oracle's and the aligned call's."""
    M, K = 3, 512
    rng = np.random.default_rng(7)
    x = acts(rng, M, K)
    x[1, :128] *= 1e-3
    rc, rs = oracle.act_quant(bf16(x).copy())
    buf = hip.DevBuf((M * K + 4) * 4)
    pad = np.zeros(M * K + 4, np.float32)
    pad[1:1 + M * K] = x.ravel()
    hip._check(hip.lib().apus_hip_h2d(buf.ptr, pad.ctypes.data, pad.nbytes), "h2d")
    for off in (0, 4):                    # bytes: aligned copy at 16, unaligned at 4
        src = hip.DevBuf.from_array(x) if off == 0 else None
        dc, ds = hip.DevBuf(M * K), hip.DevBuf(M * (K // 128) * 4)
        ptr = src.ptr if src else buf.ptr + off
        hip._check(hip.lib().apus_hip_act_quant_dev(ptr, M, K, dc.ptr, ds.ptr), "act_quant_dev")
        assert np.array_equal(dc.to_array(np.uint8, (M, K)), rc), off
        assert np.array_equal(ds.to_array(np.float32, (M, K // 128)), rs), off


@pytest.mark.parametrize("M,O,K", [(1, 512, 4096), (3, 1024, 1024), (8, 512, 8192), (2, 256, 2048)])
def test_split_linear_quant_equals_act_quant(hip, rng, M, O, K):
    """FP8 linears of at most 8 rows on tiled weights quantise x inside the
    split-K GEMV; the result equals act-quant then the same GEMV on codes,
    bit for bit, with groups of NaN only, an infinity, zeros, subnormals and
    large values among ordinary ones."""
    L = hip.lib()
    w, ws = fp8_weights(rng, O, K)
    x = acts(rng, M, K, 2.0)
    x[0, 0:128] = np.nan                                  # a group of NaN only
    x[0, 200] = np.inf                                    # an infinity
    x[M - 1, 256:384] = 0.0                               # zeros
    x[M - 1, 384:512] = np.float32(3e-39) * rng.standard_normal(128).astype(np.float32)   # subnormals
    if K >= 1024:
        x[0, 640:768] *= np.float32(1e30)                 # large values
    dx = hip.DevBuf.from_array(np.ascontiguousarray(x, np.float32))
    dw, dws = hip.DevBuf.from_array(w), hip.DevBuf.from_array(ws)
    tw = hip.DevBuf(O * K)
    hip._check(L.apus_hip_pack_weights_dev(1, dw.ptr, None, tw.ptr, None, O, K), "pack")
    wsp = hip.DevBuf(L.apus_hip_linear_workspace(M, K))
    y1 = hip.DevBuf(M * O * 4)
    hip._check(L.apus_hip_linear_dev(1 | hip.W_TILED, tw.ptr, dws.ptr, dx.ptr, y1.ptr, M, K, O, wsp.ptr),
               "linear_dev")
    dc, ds = hip.DevBuf(M * K), hip.DevBuf(M * (K // 128) * 4)
    hip._check(L.apus_hip_act_quant_dev(dx.ptr, M, K, dc.ptr, ds.ptr), "act_quant_dev")
    y2 = hip.DevBuf(M * O * 4)
    hip._check(L.apus_hip_fp8_gemm_dev(tw.ptr, dws.ptr, dc.ptr, ds.ptr, y2.ptr, M, O, K, 1 | hip.W_TILED),
               "fp8_gemm_dev")
    hip._check(L.apus_hip_synchronize(), "sync")
    a, b = y1.to_array(np.float32, (M, O)), y2.to_array(np.float32, (M, O))
    assert np.array_equal(np.isnan(a), np.isnan(b))
    fin = ~np.isnan(a)
    assert np.array_equal(a[fin].view(np.uint32), b[fin].view(np.uint32))
    assert np.isnan(a[0]).all()                           # row 0 holds an infinity
    assert np.isfinite(a[1:]).all()

