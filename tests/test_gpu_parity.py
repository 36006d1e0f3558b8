"""GPU parity: libapus_hip.so (through its C ABI) against the CPU oracle.

Bars (written into each test):
  * activation codes/scales: bit-exact;
  * raw GEMM outputs (FP32): max|d|/max|ref| <= 1e-3 (BASELINE) and per-output
    err/esc <= 1e-4 vs the float64 truth. The reference gates its sequential
    FP32 CPU kernels at err/esc < 2e-5 (tests/m3/test_fp4.c:365-503); the
    F8F6F4 matrix cores accumulate each 128-wide block in their own order and
    precision, measured at err/esc ~2e-5 on gfx950, hence the 5x margin;
  * BF16-rounded linear outputs: each element within one BF16 ulp of the
    oracle's unrounded fp32 value plus 1e-4*max|ref| (the sums differ only in
    summation order, so a value near a rounding boundary may round the other
    way), and max|d|/max|ref| <= 1e-3 + 2^-8 (one BF16 ulp) overall.
"""
import numpy as np
import pytest

from helpers import (acts, bf16_linear_ok, err_esc, fp4_weights, fp4_weights_corners,
                     fp8_weights, max_rel)

pytestmark = pytest.mark.gpu


def test_device_is_gfx950(hip):
    name, cus = hip.device_info()
    print("device:", name, "CUs:", cus)
    assert "gfx950" in name


@pytest.mark.parametrize("M,K", [(1, 128), (3, 256), (7, 4096), (64, 2048)])
def test_act_quant_bitexact(hip, oracle, rng, M, K):
    x = acts(rng, M, K, 3.0)
    x[0, :128] = 0.0                       # zero group -> amax floor path
    if M > 1:
        x[1, 128 % K:] *= 100.0            # large later groups
    x[-1, 5] = 1e-30                       # tiny value next to normal ones
    c_ref, s_ref = oracle.act_quant(x)
    c, s = hip.act_quant(x)
    assert np.array_equal(c, c_ref)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("M,O,K", [(1, 16, 128), (1, 64, 512), (3, 64, 256), (5, 40, 640),
                                   (1, 2048, 4096), (16, 256, 4096), (33, 96, 1024)])
def test_fp4_gemm(hip, oracle, rng, M, O, K):
    w, ws = fp4_weights_corners(rng, O, K)
    x = acts(rng, M, K, 3.0)
    c, s = oracle.act_quant(x)
    want = oracle.fp4_gemm(w, ws, c, s)
    truth, esc = oracle.fp4_truth(w, ws, c, s)
    got = hip.fp4_gemm(w, ws, c, s)
    mr, ee = max_rel(got, want), err_esc(got, truth, esc)
    print(f"fp4 gemm M={M} O={O} K={K}: max_rel={mr:.3g} err/esc={ee:.3g}")
    assert mr <= 1e-3
    assert ee <= 1e-4


@pytest.mark.parametrize("M,O,K", [(1, 128, 128), (2, 130, 384), (1, 4096, 4096),
                                   (17, 256, 1024)])
def test_fp8_gemm(hip, oracle, rng, M, O, K):
    w, ws = fp8_weights(rng, O, K)
    x = acts(rng, M, K, 2.0)
    c, s = oracle.act_quant(x)
    want = oracle.fp8_gemm(w, ws, c, s)
    truth, esc = oracle.fp8_truth(w, ws, c, s)
    got = hip.fp8_gemm(w, ws, c, s)
    mr, ee = max_rel(got, want), err_esc(got, truth, esc)
    print(f"fp8 gemm M={M} O={O} K={K}: max_rel={mr:.3g} err/esc={ee:.3g}")
    assert mr <= 1e-3
    assert ee <= 1e-4


def _check_linear(got, want, unrounded, tag):
    ok = bf16_linear_ok(got, unrounded, 1e-4 * np.abs(unrounded).max())
    flips = float(np.mean(got != want))
    mr = max_rel(got, want)
    print(f"{tag}: bf16 flips vs oracle {flips:.2%}, max_rel={mr:.3g}")
    assert ok.all(), np.argwhere(~ok)[:5]
    assert mr <= 1e-3 + 2.0 ** -8


# M <= 8 with K 2048/4096 runs the one-launch path (act quant inside the
# GEMM staging); the other shapes quantise first
@pytest.mark.parametrize("M,O,K", [(1, 2048, 4096), (4, 4096, 2048), (8, 256, 2048), (9, 2048, 4096),
                                   (1, 512, 8192), (3, 256, 1024)])
def test_fp4_linear(hip, oracle, rng, M, O, K):
    w, ws = fp4_weights(rng, O, K)
    x = acts(rng, M, K)
    want = oracle.fp4_linear(w, ws, x)
    c, s = oracle.act_quant(x)
    got = hip.fp4_linear(w, ws, x)
    _check_linear(got, want, oracle.fp4_gemm(w, ws, c, s), f"fp4 linear M={M} O={O} K={K}")


@pytest.mark.parametrize("M,O,K", [(1, 4096, 4096), (8, 4096, 2048), (3, 256, 512), (12, 1024, 4096),
                                   (1, 1024, 8192), (8, 512, 8192), (4, 512, 1024), (1, 2048, 1024)])
def test_fp8_linear(hip, oracle, rng, M, O, K):
    w, ws = fp8_weights(rng, O, K)
    x = acts(rng, M, K)
    want = oracle.fp8_linear(w, ws, x)
    c, s = oracle.act_quant(x)
    got = hip.fp8_linear(w, ws, x)
    _check_linear(got, want, oracle.fp8_gemm(w, ws, c, s), f"fp8 linear M={M} O={O} K={K}")


def test_fp4_gemm_m_independent(hip, oracle, rng):
    """Within a schedule, a row's result does not depend on the batch (the
    reference's M-independence gate, tests/m12/README.md:331-354): up to 8
    rows (split-K schedule) and more than 8 rows (tile schedule) are each
    checked bitwise. Across the two schedules the K split differs, so the
    bits may differ within the GEMM tolerance."""
    O, K = 256, 2048
    w, ws = fp4_weights(rng, O, K)
    c, s = oracle.act_quant(acts(rng, 40, K))
    big = hip.fp4_gemm(w, ws, c, s)                         # tile schedule
    mid = hip.fp4_gemm(w, ws, c[5:25].copy(), s[5:25].copy())
    assert np.array_equal(mid.view(np.uint32), big[5:25].view(np.uint32))
    few = hip.fp4_gemm(w, ws, c[:6].copy(), s[:6].copy())  # few-row schedule
    for m in (0, 5):
        one = hip.fp4_gemm(w, ws, c[m:m + 1].copy(), s[m:m + 1].copy())
        assert np.array_equal(one.view(np.uint32), few[m:m + 1].view(np.uint32))
    assert max_rel(few, big[:6]) <= 1e-3


@pytest.mark.parametrize("fmt,M,O,K", [("fp8", 100, 256, 4096), ("fp8", 64, 384, 2048),
                                       ("fp4", 77, 256, 4096), ("fp4", 9, 128, 2048),
                                       ("fp8", 70, 256, 8192), ("fp8", 33, 128, 1024),
                                       ("fp4", 20, 256, 1024), ("fp4", 65, 128, 8192)])
def test_gemm_tile_schedule(hip, oracle, rng, fmt, M, O, K):
    """More than 8 rows, K 1024/2048/4096/8192: the 64 x 128 tile schedule,
    ragged M."""
    c, s = oracle.act_quant(acts(rng, M, K, 2.0))
    if fmt == "fp8":
        w, ws = fp8_weights(rng, O, K)
        got, want = hip.fp8_gemm(w, ws, c, s), oracle.fp8_gemm(w, ws, c, s)
        truth, esc = oracle.fp8_truth(w, ws, c, s)
    else:
        w, ws = fp4_weights(rng, O, K)
        got, want = hip.fp4_gemm(w, ws, c, s), oracle.fp4_gemm(w, ws, c, s)
        truth, esc = oracle.fp4_truth(w, ws, c, s)
    assert max_rel(got, want) <= 1e-3
    assert err_esc(got, truth, esc) <= 1e-4


@pytest.mark.parametrize("fmt", ["fp4", "fp8"])
def test_linear_rows_independent(hip, rng, fmt):
    """Up to 8 rows: each row of a batched linear is bitwise the row computed
    alone (one-launch path)."""
    O, K = 1024, 4096
    w, ws = (fp4_weights if fmt == "fp4" else fp8_weights)(rng, O, K)
    x = acts(rng, 6, K)
    f = hip.fp4_linear if fmt == "fp4" else hip.fp8_linear
    full = f(w, ws, x)
    for m in (0, 5):
        one = f(w, ws, x[m:m + 1].copy())
        assert np.array_equal(one.view(np.uint32), full[m:m + 1].view(np.uint32))


def test_dense_cache_same_bytes_other_shape(hip, oracle, rng):
    """The dense weight cache is keyed by host pointer; the same buffer
    reused as a different (O, K) of equal size must not hit the copy laid out
    for the first shape (resident copies are MFMA-tiled per shape)."""
    w, ws = fp4_weights(rng, 2048, 4096)
    x1 = acts(rng, 1, 4096)
    got1 = hip.fp4_linear(w, ws, x1)
    assert max_rel(got1, oracle.fp4_linear(w, ws, x1)) <= 1e-3 + 2.0 ** -8
    w2, ws2 = w.reshape(4096, 1024), ws.reshape(4096, 64)      # same memory
    assert w2.ctypes.data == w.ctypes.data and ws2.ctypes.data == ws.ctypes.data
    x2 = acts(rng, 3, 2048)
    got2 = hip.fp4_linear(w2, ws2, x2)
    assert max_rel(got2, oracle.fp4_linear(w2, ws2, x2)) <= 1e-3 + 2.0 ** -8


def test_linear_host_staging_sizes(hip, oracle, rng):
    """Host-pointer calls alternate between transfers that go through the
    library's pinned staging buffer (up to 1 MB each) and larger ones that go
    straight to and from the caller's memory (x of 80 x 4096 fp32 = 1.3 MB,
    out of 80 x 4096 fp32), each result checked against the oracle, so a
    result staged for one call can never land in another call's buffer."""
    K = 4096
    w, ws = fp4_weights(rng, 4096, K)
    for M in (1, 80, 3, 80, 1):
        x = acts(rng, M, K)
        want = oracle.fp4_linear(w, ws, x)
        c, s = oracle.act_quant(x)
        got = hip.fp4_linear(w, ws, x)
        _check_linear(got, want, oracle.fp4_gemm(w, ws, c, s), f"fp4 linear staging M={M}")
