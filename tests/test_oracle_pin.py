"""Pin the CPU oracle (oracle/apus_oracle.c) before trusting it as the checker.

Each function of the restatement is checked three ways where possible:
  * bitwise against apus's own C kernels compiled from the apus sources
    (oracle/_ref/libapus_ref.so; skipped where that library is absent);
  * against what the mathematics fixes (exhaustive enumeration, brute-force
    nearest-value search, float64 truth, closed forms);
  * against invariants a plausible mistake would break.
CPU only.
"""
import concurrent.futures as cf
import ctypes as C
import math

import numpy as np
import pytest

from helpers import acts, fp4_weights, fp4_weights_corners, fp8_weights, moe_experts

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


def _exhaustive(oracle, which, fnptr, threads=8):
    """Run orc_pin_unary over all 2^32 inputs split across threads (ctypes
    releases the GIL during the call)."""
    step = (1 << 32) // threads
    with cf.ThreadPoolExecutor(threads) as ex:
        futs = [ex.submit(oracle.pin_unary, which, fnptr, i * step, (i + 1) * step)
                for i in range(threads)]
        res = [f.result() for f in futs]
    return sum(r[0] for r in res), [r[1] for r in res if r[0]]


# ----------------------------------------------------------------- scalars

def test_bf16_round_exhaustive_vs_reference(oracle, ref):
    bad, first = _exhaustive(oracle, 0, C.cast(ref.L.apus_bf16_round, C.c_void_p))
    assert bad == 0, [hex(x) for x in first]


def test_e4m3_quant_exhaustive_vs_reference(oracle, ref):
    bad, first = _exhaustive(oracle, 1, C.cast(ref.L.apus_e4m3_quant_f32, C.c_void_p))
    assert bad == 0, [hex(x) for x in first]


def _e4m3_values():
    return np.array([math.ldexp(1.0 + (c & 7) / 8.0, ((c >> 3) & 15) - 7) if (c >> 3) & 15
                     else (c & 7) * 2.0 ** -9 for c in range(128)])


def test_e4m3_quant_bruteforce_nearest(oracle):
    """The code is the nearest E4M3 value to clamp(x, +-448), ties to the even
    code — found by searching all 127 finite magnitudes (0x7F excluded)."""
    vals = _e4m3_values()[:127]
    rng = np.random.default_rng(5)
    xs = np.concatenate([rng.standard_normal(4000) * 50, rng.standard_normal(2000) * 0.01,
                         (rng.integers(0, 127, 2000) + 0.5).astype(np.float64),   # near ties
                         [(vals[i] + vals[i + 1]) / 2 for i in range(126)],       # exact ties
                         [448.0, 449.0, 464.0, 1e30, 2.0 ** -10, 2.0 ** -11, 0.0]])
    for x in xs.astype(np.float32):
        xa = min(abs(float(x)), 448.0)
        d = np.abs(vals - xa)
        best = np.flatnonzero(d == d.min())
        want = best[0] if len(best) == 1 else [b for b in best if b % 2 == 0][0]
        got = oracle.L.orc_e4m3_quant(float(x))
        assert (got & 0x7F) == want, (x, got, want)
        if x < 0:
            assert got & 0x80


def test_e4m3_dequant_all_codes(oracle, ref):
    vals = _e4m3_values()
    for c in range(256):
        v = oracle.e4m3_dequant(c)
        assert v == ref.L.apus_e4m3_dequant_f32(c)
        want = (480.0 if (c & 0x7F) == 0x7F else vals[c & 0x7F]) * (-1 if c & 0x80 else 1)
        assert v == want, c
    assert oracle.e4m3_dequant(0x7E) == 448.0 and oracle.e4m3_dequant(1) == 2.0 ** -9


def test_ue8m0_closed_form(oracle, ref):
    for b in range(256):
        v = oracle.ue8m0(b)
        assert v == ref.L.apus_ue8m0_f32(b)
        if b == 255:
            assert math.isinf(v)
        else:
            assert v == math.ldexp(1.0, b - 127), b


def test_fp4_values_and_dequant_exhaustive(oracle, ref):
    """E2M1 magnitudes are {0, .5, 1, 1.5, 2, 3, 4, 6} with bit 3 the sign;
    every (byte, scale byte) pair dequantises exactly (product of two
    representable numbers) and bitwise like the reference row dequant."""
    mags = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for n in range(16):
        assert oracle.fp4_value(n) == (-1 if n & 8 else 1) * mags[n & 7]
        assert math.copysign(1.0, oracle.fp4_value(n)) == (-1.0 if n & 7 and n & 8 else 1.0)
    packed = np.arange(256, dtype=np.uint8)
    packed = np.tile(packed, 1)              # 256 bytes = 512 elements = 16 groups
    for sb in range(0, 256, 1):
        scales = np.full(16, sb, np.uint8)
        got = oracle.fp4_dequant_row(packed, scales)
        want = np.empty(512, np.float32)
        ref.L.apus_fp4_dequant_row_scalar(packed.ctypes.data_as(C.POINTER(C.c_uint8)),
                                          scales.ctypes.data_as(C.POINTER(C.c_uint8)),
                                          want.ctypes.data_as(C.POINTER(C.c_float)), 512)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), sb
        if sb < 255:
            lo = np.array([mags[b & 7] * (-1 if b & 8 else 1) for b in packed & 15])
            # exact in fp32 (or +-inf where the product passes FLT_MAX)
            with np.errstate(over="ignore"):
                assert np.array_equal(got[0::2], (lo * 2.0 ** (sb - 127)).astype(np.float32))


# --------------------------------------------------------------- act quant

def _act_rows(rng, M, K):
    x = acts(rng, M, K, 3.0)
    x[0] = 0.0                                     # amax floor (1e-4)
    if M > 1:
        x[1, : min(K, 128)] *= 1e4                 # outliers in group 0
    if M > 2:
        x[2] = 1e-30                               # tiny everywhere
    if M > 3:
        x[3] = -np.abs(x[3])                       # all negative
    if M > 4:
        x[4, ::7] = 448.0 * 2.0 ** 3               # exact power-of-two amax
    return x


@pytest.mark.parametrize("M,K", [(6, 128), (6, 4096), (5, 160), (3, 96), (9, 2048)])
def test_act_quant_vs_reference(oracle, ref, rng, M, K):
    x = _act_rows(rng, M, K)
    c1, s1 = oracle.act_quant(x)
    c2, s2 = ref.act_quant(x)
    assert np.array_equal(c1, c2)
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))


def test_act_quant_invariants(oracle, rng):
    """Scales are powers of two with amax/s in (224, 448] (or the 1e-4 floor),
    and each code decodes to within half an E4M3 step of x/s."""
    from helpers import bf16
    M, K = 16, 1024
    x = _act_rows(rng, M, K)
    codes, sc = oracle.act_quant(x)
    xb = bf16(x)
    deq = np.vectorize(oracle.e4m3_dequant)(codes).astype(np.float64)
    for m in range(M):
        for b in range(K // 128):
            s = float(sc[m, b])
            assert math.frexp(s)[0] == 0.5                     # power of two
            blk = xb[m, b * 128:(b + 1) * 128].astype(np.float64)
            amax = max(np.abs(blk).max(), 1e-4)
            r = amax / s
            assert 224.0 <= r <= 448.0 * (1 + 2 ** -20), (m, b, r)
            y = blk / s
            step = np.where(np.abs(y) < 2 ** -6, 2.0 ** -9,
                            2.0 ** (np.floor(np.log2(np.maximum(np.abs(y), 2 ** -6))) - 3))
            assert np.all(np.abs(deq[m, b * 128:(b + 1) * 128] - y) <= step / 2 + 1e-12)


# ------------------------------------------------------------------- GEMMs

@pytest.mark.parametrize("M,O,K", [(3, 64, 256), (1, 96, 4096), (5, 33, 640), (8, 130, 128)])
def test_fp4_gemm_vs_reference_and_truth(oracle, ref, rng, M, O, K):
    w, ws = fp4_weights_corners(rng, O, K)
    c, s = oracle.act_quant(acts(rng, M, K, 3.0))
    got = oracle.fp4_gemm(w, ws, c, s)
    for want in (ref.fp4_gemm_scalar(w, ws, c, s), ref.fp4_gemm_mt(w, ws, c, s)):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    truth, esc = oracle.fp4_truth(w, ws, c, s)
    err = np.abs(got - truth)
    assert np.all(err <= 2e-5 * esc + 1e-30)


@pytest.mark.parametrize("M,O,K", [(8, 320, 384), (1, 256, 4096), (3, 129, 256)])
def test_fp8_gemm_vs_reference_and_truth(oracle, ref, rng, M, O, K):
    w, ws = fp8_weights(rng, O, K)
    w[0, :128] = 0                                   # zero tile row
    w[1, :16] = 0x7E                                 # +448
    w[2, :16] = 0xFE                                 # -448
    w[3, :16] = 0x01                                 # min subnormal
    ws[0, 0] = 0
    if ws.shape[1] > 1:
        ws[0, 1] = 1
    c, s = oracle.act_quant(acts(rng, M, K, 2.0))
    got = oracle.fp8_gemm(w, ws, c, s)
    for want in (ref.fp8_gemm_scalar(w, ws, c, s), ref.fp8_gemm_mt(w, ws, c, s)):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    truth, esc = oracle.fp8_truth(w, ws, c, s)
    assert np.all(np.abs(got - truth) <= 2e-5 * esc + 1e-30)


def test_linears_vs_reference(oracle, ref, rng):
    w4, ws4 = fp4_weights(rng, 128, 512)
    w8, ws8 = fp8_weights(rng, 256, 512)
    x = acts(rng, 9, 512)
    for got, want in ((oracle.fp4_linear(w4, ws4, x), ref.fp4_linear(w4, ws4, x)),
                      (oracle.fp8_linear(w8, ws8, x), ref.fp8_linear(w8, ws8, x))):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gemm_m_independent(oracle, rng):
    """Row m of a batched GEMM equals the same row computed alone (the
    reference's bitwise M-independence, tests/m12/README.md:331-354)."""
    w, ws = fp4_weights(rng, 64, 512)
    c, s = oracle.act_quant(acts(rng, 6, 512))
    full = oracle.fp4_gemm(w, ws, c, s)
    for m in range(6):
        one = oracle.fp4_gemm(w, ws, c[m:m + 1].copy(), s[m:m + 1].copy())
        assert np.array_equal(one, full[m:m + 1])


# --------------------------------------------------------------------- MoE

def test_swiglu_vs_reference_and_truth(oracle, ref, rng):
    g = (rng.standard_normal(20000) * 6).astype(np.float32)
    u = (rng.standard_normal(20000) * 6).astype(np.float32)
    g[:5] = [30.0, -30.0, 10.0, 0.0, -0.0]
    for limit in (10.0, 0.0):
        h = oracle.swiglu(g, u, limit)
        assert np.array_equal(h.view(np.uint32), ref.swiglu(g, u, limit).view(np.uint32))
        gg = g.astype(np.float64)
        uu = u.astype(np.float64)
        if limit > 0:
            uu = np.clip(uu, -limit, limit)
            gg = np.minimum(gg, limit)
        t = gg / (1 + np.exp(-gg)) * uu
        # BF16 output: within one BF16 ulp of the float64 value
        assert np.all(np.abs(h - t) <= np.abs(t) * 2.0 ** -7 + 1e-30)


@pytest.mark.parametrize("s,topk", [(1, 6), (5, 3), (20, 4)])
def test_moe_routed_vs_reference(oracle, ref, rng, s, topk):
    E, dim, inter = 8, 256, 256
    experts = moe_experts(rng, E, dim, inter)
    gate = (rng.standard_normal((E, dim)) * 0.05).astype(np.float32)
    from helpers import bf16
    x = bf16(acts(rng, s, dim))
    idx = np.stack([rng.choice(E, topk, replace=False) for _ in range(s)]).astype(np.int32)
    rw, ry = ref.moe_routed(experts, gate, x, idx, 1.5, 10.0)
    oy = oracle.moe_routed(experts, x, idx, rw, 10.0)
    assert np.array_equal(oy.view(np.uint32), ry.view(np.uint32))


def test_moe_routed_batched_equals_per_token(oracle, rng):
    E, dim, inter, s, topk = 6, 256, 128, 4, 2
    experts = moe_experts(rng, E, dim, inter)
    x = acts(rng, s, dim)
    idx = np.stack([rng.choice(E, topk, replace=False) for _ in range(s)]).astype(np.int32)
    wgt = rng.random((s, topk)).astype(np.float32)
    full = oracle.moe_routed(experts, x, idx, wgt, 10.0)
    for t in range(s):
        one = oracle.moe_routed(experts, x[t:t + 1], idx[t:t + 1], wgt[t:t + 1], 10.0)
        assert np.array_equal(one, full[t:t + 1])


# ---------------------------------------------------------------- generator

def test_fill_bytes_ranges_and_determinism(oracle):
    n = 1 << 16
    a = oracle.fill_bytes(7, 3, n, 0)
    assert np.array_equal(a, oracle.fill_bytes(7, 3, n, 0))
    assert not np.array_equal(a, oracle.fill_bytes(7, 4, n, 0))
    # offset consistency: a window starting mid-stream matches
    assert np.array_equal(a[1000:2000], oracle.fill_bytes(7, 3, 1000, 0, first=1000))
    lo, hi = np.bincount(a & 15, minlength=16), np.bincount(a >> 4, minlength=16)
    assert lo.min() > n / 16 * 0.9 and hi.min() > n / 16 * 0.9
    s1 = oracle.fill_bytes(7, 5, n, 1)
    assert s1.min() == 118 and s1.max() == 130
    s3 = oracle.fill_bytes(7, 6, n, 3)
    assert s3.min() == 117 and s3.max() == 123
    w8 = oracle.fill_bytes(7, 8, n, 2)
    vals = np.vectorize(oracle.e4m3_dequant)(w8)
    assert abs(vals.mean()) < 0.05 and 0.9 < vals.std() < 1.1
    assert not np.any((w8 & 0x7F) == 0x7F)


def _moe_case(rng, E, dim, inter, s, topk, hash_):
    from helpers import acts, fp8_weights, moe_experts
    experts = moe_experts(rng, E, dim, inter)
    sw1, sw1s = fp8_weights(rng, inter, dim)
    sw2, sw2s = fp8_weights(rng, dim, inter)
    sw3, sw3s = fp8_weights(rng, inter, dim)
    cfg = {"E": E, "topk": topk, "dim": dim, "inter": inter, "route_scale": 2.5, "limit": 10.0,
           "hash": hash_, "gate_w": (rng.standard_normal((E, dim)) / np.sqrt(dim)).astype(np.float32),
           "gate_bias": (rng.standard_normal(E) * 0.05).astype(np.float32)}
    if hash_:
        cfg["tid2eid"] = np.stack([rng.choice(E, topk, replace=False) for _ in range(11)]).astype(np.int64)
        cfg["ids"] = rng.integers(0, 11, s).astype(np.int64)
    return cfg, experts, (sw1, sw1s, sw2, sw2s, sw3, sw3s), acts(rng, s, dim)


@pytest.mark.parametrize("s,hash_", [(1, 0), (5, 0), (3, 1)])
def test_moe_forward_restatement_vs_reference(oracle, ref, rng, s, hash_):
    """orc_moe_forward (router + routed + FP8 shared + final bf16 sum) equals
    the real apus_moe_forward bit for bit, intermediates included."""
    cfg, experts, shared, x = _moe_case(rng, 16, 256, 128, s, 4, hash_)
    got = oracle.moe_forward(cfg, experts, shared, x)
    want = ref.moe_forward(cfg, experts, shared, x)
    for name, a, b in zip(("out", "routed", "shared", "sp", "idx", "wgt"), got, want):
        assert np.array_equal(a.view(np.uint32) if a.dtype != np.int32 else a,
                              b.view(np.uint32) if b.dtype != np.int32 else b), name


@pytest.mark.parametrize("case", ["ties", "large"])
def test_router_edges_restatement_vs_reference(oracle, ref, rng, case):
    """Router edge cases, restatement vs the real apus_moe_forward: exact ties
    (identical gate rows, zero bias: the lowest indices win, in order) and
    gate dot products past 20 (softplus returns its argument)."""
    E, topk, s = 16, 4, 3
    cfg, experts, shared, x = _moe_case(rng, E, 256, 128, s, topk, 0)
    if case == "ties":
        cfg["gate_w"] = np.repeat(cfg["gate_w"][:1], E, axis=0)
        cfg["gate_bias"] = np.zeros(E, np.float32)
    else:
        cfg["gate_w"] = cfg["gate_w"] * 40.0
    got = oracle.moe_forward(cfg, experts, shared, x)
    want = ref.moe_forward(cfg, experts, shared, x)
    for name, a, b in zip(("out", "routed", "shared", "sp", "idx", "wgt"), got, want):
        assert np.array_equal(a.view(np.uint32) if a.dtype != np.int32 else a,
                              b.view(np.uint32) if b.dtype != np.int32 else b), name
    if case == "ties":
        assert np.array_equal(got[4], np.tile(np.arange(topk, dtype=np.int32), (s, 1)))
    else:
        dots = x.astype(np.float64) @ cfg["gate_w"].T.astype(np.float64)
        assert (dots > 20).any()


@pytest.mark.parametrize("M,K,O", [(1, 256, 37), (3, 1000, 20), (5, 4096, 9)])
def test_wlinear_restatement_vs_reference(oracle, ref, rng, M, K, O):
    """orc_wlinear equals the reference's plain-weight linears bit for bit:
    apus_f32_linear (flags 0), apus_bf16_linear (R_IN | R_OUT),
    apus_head_gemv over F32 and BF16 views (M = 1), and the BF16-weight form
    (W_BF16, used by the wo_a hook) equals apus_f32_linear on the exactly
    widened weights."""
    from helpers import bf16
    w = (rng.standard_normal((O, K)) / np.sqrt(K)).astype(np.float32)
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    assert np.array_equal(oracle.wlinear(w, x, 0).view(np.uint32), ref.f32_linear(w, x).view(np.uint32))
    assert np.array_equal(oracle.wlinear(w, x, 3).view(np.uint32), ref.bf16_linear(w, x).view(np.uint32))
    wb = (w.view(np.uint32) >> 16).astype(np.uint16)            # BF16 bits (truncated)
    widened = (wb.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(oracle.wlinear(wb, x, 6).view(np.uint32),
                          bf16(ref.f32_linear(widened, x)).view(np.uint32))
    assert np.array_equal(oracle.wlinear(w, x[:1], 0)[0].view(np.uint32),
                          ref.head_gemv(w, x[:1]).view(np.uint32))
    assert np.array_equal(oracle.wlinear(wb, x[:1], 4)[0].view(np.uint32),
                          ref.head_gemv(wb, x[:1]).view(np.uint32))
    truth, esc = oracle.wlinear_truth(w, x, 0)
    got = oracle.wlinear(w, x, 0).astype(np.float64)
    assert np.all(np.abs(got - truth) <= K * 2.0 ** -24 * esc + 1e-30)


def test_ref_decode_layer_vs_oracle(oracle, ref, rng):
    """The config-4 CPU baseline's layer (ref_decode_layer: apus's own
    apus_fp8_linear and the one-token routed loop of apus_moe_forward)
    equals the oracle's FP8 linear and routed dispatch bit for bit."""
    from pyoracle import ref_decode_layer
    dim, inter, topk = 512, 256, 6
    experts = moe_experts(rng, topk, dim, inter)
    pw, pws = fp8_weights(rng, dim, dim)
    x = acts(rng, 1, dim)
    wgt = rng.random(topk).astype(np.float32)
    y, proj = ref_decode_layer(ref, experts, wgt, pw, pws, x, 10.0)
    want_y = oracle.moe_routed(experts, x, np.arange(topk, dtype=np.int32)[None, :], wgt[None, :], 10.0)
    want_p = oracle.fp8_linear(pw, pws, x)
    assert np.array_equal(y.view(np.uint32), want_y[0].view(np.uint32))
    assert np.array_equal(proj.view(np.uint32), want_p[0].view(np.uint32))
