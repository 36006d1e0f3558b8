"""Input generators and error metrics shared by the tests.

Metrics follow the reference's own gates:
  * max_rel  = max|got - want| / max|want|   (BASELINE tolerance 1e-3)
  * err/esc  per output, esc = sum of |block terms| (tests/m3/test_fp4.c:67-100,
             tests/m4a/README.md:78-83); the reference asserts < 2e-5.
"""
import numpy as np


# lines a test wants in the run's log whatever the capture mode (printed by
# tests/conftest.py at the end of the session)
SUMMARY_LINES = []


def fp4_weights(rng, O, K, lo=118, hi=130):
    """MXFP4 weight [O, K/2] with uniform nibbles and E8M0 bytes in lo..hi."""
    w = rng.integers(0, 256, (O, K // 2), dtype=np.uint8)
    ws = rng.integers(lo, hi + 1, (O, K // 32), dtype=np.uint8)
    return w, ws


def fp4_weights_corners(rng, O, K):
    """Random MXFP4 weights plus the corner blocks of tests/m3/gen_golden.py:179-204:
    an all-zero block under a huge scale, +6 and -6 saturation blocks, mixed
    0/0.5 codes, and extreme E8M0 bytes 0, 1, 200, 254."""
    w, ws = fp4_weights(rng, O, K)
    nb = K // 32
    w[0, 0:16] = 0x00
    ws[0, 0] = 200
    w[1 % O, 16:32] = 0x77
    w[2 % O, 32:48] = 0xFF
    w[3 % O, 48:64] = 0x10
    ws[4 % O, min(4, nb - 1)] = 0
    ws[5 % O, min(5, nb - 1)] = 1
    # 2^127 only on an all-zero block: a nonzero block would overflow to inf
    # in the CPU fold, outside the finite contract of both implementations
    b = min(6, nb - 1)
    w[6 % O, b * 16:(b + 1) * 16] = 0x00
    ws[6 % O, b] = 254
    return w, ws


def fp8_weights(rng, O, K, lo=117, hi=123):
    """E4M3 weight [O, K] = e4m3(clamp(N(0,1))) via the oracle's quantiser and
    tile scales [ceil(O/128), K/128] in lo..hi."""
    v = np.clip(rng.standard_normal((O, K)).astype(np.float32), -448, 448)
    w = e4m3_np(v)
    ws = rng.integers(lo, hi + 1, ((O + 127) // 128, K // 128), dtype=np.uint8)
    return w, ws


def e4m3_np(v):
    """Vectorised E4M3 RNE encode (same rule as orc_e4m3_quant) for big inputs."""
    v = np.clip(np.asarray(v, np.float32), -448, 448)
    u = v.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint32)
    a = u & 0x7FFFFFFF
    normal = a >= 0x3C800000
    rn = (((a.astype(np.uint64) + 0x7FFFF + ((a >> 20) & 1)) >> 20) - 960).astype(np.uint32)
    sub = np.rint(a.view(np.float32) * np.float32(512)).astype(np.uint32)
    return (sign | np.where(normal, rn, sub)).astype(np.uint8)


def acts(rng, M, K, scale=1.0):
    return (rng.standard_normal((M, K)) * scale).astype(np.float32)


def bf16(x):
    from pyoracle import bf16_round_np
    return bf16_round_np(x)


def max_rel(got, want):
    want = np.asarray(want, np.float64)
    d = np.abs(np.asarray(got, np.float64) - want).max()
    m = np.abs(want).max()
    return float(d / m) if m > 0 else float(d)


def err_esc(got, truth, esc):
    e = np.abs(np.asarray(got, np.float64) - truth)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(esc > 0, e / esc, np.where(e == 0, 0.0, np.inf))
    return float(r.max())


def bf16_ulp_diff(got, want):
    """Max distance in BF16 ulps between BF16-valued fp32 arrays."""
    def key(a):
        u = (np.asarray(a, np.float32).view(np.uint32) >> 16).astype(np.int64)
        return np.where(u & 0x8000, -(u & 0x7FFF), u)
    return int(np.abs(key(got) - key(want)).max())


def moe_experts(rng, E, dim, inter):
    """E routed experts: (w1, w1s, w2, w2s, w3, w3s)."""
    out = []
    for _ in range(E):
        w1, w1s = fp4_weights(rng, inter, dim)
        w2, w2s = fp4_weights(rng, dim, inter)
        w3, w3s = fp4_weights(rng, inter, dim)
        out.append((w1, w1s, w2, w2s, w3, w3s))
    return out


def topk_routing(rng, s, E, topk):
    """Seeded N(0,1) gating logits, top-k by logit, softmax over the chosen k
    (BASELINE config 2)."""
    logits = rng.standard_normal((s, E)).astype(np.float32)
    idx = np.argsort(-logits, axis=1, kind="stable")[:, :topk].astype(np.int32)
    sel = np.take_along_axis(logits, idx, axis=1).astype(np.float64)
    w = np.exp(sel - sel.max(axis=1, keepdims=True))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return idx, w


def bf16_linear_ok(got, v, abs_tol):
    """Elementwise bar for BF16-rounded linear outputs against the oracle's
    unrounded fp32 value v: |got - v| <= one BF16 ulp of v + abs_tol.
    A linear's output is bf16(sum); two implementations whose fp32 sums
    differ by summation order (bounded by abs_tol) round to values at most
    one BF16 ulp (2^-7 relative at worst) plus that difference apart."""
    v = np.asarray(v, np.float64)
    av = np.abs(v)
    ulp = np.where(av > 0, np.exp2(np.floor(np.log2(np.where(av > 0, av, 1.0))) - 7), 0.0)
    return np.abs(np.asarray(got, np.float64) - v) <= ulp + abs_tol
