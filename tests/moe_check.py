"""Per-element parity of the routed-expert dispatch, stage by stage.

The dispatch computes, for token t and its routed pair j (expert e, weight w):
    g, u = bf16(w1 x), bf16(w3 x)                    (c/moe.h:282-300, :198-209)
    h    = act_quant(bf16(silu(min(g, L)) * clamp(u, +-L)))   (:113-126, :309-314)
    eo   = bf16(w2 h)                                 (:316-325)
    y[t] = sum_j w_j * eo_j, mul then add, j order    (:148-158, :447-449)
The GPU forms every block sum on the matrix cores in its own order, so an
unrounded sum differs from the exact one by at most DELTA * esc, where esc =
sum of |block terms| (the reference's error measure, tests/m3/test_fp4.c:
67-100; measured on gfx950 about 2e-5, the GEMM bar is 1e-4). Each check
below turns that bound into the exact set of values a correct implementation
may produce at the next rounding point, from the oracle's float64 truth:

  stage A (w1, w3, SwiGLU, act quant): for every element, the interval of
    BF16 values g and u can round to, the interval of h over those (plus a
    2^-19 relative allowance for expf from another libm), the interval of
    group scales the group's |h| maximum allows, and, under the GPU's own
    scale, the interval of E4M3 codes. The GPU's scale byte and every code
    must lie in them; where an interval is a single value (no rounding
    boundary within reach) the GPU must match exactly.
  stage B (w2) and C (accumulation): the oracle recomputes eo from the GPU's
    own h codes, so the only freedom left is the w2 block-sum order: eo lies
    in the BF16 interval of truth +- DELTA * esc, and y[t, o] must equal the
    sequential fp32 sum bit for bit wherever every eo_j is pinned to one
    value, and lie within the weighted interval (plus fp32 rounding of the
    sum) elsewhere.

The matrix cores add the 32 products of a scale block in a fixed-point
window about 13 bits below the block's largest product (measured on gfx950:
2^8 + 2^-5 is exact, 2^8 + 2^-6 gives 2^8; products in different blocks add
in fp32): a product more than 2^13 below the block's largest can vanish, and
partial sums of such products lose their bits below the window. mfma_slack()
bounds that loss per output from the operands (a product with all its bits in
the window is exact; only the smaller ones can lose, and never more than
themselves or one window LSB per adder), and every interval below is widened
by it on top of DELTA * esc.

A systematic error in one expert (a wrong scale, index or operand) moves
far more than these bounds and fails one of these.
"""
import numpy as np

from helpers import bf16, e4m3_np

DELTA = 1e-4          # |unrounded GPU sum - exact| <= DELTA * esc (GEMM bar)
EXPF_REL = 2.0 ** -19  # relative slack of the fp32 SwiGLU element (libm expf)


def _f32_out(lo, hi):
    """float32 interval containing the float64 interval [lo, hi]."""
    lo32 = np.nextafter(np.asarray(lo, np.float64).astype(np.float32), np.float32(-np.inf))
    hi32 = np.nextafter(np.asarray(hi, np.float64).astype(np.float32), np.float32(np.inf))
    return lo32, hi32


def bf16_interval(truth, esc, delta=DELTA, extra=0.0):
    """BF16 values an fp32 sum within delta*esc + extra of truth can round
    to, as the closed interval [lo, hi] (rounding is monotone)."""
    lo, hi = _f32_out(truth - delta * esc - extra, truth + delta * esc + extra)
    return bf16(lo).astype(np.float64), bf16(hi).astype(np.float64)


E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])
WINDOW = 13          # bits kept below a block's largest product (measured)


def mfma_slack_np(w, ws, codes, scales):
    """Per output o: a bound on what the matrix cores' block-wise fixed-point
    addition can lose in sum_k W[o, k] * A[k] (one activation row), for MXFP4
    weights w [O, K/2] (low nibble first) with E8M0 scales ws [O, K/32] and
    E4M3 codes [K] with fp32 scales [K/128]. For each 32-block: LSB =
    2^(exponent of the largest |product| - WINDOW); a product of at least
    32 LSB (E4M3 x E2M1 significands: at most 6 bits) lies on the window's
    grid and is exact; each smaller product enters one addition, which can
    lose at most the product itself or one LSB, so the block loses at most
    min(sum of the smaller |products|, their count x LSB)."""
    O = w.shape[0]
    K = codes.shape[-1]
    wv = np.empty((O, K), np.float64)
    wv[:, 0::2] = E2M1[w & 0xF]
    wv[:, 1::2] = E2M1[w >> 4]
    wv *= np.repeat(np.exp2(ws.astype(np.float64) - 127.0), 32, axis=1)
    av = E4M3[np.asarray(codes).reshape(K)] * np.repeat(np.asarray(scales, np.float64).reshape(-1), 128)
    t = np.abs(wv * av[None, :]).reshape(O, K // 32, 32)
    mx = t.max(axis=2)
    with np.errstate(divide="ignore"):
        lsb = np.where(mx > 0, np.exp2(np.floor(np.log2(np.where(mx > 0, mx, 1.0))) - WINDOW), 0.0)
    sm = t < 32.0 * lsb[:, :, None]
    small = np.where(sm, t, 0.0).sum(axis=2)
    return np.minimum(small, sm.sum(axis=2) * lsb).sum(axis=1)


def mfma_slack(w, ws, codes, scales):
    """mfma_slack_np computed by the oracle library's C loop (the same bound,
    about 100x faster; the two are pinned against each other in
    tests/test_moe_check.py)."""
    from pyoracle import Oracle
    global _ORC
    if _ORC is None:
        _ORC = Oracle()
    return _ORC.fp4_mfma_slack(w, ws, codes, scales, WINDOW)


_ORC = None


def act_scale_exp(amax):
    """Biased exponent of the per-128 activation scale (c/fp4.h:300-317):
    amax floored at 1e-4, p = amax * fl(1/448), 2^ceil(log2 p) from p's bits."""
    a = np.maximum(np.asarray(amax, np.float32), np.float32(1e-4))
    pb = (a * np.float32(1.0 / 448.0)).astype(np.float32).view(np.uint32)
    return ((pb >> 23) & 0xFF).astype(np.int64) + ((pb & 0x7FFFFF) != 0)


def _e4m3_values():
    v = np.zeros(256, np.float64)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 3) & 0xF, c & 7
        v[c] = s * (m / 8.0) * 2.0 ** -6 if e == 0 else s * (1 + m / 8.0) * 2.0 ** (e - 7)
    return v


E4M3 = _e4m3_values()


def _silu_mul(g, u):
    return (g * (1.0 / (1.0 + np.exp(-g)))) * u


# silu(g) = g * sigmoid(g) falls to its minimum at g = -1.278464542761074
# and rises on both sides of it
SILU_ARGMIN = -1.278464542761074


def stage_a(g_truth, g_esc, u_truth, u_esc, limit, codes, e8m0, g_slack=0.0, u_slack=0.0):
    """Check the GPU's h codes [N] and E8M0 bytes [N/128] of one pair against
    the intervals the w1/w3 truth allows. Returns (n_exact, n_pinned, n)."""
    N = g_truth.shape[0]
    glo, ghi = bf16_interval(g_truth, g_esc, extra=g_slack)
    ulo, uhi = bf16_interval(u_truth, u_esc, extra=u_slack)
    if limit > 0:
        glo, ghi = np.minimum(glo, limit), np.minimum(ghi, limit)
        ulo, uhi = np.clip(ulo, -limit, limit), np.clip(uhi, -limit, limit)
    # h = silu(g) * u over the box [glo, ghi] x [ulo, uhi]: linear in u, and
    # in g monotone on either side of silu's minimum, so its extremes lie at
    # the corners or at g = SILU_ARGMIN (the continuous hull contains every
    # value the BF16 inputs of the box can give)
    gin = np.clip(SILU_ARGMIN, glo, ghi)
    hs = []
    with np.errstate(over="ignore"):
        for gc in (glo, ghi, gin):
            for uc in (ulo, uhi):
                hs.append(_silu_mul(gc, uc))
    hmin, hmax = np.min(hs, axis=0), np.max(hs, axis=0)
    lo, hi = _f32_out(hmin - np.abs(hmin) * EXPF_REL, hmax + np.abs(hmax) * EXPF_REL)
    hlo, hhi = bf16(lo).astype(np.float64), bf16(hi).astype(np.float64)
    G = N // 128
    alo = np.where((hlo <= 0) & (hhi >= 0), 0.0, np.minimum(np.abs(hlo), np.abs(hhi)))
    ahi = np.maximum(np.abs(hlo), np.abs(hhi))
    elo = act_scale_exp(alo.reshape(G, 128).max(1))
    ehi = act_scale_exp(ahi.reshape(G, 128).max(1))
    e = e8m0.astype(np.int64)
    bad = np.nonzero((e < elo) | (e > ehi))[0]
    assert bad.size == 0, f"scale bytes outside the allowed range at groups {bad[:8]}: " \
        f"gpu {e[bad[:8]]} allowed [{elo[bad[:8]]}, {ehi[bad[:8]]}]"
    inv = np.repeat(np.exp2(127.0 - e), 128)
    with np.errstate(invalid="ignore", over="ignore"):
        clo = E4M3[e4m3_np(np.clip(hlo * inv, -448.0, 448.0).astype(np.float32))]
        chi = E4M3[e4m3_np(np.clip(hhi * inv, -448.0, 448.0).astype(np.float32))]
    got = E4M3[codes]
    bad = np.nonzero((got < clo) | (got > chi))[0]
    assert bad.size == 0, f"h codes outside the allowed interval at {bad[:8]}: gpu {got[bad[:8]]} " \
        f"allowed [{clo[bad[:8]]}, {chi[bad[:8]]}]"
    pinned = (clo == chi) & np.repeat(elo == ehi, 128)
    return int(np.sum(pinned & (got == clo))), int(pinned.sum()), N


def stage_bc(eo_truth, eo_esc, wgt, y_gpu, eo_slack=0.0):
    """eo_truth / eo_esc [topk, dim] of one token (from the GPU's own h),
    wgt [topk]; y_gpu [dim]. Returns (n_bitexact_required, dim)."""
    lo, hi = bf16_interval(eo_truth, eo_esc, extra=eo_slack)
    pinned = np.all(lo == hi, axis=0)
    # the sequential fp32 accumulation the reference and the GPU both do
    y = np.zeros(eo_truth.shape[1], np.float32)
    for j in range(eo_truth.shape[0]):
        y = (y + (np.float32(wgt[j]) * lo[j].astype(np.float32)).astype(np.float32)).astype(np.float32)
    g = np.asarray(y_gpu, np.float32)
    bad = np.nonzero(pinned & (g.view(np.uint32) != y.view(np.uint32)))[0]
    assert bad.size == 0, f"y differs where every eo is pinned, at {bad[:8]}: {g[bad[:8]]} vs {y[bad[:8]]}"
    w = np.asarray(wgt, np.float64)[:, None]
    ylo = np.sum(np.minimum(w * lo, w * hi), axis=0)
    yhi = np.sum(np.maximum(w * lo, w * hi), axis=0)
    slack = eo_truth.shape[0] * 2.0 ** -23 * np.sum(np.abs(w) * np.maximum(np.abs(lo), np.abs(hi)), axis=0)
    gd = g.astype(np.float64)
    bad = np.nonzero((gd < ylo - slack) | (gd > yhi + slack))[0]
    assert bad.size == 0, f"y outside its interval at {bad[:8]}"
    # reported, not a bar: one BF16 flip of an eo moves y by w * ulp(eo),
    # up to a few 1e-3 of max|y| for the reference's own sum as well
    mr = float(np.abs(gd - y.astype(np.float64)).max() / max(np.abs(y).max(), 1e-30))
    return pinned, eo_truth.shape[1], mr


def check_token(oracle, experts_of, x_row, idx_row, wgt_row, limit, h_codes, h_e8m0, y_gpu):
    """Stages A, B, C for one token. experts_of(e) -> (w1, w1s, w2, w2s, w3,
    w3s) row-major; h_codes [topk, inter], h_e8m0 [topk, inter/128] from the
    GPU; y_gpu [dim]. Returns a dict of counts."""
    xc, xs = oracle.act_quant(bf16(x_row[None, :].astype(np.float32)))
    topk = len(idx_row)
    a_exact = a_pinned = a_n = 0
    eo_t, eo_e, eo_s = [], [], []
    for j in range(topk):
        w1, w1s, w2, w2s, w3, w3s = experts_of(int(idx_row[j]))
        gt, ge = oracle.fp4_truth(w1, w1s, xc, xs)
        ut, ue = oracle.fp4_truth(w3, w3s, xc, xs)
        ex, pn, n = stage_a(gt[0], ge[0], ut[0], ue[0], limit, h_codes[j], h_e8m0[j],
                            mfma_slack(w1, w1s, xc[0], xs[0]), mfma_slack(w3, w3s, xc[0], xs[0]))
        a_exact += ex
        a_pinned += pn
        a_n += n
        hsc = np.exp2(h_e8m0[j].astype(np.float64) - 127.0).astype(np.float32)[None, :]
        et, ee = oracle.fp4_truth(w2, w2s, np.ascontiguousarray(h_codes[j][None, :]), hsc)
        eo_t.append(et[0])
        eo_e.append(ee[0])
        eo_s.append(mfma_slack(w2, w2s, h_codes[j], hsc[0]))
    y_pin, dim, mr = stage_bc(np.stack(eo_t), np.stack(eo_e), wgt_row, y_gpu, np.stack(eo_s))
    assert a_exact == a_pinned
    return {"h_pinned": a_pinned / a_n, "y_pinned": float(y_pin.sum()) / dim, "y_max_rel": mr,
            "y_pinned_mask": y_pin}


def check_pair(oracle, expert, x_row, limit, h_codes, h_e8m0, eo_bf16=None):
    """Stage A (and, given the GPU's bf16 eo of the pair, stage B) for ONE
    routed pair: expert = (w1, w1s, w2, w2s, w3, w3s) row-major, h_codes
    [inter], h_e8m0 [inter/128]. Returns the fraction of h codes pinned."""
    xc, xs = oracle.act_quant(bf16(x_row[None, :].astype(np.float32)))
    w1, w1s, w2, w2s, w3, w3s = expert
    gt, ge = oracle.fp4_truth(w1, w1s, xc, xs)
    ut, ue = oracle.fp4_truth(w3, w3s, xc, xs)
    ex, pn, n = stage_a(gt[0], ge[0], ut[0], ue[0], limit, h_codes, h_e8m0,
                        mfma_slack(w1, w1s, xc[0], xs[0]), mfma_slack(w3, w3s, xc[0], xs[0]))
    assert ex == pn
    return pn / n
