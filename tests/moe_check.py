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

A systematic error in one expert (a wrong scale, index or operand) moves
far more than DELTA * esc and fails one of these.
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


def bf16_interval(truth, esc, delta=DELTA):
    """BF16 values an fp32 sum within delta*esc of truth can round to, as
    the closed interval [lo, hi] (rounding is monotone)."""
    lo, hi = _f32_out(truth - delta * esc, truth + delta * esc)
    return bf16(lo).astype(np.float64), bf16(hi).astype(np.float64)


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


def stage_a(g_truth, g_esc, u_truth, u_esc, limit, codes, e8m0):
    """Check the GPU's h codes [N] and E8M0 bytes [N/128] of one pair against
    the intervals the w1/w3 truth allows. Returns (n_exact, n_pinned, n)."""
    N = g_truth.shape[0]
    glo, ghi = bf16_interval(g_truth, g_esc)
    ulo, uhi = bf16_interval(u_truth, u_esc)
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


def stage_bc(eo_truth, eo_esc, wgt, y_gpu):
    """eo_truth / eo_esc [topk, dim] of one token (from the GPU's own h),
    wgt [topk]; y_gpu [dim]. Returns (n_bitexact_required, dim)."""
    lo, hi = bf16_interval(eo_truth, eo_esc)
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
    return int(pinned.sum()), eo_truth.shape[1], mr


def check_token(oracle, experts_of, x_row, idx_row, wgt_row, limit, h_codes, h_e8m0, y_gpu):
    """Stages A, B, C for one token. experts_of(e) -> (w1, w1s, w2, w2s, w3,
    w3s) row-major; h_codes [topk, inter], h_e8m0 [topk, inter/128] from the
    GPU; y_gpu [dim]. Returns a dict of counts."""
    xc, xs = oracle.act_quant(bf16(x_row[None, :].astype(np.float32)))
    topk = len(idx_row)
    a_exact = a_pinned = a_n = 0
    eo_t, eo_e = [], []
    for j in range(topk):
        w1, w1s, w2, w2s, w3, w3s = experts_of(int(idx_row[j]))
        gt, ge = oracle.fp4_truth(w1, w1s, xc, xs)
        ut, ue = oracle.fp4_truth(w3, w3s, xc, xs)
        ex, pn, n = stage_a(gt[0], ge[0], ut[0], ue[0], limit, h_codes[j], h_e8m0[j])
        a_exact += ex
        a_pinned += pn
        a_n += n
        hsc = np.exp2(h_e8m0[j].astype(np.float64) - 127.0).astype(np.float32)[None, :]
        et, ee = oracle.fp4_truth(w2, w2s, np.ascontiguousarray(h_codes[j][None, :]), hsc)
        eo_t.append(et[0])
        eo_e.append(ee[0])
    b_pinned, dim, mr = stage_bc(np.stack(eo_t), np.stack(eo_e), wgt_row, y_gpu)
    assert a_exact == a_pinned
    return {"h_pinned": a_pinned / a_n, "y_pinned": b_pinned / dim, "y_max_rel": mr}
