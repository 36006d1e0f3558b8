/*
 * oracle/apus_oracle.c — CPU restatement of apus's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): see the header
 * for the pinning of every function. Built with -ffp-contract=off so that no
 * multiply-add pair is fused: the reference pins the same flag
 * (Makefile:21-27) and its two-rounding scale steps depend on it.
 */
#include "apus_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---------------------------------------------------------------- scalars */

float orc_ue8m0_f32(uint8_t b) {
    /* 2^(b-127) placed straight into the exponent field; the one byte whose
     * exponent field would be 0 (b=0) is the subnormal 2^-127 = mantissa
     * bit 22. b=255 lands on the all-ones exponent with a zero mantissa,
     * i.e. +inf. (c/fp4.h:209-217) */
    return b ? u2f((uint32_t)b << 23) : u2f(1u << 22);
}

float orc_fp4_value(unsigned nib) {
    /* E2M1: e=bits[2:1], m=bit0. e=0 -> m*0.5 (subnormal), else
     * (1+m/2)*2^(e-1). Bit 3 is the sign. (c/fp4.h:204-207) */
    unsigned e = (nib >> 1) & 3u, m = nib & 1u;
    float mag = e ? (float)(2u + m) * (float)(1u << e) * 0.25f
                  : 0.5f * (float)m;
    /* the negative-zero code 0b1000 decodes to +0.0, as in the reference
     * table (c/fp4.h:204-207), so dequantised rows match it bit for bit */
    return ((nib & 8u) && mag != 0.0f) ? -mag : mag;
}

void orc_fp4_dequant_row(const uint8_t *packed, const uint8_t *scales,
                         float *out, size_t K) {
    /* (c/fp4.h:323-335): element k lives in byte k/2, low nibble for even k */
    for (size_t k = 0; k < K; k++) {
        uint8_t byte = packed[k >> 1];
        unsigned nib = (k & 1) ? (unsigned)(byte >> 4) : (unsigned)(byte & 15u);
        out[k] = orc_fp4_value(nib) * orc_ue8m0_f32(scales[k / 32]);
    }
}

float orc_bf16_round(float x) {
    /* (c/fp4.h:262-270) RNE on the upper 16 bits; NaN passes through */
    uint32_t u = f2u(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x;
    uint32_t lsb = (u >> 16) & 1u;
    return u2f((u + 0x7fffu + lsb) & 0xffff0000u);
}

uint8_t orc_e4m3_quant(float x) {
    /* (c/fp4.h:219-253) saturate to the finite range, then round to the
     * nearest E4M3 value, ties to even.
     * Normal range |x| >= 2^-6: RNE on the fp32 bits keeping 3 mantissa
     * bits; a mantissa carry walks into the exponent by itself. The E4M3
     * code is then the kept bits re-biased from 127 to 7 (120 << 3).
     * Below 2^-6 the grid is uniform with quantum 2^-9: scaling by 512 is
     * exact, and rint (ties to even) gives the subnormal code 0..8 (8 is
     * the smallest normal, continuous with the grid). */
    if (x > 448.0f) x = 448.0f;
    if (x < -448.0f) x = -448.0f;
    uint32_t u = f2u(x);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    uint32_t code;
    if (a >= 0x3c800000u) {                     /* |x| >= 2^-6 */
        uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;
        code = r - (120u << 3);
    } else {
        code = (uint32_t)rintf(u2f(a) * 512.0f);
    }
    return (uint8_t)(sign | code);
}

float orc_e4m3_dequant(uint8_t c) {
    /* (c/fp4.h:255-260) exponent field e (bias 7), mantissa m; e=0 is the
     * subnormal m*2^-9. 0x7F/0xFF are not NaN here: they decode as +-480. */
    unsigned e = (c >> 3) & 15u, m = c & 7u;
    float mag = e ? u2f(((e + 120u) << 23) | (m << 20))
                  : (float)m * (1.0f / 512.0f);
    return (c & 0x80u) ? -mag : mag;
}

size_t orc_act_blocks(size_t K) { return (K + 127) / 128; }

void orc_act_quant_row(const float *x, size_t K, uint8_t *codes,
                       float *scales) {
    /* (c/fp4.h:293-321) per 128-element group: amax (floor 1e-4),
     * s = 2^ceil(log2(amax * fl(1/448))) from the product's bits (exponent,
     * +1 when any mantissa bit is set), codes = q(x / s). */
    const float inv448 = 1.0f / 448.0f;
    for (size_t lo = 0, b = 0; lo < K; lo += 128, b++) {
        size_t hi = lo + 128 < K ? lo + 128 : K;
        float amax = 0.0f;
        for (size_t i = lo; i < hi; i++) {
            float a = fabsf(x[i]);
            amax = a > amax ? a : amax;
        }
        if (amax < 1e-4f) amax = 1e-4f;
        uint32_t pb = f2u(amax * inv448);
        uint32_t ex = ((pb >> 23) & 0xffu) + ((pb & 0x7fffffu) ? 1u : 0u);
        float s = u2f(ex << 23);
        scales[b] = s;
        for (size_t i = lo; i < hi; i++) codes[i] = orc_e4m3_quant(x[i] / s);
    }
}

void orc_act_quant_rows(const float *x, size_t M, size_t K, uint8_t *codes,
                        float *scales) {
    /* (c/attn.h:393-403) */
    float *row = malloc(K * sizeof(float));
    size_t nab = orc_act_blocks(K);
    for (size_t m = 0; m < M; m++) {
        for (size_t i = 0; i < K; i++) row[i] = orc_bf16_round(x[m * K + i]);
        orc_act_quant_row(row, K, codes + m * K, scales + m * nab);
    }
    free(row);
}

/* ------------------------------------------------------------------ GEMMs */

void orc_fp4_gemm(const uint8_t *w, const uint8_t *ws, const uint8_t *acodes,
                  const float *as, float *out, size_t M, size_t O, size_t K) {
    /* (c/fp4.h:367-395) per output: for each 32-group in K order, the group
     * dot is a running fp32 sum of exact products taken in k order; the
     * group is folded as (dot * sa) * sb, each multiply rounded on its own,
     * and added to the running fp32 total in group order. */
    size_t nb = K / 32, nab = orc_act_blocks(K);
    float *a = malloc(K * sizeof(float));
    for (size_t m = 0; m < M; m++) {
        for (size_t k = 0; k < K; k++) a[k] = orc_e4m3_dequant(acodes[m * K + k]);
        for (size_t o = 0; o < O; o++) {
            const uint8_t *row = w + o * (K / 2);
            float total = 0.0f;
            for (size_t g = 0; g < nb; g++) {
                float dot = 0.0f;
                for (size_t k = g * 32; k < g * 32 + 32; k++) {
                    uint8_t byte = row[k >> 1];
                    unsigned nib = (k & 1) ? (unsigned)(byte >> 4)
                                           : (unsigned)(byte & 15u);
                    float p = a[k] * orc_fp4_value(nib);
                    dot = dot + p;
                }
                float t = dot * as[m * nab + g / 4];
                t = t * orc_ue8m0_f32(ws[o * nb + g]);
                total = total + t;
            }
            out[m * O + o] = total;
        }
    }
    free(a);
}

void orc_fp4_linear(const uint8_t *w, const uint8_t *ws, const float *x,
                    float *out, size_t M, size_t K, size_t O) {
    /* (c/attn.h:432-448) */
    size_t nab = orc_act_blocks(K);
    uint8_t *codes = malloc(M * K);
    float *as = malloc(M * nab * sizeof(float));
    orc_act_quant_rows(x, M, K, codes, as);
    orc_fp4_gemm(w, ws, codes, as, out, M, O, K);
    for (size_t i = 0; i < M * O; i++) out[i] = orc_bf16_round(out[i]);
    free(codes);
    free(as);
}

void orc_fp8_gemm(const uint8_t *w, const uint8_t *ws, const uint8_t *acodes,
                  const float *as, float *out, size_t M, size_t O, size_t K) {
    /* (c/fp8.h:191-218) per 128-group: sequential fp32 dot of exact
     * products; the two scales are multiplied FIRST (one rounding), then
     * dot * sc, then added to the running total in group order. */
    size_t nb = orc_act_blocks(K);
    float *a = malloc(K * sizeof(float));
    for (size_t m = 0; m < M; m++) {
        for (size_t k = 0; k < K; k++) a[k] = orc_e4m3_dequant(acodes[m * K + k]);
        for (size_t o = 0; o < O; o++) {
            const uint8_t *row = w + o * K;
            const uint8_t *srow = ws + (o / 128) * nb;
            float total = 0.0f;
            for (size_t g = 0; g < nb; g++) {
                size_t hi = g * 128 + 128 < K ? g * 128 + 128 : K;
                float dot = 0.0f;
                for (size_t k = g * 128; k < hi; k++) {
                    float p = a[k] * orc_e4m3_dequant(row[k]);
                    dot = dot + p;
                }
                float sc = as[m * nb + g] * orc_ue8m0_f32(srow[g]);
                float t = dot * sc;
                total = total + t;
            }
            out[m * O + o] = total;
        }
    }
    free(a);
}

void orc_fp8_linear(const uint8_t *w, const uint8_t *ws, const float *x,
                    float *out, size_t M, size_t K, size_t O) {
    size_t nab = orc_act_blocks(K);
    uint8_t *codes = malloc(M * K);
    float *as = malloc(M * nab * sizeof(float));
    orc_act_quant_rows(x, M, K, codes, as);
    orc_fp8_gemm(w, ws, codes, as, out, M, O, K);
    for (size_t i = 0; i < M * O; i++) out[i] = orc_bf16_round(out[i]);
    free(codes);
    free(as);
}

/* ------------------------------------------------------------------- MoE */

void orc_swiglu(const float *g, const float *u, float *h, size_t n,
                float limit) {
    /* (c/moe.h:113-126): up clamped to [-limit, limit], gate clamped from
     * above only; silu(g) = g * (1/(1+exp(-g))) with the reciprocal formed
     * first; product with up, then BF16. */
    for (size_t i = 0; i < n; i++) {
        float gv = g[i], uv = u[i];
        if (limit > 0.0f) {
            uv = uv > limit ? limit : (uv < -limit ? -limit : uv);
            gv = gv > limit ? limit : gv;
        }
        float sig = 1.0f / (1.0f + expf(-gv));
        float silu = gv * sig;
        h[i] = orc_bf16_round(silu * uv);
    }
}

void orc_moe_routed(const uint8_t *const *w1, const uint8_t *const *w1s,
                    const uint8_t *const *w2, const uint8_t *const *w2s,
                    const uint8_t *const *w3, const uint8_t *const *w3s,
                    int dim, int inter, float limit, const float *x,
                    const int32_t *idx, const float *wgt, int s, int topk,
                    float *y) {
    /* (c/moe.h:433-450, :148-158): for every (t, j) in token-major order,
     * eo = w2(swiglu(w1(x_t), w3(x_t))) through the fp4 linears; the token
     * sum starts at 0 and adds wgt*eo per j in order (multiply rounded,
     * then add rounded). The reference's batched path computes the same
     * per-row values (its GEMM rows are M-independent), so one restatement
     * covers both. */
    float *g = malloc((size_t)inter * sizeof(float));
    float *u = malloc((size_t)inter * sizeof(float));
    float *h = malloc((size_t)inter * sizeof(float));
    float *eo = malloc((size_t)dim * sizeof(float));
    memset(y, 0, (size_t)s * dim * sizeof(float));
    for (int t = 0; t < s; t++) {
        const float *xt = x + (size_t)t * dim;
        float *yt = y + (size_t)t * dim;
        for (int j = 0; j < topk; j++) {
            int e = idx[t * topk + j];
            orc_fp4_linear(w1[e], w1s[e], xt, g, 1, (size_t)dim, (size_t)inter);
            orc_fp4_linear(w3[e], w3s[e], xt, u, 1, (size_t)dim, (size_t)inter);
            orc_swiglu(g, u, h, (size_t)inter, limit);
            orc_fp4_linear(w2[e], w2s[e], h, eo, 1, (size_t)inter, (size_t)dim);
            float wt = wgt[t * topk + j];
            for (int i = 0; i < dim; i++) {
                float p = wt * eo[i];
                yt[i] = yt[i] + p;
            }
        }
    }
    free(g); free(u); free(h); free(eo);
}

/* ------------------------------------------------------------ router */

/* torch softplus, beta 1, threshold 20 (c/moe.h:97-100) */
static float orc_softplus(float v) { return v > 20.0f ? v : log1pf(expf(v)); }

void orc_router(const float *gate_w, const float *gate_bias, const float *x,
                int s, int dim, int E, int topk, float route_scale, int hash,
                const int64_t *tid2eid, const int64_t *ids, float *sp,
                int32_t *idx, float *wgt) {
    /* scores: strict k-order fp32 dots, products rounded then added
     * (apus_dot_f32_scalar, c/attn.h:460-465, via apus_f32_linear), then
     * sqrt(softplus) (c/moe.h:360-361) */
    for (int t = 0; t < s; t++)
        for (int e = 0; e < E; e++) {
            const float *a = x + (size_t)t * dim, *b = gate_w + (size_t)e * dim;
            float dot = 0.0f;
            for (int k = 0; k < dim; k++) {
                float p = a[k] * b[k];
                dot = dot + p;
            }
            sp[(size_t)t * E + e] = sqrtf(orc_softplus(dot));
        }
    for (int t = 0; t < s; t++) {
        int32_t *it = idx + (size_t)t * topk;
        const float *row = sp + (size_t)t * E;
        if (hash) {
            for (int j = 0; j < topk; j++) it[j] = (int32_t)tid2eid[ids[t] * topk + j];
        } else {
            /* selection on sp + bias (c/moe.h:362-363): stable descending
             * top-k, strict greater-than, lowest index among equals
             * (c/attn.h:668-686) */
            char used[1024] = {0};
            for (int j = 0; j < topk; j++) {
                int best = -1;
                float bv = 0.0f;
                for (int e = 0; e < E; e++) {
                    if (used[e]) continue;
                    float v = row[e] + gate_bias[e];
                    if (best < 0 || v > bv) { best = e; bv = v; }
                }
                it[j] = best;
                used[best] = 1;
            }
        }
        /* weights from the unbiased scores, normalised, times route_scale
         * (c/moe.h:401-410) */
        float *wt = wgt + (size_t)t * topk, sum = 0.0f;
        for (int j = 0; j < topk; j++) { wt[j] = row[it[j]]; sum += wt[j]; }
        for (int j = 0; j < topk; j++) wt[j] = wt[j] / sum * route_scale;
    }
}

void orc_moe_forward(const float *gate_w, const float *gate_bias, int hash,
                     const int64_t *tid2eid, const int64_t *ids,
                     float route_scale, float limit,
                     const uint8_t *const *w1, const uint8_t *const *w1s,
                     const uint8_t *const *w2, const uint8_t *const *w2s,
                     const uint8_t *const *w3, const uint8_t *const *w3s,
                     const uint8_t *sw1, const uint8_t *sw1s,
                     const uint8_t *sw2, const uint8_t *sw2s,
                     const uint8_t *sw3, const uint8_t *sw3s,
                     int E, int topk, int dim, int inter, const float *x, int s,
                     float *out, float *routed, float *shared, float *sp_out,
                     int32_t *idx_out, float *wgt_out) {
    float *sp = malloc((size_t)s * E * sizeof(float));
    int32_t *idx = malloc((size_t)s * topk * sizeof(int32_t));
    float *wgt = malloc((size_t)s * topk * sizeof(float));
    float *y = malloc((size_t)s * dim * sizeof(float));
    float *sh = malloc((size_t)s * dim * sizeof(float));
    float *g = malloc((size_t)inter * sizeof(float));
    float *u = malloc((size_t)inter * sizeof(float));
    float *h = malloc((size_t)inter * sizeof(float));
    orc_router(gate_w, gate_bias, x, s, dim, E, topk, route_scale, hash, tid2eid, ids,
               sp, idx, wgt);
    orc_moe_routed(w1, w1s, w2, w2s, w3, w3s, dim, inter, limit, x, idx, wgt, s, topk, y);
    /* shared expert: FP8 linears with BF16 outputs and SwiGLU per row
     * (c/moe.h:570-585, apus_expert kind 1 c/moe.h:333-350) */
    for (int t = 0; t < s; t++) {
        const float *xt = x + (size_t)t * dim;
        orc_fp8_linear(sw1, sw1s, xt, g, 1, (size_t)dim, (size_t)inter);
        orc_fp8_linear(sw3, sw3s, xt, u, 1, (size_t)dim, (size_t)inter);
        orc_swiglu(g, u, h, (size_t)inter, limit);
        orc_fp8_linear(sw2, sw2s, h, sh + (size_t)t * dim, 1, (size_t)inter, (size_t)dim);
    }
    /* out = bf16(routed + shared) (c/moe.h:588-589) */
    for (size_t i = 0; i < (size_t)s * dim; i++) out[i] = orc_bf16_round(y[i] + sh[i]);
    if (routed) memcpy(routed, y, (size_t)s * dim * sizeof(float));
    if (shared) memcpy(shared, sh, (size_t)s * dim * sizeof(float));
    if (sp_out) memcpy(sp_out, sp, (size_t)s * E * sizeof(float));
    if (idx_out) memcpy(idx_out, idx, (size_t)s * topk * sizeof(int32_t));
    if (wgt_out) memcpy(wgt_out, wgt, (size_t)s * topk * sizeof(float));
    free(sp); free(idx); free(wgt); free(y); free(sh); free(g); free(u); free(h);
}

/* ------------------------------------------------------------ f64 truth */

void orc_fp4_truth_f64(const uint8_t *w, const uint8_t *ws,
                       const uint8_t *acodes, const float *as, double *out,
                       double *esc, size_t M, size_t O, size_t K) {
    size_t nb = K / 32, nab = orc_act_blocks(K);
    for (size_t m = 0; m < M; m++)
        for (size_t o = 0; o < O; o++) {
            double tot = 0.0, sc = 0.0;
            for (size_t g = 0; g < nb; g++) {
                double dot = 0.0;
                for (size_t k = g * 32; k < g * 32 + 32; k++) {
                    uint8_t byte = w[o * (K / 2) + (k >> 1)];
                    unsigned nib = (k & 1) ? (unsigned)(byte >> 4)
                                           : (unsigned)(byte & 15u);
                    dot += (double)orc_e4m3_dequant(acodes[m * K + k]) *
                           (double)orc_fp4_value(nib);
                }
                double term = dot * (double)as[m * nab + g / 4] *
                              (double)orc_ue8m0_f32(ws[o * nb + g]);
                tot += term;
                sc += fabs(term);
            }
            out[m * O + o] = tot;
            if (esc) esc[m * O + o] = sc;
        }
}

void orc_fp8_truth_f64(const uint8_t *w, const uint8_t *ws,
                       const uint8_t *acodes, const float *as, double *out,
                       double *esc, size_t M, size_t O, size_t K) {
    size_t nb = orc_act_blocks(K);
    for (size_t m = 0; m < M; m++)
        for (size_t o = 0; o < O; o++) {
            double tot = 0.0, sc = 0.0;
            for (size_t g = 0; g < nb; g++) {
                size_t hi = g * 128 + 128 < K ? g * 128 + 128 : K;
                double dot = 0.0, adot = 0.0;
                for (size_t k = g * 128; k < hi; k++) {
                    double p = (double)orc_e4m3_dequant(acodes[m * K + k]) *
                               (double)orc_e4m3_dequant(w[o * K + k]);
                    dot += p;
                    adot += fabs(p);
                }
                double s = (double)as[m * nb + g] *
                           (double)orc_ue8m0_f32(ws[(o / 128) * nb + g]);
                tot += dot * s;
                sc += adot * fabs(s);
            }
            out[m * O + o] = tot;
            if (esc) esc[m * O + o] = sc;
        }
}

/* --------------------------------------------------------- exhaustive pin */

uint64_t orc_pin_unary(int which, const void *ref_fn, uint64_t lo,
                       uint64_t hi, uint32_t *first_bad) {
    uint64_t bad = 0;
    if (first_bad) *first_bad = 0;
    if (which == 0) {
        float (*ref)(float) = (float (*)(float))ref_fn;
        for (uint64_t i = lo; i < hi; i++) {
            float x = u2f((uint32_t)i);
            if (f2u(orc_bf16_round(x)) != f2u(ref(x))) {
                if (!bad && first_bad) *first_bad = (uint32_t)i;
                bad++;
            }
        }
    } else {
        uint8_t (*ref)(float) = (uint8_t (*)(float))ref_fn;
        for (uint64_t i = lo; i < hi; i++) {
            uint32_t u = (uint32_t)i;
            if ((u & 0x7f800000u) == 0x7f800000u) continue;   /* inf/NaN */
            float x = u2f(u);
            if (orc_e4m3_quant(x) != ref(x)) {
                if (!bad && first_bad) *first_bad = u;
                bad++;
            }
        }
    }
    return bad;
}

/* ------------------------------------------------ counter-based generator */

uint64_t orc_hash64(uint64_t seed, uint64_t stream, uint64_t index) {
    /* splitmix64 finaliser over a (seed, stream, index) mix */
    uint64_t z = seed * 0x9e3779b97f4a7c15ull + stream * 0xd1b54a32d192ed03ull
               + index * 0xbf58476d1ce4e5b9ull + 0x94d049bb133111ebull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

void orc_fill_bytes(uint64_t seed, uint64_t stream, uint64_t first,
                    uint8_t *out, size_t n, int kind) {
    /* kind 0: uniform byte (packed FP4, nibbles uniform over 16 codes)
     * kind 1: UE8M0 byte uniform in 118..130 (MXFP4 group scales)
     * kind 2: E4M3 code of an approximately N(0,1) value (Irwin-Hall of
     *         four 16-bit uniforms, exact integer sum, one fp32 scaling)
     * kind 3: UE8M0 byte uniform in 117..123 (FP8 tile scales) */
    for (size_t i = 0; i < n; i++) {
        uint64_t pos = first + i;
        if (kind == 0) {   /* eight bytes per hash: byte (pos % 8) of h(pos / 8) */
            out[i] = (uint8_t)(orc_hash64(seed, stream, pos >> 3) >> (8 * (pos & 7)));
            continue;
        }
        uint64_t h = orc_hash64(seed, stream, pos);
        switch (kind) {
        case 1: out[i] = (uint8_t)(118u + (uint32_t)((h >> 32) % 13u)); break;
        case 2: {
            int32_t sum = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff)
                        + (int32_t)((h >> 32) & 0xffff) + (int32_t)(h >> 48);
            float v = (float)(sum - 131070) * (1.0f / 37837.6f);
            out[i] = orc_e4m3_quant(v);
            break;
        }
        default: out[i] = (uint8_t)(117u + (uint32_t)((h >> 32) % 7u)); break;
        }
    }
}


/* ---- plain-weight linears (c/attn.h:600-666, c/model.h:585-647) ---- */

static float orc_wl_weight(const void *w, size_t i, int bf16) {
    if (!bf16) return ((const float *)w)[i];
    const uint32_t u = (uint32_t)((const uint16_t *)w)[i] << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_wlinear(const void *w, const float *x, float *out, int M, int K, int O, int flags) {
    const int bf16 = (flags & ORC_W_BF16) != 0;
    for (int m = 0; m < M; m++) {
        for (int o = 0; o < O; o++) {
            float acc = 0.0f;
            for (int k = 0; k < K; k++) {
                float xv = x[(size_t)m * K + k];
                if (flags & ORC_W_R_IN) xv = orc_bf16_round(xv);
                const float p = orc_wl_weight(w, (size_t)o * K + k, bf16) * xv;
                acc = acc + p;
            }
            out[(size_t)m * O + o] = (flags & ORC_W_R_OUT) ? orc_bf16_round(acc) : acc;
        }
    }
}

void orc_wlinear_truth_f64(const void *w, const float *x, double *truth, double *esc,
                           int M, int K, int O, int flags) {
    const int bf16 = (flags & ORC_W_BF16) != 0;
    for (int m = 0; m < M; m++) {
        for (int o = 0; o < O; o++) {
            double t = 0.0, e = 0.0;
            for (int k = 0; k < K; k++) {
                float xv = x[(size_t)m * K + k];
                if (flags & ORC_W_R_IN) xv = orc_bf16_round(xv);
                const double p = (double)orc_wl_weight(w, (size_t)o * K + k, bf16) * (double)xv;
                t += p;
                e += fabs(p);
            }
            truth[(size_t)m * O + o] = t;
            esc[(size_t)m * O + o] = e;
        }
    }
}

/* ------------------------------------------------- checker bound (tests) */

/* Not a restatement of a reference function: the bound the MoE stage
 * checker (tests/moe_check.py) puts on what the matrix cores' block-wise
 * fixed-point addition can lose in sum_k W[o,k] * A[k] for one activation
 * row (MXFP4 weights w [O, K/2] low nibble first, E8M0 ws [O, K/32]; E4M3
 * codes [K], fp32 scales [K/128]). Per 32-block: lsb = 2^(exponent of the
 * largest |product| - window); products below 32 lsb can each lose at most
 * themselves or one lsb, so the block loses at most min(their sum, their
 * count x lsb). out[o] = the sum over blocks. Equal to the numpy form of the
 * checker (tests/test_moe_check.py pins the two against each other). */
void orc_fp4_mfma_slack(const uint8_t *w, const uint8_t *ws, const uint8_t *codes,
                        const float *as, double *out, size_t O, size_t K, int window) {
    const size_t nb = K / 32;
    double av[32];
    for (size_t o = 0; o < O; o++) {
        double tot = 0.0;
        for (size_t b = 0; b < nb; b++) {
            const double ws_v = (double)orc_ue8m0_f32(ws[o * nb + b]);
            double t[32], mx = 0.0;
            for (size_t i = 0; i < 32; i++) {
                const size_t k = b * 32 + i;
                av[i] = (double)orc_e4m3_dequant(codes[k]) * (double)as[k / 128];
                const uint8_t byte = w[o * (K / 2) + (k >> 1)];
                const unsigned nib = (k & 1) ? (unsigned)(byte >> 4) : (unsigned)(byte & 15u);
                t[i] = fabs((double)orc_fp4_value(nib) * ws_v * av[i]);
                if (t[i] > mx) mx = t[i];
            }
            if (!(mx > 0.0)) continue;
            int e;
            (void)frexp(mx, &e);                 /* mx = f 2^e, f in [0.5, 1) */
            const double lsb = ldexp(1.0, e - 1 - window);
            double small = 0.0;
            int cnt = 0;
            for (size_t i = 0; i < 32; i++)
                if (t[i] < 32.0 * lsb) { small += t[i]; cnt++; }
            const double cap = cnt * lsb;
            tot += small < cap ? small : cap;
        }
        out[o] = tot;
    }
}
