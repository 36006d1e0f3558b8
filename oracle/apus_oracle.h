/*
 * oracle/apus_oracle.h — CPU restatement of apus's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP backend is
 * compared against; it is never linked into, loaded by, or called from the
 * product library (libapus_hip.so). Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it.
 *
 * Each function restates the behaviour of the reference function cited next
 * to it (paths relative to the apus repository root). The code is written
 * from the stated numerics, not transcribed; where the steps have to be the
 * same (rounding rules, summation order) they are the same on purpose,
 * because bit-exact parity depends on them.
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   orc_ue8m0_f32, orc_fp4_value, orc_fp4_dequant_row, orc_e4m3_dequant:
 *       closed form + exhaustive over every input byte (pair), and bitwise
 *       against the compiled reference (oracle/_ref).
 *   orc_bf16_round, orc_e4m3_quant: exhaustive over all 2^32 float bit
 *       patterns against the compiled reference (oracle/_ref), plus a
 *       brute-force nearest-code search on a sample.
 *   orc_act_quant_row / orc_act_quant_rows: bitwise vs the compiled
 *       reference on seeded rows incl. zero rows, outliers, partial blocks;
 *       invariants (codes*scale within half a code step of x).
 *   orc_fp4_gemm, orc_fp8_gemm: bitwise vs the compiled reference scalar
 *       and AVX2/pthread kernels; float64 truth with the err/esc metric.
 *   orc_swiglu: float64 truth within bf16 half-ulp tolerance; bitwise vs the
 *       reference MoE on the same libm.
 *   orc_moe_routed: bitwise vs the compiled reference apus_moe_forward's
 *       routed output (ApusMoeInterm.moe_routed) on the same routing.
 *   orc_wlinear: bitwise vs the compiled reference apus_f32_linear,
 *       apus_bf16_linear and apus_head_gemv (F32 and BF16 views); the BF16
 *       weight form equals the FP32 form on exactly widened weights.
 */
#ifndef APUS_ORACLE_H
#define APUS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* c/fp4.h:209-217 — UE8M0 byte -> 2^(b-127); b=0 -> 2^-127, b=255 -> +inf */
float   orc_ue8m0_f32(uint8_t b);
/* c/fp4.h:204-207 — E2M1 nibble value (bit 3 = sign) */
float   orc_fp4_value(unsigned nib);
/* c/fp4.h:323-335 — exact dequant of one packed row (low nibble = even k) */
void    orc_fp4_dequant_row(const uint8_t *packed, const uint8_t *scales,
                            float *out, size_t K);
/* c/fp4.h:262-270 — fp32 -> bf16 round-to-nearest-even, kept in fp32 */
float   orc_bf16_round(float x);
/* c/fp4.h:219-253 — fp32 -> E4M3, clamp +-448, RNE, subnormal grid 2^-9 */
uint8_t orc_e4m3_quant(float x);
/* c/fp4.h:255-260 — E4M3 -> fp32, exact; 0x7F/0xFF -> +-480 */
float   orc_e4m3_dequant(uint8_t c);
/* c/fp4.h:289-291 */
size_t  orc_act_blocks(size_t K);
/* c/fp4.h:293-321 — one row, per-128 power-of-2 scale (amax floor 1e-4) */
void    orc_act_quant_row(const float *x, size_t K, uint8_t *codes,
                          float *scales);
/* c/attn.h:393-403 — BF16 round then orc_act_quant_row, per row */
void    orc_act_quant_rows(const float *x, size_t M, size_t K,
                           uint8_t *codes, float *scales);

/* c/fp4.h:367-395 — normative MXFP4 GEMM on pre-quantized activations:
 * out[m,o] = sum_kb (dot32 * as[m,kb/4]) * ue8m0(ws[o,kb]), sequential. */
void    orc_fp4_gemm(const uint8_t *w, const uint8_t *ws,
                     const uint8_t *acodes, const float *as, float *out,
                     size_t M, size_t O, size_t K);
/* c/attn.h:432-448 — bf16(x) -> act quant -> fp4 gemm -> bf16(out) */
void    orc_fp4_linear(const uint8_t *w, const uint8_t *ws, const float *x,
                       float *out, size_t M, size_t K, size_t O);

/* c/fp8.h:191-218 — normative FP8 block-scaled GEMM:
 * out[m,o] = sum_kb dot128 * (as[m,kb] * ue8m0(ws[o/128,kb])), sequential */
void    orc_fp8_gemm(const uint8_t *w, const uint8_t *ws,
                     const uint8_t *acodes, const float *as, float *out,
                     size_t M, size_t O, size_t K);
/* c/attn.h:408-430 (hook-less branch) */
void    orc_fp8_linear(const uint8_t *w, const uint8_t *ws, const float *x,
                       float *out, size_t M, size_t K, size_t O);

/* c/moe.h:113-126 — h = bf16((g * sigmoid(g)) * u) with clamps */
void    orc_swiglu(const float *g, const float *u, float *h, size_t n,
                   float limit);

/* Routed-expert dispatch, c/moe.h:433-563 (s==1 path :435-450 and the
 * batched path, which the reference proves bitwise equal to it). Expert e's
 * weights: w1/w3 [inter, dim/2] + [inter, dim/32], w2 [dim, inter/2] +
 * [dim, inter/32], addressed through the pointer tables. idx/wgt are
 * [s, topk]. y [s, dim] is the FP32 routed sum (ApusMoeInterm.moe_routed). */
void    orc_moe_routed(const uint8_t *const *w1, const uint8_t *const *w1s,
                       const uint8_t *const *w2, const uint8_t *const *w2s,
                       const uint8_t *const *w3, const uint8_t *const *w3s,
                       int dim, int inter, float limit, const float *x,
                       const int32_t *idx, const float *wgt, int s, int topk,
                       float *y);

/* float64 truth for the normative GEMMs plus the per-output error scale
 * (tests/m3/test_fp4.c:75-100, tests/m4a/README.md:78-83):
 *   fp4: esc = sum_kb |dot_kb * sa * sb|
 *   fp8: esc = sum_kb (sum_i |a_i w_i|) * sa * sb */
/* c/moe.h:352-367 apus_router_score + the routing of apus_moe_forward
 * (c/moe.h:378-413, top-k c/attn.h:668-686, softplus c/moe.h:97-100).
 * gate_w [E, dim] fp32; gate_bias [E] (unused with hash); hash: ids [s] and
 * tid2eid [*, topk] pick the experts. Out: sp [s, E] = sqrt(softplus(gate x)),
 * idx [s, topk], wgt [s, topk] = sp[idx] / sum * route_scale. */
void    orc_router(const float *gate_w, const float *gate_bias, const float *x,
                   int s, int dim, int E, int topk, float route_scale, int hash,
                   const int64_t *tid2eid, const int64_t *ids, float *sp,
                   int32_t *idx, float *wgt);
/* c/moe.h:369-595 apus_moe_forward: router, routed experts (MXFP4), FP8
 * shared expert (kind 1 of apus_expert / the batched s > 1 form, identical
 * per row), out = bf16(routed + shared). routed/shared/sp/idx/wgt optional. */
void    orc_moe_forward(const float *gate_w, const float *gate_bias, int hash,
                        const int64_t *tid2eid, const int64_t *ids,
                        float route_scale, float limit,
                        const uint8_t *const *w1, const uint8_t *const *w1s,
                        const uint8_t *const *w2, const uint8_t *const *w2s,
                        const uint8_t *const *w3, const uint8_t *const *w3s,
                        const uint8_t *sw1, const uint8_t *sw1s,
                        const uint8_t *sw2, const uint8_t *sw2s,
                        const uint8_t *sw3, const uint8_t *sw3s,
                        int E, int topk, int dim, int inter, const float *x, int s,
                        float *out, float *routed, float *shared, float *sp,
                        int32_t *idx, float *wgt);
/* Plain-weight linears: c/attn.h:600-666 apus_bf16_linear / apus_f32_linear
 * (and the wo_a rows of the f32_linear hook, c/attn.h:1690-1735),
 * c/model.h:585-647 apus_head_gemv. out[m, o] = sum_k w[o, k] * x'[m, k]
 * in k order from +0, each product and sum rounded to FP32; x' = bf16(x)
 * with ORC_W_R_IN, out rounded to BF16 with ORC_W_R_OUT; w is FP32, or BF16
 * bits widened exactly with ORC_W_BF16 (the hook flags of
 * c/backend_metal.h:56-61). */
#define ORC_W_R_IN  1
#define ORC_W_R_OUT 2
#define ORC_W_BF16  4
void    orc_wlinear(const void *w, const float *x, float *out, int M, int K, int O,
                    int flags);
/* float64 truth of the same products (x' as above) and esc = sum |w x'| */
void    orc_wlinear_truth_f64(const void *w, const float *x, double *truth, double *esc,
                              int M, int K, int O, int flags);
void    orc_fp4_truth_f64(const uint8_t *w, const uint8_t *ws,
                          const uint8_t *acodes, const float *as,
                          double *out, double *esc,
                          size_t M, size_t O, size_t K);
void    orc_fp8_truth_f64(const uint8_t *w, const uint8_t *ws,
                          const uint8_t *acodes, const float *as,
                          double *out, double *esc,
                          size_t M, size_t O, size_t K);

/* Exhaustive pin helpers: compare an oracle unary map against a function
 * pointer over every 32-bit pattern in [lo, hi). Return the number of
 * mismatches and store the first mismatching input in *first_bad.
 *   which = 0: orc_bf16_round vs float(*)(float)
 *   which = 1: orc_e4m3_quant  vs uint8_t(*)(float)   (finite inputs only) */
uint64_t orc_pin_unary(int which, const void *ref_fn, uint64_t lo,
                       uint64_t hi, uint32_t *first_bad);

/* Counter-based weight generator (splitmix64 of (seed, stream, index)).
 * The HIP library has a device twin; the host copy lets tests spot-check
 * device-initialised HBM-resident weights without copying them back. */
uint64_t orc_hash64(uint64_t seed, uint64_t stream, uint64_t index);
void     orc_fill_bytes(uint64_t seed, uint64_t stream, uint64_t first,
                        uint8_t *out, size_t n, int kind);

/* Checker bound, not a reference function: per output row, what the matrix
 * cores' block-wise fixed-point addition can lose (tests/moe_check.py). */
void     orc_fp4_mfma_slack(const uint8_t *w, const uint8_t *ws, const uint8_t *codes,
                            const float *as, double *out, size_t O, size_t K, int window);

#ifdef __cplusplus
}
#endif

#endif /* APUS_ORACLE_H */
