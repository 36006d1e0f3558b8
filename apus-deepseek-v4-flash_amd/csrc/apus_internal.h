/*
 * apus_internal.h — launchers shared between the kernel translation unit and
 * the C-ABI backend. Not part of the public interface (include/apus_hip.h).
 * All launchers are asynchronous on the given stream and take device
 * pointers only.
 */
#ifndef APUS_INTERNAL_H
#define APUS_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

/* weight formats of the block-scaled GEMM */
enum { APUS_W_FP4 = 0, APUS_W_FP8 = 1, APUS_W_F32 = 2, APUS_W_BF16 = 3 };

/* One GEMM of a (possibly grouped) launch. Output row m of this entry is
 *   out[orow(m) * ldo + o] = sum_k A[arow(m), k] * W[o, k]   (o < O)
 * with arow(m) = arows ? arows[m] : a0 + m, orow(m) = orows ? orows[m] : o0 + m.
 * W: FP4 [O, K/2] packed + [O, K/32] E8M0, or FP8 [O, K] + [ceil(O/128), K/128]
 * E8M0 tiles. A: E4M3 codes [*, K] with fp32 power-of-two scales [*, K/128]. */
typedef struct {
    const uint8_t *w, *ws;
    float *out;
    const int32_t *arows, *orows;
    int32_t a0, o0, M, pad;
} ApusGemmEnt;

typedef struct {
    const uint8_t *acodes;   /* [rows, K] */
    const float *ascale;     /* [rows, K/128] */
    const ApusGemmEnt *ents; /* grouped: device array; else NULL */
    ApusGemmEnt ent0;        /* the entry when ents == NULL */
    ApusGemmEnt ent1;        /* few-row schedule, ents and pidx NULL, two launch
                              * entries: entry 1 (same activation rows as ent0) */
    int O, K, ldo, round_out;
    int wtiled;              /* every W (and FP4 scale) in the MFMA-tiled layout of
                              * apus_launch_pack: K 2048 or 4096, O % 128 == 0 */
    int max_m;               /* upper bound on every entry's M (0 = unknown); a
                              * launch with max_m <= 8 runs only the few-row
                              * schedule */
    int min_m;               /* every entry has M = 0 or M > min_m (0 = unknown) */
    int m_min, m_max;        /* set by the launcher: a kernel computes only the
                              * entries with m_min < M <= m_max (m_max 0: no cap) */
    int kchain;              /* required accumulation order over K (grouped MXFP4
                              * launches with K 2048 / 4096 and the few-row
                              * schedule): 0 = the schedule's own; 1 = one chain
                              * over the 128-groups in order; 4 = four chains from
                              * zero over the quarters of K, added left to right.
                              * The routed MoE uses 1 for w1/w3 and 4 for w2, the
                              * orders of its one-token kernels, so a token's
                              * result does not depend on the batch around it. */
    int pad3;
    /* --- few-row schedule only (apus_launch_gemm_few) --- */
    int asrc;                /* APUS_A_*: where the activation rows come from */
    const float *ax, *au;    /* F32: rows of x [*, K]; SWIGLU: rows of g and u [*, K] */
    float limit;             /* SWIGLU clamp (<= 0: none) */
    /* pair entries (ents == NULL, pidx != NULL): launch entry y is matrix
     * y % nmat of routed pair p = y / nmat, expert e = pidx[p] (pairs with
     * e outside [0, pE) are skipped): W = pw[mat][e], pws[mat][e], M = 1,
     * activation row p / adiv, output row p of pout[mat] */
    const int32_t *pidx;
    int nmat, adiv, pE, pad2;
    const uint8_t *const *pw[2];
    const uint8_t *const *pws[2];
    float *pout[2];
    /* regularly spaced expert slabs (an expert store layer): when pbase is
     * set, W = pbase + e * pstride + pwoff[mat] and scales at psoff[mat]
     * instead of the pointer tables (one dependent load fewer) */
    const uint8_t *pbase;
    size_t pstride, pwoff[2], psoff[2];
    /* fused (t, j)-ordered accumulation (pair entries, nmat 1): after every
     * workgroup of a column tile has written its outputs, the last one adds
     * y[t, o] = sum_j acc_w[t*acc_topk + j] * out[t*acc_topk + j, o] over
     * t < acc_s (y row stride ldo); tickets: one counter per column tile,
     * zero at launch */
    const float *acc_w;
    float *acc_y;
    unsigned *tickets;
    int acc_topk, acc_s;
    /* optional fused sum (apus_moe_pair2_kernel): add_out[t, o] =
     * bf16(y[t, o] + add_src[t, o]), row stride ldo */
    const float *add_src;
    float *add_out;
    /* one-token MoE kernels: routed pairs in the launch (apus_moe_pair13 /
     * pair2), and optionally each token's FP8 shared expert fused in: w1,
     * w2, w3 = shw[0..2] with tile scales shws (MFMA-tiled when sh_tiled);
     * its h goes to h row npairs + t, sh = bf16(w2 h) to sh_out, and
     * add_out = bf16(y + sh) */
    int npairs, sh_tiled;
    const uint8_t *shw[3], *shws[3];
    float *sh_out;
    /* apus_moe_pair13 with rsp set: each workgroup chooses its pair's expert
     * itself (apus_route_token over token t's selection scores rsel[t] or
     * the hash row rt2e[rids[t]]), and the workgroups of column block 0
     * write the choice and its weight to ridx / rwgt (the w2 launch's pidx
     * and acc_w) */
    /* one-token MoE h hand-off: apus_moe_pair13 quantises h per 128-group
     * (E4M3 codes hq [rows, O], E8M0 bytes hqs [rows, O/128]) through
     * hq_tk, one counter per (row, group), zero at launch and left zero;
     * apus_moe_pair2 reads its A operands straight from hq / hqs */
    uint8_t *hq, *hqs;
    unsigned *hq_tk;
    /* apus_moe_pair13 with rdout set: launch rows after the pairs (and the
     * shared-expert rows) compute, per token t, a dense FP8 linear of the same
     * x: rdout[t, 0 : 2 O] = bf16(W x) with W = rdw [2 O, K] (tile scales
     * rdws [2 O / 128, K / 128]; MFMA-tiled when rdtiled) */
    const uint8_t *rdw, *rdws;
    float *rdout;
    int rdtiled, pad4;
    const float *rsel, *rsp;
    const int64_t *rt2e, *rids;
    float rscale;
    int rE;
    int32_t *ridx;
    float *rwgt;
    unsigned *zero;          /* zeroed by workgroups of launch row 0 (the */
    int nzero;               /* tickets of a later launch) */
    /* many-row schedule work list (optional): launch row y computes rows
     * [c0, c0 + 64) of entry items[y].x, c0 = items[y].y; x < 0: nothing */
    const int2 *items;
} ApusGemmArgs;

enum { APUS_A_CODES = 0, APUS_A_F32 = 1, APUS_A_SWIGLU = 2 };

/* reduction lengths with the MFMA schedules (decode, tile) and the MFMA-tiled
 * weight layout for dense GEMMs: 512 * {2, 4, 8, 16} (the model's dense FP8
 * shapes have K 1024, 4096 and 8192; experts 2048 and 4096) */
static inline bool apus_fast_k(int K) { return K == 1024 || K == 2048 || K == 4096 || K == 8192; }
/* grouped launches (experts) keep to K 2048 and 4096 */
static inline bool apus_group_k(int K) { return K == 2048 || K == 4096; }

/* rows (tokens) per chunk of the many-row (prefill) schedule for MXFP4
 * weights: one work-list item */
#ifndef APUS_PREFILL_ROWS
#define APUS_PREFILL_ROWS 64
#endif

/* One-token-chunk MoE dispatch for few routed pairs (decode), MXFP4 experts
 * with dim and inter in {2048, 4096}, topk 6 or 8, in two launches:
 *  w1/w3: one workgroup per (16 rows of inter, pair): h = swiglu(bf16(w1 x),
 *         bf16(w3 x)) written as fp32 rows of pout[0] [s*topk, inter]; x rows
 *         quantised while staging; zero, nzero cleared.
 *  w2:    one workgroup per 16 columns of dim, looping over the tokens and
 *         their topk pairs: y[t] = sum_j acc_w[t*topk+j] * bf16(w2_j h_j).
 * Fields used: ax (x or h), pidx, pE, adiv (= topk), pw/pws or pbase/pstride/
 * pwoff/psoff, limit, acc_w/acc_y/acc_s/acc_topk, O, K, ldo, wtiled.
 * Returns hipErrorInvalidValue for other shapes. */
hipError_t apus_launch_moe_pair13(const ApusGemmArgs *a, int npairs, hipStream_t st);
hipError_t apus_launch_moe_pair2(const ApusGemmArgs *a, hipStream_t st);

/* The same one-token dispatch (dim 4096, inter 2048, topk 6, one token, no
 * shared expert or in-kernel routing; optionally the dense rider of a1) in
 * ONE launch of 256 workgroups with a grid-wide barrier between the w1/w3
 * and the w2 phases; a1 / a2 as for apus_launch_moe_pair13 / pair2. bar:
 * apus_moe_layer1_bar_words() device words, zero before the first launch
 * and left zero (but for the counter at apus_moe_layer1_fault_word() of
 * workgroups that gave up waiting at the barrier). Needs all 256
 * workgroups resident at once: callers check apus_moe_layer1_fits() and the
 * CU count, and never run two of these launches concurrently. A workgroup
 * whose barrier wait gives up after spin_lim polls writes NaN to its y (and
 * add_out) columns and sets *hflag = 1 (device-visible host memory, or
 * null). */
hipError_t apus_launch_moe_layer1(const ApusGemmArgs *a1, const ApusGemmArgs *a2, unsigned *bar,
                                  unsigned *hflag, unsigned spin_lim, hipStream_t st);
/* workgroups of apus_moe_layer1_kernel that fit on one CU; its barrier
 * buffer size and fault-counter word */
int apus_moe_layer1_fits();
int apus_moe_layer1_bar_words();
int apus_moe_layer1_fault_word();

/* The few-row schedule for every entry (each entry's M is computed in
 * chunks of up to `rows` rows; rows 1 or 8), with the activation source,
 * pair entries and fused accumulation of ApusGemmArgs. Needs K 2048 or
 * 4096 and O % 128 == 0; asrc CODES needs rows 8. ks: 0 = by launch size,
 * else 1, 2 or 4 waves per 16-row tile. Returns hipErrorInvalidValue for
 * other shapes. */
hipError_t apus_launch_gemm_few(int wfmt, const ApusGemmArgs *a, int n_ent, int rows,
                                int ks, hipStream_t st);

/* y[m] = A x W^T for every entry; n_ent entries (1 with ents == NULL). */
hipError_t apus_launch_gemm(int wfmt, const ApusGemmArgs *a, int n_ent,
                            hipStream_t st);

/* BF16 round + per-128 E4M3 act quant of rows of x (row stride ldx floats);
 * arows optional gather. codes [M, K], scales [M, K/128]. K % 128 == 0. */
hipError_t apus_launch_act_quant(const float *x, int ldx, const int32_t *arows,
                                 int M, int K, uint8_t *codes, float *scales,
                                 hipStream_t st);

/* h = bf16(silu(clamp g) * clamp u) then act quant of h (no extra bf16 step
 * needed: h is already bf16). g, u, codes: [M, N]; scales [M, N/128]. */
hipError_t apus_launch_swiglu_quant(const float *g, const float *u, int M,
                                    int N, float limit, uint8_t *codes,
                                    float *scales, hipStream_t st);

/* Counting sort of the routed pairs by expert and GEMM entry tables.
 * idx [nj] (nj = s * topk) expert ids in [0, E), E <= 1024; writes
 * pair_sorted [nj] (pair q), tok_sorted [nj] (q / topk) and two sets of
 * entry tables: experts with 1..small_max pairs go, in expert order, to the
 * front of e13s [2E] (w1 then w3 of each expert, output rows in sorted
 * order) and e2s [E] (output rows = pair ids); experts with more pairs go to
 * e13l / e2l the same way. Slots past the listed experts have M = 0.
 * items13 [2 n_items] / items2 [n_items] list (entry, first row) of every
 * APUS_PREFILL_ROWS-row chunk of the many-row entries (x = -1 past the end).
 * The weight pointer tables are device arrays of E pointers each. */
typedef struct {
    const uint8_t *const *w1, *const *w1s, *const *w2, *const *w2s,
                  *const *w3, *const *w3s;
} ApusExpertTable;

hipError_t apus_launch_moe_route(const int32_t *idx, int nj, int topk, int E,
                                 ApusExpertTable tab, float *g, float *u, float *eo,
                                 int32_t *pair_sorted, int32_t *tok_sorted,
                                 ApusGemmEnt *e13s, ApusGemmEnt *e2s, ApusGemmEnt *e13l,
                                 ApusGemmEnt *e2l, int small_max, int2 *items13, int2 *items2,
                                 int n_items, hipStream_t st);

/* work-list bound per matrix for the many-row experts of nj pairs */
static inline int apus_moe_items_bound(int nj, int E, int small_max) {
    const int nl = (nj / (small_max + 1)) < E ? nj / (small_max + 1) : E;
    return nj / APUS_PREFILL_ROWS + nl;
}

/* Row-major <-> MFMA-tiled weights (unpack = 0: w, ws -> tw, tws). FP4
 * moves the weights and the per-32 scales, FP8 the weights only (its
 * 128 x 128 tile scales keep their layout). O % 16 == 0, K % 512 == 0;
 * source and destination must not overlap. */
hipError_t apus_launch_pack(int wfmt, const uint8_t *w, const uint8_t *ws, uint8_t *tw,
                            uint8_t *tws, int O, int K, int unpack, hipStream_t st);

/* Router of one MoE layer (c/moe.h:352-410): scores, selection, weights. */
hipError_t apus_launch_router(const float *gate_w, const float *bias, const float *x, int s,
                              int dim, int E, float *sp, float *biased, hipStream_t st);
hipError_t apus_launch_topk(const float *sel, const float *sp, int s, int E, int topk,
                            const int64_t *tid2eid, const int64_t *ids, float route_scale,
                            int32_t *idx, float *wgt, hipStream_t st);
/* plain-weight linear (FP32 or BF16-bit weights [O, K], FP32 accumulate):
 * out[m, o] = sum_k w[o, k] * x'[m, k]; flags as the f32_linear hook
 * (1: x' = bf16(x), 2: bf16 output, 4: BF16 weights). K % 8 == 0. */
hipError_t apus_launch_wgemv(const void *w, const float *x, float *out, int M, int K, int O,
                             int flags, hipStream_t st);
/* hardware E4M3 conversion vs the integer encoder over |x| <= 448 */
hipError_t apus_launch_e4m3_hw_check(unsigned *bad, unsigned *last_bad, hipStream_t st);
/* out = bf16(a + b) */
hipError_t apus_launch_add_bf16(const float *a, const float *b, float *out, size_t n,
                                hipStream_t st);

/* y[t, i] = sum_j wgt[t, j] * eo[t*topk + j, i] in j order (mul, then add,
 * each rounded), starting from +0; with add_out, also add_out[t, i] =
 * bf16(y[t, i] + add_src[t, i]). */
hipError_t apus_launch_moe_accum(const float *eo, const float *wgt, int s,
                                 int topk, int dim, float *y, const float *add_src,
                                 float *add_out, hipStream_t st);

/* Counter-based fill (kind as orc_fill_bytes: 0 uniform byte, 1 E8M0
 * 118..130, 2 E4M3 of ~N(0,1), 3 E8M0 117..123). */
hipError_t apus_launch_fill(uint8_t *dst, size_t n, uint64_t seed,
                            uint64_t stream_id, uint64_t first, int kind,
                            hipStream_t st);

/* elementwise BF16 rounding in place */
hipError_t apus_launch_bf16_round(float *v, size_t n, hipStream_t st);

/* a one-wave kernel that holds the stream for `ticks` wall-clock ticks */
hipError_t apus_launch_delay(unsigned long long ticks, hipStream_t st);

/* row r of h codes / scales (fp32 when hs_f32, else E8M0 bytes) to row
 * pair_of_row[r] (identity when null) of codes / e8m0 */
hipError_t apus_launch_moe_h_gather(const uint8_t *hc, const void *hs, int hs_f32,
                                    const int32_t *pair_of_row, int rows, int N, uint8_t *codes,
                                    uint8_t *e8m0, hipStream_t st);

/* h = bf16(silu(min(g, limit)) * clamp(u, +-limit)) elementwise (no clamp
 * when limit <= 0) */
hipError_t apus_launch_swiglu(const float *g, const float *u, size_t n, float limit, float *h,
                              hipStream_t st);

/* one tensor of every expert of a store layer, generated in place (MXFP4
 * weights what 0 / E8M0 scales what 1; MFMA-tiled when tiled): equal to
 * apus_launch_fill of stream sid0 + 8 e followed by apus_launch_pack */
hipError_t apus_launch_store_fill(uint8_t *base, size_t stride, int E, int O, int K, int what,
                                  int tiled, uint64_t seed, uint64_t sid0, hipStream_t st);

#endif /* APUS_INTERNAL_H */
