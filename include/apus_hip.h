/*
 * include/apus_hip.h — C ABI of the MI355X (gfx950) backend for apus's
 * quantized-matmul path: MXFP4 expert GEMV/GEMM, FP8-E4M3 block-scaled dense
 * GEMV/GEMM and the routed-expert SwiGLU dispatch.
 *
 * The surface mirrors apus's Metal backend boundary (c/backend_metal.h):
 * a function-pointer hook table that the engine's call sites try first,
 * enable/disable/is_enabled, counters, and direct entry points for
 * kernel-level tests. Every hook returns 0 when it produced the result and
 * nonzero when the shape or state is unsupported, in which case the caller
 * runs its CPU kernel (c/backend_metal.h:63-65, c/attn.h:412-414). Nothing
 * here crashes on an unsupported request.
 *
 * Numerics contract (same as c/backend_metal.h:19-29): activations are
 * BF16-rounded and quantised per 128 along K exactly as the CPU does
 * (bit-identical codes and scales); weights are consumed in their stored
 * E2M1/E4M3 + E8M0 form (decoded values bit-identical); the block dots run
 * on the F8F6F4 matrix cores with FP32 accumulation, so matmul outputs match
 * the CPU within FP32 summation-order error; BF16 output rounding happens
 * at the same points as on the CPU.
 *
 * Threading: one HIP stream per process, hooks are synchronous at the ABI
 * (outputs written before return) and not re-entrant, like the Metal hooks
 * (c/backend_metal.mm:38-39). Host-pointer entry points copy through pinned
 * staging; *_dev entry points take device pointers, are asynchronous on the
 * backend stream and never synchronise.
 *
 * Weight residency: dense weights passed by host pointer are uploaded once
 * and cached by host pointer (stable, immutable pointers assumed, as
 * c/backend_metal.h:38-43). Routed experts are cached by (layer, expert id),
 * never by pointer, in an HBM-resident expert store.
 */
#ifndef APUS_HIP_H
#define APUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- weight views: layout-identical to the reference types. When the
 * engine's own headers are included first their definitions are used. */
#ifndef APUS_ST_H
/* c/st.h:88-89 */
typedef struct { const uint8_t *codes, *scales; int64_t O, K; } ApusFp8W;
typedef struct { const uint8_t *packed, *scales; int64_t O, K; } ApusFp4W;
/* c/st.h:40-53 — a tensor view (the head GEMV hook takes one) */
typedef enum {
    APUS_ST_I8, APUS_ST_U8, APUS_ST_F8_E8M0, APUS_ST_F8_E4M3,
    APUS_ST_BF16, APUS_ST_F16, APUS_ST_F32, APUS_ST_I32, APUS_ST_I64,
    APUS_ST_OTHER
} ApusStDtype;
typedef struct {
    char        name[160];
    ApusStDtype dtype;
    int         ndim;
    int64_t     shape[8];
    const void *data;
    size_t      nbytes;
} ApusStTensor;
#endif

/* f32_linear hook flags (c/backend_metal.h:56-61) */
#define APUS_HIP_R_IN   1      /* BF16-round the input elements */
#define APUS_HIP_R_OUT  2      /* BF16-round the output */
#define APUS_HIP_W_BF16 4      /* w holds BF16 bits (uint16), not FP32 */

#ifndef APUS_FP4_H
/* c/fp4.h:184-188 — one entry of a grouped same-(O,K) MXFP4 GEMM */
typedef struct {
    const uint8_t *w, *ws;
    float *out;
    size_t m0, M;
} ApusFp4GemmEnt;
#endif

#ifndef APUS_MOE_H
/* c/moe.h:37-63 — MoE weights (only the routed-expert fields, layer_id and
 * hook_resolve/hook_ctx are read by this backend). */
typedef struct {
    int E, topk, inter, dim, hash;
    float route_scale, limit;
    const float *gate_w;
    const float *gate_bias;
    const int64_t *tid2eid;
    ApusFp4W *w1, *w2, *w3;
    ApusFp8W sw1, sw2, sw3;
    void *hook_ctx;
    int  (*hook_resolve)(void *ctx, int layer, int eid,
                         ApusFp4W *w1, ApusFp4W *w2, ApusFp4W *w3);
    void (*hook_hint)(void *ctx, int layer, int eid);
    void (*hook_layer_end)(void *ctx, int layer);
    void *hook_hint_ctx;
    void *hook_layer_end_ctx;
    int layer_id;
} ApusMoeW;
#endif

/* ---- hook table. The first three members are ApusBackendHooks
 * (c/backend_metal.h:73-80) in the same order; the last three are the new
 * call sites this backend adds (top of apus_fp4_linear, c/attn.h:432;
 * apus_fp4_gemm_mt_grouped, c/fp4.h:936; routed dispatch in
 * apus_moe_forward before c/moe.h:433). Unimplemented members are NULL. */
typedef struct {
    int (*fp8_linear)(const ApusFp8W *w, const float *x, float *out,
                      int M, int K, int O);
    int (*f32_linear)(const float *w, const float *x, float *out,
                      int M, int K, int O, int flags);
    int (*head_gemv)(const ApusStTensor *head, const float *x, float *out,
                     int64_t O, int64_t K);
    int (*fp4_linear)(const ApusFp4W *w, const float *x, float *out,
                      int M, int K, int O);
    int (*fp4_gemm_grouped)(const ApusFp4GemmEnt *ents, size_t n_ent,
                            const uint8_t *acodes, const float *as,
                            size_t O, size_t K);
    int (*moe_routed)(const ApusMoeW *w, const float *x, const int32_t *idx,
                      const float *wgt, int s, float *y);
} ApusHipHooks;

/* ---- lifecycle (c/backend_metal.h:84-91) ---- */
/* Initialise device 0, stream and weight caches; fill the hook table.
 * 0 on success; nonzero with err filled when no usable gfx950 device. */
int  apus_hip_enable(char *err, size_t errcap);
/* Detach: drop weight caches and device state. */
void apus_hip_disable(void);
int  apus_hip_is_enabled(void);
/* The hook table (all NULL until enabled). */
const ApusHipHooks *apus_hip_hooks(void);

/* ---- counters (c/backend_metal.h:93-97) ---- */
uint64_t apus_hip_bytes_uploaded(void);   /* weight bytes copied to HBM */
uint64_t apus_hip_bytes_resident(void);   /* weight bytes held in HBM */
uint64_t apus_hip_dispatches(void);       /* kernel launches issued */

/* ---- hooks, also callable directly. Host pointers; synchronous. ----
 * Inputs the matrix cores would read differently from the reference are
 * refused with a nonzero return (the caller then runs its CPU kernel): a
 * non-finite activation, an E8M0 scale byte 255 (+inf in c/fp4.h:209-217,
 * NaN on the matrix cores), an E4M3 weight or activation code 0x7F / 0xFF
 * (+-480 in c/fp4.h:255-260, NaN on the matrix cores), and pre-quantised
 * activation scales that are not finite powers of two. */
/* c/attn.h:408-430 apus_fp8_linear: bf16(x) -> act quant -> FP8 GEMM ->
 * bf16(out). x [M,K], out [M,O]. */
int apus_hip_fp8_linear(const ApusFp8W *w, const float *x, float *out,
                        int M, int K, int O);
/* c/attn.h:432-448 apus_fp4_linear: same with an MXFP4 weight. */
int apus_hip_fp4_linear(const ApusFp4W *w, const float *x, float *out,
                        int M, int K, int O);
/* c/attn.h:600-666 plain-weight linears (the f32_linear hook): FP32
 * accumulate over w [O, K] (FP32, or BF16 bits with APUS_HIP_W_BF16) and
 * x [M, K]; APUS_HIP_R_IN / R_OUT round input / output to BF16 (router gate:
 * 0; apus_bf16_linear: R_IN|R_OUT; wo_a groups: R_OUT|W_BF16). K % 8 == 0. */
int apus_hip_f32_linear(const float *w, const float *x, float *out, int M, int K, int O,
                        int flags);
/* c/model.h:638-647 apus_head_gemv: out [O] = head [O, K] (BF16 or F32 view)
 * times x [K], FP32 accumulate, unrounded. */
int apus_hip_head_gemv(const ApusStTensor *head, const float *x, float *out, int64_t O,
                       int64_t K);
/* c/fp4.h:936-986 apus_fp4_gemm_mt_grouped on pre-quantised activations
 * acodes [rows, K] / as [rows, K/128]; entry i writes ents[i].out [M, O]
 * (unrounded FP32) from activation rows [m0, m0+M). */
int apus_hip_fp4_gemm_grouped(const ApusFp4GemmEnt *ents, size_t n_ent,
                              const uint8_t *acodes, const float *as,
                              size_t O, size_t K);
/* c/moe.h:433-563: routed-expert dispatch for s tokens with the routing
 * already decided: idx/wgt [s, topk]. y [s, dim] receives the FP32 routed
 * sum (ApusMoeInterm.moe_routed, c/moe.h:564-565). Expert weights come
 * from w->hook_resolve when set, else from w->w1/w2/w3, and are kept in
 * HBM keyed by (w->layer_id, expert id). */
int apus_hip_moe_routed(const ApusMoeW *w, const float *x, const int32_t *idx,
                        const float *wgt, int s, float *y);

/* ---- direct kernel entry points (host pointers, synchronous) ---- */
/* c/fp4.h:293-321 via c/attn.h:393-403: BF16 round + per-128 act quant.
 * codes [M,K], scales [M, K/128]. K % 128 == 0. */
int apus_hip_act_quant(const float *x, int M, int K, uint8_t *codes,
                       float *scales);
/* c/fp4.h:815-848 apus_fp4_gemm_mt (scratch not needed): unrounded FP32
 * out [M,O] from pre-quantised activations. */
int apus_hip_fp4_gemm(const uint8_t *w, const uint8_t *ws,
                      const uint8_t *acodes, const float *as, float *out,
                      int M, int O, int K);
/* c/fp8.h:557-586 apus_fp8_gemm_mt; mirrors apus_metal_fp8_gemm
 * (c/backend_metal.h:110-112). */
int apus_hip_fp8_gemm(const uint8_t *w, const uint8_t *ws,
                      const uint8_t *acodes, const float *as, float *out,
                      int M, int O, int K);

/* weight-layout flag of the device entry points: MFMA-tiled weights */
#define APUS_HIP_W_TILED 0x100

/* ---- device-pointer entry points (asynchronous on the backend stream) ----
 * Same semantics as the host versions; all pointers are device pointers.
 * They exist for callers that keep activations in HBM between layers and
 * for measurement with inputs already resident. */
/* A group holding +-inf gets the scale +inf (as the reference's does) and
 * signed-zero codes for its finite elements; the GEMMs then return NaN for
 * that row (E8M0 255 is NaN on the matrix cores). Non-finite activations are
 * outside the contract of the *_dev entry points; the host-pointer entry
 * points refuse them (nonzero), so the caller's CPU kernel handles them. */
int apus_hip_act_quant_dev(const float *x, int M, int K, uint8_t *codes,
                           float *scales);
/* c/moe.h:113-135 apus_expert_swiglu: h[i] = bf16((g' * (1 / (1 + expf(-g'))))
 * * u') with g' = min(g, limit), u' = clamp(u, +-limit) when limit > 0, each
 * step rounded as written; n elements, device pointers, asynchronous. The
 * element function of every fused MoE kernel here; expf is ROCm's, so a
 * result can differ from the CPU's by one BF16 ulp where the product lies
 * within a few fp32 ulps of a BF16 rounding boundary. */
int apus_hip_swiglu_dev(const float *g, const float *u, size_t n, float limit, float *h);
/* round_out: bit 0 BF16-rounds the outputs; | APUS_HIP_W_TILED for weights
 * in the MFMA-tiled layout (K 2048/4096, O % 128 == 0). */
int apus_hip_fp4_gemm_dev(const uint8_t *w, const uint8_t *ws,
                          const uint8_t *acodes, const float *as, float *out,
                          int M, int O, int K, int round_out);
int apus_hip_fp8_gemm_dev(const uint8_t *w, const uint8_t *ws,
                          const uint8_t *acodes, const float *as, float *out,
                          int M, int O, int K, int round_out);
/* Grouped block-scaled GEMM over an entry table in device memory (the
 * device form of c/fp4.h:936-986, for callers that keep their grouping on
 * the device). Entry i computes, for m < M,
 *   out[orow(m) * ldo + o] = sum_k acodes[arow(m), k] * W[o, k]   (o < O)
 * with arow(m) = arows ? arows[m] : a0 + m and orow(m) = orows ? orows[m] :
 * o0 + m; W is MXFP4 [O, K/2] + [O, K/32] (wfmt 0) or FP8 [O, K] +
 * [ceil(O/128), K/128] (wfmt 1). max_m is an upper bound on every entry's
 * M, or 0 when unknown (entries with M > max_m may be left uncomputed).
 * round_out: BF16-round the outputs. wfmt | APUS_HIP_W_TILED: every W (and
 * FP4 scale array) is in the MFMA-tiled layout of apus_hip_pack_weights_dev
 * (then K must be 2048 or 4096 and O % 128 == 0). */
typedef struct {
    const uint8_t *w, *ws;
    float *out;
    const int32_t *arows, *orows;
    int32_t a0, o0, M, reserved;
} ApusHipGemmEnt;
int apus_hip_gemm_grouped_dev(int wfmt, const ApusHipGemmEnt *ents, int n_ent,
                              const uint8_t *acodes, const float *as, int O, int K,
                              int ldo, int round_out, int max_m);
/* Row-major <-> MFMA-tiled weights, device to device (no counterpart in the
 * reference: a resident-weight layout of this backend). The tiled layout
 * stores, for each 16-row tile and 128-wide K group, the 16-byte pieces in
 * matrix-core lane order, so the GEMM streams them with contiguous 1 KB
 * loads. wfmt 0 (MXFP4): weights [O, K/2] and scales [O, K/32] both move;
 * wfmt 1 (FP8): the weights move, the 128 x 128 tile scales keep their
 * layout (ws/tws unused). O % 16 == 0, K % 512 == 0, no overlap. Async on
 * the backend stream. */
int apus_hip_pack_weights_dev(int wfmt, const uint8_t *w, const uint8_t *ws, uint8_t *tw,
                              uint8_t *tws, int O, int K);
int apus_hip_unpack_weights_dev(int wfmt, const uint8_t *tw, const uint8_t *tws, uint8_t *w,
                                uint8_t *ws, int O, int K);
/* Linear = act quant + GEMM (+ BF16 out) with a caller workspace of
 * apus_hip_linear_workspace(M, K) bytes. */
size_t apus_hip_linear_workspace(int M, int K);
int apus_hip_fp4_linear_dev(const uint8_t *w, const uint8_t *ws,
                            const float *x, float *out, int M, int K, int O,
                            void *workspace);
int apus_hip_fp8_linear_dev(const uint8_t *w, const uint8_t *ws,
                            const float *x, float *out, int M, int K, int O,
                            void *workspace);
/* Either format: wfmt 0 (MXFP4) or 1 (FP8), | APUS_HIP_W_TILED for weights
 * in the MFMA-tiled layout (K 2048/4096, O % 128 == 0). */
int apus_hip_linear_dev(int wfmt, const uint8_t *w, const uint8_t *ws,
                        const float *x, float *out, int M, int K, int O,
                        void *workspace);

/* ---- HBM-resident expert store (replaces the NVMe/RAM tiers of
 * c/cache.h for the routed experts; keyed by (layer, expert id)) ---- */
typedef struct ApusHipStore ApusHipStore;
/* Reserve n_layers x E experts of shape gate/up [inter, dim], down
 * [dim, inter] (MXFP4), laid out as one slab per expert in HBM. When dim
 * and inter are 2048 or 4096 the matrices are held in the MFMA-tiled layout
 * of apus_hip_pack_weights_dev (apus_hip_store_tiled returns 1); otherwise
 * row-major. Returns NULL (err filled) when HBM cannot hold it. */
ApusHipStore *apus_hip_store_create(int n_layers, int E, int dim, int inter,
                                    char *err, size_t errcap);
void     apus_hip_store_free(ApusHipStore *st);
uint64_t apus_hip_store_bytes(const ApusHipStore *st);
/* Fill every expert with counter-based synthetic weights on the device
 * (nibbles uniform, E8M0 scales uniform in 118..130). Tensor t of
 * (layer, e) uses stream id ((layer * E + e) * 8 + t), t = 0..5 for
 * w1, w1s, w2, w2s, w3, w3s. */
int      apus_hip_store_fill_random(ApusHipStore *st, uint64_t seed);
/* Upload one expert from host memory (row-major, c/st.h ApusFp4W); packed
 * into the store's layout. */
int      apus_hip_store_put(ApusHipStore *st, int layer, int eid,
                            const ApusFp4W *w1, const ApusFp4W *w2,
                            const ApusFp4W *w3);
/* Device pointers of one expert's six tensors (w1, w1s, w2, w2s, w3, w3s),
 * in the store's layout (apus_hip_unpack_weights_dev turns a tiled matrix
 * back into the row-major form of c/st.h). */
int      apus_hip_store_get(const ApusHipStore *st, int layer, int eid,
                            const uint8_t *ptrs[6]);
/* 1 when the store holds its matrices MFMA-tiled. */
int      apus_hip_store_tiled(const ApusHipStore *st);
/* Workspace bytes for apus_hip_moe_routed_dev with s tokens x topk. */
size_t   apus_hip_moe_workspace(const ApusHipStore *st, int s, int topk);
/* Routed dispatch of one layer with everything in HBM: x [s, dim] f32,
 * idx/wgt [s, topk] (device), y [s, dim] f32 (device). Asynchronous. */
int      apus_hip_moe_routed_dev(const ApusHipStore *st, int layer,
                                 const float *x, const int32_t *idx,
                                 const float *wgt, int s, int topk,
                                 float limit, float *y, void *workspace);

/* apus_hip_moe_routed_dev plus a dense FP8 linear of the same x, e.g. a
 * shared expert's fused gate/up projection: dense_out [s, 2*inter] =
 * bf16(W x) (c/attn.h:408-430 semantics) for W [2*inter, dim] E4M3 with
 * 128 x 128 E8M0 tile scales dws (MFMA-tiled when dense_tiled). With the
 * one-token kernels (s * topk <= 32, topk 6 or 8, dim and inter 2048 or
 * 4096) the linear runs inside the routed w1/w3 launch, so the pair costs
 * two launches instead of three; otherwise it is its own launch on the
 * quantised x. No counterpart in the reference (a co-scheduling of two of
 * its calls). Device pointers, asynchronous. */
int      apus_hip_moe_routed_dense_dev(const ApusHipStore *st, int layer, const float *x,
                                       const int32_t *idx, const float *wgt, int s, int topk,
                                       float limit, float *y, void *workspace,
                                       const uint8_t *dw, const uint8_t *dws, int dense_tiled,
                                       float *dense_out);

/* apus_hip_moe_routed_dev without a caller workspace, for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The
 * workspace is a library-owned static device array of
 * apus_hip_moe_noalloc_max() bytes (64 MiB: the routed dispatch of up to
 * ~256 tokens x top-6 at dim 4096, inter 2048; larger calls are refused
 * with an error naming the bytes needed); the call itself allocates nothing
 * (apus_hip_enable must have run first). Every call on a GPU shares that
 * GPU's array and it keeps the last call's contents (nothing in it needs
 * to start at zero): calls that overlap on one GPU (other threads, other
 * processes) race; with a concurrency lane other than lane 0 selected the
 * call is refused. Results are bit-identical to apus_hip_moe_routed_dev. */
size_t   apus_hip_moe_noalloc_max(void);
int      apus_hip_moe_routed_dev_noalloc(const ApusHipStore *st, int layer,
                                         const float *x, const int32_t *idx,
                                         const float *wgt, int s, int topk,
                                         float limit, float *y);

/* Read-back of the routed dispatch's quantised SwiGLU activations (the w2
 * input h = act_quant(swiglu(bf16 g, bf16 u)), c/moe.h:113-126, :309-314)
 * from the workspace of the latest apus_hip_moe_routed_dev call with the same
 * store, s, topk and workspace: codes [s*topk, inter] E4M3 and e8m0
 * [s*topk, inter/128] scale bytes, row p = t*topk + j (device pointers,
 * asynchronous, stream-ordered after that call). No counterpart in the
 * reference (which keeps h internal): it lets a checker test the w1/w3 and
 * w2 stages of the dispatch separately. Pairs with an expert id outside
 * [0, E) are not written. */
int      apus_hip_moe_routed_h(const ApusHipStore *st, int s, int topk, const void *workspace,
                               uint8_t *codes, uint8_t *e8m0);

/* Plain-weight linear on device pointers (asynchronous): same semantics and
 * flags as apus_hip_f32_linear. */
int      apus_hip_wlinear_dev(const void *w, const float *x, float *out, int M, int K,
                              int O, int flags);

/* ---- apus model containers: routed-expert slabs on disk -> the store ----
 *
 * An apus container is a directory with model.safetensors.index.json (or
 * <dir>/weights/...) whose "weight_map" names the shard of every tensor; the
 * six tensors of a routed expert (layers.L.ffn.experts.E.w{1,2,3}.{weight,
 * scale}; MTP blocks: mtp.K.ffn.experts..., store layer n_main + K) lie back
 * to back in one shard (tools/convert.py:91-93), forming one slab per expert.
 * The index follows apus_store_open (c/cache.h:1030-1110, slab derivation
 * :431-509): 6 of 6 tensors per expert, one shard, contiguous, I8 weights
 * [O, K/2] with F8_E8M0 scales [O, K/32], one slab size for all experts. */
typedef struct {
    int32_t  shard;           /* index of the shard file (apus_hip_container_shard) */
    int32_t  pad;
    uint64_t off, len;        /* absolute file offset and bytes of the slab */
    uint32_t rel[6];          /* offsets of w1, w1s, w2, w2s, w3, w3s in the slab */
    int64_t  O[3], K[3];      /* logical shapes of w1, w2, w3 */
} ApusHipSlabRec;
typedef struct ApusHipContainer ApusHipContainer;
/* Host only (no device use). n_layers counts main + MTP expert layers. */
ApusHipContainer *apus_hip_container_open(const char *model_dir, int n_layers, int n_mtp,
                                          int n_experts, char *err, size_t errcap);
void     apus_hip_container_close(ApusHipContainer *c);
int      apus_hip_container_slab(const ApusHipContainer *c, int layer, int eid,
                                 ApusHipSlabRec *out);
/* path of shard i (NULL when out of range) */
const char *apus_hip_container_shard(const ApusHipContainer *c, int i);
/* Read every expert slab of the container into the store (its layers and
 * experts must match; w1/w3 [inter, dim], w2 [dim, inter]), re-laid out as
 * the store keeps them. io_threads readers (<= 0: 4) pread slabs into pinned
 * host buffers while earlier ones upload. Synchronous; 0 on success. */
int      apus_hip_store_load(ApusHipStore *st, const ApusHipContainer *c, int io_threads,
                             char *err, size_t errcap);

/* The whole MoE sublayer of one layer on the device (c/moe.h:369-595,
 * apus_moe_forward): router scores sqrt(softplus(gate_w x)) (c/moe.h:352-367),
 * expert choice by stable top-k of the scores plus gate_bias or by the hash
 * table (tid2eid[ids[t]]), weights sp / sum * route_scale, routed experts from
 * the store, the FP8 shared expert, and out = bf16(routed + shared). All
 * pointers are device pointers; asynchronous. Router scores agree with the
 * CPU's within fp32 rounding (different summation order, ROCm libm), so a
 * near-tie at the top-k boundary can choose differently. */
typedef struct {
    const float *gate_w;      /* [E, dim] fp32 */
    const float *gate_bias;   /* [E] selection bias (routing by scores) */
    const int64_t *tid2eid;   /* [*, topk] expert ids per token id (hash != 0) */
    int hash;
    float route_scale, limit;
    /* shared expert, FP8-E4M3 with 128 x 128 E8M0 tile scales:
     * w1, w3 [inter, dim], w2 [dim, inter] */
    const uint8_t *sw1, *sw1s, *sw2, *sw2s, *sw3, *sw3s;
    int shared_tiled;         /* shared weights in the MFMA-tiled layout */
} ApusHipMoeLayer;
/* Optional intermediates (c/moe.h:64-71 ApusMoeInterm); NULL members skipped. */
typedef struct {
    float *router_scores;     /* [s, E] */
    int32_t *router_idx;      /* [s, topk] */
    float *router_w;          /* [s, topk] */
    float *moe_routed;        /* [s, dim] */
    float *moe_shared;        /* [s, dim] */
} ApusHipMoeInterm;
size_t   apus_hip_moe_forward_workspace(const ApusHipStore *st, int s, int topk);
int      apus_hip_moe_forward_dev(const ApusHipStore *st, int layer,
                                  const ApusHipMoeLayer *ml, const float *x,
                                  const int64_t *ids, int s, int topk, float *out,
                                  const ApusHipMoeInterm *interm, void *workspace);

/* ---- device memory and timing helpers (tests and benchmarks) ---- */
void *apus_hip_malloc(size_t bytes);
int   apus_hip_free(void *p);
int   apus_hip_h2d(void *dst, const void *src, size_t bytes);
int   apus_hip_d2h(void *dst, const void *src, size_t bytes);
/* Asynchronous memset on the backend stream; returns nonzero (and does
 * nothing) while a graph capture is open on the backend stream or the
 * selected lane: memset nodes are not recorded into graphs. */
int   apus_hip_memset(void *dst, int value, size_t bytes);
/* device-to-device copy on the current lane (asynchronous) */
int   apus_hip_d2d(void *dst, const void *src, size_t bytes);
int   apus_hip_fill_random(void *dst, size_t bytes, uint64_t seed,
                           uint64_t stream_id, int kind);
int   apus_hip_synchronize(void);
/* Events on the backend stream: record a start mark, later the elapsed
 * milliseconds since it (synchronises on the end event). */
int   apus_hip_timer_start(void);
float apus_hip_timer_stop(void);
/* Hold the backend stream on the device for delay_us microseconds
 * (0..10^6): a one-wave kernel sleeps that long. Work the host queues right
 * after this call (warm-up launches, a timer start, a graph replay) then
 * runs back to back once the delay ends, so a timed interval measures the
 * device's execution, not the host's submission. No counterpart in the
 * reference (measurement helper). */
int   apus_hip_stream_delay(int delay_us);
/* Concurrency lanes: extra HIP streams for the *_dev entry points, so that
 * independent work (e.g. GEMVs of different experts) can overlap. Lane 0 is
 * the backend stream. apus_hip_lanes(n) creates lanes 1..n-1 (n <= 8);
 * apus_hip_lane(i) routes later *_dev launches to lane i; apus_hip_fork()
 * makes every lane wait for the work issued so far on lane 0; apus_hip_join()
 * makes lane 0 wait for every lane and selects lane 0 again. Fork/join are
 * recorded into a graph when issued during capture. Host-pointer entry points
 * always use lane 0. */
int   apus_hip_lanes(int n);
int   apus_hip_lane(int i);
int   apus_hip_fork(void);
int   apus_hip_join(void);
/* Capture the launches issued on the backend stream between begin and end
 * into one HIP graph, then replay it (asynchronously) `times` times. Only
 * *_dev entry points may be issued while capturing. */
int   apus_hip_graph_begin(void);
int   apus_hip_graph_end(void);
int   apus_hip_graph_replay(int times);
/* Last error message of this thread ("" when none). */
const char *apus_hip_last_error(void);
/* The one-launch one-token MoE layer (dim 4096, inter 2048, top-6, one
 * token, no fused shared expert or routing: w1/w3, a grid-wide barrier and
 * w2 in one kernel of 256 resident workgroups, on lane 0; y bit-identical to
 * the two-launch path). mode 1 turns it on (only where 256 workgroups fit
 * at once), 0 off (two launches per layer), -1 leaves it; the environment
 * variable APUS_HIP_LAYER1=0 turns it off at start-up. The barrier wait is
 * bounded (about a second); a workgroup that gives up writes NaN into its
 * 16 columns of y (and of the fused bf16(y + add) output) and flags the
 * fault, so a result is never wrong and finite. The next
 * apus_hip_synchronize (and every host-pointer hook's own wait) then returns
 * nonzero with an error naming the fault; a caller that waits on the stream
 * by other means polls the count here. With faults: waits for lane 0 and
 * stores the number of workgroups that gave up since the last such read
 * (the barrier words are then reset). Returns 1 when on, 0 when off, -1 on
 * error. No counterpart in the reference (a launch-structure switch). */
int   apus_hip_layer1(int mode, unsigned *faults);
/* Polls of the release word before a one-launch layer's barrier wait gives
 * up (default 2^23, about a second); 0 makes every wait give up at once.
 * A test hook for the fault path above (every kernel still exits normally).
 * No counterpart in the reference. */
int   apus_hip_layer1_spin_limit(unsigned spins);
/* Device name and compute-unit count of the current device. */
int   apus_hip_device_info(char *name, size_t cap, int *cus);

/* Device self-check: the hardware E4M3 conversion the kernels use for
 * activation codes equals the integer round-to-nearest-even encoder
 * (apus_hip_host_e4m3_quant, c/fp4.h:219-253) for every fp32 input with
 * |x| <= 448, both signs. No counterpart in the reference: it proves the
 * precondition of using the hardware instruction. Synchronous. */
int   apus_hip_check_e4m3_hw(unsigned *mismatches, unsigned *last_bad_bits);

/* ---- host twins of the device numerics (no GPU needed) ---- */
float    apus_hip_host_bf16_round(float x);
uint8_t  apus_hip_host_e4m3_quant(float x);
float    apus_hip_host_act_scale(float amax);

#ifdef __cplusplus
}
#endif

#endif /* APUS_HIP_H */
