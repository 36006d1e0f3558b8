/*
 * oracle/ref_shim.c — builds the reference's OWN CPU kernels (c/fp4.h,
 * c/fp8.h, c/attn.h linears, c/moe.h dispatch, c/cache.h expert store,
 * c/model.h head GEMV (with c/layer.h, which it needs),
 * c/pool.h, c/x86.h) from the
 * sources where they lie under the apus checkout (-I <apus>/c) into
 * oracle/_ref/libapus_ref.so. Nothing from the reference is copied here:
 * this file only instantiates the header-only implementations and adds a
 * few exported wrappers for entry points the headers keep static.
 *
 * TEST INFRASTRUCTURE ONLY: used to pin the oracle restatement and as the
 * measured CPU baseline (kind "reference") in bench.py.
 */
#define APUS_COMPAT_IMPLEMENTATION
#define APUS_FP4_IMPLEMENTATION
#define APUS_FP8_IMPLEMENTATION
#define APUS_JSON_IMPLEMENTATION
#define APUS_ST_IMPLEMENTATION
#define APUS_MHC_IMPLEMENTATION
#define APUS_ATTN_IMPLEMENTATION
#define APUS_MOE_IMPLEMENTATION
#define APUS_CACHE_IMPLEMENTATION
#define APUS_LAYER_IMPLEMENTATION
#define APUS_MODEL_IMPLEMENTATION
#include "compat.h"
#include "fp4.h"
#include "fp8.h"
#include "json.h"
#include "st.h"
#include "mhc.h"
#include "attn.h"
#include "moe.h"
#include "cache.h"
#include "layer.h"
#include "model.h"

#include <stdlib.h>
#include <string.h>

/* c/moe.h:113-126 is static; expose the elementwise SwiGLU range */
void ref_swiglu(const float *g, const float *u, float *h, size_t n,
                float limit) {
    ApusSwigluJob j = { g, u, h, limit };
    apus_expert_swiglu_range(&j, 0, n);
}

unsigned long ref_x86_avx2_hits(void) { return apus_x86_avx2_hits(); }
int ref_pool_threads(void) { return apus_pool_threads(); }

/* Run the real apus_moe_forward (c/moe.h:369) with hash routing so the
 * caller fixes the expert ids: tid2eid[t*topk+j] = idx[t*topk+j], ids[t]=t.
 * Routing weights come from the gate scores as in the reference; they are
 * returned in router_w so a restatement can use the identical weights.
 * The shared expert runs on all-zero FP8 weights (its output is not used:
 * routed_y is ApusMoeInterm.moe_routed, the routed-only FP32 sum). */
int ref_moe_routed(int E, int topk, int dim, int inter, float route_scale,
                   float limit, const float *gate_w,
                   const uint8_t *const *w1, const uint8_t *const *w1s,
                   const uint8_t *const *w2, const uint8_t *const *w2s,
                   const uint8_t *const *w3, const uint8_t *const *w3s,
                   const float *x, const int32_t *idx, int s,
                   float *router_w, float *routed_y, float *out) {
    ApusMoeW w;
    memset(&w, 0, sizeof w);
    w.E = E; w.topk = topk; w.inter = inter; w.dim = dim; w.hash = 1;
    w.route_scale = route_scale; w.limit = limit;
    w.gate_w = gate_w;
    int64_t *tid2eid = malloc((size_t)s * topk * sizeof(int64_t));
    int64_t *ids = malloc((size_t)s * sizeof(int64_t));
    for (int i = 0; i < s * topk; i++) tid2eid[i] = idx[i];
    for (int t = 0; t < s; t++) ids[t] = t;
    w.tid2eid = tid2eid;
    ApusFp4W *a1 = calloc((size_t)E, sizeof(ApusFp4W));
    ApusFp4W *a2 = calloc((size_t)E, sizeof(ApusFp4W));
    ApusFp4W *a3 = calloc((size_t)E, sizeof(ApusFp4W));
    for (int e = 0; e < E; e++) {
        a1[e] = (ApusFp4W){ w1[e], w1s[e], inter, dim };
        a2[e] = (ApusFp4W){ w2[e], w2s[e], dim, inter };
        a3[e] = (ApusFp4W){ w3[e], w3s[e], inter, dim };
    }
    w.w1 = a1; w.w2 = a2; w.w3 = a3;
    size_t nsd = (size_t)((inter + 127) / 128) * (size_t)((dim + 127) / 128);
    uint8_t *z1 = calloc((size_t)inter * dim, 1), *z2 = calloc((size_t)inter * dim, 1);
    uint8_t *z3 = calloc((size_t)inter * dim, 1);
    uint8_t *zs = malloc(nsd);
    memset(zs, 127, nsd);
    w.sw1 = (ApusFp8W){ z1, zs, inter, dim };
    w.sw2 = (ApusFp8W){ z2, zs, dim, inter };
    w.sw3 = (ApusFp8W){ z3, zs, inter, dim };
    int32_t *ridx = malloc((size_t)s * topk * sizeof(int32_t));
    ApusMoeInterm im;
    memset(&im, 0, sizeof im);
    im.router_w = router_w;
    im.router_idx = ridx;
    im.moe_routed = routed_y;
    apus_moe_forward(&w, x, ids, s, out, &im);
    int ok = memcmp(ridx, idx, (size_t)s * topk * sizeof(int32_t)) == 0;
    free(tid2eid); free(ids); free(a1); free(a2); free(a3);
    free(z1); free(z2); free(z3); free(zs); free(ridx);
    return ok ? 0 : -1;
}

/* The real apus_moe_forward with every part live: gate (+bias) or hash
 * routing, MXFP4 routed experts, FP8 shared expert. Returns the layer output
 * and the intermediates the reference exposes (ApusMoeInterm, c/moe.h:64-71). */
void ref_moe_forward(int E, int topk, int dim, int inter, float route_scale,
                     float limit, int hash, const float *gate_w, const float *gate_bias,
                     const int64_t *tid2eid, const int64_t *ids,
                     const uint8_t *const *w1, const uint8_t *const *w1s,
                     const uint8_t *const *w2, const uint8_t *const *w2s,
                     const uint8_t *const *w3, const uint8_t *const *w3s,
                     const uint8_t *sw1, const uint8_t *sw1s, const uint8_t *sw2,
                     const uint8_t *sw2s, const uint8_t *sw3, const uint8_t *sw3s,
                     const float *x, int s, float *out, float *routed, float *shared,
                     float *sp, int32_t *idx, float *wgt) {
    ApusMoeW w;
    memset(&w, 0, sizeof w);
    w.E = E; w.topk = topk; w.inter = inter; w.dim = dim; w.hash = hash;
    w.route_scale = route_scale; w.limit = limit;
    w.gate_w = gate_w; w.gate_bias = gate_bias; w.tid2eid = tid2eid;
    ApusFp4W *a1 = calloc((size_t)E, sizeof(ApusFp4W));
    ApusFp4W *a2 = calloc((size_t)E, sizeof(ApusFp4W));
    ApusFp4W *a3 = calloc((size_t)E, sizeof(ApusFp4W));
    for (int e = 0; e < E; e++) {
        a1[e] = (ApusFp4W){ w1[e], w1s[e], inter, dim };
        a2[e] = (ApusFp4W){ w2[e], w2s[e], dim, inter };
        a3[e] = (ApusFp4W){ w3[e], w3s[e], inter, dim };
    }
    w.w1 = a1; w.w2 = a2; w.w3 = a3;
    w.sw1 = (ApusFp8W){ sw1, sw1s, inter, dim };
    w.sw2 = (ApusFp8W){ sw2, sw2s, dim, inter };
    w.sw3 = (ApusFp8W){ sw3, sw3s, inter, dim };
    ApusMoeInterm im;
    memset(&im, 0, sizeof im);
    im.router_scores = sp;
    im.router_idx = idx;
    im.router_w = wgt;
    im.moe_routed = routed;
    im.moe_shared = shared;
    apus_moe_forward(&w, x, ids, s, out, &im);
    free(a1); free(a2); free(a3);
}

/* c/attn.h:393-403 apus_act_quant_rows is static; run it over M rows
 * exactly as apus_fp4_linear / apus_fp8_linear do (BF16 round + act quant). */
void ref_act_quant_rows(const float *x, int M, int K, float *xb, uint8_t *codes,
                        float *scales) {
    ApusActQuantJob aq = { x, xb, codes, scales, K, apus_fp4_act_blocks((size_t)K) };
    apus_act_quant_rows(&aq, 0, (size_t)M);
}


/* The reference expert store's slab index (c/cache.h:1030-1110
 * apus_store_open, :431-509 derivation), opened synchronously with no usage
 * file. Writes, per (layer, expert) in layer-major order: the shard name's
 * index in `names` (first-use order, each name NUL-terminated in a
 * name_cap-byte field), the slab's file offset, length, member offsets and
 * w1..w3 shapes, and the expert's slab bytes read through
 * apus_store_resolve when `slabs` is non-NULL. Returns 0, or -1 with err. */
int ref_store_index(const char *dir, int n_layers, int n_mtp, int E, int32_t *shard,
                    uint64_t *off, uint64_t *len, uint32_t *rel, int64_t *O, int64_t *K,
                    char *names, int name_cap, int *n_names, uint8_t *slabs,
                    char *err, size_t errcap) {
    ApusStoreCfg cfg = {0};
    cfg.n_layers = n_layers;
    cfg.n_experts = E;
    cfg.n_mtp = n_mtp;
    cfg.io_threads = -1;
    cfg.nocache = -1;
    cfg.usage_path = "";
    ApusStore *st = apus_store_open(dir, &cfg, err, errcap);
    if (!st) return -1;
    *n_names = 0;
    for (int i = 0; i < n_layers * E; i++) {
        const ApusSlabRec *r = &st->recs[i];
        int sid = -1;
        for (int k = 0; k < st->shards_n; k++)
            if (st->shards[k].lz == r->lz) sid = k;
        shard[i] = sid;
        off[i] = r->off;
        len[i] = r->len;
        for (int j = 0; j < 6; j++) rel[6 * i + j] = r->rel[j];
        for (int t = 0; t < 3; t++) { O[3 * i + t] = r->O[t]; K[3 * i + t] = r->K[t]; }
    }
    for (int k = 0; k < st->shards_n; k++)
        snprintf(names + (size_t)k * name_cap, (size_t)name_cap, "%s", st->shards[k].name);
    *n_names = st->shards_n;
    if (slabs) {
        for (int i = 0; i < n_layers * E; i++) {
            ApusFp4W w[3];
            if (apus_store_resolve(st, i / E, i % E, &w[0], &w[1], &w[2])) {
                snprintf(err, errcap, "resolve %d.%d failed", i / E, i % E);
                apus_store_close(st);
                return -1;
            }
            /* members in canonical order at their slab offsets */
            const uint8_t *src[6] = {w[0].packed, w[0].scales, w[1].packed, w[1].scales,
                                     w[2].packed, w[2].scales};
            const ApusSlabRec *r = &st->recs[i];
            const size_t sz[6] = {
                (size_t)(r->O[0] * r->K[0] / 2), (size_t)(r->O[0] * r->K[0] / 32),
                (size_t)(r->O[1] * r->K[1] / 2), (size_t)(r->O[1] * r->K[1] / 32),
                (size_t)(r->O[2] * r->K[2] / 2), (size_t)(r->O[2] * r->K[2] / 32)};
            for (int j = 0; j < 6; j++)
                memcpy(slabs + (size_t)i * r->len + r->rel[j], src[j], sz[j]);
            apus_store_layer_end(st, i / E);
        }
    }
    apus_store_close(st);
    return 0;
}

/* One token through one decode layer of BASELINE config 4 on apus's own CPU
 * kernels: the FP8 [O8, dim] projection of x (apus_fp8_linear, c/attn.h:
 * 408-430) and the routed experts of the token as apus_moe_forward's s == 1
 * path runs them (c/moe.h:435-450: apus_expert per pair, then y += w * eo
 * in j order). w1..w3s hold the topk experts' tensors. Used as the timed
 * CPU baseline of config 4. */
void ref_decode_layer(int topk, int dim, int inter, float limit,
                      const uint8_t *const *w1, const uint8_t *const *w1s,
                      const uint8_t *const *w2, const uint8_t *const *w2s,
                      const uint8_t *const *w3, const uint8_t *const *w3s,
                      const float *wgt, const uint8_t *pw, const uint8_t *pws, int O8,
                      const float *x, float *y, float *proj) {
    ApusFp8W p = { pw, pws, O8, dim };
    apus_fp8_linear(&p, x, proj, 1, dim, O8);
    float *eo = malloc((size_t)dim * sizeof(float));
    memset(y, 0, (size_t)dim * sizeof(float));
    for (int j = 0; j < topk; j++) {
        ApusFp4W e1 = { w1[j], w1s[j], inter, dim };
        ApusFp4W e2 = { w2[j], w2s[j], dim, inter };
        ApusFp4W e3 = { w3[j], w3s[j], inter, dim };
        apus_expert(&e1, &e2, &e3, 0, limit, x, dim, inter, eo);
        for (int i = 0; i < dim; i++) y[i] += wgt[j] * eo[i];
    }
    free(eo);
}
