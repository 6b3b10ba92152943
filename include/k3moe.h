/* k3moe.h - C ABI of the MI355X routed-expert MoE layer.
 *
 * Three groups of entry points live here.
 *
 *  1. DROP-IN. The engine's own MoE entry points, with the engine's names, signatures,
 *     struct layouts and error behaviour, so a decoder layer that calls k3_moe() links
 *     against this library unchanged. Host pointers, synchronous. Each one cites the
 *     reference declaration it replaces.
 *
 *  2. DEVICE API (k3g_*). The same layer with device pointers, an explicit HIP stream and
 *     a preallocated workspace: no allocation and no host synchronisation on the hot
 *     path. The drop-in functions are built on it.
 *
 *  3. HBM EXPERT CACHE (k3gc_*). The engine's expert cache re-planned for HBM: slots in
 *     device memory, misses copied from a pinned host bank on a side stream. It is a
 *     K3ExpertSrc whose get() hands back DEVICE pointers.
 *
 * Types shared with the engine (K3Cfg, K3ExpertQ, K3ExpertSrc, K3MoeW) are declared
 * only when the engine's k3.h has not already been included; the layouts are the
 * engine's, field for field, because callers build these structs and pass them in.
 */
#ifndef K3MOE_H
#define K3MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ===================================================================== engine types == */
#ifndef K3_H
/* Layout of include/k3/k3.h:73-120. Only the MoE fields (n_experts .. latent_norm,
 * hidden, rms_eps, situ_b1/b2) are read by this library; the rest are carried so that a
 * K3Cfg built by the engine's config loader can be passed straight in. */
typedef struct {
    int hidden;
    int n_layers;
    int vocab;
    float rms_eps;

    int kda_heads;
    int kda_head_dim;
    int conv_k;
    float gate_lb;

    int n_heads;
    int q_lora;
    int kv_lora;
    int qk_nope;
    int qk_rope;
    int v_head;
    int mla_out_gate;

    int n_experts;
    int topk;
    int n_shared;
    int latent;
    int moe_inter;
    float routed_scale;
    int moe_renorm;
    int latent_norm;

    int first_dense;
    int dense_inter;

    int attn_res_block;

    float situ_b1;
    float situ_b2;

    int  n_full_attn;
    int *full_attn;
} K3Cfg;

/* Weight tags, include/k3/k3.h:270. */
enum { K3_WF32 = 0, K3_WBF16 = 1, K3_WI8 = 2 };

/* One MXFP4 expert, include/k3/k3.h:323-327. Row-major packed nibbles (low nibble is
 * the even element) plus one E8M0 byte per 32 elements of a row. */
typedef struct {
    const unsigned char *p1, *s1;        /* w1 gate  [inter][latent/2], [inter][latent/32] */
    const unsigned char *p3, *s3;        /* w3 up                                          */
    const unsigned char *p2, *s2;        /* w2 down  [latent][inter/2], [latent][inter/32] */
} K3ExpertQ;

/* Expert source plugin, include/k3/k3.h:332-355. */
typedef struct K3ExpertSrc {
    int (*get)(struct K3ExpertSrc *self, int layer, int expert, K3ExpertQ *out);
    int (*getmany)(struct K3ExpertSrc *self, int layer, const int *experts, int n);
    int (*resident)(struct K3ExpertSrc *self, int layer, int expert, K3ExpertQ *out);
    void *ctx;
} K3ExpertSrc;

/* One MoE layer's weights, include/k3/k3.h:357-380. Zero it before filling it.
 *
 * Extension, backward compatible because the engine would dereference NULL here:
 *   down == NULL  no latent down-projection (z = x; requires latent == hidden)
 *   up   == NULL  no latent up-projection   (out = routed aggregate)
 * That is the Kimi-K2 layer shape, which the engine otherwise expresses with bf16
 * identity matrices (exactly, at twice the traffic). */
typedef struct {
    const float *gate, *bias;
    const float *w1, *w3, *w2;
    const float *latent_norm;
    const void  *down, *up;
    const void  *sh1, *sh3, *sh2;
    int          wdt;
    struct K3ExpertSrc *src;
    int          layer;
    int          cache_only;
} K3MoeW;

#define K3_MXFP4_GROUP 32
#define K3_MAX_TOPK 64
#endif /* K3_H */

/* ================================================================ 1. drop-in ABI == */

/* Routed experts that could not be fetched and were left out of a sum.
 * Replaces include/k3/k3.h:388 (defined at src/core/k3_ops.c:108). Callers must check
 * it and fail the run when it changes. */
extern long k3_expert_drops;

/* Replaces include/k3/k3.h:241-243 (src/core/k3_ops.c:419-478). One token: logits =
 * W x (fp32 weights, double accumulation), sigmoid scores, top-k on score + bias,
 * weights gathered from the UNBIASED scores, renormalised with +1e-20, times
 * routed_scale. idx/w are written in descending biased-score order, ties to the lower
 * expert index. Runs on the GPU; the selection is bit-exact with the engine's. */
void k3_router(int *idx, float *w, const float *x, const float *W,
               const float *bias, int hidden, int n_experts, int topk,
               int renorm, float routed_scale);

/* Replaces include/k3/k3.h:382 (src/core/k3_ops.c:658-666). Same value. */
size_t k3_moe_scratch(const K3Cfg *c);

/* Replaces include/k3/k3.h:418-419 (src/core/k3_ops.c:556-656). x, out are host
 * [T][hidden] fp32. idx/wt receive the LAST token's routing, as in the engine. scratch
 * is accepted for ABI compatibility and not used: the GPU workspace is preallocated
 * per device. Weights are uploaded to HBM on first use and keyed by host address and
 * size; a sampled fingerprint of the bytes is checked every call, and a caller that
 * rewrites a weight buffer in place (a ring of layer buffers) calls
 * k3moe_invalidate_weights() on it. Experts come from w->src (MXFP4) or from the fp32
 * resident bank w->w1/w3/w2. A source that fails to deliver an expert bumps
 * k3_expert_drops, as the engine does.
 *
 * With bf16 shared and latent weights (wdt K3_WBF16) and experts from a source, the layer
 * runs on the matrix cores: the fused decode kernel (no latent, up to 4 tokens) or the
 * grouped GEMMs; an HBM expert cache (k3gc_*) with a tiled bank serves its experts in
 * place, any other source's experts are copied and tiled per call. Through an HBM cache
 * the tokens are run in groups whose experts fit the cache's unpinned slots, one cache
 * step each, so a cache of top-k + 1 slots serves any T without dropping an expert.
 * fp32 and int8-draft (K3_WI8) shared and latent weights run as per-row GEMVs; the int8
 * rows are summed in float in the GPU's order, within float rounding of the engine's
 * k3_matmul_q8 (which itself differs between its AVX2, NEON and plain builds). */
void k3_moe(float *out, const float *x, const K3MoeW *w, const K3Cfg *c,
            int T, int *idx, float *wt, float *scratch);

/* Replaces include/k3/k3.h:425-426 (src/core/k3_ops.c:689-808). Bit-identical routing
 * to k3_moe and the same per-token arithmetic; all T tokens go to the GPU as one batch. */
void k3_moe_prefill(float *out, const float *x, const K3MoeW *w, const K3Cfg *c,
                    int T, int *idx, float *wt, float *scratch);

/* Replaces include/k3/k3.h:559-560 (src/core/k3_ops.c:1770-1800). Exact. */
void k3_mxfp4_dequant(float *out, const unsigned char *packed,
                      const unsigned char *scales, int rows, int pcols, int group);

/* Replaces include/k3/k3.h:565-566 (src/core/k3_ops.c:1363-1768). Aborts on odd `in`
 * or group > 64, as the engine does (and on group < 1, which the engine divides by).
 * Each row carries ceil(in / group) E8M0 scale bytes; group 32 (the format's block,
 * K3_MXFP4_GROUP) runs the vectorised kernel, any other group one wave per row, reading
 * the nibbles as the engine's grouped path does (group g from byte g * (group / 2)).
 * Sums in float, within float rounding of the engine's double sums. */
void k3_matmul_mxfp4(float *y, const float *x, const unsigned char *packed,
                     const unsigned char *scales, int in, int rows, int group);

/* Drop every HBM copy of host weights made by k3_moe/k3_router. No reference
 * counterpart: the engine reads host weights in place. */
void k3moe_forget_weights(void);

/* Which kernels the last k3_moe / k3_moe_prefill call ran, as bits: 1 the staged VALU
 * kernels, 2 the fused decode kernel, 4 the grouped matrix-core GEMMs. No reference
 * counterpart (diagnostics). */
int k3moe_last_kernels(void);

/* Drop the HBM copies of host weights overlapping [host, host + bytes): the next call
 * uploads them again. For callers that reuse a weight buffer for other weights at the
 * same address (the engine's trunk ring, src/io/k3_trunk.c). The copies are also kept
 * within K3MOE_MIRROR_BYTES of device memory (default 64 GiB), least recently used
 * dropped first. No reference counterpart: the engine reads host weights in place. */
void k3moe_invalidate_weights(const void *host, size_t bytes);

/* ================================================= 1b. the engine's expert cache == */
/* The engine's checkpoint index and expert geometry, field for field
 * (src/io/k3_st.h:29-70, src/io/k3_load.h:29-43), declared only when the engine's own
 * headers have not been included: k3_cache_init reads the K3St that the engine's
 * k3_st_open filled in. */
#ifndef K3_ST_H
typedef enum { K3_DT_UNKNOWN = 0, K3_DT_U8, K3_DT_BF16, K3_DT_F16, K3_DT_F32,
               K3_DT_I8R } K3Dtype;
typedef struct {
    char     *name;
    int       shard;          /* index into K3St.fd[] */
    K3Dtype   dtype;
    int       ndim;
    int64_t   shape[4];
    int64_t   off;            /* absolute byte offset in the shard */
    int64_t   nbytes;
} K3Tensor;
#define K3_ST_ALIGN 4096
typedef struct {
    int       *fd;            /* one descriptor per shard */
    int       *dfd;           /* the same shards opened O_DIRECT, or -1 */
    char     **path;
    int        nshard;
    K3Tensor  *t;             /* every tensor */
    int        nt;
    int32_t   *bucket;        /* the engine's hash index (not read here) */
    int        nbucket;
    char      *strpool;
    size_t     strcap, strlen_;
} K3St;
#endif /* K3_ST_H */
#ifndef K3_LOAD_H
typedef struct {
    int64_t p_off, p_bytes;   /* packed nibbles, offset within the run */
    int64_t s_off, s_bytes;   /* E8M0 scales, offset within the run */
    int     rows, pcols;
    int     scols;
} K3QMat;
typedef struct {
    int     layer, expert;
    int     shard;
    int64_t off;              /* file offset of the run */
    int64_t nbytes;
    int     contiguous;
    K3QMat  m[3];             /* w1, w2, w3 */
} K3ExpertRef;
#endif /* K3_LOAD_H */

/* The engine's expert cache, src/cache/k3_cache.h:47-96, field for field, so that the
 * engine's main() (src/cli/k3_run.c:1144-1155, :1524-1534) reads nslot, slot_bytes and
 * the counters and wires &cache->src into every K3MoeW unchanged. Here the slots are in
 * HBM: arena is a DEVICE pointer, get() hands out device pointers (the tiled MXFP4 layout
 * when the checkpoint's experts have one, the checkpoint layout otherwise), and k3_moe /
 * k3_moe_prefill of this library run on them in place. A miss is read from the
 * checkpoint (O_DIRECT where the shard has it, the misses of one getmany in parallel)
 * into pinned staging and copied to its slot on a side stream. The fields mean what the
 * engine's mean; slot_of, key_of, used_at, pinned and hist are the cache's live arrays,
 * the counters are brought up to date by every call, ref[slot] is the geometry of the
 * expert a slot holds as k3_expert_ref gives it for a run in the checkpoint order
 * (w1p w1s w2p w2s w3p w3s; a run whose tensors are stored in another order is read as
 * six spans into that order) and pad[] stays 0. src.ctx belongs to the cache. */
#ifndef K3_CACHE_H
#define K3_SLOT_EMPTY     (-1)
#define K3_SLOT_INFLIGHT  (-2)
typedef struct {
    K3ExpertSrc  src;         /* first: pass &cache->src to K3MoeW */
    const K3St  *st;
    int          n_layers, n_experts;
    unsigned char *arena;     /* nslot * slot_bytes of HBM */
    int64_t      slot_bytes;
    int          nslot;
    int32_t     *slot_of;     /* [n_layers * n_experts] -> slot, or -1 */
    int32_t     *key_of;      /* [nslot] -> layer * n_experts + expert, EMPTY or INFLIGHT */
    uint64_t    *used_at;     /* [nslot] LRU stamp */
    unsigned char *pinned;    /* [nslot] */
    K3ExpertRef *ref;         /* [nslot] */
    int32_t     *pad;         /* [nslot] */
    uint64_t     clock;
    uint64_t     hits, misses, evictions, bytes_read;
    uint64_t     prefetch_reads;   /* misses brought in by getmany */
    double       load_seconds;     /* host time spent reading the checkpoint */
    uint32_t    *hist;        /* [n_layers * n_experts] requests */
    int32_t     *trace;       /* (layer, expert) pairs in request order */
    int64_t      ntrace, captrace;
} K3Cache;
#endif /* K3_CACHE_H */

/* Replaces src/cache/k3_cache.h:97-100 (src/cache/k3_cache.c:262-345). Sizes a slot from
 * the first routed expert found in the checkpoint (layers from cfg->first_dense on),
 * takes budget_bytes of HBM on the current device, and fails with a message when that is
 * fewer than topk + 1 slots. K3_NOPREFETCH set: no getmany, as in the engine. */
int  k3_cache_init(K3Cache *c, const K3St *st, const K3Cfg *cfg, int64_t budget_bytes);
/* Replaces src/cache/k3_cache.h:101 (k3_cache.c:347-353); call before the engine's
 * k3_st_close. */
void k3_cache_free(K3Cache *c);
/* Replaces src/cache/k3_cache.h:103-105 (k3_cache.c:367-375): 1 when the expert was
 * resident (and is now pinned or unpinned), 0 otherwise. */
int  k3_cache_pin(K3Cache *c, int layer, int expert, int pin);
/* Replaces src/cache/k3_cache.h:107-108 (k3_cache.c:377-380): 0, or -1 when it could
 * not be brought in. */
int  k3_cache_prefetch(K3Cache *c, int layer, int expert);
/* Replaces src/cache/k3_cache.h:110-111 (k3_cache.c:382-394, :396-424). */
void k3_cache_reset_stats(K3Cache *c);
void k3_cache_report(const K3Cache *c, const char *label);
/* Replaces src/cache/k3_cache.h:113-118 (k3_cache.c:355-365, :426-446): the engine's
 * JSON histogram and flat int32 (layer, expert) trace. */
int  k3_cache_dump_hist(const K3Cache *c, const char *path);
int  k3_cache_dump_trace(const K3Cache *c, const char *path);

/* ============================================================== 2. device API == */

typedef struct K3gCtx K3gCtx;        /* device, streams, workspace; opaque */

/* Byte geometry of one expert run in the order the checkpoint stores it
 * (src/io/k3_load.h:3-9): w1.packed w1.scale w2.packed w2.scale w3.packed w3.scale.
 * Offsets are relative to the run start. */
typedef struct {
    int64_t p1_off, s1_off, p2_off, s2_off, p3_off, s3_off;
    int64_t nbytes;
} K3gExpertLayout;

K3gExpertLayout k3g_expert_layout(int hidden, int inter);

/* A layer whose weights are already in HBM. All pointers are device pointers.
 *
 *   gate [n_experts][hidden] fp32, bias [n_experts] fp32 or NULL
 *   routed experts, running at width `latent`:
 *     expert_fmt 0: `experts`, a device array of n_experts K3ExpertQ holding device
 *                   pointers to MXFP4 matrices (entries of unrouted experts unused)
 *     expert_fmt 1: the fp32 resident bank w1/w3 [n_experts][inter][latent] and
 *                   w2 [n_experts][latent][inter] (the engine's fixture path)
 *     expert_fmt 2: as 0, but p1/p3/p2 point at matrices in the tiled MXFP4 layout
 *                   k3g_tile_mxfp4 writes (they carry their own scales; s1/s3/s2
 *                   unused). The fused decode kernel streams this layout at full line
 *                   granularity into the matrix cores; it serves up to 4 tokens a call.
 *   shared expert, tagged by wdt (K3_WF32, K3_WBF16, or K3_WI8: rows of an f32 scale
 *     then the row's int8 weights, as the engine's draft model stores them, summed in
 *     float with no bit-exactness promise, as the engine's k3_matmul_q8 gives none):
 *     sh1/sh3 [shared_inter][hidden], sh2 [hidden][shared_inter]; shared_inter == 0
 *     means none. shared_fmt 0: row-major;
 *     1: bf16 in the tiled layout k3g_tile_bf16 writes, for the shared expert and the
 *     latent projections alike (goes with expert_fmt 2)
 *   latent projections, tagged by wdt: down [latent][hidden], up [hidden][latent];
 *     NULL for the Kimi-K2 shape (latent == hidden). latent_norm [latent] or NULL.
 *   act_b1/act_b2: SiTU caps; a value >= 2^64 means uncapped (SwiGLU). */
typedef struct {
    int hidden, n_experts, topk, inter, shared_inter, latent;
    int renorm;
    float routed_scale;
    float act_b1, act_b2;
    float rms_eps;
    const float *gate, *bias;
    int expert_fmt;
    const K3ExpertQ *experts;
    const float *w1, *w3, *w2;
    int wdt;
    const void *sh1, *sh3, *sh2;
    const void *down, *up;
    const float *latent_norm;
    int shared_fmt;
} K3gLayer;

enum { K3G_EXPERT_MXFP4 = 0, K3G_EXPERT_F32 = 1, K3G_EXPERT_MXFP4_TILED = 2 };

/* Repack a device matrix from the checkpoint layout into the tiled layout the matrix
 * cores stream (asynchronous on `stream`; dst must not overlap the source).
 * MXFP4: rows % 16 == 0, cols % 32 == 0, packed [rows][cols/2] + scales [rows][cols/32]
 * (group 32); the tiled matrix takes k3g_tiled_mxfp4_bytes (cols padded to a multiple of
 * 512). bf16: rows % 16 == 0, cols % 32 == 0, [rows][cols] -> the same number of bytes.
 * Sizes are 0 and the calls return -1 for other shapes. No reference counterpart: the
 * engine reads the checkpoint layout in place. */
size_t k3g_tiled_mxfp4_bytes(int rows, int cols);
int  k3g_tile_mxfp4(void *dst, const void *packed, const void *scales, int rows, int cols,
                    void *stream);
size_t k3g_tiled_bf16_bytes(int rows, int cols);
int  k3g_tile_bf16(void *dst, const void *src, int rows, int cols, void *stream);

/* Create a context on `device` for layers of this shape (only the size fields of
 * `shape` are read) and up to max_tokens tokens per call. Allocates the whole workspace
 * once. Returns 0, or -1 with a message on stderr. */
int  k3g_ctx_create(K3gCtx **ctx, int device, const K3gLayer *shape, int max_tokens);
void k3g_ctx_destroy(K3gCtx *ctx);
void *k3g_ctx_stream(K3gCtx *ctx);   /* the context's compute stream (hipStream_t) */

/* Routing statistics since the context was created. Calls of up to 511 tokens (fp64
 * logits and a certified selection): [0] tokens whose certificate failed and were
 * re-routed in the engine's serial order, [1] selected experts of certified tokens whose
 * score the bound left unsettled and was recomputed exactly. Calls of 512 tokens or more
 * (bounded bf16 logits, then fp64 logits for the candidates only): [0] tokens with more
 * candidates than k, [1] candidate logits the any-order bound left open (settled by the
 * partial-sum bound or the serial chain), [2] candidates whose fp64 logit fell outside
 * its bounded interval (a live check of the bound; never expected). */
void k3g_ctx_stats(K3gCtx *ctx, int64_t *out, int n);

/* Per-stage timing with HIP events on the call's stream (off by default; turning it on
 * or off clears the totals). Stages: 0 router, 1 dispatch, 2 routed gate/up, 3 routed
 * down, 4 shared gate/up, 5 shared down, 6 combine, 7 latent projections, 8 the fused
 * decode kernel (the whole layer in one launch). */
void k3g_ctx_profile(K3gCtx *ctx, int on);
/* Totals since profiling was turned on: milliseconds and call counts per stage. Returns
 * the number of stages. */
int  k3g_ctx_stage_ms(K3gCtx *ctx, double *ms, int64_t *count, int n);

/* k3g_moe runs a Kimi-K2-shaped layer at up to 4 tokens as one fused persistent kernel
 * (default on); off forces the staged kernels. No reference counterpart. */
void k3g_ctx_set_fused(K3gCtx *ctx, int on);
/* The kernels the context's calls ran since the last clear: bit 0 the staged VALU kernels,
 * bit 1 the fused decode kernel, bit 2 the grouped GEMMs; clear != 0 resets it. */
int  k3g_ctx_paths(K3gCtx *ctx, int clear);

/* Routed experts of calls beyond the fused decode kernel on the FP4 x FP8 matrix cores
 * (v_mfma_scale_f32_16x16x128_f8f6f4): MXFP4 weights as stored, x and the activation h
 * quantised to MXFP8 (OCP MX: E4M3, an E8M0 scale per 32 values). Off by default (the
 * bf16 matrix cores, activations exact to 2^-17). The shared expert stays bf16. No
 * reference counterpart. */
void k3g_ctx_set_fp8(K3gCtx *ctx, int on);

/* Instrumentation: with a device buffer of 3 * tickets + 5 uint64, the fused kernel writes
 * for each ticket its start, the end of its waits and its end as wall-clock stamps
 * (100 MHz counter), then the top-k ticket's stamps after its wait, after its selection
 * and inside the selection. Calls on the grouped GEMMs write 4 uint64 per workgroup of
 * the routed gate/up launch (8 * 4 ceil(tiles / 32) * ceil(inter / 128) workgroups, tiles =
 * ceil(T topk / 128) + min(n_experts, T topk)), then of the routed down launch: wave 0's
 * start and end, column tile << 32 | feature tile, XCC << 32 | HW_ID. NULL turns it off.
 * No reference counterpart. */
void k3g_ctx_set_trace(K3gCtx *ctx, void *dev_buf);

/* Force the router's exact re-routing path (testing only): 0 normal, 1 every token
 * re-routes its candidate set, 2 every token recomputes the engine's float logit of every
 * expert (from a bounded sum in any order, the serial chain where the bound leaves the
 * float open), 3 as 2 with the serial chain for every logit. */
void k3g_ctx_force_exact(K3gCtx *ctx, int mode);

/* Router on the GPU for T tokens: x [T][hidden] fp32 -> idx [T][topk] int32,
 * wt [T][topk] fp32, device pointers. Bit-exact selection (see k3_router). */
int  k3g_router(K3gCtx *ctx, const K3gLayer *L, const float *x, int T,
                int32_t *idx, float *wt, void *stream);

/* The whole layer for T tokens: out [T][hidden] fp32 = routed combine + shared expert.
 * idx/wt (device, [T][topk]) receive the routing. Asynchronous on `stream`
 * (NULL = the context's stream). Returns 0, or -1 on a launch error. */
int  k3g_moe(K3gCtx *ctx, const K3gLayer *L, const float *x, int T,
             float *out, int32_t *idx, float *wt, void *stream);

/* The layer's steps one at a time (the expert-major prefill, src/core/k3_ops.c:717-807),
 * all device pointers, asynchronous on `stream` (NULL = the context's stream), sizes
 * within what the context was created for. Each returns 0, or -1 on a bad argument or a
 * launch error; device-side errors surface at k3g_sync. */

/* Token -> expert dispatch (the unique-expert collection of src/core/k3_ops.c:733-749,
 * made a counting sort): for P = T * topk (token, slot) pairs with expert ids idx [P],
 * off [n_experts + 1] receives each expert's first position and perm [P] the pair numbers
 * t * topk + j grouped by expert, ascending within each expert (a stable sort on idx).
 * Pairs with idx < 0 are left out (off[n_experts] counts the pairs placed); an id >=
 * n_experts is left out too and raises the device error that k3g_sync reports. */
int  k3g_dispatch(K3gCtx *ctx, const int32_t *idx, int T, int topk, int n_experts,
                  int32_t *perm, int32_t *off, void *stream);

/* Routed experts as per-expert GEMVs over each expert's pairs (the expert-major loop of
 * src/core/k3_ops.c:751-778, k3_matmul_mxfp4 at src/core/k3_ops.c:108): contrib
 * [T * topk][hidden] receives w2 . act(w1 . x_t, w3 . x_t) for each pair (t, j) with
 * e = idx[t * topk + j] valid; other rows are left alone. Experts in the checkpoint MXFP4
 * layout (K3G_EXPERT_MXFP4) or fp32; no latent projection. */
int  k3g_expert_gemv(K3gCtx *ctx, const K3gLayer *L, const float *x, int T,
                     const int32_t *idx, float *contrib, void *stream);

/* The same contrib rows as grouped GEMMs over 128-pair column tiles: gate/up with the
 * activation fused, then down, bf16 matrix cores (weights decoded from MXFP4 exactly,
 * x as two bf16 pieces, h as a bf16 piece plus its MXFP8 remainder on the scaled FP8
 * matrix cores, fp32 accumulation; rel-L2 about 4e-5) or, for _f8f6f4, the
 * scaled FP4 x FP8 ones with x and h quantised to MXFP8. Experts in the tiled layout
 * (K3G_EXPERT_MXFP4_TILED), hidden and inter multiples of 32. */
int  k3g_grouped_gemm_bf16(K3gCtx *ctx, const K3gLayer *L, const float *x, int T,
                           const int32_t *idx, float *contrib, void *stream);
int  k3g_grouped_gemm_f8f6f4(K3gCtx *ctx, const K3gLayer *L, const float *x, int T,
                             const int32_t *idx, float *contrib, void *stream);

/* Deterministic combine (src/core/k3_ops.c:780-792): out [T][n] = sum over j in top-k
 * order of wt[t][j] * contrib[t * topk + j] in fp32, starting from 0, then + add[t]
 * when add (the shared expert's output) is given. Slots with idx < 0 are skipped; n is a
 * multiple of 4. */
int  k3g_combine(K3gCtx *ctx, const float *contrib, const int32_t *idx, const float *wt,
                 int T, int topk, int n, const float *add, float *out, void *stream);

/* k3g_moe at decode sizes WITHOUT ANY ALLOCATION. No reference counterpart: it is for
 * callers that cannot allocate (code under HIP graph capture, serving loops that forbid
 * hipMalloc). It runs the fused decode kernel (1 <= T <= 4; Kimi-K2 layer shape: experts
 * in the tiled MXFP4 layout, shared expert in the tiled bf16 layout, no latent
 * projection) with every buffer beyond x, out, idx and wt in one fixed device array of
 * 16 MiB per GPU, set up on the first call on a device and held until the process ends.
 * A layer whose buffers exceed it (e.g. top-k 64 at hidden 7168) is rejected with -1 and
 * a message, as is any other shape or T. idx/wt (device, [T][topk]) may be NULL (the
 * routing then stays in the array); err (device int, may be NULL) receives a device
 * error the kernel raises (an exhausted bounded wait), as k3g_sync reports it for a
 * context. Asynchronous on `stream` (NULL = the null stream). Every call on a GPU shares
 * that GPU's array and it keeps the last call's contents: calls that overlap on one GPU
 * race and must be ordered by the caller. Returns 0, or -1. */
int  k3g_moe_noalloc(const K3gLayer *L, const float *x, int T, float *out, int32_t *idx,
                     float *wt, int *err, void *stream);

/* Synchronise the stream and report any error a kernel raised on the device
 * (an exhausted bounded wait, a bad expert index). Returns 0 when clean. */
int  k3g_sync(K3gCtx *ctx, void *stream);

/* ========================================================== 3. HBM expert cache == */

/* The engine's expert cache (src/cache/k3_cache.h, src/cache/k3_cache.c) re-planned for
 * one GPU: the slot arena is HBM, the backing store is a pinned host bank holding every
 * (layer, expert) run, and a miss is a hipMemcpyAsync on the cache's own copy stream.
 * Policy and accounting follow the engine: LRU with pinning over a linear victim scan,
 * slots that are EMPTY, INFLIGHT (reserved by a batch) or hold a key, batch prefetch in
 * three phases (reserve, copy, publish), a per-(layer, expert) request histogram and a
 * (layer, expert) request trace, and the true hit rate (hits - prefetch_reads) /
 * requests. get() hands back DEVICE pointers that stay valid until the step that got
 * them ends (k3gc_step_end). */
typedef struct K3gcBank K3gcBank;
typedef struct K3gCache K3gCache;

/* A host bank for n_layers x n_experts expert runs of `layout`, pinned per layer as far
 * as the driver allows: K3G_EXPERT_MXFP4
 * (the checkpoint run, src/io/k3_load.h:3-9) or K3G_EXPERT_MXFP4_TILED (w1, w3, w2 each
 * in the tiled MXFP4 layout, back to back). No reference counterpart: the engine reads
 * experts from the checkpoint files. */
int  k3gc_bank_create(K3gcBank **bank, int n_layers, int n_experts, int hidden, int inter,
                      int layout);
/* The same with at most max_pinned_layers layers pinned (< 0: as many as the driver
 * grants). Misses from pageable layers are copied through K3GC_NSTAGE pinned staging
 * buffers of the bank (taken before the layers): the host copies the run in with all
 * threads and the DMA engine copies it out at the pinned rate. Caches sharing a bank
 * must not copy at the same time. No reference counterpart. */
int  k3gc_bank_create_ex(K3gcBank **bank, int n_layers, int n_experts, int hidden,
                         int inter, int layout, int max_pinned_layers);
/* A bank of checkpoint-layout runs of expert_bytes each with no layer shape: it holds and
 * serves bytes (k3gc_bank_load, a cache's get) but a layer cannot run on it. For
 * checkpoints whose expert matrices do not form a layer (test fixtures). */
int  k3gc_bank_create_raw(K3gcBank **bank, int n_layers, int n_experts, int64_t expert_bytes,
                          int max_pinned_layers);
/* A bank with the geometry only (no memory), for caches that keep the bookkeeping only
 * (k3gc_init with device < 0): replays of a request trace at any capacity, as the
 * engine's offline simulator does. */
int  k3gc_bank_geometry(K3gcBank **bank, int n_layers, int n_experts, int64_t expert_bytes);
void k3gc_bank_free(K3gcBank *bank);
/* host pointer to the run of (layer, expert), expert_bytes long, for the caller to fill */
void *k3gc_bank_expert(K3gcBank *bank, int layer, int expert);
int64_t k3gc_bank_expert_bytes(const K3gcBank *bank);
/* layers whose runs sit in pinned memory (the rest are pageable when the driver caps
 * pinned memory below the bank's size) */
int  k3gc_bank_pinned_layers(const K3gcBank *bank);

/* Routed experts from safetensors checkpoint shards. An index of every tensor of every
 * *.safetensors file of a directory, shards numbered in name order (the engine's
 * k3_st_open / k3_st_find, src/io/k3_st.c:364-452). Returns 0, or -1 with a message (no
 * shards, a malformed header, a span that disagrees with its shape, duplicate names). */
typedef struct K3gcSt K3gcSt;
int  k3gc_st_open(K3gcSt **st, const char *dir);
void k3gc_st_close(K3gcSt *st);
int  k3gc_st_count(const K3gcSt *st);            /* tensors indexed */
/* Shards read with O_DIRECT (contiguous runs, through the enclosing 4096-byte window, as
 * the engine's k3_st_read_aligned, src/io/k3_st.c:457-497); the others, and every shard
 * when K3GC_NO_DIRECT is set at open, use ordinary reads. */
int  k3gc_st_direct(const K3gcSt *st);

/* One routed expert's six U8 tensors (w1, w2, w3: weight_packed, weight_scale), validated
 * as the engine's k3_expert_ref does (src/io/k3_load.c:15-100): 2-D, rows agreeing, one
 * scale byte per 32 elements, one shard. contiguous: the six spans tile one run in the
 * order w1.packed w1.scale w2.packed w2.scale w3.packed w3.scale (src/io/k3_load.h:3-9). */
typedef struct {
    int shard;
    int64_t off, nbytes;          /* the run: first byte in the shard, total bytes */
    int contiguous;
    int rows[3], pcols[3];        /* w1, w2, w3: packed [rows][pcols] */
    int64_t p_bytes[3], s_bytes[3], p_file[3], s_file[3];
} K3gcExpertRun;
int  k3gc_st_expert(const K3gcSt *st, int layer, int expert, K3gcExpertRun *run);
/* The run's bytes in the checkpoint order into dst (run->nbytes): one read when
 * contiguous, six otherwise (src/io/k3_load.c:105-136). Returns 0, or -1 on a short read. */
int  k3gc_st_read_run(const K3gcSt *st, const K3gcExpertRun *run, unsigned char *dst);
/* The same into buf (cap bytes): a contiguous run with O_DIRECT straight into buf when
 * buf is 4096-aligned and holds the run's enclosing 4096-byte window, the run then at
 * buf + *pad (src/io/k3_st.c:457-497); ordinary reads at buf otherwise (*pad = 0). */
int  k3gc_st_read_run_into(const K3gcSt *st, const K3gcExpertRun *run, unsigned char *buf,
                           int64_t cap, int64_t *pad);
/* An index over the engine's own K3St (as its k3_st_open filled it): names and spans
 * copied, the shard descriptors borrowed, so the engine's index must outlive this one. */
int  k3gc_st_from_engine(K3gcSt **st, const K3St *engine_index);
/* A bank that holds nothing in host memory: every miss is read from the checkpoint into
 * pinned staging (the misses of one getmany in parallel) and copied to its slot. The
 * layout follows expert 0 of checkpoint layer probe_layer: the tiled MXFP4 layout (tiled
 * on the GPU after the copy) when it is an expert of a hidden x inter layer with a tiled
 * layout, its own run layout otherwise; every later run must match it. Cache layer l
 * reads checkpoint layer l. st must outlive the bank. No reference counterpart as a
 * bank: the engine's k3_cache_init reads misses from the K3St itself. */
int  k3gc_bank_create_disk(K3gcBank **bank, const K3gcSt *st, int n_layers, int n_experts,
                           int probe_layer);
/* Bank layers [bank_layer0, + n_layers) from checkpoint layers [ck_layer0, + n_layers):
 * every expert's run read straight into the bank's host memory (checkpoint layout), or
 * read and tiled on the host (tiled layout). A bank with a layer shape takes only experts
 * of that shape. Returns 0, or -1 with a message. No reference counterpart: the engine
 * reads experts from the checkpoint on each miss (k3_expert_load_direct). */
int  k3gc_bank_load(K3gcBank *bank, const K3gcSt *st, int ck_layer0, int bank_layer0,
                    int n_layers);
/* The tiled MXFP4 layout of k3g_tile_mxfp4, written by the host (same bytes). */
int  k3gc_tile_mxfp4_host(unsigned char *dst, const unsigned char *packed,
                          const unsigned char *scales, int rows, int cols);

/* Replaces k3_cache_init (src/cache/k3_cache.h:97, src/cache/k3_cache.c:263-353):
 * budget_bytes of HBM rounded down to whole slots; fails (-1) below topk + 1 slots.
 * device < 0 keeps the bookkeeping only (no memory is moved; for policy replays). */
int  k3gc_init(K3gCache **cache, int device, K3gcBank *bank, int topk, int64_t budget_bytes);
/* Replaces k3_cache_free. */
void k3gc_free(K3gCache *cache);
/* The K3ExpertSrc to pass as K3MoeW.src (get/getmany/resident, device pointers). */
K3ExpertSrc *k3gc_src(K3gCache *cache);
/* Replaces k3_cache_pin: pin or unpin the slot holding (layer, expert); 0 if not
 * resident. */
int  k3gc_pin(K3gCache *cache, int layer, int expert, int pin);
/* Replaces k3_cache_prefetch: bring (layer, expert) resident without returning it. */
int  k3gc_prefetch(K3gCache *cache, int layer, int expert);
/* Replaces k3_cache_reset_stats, k3_cache_report, k3_cache_dump_hist,
 * k3_cache_dump_trace (same formats). */
void k3gc_reset_stats(K3gCache *cache);
void k3gc_report(K3gCache *cache, const char *label);
int  k3gc_dump_hist(const K3gCache *cache, const char *path);
int  k3gc_dump_trace(const K3gCache *cache, const char *path);

/* Histogram-driven pinning: make the npin most requested (layer, expert) of a histogram
 * [n_layers][n_experts] resident and pin them (ties to the lower layer, then expert). The
 * histogram is a previous workload's (the cache's own, k3gc_hist, or one read back from
 * k3gc_dump_hist); pinning stops short of leaving fewer than top-k + 1 unpinned slots.
 * Returns the number pinned. The use the engine's request histogram and k3_cache_pin are
 * for (src/cache/k3_cache.h:29-31, :100-102); the engine has no such call itself. */
int  k3gc_pin_hottest(K3gCache *cache, const uint32_t *hist, int npin);
/* The cache's request histogram, [n_layers][n_experts] counts of get() calls. */
const uint32_t *k3gc_hist(const K3gCache *cache);

/* Offline replays of a (layer, expert) request trace (int32 pairs, the format
 * k3gc_dump_trace writes) at `capacity` experts; each returns the hits, first touches
 * counted as misses. The engine's tools/sim_cache.py:36-110 with the same definitions:
 *   lru         least recently used;
 *   belady      the optimal offline policy: evict the expert used furthest in the
 *               future, and do not cache a request used later than every resident one;
 *   pinned_lru  the npin most requested experts of the trace (ties to the first seen)
 *               held once read, LRU in the remaining capacity - npin slots (at least 1);
 *               npin >= capacity is taken as capacity - 1.
 * Belady and pinned_lru see the whole trace, so they are ceilings for the policies a
 * cache can run. */
int64_t k3gc_replay_lru(const int32_t *trace_pairs, int64_t n, int64_t capacity);
int64_t k3gc_replay_belady(const int32_t *trace_pairs, int64_t n, int64_t capacity);
int64_t k3gc_replay_pinned_lru(const int32_t *trace_pairs, int64_t n, int64_t capacity,
                               int64_t npin);

typedef struct {
    int64_t requests, hits, misses, evictions, prefetch_reads, bytes_read;
    double load_seconds;          /* copy-stream time spent on misses */
    int nslot, resident, pinned;
    int64_t slot_bytes;
    int64_t staged;               /* misses copied through the bank's pinned staging */
} K3gcStats;
void k3gc_stats(K3gCache *cache, K3gcStats *out);

/* A step: experts handed out between begin and end are not evicted until the work
 * enqueued on `stream` before end() has finished with them. k3gc_wait makes `stream`
 * wait for every copy issued so far. No reference counterpart (the engine's reads are
 * synchronous). */
void k3gc_step_begin(K3gCache *cache);
void k3gc_step_end(K3gCache *cache, void *stream);
void k3gc_wait(K3gCache *cache, void *stream);

/* One streamed layer through the cache (experts in the bank's tiled layout): the
 * router (or, with route_idx/route_wt given, that routing: host arrays [T][topk]),
 * then the step's unique experts in first-seen order through getmany + get (the
 * engine's call pattern, src/core/k3_ops.c:604-627), the shared expert while the misses
 * copy, then the routed experts. L->experts is ignored; idx/wt are device outputs. */
int  k3gc_moe(K3gCtx *ctx, K3gCache *cache, const K3gLayer *L, int layer, const float *x,
              int T, float *out, int32_t *idx, float *wt, const int32_t *route_idx,
              const float *route_wt, void *stream);

/* A synthetic stack of MoE halves on a hidden state h [T][hidden] (device, fp32) that
 * stays in HBM, with no attention and no AttnRes aggregation between them: for each
 * layer l, hin = RMSNorm(h) x post_norm[l] (double sum, as the engine's k3_rmsnorm;
 * skipped when post_norm or post_norm[l] is NULL), the layer's MoE output on hin through
 * the cache (cache layer first_layer + l), then h += that output. The norm and MoE call
 * are k3_decoder_layer_inc's (src/core/k3_ops.c:1015-1024), the layer walk with the cache
 * as every layer's expert source is forward()'s (src/cli/k3_run.c:582-618); the engine
 * adds the MoE output to its block prefix pref (src/core/k3_ops.c:1035-1036), which its
 * attention and AttnRes steps keep apart from h, where this chain adds it to h itself.
 * Between layers the residual add and the next layer's norm are one launch. Only the
 * routing crosses to the host (for the cache's get calls). When every expert of every
 * layer in the chain is resident, the layers run back to back with no host
 * synchronisation, every layer's routing comes back in one copy, and the cache's get
 * calls follow, one step per layer, all hits. Layers in the tiled layout of the cache's
 * bank. */
int  k3gc_chain(K3gCtx *ctx, K3gCache *cache, const K3gLayer *layers,
                const float *const *post_norm, int first_layer, int n_layers, float *h,
                int T, float rms_eps, void *stream);

/* Seeded synthetic data, generated identically on host and device from a counter
 * hash, so a CPU check can regenerate any slice of what the GPU holds.
 * byte i of stream `stream` under `seed` is k3s_byte(seed, stream, i). */
uint8_t k3s_byte(uint64_t seed, uint64_t stream, uint64_t i);
void k3s_fill_bytes(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream, uint64_t first);
/* MXFP4 E8M0 scale bytes: 127 + uniform{lo..hi}. */
void k3s_fill_scales(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream, uint64_t first,
                     int lo, int hi);
/* N(mean, std) fp32 values (Box-Muller over the same counter hash). bf16_round != 0
 * rounds each value to bf16 (nearest-even) and returns it widened. */
void k3s_fill_normal(float *dst, size_t n, uint64_t seed, uint64_t stream, uint64_t first,
                     float mean, float std, int bf16_round);
/* Device fills, same values as the host fills. */
int  k3g_fill_bytes(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream, uint64_t first,
                    void *hstream);
int  k3g_fill_scales(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream, uint64_t first,
                     int lo, int hi, void *hstream);

#ifdef __cplusplus
}
#endif

#endif /* K3MOE_H */
