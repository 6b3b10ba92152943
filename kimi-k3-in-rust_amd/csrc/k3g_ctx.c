/* k3g_ctx.c - device context and the k3g_* layer API (C99 host code).
 *
 * The layer runs as a fixed sequence of kernels on one stream:
 *   router (fp64 logits, certified top-k)  ->  dispatch (stable counting sort)
 *   -> [latent down] -> routed gate/up + activation -> routed down
 *   -> shared gate/up + activation -> shared down -> combine (slot order, + shared)
 *   -> [aggregate RMSNorm, latent up, + shared]
 * All buffers come from one workspace allocated at context creation; a call allocates
 * nothing. */
#include "k3g_ctx.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

void k3g_fatal_hip(const char *what, hipError_t e, const char *file, int line)
{
    fprintf(stderr,
            "k3moe: FATAL, %s failed: %s (%s:%d).\n"
            "    Aborting rather than returning an output the GPU did not finish.\n",
            what, hipGetErrorString(e), file, line);
    abort();
}

void k3g_fatal(const char *what)
{
    fprintf(stderr, "k3moe: FATAL, %s\n", what);
    abort();
}

K3gExpertLayout k3g_expert_layout(int hidden, int inter)
{
    /* src/io/k3_load.h:3-9: w1.packed w1.scale w2.packed w2.scale w3.packed w3.scale */
    K3gExpertLayout l;
    const int64_t p13 = (int64_t)inter * (hidden / 2), s13 = (int64_t)inter * ((hidden + 31) / 32);
    const int64_t p2 = (int64_t)hidden * (inter / 2), s2 = (int64_t)hidden * ((inter + 31) / 32);
    l.p1_off = 0;
    l.s1_off = l.p1_off + p13;
    l.p2_off = l.s1_off + s13;
    l.s2_off = l.p2_off + p2;
    l.p3_off = l.s2_off + s2;
    l.s3_off = l.p3_off + p13;
    l.nbytes = l.s3_off + s13;
    return l;
}

size_t k3g_tiled_mxfp4_bytes(int rows, int cols) { return k3k_tiled_mxfp4_bytes(rows, cols); }
size_t k3g_tiled_bf16_bytes(int rows, int cols) { return k3k_tiled_bf16_bytes(rows, cols); }

int k3g_tile_mxfp4(void *dst, const void *packed, const void *scales, int rows, int cols,
                   void *stream)
{
    return k3k_tile_mxfp4((uint8_t *)dst, (const uint8_t *)packed, (const uint8_t *)scales,
                          rows, cols, (hipStream_t)stream);
}

int k3g_tile_bf16(void *dst, const void *src, int rows, int cols, void *stream)
{
    return k3k_tile_bf16((uint16_t *)dst, (const uint16_t *)src, rows, cols,
                         (hipStream_t)stream);
}

static size_t carve(size_t *at, size_t bytes)
{
    const size_t o = *at;
    *at += (bytes + 255) & ~(size_t)255;
    return o;
}

int k3g_ctx_create(K3gCtx **out, int device, const K3gLayer *s, int max_tokens)
{
    *out = NULL;
    if (!s || max_tokens < 1 || s->topk < 1 || s->topk > K3G_MAX_TOPK || s->n_experts < 1 ||
        s->n_experts > 1024 || s->hidden < 1) {
        fprintf(stderr, "k3moe: k3g_ctx_create: unsupported shape\n");
        return -1;
    }
    K3gCtx *c = (K3gCtx *)calloc(1, sizeof *c);
    if (!c) return -1;
    c->device = device;
    c->hidden = s->hidden;
    c->n_experts = s->n_experts;
    c->topk = s->topk;
    c->inter = s->inter;
    c->shared_inter = s->shared_inter;
    c->latent = s->latent > 0 ? s->latent : s->hidden;
    c->max_tokens = max_tokens;

    if (hipSetDevice(device) != hipSuccess) { free(c); return -1; }
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        free(c);
        return -1;
    }
    if (hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_in, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c->ev_shared, hipEventDisableTiming) != hipSuccess) {
        fprintf(stderr, "k3moe: k3g_ctx_create: cannot create the side stream\n");
        return -1;
    }
    const size_t T = (size_t)max_tokens, E = (size_t)c->n_experts, k = (size_t)c->topk;
    const size_t P = T * k, nch = (P + 255) / 256;
    const size_t L = (size_t)c->latent, I = (size_t)c->inter, SI = (size_t)c->shared_inter;
    const size_t d = (size_t)c->hidden;
    size_t at = 0;
    const size_t o_rs = carve(&at, T * E * 16);
    const size_t o_idx = carve(&at, P * 4), o_wt = carve(&at, P * 4);
    const size_t o_cnt = carve(&at, nch * E * 4), o_base = carve(&at, (nch + 1) * E * 4);
    const size_t o_off = carve(&at, (E + 1) * 4), o_act = carve(&at, E * 4);
    const size_t o_nact = carve(&at, 4), o_perm = carve(&at, P * 4);
    const size_t o_z = carve(&at, T * L * 4), o_h = carve(&at, P * I * 4);
    const size_t o_contrib = carve(&at, P * L * 4), o_accl = carve(&at, T * L * 4);
    const size_t o_shh = carve(&at, T * (SI ? SI : 1) * 4), o_sho = carve(&at, T * d * 4);
    const size_t o_err = carve(&at, 4), o_stats = carve(&at, 16 * 4);
    /* the fused decode kernel's buffers, for up to 4 tokens */
    const int T4 = max_tokens < 4 ? max_tokens : 4;
    const size_t P4 = (size_t)T4 * k;
    const size_t nQd = (d + 511) / 512, nQi = (I + 511) / 512;
    const size_t o_xq8 = carve(&at, (size_t)T4 * nQd * 8448), o_hq8 = carve(&at, P4 * nQi * 8448);
    const size_t o_xq16 = carve(&at, (d / 32) * 1024), o_hq16 = carve(&at, (SI / 32 + 1) * 1024);
    const size_t o_gpart = carve(&at, P4 * K3G_KS_G_MAX * 2 * I * 4);
    const size_t o_sgpart = carve(&at, (size_t)K3G_KS_SG_MAX * T4 * 2 * (SI ? SI : 1) * 4);
    const size_t o_shpart = carve(&at, (size_t)K3G_KS_SD_MAX * T4 * d * 4);
    const size_t o_rpart = carve(&at, (size_t)T4 * E * K3G_KS_R_MAX * 16);
    const size_t dl = d > L ? d : L;       /* the routed down's output rows */
    const size_t o_dcontrib = carve(&at, P4 * K3G_KS_D_MAX * dl * 4);
    /* the latent layer's: z's slices and FP8 pieces, the aggregate, its tiles' sums of
     * squares, its bf16 pieces, the latent up's slices */
    const int lat = L != d;
    const size_t nQL = (L + 511) / 512;
    const size_t o_dzpart = carve(&at, lat ? (size_t)K3G_KS_LD * T4 * L * 4 : 16);
    const size_t o_dzq8 = carve(&at, lat ? (size_t)T4 * nQL * 8448 : 16);
    const size_t o_daccl = carve(&at, lat ? (size_t)T4 * L * 4 : 16);
    const size_t o_dnss = carve(&at, lat ? (size_t)T4 * (L / 32) * 8 : 16);
    const size_t o_daq16 = carve(&at, lat ? (L / 32 + 1) * 1024 : 16);
    const size_t o_dupart = carve(&at, lat ? (size_t)K3G_KS_LU * T4 * d * 4 : 16);
    /* the grouped GEMMs' activation pieces and column tiles */
    const size_t d128 = (d + 127) / 128 * 128, I128 = (I + 127) / 128 * 128;
    const size_t SI128 = (SI + 127) / 128 * 128;
    const size_t maxt = (P + 127) / 128 + E;
    const size_t o_xb = carve(&at, 2 * T * d128 * 2), o_hb = carve(&at, 2 * P * I128 * 2);
    const size_t o_hsb = carve(&at, 2 * T * (SI128 ? SI128 : 128) * 2);
    /* the dense GEMMs' K-slice sums when few columns leave the GPU idle: the shared
     * expert's gate/up and down, the latent down and up projections */
    size_t part = 0;
    if (SI) {
        const size_t pg = k3k_gemm_part_bytes((int)((SI + 255) / 256), (int)(2 * SI));
        const size_t pd = k3k_gemm_part_bytes((int)((d + 511) / 512), (int)d);
        part = pg > pd ? pg : pd;
    }
    if (L != d) {
        const size_t pz = k3k_gemm_part_bytes((int)((L + 511) / 512), (int)L);
        const size_t pu = k3k_gemm_part_bytes((int)((d + 511) / 512), (int)d);
        if (pz > part) part = pz;
        if (pu > part) part = pu;
    }
    const size_t o_kpart = carve(&at, part ? part : 16);
    size_t part2 = 0;      /* the shared expert's, when it runs on the side stream */
    if (SI) {
        const size_t pg = k3k_gemm_part_bytes((int)((SI + 255) / 256), (int)(2 * SI));
        const size_t pd = k3k_gemm_part_bytes((int)((d + 511) / 512), (int)d);
        part2 = pg > pd ? pg : pd;
    }
    const size_t o_kpart2 = carve(&at, part2 ? part2 : 16);
    const size_t L128 = (L + 127) / 128 * 128;
    const size_t o_zb = carve(&at, L != d ? 2 * T * L128 * 2 : 16);
    const size_t o_zflag = carve(&at, 4);
    const size_t o_rtpart = carve(&at, k3k_router_part_bytes());
    const size_t o_rtctr = carve(&at, 512 * 128);
    const size_t rbf = k3k_router_bf3_floats((int)T, (int)E);
    const size_t o_rbpart = carve(&at, rbf ? rbf * 4 : 16);
    const size_t o_tiles = carve(&at, maxt * 16), o_ntiles = carve(&at, 4);
    const size_t o_xflag = carve(&at, 4);
    const size_t d512 = (d + 511) / 512 * 512, I512 = (I + 511) / 512 * 512;
    const size_t L512 = (L + 511) / 512 * 512, q512 = d512 > L512 ? d512 : L512;
    const size_t o_xq8b = carve(&at, T * q512 + T * q512 / 32);
    const size_t o_hq8b = carve(&at, P * I512 + P * I512 / 32);
    /* two banks of counters, one per call in turn; each a multiple of 256 bytes */
    /* the larger of the latent layer's geometry and the plain one (a layer without the
     * latent projections may run on a context sized for them) */
    const size_t sb_l = k3k_decode_sync_bytes(T4, (int)d, (int)E, (int)k, (int)I, (int)SI, (int)L);
    const size_t sb_d = k3k_decode_sync_bytes(T4, (int)d, (int)E, (int)k, (int)I, (int)SI, (int)d);
    c->sync_bytes = ((sb_l > sb_d ? sb_l : sb_d) + 255) & ~(size_t)255;
    const size_t o_sync = carve(&at, 2 * c->sync_bytes);
    c->ws_bytes = at;
    if (hipMalloc(&c->ws, at) != hipSuccess) {
        fprintf(stderr, "k3moe: cannot allocate %.2f GB of device workspace\n", at / 1e9);
        hipStreamDestroy(c->stream);
        free(c);
        return -1;
    }
    char *b = (char *)c->ws;
    c->rs = (float *)(b + o_rs);
    c->idx = (int32_t *)(b + o_idx);
    c->wt = (float *)(b + o_wt);
    c->cnt = (int32_t *)(b + o_cnt);
    c->base = (int32_t *)(b + o_base);
    c->off = (int32_t *)(b + o_off);
    c->act = (int32_t *)(b + o_act);
    c->nact = (int32_t *)(b + o_nact);
    c->perm = (int32_t *)(b + o_perm);
    c->z = (float *)(b + o_z);
    c->h = (float *)(b + o_h);
    c->contrib = (float *)(b + o_contrib);
    c->accl = (float *)(b + o_accl);
    c->sh_h = (float *)(b + o_shh);
    c->sh_out = (float *)(b + o_sho);
    c->err = (int *)(b + o_err);
    c->stats = (int *)(b + o_stats);
    c->xq8 = (uint8_t *)(b + o_xq8);
    c->hq8 = (uint8_t *)(b + o_hq8);
    c->xq16 = (uint16_t *)(b + o_xq16);
    c->hq16 = (uint16_t *)(b + o_hq16);
    c->gpart = (float *)(b + o_gpart);
    c->sgpart = (float *)(b + o_sgpart);
    c->shpart = (float *)(b + o_shpart);
    c->rpart = (double *)(b + o_rpart);
    c->dcontrib = (float *)(b + o_dcontrib);
    c->dzpart = (float *)(b + o_dzpart);
    c->dzq8 = (uint8_t *)(b + o_dzq8);
    c->daccl = (float *)(b + o_daccl);
    c->dnss = (double *)(b + o_dnss);
    c->daq16 = (uint16_t *)(b + o_daq16);
    c->dupart = (float *)(b + o_dupart);
    c->sync = (int *)(b + o_sync);
    c->xb = (uint16_t *)(b + o_xb);
    c->hb = (uint16_t *)(b + o_hb);
    c->hsb = (uint16_t *)(b + o_hsb);
    c->zb = (uint16_t *)(b + o_zb);
    c->zflag = (int32_t *)(b + o_zflag);
    c->kpart = (float *)(b + o_kpart);
    c->kpart2 = (float *)(b + o_kpart2);
    c->rtpart = (double *)(b + o_rtpart);
    c->rtctr = (int32_t *)(b + o_rtctr);
    c->rbpart = rbf ? (float *)(b + o_rbpart) : NULL;
    c->rbpart_floats = rbf;
    c->tiles = (int32_t *)(b + o_tiles);
    c->ntiles = (int32_t *)(b + o_ntiles);
    c->xflag = (int32_t *)(b + o_xflag);
    c->max_tiles = (int)maxt;
    c->xq8b = (uint8_t *)(b + o_xq8b);
    c->hq8b = (uint8_t *)(b + o_hq8b);
    c->fused = 1;
    if (hipMemset(c->ws, 0, at) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        hipFree(c->ws);
        hipStreamDestroy(c->stream);
        free(c);
        return -1;
    }
    *out = c;
    return 0;
}

/* Stage timing: each stage owns a ring of K3G_RING event pairs. A pair is harvested
 * (its elapsed time added to the stage total) only when the ring comes back to it or
 * the totals are read, so a timed loop of up to K3G_RING calls never blocks on its own
 * events. */
static void harvest_one(K3gCtx *c, int s, int i)
{
    float ms = 0.0f;
    K3G_CHECK(hipEventSynchronize(c->ev[s][i][1]));
    K3G_CHECK(hipEventElapsedTime(&ms, c->ev[s][i][0], c->ev[s][i][1]));
    c->stage_ms[s] += ms;
    c->stage_n[s]++;
}

static void harvest(K3gCtx *c, int s)
{
    const int n = c->ev_used[s];
    for (int k = 0; k < n; k++)
        harvest_one(c, s, (c->ev_head[s] - n + k + K3G_RING) % K3G_RING);
    c->ev_used[s] = 0;
}

void k3g_stage_begin(K3gCtx *c, int s, hipStream_t st)
{
    if (!c->prof) return;
    const int i = c->ev_head[s];
    if (!c->ev[s][i][0]) {
        K3G_CHECK(hipEventCreate(&c->ev[s][i][0]));
        K3G_CHECK(hipEventCreate(&c->ev[s][i][1]));
    }
    if (c->ev_used[s] == K3G_RING) {        /* the oldest pair is this one */
        harvest_one(c, s, i);
        c->ev_used[s]--;
    }
    K3G_CHECK(hipEventRecord(c->ev[s][i][0], st));
}

void k3g_stage_end(K3gCtx *c, int s, hipStream_t st)
{
    if (!c->prof) return;
    const int i = c->ev_head[s];
    K3G_CHECK(hipEventRecord(c->ev[s][i][1], st));
    c->ev_head[s] = (i + 1) % K3G_RING;
    c->ev_used[s]++;
}

void k3g_ctx_profile(K3gCtx *c, int on)
{
    if (!c) return;
    for (int s = 0; s < K3G_NSTAGE; s++) harvest(c, s);
    c->prof = on;
    for (int s = 0; s < K3G_NSTAGE; s++) { c->stage_ms[s] = 0.0; c->stage_n[s] = 0; }
}

int k3g_ctx_stage_ms(K3gCtx *c, double *ms, int64_t *count, int n)
{
    if (!c) return 0;
    for (int s = 0; s < K3G_NSTAGE; s++) harvest(c, s);
    for (int s = 0; s < n && s < K3G_NSTAGE; s++) {
        if (ms) ms[s] = c->stage_ms[s];
        if (count) count[s] = c->stage_n[s];
    }
    return K3G_NSTAGE;
}

void k3g_ctx_destroy(K3gCtx *c)
{
    if (!c) return;
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
    for (int s = 0; s < K3G_NSTAGE; s++)
        for (int i = 0; i < K3G_RING; i++)
            if (c->ev[s][i][0]) {
                hipEventDestroy(c->ev[s][i][0]);
                hipEventDestroy(c->ev[s][i][1]);
            }
    hipFree(c->ws);
    hipStreamSynchronize(c->side);
    hipEventDestroy(c->ev_in);
    hipEventDestroy(c->ev_shared);
    hipStreamDestroy(c->side);
    hipStreamDestroy(c->stream);
    free(c);
}

void *k3g_ctx_stream(K3gCtx *c) { return c ? (void *)c->stream : NULL; }

void k3g_ctx_force_exact(K3gCtx *c, int mode) { if (c) c->force_exact = mode; }

void k3g_ctx_set_fused(K3gCtx *c, int on) { if (c) c->fused = on; }

int k3g_ctx_paths(K3gCtx *c, int clear)
{
    if (!c) return 0;
    const int p = c->paths;
    if (clear) c->paths = 0;
    return p;
}

void k3g_ctx_set_trace(K3gCtx *c, void *dev_buf) { if (c) c->trace = (unsigned long long *)dev_buf; }

/* The fused kernel covers decode token counts with the routed experts and the shared
 * expert in the tiled layouts: the Kimi-K2 layer shape (no latent), and the LatentMoE
 * layer (Kimi-K3: both latent projections in the tiled bf16 layout, the aggregate's
 * RMSNorm when given). */
static int fusable(const K3gCtx *c, const K3gLayer *L, int T)
{
    const int lat = L->latent > 0 ? L->latent : L->hidden;
    const int plain = !L->down && !L->up && !L->latent_norm && lat == L->hidden;
    const int latent = L->down && L->up && lat != L->hidden && lat % 32 == 0 &&
                       lat <= c->latent && L->wdt == K3_WBF16 && L->shared_fmt == 1;
    return c->fused && T <= 4 && L->expert_fmt == K3G_EXPERT_MXFP4_TILED && (plain || latent) &&
           L->hidden % 32 == 0 && L->inter % 32 == 0 &&
           (L->shared_inter == 0 || (L->wdt == K3_WBF16 && L->shared_fmt == 1 &&
                                     L->shared_inter % 32 == 0));
}

/* The grouped GEMMs cover any token count on tiled experts, with the shared expert and
 * the latent projections (when present) in the tiled bf16 layout. */
static int gemmable(const K3gCtx *c, const K3gLayer *L)
{
    const int lat = L->latent > 0 ? L->latent : L->hidden;
    if (!c->fused || L->expert_fmt != K3G_EXPERT_MXFP4_TILED || L->hidden % 32 ||
        L->inter % 32 || lat % 32)
        return 0;
    const int bf16_tiled = L->wdt == K3_WBF16 && L->shared_fmt == 1;
    if (L->shared_inter && (!bf16_tiled || L->shared_inter % 32)) return 0;
    if ((L->down || L->up) && !bf16_tiled) return 0;
    return 1;
}

static int run_fused(K3gCtx *c, const K3gLayer *L, const float *x, int T, float *out,
                     int32_t *idx, float *wt, int given, hipStream_t st);

static int r128(int v) { return (v + 127) / 128 * 128; }
static int r512(int v) { return (v + 511) / 512 * 512; }

void k3g_ctx_set_fp8(K3gCtx *c, int on) { if (c) c->gemm_fp8 = on; }

/* K slices of a dense GEMM (whole 128-column steps only) */
static int dense_ksplit(int nft, int T, int K)
{
    return K % 128 ? 1 : k3k_gemm_ksplit(nft, (T + 127) / 128, K);
}

/* out [T][rows] = W B for a dense tiled-bf16 matrix W [rows][K] and two-piece B [2][T][ldb]
 * (piece 1 skipped when *lo_flag == 0), fp32 rows at stride ldo. */
static int dense_gemm(K3gCtx *c, const void *W, int rows, int K, const uint16_t *b, int ldb,
                      const int32_t *lo_flag, int T, float *out, int ldo, hipStream_t st)
{
    K3kGemm s;
    memset(&s, 0, sizeof s);
    s.mode = 1;
    s.afmt = 1;
    s.rows = rows;
    s.K = K;
    s.ldb = ldb;
    s.wa = (const uint16_t *)W;
    s.b = b;
    s.bpiece = (long long)T * ldb;
    s.dense_rows = T;
    s.npieces = 2;
    s.lo_flag = lo_flag;
    s.out = out;
    s.ldo = ldo;
    s.nft = (rows + 511) / 512;
    s.ksplit = dense_ksplit(s.nft, T, K);
    s.part = c->kpart;
    return k3k_gemm(&s, st);
}

/* Routed and shared experts as grouped GEMMs on the bf16 matrix cores (k3g_gemm.hip), or
 * the routed experts on the FP4 x FP8 ones (fp8): dispatch -> column tiles -> x pieces ->
 * [shared gate/up, down] -> routed gate/up (+act) -> down -> [combine]. full = 0 stops at
 * the routed experts' per-pair rows in contrib. */
static int gemm_body(K3gCtx *c, const K3gLayer *L, const float *x, int T,
                     const int32_t *idx, const float *wt, float *out, float *contrib, int fp8,
                     int full, int shared_side, hipStream_t st);

static int experts_gemm(K3gCtx *c, const K3gLayer *L, const float *x, int T,
                        const int32_t *idx, const float *wt, float *out, float *contrib,
                        int fp8, int full, hipStream_t st)
{
    int rc = 0;
    k3g_stage_begin(c, K3G_ST_DISPATCH, st);
    rc |= k3k_dispatch_tiles(idx, T * L->topk, L->n_experts, c->cnt, c->base, c->off, c->act,
                             c->nact, c->perm, c->err, c->tiles, c->ntiles, c->xflag, st);
    k3g_stage_end(c, K3G_ST_DISPATCH, st);
    return rc | gemm_body(c, L, x, T, idx, wt, out, contrib, fp8, full, 0, st);
}

/* The shared expert's dense gate/up (+ activation -> h pieces) and down GEMMs on x's
 * pieces, into c->sh_out; part: the K-slice sums' buffer. */
static int shared_expert(K3gCtx *c, const K3gLayer *L, int T, float *part, hipStream_t st)
{
    const int d = L->hidden, SI = L->shared_inter;
    const int d128 = r128(d), SI128 = r128(c->shared_inter);
    int rc = 0;
    K3kGemm s;
    memset(&s, 0, sizeof s);
    s.mode = 0;
    s.afmt = 1;
    s.rows = SI;
    s.K = d;
    s.ldb = d128;
    s.b = c->xb;
    s.bpiece = (long long)T * d128;
    s.npieces = 2;
    s.lo_flag = c->xflag;
    s.wa = (const uint16_t *)L->sh1;
    s.wb = (const uint16_t *)L->sh3;
    s.dense_rows = T;
    s.h = c->hsb;
    s.hpiece = (long long)T * SI128;
    s.ldh = SI128;
    s.b1 = L->act_b1;
    s.b2 = L->act_b2;
    s.nft = (SI + 255) / 256;
    s.ksplit = dense_ksplit(s.nft, T, d);
    s.part = part;
    k3g_stage_begin(c, K3G_ST_SH_GATEUP, st);
    rc |= k3k_gemm(&s, st);
    k3g_stage_end(c, K3G_ST_SH_GATEUP, st);
    s.mode = 1;
    s.rows = d;
    s.K = SI;
    s.ldb = SI128;
    s.wa = (const uint16_t *)L->sh2;
    s.wb = NULL;
    s.b = c->hsb;
    s.bpiece = (long long)T * SI128;
    s.lo_flag = NULL;
    s.h = NULL;
    s.out = c->sh_out;
    s.ldo = d;
    s.nft = (d + 511) / 512;
    s.ksplit = dense_ksplit(s.nft, T, SI);
    k3g_stage_begin(c, K3G_ST_SH_DOWN, st);
    rc |= k3k_gemm(&s, st);
    k3g_stage_end(c, K3G_ST_SH_DOWN, st);
    return rc;
}

/* x's two bf16 pieces (the piece-1 flag cleared before) and, for the FP4 x FP8 routed
 * experts on x itself, its MXFP8 copy. */
static int gemm_pieces(K3gCtx *c, const K3gLayer *L, const float *x, int T, int fp8,
                       hipStream_t st)
{
    const int d = L->hidden, d128 = r128(d), d512 = r512(d);
    int rc = 0;
    k3g_stage_begin(c, K3G_ST_PIECES, st);
    rc |= k3k_xpieces(x, T, d, d128, c->xb, (long long)T * d128, c->xflag, st);
    if (fp8 && !L->down)
        rc |= k3k_xq8(x, T, d, d512, c->xq8b, c->xq8b + (size_t)T * d512, st);
    k3g_stage_end(c, K3G_ST_PIECES, st);
    return rc;
}

/* The grouped GEMMs after the dispatch (column tiles built, x's piece-1 flag cleared):
 * x pieces, [latent down], the shared expert, the routed gate/up and down, [combine,
 * latent up, + shared]. shared_side: x's pieces are already made and the shared expert
 * runs on the side stream (ev_shared marks its end; the combine waits for it). */
static int gemm_body(K3gCtx *c, const K3gLayer *L, const float *x, int T,
                     const int32_t *idx, const float *wt, float *out, float *contrib, int fp8,
                     int full, int shared_side, hipStream_t st)
{
    const int d = L->hidden, E = L->n_experts, k = L->topk, I = L->inter;
    const int SI = full ? L->shared_inter : 0, P = T * k;
    const int d128 = r128(d), I128 = r128(c->inter);
    const int lat = L->latent > 0 ? L->latent : d, lat128 = r128(lat);
    const int projected = L->down != NULL;
    int rc = 0;
    const int I512 = r512(c->inter);
    if (!shared_side) rc |= gemm_pieces(c, L, x, T, fp8, st);
    /* the routed experts' input: x, or its latent projection z = down x as two bf16
     * pieces (piece 1 always taken) */
    const uint16_t *rb = c->xb;
    int ldr = d128;
    const int32_t *rflag = c->xflag;
    if (projected) {
        k3g_stage_begin(c, K3G_ST_LATENT, st);
        rc |= dense_gemm(c, L->down, lat, d, c->xb, d128, c->xflag, T, c->z, lat, st);
        rc |= k3k_xpieces(c->z, T, lat, lat128, c->zb, (long long)T * lat128, c->zflag, st);
        if (fp8) {
            const int l512 = r512(lat);
            rc |= k3k_xq8(c->z, T, lat, l512, c->xq8b, c->xq8b + (size_t)T * l512, st);
        }
        k3g_stage_end(c, K3G_ST_LATENT, st);
        rb = c->zb;
        ldr = lat128;
        rflag = NULL;
    }

    K3kGemm g;
    memset(&g, 0, sizeof g);
    g.mode = 0;
    g.afmt = 0;
    g.rows = I;
    g.K = lat;
    g.ldb = ldr;
    g.eq = L->experts;
    g.b = rb;
    g.bpiece = (long long)T * ldr;
    g.perm = c->perm;
    g.topk = k;
    g.tiles = c->tiles;
    g.ntiles = c->ntiles;
    g.max_tiles = (P + 127) / 128 + (E < P ? E : P);
    g.npieces = 2;
    g.lo_flag = rflag;
    g.h = c->hb;
    g.hpiece = (long long)P * I128;
    g.ldh = I128;
    g.b1 = L->act_b1;
    g.b2 = L->act_b2;
    g.nft = (I + 255) / 256;

    if (SI > 0 && !shared_side) rc |= shared_expert(c, L, T, c->kpart, st);
    /* routed experts last, after any copies they wait for (the shared expert above
     * overlaps them) */
    if (c->routed_wait) {
        if (hipStreamWaitEvent(st, c->routed_wait, 0) != hipSuccess) rc = -1;
        c->routed_wait = NULL;
    }
    if (fp8) {
        const int l512 = r512(lat);
        g.bq = c->xq8b;
        g.bs = c->xq8b + (size_t)T * l512;
        g.ldb = l512;
        g.hq = c->hq8b;
        g.hs = c->hq8b + (size_t)P * I512;
        g.ldhq = I512;
    } else {
        /* h leaves gate/up as bf16 plus its MXFP8 remainder */
        g.hmix = 1;
        g.hq = c->hq8b;
        g.hs = c->hq8b + (size_t)P * I512;
        g.ldhq = I512;
    }
    k3g_stage_begin(c, K3G_ST_GATEUP, st);
    g.trace = fp8 ? NULL : c->trace;
    rc |= fp8 ? k3k_gemm_f8(&g, st) : k3k_gemm(&g, st);
    k3g_stage_end(c, K3G_ST_GATEUP, st);
    /* the down launch's stamps follow the widest gate/up launch's (4-wave workgroups) */
    if (g.trace) g.trace += 4 * 8 * (size_t)K3G_TILE_ROUNDS(g.max_tiles) * (size_t)((I + 127) / 128);

    g.mode = 1;
    g.rows = lat;
    g.K = I;
    g.ldb = I128;
    g.b = c->hb;
    g.bpiece = (long long)P * I128;
    g.lo_flag = NULL;
    g.h = NULL;
    g.out = contrib;
    g.ldo = lat;
    g.scatter = 1;
    g.nft = (lat + 511) / 512;
    if (fp8) {
        g.bq = c->hq8b;
        g.bs = c->hq8b + (size_t)P * I512;
        g.ldb = I512;
        g.hq = NULL;
        g.hs = NULL;
    } else {
        g.npieces = 1;
        g.bq = c->hq8b;
        g.bs = c->hq8b + (size_t)P * I512;
    }
    k3g_stage_begin(c, K3G_ST_DOWN, st);
    rc |= fp8 ? k3k_gemm_f8(&g, st) : k3k_gemm(&g, st);
    k3g_stage_end(c, K3G_ST_DOWN, st);

    if (SI > 0 && shared_side && hipStreamWaitEvent(st, c->ev_shared, 0) != hipSuccess) rc = -1;
    if (full && !projected && !L->up && !L->latent_norm) {
        k3g_stage_begin(c, K3G_ST_COMBINE, st);
        rc |= k3k_combine(contrib, idx, wt, T, k, d, SI > 0 ? c->sh_out : NULL, out, st);
        k3g_stage_end(c, K3G_ST_COMBINE, st);
    } else if (full) {
        /* the routed aggregate at latent width, its RMSNorm, up = the up projection as a
         * dense GEMM on its two bf16 pieces, then + the shared expert */
        k3g_stage_begin(c, K3G_ST_COMBINE, st);
        rc |= k3k_combine(contrib, idx, wt, T, k, lat, NULL, c->accl, st);
        if (L->latent_norm)
            rc |= k3k_rmsnorm(c->accl, c->accl, L->latent_norm, lat, T, L->rms_eps, st);
        k3g_stage_end(c, K3G_ST_COMBINE, st);
        if (L->up) {
            k3g_stage_begin(c, K3G_ST_LATENT, st);
            rc |= k3k_xpieces(c->accl, T, lat, lat128, c->zb, (long long)T * lat128, c->zflag,
                              st);
            rc |= dense_gemm(c, L->up, d, lat, c->zb, lat128, NULL, T, out, d, st);
            k3g_stage_end(c, K3G_ST_LATENT, st);
        } else if (hipMemcpyAsync(out, c->accl, (size_t)T * d * 4, hipMemcpyDeviceToDevice, st) !=
                   hipSuccess) {
            rc = -1;
        }
        if (SI > 0) rc |= k3k_add(out, c->sh_out, (size_t)T * d, st);
    }
    return rc ? -1 : 0;
}

void k3g_ctx_routed_wait(K3gCtx *c, hipEvent_t ev) { if (c) c->routed_wait = ev; }

void k3g_ctx_stats(K3gCtx *c, int64_t *out, int n)
{
    int s[16] = {0};
    if (!c || n <= 0) return;
    hipSetDevice(c->device);
    K3G_CHECK(hipStreamSynchronize(c->stream));
    K3G_CHECK(hipMemcpy(s, c->stats, sizeof s, hipMemcpyDeviceToHost));
    for (int i = 0; i < n && i < 16; i++) out[i] = s[i];
}

static int fits(const K3gCtx *c, const K3gLayer *L, int T)
{
    const int lat = L->latent > 0 ? L->latent : L->hidden;
    if (T < 1 || T > c->max_tokens || L->hidden != c->hidden || L->n_experts > c->n_experts ||
        L->topk > c->topk || L->inter > c->inter || L->shared_inter > c->shared_inter ||
        lat > c->latent) {
        fprintf(stderr, "k3moe: layer or token count exceeds the context's workspace\n");
        return 0;
    }
    if (lat != L->hidden && (!L->down || !L->up)) {
        fprintf(stderr, "k3moe: latent %d != hidden %d needs both down and up\n", lat,
                L->hidden);
        return 0;
    }
    return 1;
}

/* fits() for the calls that read the routed experts: a layer whose experts are missing
 * (no table for the MXFP4 formats, no w1/w3/w2 for the fp32 bank; a caller that freed
 * its experts and serves them from an HBM cache passes the cache's table instead) is
 * refused here rather than read on the device */
static int fits_experts(const K3gCtx *c, const K3gLayer *L, int T)
{
    const int have = L->expert_fmt == K3G_EXPERT_F32 ? (L->w1 && L->w3 && L->w2)
                                                     : L->experts != NULL;
    if (!have) {
        fprintf(stderr, "k3moe: the layer has no routed experts (table or fp32 bank)\n");
        return 0;
    }
    return fits(c, L, T);
}

int k3g_route(K3gCtx *c, const K3gLayer *L, const float *x, int T, int32_t *idx, float *wt,
              hipStream_t st)
{
    if (!fits(c, L, T)) return -1;
    k3g_stage_begin(c, K3G_ST_ROUTER, st);
    const int rc = k3k_router(x, T, L->gate, L->bias, L->hidden, L->n_experts, L->topk,
                              L->renorm, L->routed_scale, c->rs, idx, wt, c->force_exact,
                              c->stats, c->rtpart, c->rtctr, c->rbpart, c->rbpart_floats,
                              c->route_x1flag, st);
    k3g_stage_end(c, K3G_ST_ROUTER, st);
    return rc;
}

int k3g_router(K3gCtx *c, const K3gLayer *L, const float *x, int T, int32_t *idx, float *wt,
               void *stream)
{
    hipStream_t st = stream ? (hipStream_t)stream : c->stream;
    return k3g_route(c, L, x, T, idx, wt, st);
}

static int wfmt(int wdt)
{
    return wdt == K3_WBF16 ? K3K_BF16 : wdt == K3_WI8 ? K3K_I8R : K3K_F32;
}

/* The routed experts of checkpoint-layout (or fp32) weights as per-expert GEMVs over each
 * expert's pairs (k3g_gemv.hip): dispatch -> gate/up (+act) -> down -> contrib rows. */
static int routed_staged(K3gCtx *c, const K3gLayer *L, const float *z, int lat, int T,
                         const int32_t *idx, float *contrib, hipStream_t st)
{
    const int E = L->n_experts, k = L->topk, P = T * k;
    int rc = 0;
    k3g_stage_begin(c, K3G_ST_DISPATCH, st);
    rc |= k3k_dispatch(idx, P, E, c->cnt, c->base, c->off, c->act, c->nact, c->perm, c->err,
                       st);
    k3g_stage_end(c, K3G_ST_DISPATCH, st);
    K3kRouted a;
    memset(&a, 0, sizeof a);
    a.fmt = L->expert_fmt == 1 ? K3K_F32 : K3K_MXFP4;
    a.eq = L->experts;
    a.w1 = L->w1;
    a.w3 = L->w3;
    a.w2 = L->w2;
    a.act = c->act;
    a.nact = c->nact;
    a.off = c->off;
    a.perm = c->perm;
    a.topk = k;
    a.inter = L->inter;
    a.latent = lat;
    a.z = z;
    a.h = c->h;
    a.contrib = contrib;
    a.b1 = L->act_b1;
    a.b2 = L->act_b2;
    a.err = c->err;
    const int maxU = P < E ? P : E;
    k3g_stage_begin(c, K3G_ST_GATEUP, st);
    rc |= k3k_routed_gateup(&a, maxU, T, st);
    k3g_stage_end(c, K3G_ST_GATEUP, st);
    k3g_stage_begin(c, K3G_ST_DOWN, st);
    rc |= k3k_routed_down(&a, maxU, T, st);
    k3g_stage_end(c, K3G_ST_DOWN, st);
    return rc;
}

int k3g_experts(K3gCtx *c, const K3gLayer *L, const float *x, int T, const int32_t *idx,
                const float *wt, float *out, hipStream_t st)
{
    if (!fits_experts(c, L, T)) return -1;
    const int d = L->hidden, k = L->topk;
    const int SI = L->shared_inter, lat = L->latent > 0 ? L->latent : d;
    const int projected = L->down != NULL;
    int rc = 0;
    if (fusable(c, L, T)) {
        /* one launch: the copies it needs must be in before it starts */
        if (c->routed_wait) {
            if (hipStreamWaitEvent(st, c->routed_wait, 0) != hipSuccess) return -1;
            c->routed_wait = NULL;
        }
        c->paths |= 2;
        return run_fused(c, L, x, T, out, (int32_t *)idx, (float *)wt, 1, st);
    }
    if (gemmable(c, L)) {
        c->paths |= 4;
        return experts_gemm(c, L, x, T, idx, wt, out, c->contrib, c->gemm_fp8, 1, st);
    }
    c->paths |= 1;
    if (c->routed_wait) {
        if (hipStreamWaitEvent(st, c->routed_wait, 0) != hipSuccess) return -1;
        c->routed_wait = NULL;
    }
    if (L->expert_fmt == K3G_EXPERT_MXFP4_TILED || L->shared_fmt != 0) {
        fprintf(stderr, "k3moe: tiled experts need the Kimi-K2 layer shape (no latent "
                        "projection, bf16 shared expert, widths multiple of 32)\n");
        return -1;
    }

    const float *z = x;
    if (projected) {
        k3g_stage_begin(c, K3G_ST_LATENT, st);
        rc |= k3k_dense(wfmt(L->wdt), L->down, NULL, lat, d, x, d, T, c->z, lat, 0.f, 0.f, st);
        k3g_stage_end(c, K3G_ST_LATENT, st);
        z = c->z;
    }
    rc |= routed_staged(c, L, z, lat, T, idx, c->contrib, st);
    if (SI > 0) {
        k3g_stage_begin(c, K3G_ST_SH_GATEUP, st);
        rc |= k3k_dense(wfmt(L->wdt), L->sh1, L->sh3, SI, d, x, d, T, c->sh_h, SI,
                        L->act_b1, L->act_b2, st);
        k3g_stage_end(c, K3G_ST_SH_GATEUP, st);
        k3g_stage_begin(c, K3G_ST_SH_DOWN, st);
        rc |= k3k_dense(wfmt(L->wdt), L->sh2, NULL, d, SI, c->sh_h, SI, T, c->sh_out, d,
                        0.f, 0.f, st);
        k3g_stage_end(c, K3G_ST_SH_DOWN, st);
    }
    if (!projected && !L->up && !L->latent_norm) {
        k3g_stage_begin(c, K3G_ST_COMBINE, st);
        rc |= k3k_combine(c->contrib, idx, wt, T, k, d, SI > 0 ? c->sh_out : NULL, out, st);
        k3g_stage_end(c, K3G_ST_COMBINE, st);
    } else {
        rc |= k3k_combine(c->contrib, idx, wt, T, k, lat, NULL, c->accl, st);
        if (L->latent_norm) rc |= k3k_rmsnorm(c->accl, c->accl, L->latent_norm, lat, T,
                                              L->rms_eps, st);
        if (L->up)
            rc |= k3k_dense(wfmt(L->wdt), L->up, NULL, d, lat, c->accl, lat, T, out, d, 0.f,
                            0.f, st);
        else if (hipMemcpyAsync(out, c->accl, (size_t)T * d * 4, hipMemcpyDeviceToDevice, st) !=
                 hipSuccess)
            rc = -1;
        if (SI > 0) rc |= k3k_add(out, c->sh_out, (size_t)T * d, st);
    }
    return rc ? -1 : 0;
}

/* The fused decode kernel for T <= 4 tokens: with given = 0 it routes inside (idx/wt
 * receive the routing), with given = 1 it takes the routing in idx/wt. */
static int run_fused(K3gCtx *c, const K3gLayer *L, const float *x, int T, float *out,
                     int32_t *idx, float *wt, int given, hipStream_t st)
{
    K3kDecode a;
    memset(&a, 0, sizeof a);
    a.T = T;
    a.d = L->hidden;
    a.E = L->n_experts;
    a.k = L->topk;
    a.I = L->inter;
    a.SI = L->shared_inter;
    a.renorm = L->renorm;
    a.routed_scale = L->routed_scale;
    a.b1 = L->act_b1;
    a.b2 = L->act_b2;
    a.gate = L->gate;
    a.bias = L->bias;
    a.eq = L->experts;
    a.sh1 = (const uint16_t *)L->sh1;
    a.sh3 = (const uint16_t *)L->sh3;
    a.sh2 = (const uint16_t *)L->sh2;
    a.x = x;
    a.out = out;
    a.idx = idx;
    a.wt = wt;
    a.rs = c->rs;
    a.xq8 = c->xq8;
    a.xq16 = c->xq16;
    a.gpart = c->gpart;
    a.hq8 = c->hq8;
    a.sgpart = c->sgpart;
    a.hq16 = c->hq16;
    a.contrib = c->dcontrib;
    a.shpart = c->shpart;
    a.rpart = c->rpart;
    const int lat = L->latent > 0 ? L->latent : L->hidden;
    a.L = lat;
    if (lat != L->hidden) {
        a.down = (const uint16_t *)L->down;
        a.up = (const uint16_t *)L->up;
        a.lnorm = L->latent_norm;
        a.rms_eps = L->rms_eps;
        a.zpart = c->dzpart;
        a.zq8 = c->dzq8;
        a.accl = c->daccl;
        a.nss = c->dnss;
        a.aq16 = c->daq16;
        a.upart = c->dupart;
    }
    const int words = (int)(c->sync_bytes / 4);
    a.sync = c->sync + (size_t)(c->epoch & 1) * words;
    a.sync_clear = c->sync + (size_t)((c->epoch & 1) ^ 1) * words;
    a.sync_words = words;
    a.err = c->err;
    a.stats = c->stats;
    a.force = c->force_exact;
    a.given = given;
    a.spin_limit = 1ll << 21;
    a.trace = c->trace;
    a.hidx = c->host_idx;
    a.hwt = c->host_idx ? c->host_wt : NULL;
    a.herr = c->host_err;
    a.hflag = c->host_idx && c->host_wt ? c->host_flag : NULL;
    k3g_stage_begin(c, K3G_ST_FUSED, st);
    const int rc = k3k_decode_fused(&a, st);
    k3g_stage_end(c, K3G_ST_FUSED, st);
    if (rc == 0) c->epoch = (c->epoch + 1) & 0x3fffffff;   /* the next call's bank */
    return rc;
}

int k3g_await_flag(const volatile int *flag, double limit_s)
{
    struct timespec t0, t1;
    clock_gettime(CLOCK_MONOTONIC, &t0);
    for (unsigned i = 1;; i++) {
        if (*flag) {
            __atomic_thread_fence(__ATOMIC_ACQUIRE);
            return 1;
        }
        if (!(i & 1023)) {
            clock_gettime(CLOCK_MONOTONIC, &t1);
            if ((double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec) >
                limit_s)
                return 0;
        }
    }
}

int k3g_err_read(K3gCtx *c)
{
    int e = 0;
    if (hipSetDevice(c->device) != hipSuccess ||
        hipMemcpy(&e, c->err, sizeof e, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    return e;
}

int k3g_fuses(const K3gCtx *c, const K3gLayer *L, int T)
{
    const int have = L->expert_fmt == K3G_EXPERT_F32 ? (L->w1 && L->w3 && L->w2)
                                                     : L->experts != NULL;
    return have && fits(c, L, T) && fusable(c, L, T);
}

int k3g_moe(K3gCtx *c, const K3gLayer *L, const float *x, int T, float *out, int32_t *idx,
            float *wt, void *stream)
{
    hipStream_t st = stream ? (hipStream_t)stream : c->stream;
    if (!idx) idx = c->idx;
    if (!wt) wt = c->wt;
    if (!fits_experts(c, L, T)) return -1;
    if (fusable(c, L, T)) {
        c->paths |= 2;
        return run_fused(c, L, x, T, out, idx, wt, 0, st);
    }
    if (gemmable(c, L) && !c->routed_wait) {
        /* x's pieces, then the shared expert on the side stream (only the final combine
         * needs it) beside the router, the dispatch and the routed experts on this one */
        c->paths |= 4;
        int rc = k3k_set_i32(c->xflag, 0, st);
        rc |= gemm_pieces(c, L, x, T, c->gemm_fp8, st);
        if (L->shared_inter > 0) {
            if (hipEventRecord(c->ev_in, st) != hipSuccess ||
                hipStreamWaitEvent(c->side, c->ev_in, 0) != hipSuccess)
                rc = -1;
            rc |= shared_expert(c, L, T, c->kpart2, c->side);
            if (hipEventRecord(c->ev_shared, c->side) != hipSuccess) rc = -1;
        }
        /* x's piece-1 flag is this x's: the router skips the product of x's second piece
         * when every x is a bf16 value */
        c->route_x1flag = c->xflag;
        rc |= k3g_route(c, L, x, T, idx, wt, st);
        c->route_x1flag = NULL;
        /* the dispatch's flag argument (cleared) is the spare one: x's is set above */
        k3g_stage_begin(c, K3G_ST_DISPATCH, st);
        rc |= k3k_dispatch_tiles(idx, T * L->topk, L->n_experts, c->cnt, c->base, c->off,
                                 c->act, c->nact, c->perm, c->err, c->tiles, c->ntiles,
                                 c->zflag, st);
        k3g_stage_end(c, K3G_ST_DISPATCH, st);
        rc |= gemm_body(c, L, x, T, idx, wt, out, c->contrib, c->gemm_fp8, 1, 1, st);
        return rc ? -1 : 0;
    }
    if (k3g_route(c, L, x, T, idx, wt, st) != 0) return -1;
    return k3g_experts(c, L, x, T, idx, wt, out, st);
}

int k3g_sync(K3gCtx *c, void *stream)
{
    hipStream_t st = stream ? (hipStream_t)stream : c->stream;
    if (hipStreamSynchronize(st) != hipSuccess) return -1;
    int e = 0;
    if (hipMemcpy(&e, c->err, sizeof e, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    return k3g_err_settle(c, e);
}

int k3g_err_settle(K3gCtx *c, int e)
{
    if (e) {
        fprintf(stderr, "k3moe: device reported error %d (%s)\n", e,
                e == 1 ? "routed expert index out of range" : "bounded wait ran out");
        int z = 0;
        hipMemcpy(c->err, &z, sizeof z, hipMemcpyHostToDevice);
        /* a call cut short leaves the fused kernel's counters short: start over */
        hipMemset(c->sync, 0, 2 * c->sync_bytes);
        c->epoch = 0;
        return e;
    }
    return 0;
}

/* ------------------------------------------------------ device API, step by step ---- */
/* The layer's steps one at a time, device pointers on `stream` (NULL: the context's). */

int k3g_dispatch(K3gCtx *c, const int32_t *idx, int T, int topk, int n_experts, int32_t *perm,
                 int32_t *off, void *stream)
{
    if (!c || !idx || !perm || !off || T < 1 || topk < 1 || T > c->max_tokens ||
        topk > c->topk || n_experts < 1 || n_experts > c->n_experts)
        return -1;
    hipStream_t st = stream ? (hipStream_t)stream : c->stream;
    hipSetDevice(c->device);
    return k3k_dispatch(idx, T * topk, n_experts, c->cnt, c->base, off, c->act, c->nact, perm,
                        c->err, st);
}

int k3g_expert_gemv(K3gCtx *c, const K3gLayer *L, const float *x, int T, const int32_t *idx,
                    float *contrib, void *stream)
{
    if (!c || !L || !x || !idx || !contrib || !fits_experts(c, L, T)) return -1;
    if (L->expert_fmt == K3G_EXPERT_MXFP4_TILED || L->down ||
        (L->latent > 0 && L->latent != L->hidden)) {
        fprintf(stderr, "k3g_expert_gemv: needs checkpoint-layout (or fp32) experts and no "
                        "latent projection\n");
        return -1;
    }
    hipStream_t st = stream ? (hipStream_t)stream : c->stream;
    hipSetDevice(c->device);
    return routed_staged(c, L, x, L->hidden, T, idx, contrib, st) ? -1 : 0;
}

static int grouped(K3gCtx *c, const K3gLayer *L, const float *x, int T, const int32_t *idx,
                   float *contrib, int fp8, void *stream)
{
    if (!c || !L || !x || !idx || !contrib || !fits_experts(c, L, T)) return -1;
    if (L->expert_fmt != K3G_EXPERT_MXFP4_TILED || L->down || L->up || L->latent_norm ||
        (L->latent > 0 && L->latent != L->hidden) || L->hidden % 32 || L->inter % 32) {
        fprintf(stderr, "k3g_grouped_gemm: needs experts in the tiled MXFP4 layout and no "
                        "latent projection\n");
        return -1;
    }
    hipStream_t st = stream ? (hipStream_t)stream : c->stream;
    hipSetDevice(c->device);
    return experts_gemm(c, L, x, T, idx, NULL, NULL, contrib, fp8, 0, st);
}

int k3g_grouped_gemm_bf16(K3gCtx *c, const K3gLayer *L, const float *x, int T,
                          const int32_t *idx, float *contrib, void *stream)
{
    return grouped(c, L, x, T, idx, contrib, 0, stream);
}

int k3g_grouped_gemm_f8f6f4(K3gCtx *c, const K3gLayer *L, const float *x, int T,
                            const int32_t *idx, float *contrib, void *stream)
{
    return grouped(c, L, x, T, idx, contrib, 1, stream);
}

int k3g_combine(K3gCtx *c, const float *contrib, const int32_t *idx, const float *wt, int T,
                int topk, int n, const float *add, float *out, void *stream)
{
    if (!c || !contrib || !idx || !wt || !out || T < 1 || topk < 1 || n < 1) return -1;
    hipStream_t st = stream ? (hipStream_t)stream : c->stream;
    hipSetDevice(c->device);
    return k3k_combine(contrib, idx, wt, T, topk, n, add, out, st);
}
