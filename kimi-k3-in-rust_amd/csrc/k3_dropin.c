/* k3_dropin.c - the engine's MoE entry points (k3_router, k3_moe, k3_moe_prefill,
 * k3_matmul_mxfp4, k3_mxfp4_dequant, k3_moe_scratch, k3_expert_drops) on the GPU,
 * with the engine's host-pointer signatures, synchronous semantics and error
 * behaviour (C99).
 *
 * Host weights are mirrored into HBM on first use, keyed by (address, size), and then
 * reused: the engine binds a layer's weights once and passes the same pointers every
 * token. Experts from a K3ExpertSrc are fetched with the engine's own call pattern
 * (getmany then get per slot for k3_moe, per unique expert per 64-token chunk for
 * k3_moe_prefill, src/core/k3_ops.c:604-627 and :756-766), so a cache behind the source
 * sees the same requests. A source returning host pointers has each expert copied to
 * HBM right after get(), before the next get() can evict it; the HBM expert cache
 * (k3gc_*) returns device pointers and is used in place. */
#include "k3g_ctx.h"
#include "k3gc_cache.h"

#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

long k3_expert_drops = 0;

static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;

/* ----------------------------------------------------------- per-device state ---- */
typedef struct {
    const void *host;
    size_t bytes;
    uint64_t print;              /* sampled fingerprint of the host bytes at upload */
    void *dev;
} Mirror;

typedef struct {
    int used;
    K3gCtx *ctx;
    K3gLayer shape;              /* what ctx was sized for */
    int ctx_tokens;
    Mirror *mir;
    int nmir, capmir;
    void *stage;                 /* scratch device buffer, grow-only */
    size_t stage_bytes;
    K3ExpertQ *eq_dev;           /* [cap_e] device expert table */
    int cap_e;
} DevState;

#define K3_MAX_DEV 16
static DevState g_dev[K3_MAX_DEV];

static DevState *dev_state(void)
{
    int d = 0;
    K3G_CHECK(hipGetDevice(&d));
    if (d < 0 || d >= K3_MAX_DEV) k3g_fatal("device ordinal beyond the drop-in's table");
    g_dev[d].used = 1;
    return &g_dev[d];
}

/* FNV-1a over 64 eight-byte samples spread across the buffer (all of it when short):
 * cheap enough to check on every call, and it catches a buffer that was freed and
 * reused for other weights at the same address. */
static uint64_t fingerprint(const void *host, size_t bytes)
{
    const unsigned char *b = (const unsigned char *)host;
    uint64_t h = 1469598103934665603ull;
    if (bytes <= 512) {
        for (size_t i = 0; i < bytes; i++) { h ^= b[i]; h *= 1099511628211ull; }
        return h;
    }
    for (int k = 0; k < 64; k++) {
        const size_t at = (size_t)k * ((bytes - 8) / 63);
        for (int i = 0; i < 8; i++) { h ^= b[at + i]; h *= 1099511628211ull; }
    }
    return h;
}

/* Device copy of `bytes` of host memory at `host`, uploaded on first use and again
 * whenever the sampled fingerprint shows the host bytes changed. */
static const void *mirror(DevState *s, const void *host, size_t bytes)
{
    if (!host || !bytes) return NULL;
    const uint64_t fp = fingerprint(host, bytes);
    for (int i = 0; i < s->nmir; i++)
        if (s->mir[i].host == host && s->mir[i].bytes == bytes) {
            if (s->mir[i].print != fp) {
                K3G_CHECK(hipMemcpy(s->mir[i].dev, host, bytes, hipMemcpyHostToDevice));
                s->mir[i].print = fp;
            }
            return s->mir[i].dev;
        }
    if (s->nmir == s->capmir) {
        const int nc = s->capmir ? 2 * s->capmir : 32;
        Mirror *m = (Mirror *)realloc(s->mir, (size_t)nc * sizeof *m);
        if (!m) k3g_fatal("out of host memory for the weight mirror table");
        s->mir = m;
        s->capmir = nc;
    }
    void *dev = NULL;
    K3G_CHECK(hipMalloc(&dev, bytes));
    K3G_CHECK(hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice));
    s->mir[s->nmir].host = host;
    s->mir[s->nmir].bytes = bytes;
    s->mir[s->nmir].print = fp;
    s->mir[s->nmir].dev = dev;
    s->nmir++;
    return dev;
}

static void *stage(DevState *s, size_t bytes)
{
    if (bytes > s->stage_bytes) {
        if (s->stage) K3G_CHECK(hipFree(s->stage));
        s->stage = NULL;
        const size_t nb = bytes + bytes / 4;
        K3G_CHECK(hipMalloc(&s->stage, nb));
        s->stage_bytes = nb;
    }
    return s->stage;
}

void k3moe_forget_weights(void)
{
    pthread_mutex_lock(&g_lock);
    int cur = 0;
    hipGetDevice(&cur);
    for (int d = 0; d < K3_MAX_DEV; d++) {
        DevState *s = &g_dev[d];
        if (!s->used) continue;
        hipSetDevice(d);
        hipDeviceSynchronize();
        for (int i = 0; i < s->nmir; i++) hipFree(s->mir[i].dev);
        s->nmir = 0;
    }
    hipSetDevice(cur);
    pthread_mutex_unlock(&g_lock);
}

/* A context at least as large as this layer and token count. */
static K3gCtx *ctx_for(DevState *s, const K3gLayer *L, int T)
{
    const int lat = L->latent > 0 ? L->latent : L->hidden;
    const K3gLayer *o = &s->shape;
    if (s->ctx && o->hidden == L->hidden && o->n_experts >= L->n_experts && o->topk >= L->topk &&
        o->inter >= L->inter && o->shared_inter >= L->shared_inter && o->latent >= lat &&
        s->ctx_tokens >= T)
        return s->ctx;
    K3gLayer n = *L;
    n.latent = lat;
    if (s->ctx && o->hidden == L->hidden) {
        if (o->n_experts > n.n_experts) n.n_experts = o->n_experts;
        if (o->topk > n.topk) n.topk = o->topk;
        if (o->inter > n.inter) n.inter = o->inter;
        if (o->shared_inter > n.shared_inter) n.shared_inter = o->shared_inter;
        if (o->latent > n.latent) n.latent = o->latent;
        if (s->ctx_tokens > T) T = s->ctx_tokens;
    }
    if (s->ctx) k3g_ctx_destroy(s->ctx);
    s->ctx = NULL;
    int dev = 0;
    K3G_CHECK(hipGetDevice(&dev));
    if (k3g_ctx_create(&s->ctx, dev, &n, T) != 0) k3g_fatal("cannot create a device context");
    s->shape = n;
    s->ctx_tokens = T;
    return s->ctx;
}

/* ----------------------------------------------------------------- router ---- */
void k3_router(int *idx, float *w, const float *x, const float *W, const float *bias,
               int hidden, int n_experts, int topk, int renorm, float routed_scale)
{
    if (topk < 1 || topk > K3G_MAX_TOPK || n_experts < 1 || n_experts > 1024)
        k3g_fatal("k3_router: top-k or expert count outside what the GPU router supports");
    pthread_mutex_lock(&g_lock);
    DevState *s = dev_state();
    K3gLayer L;
    memset(&L, 0, sizeof L);
    L.hidden = hidden;
    L.latent = hidden;
    L.n_experts = n_experts;
    L.topk = topk;
    L.inter = 16;
    L.renorm = renorm;
    L.routed_scale = routed_scale;
    L.gate = (const float *)mirror(s, W, (size_t)n_experts * hidden * 4);
    L.bias = (const float *)mirror(s, bias, bias ? (size_t)n_experts * 4 : 0);
    K3gCtx *c = ctx_for(s, &L, 1);
    float *xd = (float *)stage(s, (size_t)hidden * 4);
    K3G_CHECK(hipMemcpyAsync(xd, x, (size_t)hidden * 4, hipMemcpyHostToDevice, c->stream));
    if (k3g_route(c, &L, xd, 1, c->idx, c->wt, c->stream) != 0)
        k3g_fatal("k3_router: launch failed");
    K3G_CHECK(hipMemcpyAsync(idx, c->idx, (size_t)topk * 4, hipMemcpyDeviceToHost, c->stream));
    K3G_CHECK(hipMemcpyAsync(w, c->wt, (size_t)topk * 4, hipMemcpyDeviceToHost, c->stream));
    if (k3g_sync(c, NULL) != 0) k3g_fatal("k3_router: device error");
    pthread_mutex_unlock(&g_lock);
}

size_t k3_moe_scratch(const K3Cfg *c)
{
    /* src/core/k3_ops.c:658-666 */
    const int SI = c->moe_inter * c->n_shared;
    return (size_t)2 * c->latent + (size_t)3 * c->moe_inter + (size_t)c->latent +
           (size_t)3 * SI + (size_t)c->hidden;
}

/* ---------------------------------------------------------------- MoE layer ---- */
static size_t wsz(int wdt) { return wdt == K3_WBF16 ? 2 : 4; }

/* Copy one host-resident expert into staging slot `slot` and record its device
 * pointers. */
static K3ExpertQ stage_expert(const K3ExpertQ *q, unsigned char *base, const K3gExpertLayout *g,
                              int I, int L, hipStream_t st)
{
    K3ExpertQ d;
    const size_t p13 = (size_t)I * (L / 2), s13 = (size_t)I * ((L + 31) / 32);
    const size_t p2 = (size_t)L * (I / 2), s2 = (size_t)L * ((I + 31) / 32);
    K3G_CHECK(hipMemcpyAsync(base + g->p1_off, q->p1, p13, hipMemcpyHostToDevice, st));
    K3G_CHECK(hipMemcpyAsync(base + g->s1_off, q->s1, s13, hipMemcpyHostToDevice, st));
    K3G_CHECK(hipMemcpyAsync(base + g->p2_off, q->p2, p2, hipMemcpyHostToDevice, st));
    K3G_CHECK(hipMemcpyAsync(base + g->s2_off, q->s2, s2, hipMemcpyHostToDevice, st));
    K3G_CHECK(hipMemcpyAsync(base + g->p3_off, q->p3, p13, hipMemcpyHostToDevice, st));
    K3G_CHECK(hipMemcpyAsync(base + g->s3_off, q->s3, s13, hipMemcpyHostToDevice, st));
    /* the source may evict these bytes at its next get(); finish the copy first */
    K3G_CHECK(hipStreamSynchronize(st));
    d.p1 = base + g->p1_off; d.s1 = base + g->s1_off;
    d.p2 = base + g->p2_off; d.s2 = base + g->s2_off;
    d.p3 = base + g->p3_off; d.s3 = base + g->s3_off;
    return d;
}

typedef struct {
    DevState *s;
    const K3MoeW *w;
    int E, I, L, device_src;
    K3gExpertLayout geo;
    unsigned char *slots;        /* staging slots for host-resident experts */
    int nslot, maxslot;
    int *slot_of;                /* [E] */
    K3ExpertQ *table;            /* host copy of the device table [E] */
    unsigned char *have;         /* [E] expert resolved in this call */
    hipStream_t st;
} Fetcher;

/* get() one expert and resolve it to device pointers. Returns 0, or -1 on a miss. */
static int fetch_one(Fetcher *f, int e, int resident_only)
{
    K3ExpertQ q;
    const K3MoeW *w = f->w;
    const int miss = resident_only ? !w->src->resident(w->src, w->layer, e, &q)
                                   : (w->src->get(w->src, w->layer, e, &q) != 0);
    if (miss) return -1;
    if (f->device_src) {
        f->table[e] = q;
    } else if (!f->have[e]) {
        if (f->nslot >= f->maxslot) k3g_fatal("expert staging overflow");
        const int sl = f->nslot++;
        f->slot_of[e] = sl;
        f->table[e] = stage_expert(&q, f->slots + (size_t)sl * f->geo.nbytes, &f->geo, f->I,
                                   f->L, f->st);
    }
    f->have[e] = 1;
    return 0;
}

static void drop_msg(int layer, int e, const char *what)
{
    k3_expert_drops++;
    fprintf(stderr, "EXPERT DROP: layer %d expert %d failed to load; this %s is CORRUPT\n",
            layer, e, what);
}

/* mode 0: k3_moe semantics; mode 1: k3_moe_prefill semantics. */
static void moe_run(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T,
                    int *idx_out, float *wt_out, int mode)
{
    if (T <= 0) return;
    if (c->topk < 1 || c->topk > K3_MAX_TOPK) k3g_fatal("k3_moe: topk outside 1..64");
    if (w->wdt == K3_WI8) k3g_fatal("k3_moe: int8 draft weights are not on the GPU path");
    const int d = c->hidden, E = c->n_experts, k = c->topk, I = c->moe_inter;
    const int L = w->down ? c->latent : d;
    const int SI = c->moe_inter * c->n_shared;
    if (!w->down && c->latent != d && c->latent != 0)
        k3g_fatal("k3_moe: down == NULL (no latent) needs latent == hidden");

    pthread_mutex_lock(&g_lock);
    DevState *s = dev_state();
    K3gLayer G;
    memset(&G, 0, sizeof G);
    G.hidden = d;
    G.n_experts = E;
    G.topk = k;
    G.inter = I;
    G.shared_inter = SI;
    G.latent = L;
    G.renorm = c->moe_renorm;
    G.routed_scale = c->routed_scale;
    G.act_b1 = c->situ_b1;
    G.act_b2 = c->situ_b2;
    G.rms_eps = c->rms_eps;
    G.wdt = w->wdt;
    G.gate = (const float *)mirror(s, w->gate, (size_t)E * d * 4);
    G.bias = (const float *)mirror(s, w->bias, w->bias ? (size_t)E * 4 : 0);
    G.down = mirror(s, w->down, w->down ? (size_t)L * d * wsz(w->wdt) : 0);
    G.up = mirror(s, w->up, w->up ? (size_t)d * L * wsz(w->wdt) : 0);
    G.latent_norm = c->latent_norm ? (const float *)mirror(s, w->latent_norm, (size_t)L * 4)
                                   : NULL;
    if (SI > 0) {
        G.sh1 = mirror(s, w->sh1, (size_t)SI * d * wsz(w->wdt));
        G.sh3 = mirror(s, w->sh3, (size_t)SI * d * wsz(w->wdt));
        G.sh2 = mirror(s, w->sh2, (size_t)d * SI * wsz(w->wdt));
    }
    if (!w->src) {
        G.expert_fmt = 1;
        G.w1 = (const float *)mirror(s, w->w1, (size_t)E * I * L * 4);
        G.w3 = (const float *)mirror(s, w->w3, (size_t)E * I * L * 4);
        G.w2 = (const float *)mirror(s, w->w2, (size_t)E * L * I * 4);
    }
    K3gCtx *ctx = ctx_for(s, &G, T);
    hipStream_t st = ctx->stream;

    /* one staging buffer: x [T][d], out [T][d], then the host-resident experts' slots */
    const int device_src = w->src ? k3gc_is_device_src(w->src) : 0;
    const K3gExpertLayout geo = k3g_expert_layout(L, I);
    const int maxslot = (w->src && !device_src) ? (T * k < E ? T * k : E) : 0;
    const size_t xb = ((size_t)T * d * 4 + 255) & ~(size_t)255;
    unsigned char *sb = (unsigned char *)stage(s, 2 * xb + (size_t)maxslot * geo.nbytes);
    float *xd = (float *)sb, *od = (float *)(sb + xb);
    K3G_CHECK(hipMemcpyAsync(xd, x, (size_t)T * d * 4, hipMemcpyHostToDevice, st));
    if (k3g_route(ctx, &G, xd, T, ctx->idx, ctx->wt, st) != 0) k3g_fatal("k3_moe: router launch");

    int *ridx = (int *)malloc((size_t)T * k * sizeof(int));
    float *rwt = (float *)malloc((size_t)T * k * sizeof(float));
    int *last = (int *)malloc((size_t)k * sizeof(int));
    float *lastw = (float *)malloc((size_t)k * sizeof(float));
    if (!ridx || !rwt || !last || !lastw) k3g_fatal("k3_moe: out of host memory");
    K3G_CHECK(hipMemcpyAsync(ridx, ctx->idx, (size_t)T * k * 4, hipMemcpyDeviceToHost, st));
    K3G_CHECK(hipMemcpyAsync(rwt, ctx->wt, (size_t)T * k * 4, hipMemcpyDeviceToHost, st));
    if (k3g_sync(ctx, NULL) != 0) k3g_fatal("k3_moe: device error in the router");
    memcpy(last, ridx + (size_t)(T - 1) * k, (size_t)k * sizeof(int));
    memcpy(lastw, rwt + (size_t)(T - 1) * k, (size_t)k * sizeof(float));

    const int cache_only = w->cache_only && w->src && w->src->resident;
    if (cache_only) {
        /* src/core/k3_ops.c:585-594: keep the resident subset in slot order and divide
         * its weights by their float sum */
        for (int t = 0; t < T; t++) {
            int *it = ridx + (size_t)t * k;
            float *wt = rwt + (size_t)t * k;
            int keep[K3_MAX_TOPK], m = 0;
            float wsum = 0.0f;
            for (int j = 0; j < k; j++) {
                keep[j] = w->src->resident(w->src, w->layer, it[j], NULL);
                if (keep[j]) wsum += wt[j];
            }
            for (int j = 0; j < k; j++) {
                if (!keep[j]) { it[j] = -1; continue; }
                if (wsum > 0.0f) wt[j] /= wsum;
                if (t == T - 1) { last[m] = it[j]; lastw[m] = wt[j]; }
                m++;
            }
        }
    }

    K3gCache *hc_end = NULL;
    if (w->src) {
        Fetcher f;
        memset(&f, 0, sizeof f);
        f.s = s;
        f.w = w;
        f.E = E;
        f.I = I;
        f.L = L;
        f.st = st;
        f.device_src = device_src;
        f.geo = geo;
        f.slots = sb + 2 * xb;
        f.maxslot = maxslot;
        f.slot_of = (int *)malloc((size_t)E * sizeof(int));
        f.table = (K3ExpertQ *)calloc((size_t)E, sizeof(K3ExpertQ));
        f.have = (unsigned char *)calloc((size_t)E, 1);
        if (!f.slot_of || !f.table || !f.have) k3g_fatal("k3_moe: out of host memory");
        K3gCache *hc = device_src ? k3gc_of_src(w->src) : NULL;
        if (hc && hc->bank->layout != K3G_EXPERT_MXFP4)
            k3g_fatal("k3_moe: an HBM cache used through the drop-in must hold checkpoint-"
                      "layout expert runs");
        /* every slot handed out during this call stays put until its kernels are done */
        if (hc) k3gc_step_begin(hc);
        const int per_token = mode == 0 || T <= 1 || cache_only;
        if (per_token) {
            /* src/core/k3_ops.c:604-627 */
            for (int t = 0; t < T; t++) {
                int *it = ridx + (size_t)t * k;
                int ids[K3_MAX_TOPK], nk = 0;
                for (int j = 0; j < k; j++) if (it[j] >= 0) ids[nk++] = it[j];
                if (!cache_only && w->src->getmany) w->src->getmany(w->src, w->layer, ids, nk);
                for (int j = 0; j < k; j++) {
                    if (it[j] < 0) continue;
                    if (fetch_one(&f, it[j], cache_only) != 0) {
                        if (!cache_only) drop_msg(w->layer, it[j], "token");
                        it[j] = -1;
                    }
                }
            }
        } else {
            /* src/core/k3_ops.c:707-766: 64-token chunks, unique experts in first-seen
             * order, one get() each */
            int *uniq = (int *)malloc((size_t)64 * k * sizeof(int));
            unsigned char *seen = (unsigned char *)malloc((size_t)E);
            if (!uniq || !seen) k3g_fatal("k3_moe_prefill: out of host memory");
            for (int t0 = 0; t0 < T; t0 += 64) {
                const int n = T - t0 < 64 ? T - t0 : 64;
                memset(seen, 0, (size_t)E);
                int nu = 0;
                for (int t = t0; t < t0 + n; t++)
                    for (int j = 0; j < k; j++) {
                        const int e = ridx[(size_t)t * k + j];
                        if (e >= 0 && e < E && !seen[e]) { seen[e] = 1; uniq[nu++] = e; }
                    }
                if (n > 1 && w->src->getmany) w->src->getmany(w->src, w->layer, uniq, nu);
                if (n == 1 && w->src->getmany) w->src->getmany(w->src, w->layer, ridx + (size_t)t0 * k, k);
                if (n == 1) {
                    /* a one-token chunk takes k3_moe's per-slot path (:709-710) */
                    for (int j = 0; j < k; j++) {
                        int *e = ridx + (size_t)t0 * k + j;
                        if (*e >= 0 && fetch_one(&f, *e, 0) != 0) {
                            drop_msg(w->layer, *e, "token");
                            *e = -1;
                        }
                    }
                    continue;
                }
                for (int u = 0; u < nu; u++) {
                    if (fetch_one(&f, uniq[u], 0) == 0) continue;
                    drop_msg(w->layer, uniq[u], "chunk");
                    for (int t = t0; t < t0 + n; t++)
                        for (int j = 0; j < k; j++)
                            if (ridx[(size_t)t * k + j] == uniq[u]) ridx[(size_t)t * k + j] = -1;
                }
            }
            free(uniq);
            free(seen);
        }
        if (s->cap_e < E) {
            if (s->eq_dev) K3G_CHECK(hipFree(s->eq_dev));
            K3G_CHECK(hipMalloc((void **)&s->eq_dev, (size_t)E * sizeof(K3ExpertQ)));
            s->cap_e = E;
        }
        K3G_CHECK(hipMemcpyAsync(s->eq_dev, f.table, (size_t)E * sizeof(K3ExpertQ),
                                 hipMemcpyHostToDevice, st));
        G.expert_fmt = 0;
        G.experts = s->eq_dev;
        K3G_CHECK(hipStreamSynchronize(st));
        free(f.slot_of);
        free(f.table);
        free(f.have);
        /* the misses copy on the cache's stream: the expert kernels wait for them */
        if (hc) k3gc_wait(hc, st);
        hc_end = hc;
    }

    K3G_CHECK(hipMemcpyAsync(ctx->idx, ridx, (size_t)T * k * 4, hipMemcpyHostToDevice, st));
    K3G_CHECK(hipMemcpyAsync(ctx->wt, rwt, (size_t)T * k * 4, hipMemcpyHostToDevice, st));
    if (k3g_experts(ctx, &G, xd, T, ctx->idx, ctx->wt, od, st) != 0)
        k3g_fatal("k3_moe: launch failed");
    if (hc_end) k3gc_step_end(hc_end, st);
    K3G_CHECK(hipMemcpyAsync(out, od, (size_t)T * d * 4, hipMemcpyDeviceToHost, st));
    if (k3g_sync(ctx, NULL) != 0) k3g_fatal("k3_moe: device error");

    /* idx/wt hold the last token's routing when the engine's per-token path produced
     * it; the batched prefill path leaves them untouched (src/core/k3_ops.c:699-714).
     * After a cache-only filter the resident subset is compacted to the front and the
     * rest keeps the router's values, as in the engine. */
    const int batched = mode == 1 && w->src && T > 1 && !cache_only;
    if (!batched || (T - 1) % 64 == 0) {
        memcpy(idx_out, last, (size_t)k * sizeof(int));
        memcpy(wt_out, lastw, (size_t)k * sizeof(float));
    }
    free(ridx);
    free(rwt);
    free(last);
    free(lastw);
    pthread_mutex_unlock(&g_lock);
}

void k3_moe(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T, int *idx,
            float *wt, float *scratch)
{
    (void)scratch;
    moe_run(out, x, w, c, T, idx, wt, 0);
}

void k3_moe_prefill(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T,
                    int *idx, float *wt, float *scratch)
{
    (void)scratch;
    moe_run(out, x, w, c, T, idx, wt, 1);
}

/* ------------------------------------------------------------ MXFP4 kernels ---- */
void k3_matmul_mxfp4(float *y, const float *x, const unsigned char *packed,
                     const unsigned char *scales, int in, int rows, int group)
{
    if (in & 1) {
        fprintf(stderr, "k3: FATAL, k3_matmul_mxfp4 called with in=%d, which is odd.\n", in);
        abort();
    }
    if (group > 64) {
        fprintf(stderr, "k3: FATAL, k3_matmul_mxfp4 called with group=%d, which exceeds 64.\n",
                group);
        abort();
    }
    if (group != K3_MXFP4_GROUP) {
        fprintf(stderr, "k3moe: FATAL, k3_matmul_mxfp4 on the GPU needs group 32, got %d.\n",
                group);
        abort();
    }
    if (rows <= 0 || in <= 0) return;
    pthread_mutex_lock(&g_lock);
    DevState *s = dev_state();
    K3gLayer L;
    memset(&L, 0, sizeof L);
    L.hidden = in;
    L.latent = in;
    L.n_experts = 1;
    L.topk = 1;
    L.inter = 16;
    K3gCtx *c = ctx_for(s, &L, 1);
    const size_t pb = (size_t)rows * (in / 2), sb = (size_t)rows * ((in + 31) / 32);
    const size_t xb = (size_t)in * 4, yb = (size_t)rows * 4;
    const size_t a0 = 0, a1 = (pb + 255) & ~(size_t)255, a2 = a1 + ((sb + 255) & ~(size_t)255);
    const size_t a3 = a2 + ((xb + 255) & ~(size_t)255);
    unsigned char *b = (unsigned char *)stage(s, a3 + yb);
    K3G_CHECK(hipMemcpyAsync(b + a0, packed, pb, hipMemcpyHostToDevice, c->stream));
    K3G_CHECK(hipMemcpyAsync(b + a1, scales, sb, hipMemcpyHostToDevice, c->stream));
    K3G_CHECK(hipMemcpyAsync(b + a2, x, xb, hipMemcpyHostToDevice, c->stream));
    if (k3k_mxfp4_gemv((float *)(b + a3), (const float *)(b + a2), b + a0, b + a1, in, rows,
                       c->stream) != 0)
        k3g_fatal("k3_matmul_mxfp4: launch failed");
    K3G_CHECK(hipMemcpyAsync(y, b + a3, yb, hipMemcpyDeviceToHost, c->stream));
    K3G_CHECK(hipStreamSynchronize(c->stream));
    pthread_mutex_unlock(&g_lock);
}

void k3_mxfp4_dequant(float *out, const unsigned char *packed, const unsigned char *scales,
                      int rows, int pcols, int group)
{
    if (rows <= 0 || pcols <= 0) return;
    if (group < 1) k3g_fatal("k3_mxfp4_dequant: group < 1");
    pthread_mutex_lock(&g_lock);
    DevState *s = dev_state();
    K3gLayer L;
    memset(&L, 0, sizeof L);
    L.hidden = 16;
    L.latent = 16;
    L.n_experts = 1;
    L.topk = 1;
    L.inter = 16;
    const int width = pcols * 2, ngrp = (width + group - 1) / group;
    const size_t pb = (size_t)rows * pcols, sb = (size_t)rows * ngrp;
    const size_t ob = (size_t)rows * width * 4;
    const size_t a1 = (pb + 255) & ~(size_t)255, a2 = a1 + ((sb + 255) & ~(size_t)255);
    K3gCtx *c = ctx_for(s, &L, 1);
    unsigned char *b = (unsigned char *)stage(s, a2 + ob);
    K3G_CHECK(hipMemcpyAsync(b, packed, pb, hipMemcpyHostToDevice, c->stream));
    K3G_CHECK(hipMemcpyAsync(b + a1, scales, sb, hipMemcpyHostToDevice, c->stream));
    if (k3k_dequant((float *)(b + a2), b, b + a1, rows, pcols, group, c->stream) != 0)
        k3g_fatal("k3_mxfp4_dequant: launch failed");
    K3G_CHECK(hipMemcpyAsync(out, b + a2, ob, hipMemcpyDeviceToHost, c->stream));
    K3G_CHECK(hipStreamSynchronize(c->stream));
    pthread_mutex_unlock(&g_lock);
}
