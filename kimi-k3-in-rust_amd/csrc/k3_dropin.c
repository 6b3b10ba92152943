/* k3_dropin.c - the engine's MoE entry points (k3_router, k3_moe, k3_moe_prefill,
 * k3_matmul_mxfp4, k3_mxfp4_dequant, k3_moe_scratch, k3_expert_drops) on the GPU,
 * with the engine's host-pointer signatures, synchronous semantics and error
 * behaviour (C99).
 *
 * Host weights are mirrored into HBM on first use, keyed by (address, size, layout), and
 * then reused: the engine binds a layer's weights once and passes the same pointers every
 * token. A sampled fingerprint of the host bytes is checked on every call and
 * k3moe_invalidate_weights() drops a mirror explicitly (a buffer reused for other weights
 * at the same address, as a ring of layer buffers does).
 *
 * Experts from a K3ExpertSrc are fetched with the engine's own call pattern (getmany then
 * get per slot for k3_moe, per unique expert per 64-token chunk for k3_moe_prefill,
 * src/core/k3_ops.c:604-627 and :756-766), so a cache behind the source sees the same
 * requests. A layer with bf16 shared/latent weights and MXFP4 experts from a source runs
 * on the matrix-core kernels: the fused decode kernel (Kimi-K2 shape, up to 4 tokens,
 * the routing given) or the grouped GEMMs. Their weights are in the tiled layouts: the
 * mirrors of the bf16 matrices are tiled once at upload; an HBM expert cache (k3gc_*)
 * with a tiled bank hands out tiled experts as they are; any other expert is copied to
 * HBM (a host source) and tiled into a staging slot before the next get() can evict it.
 * Other layers (fp32 weights, the fp32 resident expert bank, int8 draft weights) run on
 * the staged VALU kernels with experts in the checkpoint layout.
 *
 * Through an HBM cache the tokens of a call are cut into groups whose experts fit the
 * cache's unpinned slots at once; each group is one cache step: its experts stay put
 * until its kernels are done, then the next group fetches. */
#include "k3g_ctx.h"
#include "k3gc_cache.h"

#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

long k3_expert_drops = 0;

static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;
static int g_last_paths = 0;     /* kernels the last k3_moe / k3_moe_prefill call ran */

int k3moe_last_kernels(void) { return g_last_paths; }

/* ----------------------------------------------------------- per-device state ---- */
enum { MIR_ROWMAJOR = 0, MIR_TILED_BF16 = 1 };

typedef struct {
    const void *host;
    size_t bytes;                /* host bytes mirrored */
    int kind, rows, cols;
    uint64_t print;              /* sampled fingerprint of the host bytes at upload */
    uint64_t used;               /* call stamp of the last use */
    void *dev;
    size_t dev_bytes;
} Mirror;

typedef struct {
    int used;
    K3gCtx *ctx;
    K3gLayer shape;              /* what ctx was sized for */
    int ctx_tokens;
    Mirror *mir;
    int nmir, capmir;
    size_t mir_bytes;            /* device bytes the mirrors hold */
    uint64_t calls;
    void *stage;                 /* scratch device buffer of a call, grow-only */
    size_t stage_bytes;
    void *mstage;                /* the mirrors' upload buffer, grow-only: a mirror checked
                                    while a call runs uploads without touching its stage */
    size_t mstage_bytes;
    K3ExpertQ *eq_dev;           /* [cap_e] device expert table */
    int cap_e;
    /* host scratch of a call, grow-only; the routing and the activations travel through
     * pinned memory (asynchronous copies at the DMA rate) */
    unsigned char *pin;
    size_t pin_bytes;
    unsigned char *io;           /* device I/O area of a call, grow-only, starts zeroed */
    size_t io_bytes;
    int *ridx;
    float *rwt;
    size_t cap_pairs;
    int *slot_of, *uniq;
    K3ExpertQ *table;
    unsigned char *have, *seen;
    int cap_host_e;
    int defer;                   /* mirror lookups skip the fingerprint (checked later) */
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

static void *xgrow(void *p, size_t bytes)
{
    void *q = realloc(p, bytes ? bytes : 1);
    if (!q) k3g_fatal("out of host memory in the drop-in");
    return q;
}

/* dst <- src, with every host thread for large copies (the activations of a prefill) */
static void host_copy(void *dst, const void *src, size_t n)
{
    if (n < ((size_t)1 << 20)) {
        memcpy(dst, src, n);
        return;
    }
    const int parts = 16;
    const size_t per = ((n + parts - 1) / parts + 4095) & ~(size_t)4095;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < parts; i++) {
        const size_t a = (size_t)i * per;
        if (a < n) memcpy((char *)dst + a, (const char *)src + a, a + per < n ? per : n - a);
    }
}

/* Activations between the call's pinned staging and HBM: up to 1 MB by a copy kernel on
 * the compute stream (the kernels before and after it need no hand-over to a copy engine
 * and back, ~10 us each way at one token), larger ones by the copy engine. */
#define XFER_KERNEL_MAX ((size_t)1 << 20)
static void xfer(void *dst, const void *src, size_t n, hipMemcpyKind kind, hipStream_t st)
{
    if (!n) return;
    if (n <= XFER_KERNEL_MAX && k3k_copy(dst, src, n, st) == 0) return;
    K3G_CHECK(hipMemcpyAsync(dst, src, n, kind, st));
}

/* pinned host memory of at least `bytes`, grow-only; coherent (fine-grained), since the
 * fused decode kernel writes results and flags into it that the host reads while the
 * launch still runs */
static unsigned char *pinned(DevState *s, size_t bytes)
{
    if (bytes > s->pin_bytes) {
        if (s->pin) {
            K3G_CHECK(hipDeviceSynchronize());
            K3G_CHECK(hipHostFree(s->pin));
        }
        s->pin = NULL;
        const size_t nb = bytes + bytes / 4;
        K3G_CHECK(hipHostMalloc((void **)&s->pin, nb, hipHostMallocCoherent));
        s->pin_bytes = nb;
    }
    return s->pin;
}

/* The device I/O area of a call, grow-only. Its first word is the device error word of
 * the drop-in's context: zero, since any error aborts the process. */
static unsigned char *io_area(DevState *s, size_t bytes)
{
    if (bytes > s->io_bytes) {
        if (s->io) {
            K3G_CHECK(hipDeviceSynchronize());
            K3G_CHECK(hipFree(s->io));
        }
        s->io = NULL;
        const size_t nb = bytes + bytes / 4;
        K3G_CHECK(hipMalloc((void **)&s->io, nb));
        K3G_CHECK(hipMemset(s->io, 0, nb));
        s->io_bytes = nb;
    }
    return s->io;
}

/* host scratch for T * k pairs and E experts */
static void host_scratch(DevState *s, size_t pairs, int E)
{
    if (pairs > s->cap_pairs) {
        s->uniq = (int *)xgrow(s->uniq, pairs * sizeof(int));
        s->cap_pairs = pairs;
    }
    if (E > s->cap_host_e) {
        s->slot_of = (int *)xgrow(s->slot_of, (size_t)E * sizeof(int));
        s->table = (K3ExpertQ *)xgrow(s->table, (size_t)E * sizeof(K3ExpertQ));
        s->have = (unsigned char *)xgrow(s->have, (size_t)E);
        s->seen = (unsigned char *)xgrow(s->seen, (size_t)E);
        s->cap_host_e = E;
    }
}

/* FNV-1a over 64 eight-byte samples spread across the buffer (all of it when short):
 * cheap enough to check on every call, and it catches a buffer that was rewritten with
 * other weights at the same address. */
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

static void *stage(DevState *s, size_t bytes);

/* Bytes the mirrors may hold on one device (K3MOE_MIRROR_BYTES; default 64 GB): beyond
 * it the least recently used mirrors not used by the current call are dropped. */
static size_t mirror_budget(void)
{
    static size_t budget = 0;
    if (!budget) {
        const char *e = getenv("K3MOE_MIRROR_BYTES");
        const double v = e ? atof(e) : 0.0;
        budget = v > 0.0 ? (size_t)v : (size_t)64 << 30;
    }
    return budget;
}

static void mirror_drop(DevState *s, int i)
{
    K3G_CHECK(hipDeviceSynchronize());
    K3G_CHECK(hipFree(s->mir[i].dev));
    s->mir_bytes -= s->mir[i].dev_bytes;
    s->mir[i] = s->mir[--s->nmir];
}

static void mirror_make_room(DevState *s, size_t need)
{
    while (s->nmir > 0 && s->mir_bytes + need > mirror_budget()) {
        int victim = -1;
        for (int i = 0; i < s->nmir; i++)
            if (s->mir[i].used < s->calls && (victim < 0 || s->mir[i].used < s->mir[victim].used))
                victim = i;
        if (victim < 0) break;          /* everything is this call's: go over the budget */
        mirror_drop(s, victim);
    }
}

/* (Re)fill a mirror's device copy from the host bytes. */
static void mirror_upload(DevState *s, Mirror *m, hipStream_t st)
{
    if (m->kind == MIR_ROWMAJOR) {
        K3G_CHECK(hipMemcpy(m->dev, m->host, m->bytes, hipMemcpyHostToDevice));
        return;
    }
    /* row-major bf16 to the mirrors' upload buffer, then tiled into the mirror */
    if (m->bytes > s->mstage_bytes) {
        if (s->mstage) {
            K3G_CHECK(hipDeviceSynchronize());
            K3G_CHECK(hipFree(s->mstage));
        }
        s->mstage = NULL;
        K3G_CHECK(hipMalloc(&s->mstage, m->bytes));
        s->mstage_bytes = m->bytes;
    }
    void *tmp = s->mstage;
    K3G_CHECK(hipMemcpy(tmp, m->host, m->bytes, hipMemcpyHostToDevice));
    if (k3k_tile_bf16((uint16_t *)m->dev, (const uint16_t *)tmp, m->rows, m->cols, st) != 0)
        k3g_fatal("tiling a bf16 weight matrix failed");
    K3G_CHECK(hipStreamSynchronize(st));
}

/* Device copy of host weights: row-major (`bytes` of them), or for MIR_TILED_BF16 a bf16
 * [rows][cols] matrix in the tiled layout. Uploaded on first use and again whenever the
 * sampled fingerprint shows the host bytes changed. */
static const void *mirror_kind(DevState *s, const void *host, size_t bytes, int kind, int rows,
                               int cols, hipStream_t st)
{
    if (!host || !bytes) return NULL;
    for (int i = 0; i < s->nmir; i++) {
        Mirror *m = &s->mir[i];
        if (m->host == host && m->bytes == bytes && m->kind == kind && m->rows == rows &&
            m->cols == cols) {
            m->used = s->calls;
            if (!s->defer) {
                const uint64_t fp = fingerprint(host, bytes);
                if (m->print != fp) {
                    m->print = fp;
                    mirror_upload(s, m, st);
                }
            }
            return m->dev;
        }
    }
    const uint64_t fp = fingerprint(host, bytes);
    const size_t db = kind == MIR_ROWMAJOR ? bytes : k3k_tiled_bf16_bytes(rows, cols);
    if (!db) k3g_fatal("a bf16 weight matrix has no tiled layout (rows % 16, cols % 32)");
    mirror_make_room(s, db);
    if (s->nmir == s->capmir) {
        const int nc = s->capmir ? 2 * s->capmir : 32;
        s->mir = (Mirror *)xgrow(s->mir, (size_t)nc * sizeof(Mirror));
        s->capmir = nc;
    }
    Mirror *m = &s->mir[s->nmir];
    memset(m, 0, sizeof *m);
    m->host = host;
    m->bytes = bytes;
    m->kind = kind;
    m->rows = rows;
    m->cols = cols;
    m->print = fp;
    m->used = s->calls;
    m->dev_bytes = db;
    K3G_CHECK(hipMalloc(&m->dev, db));
    s->nmir++;
    s->mir_bytes += db;
    mirror_upload(s, m, st);
    return m->dev;
}

static const void *mirror(DevState *s, const void *host, size_t bytes)
{
    return mirror_kind(s, host, bytes, MIR_ROWMAJOR, 0, 0, NULL);
}

static const void *mirror_tiled(DevState *s, const void *host, int rows, int cols,
                                hipStream_t st)
{
    return mirror_kind(s, host, (size_t)rows * cols * 2, MIR_TILED_BF16, rows, cols, st);
}

/* The fingerprints of the mirrors this call uses, checked while its kernels run: on a
 * change the stream is drained (the kernels read the old bytes) and the changed mirrors
 * are uploaded again. Returns how many were; the caller then runs its work again. */
static int verify_mirrors(DevState *s, hipStream_t st)
{
    int n = 0;
    for (int i = 0; i < s->nmir; i++) {
        Mirror *m = &s->mir[i];
        if (m->used != s->calls) continue;
        const uint64_t fp = fingerprint(m->host, m->bytes);
        if (fp == m->print) continue;
        if (!n) K3G_CHECK(hipStreamSynchronize(st));
        m->print = fp;
        mirror_upload(s, m, st);
        n++;
    }
    return n;
}

static void *stage(DevState *s, size_t bytes)
{
    if (bytes > s->stage_bytes) {
        if (s->stage) {
            K3G_CHECK(hipDeviceSynchronize());
            K3G_CHECK(hipFree(s->stage));
        }
        s->stage = NULL;
        const size_t nb = bytes + bytes / 4;
        K3G_CHECK(hipMalloc(&s->stage, nb));
        s->stage_bytes = nb;
    }
    return s->stage;
}

/* A decode call on the flags' path returns while its launch's last waves still retire:
 * before the process ends it waits for every stream the drop-in used. Registered at the
 * first such call, after the HIP runtime has set itself up, so it runs before the
 * runtime's own exit work. Takes no lock: a fatal error exits with the lock held. */
static void drain_at_exit(void)
{
    for (int d = 0; d < K3_MAX_DEV; d++)
        if (g_dev[d].used && g_dev[d].ctx) {
            hipSetDevice(d);
            hipStreamSynchronize(g_dev[d].ctx->stream);
        }
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
        s->mir_bytes = 0;
        if (s->mstage) hipFree(s->mstage);
        s->mstage = NULL;
        s->mstage_bytes = 0;
    }
    hipSetDevice(cur);
    pthread_mutex_unlock(&g_lock);
}

void k3moe_invalidate_weights(const void *host, size_t bytes)
{
    if (!host || !bytes) return;
    const uintptr_t a = (uintptr_t)host, b = a + bytes;
    pthread_mutex_lock(&g_lock);
    int cur = 0;
    hipGetDevice(&cur);
    for (int d = 0; d < K3_MAX_DEV; d++) {
        DevState *s = &g_dev[d];
        if (!s->used) continue;
        hipSetDevice(d);
        for (int i = 0; i < s->nmir;) {
            const uintptr_t ma = (uintptr_t)s->mir[i].host, mb = ma + s->mir[i].bytes;
            if (ma < b && a < mb) mirror_drop(s, i);
            else i++;
        }
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
    s->calls++;
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
/* bytes of a rows x in weight matrix tagged wdt (include/k3/k3.h:299-303: per-row int8
 * draft rows are an f32 scale then `in` int8 weights) */
static size_t mat_bytes(int wdt, int rows, int in)
{
    const size_t row = wdt == K3_WI8 ? (size_t)4 + (size_t)in
                                     : (size_t)in * (wdt == K3_WBF16 ? 2u : 4u);
    return (size_t)rows * row;
}

/* How a fetched expert reaches the kernels. */
enum {
    F_DIRECT = 0,      /* device pointers in the layout the kernels read */
    F_DEV_TILE,        /* device pointers in the checkpoint layout, tiled into a slot */
    F_HOST_STAGE,      /* host pointers, copied into a checkpoint-layout slot */
    F_HOST_TILE        /* host pointers, copied to a ring buffer and tiled into a slot */
};

typedef struct {
    const K3MoeW *w;
    int I, L, how;
    K3gExpertLayout geo;
    size_t t13, t2, slot_bytes;  /* tiled matrix sizes; bytes per staging slot */
    unsigned char *slots;        /* staging slots */
    unsigned char *ring[2];      /* checkpoint-layout buffers for F_HOST_TILE */
    int nring;
    int nslot, maxslot;
    int *slot_of;                /* [E] */
    K3ExpertQ *table;            /* [E] the pointers the kernels read */
    unsigned char *have;         /* [E] expert resolved in this call */
    K3gCache *hc;
    hipStream_t st;
} Fetcher;

/* Tile one checkpoint-layout expert (device pointers) into tiled slot memory. */
static K3ExpertQ tile_expert(Fetcher *f, const K3ExpertQ *q, unsigned char *dst)
{
    K3ExpertQ d;
    memset(&d, 0, sizeof d);
    if (k3k_tile_mxfp4(dst, q->p1, q->s1, f->I, f->L, f->st) != 0 ||
        k3k_tile_mxfp4(dst + f->t13, q->p3, q->s3, f->I, f->L, f->st) != 0 ||
        k3k_tile_mxfp4(dst + 2 * f->t13, q->p2, q->s2, f->L, f->I, f->st) != 0)
        k3g_fatal("k3_moe: tiling an expert failed");
    d.p1 = dst;
    d.p3 = dst + f->t13;
    d.p2 = dst + 2 * f->t13;
    return d;
}

/* Copy one host-resident expert to the device in the checkpoint layout at `base`. */
static K3ExpertQ upload_expert(Fetcher *f, const K3ExpertQ *q, unsigned char *base)
{
    const K3gExpertLayout *g = &f->geo;
    const int I = f->I, L = f->L;
    const size_t p13 = (size_t)I * (L / 2), s13 = (size_t)I * ((L + 31) / 32);
    const size_t p2 = (size_t)L * (I / 2), s2 = (size_t)L * ((I + 31) / 32);
    hipStream_t st = f->st;
    K3G_CHECK(hipMemcpyAsync(base + g->p1_off, q->p1, p13, hipMemcpyHostToDevice, st));
    K3G_CHECK(hipMemcpyAsync(base + g->s1_off, q->s1, s13, hipMemcpyHostToDevice, st));
    K3G_CHECK(hipMemcpyAsync(base + g->p2_off, q->p2, p2, hipMemcpyHostToDevice, st));
    K3G_CHECK(hipMemcpyAsync(base + g->s2_off, q->s2, s2, hipMemcpyHostToDevice, st));
    K3G_CHECK(hipMemcpyAsync(base + g->p3_off, q->p3, p13, hipMemcpyHostToDevice, st));
    K3G_CHECK(hipMemcpyAsync(base + g->s3_off, q->s3, s13, hipMemcpyHostToDevice, st));
    /* the source may evict these bytes at its next get(); finish the copy first */
    K3G_CHECK(hipStreamSynchronize(st));
    K3ExpertQ d;
    d.p1 = base + g->p1_off; d.s1 = base + g->s1_off;
    d.p2 = base + g->p2_off; d.s2 = base + g->s2_off;
    d.p3 = base + g->p3_off; d.s3 = base + g->s3_off;
    return d;
}

/* get() one expert and resolve it to device pointers. Returns 0, or -1 on a miss. */
static int fetch_one(Fetcher *f, int e, int resident_only)
{
    K3ExpertQ q;
    const K3MoeW *w = f->w;
    const int miss = resident_only ? !w->src->resident(w->src, w->layer, e, &q)
                                   : (w->src->get(w->src, w->layer, e, &q) != 0);
    if (miss) return -1;
    if (f->how == F_DIRECT) {
        f->table[e] = q;
    } else if (!f->have[e]) {
        if (f->nslot >= f->maxslot) k3g_fatal("expert staging overflow");
        const int sl = f->nslot++;
        f->slot_of[e] = sl;
        unsigned char *slot = f->slots + (size_t)sl * f->slot_bytes;
        if (f->how == F_HOST_STAGE) {
            f->table[e] = upload_expert(f, &q, slot);
        } else if (f->how == F_HOST_TILE) {
            /* two ring buffers alternate: the copy into one waits (stream order) for the
             * tiling that read it two experts ago */
            const K3ExpertQ d = upload_expert(f, &q, f->ring[f->nring++ & 1]);
            f->table[e] = tile_expert(f, &d, slot);
        } else {
            /* the cache's copy of this expert may still be in flight */
            k3gc_wait(f->hc, f->st);
            f->table[e] = tile_expert(f, &q, slot);
        }
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

/* The engine's fetch calls for tokens [t0, t1) (per-token pattern) or for whole 64-token
 * prefill chunks starting at t0 (mode 1). Routing entries of dropped experts become -1. */
static void fetch_tokens(Fetcher *f, DevState *s, int *ridx, int k, int E, int t0, int t1,
                         int batched, int cache_only)
{
    const K3MoeW *w = f->w;
    if (!batched) {
        /* src/core/k3_ops.c:604-627 */
        for (int t = t0; t < t1; t++) {
            int *it = ridx + (size_t)t * k;
            int ids[K3_MAX_TOPK], nk = 0;
            for (int j = 0; j < k; j++) if (it[j] >= 0) ids[nk++] = it[j];
            if (!cache_only && w->src->getmany) w->src->getmany(w->src, w->layer, ids, nk);
            for (int j = 0; j < k; j++) {
                if (it[j] < 0) continue;
                if (fetch_one(f, it[j], cache_only) != 0) {
                    if (!cache_only) drop_msg(w->layer, it[j], "token");
                    it[j] = -1;
                }
            }
        }
        return;
    }
    /* src/core/k3_ops.c:707-766: 64-token chunks, unique experts in first-seen order,
     * one get() each; the chunks are the engine's [64 m, 64 m + 64) whatever token a
     * group starts at (a group that began inside a chunk the cache could not hold at
     * once ends at its boundary) */
    for (int c0 = t0, c1; c0 < t1; c0 = c1) {
        c1 = (c0 / 64 + 1) * 64 < t1 ? (c0 / 64 + 1) * 64 : t1;
        const int n = c1 - c0;
        if (n == 1) {
            /* a one-token chunk takes k3_moe's per-slot path (:709-710) */
            fetch_tokens(f, s, ridx, k, E, c0, c0 + 1, 0, 0);
            continue;
        }
        memset(s->seen, 0, (size_t)E);
        int nu = 0;
        for (int t = c0; t < c0 + n; t++)
            for (int j = 0; j < k; j++) {
                const int e = ridx[(size_t)t * k + j];
                if (e >= 0 && e < E && !s->seen[e]) { s->seen[e] = 1; s->uniq[nu++] = e; }
            }
        if (w->src->getmany) w->src->getmany(w->src, w->layer, s->uniq, nu);
        for (int u = 0; u < nu; u++) {
            if (fetch_one(f, s->uniq[u], 0) == 0) continue;
            drop_msg(w->layer, s->uniq[u], "chunk");
            for (int t = c0; t < c0 + n; t++)
                for (int j = 0; j < k; j++)
                    if (ridx[(size_t)t * k + j] == s->uniq[u]) ridx[(size_t)t * k + j] = -1;
        }
    }
}

/* Tentatively add the experts of tokens [t0, t1) to the set in seen[] (1: in the group,
 * 2: tentative); returns how many are new. */
static int add_tokens(unsigned char *seen, const int *ridx, int k, int E, int t0, int t1)
{
    int n = 0;
    for (size_t p = (size_t)t0 * k; p < (size_t)t1 * k; p++) {
        const int e = ridx[p];
        if (e >= 0 && e < E && !seen[e]) { seen[e] = 2; n++; }
    }
    return n;
}

static void settle_tokens(unsigned char *seen, const int *ridx, int k, int E, int t0, int t1,
                          int keep)
{
    for (size_t p = (size_t)t0 * k; p < (size_t)t1 * k; p++) {
        const int e = ridx[p];
        if (e >= 0 && e < E && seen[e] == 2) seen[e] = keep ? 1 : 0;
    }
}

/* The engine's getmany/get calls for a layer that ran with every expert resident: all
 * hits, in the engine's order, with the cache's counters and clock as when fetching
 * first. */
static void fetch_resident(Fetcher *f, DevState *s, K3gCache *hc, int *ridx, int k, int E,
                           int T, int mode, hipStream_t st)
{
    f->table = s->table;
    f->have = s->have;
    const long d0 = k3_expert_drops;
    k3gc_step_begin(hc);
    fetch_tokens(f, s, ridx, k, E, 0, T, mode == 1 && T > 1, 0);
    k3gc_step_end(hc, st);
    if (k3_expert_drops != d0) k3g_fatal("k3_moe: a resident expert was not served");
}

/* The end of the next token group from t0: whole units (one token, or a 64-token prefill
 * chunk, the engine's [64 m, 64 m + 64)) while the group's distinct experts fit in cap
 * slots; a unit that alone exceeds cap is split into tokens (at least one: the cache
 * holds top-k + 1 slots), and the group after a split ends at the chunk's boundary, so
 * later chunks keep the engine's alignment. */
static int next_group(DevState *s, const int *ridx, int k, int E, int T, int t0, int unit,
                      int cap)
{
    unsigned char *seen = s->seen;
    memset(seen, 0, (size_t)E);
    int n = 0, t1 = t0;
    while (t1 < T) {
        const int ue = (t1 / unit + 1) * unit;
        const int u1 = ue < T ? ue : T;
        const int add = add_tokens(seen, ridx, k, E, t1, u1);
        const int fits = n + add <= cap;
        settle_tokens(seen, ridx, k, E, t1, u1, fits);
        if (fits) { n += add; t1 = u1; continue; }
        if (t1 > t0) break;
        /* the first unit alone is too wide: as many of its tokens as fit */
        int t = t0;
        while (t < u1) {
            const int a = add_tokens(seen, ridx, k, E, t, t + 1);
            const int ok = n + a <= cap || t == t0;
            settle_tokens(seen, ridx, k, E, t, t + 1, ok);
            if (!ok) break;
            n += a;
            t++;
        }
        return t;
    }
    return t1 > t0 ? t1 : t0 + 1;
}

/* The fast path: bf16 shared/latent weights (tiled mirrors) and MXFP4 experts from a
 * source in the tiled layout, on the matrix-core kernels. */
static int fast_layer(const K3MoeW *w, const K3Cfg *c, int L, int SI)
{
    static int staged = -1;
    if (staged < 0) staged = getenv("K3MOE_DROPIN_STAGED") ? 1 : 0;
    const int d = c->hidden, I = c->moe_inter;
    if (staged || !w->src || d % 32 || I % 32 || L % 32) return 0;
    if ((SI > 0 || w->down || w->up) && w->wdt != K3_WBF16) return 0;
    if (SI % 32) return 0;
    return k3k_tiled_mxfp4_bytes(I, L) > 0 && k3k_tiled_mxfp4_bytes(L, I) > 0;
}

/* mode 0: k3_moe semantics; mode 1: k3_moe_prefill semantics. */
static void moe_run(float *out, const float *x, const K3MoeW *w, const K3Cfg *c, int T,
                    int *idx_out, float *wt_out, int mode)
{
    if (T <= 0) return;
    if (c->topk < 1 || c->topk > K3_MAX_TOPK) k3g_fatal("k3_moe: topk outside 1..64");
    if (w->wdt != K3_WF32 && w->wdt != K3_WBF16 && w->wdt != K3_WI8)
        k3g_fatal("k3_moe: unknown weight type (wdt)");
    const int d = c->hidden, E = c->n_experts, k = c->topk, I = c->moe_inter;
    const int L = w->down ? c->latent : d;
    const int SI = c->moe_inter * c->n_shared;
    if (!w->down && c->latent != d && c->latent != 0)
        k3g_fatal("k3_moe: down == NULL (no latent) needs latent == hidden");
    if (mode == 1) {
        /* src/core/k3_ops.c:692-695: one binary gives both token streams for an A/B */
        static int no_batch = -1;
        if (no_batch < 0) no_batch = getenv("K3_NO_BATCH_PREFILL") ? 1 : 0;
        if (no_batch) mode = 0;
    }

    pthread_mutex_lock(&g_lock);
    DevState *s = dev_state();
    s->calls++;
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
    const int device_src = w->src ? k3gc_is_device_src(w->src) : 0;
    K3gCache *hc = device_src ? k3gc_of_src(w->src) : NULL;
    const int fast = fast_layer(w, c, L, SI);
    if (hc && (hc->bank->hidden != L || hc->bank->inter != I || hc->n_experts < E))
        k3g_fatal("k3_moe: the HBM cache's bank does not hold this layer's expert shape");
    if (hc && hc->bank->layout == K3G_EXPERT_MXFP4_TILED && !fast)
        k3g_fatal("k3_moe: experts in the tiled layout need bf16 shared and latent weights "
                  "(widths multiples of 32)");
    /* sizes first (the context may be recreated), then the mirrors on its stream */
    K3gCtx *ctx = ctx_for(s, &G, T);
    hipStream_t st = ctx->stream;
    const int cache_only = w->cache_only && w->src && w->src->resident;
    /* Every expert of the layer in the HBM cache: the whole layer runs at once (below);
     * the mirrors' fingerprints are then checked while it runs */
    const int resident = hc && fast && hc->bank->layout == K3G_EXPERT_MXFP4_TILED &&
                         !cache_only && k3gc_layer_all_resident(hc, w->layer);
    s->defer = resident;
    G.gate = (const float *)mirror(s, w->gate, (size_t)E * d * 4);
    G.bias = (const float *)mirror(s, w->bias, w->bias ? (size_t)E * 4 : 0);
    G.latent_norm = c->latent_norm ? (const float *)mirror(s, w->latent_norm, (size_t)L * 4)
                                   : NULL;
    if (fast) {
        G.shared_fmt = 1;
        G.expert_fmt = K3G_EXPERT_MXFP4_TILED;
        if (w->down) G.down = mirror_tiled(s, w->down, L, d, st);
        if (w->up) G.up = mirror_tiled(s, w->up, d, L, st);
        if (SI > 0) {
            G.sh1 = mirror_tiled(s, w->sh1, SI, d, st);
            G.sh3 = mirror_tiled(s, w->sh3, SI, d, st);
            G.sh2 = mirror_tiled(s, w->sh2, d, SI, st);
        }
    } else {
        G.down = mirror(s, w->down, w->down ? mat_bytes(w->wdt, L, d) : 0);
        G.up = mirror(s, w->up, w->up ? mat_bytes(w->wdt, d, L) : 0);
        if (SI > 0) {
            G.sh1 = mirror(s, w->sh1, mat_bytes(w->wdt, SI, d));
            G.sh3 = mirror(s, w->sh3, mat_bytes(w->wdt, SI, d));
            G.sh2 = mirror(s, w->sh2, mat_bytes(w->wdt, d, SI));
        }
        if (!w->src) {
            G.expert_fmt = 1;
            G.w1 = (const float *)mirror(s, w->w1, (size_t)E * I * L * 4);
            G.w3 = (const float *)mirror(s, w->w3, (size_t)E * I * L * 4);
            G.w2 = (const float *)mirror(s, w->w2, (size_t)E * L * I * 4);
        }
    }
    s->defer = 0;

    /* how fetched experts reach the kernels, and the staging this call needs */
    Fetcher f;
    memset(&f, 0, sizeof f);
    f.w = w;
    f.I = I;
    f.L = L;
    f.st = st;
    f.hc = hc;
    f.geo = k3g_expert_layout(L, I);
    f.t13 = fast ? k3k_tiled_mxfp4_bytes(I, L) : 0;
    f.t2 = fast ? k3k_tiled_mxfp4_bytes(L, I) : 0;
    if (!w->src) f.how = F_DIRECT;
    else if (hc) f.how = (fast && hc->bank->layout != K3G_EXPERT_MXFP4_TILED) ? F_DEV_TILE : F_DIRECT;
    else f.how = fast ? F_HOST_TILE : F_HOST_STAGE;
    const size_t geo_b = ((size_t)f.geo.nbytes + 255) & ~(size_t)255;
    f.slot_bytes = fast ? ((2 * f.t13 + f.t2 + 255) & ~(size_t)255) : geo_b;
    const int pairs = T * k < E ? T * k : E;
    f.maxslot = f.how == F_DIRECT ? 0 : pairs;
    const size_t xb = ((size_t)T * d * 4 + 255) & ~(size_t)255;
    const size_t nring = f.how == F_HOST_TILE ? 2 : 0;
    unsigned char *sb = (unsigned char *)stage(
        s, xb + nring * geo_b + (size_t)f.maxslot * f.slot_bytes);
    float *xd = (float *)sb;
    f.ring[0] = sb + xb;
    f.ring[1] = sb + xb + geo_b;
    f.slots = sb + xb + nring * geo_b;

    /* The call's device I/O area and its pinned twin, one transfer each way:
     * [error word | idx [T][k] | wt [T][k] | out [T][d]], x after it on the host side.
     * The context reports device errors into the area's first word. */
    const size_t xbytes = (size_t)T * d * 4, pbytes = (size_t)T * k * 4;
    const size_t o_idx = 256, o_wt = o_idx + ((pbytes + 255) & ~(size_t)255);
    const size_t o_out = o_wt + ((pbytes + 255) & ~(size_t)255), io_n = o_out + xbytes;
    unsigned char *io = io_area(s, io_n);
    unsigned char *pin = pinned(s, io_n + xbytes);
    ctx->err = (int *)io;
    int32_t *didx = (int32_t *)(io + o_idx);
    float *dwt = (float *)(io + o_wt), *od = (float *)(io + o_out);
    int *perr = (int *)pin, *ridx = (int *)(pin + o_idx);
    float *rwt = (float *)(pin + o_wt), *pout = (float *)(pin + o_out);
    float *px = (float *)(pin + io_n);
    host_copy(px, x, xbytes);
    ctx->paths = 0;
    host_scratch(s, (size_t)T * k, E);
    int last[K3_MAX_TOPK];
    float lastw[K3_MAX_TOPK];

    /* Every expert of the layer in the HBM cache: the whole layer runs at once against
     * the cache's device expert table (the fused decode kernel routes inside), and the
     * engine's getmany/get calls follow on the host in the engine's order, all hits: the
     * same results and the same cache state and accounting as fetching first. A weight
     * buffer found changed while the layer ran is uploaded again and the layer rerun. */
    if (resident) {
        k3gc_wait(hc, st);
        G.experts = k3gc_layer_table(hc, w->layer, st);
        if (!G.experts) k3g_fatal("k3_moe: expert table update failed");
        /* One fused decode launch writes out, the routing, a nonzero error code and two
         * flags straight into the pinned twin (no transfer back): the engine's get calls
         * go out as soon as the routing is there, while the layer still runs, and the
         * call returns once the outputs are (work queued on the stream later still
         * waits for the launch's last waves). Without the flags (a rerun, a launch cut
         * short by an error) the stream is waited for. */
        const int direct = k3g_fuses(ctx, &G, T);
        volatile int *flag = (volatile int *)(pin + 128);
        static int drain_registered = 0;
        if (direct && !drain_registered) drain_registered = atexit(drain_at_exit) == 0;
        if (direct) {
            *perr = 0;
            flag[K3K_HFLAG_ROUTED] = 0;
            flag[K3K_HFLAG_DONE] = 0;
            ctx->host_idx = ridx;
            ctx->host_wt = rwt;
            ctx->host_err = perr;
            ctx->host_flag = (int *)flag;
        }
        /* x goes in right before the layer, so the two launches reach the GPU back to
         * back (host work between them would leave it idle) */
        xfer(xd, px, xbytes, hipMemcpyHostToDevice, st);
        int reran = 0;
        for (int pass = 0;; pass++) {
            if (k3g_moe(ctx, &G, xd, T, direct ? pout : od, didx, dwt, st) != 0)
                k3g_fatal("k3_moe: launch failed");
            if (!direct) xfer(pin, io, io_n, hipMemcpyDeviceToHost, st);
            reran = pass > 0;
            if (pass > 0 || !verify_mirrors(s, st)) break;
        }
        ctx->host_idx = NULL;
        ctx->host_wt = NULL;
        ctx->host_err = NULL;
        ctx->host_flag = NULL;
        const int early = direct && !reran && k3g_await_flag(&flag[K3K_HFLAG_ROUTED], 0.1);
        if (early) fetch_resident(&f, s, hc, ridx, k, E, T, mode, st);
        int e = *perr;
        if (!early || !k3g_await_flag(&flag[K3K_HFLAG_DONE], 0.1)) {
            K3G_CHECK(hipStreamSynchronize(st));
            /* the error word came back with the copy, or with the outputs' flag of a
             * single launch; else it is read */
            if (direct && (reran || !flag[K3K_HFLAG_DONE])) e = k3g_err_read(ctx);
            else e = *perr;
        }
        if (k3g_err_settle(ctx, e) != 0) k3g_fatal("k3_moe: device error");
        if (!early) fetch_resident(&f, s, hc, ridx, k, E, T, mode, st);
        host_copy(out, pout, xbytes);
        g_last_paths = ctx->paths;
        const int batched = mode == 1 && T > 1;
        if (!batched || (T - 1) % 64 == 0) {
            memcpy(idx_out, ridx + (size_t)(T - 1) * k, (size_t)k * sizeof(int));
            memcpy(wt_out, rwt + (size_t)(T - 1) * k, (size_t)k * sizeof(float));
        }
        pthread_mutex_unlock(&g_lock);
        return;
    }

    xfer(xd, px, xbytes, hipMemcpyHostToDevice, st);
    if (k3g_route(ctx, &G, xd, T, didx, dwt, st) != 0) k3g_fatal("k3_moe: router launch");
    xfer(pin, io, o_out, hipMemcpyDeviceToHost, st);
    K3G_CHECK(hipStreamSynchronize(st));
    if (k3g_err_settle(ctx, *perr) != 0) k3g_fatal("k3_moe: device error in the router");
    memcpy(last, ridx + (size_t)(T - 1) * k, (size_t)k * sizeof(int));
    memcpy(lastw, rwt + (size_t)(T - 1) * k, (size_t)k * sizeof(float));

    /* the device keeps the router's idx/wt; they travel again only where the host
     * changed them (drops, the cache-only filter) */
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

    if (!w->src) {
        if (k3g_experts(ctx, &G, xd, T, didx, dwt, od, st) != 0)
            k3g_fatal("k3_moe: launch failed");
    } else {
        f.slot_of = s->slot_of;
        f.table = s->table;
        f.have = s->have;
        memset(f.have, 0, (size_t)E);
        if (s->cap_e < E) {
            if (s->eq_dev) {
                K3G_CHECK(hipDeviceSynchronize());
                K3G_CHECK(hipFree(s->eq_dev));
            }
            K3G_CHECK(hipMalloc((void **)&s->eq_dev, (size_t)E * sizeof(K3ExpertQ)));
            s->cap_e = E;
        }
        G.experts = s->eq_dev;
        const long drops0 = k3_expert_drops;
        const int batched = mode == 1 && T > 1 && !cache_only;
        /* every slot a group fetches stays put until the group's kernels are done: a
         * group's experts must fit the cache's unpinned slots together */
        int cap = E;
        if (hc) {
            int npinned = 0;
            for (int i = 0; i < hc->nslot; i++) npinned += hc->pinned[i] != 0;
            cap = hc->nslot - npinned;
            if (cap < 1) k3g_fatal("k3_moe: every slot of the HBM cache is pinned");
        }
        for (int t0 = 0; t0 < T;) {
            const int t1 = hc ? next_group(s, ridx, k, E, T, t0, batched ? 64 : 1, cap) : T;
            if (hc) k3gc_step_begin(hc);
            fetch_tokens(&f, s, ridx, k, E, t0, t1, batched, cache_only);
            /* the group's experts into the device table, as kernel arguments */
            K3kEqSet set;
            memset(&set, 0, sizeof set);
            memset(s->seen, 0, (size_t)E);
            for (size_t p = (size_t)t0 * k; p < (size_t)t1 * k; p++) {
                const int e = ridx[p];
                if (e < 0 || e >= E || s->seen[e]) continue;
                s->seen[e] = 1;
                set.e[set.n] = e;
                set.q[set.n] = f.table[e];
                if (++set.n == K3K_EQSET) {
                    if (k3k_set_experts(s->eq_dev, &set, st) != 0)
                        k3g_fatal("k3_moe: expert table update failed");
                    set.n = 0;
                }
            }
            if (set.n && k3k_set_experts(s->eq_dev, &set, st) != 0)
                k3g_fatal("k3_moe: expert table update failed");
            const size_t pk = (size_t)t0 * k, np = (size_t)(t1 - t0) * k;
            if (cache_only || drops0 != k3_expert_drops) {
                xfer(didx + pk, ridx + pk, np * 4, hipMemcpyHostToDevice, st);
                xfer(dwt + pk, rwt + pk, np * 4, hipMemcpyHostToDevice, st);
            }
            /* the misses copy on the cache's stream: the routed experts wait for them
             * (the shared expert does not) */
            if (hc && hc->copies_pending) {
                k3g_ctx_routed_wait(ctx, hc->last_copy);
                hc->copies_pending = 0;
            }
            if (k3g_experts(ctx, &G, xd + (size_t)t0 * d, t1 - t0, didx + pk, dwt + pk,
                            od + (size_t)t0 * d, st) != 0)
                k3g_fatal("k3_moe: launch failed");
            if (hc) k3gc_step_end(hc, st);
            /* the pinned routing of this group travels before the next group edits it */
            if (t1 < T) K3G_CHECK(hipStreamSynchronize(st));
            t0 = t1;
        }
    }
    xfer(pout, od, xbytes, hipMemcpyDeviceToHost, st);
    xfer(perr, io, 4, hipMemcpyDeviceToHost, st);
    K3G_CHECK(hipStreamSynchronize(st));
    if (k3g_err_settle(ctx, *perr) != 0) k3g_fatal("k3_moe: device error");
    host_copy(out, pout, xbytes);
    g_last_paths = ctx->paths;

    /* idx/wt hold the last token's routing when the engine's per-token path produced
     * it; the batched prefill path leaves them untouched (src/core/k3_ops.c:699-714).
     * After a cache-only filter the resident subset is compacted to the front and the
     * rest keeps the router's values, as in the engine. */
    const int batched = mode == 1 && w->src && T > 1 && !cache_only;
    if (!batched || (T - 1) % 64 == 0) {
        memcpy(idx_out, last, (size_t)k * sizeof(int));
        memcpy(wt_out, lastw, (size_t)k * sizeof(float));
    }
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
    if (group < 1) {
        /* the engine divides by it (src/core/k3_ops.c:1387) */
        fprintf(stderr, "k3moe: FATAL, k3_matmul_mxfp4 called with group=%d.\n", group);
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
    const size_t pb = (size_t)rows * (in / 2), sb = (size_t)rows * ((in + group - 1) / group);
    const size_t xb = (size_t)in * 4, yb = (size_t)rows * 4;
    const size_t a0 = 0, a1 = (pb + 255) & ~(size_t)255, a2 = a1 + ((sb + 255) & ~(size_t)255);
    const size_t a3 = a2 + ((xb + 255) & ~(size_t)255);
    unsigned char *b = (unsigned char *)stage(s, a3 + yb);
    K3G_CHECK(hipMemcpyAsync(b + a0, packed, pb, hipMemcpyHostToDevice, c->stream));
    K3G_CHECK(hipMemcpyAsync(b + a1, scales, sb, hipMemcpyHostToDevice, c->stream));
    K3G_CHECK(hipMemcpyAsync(b + a2, x, xb, hipMemcpyHostToDevice, c->stream));
    if (k3k_mxfp4_gemv((float *)(b + a3), (const float *)(b + a2), b + a0, b + a1, in, rows,
                       group, c->stream) != 0)
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
