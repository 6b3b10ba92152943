/* k3_cache_dropin.c - the engine's expert cache entry points (src/cache/k3_cache.h:97-118)
 * with the engine's K3Cache layout, on the HBM expert cache (C99).
 *
 * The engine's main() builds its cache with k3_cache_init(&cache, &st, &cfg, budget), reads
 * cache.nslot / cache.slot_bytes / the hit and read counters directly, hands &cache.src to
 * every MoE layer and reports with k3_cache_report (src/cli/k3_run.c:1144-1155, :582-590,
 * :1524-1534, :1608). Those call sites link against this file unchanged. Inside, a K3Cache
 * wraps a k3gc cache over a checkpoint bank: the misses are read from the engine's own
 * index (the K3St its k3_st_open filled) into pinned staging and copied into HBM slots,
 * and get() hands out device pointers that this library's k3_moe runs on in place. The
 * policy, the counters and the request trace are the HBM cache's, which follow the
 * engine's (src/cache/k3_cache.c:49-260); this file keeps the K3Cache fields in step with
 * them after every call. */
#include "k3gc_cache.h"
#include "k3g_ctx.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    K3gCache *inner;
    K3gcBank *bank;
    K3gcSt *st;
} KcPriv;

static KcPriv *kc_priv(const K3Cache *c) { return (KcPriv *)c->src.ctx; }

static int kc_get(K3ExpertSrc *self, int layer, int expert, K3ExpertQ *out);

K3gCache *k3_cache_inner_of(const K3ExpertSrc *src)
{
    if (!src || src->get != kc_get || !src->ctx) return NULL;
    return ((KcPriv *)src->ctx)->inner;
}

/* the engine-visible fields from the HBM cache's state */
static void kc_sync(K3Cache *c)
{
    const K3gCache *h = kc_priv(c)->inner;
    c->clock = h->clock;
    c->hits = h->hits;
    c->misses = h->misses;
    c->evictions = h->evictions;
    c->bytes_read = h->bytes_read;
    c->prefetch_reads = h->prefetch_reads;
    c->load_seconds = h->disk_seconds;
    c->trace = h->trace;
    c->ntrace = h->ntrace;
    c->captrace = h->captrace;
}

/* ref[slot]: the checkpoint geometry of the expert the slot now holds */
static void kc_note(K3Cache *c, int layer, int expert)
{
    const K3gCache *h = kc_priv(c)->inner;
    if (layer < 0 || layer >= h->n_layers || expert < 0 || expert >= h->n_experts) return;
    const int slot = h->slot_of[layer * h->n_experts + expert];
    if (slot < 0 || (c->ref[slot].nbytes > 0 && c->ref[slot].layer == layer &&
                         c->ref[slot].expert == expert))
        return;
    K3gcExpertRun r;
    K3ExpertRef *f = &c->ref[slot];
    memset(f, 0, sizeof *f);
    if (k3gc_st_expert(kc_priv(c)->st, layer, expert, &r) != 0) return;
    f->layer = layer;
    f->expert = expert;
    f->shard = r.shard;
    f->off = r.off;
    f->nbytes = r.nbytes;
    f->contiguous = r.contiguous;
    int64_t at = 0;
    for (int i = 0; i < 3; i++) {
        f->m[i].p_off = at;
        f->m[i].p_bytes = r.p_bytes[i];
        at += r.p_bytes[i];
        f->m[i].s_off = at;
        f->m[i].s_bytes = r.s_bytes[i];
        at += r.s_bytes[i];
        f->m[i].rows = r.rows[i];
        f->m[i].pcols = r.pcols[i];
        f->m[i].scols = r.pcols[i] * 2 / 32;
    }
}

static int kc_get(K3ExpertSrc *self, int layer, int expert, K3ExpertQ *out)
{
    K3Cache *c = (K3Cache *)self;            /* src is the first member */
    K3gCache *h = kc_priv(c)->inner;
    const int rc = h->src.get(&h->src, layer, expert, out);
    if (rc == 0) kc_note(c, layer, expert);
    kc_sync(c);
    return rc;
}

static int kc_getmany(K3ExpertSrc *self, int layer, const int *experts, int n)
{
    K3Cache *c = (K3Cache *)self;
    K3gCache *h = kc_priv(c)->inner;
    const int rc = h->src.getmany ? h->src.getmany(&h->src, layer, experts, n) : 0;
    for (int i = 0; i < n; i++) kc_note(c, layer, experts[i]);
    kc_sync(c);
    return rc;
}

static int kc_resident(K3ExpertSrc *self, int layer, int expert, K3ExpertQ *out)
{
    K3Cache *c = (K3Cache *)self;
    K3gCache *h = kc_priv(c)->inner;
    return h->src.resident(&h->src, layer, expert, out);
}

int k3_cache_init(K3Cache *c, const K3St *st, const K3Cfg *cfg, int64_t budget_bytes)
{
    memset(c, 0, sizeof *c);
    if (!st || !cfg || cfg->n_layers < 1 || cfg->n_experts < 1 || cfg->topk < 1) return -1;
    KcPriv *p = (KcPriv *)calloc(1, sizeof *p);
    if (!p) return -1;
    if (k3gc_st_from_engine(&p->st, st) != 0) { free(p); return -1; }
    /* a slot sized from the checkpoint: the first routed expert of the first MoE layer
     * that has one (k3_cache.c:281-289) */
    int probe = -1;
    for (int l = cfg->first_dense > 0 ? cfg->first_dense : 0; l < cfg->n_layers && probe < 0; l++) {
        K3gcExpertRun r;
        if (k3gc_st_expert(p->st, l, 0, &r) == 0) probe = l;
    }
    if (probe < 0) {
        fprintf(stderr, "k3_cache: no routed experts in this shard set\n");
        k3gc_st_close(p->st);
        free(p);
        return -1;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    if (k3gc_bank_create_disk(&p->bank, p->st, cfg->n_layers, cfg->n_experts, probe) != 0 ||
        k3gc_init(&p->inner, dev, p->bank, cfg->topk, budget_bytes) != 0) {
        if (p->bank) k3gc_bank_free(p->bank);
        k3gc_st_close(p->st);
        free(p);
        return -1;
    }
    K3gCache *h = p->inner;
    c->src.get = kc_get;
    c->src.getmany = h->src.getmany ? kc_getmany : NULL;   /* K3_NOPREFETCH, k3_cache.c:268 */
    c->src.resident = kc_resident;
    c->src.ctx = p;
    c->st = st;
    c->n_layers = h->n_layers;
    c->n_experts = h->n_experts;
    c->arena = h->arena;
    c->slot_bytes = h->slot_bytes;
    c->nslot = h->nslot;
    c->slot_of = h->slot_of;
    c->key_of = h->key_of;
    c->used_at = h->used_at;
    c->pinned = h->pinned;
    c->hist = h->hist;
    c->ref = (K3ExpertRef *)calloc((size_t)h->nslot, sizeof(K3ExpertRef));
    c->pad = (int32_t *)calloc((size_t)h->nslot, sizeof(int32_t));
    if (!c->ref || !c->pad) {
        k3_cache_free(c);
        return -1;
    }
    kc_sync(c);
    return 0;
}

void k3_cache_free(K3Cache *c)
{
    if (!c) return;
    KcPriv *p = kc_priv(c);
    if (p && c->src.get == kc_get) {
        k3gc_free(p->inner);
        k3gc_bank_free(p->bank);
        k3gc_st_close(p->st);
        free(p);
    }
    free(c->ref);
    free(c->pad);
    memset(c, 0, sizeof *c);
}

int k3_cache_pin(K3Cache *c, int layer, int expert, int pin)
{
    return k3gc_pin(kc_priv(c)->inner, layer, expert, pin);
}

int k3_cache_prefetch(K3Cache *c, int layer, int expert)
{
    const int rc = k3gc_prefetch(kc_priv(c)->inner, layer, expert);
    if (rc == 0) kc_note(c, layer, expert);
    kc_sync(c);
    return rc;
}

void k3_cache_reset_stats(K3Cache *c)
{
    k3gc_reset_stats(kc_priv(c)->inner);
    kc_sync(c);
}

void k3_cache_report(const K3Cache *c, const char *label)
{
    const K3gCache *h = kc_priv(c)->inner;
    const uint64_t n = h->hits + h->misses;
    int resident = 0, pinned = 0;
    for (int i = 0; i < h->nslot; i++) {
        resident += h->key_of[i] >= 0;
        pinned += h->pinned[i] != 0;
    }
    printf("cache [%s]\n", label ? label : "");
    printf("  slots        : %d of %.2f MB = %.2f GB of HBM (%d resident, %d pinned)\n",
           h->nslot, (double)h->slot_bytes / 1e6, (double)h->nslot * h->slot_bytes / 1e9,
           resident, pinned);
    printf("  requests     : %llu  hits %llu (%.2f%%)  misses %llu  evictions %llu\n",
           (unsigned long long)n, (unsigned long long)h->hits, n ? 100.0 * h->hits / n : 0.0,
           (unsigned long long)h->misses, (unsigned long long)h->evictions);
    if (h->prefetch_reads) {
        const uint64_t served = h->hits > h->prefetch_reads ? h->hits - h->prefetch_reads : 0;
        printf("  of those hits : %llu were read by the batch prefetch this step; true "
               "resident hit rate %.2f%%\n",
               (unsigned long long)h->prefetch_reads, n ? 100.0 * served / n : 0.0);
    }
    printf("  read from disk: %.2f GB in %.2f s (%.0f MB/s while reading)%s\n",
           (double)h->bytes_read / 1e9, h->disk_seconds,
           h->disk_seconds > 0 ? (double)h->bytes_read / 1e6 / h->disk_seconds : 0.0,
           h->failed_reads ? ", some runs could not be read" : "");
}

int k3_cache_dump_hist(const K3Cache *c, const char *path)
{
    return k3gc_dump_hist(kc_priv(c)->inner, path);
}

int k3_cache_dump_trace(const K3Cache *c, const char *path)
{
    return k3gc_dump_trace(kc_priv(c)->inner, path);
}
