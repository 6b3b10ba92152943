/* k3gc_cache.c - the engine's expert cache (src/cache/k3_cache.c) re-planned for HBM.
 *
 * What stays the engine's: the policy and the accounting. Slots hold a key, are EMPTY or
 * are INFLIGHT (reserved by a batch); the victim is the first EMPTY slot, else the least
 * recently used slot that is neither pinned nor INFLIGHT (a linear scan, as in
 * k3_cache.c:49-60); a batch prefetch reserves serially, copies, then publishes
 * (k3_cache.c:131-218); every get() counts a histogram entry and appends (layer, expert)
 * to the trace before it is served (k3_cache.c:235-261); prefetched experts are counted
 * apart so the true hit rate is (hits - prefetch_reads) / requests (k3_cache.c:403-429).
 *
 * What is new for a GPU. The slots are HBM; the backing store is a pinned host bank; a
 * miss is a hipMemcpyAsync on the cache's own copy stream, ordered after the last step
 * that read the victim slot (an event recorded on the compute stream when that step
 * ended), and a consumer makes its stream wait for the copies with one event. A slot
 * handed out in the open step is never a victim, which is the engine's "capacity above
 * top-k" rule (k3_cache.c:304-313) applied to a whole step's working set. */
#include "k3gc_cache.h"
#include "k3g_ctx.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static int has_device(const K3gCache *c) { return c->device >= 0; }

static int64_t run_bytes(int hidden, int inter, int layout)
{
    if (layout == K3G_EXPERT_MXFP4_TILED)
        return 2 * (int64_t)k3k_tiled_mxfp4_bytes(inter, hidden) +
               (int64_t)k3k_tiled_mxfp4_bytes(hidden, inter);
    return k3g_expert_layout(hidden, inter).nbytes;
}

/* ------------------------------------------------------------------ host bank ---- */
int k3gc_bank_create(K3gcBank **out, int n_layers, int n_experts, int hidden, int inter,
                     int layout)
{
    return k3gc_bank_create_ex(out, n_layers, n_experts, hidden, inter, layout, -1);
}

static int bank_alloc(K3gcBank **out, int n_layers, int n_experts, int hidden, int inter,
                      int layout, int64_t eb, int max_pinned_layers);

int k3gc_bank_create_ex(K3gcBank **out, int n_layers, int n_experts, int hidden, int inter,
                        int layout, int max_pinned_layers)
{
    *out = NULL;
    if (n_layers < 1 || n_experts < 1 || hidden < 32 || inter < 32 ||
        (layout != K3G_EXPERT_MXFP4 && layout != K3G_EXPERT_MXFP4_TILED)) {
        fprintf(stderr, "k3gc_bank_create: unsupported shape\n");
        return -1;
    }
    const int64_t eb = run_bytes(hidden, inter, layout);
    if (eb <= 0) {
        fprintf(stderr, "k3gc_bank_create: no tiled layout for hidden %d inter %d\n", hidden,
                inter);
        return -1;
    }
    return bank_alloc(out, n_layers, n_experts, hidden, inter, layout, eb, max_pinned_layers);
}

int k3gc_bank_create_raw(K3gcBank **out, int n_layers, int n_experts, int64_t expert_bytes,
                         int max_pinned_layers)
{
    *out = NULL;
    if (n_layers < 1 || n_experts < 1 || expert_bytes < 1) return -1;
    return bank_alloc(out, n_layers, n_experts, 0, 0, K3G_EXPERT_MXFP4, expert_bytes,
                      max_pinned_layers);
}

static int bank_alloc(K3gcBank **out, int n_layers, int n_experts, int hidden, int inter,
                      int layout, int64_t eb, int max_pinned_layers)
{
    K3gcBank *b = (K3gcBank *)calloc(1, sizeof *b);
    if (!b) return -1;
    b->n_layers = n_layers;
    b->n_experts = n_experts;
    b->hidden = hidden;
    b->inter = inter;
    b->layout = layout;
    b->expert_bytes = eb;
    /* one allocation per layer: pinned while the driver grants it (a machine may cap pinned
     * memory well below the bank's size) and max_pinned_layers allows (< 0: no limit),
     * pageable beyond that. The staging buffers the pageable layers' misses go through
     * are taken first, so the pinned layers cannot use up what they need. */
    const size_t per_layer = (size_t)n_experts * (size_t)eb;
    b->layer_host = (unsigned char **)calloc((size_t)n_layers, sizeof(unsigned char *));
    b->layer_pinned = (unsigned char *)calloc((size_t)n_layers, 1);
    if (!b->layer_host || !b->layer_pinned) { k3gc_bank_free(b); return -1; }
    for (int i = 0; i < K3GC_NSTAGE; i++) {
        void *p = NULL;
        if (hipHostMalloc(&p, (size_t)eb, hipHostMallocDefault) != hipSuccess || !p) {
            (void)hipGetLastError();
            break;
        }
        b->stage[b->nstage++] = (unsigned char *)p;
    }
    int pinned_ok = max_pinned_layers != 0;
    for (int l = 0; l < n_layers; l++) {
        void *p = NULL;
        if (max_pinned_layers >= 0 && b->pinned_layers >= max_pinned_layers) pinned_ok = 0;
        if (pinned_ok && hipHostMalloc(&p, per_layer, hipHostMallocDefault) == hipSuccess && p) {
            b->layer_pinned[l] = 1;
            b->pinned_layers++;
        } else {
            if (pinned_ok) (void)hipGetLastError();   /* clear the refused allocation */
            pinned_ok = 0;
            p = malloc(per_layer);
            if (!p) {
                fprintf(stderr, "k3gc_bank_create: cannot allocate %.2f GB of host memory\n",
                        (double)per_layer * n_layers / 1e9);
                k3gc_bank_free(b);
                return -1;
            }
        }
        b->layer_host[l] = (unsigned char *)p;
    }
    if (b->pinned_layers < n_layers)
        fprintf(stderr, "k3gc_bank_create: %d of %d layers pinned, the rest pageable\n",
                b->pinned_layers, n_layers);
    *out = b;
    return 0;
}

int k3gc_bank_geometry(K3gcBank **out, int n_layers, int n_experts, int64_t expert_bytes)
{
    *out = NULL;
    if (n_layers < 1 || n_experts < 1 || expert_bytes < 1) return -1;
    K3gcBank *b = (K3gcBank *)calloc(1, sizeof *b);
    if (!b) return -1;
    b->n_layers = n_layers;
    b->n_experts = n_experts;
    b->layout = K3G_EXPERT_MXFP4;
    b->expert_bytes = expert_bytes;
    *out = b;
    return 0;
}

/* ------------------------------------------------------------ checkpoint bank ---- */
int k3gc_bank_create_disk(K3gcBank **out, const K3gcSt *st, int n_layers, int n_experts,
                          int probe_layer)
{
    *out = NULL;
    if (!st || n_layers < 1 || n_experts < 1 || probe_layer < 0 || probe_layer >= n_layers)
        return -1;
    K3gcExpertRun r;
    if (k3gc_st_expert(st, probe_layer, 0, &r) != 0) return -1;
    const int inter = r.rows[0], hidden = 2 * r.pcols[0];
    const int shaped = r.rows[2] == inter && r.pcols[2] == r.pcols[0] && r.rows[1] == hidden &&
                       2 * r.pcols[1] == inter;
    const int tiled = shaped && hidden >= 32 && inter >= 32 &&
                      k3k_tiled_mxfp4_bytes(inter, hidden) > 0 &&
                      k3k_tiled_mxfp4_bytes(hidden, inter) > 0;
    K3gcBank *b = (K3gcBank *)calloc(1, sizeof *b);
    if (!b) return -1;
    b->n_layers = n_layers;
    b->n_experts = n_experts;
    b->st = st;
    b->run_bytes = r.nbytes;
    b->layout = tiled ? K3G_EXPERT_MXFP4_TILED : K3G_EXPERT_MXFP4;
    if (tiled) {
        b->hidden = hidden;
        b->inter = inter;
        b->expert_bytes = run_bytes(hidden, inter, K3G_EXPERT_MXFP4_TILED);
    } else {
        /* the run's own layout: its six matrices' offsets, which every run must share */
        int64_t at = 0;
        for (int i = 0; i < 3; i++) {
            b->raw_off[2 * i] = at;
            at += r.p_bytes[i];
            b->raw_off[2 * i + 1] = at;
            at += r.s_bytes[i];
        }
        b->raw_geometry = 1;
        b->expert_bytes = r.nbytes;
    }
    b->stage_cap = ((r.nbytes + 4095) & ~(int64_t)4095) + 2 * 4096;
    for (int i = 0; i < K3GC_NSTAGE; i++) {
        void *p = NULL;
        if (hipHostMalloc(&p, (size_t)b->stage_cap, hipHostMallocDefault) != hipSuccess || !p) {
            (void)hipGetLastError();
            fprintf(stderr, "k3gc_bank_create_disk: cannot pin %.1f MB of staging\n",
                    (double)b->stage_cap / 1e6);
            k3gc_bank_free(b);
            return -1;
        }
        b->stage[b->nstage++] = (unsigned char *)p;
        if (tiled && hipMalloc((void **)&b->dstage[i], (size_t)r.nbytes) != hipSuccess) {
            (void)hipGetLastError();
            b->dstage[i] = NULL;
            k3gc_bank_free(b);
            return -1;
        }
    }
    *out = b;
    return 0;
}

/* A run of a checkpoint bank has the bank's geometry. */
static int disk_run_fits(const K3gcBank *b, const K3gcExpertRun *r)
{
    if (b->layout == K3G_EXPERT_MXFP4_TILED)
        return r->rows[0] == b->inter && 2 * r->pcols[0] == b->hidden && r->rows[2] == b->inter &&
               2 * r->pcols[2] == b->hidden && r->rows[1] == b->hidden &&
               2 * r->pcols[1] == b->inter && r->nbytes == b->run_bytes;
    int64_t at = 0;
    for (int i = 0; i < 3; i++) {
        if (b->raw_off[2 * i] != at) return 0;
        at += r->p_bytes[i];
        if (b->raw_off[2 * i + 1] != at) return 0;
        at += r->s_bytes[i];
    }
    return r->nbytes == b->run_bytes;
}

void k3gc_bank_free(K3gcBank *b)
{
    if (!b) return;
    if (b->layer_host)
        for (int l = 0; l < b->n_layers; l++) {
            if (!b->layer_host[l]) continue;
            if (b->layer_pinned[l]) hipHostFree(b->layer_host[l]);
            else free(b->layer_host[l]);
        }
    for (int i = 0; i < b->nstage; i++) hipHostFree(b->stage[i]);
    for (int i = 0; i < K3GC_NSTAGE; i++)
        if (b->dstage[i]) hipFree(b->dstage[i]);
    free(b->layer_host);
    free(b->layer_pinned);
    free(b);
}

void *k3gc_bank_expert(K3gcBank *b, int layer, int expert)
{
    if (!b || !b->layer_host || layer < 0 || layer >= b->n_layers || expert < 0 ||
        expert >= b->n_experts)
        return NULL;
    return b->layer_host[layer] + (size_t)expert * (size_t)b->expert_bytes;
}

int k3gc_bank_pinned_layers(const K3gcBank *b) { return b ? b->pinned_layers : 0; }

int64_t k3gc_bank_expert_bytes(const K3gcBank *b) { return b ? b->expert_bytes : 0; }

/* ------------------------------------------------------------------- policy ---- */
/* The first EMPTY slot; else the least recently used one that is not INFLIGHT, not
 * pinned and not handed out in the open step. -1 when there is none. */
static int pick_victim(const K3gCache *c)
{
    int best = -1;
    uint64_t oldest = UINT64_MAX;
    for (int i = 0; i < c->nslot; i++) {
        if (c->key_of[i] == K3GC_INFLIGHT) continue;
        if (c->key_of[i] == K3GC_EMPTY) return i;
        if (c->pinned[i]) continue;
        if (c->step_open && c->used_at[i] >= c->step_clock) continue;
        if (c->used_at[i] < oldest) { oldest = c->used_at[i]; best = i; }
    }
    return best;
}

static void fill_q(const K3gCache *c, int slot, K3ExpertQ *q)
{
    const uintptr_t base = (uintptr_t)c->arena + (uintptr_t)slot * (uintptr_t)c->slot_bytes;
    const K3gcBank *b = c->bank;
    memset(q, 0, sizeof *q);
    if (b->layout == K3G_EXPERT_MXFP4_TILED) {
        const uintptr_t t13 = (uintptr_t)k3k_tiled_mxfp4_bytes(b->inter, b->hidden);
        q->p1 = (const unsigned char *)base;
        q->p3 = (const unsigned char *)(base + t13);
        q->p2 = (const unsigned char *)(base + 2 * t13);
    } else if (b->hidden == 0) {
        q->p1 = (const unsigned char *)(base + b->raw_off[0]);
        q->s1 = (const unsigned char *)(base + b->raw_off[1]);
        q->p2 = (const unsigned char *)(base + b->raw_off[2]);
        q->s2 = (const unsigned char *)(base + b->raw_off[3]);
        q->p3 = (const unsigned char *)(base + b->raw_off[4]);
        q->s3 = (const unsigned char *)(base + b->raw_off[5]);
    } else {
        const K3gExpertLayout g = k3g_expert_layout(b->hidden, b->inter);
        q->p1 = (const unsigned char *)(base + g.p1_off);
        q->s1 = (const unsigned char *)(base + g.s1_off);
        q->p2 = (const unsigned char *)(base + g.p2_off);
        q->s2 = (const unsigned char *)(base + g.s2_off);
        q->p3 = (const unsigned char *)(base + g.p3_off);
        q->s3 = (const unsigned char *)(base + g.s3_off);
    }
}

/* slot bookkeeping: a key enters or leaves a slot */
static void key_in(K3gCache *c, int32_t key)
{
    const int layer = key / c->n_experts;
    c->layer_resident[layer]++;
    c->table_dirty[layer] = 1;
}

static void key_out(K3gCache *c, int32_t key)
{
    const int layer = key / c->n_experts;
    c->layer_resident[layer]--;
    c->table_dirty[layer] = 1;
}

/* ------------------------------------------------------------- data movement ---- */
static void harvest_timers(K3gCache *c, int all)
{
    while (c->t_used > 0 && (all || c->t_used == K3GC_TIMER_RING)) {
        const int i = (c->t_head - c->t_used + K3GC_TIMER_RING) % K3GC_TIMER_RING;
        float ms = 0.0f;
        K3G_CHECK(hipEventSynchronize(c->tev[i][1]));
        K3G_CHECK(hipEventElapsedTime(&ms, c->tev[i][0], c->tev[i][1]));
        c->load_seconds += ms * 1e-3;
        c->t_used--;
    }
}

/* Open a timed batch of copies (once per get/getmany/prefetch that copies). */
static void batch_open(K3gCache *c)
{
    if (!has_device(c) || c->t_open) return;
    harvest_timers(c, 0);
    K3G_CHECK(hipEventRecord(c->tev[c->t_head][0], c->copy));
    c->t_open = 1;
}

static void batch_close(K3gCache *c)
{
    if (!has_device(c) || !c->t_open) return;
    K3G_CHECK(hipEventRecord(c->tev[c->t_head][1], c->copy));
    c->t_head = (c->t_head + 1) % K3GC_TIMER_RING;
    c->t_used++;
    c->t_open = 0;
    K3G_CHECK(hipEventRecord(c->last_copy, c->copy));
    c->copies_pending = 1;
}

/* dst <- src with every host thread (a run is tens of MB) */
static void par_copy(unsigned char *dst, const unsigned char *src, size_t n)
{
    const int parts = 16;
    const size_t per = ((n + parts - 1) / parts + 4095) & ~(size_t)4095;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < parts; i++) {
        const size_t a = (size_t)i * per;
        if (a < n) memcpy(dst + a, src + a, (a + per < n ? per : n - a));
    }
}

/* Copy (layer, expert) from the bank into `slot`, after the last step that read it. A run
 * in a pageable layer goes through the next pinned staging buffer: once the DMA engine
 * has copied that buffer's previous run out, the host copies this run in, and the DMA
 * engine copies it to the slot at the pinned rate (the host copy of the next miss
 * overlaps this one's DMA). */
static double now_s(void)
{
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

/* Misses of a checkpoint bank into their slots: in groups of the staging buffers, the
 * runs resolved and read in parallel (one thread each, O_DIRECT where the shard has it),
 * then each copied to its slot after the last step that read the slot, and tiled there
 * for the tiled layout. ok[i] = 1 when slots[i] now holds keys[i]. */
static void disk_fetch(K3gCache *c, int n, const int *slots, const int32_t *keys, int *ok)
{
    K3gcBank *b = c->bank;
    for (int i0 = 0; i0 < n; i0 += b->nstage) {
        const int m = n - i0 < b->nstage ? n - i0 : b->nstage;
        int js[K3GC_NSTAGE], good[K3GC_NSTAGE];
        int64_t pad[K3GC_NSTAGE];
        K3gcExpertRun r[K3GC_NSTAGE];
        for (int k = 0; k < m; k++) {
            const int32_t key = keys[i0 + k];
            js[k] = (int)(c->stage_next++ % (unsigned)b->nstage);
            if (has_device(c)) K3G_CHECK(hipEventSynchronize(c->stage_ev[js[k]]));
            good[k] = k3gc_st_expert(b->st, key / c->n_experts, key % c->n_experts, &r[k]) == 0 &&
                      disk_run_fits(b, &r[k]);
            pad[k] = 0;
        }
        const double t0 = now_s();
#pragma omp parallel for schedule(static, 1) num_threads(m) if (m > 1)
        for (int k = 0; k < m; k++)
            if (good[k])
                good[k] = k3gc_st_read_run_into(b->st, &r[k], b->stage[js[k]], b->stage_cap,
                                                &pad[k]) == 0;
        c->disk_seconds += now_s() - t0;
        for (int k = 0; k < m; k++) {
            const int32_t key = keys[i0 + k];
            const int slot = slots[i0 + k];
            ok[i0 + k] = good[k];
            if (!good[k]) {
                c->failed_reads++;
                fprintf(stderr, "k3gc: cannot read L%d expert %d from the checkpoint (or its "
                                "geometry differs from the cache's)\n",
                        key / c->n_experts, key % c->n_experts);
                continue;
            }
            c->bytes_read += (uint64_t)r[k].nbytes;
            if (!has_device(c)) continue;
            batch_open(c);
            const int64_t s = c->use_step[slot];
            if (s >= 0 && c->step - s <= K3GC_STEP_RING)
                K3G_CHECK(hipStreamWaitEvent(c->copy, c->step_ev[s % K3GC_STEP_RING], 0));
            const unsigned char *src = b->stage[js[k]] + pad[k];
            unsigned char *dst = c->arena + (size_t)slot * c->slot_bytes;
            if (b->layout == K3G_EXPERT_MXFP4_TILED) {
                /* the run in the checkpoint order (w1p w1s w2p w2s w3p w3s), then w1, w3,
                 * w2 tiled back to back as fill_q hands them out */
                unsigned char *d = b->dstage[js[k]];
                K3G_CHECK(hipMemcpyAsync(d, src, (size_t)r[k].nbytes, hipMemcpyHostToDevice,
                                         c->copy));
                const int64_t o1 = 0, o2 = r[k].p_bytes[0] + r[k].s_bytes[0];
                const int64_t o3 = o2 + r[k].p_bytes[1] + r[k].s_bytes[1];
                const size_t t13 = k3k_tiled_mxfp4_bytes(b->inter, b->hidden);
                if (k3k_tile_mxfp4(dst, d + o1, d + o1 + r[k].p_bytes[0], b->inter, b->hidden,
                                   c->copy) != 0 ||
                    k3k_tile_mxfp4(dst + t13, d + o3, d + o3 + r[k].p_bytes[2], b->inter,
                                   b->hidden, c->copy) != 0 ||
                    k3k_tile_mxfp4(dst + 2 * t13, d + o2, d + o2 + r[k].p_bytes[1], b->hidden,
                                   b->inter, c->copy) != 0)
                    k3g_fatal("k3gc: tiling a checkpoint run failed");
            } else {
                K3G_CHECK(hipMemcpyAsync(dst, src, (size_t)r[k].nbytes, hipMemcpyHostToDevice,
                                         c->copy));
            }
            K3G_CHECK(hipEventRecord(c->stage_ev[js[k]], c->copy));
        }
    }
}

static int copy_in(K3gCache *c, int slot, int32_t key)
{
    if (c->bank->st) {
        int ok = 0;
        disk_fetch(c, 1, &slot, &key, &ok);
        return ok ? 0 : -1;
    }
    c->bytes_read += (uint64_t)c->bank->expert_bytes;
    if (!has_device(c)) return 0;
    batch_open(c);
    const int64_t s = c->use_step[slot];
    if (s >= 0 && c->step - s <= K3GC_STEP_RING)
        K3G_CHECK(hipStreamWaitEvent(c->copy, c->step_ev[s % K3GC_STEP_RING], 0));
    const int layer = key / c->n_experts;
    const unsigned char *src =
        (const unsigned char *)k3gc_bank_expert(c->bank, layer, key % c->n_experts);
    const size_t n = (size_t)c->bank->expert_bytes;
    unsigned char *dst = c->arena + (size_t)slot * c->slot_bytes;
    if (!c->bank->layer_pinned[layer] && c->bank->nstage > 0) {
        const int j = (int)(c->stage_next++ % (unsigned)c->bank->nstage);
        K3G_CHECK(hipEventSynchronize(c->stage_ev[j]));
        par_copy(c->bank->stage[j], src, n);
        K3G_CHECK(hipMemcpyAsync(dst, c->bank->stage[j], n, hipMemcpyHostToDevice, c->copy));
        K3G_CHECK(hipEventRecord(c->stage_ev[j], c->copy));
        c->staged++;
    } else {
        K3G_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->copy));
    }
    return 0;
}

/* A slot handed out: its LRU stamp, and, inside a step, the step whose end event any later
 * copy into the slot must wait for (a slot used in the open step is never evicted before
 * the step ends, so no copy waits on that event before it is recorded) */
static void touch(K3gCache *c, int slot)
{
    c->used_at[slot] = ++c->clock;
    if (c->step_open) c->use_step[slot] = c->step;
}

/* Bring (layer, expert) resident; returns its slot or -1. src/cache/k3_cache.c:63-110 */
static int admit(K3gCache *c, int layer, int expert)
{
    const int32_t key = layer * c->n_experts + expert;
    int slot = c->slot_of[key];
    if (slot >= 0) {
        c->hits++;
        touch(c, slot);
        return slot;
    }
    c->misses++;
    slot = pick_victim(c);
    if (slot < 0) {
        fprintf(stderr, "k3gc: no evictable slot for L%d expert %d (all pinned or in use by "
                        "this step)\n", layer, expert);
        return -1;
    }
    if (c->key_of[slot] >= 0) {
        key_out(c, c->key_of[slot]);
        c->slot_of[c->key_of[slot]] = -1;
        c->evictions++;
    }
    if (copy_in(c, slot, key) != 0) {
        c->key_of[slot] = K3GC_EMPTY;        /* holds nothing: k3_cache.c:96-101 */
        return -1;
    }
    c->key_of[slot] = key;
    c->slot_of[key] = slot;
    key_in(c, key);
    touch(c, slot);
    return slot;
}

/* --------------------------------------------------------- K3ExpertSrc vtable ---- */
static int cache_get(K3ExpertSrc *self, int layer, int expert, K3ExpertQ *out)
{
    K3gCache *c = (K3gCache *)self;
    if (layer < 0 || layer >= c->n_layers || expert < 0 || expert >= c->n_experts) {
        fprintf(stderr, "k3gc: out of range L%d expert %d\n", layer, expert);
        return -1;
    }
    c->hist[layer * c->n_experts + expert]++;
    /* the request as the model made it, before it is served (k3_cache.c:244-255) */
    if (c->ntrace + 2 > c->captrace) {
        const int64_t nc = c->captrace ? c->captrace * 2 : (1 << 16);
        int32_t *nt = (int32_t *)realloc(c->trace, (size_t)nc * sizeof(int32_t));
        if (nt) { c->trace = nt; c->captrace = nc; }
    }
    if (c->ntrace + 2 <= c->captrace) {
        c->trace[c->ntrace++] = layer;
        c->trace[c->ntrace++] = expert;
    }
    const int slot = admit(c, layer, expert);
    batch_close(c);
    if (slot < 0) return -1;
    if (out) fill_q(c, slot, out);
    return 0;
}

/* src/cache/k3_cache.c:131-218: reserve serially, copy, publish. The copies are queued
 * back to back on the copy stream, so the DMA engine sees the whole batch at once. */
static int cache_getmany(K3ExpertSrc *self, int layer, const int *ids, int n)
{
    K3gCache *c = (K3gCache *)self;
    if (n <= 0 || layer < 0 || layer >= c->n_layers) return 0;
    int slots[K3_MAX_TOPK], experts[K3_MAX_TOPK];
    int nw = 0;
    for (int i = 0; i < n && nw < K3_MAX_TOPK; i++) {
        const int e = ids[i];
        if (e < 0 || e >= c->n_experts) continue;
        const int32_t key = layer * c->n_experts + e;
        if (c->slot_of[key] >= 0) continue;
        int dup = 0;
        for (int j = 0; j < nw; j++) if (experts[j] == e) { dup = 1; break; }
        if (dup) continue;
        const int slot = pick_victim(c);
        if (slot < 0) break;
        if (c->key_of[slot] >= 0) {
            key_out(c, c->key_of[slot]);
            c->slot_of[c->key_of[slot]] = -1;
            c->evictions++;
        }
        c->key_of[slot] = K3GC_INFLIGHT;
        /* the LRU stamp only: the copy below waits on the step of the slot's last user,
         * and the step of this use is marked when the slot is published */
        c->used_at[slot] = ++c->clock;
        slots[nw] = slot;
        experts[nw] = e;
        nw++;
    }
    int ok[K3_MAX_TOPK];
    int32_t keys[K3_MAX_TOPK];
    for (int i = 0; i < nw; i++) keys[i] = layer * c->n_experts + experts[i];
    if (c->bank->st) {
        disk_fetch(c, nw, slots, keys, ok);
    } else {
        for (int i = 0; i < nw; i++) ok[i] = copy_in(c, slots[i], layer * c->n_experts + experts[i]) == 0;
    }
    batch_close(c);
    int pub = 0;
    for (int i = 0; i < nw; i++) {
        const int32_t key = layer * c->n_experts + experts[i];
        if (!ok[i]) {
            c->key_of[slots[i]] = K3GC_EMPTY;   /* a failed read publishes nothing */
            continue;
        }
        pub++;
        c->key_of[slots[i]] = key;
        c->slot_of[key] = slots[i];
        key_in(c, key);
        touch(c, slots[i]);
        c->prefetch_reads++;
    }
    return pub;
}

static int cache_resident(K3ExpertSrc *self, int layer, int expert, K3ExpertQ *out)
{
    K3gCache *c = (K3gCache *)self;
    if (layer < 0 || layer >= c->n_layers || expert < 0 || expert >= c->n_experts) return 0;
    const int slot = c->slot_of[layer * c->n_experts + expert];
    if (slot < 0) return 0;
    if (out) fill_q(c, slot, out);
    return 1;
}

int k3gc_is_device_src(const K3ExpertSrc *src)
{
    return src && (src->get == cache_get || k3_cache_inner_of(src) != NULL);
}

int k3gc_layer_all_resident(const K3gCache *c, int layer)
{
    return c && layer >= 0 && layer < c->n_layers && c->layer_resident[layer] == c->n_experts;
}

const K3ExpertQ *k3gc_layer_table(K3gCache *c, int layer, hipStream_t st)
{
    if (!c || !has_device(c) || layer < 0 || layer >= c->n_layers) return NULL;
    K3ExpertQ *row = c->dev_table + (size_t)layer * c->n_experts;
    if (!c->table_dirty[layer]) return row;
    K3kEqSet set;
    memset(&set, 0, sizeof set);
    for (int e = 0; e < c->n_experts; e++) {
        const int slot = c->slot_of[layer * c->n_experts + e];
        set.e[set.n] = e;
        if (slot >= 0) fill_q(c, slot, &set.q[set.n]);
        else memset(&set.q[set.n], 0, sizeof set.q[set.n]);
        if (++set.n == K3K_EQSET || e == c->n_experts - 1) {
            if (k3k_set_experts(row, &set, st) != 0) return NULL;
            set.n = 0;
        }
    }
    c->table_dirty[layer] = 0;
    return row;
}

K3gCache *k3gc_of_src(K3ExpertSrc *src)
{
    if (src && src->get == cache_get) return (K3gCache *)src;
    return k3_cache_inner_of(src);
}

K3ExpertSrc *k3gc_src(K3gCache *c) { return c ? &c->src : NULL; }

/* ------------------------------------------------------------- construction ---- */
int k3gc_init(K3gCache **out, int device, K3gcBank *bank, int topk, int64_t budget_bytes)
{
    *out = NULL;
    if (!bank || topk < 1) return -1;
    if (device >= 0 && !bank->layer_host && !bank->st) {
        fprintf(stderr, "k3gc_init: the bank holds no host memory\n");
        return -1;
    }
    K3gCache *c = (K3gCache *)calloc(1, sizeof *c);
    if (!c) return -1;
    c->src.get = cache_get;
    /* K3_NOPREFETCH set: no batch path (src/cache/k3_cache.c:268-274), so one binary can
     * time the layer with and without it; get() then copies each miss itself */
    c->src.getmany = getenv("K3_NOPREFETCH") ? NULL : cache_getmany;
    if (!c->src.getmany) fprintf(stderr, "k3gc: batch prefetch disabled by K3_NOPREFETCH\n");
    c->src.resident = cache_resident;
    c->src.ctx = c;
    c->bank = bank;
    c->device = device;
    c->n_layers = bank->n_layers;
    c->n_experts = bank->n_experts;
    c->topk = topk;
    /* a slot is one run rounded up to 64 KB, so every slot starts on a 64 KB boundary */
    c->slot_bytes = (bank->expert_bytes + 65535) & ~(int64_t)65535;
    c->nslot = (int)(budget_bytes / c->slot_bytes);
    if (c->nslot < topk + 1) {
        fprintf(stderr,
                "k3gc_init: budget %.2f GB gives %d slots of %.2f MB, but top-%d needs at "
                "least %d\n", (double)budget_bytes / 1e9, c->nslot, c->slot_bytes / 1e6, topk,
                topk + 1);
        free(c);
        return -1;
    }
    const size_t nkey = (size_t)c->n_layers * c->n_experts;
    c->slot_of = (int32_t *)malloc(nkey * sizeof(int32_t));
    c->key_of = (int32_t *)malloc((size_t)c->nslot * sizeof(int32_t));
    c->used_at = (uint64_t *)calloc((size_t)c->nslot, sizeof(uint64_t));
    c->pinned = (unsigned char *)calloc((size_t)c->nslot, 1);
    c->use_step = (int64_t *)malloc((size_t)c->nslot * sizeof(int64_t));
    c->hist = (uint32_t *)calloc(nkey, sizeof(uint32_t));
    c->layer_resident = (int32_t *)calloc((size_t)c->n_layers, sizeof(int32_t));
    c->table_dirty = (unsigned char *)malloc((size_t)c->n_layers);
    if (c->table_dirty) memset(c->table_dirty, 1, (size_t)c->n_layers);
    if (!c->slot_of || !c->key_of || !c->used_at || !c->pinned || !c->use_step || !c->hist ||
        !c->layer_resident || !c->table_dirty) {
        k3gc_free(c);
        return -1;
    }
    for (size_t i = 0; i < nkey; i++) c->slot_of[i] = -1;
    for (int i = 0; i < c->nslot; i++) { c->key_of[i] = K3GC_EMPTY; c->use_step[i] = -1; }
    if (device >= 0) {
        if (hipSetDevice(device) != hipSuccess ||
            hipMalloc((void **)&c->arena, (size_t)c->nslot * c->slot_bytes) != hipSuccess) {
            fprintf(stderr, "k3gc_init: cannot allocate %.2f GB of HBM slots\n",
                    (double)c->nslot * c->slot_bytes / 1e9);
            c->arena = NULL;
            k3gc_free(c);
            return -1;
        }
        K3G_CHECK(hipStreamCreateWithFlags(&c->copy, hipStreamNonBlocking));
        for (int i = 0; i < K3GC_STEP_RING; i++)
            K3G_CHECK(hipEventCreateWithFlags(&c->step_ev[i], hipEventDisableTiming));
        K3G_CHECK(hipEventCreateWithFlags(&c->last_copy, hipEventDisableTiming));
        for (int i = 0; i < K3GC_NSTAGE; i++) {
            K3G_CHECK(hipEventCreateWithFlags(&c->stage_ev[i], hipEventDisableTiming));
            K3G_CHECK(hipEventRecord(c->stage_ev[i], c->copy));
        }
        for (int i = 0; i < K3GC_TIMER_RING; i++) {
            K3G_CHECK(hipEventCreate(&c->tev[i][0]));
            K3G_CHECK(hipEventCreate(&c->tev[i][1]));
        }
        const size_t tb = nkey * sizeof(K3ExpertQ);
        if (hipMalloc((void **)&c->dev_table, tb) != hipSuccess ||
            hipMemset(c->dev_table, 0, tb) != hipSuccess) {
            c->dev_table = NULL;
            k3gc_free(c);
            return -1;
        }
    }
    *out = c;
    return 0;
}

void k3gc_free(K3gCache *c)
{
    if (!c) return;
    if (has_device(c)) {
        hipSetDevice(c->device);
        if (c->copy) {
            hipStreamSynchronize(c->copy);
            for (int i = 0; i < K3GC_STEP_RING; i++)
                if (c->step_ev[i]) hipEventDestroy(c->step_ev[i]);
            if (c->last_copy) hipEventDestroy(c->last_copy);
            for (int i = 0; i < K3GC_NSTAGE; i++)
                if (c->stage_ev[i]) hipEventDestroy(c->stage_ev[i]);
            for (int i = 0; i < K3GC_TIMER_RING; i++) {
                if (c->tev[i][0]) hipEventDestroy(c->tev[i][0]);
                if (c->tev[i][1]) hipEventDestroy(c->tev[i][1]);
            }
            hipStreamDestroy(c->copy);
        }
        hipDeviceSynchronize();
        if (c->arena) hipFree(c->arena);
        if (c->dev_table) hipFree(c->dev_table);
        if (c->host_idx) hipHostFree(c->host_idx);
        if (c->chain_dev) hipFree(c->chain_dev);
        if (c->chain_host) hipHostFree(c->chain_host);
    }
    free(c->slot_of);
    free(c->key_of);
    free(c->used_at);
    free(c->pinned);
    free(c->use_step);
    free(c->hist);
    free(c->trace);
    free(c->layer_resident);
    free(c->table_dirty);
    free(c);
}

/* ------------------------------------------------------------------- steps ---- */
void k3gc_step_begin(K3gCache *c)
{
    if (!c) return;
    c->step_open = 1;
    c->step_clock = c->clock + 1;
}

void k3gc_step_end(K3gCache *c, void *stream)
{
    if (!c) return;
    if (has_device(c)) {
        hipEvent_t ev = c->step_ev[c->step % K3GC_STEP_RING];
        /* the event last marked step - RING: its waits are long satisfied, but make
         * sure before it is re-recorded */
        if (c->step >= K3GC_STEP_RING) K3G_CHECK(hipEventSynchronize(ev));
        K3G_CHECK(hipEventRecord(ev, (hipStream_t)stream));
    }
    c->step++;
    c->step_open = 0;
}

void k3gc_wait(K3gCache *c, void *stream)
{
    if (!c || !has_device(c) || !c->copies_pending) return;
    K3G_CHECK(hipStreamWaitEvent((hipStream_t)stream, c->last_copy, 0));
    c->copies_pending = 0;
}

/* --------------------------------------------------------------- management ---- */
int k3gc_pin(K3gCache *c, int layer, int expert, int pin)
{
    if (!c || layer < 0 || layer >= c->n_layers || expert < 0 || expert >= c->n_experts)
        return 0;
    const int slot = c->slot_of[layer * c->n_experts + expert];
    if (slot < 0) return 0;
    c->pinned[slot] = pin ? 1 : 0;
    return 1;
}

int k3gc_prefetch(K3gCache *c, int layer, int expert)
{
    if (!c || layer < 0 || layer >= c->n_layers || expert < 0 || expert >= c->n_experts)
        return -1;
    const int slot = admit(c, layer, expert);
    batch_close(c);
    return slot >= 0 ? 0 : -1;
}

void k3gc_reset_stats(K3gCache *c)
{
    if (!c) return;
    if (has_device(c)) harvest_timers(c, 1);
    /* prefetch_reads covers the same window as hits (k3_cache.c:384-394) */
    c->hits = c->misses = c->evictions = c->bytes_read = c->prefetch_reads = 0;
    c->load_seconds = c->disk_seconds = 0.0;
    c->failed_reads = 0;
}

void k3gc_stats(K3gCache *c, K3gcStats *o)
{
    memset(o, 0, sizeof *o);
    if (!c) return;
    if (has_device(c)) harvest_timers(c, 1);
    o->requests = (int64_t)(c->hits + c->misses);
    o->hits = (int64_t)c->hits;
    o->misses = (int64_t)c->misses;
    o->evictions = (int64_t)c->evictions;
    o->prefetch_reads = (int64_t)c->prefetch_reads;
    o->bytes_read = (int64_t)c->bytes_read;
    o->load_seconds = c->load_seconds;
    o->nslot = c->nslot;
    o->slot_bytes = c->slot_bytes;
    o->staged = (int64_t)c->staged;
    for (int i = 0; i < c->nslot; i++) {
        if (c->key_of[i] >= 0) o->resident++;
        if (c->pinned[i]) o->pinned++;
    }
}

void k3gc_report(K3gCache *c, const char *label)
{
    K3gcStats s;
    k3gc_stats(c, &s);
    const double n = (double)s.requests;
    printf("cache [%s]\n", label ? label : "");
    printf("  slots        : %d of %.2f MB = %.2f GB HBM (%d resident, %d pinned)\n", s.nslot,
           s.slot_bytes / 1e6, (double)s.nslot * s.slot_bytes / 1e9, s.resident, s.pinned);
    printf("  requests     : %lld  hits %lld (%.2f%%)  misses %lld  evictions %lld\n",
           (long long)s.requests, (long long)s.hits, n > 0 ? 100.0 * s.hits / n : 0.0,
           (long long)s.misses, (long long)s.evictions);
    if (s.prefetch_reads) {
        const long long served = s.hits > s.prefetch_reads ? s.hits - s.prefetch_reads : 0;
        printf("  of those hits : %lld came from the batch prefetch, i.e. copied this step;\n"
               "                  TRUE resident hit rate %.2f%%\n",
               (long long)s.prefetch_reads, n > 0 ? 100.0 * served / n : 0.0);
    }
    printf("  copied H2D   : %.2f GB in %.3f s of copy-stream time (%.1f GB/s)\n",
           s.bytes_read / 1e9, s.load_seconds,
           s.load_seconds > 0 ? s.bytes_read / 1e9 / s.load_seconds : 0.0);
}

int k3gc_dump_hist(const K3gCache *c, const char *path)
{
    FILE *f = fopen(path, "w");
    if (!f) return -1;
    fprintf(f, "{\"n_layers\":%d,\"n_experts\":%d,\"counts\":{", c->n_layers, c->n_experts);
    int first = 1;
    for (int L = 0; L < c->n_layers; L++)
        for (int e = 0; e < c->n_experts; e++) {
            const uint32_t v = c->hist[L * c->n_experts + e];
            if (!v) continue;
            fprintf(f, "%s\"%d,%d\":%u", first ? "" : ",", L, e, v);
            first = 0;
        }
    fprintf(f, "}}\n");
    fclose(f);
    return 0;
}

int k3gc_dump_trace(const K3gCache *c, const char *path)
{
    if (!c->trace || c->ntrace == 0) return -1;
    FILE *f = fopen(path, "wb");
    if (!f) return -1;
    const size_t n = fwrite(c->trace, sizeof(int32_t), (size_t)c->ntrace, f);
    fclose(f);
    return n == (size_t)c->ntrace ? 0 : -1;
}

/* ------------------------------------------------------------ streamed layer ---- */
int k3gc_moe(K3gCtx *ctx, K3gCache *c, const K3gLayer *L, int layer, const float *x, int T,
             float *out, int32_t *idx, float *wt, const int32_t *route_idx,
             const float *route_wt, void *stream)
{
    if (!ctx || !c || !has_device(c) || !L || layer < 0 || layer >= c->n_layers) return -1;
    if (c->bank->layout != K3G_EXPERT_MXFP4_TILED || L->n_experts != c->n_experts ||
        L->hidden != c->bank->hidden || L->inter != c->bank->inter) {
        fprintf(stderr, "k3gc_moe: the layer does not match the cache's tiled bank\n");
        return -1;
    }
    hipStream_t st = stream ? (hipStream_t)stream : (hipStream_t)k3g_ctx_stream(ctx);
    const int k = L->topk, P = T * k;
    if (T < 1 || k < 1 || P > 65536) return -1;
    if (c->host_idx_cap < P) {
        if (c->host_idx) hipHostFree(c->host_idx);
        c->host_idx = NULL;
        if (hipHostMalloc((void **)&c->host_idx, (size_t)P * 4, hipHostMallocDefault) !=
            hipSuccess) return -1;
        c->host_idx_cap = P;
    }
    if (!route_idx) {
        if (k3g_route(ctx, L, x, T, idx, wt, st) != 0) return -1;
        K3G_CHECK(hipMemcpyAsync(c->host_idx, idx, (size_t)P * 4, hipMemcpyDeviceToHost, st));
        K3G_CHECK(hipStreamSynchronize(st));
    } else {
        memcpy(c->host_idx, route_idx, (size_t)P * 4);
        K3G_CHECK(hipMemcpyAsync(idx, c->host_idx, (size_t)P * 4, hipMemcpyHostToDevice, st));
        K3G_CHECK(hipMemcpyAsync(wt, route_wt, (size_t)P * 4, hipMemcpyHostToDevice, st));
        /* the staging buffer is reused by the next call: let the copies finish */
        K3G_CHECK(hipStreamSynchronize(st));
    }
    /* tokens in groups whose experts fit the unpinned slots together (every slot a
     * group gets stays put until the group's kernels are done); per group, its unique
     * experts in first-seen order: getmany, then one get each */
    int npinned = 0;
    for (int i = 0; i < c->nslot; i++) npinned += c->pinned[i] != 0;
    const int cap = c->nslot - npinned;
    int *uniq = (int *)malloc((size_t)P * sizeof(int));
    unsigned char *seen = (unsigned char *)calloc((size_t)c->n_experts, 1);
    if (!uniq || !seen || cap < 1) { free(uniq); free(seen); return -1; }
    K3ExpertQ *table = c->dev_table + (size_t)layer * c->n_experts;
    const int d = L->hidden;
    int rc = 0;
    for (int t0 = 0; t0 < T && rc == 0;) {
        memset(seen, 0, (size_t)c->n_experts);
        int nu = 0, t1 = t0;
        while (t1 < T) {
            int add = 0;
            for (int j = 0; j < k; j++) {
                const int e = c->host_idx[t1 * k + j];
                if (e >= 0 && e < c->n_experts && !seen[e]) {
                    int dup = 0;
                    for (int q = 0; q < j; q++) dup |= c->host_idx[t1 * k + q] == e;
                    add += !dup;
                }
            }
            if (nu + add > cap && t1 > t0) break;
            for (int j = 0; j < k; j++) {
                const int e = c->host_idx[t1 * k + j];
                if (e >= 0 && e < c->n_experts && !seen[e]) { seen[e] = 1; uniq[nu++] = e; }
            }
            t1++;
        }
        k3gc_step_begin(c);
        for (int i = 0; i < nu; i += K3_MAX_TOPK)
            if (c->src.getmany)
                c->src.getmany(&c->src, layer, uniq + i, nu - i < K3_MAX_TOPK ? nu - i : K3_MAX_TOPK);
        K3kEqSet set;
        memset(&set, 0, sizeof set);
        for (int i = 0; i < nu && rc == 0; i++) {
            K3ExpertQ q;
            if (cache_get(&c->src, layer, uniq[i], &q) != 0) { rc = -1; break; }
            set.e[set.n] = uniq[i];
            set.q[set.n] = q;
            if (++set.n == K3K_EQSET) {
                rc |= k3k_set_experts(table, &set, st);
                set.n = 0;
            }
        }
        if (rc == 0 && set.n) rc |= k3k_set_experts(table, &set, st);
        if (rc == 0) {
            K3gLayer Lc = *L;
            Lc.experts = table;
            Lc.expert_fmt = K3G_EXPERT_MXFP4_TILED;
            /* the shared expert runs while the misses copy; the routed experts wait */
            if (c->copies_pending) {
                k3g_ctx_routed_wait(ctx, c->last_copy);
                c->copies_pending = 0;
            }
            rc = k3g_experts(ctx, &Lc, x + (size_t)t0 * d, t1 - t0, idx + (size_t)t0 * k,
                             wt + (size_t)t0 * k, out + (size_t)t0 * d, st);
        }
        k3gc_step_end(c, st);
        t0 = t1;
    }
    free(uniq);
    free(seen);
    return rc;
}

/* ------------------------------------------------------------- chained layers ---- */
/* The step's unique experts of routing idx [T][k] in first-seen order, through getmany
 * then one get each (the calls k3gc_moe makes); returns 0 or -1 on a failed get. */
static int account_step(K3gCache *c, int layer, const int32_t *idx, int P, hipStream_t st)
{
    int uniq[4 * K3_MAX_TOPK * 4];
    int nu = 0, rc = 0;
    for (int p = 0; p < P && nu < (int)(sizeof uniq / sizeof uniq[0]); p++) {
        const int e = idx[p];
        if (e < 0 || e >= c->n_experts) continue;
        int dup = 0;
        for (int j = 0; j < nu; j++) if (uniq[j] == e) { dup = 1; break; }
        if (!dup) uniq[nu++] = e;
    }
    k3gc_step_begin(c);
    for (int i = 0; i < nu; i += K3_MAX_TOPK)
        if (c->src.getmany)
            c->src.getmany(&c->src, layer, uniq + i, nu - i < K3_MAX_TOPK ? nu - i : K3_MAX_TOPK);
    for (int i = 0; i < nu; i++)
        if (cache_get(&c->src, layer, uniq[i], NULL) != 0) rc = -1;
    k3gc_step_end(c, st);
    return rc;
}

int k3gc_chain(K3gCtx *ctx, K3gCache *c, const K3gLayer *layers, const float *const *post_norm,
               int first_layer, int n_layers, float *h, int T, float rms_eps, void *stream)
{
    if (!ctx || !c || !has_device(c) || !layers || !h || n_layers < 1 || T < 1 ||
        first_layer < 0 || first_layer + n_layers > c->n_layers)
        return -1;
    hipStream_t st = stream ? (hipStream_t)stream : (hipStream_t)k3g_ctx_stream(ctx);
    const int d = layers[0].hidden;
    int kmax = 1;
    for (int l = 0; l < n_layers; l++) {
        if (layers[l].hidden != d) return -1;
        if (layers[l].topk > kmax) kmax = layers[l].topk;
    }
    const size_t act = ((size_t)T * d * 4 + 255) & ~(size_t)255;
    const size_t rt = ((size_t)T * kmax * 4 + 255) & ~(size_t)255;
    const size_t need = 2 * act + 2 * rt * (size_t)n_layers;
    if (need > c->chain_dev_bytes) {
        if (c->chain_dev) {
            K3G_CHECK(hipDeviceSynchronize());
            K3G_CHECK(hipFree(c->chain_dev));
        }
        c->chain_dev = NULL;
        if (hipMalloc((void **)&c->chain_dev, need) != hipSuccess) return -1;
        c->chain_dev_bytes = need;
    }
    const size_t hneed = rt * (size_t)n_layers;
    if (hneed > c->chain_host_bytes) {
        if (c->chain_host) {
            K3G_CHECK(hipDeviceSynchronize());
            K3G_CHECK(hipHostFree(c->chain_host));
        }
        c->chain_host = NULL;
        if (hipHostMalloc((void **)&c->chain_host, hneed, hipHostMallocDefault) != hipSuccess)
            return -1;
        c->chain_host_bytes = hneed;
    }
    float *hin = (float *)c->chain_dev, *tmp = (float *)(c->chain_dev + act);
    /* the layers' routing: idx of layer l at rbase + rt l, its weights after all idx */
    unsigned char *rbase = c->chain_dev + 2 * act;
    /* every expert of every layer resident: the layers run back to back on the cache's
     * device tables with no host synchronisation, the accounting after them */
    int resident = c->bank->layout == K3G_EXPERT_MXFP4_TILED;
    for (int l = 0; l < n_layers && resident; l++)
        resident = k3gc_layer_all_resident(c, first_layer + l);
    if (resident) k3gc_wait(c, st);
    int rc = 0;
    /* hin = RMSNorm(h) x post_norm (src/core/k3_ops.c:1015-1016); between layers the
     * residual add and the next layer's norm are one launch */
    if (post_norm && post_norm[0] &&
        k3k_add_rmsnorm(h, NULL, hin, post_norm[0], d, T, rms_eps, st) != 0)
        return -1;
    for (int l = 0; l < n_layers && rc == 0; l++) {
        const K3gLayer *L = &layers[l];
        const int layer = first_layer + l;
        int32_t *idx = (int32_t *)(rbase + rt * (size_t)l);
        float *wt = (float *)(rbase + rt * (size_t)(n_layers + l));
        const float *in = post_norm && post_norm[l] ? hin : h;
        if (resident) {
            K3gLayer G = *L;
            G.experts = k3gc_layer_table(c, layer, st);
            G.expert_fmt = K3G_EXPERT_MXFP4_TILED;
            if (!G.experts) return -1;
            rc = k3g_moe(ctx, &G, in, T, tmp, idx, wt, st);
        } else {
            rc = k3gc_moe(ctx, c, L, layer, in, T, tmp, idx, wt, NULL, NULL, st);
        }
        /* h += the layer's MoE output (src/core/k3_ops.c:1035-1036), then the next
         * layer's hin */
        const float *next = post_norm && l + 1 < n_layers ? post_norm[l + 1] : NULL;
        if (rc == 0) rc = k3k_add_rmsnorm(h, tmp, next ? hin : NULL, next, d, T, rms_eps, st);
    }
    if (resident && rc == 0) {
        /* every layer's routing to the host in one copy on the compute stream */
        if (k3k_copy(c->chain_host, rbase, rt * (size_t)n_layers, st) != 0)
            K3G_CHECK(hipMemcpyAsync(c->chain_host, rbase, rt * (size_t)n_layers,
                                     hipMemcpyDeviceToHost, st));
        K3G_CHECK(hipStreamSynchronize(st));
        for (int l = 0; l < n_layers && rc == 0; l++)
            rc = account_step(c, first_layer + l,
                              (const int32_t *)((unsigned char *)c->chain_host + rt * (size_t)l),
                              T * layers[l].topk, st);
    }
    return rc;
}

