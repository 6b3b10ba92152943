/* k3gc_policy.c - replacement policy beyond LRU for the HBM expert cache (C99).
 *
 * Two parts:
 *  - offline replays of a recorded (layer, expert) request trace (the cache's own trace,
 *    k3gc_dump_trace, in the engine's format) at any capacity: LRU, Belady (the optimal
 *    offline policy; a request whose next use is later than every resident expert's is
 *    not cached), and the hottest experts pinned with LRU for the rest. These answer the
 *    sizing question the engine's tools/sim_cache.py answers (its lru, belady and
 *    pinned_lru at :36-110), with the same definitions, so the numbers compare with the
 *    engine's published table;
 *  - histogram-driven pinning: the purpose of the engine's per-(layer, expert) request
 *    histogram and k3_cache_pin (src/cache/k3_cache.h:29-31, :100-102): the hot set of a
 *    previous workload made resident and never evicted.
 *
 * The replays run in O(n log n): keys are made dense by sorting, LRU is a doubly linked
 * list, Belady a max-heap of next uses with stale entries skipped on the way out. */
#include "k3gc_cache.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ dense keys ---- */
typedef struct {
    int64_t key;
    int64_t at;
} KeyAt;

static int cmp_keyat(const void *a, const void *b)
{
    const KeyAt *x = (const KeyAt *)a, *y = (const KeyAt *)b;
    if (x->key != y->key) return x->key < y->key ? -1 : 1;
    return x->at < y->at ? -1 : (x->at > y->at);
}

/* ids[i] in 0..U-1 for request i, numbered in order of first occurrence; returns U, or
 * -1 on allocation failure. */
static int64_t dense_ids(const int32_t *pairs, int64_t n, int64_t *ids)
{
    KeyAt *ka = (KeyAt *)malloc((size_t)n * sizeof *ka);
    int64_t *first = (int64_t *)malloc((size_t)n * sizeof *first);
    if (!ka || !first) { free(ka); free(first); return -1; }
    for (int64_t i = 0; i < n; i++) {
        ka[i].key = ((int64_t)pairs[2 * i] << 20) | (int64_t)(uint32_t)pairs[2 * i + 1];
        ka[i].at = i;
    }
    qsort(ka, (size_t)n, sizeof *ka, cmp_keyat);
    /* group g's first occurrence is its first element (sorted by position within a key) */
    int64_t ng = 0;
    for (int64_t i = 0; i < n; i++) {
        if (i == 0 || ka[i].key != ka[i - 1].key) first[ng++] = ka[i].at;
        ids[ka[i].at] = ng - 1;               /* group number for now */
    }
    /* renumber groups by first occurrence: walk the trace, a group's first request
     * gets the next id */
    int64_t *rank = (int64_t *)malloc((size_t)ng * sizeof *rank);
    if (!rank) { free(ka); free(first); return -1; }
    for (int64_t g = 0; g < ng; g++) rank[g] = -1;
    int64_t next = 0;
    for (int64_t i = 0; i < n; i++) {
        const int64_t g = ids[i];
        if (rank[g] < 0) rank[g] = next++;
        ids[i] = rank[g];
    }
    free(rank);
    free(ka);
    free(first);
    return ng;
}

/* -------------------------------------------------------------------- LRU core ---- */
/* A doubly linked recency list over dense ids (head = most recent). */
typedef struct {
    int64_t *prev, *next;
    unsigned char *in;
    int64_t head, tail, size;
} Lru;

static int lru_init(Lru *l, int64_t u)
{
    l->prev = (int64_t *)malloc((size_t)u * sizeof(int64_t));
    l->next = (int64_t *)malloc((size_t)u * sizeof(int64_t));
    l->in = (unsigned char *)calloc((size_t)u, 1);
    l->head = l->tail = -1;
    l->size = 0;
    return l->prev && l->next && l->in ? 0 : -1;
}

static void lru_free(Lru *l) { free(l->prev); free(l->next); free(l->in); }

static void lru_unlink(Lru *l, int64_t k)
{
    if (l->prev[k] >= 0) l->next[l->prev[k]] = l->next[k]; else l->head = l->next[k];
    if (l->next[k] >= 0) l->prev[l->next[k]] = l->prev[k]; else l->tail = l->prev[k];
    l->in[k] = 0;
    l->size--;
}

static void lru_push(Lru *l, int64_t k)
{
    l->prev[k] = -1;
    l->next[k] = l->head;
    if (l->head >= 0) l->prev[l->head] = k; else l->tail = k;
    l->head = k;
    l->in[k] = 1;
    l->size++;
}

/* One request: returns 1 on a hit. cap >= 1. */
static int lru_touch(Lru *l, int64_t k, int64_t cap)
{
    if (l->in[k]) {
        lru_unlink(l, k);
        lru_push(l, k);
        return 1;
    }
    if (l->size >= cap) lru_unlink(l, l->tail);
    lru_push(l, k);
    return 0;
}

int64_t k3gc_replay_lru(const int32_t *pairs, int64_t n, int64_t capacity)
{
    if (!pairs || n <= 0 || capacity < 1) return 0;
    int64_t *ids = (int64_t *)malloc((size_t)n * sizeof *ids);
    if (!ids) return -1;
    const int64_t u = dense_ids(pairs, n, ids);
    Lru l;
    int64_t hits = -1;
    if (u >= 0 && lru_init(&l, u) == 0) {
        hits = 0;
        for (int64_t i = 0; i < n; i++) hits += lru_touch(&l, ids[i], capacity);
    }
    if (u >= 0) lru_free(&l);
    free(ids);
    return hits;
}

/* ------------------------------------------------------------------ Belady ---- */
typedef struct {
    int64_t nu, id;
} HeapE;

static void heap_push(HeapE *h, int64_t *n, HeapE e)
{
    int64_t i = (*n)++;
    while (i > 0) {
        const int64_t p = (i - 1) / 2;
        if (h[p].nu >= e.nu) break;
        h[i] = h[p];
        i = p;
    }
    h[i] = e;
}

static void heap_pop(HeapE *h, int64_t *n)
{
    const HeapE last = h[--(*n)];
    int64_t i = 0;
    for (;;) {
        int64_t c = 2 * i + 1;
        if (c >= *n) break;
        if (c + 1 < *n && h[c + 1].nu > h[c].nu) c++;
        if (h[c].nu <= last.nu) break;
        h[i] = h[c];
        i = c;
    }
    if (*n > 0) h[i] = last;
}

int64_t k3gc_replay_belady(const int32_t *pairs, int64_t n, int64_t capacity)
{
    if (!pairs || n <= 0 || capacity < 1) return 0;
    int64_t *ids = (int64_t *)malloc((size_t)n * sizeof *ids);
    int64_t *nxt = (int64_t *)malloc((size_t)n * sizeof *nxt);
    if (!ids || !nxt) { free(ids); free(nxt); return -1; }
    const int64_t u = dense_ids(pairs, n, ids);
    int64_t *last = u > 0 ? (int64_t *)malloc((size_t)u * sizeof *last) : NULL;
    int64_t *cur = u > 0 ? (int64_t *)malloc((size_t)u * sizeof *cur) : NULL;
    unsigned char *res = u > 0 ? (unsigned char *)calloc((size_t)u, 1) : NULL;
    /* one heap entry per request at most */
    HeapE *heap = (HeapE *)malloc((size_t)n * sizeof *heap);
    int64_t hits = -1;
    if (u > 0 && last && cur && res && heap) {
        /* next use of each request's key (n: never again) */
        for (int64_t k = 0; k < u; k++) last[k] = n;
        for (int64_t i = n - 1; i >= 0; i--) {
            nxt[i] = last[ids[i]];
            last[ids[i]] = i;
        }
        int64_t hn = 0, size = 0;
        hits = 0;
        for (int64_t i = 0; i < n; i++) {
            const int64_t k = ids[i];
            if (res[k]) {
                hits++;
                cur[k] = nxt[i];
                heap_push(heap, &hn, (HeapE){nxt[i], k});
                continue;
            }
            if (size >= capacity) {
                /* the resident expert used furthest in the future (stale entries out) */
                while (hn > 0 && (!res[heap[0].id] || cur[heap[0].id] != heap[0].nu))
                    heap_pop(heap, &hn);
                const int64_t v = heap[0].id;
                /* every resident expert is needed sooner than this one: do not cache it */
                if (cur[v] < nxt[i]) continue;
                heap_pop(heap, &hn);
                res[v] = 0;
                size--;
            }
            res[k] = 1;
            cur[k] = nxt[i];
            heap_push(heap, &hn, (HeapE){nxt[i], k});
            size++;
        }
    }
    free(ids); free(nxt); free(last); free(cur); free(res); free(heap);
    return hits;
}

/* -------------------------------------------------------------- pinned + LRU ---- */
typedef struct {
    int64_t count, id;
} CountId;

static int cmp_hot(const void *a, const void *b)
{
    const CountId *x = (const CountId *)a, *y = (const CountId *)b;
    if (x->count != y->count) return x->count > y->count ? -1 : 1;
    return x->id < y->id ? -1 : (x->id > y->id);     /* ids are first-occurrence order */
}

int64_t k3gc_replay_pinned_lru(const int32_t *pairs, int64_t n, int64_t capacity, int64_t npin)
{
    if (!pairs || n <= 0 || capacity < 1) return 0;
    if (npin >= capacity) npin = capacity - 1;
    if (npin < 0) npin = 0;
    int64_t *ids = (int64_t *)malloc((size_t)n * sizeof *ids);
    if (!ids) return -1;
    const int64_t u = dense_ids(pairs, n, ids);
    CountId *c = u > 0 ? (CountId *)calloc((size_t)u, sizeof *c) : NULL;
    unsigned char *hot = u > 0 ? (unsigned char *)calloc((size_t)u, 1) : NULL;
    unsigned char *loaded = u > 0 ? (unsigned char *)calloc((size_t)u, 1) : NULL;
    Lru l;
    int64_t hits = -1;
    if (u > 0 && c && hot && loaded && lru_init(&l, u) == 0) {
        /* the npin most requested experts of this trace, ties to the first seen */
        for (int64_t k = 0; k < u; k++) c[k].id = k;
        for (int64_t i = 0; i < n; i++) c[ids[i]].count++;
        qsort(c, (size_t)u, sizeof *c, cmp_hot);
        const int64_t nhot = npin < u ? npin : u;
        for (int64_t j = 0; j < nhot; j++) hot[c[j].id] = 1;
        const int64_t room = capacity - nhot > 1 ? capacity - nhot : 1;
        hits = 0;
        for (int64_t i = 0; i < n; i++) {
            const int64_t k = ids[i];
            if (hot[k]) {
                /* a pinned expert is still read once: its first touch is a miss */
                if (loaded[k]) hits++;
                loaded[k] = 1;
                continue;
            }
            hits += lru_touch(&l, k, room);
        }
        lru_free(&l);
    }
    free(ids); free(c); free(hot); free(loaded);
    return hits;
}

/* ------------------------------------------------------ histogram-driven pin ---- */
typedef struct {
    uint32_t count;
    int32_t key;
} HistE;

static int cmp_hist(const void *a, const void *b)
{
    const HistE *x = (const HistE *)a, *y = (const HistE *)b;
    if (x->count != y->count) return x->count > y->count ? -1 : 1;
    return x->key < y->key ? -1 : (x->key > y->key);
}

const uint32_t *k3gc_hist(const K3gCache *c) { return c ? c->hist : NULL; }

int k3gc_pin_hottest(K3gCache *c, const uint32_t *hist, int npin)
{
    if (!c || !hist || npin <= 0) return 0;
    /* a token's experts must still find room: never pin past nslot - (top-k + 1) */
    int already = 0;
    for (int i = 0; i < c->nslot; i++) already += c->pinned[i] != 0;
    const int limit = c->nslot - (c->topk + 1) - already;
    if (npin > limit) npin = limit;
    if (npin <= 0) return 0;
    const int nkey = c->n_layers * c->n_experts;
    HistE *h = (HistE *)malloc((size_t)nkey * sizeof *h);
    if (!h) return 0;
    int m = 0;
    for (int k = 0; k < nkey; k++)
        if (hist[k]) { h[m].count = hist[k]; h[m].key = k; m++; }
    qsort(h, (size_t)m, sizeof *h, cmp_hist);
    int pinned = 0;
    for (int j = 0; j < m && pinned < npin; j++) {
        const int layer = h[j].key / c->n_experts, e = h[j].key % c->n_experts;
        if (k3gc_prefetch(c, layer, e) != 0) break;
        if (k3gc_pin(c, layer, e, 1)) pinned++;
    }
    free(h);
    return pinned;
}
