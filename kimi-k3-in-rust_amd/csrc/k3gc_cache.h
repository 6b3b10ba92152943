/* k3gc_cache.h - HBM expert cache (private declarations shared with the drop-in and the
 * context). The public API is in include/k3moe.h. */
#ifndef K3GC_CACHE_H
#define K3GC_CACHE_H

#include "../../include/k3moe.h"

#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>

/* Slot states in key_of[] (src/cache/k3_cache.h:40-45 keeps the same three): a key,
 * EMPTY, or INFLIGHT (reserved by a batch whose copies are not yet issued). */
#define K3GC_EMPTY (-1)
#define K3GC_INFLIGHT (-2)

#define K3GC_STEP_RING 1024
#define K3GC_TIMER_RING 256
#define K3GC_NSTAGE 4          /* pinned staging buffers for misses from pageable layers */

struct K3gcBank {
    int n_layers, n_experts, hidden, inter, layout;
    int64_t expert_bytes;
    /* a bank without a layer shape (hidden == 0): the six matrices' offsets in a run,
     * w1p w1s w2p w2s w3p w3s, as the checkpoint's runs have them (k3gc_bank_load) */
    int64_t raw_off[6];
    int raw_geometry;
    unsigned char **layer_host;   /* [n_layers]: [n_experts][expert_bytes] each */
    unsigned char *layer_pinned;  /* [n_layers]: 1 hipHostMalloc, 0 pageable malloc */
    int pinned_layers;
    /* pinned staging for the pageable layers' runs: the host copies a run in (all
     * threads), the DMA engine copies it out at the pinned rate */
    unsigned char *stage[K3GC_NSTAGE];
    int nstage;
    /* a checkpoint bank (k3gc_bank_create_disk): no host copy of the experts; a miss is
     * read from st into a pinned staging buffer (stage_cap bytes, room for the run's
     * enclosing 4096-byte window) and, for the tiled layout, copied to a device staging
     * buffer and tiled into its slot */
    const K3gcSt *st;
    int64_t run_bytes;            /* checkpoint bytes of one run */
    int64_t stage_cap;
    unsigned char *dstage[K3GC_NSTAGE];
};

struct K3gCache {
    K3ExpertSrc src;              /* first: callers pass &cache->src as K3MoeW.src */
    K3gcBank *bank;
    int device;                   /* < 0: bookkeeping only (no device memory, no copies) */
    int n_layers, n_experts, topk;
    int64_t slot_bytes;
    int nslot;
    unsigned char *arena;         /* device, nslot * slot_bytes */
    int32_t *slot_of;             /* [n_layers * n_experts] -> slot or -1 */
    int32_t *key_of;              /* [nslot] -> key, K3GC_EMPTY or K3GC_INFLIGHT */
    uint64_t *used_at;            /* [nslot] LRU stamp */
    unsigned char *pinned;        /* [nslot] */
    int64_t *use_step;            /* [nslot] last step that handed the slot out, -1 none */
    uint64_t clock;
    int step_open;
    uint64_t step_clock;          /* used_at >= step_clock: handed out in the open step */
    int64_t step;                 /* steps ended so far */
    /* device side */
    hipStream_t copy;             /* the side stream the misses are copied on */
    hipEvent_t step_ev[K3GC_STEP_RING];   /* compute stream, end of each step */
    hipEvent_t last_copy;         /* copy stream, after the latest copy */
    int copies_pending;           /* copies issued since the last k3gc_wait */
    hipEvent_t tev[K3GC_TIMER_RING][2];   /* copy-stream timing per batch of copies */
    hipEvent_t stage_ev[K3GC_NSTAGE];     /* copy stream, after the copy out of a stage */
    unsigned stage_next;
    uint64_t staged;              /* misses copied through the staging buffers */
    int t_head, t_used, t_open;
    K3ExpertQ *dev_table;         /* [n_layers][n_experts] device pointers (k3gc_moe) */
    int32_t *layer_resident;      /* [n_layers] experts of the layer holding a slot */
    unsigned char *table_dirty;   /* [n_layers] dev_table row behind the slots */
    int32_t *host_idx;            /* pinned staging of a step's routing */
    int host_idx_cap;
    /* k3gc_chain's buffers, grow-only: device hin/tmp [T][hidden] and idx/wt per layer;
     * pinned routing per layer */
    unsigned char *chain_dev;
    size_t chain_dev_bytes;
    int32_t *chain_host;
    size_t chain_host_bytes;
    /* stats (src/cache/k3_cache.h:74-83) */
    uint64_t hits, misses, evictions, bytes_read, prefetch_reads;
    double load_seconds;
    double disk_seconds;          /* checkpoint bank: host time in checkpoint reads */
    uint64_t failed_reads;        /* checkpoint bank: runs that could not be read */
    uint32_t *hist;               /* [n_layers * n_experts] requests */
    int32_t *trace;               /* (layer, expert) pairs in request order */
    int64_t ntrace, captrace;
};

/* The HBM cache inside an engine-layout K3Cache whose src this is, or NULL
 * (k3_cache_dropin.c). */
K3gCache *k3_cache_inner_of(const K3ExpertSrc *src);
/* 1 when src is an HBM expert cache, whose get() hands out device pointers. */
int k3gc_is_device_src(const K3ExpertSrc *src);
/* The cache behind a device source (NULL otherwise). */
K3gCache *k3gc_of_src(K3ExpertSrc *src);
/* 1 when every expert of the layer holds a slot (a get() of any of them is a hit). */
int k3gc_layer_all_resident(const K3gCache *c, int layer);
/* The layer's row of the device expert table, brought up to date with the slots on
 * `stream` when they changed since it was last written. */
const K3ExpertQ *k3gc_layer_table(K3gCache *c, int layer, hipStream_t stream);

#endif
