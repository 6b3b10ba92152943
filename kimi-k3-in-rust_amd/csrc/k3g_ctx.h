/* k3g_ctx.h - the device context behind the k3g_* API (private to the library). */
#ifndef K3G_CTX_H
#define K3G_CTX_H

#include "k3g_kernels.h"

/* Abort with a message when a HIP call fails on the hot path: the engine's rule is that
 * a kernel never returns a partial or stale output (src/core/k3_ops.c:37-78). */
#define K3G_CHECK(call)                                                                   \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess) k3g_fatal_hip(#call, e_, __FILE__, __LINE__);               \
    } while (0)

void k3g_fatal_hip(const char *what, hipError_t e, const char *file, int line);
void k3g_fatal(const char *what);

/* stages of a layer call, for the optional per-stage timing */
enum {
    K3G_ST_ROUTER = 0, K3G_ST_DISPATCH, K3G_ST_GATEUP, K3G_ST_DOWN, K3G_ST_SH_GATEUP,
    K3G_ST_SH_DOWN, K3G_ST_COMBINE, K3G_ST_LATENT, K3G_ST_FUSED, K3G_ST_PIECES, K3G_NSTAGE
};

#define K3G_RING 256

struct K3gCtx {
    int device;
    hipStream_t stream;
    /* shape the workspace was sized for */
    int hidden, n_experts, topk, inter, shared_inter, latent, max_tokens;
    int force_exact;
    /* one device allocation, carved below */
    void *ws;
    size_t ws_bytes;
    float *rs;                   /* [T][E][4] router score intervals */
    int32_t *idx;                /* [T][k] when the caller passes none */
    float *wt;
    int32_t *cnt, *base;         /* [nch][E] */
    int32_t *off, *act, *nact;   /* [E+1], [E], [1] */
    int32_t *perm;               /* [T*k] */
    float *z;                    /* [T][latent] when projected */
    float *h;                    /* [T*k][inter] */
    float *contrib;              /* [T*k][latent] */
    float *accl;                 /* [T][latent] */
    float *sh_h;                 /* [T][shared_inter] */
    float *sh_out;               /* [T][hidden] */
    int *err;                    /* device error word */
    int *stats;                  /* device counters */
    /* fused decode kernel: activation pieces, partial sums, counters */
    uint8_t *xq8, *hq8;
    uint16_t *xq16, *hq16;
    float *gpart, *sgpart, *shpart, *dcontrib;
    /* the fused kernel's latent-layer buffers (k3g_decode.hip) */
    float *dzpart, *daccl, *dupart;
    uint8_t *dzq8;
    double *dnss;
    uint16_t *daq16;
    double *rpart;
    int *sync;
    size_t sync_bytes;
    int epoch;                   /* fused-kernel calls; its parity picks the counter bank */
    int fused;                   /* use the fused decode kernel when the layer allows */
    int paths;                   /* kernels the calls ran since it was cleared: bit 0 the
                                  * staged kernels, 1 the fused decode kernel, 2 the
                                  * grouped GEMMs */
    /* grouped GEMMs on the matrix cores (more than 4 tokens, tiled layouts) */
    uint16_t *xb, *hb, *hsb;     /* bf16 pieces of x [2][T][d128], h [2][T*k][I128], shared h */
    uint16_t *zb;                /* bf16 pieces of the latent input / aggregate [2][T][L128] */
    int32_t *zflag;              /* their piece-1 flag (written, not read) */
    float *kpart;                /* K-slice sums of the dense GEMMs */
    float *kpart2;               /* the shared expert's, when it runs on the side stream */
    double *rtpart;              /* K-slice sums of the router's matrix-core logits */
    int32_t *rtctr;              /* their per-tile arrival counts (zero between calls) */
    float *rbpart;               /* the bounded bf16 logits' K-slice sums and norms */
    const int32_t *route_x1flag; /* x's piece-1 flag for the call being routed, or NULL */
    size_t rbpart_floats;
    int32_t *tiles, *ntiles, *xflag;
    int max_tiles;
    hipEvent_t routed_wait;      /* the next k3g_experts waits for it before routed work */
    /* a second compute stream (default priority): the shared expert of a grouped call
     * runs on it beside the router and the routed experts; ev_in orders it after x's
     * pieces, ev_shared marks its end */
    hipStream_t side;
    hipEvent_t ev_in, ev_shared;
    int gemm_fp8;                /* routed experts on the FP4 x FP8 matrix cores */
    uint8_t *xq8b, *hq8b;        /* MXFP8 x [T][d512] + scales, h [T*k][I512] + scales */
    unsigned long long *trace;   /* optional per-ticket timestamps of the fused kernel */
    /* optional pinned host copies that the fused kernel writes directly (the routing, a
     * nonzero error code), for callers reading the results on the host with no transfer */
    int32_t *host_idx;
    float *host_wt;
    int *host_err;
    int *host_flag;              /* with host_idx/host_wt: K3K_HFLAG_INTS pinned flags
                                  * (the outputs' flag only with host_err too) */
    /* optional per-stage timing: a ring of event pairs around each stage of a call,
     * harvested only when the ring wraps or the totals are read */
    int prof;
    hipEvent_t ev[K3G_NSTAGE][K3G_RING][2];
    int ev_head[K3G_NSTAGE], ev_used[K3G_NSTAGE];
    double stage_ms[K3G_NSTAGE];
    int64_t stage_n[K3G_NSTAGE];
};

void k3g_stage_begin(K3gCtx *c, int stage, hipStream_t st);
void k3g_stage_end(K3gCtx *c, int stage, hipStream_t st);

/* Stages of k3g_moe, for callers (the drop-in) that must act on the routing between
 * them. idx/wt are device arrays [T][topk]; entries with idx < 0 are skipped. */
int k3g_route(K3gCtx *c, const K3gLayer *L, const float *x, int T, int32_t *idx, float *wt,
              hipStream_t st);
int k3g_experts(K3gCtx *c, const K3gLayer *L, const float *x, int T, const int32_t *idx,
                const float *wt, float *out, hipStream_t st);
/* Make the next k3g_experts wait for `ev` (recorded on another stream) before its routed
 * expert kernels; the shared expert does not wait. */
void k3g_ctx_routed_wait(K3gCtx *c, hipEvent_t ev);
/* The device error word `e`, read back by the caller (c->err): 0 when clean; otherwise
 * reports it, clears it on the device and resets the fused kernel's counters, and
 * returns it (what k3g_sync does after its own read). */
int k3g_err_settle(K3gCtx *c, int e);
/* 1 when k3g_moe runs this layer at T tokens as one fused decode launch (the launch that
 * writes c->host_idx/host_wt/host_err when they are set) */
int k3g_fuses(const K3gCtx *c, const K3gLayer *L, int T);
/* Spin until a running launch sets a pinned host flag (host_flag above): 1 when set, 0 when
 * not within limit_s seconds (a launch cut short by an error, a GPU busy with other work:
 * the caller then waits for the stream instead). */
int k3g_await_flag(const volatile int *flag, double limit_s);
/* The device error word, read back synchronously (-1 when it cannot be read), once the
 * caller has waited for its stream: for callers whose flags did not come */
int k3g_err_read(K3gCtx *c);

#endif /* K3G_CTX_H */
