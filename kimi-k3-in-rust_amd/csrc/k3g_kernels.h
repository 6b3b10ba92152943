/* k3g_kernels.h - launchers of the gfx950 kernels, callable from the C99 host code.
 * Every launcher enqueues on the given stream and returns 0, or -1 when the arguments
 * are outside what the kernel supports (nothing is launched then). */
#ifndef K3G_KERNELS_H
#define K3G_KERNELS_H

#include <stdint.h>
#ifndef __HIPCC__
#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#endif
#include <hip/hip_runtime_api.h>

#include "../../include/k3moe.h"

#ifdef __cplusplus
extern "C" {
#endif

#define K3G_MAX_TOPK 64

/* The grouped GEMMs deal consecutive column tiles to one XCD in groups of this many (an
 * expert's full tiles are consecutive, so they run at once on one XCD and share its
 * weights in that L2); K3G_TILE_ROUNDS(n) is the rounds of workgroups per XCD for up to n
 * column tiles. */
#define K3G_TILE_GROUP 4
#define K3G_TILE_ROUNDS(n) (K3G_TILE_GROUP * (((n) + 8 * K3G_TILE_GROUP - 1) / (8 * K3G_TILE_GROUP)))

/* weight formats */
enum { K3K_MXFP4 = 0, K3K_F32 = 1, K3K_BF16 = 2,
       K3K_I8R = 3 };    /* K3K_I8R: rows of [f32 scale][int8 x in] (the engine's K3_WI8) */

/* Everything the routed-expert kernels read, device pointers. */
typedef struct {
    int fmt;                          /* K3K_MXFP4: eq table; K3K_F32: w1/w3/w2 bank */
    const K3ExpertQ *eq;              /* [n_experts] */
    const float *w1, *w3, *w2;        /* [n_experts][inter][latent], [..][latent][inter] */
    const int32_t *act, *nact;        /* active experts, ascending, and their count */
    const int32_t *off;               /* [n_experts + 1] pair ranges per expert */
    const int32_t *perm;              /* pair ids p = t*topk + j, grouped by expert */
    int topk, inter, latent;
    const float *z;                   /* [T][latent] routed input */
    float *h;                         /* [T*topk][inter] after the activation */
    float *contrib;                   /* [T*topk][latent] per-slot expert outputs */
    float b1, b2;                     /* SiTU caps (>= 2^64: uncapped) */
    int *err;
} K3kRouted;

/* The fused decode kernel (k3g_decode.hip): the whole Kimi-K2-shaped layer for T <= 4
 * tokens in one persistent launch, on experts in the tiled MXFP4 layout and a shared
 * expert in the tiled bf16 layout (k3g_tile.hip). */
typedef struct {
    int T, d, E, k, I, SI;
    int renorm;
    float routed_scale, b1, b2;
    const float *gate, *bias;
    const K3ExpertQ *eq;          /* p1/p3/p2: tiled MXFP4 w1, w3, w2; s* unused */
    const uint16_t *sh1, *sh3, *sh2;   /* tiled bf16 */
    const float *x;
    float *out;
    int32_t *idx;
    float *wt;
    float *rs;                    /* [T][E][4] router {choice, lo, hi, score} */
    double *rpart;                /* [T][E][K3G_KS_R][2] router slice sums */
    uint8_t *xq8;                 /* [T][ceil(d/512)][8448]: x's FP8 pieces, B layout */
    uint16_t *xq16;               /* [d/32][64][8]: x's bf16 pieces, column 3t + piece */
    float *gpart;                 /* [T*k][K3G_KS_G_MAX][2][I] routed gate/up partial sums */
    uint8_t *hq8;                 /* [T*k][ceil(I/512)][8448]: h's FP8 pieces */
    float *sgpart;                /* [K3G_KS_SG][T][2][SI] shared gate/up partial sums */
    uint16_t *hq16;               /* [SI/32][64][8]: shared h's bf16 pieces */
    float *contrib;               /* [T*k][K3G_KS_D][d] per-slot expert output slices */
    float *shpart;                /* [K3G_KS_SD][T][d] shared down partial sums */
    int *sync;                    /* this call's counter bank, all zero */
    int *sync_clear;              /* the other bank, zeroed by this call for the next */
    int sync_words;               /* ints per bank */
    int *err, *stats;
    int force;
    int given;                    /* 1: idx/wt hold the routing already (entries < 0 are
                                   * left out); the router tickets do nothing */
    long long spin_limit;
    unsigned long long *trace;    /* optional: [ticket][2] start/end wall-clock stamps */
    /* the LatentMoE layer (Kimi-K3: src/core/k3_ops.c:556-656): L != d turns on the latent
     * projections. The routed experts then run on z = down x (width L), their slot-order
     * aggregate (width L) is RMSNorm-ed with lnorm (when given) and projected back by up,
     * and the shared expert's output is added to that. L == d: the Kimi-K2 shape, none of
     * the fields below is read. */
    int L;
    const uint16_t *down, *up;    /* tiled bf16 [L][d] and [d][L] */
    const float *lnorm;           /* [L], or NULL: no RMSNorm of the aggregate */
    float rms_eps;
    float *zpart;                 /* [K3G_KS_LD][T][L] latent down partial sums */
    uint8_t *zq8;                 /* [T][ceil(L/512)][8448]: z's FP8 pieces, B layout */
    float *accl;                  /* [T][L] the routed experts' slot-order aggregate */
    double *nss;                  /* [T][L/32] the aggregate's sums of squares per 32 rows */
    uint16_t *aq16;               /* [L/32][64][8]: the normalised aggregate's bf16 pieces */
    float *upart;                 /* [K3G_KS_LU][T][d] latent up partial sums */
    /* Optional copies in pinned host memory, for a caller that reads the results on the
     * host with no transfer after the launch (out may then be pinned host memory too):
     * hidx/hwt the routing [T][k] once published; with hflag, herr the error word as it
     * stands when the outputs are complete (the caller zeroes *herr before the launch). */
    int32_t *hidx;
    float *hwt;
    int *herr;
    /* With hidx/hwt: pinned host flags the caller zeroes before the launch and may poll
     * while it runs: [K3K_HFLAG_ROUTED] set once hidx/hwt are complete; with herr as well,
     * [K3K_HFLAG_DONE] once out (then written through to memory) and herr are. A launch
     * cut short by an error may never set them: the caller then waits for the stream and
     * reads the device error word itself. */
    int *hflag;
} K3kDecode;

#define K3K_HFLAG_ROUTED 0
#define K3K_HFLAG_DONE 16     /* a separate 64-byte line */
#define K3K_HFLAG_INTS 32

/* One grouped GEMM on the bf16 matrix cores (k3g_gemm.hip). Columns are (token, slot)
 * pairs grouped by expert (tiles) or all tokens (dense, the shared expert). */
typedef struct {
    int mode;                 /* 0: gate/up + activation -> h pieces; 1: down -> fp32 rows */
    int afmt;                 /* 0: tiled MXFP4 per expert (eq); 1: tiled bf16 (wa, wb) */
    int rows;                 /* output rows of one weight matrix: inter (mode 0), hidden (1) */
    int K;                    /* reduction length */
    int ldb;                  /* row stride of the B pieces (elements), K rounded up to 128 */
    const K3ExpertQ *eq;      /* mode 0: p1, p3; mode 1: p2 (tiled MXFP4) */
    const uint16_t *wa, *wb;  /* tiled bf16: mode 0 gate, up; mode 1 down */
    const uint16_t *b;        /* B pieces, piece p at b + p * bpiece */
    long long bpiece;
    const int32_t *perm;      /* sorted position -> pair id (t * topk + j) */
    int topk;
    const int32_t *tiles;     /* {expert, first sorted position, count, 0}; NULL: dense */
    const int32_t *ntiles;
    int max_tiles;            /* bound on *ntiles (grid size) */
    int dense_rows;           /* dense: the column count (tokens) */
    int npieces;              /* B pieces, 1 or 2 */
    const int32_t *lo_flag;   /* piece 1 only when *lo_flag != 0 (NULL: always) */
    uint16_t *h;              /* mode 0 out: [2][columns][ldh] bf16 pieces */
    long long hpiece;
    int ldh;
    float b1, b2;             /* activation caps */
    float *out;               /* mode 1 out: row per column, stride ldo */
    int ldo;
    int scatter;              /* mode 1: out row = perm[column] (else the column) */
    int nft;                  /* feature tiles: ceil(rows / 256) (mode 0), / 512 (mode 1) */
    /* MXFP8 activations (k3k_gemm_f8, MXFP4 weights only): E4M3 bytes [rows][ldb] and
     * E8M0 block scales [rows][ldb / 32]; mode 0 writes h the same way to hq/hs */
    const uint8_t *bq, *bs;
    uint8_t *hq, *hs;
    int ldhq;                 /* bytes per h row (scales: ldhq / 32) */
    /* k3k_gemm with MXFP4 weights: h as bf16 piece 0 (h, b) plus its remainder
     * h - bf16(h) as MXFP8 (mode 0 writes hq/hs, mode 1 reads bq/bs; row stride ldhq bytes)
     * on the scaled FP8 matrix cores; mode 1 then takes npieces = 1 */
    int hmix;
    int np_only;              /* set by k3k_gemm: 2 = a launch that runs only two-piece B */
    /* dense tiled-bf16 GEMMs only: K cut into ksplit slices of whole 128-column steps
     * (1: none); the slices' fp32 sums go to part ([ksplit][columns][2][rows] gate/up,
     * [ksplit][columns][rows] down) and k3k_gemm reduces them in slice order */
    int ksplit;
    float *part;
    /* instrumentation (NULL: off): per workgroup of the launch that does the work, wave
     * 0's start and end (wall clock), tile << 32 | feature tile, XCC << 32 | HW_ID */
    unsigned long long *trace;
} K3kGemm;

int k3k_gemm(const K3kGemm *g, hipStream_t st);
/* The K slices a dense GEMM of nft feature tiles x ntl column tiles over K columns uses
 * to give the GPU about 256 workgroups (1 = no split), and the part buffer bytes a
 * context needs for any column count (rows: the GEMM's output rows; x2 for gate/up). */
int k3k_gemm_ksplit(int nft, int ntl, int K);
size_t k3k_gemm_part_bytes(int nft, int rows2);
/* The same grouped GEMM on v_mfma_scale_f32_16x16x128_f8f6f4: MXFP4 weights as they are,
 * activations in MXFP8 (bq/bs; mode 0 quantises h to hq/hs). */
int k3k_gemm_f8(const K3kGemm *g, hipStream_t st);
/* x -> MXFP8 (OCP MX: block scale 2^(floor(log2 amax) - 8), E4M3 nearest-even, clamped
 * to +-448): bytes [T][ldq], scales [T][ldq / 32]; the padding columns stay zero. */
int k3k_xq8(const float *x, int T, int d, int ldq, uint8_t *xq, uint8_t *xs, hipStream_t st);
/* column tiles from the dispatch's per-expert ranges; clears *flag */
int k3k_gemm_tiles(const int32_t *off, int E, int32_t *tiles, int32_t *ntiles,
                   int32_t *flag, hipStream_t st);
/* x -> bf16 pieces [2][T][ldb]; *flag = 1 when some piece 1 is not zero */
int k3k_xpieces(const float *x, int T, int d, int ldb, uint16_t *xb, long long piece,
                int32_t *flag, hipStream_t st);

/* K slices of the fused kernel's ticket classes (fewer when K is short); each may be set
 * at build time (-DK3G_KS_SG=...) */
#ifndef K3G_KS_G
#define K3G_KS_G 7                /* routed gate/up: over 512-column quads of d */
#endif
#ifndef K3G_KS_G_LAT
#define K3G_KS_G_LAT 2            /* the same in the latent layer (quads of L): its 16 slots
                                   * x L/32 row tiles are many tickets already */
#endif
#define K3G_KS_G_MAX (K3G_KS_G > K3G_KS_G_LAT ? K3G_KS_G : K3G_KS_G_LAT)
#ifndef K3G_KS_SG
#define K3G_KS_SG 7               /* shared gate/up: over 32-column chunks of d */
#endif
#ifndef K3G_KS_SD
#define K3G_KS_SD 2               /* shared down: over 32-column chunks of SI */
#endif
#ifndef K3G_KS_R
#define K3G_KS_R 4                /* router: over 1024-column chunks of d */
#endif
#ifndef K3G_KS_D
#define K3G_KS_D 2                /* routed down: over 512-column quads of I */
#endif
#ifndef K3G_KS_LD
#define K3G_KS_LD 7               /* latent down: over 32-column chunks of d */
#endif
#ifndef K3G_KS_LU
#define K3G_KS_LU 8               /* latent up: over 32-column chunks of L */
#endif
/* the shared gate/up, shared down, router and routed down slices of the latent layer
 * (default: as the plain layer's) */
#ifndef K3G_KS_SG_LAT
#define K3G_KS_SG_LAT K3G_KS_SG
#endif
#ifndef K3G_KS_SD_LAT
#define K3G_KS_SD_LAT K3G_KS_SD
#endif
#ifndef K3G_KS_R_LAT
#define K3G_KS_R_LAT K3G_KS_R
#endif
#ifndef K3G_KS_D_LAT
#define K3G_KS_D_LAT K3G_KS_D
#endif
#define K3G_KS_MAX2(a, b) ((a) > (b) ? (a) : (b))
#define K3G_KS_SG_MAX K3G_KS_MAX2(K3G_KS_SG, K3G_KS_SG_LAT)
#define K3G_KS_SD_MAX K3G_KS_MAX2(K3G_KS_SD, K3G_KS_SD_LAT)
#define K3G_KS_R_MAX K3G_KS_MAX2(K3G_KS_R, K3G_KS_R_LAT)
#define K3G_KS_D_MAX K3G_KS_MAX2(K3G_KS_D, K3G_KS_D_LAT)
#define K3G_DEC_WAVES_PER_EU 4

/* bytes of counters and tickets per call of the fused kernel at this shape */
size_t k3k_decode_sync_bytes(int T, int d, int E, int k, int I, int SI, int L);
int k3k_decode_tickets(int T, int d, int E, int k, int I, int SI, int L);
int k3k_decode_fused(const K3kDecode *a, hipStream_t st);

/* Repack into the tiled layouts (k3g_tile.hip). Sizes are 0 for unsupported shapes. */
size_t k3k_tiled_mxfp4_bytes(int rows, int cols);
size_t k3k_tiled_bf16_bytes(int rows, int cols);
int k3k_tile_mxfp4(uint8_t *dst, const uint8_t *packed, const uint8_t *scales, int rows,
                   int cols, hipStream_t st);
int k3k_tile_bf16(uint16_t *dst, const uint16_t *src, int rows, int cols, hipStream_t st);

/* rs: [T][E] float4 {choice, lo, hi, score} workspace */
int k3k_router(const float *x, int T, const float *W, const float *bias, int d, int E,
               int k, int renorm, float routed_scale, float *rs, int32_t *idx, float *wt,
               int force, int *stats, double *part, int32_t *ctr, float *bpart,
               size_t bpart_floats, const int32_t *x1flag, hipStream_t st);
/* bytes of the part buffer k3k_router's sliced logits use (ctr: 512 zeroed 128-byte
 * lines, 16384 ints) */
size_t k3k_router_part_bytes(void);
/* floats of the bpart buffer the bounded bf16 logits of T tokens use (0: not taken) */
size_t k3k_router_bf3_floats(int T, int E);

/* Stable counting sort of the T*k (token, slot) pairs by expert. cnt is [ceil(P/256)][E]
 * ints of workspace, base [ceil(P/256) + 1][E] (the experts' totals in its last row). */
int k3k_dispatch(const int32_t *idx, int P, int E, int32_t *cnt, int32_t *base,
                 int32_t *off, int32_t *act, int32_t *nact, int32_t *perm, int *err,
                 hipStream_t st);
/* The same, followed by the grouped GEMMs' column tiles (as k3k_gemm_tiles), in one
 * launch when P <= 4096. */
int k3k_dispatch_tiles(const int32_t *idx, int P, int E, int32_t *cnt, int32_t *base,
                       int32_t *off, int32_t *act, int32_t *nact, int32_t *perm, int *err,
                       int32_t *tiles, int32_t *ntiles, int32_t *flag, hipStream_t st);

/* h = act(W1 z, W3 z) and contrib = W2 h for every active expert's pairs. maxU bounds
 * the number of active experts (min(E, T*k)); maxtok bounds tokens per expert. */
int k3k_routed_gateup(const K3kRouted *a, int maxU, int maxtok, hipStream_t st);
int k3k_routed_down(const K3kRouted *a, int maxU, int maxtok, hipStream_t st);

/* y[t][r] = W[r] . x[t] (fmt K3K_F32, K3K_BF16 or K3K_I8R), or with Wb != NULL
 * y[t][r] = act(Wa[r] . x[t], Wb[r] . x[t]). */
int k3k_dense(int fmt, const void *Wa, const void *Wb, int rows, int in,
              const float *x, int ldx, int T, float *y, int ldy, float b1, float b2,
              hipStream_t st);

/* out[t] = sum_j wt[t][j] * contrib[t*k+j] in slot order (float multiply, then add;
 * slots with idx < 0 skipped), then + add[t] when add != NULL. */
int k3k_combine(const float *contrib, const int32_t *idx, const float *wt, int T, int k,
                int n, const float *add, float *out, hipStream_t st);

/* Write table[e[i]] = q[i] for i < n (device expert tables updated from host-side
 * decisions without a host staging buffer: the entries travel as kernel arguments). */
#define K3K_EQSET 64
typedef struct {
    int n;
    int e[K3K_EQSET];
    K3ExpertQ q[K3K_EQSET];
} K3kEqSet;
int k3k_set_experts(K3ExpertQ *table, const K3kEqSet *s, hipStream_t st);

/* y = w * x * (float)(1/sqrt(sum x^2 / n + eps)), double sum; one token per block. */
int k3k_rmsnorm(float *y, const float *x, const float *w, int n, int T, float eps,
                hipStream_t st);

/* *p = v, in stream order */
int k3k_set_i32(int32_t *p, int32_t v, hipStream_t st);

/* y += a, elementwise */
int k3k_add(float *y, const float *a, size_t n, hipStream_t st);

/* Per token (rows of n): h += a when a is given (stored back), then y = RMSNorm(h) * w
 * when w is given (k3k_rmsnorm's arithmetic); y may alias h. */
int k3k_add_rmsnorm(float *h, const float *a, float *y, const float *w, int n, int T, float eps,
                    hipStream_t st);

/* dst <- src, n bytes, by a kernel on the stream (16-byte aligned pointers; either side may
 * be pinned host memory). -1 on misaligned pointers. */
int k3k_copy(void *dst, const void *src, size_t n, hipStream_t st);

/* MXFP4 -> fp32, exact (k3_mxfp4_dequant semantics). */
int k3k_dequant(float *out, const uint8_t *packed, const uint8_t *scales, int rows,
                int pcols, int group, hipStream_t st);

/* y[rows] = W x for one MXFP4 matrix (group 32), any even `in`. */
int k3k_mxfp4_gemv(float *y, const float *x, const uint8_t *packed, const uint8_t *scales,
                   int in, int rows, int group, hipStream_t st);

int k3k_fill_bytes(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream, uint64_t first,
                   hipStream_t st);
int k3k_fill_scales(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream,
                    uint64_t first, int lo, int hi, hipStream_t st);

#ifdef __cplusplus
}
#endif

#endif /* K3G_KERNELS_H */
