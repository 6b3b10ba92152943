/* k3g_gemm.hip - the expert products for many tokens (prefill, batched decode) as grouped
 * GEMMs on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16, fp32 accumulation).
 *
 * The engine computes, per (token, slot) pair, three MXFP4 GEMVs per expert in its
 * moe_prefill_chunk loop (src/core/k3_ops.c:668-808); here the pairs are grouped by
 * expert (the stable counting sort of k3g_misc.hip) and each expert's pairs form the
 * columns of one GEMM against that expert's weights:
 *
 *   gate/up  (mode 0):  G = W1 X, U = W3 X  -> h = act(G, U)   (K = hidden)
 *   down     (mode 1):  Y = W2 h            -> contrib rows    (K = inter)
 *
 * The shared expert is the same GEMM over all tokens with a dense column list.
 *
 * Work unit: one workgroup of 8 waves = one (column tile of up to 128 pairs, feature
 * tile) of one expert. Wave w owns 4 row groups of 16 weight rows (mode 0: 32 gate rows
 * and the 32 up rows of the same features, so the activation is lane-local; mode 1: 64
 * output rows) and all the tile's columns: 4 x 8 accumulators of 16x16.
 *
 * Weights (A operand) go from HBM straight to registers in the tiled layouts of
 * k3g_tile.hip: one 16-byte load per lane and row group gives a 16-row x 128-column block
 * of MXFP4, which v_cvt_scalef32_pk_bf16_fp4 turns into four exact bf16 A operands (FP4
 * times a power-of-two scale is a 3-bit significand: bf16 holds it exactly). Tiled bf16
 * weights (the shared expert) load as A operands directly.
 *
 * Activations (B operand) are bf16 PIECES: x (or h) = piece0 + piece1 with piece0 =
 * bf16(v) and piece1 = bf16(v - piece0), 16 significant bits, so the products see the
 * activations to 2^-17 relative. A single bf16 piece of h would cost ~1.7e-3 rel-L2 on
 * the layer output; two cost ~2e-6. When every x is already a bf16 value (piece1 = 0
 * everywhere, recorded in a flag) the gate/up GEMMs skip piece 1: the result is the
 * same. The column tile's activations are staged in LDS, 128 columns x 128 K per piece
 * per stage, two stages, written by global_load_lds_dwordx4 (no register round trip) in a
 * row-XOR-swizzled layout that the B-operand reads (ds_read_b128) hit without bank
 * conflicts. K advances 128 per step: one barrier per step, the next step's weights and
 * activations in flight during the current step's matrix work.
 *
 * Workgroup order: the tiles of one expert are consecutive and every XCD gets one
 * contiguous run of them (blockIdx % 8 is the XCD a workgroup lands on), so the column
 * tiles that share a feature tile's weights, and the feature tiles that share a column
 * tile's activations, meet in one XCD's L2.
 */
#include "k3g_dev.h"
#include "k3g_kernels.h"

typedef float k3v4f __attribute__((ext_vector_type(4)));
typedef __bf16 k3v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 k3v2bf __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void *k3lds;

#define GM_WAVES 8
#define GM_COLS 128                       /* pair columns per tile */
#define GM_KC 128                         /* K per step */
#define GM_PIECE (GM_COLS * GM_KC * 2)    /* bytes of one piece of one stage: 32 KB */
#define GM_STAGE (2 * GM_PIECE)
#define GM_QT 4352                        /* tiled MXFP4 quad tile */

__device__ __forceinline__ int gm_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

/* 8 E2M1 values (one 32-bit word, low nibble first) times 2^(s-127) as bf16, exact */
__device__ __forceinline__ k3v8bf gm_deq8(uint32_t w, float scale)
{
    const k3v2bf a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
    const k3v2bf b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
    const k3v2bf c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
    const k3v2bf d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
    return k3v8bf{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

__device__ __forceinline__ k3v4f gm_mma(k3v8bf a, uint4 b, k3v4f acc)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(k3v8bf, b), acc, 0, 0, 0);
}

__device__ __forceinline__ uint16_t gm_bf16_rn(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float gm_bf16_f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint4 gm_ld16(const void *p)
{
    return *(const uint4 *)p;
}

/* h = act(gate, up) for 4 consecutive features of one column, stored as two bf16 pieces
 * (piece 1 at o + piece) */
__device__ __noinline__ void gm_act_store(k3v4f gt, k3v4f up, float b1, float b2, uint16_t *o,
                                          long long piece)
{
    uint16_t hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float y = k3d_act(gt[i], up[i], b1, b2);
        hi[i] = gm_bf16_rn(y);
        lo[i] = gm_bf16_rn(y - gm_bf16_f(hi[i]));
    }
    uint2 vh, vl;
    vh.x = hi[0] | ((uint32_t)hi[1] << 16); vh.y = hi[2] | ((uint32_t)hi[3] << 16);
    vl.x = lo[0] | ((uint32_t)lo[1] << 16); vl.y = lo[2] | ((uint32_t)lo[3] << 16);
    *(uint2 *)o = vh;
    *(uint2 *)(o + piece) = vl;
}

/* one DMA instruction: 64 lanes x 16 bytes from their own global addresses to 1 KB of
 * LDS at `dst` (lane l at dst + 16 l) */
__device__ __forceinline__ void gm_dma16(const void *src, void *dst)
{
    __builtin_amdgcn_global_load_lds(src, (k3lds)dst, 16, 0, 0);
}

/* s_waitcnt vmcnt(N) (expcnt, lgkmcnt not waited on) */
template <int N>
__device__ __forceinline__ void gm_wait_vm()
{
    static_assert(N >= 0 && N < 16, "vmcnt");
    __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

template <int AF>
__global__ void __launch_bounds__(GM_WAVES * 64, 1)
k_gemm(const K3kGemm g)
{
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * GM_STAGE];

    /* ---- which tile ---------------------------------------------------------------- */
    const int ntl = g.tiles ? *g.ntiles : (g.dense_rows + GM_COLS - 1) / GM_COLS;
    const int N = ntl * g.nft;
    const int per = (N + 7) >> 3;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    if (slot >= per) return;
    const int lam = xcd * per + slot;
    if (lam >= N) return;
    const int tile = lam / g.nft, f = lam - tile * g.nft;
    int e = 0, p0, np;
    if (g.tiles) {
        const int4 t = ((const int4 *)g.tiles)[tile];
        e = t.x; p0 = t.y; np = t.z;
    } else {
        p0 = tile * GM_COLS;
        np = min(GM_COLS, g.dense_rows - p0);
    }
    const int nb = (np + 15) >> 4;                       /* 16-column blocks in use */
    const int npr = (g.npieces > 1 && (!g.lo_flag || *g.lo_flag)) ? 2 : 1;
    const int lane = threadIdx.x & 63;
    const int w = gm_uniform(threadIdx.x >> 6);
    const int K = g.K;
    const int nK = (K + GM_KC - 1) / GM_KC;

    /* ---- this wave's weight rows --------------------------------------------------- */
    /* row group r: matrix base and 16-row block index; valid when inside the matrix */
    const uint8_t *abase[4];
    bool rv[4];
    int orow0;                                            /* first output row (mode 1) or feature (mode 0) */
    {
        const uint8_t *m0, *m1;
        if (AF == 0) {
            const K3ExpertQ *q = g.eq + e;
            m0 = g.mode == 0 ? q->p1 : q->p2;
            m1 = g.mode == 0 ? q->p3 : q->p2;
        } else {
            m0 = (const uint8_t *)g.wa;
            m1 = (const uint8_t *)(g.mode == 0 ? g.wb : g.wa);
        }
        /* bytes per 16-row block */
        const size_t rbb = AF == 0 ? (size_t)((K + 511) / 512) * GM_QT : (size_t)(K / 32) * 1024;
        if (g.mode == 0) {
            orow0 = 256 * f + 32 * w;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = orow0 + 16 * (r & 1);
                rv[r] = orow0 < g.rows;
                abase[r] = (r < 2 ? m0 : m1) + (size_t)(rv[r] ? row / 16 : 0) * rbb;
            }
        } else {
            orow0 = 512 * f + 64 * w;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = orow0 + 16 * r;
                rv[r] = row < g.rows;
                abase[r] = m0 + (size_t)(rv[r] ? row / 16 : 0) * rbb;
            }
        }
    }
    const bool anyv = rv[0] || rv[1] || rv[2] || rv[3];

    /* ---- the activation rows this lane's DMA reads --------------------------------- */
    /* instruction i of wave w fills LDS rows 4 (8 i + w) .. + 3; lane l writes row
     * 4 (8 i + w) + l / 16, physical 16-byte slot l % 16, which holds logical slot
     * (l % 16) ^ (row % 16). row % 16 = (4 w + l / 16) % 16 for every i. */
    const int qoff = 8 * ((lane & 15) ^ ((4 * w + (lane >> 4)) & 15));
    uint32_t boff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 4 * (8 * i + w) + (lane >> 4);
        const int p = p0 + (r < np ? r : 0);
        const int src = (g.mode == 0 && g.perm) ? g.perm[p] / g.topk : p;
        boff[i] = (uint32_t)src * (uint32_t)g.ldb + (uint32_t)qoff;
    }
    const int ndma = gm_uniform((4 * nb + 7 - w) / 8 < 4 ? (4 * nb + 7 - w) / 8 : 4);

    auto dma = [&](int c) {
        uint8_t *st = lds + (c & 1) * GM_STAGE + w * 1024;
        const uint16_t *b0 = g.b + (size_t)c * GM_KC;
        for (int pc = 0; pc < npr; ++pc) {
            const uint16_t *b = b0 + (size_t)pc * g.bpiece;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (i < ndma) gm_dma16(b + boff[i], st + pc * GM_PIECE + i * 8 * 1024);
        }
    };

    k3v4f acc[4][8];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) acc[r][cb] = k3v4f{0.f, 0.f, 0.f, 0.f};

    /* B operand read: column block cb, logical slot q of the step's 16 */
    const int brow = (lane & 15) * 256;
    auto bread = [&](int c, int pc, int cb, int q) -> uint4 {
        const uint8_t *p = lds + (c & 1) * GM_STAGE + pc * GM_PIECE + cb * 16 * 256 + brow +
                           16 * (q ^ (lane & 15));
        return *(const uint4 *)p;
    };
    const int g4 = lane >> 4;

    if (AF == 0) {
        /* ------------------------------------------------ MXFP4 weights ---------- */
        uint4 ar[4];
        uint32_t sw[4];
        auto aload = [&](int c, uint4 *dst, uint32_t *sdst) {
            const size_t qo = (size_t)(c >> 2) * GM_QT;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint8_t *t = abase[r] + qo;
                dst[r] = gm_ld16(t + 1024 * (c & 3) + 16 * lane);
                if ((c & 3) == 0) sdst[r] = *(const uint32_t *)(t + 4096 + 4 * lane);
            }
        };
        aload(0, ar, sw);
        dma(0);
        for (int c = 0; c < nK; ++c) {
            gm_wait_vm<0>();
            __syncthreads();
            uint4 cur[4];
            uint32_t scl[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) { cur[r] = ar[r]; scl[r] = sw[r]; }
            if (c + 1 < nK) {
                aload(c + 1, ar, sw);
                dma(c + 1);
            }
            const int j = c & 3;
            float sc[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) sc[r] = k3d_e8m0((scl[r] >> (8 * j)) & 0xffu);
            if (anyv) {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    k3v8bf a[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint32_t wd = s == 0 ? cur[r].x : s == 1 ? cur[r].y
                                          : s == 2 ? cur[r].z : cur[r].w;
                        a[r] = gm_deq8(wd, sc[r]);
                    }
                    const int q = 4 * g4 + s;
#pragma unroll
                    for (int cb = 0; cb < 8; ++cb) {
                        if (cb < nb) {
                            for (int pc = 0; pc < npr; ++pc) {
                                const uint4 bv = bread(c, pc, cb, q);
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    if (rv[r]) acc[r][cb] = gm_mma(a[r], bv, acc[r][cb]);
                            }
                        }
                    }
                }
            }
        }
    } else {
        /* ------------------------------------------------ bf16 weights ----------- */
        /* A operands per (step, sub-step): 4 row groups x 16 bytes; a ring of 4
         * sub-steps, loaded two sub-steps ahead */
        const int nC32 = K / 32;
        uint4 ring[4][4];
        auto aload = [&](int c, int s, uint4 *dst) {
            const int c32 = 4 * c + s;
            const int cc = c32 < nC32 ? c32 : nC32 - 1;
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[r] = gm_ld16(abase[r] + (size_t)cc * 1024 + 16 * lane);
        };
        dma(0);
        aload(0, 0, ring[0]);
        aload(0, 1, ring[1]);
        for (int c = 0; c < nK; ++c) {
            /* DMA(c) was followed by the loads of sub-steps (c,0) and (c,1): 8 loads */
            gm_wait_vm<8>();
            __syncthreads();
            if (c + 1 < nK) dma(c + 1);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                /* sub-step s + 2 (wrapping into the next step) */
                const int s2 = (s + 2) & 3;
                const int c2 = c + ((s + 2) >> 2);
                aload(c2 < nK ? c2 : nK - 1, s2, ring[s2]);
                const bool live = 4 * c + s < nC32;
                if (anyv && live) {
                    k3v8bf a[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) a[r] = __builtin_bit_cast(k3v8bf, ring[s][r]);
                    const int q = 4 * s + g4;
#pragma unroll
                    for (int cb = 0; cb < 8; ++cb) {
                        if (cb < nb) {
                            for (int pc = 0; pc < npr; ++pc) {
                                const uint4 bv = bread(c, pc, cb, q);
#pragma unroll
                                for (int r = 0; r < 4; ++r)
                                    if (rv[r]) acc[r][cb] = gm_mma(a[r], bv, acc[r][cb]);
                            }
                        }
                    }
                }
            }
        }
        gm_wait_vm<0>();
    }

    /* ---- epilogue -------------------------------------------------------------------- */
    const int col0 = lane & 15;
    if (g.mode == 0) {
        if (!rv[0]) return;
        const int n = orow0 + 4 * g4;
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) {
            const int col = 16 * cb + col0;
            if (cb < nb && col < np) {
                uint16_t *o = g.h + (size_t)(p0 + col) * g.ldh + n;
                gm_act_store(acc[0][cb], acc[2][cb], g.b1, g.b2, o, g.hpiece);
                gm_act_store(acc[1][cb], acc[3][cb], g.b1, g.b2, o + 16, g.hpiece);
            }
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (!rv[r]) continue;
            const int orow = orow0 + 16 * r + 4 * g4;
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) {
                const int col = 16 * cb + col0;
                if (cb < nb && col < np) {
                    const int p = p0 + col;
                    const int dst = g.scatter ? g.perm[p] : p;
                    *(k3v4f *)(g.out + (size_t)dst * g.ldo + orow) = acc[r][cb];
                }
            }
        }
    }
}

/* ------------------------------------------------------------------ helpers ------ */
/* Column tiles of up to 128 pairs per active expert, in expert order; also clears the
 * flag the activation pieces raise. One block of 1024 threads (n_experts <= 1024). */
__global__ void __launch_bounds__(1024)
k_gemm_tiles(const int32_t *__restrict__ off, int E, int4 *__restrict__ tiles,
             int32_t *__restrict__ ntiles, int32_t *__restrict__ flag)
{
    __shared__ int s[1024];
    const int e = threadIdx.x;
    const int cnt = e < E ? off[e + 1] - off[e] : 0;
    const int nt = (cnt + GM_COLS - 1) / GM_COLS;
    s[e] = nt;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        const int v = e >= d ? s[e - d] : 0;
        __syncthreads();
        s[e] += v;
        __syncthreads();
    }
    const int first = s[e] - nt;
    for (int i = 0; i < nt; ++i) {
        const int p0 = off[e] + GM_COLS * i;
        tiles[first + i] = make_int4(e, p0, min(GM_COLS, off[e + 1] - p0), 0);
    }
    if (e == 1023) { *ntiles = s[1023]; *flag = 0; }
}

/* x (fp32 [T][d]) -> two bf16 pieces [2][T][ldb]; raises *flag when any piece 1 is not
 * zero. The padding columns d..ldb are never written (the workspace starts zeroed). */
__global__ void __launch_bounds__(256)
k_xpieces(const float *__restrict__ x, int T, int d, int ldb, uint16_t *__restrict__ xb,
          long long piece, int32_t *__restrict__ flag)
{
    const size_t n = (size_t)T * d;
    bool nz = false;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t t = i / d, c = i - t * d;
        const float v = x[i];
        const uint16_t hi = gm_bf16_rn(v);
        const uint16_t lo = gm_bf16_rn(v - gm_bf16_f(hi));
        xb[t * ldb + c] = hi;
        xb[piece + t * ldb + c] = lo;
        nz |= lo != 0;
    }
    if (__any(nz) && (threadIdx.x & 63) == 0) *flag = 1;
}

/* ------------------------------------------------------------------ launchers ---- */
extern "C" int k3k_gemm_tiles(const int32_t *off, int E, int32_t *tiles, int32_t *ntiles,
                              int32_t *flag, hipStream_t st)
{
    if (E < 1 || E > 1024) return -1;
    hipLaunchKernelGGL(k_gemm_tiles, dim3(1), dim3(1024), 0, st, off, E, (int4 *)tiles, ntiles,
                       flag);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int k3k_xpieces(const float *x, int T, int d, int ldb, uint16_t *xb,
                           long long piece, int32_t *flag, hipStream_t st)
{
    if (T < 1 || d < 1 || ldb < d) return -1;
    const size_t n = (size_t)T * d;
    const int blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    hipLaunchKernelGGL(k_xpieces, dim3(blocks), dim3(256), 0, st, x, T, d, ldb, xb, piece, flag);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int k3k_gemm(const K3kGemm *g, hipStream_t st)
{
    /* shapes the kernel's indexing assumes */
    if (g->mode < 0 || g->mode > 1 || g->afmt < 0 || g->afmt > 1) return -1;
    if (g->K < 32 || g->K % 32 || g->rows < 16 || g->ldb < g->K || g->ldb % GM_KC ||
        g->npieces < 1 || g->npieces > 2 || !g->b || g->nft < 1)
        return -1;
    if (g->mode == 0 && (g->rows % 32 || g->nft * 256 < g->rows || !g->h || g->ldh < g->rows))
        return -1;
    if (g->mode == 1 && (g->rows % 16 || g->nft * 512 < g->rows || !g->out || g->ldo < g->rows ||
                         g->ldo % 4))
        return -1;
    if (g->afmt == 0 && !g->eq) return -1;
    if (g->afmt == 1 && (!g->wa || (g->mode == 0 && !g->wb))) return -1;
    if (g->tiles ? (!g->ntiles || g->max_tiles < 1) : g->dense_rows < 1) return -1;
    if ((g->scatter || (g->mode == 0 && g->tiles)) && !g->perm) return -1;
    const long long maxt = g->tiles ? g->max_tiles : (g->dense_rows + GM_COLS - 1) / GM_COLS;
    const long long nwg = maxt * g->nft;
    const long long grid = 8 * ((nwg + 7) / 8);
    if (grid > 0x7fffffff) return -1;
    if (g->afmt == 0)
        hipLaunchKernelGGL(k_gemm<0>, dim3((unsigned)grid), dim3(GM_WAVES * 64), 0, st, *g);
    else
        hipLaunchKernelGGL(k_gemm<1>, dim3((unsigned)grid), dim3(GM_WAVES * 64), 0, st, *g);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
