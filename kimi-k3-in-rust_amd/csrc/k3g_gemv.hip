/* k3g_gemv.hip - matrix-vector kernels for decode-sized token counts.
 *
 * Layout of the work. A wave owns a tile of rows and walks the row's columns in blocks
 * of 1024: lane l holds columns [16l, 16l+16) of the block, so one block of one row is
 * a single coalesced 512 B read of MXFP4 (8 B per lane plus one scale byte), 2 KB of
 * bf16 or 4 KB of fp32. The lane's slice of x stays in registers for every row of the
 * tile, each lane keeps one fp32 partial per (row, token), and a transposed reduction
 * leaves one finished output per lane at the end. The weights are read once per
 * launch; x and the partial sums never touch LDS.
 *
 * MXFP4 decode is gfx950's v_cvt_scalef32_pk_f32_fp4, which applies the E8M0 scale
 * exactly, so every product is the same value the engine's exact dequantisation gives;
 * accumulation is fp32 fused multiply-add.
 */
#include "k3g_dev.h"
#include "k3g_kernels.h"

#define K3G_CB 1024   /* columns per block: 64 lanes x 16 */

/* 16 consecutive weights of a row starting at column col (col % 16 == 0). */
template <int FMT>
__device__ __forceinline__ void k3d_load16(const void *row, const uint8_t *srow, int col,
                                           float *w)
{
    if constexpr (FMT == K3K_MXFP4) {
        const uint2 q = *(const uint2 *)((const uint8_t *)row + (col >> 1));
        const float sc = k3d_e8m0(srow[col >> 5]);
        k3d_fp4x8(q.x, sc, w);
        k3d_fp4x8(q.y, sc, w + 8);
    } else if constexpr (FMT == K3K_F32) {
        const float4 *p = (const float4 *)((const float *)row + col);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = p[i];
            w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        }
    } else {
        const uint4 *p = (const uint4 *)((const uint16_t *)row + col);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint4 v = p[i];
            w[8 * i + 0] = k3d_bf16lo(v.x); w[8 * i + 1] = k3d_bf16hi(v.x);
            w[8 * i + 2] = k3d_bf16lo(v.y); w[8 * i + 3] = k3d_bf16hi(v.y);
            w[8 * i + 4] = k3d_bf16lo(v.z); w[8 * i + 5] = k3d_bf16hi(v.z);
            w[8 * i + 6] = k3d_bf16lo(v.w); w[8 * i + 7] = k3d_bf16hi(v.w);
        }
    }
}

/* Row r of a matrix with `in` columns, in the given format. */
template <int FMT>
__device__ __forceinline__ const void *k3d_row(const void *base, int r, int in)
{
    if constexpr (FMT == K3K_MXFP4) return (const uint8_t *)base + (size_t)r * (in >> 1);
    else if constexpr (FMT == K3K_F32) return (const float *)base + (size_t)r * in;
    else return (const uint16_t *)base + (size_t)r * in;
}

__device__ __forceinline__ const uint8_t *k3d_srow(const uint8_t *s, int r, int in)
{
    return s ? s + (size_t)r * ((in + 31) >> 5) : nullptr;
}

/* 16 consecutive x values of token row xr at column col, or zeros. */
__device__ __forceinline__ void k3d_x16(const float *xr, int col, float *xv)
{
    if (xr) {
        const float4 *p = (const float4 *)(xr + col);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = p[i];
            xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) xv[i] = 0.0f;
    }
}

template <int V>
struct K3Log2 { static constexpr int v = 1 + K3Log2<V / 2>::v; };
template <>
struct K3Log2<1> { static constexpr int v = 0; };

/* Accumulator type: fp32 for the streamed formats (MXFP4, bf16), double for fp32
 * weights, whose products are exact in double as in the engine's fixture path. */
template <int FMT> struct K3Acc { typedef float T; };
template <> struct K3Acc<K3K_F32> { typedef double T; };

__device__ __forceinline__ float k3d_fma(float w, float x, float a) { return fmaf(w, x, a); }
__device__ __forceinline__ double k3d_fma(float w, float x, double a)
{
    return fma((double)w, (double)x, a);
}

/* Tile core: NRT rows (rows[] pointers, NULL = out of range) x NT tokens (xr[] rows,
 * NULL = absent), accumulated into acc[r*NT + t] over all column blocks. */
template <int FMT, int NRT, int NT, typename A>
__device__ __forceinline__ void k3d_tile(const void *const *rows, const uint8_t *const *srows,
                                         const float *const *xr, int in, int lane,
                                         A *acc)
{
#pragma unroll
    for (int i = 0; i < NRT * NT; ++i) acc[i] = (A)0;
    for (int cb = 0; cb < in; cb += K3G_CB) {
        const int col = cb + lane * 16;
        if (col >= in) continue;
        float xv[NT][16];
#pragma unroll
        for (int t = 0; t < NT; ++t) k3d_x16(xr[t], col, xv[t]);
#pragma unroll
        for (int r = 0; r < NRT; ++r) {
            if (!rows[r]) continue;
            float w[16];
            k3d_load16<FMT>(rows[r], srows[r], col, w);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                A a = acc[r * NT + t];
#pragma unroll
                for (int i = 0; i < 16; ++i) a = k3d_fma(w[i], xv[t][i], a);
                acc[r * NT + t] = a;
            }
        }
    }
}

/* ------------------------------------------------------------ routed experts ---- */
/* grid (ceil(inter / (4*NR)), maxU), block 256: wave w of block b owns gate rows and
 * up rows [row0, row0 + NR) of active expert blockIdx.y, for its tokens NT at a time. */
template <int FMT, int NR, int NT>
__global__ void __launch_bounds__(256)
k_routed_gateup(K3kRouted a)
{
    const int u = blockIdx.y;
    if (u >= *a.nact) return;
    const int e = a.act[u];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int I = a.inter, L = a.latent;
    const int row0 = (blockIdx.x * 4 + wave) * NR;
    if (row0 >= I) return;

    const void *Wg, *Wu;
    const uint8_t *Sg = nullptr, *Su = nullptr;
    if constexpr (FMT == K3K_MXFP4) {
        const K3ExpertQ q = a.eq[e];
        Wg = q.p1; Wu = q.p3; Sg = q.s1; Su = q.s3;
    } else {
        Wg = a.w1 + (size_t)e * I * L;
        Wu = a.w3 + (size_t)e * I * L;
    }
    const void *rows[2 * NR];
    const uint8_t *srows[2 * NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const bool ok = row0 + r < I;
        rows[r] = ok ? k3d_row<FMT>(Wg, row0 + r, L) : nullptr;
        rows[NR + r] = ok ? k3d_row<FMT>(Wu, row0 + r, L) : nullptr;
        srows[r] = ok ? k3d_srow(Sg, row0 + r, L) : nullptr;
        srows[NR + r] = ok ? k3d_srow(Su, row0 + r, L) : nullptr;
    }

    constexpr int V = 2 * NR * NT;
    constexpr int SH = 6 - K3Log2<V>::v;
    const int beg = a.off[e], end = a.off[e + 1];
    for (int c0 = beg; c0 < end; c0 += NT) {
        int pr[NT];
        const float *xr[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            pr[t] = c0 + t < end ? a.perm[c0 + t] : -1;
            xr[t] = pr[t] >= 0 ? a.z + (size_t)(pr[t] / a.topk) * L : nullptr;
        }
        typename K3Acc<FMT>::T acc[V];
        k3d_tile<FMT, 2 * NR, NT>(rows, srows, xr, L, lane, acc);
        k3d_transpose_reduce<V>(acc, lane);
        const float gv = (float)acc[0];
        const float upv = __shfl_xor(gv, 32, K3G_WAVE);
        const int v = lane >> SH;
        if ((lane & ((1 << SH) - 1)) == 0 && v < NR * NT) {
            const int r = v / NT, t = v % NT;
            int p = -1;
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) if (tt == t) p = pr[tt];
            if (row0 + r < I && p >= 0)
                a.h[(size_t)p * I + row0 + r] = k3d_act(gv, upv, a.b1, a.b2);
        }
    }
}

/* grid (ceil(latent / (4*NR)), maxU): wave owns W2 rows [row0, row0+NR). */
template <int FMT, int NR, int NT>
__global__ void __launch_bounds__(256)
k_routed_down(K3kRouted a)
{
    const int u = blockIdx.y;
    if (u >= *a.nact) return;
    const int e = a.act[u];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int I = a.inter, L = a.latent;
    const int row0 = (blockIdx.x * 4 + wave) * NR;
    if (row0 >= L) return;

    const void *W;
    const uint8_t *S = nullptr;
    if constexpr (FMT == K3K_MXFP4) {
        const K3ExpertQ q = a.eq[e];
        W = q.p2; S = q.s2;
    } else {
        W = a.w2 + (size_t)e * L * I;
    }
    const void *rows[NR];
    const uint8_t *srows[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const bool ok = row0 + r < L;
        rows[r] = ok ? k3d_row<FMT>(W, row0 + r, I) : nullptr;
        srows[r] = ok ? k3d_srow(S, row0 + r, I) : nullptr;
    }
    constexpr int V = NR * NT;
    constexpr int SH = 6 - K3Log2<V>::v;
    const int beg = a.off[e], end = a.off[e + 1];
    for (int c0 = beg; c0 < end; c0 += NT) {
        int pr[NT];
        const float *xr[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            pr[t] = c0 + t < end ? a.perm[c0 + t] : -1;
            xr[t] = pr[t] >= 0 ? a.h + (size_t)pr[t] * I : nullptr;
        }
        typename K3Acc<FMT>::T acc[V];
        k3d_tile<FMT, NR, NT>(rows, srows, xr, I, lane, acc);
        k3d_transpose_reduce<V>(acc, lane);
        const int v = lane >> SH;
        if ((lane & ((1 << SH) - 1)) == 0 && v < V) {
            const int r = v / NT, t = v % NT;
            int p = -1;
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) if (tt == t) p = pr[tt];
            if (row0 + r < L && p >= 0) a.contrib[(size_t)p * L + row0 + r] = (float)acc[0];
        }
    }
}

/* ----------------------------------------------------------------- dense ---- */
/* grid (ceil(rows / (4*NR)), ceil(T / NT)). With PAIR the wave owns rows of Wa and Wb
 * and writes act(a, b). */
template <int FMT, int NR, int NT, bool PAIR>
__global__ void __launch_bounds__(256)
k_dense(const void *Wa, const void *Wb, const uint8_t *Sa, const uint8_t *Sb, int nrows,
        int in, const float *x, int ldx, int T, float *y, int ldy, float b1, float b2)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row0 = (blockIdx.x * 4 + wave) * NR;
    if (row0 >= nrows) return;
    const int t0 = blockIdx.y * NT;
    constexpr int NRT = PAIR ? 2 * NR : NR;
    const void *rows[NRT];
    const uint8_t *srows[NRT];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const bool ok = row0 + r < nrows;
        rows[r] = ok ? k3d_row<FMT>(Wa, row0 + r, in) : nullptr;
        srows[r] = ok ? k3d_srow(Sa, row0 + r, in) : nullptr;
        if constexpr (PAIR) {
            rows[NR + r] = ok ? k3d_row<FMT>(Wb, row0 + r, in) : nullptr;
            srows[NR + r] = ok ? k3d_srow(Sb, row0 + r, in) : nullptr;
        }
    }
    const float *xr[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) xr[t] = t0 + t < T ? x + (size_t)(t0 + t) * ldx : nullptr;
    constexpr int V = NRT * NT;
    constexpr int SH = 6 - K3Log2<V>::v;
    typename K3Acc<FMT>::T acc[V];
    k3d_tile<FMT, NRT, NT>(rows, srows, xr, in, lane, acc);
    k3d_transpose_reduce<V>(acc, lane);
    const int v = lane >> SH;
    const float av = (float)acc[0];
    if constexpr (PAIR) {
        const float bv = __shfl_xor(av, 32, K3G_WAVE);
        if ((lane & ((1 << SH) - 1)) == 0 && v < NR * NT) {
            const int r = v / NT, t = v % NT;
            if (row0 + r < nrows && t0 + t < T)
                y[(size_t)(t0 + t) * ldy + row0 + r] = k3d_act(av, bv, b1, b2);
        }
    } else {
        if ((lane & ((1 << SH) - 1)) == 0 && v < V) {
            const int r = v / NT, t = v % NT;
            if (row0 + r < nrows && t0 + t < T)
                y[(size_t)(t0 + t) * ldy + row0 + r] = av;
        }
    }
}

/* --------------------------------------------------- int8 draft rows (K3_WI8) ---- */
/* Rows of [f32 scale][int8 x in] (stride 4 + in bytes, so 4-byte aligned when in % 4 == 0):
 * y[t][r] = (sum_i w[r][i] x[t][i]) * scale[r], summed in float in any order (the engine's
 * k3_matmul_q8, src/core/k3_ops.c:1198-1272, gives these draft weights no determinism
 * contract). One wave per row and up to NT tokens, lane l taking columns 4 l + 256 j; with
 * PAIR the wave also takes the same row of Wb and writes act(a, b). grid (ceil(rows / 4),
 * ceil(T / NT)), 4 waves per block. */
template <int NT, bool PAIR>
__global__ void __launch_bounds__(256)
k_dense_q8(const uint8_t *Wa, const uint8_t *Wb, int nrows, int in, const float *x, int ldx,
           int T, float *y, int ldy, float b1, float b2)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= nrows) return;
    const int t0 = blockIdx.y * NT;
    const size_t rowb = (size_t)4 + (size_t)in;
    const uint8_t *ra = Wa + (size_t)row * rowb;
    const uint8_t *rb = PAIR ? Wb + (size_t)row * rowb : nullptr;
    float acc[NT], accb[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) { acc[t] = 0.0f; accb[t] = 0.0f; }
    for (int i = 4 * lane; i < in; i += 256) {
        const uint32_t wa = *(const uint32_t *)(ra + 4 + i);
        const float a[4] = {(float)(int8_t)(wa & 0xff), (float)(int8_t)((wa >> 8) & 0xff),
                            (float)(int8_t)((wa >> 16) & 0xff), (float)(int8_t)(wa >> 24)};
        float bw[4] = {0.f, 0.f, 0.f, 0.f};
        if (PAIR) {
            const uint32_t wb = *(const uint32_t *)(rb + 4 + i);
            bw[0] = (float)(int8_t)(wb & 0xff); bw[1] = (float)(int8_t)((wb >> 8) & 0xff);
            bw[2] = (float)(int8_t)((wb >> 16) & 0xff); bw[3] = (float)(int8_t)(wb >> 24);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t0 + t < T) {
                const float4 xv = *(const float4 *)(x + (size_t)(t0 + t) * ldx + i);
                acc[t] = fmaf(a[0], xv.x, fmaf(a[1], xv.y, fmaf(a[2], xv.z, fmaf(a[3], xv.w, acc[t]))));
                if (PAIR)
                    accb[t] = fmaf(bw[0], xv.x, fmaf(bw[1], xv.y,
                                   fmaf(bw[2], xv.z, fmaf(bw[3], xv.w, accb[t]))));
            }
        }
    }
    const float sa = *(const float *)ra, sb = PAIR ? *(const float *)rb : 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float va = k3d_wave_sum(acc[t]) * sa;
        const float vb = PAIR ? k3d_wave_sum(accb[t]) * sb : 0.0f;
        if (lane == 0 && t0 + t < T)
            y[(size_t)(t0 + t) * ldy + row] = PAIR ? k3d_act(va, vb, b1, b2) : va;
    }
}

/* ------------------------------------------------------------- launchers ---- */
static bool k3_aligned(const void *p, int a) { return ((uintptr_t)p & (uintptr_t)(a - 1)) == 0; }

extern "C" int k3k_routed_gateup(const K3kRouted *a, int maxU, int maxtok, hipStream_t st)
{
    if (maxU <= 0) return 0;
    if (a->latent % 16 || !k3_aligned(a->z, 16)) return -1;
    if (a->fmt == K3K_MXFP4) {
        if (maxtok <= 1) {
            constexpr int NR = 8;
            dim3 g((a->inter + 4 * NR - 1) / (4 * NR), maxU);
            hipLaunchKernelGGL((k_routed_gateup<K3K_MXFP4, NR, 1>), g, dim3(256), 0, st, *a);
        } else {
            constexpr int NR = 8;
            dim3 g((a->inter + 4 * NR - 1) / (4 * NR), maxU);
            hipLaunchKernelGGL((k_routed_gateup<K3K_MXFP4, NR, 4>), g, dim3(256), 0, st, *a);
        }
    } else if (a->fmt == K3K_F32) {
        constexpr int NR = 4;
        dim3 g((a->inter + 4 * NR - 1) / (4 * NR), maxU);
        hipLaunchKernelGGL((k_routed_gateup<K3K_F32, NR, 4>), g, dim3(256), 0, st, *a);
    } else {
        return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int k3k_routed_down(const K3kRouted *a, int maxU, int maxtok, hipStream_t st)
{
    if (maxU <= 0) return 0;
    if (a->inter % 16) return -1;
    if (a->fmt == K3K_MXFP4) {
        if (maxtok <= 1) {
            constexpr int NR = 16;
            dim3 g((a->latent + 4 * NR - 1) / (4 * NR), maxU);
            hipLaunchKernelGGL((k_routed_down<K3K_MXFP4, NR, 1>), g, dim3(256), 0, st, *a);
        } else {
            constexpr int NR = 16;
            dim3 g((a->latent + 4 * NR - 1) / (4 * NR), maxU);
            hipLaunchKernelGGL((k_routed_down<K3K_MXFP4, NR, 4>), g, dim3(256), 0, st, *a);
        }
    } else if (a->fmt == K3K_F32) {
        constexpr int NR = 8;
        dim3 g((a->latent + 4 * NR - 1) / (4 * NR), maxU);
        hipLaunchKernelGGL((k_routed_down<K3K_F32, NR, 4>), g, dim3(256), 0, st, *a);
    } else {
        return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int k3k_dense(int fmt, const void *Wa, const void *Wb, int rows, int in,
                         const float *x, int ldx, int T, float *y, int ldy, float b1,
                         float b2, hipStream_t st)
{
    if (rows <= 0 || T <= 0) return 0;
    if (fmt == K3K_I8R) {
        /* 4-byte int8 groups and float4 activations: in % 4, 16-byte x rows */
        if (in % 4 || ldx % 4 || !k3_aligned(x, 16) || !k3_aligned(Wa, 4) ||
            (Wb && !k3_aligned(Wb, 4)))
            return -1;
        constexpr int NT = 4;
        const dim3 g((rows + 3) / 4, (T + NT - 1) / NT);
        if (Wb)
            hipLaunchKernelGGL((k_dense_q8<NT, true>), g, dim3(256), 0, st, (const uint8_t *)Wa,
                               (const uint8_t *)Wb, rows, in, x, ldx, T, y, ldy, b1, b2);
        else
            hipLaunchKernelGGL((k_dense_q8<NT, false>), g, dim3(256), 0, st, (const uint8_t *)Wa,
                               (const uint8_t *)nullptr, rows, in, x, ldx, T, y, ldy, b1, b2);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    if (in % 16 || ldx % 4 || !k3_aligned(x, 16) || !k3_aligned(Wa, 16) ||
        (Wb && !k3_aligned(Wb, 16)))
        return -1;
    if (fmt == K3K_BF16 && in % 8) return -1;
    constexpr int NR = 8, NT = 4;
    dim3 g((rows + 4 * NR - 1) / (4 * NR), (T + NT - 1) / NT);
    if (fmt == K3K_BF16) {
        if (Wb) {
            if (T == 1)
                hipLaunchKernelGGL((k_dense<K3K_BF16, NR, 1, true>),
                                   dim3(g.x, T), dim3(256), 0, st, Wa, Wb, nullptr, nullptr,
                                   rows, in, x, ldx, T, y, ldy, b1, b2);
            else
                hipLaunchKernelGGL((k_dense<K3K_BF16, NR, NT, true>), g, dim3(256), 0, st,
                                   Wa, Wb, nullptr, nullptr, rows, in, x, ldx, T, y, ldy,
                                   b1, b2);
        } else {
            if (T == 1)
                hipLaunchKernelGGL((k_dense<K3K_BF16, 2 * NR, 1, false>),
                                   dim3((rows + 8 * NR - 1) / (8 * NR), T), dim3(256), 0, st,
                                   Wa, Wb, nullptr, nullptr, rows, in, x, ldx, T, y, ldy,
                                   b1, b2);
            else
                hipLaunchKernelGGL((k_dense<K3K_BF16, NR, NT, false>), g, dim3(256), 0, st,
                                   Wa, Wb, nullptr, nullptr, rows, in, x, ldx, T, y, ldy,
                                   b1, b2);
        }
    } else if (fmt == K3K_F32) {
        if (Wb)
            hipLaunchKernelGGL((k_dense<K3K_F32, NR / 2, NT, true>),
                               dim3((rows + 2 * NR - 1) / (2 * NR), g.y), dim3(256), 0, st,
                               Wa, Wb, nullptr, nullptr, rows, in, x, ldx, T, y, ldy, b1,
                               b2);
        else
            hipLaunchKernelGGL((k_dense<K3K_F32, NR, NT, false>), g, dim3(256), 0, st,
                               Wa, Wb, nullptr, nullptr, rows, in, x, ldx, T, y, ldy, b1,
                               b2);
    } else {
        return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

/* One MXFP4 matrix times one vector (k3_matmul_mxfp4 on the GPU). Fast path for
 * group 32, in % 16 == 0 with aligned operands; otherwise one wave per row decoding
 * nibbles one at a time the way the engine's grouped path does (src/core/k3_ops.c:
 * 1386-1388, 1515-1520): a row has ceil(in / group) scale bytes, element j of group g
 * is nibble j of the bytes from g * (group / 2) on (low nibble first) scaled by byte g --
 * for an even group the row's plain packing, for an odd one what the engine reads. */
__global__ void __launch_bounds__(64)
k_mxfp4_gemv_any(float *y, const float *x, const uint8_t *packed, const uint8_t *scales,
                 int in, int rows, int group)
{
    const int r = blockIdx.x, lane = threadIdx.x;
    const uint8_t *pr = packed + (size_t)r * (in / 2);
    const uint8_t *sr = scales + (size_t)r * ((in + group - 1) / group);
    float acc = 0.0f;
    for (int i = lane; i < in; i += 64) {
        const int g = i / group, j = i - g * group;
        const uint8_t b = pr[g * (group >> 1) + (j >> 1)];
        const uint32_t code = (j & 1) ? (b >> 4) : (b & 15);
        const float m = k3d_e8m0(sr[g]);
        const float mag = (code & 7) == 0 ? 0.0f
                        : (code & 7) == 1 ? 0.5f
                        : __uint_as_float((((code & 7) >> 1) + 126u) << 23 | (code & 1u) << 22);
        const float wv = (code & 8) ? -mag : mag;
        acc = fmaf(__fmul_rn(wv, m), x[i], acc);
    }
    acc = k3d_wave_sum(acc);
    if (lane == 0) y[r] = acc;
}

extern "C" int k3k_mxfp4_gemv(float *y, const float *x, const uint8_t *packed,
                              const uint8_t *scales, int in, int rows, int group,
                              hipStream_t st)
{
    if (rows <= 0 || in <= 0) return 0;
    if (group < 1) return -1;
    if (group == 32 && in % 16 == 0 && k3_aligned(x, 16) && k3_aligned(packed, 8)) {
        constexpr int NR = 16;
        hipLaunchKernelGGL((k_dense<K3K_MXFP4, NR, 1, false>),
                           dim3((rows + 4 * NR - 1) / (4 * NR), 1), dim3(256), 0, st,
                           (const void *)packed, (const void *)nullptr, scales, nullptr, rows,
                           in, x, in, 1, y, rows, 0.f, 0.f);
    } else {
        hipLaunchKernelGGL(k_mxfp4_gemv_any, dim3(rows), dim3(64), 0, st, y, x, packed, scales,
                           in, rows, group);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
