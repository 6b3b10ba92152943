/* k3g_dev.h - device-side helpers shared by the gfx950 kernels. */
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "k3g_expf.h"

#define K3G_WAVE 64
#define K3G_TILE_COLS 128      /* pairs per column tile of the grouped GEMMs */


typedef float k3v2f __attribute__((ext_vector_type(2)));

/* Error codes a kernel may raise into the context's device error word. The host reads
 * it in k3g_sync() and reports it. */
enum {
    K3G_ERR_NONE = 0,
    K3G_ERR_EXPERT_RANGE = 1,   /* a routed index outside [0, n_experts) reached a kernel */
    K3G_ERR_WAIT = 2,           /* a bounded device wait ran out */
};

__device__ __forceinline__ void k3d_raise(int *err, int code)
{
    if (err) atomicCAS(err, 0, code);
}

/* Device-coherent (sc1) 64-bit load and store, for values other waves exchange inside
 * one kernel without a device-wide cache writeback. */
__device__ __forceinline__ double k3d_ld_dev64(const double *p)
{
    const unsigned long long v = __hip_atomic_load((const unsigned long long *)p,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __longlong_as_double((long long)v);
}

__device__ __forceinline__ void k3d_st_dev64(double *p, double v)
{
    __hip_atomic_store((unsigned long long *)p, (unsigned long long)__double_as_longlong(v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* E8M0 byte -> 2^(b-127) as fp32; 255 (NaN by the OCP spec) -> 0, matching the engine's
 * table (src/core/k3_ops.c:1315-1322). b = 0 gives the denormal 2^-127. */
__device__ __forceinline__ float k3d_e8m0(uint32_t b)
{
    return b == 255u ? 0.0f
         : (b == 0u ? __uint_as_float(0x00400000u) : __uint_as_float(b << 23));
}

/* Eight E2M1 values from one 32-bit word (bytes in memory order; low nibble is the even
 * element), each times `scale`, using gfx950's v_cvt_scalef32_pk_f32_fp4. The product
 * with a power-of-two scale is exact. */
__device__ __forceinline__ void k3d_fp4x8(uint32_t w, float scale, float *o)
{
    k3v2f a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 0);
    k3v2f b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 1);
    k3v2f c = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 2);
    k3v2f d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, scale, 3);
    o[0] = a.x; o[1] = a.y; o[2] = b.x; o[3] = b.y;
    o[4] = c.x; o[5] = c.y; o[6] = d.x; o[7] = d.y;
}

/* One DMA instruction: 64 lanes x 16 bytes from their own global addresses to 1 KB of LDS
 * at byte address `lds` (lane l at lds + 16 l), M0 saved and restored around it. */
__device__ __forceinline__ void k3d_dma16(const void *src, uint32_t lds)
{
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %2\n\t"
                 "global_load_lds_dwordx4 %1, off\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(keep) : "v"(src), "s"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}

/* s_waitcnt vmcnt(n) for a wave-uniform n in 0..15 */
__device__ __forceinline__ void k3d_wait_vm(int n)
{
    switch (n) {
#define K3_WVM(N) case N: __builtin_amdgcn_s_waitcnt(0x0F70 | N); break;
        K3_WVM(1) K3_WVM(2) K3_WVM(3) K3_WVM(4) K3_WVM(5) K3_WVM(6) K3_WVM(7) K3_WVM(8)
        K3_WVM(9) K3_WVM(10) K3_WVM(11) K3_WVM(12) K3_WVM(13) K3_WVM(14) K3_WVM(15)
#undef K3_WVM
        default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    }
}

__device__ __forceinline__ float k3d_bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float k3d_bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

/* Wave-wide sum, every lane gets the total. */
/* Exclusive scans, across a block of NW <= 64 waves, of N ints per thread at once: wave
 * scans by shuffles, the waves' totals scanned by wave 0 through lds[(NW + 1) * N]; tot
 * receives the block sums. Every thread of the block takes part. */
template <int N, int NW>
__device__ __forceinline__ void k3d_block_exscan_n(int (&v)[N], int (&tot)[N], int *lds)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc[N];
#pragma unroll
    for (int i = 0; i < N; ++i) inc[i] = v[i];
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int o = __shfl_up(inc[i], m, K3G_WAVE);
            if (lane >= m) inc[i] += o;
        }
    }
    if (lane == 63) {
#pragma unroll
        for (int i = 0; i < N; ++i) lds[wave * N + i] = inc[i];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int t = lane < NW ? lds[lane * N + i] : 0;
            int s = t;
#pragma unroll
            for (int m = 1; m < NW; m <<= 1) {
                const int o = __shfl_up(s, m, K3G_WAVE);
                if (lane >= m) s += o;
            }
            if (lane < NW) lds[lane * N + i] = s - t;
            if (lane == NW - 1) lds[NW * N + i] = s;
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < N; ++i) {
        v[i] = lds[wave * N + i] + inc[i] - v[i];
        tot[i] = lds[NW * N + i];
    }
    __syncthreads();
}

/* Column tiles of up to K3G_TILE_COLS pairs per expert, largest first: every full tile
 * (in expert order), then the experts' last partial tiles by their count of 16-column
 * blocks, 8 down to 1 (in expert order within a count); clears *flag. Called by every
 * thread of a block of 1024 (thread e < E for expert e, its pair count and first sorted
 * position); lds holds (16 + 1) * 9 ints. */
__device__ __forceinline__ void k3d_build_tiles(int e, int E, int cnt, int off_e, int4 *tiles,
                                                int32_t *ntiles, int32_t *flag, int *lds)
{
    if (e >= E) cnt = 0;
    const int nfull = cnt / K3G_TILE_COLS, rem = cnt - nfull * K3G_TILE_COLS;
    const int cls = rem ? (rem + 15) / 16 : 0;          /* block count of the last tile */
    int v[9], tot[9];
    v[0] = nfull;
#pragma unroll
    for (int j = 1; j < 9; ++j) v[j] = cls == 9 - j;
    k3d_block_exscan_n<9, 16>(v, tot, lds);
    for (int i = 0; i < nfull; ++i)
        tiles[v[0] + i] = make_int4(e, off_e + K3G_TILE_COLS * i, K3G_TILE_COLS, 0);
    int base = tot[0];
#pragma unroll
    for (int j = 1; j < 9; ++j) {
        if (cls == 9 - j)
            tiles[base + v[j]] = make_int4(e, off_e + K3G_TILE_COLS * nfull, rem, 0);
        base += tot[j];
    }
    if (e == 0) { *ntiles = base; *flag = 0; }
}

__device__ __forceinline__ float k3d_wave_sum(float v)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, K3G_WAVE);
    return v;
}

__device__ __forceinline__ double k3d_wave_sumd(double v)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, K3G_WAVE);
    return v;
}

/* Transposed wave reduction of V partial sums per lane (V a power of two, <= 64).
 * Afterwards lane l holds the full 64-lane sum of value index (l >> (6 - log2 V)) in
 * v[0]. Each halving round trades half the values with the partner lane, so the whole
 * reduction costs about V shuffles instead of 6*V. */
template <int V, typename A>
__device__ __forceinline__ void k3d_transpose_reduce(A *v, int lane)
{
    int n = V;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        if (n > 1) {
            const int h = n >> 1;
            const bool upper = (lane & m) != 0;
#pragma unroll
            for (int i = 0; i < V / 2; ++i) {
                if (i < h) {
                    const A send = upper ? v[i] : v[i + h];
                    const A keep = upper ? v[i + h] : v[i];
                    v[i] = keep + __shfl_xor(send, m, K3G_WAVE);
                }
            }
            n = h;
        } else {
            v[0] += __shfl_xor(v[0], m, K3G_WAVE);
        }
    }
}

/* The engine's expf bit for bit (the C library's algorithm, k3g_expf.h), and tanhf
 * correctly rounded but for a vanishing set of near-midpoint inputs (the double tanh is
 * within an ulp of double, far inside a float rounding interval). */
__device__ __forceinline__ float k3d_expf(float v) { return k3x_expf(v); }
__device__ __forceinline__ float k3d_tanhf_cr(float v) { return (float)tanh((double)v); }

/* 1/(1+expf(-v)) with the engine's float operation order (src/core/k3_ops.c:105) */
__device__ __forceinline__ float k3d_sigmoid(float v)
{
    return __fdiv_rn(1.0f, __fadd_rn(1.0f, k3d_expf(-v)));
}

/* SiTU-GLU on one (gate, up) pair, src/core/k3_ops.c:110-123, in the engine's float
 * operation order: a = (b1 * tanh(g / b1)) * sigmoid(g), u = b2 * tanh(up / b2), y = a * u.
 * A cap >= 2^64 is treated as absent, the exact limit the engine reaches for its SwiGLU
 * setting b = 2^100 (tanh(t) = t for tiny t, and scaling by a power of two is exact):
 * a = g * sigmoid(g), u = up. The sigmoid takes the uncapped gate. */
__device__ __forceinline__ float k3d_act(float g, float up, float b1, float b2)
{
    const float sg = k3d_sigmoid(g);
    float a, u;
    if (b1 >= 18446744073709551616.0f) a = __fmul_rn(g, sg);
    else a = __fmul_rn(__fmul_rn(b1, k3d_tanhf_cr(__fdiv_rn(g, b1))), sg);
    if (b2 >= 18446744073709551616.0f) u = up;
    else u = __fmul_rn(b2, k3d_tanhf_cr(__fdiv_rn(up, b2)));
    return __fmul_rn(a, u);
}
