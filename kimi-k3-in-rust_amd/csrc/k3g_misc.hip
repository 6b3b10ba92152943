/* k3g_misc.hip - dispatch (counting sort of token slots by expert), the weighted
 * combine, RMSNorm, dequantisation and the seeded synthetic fills. */
#include "k3g_dev.h"
#include "k3g_kernels.h"
#include "k3s_hash.h"

#define K3G_DCH 256          /* pairs per dispatch chunk */
#define K3G_MAX_EXPERTS 1024

/* --------------------------------------------------------------- dispatch ---- */
/* The engine's prefill groups (token, slot) pairs by expert in first-seen order and
 * scans for matches (src/core/k3_ops.c:738-775). Here the grouping is a stable counting
 * sort in expert order: within an expert the pairs keep their (t, j) order, so every
 * expert's token list is deterministic and its outputs land in per-pair slots that the
 * combine reads back in the engine's slot order. */

__device__ __forceinline__ int k3d_key(const int32_t *idx, int p, int P, int E, int *err)
{
    if (p >= P) return -1;
    const int k = idx[p];
    if (k >= E) { k3d_raise(err, K3G_ERR_EXPERT_RANGE); return -1; }
    return k;   /* negative keys (dropped slots) are skipped */
}

/* One block of 1024 threads for P <= K3G_DSORT pairs: the pairs, as key << 12 | pair
 * (key = expert, or E for a dropped slot and for the padding of the last 64-pair chunk),
 * are sorted by key in LDS with one stable split per key bit: a pair's place is the
 * zeros (or ones) before its chunk plus those before its lane in the chunk's ballot.
 * Per-expert counts come from LDS atomics; block scans give the expert ranges and the
 * active list. */
#define K3G_DSORT 4096
__global__ void __launch_bounds__(1024)
k_disp_sort(const int32_t *idx, int P, int E, int32_t *off, int32_t *act, int32_t *nact,
            int32_t *perm, int *err, int4 *tiles, int32_t *ntiles, int32_t *flag)
{
    __shared__ uint32_t kv[2][K3G_DSORT];
    __shared__ int cnt[K3G_MAX_EXPERTS];
    __shared__ int zc[K3G_DSORT / 64];
    __shared__ int red[17 * 9];
    __shared__ int ztot;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nch = (P + 63) / 64;
    cnt[tid] = 0;
    __syncthreads();
    for (int i = tid; i < 64 * nch; i += 1024) {
        int key = E;
        if (i < P) {
            const int k = idx[i];
            if (k >= E) k3d_raise(err, K3G_ERR_EXPERT_RANGE);
            else if (k >= 0) { key = k; atomicAdd(&cnt[k], 1); }
        }
        kv[0][i] = ((uint32_t)key << 12) | (uint32_t)i;
    }
    __syncthreads();
    const int nb = 32 - __clz(E);               /* bits of the largest key, E */
    int cur = 0;
    for (int b = 0; b < nb; ++b) {
        const uint32_t bit = 1u << (12 + b);
        for (int c = w; c < nch; c += 16) {
            const uint64_t m = __ballot(!(kv[cur][64 * c + lane] & bit));
            if (lane == 0) zc[c] = __popcll(m);
        }
        __syncthreads();
        if (w == 0) {
            const int z = lane < nch ? zc[lane] : 0;
            int inc = z;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int o = __shfl_up(inc, d, K3G_WAVE);
                if (lane >= d) inc += o;
            }
            if (lane < nch) zc[lane] = inc - z;
            if (lane == 63) ztot = inc;
        }
        __syncthreads();
        const int Z = ztot;
        const uint64_t lt = (1ull << lane) - 1;
        for (int c = w; c < nch; c += 16) {
            const uint32_t v = kv[cur][64 * c + lane];
            const bool zero = !(v & bit);
            const uint64_t m = __ballot(zero);
            const int zb = zc[c];
            const int pos = zero ? zb + __popcll(m & lt) : Z + 64 * c - zb + __popcll(~m & lt);
            kv[cur ^ 1][pos] = v;
        }
        __syncthreads();
        cur ^= 1;
    }
    /* expert ranges and the active list */
    const int ce = tid < E ? cnt[tid] : 0;
    int v[2] = {ce, ce > 0}, tot[2];
    k3d_block_exscan_n<2, 16>(v, tot, red);
    if (tid < E) {
        off[tid] = v[0];
        if (ce > 0) act[v[1]] = tid;
    }
    if (tid == 0) { off[E] = tot[0]; *nact = tot[1]; }
    /* the pairs of real experts come first, in expert order, each expert's in pair order */
    for (int i = tid; i < tot[0]; i += 1024) perm[i] = (int32_t)(kv[cur][i] & 4095u);
    if (tiles) k3d_build_tiles(tid, E, ce, v[0], tiles, ntiles, flag, red);
}

/* Large P: three passes over chunks of 256 pairs, no single-block step (a lone large
 * block waits long for a CU when other kernels fill the GPU beside it):
 *   count   one block per chunk: the chunk's per-expert counts from LDS atomics;
 *   scan    one wave per 64 experts, a lane per expert: its counts over all chunks (every
 *           load of a batch in flight), their running sum as each chunk's base within the
 *           expert, and the expert's total;
 *   scatter one block per chunk: the expert ranges from a block scan of the totals (block
 *           0 also writes them and the active list), then each pair's place = its expert's
 *           start + its chunk's base + its rank among the chunk's earlier pairs of that
 *           expert (ballots over the key bits within a wave, per-wave counts in LDS across
 *           waves), so the order within an expert is the pair order. */
__global__ void __launch_bounds__(256)
k_disp_count(const int32_t *idx, int P, int E, int32_t *cnt, int *err)
{
    __shared__ int h[K3G_MAX_EXPERTS];
    const int c = blockIdx.x;
    for (int e = threadIdx.x; e < E; e += 256) h[e] = 0;
    __syncthreads();
    const int key = k3d_key(idx, c * K3G_DCH + threadIdx.x, P, E, err);
    if (key >= 0) atomicAdd(&h[key], 1);
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += 256) cnt[(size_t)c * E + e] = h[e];
}

__global__ void __launch_bounds__(64)
k_disp_scan(const int32_t *cnt, int nch, int E, int32_t *base, int32_t *tot)
{
    const int e = blockIdx.x * 64 + threadIdx.x;
    if (e >= E) return;
    int b = 0;
    for (int c = 0; c < nch; c += 32) {
        int v[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) v[u] = c + u < nch ? cnt[(size_t)(c + u) * E + e] : 0;
#pragma unroll
        for (int u = 0; u < 32; ++u)
            if (c + u < nch) { base[(size_t)(c + u) * E + e] = b; b += v[u]; }
    }
    tot[e] = b;
}

__global__ void __launch_bounds__(256)
k_disp_scatter(const int32_t *idx, int P, int E, const int32_t *base, const int32_t *tot,
               int32_t *off, int32_t *act, int32_t *nact, int32_t *perm)
{
    __shared__ int wc[4][K3G_MAX_EXPERTS];
    __shared__ int first[K3G_MAX_EXPERTS];
    __shared__ int red[5 * 2];
    const int c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    for (int e = tid; e < E; e += 256) wc[0][e] = wc[1][e] = wc[2][e] = wc[3][e] = 0;
    /* the expert ranges: thread i scans experts 4 i .. 4 i + 3 (E <= 1024) */
    {
        int t4[4], run = 0, nz = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = 4 * tid + u;
            t4[u] = e < E ? tot[e] : 0;
            run += t4[u];
            nz += t4[u] > 0;
        }
        int v[2] = {run, nz}, all[2];
        k3d_block_exscan_n<2, 4>(v, all, red);
        int s0 = v[0], a0 = v[1];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = 4 * tid + u;
            if (e < E) {
                first[e] = s0;
                if (c == 0) {
                    off[e] = s0;
                    if (t4[u] > 0) act[a0] = e;
                }
            }
            s0 += t4[u];
            a0 += t4[u] > 0;
        }
        if (c == 0 && tid == 0) { off[E] = all[0]; *nact = all[1]; }
    }
    const int key = k3d_key(idx, c * K3G_DCH + tid, P, E, nullptr);
    /* the lanes of this wave holding the same key: ballots over the key's bits (skipped
     * slots, key -1, form their own group and are not placed) */
    uint64_t peers = __ballot(key >= 0);
    if (key < 0) peers = ~peers;
    const int nb = 32 - __clz(E > 1 ? E - 1 : 1);
    for (int b = 0; b < nb; ++b) {
        const bool one = key >= 0 && ((key >> b) & 1);
        const uint64_t m = __ballot(one);
        peers &= one ? m : ~m;
    }
    const uint64_t lt = (1ull << lane) - 1;
    const int r = __popcll(peers & lt);
    __syncthreads();
    if (key >= 0 && r == 0) wc[w][key] = __popcll(peers);
    __syncthreads();
    if (key >= 0) {
        int before = r;
        for (int q = 0; q < w; ++q) before += wc[q][key];
        perm[first[key] + base[(size_t)c * E + key] + before] = c * K3G_DCH + tid;
    }
}

extern "C" int k3k_dispatch_tiles(const int32_t *idx, int P, int E, int32_t *cnt,
                                  int32_t *base, int32_t *off, int32_t *act, int32_t *nact,
                                  int32_t *perm, int *err, int32_t *tiles, int32_t *ntiles,
                                  int32_t *flag, hipStream_t st)
{
    if (E < 1 || E > K3G_MAX_EXPERTS || P < 1) return -1;
    if (P <= K3G_DSORT) {
        hipLaunchKernelGGL(k_disp_sort, dim3(1), dim3(1024), 0, st, idx, P, E, off, act, nact,
                           perm, err, (int4 *)tiles, ntiles, flag);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    const int nch = (P + K3G_DCH - 1) / K3G_DCH;
    /* the experts' totals follow the chunk bases (base holds (nch + 1) E entries) */
    int32_t *tot = base + (size_t)nch * E;
    hipLaunchKernelGGL(k_disp_count, dim3(nch), dim3(256), 0, st, idx, P, E, cnt, err);
    hipLaunchKernelGGL(k_disp_scan, dim3((E + 63) / 64), dim3(64), 0, st, cnt, nch, E, base,
                       tot);
    hipLaunchKernelGGL(k_disp_scatter, dim3(nch), dim3(256), 0, st, idx, P, E, base, tot, off,
                       act, nact, perm);
    if (hipGetLastError() != hipSuccess) return -1;
    return tiles ? k3k_gemm_tiles(off, E, tiles, ntiles, flag, st) : 0;
}

extern "C" int k3k_dispatch(const int32_t *idx, int P, int E, int32_t *cnt, int32_t *base,
                            int32_t *off, int32_t *act, int32_t *nact, int32_t *perm,
                            int *err, hipStream_t st)
{
    return k3k_dispatch_tiles(idx, P, E, cnt, base, off, act, nact, perm, err, nullptr,
                              nullptr, nullptr, st);
}

/* ---------------------------------------------------------------- combine ---- */
/* src/core/k3_ops.c:641-642 and :786-793: acc = 0; acc += w_j * edn_j for j in slot
 * order, multiply and add rounded separately; then the shared expert is added
 * (:654). grid (ceil(n / 1024), T); a thread owns four columns. */
__global__ void __launch_bounds__(256)
k_combine(const float *__restrict__ contrib, const int32_t *__restrict__ idx,
          const float *__restrict__ wt, int k, int n, const float *__restrict__ add,
          float *__restrict__ out)
{
    const int t = blockIdx.y;
    const int col = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (col >= n) return;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    for (int j = 0; j < k; ++j) {
        const size_t p = (size_t)t * k + j;
        if (idx[p] < 0) continue;
        const float w = wt[p];
        const float4 c = *(const float4 *)(contrib + p * n + col);
        a0 = __fadd_rn(a0, __fmul_rn(w, c.x));
        a1 = __fadd_rn(a1, __fmul_rn(w, c.y));
        a2 = __fadd_rn(a2, __fmul_rn(w, c.z));
        a3 = __fadd_rn(a3, __fmul_rn(w, c.w));
    }
    if (add) {
        const float4 s = *(const float4 *)(add + (size_t)t * n + col);
        a0 = __fadd_rn(a0, s.x); a1 = __fadd_rn(a1, s.y);
        a2 = __fadd_rn(a2, s.z); a3 = __fadd_rn(a3, s.w);
    }
    *(float4 *)(out + (size_t)t * n + col) = make_float4(a0, a1, a2, a3);
}

extern "C" int k3k_combine(const float *contrib, const int32_t *idx, const float *wt, int T,
                           int k, int n, const float *add, float *out, hipStream_t st)
{
    if (n % 4 || T < 1) return -1;
    hipLaunchKernelGGL(k_combine, dim3((n + 1023) / 1024, T), dim3(256), 0, st, contrib, idx,
                       wt, k, n, add, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

/* ---------------------------------------------------------------- rmsnorm ---- */
/* One token per block of 1024 threads: h += a (when a is given, stored back: the residual
 * add of src/core/k3_ops.c:1035-1036), then y = w * h * inv with
 * inv = (float)(1 / sqrt(sum_double h^2 / n + eps)) (src/core/k3_ops.c:94-102, float
 * multiplies in the engine's order) when w is given. Every load of the token is issued
 * before the first use; each thread owns elements 4 (tid + 1024 j) .. + 3 and is the only
 * one to read or write them, so y may alias h. The sum of squares is fp64 (the squares of
 * floats are exact in it) in a fixed order: per thread, then the wave, then the 16 waves
 * in index order. NV = float4s per thread held in registers (n <= 4096 NV). */
template <int NV>
__global__ void __launch_bounds__(1024)
k_add_rmsnorm(float *h, const float *a, float *y, const float *w, int n, float eps)
{
    __shared__ double part[16];
    const size_t base = (size_t)blockIdx.x * n;
    float4 *h4 = (float4 *)(h + base);
    const float4 *a4 = a ? (const float4 *)(a + base) : nullptr;
    const int n4 = n >> 2, tid = threadIdx.x;
    float4 v[NV], av[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = tid + 1024 * j;
        if (i < n4) {
            v[j] = h4[i];
            if (a4) av[j] = a4[i];
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = tid + 1024 * j;
        if (i < n4) {
            if (a4) {
                v[j].x = __fadd_rn(v[j].x, av[j].x);
                v[j].y = __fadd_rn(v[j].y, av[j].y);
                v[j].z = __fadd_rn(v[j].z, av[j].z);
                v[j].w = __fadd_rn(v[j].w, av[j].w);
                h4[i] = v[j];
            }
            ss = fma((double)v[j].x, (double)v[j].x, ss);
            ss = fma((double)v[j].y, (double)v[j].y, ss);
            ss = fma((double)v[j].z, (double)v[j].z, ss);
            ss = fma((double)v[j].w, (double)v[j].w, ss);
        }
    }
    if (!w) return;
    ss = k3d_wave_sumd(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int q = 0; q < 16; ++q) tot += part[q];
    const float inv = (float)(1.0 / sqrt(tot / (double)n + (double)eps));
    float4 *y4 = (float4 *)(y + base);
    const float4 *w4 = (const float4 *)w;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int i = tid + 1024 * j;
        if (i < n4) {
            const float4 wv = w4[i];
            float4 o;
            o.x = __fmul_rn(__fmul_rn(wv.x, v[j].x), inv);
            o.y = __fmul_rn(__fmul_rn(wv.y, v[j].y), inv);
            o.z = __fmul_rn(__fmul_rn(wv.z, v[j].z), inv);
            o.w = __fmul_rn(__fmul_rn(wv.w, v[j].w), inv);
            y4[i] = o;
        }
    }
}

/* Any width: the same sums and products, element by element, in the same per-thread
 * order (thread tid owns elements tid + 1024 j). */
__global__ void __launch_bounds__(1024)
k_add_rmsnorm_any(float *h, const float *a, float *y, const float *w, int n, float eps)
{
    __shared__ double part[16];
    const size_t base = (size_t)blockIdx.x * n;
    float *ht = h + base;
    const float *at = a ? a + base : nullptr;
    const int tid = threadIdx.x;
    double ss = 0.0;
    for (int i = tid; i < n; i += 1024) {
        float v = ht[i];
        if (at) {
            v = __fadd_rn(v, at[i]);
            ht[i] = v;
        }
        ss = fma((double)v, (double)v, ss);
    }
    if (!w) return;
    ss = k3d_wave_sumd(ss);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int q = 0; q < 16; ++q) tot += part[q];
    const float inv = (float)(1.0 / sqrt(tot / (double)n + (double)eps));
    float *yt = y + base;
    for (int i = tid; i < n; i += 1024) yt[i] = __fmul_rn(__fmul_rn(w[i], ht[i]), inv);
}

extern "C" int k3k_add_rmsnorm(float *h, const float *a, float *y, const float *w, int n, int T,
                               float eps, hipStream_t st)
{
    if (T < 1 || n < 1) return 0;
    if (!a && !w) return 0;
    const bool v4 = n % 4 == 0 && (((uintptr_t)h | (uintptr_t)a | (uintptr_t)y | (uintptr_t)w) & 15) == 0;
    const int nv = (n / 4 + 1023) / 1024;
    if (v4 && nv <= 1)
        hipLaunchKernelGGL(k_add_rmsnorm<1>, dim3(T), dim3(1024), 0, st, h, a, y, w, n, eps);
    else if (v4 && nv <= 2)
        hipLaunchKernelGGL(k_add_rmsnorm<2>, dim3(T), dim3(1024), 0, st, h, a, y, w, n, eps);
    else if (v4 && nv <= 4)
        hipLaunchKernelGGL(k_add_rmsnorm<4>, dim3(T), dim3(1024), 0, st, h, a, y, w, n, eps);
    else
        hipLaunchKernelGGL(k_add_rmsnorm_any, dim3(T), dim3(1024), 0, st, h, a, y, w, n, eps);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

/* y = RMSNorm(x) * w, one token per block (y may alias x) */
extern "C" int k3k_rmsnorm(float *y, const float *x, const float *w, int n, int T, float eps,
                           hipStream_t st)
{
    if (T < 1 || n < 1) return 0;
    if (!w) return -1;
    /* with no addend the kernel only reads x */
    return k3k_add_rmsnorm(const_cast<float *>(x), nullptr, y, w, n, T, eps, st);
}

__global__ void k_add(float *y, const float *a, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        y[i] = __fadd_rn(y[i], a[i]);
}

extern "C" int k3k_add(float *y, const float *a, size_t n, hipStream_t st)
{
    if (!n) return 0;
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_add, dim3(blocks < 4096 ? (unsigned)blocks : 4096u), dim3(256), 0, st,
                       y, a, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

/* dst <- src (n bytes) by a kernel on the stream: between pinned host memory and device
 * memory this stays on the compute queue, with no hand-over to a copy engine and back.
 * Both 16-byte aligned. */
__global__ void __launch_bounds__(256) k_copy(uint4 *dst, const uint4 *src, size_t n16,
                                              uint8_t *dtail, const uint8_t *stail, int ntail)
{
    const size_t g = (size_t)blockIdx.x * 256 + threadIdx.x, stride = (size_t)gridDim.x * 256;
    for (size_t i = g; i < n16; i += stride) dst[i] = src[i];
    if (g < (size_t)ntail) dtail[g] = stail[g];
}

extern "C" int k3k_copy(void *dst, const void *src, size_t n, hipStream_t st)
{
    if (!n) return 0;
    if ((((uintptr_t)dst | (uintptr_t)src) & 15) != 0) return -1;
    const size_t n16 = n / 16;
    const int ntail = (int)(n - 16 * n16);
    size_t blocks = (n16 + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL(k_copy, dim3((unsigned)blocks), dim3(256), 0, st, (uint4 *)dst,
                       (const uint4 *)src, n16, (uint8_t *)dst + 16 * n16,
                       (const uint8_t *)src + 16 * n16, ntail);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

/* *p = v (a flag cleared in stream order by a kernel, which a captured graph replays
 * the same way every time) */
__global__ void __launch_bounds__(64) k_set_i32(int32_t *p, int32_t v)
{
    if (threadIdx.x == 0) *p = v;
}

extern "C" int k3k_set_i32(int32_t *p, int32_t v, hipStream_t st)
{
    if (!p) return -1;
    hipLaunchKernelGGL(k_set_i32, dim3(1), dim3(64), 0, st, p, v);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

/* ---------------------------------------------------------------- dequant ---- */
/* src/core/k3_ops.c:1770-1800: out = E2M1[nibble] * 2^(s-127), s = 255 gives a
 * (signed) zero; element i takes scale i / group of its row. One packed byte per
 * thread. */
__constant__ float k3c_e2m1[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                                   -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

__global__ void k_dequant(float *out, const uint8_t *packed, const uint8_t *scales, int rows,
                          int pcols, int group)
{
    const int width = pcols * 2, ngrp = (width + group - 1) / group;
    const size_t n = (size_t)rows * pcols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        const size_t r = i / pcols;
        const int c = (int)(i - r * pcols);
        const uint8_t b = packed[i];
        const float m0 = k3d_e8m0(scales[r * ngrp + (2 * c) / group]);
        const float m1 = k3d_e8m0(scales[r * ngrp + (2 * c + 1) / group]);
        out[r * width + 2 * c] = __fmul_rn(k3c_e2m1[b & 15], m0);
        out[r * width + 2 * c + 1] = __fmul_rn(k3c_e2m1[b >> 4], m1);
    }
}

extern "C" int k3k_dequant(float *out, const uint8_t *packed, const uint8_t *scales, int rows,
                           int pcols, int group, hipStream_t st)
{
    const size_t n = (size_t)rows * pcols;
    if (!n) return 0;
    const size_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_dequant, dim3(blocks < 16384 ? (unsigned)blocks : 16384u), dim3(256),
                       0, st, out, packed, scales, rows, pcols, group);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

/* ------------------------------------------------------------------ fills ---- */
__global__ void k_fill_bytes(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream,
                             uint64_t first)
{
    /* thread writes the 8 bytes of one hash word that fall inside [first, first+n) */
    const uint64_t w0 = first >> 3, w1 = (first + n + 7) >> 3;
    for (uint64_t w = w0 + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; w < w1;
         w += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t h = k3s_word(seed, stream, w);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint64_t i = w * 8 + b;
            if (i >= first && i < first + n) dst[i - first] = (uint8_t)(h >> (8 * b));
        }
    }
}

__global__ void k_fill_scales(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream,
                              uint64_t first, int lo, int hi)
{
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = k3s_scale_byte(seed, stream, first + i, lo, hi);
}

extern "C" int k3k_fill_bytes(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream,
                              uint64_t first, hipStream_t st)
{
    if (!n) return 0;
    hipLaunchKernelGGL(k_fill_bytes, dim3(4096), dim3(256), 0, st, dst, n, seed, stream, first);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int k3k_fill_scales(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream,
                               uint64_t first, int lo, int hi, hipStream_t st)
{
    if (!n) return 0;
    if (hi < lo) return -1;
    hipLaunchKernelGGL(k_fill_scales, dim3(4096), dim3(256), 0, st, dst, n, seed, stream,
                       first, lo, hi);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

/* ------------------------------------------------------------ expert tables ---- */
__global__ void __launch_bounds__(64)
k_set_experts(K3ExpertQ *table, const K3kEqSet s)
{
    const int i = threadIdx.x;
    if (i < s.n) table[s.e[i]] = s.q[i];
}

extern "C" int k3k_set_experts(K3ExpertQ *table, const K3kEqSet *s, hipStream_t st)
{
    if (!table || s->n < 0 || s->n > K3K_EQSET) return -1;
    if (s->n == 0) return 0;
    hipLaunchKernelGGL(k_set_experts, dim3(1), dim3(64), 0, st, table, *s);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
