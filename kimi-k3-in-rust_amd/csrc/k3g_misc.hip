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

/* Block-wide exclusive scan of one int per thread (256 threads). */
__device__ __forceinline__ int k3d_block_exscan(int v, int *total)
{
    __shared__ int wsum[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int inc = v;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const int o = __shfl_up(inc, m, K3G_WAVE);
        if (lane >= m) inc += o;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        if (w < wave) before += wsum[w];
        all += wsum[w];
    }
    __syncthreads();
    *total = all;
    return before + inc - v;
}

/* Single block, P <= 256: count, scan and scatter in one pass. */
__global__ void __launch_bounds__(256)
k_disp_small(const int32_t *idx, int P, int E, int32_t *off, int32_t *act, int32_t *nact,
             int32_t *perm, int *err)
{
    __shared__ int keys[K3G_DCH];
    __shared__ int tot[K3G_MAX_EXPERTS];
    const int tid = threadIdx.x;
    keys[tid] = k3d_key(idx, tid, P, E, err);
    __syncthreads();
    const int n = P < K3G_DCH ? P : K3G_DCH;
    for (int e = tid; e < E; e += 256) {
        int m = 0;
        for (int i = 0; i < n; ++i) m += keys[i] == e;
        tot[e] = m;
    }
    __syncthreads();
    /* each thread owns experts [tid*per, tid*per + per) */
    const int per = (E + 255) / 256;
    int s = 0, a = 0;
    for (int q = 0; q < per; ++q) {
        const int e = tid * per + q;
        if (e < E) { s += tot[e]; a += tot[e] > 0; }
    }
    int stot, atot;
    int sb = k3d_block_exscan(s, &stot);
    int ab = k3d_block_exscan(a, &atot);
    for (int q = 0; q < per; ++q) {
        const int e = tid * per + q;
        if (e < E) {
            off[e] = sb;
            if (tot[e] > 0) act[ab++] = e;
            const int base = sb;
            sb += tot[e];
            int pos = base;
            for (int i = 0; i < n; ++i)
                if (keys[i] == e) perm[pos++] = i;
        }
    }
    if (tid == 0) { off[E] = stot; *nact = atot; }
}

/* Single block of 1024 threads, P <= K3G_DONE: the pairs' keys in LDS, one thread per
 * expert counts its pairs, a block scan places the experts, and each expert thread writes
 * its pairs in pair order (stable). One launch instead of three for mid-size batches. */
#define K3G_DONE 4096
__global__ void __launch_bounds__(1024)
k_disp_one(const int32_t *idx, int P, int E, int32_t *off, int32_t *act, int32_t *nact,
           int32_t *perm, int *err)
{
    __shared__ __attribute__((aligned(16))) int keys[K3G_DONE];
    __shared__ int sc[1024], sa[1024];
    const int e = threadIdx.x;
    const int P4 = (P + 3) / 4;
    for (int i = e; i < 4 * P4; i += 1024) keys[i] = k3d_key(idx, i, P, E, err);
    __syncthreads();
    /* every thread reads the same keys (LDS broadcasts), four at a time */
    const int4 *k4 = (const int4 *)keys;
    int tot = 0;
    if (e < E) {
#pragma unroll 8
        for (int i = 0; i < P4; ++i) {
            const int4 v = k4[i];
            tot += (v.x == e) + (v.y == e) + (v.z == e) + (v.w == e);
        }
    }
    sc[e] = tot;
    sa[e] = tot > 0;
    __syncthreads();
    for (int dd = 1; dd < 1024; dd <<= 1) {
        const int a = e >= dd ? sc[e - dd] : 0, b = e >= dd ? sa[e - dd] : 0;
        __syncthreads();
        sc[e] += a;
        sa[e] += b;
        __syncthreads();
    }
    if (e < E) {
        const int first = sc[e] - tot;
        off[e] = first;
        if (tot > 0) act[sa[e] - 1] = e;
        int pos = first;
#pragma unroll 4
        for (int i = 0; i < P4 && pos < first + tot; ++i) {
            const int4 v = k4[i];
            if (v.x == e) perm[pos++] = 4 * i;
            if (v.y == e) perm[pos++] = 4 * i + 1;
            if (v.z == e) perm[pos++] = 4 * i + 2;
            if (v.w == e) perm[pos++] = 4 * i + 3;
        }
    }
    if (e == 1023) { off[E] = sc[1023]; *nact = sa[1023]; }
}

/* Large P, three passes over chunks of 256 pairs. */
__global__ void __launch_bounds__(256)
k_disp_count(const int32_t *idx, int P, int E, int32_t *cnt, int *err)
{
    __shared__ int keys[K3G_DCH];
    const int c = blockIdx.x;
    keys[threadIdx.x] = k3d_key(idx, c * K3G_DCH + threadIdx.x, P, E, err);
    __syncthreads();
    const int n = min(K3G_DCH, P - c * K3G_DCH);
    for (int e = threadIdx.x; e < E; e += 256) {
        int m = 0;
        for (int i = 0; i < n; ++i) m += keys[i] == e;
        cnt[(size_t)c * E + e] = m;
    }
}

/* One block, a thread per expert: per-chunk bases of each expert's pairs, the expert
 * ranges and the active list. The chunk counts are read 8 at a time so the loads of a
 * thread overlap instead of forming one long dependent chain. */
__global__ void __launch_bounds__(1024)
k_disp_scan(const int32_t *cnt, int nch, int E, int32_t *base, int32_t *off,
            int32_t *act, int32_t *nact)
{
    __shared__ int sc[1024], sa[1024];
    const int e = threadIdx.x;
    int tot = 0;
    if (e < E) {
        int c = 0;
        for (; c + 8 <= nch; c += 8) {
            int v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = cnt[(size_t)(c + u) * E + e];
#pragma unroll
            for (int u = 0; u < 8; ++u) tot += v[u];
        }
        for (; c < nch; ++c) tot += cnt[(size_t)c * E + e];
    }
    /* block-wide inclusive scans of the totals and of the active flags */
    sc[e] = tot;
    sa[e] = tot > 0;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        const int a = e >= d ? sc[e - d] : 0, b = e >= d ? sa[e - d] : 0;
        __syncthreads();
        sc[e] += a;
        sa[e] += b;
        __syncthreads();
    }
    if (e < E) {
        const int first = sc[e] - tot;
        off[e] = first;
        if (tot > 0) act[sa[e] - 1] = e;
        int s = first;
        int c = 0;
        for (; c + 8 <= nch; c += 8) {
            int v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = cnt[(size_t)(c + u) * E + e];
#pragma unroll
            for (int u = 0; u < 8; ++u) { base[(size_t)(c + u) * E + e] = s; s += v[u]; }
        }
        for (; c < nch; ++c) { base[(size_t)c * E + e] = s; s += cnt[(size_t)c * E + e]; }
    }
    if (e == 1023) { off[E] = sc[1023]; *nact = sa[1023]; }
}

__global__ void __launch_bounds__(256)
k_disp_scatter(const int32_t *idx, int P, int E, const int32_t *base, int32_t *perm)
{
    __shared__ int keys[K3G_DCH];
    const int c = blockIdx.x;
    keys[threadIdx.x] = k3d_key(idx, c * K3G_DCH + threadIdx.x, P, E, nullptr);
    __syncthreads();
    const int n = min(K3G_DCH, P - c * K3G_DCH);
    for (int e = threadIdx.x; e < E; e += 256) {
        int pos = base[(size_t)c * E + e];
        for (int i = 0; i < n; ++i)
            if (keys[i] == e) perm[pos++] = c * K3G_DCH + i;
    }
}

extern "C" int k3k_dispatch(const int32_t *idx, int P, int E, int32_t *cnt, int32_t *base,
                            int32_t *off, int32_t *act, int32_t *nact, int32_t *perm,
                            int *err, hipStream_t st)
{
    if (E < 1 || E > K3G_MAX_EXPERTS || P < 1) return -1;
    if (P <= K3G_DCH) {
        hipLaunchKernelGGL(k_disp_small, dim3(1), dim3(256), 0, st, idx, P, E, off, act, nact,
                           perm, err);
    } else if (P <= K3G_DONE) {
        hipLaunchKernelGGL(k_disp_one, dim3(1), dim3(1024), 0, st, idx, P, E, off, act, nact,
                           perm, err);
    } else {
        const int nch = (P + K3G_DCH - 1) / K3G_DCH;
        hipLaunchKernelGGL(k_disp_count, dim3(nch), dim3(256), 0, st, idx, P, E, cnt, err);
        hipLaunchKernelGGL(k_disp_scan, dim3(1), dim3(1024), 0, st, cnt, nch, E, base, off,
                           act, nact);
        hipLaunchKernelGGL(k_disp_scatter, dim3(nch), dim3(256), 0, st, idx, P, E, base, perm);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
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
/* src/core/k3_ops.c:94-102; one token per block. */
__global__ void __launch_bounds__(256)
k_rmsnorm(float *y, const float *x, const float *w, int n, float eps)
{
    __shared__ double part[4];
    const float *xt = x + (size_t)blockIdx.x * n;
    float *yt = y + (size_t)blockIdx.x * n;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) ss = fma((double)xt[i], (double)xt[i], ss);
    ss = k3d_wave_sumd(ss);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const double tot = (part[0] + part[1]) + (part[2] + part[3]);
    const float inv = (float)(1.0 / sqrt(tot / (double)n + (double)eps));
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += 256) yt[i] = __fmul_rn(__fmul_rn(w[i], xt[i]), inv);
}

extern "C" int k3k_rmsnorm(float *y, const float *x, const float *w, int n, int T, float eps,
                           hipStream_t st)
{
    if (T < 1 || n < 1) return 0;
    hipLaunchKernelGGL(k_rmsnorm, dim3(T), dim3(256), 0, st, y, x, w, n, eps);
    return hipGetLastError() == hipSuccess ? 0 : -1;
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
