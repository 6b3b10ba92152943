/* k3g_router.hip - routing on the GPU with a selection bit-exact to the engine's
 * k3_router (src/core/k3_ops.c:419-478).
 *
 * The engine's logit is a SEQUENTIAL double sum of exact products rounded to float,
 * then sigmoid with float expf. A GPU computes the same sum in another order, and a
 * different summation order can move the double result by up to (n-1)*2^-53*sum|p|,
 * enough to change the float logit by one ulp once in a few hundred experts. That only
 * matters for the routing when two choice scores are within a few ulps of each other
 * at a place the top-k depends on, so each token carries a CERTIFICATE:
 *
 *   1. logits in fp64 (one wave per expert row) with sum|w*x| alongside;
 *   2. per expert an interval [lo, hi] that is guaranteed to hold the engine's choice
 *      score: the summation bound of both orders, pushed monotonically through the
 *      float rounding, the sigmoid (+-4 ulp for a libm expf that differs from a
 *      correctly rounded one) and the bias add;
 *   3. top-k on the best guess, accepted when every selected expert's lo is strictly
 *      above the hi of every expert ranked after it.
 *
 * A token that fails recomputes, in the engine's exact serial order, every expert whose
 * interval reaches the weakest selected lo (the only experts that can be in its top-k),
 * and selects among those with the engine's strict-max, lowest-index rule.
 */
#include "k3g_dev.h"
#include "k3g_kernels.h"
#include "k3g_select.h"

#include <math.h>

/* ------------------------------------------------------------------ logits ---- */
/* grid (n_experts, ceil(T / RT)), block = one wave. Lane l reads float4 column chunks
 * 4l, 4l+256, ... of the expert row and of each token's x. */
template <int RT>
__global__ void __launch_bounds__(64)
k_router_logits(const float *__restrict__ x, int T, const float *__restrict__ W,
                const float *__restrict__ bias, int d, int vec, float4 *__restrict__ rs,
                int E)
{
    const int e = blockIdx.x;
    const int t0 = blockIdx.y * RT;
    const int lane = threadIdx.x;
    const float *w = W + (size_t)e * d;
    double acc[RT], ab[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) { acc[t] = 0.0; ab[t] = 0.0; }
    const int d4 = vec ? (d & ~3) : 0;
#ifndef K3R_VALU_UNROLL
#define K3R_VALU_UNROLL 4
#endif
#pragma unroll K3R_VALU_UNROLL
    for (int i = lane * 4; i < d4; i += 256) {
        const float4 wv = *(const float4 *)(w + i);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            if (t0 + t < T) {
                const float4 xv = *(const float4 *)(x + (size_t)(t0 + t) * d + i);
                acc[t] = fma((double)wv.x, (double)xv.x, acc[t]);
                acc[t] = fma((double)wv.y, (double)xv.y, acc[t]);
                acc[t] = fma((double)wv.z, (double)xv.z, acc[t]);
                acc[t] = fma((double)wv.w, (double)xv.w, acc[t]);
                ab[t] = fma(fabs((double)wv.x), fabs((double)xv.x), ab[t]);
                ab[t] = fma(fabs((double)wv.y), fabs((double)xv.y), ab[t]);
                ab[t] = fma(fabs((double)wv.z), fabs((double)xv.z), ab[t]);
                ab[t] = fma(fabs((double)wv.w), fabs((double)xv.w), ab[t]);
            }
        }
    }
    for (int i = d4 + lane; i < d; i += 64) {
#pragma unroll
        for (int t = 0; t < RT; ++t)
            if (t0 + t < T) {
                const double p = (double)w[i] * (double)x[(size_t)(t0 + t) * d + i];
                acc[t] += p;
                ab[t] += fabs(p);
            }
    }
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const double s = k3d_wave_sumd(acc[t]);
        const double a = k3d_wave_sumd(ab[t]);
        if (lane == 0 && t0 + t < T)
            rs[(size_t)(t0 + t) * E + e] = k3d_route_score(s, a, bias ? bias[e] : 0.0f, d);
    }
}

/* ------------------------------------------------- logits on the matrix cores ---- */
/* Many tokens: the logits as a GEMM on v_mfma_f64_16x16x4f64 (fp32 x fp32 products are
 * exact in fp64, the sums are fp64 fused multiply-adds). One wave per 16 experts x 32
 * tokens. In each 16-column step lane L holds columns 4 (L / 16) .. + 3 of expert row
 * L % 16 (A operand) and of token L % 16 (+ 16) (B operand); the four MFMAs of a step
 * take one column each, so both operands come from one 16-byte load per row. The
 * f64 MFMA result puts expert 4 i + L / 16, token L % 16 in item i of lane L.
 * sum|w*x| is bounded by ||w|| ||x|| (Cauchy-Schwarz), both norms summed alongside.
 * With few tiles (S > 1) each tile's columns are cut into S slices taken by S waves; a
 * slice stores its partial sums, and the wave that completes the tile's count (a device
 * atomic) sums the S partials in slice order and forms the scores (any summation order
 * stays inside the interval's bound), then resets the count for the next call. */
typedef double k3v4d __attribute__((ext_vector_type(4)));

#define K3R_RING 4
/* below this many tokens the 16 x 32 tiles are too few to fill the GPU (T = 64: 48
 * waves) and the one-wave-per-(expert, 4 tokens) kernel is faster */
#ifndef K3R_MFMA_MIN_T
#define K3R_MFMA_MIN_T 512
#endif

#define K3R_PART 11    /* doubles per lane of a slice's partial sums */
#define K3R_WPB 4      /* waves per workgroup when K is sliced */

/* A 16-expert x 32-token tile, its K cut into S slices of whole 16-column steps: the
 * workgroups of a tile (G of them, blockDim / 64 waves each, one slice per wave; a wave
 * past S only adds zeros) first add their waves' sums in LDS, then, when G > 1, meet
 * through device-coherent partial sums where the last arrival adds them in group order. */
__global__ void __launch_bounds__(64 * K3R_WPB)
k_router_logits_mfma(const float *__restrict__ x, int T, const float *__restrict__ W,
                     const float *__restrict__ bias, int d, int E, float4 *__restrict__ rs,
                     int S, int G, double *__restrict__ part, int32_t *__restrict__ ctr)
{
    extern __shared__ double k3r_red[];
    const int wpb = blockDim.x >> 6;
    const int nte = E / 16, ntt = (T + 31) / 32, N = nte * ntt * G;
    const int per = (N + 7) >> 3;
    /* block b runs on XCD b % 8: give each XCD a contiguous run, so the expert tiles of
     * one token tile (consecutive) share its x rows in one L2 */
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    if (slot >= per) return;
    const int lam = xcd * per + slot;
    if (lam >= N) return;
    const int tl = lam / G, grp = lam - tl * G;
    const int wv = threadIdx.x >> 6, sl = grp * wpb + wv;
    const int tt = tl / nte, et = tl - tt * nte;
    const int e0 = 16 * et, t0 = 32 * tt;
    const int L = threadIdx.x & 63, g = L >> 4, r = L & 15;
    const int nsteps = d / 16, spp = (nsteps + S - 1) / S;
    const int s_begin = min(nsteps, sl * spp);
    const int s_addr = min(s_begin, nsteps - 1);         /* in the rows even for no steps */
    const float4 *wp = (const float4 *)(W + (size_t)(e0 + r) * d) + g + 4 * s_addr;
    const float4 *ap = (const float4 *)(x + (size_t)min(t0 + r, T - 1) * d) + g + 4 * s_addr;
    const float4 *bp = (const float4 *)(x + (size_t)min(t0 + 16 + r, T - 1) * d) + g + 4 * s_addr;
    const int ns = max(0, min(nsteps, s_begin + spp) - s_begin);
    float4 wq[K3R_RING], av[K3R_RING], bv[K3R_RING];
#pragma unroll
    for (int u = 0; u < K3R_RING; ++u) {
        const int s = max(0, min(u, ns - 1));
        wq[u] = wp[4 * s]; av[u] = ap[4 * s]; bv[u] = bp[4 * s];
    }
    /* two chains per output (even and odd columns of a step), so consecutive MFMAs do
     * not wait for each other's results; they are added at the end */
    k3v4d acc0 = {0.0, 0.0, 0.0, 0.0}, acc1 = {0.0, 0.0, 0.0, 0.0};
    k3v4d acc2 = {0.0, 0.0, 0.0, 0.0}, acc3 = {0.0, 0.0, 0.0, 0.0};
    double ssw = 0.0, ssa = 0.0, ssb = 0.0;
    for (int s0 = 0; s0 < ns; s0 += K3R_RING) {
#pragma unroll
        for (int u = 0; u < K3R_RING; ++u) {
            const float4 w4 = wq[u], a4 = av[u], b4 = bv[u];
            const int sn = max(0, min(s0 + u + K3R_RING, ns - 1));
            wq[u] = wp[4 * sn]; av[u] = ap[4 * sn]; bv[u] = bp[4 * sn];
            if (s0 + u < ns) {
                const double w[4] = {w4.x, w4.y, w4.z, w4.w};
                const double a[4] = {a4.x, a4.y, a4.z, a4.w};
                const double b[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
                for (int k = 0; k < 4; k += 2) {
                    acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64(w[k], a[k], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64(w[k], b[k], acc1, 0, 0, 0);
                    acc2 = __builtin_amdgcn_mfma_f64_16x16x4f64(w[k + 1], a[k + 1], acc2, 0, 0, 0);
                    acc3 = __builtin_amdgcn_mfma_f64_16x16x4f64(w[k + 1], b[k + 1], acc3, 0, 0, 0);
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    ssw = fma(w[k], w[k], ssw);
                    ssa = fma(a[k], a[k], ssa);
                    ssb = fma(b[k], b[k], ssb);
                }
            }
        }
    }
    acc0 += acc2;
    acc1 += acc3;
    if (S > 1) {
        double v[K3R_PART] = {acc0[0], acc0[1], acc0[2], acc0[3], acc1[0], acc1[1],
                              acc1[2], acc1[3], ssw, ssa, ssb};
        if (wpb > 1) {
            /* the workgroup's slices, added in slice order by wave 0 */
            double *mine = k3r_red + ((size_t)wv * 64 + L) * K3R_PART;
#pragma unroll
            for (int i = 0; i < K3R_PART; ++i) mine[i] = v[i];
            __syncthreads();
            if (wv != 0) return;
#pragma unroll
            for (int i = 0; i < K3R_PART; ++i) v[i] = 0.0;
            for (int q = 0; q < wpb; ++q) {
                const double *o = k3r_red + ((size_t)q * 64 + L) * K3R_PART;
#pragma unroll
                for (int i = 0; i < K3R_PART; ++i) v[i] += o[i];
            }
        }
        if (G > 1) {
            /* device-coherent stores of the group's sums, complete before the count moves
             * (no cache writeback or invalidate: the data never sits in a non-coherent
             * cache); the last arrival adds the groups' sums in group order */
            double *pp = part + ((size_t)tl * G + grp) * (64 * K3R_PART) + L * K3R_PART;
#pragma unroll
            for (int i = 0; i < K3R_PART; ++i)
                __hip_atomic_store(pp + i, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);
            asm volatile("" ::: "memory");
            int old = 0;
            /* one count per 128-byte line: counts sharing a line would queue at the L2 */
            if (L == 0) old = __hip_atomic_fetch_add(&ctr[32 * tl], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (__builtin_amdgcn_readfirstlane(old) != G - 1) return;
            asm volatile("" ::: "memory");
            double u[K3R_WPB][K3R_PART];
#pragma unroll
            for (int q = 0; q < K3R_WPB; ++q) {
                const double *qq = part + ((size_t)tl * G + min(q, G - 1)) * (64 * K3R_PART) + L * K3R_PART;
#pragma unroll
                for (int i = 0; i < K3R_PART; ++i)
                    u[q][i] = __hip_atomic_load(qq + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int i = 0; i < K3R_PART; ++i) v[i] = 0.0;
#pragma unroll
            for (int q = 0; q < K3R_WPB; ++q)
                if (q < G) {
#pragma unroll
                    for (int i = 0; i < K3R_PART; ++i) v[i] += u[q][i];
                }
            if (L == 0) __hip_atomic_store(&ctr[32 * tl], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) { acc0[i] = v[i]; acc1[i] = v[4 + i]; }
        ssw = v[8]; ssa = v[9]; ssb = v[10];
    }
    /* norms: sum the four column groups; lane L then holds expert e0 + L % 16 and tokens
     * t0 + L % 16, t0 + 16 + L % 16 */
#pragma unroll
    for (int m = 16; m <= 32; m <<= 1) {
        ssw += __shfl_xor(ssw, m, K3G_WAVE);
        ssa += __shfl_xor(ssa, m, K3G_WAVE);
        ssb += __shfl_xor(ssb, m, K3G_WAVE);
    }
    const double nw = sqrt(ssw), na = sqrt(ssa), nb = sqrt(ssb);
    const double nround = 2.0 * d + 16.0;
    const double margin = 1.0 + 0x1p-40;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int er = 4 * i + g;                         /* expert row of item i */
        const double nwe = __shfl(nw, er, K3G_WAVE);
        const int e = e0 + er;
        const float be = bias ? bias[e] : 0.0f;
        const int ta = t0 + r, tb = t0 + 16 + r;
        if (ta < T) rs[(size_t)ta * E + e] = k3d_route_score_n(acc0[i], nwe * na * margin, be, nround);
        if (tb < T) rs[(size_t)tb * E + e] = k3d_route_score_n(acc1[i], nwe * nb * margin, be, nround);
    }
}

/* ------------------------------------------------------------------ select ---- */
/* One wave per token; a token whose certificate fails computes its candidates' exact
 * logits from rows staged through LDS. */
__global__ void __launch_bounds__(64)
k_router_select(const float4 *__restrict__ rs, const float *__restrict__ bias,
                const float *__restrict__ W, const float *__restrict__ x, int d, int E, int k,
                int renorm, float routed_scale, int32_t *__restrict__ idx,
                float *__restrict__ wt, int force, int *__restrict__ stats)
{
    __shared__ K3SelectLds lds;
    __shared__ __attribute__((aligned(16))) uint8_t stage[K3G_XD_BYTES];
    k3d_select_token(&lds, blockIdx.x, rs, bias, W, x, d, E, k, renorm, routed_scale, idx, wt,
                     force, stats, threadIdx.x, nullptr, stage);
}

/* K slices for the matrix-core logits when the tiles are few: about K3R_WAVES waves, at
 * most K3R_MAXS slices per tile; tiles x groups stays below K3R_WAVES (groups' sums in
 * memory: tiles < 512 and groups <= slices / 4 + 1 <= 1024 / (4 tiles) + 1) */
#define K3R_WAVES 1024
#define K3R_MAXS 16
extern "C" size_t k3k_router_part_bytes(void) { return (size_t)K3R_WAVES * 64 * K3R_PART * 8; }

static int router_slices(int N)
{
    if (N >= 512) return 1;
    const int s = K3R_WAVES / N;
    return s > K3R_MAXS ? K3R_MAXS : (s < 2 ? 2 : s);
}

extern "C" int k3k_router(const float *x, int T, const float *W, const float *bias, int d,
                          int E, int k, int renorm, float routed_scale, float *rs,
                          int32_t *idx, float *wt, int force, int *stats, double *part,
                          int32_t *ctr, hipStream_t st)
{
    if (E > K3G_MAX_E || k > K3G_MAX_TOPK || k < 1 || T < 1 || d < 1) return -1;
    /* the score intervals of token t live at [t][E] */
    /* float4 loads need 16-byte aligned rows; anything else takes the scalar loop */
    const int vec = ((((uintptr_t)x | (uintptr_t)W) & 15) == 0) && ((d & 3) == 0);
    const long long N1 = (long long)(E / 16) * ((T + 31) / 32);
    const bool mfma_ok = T >= 16 && vec && E >= 16 && E % 16 == 0 && d % 64 == 0;
    int S = (mfma_ok && part && ctr && N1 < 512) ? router_slices((int)N1) : 1;
    if (S > 1) {
        /* whole 16-column steps per slice and no empty slice */
        const int nsteps = d / 16;
        if (S > nsteps) S = nsteps;
        const int spp = (nsteps + S - 1) / S;
        S = (nsteps + spp - 1) / spp;
    }
    if (mfma_ok && (S > 1 || T >= K3R_MFMA_MIN_T)) {
        /* slices as the waves of a workgroup (summed in LDS), workgroups of a tile summed
         * through memory */
        const int wpb = S < K3R_WPB ? S : K3R_WPB, G = (S + wpb - 1) / wpb;
        const long long N = N1 * G;
        if (G > 1 && N > K3R_WAVES) return -1;     /* the groups' sums would not fit */
        const size_t lds = wpb > 1 ? (size_t)wpb * 64 * K3R_PART * sizeof(double) : 0;
        hipLaunchKernelGGL(k_router_logits_mfma, dim3((unsigned)(8 * ((N + 7) / 8))),
                           dim3(64 * wpb), lds, st, x, T, W, bias, d, E, (float4 *)rs, S, G,
                           part, ctr);
    } else if (T >= 4) {
        hipLaunchKernelGGL(k_router_logits<4>, dim3(E, (T + 3) / 4), dim3(64), 0, st,
                           x, T, W, bias, d, vec, (float4 *)rs, E);
    } else {
        hipLaunchKernelGGL(k_router_logits<1>, dim3(E, T), dim3(64), 0, st,
                           x, T, W, bias, d, vec, (float4 *)rs, E);
    }
    hipLaunchKernelGGL(k_router_select, dim3(T), dim3(64), 0, st, (const float4 *)rs, bias, W,
                       x, d, E, k, renorm, routed_scale, idx, wt, force, stats);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
