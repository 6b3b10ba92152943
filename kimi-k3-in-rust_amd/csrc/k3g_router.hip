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

#include <math.h>

/* ------------------------------------------------------------------ logits ---- */
/* grid (n_experts, ceil(T / RT)), block = one wave. Lane l reads float4 column chunks
 * 4l, 4l+256, ... of the expert row and of each token's x. */
template <int RT>
__global__ void __launch_bounds__(64)
k_router_logits(const float *__restrict__ x, int T, const float *__restrict__ W,
                int d, int vec, double *__restrict__ logit, double *__restrict__ asum,
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
        if (lane == 0 && t0 + t < T) {
            logit[(size_t)(t0 + t) * E + e] = s;
            asum[(size_t)(t0 + t) * E + e] = a;
        }
    }
}

/* ------------------------------------------------------------------ select ---- */
#define K3G_MAX_E 1024

/* (value, index) argmax with the engine's rule: larger value wins, equal values go to
 * the lower index. NaN and -inf never win (the engine's strict > against -inf). */
__device__ __forceinline__ void k3d_argmax(float &v, int &i)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(v, m, K3G_WAVE);
        const int oi = __shfl_xor(i, m, K3G_WAVE);
        if (ov > v || (ov == v && oi >= 0 && (i < 0 || oi < i))) { v = ov; i = oi; }
    }
}

/* One wave per token. */
__global__ void __launch_bounds__(64)
k_router_select(const double *__restrict__ logit, const double *__restrict__ asum,
                const float *__restrict__ bias, const float *__restrict__ W,
                const float *__restrict__ x, int d, int E, int k, int renorm,
                float routed_scale, int32_t *__restrict__ idx, float *__restrict__ wt,
                int force, int *__restrict__ stats)
{
    __shared__ float s_choice[K3G_MAX_E];
    __shared__ float s_lo[K3G_MAX_E];
    __shared__ float s_hi[K3G_MAX_E];
    __shared__ float s_score[K3G_MAX_E];
    __shared__ unsigned char s_taken[K3G_MAX_E];
    __shared__ int s_sel[K3G_MAX_TOPK];
    __shared__ int s_cand[K3G_MAX_E];
    __shared__ int s_ncand;
    __shared__ int s_cert;

    const int t = blockIdx.x;
    const int lane = threadIdx.x;
    const double *lg = logit + (size_t)t * E;
    const double *as = asum + (size_t)t * E;
    const double kB = ((double)d * (1.0 + 1.0 / 64.0) + 16.0) * 0x1p-53 * 1.01;

    for (int e = lane; e < E; e += 64) {
        const double acc = lg[e];
        const double B = kB * as[e] + fabs(acc) * 0x1p-51 + 0x1p-1000;
        const float b = bias ? bias[e] : 0.0f;
        const float s = k3d_sigmoid((float)acc);
        float slo = k3d_sigmoid((float)(acc - B));
        float shi = k3d_sigmoid((float)(acc + B));
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            slo = nextafterf(slo, -INFINITY);
            shi = nextafterf(shi, INFINITY);
        }
        s_score[e] = s;
        s_choice[e] = __fadd_rn(s, b);
        s_lo[e] = __fadd_rn(slo, b);
        s_hi[e] = __fadd_rn(shi, b);
        s_taken[e] = 0;
    }
    __syncthreads();

    /* top-k on the best guess */
    for (int j = 0; j < k; ++j) {
        float bv = -INFINITY;
        int bi = -1;
        for (int e = lane; e < E; e += 64) {
            const float c = s_choice[e];
            if (!s_taken[e] && c > bv) { bv = c; bi = e; }
        }
        k3d_argmax(bv, bi);
        if (lane == 0) {
            s_sel[j] = bi;
            if (bi >= 0) s_taken[bi] = 1;
        }
        __syncthreads();
    }

    /* certificate: every selected lo strictly above the hi of everything ranked after */
    float hrest = -INFINITY;
    for (int e = lane; e < E; e += 64)
        if (!s_taken[e] && s_hi[e] > hrest) hrest = s_hi[e];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) hrest = fmaxf(hrest, __shfl_xor(hrest, m, K3G_WAVE));
    if (lane == 0) {
        int ok = force ? 0 : 1;
        float M = hrest;
        for (int j = k - 1; j >= 0 && ok; --j) {
            const int e = s_sel[j];
            if (e < 0) { ok = 0; break; }
            if (!(s_lo[e] > M)) ok = 0;
            M = fmaxf(M, s_hi[e]);
        }
        s_cert = ok;
    }
    __syncthreads();

    if (!s_cert) {
        /* candidates: every expert whose interval reaches the weakest selected lo */
        if (lane == 0) {
            float theta = INFINITY;
            for (int j = 0; j < k; ++j) {
                const int e = s_sel[j];
                theta = e < 0 ? -INFINITY : fminf(theta, s_lo[e]);
            }
            int n = 0;
            for (int e = 0; e < E; ++e)
                if (force == 2 || s_hi[e] >= theta || s_taken[e]) s_cand[n++] = e;
            s_ncand = n;
            if (stats) atomicAdd(&stats[0], 1);
        }
        __syncthreads();
        const int nc = s_ncand;
        const float *xt = x + (size_t)t * d;
        for (int c0 = 0; c0 < nc; c0 += 64) {
            const int c = c0 + lane;
            if (c < nc) {
                const int e = s_cand[c];
                const float *w = W + (size_t)e * d;
                double acc = 0.0;
                for (int i = 0; i < d; ++i) acc = fma((double)w[i], (double)xt[i], acc);
                const float s = k3d_sigmoid((float)acc);
                s_score[e] = s;
                s_choice[e] = __fadd_rn(s, bias ? bias[e] : 0.0f);
            }
        }
        __syncthreads();
        for (int c = lane; c < nc; c += 64) s_taken[s_cand[c]] = 0;
        __syncthreads();
        for (int j = 0; j < k; ++j) {
            float bv = -INFINITY;
            int bi = -1;
            for (int c = lane; c < nc; c += 64) {
                const int e = s_cand[c];
                const float v = s_choice[e];
                if (!s_taken[e] && (v > bv || (v == bv && bi >= 0 && e < bi))) { bv = v; bi = e; }
            }
            k3d_argmax(bv, bi);
            if (lane == 0) {
                s_sel[j] = bi;
                if (bi >= 0) s_taken[bi] = 1;
            }
            __syncthreads();
        }
    }

    /* weights from the unbiased scores, renormalised in double, then scaled */
    if (lane == 0) {
        float w[K3G_MAX_TOPK];
        for (int j = 0; j < k; ++j) w[j] = s_sel[j] >= 0 ? s_score[s_sel[j]] : 0.0f;
        if (renorm && k > 1) {
            double s = 0.0;
            for (int j = 0; j < k; ++j) s += (double)w[j];
            const float inv = (float)(1.0 / (s + 1e-20));
            for (int j = 0; j < k; ++j) w[j] = __fmul_rn(w[j], inv);
        }
        for (int j = 0; j < k; ++j) {
            idx[(size_t)t * k + j] = s_sel[j] >= 0 ? s_sel[j] : 0;
            wt[(size_t)t * k + j] = __fmul_rn(w[j], routed_scale);
        }
    }
}

extern "C" int k3k_router(const float *x, int T, const float *W, const float *bias, int d,
                          int E, int k, int renorm, float routed_scale, double *logit,
                          double *asum, int32_t *idx, float *wt, int force, int *stats,
                          hipStream_t st)
{
    if (E > K3G_MAX_E || k > K3G_MAX_TOPK || k < 1 || T < 1 || d < 1) return -1;
    /* float4 loads need 16-byte aligned rows; anything else takes the scalar loop */
    const int vec = ((((uintptr_t)x | (uintptr_t)W) & 15) == 0) && ((d & 3) == 0);
    if (T >= 4) {
        hipLaunchKernelGGL(k_router_logits<4>, dim3(E, (T + 3) / 4), dim3(64), 0, st,
                           x, T, W, d, vec, logit, asum, E);
    } else {
        hipLaunchKernelGGL(k_router_logits<1>, dim3(E, T), dim3(64), 0, st,
                           x, T, W, d, vec, logit, asum, E);
    }
    hipLaunchKernelGGL(k_router_select, dim3(T), dim3(64), 0, st, logit, asum, bias, W, x,
                       d, E, k, renorm, routed_scale, idx, wt, force, stats);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
