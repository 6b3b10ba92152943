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

/* ------------------------------------------------------------------ select ---- */
/* One wave per token. */
__global__ void __launch_bounds__(64)
k_router_select(const float4 *__restrict__ rs, const float *__restrict__ bias,
                const float *__restrict__ W, const float *__restrict__ x, int d, int E, int k,
                int renorm, float routed_scale, int32_t *__restrict__ idx,
                float *__restrict__ wt, int force, int *__restrict__ stats)
{
    __shared__ K3SelectLds lds;
    k3d_select_token(&lds, blockIdx.x, rs, bias, W, x, d, E, k, renorm, routed_scale, idx, wt,
                     force, stats, threadIdx.x);
}

extern "C" int k3k_router(const float *x, int T, const float *W, const float *bias, int d,
                          int E, int k, int renorm, float routed_scale, float *rs,
                          int32_t *idx, float *wt, int force, int *stats, hipStream_t st)
{
    if (E > K3G_MAX_E || k > K3G_MAX_TOPK || k < 1 || T < 1 || d < 1) return -1;
    /* the score intervals of token t live at [t][E] */
    /* float4 loads need 16-byte aligned rows; anything else takes the scalar loop */
    const int vec = ((((uintptr_t)x | (uintptr_t)W) & 15) == 0) && ((d & 3) == 0);
    if (T >= 4) {
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
