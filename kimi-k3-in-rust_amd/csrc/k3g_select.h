/* k3g_select.h - certified top-k selection for one token, run by one wave. Shared by
 * the standalone router and the fused decode kernel.
 *
 * Inputs are `nparts` partial fp64 logits and partial sum|w*x| per expert, laid out
 * [part][T][E] and added in part order. See k3g_router.hip for the certificate. */
#pragma once

#include "k3g_dev.h"

#define K3G_MAX_E 1024

struct K3SelectLds {
    float choice[K3G_MAX_E];
    float lo[K3G_MAX_E];
    float hi[K3G_MAX_E];
    float score[K3G_MAX_E];
    unsigned char taken[K3G_MAX_E];
    int sel[64];
    int cand[K3G_MAX_E];
    int ncand;
    int cert;
};

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

/* Selection for token t. Only this wave touches `s`; the wave synchronises itself with
 * wave-level barriers (LDS traffic within one wave is ordered by s_waitcnt). */
__device__ __forceinline__ void
k3d_select_token(K3SelectLds *s, int t, int T, int nparts, const double *logit,
                 const double *asum, const float *bias, const float *W, const float *x,
                 int d, int E, int k, int renorm, float routed_scale, int32_t *idx,
                 float *wt, int force, int *stats, int lane)
{
    const double kB = ((double)d * (1.0 + 1.0 / 64.0) + 16.0) * 0x1p-53 * 1.01;
    for (int e = lane; e < E; e += 64) {
        double acc = 0.0, ab = 0.0;
        for (int q = 0; q < nparts; ++q) {
            acc += k3d_ld_dev64(&logit[((size_t)q * T + t) * E + e]);
            ab += k3d_ld_dev64(&asum[((size_t)q * T + t) * E + e]);
        }
        const double B = kB * ab + fabs(acc) * 0x1p-51 + 0x1p-1000;
        const float b = bias ? bias[e] : 0.0f;
        const float sc = k3d_sigmoid((float)acc);
        float slo = k3d_sigmoid((float)(acc - B));
        float shi = k3d_sigmoid((float)(acc + B));
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            slo = nextafterf(slo, -INFINITY);
            shi = nextafterf(shi, INFINITY);
        }
        s->score[e] = sc;
        s->choice[e] = __fadd_rn(sc, b);
        s->lo[e] = __fadd_rn(slo, b);
        s->hi[e] = __fadd_rn(shi, b);
        s->taken[e] = 0;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();

    /* top-k on the best guess */
    for (int j = 0; j < k; ++j) {
        float bv = -INFINITY;
        int bi = -1;
        for (int e = lane; e < E; e += 64) {
            const float c = s->choice[e];
            if (!s->taken[e] && c > bv) { bv = c; bi = e; }
        }
        k3d_argmax(bv, bi);
        if (lane == 0) {
            s->sel[j] = bi;
            if (bi >= 0) s->taken[bi] = 1;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
    }

    /* certificate: every selected lo strictly above the hi of everything ranked after */
    float hrest = -INFINITY;
    for (int e = lane; e < E; e += 64)
        if (!s->taken[e] && s->hi[e] > hrest) hrest = s->hi[e];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) hrest = fmaxf(hrest, __shfl_xor(hrest, m, K3G_WAVE));
    if (lane == 0) {
        int ok = force ? 0 : 1;
        float M = hrest;
        for (int j = k - 1; j >= 0 && ok; --j) {
            const int e = s->sel[j];
            if (e < 0) { ok = 0; break; }
            if (!(s->lo[e] > M)) ok = 0;
            M = fmaxf(M, s->hi[e]);
        }
        s->cert = ok;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();

    if (!s->cert) {
        /* candidates: every expert whose interval reaches the weakest selected lo */
        if (lane == 0) {
            float theta = INFINITY;
            for (int j = 0; j < k; ++j) {
                const int e = s->sel[j];
                theta = e < 0 ? -INFINITY : fminf(theta, s->lo[e]);
            }
            int n = 0;
            for (int e = 0; e < E; ++e)
                if (force == 2 || s->hi[e] >= theta || s->taken[e]) s->cand[n++] = e;
            s->ncand = n;
            if (stats) atomicAdd(&stats[0], 1);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        const int nc = s->ncand;
        const float *xt = x + (size_t)t * d;
        for (int c0 = 0; c0 < nc; c0 += 64) {
            const int c = c0 + lane;
            if (c < nc) {
                const int e = s->cand[c];
                const float *w = W + (size_t)e * d;
                double acc = 0.0;
                for (int i = 0; i < d; ++i) acc = fma((double)w[i], (double)xt[i], acc);
                const float sc = k3d_sigmoid((float)acc);
                s->score[e] = sc;
                s->choice[e] = __fadd_rn(sc, bias ? bias[e] : 0.0f);
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        for (int c = lane; c < nc; c += 64) s->taken[s->cand[c]] = 0;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        for (int j = 0; j < k; ++j) {
            float bv = -INFINITY;
            int bi = -1;
            for (int c = lane; c < nc; c += 64) {
                const int e = s->cand[c];
                const float v = s->choice[e];
                if (!s->taken[e] && (v > bv || (v == bv && bi >= 0 && e < bi))) { bv = v; bi = e; }
            }
            k3d_argmax(bv, bi);
            if (lane == 0) {
                s->sel[j] = bi;
                if (bi >= 0) s->taken[bi] = 1;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_wave_barrier();
        }
    }

    /* weights from the unbiased scores, renormalised in double, then scaled */
    if (lane == 0) {
        float w[64];
        for (int j = 0; j < k; ++j) w[j] = s->sel[j] >= 0 ? s->score[s->sel[j]] : 0.0f;
        if (renorm && k > 1) {
            double sum = 0.0;
            for (int j = 0; j < k; ++j) sum += (double)w[j];
            const float inv = (float)(1.0 / (sum + 1e-20));
            for (int j = 0; j < k; ++j) w[j] = __fmul_rn(w[j], inv);
        }
        for (int j = 0; j < k; ++j) {
            __hip_atomic_store(&idx[(size_t)t * k + j], s->sel[j] >= 0 ? s->sel[j] : 0,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&wt[(size_t)t * k + j], __fmul_rn(w[j], routed_scale),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
}
