/* k3g_select.h - the router's score intervals and the certified top-k for one token, run
 * by one wave. Shared by the standalone router and the fused decode kernel.
 *
 * The engine's logit is a SEQUENTIAL double sum of exact products rounded to float,
 * then sigmoid with float expf (src/core/k3_ops.c:419-478). A GPU sums in another order,
 * so the kernels that form the logits (one wave per expert row) also form, per expert, an
 * interval [lo, hi] guaranteed to hold the engine's choice score, and store
 * {choice, lo, hi, score} per (token, expert). The selection then runs on the best
 * guess and accepts it when every selected lo is strictly above the hi of every expert
 * ranked after it; otherwise it recomputes the candidates in the engine's exact serial
 * order. */
#pragma once

#include "k3g_dev.h"

#define K3G_MAX_E 1024

/* 0: always the k rounds of k3d_select_token_n (the threshold path is skipped) */
#ifndef K3G_SELECT_FAST
#define K3G_SELECT_FAST 1
#endif

/* k3d_select_fast's LDS: the candidates (keys, lo, hi, score) and the selection by rank */
struct K3RankLds {
    unsigned long long ckey[64], rkey[64];
    float clo[64], chi[64], csc[64];
    float rlo[64], rhi[64], rsc[64];
    int rsel[64];
};

struct K3SelectLds {
    float choice[K3G_MAX_E];
    float lo[K3G_MAX_E];
    float hi[K3G_MAX_E];
    float score[K3G_MAX_E];
    unsigned char taken[K3G_MAX_E];
    int sel[64];
    int cand[K3G_MAX_E];
    int redo[K3G_MAX_E];
    int ncand, nredo;
    int cert;
    double wsum;
    K3RankLds rk;
};

/* {choice, lo, hi, score} of one expert from its fp64 logit sum `acc` and a bound `ab` on
 * sum|w*x|:
 *   |acc - engine's double sum| <= B = nround 2^-53 ab 1.01 + |acc| 2^-51,
 * where nround counts the roundings of both summation orders (d (1 + 1/64) + 16 for a
 * lane-strided tree of d products, 2 d + 16 for a chain of fused multiply-adds); the
 * bound is pushed through the float rounding and the sigmoid (monotone) and widened by
 * 4 ulp for a libm expf that differs from a correctly rounded one, then the bias is added
 * (monotone again). When acc -/+ B round to the same float, that float is the engine's
 * float logit and score/choice are the engine's values (with its expf): the interval's
 * upper end then carries an even bit pattern, otherwise an odd one (moving it up by at
 * most one ulp, so it stays an upper bound); k3d_settled reads the mark. */
__device__ __forceinline__ float4 k3d_route_score_n(double acc, double ab, float bias,
                                                     double nround)
{
    const double kB = nround * 0x1p-53 * 1.01;
    const double B = kB * ab + fabs(acc) * 0x1p-51 + 0x1p-1000;
    const float sc = k3d_sigmoid((float)acc);
    float slo = k3d_sigmoid((float)(acc - B));
    float shi = k3d_sigmoid((float)(acc + B));
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        slo = nextafterf(slo, -INFINITY);
        shi = nextafterf(shi, INFINITY);
    }
    float hi = __fadd_rn(shi, bias);
    const bool settled = (float)(acc - B) == (float)(acc + B);
    if ((int)(__float_as_uint(hi) & 1u) != (settled ? 0 : 1)) hi = nextafterf(hi, INFINITY);
    return make_float4(__fadd_rn(sc, bias), __fadd_rn(slo, bias), hi, sc);
}

/* The mark k3d_route_score_n leaves on an interval's upper end: true when the score and
 * choice were formed from the engine's own float logit. */
__device__ __forceinline__ bool k3d_settled(float hi)
{
    return __builtin_isfinite(hi) && !(__float_as_uint(hi) & 1u);
}

__device__ __forceinline__ float4 k3d_route_score(double acc, double ab, float bias, int d)
{
    return k3d_route_score_n(acc, ab, bias, (double)d * (1.0 + 1.0 / 64.0) + 16.0);
}

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

/* Wave-wide maximum with DPP row shifts and row broadcasts (no LDS round trips): every
 * lane returns the maximum. */
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t k3d_dpp(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROWS, 0xf, false);
}

template <int CTRL, int ROWS>
__device__ __forceinline__ uint64_t k3d_dpp_max_step(uint64_t k)
{
    const uint64_t o = ((uint64_t)k3d_dpp<CTRL, ROWS>((uint32_t)(k >> 32)) << 32) |
                       k3d_dpp<CTRL, ROWS>((uint32_t)k);
    return o > k ? o : k;
}

__device__ __forceinline__ uint64_t k3d_wave_max_u64(uint64_t k)
{
    k = k3d_dpp_max_step<0x111, 0xf>(k);   /* row_shr:1 */
    k = k3d_dpp_max_step<0x112, 0xf>(k);   /* row_shr:2 */
    k = k3d_dpp_max_step<0x114, 0xf>(k);   /* row_shr:4 */
    k = k3d_dpp_max_step<0x118, 0xf>(k);   /* row_shr:8 */
    k = k3d_dpp_max_step<0x142, 0xa>(k);   /* row_bcast:15 */
    k = k3d_dpp_max_step<0x143, 0xc>(k);   /* row_bcast:31 */
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(k >> 32), 63);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)k, 63);
    return ((uint64_t)hi << 32) | lo;
}

/* fmaxf over the wave (NaN ignored, as fmaxf does) */
__device__ __forceinline__ float k3d_wave_fmax(float v)
{
#define K3_FMAX_STEP(C, R) v = fmaxf(v, __uint_as_float(k3d_dpp<C, R>(__float_as_uint(v))));
    K3_FMAX_STEP(0x111, 0xf) K3_FMAX_STEP(0x112, 0xf) K3_FMAX_STEP(0x114, 0xf)
    K3_FMAX_STEP(0x118, 0xf) K3_FMAX_STEP(0x142, 0xa) K3_FMAX_STEP(0x143, 0xc)
#undef K3_FMAX_STEP
    return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 63));
}

/* float -> uint32 with the same order (for finite and infinite values) */
__device__ __forceinline__ uint32_t k3d_ordered(float f)
{
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* The engine's logit: sum_i w[i] x[i] in double, strictly in index order (each product
 * is exact, so a fused multiply-add rounds exactly like the engine's add). The sum is one
 * dependent chain; the operands stream in 16-byte loads issued two groups ahead so the
 * chain, not the loads, sets the pace. */
__device__ __noinline__ double k3d_serial_dot(const float *w, const float *x, int d)
{
    double acc = 0.0;
    int i = 0;
    if (((((uintptr_t)w | (uintptr_t)x) & 15) == 0) && d >= 32) {
        const float4 *w4 = (const float4 *)w, *x4 = (const float4 *)x;
        const int n4 = d / 4;
        float4 wa[4], xa[4], wb[4], xb[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) { wa[u] = w4[u]; xa[u] = x4[u]; }
#pragma unroll
        for (int u = 0; u < 4; ++u) { wb[u] = w4[4 + u]; xb[u] = x4[4 + u]; }
        int q = 0;
        for (; q + 8 <= n4; q += 4) {
            float4 wn[4], xn[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int qq = min(q + 8 + u, n4 - 1);
                wn[u] = w4[qq]; xn[u] = x4[qq];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                acc = fma((double)wa[u].x, (double)xa[u].x, acc);
                acc = fma((double)wa[u].y, (double)xa[u].y, acc);
                acc = fma((double)wa[u].z, (double)xa[u].z, acc);
                acc = fma((double)wa[u].w, (double)xa[u].w, acc);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) { wa[u] = wb[u]; xa[u] = xb[u]; wb[u] = wn[u]; xb[u] = xn[u]; }
        }
        i = 4 * q;
    }
    for (; i < d; ++i) acc = fma((double)w[i], (double)x[i], acc);
    return acc;
}

/* LDS staging for the candidates' logits (k3d_fast_dots_staged): two stages of up to
 * K3G_XD_ROWS candidate rows + the token's x, 256 fp32 columns each. Rows are skewed by
 * 16 bytes so that the lanes' row reads fall on different banks. */
#define K3G_XD_ROWS 6
#define K3G_XD_ROWB 1040                                  /* 256 fp32 + 16 */
#define K3G_XD_STAGE ((K3G_XD_ROWS + 1) * K3G_XD_ROWB)
#define K3G_XD_BYTES (2 * K3G_XD_STAGE)

/* Logits of nb <= K3G_XD_ROWS candidate rows against x in any summation order, with what
 * bounds their distance from the engine's serial sums: lane j < nb returns in s row j's
 * sum of exact fp64 products w_i x_i and in a the sum of their magnitudes. Any two
 * summation orders of n terms differ by at most 2 gamma_(n-1) sum |w_i x_i|, so when the
 * float roundings of s -/+ that bound agree, they are the float the engine casts its
 * serial sum to. The rows and x stream through LDS by DMA, 256 columns per stage with the
 * next stage in flight; every lane multiplies its 4 columns of each row and keeps the row
 * sums in registers, and a wave reduction ends the row. d a multiple of 4, rows and x
 * 16-byte aligned. */
__device__ __forceinline__ void k3d_fast_dots_staged(uint8_t *stage,
                                                    const float *const (&rows)[K3G_XD_ROWS],
                                                    int nb, const float *x, int d, int lane,
                                                    double &s, double &a)
{
    const uint32_t base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)stage;
    const int nch = (d + 255) / 256;
    auto issue = [&](int k) {
        const int col = min(256 * k + 4 * lane, d - 4);
        const uint32_t st = base + (uint32_t)(k & 1) * K3G_XD_STAGE;
#pragma unroll
        for (int j = 0; j < K3G_XD_ROWS; ++j)
            if (j < nb) k3d_dma16(rows[j] + col, st + j * K3G_XD_ROWB);
        k3d_dma16(x + col, st + nb * K3G_XD_ROWB);
    };
    double rs[K3G_XD_ROWS], ra[K3G_XD_ROWS];
#pragma unroll
    for (int j = 0; j < K3G_XD_ROWS; ++j) { rs[j] = 0.0; ra[j] = 0.0; }
    issue(0);
    for (int k = 0; k < nch; ++k) {
        if (k + 1 < nch) {
            issue(k + 1);
            k3d_wait_vm(nb + 1);          /* stage k landed; stage k + 1 in flight */
        } else {
            k3d_wait_vm(0);
        }
        __builtin_amdgcn_wave_barrier();
        const uint8_t *st = stage + (k & 1) * K3G_XD_STAGE;
        /* columns past d (a re-read of the row's last 16 bytes) are not summed */
        if (256 * k + 4 * lane < d) {
            const float4 xv = *(const float4 *)(st + nb * K3G_XD_ROWB + 16 * lane);
#pragma unroll
            for (int j = 0; j < K3G_XD_ROWS; ++j) {
                if (j < nb) {
                    const float4 wv = *(const float4 *)(st + j * K3G_XD_ROWB + 16 * lane);
                    const double p0 = (double)wv.x * xv.x, p1 = (double)wv.y * xv.y;
                    const double p2 = (double)wv.z * xv.z, p3 = (double)wv.w * xv.w;
                    rs[j] += (p0 + p1) + (p2 + p3);
                    ra[j] += (fabs(p0) + fabs(p1)) + (fabs(p2) + fabs(p3));
                }
            }
        }
        /* every lane is done with this stage before the next issue refills it */
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }
    s = 0.0;
    a = 0.0;
#pragma unroll
    for (int j = 0; j < K3G_XD_ROWS; ++j) {
        if (j < nb) {
            const double vs = k3d_wave_sumd(rs[j]), va = k3d_wave_sumd(ra[j]);
            if (lane == j) { s = vs; a = va; }
        }
    }
}

/* The engine's float logit for one row, from a wave. The engine adds the row's d exact
 * products p_i serially in double, s^_i = fl(s^_(i-1) + p_i), and that sum is within
 * u sum_i |s^_i| of the exact one (u = 2^-53; Higham, Accuracy and Stability, 4.2) --
 * a bound in the partial sums' magnitudes, far tighter than one in sum |p_i|. Lane l adds
 * a contiguous block of the row in the engine's order, keeping its block sum b_l and the
 * sum L_l of its local partial sums' magnitudes; a wave scan gives each block its starting
 * partial sum P_l, so sum_i |s_i| <= sum_l (n_l |P_l| + L_l). The lanes' own sums err by
 * at most u L_l each and the scan by gamma_7 sum_l |b_l|. When s -/+ that total bound
 * round to the same float, that float is the engine's; returns false otherwise. d a
 * multiple of 4, w and x 16-byte aligned. */
__device__ __forceinline__ bool k3d_row_logit(const float *w, const float *x, int d, int lane,
                                             float *f)
{
    const float4 *w4 = (const float4 *)w, *x4 = (const float4 *)x;
    const int n4 = d / 4, per = (n4 + 63) / 64;
    const int q0 = min(lane * per, n4), q1 = min(q0 + per, n4);
    double b = 0.0, L = 0.0;
    for (int q = q0; q < q1; q += 8) {
        float4 wv[8], xv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int qq = min(q + u, q1 - 1);
            wv[u] = w4[qq];
            xv[u] = x4[qq];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (q + u < q1) {
                b += (double)wv[u].x * xv[u].x; L += fabs(b);
                b += (double)wv[u].y * xv[u].y; L += fabs(b);
                b += (double)wv[u].z * xv[u].z; L += fabs(b);
                b += (double)wv[u].w * xv[u].w; L += fabs(b);
            }
        }
    }
    /* inclusive scan of the block sums; P = the partial sum before this block */
    double inc = b;
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) {
        const double o = __shfl_up(inc, m, K3G_WAVE);
        if (lane >= m) inc += o;
    }
    const double P = inc - b;
    const double nl = 4.0 * (q1 - q0);
    const double part = nl * fabs(P) + 2.0 * L, mag = fabs(b);
    const double sp = k3d_wave_sumd(part), sm = k3d_wave_sumd(mag);
    const double sum = __shfl(inc, 63, K3G_WAVE);
    const double B = 1.05 * 0x1p-53 * sp + 8.0 * 0x1p-53 * sm + fabs(sum) * 0x1p-52 + 0x1p-1060;
    const float lo = (float)(sum - B), hi = (float)(sum + B);
    *f = lo;
    return lo == hi;
}

/* The float the engine casts its serial fp64 sum to, from a sum s of the same n exact
 * products in another order and the sum a of their magnitudes: true when the bound
 * settles it (*f set), false when s lies too close to a float rounding boundary. */
__device__ __forceinline__ bool k3d_settled_float(double s, double a, int n, float *f)
{
    /* 2 gamma_(n-1) a, with a itself a rounded sum (a factor 1.01 covers both), plus the
     * rounding of s -/+ B */
    const double B = 2.02 * (double)n * 0x1p-53 * a + fabs(s) * 0x1p-52 + 0x1p-1060;
    const float lo = (float)(s - B), hi = (float)(s + B);
    *f = lo;
    return lo == hi;
}

/* The top-k and its certificate without k dependent rounds. th = the k-th largest of the
 * 64 lanes' best ordered choices (a bitwise search on ballot counts) is at most the k-th
 * largest choice overall, so the keys whose ordered choice reaches th hold the top k.
 * When there are at most 64 of them they go to LDS, and each one's rank is the number of
 * candidates with a larger key (the keys are distinct: they carry the index), which is
 * its round in the engine's order. Lane r < k then holds the r-th selection, and the
 * certificate is the rounds' one: every selected hi (r > 0) below the smallest lo
 * selected before it (a prefix minimum over the lanes), no NaN lo. Returns false, with
 * nothing changed, when fewer than k lanes hold a key or the candidates are more than 64;
 * the rounds then run as before. */
template <int NPL>
__device__ __forceinline__ bool k3d_select_fast(K3RankLds *s, const uint64_t (&key)[NPL],
                                                const float4 (&v)[NPL], int k, int lane,
                                                uint32_t &taken, bool &ok, float &minlo,
                                                double &wsum, int &my_sel, float &my_score,
                                                float &my_hi)
{
    uint64_t m = key[0];
#pragma unroll
    for (int i = 1; i < NPL; ++i) m = key[i] > m ? key[i] : m;
    const uint32_t mh = (uint32_t)(m >> 32);
    uint32_t th = 0;
    for (int b = 31; b >= 0; --b) {
        const uint32_t c = th | (1u << b);
        if (__popcll(__ballot(mh >= c)) >= k) th = c;
    }
    if (th == 0) return false;              /* fewer than k lanes hold a valid key */
    int total = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) total += __popcll(__ballot((uint32_t)(key[i] >> 32) >= th));
    if (total > 64) return false;
    const uint64_t lt = (1ull << lane) - 1;
    int base = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const bool c = (uint32_t)(key[i] >> 32) >= th;
        const uint64_t bm = __ballot(c);
        if (c) {
            const int pos = base + __popcll(bm & lt);
            s->ckey[pos] = key[i];
            s->clo[pos] = v[i].y;
            s->chi[pos] = v[i].z;
            s->csc[pos] = v[i].w;
        }
        base += __popcll(bm);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    /* lane j holds candidate j; its rank from the other candidates' keys read across the
     * wave (register reads, no LDS round trip per candidate) */
    const uint64_t mine = lane < total ? s->ckey[lane] : 0;
    const uint32_t mhi = (uint32_t)(mine >> 32), mlo = (uint32_t)mine;
    int rank = 0;
    for (int q = 0; q < total; ++q) {
        const uint32_t oh = (uint32_t)__builtin_amdgcn_readlane((int)mhi, q);
        const uint32_t ol = (uint32_t)__builtin_amdgcn_readlane((int)mlo, q);
        rank += (((uint64_t)oh << 32) | ol) > mine ? 1 : 0;
    }
    if (lane < total && rank < k) {
        s->rkey[rank] = mine;
        s->rsel[rank] = (int)~(uint32_t)mine;
        s->rlo[rank] = s->clo[lane];
        s->rhi[rank] = s->chi[lane];
        s->rsc[rank] = s->csc[lane];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    float lo = INFINITY, hi = 0.0f, sc = 0.0f;
    if (lane < k) {
        my_sel = s->rsel[lane];
        lo = s->rlo[lane];
        hi = s->rhi[lane];
        sc = s->rsc[lane];
        my_score = sc;
        my_hi = hi;
    }
    /* inclusive prefix minimum of the selected lo (fminf: NaN ignored, as the rounds'
     * running minimum ignores it), and the exclusive one for the check */
    float inc = lo;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float u = __shfl_up(inc, o, K3G_WAVE);
        if (lane >= o) inc = fminf(inc, u);
    }
    float ex = __shfl_up(inc, 1, K3G_WAVE);
    if (lane == 0) ex = INFINITY;
    const bool bad = lane < k && ((lane > 0 && !__builtin_isnan(hi) && !(hi < ex)) ||
                                  __builtin_isnan(lo));
    if (__ballot(bad)) ok = false;
    minlo = __shfl(inc, k - 1, K3G_WAVE);
    /* the engine's sequential double sum in selection order */
    double ws = 0.0;
    for (int r = 0; r < k; ++r)
        ws += (double)__uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(sc), r));
    wsum = ws;
    /* the k-th selected key (readfirstlane returns int: widen each half unsigned) */
    const uint32_t kh = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(s->rkey[k - 1] >> 32));
    const uint32_t kl = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)s->rkey[k - 1]);
    const uint64_t kth = ((uint64_t)kh << 32) | kl;
#pragma unroll
    for (int i = 0; i < NPL; ++i)
        if (key[i] != 0 && key[i] >= kth) taken |= 1u << i;
    return true;
}

/* Selection for token t from rs [T][E] {choice, lo, hi, score} (read at device
 * coherence: the fused kernel's router tickets write them in the same launch). Each lane
 * owns experts lane, lane + 64, ... (NPL of them); all loads are issued before any is
 * used. The top-k runs in registers: per round a lane proposes its best untaken choice and
 * a DPP maximum over (ordered choice, ~index) keys picks the engine's winner (larger
 * value, then lower index). The certificate is checked along the way: with the rounds in
 * choice order, "every selected lo above the hi of everything ranked after it" is "each
 * new hi below the smallest lo selected before it" plus "the smallest selected lo above
 * the largest unselected hi". LDS is only used when the certificate fails. Returns the
 * certified selections whose scores are not settled (bit j: round j; 0 after the exact
 * path), for k3d_fix_unsettled. */
template <int NPL>
__device__ __noinline__ uint64_t
k3d_select_token_n(K3SelectLds *s, int t, const float4 *rs, const float *bias,
                   const float *W, const float *x, int d, int E, int k, int renorm,
                   float routed_scale, int32_t *idx, float *wt, int force, int *stats,
                   int lane, unsigned long long *stamp, uint8_t *stage)
{
    const int nb = (t + 1) * E * 16;
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float4 *>(rs), (short)0, nb, 0x00020000);
    float4 v[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int e = lane + 64 * i;
        /* experts past E read past the descriptor's bound: zero, no memory access */
        const int off = e < E ? (t * E + e) * 16 : nb;
        v[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rr, off, 0, 16));
    }
    if (stamp && lane == 0) stamp[0] = wall_clock64();

    /* the engine's order as one unsigned key per expert: (ordered choice, ~index); 0 for
     * experts that cannot win (past E, NaN or -inf choice) or are taken */
    uint64_t key[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int e = lane + 64 * i;
        key[i] = e < E && v[i].x > -INFINITY
                     ? ((uint64_t)k3d_ordered(v[i].x) << 32) | (uint32_t)~e : 0;
    }
    uint32_t taken = 0;
    bool ok = !force;
    float minlo = INFINITY;
    double wsum = 0.0;
    int my_sel = -1;          /* lane j: the j-th selected expert */
    float my_score = 0.0f, my_hi = 0.0f;
    const bool fast = K3G_SELECT_FAST &&
                      k3d_select_fast<NPL>(&s->rk, key, v, k, lane, taken, ok, minlo, wsum, my_sel,
                                           my_score, my_hi);
    for (int j = 0; j < (fast ? 0 : k); ++j) {
        /* this lane's best untaken key: a tree over the slots */
        uint64_t m[NPL];
#pragma unroll
        for (int i = 0; i < NPL; ++i) m[i] = key[i];
#pragma unroll
        for (int h = NPL / 2; h >= 1; h /= 2)
#pragma unroll
            for (int i = 0; i < h; ++i) m[i] = m[i + h] > m[i] ? m[i + h] : m[i];
        const uint64_t win = k3d_wave_max_u64(m[0]);
        const int w = win ? (int)~(uint32_t)win : -1;       /* uniform */
        float wlo = 0.0f, whi = 0.0f, wsc = 0.0f;
        if (w >= 0) {
            const int slot = w >> 6, wl = w & 63;           /* uniform */
            float lo = 0.0f, hi = 0.0f, sc = 0.0f;
#pragma unroll
            for (int i = 0; i < NPL; ++i)
                if (i == slot) {
                    lo = v[i].y; hi = v[i].z; sc = v[i].w;
                    if (lane == wl) key[i] = 0;
                }
            wlo = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(lo), wl));
            whi = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(hi), wl));
            wsc = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(sc), wl));
            if (lane == wl) taken |= 1u << slot;
            if (j > 0 && !__builtin_isnan(whi) && !(whi < minlo)) ok = false;
            if (__builtin_isnan(wlo)) ok = false;
            minlo = fminf(minlo, wlo);
            wsum += (double)wsc;
        } else {
            ok = false;
        }
        if (lane == j) { my_sel = w; my_score = w >= 0 ? wsc : 0.0f; my_hi = whi; }
    }
    /* the selections whose score is not settled (bit j: round j) */
    const uint64_t unsettled = __ballot(lane < k && my_sel >= 0 && !k3d_settled(my_hi));
    float hrest = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPL; ++i)
        if (lane + 64 * i < E && !((taken >> i) & 1u)) hrest = fmaxf(hrest, v[i].z);
    hrest = k3d_wave_fmax(hrest);
    if (!(minlo > hrest)) ok = false;
    if (stamp && lane == 0) stamp[1] = wall_clock64();

    if (!ok) {
        /* the exact path: LDS copies, candidates (every expert whose interval reaches the
         * weakest selected lo), their logits in the engine's serial order, and the
         * engine's selection among them */
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int e = lane + 64 * i;
            if (e < E) {
                s->choice[e] = v[i].x;
                s->lo[e] = v[i].y;
                s->hi[e] = v[i].z;
                s->score[e] = v[i].w;
                s->taken[e] = (taken >> i) & 1u;
            }
        }
        if (lane < k) s->sel[lane] = my_sel;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        /* theta: the weakest selected lo (lane j < k holds the j-th selection) */
        float nth = -INFINITY;
        if (lane < k) nth = my_sel < 0 ? INFINITY : -s->lo[my_sel];
        const float theta = -k3d_wave_fmax(nth);
        /* candidates in expert order, and among them those whose float logit the bound
         * left open (all when forced), by ballots over the lanes' slots */
        int nc = 0, nr = 0;
        const uint64_t lt = (1ull << lane) - 1;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
            const int e = lane + 64 * i;
            const bool cf = e < E && (force >= 2 || v[i].z >= theta || ((taken >> i) & 1u));
            const bool rf = cf && (force >= 2 || !k3d_settled(v[i].z));
            const uint64_t cm = __ballot(cf), rm = __ballot(rf);
            if (cf) s->cand[nc + __popcll(cm & lt)] = e;
            if (rf) s->redo[nr + __popcll(rm & lt)] = e;
            nc += __popcll(cm);
            nr += __popcll(rm);
        }
        if (lane == 0) {
            s->ncand = nc;
            s->nredo = nr;
            if (stats) atomicAdd(&stats[0], 1);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        const float *xt = x + (size_t)t * d;
        const bool staged = stage && d % 4 == 0 && d >= 4 &&
                            ((((uintptr_t)W | (uintptr_t)x) & 15) == 0);
        const int per = staged ? K3G_XD_ROWS : 64;
        /* the settled candidates' scores and choices are the engine's already; the rest
         * get the engine's float logit */
        for (int c0 = 0; c0 < nr; c0 += per) {
            const int c = c0 + lane;
            double ps = 0.0, pa = 0.0;
            if (staged) {
                const float *rows[K3G_XD_ROWS];
                const int nb = min(K3G_XD_ROWS, nr - c0);
#pragma unroll
                for (int j = 0; j < K3G_XD_ROWS; ++j)
                    rows[j] = W + (size_t)__builtin_amdgcn_readfirstlane(
                                      s->redo[c0 + (j < nb ? j : 0)]) * d;
                k3d_fast_dots_staged(stage, rows, nb, xt, d, lane, ps, pa);
            }
            if (lane < per && c < nr) {
                const int e = s->redo[c];
                /* the engine's float logit: settled by the bound, else its serial chain
                 * (always the chain when force > 2) */
                float logit;
                if (!staged || force > 2 || !k3d_settled_float(ps, pa, d, &logit))
                    logit = (float)k3d_serial_dot(W + (size_t)e * d, xt, d);
                const float sc = k3d_sigmoid(logit);
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
                const float cv = s->choice[e];
                if (!s->taken[e] && (cv > bv || (cv == bv && bi >= 0 && e < bi))) { bv = cv; bi = e; }
            }
            k3d_argmax(bv, bi);
            if (lane == 0) {
                s->sel[j] = bi;
                if (bi >= 0) s->taken[bi] = 1;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_wave_barrier();
        }
        /* the engine's sequential double sum over the new selection */
        if (lane == 0) {
            double sum = 0.0;
            for (int j = 0; j < k; ++j) sum += s->sel[j] >= 0 ? (double)s->score[s->sel[j]] : 0.0;
            s->wsum = sum;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        wsum = s->wsum;
        if (lane < k) {
            my_sel = s->sel[lane];
            my_score = my_sel >= 0 ? s->score[my_sel] : 0.0f;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
    }

    /* weights from the unbiased scores, renormalised by the engine's sequential double
     * sum (taken in selection order above), then scaled; lane j writes slot j */
    if (stamp && lane == 0) stamp[2] = wall_clock64();
    if (lane < k) {
        float w = my_score;
        if (renorm && k > 1) w = __fmul_rn(w, (float)(1.0 / (wsum + 1e-20)));
        __hip_atomic_store(&idx[(size_t)t * k + lane], my_sel >= 0 ? my_sel : 0,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&wt[(size_t)t * k + lane], __fmul_rn(w, routed_scale),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    /* the exact path formed every score it selected from the engine's float logit */
    return ok ? unsettled : 0;
}

/* A certified selection's weights are its scores, and a score the bound left unsettled
 * may not be the engine's (its float logit within the bound of a rounding boundary): the
 * order stands (the intervals hold the engine's choices), so only those scores are
 * recomputed -- k3d_row_logit reads the row straight from memory, one block per lane, and
 * its partial-sum bound settles the engine's float logit; the serial chain only when it
 * does not -- and the token's weights are formed again from all k scores (the engine's
 * sequential double sum in selection order). Out of line and after the selection, so the
 * selection's common path keeps its registers. */
__device__ __noinline__ void k3d_fix_unsettled(int t, const float4 *rs, const float *W,
                                               const float *x, int d, int E, int k, int renorm,
                                               float routed_scale, int32_t *idx, float *wt,
                                               int *stats, int lane, uint64_t unsettled)
{
    if (stats && lane == 0) atomicAdd(&stats[1], __popcll(unsettled));
    const float *xt = x + (size_t)t * d;
    int sel = 0;
    float score = 0.0f;
    if (lane < k) {
        sel = __hip_atomic_load(&idx[(size_t)t * k + lane], __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
        score = rs[(size_t)t * E + sel].w;
    }
    const bool vec = d % 4 == 0 && ((((uintptr_t)W | (uintptr_t)x) & 15) == 0);
    for (uint64_t m = unsettled; m; m &= m - 1) {
        const int j = __builtin_ctzll(m);
        const int e = __builtin_amdgcn_readlane(sel, j);
        float logit;
        if (!vec || !k3d_row_logit(W + (size_t)e * d, xt, d, lane, &logit))
            logit = (float)k3d_serial_dot(W + (size_t)e * d, xt, d);
        if (lane == j) score = k3d_sigmoid(logit);
    }
    double wsum = 0.0;
    for (int j = 0; j < k; ++j)
        wsum += (double)__uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(score), j));
    if (lane < k) {
        float w = score;
        if (renorm && k > 1) w = __fmul_rn(w, (float)(1.0 / (wsum + 1e-20)));
        __hip_atomic_store(&wt[(size_t)t * k + lane], __fmul_rn(w, routed_scale),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

/* k3d_select_token_n with the per-lane count chosen for E (<= K3G_MAX_E), then the
 * unsettled scores of a certified selection recomputed. */
__device__ __forceinline__ void
k3d_select_token(K3SelectLds *s, int t, const float4 *rs, const float *bias, const float *W,
                 const float *x, int d, int E, int k, int renorm, float routed_scale,
                 int32_t *idx, float *wt, int force, int *stats, int lane,
                 unsigned long long *stamp = nullptr, uint8_t *stage = nullptr)
{
    uint64_t um;
    if (E <= 256)
        um = k3d_select_token_n<4>(s, t, rs, bias, W, x, d, E, k, renorm, routed_scale, idx,
                                   wt, force, stats, lane, stamp, stage);
    else if (E <= 512)
        um = k3d_select_token_n<8>(s, t, rs, bias, W, x, d, E, k, renorm, routed_scale, idx,
                                   wt, force, stats, lane, stamp, stage);
    else
        um = k3d_select_token_n<16>(s, t, rs, bias, W, x, d, E, k, renorm, routed_scale, idx,
                                    wt, force, stats, lane, stamp, stage);
    if (um)
        k3d_fix_unsettled(t, rs, W, x, d, E, k, renorm, routed_scale, idx, wt, stats, lane, um);
}

#define K3G_PICK_RB 8     /* candidate rows per pass of the exact logits */

/* a candidate's float logit the any-order bound left open: the partial-sum bound, else the
 * engine's serial chain (always the chain when force > 2). Inline, so that the kernel's
 * register budget holds for it too (a call would size the kernel by its callee). */
__device__ __forceinline__ float k3d_open_logit(const float *row, const float *xt, int d,
                                               int lane, int force)
{
    float g;
    if (force <= 2 && k3d_row_logit(row, xt, d, lane, &g)) return g;
    const float4 *w4 = (const float4 *)row, *x4 = (const float4 *)xt;
    double acc = 0.0;
#pragma unroll 8
    for (int q = 0; q < d / 4; ++q) {
        const float4 wv = w4[q], xv = x4[q];
        acc = fma((double)wv.x, (double)xv.x, acc);
        acc = fma((double)wv.y, (double)xv.y, acc);
        acc = fma((double)wv.z, (double)xv.z, acc);
        acc = fma((double)wv.w, (double)xv.w, acc);
    }
    return (float)acc;
}

/* 1 / (1 + e^-v) with the hardware exponential: within a few float ulps */
__device__ __forceinline__ float k3d_sig_fast(float v) { return 1.0f / (1.0f + __expf(-v)); }

/* Row j < NB's fp64 dot product with x (acc[2 j]) and the sum of its products' magnitudes
 * (acc[2 j + 1]), this lane's share: columns 2 lane + 128 q, two per 128-column stage,
 * with two stages in flight. d a multiple of 256, rows and x 8-byte aligned. */
template <int NB>
__device__ __forceinline__ void k3d_cand_dots(const float *const *rows, const float *xt, int d,
                                        int lane, double *acc)
{
    const float2 *x2 = (const float2 *)xt;
    const int nq = d / 128;
    float2 xs[3], ws[3][NB];
    auto ld = [&](int slot, int q) {
        const int o = min(q, nq - 1) * 64 + lane;
        xs[slot] = x2[o];
#pragma unroll
        for (int j = 0; j < NB; ++j) ws[slot][j] = ((const float2 *)rows[j])[o];
    };
    ld(0, 0);
    ld(1, 1);
    for (int q0 = 0; q0 < nq; q0 += 3) {
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            ld((u + 2) % 3, q0 + u + 2);
            if (q0 + u < nq) {
                const double x0 = xs[u].x, x1 = xs[u].y;
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const double w0 = ws[u][j].x, w1 = ws[u][j].y;
                    acc[2 * j] = fma(w1, x1, fma(w0, x0, acc[2 * j]));
                    acc[2 * j + 1] = fma(fabs(w1), fabs(x1), fma(fabs(w0), fabs(x0), acc[2 * j + 1]));
                }
            }
        }
    }
}

/* One token's routing from bounded approximate logits, run by one wave: part holds the
 * approximate logits [T][E] (fp32), wn2 the experts' squared norms, xn2 the tokens'; the
 * logit of (t, e) is within nround 2^-53 1.01 ||w_e|| ||x_t|| + |a| 2^-51 of the engine's
 * double sum (the norms widened by 2^-10 here). Choice bounds from that interval, top-k
 * on the guesses, the candidates (every expert whose upper bound reaches the weakest
 * selected lower bound: the engine's top-k lies among them; all experts when the guesses
 * cannot select k or are not numbers, or when force >= 2), their fp64 logits (the
 * engine's float logit settled by the any-order bound, else by the partial-sum bound,
 * else the serial chain; always the chain when force > 2), and the engine's selection
 * among the candidates with its weights. cand, cch and csc are this wave's LDS lists of
 * K3G_MAX_E entries. cnt: [0] more candidates than k, [1] candidate logits the any-order
 * bound left open, [2] candidates whose fp64 logit fell outside the bounded interval. */
template <int NPL>
__device__ __forceinline__ void
k3d_pick_token(int t, const float *part, const float *xn2, const float *wn2, const float *bias,
               const float *W, const float *x, int d, int E, int k, int renorm,
               float routed_scale, int32_t *idx, float *wt, int force, double nround, int *cand,
               float *cch, float *csc, int lane, int (&cnt)[3])
{
    const double xn = sqrt((double)xn2[t]) * (1.0 + 0x1p-10);
    /* the approximate logit and its norm product */
    auto approx = [&](int e, float &a, double &ab) {
        a = part[(size_t)t * E + e];
        ab = sqrt((double)wn2[e]) * (1.0 + 0x1p-10) * xn;
    };
    /* every load issued before any is used */
    float av[NPL], wv[NPL], bv[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int e = min(lane + 64 * i, E - 1);
        av[i] = part[(size_t)t * E + e];
        wv[i] = wn2[e];
        bv[i] = bias ? bias[e] : 0.0f;
    }
    float4 v[NPL];
    uint64_t key[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int e = lane + 64 * i;
        v[i] = make_float4(-INFINITY, -INFINITY, -INFINITY, 0.0f);
        key[i] = 0;
        if (e < E) {
            /* the engine's float logit lies in [fl(a - B), fl(a + B)] (rounding is
             * monotone); the choice bounds follow in fast float arithmetic with 2^-16
             * (1 + |bias|) of slack, which covers the fast exp, the engine's expf and the
             * roundings of the sigmoid and the bias add. Only the candidate set depends on
             * them. */
            const double a = av[i];
            const double B = nround * 0x1p-53 * 1.01 * (sqrt((double)wv[i]) * (1.0 + 0x1p-10) * xn) +
                             fabs(a) * 0x1p-51 + 0x1p-1000;
            const float slack = 0x1p-16f * (1.0f + fabsf(bv[i]));
            v[i].x = k3d_sig_fast((float)a) + bv[i];
            v[i].y = k3d_sig_fast((float)(a - B)) + bv[i] - slack;
            v[i].z = k3d_sig_fast((float)(a + B)) + bv[i] + slack;
            if (v[i].x > -INFINITY)
                key[i] = ((uint64_t)k3d_ordered(v[i].x) << 32) | (uint32_t)~e;
        }
    }
    /* top-k on the guesses: theta = the weakest selected lower end */
    uint32_t taken = 0;
    bool valid = true;
    float theta = INFINITY;
    for (int j = 0; j < k; ++j) {
        uint64_t m[NPL];
#pragma unroll
        for (int i = 0; i < NPL; ++i) m[i] = key[i];
#pragma unroll
        for (int h = NPL / 2; h >= 1; h /= 2)
#pragma unroll
            for (int i = 0; i < h; ++i) m[i] = m[i + h] > m[i] ? m[i + h] : m[i];
        const uint64_t win = k3d_wave_max_u64(m[0]);
        if (!win) { valid = false; break; }
        const int w = (int)~(uint32_t)win, slot = w >> 6, wl = w & 63;
        float lo = 0.0f;
#pragma unroll
        for (int i = 0; i < NPL; ++i)
            if (i == slot) {
                lo = v[i].y;
                if (lane == wl) { key[i] = 0; taken |= 1u << i; }
            }
        const float wlo = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(lo), wl));
        if (__builtin_isnan(wlo)) valid = false;
        theta = fminf(theta, wlo);
    }
    if (!valid || force >= 2) theta = -INFINITY;
    /* candidates in expert order (a NaN upper end is a candidate) */
    int nc = 0;
    const uint64_t lt = (1ull << lane) - 1;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        const int e = lane + 64 * i;
        const bool cf = e < E && (((taken >> i) & 1u) || !(v[i].z < theta));
        const uint64_t cm = __ballot(cf);
        if (cf) cand[nc + __popcll(cm & lt)] = e;
        nc += __popcll(cm);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();

    /* the candidates' float logits */
    const float *xt = x + (size_t)t * d;
    int nopen = 0, nviol = 0;
    for (int c0 = 0; c0 < nc; c0 += K3G_PICK_RB) {
        const int nb = min(K3G_PICK_RB, nc - c0);
        const float *rows[K3G_PICK_RB];
#pragma unroll
        for (int j = 0; j < K3G_PICK_RB; ++j)
            rows[j] = W + (size_t)__builtin_amdgcn_readfirstlane(cand[c0 + min(j, nb - 1)]) * d;
        double acc[2 * K3G_PICK_RB];
#pragma unroll
        for (int j = 0; j < 2 * K3G_PICK_RB; ++j) acc[j] = 0.0;
        switch (nb) {
        case 1: k3d_cand_dots<1>(rows, xt, d, lane, acc); break;
        case 2: k3d_cand_dots<2>(rows, xt, d, lane, acc); break;
        case 3: k3d_cand_dots<3>(rows, xt, d, lane, acc); break;
        case 4: k3d_cand_dots<4>(rows, xt, d, lane, acc); break;
        case 5: k3d_cand_dots<5>(rows, xt, d, lane, acc); break;
        case 6: k3d_cand_dots<6>(rows, xt, d, lane, acc); break;
        case 7: k3d_cand_dots<7>(rows, xt, d, lane, acc); break;
        default: k3d_cand_dots<8>(rows, xt, d, lane, acc); break;
        }
        /* lane l then holds value l >> 2: row j's sum at lane 8 j, its magnitude at 8 j + 4 */
        k3d_transpose_reduce<2 * K3G_PICK_RB>(acc, lane);
        const double sj = __shfl(acc[0], (8 * lane) & 63, K3G_WAVE);
        const double aj = __shfl(acc[0], (8 * lane + 4) & 63, K3G_WAVE);
        float f = 0.0f;
        bool ok = false;
        if (lane < nb) ok = force <= 2 && k3d_settled_float(sj, aj, d, &f);
        const uint64_t um = __ballot(lane < nb && !ok);
        nopen += __popcll(um);
        for (uint64_t m = um; m; m &= m - 1) {
            const int j = __builtin_ctzll(m);
            const float *row = W + (size_t)__builtin_amdgcn_readfirstlane(cand[c0 + j]) * d;
            const float g = k3d_open_logit(row, xt, d, lane, force);
            if (lane == j) f = g;
        }
        bool viol = false;
        if (lane < nb) {
            const int e = cand[c0 + lane];
            const float sc = k3d_sigmoid(f);
            csc[c0 + lane] = sc;
            cch[c0 + lane] = __fadd_rn(sc, bias ? bias[e] : 0.0f);
            float a;
            double ab;
            approx(e, a, ab);
            const double B = nround * 0x1p-53 * 1.01 * ab + fabs((double)a) * 0x1p-51;
            const double df = fabs((double)f - (double)a);
            viol = __builtin_isfinite(f) && __builtin_isfinite(a) && __builtin_isfinite(B) &&
                   df > B + fabs((double)f) * 0x1p-23;
        }
        nviol += __popcll(__ballot(viol));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();

    /* the engine's selection among the candidates: larger choice, then lower index (the
     * candidates are in expert order, so the lower candidate slot); NaN and -inf never win */
    const int nsl = (nc + 63) >> 6;
    uint32_t tk = 0;
    int my_sel = -1;
    float my_score = 0.0f;
    for (int j = 0; j < k; ++j) {
        uint64_t best = 0;
        for (int q = 0; q < nsl; ++q) {
            const int c = lane + 64 * q;
            if (c < nc && !((tk >> q) & 1u)) {
                const float ch = cch[c];
                if (ch > -INFINITY) {
                    const uint64_t kk = ((uint64_t)k3d_ordered(ch) << 32) | (uint32_t)~c;
                    best = kk > best ? kk : best;
                }
            }
        }
        const uint64_t win = k3d_wave_max_u64(best);
        int sel = -1;
        float sc = 0.0f;
        if (win) {
            const int c = (int)~(uint32_t)win;
            sel = cand[c];
            sc = csc[c];
            if (lane == (c & 63)) tk |= 1u << (c >> 6);
        }
        if (lane == j) { my_sel = sel; my_score = sc; }
    }
    /* weights from the unbiased scores, renormalised by the engine's sequential double sum
     * in selection order, then scaled */
    double wsum = 0.0;
    for (int j = 0; j < k; ++j)
        wsum += (double)__uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(my_score), j));
    if (lane < k) {
        float wgt = my_score;
        if (renorm && k > 1) wgt = __fmul_rn(wgt, (float)(1.0 / (wsum + 1e-20)));
        idx[(size_t)t * k + lane] = my_sel >= 0 ? my_sel : 0;
        wt[(size_t)t * k + lane] = __fmul_rn(wgt, routed_scale);
    }
    cnt[0] = nc > k;
    cnt[1] = nopen;
    cnt[2] = nviol;
}
