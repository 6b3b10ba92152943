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

/* ------------------------------ many tokens: bounded logits on the bf16 matrix cores ---- */
/* From a few hundred tokens on, the fp64 logits of every (token, expert) pair cost more
 * than the routing needs: only the k selected scores must be the engine's exactly, and
 * which experts those are is decided by a handful per token. So the logits are first
 * formed on the bf16 matrix cores with a rigorous error bound (k_router_bf3), and only the
 * experts whose bounded choice score can reach the token's top-k get their fp64 logit
 * (k_router_pick).
 *
 * With w = w0 + w1 + ew and x = x0 + x1 + ex split into bf16 pieces, each rounded to
 * nearest even (|w1| <= 2^-8 |w|, |ew| <= 2^-16 |w|, likewise for x), the three products
 * w0 x0 + w0 x1 + w1 x0 differ from w x by at most 3.02 2^-16 |w x|, and each is exact in
 * fp32. v_mfma_f32_16x16x32_bf16 sums them into fp32 accumulators that restart every 128
 * columns (384 terms per chunk); the chunk sums are added in fp32, within a K slice and
 * then over the slices in slice order. With each addition within 2^-23 of its result (an
 * accumulator that aligns and truncates its products stays within that per product), the
 * total errs by at most 1.02 (384 + d/128) 2^-23 sum |w x|. The bound used is twice the sum
 * of both terms, on ||w|| ||x|| >= sum |w x| (norms from fp32 sums of squares, widened by
 * 2^-10); it also covers the engine's own double rounding (< 2^-40 relative). */
#define RB_TILE 128                 /* experts x tokens per workgroup tile */
#define RB_OPB 16384                /* one operand's two pieces, 128 rows x 64 B each */
#define RB_MIN_T 512                /* from this many tokens on */

typedef __bf16 k3v2bfr __attribute__((ext_vector_type(2)));
typedef __bf16 k3v8bfr __attribute__((ext_vector_type(8)));
typedef float k3v4fr __attribute__((ext_vector_type(4)));

static double rb_bound(int d)
{
    return 2.0 * (3.02 * 0x1p-16 + 1.02 * (400.0 + d / 128) * 0x1p-23);
}

/* 8 fp32 values -> their two bf16 pieces, 16 bytes each */
__device__ __forceinline__ void rb_pieces(float4 a, float4 b, uint4 &p0, uint4 &p1)
{
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const k3v2f f = {v[2 * i], v[2 * i + 1]};
        const k3v2bfr hb = __builtin_convertvector(f, k3v2bfr);
        const k3v2f r = f - __builtin_convertvector(hb, k3v2f);      /* exact */
        const k3v2bfr lb = __builtin_convertvector(r, k3v2bfr);
        h[i] = __builtin_bit_cast(uint32_t, hb);
        l[i] = __builtin_bit_cast(uint32_t, lb);
    }
    p0 = make_uint4(h[0], h[1], h[2], h[3]);
    p1 = make_uint4(l[0], l[1], l[2], l[3]);
}

__device__ __forceinline__ float rb_sq(float4 a, float4 b, float s)
{
    s = fmaf(a.x, a.x, s); s = fmaf(a.y, a.y, s); s = fmaf(a.z, a.z, s); s = fmaf(a.w, a.w, s);
    s = fmaf(b.x, b.x, s); s = fmaf(b.y, b.y, s); s = fmaf(b.z, b.z, s); s = fmaf(b.w, b.w, s);
    return s;
}

__device__ __forceinline__ k3v4fr rb_mma(uint4 a, uint4 b, k3v4fr c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(k3v8bfr, a),
                                                   __builtin_bit_cast(k3v8bfr, b), c, 0, 0, 0);
}

/* One workgroup = a 128-expert x 128-token tile over one K slice of whole 128-column
 * chunks; wave w takes experts 64 (w >> 1) .. + 63 and tokens 64 (w & 1) .. + 63 as 4 x 4
 * blocks of 16 x 16. Per 32-column step the workgroup converts its W and x rows to bf16
 * pieces in registers and stores them in LDS (two stages; each row's four 16-byte column
 * groups XOR-swizzled by (row >> 2) & 3, so that the operand reads of 16 consecutive rows
 * hit 64 distinct banks); the next step's rows are loaded before the current step's matrix
 * work. Partial sums go to part[s][t][e]; the workgroups of expert tile 0 also sum x's
 * squares (xn2[s][t]) and those of token tile 0 W's (wn2[s][e]). Workgroups of one token
 * tile and slice are consecutive on one XCD, sharing its x rows in that L2. */
template <bool X1>
__device__ __forceinline__ void
rb_tile(const float *__restrict__ x, int T, const float *__restrict__ W, int d, int E, int S,
        float *__restrict__ part, float *__restrict__ xn2, float *__restrict__ wn2, uint8_t *lds)
{
    const int nte = (E + RB_TILE - 1) / RB_TILE, ntt = (T + RB_TILE - 1) / RB_TILE;
    const int N = nte * ntt * S, per = (N + 7) >> 3;
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int lam = xcd * per + slot;
    if (slot >= per || lam >= N) return;
    const int et = lam % nte, rest = lam / nte, s = rest % S, tt = rest / S;
    const int e0 = RB_TILE * et, t0 = RB_TILE * tt;
    const int nch = d / 128, cps = (nch + S - 1) / S;
    const int cb = min(nch, s * cps), ce = min(nch, cb + cps);
    const int nst = 4 * (ce - cb);
    const int tid = threadIdx.x, w = tid >> 6, L = tid & 63;

    /* staging units tid and tid + 256: row u >> 2, columns 8 (u & 3) .. + 7 of the step */
    const int r0 = tid >> 2, r1 = r0 + 64, cc = tid & 3;
    const bool we0 = e0 + r0 < E, we1 = e0 + r1 < E, xe0 = t0 + r0 < T, xe1 = t0 + r1 < T;
    const size_t kb = (size_t)cb * 128 + 8 * cc;
    const float *wp0 = W + (size_t)min(e0 + r0, E - 1) * d + kb;
    const float *wp1 = W + (size_t)min(e0 + r1, E - 1) * d + kb;
    const float *xp0 = x + (size_t)min(t0 + r0, T - 1) * d + kb;
    const float *xp1 = x + (size_t)min(t0 + r1, T - 1) * d + kb;
    const uint32_t so0 = r0 * 64 + 16 * (cc ^ ((r0 >> 2) & 3));
    const uint32_t so1 = r1 * 64 + 16 * (cc ^ ((r1 >> 2) & 3));
    const bool do_x = et == 0, do_w = tt == 0;
    float xs0 = 0.0f, xs1 = 0.0f, ws0 = 0.0f, ws1 = 0.0f;

    float4 g[8];
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    /* rows past E or T load a valid row (the pointers are clamped) and are zeroed after */
    auto gload = [&](int st) {
        const int k = 32 * st;
        g[0] = *(const float4 *)(wp0 + k);
        g[1] = *(const float4 *)(wp0 + k + 4);
        g[2] = *(const float4 *)(wp1 + k);
        g[3] = *(const float4 *)(wp1 + k + 4);
        g[4] = *(const float4 *)(xp0 + k);
        g[5] = *(const float4 *)(xp0 + k + 4);
        g[6] = *(const float4 *)(xp1 + k);
        g[7] = *(const float4 *)(xp1 + k + 4);
    };
    auto stage = [&](int buf) {
        uint8_t *b = lds + buf * 2 * RB_OPB;
        if (!we0) { g[0] = z4; g[1] = z4; }
        if (!we1) { g[2] = z4; g[3] = z4; }
        if (!xe0) { g[4] = z4; g[5] = z4; }
        if (!xe1) { g[6] = z4; g[7] = z4; }
        uint4 p0, p1;
        rb_pieces(g[0], g[1], p0, p1);
        *(uint4 *)(b + so0) = p0;
        *(uint4 *)(b + 8192 + so0) = p1;
        rb_pieces(g[2], g[3], p0, p1);
        *(uint4 *)(b + so1) = p0;
        *(uint4 *)(b + 8192 + so1) = p1;
        rb_pieces(g[4], g[5], p0, p1);
        *(uint4 *)(b + RB_OPB + so0) = p0;
        *(uint4 *)(b + RB_OPB + 8192 + so0) = p1;
        rb_pieces(g[6], g[7], p0, p1);
        *(uint4 *)(b + RB_OPB + so1) = p0;
        *(uint4 *)(b + RB_OPB + 8192 + so1) = p1;
        if (do_w) { ws0 = rb_sq(g[0], g[1], ws0); ws1 = rb_sq(g[2], g[3], ws1); }
        if (do_x) { xs0 = rb_sq(g[4], g[5], xs0); xs1 = rb_sq(g[6], g[7], xs1); }
    };

    const int wr = w >> 1, wc = w & 1, rr = L & 15, cq = L >> 4;
    const uint32_t sw = 16 * (cq ^ ((rr >> 2) & 3));
    const uint32_t ao = (64 * wr + rr) * 64 + sw, bo = RB_OPB + (64 * wc + rr) * 64 + sw;
    k3v4fr acc[4][4], tot[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) tot[i][j] = k3v4fr{0.0f, 0.0f, 0.0f, 0.0f};

    if (nst > 0) {
        gload(0);
        stage(0);
        if (nst > 1) gload(1);
        __syncthreads();
    }
    for (int st0 = 0; st0 < nst; st0 += 4) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int st = st0 + q;
            /* the next step's rows into the other stage (free since the last barrier), the
             * one after into registers, then this step's matrix work */
            if (st + 1 < nst) stage((st + 1) & 1);
            if (st + 2 < nst) gload(st + 2);
            const uint8_t *b = lds + (st & 1) * 2 * RB_OPB;
            uint4 b0[4], b1[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                b0[j] = *(const uint4 *)(b + bo + j * 1024);
                if (X1) b1[j] = *(const uint4 *)(b + bo + 8192 + j * 1024);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 a0 = *(const uint4 *)(b + ao + i * 1024);
                const uint4 a1 = *(const uint4 *)(b + ao + 8192 + i * 1024);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    k3v4fr c = q == 0 ? k3v4fr{0.0f, 0.0f, 0.0f, 0.0f} : acc[i][j];
                    c = rb_mma(a0, b0[j], c);
                    if (X1) c = rb_mma(a0, b1[j], c);
                    acc[i][j] = rb_mma(a1, b0[j], c);
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) tot[i][j] += acc[i][j];
    }

    /* lane L of block (i, j): experts 4 (L >> 4) + 0..3, token L & 15 */
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int t = t0 + 64 * wc + 16 * j + rr;
        if (t < T) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = e0 + 64 * wr + 16 * i + 4 * cq;
                if (e < E) *(k3v4fr *)(part + ((size_t)s * T + t) * E + e) = tot[i][j];
            }
        }
    }
    if (do_x || do_w) {
        /* the four units of a row are lanes 4m .. 4m + 3 */
        xs0 += __shfl_xor(xs0, 1, K3G_WAVE); xs0 += __shfl_xor(xs0, 2, K3G_WAVE);
        xs1 += __shfl_xor(xs1, 1, K3G_WAVE); xs1 += __shfl_xor(xs1, 2, K3G_WAVE);
        ws0 += __shfl_xor(ws0, 1, K3G_WAVE); ws0 += __shfl_xor(ws0, 2, K3G_WAVE);
        ws1 += __shfl_xor(ws1, 1, K3G_WAVE); ws1 += __shfl_xor(ws1, 2, K3G_WAVE);
        if (cc == 0) {
            if (do_x && xe0) xn2[(size_t)s * T + t0 + r0] = xs0;
            if (do_x && xe1) xn2[(size_t)s * T + t0 + r1] = xs1;
            if (do_w && we0) wn2[(size_t)s * E + e0 + r0] = ws0;
            if (do_w && we1) wn2[(size_t)s * E + e0 + r1] = ws1;
        }
    }
}

/* x1flag (optional): nonzero when some x has a nonzero second bf16 piece; when it reads
 * zero every x is a bf16 value and its w0 x1 product is skipped (it would add zeros). */
__global__ void __launch_bounds__(256, 2)
k_router_bf3(const float *__restrict__ x, int T, const float *__restrict__ W, int d, int E,
             int S, float *__restrict__ part, float *__restrict__ xn2, float *__restrict__ wn2,
             const int32_t *__restrict__ x1flag)
{
    __shared__ __attribute__((aligned(16))) uint8_t lds[4 * RB_OPB];
    if (!x1flag || *x1flag)
        rb_tile<true>(x, T, W, d, E, S, part, xn2, wn2, lds);
    else
        rb_tile<false>(x, T, W, d, E, S, part, xn2, wn2, lds);
}

/* The K slices' sums of k_router_bf3 added in slice order into slice 0 (the logits four
 * experts per thread, then the squared norms), so that the per-token pass reads one value
 * per expert. */
__global__ void __launch_bounds__(256)
k_router_bf3_sum(float *__restrict__ part, int S, int T, int E, float *__restrict__ xn2,
                 float *__restrict__ wn2)
{
    const size_t n4 = (size_t)T * E / 4, stride = (size_t)gridDim.x * 256;
    const size_t TE = (size_t)T * E;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4 + T + E; i += stride) {
        if (i < n4) {
            k3v4fr a = *(const k3v4fr *)(part + 4 * i);
            for (int s = 1; s < S; ++s) a += *(const k3v4fr *)(part + s * TE + 4 * i);
            *(k3v4fr *)(part + 4 * i) = a;
        } else if (i < n4 + T) {
            const size_t t = i - n4;
            float a = xn2[t];
            for (int s = 1; s < S; ++s) a += xn2[(size_t)s * T + t];
            xn2[t] = a;
        } else {
            const size_t e = i - n4 - T;
            float a = wn2[e];
            for (int s = 1; s < S; ++s) a += wn2[(size_t)s * E + e];
            wn2[e] = a;
        }
    }
}

/* One wave per token after k_router_bf3 (k3d_pick_token), four tokens per workgroup. */
template <int NPL>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
k_router_pick(const float *__restrict__ part, const float *__restrict__ xn2,
              const float *__restrict__ wn2, const float *__restrict__ bias,
              const float *__restrict__ W, const float *__restrict__ x, int T, int d, int E, int k,
              int renorm, float routed_scale, int32_t *__restrict__ idx,
              float *__restrict__ wt, int force, int *__restrict__ tstat, double nround)
{
    /* each wave with its own LDS lists */
    __shared__ int cand_s[4][K3G_MAX_E];
    __shared__ float cch_s[4][K3G_MAX_E], csc_s[4][K3G_MAX_E];
    const int wq = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t = 4 * blockIdx.x + wq;
    if (t >= T) return;
    int cnt[3];
    k3d_pick_token<NPL>(t, part, xn2, wn2, bias, W, x, d, E, k, renorm, routed_scale, idx, wt,
                        force, nround, cand_s[wq], cch_s[wq], csc_s[wq], lane, cnt);
    /* per-token counts (4096 waves adding into one address would queue at the L2) */
    if (lane == 0) *(int4 *)(tstat + 4 * (size_t)t) = make_int4(cnt[0], cnt[1], cnt[2], 0);
}

/* The per-token counts of k_router_pick added into the context's statistics */
__global__ void __launch_bounds__(256)
k_router_stats(const int4 *__restrict__ tstat, int T, int *__restrict__ stats)
{
    __shared__ int red[3][4];
    int a = 0, b = 0, c = 0;
    for (int t = threadIdx.x; t < T; t += 256) {
        const int4 v = tstat[t];
        a += v.x; b += v.y; c += v.z;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        a += __shfl_xor(a, m, K3G_WAVE);
        b += __shfl_xor(b, m, K3G_WAVE);
        c += __shfl_xor(c, m, K3G_WAVE);
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { red[0][w] = a; red[1][w] = b; red[2][w] = c; }
    __syncthreads();
    if (threadIdx.x < 3) {
        const int s = red[threadIdx.x][0] + red[threadIdx.x][1] + red[threadIdx.x][2] +
                      red[threadIdx.x][3];
        if (s) atomicAdd(&stats[threadIdx.x], s);
    }
}

/* K slices of the bounded logits wanted for T tokens: about 512 (tile, slice) workgroups,
 * at least one slice (the launch further bounds it by the workspace and by d / 128) */
static int rb_slices(int T, int E)
{
    const int nmn = ((E + RB_TILE - 1) / RB_TILE) * ((T + RB_TILE - 1) / RB_TILE);
    const int s = 512 / nmn;
    return s < 1 ? 1 : s;
}

/* floats of workspace the bounded-logit path needs for T tokens (0 below its range): its
 * K slices of partial sums and norms, then 4 ints of counts per token */
extern "C" size_t k3k_router_bf3_floats(int T, int E)
{
    if (T < RB_MIN_T) return 0;
    const int S = rb_slices(T, E);
    return (size_t)(S < 8 ? S : 8) * ((size_t)T * E + T + E) + 4 * (size_t)T;
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
                          int32_t *ctr, float *bpart, size_t bpart_floats,
                          const int32_t *x1flag, hipStream_t st)
{
    if (E > K3G_MAX_E || k > K3G_MAX_TOPK || k < 1 || T < 1 || d < 1) return -1;
    /* float4 loads need 16-byte aligned rows; anything else takes the scalar loop */
    const int vec = ((((uintptr_t)x | (uintptr_t)W) & 15) == 0) && ((d & 3) == 0);
    if (bpart && T >= RB_MIN_T && vec && E % 16 == 0 && d % 256 == 0) {
        /* bounded bf16 logits, then the candidates' fp64 logits: about two workgroups per
         * CU of K slices, whole 128-column chunks each, no empty slice */
        const int nmn = ((E + RB_TILE - 1) / RB_TILE) * ((T + RB_TILE - 1) / RB_TILE);
        const int nch = d / 128;
        const size_t per_s = (size_t)T * E + T + E;
        const size_t room = bpart_floats > 4 * (size_t)T ? bpart_floats - 4 * (size_t)T : 0;
        int *tstat = (int *)(bpart + room);
        int S = rb_slices(T, E);
        if ((size_t)S * per_s > room) S = (int)(room / per_s);
        if (S > nch) S = nch;
        if (S >= 1) {
            const int cps = (nch + S - 1) / S;
            S = (nch + cps - 1) / cps;
            float *xn2 = bpart + (size_t)S * T * E, *wn2 = xn2 + (size_t)S * T;
            const long long N = (long long)nmn * S;
            hipLaunchKernelGGL(k_router_bf3, dim3((unsigned)(8 * ((N + 7) / 8))), dim3(256), 0,
                               st, x, T, W, d, E, S, bpart, xn2, wn2, x1flag);
            if (S > 1) {
                const size_t n = (size_t)T * E / 4 + T + E;
                const unsigned g = (unsigned)((n + 255) / 256 < 2048 ? (n + 255) / 256 : 2048);
                hipLaunchKernelGGL(k_router_bf3_sum, dim3(g), dim3(256), 0, st, bpart, S, T, E,
                                   xn2, wn2);
            }
            const double nround = rb_bound(d) / (1.01 * 0x1p-53);
            if (E <= 256)
                hipLaunchKernelGGL(k_router_pick<4>, dim3((T + 3) / 4), dim3(256), 0, st, bpart,
                                   xn2, wn2, bias, W, x, T, d, E, k, renorm, routed_scale, idx, wt,
                                   force, tstat, nround);
            else if (E <= 512)
                hipLaunchKernelGGL(k_router_pick<8>, dim3((T + 3) / 4), dim3(256), 0, st, bpart,
                                   xn2, wn2, bias, W, x, T, d, E, k, renorm, routed_scale, idx, wt,
                                   force, tstat, nround);
            else
                hipLaunchKernelGGL(k_router_pick<16>, dim3((T + 3) / 4), dim3(256), 0, st, bpart,
                                   xn2, wn2, bias, W, x, T, d, E, k, renorm, routed_scale, idx, wt,
                                   force, tstat, nround);
            if (stats)
                hipLaunchKernelGGL(k_router_stats, dim3(1), dim3(256), 0, st, (const int4 *)tstat,
                                   T, stats);
            return hipGetLastError() == hipSuccess ? 0 : -1;
        }
    }
    /* the score intervals of token t live at [t][E] */
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
