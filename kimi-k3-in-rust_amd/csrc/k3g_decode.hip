/* k3g_decode.hip - the whole decode-sized MoE layer (Kimi-K2 shape: no latent, MXFP4
 * routed experts, bf16 shared expert) as ONE persistent kernel.
 *
 * Why one kernel. At one token the layer streams ~286 MB and does almost no arithmetic,
 * so it is a pure HBM-streaming problem, and a chain of separate kernels loses the
 * machine at every boundary: each launch ramps up, drains, and waits for its slowest
 * wave. Here the work is cut into tickets, ordered so that whatever a ticket depends on
 * has a smaller ticket, and wave w of a co-resident persistent grid of W waves takes
 * tickets w, w + W, w + 2W, ... in order (a shared ticket counter costs one contended
 * device atomic per ticket, which at ~10^4 tickets per call is the bottleneck itself):
 *
 *   R   router logits: (expert, 1024-column chunk) per ticket, fp64 partial sums
 *   S   the certified top-k for every token (one ticket); waits for all R
 *   SG  shared-expert gate/up, 4 row pairs per ticket, SwiGLU/SiTU epilogue
 *   G   routed gate/up of one (token, slot) pair, 8 row pairs per ticket; waits for
 *       the routing
 *   SD  shared-expert down, 8 output rows per ticket; waits for all SG
 *   D   routed down of one pair, 16 output rows per ticket; waits for that pair's G
 *   C   combine, 256 output rows per ticket: slots in the engine's order (float
 *       multiply, then add), then + shared; waits for every D and SD
 *
 * The shared expert does not depend on the routing, so it streams while the top-k is
 * being chosen, and the G tickets of slot 0 finish first, so its D tickets start while
 * later slots still stream their gate/up rows.
 *
 * Cross-wave data (partial logits, the routing, h, per-slot outputs) is written and read
 * at device coherence (sc1 stores and loads), and a producer waits for its stores to
 * complete before it bumps a counter, so no device-wide cache writeback or invalidate is
 * ever issued and the L2s keep streaming.
 *
 * Completion counters are spread over separate cache lines (sub-counters per ticket
 * class, summed by the waiter) and never reset: launch n waits for n times the per-call
 * count (the host passes n as the epoch and clears the counters when it wraps or after
 * a device error).
 *
 * Deadlock freedom: a ticket only waits on smaller tickets; the owner of a smaller ticket
 * reaches it after its own even smaller tickets, all waves are resident at once (the grid
 * is sized by the occupancy calculator), and every wait is bounded (an exhausted wait
 * raises K3G_ERR_WAIT and the wave moves on, so every wave reaches the exit).
 */
#include "k3g_dev.h"
#include "k3g_kernels.h"
#include "k3g_select.h"

/* counter layout: every counter on its own 128-byte line (32 ints) */
#define SY_LINE 32
#define NSUB 16           /* sub-counters per ticket class */
enum { SY_R = 0, SY_SEL = SY_R + NSUB, SY_SG = SY_SEL + 1, SY_SD = SY_SG + NSUB,
       SY_G = SY_SD + NSUB, SY_D = SY_G + 256, SY_NLINES = SY_D + 256 };

#define R_CHUNK 1024      /* router columns per ticket: 64 lanes x 16 */
#define SG_PAIRS 4        /* shared gate/up row pairs per ticket */
#define G_PAIRS 8         /* routed gate/up row pairs per ticket */
#define SD_ROWS 8         /* shared down rows per ticket */
#define D_ROWS 16         /* routed down rows per ticket */
#define C_ROWS 256        /* combine rows per ticket: 64 lanes x 4 */

/* ------------------------------------------------------------ coherence ---- */
__device__ __forceinline__ int k3d_ld_relaxed(const int *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void k3d_st_dev(float *p, float v)
{
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ int *k3d_line(int *sync, int i) { return sync + (size_t)i * SY_LINE; }

/* All of this wave's memory operations complete, then the counter moves. */
__device__ __forceinline__ void k3d_signal(int *ctr, int lane)
{
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("" ::: "memory");
    if (lane == 0)
        __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Wait until the counters line(first) .. line(first + n - 1) sum to at least target.
 * Bounded: false (and an error raised) when the limit runs out. Wave-uniform. */
__device__ __forceinline__ bool k3d_wait_sum(int *sync, int first, int n, long long target,
                                             long long limit, int *err, int lane)
{
    long long spins = 0;
    for (;;) {
        long long v = lane < n ? k3d_ld_relaxed(k3d_line(sync, first + lane)) : 0;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, K3G_WAVE);
        if (__builtin_amdgcn_readfirstlane((int)(v >= target))) break;
        __builtin_amdgcn_s_sleep(2);
        if (++spins > limit) {
            k3d_raise(err, K3G_ERR_WAIT);
            return false;
        }
    }
    asm volatile("" ::: "memory");
    return true;
}

/* ----------------------------------------------------------- buffer loads ---- */
/* Every weight row is read through a raw buffer descriptor: the matrix base lives in
 * scalar registers, each row is a scalar offset, and only the lane's column offset is a
 * vector register, so a tile of 16 rows costs 16 scalar offsets instead of 16 vector
 * pointer pairs. Out-of-range offsets read zero (the descriptor's byte bound). */
typedef __amdgpu_buffer_rsrc_t K3Rsrc;

__device__ __forceinline__ K3Rsrc k3d_rsrc(const void *p, size_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(bytes < 0x7fffffffu ? bytes : 0x7fffffffu),
                                             0x00020000);
}

#define K3_SC1 16   /* cache policy: device-coherent load */

template <int AUX = 0>
__device__ __forceinline__ uint4 k3d_b128(K3Rsrc r, int voff, int soff)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX));
}

__device__ __forceinline__ uint32_t k3d_b8(K3Rsrc r, int voff, int soff)
{
    return __builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, 0);
}

/* n4 float4 (16-byte) loads at byte offset voff + soff */
template <int AUX = 0>
__device__ __forceinline__ void k3d_bx(K3Rsrc r, int voff, int soff, float *x, int n4)
{
    for (int i = 0; i < n4; ++i) {
        const uint4 v = k3d_b128<AUX>(r, voff + 16 * i, soff);
        x[4 * i] = __uint_as_float(v.x); x[4 * i + 1] = __uint_as_float(v.y);
        x[4 * i + 2] = __uint_as_float(v.z); x[4 * i + 3] = __uint_as_float(v.w);
    }
}

/* acc + the 32 products of one MXFP4 group (16 bytes, scale byte s), decoding one
 * 8-element word at a time */
__device__ __forceinline__ float k3d_dot32(uint4 q, uint32_t s, const float *x, float acc)
{
    const float sc = k3d_e8m0(s);
    const uint32_t wd[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        float w[8];
        k3d_fp4x8(wd[h], sc, w);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = fmaf(w[i], x[8 * h + i], acc);
    }
    return acc;
}

/* 16 bf16 weights (32 bytes) dotted with 16 x values */
__device__ __forceinline__ float k3d_dot16bf(const uint4 &a, const uint4 &b, const float *x,
                                             float s)
{
    const uint32_t wd[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        s = fmaf(k3d_bf16lo(wd[i]), x[2 * i], s);
        s = fmaf(k3d_bf16hi(wd[i]), x[2 * i + 1], s);
    }
    return s;
}

template <int V>
struct K3L2 { static constexpr int v = 1 + K3L2<V / 2>::v; };
template <>
struct K3L2<1> { static constexpr int v = 0; };

__device__ __forceinline__ int k3d_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

/* A pointer every lane holds the same value of, moved to scalar registers (a pointer
 * loaded from memory the kernel also writes comes back in vector registers). */
template <typename P>
__device__ __forceinline__ P *k3d_uniform_ptr(P *p)
{
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (P *)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ K3ExpertQ k3d_expert(const K3ExpertQ *eq, int e)
{
    const K3ExpertQ q = eq[e];
    K3ExpertQ u;
    u.p1 = k3d_uniform_ptr(q.p1); u.s1 = k3d_uniform_ptr(q.s1);
    u.p3 = k3d_uniform_ptr(q.p3); u.s3 = k3d_uniform_ptr(q.s3);
    u.p2 = k3d_uniform_ptr(q.p2); u.s2 = k3d_uniform_ptr(q.s2);
    return u;
}

template <int NT>
struct K3Dec {
    /* ----------------------------------------------------------------- R ---- */
    static __device__ void router(const K3kDecode &a, int tk, int lane)
    {
        const int nch = (a.d + R_CHUNK - 1) / R_CHUNK;
        const int e = tk / nch, c = tk - e * nch;
        const int col = c * R_CHUNK + lane * 16;
        const K3Rsrc rg = k3d_rsrc(a.gate, (size_t)a.E * a.d * 4);
        const K3Rsrc rx = k3d_rsrc(a.x, (size_t)a.T * a.d * 4);
        double acc[NT], ab[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) { acc[t] = 0.0; ab[t] = 0.0; }
        float w[16];
        k3d_bx(rg, col * 4, e * a.d * 4, w, 4);
        const bool on = col < a.d;     /* lanes past the row end read the next row */
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t < a.T && on) {
                float xv[16];
                k3d_bx(rx, col * 4, t * a.d * 4, xv, 4);
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    acc[t] = fma((double)w[i], (double)xv[i], acc[t]);
                    ab[t] = fma(fabs((double)w[i]), fabs((double)xv[i]), ab[t]);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const double s = k3d_wave_sumd(acc[t]);
            const double b = k3d_wave_sumd(ab[t]);
            if (lane == 0 && t < a.T) {
                k3d_st_dev64(&a.plogit[((size_t)c * a.T + t) * a.E + e], s);
                k3d_st_dev64(&a.pasum[((size_t)c * a.T + t) * a.E + e], b);
            }
        }
        k3d_signal(k3d_line(a.sync, SY_R + tk % NSUB), lane);
    }

    /* ----------------------------------------------------------------- S ---- */
    static __device__ void select(const K3kDecode &a, int lane, K3SelectLds *lds, int nR)
    {
        const int nch = (a.d + R_CHUNK - 1) / R_CHUNK;
        if (!k3d_wait_sum(a.sync, SY_R, NSUB, (long long)a.epoch * nR, a.spin_limit, a.err,
                          lane))
            return;
        for (int t = 0; t < a.T; ++t)
            k3d_select_token(lds, t, a.T, nch, a.plogit, a.pasum, a.bias, a.gate, a.x, a.d,
                             a.E, a.k, a.renorm, a.routed_scale, a.idx, a.wt, a.force,
                             a.stats, lane);
        __builtin_amdgcn_s_waitcnt(0);
        asm volatile("" ::: "memory");
        if (lane == 0)
            __hip_atomic_store(k3d_line(a.sync, SY_SEL), a.epoch, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }

    /* ---------------------------------------------------------------- SG ---- */
    static __device__ void shared_gateup(const K3kDecode &a, int tk, int lane)
    {
        const int r0 = tk * SG_PAIRS;
        constexpr int V = 2 * SG_PAIRS * NT;
        constexpr int SH = 6 - K3L2<V>::v;
        const K3Rsrc r1 = k3d_rsrc(a.sh1, (size_t)a.SI * a.d * 2);
        const K3Rsrc r3 = k3d_rsrc(a.sh3, (size_t)a.SI * a.d * 2);
        const K3Rsrc rx = k3d_rsrc(a.x, (size_t)a.T * a.d * 4);
        const int rowb = a.d * 2;
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = 0.0f;
        for (int cb = 0; cb < a.d; cb += 1024) {
            const int col = cb + lane * 16;
            uint4 q[2 * SG_PAIRS][2];
#pragma unroll
            for (int r = 0; r < SG_PAIRS; ++r) {
                q[r][0] = k3d_b128(r1, col * 2, (r0 + r) * rowb);
                q[r][1] = k3d_b128(r1, col * 2 + 16, (r0 + r) * rowb);
                q[SG_PAIRS + r][0] = k3d_b128(r3, col * 2, (r0 + r) * rowb);
                q[SG_PAIRS + r][1] = k3d_b128(r3, col * 2 + 16, (r0 + r) * rowb);
            }
            if (col >= a.d) continue;   /* lanes past the row end read the next row */
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float xv[16];
                k3d_bx(rx, col * 4, (t < a.T ? t : 0) * a.d * 4, xv, 4);
#pragma unroll
                for (int r = 0; r < 2 * SG_PAIRS; ++r)
                    acc[r * NT + t] = k3d_dot16bf(q[r][0], q[r][1], xv, acc[r * NT + t]);
            }
        }
        k3d_transpose_reduce<V>(acc, lane);
        const float upv = __shfl_xor(acc[0], 32, K3G_WAVE);
        const int v = lane >> SH;
        if ((lane & ((1 << SH) - 1)) == 0 && v < SG_PAIRS * NT) {
            const int r = v / NT, t = v % NT;
            if (r0 + r < a.SI && t < a.T)
                k3d_st_dev(&a.sh_h[(size_t)t * a.SI + r0 + r], k3d_act(acc[0], upv, a.b1, a.b2));
        }
        k3d_signal(k3d_line(a.sync, SY_SG + tk % NSUB), lane);
    }

    /* ----------------------------------------------------------------- G ---- */
    static __device__ void routed_gateup(const K3kDecode &a, int tk, int lane)
    {
        const int tiles = (a.I + G_PAIRS - 1) / G_PAIRS;
        const int p = tk / tiles, g = tk - p * tiles;
        const int r0 = g * G_PAIRS;
        if (!k3d_wait_sum(a.sync, SY_SEL, 1, a.epoch, a.spin_limit, a.err, lane)) return;
        const int e = k3d_uniform(__hip_atomic_load(&a.idx[p], __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT));
        if (e >= 0 && e < a.E) {
            const K3ExpertQ q = k3d_expert(a.eq, e);
            const int t = p / a.k;
            const int pc = a.d >> 1, sc = (a.d + 31) >> 5;
            const K3Rsrc rp1 = k3d_rsrc(q.p1, (size_t)a.I * pc), rs1 = k3d_rsrc(q.s1, (size_t)a.I * sc);
            const K3Rsrc rp3 = k3d_rsrc(q.p3, (size_t)a.I * pc), rs3 = k3d_rsrc(q.s3, (size_t)a.I * sc);
            const K3Rsrc rx = k3d_rsrc(a.x, (size_t)a.T * a.d * 4);
            float acc[2 * G_PAIRS];
#pragma unroll
            for (int i = 0; i < 2 * G_PAIRS; ++i) acc[i] = 0.0f;
            for (int cb = 0; cb < a.d; cb += 2048) {
                const int col = cb + lane * 32;
                const bool on = col < a.d;
                uint4 w[2 * G_PAIRS];
                uint32_t s[2 * G_PAIRS];
#pragma unroll
                for (int r = 0; r < G_PAIRS; ++r) {
                    w[r] = k3d_b128(rp1, col >> 1, (r0 + r) * pc);
                    s[r] = k3d_b8(rs1, col >> 5, (r0 + r) * sc);
                    w[G_PAIRS + r] = k3d_b128(rp3, col >> 1, (r0 + r) * pc);
                    s[G_PAIRS + r] = k3d_b8(rs3, col >> 5, (r0 + r) * sc);
                }
                float xv[32];
                k3d_bx(rx, col * 4, t * a.d * 4, xv, 8);
                if (on) {
#pragma unroll
                    for (int r = 0; r < 2 * G_PAIRS; ++r) acc[r] = k3d_dot32(w[r], s[r], xv, acc[r]);
                }
            }
            k3d_transpose_reduce<2 * G_PAIRS>(acc, lane);
            const float upv = __shfl_xor(acc[0], 32, K3G_WAVE);
            const int v = lane >> 2;     /* V = 16: lane l holds row l >> 2 */
            if ((lane & 3) == 0 && v < G_PAIRS && r0 + v < a.I)
                k3d_st_dev(&a.h[(size_t)p * a.I + r0 + v], k3d_act(acc[0], upv, a.b1, a.b2));
        } else if (e >= a.E) {
            k3d_raise(a.err, K3G_ERR_EXPERT_RANGE);
        }
        k3d_signal(k3d_line(a.sync, SY_G + p), lane);
    }

    /* ---------------------------------------------------------------- SD ---- */
    static __device__ void shared_down(const K3kDecode &a, int tk, int lane, int nSG)
    {
        const int r0 = tk * SD_ROWS;
        if (!k3d_wait_sum(a.sync, SY_SG, NSUB, (long long)a.epoch * nSG, a.spin_limit, a.err,
                          lane))
            return;
        constexpr int V = SD_ROWS * NT;
        constexpr int SH = 6 - K3L2<V>::v;
        const K3Rsrc r2 = k3d_rsrc(a.sh2, (size_t)a.d * a.SI * 2);
        const K3Rsrc rh = k3d_rsrc(a.sh_h, (size_t)a.T * a.SI * 4);
        const int rowb = a.SI * 2;
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = 0.0f;
        for (int cb = 0; cb < a.SI; cb += 1024) {
            const int col = cb + lane * 16;
            uint4 qv[SD_ROWS][2];
#pragma unroll
            for (int r = 0; r < SD_ROWS; ++r) {
                qv[r][0] = k3d_b128(r2, col * 2, (r0 + r) * rowb);
                qv[r][1] = k3d_b128(r2, col * 2 + 16, (r0 + r) * rowb);
            }
            if (col >= a.SI) continue;  /* lanes past the row end read the next row */
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float xv[16];
                k3d_bx<K3_SC1>(rh, col * 4, (t < a.T ? t : 0) * a.SI * 4, xv, 4);
#pragma unroll
                for (int r = 0; r < SD_ROWS; ++r)
                    acc[r * NT + t] = k3d_dot16bf(qv[r][0], qv[r][1], xv, acc[r * NT + t]);
            }
        }
        k3d_transpose_reduce<V>(acc, lane);
        const int v = lane >> SH;
        if ((lane & ((1 << SH) - 1)) == 0 && v < V) {
            const int r = v / NT, t = v % NT;
            if (r0 + r < a.d && t < a.T) k3d_st_dev(&a.sh_out[(size_t)t * a.d + r0 + r], acc[0]);
        }
        k3d_signal(k3d_line(a.sync, SY_SD + tk % NSUB), lane);
    }

    /* ----------------------------------------------------------------- D ---- */
    static __device__ void routed_down(const K3kDecode &a, int tk, int lane, int tilesG)
    {
        const int tiles = (a.d + D_ROWS - 1) / D_ROWS;
        const int p = tk / tiles, g = tk - p * tiles;
        const int r0 = g * D_ROWS;
        if (!k3d_wait_sum(a.sync, SY_G + p, 1, (long long)a.epoch * tilesG, a.spin_limit,
                          a.err, lane))
            return;
        const int e = k3d_uniform(__hip_atomic_load(&a.idx[p], __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT));
        if (e >= 0 && e < a.E) {
            const K3ExpertQ q = k3d_expert(a.eq, e);
            const int ipc = a.I >> 1, isc = (a.I + 31) >> 5;
            const K3Rsrc rp = k3d_rsrc(q.p2, (size_t)a.d * ipc), rs = k3d_rsrc(q.s2, (size_t)a.d * isc);
            const K3Rsrc rh = k3d_rsrc(a.h + (size_t)p * a.I, (size_t)a.I * 4);
            float acc[D_ROWS];
#pragma unroll
            for (int i = 0; i < D_ROWS; ++i) acc[i] = 0.0f;
            for (int cb = 0; cb < a.I; cb += 2048) {
                const int col = cb + lane * 32;
                const bool on = col < a.I;
                uint4 w[D_ROWS];
                uint32_t s[D_ROWS];
#pragma unroll
                for (int r = 0; r < D_ROWS; ++r) {
                    w[r] = k3d_b128(rp, col >> 1, (r0 + r) * ipc);
                    s[r] = k3d_b8(rs, col >> 5, (r0 + r) * isc);
                }
                float xv[32];
                k3d_bx<K3_SC1>(rh, col * 4, 0, xv, 8);
                if (on) {
#pragma unroll
                    for (int r = 0; r < D_ROWS; ++r) acc[r] = k3d_dot32(w[r], s[r], xv, acc[r]);
                }
            }
            k3d_transpose_reduce<D_ROWS>(acc, lane);
            const int v = lane >> 2;     /* V = 16: lane l holds row l >> 2 */
            if ((lane & 3) == 0 && r0 + v < a.d)
                k3d_st_dev(&a.contrib[(size_t)p * a.d + r0 + v], acc[0]);
        }
        k3d_signal(k3d_line(a.sync, SY_D + p), lane);
    }

    /* ----------------------------------------------------------------- C ---- */
    static __device__ void combine(const K3kDecode &a, int tk, int lane, int nSD)
    {
        const int P = a.T * a.k, tilesD = (a.d + D_ROWS - 1) / D_ROWS;
        for (int p0 = 0; p0 < P; p0 += 64)
            if (!k3d_wait_sum(a.sync, SY_D + p0, min(64, P - p0),
                              (long long)a.epoch * tilesD * min(64, P - p0), a.spin_limit,
                              a.err, lane))
                return;
        if (a.SI > 0 && !k3d_wait_sum(a.sync, SY_SD, NSUB, (long long)a.epoch * nSD,
                                      a.spin_limit, a.err, lane))
            return;
        const int row = tk * C_ROWS + lane * 4;
        const K3Rsrc rc = k3d_rsrc(a.contrib, (size_t)a.T * a.k * a.d * 4);
        const K3Rsrc rs = k3d_rsrc(a.sh_out, (size_t)a.T * a.d * 4);
        for (int t = 0; t < a.T; ++t) {
            float c0 = 0.0f, c1 = 0.0f, c2 = 0.0f, c3 = 0.0f;
            for (int j = 0; j < a.k; ++j) {
                const int p = t * a.k + j;
                const int e = k3d_uniform(__hip_atomic_load(&a.idx[p], __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT));
                if (e < 0 || e >= a.E) continue;
                const float w = __hip_atomic_load(&a.wt[p], __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
                const uint4 y = k3d_b128<K3_SC1>(rc, row * 4, p * a.d * 4);
                c0 = __fadd_rn(c0, __fmul_rn(w, __uint_as_float(y.x)));
                c1 = __fadd_rn(c1, __fmul_rn(w, __uint_as_float(y.y)));
                c2 = __fadd_rn(c2, __fmul_rn(w, __uint_as_float(y.z)));
                c3 = __fadd_rn(c3, __fmul_rn(w, __uint_as_float(y.w)));
            }
            if (a.SI > 0) {
                const uint4 sv = k3d_b128<K3_SC1>(rs, row * 4, t * a.d * 4);
                c0 = __fadd_rn(c0, __uint_as_float(sv.x)); c1 = __fadd_rn(c1, __uint_as_float(sv.y));
                c2 = __fadd_rn(c2, __uint_as_float(sv.z)); c3 = __fadd_rn(c3, __uint_as_float(sv.w));
            }
            if (row < a.d)
                *(float4 *)(a.out + (size_t)t * a.d + row) = make_float4(c0, c1, c2, c3);
        }
    }
};

template <int NT>
__global__ void __launch_bounds__(256)
k_decode_fused(K3kDecode a)
{
    __shared__ K3SelectLds lds;
    const int lane = threadIdx.x & 63;
    const int P = a.T * a.k;
    const int nch = (a.d + R_CHUNK - 1) / R_CHUNK;
    const int nR = a.E * nch;
    const int nSG = a.SI > 0 ? (a.SI + SG_PAIRS - 1) / SG_PAIRS : 0;
    const int tilesG = (a.I + G_PAIRS - 1) / G_PAIRS;
    const int nG = P * tilesG;
    const int nSD = a.SI > 0 ? (a.d + SD_ROWS - 1) / SD_ROWS : 0;
    const int nD = P * ((a.d + D_ROWS - 1) / D_ROWS);
    const int nC = (a.d + C_ROWS - 1) / C_ROWS;
    const int total = nR + 1 + nSG + nG + nSD + nD + nC;
    const int W = gridDim.x * (blockDim.x >> 6);
    const int w = k3d_uniform(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
    for (int tk = w; tk < total; tk += W) {
        if (a.trace && lane == 0) a.trace[2 * tk] = wall_clock64();
        int t = tk;
        if (t < nR) K3Dec<NT>::router(a, t, lane);
        else if ((t -= nR) < 1) K3Dec<NT>::select(a, lane, &lds, nR);
        else if ((t -= 1) < nSG) K3Dec<NT>::shared_gateup(a, t, lane);
        else if ((t -= nSG) < nG) K3Dec<NT>::routed_gateup(a, t, lane);
        else if ((t -= nG) < nSD) K3Dec<NT>::shared_down(a, t, lane, nSG);
        else if ((t -= nSD) < nD) K3Dec<NT>::routed_down(a, t, lane, tilesG);
        else K3Dec<NT>::combine(a, t - nD, lane, nSD);
        if (a.trace && lane == 0) a.trace[2 * tk + 1] = wall_clock64();
    }
}

extern "C" int k3k_decode_fused(const K3kDecode *a, hipStream_t st)
{
    if (a->T < 1 || a->T > 4 || a->d % 256 || a->I % 32 || (a->SI % 16) || a->k < 1 ||
        a->k > K3G_MAX_TOPK || a->E < 1 || a->E > K3G_MAX_E ||
        a->T * a->k > 256 || SY_NLINES * SY_LINE > K3G_SYNC_WORDS || a->epoch < 1)
        return -1;
    static int grid[5] = {0, 0, 0, 0, 0};
    const int NT = a->T <= 1 ? 1 : a->T <= 2 ? 2 : 4;
    const void *fn = NT == 1 ? (const void *)k_decode_fused<1>
                   : NT == 2 ? (const void *)k_decode_fused<2> : (const void *)k_decode_fused<4>;
    if (!grid[NT]) {
        int dev = 0, cus = 0, per = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, fn, 256, 0) != hipSuccess)
            return -1;
        grid[NT] = cus * (per > 0 ? per : 1);
    }
    if (NT == 1) hipLaunchKernelGGL(k_decode_fused<1>, dim3(grid[1]), dim3(256), 0, st, *a);
    else if (NT == 2) hipLaunchKernelGGL(k_decode_fused<2>, dim3(grid[2]), dim3(256), 0, st, *a);
    else hipLaunchKernelGGL(k_decode_fused<4>, dim3(grid[4]), dim3(256), 0, st, *a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
