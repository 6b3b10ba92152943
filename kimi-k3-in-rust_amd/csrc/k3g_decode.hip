/* k3g_decode.hip - the whole decode-sized MoE layer (Kimi-K2 shape: no latent, MXFP4
 * routed experts, bf16 shared expert) as ONE persistent kernel on the matrix cores.
 *
 * At one token the layer streams ~286 MB and does almost no arithmetic, so it is an
 * HBM-streaming problem. Two things decide the speed: every wave must keep bytes in
 * flight all the time, and no phase boundary may drain the machine. So:
 *
 * 1. The weights are consumed by MFMAs straight from the load registers. Routed experts
 *    are in the tiled MXFP4 layout (k3g_tile.hip) and go to
 *    v_mfma_scale_f32_16x16x128_f8f6f4 as FP4 A operands with their own E8M0 scales;
 *    the shared expert is in the tiled bf16 layout and goes to v_mfma_f32_16x16x32_bf16.
 *    The activations are the B operand, split into pieces so the products keep fp32
 *    accuracy: for FP4 x FP8, v = sum of 6 E4M3 pieces, each with its own per-32-block
 *    E8M0 scale (B columns 0..5); for bf16, v = sum of 3 bf16 pieces (columns 3t..3t+2 of
 *    token t). A GEMV row is the sum of its piece columns. Products of an E2M1 and an
 *    E4M3 (or two bf16) are exact in fp32, so the only error left is the pieces' residual
 *    (below 2^-24 of the block maximum) and fp32 accumulation.
 *    No weight is ever decoded by the vector ALUs.
 *
 * 2. The work is cut into tickets, ordered so that whatever a ticket depends on has a
 *    smaller ticket, and wave w of a co-resident persistent grid of W waves takes
 *    tickets w, w + W, w + 2W, ... (a shared ticket counter would cost one contended
 *    device atomic per ticket):
 *
 *      X   x -> FP8 pieces (per token, per 512 columns) and bf16 pieces
 *      R   router logits of one expert row (all tokens), fp64 with an error bound
 *      S   the certified top-k for every token (one ticket); waits for all R
 *      SG  shared gate/up: 16 SG_TILES rows x a K slice; the last slice of a row group
 *          (found with a returning atomic) sums the slices in slice order, applies the
 *          activation and writes the shared h as bf16 pieces
 *      SD  shared down: 32 rows x a K slice, partial sums per slice
 *      G   routed gate/up of one (token, slot) pair: 32 rows x a K slice of 512-column
 *          quads; the last slice of a tile sums, activates and writes h's FP8 pieces
 *      D   routed down of one pair: 32 output rows x a K slice of 512-column quads;
 *          waits for that pair's h. The last arrival of an output tile (over every
 *          pair's slices and the shared expert's) combines it: slots in the engine's
 *          order (float multiply, then add), then + the shared output (its slices
 *          summed in slice order)
 *
 *    The shared expert needs no routing, so SG and then SD stream while the router and
 *    top-k run.
 *
 * Cross-wave data (logits, routing, partial sums, pieces, per-slot outputs) is written
 * and read at device coherence (sc1 stores and loads) and a producer waits for its stores
 * to complete before it bumps a counter, so no device-wide cache writeback or invalidate
 * is ever issued. Completion counters sit on separate 128-byte lines. They come in two
 * banks that calls alternate between: a call counts from zero in its bank and, at its
 * start, zeroes the other bank (which the previous call used and, the launches being
 * ordered on the stream, has finished with) for the next call. So the per-call counts
 * may change from call to call (a different token count or layer).
 *
 * Deadlock freedom: a ticket only waits on smaller tickets, all waves are resident at
 * once (the grid is sized by the occupancy calculator), and every wait is bounded (an
 * exhausted wait raises K3G_ERR_WAIT and the wave moves on, so every wave reaches the
 * exit).
 */
#include "k3g_dev.h"
#include "k3g_kernels.h"
#include "k3g_select.h"

#include <stdlib.h>

typedef int k3v8i __attribute__((ext_vector_type(8)));
typedef float k3v4f __attribute__((ext_vector_type(4)));
typedef __bf16 k3v8bf __attribute__((ext_vector_type(8)));
typedef unsigned int k3v4u __attribute__((ext_vector_type(4)));

#define K3G_QT 4352       /* MXFP4 quad tile: 4 x 1 KB chunks + 256 B of scales */
#define K3G_BQ 8448       /* FP8 B quad: 4 x 2 KB chunks + 256 B of scales */
#define NPC8 6            /* FP8 pieces per value */
#define NPC16 3           /* bf16 pieces per value */
/* up to this many tokens the shared gate/up and latent down tickets make x's bf16 pieces
 * in registers from fp32 x; above it they read the prep tickets' pieces */
#ifndef K3G_XREG
#define K3G_XREG 2
#endif
#define SG_TILES 1        /* shared gate/up: 16-row tiles per ticket */
#define SG_BATCH 8        /* shared gate/up: 32-column chunks per load batch */

#define SY_LINE 32        /* ints per counter line (128 bytes) */
#define NSUB 16           /* sub-counters per ticket class with many signalers */
/* An event that thousands of waves wait for is published as NREP flag copies, 512 bytes
 * apart, and each waiter polls the copy its ticket number picks: one hot line polled by
 * every waiting wave would serialise at one memory channel and slow every other access
 * to it. */
#define NREP 16
#define REP_STRIDE 4      /* lines between copies */
#define K3_EVLINES (NREP * REP_STRIDE)

/* ------------------------------------------------------------ geometry ---- */
/* Ticket classes in order: X R S [LD] SG SD G D [NR LU]. The bracketed ones exist only for
 * the LatentMoE layer (L != d): LD the latent down projection z = down x (32 rows x a K
 * slice; the last slice of a row tile writes z's FP8 pieces for the routed gate/up), NR
 * the aggregate's RMSNorm into bf16 pieces (64 columns each), LU the latent up projection
 * (32 output rows x a K slice; the last arrival of an output tile, over LU's and the shared
 * down's slices, writes out). There the routed gate/up reads z (K = L), the routed down
 * produces L rows, and its last arrival per 32 rows writes the slot-order aggregate. */
struct K3Geo {
    int T, P, nQd, nCd, nQi, nCsi;
    int KSS, KSG, KSD, KSR, KSDN; /* K slices of SG, G, SD, R, D tickets */
    int nRc;                     /* router 1024-column chunks */
    int nSGt, nGt, nSDt, nDt;    /* row tiles (SG: row groups of SG_TILES tiles) */
    int nX, nR, nSG, nG, nSD, nD, total;
    int oSG, oG, oSD, oD;        /* first ticket of each class after S */
    /* the latent layer */
    int lat, L, Dout, nQk;       /* L; D's output rows (L or d); G's K in 512-column quads */
    int nCL, KSLD, KSLU, nLDt, nLUt, nNR, nLD, nLU, oLD, oNR, oLU;
    /* counter lines */
    int lR, lSD, lD, lTSG, lTG, lRE, lDT, lLD, lLU, cX, cX16, cR, cSGF, cGF, cZ, cA, cN, eX,
        eX16, eR, eSEL, eSGF, eGF, eZ, eA, eN, cOD, nlines;
};

__host__ __device__ inline K3Geo k3_geo(int T, int d, int E, int k, int I, int SI, int L)
{
    K3Geo g;
    g.T = T;
    g.P = T * k;
    if (L <= 0) L = d;           /* 0: no latent layer */
    g.lat = L != d;
    g.L = L;
    g.Dout = g.lat ? L : d;
    g.nQd = (d + 511) / 512;
    g.nQk = g.lat ? (L + 511) / 512 : g.nQd;
    g.nCd = d / 32;
    g.nCL = L / 32;
    g.nQi = (I + 511) / 512;
    g.nCsi = SI / 32;
    const int kss = g.lat ? K3G_KS_SG_LAT : K3G_KS_SG, ksd = g.lat ? K3G_KS_SD_LAT : K3G_KS_SD;
    const int ksr = g.lat ? K3G_KS_R_LAT : K3G_KS_R, ksdn = g.lat ? K3G_KS_D_LAT : K3G_KS_D;
    g.KSS = SI > 0 ? (kss < g.nCd ? kss : g.nCd) : 0;
    {
        const int ks = g.lat ? K3G_KS_G_LAT : K3G_KS_G;
        g.KSG = ks < g.nQk ? ks : g.nQk;
    }
    g.KSD = SI > 0 ? (ksd < g.nCsi ? ksd : g.nCsi) : 0;
    g.nRc = (d + 1023) / 1024;
    g.KSR = ksr < g.nRc ? ksr : g.nRc;
    g.KSDN = ksdn < g.nQi ? ksdn : g.nQi;
    g.KSLD = g.lat ? (K3G_KS_LD < g.nCd ? K3G_KS_LD : g.nCd) : 0;
    g.KSLU = g.lat ? (K3G_KS_LU < g.nCL ? K3G_KS_LU : g.nCL) : 0;
    g.nSGt = (SI + 16 * SG_TILES - 1) / (16 * SG_TILES);
    g.nGt = I / 32;
    g.nSDt = SI > 0 ? d / 32 : 0;
    g.nDt = g.Dout / 32;
    g.nLDt = g.lat ? L / 32 : 0;
    g.nLUt = g.lat ? d / 32 : 0;
    g.nNR = g.lat ? (L + 63) / 64 : 0;
    g.nX = T * ((g.nCd + 1) / 2);
    g.nR = E * g.KSR;
    g.nLD = g.nLDt * g.KSLD;
    g.nSG = g.nSGt * g.KSS;
    g.nG = g.P * g.nGt * g.KSG;
    g.nSD = g.nSDt * g.KSD;
    g.nD = g.P * g.nDt * g.KSDN;
    g.nLU = g.nLUt * g.KSLU;
    g.oLD = g.nX + g.nR + 1;
    g.oSG = g.oLD + g.nLD;
    g.oSD = g.oSG + g.nSG;
    g.oG = g.oSD + g.nSD;
    g.oD = g.oG + g.nG;
    g.oNR = g.oD + g.nD;
    g.oLU = g.oNR + g.nNR;
    g.total = g.oLU + g.nLU;
    /* counters: one 128-byte line each; events: a counter plus NREP replicated flags */
    g.lR = 0;
    g.lSD = g.lR + NSUB;
    g.lD = g.lSD + NSUB;
    g.lTSG = g.lD + g.P;
    g.lTG = g.lTSG + g.nSGt;
    g.lRE = g.lTG + g.P * g.nGt;
    g.lDT = g.lRE + E;
    g.lLD = g.lDT + g.nDt;
    g.lLU = g.lLD + g.nLDt;
    /* event counters: a top line and NSUB sub-counter lines each (k3d_arrive_event2) */
    g.cX = g.lLU + g.nLUt;
    g.cX16 = g.cX + 1 + NSUB;
    g.cR = g.cX16 + 1 + NSUB;
    g.cSGF = g.cR + 1 + NSUB;
    g.cZ = g.cSGF + 1 + NSUB;
    g.cA = g.cZ + 1 + NSUB;
    g.cN = g.cA + 1 + NSUB;
    g.cGF = g.cN + 1 + NSUB;
    g.eX = g.cGF + g.P * (1 + NSUB);
    g.eX16 = g.eX + K3_EVLINES;
    g.eR = g.eX16 + K3_EVLINES;
    g.eSEL = g.eR + K3_EVLINES;
    g.eSGF = g.eSEL + K3_EVLINES;
    g.eZ = g.eSGF + K3_EVLINES;
    g.eA = g.eZ + K3_EVLINES;
    g.eN = g.eA + K3_EVLINES;
    g.eGF = g.eN + K3_EVLINES;
    g.cOD = g.eGF + g.P * K3_EVLINES;   /* output tiles written (host copies only) */
    g.nlines = g.cOD + 1 + NSUB;
    return g;
}

/* ------------------------------------------------------------ coherence ---- */
__device__ __forceinline__ int k3d_ld_relaxed(const int *p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

/* All of this wave's memory operations complete, then it arrives at a tile counter;
 * true (in every lane) for the arrival that completes the tile in this call. */
__device__ __forceinline__ bool k3d_arrive(int *ctr, int last_old, int lane)
{
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("" ::: "memory");
    int old = 0;
    if (lane == 0)
        old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    asm volatile("" ::: "memory");
    return old == last_old;
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

/* Wait until the event's flag copy picked by `who` is set. Bounded like k3d_wait_sum. */
__device__ __forceinline__ bool k3d_wait_event(int *sync, int ev, int who, long long limit,
                                               int *err, int lane)
{
    const int *f = k3d_line(sync, ev + (who % NREP) * REP_STRIDE);
    long long spins = 0;
    for (;;) {
        int v = lane == 0 ? k3d_ld_relaxed(f) : 0;
        if (__builtin_amdgcn_readfirstlane(v)) break;
        __builtin_amdgcn_s_sleep(8);
        if (++spins > limit) {
            k3d_raise(err, K3G_ERR_WAIT);
            return false;
        }
    }
    asm volatile("" ::: "memory");
    return true;
}

/* Set every flag copy of an event (after this wave's stores completed). */
__device__ __forceinline__ void k3d_set_event(int *sync, int ev, int lane)
{
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("" ::: "memory");
    if (lane < NREP)
        __hip_atomic_store(k3d_line(sync, ev + lane * REP_STRIDE), 1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

/* Arrive at an event that `count` arrivals complete, arrival `who` (0 .. count - 1) at
 * sub-counter line ctr + 1 + who % NSUB; the arrival that completes a sub-counter arrives
 * at the top line ctr, and the one that completes the top count (one per non-empty
 * sub-counter) sets the event. Same-address atomics serialise at the memory side, so a
 * few hundred arrivals on one line would take microseconds; here at most
 * ceil(count / NSUB) + NSUB meet on one line. */
__device__ __forceinline__ bool k3d_arrive2(int *sync, int ctr, int count, int who, int lane)
{
    const int sub = who % NSUB;
    const int members = count / NSUB + (sub < count % NSUB ? 1 : 0);
    if (!k3d_arrive(k3d_line(sync, ctr + 1 + sub), members - 1, lane)) return false;
    const int tops = count < NSUB ? count : NSUB;
    return k3d_arrive(k3d_line(sync, ctr), tops - 1, lane);
}

__device__ __forceinline__ void k3d_arrive_event2(int *sync, int ctr, int count, int who,
                                                  int ev, int lane)
{
    if (k3d_arrive2(sync, ctr, count, who, lane)) k3d_set_event(sync, ev, lane);
}

/* Instrumentation: the moment a ticket's waits are over (its second trace stamp). */
__device__ __forceinline__ void k3d_trace_go(unsigned long long *trace, int tkg, int lane)
{
    if (trace && lane == 0) trace[3 * tkg + 1] = wall_clock64();
}

/* A workgroup's reduction of one router row's slices (4 waves = 4 slices, up to 4 tokens):
 * {sum, sum|w x|} per slice and token, and the arrival count. */
struct K3RouterLds {
    double part[4][4][2];
    int count;
};

/* ----------------------------------------------------------- buffer access ---- */
/* Weights and pieces are read through raw buffer descriptors: the base lives in scalar
 * registers and each lane adds its own byte offset. An offset at or past the
 * descriptor's size reads zero without touching memory, which is how unused B columns
 * are skipped. */
typedef __amdgpu_buffer_rsrc_t K3Rsrc;

__device__ __forceinline__ K3Rsrc k3d_rsrc(const void *p, size_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(bytes < 0x7fffffffu ? bytes : 0x7fffffffu),
                                             0x00020000);
}

#define K3_SC1 16   /* cache policy: device-coherent access */
/* Cache policy of the loads of activation pieces and per-slot outputs (xq8, xq16, hq8,
 * hq16, contrib, shpart): ordinary cached loads. Each of those lines is written once per
 * launch and read only after the counter that covers all of its writers has moved, and
 * every launch starts with the L2s invalidated, so no XCD can hold a stale copy; cached
 * loads keep these small, hot arrays in each XCD's L2 instead of going to memory for
 * every read. (sgpart lines span two row tiles that finish at different times, and the
 * router scores are read once; those stay device-coherent.) */
#define K3_BPOL 0
#define K3_OOB 0x7ffffff0

template <int AUX = 0>
__device__ __forceinline__ uint4 k3d_b128(K3Rsrc r, int voff)
{
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, AUX));
}

template <int AUX = 0>
__device__ __forceinline__ uint32_t k3d_b32(K3Rsrc r, int voff)
{
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, AUX);
}

__device__ __forceinline__ float k3d_f32_sc1(K3Rsrc r, int voff)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, K3_SC1));
}

/* sum over q < n (n <= N) of the fp32 at byte offset off + q * stride, device-coherent,
 * in q order from 0.0f; every load is issued before the first add (a loop of dependent
 * loads would cost one memory round trip per term) */
template <int N>
__device__ __forceinline__ float k3d_sum_sc1(K3Rsrc r, int off, int stride, int n)
{
    float v[N];
#pragma unroll
    for (int q = 0; q < N; ++q)
        v[q] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(r, q < n ? off + q * stride : K3_OOB, 0, K3_SC1));
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < N; ++q)
        if (q < n) s += v[q];
    return s;
}

__device__ __forceinline__ void k3d_st4_sc1(K3Rsrc r, int voff, k3v4f v)
{
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(k3v4u, v), r, voff, 0, K3_SC1);
}

__device__ __forceinline__ void k3d_st8_sc1(K3Rsrc r, int voff, uint32_t v)
{
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)v, r, voff, 0, K3_SC1);
}

__device__ __forceinline__ void k3d_st16_sc1(K3Rsrc r, int voff, uint32_t v)
{
    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)v, r, voff, 0, K3_SC1);
}

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

/* ----------------------------------------------------------- MFMA helpers ---- */
__device__ __forceinline__ k3v8i k3d_a4(uint4 a) { return k3v8i{(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0}; }

__device__ __forceinline__ k3v8i k3d_b8(uint4 lo, uint4 hi)
{
    return k3v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
}

/* acc += A(FP4, scale byte J of sa) x B(FP8, scale byte J of sb) */
template <int J>
__device__ __forceinline__ k3v4f k3d_mma4(uint4 a, k3v8i b, k3v4f acc, uint32_t sa, uint32_t sb)
{
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(k3d_a4(a), b, acc, 4, 0, J, (int)sa,
                                                            J, (int)sb);
}

__device__ __forceinline__ k3v4f k3d_mma16(uint4 a, uint4 b, k3v4f acc)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(k3v8bf, a),
                                                   __builtin_bit_cast(k3v8bf, b), acc, 0, 0, 0);
}

/* Sum of the 16 columns of a 16x16 accumulator: afterwards the lanes of column 0
 * (lane & 15 == 0) hold, in register i, row 4 (lane >> 4) + i. */
__device__ __forceinline__ k3v4f k3d_colsum(k3v4f v)
{
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
        v[0] += __shfl_xor(v[0], m, K3G_WAVE);
        v[1] += __shfl_xor(v[1], m, K3G_WAVE);
        v[2] += __shfl_xor(v[2], m, K3G_WAVE);
        v[3] += __shfl_xor(v[3], m, K3G_WAVE);
    }
    return v;
}

/* Token t = lane & 15's sum of columns 3t, 3t+1, 3t+2 (lanes with t >= T get junk). */
__device__ __forceinline__ k3v4f k3d_colsum3(k3v4f v, int lane)
{
    const int base = (lane & 48) + 3 * (lane & 15);
    k3v4f r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = __shfl(v[i], base & 63, K3G_WAVE);
        const float b = __shfl(v[i], (base + 1) & 63, K3G_WAVE);
        const float c = __shfl(v[i], (base + 2) & 63, K3G_WAVE);
        r[i] = (a + b) + c;
    }
    return r;
}

/* E8M0 exponent s such that max / 2^s <= 448 (the largest E4M3 value), for max > 0. */
__device__ __forceinline__ int k3d_fp8_scale(float m)
{
    if (!(m > 0.0f)) return -127;
    int e;
    const float f = frexpf(m, &e);        /* m = f 2^e, f in [0.5, 1) */
    int s = f <= 0.875f ? e - 9 : e - 8;  /* 448 = 0.875 * 2^9 */
    return s < -127 ? -127 : (s > 127 ? 127 : s);
}

/* One FP8 piece of r (a block of 32 lanes shares the scale): returns the E4M3 byte,
 * sets *sx to the block's scale exponent and removes the piece from r (exactly). */
__device__ __forceinline__ uint32_t k3d_fp8_piece(float &r, int &sx)
{
    float m = fabsf(r);
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, K3G_WAVE));
    sx = k3d_fp8_scale(m);
    const int pk = __builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(r, -sx), 0.0f, 0, false);
    r = r - ldexpf(__builtin_amdgcn_cvt_f32_fp8(pk, 0), sx);
    return (uint32_t)pk & 0xffu;
}

/* bf16 nearest-even of v (finite v) as bits, and its value */
__device__ __forceinline__ uint32_t k3d_bf16_rn(float v, float &back)
{
    uint32_t u = __float_as_uint(v);
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    back = __uint_as_float(u);
    return u >> 16;
}

/* Byte offset inside an FP8 B quad of element e (0..31) of MX block b (of the whole
 * vector) for piece column pc, and of that block's scale byte. The B operand pairs with
 * the tiled A layout: chunk j = (b % 16) / 4 holds blocks 16Q + 4j + g in lane group g,
 * and the MFMA pairs A group g's nibbles 0-15 / 16-31 with B lanes 16 (2 (g & 1)) + c /
 * 16 (2 (g & 1) + 1) + c, bytes 16 (g >> 1) .. + 16 of column c. */
__device__ __forceinline__ int k3d_bq_data(int b, int e, int pc)
{
    const int j = (b & 15) >> 2, g = b & 3;
    const int M = 16 * (2 * (g & 1) + (e >> 4)) + pc;
    return j * 2048 + M * 32 + 16 * (g >> 1) + (e & 15);
}

__device__ __forceinline__ int k3d_bq_scale(int b, int pc)
{
    const int j = (b & 15) >> 2, g = b & 3;
    return 8192 + (16 * g + pc) * 4 + j;
}

/* Byte offset in a bf16 B array (chunks of 32 values, 1 KB each) of value k, column col */
__device__ __forceinline__ int k3d_b16_off(int k, int col)
{
    return (k >> 5) * 1024 + (16 * ((k & 31) >> 3) + col) * 16 + 2 * (k & 7);
}

/* x's bf16 pieces as the B operand of one 32-column chunk, made in registers from fp32 x
 * (T <= 2, when 3T columns and their 3T neighbours 8 lanes on fit in a 16-lane row).
 * Lane (kg, col) with col < 3T needs piece col % 3 of token col / 3's values
 * 32 c + 8 kg .. + 7: lane col loads the first four, lane col + 8 the last four, and a
 * DPP rotation by 8 inside the row brings the second half over. The pieces are the prep
 * tickets' (bf16 nearest-even of the value, then of each remainder), so the products are
 * the same bits. k3d_xb16_off: this lane's load offset (past the end when it loads
 * nothing); k3d_xb16_make: the operand from the loaded half. */
__device__ __forceinline__ int k3d_xb16_off(int T, int d, int c, int lane)
{
    const int col = lane & 15, half = col >> 3, cl = col & 7;
    if (cl >= 3 * T) return K3_OOB;
    return ((cl / 3) * d + 32 * c + 8 * (lane >> 4) + 4 * half) * 4;
}

__device__ __forceinline__ uint4 k3d_xb16_make(uint4 raw, int T, int lane)
{
    typedef __bf16 k3v2bf __attribute__((ext_vector_type(2)));
    const uint4 up = make_uint4(__builtin_amdgcn_mov_dpp(raw.x, 0x128, 0xf, 0xf, false),
                                __builtin_amdgcn_mov_dpp(raw.y, 0x128, 0xf, 0xf, false),
                                __builtin_amdgcn_mov_dpp(raw.z, 0x128, 0xf, 0xf, false),
                                __builtin_amdgcn_mov_dpp(raw.w, 0x128, 0xf, 0xf, false));
    float v[8] = {__uint_as_float(raw.x), __uint_as_float(raw.y), __uint_as_float(raw.z),
                  __uint_as_float(raw.w), __uint_as_float(up.x),  __uint_as_float(up.y),
                  __uint_as_float(up.z),  __uint_as_float(up.w)};
    const int col = lane & 15, pc = col % 3;
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int lv = 0; lv < NPC16; ++lv) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const k3v2bf h = {(__bf16)v[2 * m], (__bf16)v[2 * m + 1]};
            const uint32_t hb = __builtin_bit_cast(uint32_t, h);
            if (pc == lv) w[m] = hb;
            if (lv + 1 < NPC16) {
                v[2 * m] -= __uint_as_float(hb << 16);
                v[2 * m + 1] -= __uint_as_float(hb & 0xffff0000u);
            }
        }
    }
    const bool on = col < 3 * T;
    return on ? make_uint4(w[0], w[1], w[2], w[3]) : make_uint4(0, 0, 0, 0);
}

/* The kernel's arguments, addressed in the constant address space: a phase function
 * moves the pointer to scalar registers and every field it reads comes back in scalar
 * registers (scalar loads), so buffer descriptors and loop bounds never become per-lane
 * values (which would turn each buffer load into a loop over lanes). */
#ifdef __HIP_DEVICE_COMPILE__
typedef const __attribute__((address_space(4))) K3kDecode *K3ArgPtr;
#else
typedef const K3kDecode *K3ArgPtr;   /* the host pass only parses the device code */
#endif

__device__ __forceinline__ K3ArgPtr k3d_uniform_cptr(K3ArgPtr p)
{
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (K3ArgPtr)(((uint64_t)hi << 32) | lo);
}

/* The slices of the bf16 ticket classes start at multiples of 32 KB of their tiled
 * matrices, and every wave of a class streams its slice from the first 8 KB batch to the
 * last at about the same pace: left alone, the waves' reads would all fall in the same
 * 8 KB of every 32 KB at once. With K3G_ROT, batch bi of a ticket's nb is taken at
 * position (bi + rot) mod nb, rot = ticket mod nb, so waves running together start at
 * different offsets (measured: no gain at the K2 and K3 shapes, so it is off). */
#ifndef K3G_ROT
#define K3G_ROT 0
#endif
__device__ __forceinline__ int k3d_batch_rot(int tk, int nb) { return K3G_ROT && nb > 0 ? tk % nb : 0; }
__device__ __forceinline__ int k3d_batch_at(int bi, int nb, int rot)
{
    const int b = bi + rot;
    return b >= nb ? b - nb : b;
}

template <int NT>
struct K3Dec {
    /* ----------------------------------------------------------------- X ---- */
    static __device__ __noinline__ void prep(K3ArgPtr ap, int tk_, int lane)
    {
        const K3kDecode a = *k3d_uniform_cptr(ap);
        const int tk = k3d_uniform(tk_);
        const K3Geo G = k3_geo(a.T, a.d, a.E, a.k, a.I, a.SI, a.L);
        const int npair = (G.nCd + 1) / 2;
        const int t = tk / npair, i = tk - t * npair;
        const K3Rsrc r8 = k3d_rsrc(a.xq8 + (size_t)t * G.nQd * K3G_BQ, (size_t)G.nQd * K3G_BQ);
        const K3Rsrc r16 = k3d_rsrc(a.xq16, (size_t)G.nCd * 1024);
        /* lanes 0-31: block 2i, lanes 32-63: block 2i + 1 (absent when nCd is odd) */
        const int b = 2 * i + (lane >> 5), e = lane & 31;
        const int col = 32 * b + e;
        const bool on = col < a.d;
        const float v = on ? a.x[(size_t)t * a.d + col] : 0.0f;
        const int Q = b >> 4;
        /* the bf16 pieces first: the shared expert's tickets wait only for these (up to
         * two tokens they make them themselves) */
        if (NT > K3G_XREG) {
            float r2 = v;
#pragma unroll
            for (int pc = 0; pc < NPC16; ++pc) {
                float back;
                const uint32_t h = k3d_bf16_rn(r2, back);
                r2 -= back;
                if (on) k3d_st16_sc1(r16, k3d_b16_off(col, NPC16 * t + pc), h);
            }
            k3d_arrive_event2(a.sync, G.cX16, G.nX, tk, G.eX16, lane);
        }
        /* x's FP8 pieces feed the routed gate/up; the latent layer's routed experts read
         * z's instead (the LD tickets make them) */
        if (!G.lat) {
            float r = v;
#pragma unroll
            for (int pc = 0; pc < NPC8; ++pc) {
                int sx;
                const uint32_t q = k3d_fp8_piece(r, sx);
                if (on) {
                    k3d_st8_sc1(r8, Q * K3G_BQ + k3d_bq_data(b, e, pc), q);
                    if (e == 0) k3d_st8_sc1(r8, Q * K3G_BQ + k3d_bq_scale(b, pc), sx + 127);
                }
            }
        }
        k3d_arrive_event2(a.sync, G.cX, G.nX, tk, G.eX, lane);
    }

    /* ----------------------------------------------------------------- R ---- */
    static __device__ __noinline__ void router(K3ArgPtr ap, int tk_, int lane, K3RouterLds *rl,
                                               bool wg_slices)
    {
        const K3kDecode a = *k3d_uniform_cptr(ap);
        if (a.given) return;
        const int tk = k3d_uniform(tk_);
        const K3Geo G = k3_geo(a.T, a.d, a.E, a.k, a.I, a.SI, a.L);
        const int e = tk / G.KSR, r = tk - e * G.KSR;
        const int ch0 = r * G.nRc / G.KSR, ch1 = (r + 1) * G.nRc / G.KSR;
        const K3Rsrc rg = k3d_rsrc(a.gate + (size_t)e * a.d, (size_t)a.d * 4);
        const K3Rsrc rx = k3d_rsrc(a.x, (size_t)a.T * a.d * 4);
        double acc[NT], ab[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) { acc[t] = 0.0; ab[t] = 0.0; }
        for (int cb = ch0; cb < ch1; cb += 2) {
            /* two 1024-column chunks per batch; columns past the slice or the row read
             * zero */
            uint4 W[8];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int col = (cb + h) * 1024 + lane * 16;
                const bool on = cb + h < ch1 && col < a.d;
#pragma unroll
                for (int i = 0; i < 4; ++i) W[4 * h + i] = k3d_b128(rg, on ? col * 4 + 16 * i : K3_OOB);
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (t < a.T) {
                    uint4 X[8];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int col = (cb + h) * 1024 + lane * 16;
                        const bool on = cb + h < ch1 && col < a.d;
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            X[4 * h + i] = k3d_b128(rx, on ? (t * a.d + col) * 4 + 16 * i : K3_OOB);
                    }
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const float w4[4] = {__uint_as_float(W[i].x), __uint_as_float(W[i].y),
                                             __uint_as_float(W[i].z), __uint_as_float(W[i].w)};
                        const float x4[4] = {__uint_as_float(X[i].x), __uint_as_float(X[i].y),
                                             __uint_as_float(X[i].z), __uint_as_float(X[i].w)};
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            acc[t] = fma((double)w4[q], (double)x4[q], acc[t]);
                            ab[t] = fma(fabs((double)w4[q]), fabs((double)x4[q]), ab[t]);
                        }
                    }
                }
            }
        }
        /* the slice's partial sums {sum, sum|w x|}: in LDS when the row's slices are the
         * four waves of this workgroup, else in memory, [t][e][slice] */
        const K3Rsrc rp = k3d_rsrc(a.rpart, (size_t)a.T * a.E * G.KSR * 16);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const double sv = k3d_wave_sumd(acc[t]);
            const double bv = k3d_wave_sumd(ab[t]);
            if (lane == 0 && t < a.T) {
                if (wg_slices) {
                    rl->part[r][t][0] = sv;
                    rl->part[r][t][1] = bv;
                } else {
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(k3v4u, make_double2(sv, bv)), rp,
                        ((t * a.E + e) * G.KSR + r) * 16, 0, K3_SC1);
                }
            }
        }
        if (wg_slices) {
            /* the workgroup's arrival count, in LDS: the wave that completes it has every
             * slice's partial sums (each wave's LDS writes are done before its count) */
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            int old = 0;
            if (lane == 0)
                old = __hip_atomic_fetch_add(&rl->count, 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_WORKGROUP);
            if (k3d_uniform(old) != G.KSR - 1) return;
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        } else if (!k3d_arrive(k3d_line(a.sync, G.lRE + e), G.KSR - 1, lane)) {
            return;
        }
        /* the last slice of the row: the slices summed in slice order, then the score
         * interval (any summation order is inside the interval's bound) */
        if (lane < a.T) {
            double2 pv[K3G_KS_R_MAX];
#pragma unroll
            for (int q = 0; q < K3G_KS_R_MAX; ++q) {
                if (wg_slices)
                    pv[q] = q < G.KSR ? make_double2(rl->part[q][lane][0], rl->part[q][lane][1])
                                     : make_double2(0.0, 0.0);
                else
                    pv[q] = __builtin_bit_cast(
                        double2, __builtin_amdgcn_raw_buffer_load_b128(
                                     rp, q < G.KSR ? ((lane * a.E + e) * G.KSR + q) * 16 : K3_OOB,
                                     0, K3_SC1));
            }
            double sv = 0.0, bv = 0.0;
#pragma unroll
            for (int q = 0; q < K3G_KS_R_MAX; ++q) {
                if (q < G.KSR) {
                    sv += pv[q].x;
                    bv += pv[q].y;
                }
            }
            const K3Rsrc rr = k3d_rsrc(a.rs, (size_t)a.T * a.E * 16);
            const float4 v = k3d_route_score(sv, bv, a.bias ? a.bias[e] : 0.0f, a.d);
            k3d_st4_sc1(rr, (lane * a.E + e) * 16, k3v4f{v.x, v.y, v.z, v.w});
        }
        k3d_arrive_event2(a.sync, G.cR, a.E, e, G.eR, lane);
    }

    /* ----------------------------------------------------------------- S ---- */
    static __device__ __noinline__ void select(K3ArgPtr ap, int lane, K3SelectLds *lds)
    {
        const K3kDecode a = *k3d_uniform_cptr(ap);
        const K3Geo G = k3_geo(a.T, a.d, a.E, a.k, a.I, a.SI, a.L);
        if (a.given) {
            /* the routing came with the call: publish it once x's pieces exist */
            if (!k3d_wait_event(a.sync, G.eX, 0, a.spin_limit, a.err, lane)) return;
            k3d_set_event(a.sync, G.eSEL, lane);
            host_routing(a, lane);
            return;
        }
        /* the routed tickets also need x's pieces: the routing is published once both
         * exist. x's pieces are done long before the router rows, so their event is
         * checked first, off the path from the last row to the publication. */
        if (!k3d_wait_event(a.sync, G.eX, 0, a.spin_limit, a.err, lane)) return;
        /* every router row in: the select is the only waiter, so it reads the rows'
         * sub-counters itself instead of waiting for the top count and the event flags
         * (one returning atomic and a flag store less on the routed experts' path) */
        if (!k3d_wait_sum(a.sync, G.cR + 1, NSUB, a.E, a.spin_limit, a.err, lane)) return;
        /* instrumentation: after the trace's [ticket][2] stamps, the select's own phases */
        if (a.trace && lane == 0) a.trace[3 * G.total] = wall_clock64();
        /* everything routed waits for this wave: let it issue ahead of its SIMD's others */
        __builtin_amdgcn_s_setprio(3);
        for (int t = 0; t < a.T; ++t)
            k3d_select_token(lds, t, (const float4 *)a.rs, a.bias, a.gate, a.x, a.d, a.E, a.k,
                             a.renorm, a.routed_scale, a.idx, a.wt, a.force, a.stats, lane,
                             a.trace && t == 0 ? a.trace + 3 * G.total + 2 : nullptr);
        if (a.trace && lane == 0) a.trace[3 * G.total + 1] = wall_clock64();
        k3d_set_event(a.sync, G.eSEL, lane);
        __builtin_amdgcn_s_setprio(0);
        host_routing(a, lane);
    }

    /* the published routing to the caller's host copies (after the event, off the routed
     * tickets' path); the event's release has made this wave's writes readable */
    static __device__ __forceinline__ void host_routing(const K3kDecode &a, int lane)
    {
        if (!a.hidx) return;
        /* system-scope stores are written through to the host's memory; the flag follows
         * once they are complete */
        for (int i = lane; i < a.T * a.k; i += 64) {
            const int e = __hip_atomic_load(&a.idx[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float w = __hip_atomic_load(&a.wt[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&a.hidx[i], e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(&a.hwt[i], w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        if (!a.hflag) return;
        __builtin_amdgcn_s_waitcnt(0);
        if (lane == 0)
            __hip_atomic_store(&a.hflag[K3K_HFLAG_ROUTED], 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
    }

    /* out[i] = v: with the host flags, a store written through to the host's memory (the
     * completion flag must not overtake it) */
    static __device__ __forceinline__ void put_out(const K3kDecode &a, size_t i, float v)
    {
        if (a.hflag && a.herr)
            __hip_atomic_store(&a.out[i], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        else a.out[i] = v;
    }

    /* With the host flags and herr: an output tile of 32 rows counts itself out once its
     * stores are complete (k3d_arrive waits for them); the last of the d/32 tiles passes the
     * device error word on to the host copy and marks the outputs complete. The tiles are the
     * last work of the launch (every other ticket feeds them), so the flag means the
     * caller's results are all there. */
    static __device__ __forceinline__ void out_done(const K3kDecode &a, const K3Geo &G, int tile,
                                                    int lane)
    {
        if (!a.hflag || !a.herr || !k3d_arrive2(a.sync, G.cOD, a.d / 32, tile, lane)) return;
        if (lane == 0) {
            const int e = a.err ? __hip_atomic_load(a.err, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT) : 0;
            if (e) __hip_atomic_store(a.herr, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __builtin_amdgcn_s_waitcnt(0);
            __hip_atomic_store(&a.hflag[K3K_HFLAG_DONE], 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }

    /* ---------------------------------------------------------------- SG ---- */
    static __device__ __noinline__ void shared_gateup(K3ArgPtr ap, int tk_, int lane)
    {
        const K3kDecode a = *k3d_uniform_cptr(ap);
        const int tk = k3d_uniform(tk_);
        const K3Geo G = k3_geo(a.T, a.d, a.E, a.k, a.I, a.SI, a.L);
        const int rg = tk / G.KSS, ks = tk - rg * G.KSS;    /* row group, K slice */
        const int c0 = ks * G.nCd / G.KSS, c1 = (ks + 1) * G.nCd / G.KSS;
        const size_t mb = (size_t)a.SI * a.d * 2;
        const K3Rsrc r1 = k3d_rsrc(a.sh1, mb), r3 = k3d_rsrc(a.sh3, mb);
        const K3Rsrc rb = k3d_rsrc(a.xq16, (size_t)G.nCd * 1024);
        const K3Rsrc rx = k3d_rsrc(a.x, (size_t)a.T * a.d * 4);
        const bool bon = (lane & 15) < NPC16 * a.T;
        k3v4f g[SG_TILES], u[SG_TILES];
#pragma unroll
        for (int j = 0; j < SG_TILES; ++j) {
            g[j] = k3v4f{0, 0, 0, 0};
            u[j] = k3v4f{0, 0, 0, 0};
        }
        /* tile j's chunk c: (SG_TILES rg + j) nCd + c KB in; tiles past SI read zero */
        const int abase = SG_TILES * rg * G.nCd * 1024 + lane * 16, tstride = G.nCd * 1024;
        bool first = true;
        if (NT <= K3G_XREG) k3d_trace_go(a.trace, G.oSG + tk, lane);
        const int nb = (c1 - c0 + SG_BATCH - 1) / SG_BATCH, rot = k3d_batch_rot(tk, nb);
        for (int bi = 0; bi < nb; ++bi) {
            const int cb = c0 + SG_BATCH * k3d_batch_at(bi, nb, rot);
            uint4 A1[SG_TILES][SG_BATCH], A3[SG_TILES][SG_BATCH], B[SG_BATCH];
            if (NT <= K3G_XREG) {
                /* x's halves first, so they can be used before the weights land */
#pragma unroll
                for (int i = 0; i < SG_BATCH; ++i)
                    B[i] = k3d_b128(rx, cb + i < c1 ? k3d_xb16_off(a.T, a.d, cb + i, lane)
                                                   : K3_OOB);
            }
#pragma unroll
            for (int i = 0; i < SG_BATCH; ++i) {
                const int c = cb + i;
#pragma unroll
                for (int j = 0; j < SG_TILES; ++j) {
                    const int o = abase + j * tstride + c * 1024;
                    A1[j][i] = k3d_b128(r1, c < c1 ? o : K3_OOB);
                    A3[j][i] = k3d_b128(r3, c < c1 ? o : K3_OOB);
                }
            }
            if (NT <= K3G_XREG) {
#pragma unroll
                for (int i = 0; i < SG_BATCH; ++i) B[i] = k3d_xb16_make(B[i], a.T, lane);
            } else {
                if (first) {
                    /* the first weights stream in while x's bf16 pieces are made */
                    if (!k3d_wait_event(a.sync, G.eX16, tk, a.spin_limit, a.err, lane))
                        return;
                    k3d_trace_go(a.trace, G.oSG + tk, lane);
                    first = false;
                }
#pragma unroll
                for (int i = 0; i < SG_BATCH; ++i) {
                    const int c = cb + i;
                    B[i] = k3d_b128<K3_BPOL>(rb, bon && c < c1 ? c * 1024 + lane * 16 : K3_OOB);
                }
            }
#pragma unroll
            for (int i = 0; i < SG_BATCH; ++i)
#pragma unroll
                for (int j = 0; j < SG_TILES; ++j) {
                    g[j] = k3d_mma16(A1[j][i], B[i], g[j]);
                    u[j] = k3d_mma16(A3[j][i], B[i], u[j]);
                }
        }
        const int t = lane & 15;
        const K3Rsrc rp = k3d_rsrc(a.sgpart, (size_t)G.KSS * a.T * 2 * a.SI * 4);
#pragma unroll
        for (int j = 0; j < SG_TILES; ++j) {
            g[j] = k3d_colsum3(g[j], lane);
            u[j] = k3d_colsum3(u[j], lane);
            const int row = 16 * (SG_TILES * rg + j) + 4 * (lane >> 4);
            if (t < a.T && row < a.SI) {
                k3d_st4_sc1(rp, (((ks * a.T + t) * 2 + 0) * a.SI + row) * 4, g[j]);
                k3d_st4_sc1(rp, (((ks * a.T + t) * 2 + 1) * a.SI + row) * 4, u[j]);
            }
        }
        if (!k3d_arrive(k3d_line(a.sync, G.lTSG + rg), G.KSS - 1, lane)) return;
        /* last slice of the row group: h = act(gate, up) for its 64 rows x T tokens (lane:
         * row) -> bf16 pieces */
        const int row = 16 * SG_TILES * rg + lane;
        const K3Rsrc rh = k3d_rsrc(a.hq16, (size_t)G.nCsi * 1024);
        for (int tt = 0; tt < a.T; ++tt) {
            if (lane < 16 * SG_TILES && row < a.SI) {
                const int qs = a.T * 2 * a.SI * 4;
                const float gs = k3d_sum_sc1<K3G_KS_SG_MAX>(rp, ((tt * 2 + 0) * a.SI + row) * 4, qs,
                                                        G.KSS);
                const float us = k3d_sum_sc1<K3G_KS_SG_MAX>(rp, ((tt * 2 + 1) * a.SI + row) * 4, qs,
                                                        G.KSS);
                float r2 = k3d_act(gs, us, a.b1, a.b2);
#pragma unroll
                for (int pc = 0; pc < NPC16; ++pc) {
                    float back;
                    const uint32_t h = k3d_bf16_rn(r2, back);
                    r2 -= back;
                    k3d_st16_sc1(rh, k3d_b16_off(row, NPC16 * tt + pc), h);
                }
            }
        }
        k3d_arrive_event2(a.sync, G.cSGF, G.nSGt, rg, G.eSGF, lane);
    }

    /* ----------------------------------------------------------------- G ---- */
    static __device__ __noinline__ void routed_gateup(K3ArgPtr ap, int tk_, int lane)
    {
        const K3kDecode a = *k3d_uniform_cptr(ap);
        const int tk = k3d_uniform(tk_);
        const K3Geo G = k3_geo(a.T, a.d, a.E, a.k, a.I, a.SI, a.L);
        const int per = G.nGt * G.KSG;
        const int p = tk / per, rem = tk - p * per;
        const int gt = rem / G.KSG, ks = rem - gt * G.KSG;
        const int q0 = ks * G.nQk / G.KSG, q1 = (ks + 1) * G.nQk / G.KSG;
        const int t = p / a.k;
        if (!k3d_wait_event(a.sync, G.eSEL, tk, a.spin_limit, a.err, lane)) return;
        /* the latent layer's routed input is z = down x */
        if (G.lat && !k3d_wait_event(a.sync, G.eZ, tk, a.spin_limit, a.err, lane)) return;
        k3d_trace_go(a.trace, G.oG + tk, lane);
        const int e = k3d_uniform(__hip_atomic_load(&a.idx[p], __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT));
        k3v4f acc[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
        if (e >= 0 && e < a.E) {
            const uint8_t *w1 = k3d_uniform_ptr((const uint8_t *)a.eq[e].p1);
            const uint8_t *w3 = k3d_uniform_ptr((const uint8_t *)a.eq[e].p3);
            const size_t mb = (size_t)(a.I / 16) * G.nQk * K3G_QT;
            const K3Rsrc r1 = k3d_rsrc(w1, mb), r3 = k3d_rsrc(w3, mb);
            const uint8_t *bsrc = G.lat ? a.zq8 : a.xq8;
            const K3Rsrc rb = k3d_rsrc(bsrc + (size_t)t * G.nQk * K3G_BQ, (size_t)G.nQk * K3G_BQ);
            const bool bon = (lane & 15) < NPC8;
            const int rs = G.nQk * K3G_QT;                    /* bytes per row block */
            const int o0 = 2 * gt * rs + lane * 16, o1 = o0 + rs;
            for (int Q = q0; Q < q1; ++Q) {
                const int qo = Q * K3G_QT;
                uint4 A[4][4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    A[0][j] = k3d_b128(r1, o0 + qo + 1024 * j);
                    A[1][j] = k3d_b128(r1, o1 + qo + 1024 * j);
                    A[2][j] = k3d_b128(r3, o0 + qo + 1024 * j);
                    A[3][j] = k3d_b128(r3, o1 + qo + 1024 * j);
                }
                const int so = qo + 4096 + lane * 4 - lane * 16;
                const uint32_t s0 = k3d_b32(r1, o0 + so), s1 = k3d_b32(r1, o1 + so);
                const uint32_t s2 = k3d_b32(r3, o0 + so), s3 = k3d_b32(r3, o1 + so);
                uint4 B[4][2];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    B[j][0] = k3d_b128<K3_BPOL>(rb, bon ? Q * K3G_BQ + j * 2048 + lane * 32 : K3_OOB);
                    B[j][1] = k3d_b128<K3_BPOL>(rb, bon ? Q * K3G_BQ + j * 2048 + lane * 32 + 16 : K3_OOB);
                }
                const uint32_t sb = k3d_b32<K3_BPOL>(rb, Q * K3G_BQ + 8192 + lane * 4);
                const k3v8i b0 = k3d_b8(B[0][0], B[0][1]), b1 = k3d_b8(B[1][0], B[1][1]);
                const k3v8i b2 = k3d_b8(B[2][0], B[2][1]), b3 = k3d_b8(B[3][0], B[3][1]);
                acc[0] = k3d_mma4<0>(A[0][0], b0, acc[0], s0, sb);
                acc[1] = k3d_mma4<0>(A[1][0], b0, acc[1], s1, sb);
                acc[2] = k3d_mma4<0>(A[2][0], b0, acc[2], s2, sb);
                acc[3] = k3d_mma4<0>(A[3][0], b0, acc[3], s3, sb);
                acc[0] = k3d_mma4<1>(A[0][1], b1, acc[0], s0, sb);
                acc[1] = k3d_mma4<1>(A[1][1], b1, acc[1], s1, sb);
                acc[2] = k3d_mma4<1>(A[2][1], b1, acc[2], s2, sb);
                acc[3] = k3d_mma4<1>(A[3][1], b1, acc[3], s3, sb);
                acc[0] = k3d_mma4<2>(A[0][2], b2, acc[0], s0, sb);
                acc[1] = k3d_mma4<2>(A[1][2], b2, acc[1], s1, sb);
                acc[2] = k3d_mma4<2>(A[2][2], b2, acc[2], s2, sb);
                acc[3] = k3d_mma4<2>(A[3][2], b2, acc[3], s3, sb);
                acc[0] = k3d_mma4<3>(A[0][3], b3, acc[0], s0, sb);
                acc[1] = k3d_mma4<3>(A[1][3], b3, acc[1], s1, sb);
                acc[2] = k3d_mma4<3>(A[2][3], b3, acc[2], s2, sb);
                acc[3] = k3d_mma4<3>(A[3][3], b3, acc[3], s3, sb);
            }
        } else if (e >= a.E) {
            k3d_raise(a.err, K3G_ERR_EXPERT_RANGE);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) acc[m] = k3d_colsum(acc[m]);
        const K3Rsrc rp = k3d_rsrc(a.gpart, (size_t)G.P * G.KSG * 2 * a.I * 4);
        if ((lane & 15) == 0) {
            const int r4 = 32 * gt + 4 * (lane >> 4);
#pragma unroll
            for (int m = 0; m < 4; ++m)
                k3d_st4_sc1(rp, (((p * G.KSG + ks) * 2 + (m >> 1)) * a.I + r4 + 16 * (m & 1)) * 4,
                            acc[m]);
        }
        if (!k3d_arrive(k3d_line(a.sync, G.lTG + p * G.nGt + gt), G.KSG - 1, lane))
            return;
        /* last slice of the tile: 32 rows of h = act(gate, up) -> FP8 pieces (one block) */
        const int r = lane & 31, row = 32 * gt + r;
        const float gs = k3d_sum_sc1<K3G_KS_G_MAX>(rp, ((p * G.KSG * 2 + 0) * a.I + row) * 4,
                                               2 * a.I * 4, G.KSG);
        const float us = k3d_sum_sc1<K3G_KS_G_MAX>(rp, ((p * G.KSG * 2 + 1) * a.I + row) * 4,
                                               2 * a.I * 4, G.KSG);
        float h = lane < 32 ? k3d_act(gs, us, a.b1, a.b2) : 0.0f;
        const K3Rsrc rh = k3d_rsrc(a.hq8 + (size_t)p * G.nQi * K3G_BQ, (size_t)G.nQi * K3G_BQ);
        const int Qh = gt >> 4;
#pragma unroll
        for (int pc = 0; pc < NPC8; ++pc) {
            int sx;
            const uint32_t q = k3d_fp8_piece(h, sx);
            if (lane < 32) {
                k3d_st8_sc1(rh, Qh * K3G_BQ + k3d_bq_data(gt, r, pc), q);
                if (lane == 0) k3d_st8_sc1(rh, Qh * K3G_BQ + k3d_bq_scale(gt, pc), sx + 127);
            }
        }
        k3d_arrive_event2(a.sync, G.cGF + p * (1 + NSUB), G.nGt, gt, G.eGF + p * K3_EVLINES, lane);
    }

    /* ---------------------------------------------------------------- SD ---- */
    static __device__ __noinline__ void shared_down(K3ArgPtr ap, int tk_, int lane)
    {
        const K3kDecode a = *k3d_uniform_cptr(ap);
        const int tk = k3d_uniform(tk_);
        const K3Geo G = k3_geo(a.T, a.d, a.E, a.k, a.I, a.SI, a.L);
        const int rt = tk / G.KSD, ks = tk - rt * G.KSD;
        const int c0 = ks * G.nCsi / G.KSD, c1 = (ks + 1) * G.nCsi / G.KSD;
        const K3Rsrc r2 = k3d_rsrc(a.sh2, (size_t)a.d * a.SI * 2);
        const K3Rsrc rb = k3d_rsrc(a.hq16, (size_t)G.nCsi * 1024);
        const bool bon = (lane & 15) < NPC16 * a.T;
        k3v4f y0 = {0, 0, 0, 0}, y1 = {0, 0, 0, 0};
        const int o0 = 2 * rt * G.nCsi * 1024 + lane * 16, o1 = o0 + G.nCsi * 1024;
        bool first = true;
        const int nb = (c1 - c0 + 7) / 8, rot = k3d_batch_rot(tk, nb);
        for (int bi = 0; bi < nb; ++bi) {
            const int cb = c0 + 8 * k3d_batch_at(bi, nb, rot);
            uint4 A0[8], A1[8], B[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int c = cb + i;
                A0[i] = k3d_b128(r2, c < c1 ? o0 + c * 1024 : K3_OOB);
                A1[i] = k3d_b128(r2, c < c1 ? o1 + c * 1024 : K3_OOB);
            }
            if (first) {   /* the first weights stream in while the shared h is finished */
                if (!k3d_wait_event(a.sync, G.eSGF, tk, a.spin_limit, a.err, lane)) return;
                k3d_trace_go(a.trace, G.oSD + tk, lane);
                first = false;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int c = cb + i;
                B[i] = k3d_b128<K3_BPOL>(rb, bon && c < c1 ? c * 1024 + lane * 16 : K3_OOB);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                y0 = k3d_mma16(A0[i], B[i], y0);
                y1 = k3d_mma16(A1[i], B[i], y1);
            }
        }
        y0 = k3d_colsum3(y0, lane);
        y1 = k3d_colsum3(y1, lane);
        const int t = lane & 15;
        if (t < a.T) {
            const K3Rsrc rp = k3d_rsrc(a.shpart, (size_t)G.KSD * a.T * a.d * 4);
            const int row = 32 * rt + 4 * (lane >> 4);
            k3d_st4_sc1(rp, ((ks * a.T + t) * a.d + row) * 4, y0);
            k3d_st4_sc1(rp, ((ks * a.T + t) * a.d + row + 16) * 4, y1);
        }
        if (G.lat) {
            if (k3d_arrive(k3d_line(a.sync, G.lLU + rt), G.KSLU + G.KSD - 1, lane))
                combine_out(a, G, rt, lane);
        } else if (k3d_arrive(k3d_line(a.sync, G.lDT + rt), G.P * G.KSDN + G.KSD - 1, lane)) {
            combine_rows(a, G, rt, lane);
        }
    }

    /* ----------------------------------------------------------------- D ---- */
    static __device__ __noinline__ void routed_down(K3ArgPtr ap, int tk_, int lane)
    {
        const K3kDecode a = *k3d_uniform_cptr(ap);
        const int tk = k3d_uniform(tk_);
        const K3Geo G = k3_geo(a.T, a.d, a.E, a.k, a.I, a.SI, a.L);
        const int per = G.nDt * G.KSDN;
        const int p = tk / per, rem = tk - p * per;
        const int dt = rem / G.KSDN, ks = rem - dt * G.KSDN;
        const int q0 = ks * G.nQi / G.KSDN, q1 = (ks + 1) * G.nQi / G.KSDN;
        if (!k3d_wait_event(a.sync, G.eSEL, tk, a.spin_limit, a.err, lane)) return;
        const int e = k3d_uniform(__hip_atomic_load(&a.idx[p], __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT));
        k3v4f y0 = {0, 0, 0, 0}, y1 = {0, 0, 0, 0};
        if (e >= 0 && e < a.E) {
            const uint8_t *w2 = k3d_uniform_ptr((const uint8_t *)a.eq[e].p2);
            const K3Rsrc r2 = k3d_rsrc(w2, (size_t)(G.Dout / 16) * G.nQi * K3G_QT);
            const K3Rsrc rb = k3d_rsrc(a.hq8 + (size_t)p * G.nQi * K3G_BQ, (size_t)G.nQi * K3G_BQ);
            const bool bon = (lane & 15) < NPC8;
            const int rs = G.nQi * K3G_QT;
            const int o0 = 2 * dt * rs + lane * 16, o1 = o0 + rs;
            bool first = true;
            for (int Q = q0; Q < q1; ++Q) {
                const int qo = Q * K3G_QT;
                uint4 A[2][4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    A[0][j] = k3d_b128(r2, o0 + qo + 1024 * j);
                    A[1][j] = k3d_b128(r2, o1 + qo + 1024 * j);
                }
                const int so = qo + 4096 + lane * 4 - lane * 16;
                const uint32_t s0 = k3d_b32(r2, o0 + so), s1 = k3d_b32(r2, o1 + so);
                if (first) {   /* the first weights stream in while this pair's h finishes */
                    if (!k3d_wait_event(a.sync, G.eGF + p * K3_EVLINES, tk, a.spin_limit,
                                        a.err, lane))
                        return;
                    k3d_trace_go(a.trace, G.oD + tk, lane);
                    first = false;
                }
                uint4 B[4][2];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    B[j][0] = k3d_b128<K3_BPOL>(rb, bon ? Q * K3G_BQ + j * 2048 + lane * 32 : K3_OOB);
                    B[j][1] = k3d_b128<K3_BPOL>(rb, bon ? Q * K3G_BQ + j * 2048 + lane * 32 + 16 : K3_OOB);
                }
                const uint32_t sb = k3d_b32<K3_BPOL>(rb, Q * K3G_BQ + 8192 + lane * 4);
                const k3v8i b0 = k3d_b8(B[0][0], B[0][1]), b1 = k3d_b8(B[1][0], B[1][1]);
                const k3v8i b2 = k3d_b8(B[2][0], B[2][1]), b3 = k3d_b8(B[3][0], B[3][1]);
                y0 = k3d_mma4<0>(A[0][0], b0, y0, s0, sb);
                y1 = k3d_mma4<0>(A[1][0], b0, y1, s1, sb);
                y0 = k3d_mma4<1>(A[0][1], b1, y0, s0, sb);
                y1 = k3d_mma4<1>(A[1][1], b1, y1, s1, sb);
                y0 = k3d_mma4<2>(A[0][2], b2, y0, s0, sb);
                y1 = k3d_mma4<2>(A[1][2], b2, y1, s1, sb);
                y0 = k3d_mma4<3>(A[0][3], b3, y0, s0, sb);
                y1 = k3d_mma4<3>(A[1][3], b3, y1, s1, sb);
            }
        }
        y0 = k3d_colsum(y0);
        y1 = k3d_colsum(y1);
        if ((lane & 15) == 0) {
            const K3Rsrc rc = k3d_rsrc(a.contrib, (size_t)G.P * G.KSDN * G.Dout * 4);
            const int row = 32 * dt + 4 * (lane >> 4);
            k3d_st4_sc1(rc, ((p * G.KSDN + ks) * G.Dout + row) * 4, y0);
            k3d_st4_sc1(rc, ((p * G.KSDN + ks) * G.Dout + row + 16) * 4, y1);
        }
        if (G.lat) {
            /* the latent layer: the slots' aggregate (the shared expert joins after up) */
            if (k3d_arrive(k3d_line(a.sync, G.lDT + dt), G.P * G.KSDN - 1, lane))
                combine_latent(a, G, dt, lane);
        } else if (k3d_arrive(k3d_line(a.sync, G.lDT + dt), G.P * G.KSDN + G.KSD - 1, lane)) {
            combine_rows(a, G, dt, lane);
        }
    }

    /* ---------------------------------------------------------------- LD ---- */
    /* z = down x for 32 latent rows x a K slice (tiled bf16 down [L][d], B = x's bf16
     * pieces, as the shared gate/up reads them); the last slice of a row tile sums the
     * slices in slice order and writes the 32 values' FP8 pieces (one MX block) for the
     * routed gate/up (src/core/k3_ops.c:600: z = down x). */
    static __device__ __noinline__ void latent_down(K3ArgPtr ap, int tk_, int lane)
    {
        const K3kDecode a = *k3d_uniform_cptr(ap);
        const int tk = k3d_uniform(tk_);
        const K3Geo G = k3_geo(a.T, a.d, a.E, a.k, a.I, a.SI, a.L);
        const int rt = tk / G.KSLD, ks = tk - rt * G.KSLD;
        const int c0 = ks * G.nCd / G.KSLD, c1 = (ks + 1) * G.nCd / G.KSLD;
        const K3Rsrc rw = k3d_rsrc(a.down, (size_t)G.L * a.d * 2);
        const K3Rsrc rb = k3d_rsrc(a.xq16, (size_t)G.nCd * 1024);
        const K3Rsrc rx = k3d_rsrc(a.x, (size_t)a.T * a.d * 4);
        const bool bon = (lane & 15) < NPC16 * a.T;
        k3v4f y0 = {0, 0, 0, 0}, y1 = {0, 0, 0, 0};
        const int o0 = 2 * rt * G.nCd * 1024 + lane * 16, o1 = o0 + G.nCd * 1024;
        bool first = true;
        if (NT <= K3G_XREG) k3d_trace_go(a.trace, G.oLD + tk, lane);
        const int nb = (c1 - c0 + 7) / 8, rot = k3d_batch_rot(tk, nb);
        for (int bi = 0; bi < nb; ++bi) {
            const int cb = c0 + 8 * k3d_batch_at(bi, nb, rot);
            uint4 A0[8], A1[8], B[8];
            if (NT <= K3G_XREG) {
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    B[i] = k3d_b128(rx, cb + i < c1 ? k3d_xb16_off(a.T, a.d, cb + i, lane)
                                                   : K3_OOB);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int c = cb + i;
                A0[i] = k3d_b128(rw, c < c1 ? o0 + c * 1024 : K3_OOB);
                A1[i] = k3d_b128(rw, c < c1 ? o1 + c * 1024 : K3_OOB);
            }
            if (NT <= K3G_XREG) {
#pragma unroll
                for (int i = 0; i < 8; ++i) B[i] = k3d_xb16_make(B[i], a.T, lane);
            } else {
                if (first) {
                    if (!k3d_wait_event(a.sync, G.eX16, tk, a.spin_limit, a.err, lane))
                        return;
                    k3d_trace_go(a.trace, G.oLD + tk, lane);
                    first = false;
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int c = cb + i;
                    B[i] = k3d_b128<K3_BPOL>(rb, bon && c < c1 ? c * 1024 + lane * 16 : K3_OOB);
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                y0 = k3d_mma16(A0[i], B[i], y0);
                y1 = k3d_mma16(A1[i], B[i], y1);
            }
        }
        y0 = k3d_colsum3(y0, lane);
        y1 = k3d_colsum3(y1, lane);
        const K3Rsrc rp = k3d_rsrc(a.zpart, (size_t)G.KSLD * a.T * G.L * 4);
        if ((lane & 15) < a.T) {
            const int t = lane & 15, row = 32 * rt + 4 * (lane >> 4);
            k3d_st4_sc1(rp, ((ks * a.T + t) * G.L + row) * 4, y0);
            k3d_st4_sc1(rp, ((ks * a.T + t) * G.L + row + 16) * 4, y1);
        }
        if (!k3d_arrive(k3d_line(a.sync, G.lLD + rt), G.KSLD - 1, lane)) return;
        /* last slice of the row tile: rows 32 rt + r (lane r < 32) of z -> FP8 pieces */
        const int r = lane & 31, row = 32 * rt + r;
        const K3Rsrc rz = k3d_rsrc(a.zq8, (size_t)a.T * G.nQk * K3G_BQ);
        const int Qz = rt >> 4;
        for (int tt = 0; tt < a.T; ++tt) {
            const float zs = k3d_sum_sc1<K3G_KS_LD>(rp, (tt * G.L + row) * 4, a.T * G.L * 4,
                                                    G.KSLD);
            float h = lane < 32 ? zs : 0.0f;
            const int qb = (tt * G.nQk + Qz) * K3G_BQ;
#pragma unroll
            for (int pc = 0; pc < NPC8; ++pc) {
                int sx;
                const uint32_t q = k3d_fp8_piece(h, sx);
                if (lane < 32) {
                    k3d_st8_sc1(rz, qb + k3d_bq_data(rt, r, pc), q);
                    if (lane == 0) k3d_st8_sc1(rz, qb + k3d_bq_scale(rt, pc), sx + 127);
                }
            }
        }
        k3d_arrive_event2(a.sync, G.cZ, G.nLDt, rt, G.eZ, lane);
    }

    /* ---------------------------------------------------------------- NR ---- */
    /* The aggregate's RMSNorm for 64 latent columns of every token (src/core/k3_ops.c:
     * 94-102 on accL, :646): inv = (float)(1 / sqrt(sum_double a^2 / L + eps)) from the
     * row tiles' sums (added in tile order), y = lnorm * a * inv (float, the engine's
     * order), then y's bf16 pieces (the latent up's B operand). No lnorm: y = a. */
    static __device__ __noinline__ void norm(K3ArgPtr ap, int tk_, int lane)
    {
        const K3kDecode a = *k3d_uniform_cptr(ap);
        const int tk = k3d_uniform(tk_);
        const K3Geo G = k3_geo(a.T, a.d, a.E, a.k, a.I, a.SI, a.L);
        if (!k3d_wait_event(a.sync, G.eA, tk, a.spin_limit, a.err, lane)) return;
        k3d_trace_go(a.trace, G.oNR + tk, lane);
        const int col = 64 * tk + lane;
        const bool on = col < G.L;
        const K3Rsrc rn = k3d_rsrc(a.nss, (size_t)a.T * G.nDt * 8);
        const K3Rsrc ra = k3d_rsrc(a.accl, (size_t)a.T * G.L * 4);
        const K3Rsrc rq = k3d_rsrc(a.aq16, (size_t)G.nCL * 1024);
        for (int t = 0; t < a.T; ++t) {
            float inv = 1.0f;
            if (a.lnorm) {
                /* every tile's sum, lane l taking tiles l, l + 64, ..., in that order, then
                 * the wave's fixed-order reduction: the same sum in every NR ticket */
                double s = 0.0;
                for (int q = lane; q < G.nDt; q += 64)
                    s += __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(
                                                        rn, (t * G.nDt + q) * 8, 0, K3_SC1));
                s = k3d_wave_sumd(s);
                inv = (float)(1.0 / sqrt(s / (double)G.L + (double)a.rms_eps));
            }
            const float v = k3d_f32_sc1(ra, on ? (t * G.L + col) * 4 : K3_OOB);
            float y = a.lnorm && on ? __fmul_rn(__fmul_rn(a.lnorm[col], v), inv) : v;
#pragma unroll
            for (int pc = 0; pc < NPC16; ++pc) {
                float back;
                const uint32_t h = k3d_bf16_rn(y, back);
                y -= back;
                if (on) k3d_st16_sc1(rq, k3d_b16_off(col, NPC16 * t + pc), h);
            }
        }
        k3d_arrive_event2(a.sync, G.cN, G.nNR, tk, G.eN, lane);
    }

    /* ---------------------------------------------------------------- LU ---- */
    /* out = up * aggregate for 32 output rows x a K slice (tiled bf16 up [d][L], B = the
     * normalised aggregate's bf16 pieces): the first weights stream in while the norm
     * finishes. The last arrival of an output tile (LU's and the shared down's slices)
     * writes out (src/core/k3_ops.c:647-654). */
    static __device__ __noinline__ void latent_up(K3ArgPtr ap, int tk_, int lane)
    {
        const K3kDecode a = *k3d_uniform_cptr(ap);
        const int tk = k3d_uniform(tk_);
        const K3Geo G = k3_geo(a.T, a.d, a.E, a.k, a.I, a.SI, a.L);
        const int rt = tk / G.KSLU, ks = tk - rt * G.KSLU;
        const int c0 = ks * G.nCL / G.KSLU, c1 = (ks + 1) * G.nCL / G.KSLU;
        const K3Rsrc rw = k3d_rsrc(a.up, (size_t)a.d * G.L * 2);
        const K3Rsrc rb = k3d_rsrc(a.aq16, (size_t)G.nCL * 1024);
        const bool bon = (lane & 15) < NPC16 * a.T;
        k3v4f y0 = {0, 0, 0, 0}, y1 = {0, 0, 0, 0};
        const int o0 = 2 * rt * G.nCL * 1024 + lane * 16, o1 = o0 + G.nCL * 1024;
        bool first = true;
        const int nb = (c1 - c0 + 7) / 8, rot = k3d_batch_rot(tk, nb);
        for (int bi = 0; bi < nb; ++bi) {
            const int cb = c0 + 8 * k3d_batch_at(bi, nb, rot);
            uint4 A0[8], A1[8], B[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int c = cb + i;
                A0[i] = k3d_b128(rw, c < c1 ? o0 + c * 1024 : K3_OOB);
                A1[i] = k3d_b128(rw, c < c1 ? o1 + c * 1024 : K3_OOB);
            }
            if (first) {
                if (!k3d_wait_event(a.sync, G.eN, tk, a.spin_limit, a.err, lane)) return;
                k3d_trace_go(a.trace, G.oLU + tk, lane);
                first = false;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int c = cb + i;
                B[i] = k3d_b128<K3_BPOL>(rb, bon && c < c1 ? c * 1024 + lane * 16 : K3_OOB);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                y0 = k3d_mma16(A0[i], B[i], y0);
                y1 = k3d_mma16(A1[i], B[i], y1);
            }
        }
        y0 = k3d_colsum3(y0, lane);
        y1 = k3d_colsum3(y1, lane);
        if ((lane & 15) < a.T) {
            const K3Rsrc rp = k3d_rsrc(a.upart, (size_t)G.KSLU * a.T * a.d * 4);
            const int t = lane & 15, row = 32 * rt + 4 * (lane >> 4);
            k3d_st4_sc1(rp, ((ks * a.T + t) * a.d + row) * 4, y0);
            k3d_st4_sc1(rp, ((ks * a.T + t) * a.d + row + 16) * 4, y1);
        }
        if (k3d_arrive(k3d_line(a.sync, G.lLU + rt), G.KSLU + G.KSD - 1, lane))
            combine_out(a, G, rt, lane);
    }

    /* The latent layer's aggregate for latent rows 32 dt .. + 31, once every slot's
     * down-projection slices are in: slots in the engine's order (float multiply, then
     * add, src/core/k3_ops.c:641-642), stored for the norm, with the rows' sum of squares
     * (fp64; a float's square is exact in it). Lane r < 32 owns row 32 dt + r. */
    static __device__ void combine_latent(const K3kDecode &a, const K3Geo &G, int dt, int lane)
    {
        const int row = 32 * dt + (lane & 31);
        const K3Rsrc rc = k3d_rsrc(a.contrib, (size_t)G.P * G.KSDN * G.Dout * 4);
        const K3Rsrc ra = k3d_rsrc(a.accl, (size_t)a.T * G.L * 4);
        const K3Rsrc rn = k3d_rsrc(a.nss, (size_t)a.T * G.nDt * 8);
        for (int t = 0; t < a.T; ++t) {
            int ev = -1;
            float wv = 0.0f;
            if (lane < a.k) {
                ev = __hip_atomic_load(&a.idx[t * a.k + lane], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                wv = __hip_atomic_load(&a.wt[t * a.k + lane], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
            float c = 0.0f;
            for (int j0 = 0; j0 < a.k; j0 += 8) {
                float y[8][K3G_KS_D_MAX];
#pragma unroll
                for (int jj = 0; jj < 8; ++jj)
#pragma unroll
                    for (int q = 0; q < K3G_KS_D_MAX; ++q) {
                        const int p = t * a.k + j0 + jj;
                        y[jj][q] = __uint_as_float(k3d_b32<K3_BPOL>(
                            rc, j0 + jj < a.k && q < G.KSDN
                                    ? ((p * G.KSDN + q) * G.Dout + row) * 4 : K3_OOB));
                    }
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const int j = j0 + jj;
                    if (j >= a.k) break;
                    const int e = __builtin_amdgcn_readlane(ev, j);
                    if (e < 0 || e >= a.E) continue;
                    const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wv), j));
                    float yy = 0.0f;
#pragma unroll
                    for (int q = 0; q < K3G_KS_D_MAX; ++q)
                        if (q < G.KSDN) yy += y[jj][q];
                    c = __fadd_rn(c, __fmul_rn(w, yy));
                }
            }
            if (lane < 32)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(c), ra, (t * G.L + row) * 4,
                                                      0, K3_SC1);
            const double sq = k3d_wave_sumd(lane < 32 ? (double)c * (double)c : 0.0);
            if (lane == 0)
                __builtin_amdgcn_raw_buffer_store_b64(
                    __builtin_bit_cast(unsigned int __attribute__((ext_vector_type(2))), sq), rn,
                    (t * G.nDt + dt) * 8, 0, K3_SC1);
        }
        k3d_arrive_event2(a.sync, G.cA, G.nDt, dt, G.eA, lane);
    }

    /* The latent layer's output rows 32 rt .. + 31, once the latent up's and the shared
     * down's slices for them are in: up * aggregate (slices in order), then + the shared
     * output (slices in order), one float add (src/core/k3_ops.c:654). */
    static __device__ void combine_out(const K3kDecode &a, const K3Geo &G, int rt, int lane)
    {
        const int row = 32 * rt + (lane & 31);
        const K3Rsrc ru = k3d_rsrc(a.upart, (size_t)G.KSLU * a.T * a.d * 4);
        const K3Rsrc rs = k3d_rsrc(a.shpart, (size_t)(G.KSD > 0 ? G.KSD : 1) * a.T * a.d * 4);
        for (int t = 0; t < a.T; ++t) {
            float uv[K3G_KS_LU], sh[K3G_KS_SD_MAX];
#pragma unroll
            for (int q = 0; q < K3G_KS_LU; ++q)
                uv[q] = __uint_as_float(k3d_b32<K3_BPOL>(
                    ru, q < G.KSLU ? ((q * a.T + t) * a.d + row) * 4 : K3_OOB));
#pragma unroll
            for (int q = 0; q < K3G_KS_SD_MAX; ++q)
                sh[q] = __uint_as_float(k3d_b32<K3_BPOL>(
                    rs, a.SI > 0 && q < G.KSD ? ((q * a.T + t) * a.d + row) * 4 : K3_OOB));
            float c = 0.0f;
#pragma unroll
            for (int q = 0; q < K3G_KS_LU; ++q)
                if (q < G.KSLU) c += uv[q];
            if (a.SI > 0) {
                float s2 = 0.0f;
#pragma unroll
                for (int q = 0; q < K3G_KS_SD_MAX; ++q)
                    if (q < G.KSD) s2 += sh[q];
                c = __fadd_rn(c, s2);
            }
            if (lane < 32) put_out(a, (size_t)t * a.d + row, c);
        }
        out_done(a, G, rt, lane);
    }

    /* ------------------------------------------------------------ combine ---- */
    /* Rows 32 dt .. 32 dt + 31 of the output, once every routed slot's down-projection
     * slices and the shared expert's slices for them are in: slots in the engine's order
     * (float multiply, then add), then + the shared output (slices summed in order).
     * Lane r < 32 owns row 32 dt + r. */
    static __device__ void combine_rows(const K3kDecode &a, const K3Geo &G, int dt, int lane)
    {
        const int row = 32 * dt + (lane & 31);
        const K3Rsrc rc = k3d_rsrc(a.contrib, (size_t)G.P * G.KSDN * a.d * 4);
        const K3Rsrc rs = k3d_rsrc(a.shpart, (size_t)(G.KSD > 0 ? G.KSD : 1) * a.T * a.d * 4);
        for (int t = 0; t < a.T; ++t) {
            /* every load is issued before any is used: lane j < k holds slot j's routing,
             * then the slices of 8 slots (and the shared expert's) are read at once */
            int ev = -1;
            float wv = 0.0f;
            if (lane < a.k) {
                ev = __hip_atomic_load(&a.idx[t * a.k + lane], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                wv = __hip_atomic_load(&a.wt[t * a.k + lane], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
            float sh[K3G_KS_SD_MAX];
#pragma unroll
            for (int q = 0; q < K3G_KS_SD_MAX; ++q)
                sh[q] = __uint_as_float(k3d_b32<K3_BPOL>(
                    rs, a.SI > 0 && q < G.KSD ? ((q * a.T + t) * a.d + row) * 4 : K3_OOB));
            float c = 0.0f;
            for (int j0 = 0; j0 < a.k; j0 += 8) {
                float y[8][K3G_KS_D_MAX];
#pragma unroll
                for (int jj = 0; jj < 8; ++jj)
#pragma unroll
                    for (int q = 0; q < K3G_KS_D_MAX; ++q) {
                        const int p = t * a.k + j0 + jj;
                        y[jj][q] = __uint_as_float(k3d_b32<K3_BPOL>(
                            rc, j0 + jj < a.k && q < G.KSDN ? ((p * G.KSDN + q) * a.d + row) * 4
                                                            : K3_OOB));
                    }
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const int j = j0 + jj;
                    if (j >= a.k) break;
                    const int e = __builtin_amdgcn_readlane(ev, j);
                    if (e < 0 || e >= a.E) continue;
                    const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wv), j));
                    float yy = 0.0f;
#pragma unroll
                    for (int q = 0; q < K3G_KS_D_MAX; ++q)
                        if (q < G.KSDN) yy += y[jj][q];
                    c = __fadd_rn(c, __fmul_rn(w, yy));
                }
            }
            if (a.SI > 0) {
                float s2 = 0.0f;
#pragma unroll
                for (int q = 0; q < K3G_KS_SD_MAX; ++q)
                    if (q < G.KSD) s2 += sh[q];
                c = __fadd_rn(c, s2);
            }
            if (lane < 32) put_out(a, (size_t)t * a.d + row, c);
        }
        out_done(a, G, dt, lane);
    }
};

template <int NT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(K3G_DEC_WAVES_PER_EU)))
k_decode_fused(K3kDecode a)
{
    __shared__ K3SelectLds lds;
    __shared__ K3RouterLds rl;
    const int lane = threadIdx.x & 63;
    const K3ArgPtr ap = (K3ArgPtr)__builtin_amdgcn_kernarg_segment_ptr();
    const K3Geo G = k3_geo(a.T, a.d, a.E, a.k, a.I, a.SI, a.L);
    const int W = gridDim.x * (blockDim.x >> 6);
    const int w = k3d_uniform(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
    {
        /* zero this wave's slice of the other counter bank for the next call */
        const int per = (a.sync_words + W - 1) / W;
        const int lo = w * per, hi = min(a.sync_words, lo + per);
        for (int i = lo + lane; i < hi; i += 64) a.sync_clear[i] = 0;
    }
    /* A router row's K3G_KS_R slices are tickets nX + KSR e .. + KSR - 1: when they are
     * the four waves of one workgroup, all taking them in the first round, the slices are
     * reduced in the workgroup's LDS instead of through memory. */
    const bool wg_slices = G.KSR == (int)(blockDim.x >> 6) && G.nX % G.KSR == 0 &&
                           G.nX + G.nR <= W;
    if (threadIdx.x == 0) rl.count = 0;
    __syncthreads();
    for (int tk = w; tk < G.total; tk += W) {
        if (a.trace && lane == 0) {
            const unsigned long long now = wall_clock64();
            a.trace[3 * tk] = now;
            a.trace[3 * tk + 1] = now;
        }
        int t = tk;
        if (t < G.nX) K3Dec<NT>::prep(ap, t, lane);
        else if ((t -= G.nX) < G.nR) K3Dec<NT>::router(ap, t, lane, &rl, wg_slices);
        else if ((t -= G.nR) < 1) K3Dec<NT>::select(ap, lane, &lds);
        else if ((t -= 1) < G.nLD) K3Dec<NT>::latent_down(ap, t, lane);
        else if ((t -= G.nLD) < G.nSG) K3Dec<NT>::shared_gateup(ap, t, lane);
        else if ((t -= G.nSG) < G.nSD) K3Dec<NT>::shared_down(ap, t, lane);
        else if ((t -= G.nSD) < G.nG) K3Dec<NT>::routed_gateup(ap, t, lane);
        else if ((t -= G.nG) < G.nD) K3Dec<NT>::routed_down(ap, t, lane);
        else if ((t -= G.nD) < G.nNR) K3Dec<NT>::norm(ap, t, lane);
        else K3Dec<NT>::latent_up(ap, t - G.nNR, lane);
        if (a.trace && lane == 0) a.trace[3 * tk + 2] = wall_clock64();
    }
}

extern "C" size_t k3k_decode_sync_bytes(int T, int d, int E, int k, int I, int SI, int L)
{
    const K3Geo G = k3_geo(T, d, E, k, I, SI, L);
    return (size_t)G.nlines * SY_LINE * 4;
}

extern "C" int k3k_decode_tickets(int T, int d, int E, int k, int I, int SI, int L)
{
    return k3_geo(T, d, E, k, I, SI, L).total;
}

extern "C" int k3k_decode_fused(const K3kDecode *a, hipStream_t st)
{
    if (a->T < 1 || a->T > 4 || a->d % 32 || a->I % 32 || a->SI % 32 || a->k < 1 ||
        a->k > K3G_MAX_TOPK || a->E < 1 || a->E > K3G_MAX_E || a->T * a->k > 256 ||
        !a->sync || !a->sync_clear ||
        (size_t)a->sync_words * 4 <
            k3k_decode_sync_bytes(a->T, a->d, a->E, a->k, a->I, a->SI, a->L))
        return -1;
    /* the latent layer: both projections, widths the tiles and blocks divide, and every
     * buffer its tickets write */
    if (a->L > 0 && a->L != a->d &&
        (a->L % 32 || !a->down || !a->up || !a->zpart || !a->zq8 || !a->accl || !a->nss ||
         !a->aq16 || !a->upart))
        return -1;
    /* the co-resident grid, per device and token-count instance, found once */
    static int grids[16][5];
    const int NT = a->T <= 1 ? 1 : a->T <= 2 ? 2 : 4;
    const void *fn = NT == 1 ? (const void *)k_decode_fused<1>
                   : NT == 2 ? (const void *)k_decode_fused<2> : (const void *)k_decode_fused<4>;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return -1;
    int *grid = grids[dev];
    if (!grid[NT]) {
        int cus = 0, per = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, fn, 256, 0) != hipSuccess)
            return -1;
        if (per < 1) per = 1;
        /* K3MOE_DECODE_BPC: blocks per CU, at most what fits at once (tuning knob) */
        const char *env = getenv("K3MOE_DECODE_BPC");
        const int want = env ? atoi(env) : 0;
        grid[NT] = cus * (want > 0 && want < per ? want : per);
    }
    if (NT == 1) hipLaunchKernelGGL(k_decode_fused<1>, dim3(grid[1]), dim3(256), 0, st, *a);
    else if (NT == 2) hipLaunchKernelGGL(k_decode_fused<2>, dim3(grid[2]), dim3(256), 0, st, *a);
    else hipLaunchKernelGGL(k_decode_fused<4>, dim3(grid[4]), dim3(256), 0, st, *a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
