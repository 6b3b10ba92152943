/* k3g_dev_host.h - a CPU stand-in for the device primitives k3g_select.h uses, so the
 * selection code compiles with g++ and runs on the host under AddressSanitizer and the
 * array-bounds checker (test infrastructure; never linked into the library).
 *
 * One wave is 64 host threads, one per lane. Every cross-lane operation (shuffle, DPP,
 * readlane, ballot, wave barrier) is a rendezvous of all 64 threads: each lane posts its
 * value, all meet at a barrier, each reads what it needs, all meet again. The selection
 * code only issues cross-lane operations under wave-uniform control flow, which is what
 * makes the rendezvous well defined (a divergent one would deadlock, and the audit's
 * per-case time limit would report it).
 *
 * Buffer loads keep the hardware's range check: a raw buffer load at or past the
 * descriptor's size returns zero without touching memory. The audit also counts loads
 * that the range check stopped, so the driver can tell a deliberate out-of-range read
 * (lanes past n_experts) from an accidental one.
 *
 * The test copies this file next to a copy of k3g_select.h as "k3g_dev.h". */
#pragma once

#include "k3g_expf.h"

#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>

#define K3G_WAVE 64
#define __device__
#define __forceinline__ inline __attribute__((always_inline))
#define __noinline__ __attribute__((noinline))

#include <sched.h>

struct float4 { float x, y, z, w; };
struct float2 { float x, y; };
struct double2 { double x, y; };
inline float4 make_float4(float a, float b, float c, float d) { return float4{a, b, c, d}; }

inline float __uint_as_float(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t __float_as_uint(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float __fadd_rn(float a, float b) { volatile float r = a + b; return r; }
inline float __fmul_rn(float a, float b) { volatile float r = a * b; return r; }
inline float __fdiv_rn(float a, float b) { volatile float r = a / b; return r; }
inline int __popcll(unsigned long long v) { return __builtin_popcountll(v); }
inline int min(int a, int b) { return a < b ? a : b; }
inline unsigned long long wall_clock64() { return 0; }

/* ----------------------------------------------------------------- the wave ---- */
/* A sense-reversing barrier for the 64 lane threads that spins with yields (a futex per
 * rendezvous makes the audit tens of times slower with 64 threads on a few cores). */
struct EmuBarrier {
    std::atomic<int> count{0};
    std::atomic<int> sense{0};
    void arrive_and_wait()
    {
        const int s = sense.load(std::memory_order_relaxed);
        if (count.fetch_add(1, std::memory_order_acq_rel) == 63) {
            count.store(0, std::memory_order_relaxed);
            sense.store(s ^ 1, std::memory_order_release);
        } else {
            while (sense.load(std::memory_order_acquire) == s) sched_yield();
        }
    }
};

struct EmuWave {
    EmuBarrier bar;
    uint64_t slot[64];
    void *lds_base = nullptr;        /* host memory standing in for the LDS window */
    std::atomic<long> oob_loads{0};  /* buffer loads the range check stopped */
    std::atomic<long> dma_ops{0};
};
extern EmuWave *g_wave;
extern thread_local int t_lane;

inline uint64_t emu_exchange(uint64_t mine, int from)
{
    g_wave->slot[t_lane] = mine;
    g_wave->bar.arrive_and_wait();
    const uint64_t v = g_wave->slot[from];
    g_wave->bar.arrive_and_wait();
    return v;
}

template <typename T>
inline T emu_shfl_xor(T v, int m)
{
    uint64_t u = 0;
    std::memcpy(&u, &v, sizeof(T));
    const uint64_t o = emu_exchange(u, t_lane ^ m);
    T r;
    std::memcpy(&r, &o, sizeof(T));
    return r;
}
#define __shfl_xor(v, m, w) emu_shfl_xor(v, m)

/* lane l takes lane l - m (lanes below m keep their own value), and any lane's value */
template <typename T>
inline T emu_shfl_from(T v, int from)
{
    uint64_t u = 0;
    std::memcpy(&u, &v, sizeof(T));
    const uint64_t o = emu_exchange(u, from);
    T r;
    std::memcpy(&r, &o, sizeof(T));
    return r;
}
#define __shfl_up(v, m, w) emu_shfl_from(v, t_lane >= (m) ? t_lane - (m) : t_lane)
#define __shfl(v, l, w) emu_shfl_from(v, (l))

inline uint32_t emu_readlane(uint32_t v, int l) { return (uint32_t)emu_exchange(v, l); }
#define __builtin_amdgcn_readlane(v, l) emu_readlane((uint32_t)(v), (l))
/* every lane of the selection code is active wherever it reads the first lane */
#define __builtin_amdgcn_readfirstlane(v) emu_readlane((uint32_t)(v), 0)

inline unsigned long long emu_ballot(bool p)
{
    g_wave->slot[t_lane] = p ? 1 : 0;
    g_wave->bar.arrive_and_wait();
    unsigned long long m = 0;
    for (int l = 0; l < 64; ++l) m |= (unsigned long long)(g_wave->slot[l] & 1) << l;
    g_wave->bar.arrive_and_wait();
    return m;
}
#define __ballot(p) emu_ballot(p)

/* DPP with bound_ctrl off and bank_mask 0xf: row_shr:n (lane i of a 16-lane row takes lane
 * i - n of its row, lanes i < n keep `old`), row_bcast:15 (rows 1..3 take lane 15 of the
 * row below) and row_bcast:31 (rows 2, 3 take lane 31); rows outside row_mask keep `old`. */
inline int emu_update_dpp(int old, int src, int ctrl, int row_mask)
{
    g_wave->slot[t_lane] = (uint32_t)src;
    g_wave->bar.arrive_and_wait();
    const int row = t_lane >> 4, i = t_lane & 15;
    int r = old;
    if ((row_mask >> row) & 1) {
        if (ctrl >= 0x111 && ctrl <= 0x11f) {
            const int n = ctrl - 0x110;
            if (i >= n) r = (int)(uint32_t)g_wave->slot[t_lane - n];
        } else if (ctrl == 0x142) {
            if (row >= 1) r = (int)(uint32_t)g_wave->slot[16 * row - 1];
        } else if (ctrl == 0x143) {
            if (row >= 2) r = (int)(uint32_t)g_wave->slot[31];
        } else {
            std::abort();            /* a DPP control this stand-in does not model */
        }
    }
    g_wave->bar.arrive_and_wait();
    return r;
}
#define __builtin_amdgcn_update_dpp(old, src, ctrl, rm, bm, bc) emu_update_dpp(old, src, ctrl, rm)

inline void emu_wave_barrier() { g_wave->bar.arrive_and_wait(); }
#define __builtin_amdgcn_wave_barrier() emu_wave_barrier()
#define __builtin_amdgcn_fence(order, scope) std::atomic_thread_fence(std::memory_order_seq_cst)
#define __builtin_amdgcn_s_waitcnt(n) ((void)0)

/* stores other waves read at device coherence: plain stores here (one wave) */
#define __HIP_MEMORY_SCOPE_AGENT 0
#define __hip_atomic_store(p, v, order, scope) (*(p) = (v))
#define __hip_atomic_load(p, order, scope) (*(p))
inline int atomicAdd(int *p, int v)
{
    return std::atomic_ref<int>(*p).fetch_add(v);
}

/* ------------------------------------------------------- buffer descriptors ---- */
struct __amdgpu_buffer_rsrc_t { const char *base; int bytes; };
struct emu_u4 { uint32_t x, y, z, w; };
inline __amdgpu_buffer_rsrc_t __builtin_amdgcn_make_buffer_rsrc(void *p, short, int n, int)
{
    return __amdgpu_buffer_rsrc_t{(const char *)p, n};
}
inline emu_u4 __builtin_amdgcn_raw_buffer_load_b128(__amdgpu_buffer_rsrc_t r, int off, int soff,
                                                    int)
{
    emu_u4 v{0, 0, 0, 0};
    const long o = (long)off + soff;
    if (o < 0 || o + 16 > r.bytes) {
        g_wave->oob_loads++;
        return v;
    }
    std::memcpy(&v, r.base + o, 16);
    return v;
}

/* ------------------------------------------------------------------ helpers ---- */
inline float k3d_expf(float v) { return k3x_expf(v); }
inline float k3d_sigmoid(float v) { return __fdiv_rn(1.0f, __fadd_rn(1.0f, k3d_expf(-v))); }

inline double k3d_wave_sumd(double v)
{
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, K3G_WAVE);
    return v;
}

/* the device's hardware exponential stands in as the host's float exp */
inline float __expf(float v) { return std::exp(v); }

/* Transposed wave reduction of V partial sums per lane (the device helper's halving
 * rounds): lane l ends with the 64-lane sum of value index l >> (6 - log2 V) in v[0]. */
template <int V, typename A>
inline void k3d_transpose_reduce(A *v, int lane)
{
    int n = V;
    for (int m = 32; m >= 1; m >>= 1) {
        if (n > 1) {
            const int h = n >> 1;
            const bool upper = (lane & m) != 0;
            for (int i = 0; i < V / 2; ++i) {
                if (i < h) {
                    const A send = upper ? v[i] : v[i + h];
                    const A keep = upper ? v[i + h] : v[i];
                    v[i] = keep + __shfl_xor(send, m, K3G_WAVE);
                }
            }
            n = h;
        } else {
            v[0] += __shfl_xor(v[0], m, K3G_WAVE);
        }
    }
}

/* global_load_lds_dwordx4: lane l's 16 bytes land at LDS byte address lds + 16 l; the
 * address is the low 32 bits of a pointer into the host block standing in for the LDS */
inline void k3d_dma16(const void *src, uint32_t lds)
{
    const uint32_t base = (uint32_t)(uintptr_t)g_wave->lds_base;
    char *dst = (char *)g_wave->lds_base + (uint32_t)(lds - base) + 16 * t_lane;
    std::memcpy(dst, src, 16);
    g_wave->dma_ops++;
    emu_wave_barrier();              /* the instruction is issued by the whole wave */
}
inline void k3d_wait_vm(int) {}
