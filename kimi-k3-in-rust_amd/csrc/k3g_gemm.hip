/* k3g_gemm.hip - the expert products for many tokens (prefill, batched decode) as grouped
 * GEMMs on the bf16 matrix cores (v_mfma_f32_16x16x32_bf16, fp32 accumulation).
 *
 * The engine computes, per (token, slot) pair, three MXFP4 GEMVs per expert in its
 * moe_prefill_chunk loop (src/core/k3_ops.c:668-808); here the pairs are grouped by
 * expert (the stable counting sort of k3g_misc.hip) and each expert's pairs form the
 * columns of one GEMM against that expert's weights:
 *
 *   gate/up  (mode 0):  G = W1 X, U = W3 X  -> h = act(G, U)   (K = hidden)
 *   down     (mode 1):  Y = W2 h            -> contrib rows    (K = inter)
 *
 * The shared expert is the same GEMM over all tokens with a dense column list.
 *
 * Work unit: one workgroup = one (column tile of up to 128 pairs, feature tile) of one
 * expert. Wave w owns 4 row groups of 16 weight rows (mode 0: 32 gate rows and the 32 up
 * rows of the same features, so the activation is lane-local; mode 1: 64 output rows)
 * and all the tile's columns: 4 x 8 accumulators of 16x16. Gate/up with one-piece
 * activations runs 4-wave workgroups (128 features), two per CU, so that one
 * workgroup's matrix work covers the other's barrier and load waits; two-piece
 * activations and the down GEMM run 8-wave workgroups (256 features / 512 rows), one per
 * CU (their stages need 128 KB of LDS).
 *
 * Weights (A operand) go from HBM straight to registers in the tiled layouts of
 * k3g_tile.hip: one 16-byte load per lane and row group gives a 16-row x 128-column block
 * of MXFP4, which v_cvt_scalef32_pk_bf16_fp4 turns into four exact bf16 A operands (FP4
 * times a power-of-two scale is a 3-bit significand: bf16 holds it exactly). Tiled bf16
 * weights (the shared expert) load as A operands directly.
 *
 * Activations (B operand) are bf16 PIECES: x (or h) = piece0 + piece1 with piece0 =
 * bf16(v) and piece1 = bf16(v - piece0), 16 significant bits, so the products see the
 * activations to 2^-17 relative. A single bf16 piece of h would cost ~1.7e-3 rel-L2 on
 * the layer output; two cost ~2e-6. When every x is already a bf16 value (piece1 = 0
 * everywhere, recorded in a flag) the gate/up GEMMs skip piece 1: the result is the
 * same. The column tile's activations are staged in LDS, 128 columns x 128 K per piece
 * per stage, two stages, written by global_load_lds_dwordx4 (no register round trip) in a
 * row-XOR-swizzled layout that the B-operand reads (ds_read_b128) hit without bank
 * conflicts. K advances 128 per step: one barrier per step, the next step's weights and
 * activations in flight during the current step's matrix work.
 *
 * Workgroup order: column tiles are sorted largest first (an expert's full tiles next to
 * each other) and dealt to the 8 XCDs in groups of K3G_TILE_GROUP consecutive tiles, the
 * groups in a snake, so every XCD gets the same amount of work and runs its largest tiles
 * first (the contiguous alternative left the busiest XCD ~10% behind on the Zipf-skewed
 * prefill), and a hot expert's tiles run at once on one XCD, sharing its weights in that
 * XCD's L2; the feature tiles of one column tile run back to back on one XCD and share
 * the tile's activations there.
 */
#include "k3g_dev.h"
#include "k3g_kernels.h"

typedef float k3v4f __attribute__((ext_vector_type(4)));
typedef __bf16 k3v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 k3v2bf __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void *k3lds;

#define GM_WAVES 8
#define GM_COLS 128                       /* pair columns per tile */
#define GM_KC 128                         /* K per step */
#define GM_PIECE (GM_COLS * GM_KC * 2)    /* bytes of one piece of one stage: 32 KB */
#define GM_STAGE (2 * GM_PIECE)
#define GM_QT 4352                        /* tiled MXFP4 quad tile */

__device__ __forceinline__ int gm_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

/* E8M0 byte -> 2^(b-127) as fp32 without branches (the tiled layout holds no 255) */
__device__ __forceinline__ float gm_scale(uint32_t b)
{
    return __uint_as_float(b ? b << 23 : 0x00400000u);
}

/* 8 E2M1 values (one 32-bit word, low nibble first) times 2^(s-127) as bf16, exact */
__device__ __forceinline__ k3v8bf gm_deq8(uint32_t w, float scale)
{
    const k3v2bf a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0);
    const k3v2bf b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1);
    const k3v2bf c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2);
    const k3v2bf d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3);
    return k3v8bf{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

__device__ __forceinline__ k3v4f gm_mma(k3v8bf a, uint4 b, k3v4f acc)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(k3v8bf, b), acc, 0, 0, 0);
}

__device__ __forceinline__ uint16_t gm_bf16_rn(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float gm_bf16_f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

/* Loads through pointers the compiler cannot prove global (they come from the expert
 * table) would be flat loads, which also count against the LDS counter and make every
 * ds_read wait for outstanding HBM loads: address them as global memory explicitly. */
typedef unsigned int gm_v4u __attribute__((ext_vector_type(4)));
#ifdef __HIP_DEVICE_COMPILE__
typedef const __attribute__((address_space(1))) gm_v4u *gm_g4;
typedef const __attribute__((address_space(1))) uint32_t *gm_g1;
#else
typedef const gm_v4u *gm_g4;       /* the host pass only parses device code */
typedef const uint32_t *gm_g1;
#endif

__device__ __forceinline__ uint4 gm_ld16(const void *p)
{
    const gm_v4u v = *(gm_g4)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t gm_ld4(const void *p) { return *(gm_g1)p; }

/* h = act(gate, up) for 4 consecutive features of one column, stored as two bf16 pieces
 * (piece 1 at o + piece) */
__device__ __noinline__ void gm_act_store(k3v4f gt, k3v4f up, float b1, float b2, uint16_t *o,
                                          long long piece)
{
    uint16_t hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float y = k3d_act(gt[i], up[i], b1, b2);
        hi[i] = gm_bf16_rn(y);
        lo[i] = gm_bf16_rn(y - gm_bf16_f(hi[i]));
    }
    uint2 vh, vl;
    vh.x = hi[0] | ((uint32_t)hi[1] << 16); vh.y = hi[2] | ((uint32_t)hi[3] << 16);
    vl.x = lo[0] | ((uint32_t)lo[1] << 16); vl.y = lo[2] | ((uint32_t)lo[3] << 16);
    *(uint2 *)o = vh;
    *(uint2 *)(o + piece) = vl;
}

/* One DMA instruction: 64 lanes x 16 bytes from their own global addresses to 1 KB of LDS
 * at byte address `lds` (lane l at lds + 16 l). Issued as inline assembly so the
 * compiler does not treat every later LDS read as waiting on it (it would drain all
 * outstanding loads before each ds_read); completion is awaited explicitly with
 * s_waitcnt vmcnt before the barrier that publishes the stage. M0 is saved and restored
 * around the instruction. */
__device__ __forceinline__ void gm_dma16(const void *src, uint32_t lds)
{
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %2\n\t"
                 "global_load_lds_dwordx4 %1, off\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(keep) : "v"(src), "s"(lds) : "memory");
}

/* The same DMA with a wave-uniform base in scalar registers and this lane's 32-bit byte
 * offset in one vector register: no per-lane 64-bit address to build or keep. */
__device__ __forceinline__ void gm_dma16s(const void *sbase, uint32_t voff, uint32_t lds)
{
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %3\n\t"
                 "global_load_lds_dwordx4 %1, %2\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(keep) : "v"(voff), "s"(sbase), "s"(lds) : "memory");
}

__device__ __forceinline__ void gm_dma4s(const void *sbase, uint32_t voff, uint32_t lds)
{
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %3\n\t"
                 "global_load_lds_dword %1, %2\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(keep) : "v"(voff), "s"(sbase), "s"(lds) : "memory");
}

/* a wave-uniform pointer, in scalar registers */
template <typename P>
__device__ __forceinline__ P *gm_uniform_ptr(P *p)
{
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (P *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

/* raw buffer descriptor over `bytes` at p (p wave-uniform): loads take a scalar offset
 * and this lane's vector offset */
typedef __amdgpu_buffer_rsrc_t gm_rsrc;
__device__ __forceinline__ gm_rsrc gm_make_rsrc(const void *p, size_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0,
                                             (int)(bytes < 0x7fffffffu ? bytes : 0x7fffffffu),
                                             0x00020000);
}

/* s_waitcnt vmcnt(N) (expcnt, lgkmcnt not waited on) */
template <int N>
__device__ __forceinline__ void gm_wait_vm()
{
    static_assert(N >= 0 && N < 16, "vmcnt");
    __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

/* s_waitcnt vmcnt(n) for a wave-uniform n in 8..16 */
__device__ __forceinline__ void gm_wait_vm_n(int n)
{
    switch (n) {
        case 8: gm_wait_vm<8>(); break;
        case 9: gm_wait_vm<9>(); break;
        case 10: gm_wait_vm<10>(); break;
        case 11: gm_wait_vm<11>(); break;
        case 12: gm_wait_vm<12>(); break;
        case 13: gm_wait_vm<13>(); break;
        case 14: gm_wait_vm<14>(); break;
        case 15: gm_wait_vm<15>(); break;
        default: gm_wait_vm<8>(); break;
    }
}

/* ============================================================ scaled FP8 MFMA ====== */
/* Used by the FP4 x FP8 variant and by the remainder piece of h in the bf16 path.
 * v_mfma_scale_f32_16x16x128_f8f6f4 with cbsz 4 (A: FP4) and blgp 0 (B: FP8 E4M3), each
 * 32-column block carrying its E8M0 scale. One instruction covers a whole 128-column
 * step: the tiled MXFP4 chunk is its A operand unchanged (lane L: row L % 16, block
 * L / 16), and lane 16 q + c of B holds column c's bytes 16 q .. + 15 and 64 + 16 q .. + 15
 * of the step, with lane 16 g + c giving column c's scale of block g.
 * LDS per stage: 128 columns x 128 bytes, the 16-byte units stored so each lane's two
 * units are one logical pair (logical slot 2 q: unit q, 2 q + 1: unit 4 + q), physical
 * slot = logical ^ ((row / 2) % 8) (conflict-free: 16 lanes of one unit index cover 16
 * distinct bank groups); then 128 x 4 scale bytes. */
#define GM_F8_DATA (GM_COLS * GM_KC)
#define GM_F8_STAGE (GM_F8_DATA + GM_COLS * 4)

__device__ __forceinline__ void gm_dma4(const void *src, uint32_t lds)
{
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %2\n\t"
                 "global_load_lds_dword %1, off\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(keep) : "v"(src), "s"(lds) : "memory");
}

typedef int gm_v8i __attribute__((ext_vector_type(8)));

__device__ __forceinline__ k3v4f gm_mma_f8(uint4 a, uint32_t sa, const gm_v8i &b, uint32_t sb,
                                           k3v4f acc)
{
    const gm_v8i av = {(int)a.x, (int)a.y, (int)a.z, (int)a.w, 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, b, acc, 4, 0, 0, (int)sa, 0,
                                                            (int)sb);
}

/* E8M0 exponent (2^sx) and E4M3 bytes of four values x 2^-sx, nearest-even, clamped to
 * +-448 first (the OCP MX conversion) */
__device__ __forceinline__ int gm_mx_exp(float amax)
{
    if (!(amax > 0.0f)) return -127;
    int e;
    frexpf(amax, &e);
    const int sx = e - 1 - 8;
    return sx < -127 ? -127 : (sx > 127 ? 127 : sx);
}

__device__ __forceinline__ uint32_t gm_e4m3x4(float a, float b, float c, float d, int sx)
{
    const float k = ldexpf(1.0f, -sx);
    a = fminf(fmaxf(a * k, -448.0f), 448.0f);
    b = fminf(fmaxf(b * k, -448.0f), 448.0f);
    c = fminf(fmaxf(c * k, -448.0f), 448.0f);
    d = fminf(fmaxf(d * k, -448.0f), 448.0f);
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
}

/* h = act(gate, up) for the wave's 32 features of one column (this lane's features
 * 4 g + i and 16 + 4 g + i, g = g4): bf16(h) at o (piece 0, bf16 row at o) and the
 * remainder h - bf16(h) as one MX block: E4M3 bytes at oq, E8M0 scale at *os. The block
 * exponent puts the largest remainder in [128, 256), under E4M3's 448, so nothing clamps;
 * the remainder keeps 4 significant bits, h about 12. */
__device__ __noinline__ void gm_act_store_mix(k3v4f g0, k3v4f g1, k3v4f u0, k3v4f u1, float b1,
                                              float b2, uint16_t *o, uint8_t *oq, uint8_t *os,
                                              int g4)
{
    uint16_t hi[8];
    float rr[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float y0 = k3d_act(g0[i], u0[i], b1, b2), y1 = k3d_act(g1[i], u1[i], b1, b2);
        hi[i] = gm_bf16_rn(y0);
        hi[4 + i] = gm_bf16_rn(y1);
        rr[i] = y0 - gm_bf16_f(hi[i]);
        rr[4 + i] = y1 - gm_bf16_f(hi[4 + i]);
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(rr[i]));
    m = fmaxf(m, __shfl_xor(m, 16, K3G_WAVE));
    m = fmaxf(m, __shfl_xor(m, 32, K3G_WAVE));
    int sx = -127;
    if (m > 0.0f) {
        int e;
        frexpf(m, &e);
        sx = e - 8 < -127 ? -127 : (e - 8 > 127 ? 127 : e - 8);
    }
    uint2 v0, v1;
    v0.x = hi[0] | ((uint32_t)hi[1] << 16); v0.y = hi[2] | ((uint32_t)hi[3] << 16);
    v1.x = hi[4] | ((uint32_t)hi[5] << 16); v1.y = hi[6] | ((uint32_t)hi[7] << 16);
    *(uint2 *)(o + 4 * g4) = v0;
    *(uint2 *)(o + 16 + 4 * g4) = v1;
    *(uint32_t *)(oq + 4 * g4) = gm_e4m3x4(rr[0], rr[1], rr[2], rr[3], sx);
    *(uint32_t *)(oq + 16 + 4 * g4) = gm_e4m3x4(rr[4], rr[5], rr[6], rr[7], sx);
    if (g4 == 0) *os = (uint8_t)(sx + 127);
}

/* Instruction order of one step's matrix work (NR B-operand reads from LDS, 4 MFMAs
 * each): the reads run two ahead of the MFMAs that use them, and the conversions of the
 * next sub-step's weights fill the issue slots between MFMAs, so neither an LDS round
 * trip nor a run of conversions sits between two MFMAs. */
template <int NR, int GM_AHEAD>
__device__ __forceinline__ void gm_pipeline()
{
    __builtin_amdgcn_sched_group_barrier(0x100, GM_AHEAD, 0);   /* DS read */
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);      /* MFMA */
        if (i + GM_AHEAD < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
}

/* Everything one workgroup's tile needs, uniform across the workgroup except the
 * per-lane DMA row offsets. */
struct GmTile {
    int p0, np, lane, w, g4, nK, ndma;
    int ks, kstep0, nC32;      /* K slice: its index, first 128-column step, 32-chunks */
    int orow0;                 /* mode 0: first feature; mode 1: first output row */
    const uint8_t *abase[4];   /* row group r: its 16-row block of the weight matrix */
    bool rv[4];                /* row group inside the matrix */
    uint32_t boff[8];          /* element offsets of this lane's DMA rows (+ swizzled slot) */
    uint32_t lds;              /* LDS byte address of the staging buffers */
    uint8_t *ldsp;
    uint32_t rbb;              /* bytes of one 16-row block of the weight matrix */
};

/* The tile's GEMM with NB 16-column blocks and NP activation pieces in a workgroup of WV
 * waves, then its epilogue. */
template <int AF, int NP, int NB, int WV>
__device__ __forceinline__ void gm_tile(const K3kGemm &g, const GmTile &t)
{
    k3v4f acc[4][NB];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) acc[r][cb] = k3v4f{0.f, 0.f, 0.f, 0.f};
    const int lane = t.lane;

    /* stages: 8 waves: three of one piece (activations two steps ahead) or two of two
     * pieces; 4 waves (two workgroups per CU): two of one piece */
    constexpr int SN = (NP == 1 && WV == 8) ? 3 : 2;
    constexpr int NI = 32 / WV;                  /* DMA instructions per wave and piece */
    auto stage = [](int c) { return (uint32_t)((c % SN) * (NP * GM_PIECE)); };
    auto dma = [&](int c) {
        const uint32_t st = t.lds + stage(c) + t.w * 1024;
        const uint16_t *b0 = g.b + (size_t)(t.kstep0 + c) * GM_KC;
#pragma unroll
        for (int pc = 0; pc < NP; ++pc) {
            const uint16_t *b = b0 + (size_t)pc * g.bpiece;
#pragma unroll
            for (int i = 0; i < NI; ++i)
                if (i < t.ndma) gm_dma16(b + t.boff[i], st + pc * GM_PIECE + i * WV * 1024);
        }
    };
    /* B operand: column block cb, logical 16-byte slot q of the step's row */
    const uint8_t *brow = t.ldsp + (lane & 15) * 256;
    auto bread = [&](int c, int pc, int cb, int q) -> uint4 {
        return *(const uint4 *)(brow + stage(c) + pc * GM_PIECE + cb * 16 * 256 +
                                16 * (q ^ (lane & 15)));
    };
    auto mma_step = [&](int c, int q, const k3v8bf *a) {
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) {
#pragma unroll
            for (int pc = 0; pc < NP; ++pc) {
                const uint4 bv = bread(c, pc, cb, q);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[r][cb] = gm_mma(a[r], bv, acc[r][cb]);
            }
        }
    };
    const uint4 z4 = make_uint4(0, 0, 0, 0);

    if (AF == 0) {
        /* ------------------------------------------------ MXFP4 weights ---------- */
        /* step c's weights are loaded two steps ahead (8 loads per step: 4 row groups'
         * 16 data bytes and their scale dwords); the activations one step ahead. Issue
         * order per step: DMA(c + 1), then weights(c + 2), so "all but the last 8 loads
         * done" means step c + 1's stage and weights have landed. */
        uint4 ab[3][4];
        uint32_t sb[3][4];
        auto aload = [&](int c, uint4 (&dst)[4], uint32_t (&sdst)[4]) {
            const size_t qo = (size_t)(c >> 2) * GM_QT;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint8_t *p = t.abase[r] + qo;
                dst[r] = gm_ld16(p + 1024 * (c & 3) + 16 * lane);
                sdst[r] = gm_ld4(p + 4096 + 4 * lane);
            }
        };
        /* One step: weights of step c in cur, weights of step c + 2 loaded into nxt. The
         * buffers rotate by unrolling (never by register moves, which would wait for the
         * loads in flight), and every step issues the same loads (clamped to the last step;
         * the padding steps past nK only skip their matrix work), so the compiler's load
         * counters agree on every path and its waits stay on the step that is due. */
        /* loads after the ones step c needs: SN == 3: DMA(c + 1) then weights(c + 1);
         * SN == 2: weights(c + 1) only (DMA(c) came after them) */
        const int after = SN == 3 ? 8 + NP * t.ndma : 8;
        auto step = [&](int c, const uint4 (&cur)[4], const uint32_t (&scl)[4], uint4 (&nxt)[4],
                        uint32_t (&nsc)[4]) {
            gm_wait_vm_n(after);
            __syncthreads();
            dma(min(c + SN - 1, t.nK - 1));
            aload(min(c + 2, t.nK - 1), nxt, nsc);
            __builtin_amdgcn_sched_barrier(0);
            if (c < t.nK) {
                /* rows outside the matrix read row block 0 and are never stored */
                const int j = c & 3;
                float sc[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) sc[r] = gm_scale((scl[r] >> (8 * j)) & 0xffu);
                const uint4 (&wv)[4] = cur;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    k3v8bf a[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint32_t wd = s == 0 ? wv[r].x : s == 1 ? wv[r].y
                                          : s == 2 ? wv[r].z : wv[r].w;
                        a[r] = gm_deq8(wd, sc[r]);
                    }
                    mma_step(c, 4 * s + t.g4, a);
                }
                gm_pipeline<4 * NB * NP, 3>();
            }
        };
        aload(0, ab[0], sb[0]);
        dma(0);
        aload(min(1, t.nK - 1), ab[1], sb[1]);
        if (SN == 3) dma(min(1, t.nK - 1));
        for (int c = 0; c < t.nK; c += 3) {
            step(c, ab[0], sb[0], ab[2], sb[2]);
            step(c + 1, ab[1], sb[1], ab[0], sb[0]);
            step(c + 2, ab[2], sb[2], ab[1], sb[1]);
        }
        gm_wait_vm<0>();
    } else {
        /* ------------------------------------------------ bf16 weights ----------- */
        /* A operands per (step, sub-step): 4 row groups x 16 bytes; a ring of the 4
         * sub-steps of a step, each loaded two sub-steps ahead */
        const int nC32 = t.nC32;
        uint4 ring[4][4];
        auto aload = [&](int c, int s, uint4 *dst) {
            const int c32 = 4 * c + s;
            const int cc = 4 * t.kstep0 + (c32 < nC32 ? c32 : nC32 - 1);
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[r] = gm_ld16(t.abase[r] + (size_t)cc * 1024 + 16 * lane);
        };
        dma(0);
        aload(0, 0, ring[0]);
        aload(0, 1, ring[1]);
        for (int c = 0; c < t.nK; ++c) {
            /* the stage's DMA was followed by the loads of sub-steps (c, 0) and (c, 1) */
            gm_wait_vm<8>();
            __syncthreads();
            if (c + 1 < t.nK) dma(c + 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int s2 = (s + 2) & 3;
                aload(c + ((s + 2) >> 2), s2, ring[s2]);
                __builtin_amdgcn_sched_barrier(0);
                /* rows outside the matrix and columns past K multiply as zeros */
                const bool kin = 4 * c + s < nC32;
                k3v8bf a[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    a[r] = __builtin_bit_cast(k3v8bf, (t.rv[r] && kin) ? ring[s][r] : z4);
                mma_step(c, 4 * s + t.g4, a);
            }
        }
        gm_wait_vm<0>();
    }

    /* ---- epilogue -------------------------------------------------------------------- */
    const int col0 = lane & 15;
    if (g.ksplit > 1) {
        /* a K slice: its fp32 sums, reduced in slice order by k_gemm_reduce */
        const int R = g.rows, ncol = g.dense_rows;
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) {
            const int col = 16 * cb + col0;
            if (col < t.np) {
                const size_t cix = (size_t)t.ks * ncol + t.p0 + col;
                if (g.mode == 0) {
                    if (!t.rv[0]) continue;
                    float *o = g.part + cix * 2 * R + t.orow0 + 4 * t.g4;
                    *(k3v4f *)o = acc[0][cb];
                    *(k3v4f *)(o + 16) = acc[1][cb];
                    *(k3v4f *)(o + R) = acc[2][cb];
                    *(k3v4f *)(o + R + 16) = acc[3][cb];
                } else {
                    float *o = g.part + cix * R + t.orow0 + 4 * t.g4;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (t.rv[r]) *(k3v4f *)(o + 16 * r) = acc[r][cb];
                }
            }
        }
        return;
    }
    if (g.mode == 0) {
        if (!t.rv[0]) return;
        const int n = t.orow0 + 4 * t.g4;
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) {
            const int col = 16 * cb + col0;
            if (col < t.np) {
                const size_t row = (size_t)(t.p0 + col);
                if (AF == 0 && g.hmix) {
                    gm_act_store_mix(acc[0][cb], acc[1][cb], acc[2][cb], acc[3][cb], g.b1, g.b2,
                                     g.h + row * g.ldh + t.orow0, g.hq + row * g.ldhq + t.orow0,
                                     g.hs + row * (g.ldhq / 32) + t.orow0 / 32, t.g4);
                } else {
                    uint16_t *o = g.h + row * g.ldh + n;
                    gm_act_store(acc[0][cb], acc[2][cb], g.b1, g.b2, o, g.hpiece);
                    gm_act_store(acc[1][cb], acc[3][cb], g.b1, g.b2, o + 16, g.hpiece);
                }
            }
        }
    } else {
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) {
            const int col = 16 * cb + col0;
            if (col < t.np) {
                const int p = t.p0 + col;
                float *o = g.out + (size_t)(g.scatter ? g.perm[p] : p) * g.ldo + t.orow0 + 4 * t.g4;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (t.rv[r]) *(k3v4f *)(o + 16 * r) = acc[r][cb];
            }
        }
    }
}

/* Instruction order of one step of the down GEMM's matrix work: NB FP8 groups (the
 * remainder: 3 LDS reads, 4 scaled MFMAs each), then 4 NB bf16 groups (piece 0: 1 LDS
 * read, 4 MFMAs each), the reads AH groups ahead of the MFMAs that use them. */
template <int NB, int AH>
__device__ __forceinline__ void gm_pipeline_mix()
{
    constexpr int NG = 5 * NB;
    constexpr int PRO = AH <= NB ? 3 * AH : 3 * NB + (AH - NB);
    __builtin_amdgcn_sched_group_barrier(0x100, PRO, 0);     /* DS read */
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);   /* MFMA */
        if (j + AH < NB) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
        else if (j + AH < NG) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
}

/* The down GEMM of MXFP4 experts with h as bf16 piece 0 (bf16 matrix cores, as gm_tile)
 * plus its MX remainder (scaled FP8 matrix cores, one 16x16x128 instruction per step
 * on the same weight registers, at twice the bf16 rate): three quarters of the matrix
 * time of two bf16 pieces. Stage c % 2: piece 0 (GM_PIECE, gm_tile's layout), then the
 * remainder's bytes and scales (GM_F8_STAGE, k_gemm_f8's layout). The weight and DMA
 * pipeline is gm_tile's with two stages: a step waits for all but the 8 weight loads
 * issued after its stage's DMA.
 *
 * The tile's B rows are sorted positions p0 .. p0 + 127, contiguous: every DMA takes a
 * uniform base in scalar registers (the tile's first row, advanced per step) and a
 * loop-invariant byte offset per lane (bofb: piece 0, doff: remainder bytes, soff:
 * remainder scales, all relative to row p0); the weights load through one buffer
 * descriptor per row group with the step in the scalar offset. No per-lane 64-bit
 * address is kept, which leaves the registers for the LDS read-ahead. */
template <int NB>
__device__ __forceinline__ void gm_tile_mix(const K3kGemm &g, const GmTile &t,
                                            const uint32_t (&bofb)[4], const uint32_t (&doff)[2],
                                            uint32_t soff, int nd, int ns)
{
    k3v4f acc[4][NB];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) acc[r][cb] = k3v4f{0.f, 0.f, 0.f, 0.f};
    const int lane = t.lane;
    constexpr uint32_t ST = GM_PIECE + GM_F8_STAGE;
    const uint8_t *b0 = gm_uniform_ptr((const uint8_t *)(g.b + (size_t)t.p0 * g.ldb));
    const uint8_t *q0 = gm_uniform_ptr(g.bq + (size_t)t.p0 * g.ldhq);
    const uint8_t *s0 = gm_uniform_ptr(g.bs + (size_t)t.p0 * (g.ldhq / 32));
    auto dma = [&](int c) {
        const uint32_t st = t.lds + (c & 1) * ST;
        const uint8_t *b = b0 + (size_t)c * (2 * GM_KC);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < t.ndma) gm_dma16s(b, bofb[i], st + t.w * 1024 + i * 8 * 1024);
        const uint8_t *q = q0 + (size_t)c * GM_KC;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            if (i < nd) gm_dma16s(q, doff[i], st + GM_PIECE + (8 * i + t.w) * 1024);
        if (t.w < ns) gm_dma4s(s0 + 4 * c, soff, st + GM_PIECE + GM_F8_DATA + t.w * 256);
    };
    const uint8_t *brow = t.ldsp + (lane & 15) * 256;
    const int q4 = lane >> 4, c0 = lane & 15;
    gm_rsrc ar[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ar[r] = gm_make_rsrc(t.abase[r], t.rbb);
    const int v16 = 16 * lane, v4 = 4 * lane;
    uint4 ab[3][4];
    uint32_t sbuf[3][4];
    auto aload = [&](int c, uint4 (&dst)[4], uint32_t (&sdst)[4]) {
        const int so = (c >> 2) * GM_QT;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            dst[r] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(ar[r], v16, so + 1024 * (c & 3), 0));
            sdst[r] = __builtin_amdgcn_raw_buffer_load_b32(ar[r], v4, so + 4096, 0);
        }
    };
    auto step = [&](int c, const uint4 (&cur)[4], const uint32_t (&scl)[4], uint4 (&nxt)[4],
                    uint32_t (&nsc)[4]) {
        gm_wait_vm<8>();
        __syncthreads();
        dma(min(c + 1, t.nK - 1));
        aload(min(c + 2, t.nK - 1), nxt, nsc);
        __builtin_amdgcn_sched_barrier(0);
        if (c < t.nK) {
            /* rows outside the matrix read row block 0 and are never stored */
            const int j = c & 3;
            const uint32_t so = (c & 1) * ST;
            /* the remainder first: the weight words then die sub-step by sub-step */
#pragma unroll
            for (int cb = 0; cb < NB; ++cb) {
                const int row = 16 * cb + c0;
                const int hsw = (row >> 1) & 7;
                const uint8_t *base = t.ldsp + so + GM_PIECE + row * 128;
                const uint4 lo = *(const uint4 *)(base + 16 * ((2 * q4) ^ hsw));
                const uint4 hi = *(const uint4 *)(base + 16 * ((2 * q4 + 1) ^ hsw));
                const gm_v8i bv = {(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                                   (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
                const uint32_t sb = t.ldsp[so + GM_PIECE + GM_F8_DATA + row * 4 + q4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[r][cb] = gm_mma_f8(cur[r], (scl[r] >> (8 * j)) & 0xffu, bv, sb, acc[r][cb]);
            }
            float sc[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) sc[r] = gm_scale((scl[r] >> (8 * j)) & 0xffu);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                k3v8bf a[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t wd = s == 0 ? cur[r].x : s == 1 ? cur[r].y
                                      : s == 2 ? cur[r].z : cur[r].w;
                    a[r] = gm_deq8(wd, sc[r]);
                }
                const int qs = 4 * s + t.g4;
#pragma unroll
                for (int cb = 0; cb < NB; ++cb) {
                    const uint4 bv = *(const uint4 *)(brow + so + cb * 16 * 256 + 16 * (qs ^ c0));
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[r][cb] = gm_mma(a[r], bv, acc[r][cb]);
                }
            }
            /* the reads three groups ahead (where the registers allow it: a full tile of 8
             * column blocks keeps the compiler's own order, without spilling) */
            gm_pipeline_mix<NB, 3>();
        }
    };
    aload(0, ab[0], sbuf[0]);
    dma(0);
    aload(min(1, t.nK - 1), ab[1], sbuf[1]);
    for (int c = 0; c < t.nK; c += 3) {
        step(c, ab[0], sbuf[0], ab[2], sbuf[2]);
        step(c + 1, ab[1], sbuf[1], ab[0], sbuf[0]);
        step(c + 2, ab[2], sbuf[2], ab[1], sbuf[1]);
    }
    gm_wait_vm<0>();

#pragma unroll
    for (int cb = 0; cb < NB; ++cb) {
        const int col = 16 * cb + c0;
        if (col < t.np) {
            const int p = t.p0 + col;
            float *o = g.out + (size_t)(g.scatter ? g.perm[p] : p) * g.ldo + t.orow0 + 4 * t.g4;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (t.rv[r]) *(k3v4f *)(o + 16 * r) = acc[r][cb];
        }
    }
}

/* The workgroup's tile and this wave's weight rows. Workgroup b runs on XCD b % 8 and is
 * dispatched there in the order of b / 8. The tiles (largest first) are dealt to the XCDs
 * in groups of G = K3G_TILE_GROUP consecutive tiles, the groups in a snake: round r of XCD
 * x takes tile G (8 q + x) + r % G (q = r / G even) or G (8 q + 7 - x) + r % G (q odd), so
 * every XCD gets the same mix, largest first, and an expert's consecutive full tiles land
 * on one XCD in consecutive rounds; the feature tiles of one column tile run back to back
 * on one XCD, sharing its activations in that XCD's L2. Returns false when the workgroup
 * has no tile. */
template <int AF, int WV>
__device__ __forceinline__ bool gm_setup(const K3kGemm &g, GmTile &t, uint8_t *lds, int &nb,
                                         bool halves = false)
{
    /* dense GEMMs cut into K slices take (column tile, slice) pairs as their tiles; with
     * halves, every column tile is two work items of up to 64 columns, dealt one after
     * the other to the same XCD */
    const int ks_n = g.tiles ? 1 : max(1, g.ksplit);
    const int ntl = (g.tiles ? *g.ntiles : (g.dense_rows + GM_COLS - 1) / GM_COLS) * ks_n *
                    (halves ? 2 : 1);
    const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
    const int rnd = slot / g.nft, f = slot - rnd * g.nft;
    const int grp = rnd / K3G_TILE_GROUP, gi = rnd - grp * K3G_TILE_GROUP;
    int tks = K3G_TILE_GROUP * (8 * grp + ((grp & 1) ? 7 - xcd : xcd)) + gi;
    if (tks >= ntl) return false;
    const int hf = halves ? (tks & 1) : 0;
    if (halves) tks >>= 1;
    const int tile = tks / ks_n;
    t.ks = tks - tile * ks_n;
    int e = 0;
    if (g.tiles) {
        const int4 tv = ((const int4 *)g.tiles)[tile];
        e = gm_uniform(tv.x); t.p0 = gm_uniform(tv.y); t.np = gm_uniform(tv.z);
    } else {
        t.p0 = tile * GM_COLS;
        t.np = min(GM_COLS, g.dense_rows - t.p0);
    }
    if (halves) {
        if (64 * hf >= t.np) return false;               /* a tile of 64 columns or fewer */
        t.p0 += 64 * hf;
        t.np = min(64, t.np - 64 * hf);
    }
    nb = (t.np + 15) >> 4;                               /* 16-column blocks in use */
    t.lane = threadIdx.x & 63;
    t.w = gm_uniform(threadIdx.x >> 6);
    t.g4 = t.lane >> 4;
    {
        const int steps = (g.K + GM_KC - 1) / GM_KC, per = (steps + ks_n - 1) / ks_n;
        t.kstep0 = t.ks * per;
        t.nK = max(0, min(per, steps - t.kstep0));
        t.nC32 = min(4 * t.nK, g.K / 32 - 4 * t.kstep0);
    }
    t.ldsp = lds;
    t.lds = (uint32_t)(uintptr_t)(k3lds)lds;
    const uint8_t *m0, *m1;
    if (AF == 0) {
        const K3ExpertQ *q = g.eq + e;
        m0 = g.mode == 0 ? q->p1 : q->p2;
        m1 = g.mode == 0 ? q->p3 : q->p2;
    } else {
        m0 = (const uint8_t *)g.wa;
        m1 = (const uint8_t *)(g.mode == 0 ? g.wb : g.wa);
    }
    /* bytes per 16-row block */
    const size_t rbb = AF == 0 ? (size_t)((g.K + 511) / 512) * GM_QT : (size_t)(g.K / 32) * 1024;
    t.rbb = (uint32_t)rbb;
    if (g.mode == 0) {
        t.orow0 = 32 * WV * f + 32 * t.w;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = t.orow0 + 16 * (r & 1);
            t.rv[r] = t.orow0 < g.rows;
            t.abase[r] = gm_uniform_ptr((r < 2 ? m0 : m1) + (size_t)(t.rv[r] ? row / 16 : 0) * rbb);
        }
    } else {
        t.orow0 = 64 * WV * f + 64 * t.w;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = t.orow0 + 16 * r;
            t.rv[r] = row < g.rows;
            t.abase[r] = gm_uniform_ptr(m0 + (size_t)(t.rv[r] ? row / 16 : 0) * rbb);
        }
    }
    return true;
}

/* the activation row a tile column reads: the token (gate/up of routed pairs) or the
 * column itself */
__device__ __forceinline__ int gm_src_row(const K3kGemm &g, const GmTile &t, int r)
{
    const int p = t.p0 + (r < t.np ? r : 0);
    return (g.mode == 0 && g.perm) ? g.perm[p] / g.topk : p;
}

/* WV = 8: one workgroup per CU, any piece count. WV = 4 (one-piece B only): two
 * workgroups of 4 waves per CU, each with 64 KB of stages, so one workgroup's matrix work
 * fills the other's barrier and load waits. */
template <int AF, int WV>
__global__ void __launch_bounds__(WV * 64, 8 / WV)
k_gemm(const K3kGemm g)
{
    __shared__ __attribute__((aligned(1024))) uint8_t lds[WV == 8 ? 2 * GM_STAGE : 2 * GM_PIECE];
    const int npr = (g.npieces > 1 && (!g.lo_flag || *g.lo_flag)) ? 2 : 1;
    if (WV == 4 ? npr != 1 : (g.np_only == 2 && npr != 2)) return;
    GmTile t;
    int nb;
    if (!gm_setup<AF, WV>(g, t, lds, nb)) return;
    const unsigned long long t_start = g.trace ? wall_clock64() : 0;

    /* ---- the activation rows this lane's DMA reads --------------------------------- */
    /* instruction i of wave w fills LDS rows 4 (WV i + w) .. + 3; lane l writes row
     * 4 (WV i + w) + l / 16, physical 16-byte slot l % 16, which holds logical slot
     * (l % 16) ^ (row % 16). row % 16 = (4 w + l / 16) % 16 for every i (WV = 4 or 8).
     * The B operand of sub-step s in lane group g is read from logical slot 4 s + g (the
     * conflict-free order); for MXFP4 weights that slot holds the 8 columns at
     * 32 g + 8 s of the step (the A operand's column order), i.e. logical slot q holds
     * columns 8 (4 (q % 4) + q / 4). */
    const int qlog = (t.lane & 15) ^ ((4 * t.w + (t.lane >> 4)) & 15);
    const int qoff = 8 * (AF == 0 ? 4 * (qlog & 3) + (qlog >> 2) : qlog);
    constexpr int NI = 32 / WV;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int r = 4 * (WV * i + t.w) + (t.lane >> 4);
        t.boff[i] = (uint32_t)gm_src_row(g, t, r) * (uint32_t)g.ldb + (uint32_t)qoff;
    }
    /* instructions whose first row is inside the tile's 16 nb rows */
    t.ndma = min(NI, (4 * nb + WV - 1 - t.w) / WV);

    bool mixed = false;
    if constexpr (AF == 0 && WV == 8) {
        if (g.mode == 1 && g.hmix) {
            /* the remainder's DMA (k_gemm_f8's layout, 128 rows): instruction i of wave w
             * fills rows 8 (8 i + w) .. + 7; waves 0 and 1 fill the scales of rows 0 .. 63
             * and 64 .. 127 */
            mixed = true;
            /* offsets relative to the tile's first row p0 (its rows are p0 .. p0 + 127) */
            auto rel = [&](int r) { return r < t.np ? r : 0; };
            uint32_t bofb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = 4 * (8 * i + t.w) + (t.lane >> 4);
                bofb[i] = 2u * ((uint32_t)rel(r) * (uint32_t)g.ldb + (uint32_t)qoff);
            }
            uint32_t doff[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int r = 8 * (8 * i + t.w) + (t.lane >> 3);
                const int ls = (t.lane & 7) ^ ((r >> 1) & 7);
                const int u = (ls & 1) ? 4 + (ls >> 1) : (ls >> 1);
                doff[i] = (uint32_t)rel(r) * (uint32_t)g.ldhq + 16 * u;
            }
            const int nd = min(2, (2 * nb + 7 - t.w) / 8);
            const int ns = nb > 4 ? 2 : 1;
            const uint32_t soff =
                (uint32_t)rel(64 * min(t.w, 1) + t.lane) * (uint32_t)(g.ldhq / 32);
            switch (nb) {
                case 1: gm_tile_mix<1>(g, t, bofb, doff, soff, nd, ns); break;
                case 2: gm_tile_mix<2>(g, t, bofb, doff, soff, nd, ns); break;
                case 3: gm_tile_mix<3>(g, t, bofb, doff, soff, nd, ns); break;
                case 4: gm_tile_mix<4>(g, t, bofb, doff, soff, nd, ns); break;
                case 5: gm_tile_mix<5>(g, t, bofb, doff, soff, nd, ns); break;
                case 6: gm_tile_mix<6>(g, t, bofb, doff, soff, nd, ns); break;
                case 7: gm_tile_mix<7>(g, t, bofb, doff, soff, nd, ns); break;
                case 8: gm_tile_mix<8>(g, t, bofb, doff, soff, nd, ns); break;
                default: break;
            }
        }
    }
#define GM_CASE(P, B) case (P) * 16 + (B): gm_tile<AF, P, B, WV>(g, t); break;
    if (mixed) {
    } else if constexpr (WV == 8) {
        switch (npr * 16 + nb) {
            GM_CASE(1, 1) GM_CASE(1, 2) GM_CASE(1, 3) GM_CASE(1, 4)
            GM_CASE(1, 5) GM_CASE(1, 6) GM_CASE(1, 7) GM_CASE(1, 8)
            GM_CASE(2, 1) GM_CASE(2, 2) GM_CASE(2, 3) GM_CASE(2, 4)
            GM_CASE(2, 5) GM_CASE(2, 6) GM_CASE(2, 7) GM_CASE(2, 8)
            default: break;
        }
    } else {
        switch (16 + nb) {
            GM_CASE(1, 1) GM_CASE(1, 2) GM_CASE(1, 3) GM_CASE(1, 4)
            GM_CASE(1, 5) GM_CASE(1, 6) GM_CASE(1, 7) GM_CASE(1, 8)
            default: break;
        }
    }
#undef GM_CASE
    if (g.trace && threadIdx.x == 0) {
        const int slot = blockIdx.x >> 3;
        const int rnd = slot / g.nft, xcd = blockIdx.x & 7;
        const int grp = rnd / K3G_TILE_GROUP, gi = rnd - grp * K3G_TILE_GROUP;
        unsigned long long *o = g.trace + 4 * (size_t)blockIdx.x;
        o[0] = t_start;
        o[1] = wall_clock64();
        o[2] = (unsigned long long)(K3G_TILE_GROUP * (8 * grp + ((grp & 1) ? 7 - xcd : xcd)) +
                                    gi) << 32 |
               (unsigned)(slot - rnd * g.nft);
        o[3] = (unsigned long long)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15) << 32 |
               (unsigned)__builtin_amdgcn_s_getreg((31 << 11) | 4);
    }
}

/* ============================================================ FP4 x FP8 variant ==== */
/* h = act(gate, up) for the wave's 32 features of one column, quantised as one MX block:
 * this lane's 4 + 4 values (features 4 g + i and 16 + 4 g + i) */
__device__ __noinline__ void gm_act_store_f8(k3v4f g0, k3v4f g1, k3v4f u0, k3v4f u1, float b1,
                                             float b2, uint8_t *o, uint8_t *os, int g4)
{
    float y[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        y[i] = k3d_act(g0[i], u0[i], b1, b2);
        y[4 + i] = k3d_act(g1[i], u1[i], b1, b2);
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(y[i]));
    m = fmaxf(m, __shfl_xor(m, 16, K3G_WAVE));
    m = fmaxf(m, __shfl_xor(m, 32, K3G_WAVE));
    const int sx = gm_mx_exp(m);
    *(uint32_t *)(o + 4 * g4) = gm_e4m3x4(y[0], y[1], y[2], y[3], sx);
    *(uint32_t *)(o + 16 + 4 * g4) = gm_e4m3x4(y[4], y[5], y[6], y[7], sx);
    if (g4 == 0) *os = (uint8_t)(sx + 127);
}

template <int NB>
__device__ __forceinline__ void gm_tile_f8(const K3kGemm &g, const GmTile &t,
                                           const uint32_t (&doff)[2], uint32_t soff, int nd,
                                           int ns)
{
    k3v4f acc[4][NB];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) acc[r][cb] = k3v4f{0.f, 0.f, 0.f, 0.f};
    const int lane = t.lane;
    auto dma = [&](int c) {
        const uint32_t st = t.lds + (c & 1) * GM_F8_STAGE;
        const uint8_t *b = g.bq + (size_t)c * GM_KC;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            if (i < nd) gm_dma16(b + doff[i], st + (8 * i + t.w) * 1024);
        if (t.w < ns) gm_dma4(g.bs + soff + 4 * c, st + GM_F8_DATA + t.w * 256);
    };
    /* B operand of column block cb: the lane's unit pair and its block scale */
    const int q = lane >> 4, c0 = lane & 15;
    auto bread = [&](int c, int cb, gm_v8i &bv, uint32_t &sb) {
        const int row = 16 * cb + c0;
        const int hsw = (row >> 1) & 7;
        const uint8_t *base = t.ldsp + (c & 1) * GM_F8_STAGE + row * 128;
        const uint4 lo = *(const uint4 *)(base + 16 * ((2 * q) ^ hsw));
        const uint4 hi = *(const uint4 *)(base + 16 * ((2 * q + 1) ^ hsw));
        bv = gm_v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w,
                    (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        sb = t.ldsp[(c & 1) * GM_F8_STAGE + GM_F8_DATA + row * 4 + q];
    };
    uint4 ab[3][4];
    uint32_t sbuf[3][4];
    auto aload = [&](int c, uint4 (&dst)[4], uint32_t (&sdst)[4]) {
        const size_t qo = (size_t)(c >> 2) * GM_QT;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const uint8_t *p = t.abase[r] + qo;
            dst[r] = gm_ld16(p + 1024 * (c & 3) + 16 * lane);
            sdst[r] = gm_ld4(p + 4096 + 4 * lane);
        }
    };
    /* the same pipeline as the bf16 kernel: weights two steps ahead (8 loads per step,
     * rotating by unrolling), activations one step ahead, every step issuing the same
     * loads */
    auto step = [&](int c, const uint4 (&cur)[4], const uint32_t (&scl)[4], uint4 (&nxt)[4],
                    uint32_t (&nsc)[4]) {
        gm_wait_vm<8>();
        __syncthreads();
        dma(min(c + 1, t.nK - 1));
        aload(min(c + 2, t.nK - 1), nxt, nsc);
        __builtin_amdgcn_sched_barrier(0);
        if (c < t.nK) {
            /* rows outside the matrix read row block 0 and are never stored */
            const int j = c & 3;
            /* B operands two column blocks at a time: reading all of them ahead would not
             * fit beside the accumulators */
#pragma unroll
            for (int cb = 0; cb < NB; ++cb) {
                gm_v8i bv;
                uint32_t sb;
                bread(c, cb, bv, sb);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    acc[r][cb] = gm_mma_f8(cur[r], (scl[r] >> (8 * j)) & 0xffu, bv, sb, acc[r][cb]);
                if (cb & 1) __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    aload(0, ab[0], sbuf[0]);
    dma(0);
    aload(min(1, t.nK - 1), ab[1], sbuf[1]);
    for (int c = 0; c < t.nK; c += 3) {
        step(c, ab[0], sbuf[0], ab[2], sbuf[2]);
        step(c + 1, ab[1], sbuf[1], ab[0], sbuf[0]);
        step(c + 2, ab[2], sbuf[2], ab[1], sbuf[1]);
    }
    gm_wait_vm<0>();

    /* ---- epilogue -------------------------------------------------------------------- */
    if (g.mode == 0) {
        if (!t.rv[0]) return;
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) {
            const int col = 16 * cb + c0;
            /* all four lane groups of the column take part in the block maximum */
            const size_t row = (size_t)(t.p0 + min(col, t.np - 1));
            uint8_t *o = g.hq + row * g.ldhq + t.orow0;
            uint8_t *os = g.hs + row * (g.ldhq / 32) + t.orow0 / 32;
            if (col < t.np)
                gm_act_store_f8(acc[0][cb], acc[1][cb], acc[2][cb], acc[3][cb], g.b1, g.b2, o,
                                os, t.g4);
        }
    } else {
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) {
            const int col = 16 * cb + c0;
            if (col < t.np) {
                const int p = t.p0 + col;
                float *o = g.out + (size_t)(g.scatter ? g.perm[p] : p) * g.ldo + t.orow0 + 4 * t.g4;
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (t.rv[r]) *(k3v4f *)(o + 16 * r) = acc[r][cb];
            }
        }
    }
}

__global__ void __launch_bounds__(GM_WAVES * 64, 1)
k_gemm_f8(const K3kGemm g)
{
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * GM_F8_STAGE];
    /* the tile's two 64-column halves are separate work items on one XCD, one after the
     * other in its dispatch order (4 x 4 accumulators fit beside the weight pipeline, 4 x 8
     * do not), so they stream the same weights at about the same time and the second
     * finds them in the XCD's L2 */
    GmTile t;
    int nb;
    if (!gm_setup<0, GM_WAVES>(g, t, lds, nb, true)) return;
    /* data DMA: instruction i of wave w fills rows 8 (8 i + w) .. + 7 (only i = 0 is
     * needed for 64 rows); lane l writes row 8 (8 i + w) + l / 8, physical unit l % 8 =
     * logical unit (l % 8) ^ ((row / 2) % 8); logical unit 2 q holds column unit q,
     * 2 q + 1 holds unit 4 + q */
    uint32_t doff[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 8 * (8 * i + t.w) + (t.lane >> 3);
        const int ls = (t.lane & 7) ^ ((r >> 1) & 7);
        const int u = (ls & 1) ? 4 + (ls >> 1) : (ls >> 1);
        doff[i] = (uint32_t)gm_src_row(g, t, r) * (uint32_t)g.ldb + 16 * u;
    }
    const int nd = min(2, (2 * nb + 7 - t.w) / 8);
    /* scales: wave 0 fills rows 0 .. 63, 4 bytes each */
    const uint32_t soff = (uint32_t)gm_src_row(g, t, t.lane) * (uint32_t)(g.ldb / 32);
    switch (nb) {
        case 1: gm_tile_f8<1>(g, t, doff, soff, nd, 1); break;
        case 2: gm_tile_f8<2>(g, t, doff, soff, nd, 1); break;
        case 3: gm_tile_f8<3>(g, t, doff, soff, nd, 1); break;
        case 4: gm_tile_f8<4>(g, t, doff, soff, nd, 1); break;
        default: break;
    }
}

/* ------------------------------------------------------------------ helpers ------ */
/* Column tiles from the expert ranges (k3d_build_tiles). One block of 1024 threads
 * (n_experts <= 1024). */
static_assert(GM_COLS == K3G_TILE_COLS, "column tile width");
__global__ void __launch_bounds__(1024)
k_gemm_tiles(const int32_t *__restrict__ off, int E, int4 *__restrict__ tiles,
             int32_t *__restrict__ ntiles, int32_t *__restrict__ flag)
{
    __shared__ int red[17 * 9];
    const int e = threadIdx.x;
    const int cnt = e < E ? off[e + 1] - off[e] : 0;
    k3d_build_tiles(e, E, cnt, e < E ? off[e] : 0, tiles, ntiles, flag, red);
}

/* x (fp32 [T][d]) -> two bf16 pieces [2][T][ldb]; raises *flag when any piece 1 is not
 * zero. The padding columns d..ldb are never written (the workspace starts zeroed). */
__global__ void __launch_bounds__(256)
k_xpieces(const float *__restrict__ x, int T, int d, int ldb, uint16_t *__restrict__ xb,
          long long piece, int32_t *__restrict__ flag)
{
    const size_t n = (size_t)T * d;
    bool nz = false;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t t = i / d, c = i - t * d;
        const float v = x[i];
        const uint16_t hi = gm_bf16_rn(v);
        const uint16_t lo = gm_bf16_rn(v - gm_bf16_f(hi));
        xb[t * ldb + c] = hi;
        xb[piece + t * ldb + c] = lo;
        nz |= lo != 0;
    }
    if (__any(nz) && (threadIdx.x & 63) == 0) *flag = 1;
}

/* The same, eight columns per thread (two 16-byte loads, one 16-byte store per piece):
 * d a multiple of 8, x 16-byte aligned. */
__global__ void __launch_bounds__(256)
k_xpieces8(const float *__restrict__ x, int T, int d, int ldb, uint16_t *__restrict__ xb,
           long long piece, int32_t *__restrict__ flag)
{
    const int d8 = d / 8;
    const size_t n = (size_t)T * d8;
    bool nz = false;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t t = i / d8, c = 8 * (i - t * d8);
        const float4 a = *(const float4 *)(x + t * d + c), b = *(const float4 *)(x + t * d + c + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint16_t h0 = gm_bf16_rn(v[2 * j]), h1 = gm_bf16_rn(v[2 * j + 1]);
            const uint16_t l0 = gm_bf16_rn(v[2 * j] - gm_bf16_f(h0));
            const uint16_t l1 = gm_bf16_rn(v[2 * j + 1] - gm_bf16_f(h1));
            hi[j] = (uint32_t)h0 | ((uint32_t)h1 << 16);
            lo[j] = (uint32_t)l0 | ((uint32_t)l1 << 16);
            nz |= (lo[j] != 0);
        }
        *(uint4 *)(xb + t * ldb + c) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        *(uint4 *)(xb + piece + t * ldb + c) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
    if (__any(nz) && (threadIdx.x & 63) == 0) *flag = 1;
}

/* The K slices of a dense GEMM summed in slice order: gate/up (mode 0) -> act -> h as two
 * bf16 pieces; down (mode 1) -> out rows. One thread per 4 consecutive rows of a column. */
__global__ void __launch_bounds__(256)
k_gemm_reduce(const float *__restrict__ part, int ks_n, int ncol, int R, int mode, float b1,
              float b2, uint16_t *__restrict__ h, long long hpiece, int ldh,
              float *__restrict__ out, int ldo)
{
    const int r4 = R / 4;
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long long)ncol * r4) return;
    const int col = (int)(i / r4), n = 4 * (int)(i - (long long)col * r4);
    if (mode == 0) {
        k3v4f gs = {0, 0, 0, 0}, us = {0, 0, 0, 0};
        for (int k = 0; k < ks_n; ++k) {
            const float *p = part + ((size_t)k * ncol + col) * 2 * R + n;
            gs += *(const k3v4f *)p;
            us += *(const k3v4f *)(p + R);
        }
        gm_act_store(gs, us, b1, b2, h + (size_t)col * ldh + n, hpiece);
    } else {
        k3v4f y = {0, 0, 0, 0};
        for (int k = 0; k < ks_n; ++k) y += *(const k3v4f *)(part + ((size_t)k * ncol + col) * R + n);
        *(k3v4f *)(out + (size_t)col * ldo + n) = y;
    }
}

extern "C" int k3k_gemm_ksplit(int nft, int ntl, int K)
{
    const int steps = (K + GM_KC - 1) / GM_KC;
    const int want = nft * ntl >= 256 ? 1 : 256 / (nft * ntl);
    int ks = want < steps ? want : steps;
    if (ks < 1) ks = 1;
    /* whole steps per slice, no empty slice */
    const int per = (steps + ks - 1) / ks;
    return (steps + per - 1) / per;
}

extern "C" size_t k3k_gemm_part_bytes(int nft, int rows2)
{
    /* ksplit x column tiles <= 256 / nft + 1 whenever ksplit > 1 */
    return (size_t)(256 / nft + 1) * GM_COLS * (size_t)rows2 * 4;
}

/* ------------------------------------------------------------------ launchers ---- */
extern "C" int k3k_gemm_tiles(const int32_t *off, int E, int32_t *tiles, int32_t *ntiles,
                              int32_t *flag, hipStream_t st)
{
    if (E < 1 || E > 1024) return -1;
    hipLaunchKernelGGL(k_gemm_tiles, dim3(1), dim3(1024), 0, st, off, E, (int4 *)tiles, ntiles,
                       flag);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int k3k_xpieces(const float *x, int T, int d, int ldb, uint16_t *xb,
                           long long piece, int32_t *flag, hipStream_t st)
{
    if (T < 1 || d < 1 || ldb < d) return -1;
    if (d % 8 == 0 && ldb % 8 == 0 && piece % 8 == 0 && ((uintptr_t)x & 15) == 0 &&
        ((uintptr_t)xb & 15) == 0) {
        const size_t n = (size_t)T * (d / 8);
        const int blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
        hipLaunchKernelGGL(k_xpieces8, dim3(blocks), dim3(256), 0, st, x, T, d, ldb, xb, piece,
                           flag);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    const size_t n = (size_t)T * d;
    const int blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    hipLaunchKernelGGL(k_xpieces, dim3(blocks), dim3(256), 0, st, x, T, d, ldb, xb, piece, flag);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

/* x -> MXFP8, one thread per 32-column block */
__global__ void __launch_bounds__(256)
k_xq8(const float *__restrict__ x, int T, int d, int ldq, uint8_t *__restrict__ xq,
      uint8_t *__restrict__ xs)
{
    const int nbk = d / 32;
    const long long b = (long long)blockIdx.x * 256 + threadIdx.x;
    if (b >= (long long)T * nbk) return;
    const int t = (int)(b / nbk), k = (int)(b - (long long)t * nbk);
    const float4 *p = (const float4 *)(x + (size_t)t * d + 32 * k);
    float4 v[8];
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[i] = p[i];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    }
    const int sx = gm_mx_exp(m);
    uint32_t *o = (uint32_t *)(xq + (size_t)t * ldq + 32 * k);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = gm_e4m3x4(v[i].x, v[i].y, v[i].z, v[i].w, sx);
    xs[(size_t)t * (ldq / 32) + k] = (uint8_t)(sx + 127);
}

extern "C" int k3k_xq8(const float *x, int T, int d, int ldq, uint8_t *xq, uint8_t *xs,
                       hipStream_t st)
{
    if (T < 1 || d < 32 || d % 32 || ldq < d || ldq % 32 || ((uintptr_t)x & 15)) return -1;
    const long long n = (long long)T * (d / 32);
    hipLaunchKernelGGL(k_xq8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, T, d, ldq,
                       xq, xs);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int k3k_gemm_f8(const K3kGemm *g, hipStream_t st)
{
    if (g->mode < 0 || g->mode > 1 || g->afmt != 0 || !g->eq || !g->bq || !g->bs) return -1;
    if (g->K < 32 || g->K % 32 || g->rows < 16 || g->ldb < g->K || g->ldb % 512 || g->nft < 1)
        return -1;
    if (g->mode == 0 && (g->rows % 32 || g->nft * 256 < g->rows || !g->hq || !g->hs ||
                         g->ldhq < g->rows || g->ldhq % 512))
        return -1;
    if (g->mode == 1 && (g->rows % 16 || g->nft * 512 < g->rows || !g->out || g->ldo < g->rows ||
                         g->ldo % 4))
        return -1;
    if (g->tiles ? (!g->ntiles || g->max_tiles < 1) : g->dense_rows < 1) return -1;
    if ((g->scatter || (g->mode == 0 && g->tiles)) && !g->perm) return -1;
    const long long maxt = g->tiles ? g->max_tiles : (g->dense_rows + GM_COLS - 1) / GM_COLS;
    const long long grid = 8 * (long long)K3G_TILE_ROUNDS(2 * maxt) * g->nft;   /* halves */
    if (grid > 0x7fffffff) return -1;
    hipLaunchKernelGGL(k_gemm_f8, dim3((unsigned)grid), dim3(GM_WAVES * 64), 0, st, *g);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int k3k_gemm(const K3kGemm *g, hipStream_t st)
{
    /* shapes the kernel's indexing assumes */
    if (g->mode < 0 || g->mode > 1 || g->afmt < 0 || g->afmt > 1) return -1;
    if (g->K < 32 || g->K % 32 || g->rows < 16 || g->ldb < g->K || g->ldb % GM_KC ||
        g->npieces < 1 || g->npieces > 2 || !g->b || g->nft < 1)
        return -1;
    if (g->mode == 0 && (g->rows % 32 || g->nft * 256 < g->rows || !g->h || g->ldh < g->rows))
        return -1;
    if (g->mode == 1 && (g->rows % 16 || g->nft * 512 < g->rows || !g->out || g->ldo < g->rows ||
                         g->ldo % 4))
        return -1;
    if (g->afmt == 0 && !g->eq) return -1;
    if (g->hmix && (g->afmt != 0 || g->ldhq % 512 ||
                    (g->mode == 0 ? (!g->hq || !g->hs || g->ldhq < g->rows)
                                  : (!g->bq || !g->bs || g->ldhq < g->K || g->npieces != 1))))
        return -1;
    if (g->afmt == 1 && (!g->wa || (g->mode == 0 && !g->wb))) return -1;
    if (g->tiles ? (!g->ntiles || g->max_tiles < 1) : g->dense_rows < 1) return -1;
    if ((g->scatter || (g->mode == 0 && g->tiles)) && !g->perm) return -1;
    const int ks_n = g->ksplit > 1 ? g->ksplit : 1;
    if (ks_n > 1 && (g->tiles || g->afmt != 1 || !g->part || g->K % GM_KC ||
                     ks_n > g->K / GM_KC || (g->mode == 0 && g->rows % 4)))
        return -1;
    const long long maxt = g->tiles ? g->max_tiles
                                    : (long long)((g->dense_rows + GM_COLS - 1) / GM_COLS) * ks_n;
    const long long grid = 8 * (long long)K3G_TILE_ROUNDS(maxt) * g->nft;
    if (grid > 0x7fffffff) return -1;
    if (g->afmt == 0 && g->mode == 0) {
        /* gate/up of MXFP4 experts: 4-wave workgroups when x is one piece (the usual case:
         * decided on the device from the flag), 8-wave ones for two pieces; each launch
         * leaves at once when the other one's case holds */
        K3kGemm g4 = *g, g8 = *g;
        g4.nft = (g->rows + 127) / 128;
        g8.np_only = 2;
        const long long grid4 = 8 * (long long)K3G_TILE_ROUNDS(maxt) * g4.nft;
        if (grid4 > 0x7fffffff) return -1;
        hipLaunchKernelGGL((k_gemm<0, 4>), dim3((unsigned)grid4), dim3(4 * 64), 0, st, g4);
        if (g->npieces > 1)
            hipLaunchKernelGGL((k_gemm<0, 8>), dim3((unsigned)grid), dim3(GM_WAVES * 64), 0, st, g8);
    } else if (g->afmt == 0) {
        hipLaunchKernelGGL((k_gemm<0, 8>), dim3((unsigned)grid), dim3(GM_WAVES * 64), 0, st, *g);
    } else {
        K3kGemm g1 = *g;
        g1.ksplit = ks_n;
        hipLaunchKernelGGL((k_gemm<1, 8>), dim3((unsigned)grid), dim3(GM_WAVES * 64), 0, st, g1);
        if (ks_n > 1) {
            const long long n = (long long)g->dense_rows * (g->rows / 4);
            hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                               g->part, ks_n, g->dense_rows, g->rows, g->mode, g->b1, g->b2,
                               g->h, g->hpiece, g->ldh, g->out, g->ldo);
        }
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
