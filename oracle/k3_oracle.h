/* k3_oracle.h - CPU restatement of the engine's routed-expert MoE arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This is what the GPU path is compared against. Only
 * tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may load it; the
 * product library never links it and never falls back to it.
 *
 * Every function restates one reference function (file:line given at each definition)
 * with the same operation order, the same double accumulators and the same reduction
 * trees, and is compiled with -ffp-contract=off as the engine is (Makefile:127-139).
 * Where the engine has an AVX2 and a scalar form that differ in the last bits
 * (k3_matmul_mxfp4), the AVX2 form is restated: it is what an x86-64 host runs.
 */
#ifndef K3_ORACLE_H
#define K3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "../include/k3moe.h"

#ifdef __cplusplus
extern "C" {
#endif

extern long ork3_expert_drops;

void   ork3_mxfp4_dequant(float *out, const unsigned char *packed,
                          const unsigned char *scales, int rows, int pcols, int group);
void   ork3_matmul_mxfp4(float *y, const float *x, const unsigned char *packed,
                         const unsigned char *scales, int in, int rows, int group);
void   ork3_matmul_bf16(float *y, const float *x, const uint16_t *W, int in, int out);
/* per-row int8 draft weights: `out` rows of [f32 scale][int8 * in] */
void   ork3_matmul_q8(float *y, const float *x, const void *W, int in, int out);
void   ork3_matmul(float *y, const float *x, const float *W, int in, int out);
void   ork3_situ_glu(float *y, const float *x, int n, float b1, float b2);
void   ork3_rmsnorm(float *y, const float *x, const float *w, int n, float eps);
void   ork3_router(int *idx, float *w, const float *x, const float *W,
                   const float *bias, int hidden, int n_experts, int topk,
                   int renorm, float routed_scale);
size_t ork3_moe_scratch(const K3Cfg *c);
void   ork3_moe(float *out, const float *x, const K3MoeW *w, const K3Cfg *c,
                int T, int *idx, float *wt, float *scratch);
void   ork3_moe_prefill(float *out, const float *x, const K3MoeW *w, const K3Cfg *c,
                        int T, int *idx, float *wt, float *scratch);

/* The kernels ork3_moe composes. By default the restatements above; the CPU baseline
 * swaps in the engine's own compiled kernels so that the composition (which the engine
 * can only express with identity latent matrices for the K2 shape) runs the engine's
 * arithmetic. Passing NULL restores the restatements. */
typedef struct {
    void (*router)(int *, float *, const float *, const float *, const float *,
                   int, int, int, int, float);
    void (*matmul_mxfp4)(float *, const float *, const unsigned char *,
                         const unsigned char *, int, int, int);
    void (*matmul_bf16)(float *, const float *, const uint16_t *, int, int);
    void (*matmul)(float *, const float *, const float *, int, int);
    void (*situ_glu)(float *, const float *, int, float, float);
    void (*rmsnorm)(float *, const float *, const float *, int, float);
    void (*matmul_q8)(float *, const float *, const void *, int, int);
} OrKernels;
void ork3_set_kernels(const OrKernels *k);

/* An in-memory K3ExpertSrc over expert runs: expert e of layer L starts at
 * bases[L * n_experts + e] (NULL: get() fails, which is how a test forces an expert drop),
 * with the six matrices at the given offsets. `src` is the first member, so &s->src is
 * what K3MoeW.src takes. */
typedef struct {
    K3ExpertSrc src;
    const unsigned char *const *bases;
    int64_t p1_off, s1_off, p2_off, s2_off, p3_off, s3_off;
    int n_layers, n_experts;
    int64_t gets, getmanys, residents;   /* call counts */
} OrMemSrc;
void ork3_memsrc_init(OrMemSrc *s, const unsigned char *const *bases, int n_layers,
                      int n_experts, const int64_t offs[6]);

/* Textbook LRU replay (tools/sim_cache.py:36-48): hits for a trace of keys at a given
 * capacity in slots. */
int64_t ork3_lru_hits(const int32_t *keys, int64_t n, int64_t nkeys, int64_t capacity);

/* Quantisation-aware restatement for the MXFP8 activation variant: x rounded to OCP
 * E4M3 with one E8M0 scale per 32 elements (scale = 2^(floor(log2 amax) - 8), the OCP
 * MX rule with emax(E4M3) = 8), nearest-even, saturating at 448. In place; n % 32 == 0. */
void ork3_quant_mxfp8(float *x, int n);

/* The benchmark's known-answer inputs and output hash (benchmarks/bench_kernels.c:44-89). */
void ork3_kat_fillf(float *p, size_t n, unsigned s);
void ork3_kat_fillb(unsigned char *p, size_t n, unsigned s);
void ork3_kat_fillbf16(uint16_t *p, size_t n, unsigned s);
unsigned long long ork3_fnv1a(const float *v, int n);

#ifdef __cplusplus
}
#endif

#endif /* K3_ORACLE_H */
