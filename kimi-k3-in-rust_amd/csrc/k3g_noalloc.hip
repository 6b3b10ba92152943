/* k3g_noalloc.hip - k3g_moe at decode sizes without any allocation: every buffer of the
 * fused decode kernel beyond the caller's x, out, idx and wt lives in one fixed device
 * array, `scratch`, of K3G_NOALLOC_BYTES per GPU, held until the process ends.
 *
 * For callers that cannot call hipMalloc (code under HIP graph capture, serving loops
 * that forbid allocation). The engine has no such entry point: its k3_moe takes a
 * caller-provided scratch of host floats.
 *
 * Layout of the array (per GPU): two counter banks of K3G_NOALLOC_BANK bytes at the front
 * (the fused kernel counts in one bank and zeroes the other for the next call), then the
 * kernel's buffers carved for the call's layer shape at 4 tokens, so every token count of
 * one shape finds them at the same offsets. Cleared by a fill kernel the first time a GPU
 * is used and whenever the layer shape changes (the activation pieces' padding must read
 * as zero). Calls that overlap on one GPU share the array and race: they must be ordered
 * on one stream (or otherwise serialised) by the caller. */
#include "k3g_dev.h"
#include "k3g_kernels.h"

#include <pthread.h>
#include <stdio.h>
#include <string.h>

#define K3G_NOALLOC_BYTES (16u << 20)
#define K3G_NOALLOC_BANK (1u << 20)
#define K3G_NOALLOC_DEV 16

static __device__ __align__(256) uint8_t scratch[K3G_NOALLOC_BYTES];

namespace {

struct NoallocDev {
    uint8_t *ptr;          /* this GPU's copy of `scratch` (hipGetSymbolAddress) */
    int epoch;             /* counter bank of the next call */
    int key[6];            /* layer shape the buffers were last cleared for */
    bool have_key;
};

NoallocDev g_na[K3G_NOALLOC_DEV];
pthread_mutex_t g_na_lock = PTHREAD_MUTEX_INITIALIZER;

__global__ void __launch_bounds__(256) k_noalloc_zero(uint4 *p, size_t n16)
{
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
        p[i] = make_uint4(0, 0, 0, 0);
}

size_t carve(size_t *at, size_t bytes)
{
    const size_t o = *at;
    *at += (bytes + 255) & ~(size_t)255;
    return o;
}

/* byte offsets of the fused kernel's buffers for a layer shape at 4 tokens */
struct NoallocLayout {
    size_t rs, rpart, xq8, xq16, gpart, hq8, sgpart, hq16, contrib, shpart, idx, wt, err, stats;
    size_t total;
};

NoallocLayout layout_for(int d, int E, int k, int I, int SI)
{
    const size_t T4 = 4, P4 = T4 * (size_t)k;
    const size_t nQd = ((size_t)d + 511) / 512, nQi = ((size_t)I + 511) / 512;
    NoallocLayout l;
    size_t at = 2 * (size_t)K3G_NOALLOC_BANK;
    l.rs = carve(&at, T4 * E * 16);
    l.rpart = carve(&at, T4 * E * K3G_KS_R_MAX * 16);
    l.xq8 = carve(&at, T4 * nQd * 8448);
    l.xq16 = carve(&at, ((size_t)d / 32) * 1024);
    l.gpart = carve(&at, P4 * K3G_KS_G_MAX * 2 * (size_t)I * 4);
    l.hq8 = carve(&at, P4 * nQi * 8448);
    l.sgpart = carve(&at, (size_t)K3G_KS_SG_MAX * T4 * 2 * (SI ? SI : 1) * 4);
    l.hq16 = carve(&at, ((size_t)SI / 32 + 1) * 1024);
    l.contrib = carve(&at, P4 * K3G_KS_D_MAX * (size_t)d * 4);
    l.shpart = carve(&at, (size_t)K3G_KS_SD_MAX * T4 * d * 4);
    l.idx = carve(&at, P4 * 4);
    l.wt = carve(&at, P4 * 4);
    l.err = carve(&at, 4);
    l.stats = carve(&at, 16 * 4);
    l.total = at;
    return l;
}

}  // namespace

extern "C" int k3g_moe_noalloc(const K3gLayer *L, const float *x, int T, float *out,
                               int32_t *idx, float *wt, int *err, void *stream)
{
    if (!L || !x || !out || T < 1 || T > 4) {
        fprintf(stderr, "k3g_moe_noalloc: needs a layer, x and out, and 1 <= T <= 4 (T = %d)\n",
                T);
        return -1;
    }
    const int lat = L->latent > 0 ? L->latent : L->hidden;
    if (L->expert_fmt != K3G_EXPERT_MXFP4_TILED || !L->experts || !L->gate || L->down ||
        L->up || L->latent_norm || lat != L->hidden || L->hidden % 32 || L->inter % 32 ||
        L->inter < 32 || L->topk < 1 || L->topk > K3G_MAX_TOPK || L->n_experts < 1 ||
        L->n_experts > 1024 || T * L->topk > 256 ||
        (L->shared_inter && (L->wdt != K3_WBF16 || L->shared_fmt != 1 || L->shared_inter % 32 ||
                             !L->sh1 || !L->sh3 || !L->sh2))) {
        fprintf(stderr, "k3g_moe_noalloc: the layer is not the fused decode kernel's shape "
                        "(tiled MXFP4 experts, tiled bf16 shared expert, no latent projection, "
                        "widths multiples of 32)\n");
        return -1;
    }
    const int d = L->hidden, E = L->n_experts, k = L->topk, I = L->inter, SI = L->shared_inter;
    const NoallocLayout lo = layout_for(d, E, k, I, SI);
    const size_t sync_bytes = k3k_decode_sync_bytes(4, d, E, k, I, SI, d);
    if (lo.total > K3G_NOALLOC_BYTES || sync_bytes > K3G_NOALLOC_BANK) {
        fprintf(stderr, "k3g_moe_noalloc: the layer needs %zu bytes of scratch (%zu of "
                        "counters), beyond the fixed %u (%u per counter bank)\n",
                lo.total, sync_bytes, K3G_NOALLOC_BYTES, K3G_NOALLOC_BANK);
        return -1;
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= K3G_NOALLOC_DEV) {
        fprintf(stderr, "k3g_moe_noalloc: no current device below %d\n", K3G_NOALLOC_DEV);
        return -1;
    }
    hipStream_t st = (hipStream_t)stream;
    pthread_mutex_lock(&g_na_lock);
    NoallocDev &s = g_na[dev];
    if (!s.ptr) {
        /* this GPU's copy of the array: kernels get its address, never the symbol */
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            pthread_mutex_unlock(&g_na_lock);
            fprintf(stderr, "k3g_moe_noalloc: hipGetSymbolAddress failed: %s\n",
                    hipGetErrorString(e));
            return -1;
        }
        s.ptr = (uint8_t *)p;
        s.have_key = false;
    }
    const int key[6] = {d, E, k, I, SI, L->shared_inter ? 1 : 0};
    bool same = s.have_key;
    for (int i = 0; i < 6 && same; ++i) same = s.key[i] == key[i];
    if (!same) {
        const size_t n16 = K3G_NOALLOC_BYTES / 16;
        hipLaunchKernelGGL(k_noalloc_zero, dim3(1024), dim3(256), 0, st, (uint4 *)s.ptr, n16);
        if (hipGetLastError() != hipSuccess) {
            pthread_mutex_unlock(&g_na_lock);
            fprintf(stderr, "k3g_moe_noalloc: clearing the scratch array failed\n");
            return -1;
        }
        for (int i = 0; i < 6; ++i) s.key[i] = key[i];
        s.have_key = true;
        s.epoch = 0;
    }
    uint8_t *b = s.ptr;
    K3kDecode a;
    memset(&a, 0, sizeof a);
    a.T = T;
    a.d = d;
    a.E = E;
    a.k = k;
    a.I = I;
    a.SI = SI;
    a.renorm = L->renorm;
    a.routed_scale = L->routed_scale;
    a.b1 = L->act_b1;
    a.b2 = L->act_b2;
    a.gate = L->gate;
    a.bias = L->bias;
    a.eq = L->experts;
    a.sh1 = (const uint16_t *)L->sh1;
    a.sh3 = (const uint16_t *)L->sh3;
    a.sh2 = (const uint16_t *)L->sh2;
    a.x = x;
    a.out = out;
    a.idx = idx ? idx : (int32_t *)(b + lo.idx);
    a.wt = wt ? wt : (float *)(b + lo.wt);
    a.rs = (float *)(b + lo.rs);
    a.rpart = (double *)(b + lo.rpart);
    a.xq8 = b + lo.xq8;
    a.xq16 = (uint16_t *)(b + lo.xq16);
    a.gpart = (float *)(b + lo.gpart);
    a.hq8 = b + lo.hq8;
    a.sgpart = (float *)(b + lo.sgpart);
    a.hq16 = (uint16_t *)(b + lo.hq16);
    a.contrib = (float *)(b + lo.contrib);
    a.shpart = (float *)(b + lo.shpart);
    /* the whole other bank is zeroed, whatever this call's geometry uses of it */
    a.sync = (int *)(b + (size_t)(s.epoch & 1) * K3G_NOALLOC_BANK);
    a.sync_clear = (int *)(b + (size_t)((s.epoch & 1) ^ 1) * K3G_NOALLOC_BANK);
    a.sync_words = (int)(K3G_NOALLOC_BANK / 4);
    a.err = err ? err : (int *)(b + lo.err);
    a.stats = (int *)(b + lo.stats);
    a.force = 0;
    a.spin_limit = 1ll << 21;
    a.trace = nullptr;
    const int rc = k3k_decode_fused(&a, st);
    if (rc == 0) s.epoch ^= 1;
    pthread_mutex_unlock(&g_na_lock);
    if (rc != 0) fprintf(stderr, "k3g_moe_noalloc: launch failed\n");
    return rc;
}
