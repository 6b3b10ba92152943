/* select_audit.cpp - runs the router's certified top-k (k3g_select.h, the code the GPU
 * kernels run) on the host, one 64-thread wave per token, under AddressSanitizer and the
 * array-bounds checker, and compares every token's routing with the oracle's k3_router
 * restatement (test infrastructure).
 *
 * Each case builds a router (W [E][d], bias [E], x [T][d]) in exactly sized heap blocks,
 * forms the score intervals the logit kernels store (k3d_route_score on an fp64 sum taken
 * in a lane-strided order, as the GPU takes it), then selects every token with and without
 * the LDS staging of the exact path, in the normal and the three forced modes. Inputs can
 * carry duplicated router rows and tied biases (exact ties in the choice scores, which fail
 * the certificate and exercise the exact path and its lowest-index rule).
 *
 * usage: select_audit E k d T ties seed [wide]   (prints one line per case; exit 1 on a
 *                                             mismatch, the sanitizers abort on a fault) */
#include "k3g_select.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <thread>
#include <vector>

extern "C" void ork3_router(int *idx, float *w, const float *x, const float *W,
                            const float *bias, int hidden, int n_experts, int topk, int renorm,
                            float routed_scale);

EmuWave *g_wave;
thread_local int t_lane;

/* The fp64 sum of exact products in the order of a wave that takes 4 columns per lane per
 * 256-column step and reduces the lanes by a butterfly; also sum |w x|. */
static void strided_dot(const float *w, const float *x, int d, double *s, double *a)
{
    double ls[64] = {0}, la[64] = {0};
    for (int i0 = 0; i0 < d; i0 += 256)
        for (int l = 0; l < 64; ++l)
            for (int q = 0; q < 4; ++q) {
                const int i = i0 + 4 * l + q;
                if (i < d) {
                    const double p = (double)w[i] * (double)x[i];
                    ls[l] += p;
                    la[l] += std::fabs(p);
                }
            }
    for (int m = 32; m >= 1; m >>= 1)
        for (int l = 0; l < 64; ++l)
            if (!(l & m)) { ls[l] += ls[l + m]; la[l] += la[l + m]; }
    *s = ls[0];
    *a = la[0];
}

int main(int argc, char **argv)
{
    if (argc != 7 && argc != 8) {
        std::fprintf(stderr, "usage: select_audit E k d T ties seed [wide]\n");
        return 2;
    }
    /* wide: every interval's bound is widened to many float ulps of the logit and its best
     * guess moved by 0.7 of the bound (still inside it), so no score is settled and the
     * guessed scores are not the engine's: a weight taken from a guess is a mismatch */
    const int wide = argc == 8 ? std::atoi(argv[7]) : 0;
    const int E = std::atoi(argv[1]), k = std::atoi(argv[2]), d = std::atoi(argv[3]);
    const int T = std::atoi(argv[4]), ties = std::atoi(argv[5]);
    const unsigned seed = (unsigned)std::atoi(argv[6]);
    if (E < 1 || E > K3G_MAX_E || k < 1 || k > 64 || d < 4 || d % 4 || T < 1) return 2;

    std::mt19937_64 rng(seed);
    std::normal_distribution<float> nw(0.0f, 0.02f), nx(0.0f, 1.0f), nb(0.0f, 0.01f);
    /* exactly sized blocks: any read past them is an AddressSanitizer report */
    float *W = new float[(size_t)E * d];
    float *x = new float[(size_t)T * d];
    float *bias = new float[E];
    for (size_t i = 0; i < (size_t)E * d; ++i) W[i] = nw(rng);
    for (size_t i = 0; i < (size_t)T * d; ++i) x[i] = nx(rng);
    for (int e = 0; e < E; ++e) bias[e] = nb(rng);
    if (ties) {
        /* every third row repeats its predecessor (equal logits, equal scores) with the same
         * bias (equal choices), and a few biases are set so that a choice ties another's */
        for (int e = 1; e < E; e += 3) {
            std::memcpy(W + (size_t)e * d, W + (size_t)(e - 1) * d, (size_t)d * 4);
            bias[e] = bias[e - 1];
        }
    }

    float4 *rs = new float4[(size_t)T * E];
    for (int t = 0; t < T; ++t)
        for (int e = 0; e < E; ++e) {
            double s, a;
            strided_dot(W + (size_t)e * d, x + (size_t)t * d, d, &s, &a);
            if (wide) {
                const double nr = 1e8, B = nr * 0x1p-53 * 1.01 * a + std::fabs(s) * 0x1p-51;
                rs[(size_t)t * E + e] = k3d_route_score_n(s + ((e & 1) ? 0.7 : -0.7) * B, a,
                                                          bias[e], nr);
            } else {
                rs[(size_t)t * E + e] = k3d_route_score(s, a, bias[e], d);
            }
        }

    std::vector<int> ref_idx((size_t)T * k);
    std::vector<float> ref_w((size_t)T * k);
    for (int t = 0; t < T; ++t)
        ork3_router(&ref_idx[(size_t)t * k], &ref_w[(size_t)t * k], x + (size_t)t * d, W, bias,
                    d, E, k, 1, 2.5f);

    K3SelectLds *lds = new K3SelectLds;
    alignas(16) static uint8_t stage_mem[K3G_XD_BYTES];
    int bad = 0;
    for (int staged = 0; staged < 2; ++staged)
        for (int force = 0; force <= 3; ++force) {
            int32_t *idx = new int32_t[(size_t)T * k];
            float *wt = new float[(size_t)T * k];
            int stats[16] = {0};
            EmuWave wave;
            wave.lds_base = stage_mem;
            g_wave = &wave;
            for (int t = 0; t < T; ++t) {
                std::memset((void *)lds, 0xA5, sizeof *lds);   /* stale LDS contents */
                std::vector<std::thread> th;
                for (int l = 0; l < 64; ++l)
                    th.emplace_back([&, l] {
                        t_lane = l;
                        k3d_select_token(lds, t, rs, bias, W, x, d, E, k, 1, 2.5f, idx, wt, force,
                                         stats, l, nullptr, staged ? stage_mem : nullptr);
                    });
                for (auto &h : th) h.join();
            }
            int mism = 0;
            for (size_t i = 0; i < (size_t)T * k; ++i)
                if (idx[i] != ref_idx[i] || __float_as_uint(wt[i]) != __float_as_uint(ref_w[i]))
                    ++mism;
            /* lanes past E read past the descriptor on purpose; nothing else may */
            const int npl = E <= 256 ? 4 : E <= 512 ? 8 : 16;
            const long deliberate = (long)T * (64L * npl - E);
            std::printf("E=%d k=%d d=%d T=%d ties=%d staged=%d force=%d: rerouted %d, "
                        "recomputed %d, dma %ld, range-checked loads %ld (deliberate %ld), "
                        "mismatches %d\n",
                        E, k, d, T, ties, staged, force, stats[0], stats[1], (long)wave.dma_ops,
                        (long)wave.oob_loads, deliberate, mism);
            if (mism || wave.oob_loads != deliberate) bad = 1;
            delete[] idx;
            delete[] wt;
        }
    delete lds;
    delete[] rs;
    delete[] W;
    delete[] x;
    delete[] bias;
    return bad;
}
