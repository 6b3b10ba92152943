/* pick_audit.cpp - runs the router's many-token selection (k3d_pick_token in k3g_select.h,
 * the code k_router_pick runs after the bounded bf16 logits) on the host, one emulated
 * 64-lane wave per token, under AddressSanitizer and the array-bounds checker, and
 * compares every token's routing bit for bit with the oracle's k3_router restatement
 * (test infrastructure).
 *
 * The approximate logits are placed adversarially inside their bound: the exact fp64 sum
 * moved by 0.9 of the bound, up for odd experts and down for even ones, then rounded to
 * float as the GPU's logits are. mode 0 takes the bound the GPU path uses for this d
 * (about 2e-4 ||w|| ||x||: many candidates per token); mode 1 a bound 200 times tighter
 * (most tokens with exactly k candidates). Inputs can carry duplicated router rows and
 * tied biases (exact ties in the choice scores).
 *
 * usage: pick_audit E k d T ties seed mode   (one line per forced mode; exit 1 on a
 *                                             mismatch or a counted bound violation) */
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

int main(int argc, char **argv)
{
    if (argc != 8) {
        std::fprintf(stderr, "usage: pick_audit E k d T ties seed mode\n");
        return 2;
    }
    const int E = std::atoi(argv[1]), k = std::atoi(argv[2]), d = std::atoi(argv[3]);
    const int T = std::atoi(argv[4]), ties = std::atoi(argv[5]);
    const unsigned seed = (unsigned)std::atoi(argv[6]);
    const int mode = std::atoi(argv[7]);
    if (E < 16 || E > K3G_MAX_E || E % 16 || k < 1 || k > 64 || d < 256 || d % 256 || T < 1)
        return 2;

    std::mt19937_64 rng(seed);
    std::normal_distribution<float> nw(0.0f, 0.02f), nx(0.0f, 1.0f), nb(0.0f, 0.01f);
    float *W = new float[(size_t)E * d];
    float *x = new float[(size_t)T * d];
    float *bias = new float[E];
    for (size_t i = 0; i < (size_t)E * d; ++i) W[i] = nw(rng);
    for (size_t i = 0; i < (size_t)T * d; ++i) x[i] = nx(rng);
    for (int e = 0; e < E; ++e) bias[e] = nb(rng);
    if (ties) {
        for (int e = 1; e < E; e += 3) {
            std::memcpy(W + (size_t)e * d, W + (size_t)(e - 1) * d, (size_t)d * 4);
            bias[e] = bias[e - 1];
        }
    }
    /* the GPU path's bound for this d (twice the analysed error), or a tighter one */
    const double gpu_b = 2.0 * (3.02 * 0x1p-16 + 1.02 * (400.0 + d / 128) * 0x1p-23);
    const double nround = mode == 0 ? gpu_b / (1.01 * 0x1p-53) : 1e10;

    float *part = new float[(size_t)T * E];
    float *wn2 = new float[E];
    float *xn2 = new float[T];
    for (int e = 0; e < E; ++e) {
        double s = 0.0;
        for (int i = 0; i < d; ++i) s += (double)W[(size_t)e * d + i] * W[(size_t)e * d + i];
        wn2[e] = (float)s;
    }
    for (int t = 0; t < T; ++t) {
        double s = 0.0;
        for (int i = 0; i < d; ++i) s += (double)x[(size_t)t * d + i] * x[(size_t)t * d + i];
        xn2[t] = (float)s;
    }
    for (int t = 0; t < T; ++t)
        for (int e = 0; e < E; ++e) {
            const float *w = W + (size_t)e * d, *xt = x + (size_t)t * d;
            double s = 0.0;
            for (int i = 0; i < d; ++i) s += (double)w[i] * xt[i];
            const double B0 = nround * 0x1p-53 * 1.01 * std::sqrt((double)wn2[e]) *
                              std::sqrt((double)xn2[t]);
            part[(size_t)t * E + e] = (float)(s + ((e & 1) ? 0.9 : -0.9) * B0);
        }

    std::vector<int> ref_idx((size_t)T * k);
    std::vector<float> ref_w((size_t)T * k);
    for (int t = 0; t < T; ++t)
        ork3_router(&ref_idx[(size_t)t * k], &ref_w[(size_t)t * k], x + (size_t)t * d, W, bias,
                    d, E, k, 1, 2.5f);

    int *cand = new int[K3G_MAX_E];
    float *cch = new float[K3G_MAX_E], *csc = new float[K3G_MAX_E];
    int bad = 0;
    for (int force : {0, 2, 3}) {
        int32_t *idx = new int32_t[(size_t)T * k];
        float *wt = new float[(size_t)T * k];
        long extra = 0, open = 0, viol = 0;
        EmuWave wave;
        g_wave = &wave;
        for (int t = 0; t < T; ++t) {
            std::memset(cand, 0xA5, K3G_MAX_E * sizeof(int));      /* stale LDS contents */
            std::memset(cch, 0xA5, K3G_MAX_E * sizeof(float));
            std::memset(csc, 0xA5, K3G_MAX_E * sizeof(float));
            int cnt[64][3];
            std::vector<std::thread> th;
            for (int l = 0; l < 64; ++l)
                th.emplace_back([&, l] {
                    t_lane = l;
                    if (E <= 256)
                        k3d_pick_token<4>(t, part, xn2, wn2, bias, W, x, d, E, k, 1, 2.5f, idx,
                                          wt, force, nround, cand, cch, csc, l, cnt[l]);
                    else if (E <= 512)
                        k3d_pick_token<8>(t, part, xn2, wn2, bias, W, x, d, E, k, 1, 2.5f, idx,
                                          wt, force, nround, cand, cch, csc, l, cnt[l]);
                    else
                        k3d_pick_token<16>(t, part, xn2, wn2, bias, W, x, d, E, k, 1, 2.5f, idx,
                                           wt, force, nround, cand, cch, csc, l, cnt[l]);
                });
            for (auto &h : th) h.join();
            extra += cnt[0][0];
            open += cnt[0][1];
            viol += cnt[0][2];
        }
        int mism = 0;
        for (size_t i = 0; i < (size_t)T * k; ++i)
            if (idx[i] != ref_idx[i] || __float_as_uint(wt[i]) != __float_as_uint(ref_w[i]))
                ++mism;
        std::printf("E=%d k=%d d=%d T=%d ties=%d mode=%d force=%d: extra %ld, open %ld, "
                    "violations %ld, mismatches %d\n",
                    E, k, d, T, ties, mode, force, extra, open, viol, mism);
        if (mism || viol) bad = 1;
        delete[] idx;
        delete[] wt;
    }
    delete[] cand;
    delete[] cch;
    delete[] csc;
    delete[] part;
    delete[] wn2;
    delete[] xn2;
    delete[] W;
    delete[] x;
    delete[] bias;
    return bad;
}
