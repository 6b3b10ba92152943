/* k3s_synth.c - seeded synthetic tensors (host side). The same (seed, stream, index)
 * gives the same byte on the host and on the device (k3s_hash.h), so a CPU check can
 * regenerate exactly the experts a GPU run used. */
#include "k3g_kernels.h"
#include "k3s_hash.h"

#include <math.h>
#include <string.h>

uint8_t k3s_byte(uint64_t seed, uint64_t stream, uint64_t i)
{
    return k3s_byte_at(seed, stream, i);
}

void k3s_fill_bytes(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream, uint64_t first)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > (1u << 20))
#endif
    for (int64_t i = 0; i < (int64_t)n; i++) dst[i] = k3s_byte_at(seed, stream, first + (uint64_t)i);
}

void k3s_fill_scales(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream, uint64_t first,
                     int lo, int hi)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > (1u << 20))
#endif
    for (int64_t i = 0; i < (int64_t)n; i++)
        dst[i] = k3s_scale_byte(seed, stream, first + (uint64_t)i, lo, hi);
}

static float bf16_rne(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) != 0x7F800000u) u += 0x7FFFu + ((u >> 16) & 1u);
    u &= 0xFFFF0000u;
    memcpy(&f, &u, 4);
    return f;
}

/* Box-Muller: element 2m uses r*cos(theta), element 2m+1 r*sin(theta), with
 * u1 = (word(2m) >> 11 + 1) * 2^-53 in (0, 1] and u2 = (word(2m+1) >> 11) * 2^-53. */
void k3s_fill_normal(float *dst, size_t n, uint64_t seed, uint64_t stream, uint64_t first,
                     float mean, float std, int bf16_round)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (n > (1u << 18))
#endif
    for (int64_t ii = 0; ii < (int64_t)n; ii++) {
        const uint64_t i = first + (uint64_t)ii;
        const uint64_t m = i >> 1;
        const double u1 = ((double)(k3s_word(seed, stream, 2 * m) >> 11) + 1.0) * 0x1p-53;
        const double u2 = (double)(k3s_word(seed, stream, 2 * m + 1) >> 11) * 0x1p-53;
        const double r = sqrt(-2.0 * log(u1));
        const double th = 6.283185307179586476925286766559 * u2;
        const double z = (i & 1) ? r * sin(th) : r * cos(th);
        const float v = (float)((double)mean + (double)std * z);
        dst[ii] = bf16_round ? bf16_rne(v) : v;
    }
}

int k3g_fill_bytes(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream, uint64_t first,
                   void *hstream)
{
    return k3k_fill_bytes(dst, n, seed, stream, first, (hipStream_t)hstream);
}

int k3g_fill_scales(uint8_t *dst, size_t n, uint64_t seed, uint64_t stream, uint64_t first,
                    int lo, int hi, void *hstream)
{
    return k3k_fill_scales(dst, n, seed, stream, first, lo, hi, (hipStream_t)hstream);
}
