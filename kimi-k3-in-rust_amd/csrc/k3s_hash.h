/* k3s_hash.h - counter-based hash behind the seeded synthetic data. Shared verbatim by
 * the C99 host fills and the HIP device fills, so any byte of a generated tensor can be
 * regenerated on either side from (seed, stream, index) alone. Integer-only: host and
 * device agree bit for bit. */
#ifndef K3S_HASH_H
#define K3S_HASH_H

#include <stdint.h>

#ifdef __HIPCC__
#define K3S_HD __host__ __device__ __forceinline__
#else
#define K3S_HD static inline
#endif

/* splitmix64 finaliser (Steele, Lea, Flood, "Fast splittable pseudorandom number
 * generators", OOPSLA 2014) */
K3S_HD uint64_t k3s_mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* 64-bit word w of stream `stream` under `seed` */
K3S_HD uint64_t k3s_word(uint64_t seed, uint64_t stream, uint64_t w)
{
    const uint64_t key = k3s_mix64(seed + 0x9E3779B97F4A7C15ull * (stream + 1));
    return k3s_mix64(key + 0x9E3779B97F4A7C15ull * (w + 1));
}

K3S_HD uint8_t k3s_byte_at(uint64_t seed, uint64_t stream, uint64_t i)
{
    return (uint8_t)(k3s_word(seed, stream, i >> 3) >> (8 * (i & 7)));
}

/* E8M0 byte 127 + v with v uniform over [lo, hi] (16 bits of hash per element,
 * multiply-shift range reduction). */
K3S_HD uint8_t k3s_scale_byte(uint64_t seed, uint64_t stream, uint64_t i, int lo, int hi)
{
    const uint32_t u = (uint32_t)(k3s_word(seed, stream, i >> 2) >> (16 * (i & 3))) & 0xFFFFu;
    const uint32_t span = (uint32_t)(hi - lo + 1);
    return (uint8_t)(127 + lo + (int)((u * span) >> 16));
}

#endif /* K3S_HASH_H */
