// Philox4x32-10 (Salmon et al., "Parallel random numbers: as easy as 1, 2, 3", SC 2011),
// counter-based: element i of the stream under key `seed` is word i % 4 of the block for
// counter (i / 4, 0), so any element is drawn independently of the others.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace glif {

constexpr uint32_t kPhM0 = 0xD2511F53u, kPhM1 = 0xCD9E8D57u;  // round multipliers
constexpr uint32_t kPhW0 = 0x9E3779B9u, kPhW1 = 0xBB67AE85u;  // key increments (Weyl)

__device__ inline uint32_t philox_word(uint64_t seed, uint64_t i) {
    const uint64_t blk = i >> 2;
    uint32_t c0 = static_cast<uint32_t>(blk), c1 = static_cast<uint32_t>(blk >> 32), c2 = 0u, c3 = 0u;
    uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t lo0 = kPhM0 * c0, hi0 = __umulhi(kPhM0, c0);
        const uint32_t lo1 = kPhM1 * c2, hi1 = __umulhi(kPhM1, c2);
        const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
        c0 = n0;
        c1 = lo1;
        c2 = n2;
        c3 = lo0;
        k0 += kPhW0;
        k1 += kPhW1;
    }
    const uint32_t w = static_cast<uint32_t>(i & 3u);
    return w == 0 ? c0 : (w == 1 ? c1 : (w == 2 ? c2 : c3));
}

// fp32 in [0, 1): the word's top 24 bits times 2^-24 (exact)
__device__ inline float philox_uniform(uint64_t seed, uint64_t i) {
    return static_cast<float>(philox_word(seed, i) >> 8) * 5.9604644775390625e-08f;
}

}  // namespace glif
