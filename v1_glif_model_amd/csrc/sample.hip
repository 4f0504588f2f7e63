// Counter-based input sampling on the device: LGN Bernoulli spikes (stim_dataset.py:182-197:
// p = 1 - exp(-rate * dt / 1000), spike where u < p) and background Poisson counts
// (models.py:865-887, lambda = rate * dt / 1000).  The generator is Philox4x32-10 (Salmon et
// al., "Parallel random numbers: as easy as 1, 2, 3", SC 2011): element i of a stream takes
// word i % 4 of the block for counter (i / 4, 0) under key seed, so any element can be drawn
// independently and a stream can be continued at an offset.  TF's stateless streams cannot
// be reproduced; these replace them.
#include "glif_internal.h"

namespace glif {

namespace {
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
}  // namespace

__global__ void __launch_bounds__(kBlock)
    k_bernoulli(const float *__restrict__ p, int64_t n, uint64_t seed, uint64_t offset, uint8_t *__restrict__ out) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = philox_uniform(seed, offset + static_cast<uint64_t>(i)) < p[i] ? 1 : 0;
}

// Sequential inverse CDF in fp32 (counts capped at 255):
//   k = 0, pk = exp(-lam), cdf = pk;  while u > cdf and k < 255: k++, pk *= lam / k, cdf += pk
__global__ void __launch_bounds__(kBlock)
    k_poisson(float lam, float exp_neg_lam, int64_t n, uint64_t seed, uint64_t offset, uint8_t *__restrict__ out) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float u = philox_uniform(seed, offset + static_cast<uint64_t>(i));
        int k = 0;
        float pk = exp_neg_lam, cdf = pk;
        while (u > cdf && k < 255) {
            ++k;
            pk = pk * (lam / static_cast<float>(k));
            cdf = cdf + pk;
        }
        out[i] = static_cast<uint8_t>(k);
    }
}

static dim3 sample_grid(int64_t n) {
    return dim3(static_cast<unsigned>(std::min<int64_t>((n + kBlock - 1) / kBlock, 8192)));
}

}  // namespace glif

using namespace glif;

extern "C" {

int glif_sample_bernoulli(const float *p, int64_t n, uint64_t seed, uint64_t offset, uint8_t *out, void *stream) {
    if (n < 0) return fail(GLIF_EINVAL, "n must be >= 0");
    if (n == 0) return GLIF_OK;
    if (!p || !out) return fail(GLIF_EINVAL, "NULL argument");
    hipLaunchKernelGGL(k_bernoulli, sample_grid(n), dim3(kBlock), 0, static_cast<hipStream_t>(stream), p, n, seed,
                       offset, out);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

int glif_sample_poisson(float lam, float exp_neg_lam, int64_t n, uint64_t seed, uint64_t offset, uint8_t *out,
                        void *stream) {
    if (n < 0 || !(lam >= 0.0f)) return fail(GLIF_EINVAL, "n must be >= 0 and lambda >= 0");
    if (n == 0) return GLIF_OK;
    if (!out) return fail(GLIF_EINVAL, "NULL argument");
    hipLaunchKernelGGL(k_poisson, sample_grid(n), dim3(kBlock), 0, static_cast<hipStream_t>(stream), lam,
                       exp_neg_lam, n, seed, offset, out);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

}  // extern "C"
