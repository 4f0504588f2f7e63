// Counter-based input sampling on the device: LGN Bernoulli spikes (stim_dataset.py:182-197:
// p = 1 - exp(-rate * dt / 1000), spike where u < p) and background Poisson counts
// (models.py:865-887, lambda = rate * dt / 1000).  The generator is Philox4x32-10 (Salmon et
// al., "Parallel random numbers: as easy as 1, 2, 3", SC 2011): element i of a stream takes
// word i % 4 of the block for counter (i / 4, 0) under key seed, so any element can be drawn
// independently and a stream can be continued at an offset.  TF's stateless streams cannot
// be reproduced; these replace them.
#include "glif_internal.h"
#include "philox.h"

namespace glif {

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
