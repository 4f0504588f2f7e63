// Rate-distribution loss of the cell's spikes (SpikeRateDistributionTarget,
// loss_functions.py:782-889, through compute_spike_rate_target_loss :634-664,
// compute_spike_rate_distribution_loss :666-681 and huber_quantile_loss :626-632):
//
//   rate[n]   = (sum over the window of z[t][b][n]) / S            (S = window ticks x B)
//   per population k (n_k selected neurons, sorted targets tgt_k):
//     sorted  = ascending sort of the population's rates, ties in shuffled order
//     u_r     = sorted_r - tgt_k[r],  tau_r = (r + 1) / n_k
//     h(u)    = |u| <= kappa ? |tau - [u <= 0]| / (2 kappa) * u^2
//                            : |tau - [u <= 0]| * (|u| - kappa / 2)
//   loss      = rate_cost * (sum_k sum_r h(u_r)) / sum_k n_k
//
// Rates are exact integer counts over S, so the sort runs on integer keys:
//   key = (k * (S + 1) + count) << 32 | tie
// with tie a Philox4x32-10 word (a uniformly random order among equal rates, the
// reference's tf.random.shuffle before its sort) or 0 (input order: the caller's own
// shuffle).  One stable LSD radix sort over the whole selection (hipCUB) then yields every
// population's sorted segment in place.  The gradient of each sorted position goes back to
// the neuron that holds it: gz_neuron[n] += dL/drate[n] / S, the dL/dz the cell's backward
// broadcasts over the window.  The loss sum runs in a fixed order (deterministic).
#include <hipcub/hipcub.hpp>

#include "glif_internal.h"
#include "philox.h"

namespace glif {

namespace {
constexpr int kMaxPop = 64;
constexpr int kLossParts = 256;   // workgroups of the loss pass = partial sums

struct RateArgs {
    const int32_t *count;   // [rows][N]
    int32_t rows, N;
    int32_t S;              // samples per rate (window ticks x batch)
    uint32_t span;          // S + 1
    const int32_t *ids;     // [n_sel]
    int64_t n_sel;
    int32_t n_pop;
    int32_t pop_ptr[kMaxPop + 1];
    const float *targets;   // [n_sel], each population's segment ascending
    float kappa, rate_cost;
    int32_t shuffle;
    uint64_t seed, offset;
    uint64_t *key_in, *key_out;
    int32_t *val_in, *val_out;
    float *partial;         // [kLossParts]
    uint32_t *bad;          // ids outside [0, N) seen
    float *gz_neuron;
    float *loss;
};

// population of selection position i: the largest k with pop_ptr[k] <= i (empty
// populations share their start with the next one, which is the one holding i)
__device__ inline int pop_of(const RateArgs &a, int64_t i) {
    int lo = 0, hi = a.n_pop - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (a.pop_ptr[mid] <= i) lo = mid; else hi = mid - 1;
    }
    return lo;
}

__global__ void __launch_bounds__(kBlock) k_rate_keys(RateArgs a) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= a.n_sel) return;
    const int k = pop_of(a, i);
    const int32_t id = a.ids[i];
    uint32_t c = 0;
    if (id >= 0 && id < a.N) {
        for (int r = 0; r < a.rows; ++r) c += static_cast<uint32_t>(a.count[static_cast<int64_t>(r) * a.N + id]);
        if (c > static_cast<uint32_t>(a.S)) c = static_cast<uint32_t>(a.S), atomicOr(a.bad, 2u);
    } else {
        atomicOr(a.bad, 1u);
    }
    const uint64_t hi = static_cast<uint64_t>(k) * a.span + c;
    const uint32_t tie = a.shuffle ? philox_word(a.seed, a.offset + static_cast<uint64_t>(i)) : 0u;
    a.key_in[i] = hi << 32 | tie;
    a.val_in[i] = static_cast<int32_t>(i);
}

// One loss term per sorted position, in the reference's fp32 operation order (the
// library builds without contraction); the per-thread sums (fixed strides) and the workgroup tree give a
// deterministic partial per workgroup.
__global__ void __launch_bounds__(kBlock) k_rate_terms(RateArgs a) {
    __shared__ float red[kBlock];
    const float kappa = a.kappa, two_kappa = 2.0f * a.kappa, half_kappa = 0.5f * a.kappa;
    const float g = a.rate_cost / static_cast<float>(a.n_sel);   // dL/dh
    const float S = static_cast<float>(a.S);
    float acc = 0.0f;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < a.n_sel; p += stride) {
        const uint64_t hi = a.key_out[p] >> 32;
        const int k = static_cast<int>(hi / a.span);
        const uint32_t c = static_cast<uint32_t>(hi - static_cast<uint64_t>(k) * a.span);
        const float rate = static_cast<float>(c) / S;
        const int32_t p0 = a.pop_ptr[k], nk = a.pop_ptr[k + 1] - p0;
        const float tau = static_cast<float>(static_cast<int32_t>(p) - p0 + 1) / static_cast<float>(nk);
        const float u = rate - a.targets[p];
        const float au = fabsf(u);
        const float num = fabsf(tau - (u <= 0.0f ? 1.0f : 0.0f));
        float h, dh;
        if (au <= kappa) {
            h = num / two_kappa * (u * u);
            dh = (g * (num / two_kappa)) * (2.0f * u);
        } else {
            h = num * (au - half_kappa);
            dh = (g * num) * (u > 0.0f ? 1.0f : -1.0f);
        }
        acc = acc + h;
        const int32_t id = a.ids[a.val_out[p]];
        if (id >= 0 && id < a.N) a.gz_neuron[id] = a.gz_neuron[id] + dh / S;
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = kBlock / 2; w > 0; w >>= 1) {
        if (static_cast<int>(threadIdx.x) < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) a.partial[blockIdx.x] = red[0];
}

__global__ void __launch_bounds__(kBlock) k_rate_final(RateArgs a, int parts) {
    __shared__ float red[kBlock];
    float acc = 0.0f;
    for (int i = threadIdx.x; i < parts; i += kBlock) acc = acc + a.partial[i];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = kBlock / 2; w > 0; w >>= 1) {
        if (static_cast<int>(threadIdx.x) < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const float loss = red[0] / static_cast<float>(a.n_sel) * a.rate_cost;
        a.loss[0] = *a.bad ? __builtin_nanf("") : loss;
    }
}

// Mean-squared firing-rate error (the benchmark's configuration-2 loss): per neuron
// rbar = count / S, diff = rbar - target; loss = sum diff^2 / N in a fixed order,
// gz_neuron += diff * scale with scale = 2 / (N * S) (the per-tick dL/dz).
__global__ void __launch_bounds__(kBlock)
    k_rate_mse(const int32_t *__restrict__ count, int32_t rows, int32_t N, float S, const float *__restrict__ tgt,
               float scale, float *__restrict__ gz, float *__restrict__ partial) {
    __shared__ float red[kBlock];
    float acc = 0.0f;
    for (int32_t n = blockIdx.x * blockDim.x + threadIdx.x; n < N; n += gridDim.x * blockDim.x) {
        int32_t c = 0;
        for (int32_t r = 0; r < rows; ++r) c += count[static_cast<int64_t>(r) * N + n];
        const float diff = static_cast<float>(c) / S - tgt[n];
        acc = acc + diff * diff;
        gz[n] = gz[n] + diff * scale;
    }
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = kBlock / 2; w > 0; w >>= 1) {
        if (static_cast<int>(threadIdx.x) < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) partial[blockIdx.x] = red[0];
}

__global__ void __launch_bounds__(kBlock) k_rate_mse_final(const float *__restrict__ partial, int parts, float N,
                                                            float *__restrict__ loss) {
    __shared__ float red[kBlock];
    float acc = 0.0f;
    for (int i = threadIdx.x; i < parts; i += kBlock) acc = acc + partial[i];
    red[threadIdx.x] = acc;
    __syncthreads();
    for (int w = kBlock / 2; w > 0; w >>= 1) {
        if (static_cast<int>(threadIdx.x) < w) red[threadIdx.x] = red[threadIdx.x] + red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) loss[0] = red[0] / N;
}

int bits_for(uint64_t v) {   // bits needed to hold values < v
    int b = 0;
    while (b < 64 && (uint64_t(1) << b) < v) ++b;
    return b;
}

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

int sort_temp_bytes(int64_t n, int begin_bit, int end_bit, size_t *bytes) {
    size_t tb = 0;
    GLIF_HIP(hipcub::DeviceRadixSort::SortPairs(nullptr, tb, static_cast<const uint64_t *>(nullptr),
                                                static_cast<uint64_t *>(nullptr),
                                                static_cast<const int32_t *>(nullptr),
                                                static_cast<int32_t *>(nullptr), static_cast<int>(n), begin_bit,
                                                end_bit, hipStream_t(nullptr)));
    *bytes = tb;
    return GLIF_OK;
}

size_t fixed_bytes(int64_t n) {
    const size_t un = static_cast<size_t>(n);
    return 2 * align256(un * 8) + 2 * align256(un * 4) + align256(kLossParts * 4) + 256;
}
}  // namespace

}  // namespace glif

using namespace glif;

extern "C" {

size_t glif_rate_loss_workspace(int64_t n_sel) {
    if (n_sel <= 0 || n_sel >= INT32_MAX) return 0;
    size_t tb = 0;
    if (sort_temp_bytes(n_sel, 0, 64, &tb)) return 0;
    return fixed_bytes(n_sel) + align256(tb);
}

int glif_rate_dist_loss(const int32_t *count, int32_t count_rows, int32_t n_neurons, int32_t n_samples,
                        const int32_t *ids, const int32_t *pop_ptr, int32_t n_pop, const float *targets,
                        float kappa, float rate_cost, int32_t shuffle, uint64_t seed, uint64_t offset,
                        float *loss_out, float *gz_neuron, void *ws, size_t ws_bytes, void *stream) {
    if (!count || !ids || !pop_ptr || !targets || !loss_out || !gz_neuron) return fail(GLIF_EINVAL, "NULL argument");
    if (count_rows <= 0 || n_neurons <= 0) return fail(GLIF_EINVAL, "count_rows and n_neurons must be > 0");
    if (n_pop <= 0 || n_pop > kMaxPop) return fail(GLIF_EINVAL, "n_pop must be in [1, 64]");
    if (n_samples <= 0 || n_samples >= (1 << 22))
        return fail(GLIF_EINVAL, "n_samples must be in [1, 2^22) (rates are exact count / n_samples)");
    if (!(kappa > 0.0f)) return fail(GLIF_EINVAL, "kappa must be > 0");
    if (pop_ptr[0] != 0) return fail(GLIF_EINVAL, "pop_ptr[0] must be 0");
    for (int k = 0; k < n_pop; ++k)
        if (pop_ptr[k + 1] < pop_ptr[k]) return fail(GLIF_EINVAL, "pop_ptr must be non-decreasing");
    const int64_t n_sel = pop_ptr[n_pop];
    if (n_sel <= 0) return fail(GLIF_EINVAL, "no neuron selected");
    const uint64_t span = static_cast<uint64_t>(n_samples) + 1;
    const int hi_bits = bits_for(static_cast<uint64_t>(n_pop) * span);
    if (hi_bits > 32) return fail(GLIF_ERANGE, "n_pop * (n_samples + 1) must be < 2^32");
    const size_t need = glif_rate_loss_workspace(n_sel);
    if (!need) return fail(GLIF_EINVAL, "selection too large");
    if (!ws || ws_bytes < need) return fail(GLIF_ENOMEM, "workspace too small");
    const int begin_bit = shuffle ? 0 : 32, end_bit = 32 + hi_bits;
    size_t temp = 0;
    if (int rc = sort_temp_bytes(n_sel, begin_bit, end_bit, &temp)) return rc;
    if (fixed_bytes(n_sel) + align256(temp) > ws_bytes) return fail(GLIF_ENOMEM, "workspace too small for the sort");

    hipStream_t s = static_cast<hipStream_t>(stream);
    RateArgs a{};
    a.count = count;
    a.rows = count_rows;
    a.N = n_neurons;
    a.S = n_samples;
    a.span = static_cast<uint32_t>(span);
    a.ids = ids;
    a.n_sel = n_sel;
    a.n_pop = n_pop;
    for (int k = 0; k <= n_pop; ++k) a.pop_ptr[k] = pop_ptr[k];
    a.targets = targets;
    a.kappa = kappa;
    a.rate_cost = rate_cost;
    a.shuffle = shuffle;
    a.seed = seed;
    a.offset = offset;
    a.gz_neuron = gz_neuron;
    a.loss = loss_out;
    char *p = static_cast<char *>(ws);
    const size_t un = static_cast<size_t>(n_sel);
    a.key_in = reinterpret_cast<uint64_t *>(p);  p += align256(un * 8);
    a.key_out = reinterpret_cast<uint64_t *>(p); p += align256(un * 8);
    a.val_in = reinterpret_cast<int32_t *>(p);   p += align256(un * 4);
    a.val_out = reinterpret_cast<int32_t *>(p);  p += align256(un * 4);
    a.partial = reinterpret_cast<float *>(p);    p += align256(kLossParts * 4);
    a.bad = reinterpret_cast<uint32_t *>(p);     p += 256;
    void *sort_tmp = p;

    if (int rc = launch_fill_u32(a.bad, 0u, 1, s)) return rc;
    const unsigned blocks = static_cast<unsigned>((n_sel + kBlock - 1) / kBlock);
    hipLaunchKernelGGL(k_rate_keys, dim3(blocks), dim3(kBlock), 0, s, a);
    GLIF_HIP(hipGetLastError());
    GLIF_HIP(hipcub::DeviceRadixSort::SortPairs(sort_tmp, temp, a.key_in, a.key_out, a.val_in, a.val_out,
                                                static_cast<int>(n_sel), begin_bit, end_bit, s));
    const int parts = static_cast<int>(std::min<int64_t>(kLossParts, blocks));
    hipLaunchKernelGGL(k_rate_terms, dim3(parts), dim3(kBlock), 0, s, a);
    GLIF_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_rate_final, dim3(1), dim3(kBlock), 0, s, a, parts);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

size_t glif_rate_mse_workspace(void) { return kLossParts * sizeof(float); }

int glif_rate_mse_loss(const int32_t *count, int32_t count_rows, int32_t n_neurons, int32_t n_samples,
                       const float *targets, float *loss_out, float *gz_neuron, void *ws, size_t ws_bytes,
                       void *stream) {
    if (!count || !targets || !loss_out || !gz_neuron) return fail(GLIF_EINVAL, "NULL argument");
    if (count_rows <= 0 || n_neurons <= 0 || n_samples <= 0)
        return fail(GLIF_EINVAL, "count_rows, n_neurons and n_samples must be > 0");
    if (!ws || ws_bytes < glif_rate_mse_workspace()) return fail(GLIF_ENOMEM, "workspace too small");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int parts = std::min<int>(kLossParts, (n_neurons + kBlock - 1) / kBlock);
    const float scale = static_cast<float>(2.0 / (static_cast<double>(n_neurons) * n_samples));
    hipLaunchKernelGGL(k_rate_mse, dim3(parts), dim3(kBlock), 0, s, count, count_rows, n_neurons,
                       static_cast<float>(n_samples), targets, scale, gz_neuron, static_cast<float *>(ws));
    GLIF_HIP(hipGetLastError());
    hipLaunchKernelGGL(k_rate_mse_final, dim3(1), dim3(kBlock), 0, s, static_cast<const float *>(ws), parts,
                       static_cast<float>(n_neurons), loss_out);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}

}  // extern "C"
