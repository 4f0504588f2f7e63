// Fused ExponentiatedAdam step + SignedConstraint (v1_model_utils/optimizers.py:268-376,
// dense branch :354-376, models.py:419-427): one streaming pass over a weight vector.
#include "glif_internal.h"

namespace glif {

// Per element, in TF's operation order (fp32, separate roundings):
//   m += (g - m) * (1 - beta_1);   v += (g * g - v) * (1 - beta_2)
//   vhat = max(vhat, v) (AMSGrad);  u = vhat or v
//   s = sign(w) with sign(0) = +1;  w = w * exp(((-alpha) * (m / (sqrt(u) + eps))) * s)
//   positive: w = positive ? relu(w) : -relu(-w)   (the variable's constraint, applied
//   by Keras after the update)
__global__ void __launch_bounds__(kBlock)
    k_exp_adam(float *__restrict__ w, float *__restrict__ m, float *__restrict__ v, float *__restrict__ vhat,
               const float *__restrict__ g, const uint8_t *__restrict__ positive, int64_t n, float alpha,
               float one_m_b1, float one_m_b2, float eps) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float gi = g[i];
        float mi = m[i], vi = v[i];
        mi = mi + (gi - mi) * one_m_b1;
        vi = vi + (gi * gi - vi) * one_m_b2;
        m[i] = mi;
        v[i] = vi;
        float u = vi;
        if (vhat) {
            u = fmaxf(vhat[i], vi);
            vhat[i] = u;
        }
        const float ag = mi / (sqrtf(u) + eps);
        const float wi = w[i];
        const float s = wi > 0.0f ? 1.0f : (wi < 0.0f ? -1.0f : 1.0f);
        float wn = wi * expf((-alpha * ag) * s);
        if (positive) wn = positive[i] ? fmaxf(wn, 0.0f) : -fmaxf(-wn, 0.0f);
        w[i] = wn;
    }
}

}  // namespace glif

using namespace glif;

extern "C" int glif_exp_adam(float *w, float *m, float *v, float *vhat, const float *g, const uint8_t *positive,
                             int64_t n, float alpha, float beta_1, float beta_2, float epsilon, void *stream) {
    if (n < 0) return fail(GLIF_EINVAL, "n must be >= 0");
    if (n == 0) return GLIF_OK;
    if (!w || !m || !v || !g) return fail(GLIF_EINVAL, "NULL argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t blocks = std::min<int64_t>((n + kBlock - 1) / kBlock, 8192);
    hipLaunchKernelGGL(k_exp_adam, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, w, m, v, vhat, g,
                       positive, n, alpha, 1.0f - beta_1, 1.0f - beta_2, epsilon);
    GLIF_HIP(hipGetLastError());
    return GLIF_OK;
}
