// fixed_ppo.hip — the reference's fixed-shape PPO operators (ppo.hpp:65-181,
// 310-324) as batched kernels over caller arrays: actor and critic forward,
// Gaussian log-probability, per-sample clipped-surrogate loss and derivatives,
// and Adam.  They back the mdn_op_* entry points that stand in for the header
// functions a host harness calls (fixed_ppo::actor_forward, ...); the training
// path uses the fused kernels of ppo.hip and large.hip.
//
// The arithmetic is the canonical form the rest of the library and the CPU
// oracle share: dot products are fma chains from the bias with inputs in
// ascending order, tanh/exp are this project's own (mdnav_math.h), divisions
// and square roots are correctly rounded.
#include <hip/hip_runtime.h>

#include "kernel_args.h"
#include "mdnav_math.h"
#include "mdnav_types.h"

namespace fppo {
using namespace mdn;

constexpr float LOG_TWO_PI = 1.8378770664093453f;
constexpr uint32_t MAX_IN = 1024, MAX_HIDDEN = 8192;

// One workgroup per row: the row's inputs in LDS, hidden units strided over
// the 256 threads, then one thread per output (means, or the value) runs the
// output chain over the hidden units in order.  Layouts (ppo.hpp:35-45):
// W1[H][D] at 0, b1[H], W2[O][H], b2[O]; the actor (O = 4) then has
// log_std[4], the critic (O = 1) nothing.
__global__ __launch_bounds__(256) void mlp_forward_kernel(const float* __restrict__ w, const float* __restrict__ x,
                                                          uint32_t D, uint32_t H, uint32_t O, uint32_t prior,
                                                          uint64_t B, float* __restrict__ hidden,
                                                          float* __restrict__ out) {
    __shared__ float s_x[MAX_IN];
    __shared__ float s_h[MAX_HIDDEN];
    const uint64_t row = blockIdx.x;
    if (row >= B) return;  // the whole workgroup leaves together
    const uint32_t t = threadIdx.x;
    const float* xr = x + row * D;
    for (uint32_t i = t; i < D; i += 256) s_x[i] = xr[i];
    __syncthreads();
    const float* b1 = w + size_t(H) * D;
    for (uint32_t h = t; h < H; h += 256) {
        const float* wr = w + size_t(h) * D;
        float z = b1[h];
        for (uint32_t i = 0; i < D; i++) z = fma_f(wr[i], s_x[i], z);
        const float a = tanh_f(z);
        s_h[h] = a;
        if (hidden) hidden[row * H + h] = a;
    }
    __syncthreads();
    if (t < O) {
        const float* w2 = b1 + H + size_t(t) * H;
        float z = b1[H + size_t(O) * H + t];
        for (uint32_t h = 0; h < H; h++) z = fma_f(w2[h], s_h[h], z);
        // geometry prior (ppo.hpp:30-34, 77): the hint inputs join the first three means
        if (prior && t < 3) z += s_x[D - 3 + t];
        out[row * O + t] = z;
    }
}

__device__ __forceinline__ float log_prob(const float* a, const float* m, const float* ls) {
    float r = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) {
        const float inv_std = exp_f(-ls[q]);
        const float d = (a[q] - m[q]) * inv_std;
        r += -0.5f * (d * d + 2.0f * ls[q] + LOG_TWO_PI);
    }
    return r;
}

// ppo.hpp:95-103; log_std is shared ([4], stride 0) or per row ([B][4]).
__global__ __launch_bounds__(256) void log_prob_kernel(const float* __restrict__ act, const float* __restrict__ mean,
                                                       const float* __restrict__ log_std, uint32_t ls_stride,
                                                       uint64_t B, float* __restrict__ out) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= B) return;
    out[i] = log_prob(act + 4 * i, mean + 4 * i, log_std + ls_stride * i);
}

// ppo.hpp:144-181 per row: d_mean[4], d_log_std[4], d_value and the losses
// [policy, value, entropy, ratio].
__global__ __launch_bounds__(256) void loss_grad_kernel(fppo_loss_args a) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= a.b) return;
    const float* act = a.actions + 4 * i;
    const float* mean = a.means + 4 * i;
    const float* ls = a.log_std + a.ls_stride * i;
    const float adv = a.advantages[i];
    const float value = a.values[i], target = a.returns[i];
    const float logp = log_prob(act, mean, ls);
    const float raw = logp - a.old_logp[i];
    const float ratio = exp_f(clamp_f(raw, -20.0f, 20.0f));
    const float clipped = clamp_f(ratio, 1.0f - a.clip, 1.0f + a.clip);
    const float chosen = min_f(ratio * adv, clipped * adv);
    const bool in_range = raw >= -20.0f && raw <= 20.0f;
    const bool active = in_range && (adv >= 0.0f ? ratio <= 1.0f + a.clip : ratio >= 1.0f - a.clip);
    const float scale = 1.0f / max_f(a.batch_size, 1.0f);
    float entropy = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) {
        const float inv_var = exp_f(-2.0f * ls[q]);
        const float diff = act[q] - mean[q];
        float dm = 0.0f, dl = 0.0f;
        if (active) {
            const float dlogp = -ratio * adv * scale;
            dm = dlogp * diff * inv_var;
            dl = dlogp * (diff * diff * inv_var - 1.0f);
        }
        dl -= a.ecoef * scale;
        entropy += -a.ecoef * (ls[q] + 0.5f * (1.0f + LOG_TWO_PI)) * scale;
        a.d_mean[4 * i + q] = dm;
        a.d_log_std[4 * i + q] = dl;
    }
    a.d_value[i] = a.vcoef * (value - target) * scale;
    a.losses[4 * i] = -chosen * scale;
    a.losses[4 * i + 1] = 0.5f * a.vcoef * (value - target) * (value - target) * scale;
    a.losses[4 * i + 2] = entropy;
    a.losses[4 * i + 3] = ratio;
}

// ppo.hpp:310-324 elementwise; c1, c2 = 1 - beta^step from the host.
__global__ __launch_bounds__(256) void adam_op_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                      float* __restrict__ m, float* __restrict__ v, uint64_t n,
                                                      float lr, float b1, float b2, float eps, float wd, float c1,
                                                      float c2) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const float gi = g[i] + wd * p[i];
    const float mi = b1 * m[i] + (1.0f - b1) * gi;
    const float vi = b2 * v[i] + (1.0f - b2) * gi * gi;
    m[i] = mi;
    v[i] = vi;
    p[i] -= lr * (mi / c1) / (sqrt_f(vi / c2) + eps);
}

}  // namespace fppo

extern "C" {

hipError_t fppo_launch_forward(const float* w, const float* x, uint32_t D, uint32_t H, uint32_t O, uint32_t prior,
                               uint64_t B, float* hidden, float* out, hipStream_t st) {
    if (B == 0) return hipSuccess;
    if (D == 0 || D > fppo::MAX_IN || H == 0 || H > fppo::MAX_HIDDEN || O == 0 || O > 256 || B > 0x7fffffffull ||
        (prior && D < 3))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(fppo::mlp_forward_kernel, dim3(uint32_t(B)), dim3(256), 0, st, w, x, D, H, O, prior, B, hidden,
                       out);
    return hipGetLastError();
}

hipError_t fppo_launch_log_prob(const float* act, const float* mean, const float* log_std, uint32_t ls_stride,
                                uint64_t B, float* out, hipStream_t st) {
    if (B == 0) return hipSuccess;
    hipLaunchKernelGGL(fppo::log_prob_kernel, dim3(uint32_t((B + 255) / 256)), dim3(256), 0, st, act, mean, log_std,
                       ls_stride, B, out);
    return hipGetLastError();
}

hipError_t fppo_launch_loss_grad(const fppo_loss_args* a, hipStream_t st) {
    if (a->b == 0) return hipSuccess;
    hipLaunchKernelGGL(fppo::loss_grad_kernel, dim3(uint32_t((a->b + 255) / 256)), dim3(256), 0, st, *a);
    return hipGetLastError();
}

hipError_t fppo_launch_adam(float* p, const float* g, float* m, float* v, uint64_t n, float lr, float b1, float b2,
                            float eps, float wd, float c1, float c2, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fppo::adam_op_kernel, dim3(uint32_t((n + 255) / 256)), dim3(256), 0, st, p, g, m, v, n, lr, b1,
                       b2, eps, wd, c1, c2);
    return hipGetLastError();
}

}  // extern "C"
