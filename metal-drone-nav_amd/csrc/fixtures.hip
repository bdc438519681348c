// fixtures.hip — stateless operators over caller arrays, built from the same
// device functions as the rollout kernel.  They play the role of the
// reference's fixture kernels (physics_fixture, raptor_fixture, world_depth,
// world_clearance; main.mm:29-43, 74-81) for golden-vector tests.
#include "nav_device.h"

namespace nav {

__device__ __forceinline__ void fx_sync() { __syncthreads(); }

// One thread per sample: physics_step on AoS states (physics.hpp:149-179).
__global__ __launch_bounds__(256) void physics_fixture_kernel(const MdnPhysicsState* __restrict__ in,
                                                              const float* __restrict__ actions,
                                                              const float* __restrict__ winds, MdnPhysicsParams P,
                                                              MdnPhysicsState* __restrict__ out, uint64_t n) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    State s, nx;
    const float* src = &in[i].position[0];
    float* d = &s.p[0];
#pragma unroll
    for (int j = 0; j < 17; j++) d[j] = src[j];
    float act[4], wind[3];
#pragma unroll
    for (int j = 0; j < 4; j++) act[j] = actions[4 * i + j];
#pragma unroll
    for (int j = 0; j < 3; j++) wind[j] = winds[3 * i + j];
    physics_step(P, phys_recip(P), s, act, wind, nx);
    float* dst = &out[i].position[0];
    const float* o = &nx.p[0];
#pragma unroll
    for (int j = 0; j < 17; j++) dst[j] = o[j];
}

// One workgroup per world: obstacles and their centres in LDS exactly as the
// rollout kernel holds them; threads stride over the world's rays.
__global__ __launch_bounds__(256) void ray_fixture_kernel(const float* __restrict__ worlds,
                                                          const float* __restrict__ rays,
                                                          const float* __restrict__ times, uint32_t rays_per_world,
                                                          float* __restrict__ out, uint64_t n) {
    __shared__ float w[WORLD_WORDS + 3];
    __shared__ float cent[48];
    const uint64_t wi = blockIdx.x;
    for (uint32_t i = threadIdx.x; i < WORLD_WORDS; i += 256) w[i] = worlds[wi * WORLD_WORDS + i];
    fx_sync();
    const uint32_t count = min(float_bits(w[160]), 16u);
    if (threadIdx.x < count) {
        const V c = obstacle_center(w + 10 * threadIdx.x, times[wi]);
        cent[3 * threadIdx.x] = c.x; cent[3 * threadIdx.x + 1] = c.y; cent[3 * threadIdx.x + 2] = c.z;
    }
    fx_sync();
    for (uint32_t k = threadIdx.x; k < rays_per_world; k += 256) {
        const uint64_t i = wi * rays_per_world + k;
        if (i >= n) break;
        const float* r = rays + 6 * i;
        out[i] = cast_ray(w, cent, count, mk(r[0], r[1], r[2]), mk(r[3], r[4], r[5]));
    }
}

__global__ __launch_bounds__(256) void clearance_fixture_kernel(const float* __restrict__ worlds,
                                                                const float* __restrict__ points,
                                                                const float* __restrict__ times,
                                                                float* __restrict__ out, uint64_t n) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const float* w = worlds + i * WORLD_WORDS;
    out[i] = clearance_at(w, min(float_bits(w[160]), 16u), mk(points[3 * i], points[3 * i + 1], points[3 * i + 2]), times[i]);
}

}  // namespace nav

// The RAPTOR fixture needs the lane-group step of the rollout kernel, which
// lives in rollout.hip; it is launched from there (nav_launch_raptor_fixture).
extern "C" {

hipError_t nav_launch_physics_fixture(const MdnPhysicsState* in, const float* actions, const float* winds,
                                      const MdnPhysicsParams* P, MdnPhysicsState* out, uint64_t n, hipStream_t st) {
    hipLaunchKernelGGL(nav::physics_fixture_kernel, dim3(uint32_t((n + 255) / 256)), dim3(256), 0, st, in, actions, winds,
                       *P, out, n);
    return hipGetLastError();
}

hipError_t nav_launch_ray_fixture(const float* worlds, const float* rays, const float* times, uint32_t rays_per_world,
                                  float* out, uint64_t n, hipStream_t st) {
    const uint64_t nw = (n + rays_per_world - 1) / rays_per_world;
    hipLaunchKernelGGL(nav::ray_fixture_kernel, dim3(uint32_t(nw)), dim3(256), 0, st, worlds, rays, times, rays_per_world,
                       out, n);
    return hipGetLastError();
}

hipError_t nav_launch_clearance_fixture(const float* worlds, const float* points, const float* times, float* out,
                                        uint64_t n, hipStream_t st) {
    hipLaunchKernelGGL(nav::clearance_fixture_kernel, dim3(uint32_t((n + 255) / 256)), dim3(256), 0, st, worlds, points,
                       times, out, n);
    return hipGetLastError();
}

}  // extern "C"

// ---------------------------------------------------------------- calibration copy
namespace nav {
__global__ __launch_bounds__(256) void calib_copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                         uint64_t n) {
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += uint64_t(gridDim.x) * 256)
        dst[i] = src[i];
}
// Counts the fp32 bit patterns a (all 2^32) for which div_r(a, RN64(1/b)) is
// not bitwise the correctly rounded a / b (NaN results compare equal).
__global__ __launch_bounds__(256) void div_check_kernel(float b, double r, unsigned long long* count) {
    __shared__ unsigned long long block;
    if (threadIdx.x == 0) block = 0;
    __syncthreads();
    unsigned long long bad = 0;
    const uint64_t base = (uint64_t(blockIdx.x) * 256 + threadIdx.x) * 64;
    for (uint32_t i = 0; i < 64; i++) {
        const float a = __uint_as_float(uint32_t(base + i));
        const float want = a / b, got = div_r(a, r);
        const bool same = (want != want && got != got) || __float_as_uint(want) == __float_as_uint(got);
        bad += same ? 0 : 1;
    }
    atomicAdd(&block, bad);
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd(count, block);
}
}  // namespace nav

extern "C" int mdn_op_check_division(const float* divisors, uint32_t n, uint64_t* mismatches) {
    if (!divisors || !mismatches) return -1;
    if (n == 0) return 0;
    unsigned long long* d = nullptr;
    if (hipMalloc(&d, size_t(n) * 8) != hipSuccess) return -2;
    int rc = hipMemset(d, 0, size_t(n) * 8) == hipSuccess ? 0 : -2;
    const uint32_t blocks = uint32_t((uint64_t(1) << 32) / 64 / 256);
    for (uint32_t i = 0; i < n && rc == 0; i++) {
        hipLaunchKernelGGL(nav::div_check_kernel, dim3(blocks), dim3(256), 0, nullptr, divisors[i],
                           1.0 / double(divisors[i]), d + i);
        if (hipGetLastError() != hipSuccess) rc = -3;
    }
    if (rc == 0 && hipDeviceSynchronize() != hipSuccess) rc = -3;
    if (rc == 0 && hipMemcpy(mismatches, d, size_t(n) * 8, hipMemcpyDeviceToHost) != hipSuccess) rc = -3;
    hipFree(d);
    return rc;
}

extern "C" int mdn_calib_copy(uint64_t bytes, uint32_t repeats, double* ms) {
    if (bytes == 0 || bytes % 16 || repeats == 0 || !ms) return -1;
    void *a = nullptr, *b = nullptr;
    if (hipMalloc(&a, bytes) != hipSuccess) return -2;
    if (hipMalloc(&b, bytes) != hipSuccess) { hipFree(a); return -2; }
    hipMemset(a, 1, bytes);
    hipEvent_t e0, e1;
    hipEventCreate(&e0);
    hipEventCreate(&e1);
    const uint64_t n = bytes / 16;
    hipLaunchKernelGGL(nav::calib_copy_kernel, dim3(2048), dim3(256), 0, nullptr, (const uint4*)a, (uint4*)b, n);
    hipEventRecord(e0, nullptr);
    for (uint32_t r = 0; r < repeats; r++)
        hipLaunchKernelGGL(nav::calib_copy_kernel, dim3(2048), dim3(256), 0, nullptr, (const uint4*)a, (uint4*)b, n);
    hipEventRecord(e1, nullptr);
    hipEventSynchronize(e1);
    float t = 0;
    hipEventElapsedTime(&t, e0, e1);
    *ms = double(t) / repeats;
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipFree(a);
    hipFree(b);
    return 0;
}
