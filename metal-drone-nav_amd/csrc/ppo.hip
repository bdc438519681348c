// ppo.hip — GAE, advantage normalisation and the PPO minibatch update for gfx950.
//
// Reductions follow one canonical order shared with the CPU oracle so both
// round identically:
//   * dot products accumulate from the bias, inputs ascending (ppo.hpp:65-93);
//   * sums over minibatch rows: sequential within 256-row chunks, chunk
//     partials sequential within groups of 32 chunks, then over the groups
//     (a single chunk at the reference's 256-row minibatch, i.e.
//     ppo_actor_grad_direct's order, ppo.metal:497-519);
//   * squared gradient norm: 256 strided partials then a pairwise tree;
//   * advantage statistics in double: within each 256-element chunk, lane
//     sums of 4 elements combined by a wavefront xor butterfly; chunk
//     partials sequential within groups of 64, then over the groups.
// The 64-wide hidden layers are evaluated on the VALU with weights as
// wave-uniform scalar loads: one lane owns one row (forward) or one input
// feature (weight gradient), so every accumulation is a private serial chain.
#include <hip/hip_runtime.h>

#include "mdnav_math.h"
#include "mdnav_types.h"
#include "kernel_args.h"

namespace ppo {
using namespace mdn;

constexpr uint32_t OBS = MDN_ACTOR_OBS_POOLED;
constexpr uint32_t COBS = MDN_CRITIC_OBS;
constexpr uint32_t HID = MDN_HIDDEN;
constexpr uint32_t CHUNK = 256;
constexpr uint32_t GRAD_GROUP = 32;   // chunk partials per group (gradient sums)
constexpr uint32_t NORM_GROUP = 64;   // chunk partials per group (advantage statistics)
constexpr float LOG_TWO_PI = 1.8378770664093453f;

constexpr uint32_t A_B1 = HID * OBS, A_W2 = A_B1 + HID, A_B2 = A_W2 + 4 * HID, A_LS = A_B2 + 4, A_COUNT = A_LS + 4;
constexpr uint32_t C_B1 = HID * COBS, C_W2 = C_B1 + HID, C_B2 = C_W2 + HID, C_COUNT = C_B2 + 1;
// Per-chunk partial layout: actor params, critic params, 4 metric sums.
constexpr uint32_t P_TOTAL = A_COUNT + C_COUNT + 4;

// ---------------------------------------------------------------- GAE
// ppo.hpp:108-126 == ppo.metal:279-304, reverse scan per env.  A workgroup
// owns 32 envs and walks the horizon backwards in tiles of 32 ticks: all 256
// threads load the tile coalesced and form delta = r + gamma*V'(s') - V(s)
// in LDS, one lane per env then runs the carry recurrence over the tile (the
// only serial part), and the tile of advantages/returns is stored coalesced.
constexpr uint32_t GAE_ENVS = 32, GAE_TICKS = 32, GAE_PER = GAE_ENVS * GAE_TICKS / 256;
struct GaeTile {
    float delta[GAE_PER], value[GAE_PER];
    uint32_t boundary[GAE_PER];
};
// Loads the tile [t0, t1) x [e0, e0+32) into registers (4 elements per
// thread) and forms the deltas.
__device__ __forceinline__ void gae_load(GaeTile& g, const float* __restrict__ r, const float* __restrict__ v,
                                         const float* __restrict__ nv, const uint8_t* __restrict__ te,
                                         const uint8_t* __restrict__ tr, uint32_t t0, uint32_t t1, uint32_t e0,
                                         uint32_t n, float gamma) {
#pragma unroll
    for (uint32_t j = 0; j < GAE_PER; j++) {
        const uint32_t i = threadIdx.x + 256 * j;
        const uint32_t t = t0 + i / GAE_ENVS, env = e0 + i % GAE_ENVS;
        g.delta[j] = 0.0f; g.value[j] = 0.0f; g.boundary[j] = 0;
        if (t < t1 && env < n) {
            const size_t k = size_t(t) * n + env;
            const bool term = te[k] != 0;
            const bool boundary = term || tr[k] != 0;
            const float bootstrap = term ? 0.0f : nv[k];
            const float value = v[k];
            g.delta[j] = r[k] + gamma * bootstrap - value;
            g.value[j] = value;
            g.boundary[j] = boundary;
        }
    }
}
__global__ __launch_bounds__(256) void gae_kernel(const float* __restrict__ r, const float* __restrict__ v,
                                                  const float* __restrict__ nv, const uint8_t* __restrict__ te,
                                                  const uint8_t* __restrict__ tr, float* __restrict__ adv,
                                                  float* __restrict__ ret, uint32_t horizon, uint32_t n,
                                                  float gamma, float lambda) {
    __shared__ float s_delta[GAE_TICKS][GAE_ENVS + 1];
    __shared__ float s_val[GAE_TICKS][GAE_ENVS + 1];
    __shared__ float s_adv[GAE_TICKS][GAE_ENVS + 1];
    __shared__ uint32_t s_bnd[GAE_TICKS][GAE_ENVS + 1];
    const uint32_t e0 = blockIdx.x * GAE_ENVS, tid = threadIdx.x;
    float carry = 0.0f;
    GaeTile cur;
    uint32_t t1 = horizon, t0 = t1 > GAE_TICKS ? t1 - GAE_TICKS : 0;
    gae_load(cur, r, v, nv, te, tr, t0, t1, e0, n, gamma);
    while (t1 > 0) {
#pragma unroll
        for (uint32_t j = 0; j < GAE_PER; j++) {
            const uint32_t i = tid + 256 * j, tt = i / GAE_ENVS, e = i % GAE_ENVS;
            s_delta[tt][e] = cur.delta[j];
            s_val[tt][e] = cur.value[j];
            s_bnd[tt][e] = cur.boundary[j];
        }
        __syncthreads();
        // the next (earlier) tile's loads are in flight during the scan
        const uint32_t n1 = t0, n0 = n1 > GAE_TICKS ? n1 - GAE_TICKS : 0;
        if (n1 > 0) gae_load(cur, r, v, nv, te, tr, n0, n1, e0, n, gamma);
        if (tid < GAE_ENVS && e0 + tid < n) {
            for (uint32_t tt = t1 - t0; tt-- > 0;) {
                carry = s_delta[tt][tid] + (s_bnd[tt][tid] ? 0.0f : gamma * lambda * carry);
                s_adv[tt][tid] = carry;
            }
        }
        __syncthreads();
#pragma unroll
        for (uint32_t j = 0; j < GAE_PER; j++) {
            const uint32_t i = tid + 256 * j, tt = i / GAE_ENVS, e = i % GAE_ENVS;
            const uint32_t t = t0 + tt, env = e0 + e;
            if (t < t1 && env < n) {
                const size_t k = size_t(t) * n + env;
                const float a = s_adv[tt][e];
                adv[k] = a;
                ret[k] = a + s_val[tt][e];
            }
        }
        __syncthreads();
        t1 = n1;
        t0 = n0;
    }
}

// ---------------------------------------------------------------- normalisation
// ppo.hpp:128-140 with double statistics.  One wavefront per 256-element
// chunk: lane l adds elements 4l..4l+3 in order, then an xor butterfly over
// the 64 lanes (pass 0: sum a; pass 1: sum (a-mean)^2).
__global__ __launch_bounds__(256) void norm_chunks_kernel(const float* __restrict__ a, uint64_t count,
                                                          double* __restrict__ part, const float* __restrict__ stats,
                                                          int pass) {
    const uint64_t c = uint64_t(blockIdx.x) * 4 + threadIdx.x / 64;
    const uint32_t l = threadIdx.x % 64;
    const uint64_t chunks = (count + CHUNK - 1) / CHUNK;
    if (c >= chunks) return;  // whole wavefronts leave together
    const uint64_t begin = c * CHUNK + 4 * l;
    const float mean = pass == 0 ? 0.0f : stats[0];
    double s = 0.0;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        const uint64_t i = begin + j;
        if (i < count) {
            if (pass == 0) {
                s += double(a[i]);
            } else {
                const double d = double(a[i] - mean);
                s += d * d;
            }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s = s + __shfl_xor(s, off, 64);
    if (l == 0) part[c] = s;
}
// Chunk partials summed sequentially within groups of NORM_GROUP, then the
// group sums sequentially; pass 0 writes the float mean, pass 1 the inverse
// standard deviation 1/sqrt(var + eps).
__global__ __launch_bounds__(256) void norm_finish_kernel(const double* __restrict__ part, uint64_t count,
                                                          float* __restrict__ stats, float eps, int pass) {
    __shared__ double gs[256];
    const uint64_t chunks = (count + CHUNK - 1) / CHUNK;
    const uint64_t groups = (chunks + NORM_GROUP - 1) / NORM_GROUP;
    double total = 0.0;
    for (uint64_t g0 = 0; g0 < groups; g0 += 256) {
        const uint64_t g = g0 + threadIdx.x;
        if (g < groups) {
            const uint64_t c0 = g * NORM_GROUP, end = c0 + NORM_GROUP < chunks ? c0 + NORM_GROUP : chunks;
            double s = 0.0;
            for (uint64_t c = c0; c < end; ++c) s += part[c];
            gs[threadIdx.x] = s;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            const uint64_t m = groups - g0 < 256 ? groups - g0 : 256;
            for (uint64_t j = 0; j < m; ++j) total += gs[j];
        }
        __syncthreads();
    }
    if (threadIdx.x != 0) return;
    if (pass == 0) stats[0] = float(total / double(count));
    else stats[1] = 1.0f / sqrt_f(float(total / double(count)) + eps);
}
__global__ __launch_bounds__(256) void norm_apply_kernel(float* __restrict__ a, uint64_t count,
                                                         const float* __restrict__ stats) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= count) return;
    a[i] = (a[i] - stats[0]) * stats[1];
}

// ---------------------------------------------------------------- minibatch rows


// Forward, per-row loss/derivatives (ppo.hpp:144-181) and hidden deltas
// (ppo.metal:470-485, 618-631); one lane per row.
// Writes one 64-float value per row of the block's 256-row tile, transposed
// through LDS so that global stores are contiguous across lanes (the row-major
// [row][64] layout the gradient kernels read).
__device__ __forceinline__ void store_rows64(float* lds, const float (&v)[HID], float* __restrict__ dst, uint32_t n0,
                                             uint32_t rows) {
    const uint32_t t = threadIdx.x;
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < HID; k++) lds[t * (HID + 1) + k] = v[k];
    __syncthreads();
    float* out = dst + size_t(n0) * HID;
    for (uint32_t e = t; e < rows * HID; e += 256) out[e] = lds[(e / HID) * (HID + 1) + e % HID];
}

__global__ __launch_bounds__(256) void rows_kernel(RowArgs a) {
    // Row tiles are staged through LDS 16 features at a time with coalesced
    // loads; each lane then walks its own row (padding 17 avoids bank
    // conflicts) while the weights arrive as wave-uniform scalar loads.  The
    // same LDS then stages the per-row outputs.
    __shared__ float lds[256 * (HID + 1)];
    float(*tile)[17] = reinterpret_cast<float(*)[17]>(lds);
    const uint32_t t = threadIdx.x, n0 = blockIdx.x * 256;
    const uint32_t n = n0 + t;
    const bool live = n < a.b;
    const uint32_t rows = a.b - n0 < 256 ? a.b - n0 : 256;
    float h[HID];
#pragma unroll
    for (uint32_t k = 0; k < HID; k++) h[k] = a.actor[A_B1 + k];
    for (uint32_t i0 = 0; i0 < OBS; i0 += 16) {
        for (uint32_t e = t; e < 256 * 16; e += 256) {
            const uint32_t rr = e / 16, cc = e % 16;
            const uint32_t row = n0 + rr, col = i0 + cc;
            tile[rr][cc] = (row < a.b && col < OBS) ? a.obs[size_t(row) * OBS + col] : 0.0f;
        }
        __syncthreads();
        const uint32_t cnt = OBS - i0 < 16 ? OBS - i0 : 16;
#pragma unroll
        for (uint32_t c = 0; c < 16; c++) {
            if (c < cnt) {
                const float xi = tile[t][c];
                const float* w = a.actor_w1t + size_t(i0 + c) * HID;
#pragma unroll
                for (uint32_t k = 0; k < HID; k++) h[k] += w[k] * xi;
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (uint32_t k = 0; k < HID; k++) h[k] = tanh_f(h[k]);
    float mean[4];
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) {
        float z = a.actor[A_B2 + q];
#pragma unroll
        for (uint32_t k = 0; k < HID; k++) z += a.actor[A_W2 + q * HID + k] * h[k];
        mean[q] = z;
    }
    float g[HID];
#pragma unroll
    for (uint32_t k = 0; k < HID; k++) g[k] = a.critic[C_B1 + k];
    for (uint32_t i0 = 0; i0 < COBS; i0 += 16) {
        for (uint32_t e = t; e < 256 * 16; e += 256) {
            const uint32_t rr = e / 16, cc = e % 16;
            const uint32_t row = n0 + rr;
            tile[rr][cc] = row < a.b ? a.co[size_t(row) * COBS + i0 + cc] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (uint32_t c = 0; c < 16; c++) {
            const float xi = tile[t][c];
            const float* w = a.critic_w1t + size_t(i0 + c) * HID;
#pragma unroll
            for (uint32_t k = 0; k < HID; k++) g[k] += w[k] * xi;
        }
        __syncthreads();
    }
#pragma unroll
    for (uint32_t k = 0; k < HID; k++) g[k] = tanh_f(g[k]);
    float value = a.critic[C_B2];
#pragma unroll
    for (uint32_t k = 0; k < HID; k++) value += a.critic[C_W2 + k] * g[k];

    // sample_loss_and_grad (rows past the minibatch compute on index 0 and
    // store nothing)
    const uint32_t m = live ? n : 0;
    const float* act = a.actions + size_t(m) * 4;
    const float* ls = a.actor + A_LS;
    float logp = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) {
        const float inv_std = exp_f(-ls[q]);
        const float d = (act[q] - mean[q]) * inv_std;
        logp += -0.5f * (d * d + 2.0f * ls[q] + LOG_TWO_PI);
    }
    const float raw = logp - a.old_logp[m];
    const float lr = clamp_f(raw, -20.0f, 20.0f);
    const float ratio = exp_f(lr);
    const float adv = a.adv[m], target = a.ret[m];
    const float clipped = clamp_f(ratio, 1.0f - a.clip, 1.0f + a.clip);
    const float chosen = min_f(ratio * adv, clipped * adv);
    const bool in_range = raw >= -20.0f && raw <= 20.0f;
    const bool active = in_range && (adv >= 0.0f ? ratio <= 1.0f + a.clip : ratio >= 1.0f - a.clip);
    const float scale = 1.0f / max_f(float(a.b), 1.0f);
    float dmean[4], dlog[4], entropy = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) {
        const float inv_var = exp_f(-2.0f * ls[q]);
        const float diff = act[q] - mean[q];
        if (active) {
            const float dlogp = -ratio * adv * scale;
            dmean[q] = dlogp * diff * inv_var;
            dlog[q] = dlogp * (diff * diff * inv_var - 1.0f);
        } else {
            dmean[q] = 0.0f;
            dlog[q] = 0.0f;
        }
        dlog[q] -= a.ecoef * scale;
        entropy += -a.ecoef * (ls[q] + 0.5f * (1.0f + LOG_TWO_PI)) * scale;
    }
    const float dvalue = a.vcoef * (value - target) * scale;
    if (live) {
        float* lo = a.loss + size_t(n) * 4;
        lo[0] = -chosen * scale;
        lo[1] = 0.5f * a.vcoef * (value - target) * (value - target) * scale;
        lo[2] = entropy;
        lo[3] = ratio;
#pragma unroll
        for (uint32_t q = 0; q < 4; q++) {
            a.dm[size_t(n) * 4 + q] = dmean[q];
            a.dls[size_t(n) * 4 + q] = dlog[q];
        }
        a.dv[n] = dvalue;
    }
    store_rows64(lds, h, a.ah, n0, rows);
#pragma unroll
    for (uint32_t k = 0; k < HID; k++) {
        float d = 0.0f;
#pragma unroll
        for (uint32_t q = 0; q < 4; q++) d += dmean[q] * a.actor[A_W2 + q * HID + k];
        h[k] = d * (1.0f - h[k] * h[k]);
    }
    store_rows64(lds, h, a.adelta, n0, rows);
    store_rows64(lds, g, a.ch, n0, rows);
#pragma unroll
    for (uint32_t k = 0; k < HID; k++) g[k] = dvalue * a.critic[C_W2 + k] * (1.0f - g[k] * g[k]);
    store_rows64(lds, g, a.cdelta, n0, rows);
}

// ---------------------------------------------------------------- gradient partials
// First-layer weight gradients of one 256-row chunk: lane = input feature,
// 64 accumulators (one per hidden unit), rows ascending; deltas are
// wave-uniform scalar loads.  grid.x = chunk, grid.y = 0 actor / 1 critic.
__global__ __launch_bounds__(192) void w1_grad_kernel(const float* __restrict__ obs, const float* __restrict__ co,
                                                      const float* __restrict__ adelta,
                                                      const float* __restrict__ cdelta, float* __restrict__ part,
                                                      uint32_t b) {
    const uint32_t c = blockIdx.x;
    const bool critic = blockIdx.y == 1;
    const uint32_t D = critic ? COBS : OBS;
    const uint32_t i = threadIdx.x;
    if (i >= D) return;
    const float* X = critic ? co : obs;
    const float* delta = critic ? cdelta : adelta;
    float acc[HID];
#pragma unroll
    for (uint32_t k = 0; k < HID; k++) acc[k] = 0.0f;
    const uint32_t end = (c + 1) * CHUNK < b ? (c + 1) * CHUNK : b;
    for (uint32_t n = c * CHUNK; n < end; n++) {
        const float x = X[size_t(n) * D + i];
        const float* d = delta + size_t(n) * HID;
#pragma unroll
        for (uint32_t k = 0; k < HID; k++) acc[k] += d[k] * x;
    }
    float* out = part + size_t(c) * P_TOTAL + (critic ? A_COUNT : 0);
#pragma unroll
    for (uint32_t k = 0; k < HID; k++) out[size_t(k) * D + i] = acc[k];
}

// The remaining sums of one chunk: actor b1, W2, b2, log_std; critic b1, w2,
// b2; the four metric sums.  One thread per output slot.
constexpr uint32_t SMALL_SLOTS = HID + 4 * HID + 4 + 4 + HID + HID + 1 + 4;  // 461
__global__ __launch_bounds__(512) void small_grad_kernel(const float* __restrict__ ah, const float* __restrict__ adelta,
                                                         const float* __restrict__ ch, const float* __restrict__ cdelta,
                                                         const float* __restrict__ dm, const float* __restrict__ dls,
                                                         const float* __restrict__ dv, const float* __restrict__ loss,
                                                         float* __restrict__ part, uint32_t b) {
    const uint32_t c = blockIdx.x;
    uint32_t s = threadIdx.x;
    if (s >= SMALL_SLOTS) return;
    const uint32_t begin = c * CHUNK, end = (c + 1) * CHUNK < b ? (c + 1) * CHUNK : b;
    float acc = 0.0f;
    size_t out;
    float* P = part + size_t(c) * P_TOTAL;
    if (s < HID) {  // actor b1
        for (uint32_t n = begin; n < end; n++) acc += adelta[size_t(n) * HID + s];
        out = A_B1 + s;
    } else if ((s -= HID) < 4 * HID) {  // actor W2[a][h]
        const uint32_t q = s / HID, h = s % HID;
        for (uint32_t n = begin; n < end; n++) acc += dm[size_t(n) * 4 + q] * ah[size_t(n) * HID + h];
        out = A_W2 + s;
    } else if ((s -= 4 * HID) < 4) {  // actor b2
        for (uint32_t n = begin; n < end; n++) acc += dm[size_t(n) * 4 + s];
        out = A_B2 + s;
    } else if ((s -= 4) < 4) {  // actor log_std
        for (uint32_t n = begin; n < end; n++) acc += dls[size_t(n) * 4 + s];
        out = A_LS + s;
    } else if ((s -= 4) < HID) {  // critic b1
        for (uint32_t n = begin; n < end; n++) acc += cdelta[size_t(n) * HID + s];
        out = A_COUNT + C_B1 + s;
    } else if ((s -= HID) < HID) {  // critic w2
        for (uint32_t n = begin; n < end; n++) acc += dv[n] * ch[size_t(n) * HID + s];
        out = A_COUNT + C_W2 + s;
    } else if ((s -= HID) < 1) {  // critic b2
        for (uint32_t n = begin; n < end; n++) acc += dv[n];
        out = A_COUNT + C_B2;
    } else {  // metric sums (main.mm:941-951)
        s -= 1;
        for (uint32_t n = begin; n < end; n++) acc += loss[size_t(n) * 4 + s];
        out = A_COUNT + C_COUNT + s;
    }
    P[out] = acc;
}

// Chunk partials summed within groups of GRAD_GROUP chunks, in place into
// the group's first chunk row; grid (param blocks, groups).
__global__ __launch_bounds__(256) void group_reduce_kernel(float* __restrict__ part, uint32_t chunks) {
    const uint32_t p = blockIdx.x * 256 + threadIdx.x;
    const uint32_t c0 = blockIdx.y * GRAD_GROUP;
    if (p >= P_TOTAL || c0 >= chunks) return;
    const uint32_t end = c0 + GRAD_GROUP < chunks ? c0 + GRAD_GROUP : chunks;
    float s = 0.0f;
    for (uint32_t c = c0; c < end; c++) s += part[size_t(c) * P_TOTAL + p];
    part[size_t(c0) * P_TOTAL + p] = s;
}
// Sequential sum over the group sums: grad[p] = 0 + g0[p] + g1[p] + ...
__global__ __launch_bounds__(256) void chunk_reduce_kernel(const float* __restrict__ part, float* __restrict__ grad,
                                                           uint32_t chunks) {
    const uint32_t p = blockIdx.x * 256 + threadIdx.x;
    if (p >= P_TOTAL) return;
    float total = 0.0f;
    for (uint32_t c = 0; c < chunks; c += GRAD_GROUP) total += part[size_t(c) * P_TOTAL + p];
    grad[p] = total;
}

// ---------------------------------------------------------------- clip + Adam
// cpu_reference.hpp:553-567 + log-std clamp (603); block 0 = actor, 1 = critic.
// Also refreshes the transposed first-layer copy and the metric row.

__global__ __launch_bounds__(256) void adam_kernel(AdamArgs a) {
    const bool critic = blockIdx.x == 1;
    const uint32_t P = critic ? C_COUNT : A_COUNT;
    float* params = critic ? a.critic : a.actor;
    float* m = critic ? a.cm : a.am;
    float* v = critic ? a.cv : a.av;
    const float* g = a.grad + (critic ? A_COUNT : 0);
    __shared__ float part[256];
    const uint32_t t = threadIdx.x;
    float s = 0.0f;
    for (uint32_t i = t; i < P; i += 256) s += g[i] * g[i];
    part[t] = s;
    __syncthreads();
    for (uint32_t stride = 128; stride > 0; stride >>= 1) {
        if (t < stride) part[t] = part[t] + part[t + stride];
        __syncthreads();
    }
    const float norm = sqrt_f(part[0] + 1.0e-20f);
    const float scale = min_f(1.0f, 0.5f / norm);
    const float b1 = 0.9f, b2 = 0.999f;
    for (uint32_t i = t; i < P; i += 256) {
        const float gi = g[i] * scale;
        m[i] = b1 * m[i] + (1.0f - b1) * gi;
        v[i] = b2 * v[i] + (1.0f - b2) * gi * gi;
        const float mh = m[i] / a.c1, vh = v[i] / a.c2;
        params[i] -= a.lr * mh / (sqrt_f(vh) + 1.0e-8f);
    }
    __syncthreads();
    if (!critic) {
        if (t < 4) params[A_LS + t] = clamp_f(params[A_LS + t], -2.0f, .5f);
        for (uint32_t e = t; e < HID * OBS; e += 256) {
            const uint32_t h = e / OBS, i = e % OBS;
            a.actor_w1t[size_t(i) * HID + h] = params[e];
        }
        if (t == 0) {
            const float* ms = a.grad + A_COUNT + C_COUNT;
            a.metric_row[0] = ms[0];
            a.metric_row[1] = ms[1];
            a.metric_row[2] = ms[2];
            a.metric_row[3] = ms[3] / float(a.b);
        }
    } else {
        for (uint32_t e = t; e < HID * COBS; e += 256) {
            const uint32_t h = e / COBS, i = e % COBS;
            a.critic_w1t[size_t(i) * HID + h] = params[e];
        }
    }
}

// Transposed first-layer copies from the flat vectors (after uploads/init).
__global__ __launch_bounds__(256) void transpose_w1_kernel(const float* __restrict__ actor,
                                                           const float* __restrict__ critic, float* __restrict__ aw,
                                                           float* __restrict__ cw) {
    const uint32_t e = blockIdx.x * 256 + threadIdx.x;
    if (e < HID * OBS) {
        const uint32_t h = e / OBS, i = e % OBS;
        aw[size_t(i) * HID + h] = actor[e];
    }
    if (e < HID * COBS) {
        const uint32_t h = e / COBS, i = e % COBS;
        cw[size_t(i) * HID + h] = critic[e];
    }
}

// metric_mean (main.mm:952-962): sequential over updates.
__global__ void metric_mean_kernel(const float* __restrict__ rows, float* __restrict__ mean, uint32_t updates) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    float s[4] = {0, 0, 0, 0};
    for (uint32_t u = 0; u < updates; u++)
        for (int k = 0; k < 4; k++) s[k] += rows[size_t(u) * 4 + k];
    for (int k = 0; k < 4; k++) mean[k] = updates ? s[k] / float(updates) : 0.0f;
}

}  // namespace ppo

// ---------------------------------------------------------------- launchers
extern "C" {

hipError_t ppo_launch_gae(const float* r, const float* v, const float* nv, const uint8_t* te, const uint8_t* tr,
                          float* adv, float* ret, uint32_t horizon, uint32_t n, float gamma, float lambda,
                          hipStream_t st) {
    if (n == 0 || horizon == 0) return hipSuccess;
    hipLaunchKernelGGL(ppo::gae_kernel, dim3((n + ppo::GAE_ENVS - 1) / ppo::GAE_ENVS), dim3(256), 0, st, r, v, nv, te, tr,
                       adv, ret, horizon, n, gamma, lambda);
    return hipGetLastError();
}

// stats: device float[2] (mean, inv_std); part: device double[ceil(count/256)]
hipError_t ppo_launch_normalize(float* a, uint64_t count, double* part, float* stats, float eps, hipStream_t st) {
    if (count == 0) return hipSuccess;
    const uint64_t chunks = (count + ppo::CHUNK - 1) / ppo::CHUNK;
    const uint32_t cb = uint32_t((chunks + 3) / 4);  // one wavefront per chunk
    for (int pass = 0; pass < 2; pass++) {
        hipLaunchKernelGGL(ppo::norm_chunks_kernel, dim3(cb), dim3(256), 0, st, a, count, part, stats, pass);
        hipLaunchKernelGGL(ppo::norm_finish_kernel, dim3(1), dim3(256), 0, st, part, count, stats, eps, pass);
    }
    hipLaunchKernelGGL(ppo::norm_apply_kernel, dim3(uint32_t((count + 255) / 256)), dim3(256), 0, st, a, count, stats);
    return hipGetLastError();
}

hipError_t ppo_launch_rows(const ppo::RowArgs* a, hipStream_t st) {
    hipLaunchKernelGGL(ppo::rows_kernel, dim3((a->b + 255) / 256), dim3(256), 0, st, *a);
    return hipGetLastError();
}

hipError_t ppo_launch_grads(const float* obs, const float* co, const float* ah, const float* adelta, const float* ch,
                            const float* cdelta, const float* dm, const float* dls, const float* dv, const float* loss,
                            float* part, float* grad, uint32_t b, hipStream_t st) {
    const uint32_t chunks = (b + ppo::CHUNK - 1) / ppo::CHUNK;
    hipLaunchKernelGGL(ppo::w1_grad_kernel, dim3(chunks, 2), dim3(192), 0, st, obs, co, adelta, cdelta, part, b);
    hipLaunchKernelGGL(ppo::small_grad_kernel, dim3(chunks), dim3(512), 0, st, ah, adelta, ch, cdelta, dm, dls, dv, loss,
                       part, b);
    const uint32_t groups = (chunks + ppo::GRAD_GROUP - 1) / ppo::GRAD_GROUP;
    hipLaunchKernelGGL(ppo::group_reduce_kernel, dim3((ppo::P_TOTAL + 255) / 256, groups), dim3(256), 0, st, part, chunks);
    hipLaunchKernelGGL(ppo::chunk_reduce_kernel, dim3((ppo::P_TOTAL + 255) / 256), dim3(256), 0, st, part, grad, chunks);
    return hipGetLastError();
}

hipError_t ppo_launch_adam(const ppo::AdamArgs* a, hipStream_t st) {
    hipLaunchKernelGGL(ppo::adam_kernel, dim3(2), dim3(256), 0, st, *a);
    return hipGetLastError();
}

hipError_t ppo_launch_transpose(const float* actor, const float* critic, float* aw, float* cw, hipStream_t st) {
    hipLaunchKernelGGL(ppo::transpose_w1_kernel, dim3((ppo::HID * ppo::OBS + 255) / 256), dim3(256), 0, st, actor, critic,
                       aw, cw);
    return hipGetLastError();
}

hipError_t ppo_launch_metric_mean(const float* rows, float* mean, uint32_t updates, hipStream_t st) {
    hipLaunchKernelGGL(ppo::metric_mean_kernel, dim3(1), dim3(64), 0, st, rows, mean, updates);
    return hipGetLastError();
}

uint32_t ppo_partial_stride() { return ppo::P_TOTAL; }

}  // extern "C"
