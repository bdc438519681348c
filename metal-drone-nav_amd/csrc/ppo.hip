// ppo.hip — GAE, advantage normalisation and the PPO minibatch update for gfx950.
//
// Reductions follow one canonical order shared with the CPU oracle so both
// round identically:
//   * dot products: fma chain from the bias, inputs ascending (ppo.hpp:65-93);
//   * weight gradients: fma chain over rows in the row order below;
//   * sums over minibatch rows: sequential within 256-row chunks, chunk
//     partials sequential within groups of 32 chunks, then over the groups
//     (a single chunk at the reference's 256-row minibatch, i.e.
//     ppo_actor_grad_direct's order, ppo.metal:497-519);
//   * squared gradient norm: 256 strided partials then a pairwise tree;
//   * advantage statistics in double: within each 256-element chunk, lane
//     sums of 4 elements combined by a pairwise tree over adjacent lanes;
//     chunk partials sequential within groups of 64, then over the groups.
// Dot products and weight-gradient sums are fma chains (one rounding per
// step), which the fp32 matrix-core GEMMs below reproduce exactly.
#include <hip/hip_runtime.h>

#include "mdnav_math.h"
#include "mdnav_types.h"
#include "kernel_args.h"

namespace ppo {
using namespace mdn;

constexpr uint32_t COBS = MDN_CRITIC_OBS;
constexpr uint32_t HID = MDN_HIDDEN;
constexpr uint32_t CHUNK = 256;
constexpr uint32_t GRAD_GROUP = 32;   // chunk partials per group (gradient sums)
constexpr uint32_t NORM_GROUP = 64;   // chunk partials per group (advantage statistics)
constexpr float LOG_TWO_PI = 1.8378770664093453f;

constexpr uint32_t C_B1 = HID * COBS, C_W2 = C_B1 + HID, C_B2 = C_W2 + HID, C_COUNT = C_B2 + 1;
// Flat actor layout (ppo.hpp:35-40) for D inputs: 181 (pooled observation) or
// 184 (with the geometry-prior hint).  Per-chunk partial layout: actor
// params, critic params, 4 metric sums.
template <uint32_t D>
struct AL {
    static constexpr uint32_t B1 = HID * D, W2 = B1 + HID, B2 = W2 + 4 * HID, LS = B2 + 4, COUNT = LS + 4;
    static constexpr uint32_t P_TOTAL = COUNT + C_COUNT + 4;
};

// ---------------------------------------------------------------- GAE
// ppo.hpp:108-126 == ppo.metal:279-304, reverse scan per env.  A workgroup
// owns a slice of 32 envs and walks the horizon backwards in tiles of 128
// ticks: all 256 threads load the tile coalesced and form
// delta = r + gamma*V'(s') - V(s) in LDS, one lane per env then runs the
// carry recurrence over the tile (the only serial part), and the tile of
// advantages/returns is stored coalesced.
constexpr uint32_t GAE_ENVS = 32, GAE_TICKS = 128, GAE_PER = GAE_ENVS * GAE_TICKS / 256, GAE_SCAN = 32;
struct GaeTile {
    float delta[GAE_PER], value[GAE_PER];
    uint32_t boundary[GAE_PER];
};
// Loads the tile [t0, t1) x [e0, e0+32) into registers (16 elements per
// thread) and forms the deltas.  Every load is issued before any is used
// (the bootstrap value is read whether or not the step terminated, then
// selected).  V4: n % 4 == 0, so each thread takes four consecutive envs of
// four rows with 16-byte (float) and 4-byte (flag) loads; thread tid holds
// envs 4 (tid % 8) + c of rows tid / 8 + 32 j as element 4 j + c.
template <bool V4>
__device__ __forceinline__ void gae_load(GaeTile& g, const float* __restrict__ r, const float* __restrict__ v,
                                         const float* __restrict__ nv, const uint8_t* __restrict__ te,
                                         const uint8_t* __restrict__ tr, uint32_t t0, uint32_t t1, uint32_t e0,
                                         uint32_t n, float gamma) {
    if constexpr (V4) {
        const uint32_t eq = threadIdx.x % 8, row = threadIdx.x / 8;
        float4 rr[GAE_PER / 4], vv[GAE_PER / 4], nn[GAE_PER / 4];
        uint32_t tt4[GAE_PER / 4], tu4[GAE_PER / 4];
        bool in[GAE_PER / 4];
#pragma unroll
        for (uint32_t j = 0; j < GAE_PER / 4; j++) {
            const uint32_t t = t0 + row + 32 * j, env = e0 + 4 * eq;
            in[j] = t < t1 && env < n;
            const size_t k = in[j] ? size_t(t) * n + env : 0;
            rr[j] = *reinterpret_cast<const float4*>(r + k);
            vv[j] = *reinterpret_cast<const float4*>(v + k);
            nn[j] = *reinterpret_cast<const float4*>(nv + k);
            tt4[j] = *reinterpret_cast<const uint32_t*>(te + k);
            tu4[j] = *reinterpret_cast<const uint32_t*>(tr + k);
        }
#pragma unroll
        for (uint32_t j = 0; j < GAE_PER / 4; j++) {
            const float rc[4] = {rr[j].x, rr[j].y, rr[j].z, rr[j].w};
            const float vc[4] = {vv[j].x, vv[j].y, vv[j].z, vv[j].w};
            const float nc[4] = {nn[j].x, nn[j].y, nn[j].z, nn[j].w};
#pragma unroll
            for (uint32_t c = 0; c < 4; c++) {
                const bool term = ((tt4[j] >> (8 * c)) & 0xffu) != 0;
                const bool boundary = term || ((tu4[j] >> (8 * c)) & 0xffu) != 0;
                const float bootstrap = term ? 0.0f : nc[c];
                g.delta[4 * j + c] = in[j] ? rc[c] + gamma * bootstrap - vc[c] : 0.0f;
                g.value[4 * j + c] = in[j] ? vc[c] : 0.0f;
                g.boundary[4 * j + c] = in[j] && boundary;
            }
        }
    } else {
#pragma unroll
        for (uint32_t j = 0; j < GAE_PER; j++) {
            const uint32_t i = threadIdx.x + 256 * j;
            const uint32_t t = t0 + i / GAE_ENVS, env = e0 + i % GAE_ENVS;
            g.delta[j] = 0.0f; g.value[j] = 0.0f; g.boundary[j] = 0;
            if (t < t1 && env < n) {
                const size_t k = size_t(t) * n + env;
                const bool term = te[k] != 0;
                const bool boundary = term || tr[k] != 0;
                const float nvk = nv[k];
                const float bootstrap = term ? 0.0f : nvk;
                const float value = v[k];
                g.delta[j] = r[k] + gamma * bootstrap - value;
                g.value[j] = value;
                g.boundary[j] = boundary;
            }
        }
    }
}
// LDS position (tick, env) of a thread's element j in either load layout.
template <bool V4>
__device__ __forceinline__ void gae_pos(uint32_t j, uint32_t& tt, uint32_t& e) {
    if constexpr (V4) {
        tt = threadIdx.x / 8 + 32 * (j / 4);
        e = 4 * (threadIdx.x % 8) + j % 4;
    } else {
        const uint32_t i = threadIdx.x + 256 * j;
        tt = i / GAE_ENVS;
        e = i % GAE_ENVS;
    }
}
// The slice workgroup b takes out of S.  Workgroups go to the eight XCDs
// round-robin (b % 8); with S % 64 == 0 the eight slices of each 256-env
// block run on one XCD, so a 128-byte line of flags (four slices) is fetched
// into one L2.
__device__ __forceinline__ uint32_t gae_slice(uint32_t b, uint32_t S) {
    if (S % 64 != 0) return b;
    const uint32_t k = b / 8;
    return 8 * (b % 8 + 8 * (k / 8)) + k % 8;
}

template <bool V4>
__global__ __launch_bounds__(256) void gae_kernel(const float* __restrict__ r, const float* __restrict__ v,
                                                  const float* __restrict__ nv, const uint8_t* __restrict__ te,
                                                  const uint8_t* __restrict__ tr, float* __restrict__ adv,
                                                  float* __restrict__ ret, uint32_t horizon, uint32_t n,
                                                  float gamma, float lambda) {
    __shared__ float s_delta[GAE_TICKS][GAE_ENVS + 1];
    __shared__ float s_val[GAE_TICKS][GAE_ENVS + 1];
    __shared__ float s_adv[GAE_TICKS][GAE_ENVS + 1];
    __shared__ uint32_t s_bnd[GAE_TICKS][GAE_ENVS + 1];
    const uint32_t S = (n + GAE_ENVS - 1) / GAE_ENVS;
    const uint32_t slice = gae_slice(blockIdx.x, S);
    const uint32_t e0 = slice * GAE_ENVS, tid = threadIdx.x;
    float carry = 0.0f;
    GaeTile cur;
    uint32_t t1 = horizon, t0 = t1 > GAE_TICKS ? t1 - GAE_TICKS : 0;
    gae_load<V4>(cur, r, v, nv, te, tr, t0, t1, e0, n, gamma);
    while (t1 > 0) {
#pragma unroll
        for (uint32_t j = 0; j < GAE_PER; j++) {
            uint32_t tt, e;
            gae_pos<V4>(j, tt, e);
            s_delta[tt][e] = cur.delta[j];
            s_val[tt][e] = cur.value[j];
            s_bnd[tt][e] = cur.boundary[j];
        }
        __syncthreads();
        // the next (earlier) tile's loads are in flight during the scan
        const uint32_t n1 = t0, n0 = n1 > GAE_TICKS ? n1 - GAE_TICKS : 0;
        if (n1 > 0) gae_load<V4>(cur, r, v, nv, te, tr, n0, n1, e0, n, gamma);
        if (tid < GAE_ENVS && e0 + tid < n) {
            // the column in registers GAE_SCAN ticks at a time (one LDS round
            // trip each), the carry chain without memory operations
            const uint32_t len = t1 - t0;
            for (uint32_t b1 = (len + GAE_SCAN - 1) / GAE_SCAN * GAE_SCAN; b1 > 0; b1 -= GAE_SCAN) {
                const uint32_t b0 = b1 - GAE_SCAN;
                float dl[GAE_SCAN];
                uint32_t bd[GAE_SCAN];
#pragma unroll
                for (uint32_t k = 0; k < GAE_SCAN; k++) {
                    dl[k] = s_delta[b0 + k][tid];
                    bd[k] = s_bnd[b0 + k][tid];
                }
#pragma unroll
                for (uint32_t k = GAE_SCAN; k-- > 0;) {
                    if (b0 + k < len) {
                        carry = dl[k] + (bd[k] ? 0.0f : gamma * lambda * carry);
                        dl[k] = carry;
                    }
                }
#pragma unroll
                for (uint32_t k = 0; k < GAE_SCAN; k++) s_adv[b0 + k][tid] = dl[k];
            }
        }
        __syncthreads();
        if constexpr (V4) {
            // thread tid stores envs 4 (tid % 8) .. + 3 of rows tid / 8 + 32 j
            // with 16-byte stores
            const uint32_t e = 4 * (tid % 8);
#pragma unroll
            for (uint32_t j = 0; j < GAE_PER / 4; j++) {
                const uint32_t tt = tid / 8 + 32 * j, t = t0 + tt, env = e0 + e;
                const float4 a4 = make_float4(s_adv[tt][e], s_adv[tt][e + 1], s_adv[tt][e + 2], s_adv[tt][e + 3]);
                const float4 r4 = make_float4(a4.x + s_val[tt][e], a4.y + s_val[tt][e + 1], a4.z + s_val[tt][e + 2],
                                              a4.w + s_val[tt][e + 3]);
                if (t < t1 && env < n) {
                    const size_t k = size_t(t) * n + env;
                    *reinterpret_cast<float4*>(adv + k) = a4;
                    *reinterpret_cast<float4*>(ret + k) = r4;
                }
            }
        } else {
#pragma unroll
            for (uint32_t j = 0; j < GAE_PER; j++) {
                uint32_t tt, e;
                gae_pos<V4>(j, tt, e);
                const uint32_t t = t0 + tt, env = e0 + e;
                if (t < t1 && env < n) {
                    const size_t k = size_t(t) * n + env;
                    const float a = s_adv[tt][e];
                    adv[k] = a;
                    ret[k] = a + s_val[tt][e];
                }
            }
        }
        __syncthreads();
        t1 = n1;
        t0 = n0;
    }
}

// ---------------------------------------------------------------- advantage statistics
// ppo.hpp:128-140 with double statistics in the canonical order: a chunk of
// 256 elements is summed by one wavefront (lane l adds elements 4l..4l+3 in
// order, then xor levels 1, 2, ..., 32: a pairwise tree over adjacent
// lanes); chunk partials are added sequentially within groups of NORM_GROUP
// chunks, then the group sums sequentially.
//
// Two passes, each storing one partial per group (a 1024-thread workgroup
// per group of 64 chunks): the values, then the squared deviations.  The
// second pass forms the mean from the first's group partials (64 per
// million values) in every workgroup while its own values load; its last
// workgroup to finish forms 1 / sqrt(var + eps).  The rescale itself is a
// third launch or, in PPOTrainer::rollout_update, part of the first epoch's
// minibatch kernels.
//
// part: a 32-bit ticket (zero when allocated; the last workgroup of each
// second pass resets it), then pass 0's group partials, then pass 1's.
constexpr uint32_t NORM_THREADS = 1024, NORM_WAVE_CHUNKS = NORM_GROUP / (NORM_THREADS / 64);
static_assert(NORM_WAVE_CHUNKS * (NORM_THREADS / 64) == NORM_GROUP, "a workgroup per group of chunks");

// Sum of the 64 lanes' values in the canonical tree (xor levels 1..32).
__device__ __forceinline__ double chunk_tree(double v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) v = v + __shfl_xor(v, off, 64);
    return v;
}
// Sequential sum of p[0, m) (the group partials, in order), returned to
// every thread: rounds of 256 loaded coalesced into LDS, thread 0 adds them
// 16 at a time.  `first` holds p[threadIdx.x] (0 past m), loaded by the
// caller before its own values so that this wait does not include them.
// sp: LDS double[257].
__device__ double sequential_total(const double* __restrict__ p, uint64_t m, double first, double* sp) {
    double total = 0.0;
#pragma unroll 1
    for (uint64_t c0 = 0; c0 < m; c0 += 256) {
        const uint32_t k = uint32_t(m - c0 < 256 ? m - c0 : 256);
        if (threadIdx.x < 256) sp[threadIdx.x] = c0 == 0 ? first : (threadIdx.x < k ? p[c0 + threadIdx.x] : 0.0);
        __syncthreads();
        if (threadIdx.x == 0) {
#pragma unroll 1
            for (uint32_t j0 = 0; j0 < k; j0 += 16) {
                double y[16];
#pragma unroll
                for (uint32_t j = 0; j < 16; j++) y[j] = sp[j0 + j];
                if (j0 + 16 <= k) {
#pragma unroll
                    for (uint32_t j = 0; j < 16; j++) total += y[j];
                } else {
#pragma unroll
                    for (uint32_t j = 0; j < 16; j++)
                        if (j0 + j < k) total += y[j];
                }
            }
            sp[256] = total;
        }
        __syncthreads();
        total = sp[256];
        __syncthreads();
    }
    return total;
}
// One pass over a[0, count): workgroup g sums chunks 64g..64g+63 (wavefront
// w the four chunks from 64g + 4w, loads issued together), then thread 0
// adds the 64 chunk partials in order into the pass's group partial g.
// Pass 0 sums a; pass 1 first forms the mean from pass 0's group partials
// (workgroup 0 stores it in stats[0]) and sums (a - mean)^2, and its last
// workgroup stores inv in stats[1].  A16: a is 16-byte aligned (each lane's
// four elements in one load).
template <bool A16>
__global__ __launch_bounds__(NORM_THREADS) void norm_pass_kernel(const float* __restrict__ a, uint64_t count,
                                                                 double* __restrict__ part, float* __restrict__ stats,
                                                                 float eps, int pass) {
    __shared__ double sp[257];
    __shared__ double s_chunk[NORM_GROUP];
    __shared__ uint32_t s_last;
    const uint64_t chunks = (count + CHUNK - 1) / CHUNK, groups = (chunks + NORM_GROUP - 1) / NORM_GROUP;
    uint32_t* ticket = reinterpret_cast<uint32_t*>(part);
    double* p0 = part + 1;
    double* p1 = p0 + groups;
    const uint32_t w = threadIdx.x / 64, l = threadIdx.x % 64;
    const double first = pass != 0 && threadIdx.x < groups ? p0[threadIdx.x] : 0.0;
    const uint64_t c0 = uint64_t(blockIdx.x) * NORM_GROUP + NORM_WAVE_CHUNKS * w;
    float x[NORM_WAVE_CHUNKS][4];
#pragma unroll
    for (uint32_t i = 0; i < NORM_WAVE_CHUNKS; i++) {
        const uint64_t e = (c0 + i) * CHUNK + 4 * l;
        if (A16 && e + 3 < count) {
            const float4 v4 = *reinterpret_cast<const float4*>(a + e);
            x[i][0] = v4.x; x[i][1] = v4.y; x[i][2] = v4.z; x[i][3] = v4.w;
        } else {
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) x[i][j] = e + j < count ? a[e + j] : 0.0f;
        }
    }
    float mean = 0.0f;
    if (pass != 0) {
        mean = float(sequential_total(p0, groups, first, sp) / double(count));
        if (blockIdx.x == 0 && threadIdx.x == 0) stats[0] = mean;
    }
#pragma unroll
    for (uint32_t i = 0; i < NORM_WAVE_CHUNKS; i++) {
        const uint64_t e = (c0 + i) * CHUNK + 4 * l;
        double s = 0.0;
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
            if (e + j < count) {
                if (pass == 0) {
                    s += double(x[i][j]);
                } else {
                    const double d = double(x[i][j] - mean);
                    s += d * d;
                }
            }
        }
        s = chunk_tree(s);
        if (l == 0) s_chunk[NORM_WAVE_CHUNKS * w + i] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint64_t cg = uint64_t(blockIdx.x) * NORM_GROUP;
        const uint32_t k = uint32_t(chunks - cg < NORM_GROUP ? chunks - cg : NORM_GROUP);
        double v = 0.0;
#pragma unroll 1
        for (uint32_t c = 0; c < NORM_GROUP; c += 16) {
            double y[16];
#pragma unroll
            for (uint32_t j = 0; j < 16; j++) y[j] = s_chunk[c + j];
            if (c + 16 <= k) {
#pragma unroll
                for (uint32_t j = 0; j < 16; j++) v += y[j];
            } else {
#pragma unroll
                for (uint32_t j = 0; j < 16; j++)
                    if (c + j < k) v += y[j];
            }
        }
        if (pass == 0) {
            p0[blockIdx.x] = v;
        } else {
            // the partial is released with the count; the workgroup that
            // takes the last ticket acquires every other one's partial
            p1[blockIdx.x] = v;
            const uint32_t taken = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            s_last = taken == groups - 1;
            if (s_last) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (pass == 0) return;
    __syncthreads();
    if (!s_last) return;
    const double total = sequential_total(p1, groups, threadIdx.x < groups ? p1[threadIdx.x] : 0.0, sp);
    if (threadIdx.x == 0) stats[1] = 1.0f / sqrt_f(float(total / double(count)) + eps);
}
// (a - mean) * inv over the workgroup's NORM_APPLY elements (loaded at
// once), with (mean, inv) from stats.
constexpr uint32_t NORM_APPLY = 4096;
__global__ __launch_bounds__(256) void norm_apply_kernel(float* __restrict__ a, uint64_t count,
                                                         const float* __restrict__ stats) {
    const uint64_t e0 = uint64_t(blockIdx.x) * NORM_APPLY;
    float x[NORM_APPLY / 256];
#pragma unroll
    for (uint32_t j = 0; j < NORM_APPLY / 256; j++) {
        const uint64_t i = e0 + threadIdx.x + 256 * j;
        x[j] = i < count ? a[i] : 0.0f;
    }
    const float mean = stats[0], inv = stats[1];
#pragma unroll
    for (uint32_t j = 0; j < NORM_APPLY / 256; j++) {
        const uint64_t i = e0 + threadIdx.x + 256 * j;
        if (i < count) a[i] = (x[j] - mean) * inv;
    }
}

// ---------------------------------------------------------------- minibatch chunk
// One workgroup per 256-row chunk of a minibatch: critic and actor forward,
// per-row loss and derivatives (ppo.hpp:144-181), hidden deltas
// (ppo.metal:470-485, 618-631) and every parameter's partial sum over the
// chunk's rows (cpu_reference.hpp:515-551), written to the chunk's partial
// vector.  Activations and deltas stay in LDS.
//
// The GEMMs run on the fp32 matrix cores.  v_mfma_f32_32x32x2_f32 applies
// acc = fma(a[k], b[k], acc) for k = 0 then 1 with one rounding per step, so
// a chain of them over k ascending is exactly the canonical fma chain:
//   forward:  h[row][j] = fma over inputs i ascending, from b1[j];
//   backward: dW1[j][i] = fma over the chunk's rows ascending, from 0.
// Operand layout (per wavefront, one 32x32 tile): A lane a holds A[a%32][k0 +
// a/32], B lane a holds B[k0 + a/32][a%32]; accumulator register r of lane l
// holds D[8(r/4) + 4(l/32) + r%4][l%32].  Padding steps multiply by -0.0,
// which leaves every accumulator (including -0.0) unchanged.
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ v16f mfma32(float a, float b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t acc_row(uint32_t l, uint32_t r) { return 8 * (r / 4) + 4 * (l / 32) + (r % 4); }

constexpr uint32_t HS = HID + 1;       // row stride of the [256][64] activation buffer
constexpr uint32_t CHUNK_PF = 3;       // MFMA steps between an operand's LDS read and its use
constexpr uint32_t BR = 32;            // backward: rows per row-slab
constexpr uint32_t OBS_PAD = 192;      // inputs rounded up to whole 32-wide tiles
constexpr uint32_t XRS = OBS_PAD + 32; // stride of the backward row slab [32][192]
constexpr uint32_t RS = 12;            // per-row scalars: dm[4], dls[4], loss terms and ratio[4]

// A chunk's workgroup: CW = 8 wavefronts, two per SIMD, so that one
// wavefront's LDS reads and VALU work overlap the other's matrix-core work.
// Row-wise phases run on threads 0-255 (thread t owns row t of the chunk).
constexpr uint32_t CW = 8, CT = 64 * CW;
// shared scratch: the critic's staged first layer and the forwards' input
// tiles (one [32][XWS] tile per wavefront), the backward row slabs, after
// the actor forward the per-row scalars
constexpr uint32_t XWS = 17;  // row stride of a wavefront's input tile
constexpr uint32_t XW_BASE = COBS * HID;
constexpr uint32_t U_WORDS = BR * XRS > XW_BASE + CW * 32 * XWS ? BR * XRS : XW_BASE + CW * 32 * XWS;
static_assert(256 * RS <= U_WORDS, "the per-row scalars fit the shared scratch");

// A first layer staged in LDS, transposed: W1[u][k] at w1_pos(k, u) =
// 64 k + (u ^ 32 (k & 1)), so the two input rows of one MFMA step's B
// operand (k even in lanes 0-31, odd in lanes 32-63) fall in different halves
// of the banks.
__device__ __forceinline__ uint32_t w1_pos(uint32_t k, uint32_t u) { return k * HID + (u ^ (32u * (k & 1u))); }
// W1T [D][64] (global, input-major) into LDS for inputs 0 .. KP-1, the
// inputs past D as -0, in two halves so that a kernel can issue every load
// of its prologue before the first store.
template <uint32_t D, uint32_t KP>
__device__ __forceinline__ void stage_w1_load(const float* __restrict__ W1T, float (&v)[KP * HID / CT]) {
    static_assert(KP * HID % CT == 0, "whole staging rounds");
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (uint32_t j = 0; j < KP * HID / CT; j++) {
        const uint32_t e = t + CT * j;
        v[j] = e / HID < D ? W1T[e] : -0.0f;
    }
}
template <uint32_t D, uint32_t KP>
__device__ __forceinline__ void stage_w1_store(const float (&v)[KP * HID / CT], float* sw) {
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (uint32_t j = 0; j < KP * HID / CT; j++) {
        const uint32_t e = t + CT * j;
        sw[w1_pos(e / HID, e % HID)] = v[j];
    }
}

// h[256][64] = tanh(X W1^T + b1) for the chunk's rows (rows past b read as
// 0), with W1 staged by stage_w1_load/stage_w1_store<D, KP>.  Wavefront w owns rows 32w..32w+31
// as two 32x32 tiles (hidden units 0-31, 32-63).  It fetches its rows'
// inputs in blocks of 16 (each load instruction covering 4 rows x 16
// consecutive inputs), two blocks ahead of the matrix cores, and passes each
// block through its own LDS tile xw [32][17] into the A operand (lane l: row
// l % 32, the inputs of parity l / 32); each step's B operand comes from the
// staged layer.  Every block runs all 16 inputs (inputs past D hold x = +0
// and w = -0, whose product -0 leaves each accumulator unchanged).  No
// workgroup barrier falls before the activations (tanh) are formed, so one
// wavefront's activations overlap the other's MFMAs on a SIMD; with WAIT a
// barrier separates them from the stores into s_h (whose previous readers
// may still run).
template <uint32_t D, uint32_t KP, bool WAIT>
__device__ __forceinline__ void chunk_forward(const float* __restrict__ X, const float* sw, float* xw_all,
                                              const float* __restrict__ b1, uint32_t n0, uint32_t b, float* s_h) {
    static_assert(KP % 16 == 0 && KP >= D, "whole input blocks");
    constexpr uint32_t NB = KP / 16;
    const uint32_t t = threadIdx.x, wv = t / 64, l = t % 64, hf = l / 32;
    float* xw = xw_all + wv * 32 * XWS;
    v16f acc[2];
#pragma unroll
    for (uint32_t ct = 0; ct < 2; ct++) {
        const float bias = b1[32 * ct + l % 32];
#pragma unroll
        for (uint32_t r = 0; r < 16; r++) acc[ct][r] = bias;
    }
    // load i of a block: row 4 i + l / 16 of the wavefront's rows, input l % 16
    const uint32_t lr = l / 16, lk = l % 16;
    float xg[3][8];
    auto xload = [&](uint32_t p, uint32_t blk) {
        const uint32_t k = 16 * blk + lk;
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            const uint32_t row = n0 + 32 * wv + 4 * i + lr;
            const bool ok = row < b && k < D;
            const float v = X[size_t(row < b ? row : n0) * D + (k < D ? k : D - 1)];
            xg[p][i] = ok ? v : 0.0f;
        }
    };
    xload(0, 0);
    if (NB > 1) xload(1, 1);
    for (uint32_t j0 = 0; j0 < NB; j0 += 3) {
#pragma unroll
        for (uint32_t p = 0; p < 3; p++) {
            const uint32_t j = j0 + p;
            if (j >= NB) break;
#pragma unroll
            for (uint32_t i = 0; i < 8; i++) xw[(4 * i + lr) * XWS + lk] = xg[p][i];
            if (j + 2 < NB) xload((p + 2) % 3, j + 2);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            float av[8], bv[8][2];
#pragma unroll
            for (uint32_t i = 0; i < 8; i++) {
                av[i] = xw[(l % 32) * XWS + 2 * i + hf];
                const uint32_t k = 16 * j + 2 * i + hf;
#pragma unroll
                for (uint32_t ct = 0; ct < 2; ct++) bv[i][ct] = sw[k * HID + 32 * (ct ^ hf) + l % 32];
            }
#pragma unroll
            for (uint32_t i = 0; i < 8; i++)
#pragma unroll
                for (uint32_t ct = 0; ct < 2; ct++) acc[ct] = mfma32(av[i], bv[i][ct], acc[ct]);
            // this block's tile reads precede the next block's writes
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
#pragma unroll
    for (uint32_t ct = 0; ct < 2; ct++)
#pragma unroll
        for (uint32_t r = 0; r < 16; r++) acc[ct][r] = tanh_f(acc[ct][r]);
    if (WAIT) __syncthreads();  // s_h's previous readers are done
#pragma unroll
    for (uint32_t ct = 0; ct < 2; ct++)
#pragma unroll
        for (uint32_t r = 0; r < 16; r++) s_h[(32 * wv + acc_row(l, r)) * HS + 32 * ct + l % 32] = acc[ct][r];
    __syncthreads();
}

// s = fma(a[r], b[r * bs], s) (MUL) or s = s + b[r * bs] for r = r0 .. r1-1
// ascending, operands in LDS; a is read four rows at a time (16-byte reads,
// r0 a multiple of 4).  The reads of a block of CH_NB rows are issued before
// the previous block's arithmetic, so a dependent chain does not wait on
// every read.  A span of exactly FULL rows (a whole chunk or slab) takes a
// loop with a fixed trip count; other spans take the general loop.
constexpr uint32_t CH_NB = 8;
template <bool MUL, uint32_t FULL>
__device__ __forceinline__ float lds_chain(const float* a, const float* b, uint32_t bs, uint32_t r0, uint32_t r1,
                                           float s) {
    static_assert(FULL % (2 * CH_NB) == 0, "whole block pairs");
    float4 av[2][CH_NB / 4];
    float bv[2][CH_NB];
    auto load = [&](uint32_t p, uint32_t r) {
        if (MUL)
#pragma unroll
            for (uint32_t i = 0; i < CH_NB / 4; i++) av[p][i] = *reinterpret_cast<const float4*>(a + r + 4 * i);
#pragma unroll
        for (uint32_t i = 0; i < CH_NB; i++) bv[p][i] = b[(r + i) * bs];
    };
    auto use = [&](uint32_t p) {
#pragma unroll
        for (uint32_t i = 0; i < CH_NB; i++) {
            if (MUL) s = fma_f(av[p][i / 4][i % 4], bv[p][i], s);
            else s = s + bv[p][i];
        }
    };
    if (r1 - r0 == FULL) {
        load(0, r0);
#pragma unroll 4
        for (uint32_t j = 0; j < FULL; j += 2 * CH_NB) {
            load(1, r0 + j + CH_NB);
            use(0);
            if (j + 2 * CH_NB < FULL) load(0, r0 + j + 2 * CH_NB);
            use(1);
        }
        return s;
    }
    const uint32_t nfull = r0 + (r1 - r0) / CH_NB * CH_NB;
    uint32_t r = r0;
    if (r < nfull) load(0, r);
    while (r < nfull) {
        const bool more = r + CH_NB < nfull;
        if (more) load(1, r + CH_NB);
        use(0);
        r += CH_NB;
        if (!more) break;
        const bool more2 = r + CH_NB < nfull;
        if (more2) load(0, r + CH_NB);
        use(1);
        r += CH_NB;
        if (!more2) break;
    }
    for (; r < r1; r++) s = MUL ? fma_f(a[r], b[r * bs], s) : s + b[r * bs];
    return s;
}

// Backward row slab in registers: BR rows x W columns, element e = t + CT j.
template <uint32_t W>
struct RowSlab {
    float x[BR * W / CT];
};
// Column D (inside the padding, D < W) holds 1 for the chunk's rows: its
// products with the deltas form the first-layer bias gradient in the same
// chain (fma(d, 1, s) rounds as s + d).
template <uint32_t D, uint32_t W>
__device__ __forceinline__ void row_load(RowSlab<W>& f, const float* __restrict__ X, uint32_t n0, uint32_t rows,
                                         uint32_t r0) {
    static_assert(D < W, "a padding column for the bias");
#pragma unroll
    for (uint32_t j = 0; j < BR * W / CT; j++) {
        const uint32_t e = threadIdx.x + CT * j, rr = e / W, cc = e % W;
        const bool rok = r0 + rr < rows;
        const float v = X[size_t(n0 + (rok ? r0 + rr : 0)) * D + (cc < D ? cc : 0)];
        f.x[j] = rok && cc < D ? v : (rok && cc == D ? 1.0f : -0.0f);
    }
}

// dW1[j][i] partial over the chunk's rows: A = delta^T (s_h, [row][64]),
// B = the input rows streamed from global in slabs of 32 rows (W columns, a
// multiple of 32 covering D and the ones column D) through LDS; the first
// slab arrives in f, fetched by the caller ahead of time.  Wavefront tiles
// are the (jt[q], it[q]) pairs; the tile holding column D also yields b1
// (into b1_out).
template <uint32_t D, uint32_t W, uint32_t T>
__device__ __forceinline__ void chunk_weight_grad(RowSlab<W>& f, const float* __restrict__ X, uint32_t n0,
                                                  uint32_t rows, const uint32_t (&jt)[T], const uint32_t (&it)[T],
                                                  bool owner, float* s_u, const float* s_h, float* __restrict__ out,
                                                  float* __restrict__ b1_out) {
    constexpr uint32_t WS = W + 32;  // slab row stride: the two k halves fall in different banks
    const uint32_t t = threadIdx.x, l = t % 64;
    float* sx = s_u;  // [BR][WS]
    v16f acc[T];
#pragma unroll
    for (uint32_t q = 0; q < T; q++)
#pragma unroll
        for (uint32_t r = 0; r < 16; r++) acc[q][r] = 0.0f;
    for (uint32_t r0 = 0; r0 < rows; r0 += BR) {
#pragma unroll
        for (uint32_t j = 0; j < BR * W / CT; j++) {
            const uint32_t e = t + CT * j;
            sx[(e / W) * WS + e % W] = f.x[j];
        }
        __syncthreads();
        if (r0 + BR < rows) row_load<D, W>(f, X, n0, rows, r0 + BR);
        if (owner) {
            // every slab runs all BR rows (rows past the chunk's hold
            // deltas +0 and inputs -0: a -0 product, no change); each step's
            // LDS operands are read CHUNK_PF steps ahead of its MFMAs
            constexpr uint32_t NS = BR / 2;
            float av[NS][T], bv[NS][T];
#pragma unroll
            for (uint32_t st = 0; st < NS + CHUNK_PF; st++) {
                if (st < NS) {
                    const uint32_t rr = 2 * st + l / 32;
#pragma unroll
                    for (uint32_t q = 0; q < T; q++) {
                        av[st][q] = s_h[(r0 + rr) * HS + 32 * jt[q] + l % 32];
                        bv[st][q] = sx[rr * WS + 32 * it[q] + l % 32];
                    }
                }
                if (st >= CHUNK_PF) {
                    const uint32_t u = st - CHUNK_PF;
#pragma unroll
                    for (uint32_t q = 0; q < T; q++) acc[q] = mfma32(av[u][q], bv[u][q], acc[q]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        __syncthreads();
    }
    if (!owner) return;
#pragma unroll
    for (uint32_t q = 0; q < T; q++) {
        const uint32_t i = 32 * it[q] + l % 32;
        if (i < D) {
#pragma unroll
            for (uint32_t r = 0; r < 16; r++) out[(32 * jt[q] + acc_row(l, r)) * D + i] = acc[q][r];
        } else if (i == D) {
#pragma unroll
            for (uint32_t r = 0; r < 16; r++) b1_out[32 * jt[q] + acc_row(l, r)] = acc[q][r];
        }
    }
}

// A stored advantage, normalised on the fly when a.norm is set (ppo.hpp:139).
__device__ __forceinline__ float normalized_advantage(const RowArgs& a, float adv) {
    return a.norm ? (adv - a.norm[0]) * a.norm[1] : adv;
}
// Row m's advantage, normalised when a.norm is set.
__device__ __forceinline__ float row_advantage(const RowArgs& a, uint32_t m) {
    return normalized_advantage(a, a.adv[m]);
}
// exp_f(-ls[j]) for j < 4, exp_f(-2 ls[j - 4]) for j = 4..7: the per-action
// scale factors of row_objective, the same for every row, formed once per
// workgroup
__device__ __forceinline__ float row_scale_exp(const float* ls, uint32_t j) {
    return j < 4 ? exp_f(-ls[j]) : exp_f(-2.0f * ls[j - 4]);
}
// Per-row objective (ppo.hpp:144-181): log-probability of the stored
// action, clipped surrogate with its active branch, value loss, and the
// derivatives of the minibatch-mean objective (scale = 1/b).  ex holds
// row_scale_exp of j = 0..7; act and old_logp are the row's stored action
// and log-probability.  Writes scalar i at rs[RSTRIDE i]: 0..3 d mean,
// 4..7 d log_std, 8..11 the row's policy, value and entropy terms and its
// ratio.
template <uint32_t RSTRIDE = 1>
__device__ __forceinline__ void row_objective(const RowArgs& a, const float* ls, const float* ex,
                                              const float (&act)[4], float old_logp, float adv,
                                              const float (&mean)[4], float value, float target, float scale,
                                              float (&dmean)[4], float* rs) {
    float logp = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) {
        const float inv_std = ex[q];  // exp_f(-ls[q])
        const float d = (act[q] - mean[q]) * inv_std;
        logp += -0.5f * (d * d + 2.0f * ls[q] + LOG_TWO_PI);
    }
    const float raw = logp - old_logp;
    const float lr = clamp_f(raw, -20.0f, 20.0f);
    const float ratio = exp_f(lr);
    const float clipped = clamp_f(ratio, 1.0f - a.clip, 1.0f + a.clip);
    const float chosen = min_f(ratio * adv, clipped * adv);
    const bool in_range = raw >= -20.0f && raw <= 20.0f;
    const bool active = in_range && (adv >= 0.0f ? ratio <= 1.0f + a.clip : ratio >= 1.0f - a.clip);
    float entropy = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) {
        const float inv_var = ex[4 + q];  // exp_f(-2.0f * ls[q])
        const float diff = act[q] - mean[q];
        float dl;
        if (active) {
            const float dlogp = -ratio * adv * scale;
            dmean[q] = dlogp * diff * inv_var;
            dl = dlogp * (diff * diff * inv_var - 1.0f);
        } else {
            dmean[q] = 0.0f;
            dl = 0.0f;
        }
        dl -= a.ecoef * scale;
        entropy += -a.ecoef * (ls[q] + 0.5f * (1.0f + LOG_TWO_PI)) * scale;
        rs[RSTRIDE * q] = dmean[q];
        rs[RSTRIDE * (4 + q)] = dl;
    }
    rs[RSTRIDE * 8] = -chosen * scale;
    rs[RSTRIDE * 9] = 0.5f * a.vcoef * (value - target) * (value - target) * scale;
    rs[RSTRIDE * 10] = entropy;
    rs[RSTRIDE * 11] = ratio;
}

template <uint32_t D>
__global__ __launch_bounds__(CT) void chunk_kernel(RowArgs a) {
    using L = AL<D>;
    __shared__ float s_h[256 * HS];
    __shared__ __attribute__((aligned(16))) float s_u[U_WORDS];
    __shared__ float s_aw[OBS_PAD * HID];  // the actor's first layer (stage_w1_store)
    __shared__ __attribute__((aligned(16))) float s_dv[256];
    // the critic's w2 and the actor's W2 [4][64], read by every row's chains:
    // one LDS copy (broadcast reads) instead of per-step global loads
    __shared__ __attribute__((aligned(16))) float s_w2[5 * HID];
    __shared__ float s_ex[8];  // exp(-log_std), exp(-2 log_std): the same for every row
    const uint32_t t = threadIdx.x, wv = t / 64;
    const bool rowt = t < 256;  // the row-wise phases' threads
    const uint32_t n0 = blockIdx.x * 256;
    const uint32_t rows = a.b - n0 < 256 ? a.b - n0 : 256;
    const bool live = t < rows;
    const uint32_t n = n0 + t, m = live ? n : n0;
    float* P = a.part + size_t(blockIdx.x) * L::P_TOTAL;
    const float scale = 1.0f / max_f(float(a.b), 1.0f);
    // every global load of the prologue issued before its first LDS store:
    // the output layers' weights (thread t < 5 HID) or a log-std (the next
    // 8), both first layers, and the row's advantage (read before the first
    // barrier, stored back for live rows after it) and return
    const uint32_t xj = t - 5 * HID;  // row_scale_exp index of threads 5 HID .. 5 HID + 7
    const float w2v = t < HID ? a.critic[C_W2 + t]
                    : t < 5 * HID ? a.actor[L::W2 + t - HID]
                                  : a.actor[L::LS + (t < 5 * HID + 8 ? xj % 4 : 0)];
    float cwv[COBS * HID / CT], awv[OBS_PAD * HID / CT];
    stage_w1_load<COBS, COBS>(a.critic_w1t, cwv);
    stage_w1_load<D, OBS_PAD>(a.actor_w1t, awv);
    const float adv_raw = a.adv[m];
    const float target = a.ret[m];
    if (t < 5 * HID) s_w2[t] = w2v;
    else if (t < 5 * HID + 8) s_ex[xj] = xj < 4 ? exp_f(-w2v) : exp_f(-2.0f * w2v);  // row_scale_exp
    stage_w1_store<COBS, COBS>(cwv, s_u);
    stage_w1_store<D, OBS_PAD>(awv, s_aw);
    const float adv = normalized_advantage(a, adv_raw);

    // ---- critic: forward, value, dV (ppo.hpp:82-93, 176-180)
    __syncthreads();
    chunk_forward<COBS, COBS, false>(a.co, s_u, s_u + XW_BASE, a.critic + C_B1, n0, a.b, s_h);
    RowSlab<2 * COBS> fc;  // the critic inputs' first row slab, fetched ahead of the W1 gradient
    row_load<COBS, 2 * COBS>(fc, a.co, n0, rows, 0);
    float value = a.critic[C_B2];
    if (rowt) value = lds_chain<true, HID>(s_w2, s_h + t * HS, 1, 0, HID, value);
    const float dvalue = a.vcoef * (value - target) * scale;
    if (rowt) s_dv[t] = live ? dvalue : 0.0f;
    __syncthreads();
    if (t < HID)  // critic w2: fma over rows
        P[L::COUNT + C_W2 + t] = lds_chain<true, 256>(s_dv, s_h + t, HS, 0, rows, 0.0f);
    else if (t == 256)  // critic b2
        P[L::COUNT + C_B2] = lds_chain<false, 256>(nullptr, s_dv, 1, 0, rows, 0.0f);
    __syncthreads();
    // critic hidden delta in place, row t % 256, units 32 (t / 256) .. + 31
    const uint32_t hrow = t % 256, hk0 = 32 * (t / 256);
    const bool hlive = hrow < rows;
    {
        const float dv = s_dv[hrow];
#pragma unroll 8
        for (uint32_t k = hk0; k < hk0 + 32; k++) {
            const float g = s_h[hrow * HS + k];
            const float d = dv * s_w2[k] * (1.0f - g * g);
            s_h[hrow * HS + k] = hlive ? d : 0.0f;
        }
    }
    // critic W1 [64][32] and b1: wavefronts 0-3 own one 32x32 tile each
    // (inputs 0-31, then the ones column and its padding)
    {
        const uint32_t jt[1] = {wv & 1}, it[1] = {(wv / 2) & 1};
        chunk_weight_grad<COBS, 2 * COBS, 1>(fc, a.co, n0, rows, jt, it, wv < 4, s_u, s_h, P + L::COUNT,
                                             P + L::COUNT + C_B1);
    }

    // ---- actor: forward, means, loss and derivatives
    chunk_forward<D, OBS_PAD, false>(a.obs, s_aw, s_u + XW_BASE, a.actor + L::B1, n0, a.b, s_h);
    RowSlab<OBS_PAD> fa;  // the inputs' first row slab, fetched ahead of the W1 gradient
    row_load<D, OBS_PAD>(fa, a.obs, n0, rows, 0);
    float* rs_t = s_u;  // per-row scalars [12][256] (scalar-major): the row slabs are done with
    if (rowt) {
        float mean[4];
#pragma unroll
        for (uint32_t q = 0; q < 4; q++) mean[q] = a.actor[L::B2 + q];
        {   // the four chains over the hidden units side by side, each block
            // of 8 units read before the previous block's fmas
            constexpr uint32_t MB = 8;
            float hv[2][MB];
            float4 wv4[2][4][MB / 4];
            auto load = [&](uint32_t p, uint32_t k0) {
#pragma unroll
                for (uint32_t i = 0; i < MB; i++) hv[p][i] = s_h[t * HS + k0 + i];
#pragma unroll
                for (uint32_t q = 0; q < 4; q++)
#pragma unroll
                    for (uint32_t i = 0; i < MB / 4; i++)
                        wv4[p][q][i] = *reinterpret_cast<const float4*>(s_w2 + HID + q * HID + k0 + 4 * i);
            };
            auto use = [&](uint32_t p) {
#pragma unroll
                for (uint32_t i = 0; i < MB; i++)
#pragma unroll
                    for (uint32_t q = 0; q < 4; q++) mean[q] = fma_f(wv4[p][q][i / 4][i % 4], hv[p][i], mean[q]);
            };
            load(0, 0);
#pragma unroll
            for (uint32_t k0 = 0; k0 < HID; k0 += 2 * MB) {
                load(1, k0 + MB);
                use(0);
                if (k0 + 2 * MB < HID) load(0, k0 + 2 * MB);
                use(1);
            }
        }
        // geometry prior (ppo.hpp:77): the hint inputs add to the first three means
        if (D == MDN_ACTOR_OBS_PRIOR)
#pragma unroll
            for (uint32_t q = 0; q < 3; q++) mean[q] += a.obs[size_t(m) * D + D - 3 + q];
        float dmean[4];
        const float* ap = a.actions + size_t(m) * 4;
        const float act[4] = {ap[0], ap[1], ap[2], ap[3]};
        row_objective<256>(a, a.actor + L::LS, s_ex, act, a.old_logp[m], adv, mean, value, target, scale, dmean,
                           rs_t + t);
        if (a.norm && live) a.adv_out[m] = adv;
    }
    __syncthreads();
    // the d means of row t % 256, read before the barrier after which the
    // weight gradient's row slabs overwrite the per-row scalars
    float dm[4];
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) dm[q] = rs_t[q * 256 + hrow];
    if (rowt) {   // actor W2[q][k]: fma over rows
        const uint32_t q = t / HID, k = t % HID;
        P[L::W2 + q * HID + k] = lds_chain<true, 256>(rs_t + q * 256, s_h + k, HS, 0, rows, 0.0f);
    } else if (t < 256 + 12) {  // b2, log_std and the metric sums: sums over rows
        const uint32_t col = t - 256;
        P[col < 4 ? L::B2 + col : col < 8 ? L::LS + (col - 4) : L::COUNT + C_COUNT + (col - 8)] =
            lds_chain<false, 256>(nullptr, rs_t + col * 256, 1, 0, rows, 0.0f);
    }
    __syncthreads();
    {   // actor hidden delta in place, row t % 256, units 32 (t / 256) .. + 31
#pragma unroll 8
        for (uint32_t k = hk0; k < hk0 + 32; k++) {
            float d = 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < 4; q++) d = fma_f(dm[q], s_w2[HID + q * HID + k], d);
            const float h = s_h[hrow * HS + k];
            const float dh = d * (1.0f - h * h);
            s_h[hrow * HS + k] = hlive ? dh : 0.0f;
        }
    }
    // actor W1 [64][D] and b1 (the ones column D in tiles (j, 5)): 2 x 6
    // tiles of 32x32.  Wavefronts w and w + 4 share a SIMD and take three
    // tiles between them: tiles 2w and 2w + 1 for w < 4, tile w + 4 for the
    // others.  Both paths run the same slabs and barriers (a workgroup
    // barrier counts arrivals, not code positions); the first slab's barrier
    // also orders the deltas before their reads.
    if (wv < 4) {
        const uint32_t jt[2] = {(2 * wv) / 6, (2 * wv + 1) / 6};
        const uint32_t it[2] = {(2 * wv) % 6, (2 * wv + 1) % 6};
        chunk_weight_grad<D, OBS_PAD, 2>(fa, a.obs, n0, rows, jt, it, true, s_u, s_h, P, P + L::B1);
    } else {
        const uint32_t jt[1] = {(wv + 4) / 6}, it[1] = {(wv + 4) % 6};
        chunk_weight_grad<D, OBS_PAD, 1>(fa, a.obs, n0, rows, jt, it, true, s_u, s_h, P, P + L::B1);
    }
}

// Chunk partials summed within groups of GRAD_GROUP chunks, in place into
// the group's first chunk row; grid (param blocks, groups).
__global__ __launch_bounds__(256) void group_reduce_kernel(float* __restrict__ part, uint32_t chunks, uint32_t ptot) {
    const uint32_t p = blockIdx.x * 256 + threadIdx.x;
    const uint32_t c0 = blockIdx.y * GRAD_GROUP;
    if (p >= ptot || c0 >= chunks) return;
    const uint32_t end = c0 + GRAD_GROUP < chunks ? c0 + GRAD_GROUP : chunks;
    float s = 0.0f;
    for (uint32_t c = c0; c < end; c++) s += part[size_t(c) * ptot + p];
    part[size_t(c0) * ptot + p] = s;
}
// Sequential sum over the group sums: grad[p] = 0 + g0[p] + g1[p] + ...
__global__ __launch_bounds__(256) void chunk_reduce_kernel(const float* __restrict__ part, float* __restrict__ grad,
                                                           uint32_t chunks, uint32_t ptot) {
    const uint32_t p = blockIdx.x * 256 + threadIdx.x;
    if (p >= ptot) return;
    float total = 0.0f;
    for (uint32_t c = 0; c < chunks; c += GRAD_GROUP) total += part[size_t(c) * ptot + p];
    grad[p] = total;
}

// ---------------------------------------------------------------- minibatches of one chunk
// A minibatch of at most 256 rows is one gradient chunk, so every parameter's
// sum runs over its rows in order (the reference's own order at its 256-row
// minibatch).  chunk_kernel would run it in one workgroup; here the rows'
// forward, objective and hidden deltas run in ceil(b/16) workgroups and the
// parameter sums in 69 more, each chain still over the rows ascending:
//   mb_forward_kernel: 16 rows per workgroup, wavefronts 0-3 take the actor's
//     hidden units 16w..16w+15 and 4-7 the critic's on 16x16x4 fp32 MFMA
//     chains over the inputs from the bias (the fma chain of chunk_forward);
//     then means and value (fma chains over the 64 units), row_objective and
//     the hidden deltas, all written to the row records;
//   mb_grad_kernel: every parameter's sum as a 16x16x4 MFMA chain over the
//     rows, one 16x16 tile per wavefront (below).
// Each gradient is stored as 0 + (0 + sum), the value the chunk reduction
// (group sum from 0, then the sum of groups from 0) gives for one chunk.
constexpr uint32_t MB_HA = 0, MB_DA = 256 * 64, MB_HC = 2 * 256 * 64, MB_DC = 3 * 256 * 64, MB_RS = 4 * 256 * 64;
constexpr uint32_t MB_FWD_ROWS = 16;
template <uint32_t D>
__global__ __launch_bounds__(512) void mb_forward_kernel(MbArgs m) {
    using L = AL<D>;
    const RowArgs& a = m.r;
    constexpr uint32_t XS = D | 1u, WS = HID + 1;  // odd strides: rows fall in distinct banks
    __shared__ float s_w[D * WS];                  // actor W1^T [input][unit]
    __shared__ float s_cw[COBS * WS];              // critic W1^T
    __shared__ float s_t[5 * HID + 8 + 2 * HID + 1];  // actor b1, W2, b2, log_std; critic b1, w2, b2
    __shared__ float s_x[MB_FWD_ROWS][XS];
    __shared__ float s_c[MB_FWD_ROWS][COBS + 1];
    __shared__ float s_ha[MB_FWD_ROWS][HID + 1];
    __shared__ float s_hc[MB_FWD_ROWS][HID + 1];
    __shared__ float s_mv[MB_FWD_ROWS][5];   // means, value
    __shared__ float s_rs[MB_FWD_ROWS][16];  // d mean, d log_std, metric terms, d value
    __shared__ float s_ex[8];                 // row_scale_exp
    const uint32_t t = threadIdx.x, wv = t / 64, l = t % 64;
    const uint32_t n0 = blockIdx.x * MB_FWD_ROWS;
    const uint32_t live_rows = a.b - n0 < MB_FWD_ROWS ? a.b - n0 : MB_FWD_ROWS;
    constexpr uint32_t AT = 5 * HID + 8;  // actor tail words from b1 on
    float* s_at = s_t;
    float* s_ct = s_t + AT;
    float ract[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float rolp = 0.0f, radv = 0.0f, rret = 0.0f;
    {   // every load of the staging issued before any store
        constexpr uint32_t NW = (D * HID + 511) / 512, NCW = COBS * HID / 512, NX = (MB_FWD_ROWS * D + 511) / 512;
        float w[NW], cw[NCW], xv[NX], cv, tv[2];
        // the first layers from the flat vectors ([unit][input]), transposed
        // into LDS (the transposed copies are refreshed once per update)
#pragma unroll
        for (uint32_t k = 0; k < NW; k++) {
            const uint32_t e = t + 512 * k;
            w[k] = e < D * HID ? a.actor[e] : 0.0f;
        }
#pragma unroll
        for (uint32_t k = 0; k < NCW; k++) cw[k] = a.critic[t + 512 * k];
#pragma unroll
        for (uint32_t k = 0; k < NX; k++) {
            const uint32_t e = t + 512 * k, r = e / D;
            xv[k] = e < MB_FWD_ROWS * D && r < live_rows ? a.obs[size_t(n0) * D + e] : 0.0f;
        }
        {
            const uint32_t r = t / COBS;
            cv = r < live_rows ? a.co[size_t(n0) * COBS + t] : 0.0f;  // 512 = 16 rows x 32
        }
        tv[0] = t < AT ? a.actor[L::B1 + t] : 0.0f;
        tv[1] = t < 2 * HID + 1 ? a.critic[C_B1 + t] : 0.0f;
        if (t < live_rows) {  // the row's objective inputs, used after the layers
            const uint32_t mrow = n0 + t;
#pragma unroll
            for (uint32_t q = 0; q < 4; q++) ract[q] = a.actions[size_t(mrow) * 4 + q];
            rolp = a.old_logp[mrow];
            radv = a.adv[mrow];  // normalised where it is used, so no load waits on it here
            rret = a.ret[mrow];
        }
#pragma unroll
        for (uint32_t k = 0; k < NW; k++) {
            const uint32_t e = t + 512 * k;
            if (e < D * HID) s_w[(e % D) * WS + e / D] = w[k];
        }
#pragma unroll
        for (uint32_t k = 0; k < NCW; k++) {
            const uint32_t e = t + 512 * k;
            s_cw[(e % COBS) * WS + e / COBS] = cw[k];
        }
#pragma unroll
        for (uint32_t k = 0; k < NX; k++) {
            const uint32_t e = t + 512 * k;
            if (e < MB_FWD_ROWS * D) s_x[e / D][e % D] = xv[k];
        }
        s_c[t / COBS][t % COBS] = cv;
        if (t < AT) s_at[t] = tv[0];
        if (t < 2 * HID + 1) s_ct[t] = tv[1];
    }
    static_assert(MB_FWD_ROWS * COBS == 512 && COBS * HID % 512 == 0 && 5 * HID + 8 <= 512, "staging map");
    __syncthreads();
    {
        const bool actor = wv < 4;
        const uint32_t unit = 16 * (wv % 4) + l % 16;
        const float bias = actor ? s_at[unit] : s_ct[unit];
        v4f acc = {bias, bias, bias, bias};
        if (actor) {
            constexpr uint32_t NK = (D + 3) / 4;
#pragma unroll 8
            for (uint32_t st = 0; st < NK; st++) {
                const uint32_t k = 4 * st + l / 16;
                const float av = k < D ? s_x[l % 16][k] : 0.0f;
                const float bv = k < D ? s_w[k * WS + unit] : -0.0f;
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (uint32_t st = 0; st < COBS / 4; st++) {
                const uint32_t k = 4 * st + l / 16;
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(s_c[l % 16][k], s_cw[k * WS + unit], acc, 0, 0, 0);
            }
        }
#pragma unroll
        for (uint32_t r = 0; r < 4; r++) {
            const float h = tanh_f(acc[r]);
            if (actor) s_ha[4 * (l / 16) + r][unit] = h;
            else s_hc[4 * (l / 16) + r][unit] = h;
        }
    }
    __syncthreads();
    const float* w2 = s_at + HID;          // actor W2 [4][64]
    const float* cw2 = s_ct + HID;         // critic w2 [64]
    if (t < 4 * MB_FWD_ROWS) {  // means (ppo.hpp:73-78)
        const uint32_t r = t / 4, q = t % 4;
        float z = s_at[5 * HID + q];
        for (uint32_t k = 0; k < HID; k++) z = fma_f(w2[q * HID + k], s_ha[r][k], z);
        if (D == MDN_ACTOR_OBS_PRIOR && q < 3) z += s_x[r][D - 3 + q];
        s_mv[r][q] = z;
    } else if (t < 5 * MB_FWD_ROWS) {  // value (ppo.hpp:82-93)
        const uint32_t r = t - 4 * MB_FWD_ROWS;
        float v = s_ct[2 * HID];
        for (uint32_t k = 0; k < HID; k++) v = fma_f(cw2[k], s_hc[r][k], v);
        s_mv[r][4] = v;
    } else if (t < 5 * MB_FWD_ROWS + 8) {
        s_ex[t - 5 * MB_FWD_ROWS] = row_scale_exp(s_at + 5 * HID + 4, t - 5 * MB_FWD_ROWS);
    }
    __syncthreads();
    const float scale = 1.0f / max_f(float(a.b), 1.0f);
    if (t < MB_FWD_ROWS) {
        float* rs = s_rs[t];
        if (t < live_rows) {
            const uint32_t mrow = n0 + t;
            const float mean[4] = {s_mv[t][0], s_mv[t][1], s_mv[t][2], s_mv[t][3]};
            const float value = s_mv[t][4], target = rret;
            float dmean[4];
            const float adv = normalized_advantage(a, radv);
            if (a.norm) a.adv_out[mrow] = adv;
            row_objective(a, s_at + 5 * HID + 4, s_ex, ract, rolp, adv, mean, value, target, scale, dmean, rs);
            rs[12] = a.vcoef * (value - target) * scale;
        } else {
            for (uint32_t c = 0; c < 13; c++) rs[c] = 0.0f;
        }
    }
    __syncthreads();
    {   // hidden deltas (ppo.metal:470-485, 618-631) and the row records
        const uint32_t r = t / 32, k0 = t % 32;
        const bool live = r < live_rows;
        const size_t row = n0 + r;
#pragma unroll
        for (uint32_t u = 0; u < 2; u++) {
            const uint32_t k = k0 + 32 * u;
            float d = 0.0f;
#pragma unroll
            for (uint32_t q = 0; q < 4; q++) d = fma_f(s_rs[r][q], w2[q * HID + k], d);
            const float ha = s_ha[r][k], hc = s_hc[r][k];
            m.rec[MB_HA + row * HID + k] = ha;
            m.rec[MB_DA + row * HID + k] = live ? d * (1.0f - ha * ha) : 0.0f;
            m.rec[MB_HC + row * HID + k] = hc;
            m.rec[MB_DC + row * HID + k] = live ? s_rs[r][12] * cw2[k] * (1.0f - hc * hc) : 0.0f;
        }
        if (k0 < 16) m.rec[MB_RS + row * 16 + k0] = s_rs[r][k0];
    }
}

// Every gradient of the minibatch is a chain over its rows, so all of them
// run as 16x16x4 MFMA chains with the rows as the reduction index:
//   first layers: A = deltas^T (unit rows), B = inputs with a column of ones
//     after the last input, so the tile holding that column also yields the
//     first-layer bias sums (fma(d, 1, s) rounds as s + d);
//   row scalars: A = the records' scalars^T (rows dmean 0-3, dlog_std 4-7,
//     metric terms 8-11, dvalue 12), B = [actor h | 1] or critic h: actor W2
//     (rows 0-3 x h), b2, log_std, metrics and critic b2 (x the ones column),
//     critic w2 (row 12 x critic h).
// Rows past b multiply 0 by -0.0 and leave every chain unchanged.  Tiles:
// actor inputs ceil((D+1)/16) x 4 unit blocks, critic 3 x 4, actor row
// scalars 5 (h blocks 0-3 and the ones column), critic row scalars 4.
template <uint32_t D>
constexpr uint32_t mb_actor_in_tiles() { return (D + 1 + 15) / 16; }
template <uint32_t D>
constexpr uint32_t mb_tiles() { return 4 * mb_actor_in_tiles<D>() + 4 * ((COBS + 1 + 15) / 16) + 5 + 4; }
template <uint32_t D>
__global__ __launch_bounds__(64) void mb_grad_kernel(MbArgs m) {
    using L = AL<D>;
    const RowArgs& a = m.r;
    const uint32_t l = threadIdx.x, rows = a.b;
    constexpr uint32_t AIT = mb_actor_in_tiles<D>(), CIT = (COBS + 1 + 15) / 16;
    constexpr uint32_t A_W1 = 4 * AIT, C_W1 = A_W1 + 4 * CIT, A_RS = C_W1 + 5;
    const float* RS = m.rec + MB_RS;
    uint32_t tile = blockIdx.x;
    // operand sources: A[row][r] = arow(r), B[r][col] = bcol(r)
    uint32_t kind;  // 0 actor W1, 1 critic W1, 2 actor row scalars, 3 critic row scalars
    if (tile < A_W1) kind = 0;
    else if (tile < C_W1) { kind = 1; tile -= A_W1; }
    else if (tile < A_RS) { kind = 2; tile -= C_W1; }
    else { kind = 3; tile -= A_RS; }
    const uint32_t jt = kind < 2 ? tile % 4 : 0, it = kind < 2 ? tile / 4 : tile;
    const uint32_t ar = 16 * jt + l % 16;        // A row (unit, or row-scalar index)
    const uint32_t bc = 16 * it + l % 16;        // B column
    // per-lane operand columns, resolved once so the row loop is branch-free:
    // A[ar][r] = pa[r * sa] when a_ok; B[r][bc] = pb[r * sb] when b_ok, else
    // 1 for the ones column, else -0 (an out-of-range lane reads column 0)
    const float* pa;
    const float* pb;
    uint32_t sa, sb;
    bool a_ok = true, b_ok, b_one;
    if (kind == 0) {
        pa = m.rec + MB_DA + ar; sa = HID;
        b_ok = bc < D; b_one = bc == D; pb = a.obs + (b_ok ? bc : 0); sb = D;
    } else if (kind == 1) {
        pa = m.rec + MB_DC + ar; sa = HID;
        b_ok = bc < COBS; b_one = bc == COBS; pb = a.co + (b_ok ? bc : 0); sb = COBS;
    } else if (kind == 2) {
        a_ok = ar < 13; pa = RS + (a_ok ? ar : 0); sa = 16;
        b_ok = bc < HID; b_one = bc == HID; pb = m.rec + MB_HA + (b_ok ? bc : 0); sb = HID;
    } else {
        a_ok = ar < 13; pa = RS + (a_ok ? ar : 0); sa = 16;
        b_ok = true; b_one = false; pb = m.rec + MB_HC + bc; sb = HID;
    }
    const float b_pad = b_one ? 1.0f : -0.0f;
    float xv[64], yv[64];
#pragma unroll
    for (uint32_t s = 0; s < 64; s++) {
        const uint32_t r = 4 * s + l / 16;
        const size_t rr = r < rows ? r : 0;
        xv[s] = pa[rr * sa];
        yv[s] = pb[rr * sb];
    }
    // every operand load issued before the chain selects and consumes the
    // first (the scheduler would otherwise interleave them in short batches)
    __builtin_amdgcn_sched_barrier(0);
    // rows past b contribute fma(0, -0, acc) = acc
    v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t s = 0; s < 64; s++) {
        const bool rv = 4 * s + l / 16 < rows;
        const float av = rv && a_ok ? xv[s] : 0.0f;
        const float bv = rv ? (b_ok ? yv[s] : b_pad) : -0.0f;
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
    }
    float* g = m.grad;
    // accumulator register r of lane l holds D[4 (l/16) + r][l % 16]
#pragma unroll
    for (uint32_t r = 0; r < 4; r++) {
        const uint32_t row = 16 * jt + 4 * (l / 16) + r;  // A row of this value
        const uint32_t col = bc;
        const float val = 0.0f + (0.0f + acc[r]);
        int32_t out = -1;
        if (kind == 0) {
            if (col < D) out = int32_t(row * D + col);
            else if (col == D) out = int32_t(L::B1 + row);
        } else if (kind == 1) {
            if (col < COBS) out = int32_t(L::COUNT + row * COBS + col);
            else if (col == COBS) out = int32_t(L::COUNT + C_B1 + row);
        } else if (kind == 2) {
            if (col < HID && row < 4) out = int32_t(L::W2 + row * HID + col);
            else if (col == HID && row < 4) out = int32_t(L::B2 + row);
            else if (col == HID && row < 8) out = int32_t(L::LS + row - 4);
            else if (col == HID && row < 12) out = int32_t(L::COUNT + C_COUNT + row - 8);
            else if (col == HID && row == 12) out = int32_t(L::COUNT + C_B2);
        } else {
            if (row == 12) out = int32_t(L::COUNT + C_W2 + col);
        }
        if (out >= 0) g[out] = val;
    }
}

// ---------------------------------------------------------------- clip + Adam
// cpu_reference.hpp:553-567 + log-std clamp (603), over many workgroups: the
// first AW take slices of the actor, the rest slices of the critic.  Each
// recomputes its net's squared gradient norm in the canonical order (256
// strided partials, then the pairwise tree) and updates a slice of ADAM_SLICE
// parameters, clamping the log-stds it owns and, unless keep_w1t is 0 (the
// 256-row path, which transposes once after the update), refreshing the
// transposed first-layer copy; workgroup 0 writes the metric row.
constexpr uint32_t ADAM_SLICE = 256;
template <uint32_t D>
constexpr uint32_t adam_groups() {
    return (AL<D>::COUNT + ADAM_SLICE - 1) / ADAM_SLICE + (C_COUNT + ADAM_SLICE - 1) / ADAM_SLICE;
}
template <uint32_t D>
__global__ __launch_bounds__(256) void adam_slices_kernel(AdamArgs a) {
    using L = AL<D>;
    constexpr uint32_t AW = (L::COUNT + ADAM_SLICE - 1) / ADAM_SLICE;
    constexpr uint32_t NA = (L::COUNT + 255) / 256, NC = (C_COUNT + 255) / 256;
    const bool critic = blockIdx.x >= AW;
    const uint32_t P = critic ? C_COUNT : L::COUNT;
    const uint32_t i0 = (critic ? blockIdx.x - AW : blockIdx.x) * ADAM_SLICE;
    float* params = critic ? a.critic : a.actor;
    float* m = critic ? a.cm : a.am;
    float* v = critic ? a.cv : a.av;
    const float* g = a.grad + (critic ? L::COUNT : 0);
    __shared__ float part[256];
    const uint32_t t = threadIdx.x;
    // this slice's operands, loaded while the norm is formed
    constexpr uint32_t PER = ADAM_SLICE / 256;
    float gv[PER], mv[PER], vv[PER], pv[PER];
#pragma unroll
    for (uint32_t k = 0; k < PER; k++) {
        const uint32_t i = i0 + t + 256 * k;
        if (i < P) { gv[k] = g[i]; mv[k] = m[i]; vv[k] = v[i]; pv[k] = params[i]; }
    }
    // the metric row's sums (workgroup 0) read with the first loads
    float met[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (blockIdx.x == 0 && t == 0) {
        const float* ms = a.grad + L::COUNT + C_COUNT;
#pragma unroll
        for (uint32_t q = 0; q < 4; q++) met[q] = ms[q];
    }
    float s = 0.0f;
    if (critic) {
        float x[NC];
#pragma unroll
        for (uint32_t k = 0; k < NC; k++) x[k] = t + 256 * k < C_COUNT ? g[t + 256 * k] : 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < NC; k++)
            if (t + 256 * k < C_COUNT) s += x[k] * x[k];
    } else {
        float x[NA];
#pragma unroll
        for (uint32_t k = 0; k < NA; k++) x[k] = t + 256 * k < L::COUNT ? g[t + 256 * k] : 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < NA; k++)
            if (t + 256 * k < L::COUNT) s += x[k] * x[k];
    }
    part[t] = s;
    __syncthreads();
    // the pairwise tree: strides 128 and 64 through LDS, 32 to 1 by shuffles
    // within wavefront 0 (lane t adds lane t + stride, as the LDS steps do)
    if (t < 128) part[t] = part[t] + part[t + 128];
    __syncthreads();
    if (t < 64) {
        float v = part[t] + part[t + 64];
#pragma unroll
        for (uint32_t stride = 32; stride > 0; stride >>= 1) v = v + __shfl_down(v, stride, 64);
        if (t == 0) part[0] = v;
    }
    __syncthreads();
    const float norm = sqrt_f(part[0] + 1.0e-20f);
    const float scale = min_f(1.0f, 0.5f / norm);
    if (i0 == 0 && t == 0) a.norm_row[critic ? 1 : 0] = norm;  // ppo_grad_norm's row (main.mm:963-975)
    const float b1 = 0.9f, b2 = 0.999f;
#pragma unroll
    for (uint32_t k = 0; k < PER; k++) {
        const uint32_t i = i0 + t + 256 * k;
        if (i < P) {
            const float gi = gv[k] * scale;
            const float mi = b1 * mv[k] + (1.0f - b1) * gi;
            const float vi = b2 * vv[k] + (1.0f - b2) * gi * gi;
            const float mh = mi / a.c1, vh = vi / a.c2;
            m[i] = mi;
            v[i] = vi;
            float p = pv[k] - a.lr * mh / (sqrt_f(vh) + 1.0e-8f);
            if (!critic && i >= L::LS && i < L::LS + 4) p = clamp_f(p, -2.0f, .5f);
            params[i] = p;
            if (a.keep_w1t) {
                if (!critic && i < HID * D) a.actor_w1t[size_t(i % D) * HID + i / D] = p;
                if (critic && i < HID * COBS) a.critic_w1t[size_t(i % COBS) * HID + i / COBS] = p;
            }
        }
    }
    if (!critic && blockIdx.x == 0 && t == 0) {
        a.metric_row[0] = met[0];
        a.metric_row[1] = met[1];
        a.metric_row[2] = met[2];
        a.metric_row[3] = met[3] / float(a.b);
    }
}

// Transposed first-layer copies from the flat vectors (after uploads/init).
template <uint32_t D>
__global__ __launch_bounds__(256) void transpose_w1_kernel(const float* __restrict__ actor,
                                                           const float* __restrict__ critic, float* __restrict__ aw,
                                                           float* __restrict__ cw) {
    const uint32_t e = blockIdx.x * 256 + threadIdx.x;
    if (e < HID * D) {
        const uint32_t h = e / D, i = e % D;
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

namespace {
bool gae_v4(const float* r, const float* v, const float* nv, const uint8_t* te, const uint8_t* tr, uint32_t n) {
    return n % 4 == 0 && (reinterpret_cast<uintptr_t>(r) | reinterpret_cast<uintptr_t>(v) |
                          reinterpret_cast<uintptr_t>(nv) | reinterpret_cast<uintptr_t>(te) |
                          reinterpret_cast<uintptr_t>(tr)) % 16 == 0;
}
}  // namespace

hipError_t ppo_launch_gae(const float* r, const float* v, const float* nv, const uint8_t* te, const uint8_t* tr,
                          float* adv, float* ret, uint32_t horizon, uint32_t n, float gamma, float lambda,
                          hipStream_t st) {
    if (n == 0 || horizon == 0) return hipSuccess;
    const dim3 grid((n + ppo::GAE_ENVS - 1) / ppo::GAE_ENVS);
    // 16-byte row loads when every row starts 16-byte aligned
    if (gae_v4(r, v, nv, te, tr, n))
        hipLaunchKernelGGL(ppo::gae_kernel<true>, grid, dim3(256), 0, st, r, v, nv, te, tr, adv, ret, horizon, n,
                           gamma, lambda);
    else
        hipLaunchKernelGGL(ppo::gae_kernel<false>, grid, dim3(256), 0, st, r, v, nv, te, tr, adv, ret, horizon, n,
                           gamma, lambda);
    return hipGetLastError();
}

// stats: device float[2] (mean, inv_std); part: device
// double[ppo_normalize_part_words(count)] (the ticket, zero when allocated,
// and both passes' group partials).  `apply` = 0 leaves the rescale to the
// caller's consumers.
hipError_t ppo_launch_normalize_stats(float* a, uint64_t count, double* part, float* stats, float eps, int apply,
                                      hipStream_t st) {
    if (count == 0) return hipSuccess;
    const uint64_t chunks = (count + ppo::CHUNK - 1) / ppo::CHUNK;
    const uint64_t groups = (chunks + ppo::NORM_GROUP - 1) / ppo::NORM_GROUP;
    const uint64_t applies = (count + ppo::NORM_APPLY - 1) / ppo::NORM_APPLY;
    if (groups > 0x7fffffffull || applies > 0x7fffffffull) return hipErrorInvalidValue;
    const bool a16 = reinterpret_cast<uintptr_t>(a) % 16 == 0;
    for (int pass = 0; pass < 2; pass++) {
        if (a16)
            hipLaunchKernelGGL(ppo::norm_pass_kernel<true>, dim3(uint32_t(groups)), dim3(ppo::NORM_THREADS), 0, st, a,
                               count, part, stats, eps, pass);
        else
            hipLaunchKernelGGL(ppo::norm_pass_kernel<false>, dim3(uint32_t(groups)), dim3(ppo::NORM_THREADS), 0, st,
                               a, count, part, stats, eps, pass);
    }
    if (apply)
        hipLaunchKernelGGL(ppo::norm_apply_kernel, dim3(uint32_t(applies)), dim3(256), 0, st, a, count, stats);
    return hipGetLastError();
}

hipError_t ppo_launch_normalize(float* a, uint64_t count, double* part, float* stats, float eps, hipStream_t st) {
    return ppo_launch_normalize_stats(a, count, part, stats, eps, 1, st);
}

// Actor input widths built: 181 (pooled observation) and 184 (with the
// geometry-prior hint).
hipError_t ppo_launch_rows(const ppo::RowArgs* a, hipStream_t st) {
    if (a->b == 0) return hipSuccess;
    if (a->d == MDN_ACTOR_OBS_POOLED)
        hipLaunchKernelGGL(ppo::chunk_kernel<MDN_ACTOR_OBS_POOLED>, dim3((a->b + 255) / 256), dim3(ppo::CT), 0, st, *a);
    else if (a->d == MDN_ACTOR_OBS_PRIOR)
        hipLaunchKernelGGL(ppo::chunk_kernel<MDN_ACTOR_OBS_PRIOR>, dim3((a->b + 255) / 256), dim3(ppo::CT), 0, st, *a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// A minibatch of at most 256 rows: forward/objective/deltas, then the
// finished gradient in grad (no chunk reduction).
hipError_t ppo_launch_minibatch(const ppo::MbArgs* m, hipStream_t st) {
    const uint32_t b = m->r.b;
    if (b == 0 || b > ppo::MB_ROWS) return hipErrorInvalidValue;
    const dim3 fwd((b + ppo::MB_FWD_ROWS - 1) / ppo::MB_FWD_ROWS);
    if (m->r.d == MDN_ACTOR_OBS_POOLED) {
        hipLaunchKernelGGL(ppo::mb_forward_kernel<MDN_ACTOR_OBS_POOLED>, fwd, dim3(512), 0, st, *m);
        hipLaunchKernelGGL(ppo::mb_grad_kernel<MDN_ACTOR_OBS_POOLED>,
                           dim3(ppo::mb_tiles<MDN_ACTOR_OBS_POOLED>()), dim3(64), 0, st, *m);
    } else if (m->r.d == MDN_ACTOR_OBS_PRIOR) {
        hipLaunchKernelGGL(ppo::mb_forward_kernel<MDN_ACTOR_OBS_PRIOR>, fwd, dim3(512), 0, st, *m);
        hipLaunchKernelGGL(ppo::mb_grad_kernel<MDN_ACTOR_OBS_PRIOR>,
                           dim3(ppo::mb_tiles<MDN_ACTOR_OBS_PRIOR>()), dim3(64), 0, st, *m);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t ppo_launch_grads(float* part, float* grad, uint32_t b, uint32_t d, hipStream_t st) {
    const uint32_t chunks = (b + ppo::CHUNK - 1) / ppo::CHUNK;
    const uint32_t groups = (chunks + ppo::GRAD_GROUP - 1) / ppo::GRAD_GROUP;
    const uint32_t ptot = ppo_partial_stride(d);
    hipLaunchKernelGGL(ppo::group_reduce_kernel, dim3((ptot + 255) / 256, groups), dim3(256), 0, st, part, chunks, ptot);
    hipLaunchKernelGGL(ppo::chunk_reduce_kernel, dim3((ptot + 255) / 256), dim3(256), 0, st, part, grad, chunks, ptot);
    return hipGetLastError();
}

hipError_t ppo_launch_adam(const ppo::AdamArgs* a, hipStream_t st) {
    if (a->d == MDN_ACTOR_OBS_POOLED)
        hipLaunchKernelGGL(ppo::adam_slices_kernel<MDN_ACTOR_OBS_POOLED>,
                           dim3(ppo::adam_groups<MDN_ACTOR_OBS_POOLED>()), dim3(256), 0, st, *a);
    else if (a->d == MDN_ACTOR_OBS_PRIOR)
        hipLaunchKernelGGL(ppo::adam_slices_kernel<MDN_ACTOR_OBS_PRIOR>,
                           dim3(ppo::adam_groups<MDN_ACTOR_OBS_PRIOR>()), dim3(256), 0, st, *a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t ppo_launch_transpose(const float* actor, const float* critic, float* aw, float* cw, uint32_t d,
                                hipStream_t st) {
    if (d == MDN_ACTOR_OBS_POOLED)
        hipLaunchKernelGGL(ppo::transpose_w1_kernel<MDN_ACTOR_OBS_POOLED>, dim3((ppo::HID * d + 255) / 256), dim3(256), 0,
                           st, actor, critic, aw, cw);
    else if (d == MDN_ACTOR_OBS_PRIOR)
        hipLaunchKernelGGL(ppo::transpose_w1_kernel<MDN_ACTOR_OBS_PRIOR>, dim3((ppo::HID * d + 255) / 256), dim3(256), 0,
                           st, actor, critic, aw, cw);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t ppo_launch_metric_mean(const float* rows, float* mean, uint32_t updates, hipStream_t st) {
    hipLaunchKernelGGL(ppo::metric_mean_kernel, dim3(1), dim3(64), 0, st, rows, mean, updates);
    return hipGetLastError();
}

uint32_t ppo_partial_stride(uint32_t d) {
    return d == MDN_ACTOR_OBS_PRIOR ? ppo::AL<MDN_ACTOR_OBS_PRIOR>::P_TOTAL : ppo::AL<MDN_ACTOR_OBS_POOLED>::P_TOTAL;
}

}  // extern "C"
