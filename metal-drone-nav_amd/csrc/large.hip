// large.hip — PPO with a wide single hidden layer (the reference's
// FIXED_PPO_HIDDEN_DIM, ppo.hpp:17-45, e.g. 5120 for the 967,688-parameter
// capacity actor) on gfx950 bf16 matrix cores.
//
// Parameters stay fp32 in the reference's flat layout (actor: W1 [H][D] with
// D = 181 or 184 inputs, b1 [H], W2 [4][H], b2 [4], log_std [4]; critic:
// W1 [H][32], b1 [H], w2 [H], b2) with fp32 Adam moments.  The 184-input
// actor adds its last three inputs (the geometry-prior hint) to the first
// three means (ppo.hpp:77) in fp32.  The first-layer matrices are also
// kept as bf16 copies [H][K] (inputs zero-padded to K = 192 / 32, scaled by
// 2 log2(e) for the activation's base-2 form) for the GEMMs, refreshed by
// every Adam step.  GEMMs accumulate in fp32
// (v_mfma_f32_32x32x16_bf16); activations use a fast exp-based tanh; the
// hidden activations are never written to HBM: the backward pass recomputes
// each tile.  Results match the fp32 CPU oracle within bf16 tolerance, not
// bit for bit.
//
// MFMA operand layout (32x32x16): A lane a holds A[a%32][8(a/32) .. +7],
// B lane b holds B[8(b/32) .. +7][b%32], accumulator r of lane l holds
// D[8(r/4) + 4(l/32) + r%4][l%32].
#include <hip/hip_runtime.h>

#include <algorithm>

#include "mdnav_math.h"
#include "mdnav_types.h"
#include "kernel_args.h"

namespace lp {
using namespace mdn;

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr uint32_t COBS = MDN_CRITIC_OBS;
constexpr uint32_t KA = 192, KC = 32;  // first-layer inputs padded to whole 32-wide tiles
constexpr uint32_t RB = 64;            // rows per block (two 32-row tiles); 2 workgroups fit a CU
constexpr uint32_t RT = RB / 32;       // 32-row tiles per block
constexpr uint32_t UT = 128;           // hidden units per tile: four wavefronts x 32
constexpr float LOG_TWO_PI = 1.8378770664093453f;

__device__ __forceinline__ v16f mfma(bf8 a, bf8 b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ uint32_t acc_row(uint32_t l, uint32_t r) { return 8 * (r / 4) + 4 * (l / 32) + (r % 4); }
// tanh(x) = 1 - 2 / (2^y + 1) with y = 2 log2(e) x, on the hardware base-2
// exponential and reciprocal (v_exp_f32, v_rcp_f32; about 1 ulp each).  The
// first layers' bf16 copies and biases are held multiplied by TANH_SCALE =
// 2 log2(e) (pack_kernel, adam_kernel, the kernels' bias loads), so a hidden
// unit's accumulator already holds y and the activation costs no multiply.
constexpr float TANH_SCALE = 2.8853900817779268f;

__device__ __forceinline__ float tanh_scaled(float y) {
    const float e = __builtin_amdgcn_exp2f(y);
    return fma_f(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
}

// bf16 copies of the B rows of X[B][D] prepared once per minibatch: Xb
// [BP][K] row-major and XbT [K][BP] transposed (BP = B rounded up to RB; inputs
// past D and rows past B are zero).  Every hidden tile reads these instead of
// converting the rows itself.  A workgroup takes RB rows: each thread reads 8
// consecutive inputs of a row (consecutive threads, consecutive inputs) and
// writes them as one 16-byte bf16 chunk of Xb; the transposed copy goes
// through an LDS tile so that each row of XbT is written in 16-byte chunks
// of 8 rows.
template <uint32_t D, uint32_t K>
__global__ __launch_bounds__(256) void prep_kernel(const float* __restrict__ X, uint32_t B, uint32_t BP,
                                                   __bf16* __restrict__ Xb, __bf16* __restrict__ XbT) {
    constexpr uint32_t CH = K / 8, TS = K + 8;  // chunks per row; tile row stride (bf16)
    __shared__ __attribute__((aligned(16))) __bf16 tile[RB * TS];
    const uint32_t t = threadIdx.x, r0 = blockIdx.x * RB;
    for (uint32_t e = t; e < RB * CH; e += 256) {
        const uint32_t rr = e / CH, c = e % CH, row = r0 + rr;
        bf8 v;
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) {
            const uint32_t k = 8 * c + j;
            const float x = X[size_t(row < B ? row : 0) * D + (k < D ? k : 0)];
            v[j] = (__bf16)((row < B && k < D) ? x : 0.0f);
        }
        *reinterpret_cast<bf8*>(Xb + size_t(row) * K + 8 * c) = v;
        // the transposed copy carries a one in the first padding input: the
        // backward's bias column (rows past B have zero deltas)
        if (D < K && c == D / 8) v[D % 8] = (__bf16)1.0f;
        if (XbT) *reinterpret_cast<bf8*>(tile + rr * TS + 8 * c) = v;
    }
    if (!XbT) return;
    __syncthreads();
    for (uint32_t e = t; e < K * (RB / 8); e += 256) {
        const uint32_t k = e / (RB / 8), r8 = e % (RB / 8);
        bf8 v;
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) v[j] = tile[(8 * r8 + j) * TS + k];
        *reinterpret_cast<bf8*>(XbT + size_t(k) * BP + r0 + 8 * r8) = v;
    }
}

// ---------------------------------------------------------------- weights
// The bf16 copy of a first-layer matrix W [H][D] (inputs zero-padded to K) is
// stored in fragment order: for each group of 32 units and each 16-wide k
// step, the 64 lanes' 8-element matrix-core fragments (lane l: unit l % 32,
// inputs 8(l / 32) ..) lie contiguously, so a wavefront's fragment load reads
// 1 KB in one piece.  wsw(u, k) is the position of W[u][k]; frag(ub, ks, l)
// the first element of lane l's fragment for units ub .. ub+31 (ub % 32 == 0).
__device__ __forceinline__ size_t frag(uint32_t ub, uint32_t ks, uint32_t l, uint32_t K) {
    return ((size_t(ub / 32) * (K / 16) + ks) * 64 + l) * 8;
}
__device__ __forceinline__ size_t wsw(uint32_t u, uint32_t k, uint32_t K) {
    return frag(u - u % 32, k / 16, u % 32 + 32 * ((k % 16) / 8), K) + k % 8;
}
__global__ __launch_bounds__(256) void pack_kernel(const float* __restrict__ W, uint32_t H, uint32_t D, uint32_t K,
                                                   __bf16* __restrict__ out) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= uint64_t(H) * K) return;
    const uint32_t u = uint32_t(i / K), k = uint32_t(i % K);
    out[wsw(u, k, K)] = (__bf16)(k < D ? W[uint64_t(u) * D + k] * TANH_SCALE : 0.0f);
}

// ---------------------------------------------------------------- forward
// out[row][q] = b2[q] + sum_u W2[q][u] tanh(b1[u] + sum_k W1[u][k] X[row][k])
// for q < NQ (actor means: NQ = 4 over W2 [4][H]; critic value: NQ = 1).
//
// Both layers run on the matrix cores.  The first is computed transposed,
// hT[unit][row] = W1 X^T (weights as the A operand, rows as B), so that a
// wavefront's accumulator (lane -> row l%32, register r -> unit
// 8(r/4) + 4(l/32) + r%4) is, rounded to bf16, already the B operand of the
// second product zT[q][row] += W2[q][units] hT[units][row]: k slot
// 8(l/32) + e of product m is register 8m + e, and the A operand holds W2
// columns in that same unit order (rows q >= NQ zero).  A workgroup of eight
// wavefronts owns FWD_RB = 2 RB rows: wavefronts g and g + 4 take the same
// 32 units of every 128-unit tile for their own RB rows, whose fragments stay
// in registers, and the tile's W1 fragments (4 x K/16 x 1 KB, contiguous in
// Wb), biases and W2 columns are staged once in LDS for both (double-
// buffered, one barrier per tile).  The four wavefronts of a row half meet
// in LDS at the end, their partial sums added in unit-group order.
// blockIdx.y splits the hidden units into gridDim.y slices when there are
// too few rows to fill the GPU: each slice writes part [S][BP][NQ] and
// part_sum_kernel adds them in slice order.
constexpr uint32_t FWD_RB = 2 * RB;
template <uint32_t K, uint32_t NQ>
__global__ __launch_bounds__(512, 1) void forward_kernel(const __bf16* __restrict__ Xb, uint32_t BP,
                                                          const __bf16* __restrict__ Wb,
                                                          const float* __restrict__ b1, const float* __restrict__ W2,
                                                          const float* __restrict__ b2, uint32_t H, uint32_t B,
                                                          float* __restrict__ out, float* __restrict__ part,
                                                          const float* __restrict__ prior, uint32_t prior_stride) {
    constexpr uint32_t KS = K / 16, NTH = 512, RBW = FWD_RB;
    __shared__ float zs[8][RB * NQ];
    const uint32_t t = threadIdx.x, wv = t / 64, l = t % 64, half = l / 32, lr = l % 32;
    const uint32_t grp = wv % 4, rh = wv / 4;
    const uint32_t r0 = blockIdx.x * RBW + rh * RB;
    const uint32_t span = H / gridDim.y, h0 = blockIdx.y * span, h1 = h0 + span;
    bf8 xf[RT][KS];  // B operand: X[row r0 + 32 rt + l%32][16 ks + 8(l/32) ..]
#pragma unroll
    for (uint32_t rt = 0; rt < RT; rt++) {
        const uint32_t row = r0 + 32 * rt + lr;
#pragma unroll
        for (uint32_t ks = 0; ks < KS; ks++) {
            const bf8 v = *reinterpret_cast<const bf8*>(Xb + size_t(row < BP ? row : 0) * K + 16 * ks + 8 * half);
            xf[rt][ks] = row < BP ? v : bf8{};
        }
    }
    v16f z[RT];
#pragma unroll
    for (uint32_t rt = 0; rt < RT; rt++)
#pragma unroll
        for (uint32_t r = 0; r < 16; r++) z[rt][r] = 0.0f;
    const uint32_t ntile = span / UT;
    {
        constexpr uint32_t NF = 4 * KS * 64, PER = (NF + NTH - 1) / NTH;  // 16-byte fragments per tile
        // per tile: the W1 fragments, b1 of the tile's units, and the second
        // layer's A operand as bf16 fragments: thread t = (group g, product m,
        // lane l) holds W2[q = l%32][unit 32 g + 16 m + 4(l/32) + {0..3, 8..11}]
        // (zero for q >= NQ)
        __shared__ bf8 ws[2][NF];
        __shared__ __attribute__((aligned(16))) float wb1[2][UT];
        __shared__ bf8 wfa[2][4 * 2 * 64];
        static_assert(NTH == 4 * 2 * 64 && UT <= NTH, "one second-layer fragment and one bias per thread");
        static_assert(NF % NTH == 0, "whole fragment rounds");
        auto tile_base = [&](uint32_t i) { return h0 + UT * i; };
        float sb1 = 0.0f;
        float4 sw2[2];
        const uint32_t fg = t / 128, fm = (t / 64) % 2, fl = t % 64, fq = fl % 32, fh = fl / 32;
        bf8 stg[PER];
        auto fetch = [&](uint32_t i) {
            const uint32_t base = tile_base(i);
            const bf8* src = reinterpret_cast<const bf8*>(Wb + frag(base, 0, 0, K));
#pragma unroll
            for (uint32_t j = 0; j < PER; j++) stg[j] = src[t + NTH * j];
            if (t < UT) sb1 = b1[base + t];
            const float* w2 = W2 + size_t(min(fq, NQ - 1)) * H + base + 32 * fg + 16 * fm + 4 * fh;
            sw2[0] = *reinterpret_cast<const float4*>(w2);
            sw2[1] = *reinterpret_cast<const float4*>(w2 + 8);
        };
        auto stage = [&](uint32_t buf) {
#pragma unroll
            for (uint32_t j = 0; j < PER; j++) ws[buf][t + NTH * j] = stg[j];
            if (t < UT) wb1[buf][t] = sb1 * TANH_SCALE;
            const bool on = fq < NQ;
            bf8 a;
            a[0] = (__bf16)(on ? sw2[0].x : 0.0f); a[1] = (__bf16)(on ? sw2[0].y : 0.0f);
            a[2] = (__bf16)(on ? sw2[0].z : 0.0f); a[3] = (__bf16)(on ? sw2[0].w : 0.0f);
            a[4] = (__bf16)(on ? sw2[1].x : 0.0f); a[5] = (__bf16)(on ? sw2[1].y : 0.0f);
            a[6] = (__bf16)(on ? sw2[1].z : 0.0f); a[7] = (__bf16)(on ? sw2[1].w : 0.0f);
            wfa[buf][t] = a;
        };
        // activations of one row tile and their second-layer products
        auto activate = [&](const v16f& a, const bf8 (&w)[2], v16f& zz) {
#pragma unroll
            for (uint32_t m = 0; m < 2; m++) {
                bf8 hb;
#pragma unroll
                for (uint32_t e = 0; e < 8; e++) hb[e] = (__bf16)tanh_scaled(a[8 * m + e]);
                zz = mfma(w[m], hb, zz);
            }
        };
        fetch(0);
        stage(0);
        for (uint32_t i = 0; i < ntile; i++) {
            __syncthreads();  // tile i staged in buffer i & 1; the other is no longer read
            if (i + 1 < ntile) fetch(i + 1);
            const float* tv = wb1[i & 1];
            const uint32_t uo = 32 * grp;  // the wavefront's units within the tile
            v16f bias;
#pragma unroll
            for (uint32_t g = 0; g < 4; g++) {
                const float4 b4 = *reinterpret_cast<const float4*>(tv + uo + 8 * g + 4 * half);
                bias[4 * g] = b4.x; bias[4 * g + 1] = b4.y; bias[4 * g + 2] = b4.z; bias[4 * g + 3] = b4.w;
            }
            // second-layer A operand: W2[q = l%32][unit of k slot 8(l/32) + e] (zero for q >= NQ)
            const bf8 wa[2] = {wfa[i & 1][(grp * 2 + 0) * 64 + l], wfa[i & 1][(grp * 2 + 1) * 64 + l]};
            const bf8* wt = ws[i & 1] + grp * KS * 64 + l;
            v16f acc[RT];
#pragma unroll
            for (uint32_t rt = 0; rt < RT; rt++) acc[rt] = bias;
            bf8 wv[KS];  // the tile's W1 fragments, all requested before the first product
#pragma unroll
            for (uint32_t ks = 0; ks < KS; ks++) wv[ks] = wt[ks * 64];
#pragma unroll
            for (uint32_t ks = 0; ks < KS; ks++)
#pragma unroll
                for (uint32_t rt = 0; rt < RT; rt++) acc[rt] = mfma(wv[ks], xf[rt][ks], acc[rt]);
#pragma unroll
            for (uint32_t rt = 0; rt < RT; rt++) activate(acc[rt], wa, z[rt]);
            if (i + 1 < ntile) stage((i + 1) & 1);
        }
    }
    // zT[q][row]: lanes 0-31, registers q
    if (half == 0)
#pragma unroll
        for (uint32_t rt = 0; rt < RT; rt++)
#pragma unroll
            for (uint32_t q = 0; q < NQ; q++) zs[wv][(32 * rt + lr) * NQ + q] = z[rt][q];
    __syncthreads();
    for (uint32_t i = t; i < RBW * NQ; i += NTH) {
        const uint32_t hr = i / (RB * NQ), li = i % (RB * NQ);  // row half, entry within it
        const uint32_t row = blockIdx.x * RBW + i / NQ, q = i % NQ;
        const float v = ((zs[4 * hr][li] + zs[4 * hr + 1][li]) + zs[4 * hr + 2][li]) + zs[4 * hr + 3][li];
        if (row >= B) continue;
        if (gridDim.y == 1)
            out[size_t(row) * NQ + q] = prior && q < 3 ? (b2[q] + v) + prior[size_t(row) * prior_stride + q] : b2[q] + v;
        else
            part[(size_t(blockIdx.y) * BP + row) * NQ + q] = v;
    }
}

// out[row][q] = b2[q] + the hidden slices' partial sums, in slice order
// (+ prior[row][q] for q < 3 when given: the geometry-prior hint).
__global__ __launch_bounds__(256) void part_sum_kernel(const float* __restrict__ part, uint32_t S, uint32_t BP,
                                                       uint32_t B, uint32_t NQ, const float* __restrict__ b2,
                                                       float* __restrict__ out, const float* __restrict__ prior,
                                                       uint32_t prior_stride) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= B * NQ) return;
    // the slices in order, 8 loads in flight at a time; slices past the
    // last are loaded as 0 and not added (the first slice may be -0)
    float v = part[i];
    for (uint32_t s0 = 1; s0 < S; s0 += 8) {
        float x[8];
#pragma unroll
        for (uint32_t k = 0; k < 8; k++) x[k] = s0 + k < S ? part[size_t(s0 + k) * BP * NQ + i] : 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < 8; k++)
            if (s0 + k < S) v += x[k];
    }
    const uint32_t row = i / NQ, q = i % NQ;
    out[i] = prior && q < 3 ? (b2[q] + v) + prior[size_t(row) * prior_stride + q] : b2[q] + v;
}

// ---------------------------------------------------------------- loss
// sample_loss_and_grad (ppo.hpp:144-181) per minibatch row from the means and
// values of the forward kernels.  Writes dmean[4], dlog_std[4], dvalue and the
// four loss terms.
// Per-row clipped-surrogate, value and entropy terms (ppo.hpp:144-181) of
// row n, written to the row records and to column t of cs.
__device__ __forceinline__ void row_loss(const float* __restrict__ mean, const float* __restrict__ value,
                                         const float* __restrict__ actions, const float* __restrict__ old_logp,
                                         const float* __restrict__ adv, const float* __restrict__ ret,
                                         const float* __restrict__ log_std, uint32_t B, float clip, float vcoef,
                                         float ecoef, uint32_t n, float* __restrict__ dm, float* __restrict__ dls,
                                         float* __restrict__ dv, float* __restrict__ loss, float (*cs)[RB + 1],
                                         uint32_t t) {
    const float* act = actions + size_t(n) * 4;
    const float* mu = mean + size_t(n) * 4;
    const float scale = 1.0f / max_f(float(B), 1.0f);
    float logp = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) {
        const float d = (act[q] - mu[q]) * exp_f(-log_std[q]);
        logp += -0.5f * (d * d + 2.0f * log_std[q] + LOG_TWO_PI);
    }
    const float raw = logp - old_logp[n];
    const float ratio = exp_f(clamp_f(raw, -20.0f, 20.0f));
    const float a = adv[n], target = ret[n], v = value[n];
    const float clipped = clamp_f(ratio, 1.0f - clip, 1.0f + clip);
    const float chosen = min_f(ratio * a, clipped * a);
    const bool in_range = raw >= -20.0f && raw <= 20.0f;
    const bool active = in_range && (a >= 0.0f ? ratio <= 1.0f + clip : ratio >= 1.0f - clip);
    float entropy = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) {
        const float inv_var = exp_f(-2.0f * log_std[q]);
        const float diff = act[q] - mu[q];
        float g = 0.0f, gl = 0.0f;
        if (active) {
            const float dlogp = -ratio * a * scale;
            g = dlogp * diff * inv_var;
            gl = dlogp * (diff * diff * inv_var - 1.0f);
        }
        gl -= ecoef * scale;
        entropy += -ecoef * (log_std[q] + 0.5f * (1.0f + LOG_TWO_PI)) * scale;
        dm[size_t(n) * 4 + q] = g;
        dls[size_t(n) * 4 + q] = gl;
        cs[q][t] = g;
        cs[4 + q][t] = gl;
    }
    const float dvn = vcoef * (v - target) * scale;
    const float l0 = -chosen * scale, l1 = 0.5f * vcoef * (v - target) * (v - target) * scale;
    dv[n] = dvn;
    float* lo = loss + size_t(n) * 4;
    lo[0] = l0;
    lo[1] = l1;
    lo[2] = entropy;
    lo[3] = ratio;
    cs[8][t] = dvn;
    cs[9][t] = l0;
    cs[10][t] = l1;
    cs[11][t] = entropy;
    cs[12][t] = ratio;
}

__global__ __launch_bounds__(RB) void loss_kernel(const float* __restrict__ mean, const float* __restrict__ value,
                                                  const float* __restrict__ actions, const float* __restrict__ old_logp,
                                                  const float* __restrict__ adv, const float* __restrict__ ret,
                                                  const float* __restrict__ log_std, uint32_t B, float clip,
                                                  float vcoef, float ecoef, float* __restrict__ dm,
                                                  float* __restrict__ dls, float* __restrict__ dv,
                                                  float* __restrict__ loss, float* __restrict__ col_part) {
    // block b takes rows b*RB ..; its 13 per-row terms (dm[4] -> b2,
    // dls[4] -> log_std, dv -> critic b2, loss[4] -> metrics) are then summed
    // over those rows in order into col_part[b][13] (column_finish_kernel
    // adds the blocks in order)
    __shared__ float cs[13][RB + 1];
    const uint32_t t = threadIdx.x, n = blockIdx.x * RB + t;
    if (n >= B) {
        for (uint32_t c = 0; c < 13; c++) cs[c][t] = 0.0f;
    } else {
        row_loss(mean, value, actions, old_logp, adv, ret, log_std, B, clip, vcoef, ecoef, n, dm, dls, dv, loss, cs, t);
    }
    __syncthreads();
    if (t < 13) {
        float a = 0.0f;
        for (uint32_t rr = 0; rr < RB; rr++) a += cs[t][rr];
        col_part[size_t(blockIdx.x) * 13 + t] = a;
    }
}

// gaussian_log_prob (ppo.hpp:95-103) of the stored actions under the means.
__global__ __launch_bounds__(256) void logp_kernel(const float* __restrict__ mean, const float* __restrict__ actions,
                                                   const float* __restrict__ log_std, uint32_t B,
                                                   float* __restrict__ logp) {
    const uint32_t n = blockIdx.x * 256 + threadIdx.x;
    if (n >= B) return;
    float lp = 0.0f;
#pragma unroll
    for (uint32_t q = 0; q < 4; q++) {
        const float d = (actions[size_t(n) * 4 + q] - mean[size_t(n) * 4 + q]) * exp_f(-log_std[q]);
        lp += -0.5f * (d * d + 2.0f * log_std[q] + LOG_TWO_PI);
    }
    logp[n] = lp;
}

// ---------------------------------------------------------------- backward
// Partial gradients of one (hidden tile, row chunk).  The workgroup's 128
// units are four groups of 32; with WV = 4 wavefronts wavefront g owns group
// g and both 32-row tiles of each RB-row block, with WV = 8 wavefronts g and
// g + 4 share group g (each holding its W1 rows) and take one 32-row tile
// each, so that two wavefronts per SIMD overlap one's matrix-core work with
// the other's activations.  Everything runs in one accumulator layout
// (lane -> unit l%32, register r -> row 32 rt + 8(r/4) + 4(l/32) + r%4):
//   h      = tanh(X W1^T + b1)            bf16 MFMA, rows as A (from LDS)
//   g      = dm W2^T                      fp32 MFMA 32x32x2 (the fma chain over q)
//   delta  = g (1 - h^2)                  VALU, per lane
//   dW2^T += dm^T h                       bf16 MFMA, h from registers as B
//   dW1   += delta^T X                    bf16 MFMA, delta from registers as A,
//                                         X^T rows from LDS as B
//   db1   += delta                        the dW1 product's column of ones
//                                         (input D) when the inputs are
//                                         padded (D < K), else VALU per lane
// The rows are the reduction dimension of the last two products; their k
// slots follow the accumulator's row order (slot 8(l/32) + e of product m is
// register 8m + e), and the LDS operands are read in that order.  Rows of the
// next block are fetched into registers during the current block (two LDS
// buffers, one barrier per block).  Rows past the chunk carry dm = 0 and
// contribute nothing.  With WV = 8 the second wavefront of each group adds
// its sums to the first's through LDS at the end.  Output: partial slot c =
// blockIdx.y of dW1p [c][H][D], db1p [c][H], dW2p [c][NQ][H].
template <uint32_t K, uint32_t NQ, uint32_t NTH>
struct BwdStage {
    static constexpr uint32_t XS = K + 8, TS = RB + 8;   // row strides (bf16) of xs and xt (16-byte multiples)
    static constexpr uint32_t XCH = RB * K / 8;          // 16-byte chunks of a block's rows
    static constexpr uint32_t TCH = K * RB / 8;
    static constexpr uint32_t NX = (XCH + NTH - 1) / NTH, NT = (TCH + NTH - 1) / NTH;
    bf8 x[NX], xt[NT];
    float d;
};

template <uint32_t K, uint32_t NQ, uint32_t NTH>
__device__ __forceinline__ void bwd_fetch(BwdStage<K, NQ, NTH>& f, const __bf16* __restrict__ Xb,
                                          const __bf16* __restrict__ XbT, uint32_t BP, uint32_t r0, uint32_t rend,
                                          const float* __restrict__ dm, uint32_t t) {
    using S = BwdStage<K, NQ, NTH>;
    constexpr uint32_t CH = K / 8;
#pragma unroll
    for (uint32_t i = 0; i < S::NX; i++) {
        const uint32_t e = min(t + NTH * i, S::XCH - 1);
        f.x[i] = *reinterpret_cast<const bf8*>(Xb + size_t(r0 + e / CH) * K + 8 * (e % CH));
    }
#pragma unroll
    for (uint32_t i = 0; i < S::NT; i++) {
        const uint32_t e = min(t + NTH * i, S::TCH - 1);
        f.xt[i] = *reinterpret_cast<const bf8*>(XbT + size_t(e / (RB / 8)) * BP + r0 + 8 * (e % (RB / 8)));
    }
    const uint32_t row = r0 + t / NQ;  // t < RB * NQ (256 threads cover RB * 4)
    f.d = (t < RB * NQ && row < rend) ? dm[size_t(min(row, rend - 1)) * NQ + t % NQ] : 0.0f;
}

// Position of a block row in the transposed LDS copies (xt, the bf16 dm):
// bits 2 and 3 of the row swapped, so that the rows of one product's k slots
// (16 m + 4 (l/32) + {0..3, 8..11}) lie in 8 consecutive positions and a
// lane reads its B (or A) operand in one 16-byte load.
__device__ __forceinline__ uint32_t kpos(uint32_t row) {
    return (row & ~15u) | ((row & 4u) << 1) | ((row & 8u) >> 1) | (row & 3u);
}

template <uint32_t K, uint32_t NQ, uint32_t NTH>
__device__ __forceinline__ void bwd_store(const BwdStage<K, NQ, NTH>& f, __bf16* xs, __bf16* xt, float* dmt,
                                          __bf16* dmb, uint32_t t) {
    using S = BwdStage<K, NQ, NTH>;
    constexpr uint32_t CH = K / 8;
    typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (uint32_t i = 0; i < S::NX; i++) {
        const uint32_t e = t + NTH * i;
        if (e < S::XCH) *reinterpret_cast<bf8*>(xs + (e / CH) * S::XS + 8 * (e % CH)) = f.x[i];
    }
#pragma unroll
    for (uint32_t i = 0; i < S::NT; i++) {
        const uint32_t e = t + NTH * i;
        if (e < S::TCH) {
            __bf16* dst = xt + (e / (RB / 8)) * S::TS;
            const uint32_t r8 = 8 * (e % (RB / 8));
            const bf8 v = f.xt[i];
            *reinterpret_cast<bf4*>(dst + kpos(r8)) = bf4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<bf4*>(dst + kpos(r8 + 4)) = bf4{v[4], v[5], v[6], v[7]};
        }
    }
    if (t < RB * NQ) {  // transposed: dmt [q][row] (fp32), dmb [q][kpos(row)] (bf16)
        dmt[(t % NQ) * RB + t / NQ] = f.d;
        dmb[(t % NQ) * RB + kpos(t / NQ)] = (__bf16)f.d;
    }
}

template <uint32_t D, uint32_t K, uint32_t NQ, uint32_t WV>
__global__ __launch_bounds__(64 * WV, WV == 4 && NQ == 1 ? 2 : 1) void backward_kernel(
    const __bf16* __restrict__ Xb, const __bf16* __restrict__ XbT, uint32_t BP, const __bf16* __restrict__ Wb,
    const float* __restrict__ b1, const float* __restrict__ W2, const float* __restrict__ dm, uint32_t H, uint32_t B,
    uint32_t RC, float* __restrict__ dW1p, float* __restrict__ db1p, float* __restrict__ dW2p) {
    static_assert(WV == 4 || WV == 8, "one or two wavefronts per unit group");
    constexpr uint32_t NTH = 64 * WV, RTW = RT * 4 / WV;  // threads; 32-row tiles per wavefront and block
    using S = BwdStage<K, NQ, NTH>;
    constexpr uint32_t XS = S::XS, TS = S::TS, JT = K / 32;
    __shared__ __bf16 xs[2][RB * XS];   // [row][k]
    __shared__ __bf16 xt[2][K * TS];    // [k][row]
    __shared__ __attribute__((aligned(16))) float dmt[2][NQ * RB];  // [q][row]
    __shared__ __attribute__((aligned(16))) __bf16 dmb[2][(NQ + 1) * RB];  // [q][kpos(row)]; row NQ zero
    const uint32_t t = threadIdx.x, wv = t / 64, l = t % 64, half = l / 32, lr = l % 32;
    const uint32_t grp = wv % 4, rh = wv / 4;  // unit group; row tiles rh * RTW ..
    const uint32_t u0 = blockIdx.x * UT, c = blockIdx.y;
    const uint32_t unit = u0 + 32 * grp + lr;
    const uint32_t rbeg = c * RC, rend = min(B, rbeg + RC);
    const float bias = b1[unit] * TANH_SCALE;
    // B operand of h: W1[unit][16 ks + 8(l/32) ..].  WV = 4: in registers;
    // WV = 8: the workgroup's 128 units (48 KB in fragment order, contiguous
    // in Wb) staged once in LDS and read per step, which leaves the registers
    // to the two wavefronts per SIMD.
    constexpr uint32_t WF = WV == 8 ? 4 * (K / 16) * 64 : 1;  // 16-byte fragments staged
    __shared__ bf8 ws[WF];
    bf8 bw[WV == 8 ? 1 : K / 16];
    if constexpr (WV == 8) {
        const bf8* src = reinterpret_cast<const bf8*>(Wb + frag(u0, 0, 0, K));
#pragma unroll 4
        for (uint32_t i = t; i < WF; i += NTH) ws[i] = src[i];
    } else {
#pragma unroll
        for (uint32_t ks = 0; ks < K / 16; ks++)
            bw[ks] = *reinterpret_cast<const bf8*>(Wb + frag(u0 + 32 * grp, ks, l, K));
    }
    // B operand of g: W2[q = 2 p + l/32][unit] (zero for q >= NQ)
    constexpr uint32_t NP = (NQ + 1) / 2;
    float w2f[NP];
#pragma unroll
    for (uint32_t p = 0; p < NP; p++) {
        const uint32_t q = 2 * p + half;
        w2f[p] = q < NQ ? W2[size_t(min(q, NQ - 1)) * H + unit] : 0.0f;
    }
    v16f gacc[JT], w2acc;
#pragma unroll
    for (uint32_t jt = 0; jt < JT; jt++)
#pragma unroll
        for (uint32_t r = 0; r < 16; r++) gacc[jt][r] = 0.0f;
#pragma unroll
    for (uint32_t r = 0; r < 16; r++) w2acc[r] = 0.0f;
    // db1: with padding inputs (D < K) the transposed rows carry ones in
    // input column D (prep_kernel), so the dW1 tile holding that column also
    // yields the bias sums; otherwise the deltas are summed per lane
    constexpr bool ONES = D < K;
    float db1a = 0.0f;
    for (uint32_t i = t; i < 2 * RB; i += NTH) dmb[i / RB][NQ * RB + i % RB] = (__bf16)0.0f;

    S st;
    if (rbeg < rend) {
        bwd_fetch(st, Xb, XbT, BP, rbeg, rend, dm, t);
        bwd_store(st, xs[0], xt[0], dmt[0], dmb[0], t);
    }
    uint32_t buf = 0;
    for (uint32_t r0 = rbeg; r0 < rend; r0 += RB, buf ^= 1) {
        __syncthreads();  // block r0 staged in buf; buf ^ 1 no longer read
        const bool more = r0 + RB < rend;
        const __bf16* X = xs[buf];
        const __bf16* XT = xt[buf];
        const float* DM = dmt[buf];
        const __bf16* DMB = dmb[buf];
#pragma unroll
        for (uint32_t ri = 0; ri < RTW; ri++) {
            const uint32_t rt = rh * RTW + ri;
            v16f h;
#pragma unroll
            for (uint32_t r = 0; r < 16; r++) h[r] = bias;
            bf8 av[K / 16], bv[K / 16];  // requested ahead of the products (the compiler keeps several in flight)
#pragma unroll
            for (uint32_t ks = 0; ks < K / 16; ks++) {
                av[ks] = *reinterpret_cast<const bf8*>(X + (32 * rt + lr) * XS + 16 * ks + 8 * half);
                bv[ks] = WV == 8 ? ws[(grp * (K / 16) + ks) * 64 + l] : bw[WV == 8 ? 0 : ks];
            }
#pragma unroll
            for (uint32_t ks = 0; ks < K / 16; ks++) h = mfma(av[ks], bv[ks], h);
            // the next block's rows, requested once the products no longer
            // need the registers
            if (ri == 0 && more) bwd_fetch(st, Xb, XbT, BP, r0 + RB, rend, dm, t);
            v16f g;
#pragma unroll
            for (uint32_t r = 0; r < 16; r++) g[r] = 0.0f;
#pragma unroll
            for (uint32_t p = 0; p < NP; p++) {
                const uint32_t q = 2 * p + half;
                const float a = q < NQ ? DM[min(q, NQ - 1) * RB + 32 * rt + lr] : 0.0f;
                g = __builtin_amdgcn_mfma_f32_32x32x2f32(a, w2f[p], g, 0, 0, 0);
            }
#pragma unroll
            for (uint32_t m = 0; m < 2; m++) {
                bf8 hb, db;
#pragma unroll
                for (uint32_t e = 0; e < 8; e++) {
                    const float hv = tanh_scaled(h[8 * m + e]);
                    const float d = g[8 * m + e] * fma_f(-hv, hv, 1.0f);
                    if constexpr (!ONES) db1a += d;
                    hb[e] = (__bf16)hv;
                    db[e] = (__bf16)d;
                }
                // rows of this product's k slots: 32 rt + 16 m + 4(l/32) + {0..3, 8..11},
                // consecutive at kpos 32 rt + 16 m + 8(l/32) of the transposed copies
                const uint32_t kp = 32 * rt + 16 * m + 8 * half;
                {   // dW2^T: A = dm^T [q][rows] (q = l%32, zero past NQ)
                    const bf8 am = *reinterpret_cast<const bf8*>(DMB + min(lr, NQ) * RB + kp);
                    w2acc = mfma(am, hb, w2acc);
                }
#pragma unroll
                for (uint32_t jt = 0; jt < JT; jt++) {  // dW1: B = X [rows][k = 32 jt + l%32]
                    const bf8 xb = *reinterpret_cast<const bf8*>(XT + (32 * jt + lr) * TS + kp);
                    gacc[jt] = mfma(db, xb, gacc[jt]);
                }
            }
        }
        if (more) bwd_store(st, xs[buf ^ 1], xt[buf ^ 1], dmt[buf ^ 1], dmb[buf ^ 1], t);
    }
    // lanes l and l + 32 hold the same unit
    if constexpr (!ONES) db1a += __shfl_xor(db1a, 32, 64);
    if constexpr (WV == 8) {
        // the second wavefront of each group hands its sums to the first
        // through the (now idle) row staging buffer, three 16-register
        // pieces (dW1 tiles, then dW2^T) per round: hand [piece][group][16][64],
        // then db1 [group][64] in the first round
        constexpr uint32_t NPC = JT + 1, PIECE = 4 * 16 * 64, ROOM = (sizeof(xs) / 4 - 4 * 64) / PIECE;
        static_assert(ROOM >= 1, "the staging buffer holds a hand-over round");
        constexpr uint32_t PR = ROOM < 3 ? ROOM : 3;
        float* hand = reinterpret_cast<float*>(&xs[0][0]);
#pragma unroll
        for (uint32_t p0 = 0; p0 < NPC; p0 += PR) {
            __syncthreads();  // the staging buffers (or the previous round) are free
            if (rh == 1) {
#pragma unroll
                for (uint32_t pi = 0; pi < PR; pi++) {
                    if (p0 + pi >= NPC) break;
                    const v16f& v = p0 + pi < JT ? gacc[p0 + pi] : w2acc;
#pragma unroll
                    for (uint32_t r = 0; r < 16; r++) hand[((pi * 4 + grp) * 16 + r) * 64 + l] = v[r];
                }
                if (!ONES && p0 == 0) hand[PR * 4 * 16 * 64 + grp * 64 + l] = db1a;
            }
            __syncthreads();
            if (rh == 0) {
#pragma unroll
                for (uint32_t pi = 0; pi < PR; pi++) {
                    if (p0 + pi >= NPC) break;
                    v16f& v = p0 + pi < JT ? gacc[p0 + pi] : w2acc;
#pragma unroll
                    for (uint32_t r = 0; r < 16; r++) v[r] += hand[((pi * 4 + grp) * 16 + r) * 64 + l];
                }
                if (!ONES && p0 == 0) db1a += hand[PR * 4 * 16 * 64 + grp * 64 + l];
            }
        }
        if (rh == 1) return;
    }
#pragma unroll
    for (uint32_t jt = 0; jt < JT; jt++) {
        const uint32_t j = 32 * jt + lr;
        if (j < D) {
#pragma unroll
            for (uint32_t r = 0; r < 16; r++)
                dW1p[(size_t(c) * H + u0 + 32 * grp + acc_row(l, r)) * D + j] = gacc[jt][r];
        } else if (ONES && j == D) {
#pragma unroll
            for (uint32_t r = 0; r < 16; r++) db1p[size_t(c) * H + u0 + 32 * grp + acc_row(l, r)] = gacc[jt][r];
        }
    }
    // dW2^T[q][unit] sits in lanes 0-31, registers q
    if (half == 0) {
        if (!ONES) db1p[size_t(c) * H + unit] = db1a;
#pragma unroll
        for (uint32_t q = 0; q < NQ; q++) dW2p[(size_t(c) * NQ + q) * H + unit] = w2acc[q];
    }
}

// ---------------------------------------------------------------- values at s'
// Rows [tick][N]: a row whose next-state critic observation equals the next
// tick's critic observation of the same env bit for bit takes that row's
// value (the same input through the same network gives the same value); the
// others (the last tick, resets) are gathered, in any order, for their own
// evaluation: idx[i] the row, gather[i] its 32 inputs, *count of them.
__global__ __launch_bounds__(256) void next_value_split_kernel(const float* __restrict__ co,
                                                               const float* __restrict__ nco,
                                                               const float* __restrict__ values, uint32_t ticks,
                                                               uint32_t N, float* __restrict__ next_values,
                                                               uint32_t* __restrict__ count, uint32_t* __restrict__ idx,
                                                               float* __restrict__ gather) {
    // eight lanes per row, one 16-byte piece each (each load instruction
    // covers eight whole rows)
    static_assert(COBS == 32, "eight 16-byte pieces per row");
    const uint64_t e = uint64_t(blockIdx.x) * 256 + threadIdx.x, r = e / 8;
    const uint32_t k = threadIdx.x % 8, lane = threadIdx.x % 64;
    const bool live = r < uint64_t(ticks) * N;
    const uint64_t rr = live ? r : 0;
    const uint4 v = reinterpret_cast<const uint4*>(nco)[rr * 8 + k];
    bool same = live && rr / N + 1 < ticks;
    if (same) {
        const uint4 w = reinterpret_cast<const uint4*>(co)[(rr + N) * 8 + k];
        same = v.x == w.x && v.y == w.y && v.z == w.z && v.w == w.w;
    }
    const uint64_t differ = __ballot(live && !same);
    const bool row_same = ((differ >> (lane & ~7u)) & 0xffull) == 0;
    if (!live) return;
    if (row_same) {
        if (k == 0) next_values[r] = values[r + N];
        return;
    }
    uint32_t i = 0;
    if (k == 0) {
        i = atomicAdd(count, 1u);
        idx[i] = uint32_t(r);
    }
    i = __shfl(i, lane & ~7u, 64);
    reinterpret_cast<uint4*>(gather)[size_t(i) * 8 + k] = v;
}
__global__ __launch_bounds__(256) void next_value_scatter_kernel(const uint32_t* __restrict__ idx,
                                                                 const float* __restrict__ vals, uint32_t n,
                                                                 float* __restrict__ next_values) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) next_values[idx[i]] = vals[i];
}

// ---------------------------------------------------------------- reductions
constexpr uint32_t NP = 4096;  // most squared-norm partial slots (workgroups) per network

// The six gradient segments (actor W1, b1, W2, then critic W1, b1, w2) in
// one launch of at most NP workgroups striding over their elements: dst[s][j] = the
// sum over the segment's `slots` partial slots (slot-major, stride n_s) in
// slot order.  Each workgroup also leaves the sums of squares of what it
// wrote, per network, in norm_part[net][blockIdx.x] (workgroup 0 adds the
// column-sum parameters written before the launch: actor b2 and log_std,
// critic b2), the partials of the clip norm.
struct SumSegs {
    const float* src[6];
    float* dst[6];
    uint64_t start[7];  // element offsets of the segments in the launch; start[6] = total
    uint32_t slots[6];
    const float* cols_a;  // actor b2, log_std (8 values)
    const float* cols_c;  // critic b2
    float* norm_part;     // [2][NP], the first gridDim.x slots of each
};
__global__ __launch_bounds__(256) void sum_segments_kernel(SumSegs g) {
    const uint32_t t = threadIdx.x;
    float sq[2] = {0.0f, 0.0f};
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + t; i < g.start[6]; i += uint64_t(gridDim.x) * 256) {
        // the element's segment (the starts ascend), its fields picked with
        // constant indices so they stay in scalar registers (an indexed read
        // of the argument arrays is a memory load the sums would wait on)
        uint32_t sg = 0;
#pragma unroll
        for (uint32_t q = 1; q < 6; q++) sg += i >= g.start[q] ? 1u : 0u;
        const float* src = g.src[0];
        float* dst = g.dst[0];
        uint64_t s0 = g.start[0], s1 = g.start[1];
        uint32_t slots = g.slots[0];
#pragma unroll
        for (uint32_t q = 1; q < 6; q++) {
            const bool h = sg == q;
            src = h ? g.src[q] : src;
            dst = h ? g.dst[q] : dst;
            s0 = h ? g.start[q] : s0;
            s1 = h ? g.start[q + 1] : s1;
            slots = h ? g.slots[q] : slots;
        }
        const uint64_t j = i - s0, n = s1 - s0;
        // the slots in order, 32 loads in flight at a time; a slot past the
        // last adds +0, which leaves the sum (never -0) unchanged
        float s = 0.0f;
        for (uint32_t c0 = 0; c0 < slots; c0 += 32) {
            float v[32];
#pragma unroll
            for (uint32_t k = 0; k < 32; k++) v[k] = c0 + k < slots ? src[uint64_t(c0 + k) * n + j] : 0.0f;
#pragma unroll
            for (uint32_t k = 0; k < 32; k++) s += v[k];
        }
        dst[j] = s;
        sq[sg < 3 ? 0 : 1] += s * s;
    }
    if (blockIdx.x == 0 && t == 0)
        for (uint32_t k = 0; k < 8; k++) sq[0] += g.cols_a[k] * g.cols_a[k];
    if (blockIdx.x == 0 && t == 1) sq[1] += g.cols_c[0] * g.cols_c[0];
    __shared__ float red[2][256];
    red[0][t] = sq[0];
    red[1][t] = sq[1];
    __syncthreads();
    for (uint32_t w = 128; w > 0; w >>= 1) {
        if (t < w) {
            red[0][t] += red[0][t + w];
            red[1][t] += red[1][t + w];
        }
        __syncthreads();
    }
    if (t < 2) g.norm_part[t * NP + blockIdx.x] = red[t][0];
}
// Adds the column partials in block order and writes the per-row-column
// gradients into the flat vectors (actor b2, log_std; critic b2) and the four
// metric sums into metric_sums.
__global__ __launch_bounds__(64) void column_finish_kernel(const float* __restrict__ col_part, uint32_t blocks,
                                                           uint32_t H, uint32_t D, float* __restrict__ ga,
                                                           float* __restrict__ gc, float* __restrict__ metric_sums) {
    const uint32_t t = blockIdx.x, l = threadIdx.x;  // column t, lane l adds blocks l, l + 64, ...
    float s = 0.0f;
    for (uint32_t b = l; b < blocks; b += 64) s += col_part[size_t(b) * 13 + t];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (l != 0) return;
    const uint32_t A_B2 = H * D + H + 4 * H, A_LS = A_B2 + 4, C_B2 = H * COBS + 2 * H;
    if (t < 4) ga[A_B2 + t] = s;
    else if (t < 8) ga[A_LS + t - 4] = s;
    else if (t == 8) gc[C_B2] = s;
    else metric_sums[t - 9] = s;
}

// Clip scales min(1, 0.5 / ||g||) of both networks, their pre-clip norms
// ||g|| = sqrt(|g|^2 + 1e-20) (ppo_grad_norm, main.mm:963-975) and the
// update's metric row.  One wavefront per network: each lane adds every
// 64th of the `parts` partials (of the NP slots), then a butterfly over the
// lanes.
__global__ __launch_bounds__(128) void norm_finish_kernel(const float* __restrict__ part,
                                                          const float* __restrict__ metric_sums, uint32_t b,
                                                          uint32_t parts, float* __restrict__ scale,
                                                          float* __restrict__ metric_row, float* __restrict__ norm_row) {
    const uint32_t t = threadIdx.x, net = t / 64, l = t % 64;
    float s = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < NP / 64; k++) {  // every load in flight; slots past `parts` add 0
        const float v = part[net * NP + l + 64 * k];
        s += l + 64 * k < parts ? v : 0.0f;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if (l == 0) {
        const float norm = sqrt_f(s + 1.0e-20f);
        scale[net] = min_f(1.0f, 0.5f / norm);
        norm_row[net] = norm;
    }
    if (net == 1 && l < 4) metric_row[l] = l == 3 ? metric_sums[3] / float(b) : metric_sums[l];
}

struct LargeAdamArgs {
    float* actor; float* critic;
    float* am; float* av; float* cm; float* cv;
    __bf16* actor_wb; __bf16* critic_wb;
    const float* ga; const float* gc;   // gradients in the flat layouts
    const float* scale;                 // [2] clip scales
    uint32_t H, PA, PC;
    float lr, c1, c2;
};

// cpu_reference.hpp:553-567 per element: clipped gradient, Adam (0.9, 0.999,
// 1e-8) with host bias corrections, log-std clamp (603), bf16 refresh of the
// first-layer copies.  D: actor inputs.
template <uint32_t D>
__global__ __launch_bounds__(256) void adam_kernel(LargeAdamArgs a) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= uint64_t(a.PA) + a.PC) return;
    const bool critic = i >= a.PA;
    const uint32_t p = uint32_t(critic ? i - a.PA : i);
    const uint32_t A_B1 = a.H * D, A_LS = A_B1 + a.H + 4 * a.H + 4, C_B1 = a.H * COBS;
    const float gi = (critic ? a.gc[p] : a.ga[p]) * a.scale[critic ? 1 : 0];
    float* params = critic ? a.critic : a.actor;
    float* m = critic ? a.cm : a.am;
    float* v = critic ? a.cv : a.av;
    const float mi = 0.9f * m[p] + (1.0f - 0.9f) * gi;
    const float vi = 0.999f * v[p] + (1.0f - 0.999f) * gi * gi;
    m[p] = mi;
    v[p] = vi;
    float w = params[p] - a.lr * (mi / a.c1) / (sqrt_f(vi / a.c2) + 1.0e-8f);
    if (!critic && p >= A_LS) w = clamp_f(w, -2.0f, 0.5f);
    params[p] = w;
    if (!critic && p < A_B1) a.actor_wb[wsw(p / D, p % D, KA)] = (__bf16)(w * TANH_SCALE);
    if (critic && p < C_B1) a.critic_wb[wsw(p / COBS, p % COBS, KC)] = (__bf16)(w * TANH_SCALE);
}

}  // namespace lp

// ---------------------------------------------------------------- launchers
extern "C" {

hipError_t lp_launch_pack(const float* W, uint32_t H, uint32_t D, uint32_t K, __bf16* out, hipStream_t st) {
    const uint64_t n = uint64_t(H) * K;
    hipLaunchKernelGGL(lp::pack_kernel, dim3(uint32_t((n + 255) / 256)), dim3(256), 0, st, W, H, D, K, out);
    return hipGetLastError();
}

// bf16 copies of the B rows (actor inputs of width d and critic inputs): xa
// [BP][192], xaT [192][BP], xc [BP][32], xcT [32][BP] with BP = B rounded up
// to 128.  `transposed` = false skips the transposed copies (forward-only use).
hipError_t lp_launch_prep(const float* obs, const float* co, uint32_t B, uint32_t d, __bf16* xa, __bf16* xaT,
                          __bf16* xc, __bf16* xcT, bool transposed, hipStream_t st) {
    if (B == 0) return hipSuccess;
    if (obs && d != MDN_ACTOR_OBS_POOLED && d != MDN_ACTOR_OBS_PRIOR) return hipErrorInvalidValue;
    const uint32_t BP = (B + lp::RB - 1) / lp::RB * lp::RB;
    const uint32_t gx = BP / lp::RB;
    if (obs && d == MDN_ACTOR_OBS_POOLED)
        hipLaunchKernelGGL((lp::prep_kernel<MDN_ACTOR_OBS_POOLED, lp::KA>), dim3(gx), dim3(256), 0, st, obs, B, BP, xa,
                           transposed ? xaT : nullptr);
    if (obs && d == MDN_ACTOR_OBS_PRIOR)
        hipLaunchKernelGGL((lp::prep_kernel<MDN_ACTOR_OBS_PRIOR, lp::KA>), dim3(gx), dim3(256), 0, st, obs, B, BP, xa,
                           transposed ? xaT : nullptr);
    if (co)
        hipLaunchKernelGGL((lp::prep_kernel<lp::COBS, lp::KC>), dim3(gx), dim3(256), 0, st, co, B, BP, xc,
                           transposed ? xcT : nullptr);
    return hipGetLastError();
}

// Actor means [B][4] and critic values [B] of B prepared rows; a d = 184
// actor adds prior[row][0..2] (its fp32 hint inputs, row stride d) to the
// first three means.  When the
// row blocks alone would leave CUs short of two workgroups each, the hidden
// units are split in up to 8
// slices; `part` then holds the slices' partial sums (capacity
// lp_forward_part_floats(B)).
// Hidden-unit slices of a forward launch of B rows (workgroups of FWD_ROWS
// rows): enough workgroups for one per CU where the tiles divide evenly.
constexpr uint32_t FWD_ROWS = lp::FWD_RB;
static uint32_t forward_slices(uint32_t B, uint32_t H) {
    const uint32_t blocks = (B + FWD_ROWS - 1) / FWD_ROWS, tiles = H / lp::UT;
    uint32_t S = 1;
    while (blocks * S < 256 && S < 8 && tiles % (2 * S) == 0) S *= 2;
    return S;
}

uint64_t lp_forward_part_floats(uint32_t B) {
    const uint32_t BP = (B + lp::RB - 1) / lp::RB * lp::RB;
    return uint64_t(8) * BP * 4;
}

hipError_t lp_launch_forward(const __bf16* xa, const __bf16* xc, const __bf16* awb, const __bf16* cwb,
                             const float* actor, const float* critic, uint32_t H, uint32_t d, uint32_t B,
                             const float* prior, float* means, float* values, float* part, hipStream_t st) {
    if (B == 0) return hipSuccess;
    if ((d == MDN_ACTOR_OBS_PRIOR) != (prior != nullptr) && means) return hipErrorInvalidValue;
    const uint32_t BP = (B + lp::RB - 1) / lp::RB * lp::RB;
    const uint32_t S = forward_slices(B, H);
    const dim3 grid((BP + FWD_ROWS - 1) / FWD_ROWS, S);
    const uint32_t A_B1 = H * d, A_W2 = A_B1 + H, A_B2 = A_W2 + 4 * H;
    const uint32_t C_B1 = H * lp::COBS, C_W2 = C_B1 + H, C_B2 = C_W2 + H;
    if (means) {
        hipLaunchKernelGGL((lp::forward_kernel<lp::KA, 4>), grid, dim3(512), 0, st, xa, BP, awb, actor + A_B1,
                           actor + A_W2, actor + A_B2, H, B, means, part, prior, d);
        if (S > 1)
            hipLaunchKernelGGL(lp::part_sum_kernel, dim3((B * 4 + 255) / 256), dim3(256), 0, st, part, S, BP, B, 4u,
                               actor + A_B2, means, prior, d);
    }
    if (values) {
        hipLaunchKernelGGL((lp::forward_kernel<lp::KC, 1>), grid, dim3(512), 0, st, xc, BP, cwb, critic + C_B1,
                           critic + C_W2, critic + C_B2, H, B, values, part, nullptr, 0u);
        if (S > 1)
            hipLaunchKernelGGL(lp::part_sum_kernel, dim3((B + 255) / 256), dim3(256), 0, st, part, S, BP, B, 1u,
                               critic + C_B2, values, nullptr, 0u);
    }
    return hipGetLastError();
}

hipError_t lp_launch_next_value_split(const float* co, const float* nco, const float* values, uint32_t ticks,
                                      uint32_t N, float* next_values, uint32_t* count, uint32_t* idx, float* gather,
                                      hipStream_t st) {
    const uint64_t rows = uint64_t(ticks) * N;
    if (rows == 0) return hipSuccess;
    if (rows > 0xffffffffull || (reinterpret_cast<uintptr_t>(co) | reinterpret_cast<uintptr_t>(nco) |
                                 reinterpret_cast<uintptr_t>(gather)) % 16)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(lp::next_value_split_kernel, dim3(uint32_t((rows * 8 + 255) / 256)), dim3(256), 0, st, co,
                       nco, values, ticks, N, next_values, count, idx, gather);
    return hipGetLastError();
}

hipError_t lp_launch_next_value_scatter(const uint32_t* idx, const float* vals, uint32_t n, float* next_values,
                                        hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(lp::next_value_scatter_kernel, dim3((n + 255) / 256), dim3(256), 0, st, idx, vals, n,
                       next_values);
    return hipGetLastError();
}

hipError_t lp_launch_logp(const float* means, const float* actions, const float* log_std, uint32_t B, float* logp,
                          hipStream_t st) {
    if (B == 0) return hipSuccess;
    hipLaunchKernelGGL(lp::logp_kernel, dim3((B + 255) / 256), dim3(256), 0, st, means, actions, log_std, B, logp);
    return hipGetLastError();
}

hipError_t lp_launch_loss(const float* means, const float* values, const float* actions, const float* old_logp,
                          const float* adv, const float* ret, const float* log_std, uint32_t B, float clip,
                          float vcoef, float ecoef, float* dm, float* dls, float* dv, float* loss, float* col_part,
                          hipStream_t st) {
    if (B == 0) return hipSuccess;
    hipLaunchKernelGGL(lp::loss_kernel, dim3((B + lp::RB - 1) / lp::RB), dim3(lp::RB), 0, st, means, values, actions,
                       old_logp, adv, ret, log_std, B, clip, vcoef, ecoef, dm, dls, dv, loss, col_part);
    return hipGetLastError();
}

// The column sums of the per-row terms (col_part, as written by
// lp_launch_loss) into ga / gc and the metric sums, the backward of both
// networks into the partial slots, then the slot sums into the flat
// gradients ga (actor layout) and gc (critic layout) with the clip norm's
// partials.  part >= lp_backward_part_floats(B, H, d) floats; scratch >=
// lp_adam_scratch_floats() (norm partials, clip scales, metric sums), read by
// lp_launch_adam.
// Row chunks of the backward for B rows: the actor's (hidden tile, chunk)
// workgroups fill one round at one per CU; the critic, whose blocks are light,
// takes four times as many chunks and runs two workgroups per CU.
// workgroups of the segment sums (one element per thread up to NP of them),
// the number of clip-norm partials per network
static uint32_t lp_norm_parts(uint32_t H, uint32_t d) {
    const uint64_t total = uint64_t(H) * (d + 1 + 4) + uint64_t(H) * (lp::COBS + 1 + 1);
    return uint32_t(std::min<uint64_t>(lp::NP, (total + 255) / 256));
}

uint64_t lp_adam_scratch_floats() { return 2 * uint64_t(lp::NP) + 2 + 4; }

void lp_backward_chunks(uint32_t B, uint32_t H, uint32_t* actor_chunks, uint32_t* critic_chunks) {
    const uint32_t tiles = H / lp::UT, blocks = (B + lp::RB - 1) / lp::RB;
    *actor_chunks = std::max(1u, std::min(blocks, 256 / tiles));
    *critic_chunks = std::max(1u, std::min(blocks, 4 * (256 / tiles)));
}

uint64_t lp_backward_part_floats(uint32_t B, uint32_t H, uint32_t d) {
    uint32_t na, nc;
    lp_backward_chunks(B, H, &na, &nc);
    return uint64_t(na) * H * (d + 1 + 4) + uint64_t(nc) * H * (lp::COBS + 1 + 1);
}

hipError_t lp_launch_backward(const __bf16* xa, const __bf16* xaT, const __bf16* xc, const __bf16* xcT,
                              const __bf16* awb, const __bf16* cwb, const float* actor, const float* critic,
                              const float* dm, const float* dv, const float* col_part, uint32_t H, uint32_t d,
                              uint32_t B, float* part, float* ga, float* gc, float* scratch, hipStream_t st) {
    if (B == 0) return hipSuccess;
    if (d != MDN_ACTOR_OBS_POOLED && d != MDN_ACTOR_OBS_PRIOR) return hipErrorInvalidValue;
    float* metric_sums = scratch + 2 * lp::NP + 2;
    hipLaunchKernelGGL(lp::column_finish_kernel, dim3(13), dim3(64), 0, st, col_part, (B + lp::RB - 1) / lp::RB, H, d,
                       ga, gc, metric_sums);
    const uint32_t BP = (B + lp::RB - 1) / lp::RB * lp::RB;
    uint32_t ca, cc;
    lp_backward_chunks(B, H, &ca, &cc);
    auto rows_per = [&](uint32_t chunks) { return ((B + chunks - 1) / chunks + lp::RB - 1) / lp::RB * lp::RB; };
    const uint32_t RA = rows_per(ca), RCc = rows_per(cc);
    const uint32_t na = (B + RA - 1) / RA, nc = (B + RCc - 1) / RCc;
    const uint32_t A_B1 = H * d, A_W2 = A_B1 + H;
    const uint32_t C_B1 = H * lp::COBS, C_W2 = C_B1 + H;
    // partial slot layout: actor [na][H*d], [na][H], [na][4][H]; critic [nc][H*32], [nc][H], [nc][1][H]
    float* aW1 = part;
    float* ab1 = aW1 + size_t(na) * H * d;
    float* aW2 = ab1 + size_t(na) * H;
    float* cW1 = aW2 + size_t(na) * 4 * H;
    float* cb1 = cW1 + size_t(nc) * H * lp::COBS;
    float* cw2 = cb1 + size_t(nc) * H;
    if (d == MDN_ACTOR_OBS_POOLED)
        hipLaunchKernelGGL((lp::backward_kernel<MDN_ACTOR_OBS_POOLED, lp::KA, 4, 8>), dim3(H / lp::UT, na), dim3(512), 0,
                           st, xa, xaT, BP, awb, actor + A_B1, actor + A_W2, dm, H, B, RA, aW1, ab1, aW2);
    else
        hipLaunchKernelGGL((lp::backward_kernel<MDN_ACTOR_OBS_PRIOR, lp::KA, 4, 8>), dim3(H / lp::UT, na), dim3(512), 0,
                           st, xa, xaT, BP, awb, actor + A_B1, actor + A_W2, dm, H, B, RA, aW1, ab1, aW2);
    hipLaunchKernelGGL((lp::backward_kernel<lp::COBS, lp::KC, 1, 4>), dim3(H / lp::UT, nc), dim3(256), 0, st, xc, xcT,
                       BP, cwb, critic + C_B1, critic + C_W2, dv, H, B, RCc, cW1, cb1, cw2);
    lp::SumSegs g;
    const float* srcs[6] = {aW1, ab1, aW2, cW1, cb1, cw2};
    float* dsts[6] = {ga, ga + A_B1, ga + A_W2, gc, gc + C_B1, gc + C_W2};
    const uint64_t ns[6] = {uint64_t(H) * d, H, 4ull * H, uint64_t(H) * lp::COBS, H, H};
    const uint32_t slots[6] = {na, na, na, nc, nc, nc};
    g.start[0] = 0;
    for (int k = 0; k < 6; k++) {
        g.src[k] = srcs[k];
        g.dst[k] = dsts[k];
        g.slots[k] = slots[k];
        g.start[k + 1] = g.start[k] + ns[k];
    }
    g.cols_a = ga + A_W2 + 4 * H;
    g.cols_c = gc + C_W2 + H;
    g.norm_part = scratch;
    hipLaunchKernelGGL(lp::sum_segments_kernel, dim3(lp_norm_parts(H, d)), dim3(256), 0, st, g);
    return hipGetLastError();
}

// Clip + Adam of both networks from the gradients, norm partials and metric
// sums lp_launch_backward left in ga, gc and scratch.
hipError_t lp_launch_adam(float* actor, float* critic, float* am, float* av, float* cm, float* cv, __bf16* awb,
                          __bf16* cwb, float* ga, float* gc, float* scratch, uint32_t B, uint32_t H, uint32_t d,
                          float lr, float c1, float c2, float* metric_row, float* norm_row, hipStream_t st) {
    if (d != MDN_ACTOR_OBS_POOLED && d != MDN_ACTOR_OBS_PRIOR) return hipErrorInvalidValue;
    const uint32_t PA = H * d + H + 4 * H + 8, PC = H * lp::COBS + 2 * H + 1;
    float* norm_part = scratch;
    float* scale = scratch + 2 * lp::NP;
    float* metric_sums = scale + 2;
    hipLaunchKernelGGL(lp::norm_finish_kernel, dim3(1), dim3(128), 0, st, norm_part, metric_sums, B,
                       lp_norm_parts(H, d), scale, metric_row, norm_row);
    lp::LargeAdamArgs a;
    a.actor = actor; a.critic = critic; a.am = am; a.av = av; a.cm = cm; a.cv = cv;
    a.actor_wb = awb; a.critic_wb = cwb; a.ga = ga; a.gc = gc; a.scale = scale;
    a.H = H; a.PA = PA; a.PC = PC; a.lr = lr; a.c1 = c1; a.c2 = c2;
    if (d == MDN_ACTOR_OBS_POOLED)
        hipLaunchKernelGGL(lp::adam_kernel<MDN_ACTOR_OBS_POOLED>, dim3((PA + PC + 255) / 256), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL(lp::adam_kernel<MDN_ACTOR_OBS_PRIOR>, dim3((PA + PC + 255) / 256), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // extern "C"
