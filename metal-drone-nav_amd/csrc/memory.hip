// memory.hip — the geometry-memory hint of the 184-input actor
// (guidance.hpp:100-194 nav_memory_clearance / nav_guidance_memory, as the CPU
// reference calls it: cpu_reference.hpp:353-375; the reference's GPU splits it
// into memory.metal:9-153 + sim.metal:226).
//
// One 256-thread workgroup per env, run between the env kernel's observation
// of a tick and the launch that acts on it:
//   1. the env's up to 8 x 80 remembered range hits become body-frame points
//      (position, |p|^2, 3 + radius, radius^2), built once instead of once
//      per candidate direction.  Only points that some sweep could touch are
//      kept (compacted into LDS): a contact needs along <= 3 + radius and
//      |p|^2 - along^2 < radius^2, so a point with |p|^2 above
//      (3 + radius)^2 + radius^2 (with a 0.1 % margin for rounding) is never
//      one, whatever the sweep.  The kept points are grouped nearest first
//      in four distance shells, and padded with points no sweep touches to a
//      multiple of three;
//   2. 255 threads = 85 candidate sweeps x 3 interleaved thirds of the kept
//      points scan them (every lane of a third reads the same point: LDS
//      broadcast) with one trip count for the whole workgroup; the nearest
//      contacts are combined with a min, which is exact in any order, so the
//      order of the points does not change the result.  Near points first
//      lower each sweep's running nearest contact early, which lets the
//      exact skip test (below) drop most later contacts before their square
//      root;
//   3. the 85 candidates are scored and reduced with the sequential scan's
//      rule (maximum score, first candidate on ties), and one lane writes the
//      hint to the row's last three inputs.
// Every value is computed with the operations and order of the oracle's
// restatement, so the hint is bit-identical to it.
#include <hip/hip_runtime.h>

#include "kernel_args.h"
#include "mdnav_math.h"
#include "mdnav_types.h"

namespace mem {
using namespace mdn;

constexpr uint32_t OBS = MDN_ACTOR_OBS_PRIOR;
constexpr uint32_t POINTS = 640, CANDIDATES = 85, PARTS = 3;
constexpr uint32_t THREADS = 256;

__device__ __forceinline__ float fbits(uint32_t u) { return __builtin_bit_cast(float, u); }
// Correctly rounded square root of a positive normal x >= 2^-96: the
// hardware estimate and the one-ulp correction of the compiler's own
// correctly rounded sqrt lowering, without its scaling of tiny inputs and its
// zero / infinity fix-up, neither of which applies in that range (the
// instruction sequence is otherwise the same, so the results are equal).
__device__ __forceinline__ float sqrt_pos(float x) {
    const float s = __builtin_amdgcn_sqrtf(x);
    const uint32_t b = __builtin_bit_cast(uint32_t, s);
    const float dn = fbits(b - 1u), up = fbits(b + 1u);
    float r = __builtin_fmaf(-dn, s, x) <= 0.0f ? dn : s;
    r = __builtin_fmaf(-up, s, x) > 0.0f ? up : r;
    return r;
}
constexpr uint32_t SHELLS = 4;
// distance shell of a kept point by |p|^2: (< 1 m, < 2 m, < 3 m, beyond)
__device__ __forceinline__ uint32_t shell_of(float p2) {
    return p2 < 1.0f ? 0u : (p2 < 4.0f ? 1u : (p2 < 9.0f ? 2u : 3u));
}
__device__ __forceinline__ float div_r(float x, double r) { return float(double(x) * r); }

struct Point {
    float4 xyz2;  // body-frame x, y, z and x^2 + y^2 + z^2
    float4 lim;   // 3 + radius, radius^2, an upper bound of sqrt(radius^2), unused
};

// guidance.hpp:27-34 over the LDS copy of the current ranges (already x 12)
__device__ __forceinline__ float min3x3(const float* cur, int row, int col) {
    float nearest = 12.0f;
    for (int dr = -1; dr <= 1; dr++)
        for (int dc = -1; dc <= 1; dc++) {
            const int r = row + dr, c = col + dc;
            if (r >= 0 && r < 8 && c >= 0 && c < 10) nearest = fmin_f(nearest, cur[r * 10 + c]);
        }
    return nearest;
}
// guidance.hpp:55-63 over the per-cell risk contributions (0 or min(0.2 u, 1))
__device__ __forceinline__ float max3x3(const float* v, int row, int col) {
    float risk = 0.0f;
    for (int dr = -1; dr <= 1; dr++)
        for (int dc = -1; dc <= 1; dc++) {
            const int r = row + dr, c = col + dc;
            if (r >= 0 && r < 8 && c >= 0 && c < 10) risk = fmax_f(risk, v[r * 10 + c]);
        }
    return risk;
}

// arg-max over a wavefront with the first index winning ties
__device__ __forceinline__ void wave_argmax(float& v, uint32_t& idx) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const uint32_t oi = __shfl_xor(idx, off, 64);
        if (ov > v || (ov == v && oi < idx)) { v = ov; idx = oi; }
    }
}

__global__ __launch_bounds__(THREADS) void memory_hint_kernel(nav::MemoryArgs a) {
    __shared__ Point pts[POINTS + 2];  // + padding to a multiple of three
    __shared__ float cur[80], risk_v[80], part_near[PARTS][CANDIDATES];
    __shared__ float cand_score[2], cand_free[CANDIDATES];
    __shared__ uint32_t cand_idx[2], goal_cell_s[2];
    __shared__ float goal_al_s[2];
    __shared__ uint32_t shell_count[SHELLS], shell_base[SHELLS + 1];
    const uint32_t n = blockIdx.x, t = threadIdx.x, wv = t / 64, lane = t % 64;
    const uint32_t* hd = a.head + size_t(n) * nav::MEM_HEAD_WORDS;
    if (hd[nav::MEM_HEAD_OBSERVED] == 0u) return;  // uniform over the workgroup
    float* og = a.obs + size_t(n) * OBS;
    const float* ctx = og + 160;
    const float distance = fbits(hd[nav::MEM_HEAD_DISTANCE]);
    const float gin[3] = {ctx[0], ctx[1], ctx[2]};
    const float vel[3] = {ctx[4] * 4.0f, ctx[5] * 4.0f, ctx[6] * 4.0f};
    const float gnorm = sqrt_f(gin[0] * gin[0] + gin[1] * gin[1] + gin[2] * gin[2]);
    if (gnorm < 1e-6f || distance < 0.05f) {
        if (t < 3) og[OBS - 3 + t] = 0.0f;
        return;
    }
    const float goal[3] = {gin[0] / gnorm, gin[1] / gnorm, gin[2] / gnorm};
    const float speed = sqrt_f(vel[0] * vel[0] + vel[1] * vel[1] + vel[2] * vel[2]);
    const float sensor_dt = a.sensor_dt;
    const float stop_margin = 0.28f + speed * fmax_f(sensor_dt, 0.0f) + 0.25f * speed * speed;
    const uint32_t latest = hd[nav::MEM_HEAD_FRAME], valid = hd[nav::MEM_HEAD_VALID];
    float pose[12];
#pragma unroll
    for (int j = 0; j < 12; j++) pose[j] = fbits(hd[nav::MEM_HEAD_POSE + j]);

    if (t < SHELLS) shell_count[t] = 0;
    __syncthreads();
    // 1. remembered points (guidance.hpp:113-139 up to the sweep test); each
    // thread keeps its up to three points in registers while the shells are
    // counted
    constexpr uint32_t PER = (POINTS + THREADS - 1) / THREADS;
    Point held[PER];
    uint32_t held_shell[PER], held_slot[PER];
#pragma unroll
    for (uint32_t k = 0; k < PER; k++) {
        const uint32_t j = k * THREADS + t;
        const uint32_t back = j / 80, cell = j % 80, row = cell / 10, col = cell % 10;
        Point p;
        bool keep = false;
        if (j < POINTS && back < valid) {
            const uint32_t frame = (latest + 8u - back) % 8u;
            const float* old_pose = a.poses + (size_t(n) * 8 + frame) * 12;
            const float* ranges = a.sensors + (size_t(n) * 8 + frame) * 320;
            const uint32_t px = row * 2 * 20 + col * 2;
            uint32_t hit = px;
            float range = ranges[px];
            const uint32_t pixels[3] = {px + 1, px + 20, px + 21};
#pragma unroll
            for (int k = 0; k < 3; k++)
                if (ranges[pixels[k]] < range) { range = ranges[pixels[k]]; hit = pixels[k]; }
            if (!(range <= 0.01f || range >= 11.9f)) {
                const float* ray = a.pix_rays + 3 * hit;
                const float wx = old_pose[3] * ray[0] + old_pose[4] * ray[1] + old_pose[5] * ray[2];
                const float wy = old_pose[6] * ray[0] + old_pose[7] * ray[1] + old_pose[8] * ray[2];
                const float wz = old_pose[9] * ray[0] + old_pose[10] * ray[1] + old_pose[11] * ray[2];
                const float dx = old_pose[0] + range * wx - pose[0];
                const float dy = old_pose[1] + range * wy - pose[1];
                const float dz = old_pose[2] + range * wz - pose[2];
                const float x = pose[3] * dx + pose[6] * dy + pose[9] * dz;
                const float y = pose[4] * dx + pose[7] * dy + pose[10] * dz;
                const float z = pose[5] * dx + pose[8] * dy + pose[11] * dz;
                // nav_memory_point_radius with the capture-age term off
                const float age = fmax_f(float(back) * fmax_f(sensor_dt, 0.0f), 0.0f) + 0.0f;
                const float radius = 0.20f + 0.015f * range + 0.15f * age;
                p.xyz2 = make_float4(x, y, z, x * x + y * y + z * z);
                p.lim = make_float4(3.0f + radius, radius * radius, radius * 1.0001f + 1e-6f, 0.0f);
                keep = p.xyz2.w <= 1.001f * (p.lim.x * p.lim.x + p.lim.y);
            }
        }
        held[k] = p;
        held_shell[k] = keep ? shell_of(p.xyz2.w) : SHELLS;
        held_slot[k] = keep ? atomicAdd(&shell_count[held_shell[k]], 1u) : 0u;
    }
    __syncthreads();
    if (t == 0) {
        shell_base[0] = 0;
        for (uint32_t k = 0; k < SHELLS; k++) shell_base[k + 1] = shell_base[k] + shell_count[k];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t k = 0; k < PER; k++)
        if (held_shell[k] < SHELLS) pts[shell_base[held_shell[k]] + held_slot[k]] = held[k];
    {   // padding to a multiple of three: at the origin, no sweep has along > 0
        const uint32_t total = shell_base[SHELLS], padded = (total + 2u) / 3u * 3u;
        if (t < padded - total) {
            Point z;
            z.xyz2 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            z.lim = make_float4(-1.0f, 0.0f, 0.0f, 0.0f);
            pts[total + t] = z;
        }
    }
    // per-cell current range x 12 and closing-speed risk contribution
    if (t < 80) {
        const float now = og[t] * 12.0f, old = og[80 + t] * 12.0f;
        cur[t] = now;
        const float* ray = a.cells + 3 * t;
        const float unexpected = div_r(old - now, a.inv_sensor_dt) - (vel[0] * ray[0] + vel[1] * ray[1] + vel[2] * ray[2]);
        const bool hit = (sensor_dt > 1e-4f) & (old < 11.9f) & (now < 11.9f) & (unexpected > 0.5f);
        risk_v[t] = hit ? fmin_f(0.20f * unexpected, 1.0f) : 0.0f;
    }
    // goal cell: the cell ray best aligned with the goal (first on ties), wave 0 and 1
    if (t < 128) {
        float al = -1e20f;
        uint32_t c = 80;
        if (t < 80) {
            const float* d = a.cells + 3 * t;
            al = d[0] * goal[0] + d[1] * goal[1] + d[2] * goal[2];
            if (!(al == al)) al = -INFINITY;  // the scan never selects a NaN
            c = t;
        }
        wave_argmax(al, c);
        if ((t & 63) == 0) { goal_al_s[wv] = al; goal_cell_s[wv] = c; }
    }
    __syncthreads();
    uint32_t gcell = goal_cell_s[0];
    if (goal_al_s[1] > goal_al_s[0] || (goal_al_s[1] == goal_al_s[0] && goal_cell_s[1] < gcell)) gcell = goal_cell_s[1];
    const float gsel = goal_al_s[1] > goal_al_s[0] || (goal_al_s[1] == goal_al_s[0] && goal_cell_s[1] < goal_cell_s[0])
                           ? goal_al_s[1] : goal_al_s[0];
    // scan's fallback without any finite alignment: cell (0, 0)
    const uint32_t goal_row = gsel > -1e20f ? gcell / 10 : 0, goal_col = gsel > -1e20f ? gcell % 10 : 0;

    // candidate direction (guidance.hpp:164-166)
    auto direction = [&](uint32_t c, float d[3]) {
        if (c < 80) {
            d[0] = a.cells[3 * c]; d[1] = a.cells[3 * c + 1]; d[2] = a.cells[3 * c + 2];
        } else if (c == 80) {
            d[0] = goal[0]; d[1] = goal[1]; d[2] = goal[2];
        } else {
            d[0] = 0.0f;
            d[1] = c >= 83 ? (c == 83 ? 1.0f : -1.0f) : 0.0f;
            d[2] = c < 83 ? (c == 81 ? 1.0f : -1.0f) : 0.0f;
        }
    };

    // 2. swept-sphere clearance of every candidate over a third of the points
    // (guidance.hpp:134-139)
    const uint32_t iters = __builtin_amdgcn_readfirstlane((shell_base[SHELLS] + 2u) / 3u);
    if (t < PARTS * CANDIDATES) {
        const uint32_t c = t % CANDIDATES, part = t / CANDIDATES;
        float d[3];
        direction(c, d);
        float sw[3] = {1.2f * d[0] + 0.35f * vel[0], 1.2f * d[1] + 0.35f * vel[1], 1.2f * d[2] + 0.35f * vel[2]};
        const float sn = sqrt_f(sw[0] * sw[0] + sw[1] * sw[1] + sw[2] * sw[2]);
#pragma unroll
        for (int j = 0; j < 3; j++) sw[j] /= fmax_f(sn, 1e-6f);
        // A contact is along - sqrt(radius^2 - lateral^2) >= along - radius
        // (rounded values included: sqrt of at most radius^2 rounds to at most
        // radius (1 + 2^-23)), so a point with along - 1.0001 radius >= nearest
        // cannot lower nearest and its square root is skipped.  The state is
        // finite at an observation (the advance resets non-finite states), so
        // `along` is never NaN.
        // The argument of the square root is l.y - lateral2 > 0 with
        // l.y = radius^2 >= 0.04, so it is at least half an ulp of 0.04
        // (about 2e-9), a normal number: sqrt_pos applies.  No operand of
        // the min / max below is NaN (finite points and sweeps) or -0 (a
        // difference of equal values rounds to +0), so the hardware min and
        // max equal the oracle's fmin / fmax.
        float nearest = 3.0f;
        const Point* pp = pts + part;
#pragma unroll 2
        for (uint32_t i = 0; i < iters; i++) {
            const float4 q = pp[3 * i].xyz2;
            const float4 l = pp[3 * i].lim;
            const float along = q.x * sw[0] + q.y * sw[1] + q.z * sw[2];
            const float lateral2 = __builtin_fmaxf(q.w - along * along, 0.0f);
            const bool contact = (along > 0.0f) & (along <= l.x) & (lateral2 < l.y) & (along - l.z < nearest);
            if (contact) nearest = __builtin_fminf(nearest, __builtin_fmaxf(along - sqrt_pos(l.y - lateral2), 0.0f));
        }
        part_near[part][c] = nearest;
    }
    __syncthreads();

    // 3. candidate scores (guidance.hpp:167-183) and the best candidate
    const float desired_speed = fmin_f(1.6f, sqrt_f(4.0f * fmax_f(distance - 0.28f, 0.0f)));
    float score = -1e20f;
    uint32_t ci = CANDIDATES;
    if (t < CANDIDATES) {
        float d[3];
        direction(t, d);
        const int row = t < 80 ? int(t / 10) : int(goal_row), col = t < 80 ? int(t % 10) : int(goal_col);
        float free = fmin_f(fmin_f(part_near[0][t], part_near[1][t]), part_near[2][t]);
        const float observed = min3x3(cur, row, col);
        if (t < 81) free = fmin_f(free, observed);
        const float temporal_risk = max3x3(risk_v, row, col);
        free = fmax_f(free - temporal_risk, 0.0f);
        const float alignment = d[0] * goal[0] + d[1] * goal[1] + d[2] * goal[2];
        const float required = stop_margin + 0.15f + desired_speed * desired_speed * .25f;
        score = 1.4f * alignment + 0.20f * fmin_f(free, 3.0f) - (free < required ? 3.0f * (required - free) / required : 0.0f);
        if (!(score == score)) score = -INFINITY;  // the scan never selects a NaN
        ci = t;
        cand_free[t] = free;
    }
    if (t < 128) {
        wave_argmax(score, ci);
        if ((t & 63) == 0) { cand_score[wv] = score; cand_idx[wv] = ci; }
    }
    __syncthreads();
    if (t == 0) {
        uint32_t best = cand_idx[0];
        if (cand_score[1] > cand_score[0] || (cand_score[1] == cand_score[0] && cand_idx[1] < best)) best = cand_idx[1];
        const bool any = (cand_score[0] > -1e20f) | (cand_score[1] > -1e20f);
        float best_dir[3] = {1.0f, 0.0f, 0.0f}, best_free = 0.0f;
        if (any) {
            direction(best, best_dir);
            best_free = cand_free[best];
        }
        const float tan_v = a.tan_v;
        const bool goal_in_fov = goal[0] > 0.0f && fabs_f(goal[1]) <= goal[0] && fabs_f(goal[2]) <= tan_v * goal[0];
        const float after_stop = fmax_f(best_free - stop_margin - 0.15f, 0.0f);
        float command_speed = fmin_f(desired_speed, sqrt_f(4.0f * after_stop));
        if (!goal_in_fov) command_speed = fmin_f(command_speed, 0.25f);
        const float fraction = fmin_f(0.8f, command_speed * 0.5f);
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const float x = fraction * best_dir[i];
            og[OBS - 3 + i] = 0.5f * log_f((1.0f + x) / (1.0f - x));
        }
    }
}

}  // namespace mem

extern "C" hipError_t nav_launch_memory_hint(const nav::MemoryArgs* a, hipStream_t st) {
    if (a->n == 0) return hipSuccess;
    hipLaunchKernelGGL(mem::memory_hint_kernel, dim3(a->n), dim3(mem::THREADS), 0, st, *a);
    return hipGetLastError();
}
