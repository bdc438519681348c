// nav_episode.h — per-episode work that runs once per reset, one thread per
// env: the episode's plant draw (physics_domain.hpp:42-155 with the Metal
// seed hash of sim.metal:50-54) and the goal-conditioned navigation task
// (navigation_tasks.hpp:209-548) over the env's WWorld word row; plus the
// task's per-tick step, evaluated inside the rollout kernel.
//
// Arithmetic follows the reference's statement order with this library's
// own correctly rounded sqrt / sin / cos; several RNG draws inside one
// argument list are sequenced left to right, as the Metal compiler orders
// them.
#pragma once

#include "nav_device.h"

namespace nav {

// ---------------------------------------------------------------- plant draw
// xorshift 13/17/5 that never yields or keeps 0 (physics_domain.hpp:42-47)
__device__ __forceinline__ uint32_t dom_next(uint32_t& s) {
    uint32_t v = s ? s : 1u;
    v ^= v << 13; v ^= v >> 17; v ^= v << 5;
    s = v ? v : 1u;
    return s;
}
__device__ __forceinline__ float dom_scale(uint32_t& s, float lo, float hi, float amp) {
    const float u = float(dom_next(s) >> 8) * (1.0f / 16777216.0f);
    const float draw = lo + (hi - lo) * u;
    return 1.0f + amp * (draw - 1.0f);
}
__device__ __forceinline__ bool dom_range_ok(float lo, float hi) {
    return isfinite_f(lo) && isfinite_f(hi) && lo > 0.0f && lo <= hi;
}
// physics_domain.hpp:98-155: `out` is the drawn plant when the draw is
// accepted (returns true)
__device__ bool dom_sample(const MdnPhysicsParams& p, uint32_t rng, float amp, const MdnDomainRange& R,
                           MdnPhysicsParams& out) {
    if (!isfinite_f(amp) || amp < 0.0f || amp > 1.0f || !isfinite_f(R.minimum_thrust_to_weight) ||
        R.minimum_thrust_to_weight < 1.0f || !dom_range_ok(R.mass_scale_min, R.mass_scale_max) ||
        !dom_range_ok(R.inertia_axis_scale_min, R.inertia_axis_scale_max) ||
        !dom_range_ok(R.thrust_gain_min, R.thrust_gain_max) ||
        !dom_range_ok(R.rising_lag_scale_min, R.rising_lag_scale_max) ||
        !dom_range_ok(R.falling_lag_scale_min, R.falling_lag_scale_max))
        return false;
    out = p;
    if (amp > 0.0f) {
        const float mass_scale = dom_scale(rng, R.mass_scale_min, R.mass_scale_max, amp);
        float axis[3], gain[4], rise[4], fall[4];
        for (int k = 0; k < 3; k++) axis[k] = dom_scale(rng, R.inertia_axis_scale_min, R.inertia_axis_scale_max, amp);
        for (int r = 0; r < 4; r++) {
            gain[r] = dom_scale(rng, R.thrust_gain_min, R.thrust_gain_max, amp);
            rise[r] = dom_scale(rng, R.rising_lag_scale_min, R.rising_lag_scale_max, amp);
            fall[r] = dom_scale(rng, R.falling_lag_scale_min, R.falling_lag_scale_max, amp);
        }
        out.mass = p.mass * mass_scale;
        float root[3];
        for (int k = 0; k < 3; k++) root[k] = sqrt_f(axis[k]);
        float* I = out.inertia;
        for (int row = 0; row < 3; row++)
            for (int col = 0; col < 3; col++) I[3 * row + col] = p.inertia[3 * row + col] * mass_scale * root[row] * root[col];
        // physics_domain.hpp:59-80: cofactor inverse of a symmetric
        // positive-definite inertia
        for (int j = 0; j < 9; j++) if (!isfinite_f(I[j])) return false;
        const float a = I[0], b = I[1], c = I[2], d = I[3], e = I[4], f = I[5], g = I[6], h = I[7], i = I[8];
        if (fabs_f(b - d) > 1.0e-6f || fabs_f(c - g) > 1.0e-6f || fabs_f(f - h) > 1.0e-6f) return false;
        const float minor2 = a * e - b * d;
        const float det = a * (e * i - f * h) - b * (d * i - f * g) + c * (d * h - e * g);
        if (!(a > 0.0f) || !(minor2 > 0.0f) || !(det > 0.0f) || !isfinite_f(det)) return false;
        const float rd = 1.0f / det;
        float* J = out.inertia_inverse;
        J[0] = (e * i - f * h) * rd; J[1] = (c * h - b * i) * rd; J[2] = (b * f - c * e) * rd;
        J[3] = (f * g - d * i) * rd; J[4] = (a * i - c * g) * rd; J[5] = (c * d - a * f) * rd;
        J[6] = (d * h - e * g) * rd; J[7] = (b * g - a * h) * rd; J[8] = (a * e - b * d) * rd;
        for (int j = 0; j < 9; j++) if (!isfinite_f(J[j])) return false;
        for (int r = 0; r < 4; r++) {
            for (int k = 0; k < 3; k++)
                out.rotor_thrust_coefficients[3 * r + k] = p.rotor_thrust_coefficients[3 * r + k] * gain[r];
            out.rotor_time_constants_rising[r] = p.rotor_time_constants_rising[r] * rise[r];
            out.rotor_time_constants_falling[r] = p.rotor_time_constants_falling[r] * fall[r];
        }
    }
    // physics_domain.hpp:82-93: vertical thrust at full action over the weight
    float lift = 0.0f;
    const float u = out.action_max;
    for (int r = 0; r < 4; r++) {
        const float* c = &out.rotor_thrust_coefficients[3 * r];
        lift += out.rotor_thrust_directions[3 * r + 2] * (c[0] + c[1] * u + c[2] * u * u);
    }
    const float weight = out.mass * fabs_f(out.gravity_world[2]);
    const float t2w = weight > 0.0f ? lift / weight : 0.0f;
    return t2w >= R.minimum_thrust_to_weight;
}
// sim.metal:50-54
__device__ __forceinline__ uint32_t dom_seed(const MdnRuntimeConfig& rt, uint32_t cfg_seed, uint32_t env,
                                             uint32_t episode) {
    uint32_t h = rt.domain_seed ^ cfg_seed ^ ((env + 1u) * 0x9e3779b9u) ^ ((episode + 1u) * 0x85ebca6bu);
    h ^= h >> 16; h *= 0x7feb352du; h ^= h >> 15; h *= 0x846ca68bu; h ^= h >> 16;
    return h ? h : 1u;
}

// ---------------------------------------------------------------- tasks
__device__ __forceinline__ V add3(V a, V b) { return mk(a.x + b.x, a.y + b.y, a.z + b.z); }
__device__ __forceinline__ V mul3(V a, float s) { return mk(a.x * s, a.y * s, a.z * s); }
__device__ __forceinline__ float task_clamp(float v, float lo, float hi) { return fmin_f(fmax_f(v, lo), hi); }
__device__ __forceinline__ bool task_inside(V p, const float* lo, const float* hi) {
    return p.x >= lo[0] && p.x <= hi[0] && p.y >= lo[1] && p.y <= hi[1] && p.z >= lo[2] && p.z <= hi[2];
}
// navigation_tasks.hpp:243-255: clearance of the static scene along a
// segment, sampled at most 5 cm apart.  The episode kernel runs one
// wavefront per env with every lane on the same values; the samples are
// split over the 64 lanes and their minimum taken with xor shuffles (every
// clearance is finite and none is -0, so the minimum does not depend on the
// order).
__device__ float task_segment_clearance(const float* w, uint32_t count, V a, V b) {
    const V d = sub3(b, a);
    const float distance = len3(d);
    uint32_t samples = uint32_t(__builtin_ceilf(distance / 0.05f));
    if (samples < 1u) samples = 1u;
    if (samples > 512u) return -1e6f;
    float minimum = 1e20f;
    for (uint32_t k = threadIdx.x % 64u; k <= samples; k += 64u) {
        const float t = float(k) / float(samples);
        minimum = fmin_f(minimum, clearance_at(w, count, add3(a, mul3(d, t)), 0.0f));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) minimum = fmin_f(minimum, __shfl_xor(minimum, off, 64));
    return minimum;
}
// navigation_tasks.hpp:257-263 over 2 to 4 points
__device__ float task_path_clearance(const float* w, uint32_t count, const V* p, uint32_t n) {
    float minimum = 1e20f;
    for (uint32_t s = 0; s + 1u < n; s++) minimum = fmin_f(minimum, task_segment_clearance(w, count, p[s], p[s + 1]));
    return minimum;
}
struct TaskWitness { V p[4]; uint32_t n; float clearance, length; };
// navigation_tasks.hpp:265-277
__device__ __forceinline__ void task_save(TaskWitness& out, const V* path, uint32_t n, float cl) {
    out.n = n;
    out.clearance = cl;
    float total = 0;
    for (uint32_t s = 0; s + 1u < n; s++) total += len3(sub3(path[s + 1], path[s]));
    out.length = total;
    for (uint32_t i = 0; i < 4; i++) out.p[i] = i < n ? path[i] : mk(0, 0, 0);
}
__device__ __forceinline__ bool task_accept(const float* w, uint32_t count, const V* path, uint32_t n, float thr,
                                            TaskWitness& out) {
    const float cl = task_path_clearance(w, count, path, n);
    if (!(cl > thr)) return false;
    task_save(out, path, n, cl);
    return true;
}
// navigation_tasks.hpp:281-345: the direct line, else the first clear path
// of a fixed list of doglegs
__device__ bool task_witness(const float* w, uint32_t count, V start, V goal, const MdnTaskConfig& c,
                             TaskWitness& out, float& direct) {
    const float thr = c.minimum_witness_clearance_m;
    // the candidate path in the wavefront's LDS (every lane holds the same
    // points; indexed by segment, it would otherwise live in scratch)
    __shared__ V path[4];
    path[0] = start; path[1] = goal; path[2] = goal; path[3] = goal;
    direct = task_path_clearance(w, count, path, 2);
    if (direct > thr && c.require_detour == 0u) {
        task_save(out, path, 2, direct);
        return true;
    }
    if (direct > thr) return false;
    const V dl = sub3(goal, start);
    const float xf[5] = {0.10f, 0.25f, 0.50f, 0.75f, 0.90f};
    path[2] = goal;
    for (int side = 0; side < 2; side++) {
        const float y = side ? 4.60f : -4.60f;
        for (int i = 0; i < 5; i++) {
            path[1] = mk(start.x + xf[i] * dl.x, y, start.z + xf[i] * dl.z);
            if (task_accept(w, count, path, 3, thr, out)) return true;
        }
    }
    const float off[4] = {-2.4f, -1.2f, 1.2f, 2.4f};
    for (int i = 0; i < 4; i++) {
        path[1] = mk(start.x + 0.5f * dl.x, task_clamp((start.y + goal.y) * 0.5f + off[i], -4.60f, 4.60f),
                     start.z + 0.5f * dl.z);
        if (task_accept(w, count, path, 3, thr, out)) return true;
    }
    for (int i = 0; i < 2; i++) {
        path[1] = mk(start.x + 0.5f * dl.x, start.y + 0.5f * dl.y, i ? 4.45f : 0.55f);
        if (task_accept(w, count, path, 3, thr, out)) return true;
    }
    for (int side = 0; side < 2; side++) {
        const float y = side ? 4.60f : -4.60f;
        path[1] = mk(start.x + 0.20f * dl.x, y, start.z + 0.20f * dl.z);
        path[2] = mk(start.x + 0.80f * dl.x, y, start.z + 0.80f * dl.z);
        path[3] = goal;
        if (task_accept(w, count, path, 4, thr, out)) return true;
    }
    return false;
}
__device__ __forceinline__ bool task_fin(float x) { return isfinite_f(x); }
// navigation_tasks.hpp:355-388 (version 0, the generator without the
// clutter-goal conditioning, is accepted besides version 1)
__device__ bool task_config_valid(const MdnTaskConfig& c) {
    if (c.generation_version > 1u || c.stage > MDN_TASK_STAGE_CLUTTER_GOAL ||
        c.objective > MDN_TASK_OBJECTIVE_FINAL_HOLD || c.family > 16u || c.require_detour > 1u ||
        !task_fin(c.scene_distance_m) || c.scene_distance_m < 3.0f || c.scene_distance_m > 10.0f ||
        !task_fin(c.difficulty) || c.difficulty < 0.0f || c.difficulty > 1.0f || !task_fin(c.goal_distance_min_m) ||
        !task_fin(c.goal_distance_max_m) || c.goal_distance_min_m <= c.goal_radius_m ||
        c.goal_distance_max_m < c.goal_distance_min_m || !task_fin(c.minimum_endpoint_clearance_m) ||
        c.minimum_endpoint_clearance_m < 0.30f || !task_fin(c.minimum_witness_clearance_m) ||
        c.minimum_witness_clearance_m < 0.02f || !task_fin(c.goal_radius_m) || c.goal_radius_m <= 0.0f ||
        !task_fin(c.stable_speed_mps) || c.stable_speed_mps < 0.0f || !task_fin(c.stable_hold_s) ||
        c.stable_hold_s < 0.0f || !task_fin(c.nav_period_s) || c.nav_period_s <= 0.0f ||
        !task_fin(c.initial_speed_min_mps) || !task_fin(c.initial_speed_max_mps) || c.initial_speed_min_mps < 0.0f ||
        c.initial_speed_max_mps < c.initial_speed_min_mps || !task_fin(c.progress_reward_per_m) ||
        c.progress_reward_per_m < 0.0f || !task_fin(c.time_cost_per_s) || c.time_cost_per_s < 0.0f ||
        !task_fin(c.contact_penalty) || c.contact_penalty < 0.0f || !task_fin(c.stable_arrival_bonus) ||
        c.stable_arrival_bonus < 0.0f || !task_fin(c.command_smoothness_weight) || c.command_smoothness_weight < 0.0f ||
        c.max_nav_steps == 0u || c.max_generation_attempts == 0u)
        return false;
    return true;
}
__device__ __forceinline__ V task_direction(uint32_t& rng) {
    const float z = 2.0f * ur(rng) - 1.0f;
    const float angle = 6.28318530718f * ur(rng);
    const float radial = sqrt_f(fmax_f(0.0f, 1.0f - z * z));
    float s, co;
    sincos_f(angle, &s, &co);
    return mk(radial * co, radial * s, z);
}
__device__ __forceinline__ V task_point(uint32_t& rng, const float* lo, const float* hi) {
    const float x = lo[0] + (hi[0] - lo[0]) * ur(rng);
    const float y = lo[1] + (hi[1] - lo[1]) * ur(rng);
    const float z = lo[2] + (hi[2] - lo[2]) * ur(rng);
    return mk(x, y, z);
}
// navigation_tasks.hpp:355-491: a safe world, start and goal (the world row
// `w` is regenerated in place), or an explicit failure status
__device__ uint32_t task_generate(float* w, MdnTaskState& t, uint32_t& rng, const MdnTaskConfig& c) {
    t.generation_status = MDN_TASK_INVALID_CONFIG;
    t.generation_attempts = 0;
    t.valid = 0;
    if (!task_config_valid(c)) return MDN_TASK_INVALID_CONFIG;
    const bool clutter = c.stage == MDN_TASK_STAGE_CLUTTER_GOAL;
    if (!clutter && c.family != 0u) return MDN_TASK_INVALID_CONFIG;
    if (clutter && !(c.family == 1u || c.family == 2u || c.family == 4u || c.family == 5u || c.family == 12u))
        return MDN_TASK_UNSUPPORTED_FAMILY;
    for (int k = 0; k < 3; k++) {
        const float room_min = k == 0 ? -2.0f : (k == 1 ? -5.0f : 0.0f), room_max = k == 0 ? 14.0f : 5.0f;
        const float m = c.minimum_endpoint_clearance_m;
        if (!task_fin(c.start_min_xyz[k]) || !task_fin(c.start_max_xyz[k]) || !task_fin(c.goal_min_xyz[k]) ||
            !task_fin(c.goal_max_xyz[k]) || c.start_min_xyz[k] >= c.start_max_xyz[k] ||
            c.goal_min_xyz[k] >= c.goal_max_xyz[k] || c.start_min_xyz[k] < room_min + m ||
            c.start_max_xyz[k] > room_max - m || c.goal_min_xyz[k] < room_min + m || c.goal_max_xyz[k] > room_max - m)
            return MDN_TASK_INVALID_CONFIG;
    }
    const uint32_t attempts = min(c.max_generation_attempts, MDN_TASK_MAX_ATTEMPTS);
    WorldGen wg{w};
    for (uint32_t attempt = 0; attempt < attempts; attempt++) {
        t.generation_attempts = attempt + 1;
        const uint32_t scene_seed = xs(rng);
        uint32_t family = c.family;
        if (c.family == 12u) {
            const uint32_t sel = xs(rng) % 4u;
            family = sel == 0 ? 1u : (sel == 1 ? 2u : (sel == 2 ? 4u : 5u));
        }
        wg.generate(scene_seed, family, c.scene_distance_m);
        const uint32_t count = min(wg.count(), 16u);
        if (clutter) {
            bool moving = false;
            for (uint32_t o = 0; o < count; o++)
                for (int k = 0; k < 3; k++) moving = moving || fabs_f(w[10 * o + 7 + k]) > 1e-8f;
            if (moving) {
                t.generation_status = MDN_TASK_UNSUPPORTED_DYNAMIC;
                return t.generation_status;
            }
        }
        V dir = task_direction(rng);
        const float span = c.goal_distance_max_m - c.goal_distance_min_m;
        const float center = c.goal_distance_min_m + c.difficulty * span;
        const float jitter = (ur(rng) - 0.5f) * 0.20f * span;
        const float distance = task_clamp(center + jitter, c.goal_distance_min_m, c.goal_distance_max_m);
        V start, goal;
        if (c.stage == MDN_TASK_STAGE_NEAR_GOAL_HOLD) {
            goal = task_point(rng, c.goal_min_xyz, c.goal_max_xyz);
            start = sub3(goal, mul3(dir, distance));
        } else {
            start = task_point(rng, c.start_min_xyz, c.start_max_xyz);
            goal = add3(start, mul3(dir, distance));
            if (clutter && c.generation_version >= 1u) {
                bool in = task_inside(goal, c.goal_min_xyz, c.goal_max_xyz);
                for (uint32_t k = 1; !in && k < MDN_TASK_MAX_ATTEMPTS; k++) {
                    dir = task_direction(rng);
                    goal = add3(start, mul3(dir, distance));
                    in = task_inside(goal, c.goal_min_xyz, c.goal_max_xyz);
                }
                if (!in) continue;
            }
        }
        if (!task_fin(goal.x) || !task_fin(goal.y) || !task_fin(goal.z)) continue;
        if (!task_inside(start, c.start_min_xyz, c.start_max_xyz) || !task_inside(goal, c.goal_min_xyz, c.goal_max_xyz))
            continue;
        const float start_clear = clearance_at(w, count, start, 0.0f), goal_clear = clearance_at(w, count, goal, 0.0f);
        if (start_clear <= c.minimum_endpoint_clearance_m || goal_clear <= c.minimum_endpoint_clearance_m) continue;
        const float actual = len3(sub3(goal, start));
        if (actual < c.goal_distance_min_m || actual > c.goal_distance_max_m) continue;
        TaskWitness wit;
        float direct = 0.0f;
        if (!task_witness(w, count, start, goal, c, wit, direct)) continue;
        w[163] = goal.x; w[164] = goal.y; w[165] = goal.z;
        t.family = family; t.stage = c.stage; t.objective = c.objective;
        t.max_nav_steps = c.max_nav_steps; t.step_count = 0; t.stable_ticks = 0;
        t.was_inside_goal = 0; t.waypoint_event_latched = 0; t.terminal = 0;
        t.start_position[0] = start.x; t.start_position[1] = start.y; t.start_position[2] = start.z;
        t.start_yaw_rad = (ur(rng) * 2.0f - 1.0f) * 3.14159265359f;
        const float speed = c.initial_speed_min_mps + (c.initial_speed_max_mps - c.initial_speed_min_mps) * ur(rng);
        t.start_velocity_world[0] = dir.x * speed;
        t.start_velocity_world[1] = dir.y * speed;
        t.start_velocity_world[2] = dir.z * speed;
        t.goal_position[0] = goal.x; t.goal_position[1] = goal.y; t.goal_position[2] = goal.z;
        t.initial_distance_m = actual; t.previous_distance_m = actual;
        t.difficulty = c.difficulty;
        t.start_clearance_m = start_clear; t.goal_clearance_m = goal_clear;
        t.direct_segment_clearance_m = direct;
        t.witness_min_clearance_m = wit.clearance; t.witness_length_m = wit.length;
        t.stable_time_s = 0.0f;
        for (int k = 0; k < 3; k++) t.last_executed_world_command[k] = t.start_velocity_world[k];
        t.last_executed_world_command[3] = 0.0f;
        t.witness_point_count = wit.n;
        for (uint32_t p = 0; p < 4; p++) {
            t.witness_points[p][0] = wit.p[p].x;
            t.witness_points[p][1] = wit.p[p].y;
            t.witness_points[p][2] = wit.p[p].z;
        }
        t.valid = 1;
        t.generation_status = MDN_TASK_READY;
        return t.generation_status;
    }
    t.generation_status = MDN_TASK_EXHAUSTED;
    return t.generation_status;
}

// navigation_tasks.hpp:509-548, evaluated redundantly by every lane of the
// env's group from the state in global memory; lane `writer` stores the
// updated state.  Returns the reward; sets success / timeout per
// sim.metal:307-315.
struct TaskOutcome { float reward; bool stable_success, timeout; };
__device__ __forceinline__ TaskOutcome task_step(MdnTaskState* tg, const MdnTaskConfig& c, const float* pos,
                                                 const float* vel, const float* executed, bool contact, bool forced,
                                                 bool writer) {
    TaskOutcome o = {0.0f, false, false};
    MdnTaskState t = *tg;
    if (t.generation_status != MDN_TASK_READY || t.terminal != 0u) return o;
    const float dx = t.goal_position[0] - pos[0], dy = t.goal_position[1] - pos[1], dz = t.goal_position[2] - pos[2];
    const float distance = sqrt_f(dx * dx + dy * dy + dz * dz);
    const float speed = sqrt_f(vel[0] * vel[0] + vel[1] * vel[1] + vel[2] * vel[2]);
    if (!task_fin(distance) || !task_fin(speed)) {
        if (writer) tg->terminal = 1u;
        return o;
    }
    t.step_count++;
    float reward = c.progress_reward_per_m * (t.previous_distance_m - distance) - c.time_cost_per_s * c.nav_period_s;
    t.previous_distance_m = distance;
    const bool inside = distance <= c.goal_radius_m;
    if (t.objective == MDN_TASK_OBJECTIVE_WAYPOINT && inside && t.waypoint_event_latched == 0u)
        t.waypoint_event_latched = 1u;
    const bool stable = inside && speed <= c.stable_speed_mps;
    if (t.objective == MDN_TASK_OBJECTIVE_FINAL_HOLD && stable) t.stable_time_s += c.nav_period_s;
    else t.stable_time_s = 0.0f;
    t.stable_ticks = uint32_t(__builtin_ceilf(t.stable_time_s / fmax_f(c.nav_period_s, 1e-6f) - 1e-5f));
    o.stable_success = t.objective == MDN_TASK_OBJECTIVE_FINAL_HOLD && stable && t.stable_time_s + 1e-6f >= c.stable_hold_s;
    o.timeout = forced || t.step_count >= t.max_nav_steps;
    if (c.command_smoothness_weight > 0.0f) {
        float diff = 0.0f;
        for (int k = 0; k < 4; k++) {
            const float d = executed[k] - t.last_executed_world_command[k];
            diff += d * d;
            t.last_executed_world_command[k] = executed[k];
        }
        reward -= c.command_smoothness_weight * diff * c.nav_period_s;
    }
    if (contact) reward -= c.contact_penalty;
    if (o.stable_success && !contact) reward += c.stable_arrival_bonus;
    t.terminal = (contact || o.stable_success || o.timeout) ? 1u : 0u;
    o.reward = reward;
    if (writer) *tg = t;
    return o;
}

}  // namespace nav
