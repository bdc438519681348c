/*
 * oracle_tasks.h — CPU oracle, part 3: episode dynamics variation and
 * goal-conditioned navigation tasks.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker for the HIP path: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * It restates, in plain scalar C++, the reference functions cited on each
 * definition (physics_domain.hpp, navigation_tasks.hpp and the Metal seed
 * hashes of sim.metal); paths are relative to the reference repository.
 * Several RNG draws inside one argument list are sequenced left to right, as
 * for the world generator.
 */
#ifndef MDNAV_ORACLE_TASKS_H
#define MDNAV_ORACLE_TASKS_H

#include <cmath>
#include <cstdint>
#include <cstring>

#include "oracle_world.h"

namespace orc {

// ---- episode dynamics: physics_domain.hpp --------------------------------
struct DomainSample {
    float mass_scale, inertia_axis_scale[3], thrust_gain[4], rising_lag_scale[4], falling_lag_scale[4];
    float thrust_to_weight;
};
// physics_domain.hpp:37-40
inline MdnDomainRange domain_stress_range() {
    return {0.90f, 1.10f, 0.90f, 1.10f, 0.90f, 1.10f, 0.75f, 1.35f, 0.75f, 1.35f, 1.15f};
}
// physics_domain.hpp:42-47 (xorshift 13/17/5 that never yields or keeps 0)
inline uint32_t domain_next(uint32_t& state) {
    uint32_t v = state ? state : 1u;
    v ^= v << 13; v ^= v >> 17; v ^= v << 5;
    state = v ? v : 1u;
    return state;
}
// physics_domain.hpp:49-57
inline float domain_uniform(uint32_t& state) { return float(domain_next(state) >> 8) * (1.0f / 16777216.0f); }
inline float domain_scale(uint32_t& state, float low, float high, float amplitude) {
    const float draw = low + (high - low) * domain_uniform(state);
    return 1.0f + amplitude * (draw - 1.0f);
}
// physics_domain.hpp:59-80 (symmetric positive-definite 3x3 inverse by cofactors)
inline bool domain_inverse3(const float* m, float* inv) {
    for (int j = 0; j < 9; j++) if (!isfinite_f(m[j])) return false;
    const float a = m[0], b = m[1], c = m[2], d = m[3], e = m[4], f = m[5], g = m[6], h = m[7], i = m[8];
    if (fabs_f(b - d) > 1.0e-6f || fabs_f(c - g) > 1.0e-6f || fabs_f(f - h) > 1.0e-6f) return false;
    const float minor2 = a * e - b * d;
    const float det = a * (e * i - f * h) - b * (d * i - f * g) + c * (d * h - e * g);
    if (!(a > 0.0f) || !(minor2 > 0.0f) || !(det > 0.0f) || !isfinite_f(det)) return false;
    const float r = 1.0f / det;
    inv[0] = (e * i - f * h) * r; inv[1] = (c * h - b * i) * r; inv[2] = (b * f - c * e) * r;
    inv[3] = (f * g - d * i) * r; inv[4] = (a * i - c * g) * r; inv[5] = (c * d - a * f) * r;
    inv[6] = (d * h - e * g) * r; inv[7] = (b * g - a * h) * r; inv[8] = (a * e - b * d) * r;
    for (int j = 0; j < 9; j++) if (!isfinite_f(inv[j])) return false;
    return true;
}
// physics_domain.hpp:82-93 — vertical thrust at full action over the weight
inline float domain_thrust_to_weight(const MdnPhysicsParams& p) {
    float lift = 0.0f;
    const float u = p.action_max;
    for (int r = 0; r < 4; r++) {
        const float* c = &p.rotor_thrust_coefficients[3 * r];
        lift += p.rotor_thrust_directions[3 * r + 2] * (c[0] + c[1] * u + c[2] * u * u);
    }
    const float weight = p.mass * fabs_f(p.gravity_world[2]);
    return weight > 0.0f ? lift / weight : 0.0f;
}
inline bool range_ok(float lo, float hi) { return isfinite_f(lo) && isfinite_f(hi) && lo > 0.0f && lo <= hi; }
// physics_domain.hpp:98-155
inline bool sample_domain(const MdnPhysicsParams& nominal, uint32_t& rng, float amplitude, const MdnDomainRange& R,
                          MdnPhysicsParams& varied, DomainSample& s) {
    if (!isfinite_f(amplitude) || amplitude < 0.0f || amplitude > 1.0f || !isfinite_f(R.minimum_thrust_to_weight) ||
        R.minimum_thrust_to_weight < 1.0f || !range_ok(R.mass_scale_min, R.mass_scale_max) ||
        !range_ok(R.inertia_axis_scale_min, R.inertia_axis_scale_max) || !range_ok(R.thrust_gain_min, R.thrust_gain_max) ||
        !range_ok(R.rising_lag_scale_min, R.rising_lag_scale_max) ||
        !range_ok(R.falling_lag_scale_min, R.falling_lag_scale_max))
        return false;
    varied = nominal;
    s.mass_scale = 1.0f;
    s.thrust_to_weight = 0.0f;
    for (int k = 0; k < 3; k++) s.inertia_axis_scale[k] = 1.0f;
    for (int r = 0; r < 4; r++) s.thrust_gain[r] = s.rising_lag_scale[r] = s.falling_lag_scale[r] = 1.0f;
    if (amplitude > 0.0f) {
        s.mass_scale = domain_scale(rng, R.mass_scale_min, R.mass_scale_max, amplitude);
        for (int k = 0; k < 3; k++)
            s.inertia_axis_scale[k] = domain_scale(rng, R.inertia_axis_scale_min, R.inertia_axis_scale_max, amplitude);
        for (int r = 0; r < 4; r++) {
            s.thrust_gain[r] = domain_scale(rng, R.thrust_gain_min, R.thrust_gain_max, amplitude);
            s.rising_lag_scale[r] = domain_scale(rng, R.rising_lag_scale_min, R.rising_lag_scale_max, amplitude);
            s.falling_lag_scale[r] = domain_scale(rng, R.falling_lag_scale_min, R.falling_lag_scale_max, amplitude);
        }
        varied.mass = nominal.mass * s.mass_scale;
        float root[3];
        for (int k = 0; k < 3; k++) root[k] = sqrt_f(s.inertia_axis_scale[k]);
        for (int row = 0; row < 3; row++)
            for (int col = 0; col < 3; col++)
                varied.inertia[3 * row + col] = nominal.inertia[3 * row + col] * s.mass_scale * root[row] * root[col];
        if (!domain_inverse3(varied.inertia, varied.inertia_inverse)) return false;
        for (int r = 0; r < 4; r++) {
            for (int c = 0; c < 3; c++)
                varied.rotor_thrust_coefficients[3 * r + c] = nominal.rotor_thrust_coefficients[3 * r + c] * s.thrust_gain[r];
            varied.rotor_time_constants_rising[r] = nominal.rotor_time_constants_rising[r] * s.rising_lag_scale[r];
            varied.rotor_time_constants_falling[r] = nominal.rotor_time_constants_falling[r] * s.falling_lag_scale[r];
        }
    }
    s.thrust_to_weight = domain_thrust_to_weight(varied);
    return s.thrust_to_weight >= R.minimum_thrust_to_weight;
}
// sim.metal:50-54 — per-env, per-episode seed of the dynamics draw
inline uint32_t domain_episode_seed(const MdnRuntimeConfig& rt, uint32_t cfg_seed, uint32_t env, uint32_t episode) {
    uint32_t h = rt.domain_seed ^ cfg_seed ^ ((env + 1u) * 0x9e3779b9u) ^ ((episode + 1u) * 0x85ebca6bu);
    h ^= h >> 16; h *= 0x7feb352du; h ^= h >> 15; h *= 0x846ca68bu; h ^= h >> 16;
    return h ? h : 1u;
}
// sim.metal:62-69 — the episode's plant: the nominal one, or a draw (a
// rejected draw keeps the nominal plant with a NaN mass, which the host's
// validation reports)
inline MdnPhysicsParams episode_params(const MdnRuntimeConfig& rt, const MdnPhysicsParams& p, uint32_t cfg_seed,
                                       uint32_t env, uint32_t episode) {
    MdnPhysicsParams out = p;
    if (rt.enabled != 0 && rt.domain_amplitude > 0.0f) {
        uint32_t rng = domain_episode_seed(rt, cfg_seed, env, episode);
        MdnPhysicsParams varied;
        DomainSample s;
        if (sample_domain(p, rng, rt.domain_amplitude, rt.domain_range, varied, s)) out = varied;
        else out.mass = nan_f();
    }
    return out;
}
// sim.metal:70-81 — hover rpm: one root for the nominal plant, one per rotor
// (full action where the discriminant is negative) for per-episode plants
inline void hover_rpm(const MdnRuntimeConfig& rt, const MdnPhysicsParams& p, const MdnPhysicsParams& ep, float out[4]) {
    if (rt.enabled == 0) {
        const float target = p.mass * 9.81f / 4;
        const float c0 = p.rotor_thrust_coefficients[0], c1 = p.rotor_thrust_coefficients[1],
                    c2 = p.rotor_thrust_coefficients[2];
        const float h = clamp_f((-c1 + sqrt_f(c1 * c1 - 4 * c2 * (c0 - target))) / (2 * c2), p.action_min, p.action_max);
        for (int r = 0; r < 4; r++) out[r] = h;
        return;
    }
    const float target = ep.mass * 9.81f / 4;
    for (int r = 0; r < 4; r++) {
        const float c0 = ep.rotor_thrust_coefficients[3 * r], c1 = ep.rotor_thrust_coefficients[3 * r + 1],
                    c2 = ep.rotor_thrust_coefficients[3 * r + 2];
        const float disc = c1 * c1 - 4 * c2 * (c0 - target);
        out[r] = disc >= 0.0f ? clamp_f((-c1 + sqrt_f(disc)) / (2 * c2), ep.action_min, ep.action_max) : ep.action_max;
    }
}

// ---- navigation tasks: navigation_tasks.hpp ------------------------------
// navigation_tasks.hpp:99-140
inline bool task_default_config(MdnTaskConfig& c, uint32_t stage, uint32_t family, float difficulty) {
    if (stage > MDN_TASK_STAGE_CLUTTER_GOAL || !isfinite_f(difficulty) || difficulty < 0.0f || difficulty > 1.0f)
        return false;
    if (stage == MDN_TASK_STAGE_OPEN_GOAL || stage == MDN_TASK_STAGE_NEAR_GOAL_HOLD) {
        if (family != 0u) return false;
    } else if (!(family == 1u || family == 2u || family == 4u || family == 5u || family == 12u)) {
        return false;
    }
    std::memset(&c, 0, sizeof(c));
    c.generation_version = 1; c.family = family; c.stage = stage; c.objective = MDN_TASK_OBJECTIVE_FINAL_HOLD;
    c.require_detour = 0; c.max_generation_attempts = MDN_TASK_MAX_ATTEMPTS;
    c.max_nav_steps = 400; c.scene_distance_m = 8.0f; c.difficulty = difficulty;
    c.minimum_endpoint_clearance_m = 0.30f; c.minimum_witness_clearance_m = 0.02f;
    c.goal_radius_m = 0.35f; c.stable_speed_mps = 0.50f; c.stable_hold_s = 0.20f;
    c.nav_period_s = 0.05f; c.initial_speed_min_mps = 0.0f; c.initial_speed_max_mps = 0.0f;
    c.progress_reward_per_m = 2.0f; c.time_cost_per_s = 0.20f;
    c.contact_penalty = 10.0f; c.stable_arrival_bonus = 10.0f; c.command_smoothness_weight = 0.05f;
    const float slo[3] = {-1.0f, -2.0f, 0.8f}, shi[3] = {1.0f, 2.0f, 2.4f};
    const float glo[3] = {-1.2f, -4.0f, 0.5f}, ghi[3] = {13.2f, 4.0f, 4.5f};
    for (int k = 0; k < 3; k++) {
        c.start_min_xyz[k] = slo[k]; c.start_max_xyz[k] = shi[k];
        c.goal_min_xyz[k] = glo[k]; c.goal_max_xyz[k] = ghi[k];
    }
    if (stage == MDN_TASK_STAGE_NEAR_GOAL_HOLD) {
        c.goal_distance_min_m = 0.8f; c.goal_distance_max_m = 2.0f;
        for (int k = 0; k < 3; k++) { c.start_min_xyz[k] = glo[k]; c.start_max_xyz[k] = ghi[k]; }
    } else if (stage == MDN_TASK_STAGE_CLUTTER_GOAL) {
        c.goal_distance_min_m = 2.0f; c.goal_distance_max_m = 7.0f;
    } else {
        c.goal_distance_min_m = 2.0f; c.goal_distance_max_m = 6.0f;
    }
    return true;
}
// navigation_training.hpp:7-14 — the training and evaluation task settings
inline MdnTaskControl task_settings(uint32_t stage, uint32_t family, bool& ok) {
    MdnTaskControl t;
    std::memset(&t, 0, sizeof(t));
    t.enabled = 1;
    ok = task_default_config(t.config, stage, family, .5f);
    t.config.time_cost_per_s = .2f;
    t.config.command_smoothness_weight = .05f;
    t.config.initial_speed_max_mps = stage == 1 ? .5f : 1.0f;
    return t;
}

inline float task_clamp(float v, float lo, float hi) { return fmin_f(fmax_f(v, lo), hi); }
// navigation_tasks.hpp:213-218
inline V3 task_random_direction(uint32_t& rng) {
    const float z = 2.0f * urand(rng) - 1.0f;
    const float angle = 6.28318530718f * urand(rng);
    const float radial = sqrt_f(fmax_f(0.0f, 1.0f - z * z));
    float s, c;
    sincos_f(angle, &s, &c);
    return v3(radial * c, radial * s, z);
}
// navigation_tasks.hpp:220-224
inline V3 task_random_point(uint32_t& rng, const float* lo, const float* hi) {
    const float x = lo[0] + (hi[0] - lo[0]) * urand(rng);
    const float y = lo[1] + (hi[1] - lo[1]) * urand(rng);
    const float z = lo[2] + (hi[2] - lo[2]) * urand(rng);
    return v3(x, y, z);
}
// navigation_tasks.hpp:231-234
inline bool task_inside(V3 p, const float* lo, const float* hi) {
    return p.x >= lo[0] && p.x <= hi[0] && p.y >= lo[1] && p.y <= hi[1] && p.z >= lo[2] && p.z <= hi[2];
}
// navigation_tasks.hpp:236-241
inline float task_goal_distance(uint32_t& rng, const MdnTaskConfig& c) {
    const float span = c.goal_distance_max_m - c.goal_distance_min_m;
    const float center = c.goal_distance_min_m + c.difficulty * span;
    const float jitter = (urand(rng) - 0.5f) * 0.20f * span;
    return task_clamp(center + jitter, c.goal_distance_min_m, c.goal_distance_max_m);
}
// navigation_tasks.hpp:243-255 — clearance along a segment sampled every
// 5 cm or closer (static scene, time 0)
inline float task_segment_clearance(const MdnWorld& w, V3 a, V3 b) {
    const float distance = vlen(vsub(b, a));
    uint32_t count = uint32_t(std::ceil(distance / 0.05f));
    if (count < 1u) count = 1u;
    if (count > 512u) return -1e6f;
    float minimum = 1e20f;
    for (uint32_t k = 0; k <= count; k++) {
        const float t = float(k) / float(count);
        minimum = fmin_f(minimum, clearance(w, vadd(a, vmul(vsub(b, a), t)), 0.0f));
    }
    return minimum;
}
// navigation_tasks.hpp:257-263
inline float task_test_path(const MdnWorld& w, const V3* p, uint32_t count) {
    if (count < 2u || count > MDN_TASK_MAX_WITNESS_POINTS) return -1e6f;
    float minimum = 1e20f;
    for (uint32_t s = 0; s + 1u < count; s++) minimum = fmin_f(minimum, task_segment_clearance(w, p[s], p[s + 1]));
    return minimum;
}
struct Witness { V3 points[4]; uint32_t count; float min_clearance, length; };
// navigation_tasks.hpp:265-277
inline void task_save_witness(Witness& out, const V3* p, uint32_t count, float clearance_m) {
    out.count = count;
    out.min_clearance = clearance_m;
    float total = 0;
    for (uint32_t s = 0; s + 1u < count; s++) total += vlen(vsub(p[s + 1], p[s]));
    out.length = total;
    for (uint32_t i = 0; i < 4; i++) out.points[i] = i < count ? p[i] : v3(0, 0, 0);
}
// navigation_tasks.hpp:281-345 — the direct line, else the first clear
// dogleg of a fixed list
inline bool task_find_witness(const MdnWorld& w, V3 start, V3 goal, const MdnTaskConfig& c, Witness& out,
                              float& direct) {
    const float thr = c.minimum_witness_clearance_m;
    const V3 line[2] = {start, goal};
    direct = task_test_path(w, line, 2);
    if (direct > thr && c.require_detour == 0u) { task_save_witness(out, line, 2, direct); return true; }
    if (direct > thr) return false;
    const V3 delta = vsub(goal, start);
    auto try3 = [&](V3 mid) {
        const V3 path[3] = {start, mid, goal};
        const float cl = task_test_path(w, path, 3);
        if (cl > thr) { task_save_witness(out, path, 3, cl); return true; }
        return false;
    };
    const float xf[5] = {0.10f, 0.25f, 0.50f, 0.75f, 0.90f};
    const float side_y[2] = {-4.60f, 4.60f};
    for (int side = 0; side < 2; side++)
        for (int i = 0; i < 5; i++)
            if (try3(v3(start.x + xf[i] * delta.x, side_y[side], start.z + xf[i] * delta.z))) return true;
    const float off[4] = {-2.4f, -1.2f, 1.2f, 2.4f};
    for (int i = 0; i < 4; i++)
        if (try3(v3(start.x + 0.5f * delta.x, task_clamp((start.y + goal.y) * 0.5f + off[i], -4.60f, 4.60f),
                    start.z + 0.5f * delta.z)))
            return true;
    const float dz[2] = {0.55f, 4.45f};
    for (int i = 0; i < 2; i++)
        if (try3(v3(start.x + 0.5f * delta.x, start.y + 0.5f * delta.y, dz[i]))) return true;
    for (int side = 0; side < 2; side++) {
        const float y = side_y[side];
        const V3 path[4] = {start, v3(start.x + 0.20f * delta.x, y, start.z + 0.20f * delta.z),
                            v3(start.x + 0.80f * delta.x, y, start.z + 0.80f * delta.z), goal};
        const float cl = task_test_path(w, path, 4);
        if (cl > thr) { task_save_witness(out, path, 4, cl); return true; }
    }
    return false;
}
// navigation_tasks.hpp:347-351
inline bool task_static_world(const MdnWorld& w) {
    for (uint32_t o = 0; o < w.count; o++)
        for (int k = 0; k < 3; k++)
            if (fabs_f(w.obstacles[o].velocity[k]) > 1e-8f) return false;
    return true;
}
inline bool fin(float x) { return isfinite_f(x); }
// navigation_tasks.hpp:355-388 — configuration checks of the generator.
// Version 0 is also accepted: the generator before the clutter goals were
// conditioned on the goal bounds (navigation_tasks.hpp:435-446 absent), the
// one that produced the reference's published goal-arrival evaluations
// (evidence/inputs/arrival-training, whose manifest records that older
// source); the reference's current header accepts version 1 only.
inline bool task_config_valid(const MdnTaskConfig& c) {
    return !(c.generation_version > 1u || c.stage > MDN_TASK_STAGE_CLUTTER_GOAL ||
             c.objective > MDN_TASK_OBJECTIVE_FINAL_HOLD || c.family > 16u || c.require_detour > 1u ||
             !fin(c.scene_distance_m) || c.scene_distance_m < 3.0f || c.scene_distance_m > 10.0f ||
             !fin(c.difficulty) || c.difficulty < 0.0f || c.difficulty > 1.0f || !fin(c.goal_distance_min_m) ||
             !fin(c.goal_distance_max_m) || c.goal_distance_min_m <= c.goal_radius_m ||
             c.goal_distance_max_m < c.goal_distance_min_m || !fin(c.minimum_endpoint_clearance_m) ||
             c.minimum_endpoint_clearance_m < 0.30f || !fin(c.minimum_witness_clearance_m) ||
             c.minimum_witness_clearance_m < 0.02f || !fin(c.goal_radius_m) || c.goal_radius_m <= 0.0f ||
             !fin(c.stable_speed_mps) || c.stable_speed_mps < 0.0f || !fin(c.stable_hold_s) || c.stable_hold_s < 0.0f ||
             !fin(c.nav_period_s) || c.nav_period_s <= 0.0f || !fin(c.initial_speed_min_mps) ||
             !fin(c.initial_speed_max_mps) || c.initial_speed_min_mps < 0.0f ||
             c.initial_speed_max_mps < c.initial_speed_min_mps || !fin(c.progress_reward_per_m) ||
             c.progress_reward_per_m < 0.0f || !fin(c.time_cost_per_s) || c.time_cost_per_s < 0.0f ||
             !fin(c.contact_penalty) || c.contact_penalty < 0.0f || !fin(c.stable_arrival_bonus) ||
             c.stable_arrival_bonus < 0.0f || !fin(c.command_smoothness_weight) || c.command_smoothness_weight < 0.0f ||
             c.max_nav_steps == 0u || c.max_generation_attempts == 0u);
}
// navigation_tasks.hpp:355-491
inline uint32_t generate_task(MdnWorld& w, MdnTaskState& t, uint32_t& rng, const MdnTaskConfig& c) {
    t.generation_status = MDN_TASK_INVALID_CONFIG;
    t.generation_attempts = 0;
    t.valid = 0;
    if (!task_config_valid(c)) return MDN_TASK_INVALID_CONFIG;
    if ((c.stage == MDN_TASK_STAGE_OPEN_GOAL || c.stage == MDN_TASK_STAGE_NEAR_GOAL_HOLD) && c.family != 0u)
        return MDN_TASK_INVALID_CONFIG;
    if (c.stage == MDN_TASK_STAGE_CLUTTER_GOAL &&
        !(c.family == 1u || c.family == 2u || c.family == 4u || c.family == 5u || c.family == 12u))
        return MDN_TASK_UNSUPPORTED_FAMILY;
    for (int k = 0; k < 3; k++) {
        const float room_min = k == 0 ? -2.0f : (k == 1 ? -5.0f : 0.0f);
        const float room_max = k == 0 ? 14.0f : 5.0f;
        const float m = c.minimum_endpoint_clearance_m;
        if (!fin(c.start_min_xyz[k]) || !fin(c.start_max_xyz[k]) || !fin(c.goal_min_xyz[k]) ||
            !fin(c.goal_max_xyz[k]) || c.start_min_xyz[k] >= c.start_max_xyz[k] ||
            c.goal_min_xyz[k] >= c.goal_max_xyz[k] || c.start_min_xyz[k] < room_min + m ||
            c.start_max_xyz[k] > room_max - m || c.goal_min_xyz[k] < room_min + m || c.goal_max_xyz[k] > room_max - m)
            return MDN_TASK_INVALID_CONFIG;
    }
    const uint32_t attempts = c.max_generation_attempts < MDN_TASK_MAX_ATTEMPTS ? c.max_generation_attempts
                                                                                : MDN_TASK_MAX_ATTEMPTS;
    for (uint32_t attempt = 0; attempt < attempts; attempt++) {
        t.generation_attempts = attempt + 1;
        const uint32_t scene_seed = xorshift(rng);
        uint32_t family = c.family;
        if (c.family == 12u) {
            const uint32_t sel = xorshift(rng) % 4u;
            family = sel == 0 ? 1u : (sel == 1 ? 2u : (sel == 2 ? 4u : 5u));
        }
        generate_world(w, scene_seed, family, c.scene_distance_m);
        if (c.stage == MDN_TASK_STAGE_CLUTTER_GOAL && !task_static_world(w)) {
            t.generation_status = MDN_TASK_UNSUPPORTED_DYNAMIC;
            return t.generation_status;
        }
        V3 dir = task_random_direction(rng);
        const float distance = task_goal_distance(rng, c);
        V3 start, goal;
        if (c.stage == MDN_TASK_STAGE_NEAR_GOAL_HOLD) {
            goal = task_random_point(rng, c.goal_min_xyz, c.goal_max_xyz);
            start = vsub(goal, vmul(dir, distance));
        } else {
            start = task_random_point(rng, c.start_min_xyz, c.start_max_xyz);
            goal = vadd(start, vmul(dir, distance));
            if (c.stage == MDN_TASK_STAGE_CLUTTER_GOAL && c.generation_version >= 1u) {
                bool in = task_inside(goal, c.goal_min_xyz, c.goal_max_xyz);
                for (uint32_t k = 1; !in && k < MDN_TASK_MAX_ATTEMPTS; k++) {
                    dir = task_random_direction(rng);
                    goal = vadd(start, vmul(dir, distance));
                    in = task_inside(goal, c.goal_min_xyz, c.goal_max_xyz);
                }
                if (!in) continue;
            }
        }
        if (!fin(goal.x) || !fin(goal.y) || !fin(goal.z)) continue;
        if (!task_inside(start, c.start_min_xyz, c.start_max_xyz) || !task_inside(goal, c.goal_min_xyz, c.goal_max_xyz))
            continue;
        const float start_clear = clearance(w, start, 0.0f), goal_clear = clearance(w, goal, 0.0f);
        if (start_clear <= c.minimum_endpoint_clearance_m || goal_clear <= c.minimum_endpoint_clearance_m) continue;
        const float actual = vlen(vsub(goal, start));
        if (actual < c.goal_distance_min_m || actual > c.goal_distance_max_m) continue;
        Witness wit;
        std::memset(&wit, 0, sizeof(wit));
        float direct = 0.0f;
        if (!task_find_witness(w, start, goal, c, wit, direct)) continue;
        w.goal[0] = goal.x; w.goal[1] = goal.y; w.goal[2] = goal.z;
        t.family = family; t.stage = c.stage; t.objective = c.objective;
        t.max_nav_steps = c.max_nav_steps; t.step_count = 0; t.stable_ticks = 0;
        t.was_inside_goal = 0; t.waypoint_event_latched = 0; t.terminal = 0;
        t.start_position[0] = start.x; t.start_position[1] = start.y; t.start_position[2] = start.z;
        t.start_yaw_rad = (urand(rng) * 2.0f - 1.0f) * 3.14159265359f;
        const float speed = c.initial_speed_min_mps + (c.initial_speed_max_mps - c.initial_speed_min_mps) * urand(rng);
        t.start_velocity_world[0] = dir.x * speed;
        t.start_velocity_world[1] = dir.y * speed;
        t.start_velocity_world[2] = dir.z * speed;
        t.goal_position[0] = goal.x; t.goal_position[1] = goal.y; t.goal_position[2] = goal.z;
        t.initial_distance_m = actual; t.previous_distance_m = actual;
        t.difficulty = c.difficulty;
        t.start_clearance_m = start_clear; t.goal_clearance_m = goal_clear;
        t.direct_segment_clearance_m = direct;
        t.witness_min_clearance_m = wit.min_clearance; t.witness_length_m = wit.length;
        t.stable_time_s = 0.0f;
        for (int k = 0; k < 3; k++) t.last_executed_world_command[k] = t.start_velocity_world[k];
        t.last_executed_world_command[3] = 0.0f;
        t.witness_point_count = wit.count;
        for (uint32_t p = 0; p < 4; p++) {
            t.witness_points[p][0] = p < wit.count ? wit.points[p].x : 0.0f;
            t.witness_points[p][1] = p < wit.count ? wit.points[p].y : 0.0f;
            t.witness_points[p][2] = p < wit.count ? wit.points[p].z : 0.0f;
        }
        t.valid = 1;
        t.generation_status = MDN_TASK_READY;
        return t.generation_status;
    }
    t.generation_status = MDN_TASK_EXHAUSTED;
    return t.generation_status;
}
// navigation_tasks.hpp:495-505 — physical start state only
inline void task_apply_start(const MdnTaskState& t, MdnPhysicsState& s) {
    for (int k = 0; k < 3; k++) {
        s.position[k] = t.start_position[k];
        s.linear_velocity[k] = t.start_velocity_world[k];
        s.angular_velocity_body[k] = 0.0f;
    }
    float sh, ch;
    sincos_f(t.start_yaw_rad * 0.5f, &sh, &ch);
    s.orientation_wxyz[0] = ch; s.orientation_wxyz[1] = 0.0f; s.orientation_wxyz[2] = 0.0f; s.orientation_wxyz[3] = sh;
}
struct TaskStep { float reward, goal_distance, speed; uint32_t waypoint_passed, stable_success, collision, timeout, done; };
// navigation_tasks.hpp:509-548
inline TaskStep task_step(MdnTaskState& t, const MdnTaskConfig& c, const float* pos, const float* vel,
                          const float* executed, uint32_t contact, uint32_t forced_timeout) {
    TaskStep r;
    std::memset(&r, 0, sizeof(r));
    if (t.generation_status != MDN_TASK_READY || t.terminal != 0u) { r.done = 1; return r; }
    const float dx = t.goal_position[0] - pos[0], dy = t.goal_position[1] - pos[1], dz = t.goal_position[2] - pos[2];
    const float distance = sqrt_f(dx * dx + dy * dy + dz * dz);
    const float speed = sqrt_f(vel[0] * vel[0] + vel[1] * vel[1] + vel[2] * vel[2]);
    if (!fin(distance) || !fin(speed)) { r.collision = 1; r.done = 1; t.terminal = 1; return r; }
    t.step_count++;
    r.goal_distance = distance; r.speed = speed;
    const float progress = t.previous_distance_m - distance;
    r.reward = c.progress_reward_per_m * progress - c.time_cost_per_s * c.nav_period_s;
    t.previous_distance_m = distance;
    const uint32_t inside = distance <= c.goal_radius_m ? 1u : 0u;
    r.waypoint_passed = (t.objective == MDN_TASK_OBJECTIVE_WAYPOINT && inside && t.waypoint_event_latched == 0u) ? 1u : 0u;
    if (r.waypoint_passed) t.waypoint_event_latched = 1;
    const uint32_t stable = (inside && speed <= c.stable_speed_mps) ? 1u : 0u;
    if (t.objective == MDN_TASK_OBJECTIVE_FINAL_HOLD && stable) t.stable_time_s += c.nav_period_s;
    else t.stable_time_s = 0.0f;
    t.stable_ticks = uint32_t(std::ceil(t.stable_time_s / fmax_f(c.nav_period_s, 1e-6f) - 1e-5f));
    r.stable_success =
        (t.objective == MDN_TASK_OBJECTIVE_FINAL_HOLD && stable && t.stable_time_s + 1e-6f >= c.stable_hold_s) ? 1u : 0u;
    r.collision = contact ? 1u : 0u;
    r.timeout = (forced_timeout || t.step_count >= t.max_nav_steps) ? 1u : 0u;
    if (c.command_smoothness_weight > 0.0f) {
        float diff = 0.0f;
        for (int k = 0; k < 4; k++) {
            const float d = executed[k] - t.last_executed_world_command[k];
            diff += d * d;
            t.last_executed_world_command[k] = executed[k];
        }
        r.reward -= c.command_smoothness_weight * diff * c.nav_period_s;
    }
    if (r.collision) r.reward -= c.contact_penalty;
    if (r.stable_success && !r.collision) r.reward += c.stable_arrival_bonus;
    r.done = (r.collision || r.stable_success || r.timeout) ? 1u : 0u;
    t.terminal = r.done;
    return r;
}
// sim.metal:122-141 — new task for an env after its reset: world, start
// state, yaw, reference point, desired velocity, initial distance, wind
inline void reset_task(const MdnTaskControl& tc, uint32_t cfg_seed, float wind, uint32_t env, MdnPhysicsState& s,
                       MdnSimRun& run, MdnWorld& w, MdnTaskState& t) {
    std::memset(&t, 0, sizeof(t));
    if (tc.enabled == 0) return;
    uint32_t rng = cfg_seed ^ ((env + 1u) * 0x27d4eb2du) ^ ((run.episodes + 1u) * 0x165667b1u);
    generate_task(w, t, rng, tc.config);
    if (t.valid == 0) return;
    task_apply_start(t, s);
    run.yaw = t.start_yaw_rad;
    run.initial_distance = t.initial_distance_m;
    for (int k = 0; k < 3; k++) {
        run.reference_position[k] = s.position[k];
        run.desired_velocity[k] = s.linear_velocity[k];
    }
    w.wind[0] = wind; w.wind[1] = 0; w.wind[2] = 0;
}

}  // namespace orc

#endif  // MDNAV_ORACLE_TASKS_H
