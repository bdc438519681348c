/*
 * mdnav_host.h — host-side definitions that both the HIP library and the CPU
 * oracle must agree on bit for bit: default plant parameters, the policy
 * initialisation stream, and the minibatch order of a PPO update.
 * Header-only C++17; no GPU code.
 */
#ifndef MDNAV_HOST_H
#define MDNAV_HOST_H

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "mdnav_math.h"
#include "mdnav_plant.h"
#include "mdnav_types.h"

namespace mdn {

// Layout of the flat actor/critic parameter vectors (ppo.hpp:35-45): actor
// W1[hidden][obs] @0, b1, W2[4][hidden], b2, log_std[4]; critic W1[hidden][32],
// b1, w2[hidden], b2.
struct PolicyShape {
    uint32_t obs = MDN_ACTOR_OBS_POOLED;
    uint32_t hidden = MDN_HIDDEN;
    uint32_t critic_obs = MDN_CRITIC_OBS;
    uint32_t critic_hidden = MDN_HIDDEN;
    uint32_t actor_b1() const { return hidden * obs; }
    uint32_t actor_w2() const { return actor_b1() + hidden; }
    uint32_t actor_b2() const { return actor_w2() + MDN_ACTIONS * hidden; }
    uint32_t actor_log_std() const { return actor_b2() + MDN_ACTIONS; }
    uint32_t actor_count() const { return actor_log_std() + MDN_ACTIONS; }
    uint32_t critic_b1() const { return critic_hidden * critic_obs; }
    uint32_t critic_w2() const { return critic_b1() + critic_hidden; }
    uint32_t critic_b2() const { return critic_w2() + critic_hidden; }
    uint32_t critic_count() const { return critic_b2() + 1; }
};

// xorshift32 (13,17,5) and its 24-bit uniform (world.hpp:30-31).
MDN_HD uint32_t xorshift(uint32_t& s) { s ^= s << 13; s ^= s >> 17; s ^= s << 5; return s; }
MDN_HD float urand(uint32_t& s) { return float(xorshift(s) >> 8) * (1.0f / 16777216.0f); }

// L2F Crazyflie profile (physics.hpp:184-219).
inline MdnPhysicsParams crazyflie_params() { return crazyflie_profile(); }

// Whether a plant has the standard quadrotor structure the device's
// specialised derivative assumes: thrust directions (0, 0, 1), torque
// directions (0, 0, +-1), rotors in the z = 0 plane, diagonal inertia and
// inverse, gravity along z (zeros as +0.0 bit patterns).
inline bool quad_structure(const MdnPhysicsParams& p) {
    auto bits = [](float x) { uint32_t u; std::memcpy(&u, &x, 4); return u; };
    bool ok = true;
    for (int r = 0; r < 4; ++r) {
        ok = ok && bits(p.rotor_thrust_directions[3 * r]) == 0u && bits(p.rotor_thrust_directions[3 * r + 1]) == 0u &&
             bits(p.rotor_thrust_directions[3 * r + 2]) == bits(1.0f);
        ok = ok && bits(p.rotor_torque_directions[3 * r]) == 0u && bits(p.rotor_torque_directions[3 * r + 1]) == 0u &&
             (bits(p.rotor_torque_directions[3 * r + 2]) == bits(1.0f) ||
              bits(p.rotor_torque_directions[3 * r + 2]) == bits(-1.0f));
        ok = ok && bits(p.rotor_positions[3 * r + 2]) == 0u;
    }
    for (int i = 0; i < 9; ++i)
        if (i % 4 != 0) ok = ok && bits(p.inertia[i]) == 0u && bits(p.inertia_inverse[i]) == 0u;
    return ok && bits(p.gravity_world[0]) == 0u && bits(p.gravity_world[1]) == 0u;
}

// Default run configuration of main.mm:461-464.
inline MdnSimConfig default_config() {
    MdnSimConfig c;
    std::memset(&c, 0, sizeof(c));
    c.n = 128; c.tick = 0; c.mode = 0; c.family = 0; c.substeps = 5; c.sensor_period = 1;
    c.sensor_delay = 0; c.command_delay = 0; c.max_steps = 200; c.seed = 42; c.eval = 0;
    c.speed = 2; c.distance = 4; c.wind = 0; c.depth_noise = 0; c.dropout = 0; c.risk_coef = 0;
    c.entropy_coef = .005f; c.learning_rate = .0003f; c.velocity_contract = 1; c.geometry_memory = 0;
    return c;
}

// Policy initialisation (cpu_reference.hpp:89-103 == main.mm:548-554): seed
// 1789 xorshift Box–Muller; actor W1*0.04, W2*0.01, log_std=-1; critic
// W1*0.15, w2*0.1; biases zero.
inline void init_policy(const PolicyShape& s, float* actor, float* critic) {
    std::fill(actor, actor + s.actor_count(), 0.0f);
    std::fill(critic, critic + s.critic_count(), 0.0f);
    uint32_t seed = 1789;
    auto normal = [&]() {
        const float u = max_f(urand(seed), 1.0e-7f);
        const float lu = log_f(u);
        const float v = urand(seed);
        return sqrt_f(-2.0f * lu) * cos_f(6.2831853f * v);
    };
    for (uint32_t i = 0; i < s.actor_b1(); i++) actor[i] = normal() * 0.04f;
    for (uint32_t i = s.actor_w2(); i < s.actor_b2(); i++) actor[i] = normal() * 0.01f;
    for (uint32_t i = 0; i < MDN_ACTIONS; i++) actor[s.actor_log_std() + i] = -1.0f;
    for (uint32_t i = 0; i < s.critic_b1(); i++) critic[i] = normal() * 0.15f;
    for (uint32_t i = s.critic_w2(); i < s.critic_b2(); i++) critic[i] = normal() * 0.1f;
}

// Minibatch order of one rollout update (cpu_reference.hpp:569-579 ==
// main.mm:1331-1338): contiguous row blocks, shuffled with
// mt19937(0x9e3779b9 + rollout*0x85ebca6b), reshuffled only before epoch 1.
// The reference is built with Apple clang against libc++, so its std::shuffle
// is libc++'s, restated here over the mt19937 stream (whose output the C++
// standard fixes):
//   for k = 0 .. n-2: i = uniform integer in [0, n-1-k]; if i != 0, swap
//   v[k] and v[k+i];
// and libc++'s uniform_int_distribution<ptrdiff_t> over a 32-bit engine
// draws an integer in [0, range) as the low w = ceil(log2(range)) bits of one
// engine output, drawing again while the value is >= range (a range of 1
// draws nothing).  Returns the start row of every update in execution order.
inline uint32_t libcxx_uniform_below(std::mt19937& rng, uint64_t range) {
    if (range <= 1) return 0;
    uint32_t w = 0;
    while ((uint64_t(1) << w) < range) ++w;  // ceil(log2(range)), range <= 2^32
    const uint32_t mask = w >= 32 ? 0xffffffffu : ((1u << w) - 1u);
    uint32_t u;
    do {
        u = uint32_t(rng()) & mask;
    } while (u >= range);
    return u;
}

inline void libcxx_shuffle(std::vector<uint32_t>& v, std::mt19937& rng) {
    const size_t n = v.size();
    for (size_t k = 0; k + 1 < n; ++k) {
        const uint32_t i = libcxx_uniform_below(rng, uint64_t(n - k));
        if (i != 0) std::swap(v[k], v[k + i]);
    }
}

inline std::vector<uint32_t> minibatch_schedule(uint32_t rows, uint32_t minibatch, uint32_t epochs,
                                                uint32_t rollout_index) {
    std::vector<uint32_t> starts;
    for (uint32_t s = 0; s < rows; s += minibatch) starts.push_back(s);
    std::mt19937 rng(0x9e3779b9u + rollout_index * 0x85ebca6bu);
    libcxx_shuffle(starts, rng);
    std::vector<uint32_t> order;
    order.reserve(size_t(starts.size()) * epochs);
    for (uint32_t e = 0; e < epochs; ++e) {
        if (e == 1) libcxx_shuffle(starts, rng);
        order.insert(order.end(), starts.begin(), starts.end());
    }
    return order;
}

// Adam bias corrections 1 - beta^step, evaluated on the host in float with the
// platform pow exactly as cpu_reference.hpp:558-559 does.
inline void adam_corrections(uint64_t step, float beta1, float beta2, float* c1, float* c2) {
    *c1 = 1.0f - std::pow(beta1, float(step));
    *c2 = 1.0f - std::pow(beta2, float(step));
}

// RAPTOR1 loader (raptor.hpp:25-40).
inline bool load_raptor_file(const char* path, MdnRaptorWeights* w) {
    if (!path || !w) return false;
    FILE* f = std::fopen(path, "rb");
    if (!f) return false;
    unsigned char header[16];
    bool ok = std::fread(header, 1, 16, f) == 16;
    static const unsigned char magic[8] = {'R', 'A', 'P', 'T', 'O', 'R', '1', 0};
    ok = ok && std::memcmp(header, magic, 8) == 0;
    uint32_t version = 0, count = 0;
    std::memcpy(&version, header + 8, 4);
    std::memcpy(&count, header + 12, 4);
    ok = ok && version == 1 && count == 2084;
    ok = ok && std::fread(w, 1, sizeof(*w), f) == sizeof(*w);
    std::fclose(f);
    return ok;
}

// physics_domain.hpp:37-40 — the stress bounds of the episode plant draw
inline MdnDomainRange domain_stress_range() {
    return {0.90f, 1.10f, 0.90f, 1.10f, 0.90f, 1.10f, 0.75f, 1.35f, 0.75f, 1.35f, 1.15f};
}

// navigation_tasks.hpp:99-140 — baseline task parameters per stage
inline bool task_default_config(MdnTaskConfig& c, uint32_t stage, uint32_t family, float difficulty) {
    if (stage > MDN_TASK_STAGE_CLUTTER_GOAL || !(difficulty >= 0.0f && difficulty <= 1.0f)) return false;
    const bool open = stage != MDN_TASK_STAGE_CLUTTER_GOAL;
    if (open ? family != 0u : !(family == 1u || family == 2u || family == 4u || family == 5u || family == 12u))
        return false;
    c = MdnTaskConfig{};
    c.generation_version = 1; c.family = family; c.stage = stage;
    c.objective = MDN_TASK_OBJECTIVE_FINAL_HOLD; c.require_detour = 0;
    c.max_generation_attempts = MDN_TASK_MAX_ATTEMPTS; c.max_nav_steps = 400;
    c.scene_distance_m = 8.0f; c.difficulty = difficulty;
    c.minimum_endpoint_clearance_m = 0.30f; c.minimum_witness_clearance_m = 0.02f;
    c.goal_radius_m = 0.35f; c.stable_speed_mps = 0.50f; c.stable_hold_s = 0.20f; c.nav_period_s = 0.05f;
    c.progress_reward_per_m = 2.0f; c.time_cost_per_s = 0.20f; c.contact_penalty = 10.0f;
    c.stable_arrival_bonus = 10.0f; c.command_smoothness_weight = 0.05f;
    const float start_lo[3] = {-1.0f, -2.0f, 0.8f}, start_hi[3] = {1.0f, 2.0f, 2.4f};
    const float goal_lo[3] = {-1.2f, -4.0f, 0.5f}, goal_hi[3] = {13.2f, 4.0f, 4.5f};
    const bool near = stage == MDN_TASK_STAGE_NEAR_GOAL_HOLD;
    for (int k = 0; k < 3; k++) {
        c.start_min_xyz[k] = near ? goal_lo[k] : start_lo[k];
        c.start_max_xyz[k] = near ? goal_hi[k] : start_hi[k];
        c.goal_min_xyz[k] = goal_lo[k];
        c.goal_max_xyz[k] = goal_hi[k];
    }
    c.goal_distance_min_m = near ? 0.8f : 2.0f;
    c.goal_distance_max_m = near ? 2.0f : (stage == MDN_TASK_STAGE_CLUTTER_GOAL ? 7.0f : 6.0f);
    return true;
}

// nav_sensor::legacy / native (sensor_profile.hpp:118-126)
inline MdnCameraProfile camera_profile(uint32_t id) {
    MdnCameraProfile c;
    c.id = id == MDN_CAMERA_NATIVE ? MDN_CAMERA_NATIVE : MDN_CAMERA_LEGACY;
    c.tan_h = MDN_SENSOR_TAN_H;
    c.tan_v = id == MDN_CAMERA_NATIVE ? MDN_SENSOR_NATIVE_TAN_V : MDN_SENSOR_TAN_V;
    c.mount_x_m = id == MDN_CAMERA_NATIVE ? MDN_SENSOR_NATIVE_MOUNT_X : 0.0f;
    c.min_range_m = MDN_SENSOR_MIN_RANGE;
    c.max_range_m = MDN_SENSOR_MAX_RANGE;
    return c;
}

} // namespace mdn

#endif /* MDNAV_HOST_H */
