/*
 * oracle.cpp — CPU oracle, part 2: the batched simulator tick, the PPO
 * operators and the rollout+update trainer, with a C ABI for ctypes.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path.  It restates
 * cpu_reference.hpp (Trainer, OpenMP in place of GCD, plain loops in place of
 * Accelerate SGEMM) and, where the GPU path of the reference differs, the
 * kernels of sim.metal.  Reductions follow the canonical orders the HIP path
 * also uses (one definition, so both produce the same bits):
 *   - dot products:   z = b; z = fma(w[i], x[i], z) for i ascending
 *     (ppo.hpp:65-93, one rounding per step);
 *   - weight-gradient sums: g = fma(delta, x, g) over rows, same row order
 *     as the sums below;
 *   - sums over the rows of a minibatch: sequential within 256-row chunks,
 *     chunk partials summed sequentially within groups of 32 chunks, group
 *     sums sequentially (a single chunk at the reference's 256-row
 *     minibatch, i.e. the order of ppo_actor_grad_direct,
 *     ppo.metal:497-519);
 *   - squared gradient norm: 256 strided partial sums, then a pairwise tree;
 *   - advantage mean/variance: double; within each 256-row chunk 64 slots
 *     of 4 sequential rows combined by a pairwise tree over adjacent slots,
 *     chunk partials sequential within groups of 64 chunks, then over the
 *     groups.
 * Build: g++ -O2 -fopenmp -ffp-contract=off (see oracle/Makefile).
 */
#include <omp.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstring>
#include <vector>

#include "oracle_world.h"
#include "oracle_guidance.h"
#include "oracle_tasks.h"

namespace orc {

constexpr uint32_t kChunk = 256;
constexpr uint32_t kGradGroup = 32;   // chunk partials per group (gradient sums)
constexpr uint32_t kNormGroup = 64;   // chunk partials per group (advantage statistics)
constexpr float kGamma = 0.99f, kLambda = 0.95f, kClip = 0.2f, kValueCoef = 0.5f, kGradClip = 0.5f;
constexpr float kBeta1 = 0.9f, kBeta2 = 0.999f, kAdamEps = 1.0e-8f;
constexpr float kLogTwoPi = 1.8378770664093453f;

// ---- PPO operators: ppo.hpp:65-181 ---------------------------------------
inline void actor_forward(const PolicyShape& s, const float* w, const float* obs, float* hidden, float* mean) {
    for (uint32_t h = 0; h < s.hidden; ++h) {
        float z = w[s.actor_b1() + h];
        const float* row = w + size_t(h) * s.obs;
        for (uint32_t i = 0; i < s.obs; ++i) z = fma_f(row[i], obs[i], z);
        hidden[h] = tanh_f(z);
    }
    for (uint32_t a = 0; a < MDN_ACTIONS; ++a) {
        float z = w[s.actor_b2() + a];
        const float* row = w + s.actor_w2() + size_t(a) * s.hidden;
        for (uint32_t h = 0; h < s.hidden; ++h) z = fma_f(row[h], hidden[h], z);
        // geometry prior (ppo.hpp:30-34, 77): a 184-input actor adds the
        // observation's guidance hint to the first three means
        if (s.obs == MDN_ACTOR_OBS_PRIOR && a < 3) z += obs[s.obs - 3 + a];
        mean[a] = z;
    }
}
inline float critic_forward(const PolicyShape& s, const float* w, const float* obs, float* hidden) {
    for (uint32_t h = 0; h < s.critic_hidden; ++h) {
        float z = w[s.critic_b1() + h];
        const float* row = w + size_t(h) * s.critic_obs;
        for (uint32_t i = 0; i < s.critic_obs; ++i) z = fma_f(row[i], obs[i], z);
        hidden[h] = tanh_f(z);
    }
    float value = w[s.critic_b2()];
    for (uint32_t h = 0; h < s.critic_hidden; ++h) value = fma_f(w[s.critic_w2() + h], hidden[h], value);
    return value;
}
inline float gaussian_log_prob(const float* action, const float* mean, const float* log_std) {
    float result = 0.0f;
    for (uint32_t a = 0; a < MDN_ACTIONS; ++a) {
        const float inv_std = exp_f(-log_std[a]);
        const float d = (action[a] - mean[a]) * inv_std;
        result += -0.5f * (d * d + 2.0f * log_std[a] + kLogTwoPi);
    }
    return result;
}
struct Loss { float policy, value, entropy, ratio; };
inline Loss sample_loss_and_grad(const float* action, const float* mean, const float* log_std, float old_logp,
                                 float value, float advantage, float target, float batch, float clip,
                                 float vcoef, float ecoef, float* d_mean, float* d_log_std, float* d_value) {
    const float logp = gaussian_log_prob(action, mean, log_std);
    const float raw = logp - old_logp;
    const float lr = clamp_f(raw, -20.0f, 20.0f);
    const float ratio = exp_f(lr);
    const float clipped = clamp_f(ratio, 1.0f - clip, 1.0f + clip);
    const float chosen = min_f(ratio * advantage, clipped * advantage);
    const bool in_range = raw >= -20.0f && raw <= 20.0f;
    const bool active = in_range && (advantage >= 0.0f ? ratio <= 1.0f + clip : ratio >= 1.0f - clip);
    const float scale = 1.0f / max_f(batch, 1.0f);
    Loss loss;
    loss.policy = -chosen * scale;
    loss.value = 0.5f * vcoef * (value - target) * (value - target) * scale;
    loss.ratio = ratio;
    loss.entropy = 0.0f;
    for (uint32_t a = 0; a < MDN_ACTIONS; ++a) {
        const float inv_var = exp_f(-2.0f * log_std[a]);
        const float diff = action[a] - mean[a];
        if (active) {
            const float dlogp = -ratio * advantage * scale;
            d_mean[a] = dlogp * diff * inv_var;
            d_log_std[a] = dlogp * (diff * diff * inv_var - 1.0f);
        } else {
            d_mean[a] = 0.0f;
            d_log_std[a] = 0.0f;
        }
        d_log_std[a] -= ecoef * scale;
        loss.entropy += -ecoef * (log_std[a] + 0.5f * (1.0f + kLogTwoPi)) * scale;
    }
    *d_value = vcoef * (value - target) * scale;
    return loss;
}
// ppo.hpp:108-126
inline void compute_gae(uint32_t horizon, uint32_t n, const float* r, const float* v, const float* nv,
                        const uint8_t* term, const uint8_t* trunc, float gamma, float lambda, float* adv,
                        float* ret) {
#pragma omp parallel for schedule(static)
    for (int64_t env = 0; env < int64_t(n); ++env) {
        float carry = 0.0f;
        for (uint32_t rev = 0; rev < horizon; ++rev) {
            const uint32_t t = horizon - 1 - rev;
            const size_t k = size_t(t) * n + size_t(env);
            const bool te = term[k] != 0;
            const bool boundary = te || trunc[k] != 0;
            const float bootstrap = te ? 0.0f : nv[k];
            const float delta = r[k] + gamma * bootstrap - v[k];
            carry = delta + (boundary ? 0.0f : gamma * lambda * carry);
            adv[k] = carry;
            ret[k] = carry + v[k];
        }
    }
}
// Sequential within groups of `group` partials, then over the group sums.
template <class T>
inline T grouped_sum(const std::vector<T>& part, size_t group) {
    T total = T(0);
    for (size_t g0 = 0; g0 < part.size(); g0 += group) {
        T s = T(0);
        for (size_t c = g0; c < std::min(part.size(), g0 + group); ++c) s += part[c];
        total += s;
    }
    return total;
}
// Sum of f(a[i]) over one 256-element chunk in the canonical order: slot l
// (0..63) adds elements 4l..4l+3 sequentially from 0.0, then six butterfly
// levels s[l] = s[l] + s[l ^ off] for off = 1, 2, ..., 32 (a wavefront xor
// reduction; every slot ends with the same value since + is commutative).
// Adjacent slots pair first, so slots 8k..8k+7 (elements 32k..32k+31) form a
// subtree after three levels and the chunk's sum is the pairwise tree
// ((u0 + u1) + (u2 + u3)) + ((u4 + u5) + (u6 + u7)) of those eight subtrees.
template <class F>
inline double chunk_tree_sum(const float* a, size_t begin, size_t end, F f) {
    double s[64];
    for (size_t l = 0; l < 64; ++l) {
        s[l] = 0.0;
        for (size_t j = 0; j < 4; ++j) {
            const size_t i = begin + 4 * l + j;
            if (i < end) s[l] += f(a[i]);
        }
    }
    for (size_t off = 1; off < 64; off <<= 1) {
        double t[64];
        for (size_t l = 0; l < 64; ++l) t[l] = s[l] + s[l ^ off];
        for (size_t l = 0; l < 64; ++l) s[l] = t[l];
    }
    return s[0];
}
// ppo.hpp:128-140 with the canonical double sums: chunk tree sums, chunk
// partials sequential within groups of 64, then over the groups.
inline void normalize_advantages(float* a, size_t count, float eps) {
    if (count == 0) return;
    const size_t chunks = (count + kChunk - 1) / kChunk;
    std::vector<double> part(chunks);
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < int64_t(chunks); ++c)
        part[c] = chunk_tree_sum(a, size_t(c) * kChunk, std::min(count, size_t(c + 1) * kChunk),
                                 [](float x) { return double(x); });
    const double sum = grouped_sum(part, kNormGroup);
    const float mean = float(sum / double(count));
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < int64_t(chunks); ++c)
        part[c] = chunk_tree_sum(a, size_t(c) * kChunk, std::min(count, size_t(c + 1) * kChunk), [mean](float x) {
            const double d = double(x - mean);
            return d * d;
        });
    const double sq = grouped_sum(part, kNormGroup);
    const float inv = 1.0f / sqrt_f(float(sq / double(count)) + eps);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < int64_t(count); ++i) a[i] = (a[i] - mean) * inv;
}
// Squared L2 norm in the canonical order: 256 strided partials, pairwise tree.
inline float squared_norm(const float* g, size_t count) {
    float part[256];
    for (uint32_t t = 0; t < 256; ++t) {
        float s = 0.0f;
        for (size_t i = t; i < count; i += 256) s += g[i] * g[i];
        part[t] = s;
    }
    for (uint32_t stride = 128; stride > 0; stride >>= 1)
        for (uint32_t t = 0; t < stride; ++t) part[t] = part[t] + part[t + stride];
    return part[0];
}
// cpu_reference.hpp:553-567 (norm clip then Adam; corrections from the host).
// Returns the pre-clip norm sqrt(|g|^2 + 1e-20) (ppo_grad_norm, main.mm:963-975).
inline float clip_and_adam(std::vector<float>& grad, float* params, float* m, float* v, uint64_t step, float lr) {
    const float sum = squared_norm(grad.data(), grad.size());
    const float norm = sqrt_f(sum + 1.0e-20f);
    const float scale = min_f(1.0f, kGradClip / norm);
    for (float& g : grad) g *= scale;
    float c1, c2;
    adam_corrections(step, kBeta1, kBeta2, &c1, &c2);
    for (size_t i = 0; i < grad.size(); i++) {
        m[i] = kBeta1 * m[i] + (1.0f - kBeta1) * grad[i];
        v[i] = kBeta2 * v[i] + (1.0f - kBeta2) * grad[i] * grad[i];
        const float mh = m[i] / c1, vh = v[i] / c2;
        params[i] -= lr * mh / (sqrt_f(vh) + kAdamEps);
    }
    return norm;
}

// ---- Trainer: cpu_reference.hpp:112-615 + sim.metal semantics ------------
// Default-mode shaping reward of one env-step (cpu_reference.hpp:497-500 ==
// sim.metal:305): progress toward the goal doubled, a 0.01 step cost, a risk
// penalty growing linearly as the step's minimum clearance falls below
// 0.6 m, +10 on success and -10 on collision.
inline float step_reward(float before, float after, float step_clearance, float risk_coef, bool success,
                         bool collision) {
    return (before - after) * 2.0f - .01f - risk_coef * clamp_f((0.6f - step_clearance) / 0.6f, 0.0f, 1.0f) +
           (success ? 10.0f : 0.0f) - (collision ? 10.0f : 0.0f);
}

struct Trainer {
    MdnSimConfig cfg;
    uint32_t horizon, epochs, minibatch;
    MdnRaptorWeights raptor;
    MdnPhysicsParams physics;
    PolicyShape shape;
    std::vector<float> actor, critic, actor_m, actor_v, critic_m, critic_v;
    uint64_t optimizer_step = 0;
    std::vector<MdnPhysicsState> states;
    std::vector<MdnSimRun> runs;
    std::vector<MdnWorld> worlds;
    std::vector<float> sensors, poses, commands;
    std::vector<float> obs, co, nco, actions, logp, values, rewards, next_values, advantages, returns;
    std::vector<uint8_t> terminated, truncated;
    std::vector<float> metric_rows;
    std::vector<float> grad_norm_rows;  // [updates][2] pre-clip norms (main.mm:1370-1373)
    float metric_mean[4] = {0, 0, 0, 0};
    std::vector<float> means, camera;
    // camera profile (sensor_profile.hpp:46-51): legacy unless set_camera
    float camera_tan_v = MDN_SENSOR_TAN_V, camera_mount_x = 0.0f;
    // episode dynamics and navigation tasks (sim.metal:55-141, 287, 307-315)
    MdnRuntimeConfig runtime;
    MdnTaskControl tasks;
    std::vector<MdnPhysicsParams> env_physics;
    std::vector<MdnTaskState> task_states;
    // frozen challenge bank (sim.metal:95-121, 317)
    MdnBankControl bank;
    std::vector<MdnWorld> bank_worlds;
    std::vector<uint32_t> bank_schedule, bank_active, bank_transition;

    Trainer(const MdnSimConfig& c, uint32_t h, const MdnRaptorWeights& r, const MdnPhysicsParams& p,
            uint32_t ep, uint32_t mb)
        : cfg(c), horizon(h), epochs(ep), minibatch(mb), raptor(r), physics(p) {
        const size_t n = cfg.n, rows = n * horizon;
        actor.resize(shape.actor_count());
        critic.resize(shape.critic_count());
        init_policy(shape, actor.data(), critic.data());
        actor_m.assign(actor.size(), 0.0f); actor_v.assign(actor.size(), 0.0f);
        critic_m.assign(critic.size(), 0.0f); critic_v.assign(critic.size(), 0.0f);
        states.resize(n); runs.resize(n); worlds.resize(n);
        std::memset(states.data(), 0, n * sizeof(MdnPhysicsState));
        std::memset(runs.data(), 0, n * sizeof(MdnSimRun));
        std::memset(worlds.data(), 0, n * sizeof(MdnWorld));
        sensors.assign(n * MDN_SENSOR_FRAMES * MDN_SENSOR_PIXELS, 12.0f);
        poses.assign(n * MDN_SENSOR_FRAMES * 12, 0.0f);
        commands.assign(n * MDN_SENSOR_FRAMES * MDN_ACTIONS, 0.0f);
        obs.assign(rows * shape.obs, 0.0f); co.assign(rows * shape.critic_obs, 0.0f);
        nco.assign(rows * shape.critic_obs, 0.0f);
        actions.assign(rows * MDN_ACTIONS, 0.0f); logp.assign(rows, 0.0f); values.assign(rows, 0.0f);
        rewards.assign(rows, 0.0f); next_values.assign(rows, 0.0f); advantages.assign(rows, 0.0f);
        returns.assign(rows, 0.0f); terminated.assign(rows, 0); truncated.assign(rows, 0);
        means.assign(n * MDN_ACTIONS, 0.0f);
        std::memset(&runtime, 0, sizeof(runtime));
        std::memset(&tasks, 0, sizeof(tasks));
        env_physics.assign(n, p);
        task_states.resize(n);
        std::memset(task_states.data(), 0, n * sizeof(MdnTaskState));
        std::memset(&bank, 0, sizeof(bank));
        bank_active.assign(n, MDN_BANK_REHEARSAL);
        bank_transition.assign(rows, MDN_BANK_REHEARSAL);
        set_camera(MDN_SENSOR_TAN_V, 0.0f);
        for (uint32_t e = 0; e < cfg.n; e++) reset_env(e, true, 0);
    }

    // the profile's pixel rays and mount (sim.metal:147-152)
    void set_camera(float tan_v, float mount_x) {
        camera_tan_v = tan_v;
        camera_mount_x = mount_x;
        camera.resize(MDN_SENSOR_PIXELS * 3);
        for (uint32_t k = 0; k < MDN_SENSOR_PIXELS; k++) {
            const V3 ray = camera_ray(k, tan_v);
            camera[3 * k] = ray.x; camera[3 * k + 1] = ray.y; camera[3 * k + 2] = ray.z;
        }
    }

    // cpu_reference.hpp:219-238 == sim.metal:17-36
    bool clean_env(uint32_t n) const {
        return cfg.eval == 0 && ((cfg.family == 12 || cfg.family == 13) && n % 2 == 0);
    }
    uint32_t sensor_delay(uint32_t n) const { return clean_env(n) ? 0 : cfg.sensor_delay; }
    uint32_t command_delay(uint32_t n) const { return clean_env(n) ? 0 : cfg.command_delay; }
    float wind_param(uint32_t n) const { return clean_env(n) ? 0.0f : cfg.wind; }
    float depth_noise(uint32_t n) const { return clean_env(n) ? 0.0f : cfg.depth_noise; }
    float dropout(uint32_t n) const { return clean_env(n) ? 0.0f : cfg.dropout; }
    bool active(uint32_t n) const { return !(cfg.eval && runs[n].episodes); }

    // cpu_reference.hpp:240-273 == sim.metal:55-94 (runtime domain off)
    // sim.metal:95-121: the bank world of the env's schedule slot (a
    // generated rehearsal world for MDN_BANK_REHEARSAL)
    void apply_bank(uint32_t n, uint32_t slot) {
        if (bank.bank_count == 0 || n >= cfg.n || slot >= bank.schedule_stride) return;
        MdnPhysicsState& s = states[n];
        MdnSimRun& run = runs[n];
        MdnWorld& world = worlds[n];
        const uint32_t level = bank_schedule[size_t(n) * bank.schedule_stride + slot];
        if (level == MDN_BANK_REHEARSAL) {
            uint32_t rng = run.rng;
            const uint32_t family = training_family(n % 2 == 0 ? 12u : 13u, rng);
            const uint32_t seed = xorshift(rng);
            generate_world(world, seed, family, 4.0f);
            run.rng = rng;
        } else {
            if (level >= bank.bank_count) return;
            world = bank_worlds[level];
        }
        world.wind[0] = wind_param(n); world.wind[1] = 0; world.wind[2] = 0;
        run.initial_distance = vlen(v3(world.goal[0], world.goal[1], world.goal[2] - 1.5f));
        if (world.family == 10 || world.family == 11) {
            s.linear_velocity[0] = cfg.speed;
            run.desired_velocity[0] = cfg.speed;
            run.previous_nav[0] = 1.0f;
        }
        bank_active[n] = level;
    }

    void reset_env(uint32_t n, bool first, uint32_t slot) {
        MdnPhysicsState& s = states[n];
        MdnSimRun& run = runs[n];
        MdnWorld& world = worlds[n];
        uint32_t rng = first ? cfg.seed + n * 747796405u + 2891336453u : run.rng;
        // the moving-threat mix takes its family from the env's lane
        const uint32_t family = cfg.family == MDN_FAMILY_C3_MIX ? MDN_C3_LANE_FAMILY(n) : training_family(cfg.family, rng);
        const uint32_t world_seed = xorshift(rng);
        generate_world(world, world_seed, family, cfg.distance);
        world.wind[0] = wind_param(n); world.wind[1] = 0; world.wind[2] = 0;
        for (int j = 0; j < 3; j++) {
            s.position[j] = j == 2 ? 1.5f : 0;
            s.linear_velocity[j] = 0;
            s.angular_velocity_body[j] = 0;
            run.desired_velocity[j] = 0;
            run.reference_position[j] = s.position[j];
        }
        s.orientation_wxyz[0] = 1;
        for (int j = 1; j < 4; j++) s.orientation_wxyz[j] = 0;
        env_physics[n] = episode_params(runtime, physics, cfg.seed, n, first ? 0u : run.episodes);
        float hover[4];
        hover_rpm(runtime, physics, env_physics[n], hover);
        raptor_reset(raptor, run.hidden);
        for (int j = 0; j < 4; j++) { s.rpm[j] = hover[j]; run.motors[j] = 0; run.previous_nav[j] = 0; }
        if (world.family == 10 || world.family == 11) {
            s.linear_velocity[0] = cfg.speed;
            run.desired_velocity[0] = cfg.speed;
            run.previous_nav[0] = 1.0f;
        }
        std::fill(sensors.begin() + size_t(n) * 8 * 320, sensors.begin() + size_t(n + 1) * 8 * 320, 12.0f);
        std::fill(commands.begin() + size_t(n) * 8 * 4, commands.begin() + size_t(n + 1) * 8 * 4, 0.0f);
        run.yaw = 0; run.rng = rng; run.steps = 0; run.path = run.elapsed = run.peak_speed = 0;
        run.min_clearance = 12;
        run.initial_distance = vlen(v3(world.goal[0], world.goal[1], world.goal[2] - 1.5f));
        if (first) {
            run.successes = run.collisions = run.timeouts = run.episodes = 0;
            run.success_time = run.total_path = run.total_elapsed = run.final_progress = 0;
            std::fill(poses.begin() + size_t(n) * 96, poses.begin() + size_t(n + 1) * 96, 0.0f);
        }
        if (bank.enabled != 0) apply_bank(n, slot);
        else bank_active[n] = MDN_BANK_REHEARSAL;
        reset_task(tasks, cfg.seed, wind_param(n), n, s, run, world, task_states[n]);
    }
    void reset_all() {
        for (uint32_t e = 0; e < cfg.n; e++) reset_env(e, true, 0);
    }

    // sim.metal:159-181 == cpu_reference.hpp:379-394
    static void critic_observation(const MdnPhysicsState& s, const MdnWorld& w, const MdnSimRun& run, float* out) {
        for (uint32_t j = 0; j < MDN_CRITIC_OBS; j++) out[j] = 0;
        for (int j = 0; j < 3; j++) {
            out[j] = (w.goal[j] - s.position[j]) / 10.0f;
            out[j + 3] = s.linear_velocity[j] / 4.0f;
            out[j + 6] = s.angular_velocity_body[j] / 4.0f;
            out[j + 13] = s.position[j] / 10.0f;
            out[j + 16] = (run.reference_position[j] - s.position[j]) * 2.0f;
        }
        for (int j = 0; j < 4; j++) out[9 + j] = s.orientation_wxyz[j];
        out[30] = w.wind[0];
        out[31] = w.wind[1];
        out[19] = clearance(w, v3(s.position[0], s.position[1], s.position[2]), run.elapsed) / 5.0f;
        out[20] = float(run.steps) / 200.0f;
        for (uint32_t j = 0; j < std::min(w.count, 3u); j++) {
            const V3 c = obstacle_center(w.obstacles[j], run.elapsed);
            out[21 + j * 3] = (c.x - s.position[0]) / 10.0f;
            out[22 + j * 3] = (c.y - s.position[1]) / 10.0f;
            out[23 + j * 3] = (c.z - s.position[2]) / 10.0f;
        }
    }

    // sim.metal:145-158 + 182-228 == cpu_reference.hpp:275-377 (pooled 181 obs)
    void depth_and_observe(uint32_t tick, uint32_t n) {
        MdnSimRun& run = runs[n];
        const MdnPhysicsState& s = states[n];
        const MdnWorld& world = worlds[n];
        float r[9];
        rotation(s.orientation_wxyz, r);
        if (run.steps % cfg.sensor_period == 0) {
            const uint32_t frame = (run.steps / cfg.sensor_period) % 8;
            const float mx = camera_mount_x;
            const V3 origin = v3(s.position[0] + mx * r[0], s.position[1] + mx * r[3], s.position[2] + mx * r[6]);
            float* pose = &poses[(size_t(n) * 8 + frame) * 12];
            pose[0] = origin.x; pose[1] = origin.y; pose[2] = origin.z;
            for (int j = 0; j < 9; j++) pose[3 + j] = r[j];
            const float noise = depth_noise(n), drop = dropout(n);
            for (uint32_t k = 0; k < MDN_SENSOR_PIXELS; k++) {
                const float rx = camera[3 * k], ry = camera[3 * k + 1], rz = camera[3 * k + 2];
                const V3 d = v3(r[0] * rx + r[1] * ry + r[2] * rz, r[3] * rx + r[4] * ry + r[5] * rz,
                                r[6] * rx + r[7] * ry + r[8] * rz);
                float depth = ray_world(world, origin, d, run.elapsed);
                if (noise != 0 || drop != 0) {
                    uint32_t rng = run.rng + k * 1664525u + run.steps * 1013904223u;
                    depth = clamp_f(depth + noise * sim_normal(rng), 0.0f, 12.0f);
                    if (urand(rng) < drop) depth = 12.0f;
                }
                sensors[(size_t(n) * 8 + frame) * 320 + k] = depth;
            }
        }
        const uint32_t available = run.steps / cfg.sensor_period;
        const uint32_t delay = sensor_delay(n);
        const uint32_t frame = available > delay ? available - delay : 0;
        const uint32_t prev = frame > 0 ? frame - 1 : 0;
        float* o = &obs[(size_t(tick) * cfg.n + n) * shape.obs];
        const float* cur_f = &sensors[(size_t(n) * 8 + frame % 8) * 320];
        const float* prev_f = &sensors[(size_t(n) * 8 + prev % 8) * 320];
        for (uint32_t k = 0; k < MDN_POOLED_FEATURES; k++) {
            float current = 12.0f, previous = 12.0f;
            const uint32_t y = (k / 10) * 2, x = (k % 10) * 2;
            for (uint32_t dy = 0; dy < 2; dy++)
                for (uint32_t dx = 0; dx < 2; dx++) {
                    const uint32_t pixel = (y + dy) * 20 + x + dx;
                    current = min_f(current, cur_f[pixel]);
                    previous = min_f(previous, prev_f[pixel]);
                }
            o[k] = available >= delay ? current / 12.0f : 1.0f;
            o[80 + k] = available >= delay ? previous / 12.0f : 1.0f;
        }
        if (cfg.mode == 18)  // sim.metal:211-213: evaluation ablation without the previous frame
            for (uint32_t k = 0; k < MDN_POOLED_FEATURES; k++) o[80 + k] = o[k];
        const V3 delta = v3(world.goal[0] - s.position[0], world.goal[1] - s.position[1], world.goal[2] - s.position[2]);
        const float distance = max_f(vlen(delta), 1.0e-6f);
        float* c = o + 160;
        for (int j = 0; j < 3; j++) {
            c[j] = (r[j] * delta.x + r[3 + j] * delta.y + r[6 + j] * delta.z) / distance;
            c[4 + j] = (r[j] * s.linear_velocity[0] + r[3 + j] * s.linear_velocity[1] + r[6 + j] * s.linear_velocity[2]) / 4.0f;
            c[7 + j] = s.angular_velocity_body[j] / 4.0f;
            c[10 + j] = r[6 + j];
        }
        c[3] = min_f(distance / 10.0f, 1.5f);
        for (int j = 0; j < 4; j++) c[13 + j] = run.previous_nav[j];
        c[17] = float(run.steps - frame * cfg.sensor_period) * physics.dt * float(cfg.substeps);
        const float ref[3] = {run.reference_position[0] - s.position[0], run.reference_position[1] - s.position[1],
                              run.reference_position[2] - s.position[2]};
        for (int j = 0; j < 3; j++) c[18 + j] = clamp_f((r[j] * ref[0] + r[3 + j] * ref[1] + r[6 + j] * ref[2]) * 2.0f, -1.0f, 1.0f);
        if (shape.obs == MDN_ACTOR_OBS_PRIOR) {  // guidance hint (cpu_reference.hpp:353-375)
            float cur[80], prv[80], goal[3], vel[3], hint[3];
            for (int j = 0; j < 80; j++) { cur[j] = o[j] * 12.0f; prv[j] = o[80 + j] * 12.0f; }
            for (int j = 0; j < 3; j++) { goal[j] = c[j]; vel[j] = c[4 + j] * 4.0f; }
            const float sensor_dt = float(cfg.sensor_period) * physics.dt * float(cfg.substeps);
            if (cfg.geometry_memory) {
                float pose[12];
                for (int j = 0; j < 3; j++) pose[j] = s.position[j];
                for (int j = 0; j < 9; j++) pose[3 + j] = r[j];
                uint32_t valid = available >= delay ? std::min(frame + 1, 8u - delay) : 0u;
                if (cfg.mode == 18) valid = std::min(valid, 1u);  // memory.metal:34: newest frame only
                nav_guidance_memory(cur, prv, goal, distance, vel, sensor_dt, camera_tan_v,
                                    &sensors[size_t(n) * 8 * 320], &poses[size_t(n) * 8 * 12], pose, frame, valid, hint);
            } else {
                nav_guidance(cur, prv, goal, distance, vel, sensor_dt, camera_tan_v, hint);
            }
            for (int j = 0; j < 3; j++) o[shape.obs - 3 + j] = hint[j];
        }
        critic_observation(s, world, run, &co[(size_t(tick) * cfg.n + n) * shape.critic_obs]);
    }

    // Pooled cells of the top two grid rows farther than 2.5 m (sim.metal:233, 236).
    static float overhead_cells(const float* o) {
        float overhead = 0.0f;
        for (int k = 0; k < 20; k++) overhead += o[k] * 12.0f > 2.5f ? 1.0f : 0.0f;
        return overhead;
    }
    // sim.metal:233: evaluation modes 9-21 of the 184-input actor pull the
    // means toward the hint (inputs 181-183) by a mode-dependent scale.
    // Only the reference's GPU path has them (cpu_reference.hpp samples in
    // mode 0 only); restated from the Metal source.
    static void guided_mode_means(uint32_t mode, const float* o, float* mean) {
        float scale = (mode == 9 || mode == 13) ? 0.0f
                      : ((mode == 10 || mode == 14 || mode == 16) ? 0.25f : (mode == 15 ? 1.0f : 0.5f));
        if (mode >= 17) scale = 0.25f + 0.75f * (overhead_cells(o) / 20.0f);
        if (mode == 12) {
            float near = 12.0f;
            for (int k = 0; k < 80; k++) near = fmin_f(near, o[k] * 12.0f);
            scale = clamp_f((near - .3f) / 2, 0.2f, 1.0f);
        }
        for (int j = 0; j < 3; j++) {
            const float prior = o[MDN_ACTOR_OBS_PRIOR - 3 + j];
            mean[j] = prior + scale * (mean[j] - prior);
        }
        mean[3] *= scale;
        if (mode == 16) {
            const float yaw = atan2_f(o[161], o[160]);
            mean[3] += nav_atanh(clamp_f(yaw * 1.5f, -.85f, .85f));
        }
    }

    // sim.metal:229-271 == cpu_reference.hpp:404-429
    void act(uint32_t tick, uint32_t n) {
        MdnSimRun& run = runs[n];
        const size_t row = size_t(tick) * cfg.n + n;
        float hidden[8192];
        float mean[4];
        if (ext_means)  // means supplied from outside (a policy evaluated elsewhere)
            for (int j = 0; j < 4; j++) mean[j] = ext_means[row * 4 + j];
        else
            actor_forward(shape, actor.data(), &obs[row * shape.obs], hidden, mean);
        values[row] = critic_forward(shape, critic.data(), &co[row * shape.critic_obs], hidden);
        const float* o = &obs[row * shape.obs];
        const bool guided = shape.obs == MDN_ACTOR_OBS_PRIOR;
        if (guided && cfg.mode >= 9 && cfg.mode <= 21) guided_mode_means(cfg.mode, o, mean);
        // sim.metal:234-238, 246-252: mode 22 trains through the deployed
        // mode-17 map of the sampled action (the log-probability stays on the
        // raw sample)
        const float deployed = guided && cfg.mode == 22 ? 0.25f + 0.75f * (overhead_cells(o) / 20.0f) : 1.0f;
        const float* log_std = &actor[shape.actor_log_std()];
        uint32_t rng = run.rng;
        float lp = 0, a[4];
        for (int j = 0; j < 4; j++) {
            a[j] = mean[j] + ((cfg.mode == 0 || cfg.mode == 22) ? exp_f(log_std[j]) * sim_normal(rng) : 0.0f);
            if (cfg.mode == 1) a[j] = sim_normal(rng);
            const float diff = (a[j] - mean[j]) * exp_f(-log_std[j]);
            lp += -0.5f * (diff * diff + 2 * log_std[j] + kLogTwoPi);
            actions[row * 4 + j] = a[j];
            float executed = a[j];
            if (guided && cfg.mode == 22)
                executed = j < 3 ? o[MDN_ACTOR_OBS_PRIOR - 3 + j] + deployed * (a[j] - o[MDN_ACTOR_OBS_PRIOR - 3 + j])
                                 : deployed * a[j];
            commands[(size_t(n) * 8 + run.steps % 8) * 4 + j] = tanh_f(executed);
        }
        logp[row] = lp;
        run.rng = rng;
        const MdnPhysicsState& s = states[n];
        float r[9];
        rotation(s.orientation_wxyz, r);
        if (cfg.mode == 2 || cfg.mode == 3 || cfg.mode == 20) {
            const MdnWorld& w = worlds[n];
            V3 d = v3(w.goal[0] - s.position[0], w.goal[1] - s.position[1], w.goal[2] - s.position[2]);
            const float len = vlen(d);
            d = vmul(vmul(d, 1.0f / len), min_f(len, cfg.speed));
            a[0] = (r[0] * d.x + r[3] * d.y + r[6] * d.z) / cfg.speed;
            a[1] = (r[1] * d.x + r[4] * d.y + r[7] * d.z) / cfg.speed;
            a[2] = (r[2] * d.x + r[5] * d.y + r[8] * d.z) / cfg.speed;
            a[3] = 0;
            for (int j = 0; j < 4; j++) commands[(size_t(n) * 8 + run.steps % 8) * 4 + j] = a[j];
        }
        const uint32_t delay = command_delay(n);
        const uint32_t applied = run.steps > delay ? run.steps - delay : 0;
        for (int j = 0; j < 4; j++)
            run.previous_nav[j] = run.steps < delay ? 0.0f : commands[(size_t(n) * 8 + applied % 8) * 4 + j];
        float v[3] = {run.previous_nav[0] * cfg.speed, run.previous_nav[1] * cfg.speed,
                      run.previous_nav[2] * cfg.speed * (cfg.velocity_contract == 0 ? 0.5f : 1.0f)};
        if (cfg.velocity_contract == 1) {
            const float scale = min_f(1.0f, cfg.speed / max_f(vlen(v3(v[0], v[1], v[2])), 1e-8f));
            for (float& x : v) x *= scale;
        }
        if (cfg.mode == 19) {
            const float magnitude = vlen(v3(v[0], v[1], v[2]));
            if (magnitude > 1e-8f) {
                const float scale = cfg.speed / magnitude;
                for (float& x : v) x *= scale;
            }
        }
        for (int j = 0; j < 3; j++) run.desired_velocity[j] = r[j * 3] * v[0] + r[j * 3 + 1] * v[1] + r[j * 3 + 2] * v[2];
        run.yaw += run.previous_nav[3] * physics.dt * float(cfg.substeps) * 0.5f;
    }

    // sim.metal:272-332 == cpu_reference.hpp:460-513 (+ next value, reset)
    void advance(uint32_t tick, uint32_t n) {
        MdnSimRun& run = runs[n];
        MdnPhysicsState s = states[n];
        MdnWorld& world = worlds[n];
        float h[16], motors[4];
        for (int j = 0; j < 16; j++) h[j] = run.hidden[j];
        for (int j = 0; j < 4; j++) motors[j] = run.motors[j];
        const V3 goal = v3(world.goal[0], world.goal[1], world.goal[2]);
        const float before = vlen(vsub(goal, v3(s.position[0], s.position[1], s.position[2])));
        const float yaw = run.yaw;
        float si, c;
        sincos_f(yaw, &si, &c);
        float sh, ch;
        sincos_f(yaw * 0.5f, &sh, &ch);
        bool collision = false;
        float step_clearance = 12.0f;
        const MdnPhysicsParams& sp = runtime.enabled != 0 ? env_physics[n] : physics;
        const float wind[3] = {world.wind[0] * sp.mass, world.wind[1] * sp.mass, world.wind[2] * sp.mass};
        for (uint32_t step = 0; step < cfg.substeps; step++) {
            float mo[22];
            const float v[3] = {run.desired_velocity[0], run.desired_velocity[1], run.desired_velocity[2]};
            for (int j = 0; j < 3; j++) run.reference_position[j] += v[j] * physics.dt;
            const float dp[3] = {s.position[0] - run.reference_position[0], s.position[1] - run.reference_position[1],
                                 s.position[2] - run.reference_position[2]};
            const float dv[3] = {s.linear_velocity[0] - v[0], s.linear_velocity[1] - v[1], s.linear_velocity[2] - v[2]};
            mo[0] = clamp_f(c * dp[0] + si * dp[1], -.5f, .5f);
            mo[1] = clamp_f(-si * dp[0] + c * dp[1], -.5f, .5f);
            mo[2] = clamp_f(dp[2], -.5f, .5f);
            const float* sq = s.orientation_wxyz;
            const float q[4] = {ch * sq[0] + sh * sq[3], ch * sq[1] + sh * sq[2], ch * sq[2] - sh * sq[1],
                                ch * sq[3] - sh * sq[0]};
            float r[9];
            rotation(q, r);
            for (int j = 0; j < 9; j++) mo[3 + j] = r[j];
            mo[12] = clamp_f(c * dv[0] + si * dv[1], -1.0f, 1.0f);
            mo[13] = clamp_f(-si * dv[0] + c * dv[1], -1.0f, 1.0f);
            mo[14] = clamp_f(dv[2], -1.0f, 1.0f);
            for (int j = 0; j < 3; j++) mo[15 + j] = s.angular_velocity_body[j];
            for (int j = 0; j < 4; j++) mo[18 + j] = motors[j];
            raptor_forward(raptor, mo, h, motors);
            raptor_clip(motors);
            MdnPhysicsState next;
            physics_step(s, motors, wind, sp, next);
            bool valid = true;
            const float* nf = &next.position[0];
            for (int j = 0; j < 17; j++) valid = valid && isfinite_f(nf[j]);
            if (!valid) { collision = true; break; }
            run.path += vlen(vsub(v3(s.position[0], s.position[1], s.position[2]),
                                  v3(next.position[0], next.position[1], next.position[2])));
            s = next;
            run.elapsed += physics.dt;
            const float cl = clearance(world, v3(s.position[0], s.position[1], s.position[2]), run.elapsed);
            step_clearance = min_f(step_clearance, cl);
            run.min_clearance = min_f(run.min_clearance, cl);
            run.peak_speed = max_f(run.peak_speed, vlen(v3(s.linear_velocity[0], s.linear_velocity[1], s.linear_velocity[2])));
            if (cl <= 0) { collision = true; break; }
        }
        run.steps++;
        states[n] = s;
        for (int j = 0; j < 16; j++) run.hidden[j] = h[j];
        for (int j = 0; j < 4; j++) run.motors[j] = motors[j];
        const float after = vlen(vsub(goal, v3(s.position[0], s.position[1], s.position[2])));
        bool success = after < (cfg.mode == 20 ? .10f : .35f) && !collision;
        bool timeout = run.steps >= cfg.max_steps;
        const size_t row = size_t(tick) * cfg.n + n;
        rewards[row] = step_reward(before, after, step_clearance, cfg.risk_coef, success, collision);
        terminated[row] = uint8_t(collision || success);
        truncated[row] = uint8_t(timeout && !terminated[row]);
        if (tasks.enabled != 0) {  // sim.metal:307-315
            const float executed[4] = {run.desired_velocity[0], run.desired_velocity[1], run.desired_velocity[2],
                                       run.previous_nav[3] * 0.5f};
            const TaskStep o = task_step(task_states[n], tasks.config, s.position, s.linear_velocity, executed,
                                         uint32_t(collision), uint32_t(timeout));
            success = o.stable_success != 0 && !collision;
            timeout = o.timeout != 0;
            rewards[row] = o.reward;
            terminated[row] = uint8_t(collision || success);
            truncated[row] = uint8_t(timeout && !terminated[row]);
        }
        bank_transition[row] = bank.enabled != 0 ? bank_active[n] : MDN_BANK_REHEARSAL;  // sim.metal:317
        float hidden[8192];
        float* cobs = &nco[row * shape.critic_obs];
        critic_observation(s, world, run, cobs);
        next_values[row] = critic_forward(shape, critic.data(), cobs, hidden);
        if (success || collision || timeout) {
            run.successes += success;
            run.collisions += collision;
            run.timeouts += timeout && !terminated[row];
            run.episodes++;
            run.success_time += success ? run.elapsed : 0;
            run.total_path += run.path;
            run.total_elapsed += run.elapsed;
            run.final_progress += 1.0f - after / max_f(run.initial_distance, 1.0e-4f);
            if (!cfg.eval) reset_env(n, false, tick + 1);
        }
    }

    // Sim::collect (main.mm:573-598): tick t writes row block t % horizon.
    void collect(uint32_t count) {
        if (count == 0) count = horizon;
        for (uint32_t t = 0; t < count; t++) {
            const uint32_t tick = t % horizon;
#pragma omp parallel for schedule(dynamic, 16)
            for (int64_t n = 0; n < int64_t(cfg.n); n++) {
                if (!active(uint32_t(n))) continue;
                depth_and_observe(tick, uint32_t(n));
                act(tick, uint32_t(n));
                advance(tick, uint32_t(n));
            }
        }
    }

    void gae() {
        compute_gae(horizon, cfg.n, rewards.data(), values.data(), next_values.data(), terminated.data(),
                    truncated.data(), kGamma, kLambda, advantages.data(), returns.data());
    }
    void normalize() { normalize_advantages(advantages.data(), advantages.size(), 1.0e-8f); }

    // Loss, per-row derivatives and reduced gradients of one minibatch
    // (main.mm:1349-1364 == cpu_reference.hpp:586-599).  Optional outputs:
    // per-row d_mean/d_log_std (b*4) and d_value (b).
    void minibatch_grads(uint32_t begin, uint32_t b, std::vector<float>& ag, std::vector<float>& cg,
                         float* metric_row, float* dm_out = nullptr, float* dls_out = nullptr,
                         float* dv_out = nullptr) {
        const PolicyShape& S = shape;
        const uint32_t H = S.hidden, D = S.obs, CH = S.critic_hidden, CD = S.critic_obs;
        std::vector<float> ah(size_t(b) * H), am(size_t(b) * 4), ch(size_t(b) * CH), cv(b);
        std::vector<float> dm(size_t(b) * 4), dls(size_t(b) * 4), dv(b), losses(size_t(b) * 4);
        std::vector<float> adelta(size_t(b) * H), cdelta(size_t(b) * CH);
        const float* X = &obs[size_t(begin) * D];
        const float* C = &co[size_t(begin) * CD];
        const float* log_std = &actor[S.actor_log_std()];
#pragma omp parallel for schedule(static)
        for (int64_t n = 0; n < int64_t(b); n++) {
            actor_forward(S, actor.data(), X + size_t(n) * D, &ah[size_t(n) * H], &am[size_t(n) * 4]);
            cv[n] = critic_forward(S, critic.data(), C + size_t(n) * CD, &ch[size_t(n) * CH]);
            const size_t row = size_t(begin) + size_t(n);
            const Loss l = sample_loss_and_grad(&actions[row * 4], &am[size_t(n) * 4], log_std, logp[row], cv[n],
                                                advantages[row], returns[row], float(b), kClip, kValueCoef,
                                                cfg.entropy_coef, &dm[size_t(n) * 4], &dls[size_t(n) * 4], &dv[n]);
            losses[size_t(n) * 4 + 0] = l.policy; losses[size_t(n) * 4 + 1] = l.value;
            losses[size_t(n) * 4 + 2] = l.entropy; losses[size_t(n) * 4 + 3] = l.ratio;
            // ppo.metal:470-485 and 618-631
            for (uint32_t h = 0; h < H; h++) {
                float d = 0.0f;
                for (uint32_t a = 0; a < 4; a++) d = fma_f(dm[size_t(n) * 4 + a], actor[S.actor_w2() + a * H + h], d);
                const float act = ah[size_t(n) * H + h];
                adelta[size_t(n) * H + h] = d * (1.0f - act * act);
            }
            for (uint32_t h = 0; h < CH; h++) {
                const float act = ch[size_t(n) * CH + h];
                cdelta[size_t(n) * CH + h] = dv[n] * critic[S.critic_w2() + h] * (1.0f - act * act);
            }
        }
        // metrics row (main.mm:941-951) with chunked sums
        const uint32_t chunks = (b + kChunk - 1) / kChunk;
        float msum[4] = {0, 0, 0, 0};
        for (int k = 0; k < 4; k++) {
            std::vector<float> part(chunks, 0.0f);
            for (uint32_t c = 0; c < chunks; c++)
                for (uint32_t n = c * kChunk; n < std::min(b, (c + 1) * kChunk); n++) part[c] += losses[size_t(n) * 4 + k];
            msum[k] = grouped_sum(part, kGradGroup);
        }
        msum[3] /= float(b);
        for (int k = 0; k < 4; k++) metric_row[k] = msum[k];
        // Gradients: every parameter is a chunked sum over the minibatch rows
        // (sequential within a 256-row chunk, then sequential over chunks).
        // Rows run in the outer loop for locality; each parameter's own
        // accumulation order is unchanged by that.
        const uint32_t AP = S.actor_count(), CP = S.critic_count();
        std::vector<float> apart(size_t(chunks) * AP, 0.0f), cpart(size_t(chunks) * CP, 0.0f);
#pragma omp parallel for schedule(dynamic, 1)
        for (int64_t c = 0; c < int64_t(chunks); c++) {
            float* ga = &apart[size_t(c) * AP];
            float* gc = &cpart[size_t(c) * CP];
            for (uint32_t n = uint32_t(c) * kChunk; n < std::min(b, uint32_t(c + 1) * kChunk); n++) {
                const float* x = X + size_t(n) * D;
                const float* cx = C + size_t(n) * CD;
                for (uint32_t h = 0; h < H; h++) {
                    const float d = adelta[size_t(n) * H + h];
                    float* row = ga + size_t(h) * D;
                    for (uint32_t i = 0; i < D; i++) row[i] = fma_f(d, x[i], row[i]);
                    ga[S.actor_b1() + h] += d;
                }
                for (uint32_t a = 0; a < 4; a++) {
                    const float g = dm[size_t(n) * 4 + a];
                    for (uint32_t h = 0; h < H; h++)
                        ga[S.actor_w2() + a * H + h] = fma_f(g, ah[size_t(n) * H + h], ga[S.actor_w2() + a * H + h]);
                    ga[S.actor_b2() + a] += g;
                    ga[S.actor_log_std() + a] += dls[size_t(n) * 4 + a];
                }
                for (uint32_t h = 0; h < CH; h++) {
                    const float d = cdelta[size_t(n) * CH + h];
                    float* row = gc + size_t(h) * CD;
                    for (uint32_t i = 0; i < CD; i++) row[i] = fma_f(d, cx[i], row[i]);
                    gc[S.critic_b1() + h] += d;
                    gc[S.critic_w2() + h] = fma_f(dv[n], ch[size_t(n) * CH + h], gc[S.critic_w2() + h]);
                }
                gc[S.critic_b2()] += dv[n];
            }
        }
        ag.assign(AP, 0.0f);
        cg.assign(CP, 0.0f);
#pragma omp parallel for schedule(static)
        for (int64_t p = 0; p < int64_t(AP); p++) {
            float total = 0.0f;
            for (uint32_t g0 = 0; g0 < chunks; g0 += kGradGroup) {
                float s = 0.0f;
                for (uint32_t c = g0; c < std::min(chunks, g0 + kGradGroup); c++) s += apart[size_t(c) * AP + size_t(p)];
                total += s;
            }
            ag[p] = total;
        }
        for (uint32_t p = 0; p < CP; p++) {
            float total = 0.0f;
            for (uint32_t g0 = 0; g0 < chunks; g0 += kGradGroup) {
                float s = 0.0f;
                for (uint32_t c = g0; c < std::min(chunks, g0 + kGradGroup); c++) s += cpart[size_t(c) * CP + p];
                total += s;
            }
            cg[p] = total;
        }
        if (dm_out) std::copy(dm.begin(), dm.end(), dm_out);
        if (dls_out) std::copy(dls.begin(), dls.end(), dls_out);
        if (dv_out) std::copy(dv.begin(), dv.end(), dv_out);
    }

    // One minibatch update (main.mm:1349-1378 == cpu_reference.hpp:580-603).
    void update_minibatch(uint32_t begin, uint32_t b, float* metric_row, float* norm_row) {
        const PolicyShape& S = shape;
        std::vector<float> ag, cg;
        minibatch_grads(begin, b, ag, cg, metric_row);
        ++optimizer_step;
        norm_row[0] = clip_and_adam(ag, actor.data(), actor_m.data(), actor_v.data(), optimizer_step, cfg.learning_rate);
        norm_row[1] = clip_and_adam(cg, critic.data(), critic_m.data(), critic_v.data(), optimizer_step, cfg.learning_rate);
        for (uint32_t a = 0; a < 4; a++) {
            float& x = actor[S.actor_log_std() + a];
            x = clamp_f(x, -2.0f, .5f);
        }
    }

    // PPOTrainer::rollout_update (main.mm:1321-1384) without the optional
    // anchor/auxiliary terms.
    void update(uint32_t rollout_index) {
        const uint32_t rows = cfg.n * horizon;
        const std::vector<uint32_t> order = minibatch_schedule(rows, minibatch, epochs, rollout_index);
        metric_rows.assign(order.size() * 4, 0.0f);
        grad_norm_rows.assign(order.size() * 2, 0.0f);
        for (size_t u = 0; u < order.size(); u++) {
            const uint32_t begin = order[u];
            const uint32_t b = std::min(minibatch, rows - begin);
            update_minibatch(begin, b, &metric_rows[u * 4], &grad_norm_rows[u * 2]);
        }
        // main.mm:952-962
        for (int k = 0; k < 4; k++) metric_mean[k] = 0.0f;
        for (size_t u = 0; u < order.size(); u++)
            for (int k = 0; k < 4; k++) metric_mean[k] += metric_rows[u * 4 + k];
        if (!order.empty())
            for (int k = 0; k < 4; k++) metric_mean[k] /= float(order.size());
    }

    // Means [T][N][4] that act() uses in place of the actor's forward pass
    // (nullptr: the actor).  The sampling, log-probability and everything
    // downstream are unchanged (sim.metal:229-256 with mean given).
    const float* ext_means = nullptr;

    // A policy of hidden width h (ppo.hpp:17-45 FIXED_PPO_HIDDEN_DIM) in
    // place of the current one: fresh initialisation, zero Adam moments.
    void set_hidden(uint32_t h) {
        shape.hidden = shape.critic_hidden = h;
        actor.assign(shape.actor_count(), 0.0f);
        critic.assign(shape.critic_count(), 0.0f);
        init_policy(shape, actor.data(), critic.data());
        actor_m.assign(actor.size(), 0.0f); actor_v.assign(actor.size(), 0.0f);
        critic_m.assign(critic.size(), 0.0f); critic_v.assign(critic.size(), 0.0f);
        optimizer_step = 0;
    }
    // Actor input width (ppo.hpp:11-34 FIXED_PPO_ACTOR_OBS_DIM): 181 (pooled
    // observation) or 184 (with the geometry-prior hint).  Fresh policy and
    // moments; observation rows resized.
    void set_actor_obs(uint32_t d) {
        shape.obs = d;
        obs.assign(size_t(cfg.n) * horizon * d, 0.0f);
        set_hidden(shape.hidden);
    }
    // Log-probabilities of the stored actions and values at s and s' under the
    // current policy for every rollout row (the rollout's act and next-value
    // outputs re-evaluated with this policy).
    void evaluate() {
        const int64_t rows = int64_t(cfg.n) * horizon;
        const float* log_std = &actor[shape.actor_log_std()];
#pragma omp parallel for schedule(static)
        for (int64_t row = 0; row < rows; row++) {
            float hidden[8192], mean[4];
            actor_forward(shape, actor.data(), &obs[size_t(row) * shape.obs], hidden, mean);
            logp[row] = gaussian_log_prob(&actions[size_t(row) * 4], mean, log_std);
            values[row] = critic_forward(shape, critic.data(), &co[size_t(row) * shape.critic_obs], hidden);
            next_values[row] = critic_forward(shape, critic.data(), &nco[size_t(row) * shape.critic_obs], hidden);
        }
    }

    void iteration(uint32_t rollout_index) {
        collect(horizon);
        gae();
        normalize();
        update(rollout_index);
    }
};

} // namespace orc

// =========================== C ABI for ctypes ===============================
extern "C" {

using orc::Trainer;

void* orc_trainer_create(const MdnSimConfig* cfg, uint32_t horizon, const MdnRaptorWeights* raptor,
                         const MdnPhysicsParams* physics, uint32_t epochs, uint32_t minibatch) {
    return new Trainer(*cfg, horizon, *raptor, *physics, epochs, minibatch);
}
void orc_trainer_destroy(void* h) { delete static_cast<Trainer*>(h); }
void orc_trainer_collect(void* h, uint32_t count) { static_cast<Trainer*>(h)->collect(count); }
void orc_trainer_gae(void* h) { static_cast<Trainer*>(h)->gae(); }
void orc_trainer_normalize(void* h) { static_cast<Trainer*>(h)->normalize(); }
void orc_trainer_update(void* h, uint32_t rollout_index) { static_cast<Trainer*>(h)->update(rollout_index); }
void orc_trainer_iteration(void* h, uint32_t rollout_index) { static_cast<Trainer*>(h)->iteration(rollout_index); }
void orc_trainer_minibatch_grads(void* h, uint32_t begin, uint32_t b, float* actor_grad, float* critic_grad,
                                 float* metric_row, float* d_mean, float* d_log_std, float* d_value) {
    Trainer* t = static_cast<Trainer*>(h);
    std::vector<float> ag, cg;
    t->minibatch_grads(begin, b, ag, cg, metric_row, d_mean, d_log_std, d_value);
    std::copy(ag.begin(), ag.end(), actor_grad);
    std::copy(cg.begin(), cg.end(), critic_grad);
}
void orc_trainer_set_config(void* h, const MdnSimConfig* cfg) { static_cast<Trainer*>(h)->cfg = *cfg; }
void orc_trainer_set_hidden(void* h, uint32_t hidden) { static_cast<Trainer*>(h)->set_hidden(hidden); }
void orc_trainer_set_actor_obs(void* h, uint32_t d) { static_cast<Trainer*>(h)->set_actor_obs(d); }
void orc_trainer_set_camera(void* h, uint32_t profile_id) {
    const MdnCameraProfile c = mdn::camera_profile(profile_id);
    static_cast<Trainer*>(h)->set_camera(c.tan_v, c.mount_x_m);
}
void orc_guidance(const float* cur, const float* prev, const float* goal, float distance, const float* vel,
                  float sensor_dt, float* hint) {
    orc::nav_guidance(cur, prev, goal, distance, vel, sensor_dt, MDN_SENSOR_TAN_V, hint);
}
void orc_memory_clearance(const float* direction, const float* range_ring, const float* pose_ring, const float* pose,
                          uint32_t latest_frame, uint32_t valid_frames, float sensor_dt, float* out) {
    *out = orc::nav_memory_clearance(direction, range_ring, pose_ring, pose, latest_frame, valid_frames, sensor_dt,
                                     MDN_SENSOR_TAN_V);
}
void orc_guidance_memory(const float* cur, const float* prev, const float* goal, float distance, const float* vel,
                         float sensor_dt, const float* range_ring, const float* pose_ring, const float* pose,
                         uint32_t latest_frame, uint32_t valid_frames, float* hint) {
    orc::nav_guidance_memory(cur, prev, goal, distance, vel, sensor_dt, MDN_SENSOR_TAN_V, range_ring, pose_ring, pose,
                             latest_frame, valid_frames, hint);
}
void orc_trainer_set_runtime(void* h, const MdnRuntimeConfig* r) { static_cast<Trainer*>(h)->runtime = *r; }
void orc_trainer_set_tasks(void* h, const MdnTaskControl* t) { static_cast<Trainer*>(h)->tasks = *t; }
void orc_trainer_reset(void* h) { static_cast<Trainer*>(h)->reset_all(); }
void orc_trainer_set_bank(void* h, const MdnWorld* worlds, uint32_t count, const uint32_t* schedule, uint32_t stride) {
    Trainer* t = static_cast<Trainer*>(h);
    t->bank.enabled = count > 0 ? 1u : 0u;
    t->bank.bank_count = count;
    t->bank.schedule_stride = stride;
    t->bank.horizon = t->horizon;
    t->bank_worlds.assign(worlds, worlds + count);
    t->bank_schedule.assign(schedule, schedule + size_t(t->cfg.n) * stride);
}
// standalone operators of the dynamics draw and the task generator
int orc_sample_domain(const MdnPhysicsParams* nominal, uint32_t* rng, float amplitude, const MdnDomainRange* range,
                      MdnPhysicsParams* varied, float* sample) {
    orc::DomainSample s;
    std::memset(&s, 0, sizeof(s));
    const bool ok = orc::sample_domain(*nominal, *rng, amplitude, *range, *varied, s);
    std::memcpy(sample, &s, sizeof(s));
    return ok ? 1 : 0;
}
uint32_t orc_domain_episode_seed(const MdnRuntimeConfig* r, uint32_t cfg_seed, uint32_t env, uint32_t episode) {
    return orc::domain_episode_seed(*r, cfg_seed, env, episode);
}
void orc_domain_stress_range(MdnDomainRange* r) { *r = orc::domain_stress_range(); }
int orc_task_default_config(MdnTaskConfig* c, uint32_t stage, uint32_t family, float difficulty) {
    return orc::task_default_config(*c, stage, family, difficulty) ? 1 : 0;
}
int orc_task_settings(MdnTaskControl* t, uint32_t stage, uint32_t family) {
    bool ok = false;
    *t = orc::task_settings(stage, family, ok);
    return ok ? 1 : 0;
}
uint32_t orc_generate_task(MdnWorld* w, MdnTaskState* t, uint32_t* rng, const MdnTaskConfig* c) {
    return orc::generate_task(*w, *t, *rng, *c);
}
void orc_task_step(MdnTaskState* t, const MdnTaskConfig* c, const float* pos, const float* vel, const float* executed,
                   uint32_t contact, uint32_t forced_timeout, float* out) {
    const orc::TaskStep r = orc::task_step(*t, *c, pos, vel, executed, contact, forced_timeout);
    out[0] = r.reward; out[1] = r.goal_distance; out[2] = r.speed;
    out[3] = float(r.waypoint_passed); out[4] = float(r.stable_success); out[5] = float(r.collision);
    out[6] = float(r.timeout); out[7] = float(r.done);
}
void orc_trainer_evaluate(void* h) { static_cast<Trainer*>(h)->evaluate(); }
void orc_trainer_set_ext_means(void* h, const float* means) { static_cast<Trainer*>(h)->ext_means = means; }
uint64_t orc_trainer_optimizer_step(void* h) { return static_cast<Trainer*>(h)->optimizer_step; }
void orc_trainer_set_optimizer_step(void* h, uint64_t step) { static_cast<Trainer*>(h)->optimizer_step = step; }
void orc_trainer_metric_mean(void* h, float* out) {
    for (int k = 0; k < 4; k++) out[k] = static_cast<Trainer*>(h)->metric_mean[k];
}

// Buffer ids match the HIP library (mdnav.h MDN_BUF_*).
void* orc_trainer_buffer(void* hp, uint32_t id, uint64_t* bytes) {
    Trainer* t = static_cast<Trainer*>(hp);
    auto ret = [&](auto& v) -> void* {
        *bytes = v.size() * sizeof(v[0]);
        return v.data();
    };
    switch (id) {
        case 0: return ret(t->states);
        case 1: return ret(t->runs);
        case 2: return ret(t->worlds);
        case 3: return ret(t->sensors);
        case 4: return ret(t->poses);
        case 5: return ret(t->commands);
        case 6: return ret(t->actor);
        case 7: return ret(t->critic);
        case 8: return ret(t->obs);
        case 9: return ret(t->co);
        case 10: return ret(t->actions);
        case 11: return ret(t->logp);
        case 12: return ret(t->values);
        case 13: return ret(t->rewards);
        case 14: return ret(t->next_values);
        case 15: return ret(t->terminated);
        case 16: return ret(t->truncated);
        case 17: return ret(t->advantages);
        case 18: return ret(t->returns);
        case 19: return ret(t->actor_m);
        case 20: return ret(t->actor_v);
        case 21: return ret(t->critic_m);
        case 22: return ret(t->critic_v);
        case 23: return ret(t->metric_rows);
        case 24: return ret(t->nco);
        case 25: return ret(t->env_physics);
        case 26: return ret(t->task_states);
        case 27: return ret(t->bank_active);
        case 28: return ret(t->bank_transition);
        case 29: return ret(t->bank_schedule);
        case 30: return ret(t->grad_norm_rows);
        default: *bytes = 0; return nullptr;
    }
}

// ---- standalone operators (fixtures and closed-form checks) ----
void orc_physics_step_batch(const MdnPhysicsState* s, const float* actions, const float* winds,
                            const MdnPhysicsParams* p, MdnPhysicsState* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) orc::physics_step(s[i], actions + 4 * i, winds + 3 * i, *p, out[i]);
}
void orc_raptor_sequence(const MdnRaptorWeights* w, const float* obs, uint32_t steps, float* actions,
                         float* hidden_out) {
    float h[16];
    orc::raptor_reset(*w, h);
    for (uint32_t t = 0; t < steps; t++) orc::raptor_forward(*w, obs + 22 * t, h, actions + 4 * t);
    for (int j = 0; j < 16; j++) hidden_out[j] = h[j];
}
void orc_generate_world(MdnWorld* w, uint32_t seed, uint32_t family, float distance) {
    std::memset(w, 0, sizeof(*w));
    orc::generate_world(*w, seed, family, distance);
}
// rays: origin[3] + dir[3] per ray; world per ray index/worlds_per
void orc_ray_world_batch(const MdnWorld* worlds, const float* rays, const float* times, uint32_t rays_per_world,
                         float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        const MdnWorld& w = worlds[i / rays_per_world];
        const float* r = rays + 6 * i;
        out[i] = orc::ray_world(w, orc::v3(r[0], r[1], r[2]), orc::v3(r[3], r[4], r[5]), times[i / rays_per_world]);
    }
}
void orc_atan2_batch(const float* y, const float* x, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) out[i] = mdn::atan2_f(y[i], x[i]);
}
// sim.metal:233: the guided evaluation modes' means for one 184-input row
void orc_guided_mode_means(uint32_t mode, const float* obs, float* mean) { orc::Trainer::guided_mode_means(mode, obs, mean); }
void orc_obstacle_center(const MdnWorld* w, uint32_t i, float t, float* out) {
    const orc::V3 c = orc::obstacle_center(w->obstacles[i], t);
    out[0] = c.x; out[1] = c.y; out[2] = c.z;
}
void orc_clearance_batch(const MdnWorld* worlds, const float* points, const float* times, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++)
        out[i] = orc::clearance(worlds[i], orc::v3(points[3 * i], points[3 * i + 1], points[3 * i + 2]), times[i]);
}
float orc_ray_box(const float* p, const float* d, const float* c, const float* e) {
    return orc::ray_box(orc::v3(p[0], p[1], p[2]), orc::ray_inverse(orc::v3(d[0], d[1], d[2])),
                        orc::v3(c[0], c[1], c[2]), orc::v3(e[0], e[1], e[2]));
}
float orc_ray_sphere(const float* p, const float* d, const float* c, float r) {
    return orc::ray_sphere(orc::v3(p[0], p[1], p[2]), orc::v3(d[0], d[1], d[2]), orc::v3(c[0], c[1], c[2]), r);
}
float orc_ray_cylinder(const float* p, const float* d, const float* c, float r, float h) {
    return orc::ray_cylinder(orc::v3(p[0], p[1], p[2]), orc::v3(d[0], d[1], d[2]), orc::v3(c[0], c[1], c[2]), r, h);
}
void orc_camera_rays(float* out) {
    for (uint32_t k = 0; k < MDN_SENSOR_PIXELS; k++) {
        const orc::V3 r = orc::camera_ray(k);
        out[3 * k] = r.x; out[3 * k + 1] = r.y; out[3 * k + 2] = r.z;
    }
}
void orc_camera_rays_tan(float tan_v, float* out) {
    for (uint32_t k = 0; k < MDN_SENSOR_PIXELS; k++) {
        const orc::V3 r = orc::camera_ray(k, tan_v);
        out[3 * k] = r.x; out[3 * k + 1] = r.y; out[3 * k + 2] = r.z;
    }
}
void orc_math_batch(uint32_t fn, const float* x, float* y, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        switch (fn) {
            case 0: y[i] = mdn::exp_f(x[i]); break;
            case 1: y[i] = mdn::log_f(x[i]); break;
            case 2: y[i] = mdn::sin_f(x[i]); break;
            case 3: y[i] = mdn::cos_f(x[i]); break;
            case 4: y[i] = mdn::tanh_f(x[i]); break;
            case 5: y[i] = mdn::expm1_f(x[i]); break;
            case 6: y[i] = mdn::sigmoid_f(x[i]); break;
            default: y[i] = 0; break;
        }
    }
}
void orc_compute_gae(uint32_t horizon, uint32_t n, const float* r, const float* v, const float* nv,
                     const uint8_t* te, const uint8_t* tr, float gamma, float lambda, float* adv, float* ret) {
    orc::compute_gae(horizon, n, r, v, nv, te, tr, gamma, lambda, adv, ret);
}
void orc_normalize_advantages(float* a, uint64_t count, float eps) { orc::normalize_advantages(a, count, eps); }
float orc_squared_norm(const float* g, uint64_t count) { return orc::squared_norm(g, count); }
void orc_sample_loss_and_grad(const float* action, const float* mean, const float* log_std, float old_logp,
                              float value, float advantage, float target, float batch, float clip, float vcoef,
                              float ecoef, float* d_mean, float* d_log_std, float* d_value, float* losses4) {
    const orc::Loss l = orc::sample_loss_and_grad(action, mean, log_std, old_logp, value, advantage, target, batch,
                                                  clip, vcoef, ecoef, d_mean, d_log_std, d_value);
    losses4[0] = l.policy; losses4[1] = l.value; losses4[2] = l.entropy; losses4[3] = l.ratio;
}
void orc_actor_forward_batch(const float* params, const float* obs, uint32_t obs_dim, uint32_t hidden_dim,
                             uint64_t batch, float* hidden, float* means) {
    mdn::PolicyShape s;
    s.obs = obs_dim;
    s.hidden = hidden_dim;
    for (uint64_t n = 0; n < batch; n++)
        orc::actor_forward(s, params, obs + n * obs_dim, hidden + n * hidden_dim, means + n * 4);
}
void orc_critic_forward_batch(const float* params, const float* obs, uint64_t batch, float* hidden, float* values) {
    mdn::PolicyShape s;
    for (uint64_t n = 0; n < batch; n++) values[n] = orc::critic_forward(s, params, obs + n * 32, hidden + n * 64);
}
void orc_init_policy(float* actor, float* critic) {
    mdn::PolicyShape s;
    mdn::init_policy(s, actor, critic);
}
void orc_minibatch_schedule(uint32_t rows, uint32_t minibatch, uint32_t epochs, uint32_t rollout, uint32_t* out) {
    const auto v = mdn::minibatch_schedule(rows, minibatch, epochs, rollout);
    std::copy(v.begin(), v.end(), out);
}
// fixed_ppo::adam_update (ppo.hpp:310-324) with weight decay; bias
// corrections 1 - beta^step in float as the reference computes them.
void orc_adam_update(float* p, const float* g, float* m, float* v, uint64_t n, uint64_t step, float lr, float b1,
                     float b2, float eps, float wd) {
    float c1 = 0.0f, c2 = 0.0f;
    mdn::adam_corrections(step, b1, b2, &c1, &c2);
    for (uint64_t i = 0; i < n; i++) {
        const float gi = g[i] + wd * p[i];
        m[i] = b1 * m[i] + (1.0f - b1) * gi;
        v[i] = b2 * v[i] + (1.0f - b2) * gi * gi;
        p[i] -= lr * (m[i] / c1) / (mdn::sqrt_f(v[i] / c2) + eps);
    }
}
float orc_step_reward(float before, float after, float step_clearance, float risk_coef, int success, int collision) {
    return orc::step_reward(before, after, step_clearance, risk_coef, success != 0, collision != 0);
}
void orc_critic_observation(const MdnPhysicsState* s, const MdnWorld* w, const MdnSimRun* run, float* out) {
    orc::Trainer::critic_observation(*s, *w, *run, out);
}
void orc_crazyflie_params(MdnPhysicsParams* p) { *p = mdn::crazyflie_params(); }
void orc_default_config(MdnSimConfig* c) { *c = mdn::default_config(); }
int orc_num_threads() { return omp_get_max_threads(); }
void orc_set_num_threads(int n) { omp_set_num_threads(n); }

} // extern "C"
