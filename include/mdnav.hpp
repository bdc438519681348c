/*
 * mdnav.hpp — header-only C++ façade over the C ABI (mdnav.h) that restores
 * the reference's host interfaces:
 *   mdnav::Sim         ~ Sim (main.mm:516-603)
 *   mdnav::PPOTrainer  ~ PPOTrainer (main.mm:1110-1474)
 *   mdnav::Trainer     ~ cpu_reference::Trainer (cpu_reference.hpp:112-615),
 *                        same constructor and run() -> Metrics, on the GPU.
 * Non-zero status codes become std::runtime_error, the reference's require()
 * convention (main.mm:27).  The reference exposes shared buffers as public
 * members; here they are methods returning host copies (sim.states() for
 * sim.states.contents).
 */
#ifndef MDNAV_HPP
#define MDNAV_HPP

#include <array>
#include <chrono>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "mdnav.h"

namespace mdnav {

inline void require(int rc) {
    if (rc != MDN_OK) throw std::runtime_error(std::string("mdnav: ") + mdn_last_error());
}

class Sim {
public:
    Sim(const MdnSimConfig& config, uint32_t horizon, const MdnRaptorWeights& raptor,
        const MdnPhysicsParams& physics)
        : cfg(config), horizon(horizon) {
        require(mdn_sim_create(&config, horizon, &raptor, &physics, &handle_));
    }
    ~Sim() { mdn_sim_destroy(handle_); }
    Sim(const Sim&) = delete;
    Sim& operator=(const Sim&) = delete;

    void set_config(const MdnSimConfig& config) {
        require(mdn_sim_set_config(handle_, &config));
        cfg = config;
    }
    void reset() { require(mdn_sim_reset(handle_)); }
    // The guided build's FIXED_PPO_ACTOR_OBS_DIM = 184 (ppo.hpp:11-34), chosen at run time.
    void set_actor_obs(uint32_t d) { require(mdn_sim_set_actor_obs(handle_, d)); }
    // Sim::runtime_control / task_control (main.mm:523-537): per-episode
    // plants and navigation tasks, effective at the next reset().
    void set_runtime(const MdnRuntimeConfig& r) { require(mdn_sim_set_runtime(handle_, &r)); }
    void set_tasks(const MdnTaskControl& t) { require(mdn_sim_set_tasks(handle_, &t)); }
    // Sim::collect(cmdbuf, count): enqueue; finish() waits like Metal::finish.
    void collect(uint32_t count = 0) { require(mdn_sim_collect(handle_, count)); }
    double finish() {
        double s = 0;
        require(mdn_sim_sync(handle_, &s));
        return s;
    }

    template <class T>
    std::vector<T> download(MdnBuffer id) {
        uint64_t bytes = 0;
        require(mdn_sim_buffer_bytes(handle_, id, &bytes));
        std::vector<T> out(bytes / sizeof(T));
        require(mdn_sim_download(handle_, id, out.data(), bytes));
        return out;
    }
    template <class T>
    void upload(MdnBuffer id, const std::vector<T>& v) {
        require(mdn_sim_upload(handle_, id, v.data(), uint64_t(v.size()) * sizeof(T)));
    }
    std::vector<MdnPhysicsState> states() { return download<MdnPhysicsState>(MDN_BUF_STATES); }
    std::vector<MdnSimRun> runs() { return download<MdnSimRun>(MDN_BUF_RUNS); }
    std::vector<MdnWorld> worlds() { return download<MdnWorld>(MDN_BUF_WORLDS); }
    std::vector<float> actor() { return download<float>(MDN_BUF_ACTOR); }
    std::vector<float> critic() { return download<float>(MDN_BUF_CRITIC); }
    std::vector<float> rewards() { return download<float>(MDN_BUF_REWARDS); }

    MdnSim* handle() const { return handle_; }
    MdnSimConfig cfg;
    uint32_t horizon;

private:
    MdnSim* handle_ = nullptr;
};

class PPOTrainer {
public:
    explicit PPOTrainer(Sim& sim, uint32_t epochs = 2, uint32_t minibatch = 256) : sim_(sim) {
        require(mdn_ppo_create(sim.handle(), epochs, minibatch, &handle_));
    }
    ~PPOTrainer() { mdn_ppo_destroy(handle_); }
    PPOTrainer(const PPOTrainer&) = delete;
    PPOTrainer& operator=(const PPOTrainer&) = delete;

    void rollout_update(uint32_t rollout_index) { require(mdn_ppo_rollout_update(handle_, rollout_index)); }
    std::array<float, 4> metric_mean() {
        std::array<float, 4> m{};
        require(mdn_ppo_metric_mean(handle_, m.data()));
        return m;
    }
    uint64_t optimizer_step() const {
        uint64_t s = 0;
        require(mdn_ppo_optimizer_step(handle_, &s));
        return s;
    }
    // PPOTrainer::save_checkpoint / load_checkpoint (main.mm:1218-1317); the
    // load returns the completed rollouts (0 without a file).
    void save_checkpoint(const std::string& path, uint32_t family, uint32_t seed, uint32_t completed_rollouts) {
        require(mdn_ppo_save_checkpoint(handle_, path.c_str(), family, seed, completed_rollouts));
    }
    uint32_t load_checkpoint(const std::string& path, uint32_t family, uint32_t horizon, uint32_t n, uint32_t seed) {
        uint32_t done = 0;
        require(mdn_ppo_load_checkpoint(handle_, path.c_str(), family, horizon, n, seed, &done));
        return done;
    }

private:
    Sim& sim_;
    MdnPPO* handle_ = nullptr;
};

// nav_deployment::NavigationPolicy::load (deployment.hpp:142-166): metadata,
// the 12,104 weights of the 184-64-4 actor, the source checkpoint's hash.
struct NavigationPolicy {
    MdnNavPolicyMeta metadata{};
    std::vector<float> weights;
    uint64_t source_hash = 0;
    void load(const std::string& path) {
        weights.assign(184 * 64 + 64 + 4 * 64 + 4 + 4, 0.0f);
        require(mdn_navpol_read(path.c_str(), &metadata, weights.data(), weights.size(), &source_hash));
    }
};

// cpu_reference::Trainer on the GPU: Trainer(cfg, horizon, raptor, physics),
// run(rollouts) -> Metrics (cpu_reference.hpp:132-185).
class Trainer {
public:
    Trainer(const MdnSimConfig& config, uint32_t rollout_horizon, const MdnRaptorWeights& motor_policy,
            const MdnPhysicsParams& dynamics, uint32_t epochs = 2, uint32_t minibatch = 256)
        : sim(config, rollout_horizon, motor_policy, dynamics), ppo(sim, epochs, minibatch) {}

    MdnMetrics run(uint32_t rollouts) {
        MdnMetrics m{};
        const auto start = std::chrono::steady_clock::now();
        for (uint32_t r = 0; r < rollouts; r++) {
            sim.collect();
            ppo.rollout_update(r);
        }
        sim.finish();
        m.wall_seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count();
        m.updates = ppo.optimizer_step();
        for (const MdnSimRun& run : sim.runs()) {
            m.episodes += run.episodes; m.successes += run.successes;
            m.collisions += run.collisions; m.timeouts += run.timeouts;
            m.final_progress += run.final_progress; m.total_path += run.total_path;
            m.total_elapsed += run.total_elapsed; m.success_time += run.success_time;
        }
        const auto mean = ppo.metric_mean();
        m.policy_loss = mean[0]; m.value_loss = mean[1]; m.entropy_loss = mean[2]; m.ratio = mean[3];
        return m;
    }
    void reset_all() { sim.reset(); }

    Sim sim;
    PPOTrainer ppo;
};

// navigation_training::task_settings and configure (navigation_training.hpp:7-24):
// the stage's default task with the training's costs, and the runtime with
// the stress range and seed 0x3f84d5b5, installed before a reset.
inline MdnTaskControl task_settings(uint32_t stage, uint32_t family) {
    MdnTaskControl t{};
    t.enabled = 1;
    require(mdn_task_default_config(stage, family, .5f, &t.config));
    t.config.time_cost_per_s = .2f;
    t.config.command_smoothness_weight = .05f;
    t.config.initial_speed_max_mps = stage == 1 ? .5f : 1.0f;
    return t;
}
inline void configure(Sim& sim, const MdnTaskControl& tasks, float amplitude) {
    if (!(amplitude >= 0.0f && amplitude <= 1.0f)) throw std::runtime_error("domain amplitude must be 0..1");
    MdnRuntimeConfig r{};
    r.enabled = 1;
    r.domain_amplitude = amplitude;
    r.domain_seed = 0x3f84d5b5u;
    require(mdn_domain_stress_range(&r.domain_range));
    sim.set_runtime(r);
    sim.set_tasks(tasks);
    sim.reset();
}

}  // namespace mdnav

#endif /* MDNAV_HPP */
