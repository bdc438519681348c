/*
 * mdnav.hpp — header-only C++ façade over the C ABI (mdnav.h) that restores
 * the reference's host interfaces:
 *   mdnav::Sim         ~ Sim (main.mm:516-603)
 *   mdnav::PPOTrainer  ~ PPOTrainer (main.mm:1110-1474)
 *   mdnav::Trainer     ~ cpu_reference::Trainer (cpu_reference.hpp:112-615),
 *                        same constructor and run() -> Metrics, on the GPU.
 *   mdnav::navigation_training ~ navigation_training (navigation_training.hpp):
 *                        task_settings, configure, validate_rollout, load_actor,
 *                        evaluate, train.
 * Non-zero status codes become std::runtime_error, the reference's require()
 * convention (main.mm:27).  The reference exposes shared buffers as public
 * members; here they are methods returning host copies (sim.states() for
 * sim.states.contents).
 */
#ifndef MDNAV_HPP
#define MDNAV_HPP

#include <algorithm>
#include <array>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "mdnav.h"
#include "mdnav_host.h"

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

    // Sim::report (main.mm:599-602): episode totals of every env, printed as
    // the reference prints them (and returned).
    std::string report(const std::string& label, double wall) {
        const std::vector<MdnSimRun> r = runs();
        uint64_t success = 0, collision = 0, timeout = 0, ep = 0;
        double time = 0, path = 0, total = 0, progress = 0;
        float clearance = 12, peak = 0;
        for (const MdnSimRun& x : r) {
            success += x.successes; collision += x.collisions; timeout += x.timeouts; ep += x.episodes;
            time += x.success_time; path += x.total_path; total += x.total_elapsed; progress += x.final_progress;
            clearance = std::fmin(clearance, x.min_clearance);
            peak = std::fmax(peak, x.peak_speed);
        }
        std::ostringstream line;
        line << label << " episodes=" << ep << " success=" << (ep ? double(success) / ep : 0)
             << " collision=" << (ep ? double(collision) / ep : 0) << " timeout=" << (ep ? double(timeout) / ep : 0)
             << " progress=" << (ep ? progress / ep : 0) << " mean_goal_time=" << (success ? time / success : 0)
             << " mean_speed=" << (total ? path / total : 0) << " peak_speed=" << peak
             << " min_clearance=" << clearance << " wall_s=" << wall << "\n";
        std::cout << line.str();
        return line.str();
    }

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
    // PPOTrainer::grad_norm_summary (main.mm:1443-1465); throws on a
    // non-finite pre-clip norm like the reference's require.
    using GradNormSummary = MdnGradNormSummary;
    GradNormSummary grad_norm_summary() const {
        GradNormSummary s{};
        require(mdn_ppo_grad_norm_summary(handle_, &s));
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

    // Trainer::validate_batched_forward (cpu_reference.hpp:187-208): the
    // batched forward of the current actor and critic (on the GPU, over three
    // synthetic rows obs[i] = 0.2 sin(0.0037 i), critic obs[i] = 0.3 cos(0.17 i))
    // against the scalar fixed_ppo forward of each row (ppo.hpp:65-93); true
    // when hidden activations, means and values agree within `tolerance`.
    bool validate_batched_forward(float tolerance = 2.0e-5f) {
        constexpr uint32_t b = 3, H = MDN_HIDDEN, A = MDN_ACTIONS, C = MDN_CRITIC_OBS;
        uint32_t D = 0;
        require(mdn_sim_get_actor_obs(sim.handle(), &D));
        const std::vector<float> actor = sim.actor(), critic = sim.critic();
        std::vector<float> obs(size_t(b) * D), co(size_t(b) * C);
        for (size_t i = 0; i < obs.size(); i++) obs[i] = .2f * std::sin(float(i) * .0037f);
        for (size_t i = 0; i < co.size(); i++) co[i] = .3f * std::cos(float(i) * .17f);
        std::vector<float> ah(size_t(b) * H), am(size_t(b) * A), ch(size_t(b) * H), cv(b);
        require(mdn_op_actor_forward(actor.data(), D, H, obs.data(), b, ah.data(), am.data()));
        require(mdn_op_critic_forward(critic.data(), C, H, co.data(), b, ch.data(), cv.data()));
        float error = 0.0f;
        std::vector<float> h(H);
        for (uint32_t n = 0; n < b; n++) {
            const float* x = obs.data() + size_t(n) * D;
            for (uint32_t j = 0; j < H; j++) {  // ppo.hpp:66-72
                float z = actor[size_t(H) * D + j];
                for (uint32_t i = 0; i < D; i++) z += actor[size_t(j) * D + i] * x[i];
                h[j] = std::tanh(z);
                error = std::max(error, std::fabs(h[j] - ah[size_t(n) * H + j]));
            }
            for (uint32_t a = 0; a < A; a++) {  // ppo.hpp:73-79, the hint of a 184-input actor
                float z = actor[size_t(H) * D + H + size_t(A) * H + a];
                for (uint32_t j = 0; j < H; j++) z += actor[size_t(H) * D + H + size_t(a) * H + j] * h[j];
                if (D == MDN_ACTOR_OBS_PRIOR && a < 3) z += x[D - 3 + a];
                error = std::max(error, std::fabs(z - am[size_t(n) * A + a]));
            }
            const float* c = co.data() + size_t(n) * C;
            float value = critic[size_t(H) * C + 2 * H];
            for (uint32_t j = 0; j < H; j++) {  // ppo.hpp:82-93
                float z = critic[size_t(H) * C + j];
                for (uint32_t i = 0; i < C; i++) z += critic[size_t(j) * C + i] * c[i];
                h[j] = std::tanh(z);
                error = std::max(error, std::fabs(h[j] - ch[size_t(n) * H + j]));
            }
            for (uint32_t j = 0; j < H; j++) value += critic[size_t(H) * C + H + j] * h[j];
            error = std::max(error, std::fabs(value - cv[n]));
        }
        return error <= tolerance;
    }

    Sim sim;
    PPOTrainer ppo;
};

// The reference's Sim constructor loads the RAPTOR controller and the nominal
// plant itself (main.mm:531) and its free functions take a Metal&; here the
// controller and plant travel in this context instead.
struct Context {
    MdnRaptorWeights raptor;
    MdnPhysicsParams physics;
};

// navigation_training (navigation_training.hpp:5-173): goal-conditioned task
// set-up, validation, evaluation and the task-training loop, on the C ABI.
namespace navigation_training {

inline void require_that(bool ok, const std::string& message) {
    if (!ok) throw std::runtime_error(message);
}

// task_settings (navigation_training.hpp:7-14): the stage's default task with
// the training's time cost, smoothness weight and initial-speed cap.
inline MdnTaskControl task_settings(uint32_t stage, uint32_t family) {
    MdnTaskControl t{};
    t.enabled = 1;
    if (mdn_task_default_config(stage, family, .5f, &t.config) != MDN_OK)
        throw std::runtime_error("unsupported task stage/family");
    t.config.time_cost_per_s = .2f;
    t.config.command_smoothness_weight = .05f;
    t.config.initial_speed_max_mps = stage == 1 ? .5f : 1.0f;
    return t;
}

// configure (navigation_training.hpp:16-25): per-episode plants with the
// stress range and seed 0x3f84d5b5 at `amplitude`, the tasks, then a reset.
inline void configure(Sim& sim, const MdnTaskControl& tasks, float amplitude) {
    require_that(std::isfinite(amplitude) && amplitude >= 0.0f && amplitude <= 1.0f, "domain amplitude must be0..1");
    require_that(std::fabs(tasks.config.nav_period_s - float(sim.cfg.substeps) * .01f) < 1e-6f,
                 "task/simulator clock mismatch");
    MdnBankControl bank{};
    require(mdn_sim_get_bank(sim.handle(), &bank));
    require_that(bank.enabled == 0, "task generator and frozen bank cannot both own the world");
    MdnRuntimeConfig r{};
    r.enabled = 1;
    r.domain_amplitude = amplitude;
    r.domain_seed = 0x3f84d5b5u;
    require(mdn_domain_stress_range(&r.domain_range));
    sim.set_runtime(r);
    sim.set_tasks(tasks);
    sim.reset();
}

// validate_rollout (navigation_training.hpp:27-35).
inline void validate_rollout(Sim& sim) {
    if (mdn_sim_validate_rollout(sim.handle()) != MDN_OK) throw std::runtime_error(mdn_last_error());
}

// load_actor (navigation_training.hpp:37-62): a checkpoint's actor (and
// critic) as the sim's parameters.  The 32-to-64-input critic migration of
// the reference's control-state build has no counterpart: its critic takes
// 32 inputs here, so another critic size is an incompatible warm start.
inline void load_actor(Sim& sim, const std::string& path, bool critic = false) {
    MdnCheckpointHeader header{};
    if (mdn_checkpoint_read_params(path.c_str(), &header, nullptr, 0, nullptr, 0) != MDN_OK)
        throw std::runtime_error(mdn_last_error());
    std::vector<float> actor = sim.actor(), crit = sim.critic();
    require_that(header.actor_count == actor.size(), "task actor dimensions");
    require_that(!critic || header.critic_count == crit.size(), "task critic dimensions: incompatible warmstart");
    if (mdn_checkpoint_read_params(path.c_str(), &header, actor.data(), actor.size(), critic ? crit.data() : nullptr,
                                   critic ? crit.size() : 0) != MDN_OK)
        throw std::runtime_error("task parameter load failed");
    sim.upload(MDN_BUF_ACTOR, actor);
    if (critic) sim.upload(MDN_BUF_CRITIC, crit);
}

struct Score {
    double success = 0, collision = 0, timeout = 0, successful_time_s = 0;
};

// evaluate (navigation_training.hpp:68-115): 128 tasks of one stage and
// family with per-episode plants at `amplitude`, one episode each over 400
// ticks in `mode` (17: the deployed action map) with the geometry memory;
// the score, and the per-env task CSV when `output` is given.
inline Score evaluate(const Context& ctx, const float* actor, uint32_t stage, uint32_t family, float amplitude,
                      uint32_t seed, const std::string& output = "", uint32_t mode = 17) {
    MdnSimConfig config = mdn::default_config();
    config.n = 128; config.eval = 1; config.mode = mode; config.seed = seed; config.family = family;
    config.speed = 1.5f; config.distance = 8; config.max_steps = 400; config.geometry_memory = 1;
    Sim sim(config, 32, ctx.raptor, ctx.physics);
    sim.set_actor_obs(184);
    const MdnTaskControl settings = task_settings(stage, family);
    configure(sim, settings, amplitude);
    std::vector<float> a = sim.actor();
    std::copy(actor, actor + a.size(), a.begin());
    sim.upload(MDN_BUF_ACTOR, a);
    validate_rollout(sim);
    const std::vector<MdnTaskState> tasks = sim.download<MdnTaskState>(MDN_BUF_TASK_STATES);
    sim.collect(400);
    sim.finish();
    validate_rollout(sim);
    std::ofstream file;
    if (!output.empty()) {
        const std::filesystem::path destination(output);
        if (destination.has_parent_path()) std::filesystem::create_directories(destination.parent_path());
        file.open(output);
        require_that(bool(file), "cannot write task evaluation");
        file << "seed,env,stage,family,mode,domain_amplitude,start_x,start_y,start_z,start_yaw,initial_vx,"
                "initial_vy,initial_vz,goal_x,goal_y,goal_z,initial_distance_m,direct_clearance_m,"
                "witness_length_m,mass_kg,success,collision,timeout,time_s,path_m,goal_error_m,final_speed_mps,"
                "hold_s,peak_speed_mps,min_sphere_clearance_m,success_rule\n";
    }
    Score result;
    const std::vector<MdnSimRun> runs = sim.runs();
    const std::vector<MdnPhysicsState> states = sim.states();
    const std::vector<MdnTaskState> final_tasks = sim.download<MdnTaskState>(MDN_BUF_TASK_STATES);
    const std::vector<MdnPhysicsParams> plants = sim.download<MdnPhysicsParams>(MDN_BUF_ENV_PHYSICS);
    for (uint32_t env = 0; env < config.n; env++) {
        const MdnSimRun& run = runs[env];
        const MdnTaskState& task = tasks[env];
        const MdnPhysicsState& state = states[env];
        require_that(run.episodes == 1, "evaluation must complete exactly one task per environment");
        result.success += run.successes;
        result.collision += run.collisions;
        result.timeout += run.timeouts;
        result.successful_time_s += run.success_time;
        const float dx = task.goal_position[0] - state.position[0], dy = task.goal_position[1] - state.position[1],
                    dz = task.goal_position[2] - state.position[2];
        const float error = std::sqrt(dx * dx + dy * dy + dz * dz);
        const float* v = state.linear_velocity;
        const float speed = std::sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
        if (run.successes)
            require_that(error <= settings.config.goal_radius_m + 1e-5f &&
                             speed <= settings.config.stable_speed_mps + 1e-5f &&
                             final_tasks[env].stable_time_s >= .2f - 1e-6f,
                         "stable-arrival invariant failed");
        if (file.is_open()) {
            file << seed << ',' << env << ',' << stage << ',' << task.family << ',' << mode << ',' << amplitude;
            for (float x : task.start_position) file << ',' << x;
            file << ',' << task.start_yaw_rad;
            for (float x : task.start_velocity_world) file << ',' << x;
            for (float x : task.goal_position) file << ',' << x;
            file << ',' << task.initial_distance_m << ',' << task.direct_segment_clearance_m << ','
                 << task.witness_length_m << ',' << plants[env].mass << ',' << run.successes << ','
                 << run.collisions << ',' << run.timeouts << ',' << run.elapsed << ',' << run.path << ',' << error
                 << ',' << speed << ',' << final_tasks[env].stable_time_s << ',' << run.peak_speed << ','
                 << run.min_clearance << ",radius0.35_speed0.5_hold0.2\n";
        }
    }
    result.success /= config.n;
    result.collision /= config.n;
    result.timeout /= config.n;
    if (result.success > 0) result.successful_time_s /= result.success * config.n;
    std::cout << "task_eval stage=" << stage << " family=" << family << " seed=" << seed << " amplitude=" << amplitude
              << " mode=" << mode << " success=" << result.success << " collision=" << result.collision
              << " timeout=" << result.timeout << " mean_arrival_s=" << result.successful_time_s << "\n";
    return result;
}

// train (navigation_training.hpp:117-171): goal-arrival PPO on 128 envs x 32
// ticks in mode 22 with per-episode plants; resumes `checkpoint` when it
// exists, else warm-starts from `warmstart` with log-std -1; validates every
// rollout before its update; every 50 rollouts (and at the end) saves the
// checkpoint, evaluates on seed 800001 and keeps the best by success, then
// collisions, then arrival time; appends to `checkpoint`.history.csv.
inline void train(const Context& ctx, uint32_t rollouts, const std::string& checkpoint, const std::string& warmstart,
                  uint32_t stage, uint32_t family, float amplitude, uint32_t seed) {
    require_that(rollouts > 0, "task training requires positive rollouts and guided build");
    MdnSimConfig config = mdn::default_config();
    config.n = 128; config.mode = 22; config.family = family; config.seed = seed;
    config.speed = 1.5f; config.distance = 8; config.max_steps = 400; config.geometry_memory = 1;
    config.entropy_coef = .001f; config.learning_rate = .0001f;
    Sim sim(config, 32, ctx.raptor, ctx.physics);
    sim.set_actor_obs(184);
    const MdnTaskControl settings = task_settings(stage, family);
    configure(sim, settings, amplitude);
    PPOTrainer trainer(sim);
    const bool resume = std::filesystem::exists(checkpoint);
    uint32_t completed = 0;
    if (resume) {
        completed = trainer.load_checkpoint(checkpoint, family, 32, config.n, seed);
    } else {
        load_actor(sim, warmstart, true);
        std::vector<float> a = sim.actor();
        for (size_t axis = 0; axis < 4; axis++) a[a.size() - 4 + axis] = -1.0f;
        sim.upload(MDN_BUF_ACTOR, a);
    }
    validate_rollout(sim);
    const std::filesystem::path path(checkpoint);
    if (path.has_parent_path()) std::filesystem::create_directories(path.parent_path());
    std::ofstream history(checkpoint + ".history.csv", std::ios::app);
    require_that(bool(history), "task history write");
    if (!resume)
        history << "rollout,total_transitions,wall_s,collect_gpu_s,update_gpu_s,policy_loss,value_loss,ratio,"
                   "success,collision,timeout,mean_arrival_s\n";
    const auto start = std::chrono::steady_clock::now();
    const auto wall = [&] { return std::chrono::duration<double>(std::chrono::steady_clock::now() - start).count(); };
    const uint32_t finish = completed + rollouts;
    const auto evaluate_current = [&](const std::string& output) {
        const std::vector<float> a = sim.actor();
        return evaluate(ctx, a.data(), stage, family, amplitude, 800001, output);
    };
    Score best;
    if (resume && std::filesystem::exists(checkpoint + ".best")) {
        Sim selected(config, 32, ctx.raptor, ctx.physics);
        selected.set_actor_obs(184);
        load_actor(selected, checkpoint + ".best");
        const std::vector<float> a = selected.actor();
        best = evaluate(ctx, a.data(), stage, family, amplitude, 800001);
    }
    if (!resume) {
        const Score baseline = evaluate_current(checkpoint + ".initial-dev.csv");
        best = baseline;
        trainer.save_checkpoint(checkpoint + ".best", family, seed, completed);
        history << 0 << ",0,0,0,0,0,0,1," << baseline.success << ',' << baseline.collision << ','
                << baseline.timeout << ',' << baseline.successful_time_s << '\n';
        history.flush();
    }
    for (uint32_t rollout = completed; rollout < finish; rollout++) {
        // generation and dynamics errors are rejected before their transitions reach PPO
        sim.collect();
        const double collection_gpu = sim.finish();
        validate_rollout(sim);
        trainer.rollout_update(rollout);
        const double update_gpu = sim.finish();
        if ((rollout + 1) % 50 == 0 || rollout + 1 == finish) {
            trainer.save_checkpoint(checkpoint, family, seed, rollout + 1);
            const Score score = evaluate_current(checkpoint + ".dev.csv");
            if (score.success > best.success || (score.success == best.success && score.collision < best.collision) ||
                (score.success == best.success && score.collision == best.collision &&
                 score.successful_time_s < best.successful_time_s)) {
                best = score;
                trainer.save_checkpoint(checkpoint + ".best", family, seed, rollout + 1);
                std::filesystem::copy_file(checkpoint + ".dev.csv", checkpoint + ".best-dev.csv",
                                           std::filesystem::copy_options::overwrite_existing);
            }
            const std::array<float, 4> metrics = trainer.metric_mean();
            history << rollout + 1 << ',' << uint64_t(rollout + 1) * config.n * 32 << ',' << wall() << ','
                    << collection_gpu << ',' << update_gpu << ',' << metrics[0] << ',' << metrics[1] << ','
                    << metrics[3] << ',' << score.success << ',' << score.collision << ',' << score.timeout << ','
                    << score.successful_time_s << '\n';
            history.flush();
            std::cout << "task_train rollout=" << rollout + 1 << " policy_loss=" << metrics[0]
                      << " value_loss=" << metrics[1] << " ratio=" << metrics[3] << " wall_s=" << wall() << "\n";
            sim.report("train-arrival", 0);
        }
    }
}

}  // namespace navigation_training

// The reference's names at namespace scope of its own files.
using navigation_training::configure;
using navigation_training::task_settings;

}  // namespace mdnav

#endif /* MDNAV_HPP */
