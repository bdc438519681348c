// capi.hip — host side of the C ABI (include/mdnav.h).
//
// MdnSim owns the environment, rollout and policy buffers of one simulator on
// one HIP stream (the reference's Sim, main.mm:516-603); MdnPPO owns the
// optimiser state and minibatch workspaces (PPOTrainer, main.mm:1110-1474).
// Device layouts: physics state and SimRun as struct-of-arrays [word][env];
// worlds, rings and rollout rows in the reference's host layouts.  Downloads
// and uploads transpose to and from the reference's AoS structs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "kernel_args.h"
#include "mdnav.h"
#include "mdnav_host.h"

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}

#define HIP_TRY(call)                                                                    \
    do {                                                                                 \
        hipError_t e_ = (call);                                                          \
        if (e_ != hipSuccess) return fail(MDN_E_HIP, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

constexpr uint32_t OBS = MDN_ACTOR_OBS_POOLED;
constexpr uint32_t COBS = MDN_CRITIC_OBS;
constexpr uint32_t HID = MDN_HIDDEN;
constexpr uint32_t STATE_WORDS = 17, RUN_WORDS = 46, WORLD_WORDS = 169;
constexpr uint64_t kNavPolicyWeights = 184 * 64 + 64 + 4 * 64 + 4 + 4;  // deployment.hpp:26-38

template <class T>
int dev_alloc(T** p, size_t count) {
    *p = nullptr;
    if (count == 0) count = 1;
    HIP_TRY(hipMalloc(reinterpret_cast<void**>(p), count * sizeof(T)));
    HIP_TRY(hipMemset(*p, 0, count * sizeof(T)));
    return MDN_OK;
}

struct Timing {
    bool enabled = false;
    struct Pending { uint32_t id; hipEvent_t a, b; };
    std::vector<Pending> pending;
    std::vector<hipEvent_t> spare;
    double total_ms[MDN_K_COUNT] = {0};
    uint64_t launches[MDN_K_COUNT] = {0};
    hipEvent_t get() {
        if (!spare.empty()) {
            hipEvent_t e = spare.back();
            spare.pop_back();
            return e;
        }
        hipEvent_t e;
        hipEventCreate(&e);
        return e;
    }
};

}  // namespace

struct MdnSim {
    MdnSimConfig cfg;
    uint32_t horizon = 0;
    uint32_t lanes = 8;
    MdnPhysicsParams phys;
    mdn::PolicyShape shape;
    hipStream_t stream = nullptr;
    hipEvent_t sync_start = nullptr, sync_stop = nullptr;
    bool sync_open = false;
    Timing timing;
    // environment
    float* state = nullptr;
    uint32_t* run = nullptr;
    float* world = nullptr;
    float* sensors = nullptr;
    float* pool_ring = nullptr;  // [N][8][80]
    float* poses = nullptr;
    float* commands = nullptr;
    float* raptor = nullptr;
    float* camera = nullptr;
    float* cells = nullptr;     // pooled-cell directions of the guidance hint [80][3]
    MdnCameraProfile camera_profile{};  // legacy unless mdn_sim_set_camera chose native
    float* pix_rays = nullptr;  // raw-pixel directions of the geometry memory [320][3]
    uint32_t* mem_head = nullptr;  // per-env memory header [N][16]
    // per-episode plants and navigation tasks (NavigationRuntimeConfig and
    // NavigationTaskControl of the reference's Sim, main.mm:523-537)
    MdnRuntimeConfig runtime{};
    MdnTaskControl task{};
    MdnPhysicsParams* env_phys = nullptr;   // [N]
    MdnTaskState* task_states = nullptr;    // [N]
    MdnTaskConfig* task_cfg = nullptr;      // device copy of task.config
    // challenge bank (main.mm:522, 543-545)
    MdnBankControl bank{};
    float* bank_worlds = nullptr;           // [count][WORLD_WORDS]
    uint32_t* bank_schedule = nullptr;      // [N][stride]
    uint32_t* bank_active = nullptr;        // [N]
    uint32_t* bank_transition = nullptr;    // [T][N]
    uint32_t* validate_out = nullptr;       // [2] first failing env of validate_rollout
    bool episodic() const { return runtime.enabled != 0u || task.enabled != 0u || bank.enabled != 0u; }
    // policy
    float* actor = nullptr;
    float* critic = nullptr;
    float* actor_w1t = nullptr;
    float* critic_w1t = nullptr;
    // rollout rows
    float *obs = nullptr, *co = nullptr, *nco = nullptr, *actions = nullptr, *logp = nullptr, *values = nullptr;
    float *rewards = nullptr, *next_values = nullptr, *advantages = nullptr, *returns = nullptr;
    uint8_t *terminated = nullptr, *truncated = nullptr;
    MdnPPO* ppo = nullptr;

    size_t rows() const { return size_t(cfg.n) * horizon; }
    nav::RolloutArgs args(uint32_t count) const {
        nav::RolloutArgs a;
        a.state = state; a.run = run; a.world = world; a.sensors = sensors; a.pool_ring = pool_ring; a.poses = poses; a.commands = commands;
        a.raptor = raptor; a.actor = actor; a.actor_w1t = actor_w1t; a.critic = critic; a.critic_w1t = critic_w1t;
        a.camera = camera; a.cells = cells; a.obs = obs; a.co = co; a.nco = nco; a.actions = actions; a.logp = logp; a.values = values;
        a.rewards = rewards; a.next_values = next_values; a.terminated = terminated; a.truncated = truncated;
        a.cfg = cfg; a.phys = phys; a.count = count; a.horizon = horizon;
        a.recip_mass = 1.0 / double(phys.mass);  // IEEE fp64 division: the device's phys_recip values
        for (int i = 0; i < 4; i++) {
            a.recip_rise[i] = 1.0 / double(phys.rotor_time_constants_rising[i]);
            a.recip_fall[i] = 1.0 / double(phys.rotor_time_constants_falling[i]);
        }
        a.quad = mdn::quad_structure(phys) ? 1u : 0u;
        a.ext_means = nullptr; a.ext_log_std = nullptr; a.tick0 = 0; a.split = 0;
        a.sensor_dt = float(cfg.sensor_period) * phys.dt * float(cfg.substeps);
        a.mount_x = camera_profile.mount_x_m;
        a.tan_v = camera_profile.tan_v;
        a.inv_sensor_dt = 1.0 / double(std::max(a.sensor_dt, 1e-3f));
        a.mem_head = nullptr;
        a.env_phys = episodic() ? env_phys : nullptr;
        a.task_states = task_states;
        a.task_cfg = task.enabled ? task_cfg : nullptr;
        a.bank_active = bank.enabled ? bank_active : nullptr;
        a.bank_transition = bank_transition;
        return a;
    }
    nav::EpisodeArgs episode_args(bool first) const {
        nav::EpisodeArgs e;
        e.state = state; e.run = run; e.world = world; e.env_phys = env_phys; e.task_states = task_states;
        e.cfg = cfg; e.phys = phys; e.runtime = runtime; e.task = task; e.first = first ? 1u : 0u;
        e.bank_worlds = bank_worlds; e.bank_schedule = bank_schedule; e.bank_active = bank_active;
        e.bank = bank; e.slot = 0;
        return e;
    }
};

struct MdnPPO {
    MdnSim* sim = nullptr;
    uint32_t epochs = 2, minibatch = 256;
    uint64_t optimizer_step = 0;
    uint32_t updates = 0;
    float *am = nullptr, *av = nullptr, *cm = nullptr, *cv = nullptr;
    // minibatch workspaces: per-chunk partials and the reduced gradient; row
    // records of the one-chunk path (minibatches of at most 256 rows)
    float *part = nullptr, *grad = nullptr, *mb_rec = nullptr;
    double* norm_part = nullptr;
    float* norm_stats = nullptr;
    float *metric_rows = nullptr, *metric_mean = nullptr;
    float* grad_norm_rows = nullptr;  // [updates][2] pre-clip norms of the last rollout_update
};

namespace {

// Record a timed launch on the sim's stream.
template <class F>
int timed(MdnSim* s, uint32_t id, F launch) {
    hipEvent_t a = nullptr, b = nullptr;
    if (s->timing.enabled) {
        a = s->timing.get();
        b = s->timing.get();
        HIP_TRY(hipEventRecord(a, s->stream));
    }
    const hipError_t e = launch();
    if (e != hipSuccess) return fail(MDN_E_HIP, std::string("kernel launch: ") + hipGetErrorString(e));
    if (s->timing.enabled) {
        HIP_TRY(hipEventRecord(b, s->stream));
        s->timing.pending.push_back({id, a, b});
    }
    return MDN_OK;
}

int open_sync_window(MdnSim* s) {
    if (!s->sync_open) {
        HIP_TRY(hipEventRecord(s->sync_start, s->stream));
        s->sync_open = true;
    }
    return MDN_OK;
}

int refresh_transposes(MdnSim* s) {
    HIP_TRY(ppo_launch_transpose(s->actor, s->critic, s->actor_w1t, s->critic_w1t, s->shape.obs, s->stream));
    return MDN_OK;
}

int ring_slots(const MdnSimConfig& c) {
    const uint32_t need = c.sensor_delay + 2;
    return need <= 2 ? 2 : (need <= 4 ? 4 : 8);
}

struct BufInfo { void* dev; size_t bytes; };

BufInfo row_buffer(MdnSim* s, uint32_t id) {
    const size_t R = s->rows();
    switch (id) {
        case MDN_BUF_OBS: return {s->obs, R * s->shape.obs * 4};
        case MDN_BUF_CRITIC_OBS: return {s->co, R * COBS * 4};
        case MDN_BUF_NEXT_CRITIC_OBS: return {s->nco, R * COBS * 4};
        case MDN_BUF_ACTIONS: return {s->actions, R * 4 * 4};
        case MDN_BUF_LOGP: return {s->logp, R * 4};
        case MDN_BUF_VALUES: return {s->values, R * 4};
        case MDN_BUF_REWARDS: return {s->rewards, R * 4};
        case MDN_BUF_NEXT_VALUES: return {s->next_values, R * 4};
        case MDN_BUF_TERMINATED: return {s->terminated, R};
        case MDN_BUF_TRUNCATED: return {s->truncated, R};
        case MDN_BUF_ADVANTAGES: return {s->advantages, R * 4};
        case MDN_BUF_RETURNS: return {s->returns, R * 4};
        case MDN_BUF_SENSORS: return {s->sensors, size_t(s->cfg.n) * 8 * 320 * 4};
        case MDN_BUF_POSES: return {s->poses, size_t(s->cfg.n) * 96 * 4};
        case MDN_BUF_COMMANDS: return {s->commands, size_t(s->cfg.n) * 32 * 4};
        case MDN_BUF_WORLDS: return {s->world, size_t(s->cfg.n) * WORLD_WORDS * 4};
        case MDN_BUF_ACTOR: return {s->actor, size_t(s->shape.actor_count()) * 4};
        case MDN_BUF_CRITIC: return {s->critic, size_t(s->shape.critic_count()) * 4};
        case MDN_BUF_ENV_PHYSICS: return {s->env_phys, size_t(s->cfg.n) * sizeof(MdnPhysicsParams)};
        case MDN_BUF_TASK_STATES: return {s->task_states, size_t(s->cfg.n) * sizeof(MdnTaskState)};
        case MDN_BUF_BANK_ACTIVE_IDS: return {s->bank_active, size_t(s->cfg.n) * 4};
        case MDN_BUF_BANK_TRANSITION_IDS: return {s->bank_transition, R * 4};
        case MDN_BUF_BANK_SCHEDULE:
            return {s->bank_schedule, s->bank_schedule ? size_t(s->cfg.n) * s->bank.schedule_stride * 4 : 0};
        default: break;
    }
    if (s->ppo) {
        MdnPPO* p = s->ppo;
        switch (id) {
            case MDN_BUF_ACTOR_M: return {p->am, size_t(s->shape.actor_count()) * 4};
            case MDN_BUF_ACTOR_V: return {p->av, size_t(s->shape.actor_count()) * 4};
            case MDN_BUF_CRITIC_M: return {p->cm, size_t(s->shape.critic_count()) * 4};
            case MDN_BUF_CRITIC_V: return {p->cv, size_t(s->shape.critic_count()) * 4};
            case MDN_BUF_METRIC_ROWS: return {p->metric_rows, size_t(p->updates) * 16};
            case MDN_BUF_GRAD_NORM_ROWS: return {p->grad_norm_rows, size_t(p->updates) * 8};
            default: break;
        }
    }
    return {nullptr, 0};
}

}  // namespace

extern "C" {

const char* mdn_last_error(void) { return g_error.c_str(); }
const char* mdn_version(void) { return "mdnav 0.1 gfx950"; }

namespace {
// Camera tables of the sim's profile (sensor_profile.hpp:81-97,
// guidance.hpp:21-26, 122): unit pixel rays (nav_sensor_pixel_ray), the
// pooled-cell directions of the guidance hint and the raw-pixel directions
// of the geometry memory.  Synchronous copies.
int upload_camera(MdnSim* s) {
    const float tan_h = s->camera_profile.tan_h, tan_v = s->camera_profile.tan_v;
    std::vector<float> cam(960);
    for (uint32_t k = 0; k < 320; k++) {
        const uint32_t row = k / 20, col = k % 20;
        const float y = ((float(col) + 0.5f) / 20.0f * 2.0f - 1.0f) * tan_h;
        const float z = ((float(row) + 0.5f) / 16.0f * 2.0f - 1.0f) * tan_v;
        const float dx = 1.0f, dy = -y, dz = -z;
        const float len = mdn::sqrt_f(dx * dx + dy * dy + dz * dz);
        const float inv = 1.0f / mdn::fmax_f(len, 1e-8f);
        cam[3 * k] = dx * inv; cam[3 * k + 1] = dy * inv; cam[3 * k + 2] = dz * inv;
    }
    std::vector<float> cells(240);
    for (uint32_t k = 0; k < 80; k++) {
        const uint32_t row = k / 10, col = k % 10;
        const float y = 0.9f - 0.2f * float(col), z = (0.875f - 0.25f * float(row)) * tan_v;
        const float inv = 1.0f / mdn::sqrt_f(1.0f + y * y + z * z);
        cells[3 * k] = inv; cells[3 * k + 1] = y * inv; cells[3 * k + 2] = z * inv;
    }
    std::vector<float> pix(960);
    for (uint32_t hit = 0; hit < 320; hit++) {
        const float ry = 1.0f - (float(hit % 20) + .5f) / 10.0f;
        const float rz = tan_v * (1.0f - (float(hit / 20) + .5f) / 8.0f);
        const float inv = 1.0f / mdn::sqrt_f(1 + ry * ry + rz * rz);
        pix[3 * hit] = inv; pix[3 * hit + 1] = ry * inv; pix[3 * hit + 2] = rz * inv;
    }
    if (hipMemcpy(s->camera, cam.data(), cam.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(s->cells, cells.data(), cells.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(s->pix_rays, pix.data(), pix.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
        return fail(MDN_E_HIP, "camera table upload failed");
    return MDN_OK;
}
}  // namespace

int mdn_sim_create(const MdnSimConfig* cfg, uint32_t horizon, const MdnRaptorWeights* raptor,
                   const MdnPhysicsParams* physics, MdnSim** out) {
    if (!cfg || !raptor || !physics || !out) return fail(MDN_E_ARG, "mdn_sim_create: null argument");
    *out = nullptr;
    if (cfg->n == 0 || horizon == 0) return fail(MDN_E_ARG, "mdn_sim_create: n and horizon must be positive");
    if (cfg->sensor_period == 0) return fail(MDN_E_ARG, "mdn_sim_create: sensor_period must be positive");
    if (cfg->sensor_delay > 6 || cfg->command_delay > 7)
        return fail(MDN_E_ARG, "delay rings support <=6 sensor frames and <=7 command steps");
    MdnSim* s = new MdnSim();
    s->cfg = *cfg;
    s->horizon = horizon;
    s->phys = *physics;
    const uint32_t N = cfg->n;
    const size_t R = size_t(N) * horizon;
    int rc = MDN_OK;
    auto guard = [&](int r) { if (r != MDN_OK && rc == MDN_OK) rc = r; };
    guard(hipStreamCreate(&s->stream) == hipSuccess ? MDN_OK : fail(MDN_E_HIP, "hipStreamCreate failed"));
    guard(hipEventCreate(&s->sync_start) == hipSuccess ? MDN_OK : fail(MDN_E_HIP, "hipEventCreate"));
    guard(hipEventCreate(&s->sync_stop) == hipSuccess ? MDN_OK : fail(MDN_E_HIP, "hipEventCreate"));
    guard(dev_alloc(&s->state, size_t(STATE_WORDS) * N));
    guard(dev_alloc(&s->run, size_t(RUN_WORDS) * N));
    guard(dev_alloc(&s->world, size_t(WORLD_WORDS) * N));
    guard(dev_alloc(&s->sensors, size_t(N) * 8 * 320));
    guard(dev_alloc(&s->pool_ring, size_t(N) * 8 * 80));
    guard(dev_alloc(&s->poses, size_t(N) * 96));
    guard(dev_alloc(&s->commands, size_t(N) * 32));
    guard(dev_alloc(&s->raptor, 2084));
    guard(dev_alloc(&s->camera, 960));
    guard(dev_alloc(&s->cells, 240));
    guard(dev_alloc(&s->pix_rays, 960));
    guard(dev_alloc(&s->mem_head, size_t(N) * nav::MEM_HEAD_WORDS));
    guard(dev_alloc(&s->env_phys, N));
    guard(dev_alloc(&s->task_states, N));
    guard(dev_alloc(&s->task_cfg, 1));
    guard(dev_alloc(&s->bank_active, N));
    guard(dev_alloc(&s->bank_transition, R));
    guard(dev_alloc(&s->validate_out, 2));
    if (rc == MDN_OK) {  // no bank: every id is MDN_BANK_REHEARSAL (sim.metal:143, 317)
        guard(hipMemset(s->bank_active, 0xff, size_t(N) * 4) == hipSuccess ? MDN_OK : fail(MDN_E_HIP, "hipMemset"));
        guard(hipMemset(s->bank_transition, 0xff, R * 4) == hipSuccess ? MDN_OK : fail(MDN_E_HIP, "hipMemset"));
    }
    guard(dev_alloc(&s->actor, s->shape.actor_count()));
    guard(dev_alloc(&s->critic, s->shape.critic_count()));
    guard(dev_alloc(&s->actor_w1t, size_t(OBS) * HID));
    guard(dev_alloc(&s->critic_w1t, size_t(COBS) * HID));
    guard(dev_alloc(&s->obs, R * OBS));
    guard(dev_alloc(&s->co, R * COBS));
    guard(dev_alloc(&s->nco, R * COBS));
    guard(dev_alloc(&s->actions, R * 4));
    guard(dev_alloc(&s->logp, R));
    guard(dev_alloc(&s->values, R));
    guard(dev_alloc(&s->rewards, R));
    guard(dev_alloc(&s->next_values, R));
    guard(dev_alloc(&s->advantages, R));
    guard(dev_alloc(&s->returns, R));
    guard(dev_alloc(&s->terminated, R));
    guard(dev_alloc(&s->truncated, R));
    if (rc == MDN_OK && hipDeviceSynchronize() != hipSuccess) rc = fail(MDN_E_HIP, "mdn_sim_create: allocation sync");
    if (rc != MDN_OK) {
        mdn_sim_destroy(s);
        return rc;
    }
    s->camera_profile = mdn::camera_profile(MDN_CAMERA_LEGACY);
    if (upload_camera(s) != MDN_OK) {
        mdn_sim_destroy(s);
        return MDN_E_HIP;
    }
    // policy initialisation is a host computation shared with the oracle
    // (mdnav_host.h); copies are synchronous.
    std::vector<float> actor(s->shape.actor_count()), critic(s->shape.critic_count());
    mdn::init_policy(s->shape, actor.data(), critic.data());
    if (hipMemcpy(s->raptor, raptor, sizeof(MdnRaptorWeights), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(s->actor, actor.data(), actor.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(s->critic, critic.data(), critic.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
        mdn_sim_destroy(s);
        return fail(MDN_E_HIP, "mdn_sim_create: upload failed");
    }
    rc = refresh_transposes(s);
    if (rc == MDN_OK) rc = mdn_sim_reset(s);
    if (rc == MDN_OK && hipStreamSynchronize(s->stream) != hipSuccess) rc = fail(MDN_E_HIP, "mdn_sim_create: sync");
    if (rc != MDN_OK) {
        mdn_sim_destroy(s);
        return rc;
    }
    *out = s;
    return MDN_OK;
}

void mdn_sim_destroy(MdnSim* s) {
    if (!s) return;
    if (s->stream) hipStreamSynchronize(s->stream);
    if (s->ppo) mdn_ppo_destroy(s->ppo);
    void* bufs[] = {s->state, s->run, s->world, s->sensors, s->pool_ring, s->poses, s->commands, s->raptor, s->camera, s->cells,
                    s->pix_rays, s->mem_head, s->env_phys, s->task_states, s->task_cfg, s->bank_worlds,
                    s->bank_schedule, s->bank_active, s->bank_transition, s->validate_out,
                    s->actor, s->critic, s->actor_w1t, s->critic_w1t, s->obs, s->co, s->nco, s->actions, s->logp,
                    s->values, s->rewards, s->next_values, s->advantages, s->returns, s->terminated, s->truncated};
    for (void* b : bufs)
        if (b) hipFree(b);
    for (auto& p : s->timing.pending) { hipEventDestroy(p.a); hipEventDestroy(p.b); }
    for (auto e : s->timing.spare) hipEventDestroy(e);
    if (s->sync_start) hipEventDestroy(s->sync_start);
    if (s->sync_stop) hipEventDestroy(s->sync_stop);
    if (s->stream) hipStreamDestroy(s->stream);
    delete s;
}

int mdn_sim_set_config(MdnSim* s, const MdnSimConfig* cfg) {
    if (!s || !cfg) return fail(MDN_E_ARG, "mdn_sim_set_config: null argument");
    if (cfg->n != s->cfg.n) return fail(MDN_E_ARG, "cannot resize simulator");
    if (cfg->sensor_period == 0) return fail(MDN_E_ARG, "sensor_period must be positive");
    if (cfg->sensor_delay > 6 || cfg->command_delay > 7)
        return fail(MDN_E_ARG, "delay rings support <=6 sensor frames and <=7 command steps");
    s->cfg = *cfg;
    return MDN_OK;
}

int mdn_sim_get_config(const MdnSim* s, MdnSimConfig* cfg, uint32_t* horizon) {
    if (!s) return fail(MDN_E_ARG, "mdn_sim_get_config: null sim");
    if (cfg) *cfg = s->cfg;
    if (horizon) *horizon = s->horizon;
    return MDN_OK;
}

int mdn_sim_set_actor_obs(MdnSim* s, uint32_t actor_obs) {
    if (!s) return fail(MDN_E_ARG, "mdn_sim_set_actor_obs: null sim");
    if (actor_obs != MDN_ACTOR_OBS_POOLED && actor_obs != MDN_ACTOR_OBS_PRIOR)
        return fail(MDN_E_ARG, "actor inputs must be 181 (pooled) or 184 (with the geometry-prior hint)");
    if (s->ppo) return fail(MDN_E_STATE, "set the actor's inputs before creating the PPO trainer");
    HIP_TRY(hipStreamSynchronize(s->stream));
    mdn::PolicyShape shape = s->shape;
    shape.obs = actor_obs;
    float *obs = nullptr, *actor = nullptr, *w1t = nullptr;
    int rc = dev_alloc(&obs, s->rows() * actor_obs);
    if (!rc) rc = dev_alloc(&actor, shape.actor_count());
    if (!rc) rc = dev_alloc(&w1t, size_t(actor_obs) * HID);
    std::vector<float> a(shape.actor_count()), c(shape.critic_count());
    mdn::init_policy(shape, a.data(), c.data());
    if (!rc && (hipMemcpy(actor, a.data(), a.size() * 4, hipMemcpyHostToDevice) != hipSuccess ||
                hipMemcpy(s->critic, c.data(), c.size() * 4, hipMemcpyHostToDevice) != hipSuccess))
        rc = fail(MDN_E_HIP, "mdn_sim_set_actor_obs: policy upload");
    if (rc) {
        hipFree(obs); hipFree(actor); hipFree(w1t);
        return rc;
    }
    hipFree(s->obs); hipFree(s->actor); hipFree(s->actor_w1t);
    s->obs = obs; s->actor = actor; s->actor_w1t = w1t;
    s->shape = shape;
    rc = refresh_transposes(s);
    if (!rc) HIP_TRY(hipStreamSynchronize(s->stream));
    return rc;
}

int mdn_sim_get_actor_obs(const MdnSim* s, uint32_t* actor_obs) {
    if (!s || !actor_obs) return fail(MDN_E_ARG, "mdn_sim_get_actor_obs: null argument");
    *actor_obs = s->shape.obs;
    return MDN_OK;
}

int mdn_sim_set_lanes(MdnSim* s, uint32_t lanes) {
    if (!s || (lanes != 4 && lanes != 8 && lanes != 16)) return fail(MDN_E_ARG, "lanes per env must be 4, 8 or 16");
    s->lanes = lanes;
    return MDN_OK;
}

int mdn_sim_reset(MdnSim* s) {
    if (!s) return fail(MDN_E_ARG, "mdn_sim_reset: null sim");
    int rc = open_sync_window(s);
    if (rc) return rc;
    const nav::RolloutArgs a = s->args(0);
    HIP_TRY(nav_launch_reset(&a, s->stream));
    // Always, as sim_reset_one writes every env's plant (sim.metal:69): with
    // per-episode plants, tasks and banks off, the episode kernel writes the
    // nominal plant, a zero task state and the rehearsal level, so that a bank
    // or a resume set later starts from the reference's buffers.
    const nav::EpisodeArgs e = s->episode_args(true);
    HIP_TRY(nav_launch_episode(&e, s->stream));
    return MDN_OK;
}

int mdn_sim_set_camera(MdnSim* s, uint32_t profile_id) {
    if (!s) return fail(MDN_E_ARG, "mdn_sim_set_camera: null");
    if (profile_id != MDN_CAMERA_LEGACY && profile_id != MDN_CAMERA_NATIVE)
        return fail(MDN_E_ARG, "camera profile must be 1 (legacy) or 2 (native)");
    HIP_TRY(hipStreamSynchronize(s->stream));  // no launch in flight reads the tables
    s->camera_profile = mdn::camera_profile(profile_id);
    return upload_camera(s);
}

int mdn_sim_get_camera(const MdnSim* s, MdnCameraProfile* out) {
    if (!s || !out) return fail(MDN_E_ARG, "mdn_sim_get_camera: null");
    *out = s->camera_profile;
    return MDN_OK;
}

int mdn_sim_set_runtime(MdnSim* s, const MdnRuntimeConfig* runtime) {
    if (!s || !runtime) return fail(MDN_E_ARG, "mdn_sim_set_runtime: null argument");
    s->runtime = *runtime;
    return MDN_OK;
}

int mdn_sim_get_runtime(const MdnSim* s, MdnRuntimeConfig* runtime) {
    if (!s || !runtime) return fail(MDN_E_ARG, "mdn_sim_get_runtime: null argument");
    *runtime = s->runtime;
    return MDN_OK;
}

int mdn_sim_set_tasks(MdnSim* s, const MdnTaskControl* tasks) {
    if (!s || !tasks) return fail(MDN_E_ARG, "mdn_sim_set_tasks: null argument");
    if (tasks->enabled != 0u && s->bank.enabled != 0u)  // navigation_training.hpp:19
        return fail(MDN_E_ARG, "task generator and frozen bank cannot both own the world");
    int rc = open_sync_window(s);
    if (rc) return rc;
    s->task = *tasks;
    HIP_TRY(hipMemcpyAsync(s->task_cfg, &s->task.config, sizeof(MdnTaskConfig), hipMemcpyHostToDevice, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    return MDN_OK;
}

int mdn_sim_get_tasks(const MdnSim* s, MdnTaskControl* tasks) {
    if (!s || !tasks) return fail(MDN_E_ARG, "mdn_sim_get_tasks: null argument");
    *tasks = s->task;
    return MDN_OK;
}

int mdn_sim_set_bank(MdnSim* s, const MdnWorld* worlds, uint32_t count, const uint32_t* schedule,
                     uint32_t schedule_stride) {
    if (!s || (count && (!worlds || !schedule || schedule_stride == 0)))
        return fail(MDN_E_ARG, "mdn_sim_set_bank: null argument or zero schedule stride");
    if (count && s->task.enabled != 0u)  // navigation_training.hpp:19
        return fail(MDN_E_ARG, "task generator and frozen bank cannot both own the world");
    int rc = open_sync_window(s);
    if (rc) return rc;
    HIP_TRY(hipStreamSynchronize(s->stream));
    if (s->bank_worlds) HIP_TRY(hipFree(s->bank_worlds));
    if (s->bank_schedule) HIP_TRY(hipFree(s->bank_schedule));
    s->bank_worlds = nullptr;
    s->bank_schedule = nullptr;
    s->bank = MdnBankControl{};
    const size_t N = s->cfg.n;
    if (count == 0) {
        HIP_TRY(hipMemset(s->bank_active, 0xff, N * 4));
        return MDN_OK;
    }
    if ((rc = dev_alloc(&s->bank_worlds, size_t(count) * WORLD_WORDS)) != MDN_OK) return rc;
    if ((rc = dev_alloc(&s->bank_schedule, N * schedule_stride)) != MDN_OK) return rc;
    HIP_TRY(hipMemcpy(s->bank_worlds, worlds, size_t(count) * sizeof(MdnWorld), hipMemcpyHostToDevice));
    HIP_TRY(hipMemcpy(s->bank_schedule, schedule, N * schedule_stride * 4, hipMemcpyHostToDevice));
    s->bank.enabled = 1;
    s->bank.bank_count = count;
    s->bank.schedule_stride = schedule_stride;
    s->bank.horizon = s->horizon;
    return MDN_OK;
}

int mdn_sim_get_bank(const MdnSim* s, MdnBankControl* bank) {
    if (!s || !bank) return fail(MDN_E_ARG, "mdn_sim_get_bank: null argument");
    *bank = s->bank;
    return MDN_OK;
}

int mdn_task_default_config(uint32_t stage, uint32_t family, float difficulty, MdnTaskConfig* out) {
    if (!out) return fail(MDN_E_ARG, "mdn_task_default_config: null argument");
    if (!mdn::task_default_config(*out, stage, family, difficulty))
        return fail(MDN_E_ARG, "unsupported task stage/family or difficulty outside [0, 1]");
    return MDN_OK;
}

int mdn_domain_stress_range(MdnDomainRange* out) {
    if (!out) return fail(MDN_E_ARG, "mdn_domain_stress_range: null argument");
    *out = mdn::domain_stress_range();
    return MDN_OK;
}

// Per-episode plants and navigation tasks: one tick per launch.  Per tick:
// depth and observation (ending there), the geometry-memory hint if on, act
// + advance + (task step) + reset, then the episode kernel for the envs that
// were reset (sim.metal:328-331: the new episode's plant and task).
int collect_episodic(MdnSim* s, uint32_t count, int slots) {
    nav::RolloutArgs b = s->args(1);
    const bool memory = s->shape.obs == MDN_ACTOR_OBS_PRIOR && s->cfg.geometry_memory;
    if (memory) b.mem_head = s->mem_head;
    nav::MemoryArgs m;
    m.head = s->mem_head; m.sensors = s->sensors; m.poses = s->poses; m.pix_rays = s->pix_rays; m.cells = s->cells;
    m.sensor_dt = b.sensor_dt; m.inv_sensor_dt = b.inv_sensor_dt; m.n = s->cfg.n;
    m.tan_v = s->camera_profile.tan_v;
    nav::EpisodeArgs e = s->episode_args(false);
    int rc = MDN_OK;
    for (uint32_t t = 0; t < count && rc == MDN_OK; t++) {
        b.tick0 = t;
        b.count = 1;
        b.split = nav::SPLIT_END_AFTER_OBSERVE;
        rc = timed(s, MDN_K_ROLLOUT, [&] { return nav_launch_rollout(&b, 8, slots, s->shape.obs, s->stream); });
        if (rc) break;
        if (memory) {
            m.obs = s->obs + size_t(t % s->horizon) * s->cfg.n * s->shape.obs;
            rc = timed(s, MDN_K_MEMORY, [&] { return nav_launch_memory_hint(&m, s->stream); });
            if (rc) break;
        }
        b.split = nav::SPLIT_BEGIN_AT_ACT;
        rc = timed(s, MDN_K_ROLLOUT, [&] { return nav_launch_rollout(&b, 8, slots, s->shape.obs, s->stream); });
        if (rc) break;
        e.slot = t % s->horizon + 1;  // the reset at tick t takes schedule slot tick + 1
        rc = timed(s, MDN_K_EPISODE, [&] { return nav_launch_episode(&e, s->stream); });
    }
    return rc;
}

int mdn_sim_collect(MdnSim* s, uint32_t count) {
    if (!s) return fail(MDN_E_ARG, "mdn_sim_collect: null sim");
    if (count == 0) count = s->horizon;
    int rc = open_sync_window(s);
    if (rc) return rc;
    const nav::RolloutArgs a = s->args(count);
    const int lanes = int(s->lanes), slots = ring_slots(s->cfg);
    if (s->shape.obs == MDN_ACTOR_OBS_PRIOR && lanes != 8)
        return fail(MDN_E_ARG, "the 184-input actor's rollout runs 8 lanes per env");
    if (s->episodic()) {
        if (lanes != 8) return fail(MDN_E_ARG, "per-episode plants and tasks run 8 lanes per env");
        return collect_episodic(s, count, slots);
    }
    if (s->shape.obs != MDN_ACTOR_OBS_PRIOR || !s->cfg.geometry_memory)
        return timed(s, MDN_K_ROLLOUT, [&] { return nav_launch_rollout(&a, lanes, slots, s->shape.obs, s->stream); });
    // Geometry-memory hint: split ticks.  Tick 0 up to its observation; then
    // per tick: the memory kernel writes the hint of the tick's rows, and one
    // launch acts, advances, resets and observes the next tick.
    nav::RolloutArgs b = s->args(1);
    b.mem_head = s->mem_head;
    b.split = nav::SPLIT_END_AFTER_OBSERVE;
    rc = timed(s, MDN_K_ROLLOUT, [&] { return nav_launch_rollout(&b, 8, slots, s->shape.obs, s->stream); });
    nav::MemoryArgs m;
    m.head = s->mem_head; m.sensors = s->sensors; m.poses = s->poses; m.pix_rays = s->pix_rays; m.cells = s->cells;
    m.sensor_dt = b.sensor_dt; m.inv_sensor_dt = b.inv_sensor_dt; m.n = s->cfg.n;
    m.tan_v = s->camera_profile.tan_v;
    for (uint32_t t = 0; t < count && rc == MDN_OK; t++) {
        m.obs = s->obs + size_t(t % s->horizon) * s->cfg.n * s->shape.obs;
        rc = timed(s, MDN_K_MEMORY, [&] { return nav_launch_memory_hint(&m, s->stream); });
        if (rc) break;
        const bool more = t + 1 < count;
        b.count = more ? 2 : 1;
        b.tick0 = t;
        b.split = nav::SPLIT_BEGIN_AT_ACT | (more ? nav::SPLIT_END_AFTER_OBSERVE : 0u);
        rc = timed(s, MDN_K_ROLLOUT, [&] { return nav_launch_rollout(&b, 8, slots, s->shape.obs, s->stream); });
    }
    return rc;
}

int mdn_sim_sync(MdnSim* s, double* gpu_seconds) {
    if (!s) return fail(MDN_E_ARG, "mdn_sim_sync: null sim");
    double seconds = 0.0;
    if (s->sync_open) {
        HIP_TRY(hipEventRecord(s->sync_stop, s->stream));
        HIP_TRY(hipEventSynchronize(s->sync_stop));
        float ms = 0;
        HIP_TRY(hipEventElapsedTime(&ms, s->sync_start, s->sync_stop));
        seconds = ms * 1e-3;
        s->sync_open = false;
    } else {
        HIP_TRY(hipStreamSynchronize(s->stream));
    }
    for (auto& p : s->timing.pending) {
        float ms = 0;
        HIP_TRY(hipEventElapsedTime(&ms, p.a, p.b));
        s->timing.total_ms[p.id] += ms;
        s->timing.launches[p.id] += 1;
        s->timing.spare.push_back(p.a);
        s->timing.spare.push_back(p.b);
    }
    s->timing.pending.clear();
    if (gpu_seconds) *gpu_seconds = seconds;
    return MDN_OK;
}

int mdn_sim_set_timing(MdnSim* s, int enabled) {
    if (!s) return fail(MDN_E_ARG, "mdn_sim_set_timing: null sim");
    s->timing.enabled = enabled != 0;
    return MDN_OK;
}

int mdn_sim_kernel_time(MdnSim* s, uint32_t kernel, double* total_ms, uint64_t* launches) {
    if (!s || kernel >= MDN_K_COUNT) return fail(MDN_E_ARG, "mdn_sim_kernel_time: bad kernel id");
    if (total_ms) *total_ms = s->timing.total_ms[kernel];
    if (launches) *launches = s->timing.launches[kernel];
    return MDN_OK;
}

int mdn_sim_reset_timing(MdnSim* s) {
    if (!s) return fail(MDN_E_ARG, "mdn_sim_reset_timing: null sim");
    for (int i = 0; i < MDN_K_COUNT; i++) { s->timing.total_ms[i] = 0; s->timing.launches[i] = 0; }
    return MDN_OK;
}

int mdn_sim_validate_rollout(MdnSim* s) {
    if (!s) return fail(MDN_E_ARG, "mdn_sim_validate_rollout: null");
    int rc = open_sync_window(s);
    if (rc) return rc;
    uint32_t bad[2];
    HIP_TRY(nav_launch_validate(s->task_states, s->env_phys, s->cfg.n, s->validate_out, s->stream));
    HIP_TRY(hipMemcpyAsync(bad, s->validate_out, 8, hipMemcpyDeviceToHost, s->stream));
    HIP_TRY(hipStreamSynchronize(s->stream));
    if (bad[0] != 0xffffffffu) {
        MdnTaskState t;
        HIP_TRY(hipMemcpy(&t, s->task_states + bad[0], sizeof(t), hipMemcpyDeviceToHost));
        return fail(MDN_E_STATE, "task generation rejected env=" + std::to_string(bad[0]) +
                                     " status=" + std::to_string(t.generation_status));
    }
    if (bad[1] != 0xffffffffu)
        return fail(MDN_E_STATE, "episode dynamics sample rejected env=" + std::to_string(bad[1]));
    return MDN_OK;
}

int mdn_sim_buffer_bytes(const MdnSim* s, uint32_t buffer, uint64_t* bytes) {
    if (!s || !bytes) return fail(MDN_E_ARG, "mdn_sim_buffer_bytes: null argument");
    const uint32_t N = s->cfg.n;
    if (buffer == MDN_BUF_STATES) { *bytes = uint64_t(N) * sizeof(MdnPhysicsState); return MDN_OK; }
    if (buffer == MDN_BUF_RUNS) { *bytes = uint64_t(N) * sizeof(MdnSimRun); return MDN_OK; }
    const BufInfo b = row_buffer(const_cast<MdnSim*>(s), buffer);
    if (!b.dev) return fail(MDN_E_ARG, "unknown buffer id " + std::to_string(buffer) + " (Adam buffers need a PPO handle)");
    *bytes = b.bytes;
    return MDN_OK;
}

int mdn_sim_download(MdnSim* s, uint32_t buffer, void* host, uint64_t bytes) {
    uint64_t need = 0;
    int rc = mdn_sim_buffer_bytes(s, buffer, &need);
    if (rc) return rc;
    if (!host || bytes != need) return fail(MDN_E_ARG, "download size mismatch: need " + std::to_string(need));
    HIP_TRY(hipStreamSynchronize(s->stream));
    const uint32_t N = s->cfg.n;
    if (buffer == MDN_BUF_STATES || buffer == MDN_BUF_RUNS) {
        const uint32_t W = buffer == MDN_BUF_STATES ? STATE_WORDS : RUN_WORDS;
        std::vector<uint32_t> soa(size_t(W) * N);
        HIP_TRY(hipMemcpy(soa.data(), buffer == MDN_BUF_STATES ? static_cast<void*>(s->state) : static_cast<void*>(s->run),
                          soa.size() * 4, hipMemcpyDeviceToHost));
        uint32_t* aos = static_cast<uint32_t*>(host);
        for (uint32_t n = 0; n < N; n++)
            for (uint32_t w = 0; w < W; w++) aos[size_t(n) * W + w] = soa[size_t(w) * N + n];
        return MDN_OK;
    }
    const BufInfo b = row_buffer(s, buffer);
    HIP_TRY(hipMemcpy(host, b.dev, b.bytes, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_sim_upload(MdnSim* s, uint32_t buffer, const void* host, uint64_t bytes) {
    uint64_t need = 0;
    int rc = mdn_sim_buffer_bytes(s, buffer, &need);
    if (rc) return rc;
    if (!host || bytes != need) return fail(MDN_E_ARG, "upload size mismatch: need " + std::to_string(need));
    HIP_TRY(hipStreamSynchronize(s->stream));
    const uint32_t N = s->cfg.n;
    if (buffer == MDN_BUF_STATES || buffer == MDN_BUF_RUNS) {
        const uint32_t W = buffer == MDN_BUF_STATES ? STATE_WORDS : RUN_WORDS;
        std::vector<uint32_t> soa(size_t(W) * N);
        const uint32_t* aos = static_cast<const uint32_t*>(host);
        for (uint32_t n = 0; n < N; n++)
            for (uint32_t w = 0; w < W; w++) soa[size_t(w) * N + n] = aos[size_t(n) * W + w];
        HIP_TRY(hipMemcpy(buffer == MDN_BUF_STATES ? static_cast<void*>(s->state) : static_cast<void*>(s->run), soa.data(),
                          soa.size() * 4, hipMemcpyHostToDevice));
        return MDN_OK;
    }
    const BufInfo b = row_buffer(s, buffer);
    HIP_TRY(hipMemcpy(b.dev, host, b.bytes, hipMemcpyHostToDevice));
    if (buffer == MDN_BUF_ACTOR || buffer == MDN_BUF_CRITIC) {
        rc = refresh_transposes(s);
        if (rc) return rc;
        HIP_TRY(hipStreamSynchronize(s->stream));
    }
    return MDN_OK;
}

// ---------------------------------------------------------------- PPO
int mdn_ppo_create(MdnSim* s, uint32_t epochs, uint32_t minibatch, MdnPPO** out) {
    if (!s || !out) return fail(MDN_E_ARG, "mdn_ppo_create: null argument");
    *out = nullptr;
    if (epochs < 1 || epochs > 4) return fail(MDN_E_ARG, "PPO epochs must be1..4");
    if (minibatch == 0) return fail(MDN_E_ARG, "minibatch must be positive");
    if (s->ppo) return fail(MDN_E_STATE, "simulator already has a PPO trainer");
    MdnPPO* p = new MdnPPO();
    p->sim = s;
    p->epochs = epochs;
    p->minibatch = uint32_t(std::min<size_t>(minibatch, s->rows()));
    const size_t M = p->minibatch;
    const uint32_t minibatches = uint32_t((s->rows() + p->minibatch - 1) / p->minibatch);
    p->updates = minibatches * epochs;
    const uint32_t chunks = uint32_t((M + 255) / 256);
    int rc = MDN_OK;
    auto guard = [&](int r) { if (r != MDN_OK && rc == MDN_OK) rc = r; };
    guard(dev_alloc(&p->am, s->shape.actor_count()));
    guard(dev_alloc(&p->av, s->shape.actor_count()));
    guard(dev_alloc(&p->cm, s->shape.critic_count()));
    guard(dev_alloc(&p->cv, s->shape.critic_count()));
    guard(dev_alloc(&p->part, size_t(chunks) * ppo_partial_stride(s->shape.obs)));
    guard(dev_alloc(&p->grad, ppo_partial_stride(s->shape.obs)));
    if (M <= ppo::MB_ROWS) guard(dev_alloc(&p->mb_rec, ppo::MB_REC_WORDS));
    guard(dev_alloc(&p->norm_part, ppo_normalize_part_words(s->rows())));
    guard(dev_alloc(&p->norm_stats, 2));
    guard(dev_alloc(&p->metric_rows, size_t(p->updates) * 4));
    guard(dev_alloc(&p->metric_mean, 4));
    guard(dev_alloc(&p->grad_norm_rows, size_t(p->updates) * 2));
    s->ppo = p;
    if (rc == MDN_OK && hipDeviceSynchronize() != hipSuccess) rc = fail(MDN_E_HIP, "mdn_ppo_create: allocation sync");
    if (rc != MDN_OK) {
        mdn_ppo_destroy(p);
        return rc;
    }
    *out = p;
    return MDN_OK;
}

void mdn_ppo_destroy(MdnPPO* p) {
    if (!p) return;
    if (p->sim) {
        hipStreamSynchronize(p->sim->stream);
        if (p->sim->ppo == p) p->sim->ppo = nullptr;
    }
    void* bufs[] = {p->am, p->av, p->cm, p->cv, p->part, p->grad, p->mb_rec, p->norm_part, p->norm_stats,
                    p->metric_rows, p->metric_mean, p->grad_norm_rows};
    for (void* b : bufs)
        if (b) hipFree(b);
    delete p;
}

int mdn_ppo_gae(MdnPPO* p) {
    if (!p) return fail(MDN_E_ARG, "mdn_ppo_gae: null");
    MdnSim* s = p->sim;
    int rc = open_sync_window(s);
    if (rc) return rc;
    return timed(s, MDN_K_GAE, [&] {
        return ppo_launch_gae(s->rewards, s->values, s->next_values, s->terminated, s->truncated, s->advantages,
                              s->returns, s->horizon, s->cfg.n, 0.99f, 0.95f, s->stream);
    });
}

int mdn_ppo_normalize(MdnPPO* p) {
    if (!p) return fail(MDN_E_ARG, "mdn_ppo_normalize: null");
    MdnSim* s = p->sim;
    int rc = open_sync_window(s);
    if (rc) return rc;
    return timed(s, MDN_K_NORMALIZE, [&] {
        return ppo_launch_normalize(s->advantages, s->rows(), p->norm_part, p->norm_stats, 1.0e-8f, s->stream);
    });
}

}  // extern "C"

namespace {
// main.mm:1331-1384.  normalize_rows: the advantages hold GAE's values and
// norm_stats (mean, inv); the first epoch's minibatches (which together
// cover every row once) normalise their rows as they read them and store
// them back (ppo.hpp:139), so no separate rescale pass runs.
int ppo_update(MdnPPO* p, uint32_t rollout_index, bool normalize_rows) {
    MdnSim* s = p->sim;
    int rc = open_sync_window(s);
    if (rc) return rc;
    const uint32_t rows = uint32_t(s->rows());
    const std::vector<uint32_t> order = mdn::minibatch_schedule(rows, p->minibatch, p->epochs, rollout_index);
    if (order.size() != p->updates) return fail(MDN_E_STATE, "PPO update count mismatch");
    const size_t first_epoch = order.size() / p->epochs;
    bool stale_w1t = false;  // transposed first layers behind the flat vectors
    for (size_t u = 0; u < order.size(); u++) {
        const uint32_t begin = order[u];
        const uint32_t b = std::min(p->minibatch, rows - begin);
        ppo::RowArgs ra;
        ra.obs = s->obs + size_t(begin) * s->shape.obs;
        ra.co = s->co + size_t(begin) * COBS;
        ra.actions = s->actions + size_t(begin) * 4;
        ra.old_logp = s->logp + begin;
        ra.adv = s->advantages + begin;
        ra.ret = s->returns + begin;
        if (normalize_rows && u < first_epoch) {
            ra.norm = p->norm_stats;
            ra.adv_out = s->advantages + begin;
        }
        ra.actor = s->actor; ra.actor_w1t = s->actor_w1t; ra.critic = s->critic; ra.critic_w1t = s->critic_w1t;
        ra.part = p->part;
        ra.b = b; ra.d = s->shape.obs; ra.clip = 0.2f; ra.vcoef = 0.5f; ra.ecoef = s->cfg.entropy_coef;
        const bool one_chunk = p->mb_rec && b <= ppo::MB_ROWS;
        if (one_chunk) {  // one chunk: row and parameter passes over many CUs
            ppo::MbArgs ma;
            ma.r = ra;
            ma.rec = p->mb_rec;
            ma.grad = p->grad;
            rc = timed(s, MDN_K_ROWS, [&] { return ppo_launch_minibatch(&ma, s->stream); });
            if (rc) return rc;
        } else {
            if (stale_w1t) {  // the chunk kernel stages the transposed copies
                rc = refresh_transposes(s);
                if (rc) return rc;
                stale_w1t = false;
            }
            rc = timed(s, MDN_K_ROWS, [&] { return ppo_launch_rows(&ra, s->stream); });
            if (rc) return rc;
            rc = timed(s, MDN_K_GRADS, [&] {
                return ppo_launch_grads(p->part, p->grad, b, s->shape.obs, s->stream);
            });
            if (rc) return rc;
        }
        ++p->optimizer_step;
        ppo::AdamArgs aa;
        aa.actor = s->actor; aa.critic = s->critic; aa.actor_w1t = s->actor_w1t; aa.critic_w1t = s->critic_w1t;
        aa.am = p->am; aa.av = p->av; aa.cm = p->cm; aa.cv = p->cv;
        aa.grad = p->grad; aa.metric_row = p->metric_rows + u * 4;
        aa.norm_row = p->grad_norm_rows + u * 2;
        aa.lr = s->cfg.learning_rate;
        mdn::adam_corrections(p->optimizer_step, 0.9f, 0.999f, &aa.c1, &aa.c2);
        aa.b = b;
        aa.d = s->shape.obs;
        // the one-chunk forward stages the flat first layers, so their
        // transposed copies are formed once, after the last step
        aa.keep_w1t = one_chunk ? 0u : 1u;
        stale_w1t = stale_w1t || one_chunk;
        rc = timed(s, MDN_K_ADAM, [&] { return ppo_launch_adam(&aa, s->stream); });
        if (rc) return rc;
    }
    if (stale_w1t) {
        rc = refresh_transposes(s);
        if (rc) return rc;
    }
    HIP_TRY(ppo_launch_metric_mean(p->metric_rows, p->metric_mean, p->updates, s->stream));
    return MDN_OK;
}
}  // namespace

extern "C" {

int mdn_ppo_update(MdnPPO* p, uint32_t rollout_index) {
    if (!p) return fail(MDN_E_ARG, "mdn_ppo_update: null");
    return ppo_update(p, rollout_index, false);
}

int mdn_ppo_rollout_update(MdnPPO* p, uint32_t rollout_index) {
    int rc = mdn_ppo_gae(p);
    if (rc) return rc;
    MdnSim* s = p->sim;
    rc = timed(s, MDN_K_NORMALIZE, [&] {
        return ppo_launch_normalize_stats(s->advantages, s->rows(), p->norm_part, p->norm_stats, 1.0e-8f, 0,
                                          s->stream);
    });
    if (rc) return rc;
    return ppo_update(p, rollout_index, true);
}

}  // extern "C"

namespace {
// main.mm:1443-1465 over `updates` rows of (actor, critic) pre-clip norms.
int grad_norm_summary(const float* dev_rows, uint32_t updates, hipStream_t stream, MdnGradNormSummary* out) {
    HIP_TRY(hipStreamSynchronize(stream));
    std::vector<float> rows(size_t(updates) * 2);
    if (!rows.empty()) HIP_TRY(hipMemcpy(rows.data(), dev_rows, rows.size() * 4, hipMemcpyDeviceToHost));
    const float limit = 0.5f;  // the clip norm of both networks (cpu_reference.hpp:47)
    MdnGradNormSummary s{};
    double actor_sum = 0.0, critic_sum = 0.0;
    uint32_t actor_clipped = 0, critic_clipped = 0;
    for (uint32_t u = 0; u < updates; u++) {
        const float a = rows[2 * u], c = rows[2 * u + 1];
        if (!std::isfinite(a) || !std::isfinite(c)) return fail(MDN_E_STATE, "non-finite pre-clip gradient norm");
        actor_sum += a;
        critic_sum += c;
        actor_clipped += a > limit ? 1u : 0u;
        critic_clipped += c > limit ? 1u : 0u;
        s.actor_max = std::max(s.actor_max, a);
        s.critic_max = std::max(s.critic_max, c);
    }
    if (updates > 0) {
        s.actor_mean = float(actor_sum / double(updates));
        s.critic_mean = float(critic_sum / double(updates));
        s.actor_clip_frac = float(actor_clipped) / float(updates);
        s.critic_clip_frac = float(critic_clipped) / float(updates);
    }
    *out = s;
    return MDN_OK;
}
}  // namespace

extern "C" {

int mdn_ppo_grad_norm_summary(MdnPPO* p, MdnGradNormSummary* out) {
    if (!p || !out) return fail(MDN_E_ARG, "mdn_ppo_grad_norm_summary: null");
    return grad_norm_summary(p->grad_norm_rows, p->updates, p->sim->stream, out);
}

int mdn_ppo_metric_mean(MdnPPO* p, float out[4]) {
    if (!p || !out) return fail(MDN_E_ARG, "mdn_ppo_metric_mean: null");
    HIP_TRY(hipStreamSynchronize(p->sim->stream));
    HIP_TRY(hipMemcpy(out, p->metric_mean, 16, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_ppo_optimizer_step(const MdnPPO* p, uint64_t* step) {
    if (!p || !step) return fail(MDN_E_ARG, "mdn_ppo_optimizer_step: null");
    *step = p->optimizer_step;
    return MDN_OK;
}

int mdn_ppo_updates_per_rollout(const MdnPPO* p, uint32_t* updates) {
    if (!p || !updates) return fail(MDN_E_ARG, "mdn_ppo_updates_per_rollout: null");
    *updates = p->updates;
    return MDN_OK;
}

// ---------------------------------------------------------------- operators
namespace {
struct DevBuf {
    void* p = nullptr;
    ~DevBuf() { if (p) hipFree(p); }
};
int upload_tmp(DevBuf& d, const void* host, size_t bytes) {
    HIP_TRY(hipMalloc(&d.p, bytes ? bytes : 4));
    if (host && bytes) HIP_TRY(hipMemcpy(d.p, host, bytes, hipMemcpyHostToDevice));
    return MDN_OK;
}
}  // namespace

int mdn_op_physics_step(const MdnPhysicsState* states, const float* actions, const float* winds,
                        const MdnPhysicsParams* params, MdnPhysicsState* out, uint64_t n) {
    if (!states || !actions || !winds || !params || !out) return fail(MDN_E_ARG, "mdn_op_physics_step: null");
    if (n == 0) return MDN_OK;
    DevBuf ds, da, dw, dout;
    int rc = upload_tmp(ds, states, n * sizeof(MdnPhysicsState));
    if (!rc) rc = upload_tmp(da, actions, n * 16);
    if (!rc) rc = upload_tmp(dw, winds, n * 12);
    if (!rc) rc = upload_tmp(dout, nullptr, n * sizeof(MdnPhysicsState));
    if (rc) return rc;
    HIP_TRY(nav_launch_physics_fixture(static_cast<const MdnPhysicsState*>(ds.p), static_cast<const float*>(da.p),
                                       static_cast<const float*>(dw.p), params, static_cast<MdnPhysicsState*>(dout.p), n,
                                       nullptr));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(out, dout.p, n * sizeof(MdnPhysicsState), hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_op_raptor_sequence(const MdnRaptorWeights* weights, const float* obs, uint32_t steps, uint32_t copies,
                           float* actions, float* hidden) {
    if (!weights || !obs || !actions || !hidden) return fail(MDN_E_ARG, "mdn_op_raptor_sequence: null");
    if (steps == 0 || copies == 0) return MDN_OK;
    DevBuf dw, dobs, dact, dh;
    int rc = upload_tmp(dw, weights, sizeof(MdnRaptorWeights));
    if (!rc) rc = upload_tmp(dobs, obs, size_t(steps) * 22 * 4);
    if (!rc) rc = upload_tmp(dact, nullptr, size_t(copies) * steps * 16);
    if (!rc) rc = upload_tmp(dh, nullptr, size_t(copies) * 64);
    if (rc) return rc;
    // copies are spread over the three lane-group widths the rollout uses
    const uint32_t third = (copies + 2) / 3;
    const int widths[3] = {4, 8, 16};
    for (int k = 0; k < 3; k++) {
        const uint32_t first = third * uint32_t(k);
        if (first >= copies) break;
        const uint32_t cnt = std::min(third, copies - first);
        HIP_TRY(nav_launch_raptor_fixture(static_cast<const float*>(dw.p), static_cast<const float*>(dobs.p), steps, cnt,
                                          static_cast<float*>(dact.p) + size_t(first) * steps * 4,
                                          static_cast<float*>(dh.p) + size_t(first) * 16, widths[k], nullptr));
    }
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(actions, dact.p, size_t(copies) * steps * 16, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(hidden, dh.p, size_t(copies) * 64, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_op_ray_world(const MdnWorld* worlds, const float* rays, const float* times, uint32_t rays_per_world,
                     float* out, uint64_t n) {
    if (!worlds || !rays || !times || !out || rays_per_world == 0) return fail(MDN_E_ARG, "mdn_op_ray_world: bad argument");
    if (n == 0) return MDN_OK;
    const uint64_t nw = (n + rays_per_world - 1) / rays_per_world;
    DevBuf dw, dr, dt, dout;
    int rc = upload_tmp(dw, worlds, nw * sizeof(MdnWorld));
    if (!rc) rc = upload_tmp(dr, rays, n * 24);
    if (!rc) rc = upload_tmp(dt, times, nw * 4);
    if (!rc) rc = upload_tmp(dout, nullptr, n * 4);
    if (rc) return rc;
    HIP_TRY(nav_launch_ray_fixture(static_cast<const float*>(dw.p), static_cast<const float*>(dr.p),
                                   static_cast<const float*>(dt.p), rays_per_world, static_cast<float*>(dout.p), n,
                                   nullptr));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(out, dout.p, n * 4, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_op_clearance(const MdnWorld* worlds, const float* points, const float* times, float* out, uint64_t n) {
    if (!worlds || !points || !times || !out) return fail(MDN_E_ARG, "mdn_op_clearance: null");
    if (n == 0) return MDN_OK;
    DevBuf dw, dp, dt, dout;
    int rc = upload_tmp(dw, worlds, n * sizeof(MdnWorld));
    if (!rc) rc = upload_tmp(dp, points, n * 12);
    if (!rc) rc = upload_tmp(dt, times, n * 4);
    if (!rc) rc = upload_tmp(dout, nullptr, n * 4);
    if (rc) return rc;
    HIP_TRY(nav_launch_clearance_fixture(static_cast<const float*>(dw.p), static_cast<const float*>(dp.p),
                                         static_cast<const float*>(dt.p), static_cast<float*>(dout.p), n, nullptr));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(out, dout.p, n * 4, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_op_gae(uint32_t horizon, uint32_t n, const float* rewards, const float* values, const float* next_values,
               const uint8_t* terminated, const uint8_t* truncated, float gamma, float lambda, float* advantages,
               float* returns) {
    if (!rewards || !values || !next_values || !terminated || !truncated || !advantages || !returns)
        return fail(MDN_E_ARG, "mdn_op_gae: null");
    const size_t R = size_t(horizon) * n;
    if (R == 0) return MDN_OK;
    DevBuf r, v, nv, te, tr, adv, ret;
    int rc = upload_tmp(r, rewards, R * 4);
    if (!rc) rc = upload_tmp(v, values, R * 4);
    if (!rc) rc = upload_tmp(nv, next_values, R * 4);
    if (!rc) rc = upload_tmp(te, terminated, R);
    if (!rc) rc = upload_tmp(tr, truncated, R);
    if (!rc) rc = upload_tmp(adv, nullptr, R * 4);
    if (!rc) rc = upload_tmp(ret, nullptr, R * 4);
    if (rc) return rc;
    HIP_TRY(ppo_launch_gae(static_cast<float*>(r.p), static_cast<float*>(v.p), static_cast<float*>(nv.p),
                           static_cast<uint8_t*>(te.p), static_cast<uint8_t*>(tr.p), static_cast<float*>(adv.p),
                           static_cast<float*>(ret.p), horizon, n, gamma, lambda, nullptr));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(advantages, adv.p, R * 4, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(returns, ret.p, R * 4, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_op_normalize(float* advantages, uint64_t count, float epsilon) {
    if (!advantages) return fail(MDN_E_ARG, "mdn_op_normalize: null");
    if (count == 0) return MDN_OK;
    DevBuf a, part, stats;
    int rc = upload_tmp(a, advantages, count * 4);
    if (!rc) rc = upload_tmp(part, nullptr, ppo_normalize_part_words(count) * 8);
    if (!rc) rc = upload_tmp(stats, nullptr, 8);
    if (rc) return rc;
    HIP_TRY(hipMemset(part.p, 0, ppo_normalize_part_words(count) * 8));  // the ticket starts at zero
    HIP_TRY(ppo_launch_normalize(static_cast<float*>(a.p), count, static_cast<double*>(part.p),
                                 static_cast<float*>(stats.p), epsilon, nullptr));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(advantages, a.p, count * 4, hipMemcpyDeviceToHost));
    return MDN_OK;
}

// ---------------------------------------------------------------- normalisation without allocation
}  // extern "C"

namespace {
// Scratch of mdn_op_normalize_noalloc: a 32-bit ticket and the group
// partials of the advantage statistics (two doubles per 16,384 rows),
// followed by the two statistics (mean, inverse deviation).  Every GPU the library runs on holds its own
// copy for the life of the process.
constexpr uint64_t kNoallocPartials = ppo_normalize_part_words(MDN_NORMALIZE_NOALLOC_MAX);
constexpr size_t kNoallocBytes = kNoallocPartials * sizeof(double) + 2 * sizeof(float);
static __device__ __align__(256) unsigned char scratch[kNoallocBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
unsigned char* g_scratch[kMaxDevices] = {};

// The device address of the current GPU's scratch (host code never uses the
// symbol itself: its host-side name is not a device address).
int scratch_address(unsigned char** out) {
    int dev = 0;
    HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(MDN_E_ARG, "device ordinal beyond the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(MDN_E_HIP, "hipGetSymbolAddress returned no address for the scratch array");
        g_scratch[dev] = static_cast<unsigned char*>(p);
    }
    *out = g_scratch[dev];
    return MDN_OK;
}
}  // namespace

extern "C" {

int mdn_op_normalize_noalloc(float* advantages, uint64_t count, float epsilon, void* stream) {
    if (!advantages) return fail(MDN_E_ARG, "mdn_op_normalize_noalloc: null");
    if (count > MDN_NORMALIZE_NOALLOC_MAX)
        return fail(MDN_E_ARG, "mdn_op_normalize_noalloc: count " + std::to_string(count) + " exceeds the scratch limit of " +
                                   std::to_string(uint64_t(MDN_NORMALIZE_NOALLOC_MAX)) + " rows");
    if (count == 0) return MDN_OK;
    unsigned char* base = nullptr;
    int rc = scratch_address(&base);
    if (rc) return rc;
    // partials are written by each pass before the next reads them and the
    // statistics by the passes; the ticket is zero from load time and each
    // call leaves it zero, so nothing needs clearing
    double* part = reinterpret_cast<double*>(base);
    float* stats = reinterpret_cast<float*>(base + kNoallocPartials * sizeof(double));
    HIP_TRY(ppo_launch_normalize(advantages, count, part, stats, epsilon, static_cast<hipStream_t>(stream)));
    return MDN_OK;
}

// ---------------------------------------------------------------- fixed_ppo operators
int mdn_op_actor_forward(const float* params, uint32_t obs_dim, uint32_t hidden_dim, const float* obs, uint64_t batch,
                         float* hidden, float* means) {
    if (!params || !obs || !means) return fail(MDN_E_ARG, "mdn_op_actor_forward: null");
    if (obs_dim < 1 || obs_dim > 1024 || hidden_dim < 1 || hidden_dim > 8192)
        return fail(MDN_E_ARG, "mdn_op_actor_forward: inputs must be 1..1024 and hidden units 1..8192");
    if (batch == 0) return MDN_OK;
    if (batch > 0x7fffffffull) return fail(MDN_E_ARG, "mdn_op_actor_forward: batch too large");
    const size_t P = size_t(hidden_dim) * obs_dim + hidden_dim + 4 * size_t(hidden_dim) + 4 + 4;
    DevBuf w, x, h, m;
    int rc = upload_tmp(w, params, P * 4);
    if (!rc) rc = upload_tmp(x, obs, batch * obs_dim * 4);
    if (!rc) rc = upload_tmp(h, nullptr, batch * hidden_dim * 4);
    if (!rc) rc = upload_tmp(m, nullptr, batch * 16);
    if (rc) return rc;
    // ppo.hpp:30: the 184 and 824 input layouts end in the geometry-prior hint
    const uint32_t prior = obs_dim == 184 || obs_dim == 824;
    HIP_TRY(fppo_launch_forward(static_cast<float*>(w.p), static_cast<float*>(x.p), obs_dim, hidden_dim, 4, prior,
                                batch, static_cast<float*>(h.p), static_cast<float*>(m.p), nullptr));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(means, m.p, batch * 16, hipMemcpyDeviceToHost));
    if (hidden) HIP_TRY(hipMemcpy(hidden, h.p, batch * hidden_dim * 4, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_op_critic_forward(const float* params, uint32_t obs_dim, uint32_t hidden_dim, const float* obs, uint64_t batch,
                          float* hidden, float* values) {
    if (!params || !obs || !values) return fail(MDN_E_ARG, "mdn_op_critic_forward: null");
    if (obs_dim < 1 || obs_dim > 1024 || hidden_dim < 1 || hidden_dim > 8192)
        return fail(MDN_E_ARG, "mdn_op_critic_forward: inputs must be 1..1024 and hidden units 1..8192");
    if (batch == 0) return MDN_OK;
    if (batch > 0x7fffffffull) return fail(MDN_E_ARG, "mdn_op_critic_forward: batch too large");
    const size_t P = size_t(hidden_dim) * obs_dim + 2 * size_t(hidden_dim) + 1;
    DevBuf w, x, h, v;
    int rc = upload_tmp(w, params, P * 4);
    if (!rc) rc = upload_tmp(x, obs, batch * obs_dim * 4);
    if (!rc) rc = upload_tmp(h, nullptr, batch * hidden_dim * 4);
    if (!rc) rc = upload_tmp(v, nullptr, batch * 4);
    if (rc) return rc;
    HIP_TRY(fppo_launch_forward(static_cast<float*>(w.p), static_cast<float*>(x.p), obs_dim, hidden_dim, 1, 0, batch,
                                static_cast<float*>(h.p), static_cast<float*>(v.p), nullptr));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(values, v.p, batch * 4, hipMemcpyDeviceToHost));
    if (hidden) HIP_TRY(hipMemcpy(hidden, h.p, batch * hidden_dim * 4, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_op_gaussian_log_prob(const float* actions, const float* means, const float* log_std, uint32_t log_std_stride,
                             uint64_t batch, float* logp) {
    if (!actions || !means || !log_std || !logp) return fail(MDN_E_ARG, "mdn_op_gaussian_log_prob: null");
    if (log_std_stride != 0 && log_std_stride != 4) return fail(MDN_E_ARG, "log_std stride must be 0 or 4");
    if (batch == 0) return MDN_OK;
    DevBuf a, m, l, o;
    int rc = upload_tmp(a, actions, batch * 16);
    if (!rc) rc = upload_tmp(m, means, batch * 16);
    if (!rc) rc = upload_tmp(l, log_std, (log_std_stride ? batch : 1) * 16);
    if (!rc) rc = upload_tmp(o, nullptr, batch * 4);
    if (rc) return rc;
    HIP_TRY(fppo_launch_log_prob(static_cast<float*>(a.p), static_cast<float*>(m.p), static_cast<float*>(l.p),
                                 log_std_stride, batch, static_cast<float*>(o.p), nullptr));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(logp, o.p, batch * 4, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_op_sample_loss_and_grad(const float* actions, const float* means, const float* log_std,
                                uint32_t log_std_stride, const float* old_logp, const float* old_values,
                                const float* values, const float* advantages, const float* returns, uint64_t batch,
                                float batch_size, float clip_epsilon, float value_coefficient,
                                float entropy_coefficient, float* d_mean, float* d_log_std, float* d_value,
                                float* losses) {
    (void)old_values;  // kept in the ABI like the reference's unused old_value (ppo.hpp:180)
    if (!actions || !means || !log_std || !old_logp || !values || !advantages || !returns || !d_mean || !d_log_std ||
        !d_value || !losses)
        return fail(MDN_E_ARG, "mdn_op_sample_loss_and_grad: null");
    if (log_std_stride != 0 && log_std_stride != 4) return fail(MDN_E_ARG, "log_std stride must be 0 or 4");
    if (batch == 0) return MDN_OK;
    DevBuf a, m, l, ol, v, ad, re, dm, dl, dv, lo;
    int rc = upload_tmp(a, actions, batch * 16);
    if (!rc) rc = upload_tmp(m, means, batch * 16);
    if (!rc) rc = upload_tmp(l, log_std, (log_std_stride ? batch : 1) * 16);
    if (!rc) rc = upload_tmp(ol, old_logp, batch * 4);
    if (!rc) rc = upload_tmp(v, values, batch * 4);
    if (!rc) rc = upload_tmp(ad, advantages, batch * 4);
    if (!rc) rc = upload_tmp(re, returns, batch * 4);
    if (!rc) rc = upload_tmp(dm, nullptr, batch * 16);
    if (!rc) rc = upload_tmp(dl, nullptr, batch * 16);
    if (!rc) rc = upload_tmp(dv, nullptr, batch * 4);
    if (!rc) rc = upload_tmp(lo, nullptr, batch * 16);
    if (rc) return rc;
    fppo_loss_args g;
    g.actions = static_cast<float*>(a.p); g.means = static_cast<float*>(m.p); g.log_std = static_cast<float*>(l.p);
    g.old_logp = static_cast<float*>(ol.p); g.values = static_cast<float*>(v.p);
    g.advantages = static_cast<float*>(ad.p); g.returns = static_cast<float*>(re.p);
    g.d_mean = static_cast<float*>(dm.p); g.d_log_std = static_cast<float*>(dl.p);
    g.d_value = static_cast<float*>(dv.p); g.losses = static_cast<float*>(lo.p);
    g.b = batch; g.ls_stride = log_std_stride;
    g.batch_size = batch_size; g.clip = clip_epsilon; g.vcoef = value_coefficient; g.ecoef = entropy_coefficient;
    HIP_TRY(fppo_launch_loss_grad(&g, nullptr));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(d_mean, dm.p, batch * 16, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(d_log_std, dl.p, batch * 16, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(d_value, dv.p, batch * 4, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(losses, lo.p, batch * 16, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_op_adam_update(float* params, const float* grad, float* first, float* second, uint64_t count, uint64_t step,
                       float learning_rate, float beta1, float beta2, float epsilon, float weight_decay) {
    if (!params || !grad || !first || !second) return fail(MDN_E_ARG, "mdn_op_adam_update: null");
    if (count == 0) return MDN_OK;
    float c1 = 0.0f, c2 = 0.0f;
    mdn::adam_corrections(step, beta1, beta2, &c1, &c2);
    DevBuf p, g, m, v;
    int rc = upload_tmp(p, params, count * 4);
    if (!rc) rc = upload_tmp(g, grad, count * 4);
    if (!rc) rc = upload_tmp(m, first, count * 4);
    if (!rc) rc = upload_tmp(v, second, count * 4);
    if (rc) return rc;
    HIP_TRY(fppo_launch_adam(static_cast<float*>(p.p), static_cast<float*>(g.p), static_cast<float*>(m.p),
                             static_cast<float*>(v.p), count, learning_rate, beta1, beta2, epsilon, weight_decay, c1,
                             c2, nullptr));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(params, p.p, count * 4, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(first, m.p, count * 4, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(second, v.p, count * 4, hipMemcpyDeviceToHost));
    return MDN_OK;
}

// fixed_ppo::run_cpu_self_tests (ppo.hpp:204-267) with the GPU operators
// above: central differences of the per-sample objective (the sum of the
// policy, value and entropy losses at batch size 1, which is
// sample_objective) against the analytic derivatives on the four surrogate
// branches, the value derivative, and Adam's closed-form first step.
int mdn_op_ppo_self_tests(float tolerance, int* passed) {
    if (!passed) return fail(MDN_E_ARG, "mdn_op_ppo_self_tests: null");
    *passed = 0;
    float action[4] = {0.4f, 0, 0, 0}, mean[4] = {0.1f, 0, 0, 0}, log_std[4] = {0, 0, 0, 0};
    const float clip = 0.2f, vcoef = 0.7f, ecoef = 0.03f, value = 0.25f, target = -0.3f, h = 1.0e-3f;
    float base_logp = 0.0f;
    int rc = mdn_op_gaussian_log_prob(action, mean, log_std, 0, 1, &base_logp);
    if (rc) return rc;
    float dm[4], dl[4], dv, loss[4];
    auto run = [&](float old_logp, float adv, float* objective) {
        const int r = mdn_op_sample_loss_and_grad(action, mean, log_std, 0, &old_logp, &value, &value, &adv, &target, 1,
                                                  1.0f, clip, vcoef, ecoef, dm, dl, &dv, loss);
        if (objective) *objective = loss[0] + loss[1] + loss[2];
        return r;
    };
    const float old_values[4] = {base_logp - std::log(1.1f), base_logp - std::log(0.9f), base_logp - std::log(1.3f),
                                 base_logp - std::log(0.7f)};
    const float advantages[4] = {1.0f, -1.0f, 1.0f, -1.0f};
    for (int branch = 0; branch < 4; branch++) {
        float grad_mean[4], grad_std[4], plus = 0, minus = 0;
        if ((rc = run(old_values[branch], advantages[branch], nullptr)) != MDN_OK) return rc;
        std::copy(dm, dm + 4, grad_mean);
        std::copy(dl, dl + 4, grad_std);
        for (int which = 0; which < 2; which++) {
            float* x = which == 0 ? &mean[0] : &log_std[0];
            const float saved = *x;
            *x = saved + h;
            if ((rc = run(old_values[branch], advantages[branch], &plus)) != MDN_OK) return rc;
            *x = saved - h;
            if ((rc = run(old_values[branch], advantages[branch], &minus)) != MDN_OK) return rc;
            *x = saved;
            const float numeric = (plus - minus) / (2.0f * h);
            if (std::fabs(numeric - (which == 0 ? grad_mean[0] : grad_std[0])) > tolerance) return MDN_OK;
        }
    }
    if ((rc = run(base_logp, 0.0f, nullptr)) != MDN_OK) return rc;
    if (std::fabs(vcoef * (value - target) - dv) > tolerance) return MDN_OK;
    float parameter = 1.0f, gradient = 0.25f, first = 0.0f, second = 0.0f;
    if ((rc = mdn_op_adam_update(&parameter, &gradient, &first, &second, 1, 1, 0.01f, 0.9f, 0.999f, 1.0e-8f, 0.0f)))
        return rc;
    const float want_first = 0.1f * gradient, want_second = 0.001f * gradient * gradient;
    const float want_parameter = 1.0f - 0.01f * (want_first / 0.1f) / (std::sqrt(want_second / 0.001f) + 1.0e-8f);
    *passed = std::fabs(first - want_first) <= tolerance && std::fabs(second - want_second) <= tolerance &&
              std::fabs(parameter - want_parameter) <= tolerance;
    return MDN_OK;
}

// ---------------------------------------------------------------- wide policy
}  // extern "C"

struct MdnLargePPO {
    MdnSim* sim = nullptr;
    uint32_t hidden = 0, epochs = 1, minibatch = 0, updates = 0;
    uint64_t optimizer_step = 0;
    mdn::PolicyShape shape;
    float *actor = nullptr, *critic = nullptr, *am = nullptr, *av = nullptr, *cm = nullptr, *cv = nullptr;
    __bf16 *awb = nullptr, *cwb = nullptr;
    __bf16 *xa = nullptr, *xaT = nullptr, *xc = nullptr, *xcT = nullptr;  // bf16 rows of one minibatch
    float* eval_means = nullptr;                         // [rows][4]
    float* fwd_part = nullptr;                           // forward partial sums over hidden slices
    float *means = nullptr, *values = nullptr, *dm = nullptr, *dls = nullptr, *dv = nullptr, *loss = nullptr;
    float *part = nullptr, *ga = nullptr, *gc = nullptr, *col_part = nullptr, *scratch = nullptr;
    double* norm_part = nullptr;
    float* norm_stats = nullptr;
    float *metric_rows = nullptr, *metric_mean = nullptr;
    float* grad_norm_rows = nullptr;  // [updates][2] pre-clip norms of the last rollout_update
    // values at s': the rows evaluated on their own (count, row indices,
    // their critic inputs, their values)
    uint32_t* nv_count = nullptr;
    uint32_t* nv_idx = nullptr;
    float *nv_gather = nullptr, *nv_vals = nullptr;
};

namespace {
int lp_pack(MdnLargePPO* p) {
    MdnSim* s = p->sim;
    HIP_TRY(lp_launch_pack(p->actor, p->hidden, p->shape.obs, 192, p->awb, s->stream));
    HIP_TRY(lp_launch_pack(p->critic, p->hidden, COBS, 32, p->cwb, s->stream));
    return MDN_OK;
}
// The 184-input actor's hint inputs (the last three of each obs row, added
// to the first three means), or nullptr.
const float* lp_prior(const MdnLargePPO* p, const float* obs) {
    return obs && p->shape.obs == MDN_ACTOR_OBS_PRIOR ? obs + p->shape.obs - 3 : nullptr;
}
// Wide forward over `rows` stored rows in slices of one minibatch (the size of
// the prepared-copy buffers): actor means from obs rows and/or critic values
// from critic-observation rows.
hipError_t lp_forward_rows(MdnLargePPO* p, const float* obs, const float* co, uint32_t rows, float* means,
                           float* values) {
    MdnSim* s = p->sim;
    const uint32_t D = p->shape.obs;
    hipError_t e = hipSuccess;
    for (uint32_t r0 = 0; r0 < rows && e == hipSuccess; r0 += p->minibatch) {
        const uint32_t b = std::min(p->minibatch, rows - r0);
        const float* x = obs ? obs + size_t(r0) * D : nullptr;
        e = lp_launch_prep(x, co ? co + size_t(r0) * COBS : nullptr, b, D, p->xa, p->xaT, p->xc, p->xcT, false,
                           s->stream);
        if (e == hipSuccess)
            e = lp_launch_forward(p->xa, p->xc, p->awb, p->cwb, p->actor, p->critic, p->hidden, D, b, lp_prior(p, x),
                                  means ? means + size_t(r0) * 4 : nullptr, values ? values + r0 : nullptr,
                                  p->fwd_part, s->stream);
    }
    return e;
}

// Values at s and s' of the first `ticks` ticks' rows: the critic over the
// critic observations, then only the rows whose next-state observation is
// not the next tick's observation (the last tick, resets) over theirs; the
// others take the next tick's value (next_value_split_kernel).
hipError_t lp_values(MdnLargePPO* p, uint32_t ticks) {
    MdnSim* s = p->sim;
    const uint32_t N = s->cfg.n, rows = ticks * N;
    hipError_t e = lp_forward_rows(p, nullptr, s->co, rows, nullptr, s->values);
    if (e == hipSuccess) e = hipMemsetAsync(p->nv_count, 0, sizeof(uint32_t), s->stream);
    if (e == hipSuccess)
        e = lp_launch_next_value_split(s->co, s->nco, s->values, ticks, N, s->next_values, p->nv_count, p->nv_idx,
                                       p->nv_gather, s->stream);
    uint32_t n = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&n, p->nv_count, sizeof(n), hipMemcpyDeviceToHost, s->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
    if (e == hipSuccess && n > rows) e = hipErrorInvalidValue;
    if (e == hipSuccess) e = lp_forward_rows(p, nullptr, p->nv_gather, n, nullptr, p->nv_vals);
    if (e == hipSuccess) e = lp_launch_next_value_scatter(p->nv_idx, p->nv_vals, n, s->next_values, s->stream);
    return e;
}

float* lp_param(MdnLargePPO* p, uint32_t which, uint64_t* count) {
    const uint64_t A = p->shape.actor_count(), C = p->shape.critic_count();
    switch (which) {
        case 0: *count = A; return p->actor;
        case 1: *count = C; return p->critic;
        case 2: *count = A; return p->am;
        case 3: *count = A; return p->av;
        case 4: *count = C; return p->cm;
        case 5: *count = C; return p->cv;
        default: *count = 0; return nullptr;
    }
}
}  // namespace

extern "C" {

void mdn_lppo_destroy(MdnLargePPO* p) {
    if (!p) return;
    if (p->sim) hipStreamSynchronize(p->sim->stream);
    void* bufs[] = {p->actor, p->critic, p->am, p->av, p->cm, p->cv, p->awb, p->cwb, p->xa, p->xaT, p->xc, p->xcT,
                    p->eval_means, p->fwd_part, p->means,
                    p->values, p->dm, p->dls, p->dv, p->loss, p->part, p->ga, p->gc, p->col_part, p->scratch,
                    p->norm_part, p->norm_stats, p->metric_rows, p->metric_mean, p->grad_norm_rows,
                    p->nv_count, p->nv_idx, p->nv_gather, p->nv_vals};
    for (void* b : bufs)
        if (b) hipFree(b);
    delete p;
}

int mdn_lppo_create(MdnSim* s, uint32_t hidden, uint32_t epochs, uint32_t minibatch, MdnLargePPO** out) {
    if (!s || !out) return fail(MDN_E_ARG, "mdn_lppo_create: null argument");
    *out = nullptr;
    if (hidden == 0 || hidden % 128) return fail(MDN_E_ARG, "mdn_lppo_create: hidden must be a positive multiple of 128");
    if (hidden > 8192) return fail(MDN_E_ARG, "mdn_lppo_create: hidden above 8192");
    if (epochs < 1 || epochs > 8) return fail(MDN_E_ARG, "mdn_lppo_create: epochs must be 1..8");
    if (minibatch == 0) return fail(MDN_E_ARG, "mdn_lppo_create: minibatch must be positive");
    MdnLargePPO* p = new MdnLargePPO();
    p->sim = s;
    p->hidden = hidden;
    p->epochs = epochs;
    p->minibatch = uint32_t(std::min<size_t>(minibatch, s->rows()));
    p->shape.hidden = p->shape.critic_hidden = hidden;
    p->shape.obs = s->shape.obs;
    p->updates = uint32_t((s->rows() + p->minibatch - 1) / p->minibatch) * epochs;
    const size_t A = p->shape.actor_count(), C = p->shape.critic_count(), M = p->minibatch, R = s->rows();
    int rc = MDN_OK;
    auto guard = [&](int r) { if (r != MDN_OK && rc == MDN_OK) rc = r; };
    guard(dev_alloc(&p->actor, A));
    guard(dev_alloc(&p->critic, C));
    guard(dev_alloc(&p->am, A));
    guard(dev_alloc(&p->av, A));
    guard(dev_alloc(&p->cm, C));
    guard(dev_alloc(&p->cv, C));
    guard(dev_alloc(&p->awb, size_t(hidden) * 192));
    guard(dev_alloc(&p->cwb, size_t(hidden) * 32));
    const size_t MP = (M + 127) / 128 * 128;
    guard(dev_alloc(&p->xa, MP * 192));
    guard(dev_alloc(&p->xaT, MP * 192));
    guard(dev_alloc(&p->xc, MP * 32));
    guard(dev_alloc(&p->xcT, MP * 32));
    guard(dev_alloc(&p->eval_means, R * 4));
    guard(dev_alloc(&p->nv_count, 1));
    guard(dev_alloc(&p->nv_idx, R));
    guard(dev_alloc(&p->nv_gather, R * COBS));
    guard(dev_alloc(&p->nv_vals, R));
    guard(dev_alloc(&p->fwd_part, size_t(lp_forward_part_floats(p->minibatch))));
    guard(dev_alloc(&p->means, M * 4));
    guard(dev_alloc(&p->values, M));
    guard(dev_alloc(&p->dm, M * 4));
    guard(dev_alloc(&p->dls, M * 4));
    guard(dev_alloc(&p->dv, M));
    guard(dev_alloc(&p->loss, M * 4));
    guard(dev_alloc(&p->part, size_t(lp_backward_part_floats(p->minibatch, hidden, p->shape.obs))));
    guard(dev_alloc(&p->ga, A));
    guard(dev_alloc(&p->gc, C));
    guard(dev_alloc(&p->col_part, ((M + 63) / 64) * 13));
    guard(dev_alloc(&p->scratch, lp_adam_scratch_floats()));
    guard(dev_alloc(&p->norm_part, ppo_normalize_part_words(R)));
    guard(dev_alloc(&p->norm_stats, 2));
    guard(dev_alloc(&p->metric_rows, size_t(p->updates) * 4));
    guard(dev_alloc(&p->metric_mean, 4));
    guard(dev_alloc(&p->grad_norm_rows, size_t(p->updates) * 2));
    if (rc == MDN_OK) {
        std::vector<float> a(A), c(C);
        mdn::init_policy(p->shape, a.data(), c.data());
        if (hipMemcpy(p->actor, a.data(), A * 4, hipMemcpyHostToDevice) != hipSuccess ||
            hipMemcpy(p->critic, c.data(), C * 4, hipMemcpyHostToDevice) != hipSuccess)
            rc = fail(MDN_E_HIP, "mdn_lppo_create: policy upload");
    }
    if (rc == MDN_OK) rc = lp_pack(p);
    if (rc == MDN_OK && hipStreamSynchronize(s->stream) != hipSuccess) rc = fail(MDN_E_HIP, "mdn_lppo_create: sync");
    if (rc != MDN_OK) {
        mdn_lppo_destroy(p);
        return rc;
    }
    *out = p;
    return MDN_OK;
}

int mdn_lppo_evaluate(MdnLargePPO* p) {
    if (!p) return fail(MDN_E_ARG, "mdn_lppo_evaluate: null");
    MdnSim* s = p->sim;
    int rc = open_sync_window(s);
    if (rc) return rc;
    const uint32_t R = uint32_t(s->rows());
    return timed(s, MDN_K_LP_FORWARD, [&] {
        hipError_t e = lp_forward_rows(p, s->obs, nullptr, R, p->eval_means, nullptr);
        if (e == hipSuccess) e = lp_values(p, s->horizon);
        if (e == hipSuccess)
            e = lp_launch_logp(p->eval_means, s->actions, p->actor + p->shape.actor_log_std(), R, s->logp, s->stream);
        return e;
    });
}

int mdn_lppo_collect(MdnLargePPO* p, uint32_t count) {
    if (!p) return fail(MDN_E_ARG, "mdn_lppo_collect: null");
    MdnSim* s = p->sim;
    if (s->lanes != 8) return fail(MDN_E_ARG, "mdn_lppo_collect: the split-tick env step runs 8 lanes per env");
    if (count == 0) count = s->horizon;
    int rc = open_sync_window(s);
    if (rc) return rc;
    const uint32_t N = s->cfg.n;
    const int slots = ring_slots(s->cfg);
    nav::RolloutArgs a = s->args(1);
    a.ext_means = p->eval_means;
    a.ext_log_std = p->actor + p->shape.actor_log_std();
    const bool memory = s->shape.obs == MDN_ACTOR_OBS_PRIOR && s->cfg.geometry_memory;
    if (memory) a.mem_head = s->mem_head;
    nav::MemoryArgs m;
    m.head = s->mem_head; m.sensors = s->sensors; m.poses = s->poses; m.pix_rays = s->pix_rays; m.cells = s->cells;
    m.sensor_dt = a.sensor_dt; m.inv_sensor_dt = a.inv_sensor_dt; m.n = N;
    m.tan_v = s->camera_profile.tan_v;
    // tick 0 up to its observation; then per tick: wide actor means of the
    // tick's rows, and one launch that acts, advances, resets and observes the
    // next tick
    a.split = nav::SPLIT_END_AFTER_OBSERVE;
    rc = timed(s, MDN_K_ROLLOUT, [&] { return nav_launch_rollout(&a, 8, slots, s->shape.obs, s->stream); });
    for (uint32_t t = 0; t < count && rc == MDN_OK; t++) {
        const size_t row0 = size_t(t % s->horizon) * N;
        if (memory) {  // the geometry-memory hint of the tick's rows
            m.obs = s->obs + row0 * s->shape.obs;
            rc = timed(s, MDN_K_MEMORY, [&] { return nav_launch_memory_hint(&m, s->stream); });
            if (rc) break;
        }
        rc = timed(s, MDN_K_LP_FORWARD, [&] {
            return lp_forward_rows(p, s->obs + row0 * s->shape.obs, nullptr, N, p->eval_means + row0 * 4, nullptr);
        });
        if (rc) break;
        const bool more = t + 1 < count;
        a.count = more ? 2 : 1;
        a.tick0 = t;
        a.split = nav::SPLIT_BEGIN_AT_ACT | (more ? nav::SPLIT_END_AFTER_OBSERVE : 0u);
        rc = timed(s, MDN_K_ROLLOUT, [&] { return nav_launch_rollout(&a, 8, slots, s->shape.obs, s->stream); });
    }
    if (rc) return rc;
    // values at s and s' (sim.metal:254, 322) under the wide critic (a row
    // reuses the next row's value only where their inputs are equal bit for
    // bit, so a collect that wrapped the horizon is handled too)
    return timed(s, MDN_K_LP_FORWARD, [&] { return lp_values(p, std::min(count, s->horizon)); });
}

int mdn_lppo_means(MdnLargePPO* p, float* host, uint64_t count) {
    if (!p || !host) return fail(MDN_E_ARG, "mdn_lppo_means: null");
    const uint64_t n = uint64_t(p->sim->rows()) * 4;
    if (count != n) return fail(MDN_E_ARG, "mdn_lppo_means: count must be rows * 4");
    HIP_TRY(hipStreamSynchronize(p->sim->stream));
    HIP_TRY(hipMemcpy(host, p->eval_means, n * 4, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_lppo_rollout_update(MdnLargePPO* p, uint32_t rollout_index) {
    if (!p) return fail(MDN_E_ARG, "mdn_lppo_rollout_update: null");
    MdnSim* s = p->sim;
    int rc = open_sync_window(s);
    if (rc) return rc;
    const uint32_t rows = uint32_t(s->rows());
    rc = timed(s, MDN_K_GAE, [&] {
        return ppo_launch_gae(s->rewards, s->values, s->next_values, s->terminated, s->truncated, s->advantages,
                              s->returns, s->horizon, s->cfg.n, 0.99f, 0.95f, s->stream);
    });
    if (rc) return rc;
    rc = timed(s, MDN_K_NORMALIZE, [&] {
        return ppo_launch_normalize(s->advantages, rows, p->norm_part, p->norm_stats, 1.0e-8f, s->stream);
    });
    if (rc) return rc;
    const std::vector<uint32_t> order = mdn::minibatch_schedule(rows, p->minibatch, p->epochs, rollout_index);
    if (order.size() != p->updates) return fail(MDN_E_STATE, "wide PPO update count mismatch");
    const uint32_t H = p->hidden, D = p->shape.obs;
    for (size_t u = 0; u < order.size(); u++) {
        const uint32_t begin = order[u];
        const uint32_t b = std::min(p->minibatch, rows - begin);
        const float* obs = s->obs + size_t(begin) * D;
        const float* co = s->co + size_t(begin) * COBS;
        rc = timed(s, MDN_K_LP_FORWARD, [&] {
            hipError_t e = lp_launch_prep(obs, co, b, D, p->xa, p->xaT, p->xc, p->xcT, true, s->stream);
            if (e == hipSuccess)
                e = lp_launch_forward(p->xa, p->xc, p->awb, p->cwb, p->actor, p->critic, H, D, b, lp_prior(p, obs),
                                      p->means, p->values, p->fwd_part, s->stream);
            if (e == hipSuccess)
                e = lp_launch_loss(p->means, p->values, s->actions + size_t(begin) * 4, s->logp + begin,
                                   s->advantages + begin, s->returns + begin, p->actor + p->shape.actor_log_std(), b,
                                   0.2f, 0.5f, s->cfg.entropy_coef, p->dm, p->dls, p->dv, p->loss, p->col_part,
                                   s->stream);
            return e;
        });
        if (rc) return rc;
        rc = timed(s, MDN_K_LP_BACKWARD, [&] {
            return lp_launch_backward(p->xa, p->xaT, p->xc, p->xcT, p->awb, p->cwb, p->actor, p->critic, p->dm, p->dv,
                                      p->col_part, H, D, b, p->part, p->ga, p->gc, p->scratch, s->stream);
        });
        if (rc) return rc;
        ++p->optimizer_step;
        float c1 = 1.0f, c2 = 1.0f;
        mdn::adam_corrections(p->optimizer_step, 0.9f, 0.999f, &c1, &c2);
        rc = timed(s, MDN_K_LP_ADAM, [&] {
            return lp_launch_adam(p->actor, p->critic, p->am, p->av, p->cm, p->cv, p->awb, p->cwb, p->ga, p->gc,
                                  p->scratch, b, H, D, s->cfg.learning_rate, c1, c2, p->metric_rows + u * 4,
                                  p->grad_norm_rows + u * 2, s->stream);
        });
        if (rc) return rc;
    }
    HIP_TRY(ppo_launch_metric_mean(p->metric_rows, p->metric_mean, p->updates, s->stream));
    return MDN_OK;
}

int mdn_lppo_param_count(const MdnLargePPO* p, uint32_t which, uint64_t* count) {
    if (!p || !count) return fail(MDN_E_ARG, "mdn_lppo_param_count: null");
    if (!lp_param(const_cast<MdnLargePPO*>(p), which, count)) return fail(MDN_E_ARG, "mdn_lppo_param_count: bad id");
    return MDN_OK;
}

int mdn_lppo_get_params(MdnLargePPO* p, uint32_t which, float* host, uint64_t count) {
    if (!p || !host) return fail(MDN_E_ARG, "mdn_lppo_get_params: null");
    uint64_t n = 0;
    float* d = lp_param(p, which, &n);
    if (!d) return fail(MDN_E_ARG, "mdn_lppo_get_params: bad id");
    if (count != n) return fail(MDN_E_ARG, "mdn_lppo_get_params: count mismatch");
    HIP_TRY(hipStreamSynchronize(p->sim->stream));
    HIP_TRY(hipMemcpy(host, d, n * 4, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_lppo_set_params(MdnLargePPO* p, uint32_t which, const float* host, uint64_t count) {
    if (!p || !host) return fail(MDN_E_ARG, "mdn_lppo_set_params: null");
    uint64_t n = 0;
    float* d = lp_param(p, which, &n);
    if (!d) return fail(MDN_E_ARG, "mdn_lppo_set_params: bad id");
    if (count != n) return fail(MDN_E_ARG, "mdn_lppo_set_params: count mismatch");
    HIP_TRY(hipStreamSynchronize(p->sim->stream));
    HIP_TRY(hipMemcpy(d, host, n * 4, hipMemcpyHostToDevice));
    if (which <= 1) {
        const int rc = lp_pack(p);
        if (rc) return rc;
        HIP_TRY(hipStreamSynchronize(p->sim->stream));
    }
    return MDN_OK;
}

int mdn_lppo_grad_norm_summary(MdnLargePPO* p, MdnGradNormSummary* out) {
    if (!p || !out) return fail(MDN_E_ARG, "mdn_lppo_grad_norm_summary: null");
    return grad_norm_summary(p->grad_norm_rows, p->updates, p->sim->stream, out);
}

int mdn_lppo_metric_mean(MdnLargePPO* p, float out[4]) {
    if (!p || !out) return fail(MDN_E_ARG, "mdn_lppo_metric_mean: null");
    HIP_TRY(hipStreamSynchronize(p->sim->stream));
    HIP_TRY(hipMemcpy(out, p->metric_mean, 16, hipMemcpyDeviceToHost));
    return MDN_OK;
}

int mdn_lppo_optimizer_step(const MdnLargePPO* p, uint64_t* step) {
    if (!p || !step) return fail(MDN_E_ARG, "mdn_lppo_optimizer_step: null");
    *step = p->optimizer_step;
    return MDN_OK;
}


// ---------------------------------------------------------------- files
}  // extern "C"

namespace {

struct File {
    std::FILE* f = nullptr;
    explicit File(const char* path, const char* mode) : f(std::fopen(path, mode)) {}
    ~File() { if (f) std::fclose(f); }
    bool read(void* p, size_t n) { return std::fread(p, 1, n, f) == n; }
    bool write(const void* p, size_t n) { return std::fwrite(p, 1, n, f) == n; }
    bool at_end() { unsigned char c; return std::fread(&c, 1, 1, f) == 0 && std::feof(f); }
};

// read_checkpoint_header (main.mm:986-994): the 48-byte prefix, the first 64
// config bytes, then what each version adds; older versions default the rest.
int read_checkpoint_header(File& file, MdnCheckpointHeader* h) {
    std::memset(h, 0, sizeof(*h));
    unsigned char* b = reinterpret_cast<unsigned char*>(h);
    if (!file.read(b, 48) || std::memcmp(h->magic, "PPOFIX1", 7) != 0 || h->version < 3 || h->version > 10)
        return fail(MDN_E_ARG, "checkpoint prefix/version");
    if (!file.read(&h->config, 64)) return fail(MDN_E_ARG, "checkpoint header truncated");
    if (h->version >= 4) {
        if (!file.read(b + 112, 16)) return fail(MDN_E_ARG, "checkpoint header truncated");
        if (h->version >= 6) {
            if (!file.read(b + 128, 8)) return fail(MDN_E_ARG, "checkpoint header truncated");
        } else {
            h->config.geometry_memory = 0;
        }
        if (h->version == 4) h->config.velocity_contract = 0;
    } else {
        h->config.risk_coef = 0;
        h->config.entropy_coef = h->family == 7 ? .002f : .005f;
        h->config.learning_rate = .0003f;
        h->config.velocity_contract = 0;
        h->config.geometry_memory = 0;
    }
    return MDN_OK;
}

// Simulator settings a resume must match (main.mm:1224-1229).
bool same_run_settings(const MdnSimConfig& a, const MdnSimConfig& b) {
    return a.family == b.family && a.n == b.n && a.substeps == b.substeps && a.sensor_period == b.sensor_period &&
           a.sensor_delay == b.sensor_delay && a.command_delay == b.command_delay && a.max_steps == b.max_steps &&
           a.mode == b.mode && a.speed == b.speed && a.distance == b.distance && a.wind == b.wind &&
           a.depth_noise == b.depth_noise && a.dropout == b.dropout && a.risk_coef == b.risk_coef &&
           a.entropy_coef == b.entropy_coef && a.learning_rate == b.learning_rate &&
           a.velocity_contract == b.velocity_contract && a.geometry_memory == b.geometry_memory;
}

// Buffers of a checkpoint body after the header, in file order
// (main.mm:1302-1306): actor, critic, their Adam moments, then the
// simulator's states, runs, worlds, sensor ring, pose ring, command ring.
// TrainingPotentialControl (16 B) + TrainingPotentialGridSpec (44 B) + the
// 64-byte field hash (training_potential.hpp:33-52; main.mm:1259-1262)
constexpr size_t kShapingBlockBytes = 16 + 44 + 64;
const uint32_t kCheckpointBuffers[] = {MDN_BUF_ACTOR, MDN_BUF_CRITIC, MDN_BUF_ACTOR_M, MDN_BUF_ACTOR_V,
                                       MDN_BUF_CRITIC_M, MDN_BUF_CRITIC_V, MDN_BUF_STATES, MDN_BUF_RUNS,
                                       MDN_BUF_WORLDS, MDN_BUF_SENSORS, MDN_BUF_POSES, MDN_BUF_COMMANDS};

bool valid_navpol_meta(const MdnNavPolicyMeta& m) {  // deployment.hpp:260-267
    return m.version == 1 && m.observation_count == MDN_ACTOR_OBS_PRIOR && m.hidden_count == MDN_HIDDEN &&
           m.action_count == MDN_ACTIONS && m.policy_mode == 17 && m.weight_count == kNavPolicyWeights &&
           std::isfinite(m.max_speed_mps) && m.max_speed_mps > 0 && m.sensor_rows == 16 && m.sensor_columns == 20 &&
           std::fabs(m.range_max_m - 12.0f) < 1.0e-6f && std::fabs(m.navigation_period_s - 0.05f) < 1.0e-6f &&
           std::fabs(m.native_period_s - 0.01f) < 1.0e-6f && m.memory_frames == 8 && m.body_frame == 0x00554c46u;
}

}  // namespace

extern "C" {

int mdn_checkpoint_read(const char* path, MdnCheckpointHeader* header, float* actor, uint64_t actor_count) {
    if (!path || !header) return fail(MDN_E_ARG, "mdn_checkpoint_read: null argument");
    File file(path, "rb");
    if (!file.f) return fail(MDN_E_ARG, std::string("cannot open checkpoint: ") + path);
    int rc = read_checkpoint_header(file, header);
    if (rc) return rc;
    if (actor) {
        if (actor_count != header->actor_count) return fail(MDN_E_ARG, "actor count differs from the checkpoint's");
        if (!file.read(actor, size_t(actor_count) * 4)) return fail(MDN_E_ARG, "evaluation policy read");
    }
    return MDN_OK;
}

int mdn_checkpoint_read_params(const char* path, MdnCheckpointHeader* header, float* actor, uint64_t actor_count,
                               float* critic, uint64_t critic_count) {
    if (!path || !header) return fail(MDN_E_ARG, "mdn_checkpoint_read_params: null argument");
    File file(path, "rb");
    if (!file.f) return fail(MDN_E_ARG, std::string("cannot open checkpoint: ") + path);
    int rc = read_checkpoint_header(file, header);
    if (rc) return rc;
    if (actor && actor_count != header->actor_count) return fail(MDN_E_ARG, "task actor dimensions");
    if (critic && critic_count != header->critic_count)
        return fail(MDN_E_ARG, "task critic dimensions: incompatible warmstart");
    std::vector<float> skip;
    if (!actor && critic) skip.resize(header->actor_count);
    float* first = actor ? actor : skip.data();
    if ((actor || critic) && !file.read(first, size_t(header->actor_count) * 4))
        return fail(MDN_E_ARG, "task parameter load failed");
    if (critic && !file.read(critic, size_t(critic_count) * 4)) return fail(MDN_E_ARG, "task parameter load failed");
    return MDN_OK;
}

int mdn_ppo_load_checkpoint(MdnPPO* p, const char* path, uint32_t family, uint32_t horizon, uint32_t n, uint32_t seed,
                            uint32_t* completed_rollouts) {
    if (!p || !path) return fail(MDN_E_ARG, "mdn_ppo_load_checkpoint: null argument");
    MdnSim* s = p->sim;
    if (completed_rollouts) *completed_rollouts = 0;
    File file(path, "rb");
    if (!file.f) return MDN_OK;  // no checkpoint: a fresh start (main.mm:1219)
    MdnCheckpointHeader h;
    int rc = read_checkpoint_header(file, &h);
    if (rc) return rc;
    if (h.actor_count != s->shape.actor_count() || h.critic_count != s->shape.critic_count())
        return fail(MDN_E_ARG, "PPO checkpoint dimensions mismatch");
    if (h.family != family || h.horizon != horizon || h.n != n || h.base_seed != seed)
        return fail(MDN_E_ARG, "PPO checkpoint config mismatch");
    // main.mm:1225-1226: before version 10 a checkpoint had the legacy camera
    if (h.version < 10 && s->camera_profile.id != MDN_CAMERA_LEGACY)
        return fail(MDN_E_ARG, "legacy checkpoint cannot resume with calibrated sensors; use an explicit parameter "
                               "warmstart");
    if (h.horizon != s->horizon || !same_run_settings(h.config, s->cfg))
        return fail(MDN_E_ARG, "PPO checkpoint simulator settings mismatch");
    if (h.optimizer_step > uint64_t(UINT32_MAX)) return fail(MDN_E_ARG, "PPO checkpoint Adam step is too large");
    std::vector<std::vector<unsigned char>> body;
    for (uint32_t id : kCheckpointBuffers) {
        uint64_t bytes = 0;
        rc = mdn_sim_buffer_bytes(s, id, &bytes);
        if (rc) return rc;
        body.emplace_back(bytes, 0);
        if (id == MDN_BUF_POSES && h.version < 6) continue;  // older files have no pose ring
        if (!file.read(body.back().data(), bytes)) return fail(MDN_E_ARG, "truncated PPO checkpoint");
    }
    // versions 7-8 (main.mm:1237-1257): the runtime and task configuration
    // (version 7 stored the 144-byte task control of its time and resumes
    // only without tasks), every env's plant and task state, then the
    // nominal plant and controller, all of which must equal this sim's
    std::vector<unsigned char> env_phys, task_states;
    if (h.version >= 7) {
        MdnRuntimeConfig saved_runtime;
        MdnTaskControl saved_tasks;
        std::memset(&saved_runtime, 0, sizeof(saved_runtime));
        std::memset(&saved_tasks, 0, sizeof(saved_tasks));
        if (!file.read(&saved_runtime, sizeof(saved_runtime)) ||
            !file.read(&saved_tasks, h.version >= 8 ? sizeof(saved_tasks) : 144))
            return fail(MDN_E_ARG, "truncated navigation runtime configuration");
        if (h.version < 8 && saved_tasks.enabled != 0)
            return fail(MDN_E_ARG, "task-generator semantics changed; use an explicit parameter warmstart from "
                                   "version 7");
        if (std::memcmp(&saved_runtime, &s->runtime, sizeof(saved_runtime)) != 0 ||
            std::memcmp(&saved_tasks, &s->task, sizeof(saved_tasks)) != 0)
            return fail(MDN_E_ARG, "checkpoint dynamics/task configuration mismatch");
        env_phys.resize(size_t(s->cfg.n) * sizeof(MdnPhysicsParams));
        task_states.resize(size_t(s->cfg.n) * sizeof(MdnTaskState));
        MdnPhysicsParams saved_nominal;
        std::vector<float> saved_raptor(2084), raptor(2084);
        if (!file.read(env_phys.data(), env_phys.size()) || !file.read(task_states.data(), task_states.size()) ||
            !file.read(&saved_nominal, sizeof(saved_nominal)) || !file.read(saved_raptor.data(), 2084 * 4))
            return fail(MDN_E_ARG, "truncated checkpoint nominal plant/controller");
        HIP_TRY(hipMemcpy(raptor.data(), s->raptor, 2084 * 4, hipMemcpyDeviceToHost));
        if (std::memcmp(&saved_nominal, &s->phys, sizeof(saved_nominal)) != 0 ||
            std::memcmp(saved_raptor.data(), raptor.data(), 2084 * 4) != 0)
            return fail(MDN_E_ARG, "checkpoint nominal plant/controller mismatch");
    } else if (s->runtime.enabled != 0u || s->task.enabled != 0u) {  // main.mm:1254-1257: a bank alone is fine
        return fail(MDN_E_ARG, "legacy resume cannot infer new dynamics/task state; use explicit parameter warmstart");
    }
    // version 9 (main.mm:1258-1266): the shaping control, grid spec and field
    // hash, which must equal this sim's.  This sim trains without the
    // training potential, i.e. with the reference's disabled block: a
    // value-initialised control and grid and a zeroed hash (main.mm:534-536).
    if (h.version >= 9) {
        unsigned char shaping[kShapingBlockBytes];
        if (!file.read(shaping, sizeof(shaping))) return fail(MDN_E_ARG, "truncated shaping configuration");
        for (unsigned char c : shaping)
            if (c != 0)
                return fail(MDN_E_ARG, "checkpoint shaping configuration or field hash mismatch: it was trained with "
                                       "the geodesic training potential, which this build does not run; use an "
                                       "explicit parameter warmstart");
    }
    // version 10 (main.mm:1268-1277): the camera contract, which must be this
    // sim's profile
    if (h.version >= 10) {
        MdnCameraProfile saved;
        const MdnCameraProfile& c = s->camera_profile;
        if (!file.read(&saved, sizeof(saved)) || saved.id != c.id || saved.tan_h != c.tan_h ||
            saved.tan_v != c.tan_v || saved.mount_x_m != c.mount_x_m || saved.min_range_m != c.min_range_m ||
            saved.max_range_m != c.max_range_m)
            return fail(MDN_E_ARG, "checkpoint camera contract mismatch; use an explicit parameter warmstart");
    }
    if (!file.at_end()) return fail(MDN_E_ARG, "PPO checkpoint has trailing data");
    for (size_t i = 0; i < body.size(); i++) {
        rc = mdn_sim_upload(s, kCheckpointBuffers[i], body[i].data(), body[i].size());
        if (rc) return rc;
    }
    if (h.version >= 7) {
        if ((rc = mdn_sim_upload(s, MDN_BUF_ENV_PHYSICS, env_phys.data(), env_phys.size())) != MDN_OK) return rc;
        if ((rc = mdn_sim_upload(s, MDN_BUF_TASK_STATES, task_states.data(), task_states.size())) != MDN_OK)
            return rc;
    }
    rc = mdn_sim_set_config(s, &h.config);
    if (rc) return rc;
    p->optimizer_step = h.optimizer_step;
    if (completed_rollouts) *completed_rollouts = h.completed_rollouts;
    return MDN_OK;
}

int mdn_ppo_save_checkpoint(MdnPPO* p, const char* path, uint32_t family, uint32_t seed, uint32_t completed_rollouts) {
    if (!p || !path) return fail(MDN_E_ARG, "mdn_ppo_save_checkpoint: null argument");
    MdnSim* s = p->sim;
    MdnCheckpointHeader h;
    std::memset(&h, 0, sizeof(h));  // padding bytes too, so equal states give equal files
    std::memcpy(h.magic, "PPOFIX1", 7);
    // main.mm:1292-1293: version 10 with the native camera; else 8 with the
    // dynamics/task blocks when per-episode plants or tasks are on, else 6
    // (version 9 needs the training potential, which this build does not run).
    // A challenge bank alone writes version 6, as in the reference.
    h.version = s->camera_profile.id == MDN_CAMERA_NATIVE                   ? 10
                : (s->runtime.enabled != 0u || s->task.enabled != 0u) ? 8
                                                                        : 6;
    h.actor_count = s->shape.actor_count();
    h.critic_count = s->shape.critic_count();
    h.horizon = s->horizon;
    h.n = s->cfg.n;
    h.family = family;
    h.base_seed = seed;
    h.completed_rollouts = completed_rollouts;
    h.optimizer_step = p->optimizer_step;
    h.config = s->cfg;
    h.config.tick = 0;
    const std::string temp = std::string(path) + ".tmp";
    {
        File file(temp.c_str(), "wb");
        if (!file.f) return fail(MDN_E_ARG, "cannot write PPO checkpoint: " + temp);
        bool ok = file.write(&h, sizeof(h));
        for (uint32_t id : kCheckpointBuffers) {
            uint64_t bytes = 0;
            int rc = mdn_sim_buffer_bytes(s, id, &bytes);
            if (rc) return rc;
            std::vector<unsigned char> buf(bytes);
            rc = mdn_sim_download(s, id, buf.data(), bytes);
            if (rc) return rc;
            ok = ok && file.write(buf.data(), bytes);
        }
        if (h.version >= 7) {  // main.mm:1303-1307
            std::vector<unsigned char> env_phys(size_t(s->cfg.n) * sizeof(MdnPhysicsParams));
            std::vector<unsigned char> task_states(size_t(s->cfg.n) * sizeof(MdnTaskState));
            std::vector<float> raptor(2084);
            int rc = mdn_sim_download(s, MDN_BUF_ENV_PHYSICS, env_phys.data(), env_phys.size());
            if (!rc) rc = mdn_sim_download(s, MDN_BUF_TASK_STATES, task_states.data(), task_states.size());
            if (rc) return rc;
            HIP_TRY(hipMemcpy(raptor.data(), s->raptor, 2084 * 4, hipMemcpyDeviceToHost));
            ok = ok && file.write(&s->runtime, sizeof(s->runtime)) && file.write(&s->task, sizeof(s->task)) &&
                 file.write(env_phys.data(), env_phys.size()) && file.write(task_states.data(), task_states.size()) &&
                 file.write(&s->phys, sizeof(s->phys)) && file.write(raptor.data(), 2084 * 4);
        }
        if (h.version >= 9) {  // main.mm:1310-1312: the disabled shaping block
            const unsigned char shaping[kShapingBlockBytes] = {};
            ok = ok && file.write(shaping, sizeof(shaping));
        }
        if (h.version >= 10) ok = ok && file.write(&s->camera_profile, sizeof(s->camera_profile));  // 1313-1317
        ok = ok && std::fflush(file.f) == 0;
        if (!ok) {
            std::remove(temp.c_str());
            return fail(MDN_E_ARG, "PPO checkpoint write failed: " + temp);
        }
    }
    if (std::rename(temp.c_str(), path) != 0) {
        std::remove(temp.c_str());
        return fail(MDN_E_ARG, std::string("cannot replace PPO checkpoint: ") + path);
    }
    return MDN_OK;
}

int mdn_fnv1a64_file(const char* path, uint64_t* hash) {
    if (!path || !hash) return fail(MDN_E_ARG, "mdn_fnv1a64_file: null argument");
    File file(path, "rb");
    if (!file.f) return fail(MDN_E_ARG, std::string("cannot hash: ") + path);
    uint64_t h = 14695981039346656037ull;  // FNV-1a 64 (deployment.hpp:122-136)
    unsigned char buf[16384];
    size_t got;
    while ((got = std::fread(buf, 1, sizeof(buf), file.f)) > 0)
        for (size_t i = 0; i < got; i++) { h ^= buf[i]; h *= 1099511628211ull; }
    if (std::ferror(file.f)) return fail(MDN_E_ARG, std::string("read error while hashing: ") + path);
    *hash = h;
    return MDN_OK;
}

int mdn_navpol_read(const char* path, MdnNavPolicyMeta* meta, float* weights, uint64_t count, uint64_t* source_hash) {
    if (!path || !meta || !weights) return fail(MDN_E_ARG, "mdn_navpol_read: null argument");
    if (count != kNavPolicyWeights) return fail(MDN_E_ARG, "navigation policy holds 12,104 actor weights");
    File file(path, "rb");
    if (!file.f) return fail(MDN_E_ARG, std::string("cannot open navigation policy: ") + path);
    char magic[8];
    if (!file.read(magic, 8) || std::memcmp(magic, "NAVPOL1\0", 8) != 0)
        return fail(MDN_E_ARG, "navigation policy magic mismatch");
    MdnNavPolicyMeta m;
    if (!file.read(&m, sizeof(m))) return fail(MDN_E_ARG, "truncated navigation policy metadata");
    if (!valid_navpol_meta(m)) return fail(MDN_E_ARG, "unsupported navigation policy metadata");
    std::vector<float> w(kNavPolicyWeights);
    if (!file.read(w.data(), w.size() * 4)) return fail(MDN_E_ARG, "invalid navigation actor weight");
    for (float v : w)
        if (!std::isfinite(v)) return fail(MDN_E_ARG, "invalid navigation actor weight");
    char tag[8];
    uint64_t hash = 0;
    if (!file.read(tag, 8) || std::memcmp(tag, "NAVSRC1\0", 8) != 0 || !file.read(&hash, 8))
        return fail(MDN_E_ARG, "navigation source provenance is missing");
    if (!file.at_end()) return fail(MDN_E_ARG, "navigation policy has trailing bytes");
    *meta = m;
    std::memcpy(weights, w.data(), w.size() * 4);
    if (source_hash) *source_hash = hash;
    return MDN_OK;
}

int mdn_navpol_write(const char* path, const MdnNavPolicyMeta* meta, const float* weights, uint64_t count,
                     uint64_t source_hash) {
    if (!path || !meta || !weights) return fail(MDN_E_ARG, "mdn_navpol_write: null argument");
    if (count != kNavPolicyWeights || !valid_navpol_meta(*meta))
        return fail(MDN_E_ARG, "invalid NAV actor export dimensions or metadata");
    for (uint64_t i = 0; i < count; i++)
        if (!std::isfinite(weights[i])) return fail(MDN_E_ARG, "actor has a non-finite parameter");
    const std::string temp = std::string(path) + ".tmp";
    {
        File file(temp.c_str(), "wb");
        if (!file.f) return fail(MDN_E_ARG, "cannot create navigation policy: " + temp);
        const bool ok = file.write("NAVPOL1\0", 8) && file.write(meta, sizeof(*meta)) &&
                        file.write(weights, size_t(count) * 4) && file.write("NAVSRC1\0", 8) &&
                        file.write(&source_hash, 8) && std::fflush(file.f) == 0;
        if (!ok) {
            std::remove(temp.c_str());
            return fail(MDN_E_ARG, "navigation policy write failed");
        }
    }
    if (std::rename(temp.c_str(), path) != 0) {
        std::remove(temp.c_str());
        return fail(MDN_E_ARG, std::string("cannot replace navigation policy: ") + path);
    }
    return MDN_OK;
}

// navigation_wide_deployment.hpp:92-105 (WideNavigationPolicy::valid_metadata /
// valid_sensor with deployment.hpp:66-70 for the native camera)
static bool valid_navwid(const MdnNavPolicyMeta& m, const MdnSensorContract& c) {
    const bool meta = m.version == 4 && m.observation_count == 184 && m.hidden_count >= 64 && m.hidden_count <= 8192 &&
                      m.action_count == 4 && m.policy_mode == 17 && m.weight_count == 189 * m.hidden_count + 8 &&
                      std::isfinite(m.max_speed_mps) && m.max_speed_mps > 0 && m.max_speed_mps <= 10 &&
                      m.sensor_rows == 16 && m.sensor_columns == 20 && std::fabs(m.range_max_m - 12) < 1e-6f &&
                      std::fabs(m.navigation_period_s - .05f) < 1e-6f &&
                      std::fabs(m.native_period_s - .01f) < 1e-6f && m.memory_frames == 8 &&
                      m.body_frame == 0x00554C46u;
    const bool legacy = c.profile_id == 1 && std::fabs(c.tan_h - 1) < 1e-6f && std::fabs(c.tan_v - .75f) < 1e-6f &&
                        std::fabs(c.mount_x_m) < 1e-6f;
    const bool native = c.profile_id == 2 && std::fabs(c.tan_h - 1.0f) < 1e-6f && std::fabs(c.tan_v - 0.8f) < 1e-6f &&
                        std::fabs(c.mount_x_m - 0.08f) < 1e-6f;
    return meta && (legacy || native) && std::fabs(c.min_range_m - .03f) < 1e-6f &&
           std::fabs(c.max_range_m - 12) < 1e-6f && c.noise_m == 0 && c.reserved == 0;
}

int mdn_navwid_read(const char* path, MdnNavPolicyMeta* meta, MdnSensorContract* camera, float* weights,
                    uint64_t count, uint64_t* source_hash) {
    if (!path || !meta || !camera) return fail(MDN_E_ARG, "mdn_navwid_read: null argument");
    File file(path, "rb");
    if (!file.f) return fail(MDN_E_ARG, std::string("cannot open wide policy: ") + path);
    char magic[8];
    if (!file.read(magic, 8) || std::memcmp(magic, "NAVWID4\0", 8) != 0)
        return fail(MDN_E_ARG, "wide policy magic mismatch");
    MdnNavPolicyMeta m;
    MdnSensorContract c;
    if (!file.read(&m, sizeof(m))) return fail(MDN_E_ARG, "truncated wide metadata");
    if (!file.read(&c, sizeof(c))) return fail(MDN_E_ARG, "truncated camera contract");
    if (!valid_navwid(m, c)) return fail(MDN_E_ARG, "unsupported wide policy contract");
    *meta = m;
    *camera = c;
    if (!weights) return MDN_OK;  // header only: the caller sizes the weights from meta
    if (count != m.weight_count) return fail(MDN_E_ARG, "wide policy weight count differs from the buffer");
    std::vector<float> w(m.weight_count);
    if (!file.read(w.data(), w.size() * 4)) return fail(MDN_E_ARG, "truncated wide weights");
    for (float v : w)
        if (!std::isfinite(v)) return fail(MDN_E_ARG, "non-finite wide weight");
    char tag[8];
    uint64_t hash = 0;
    if (!file.read(tag, 8) || std::memcmp(tag, "NAVSRC4\0", 8) != 0 || !file.read(&hash, 8))
        return fail(MDN_E_ARG, "missing wide provenance");
    if (!file.at_end()) return fail(MDN_E_ARG, "wide policy has trailing bytes");
    std::memcpy(weights, w.data(), w.size() * 4);
    if (source_hash) *source_hash = hash;
    return MDN_OK;
}

int mdn_navwid_write(const char* path, const MdnNavPolicyMeta* meta, const MdnSensorContract* camera,
                     const float* weights, uint64_t count, uint64_t source_hash) {
    if (!path || !meta || !camera || !weights) return fail(MDN_E_ARG, "mdn_navwid_write: null argument");
    if (!valid_navwid(*meta, *camera) || count != meta->weight_count)
        return fail(MDN_E_ARG, "invalid wide policy contract or weight count");
    for (uint64_t i = 0; i < count; i++)
        if (!std::isfinite(weights[i])) return fail(MDN_E_ARG, "non-finite actor parameter");
    const std::string temp = std::string(path) + ".tmp";
    {
        File file(temp.c_str(), "wb");
        if (!file.f) return fail(MDN_E_ARG, "cannot create wide policy: " + temp);
        const bool ok = file.write("NAVWID4\0", 8) && file.write(meta, sizeof(*meta)) &&
                        file.write(camera, sizeof(*camera)) && file.write(weights, size_t(count) * 4) &&
                        file.write("NAVSRC4\0", 8) && file.write(&source_hash, 8) && std::fflush(file.f) == 0;
        if (!ok) {
            std::remove(temp.c_str());
            return fail(MDN_E_ARG, "wide policy write failed");
        }
    }
    if (std::rename(temp.c_str(), path) != 0) {
        std::remove(temp.c_str());
        return fail(MDN_E_ARG, std::string("cannot replace wide policy: ") + path);
    }
    return MDN_OK;
}

}  // extern "C"
