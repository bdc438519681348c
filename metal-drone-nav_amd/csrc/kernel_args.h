// kernel_args.h — argument blocks and launchers shared by the kernels and
// the host side of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mdnav_types.h"

namespace nav {
struct RolloutArgs {
    float* state;          // [17][N]
    uint32_t* run;         // [46][N]
    float* world;          // [N][169]
    float* sensors;        // [N][8][320]
    // pooled 2x2 minima of the last K frames, slot f % K ([N][K][80]): the
    // ring the four-wavefront kernels with K > 2 keep in HBM (their LDS has
    // no room for it); rebuilt from `sensors` at every launch
    float* pool_ring;
    float* poses;          // [N][8][12]
    float* commands;       // [N][8][4]
    const float* raptor;   // RaptorWeights, 2084 floats
    const float* actor;    // flat actor vector (ppo.hpp:35-40)
    const float* actor_w1t;   // W1 transposed [OBS][64]
    const float* critic;      // flat critic vector (ppo.hpp:41-45)
    const float* critic_w1t;  // [32][64]
    const float* camera;      // unit pixel rays [320][3]
    const float* cells;       // pooled-cell directions [80][3] (guidance.hpp:21-26 nav_ray)
    float sensor_dt;          // sensor period in seconds: period x dt x substeps (sim.metal:226)
    float mount_x;            // camera mount ahead of the body point (sim.metal:151)
    float tan_v;              // camera vertical half-tangent (sensor_profile.hpp:46-51)
    double inv_sensor_dt;     // RN64(1 / max(sensor_dt, 1e-3)), the guidance's closing-speed divisor
    float* obs;            // [T][N][181]
    float* co;             // [T][N][32]
    float* nco;            // [T][N][32] critic observation of s'
    float* actions;        // [T][N][4]
    float* logp;           // [T][N]
    float* values;
    float* rewards;
    float* next_values;
    uint8_t* terminated;
    uint8_t* truncated;
    MdnSimConfig cfg;
    MdnPhysicsParams phys;
    // RN64 reciprocals of the plant's divisors (mass, rising and falling
    // rotor time constants), computed on the host so that they arrive as
    // uniform kernel arguments (scalar registers) instead of occupying
    // vector registers for the whole launch
    double recip_mass, recip_rise[4], recip_fall[4];
    // 1 when the nominal plant has the standard quadrotor structure
    // (derivative_quad applies); set by the host per launch
    uint32_t quad;
    uint32_t count;        // ticks in this launch
    uint32_t horizon;      // row blocks of the rollout buffers
    // Split ticks (policy evaluated outside the kernel, e.g. a wide actor):
    // tick t of this launch writes row block (tick0 + t) % horizon; means come
    // from ext_means [T][N][4] and log_std from ext_log_std; values and next
    // values are left to the caller.
    // The in-kernel policy (ext_means null) runs split ticks too: a launch
    // that begins at act reloads the observation rows of its first tick.
    const float* ext_means;
    const float* ext_log_std;
    uint32_t tick0;
    uint32_t split;        // SPLIT_* flags
    // Geometry-memory hint (184-input actor, cfg.geometry_memory): instead of
    // the memory-less hint, observe writes the env's memory header [N][16]
    // (MEM_HEAD_* words) and a separate kernel writes the hint inputs of the
    // tick's rows before the launch that acts on them.
    uint32_t* mem_head;
    // Per-episode plants and navigation tasks (the rollout kernels built for
    // them, one tick per launch): env_phys [N] are the plants the envs step
    // with (sim.metal:287); with task_cfg set, task_states [N] take the
    // task's step and its outcome replaces success, timeout and reward
    // (sim.metal:307-315).
    const MdnPhysicsParams* env_phys;
    MdnTaskState* task_states;
    const MdnTaskConfig* task_cfg;
    // challenge bank: each row's level id [T][N] (sim.metal:317), from the
    // env's active level [N] (null: no bank, rows get MDN_BANK_REHEARSAL)
    const uint32_t* bank_active;
    uint32_t* bank_transition;
};
// Per-episode work after a reset (rollout.hip episode_kernel): the
// episode's plant and hover rpm (sim.metal:62-81) and its navigation task
// (sim.metal:122-141), for every env (first) or the envs whose episode
// restarted in the preceding launch (steps == 0).
struct EpisodeArgs {
    float* state;
    uint32_t* run;
    float* world;
    MdnPhysicsParams* env_phys;
    MdnTaskState* task_states;
    MdnSimConfig cfg;
    MdnPhysicsParams phys;
    MdnRuntimeConfig runtime;
    MdnTaskControl task;
    uint32_t first;
    // challenge bank (sim.metal:95-121): worlds [count][WORLD_WORDS],
    // schedule [N][stride]; a reset takes slot `slot` (0 at the first reset,
    // tick + 1 after a reset at tick)
    const float* bank_worlds;
    const uint32_t* bank_schedule;
    uint32_t* bank_active;
    MdnBankControl bank;
    uint32_t slot;
};
// memory header words
constexpr uint32_t MEM_HEAD_OBSERVED = 0;  // 1: observed this tick (else skip the env)
constexpr uint32_t MEM_HEAD_FRAME = 1;     // newest usable frame (absolute; ring slot = frame % 8)
constexpr uint32_t MEM_HEAD_VALID = 2;     // frames usable since reset (cpu_reference.hpp:366-367)
constexpr uint32_t MEM_HEAD_DISTANCE = 3;  // goal distance (float bits)
constexpr uint32_t MEM_HEAD_POSE = 4;      // position [3], body-to-world rotation row-major [9] (float bits)
constexpr uint32_t MEM_HEAD_WORDS = 16;

// Geometry-memory hint of one tick's rows (memory.hip).
struct MemoryArgs {
    const uint32_t* head;   // [N][MEM_HEAD_WORDS] written by the tick's observation
    float* obs;             // the tick's rows [N][184]; the kernel writes inputs 181-183
    const float* sensors;   // [N][8][320] range ring
    const float* poses;     // [N][8][12] pose ring
    const float* pix_rays;  // [320][3] unit rays through the raw pixels (guidance.hpp:122)
    const float* cells;     // [80][3] pooled-cell rays (nav_ray)
    float sensor_dt;
    float tan_v;            // camera vertical half-tangent (the goal's field-of-view test)
    double inv_sensor_dt;
    uint32_t n;
};
// The first tick's depth and observation were produced by the previous launch.
constexpr uint32_t SPLIT_BEGIN_AT_ACT = 1;
// The last tick stops after its observation (its means are not known yet).
constexpr uint32_t SPLIT_END_AFTER_OBSERVE = 2;
}  // namespace nav

namespace ppo {
struct RowArgs {
    const float* obs;       // minibatch rows [b][OBS]
    const float* co;        // [b][COBS]
    const float* actions;   // [b][4]
    const float* old_logp;  // [b]
    const float* adv;       // [b]
    const float* ret;       // [b]
    // (mean, inv) when the rows' advantages are still to be normalised:
    // each row's (adv - mean) * inv is used and stored back to adv_out
    const float* norm = nullptr;
    float* adv_out = nullptr;  // [b]
    const float* actor;     // flat params
    const float* actor_w1t; // [OBS][HID]
    const float* critic;
    const float* critic_w1t; // [COBS][HID]
    float* part;            // [ceil(b/256)][P_TOTAL] per-chunk gradient and metric partials
    uint32_t b;
    float clip, vcoef, ecoef;
    uint32_t d;             // actor inputs: 181, or 184 with the geometry-prior hint
};

// cpu_reference.hpp:553-567 inputs for one update of both networks.
// One minibatch of at most 256 rows (a single gradient chunk) split over many
// workgroups: the row-parallel forward writes per-row records to `rec`, the
// parameter-parallel pass writes the finished gradient to `grad`.
struct MbArgs {
    RowArgs r;
    float* rec;   // [MB_REC_WORDS]: h and delta of actor and critic [4][256][64], row scalars [256][16]
    float* grad;  // P_TOTAL: actor, critic, metric sums
};
constexpr uint32_t MB_ROWS = 256, MB_REC_WORDS = 4 * 256 * 64 + 256 * 16;

struct AdamArgs {
    float* actor; float* critic; float* actor_w1t; float* critic_w1t;
    float* am; float* av; float* cm; float* cv;
    const float* grad;   // P_TOTAL: actor, critic, metric sums
    float* metric_row;   // [4]
    float* norm_row;     // [2] pre-clip gradient norms, actor then critic (main.mm:1370-1373)
    float lr, c1, c2;    // host bias corrections 1-beta^step
    uint32_t b;
    uint32_t d;          // actor inputs
    uint32_t keep_w1t = 1;  // 0: leave actor_w1t / critic_w1t for one transpose after the update
};
}  // namespace ppo

// Per-sample loss and derivatives of fixed_ppo::sample_loss_and_grad over a
// batch (fixed_ppo.hip); log_std is shared (stride 0) or per row (stride 4).
struct fppo_loss_args {
    const float* actions; const float* means; const float* log_std; const float* old_logp;
    const float* values; const float* advantages; const float* returns;
    float* d_mean; float* d_log_std; float* d_value; float* losses;
    uint64_t b;
    uint32_t ls_stride;
    float batch_size, clip, vcoef, ecoef;
};

extern "C" {
hipError_t nav_launch_reset(const nav::RolloutArgs* a, hipStream_t stream);
hipError_t nav_launch_episode(const nav::EpisodeArgs* a, hipStream_t stream);
hipError_t nav_launch_rollout(const nav::RolloutArgs* a, int lanes_per_env, int ring_slots, uint32_t actor_obs,
                              hipStream_t stream);
hipError_t nav_launch_memory_hint(const nav::MemoryArgs* a, hipStream_t stream);
hipError_t nav_launch_validate(const MdnTaskState* tasks, const MdnPhysicsParams* phys, uint32_t n, uint32_t* out,
                               hipStream_t stream);
hipError_t nav_launch_raptor_fixture(const float* RW, const float* obs, uint32_t steps, uint32_t copies,
                                     float* actions, float* hidden, int lanes_per_env, hipStream_t st);
hipError_t nav_launch_physics_fixture(const MdnPhysicsState* in, const float* actions, const float* winds,
                                      const MdnPhysicsParams* P, MdnPhysicsState* out, uint64_t n, hipStream_t st);
hipError_t nav_launch_ray_fixture(const float* worlds, const float* rays, const float* times, uint32_t rays_per_world,
                                  float* out, uint64_t n, hipStream_t st);
hipError_t nav_launch_clearance_fixture(const float* worlds, const float* points, const float* times, float* out,
                                        uint64_t n, hipStream_t st);
hipError_t ppo_launch_gae(const float* r, const float* v, const float* nv, const uint8_t* te, const uint8_t* tr,
                          float* adv, float* ret, uint32_t horizon, uint32_t n, float gamma, float lambda,
                          hipStream_t st);
hipError_t ppo_launch_normalize(float* a, uint64_t count, double* part, float* stats, float eps, hipStream_t st);
// The statistics only (stats = mean, inv) when apply == 0.
hipError_t ppo_launch_normalize_stats(float* a, uint64_t count, double* part, float* stats, float eps, int apply,
                                      hipStream_t st);
// doubles of ppo_launch_normalize's `part` for `count` elements: a 32-bit
// ticket that must be zero when allocated, then both passes' partials, one
// per group of 64 chunks of 256 elements
constexpr uint64_t ppo_normalize_part_words(uint64_t count) { return 1 + 2 * ((count + 16383) / 16384); }
hipError_t ppo_launch_rows(const ppo::RowArgs* a, hipStream_t st);
hipError_t ppo_launch_grads(float* part, float* grad, uint32_t b, uint32_t d, hipStream_t st);
hipError_t ppo_launch_minibatch(const ppo::MbArgs* m, hipStream_t st);
hipError_t ppo_launch_adam(const ppo::AdamArgs* a, hipStream_t st);
hipError_t ppo_launch_transpose(const float* actor, const float* critic, float* aw, float* cw, uint32_t d,
                                hipStream_t st);
hipError_t ppo_launch_metric_mean(const float* rows, float* mean, uint32_t updates, hipStream_t st);
// wide-policy kernels (large.hip)
hipError_t lp_launch_pack(const float* W, uint32_t H, uint32_t D, uint32_t K, __bf16* out, hipStream_t st);
hipError_t lp_launch_prep(const float* obs, const float* co, uint32_t B, uint32_t d, __bf16* xa, __bf16* xaT,
                          __bf16* xc, __bf16* xcT, bool transposed, hipStream_t st);
hipError_t lp_launch_forward(const __bf16* xa, const __bf16* xc, const __bf16* awb, const __bf16* cwb,
                             const float* actor, const float* critic, uint32_t H, uint32_t d, uint32_t B,
                             const float* prior, float* means, float* values, float* part, hipStream_t st);
uint64_t lp_forward_part_floats(uint32_t B);
hipError_t lp_launch_next_value_split(const float* co, const float* nco, const float* values, uint32_t ticks,
                                      uint32_t N, float* next_values, uint32_t* count, uint32_t* idx, float* gather,
                                      hipStream_t st);
hipError_t lp_launch_next_value_scatter(const uint32_t* idx, const float* vals, uint32_t n, float* next_values,
                                        hipStream_t st);
hipError_t lp_launch_logp(const float* means, const float* actions, const float* log_std, uint32_t B, float* logp,
                          hipStream_t st);
hipError_t lp_launch_loss(const float* means, const float* values, const float* actions, const float* old_logp,
                          const float* adv, const float* ret, const float* log_std, uint32_t B, float clip,
                          float vcoef, float ecoef, float* dm, float* dls, float* dv, float* loss, float* col_part,
                          hipStream_t st);
hipError_t lp_launch_backward(const __bf16* xa, const __bf16* xaT, const __bf16* xc, const __bf16* xcT,
                              const __bf16* awb, const __bf16* cwb, const float* actor, const float* critic,
                              const float* dm, const float* dv, const float* col_part, uint32_t H, uint32_t d,
                              uint32_t B, float* part, float* ga, float* gc, float* scratch, hipStream_t st);
uint64_t lp_backward_part_floats(uint32_t B, uint32_t H, uint32_t d);
uint64_t lp_adam_scratch_floats();
hipError_t lp_launch_adam(float* actor, float* critic, float* am, float* av, float* cm, float* cv, __bf16* awb,
                          __bf16* cwb, float* ga, float* gc, float* scratch, uint32_t B, uint32_t H, uint32_t d,
                          float lr, float c1, float c2, float* metric_row, float* norm_row, hipStream_t st);
uint32_t ppo_partial_stride(uint32_t d);
// fixed_ppo operators over caller arrays (fixed_ppo.hip)
hipError_t fppo_launch_forward(const float* w, const float* x, uint32_t D, uint32_t H, uint32_t O, uint32_t prior,
                               uint64_t B, float* hidden, float* out, hipStream_t st);
hipError_t fppo_launch_log_prob(const float* act, const float* mean, const float* log_std, uint32_t ls_stride,
                                uint64_t B, float* out, hipStream_t st);
hipError_t fppo_launch_loss_grad(const fppo_loss_args* a, hipStream_t st);
hipError_t fppo_launch_adam(float* p, const float* g, float* m, float* v, uint64_t n, float lr, float b1, float b2,
                            float eps, float wd, float c1, float c2, hipStream_t st);
}
