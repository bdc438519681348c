/*
 * mdnav.h — C ABI of the MI355X hot path (libmdnav.so).
 *
 * Drop-in for the reference's GPU host classes: the Sim and PPOTrainer of
 * main.mm (Metal) and, through include/mdnav.hpp, the Trainer interface of
 * cpu_reference.hpp.  Plain pointers and sizes only; every function returns
 * 0 on success and a negative MDN_E_* code otherwise, with the message in
 * mdn_last_error() (the reference throws std::runtime_error through
 * require(), main.mm:27; mdnav.hpp turns codes back into exceptions).
 * Handles own their device memory; host arrays are caller-owned copies in the
 * reference's host layouts (AoS structs, time-major [T][N] rollout rows).
 * One host thread per handle; all work is ordered on the handle's stream.
 */
#ifndef MDNAV_H
#define MDNAV_H

#include <stddef.h>
#include <stdint.h>

#include "mdnav_types.h"

#ifdef __cplusplus
extern "C" {
#endif

#define MDN_OK 0
#define MDN_E_ARG -1     /* invalid argument or size */
#define MDN_E_HIP -2     /* HIP runtime error (message names the call) */
#define MDN_E_STATE -3   /* call not valid in the handle's state */

typedef struct MdnSim MdnSim;
typedef struct MdnPPO MdnPPO;
typedef struct MdnLargePPO MdnLargePPO;

/* Buffer ids for mdn_sim_download / mdn_sim_upload.  Sizes follow the
 * reference's shared buffers of Sim (main.mm:519, 540-555). */
enum MdnBuffer {
    MDN_BUF_STATES = 0,      /* MdnPhysicsState[N]            states       */
    MDN_BUF_RUNS = 1,        /* MdnSimRun[N]                  runs         */
    MDN_BUF_WORLDS = 2,      /* MdnWorld[N]                   worlds       */
    MDN_BUF_SENSORS = 3,     /* float[N][8][320]              sensors      */
    MDN_BUF_POSES = 4,       /* float[N][8][12]               poses        */
    MDN_BUF_COMMANDS = 5,    /* float[N][8][4]                commands     */
    MDN_BUF_ACTOR = 6,       /* float[actor_param_count]      actor        */
    MDN_BUF_CRITIC = 7,      /* float[critic_param_count]     critic       */
    MDN_BUF_OBS = 8,         /* float[T][N][181 or 184]       obs          */
    MDN_BUF_CRITIC_OBS = 9,  /* float[T][N][32]               co           */
    MDN_BUF_ACTIONS = 10,    /* float[T][N][4]                actions      */
    MDN_BUF_LOGP = 11,       /* float[T][N]                   logp         */
    MDN_BUF_VALUES = 12,
    MDN_BUF_REWARDS = 13,
    MDN_BUF_NEXT_VALUES = 14,
    MDN_BUF_TERMINATED = 15, /* uint8[T][N] */
    MDN_BUF_TRUNCATED = 16,  /* uint8[T][N] */
    MDN_BUF_ADVANTAGES = 17,
    MDN_BUF_RETURNS = 18,
    MDN_BUF_ACTOR_M = 19,    /* PPO Adam moments (needs a PPO handle) */
    MDN_BUF_ACTOR_V = 20,
    MDN_BUF_CRITIC_M = 21,
    MDN_BUF_CRITIC_V = 22,
    MDN_BUF_METRIC_ROWS = 23, /* float[updates][4] of the last rollout_update */
    MDN_BUF_NEXT_CRITIC_OBS = 24, /* float[T][N][32] critic observation of s' (the next_values input) */
    MDN_BUF_ENV_PHYSICS = 25, /* MdnPhysicsParams[N]  environment_physics (main.mm:537): each env's plant */
    MDN_BUF_TASK_STATES = 26, /* MdnTaskState[N]      task_states (main.mm:523) */
    MDN_BUF_BANK_ACTIVE_IDS = 27,     /* uint32[N]     bank_active_ids: each env's challenge level */
    MDN_BUF_BANK_TRANSITION_IDS = 28, /* uint32[T][N]  bank_transition_ids: the level of each row */
    MDN_BUF_BANK_SCHEDULE = 29,       /* uint32[N][stride] bank_schedule (after mdn_sim_set_bank) */
    MDN_BUF_GRAD_NORM_ROWS = 30       /* float[updates][2] grad_norm_rows (main.mm:1111, 1370-1373): the
                                         pre-clip actor and critic gradient norms of each update of the last
                                         rollout_update (needs a PPO handle; the wide policy's
                                         summary is mdn_lppo_grad_norm_summary) */
};

/* Kernel ids for mdn_sim_kernel_time. */
enum MdnKernel {
    MDN_K_ROLLOUT = 0,   /* fused env step + rollout forward, all ticks of one collect */
    MDN_K_GAE = 1,       /* ppo_gae */
    MDN_K_NORMALIZE = 2, /* ppo_normalize_advantages (all passes) */
    MDN_K_ROWS = 3,      /* minibatch forward + loss/grad + hidden deltas */
    MDN_K_GRADS = 4,     /* gradient chunk partials + reduction */
    MDN_K_ADAM = 5,      /* norm clip + Adam + log-std clamp */
    MDN_K_LP_FORWARD = 6,  /* wide-policy forward (evaluation and minibatch) + loss terms */
    MDN_K_LP_BACKWARD = 7, /* wide-policy backward partials and their sums */
    MDN_K_LP_ADAM = 8,     /* wide-policy clip + Adam + bf16 refresh */
    MDN_K_MEMORY = 9,      /* geometry-memory hint of one tick (memory.metal + guidance.hpp:152-194) */
    MDN_K_EPISODE = 10,    /* per-episode plant draw and navigation task after resets (sim.metal:62-81, 122-141) */
    MDN_K_COUNT = 11
};

const char* mdn_last_error(void);
const char* mdn_version(void);

/* Sim(Metal&, SimConfig, horizon) — main.mm:530-563: allocates the env,
 * rollout and policy buffers, initialises the policy (seed 1789,
 * main.mm:548-554) and runs the first reset (sim_reset, main.mm:565). */
int mdn_sim_create(const MdnSimConfig* cfg, uint32_t horizon, const MdnRaptorWeights* raptor,
                   const MdnPhysicsParams* physics, MdnSim** out);
void mdn_sim_destroy(MdnSim* sim);
/* Sim::set_config (main.mm:564); n cannot change. */
int mdn_sim_set_config(MdnSim* sim, const MdnSimConfig* cfg);
int mdn_sim_get_config(const MdnSim* sim, MdnSimConfig* cfg, uint32_t* horizon);
/* Sim::reset (main.mm:565): first reset of every env. */
int mdn_sim_reset(MdnSim* sim);
/* Sim::collect(cmdbuf, count) (main.mm:573-598): `count` ticks (0 = horizon),
 * tick t writes row block t % horizon.  Asynchronous on the sim's stream. */
int mdn_sim_collect(MdnSim* sim, uint32_t count);
/* Metal::finish (main.mm:71): waits for the stream, reports GPU seconds of
 * the work since the previous sync (may be NULL). */
int mdn_sim_sync(MdnSim* sim, double* gpu_seconds);
/* Shared-buffer access (the reference reads buffer.contents, e.g.
 * navigation_training.hpp:28-29): blocking copies in host layout. */
int mdn_sim_buffer_bytes(const MdnSim* sim, uint32_t buffer, uint64_t* bytes);
int mdn_sim_download(MdnSim* sim, uint32_t buffer, void* host, uint64_t bytes);
int mdn_sim_upload(MdnSim* sim, uint32_t buffer, const void* host, uint64_t bytes);
/* Per-kernel timing with HIP events on the sim's stream. */
int mdn_sim_set_timing(MdnSim* sim, int enabled);
int mdn_sim_kernel_time(MdnSim* sim, uint32_t kernel, double* total_ms, uint64_t* launches);
int mdn_sim_reset_timing(MdnSim* sim);
/* Lanes per environment in the rollout kernel (4, 8 or 16; default 8). */
int mdn_sim_set_lanes(MdnSim* sim, uint32_t lanes);
/* Actor input width, the reference's build-time FIXED_PPO_ACTOR_OBS_DIM
 * (ppo.hpp:11-13, 30-34): 181 (pooled depth + context, the default) or 184,
 * which appends the geometry-prior hint (sim.metal:226, guidance.hpp:38-96)
 * and adds it to the first three action means (ppo.hpp:77,
 * cpu_reference.hpp:446).  Replaces the policy by a fresh initialisation of
 * the new shape (actor and critic, one seed stream) and resizes the
 * observation rows.  Call before mdn_ppo_create / mdn_lppo_create.  The
 * 184-input rollout runs 8 lanes per env.  With cfg.geometry_memory = 1 the
 * hint is the history-aware one (guidance.hpp:152-194 over the 8-frame range
 * and pose rings, cpu_reference.hpp:364-372): mdn_sim_collect then runs one
 * env launch and one memory launch per tick. */
int mdn_sim_set_actor_obs(MdnSim* sim, uint32_t actor_obs);

/* Episode dynamics variation: the reference's Sim::runtime_control
 * (NavigationRuntimeConfig, navigation_runtime.hpp:9-14, written by
 * navigation_training.hpp:20-23).  With `enabled`, every env steps with its
 * own plant (MDN_BUF_ENV_PHYSICS, sim.metal:287), drawn at each reset when
 * domain_amplitude > 0 (physics_domain.hpp:98-155 seeded per env and episode,
 * sim.metal:50-54; a rejected draw leaves a NaN mass) with hover rpm per
 * rotor (sim.metal:70-81).  Takes effect at the next mdn_sim_reset, as the
 * reference's memcpy + reset does.  mdn_sim_collect then runs one tick per
 * launch with a per-episode kernel after each (8 lanes per env). */
/* Camera profile (sensor_profile.hpp:16-25, 111-126): 1 legacy (default,
 * the source model of world.hpp::wcamera), 2 native (the measured planar
 * range finder: vertical half-tangent 0.8, rays cast from 0.08 m ahead of
 * the body point).  The reference selects it at compile time
 * (NAV_SENSOR_PROFILE); here per simulator.  It sets the pixel rays, the ray
 * origin (sim.metal:147-152), the guidance hint's cell directions and the
 * geometry memory's reprojection (guidance.hpp:21-26, 110-146), and which
 * checkpoint versions resume.  Waits for the simulator's stream. */
int mdn_sim_set_camera(MdnSim* sim, uint32_t profile_id);
int mdn_sim_get_camera(const MdnSim* sim, MdnCameraProfile* profile);
int mdn_sim_set_runtime(MdnSim* sim, const MdnRuntimeConfig* runtime);
int mdn_sim_get_runtime(const MdnSim* sim, MdnRuntimeConfig* runtime);
/* Goal-conditioned navigation tasks: Sim::task_control
 * (NavigationTaskControl, navigation_tasks.hpp:93-95).  With `enabled`,
 * each reset generates the env's world, start state and goal
 * (navigation_generate_task, navigation_tasks.hpp:355-491, seeded per env and
 * episode, sim.metal:122-141; MDN_BUF_TASK_STATES holds the task and its
 * generation status), and each tick's task step (navigation_tasks.hpp:509-548)
 * replaces success (stable arrival), timeout and reward (sim.metal:307-315).
 * config.generation_version 1 is the reference's current generator; 0 is
 * the generator before clutter goals were conditioned on the goal bounds
 * (the version of the reference's published goal-arrival evidence).  Takes
 * effect at the next mdn_sim_reset.  Enabling tasks while a challenge bank is
 * set returns MDN_E_ARG (the two cannot both own the world,
 * navigation_training.hpp:19). */
int mdn_sim_set_tasks(MdnSim* sim, const MdnTaskControl* tasks);
int mdn_sim_get_tasks(const MdnSim* sim, MdnTaskControl* tasks);
/* Frozen challenge bank: Sim::bank_worlds / bank_schedule / bank_control
 * (main.mm:522, 543-545, 2175-2178).  `count` worlds and an env-major
 * schedule [N][schedule_stride] of level ids (MDN_BANK_REHEARSAL: a generated
 * rehearsal world, family 12 or 13 alternating by env); each reset takes its
 * slot (0 at mdn_sim_reset, tick + 1 after a reset at tick) and replaces the
 * world, wind and initial distance (sim.metal:95-121); every row records
 * the env's level (MDN_BUF_BANK_TRANSITION_IDS).  count = 0 disables it.
 * Upload MDN_BUF_BANK_SCHEDULE to change the schedule between rollouts.
 * Returns MDN_E_ARG for count > 0 while navigation tasks are enabled. */
int mdn_sim_set_bank(MdnSim* sim, const MdnWorld* worlds, uint32_t count, const uint32_t* schedule,
                     uint32_t schedule_stride);
/* Sim::bank_control (ChallengeBankControl, main.mm:511-514) as
 * navigation_training::configure reads it (navigation_training.hpp:19). */
int mdn_sim_get_bank(const MdnSim* sim, MdnBankControl* bank);
/* navigation_task_default_config (navigation_tasks.hpp:99-140) and
 * rl_physics_domain_stress_range (physics_domain.hpp:37-40). */
int mdn_task_default_config(uint32_t stage, uint32_t family, float difficulty, MdnTaskConfig* out);
int mdn_domain_stress_range(MdnDomainRange* out);
int mdn_sim_get_actor_obs(const MdnSim* sim, uint32_t* actor_obs);

/* PPOTrainer(Sim&, epochs) — main.mm:1166-1217, with the minibatch size
 * (PPOTrainer::minibatch, main.mm:1113) as an argument. */
int mdn_ppo_create(MdnSim* sim, uint32_t epochs, uint32_t minibatch, MdnPPO** out);
void mdn_ppo_destroy(MdnPPO* ppo);
/* PPOTrainer::rollout_update (main.mm:1321-1384): GAE, advantage
 * normalisation, epochs x minibatches of loss/grad, norm clip, Adam,
 * log-std clamp, metric mean.  Asynchronous on the sim's stream.  The
 * advantages end normalised, as with the pieces below; the rescale itself
 * runs inside the first epoch's minibatches. */
int mdn_ppo_rollout_update(MdnPPO* ppo, uint32_t rollout_index);
/* Pieces of rollout_update, for callers that validate between them
 * (navigation_training.hpp:149-152). */
int mdn_ppo_gae(MdnPPO* ppo);
int mdn_ppo_normalize(MdnPPO* ppo);
int mdn_ppo_update(MdnPPO* ppo, uint32_t rollout_index);
/* PPOTrainer::metric_mean (main.mm:1383): [policy, value, entropy, ratio]. */
int mdn_ppo_metric_mean(MdnPPO* ppo, float out[4]);
/* PPOTrainer::GradNormSummary (main.mm:1439-1442). */
typedef struct MdnGradNormSummary {
    float actor_mean, actor_max, actor_clip_frac;
    float critic_mean, critic_max, critic_clip_frac;
} MdnGradNormSummary;
/* PPOTrainer::grad_norm_summary (main.mm:1443-1465): over the last
 * rollout_update's updates, the mean (a double sum), the maximum and the
 * fraction above the clip limit 0.5 of the pre-clip actor and critic
 * gradient norms sqrt(|g|^2 + 1e-20) (MDN_BUF_GRAD_NORM_ROWS).  Waits for the
 * sim's stream.  MDN_E_STATE, "non-finite pre-clip gradient norm", when a
 * norm is NaN or infinite (main.mm:1451); all zeros before any update. */
int mdn_ppo_grad_norm_summary(MdnPPO* ppo, MdnGradNormSummary* out);
int mdn_ppo_optimizer_step(const MdnPPO* ppo, uint64_t* step);
int mdn_ppo_updates_per_rollout(const MdnPPO* ppo, uint32_t* updates);

/* On-disk formats.
 * PPOTrainer::save_checkpoint (main.mm:1285-1317): PPOFIX1 version 6 (no
 * shaping block, the legacy camera): header, actor, critic, their Adam
 * moments, then the simulator's states, runs, worlds, sensor, pose and
 * command rings, in the reference's layouts; version 8 when per-episode
 * plants or tasks are on, which appends the runtime and task configuration,
 * every env's plant and task state, the nominal plant and the RAPTOR
 * weights; version 10 with the native camera, which appends the version-8
 * blocks, the (disabled) shaping block and the camera contract.  Version 9
 * (the training potential) is never written: this build does not run the
 * potential.  Written to path.tmp and renamed. */
int mdn_ppo_save_checkpoint(MdnPPO* ppo, const char* path, uint32_t family, uint32_t seed,
                            uint32_t completed_rollouts);
/* PPOTrainer::load_checkpoint (main.mm:1218-1284) with read_checkpoint_header
 * (main.mm:986-994): versions 3-10.  A missing file is a fresh start (MDN_OK,
 * *completed_rollouts = 0), as in the reference.  The family, horizon, env
 * count and seed must match the arguments and the run settings the
 * simulator's; versions 7 and up also their runtime and task configuration,
 * nominal plant and RAPTOR weights (set them first), and a version 7 file
 * resumes only without tasks; versions 9-10 carry a shaping block, which must
 * be the disabled one (a file trained with the potential returns MDN_E_ARG);
 * version 10 carries the camera contract, which must be the simulator's
 * profile (mdn_sim_set_camera), and older versions resume only with the
 * legacy camera.  The simulator takes the file's config. */
int mdn_ppo_load_checkpoint(MdnPPO* ppo, const char* path, uint32_t family, uint32_t horizon, uint32_t n,
                            uint32_t seed, uint32_t* completed_rollouts);
/* A checkpoint's header and, if `actor` is given, its actor parameters (the
 * prefix evaluate_checkpoint reads, main.mm:1864-1866; versions 3-10). */
int mdn_checkpoint_read(const char* path, MdnCheckpointHeader* header, float* actor, uint64_t actor_count);
/* nav_deployment::NavigationPolicy::load / write_file (deployment.hpp:142-205):
 * NAVPOL1 = magic, 56-byte metadata, 12,104 finite actor weights of the
 * 184-64-4 actor, NAVSRC1 + FNV-1a 64 hash of the source checkpoint, no
 * trailing bytes. */
int mdn_navpol_read(const char* path, MdnNavPolicyMeta* meta, float* weights, uint64_t count, uint64_t* source_hash);
int mdn_navpol_write(const char* path, const MdnNavPolicyMeta* meta, const float* weights, uint64_t count,
                     uint64_t source_hash);
/* Wide deployed policy NAVWID4 (navigation_wide_deployment.hpp:15-40, written
 * by navigation_export_wide.py:40-47): magic, the 56-byte metadata (version
 * 4, 184 inputs, hidden width H in 64..8192, 189 H + 8 weights), the 32-byte
 * camera contract, the weights of the 184-H-4 actor, NAVSRC4 + FNV-1a 64 of
 * the source checkpoint, no trailing bytes.  Read with weights = NULL for
 * the header alone. */
int mdn_navwid_read(const char* path, MdnNavPolicyMeta* meta, MdnSensorContract* camera, float* weights,
                    uint64_t count, uint64_t* source_hash);
int mdn_navwid_write(const char* path, const MdnNavPolicyMeta* meta, const MdnSensorContract* camera,
                     const float* weights, uint64_t count, uint64_t source_hash);
/* fnv1a64_file (deployment.hpp:122-136). */
int mdn_fnv1a64_file(const char* path, uint64_t* hash);

/* PPOTrainer with the reference's FIXED_PPO_HIDDEN_DIM raised to `hidden`
 * (ppo.hpp:17-45; the capacity actors of ACTOR_CAPACITY_RESULTS, width 5120
 * for the 967,688-parameter actor at 184 inputs): actor 181 -> hidden -> 4,
 * critic 32 -> hidden -> 1, fp32 parameters and Adam, first-layer GEMMs on
 * bf16 matrix cores (results within bf16 tolerance of fp32).  `hidden` must
 * be a positive multiple of 128.  Parameters start from the reference's
 * initialisation stream (seed 1789, cpu_reference.hpp:89-103).  Works on the
 * rollout buffers of `sim`. */
int mdn_lppo_create(MdnSim* sim, uint32_t hidden, uint32_t epochs, uint32_t minibatch, MdnLargePPO** out);
void mdn_lppo_destroy(MdnLargePPO* lp);
/* Log-probabilities of the stored actions and values at s and s' under the
 * wide policy, written into the sim's logp, values and next_values rows
 * (the rollout's sim_act / next-value outputs for this policy). */
int mdn_lppo_evaluate(MdnLargePPO* lp);
/* Sim::collect (main.mm:573-598) of a build whose actor is the wide policy:
 * every tick the wide actor's means drive sim_act (sim.metal:229-256); the
 * wide critic gives values at s and s' (sim.metal:254, 322).  `count` ticks,
 * 0 = horizon.  Needs 8 lanes per env. */
int mdn_lppo_collect(MdnLargePPO* lp, uint32_t count);
/* Means [rows][4] of the last mdn_lppo_collect or mdn_lppo_evaluate (the
 * actor output each row's action was sampled around / re-evaluated at);
 * count = horizon * n * 4. */
int mdn_lppo_means(MdnLargePPO* lp, float* host, uint64_t count);
/* PPOTrainer::rollout_update for the wide policy: GAE, normalisation,
 * epochs x minibatches of forward, loss, backward, clip and Adam. */
int mdn_lppo_rollout_update(MdnLargePPO* lp, uint32_t rollout_index);
/* which: 0 actor, 1 critic, 2 actor Adam m, 3 actor v, 4 critic m, 5 critic v. */
int mdn_lppo_param_count(const MdnLargePPO* lp, uint32_t which, uint64_t* count);
int mdn_lppo_get_params(MdnLargePPO* lp, uint32_t which, float* host, uint64_t count);
int mdn_lppo_set_params(MdnLargePPO* lp, uint32_t which, const float* host, uint64_t count);
int mdn_lppo_metric_mean(MdnLargePPO* lp, float out[4]);
/* mdn_ppo_grad_norm_summary for the wide policy (main.mm:1443-1465). */
int mdn_lppo_grad_norm_summary(MdnLargePPO* lp, MdnGradNormSummary* out);
int mdn_lppo_optimizer_step(const MdnLargePPO* lp, uint64_t* step);

/* Stateless operators over host arrays (the reference's fixture kernels
 * physics_fixture / raptor_fixture / world_depth / world_clearance,
 * main.mm:29-43, 74-81, and ppo_gae / ppo_normalize_advantages). */
int mdn_op_physics_step(const MdnPhysicsState* states, const float* actions, const float* winds,
                        const MdnPhysicsParams* params, MdnPhysicsState* out, uint64_t n);
/* RAPTOR over `steps` observations (obs[steps][22]) from the initial hidden
 * state, evaluated by `copies` independent lane groups: actions[copies][steps][4],
 * hidden[copies][16]. */
int mdn_op_raptor_sequence(const MdnRaptorWeights* weights, const float* obs, uint32_t steps, uint32_t copies,
                           float* actions, float* hidden);
/* rays[n][6] = origin, unit direction; world of ray i = worlds[i / rays_per_world]. */
int mdn_op_ray_world(const MdnWorld* worlds, const float* rays, const float* times, uint32_t rays_per_world,
                     float* out, uint64_t n);
int mdn_op_clearance(const MdnWorld* worlds, const float* points, const float* times, float* out, uint64_t n);
int mdn_op_gae(uint32_t horizon, uint32_t n, const float* rewards, const float* values, const float* next_values,
               const uint8_t* terminated, const uint8_t* truncated, float gamma, float lambda, float* advantages,
               float* returns);
int mdn_op_normalize(float* advantages, uint64_t count, float epsilon);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): mdn_op_normalize on `count` advantages already in device
 * memory, normalised in place, enqueued on `stream` (a hipStream_t of the
 * current device; NULL for its default stream) and not waited for.  The
 * scratch is the current device's; its address is resolved once per device,
 * so like every device pointer of the library it does not survive a
 * hipDeviceReset.  It allocates nothing: the
 * statistics' scratch is a fixed array in the library (64 KiB per GPU,
 * held until the process ends) and `count` may not exceed
 * MDN_NORMALIZE_NOALLOC_MAX (MDN_E_ARG otherwise).  Calls on one GPU share
 * that array: calls that overlap in time on one GPU (other streams, other
 * threads) race and must be serialised by the caller.  Results equal
 * mdn_op_normalize's bit for bit. */
#define MDN_NORMALIZE_NOALLOC_MAX (1ull << 26)
int mdn_op_normalize_noalloc(float* advantages, uint64_t count, float epsilon, void* stream);

/* fixed_ppo's operators (ppo.hpp:24-326), batched on the GPU over host
 * arrays.  The reference's header functions take one sample; these take
 * `batch` rows of the same layouts and return what a loop over the rows of
 * the header function returns (within the fp32 tolerance of its libm
 * transcendentals: tanh and exp are this library's own).  Parameter vectors
 * use the flat layouts of ppo.hpp:35-45 at any input width D (1..1024) and
 * hidden width H (1..8192, the reference's FIXED_PPO_*_DIM):
 * actor W1[H][D], b1[H], W2[4][H], b2[4], log_std[4]; critic W1[H][D], b1[H],
 * w2[H], b2.
 *
 * fixed_ppo::actor_forward (ppo.hpp:65-80): obs[batch][D] -> hidden[batch][H]
 * (may be NULL) and mean[batch][4]; an input width of 184 (or 824) adds the
 * last three inputs, the geometry-prior hint, to the first three means
 * (ppo.hpp:30-34, 77). */
int mdn_op_actor_forward(const float* params, uint32_t obs_dim, uint32_t hidden_dim, const float* obs, uint64_t batch,
                         float* hidden, float* means);
/* fixed_ppo::critic_forward (ppo.hpp:82-93): obs[batch][D] -> hidden[batch][H]
 * (may be NULL) and values[batch]. */
int mdn_op_critic_forward(const float* params, uint32_t obs_dim, uint32_t hidden_dim, const float* obs, uint64_t batch,
                          float* hidden, float* values);
/* fixed_ppo::gaussian_log_prob (ppo.hpp:95-103) per row of actions[batch][4]
 * and means[batch][4]; log_std is one shared [4] (log_std_stride 0) or
 * per row [batch][4] (stride 4). */
int mdn_op_gaussian_log_prob(const float* actions, const float* means, const float* log_std, uint32_t log_std_stride,
                             uint64_t batch, float* logp);
/* fixed_ppo::sample_loss_and_grad (ppo.hpp:144-181) per row: the row's
 * action, mean, log_std (shared or per row as above), old log-probability,
 * old value (unused, as in the reference), value, advantage and target
 * return, with the shared batch_size, clip, value and entropy coefficients
 * -> d_mean[batch][4], d_log_std[batch][4], d_value[batch] and
 * losses[batch][4] = PpoLoss {policy, value, entropy, ratio}. */
int mdn_op_sample_loss_and_grad(const float* actions, const float* means, const float* log_std,
                                uint32_t log_std_stride, const float* old_logp, const float* old_values,
                                const float* values, const float* advantages, const float* returns, uint64_t batch,
                                float batch_size, float clip_epsilon, float value_coefficient,
                                float entropy_coefficient, float* d_mean, float* d_log_std, float* d_value,
                                float* losses);
/* fixed_ppo::adam_update (ppo.hpp:310-324): params, first and second moments
 * updated in place; bias corrections 1 - beta^step as the reference computes
 * them (float pow on the host). */
int mdn_op_adam_update(float* params, const float* grad, float* first, float* second, uint64_t count, uint64_t step,
                       float learning_rate, float beta1, float beta2, float epsilon, float weight_decay);
/* fixed_ppo::run_cpu_self_tests (ppo.hpp:204-267) run through the operators
 * above on the GPU: finite differences on the four surrogate branches, the
 * value derivative and Adam's first step.  *passed = 1 when every check is
 * within `tolerance` (the reference's default is 2e-3). */
int mdn_op_ppo_self_tests(float tolerance, int* passed);

/* navigation_training::validate_rollout (navigation_training.hpp:27-35):
 * every env's task state is valid with generation status ready and its
 * plant mass is finite and positive.  Returns MDN_E_STATE naming the first
 * failing env ("task generation rejected env=K status=S" or "episode
 * dynamics sample rejected env=K") otherwise.  Waits for the sim's stream. */
int mdn_sim_validate_rollout(MdnSim* sim);
/* The parameters of a PPOFIX1 checkpoint (read_checkpoint_header,
 * main.mm:986-994, then the actor and critic vectors that follow it, as
 * navigation_training::load_actor reads them, navigation_training.hpp:37-62):
 * actor and critic may be NULL; non-NULL ones need exactly the header's
 * counts. */
int mdn_checkpoint_read_params(const char* path, MdnCheckpointHeader* header, float* actor, uint64_t actor_count,
                               float* critic, uint64_t critic_count);

/* Test support, no counterpart in the reference: the kernels divide by
 * constants (plant mass and rotor time constants, the RK4 weight 6, the
 * observation scales) as (float)((double)x * (1.0 / (double)b)).  For each
 * of the n divisors, counts the fp32 numerators x (all 2^32 bit patterns)
 * where that differs bitwise from the correctly rounded x / b; NaN results
 * compare equal.  Returns 0, or a negative value on a HIP error. */
int mdn_op_check_division(const float* divisors, uint32_t n, uint64_t* mismatches);

#ifdef __cplusplus
}
#endif

#endif /* MDNAV_H */
