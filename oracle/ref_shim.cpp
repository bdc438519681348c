/*
 * ref_shim.cpp — C entry points over the reference's own header-only C++
 * (world.hpp, sensor_profile.hpp, physics.hpp, raptor.hpp, ppo.hpp), compiled
 * from the reference tree where it lies (oracle/Makefile target `ref`).
 * TEST INFRASTRUCTURE ONLY: used to pin the oracle's restatement against the
 * reference's code with the platform libm.  Nothing here is copied; the shim
 * only includes those headers and forwards to their functions.
 * cpu_reference.hpp and the Metal sources are not buildable here (Accelerate,
 * GCD, Metal); the oracle restates them.
 */
#ifndef FIXED_PPO_ACTOR_OBS_DIM
#define FIXED_PPO_ACTOR_OBS_DIM 181  // pooled actor; the Makefile also builds 184
#endif
#include <math.h>  // physics_domain.hpp calls the C library's isfinite unqualified
#include <cstdint>
#include <cstring>
#include <vector>

#include "world.hpp"
#include "sensor_profile.hpp"
#include "physics.hpp"
#include "raptor.hpp"
#include "ppo.hpp"
#include "guidance.hpp"
#include "physics_domain.hpp"
#include "navigation_runtime.hpp"
#include "navigation_tasks.hpp"
#include "deployment.hpp"
#include "navigation_wide_deployment.hpp"
#include "mdnav_types.h"

static_assert(sizeof(WWorld) == sizeof(MdnWorld), "world layout");
static_assert(sizeof(RLPhysicsState) == sizeof(MdnPhysicsState), "state layout");
static_assert(sizeof(RLPhysicsParams) == sizeof(MdnPhysicsParams), "params layout");
static_assert(sizeof(RaptorWeights) == sizeof(MdnRaptorWeights), "raptor layout");
static_assert(sizeof(RLPhysicsDomainRange) == sizeof(MdnDomainRange), "domain range layout");
static_assert(sizeof(NavigationRuntimeConfig) == sizeof(MdnRuntimeConfig), "runtime config layout");
static_assert(sizeof(NavigationTaskConfig) == sizeof(MdnTaskConfig), "task config layout");
static_assert(sizeof(NavigationTaskControl) == sizeof(MdnTaskControl), "task control layout");
static_assert(sizeof(NavigationTaskState) == sizeof(MdnTaskState), "task state layout");
static_assert(sizeof(nav_deployment::Metadata) == sizeof(MdnNavPolicyMeta), "NAV metadata layout");
static_assert(sizeof(nav_deployment::SensorContract) == sizeof(MdnSensorContract), "sensor contract layout");

extern "C" {

// physics_domain.hpp:98-155 and navigation_tasks.hpp:99-548
int ref_sample_domain(const MdnPhysicsParams* nominal, uint32_t* rng, float amplitude, const MdnDomainRange* range,
                      MdnPhysicsParams* varied, float* sample) {
    RLPhysicsDomainSample s{};
    const bool ok = rl_physics_sample_domain(*reinterpret_cast<const RLPhysicsParams*>(nominal), *rng, amplitude,
                                             *reinterpret_cast<const RLPhysicsDomainRange*>(range),
                                             *reinterpret_cast<RLPhysicsParams*>(varied), s);
    std::memcpy(sample, &s, sizeof(s));
    return ok ? 1 : 0;
}
void ref_domain_stress_range(MdnDomainRange* r) {
    const RLPhysicsDomainRange v = rl_physics_domain_stress_range();
    std::memcpy(r, &v, sizeof(v));
}
int ref_task_default_config(MdnTaskConfig* c, uint32_t stage, uint32_t family, float difficulty) {
    return navigation_task_default_config(*reinterpret_cast<NavigationTaskConfig*>(c), stage, family, difficulty) ? 1 : 0;
}
uint32_t ref_generate_task(MdnWorld* w, MdnTaskState* t, uint32_t* rng, const MdnTaskConfig* c) {
    return navigation_generate_task(*reinterpret_cast<WWorld*>(w), *reinterpret_cast<NavigationTaskState*>(t), *rng,
                                    *reinterpret_cast<const NavigationTaskConfig*>(c));
}
// WideNavigationPolicy::load and raw_mean (navigation_wide_deployment.hpp:15-66)
int ref_navwid_load(const char* path, MdnNavPolicyMeta* meta, MdnSensorContract* camera, uint64_t* hash,
                    const float* obs, uint32_t n, float* means) {
    nav_deployment::WideNavigationPolicy p;
    std::string error;
    if (!p.load(path, &error)) return 0;
    std::memcpy(meta, &p.metadata(), sizeof(*meta));
    std::memcpy(camera, &p.sensor_contract(), sizeof(*camera));
    *hash = p.source_checkpoint_hash();
    for (uint32_t i = 0; i < n; i++)
        if (!p.raw_mean(obs + size_t(i) * 184, means + size_t(i) * 4)) return -1;
    return 1;
}
void ref_task_apply_start(const MdnTaskState* t, MdnPhysicsState* s) {
    navigation_task_apply_start(*reinterpret_cast<const NavigationTaskState*>(t), *reinterpret_cast<RLPhysicsState*>(s));
}
void ref_task_step(MdnTaskState* t, const MdnTaskConfig* c, const float* pos, const float* vel, const float* executed,
                   uint32_t contact, uint32_t forced_timeout, float* out) {
    const NavigationTaskStep r = navigation_task_step(*reinterpret_cast<NavigationTaskState*>(t),
                                                      *reinterpret_cast<const NavigationTaskConfig*>(c), pos, vel,
                                                      executed, contact, forced_timeout);
    out[0] = r.reward; out[1] = r.goal_distance_m; out[2] = r.actual_speed_mps;
    out[3] = float(r.waypoint_passed); out[4] = float(r.stable_success); out[5] = float(r.collision);
    out[6] = float(r.timeout); out[7] = float(r.episode_done);
}

void ref_generate_world(MdnWorld* w, uint32_t seed, uint32_t family, float distance) {
    std::memset(w, 0, sizeof(*w));
    wgenerate(*reinterpret_cast<WWorld*>(w), seed, family, distance);
}
uint32_t ref_training_family(uint32_t family, uint32_t* rng) { return wtraining_family(family, *rng); }
uint32_t ref_xorshift(uint32_t* s) { return wrng(*s); }
float ref_urand(uint32_t* s) { return wurand(*s); }
void ref_ray_world_batch(const MdnWorld* worlds, const float* rays, const float* times, uint32_t rays_per_world,
                         float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) {
        const WWorld& w = reinterpret_cast<const WWorld*>(worlds)[i / rays_per_world];
        const float* r = rays + 6 * i;
        out[i] = wray(w, wv(r[0], r[1], r[2]), wv(r[3], r[4], r[5]), times[i / rays_per_world]);
    }
}
void ref_clearance_batch(const MdnWorld* worlds, const float* points, const float* times, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++)
        out[i] = wclearance(reinterpret_cast<const WWorld*>(worlds)[i], wv(points[3 * i], points[3 * i + 1], points[3 * i + 2]), times[i]);
}
// wc (world.hpp:32-41): obstacle i's centre at time t
void ref_obstacle_center(const MdnWorld* w, uint32_t i, float t, float* out) {
    const WVec c = wc(reinterpret_cast<const WWorld*>(w)->obstacles[i], t);
    out[0] = c.x; out[1] = c.y; out[2] = c.z;
}
void ref_camera_rays(float* out) {
    for (uint32_t k = 0; k < NAV_SENSOR_PIXELS; k++) {
        const WVec r = nav_sensor_pixel_ray(NAV_SENSOR_TAN_H, NAV_SENSOR_ACTIVE_TAN_V, k);
        out[3 * k] = r.x; out[3 * k + 1] = r.y; out[3 * k + 2] = r.z;
    }
}
// the native profile's rays and either profile's contract (sensor_profile.hpp:111-126)
void ref_camera_rays_native(float* out) {
    for (uint32_t k = 0; k < NAV_SENSOR_PIXELS; k++) {
        const WVec r = nav_sensor_pixel_ray(NAV_SENSOR_TAN_H, NAV_SENSOR_NATIVE_TAN_V, k);
        out[3 * k] = r.x; out[3 * k + 1] = r.y; out[3 * k + 2] = r.z;
    }
}
void ref_camera_profile(uint32_t id, void* out) {
    const nav_sensor::Profile p = nav_sensor::by_id(id);
    static_assert(sizeof(p) == 24, "nav_sensor::Profile layout");
    std::memcpy(out, &p, sizeof(p));
}
void ref_physics_step_batch(const MdnPhysicsState* s, const float* actions, const float* winds,
                            const MdnPhysicsParams* p, MdnPhysicsState* out, uint64_t n) {
    for (uint64_t i = 0; i < n; i++)
        rl_physics_step(reinterpret_cast<const RLPhysicsState*>(s)[i], actions + 4 * i, winds + 3 * i,
                        *reinterpret_cast<const RLPhysicsParams*>(p), reinterpret_cast<RLPhysicsState*>(out)[i]);
}
void ref_crazyflie_params(MdnPhysicsParams* p) {
    const RLPhysicsParams q = rl_physics_crazyflie_default();
    std::memcpy(p, &q, sizeof(q));
}
void ref_raptor_sequence(const MdnRaptorWeights* w, const float* obs, uint32_t steps, float* actions, float* hidden_out) {
    const RaptorWeights& rw = *reinterpret_cast<const RaptorWeights*>(w);
    float h[16];
    raptor_reset(rw, h);
    for (uint32_t t = 0; t < steps; t++) raptor_forward(rw, obs + 22 * t, h, actions + 4 * t);
    std::memcpy(hidden_out, h, sizeof(h));
}
void ref_raptor_forward(const MdnRaptorWeights* w, const float* obs, float* hidden, float* action) {
    raptor_forward(*reinterpret_cast<const RaptorWeights*>(w), obs, hidden, action);
}
void ref_raptor_pack_observation(const float* position, const float* orientation, const float* world_velocity,
                                 const float* body_rates, const float* target_position,
                                 const float* target_orientation, const float* target_velocity,
                                 const float* previous_action, float* observation) {
    raptor_pack_observation(position, orientation, world_velocity, body_rates, target_position, target_orientation,
                            target_velocity, previous_action, observation);
}
void ref_quaternion_matrix(const float* q, float* r) { raptor_quaternion_matrix(q, r); }

int ref_ppo_self_tests(float tolerance) { return fixed_ppo::run_cpu_self_tests(tolerance) ? 1 : 0; }
uint32_t ref_actor_param_count() { return uint32_t(fixed_ppo::actor_param_count); }
uint32_t ref_critic_param_count() { return uint32_t(fixed_ppo::critic_param_count); }
void ref_actor_forward(const float* params, const float* obs, float* hidden, float* mean) {
    fixed_ppo::ActorParams p;
    std::memcpy(p.values.data(), params, sizeof(p.values));
    fixed_ppo::actor_forward(obs, p, hidden, mean);
}
float ref_critic_forward(const float* params, const float* obs, float* hidden) {
    fixed_ppo::CriticParams p;
    std::memcpy(p.values.data(), params, sizeof(p.values));
    return fixed_ppo::critic_forward(obs, p, hidden);
}
float ref_gaussian_log_prob(const float* a, const float* m, const float* ls) { return fixed_ppo::gaussian_log_prob(a, m, ls); }
void ref_compute_gae(uint32_t horizon, uint32_t n, const float* r, const float* v, const float* nv,
                     const uint8_t* te, const uint8_t* tr, float gamma, float lambda, float* adv, float* ret) {
    fixed_ppo::compute_gae(horizon, n, r, v, nv, te, tr, gamma, lambda, adv, ret);
}
void ref_normalize_advantages(float* a, uint64_t count, float eps) { fixed_ppo::normalize_advantages(a, count, eps); }
void ref_sample_loss_and_grad(const float* action, const float* mean, const float* log_std, float old_logp,
                              float old_value, float value, float advantage, float target, float batch, float clip,
                              float vcoef, float ecoef, float* d_mean, float* d_log_std, float* d_value,
                              float* losses4) {
    const fixed_ppo::PpoLoss l = fixed_ppo::sample_loss_and_grad(action, mean, log_std, old_logp, old_value, value,
                                                                 advantage, target, batch, clip, vcoef, ecoef, d_mean,
                                                                 d_log_std, d_value);
    losses4[0] = l.policy; losses4[1] = l.value; losses4[2] = l.entropy; losses4[3] = l.ratio;
}
// Per-sample backprop reduced over the batch (ppo.hpp:269-308), the
// reference's own oracle for its batched gradient kernels.
void ref_actor_critic_grads(const float* actor, const float* critic, const float* obs, const float* cobs,
                            const float* d_mean, const float* d_log_std, const float* d_value, uint32_t batch,
                            float* actor_grad, float* critic_grad) {
    using namespace fixed_ppo;
    ActorParams ap;
    CriticParams cp;
    std::memcpy(ap.values.data(), actor, sizeof(ap.values));
    std::memcpy(cp.values.data(), critic, sizeof(cp.values));
    std::vector<float> apart(size_t(batch) * actor_param_count), cpart(size_t(batch) * critic_param_count);
    float hidden[hidden_dim], mean[action_dim];
    for (uint32_t n = 0; n < batch; n++) {
        actor_forward(obs + size_t(n) * actor_obs_dim, ap, hidden, mean);
        actor_backward_sample(obs + size_t(n) * actor_obs_dim, hidden, d_mean + 4 * n, d_log_std + 4 * n, ap,
                              apart.data() + size_t(n) * actor_param_count);
        critic_forward(cobs + size_t(n) * critic_obs_dim, cp, hidden);
        critic_backward_sample(cobs + size_t(n) * critic_obs_dim, hidden, d_value[n], cp,
                               cpart.data() + size_t(n) * critic_param_count);
    }
    reduce_sample_grads<actor_param_count>(apart.data(), batch, actor_grad);
    reduce_sample_grads<critic_param_count>(cpart.data(), batch, critic_grad);
}
void ref_adam_update(float* params, const float* grad, float* first, float* second, uint64_t count, uint64_t step,
                     float lr, float b1, float b2, float eps, float wd) {
    fixed_ppo::adam_update(params, grad, first, second, count, step, lr, b1, b2, eps, wd);
}

// guidance.hpp:38-98 and 152-194 (the CPU reference's call: clearances computed
// directly, capture age 0), legacy sensor profile
void ref_guidance(const float* cur, const float* prev, const float* goal, float distance, const float* vel,
                  float sensor_dt, float* hint) {
    nav_guidance(cur, prev, goal, distance, vel, sensor_dt, NAV_SENSOR_ACTIVE_TAN_V, hint);
}
void ref_guidance_memory(const float* cur, const float* prev, const float* goal, float distance, const float* vel,
                         float sensor_dt, const float* range_ring, const float* pose_ring, const float* pose,
                         uint32_t latest_frame, uint32_t valid_frames, float* hint) {
    nav_guidance_memory(cur, prev, goal, distance, vel, sensor_dt, NAV_SENSOR_ACTIVE_TAN_V, range_ring, pose_ring,
                        pose, latest_frame, valid_frames, hint, nullptr, 0.0f);
}
void ref_memory_clearance(const float* direction, const float* range_ring, const float* pose_ring, const float* pose,
                          uint32_t latest_frame, uint32_t valid_frames, float sensor_dt, float* out) {
    *out = nav_memory_clearance(direction, range_ring, pose_ring, pose, latest_frame, valid_frames, sensor_dt,
                                NAV_SENSOR_ACTIVE_TAN_V);
}
} // extern "C"
