/*
 * mdnav_types.h — byte layouts shared by the C ABI, the HIP kernels and the
 * CPU oracle.  Every struct reproduces the host layout of the reference so a
 * caller can hand over buffers it already holds:
 *
 *   MdnPhysicsState  == RLPhysicsState   physics.hpp:12-18   (68 B)
 *   MdnPhysicsParams == RLPhysicsParams  physics.hpp:20-38   (352 B)
 *   MdnRaptorWeights == RaptorWeights    raptor.hpp:11-21    (8336 B)
 *   MdnObstacle/World== WObstacle/WWorld world.hpp:28-29     (40 B / 676 B)
 *   MdnSimRun        == SimRun           main.mm:454-460     (184 B)
 *   MdnSimConfig     == SimConfig        main.mm:461-464     (84 B)
 *
 * Plain C so that cgo/ctypes/JNI style bindings can include it directly.
 */
#ifndef MDNAV_TYPES_H
#define MDNAV_TYPES_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Sensor contract of the legacy camera (sensor_profile.hpp:39-50). */
#define MDN_SENSOR_WIDTH 20u
#define MDN_SENSOR_HEIGHT 16u
#define MDN_SENSOR_PIXELS 320u
#define MDN_SENSOR_FRAMES 8u
#define MDN_POOLED_FEATURES 80u
#define MDN_SENSOR_TAN_H 1.0f
#define MDN_SENSOR_TAN_V 0.75f /* legacy profile (world.hpp::wcamera) */
/* native profile: the measured 20x16 planar range finder, 0.08 m forward of
 * the body reference point (sensor_profile.hpp:18-25, 46-51) */
#define MDN_SENSOR_NATIVE_TAN_V 0.8f
#define MDN_SENSOR_NATIVE_MOUNT_X 0.08f
#define MDN_SENSOR_MIN_RANGE 0.03f
#define MDN_CAMERA_LEGACY 1u
#define MDN_CAMERA_NATIVE 2u
#define MDN_SENSOR_MAX_RANGE 12.0f
#define MDN_MAX_OBSTACLES 16u

/* World families of the moving-threat mix, numbered after the reference's
 * 0-16 (world.hpp:293-318).  MDN_FAMILY_C3_MIX picks per env lane n % 4,
 * the reference's static / long / course lane split of 50/25/25
 * (navigation_training_mix.py:25-38): lanes 0 and 1 the mover world with the
 * config's goal distance, lane 2 the mover world with a long goal, lane 3 a
 * combined course.  The mover world is family 1's eight boxes plus four
 * kind-3 bounded movers (world.hpp:26-41); the course follows the combined
 * course of navigation_challenge_tasks.py:47-117. */
#define MDN_FAMILY_C3_MIX 32u
#define MDN_FAMILY_MOVERS 33u
#define MDN_FAMILY_MOVERS_LONG 34u
#define MDN_FAMILY_COURSE 35u
#define MDN_C3_LANE_FAMILY(env) \
    ((env) % 4u < 2u ? MDN_FAMILY_MOVERS : ((env) % 4u == 2u ? MDN_FAMILY_MOVERS_LONG : MDN_FAMILY_COURSE))

/* Policy shapes (ppo.hpp:26-45 with FIXED_PPO_ACTOR_OBS_DIM=181). */
#define MDN_CONTEXT_DIM 21u
#define MDN_ACTOR_OBS_POOLED 181u
/* pooled observation + the 3-value geometry-prior hint (ppo.hpp:30, 77) */
#define MDN_ACTOR_OBS_PRIOR 184u
#define MDN_CRITIC_OBS 32u
#define MDN_HIDDEN 64u
#define MDN_ACTIONS 4u

typedef struct MdnPhysicsState {
    float position[3];
    float orientation_wxyz[4];
    float linear_velocity[3];
    float angular_velocity_body[3];
    float rpm[4];
} MdnPhysicsState;

typedef struct MdnPhysicsParams {
    float rotor_positions[12];
    float rotor_thrust_directions[12];
    float rotor_torque_directions[12];
    float rotor_thrust_coefficients[12];
    float rotor_torque_constants[4];
    float rotor_time_constants_rising[4];
    float rotor_time_constants_falling[4];
    float inertia[9];
    float inertia_inverse[9];
    float gravity_world[3];
    float mass;
    float action_min;
    float action_max;
    float dt;
    float position_limit;
    float velocity_limit;
    float angular_velocity_limit;
} MdnPhysicsParams;

typedef struct MdnRaptorWeights {
    float input_weights[16 * 22];
    float input_bias[16];
    float gru_input_weights[48 * 16];
    float gru_hidden_weights[48 * 16];
    float gru_input_bias[48];
    float gru_hidden_bias[48];
    float initial_hidden_state[16];
    float output_weights[4 * 16];
    float output_bias[4];
} MdnRaptorWeights;

typedef struct MdnObstacle {
    uint32_t kind; /* 0 box, 1 sphere, 2 cylinder, 3 bounded mover */
    float center[3], size[3], velocity[3];
} MdnObstacle;

typedef struct MdnWorld {
    MdnObstacle obstacles[16];
    uint32_t count, seed, family;
    float goal[3], wind[3];
} MdnWorld;

typedef struct MdnSimRun {
    float hidden[16], motors[4], previous_nav[4], desired_velocity[3], yaw;
    uint32_t rng, steps;
    float path, elapsed, peak_speed, min_clearance, initial_distance;
    uint32_t successes, collisions, timeouts, episodes;
    float success_time, total_path, total_elapsed, final_progress, reference_position[3];
} MdnSimRun;

typedef struct MdnSimConfig {
    uint32_t n, tick, mode, family, substeps, sensor_period, sensor_delay, command_delay, max_steps, seed, eval;
    float speed, distance, wind, depth_noise, dropout, risk_coef, entropy_coef, learning_rate;
    uint32_t velocity_contract, geometry_memory;
} MdnSimConfig;

/* PPOFIX1 checkpoint header (PpoCheckpointHeader, main.mm:978-984), 136
 * bytes: magic "PPOFIX1\0", then the trainer's counters and the SimConfig. */
typedef struct MdnCheckpointHeader {
    char magic[8];
    uint32_t version, actor_count, critic_count, horizon, n, family;
    uint32_t base_seed, completed_rollouts;
    uint64_t optimizer_step;
    MdnSimConfig config;
} MdnCheckpointHeader;

/* NAVPOL1 deployed-policy metadata (nav_deployment::Metadata,
 * deployment.hpp:72-88), 56 bytes in file order. */
typedef struct MdnNavPolicyMeta {
    uint32_t version, observation_count, hidden_count, action_count, policy_mode, weight_count;
    float max_speed_mps;
    uint32_t sensor_rows, sensor_columns;
    float range_max_m, navigation_period_s, native_period_s;
    uint32_t memory_frames, body_frame;
} MdnNavPolicyMeta;

/* Episode dynamics variation (RLPhysicsDomainRange, physics_domain.hpp:17-24;
 * NavigationRuntimeConfig, navigation_runtime.hpp:9-14).  With `enabled`
 * set, every env steps with its own plant parameters, drawn at each episode
 * reset when domain_amplitude > 0 (sim.metal:63-69). */
typedef struct MdnDomainRange {
    float mass_scale_min, mass_scale_max;
    float inertia_axis_scale_min, inertia_axis_scale_max;
    float thrust_gain_min, thrust_gain_max;
    float rising_lag_scale_min, rising_lag_scale_max;
    float falling_lag_scale_min, falling_lag_scale_max;
    float minimum_thrust_to_weight;
} MdnDomainRange;

typedef struct MdnRuntimeConfig {
    uint32_t enabled;
    float domain_amplitude;
    uint32_t domain_seed;
    MdnDomainRange domain_range;
} MdnRuntimeConfig;

/* Goal-conditioned navigation tasks (navigation_tasks.hpp:64-95, 150-188):
 * a generated world, start state and goal per episode, stable-arrival
 * success and the task reward. */
#define MDN_TASK_STAGE_OPEN_GOAL 0u
#define MDN_TASK_STAGE_NEAR_GOAL_HOLD 1u
#define MDN_TASK_STAGE_CLUTTER_GOAL 2u
#define MDN_TASK_OBJECTIVE_WAYPOINT 0u
#define MDN_TASK_OBJECTIVE_FINAL_HOLD 1u
#define MDN_TASK_INVALID_CONFIG 1u
#define MDN_TASK_UNSUPPORTED_DYNAMIC 2u
#define MDN_TASK_EXHAUSTED 3u
#define MDN_TASK_READY 4u
#define MDN_TASK_UNSUPPORTED_FAMILY 5u
#define MDN_TASK_MAX_WITNESS_POINTS 4u
#define MDN_TASK_MAX_ATTEMPTS 64u

typedef struct MdnTaskConfig {
    uint32_t family, stage, objective, require_detour, max_generation_attempts, max_nav_steps;
    float scene_distance_m, difficulty, goal_distance_min_m, goal_distance_max_m;
    float minimum_endpoint_clearance_m, minimum_witness_clearance_m;
    float goal_radius_m, stable_speed_mps, stable_hold_s, nav_period_s;
    float initial_speed_min_mps, initial_speed_max_mps;
    float progress_reward_per_m, time_cost_per_s, contact_penalty, stable_arrival_bonus, command_smoothness_weight;
    float start_min_xyz[3], start_max_xyz[3], goal_min_xyz[3], goal_max_xyz[3];
    uint32_t generation_version;
} MdnTaskConfig;

typedef struct MdnTaskControl {
    uint32_t enabled;
    MdnTaskConfig config;
} MdnTaskControl;

typedef struct MdnTaskState {
    uint32_t generation_status, valid, generation_attempts, family, stage, objective, max_nav_steps;
    uint32_t step_count, stable_ticks, was_inside_goal, waypoint_event_latched, terminal;
    float start_position[3], start_yaw_rad, start_velocity_world[3], goal_position[3];
    float initial_distance_m, previous_distance_m, difficulty;
    float start_clearance_m, goal_clearance_m, direct_segment_clearance_m;
    float witness_min_clearance_m, witness_length_m, stable_time_s;
    float last_executed_world_command[4];
    uint32_t witness_point_count;
    float witness_points[4][3];
} MdnTaskState;

/* Frozen challenge bank (ChallengeBankControl, main.mm:511-514): with
 * `enabled`, every reset takes its world from the bank per schedule slot
 * (sim.metal:95-121). */
typedef struct MdnBankControl {
    uint32_t enabled, bank_count, schedule_stride, horizon;
} MdnBankControl;
#define MDN_BANK_REHEARSAL 0xffffffffu /* schedule slot: a generated rehearsal world */

/* Camera contract of a wide deployed policy (nav_deployment::SensorContract,
 * deployment.hpp:54-63), 32 bytes: profile 1 legacy, 2 native. */
typedef struct MdnSensorContract {
    uint32_t profile_id;
    float tan_h, tan_v, mount_x_m, min_range_m, max_range_m, noise_m;
    uint32_t reserved;
} MdnSensorContract;

/* Camera profile (nav_sensor::Profile, sensor_profile.hpp:113-126), 24 bytes:
 * the contract a PPOFIX1 version-10 checkpoint carries. */
typedef struct MdnCameraProfile {
    uint32_t id;
    float tan_h, tan_v, mount_x_m, min_range_m, max_range_m;
} MdnCameraProfile;

/* Rollout metrics of cpu_reference.hpp:55-70. */
typedef struct MdnMetrics {
    double wall_seconds;
    uint64_t updates, episodes, successes, collisions, timeouts;
    double final_progress, total_path, total_elapsed, success_time;
    float policy_loss, value_loss, entropy_loss, ratio;
} MdnMetrics;

#ifdef __cplusplus
}
static_assert(sizeof(MdnPhysicsState) == 68, "RLPhysicsState layout");
static_assert(sizeof(MdnPhysicsParams) == 352, "RLPhysicsParams layout");
static_assert(sizeof(MdnRaptorWeights) == 2084 * 4, "RaptorWeights layout");
static_assert(sizeof(MdnWorld) == 676, "WWorld layout");
static_assert(sizeof(MdnSimRun) == 184, "SimRun layout");
static_assert(sizeof(MdnSimConfig) == 84, "SimConfig layout");
static_assert(sizeof(MdnCheckpointHeader) == 136, "PpoCheckpointHeader layout");
static_assert(sizeof(MdnNavPolicyMeta) == 56, "NAV metadata layout");
static_assert(sizeof(MdnRuntimeConfig) == 56, "NavigationRuntimeConfig layout");
static_assert(sizeof(MdnTaskConfig) == 144, "NavigationTaskConfig layout");
static_assert(sizeof(MdnTaskControl) == 148, "NavigationTaskControl layout");
static_assert(sizeof(MdnTaskState) == 192, "NavigationTaskState layout");
static_assert(sizeof(MdnBankControl) == 16, "ChallengeBankControl layout");
static_assert(sizeof(MdnSensorContract) == 32, "SensorContract layout");
static_assert(sizeof(MdnCameraProfile) == 24, "nav_sensor::Profile layout");
#endif

#endif /* MDNAV_TYPES_H */
