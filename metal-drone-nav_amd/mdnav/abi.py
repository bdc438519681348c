"""Byte layouts of the C ABI (include/mdnav_types.h) as numpy dtypes.

Each dtype reproduces a host struct of the reference so arrays can be handed
across the boundary without conversion:

* ``PHYSICS_STATE``  == ``RLPhysicsState``  (physics.hpp:12-18, 68 B)
* ``PHYSICS_PARAMS`` == ``RLPhysicsParams`` (physics.hpp:20-38, 352 B)
* ``RAPTOR_WEIGHTS`` == ``RaptorWeights``   (raptor.hpp:11-21, 8336 B)
* ``WORLD``          == ``WWorld``          (world.hpp:28-29, 676 B)
* ``SIM_RUN``        == ``SimRun``          (main.mm:454-460, 184 B)
* ``SIM_CONFIG``     == ``SimConfig``       (main.mm:461-464, 84 B)
"""
import ctypes

import numpy as np

f4, u4 = np.float32, np.uint32

PHYSICS_STATE = np.dtype([
    ("position", f4, 3), ("orientation_wxyz", f4, 4), ("linear_velocity", f4, 3),
    ("angular_velocity_body", f4, 3), ("rpm", f4, 4)])

PHYSICS_PARAMS = np.dtype([
    ("rotor_positions", f4, 12), ("rotor_thrust_directions", f4, 12),
    ("rotor_torque_directions", f4, 12), ("rotor_thrust_coefficients", f4, 12),
    ("rotor_torque_constants", f4, 4), ("rotor_time_constants_rising", f4, 4),
    ("rotor_time_constants_falling", f4, 4), ("inertia", f4, 9), ("inertia_inverse", f4, 9),
    ("gravity_world", f4, 3), ("mass", f4), ("action_min", f4), ("action_max", f4), ("dt", f4),
    ("position_limit", f4), ("velocity_limit", f4), ("angular_velocity_limit", f4)])

RAPTOR_WEIGHTS = np.dtype([
    ("input_weights", f4, 352), ("input_bias", f4, 16), ("gru_input_weights", f4, 768),
    ("gru_hidden_weights", f4, 768), ("gru_input_bias", f4, 48), ("gru_hidden_bias", f4, 48),
    ("initial_hidden_state", f4, 16), ("output_weights", f4, 64), ("output_bias", f4, 4)])

OBSTACLE = np.dtype([("kind", u4), ("center", f4, 3), ("size", f4, 3), ("velocity", f4, 3)])
WORLD = np.dtype([("obstacles", OBSTACLE, 16), ("count", u4), ("seed", u4), ("family", u4),
                  ("goal", f4, 3), ("wind", f4, 3)])

SIM_RUN = np.dtype([
    ("hidden", f4, 16), ("motors", f4, 4), ("previous_nav", f4, 4), ("desired_velocity", f4, 3),
    ("yaw", f4), ("rng", u4), ("steps", u4), ("path", f4), ("elapsed", f4), ("peak_speed", f4),
    ("min_clearance", f4), ("initial_distance", f4), ("successes", u4), ("collisions", u4),
    ("timeouts", u4), ("episodes", u4), ("success_time", f4), ("total_path", f4),
    ("total_elapsed", f4), ("final_progress", f4), ("reference_position", f4, 3)])

SIM_CONFIG = np.dtype([
    ("n", u4), ("tick", u4), ("mode", u4), ("family", u4), ("substeps", u4), ("sensor_period", u4),
    ("sensor_delay", u4), ("command_delay", u4), ("max_steps", u4), ("seed", u4), ("eval", u4),
    ("speed", f4), ("distance", f4), ("wind", f4), ("depth_noise", f4), ("dropout", f4),
    ("risk_coef", f4), ("entropy_coef", f4), ("learning_rate", f4),
    ("velocity_contract", u4), ("geometry_memory", u4)])

# PpoCheckpointHeader (main.mm:978-984)
CHECKPOINT_HEADER = np.dtype([
    ("magic", "S8"), ("version", u4), ("actor_count", u4), ("critic_count", u4), ("horizon", u4), ("n", u4),
    ("family", u4), ("base_seed", u4), ("completed_rollouts", u4), ("optimizer_step", np.uint64),
    ("config", SIM_CONFIG), ("pad", u4)])

# nav_deployment::Metadata (deployment.hpp:72-88)
NAV_POLICY_META = np.dtype([
    ("version", u4), ("observation_count", u4), ("hidden_count", u4), ("action_count", u4),
    ("policy_mode", u4), ("weight_count", u4), ("max_speed_mps", f4), ("sensor_rows", u4),
    ("sensor_columns", u4), ("range_max_m", f4), ("navigation_period_s", f4), ("native_period_s", f4),
    ("memory_frames", u4), ("body_frame", u4)])

# RLPhysicsDomainRange / NavigationRuntimeConfig (physics_domain.hpp:17-24,
# navigation_runtime.hpp:9-14)
DOMAIN_RANGE = np.dtype([
    ("mass_scale", f4, 2), ("inertia_axis_scale", f4, 2), ("thrust_gain", f4, 2), ("rising_lag_scale", f4, 2),
    ("falling_lag_scale", f4, 2), ("minimum_thrust_to_weight", f4)])
RUNTIME_CONFIG = np.dtype([("enabled", u4), ("domain_amplitude", f4), ("domain_seed", u4),
                           ("domain_range", DOMAIN_RANGE)])
# RLPhysicsDomainSample (physics_domain.hpp:26-33)
DOMAIN_SAMPLE = np.dtype([("mass_scale", f4), ("inertia_axis_scale", f4, 3), ("thrust_gain", f4, 4),
                          ("rising_lag_scale", f4, 4), ("falling_lag_scale", f4, 4), ("thrust_to_weight", f4)])
# NavigationTaskConfig / Control / State (navigation_tasks.hpp:64-95, 150-178)
TASK_CONFIG = np.dtype([
    ("family", u4), ("stage", u4), ("objective", u4), ("require_detour", u4), ("max_generation_attempts", u4),
    ("max_nav_steps", u4), ("scene_distance_m", f4), ("difficulty", f4), ("goal_distance_min_m", f4),
    ("goal_distance_max_m", f4), ("minimum_endpoint_clearance_m", f4), ("minimum_witness_clearance_m", f4),
    ("goal_radius_m", f4), ("stable_speed_mps", f4), ("stable_hold_s", f4), ("nav_period_s", f4),
    ("initial_speed_min_mps", f4), ("initial_speed_max_mps", f4), ("progress_reward_per_m", f4),
    ("time_cost_per_s", f4), ("contact_penalty", f4), ("stable_arrival_bonus", f4),
    ("command_smoothness_weight", f4), ("start_min_xyz", f4, 3), ("start_max_xyz", f4, 3),
    ("goal_min_xyz", f4, 3), ("goal_max_xyz", f4, 3), ("generation_version", u4)])
TASK_CONTROL = np.dtype([("enabled", u4), ("config", TASK_CONFIG)])
TASK_STATE = np.dtype([
    ("generation_status", u4), ("valid", u4), ("generation_attempts", u4), ("family", u4), ("stage", u4),
    ("objective", u4), ("max_nav_steps", u4), ("step_count", u4), ("stable_ticks", u4), ("was_inside_goal", u4),
    ("waypoint_event_latched", u4), ("terminal", u4), ("start_position", f4, 3), ("start_yaw_rad", f4),
    ("start_velocity_world", f4, 3), ("goal_position", f4, 3), ("initial_distance_m", f4),
    ("previous_distance_m", f4), ("difficulty", f4), ("start_clearance_m", f4), ("goal_clearance_m", f4),
    ("direct_segment_clearance_m", f4), ("witness_min_clearance_m", f4), ("witness_length_m", f4),
    ("stable_time_s", f4), ("last_executed_world_command", f4, 4), ("witness_point_count", u4),
    ("witness_points", f4, (4, 3))])
TASK_READY = 4
# the episode dynamics seed of the reference's task training and evaluation
# (navigation_training.hpp:21)
TASK_DOMAIN_SEED = 0x3f84d5b5

assert RUNTIME_CONFIG.itemsize == 56 and DOMAIN_SAMPLE.itemsize == 68
assert TASK_CONFIG.itemsize == 144 and TASK_CONTROL.itemsize == 148 and TASK_STATE.itemsize == 192
# nav_deployment::SensorContract (deployment.hpp:54-63)
SENSOR_CONTRACT = np.dtype([("profile_id", u4), ("tan_h", f4), ("tan_v", f4), ("mount_x_m", f4),
                            ("min_range_m", f4), ("max_range_m", f4), ("noise_m", f4), ("reserved", u4)])
assert SENSOR_CONTRACT.itemsize == 32
# nav_sensor::Profile (sensor_profile.hpp:113-116): the camera of a simulator
# and of a PPOFIX1 version-10 checkpoint
CAMERA_PROFILE = np.dtype([("id", u4), ("tan_h", f4), ("tan_v", f4), ("mount_x_m", f4), ("min_range_m", f4),
                           ("max_range_m", f4)])
assert CAMERA_PROFILE.itemsize == 24
CAMERA_LEGACY, CAMERA_NATIVE = 1, 2
assert CHECKPOINT_HEADER.itemsize == 136 and NAV_POLICY_META.itemsize == 56
assert PHYSICS_STATE.itemsize == 68 and PHYSICS_PARAMS.itemsize == 352
assert RAPTOR_WEIGHTS.itemsize == 8336 and WORLD.itemsize == 676
assert SIM_RUN.itemsize == 184 and SIM_CONFIG.itemsize == 84


class GradNormSummary(ctypes.Structure):
    """PPOTrainer::GradNormSummary (main.mm:1439-1442)."""
    _fields_ = [("actor_mean", ctypes.c_float), ("actor_max", ctypes.c_float), ("actor_clip_frac", ctypes.c_float),
                ("critic_mean", ctypes.c_float), ("critic_max", ctypes.c_float), ("critic_clip_frac", ctypes.c_float)]


class Metrics(ctypes.Structure):
    """cpu_reference::Metrics (cpu_reference.hpp:55-70)."""
    _fields_ = [("wall_seconds", ctypes.c_double), ("updates", ctypes.c_uint64),
                ("episodes", ctypes.c_uint64), ("successes", ctypes.c_uint64),
                ("collisions", ctypes.c_uint64), ("timeouts", ctypes.c_uint64),
                ("final_progress", ctypes.c_double), ("total_path", ctypes.c_double),
                ("total_elapsed", ctypes.c_double), ("success_time", ctypes.c_double),
                ("policy_loss", ctypes.c_float), ("value_loss", ctypes.c_float),
                ("entropy_loss", ctypes.c_float), ("ratio", ctypes.c_float)]


def default_config(**overrides):
    """SimConfig defaults of main.mm:461-464, with keyword overrides."""
    c = np.zeros((), SIM_CONFIG)
    vals = dict(n=128, tick=0, mode=0, family=0, substeps=5, sensor_period=1, sensor_delay=0,
                command_delay=0, max_steps=200, seed=42, eval=0, speed=2.0, distance=4.0, wind=0.0,
                depth_noise=0.0, dropout=0.0, risk_coef=0.0, entropy_coef=0.005,
                learning_rate=0.0003, velocity_contract=1, geometry_memory=0)
    vals.update(overrides)
    for k, v in vals.items():
        c[k] = v
    return c


def load_raptor(path):
    """RAPTOR1 file (raptor.hpp:25-40) -> RAPTOR_WEIGHTS scalar array."""
    data = open(path, "rb").read()
    if data[:8] != b"RAPTOR1\x00":
        raise ValueError("not a RAPTOR1 file: " + str(path))
    version, count = np.frombuffer(data[8:16], np.uint32)
    if version != 1 or count != 2084:
        raise ValueError("RAPTOR1 version/count mismatch")
    return np.frombuffer(data[16:16 + 8336], RAPTOR_WEIGHTS)[0].copy()


def policy_shape(obs=181, hidden=64, critic_obs=32, critic_hidden=64):
    """Offsets of the flat actor/critic vectors (ppo.hpp:35-45)."""
    a_b1 = hidden * obs
    a_w2 = a_b1 + hidden
    a_b2 = a_w2 + 4 * hidden
    a_ls = a_b2 + 4
    c_b1 = critic_hidden * critic_obs
    c_w2 = c_b1 + critic_hidden
    c_b2 = c_w2 + critic_hidden
    return dict(obs=obs, hidden=hidden, actor_b1=a_b1, actor_w2=a_w2, actor_b2=a_b2,
                actor_log_std=a_ls, actor_count=a_ls + 4, critic_obs=critic_obs,
                critic_hidden=critic_hidden, critic_b1=c_b1, critic_w2=c_w2, critic_b2=c_b2,
                critic_count=c_b2 + 1)


# Buffer ids of mdn_sim_download/mdn_sim_upload (include/mdnav.h MDN_BUF_*).
BUFFERS = {
    "states": (0, PHYSICS_STATE), "runs": (1, SIM_RUN), "worlds": (2, WORLD),
    "sensors": (3, np.float32), "poses": (4, np.float32), "commands": (5, np.float32),
    "actor": (6, np.float32), "critic": (7, np.float32), "obs": (8, np.float32),
    "critic_obs": (9, np.float32), "actions": (10, np.float32), "logp": (11, np.float32),
    "values": (12, np.float32), "rewards": (13, np.float32), "next_values": (14, np.float32),
    "terminated": (15, np.uint8), "truncated": (16, np.uint8), "advantages": (17, np.float32),
    "returns": (18, np.float32), "actor_m": (19, np.float32), "actor_v": (20, np.float32),
    "critic_m": (21, np.float32), "critic_v": (22, np.float32), "metric_rows": (23, np.float32),
    "next_critic_obs": (24, np.float32), "environment_physics": (25, PHYSICS_PARAMS),
    "task_states": (26, TASK_STATE), "bank_active_ids": (27, np.uint32), "bank_transition_ids": (28, np.uint32),
    "bank_schedule": (29, np.uint32), "grad_norm_rows": (30, np.float32),
}
BANK_REHEARSAL = 0xFFFFFFFF
# moving-threat mix families (include/mdnav_types.h): per env lane n % 4,
# 0-1 FAMILY_MOVERS, 2 FAMILY_MOVERS_LONG, 3 FAMILY_COURSE
FAMILY_C3_MIX = 32
FAMILY_MOVERS = 33
FAMILY_MOVERS_LONG = 34
FAMILY_COURSE = 35
