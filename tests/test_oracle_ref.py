"""The oracle's restatement against the reference's own code, compiled from
world.hpp / sensor_profile.hpp / physics.hpp / raptor.hpp / ppo.hpp into
oracle/_ref (oracle/Makefile target `ref`), plus the analytic cases of
world_tests (main.mm:107-125)."""
import numpy as np
import pytest

from oracle_lib import crazyflie, oracle, physics_fixture, ptr, raptor_fixture, ref, ref_available
from mdnav import abi

needs_ref = pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built (needs the reference tree)")

F = np.float32


def gen(lib, prefix, seed, family, distance):
    w = np.zeros((), abi.WORLD)
    getattr(lib, prefix + "_generate_world")(ptr(w), seed, family, F(distance))
    return w


def test_analytic_rays_and_collision():
    """world_tests closed-form cases (main.mm:108-123)."""
    lib = oracle()
    a = lambda *v: np.array(v, F)
    assert abs(lib.orc_ray_sphere(ptr(a(0, 0, 0)), ptr(a(1, 0, 0)), ptr(a(3, 0, 0)), 1) - 2) < 1e-6
    assert abs(lib.orc_ray_sphere(ptr(a(3, 0, 0)), ptr(a(1, 0, 0)), ptr(a(3, 0, 0)), 1) - 1) < 1e-6
    assert lib.orc_ray_sphere(ptr(a(0, 2, 0)), ptr(a(1, 0, 0)), ptr(a(3, 0, 0)), 1) == 1000
    assert abs(lib.orc_ray_sphere(ptr(a(0, 1, 0)), ptr(a(1, 0, 0)), ptr(a(3, 0, 0)), 1) - 3) < 1e-6
    assert abs(lib.orc_ray_box(ptr(a(0, 0, 0)), ptr(a(1, 0, 0)), ptr(a(3, 0, 0)), ptr(a(1, 1, 1))) - 2) < 1e-6
    assert lib.orc_ray_box(ptr(a(0, 2, 0)), ptr(a(1, 0, 0)), ptr(a(3, 0, 0)), ptr(a(1, 1, 1))) == 1000
    # inside a box the ray exits through the nearest face
    assert abs(lib.orc_ray_box(ptr(a(3, 0, 0)), ptr(a(1, 0, 0)), ptr(a(3, 0, 0)), ptr(a(1, 1, 1))) - 1) < 1e-6
    assert abs(lib.orc_ray_cylinder(ptr(a(0, 0, 0)), ptr(a(1, 0, 0)), ptr(a(3, 0, 0)), 1, 1) - 2) < 1e-6
    assert abs(lib.orc_ray_cylinder(ptr(a(3, 0, 3)), ptr(a(0, 0, -1)), ptr(a(3, 0, 0)), 1, 1) - 2) < 1e-6
    # moving sphere: centre 3 - t at t=1 -> hit at 1.5; collision independent of rays; 12 m clamp
    w = np.zeros((), abi.WORLD)
    w["count"] = 1
    w["obstacles"][0]["kind"] = 1
    w["obstacles"][0]["center"] = [3, 0, 1.5]
    w["obstacles"][0]["size"] = [0.5, 0, 0]
    w["obstacles"][0]["velocity"] = [-1, 0, 0]
    ray = a(0, 0, 1.5, 1, 0, 0)
    out = np.zeros(1, F)
    lib.orc_ray_world_batch(ptr(w), ptr(ray), ptr(a(1)), 1, ptr(out), 1)
    assert abs(out[0] - 1.5) < 1e-6
    lib.orc_clearance_batch(ptr(w), ptr(a(2, 0, 1.5)), ptr(a(1)), ptr(out), 1)
    assert out[0] < 0
    w["count"] = 0
    lib.orc_ray_world_batch(ptr(w), ptr(a(0, 0, 2.5, 1, 0, 0)), ptr(a(0)), 1, ptr(out), 1)
    assert out[0] == 12


def test_room_exit_distances():
    """Inside the room x[-2,14] y[-5,5] z[0,5] every axis ray exits at the wall."""
    lib = oracle()
    w = np.zeros((), abi.WORLD)
    out = np.zeros(1, F)
    for d, want in [((0, 1, 0), 5.0), ((0, -1, 0), 5.0), ((0, 0, 1), 3.5), ((0, 0, -1), 1.5), ((-1, 0, 0), 2.0)]:
        ray = np.array([0, 0, 1.5, *d], F)
        lib.orc_ray_world_batch(ptr(w), ptr(ray), ptr(np.zeros(1, F)), 1, ptr(out), 1)
        assert abs(out[0] - want) < 1e-6, (d, out[0])


@needs_ref
@pytest.mark.parametrize("family", [0, 1, 2, 3, 4, 5, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16])
def test_world_generation_bit_exact(family):
    for seed in (1, 197, 42 + 747796405, 2891336453, 123456789):
        a = gen(oracle(), "orc", seed, family, 4.0)
        b = gen(ref(), "ref", seed, family, 4.0)
        assert a.tobytes() == b.tobytes(), (family, seed)


@needs_ref
def test_camera_rays_bit_exact():
    a = np.zeros(960, F)
    b = np.zeros(960, F)
    oracle().orc_camera_rays(ptr(a))
    ref().ref_camera_rays(ptr(b))
    assert a.tobytes() == b.tobytes()


def _world_tests_setup(n=128):
    """main.mm:115-118: 128 worlds (seed i+197, family i%4, distance 8)."""
    worlds = np.zeros(n, abi.WORLD)
    for i in range(n):
        worlds[i] = gen(oracle(), "orc", i + 197, i % 4, 8.0)
    times = np.array([(i % 7) * 0.1 for i in range(n)], F)
    cam = np.zeros((320, 3), F)
    oracle().orc_camera_rays(ptr(cam))
    rays = np.zeros((n, 320, 6), F)
    for i in range(n):
        rays[i, :, 0:3] = [0, (i % 5 - 2) * 0.3, 1.5]
        rays[i, :, 3:6] = cam
    return worlds, times, rays


@needs_ref
def test_ray_cast_against_reference():
    worlds, times, rays = _world_tests_setup()
    n = len(worlds)
    a = np.zeros(n * 320, F)
    b = np.zeros(n * 320, F)
    oracle().orc_ray_world_batch(ptr(worlds), ptr(rays), ptr(times), 320, ptr(a), n * 320)
    ref().ref_ray_world_batch(ptr(worlds), ptr(rays), ptr(times), 320, ptr(b), n * 320)
    err = np.abs(a - b).max()
    assert err < 3e-5, err  # world_tests CPU/Metal gate
    assert (a < 12).mean() > 0.3  # most rays hit something
    pts = np.ascontiguousarray(rays[:, 0, 0:3])
    ca = np.zeros(n, F)
    cb = np.zeros(n, F)
    oracle().orc_clearance_batch(ptr(worlds), ptr(pts), ptr(times), ptr(ca), n)
    ref().ref_clearance_batch(ptr(worlds), ptr(pts), ptr(times), ptr(cb), n)
    assert np.abs(ca - cb).max() < 3e-5


@needs_ref
def test_physics_against_reference_bit_exact():
    params, recs, _, _ = physics_fixture()
    p = np.array(params, abi.PHYSICS_PARAMS)
    s = np.ascontiguousarray(recs["state"])
    act = np.ascontiguousarray(recs["action"])
    wind = np.ascontiguousarray(recs["wind"])
    a = np.zeros(len(recs), abi.PHYSICS_STATE)
    b = np.zeros(len(recs), abi.PHYSICS_STATE)
    oracle().orc_physics_step_batch(ptr(s), ptr(act), ptr(wind), ptr(p), ptr(a), len(recs))
    ref().ref_physics_step_batch(ptr(s), ptr(act), ptr(wind), ptr(p), ptr(b), len(recs))
    # no transcendental functions in the plant: identical operations, identical bits
    assert a.tobytes() == b.tobytes()
    q = np.zeros((), abi.PHYSICS_PARAMS)
    ref().ref_crazyflie_params(ptr(q))
    assert q.tobytes() == crazyflie().tobytes()


@needs_ref
def test_raptor_against_reference():
    weights, obs, _ = raptor_fixture()
    w = np.array(weights, abi.RAPTOR_WEIGHTS)
    rng = np.random.default_rng(5)
    seq = np.concatenate([obs, rng.normal(0, 0.6, (48, 22)).astype(F)])
    a = np.zeros((64, 4), F)
    b = np.zeros((64, 4), F)
    ha = np.zeros(16, F)
    hb = np.zeros(16, F)
    oracle().orc_raptor_sequence(ptr(w), ptr(seq), 64, ptr(a), ptr(ha))
    ref().ref_raptor_sequence(ptr(w), ptr(seq), 64, ptr(b), ptr(hb))
    assert np.abs(a - b).max() < 2e-6 and np.abs(ha - hb).max() < 2e-6


@needs_ref
def test_native_camera_against_reference():
    """The native profile (sensor_profile.hpp:18-25, 111-126): the oracle's
    pixel rays at tan_v = 0.8 equal the reference's nav_sensor_pixel_ray bit
    for bit, and both profiles' contracts (id, tangents, mount, ranges) equal
    the reference's nav_sensor::by_id."""
    a = np.zeros(960, F)
    b = np.zeros(960, F)
    oracle().orc_camera_rays_tan(F(0.8), ptr(a))
    ref().ref_camera_rays_native(ptr(b))
    assert a.tobytes() == b.tobytes()
    for pid in (abi.CAMERA_LEGACY, abi.CAMERA_NATIVE):
        want = np.zeros((), abi.CAMERA_PROFILE)
        ref().ref_camera_profile(pid, ptr(want))
        assert int(want["id"]) == pid
        if pid == abi.CAMERA_NATIVE:
            assert float(want["tan_v"]) == F(0.8) and float(want["mount_x_m"]) == F(0.08)
        else:
            assert float(want["tan_v"]) == F(0.75) and float(want["mount_x_m"]) == 0.0
        assert float(want["tan_h"]) == 1.0 and float(want["min_range_m"]) == F(0.03)
        assert float(want["max_range_m"]) == 12.0
