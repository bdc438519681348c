"""The reference's trained assets on the GPU path: resume of the PPOFIX1
checkpoint guided-table-memory.bin.best (main.mm:1218-1284) and the
eval-policy run of the policy exported from it, assets/navigation.bin
(main.mm:1103-1108, 605-614)."""
import os
import sys

import numpy as np
import pytest

from gpu_compare import ENV_BUFFERS, ROW_BUFFERS, compare
from mdnav import PPOTrainer, Sim, abi, formats, sim_evaluate
from oracle_lib import GOLDEN, OracleTrainer, raptor_fixture

pytestmark = pytest.mark.gpu

NAVPOL = os.path.join(GOLDEN, "navigation.bin")
CKPT = os.path.join(GOLDEN, "guided-table-memory.bin.best")
PPO_BUFFERS = ["actor", "critic", "actor_m", "actor_v", "critic_m", "critic_v"]


def say(*args):
    print(*args, flush=True)
    sys.stdout.flush()


def test_checkpoint_resume_bit_exact(tmp_path):
    """Load the trained guided-memory checkpoint (128 envs mid-training: trainer
    state, Adam moments, every env's state, world and sensor/pose/command
    rings) into the GPU trainer and into the oracle, run the next rollout and
    update on both, save, reload: every buffer bit-identical throughout."""
    say("case: resume guided-table-memory.bin.best, one rollout + update, save, reload")
    hd, _ = formats.read_checkpoint(CKPT)
    cfg = np.array(hd["config"], abi.SIM_CONFIG)
    weights = raptor_fixture()[0]
    sim = Sim(cfg, 32, raptor=weights, actor_obs=184)
    ppo = PPOTrainer(sim, 2, 256)
    assert ppo.load_checkpoint(CKPT, 5, 32, 128, 42) == 1090
    assert ppo.optimizer_step == 34880
    ora = OracleTrainer(cfg, 32, weights, epochs=2, minibatch=256)
    ora.set_actor_obs(184)
    ora.load_checkpoint(CKPT)
    bad = compare(sim, ora, ENV_BUFFERS + PPO_BUFFERS, tol=0.0)
    assert not bad, ("loaded", bad)
    sim.collect()
    ppo.rollout_update(1090)
    sim.sync()
    ora.iteration(1090)
    bad = compare(sim, ora, ENV_BUFFERS + ROW_BUFFERS + PPO_BUFFERS + ["advantages", "returns", "metric_rows"], tol=0.0)
    assert not bad, ("resumed", bad)
    assert ppo.optimizer_step == ora.optimizer_step
    out = tmp_path / "resumed.bin"
    ppo.save_checkpoint(out, 5, 42, 1091)
    h2, a2 = formats.read_checkpoint(out)
    assert int(h2["version"]) == 6 and int(h2["completed_rollouts"]) == 1091
    assert int(h2["optimizer_step"]) == ppo.optimizer_step and np.array_equal(a2, sim.get("actor"))
    assert os.path.getsize(out) == os.path.getsize(CKPT)
    sim2 = Sim(cfg, 32, raptor=weights, actor_obs=184)
    ppo2 = PPOTrainer(sim2, 2, 256)
    assert ppo2.load_checkpoint(out, 5, 32, 128, 42) == 1091
    for name in ENV_BUFFERS + PPO_BUFFERS:
        assert sim2.get(name).tobytes() == sim.get(name).tobytes(), name


def test_eval_policy_known_answer():
    """eval-policy assets/navigation.bin 8 800001: 128 one-episode evaluations
    of the deployed mode-17 policy with the geometry memory, 1.5 m/s, 4 m
    goals.  The GPU run is bit-identical to the oracle's, and it reproduces
    the reference's published result of the same command exactly: 114 of 128
    successes (89.0625 %), 14 collisions (10.9375 %), no timeout, 2.83684 s
    mean goal time (docs/BENCHMARKS.md:94, printed to 6 digits).  The
    reference computed it on Metal with its own transcendental functions, so
    this agreement is not guaranteed by construction; a change that alters a
    last bit anywhere in the closed loop can move an episode, and this test
    is the place that shows it."""
    say("case: eval-policy navigation.bin family 8 seed 800001 (128 envs x 200 ticks, geometry memory)")
    meta, w, _ = formats.read_navigation_policy(NAVPOL)
    weights = raptor_fixture()[0]
    score, report = sim_evaluate(8, int(meta["policy_mode"]), w, speed=float(meta["max_speed_mps"]), distance=4.0,
                                 seed=800001, memory=1, raptor=weights)
    say("  GPU:", score, report)
    cfg = abi.default_config(n=128, family=8, mode=17, eval=1, seed=800001, distance=4.0, speed=1.5,
                             geometry_memory=1, max_steps=200)
    ora = OracleTrainer(cfg, 32, weights)
    ora.set_actor_obs(184)
    ora.set("actor", w)
    ora.collect(200)
    r = ora.get("runs")
    n = len(r)
    oscore = dict(success=r["successes"].sum() / n, collision=r["collisions"].sum() / n,
                  timeout=r["timeouts"].sum() / n,
                  goal_time=r["success_time"].astype(np.float64).sum() / max(r["successes"].sum(), 1))
    say("  oracle:", oscore)
    for k in ("success", "collision", "timeout"):
        assert score[k] == oscore[k], (k, score[k], oscore[k])
    assert abs(score["goal_time"] - oscore["goal_time"]) < 1e-9
    assert (score["success"], score["collision"], score["timeout"]) == (114 / 128, 14 / 128, 0.0), score
    assert abs(score["goal_time"] - 2.83684) < 5e-6, score


def published_evaluations():
    import csv
    return list(csv.DictReader(open(os.path.join(GOLDEN, "evaluation.csv"))))


@pytest.mark.parametrize("row", published_evaluations(), ids=lambda r: r["case_id"][:48])
def test_published_evaluations(row):
    """The reference's 28 published evaluations of this policy
    (assets/evaluation.csv: modes 2/13/17, families 3/5/7/8, two seeds,
    sensor and command delays, wind, depth noise, pixel dropout, combined),
    each 128 one-episode runs.  The outcome counts (success, collision,
    timeout) must be the reference's exactly; the continuous statistics agree
    to the printed digits in most cases and within an episode tick where a
    last-bit difference of Metal's transcendentals shifted one arrival."""
    w = formats.read_navigation_policy(NAVPOL)[1]
    score, rep = sim_evaluate(int(row["family"]), int(row["mode"]), w, speed=float(row["speed_mps"]),
                              distance=float(row["distance_m"]), seed=int(row["seed"]),
                              sensor_delay=int(row["sensor_delay_frames"]), wind=float(row["wind_param"]),
                              noise=float(row["depth_noise_m"]), dropout=float(row["dropout_probability"]),
                              command_delay=int(row["command_delay_steps"]), memory=1, raptor=raptor_fixture()[0])
    want = {k: float(row[k]) for k in ("success", "collision", "timeout", "progress", "mean_goal_time_s",
                                       "mean_speed_mps", "peak_speed_mps", "min_clearance_m")}
    say("case %s: success %.6g/%.6g collision %.6g/%.6g goal %.6g/%.6g" % (
        row["case_id"][:40], rep["success"], want["success"], rep["collision"], want["collision"],
        rep["mean_goal_time"], want["mean_goal_time_s"]))
    for k in ("success", "collision", "timeout"):  # 128 episodes: printed to 6 digits
        assert round(rep[k] * 128) == round(want[k] * 128), (k, rep[k], want[k])
    assert abs(rep["mean_goal_time"] - want["mean_goal_time_s"]) <= 0.02, rep
    assert abs(rep["progress"] - want["progress"]) <= 1e-3, rep
    assert abs(rep["mean_speed"] - want["mean_speed_mps"]) <= 5e-3, rep
    assert abs(rep["peak_speed"] - want["peak_speed_mps"]) <= 1e-3, rep
    assert abs(rep["min_clearance"] - want["min_clearance_m"]) <= 1e-5, rep


def continuation_evaluations():
    import csv
    rows = csv.DictReader(open(os.path.join(GOLDEN, "continuation-evaluation.csv")))
    return [r for r in rows if r["group"] != "controlled_threat"]


@pytest.mark.parametrize("row", continuation_evaluations(),
                         ids=lambda r: (r["candidate"] + ":" + r["case_id"])[:56])
def test_continuation_evaluations(row):
    """84 more published evaluations (assets/continuation-evaluation.csv) of
    three further trained policies (broad stress, door stress, rehearsal
    curricula; actors taken from the reference's checkpoints, identified by
    SHA-256, by tests/golden/make_actor_fixtures.py), same bar as above."""
    z = np.load(os.path.join(GOLDEN, "actors", row["candidate"] + ".npz"))
    assert bytes(z["sha256"]).hex() == row["checkpoint_sha256"]
    cfg = z["config"].view(abi.SIM_CONFIG)[0]
    rep = sim_evaluate(int(row["family"]), int(row["mode"]), z["actor"], speed=float(row["speed_mps"]),
                       distance=float(row["distance_m"]), seed=int(row["seed"]),
                       sensor_delay=int(row["sensor_delay_frames"]), wind=float(row["wind_param"]),
                       noise=float(row["depth_noise_m"]), dropout=float(row["dropout_probability"]),
                       command_delay=int(row["command_delay_steps"]), velocity_contract=int(cfg["velocity_contract"]),
                       memory=int(cfg["geometry_memory"]), raptor=raptor_fixture()[0])[1]
    want = {k: float(row[k]) for k in ("success", "collision", "timeout", "progress", "mean_goal_time_s",
                                       "mean_speed_mps", "peak_speed_mps", "min_clearance_m")}
    for k in ("success", "collision", "timeout"):
        assert round(rep[k] * 128) == round(want[k] * 128), (k, rep[k], want[k])
    assert abs(rep["mean_goal_time"] - want["mean_goal_time_s"]) <= 0.02, rep
    assert abs(rep["progress"] - want["progress"]) <= 1e-3, rep
    assert abs(rep["mean_speed"] - want["mean_speed_mps"]) <= 5e-3, rep
    assert abs(rep["peak_speed"] - want["peak_speed_mps"]) <= 1e-3, rep
    assert abs(rep["min_clearance"] - want["min_clearance_m"]) <= 1e-5, rep


def threat_evaluations():
    import csv
    rows = csv.DictReader(open(os.path.join(GOLDEN, "continuation-evaluation.csv")))
    return [r for r in rows if r["group"] == "controlled_threat"]


@pytest.mark.parametrize("row", threat_evaluations(), ids=lambda r: r["case_id"][:48])
def test_threat_evaluations(row):
    """The 24 published controlled-threat evaluations of the table-memory
    policy (continuation-evaluation.csv; threat-eval, main.mm:2711-2728 with
    threat_evaluation.hpp): one 0.35 m sphere per env on an approach or
    crossing course at 0.5 or 2 m/s, nominal time to collision 0.5 or 1 s,
    modes 2/13/17.  Outcome counts exact; statistics as above."""
    from mdnav import evaluate_threat
    w = formats.read_navigation_policy(NAVPOL)[1]
    assert row["checkpoint_sha256"].startswith("fdd62374")  # guided-table-memory, navigation.bin's source
    kind = {"approach": 0, "crossing": 1}[row["threat_kind"]]
    rep = evaluate_threat(w, int(row["mode"]), kind, float(row["threat_speed_mps"]), float(row["nominal_ttc_s"]),
                          seed=int(row["seed"]), sensor_delay=int(row["sensor_delay_frames"]),
                          command_delay=int(row["command_delay_steps"]), raptor=raptor_fixture()[0])
    want = {k: float(row[k]) for k in ("success", "collision", "timeout", "progress", "mean_goal_time_s",
                                       "mean_speed_mps", "peak_speed_mps", "min_clearance_m")}
    say("case %s: success %.6g/%.6g collision %.6g/%.6g progress %.6g/%.6g" % (
        row["case_id"][:40], rep["success"], want["success"], rep["collision"], want["collision"], rep["progress"],
        want["progress"]))
    for k in ("success", "collision", "timeout"):
        assert round(rep[k] * 128) == round(want[k] * 128), (k, rep[k], want[k])
    assert abs(rep["mean_goal_time"] - want["mean_goal_time_s"]) <= 0.02, rep
    assert abs(rep["progress"] - want["progress"]) <= 1e-3, rep
    assert abs(rep["mean_speed"] - want["mean_speed_mps"]) <= 5e-3, rep
    assert abs(rep["peak_speed"] - want["peak_speed_mps"]) <= 1e-3, rep
    assert abs(rep["min_clearance"] - want["min_clearance_m"]) <= 1e-5, rep


# Further published evaluations (evidence/inputs, copied to tests/golden/evidence):
# the speed sweep of the clean-stress policy and the inference ablations and
# controlled-threat matrix of the threat-joint policy (docs/BENCHMARKS.md:157-183
# and evidence.py:1644-1654 name the checkpoints).
EVIDENCE_POLICY = {"static-speed.csv": "clean_stress", "threat-joint-ablations.csv": "threat_joint",
                   "threat-joint-controlled.csv": "threat_joint"}


def evidence_rows():
    import csv
    out = []
    for name in sorted(EVIDENCE_POLICY):
        for r in csv.DictReader(open(os.path.join(GOLDEN, "evidence", name))):
            out.append(dict(r, _file=name))
    return out


@pytest.mark.parametrize("row", evidence_rows(), ids=lambda r: (r["_file"][:12] + ":" + r["case_id"])[:56])
def test_evidence_evaluations(row):
    """79 more published evaluations with the same bar: outcome counts exact,
    statistics to the printed digits (within a tick's shift of an arrival)."""
    from mdnav import evaluate_threat
    z = np.load(os.path.join(GOLDEN, "actors", EVIDENCE_POLICY[row["_file"]] + ".npz"))
    cfg = z["config"].view(abi.SIM_CONFIG)[0]
    if row["group"] == "controlled_threat":
        kind = {"approach": 0, "crossing": 1}[row["threat_kind"]]
        rep = evaluate_threat(z["actor"], int(row["mode"]), kind, float(row["threat_speed_mps"]),
                              float(row["nominal_ttc_s"]), seed=int(row["seed"]),
                              sensor_delay=int(row["sensor_delay_frames"]),
                              command_delay=int(row["command_delay_steps"]), raptor=raptor_fixture()[0])
    else:
        rep = sim_evaluate(int(row["family"]), int(row["mode"]), z["actor"], speed=float(row["speed_mps"]),
                           distance=float(row["distance_m"]), seed=int(row["seed"]),
                           sensor_delay=int(row["sensor_delay_frames"]), wind=float(row["wind_param"]),
                           noise=float(row["depth_noise_m"]), dropout=float(row["dropout_probability"]),
                           command_delay=int(row["command_delay_steps"]),
                           velocity_contract=int(cfg["velocity_contract"]), memory=int(cfg["geometry_memory"]),
                           raptor=raptor_fixture()[0])[1]
    want = {k: float(row[k]) for k in ("success", "collision", "timeout", "progress", "mean_goal_time_s",
                                       "mean_speed_mps", "peak_speed_mps", "min_clearance_m")}
    say("case %s: success %.6g/%.6g collision %.6g/%.6g goal %.6g/%.6g" % (
        row["case_id"][:40], rep["success"], want["success"], rep["collision"], want["collision"],
        rep["mean_goal_time"], want["mean_goal_time_s"]))
    for k in ("success", "collision", "timeout"):
        assert round(rep[k] * 128) == round(want[k] * 128), (k, rep[k], want[k])
    assert abs(rep["mean_goal_time"] - want["mean_goal_time_s"]) <= 0.02, rep
    assert abs(rep["progress"] - want["progress"]) <= 1e-3, rep
    assert abs(rep["mean_speed"] - want["mean_speed_mps"]) <= 5e-3, rep
    assert abs(rep["peak_speed"] - want["peak_speed_mps"]) <= 1e-3, rep
    assert abs(rep["min_clearance"] - want["min_clearance_m"]) <= 1e-5, rep


def test_checkpoint_versions_9_10_camera_and_shaping(tmp_path):
    """PPOFIX1 versions 9-10 (main.mm:1258-1277, 1292-1317).  With the native
    camera the trainer writes version 10: the version-8 blocks, the disabled
    shaping block (the reference's value-initialised control and grid and a
    zeroed field hash, 124 bytes, main.mm:534-536) and the 24-byte camera
    contract.  A native simulator resumes it bit for bit and continues
    identically to the simulator that wrote it; a legacy simulator refuses
    it (camera contract); a native simulator refuses an older file (legacy
    camera); a file whose shaping block is not the disabled one is refused;
    a version-9 file with the disabled block resumes in a legacy simulator."""
    from mdnav.native import MdnError
    say("case: PPOFIX1 v10 native camera save/resume, v9 shaping block, refusals")
    cfg = abi.default_config(n=64, family=1, speed=1.0, distance=3.0, max_steps=30)
    weights = raptor_fixture()[0]

    def trainer(native):
        s = Sim(cfg, 16, raptor=weights)
        if native:
            s.set_camera(abi.CAMERA_NATIVE)
        return s, PPOTrainer(s, 1, 256)

    sim, ppo = trainer(True)
    sim.collect()
    ppo.rollout_update(0)
    sim.sync()
    out = tmp_path / "native.bin"
    ppo.save_checkpoint(out, 1, 42, 1)
    h, _ = formats.read_checkpoint(out)
    assert int(h["version"]) == 10
    raw = open(out, "rb").read()
    cam = np.frombuffer(raw[-24:], abi.CAMERA_PROFILE)[0]
    assert int(cam["id"]) == 2 and float(cam["tan_v"]) == np.float32(0.8)
    assert float(cam["mount_x_m"]) == np.float32(0.08) and float(cam["max_range_m"]) == 12.0
    assert raw[-148:-24] == bytes(124)
    sim2, ppo2 = trainer(True)
    assert ppo2.load_checkpoint(out, 1, 16, 64, 42) == 1
    for name in ENV_BUFFERS + PPO_BUFFERS:
        assert sim2.get(name).tobytes() == sim.get(name).tobytes(), name
    for s_, p_ in ((sim, ppo), (sim2, ppo2)):
        s_.collect()
        p_.rollout_update(1)
        s_.sync()
    for name in ENV_BUFFERS + ROW_BUFFERS + PPO_BUFFERS:
        assert sim2.get(name).tobytes() == sim.get(name).tobytes(), ("continued", name)
    sim3, ppo3 = trainer(False)
    with pytest.raises(MdnError, match="camera contract"):
        ppo3.load_checkpoint(out, 1, 16, 64, 42)
    old = tmp_path / "legacy.bin"
    ppo3.save_checkpoint(old, 1, 42, 0)
    assert int(formats.read_checkpoint(old)[0]["version"]) == 6
    with pytest.raises(MdnError, match="calibrated sensors"):
        ppo2.load_checkpoint(old, 1, 16, 64, 42)
    shaped = bytearray(raw)
    shaped[-148] = 1  # TrainingPotentialControl.enabled
    (tmp_path / "shaped.bin").write_bytes(bytes(shaped))
    with pytest.raises(MdnError, match="shaping"):
        ppo2.load_checkpoint(tmp_path / "shaped.bin", 1, 16, 64, 42)
    v9 = bytearray(raw[:-24])
    hdr = np.frombuffer(bytes(v9[:abi.CHECKPOINT_HEADER.itemsize]), abi.CHECKPOINT_HEADER).copy()
    hdr["version"] = 9
    v9[:abi.CHECKPOINT_HEADER.itemsize] = hdr.tobytes()
    (tmp_path / "v9.bin").write_bytes(bytes(v9))
    assert ppo3.load_checkpoint(tmp_path / "v9.bin", 1, 16, 64, 42) == 1
