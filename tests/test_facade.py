"""The C++ façade (include/mdnav.hpp) compiles against the C ABI and links
libmdnav.so; error codes surface as std::runtime_error."""
import os
import subprocess

import pytest

from mdnav import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "cpp", "facade_example.cpp")
EXE = os.path.join(ROOT, "tests", "cpp", "facade_example")


def build_example():
    libdir = os.path.dirname(native.LIB_PATH)
    cmd = ["g++", "-std=c++17", "-O2", "-ffp-contract=off", "-I" + os.path.join(ROOT, "include"), SRC,
           "-L" + libdir, "-lmdnav", "-Wl,-rpath," + libdir, "-o", EXE]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return EXE


def test_facade_compiles_and_reports_usage():
    exe = build_example()
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 2 and "usage" in r.stderr


def test_facade_loads_deployed_policy():
    exe = build_example()
    r = subprocess.run([exe, "--policy", os.path.join(ROOT, "tests", "golden", "navigation.bin")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert "mode=17 observations=184 weights=12104 max_speed=1.50 source=1d991b0048dec80a" in r.stdout, r.stdout
    r = subprocess.run([exe, "--policy", os.path.join(ROOT, "tests", "golden", "raptor.bin")],
                       capture_output=True, text=True)
    assert r.returncode == 1 and "magic mismatch" in r.stderr, r.stderr


def grad_norm_summary(rows, limit=0.5):
    """main.mm:1443-1465 over [updates][2] pre-clip norms (double sums)."""
    import numpy as np
    rows = np.asarray(rows, np.float32).reshape(-1, 2)
    out = {}
    for k, name in enumerate(("actor", "critic")):
        col = rows[:, k]
        acc = 0.0  # a sequential double sum, as the reference takes it
        for x in col:
            acc += float(x)
        out[name + "_mean"] = np.float32(acc / len(col))
        out[name + "_max"] = np.float32(max(0.0, float(col.max())))
        out[name + "_clip_frac"] = np.float32(np.float32(int((col > np.float32(limit)).sum())) / np.float32(len(col)))
    return out


def report_line(label, runs, wall=0):
    """Sim::report's line (main.mm:599-602), formatted as std::ostream prints
    doubles (six significant digits)."""
    import numpy as np
    ep, succ = int(runs["episodes"].sum()), int(runs["successes"].sum())
    time_ = runs["success_time"].astype(np.float64).sum()
    path, total = runs["total_path"].astype(np.float64).sum(), runs["total_elapsed"].astype(np.float64).sum()
    progress = runs["final_progress"].astype(np.float64).sum()
    clearance = float(min(np.float32(12), runs["min_clearance"].min()))
    peak = float(max(np.float32(0), runs["peak_speed"].max()))
    g = lambda x: "%g" % x
    return ("%s episodes=%d success=%s collision=%s timeout=%s progress=%s mean_goal_time=%s mean_speed=%s "
            "peak_speed=%s min_clearance=%s wall_s=%s" % (
                label, ep, g(succ / ep if ep else 0), g(int(runs["collisions"].sum()) / ep if ep else 0),
                g(int(runs["timeouts"].sum()) / ep if ep else 0), g(progress / ep if ep else 0),
                g(time_ / succ if succ else 0), g(path / total if total else 0), g(peak), g(clearance), g(wall)))


@pytest.mark.gpu
def test_facade_trains_on_gpu():
    """cpu_reference_benchmark's use of the façade (main.mm:478-509):
    Trainer::validate_batched_forward before training (true at the reference's
    2e-5, false at 1e-9: the GPU forward is not the scalar one), run(2), then
    PPOTrainer::grad_norm_summary and Sim::report, both equal to the oracle's
    replay of the same two iterations (the GPU path is bit-exact, so the
    summary's floats and the report's text match exactly)."""
    import numpy as np
    from mdnav import abi
    from oracle_lib import OracleTrainer, raptor_fixture
    exe = build_example()
    print("case: facade example 256 envs x 2 rollouts", flush=True)
    r = subprocess.run([exe, os.path.join(ROOT, "tests", "golden", "raptor.bin"), "256", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "updates=128" in r.stdout, r.stdout  # 2 rollouts x 2 epochs x 32 minibatches
    assert "validate_batched_forward=1 strict=0" in r.stdout, r.stdout
    print("case: oracle replay of the facade run", flush=True)
    ora = OracleTrainer(abi.default_config(n=256, family=1, speed=1.0, distance=3.0), 32, raptor_fixture()[0],
                        epochs=2, minibatch=256)
    for it in range(2):
        ora.iteration(it)
    want = grad_norm_summary(ora.get("grad_norm_rows"))
    line = [l for l in r.stdout.splitlines() if l.startswith("grad_norm ")][0]
    got = dict(kv.split("=") for kv in line.split()[1:])
    for k, v in want.items():
        assert np.float32(got[k]) == v, (k, got[k], v)
    assert 0 < want["actor_mean"] and 0 <= want["actor_clip_frac"] <= 1
    rep = [l for l in r.stdout.splitlines() if l.startswith("facade-train ")]
    assert rep == [report_line("facade-train", ora.get("runs"))], (rep, report_line("facade-train", ora.get("runs")))


TRAIN_SRC = os.path.join(ROOT, "tests", "cpp", "training_example.cpp")
TRAIN_EXE = os.path.join(ROOT, "tests", "cpp", "training_example")
RAPTOR = os.path.join(ROOT, "tests", "golden", "raptor.bin")
GUIDED = os.path.join(ROOT, "tests", "golden", "guided-table-memory.bin.best")


def build_training_example():
    libdir = os.path.dirname(native.LIB_PATH)
    cmd = ["g++", "-std=c++17", "-O2", "-ffp-contract=off", "-I" + os.path.join(ROOT, "include"), TRAIN_SRC,
           "-L" + libdir, "-lmdnav", "-Wl,-rpath," + libdir, "-o", TRAIN_EXE]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return TRAIN_EXE


def test_training_example_compiles():
    exe = build_training_example()
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 2 and "usage" in r.stderr


def oracle_task_trainer(cfg_kw, horizon, stage, family, amplitude, epochs=2, minibatch=256):
    import numpy as np
    from mdnav import abi
    from mdnav.evaluate import task_runtime, task_settings
    from oracle_lib import OracleTrainer, raptor_fixture
    t = OracleTrainer(abi.default_config(**cfg_kw), horizon, raptor_fixture()[0], epochs=epochs,
                      minibatch=minibatch)
    t.set_actor_obs(184)
    t.set_runtime(task_runtime(amplitude))
    t.set_tasks(task_settings(stage, family))
    t.reset()
    return t


@pytest.mark.gpu
def test_navigation_training_facade(tmp_path):
    """navigation_training::train and evaluate through the C++ façade:
    one task-training rollout from the trained guided checkpoint (128 envs x
    32 ticks, stage 2 clutter tasks on family-1 worlds, plants at amplitude
    0.5) gives the oracle's actor and critic bit for bit; the baseline
    evaluation's per-env CSV (128 tasks, 400 ticks, mode 17) has the oracle's
    outcomes, times and paths; a second call resumes from the checkpoint."""
    import csv
    import numpy as np
    from mdnav import formats
    exe = build_training_example()
    stage, family, amp, seed = 2, 1, 0.5, 9
    ck = str(tmp_path / "task.bin")
    print("case: facade task training, 1 rollout + 2 evaluations", flush=True)
    r = subprocess.run([exe, "--task-train", RAPTOR, ck, GUIDED, "1", str(stage), str(family), str(amp), str(seed)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    assert "task_train rollout=1" in r.stdout, r.stdout
    for suffix in ("", ".best", ".history.csv", ".initial-dev.csv", ".dev.csv"):
        assert os.path.exists(ck + suffix), suffix
    hist = list(csv.DictReader(open(ck + ".history.csv")))
    assert [row["rollout"] for row in hist] == ["0", "1"] and hist[1]["total_transitions"] == str(128 * 32)
    h, actor, critic = formats.read_checkpoint_params(ck)
    assert int(h["version"]) == 8 and int(h["completed_rollouts"]) == 1 and int(h["optimizer_step"]) == 32

    print("case: oracle replay of the training rollout", flush=True)
    _, wa, wc = formats.read_checkpoint_params(GUIDED)
    wa = wa.copy()
    wa[-4:] = -1.0
    train_kw = dict(n=128, mode=22, family=family, seed=seed, speed=1.5, distance=8.0, max_steps=400,
                    geometry_memory=1, entropy_coef=0.001, learning_rate=0.0001)
    t = oracle_task_trainer(train_kw, 32, stage, family, amp)
    t.set("actor", wa)
    t.set("critic", wc)
    t.collect()
    t.gae()
    t.normalize()
    t.update(0)
    assert np.array_equal(t.get("actor"), actor) and np.array_equal(t.get("critic"), critic)

    print("case: oracle replay of the baseline evaluation", flush=True)
    e = oracle_task_trainer(dict(n=128, eval=1, mode=17, seed=800001, family=family, speed=1.5, distance=8.0,
                                 max_steps=400, geometry_memory=1), 32, stage, family, amp)
    e.set("actor", wa)
    tasks0 = e.get("task_states")
    e.collect(400)
    runs, mass = e.get("runs"), e.get("environment_physics")["mass"]
    rows = list(csv.DictReader(open(ck + ".initial-dev.csv")))
    assert len(rows) == 128
    for n, row in enumerate(rows):
        assert int(row["env"]) == n and int(row["seed"]) == 800001
        assert (int(row["success"]), int(row["collision"]), int(row["timeout"])) == (
            int(runs["successes"][n]), int(runs["collisions"][n]), int(runs["timeouts"][n])), n
        for col, want in (("time_s", runs["elapsed"][n]), ("path_m", runs["path"][n]),
                          ("goal_x", tasks0["goal_position"][n][0]), ("mass_kg", mass[n])):
            # the CSV prints six significant digits
            assert abs(float(row[col]) - float(want)) <= 1e-5 * max(1.0, abs(float(want))), (n, col)
    succ = runs["successes"].sum() / 128.0
    assert abs(float(hist[0]["success"]) - succ) < 1e-6

    print("case: facade task training resumes", flush=True)
    r = subprocess.run([exe, "--task-train", RAPTOR, ck, GUIDED, "1", str(stage), str(family), str(amp), str(seed)],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    h2, actor2, _ = formats.read_checkpoint_params(ck)
    assert int(h2["completed_rollouts"]) == 2 and int(h2["optimizer_step"]) == 64
    t.collect()
    t.gae()
    t.normalize()
    t.update(1)
    assert np.array_equal(t.get("actor"), actor2)
    assert [row["rollout"] for row in csv.DictReader(open(ck + ".history.csv"))] == ["0", "1", "2"]
