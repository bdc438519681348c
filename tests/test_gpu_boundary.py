"""The host surfaces of ppo.hpp and navigation_training.hpp through the C
ABI: fixed_ppo's operators batched on the GPU (mdn_op_actor_forward ...
mdn_op_ppo_self_tests) against the oracle (bit for bit: same canonical
arithmetic) and against the reference's own header functions built into
oracle/_ref (within fp32 tolerance: the reference uses libm's tanh/exp and
mul+add dot products); validate_rollout and the checkpoint parameter
reader."""
import os

import numpy as np
import pytest

from mdnav import MdnError, abi, formats, ops
from oracle_lib import GOLDEN, oracle, ptr, ref, ref_available

F = np.float32
needs_ref = pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built")


def say(msg):
    print(msg, flush=True)


def random_actor(rng, d, h=64):
    sh = abi.policy_shape(obs=d, hidden=h)
    w = rng.normal(0, 0.1, sh["actor_count"]).astype(F)
    w[sh["actor_log_std"]:] = rng.uniform(-1.5, 0.3, 4)
    return w, sh


@pytest.mark.gpu
@pytest.mark.parametrize("d", [181, 184])
def test_actor_critic_forward(d):
    say("case: fixed_ppo forward, %d inputs" % d)
    rng = np.random.default_rng(d)
    w, sh = random_actor(rng, d)
    obs = rng.uniform(-1, 1, (300, d)).astype(F)
    h, m = ops.actor_forward(w, obs)
    ho, mo = np.zeros((300, 64), F), np.zeros((300, 4), F)
    oracle().orc_actor_forward_batch(ptr(w), ptr(obs), d, 64, 300, ptr(ho), ptr(mo))
    assert np.array_equal(h, ho) and np.array_equal(m, mo)
    cw = rng.normal(0, 0.2, sh["critic_count"]).astype(F)
    cobs = rng.uniform(-1, 1, (300, 32)).astype(F)
    ch, v = ops.critic_forward(cw, cobs)
    cho, vo = np.zeros((300, 64), F), np.zeros(300, F)
    oracle().orc_critic_forward_batch(ptr(cw), ptr(cobs), 300, ptr(cho), ptr(vo))
    assert np.array_equal(ch, cho) and np.array_equal(v, vo)
    if not ref_available(d):
        pytest.skip("oracle/_ref not built")
    lib = ref(d)
    worst_m = worst_v = 0.0
    for k in range(0, 300, 7):
        rh, rm = np.zeros(64, F), np.zeros(4, F)
        lib.ref_actor_forward(ptr(w), ptr(obs[k]), ptr(rh), ptr(rm))
        worst_m = max(worst_m, float(np.abs(rm - m[k]).max()))
        worst_v = max(worst_v, abs(lib.ref_critic_forward(ptr(cw), ptr(cobs[k]), ptr(rh)) - float(v[k])))
    say("  max |mean - ref| %.2e, |value - ref| %.2e" % (worst_m, worst_v))
    assert worst_m < 2e-5 and worst_v < 2e-5


@pytest.mark.gpu
def test_wide_forward_matches_oracle():
    """FIXED_PPO_HIDDEN_DIM raised (the capacity actors): 184 -> 512 -> 4."""
    rng = np.random.default_rng(3)
    w, _ = random_actor(rng, 184, 512)
    obs = rng.uniform(-1, 1, (64, 184)).astype(F)
    h, m = ops.actor_forward(w, obs, hidden_dim=512)
    ho, mo = np.zeros((64, 512), F), np.zeros((64, 4), F)
    oracle().orc_actor_forward_batch(ptr(w), ptr(obs), 184, 512, 64, ptr(ho), ptr(mo))
    assert np.array_equal(h, ho) and np.array_equal(m, mo)


def loss_cases(rng, n):
    act = rng.normal(0, 0.6, (n, 4)).astype(F)
    mean = (act + rng.normal(0, 0.3, (n, 4))).astype(F)
    ls = rng.uniform(-1.5, 0.4, 4).astype(F)
    lp = ops.gaussian_log_prob(act, mean, ls)
    # old log-probabilities spanning every surrogate branch, both advantage
    # signs and the +-20 log-ratio clamp
    shift = (rng.choice([-0.5, -0.1, 0.0, 0.1, 0.5, 25.0, -25.0], n) + rng.normal(0, 0.05, n)).astype(F)
    old = (lp - shift).astype(F)
    adv = rng.normal(0, 1.5, n).astype(F)
    val = rng.normal(0, 1, n).astype(F)
    ret = rng.normal(0, 1, n).astype(F)
    return act, mean, ls, old, val, adv, ret


@pytest.mark.gpu
def test_log_prob_and_sample_loss_grad():
    say("case: fixed_ppo gaussian_log_prob and sample_loss_and_grad, 2,000 rows")
    rng = np.random.default_rng(17)
    n = 2000
    act, mean, ls, old, val, adv, ret = loss_cases(rng, n)
    dm, dl, dv, loss = ops.sample_loss_and_grad(act, mean, ls, old, val, adv, ret, batch_size=256.0,
                                                clip=0.2, value_coef=0.5, entropy_coef=0.005)
    # both surrogate branches (active: non-zero policy derivative) and the clamp occur
    active = np.abs(dm).max(axis=1) > 0
    assert 100 < active.sum() < n - 100 and np.any(np.abs(np.log(loss[:, 3])) > 19)
    for k in range(n):
        odm, odl, odv, ol = np.zeros(4, F), np.zeros(4, F), np.zeros(1, F), np.zeros(4, F)
        oracle().orc_sample_loss_and_grad(ptr(act[k]), ptr(mean[k]), ptr(ls), old[k], val[k], adv[k], ret[k], 256.0,
                                          0.2, 0.5, 0.005, ptr(odm), ptr(odl), ptr(odv), ptr(ol))
        assert np.array_equal(dm[k], odm) and np.array_equal(dl[k], odl) and dv[k] == odv[0], k
        assert np.array_equal(loss[k], ol), k
    # per-row log_std (stride 4) gives the same as the shared vector
    lsr = np.tile(ls, (n, 1))
    assert np.array_equal(ops.gaussian_log_prob(act, mean, lsr), ops.gaussian_log_prob(act, mean, ls))
    if not ref_available():
        pytest.skip("oracle/_ref not built")
    lib = ref()
    lp = ops.gaussian_log_prob(act, mean, ls)
    worst = 0.0
    for k in range(0, n, 3):
        worst = max(worst, abs(lib.ref_gaussian_log_prob(ptr(act[k]), ptr(mean[k]), ptr(ls)) - float(lp[k])))
        rdm, rdl, rdv, rl = np.zeros(4, F), np.zeros(4, F), np.zeros(1, F), np.zeros(4, F)
        lib.ref_sample_loss_and_grad(ptr(act[k]), ptr(mean[k]), ptr(ls), old[k], val[k], val[k], adv[k], ret[k],
                                     256.0, 0.2, 0.5, 0.005, ptr(rdm), ptr(rdl), ptr(rdv), ptr(rl))
        for a, b in ((dm[k], rdm), (dl[k], rdl), (dv[k:k + 1], rdv), (loss[k], rl)):
            assert np.allclose(a, b, rtol=2e-5, atol=1e-7), (k, a, b)
    assert worst < 2e-5 * max(1.0, float(np.abs(lp).max()))


@pytest.mark.gpu
def test_adam_update_matches_reference():
    say("case: fixed_ppo adam_update, 100,003 parameters, 3 steps, weight decay")
    rng = np.random.default_rng(5)
    n = 100003
    p = rng.normal(0, 1, n).astype(F)
    m, v = np.zeros(n, F), np.zeros(n, F)
    po, mo, vo = p.copy(), m.copy(), v.copy()
    for step in (1, 2, 3):
        g = rng.normal(0, 0.5, n).astype(F)
        p, m, v = ops.adam_update(p, g, m, v, step, 3e-4, weight_decay=0.01)
        oracle().orc_adam_update(ptr(po), ptr(g), ptr(mo), ptr(vo), n, step, 3e-4, 0.9, 0.999, 1e-8, 0.01)
        assert np.array_equal(p, po) and np.array_equal(m, mo) and np.array_equal(v, vo)
    if ref_available():
        pr, mr, vr = p.copy(), m.copy(), v.copy()
        g = rng.normal(0, 0.5, n).astype(F)
        p, m, v = ops.adam_update(p, g, m, v, 4, 3e-4, weight_decay=0.01)
        ref().ref_adam_update(ptr(pr), ptr(g), ptr(mr), ptr(vr), n, 4, 3e-4, 0.9, 0.999, 1e-8, 0.01)
        # same operations in the same order, correctly rounded on both
        assert np.array_equal(p, pr) and np.array_equal(m, mr) and np.array_equal(v, vr)


@pytest.mark.gpu
def test_self_tests_pass_on_gpu():
    say("case: fixed_ppo run_cpu_self_tests through the GPU operators")
    assert ops.ppo_self_tests(2e-3)
    # a tolerance no finite difference meets fails, as the reference's would
    assert not ops.ppo_self_tests(0.0)


@pytest.mark.gpu
def test_validate_rollout(raptor_weights):
    """navigation_training::validate_rollout: passes after a task reset,
    names the env whose task or plant is rejected."""
    from mdnav import Sim
    say("case: validate_rollout, 64 envs, stage 0 tasks")
    cfg = abi.default_config(n=64, family=0, mode=17, eval=1, speed=1.5, distance=8.0, max_steps=400,
                             geometry_memory=1)
    sim = Sim(cfg, 4, raptor=raptor_weights, actor_obs=184)
    with pytest.raises(MdnError, match="task generation rejected env=0 status=0"):
        sim.validate_rollout()  # no tasks: every task state is empty
    t = np.zeros((), abi.TASK_CONTROL)
    t["enabled"] = 1
    c = np.zeros((), abi.TASK_CONFIG)
    from mdnav.native import lib
    assert lib().mdn_task_default_config(0, 0, 0.5, ptr(c)) == 0
    t["config"] = c
    r = np.zeros((), abi.RUNTIME_CONFIG)
    r["enabled"], r["domain_amplitude"] = 1, 0.5
    assert lib().mdn_domain_stress_range(ptr(r["domain_range"])) == 0
    sim.set_runtime(r)
    sim.set_tasks(t)
    sim.reset()
    sim.validate_rollout()
    sim.collect(3)
    sim.validate_rollout()
    ts = sim.get("task_states")
    ts["valid"][37] = 0
    sim.set("task_states", ts)
    with pytest.raises(MdnError, match="env=37 status=4"):
        sim.validate_rollout()
    ts["valid"][37] = 1
    sim.set("task_states", ts)
    ph = sim.get("environment_physics")
    ph["mass"][5] = np.nan
    sim.set("environment_physics", ph)
    with pytest.raises(MdnError, match="episode dynamics sample rejected env=5"):
        sim.validate_rollout()


def test_checkpoint_params_reader():
    """The actor and critic that follow a PPOFIX1 header (the trained
    guided checkpoint) read back as the file's bytes."""
    path = os.path.join(GOLDEN, "guided-table-memory.bin.best")
    h, a, c = formats.read_checkpoint_params(path)
    data = open(path, "rb").read()
    na, nc = int(h["actor_count"]), int(h["critic_count"])
    assert na == 12104 and nc == 2177
    assert a.tobytes() == data[136:136 + 4 * na] and c.tobytes() == data[136 + 4 * na:136 + 4 * (na + nc)]


# ---------------------------------------------------------------- PPOTrainer::grad_norm_summary
@pytest.mark.gpu
def test_grad_norm_rows_and_summary():
    """The pre-clip gradient norms of every update (grad_norm_rows,
    main.mm:1370-1373) equal the oracle's bit for bit, for the one-chunk path
    (256-row minibatches) and the chunked path (1,024 rows), and
    grad_norm_summary (main.mm:1443-1465) is their mean, maximum and
    clipped fraction."""
    from gpu_compare import config, make_pair
    from test_facade import grad_norm_summary
    for mb in (256, 1024):
        say("case: grad-norm rows, N=64 T=32 minibatch %d" % mb)
        cfg = config(n=64, family=1, speed=1.0, distance=3.0, max_steps=25)
        sim, ppo, ora = make_pair(cfg, 32, epochs=2, minibatch=mb)
        try:
            for it in range(2):
                sim.collect()
                ppo.rollout_update(it)
                ora.iteration(it)
                rows, want = sim.get("grad_norm_rows"), ora.get("grad_norm_rows")
                assert rows.shape == (ppo.updates_per_rollout * 2,) and np.array_equal(rows, want), it
            s = ppo.grad_norm_summary()
            w = grad_norm_summary(want)
            for k, v in w.items():
                assert np.float32(getattr(s, k)) == v, (k, getattr(s, k), v)
            assert s.actor_max >= s.actor_mean > 0 and s.critic_max >= s.critic_mean > 0
        finally:
            ppo.close()
            sim.close()


@pytest.mark.gpu
def test_grad_norm_summary_rejects_non_finite():
    """A NaN reward reaches the gradients through GAE and the loss: the
    summary raises the reference's "non-finite pre-clip gradient norm"
    (main.mm:1451).  The kernels only carry the NaN as a value."""
    from gpu_compare import config, make_pair
    from mdnav.native import MdnError
    say("case: grad-norm summary with a NaN gradient")
    cfg = config(n=64, family=1, speed=1.0, distance=3.0, max_steps=25)
    sim, ppo, _ = make_pair(cfg, 16, epochs=1, minibatch=256)
    try:
        s0 = ppo.grad_norm_summary()  # before any update: all zero
        assert (s0.actor_mean, s0.actor_max, s0.critic_clip_frac) == (0, 0, 0)
        sim.collect()
        r = sim.get("rewards")
        r[5] = np.nan
        sim.set("rewards", r)
        ppo.rollout_update(0)
        with pytest.raises(MdnError, match="non-finite pre-clip gradient norm"):
            ppo.grad_norm_summary()
    finally:
        ppo.close()
        sim.close()


@pytest.mark.gpu
def test_wide_policy_grad_norm_summary():
    """The wide policy's pre-clip norms (H = 256, bf16 products) against the
    oracle's fp32 update of the same rollout: means and maxima within 2 %,
    equal clipped fractions where no norm sits within 0.01 of the limit."""
    from gpu_compare import config, make_pair
    from mdnav import LargePPOTrainer
    from test_facade import grad_norm_summary
    say("case: wide-policy grad-norm summary, H=256 N=64 T=32")
    cfg = config(n=64, family=1, speed=1.0, distance=3.0, max_steps=25)
    sim, _, ora = make_pair(cfg, 32, epochs=1, minibatch=512)
    sim.collect()
    sim.sync()
    ora.collect()
    lp = LargePPOTrainer(sim, 256, epochs=1, minibatch=512)
    ora.set_hidden(256)
    try:
        lp.evaluate()
        sim.sync()
        for name in ("logp", "values", "next_values"):
            ora.set(name, sim.get(name))
        lp.rollout_update(0)
        ora.gae()
        ora.normalize()
        ora.update(0)
        s = lp.grad_norm_summary()
        want = grad_norm_summary(ora.get("grad_norm_rows"))
        say("  gpu %s / oracle %s" % ({k: getattr(s, k) for k in want}, want))
        for k in ("actor_mean", "actor_max", "critic_mean", "critic_max"):
            assert abs(getattr(s, k) - want[k]) <= 0.02 * want[k], (k, getattr(s, k), want[k])
        rows = ora.get("grad_norm_rows").reshape(-1, 2)
        for k, name in enumerate(("actor", "critic")):
            if np.all(np.abs(rows[:, k] - 0.5) > 0.01):
                assert np.float32(getattr(s, name + "_clip_frac")) == want[name + "_clip_frac"], name
    finally:
        lp.close()
        sim.close()


@pytest.mark.gpu
@pytest.mark.parametrize("d", [181, 184])
def test_trainer_validate_batched_forward(d):
    """Trainer::validate_batched_forward (cpu_reference.hpp:187-208) on the
    freshly initialised policy and after an update: true at the reference's
    2e-5, false at 1e-9 (the GPU's fma chains and tanh are not float64's)."""
    from gpu_compare import config
    from mdnav import Trainer
    from oracle_lib import raptor_fixture
    say("case: validate_batched_forward, %d inputs" % d)
    t = Trainer(config(n=32, family=1, speed=1.0, distance=3.0), 16, raptor=raptor_fixture()[0], actor_obs=d)
    try:
        assert t.validate_batched_forward()
        assert not t.validate_batched_forward(1e-9)
        t.run(1)
        assert t.validate_batched_forward()
    finally:
        t.ppo.close()
        t.sim.close()
