"""PPO operators of the oracle: closed forms, finite differences, and the
reference's own operators from ppo.hpp compiled into oracle/_ref."""
import numpy as np
import pytest

from oracle_lib import OracleTrainer, oracle, ptr, raptor_fixture, ref, ref_available
from mdnav import abi

needs_ref = pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built")
F = np.float32
LOG2PI = 1.8378770664093453


def loss_and_grad(action, mean, log_std, old_logp, value, adv, target, batch=1.0, clip=0.2, vc=0.7, ec=0.03):
    dm = np.zeros(4, F)
    dls = np.zeros(4, F)
    dv = np.zeros(1, F)
    losses = np.zeros(4, F)
    oracle().orc_sample_loss_and_grad(ptr(np.asarray(action, F)), ptr(np.asarray(mean, F)),
                                      ptr(np.asarray(log_std, F)), F(old_logp), F(value), F(adv), F(target),
                                      F(batch), F(clip), F(vc), F(ec), ptr(dm), ptr(dls), ptr(dv), ptr(losses))
    return losses, dm, dls, float(dv[0])


def objective(*args, **kw):
    losses = loss_and_grad(*args, **kw)[0]
    return float(losses[0]) + float(losses[1]) + float(losses[2])


@needs_ref
def test_reference_self_tests_pass():
    assert ref().ref_ppo_self_tests(F(2e-3)) == 1


def test_loss_grad_finite_differences_all_branches():
    """run_cpu_self_tests (ppo.hpp:204-267) restated on the oracle's own loss
    outputs: all four clip branches, mean and log-std derivatives, value."""
    action = np.array([0.4, 0, 0, 0], F)
    mean = np.array([0.1, 0, 0, 0], F)
    log_std = np.zeros(4, F)
    base = -0.5 * (0.3 ** 2 + LOG2PI) - 3 * 0.5 * LOG2PI
    h = 1e-3
    for old, adv in [(base - np.log(1.1), 1.0), (base - np.log(0.9), -1.0), (base - np.log(1.3), 1.0),
                     (base - np.log(0.7), -1.0)]:
        _, dm, dls, _ = loss_and_grad(action, mean, log_std, old, 0.25, adv, -0.3)
        for k in (0, 2):
            mp, mm = mean.copy(), mean.copy()
            mp[k] += h
            mm[k] -= h
            num = (objective(action, mp, log_std, old, 0.25, adv, -0.3)
                   - objective(action, mm, log_std, old, 0.25, adv, -0.3)) / (2 * h)
            assert abs(num - dm[k]) < 2e-3, (adv, k, num, dm[k])
            lp, lm = log_std.copy(), log_std.copy()
            lp[k] += h
            lm[k] -= h
            num = (objective(action, mean, lp, old, 0.25, adv, -0.3)
                   - objective(action, mean, lm, old, 0.25, adv, -0.3)) / (2 * h)
            assert abs(num - dls[k]) < 2e-3, (adv, k, num, dls[k])
    _, _, _, dv = loss_and_grad(action, mean, log_std, base, 0.25, 0.0, -0.3)
    assert abs(dv - 0.7 * (0.25 + 0.3)) < 1e-6
    # a clipped sample carries no policy gradient, only the entropy term
    _, dm, dls, _ = loss_and_grad(action, mean, log_std, base - np.log(1.3), 0.25, 1.0, -0.3)
    assert np.all(dm == 0) and np.allclose(dls, -0.03)


@needs_ref
def test_loss_grad_against_reference():
    rng = np.random.default_rng(1)
    lib = ref()
    for _ in range(200):
        a, m = rng.normal(0, 0.5, 4).astype(F), rng.normal(0, 0.5, 4).astype(F)
        ls = rng.uniform(-2, 0.5, 4).astype(F)
        old, v, adv, tgt = (F(x) for x in rng.normal(0, 1, 4))
        ours = loss_and_grad(a, m, ls, old, v, adv, tgt, 256.0, 0.2, 0.5, 0.005)
        dm, dls, dv, losses = np.zeros(4, F), np.zeros(4, F), np.zeros(1, F), np.zeros(4, F)
        lib.ref_sample_loss_and_grad(ptr(a), ptr(m), ptr(ls), old, v, v, adv, tgt, F(256), F(0.2), F(0.5),
                                     F(0.005), ptr(dm), ptr(dls), ptr(dv), ptr(losses))
        assert np.allclose(ours[0], losses, rtol=1e-5, atol=1e-7)
        assert np.allclose(ours[1], dm, rtol=1e-5, atol=1e-8)
        assert np.allclose(ours[2], dls, rtol=1e-5, atol=1e-8)
        assert abs(ours[3] - dv[0]) < 1e-7


def gae(fn, T, N, r, v, nv, te, tr):
    adv = np.zeros(T * N, F)
    ret = np.zeros(T * N, F)
    args = [np.ascontiguousarray(x, F) for x in (r, v, nv)] + [np.ascontiguousarray(x, np.uint8) for x in (te, tr)]
    fn(T, N, *[ptr(x) for x in args], F(0.99), F(0.95), ptr(adv), ptr(ret))
    return adv, ret


def test_gae_hand_case():
    """main.mm:286-297: T=3, N=2 with a terminal (t=1, env 0) and a
    truncation (t=1, env 1), solved on paper."""
    adv, ret = gae(oracle().orc_compute_gae, 3, 2, [1, 2, 3, 4, 5, 6], [.1, .2, .3, .4, .5, .6],
                   [.2, .3, .4, .5, .6, .7], [0, 0, 1, 0, 0, 0], [0, 0, 0, 1, 0, 0])
    gl = 0.99 * 0.95
    e0 = [1 + .99 * .2 - .1 + gl * 2.7, None, 3 - .3, None, 5 + .99 * .6 - .5, None]
    e1 = [None, 2 + .99 * .3 - .2 + gl * (4 + .99 * .5 - .4), None, 4 + .99 * .5 - .4, None, 6 + .99 * .7 - .6]
    want = np.array([x if x is not None else y for x, y in zip(e0, e1)])
    assert np.abs(adv - want).max() < 2e-5
    assert np.abs(ret - (want + np.array([.1, .2, .3, .4, .5, .6]))).max() < 2e-5
    if ref_available():
        radv, rret = gae(ref().ref_compute_gae, 3, 2, [1, 2, 3, 4, 5, 6], [.1, .2, .3, .4, .5, .6],
                         [.2, .3, .4, .5, .6, .7], [0, 0, 1, 0, 0, 0], [0, 0, 0, 1, 0, 0])
        assert adv.tobytes() == radv.tobytes() and ret.tobytes() == rret.tobytes()


def test_gae_constant_reward_closed_form():
    T, N = 64, 3
    adv, _ = gae(oracle().orc_compute_gae, T, N, np.ones(T * N), np.zeros(T * N), np.zeros(T * N),
                 np.zeros(T * N), np.zeros(T * N))
    gl = 0.99 * 0.95
    want = np.repeat([(1 - gl ** (T - t)) / (1 - gl) for t in range(T)], N)
    assert np.abs(adv - want).max() < 1e-4


def test_normalize_closed_form():
    x = np.array([-40, -2, -1, 0, 1, 2, 10, 40], F)
    y = x.copy()
    oracle().orc_normalize_advantages(ptr(y), len(y), F(1e-8))
    x64 = x.astype(np.float64)
    want = (x64 - x64.mean()) / np.sqrt(x64.var() + 1e-8)
    assert np.abs(y - want).max() < 2e-6
    big = np.random.default_rng(3).normal(3, 7, 100_003).astype(F)
    y = big.copy()
    oracle().orc_normalize_advantages(ptr(y), len(y), F(1e-8))
    assert abs(y.astype(np.float64).mean()) < 1e-6 and abs(y.astype(np.float64).std() - 1) < 1e-5
    if ref_available():
        z = big.copy()
        ref().ref_normalize_advantages(ptr(z), len(z), F(1e-8))
        assert np.abs(y - z).max() < 1e-6


def test_squared_norm_order_and_value():
    g = np.random.default_rng(4).normal(0, 1e-2, 12_105).astype(F)
    got = oracle().orc_squared_norm(ptr(g), len(g))
    assert abs(got - float(np.sum(g.astype(np.float64) ** 2))) / got < 1e-6


@needs_ref
def test_forward_against_reference():
    rng = np.random.default_rng(7)
    actor = np.zeros(12_104 + 0, F)
    critic = np.zeros(2177, F)
    oracle().orc_init_policy(ptr(actor), ptr(critic))
    actor[:] += rng.normal(0, 0.02, actor.size).astype(F)
    critic[:] += rng.normal(0, 0.05, critic.size).astype(F)
    assert ref().ref_actor_param_count() == 181 * 64 + 64 + 256 + 4 + 4
    actor = actor[:ref().ref_actor_param_count()].copy()
    obs = rng.uniform(-1, 1, (8, 181)).astype(F)
    cobs = rng.uniform(-1, 1, (8, 32)).astype(F)
    h = np.zeros((8, 64), F)
    m = np.zeros((8, 4), F)
    oracle().orc_actor_forward_batch(ptr(actor), ptr(obs), 181, 64, 8, ptr(h), ptr(m))
    ch = np.zeros((8, 64), F)
    cv = np.zeros(8, F)
    oracle().orc_critic_forward_batch(ptr(critic), ptr(cobs), 8, ptr(ch), ptr(cv))
    for n in range(8):
        rh, rm = np.zeros(64, F), np.zeros(4, F)
        ref().ref_actor_forward(ptr(actor), ptr(obs[n]), ptr(rh), ptr(rm))
        assert np.abs(rh - h[n]).max() < 2e-6 and np.abs(rm - m[n]).max() < 2e-6
        v = ref().ref_critic_forward(ptr(critic), ptr(cobs[n]), ptr(rh))
        assert abs(v - cv[n]) < 2e-6


@pytest.mark.skipif(not ref_available(184), reason="oracle/_ref not built")
def test_guided_forward_against_reference():
    """184-input actor (ppo.hpp:30-34): the first three means carry the last
    three inputs, the hint, on top of the MLP output (ppo.hpp:77).  Checked
    against the reference built with FIXED_PPO_ACTOR_OBS_DIM=184, and the hint
    term against the same MLP with the hint inputs zeroed."""
    rng = np.random.default_rng(9)
    count = ref(184).ref_actor_param_count()
    assert count == 184 * 64 + 64 + 256 + 4 + 4
    actor = rng.normal(0, 0.05, count).astype(F)
    obs = rng.uniform(-1, 1, (8, 184)).astype(F)
    h = np.zeros((8, 64), F)
    m = np.zeros((8, 4), F)
    oracle().orc_actor_forward_batch(ptr(actor), ptr(obs), 184, 64, 8, ptr(h), ptr(m))
    for n in range(8):
        rh, rm = np.zeros(64, F), np.zeros(4, F)
        ref(184).ref_actor_forward(ptr(actor), ptr(obs[n]), ptr(rh), ptr(rm))
        assert np.abs(rh - h[n]).max() < 2e-6 and np.abs(rm - m[n]).max() < 2e-6, (rm, m[n])
    # zeroing the hint inputs and their first-layer weights removes exactly the
    # MLP's dependence on them; the means then differ by the hint itself
    a0, o0 = actor.copy(), obs.copy()
    a0[:64 * 184].reshape(64, 184)[:, 181:] = 0
    o0[:, 181:] = 0
    m0 = np.zeros((8, 4), F)
    oracle().orc_actor_forward_batch(ptr(a0), ptr(obs), 184, 64, 8, ptr(h), ptr(m))
    oracle().orc_actor_forward_batch(ptr(a0), ptr(o0), 184, 64, 8, ptr(h), ptr(m0))
    assert np.array_equal(m[:, 3], m0[:, 3])
    assert np.abs((m[:, :3] - m0[:, :3]) - obs[:, 181:]).max() < 2e-6


@pytest.mark.skipif(not ref_available(184), reason="oracle/_ref not built")
def test_guided_minibatch_grads_against_reference():
    """The 184-input trainer's batched gradients (hint inputs in the rows from
    the rollout's guidance) against the reference's per-sample backprop."""
    weights = raptor_fixture()[0]
    cfg = abi.default_config(n=16, family=1, speed=1.0, distance=3.0)
    t = OracleTrainer(cfg, 16, weights, epochs=2, minibatch=256)
    t.set_actor_obs(184)
    t.collect()
    t.gae()
    t.normalize()
    ag, cg, row, dm, dls, dv = t.minibatch_grads(0, 256)
    assert ag.size == ref(184).ref_actor_param_count()
    obs = t.get("obs")[:256 * 184].copy()
    assert np.count_nonzero(obs.reshape(256, 184)[:, 181:]) > 0
    co = t.get("critic_obs")[:256 * 32].copy()
    ra, rc = np.zeros_like(ag), np.zeros_like(cg)
    ref(184).ref_actor_critic_grads(ptr(t.get("actor")), ptr(t.get("critic")), ptr(obs), ptr(co), ptr(dm),
                                    ptr(dls), ptr(dv), 256, ptr(ra), ptr(rc))
    assert np.abs(ag - ra).max() < 3e-5 * max(1.0, np.abs(ra).max()), np.abs(ag - ra).max()
    assert np.abs(cg - rc).max() < 3e-5 * max(1.0, np.abs(rc).max())
    assert np.abs(ag[64 * 184 - 3:64 * 184]).max() > 0  # hint columns of W1 get gradient


@pytest.fixture(scope="module")
def filled_trainer():
    weights = raptor_fixture()[0]
    cfg = abi.default_config(n=16, family=1, speed=1.0, distance=3.0)
    t = OracleTrainer(cfg, 16, weights, epochs=2, minibatch=256)
    t.collect()
    t.gae()
    t.normalize()
    return t


@needs_ref
def test_minibatch_grads_against_reference_backprop(filled_trainer):
    """The oracle's batched gradients against the reference's per-sample
    backprop + reduction (ppo.hpp:269-308), fed the same row derivatives."""
    t = filled_trainer
    ag, cg, row, dm, dls, dv = t.minibatch_grads(0, 256)
    ra = np.zeros_like(ag)
    rc = np.zeros_like(cg)
    actor, critic = t.get("actor"), t.get("critic")
    obs = t.get("obs")[:256 * 181].copy()
    co = t.get("critic_obs")[:256 * 32].copy()
    ref().ref_actor_critic_grads(ptr(actor), ptr(critic), ptr(obs), ptr(co), ptr(dm), ptr(dls), ptr(dv), 256,
                                 ptr(ra), ptr(rc))
    scale = max(np.abs(ra).max(), 1e-6)
    assert np.abs(ag - ra).max() < 3e-5 * max(1.0, scale), np.abs(ag - ra).max()
    assert np.abs(cg - rc).max() < 3e-5 * max(1.0, np.abs(rc).max())
    assert np.abs(ag).max() > 0 and np.abs(cg).max() > 0


def test_minibatch_grads_finite_differences(filled_trainer):
    """Gradient of the minibatch objective sum(policy+value+entropy) through
    the whole actor and critic MLPs, by central differences on the oracle's
    own loss (old log-probs, advantages and returns held fixed)."""
    t = filled_trainer
    sh = abi.policy_shape()
    actor0, critic0 = t.get("actor"), t.get("critic")
    ag, cg, row0 = t.minibatch_grads(0, 256)[:3]
    rng = np.random.default_rng(11)

    def J():
        r = t.minibatch_grads(0, 256)[2]
        return float(r[0]) + float(r[1]) + float(r[2])

    picks = [("actor", i) for i in rng.integers(0, sh["actor_b1"], 6)]
    picks += [("actor", sh["actor_b1"] + 3), ("actor", sh["actor_w2"] + 70), ("actor", sh["actor_b2"] + 1),
              ("actor", sh["actor_log_std"] + 2)]
    picks += [("critic", i) for i in rng.integers(0, sh["critic_b1"], 4)]
    picks += [("critic", sh["critic_b1"] + 5), ("critic", sh["critic_w2"] + 9), ("critic", sh["critic_b2"])]
    for net, i in picks:
        base = (actor0 if net == "actor" else critic0).copy()
        grad = (ag if net == "actor" else cg)[i]
        h = 2e-3
        base[i] += h
        t.set(net, base)
        jp = J()
        base[i] -= 2 * h
        t.set(net, base)
        jm = J()
        base[i] += h
        t.set(net, base)
        num = (jp - jm) / (2 * h)
        assert abs(num - grad) <= 2e-2 * abs(grad) + 2e-4, (net, i, num, grad)
    t.set("actor", actor0)
    t.set("critic", critic0)


@needs_ref
def test_adam_step_against_reference():
    """One rollout update of a single minibatch equals norm-clip then the
    reference's adam_update (ppo.hpp:310-324) on the clipped gradient."""
    weights = raptor_fixture()[0]
    cfg = abi.default_config(n=16, family=1, speed=1.0, distance=3.0)
    t = OracleTrainer(cfg, 16, weights, epochs=1, minibatch=256)
    t.collect()
    t.gae()
    t.normalize()
    ag, cg = t.minibatch_grads(0, 256)[:2]
    a0, c0 = t.get("actor"), t.get("critic")
    t.update(0)
    assert t.optimizer_step == 1
    for g, p0, name in [(ag, a0, "actor"), (cg, c0, "critic")]:
        norm = np.sqrt(np.float32(oracle().orc_squared_norm(ptr(g), len(g))) + F(1e-20))
        scale = min(F(1), F(0.5) / F(norm))
        gs = (g * F(scale)).astype(F)
        p = p0.copy()
        m = np.zeros_like(p)
        v = np.zeros_like(p)
        ref().ref_adam_update(ptr(p), ptr(gs), ptr(m), ptr(v), len(p), 1, F(3e-4), F(.9), F(.999), F(1e-8), F(0))
        if name == "actor":
            ls = slice(abi.policy_shape()["actor_log_std"], None)
            p[ls] = np.clip(p[ls], -2, 0.5)
        got = t.get(name)
        assert np.abs(got - p).max() < 1e-7, name
        assert np.abs(t.get(name + "_m") - m).max() < 1e-9


def test_adam_update_operator():
    """The oracle's fixed_ppo::adam_update: the closed-form first step
    (ppo.hpp:254-266: m = 0.1 g, v = 0.001 g^2, p -= lr sign(g) at step 1),
    the weight-decay term entering the gradient, and the reference's own
    adam_update over several steps."""
    p, g, m, v = (np.array([x], F) for x in (1.0, 0.25, 0.0, 0.0))
    oracle().orc_adam_update(ptr(p), ptr(g), ptr(m), ptr(v), 1, 1, 0.01, 0.9, 0.999, 1e-8, 0.0)
    # (1 - 0.999f) = 0.00100005 in float: the second moment is within 5e-5 relative
    assert m[0] == pytest.approx(0.025, rel=1e-6) and v[0] == pytest.approx(6.25e-5, rel=1e-4)
    assert p[0] == pytest.approx(0.99, abs=1e-6)
    # weight decay 0.5 on p = 2 with g = 0 acts as a gradient of 1
    p, g, m, v = (np.array([x], F) for x in (2.0, 0.0, 0.0, 0.0))
    oracle().orc_adam_update(ptr(p), ptr(g), ptr(m), ptr(v), 1, 1, 0.01, 0.9, 0.999, 1e-8, 0.5)
    assert m[0] == pytest.approx(0.1, rel=1e-6) and p[0] == pytest.approx(1.99, abs=1e-6)
    if not ref_available():
        pytest.skip("oracle/_ref not built")
    rng = np.random.default_rng(2)
    n = 4097
    p = rng.normal(0, 1, n).astype(F)
    m, v = np.zeros(n, F), np.zeros(n, F)
    pr, mr, vr = p.copy(), m.copy(), v.copy()
    for step in range(1, 6):
        g = rng.normal(0, 1, n).astype(F)
        oracle().orc_adam_update(ptr(p), ptr(g), ptr(m), ptr(v), n, step, 1e-3, 0.9, 0.999, 1e-8, 0.02)
        ref().ref_adam_update(ptr(pr), ptr(g), ptr(mr), ptr(vr), n, step, 1e-3, 0.9, 0.999, 1e-8, 0.02)
    assert np.array_equal(p, pr) and np.array_equal(m, mr) and np.array_equal(v, vr)


def mt19937(seed):
    """std::mt19937 (the standard fixes its output sequence)."""
    mt = [0] * 624
    mt[0] = seed & 0xffffffff
    for i in range(1, 624):
        mt[i] = (1812433253 * (mt[i - 1] ^ (mt[i - 1] >> 30)) + i) & 0xffffffff
    idx = 624
    while True:
        if idx >= 624:
            for i in range(624):
                y = (mt[i] & 0x80000000) | (mt[(i + 1) % 624] & 0x7fffffff)
                mt[i] = mt[(i + 397) % 624] ^ (y >> 1) ^ (0x9908b0df if y & 1 else 0)
            idx = 0
        y = mt[idx]
        idx += 1
        y ^= y >> 11
        y ^= (y << 7) & 0x9d2c5680
        y ^= (y << 15) & 0xefc60000
        y ^= y >> 18
        yield y


def libcxx_shuffle(v, gen):
    """libc++'s std::shuffle with uniform_int_distribution<ptrdiff_t> over a
    32-bit engine: position k swaps with k + i, i drawn in [0, n-1-k] as the
    low ceil(log2(range)) bits of one engine output, redrawn while >= range."""
    n = len(v)
    for k in range(n - 1):
        rng = n - k
        w = (rng - 1).bit_length()
        while True:
            u = next(gen) & ((1 << w) - 1)
            if u < rng:
                break
        if u:
            v[k], v[k + u] = v[k + u], v[k]


def test_minibatch_schedule():
    g = mt19937(5489)
    for _ in range(9999):
        next(g)
    assert next(g) == 4123659995  # C++ standard [rand.predef]
    # Known answer worked by hand from the first nine outputs of
    # mt19937(0x9e3779b9) (rollout 0), five 256-row minibatches:
    #   1596107820 & 7 = 4 -> swap 0,4;  3571572850 & 3 = 2 -> swap 1,3;
    #   453773831 & 3 = 3 >= 3 rejected; 3932114620 & 3 = 0 -> keep;
    #   2314964120 & 1 = 0 -> keep: epoch 0 = 1024 768 512 256 0.
    #   1166738570 & 7 = 2 -> swap 0,2;  465115713 & 3 = 1 -> swap 1,2;
    #   4090974150 & 3 = 2 -> swap 2,4;  1413185717 & 1 = 1 -> swap 3,4:
    #   epoch 1 = 512 1024 0 768 256.
    g = mt19937(0x9e3779b9)
    assert [next(g) for _ in range(9)] == [1596107820, 3571572850, 453773831, 3932114620, 2314964120,
                                           1166738570, 465115713, 4090974150, 1413185717]
    got = np.zeros(10, np.uint32)
    oracle().orc_minibatch_schedule(1280, 256, 2, 0, ptr(got))
    assert got.tolist() == [1024, 768, 512, 256, 0, 512, 1024, 0, 768, 256]
    # the restatement above over larger cases (ranges that are and are not
    # powers of two, a ragged last minibatch, reshuffle only before epoch 1)
    for rows, mb, epochs, rollout in [(4096, 256, 3, 5), (1000, 96, 2, 17), (262144, 256, 2, 3),
                                      (1048576, 262144, 1, 9)]:
        nb = (rows + mb - 1) // mb
        got = np.zeros(nb * epochs, np.uint32)
        oracle().orc_minibatch_schedule(rows, mb, epochs, rollout, ptr(got))
        starts = list(range(0, rows, mb))
        gen = mt19937((0x9e3779b9 + rollout * 0x85ebca6b) & 0xffffffff)
        libcxx_shuffle(starts, gen)
        want = list(starts)
        for e in range(1, epochs):
            if e == 1:
                libcxx_shuffle(starts, gen)
            want += starts
        assert got.tolist() == want
        for e in range(epochs):
            assert sorted(got[nb * e:nb * (e + 1)].tolist()) == starts_sorted(rows, mb)


def starts_sorted(rows, mb):
    return list(range(0, rows, mb))


@needs_ref
def test_policy_initialisation_stream():
    """initialize_policy (cpu_reference.hpp:89-103): seed-1789 stream drawn
    with the reference's own wurand, transformed with float64 libm."""
    import ctypes
    actor = np.zeros(abi.policy_shape()["actor_count"], F)
    critic = np.zeros(abi.policy_shape()["critic_count"], F)
    oracle().orc_init_policy(ptr(actor), ptr(critic))
    seed = ctypes.c_uint32(1789)
    lib = ref()

    def normal():
        u = max(lib.ref_urand(ctypes.byref(seed)), 1e-7)
        v = lib.ref_urand(ctypes.byref(seed))
        return np.sqrt(-2 * np.log(np.float64(F(u)))) * np.cos(np.float64(F(6.2831853)) * np.float64(F(v)))
    sh = abi.policy_shape()
    want_a = np.zeros_like(actor, np.float64)
    for i in range(sh["actor_b1"]):
        want_a[i] = normal() * 0.04
    for i in range(sh["actor_w2"], sh["actor_b2"]):
        want_a[i] = normal() * 0.01
    want_a[sh["actor_log_std"]:] = -1
    want_c = np.zeros_like(critic, np.float64)
    for i in range(sh["critic_b1"]):
        want_c[i] = normal() * 0.15
    for i in range(sh["critic_w2"], sh["critic_b2"]):
        want_c[i] = normal() * 0.1
    assert np.abs(actor - want_a).max() < 1e-6
    assert np.abs(critic - want_c).max() < 2e-6
