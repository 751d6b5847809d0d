"""GPU parity of the on-device rollout step (zl_ppo_act): GpuPolicy::forward
(src/biped/gpu_policy.rs:210-248) plus the trainer's sampling loop
(src/bin/biped_train_gpu.rs:910-930) against the oracle's ActorCritic
(mean / value with its own running normalisers, logp; zealot-rl/src/ppo.rs:
276-306).

The GPU normalisers hold the oracle's Welford state (the same rows folded one
at a time by Normalizer::update), so normalisation is bit-exact and the nets
are compared at the forward tolerance 1e-4 of the largest |output|; actions
follow from the GPU means (mean + exp(log_std) * eps, one rounding each) and
logp is checked against the oracle's ActorCritic::logp of the GPU's own
action and mean."""

import os

import numpy as np
import pytest

from conftest import rel_amax
from oracle import zl_oracle as zo
from zealot_amd import Context, synth
from zealot_amd.rl import GpuActorCritic, GpuNormalizer

pytestmark = pytest.mark.gpu

TOL = 1e-4


def raw_obs(seed, n, dim):
    g = np.random.default_rng(seed)
    return (g.standard_normal((n, dim)) * g.uniform(0.2, 3.0, dim) + g.uniform(-3, 3, dim)).astype(np.float32)


@pytest.mark.parametrize("n,mb", [(6000, 2048), (4096, 4096), (1, 64)])
def test_act_matches_oracle_actor_critic(ctx, n, mb):
    ad, cd = synth.ACTOR_DIMS, [64, 512, 256, 128, 1]  # same depth: grouped layer launches
    g = np.random.default_rng(n)
    actor = synth.kaiming_uniform_net(g, ad, 0.1)
    critic = synth.kaiming_uniform_net(g, cd, 0.1)
    log_std = (g.uniform(-1.0, 0.0, ad[-1])).astype(np.float32)
    ac = zo.ActorCritic(ad, cd, 1.0, 1e-3, seed=3)
    ac.set(actor, critic, log_std, 1e-3)
    # Running statistics: 500 recorded observation pairs (Normalizer::update).
    hist_o, hist_c = raw_obs(1, 500, ad[0]), raw_obs(2, 500, cd[0])
    for o, c in zip(hist_o, hist_c):
        ac.record_obs(o, c)
    st_o = zo.norm_update(zo.norm_new(ad[0]), hist_o)
    st_c = zo.norm_update(zo.norm_new(cd[0]), hist_c)
    obs, cobs = raw_obs(3 + n, n, ad[0]), raw_obs(4 + n, n, cd[0])
    eps = g.standard_normal((n, ad[-1])).astype(np.float32)

    gac = GpuActorCritic(ctx, ad, cd, mb)
    gac.set_params(actor, critic, log_std, 1e-3)
    on = GpuNormalizer.from_state(ctx, st_o[:ad[0]], st_o[ad[0]:2 * ad[0]], float(st_o[-1]))
    cn = GpuNormalizer.from_state(ctx, st_c[:cd[0]], st_c[cd[0]:2 * cd[0]], float(st_c[-1]))
    A = ad[-1]
    d_act, d_lp, d_mean, d_val = ctx.alloc((n, A)), ctx.alloc(n), ctx.alloc((n, A)), ctx.alloc(n)
    gac.act(ctx.to_device(obs), n, ctx.to_device(eps), d_act, d_lp, mean=d_mean, value=d_val,
            critic_obs=ctx.to_device(cobs), obs_norm=on, critic_norm=cn)
    act, lp, mean, val = d_act.numpy(), d_lp.numpy(), d_mean.numpy(), d_val.numpy()

    rows = range(n) if n <= 1000 else np.linspace(0, n - 1, 1000).astype(int)
    ref_mean = np.stack([ac.mean(obs[r]) for r in rows])
    ref_val = np.array([ac.value(cobs[r]) for r in rows], np.float32)
    e_mean, e_val = rel_amax(mean[rows], ref_mean), rel_amax(val[rows], ref_val)
    std = np.exp(log_std).astype(np.float32)
    e_act = float(np.max(np.abs(act - (mean + std * eps))))
    ref_lp = np.array([ac.logp(act[r], mean[r]) for r in rows], np.float32)
    e_lp = rel_amax(lp[rows], ref_lp)
    print(f"[gpu] act n={n} mb={mb}: mean {e_mean:.2e} value {e_val:.2e} action {e_act:.2e} "
          f"logp {e_lp:.2e}", flush=True)
    assert e_mean <= TOL and e_val <= TOL
    assert e_act <= 1e-6 * max(1.0, float(np.max(np.abs(act))))
    assert e_lp <= 1e-5
    gac.close()


def test_act_prenormalised_actor_only(ctx):
    """NULL normaliser (rows already normalised) and no critic: the actor
    means equal zl_ppo_actor_mean's, the actions and logp zl_sample_actions'."""
    ad, cd = [37, 64, 48, 7], [37, 64, 48, 1]
    g = np.random.default_rng(11)
    actor = synth.kaiming_uniform_net(g, ad, 0.1)
    critic = synth.kaiming_uniform_net(g, cd, 0.1)
    log_std = np.full(ad[-1], -0.5, np.float32)
    n = 3000
    gac = GpuActorCritic(ctx, ad, cd, 1024)
    gac.set_params(actor, critic, log_std, 1e-3)
    obs = np.clip(g.standard_normal((n, ad[0])), -5, 5).astype(np.float32)
    eps = g.standard_normal((n, ad[-1])).astype(np.float32)
    d_obs = ctx.to_device(obs)
    d_act, d_lp, d_mean = ctx.alloc((n, 7)), ctx.alloc(n), ctx.alloc((n, 8))
    gac.act(d_obs, n, ctx.to_device(eps), d_act, d_lp, mean=d_mean, ld_mean=8)
    ref_mean = ctx.alloc((n, 7))
    gac.actor_mean(d_obs, n, ref_mean)
    assert np.array_equal(d_mean.numpy()[:, :7], ref_mean.numpy())
    ref = zo.mlp_forward(ad, actor, obs)[-1]
    assert rel_amax(ref_mean.numpy(), ref) <= TOL
    lp_ref = synth.gaussian_logp(d_act.numpy(), ref_mean.numpy(), log_std)
    assert rel_amax(d_lp.numpy(), lp_ref) <= 1e-5
    gac.close()


def test_act_rejects_critic_norm_without_value(ctx):
    from zealot_amd import ZealotError
    ad, cd = [8, 16, 3], [8, 16, 1]
    gac = GpuActorCritic(ctx, ad, cd, 64)
    cn = GpuNormalizer(ctx, 8)
    x = ctx.alloc((4, 8))
    with pytest.raises(ZealotError):
        gac.act(x, 4, ctx.alloc((4, 3)), ctx.alloc((4, 3)), ctx.alloc(4), critic_norm=cn, critic_obs=x)
    gac.close()


TRAINER_A, TRAINER_C = [265, 256, 256, 128, 12], [64, 512, 256, 128, 1]


@pytest.mark.parametrize("n,ad,cd", [(4096, synth.ACTOR_DIMS, [64, 512, 256, 128, 1]),
                                     (1000, synth.ACTOR_DIMS, [64, 512, 256, 128, 1]),
                                     (17, synth.ACTOR_DIMS, [64, 512, 256, 128, 1]),
                                     (1, synth.ACTOR_DIMS, [64, 512, 256, 128, 1]),
                                     (4096, TRAINER_A, TRAINER_C),
                                     (777, [64, 128, 64, 9], [48, 96, 48, 1]),
                                     (300, [64, 128, 64, 9], [48, 100, 1])])
def test_fused_policy_step_matches_layer_launches(ctx, n, ad, cd):
    """zk_policy (normalise, every layer of both nets and the sampling in one
    launch, 16 rows per block) against the layer-GEMM launches
    (ZL_POLICY_FUSED=0, read when a context is created: that run gets a
    context of its own), on the headline nets, the reference trainer's nets
    (a 265-wide input, 16-padded inside its 288-wide weight rows), narrow
    ones, and a critic whose 100-wide hidden layer does not fit the single
    launch (only the actor has a packed weight copy; steps with the value
    take the layer launches for both nets). Both add every reduction in the same order, so actions,
    log-probabilities, means and values are bit-identical; so are the plain
    forwards of zl_ppo_values and zl_ppo_actor_mean at these sizes."""
    g = np.random.default_rng(40 + n + ad[0])
    actor = synth.kaiming_uniform_net(g, ad, 0.1)
    critic = synth.kaiming_uniform_net(g, cd, 0.1)
    log_std = (g.uniform(-1.0, 0.0, ad[-1])).astype(np.float32)
    st_o = zo.norm_update(zo.norm_new(ad[0]), raw_obs(5, 300, ad[0]))
    st_c = zo.norm_update(zo.norm_new(cd[0]), raw_obs(6, 300, cd[0]))
    obs, cobs = raw_obs(7 + n, n, ad[0]), raw_obs(8 + n, n, cd[0])
    eps = g.standard_normal((n, ad[-1])).astype(np.float32)
    A = ad[-1]
    out = []
    for fused in (True, False):
        if not fused:
            os.environ["ZL_POLICY_FUSED"] = "0"
        try:
            cx = ctx if fused else Context(0)
        finally:
            os.environ.pop("ZL_POLICY_FUSED", None)
        gac = GpuActorCritic(cx, ad, cd, 2048)
        gac.set_params(actor, critic, log_std, 1e-3)
        on = GpuNormalizer.from_state(cx, st_o[:ad[0]], st_o[ad[0]:2 * ad[0]], float(st_o[-1]))
        cn = GpuNormalizer.from_state(cx, st_c[:cd[0]], st_c[cd[0]:2 * cd[0]], float(st_c[-1]))
        d_obs, d_cobs, d_eps = cx.to_device(obs), cx.to_device(cobs), cx.to_device(eps)
        d_act, d_lp, d_mean, d_val = cx.alloc((n, A)), cx.alloc(n), cx.alloc((n, A)), cx.alloc(n)
        gac.act(d_obs, n, d_eps, d_act, d_lp, mean=d_mean, value=d_val, critic_obs=d_cobs,
                obs_norm=on, critic_norm=cn)
        r = [d_act.numpy(), d_lp.numpy(), d_mean.numpy(), d_val.numpy()]
        # actor only, inputs already normalised
        gac.act(d_obs, n, d_eps, d_act, d_lp)
        r += [d_act.numpy(), d_lp.numpy()]
        pv, pm = cx.alloc(n), cx.alloc((n, A))
        gac.values(d_cobs, n, pv)
        gac.actor_mean(d_obs, n, pm)
        r += [pv.numpy(), pm.numpy()]
        out.append(r)
        gac.close()
        del on, cn, d_obs, d_cobs, d_eps, d_act, d_lp, d_mean, d_val, pv, pm
        if not fused:
            cx.close()
    names = ["action", "logp", "mean", "value", "action (actor only)", "logp (actor only)", "values",
             "actor mean"]
    for name, x, y in zip(names, out[0], out[1]):
        assert np.array_equal(x, y), name
    print(f"[gpu] fused policy step n={n} actor {ad}: bit-identical to the layer launches", flush=True)


def test_policy_weights_follow_parameter_changes(ctx):
    """zk_policy reads a fragment-major copy of the weights that the handle
    rewrites after every parameter change (zk_policy_pack). After
    set_params, after each of two updates (the second replays the captured
    graph), after an update that early-stops in its first epoch and after a
    checkpoint loaded into the same handle, the rollout step, zl_ppo_values
    and zl_ppo_actor_mean equal the layer launches (ZL_POLICY_FUSED=0, a
    context of its own) on the same parameters, bit for bit."""
    from test_gpu_ppo import SMALL_A, SMALL_C, _small_problem
    from zealot_amd.rl import DeviceBatch, PpoConfig

    actor, critic, log_std, batch = _small_problem(71, n=4096)
    os.environ["ZL_POLICY_FUSED"] = "0"
    try:
        cref = Context(0)
    finally:
        os.environ.pop("ZL_POLICY_FUSED", None)
    gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, 1024)
    ref = GpuActorCritic(cref, SMALL_A, SMALL_C, 1024)
    n, A = 1000, SMALL_A[-1]
    g = np.random.default_rng(72)
    obs = g.standard_normal((n, SMALL_A[0])).astype(np.float32)
    cobs = g.standard_normal((n, SMALL_C[0])).astype(np.float32)
    eps = g.standard_normal((n, A)).astype(np.float32)

    def step(h, cx):
        d_obs, d_cobs, d_eps = cx.to_device(obs), cx.to_device(cobs), cx.to_device(eps)
        d_act, d_lp, d_mean, d_val = cx.alloc((n, A)), cx.alloc(n), cx.alloc((n, A)), cx.alloc(n)
        h.act(d_obs, n, d_eps, d_act, d_lp, mean=d_mean, value=d_val, critic_obs=d_cobs)
        pv, pm = cx.alloc(n), cx.alloc((n, A))
        h.values(d_cobs, n, pv)
        h.actor_mean(d_obs, n, pm)
        return [x.numpy() for x in (d_act, d_lp, d_mean, d_val, pv, pm)]

    def check(tag):
        a, c, l, lr = gac.get_params()
        ref.set_params(a, c, l, lr)
        got, want = step(gac, ctx), step(ref, cref)
        for name, x, y in zip(["action", "logp", "mean", "value", "values", "actor mean"], got, want):
            assert np.array_equal(x, y), (tag, name)
        print(f"[gpu] policy copy current after {tag}", flush=True)

    gac.set_params(actor, critic, log_std, 1e-3)
    check("set_params")
    db = DeviceBatch(ctx, batch["obs"], batch["critic_obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    cfg = PpoConfig(epochs=2, minibatches=4)
    for i in range(2):
        gac.update(db, cfg)
        check(f"update {i + 1}")
    assert gac.graph_info()[0] == 1
    st = gac.update(db, PpoConfig.gpu_trainer(epochs=3, minibatches=4, desired_kl=1e-12))
    assert st.epochs_run == 1
    check("an early-stopped update")
    other = GpuActorCritic(ctx, SMALL_A, SMALL_C, 1024)
    other.set_params(actor * np.float32(0.5), critic, log_std - np.float32(0.25), 2e-3)
    gac.load_into(other.save_bytes())
    check("a checkpoint load")
    for h in (other, gac, ref):
        h.close()
    cref.close()
