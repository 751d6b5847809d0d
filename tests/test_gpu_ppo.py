"""GPU parity of the composed PPO path: one minibatch's gradients at the
24,576-row configuration, and whole updates under both reference semantics
(ActorCritic::update, zealot-rl/src/ppo.rs:338-510; the GPU trainer,
src/bin/biped_train_gpu.rs:1164-1553) against the CPU oracle.

Gradients are compared per tensor at 1e-4 of the tensor's max |value|, with
a float64 numpy restatement as the truth leg. Whole updates compare the
parameter change: Adam's first steps are ~lr * sign(g), so a gradient
component whose fp32 value is within rounding of zero can flip sign between
any two valid summation orders (rayon's own grouping is not fixed either);
the test bounds the fraction of such components and checks everything else
tightly, plus the scalar statistics and the adaptive learning rate."""

import os

import numpy as np
import pytest

import np_ref
from conftest import rel_amax
from oracle import zl_oracle as zo
from zealot_amd import ZealotError, synth
from zealot_amd.rl import DeviceBatch, GpuActorCritic, PpoConfig

pytestmark = pytest.mark.gpu

TOL = 1e-4
NTHREADS = min(os.cpu_count() or 1, 16)  # the GPU box gives one GPU 16 host cores


def per_tensor_err(dims, got, ref):
    o, worst = 0, 0.0
    for l in range(len(dims) - 1):
        for sz in (dims[l + 1] * dims[l], dims[l + 1]):
            worst = max(worst, rel_amax(got[o:o + sz], ref[o:o + sz]))
            o += sz
    return worst


def f32_forward(dims, packed, x):
    """Fast float32 numpy forward (input generation only)."""
    acts = np_ref.forward(dims, packed, x.astype(np.float64))
    return acts[-1].astype(np.float32)


def make_batch(n, actor_dims, critic_dims, actor, critic, seed):
    g = np.random.default_rng(seed)
    obs = synth.obs(g, n, actor_dims[0])
    means = f32_forward(actor_dims, actor, obs)
    values = f32_forward(critic_dims, critic, obs)
    mb = synth.minibatch_inputs(g, n, means, values)
    batch = dict(obs=obs, critic_obs=obs, action=mb["action"], mean_old=means,
                 logp_old=mb["logp_old"], value_old=mb["value_old"], adv=mb["adv"], ret=mb["ret"])
    return batch, mb["log_std"]


def move_off_branch_boundaries(batch, actor_dims, critic_dims, actor, critic, log_std, clip=0.2,
                               margin=1e-2):
    """The clipped objectives are discontinuous: a sample whose ratio sits on
    1 +- clip (ppo.rs:419-420), or whose clipped and unclipped value losses tie
    with v_clipped != v (ppo.rs:443), switches its whole gradient on a last-ulp
    difference of the forward pass, and any two valid fp32 evaluations (rayon's
    included) may land on either side. With N(0,1) actions the log-probs reach
    ~-500, where fp32 rounding moves log(ratio) by ~1e-3. Rows within `margin`
    of a boundary (in log-ratio, resp. relative loss gap) get logp_old / ret
    nudged clear of it; returns the number of rows moved."""
    aa = np_ref.forward(actor_dims, actor, batch["obs"])
    d = batch["action"] - aa[-1]
    ls = np.asarray(log_std, np.float64)
    lp = np.sum(-0.5 * (d / np.exp(ls)) ** 2 - ls - np_ref.LOG_SQRT_2PI, axis=1)
    logr = lp - batch["logp_old"]
    moved = 0
    for b in (np.log1p(clip), np.log1p(-clip)):
        near = np.abs(logr - b) < margin
        shift = np.where(logr >= b, 2 * margin, -2 * margin)  # push away from b
        batch["logp_old"] = np.where(near, batch["logp_old"] - shift, batch["logp_old"]).astype(np.float32)
        logr = np.where(near, logr + shift, logr)
        moved += int(near.sum())
    v = np_ref.forward(critic_dims, critic, batch["critic_obs"])[-1][:, 0]
    vo, R = batch["value_old"].astype(np.float64), batch["ret"].astype(np.float64)
    vc = vo + np.clip(v - vo, -clip, clip)
    lu, lc = (v - R) ** 2, (vc - R) ** 2
    tie = (np.abs(lc - lu) < margin * np.maximum(np.maximum(lc, lu), 1e-6)) & (np.abs(vc - v) > 1e-6)
    mid = 0.5 * (v + vc)
    away = np.where(R >= mid, 1.0, -1.0) * 0.05 * np.abs(vc - v)
    batch["ret"] = np.where(tie, R + away, R).astype(np.float32)
    return moved + int(tie.sum())


def test_minibatch_grads_config4(ctx):
    """Config 4: one 24,576-row minibatch, actor 123-512-256-128-29 + critic
    123-512-256-128-1, clip 0.2, value x1.0, entropy x0.005."""
    ad, cd = synth.ACTOR_DIMS, synth.CRITIC_DIMS
    g = synth.rng(4)
    actor = synth.kaiming_uniform_net(g, ad)
    critic = synth.kaiming_uniform_net(g, cd)
    n = 24_576
    batch, log_std = make_batch(n, ad, cd, actor, critic, seed=synth.SEED_BASE + 4)
    batch["adv"] = zo.adv_normalize(batch["adv"])
    moved = move_off_branch_boundaries(batch, ad, cd, actor, critic, log_std)
    print(f"[gpu] config4: {moved} of {n} rows moved off a clip / value-loss branch boundary", flush=True)
    assert moved < n // 1000
    gac = GpuActorCritic(ctx, ad, cd, n)
    gac.set_params(actor, critic, log_std, 1e-3)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    cfg = PpoConfig(clip=0.2, value_coef=1.0, entropy_coef=0.005)
    ga, gc, gl, st = gac.minibatch_grads(db, cfg, 0, n)
    idx = np.arange(n)
    ra, rc, rl, rst = zo.minibatch_grads(ad, cd, actor, critic, log_std, batch, idx, 0.2, 0.005, 1.0,
                                         nthreads=NTHREADS)
    ta, tc, tl, tst = np_ref.minibatch_grads(ad, cd, actor, critic, log_std, batch, idx, 0.2, 0.005, 1.0)
    e = dict(
        actor=per_tensor_err(ad, ga, ra), critic=per_tensor_err(cd, gc, rc), log_std=rel_amax(gl, rl),
        actor_gpu_vs_f64=per_tensor_err(ad, ga, ta), actor_cpu_vs_f64=per_tensor_err(ad, ra, ta),
        critic_gpu_vs_f64=per_tensor_err(cd, gc, tc), critic_cpu_vs_f64=per_tensor_err(cd, rc, tc),
    )
    print(f"[gpu] config4 grads: {e}; stats gpu {st} cpu {rst} f64 {tst}", flush=True)
    assert e["actor"] <= TOL and e["critic"] <= TOL and e["log_std"] <= TOL
    assert abs(st["surrogate"] - rst[0]) <= 1e-4 * max(1, abs(rst[0]))
    assert abs(st["value_loss"] - rst[1]) <= 1e-4 * max(1, abs(rst[1]))
    assert abs(st["kl"] - rst[2]) <= 1e-4 * max(1e-3, abs(rst[2]))
    gac.close()


@pytest.mark.parametrize("hidden", [64, 24])
def test_minibatch_grads_with_perm(ctx, hidden):
    """Row gather through a device permutation (the shuffled minibatch); a
    24-wide first layer sends the gathered rows through the narrow kernels."""
    ad, cd = [37, hidden, 48, 7], [37, hidden, 48, 1]
    g = np.random.default_rng(8)
    actor = synth.kaiming_uniform_net(g, ad, 0.1)
    critic = synth.kaiming_uniform_net(g, cd, 0.1)
    n = 5000
    batch, log_std = make_batch(n, ad, cd, actor, critic, seed=99)
    move_off_branch_boundaries(batch, ad, cd, actor, critic, log_std)
    perm = g.permutation(n).astype(np.int32)
    gac = GpuActorCritic(ctx, ad, cd, 1500)
    gac.set_params(actor, critic, log_std, 1e-3)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    ga, gc, gl, st = gac.minibatch_grads(db, PpoConfig(entropy_coef=0.01), 1000, 1500,
                                         perm=ctx.to_device(perm))
    idx = perm[1000:2500]
    ra, rc, rl, rst = zo.minibatch_grads(ad, cd, actor, critic, log_std, batch, idx, 0.2, 0.01, 1.0)
    assert per_tensor_err(ad, ga, ra) <= TOL and per_tensor_err(cd, gc, rc) <= TOL
    assert rel_amax(gl, rl) <= TOL


def _param_delta_report(p0, pg, pc, lr, steps):
    dg, dc = pg - p0, pc - p0
    diff = np.abs(dg.astype(np.float64) - dc)
    scale = lr * steps
    frac_bad = float(np.mean(diff > 1e-2 * lr))
    return dict(max_abs=float(diff.max()), bound=2 * scale, frac_gt_1pct_lr=frac_bad,
                rel_delta=rel_amax(dg, dc))


SMALL_A = [123, 128, 64, 29]
SMALL_C = [123, 128, 64, 1]


def _small_problem(seed, n=8192):
    g = np.random.default_rng(seed)
    actor = synth.kaiming_uniform_net(g, SMALL_A, 0.05)
    critic = synth.kaiming_uniform_net(g, SMALL_C, 0.05)
    batch, log_std = make_batch(n, SMALL_A, SMALL_C, actor, critic, seed + 1)
    move_off_branch_boundaries(batch, SMALL_A, SMALL_C, actor, critic, log_std)
    return actor, critic, log_std, batch


@pytest.mark.parametrize("adaptive", [False, True])
def test_update_actor_critic_semantics(ctx, adaptive):
    """ActorCritic::update: per-epoch Fisher-Yates shuffle, per-net clip, per-step
    KL-adaptive LR, log_std Adam with clamp [-1.6, 1.0]."""
    actor, critic, log_std, batch = _small_problem(41)
    lr0 = 1e-3
    ac = zo.ActorCritic(SMALL_A, SMALL_C, 1.0, lr0, 1)
    ac.set(actor, critic, log_std, lr0)
    cfg_o = zo.PpoCfg(0.99, 0.95, 0.2, 0.01, 1.0, 5, 4, 1.0, 0.01, 1e-5, 1e-2, int(adaptive))
    stats_o, adv_o = ac.update(batch, cfg_o, nthreads=NTHREADS, normalize_obs=False)
    ao, co, lso, lro, to = ac.get()

    gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, batch["obs"].shape[0] // 4)
    gac.set_params(actor, critic, log_std, lr0)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    st = gac.update(db, PpoConfig(epochs=5, minibatches=4, adaptive_lr=adaptive, shuffle=True,
                                  normalize_adv=True, clamp_log_std=True))
    ag, cg, lsg, lrg = gac.get_params()
    t, _ = gac.counters()
    rep_a = _param_delta_report(actor, ag, ao, lr0, 20)
    rep_c = _param_delta_report(critic, cg, co, lr0, 20)
    print(f"[gpu] AC update adaptive={adaptive}: actor {rep_a} critic {rep_c} "
          f"log_std {rel_amax(lsg - log_std, lso - log_std):.2e} lr {lrg} vs {lro} "
          f"stats gpu {st} cpu {stats_o}", flush=True)
    assert t == to == 20
    assert np.allclose(db.adv.numpy(), adv_o, rtol=1e-5, atol=1e-6)
    assert lrg == pytest.approx(lro, rel=1e-6)
    for rep in (rep_a, rep_c):
        assert rep["max_abs"] <= rep["bound"]
        assert rep["frac_gt_1pct_lr"] < 0.01
    assert rel_amax(lsg - log_std, lso - log_std) < 1e-2
    for k, gv in zip(("kl", "surrogate", "value_loss", "entropy"), (st.kl, st.surrogate, st.value_loss, st.entropy)):
        ov = stats_o[["kl", "surrogate", "value_loss", "entropy"].index(k)]
        assert abs(gv - ov) <= 1e-3 * max(abs(ov), 1e-2), (k, gv, ov)
    gac.close()


@pytest.mark.parametrize("early", [False, True])
def test_update_gpu_trainer_semantics(ctx, early):
    """GPU trainer update: contiguous minibatches, global clip (incl. log_std),
    per-epoch gstep bias correction, per-epoch full-Gaussian KL -> LR + early stop,
    log_std clamped to [-1.6, 0.0] after the update."""
    actor, critic, log_std, batch = _small_problem(77)
    batch["adv"] = zo.adv_normalize(batch["adv"])
    lr0 = 3e-3 if early else 1e-3
    tr = zo.Trainer(SMALL_A, SMALL_C, actor, critic, log_std, lr0)
    desired = 0.002 if early else 0.01
    cfg_o = zo.TrainerCfg(0.2, 0.01, 1.0, 5, 4, 1.0, desired, 1e-5, 1e-2, 1, int(early), 1)
    so = tr.update(batch, cfg_o, nthreads=NTHREADS)
    ao, co, lso, lro, gso = tr.get()

    gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, batch["obs"].shape[0] // 4)
    gac.set_params(actor, critic, log_std, lr0)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    cfg = PpoConfig.gpu_trainer(epochs=5, minibatches=4, entropy_coef=0.01, value_coef=1.0,
                                max_grad_norm=1.0, desired_kl=desired, early_stop=early,
                                normalize_adv=False)
    st = gac.update(db, cfg)
    ag, cg, lsg, lrg = gac.get_params()
    _, gstep = gac.counters()
    steps = int(so[5]) * 4
    rep_a = _param_delta_report(actor, ag, ao, lr0, steps)
    rep_c = _param_delta_report(critic, cg, co, lr0, steps)
    print(f"[gpu] trainer update early={early}: epochs gpu {st.epochs_run} cpu {int(so[5])} "
          f"kl {st.last_kl:.4e} vs {so[6]:.4e} lr {lrg} vs {lro} actor {rep_a} critic {rep_c}", flush=True)
    assert st.epochs_run == int(so[5])
    assert gstep == gso == 4 * st.epochs_run  # gstep += n_mb per epoch that ran (:1165)
    assert abs(st.last_kl - so[6]) <= 1e-3 * max(abs(so[6]), 1e-4)
    assert lrg == pytest.approx(lro, rel=1e-6)
    assert np.all(lsg <= 0.0) and np.all(lsg >= -1.6)
    for rep in (rep_a, rep_c):
        assert rep["max_abs"] <= rep["bound"]
        assert rep["frac_gt_1pct_lr"] < 0.01
    gac.close()


def test_update_deterministic_and_replay(ctx):
    """Two updates from the same state are bit-identical (atomic-free
    reductions), and the second runs the cached hipGraph."""
    actor, critic, log_std, batch = _small_problem(5, n=4096)
    gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, 1024)
    outs = []
    for _ in range(3):
        gac.set_params(actor, critic, log_std, 1e-3)
        gac.reset_optimizer()
        db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                         batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
        gac.update(db, PpoConfig(epochs=2, minibatches=4))
        outs.append(gac.get_params())
        del db
    for o in outs[1:]:
        for x, y in zip(o[:3], outs[0][:3]):
            assert np.array_equal(x, y)
    gac.close()


def test_values_and_actor_mean(ctx):
    """Config 2 (actor inference over 4096 rows) and critic values."""
    c2 = synth.config2()
    critic = synth.kaiming_uniform_net(synth.rng(2, 1), synth.CRITIC_DIMS)
    gac = GpuActorCritic(ctx, synth.ACTOR_DIMS, synth.CRITIC_DIMS, 1024)
    gac.set_params(c2["actor"], critic, c2["log_std"], 1e-3)
    dobs = ctx.to_device(c2["obs"])
    mean = ctx.alloc((4096, 29))
    vals = ctx.alloc(4096)
    gac.actor_mean(dobs, 4096, mean)
    gac.values(dobs, 4096, vals)
    rm = zo.mlp_forward(synth.ACTOR_DIMS, c2["actor"], c2["obs"])[-1]
    rv = zo.mlp_forward(synth.CRITIC_DIMS, critic, c2["obs"])[-1][:, 0]
    assert rel_amax(mean.numpy(), rm) <= TOL
    assert rel_amax(vals.numpy(), rv) <= TOL
    gac.close()


def test_self_test_failure_branch():
    """zl_init's failure branch (CutileGemm::init -> None, src/biped/cutile_gemm.rs:412-423)."""
    from zealot_amd import Context

    os.environ["ZL_FORCE_SELF_TEST_FAIL"] = "1"
    try:
        with pytest.raises(ZealotError) as ei:
            Context(0)
        assert ei.value.status == 4
    finally:
        del os.environ["ZL_FORCE_SELF_TEST_FAIL"]
