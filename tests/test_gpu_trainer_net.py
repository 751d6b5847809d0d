"""GPU parity at the reference trainer's own networks and at the headline
workload as stated.

The trainer's nets are asymmetric (src/bin/biped_train_gpu.rs:604-610,
zealot-env/src/tasks/velocity_flat.rs:58-72): actor [265, 256, 256, 128, 12]
on the policy observation, critic [64, 512, 256, 128, 1] on a separate
privileged critic observation, so the actor's and the critic's layers of one
depth have different K and N inside each grouped launch, and the critic
observation is staged on its own. The batches here are passed as the
trainer stages them: feature-major [dim x n] tensors.

The headline workload (4096 envs x 24 steps, actor 123-512-256-128-29,
critic 123-512-256-128-1) is run at its stated settings: critic values over
the rollout -> GAE -> advantage normalisation inside the update -> 5 epochs x
4 minibatches at clip 0.2, lr 1e-3, global clip 1.0."""

import os

import numpy as np
import pytest

import np_ref
import yardstick as ys
from conftest import rel_amax
from oracle import zl_oracle as zo
from test_gpu_ppo import (WELL_POSED_CLIP, _assert_tight, _param_delta_report, f32_forward,
                          move_off_branch_boundaries, per_tensor_err)
from zealot_amd import ops, synth
from zealot_amd.rl import DeviceBatch, GpuActorCritic, PpoConfig

pytestmark = pytest.mark.gpu

TOL = 1e-4
NTHREADS = min(os.cpu_count() or 1, 16)
TRAINER_A = [265, 256, 256, 128, 12]
TRAINER_C = [64, 512, 256, 128, 1]


def _trainer_batch(seed, n, clip_regime):
    """A batch for the trainer's nets with a separate 64-wide critic
    observation. clip_regime: config-4 style actions ~ N(0,1) (surrogate and
    value clips taken); otherwise the well-posed construction (actions
    sampled from the policy, action-correlated advantages, used with clip 100)."""
    g = np.random.default_rng(seed)
    actor = synth.kaiming_uniform_net(g, TRAINER_A, 0.05)
    critic = synth.kaiming_uniform_net(g, TRAINER_C, 0.05)
    obs = synth.obs(g, n, TRAINER_A[0])
    cobs = synth.obs(g, n, TRAINER_C[0])
    means = f32_forward(TRAINER_A, actor, obs)
    values = f32_forward(TRAINER_C, critic, cobs)[:, 0]
    A = TRAINER_A[-1]
    log_std = np.full(A, -0.5, np.float32)
    if clip_regime:
        mb = synth.minibatch_inputs(g, n, means, values)
        batch = dict(obs=obs, critic_obs=cobs, action=mb["action"], mean_old=means,
                     logp_old=mb["logp_old"], value_old=mb["value_old"], adv=mb["adv"], ret=mb["ret"])
    else:
        eps = g.standard_normal((n, A)).astype(np.float32)
        action = (means + np.exp(log_std) * eps).astype(np.float32)
        c = np.where(g.random(A) < 0.5, -1.0, 1.0)
        adv = (0.5 * (eps @ c) / np.sqrt(A) + 0.5 * g.standard_normal(n)).astype(np.float32)
        batch = dict(obs=obs, critic_obs=cobs, action=action, mean_old=means,
                     logp_old=synth.gaussian_logp(action, means, log_std),
                     value_old=(values + 0.05 * g.standard_normal(n)).astype(np.float32),
                     adv=adv, ret=g.standard_normal(n).astype(np.float32))
    return actor, critic, log_std, batch


def _device_batch(ctx, batch, fm=True):
    return DeviceBatch(ctx, batch["obs"], batch["critic_obs"], batch["action"], batch["mean_old"],
                       batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"], feature_major=fm)


def test_trainer_nets_minibatch_grads_24576(ctx):
    """One 24,576-row minibatch through the trainer's asymmetric nets (clip 0.2,
    value x1.0, entropy x0.005), feature-major inputs, against the oracle and
    the float64 truth, per tensor at 1e-4."""
    n = 24_576
    actor, critic, log_std, batch = _trainer_batch(61, n, clip_regime=True)
    batch["adv"] = zo.adv_normalize(batch["adv"])
    moved = move_off_branch_boundaries(batch, TRAINER_A, TRAINER_C, actor, critic, log_std)
    assert moved < n // 1000
    gac = GpuActorCritic(ctx, TRAINER_A, TRAINER_C, n)
    gac.set_params(actor, critic, log_std, 1e-3)
    db = _device_batch(ctx, batch)
    ga, gc, gl, st = gac.minibatch_grads(db, PpoConfig(clip=0.2, value_coef=1.0, entropy_coef=0.005), 0, n)
    idx = np.arange(n)
    ra, rc, rl, rst = zo.minibatch_grads(TRAINER_A, TRAINER_C, actor, critic, log_std, batch, idx, 0.2,
                                         0.005, 1.0, nthreads=NTHREADS)
    ta, tc, tl, tst = np_ref.minibatch_grads(TRAINER_A, TRAINER_C, actor, critic, log_std, batch, idx, 0.2,
                                             0.005, 1.0)
    e = dict(actor=per_tensor_err(TRAINER_A, ga, ra), critic=per_tensor_err(TRAINER_C, gc, rc),
             log_std=rel_amax(gl, tl), actor_f64=per_tensor_err(TRAINER_A, ga, ta),
             critic_f64=per_tensor_err(TRAINER_C, gc, tc))
    print(f"[gpu] trainer nets minibatch grads: {e}; stats gpu {st} cpu {rst}", flush=True)
    assert max(e.values()) <= TOL
    assert abs(st["surrogate"] - rst[0]) <= 1e-4 * max(1, abs(rst[0]))
    assert abs(st["value_loss"] - rst[1]) <= 1e-4 * max(1, abs(rst[1]))
    assert abs(st["kl"] - rst[2]) <= 1e-4 * max(1e-3, abs(rst[2]))
    gac.close()


@pytest.mark.parametrize("semantics", ["actor_critic", "gpu_trainer"])
def test_trainer_nets_update(ctx, semantics):
    """Whole updates (5 epochs x 4 minibatches of 6,144 rows) through the
    trainer's nets with the distinct critic observation, under both
    semantics, on the well-posed construction: parameters per component
    against the oracle. At lr 1e-3 these nets' 20-step update is chaotic in
    fp32 (on the oracle, a 1e-6 relative change of the observations moves the
    actor update by 1.7 % (ActorCritic) and 17 % (trainer) relative L2); at
    lr 1e-5 (trainer: adaptive up to 2e-5) the same change moves it by
    6e-5 / 3e-5, so per-component agreement is meaningful."""
    n, lr0 = 24_576, 1e-5
    actor, critic, log_std, batch = _trainer_batch(67, n, clip_regime=False)
    gac = GpuActorCritic(ctx, TRAINER_A, TRAINER_C, n // 4)
    gac.set_params(actor, critic, log_std, lr0)
    if semantics == "actor_critic":
        ac = zo.ActorCritic(TRAINER_A, TRAINER_C, 1.0, lr0, 1)
        ac.set(actor, critic, log_std, lr0)
        cfg_o = zo.PpoCfg(0.99, 0.95, WELL_POSED_CLIP, 0.01, 1.0, 5, 4, 1.0, 0.01, 1e-6, 1e-2, 0)
        stats_o, _ = ac.update(batch, cfg_o, nthreads=NTHREADS, normalize_obs=False)
        ao, co, lso, lro, _ = ac.get()
        cfg = PpoConfig(epochs=5, minibatches=4, clip=WELL_POSED_CLIP, adaptive_lr=False, lr_min=1e-6,
                        shuffle=True, normalize_adv=True, clamp_log_std=True)
        epochs_o = 5
    else:
        batch["adv"] = zo.adv_normalize(batch["adv"])
        tr = zo.Trainer(TRAINER_A, TRAINER_C, actor, critic, log_std, lr0)
        so = tr.update(batch, zo.TrainerCfg(WELL_POSED_CLIP, 0.01, 1.0, 5, 4, 1.0, 100.0, 1e-6, 2 * lr0, 1, 1, 1),
                       nthreads=NTHREADS)
        ao, co, lso, lro, _ = tr.get()
        cfg = PpoConfig.gpu_trainer(epochs=5, minibatches=4, clip=WELL_POSED_CLIP, entropy_coef=0.01,
                                    max_grad_norm=1.0, desired_kl=100.0, lr_min=1e-6, lr_max=2 * lr0,
                                    normalize_adv=False)
        epochs_o = int(so[5])
    db = _device_batch(ctx, batch)
    st = gac.update(db, cfg)
    ag, cg, lsg, lrg = gac.get_params()
    steps = 4 * epochs_o
    reps = dict(actor=_param_delta_report(actor, ag, ao, lr0, steps),
                critic=_param_delta_report(critic, cg, co, lr0, steps),
                log_std=_param_delta_report(log_std, lsg, lso, lr0, steps))
    print(f"[gpu] trainer nets update ({semantics}): {reps} lr {lrg} vs {lro}", flush=True)
    assert st.epochs_run == epochs_o == 5
    assert lrg == pytest.approx(lro, rel=1e-6)
    _assert_tight(reps)
    gac.close()


def test_config5_stated_settings_full_size(ctx):
    """The headline workload as the bench runs it: 4096 envs x 24 steps
    (98,304 samples), critic values over the rollout and the bootstrap
    observations, GAE (gamma 0.99, lambda 0.95), advantage normalisation
    inside the update, then 5 epochs x 4 contiguous minibatches of 24,576
    rows at clip 0.2, entropy 0.005, value x1.0, lr 1e-3 (fixed), global
    clip 1.0, log_std clamped to [-1.6, 0] after the update.

    Twenty full-size steps at lr 1e-3 with clip 0.2 are chaotic in fp32: any
    valid change of evaluation order moves the update by a few tenths of a
    percent (critic, log_std) to about 1.6 % (actor) relative L2, and more
    than half of the components by over 1 % of lr, so the parameters cannot
    be compared per component. The yardstick is the oracle's own spread
    (tests/yardstick.py): the oracle is run three more times on the same
    inputs, with another thread count (the fold grouping rayon leaves open,
    zealot-rl/src/ppo.rs:406-462) and with the observations moved by a last
    bit under two seeds, and the GPU's update must lie within 2x the largest
    distance of those runs from the oracle's, per net (a minibatch out of
    order lands 20-500x beyond it: test_update_yardstick_separates_minibatch_
    order). The fraction of components off by more than 1 % of lr is
    reported, not bounded: valid runs already reach 50-85 %. Also checked:
    two updates from one state are bit-identical; every parameter and moment
    is finite; the learning rate, gstep, epochs and the clamp range are
    exact; the value loss and entropy statistics match the oracle within
    1e-3."""
    ad, cd = synth.ACTOR_DIMS, synth.CRITIC_DIMS
    N, T = 4096, 24
    n, mb = N * T, N * T // 4
    g = synth.rng(5)
    ro = synth.rollout(g, N, T)
    actor = synth.kaiming_uniform_net(g, ad)
    critic = synth.kaiming_uniform_net(g, cd)
    log_std = np.full(ad[-1], -0.5, np.float32)
    gac = GpuActorCritic(ctx, ad, cd, mb)
    gac.set_params(actor, critic, log_std, 1e-3)
    d_obs, d_boot = ctx.to_device(ro["obs"]), ctx.to_device(ro["boot_obs"])
    d_mean, d_act, d_logp = ctx.alloc((n, ad[-1])), ctx.alloc((n, ad[-1])), ctx.alloc(n)
    gac.actor_mean(d_obs, n, d_mean)
    ops.sample_actions(ctx, d_mean, ctx.to_device(log_std), ctx.to_device(ro["eps"]), n, ad[-1], d_act, d_logp)
    d_val, d_last, d_adv, d_ret = ctx.alloc(n), ctx.alloc(N), ctx.alloc(n), ctx.alloc(n)
    gac.values(d_obs, n, d_val)
    gac.values(d_boot, N, d_last)
    ops.gae(ctx, ctx.to_device(ro["rewards"]), d_val, ctx.to_device(ro["dones"]), d_last, T, N, d_adv, d_ret,
            0.99, 0.95)
    values, adv_raw, ret = d_val.numpy(), d_adv.numpy(), d_ret.numpy()
    # The GAE inputs against the oracle: values within 1e-4, GAE of the same values bit-exact.
    rv = zo.mlp_forward(cd, critic, ro["obs"][:8192])[-1][:, 0]
    assert rel_amax(values[:8192], rv) <= TOL
    for e in range(0, N, 512):
        ra, rr = zo.gae(ro["rewards"][:, e], values.reshape(T, N)[:, e], ro["dones"][:, e],
                        float(d_last.numpy()[e]), 0.99, 0.95)
        assert np.array_equal(adv_raw.reshape(T, N)[:, e], ra)
    batch = dict(obs=ro["obs"], critic_obs=ro["obs"], action=d_act.numpy(), mean_old=d_mean.numpy(),
                 logp_old=d_logp.numpy(), value_old=values, adv=adv_raw, ret=ret)
    cfg = PpoConfig.gpu_trainer(epochs=5, minibatches=4, clip=0.2, entropy_coef=0.005, value_coef=1.0,
                                max_grad_norm=1.0, adaptive_lr=False, early_stop=False, normalize_adv=True,
                                clamp_log_std=True)
    runs = []
    for _ in range(2):
        gac.set_params(actor, critic, log_std, 1e-3)
        gac.reset_optimizer()
        db = DeviceBatch(ctx, ro["obs"], ro["obs"], batch["action"], batch["mean_old"], batch["logp_old"],
                         values, adv_raw, ret)
        st = gac.update(db, cfg)
        runs.append((gac.get_params(), gac.get_moments(), gac.counters(), st))
    (ag, cg, lsg, lrg), mom, (_, gstep), st = runs[0]
    for x, y in zip(runs[0][0][:3], runs[1][0][:3]):
        assert np.array_equal(x, y)
    assert runs[0][3] == runs[1][3]
    for x in (ag, cg, lsg, *mom):
        assert np.all(np.isfinite(x))
    assert st.epochs_run == 5 and gstep == 20 and lrg == np.float32(1e-3)
    assert np.all(lsg <= 0.0) and np.all(lsg >= -1.6)
    # The oracle on the same inputs (GPU-trainer semantics, 16 host threads),
    # then the three valid variants that measure its own spread.
    batch["adv"] = zo.adv_normalize(adv_raw)
    tcfg = zo.TrainerCfg(0.2, 0.005, 1.0, 5, 4, 1.0, 0.01, 1e-5, 1e-2, 0, 0, 1)

    def oracle(b, nth):
        tr = zo.Trainer(ad, cd, actor, critic, log_std, 1e-3)
        so_ = tr.update(b, tcfg, nthreads=nth)
        return tr.get(), so_

    (ao, co, lso, lro, gso), so = oracle(batch, NTHREADS)
    variants = [oracle(batch, max(1, NTHREADS - 4))[0]]
    for seed in (1, 2):
        b = dict(batch)
        b["obs"] = b["critic_obs"] = ys.perturb_last_bit(batch["obs"], seed)
        variants.append(oracle(b, NTHREADS)[0])
    p0, gpu, ref = (actor, critic, log_std), (ag, cg, lsg), (ao, co, lso)
    yard = {}
    for i, name in enumerate(("actor", "critic", "log_std")):
        ok, d, sp = ys.within(p0[i], ref[i], [v[i] for v in variants], gpu[i])
        yard[name] = dict(ok=ok, gpu_rel_l2=d, oracle_spread=sp,
                          frac_gt_1pct_lr=_param_delta_report(p0[i], gpu[i], ref[i], 1e-3, 20)["frac_gt_1pct_lr"])
    print(f"[gpu] config 5 stated settings: {yard}; stats gpu {st} cpu {so}", flush=True)
    assert gso == gstep and int(so[5]) == 5 and lro == lrg
    assert abs(st.value_loss - so[2]) <= 1e-3 * max(abs(so[2]), 1e-2)
    assert abs(st.entropy - so[3]) <= 1e-3 * max(abs(so[3]), 1e-2)
    for name, r in yard.items():
        assert r["ok"], (name, r)
    gac.close()
