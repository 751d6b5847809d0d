"""GPU tests of the drop-in boundary in the forms the reference trainer uses it:
feature-major [dim x n] batch tensors (src/bin/biped_train_gpu.rs:1029-1068),
fresh staging buffers on every update, the trainer's global grad-norm clip
computed on the device and applied inside a multi-tensor Adam
(src/bin/biped_train_gpu.rs:1368-1461), and the per-row outputs of the loss
operators that an operator-level swap of vortx's Ppo::actor_grad /
value_grad would consume."""

import numpy as np
import pytest

import np_ref
from conftest import rel_amax, ulp_diff
from oracle import zl_oracle as zo
from test_gpu_ppo import (SMALL_A, SMALL_C, WELL_POSED_CLIP, _small_problem, _well_posed_problem)
from zealot_amd import ops, synth
from zealot_amd.rl import DeviceBatch, GpuActorCritic, PpoConfig, packed_count

pytestmark = pytest.mark.gpu


def _batch(ctx, batch, fm, pad=0):
    return DeviceBatch(ctx, batch["obs"], batch["critic_obs"], batch["action"], batch["mean_old"],
                       batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"],
                       feature_major=fm, pad=pad)


def _run_update(ctx, actor, critic, log_std, batch, cfg, fm, gac=None, pad=0):
    own = gac is None
    if own:
        gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, batch["obs"].shape[0] // cfg.minibatches)
    gac.set_params(actor, critic, log_std, 1e-3)
    gac.reset_optimizer()
    db = _batch(ctx, batch, fm, pad)
    st = gac.update(db, cfg)
    out = gac.get_params(), gac.get_moments(), gac.counters(), st, db.adv.numpy()
    if own:
        gac.close()
    return out


@pytest.mark.parametrize("semantics", ["actor_critic", "gpu_trainer"])
def test_update_feature_major_batch_is_bit_identical(ctx, semantics):
    """The same batch passed feature-major ([dim x n], stride n: the trainer's
    f_obs / f_act / mean tensors) and batch-major gives bit-identical
    parameters, moments, counters, statistics and written-back normalised
    advantages: the update stages both into the same rows."""
    actor, critic, log_std, batch = _small_problem(23, n=4096)
    if semantics == "actor_critic":
        cfg = PpoConfig(epochs=2, minibatches=4, shuffle=True, normalize_adv=True)
    else:
        cfg = PpoConfig.gpu_trainer(epochs=2, minibatches=4, desired_kl=100.0, lr_max=2e-3)
    bm = _run_update(ctx, actor, critic, log_std, batch, cfg, False)
    fm = _run_update(ctx, actor, critic, log_std, batch, cfg, True)
    for x, y in zip(bm[0][:3], fm[0][:3]):
        assert np.array_equal(x, y)
    for x, y in zip(bm[1], fm[1]):
        assert np.array_equal(x, y)
    assert bm[0][3] == fm[0][3] and bm[2] == fm[2]
    assert bm[3] == fm[3]
    assert np.array_equal(bm[4], fm[4])
    # ... and the parameters moved (the comparison is not vacuous).
    assert np.max(np.abs(bm[0][0] - actor)) > 1e-4


@pytest.mark.parametrize("semantics", ["actor_critic", "gpu_trainer"])
def test_update_feature_major_strided_capacity(ctx, semantics):
    """Feature-major fields in tensors sized for a larger capacity: [dim x cap]
    with stride cap = n + 37 (a trainer buffer allocated for more samples than
    this update holds), the padding NaN. Bit-identical to the dense
    batch-major run."""
    actor, critic, log_std, batch = _small_problem(41, n=4096)
    if semantics == "actor_critic":
        cfg = PpoConfig(epochs=2, minibatches=4, shuffle=True, normalize_adv=True)
    else:
        cfg = PpoConfig.gpu_trainer(epochs=2, minibatches=4, desired_kl=100.0, lr_max=2e-3)
    bm = _run_update(ctx, actor, critic, log_std, batch, cfg, False)
    fm = _run_update(ctx, actor, critic, log_std, batch, cfg, True, pad=37)
    for x, y in zip(bm[0][:3], fm[0][:3]):
        assert np.array_equal(x, y)
    for x, y in zip(bm[1], fm[1]):
        assert np.array_equal(x, y)
    assert bm[0][3] == fm[0][3] and bm[2] == fm[2] and bm[3] == fm[3]
    assert np.array_equal(bm[4], fm[4])
    assert np.max(np.abs(bm[0][0] - actor)) > 1e-4


def test_update_feature_major_distinct_critic_obs(ctx):
    """Feature-major actor and critic observations of different widths (the
    trainer's f_obs [265 x n] and f_cobs [64 x n] shapes scaled down) against
    the same update on batch-major copies."""
    ad, cd = [45, 64, 32, 6], [17, 96, 32, 1]
    g = np.random.default_rng(3)
    actor = synth.kaiming_uniform_net(g, ad, 0.05)
    critic = synth.kaiming_uniform_net(g, cd, 0.05)
    n = 3000
    batch = dict(obs=synth.obs(g, n, 45), critic_obs=synth.obs(g, n, 17),
                 action=synth.normal(g, (n, 6)), mean_old=synth.normal(g, (n, 6)),
                 logp_old=synth.normal(g, n, 3.0) - 8.0, value_old=synth.normal(g, n),
                 adv=synth.normal(g, n), ret=synth.normal(g, n))
    log_std = np.full(6, -0.5, np.float32)
    outs = []
    for fm in (False, True):
        gac = GpuActorCritic(ctx, ad, cd, n // 3)
        gac.set_params(actor, critic, log_std, 1e-3)
        db = _batch(ctx, batch, fm)
        st = gac.update(db, PpoConfig.gpu_trainer(epochs=2, minibatches=3, desired_kl=100.0))
        outs.append((gac.get_params(), st))
        gac.close()
    for x, y in zip(outs[0][0][:3], outs[1][0][:3]):
        assert np.array_equal(x, y)
    assert outs[0][1] == outs[1][1]


def test_minibatch_grads_feature_major_with_perm(ctx):
    """zl_ppo_minibatch_grads on a feature-major batch, rows gathered through a
    device permutation: identical to the batch-major call, and to the oracle."""
    actor, critic, log_std, batch = _small_problem(29, n=3000)
    perm = np.random.default_rng(2).permutation(3000).astype(np.int32)
    gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, 1500)
    gac.set_params(actor, critic, log_std, 1e-3)
    dperm = ctx.to_device(perm)
    res = []
    for fm, pad in ((False, 0), (True, 0), (True, 53)):  # 53: [dim x (n + 53)] capacity stride
        db = _batch(ctx, batch, fm, pad)
        res.append(gac.minibatch_grads(db, PpoConfig(entropy_coef=0.01), 700, 1500, perm=dperm))
    for r in res[1:]:
        for x, y in zip(res[0][:3], r[:3]):
            assert np.array_equal(x, y)
        assert res[0][3] == r[3]
    idx = perm[700:2200]
    ra, rc, rl, rst = zo.minibatch_grads(SMALL_A, SMALL_C, actor, critic, log_std, batch, idx, 0.2, 0.01, 1.0)
    assert rel_amax(res[0][0], ra) <= 1e-4 and rel_amax(res[0][1], rc) <= 1e-4
    gac.close()


def test_update_new_buffers_without_recapture(ctx):
    """The reference re-stages the batch into fresh device tensors every
    iteration (src/bin/biped_train_gpu.rs:1029-1068). Updates from the same
    state on three different sets of buffers with the same contents give
    bit-identical results, the update graph is captured once, and each
    caller's adv buffer receives the normalised advantages."""
    actor, critic, log_std, batch = _well_posed_problem(7, n=4096)
    gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, 1024)
    cfg = PpoConfig.gpu_trainer(epochs=2, minibatches=4, clip=WELL_POSED_CLIP, desired_kl=100.0,
                                normalize_adv=True)
    outs, dbs = [], []
    for _ in range(3):
        gac.set_params(actor, critic, log_std, 1e-3)
        gac.reset_optimizer()
        db = _batch(ctx, batch, False)
        dbs.append(db)  # keep earlier buffers alive: the next batch gets new addresses
        st = gac.update(db, cfg)
        outs.append((gac.get_params(), st, db.adv.numpy()))
    captures, ms = gac.graph_info()
    print(f"[gpu] new-buffer updates: {captures} capture(s), last capture + instantiate {ms:.2f} ms", flush=True)
    assert captures == 1
    assert len({db.obs.ptr for db in dbs}) == 3
    for o in outs[1:]:
        for x, y in zip(o[0][:3], outs[0][0][:3]):
            assert np.array_equal(x, y)
        assert o[1] == outs[0][1]
        assert np.array_equal(o[2], outs[0][2])
    assert np.allclose(outs[0][2], zo.adv_normalize(batch["adv"]), rtol=1e-5, atol=1e-6)
    # A changed shape re-captures; going back to the first shape re-captures again.
    half = {k: v[:2048] for k, v in batch.items()}
    gac.update(_batch(ctx, half, False), cfg)
    assert gac.graph_info()[0] == 2
    gac.close()


def test_update_graph_survives_buffer_growth(ctx):
    """A buffer the captured update uses is reallocated by another entry point
    (a full-capacity minibatch_grads re-lays the split-K partial buffer the
    update's graph reads): the next update must not replay a graph that
    points at freed memory. It re-captures and matches the eager (timed)
    update bit for bit. The rollout step run in between (one zk_policy launch
    at 2048 rows) grows nothing; it checks that such a call leaves the update
    unchanged."""
    actor, critic, log_std, batch = _small_problem(31, n=2048)
    gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, 2048)
    cfg = PpoConfig(epochs=1, minibatches=4)

    def upd():
        gac.set_params(actor, critic, log_std, 1e-3)
        gac.reset_optimizer()
        gac.update(_batch(ctx, batch, False), cfg)
        return gac.get_params()

    first = upd()
    n0 = gac.graph_info()[0]
    # Grow other buffers of the handle: a 2048-row rollout step with both
    # normalisers, and a full-capacity minibatch_grads.
    from zealot_amd.rl import GpuNormalizer
    obs = ctx.to_device(batch["obs"])
    eps = ctx.to_device(np.zeros((2048, SMALL_A[-1]), np.float32))
    act, lp, val = ctx.alloc((2048, SMALL_A[-1])), ctx.alloc(2048), ctx.alloc(2048)
    norm = GpuNormalizer(ctx, SMALL_A[0])
    gac.act(obs, 2048, eps, act, lp, value=val, critic_obs=obs, obs_norm=norm, critic_norm=norm)
    gac.minibatch_grads(_batch(ctx, batch, False), PpoConfig(), 0, 2048)
    second = upd()
    assert gac.graph_info()[0] == n0 + 1
    ctx.check(ctx.lib.zl_timing_begin(ctx.h, b"zk_head"), "timing_begin")
    eager = upd()
    ctx.check(ctx.lib.zl_timing_end(ctx.h, None, None, None), "timing_end")
    for x, y, z in zip(first[:3], second[:3], eager[:3]):
        assert np.array_equal(x, y) and np.array_equal(x, z)
    gac.close()


def _grad_tensors(ad, cd, A):
    """Sizes of the trainer's gradient tensors in its norm order: actor dw[l],
    actor db[l], critic dw[l], critic db[l], dls (src/bin/biped_train_gpu.rs:1377-1397)."""
    sizes = []
    for dims in (ad, cd):
        sizes += [dims[l + 1] * dims[l] for l in range(len(dims) - 1)]
        sizes += [dims[l + 1] for l in range(len(dims) - 1)]
    return sizes + [A]


def test_config3_device_clip_and_adam_multi(ctx):
    """Config 3 as stated: Adam over actor + critic + log_std (459,323 params in
    the trainer's 17 tensors), gradients ~ N(0, 1e-2), 10 warm steps then one
    more, each with the global grad-norm clip at 1.0 computed on the device
    (zl_grad_clip_scale) and applied inside zl_adam_multi. The norm is ~6.8,
    so the clip is active every step. The norm matches float64, the scale is
    max / norm, and the parameters / moments match the oracle's Adam on the
    same scaled gradients within 2 ulp."""
    na, nc = packed_count(synth.ACTOR_DIMS), packed_count(synth.CRITIC_DIMS)
    c3 = synth.config3(na, nc)
    sizes = _grad_tensors(synth.ACTOR_DIMS, synth.CRITIC_DIMS, 29)
    n = sum(sizes)
    assert n == 459_323
    p0 = np.concatenate([c3["actor"], c3["critic"], c3["log_std"]]).astype(np.float32)
    dp, dm, dv = ctx.to_device(p0), ctx.to_device(np.zeros(n, np.float32)), ctx.to_device(np.zeros(n, np.float32))
    dg = ctx.alloc(n)
    scale, norm = ctx.alloc(1), ctx.alloc(1)
    offs = np.concatenate([[0], np.cumsum(sizes)])
    gt = [(dg.offset(int(o)), int(s)) for o, s in zip(offs[:-1], sizes)]
    at = [(dp.offset(int(o)), dg.offset(int(o)), dm.offset(int(o)), dv.offset(int(o)), int(s))
          for o, s in zip(offs[:-1], sizes)]
    hp, hm, hv = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    worst = 0.0
    for t, gr in enumerate(c3["grads"], start=1):
        bc1 = float(np.float32(1.0) - np.float32(zo.powi(0.9, t)))
        bc2 = float(np.float32(1.0) - np.float32(zo.powi(0.999, t)))
        dg.upload(gr)
        ops.grad_clip_scale(ctx, gt, 1.0, scale, norm)
        ops.adam_multi(ctx, at, 1e-3, bc1, bc2, clip_scale=scale)
        s_gpu, n_gpu = np.float32(scale.numpy()[0]), float(norm.numpy()[0])
        n64 = float(np.sqrt(np.sum(gr.astype(np.float64) ** 2)))
        worst = max(worst, abs(n_gpu - n64) / n64)
        assert n64 > 5.0  # clip active
        assert s_gpu == np.float32(1.0) / np.float32(n_gpu)
        hp, hm, hv = zo.adam_flat(hp, (gr * s_gpu).astype(np.float32), hm, hv, 1e-3, bc1, bc2)
    up, um, uv = ulp_diff(dp.numpy(), hp), ulp_diff(dm.numpy(), hm), ulp_diff(dv.numpy(), hv)
    print(f"[gpu] config3 clip+adam: norm rel err vs f64 {worst:.2e}; max ulp p={up} m={um} v={uv}", flush=True)
    assert worst < 1e-5
    assert up <= 2 and um <= 2 and uv <= 2


def test_config3_adam_multi_clip_two_launches(ctx):
    """zl_adam_multi_clip (the clipped step in two launches: sums of squares,
    then Adam blocks that each take the scale) against zl_grad_clip_scale +
    zl_adam_multi over the same 11 steps of config 3: parameters, moments,
    scale and norm bit-identical; plus a step with the clip inactive and one
    with it disabled."""
    na, nc = packed_count(synth.ACTOR_DIMS), packed_count(synth.CRITIC_DIMS)
    c3 = synth.config3(na, nc)
    sizes = _grad_tensors(synth.ACTOR_DIMS, synth.CRITIC_DIMS, 29)
    n = sum(sizes)
    p0 = np.concatenate([c3["actor"], c3["critic"], c3["log_std"]]).astype(np.float32)
    offs = np.concatenate([[0], np.cumsum(sizes)])
    runs = []
    for fused in (False, True):
        dp, dm, dv = ctx.to_device(p0), ctx.to_device(np.zeros(n, np.float32)), ctx.to_device(np.zeros(n, np.float32))
        dg = ctx.alloc(n)
        scale, norm = ctx.alloc(1), ctx.alloc(1)
        gt = [(dg.offset(int(o)), int(s)) for o, s in zip(offs[:-1], sizes)]
        at = [(dp.offset(int(o)), dg.offset(int(o)), dm.offset(int(o)), dv.offset(int(o)), int(s))
              for o, s in zip(offs[:-1], sizes)]
        trace = []
        grads = list(c3["grads"]) + [c3["grads"][0] * np.float32(1e-3), c3["grads"][1]]
        for t, gr in enumerate(grads, start=1):
            bc1 = float(np.float32(1.0) - np.float32(zo.powi(0.9, t)))
            bc2 = float(np.float32(1.0) - np.float32(zo.powi(0.999, t)))
            mx = 0.0 if t == len(grads) else 1.0
            dg.upload(gr)
            if fused:
                ops.adam_multi_clip(ctx, at, 1e-3, bc1, bc2, mx, scale, norm)
            else:
                ops.grad_clip_scale(ctx, gt, mx, scale, norm)
                ops.adam_multi(ctx, at, 1e-3, bc1, bc2, clip_scale=scale)
            trace.append((scale.numpy()[0], norm.numpy()[0]))
        runs.append((dp.numpy(), dm.numpy(), dv.numpy(), trace))
    for x, y in zip(runs[0][:3], runs[1][:3]):
        assert np.array_equal(x, y)
    assert runs[0][3] == runs[1][3]
    sc = [s for s, _ in runs[1][3]]
    assert all(s < 1.0 for s in sc[:11]) and sc[11] == 1.0 and sc[12] == 1.0


def test_clip_scale_inactive_and_disabled(ctx):
    """Below the threshold, or with max_norm <= 0, the scale is exactly 1."""
    g = (np.random.default_rng(4).standard_normal(5000) * 1e-3).astype(np.float32)
    d = ctx.to_device(g)
    scale, norm = ctx.alloc(1), ctx.alloc(1)
    for mx in (1.0, 0.0):
        ops.grad_clip_scale(ctx, [(d, 3000), (d.offset(3000), 2000)], mx, scale, norm)
        assert scale.numpy()[0] == 1.0
    assert abs(norm.numpy()[0] - np.sqrt(np.sum(g.astype(np.float64) ** 2))) < 1e-6


def _loss_case(rows, A, seed, clip=0.2):
    """Per-row loss inputs with every row kept clear of the clip and value-
    clamp branch boundaries (a row within rounding of a boundary may take
    either branch in any valid fp32 evaluation)."""
    g = np.random.default_rng(seed)
    mean = g.standard_normal((rows, A)).astype(np.float32)
    action = (mean + 0.6 * g.standard_normal((rows, A))).astype(np.float32)
    log_std = (np.full(A, -0.5) + 0.1 * g.standard_normal(A)).astype(np.float32)
    adv = g.standard_normal(rows).astype(np.float32)
    lp = np.sum(-0.5 * ((action.astype(np.float64) - mean) / np.exp(log_std.astype(np.float64))) ** 2
                - log_std - np_ref.LOG_SQRT_2PI, axis=1)
    logr = 0.3 * g.standard_normal(rows)
    for b in (np.log1p(clip), np.log1p(-clip)):
        logr = np.where(np.abs(logr - b) < 2e-2, logr + np.where(logr >= b, 4e-2, -4e-2), logr)
    logp_old = (lp - logr).astype(np.float32)
    mean_old = (mean + 0.05 * g.standard_normal((rows, A))).astype(np.float32)
    v = g.standard_normal(rows).astype(np.float32)
    vold = (v + 0.3 * g.standard_normal(rows)).astype(np.float32)
    ret = g.standard_normal(rows).astype(np.float32)
    v64, vo64, R = v.astype(np.float64), vold.astype(np.float64), ret.astype(np.float64)
    vc = vo64 + np.clip(v64 - vo64, -clip, clip)
    tie = np.abs((vc - R) ** 2 - (v64 - R) ** 2) < 1e-2 * np.maximum((vc - R) ** 2, 1e-3)
    ret = np.where(tie & (np.abs(vc - v64) > 1e-6), R + 0.05, R).astype(np.float32)
    return dict(mean=mean, action=action, log_std=log_std, adv=adv, logp_old=logp_old,
                mean_old=mean_old, v=v, vold=vold, ret=ret)


def _loss_truth(c, clip, ent, vcoef, s):
    """Per-sample float64 gradients of zealot-rl/src/ppo.rs:411-450."""
    ls = c["log_std"].astype(np.float64)
    d = c["action"].astype(np.float64) - c["mean"]
    lp = np.sum(-0.5 * (d / np.exp(ls)) ** 2 - ls - np_ref.LOG_SQRT_2PI, axis=1)
    ratio = np.exp(lp - c["logp_old"])
    A = c["adv"].astype(np.float64)
    clipped = ((A >= 0) & (ratio > 1 + clip)) | ((A < 0) & (ratio < 1 - clip))
    inv_var = np.exp(-2 * ls)
    gm = np.where(clipped[:, None], 0.0, -(A * ratio)[:, None] * d * inv_var * s)
    dls = np.where(clipped[:, None], 0.0, (A * ratio)[:, None] * (d * d * inv_var - 1.0))
    gls = (-dls * s).sum(0) - ent * s * len(A)
    v, vo, R = c["v"].astype(np.float64), c["vold"].astype(np.float64), c["ret"].astype(np.float64)
    vc = vo + np.clip(v - vo, -clip, clip)
    use_c = (vc - R) ** 2 > (v - R) ** 2
    dv = vcoef * np.where(use_c, 2 * (vc - R), 2 * (v - R)) * s
    return gm, gls, dv, clipped, use_c


@pytest.mark.parametrize("A", [29, 12, 40])
def test_loss_operators_per_row(ctx, A):
    """zl_ppo_actor_grad's d_mean [rows x A] and zl_ppo_value_grad's d_v [rows]
    element by element against the per-sample float64 gradients, with clipped
    surrogate rows and value-clamp rows present; the same call on the
    feature-major [A x rows] tensors (stride rows + 5) is bit-identical."""
    rows, clip, ent = 1777, 0.2, 0.005
    c = _loss_case(rows, A, seed=A)
    s = 1.0 / rows
    gm, gls, dv, clipped, use_c = _loss_truth(c, clip, ent, 1.0, s)
    assert clipped.sum() > rows // 20 and (~clipped).sum() > rows // 2
    assert use_c.sum() > rows // 20
    d = {k: ctx.to_device(c[k]) for k in ("mean", "action", "log_std", "adv", "logp_old", "mean_old")}
    dm, dls, st = ctx.alloc((rows, A)), ctx.alloc(A), ctx.alloc(2)
    ops.ppo_actor_grad(ctx, d["mean"], d["action"], d["log_std"], d["adv"], d["logp_old"], d["mean_old"],
                       rows, A, clip, ent, s, dm, dls, st)
    got = dm.numpy()
    scale = np.max(np.abs(gm))
    err = np.max(np.abs(got - gm)) / scale
    print(f"[gpu] actor_grad A={A}: d_mean max err {err:.2e} of max |d_mean|; "
          f"{int(clipped.sum())} clipped rows", flush=True)
    assert err <= 1e-4
    assert np.all(got[clipped] == 0.0)
    assert rel_amax(dls.numpy(), gls) <= 1e-4
    # Feature-major operands with a padded stride.
    ld = rows + 5

    def fm(x):
        out = np.zeros((A, ld), np.float32)
        out[:, :rows] = x.T
        return ctx.to_device(out)

    dmf, dlsf, stf = ctx.alloc((A, ld)), ctx.alloc(A), ctx.alloc(2)
    ops.ppo_actor_grad(ctx, fm(c["mean"]), fm(c["action"]), d["log_std"], d["adv"], d["logp_old"],
                       fm(c["mean_old"]), rows, A, clip, ent, s, dmf, dlsf, stf, ld_mean=ld,
                       ld_action=ld, ld_d_mean=ld, ld_mean_old=ld, feature_major=True)
    assert np.array_equal(dmf.numpy()[:, :rows].T, got)
    assert np.array_equal(dlsf.numpy(), dls.numpy()) and np.array_equal(stf.numpy(), st.numpy())
    # Critic half.
    dvv, vst = ctx.alloc(rows), ctx.alloc(1)
    ops.ppo_value_grad(ctx, ctx.to_device(c["v"]), ctx.to_device(c["vold"]), ctx.to_device(c["ret"]), rows,
                       clip, 1.0, s, dvv, vst)
    assert np.max(np.abs(dvv.numpy() - dv)) <= 1e-5 * np.max(np.abs(dv))


def test_sample_actions_logp_vs_oracle(ctx):
    """zl_sample_actions: action = mean + exp(log_std) * eps to one rounding,
    and logp against the oracle's ActorCritic::logp (ppo.rs:297-305) row by
    row."""
    rows, A = 1024, 29
    g = np.random.default_rng(9)
    means = g.standard_normal((rows, A)).astype(np.float32)
    eps = g.standard_normal((rows, A)).astype(np.float32)
    ac = zo.ActorCritic([4, 8, A], [4, 8, 1], 0.6, 1e-3, 5)
    _, _, log_std, _, _ = ac.get()
    act, lp = ctx.alloc((rows, A)), ctx.alloc(rows)
    ops.sample_actions(ctx, ctx.to_device(means), ctx.to_device(log_std), ctx.to_device(eps), rows, A, act, lp)
    ga, gl = act.numpy(), lp.numpy()
    ref_a = (means + np.exp(log_std).astype(np.float32) * eps).astype(np.float32)
    assert rel_amax(ga, ref_a) <= 1e-6
    ref_lp = np.array([ac.logp(ga[i], means[i]) for i in range(rows)], np.float32)
    assert rel_amax(gl, ref_lp) <= 1e-6
