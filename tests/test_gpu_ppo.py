"""GPU parity of the composed PPO path: one minibatch's gradients at the
24,576-row configuration, and whole updates under both reference semantics
(ActorCritic::update, zealot-rl/src/ppo.rs:338-510; the GPU trainer,
src/bin/biped_train_gpu.rs:1164-1553) against the CPU oracle.

Gradients are compared per tensor at 1e-4 of the tensor's max |value|, with
a float64 numpy restatement as the truth leg. Whole updates compare the
parameter change per component on a batch where a 20-step update is
well-conditioned in fp32 (Adam's first steps are ~lr * sign(g), so the test
still allows < 1 % of components to differ by more than 1 % of lr), and the
clip-0.2 regime, which is chaotic under any valid change of summation order,
by the quantities that stay well-posed there."""

import os

import numpy as np
import pytest

import np_ref
from conftest import rel_amax
from oracle import zl_oracle as zo
from zealot_amd import Context, ZealotError, synth
from zealot_amd.rl import DeviceBatch, GpuActorCritic, PpoConfig

pytestmark = pytest.mark.gpu

TOL = 1e-4
NTHREADS = min(os.cpu_count() or 1, 16)  # at most 16 host threads per GPU


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


@pytest.mark.parametrize("hidden,n,start,mb", [(64, 5000, 1000, 1500), (24, 5000, 1000, 1500),
                                                (512, 20000, 3000, 13001)])
def test_minibatch_grads_with_perm(ctx, hidden, n, start, mb):
    """Row gather through a device permutation (the shuffled minibatch); a
    24-wide first layer sends the gathered rows through the narrow kernels,
    a 512-wide one over 13,001 rows through ragged multi-wave tile grids."""
    ad, cd = [37, hidden, 48, 7], [37, hidden, 48, 1]
    g = np.random.default_rng(8)
    actor = synth.kaiming_uniform_net(g, ad, 0.1)
    critic = synth.kaiming_uniform_net(g, cd, 0.1)
    batch, log_std = make_batch(n, ad, cd, actor, critic, seed=99)
    move_off_branch_boundaries(batch, ad, cd, actor, critic, log_std)
    perm = g.permutation(n).astype(np.int32)
    gac = GpuActorCritic(ctx, ad, cd, mb)
    gac.set_params(actor, critic, log_std, 1e-3)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    ga, gc, gl, st = gac.minibatch_grads(db, PpoConfig(entropy_coef=0.01), start, mb,
                                         perm=ctx.to_device(perm))
    idx = perm[start:start + mb]
    ra, rc, rl, rst = zo.minibatch_grads(ad, cd, actor, critic, log_std, batch, idx, 0.2, 0.01, 1.0)
    assert per_tensor_err(ad, ga, ra) <= TOL and per_tensor_err(cd, gc, rc) <= TOL
    # The log_std gradient is a sum over rows with cancellation: over 13,001
    # rows the oracle's sequential fp32 sum is itself 1.6e-4 off the float64
    # truth (the GPU 1.8e-5), so that leg is judged against the truth.
    _, _, tl, _ = np_ref.minibatch_grads(ad, cd, actor, critic, log_std, batch, idx, 0.2, 0.01, 1.0)
    e_gpu, e_cpu = rel_amax(gl, tl), rel_amax(rl, tl)
    print(f"[gpu] perm grads hidden {hidden} x {mb}: log_std gpu vs f64 {e_gpu:.2e}, oracle vs f64 {e_cpu:.2e}",
          flush=True)
    assert e_gpu <= TOL


@pytest.mark.parametrize("ad,cd", [([37, 64, 160, 40], [37, 64, 160, 1]),   # H > 128, A > 32
                                   ([37, 96, 30, 3], [37, 96, 30, 1]),       # H = 30: padded tile
                                   ([37, 64, 128, 48], [37, 64, 128, 1]),    # the largest action dim
                                   ([37, 64, 128, 32], [37, 64, 128, 1])])   # the fused head's largest
def test_minibatch_grads_head_variants(ctx, ad, cd):
    """Output layers outside the fused head kernel's range (last hidden width
    > 128 or more than 32 actions: separate head GEMMs and loss kernels) and
    inside it with a hidden width that is not a multiple of 16."""
    g = np.random.default_rng(17)
    actor = synth.kaiming_uniform_net(g, ad, 0.1)
    critic = synth.kaiming_uniform_net(g, cd, 0.1)
    n = 3000
    batch, log_std = make_batch(n, ad, cd, actor, critic, seed=5)
    move_off_branch_boundaries(batch, ad, cd, actor, critic, log_std)
    gac = GpuActorCritic(ctx, ad, cd, n)
    gac.set_params(actor, critic, log_std, 1e-3)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    ga, gc, gl, st = gac.minibatch_grads(db, PpoConfig(entropy_coef=0.01), 0, n)
    idx = np.arange(n)
    ra, rc, rl, rst = zo.minibatch_grads(ad, cd, actor, critic, log_std, batch, idx, 0.2, 0.01, 1.0)
    _, _, tl, _ = np_ref.minibatch_grads(ad, cd, actor, critic, log_std, batch, idx, 0.2, 0.01, 1.0)
    e = (per_tensor_err(ad, ga, ra), per_tensor_err(cd, gc, rc), rel_amax(gl, tl))
    print(f"[gpu] head variant {ad} / {cd}: actor {e[0]:.2e} critic {e[1]:.2e} log_std {e[2]:.2e}", flush=True)
    assert max(e) <= TOL
    assert abs(st["surrogate"] - rst[0]) <= 1e-4 * max(1, abs(rst[0]))
    assert abs(st["value_loss"] - rst[1]) <= 1e-4 * max(1, abs(rst[1]))
    gac.close()


@pytest.mark.parametrize("n,shuffled", [(3001, False), (24576, False), (33000, True), (40000, False)])
def test_head_tile_schedules_match_unfused(ctx, n, shuffled):
    """zk_head's tile schedules against the separate output-layer GEMMs and
    loss kernels (ZL_FUSED_HEAD=0) on the same minibatch: a ragged last tile
    (3,001 rows), one actor tile per block with three critic tiles per block
    (24,576), and two tiles per block for both nets (33,000 shuffled,
    40,000)."""
    ad, cd = [40, 256, 128, 12], [40, 256, 128, 1]
    g = np.random.default_rng(23)
    actor = synth.kaiming_uniform_net(g, ad, 0.1)
    critic = synth.kaiming_uniform_net(g, cd, 0.1)
    batch, log_std = make_batch(n, ad, cd, actor, critic, seed=9)
    move_off_branch_boundaries(batch, ad, cd, actor, critic, log_std)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    perm = ctx.to_device(g.permutation(n).astype(np.int32)) if shuffled else None
    out = []
    for fused in (True, False):
        if not fused:
            os.environ["ZL_FUSED_HEAD"] = "0"
        try:
            gac = GpuActorCritic(ctx, ad, cd, n)
        finally:
            os.environ.pop("ZL_FUSED_HEAD", None)
        gac.set_params(actor, critic, log_std, 1e-3)
        out.append(gac.minibatch_grads(db, PpoConfig(entropy_coef=0.01), 0, n, perm=perm))
        gac.close()
    (fa, fc, fl, fs), (ua, uc, ul, us) = out
    e = (per_tensor_err(ad, fa, ua), per_tensor_err(cd, fc, uc), rel_amax(fl, ul))
    print(f"[gpu] head schedules n={n} shuffled={shuffled}: fused vs unfused actor {e[0]:.2e} "
          f"critic {e[1]:.2e} log_std {e[2]:.2e}", flush=True)
    assert max(e) <= TOL
    for key in ("surrogate", "value_loss", "kl"):
        assert abs(fs[key] - us[key]) <= 1e-5 * max(1.0, abs(us[key])), key


@pytest.mark.parametrize("n,shuffled", [(3001, True), (24576, False), (24576, True)])
def test_head_forward_fused_matches_separate(ctx, n, shuffled):
    """zk_head_fwd (the last hidden layer's forward computed tile by tile
    inside the head launch) against that layer as a GEMM launch of its own
    before zk_head (ZL_FUSED_HEAD=1): a ragged 3,001-row minibatch takes the
    masked form, 24,576 rows the exact-fit one. Every activation is summed in
    the same order, so the actor's gradients and statistics are bit-identical;
    the critic's output-layer partials are grouped per block, and its tiles
    go one per block with the forward inside (three per block otherwise at
    24,576 rows), so its gradients agree to rounding (1e-6)."""
    ad, cd = [40, 256, 128, 12], [40, 256, 128, 1]
    g = np.random.default_rng(29)
    actor = synth.kaiming_uniform_net(g, ad, 0.1)
    critic = synth.kaiming_uniform_net(g, cd, 0.1)
    batch, log_std = make_batch(n, ad, cd, actor, critic, seed=4)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    perm = ctx.to_device(g.permutation(n).astype(np.int32)) if shuffled else None
    out = []
    for fused_fwd in (True, False):
        if not fused_fwd:
            os.environ["ZL_FUSED_HEAD"] = "1"
        try:
            gac = GpuActorCritic(ctx, ad, cd, n)
        finally:
            os.environ.pop("ZL_FUSED_HEAD", None)
        gac.set_params(actor, critic, log_std, 1e-3)
        out.append(gac.minibatch_grads(db, PpoConfig(entropy_coef=0.01), 0, n, perm=perm))
        gac.close()
    (fa, fc, fl, fs), (sa, sc, sl, ss) = out
    assert np.array_equal(fa, sa) and np.array_equal(fl, sl)
    for key in ("surrogate", "kl"):
        assert fs[key] == ss[key], key
    ec = per_tensor_err(cd, fc, sc)
    print(f"[gpu] head forward fused n={n} shuffled={shuffled}: actor bit-identical, critic {ec:.2e}",
          flush=True)
    assert ec <= 1e-6
    assert abs(fs["value_loss"] - ss["value_loss"]) <= 1e-6 * max(1.0, abs(ss["value_loss"]))


@pytest.mark.parametrize("shuffled", [False, True])
def test_backward_merged_matches_separate(ctx, shuffled):
    """A layer's weight- and data-gradient GEMMs as one zk_gemm_bwd_* launch
    against the same GEMMs as two launches (ZL_MERGED_BWD=0): the 512 -> 256
    layer takes the 128 x 128 weight-gradient form, the 256 -> 128 layer the
    64 x 128 one, and both runs are bit-identical — the minibatch gradients
    and a whole update (2 epochs x 2 minibatches of 3,072 rows)."""
    ad, cd = [64, 512, 256, 128, 12], [64, 512, 256, 128, 1]
    n = 6144
    g = np.random.default_rng(31)
    actor = synth.kaiming_uniform_net(g, ad, 0.1)
    critic = synth.kaiming_uniform_net(g, cd, 0.1)
    batch, log_std = make_batch(n, ad, cd, actor, critic, seed=12)
    order = g.permutation(n).astype(np.int32)
    out = []
    for merged in (True, False):
        # The switch is read when a context is created: the separate run
        # gets a context of its own.
        if not merged:
            os.environ["ZL_MERGED_BWD"] = "0"
        try:
            cx = ctx if merged else Context(0)
        finally:
            os.environ.pop("ZL_MERGED_BWD", None)
        # A fresh batch per run: the update normalises its advantages in place.
        db = DeviceBatch(cx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                         batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
        perm = cx.to_device(order) if shuffled else None
        gac = GpuActorCritic(cx, ad, cd, n)
        gac.set_params(actor, critic, log_std, 1e-3)
        grads = gac.minibatch_grads(db, PpoConfig(entropy_coef=0.01), 0, n, perm=perm)
        gac.update(db, PpoConfig(epochs=2, minibatches=2))
        out.append((grads, gac.get_params()))
        gac.close()
        del db, perm
        if not merged:
            cx.close()
    (gm, pm), (gs, ps) = out
    for x, y in zip(gm[:3], gs[:3]):
        assert np.array_equal(x, y)
    for key in ("surrogate", "value_loss", "kl"):
        assert gm[3][key] == gs[3][key], key
    for x, y in zip(pm[:3], ps[:3]):
        assert np.array_equal(x, y)
    print(f"[gpu] merged backward shuffled={shuffled}: gradients and update bit-identical", flush=True)


def test_action_dim_limit(ctx):
    """zl_ppo_create refuses more than 48 actions, its stated maximum (the
    48-action net above is accepted)."""
    with pytest.raises(ZealotError):
        GpuActorCritic(ctx, [37, 64, 49], [37, 64, 1], 256)


def _param_delta_report(p0, pg, pc, lr, steps):
    dg, dc = (pg - p0).astype(np.float64), (pc - p0).astype(np.float64)
    diff = np.abs(dg - dc)
    nc = np.linalg.norm(dc)
    return dict(max_abs=float(diff.max()), bound=2 * lr * steps, frac_gt_1pct_lr=float(np.mean(diff > 1e-2 * lr)),
                rel_l2=float(np.linalg.norm(dg - dc) / max(nc, 1e-30)),
                cos=float(dg @ dc / max(np.linalg.norm(dg) * nc, 1e-30)))


SMALL_A = [123, 128, 64, 29]
SMALL_C = [123, 128, 64, 1]


def _small_problem(seed, n=8192):
    """Config-4 style synthetic batch (actions ~ N(0,1), advantages ~ N(0,1),
    clip 0.2 in the tests that use it). Over a 20-step update this regime is
    chaotic in fp32: perturbing the observations by 1e-5 relative changes the
    oracle's own actor update by up to 25 % (relative L2, cosine >= 0.97) and
    its last-epoch KL / surrogate by up to 7 %, because samples keep crossing
    the clip boundary and the advantage carries no signal. The critic is
    unaffected (bit-identical under the same perturbation)."""
    g = np.random.default_rng(seed)
    actor = synth.kaiming_uniform_net(g, SMALL_A, 0.05)
    critic = synth.kaiming_uniform_net(g, SMALL_C, 0.05)
    batch, log_std = make_batch(n, SMALL_A, SMALL_C, actor, critic, seed + 1)
    move_off_branch_boundaries(batch, SMALL_A, SMALL_C, actor, critic, log_std)
    return actor, critic, log_std, batch


def _well_posed_problem(seed, n=8192, ad=None, cd=None):
    """A batch on which a whole 20-step update is well-conditioned in fp32:
    actions sampled from the policy (a = mean + std * eps), logp_old the exact
    log-prob, advantages half an action-correlated signal (eps . c / sqrt(A),
    c = +-1) and half N(0,1), used with clip 100 (no surrogate or value-clip
    branch is ever taken). Measured on the oracle: perturbing the observations
    by 1e-6 relative moves no parameter by more than 1 % of lr and the update
    by < 1e-4 relative L2."""
    ad = SMALL_A if ad is None else ad
    cd = SMALL_C if cd is None else cd
    g = np.random.default_rng(seed)
    actor = synth.kaiming_uniform_net(g, ad, 0.05)
    critic = synth.kaiming_uniform_net(g, cd, 0.05)
    obs = synth.obs(g, n, ad[0])
    means = f32_forward(ad, actor, obs)
    values = f32_forward(cd, critic, obs)
    A = ad[-1]
    log_std = np.full(A, -0.5, np.float32)
    eps = g.standard_normal((n, A)).astype(np.float32)
    action = (means + np.exp(log_std) * eps).astype(np.float32)
    c = np.where(g.random(A) < 0.5, -1.0, 1.0)
    adv = (0.5 * (eps @ c) / np.sqrt(A) + 0.5 * g.standard_normal(n)).astype(np.float32)
    batch = dict(obs=obs, critic_obs=obs, action=action, mean_old=means,
                 logp_old=synth.gaussian_logp(action, means, log_std),
                 value_old=(values[:, 0] + 0.05 * g.standard_normal(n)).astype(np.float32),
                 adv=adv, ret=g.standard_normal(n).astype(np.float32))
    return actor, critic, log_std, batch


WELL_POSED_CLIP = 100.0


def _assert_tight(reps):
    for name, rep in reps.items():
        assert rep["frac_gt_1pct_lr"] < 0.01 and rep["rel_l2"] < 1e-3, (name, rep)


# Adaptive-LR settings (adaptive, desired KL, lr_max) whose every decision has
# a wide margin: "up" (KL far below desired / 2: x1.5 per minibatch up to
# lr_max, kept at 2e-3 because larger steps make the update chaotic again),
# "down" (KL far above 2 * desired after the first step: /1.5 to lr_min).
LR_RULES = {"fixed": (False, 0.01, 1e-2), "up": (True, 100.0, 2e-3), "down": (True, 1e-9, 1e-2)}


@pytest.mark.parametrize("rule", list(LR_RULES))
def test_update_actor_critic_semantics(ctx, rule):
    """ActorCritic::update: per-epoch Fisher-Yates shuffle, per-net clip, per-step
    KL-adaptive LR, log_std Adam with clamp [-1.6, 1.0], on a well-conditioned
    batch (parameters compared per component)."""
    adaptive, desired, lr_max = LR_RULES[rule]
    actor, critic, log_std, batch = _well_posed_problem(41)
    lr0 = 1e-3
    ac = zo.ActorCritic(SMALL_A, SMALL_C, 1.0, lr0, 1)
    ac.set(actor, critic, log_std, lr0)
    cfg_o = zo.PpoCfg(0.99, 0.95, WELL_POSED_CLIP, 0.01, 1.0, 5, 4, 1.0, desired, 1e-5, lr_max, int(adaptive))
    stats_o, adv_o = ac.update(batch, cfg_o, nthreads=NTHREADS, normalize_obs=False)
    ao, co, lso, lro, to = ac.get()

    gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, batch["obs"].shape[0] // 4)
    gac.set_params(actor, critic, log_std, lr0)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    st = gac.update(db, PpoConfig(epochs=5, minibatches=4, clip=WELL_POSED_CLIP, adaptive_lr=adaptive,
                                  desired_kl=desired, lr_max=lr_max, shuffle=True, normalize_adv=True,
                                  clamp_log_std=True))
    ag, cg, lsg, lrg = gac.get_params()
    t, _ = gac.counters()
    reps = dict(actor=_param_delta_report(actor, ag, ao, lr0, 20),
                critic=_param_delta_report(critic, cg, co, lr0, 20),
                log_std=_param_delta_report(log_std, lsg, lso, lr0, 20))
    print(f"[gpu] AC update lr rule {rule}: {reps} lr {lrg} vs {lro} stats gpu {st} cpu {stats_o}", flush=True)
    assert t == to == 20
    assert np.allclose(db.adv.numpy(), adv_o, rtol=1e-5, atol=1e-6)
    assert lrg == pytest.approx(lro, rel=1e-6)
    if rule == "up":
        assert lro == pytest.approx(lr_max)
    if rule == "down":
        assert lro < lr0 / 1.5 ** 10
    _assert_tight(reps)
    for k, gv in zip(("kl", "surrogate", "value_loss", "entropy"), (st.kl, st.surrogate, st.value_loss, st.entropy)):
        ov = stats_o[["kl", "surrogate", "value_loss", "entropy"].index(k)]
        assert abs(gv - ov) <= 1e-3 * max(abs(ov), 1e-2), (k, gv, ov)
    gac.close()


def test_update_actor_critic_consecutive(ctx):
    """Three ActorCritic::update calls in a row: the second takes the shuffle
    orders prepared while the first ran (its Adam step count is known), the
    third changes the minibatch count, so the prepared orders no longer match
    and are computed again. Parameters, lr and step counts against three
    oracle updates."""
    actor, critic, log_std, batch = _well_posed_problem(43)
    lr0 = 1e-3
    ac = zo.ActorCritic(SMALL_A, SMALL_C, 1.0, lr0, 1)
    ac.set(actor, critic, log_std, lr0)
    n = batch["obs"].shape[0]
    gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, n // 4)
    gac.set_params(actor, critic, log_std, lr0)
    for k, mbs in enumerate((4, 4, 8)):
        cfg_o = zo.PpoCfg(0.99, 0.95, WELL_POSED_CLIP, 0.01, 1.0, 2, mbs, 1.0, 0.01, 1e-5, 1e-2, 0)
        ac.update({key: v.copy() for key, v in batch.items()}, cfg_o, nthreads=NTHREADS,
                  normalize_obs=False)
        db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                         batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
        gac.update(db, PpoConfig(epochs=2, minibatches=mbs, clip=WELL_POSED_CLIP, adaptive_lr=False,
                                 shuffle=True, normalize_adv=True, clamp_log_std=True))
    ao, co, lso, lro, to = ac.get()
    ag, cg, lsg, lrg = gac.get_params()
    t, _ = gac.counters()
    steps = 2 * (4 + 4 + 8)
    reps = dict(actor=_param_delta_report(actor, ag, ao, lr0, steps),
                critic=_param_delta_report(critic, cg, co, lr0, steps),
                log_std=_param_delta_report(log_std, lsg, lso, lr0, steps))
    print(f"[gpu] AC consecutive updates: {reps}", flush=True)
    assert t == to == steps
    assert lrg == pytest.approx(lro, rel=1e-6)
    _assert_tight(reps)
    gac.close()


def test_update_actor_critic_full_size(ctx):
    """ActorCritic::update at the headline shapes: 98,304 rows, 5 epochs x 4
    shuffled minibatches of 24,576 rows (the observation gather fused into the
    first layer's loads and the first weight gradient), per-net clip, log_std
    Adam with clamp, on the well-posed construction at lr 1e-5 (see
    test_update_config5_full_size)."""
    ad, cd = synth.ACTOR_DIMS, synth.CRITIC_DIMS
    n, lr0 = 98304, 1e-5
    actor, critic, log_std, batch = _well_posed_problem(43, n, ad, cd)
    ac = zo.ActorCritic(ad, cd, 1.0, lr0, 1)
    ac.set(actor, critic, log_std, lr0)
    cfg_o = zo.PpoCfg(0.99, 0.95, WELL_POSED_CLIP, 0.01, 1.0, 5, 4, 1.0, 0.01, 1e-6, 1e-2, 0)
    stats_o, adv_o = ac.update(batch, cfg_o, nthreads=NTHREADS, normalize_obs=False)
    ao, co, lso, lro, to = ac.get()

    gac = GpuActorCritic(ctx, ad, cd, n // 4)
    gac.set_params(actor, critic, log_std, lr0)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    st = gac.update(db, PpoConfig(epochs=5, minibatches=4, clip=WELL_POSED_CLIP, adaptive_lr=False,
                                  desired_kl=0.01, lr_min=1e-6, lr_max=1e-2, shuffle=True,
                                  normalize_adv=True, clamp_log_std=True))
    ag, cg, lsg, lrg = gac.get_params()
    t, _ = gac.counters()
    reps = dict(actor=_param_delta_report(actor, ag, ao, lr0, 20),
                critic=_param_delta_report(critic, cg, co, lr0, 20),
                log_std=_param_delta_report(log_std, lsg, lso, lr0, 20))
    print(f"[gpu] AC update full size: {reps} stats gpu {st} cpu {stats_o}", flush=True)
    assert t == to == 20 and lrg == pytest.approx(lro, rel=1e-6)
    assert np.allclose(db.adv.numpy(), adv_o, rtol=1e-5, atol=1e-6)
    _assert_tight(reps)
    for k, gv in zip(("kl", "surrogate", "value_loss", "entropy"), (st.kl, st.surrogate, st.value_loss, st.entropy)):
        ov = stats_o[["kl", "surrogate", "value_loss", "entropy"].index(k)]
        assert abs(gv - ov) <= 1e-3 * max(abs(ov), 1e-2), (k, gv, ov)
    gac.close()


def test_update_clipped_regime(ctx):
    """ActorCritic::update at clip 0.2 on config-4 style data, where the
    surrogate and value clips are taken throughout. The regime is chaotic in
    fp32 (see _small_problem), so the actor is checked by the direction of its
    update and the KL / surrogate statistics loosely; the critic, the learning
    rate, the Adam step count, the value loss and the entropy tightly."""
    actor, critic, log_std, batch = _small_problem(41)
    lr0 = 1e-3
    ac = zo.ActorCritic(SMALL_A, SMALL_C, 1.0, lr0, 1)
    ac.set(actor, critic, log_std, lr0)
    cfg_o = zo.PpoCfg(0.99, 0.95, 0.2, 0.01, 1.0, 5, 4, 1.0, 0.01, 1e-5, 1e-2, 0)
    stats_o, adv_o = ac.update(batch, cfg_o, nthreads=NTHREADS, normalize_obs=False)
    ao, co, lso, lro, to = ac.get()
    gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, batch["obs"].shape[0] // 4)
    gac.set_params(actor, critic, log_std, lr0)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    st = gac.update(db, PpoConfig(epochs=5, minibatches=4, adaptive_lr=False, shuffle=True,
                                  normalize_adv=True, clamp_log_std=True))
    ag, cg, lsg, lrg = gac.get_params()
    t, _ = gac.counters()
    ra = _param_delta_report(actor, ag, ao, lr0, 20)
    rc = _param_delta_report(critic, cg, co, lr0, 20)
    rl = _param_delta_report(log_std, lsg, lso, lr0, 20)
    print(f"[gpu] clipped-regime update: actor {ra} critic {rc} log_std {rl} stats gpu {st} cpu {stats_o}",
          flush=True)
    assert t == to == 20 and lrg == pytest.approx(lro, rel=1e-6)
    assert ra["max_abs"] <= ra["bound"] and ra["cos"] >= 0.9
    assert rl["cos"] >= 0.9
    _assert_tight(dict(critic=rc))
    assert abs(st.value_loss - stats_o[2]) <= 1e-3 * max(abs(stats_o[2]), 1e-2)
    assert abs(st.entropy - stats_o[3]) <= 1e-2 * max(abs(stats_o[3]), 1e-2)
    for gv, ov in ((st.kl, stats_o[0]), (st.surrogate, stats_o[1])):
        assert abs(gv - ov) <= 0.25 * max(abs(ov), 1e-2), (gv, ov)
    gac.close()


@pytest.mark.parametrize("early", [False, True])
def test_update_gpu_trainer_semantics(ctx, early):
    """GPU trainer update: contiguous minibatches, global clip (incl. log_std),
    per-epoch gstep bias correction, per-epoch full-Gaussian KL -> LR + early stop,
    log_std clamped to [-1.6, 0.0] after the update. Well-conditioned batch;
    desired KL far from the epoch KLs: early=False raises the LR every epoch
    (to lr_max = 2e-3), early=True stops after the first epoch (KL > 5 * desired)."""
    actor, critic, log_std, batch = _well_posed_problem(77)
    batch["adv"] = zo.adv_normalize(batch["adv"])
    lr0 = 1e-3
    tr = zo.Trainer(SMALL_A, SMALL_C, actor, critic, log_std, lr0)
    desired = 1e-9 if early else 100.0
    cfg_o = zo.TrainerCfg(WELL_POSED_CLIP, 0.01, 1.0, 5, 4, 1.0, desired, 1e-5, 2e-3, 1, int(early), 1)
    so = tr.update(batch, cfg_o, nthreads=NTHREADS)
    ao, co, lso, lro, gso = tr.get()

    gac = GpuActorCritic(ctx, SMALL_A, SMALL_C, batch["obs"].shape[0] // 4)
    gac.set_params(actor, critic, log_std, lr0)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    cfg = PpoConfig.gpu_trainer(epochs=5, minibatches=4, clip=WELL_POSED_CLIP, entropy_coef=0.01,
                                value_coef=1.0, max_grad_norm=1.0, desired_kl=desired, lr_max=2e-3,
                                early_stop=early, normalize_adv=False)
    st = gac.update(db, cfg)
    ag, cg, lsg, lrg = gac.get_params()
    _, gstep = gac.counters()
    steps = int(so[5]) * 4
    reps = dict(actor=_param_delta_report(actor, ag, ao, lr0, steps),
                critic=_param_delta_report(critic, cg, co, lr0, steps),
                log_std=_param_delta_report(log_std, lsg, lso, lr0, steps))
    print(f"[gpu] trainer update early={early}: epochs gpu {st.epochs_run} cpu {int(so[5])} "
          f"kl {st.last_kl:.4e} vs {so[6]:.4e} lr {lrg} vs {lro} {reps}", flush=True)
    assert st.epochs_run == int(so[5]) == (1 if early else 5)
    assert gstep == gso == 4 * st.epochs_run  # gstep += n_mb per epoch that ran (:1165)
    assert abs(st.last_kl - so[6]) <= 1e-3 * max(abs(so[6]), 1e-6)
    assert lrg == pytest.approx(lro, rel=1e-6)
    assert np.all(lsg <= 0.0) and np.all(lsg >= -1.6)
    _assert_tight(reps)
    gac.close()


def test_update_config5_full_size(ctx):
    """The headline workload's shapes at full size: actor 123-512-256-128-29 +
    critic 123-512-256-128-1, 98,304 rows, 5 epochs x 4 minibatches of 24,576
    rows with GPU-trainer semantics (global clip 1.0, fixed LR, log_std clamp),
    on the well-posed batch construction at lr 1e-5. At lr 1e-3 twenty full-size
    steps are chaotic in fp32 (on the oracle, a 1e-6 relative change of the
    observations moves the actor update by 33 % relative L2), so no two correct
    implementations agree there; at 1e-5 the same perturbation moves it by
    3e-5, and the GPU update must agree with the oracle's as in the small
    trainer tests."""
    ad, cd = synth.ACTOR_DIMS, synth.CRITIC_DIMS
    n, lr0 = 98304, 1e-5
    actor, critic, log_std, batch = _well_posed_problem(11, n, ad, cd)
    batch["adv"] = zo.adv_normalize(batch["adv"])
    tr = zo.Trainer(ad, cd, actor, critic, log_std, lr0)
    cfg_o = zo.TrainerCfg(WELL_POSED_CLIP, 0.005, 1.0, 5, 4, 1.0, 0.01, 1e-5, 1e-2, 0, 0, 1)
    so = tr.update(batch, cfg_o, nthreads=NTHREADS)
    ao, co, lso, lro, _ = tr.get()

    gac = GpuActorCritic(ctx, ad, cd, n // 4)
    gac.set_params(actor, critic, log_std, lr0)
    db = DeviceBatch(ctx, batch["obs"], batch["obs"], batch["action"], batch["mean_old"],
                     batch["logp_old"], batch["value_old"], batch["adv"], batch["ret"])
    cfg = PpoConfig.gpu_trainer(epochs=5, minibatches=4, clip=WELL_POSED_CLIP, entropy_coef=0.005,
                                value_coef=1.0, max_grad_norm=1.0, adaptive_lr=False, early_stop=False,
                                normalize_adv=False, clamp_log_std=True)
    st = gac.update(db, cfg)
    ag, cg, lsg, lrg = gac.get_params()
    reps = dict(actor=_param_delta_report(actor, ag, ao, lr0, 20),
                critic=_param_delta_report(critic, cg, co, lr0, 20),
                log_std=_param_delta_report(log_std, lsg, lso, lr0, 20))
    print(f"[gpu] config 5 full size: epochs {st.epochs_run} kl {st.last_kl:.6e} vs {so[6]:.6e} {reps}", flush=True)
    assert st.epochs_run == int(so[5]) == 5 and lrg == pytest.approx(lro, rel=1e-6)
    assert abs(st.last_kl - so[6]) <= 1e-3 * max(abs(so[6]), 1e-6)
    _assert_tight(reps)
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


@pytest.mark.parametrize("n", [4096, 3500, 2500, 1024, 1000])
def test_values_and_actor_mean(ctx, n):
    """Config 2 (actor inference over 4096 rows) and critic values. With
    1024-row buffers the critic's chunks run in pairs (the second in the
    actor's buffers): n = 3500 ends in a short pair, 2500 in a lone short
    chunk, 1024 and 1000 are a single chunk."""
    c2 = synth.config2()
    obs = c2["obs"][:n]
    critic = synth.kaiming_uniform_net(synth.rng(2, 1), synth.CRITIC_DIMS)
    gac = GpuActorCritic(ctx, synth.ACTOR_DIMS, synth.CRITIC_DIMS, 1024)
    gac.set_params(c2["actor"], critic, c2["log_std"], 1e-3)
    dobs = ctx.to_device(obs)
    mean = ctx.alloc((n, 29))
    vals = ctx.alloc(n)
    gac.actor_mean(dobs, n, mean)
    gac.values(dobs, n, vals)
    rm = zo.mlp_forward(synth.ACTOR_DIMS, c2["actor"], obs)[-1]
    rv = zo.mlp_forward(synth.CRITIC_DIMS, critic, obs)[-1][:, 0]
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
