"""Benchmark: one full PPO update on one MI355X (the path's headline workload).

A step is one pass of the learning path over one synthetic rollout of
4096 envs x 24 steps (98,304 samples), all buffers resident in HBM:
critic values over the rollout + bootstrap obs -> GAE (gamma 0.99, lambda 0.95)
-> advantage normalisation -> 5 epochs x 4 minibatches (24,576 rows) of
actor 123-512-256-128-29 + critic 123-512-256-128-1 forward, PPO losses,
backward, global grad-norm clip (1.0) and Adam (lr 1e-3). GPU-trainer
semantics (src/bin/biped_train_gpu.rs:1164-1553), fixed learning rate and no
KL early stop so every step does the same work.

Prints ONE JSON line. `value` = PPO-update samples/s = 5 * 98,304 / t_step
(sample-gradient evaluations per second). `self_check` reports the post-run
check of the trained state (finite values, critic values against a float64
forward, the first Adam moment of one more step against the minibatch
gradient); the process exits 1 when it fails. Unless --no-aux, `aux` adds the
workloads around the update: the 4096-env rollout step, the observation
normaliser, the single dense layer (4096 x 123 -> 512, ELU) and the clipped
Adam step over the 459,323 parameters, the reference trainer's own nets and
the update under ActorCritic::update semantics.
"""

from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

N_ENVS, T_STEPS = 4096, 24
EPOCHS, MINIBATCHES = 5, 4
FP32_MFMA_PEAK = 157.3e12  # MI355X dense fp32 matrix, FLOP/s
HBM_PEAK = 8.0e12  # bytes/s
# HBM bytes per launch of a kernel, measured with rocprofv3 --pmc FETCH_SIZE
# and WRITE_SIZE on this workload (one counter per run), scaled by the
# readings of a 256 MiB copy kernel (FETCH_SIZE x 2.0, WRITE_SIZE x 1.0) and
# averaged over an update's launch mix; reported as roofline.traffic for the
# dominant kernel when it is one of these.
MEASURED_TRAFFIC = {
    "zk_gemm_bwd_128x128_dg128_x": 441.1e6,
    "zk_gemm_ak_bk_128x128x32_w24_x": 150.3e6,
}


def cpu_baseline(ro, actor, critic, log_std, mean_old, action, logp_old, values, adv):
    """The oracle's restatement of the same update (GPU-trainer semantics) on
    the same rollout, timed on the host cores: 5 epochs x 4 minibatches of
    24,576 rows, actor + critic fwd + bwd + global clip + Adam."""
    from oracle import zl_oracle as zo
    from zealot_amd import synth

    n = ro["obs"].shape[0]
    threads = min(os.cpu_count() or 1, 16)
    batch = dict(obs=ro["obs"], critic_obs=ro["obs"], action=action, mean_old=mean_old,
                 logp_old=logp_old, value_old=values, adv=zo.adv_normalize(adv[0]), ret=adv[1])
    tr = zo.Trainer(synth.ACTOR_DIMS, synth.CRITIC_DIMS, actor, critic, log_std, 1e-3)
    cfg = zo.TrainerCfg(0.2, 0.005, 1.0, EPOCHS, MINIBATCHES, 1.0, 0.01, 1e-5, 1e-2, 0, 0, 1)
    t0 = time.perf_counter()
    tr.update(batch, cfg, nthreads=threads)
    dt = time.perf_counter() - t0
    return {"value": EPOCHS * n / dt, "unit": "samples/s", "cores": threads, "kind": "port",
            "sample": f"the same full update ({EPOCHS} epochs x {MINIBATCHES} minibatches of "
                      f"{n // MINIBATCHES} rows, fwd+bwd+clip+Adam, GPU-trainer semantics) on "
                      f"{threads} threads: {dt:.1f} s"}


def _np_forward(dims, packed, x):
    """float64 forward of a packed MLP (w[l] row-major [out x in], then b[l];
    hidden ELU, linear output: zealot-rl/src/net.rs:88-108)."""
    a, o = np.asarray(x, np.float64), 0
    for l in range(len(dims) - 1):
        out, inp = dims[l + 1], dims[l]
        w = packed[o:o + out * inp].reshape(out, inp).astype(np.float64)
        o += out * inp
        a = a @ w.T + packed[o:o + out].astype(np.float64)
        o += out
        if l < len(dims) - 2:
            a = np.where(a > 0, a, np.expm1(np.minimum(a, 0.0)))
    return a


def self_check(ctx, gac, obs, d_obs, ld, n, mb, batch_ptrs, stats):
    """Post-run check of the timed update, outside the timed region (the
    reference harness checks its result after the timed loop,
    src/bin/iter_e2e_bench.rs:815-829):
    * the trained parameters, the Adam moments and the update's statistics
      are finite;
    * critic values of 1,024 rows spread over the rollout against a float64
      forward of the trained critic: max |err| / max |v| <= 1e-4;
    * one more update of one minibatch (rows [0, mb), the normalised
      advantages the timed updates wrote back) from the trained parameters
      with fresh moments leaves Adam's first moment at (1 - beta1) * s * g,
      where g is zl_ppo_minibatch_grads' gradient of the same rows and s the
      global clip factor min(1, 1 / |g|): max |err| / max |m| <= 1e-4 for the
      actor, the critic and log_std.
    Leaves the handle's parameters one step further on."""
    from zealot_amd import synth
    from zealot_amd.rl import PpoConfig, _ffi

    ad, cd = gac.actor_dims, gac.critic_dims
    a, c, ls, lr = gac.get_params()
    mom = gac.get_moments()
    st = [stats.kl, stats.surrogate, stats.value_loss, stats.entropy, stats.lr, stats.last_kl]
    finite = bool(all(np.all(np.isfinite(x)) for x in (a, c, ls, *mom)) and np.all(np.isfinite(st)))
    rows = np.linspace(0, n - 1, 1024).astype(np.int64)
    d_v = ctx.alloc(n)
    gac.values(d_obs, n, d_v, ld=ld)
    v = d_v.numpy()[rows].astype(np.float64)
    v_ref = _np_forward(cd, c, obs[rows])[:, 0]
    err_v = float(np.max(np.abs(v - v_ref)) / max(np.max(np.abs(v_ref)), 1e-30))
    # One minibatch: its gradient, then one update step over the same rows.
    (obs_p, ld_obs, cobs_p, ld_cobs, act_p, ld_act, mean_p, ld_mean, logp_p, val_p, adv_p, ret_p) = batch_ptrs
    one = _ffi.zl_batch(mb, obs_p, ld_obs, cobs_p, ld_cobs, act_p, ld_act, mean_p, ld_mean, logp_p, val_p,
                        adv_p, ret_p)
    cfg = PpoConfig.gpu_trainer(epochs=1, minibatches=1, clip=0.2, entropy_coef=0.005, value_coef=1.0,
                                max_grad_norm=1.0, adaptive_lr=False, early_stop=False, normalize_adv=False,
                                clamp_log_std=False).to_c()
    st3 = (C.c_float * 3)()
    ctx.check(ctx.lib.zl_ppo_minibatch_grads(gac.h, C.byref(one), C.byref(cfg), 0, mb, None, st3), "grads")
    ga, gc, gl = np.empty(gac.na, np.float32), np.empty(gac.nc, np.float32), np.empty(len(ls), np.float32)
    ctx.check(ctx.lib.zl_ppo_get_grads(gac.h, ga.ctypes.data_as(C.c_void_p), gc.ctypes.data_as(C.c_void_p),
                                       gl.ctypes.data_as(C.c_void_p)), "get_grads")
    gac.reset_optimizer()
    out = _ffi.zl_ppo_stats()
    ctx.check(ctx.lib.zl_ppo_update(gac.h, C.byref(one), C.byref(cfg), C.byref(out)), "update")
    ma, _, mc, _, mls, _ = gac.get_moments()
    g = [x.astype(np.float64) for x in (ga, gc, gl)]
    norm = np.sqrt(sum(float(np.sum(x * x)) for x in g))
    s = min(1.0, 1.0 / norm) if norm > 0 else 1.0
    err_m = {}
    for name, m, gx in (("actor", ma, g[0]), ("critic", mc, g[1]), ("log_std", mls, g[2])):
        want = 0.1 * s * gx
        err_m[name] = float(np.max(np.abs(m - want)) / max(np.max(np.abs(want)), 1e-30))
    ok = finite and err_v <= 1e-4 and max(err_m.values()) <= 1e-4
    return {"pass": bool(ok), "finite": finite, "critic_values_rel_err": err_v,
            "first_step_moment_rel_err": err_m, "grad_norm": norm, "clip_scale": s}


def _timed(ctx, fn, reps):
    fn()
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        fn()
    ctx.synchronize()
    return (time.perf_counter() - t0) / reps


def aux_measurements(ctx, gac, ro, d_obs, ld, n):
    """The rows around the update: the on-device rollout step (GpuPolicy::
    forward + sampling for 4096 envs, the actor-inference configuration) and
    the observation normaliser over one rollout step and over the whole
    update batch. Wall time over repeated calls on the context stream."""
    from zealot_amd import synth
    from zealot_amd.rl import GpuNormalizer

    ad, cd = synth.ACTOR_DIMS, synth.CRITIC_DIMS
    od = ad[0]
    envs = N_ENVS
    obs_norm = GpuNormalizer(ctx, od)
    obs_norm.update(d_obs, n, ld)  # a non-trivial transform
    eps = ctx.to_device(ro["eps"][:envs])
    act, lp, mean, val = ctx.alloc((envs, ad[-1])), ctx.alloc(envs), ctx.alloc((envs, ad[-1])), ctx.alloc(envs)
    flop_actor = 2.0 * envs * sum(ad[l] * ad[l + 1] for l in range(len(ad) - 1))
    flop_critic = 2.0 * envs * sum(cd[l] * cd[l + 1] for l in range(len(cd) - 1))
    t_act = _timed(ctx, lambda: gac.act(d_obs, envs, eps, act, lp, ld_obs=ld, obs_norm=obs_norm), 50)
    t_act_v = _timed(ctx, lambda: gac.act(d_obs, envs, eps, act, lp, mean=mean, value=val, critic_obs=d_obs,
                                          obs_norm=obs_norm, critic_norm=obs_norm, ld_obs=ld,
                                          ld_critic_obs=ld), 50)
    staged = ctx.alloc((n, od))
    t_norm = _timed(ctx, lambda: obs_norm.normalize(d_obs, n, staged, ld_x=ld, ld_out=od), 20)
    scratch = GpuNormalizer(ctx, od)
    t_upd_step = _timed(ctx, lambda: scratch.update(d_obs, envs, ld), 50)
    t_upd_all = _timed(ctx, lambda: scratch.update(d_obs, n, ld), 20)
    norm_bytes = 2.0 * n * od * 4  # read x once, write out once
    return {
        "rollout_step": {
            "workload": f"{envs} envs: normalise obs [{envs}x{od}], actor {'-'.join(map(str, ad))}, "
                        f"sample a = mean + exp(log_std) * eps, logp",
            "us": t_act * 1e6, "envs_per_s": envs / t_act,
            "gemm_tflops": flop_actor / t_act / 1e12,
            "with_critic_value_us": t_act_v * 1e6,
            "with_critic_gemm_tflops": (flop_actor + flop_critic) / t_act_v / 1e12,
        },
        "obs_normalize": {
            "workload": f"Normalizer::normalize of the update batch [{n}x{od}]",
            "us": t_norm * 1e6, "GBps": norm_bytes / t_norm / 1e9,
            "hbm_frac": norm_bytes / t_norm / 8e12,
        },
        "obs_norm_update": {
            "workload": f"Normalizer::update / PendingNorm::push of [{envs}x{od}] (one rollout step) and "
                        f"[{n}x{od}] (the batch)",
            "step_us": t_upd_step * 1e6, "batch_us": t_upd_all * 1e6,
            "batch_GBps_one_read": n * od * 4 / t_upd_all / 1e9,
        },
    }


def _kernel_ms(ctx, fn, reps, between=None):
    """Summed HIP-event kernel time per call of fn (every launch on the context
    stream bracketed by events); between(), if given, runs before each call
    outside the timed launches (a cache flush by hipMemcpyAsync)."""
    fn()
    ctx.synchronize()
    tot = C.c_double()
    ctx.check(ctx.lib.zl_timing_begin(ctx.h, b"*"), "timing_begin")
    for _ in range(reps):
        if between is not None:
            between()
        fn()
    ctx.check(ctx.lib.zl_timing_end(ctx.h, C.byref(tot), None, None), "timing_end")
    return tot.value / 1e3 / reps


def operator_measurements(ctx):
    """The two operator-level workloads: the single dense layer (X [4096 x
    123] . W [123 x 512] + b, ELU; the reference's feature-major
    gemm_bias_act, src/biped/cutile_gemm.rs:578-625) and the clipped Adam
    step over actor + critic + log_std (459,323 parameters in the trainer's
    17 tensors: zl_adam_multi_clip, the sums of squares of the gradients,
    then one tensor-list Adam launch whose blocks take the global clip scale
    at 1.0; src/bin/biped_train_gpu.rs:1368-1461). Kernel time by HIP
    events; Adam warm (working set in the Infinity Cache) and cold (a
    512 MiB device copy between calls evicts it)."""
    from zealot_amd import ops, synth

    c1 = synth.config1()
    x, w_kn, b = c1["x"], c1["w_kn"], c1["b"]
    m, n, k = 512, x.shape[0], x.shape[1]
    dwt, dxt, db = ctx.to_device(w_kn.T.copy()), ctx.to_device(x.T.copy()), ctx.to_device(b)
    out_t = ctx.alloc((m, n))
    layer = lambda: ops.gemm_bias_act(ctx, out_t, dwt, dxt, m, n, k, db, 1, True)
    t_layer = _kernel_ms(ctx, layer, 200)
    t_layer_wall = _timed(ctx, layer, 200)
    flop1 = 2.0 * m * n * k

    sizes = []
    for dims in (synth.ACTOR_DIMS, synth.CRITIC_DIMS):
        for l in range(len(dims) - 1):
            sizes += [dims[l + 1] * dims[l], dims[l + 1]]
    sizes.append(synth.ACTOR_DIMS[-1])
    npar = sum(sizes)
    c3 = synth.config3(sum(sizes[:8]), sum(sizes[8:16]))
    p0 = np.concatenate([c3["actor"], c3["critic"], c3["log_std"]]).astype(np.float32)
    dp, dg = ctx.to_device(p0), ctx.to_device(c3["grads"][0])
    dm, dv = ctx.to_device(np.zeros(npar, np.float32)), ctx.to_device(np.zeros(npar, np.float32))
    scale, norm = ctx.alloc(1), ctx.alloc(1)
    offs = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    at = [(dp.offset(int(o)), dg.offset(int(o)), dm.offset(int(o)), dv.offset(int(o)), int(s))
          for o, s in zip(offs[:-1], sizes)]
    bc1, bc2 = float(np.float32(1.0) - np.float32(0.9 ** 11)), float(np.float32(1.0) - np.float32(0.999 ** 11))

    def adam():
        ops.adam_multi_clip(ctx, at, 1e-3, bc1, bc2, 1.0, scale, norm)

    flush_bytes = 512 << 20
    fa, fb = ctx.alloc(flush_bytes, np.uint8), ctx.alloc(flush_bytes, np.uint8)
    flush = lambda: ctx.check(ctx.lib.zl_copy_d2d(ctx.h, fb.p, fa.p, flush_bytes), "zl_copy_d2d")
    t_warm = _kernel_ms(ctx, adam, 100)
    t_cold = _kernel_ms(ctx, adam, 30, between=flush)
    t_adam_wall = _timed(ctx, adam, 100)
    bytes3 = 32.0 * npar  # sum of squares 4 B + Adam 28 B per parameter
    return {
        "dense_layer": {
            "workload": f"ELU(X [{n}x{k}] . W [{k}x{m}] + b), feature-major out [{m}x{n}]",
            "kernel_us": t_layer * 1e6, "wall_us": t_layer_wall * 1e6,
            "tflops": flop1 / t_layer / 1e12, "fp32_mfma_frac": flop1 / t_layer / 157.3e12,
        },
        "adam_clip": {
            "workload": f"global grad-norm clip 1.0 + Adam over {npar} params (17 tensors), 2 launches",
            "warm_kernel_us": t_warm * 1e6, "cold_kernel_us": t_cold * 1e6, "wall_us": t_adam_wall * 1e6,
            "warm_GBps": bytes3 / t_warm / 1e9, "cold_GBps": bytes3 / t_cold / 1e9,
            "cold_hbm_frac": bytes3 / t_cold / 8e12,
        },
    }


def gemm_flop_per_row(ad, cd):
    """Layer-GEMM FLOP per minibatch row of one update step: forward and
    weight gradient of every layer, data gradient of every layer above the
    first, both nets."""
    f = 0
    for dims in (ad, cd):
        mac = [dims[l] * dims[l + 1] for l in range(len(dims) - 1)]
        f += 2 * (2 * sum(mac) + sum(mac[1:]))
    return f


def trainer_nets_measurement(ctx, steps):
    """The reference trainer's own networks (src/bin/biped_train_gpu.rs:604-610):
    actor 265-256-256-128-12 on the policy observation, critic 64-512-256-128-1
    on a separate critic observation, over a 4096 x 24 rollout staged
    feature-major ([dim x n], as the trainer stages f_obs / f_cobs / f_act),
    GPU-trainer semantics at the headline settings. Wall time per update
    (critic values + GAE + update) over `steps` updates."""
    from zealot_amd import ops, synth
    from zealot_amd.rl import GpuActorCritic, PpoConfig, _ffi

    ad, cd = [265, 256, 256, 128, 12], [64, 512, 256, 128, 1]
    N, T = N_ENVS, T_STEPS
    n, mb = N * T, N * T // MINIBATCHES
    g = synth.rng(5, 1)
    obs = synth.obs(g, n, ad[0])
    cobs = synth.obs(g, n, cd[0])
    boot = synth.obs(g, N, cd[0])
    gac = GpuActorCritic(ctx, ad, cd, mb)
    gac.set_params(synth.kaiming_uniform_net(g, ad), synth.kaiming_uniform_net(g, cd),
                   np.full(ad[-1], -0.5, np.float32), 1e-3)
    d_obs, d_cobs, d_boot = ctx.to_device(obs), ctx.to_device(cobs), ctx.to_device(boot)
    d_mean, d_act, d_logp = ctx.alloc((n, ad[-1])), ctx.alloc((n, ad[-1])), ctx.alloc(n)
    gac.actor_mean(d_obs, n, d_mean)
    ops.sample_actions(ctx, d_mean, ctx.to_device(np.full(ad[-1], -0.5, np.float32)),
                       ctx.to_device(synth.normal(g, (n, ad[-1]))), n, ad[-1], d_act, d_logp)
    # The trainer's feature-major staging of the same batch.
    fm_obs, fm_cobs = ctx.to_device(np.ascontiguousarray(obs.T)), ctx.to_device(np.ascontiguousarray(cobs.T))
    fm_act = ctx.to_device(np.ascontiguousarray(d_act.numpy().T))
    fm_mean = ctx.to_device(np.ascontiguousarray(d_mean.numpy().T))
    d_rew = ctx.to_device(synth.normal(g, (T, N)))
    d_done = ctx.to_device((g.random((T, N)) < 0.02).astype(np.uint8))
    d_val, d_last, d_adv, d_ret = ctx.alloc(n), ctx.alloc(N), ctx.alloc(n), ctx.alloc(n)
    fm = _ffi.ZL_FM_OBS | _ffi.ZL_FM_CRITIC_OBS | _ffi.ZL_FM_ACTION | _ffi.ZL_FM_MEAN_OLD
    batch = _ffi.zl_batch(n, fm_obs.ptr, n, fm_cobs.ptr, n, fm_act.ptr, n, fm_mean.ptr, n, d_logp.ptr,
                          d_val.ptr, d_adv.ptr, d_ret.ptr, fm)
    cfg = PpoConfig.gpu_trainer(epochs=EPOCHS, minibatches=MINIBATCHES, clip=0.2, entropy_coef=0.005,
                                value_coef=1.0, max_grad_norm=1.0, adaptive_lr=False, early_stop=False,
                                normalize_adv=True, clamp_log_std=True).to_c()
    stats = _ffi.zl_ppo_stats()

    def step():
        gac.values(d_cobs, n, d_val)
        gac.values(d_boot, N, d_last)
        ops.gae(ctx, d_rew, d_val, d_done, d_last, T, N, d_adv, d_ret, 0.99, 0.95)
        ctx.check(ctx.lib.zl_ppo_update(gac.h, C.byref(batch), C.byref(cfg), C.byref(stats)), "update")

    t = _timed(ctx, step, steps)
    flop = gemm_flop_per_row(ad, cd) * n * EPOCHS
    gac.close()
    return {
        "workload": f"trainer nets actor {'-'.join(map(str, ad))} / critic {'-'.join(map(str, cd))} "
                    f"(separate critic obs), {N} envs x {T} steps, feature-major batch, critic values + "
                    f"GAE + {EPOCHS} x {MINIBATCHES} minibatches of {mb} rows, global clip 1.0, lr 1e-3",
        "ms_per_update": t * 1e3,
        "samples_per_s": EPOCHS * n / t,
        "update_gemm_tflops": flop / t / 1e12,
        "fp32_mfma_frac": flop / t / FP32_MFMA_PEAK,
    }


def actor_critic_measurement(ctx, gac, batch, step_values, steps):
    """The same workload under ActorCritic::update semantics
    (zealot-rl/src/ppo.rs:338-510): a Fisher-Yates shuffle of the batch per
    epoch from Lcg(t + 1) on the host, uploaded with the update (5 x 98,304
    row indices), the observation gather fused into the first layer, clip
    per net, per-step Adam t, mean-only-KL adaptive learning rate. Wall time
    per update (critic values + GAE + update) over `steps` updates."""
    from zealot_amd.rl import PpoConfig, _ffi

    cfg = PpoConfig(epochs=EPOCHS, minibatches=MINIBATCHES, clip=0.2, entropy_coef=0.005,
                    value_coef=1.0, max_grad_norm=1.0, desired_kl=0.01, lr_min=1e-5, lr_max=1e-2,
                    shuffle=True, normalize_adv=True, clamp_log_std=True).to_c()
    stats = _ffi.zl_ppo_stats()

    def step():
        step_values()
        ctx.check(ctx.lib.zl_ppo_update(gac.h, C.byref(batch), C.byref(cfg), C.byref(stats)), "update")

    t = _timed(ctx, step, steps)
    return {
        "workload": "the headline workload under ActorCritic::update semantics (host Fisher-Yates "
                    "shuffle per epoch + index upload, gathered minibatches, per-net clip, adaptive lr)",
        "ms_per_update": t * 1e3,
        "samples_per_s": EPOCHS * N_ENVS * T_STEPS / t,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--breakdown", action="store_true", help="per-kernel time table on stderr")
    ap.add_argument("--no-aux", action="store_true",
                    help="headline workload only (no aux lines): the process the rocprofv3 profiles cover")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the update runs on a single device "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    from zealot_amd import Context, ops, synth
    from zealot_amd.rl import GpuActorCritic, PpoConfig, _ffi

    ad, cd = synth.ACTOR_DIMS, synth.CRITIC_DIMS
    n = N_ENVS * T_STEPS
    mb = n // MINIBATCHES
    g = synth.rng(5)
    ro = synth.rollout(g, N_ENVS, T_STEPS)
    actor = synth.kaiming_uniform_net(g, ad)
    critic = synth.kaiming_uniform_net(g, cd)
    log_std = np.full(ad[-1], -0.5, np.float32)
    LD = 124  # rollout rows padded to a 16-byte multiple

    ctx = Context(0)
    gac = GpuActorCritic(ctx, ad, cd, mb)
    gac.set_params(actor, critic, log_std, 1e-3)
    obs_p = np.zeros((n, LD), np.float32)
    obs_p[:, :123] = ro["obs"]
    boot_p = np.zeros((N_ENVS, LD), np.float32)
    boot_p[:, :123] = ro["boot_obs"]
    d_obs, d_boot = ctx.to_device(obs_p), ctx.to_device(boot_p)
    d_rew, d_done = ctx.to_device(ro["rewards"]), ctx.to_device(ro["dones"])
    d_mean = ctx.alloc((n, ad[-1]))
    d_act = ctx.alloc((n, ad[-1]))
    d_logp = ctx.alloc(n)
    d_val, d_last = ctx.alloc(n), ctx.alloc(N_ENVS)
    d_adv, d_ret = ctx.alloc(n), ctx.alloc(n)
    # Rollout products (setup, untimed): mean_old, sampled actions, logp_old.
    gac.actor_mean(d_obs, n, d_mean, ld=LD)
    ops.sample_actions(ctx, d_mean, ctx.to_device(log_std), ctx.to_device(ro["eps"]), n, ad[-1], d_act, d_logp)
    ctx.synchronize()

    batch = _ffi.zl_batch(n, d_obs.ptr, LD, d_obs.ptr, LD, d_act.ptr, ad[-1], d_mean.ptr, ad[-1],
                          d_logp.ptr, d_val.ptr, d_adv.ptr, d_ret.ptr)
    cfg = PpoConfig.gpu_trainer(epochs=EPOCHS, minibatches=MINIBATCHES, clip=0.2, entropy_coef=0.005,
                                value_coef=1.0, max_grad_norm=1.0, adaptive_lr=False, early_stop=False,
                                normalize_adv=True, clamp_log_std=True).to_c()
    stats = _ffi.zl_ppo_stats()

    def step():
        gac.values(d_obs, n, d_val, ld=LD)
        gac.values(d_boot, N_ENVS, d_last, ld=LD)
        ops.gae(ctx, d_rew, d_val, d_done, d_last, T_STEPS, N_ENVS, d_adv, d_ret, 0.99, 0.95)
        ctx.check(ctx.lib.zl_ppo_update(gac.h, C.byref(batch), C.byref(cfg), C.byref(stats)), "update")

    for _ in range(args.warmup):
        step()
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.synchronize()
    t_step = (time.perf_counter() - t0) / args.steps

    captures, capture_ms = gac.graph_info()
    # Per-kernel HIP-event timing: one instrumented step (eager launches),
    # every launch bracketed by events on the context stream.
    ctx.check(ctx.lib.zl_timing_begin(ctx.h, b"*"), "timing_begin")
    step()
    ctx.check(ctx.lib.zl_timing_end(ctx.h, None, None, None), "timing_end")
    ktime = {}
    for i in range(ctx.lib.zl_kernel_count()):
        name, ms, cnt, fl = C.c_char_p(), C.c_double(), C.c_longlong(), C.c_double()
        ctx.check(ctx.lib.zl_timing_kernel(ctx.h, i, C.byref(name), C.byref(ms), C.byref(cnt),
                                           C.byref(fl)), "timing_kernel")
        if cnt.value:
            ktime[name.value.decode()] = (ms.value, cnt.value, fl.value)
    # Layer GEMM work: the GEMM kernels and zk_head_fwd* (the head launch that
    # also computes the last hidden layer's forward; its FLOP count is that
    # layer's).
    gemm = {k: v for k, v in ktime.items() if k.startswith(("zk_gemm", "zk_narrow", "zk_head_fwd"))}
    gemm_ms = sum(v[0] for v in gemm.values())
    gemm_flops = sum(v[2] for v in gemm.values())
    dom = max(gemm, key=lambda k: gemm[k][0])
    dom_ms, dom_cnt, dom_flops = gemm[dom]
    dom_avg_s = dom_ms / 1e3 / dom_cnt
    dom_flop_per_launch = dom_flops / dom_cnt
    achieved = dom_flop_per_launch / dom_avg_s
    if args.breakdown:
        print(f"{'kernel':32s} {'launches':>8s} {'ms/step':>8s} {'us/launch':>9s} {'TFLOP/s':>8s}", file=sys.stderr)
        for k, (ms, cnt, fl) in sorted(ktime.items(), key=lambda kv: -kv[1][0]):
            tf = fl / (ms / 1e3) / 1e12 if ms > 0 else 0.0
            print(f"{k:32s} {cnt:8d} {ms:8.3f} {1e3 * ms / cnt:9.2f} {tf:8.2f}", file=sys.stderr)
        print(f"step {t_step * 1e3:.3f} ms; instrumented step kernels {sum(v[0] for v in ktime.values()):.3f} ms; "
              f"GEMM kernels {gemm_ms:.3f} ms", file=sys.stderr)
        shapes = {}
        for i in range(ctx.lib.zl_timing_launch_count(ctx.h)):
            name, ms, fl, sh = C.c_char_p(), C.c_double(), C.c_double(), (C.c_int * 4)()
            ctx.check(ctx.lib.zl_timing_launch(ctx.h, i, C.byref(name), C.byref(ms), C.byref(fl), sh),
                      "timing_launch")
            if sh[0]:
                key = (name.value.decode(), tuple(sh))
                acc = shapes.setdefault(key, [0.0, 0, 0.0])
                acc[0] += ms.value
                acc[1] += 1
                acc[2] += fl.value
        print(f"{'GEMM kernel':32s} {'M x N x K / splits':>24s} {'launches':>8s} {'us/launch':>9s} {'TFLOP/s':>8s}",
              file=sys.stderr)
        for (k, sh), (ms, cnt, fl) in sorted(shapes.items(), key=lambda kv: -kv[1][0]):
            print(f"{k:32s} {'%dx%dx%d/%d' % sh:>24s} {cnt:8d} {1e3 * ms / cnt:9.2f} "
                  f"{fl / (ms / 1e3) / 1e12:8.2f}", file=sys.stderr)

    out = {
        "metric": "PPO update samples/sec (fwd+bwd+Adam) on 1 MI355X; % fp32-MFMA peak",
        "value": EPOCHS * n / t_step,
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": t_step * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded numpy rollout: obs ~ N(0,1) clipped to +-5, rewards ~ N(0,1), "
                "dones ~ Bernoulli(0.02); Kaiming-uniform weights)",
        "config": {
            "workload": "full PPO update: 4096 envs x 24 steps (98,304 samples); critic values + GAE + "
                        "adv norm + 5 epochs x 4 minibatches of 24,576 rows, actor 123-512-256-128-29 + "
                        "critic 123-512-256-128-1 fwd+bwd, global clip 1.0, Adam lr 1e-3",
            "global_batch": n,
            "minibatch": mb,
            "epochs": EPOCHS,
            "semantics": "gpu_trainer",
        },
        "rollout_samples_per_s": n / t_step,
        "gemm_tflops_per_step": gemm_flops / t_step / 1e12,
        "fp32_mfma_frac_step": gemm_flops / t_step / FP32_MFMA_PEAK,
        "fp32_mfma_frac_gemm_kernels": gemm_flops / (gemm_ms / 1e3) / FP32_MFMA_PEAK,
        "roofline": {
            "kernel": dom,
            "bound": "mfma",
            "achieved": achieved / 1e12,
            "peak": FP32_MFMA_PEAK / 1e12,
            "unit": "TFLOP/s",
            "frac": achieved / FP32_MFMA_PEAK,
            "traffic": MEASURED_TRAFFIC.get(dom),
            "flop_per_launch": dom_flop_per_launch,
            "avg_launch_us": dom_avg_s * 1e6,
            "launches_per_step": dom_cnt,
        },
    }
    out["update_graph"] = {"captures": captures, "capture_instantiate_ms": capture_ms,
                           "note": "the update graph is captured once per shape / configuration; "
                                   "new batch buffers are read through a device pointer block"}
    if not args.no_aux:
        out["aux"] = aux_measurements(ctx, gac, ro, d_obs, LD, n)
        out["aux"].update(operator_measurements(ctx))
        out["aux"]["trainer_nets_update"] = trainer_nets_measurement(ctx, max(2, min(args.steps, 5)))

        def values_and_gae():
            gac.values(d_obs, n, d_val, ld=LD)
            gac.values(d_boot, N_ENVS, d_last, ld=LD)
            ops.gae(ctx, d_rew, d_val, d_done, d_last, T_STEPS, N_ENVS, d_adv, d_ret, 0.99, 0.95)

        out["aux"]["actor_critic_update"] = actor_critic_measurement(ctx, gac, batch, values_and_gae,
                                                                     max(2, min(args.steps, 5)))
    cpu_inputs = None
    if not args.no_cpu_baseline:
        # The baseline's inputs as they stand after the timed updates.
        a_now, c_now, ls_now, _ = gac.get_params()
        cpu_inputs = (ro, a_now, c_now, ls_now, d_mean.numpy(), d_act.numpy(), d_logp.numpy(),
                      d_val.numpy(), (d_adv.numpy(), d_ret.numpy()))
    out["self_check"] = self_check(
        ctx, gac, ro["obs"], d_obs, LD, n, mb,
        (d_obs.ptr, LD, d_obs.ptr, LD, d_act.ptr, ad[-1], d_mean.ptr, ad[-1], d_logp.ptr, d_val.ptr,
         d_adv.ptr, d_ret.ptr), stats)
    if cpu_inputs is not None:
        out["cpu_baseline"] = cpu_baseline(*cpu_inputs)
    gac.close()
    ctx.close()
    print(json.dumps(out), flush=True)
    if not out["self_check"]["pass"]:
        print("bench.py: post-run self-check failed: " + json.dumps(out["self_check"]), file=sys.stderr)
        sys.exit(1)


if __name__ == "__main__":
    main()
