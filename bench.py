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
(sample-gradient evaluations per second).
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
GEMM_KERNELS = [
    "zk_gemm_ak_bk_64x128", "zk_gemm_ak_bk_128x32", "zk_gemm_ak_bk_256x16",
    "zk_gemm_ak_bn_64x128", "zk_gemm_am_bn_64x128", "zk_splitk_reduce",
]
OTHER_KERNELS = ["zk_actor_loss", "zk_value_loss", "zk_sumsq", "zk_finalize", "zk_adam",
                 "zk_gae", "zk_adv_norm", "zk_epoch_begin", "zk_epoch_end", "zk_copy_rows"]


def fwd_kernel(n_out: int) -> str:
    if n_out <= 16:
        return "zk_gemm_ak_bk_256x16"
    if n_out <= 32:
        return "zk_gemm_ak_bk_128x32"
    return "zk_gemm_ak_bk_64x128"


def gemm_launches(actor_dims, critic_dims, mb, n_value_rows, chunk):
    """(kernel, algorithmic FLOP) of every GEMM launch in one step."""
    out = []
    for dims in (critic_dims,):  # value forward, chunked by the minibatch capacity
        r = n_value_rows
        while r > 0:
            rows = min(chunk, r)
            for l in range(len(dims) - 1):
                out.append((fwd_kernel(dims[l + 1]), 2 * rows * dims[l] * dims[l + 1]))
            r -= rows
    for _ in range(EPOCHS * MINIBATCHES):
        for dims in (actor_dims, critic_dims):
            for l in range(len(dims) - 1):
                out.append((fwd_kernel(dims[l + 1]), 2 * mb * dims[l] * dims[l + 1]))
            for l in range(len(dims) - 1):
                out.append(("zk_gemm_am_bn_64x128", 2 * mb * dims[l] * dims[l + 1]))
                if l > 0:
                    out.append(("zk_gemm_ak_bn_64x128", 2 * mb * dims[l] * dims[l + 1]))
    return out


def cpu_baseline(ro, actor, critic, log_std, mean_old, action, logp_old, values, adv, ret):
    """The oracle's restatement of the trainer update on a bounded sample:
    one 24,576-row minibatch (fwd + bwd + clip + Adam) of the same rollout."""
    from oracle import zl_oracle as zo
    from zealot_amd import synth

    n = 24_576
    threads = min(os.cpu_count() or 1, 16)
    batch = dict(obs=ro["obs"][:n], critic_obs=ro["obs"][:n], action=action[:n], mean_old=mean_old[:n],
                 logp_old=logp_old[:n], value_old=values[:n], adv=zo.adv_normalize(adv[:n]), ret=ret[:n])
    tr = zo.Trainer(synth.ACTOR_DIMS, synth.CRITIC_DIMS, actor, critic, log_std, 1e-3)
    cfg = zo.TrainerCfg(0.2, 0.005, 1.0, 1, 1, 1.0, 0.01, 1e-5, 1e-2, 0, 0, 1)
    t0 = time.perf_counter()
    tr.update(batch, cfg, nthreads=threads)
    dt = time.perf_counter() - t0
    return {"value": n / dt, "unit": "samples/s", "cores": threads, "kind": "port",
            "sample": f"1 minibatch of {n} rows of the same rollout (actor+critic fwd+bwd, global "
                      f"clip, Adam; trainer semantics), {dt:.1f} s on {threads} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--breakdown", action="store_true", help="per-kernel time table on stderr")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
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

    # Per-kernel HIP-event timing (one instrumented, eagerly launched step per kernel).
    launches = gemm_launches(ad, cd, mb, n + N_ENVS, mb)
    flops_by_k, count_by_k = {}, {}
    for k, f in launches:
        flops_by_k[k] = flops_by_k.get(k, 0) + f
        count_by_k[k] = count_by_k.get(k, 0) + 1
    ktime = {}
    names = GEMM_KERNELS + (OTHER_KERNELS if args.breakdown else [])
    for k in names:
        ctx.check(ctx.lib.zl_timing_begin(ctx.h, k.encode()), "timing_begin")
        step()
        ms, cnt = C.c_double(), C.c_longlong()
        ctx.check(ctx.lib.zl_timing_end(ctx.h, C.byref(ms), C.byref(cnt)), "timing_end")
        ktime[k] = (ms.value, cnt.value)
    gemm_flops = sum(f for _, f in launches)
    dom = max(flops_by_k, key=lambda k: ktime.get(k, (0, 0))[0])
    dom_ms, dom_cnt = ktime[dom]
    dom_avg_s = dom_ms / 1e3 / max(dom_cnt, 1)
    dom_flop_per_launch = flops_by_k[dom] / count_by_k[dom]
    achieved = dom_flop_per_launch / dom_avg_s
    gemm_ms = sum(ktime[k][0] for k in GEMM_KERNELS if k in ktime)
    if args.breakdown:
        print(f"{'kernel':28s} {'launches':>9s} {'ms/step':>9s} {'us/launch':>10s} {'TFLOP/s':>8s}", file=sys.stderr)
        for k, (ms, cnt) in sorted(ktime.items(), key=lambda kv: -kv[1][0]):
            tf = flops_by_k.get(k, 0) / (ms / 1e3) / 1e12 if ms > 0 and k in flops_by_k else 0.0
            print(f"{k:28s} {cnt:9d} {ms:9.3f} {1e3 * ms / max(cnt, 1):10.2f} {tf:8.2f}", file=sys.stderr)
        print(f"step {t_step * 1e3:.3f} ms; GEMM kernels {gemm_ms:.3f} ms", file=sys.stderr)

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
        "fp32_mfma_frac_gemm_kernels": gemm_flops / (gemm_ms / 1e3) / FP32_MFMA_PEAK if gemm_ms else None,
        "roofline": {
            "kernel": dom,
            "bound": "mfma",
            "achieved": achieved / 1e12,
            "peak": FP32_MFMA_PEAK / 1e12,
            "unit": "TFLOP/s",
            "frac": achieved / FP32_MFMA_PEAK,
            "traffic": None,
            "flop_per_launch": dom_flop_per_launch,
            "avg_launch_us": dom_avg_s * 1e6,
            "launches_per_step": dom_cnt,
        },
    }
    if not args.no_cpu_baseline:
        mean_old = d_mean.numpy()
        action = d_act.numpy()
        logp_old = d_logp.numpy()
        values = d_val.numpy()
        adv = d_adv.numpy()
        ret = d_ret.numpy()
        a_now, c_now, ls_now, _ = gac.get_params()
        out["cpu_baseline"] = cpu_baseline(ro, a_now, c_now, ls_now, mean_old, action, logp_old,
                                           values, adv, ret)
    gac.close()
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
