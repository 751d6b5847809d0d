"""Operator-level entry points (the cuTile adapter and vortx kernels the GPU
trainer calls), thin wrappers over the C ABI. All buffers are DeviceBuffers."""

from __future__ import annotations

import ctypes as C

from .device import Context, DeviceBuffer


def gemm(ctx: Context, out: DeviceBuffer, lhs: DeviceBuffer, lhs_t: bool, rhs: DeviceBuffer,
         rhs_t: bool, m: int, n: int, k: int):
    """out(m x n) = lhs(m x k) . rhs(k x n) (CutileGemm::gemm, src/biped/cutile_gemm.rs:477)."""
    ctx.check(ctx.lib.zl_gemm(ctx.h, out.p, lhs.p, int(lhs_t), rhs.p, int(rhs_t), m, n, k), "zl_gemm")


def gemm_bias_act(ctx: Context, out, lhs, rhs, m, n, k, bias, bias_row_stride=1, elu=True):
    """CutileGemm::gemm_bias_act (src/biped/cutile_gemm.rs:578)."""
    ctx.check(
        ctx.lib.zl_gemm_bias_act(ctx.h, out.p, lhs.p, rhs.p, m, n, k, bias.p, bias_row_stride, int(elu)),
        "zl_gemm_bias_act",
    )


def elu_backward(ctx: Context, g, y, m, n):
    ctx.check(ctx.lib.zl_elu_backward(ctx.h, g.p, y.p, m, n), "zl_elu_backward")


def row_sum(ctx: Context, out, x, m, n):
    ctx.check(ctx.lib.zl_row_sum(ctx.h, out.p, x.p, m, n), "zl_row_sum")


def ppo_actor_grad(ctx: Context, mean, action, log_std, adv, logp_old, mean_old, rows, A, clip,
                   entropy_coef, scale, d_mean, d_log_std, stats, ld_mean=None, ld_action=None,
                   ld_d_mean=None):
    ctx.check(
        ctx.lib.zl_ppo_actor_grad(
            ctx.h, mean.p, ld_mean or A, action.p, ld_action or A, log_std.p, adv.p, logp_old.p,
            mean_old.p if mean_old is not None else None, A, rows, A, clip, entropy_coef, scale,
            d_mean.p, ld_d_mean or A, d_log_std.p, stats.p,
        ),
        "zl_ppo_actor_grad",
    )


def ppo_value_grad(ctx: Context, v, value_old, ret, rows, clip, value_coef, scale, d_v, stats):
    ctx.check(
        ctx.lib.zl_ppo_value_grad(ctx.h, v.p, value_old.p, ret.p, rows, clip, value_coef, scale, d_v.p, stats.p),
        "zl_ppo_value_grad",
    )


def adam_step(ctx: Context, p, g, m, v, n, lr, bc1, bc2, beta1=0.9, beta2=0.999, eps=1e-8):
    ctx.check(ctx.lib.zl_adam_step(ctx.h, p.p, g.p, m.p, v.p, n, lr, beta1, beta2, eps, bc1, bc2), "zl_adam_step")


def grad_sqnorm(ctx: Context, x, n, out):
    ctx.check(ctx.lib.zl_grad_sqnorm(ctx.h, x.p, n, out.p), "zl_grad_sqnorm")


def gae(ctx: Context, rewards, values, dones, last_values, T, N, adv, ret, gamma=0.99, lam=0.95,
        in_strides=None, out_strides=None):
    """GAE over N envs x T steps; default layout [T x N] (time-major) in and out."""
    its, ies = in_strides if in_strides is not None else (N, 1)
    ots, oes = out_strides if out_strides is not None else (N, 1)
    ctx.check(
        ctx.lib.zl_gae(ctx.h, rewards.p, values.p, dones.p, last_values.p, T, N, its, ies, ots, oes,
                       gamma, lam, adv.p, ret.p),
        "zl_gae",
    )


def adv_normalize(ctx: Context, adv, n):
    ctx.check(ctx.lib.zl_adv_normalize(ctx.h, adv.p, n), "zl_adv_normalize")


def sample_actions(ctx: Context, mean, log_std, eps, rows, A, action, logp, ld_mean=None):
    ctx.check(
        ctx.lib.zl_sample_actions(ctx.h, mean.p, ld_mean or A, log_std.p, eps.p, rows, A, action.p, logp.p),
        "zl_sample_actions",
    )
