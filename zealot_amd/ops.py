"""Operator-level entry points (the cuTile adapter and vortx kernels the GPU
trainer calls), thin wrappers over the C ABI. All buffers are DeviceBuffers."""

from __future__ import annotations

import ctypes as C

from . import _ffi
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
                   ld_d_mean=None, ld_mean_old=None, feature_major=False):
    """Vortx Ppo::actor_grad + the dls row sum (src/bin/biped_train_gpu.rs:1257-1271,
    1350-1357). Batch-major [rows x A] operands by default (row strides ld_*,
    default A); feature_major: the trainer's [A x rows] tensors (feature
    strides ld_*, default rows)."""
    dflt = rows if feature_major else A
    ctx.check(
        ctx.lib.zl_ppo_actor_grad(
            ctx.h, mean.p, ld_mean or dflt, action.p, ld_action or dflt, log_std.p, adv.p,
            logp_old.p, mean_old.p if mean_old is not None else None, ld_mean_old or dflt, rows, A,
            clip, entropy_coef, scale, d_mean.p, ld_d_mean or dflt, d_log_std.p, stats.p,
            int(bool(feature_major)),
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


def _ptr(x):
    return x.p if isinstance(x, DeviceBuffer) else x


def grad_clip_scale(ctx: Context, tensors, max_norm, scale_out, norm_out=None):
    """The trainer's global grad-norm clip on the device (src/bin/biped_train_gpu.rs:
    1368-1452): tensors = [(buffer or pointer, n), ...]; scale_out[0] = the clip
    scale, norm_out[0] = the global norm."""
    arr = (_ffi.zl_tensor * len(tensors))(*[_ffi.zl_tensor(_ptr(t), int(n)) for t, n in tensors])
    ctx.check(ctx.lib.zl_grad_clip_scale(ctx.h, arr, len(tensors), max_norm, _ptr(scale_out),
                                         _ptr(norm_out) if norm_out is not None else None),
              "zl_grad_clip_scale")


def adam_multi(ctx: Context, tensors, lr, bc1, bc2, clip_scale=None, beta1=0.9, beta2=0.999, eps=1e-8):
    """Adam over [(p, g, m, v, n), ...] in one launch, gradients times *clip_scale."""
    arr = (_ffi.zl_adam_tensor * len(tensors))(
        *[_ffi.zl_adam_tensor(_ptr(p), _ptr(g), _ptr(m), _ptr(v), int(n)) for p, g, m, v, n in tensors])
    ctx.check(ctx.lib.zl_adam_multi(ctx.h, arr, len(tensors), lr, beta1, beta2, eps, bc1, bc2,
                                    _ptr(clip_scale) if clip_scale is not None else None),
              "zl_adam_multi")


def adam_multi_clip(ctx: Context, tensors, lr, bc1, bc2, max_norm, scale_out=None, norm_out=None,
                    beta1=0.9, beta2=0.999, eps=1e-8):
    """Global grad-norm clip + Adam over [(p, g, m, v, n), ...] in two launches."""
    arr = (_ffi.zl_adam_tensor * len(tensors))(
        *[_ffi.zl_adam_tensor(_ptr(p), _ptr(g), _ptr(m), _ptr(v), int(n)) for p, g, m, v, n in tensors])
    ctx.check(ctx.lib.zl_adam_multi_clip(ctx.h, arr, len(tensors), lr, beta1, beta2, eps, bc1, bc2, max_norm,
                                         _ptr(scale_out) if scale_out is not None else None,
                                         _ptr(norm_out) if norm_out is not None else None),
              "zl_adam_multi_clip")


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
