"""Vectorised float64 numpy restatement of the PPO minibatch gradient — the
"truth" leg of the parity tests (independent of both the C++ oracle and the
HIP kernels). Math of zealot-rl/src/net.rs:88-140 and ppo.rs:406-462."""

from __future__ import annotations

import numpy as np

LOG_SQRT_2PI = 0.9189385


def unpack(dims, packed):
    ws, bs, o = [], [], 0
    for l in range(len(dims) - 1):
        out, inp = dims[l + 1], dims[l]
        ws.append(np.asarray(packed[o:o + out * inp], np.float64).reshape(out, inp))
        o += out * inp
        bs.append(np.asarray(packed[o:o + out], np.float64))
        o += out
    return ws, bs


def pack(ws, bs):
    return np.concatenate([np.concatenate([w.ravel(), b]) for w, b in zip(ws, bs)])


def elu(z):
    return np.where(z > 0, z, np.expm1(np.minimum(z, 0)))


def forward(dims, packed, x):
    ws, bs = unpack(dims, packed)
    acts = [np.asarray(x, np.float64)]
    for l, (w, b) in enumerate(zip(ws, bs)):
        z = acts[-1] @ w.T + b
        acts.append(z if l == len(ws) - 1 else elu(z))
    return acts


def backward(dims, packed, acts, g_out):
    ws, bs = unpack(dims, packed)
    L = len(ws)
    gw, gb = [None] * L, [None] * L
    delta = np.asarray(g_out, np.float64)
    for l in range(L - 1, -1, -1):
        if l != L - 1:
            a = acts[l + 1]
            delta = delta * np.where(a > 0, 1.0, a + 1.0)
        gw[l] = delta.T @ acts[l]
        gb[l] = delta.sum(0)
        delta = delta @ ws[l]
    return pack(gw, gb)


def minibatch_grads(actor_dims, critic_dims, actor, critic, log_std, batch, idx, clip,
                    entropy_coef, value_coef):
    idx = np.asarray(idx)
    n = len(idx)
    s = 1.0 / n
    ls = np.asarray(log_std, np.float64)
    obs = np.asarray(batch["obs"], np.float64)[idx]
    cobs = np.asarray(batch["critic_obs"], np.float64)[idx]
    act = np.asarray(batch["action"], np.float64)[idx]
    adv = np.asarray(batch["adv"], np.float64)[idx]
    lpo = np.asarray(batch["logp_old"], np.float64)[idx]
    vo = np.asarray(batch["value_old"], np.float64)[idx]
    ret = np.asarray(batch["ret"], np.float64)[idx]
    aa = forward(actor_dims, actor, obs)
    mean = aa[-1]
    d = act - mean
    lp = np.sum(-0.5 * (d / np.exp(ls)) ** 2 - ls - LOG_SQRT_2PI, axis=1)
    ratio = np.exp(lp - lpo)
    surr = np.minimum(ratio * adv, np.clip(ratio, 1 - clip, 1 + clip) * adv)
    clipped = ((adv >= 0) & (ratio > 1 + clip)) | ((adv < 0) & (ratio < 1 - clip))
    keep = (~clipped)[:, None]
    inv_var = np.exp(-2 * ls)
    g_mean = np.where(keep, -(adv * ratio)[:, None] * d * inv_var * s, 0.0)
    dls = np.where(keep, (adv * ratio)[:, None] * (d * d * inv_var - 1.0), 0.0)
    gls = (-dls * s).sum(0) - entropy_coef * s * n
    ga = backward(actor_dims, actor, aa, g_mean)
    ca = forward(critic_dims, critic, cobs)
    v = ca[-1][:, 0]
    vc = vo + np.clip(v - vo, -clip, clip)
    lu, lc = (v - ret) ** 2, (vc - ret) ** 2
    use_c = lc > lu
    vloss = np.where(use_c, lc, lu)
    dv = np.where(use_c, 2 * (vc - ret), 2 * (v - ret))
    gc = backward(critic_dims, critic, ca, (value_coef * dv * s)[:, None])
    mo = batch.get("mean_old")
    kl = 0.0
    if mo is not None:
        mo = np.asarray(mo, np.float64)[idx]
        kl = float(np.sum(0.5 * ((mean - mo) * np.exp(-ls)) ** 2) * s)
    stats = np.array([float(surr.sum() * s), float(vloss.sum() * s), kl])
    return ga, gc, gls, stats
