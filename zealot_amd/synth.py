"""Seeded synthetic workloads for the PPO learning path (numpy only).

The shapes are the path's benchmark configurations: a single 123->512 ELU
layer over 4096 rows; actor inference 123-512-256-128-29 over 4096 rows with
Gaussian sampling; Adam over actor + critic (459,323 params); one PPO
minibatch of 24,576 rows; a full update over 4096 envs x 24 steps. Every
array is float32 and generated on the host from numpy's PCG64 with seed
0x2EA10000 + config index, so the device path and the CPU oracle consume
byte-identical inputs. Observations are clipped to +-5, the output range of a
fresh zealot-rl Normalizer (zealot-rl/src/ppo.rs:198-205), so that staging
them as already-normalised observations matches what the reference's update
feeds its networks.
"""

from __future__ import annotations

import numpy as np

ACTOR_DIMS = [123, 512, 256, 128, 29]
CRITIC_DIMS = [123, 512, 256, 128, 1]
SEED_BASE = 0x2EA10000
LOG_SQRT_2PI = np.float32(0.9189385)


def rng(config: int, salt: int = 0) -> np.random.Generator:
    return np.random.default_rng(SEED_BASE + config + 1000 * salt)


def normal(g: np.random.Generator, shape, std=1.0) -> np.ndarray:
    return (g.standard_normal(shape) * std).astype(np.float32)


def obs(g: np.random.Generator, rows: int, dim: int) -> np.ndarray:
    return np.clip(normal(g, (rows, dim)), -5.0, 5.0).astype(np.float32)


def kaiming_uniform_net(g: np.random.Generator, dims, bias_bound: float = 0.0) -> np.ndarray:
    """Packed params (w[0], b[0], ...; w[l] [out x in]) with w ~ U(+-sqrt(6/fan_in))
    (torch's kaiming_uniform_(a=0) bound) and b ~ U(+-bias_bound) (0: zeros)."""
    parts = []
    for l in range(len(dims) - 1):
        fan_in, fan_out = dims[l], dims[l + 1]
        bound = np.sqrt(6.0 / fan_in)
        parts.append(g.uniform(-bound, bound, fan_out * fan_in).astype(np.float32))
        if bias_bound > 0.0:
            parts.append(g.uniform(-bias_bound, bias_bound, fan_out).astype(np.float32))
        else:
            parts.append(np.zeros(fan_out, np.float32))
    return np.concatenate(parts)


def gaussian_logp(action: np.ndarray, mean: np.ndarray, log_std: np.ndarray) -> np.ndarray:
    """Row-wise Gaussian log-prob in float32 with the reference's operation order
    (zealot-rl/src/ppo.rs:297-305)."""
    std = np.exp(log_std).astype(np.float32)
    lp = np.zeros(action.shape[0], np.float32)
    for k in range(action.shape[1]):
        d = ((action[:, k] - mean[:, k]) / std[k]).astype(np.float32)
        lp = (lp + ((np.float32(-0.5) * d * d - log_std[k]) - LOG_SQRT_2PI)).astype(np.float32)
    return lp


def config1():
    """Single dense layer 4096 x 123 -> 512 + ELU."""
    g = rng(1)
    x = normal(g, (4096, 123))
    bound = np.sqrt(6.0 / 123)
    w_kn = g.uniform(-bound, bound, (123, 512)).astype(np.float32)  # W [K x N]
    b = g.uniform(-0.1, 0.1, 512).astype(np.float32)
    return dict(x=x, w_kn=w_kn, b=b)


def config2():
    """Actor rollout inference over 4096 rows with sampling noise."""
    g = rng(2)
    return dict(
        obs=obs(g, 4096, 123),
        actor=kaiming_uniform_net(g, ACTOR_DIMS),
        log_std=np.full(29, -0.5, np.float32),
        eps=normal(g, (4096, 29)),
    )


def config3(n_params_actor: int, n_params_critic: int, warm_steps: int = 10):
    """Adam over actor + critic + log_std: params, grads ~ N(0, 0.01) per step."""
    g = rng(3)
    a = kaiming_uniform_net(g, ACTOR_DIMS)
    c = kaiming_uniform_net(g, CRITIC_DIMS)
    assert a.size == n_params_actor and c.size == n_params_critic
    ls = np.full(29, -0.5, np.float32)
    grads = [normal(g, a.size + c.size + 29, 1e-2) for _ in range(warm_steps + 1)]
    return dict(actor=a, critic=c, log_std=ls, grads=grads)


def minibatch_inputs(g: np.random.Generator, rows: int, means: np.ndarray, values: np.ndarray):
    """Config-4 style per-sample inputs given the actor means / critic values of
    the observations: actions ~ N(0,1), logp_old = logp(action | mean) +
    N(0, 0.05), v_old = v + N(0, 0.05), advantages ~ N(0,1), returns ~ N(0,1)."""
    A = means.shape[1]
    log_std = np.full(A, -0.5, np.float32)
    action = normal(g, (rows, A))
    logp_old = (gaussian_logp(action, means, log_std) + normal(g, rows, 0.05)).astype(np.float32)
    value_old = (values.reshape(-1) + normal(g, rows, 0.05)).astype(np.float32)
    adv = normal(g, rows)
    ret = normal(g, rows)
    return dict(action=action, logp_old=logp_old, value_old=value_old, adv=adv, ret=ret,
                log_std=log_std)


def rollout(g: np.random.Generator, n_envs: int, T: int, obs_dim: int = 123, done_p: float = 0.02):
    """Config-5 rollout in time-major order (sample t*N + e)."""
    return dict(
        obs=obs(g, T * n_envs, obs_dim),
        boot_obs=obs(g, n_envs, obs_dim),
        rewards=normal(g, (T, n_envs)),
        dones=(g.random((T, n_envs)) < done_p).astype(np.uint8),
        eps=normal(g, (T * n_envs, ACTOR_DIMS[-1])),
    )
