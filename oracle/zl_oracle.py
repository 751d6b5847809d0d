"""ctypes binding of the CPU oracle (oracle/libzl_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the parity reference / CPU baseline, never
by the product path. The oracle restates zealot-rl (zealot-rl/src/{rng,net,ppo}.rs)
and the GPU trainer's update semantics (src/bin/biped_train_gpu.rs:1164-1553)
in scalar C++; see zl_oracle.hpp for the line-by-line citations.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# ZL_ORACLE_LIBRARY selects another build (e.g. the sanitizer build, oracle/_asan/).
LIB = os.environ.get("ZL_ORACLE_LIBRARY") or os.path.join(HERE, "libzl_oracle.so")

vp = C.c_void_p
fl = C.c_float


class PpoCfg(C.Structure):
    """zlo_ppo_cfg (PpoConfig, zealot-rl/src/ppo.rs:22-65)."""

    _fields_ = [
        ("gamma", fl), ("lam", fl), ("clip", fl), ("entropy_coef", fl), ("value_coef", fl),
        ("epochs", C.c_int), ("minibatches", C.c_int), ("max_grad_norm", fl),
        ("desired_kl", fl), ("lr_min", fl), ("lr_max", fl), ("adaptive_lr", C.c_int),
    ]


class TrainerCfg(C.Structure):
    """zlo_trainer_cfg (src/bin/biped_train_gpu.rs:53-75 and knobs)."""

    _fields_ = [
        ("clip", fl), ("entropy_coef", fl), ("value_coef", fl), ("epochs", C.c_int),
        ("minibatches", C.c_int), ("grad_clip", fl), ("desired_kl", fl), ("lr_min", fl),
        ("lr_max", fl), ("adaptive_lr", C.c_int), ("early_stop", C.c_int),
        ("clamp_after", C.c_int),
    ]


def build():
    subprocess.run(["make", "-s", "-B", "-C", HERE], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB):
        build()
    L = C.CDLL(LIB)
    sig = {
        "zlo_lcg_units": (None, [C.c_uint64, C.c_int, vp]),
        "zlo_lcg_gauss": (None, [C.c_uint64, C.c_int, vp]),
        "zlo_powi": (fl, [fl, C.c_int]),
        "zlo_elu": (fl, [fl]),
        "zlo_elu_grad_from_act": (fl, [fl]),
        "zlo_mlp_init": (None, [vp, C.c_int, fl, C.c_uint64, vp]),
        "zlo_mlp_forward": (None, [vp, C.c_int, vp, vp, C.c_int, vp]),
        "zlo_mlp_backward": (None, [vp, C.c_int, vp, vp, C.c_int, vp, vp, vp]),
        "zlo_mlpgrad_clip": (fl, [vp, C.c_int, vp, fl]),
        "zlo_adam_step": (None, [vp, C.c_int, vp, vp, vp, vp, C.c_int, fl]),
        "zlo_adam_flat": (None, [vp, vp, vp, vp, C.c_longlong, fl, fl, fl]),
        "zlo_gae": (None, [vp, vp, vp, C.c_int, fl, fl, fl, vp, vp]),
        "zlo_ac_create": (vp, [vp, C.c_int, vp, C.c_int, fl, fl, vp]),
        "zlo_ac_destroy": (None, [vp]),
        "zlo_ac_get": (None, [vp, vp, vp, vp, vp, vp]),
        "zlo_ac_set": (None, [vp, vp, vp, vp, fl]),
        "zlo_ac_get_moments": (None, [vp, vp, vp, vp, vp, vp, vp, vp]),
        "zlo_ac_record_obs": (None, [vp, vp, vp]),
        "zlo_ac_mean": (None, [vp, vp, vp]),
        "zlo_ac_value": (fl, [vp, vp]),
        "zlo_ac_entropy": (fl, [vp]),
        "zlo_ac_logp": (fl, [vp, vp, vp]),
        "zlo_ac_sample": (fl, [vp, vp, vp, vp, vp]),
        "zlo_ac_update": (None, [vp, C.c_longlong, C.c_int, C.c_int, vp, vp, vp, vp, vp, vp, vp,
                                 vp, C.POINTER(PpoCfg), C.c_int, C.c_int, vp]),
        "zlo_ac_minibatch_step": (None, [vp, C.c_longlong, C.c_int, C.c_int, vp, vp, vp, vp, vp,
                                         vp, vp, vp, vp, C.c_longlong, C.POINTER(PpoCfg),
                                         C.c_int, C.c_int, vp]),
        "zlo_tr_create": (vp, [vp, C.c_int, vp, C.c_int, vp, vp, vp, fl]),
        "zlo_tr_destroy": (None, [vp]),
        "zlo_tr_get": (None, [vp, vp, vp, vp, vp, vp]),
        "zlo_tr_get_moments": (None, [vp, vp, vp, vp, vp, vp, vp]),
        "zlo_tr_update": (None, [vp, C.c_longlong, C.c_int, C.c_int, vp, vp, vp, vp, vp, vp, vp,
                                 vp, C.POINTER(TrainerCfg), C.c_int, vp]),
        "zlo_adv_normalize": (None, [vp, C.c_longlong]),
        "zlo_norm_update_rows": (None, [vp, C.c_int, vp, C.c_int, C.c_longlong]),
        "zlo_pending_push_rows": (None, [vp, C.c_int, vp, C.c_int, C.c_longlong]),
        "zlo_norm_commit": (None, [vp, vp, C.c_int]),
        "zlo_norm_normalize_rows": (None, [vp, C.c_int, vp, C.c_int, C.c_longlong, vp, C.c_int]),
        "zlo_ppo_minibatch_grads": (None, [vp, C.c_int, vp, C.c_int, vp, vp, vp, C.c_longlong,
                                           vp, vp, vp, vp, vp, vp, vp, vp, vp, C.c_longlong, fl,
                                           fl, fl, C.c_int, vp, vp, vp, vp]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _p(a):
    return a.ctypes.data_as(vp) if a is not None else None


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def dims_arr(dims):
    return np.ascontiguousarray(dims, dtype=np.int32)


def lcg_units(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().zlo_lcg_units(seed, n, _p(out))
    return out


def lcg_gauss(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().zlo_lcg_gauss(seed, n, _p(out))
    return out


def powi(x: float, n: int) -> float:
    return lib().zlo_powi(x, n)


def packed_count(dims) -> int:
    return int(sum(dims[l + 1] * dims[l] + dims[l + 1] for l in range(len(dims) - 1)))


def mlp_init(dims, out_scale: float, seed: int) -> np.ndarray:
    d = dims_arr(dims)
    out = np.empty(packed_count(dims), np.float32)
    lib().zlo_mlp_init(_p(d), len(d), out_scale, seed, _p(out))
    return out


def mlp_forward(dims, params, x):
    """Per-row Mlp::forward over x [M x dims[0]] -> list of a[1..L] arrays."""
    d = dims_arr(dims)
    x = f32(x)
    M = x.shape[0]
    tot = sum(M * dims[l] for l in range(1, len(dims)))
    acts = np.empty(tot, np.float32)
    lib().zlo_mlp_forward(_p(d), len(d), _p(f32(params)), _p(x), M, _p(acts))
    out, o = [], 0
    for l in range(1, len(dims)):
        out.append(acts[o : o + M * dims[l]].reshape(M, dims[l]))
        o += M * dims[l]
    return out


def mlp_backward(dims, params, x, g_out, want_gin=False):
    """Sequential fold of Mlp::backward over the rows -> (packed grads, gin)."""
    d = dims_arr(dims)
    x = f32(x)
    M = x.shape[0]
    grads = np.empty(packed_count(dims), np.float32)
    gin = np.empty((M, dims[0]), np.float32) if want_gin else None
    lib().zlo_mlp_backward(_p(d), len(d), _p(f32(params)), _p(x), M, _p(f32(g_out)), _p(grads), _p(gin))
    return grads, gin


def mlpgrad_clip(dims, g, max_norm):
    g = f32(g).copy()
    d = dims_arr(dims)
    n = lib().zlo_mlpgrad_clip(_p(d), len(d), _p(g), max_norm)
    return g, n


def adam_flat(p, g, m, v, lr, bc1, bc2):
    p, m, v = f32(p).copy(), f32(m).copy(), f32(v).copy()
    g = f32(g)
    lib().zlo_adam_flat(_p(p), _p(g), _p(m), _p(v), p.size, lr, bc1, bc2)
    return p, m, v


def gae(rewards, values, dones, last_value, gamma, lam):
    r, v = f32(rewards), f32(values)
    d = np.ascontiguousarray(dones, dtype=np.uint8)
    adv = np.empty_like(r)
    ret = np.empty_like(r)
    lib().zlo_gae(_p(r), _p(v), _p(d), r.size, last_value, gamma, lam, _p(adv), _p(ret))
    return adv, ret


def adv_normalize(adv):
    a = f32(adv).copy()
    lib().zlo_adv_normalize(_p(a), a.size)
    return a


# Observation normaliser on flat states float[2 * dim + 1] = mean, m2, count
# (ppo.rs:104-206).
def norm_new(dim, unit_prior=True):
    """Normalizer::new (unit prior) or an empty PendingNorm."""
    st = np.zeros(2 * dim + 1, np.float32)
    if unit_prior:
        st[dim:] = 1.0
    return st


def norm_update(state, x):
    """Normalizer::update for each row of x [rows x dim] in order; returns the new state."""
    st, xa = f32(state).copy(), f32(x)
    dim = st.size // 2
    lib().zlo_norm_update_rows(_p(st), dim, _p(xa), xa.shape[1], xa.shape[0])
    return st


def pending_push(state, x):
    """PendingNorm::push for each row of x in order; returns the new pending state."""
    st, xa = f32(state).copy(), f32(x)
    dim = st.size // 2
    lib().zlo_pending_push_rows(_p(st), dim, _p(xa), xa.shape[1], xa.shape[0])
    return st


def norm_commit(state, pending):
    """Normalizer::commit; returns (state, pending) after the merge."""
    st, pd = f32(state).copy(), f32(pending).copy()
    lib().zlo_norm_commit(_p(st), _p(pd), st.size // 2)
    return st, pd


def norm_normalize(state, x):
    """Normalizer::normalize of each row of x [rows x dim]."""
    st, xa = f32(state), f32(x)
    out = np.empty_like(xa)
    lib().zlo_norm_normalize_rows(_p(st), st.size // 2, _p(xa), xa.shape[1], xa.shape[0], _p(out),
                                  xa.shape[1])
    return out


def minibatch_grads(actor_dims, critic_dims, actor, critic, log_std, batch: dict, idx, clip,
                    entropy_coef, value_coef, nthreads=1):
    """Fold of ppo.rs:406-462 over idx (obs already normalised) ->
    (actor grads, critic grads, log_std grads, [surrogate, value_loss, kl])."""
    a, c = dims_arr(actor_dims), dims_arr(critic_dims)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    ga = np.empty(packed_count(actor_dims), np.float32)
    gc = np.empty(packed_count(critic_dims), np.float32)
    gl = np.empty(actor_dims[-1], np.float32)
    st = np.empty(3, np.float32)
    mo = batch.get("mean_old")
    lib().zlo_ppo_minibatch_grads(
        _p(a), len(a), _p(c), len(c), _p(f32(actor)), _p(f32(critic)), _p(f32(log_std)),
        batch["obs"].shape[0], _p(f32(batch["obs"])), _p(f32(batch["critic_obs"])),
        _p(f32(batch["action"])), _p(f32(mo) if mo is not None else np.zeros_like(batch["action"])),
        _p(f32(batch["logp_old"])), _p(f32(batch["value_old"])), _p(f32(batch["adv"])),
        _p(f32(batch["ret"])), _p(idx), idx.size, clip, entropy_coef, value_coef, nthreads,
        _p(ga), _p(gc), _p(gl), _p(st),
    )
    return ga, gc, gl, st


class ActorCritic:
    """Handle to the oracle's ActorCritic (zealot-rl/src/ppo.rs:208-510)."""

    def __init__(self, actor_dims, critic_dims, init_noise_std, init_lr, seed=None, rng_state=None):
        """ActorCritic::new(.., &mut Lcg::new(seed)); pass rng_state (a 1-element
        uint64 array holding the Lcg state) instead to keep using that stream."""
        self.actor_dims = list(actor_dims)
        self.critic_dims = list(critic_dims)
        a, c = dims_arr(actor_dims), dims_arr(critic_dims)
        if rng_state is None:
            rng_state = np.array([int(seed) | 1], np.uint64)
        self.h = lib().zlo_ac_create(_p(a), len(a), _p(c), len(c), init_noise_std, init_lr,
                                     _p(rng_state))
        self.A = actor_dims[-1]

    def __del__(self):
        if getattr(self, "h", None):
            lib().zlo_ac_destroy(self.h)
            self.h = None

    def get(self):
        a = np.empty(packed_count(self.actor_dims), np.float32)
        c = np.empty(packed_count(self.critic_dims), np.float32)
        ls = np.empty(self.A, np.float32)
        lr = np.empty(1, np.float32)
        t = np.empty(1, np.int32)
        lib().zlo_ac_get(self.h, _p(a), _p(c), _p(ls), _p(lr), _p(t))
        return a, c, ls, float(lr[0]), int(t[0])

    def set(self, actor, critic, log_std, lr):
        lib().zlo_ac_set(self.h, _p(f32(actor)), _p(f32(critic)), _p(f32(log_std)), lr)

    def moments(self):
        """(m_actor, v_actor, m_critic, v_critic, m_logstd, v_logstd, [t_actor,
        t_critic, t_logstd]); the net moments are packed like the parameters."""
        na, nc = packed_count(self.actor_dims), packed_count(self.critic_dims)
        out = [np.empty(k, np.float32) for k in (na, na, nc, nc, self.A, self.A)]
        cnt = np.empty(3, np.int32)
        lib().zlo_ac_get_moments(self.h, *[_p(x) for x in out], _p(cnt))
        return out + [cnt]

    def mean(self, obs):
        out = np.empty(self.A, np.float32)
        lib().zlo_ac_mean(self.h, _p(f32(obs)), _p(out))
        return out

    def value(self, cobs):
        return lib().zlo_ac_value(self.h, _p(f32(cobs)))

    def entropy(self):
        return lib().zlo_ac_entropy(self.h)

    def logp(self, action, mean):
        return lib().zlo_ac_logp(self.h, _p(f32(action)), _p(f32(mean)))

    def sample(self, obs, rng_state: np.ndarray):
        a = np.empty(self.A, np.float32)
        m = np.empty(self.A, np.float32)
        lp = lib().zlo_ac_sample(self.h, _p(f32(obs)), _p(rng_state), _p(a), _p(m))
        return a, lp, m

    def record_obs(self, obs, cobs):
        lib().zlo_ac_record_obs(self.h, _p(f32(obs)), _p(f32(cobs)))

    def update(self, batch: dict, cfg: PpoCfg, nthreads=1, normalize_obs=True):
        """ActorCritic::update; batch['adv'] is normalised in place (returned)."""
        n = batch["obs"].shape[0]
        adv = f32(batch["adv"]).copy()
        stats = np.empty(5, np.float32)
        lib().zlo_ac_update(
            self.h, n, batch["obs"].shape[1], batch["critic_obs"].shape[1], _p(f32(batch["obs"])),
            _p(f32(batch["critic_obs"])), _p(f32(batch["action"])), _p(f32(batch["mean_old"])),
            _p(f32(batch["logp_old"])), _p(f32(batch["value_old"])), _p(adv), _p(f32(batch["ret"])),
            C.byref(cfg), nthreads, int(normalize_obs), _p(stats),
        )
        return stats, adv

    def minibatch_step(self, batch: dict, idx, cfg: PpoCfg, nthreads=1, normalize_obs=True):
        n = batch["obs"].shape[0]
        idx = np.ascontiguousarray(idx, dtype=np.int64)
        adv = f32(batch["adv"])
        stats = np.empty(5, np.float32)
        lib().zlo_ac_minibatch_step(
            self.h, n, batch["obs"].shape[1], batch["critic_obs"].shape[1], _p(f32(batch["obs"])),
            _p(f32(batch["critic_obs"])), _p(f32(batch["action"])), _p(f32(batch["mean_old"])),
            _p(f32(batch["logp_old"])), _p(f32(batch["value_old"])), _p(adv), _p(f32(batch["ret"])),
            _p(idx), idx.size, C.byref(cfg), nthreads, int(normalize_obs), _p(stats),
        )
        return stats


class Trainer:
    """Handle to the oracle's restatement of the GPU trainer's update."""

    def __init__(self, actor_dims, critic_dims, actor, critic, log_std, lr):
        self.actor_dims, self.critic_dims = list(actor_dims), list(critic_dims)
        a, c = dims_arr(actor_dims), dims_arr(critic_dims)
        self.h = lib().zlo_tr_create(_p(a), len(a), _p(c), len(c), _p(f32(actor)), _p(f32(critic)),
                                     _p(f32(log_std)), lr)
        self.A = actor_dims[-1]

    def __del__(self):
        if getattr(self, "h", None):
            lib().zlo_tr_destroy(self.h)
            self.h = None

    def get(self):
        a = np.empty(packed_count(self.actor_dims), np.float32)
        c = np.empty(packed_count(self.critic_dims), np.float32)
        ls = np.empty(self.A, np.float32)
        lr = np.empty(1, np.float32)
        g = np.empty(1, np.uint64)
        lib().zlo_tr_get(self.h, _p(a), _p(c), _p(ls), _p(lr), _p(g))
        return a, c, ls, float(lr[0]), int(g[0])

    def moments(self):
        na, nc = packed_count(self.actor_dims), packed_count(self.critic_dims)
        out = [np.empty(k, np.float32) for k in (na, na, nc, nc, self.A, self.A)]
        lib().zlo_tr_get_moments(self.h, *[_p(x) for x in out])
        return out

    def update(self, batch: dict, cfg: TrainerCfg, nthreads=1):
        n = batch["obs"].shape[0]
        stats = np.empty(7, np.float32)
        lib().zlo_tr_update(
            self.h, n, batch["obs"].shape[1], batch["critic_obs"].shape[1], _p(f32(batch["obs"])),
            _p(f32(batch["critic_obs"])), _p(f32(batch["action"])), _p(f32(batch["mean_old"])),
            _p(f32(batch["logp_old"])), _p(f32(batch["value_old"])), _p(f32(batch["adv"])),
            _p(f32(batch["ret"])), C.byref(cfg), nthreads, _p(stats),
        )
        return stats
