"""zealot-rl's learning-tier API on the MI355X path.

Names and argument meanings follow the reference (zealot-rl/src/net.rs,
ppo.rs; the GPU trainer's GpuMlp in src/bin/biped_train_gpu.rs); every call
goes through libzealot_hip.so's C ABI. Parameters cross as the packed
layout w[0], b[0], w[1], b[1], ... with w[l] row-major [dims[l+1] x dims[l]]
(zealot-rl/src/net.rs:30-34).
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _ffi
from .device import Context, DeviceBuffer, ZealotError


def _fptr(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


def packed_count(dims) -> int:
    return int(sum(dims[l + 1] * dims[l] + dims[l + 1] for l in range(len(dims) - 1)))


def unpack(dims, packed):
    """Packed params -> ([w[l] (out x in)], [b[l]])."""
    ws, bs, o = [], [], 0
    for l in range(len(dims) - 1):
        out, inp = dims[l + 1], dims[l]
        ws.append(np.asarray(packed[o : o + out * inp]).reshape(out, inp))
        o += out * inp
        bs.append(np.asarray(packed[o : o + out]))
        o += out
    return ws, bs


def pack(ws, bs) -> np.ndarray:
    parts = []
    for w, b in zip(ws, bs):
        parts.append(np.asarray(w, np.float32).ravel())
        parts.append(np.asarray(b, np.float32).ravel())
    return np.concatenate(parts).astype(np.float32)


@dataclass
class PpoConfig:
    """zealot-rl/src/ppo.rs:22-65 plus the switches between the reference's
    two update semantics (ActorCritic::update vs the GPU trainer)."""

    semantics: int = _ffi.ZL_SEMANTICS_ACTOR_CRITIC
    gamma: float = 0.99
    lam: float = 0.95
    clip: float = 0.2
    entropy_coef: float = 0.01
    value_coef: float = 1.0
    epochs: int = 5
    minibatches: int = 4
    max_grad_norm: float = 1.0
    desired_kl: float = 0.01
    lr_min: float = 1e-5
    lr_max: float = 1e-2
    adaptive_lr: bool = True
    early_stop: bool = False
    shuffle: bool = True
    normalize_adv: bool = True
    clamp_log_std: bool = True

    def to_c(self) -> _ffi.zl_ppo_config:
        return _ffi.zl_ppo_config(
            int(self.semantics), self.clip, self.entropy_coef, self.value_coef, int(self.epochs),
            int(self.minibatches), self.max_grad_norm, self.desired_kl, self.lr_min, self.lr_max,
            int(self.adaptive_lr), int(self.early_stop), int(self.shuffle),
            int(self.normalize_adv), int(self.clamp_log_std),
        )

    @staticmethod
    def gpu_trainer(**kw) -> "PpoConfig":
        """The GPU trainer's update (src/bin/biped_train_gpu.rs:53-75, :1164-1553)."""
        base = dict(
            semantics=_ffi.ZL_SEMANTICS_GPU_TRAINER, entropy_coef=0.01, value_coef=1.0,
            adaptive_lr=True, early_stop=True, shuffle=False, normalize_adv=True,
            clamp_log_std=True,
        )
        base.update(kw)
        return PpoConfig(**base)


@dataclass
class PpoStats:
    """zealot-rl/src/ppo.rs:90-102 (+ trainer epoch count / KL, pre-clip norms)."""

    kl: float
    surrogate: float
    value_loss: float
    entropy: float
    lr: float
    epochs_run: int
    last_kl: float
    grad_norm: tuple


MLP_FEATURE_MAJOR = 1  # ZL_MLP_FEATURE_MAJOR


class GpuMlp:
    """Device-resident MLP (the GpuMlp of src/bin/biped_train_gpu.rs:316-564).
    feature_major: inputs, outputs and output gradients are [dim x rows]
    with a feature stride (GpuMlp's a[0], a[L], delta[L-1]); otherwise
    [rows x dim] with a row stride."""

    def __init__(self, ctx: Context, dims, batch: int, feature_major: bool = False):
        self.ctx = ctx
        self.dims = [int(d) for d in dims]
        self.batch = int(batch)
        self.fm = bool(feature_major)
        d = (C.c_int * len(self.dims))(*self.dims)
        h = C.c_void_p()
        flags = MLP_FEATURE_MAJOR if self.fm else 0
        ctx.check(ctx.lib.zl_mlp_create_ex(ctx.h, d, len(self.dims), self.batch, flags, C.byref(h)),
                  "zl_mlp_create_ex")
        self.h = h
        self.n_params = int(ctx.lib.zl_mlp_num_params(h))

    def write_weights(self, packed):
        a = np.ascontiguousarray(packed, np.float32)
        assert a.size == self.n_params
        self.ctx.check(self.ctx.lib.zl_mlp_write_weights(self.h, _fptr(a)), "zl_mlp_write_weights")

    def read_weights(self) -> np.ndarray:
        out = np.empty(self.n_params, np.float32)
        self.ctx.check(self.ctx.lib.zl_mlp_read_weights(self.h, _fptr(out)), "zl_mlp_read_weights")
        return out

    def forward(self, x: DeviceBuffer, rows: int, ldx: int | None = None):
        if ldx is None:
            ldx = rows if self.fm else self.dims[0]
        self.ctx.check(self.ctx.lib.zl_mlp_forward(self.h, x.p, ldx, rows), "zl_mlp_forward")

    def output(self, rows: int) -> np.ndarray:
        """The last forward's output as a host [rows x dims[-1]] array (either layout)."""
        ld = C.c_int()
        p = self.ctx.lib.zl_mlp_output(self.h, C.byref(ld))
        shape = (self.dims[-1], ld.value) if self.fm else (rows, ld.value)
        buf = np.empty(shape, np.float32)
        self.ctx.check(
            self.ctx.lib.zl_download(self.ctx.h, _fptr(buf), C.c_void_p(p), buf.nbytes), "download"
        )
        return buf[:, :rows].T.copy() if self.fm else buf[:, : self.dims[-1]].copy()

    def backward(self, g_out: DeviceBuffer, ld_g: int | None = None, rows: int | None = None):
        if ld_g is None:
            ld_g = (rows if rows is not None else self.batch) if self.fm else self.dims[-1]
        self.ctx.check(self.ctx.lib.zl_mlp_backward(self.h, g_out.p, ld_g), "zl_mlp_backward")

    def read_grads(self) -> np.ndarray:
        out = np.empty(self.n_params, np.float32)
        self.ctx.check(self.ctx.lib.zl_mlp_read_grads(self.h, _fptr(out)), "zl_mlp_read_grads")
        return out

    def adam(self, lr: float, bc1: float, bc2: float):
        self.ctx.check(self.ctx.lib.zl_mlp_adam(self.h, lr, bc1, bc2), "zl_mlp_adam")

    def read_moments(self):
        m = np.empty(self.n_params, np.float32)
        v = np.empty(self.n_params, np.float32)
        self.ctx.check(self.ctx.lib.zl_mlp_read_moments(self.h, _fptr(m), _fptr(v)), "read_moments")
        return m, v

    def write_moments(self, m, v):
        m = np.ascontiguousarray(m, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self.ctx.check(self.ctx.lib.zl_mlp_write_moments(self.h, _fptr(m), _fptr(v)), "write_moments")

    def close(self):
        if self.h:
            self.ctx.lib.zl_mlp_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            if self.ctx.h:
                self.close()
        except Exception:
            pass


def _dptr(x):
    """Device pointer of a DeviceBuffer, or a raw pointer (DeviceBuffer.offset)."""
    return x.p if isinstance(x, DeviceBuffer) else x


class GpuNormalizer:
    """zealot-rl's running observation Normalizer (ppo.rs:104-206) with its
    Welford state in HBM as float[2 * dim + 1] = mean, m2, count. update /
    commit / normalize are kernels on the context's stream."""

    def __init__(self, ctx: Context, dim: int, unit_prior: bool = True):
        self.ctx = ctx
        self.dim = int(dim)
        self.buf = ctx.alloc(2 * self.dim + 1)
        ctx.check(ctx.lib.zl_norm_reset(ctx.h, self.buf.p, self.dim, int(unit_prior)), "zl_norm_reset")

    @classmethod
    def from_state(cls, ctx: Context, mean, m2, count: float) -> "GpuNormalizer":
        """Normalizer::from_state (ppo.rs:150-153)."""
        n = cls(ctx, len(mean))
        st = np.concatenate([np.asarray(mean, np.float32), np.asarray(m2, np.float32),
                             np.array([count], np.float32)])
        n.buf.upload(st)
        return n

    def state(self):
        """Normalizer::state (ppo.rs:156-158): host copies (mean, m2, count)."""
        st = self.buf.numpy()
        return st[:self.dim].copy(), st[self.dim:2 * self.dim].copy(), float(st[2 * self.dim])

    def update(self, x: DeviceBuffer, rows: int, ld: int | None = None):
        """Normalizer::update (ppo.rs:161-168) for rows of x, in order."""
        self.ctx.check(self.ctx.lib.zl_norm_update(self.ctx.h, self.buf.p, self.dim, _dptr(x),
                                                   int(ld or self.dim), int(rows)), "zl_norm_update")

    def commit(self, pending: "GpuPendingNorm"):
        """Normalizer::commit (ppo.rs:179-195): merge, then empty `pending`."""
        self.ctx.check(self.ctx.lib.zl_norm_commit(self.ctx.h, self.buf.p, pending.buf.p, self.dim),
                       "zl_norm_commit")

    def normalize(self, x: DeviceBuffer, rows: int, out: DeviceBuffer, ld_x: int | None = None,
                  ld_out: int | None = None):
        """Normalizer::normalize (ppo.rs:198-205) of each row of x into out."""
        self.ctx.check(self.ctx.lib.zl_norm_normalize(self.ctx.h, self.buf.p, self.dim, _dptr(x),
                                                      int(ld_x or self.dim), int(rows), _dptr(out),
                                                      int(ld_out or self.dim)), "zl_norm_normalize")


class GpuPendingNorm:
    """PendingNorm (ppo.rs:115-137): Welford statistics gathered while the
    live transform is frozen, merged by GpuNormalizer.commit."""

    def __init__(self, ctx: Context, dim: int):
        self.ctx = ctx
        self.dim = int(dim)
        self.buf = ctx.alloc(2 * self.dim + 1)
        ctx.check(ctx.lib.zl_norm_reset(ctx.h, self.buf.p, self.dim, 0), "zl_norm_reset")

    def push(self, x: DeviceBuffer, rows: int, ld: int | None = None):
        """PendingNorm::push for rows of x, in order."""
        self.ctx.check(self.ctx.lib.zl_norm_update(self.ctx.h, self.buf.p, self.dim, _dptr(x),
                                                   int(ld or self.dim), int(rows)), "zl_norm_update")

    @property
    def count(self) -> float:
        return float(self.buf.numpy()[2 * self.dim])


def checkpoint_dims(data: bytes):
    """(actor dims, critic dims) of a checkpoint image (host only)."""
    lib = _ffi.load_library()
    cap = 64
    ad, cd = (C.c_int * cap)(), (C.c_int * cap)()
    na, nc = C.c_int(), C.c_int()
    st = lib.zl_checkpoint_dims(data, len(data), ad, C.byref(na), cd, C.byref(nc), cap)
    if st != _ffi.ZL_OK:
        raise ZealotError(st, "zl_checkpoint_dims: " + lib.zl_global_error().decode(errors="replace"))
    return list(ad[:na.value]), list(cd[:nc.value])


class GpuActorCritic:
    """The ActorCritic of zealot-rl/src/ppo.rs:208-229 resident on one MI355X:
    actor, critic, log_std and all Adam state in one flat HBM buffer, updated
    by zl_ppo_update with no host round trip inside the update."""

    def __init__(self, ctx: Context, actor_dims, critic_dims, minibatch_rows: int):
        self.ctx = ctx
        self.actor_dims = [int(d) for d in actor_dims]
        self.critic_dims = [int(d) for d in critic_dims]
        self.action_dim = self.actor_dims[-1]
        ad = (C.c_int * len(self.actor_dims))(*self.actor_dims)
        cd = (C.c_int * len(self.critic_dims))(*self.critic_dims)
        h = C.c_void_p()
        ctx.check(
            ctx.lib.zl_ppo_create(ctx.h, ad, len(ad), cd, len(cd), int(minibatch_rows), C.byref(h)),
            "zl_ppo_create",
        )
        self.h = h
        self.na = packed_count(self.actor_dims)
        self.nc = packed_count(self.critic_dims)
        # Running normalisers of the policy and critic observations (ppo.rs:217-220).
        self.obs_norm = GpuNormalizer(ctx, self.actor_dims[0])
        self.critic_norm = GpuNormalizer(ctx, self.critic_dims[0])

    def record_obs(self, obs, critic_obs, rows: int, ld_obs: int | None = None,
                   ld_critic_obs: int | None = None):
        """ActorCritic::record_obs (ppo.rs:276-279) for `rows` observation pairs, in order."""
        self.obs_norm.update(obs, rows, ld_obs)
        self.critic_norm.update(critic_obs, rows, ld_critic_obs)

    def save(self, path: str, with_optimizer: bool = False):
        """ActorCritic::save (ppo.rs:512-570) to a .safetensors file; with_optimizer
        adds the Adam moments and counters (which the reference drops)."""
        self.ctx.check(self.ctx.lib.zl_ppo_save(self.h, self.obs_norm.buf.p, self.critic_norm.buf.p,
                                                int(with_optimizer), str(path).encode()), "zl_ppo_save")

    def save_bytes(self, with_optimizer: bool = False) -> bytes:
        n = C.c_size_t()
        lib, on, cn = self.ctx.lib, self.obs_norm.buf.p, self.critic_norm.buf.p
        self.ctx.check(lib.zl_ppo_save_bytes(self.h, on, cn, int(with_optimizer), None, 0, C.byref(n)),
                       "zl_ppo_save_bytes")
        buf = C.create_string_buffer(n.value)
        self.ctx.check(lib.zl_ppo_save_bytes(self.h, on, cn, int(with_optimizer), buf, n.value, C.byref(n)),
                       "zl_ppo_save_bytes")
        return buf.raw[:n.value]

    def load_into(self, data: bytes, restore_optimizer: bool = False):
        """ActorCritic::load_from_bytes into this handle (dims must match)."""
        self.ctx.check(self.ctx.lib.zl_ppo_load_bytes(self.h, self.obs_norm.buf.p, self.critic_norm.buf.p,
                                                      int(restore_optimizer), data, len(data)),
                       "zl_ppo_load_bytes")

    @classmethod
    def load(cls, ctx: Context, path: str, minibatch_rows: int,
             restore_optimizer: bool = False) -> "GpuActorCritic":
        """ActorCritic::load (ppo.rs:572-650): dims from the file's weight shapes."""
        with open(path, "rb") as f:
            data = f.read()
        ad, cd = checkpoint_dims(data)
        ac = cls(ctx, ad, cd, minibatch_rows)
        ac.load_into(data, restore_optimizer)
        return ac

    def set_params(self, actor, critic, log_std, lr: float):
        a = np.ascontiguousarray(actor, np.float32)
        c = np.ascontiguousarray(critic, np.float32)
        l = np.ascontiguousarray(log_std, np.float32)
        assert a.size == self.na and c.size == self.nc and l.size == self.action_dim
        self.ctx.check(self.ctx.lib.zl_ppo_set_params(self.h, _fptr(a), _fptr(c), _fptr(l), lr), "set_params")

    def get_params(self):
        a = np.empty(self.na, np.float32)
        c = np.empty(self.nc, np.float32)
        l = np.empty(self.action_dim, np.float32)
        lr = C.c_float()
        self.ctx.check(
            self.ctx.lib.zl_ppo_get_params(self.h, _fptr(a), _fptr(c), _fptr(l), C.byref(lr)), "get_params"
        )
        return a, c, l, float(lr.value)

    def get_moments(self):
        out = [np.empty(n, np.float32) for n in (self.na, self.na, self.nc, self.nc, self.action_dim, self.action_dim)]
        self.ctx.check(self.ctx.lib.zl_ppo_get_moments(self.h, *[_fptr(x) for x in out]), "get_moments")
        return out

    def reset_optimizer(self):
        self.ctx.check(self.ctx.lib.zl_ppo_reset_optimizer(self.h), "reset_optimizer")

    def counters(self):
        t = C.c_int()
        g = C.c_ulonglong()
        self.ctx.check(self.ctx.lib.zl_ppo_get_counters(self.h, C.byref(t), C.byref(g)), "counters")
        return int(t.value), int(g.value)

    def update(self, batch: "DeviceBatch", cfg: PpoConfig) -> PpoStats:
        st = _ffi.zl_ppo_stats()
        b = batch.to_c()
        c = cfg.to_c()
        self.ctx.check(self.ctx.lib.zl_ppo_update(self.h, C.byref(b), C.byref(c), C.byref(st)), "zl_ppo_update")
        return PpoStats(st.kl, st.surrogate, st.value_loss, st.entropy, st.lr, st.epochs_run,
                        st.last_kl, tuple(st.grad_norm))

    def graph_info(self):
        """(captured update graphs so far, host ms of the last capture + instantiation)."""
        n, ms = C.c_longlong(), C.c_double()
        self.ctx.check(self.ctx.lib.zl_ppo_graph_info(self.h, C.byref(n), C.byref(ms)), "graph_info")
        return int(n.value), float(ms.value)

    def minibatch_grads(self, batch: "DeviceBatch", cfg: PpoConfig, row0: int, rows: int,
                        perm: DeviceBuffer | None = None):
        """Gradients of one minibatch (no clip / Adam): returns
        (actor, critic, log_std packed grads, {surrogate, value_loss, kl})."""
        st = (C.c_float * 3)()
        b = batch.to_c()
        c = cfg.to_c()
        self.ctx.check(
            self.ctx.lib.zl_ppo_minibatch_grads(self.h, C.byref(b), C.byref(c), row0, rows,
                                                perm.p if perm is not None else None, st),
            "zl_ppo_minibatch_grads",
        )
        ga = np.empty(self.na, np.float32)
        gc = np.empty(self.nc, np.float32)
        gl = np.empty(self.action_dim, np.float32)
        self.ctx.check(self.ctx.lib.zl_ppo_get_grads(self.h, _fptr(ga), _fptr(gc), _fptr(gl)), "get_grads")
        return ga, gc, gl, dict(surrogate=st[0], value_loss=st[1], kl=st[2])

    def act(self, obs, n: int, eps, action, logp, mean=None, value=None, critic_obs=None,
            obs_norm: "GpuNormalizer | None" = None, critic_norm: "GpuNormalizer | None" = None,
            ld_obs: int | None = None, ld_critic_obs: int | None = None, ld_mean: int | None = None):
        """One rollout step for n envs (GpuPolicy::forward, src/biped/gpu_policy.rs:
        210-248, with the trainer's sampling, src/bin/biped_train_gpu.rs:910-930):
        normalise, actor mean, action = mean + exp(log_std) * eps, logp, and
        (when `value` is given) the critic value, all on the device."""
        ctx = self.ctx
        ctx.check(ctx.lib.zl_ppo_act(
            self.h, obs_norm.buf.p if obs_norm else None, _dptr(obs), int(ld_obs or self.actor_dims[0]),
            critic_norm.buf.p if critic_norm else None, _dptr(critic_obs) if critic_obs is not None else None,
            int(ld_critic_obs or self.critic_dims[0]), int(n), _dptr(eps), _dptr(action), _dptr(logp),
            _dptr(mean) if mean is not None else None, int(ld_mean or self.action_dim),
            _dptr(value) if value is not None else None), "zl_ppo_act")

    def values(self, critic_obs: DeviceBuffer, n: int, out: DeviceBuffer, ld: int | None = None):
        ld = self.critic_dims[0] if ld is None else ld
        self.ctx.check(self.ctx.lib.zl_ppo_values(self.h, critic_obs.p, ld, n, out.p), "zl_ppo_values")

    def actor_mean(self, obs: DeviceBuffer, n: int, out: DeviceBuffer, ld: int | None = None,
                   ld_out: int | None = None):
        ld = self.actor_dims[0] if ld is None else ld
        ld_out = self.action_dim if ld_out is None else ld_out
        self.ctx.check(self.ctx.lib.zl_ppo_actor_mean(self.h, obs.p, ld, n, out.p, ld_out), "actor_mean")

    def close(self):
        if self.h:
            self.ctx.lib.zl_ppo_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            if self.ctx.h:
                self.close()
        except Exception:
            pass


class DeviceBatch:
    """A rollout batch resident on the device (structure of arrays, batch
    order). Host arrays are [n x dim]; with feature_major=True the matrix
    fields are stored as the reference trainer stages them, [dim x n]
    (src/bin/biped_train_gpu.rs:1029-1030,1053-1056), with stride n."""

    def __init__(self, ctx: Context, obs, critic_obs, action, mean_old, logp_old, value_old, adv, ret,
                 feature_major: bool = False, pad: int = 0):
        """pad > 0 stores each matrix field with its stride `pad` elements past
        the rows it holds (feature-major: [dim x (n + pad)], as a trainer
        tensor sized for a larger capacity; batch-major: [n x (dim + pad)]);
        the padding holds NaN, which the update never reads."""
        self.ctx = ctx
        self.n = int(np.asarray(obs).shape[0])
        self.feature_major = bool(feature_major)
        self.pad = int(pad)

        def mat(x):
            x = np.asarray(x, np.float32)
            y = x.T if feature_major else x
            if self.pad:
                z = np.full((y.shape[0], y.shape[1] + self.pad), np.nan, np.float32)
                z[:, :y.shape[1]] = y
                y = z
            return ctx.to_device(np.ascontiguousarray(y), np.float32)

        self.obs = mat(obs)
        self.critic_obs = self.obs if critic_obs is obs else mat(critic_obs)
        self.action = mat(action)
        self.mean_old = mat(mean_old) if mean_old is not None else None
        self.logp_old = ctx.to_device(logp_old, np.float32)
        self.value_old = ctx.to_device(value_old, np.float32)
        self.adv = ctx.to_device(adv, np.float32)
        self.ret = ctx.to_device(ret, np.float32)
        self.od = np.asarray(obs).shape[1]
        self.cd = np.asarray(critic_obs).shape[1]
        self.ad = np.asarray(action).shape[1]

    def to_c(self) -> _ffi.zl_batch:
        fm = self.feature_major
        ld = (lambda d: self.n + self.pad) if fm else (lambda d: d + self.pad)
        bits = (_ffi.ZL_FM_OBS | _ffi.ZL_FM_CRITIC_OBS | _ffi.ZL_FM_ACTION | _ffi.ZL_FM_MEAN_OLD) if fm else 0
        return _ffi.zl_batch(
            self.n, self.obs.ptr, ld(self.od), self.critic_obs.ptr, ld(self.cd), self.action.ptr,
            ld(self.ad), self.mean_old.ptr if self.mean_old is not None else None, ld(self.ad),
            self.logp_old.ptr, self.value_old.ptr, self.adv.ptr, self.ret.ptr, bits,
        )
