"""GPU parity of the device observation normaliser (Normalizer / PendingNorm,
zealot-rl/src/ppo.rs:104-206) against the CPU oracle.

normalize and commit repeat the reference's operation order and are compared
bit for bit (same input state on both sides). update / push fold rows in
chunks (two-pass chunk statistics, Chan merges in row order) instead of one
row at a time, so mean and m2 are compared to the float64 closed form and to
the oracle's one-at-a-time fold at fp32 tolerance: mean within 1e-5 of the
largest |mean| (or 1e-6 absolute for near-zero means), m2 within 1e-4
relative per component. count is compared exactly."""

import numpy as np
import pytest

from conftest import rel_amax
from oracle import zl_oracle as zo
from zealot_amd.rl import GpuNormalizer, GpuPendingNorm

pytestmark = pytest.mark.gpu

MEAN_TOL = 1e-5
M2_TOL = 1e-4


def obs_rows(seed, n, dim):
    g = np.random.default_rng(seed)
    scale = g.uniform(0.1, 3.0, dim)
    shift = g.uniform(-4.0, 4.0, dim)
    return (g.standard_normal((n, dim)) * scale + shift).astype(np.float32)


def flat(norm):
    return norm.buf.numpy().copy()


def check_stats(got, ref, dim, what):
    assert got[2 * dim] == ref[2 * dim], (what, got[2 * dim], ref[2 * dim])
    e_mean = float(np.max(np.abs(got[:dim].astype(np.float64) - ref[:dim])))
    scale = max(float(np.max(np.abs(ref[:dim]))), 0.1)
    e_m2 = float(np.max(np.abs(got[dim:2 * dim].astype(np.float64) / ref[dim:2 * dim] - 1.0)))
    print(f"[gpu] {what}: mean err {e_mean / scale:.2e}, m2 rel err {e_m2:.2e}", flush=True)
    assert e_mean <= MEAN_TOL * scale, (what, e_mean)
    assert e_m2 <= M2_TOL, (what, e_m2)


def closed_form(prior, x):
    """Chan merge (float64) of a state with the rows of x."""
    dim = prior.size // 2
    n1 = float(prior[2 * dim])
    d = x.astype(np.float64)
    n2 = d.shape[0]
    xbar = d.mean(0)
    q = ((d - xbar) ** 2).sum(0)
    if n1 == 0:
        return np.concatenate([xbar, q, [n2]])
    delta = xbar - prior[:dim]
    tot = n1 + n2
    return np.concatenate([prior[:dim] + delta * n2 / tot,
                           prior[dim:2 * dim] + q + delta ** 2 * n1 * n2 / tot, [tot]])


def test_reset_states(ctx):
    n = GpuNormalizer(ctx, 123)
    assert np.array_equal(flat(n), zo.norm_new(123))
    p = GpuPendingNorm(ctx, 123)
    assert np.array_equal(flat(p), zo.norm_new(123, unit_prior=False)) and p.count == 0.0


@pytest.mark.parametrize("dim,rows", [(123, 5000), (265, 3001), (64, 1), (1, 777), (4096, 33)])
def test_normalize_bit_exact(ctx, dim, rows):
    st = zo.norm_update(zo.norm_new(dim), obs_rows(dim, 300, dim))
    st[dim] = 0.0  # component 0: variance floor
    x = (obs_rows(dim + 1, rows, dim) * np.float32(2.0)).astype(np.float32)
    norm = GpuNormalizer(ctx, dim)
    norm.buf.upload(st)
    dx = ctx.to_device(x)
    out = ctx.alloc((rows, dim))
    norm.normalize(dx, rows, out)
    ref = zo.norm_normalize(st, x)
    got = out.numpy()
    print(f"[gpu] normalize {rows} x {dim}: {int(np.sum(got != ref))} of {got.size} differ", flush=True)
    assert np.array_equal(got, ref)
    # In place.
    norm.normalize(dx, rows, dx)
    assert np.array_equal(dx.numpy(), ref)


def test_normalize_strided(ctx):
    """Rows inside wider buffers (ld_x = 130, ld_out = 128 for dim 123)."""
    dim, rows = 123, 1000
    st = zo.norm_update(zo.norm_new(dim), obs_rows(5, 400, dim))
    x = obs_rows(6, rows, 130)
    norm = GpuNormalizer.from_state(ctx, st[:dim], st[dim:2 * dim], float(st[2 * dim]))
    out = ctx.alloc((rows, 128))
    out.upload(np.full((rows, 128), 7.0, np.float32))
    norm.normalize(ctx.to_device(x), rows, out, ld_x=130, ld_out=128)
    got = out.numpy()
    assert np.array_equal(got[:, :dim], zo.norm_normalize(st, x[:, :dim]))
    assert np.all(got[:, dim:] == 7.0)  # padding columns untouched


@pytest.mark.parametrize("dim,rows", [(123, 1), (123, 255), (123, 256), (123, 257), (265, 4096),
                                      (7, 98_304), (123, 98_304)])
def test_update_vs_oracle(ctx, dim, rows):
    x = obs_rows(rows + dim, rows, dim)
    norm = GpuNormalizer(ctx, dim)
    norm.update(ctx.to_device(x), rows)
    got = flat(norm)
    prior = zo.norm_new(dim)
    ref = zo.norm_update(prior, x)
    check_stats(got, closed_form(prior, x), dim, f"update {rows} x {dim} vs f64")
    check_stats(got, ref, dim, f"update {rows} x {dim} vs oracle")


def test_update_sequence_and_empty(ctx):
    """Several updates in a row (the state's count grows between chunks) and
    a zero-row update (no-op)."""
    dim = 123
    norm = GpuNormalizer(ctx, dim)
    ref = zo.norm_new(dim)
    for i, rows in enumerate([4096, 100, 0, 3000, 1]):
        x = obs_rows(40 + i, rows, dim)
        if rows:
            norm.update(ctx.to_device(x), rows)
        else:
            ctx.check(ctx.lib.zl_norm_update(ctx.h, norm.buf.p, dim, None, dim, 0), "zl_norm_update")
        ref = zo.norm_update(ref, x)
    check_stats(flat(norm), ref, dim, "update sequence")


def test_commit_bit_exact(ctx):
    dim = 265
    base = zo.norm_update(zo.norm_new(dim), obs_rows(50, 700, dim))
    pend = zo.pending_push(zo.norm_new(dim, False), obs_rows(51, 900, dim) + np.float32(0.7))
    norm = GpuNormalizer(ctx, dim)
    norm.buf.upload(base)
    pn = GpuPendingNorm(ctx, dim)
    pn.buf.upload(pend)
    norm.commit(pn)
    st_ref, pd_ref = zo.norm_commit(base, pend)
    assert np.array_equal(flat(norm), st_ref)
    assert np.array_equal(flat(pn), pd_ref) and pn.count == 0.0
    norm.commit(pn)  # empty pending: no-op
    assert np.array_equal(flat(norm), st_ref)


def test_frozen_rollout_cycle(ctx):
    """The trainer's frozen-normaliser iteration (src/bin/biped_train_gpu.rs:
    800-801, 891-899, 1045-1052): every step's env rows are pushed to a
    pending state, the batch is normalised with the frozen transform, then the
    pending statistics are committed."""
    dim, n_env, steps = 123, 4096, 24
    live = GpuNormalizer(ctx, dim)
    pend = GpuPendingNorm(ctx, dim)
    ref_live, ref_pend = zo.norm_new(dim), zo.norm_new(dim, False)
    for it in range(2):
        obs = obs_rows(100 + it, steps * n_env, dim)
        dobs = ctx.to_device(obs)
        for t in range(steps):
            pend.push(dobs.offset(t * n_env * dim), n_env)
            ref_pend = zo.pending_push(ref_pend, obs[t * n_env:(t + 1) * n_env])
        check_stats(flat(pend), ref_pend, dim, f"iteration {it} pending")
        out = ctx.alloc((steps * n_env, dim))
        live.normalize(dobs, steps * n_env, out)
        st = flat(live)
        assert np.array_equal(out.numpy(), zo.norm_normalize(st, obs))  # same frozen state: exact
        live.commit(pend)
        ref_live, ref_pend = zo.norm_commit(ref_live, ref_pend)
        assert pend.count == 0.0
        check_stats(flat(live), ref_live, dim, f"iteration {it} committed")


def test_count_saturates_like_f32(ctx):
    dim = 3
    st = zo.norm_new(dim)
    st[2 * dim] = np.float32(2 ** 24 - 2)
    norm = GpuNormalizer(ctx, dim)
    norm.buf.upload(st)
    norm.update(ctx.to_device(obs_rows(9, 5, dim)), 5)
    assert flat(norm)[2 * dim] == np.float32(2 ** 24)


def test_bad_arguments_rejected(ctx):
    from zealot_amd import ZealotError
    norm = GpuNormalizer(ctx, 8)
    x = ctx.alloc((4, 8))
    with pytest.raises(ZealotError):
        norm.normalize(x, 4, x, ld_x=8, ld_out=9)  # in place with different strides
    with pytest.raises(ZealotError):
        norm.update(x, 4, ld=7)
    with pytest.raises(ZealotError):
        GpuNormalizer(ctx, 5000)
