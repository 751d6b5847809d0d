"""GPU checks of checkpoint I/O (ActorCritic::save / load, zealot-rl/src/ppo.rs:
512-650) for the device-resident actor-critic.

* The reference's own round-trip test (actor_critic_save_load_roundtrips,
  ppo.rs:723-758) restated: an Lcg(7) ActorCritic [4, 8, 8, 2] / [6, 8, 1]
  with 20 recorded observation pairs, saved and loaded, gives bit-identical
  means, log_std and lr.
* The image holds exactly the reference's tensors (names, shapes, F32 values
  equal to the oracle's parameters and Welford states) and is byte-identical
  to what the safetensors serializer writes for them (the Python package,
  0.8.0; the reference links the Rust crate 0.4.5); an image written by that
  package loads.
* The optional Adam state round-trips; without it load resets Adam as the
  reference does."""

import os

import numpy as np
import pytest

from oracle import zl_oracle as zo
from zealot_amd import ZealotError, synth
from zealot_amd.rl import DeviceBatch, GpuActorCritic, PpoConfig, unpack

pytestmark = pytest.mark.gpu
safetensors_numpy = pytest.importorskip("safetensors.numpy")


def roundtrip_fixture():
    """ppo.rs:727-738: Lcg(7), ActorCritic::new(&[4,8,8,2], &[6,8,1], 0.3, 1e-3),
    obs_k[j] = sin(k + j), cobs_k[j] = cos(3k + j) for k < 20."""
    ad, cd = [4, 8, 8, 2], [6, 8, 1]
    ac = zo.ActorCritic(ad, cd, 0.3, 1e-3, seed=7)
    obs = np.array([[np.sin(np.float32(k + j)) for j in range(4)] for k in range(20)], np.float32)
    cobs = np.array([[np.cos(np.float32(k * 3 + j)) for j in range(6)] for k in range(20)], np.float32)
    for o, c in zip(obs, cobs):
        ac.record_obs(o, c)
    return ad, cd, ac, obs, cobs


def gpu_from_oracle(ctx, ac, ad, cd, obs, cobs, mb=64):
    actor, critic, log_std, lr, _ = ac.get()
    gac = GpuActorCritic(ctx, ad, cd, mb)
    gac.set_params(actor, critic, log_std, lr)
    # Same rows folded one at a time: the oracle ActorCritic's own states.
    gac.obs_norm.buf.upload(zo.norm_update(zo.norm_new(ad[0]), obs))
    gac.critic_norm.buf.upload(zo.norm_update(zo.norm_new(cd[0]), cobs))
    return gac, actor, critic, log_std, lr


def gpu_means(ctx, gac, probes):
    n, A = probes.shape[0], gac.action_dim
    act, lp, mean = ctx.alloc((n, A)), ctx.alloc(n), ctx.alloc((n, A))
    gac.act(ctx.to_device(probes), n, ctx.to_device(np.zeros((n, A), np.float32)), act, lp, mean=mean,
            obs_norm=gac.obs_norm)
    return mean.numpy()


def test_reference_roundtrip(ctx, tmp_path):
    ad, cd, ac, obs, cobs = roundtrip_fixture()
    gac, actor, critic, log_std, lr = gpu_from_oracle(ctx, ac, ad, cd, obs, cobs)
    probes = np.array([[np.tanh(np.float32(k * 7 + j)) for j in range(4)] for k in range(3)], np.float32)
    before = gpu_means(ctx, gac, probes)
    ref = np.stack([ac.mean(p) for p in probes])
    assert np.max(np.abs(before - ref)) <= 1e-6
    path = os.path.join(tmp_path, "roundtrip.safetensors")
    gac.save(path)
    gac2 = GpuActorCritic.load(ctx, path, 64)
    after = gpu_means(ctx, gac2, probes)
    assert np.array_equal(after, before)  # ppo.rs:748-753 (|a - b| < 1e-9)
    a2, c2, ls2, lr2 = gac2.get_params()
    assert np.array_equal(ls2, log_std) and lr2 == np.float32(lr)  # ppo.rs:755-756
    assert np.array_equal(a2, actor) and np.array_equal(c2, critic)
    assert np.array_equal(gac2.obs_norm.buf.numpy(), gac.obs_norm.buf.numpy())
    assert np.array_equal(gac2.critic_norm.buf.numpy(), gac.critic_norm.buf.numpy())
    gac.close()
    gac2.close()


def reference_dict(ad, cd, actor, critic, log_std, lr, st_o, st_c):
    t = {}
    for prefix, dims, packed in (("actor", ad, actor), ("critic", cd, critic)):
        ws, bs = unpack(dims, packed)
        for l, (w, b) in enumerate(zip(ws, bs)):
            t[f"{prefix}.w_{l}"] = np.ascontiguousarray(w, np.float32)
            t[f"{prefix}.b_{l}"] = np.ascontiguousarray(b, np.float32)
    t["log_std"] = np.asarray(log_std, np.float32)
    for name, st, d in (("obs_norm", st_o, ad[0]), ("critic_norm", st_c, cd[0])):
        t[f"{name}.mean"] = st[:d].copy()
        t[f"{name}.m2"] = st[d:2 * d].copy()
        t[f"{name}.count"] = st[2 * d:].copy()
    t["lr"] = np.array([lr], np.float32)
    return t


def test_image_matches_reference_layout(ctx):
    ad, cd, ac, obs, cobs = roundtrip_fixture()
    gac, actor, critic, log_std, lr = gpu_from_oracle(ctx, ac, ad, cd, obs, cobs)
    img = gac.save_bytes()
    st_o = zo.norm_update(zo.norm_new(ad[0]), obs)
    st_c = zo.norm_update(zo.norm_new(cd[0]), cobs)
    want = reference_dict(ad, cd, actor, critic, log_std, lr, st_o, st_c)
    got = safetensors_numpy.load(img)
    assert sorted(got) == sorted(want)
    for k in want:
        assert got[k].dtype == np.float32 and got[k].shape == want[k].shape, k
        assert np.array_equal(got[k], want[k]), k
    assert img == safetensors_numpy.save(want)  # byte-identical image
    gac.close()


def test_load_image_written_by_safetensors(ctx):
    ad, cd = synth.ACTOR_DIMS, synth.CRITIC_DIMS
    g = np.random.default_rng(5)
    actor = synth.kaiming_uniform_net(g, ad, 0.1)
    critic = synth.kaiming_uniform_net(g, cd, 0.1)
    log_std = g.uniform(-1, 0, ad[-1]).astype(np.float32)
    st_o = zo.norm_update(zo.norm_new(ad[0]), g.standard_normal((50, ad[0])).astype(np.float32))
    st_c = zo.norm_update(zo.norm_new(cd[0]), g.standard_normal((50, cd[0])).astype(np.float32))
    img = safetensors_numpy.save(reference_dict(ad, cd, actor, critic, log_std, 2.5e-4, st_o, st_c))
    gac = GpuActorCritic(ctx, ad, cd, 1024)
    gac.load_into(img)
    a, c, ls, lr = gac.get_params()
    assert np.array_equal(a, actor) and np.array_equal(c, critic) and np.array_equal(ls, log_std)
    assert lr == np.float32(2.5e-4)
    assert np.array_equal(gac.obs_norm.buf.numpy(), st_o)
    assert np.array_equal(gac.critic_norm.buf.numpy(), st_c)
    # A handle of other dims refuses the image.
    other = GpuActorCritic(ctx, [123, 64, 29], cd, 256)
    with pytest.raises(ZealotError):
        other.load_into(img)
    gac.close()
    other.close()


def _stepped_handle(ctx):
    """A handle whose Adam moments and counters are non-trivial: one update."""
    ad, cd = [11, 32, 16, 3], [11, 32, 16, 1]
    g = np.random.default_rng(9)
    gac = GpuActorCritic(ctx, ad, cd, 256)
    gac.set_params(synth.kaiming_uniform_net(g, ad, 0.1), synth.kaiming_uniform_net(g, cd, 0.1),
                   np.full(3, -0.5, np.float32), 1e-3)
    n = 1024
    f = lambda *s: g.standard_normal(s).astype(np.float32)  # noqa: E731
    db = DeviceBatch(ctx, f(n, 11), f(n, 11), f(n, 3), f(n, 3), f(n), f(n), f(n), f(n))
    gac.update(db, PpoConfig(epochs=2, minibatches=4))
    return gac, ad, cd


def test_optimizer_state_roundtrip(ctx):
    gac, ad, cd = _stepped_handle(ctx)
    m0 = gac.get_moments()
    t0 = gac.counters()
    assert t0[0] > 0 and any(np.any(x != 0) for x in m0)
    img = gac.save_bytes(with_optimizer=True)
    names = safetensors_numpy.load(img)
    assert names["adam.t"].dtype == np.int64 and int(names["adam.t"][0]) == t0[0]
    r = GpuActorCritic(ctx, ad, cd, 256)
    r.load_into(img, restore_optimizer=True)
    for a, b in zip(r.get_moments(), m0):
        assert np.array_equal(a, b)
    assert r.counters() == t0
    # Without restore (the reference's behaviour) Adam starts fresh.
    r.load_into(img, restore_optimizer=False)
    assert all(not np.any(x) for x in r.get_moments()) and r.counters() == (0, 0)
    # The reference-layout image (no optimizer) restores nothing either.
    r.load_into(gac.save_bytes(), restore_optimizer=True)
    assert all(not np.any(x) for x in r.get_moments())
    gac.close()
    r.close()


@pytest.mark.parametrize("field,value", [("adam.t", -1), ("adam.t", 2 ** 31), ("adam.gstep", -5)])
def test_out_of_range_counters_rejected(ctx, field, value):
    """An image whose Adam counters cannot be a real step count (t outside
    [0, 2^31 - 1], the i32 exponent of the bias correction; a negative gstep)
    is refused with ZL_ERR_INVALID before any state of the handle changes."""
    gac, ad, cd = _stepped_handle(ctx)
    tensors = dict(safetensors_numpy.load(gac.save_bytes(with_optimizer=True)))
    tensors[field] = np.array([value], np.int64)
    bad = safetensors_numpy.save(tensors)
    r = GpuActorCritic(ctx, ad, cd, 256)
    before = r.get_params(), r.get_moments(), r.counters()
    with pytest.raises(ZealotError) as ei:
        r.load_into(bad, restore_optimizer=True)
    assert ei.value.status == 1
    after = r.get_params(), r.get_moments(), r.counters()
    for x, y in zip(before[0][:3], after[0][:3]):
        assert np.array_equal(x, y)
    for x, y in zip(before[1], after[1]):
        assert np.array_equal(x, y)
    assert before[2] == after[2]
    gac.close()
    r.close()
