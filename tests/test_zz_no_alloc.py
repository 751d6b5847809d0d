"""zl_grad_clip_scale_noalloc (the allocation-free variant of the device
grad-norm clip, partials in a static per-GPU device array) against
zl_grad_clip_scale through the C ABI: bit-identical scale and norm on two
calls in a row, the second with a smaller input, and an input beyond the
static array refused with ZL_ERR_INVALID."""

import ctypes as C

import numpy as np
import pytest

from zealot_amd import _ffi, synth

pytestmark = pytest.mark.gpu


def _tensors(buf, sizes):
    offs = np.concatenate([[0], np.cumsum(sizes)])
    arr = (_ffi.zl_tensor * len(sizes))(*[_ffi.zl_tensor(buf.offset(int(o)), int(s))
                                          for o, s in zip(offs[:-1], sizes)])
    return arr, len(sizes)


def _both(ctx, arr, count, max_norm):
    out = []
    for fn in (ctx.lib.zl_grad_clip_scale, ctx.lib.zl_grad_clip_scale_noalloc):
        scale, norm = ctx.alloc(1), ctx.alloc(1)
        ctx.check(fn(ctx.h, arr, count, max_norm, scale.p, norm.p), "clip scale")
        out.append((scale.numpy()[0], norm.numpy()[0]))
    return out


def test_noalloc_clip_scale_matches(ctx):
    g = np.random.default_rng(12)
    # The trainer's 17 gradient tensors at the headline nets (459,323 floats).
    sizes = []
    for dims in (synth.ACTOR_DIMS, synth.CRITIC_DIMS):
        sizes += [dims[l + 1] * dims[l] for l in range(len(dims) - 1)]
        sizes += [dims[l + 1] for l in range(len(dims) - 1)]
    sizes.append(29)
    grads = ctx.to_device((g.standard_normal(sum(sizes)) * 1e-2).astype(np.float32))
    arr, count = _tensors(grads, sizes)
    first = _both(ctx, arr, count, 1.0)
    print(f"[gpu] noalloc clip scale, 459,323 floats: {first}", flush=True)
    assert first[0] == first[1] and first[0][0] < 1.0
    # A smaller second call: 3 tensors, 5,000 floats, clip inactive.
    small = ctx.to_device((g.standard_normal(5000) * 1e-3).astype(np.float32))
    arr2, count2 = _tensors(small, [1000, 3000, 1000])
    second = _both(ctx, arr2, count2, 1.0)
    assert second[0] == second[1] and second[0][0] == 1.0
    ref = np.sqrt(np.sum(small.numpy().astype(np.float64) ** 2))
    assert abs(second[1][1] - ref) <= 1e-6 * ref


def test_noalloc_clip_scale_refuses_oversize(ctx):
    """16,384 partials of 2,048 floats fit; one more chunk is refused before
    any launch (the buffer is real: 16,385 x 2,048 floats)."""
    n = 16385 * 2048
    big = ctx.alloc(n)
    scale = ctx.alloc(1)
    arr = (_ffi.zl_tensor * 1)(_ffi.zl_tensor(big.p, n))
    st = ctx.lib.zl_grad_clip_scale_noalloc(ctx.h, arr, 1, 1.0, scale.p, None)
    assert st == _ffi.ZL_ERR_INVALID
    assert b"static scratch" in ctx.lib.zl_last_error(ctx.h)
    # The largest accepted input still works and matches the allocating call.
    ok = (_ffi.zl_tensor * 1)(_ffi.zl_tensor(big.p, 16384 * 2048))
    big.upload(np.full(n, 1e-4, np.float32))
    res = _both(ctx, ok, 1, 1.0)
    assert res[0] == res[1]


def test_noalloc_slots_per_context(ctx):
    """Every context claims one of the 4 static slots at zl_init: with 4
    contexts alive (the session's and 3 more) a fifth context's call is
    refused with ZL_ERR_INVALID, naming the slots; destroying one context
    frees its slot for the next. Each context's result matches its own
    allocating call."""
    from zealot_amd import Context

    g = np.random.default_rng(5)
    extra = [Context(0) for _ in range(3)]
    fifth = Context(0)
    try:
        for i, c in enumerate(extra):
            buf = c.to_device((g.standard_normal(7000) * (i + 1)).astype(np.float32))
            arr, count = _tensors(buf, [3000, 4000])
            res = _both(c, arr, count, 1.0)
            assert res[0] == res[1], (i, res)
        buf = fifth.to_device(np.ones(100, np.float32))
        arr, count = _tensors(buf, [100])
        scale = fifth.alloc(1)
        st = fifth.lib.zl_grad_clip_scale_noalloc(fifth.h, arr, count, 1.0, scale.p, None)
        assert st == _ffi.ZL_ERR_INVALID
        assert b"slots" in fifth.lib.zl_last_error(fifth.h)
        extra.pop().close()
        again = Context(0)
        try:
            buf2 = again.to_device(np.full(100, 0.5, np.float32))
            arr2, count2 = _tensors(buf2, [100])
            res = _both(again, arr2, count2, 1.0)
            assert res[0] == res[1] and res[0][1] == np.float32(5.0)
        finally:
            again.close()
    finally:
        fifth.close()
        for c in extra:
            c.close()
