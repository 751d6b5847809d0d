"""GPU parity of the operator-level entry points against the CPU oracle and
fp64 closed forms. Tolerances: forward/backward 1e-4 relative to the tensor's
max |value| (fp32); Adam and GAE bit-exact / 2 ulp (same operation order, no
FP contraction, correctly rounded div/sqrt on both sides)."""

import numpy as np
import pytest

from conftest import rel_amax, ulp_diff
from oracle import zl_oracle as zo
from zealot_amd import ops, synth
from zealot_amd.rl import GpuMlp, packed_count

pytestmark = pytest.mark.gpu

FWD_BWD_TOL = 1e-4


def st_val(r, c, seed, a=31, b=17, cst=101, p=97):
    i = np.arange(r)[:, None]
    j = np.arange(c)[None, :]
    h = (i * a + j * b + seed * cst) % p
    return (h.astype(np.float32) / np.float32(p / 2.0) - np.float32(1.0)).astype(np.float32)


# (m, n, k, lhs_t, rhs_t) of CutileGemm::self_test (src/biped/cutile_gemm.rs:699-708)
CUTILE_CASES = [
    (12, 300, 45, False, False),
    (45, 300, 256, True, False),
    (256, 45, 300, False, True),
    (64, 96, 4096, False, True),
    (64, 96, 3072, False, True),
    (512, 12288, 51, False, False),
]


def test_self_test_error_recorded(ctx):
    print(f"[gpu] self-test worst rel err {ctx.self_test_error:.3e}", flush=True)
    assert 0.0 <= ctx.self_test_error <= FWD_BWD_TOL


@pytest.mark.parametrize("ci,case", list(enumerate(CUTILE_CASES)))
def test_gemm_cutile_cases(ctx, ci, case):
    m, n, k, lt, rt = case
    L = st_val(m, k, ci)
    R = st_val(k, n, ci + 7)
    ref = L.astype(np.float64) @ R.astype(np.float64)
    dl = ctx.to_device(L.T.copy() if lt else L)
    dr = ctx.to_device(R.T.copy() if rt else R)
    out = ctx.alloc((m, n))
    ops.gemm(ctx, out, dl, lt, dr, rt, m, n, k)
    got = out.numpy()
    err = rel_amax(got, ref)
    print(f"[gpu] gemm case {ci} {case}: rel err {err:.2e}", flush=True)
    assert err <= FWD_BWD_TOL


@pytest.mark.parametrize("lt", [False, True])
@pytest.mark.parametrize("rt", [False, True])
@pytest.mark.parametrize("shape", [(1, 1, 1), (5, 7, 3), (33, 129, 17), (130, 70, 1000), (29, 123, 24576)])
def test_gemm_layouts_ragged(ctx, lt, rt, shape):
    m, n, k = shape
    g = np.random.default_rng(m * 1000 + n * 10 + k)
    L = g.standard_normal((m, k)).astype(np.float32)
    R = g.standard_normal((k, n)).astype(np.float32)
    ref = L.astype(np.float64) @ R.astype(np.float64)
    dl = ctx.to_device(L.T.copy() if lt else L)
    dr = ctx.to_device(R.T.copy() if rt else R)
    out = ctx.alloc((m, n))
    ops.gemm(ctx, out, dl, lt, dr, rt, m, n, k)
    err = rel_amax(out.numpy(), ref)
    assert err <= FWD_BWD_TOL, (shape, lt, rt, err)


# Shapes with several 96x128 output tiles per resident workgroup and no
# split-K (the row-major forward ak_bk and data-gradient ak_bn tiles), ragged
# in every dimension, with K tails of 12 and 4 and a single k-tile.
LARGE_CASES = [
    (50000, 300, 76, False, True),
    (50000, 300, 76, False, False),
    (13001, 1000, 132, False, True),
    (13001, 1000, 132, False, False),
    (70001, 130, 20, False, True),
    # Rollout-size forwards: the tile shrinks until every CU has a workgroup
    # (64x64 here, 32x64 when even that leaves CUs idle).
    (4001, 300, 76, False, True),
    (3001, 100, 132, False, True),
    # Weight-gradient-shaped products (A M-contiguous, long K: split-K) whose
    # widths 128-column tiles would leave partly empty: 128 x 96 and
    # 128 x 64 tiles, exact-fit (256 x 288, 512 x 64) and masked (ragged M
    # and K), and the feature-major 64 x 64 tiles with a ragged M.
    (256, 288, 24576, True, False),
    (512, 64, 24576, True, False),
    (300, 96, 5000, True, False),
    (260, 64, 7001, True, False),
    (1000, 2000, 123, False, False),
    (1000, 2000, 128, False, False),
]


@pytest.mark.parametrize("case", LARGE_CASES)
def test_gemm_large_ragged(ctx, case):
    m, n, k, lt, rt = case
    g = np.random.default_rng(m + 3 * n + 5 * k + rt)
    L = g.standard_normal((m, k)).astype(np.float32)
    R = g.standard_normal((k, n)).astype(np.float32)
    ref = L.astype(np.float64) @ R.astype(np.float64)
    dl = ctx.to_device(L.T.copy() if lt else L)
    dr = ctx.to_device(R.T.copy() if rt else R)
    out = ctx.alloc((m, n))
    ops.gemm(ctx, out, dl, lt, dr, rt, m, n, k)
    err = rel_amax(out.numpy(), ref)
    print(f"[gpu] large gemm {case}: rel err {err:.2e}", flush=True)
    assert err <= FWD_BWD_TOL, (case, err)


# Shapes whose tiles and k-tiles are all full, which run the exact-fit
# kernels (no clamps or masks): the 96 x 128 forward tile, and split-K
# weight gradients on 128 x 128 and 64 x 128 tiles.
EXACT_CASES = [
    (6144, 512, 128, False, True),
    (256, 512, 6144, True, False),
    (128, 256, 6144, True, False),
]


@pytest.mark.parametrize("case", EXACT_CASES)
def test_gemm_exact_fit(ctx, case):
    m, n, k, lt, rt = case
    g = np.random.default_rng(m + 7 * n + 11 * k)
    L = g.standard_normal((m, k)).astype(np.float32)
    R = g.standard_normal((k, n)).astype(np.float32)
    ref = L.astype(np.float64) @ R.astype(np.float64)
    dl = ctx.to_device(L.T.copy() if lt else L)
    dr = ctx.to_device(R.T.copy() if rt else R)
    out = ctx.alloc((m, n))
    ops.gemm(ctx, out, dl, lt, dr, rt, m, n, k)
    err = rel_amax(out.numpy(), ref)
    print(f"[gpu] exact-fit gemm {case}: rel err {err:.2e}", flush=True)
    assert err <= FWD_BWD_TOL, (case, err)


# Shapes routed to the register-resident narrow kernels (one dimension <= 32):
# (m, n, k, lhs_t, rhs_t) and the family each exercises.
NARROW_CASES = [
    (24576, 29, 128, False, True),   # N <= 32, float4 loads: the actor head forward
    (24576, 1, 128, False, True),    # N <= 16: the critic head forward
    (1000, 17, 50, False, True),     # N <= 32 with a K tail (element loads)
    (3, 5, 7, False, True),          # fewer rows than one strip
    (24576, 128, 29, False, False),  # K <= 32: the actor head data gradient
    (24576, 128, 1, False, False),   # the critic head data gradient
    (777, 200, 17, False, False),    # K in two 16-wide chunks, ragged N
    (29, 128, 24576, True, False),   # M <= 32: the actor head weight gradient (row slices)
    (1, 128, 24576, True, False),    # the critic head weight gradient
    (7, 300, 5000, True, False),     # three 128-column chunks, ragged last slice
    (32, 64, 100, True, False),      # one slice (direct write)
]


@pytest.mark.parametrize("case", NARROW_CASES)
def test_gemm_narrow_shapes(ctx, case):
    m, n, k, lt, rt = case
    g = np.random.default_rng(m + 7 * n + 13 * k)
    L = g.standard_normal((m, k)).astype(np.float32)
    R = g.standard_normal((k, n)).astype(np.float32)
    ref = L.astype(np.float64) @ R.astype(np.float64)
    dl = ctx.to_device(L.T.copy() if lt else L)
    dr = ctx.to_device(R.T.copy() if rt else R)
    out = ctx.alloc((m, n))
    ops.gemm(ctx, out, dl, lt, dr, rt, m, n, k)
    err = rel_amax(out.numpy(), ref)
    print(f"[gpu] narrow gemm {case}: rel err {err:.2e}", flush=True)
    assert err <= FWD_BWD_TOL, (case, err)


@pytest.fixture(scope="module")
def tiled_ctx():
    """A context with the register-resident narrow kernels switched off
    (ZL_NARROW=0, read at zl_init): N <= 32 then runs the 256 x 16 / 128 x 32
    tiles and K <= 32 / M <= 32 the general tiles."""
    import os

    from zealot_amd import Context

    os.environ["ZL_NARROW"] = "0"
    try:
        c = Context(0)
    finally:
        del os.environ["ZL_NARROW"]
    yield c
    c.close()


@pytest.mark.parametrize("case", NARROW_CASES)
def test_gemm_narrow_shapes_tiled(tiled_ctx, case):
    test_gemm_narrow_shapes(tiled_ctx, case)


def test_gemm_narrow_bias_elu(ctx):
    """K <= 32 with the strided bias column + ELU epilogue of gemm_bias_act."""
    m, n, k = 300, 100, 20
    f = lambda r, c, s: st_val(r, c, s, 29, 13, 89, 83)  # noqa: E731
    L, R, Bb = f(m, k, 5), f(k, n, 6), f(m, 8, 7)
    z = L.astype(np.float64) @ R.astype(np.float64) + Bb[:, :1].astype(np.float64)
    ref = np.where(z > 0, z, np.expm1(z))
    out = ctx.alloc((m, n))
    ops.gemm_bias_act(ctx, out, ctx.to_device(L), ctx.to_device(R), m, n, k, ctx.to_device(Bb), 8, True)
    assert rel_amax(out.numpy(), ref) <= FWD_BWD_TOL


def test_gemm_bias_elu_backward_rowsum(ctx):
    # src/biped/cutile_gemm.rs:749-826: strided bias column (stride 8), ELU, backward, row sums.
    m, n, k = 100, 300, 45
    f = lambda r, c, s: st_val(r, c, s, 29, 13, 89, 83)  # noqa: E731
    L, R, Bb, G = f(m, k, 1), f(k, n, 2), f(m, 8, 3), f(m, n, 4)
    z = L.astype(np.float64) @ R.astype(np.float64) + Bb[:, :1].astype(np.float64)
    ref = np.where(z > 0, z, np.expm1(z))
    dl, dr, db, dg = ctx.to_device(L), ctx.to_device(R), ctx.to_device(Bb), ctx.to_device(G)
    out = ctx.alloc((m, n))
    ops.gemm_bias_act(ctx, out, dl, dr, m, n, k, db, 8, True)
    y = out.numpy()
    assert rel_amax(y, ref) <= FWD_BWD_TOL
    ops.elu_backward(ctx, dg, out, m, n)
    g2 = dg.numpy()
    gref = G * np.where(y > 0, np.float32(1.0), y + np.float32(1.0))
    assert np.array_equal(g2, gref.astype(np.float32))  # one f32 multiply: exact
    rs = ctx.alloc(m)
    ops.row_sum(ctx, rs, dg, m, n)
    assert rel_amax(rs.numpy(), g2.astype(np.float64).sum(1)) <= FWD_BWD_TOL


def test_config1_single_layer(ctx):
    """X [4096 x 123] . W [123 x 512] + b, ELU (config 1) vs the oracle's Mlp::forward."""
    c1 = synth.config1()
    x, w_kn, b = c1["x"], c1["w_kn"], c1["b"]
    # Oracle: the layer as the hidden layer of an Mlp [123, 512, 1] (ELU applied).
    params = np.concatenate([w_kn.T.ravel(), b, np.zeros(513, np.float32)]).astype(np.float32)
    ref = zo.mlp_forward([123, 512, 1], params, x)[0]
    truth = x.astype(np.float64) @ w_kn.astype(np.float64) + b
    truth = np.where(truth > 0, truth, np.expm1(truth))
    # The reference's fused layer is feature-major (bias per row of out,
    # src/bin/biped_train_gpu.rs:382-394): out^T [512 x 4096] = W^T . X^T + b.
    dwt = ctx.to_device(w_kn.T.copy())
    dxt = ctx.to_device(x.T.copy())
    db = ctx.to_device(b)
    out_t = ctx.alloc((512, 4096))
    ops.gemm_bias_act(ctx, out_t, dwt, dxt, 512, 4096, 123, db, 1, True)
    got = out_t.numpy().T
    e_gpu, e_cpu = rel_amax(got, truth), rel_amax(ref, truth)
    print(f"[gpu] config1: gpu vs f64 {e_gpu:.2e}, oracle vs f64 {e_cpu:.2e}, "
          f"gpu vs oracle {rel_amax(got, ref):.2e}", flush=True)
    assert rel_amax(got, ref) <= FWD_BWD_TOL



def test_config1_aligned_and_odd_stride_agree(ctx):
    """The single layer through both feature-major tile paths: K = 123 (row
    stride 123: scalar-load 64 x 64 tiles) and the same product with K
    padded to 128 by zero columns / rows (float4 loads, 64 x 64 tiles). The
    padded terms add exact zeros in the same 16-wide chunk order, so the two
    outputs are bit-identical; both match the oracle."""
    c1 = synth.config1()
    x, w_kn, b = c1["x"], c1["w_kn"], c1["b"]
    wp = np.zeros((512, 128), np.float32)
    wp[:, :123] = w_kn.T
    xp = np.zeros((128, 4096), np.float32)
    xp[:123] = x.T
    db = ctx.to_device(b)
    o123, o128 = ctx.alloc((512, 4096)), ctx.alloc((512, 4096))
    ops.gemm_bias_act(ctx, o123, ctx.to_device(w_kn.T.copy()), ctx.to_device(x.T.copy()), 512, 4096, 123, db, 1, True)
    ops.gemm_bias_act(ctx, o128, ctx.to_device(wp), ctx.to_device(xp), 512, 4096, 128, db, 1, True)
    a, p = o123.numpy(), o128.numpy()
    params = np.concatenate([w_kn.T.ravel(), b, np.zeros(513, np.float32)]).astype(np.float32)
    ref = zo.mlp_forward([123, 512, 1], params, x)[0]
    assert np.array_equal(a, p)
    assert rel_amax(p.T, ref) <= FWD_BWD_TOL

@pytest.fixture(scope="module")
def smallk_ctx():
    """A context that takes the small-K variants also for float4-aligned A
    rows (ZL_SMALLK=2, read at zl_init)."""
    import os

    from zealot_amd import Context

    os.environ["ZL_SMALLK"] = "2"
    try:
        c = Context(0)
    finally:
        del os.environ["ZL_SMALLK"]
    yield c
    c.close()


# (m, n, k, bias): A K-contiguous (lhs as stored), B N-contiguous, K <= 128:
# ragged tiles, K tails, the padded K = 128 and the config-1 shape.
SMALLK_CASES = [(1, 1, 1, False), (5, 7, 3, True), (130, 70, 17, True), (512, 4096, 123, True),
                (512, 4096, 128, True), (300, 1000, 76, False), (64, 64, 128, False), (70, 4099, 100, True)]


@pytest.mark.parametrize("case", SMALLK_CASES)
def test_gemm_smallk_variants(ctx, smallk_ctx, case):
    """The small-K form (one round of loads for the whole K <= 128 extent)
    against float64 at 1e-4: on the default context it takes products whose
    lhs rows are not float4-aligned (K not a multiple of 4), on the
    ZL_SMALLK=2 context also the aligned ones. The same product with K padded
    to a multiple of 4 by zero columns / rows (float4 rows: the k-tiled form
    on the default context) adds exact zeros in the same 16-wide chunk order,
    so all four results are bit-identical."""
    m, n, k, bias = case
    g = np.random.default_rng(m + 7 * n + 31 * k)
    L = g.standard_normal((m, k)).astype(np.float32)
    R = g.standard_normal((k, n)).astype(np.float32)
    bb = g.uniform(-0.5, 0.5, m).astype(np.float32)
    z = L.astype(np.float64) @ R.astype(np.float64) + (bb[:, None] if bias else 0.0)
    ref = np.where(z > 0, z, np.expm1(np.minimum(z, 0))) if bias else z
    kp = -(-k // 4) * 4
    Lp = np.zeros((m, kp), np.float32)
    Lp[:, :k] = L
    Rp = np.zeros((kp, n), np.float32)
    Rp[:k] = R
    outs = []
    for cx in (ctx, smallk_ctx):
        for lhs, rhs, kk in ((L, R, k), (Lp, Rp, kp)):
            out = cx.alloc((m, n))
            dl, dr = cx.to_device(lhs), cx.to_device(rhs)
            if bias:
                ops.gemm_bias_act(cx, out, dl, dr, m, n, kk, cx.to_device(bb), 1, True)
            else:
                ops.gemm(cx, out, dl, False, dr, False, m, n, kk)
            outs.append(out.numpy())
    for o in outs:
        assert rel_amax(o, ref) <= FWD_BWD_TOL, case
    for o in outs[1:]:
        assert np.array_equal(outs[0], o), case


def _mlp_case(ctx, dims, rows, seed, bias_bound=0.1):
    g = np.random.default_rng(seed)
    params = synth.kaiming_uniform_net(g, dims, bias_bound=bias_bound)
    x = np.clip(g.standard_normal((rows, dims[0])), -5, 5).astype(np.float32)
    mlp = GpuMlp(ctx, dims, rows)
    mlp.write_weights(params)
    assert np.array_equal(mlp.read_weights(), params)
    dx = ctx.to_device(x)
    mlp.forward(dx, rows)
    return g, params, x, dx, mlp


# ([128, 512, 256, 128, 8], 6144): every 96 x 128 forward / data-gradient
# tile and every weight-gradient tile and k-tile full (the exact-fit kernels).
@pytest.mark.parametrize("dims,rows", [([4, 6, 5, 3], 7), ([123, 512, 256, 128, 29], 4096),
                                       ([123, 512, 256, 128, 1], 1000), ([17, 33, 2], 300),
                                       ([123, 512, 256, 128, 29], 13001),
                                       ([128, 512, 256, 128, 8], 6144)])
def test_mlp_forward_vs_oracle(ctx, dims, rows):
    g, params, x, dx, mlp = _mlp_case(ctx, dims, rows, seed=rows)
    got = mlp.output(rows)
    ref = zo.mlp_forward(dims, params, x)[-1]
    err = rel_amax(got, ref)
    print(f"[gpu] mlp fwd {dims} x {rows}: rel err {err:.2e}", flush=True)
    assert err <= FWD_BWD_TOL


@pytest.mark.parametrize("dims,rows", [([4, 6, 5, 3], 7), ([123, 512, 256, 128, 29], 4096),
                                       ([123, 512, 256, 128, 1], 2048), ([17, 33, 2], 300),
                                       ([123, 512, 256, 128, 29], 13001),
                                       ([128, 512, 256, 128, 8], 6144)])
def test_mlp_backward_vs_oracle(ctx, dims, rows):
    g, params, x, dx, mlp = _mlp_case(ctx, dims, rows, seed=rows + 1)
    gout = (g.standard_normal((rows, dims[-1])) / rows).astype(np.float32)
    mlp.backward(ctx.to_device(gout))
    got = mlp.read_grads()
    ref, _ = zo.mlp_backward(dims, params, x, gout)
    # per-tensor amax-normalised error
    o = 0
    worst = 0.0
    for l in range(len(dims) - 1):
        for sz in (dims[l + 1] * dims[l], dims[l + 1]):
            e = rel_amax(got[o:o + sz], ref[o:o + sz])
            worst = max(worst, e)
            o += sz
    print(f"[gpu] mlp bwd {dims} x {rows}: worst per-tensor rel err {worst:.2e}", flush=True)
    assert worst <= FWD_BWD_TOL


@pytest.mark.parametrize("dims,rows,pad", [([123, 512, 256, 128, 29], 4096, 0),
                                           ([265, 256, 256, 128, 12], 6000, 40),
                                           ([17, 33, 2], 301, 3)])
def test_mlp_feature_major_matches_batch_major(ctx, dims, rows, pad):
    """zl_mlp_create_ex(ZL_MLP_FEATURE_MAJOR): the input, the output and the
    output gradient as [dim x rows] with feature stride rows + pad, as GpuMlp
    keeps a[0], a[L] and delta[L-1] (src/bin/biped_train_gpu.rs:351-355,
    382-394, 436-492), in a handle sized for more rows than are used. The
    stride padding holds NaN (never read). Output and gradients are
    bit-identical to the batch-major handle on the same values at 16-byte
    aligned row strides, and within 1e-4 of the oracle."""
    g = np.random.default_rng(rows + 7)
    params = synth.kaiming_uniform_net(g, dims, bias_bound=0.1)
    x = np.clip(g.standard_normal((rows, dims[0])), -5, 5).astype(np.float32)
    gout = (g.standard_normal((rows, dims[-1])) / rows).astype(np.float32)
    ldx, ldg = -(-dims[0] // 4) * 4, -(-dims[-1] // 4) * 4
    xb = np.zeros((rows, ldx), np.float32)
    xb[:, :dims[0]] = x
    gb = np.zeros((rows, ldg), np.float32)
    gb[:, :dims[-1]] = gout
    mb = GpuMlp(ctx, dims, rows)
    mb.write_weights(params)
    dxb = ctx.to_device(xb)  # borrowed by the batch-major handle until its backward
    mb.forward(dxb, rows, ldx)
    out_b = mb.output(rows)
    mb.backward(ctx.to_device(gb), ldg)
    grads_b = mb.read_grads()
    ld = rows + pad
    xf = np.full((dims[0], ld), np.nan, np.float32)
    xf[:, :rows] = x.T
    gf = np.full((dims[-1], ld), np.nan, np.float32)
    gf[:, :rows] = gout.T
    mf = GpuMlp(ctx, dims, rows + 7, feature_major=True)
    mf.write_weights(params)
    dxf = ctx.to_device(xf)
    mf.forward(dxf, rows, ld)
    del dxf  # the feature-major handle staged its own copy
    out_f = mf.output(rows)
    mf.backward(ctx.to_device(gf), ld)
    grads_f = mf.read_grads()
    ref = zo.mlp_forward(dims, params, x)[-1]
    rg, _ = zo.mlp_backward(dims, params, x, gout)
    o, worst = 0, 0.0
    for l in range(len(dims) - 1):
        for sz in (dims[l + 1] * dims[l], dims[l + 1]):
            worst = max(worst, rel_amax(grads_f[o:o + sz], rg[o:o + sz]))
            o += sz
    e_fwd = rel_amax(out_f, ref)
    print(f"[gpu] mlp feature-major {dims} x {rows} (ld {ld}): fwd err {e_fwd:.2e}, bwd worst {worst:.2e}, "
          f"identical fwd {np.array_equal(out_f, out_b)} bwd {np.array_equal(grads_f, grads_b)}", flush=True)
    assert np.array_equal(out_f, out_b)
    assert np.array_equal(grads_f, grads_b)
    assert e_fwd <= FWD_BWD_TOL and worst <= FWD_BWD_TOL
    mb.close()
    mf.close()


def test_config3_adam_bit_exact(ctx):
    """Adam over actor + critic + log_std (config 3): 10 warm steps then one
    more, on identical gradients, vs net.rs:240-245 on the CPU. <= 2 ulp."""
    na = packed_count(synth.ACTOR_DIMS)
    nc = packed_count(synth.CRITIC_DIMS)
    c3 = synth.config3(na, nc)
    p = np.concatenate([c3["actor"], c3["critic"], c3["log_std"]]).astype(np.float32)
    n = p.size
    dp, dm, dv = ctx.to_device(p), ctx.to_device(np.zeros(n, np.float32)), ctx.to_device(np.zeros(n, np.float32))
    hp, hm, hv = p.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    for t, gr in enumerate(c3["grads"], start=1):
        bc1 = np.float32(1.0) - np.float32(zo.powi(0.9, t))
        bc2 = np.float32(1.0) - np.float32(zo.powi(0.999, t))
        dg = ctx.to_device(gr)
        ops.adam_step(ctx, dp, dg, dm, dv, n, 1e-3, float(bc1), float(bc2))
        hp, hm, hv = zo.adam_flat(hp, gr, hm, hv, 1e-3, float(bc1), float(bc2))
    up, um, uv = ulp_diff(dp.numpy(), hp), ulp_diff(dm.numpy(), hm), ulp_diff(dv.numpy(), hv)
    print(f"[gpu] adam 11 steps over {n} params: max ulp p={up} m={um} v={uv}", flush=True)
    assert up <= 2 and um <= 2 and uv <= 2


def test_grad_sqnorm(ctx):
    g = np.random.default_rng(3).standard_normal(459_323).astype(np.float32) * 1e-2
    d = ctx.to_device(g)
    out = ctx.alloc(1)
    ops.grad_sqnorm(ctx, d, g.size, out)
    ref = float(np.sum(g.astype(np.float64) ** 2))
    assert abs(out.numpy()[0] - ref) / ref < 1e-5


def _gae_f64(r, v, d, last_v, gamma, lam):
    """Closed form: adv_t = sum_k (gamma*lam)^k delta_{t+k}, cut at dones."""
    T = len(r)
    adv = np.zeros(T)
    for t in range(T):
        acc, coef = 0.0, 1.0
        for k in range(t, T):
            nv = last_v if k == T - 1 else v[k + 1]
            nt = 0.0 if d[k] else 1.0
            acc += coef * (r[k] + gamma * nv * nt - v[k])
            if d[k]:
                break
            coef *= gamma * lam
        adv[t] = acc
    return adv, adv + np.asarray(v, np.float64)


@pytest.mark.parametrize("T,N", [(1, 1), (2, 3), (24, 4096), (32, 333), (37, 100)])
def test_gae_bit_exact(ctx, T, N):
    g = np.random.default_rng(T * 7 + N)
    r = g.standard_normal((T, N)).astype(np.float32)
    v = g.standard_normal((T, N)).astype(np.float32)
    d = (g.random((T, N)) < 0.05).astype(np.uint8)
    lv = g.standard_normal(N).astype(np.float32)
    dr, dvv, dd, dl = ctx.to_device(r), ctx.to_device(v), ctx.to_device(d), ctx.to_device(lv)
    adv, ret = ctx.alloc((T, N)), ctx.alloc((T, N))
    ops.gae(ctx, dr, dvv, dd, dl, T, N, adv, ret, 0.99, 0.95)
    ga, gr = adv.numpy(), ret.numpy()
    # The first 64 envs and every 61st: envs of several workgroups.
    for e in sorted(set(range(min(N, 64))) | set(range(0, N, 61))):
        ra, rr = zo.gae(r[:, e], v[:, e], d[:, e], float(lv[e]), 0.99, 0.95)
        assert np.array_equal(ga[:, e], ra) and np.array_equal(gr[:, e], rr), e
        fa, fr = _gae_f64(r[:, e], v[:, e], d[:, e], float(lv[e]), 0.99, 0.95)
        assert np.allclose(ga[:, e], fa, rtol=1e-4, atol=1e-4)


def test_gae_env_major_output(ctx):
    """Output strides: write adv/ret in env-major sample order (e*T + t)."""
    T, N = 24, 257
    g = np.random.default_rng(11)
    r = g.standard_normal((T, N)).astype(np.float32)
    v = g.standard_normal((T, N)).astype(np.float32)
    d = (g.random((T, N)) < 0.02).astype(np.uint8)
    lv = g.standard_normal(N).astype(np.float32)
    adv, ret = ctx.alloc(T * N), ctx.alloc(T * N)
    ops.gae(ctx, ctx.to_device(r), ctx.to_device(v), ctx.to_device(d), ctx.to_device(lv), T, N, adv, ret,
            0.99, 0.95, in_strides=(N, 1), out_strides=(1, T))
    ga = adv.numpy().reshape(N, T)
    for e in range(N):
        ra, _ = zo.gae(r[:, e], v[:, e], d[:, e], float(lv[e]), 0.99, 0.95)
        assert np.array_equal(ga[e], ra)


def test_adv_normalize(ctx):
    a = np.random.default_rng(5).standard_normal(98_304).astype(np.float32) * 3 + 1
    d = ctx.to_device(a)
    ops.adv_normalize(ctx, d, a.size)
    got = d.numpy()
    ref = zo.adv_normalize(a)
    truth = (a - a.astype(np.float64).mean()) / a.astype(np.float64).std()
    assert rel_amax(got, ref) < 1e-5 and rel_amax(got, truth) < 1e-5
    assert abs(float(got.astype(np.float64).mean())) < 1e-5
    # constant input: sd floored at 1e-6 -> all zeros, no NaN
    d2 = ctx.to_device(np.full(1000, 2.5, np.float32))
    ops.adv_normalize(ctx, d2, 1000)
    assert np.all(d2.numpy() == 0.0)


@pytest.mark.parametrize("A", [29, 40])
def test_actor_value_grad_ops(ctx, A):
    """zl_ppo_actor_grad / zl_ppo_value_grad vs the oracle's per-sample fold
    (through a 1-layer linear actor whose output is the mean itself); A = 40
    takes the 64-lane-group loss kernel."""
    rows = 777
    g = np.random.default_rng(21)
    mean = g.standard_normal((rows, A)).astype(np.float32)
    action = (mean + 0.6 * g.standard_normal((rows, A))).astype(np.float32)
    log_std = np.full(A, -0.5, np.float32) + 0.1 * g.standard_normal(A).astype(np.float32)
    adv = g.standard_normal(rows).astype(np.float32)
    logp_old = (synth.gaussian_logp(action, mean, log_std) + 0.3 * g.standard_normal(rows)).astype(np.float32)
    mean_old = (mean + 0.05 * g.standard_normal((rows, A))).astype(np.float32)
    dm, ds_ = ctx.alloc((rows, A)), ctx.alloc(A)
    stats = ctx.alloc(2)
    ops.ppo_actor_grad(ctx, ctx.to_device(mean), ctx.to_device(action), ctx.to_device(log_std),
                       ctx.to_device(adv), ctx.to_device(logp_old), ctx.to_device(mean_old), rows, A,
                       0.2, 0.005, 1.0 / rows, dm, ds_, stats)
    # oracle: identity actor (dims [A, A], W = I, b = 0) so dL/dmean = g_out.
    ad = [A, A]
    eye = np.concatenate([np.eye(A, dtype=np.float32).ravel(), np.zeros(A, np.float32)])
    cd = [1, 1]
    crit = np.array([1.0, 0.0], np.float32)  # v = obs
    v = g.standard_normal(rows).astype(np.float32)
    vold = (v + 0.3 * g.standard_normal(rows)).astype(np.float32)
    ret = g.standard_normal(rows).astype(np.float32)
    batch = dict(obs=mean, critic_obs=v[:, None].copy(), action=action, mean_old=mean_old,
                 logp_old=logp_old, value_old=vold, adv=adv, ret=ret)
    ga, gc, gl, st = zo.minibatch_grads(ad, cd, eye, crit, log_std, batch, np.arange(rows), 0.2, 0.005, 1.0)
    # dW of the identity layer = sum_r dmean[r,k] * mean[r,i] -> compare via db = sum_r dmean
    db_ref = ga[A * A:]
    assert rel_amax(dm.numpy().astype(np.float64).sum(0), db_ref) <= FWD_BWD_TOL
    assert rel_amax(ds_.numpy(), gl) <= FWD_BWD_TOL
    s = stats.numpy()
    assert abs(s[0] - st[0]) <= 1e-4 * max(1.0, abs(st[0]))
    assert abs(s[1] - st[2]) <= 1e-4 * max(1.0, abs(st[2]))
    # value grad
    dvv, vst = ctx.alloc(rows), ctx.alloc(1)
    ops.ppo_value_grad(ctx, ctx.to_device(v), ctx.to_device(vold), ctx.to_device(ret), rows, 0.2, 1.0,
                       1.0 / rows, dvv, vst)
    # critic [1,1] with w=1,b=0: db = sum dv
    assert rel_amax(dvv.numpy().astype(np.float64).sum(), gc[1]) <= FWD_BWD_TOL
    assert abs(vst.numpy()[0] - st[1]) <= 1e-4 * max(1.0, abs(st[1]))


def test_sample_actions(ctx):
    c2 = synth.config2()
    rows, A = 4096, 29
    means = zo.mlp_forward(synth.ACTOR_DIMS, c2["actor"], c2["obs"])[-1]
    act, lp = ctx.alloc((rows, A)), ctx.alloc(rows)
    ops.sample_actions(ctx, ctx.to_device(means), ctx.to_device(c2["log_std"]), ctx.to_device(c2["eps"]),
                       rows, A, act, lp)
    std = np.exp(c2["log_std"]).astype(np.float32)
    ref_a = (means + std * c2["eps"]).astype(np.float32)
    assert rel_amax(act.numpy(), ref_a) < 1e-6
    ref_lp = synth.gaussian_logp(ref_a, means, c2["log_std"])
    assert rel_amax(lp.numpy(), ref_lp) < 1e-5
