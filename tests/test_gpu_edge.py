"""Empty and degenerate sizes through the C ABI: nothing is launched for an
empty output, an empty reduction gives zeros (an empty dot product, an empty
row sum, the norm of no elements), and an empty rollout or action batch
leaves the outputs untouched. Advantage normalisation of no elements is an
error, as the mean of an empty set is undefined (zealot-rl/src/ppo.rs:
341-348 divides by n)."""

import numpy as np
import pytest

from zealot_amd import ZealotError, ops, synth
from zealot_amd.rl import GpuActorCritic

pytestmark = pytest.mark.gpu

SENTINEL = np.float32(7.25)


def filled(ctx, n, value=SENTINEL):
    return ctx.to_device(np.full(max(n, 1), value, np.float32))


@pytest.mark.parametrize("m, n", [(0, 64), (64, 0), (0, 0), (0, 29), (3000, 0)])
def test_gemm_empty_output(ctx, m, n):
    lhs, rhs, out = filled(ctx, 64 * 32), filled(ctx, 64 * 32), filled(ctx, 1)
    ops.gemm(ctx, out, lhs, False, rhs, True, m, n, 32)
    assert out.numpy()[0] == SENTINEL  # nothing written


@pytest.mark.parametrize("n", [300, 29, 1])
@pytest.mark.parametrize("lhs_t, rhs_t", [(False, False), (False, True), (True, False)])
def test_gemm_zero_k_is_zero(ctx, n, lhs_t, rhs_t):
    """K = 0: every output is the empty sum 0 (tiled for n = 300, the narrow
    kernels for n <= 32)."""
    m = 200
    out = ctx.to_device(np.full((m, n), np.nan, np.float32))
    ops.gemm(ctx, out, filled(ctx, 1), lhs_t, filled(ctx, 1), rhs_t, m, n, 0)
    assert np.array_equal(out.numpy(), np.zeros((m, n), np.float32))


def test_gemm_bias_act_zero_k(ctx):
    """K = 0 with the bias + ELU epilogue: elu(bias) in every column."""
    m, n = 100, 40
    bias = np.linspace(-2, 2, m).astype(np.float32)
    out = ctx.to_device(np.full((m, n), np.nan, np.float32))
    ops.gemm_bias_act(ctx, out, filled(ctx, 1), filled(ctx, 1), m, n, 0, ctx.to_device(bias), 1, True)
    z = bias.astype(np.float64)[:, None] * np.ones((1, n))
    ref = np.where(z > 0, z, np.expm1(z))
    assert np.max(np.abs(out.numpy() - ref)) <= 1e-6


def test_elementwise_and_reductions_empty(ctx):
    g = filled(ctx, 1)
    ops.elu_backward(ctx, g, filled(ctx, 1), 0, 16)
    ops.elu_backward(ctx, g, filled(ctx, 1), 16, 0)
    assert g.numpy()[0] == SENTINEL
    out = ctx.to_device(np.full(37, np.nan, np.float32))
    ops.row_sum(ctx, out, filled(ctx, 1), 37, 0)  # rows of no columns
    assert np.array_equal(out.numpy(), np.zeros(37, np.float32))
    p, m, v = filled(ctx, 1), filled(ctx, 1), filled(ctx, 1)
    ops.adam_step(ctx, p, filled(ctx, 1), m, v, 0, 1e-3, 0.1, 0.001)
    assert p.numpy()[0] == SENTINEL and m.numpy()[0] == SENTINEL and v.numpy()[0] == SENTINEL
    sq = filled(ctx, 1)
    ops.grad_sqnorm(ctx, filled(ctx, 1), 0, sq)
    assert sq.numpy()[0] == 0.0
    with pytest.raises(ZealotError):
        ops.adv_normalize(ctx, filled(ctx, 1), 0)


@pytest.mark.parametrize("T, N", [(0, 64), (24, 0)])
def test_gae_empty(ctx, T, N):
    adv, ret = filled(ctx, 1), filled(ctx, 1)
    dones = ctx.to_device(np.zeros(max(T * N, 1), np.uint8))
    # last_values holds one value per env: the scan starts from it even when T = 0
    ops.gae(ctx, filled(ctx, 1), filled(ctx, 1), dones, filled(ctx, N), T, N, adv, ret)
    assert adv.numpy()[0] == SENTINEL and ret.numpy()[0] == SENTINEL


def test_sampling_and_rollout_empty(ctx):
    act, logp = filled(ctx, 1), filled(ctx, 1)
    ops.sample_actions(ctx, filled(ctx, 29), filled(ctx, 29), filled(ctx, 29), 0, 29, act, logp)
    assert act.numpy()[0] == SENTINEL and logp.numpy()[0] == SENTINEL
    ad, cd = synth.ACTOR_DIMS, synth.CRITIC_DIMS
    g = np.random.default_rng(3)
    gac = GpuActorCritic(ctx, ad, cd, 256)
    gac.set_params(synth.kaiming_uniform_net(g, ad, 0.1), synth.kaiming_uniform_net(g, cd, 0.1),
                   np.full(ad[-1], -0.5, np.float32), 1e-3)
    obs = filled(ctx, 123)
    vals = filled(ctx, 1)
    gac.values(obs, 0, vals)
    gac.act(obs, 0, filled(ctx, 29), act, logp, value=vals, critic_obs=obs,
            obs_norm=gac.obs_norm, critic_norm=gac.critic_norm)
    assert vals.numpy()[0] == SENTINEL and act.numpy()[0] == SENTINEL and logp.numpy()[0] == SENTINEL
    gac.close()
