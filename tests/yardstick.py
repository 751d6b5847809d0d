"""The oracle's own spread as the yardstick for a chaotic whole update.

Twenty Adam steps over a batch whose advantages carry little signal amplify
rounding differences: two valid evaluations of the same update (another
thread count of the oracle's fold, whose grouping zealot-rl's rayon does not
fix, zealot-rl/src/ppo.rs:406-462; or inputs differing in their last bit,
the size of difference another summation order of the first layer makes)
end with parameter changes that differ by a few tenths of a percent to a few
percent. A GPU update is accepted when its distance from the oracle is
within a factor of the largest such spread, per net. Not sharing code with
the oracle: plain numpy on its outputs."""

from __future__ import annotations

import numpy as np


def perturb_last_bit(x: np.ndarray, seed: int) -> np.ndarray:
    """x with every nonzero element moved by -1, 0 or +1 ulp (float32)."""
    x = np.ascontiguousarray(x, np.float32)
    step = np.random.default_rng(seed).integers(-1, 2, x.shape).astype(np.int32) * (x != 0)
    return (x.view(np.int32) + step).view(np.float32)


def update_distance(p0, got, ref) -> float:
    """Relative L2 distance of the parameter change got - p0 from ref - p0."""
    dg = np.asarray(got, np.float64) - np.asarray(p0, np.float64)
    dr = np.asarray(ref, np.float64) - np.asarray(p0, np.float64)
    return float(np.linalg.norm(dg - dr) / max(np.linalg.norm(dr), 1e-30))


def spread(p0, ref, variants) -> float:
    """Largest distance of a valid variant's update from the reference update."""
    return max(update_distance(p0, v, ref) for v in variants)


def within(p0, ref, variants, got, factor=2.0):
    """(ok, distance, spread) for one parameter group."""
    s = spread(p0, ref, variants)
    d = update_distance(p0, got, ref)
    return d <= factor * s, d, s
