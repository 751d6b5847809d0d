"""CPU tests of the host-side logic: synthetic workload shapes, the packed
parameter layout, the config structs, and that the product package never
reaches into the oracle."""

import ast
import os

import numpy as np

from zealot_amd import _ffi, synth
from zealot_amd.rl import PpoConfig, pack, packed_count, unpack

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_parameter_counts():
    # actor 123-512-256-128-29, critic 123-512-256-128-1 (+ log_std 29)
    assert packed_count(synth.ACTOR_DIMS) == 231_453
    assert packed_count(synth.CRITIC_DIMS) == 227_841
    assert packed_count(synth.ACTOR_DIMS) + packed_count(synth.CRITIC_DIMS) + 29 == 459_323


def test_pack_roundtrip():
    dims = [5, 4, 3]
    p = np.arange(packed_count(dims), dtype=np.float32)
    ws, bs = unpack(dims, p)
    assert ws[0].shape == (4, 5) and bs[1].shape == (3,)
    assert np.array_equal(pack(ws, bs), p)


def test_synthetic_configs():
    c1 = synth.config1()
    assert c1["x"].shape == (4096, 123) and c1["w_kn"].shape == (123, 512)
    assert np.all(np.abs(c1["w_kn"]) <= np.sqrt(6 / 123))
    assert np.all(np.abs(c1["b"]) <= 0.1)
    c2 = synth.config2()
    assert c2["obs"].shape == (4096, 123) and c2["eps"].shape == (4096, 29)
    assert np.all(c2["log_std"] == -0.5)
    g = synth.rng(5)
    ro = synth.rollout(g, 64, 24)
    assert ro["obs"].shape == (24 * 64, 123) and ro["dones"].dtype == np.uint8
    assert np.all(np.abs(ro["obs"]) <= 5.0)
    # same seed -> byte-identical inputs
    assert np.array_equal(synth.config2()["obs"], c2["obs"])


def test_gaussian_logp_closed_form():
    g = np.random.default_rng(0)
    a = g.standard_normal((10, 3)).astype(np.float32)
    m = g.standard_normal((10, 3)).astype(np.float32)
    ls = np.array([-0.5, 0.0, 0.3], np.float32)
    want = np.sum(-0.5 * ((a - m) / np.exp(ls)) ** 2 - ls - 0.5 * np.log(2 * np.pi), axis=1)
    assert np.allclose(synth.gaussian_logp(a, m, ls), want, rtol=1e-5, atol=1e-5)


def test_config_struct_fields():
    c = PpoConfig.gpu_trainer(epochs=3).to_c()
    assert c.semantics == _ffi.ZL_SEMANTICS_GPU_TRAINER and c.epochs == 3 and c.shuffle == 0
    d = PpoConfig().to_c()
    assert d.semantics == _ffi.ZL_SEMANTICS_ACTOR_CRITIC and d.shuffle == 1 and d.clamp_log_std == 1


def test_product_package_does_not_import_oracle():
    pkg = os.path.join(ROOT, "zealot_amd")
    for dirpath, _, files in os.walk(pkg):
        for fn in files:
            if fn.endswith(".py"):
                tree = ast.parse(open(os.path.join(dirpath, fn)).read())
                for node in ast.walk(tree):
                    if isinstance(node, ast.Import):
                        assert not any("oracle" in a.name for a in node.names), fn
                    if isinstance(node, ast.ImportFrom):
                        assert "oracle" not in (node.module or ""), fn
