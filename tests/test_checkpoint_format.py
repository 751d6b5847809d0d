"""CPU checks of the checkpoint image reader (zl_checkpoint_dims parses and
validates a .safetensors image without a GPU): images written by the
safetensors package (0.8.0 in this image; the reference pins the Rust crate
0.4.5, Cargo.lock:4202-4205) in the layout of ActorCritic::save
(zealot-rl/src/ppo.rs:512-570), and malformed images, which must come back
as an error status."""

import json
import struct

import numpy as np
import pytest

from zealot_amd import ZealotError
from zealot_amd.rl import checkpoint_dims

safetensors_numpy = pytest.importorskip("safetensors.numpy")


def reference_tensors(ad, cd, seed=0):
    g = np.random.default_rng(seed)
    t = {}
    for prefix, dims in (("actor", ad), ("critic", cd)):
        for l in range(len(dims) - 1):
            t[f"{prefix}.w_{l}"] = g.standard_normal((dims[l + 1], dims[l])).astype(np.float32)
            t[f"{prefix}.b_{l}"] = g.standard_normal(dims[l + 1]).astype(np.float32)
    t["log_std"] = np.full(ad[-1], -0.5, np.float32)
    for name, d in (("obs_norm", ad[0]), ("critic_norm", cd[0])):
        t[f"{name}.mean"] = g.standard_normal(d).astype(np.float32)
        t[f"{name}.m2"] = g.uniform(1, 2, d).astype(np.float32)
        t[f"{name}.count"] = np.array([37.0], np.float32)
    t["lr"] = np.array([3e-4], np.float32)
    return t


def test_dims_of_reference_layout():
    ad, cd = [123, 512, 256, 128, 29], [64, 512, 256, 128, 1]
    img = safetensors_numpy.save(reference_tensors(ad, cd))
    assert checkpoint_dims(img) == (ad, cd)


def test_metadata_is_skipped():
    ad, cd = [4, 8, 8, 2], [6, 8, 1]
    img = safetensors_numpy.save(reference_tensors(ad, cd), metadata={"format": "np", "k": "v"})
    assert checkpoint_dims(img) == (ad, cd)


def _image(header: dict, data: bytes) -> bytes:
    h = json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + data


@pytest.mark.parametrize("case", ["truncated", "header_past_end", "not_json", "gap", "overlap",
                                  "shape_mismatch", "missing_bias", "no_layers", "bad_dtype_w",
                                  "chain_mismatch"])
def test_malformed_images_rejected(case):
    w = np.ones((3, 2), np.float32).tobytes()
    b = np.ones(3, np.float32).tobytes()
    hdr = {"actor.w_0": {"dtype": "F32", "shape": [3, 2], "data_offsets": [0, 24]},
           "actor.b_0": {"dtype": "F32", "shape": [3], "data_offsets": [24, 36]},
           "critic.w_0": {"dtype": "F32", "shape": [3, 2], "data_offsets": [36, 60]},
           "critic.b_0": {"dtype": "F32", "shape": [3], "data_offsets": [60, 72]}}
    data = w + b + w + b
    good = _image(hdr, data)
    assert checkpoint_dims(good) == ([2, 3], [2, 3])
    if case == "truncated":
        img = good[:6]
    elif case == "header_past_end":
        img = struct.pack("<Q", 10 ** 6) + good[8:]
    elif case == "not_json":
        img = struct.pack("<Q", 4) + b"{abc" + data
    elif case == "gap":
        hdr["critic.b_0"]["data_offsets"] = [64, 76]
        img = _image(hdr, data + b"\0" * 4)
    elif case == "overlap":
        hdr["critic.w_0"]["data_offsets"] = [32, 56]
        img = _image(hdr, data)
    elif case == "shape_mismatch":
        hdr["actor.w_0"]["shape"] = [3, 3]
        img = _image(hdr, data)
    elif case == "missing_bias":
        del hdr["critic.b_0"]
        hdr["critic.w_0"]["data_offsets"] = [36, 60]
        img = _image(hdr, data[:60])
    elif case == "no_layers":
        img = _image({k: v for k, v in hdr.items() if k.startswith("actor")}, data[:36])
    elif case == "bad_dtype_w":
        hdr["actor.w_0"]["dtype"] = "I32"  # right size, wrong type
        img = _image(hdr, data)
    else:  # chain_mismatch: layer 1 input != layer 0 output
        hdr["actor.w_1"] = {"dtype": "F32", "shape": [2, 4], "data_offsets": [72, 104]}
        hdr["actor.b_1"] = {"dtype": "F32", "shape": [2], "data_offsets": [104, 112]}
        img = _image(hdr, data + b"\0" * 40)
    with pytest.raises(ZealotError):
        checkpoint_dims(img)


def test_mutated_images_never_crash():
    """Seeded byte mutations of a valid image (header and data): every one
    parses to dims or comes back as an error status, never a crash or an
    out-of-bounds read (run under AddressSanitizer by tests/sanitize.sh)."""
    ad, cd = [7, 16, 8, 3], [5, 16, 1]
    good = safetensors_numpy.save(reference_tensors(ad, cd))
    g = np.random.default_rng(2024)
    hlen = struct.unpack("<Q", good[:8])[0]
    ok = bad = 0
    for i in range(400):
        b = bytearray(good)
        for _ in range(int(g.integers(1, 4))):
            # Mostly inside the 8-byte length and the JSON header.
            pos = int(g.integers(0, 8 + hlen)) if g.random() < 0.9 else int(g.integers(0, len(b)))
            b[pos] = int(g.integers(0, 256))
        if i % 50 == 0:
            b = b[: int(g.integers(0, len(b)))]  # truncations
        try:
            checkpoint_dims(bytes(b))
            ok += 1
        except ZealotError:
            bad += 1
    assert ok + bad == 400 and bad > 100
