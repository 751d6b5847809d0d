"""Writes the golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

None of these come from the oracle or the HIP path:
- lcg_streams.json: zealot-rl's Lcg::unit stream (zealot-rl/src/rng.rs:21-27)
  computed with exact Python integers (the 24-bit value / 2^24 is exact in f32).
- gae_cases.json: the two hand-computed cases of zealot-rl/src/ppo.rs:709-721
  and :760-768, plus seeded random trajectories whose advantages are the
  float64 closed form adv_t = sum_k (gamma*lam)^k delta_{t+k}, truncated at
  the first done.
"""

import json
import os
import random
import struct

HERE = os.path.dirname(os.path.abspath(__file__))
MASK64 = (1 << 64) - 1


def f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def lcg_bits(seed: int, n: int):
    s = (seed | 1) & MASK64
    out = []
    for _ in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) & MASK64
        out.append(f32_bits((s >> 40) / float(1 << 24)))
    return out


def gae_closed_form(r, v, d, last_v, gamma, lam):
    T = len(r)
    adv = []
    for t in range(T):
        acc, coef = 0.0, 1.0
        for k in range(t, T):
            nv = last_v if k == T - 1 else v[k + 1]
            nt = 0.0 if d[k] else 1.0
            acc += coef * (r[k] + gamma * nv * nt - v[k])
            if d[k]:
                break
            coef *= gamma * lam
        adv.append(acc)
    return adv, [a + vv for a, vv in zip(adv, v)]


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def main():
    streams = {"units": [{"seed": s, "bits": lcg_bits(s, 64)} for s in (1, 7, 9, 123, 2024, 12345678901)]}
    with open(os.path.join(HERE, "lcg_streams.json"), "w") as f:
        json.dump(streams, f, indent=0)

    cases = [
        # ppo.rs:709-721
        dict(rewards=[1.0, 2.0], values=[0.0, 0.0], dones=[0, 0], last_value=0.0, gamma=1.0, lam=1.0,
             adv=[3.0, 2.0], ret=[3.0, 2.0]),
        # ppo.rs:760-768 (adv[0] = -4 by the test; adv[1] by the same formula)
        dict(rewards=[1.0, 1.0], values=[5.0, 5.0], dones=[1, 0], last_value=0.0, gamma=0.99, lam=0.95,
             adv=[-4.0, -4.0], ret=[1.0, 1.0]),
    ]
    rnd = random.Random(20240601)
    for T in (1, 3, 8, 24):
        for _ in range(4):
            r = [f32(rnd.uniform(-1, 1)) for _ in range(T)]
            v = [f32(rnd.uniform(-1, 1)) for _ in range(T)]
            d = [1 if rnd.random() < 0.2 else 0 for _ in range(T)]
            lv = f32(rnd.uniform(-1, 1))
            adv, ret = gae_closed_form(r, v, d, lv, 0.99, 0.95)
            cases.append(dict(rewards=r, values=v, dones=d, last_value=lv, gamma=0.99, lam=0.95,
                              adv=adv, ret=ret))
    with open(os.path.join(HERE, "gae_cases.json"), "w") as f:
        json.dump({"cases": cases}, f, indent=0)


if __name__ == "__main__":
    main()
