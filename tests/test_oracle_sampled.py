"""The oracle's sampler (orc_sample, orc_run_sampled) against the reference engine's own --gen output with
--temperature / --top-k / --top-p / --seed (tests/golden/sampled.npz, written by make_sampled.py from
oracle/_ref/rabbit2): identical ids in both orders. Plus the generator's defining properties."""
import json
import os

import numpy as np
import pytest

from oracle import pyoracle as po

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))["cases"]
SAMPLED = json.load(open(os.path.join(GOLDEN, "sampled.json")))
ORDERS = {"scalar": po.ORDER_SCALAR, "avx2": po.ORDER_AVX2}


def build(case):
    spec = MANIFEST[case]
    cfg = po.Config(**spec["config"])
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    return spec, cfg, model


@pytest.mark.parametrize("case", sorted(SAMPLED["cases"]))
def test_oracle_sampling_matches_reference_gen(case):
    spec, cfg, model = build(case)
    fx = np.load(os.path.join(GOLDEN, "sampled.npz"))
    tokens = po.prompt_tokens(spec["gen_params"]["seed"], spec["n_prompt"], cfg.vocab)
    n_gen = SAMPLED["cases"][case]["n_gen"]
    for j, (t, k, p, seed) in enumerate(SAMPLED["settings"]):
        for tag, order in ORDERS.items():
            _, _, ids = po.run(model, tokens, order=order, gen=n_gen, temperature=t, top_k=k, top_p=p, seed=seed)
            assert ids == fx[f"{case}_s{j}_{tag}"].tolist(), f"{case} setting {j} {tag}"


def test_rng_is_xorshift64_star():
    # the engine's generator: x ^= x >> 12; x ^= x << 25; x ^= x >> 27; output x * 2685821657736338717
    M = (1 << 64) - 1
    x = 12345
    st = 12345
    for _ in range(100):
        x ^= x >> 12
        x ^= (x << 25) & M
        x ^= x >> 27
        out, st = po.rng_next(st)
        assert st == x and out == (x * 2685821657736338717) & M
    # a zero state starts from the golden-ratio constant, like a zero --seed
    assert po.rng_next(0) == po.rng_next(0x9E3779B97F4A7C15)


def test_sample_special_cases():
    rng = np.random.default_rng(0)
    v = rng.standard_normal(50).astype(np.float32)
    # temperature 0: the greedy argmax, generator untouched
    assert po.sample(v, 0.0, 0, 1.0, 99) == (int(np.argmax(v)), 99)
    # top-k 1: always the largest, whatever the draw
    for s in range(1, 20):
        assert po.sample(v, 0.7, 1, 1.0, s)[0] == int(np.argmax(v))
    # a tiny top-p keeps only the first kept token (the largest under top-k)
    assert po.sample(v, 1.0, 10, 1e-6, 5)[0] == int(np.argmax(v))
    # frequencies follow softmax(v / T) (a loose check of the draw against the distribution)
    T = 1.5
    p = np.exp((v - v.max()) / T)
    p /= p.sum()
    st, counts = 7, np.zeros(v.size)
    for _ in range(20000):
        t, st = po.sample(v, T, 0, 1.0, st)
        counts[t] += 1
    assert np.abs(counts / 20000 - p).max() < 0.01
