"""The device sampler (rbt_hip_set_sampling + rbt_hip_generate / rbt_hip_generate_batch) against the
reference engine's own sampled --gen output (tests/golden/sampled.npz: --temperature / --top-k /
--top-p / --seed, rabbit2/src/rabbit2.c:569-610, :716-740): identical ids for every model, setting and
order. The device logits agree with the engine's to rounding, so a draw could only differ where it
falls within rounding of a cumulative-probability boundary; none does in these cases."""
import json
import os

import numpy as np
import pytest

from oracle import pyoracle as po

pytestmark = pytest.mark.gpu

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
def test_sampled_generate_matches_reference(dev, case):
    spec, cfg, model = build(case)
    fx = np.load(os.path.join(GOLDEN, "sampled.npz"))
    tokens = po.prompt_tokens(spec["gen_params"]["seed"], spec["n_prompt"], cfg.vocab)
    n_gen = SAMPLED["cases"][case]["n_gen"]
    dev.upload(model)
    try:
        for j, (t, k, p, seed) in enumerate(SAMPLED["settings"]):
            dev.set_sampling(t, k, p, seed)
            for tag, order in ORDERS.items():
                dev.set_router_order(order)
                dev.state_init(0)
                ids, _ = dev.generate(tokens, n_gen)
                assert ids == fx[f"{case}_s{j}_{tag}"].tolist(), f"{case} setting {j} {tag}"
    finally:
        dev.set_sampling(0.0)


def test_sampled_generate_batch_matches_reference(dev):
    """Four sequences with the fixture's prompt and the same seed each reproduce the engine's draws."""
    case = "tiny_olmoe_f32"
    spec, cfg, model = build(case)
    fx = np.load(os.path.join(GOLDEN, "sampled.npz"))
    tokens = po.prompt_tokens(spec["gen_params"]["seed"], spec["n_prompt"], cfg.vocab)
    n_gen = SAMPLED["cases"][case]["n_gen"]
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    try:
        for j, (t, k, p, seed) in enumerate(SAMPLED["settings"]):
            dev.set_sampling(t, k, p, seed)
            dev.batch_init(4, len(tokens) + n_gen)
            ids, _ = dev.generate_batch(np.tile(np.array(tokens, np.int32), (4, 1)), n_gen)
            for b in range(4):
                assert ids[b].tolist() == fx[f"{case}_s{j}_avx2"].tolist(), f"setting {j} seq {b}"
    finally:
        dev.set_sampling(0.0)
