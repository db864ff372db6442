"""The oracle against the golden fixtures written by the reference engine itself
(tests/golden/make_golden.py: oracle/_ref/rabbit2 built from rabbit2/src/rabbit2.c).

Bitwise: logits and routing of --dump, and --gen ids, in both of the engine's orders. This pins
orc_run and everything under it (matvec orders, rmsnorm, softmax, top-k, SwiGLU, combine, rope,
attention, layout) to the reference, including one OLMoE-shaped layer at full MoE size."""
import hashlib
import json
import os

import numpy as np
import pytest

from oracle import pyoracle as po

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))
ORDERS = {"scalar": po.ORDER_SCALAR, "avx2": po.ORDER_AVX2}


def build(case):
    spec = MANIFEST["cases"][case]
    cfg = po.Config(**spec["config"])
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    return spec, cfg, model


@pytest.mark.parametrize("case", sorted(MANIFEST["cases"]))
def test_oracle_matches_reference_fixtures(case):
    spec, cfg, model = build(case)
    assert model.size == spec["model_bytes"]
    assert hashlib.sha256(model.tobytes()).hexdigest() == spec["model_sha256"], "the model writer changed"
    fx = np.load(os.path.join(GOLDEN, case + ".npz"))
    tokens = fx["tokens"]
    for tag, order in ORDERS.items():
        logits, routing, gen = po.run(model, tokens, order=order, gen=spec["n_gen"])
        assert logits.tobytes() == fx[f"logits_{tag}"].tobytes(), f"{case} {tag} logits"
        assert routing.tobytes() == fx[f"routing_{tag}"].tobytes(), f"{case} {tag} routing"
        assert gen == fx[f"gen_{tag}"].tolist(), f"{case} {tag} gen"
    # the portable lane-by-lane form of the AVX2 order is bitwise the same
    logits, routing, _ = po.run(model, tokens, order=po.ORDER_LANE16)
    assert logits.tobytes() == fx["logits_avx2"].tobytes()


def test_fixture_prompt_tokens_follow_the_documented_generator():
    for case, spec in MANIFEST["cases"].items():
        fx = np.load(os.path.join(GOLDEN, case + ".npz"))
        want = po.prompt_tokens(spec["gen_params"]["seed"], spec["n_prompt"], spec["config"]["vocab"])
        assert fx["tokens"].tolist() == want
