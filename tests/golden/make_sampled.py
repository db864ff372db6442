"""Writes sampled.npz / sampled.json: the reference engine's --gen output with its sampler
(--temperature, --top-k, --top-p, --seed; rabbit2/src/rabbit2.c:558-610, :716-740) for a few golden
models, in both of its orders.

    make -C oracle && python tests/golden/make_sampled.py

The models are those of make_golden.py (same writer, same seeds; the tests rebuild them and check
their hashes against manifest.json); the engine binary is oracle/_ref/rabbit2.
"""
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle import pyoracle as po  # noqa: E402

CASES = ("tiny_olmoe_f32", "tiny_olmoe_bf16", "ref_bf16", "ref_odd_shape", "olmoe_layer_bf16")
# (temperature, top_k, top_p, seed): top-k with top-p; the whole vocabulary; top-p over the vocabulary
# order (no top-k); a small top-k with the engine's default seed (0)
SETTINGS = ((0.8, 40, 0.9, 7), (1.0, 0, 1.0, 3), (0.6, 0, 0.8, 11), (1.3, 5, 1.0, 0))


def flags(s):
    t, k, p, seed = s
    return ["--temperature", repr(t), "--top-k", str(k), "--top-p", repr(p), "--seed", str(seed)]


def main():
    if not po.have_ref():
        sys.exit("oracle/_ref/rabbit2 is not built (make -C oracle with the reference checkout present)")
    manifest = json.load(open(os.path.join(HERE, "manifest.json")))["cases"]
    arrays, meta = {}, {"settings": SETTINGS, "cases": {}}
    with tempfile.TemporaryDirectory() as tmp:
        for name in CASES:
            spec = manifest[name]
            cfg = po.Config(**spec["config"])
            g = spec["gen_params"]
            gp = po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                              emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"])
            path = os.path.join(tmp, name + ".rbt2")
            po.write_model(path, cfg, gp)
            tokens = po.prompt_tokens(g["seed"], spec["n_prompt"], cfg.vocab)
            n_gen = max(spec["n_gen"], 8)
            meta["cases"][name] = {"n_gen": n_gen}
            for j, st in enumerate(SETTINGS):
                for tag, kernel in (("scalar", None), ("avx2", "avx2")):
                    ids = po.ref_gen(path, tokens, n_gen, kernel=kernel, extra=flags(st))
                    arrays[f"{name}_s{j}_{tag}"] = np.array(ids, np.int32)
            os.remove(path)
            print("case", name, flush=True)
    np.savez_compressed(os.path.join(HERE, "sampled.npz"), **arrays)
    with open(os.path.join(HERE, "sampled.json"), "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
