"""Writes the golden fixtures in this directory from the reference engine itself.

    make -C oracle && python tests/golden/make_golden.py

For each case: the repository's own writer (oracle.pyoracle.write_model) creates a seeded .rbt2
model; the reference engine compiled from its source (oracle/_ref/rabbit2, see oracle/Makefile)
runs it with --dump and --gen, once in its scalar order (no --kernel flag, the engine default)
and once with --kernel avx2. The outputs (logits, routing, generated ids) and the SHA-256 of the
model file go into <case>.npz / manifest.json. Models are not committed; the tests regenerate
them and check the hash first.
"""
import hashlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle import pyoracle as po  # noqa: E402

C = po.Config
REF_STYLE = "ref_style"

# name: (config, gen params (seed, w_scale, fan_in, emb_scale, norm_jitter), prompt length, gen tokens)
CASES = {
    # The tiny OLMoE-style model: 2 layers, hidden 256, 4 heads, 8 experts top-2, expert hidden 128,
    # vocab 1024, fp32 weights ~N(0,0.02) from seed 0; 16 prompt ids; 32 greedy tokens.
    "tiny_olmoe_f32": (dict(vocab=1024, dim=256, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=64, n_experts=8,
                            top_k=2, expert_hidden=128, max_seq=64, dtype=0, qk_norm=1, norm_topk=0),
                       (0, 0.02, 0, 0.02, 0.0), 16, 32),
    "tiny_olmoe_bf16": (dict(vocab=1024, dim=256, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=64, n_experts=8,
                             top_k=2, expert_hidden=128, max_seq=64, dtype=1, qk_norm=1, norm_topk=0),
                        (0, 0.02, 0, 0.02, 0.0), 16, 32),
    # The shapes of the reference's engine test (rabbit2/tests/test_forward.py:80-98).
    "ref_default_f32": (dict(), (0, 1.0, 1, 0.5, 0.1), 12, 6),
    "ref_bf16": (dict(dtype=1), (0, 1.0, 1, 0.5, 0.1), 12, 6),
    "ref_qknorm_norenorm": (dict(qk_norm=1, norm_topk=0), (0, 1.0, 1, 0.5, 0.1), 12, 6),
    "ref_olmoe_like_top3of6": (dict(vocab=100, dim=48, n_layers=3, n_heads=4, n_kv_heads=4, head_dim=12, n_experts=6,
                                    top_k=3, expert_hidden=40, max_seq=32, dtype=1, qk_norm=1, norm_topk=0),
                               (0, 1.0, 1, 0.5, 0.1), 12, 6),
    "ref_odd_shape": (dict(vocab=70, dim=36, n_layers=2, n_heads=6, n_kv_heads=3, head_dim=6, n_experts=5, top_k=2,
                           expert_hidden=25, max_seq=32), (0, 1.0, 1, 0.5, 0.1), 12, 6),
    "ref_top1": (dict(vocab=64, dim=32, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=8, n_experts=4, top_k=1,
                      expert_hidden=64, max_seq=32), (0, 1.0, 1, 0.5, 0.1), 12, 6),
    # The reference's AVX2 tail cases (rabbit2/tests/test_avx2.py:52): dims 8 and 36 (< 16 / tails).
    "ref_tail_dim8": (dict(vocab=48, dim=8, n_layers=2, n_heads=2, n_kv_heads=2, head_dim=4, n_experts=4, top_k=2,
                           expert_hidden=7, max_seq=16, dtype=1, qk_norm=1, norm_topk=0), (23, 1.0, 1, 0.5, 0.1), 5, 4),
    # One OLMoE-1B-7B-shaped layer (MoE at full size: D 2048, E 64, top-8, H 1024, bf16).
    "olmoe_layer_bf16": (dict(vocab=256, dim=2048, n_layers=1, n_heads=16, n_kv_heads=16, head_dim=128, n_experts=64,
                              top_k=8, expert_hidden=1024, max_seq=16, dtype=1, qk_norm=1, norm_topk=0),
                         (1, 0.02, 0, 0.02, 0.0), 4, 2),
}


def make_case(name, spec, tmp):
    cfgd, g, nt, ngen = spec
    cfg = C(**cfgd)
    gp = po.GenParams(seed=g[0], w_scale=g[1], fan_in_scale=g[2], emb_scale=g[3], norm_jitter=g[4])
    path = os.path.join(tmp, name + ".rbt2")
    po.write_model(path, cfg, gp)
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    tokens = po.prompt_tokens(g[0], nt, cfg.vocab)
    arrays = {"tokens": np.array(tokens, np.int32)}
    for tag, kernel in (("scalar", None), ("avx2", "avx2")):
        lb, rb, _ = po.ref_dump(path, tokens, tmp, kernel=kernel)
        arrays[f"logits_{tag}"] = np.frombuffer(lb, "<f4").reshape(nt, cfg.vocab)
        arrays[f"routing_{tag}"] = np.frombuffer(rb, "<i4").reshape(nt, cfg.n_layers, cfg.top_k)
        arrays[f"gen_{tag}"] = np.array(po.ref_gen(path, tokens, ngen, kernel=kernel), np.int32)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
    os.remove(path)
    return {"config": cfg.as_dict(), "gen_params": {"seed": g[0], "w_scale": g[1], "fan_in_scale": g[2],
                                                    "emb_scale": g[3], "norm_jitter": g[4]},
            "n_prompt": nt, "n_gen": ngen, "model_sha256": h.hexdigest(), "model_bytes": po.model_file_size(cfg)}


def main():
    if not po.have_ref():
        sys.exit("oracle/_ref/rabbit2 is not built (make -C oracle with the reference checkout present)")
    manifest = {"engine": "oracle/_ref/rabbit2 built by oracle/Makefile from rabbit2/src/rabbit2.c",
                "orders": {"scalar": "no --kernel flag (engine default)", "avx2": "--kernel avx2"}, "cases": {}}
    with tempfile.TemporaryDirectory() as tmp:
        for name, spec in CASES.items():
            print("case", name, flush=True)
            manifest["cases"][name] = make_case(name, spec, tmp)
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
