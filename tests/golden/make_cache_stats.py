"""Writes cache_stats.json in this directory from the reference engine itself.

    make -C oracle && python tests/golden/make_cache_stats.py

For several golden models (regenerated from manifest.json by the repository's own writer), the
reference engine compiled from its source (oracle/_ref/rabbit2) runs --dump and --gen with
--expert-cache-mib at budgets that force evictions and at budgets that hold every expert. Its stderr
expert-cache line (rabbit2/src/rabbit2.c:745-751) is parsed into the six counters and stored with the
run's arguments. The counters depend only on the routing stream the engine walks and the budget, so
they pin an LRU replay over the same routing (tests/test_cache_replay.py) and the command line's
stats line on the GPU (tests/test_gpu_cli.py).
"""
import json
import os
import re
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle import pyoracle as po  # noqa: E402

STATS_RE = re.compile(r"(hits|misses|evictions|bytes_read|resident_bytes|capacity_bytes)=(\d+)")

# case: budgets in MiB (the first forces evictions, the last holds every expert or comes close)
RUNS = {
    "tiny_olmoe_f32": (1, 2, 8),            # expert stride 384 KiB, 16 experts
    "tiny_olmoe_bf16": (1, 4),              # 192 KiB, 16 experts
    "ref_default_f32": (1, 2),              # 96 KiB, 16 experts
    "ref_olmoe_like_top3of6": (1,),         # 12 KiB, 18 experts: everything fits
    "olmoe_layer_bf16": (24, 100, 800),     # 12 MiB, 64 experts
}
KERNELS = {"scalar": None, "avx2": "avx2"}


def run_ref(args):
    res = subprocess.run([po.REF_BIN] + [str(a) for a in args], capture_output=True, text=True, check=True)
    stats = {k: int(v) for k, v in STATS_RE.findall(res.stderr)}
    assert len(stats) == 6, res.stderr
    return stats, res.stdout


def main():
    if not po.have_ref():
        sys.exit("oracle/_ref/rabbit2 is not built (make -C oracle with the reference checkout present)")
    manifest = json.load(open(os.path.join(HERE, "manifest.json")))
    out = {"engine": manifest["engine"], "runs": []}
    with tempfile.TemporaryDirectory() as tmp:
        for case, budgets in RUNS.items():
            spec = manifest["cases"][case]
            cfg = po.Config(**spec["config"])
            g = spec["gen_params"]
            path = os.path.join(tmp, case + ".rbt2")
            po.write_model(path, cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"],
                                                   fan_in_scale=g["fan_in_scale"], emb_scale=g["emb_scale"],
                                                   norm_jitter=g["norm_jitter"]))
            tokens = po.prompt_tokens(g["seed"], spec["n_prompt"], cfg.vocab)
            for tag, kernel in KERNELS.items():
                kargs = ["--kernel", kernel] if kernel else []
                for mib in budgets:
                    print(case, tag, mib, flush=True)
                    lp, rp = os.path.join(tmp, "l.bin"), os.path.join(tmp, "r.bin")
                    dump, _ = run_ref([path, "--dump", lp, rp, "--expert-cache-mib", mib] + kargs + tokens)
                    gen, stdout = run_ref([path, "--gen", spec["n_gen"], "--expert-cache-mib", mib] + kargs + tokens)
                    out["runs"].append({"case": case, "order": tag, "budget_mib": mib, "tokens": tokens,
                                        "n_gen": spec["n_gen"], "gen_ids": [int(t) for t in stdout.split()],
                                        "dump": dump, "gen": gen})
            os.remove(path)
    with open(os.path.join(HERE, "cache_stats.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
