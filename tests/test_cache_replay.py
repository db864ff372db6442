"""The engine's expert-cache counters (rabbit2/src/rabbit2.c:236-300, stats line :745-751) replayed by
the library's host-only rbt_hip_expert_cache_replay over a routing stream.

Pinned two ways, on the CPU:
  * against the reference engine's own stats lines (tests/golden/cache_stats.json, written by the
    reference binary through make_cache_stats.py) for --dump and --gen runs at budgets that evict and
    budgets that hold every expert, replaying the routing the engine walked (the golden fixtures'
    --dump routing; for --gen, the oracle's routing over the prompt and the generated ids);
  * against an independent least-recently-used cache (an OrderedDict) on random routing streams: the
    engine's victim rule (first never-filled slot, else the smallest last-use clock) is plain LRU.
"""
import collections
import functools
import json
import os

import numpy as np
import pytest

from oracle import pyoracle as po
from rabbitm2_amd import hip

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
FIX = json.load(open(os.path.join(GOLDEN, "cache_stats.json")))
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))
ORDERS = {"scalar": po.ORDER_SCALAR, "avx2": po.ORDER_AVX2}
MIB = 1024 * 1024


@functools.lru_cache(maxsize=None)
def model_of(case):
    spec = MANIFEST["cases"][case]
    cfg = po.Config(**spec["config"])
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    return cfg, model


def lru_counts(routing, n_layers, n_experts, cap):
    """Textbook LRU over (layer, expert) keys in token, layer, slot order."""
    cache = collections.OrderedDict()
    hits = misses = ev = 0
    for tok in routing:
        for l, row in enumerate(tok):
            for e in row:
                key = (l, int(e))
                if key in cache:
                    cache.move_to_end(key)
                    hits += 1
                    continue
                misses += 1
                if len(cache) == cap:
                    cache.popitem(last=False)
                    ev += 1
                cache[key] = True
    return hits, misses, ev, min(misses, cap)


@pytest.mark.parametrize("run", FIX["runs"], ids=[f"{r['case']}_{r['order']}_{r['budget_mib']}MiB" for r in FIX["runs"]])
def test_replay_matches_the_engine_counters(run):
    cfg, model = model_of(run["case"])
    stride = po.layout(cfg)["expert_stride"]
    fx = np.load(os.path.join(GOLDEN, run["case"] + ".npz"))
    order = ORDERS[run["order"]]
    assert fx["tokens"].tolist() == run["tokens"]
    # --dump: the prompt's routing, as the reference wrote it
    got = hip.expert_cache_replay(run["budget_mib"] * MIB, stride, fx[f"routing_{run['order']}"], cfg.n_experts)
    assert got == run["dump"]
    # --gen: forward() of the prompt, then of every generated id but the last (rabbit2.c:704, :732-733)
    ids = run["gen_ids"]
    assert ids == fx[f"gen_{run['order']}"].tolist()
    seq = run["tokens"] + ids[:-1]
    _, routing, _ = po.run(model, seq, order=order, ctx=len(seq))
    assert np.array_equal(routing[:len(run["tokens"])], fx[f"routing_{run['order']}"])
    got = hip.expert_cache_replay(run["budget_mib"] * MIB, stride, routing, cfg.n_experts)
    assert got == run["gen"]


@pytest.mark.parametrize("seed", range(6))
def test_replay_is_lru(seed):
    rng = np.random.default_rng(seed)
    L, E, K, T = int(rng.integers(1, 4)), int(rng.integers(2, 12)), 0, int(rng.integers(1, 60))
    K = int(rng.integers(1, E + 1))
    routing = np.stack([np.stack([rng.permutation(E)[:K] for _ in range(L)]) for _ in range(T)]).astype(np.int32)
    stride = 4096 * int(rng.integers(1, 5))
    for cap in (1, 2, 3, L * E // 2 + 1, L * E, L * E + 7):
        got = hip.expert_cache_replay(cap * stride + stride // 2, stride, routing, E)
        hits, misses, ev, resident = lru_counts(routing, L, E, min(cap, L * E))
        assert (got["hits"], got["misses"], got["evictions"]) == (hits, misses, ev), cap
        assert got["bytes_read"] == misses * stride
        assert got["resident_bytes"] == resident * stride
        assert got["capacity_bytes"] == min(cap, L * E) * stride
        assert hits + misses == T * L * K


def test_replay_rejects_what_the_engine_rejects():
    routing = np.zeros((1, 1, 1), np.int32)
    with pytest.raises(hip.HipError, match="budget too small"):
        hip.expert_cache_replay(4095, 4096, routing, 4)  # rabbit2.c:238-242
    with pytest.raises(hip.HipError, match="out of range"):
        hip.expert_cache_replay(8192, 4096, np.full((1, 1, 1), 4, np.int32), 4)
    empty = hip.expert_cache_replay(8192, 4096, np.zeros((0, 1, 1), np.int32), 4)
    assert empty == {"hits": 0, "misses": 0, "evictions": 0, "bytes_read": 0, "resident_bytes": 0,
                     "capacity_bytes": 8192}
