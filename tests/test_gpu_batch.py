"""Batched decode (rbt_hip_batch_init / rbt_hip_forward_batch / rbt_hip_generate_batch): n_seq
independent sequences stepped together, each with its own KV cache. Each sequence must behave as the
engine's forward() on that sequence alone (rabbit2/src/rabbit2.c:453-548, the --dump and --gen loops
:703-740): the oracle (bitwise the reference engine, pinned by the golden fixtures) runs every
sequence on its own, and the batch must match it -- routing identical in every (token, layer),
logits normwise within 1e-3, greedy ids identical. Batches of 16+ tokens take the grouped MoE path.
"""
import json
import os

import numpy as np
import pytest

from oracle import pyoracle as po
from tests.common import normwise_err

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))
LOGIT_RTOL = 1e-3


def build(case):
    spec = MANIFEST["cases"][case]
    cfg = po.Config(**spec["config"])
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    return spec, cfg, model


def prompts_for(cfg, B, n, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, cfg.vocab, (B, n)).astype(np.int32)


# (case, B, positions): tiny models with the per-token fallbacks and the dense batch kernels, a tiny bf16
# model (8 experts, top-2) and the OLMoE-shaped layer at 16 sequences (grouped MoE path behind the
# decode router kernel and the top-k + split launch, batched dense matvecs, 16 heads x 128)
CASES = [("tiny_olmoe_f32", 3, 6), ("ref_odd_shape", 4, 5), ("ref_qknorm_norenorm", 5, 5),
         ("tiny_olmoe_bf16", 16, 4), ("olmoe_layer_bf16", 16, 3)]


def test_forward_batch_long_context_olmoe_heads(dev):
    """The OLMoE-shaped layer (16 heads x 128, QK-norm) over 1100 positions of two sequences: 16
    position splits of up to 69 positions, so every wave of the attention blocks takes several rounds
    of 8 positions and the splits merge; each sequence against the oracle run on it alone at every
    position (routing identical, logits normwise within 1e-3)."""
    spec = MANIFEST["cases"]["olmoe_layer_bf16"]
    conf = dict(spec["config"], max_seq=2048)
    cfg = po.Config(**conf)
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    B, n = 2, 1100
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    prompts = prompts_for(cfg, B, n, seed=11)
    want = [po.run(model, prompts[b], order=po.ORDER_AVX2, ctx=n) for b in range(B)]
    dev.batch_init(B, n)
    for p in range(n):
        logits, routing = dev.forward_batch(prompts[:, p], np.full(B, p, np.int32), cfg.vocab, cfg.n_layers,
                                            cfg.top_k)
        for b in range(B):
            wl, wr, _ = want[b]
            assert np.array_equal(routing[:, b, :], wr[p]), f"seq {b} pos {p}"
            err = normwise_err(logits[b], wl[p])
            assert err <= LOGIT_RTOL, f"seq {b} pos {p}: logits error {err:.2e}"


@pytest.mark.parametrize("case,B,n", CASES, ids=[c[0] + f"_B{c[1]}" for c in CASES])
def test_forward_batch_matches_each_sequence_alone(dev, case, B, n):
    spec, cfg, model = build(case)
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    prompts = prompts_for(cfg, B, n, seed=B)
    want = [po.run(model, prompts[b], order=po.ORDER_AVX2) for b in range(B)]
    dev.batch_init(B, 0)
    for p in range(n):
        logits, routing = dev.forward_batch(prompts[:, p], np.full(B, p, np.int32), cfg.vocab, cfg.n_layers,
                                            cfg.top_k)
        for b in range(B):
            wl, wr, _ = want[b]
            assert np.array_equal(routing[:, b, :], wr[p]), f"{case} seq {b} pos {p}"
            err = normwise_err(logits[b], wl[p])
            assert err <= LOGIT_RTOL, f"{case} seq {b} pos {p}: logits error {err:.2e}"


@pytest.mark.parametrize("B,vocab", [(33, 256), (64, 256), (33, 8192)])
def test_batch_matrix_core_matvecs_agree_with_vector_ones(dev, B, vocab):
    """The batched q/k/v, wo and lm_head on the matrix cores (option batch_mfma, the default; B = 33 fills
    a last block of 16 tokens with one sequence) against the VALU dot products: routing identical,
    logits within rounding of each other, and the first and last sequences against the oracle. Below 256
    row tiles of 16 (wo, and lm_head at vocab 256) a block takes one 16-token block, from 256 on (q/k/v,
    lm_head at vocab 8192) every token block."""
    if vocab == 256:
        spec, cfg, model = build("olmoe_layer_bf16")
    else:
        spec = MANIFEST["cases"]["olmoe_layer_bf16"]
        cfg = po.Config(**dict(spec["config"], vocab=vocab))
        g = spec["gen_params"]
        model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                                 emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    prompts = prompts_for(cfg, B, 2, seed=B + 100)
    runs = {}
    try:
        for mode in (1, 0):
            dev.set_option("batch_mfma", mode)
            dev.batch_init(B, 0)
            runs[mode] = [dev.forward_batch(prompts[:, p], np.full(B, p, np.int32), cfg.vocab, cfg.n_layers,
                                            cfg.top_k) for p in range(2)]
    finally:
        dev.set_option("batch_mfma", 1)
    for p in range(2):
        (lm, rm), (lv, rv) = runs[1][p], runs[0][p]
        assert np.array_equal(rm, rv)
        for b in range(B):
            assert normwise_err(lm[b], lv[b]) <= 1e-4
    for b in (0, B - 1):
        wl, wr, _ = po.run(model, prompts[b], order=po.ORDER_AVX2)
        for p in range(2):
            assert np.array_equal(runs[1][p][1][:, b, :], wr[p])
            assert normwise_err(runs[1][p][0][b], wl[p]) <= LOGIT_RTOL


def test_forward_batch_grouped_front_end_renormalised(dev):
    """The grouped MoE path of the batched forward with renormalised top-k weights (norm_topk = 1) and
    20 sequences: the router kernel's logits, the per-token top-k + split launch and the combine
    against the oracle run on each sequence alone."""
    spec = MANIFEST["cases"]["tiny_olmoe_bf16"]
    cfg = po.Config(**dict(spec["config"], norm_topk=1))
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"] + 7, w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    B, n = 20, 3
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    prompts = prompts_for(cfg, B, n, seed=21)
    want = [po.run(model, prompts[b], order=po.ORDER_AVX2) for b in range(B)]
    dev.batch_init(B, 0)
    for p in range(n):
        logits, routing = dev.forward_batch(prompts[:, p], np.full(B, p, np.int32), cfg.vocab, cfg.n_layers,
                                            cfg.top_k)
        for b in range(B):
            wl, wr, _ = want[b]
            assert np.array_equal(routing[:, b, :], wr[p]), f"seq {b} pos {p}"
            assert normwise_err(logits[b], wl[p]) <= LOGIT_RTOL, f"seq {b} pos {p}"


def test_forward_batch_grouped_top10_of_16(dev):
    """The grouped MoE path of the batched forward with more than 8 selected experts (16 experts,
    top-10): the per-token top-k launch, the combine's general loop and a separate RMSNorm launch
    (the fused combine + RMSNorm takes at most 8), against the oracle on each sequence alone."""
    spec = MANIFEST["cases"]["tiny_olmoe_bf16"]
    cfg = po.Config(**dict(spec["config"], n_experts=16, top_k=10))
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"] + 3, w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    B, n = 16, 3
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    prompts = prompts_for(cfg, B, n, seed=23)
    want = [po.run(model, prompts[b], order=po.ORDER_AVX2) for b in range(B)]
    dev.batch_init(B, 0)
    for p in range(n):
        logits, routing = dev.forward_batch(prompts[:, p], np.full(B, p, np.int32), cfg.vocab, cfg.n_layers,
                                            cfg.top_k)
        for b in range(B):
            wl, wr, _ = want[b]
            assert np.array_equal(routing[:, b, :], wr[p]), f"seq {b} pos {p}"
            assert normwise_err(logits[b], wl[p]) <= LOGIT_RTOL, f"seq {b} pos {p}"


def test_forward_batch_sequences_restart_independently(dev):
    """Sequence 1 starts over at position 0 every 3 steps while sequence 0 runs on: each is its own
    forward() stream (a restart overwrites only that sequence's cache)."""
    spec, cfg, model = build("tiny_olmoe_bf16")
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    prompts = prompts_for(cfg, 2, 7, seed=3)
    dev.batch_init(2, 0)
    for p in range(7):
        pos = np.array([p, p % 3], np.int32)
        logits, routing = dev.forward_batch(prompts[:, p], pos, cfg.vocab, cfg.n_layers, cfg.top_k)
        w0 = po.run(model, prompts[0, :p + 1], order=po.ORDER_AVX2)
        s1 = prompts[1, p - p % 3:p + 1]
        w1 = po.run(model, s1, order=po.ORDER_AVX2)
        assert np.array_equal(routing[:, 0, :], w0[1][p])
        assert np.array_equal(routing[:, 1, :], w1[1][len(s1) - 1])
        assert normwise_err(logits[0], w0[0][p]) <= LOGIT_RTOL
        assert normwise_err(logits[1], w1[0][len(s1) - 1]) <= LOGIT_RTOL


@pytest.mark.parametrize("case,B", [("ref_bf16", 4), ("olmoe_layer_bf16", 16)])
def test_generate_batch_matches_each_sequence_alone(dev, case, B):
    spec, cfg, model = build(case)
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    fx = np.load(os.path.join(GOLDEN, case + ".npz"))
    n = len(fx["tokens"])
    prompts = prompts_for(cfg, B, n, seed=11)
    prompts[0] = fx["tokens"]  # sequence 0: the fixture's prompt, whose --gen ids the reference wrote
    n_gen = spec["n_gen"]
    dev.batch_init(B, n + n_gen)
    ids, ms = dev.generate_batch(prompts, n_gen)
    assert ids[0].tolist() == fx["gen_avx2"].tolist()
    for b in range(1, B):
        _, _, gen = po.run(model, prompts[b], order=po.ORDER_AVX2, gen=n_gen, ctx=n + n_gen)
        assert ids[b].tolist() == gen, f"{case} seq {b}"


def test_batch_arguments_checked(dev):
    from rabbitm2_amd.hip import HipError
    spec, cfg, model = build("ref_bf16")
    dev.upload(model)
    dev.batch_init(2, 8)
    with pytest.raises(HipError):
        dev.forward(0, 0, cfg.vocab, cfg.n_layers, cfg.top_k)  # the state holds two sequences
    with pytest.raises(HipError):
        dev.forward_batch([0, cfg.vocab], [0, 0], cfg.vocab, cfg.n_layers, cfg.top_k)
    with pytest.raises(HipError):
        dev.forward_batch([0, 0], [0, 8], cfg.vocab, cfg.n_layers, cfg.top_k)
    with pytest.raises(HipError):
        dev.generate_batch(np.zeros((2, 6), np.int32), 3)  # 6 + 3 > ctx 8


def test_forward_batch_one_split_many_rounds(dev):
    """32 sequences at the OLMoE head shape (16 heads x 128, QK-norm): 512 (sequence, head) blocks take one
    position split each, and the attention kernel writes its output itself with no merge launch. Over 400
    positions every wave of a block loops over up to 13 rounds of 8 positions. Sequences 0 and 31 are
    checked against the oracle run on each alone at every position (routing identical, logits normwise
    within 1e-3)."""
    spec = MANIFEST["cases"]["olmoe_layer_bf16"]
    cfg = po.Config(**dict(spec["config"], max_seq=512))
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    B, n = 32, 400
    assert B * cfg.n_heads >= 512  # the one-split attention (kAttnDirectBlocks)
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    prompts = prompts_for(cfg, B, n, seed=41)
    want = {b: po.run(model, prompts[b], order=po.ORDER_AVX2, ctx=n) for b in (0, B - 1)}
    dev.batch_init(B, n)
    for p in range(n):
        logits, routing = dev.forward_batch(prompts[:, p], np.full(B, p, np.int32), cfg.vocab, cfg.n_layers,
                                            cfg.top_k)
        for b, (wl, wr, _) in want.items():
            assert np.array_equal(routing[:, b, :], wr[p]), f"seq {b} pos {p}"
            err = normwise_err(logits[b], wl[p])
            assert err <= LOGIT_RTOL, f"seq {b} pos {p}: logits error {err:.2e}"


def test_deferred_profile_on_the_fused_combine_path(dev):
    """Deferred profiling (mode 2) of batched steps whose combine runs fused with the next RMSNorm: every
    event pair taken is recorded, so every kernel kind reads back, and the timed steps still match the
    oracle."""
    spec, cfg, model = build("olmoe_layer_bf16")
    B = 16
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    prompts = prompts_for(cfg, B, 2, seed=5)
    dev.batch_init(B, 0)
    dev.profile(2)
    try:
        outs = [dev.forward_batch(prompts[:, p], np.full(B, p, np.int32), cfg.vocab, cfg.n_layers, cfg.top_k)
                for p in range(2)]
        counts = {}
        for name in ("router", "topk", "dispatch", "gateup", "down_combine", "combine", "qkv", "attention", "wo",
                     "lm_head"):
            ms, launches = dev.profile_get(name)
            counts[name] = launches
            assert launches == 0 or ms > 0, name
        assert counts["combine"] == 2 and counts["gateup"] == 2, counts
    finally:
        dev.profile(0)
    wl, wr, _ = po.run(model, prompts[0], order=po.ORDER_AVX2)
    for p in range(2):
        assert np.array_equal(outs[p][1][:, 0, :], wr[p])
        assert normwise_err(outs[p][0][0], wl[p]) <= LOGIT_RTOL
