"""The whole OLMoE-1B-7B-shaped model on the GPU at the sizes the benchmark runs, held to the oracle (the
engine's own forward(), rabbit2/src/rabbit2.c:453-548, bitwise the reference binary) and to its own
step-by-step results:

  * bs=1 decode: 16 layers, hidden 2048, 16 heads x 128 with QK-norm and RoPE, 64 experts top-8,
    SwiGLU 1024, vocab 50304, bf16 ~N(0, 0.02); a 128-token random prompt and 256 greedy tokens through
    the device loop (rbt_hip_generate, the engine's --gen loop :716-740).
  * batched decode on the same model: 32 sequences, at a 64-token context against the oracle run on
    sequences 0 and 31 alone, and at a 2048-token context + 64 greedy tokens against the same sequences
    decoded alone on the device (batch invariance).

Bar: routing identical to the oracle's in every (position, layer) checked, logits normwise within 1e-3,
greedy ids identical (a generated id may differ from the oracle's argmax only where the oracle's own
two largest logits are within that tolerance of each other).
"""
import numpy as np
import pytest

import bench
from oracle import pyoracle as po
from tests.common import normwise_err

pytestmark = pytest.mark.gpu
LOGIT_RTOL = 1e-3


def near_tie(logits, a, b):
    """The oracle's logits of ids a and b are equal within the tolerance (greedy may pick either)."""
    return abs(float(logits[a]) - float(logits[b])) <= LOGIT_RTOL * float(np.abs(logits).max())


@pytest.fixture(scope="module")
def full(dev):
    """The random-init model of the benchmark's whole-model legs, built once on the device."""
    from rabbitm2_amd import hip as rh
    cfg, secs = bench.make_full_model(dev)
    dev.set_router_order(rh.ORDER_AVX2)
    print(f"full model built on the device in {secs:.1f} s", flush=True)
    img = bench.read_model_image(dev, cfg)
    yield cfg, img
    del img


def test_bs1_decode_full_model(dev, full):
    cfg, img = full
    n_prompt, n_gen = bench.N_PROMPT, bench.N_GEN
    prompt = np.random.default_rng(bench.SEED).integers(0, cfg.vocab, n_prompt).astype(np.int32)
    dev.state_init(n_prompt + n_gen)
    ids, ms = dev.generate(prompt, n_gen)
    assert len(ids) == n_gen and all(0 <= t < cfg.vocab for t in ids)
    print(f"generate: {n_prompt} + {n_gen} tokens, {ms[1] / (n_gen - 1):.3f} ms per generated token", flush=True)
    # the device loop against step-by-step forwards over the whole run
    dev.state_init(n_prompt + n_gen)
    seq = prompt.tolist() + ids
    n_chk = n_prompt + 8  # positions the oracle checks: the prompt and the first 8 generated tokens
    got_l = np.zeros((n_chk, cfg.vocab), np.float32)
    got_r = np.zeros((n_chk, cfg.n_layers, cfg.top_k), np.int32)
    for pos in range(n_prompt + n_gen - 1):
        logits, routing = dev.forward(seq[pos], pos, cfg.vocab, cfg.n_layers, cfg.top_k)
        if pos < n_chk:
            got_l[pos], got_r[pos] = logits, routing
        if pos >= n_prompt - 1:
            assert int(np.argmax(logits)) == seq[pos + 1], f"pos {pos}: forward argmax vs the device loop"
    # the oracle on the same weights: the prompt and the first 8 generated tokens
    want_l, want_r, gen = po.run(img, seq[:n_chk], order=po.ORDER_AVX2, ctx=n_chk + 1, gen=1)
    worst = 0.0
    for pos in range(n_chk):
        assert np.array_equal(got_r[pos], want_r[pos]), f"pos {pos}: routing differs from the oracle"
        err = normwise_err(got_l[pos], want_l[pos])
        worst = max(worst, err)
        assert err <= LOGIT_RTOL, f"pos {pos}: logits error {err:.2e}"
    for i in range(8):
        want = int(np.argmax(want_l[n_prompt - 1 + i]))
        assert ids[i] == want or near_tie(want_l[n_prompt - 1 + i], ids[i], want), f"generated id {i}"
    assert gen == [seq[n_chk]] or near_tie(want_l[n_chk - 1], gen[0], seq[n_chk])
    print(f"bs=1: {n_chk} positions x 16 layers routing identical, worst logits error {worst:.2e}", flush=True)


def test_batched_decode_full_model(dev, full):
    cfg, img = full
    B = bench.B_SEQ
    # (a) 64-token context: sequences 0 and 31 against the oracle run on each alone, every position
    n = 64
    prompts = np.random.default_rng(bench.SEED + 9).integers(0, cfg.vocab, (B, n)).astype(np.int32)
    dev.batch_init(B, n)
    got = {b: ([], []) for b in (0, B - 1)}
    for p in range(n):
        logits, routing = dev.forward_batch(prompts[:, p], np.full(B, p, np.int32), cfg.vocab, cfg.n_layers,
                                            cfg.top_k)
        for b in got:
            got[b][0].append(logits[b].copy())
            got[b][1].append(routing[:, b, :].copy())
    for b, (gl, gr) in got.items():
        want_l, want_r, _ = po.run(img, prompts[b], order=po.ORDER_AVX2, ctx=n)
        for p in range(n):
            assert np.array_equal(gr[p], want_r[p]), f"seq {b} pos {p}: routing differs from the oracle"
            err = normwise_err(gl[p], want_l[p])
            assert err <= LOGIT_RTOL, f"seq {b} pos {p}: logits error {err:.2e}"
    print(f"batched: {B} sequences x {n} positions, sequences 0 and {B - 1} match the oracle", flush=True)
    # (b) the benchmark's 2048-token contexts + 64 greedy tokens: every sequence of the batch decodes as
    # it does alone (checked on the first and the last)
    ctx, n_gen = bench.B_CTX, bench.B_GEN
    prompts = np.random.default_rng(bench.SEED + 5).integers(0, cfg.vocab, (B, ctx)).astype(np.int32)
    dev.batch_init(B, ctx + n_gen)
    ids, (p_ms, g_ms) = dev.generate_batch(prompts, n_gen)
    print(f"batched generate: context fill {p_ms / 1e3:.1f} s, {g_ms / (n_gen - 1):.2f} ms per step", flush=True)
    for b in (0, B - 1):
        dev.state_init(ctx + n_gen)
        alone, _ = dev.generate(prompts[b], n_gen)
        assert ids[b].tolist() == alone, f"seq {b}: the batch and the sequence alone differ"
