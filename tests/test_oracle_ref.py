"""The oracle against the live reference engine (oracle/_ref/rabbit2, compiled from
rabbit2/src/rabbit2.c by oracle/Makefile). Skipped where the reference checkout was not present
to build it; the committed fixtures (test_oracle_golden.py) cover those machines.

Method of the reference's own tests: seeded models through the same writer, --dump/--gen compared
(here bitwise rather than to a tolerance, since the oracle restates the engine's fp32 order), and
--info offsets of a sparse full-size OLMoE file (rabbit2/tests/test_layout_big.py:22-65)."""
import os

import numpy as np
import pytest

from oracle import pyoracle as po

pytestmark = pytest.mark.skipif(not po.have_ref(), reason="oracle/_ref/rabbit2 not built")

C = po.Config
# rabbit2/tests/test_forward.py:80-98 shapes
SHAPES = {
    "f32_gqa_renorm": C(),
    "bf16_gqa_renorm": C(dtype=1),
    "f32_qknorm_norenorm": C(qk_norm=1, norm_topk=0),
    "bf16_olmoe_like": C(vocab=100, dim=48, n_layers=3, n_heads=4, n_kv_heads=4, head_dim=12, n_experts=6, top_k=3,
                         expert_hidden=40, max_seq=32, dtype=1, qk_norm=1, norm_topk=0),
    "odd_f32": C(vocab=70, dim=36, n_layers=2, n_heads=6, n_kv_heads=3, head_dim=6, n_experts=5, top_k=2,
                 expert_hidden=25, max_seq=32),
    "top1_mha": C(vocab=64, dim=32, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=8, n_experts=4, top_k=1,
                  expert_hidden=64, max_seq=32),
}


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_oracle_bitwise_vs_reference_engine(tmp_path, shape, seed):
    cfg = SHAPES[shape]
    path = tmp_path / "m.rbt2"
    po.write_model(str(path), cfg, po.ref_style(seed))
    model = np.fromfile(path, dtype=np.uint8)
    tokens = po.prompt_tokens(seed, min(12, cfg.max_seq - 6), cfg.vocab)
    for kernel, order in ((None, po.ORDER_SCALAR), ("scalar", po.ORDER_SCALAR), ("avx2", po.ORDER_AVX2)):
        lb, rb, _ = po.ref_dump(path, tokens, str(tmp_path), kernel=kernel)
        logits, routing, gen = po.run(model, tokens, order=order, gen=6)
        assert logits.tobytes() == lb
        assert routing.tobytes() == rb
        assert gen == po.ref_gen(path, tokens, 6, kernel=kernel)


def test_oracle_eos_and_ctx_clamp_match_reference(tmp_path):
    cfg = SHAPES["bf16_gqa_renorm"]
    path = tmp_path / "m.rbt2"
    po.write_model(str(path), cfg, po.ref_style(5))
    model = np.fromfile(path, dtype=np.uint8)
    tokens = po.prompt_tokens(5, 8, cfg.vocab)
    full = po.ref_gen(path, tokens, 20)
    eos = full[3]
    assert po.run(model, tokens, gen=20, eos=eos)[2] == po.ref_gen(path, tokens, 20, extra=["--eos", str(eos)])
    assert po.run(model, tokens, gen=20, ctx=12)[2] == po.ref_gen(path, tokens, 20, extra=["--ctx", "12"])


def test_layout_matches_reference_info_on_sparse_olmoe_file(tmp_path):
    import subprocess
    cfg = C(vocab=50304, dim=2048, n_layers=16, n_heads=16, n_kv_heads=16, head_dim=128, n_experts=64, top_k=8,
            expert_hidden=1024, max_seq=4096, dtype=1, qk_norm=1, norm_topk=0)
    L = po.layout(cfg)
    path = tmp_path / "olmoe_sparse.rbt2"
    hdr = np.zeros(68, np.uint8)
    hdr[:4] = np.frombuffer(b"RBT2", np.uint8)
    hdr[4:8] = np.frombuffer(np.uint32(2).tobytes(), np.uint8)
    hdr[8:] = np.frombuffer(bytes(cfg), np.uint8)
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.truncate(po.model_file_size(cfg))
    res = subprocess.run([po.REF_BIN, str(path), "--info"], capture_output=True, text=True, check=True)
    kv = dict(tok.split("=") for line in res.stdout.splitlines() for tok in line.split())
    assert int(kv["tok_emb"]) == L["tok_emb"]
    assert int(kv["layer0_experts"]) == L["layers"][0]["experts"]
    assert int(kv["last_layer_experts"]) == L["layers"][-1]["experts"]
    assert int(kv["expert_stride"]) == L["expert_stride"]
    assert int(kv["lm_head"]) == L["lm_head"]
    assert int(kv["layout_end"]) == L["end"]


def test_reference_rejects_what_the_oracle_rejects(tmp_path):
    cfg = SHAPES["f32_gqa_renorm"]
    path = tmp_path / "m.rbt2"
    po.write_model(str(path), cfg, po.ref_style(0))
    model = np.fromfile(path, dtype=np.uint8)
    bad = model.copy()
    bad[0] = ord("X")
    with pytest.raises(ValueError, match="bad magic"):
        po.parse_header(bad)
    with pytest.raises(RuntimeError, match="token out of range"):
        po.run(model, [cfg.vocab])
    with pytest.raises(RuntimeError, match="too small"):
        po.run(model[: model.size // 2].copy(), [1])
    os.truncate(path, model.size // 2)
    import subprocess
    res = subprocess.run([po.REF_BIN, str(path), "--gen", "1", "1"], capture_output=True, text=True)
    assert res.returncode == 1 and "too small" in res.stderr
