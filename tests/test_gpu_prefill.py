"""Parity of the grouped (prefill) MoE path: dispatch, MFMA gate/up and down GEMMs, combine.

Many tokens per call go through per-expert lists instead of per-(token, slot) GEMVs
(rabbitm2_amd/csrc/prefill.hip). The engine evaluates them one token at a time
(rabbit2/src/rabbit2.c:703-714, MoE block :511-542); per token the result must meet the same bar as
decode: routing identical except at exact CPU ties, normwise max error <= 1e-3 (tests/common.py).
The tokens-per-expert histogram must equal the count of the oracle's routing exactly.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.common import MOE_RTOL, SynthLayer, normwise_err, routing_check

pytestmark = pytest.mark.gpu

GROUPED_DEFAULT_MIN = 12  # kPrefillMinTokensDefault in rbt2_internal.h


@pytest.fixture
def grouped_from(dev):
    """Sets the smallest batch that takes the grouped path; restores the default afterwards."""
    def set_min(n):
        dev.set_option("prefill_min_tokens", n)
    yield set_min
    dev.set_option("prefill_min_tokens", GROUPED_DEFAULT_MIN)


def check_grouped(dev, layer, xb, x=None, label=""):
    dev.set_router_order(po.ORDER_AVX2)
    want = layer.oracle(xb, po.ORDER_AVX2, x=x)
    got = layer.run_gpu(xb, x=x)
    bad, unexplained = routing_check(got["routing"], want["routing"], want["probs"])
    err = normwise_err(got["moe"], want["moe"])
    # per-token bar as well: every token's output row meets the tolerance against its own scale
    tok_err = max(normwise_err(g, w) for g, w in zip(got["moe"], want["moe"])) if len(xb) else 0.0
    counts = dev.expert_counts(layer.E)
    hist = np.bincount(got["routing"].ravel(), minlength=layer.E)
    print(f"{label} T={xb.shape[0]}: routing mismatched tokens {bad} (unexplained {unexplained}), "
          f"moe err {err:.2e}, worst token err {tok_err:.2e}, max tokens/expert {hist.max()}", flush=True)
    assert unexplained == 0
    assert err <= MOE_RTOL
    assert tok_err <= MOE_RTOL
    assert counts is not None
    assert np.array_equal(counts, hist)
    if bad == 0:
        assert np.array_equal(counts, np.bincount(want["routing"].ravel(), minlength=layer.E))
    if x is not None:
        assert normwise_err(got["x"], want["x"]) <= MOE_RTOL
    return got, want


# (dim, E, K, H, norm_topk, T): whole tiles of 128 (gate/up) / 256 (down) columns
GROUPED_SHAPES = [
    (256, 8, 2, 128, 1, 3),      # one column tile each way; most experts see 0-1 pairs
    (512, 16, 4, 256, 0, 40),    # 160 pairs over 16 experts: partial row tiles
    (1024, 64, 8, 128, 1, 17),   # E 64, K 8 with 17 tokens: many experts with 1-3 rows
    (768, 256, 6, 384, 0, 33),   # E 256 (the dispatch maximum), H 384
    (2048, 64, 8, 1024, 1, 100),  # OLMoE layer, 800 pairs: ~12 rows per expert
    (768, 64, 8, 256, 0, 21),    # E <= 64: one-launch router + top-k, 768 = a full and a half column chunk
]


@pytest.mark.parametrize("shape", GROUPED_SHAPES,
                         ids=[f"D{s[0]}E{s[1]}K{s[2]}H{s[3]}n{s[4]}T{s[5]}" for s in GROUPED_SHAPES])
def test_grouped_shapes(dev, grouped_from, shape):
    D, E, K, H, nt, T = shape
    grouped_from(1)
    layer = SynthLayer(dev, D, E, K, H, po.DT_BF16, nt, seed=6, w_scale=1.0, fan_in=True)
    try:
        xb = layer.make_x(T, seed=31)
        x = layer.make_x(T, seed=32, bf16=False)
        check_grouped(dev, layer, xb, x=x, label=f"grouped D{D}E{E}K{K}H{H}")
    finally:
        layer.close()


@pytest.mark.parametrize("T", [2048, 2100])
def test_grouped_pairs_past_dispatch_registers(dev, grouped_from, T):
    """More than 16 x 64 x 4 = 4096 (token, slot) pairs: the dispatch keeps the first 4096 pairs' experts
    and ranks in registers and carries the rest through pos_of; both halves must land in the lists."""
    grouped_from(1)
    layer = SynthLayer(dev, 256, 8, 2, 128, po.DT_BF16, 1, seed=11, w_scale=1.0, fan_in=True)
    try:
        xb = layer.make_x(T, seed=41)
        check_grouped(dev, layer, xb, label=f"{T * 2} pairs")
    finally:
        layer.close()


def test_grouped_matches_gemv_path(dev, grouped_from):
    """The same 24 tokens through the grouped path and the per-pair GEMV path: same routing and
    weights (the router is shared), outputs within the bar of each other and of the oracle."""
    layer = SynthLayer(dev, 2048, 64, 8, 1024, po.DT_BF16, 1, seed=1)
    try:
        xb = layer.make_x(24, seed=8)
        grouped_from(1)
        g, want = check_grouped(dev, layer, xb, label="grouped")
        grouped_from(1 << 16)
        v = layer.run_gpu(xb)
        assert np.array_equal(g["routing"], v["routing"])
        assert np.array_equal(g["weights"], v["weights"])
        assert normwise_err(v["moe"], want["moe"]) <= MOE_RTOL
        assert normwise_err(g["moe"], v["moe"]) <= MOE_RTOL
    finally:
        layer.close()


def test_grouped_one_hot_expert_set(dev, grouped_from):
    """Every token routed to the same 8 experts (+30 on their router logits): 8 lists of 300 rows,
    5 row tiles each, 56 experts empty."""
    grouped_from(1)
    bias = np.zeros(64, np.float32)
    bias[10:18] = 30.0
    layer = SynthLayer(dev, 2048, 64, 8, 1024, po.DT_BF16, 0, seed=2, bias=bias)
    try:
        xb = layer.make_x(300, seed=9)
        got, _ = check_grouped(dev, layer, xb, label="hot set")
        counts = dev.expert_counts(64)
        assert counts[10:18].tolist() == [300] * 8 and counts.sum() == 2400
    finally:
        layer.close()


def test_grouped_deterministic(dev, grouped_from):
    grouped_from(1)
    layer = SynthLayer(dev, 1024, 64, 8, 128, po.DT_BF16, 1, seed=3)
    try:
        xb = layer.make_x(64, seed=10)
        a = layer.run_gpu(xb)
        b = layer.run_gpu(xb)
        assert a["moe"].tobytes() == b["moe"].tobytes()
        assert np.array_equal(a["routing"], b["routing"])
    finally:
        layer.close()


def test_grouped_not_taken_for_f32(dev, grouped_from):
    """f32 weights stay on the GEMV path (the MFMA path multiplies bf16 weights); results still meet
    the bar."""
    grouped_from(1)
    layer = SynthLayer(dev, 256, 8, 2, 256, po.DT_F32, 1, seed=4, w_scale=1.0, fan_in=True)
    try:
        xb = layer.make_x(20, seed=12)
        want = layer.oracle(xb, po.ORDER_AVX2)
        dev.set_router_order(po.ORDER_AVX2)
        got = layer.run_gpu(xb)
        assert routing_check(got["routing"], want["routing"], want["probs"])[1] == 0
        assert normwise_err(got["moe"], want["moe"]) <= MOE_RTOL
    finally:
        layer.close()


def test_prefill_min_tokens_option_checked(dev):
    with pytest.raises(Exception):
        dev.set_option("prefill_min_tokens", 0)


@pytest.fixture
def tile_rows(dev):
    """Forces the grouped GEMMs' tile height; restores the choice by batch afterwards."""
    def set_rows(n):
        dev.set_option("prefill_tile_rows", n)
    yield set_rows
    dev.set_option("prefill_tile_rows", 0)


@pytest.mark.parametrize("rows", [32, 64, 128])
@pytest.mark.parametrize("shape", GROUPED_SHAPES[:5],
                         ids=[f"D{s[0]}E{s[1]}K{s[2]}H{s[3]}n{s[4]}T{s[5]}" for s in GROUPED_SHAPES[:5]])
def test_grouped_every_tile_height(dev, grouped_from, tile_rows, shape, rows):
    """Each tile height (32, 64 or 128 list rows; 128-row tiles reduce in 32-wide steps through a
    four-stage ring) on the grouped shapes: lists from 0 rows to a few hundred, row tiles cut short
    at the end of each list, every expert's rows in one tile or several."""
    D, E, K, H, nt, T = shape
    grouped_from(1)
    tile_rows(rows)
    layer = SynthLayer(dev, D, E, K, H, po.DT_BF16, nt, seed=6, w_scale=1.0, fan_in=True)
    try:
        xb = layer.make_x(T, seed=31)
        x = layer.make_x(T, seed=32, bf16=False)
        check_grouped(dev, layer, xb, x=x, label=f"tile rows {rows} D{D}E{E}K{K}H{H}")
    finally:
        layer.close()


@pytest.mark.parametrize("n_tok", [128, 129, 300])
def test_grouped_tall_tiles_at_list_boundaries(dev, grouped_from, tile_rows, n_tok):
    """128-row tiles with every token on the same 8 experts: lists of exactly one tile (128), one tile
    and one row (129), and two full tiles plus a partial one (300); the other 56 experts are empty.
    Deterministic from call to call."""
    grouped_from(1)
    tile_rows(128)
    bias = np.zeros(64, np.float32)
    bias[20:28] = 30.0
    layer = SynthLayer(dev, 2048, 64, 8, 1024, po.DT_BF16, 1, seed=5, bias=bias)
    try:
        xb = layer.make_x(n_tok, seed=13)
        got, _ = check_grouped(dev, layer, xb, label=f"tall tiles {n_tok} rows")
        assert dev.expert_counts(64)[20:28].tolist() == [n_tok] * 8
        again = layer.run_gpu(xb)
        assert again["moe"].tobytes() == got["moe"].tobytes()
    finally:
        layer.close()


def test_prefill_tile_rows_option_checked(dev):
    for bad in (-1, 16, 96, 256):
        with pytest.raises(Exception):
            dev.set_option("prefill_tile_rows", bad)


@pytest.mark.parametrize("rows,wide,shape", [(64, 1, "olmoe"), (128, 1, "olmoe"), (128, 0, "olmoe"),
                                             (0, 1, "d768-h512")],
                         ids=["64-row", "128-row-wide", "128-row-256wide", "d768-h512-default"])
@pytest.mark.parametrize("biased", [False, True], ids=["uniform", "skewed"])
def test_tiled_expert_copy_is_bitwise_the_blobs(dev, grouped_from, tile_rows, biased, rows, wide, shape):
    """512 tokens on 64- and 128-row tiles, reading the experts from the row-major blobs and from the
    tiled copy (rbt_hip_prefill_layout): identical outputs, both held to the oracle; a dropped copy is
    no longer read. The OLMoE layer runs the 64-row LDS-ring tiles, the 512-row-wide register tiles
    and (option prefill_wide 0) the 256-row-wide ones (gemm_wr_tile); a layer with dim 768 and
    expert_hidden 512 has no wide tiles, so its default plan runs gemm_wr_tile over the copy."""
    grouped_from(1)
    tile_rows(rows)
    dev.set_option("prefill_wide", wide)
    D, H = (2048, 1024) if shape == "olmoe" else (768, 512)
    bias = np.zeros(64, np.float32)
    if biased:
        bias[:8] = 2.0
    layer = SynthLayer(dev, D, 64, 8, H, po.DT_BF16, 1, seed=1, bias=bias)
    try:
        xb = layer.make_x(512, seed=5)
        L = layer.desc()
        dev.prefill_layout_drop(L)
        plain, want = check_grouped(dev, layer, xb, label="blobs")
        dev.prefill_layout(L)
        tiled, _ = check_grouped(dev, layer, xb, label="tiled copy")
        assert tiled["moe"].tobytes() == plain["moe"].tobytes()
        assert np.array_equal(tiled["routing"], plain["routing"])
        dev.prefill_layout_drop(L)
        again = layer.run_gpu(xb)
        assert again["moe"].tobytes() == plain["moe"].tobytes()
    finally:
        dev.set_option("prefill_wide", 1)
        dev.prefill_layout_drop()
        layer.close()


@pytest.mark.parametrize("biased,T", [(False, 512), (True, 512), (False, 1024)],
                         ids=["uniform", "skewed", "uniform-1024"])
def test_wide_tiles_agree_with_256_row_tiles(dev, grouped_from, biased, T):
    """The OLMoE layer on 128-row tiles 512 weight rows wide (the default where the shape has them) and
    256 wide (option prefill_wide = 0): both held to the oracle, and within rounding of each other (the
    same products, summed in k-chunks rotated per tile). 512 tokens: one row tile per expert (uniform,
    expert-major slots) or three for the hot experts (skewed, column-major); 1024 evenly routed tokens:
    ~128 rows per expert, so experts span two row tiles in expert-major order."""
    grouped_from(1)
    bias = np.zeros(64, np.float32)
    if biased:
        bias[:8] = 2.0
    layer = SynthLayer(dev, 2048, 64, 8, 1024, po.DT_BF16, 1, seed=4, bias=bias)
    try:
        xb = layer.make_x(T, seed=6)
        x = layer.make_x(T, seed=16, bf16=False)
        dev.set_option("prefill_wide", 0)
        narrow, _ = check_grouped(dev, layer, xb, x=x, label="256 weight rows")
        dev.set_option("prefill_wide", 1)
        wide, _ = check_grouped(dev, layer, xb, x=x, label="512 weight rows")
        assert np.array_equal(wide["routing"], narrow["routing"])
        assert normwise_err(wide["moe"], narrow["moe"]) <= 1e-5
        if T == 1024:
            assert int((dev.expert_counts(64) > 128).sum()) > 0  # some lists span two row tiles
    finally:
        dev.set_option("prefill_wide", 1)
        layer.close()


def test_tiled_copy_follows_changed_blobs(dev, grouped_from, tile_rows):
    """Writes made through the library into a layer's blobs carry into its tiled copy by themselves:
    two experts rewritten by rbt_hip_fill_normal, then one expert's w1 overwritten by rbt_hip_h2d with
    another expert's bytes; after each, the grouped output matches the oracle on the new weights, and
    re-taking the copy changes nothing."""
    grouped_from(1)
    tile_rows(128)
    layer = SynthLayer(dev, 2048, 64, 8, 1024, po.DT_BF16, 1, seed=3)
    try:
        xb = layer.make_x(512, seed=7)
        L = layer.desc()
        dev.prefill_layout(L)
        layer.reseed_experts([5, 40], seed=99)
        followed, _ = check_grouped(dev, layer, xb, label="copy after fill_normal")
        mat = layer.H * layer.D * layer.esz
        src = layer.experts[11 * layer.stride: 11 * layer.stride + mat].copy()
        dev.h2d(layer.experts_dev, src, offset=3 * layer.stride)
        layer.experts = dev.d2h(layer.experts_dev, (layer.E * layer.stride,), np.uint8)
        followed, _ = check_grouped(dev, layer, xb, label="copy after h2d")
        dev.prefill_layout(L)
        retaken = layer.run_gpu(xb)
        assert retaken["moe"].tobytes() == followed["moe"].tobytes()
    finally:
        dev.prefill_layout_drop()
        layer.close()


def test_model_image_writes_reach_prefill_and_decode(dev, grouped_from, tile_rows):
    """A created model image with tiled copies of every layer (rbt_hip_prefill_layout(NULL)): an expert
    overwritten through rbt_hip_tensor + rbt_hip_h2d changes the host-pointer MoE block (rbt_hip_moe) at
    T = 1 (decode kernels, which read the blobs) and at T = 256 (grouped GEMMs over the copy) alike:
    both match the oracle on the image as it is after the write."""
    from rabbitm2_amd import hip as rh
    grouped_from(12)
    tile_rows(0)
    cfg = rh.Config(vocab=64, dim=512, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=128, n_experts=8, top_k=2,
                    expert_hidden=256, max_seq=64, dtype=po.DT_BF16, qk_norm=1, norm_topk=0, rope_theta=1e4,
                    rms_eps=1e-5)
    base = dev.model_create(cfg)
    img = rh.DevBuf(dev, base.value, dev.tensor("lm_head")[0] + dev.tensor("lm_head")[1])
    dev.fill_normal(img, po.DT_BF16, img.nbytes // 2, 21, 1, scale=0.02)
    dev.prefill_layout()
    stride = (3 * cfg.expert_hidden * cfg.dim * 2 + 4095) // 4096 * 4096
    r_off, r_bytes = dev.tensor("router", 1)
    e_off, e_bytes = dev.tensor("experts", 1)
    rng = np.random.default_rng(2)
    xb = rng.standard_normal((256, cfg.dim)).astype(np.float32)

    def check(label):
        router = dev.d2h(img, (cfg.n_experts, cfg.dim), np.uint16, offset=r_off)
        experts = dev.d2h(img, (e_bytes,), np.uint8, offset=e_off)
        want = po.moe_layer(cfg.dim, cfg.n_experts, cfg.top_k, cfg.expert_hidden, po.DT_BF16, 0, router, experts,
                            stride, xb, order=po.ORDER_AVX2)
        for T in (1, 256):
            x, routing = dev.moe(1, xb[:T], x=np.zeros((T, cfg.dim), np.float32))
            assert np.array_equal(routing, want["routing"][:T]), (label, T)
            err = normwise_err(x, want["moe"][:T])
            print(f"{label} T={T}: moe err {err:.2e}", flush=True)
            assert err <= MOE_RTOL
        return want

    dev.set_router_order(po.ORDER_AVX2)
    before = check("before the write")
    used = np.bincount(before["routing"].ravel(), minlength=cfg.n_experts)
    e = int(np.argmax(used))  # the most used expert gets another expert's weights
    donor = (e + 1) % cfg.n_experts
    blob = dev.d2h(img, (stride,), np.uint8, offset=e_off + donor * stride)
    dev.h2d(img, blob, offset=e_off + e * stride)
    after = check("after the write")
    assert not np.array_equal(after["moe"], before["moe"])


def test_prefill_layout_rejects_shapes_without_one(dev):
    layer = SynthLayer(dev, 768, 64, 8, 384, po.DT_BF16, 0, seed=6)
    try:
        with pytest.raises(Exception, match="no tiled layout"):
            dev.prefill_layout(layer.desc())
    finally:
        layer.close()
