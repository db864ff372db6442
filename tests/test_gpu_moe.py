"""Parity of the HIP MoE layer (rbt_hip_moe_dev through the C ABI) with the oracle.

Shapes follow the reference's engine tests (rabbit2/tests/test_forward.py:80-98 and
rabbit2/tests/test_avx2.py:52: odd dims, tails below 16 columns, top-1, top-k of few experts,
f32 and bf16) plus the OLMoE layer (D 2048, E 64, top-8, H 1024, bf16) at decode and prefill sizes.
Bar: routing identical except at exact CPU ties; normwise max error <= 1e-3 (tests/common.py).
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.common import MOE_RTOL, SynthLayer, normwise_err, routing_check

pytestmark = pytest.mark.gpu

ORDERS = [po.ORDER_AVX2, po.ORDER_SCALAR]


def check(layer, xb, order, dev, x=None, label=""):
    dev.set_router_order(order)
    want = layer.oracle(xb, order, x=x)
    got = layer.run_gpu(xb, x=x)
    bad, unexplained = routing_check(got["routing"], want["routing"], want["probs"])
    err = normwise_err(got["moe"], want["moe"])
    werr = normwise_err(got["weights"], want["weights"])
    print(f"{label} T={xb.shape[0]} order={order}: routing mismatched tokens {bad} (unexplained {unexplained}), "
          f"moe err {err:.2e}, weight err {werr:.2e}", flush=True)
    assert unexplained == 0
    assert err <= MOE_RTOL
    if bad == 0:
        assert werr <= 1e-6
    if x is not None:
        assert normwise_err(got["x"], want["x"]) <= MOE_RTOL
    return got, want


SMALL_SHAPES = [
    # (dim, E, K, H, dtype, norm_topk)
    (64, 8, 2, 128, po.DT_F32, 1),     # reference Config() defaults
    (64, 8, 2, 128, po.DT_BF16, 1),
    (48, 6, 3, 40, po.DT_BF16, 0),     # OLMoE-like top-3 of 6
    (36, 5, 2, 25, po.DT_F32, 1),      # odd dims
    (32, 4, 1, 64, po.DT_F32, 1),      # top-1
    (8, 4, 2, 7, po.DT_BF16, 0),       # dim < 16: whole row is the AVX2 tail
    (36, 4, 2, 25, po.DT_BF16, 0),
    (256, 8, 2, 128, po.DT_F32, 0),    # the tiny OLMoE-style model's MoE layer
    (100, 7, 7, 33, po.DT_BF16, 1),    # K == E
]


@pytest.mark.parametrize("shape", SMALL_SHAPES, ids=[f"D{s[0]}E{s[1]}K{s[2]}H{s[3]}dt{s[4]}n{s[5]}" for s in SMALL_SHAPES])
@pytest.mark.parametrize("order", ORDERS)
def test_small_shapes(dev, shape, order):
    D, E, K, H, dt, nt = shape
    layer = SynthLayer(dev, D, E, K, H, dt, nt, seed=3, w_scale=1.0, fan_in=True)
    try:
        for T in (1, 5):
            xb = layer.make_x(T, seed=11 + T, bf16=False)
            x = layer.make_x(T, seed=99, bf16=False)
            check(layer, xb, order, dev, x=x, label=f"D{D}E{E}K{K}H{H}")
    finally:
        layer.close()


# Shapes whose rows are whole 1 KiB wave-steps take the specialised decode kernels
# (experts_decode.hip): D, H multiples of 512 (bf16) or 256 (f32).
FAST_SHAPES = [
    (512, 8, 2, 512, po.DT_BF16, 1),    # one step per row
    (1024, 16, 4, 1536, po.DT_BF16, 0),  # 2 steps gate/up, 3 steps down
    (256, 8, 2, 256, po.DT_F32, 1),
    (768, 8, 8, 1024, po.DT_F32, 1),     # f32, 4 steps down: slots loaded 4 at a time
    (2048, 32, 12, 1024, po.DT_BF16, 1),  # K = 12: a full and a partial chunk of 8 slots
    (4096, 8, 2, 512, po.DT_BF16, 0),    # 8 steps gate/up
]


@pytest.mark.parametrize("shape", FAST_SHAPES, ids=[f"D{s[0]}E{s[1]}K{s[2]}H{s[3]}dt{s[4]}n{s[5]}" for s in FAST_SHAPES])
def test_fast_path_shapes(dev, shape):
    D, E, K, H, dt, nt = shape
    layer = SynthLayer(dev, D, E, K, H, dt, nt, seed=4, w_scale=1.0, fan_in=True)
    try:
        for T in (1, 3):
            xb = layer.make_x(T, seed=21 + T)
            x = layer.make_x(T, seed=77, bf16=False)
            check(layer, xb, po.ORDER_AVX2, dev, x=x, label=f"fast D{D}E{E}K{K}H{H}")
    finally:
        layer.close()


def test_empty_batch(dev):
    layer = SynthLayer(dev, 64, 8, 2, 128, po.DT_BF16, 1, seed=1)
    try:
        got = layer.run_gpu(np.zeros((0, 64), np.float32))
        assert got["moe"].shape == (0, 64)
    finally:
        layer.close()


@pytest.fixture(scope="module")
def olmoe_layer(dev):
    """The OLMoE-1B-7B layer shape, bf16 weights ~N(0, 0.02), seed 1, renormalised top-8."""
    layer = SynthLayer(dev, 2048, 64, 8, 1024, po.DT_BF16, 1, seed=1)
    yield layer
    layer.close()


@pytest.mark.parametrize("order", ORDERS)
def test_olmoe_decode(dev, olmoe_layer, order):
    for s in range(4):
        xb = olmoe_layer.make_x(1, seed=s)
        check(olmoe_layer, xb, order, dev, label=f"olmoe decode seed {s}")


def test_olmoe_decode_fused_and_four_launch_paths(dev, olmoe_layer):
    """Batch-1 decode runs the top-k inside the gate/up kernel by default (three launches); the
    four-launch form has a separate top-k kernel. Both meet the bar, on the same routing."""
    dev.set_router_order(po.ORDER_AVX2)
    try:
        for s in range(3):
            xb = olmoe_layer.make_x(1, seed=40 + s)
            x = olmoe_layer.make_x(1, seed=60 + s, bf16=False)
            dev.set_option("fused_decode", 1)
            got_f, want = check(olmoe_layer, xb, po.ORDER_AVX2, dev, x=x, label=f"fused seed {s}")
            dev.set_option("fused_decode", 0)
            got_u, _ = check(olmoe_layer, xb, po.ORDER_AVX2, dev, x=x, label=f"four-launch seed {s}")
            assert np.array_equal(got_f["routing"], got_u["routing"])
            assert np.array_equal(got_f["weights"], got_u["weights"])
    finally:
        dev.set_option("fused_decode", 1)


def test_profile_deferred_mode(dev, olmoe_layer):
    """Profiling mode 2 times every launch without waiting between calls: profile_get reports each
    kernel of every call since the mode was set, and the outputs are unchanged."""
    dev.set_router_order(po.ORDER_AVX2)
    L = olmoe_layer.desc()
    dev.reserve(L, 1)
    xb = dev.upload_array(olmoe_layer.make_x(1, seed=9))
    moe = dev.malloc(2048 * 4)
    try:
        dev.moe_dev(L, xb, 1, moe=moe)
        dev.synchronize()
        want = dev.d2h(moe, (2048,), np.float32)
        dev.profile(2)
        for _ in range(5):
            dev.moe_dev(L, xb, 1, moe=moe)
        for name in ("router", "gateup", "down_combine"):
            tot, n = dev.profile_get(name)
            assert n == 5 and 0 < 1000.0 * tot / n < 1000.0, (name, tot, n)
        assert dev.d2h(moe, (2048,), np.float32).tobytes() == want.tobytes()
        dev.profile(2)  # setting the mode again clears the counts
        assert dev.profile_get("gateup")[1] == 0
    finally:
        dev.profile(0)
        dev.free(xb)
        dev.free(moe)


def test_profile_deferred_mode_reuses_its_events(dev, olmoe_layer):
    """Mode 2 reads its event pairs and reuses them: past 4096 launches of one kernel every launch is
    still counted (the pool is read when it fills), and reading the counts between calls adds up."""
    dev.set_router_order(po.ORDER_AVX2)
    L = olmoe_layer.desc()
    dev.reserve(L, 1)
    xb = dev.upload_array(olmoe_layer.make_x(1, seed=9))
    moe = dev.malloc(2048 * 4)
    try:
        dev.profile(2)
        for _ in range(4100):
            dev.moe_dev(L, xb, 1, moe=moe)
        assert dev.profile_get("gateup")[1] == 4100
        for _ in range(3):
            dev.moe_dev(L, xb, 1, moe=moe)
        tot, n = dev.profile_get("router")
        assert n == 4103 and 0 < 1000.0 * tot / n < 1000.0
    finally:
        dev.profile(0)
        dev.free(xb)
        dev.free(moe)


def test_olmoe_decode_deterministic(dev, olmoe_layer):
    dev.set_router_order(po.ORDER_AVX2)
    xb = olmoe_layer.make_x(1, seed=7)
    a = olmoe_layer.run_gpu(xb)
    b = olmoe_layer.run_gpu(xb)
    assert a["moe"].tobytes() == b["moe"].tobytes()
    assert np.array_equal(a["routing"], b["routing"])


@pytest.mark.parametrize("biased", [False, True], ids=["uniform", "skewed"])
def test_olmoe_prefill(dev, biased):
    """512 tokens; skewed: +2.0 on the router logits of experts 0-7 (CPU and GPU alike)."""
    bias = np.zeros(64, np.float32)
    if biased:
        bias[:8] = 2.0
    layer = SynthLayer(dev, 2048, 64, 8, 1024, po.DT_BF16, 1, seed=1, bias=bias)
    try:
        xb = layer.make_x(512, seed=5)
        got, want = check(layer, xb, po.ORDER_AVX2, dev, label="olmoe prefill " + ("skewed" if biased else "uniform"))
        hist = np.bincount(want["routing"].ravel(), minlength=64)
        print("tokens per expert:", hist.tolist(), flush=True)
        assert hist.sum() == 512 * 8
        # 512 tokens take the grouped path, whose dispatch histogram is exposed through the C ABI
        counts = dev.expert_counts(64)
        assert counts is not None
        assert np.array_equal(counts, np.bincount(got["routing"].ravel(), minlength=64))
        if biased:
            assert hist[:8].sum() > hist[8:].sum()
    finally:
        layer.close()


# Batches of 16+ tokens take the batched router kernel (AVX2 order): the router tile is staged once per
# 8 tokens in 512-column chunks. Shapes: f32 with a 4-column tail, bf16 with an 8-column tail after a
# full and a partial chunk, f32 with a last chunk of 16 columns, and E not a multiple of 16.
ROUTER_BATCH_SHAPES = [
    (100, 8, 2, 16, po.DT_F32, 1),
    (536, 8, 3, 16, po.DT_BF16, 0),
    (1040, 6, 2, 16, po.DT_F32, 1),
    (2048, 20, 4, 16, po.DT_BF16, 1),
]


@pytest.mark.parametrize("shape", ROUTER_BATCH_SHAPES,
                         ids=[f"D{s[0]}E{s[1]}K{s[2]}dt{s[4]}" for s in ROUTER_BATCH_SHAPES])
def test_router_batch_shapes(dev, shape):
    D, E, K, H, dt, nt = shape
    bias = np.linspace(-0.5, 0.5, E).astype(np.float32)
    layer = SynthLayer(dev, D, E, K, H, dt, nt, seed=9, w_scale=1.0, fan_in=True, bias=bias)
    try:
        for T in (16, 29):
            xb = layer.make_x(T, seed=50 + T, bf16=False)
            check(layer, xb, po.ORDER_AVX2, dev, label=f"router batch D{D}E{E}")
    finally:
        layer.close()


# The engine's selection (rabbit2.c:516-528) scans with a strict '>' from index 0: among equal
# probabilities the lowest index goes first, and when the softmax sum is NaN (every probability NaN)
# each round keeps the first unused index. Every top-k on the GPU path is held to that exactly, with no
# exemption for ties: the fused decode kernel (top-k inside gate/up), the separate top-k launch, the
# few-token front end (top-k + activation split) and the one-launch grouped front end, in both orders.
TOPK_PATHS = [  # (label, tokens, option fused_decode)
    ("fused-decode", 1, 1), ("topk-launch", 1, 0), ("few-tokens", 5, 1), ("grouped-front", 16, 1),
    ("grouped-one-launch", 100, 1)]


def _selection_layer(dev, nan_row=None):
    """D 512, 64 experts, top-8, H 512, bf16, renormalised. Router rows 7, 40 and 41 copy row 3 and rows
    20 and 21 copy row 10, with biases +20 and +10 on the two groups: every token's eight largest
    probabilities are a 4-way and a 3-way exact tie and one more expert. nan_row: that router row set to
    bf16 NaN (0x7FC0), which makes the softmax sum and every probability NaN."""
    bias = np.zeros(64, np.float32)
    bias[[3, 7, 40, 41]] = 20.0
    bias[[10, 20, 21]] = 10.0
    layer = SynthLayer(dev, 512, 64, 8, 512, po.DT_BF16, 1, seed=21, bias=bias)
    r = layer.router.copy()
    r[[7, 40, 41]] = r[3]
    r[[20, 21]] = r[10]
    if nan_row is not None:
        r[nan_row] = 0x7FC0
    dev.h2d(layer.router_dev, r)
    layer.router = r
    return layer


@pytest.mark.parametrize("order", ORDERS, ids=["avx2", "scalar"])
@pytest.mark.parametrize("path", TOPK_PATHS, ids=[p[0] for p in TOPK_PATHS])
def test_topk_exact_ties_take_the_lowest_index(dev, path, order):
    label, T, fused = path
    layer = _selection_layer(dev)
    dev.set_router_order(order)
    dev.set_option("fused_decode", fused)
    try:
        xb = layer.make_x(T, seed=70 + T)
        want = layer.oracle(xb, order)
        assert (want["routing"][:, :4] == [3, 7, 40, 41]).all() and (want["routing"][:, 4:7] == [10, 20, 21]).all()
        probs = want["probs"].reshape(T, -1)
        assert (probs[:, [7, 40, 41]] == probs[:, [3]]).all() and (probs[:, [20, 21]] == probs[:, [10]]).all()
        got = layer.run_gpu(xb)
        assert np.array_equal(got["routing"], want["routing"]), f"{label}: {got['routing'][0]} vs {want['routing'][0]}"
        assert normwise_err(got["weights"], want["weights"]) <= 1e-6
        assert normwise_err(got["moe"], want["moe"]) <= MOE_RTOL
    finally:
        dev.set_option("fused_decode", 1)
        layer.close()


@pytest.mark.parametrize("order", ORDERS, ids=["avx2", "scalar"])
@pytest.mark.parametrize("path", TOPK_PATHS, ids=[p[0] for p in TOPK_PATHS])
def test_topk_nan_probabilities_keep_the_first_indices(dev, path, order):
    label, T, fused = path
    layer = _selection_layer(dev, nan_row=33)
    dev.set_router_order(order)
    dev.set_option("fused_decode", fused)
    try:
        xb = layer.make_x(T, seed=90 + T)
        want = layer.oracle(xb, order)
        assert (want["routing"] == np.arange(8)).all() and np.isnan(want["weights"]).all()
        got = layer.run_gpu(xb)
        assert np.array_equal(got["routing"], want["routing"]), f"{label}: {got['routing'][0]}"
        assert np.isnan(got["weights"]).all()
        assert np.array_equal(np.isnan(got["moe"]), np.isnan(want["moe"]))
    finally:
        dev.set_option("fused_decode", 1)
        layer.close()
