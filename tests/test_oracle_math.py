"""Pins of the oracle that do not need the reference engine: known answers, closed forms,
invariants and float64 brute force (each chosen so that a dropped term, a wrong index or a
transposed operand fails)."""
import math

import numpy as np
import pytest

from oracle import pyoracle as po


# ---------------------------------------------------------------- bf16 (rabbit2/ref/rbt2.py:106-113)

def test_bf16_known_answers():
    cases = [
        (1.0, 0x3F80),
        (-2.0, 0xC000),
        (0.0, 0x0000),
        (-0.0, 0x8000),
        (float("inf"), 0x7F80),
        (float("nan"), 0x7FC0),
        (np.float32(3.4028235e38), 0x7F80),  # largest finite rounds up to inf under RNE
    ]
    for v, want in cases:
        assert po.lib().orc_f32_to_bf16(float(v)) == want, v
    # exact halfway cases round to the even neighbour
    as_f = lambda u: np.array([u], np.uint32).view(np.float32)[0]
    assert po.lib().orc_f32_to_bf16(float(as_f(0x3F808000))) == 0x3F80
    assert po.lib().orc_f32_to_bf16(float(as_f(0x3F818000))) == 0x3F82
    assert po.lib().orc_f32_to_bf16(float(as_f(0x3F808001))) == 0x3F81
    # widening is exact and inverts encoding on representable values
    u = np.arange(0, 0x10000, 7, dtype=np.uint16)
    u = u[((u & 0x7F80) != 0x7F80)]  # finite
    f = po.bf16_to_f32(u)
    assert np.array_equal(po.f32_to_bf16(f), u)
    assert po.lib().orc_bf16_to_f32(0x3F80) == 1.0


# ---------------------------------------------------------------- layout (rabbit2.c:158-193)

def test_layout_closed_form_olmoe():
    cfg = po.Config(vocab=50304, dim=2048, n_layers=16, n_heads=16, n_kv_heads=16, head_dim=128, n_experts=64, top_k=8,
                    expert_hidden=1024, max_seq=4096, dtype=1, qk_norm=1, norm_topk=0)
    L = po.layout(cfg)
    assert L["tok_emb"] == 4096
    assert L["expert_stride"] == 12_582_912  # 3 * 1024 * 2048 * 2, already 4 KiB aligned
    assert L["layers"][0]["experts"] == 239_898_624
    assert L["layers"][-1]["experts"] == 12_827_234_304
    assert L["lm_head"] == 13_632_548_864
    assert L["end"] == 13_838_594_048
    # each layer advances by the same amount; experts are 4 KiB aligned, vectors 64 B aligned
    steps = np.diff([ly["experts"] for ly in L["layers"]])
    assert len(set(steps.tolist())) == 1
    for ly in L["layers"]:
        assert ly["experts"] % 4096 == 0
        assert all(ly[k] % 64 == 0 for k in ("attn_norm", "wq", "wk", "wv", "wo", "q_norm", "k_norm", "ffn_norm",
                                             "router"))


def test_layout_closed_form_tiny_f32():
    cfg = po.Config(vocab=1024, dim=256, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=64, n_experts=8, top_k=2,
                    expert_hidden=128, max_seq=64, dtype=0, qk_norm=1, norm_topk=0)
    L = po.layout(cfg)
    assert L["expert_stride"] == 393_216
    assert L["end"] == 10_515_456


# ---------------------------------------------------------------- generator

def test_splitmix64_published_outputs():
    # Outputs of Vigna's splitmix64.c for seed 1234567 (published test vector).
    assert po.splitmix64(1234567, 5) == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                                         4593380528125082431, 16408922859458223821]


def test_normal_samples_have_standard_normal_moments():
    z = po.fill_normal(1 << 20, po.DT_F32, 7, 3).astype(np.float64)
    assert abs(z.mean()) < 5e-3
    assert abs(z.var() - 1.0) < 5e-3
    assert abs((z ** 4).mean() - 3.0) < 0.04
    assert abs(np.mean(np.abs(z) < 1.0) - 0.6826894921) < 3e-3
    # counter-based: any sub-range regenerates identically
    assert np.array_equal(po.fill_normal(100, po.DT_F32, 7, 3, first=1000), z[1000:1100].astype(np.float32))
    # Box-Muller pair structure: element 2p and 2p+1 share the radius
    r2 = z[0::2] ** 2 + z[1::2] ** 2
    u1 = np.exp(-r2 / 2)
    assert np.all((u1 > 0) & (u1 <= 1))


def test_normal_scale_offset_and_bf16_rounding():
    a = po.fill_normal(1000, po.DT_F32, 1, 9, scale=0.02, offset=1.0)
    z = np.array([po.normal(1, 9, i) for i in range(1000)])
    assert np.array_equal(a, (1.0 + np.float64(np.float32(0.02)) * z).astype(np.float32))  # scale is an f32 argument
    b = po.fill_normal(1000, po.DT_BF16, 1, 9, scale=0.02, offset=1.0)
    assert np.array_equal(b, po.f32_to_bf16(a))


# ---------------------------------------------------------------- matvec (rabbit2.c:323-390)

@pytest.mark.parametrize("cols", [1, 3, 4, 7, 8, 15, 16, 17, 25, 36, 64, 129, 2048])
@pytest.mark.parametrize("dtype", [po.DT_F32, po.DT_BF16])
def test_matvec_float64_brute_force(cols, dtype):
    rng = np.random.default_rng(cols)
    rows = 9
    Wf = rng.standard_normal((rows, cols)).astype(np.float32)
    W = po.f32_to_bf16(Wf) if dtype == po.DT_BF16 else Wf
    Wv = po.bf16_to_f32(W) if dtype == po.DT_BF16 else Wf
    x = rng.standard_normal(cols).astype(np.float32)
    exact = Wv.astype(np.float64) @ x.astype(np.float64)
    bound = cols * 2 * np.finfo(np.float32).eps * (np.abs(Wv).astype(np.float64) @ np.abs(x).astype(np.float64))
    outs = {o: po.matvec(W, dtype, x, o) for o in (po.ORDER_SCALAR, po.ORDER_AVX2, po.ORDER_LANE16)}
    for o, out in outs.items():
        assert np.all(np.abs(out - exact) <= bound + 1e-30), o
    assert outs[po.ORDER_AVX2].tobytes() == outs[po.ORDER_LANE16].tobytes()


def test_matvec_orders_are_the_documented_sums():
    """Small cases where the two orders are written out by hand."""
    W = np.array([[1e8, 1.0, -1e8, 1.0, 1.0]], np.float32)
    x = np.ones(5, np.float32)
    # scalar: s0 = 1e8 + 1 (tail) = 1e8, s1 = 1, s2 = -1e8, s3 = 1 -> (1e8+1)+(-1e8+1) = 0
    assert po.matvec(W, po.DT_F32, x, po.ORDER_SCALAR)[0] == np.float32((np.float32(1e8) + 1) + (np.float32(-1e8) + 1))
    # avx2 with 5 columns: everything is tail, summed in order from 0: ((((0+1e8)+1)-1e8)+1)+1 = 2
    assert po.matvec(W, po.DT_F32, x, po.ORDER_AVX2)[0] == 2.0


# ---------------------------------------------------------------- softmax / top-k (rabbit2.c:399-405, 516-528)

def test_softmax_invariants():
    rng = np.random.default_rng(0)
    for n in (1, 2, 8, 64, 1000):
        v = (3 * rng.standard_normal(n)).astype(np.float32)
        p = po.softmax(v)
        assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-5
        assert np.array_equal(np.argsort(-v, kind="stable"), np.argsort(-p, kind="stable")) or n == 1
        ref = np.exp(v.astype(np.float64) - v.max())
        assert np.allclose(p, ref / ref.sum(), rtol=1e-5, atol=0)
    assert np.all(po.softmax(np.zeros(64, np.float32)) == np.float32(1.0 / 64))


def test_topk_is_a_stable_descending_sort():
    rng = np.random.default_rng(1)
    for trial in range(200):
        n = int(rng.integers(1, 70))
        k = int(rng.integers(1, min(n, 64) + 1))
        p = rng.choice(np.array([0.1, 0.2, 0.3, 0.05], np.float32), n) if trial % 2 else rng.random(n).astype(
            np.float32)
        idx, wt, ws = po.topk(p, k)
        want = np.argsort(-p, kind="stable")[:k]
        assert np.array_equal(idx, want)
        assert np.array_equal(wt, p[want])
    p = rng.random(16).astype(np.float32)
    idx, _, _ = po.topk(p, 16)
    assert np.array_equal(idx, np.argsort(-p, kind="stable"))


# ---------------------------------------------------------------- MoE layer (rabbit2.c:513-542)

def _f64_moe(router, experts, stride, D, E, K, H, dtype, norm_topk, xb, bias=None):
    """Textbook MoE in float64: softmax router, top-k, SwiGLU down(silu(gate x) * up x)."""
    esz = po.ELEM[dtype]
    dec = (lambda a: po.bf16_to_f32(a.view(np.uint16))) if dtype == po.DT_BF16 else (lambda a: a.view(np.float32))
    R = dec(router.reshape(-1).view(np.uint8)).reshape(E, D).astype(np.float64)
    out = np.zeros((xb.shape[0], D))
    routes = []
    for t, x in enumerate(xb.astype(np.float64)):
        logits = R @ x + (0 if bias is None else bias)
        p = np.exp(logits - logits.max())
        p /= p.sum()
        top = np.argsort(-p, kind="stable")[:K]
        routes.append(top)
        w = p[top] / p[top].sum() if norm_topk else p[top]
        for e, wk in zip(top, w):
            blob = experts[e * stride: e * stride + 3 * H * D * esz]
            W1 = dec(blob[: H * D * esz]).reshape(H, D).astype(np.float64)
            W3 = dec(blob[H * D * esz: 2 * H * D * esz]).reshape(H, D).astype(np.float64)
            W2 = dec(blob[2 * H * D * esz:]).reshape(D, H).astype(np.float64)
            g, u = W1 @ x, W3 @ x
            out[t] += wk * (W2 @ (g / (1 + np.exp(-g)) * u))
    return out, np.array(routes)


def _random_layer(D, E, H, dtype, seed, same_experts=False):
    rng = np.random.default_rng(seed)
    esz = po.ELEM[dtype]
    stride = (3 * H * D * esz + 4095) // 4096 * 4096
    enc = (lambda a: po.f32_to_bf16(a).view(np.uint8)) if dtype == po.DT_BF16 else (lambda a: a.view(np.uint8))
    router = enc((rng.standard_normal((E, D)) / math.sqrt(D)).astype(np.float32)).reshape(-1)
    experts = np.zeros(E * stride, np.uint8)
    blob = None
    for e in range(E):
        if blob is None or not same_experts:
            w1 = (rng.standard_normal((H, D)) / math.sqrt(D)).astype(np.float32)
            w3 = (rng.standard_normal((H, D)) / math.sqrt(D)).astype(np.float32)
            w2 = (rng.standard_normal((D, H)) / math.sqrt(H)).astype(np.float32)
            blob = np.concatenate([enc(w1).ravel(), enc(w3).ravel(), enc(w2).ravel()])
        experts[e * stride: e * stride + blob.size] = blob
    return router, experts, stride


@pytest.mark.parametrize("shape", [(64, 8, 2, 128, 0, 1), (36, 5, 2, 25, 0, 1), (48, 6, 3, 40, 1, 0), (8, 4, 4, 7, 1, 1),
                                   (256, 8, 2, 128, 0, 0)])
def test_moe_layer_float64_brute_force(shape):
    D, E, K, H, dt, nt = shape
    router, experts, stride = _random_layer(D, E, H, dt, seed=D + E)
    xb = np.random.default_rng(3).standard_normal((6, D)).astype(np.float32)
    want, routes = _f64_moe(router, experts, stride, D, E, K, H, dt, nt, xb)
    for order in (po.ORDER_SCALAR, po.ORDER_AVX2):
        got = po.moe_layer(D, E, K, H, dt, nt, router, experts, stride, xb, order=order)
        assert np.array_equal(got["routing"], routes)
        assert np.max(np.abs(got["moe"] - want)) <= 1e-5 * max(1.0, np.max(np.abs(want)))


def test_moe_layer_linearity_identical_experts():
    D, E, K, H = 32, 6, 3, 16
    router, experts, stride = _random_layer(D, E, H, po.DT_F32, seed=5, same_experts=True)
    xb = np.random.default_rng(4).standard_normal((3, D)).astype(np.float32)
    single = po.moe_layer(D, E, 1, H, 0, 1, router, experts, stride, xb)  # one expert, weight 1
    ren = po.moe_layer(D, E, K, H, 0, 1, router, experts, stride, xb)  # weights sum to 1
    raw = po.moe_layer(D, E, K, H, 0, 0, router, experts, stride, xb)  # weights sum to sum(p_top)
    assert np.allclose(ren["moe"], single["moe"], rtol=1e-5, atol=1e-6)
    wsum = raw["weights"].sum(axis=1, keepdims=True)
    assert np.allclose(raw["moe"], wsum * single["moe"], rtol=1e-5, atol=1e-6)


def test_moe_layer_zero_experts_and_residual():
    D, E, K, H = 16, 4, 2, 8
    router, _, stride = _random_layer(D, E, H, po.DT_F32, seed=6)
    experts = np.zeros(E * stride, np.uint8)
    xb = np.ones((2, D), np.float32)
    x = np.full((2, D), 3.0, np.float32)
    got = po.moe_layer(D, E, K, H, 0, 1, router, experts, stride, xb, x=x)
    assert np.all(got["moe"] == 0) and np.all(got["x"] == 3.0)


def test_moe_layer_bias_steers_routing():
    D, E, K, H = 32, 8, 2, 16
    router, experts, stride = _random_layer(D, E, H, po.DT_BF16, seed=7)
    xb = np.random.default_rng(8).standard_normal((5, D)).astype(np.float32)
    bias = np.zeros(E, np.float32)
    bias[[6, 2]] = [50.0, 40.0]
    got = po.moe_layer(D, E, K, H, 1, 1, router, experts, stride, xb, bias=bias)
    assert np.all(got["routing"] == [6, 2])


def _f64_routing(router_f64, xb, K, bias, after_softmax=False):
    """Routing and un-renormalised weights in float64: softmax over the router logits, with `bias`
    added to the logits before the softmax (after_softmax False) or to the probabilities after it."""
    routes, weights = [], []
    for x in xb.astype(np.float64):
        logits = router_f64 @ x
        if not after_softmax:
            logits = logits + bias
        p = np.exp(logits - logits.max())
        p /= p.sum()
        key = p + bias if after_softmax else p
        top = np.argsort(-key, kind="stable")[:K]
        routes.append(top)
        weights.append(p[top])
    return np.array(routes), np.array(weights)


def test_moe_layer_skew_bias_goes_before_the_softmax():
    """The skewed prefill workload's router bias (+2.0 on the logits of experts 0-7, 64 experts, top-8,
    un-renormalised weights) against the float64 brute force. The router is scaled so that logits
    spread over several units: some tokens then route past experts 0-7 despite the bias, which a bias
    added to the probabilities after the softmax (always < 1 < 2.0) could never do."""
    D, E, K, H = 64, 64, 8, 16
    rng = np.random.default_rng(11)
    router_f32 = (rng.standard_normal((E, D)) * (3.0 / math.sqrt(D))).astype(np.float32)
    router = po.f32_to_bf16(router_f32).view(np.uint8).reshape(-1)
    _, experts, stride = _random_layer(D, E, H, po.DT_BF16, seed=12)
    xb = rng.standard_normal((64, D)).astype(np.float32)
    bias = np.zeros(E, np.float32)
    bias[:8] = 2.0
    R = po.bf16_to_f32(router.view(np.uint16)).reshape(E, D).astype(np.float64)
    want_routes, want_w = _f64_routing(R, xb, K, bias.astype(np.float64))
    mutant_routes, _ = _f64_routing(R, xb, K, bias.astype(np.float64), after_softmax=True)
    unbiased_routes, _ = _f64_routing(R, xb, K, np.zeros(E))
    hot = set(range(8))
    # the workload is skewed (the bias moves routing) yet not degenerate (some tokens leave 0-7)
    assert any(set(r) != hot for r in want_routes)
    assert not np.array_equal(want_routes, unbiased_routes)
    # the mutant routes every token to exactly 0-7, so it disagrees with the brute force
    assert all(set(r) == hot for r in mutant_routes)
    assert not np.array_equal(np.sort(mutant_routes, axis=1), np.sort(want_routes, axis=1))
    for order in (po.ORDER_SCALAR, po.ORDER_AVX2):
        got = po.moe_layer(D, E, K, H, po.DT_BF16, 0, router, experts, stride, xb, order=order, bias=bias)
        assert np.array_equal(got["routing"], want_routes)
        assert np.allclose(got["weights"], want_w, rtol=1e-5, atol=1e-7)
        f64, f64_routes = _f64_moe(router, experts, stride, D, E, K, H, po.DT_BF16, 0, xb, bias=bias)
        assert np.array_equal(f64_routes, want_routes)
        assert np.max(np.abs(got["moe"] - f64)) <= 1e-5 * max(1.0, np.max(np.abs(f64)))
