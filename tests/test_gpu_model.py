"""The model-level entry points of the C ABI on uploaded .rbt2 images: rbt_hip_upload (header
checks of rabbit2/src/rabbit2.c:199-228), rbt_hip_moe (host pointers, the forward() MoE block
:513-542 with x += moe) and rbt_hip_matvec (the matvec seam :357), against the oracle on the same
bytes."""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests.common import MOE_RTOL, normwise_err, routing_check

pytestmark = pytest.mark.gpu

MODELS = {
    "tiny_olmoe_f32": (po.Config(vocab=1024, dim=256, n_layers=2, n_heads=4, n_kv_heads=4, head_dim=64, n_experts=8,
                                 top_k=2, expert_hidden=128, max_seq=64, dtype=po.DT_F32, qk_norm=1, norm_topk=0),
                       po.GenParams(seed=0, w_scale=0.02)),
    "bf16_renorm": (po.Config(dtype=po.DT_BF16), po.ref_style(4)),
    "odd_f32": (po.Config(vocab=70, dim=36, n_layers=2, n_heads=6, n_kv_heads=3, head_dim=6, n_experts=5, top_k=2,
                          expert_hidden=25, max_seq=32), po.ref_style(2)),
}


@pytest.mark.parametrize("name", list(MODELS))
def test_upload_moe_matvec(dev, name):
    cfg, gp = MODELS[name]
    model = po.build_model(cfg, gp)
    lay = po.layout(cfg)
    got_cfg = dev.upload(model)
    assert got_cfg.dim == cfg.dim and got_cfg.n_experts == cfg.n_experts
    dev.set_router_order(po.ORDER_AVX2)
    st = np.uint16 if cfg.dtype == po.DT_BF16 else np.float32
    esz = po.ELEM[cfg.dtype]
    rng = np.random.default_rng(0)
    for l in range(cfg.n_layers):
        ly = lay["layers"][l]
        router = model[ly["router"]: ly["router"] + cfg.n_experts * cfg.dim * esz].view(st).reshape(cfg.n_experts,
                                                                                                    cfg.dim)
        experts = model[ly["experts"]: ly["experts"] + cfg.n_experts * lay["expert_stride"]]
        T = 3
        xb = rng.standard_normal((T, cfg.dim)).astype(np.float32)
        x = rng.standard_normal((T, cfg.dim)).astype(np.float32)
        want = po.moe_layer(cfg.dim, cfg.n_experts, cfg.top_k, cfg.expert_hidden, cfg.dtype, cfg.norm_topk, router,
                            experts, lay["expert_stride"], xb, order=po.ORDER_AVX2, x=x)
        x_out, routing = dev.moe(l, xb, x=x)
        bad, unexplained = routing_check(routing, want["routing"], want["probs"])
        assert unexplained == 0, (bad, routing, want["routing"])
        assert normwise_err(x_out - x, want["x"] - x) <= MOE_RTOL
    # dense seam on the lm_head
    xb = rng.standard_normal(cfg.dim).astype(np.float32)
    W = model[lay["lm_head"]: lay["lm_head"] + cfg.vocab * cfg.dim * esz].view(st).reshape(cfg.vocab, cfg.dim)
    want = po.matvec(W, cfg.dtype, xb, po.ORDER_AVX2)
    got = dev.matvec(lay["lm_head"], xb, cfg.vocab)
    assert normwise_err(got, want) <= 1e-5


def test_upload_rejects_bad_images(dev):
    from rabbitm2_amd.hip import HipError
    cfg, gp = MODELS["bf16_renorm"]
    model = po.build_model(cfg, gp)
    bad = model.copy()
    bad[0] = ord("X")
    with pytest.raises(HipError, match="bad magic"):
        dev.upload(bad)
    with pytest.raises(HipError, match="too small"):
        dev.upload(model[: model.size // 2])
    bad = model.copy()
    bad[8 + 7 * 4: 8 + 8 * 4] = np.frombuffer(np.int32(99).tobytes(), np.uint8)  # top_k > n_experts
    with pytest.raises(HipError, match="invalid config"):
        dev.upload(bad)


def test_rejected_upload_keeps_the_loaded_model(dev, tmp_path):
    """A header that fails load_model's checks (rabbit2.c:199-228) leaves the handle's model and decode
    state as they were: the forward pass started before the rejected uploads continues at the next
    positions with the reference's routing and logits (the golden fixture of ref_bf16)."""
    import json
    import os
    import struct
    from rabbitm2_amd.hip import HipError
    from tests.common import normwise_err as nerr
    here = os.path.dirname(os.path.abspath(__file__))
    spec = json.load(open(os.path.join(here, "golden", "manifest.json")))["cases"]["ref_bf16"]
    cfg = po.Config(**spec["config"])
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    fx = np.load(os.path.join(here, "golden", "ref_bf16.npz"))
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    dev.state_init(0)
    tokens = fx["tokens"]

    def step(pos):
        logits, routing = dev.forward(int(tokens[pos]), pos, cfg.vocab, cfg.n_layers, cfg.top_k)
        assert np.array_equal(routing, fx["routing_avx2"][pos]), pos
        assert nerr(logits, fx["logits_avx2"][pos]) <= 1e-3, pos

    half = len(tokens) // 2
    for pos in range(half):
        step(pos)
    other = po.build_model(po.Config(dtype=po.DT_F32, dim=128, n_layers=3), po.ref_style(7))
    bad_magic = other.copy()
    bad_magic[0] = ord("X")
    huge = other.copy()  # n_layers = 2^31 - 1: the layout runs past the image
    huge[8 + 2 * 4: 8 + 3 * 4] = np.frombuffer(struct.pack("<i", 2**31 - 1), np.uint8)
    wrapped = other.copy()  # vocab * dim * 4 bytes past 2^64
    wrapped[8: 8 + 2 * 4] = np.frombuffer(struct.pack("<ii", 2**31 - 1, 2**31 - 1), np.uint8)
    for img, msg in ((bad_magic, "bad magic"), (other[: other.size // 3], "too small"), (huge, "too small"),
                     (wrapped, "too small")):
        with pytest.raises(HipError, match=msg):
            dev.upload(img)
    short = tmp_path / "short.rbt2"
    other[: other.size // 3].tofile(short)
    with pytest.raises(HipError, match="too small"):
        dev.upload_file(str(short))
    for pos in range(half, len(tokens)):
        step(pos)


def test_model_create_rejects_images_beyond_the_device(dev):
    """rbt_hip_model_create bounds the image by the device's memory before it builds the per-layer
    table: 2^31 - 1 layers of a tiny config (about 10 TB of image) fail with a message, and the handle
    stays usable."""
    from rabbitm2_amd import hip as rh
    big = rh.Config(vocab=1, dim=2, n_layers=2**31 - 1, n_heads=1, n_kv_heads=1, head_dim=2, n_experts=1, top_k=1,
                    expert_hidden=1, max_seq=1, dtype=po.DT_F32, qk_norm=0, norm_topk=0, rope_theta=1e4,
                    rms_eps=1e-5)
    with pytest.raises(rh.HipError, match="exceeds the device"):
        dev.model_create(big)
    cfg, gp = MODELS["odd_f32"]
    assert dev.upload(po.build_model(cfg, gp)).dim == cfg.dim
