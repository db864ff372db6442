"""rbt_hip_upload_file: the .rbt2 file mapped and copied into HBM once (the replacement of the
engine's mmap + get_expert reads, rabbit2/src/rabbit2.c:129-156, :261-300), its header checks
(load_model, :199-228), and the expert-cache counters in the engine's terms (:745-751; the reference's
own cache test asserts bytes_read == misses * expert_stride, rabbit2/tests/test_engine_cache.py:51).
"""
import ctypes as C
import json
import os

import numpy as np
import pytest

from oracle import pyoracle as po

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))


def build(case):
    spec = MANIFEST["cases"][case]
    cfg = po.Config(**spec["config"])
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    return spec, cfg, model


def device_bytes(dev, ptr, n):
    out = np.empty(n, np.uint8)
    assert dev.L.rbt_hip_d2h(dev.h, out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr), n)
    return out


# ref_bf16: a 1 MB file; olmoe_layer_bf16: an 841 MB one-layer file at the OLMoE shape
@pytest.mark.parametrize("case", ["ref_bf16", "olmoe_layer_bf16"])
def test_upload_file_matches_the_file_and_the_reference(dev, tmp_path, case):
    spec, cfg, model = build(case)
    path = tmp_path / f"{case}.rbt2"
    model.tofile(path)
    got = dev.upload_file(str(path))
    assert (got.dim, got.n_layers, got.n_experts) == (cfg.dim, cfg.n_layers, cfg.n_experts)
    lay = po.layout(cfg)
    # the device image holds the file's bytes: every layer's router and experts, and the lm_head
    for l in range(cfg.n_layers):
        L = dev.layer(l)
        ly = lay["layers"][l]
        nr = cfg.n_experts * cfg.dim * po.ELEM[cfg.dtype]
        assert np.array_equal(device_bytes(dev, L.router, nr), model[ly["router"]:ly["router"] + nr])
        ne = cfg.n_experts * lay["expert_stride"]
        assert np.array_equal(device_bytes(dev, L.experts, ne), model[ly["experts"]:ly["experts"] + ne])
    st = dev.expert_stats()
    assert st["misses"] == cfg.n_layers * cfg.n_experts and st["hits"] == 0 and st["evictions"] == 0
    assert st["bytes_read"] == st["misses"] * lay["expert_stride"]
    # and it runs the reference's --dump
    fx = np.load(os.path.join(GOLDEN, case + ".npz"))
    dev.set_router_order(po.ORDER_AVX2)
    dev.state_init(0)
    for pos, tok in enumerate(fx["tokens"]):
        logits, routing = dev.forward(int(tok), pos, cfg.vocab, cfg.n_layers, cfg.top_k)
        assert np.array_equal(routing, fx["routing_avx2"][pos])
    st = dev.expert_stats()
    assert st["hits"] == len(fx["tokens"]) * cfg.n_layers * cfg.top_k
    assert st["bytes_read"] == st["misses"] * lay["expert_stride"]


def test_upload_file_rejects_bad_files(dev, tmp_path):
    from rabbitm2_amd.hip import HipError
    spec, cfg, model = build("ref_bf16")
    with pytest.raises(HipError, match="cannot open"):
        dev.upload_file(str(tmp_path / "missing.rbt2"))
    short = tmp_path / "short.rbt2"
    model[: model.size // 2].tofile(short)
    with pytest.raises(HipError, match="too small"):
        dev.upload_file(str(short))
    bad = model.copy()
    bad[:4] = np.frombuffer(b"RBT3", np.uint8)
    (tmp_path / "magic.rbt2").write_bytes(bad.tobytes())
    with pytest.raises(HipError, match="magic"):
        dev.upload_file(str(tmp_path / "magic.rbt2"))
    bad = model.copy()
    bad[4:8] = np.frombuffer(np.uint32(3).tobytes(), np.uint8)
    (tmp_path / "version.rbt2").write_bytes(bad.tobytes())
    with pytest.raises(HipError, match="version"):
        dev.upload_file(str(tmp_path / "version.rbt2"))
