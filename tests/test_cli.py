"""The engine's command line over the C ABI (rabbitm2_amd/rabbit2), the parts that run without a GPU:
argument and header checks with the reference engine's exit codes and messages
(rabbit2/src/rabbit2.c:610-700), and --info against the layout rules (rabbit2.c:158-193, :668-679).
Where the reference binary built from its source is present (oracle/_ref/rabbit2), every case is also
run through it and the exit code and output compared."""
import json
import os
import subprocess

import pytest

from oracle import pyoracle as po

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "rabbitm2_amd", "rabbit2")
MANIFEST = json.load(open(os.path.join(ROOT, "tests", "golden", "manifest.json")))["cases"]

pytestmark = pytest.mark.skipif(not os.path.exists(CLI), reason="rabbit2 command line not built (rabbitm2_amd.build)")


def run(binary, *args):
    res = subprocess.run([binary] + [str(a) for a in args], capture_output=True, text=True, timeout=60)
    return res.returncode, res.stdout, res.stderr


def small_model(tmp_path, name="m.rbt2", **over):
    kw = dict(vocab=64, dim=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, n_experts=4, top_k=2,
              expert_hidden=32, max_seq=16, dtype=po.DT_BF16, qk_norm=1, norm_topk=0)
    kw.update(over)
    cfg = po.Config(**kw)
    path = tmp_path / name
    po.write_model(str(path), cfg, po.GenParams(seed=3))
    return cfg, path


def parse_info(text):
    return {k: int(v) for k, v in (kv.split("=") for kv in text.split())}


@pytest.mark.parametrize("case", sorted(MANIFEST))
def test_info_matches_layout(tmp_path, case):
    spec = MANIFEST[case]
    cfg = po.Config(**spec["config"])
    path = tmp_path / "m.rbt2"
    g = spec["gen_params"]
    po.write_model(str(path), cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                                emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    rc, out, err = run(CLI, path, "--info")
    assert rc == 0, err
    info = parse_info(out)
    lay = po.layout(cfg)
    for k, v in spec["config"].items():
        if k not in ("rope_theta", "rms_eps"):
            assert info[k] == v, k
    assert info["tok_emb"] == lay["tok_emb"]
    assert info["layer0_experts"] == lay["layers"][0]["experts"]
    assert info["last_layer_experts"] == lay["layers"][-1]["experts"]
    assert info["expert_stride"] == lay["expert_stride"]
    assert info["lm_head"] == lay["lm_head"]
    assert info["layout_end"] == lay["end"]
    assert info["file_size"] == os.path.getsize(path) == spec["model_bytes"]
    if po.have_ref():
        assert run(po.REF_BIN, path, "--info") == (rc, out, err)


def test_info_on_a_sparse_olmoe_size_file(tmp_path):
    """The OLMoE-1B-7B shape: 13.8 GB of layout, a header and a hole (the method of the reference's
    test_layout_big); offsets in closed form."""
    cfg = po.Config(vocab=50304, dim=2048, n_layers=16, n_heads=16, n_kv_heads=16, head_dim=128, n_experts=64,
                    top_k=8, expert_hidden=1024, max_seq=4096, dtype=po.DT_BF16, qk_norm=1, norm_topk=0)
    path = tmp_path / "olmoe.rbt2"
    hdr = po.build_model(po.Config(**{**{f: getattr(cfg, f) for f, _ in po.Config._fields_}, "vocab": 1,
                                      "n_layers": 1, "n_experts": 1, "top_k": 1, "expert_hidden": 1, "dim": 2,
                                      "n_heads": 1, "n_kv_heads": 1, "head_dim": 2}), po.GenParams(seed=0))[:68]
    hdr = bytearray(hdr.tobytes())
    hdr[8:68] = bytes(cfg)[:60]
    with open(path, "wb") as f:
        f.write(bytes(hdr))
        f.truncate(13_838_594_048)
    rc, out, err = run(CLI, path, "--info")
    assert rc == 0, err
    info = parse_info(out)
    assert (info["tok_emb"], info["layer0_experts"], info["last_layer_experts"], info["expert_stride"],
            info["lm_head"], info["layout_end"]) == (4096, 239_898_624, 12_827_234_304, 12_582_912, 13_632_548_864,
                                                    13_838_594_048)
    if po.have_ref():
        assert run(po.REF_BIN, path, "--info") == (rc, out, err)


def test_usage_and_option_errors(tmp_path):
    cfg, path = small_model(tmp_path)
    cases = [
        ((), 2, "usage"),
        ((path,), 2, "usage"),
        ((path, "--gen", "2"), 2, "usage"),                 # no prompt
        ((path, "1", "2"), 2, "usage"),                     # neither --dump nor --gen
        ((path, "--bogus", "1"), 2, "bad option --bogus"),
        ((path, "--gen", "2", "--kernel", "cuda", "1"), 2, "--kernel must be"),
    ]
    for value in ("0", "-1", "garbage", "18446744073709551616"):
        cases.append(((path, "--gen", "1", "--expert-cache-mib", value, "1"), 2, "--expert-cache-mib"))
    for args, code, msg in cases:
        rc, out, err = run(CLI, *args)
        assert rc == code and msg in err, (args, rc, err)
        if po.have_ref() and "--kernel" not in args:
            assert run(po.REF_BIN, *args)[0] == code


def test_runtime_errors_before_the_device(tmp_path):
    """Header, budget, context and token checks fail with exit code 1 before any device work, as the
    engine's do (rabbit2.c:199-228, :236-243, :684-691)."""
    cfg, path = small_model(tmp_path)
    stride = po.layout(cfg)["expert_stride"]
    assert stride > 0
    bad = tmp_path / "bad.rbt2"
    bad.write_bytes(b"NOPE" + bytes(100))
    short = tmp_path / "short.rbt2"
    short.write_bytes(path.read_bytes()[:4096])
    v3 = tmp_path / "v3.rbt2"
    raw = bytearray(path.read_bytes())
    raw[4:8] = (3).to_bytes(4, "little")
    v3.write_bytes(bytes(raw))
    zero = tmp_path / "zero.rbt2"
    raw = bytearray(path.read_bytes())
    raw[8:12] = (0).to_bytes(4, "little")  # vocab 0
    zero.write_bytes(bytes(raw))
    cases = [
        ((tmp_path / "missing.rbt2", "--gen", "1", "1"), "cannot"),
        ((bad, "--gen", "1", "1"), "bad magic"),
        ((short, "--gen", "1", "1"), "file too small"),
        ((v3, "--info"), "unsupported .rbt2 version 3"),
        ((zero, "--info"), "invalid config"),
        ((path, "--gen", "1", "--ctx", "4", "1", "2", "3", "4", "5"), "prompt has 5 tokens but context is 4"),
        ((path, "--gen", "1", str(cfg.vocab)), f"token {cfg.vocab} out of range"),
        ((path, "--gen", "1", "-1"), "token -1 out of range"),
    ]
    big = po.Config(vocab=8, dim=128, n_layers=1, n_heads=4, n_kv_heads=2, head_dim=32, n_experts=1, top_k=1,
                    expert_hidden=4096, max_seq=4, dtype=po.DT_F32)
    bpath = tmp_path / "big.rbt2"
    po.write_model(str(bpath), big, po.GenParams(seed=1))
    assert po.layout(big)["expert_stride"] > 1024 * 1024
    cases.append(((bpath, "--gen", "1", "--expert-cache-mib", "1", "1"), "budget too small"))
    for args, msg in cases:
        rc, out, err = run(CLI, *args)
        assert rc == 1 and msg in err, (args, rc, err)
        if po.have_ref():
            assert run(po.REF_BIN, *args)[0] == 1, args


def test_library_reports_file_info_without_a_device(tmp_path):
    """rbt_hip_file_info is host-only: it answers on a machine without a GPU."""
    from rabbitm2_amd import hip
    import ctypes as C
    cfg, path = small_model(tmp_path, dtype=po.DT_F32, qk_norm=0)
    lib = hip.lib()
    out_cfg = hip.Config()
    info = (C.c_uint64 * 7)()
    assert lib.rbt_hip_file_info(os.fsencode(str(path)), C.byref(out_cfg), info) == 1
    lay = po.layout(cfg)
    assert list(info) == [lay["tok_emb"], lay["layers"][0]["experts"], lay["layers"][-1]["experts"],
                          lay["expert_stride"], lay["lm_head"], lay["end"], os.path.getsize(path)]
    assert [getattr(out_cfg, f) for f, _ in hip.Config._fields_][:13] == [cfg.vocab, cfg.dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                  cfg.n_experts, cfg.top_k, cfg.expert_hidden, cfg.max_seq, cfg.dtype, cfg.qk_norm,
                                  cfg.norm_topk]
    assert lib.rbt_hip_file_info(os.fsencode(str(tmp_path / "none")), None, None) == 0
    assert b"cannot open" in lib.rbt_hip_last_error(None)


def test_kernel_line_as_the_engine_prints_it(tmp_path):
    """The reference's own check of the --kernel flag (rabbit2/tests/test_avx2.py:22-39) run against this
    command line: --kernel auto prints 'matvec kernel: scalar|avx2', an invalid value fails, and --kernel
    avx2 either prints 'matvec kernel: avx2' and succeeds or fails saying it is unavailable."""
    import re
    _, path = small_model(tmp_path)
    for binary in [CLI] + ([po.REF_BIN] if po.have_ref() else []):
        rc, _, err = run(binary, path, "--info", "--kernel", "auto")
        assert rc == 0 and re.search(r"matvec kernel: (scalar|avx2)", err), (binary, err)
        rc, _, err = run(binary, path, "--info", "--kernel", "invalid")
        assert rc != 0, binary
        rc, _, err = run(binary, path, "--info", "--kernel", "avx2")
        if "matvec kernel: avx2" in err:
            assert rc == 0, binary
        else:
            assert rc != 0 and "unavailable" in err, (binary, err)
        rc, _, err = run(binary, path, "--info", "--kernel", "scalar")
        assert rc == 0 and "matvec kernel: scalar" in err, (binary, err)
    # the same choice as the engine's auto on this host
    if po.have_ref():
        assert run(CLI, path, "--info", "--kernel", "auto")[2] == run(po.REF_BIN, path, "--info", "--kernel", "auto")[2]
    rc, _, err = run(CLI, path, "--info", "--kernel", "hip")
    assert rc == 0 and "matvec kernel: hip-gfx950" in err


def write_header(path, size, **over):
    """A bare .rbt2 header of the given config fields, in a (sparse) file of `size` bytes."""
    import struct
    kw = dict(vocab=8, dim=8, n_layers=1, n_heads=2, n_kv_heads=2, head_dim=4, n_experts=2, top_k=1,
              expert_hidden=8, max_seq=4, dtype=0, qk_norm=0, norm_topk=0)
    kw.update(over)
    hdr = b"RBT2" + struct.pack("<I13i2f", 2, *[kw[k] for k in ("vocab", "dim", "n_layers", "n_heads", "n_kv_heads",
                                                                "head_dim", "n_experts", "top_k", "expert_hidden",
                                                                "max_seq", "dtype", "qk_norm", "norm_topk")],
                                1e4, 1e-5)
    with open(path, "wb") as f:
        f.write(hdr)
        f.truncate(size)


@pytest.mark.parametrize("over", [dict(n_layers=2**31 - 1), dict(vocab=2**31 - 1, dim=2**31 - 1, dtype=0),
                                  dict(n_experts=2**31 - 1, expert_hidden=2**31 - 1, dim=2**31 - 1),
                                  dict(n_heads=2**30, n_kv_heads=2**30, head_dim=2**30, dim=2**31 - 1)],
                         ids=["layers", "vocab_dim", "experts", "heads"])
def test_header_with_huge_fields_fails_cleanly(tmp_path, over):
    """Header fields whose layout would run past 2^64 bytes or allocate a per-layer table the file
    cannot back: a clean 'file too small' (exit 1), never an abort or a wrapped offset."""
    path = tmp_path / "big.rbt2"
    write_header(path, 1 << 20, **over)
    rc, out, err = run(CLI, path, "--info")
    assert rc == 1 and "file too small for its own config" in err, (rc, err)
    from rabbitm2_amd import hip
    import ctypes as C
    assert hip.lib().rbt_hip_file_info(os.fsencode(str(path)), None, None) == 0
    assert b"file too small" in hip.lib().rbt_hip_last_error(None)


def test_file_too_small_reports_the_engine_end(tmp_path):
    """A header whose layout ends past the file: the message carries the layout end exactly as the
    engine computes it (rabbit2.c:221-225)."""
    cfg, path = small_model(tmp_path)
    end = po.layout(cfg)["end"]
    with open(path, "r+b") as f:
        f.truncate(end - 1)
    rc, _, err = run(CLI, path, "--info")
    assert rc == 1 and f"file too small for its own config ({end - 1} < {end})" in err
    if po.have_ref():
        rrc, _, rerr = run(po.REF_BIN, path, "--info")
        assert rrc == 1 and f"({end - 1} < {end})" in rerr
