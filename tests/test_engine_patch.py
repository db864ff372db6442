"""The integration patch (rabbitm2_amd/host/rabbit2_hip.patch) on the reference engine's own source
(rabbit2/src/rabbit2.c), on the CPU: it only inserts lines (each block guarded by RABBIT2_HIP), it
applies with GNU patch and builds with the reference's flags and -Werror against include/rbt2_hip.h and
librbt2_hip.so, and the patched engine keeps the CPU path byte for byte (--info, --dump in both of the
engine's orders) while --kernel hip fails cleanly (exit 1, the library's message) where there is no GPU.
The GPU run of --kernel hip is in test_gpu_cli.py. Needs the reference checkout for all but the first
test (skipped otherwise)."""
import ctypes as C
import os
import re
import subprocess

import pytest

from oracle import pyoracle as po

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATCH = os.path.join(ROOT, "rabbitm2_amd", "host", "rabbit2_hip.patch")
REF_SRC = "/root/reference/rabbit2/src/rabbit2.c"
need_ref = pytest.mark.skipif(not os.path.exists(REF_SRC) or not po.have_ref(),
                              reason="reference checkout (and oracle/_ref) not present")


def test_patch_only_inserts_guarded_lines():
    lines = open(PATCH).read().splitlines()
    assert lines[0].startswith("--- ") and lines[1].startswith("+++ ")
    body = lines[2:]
    hunks = [ln for ln in body if ln.startswith("@@")]
    assert hunks and all(re.fullmatch(r"@@ -\d+,0 \+\d+,\d+ @@", h) for h in hunks), hunks
    assert all(ln.startswith("+") or ln.startswith("@@") for ln in body), "the patch removes or keeps lines"
    added = [ln[1:] for ln in body if ln.startswith("+")]
    assert added.count("#ifdef RABBIT2_HIP") == added.count("#endif") == len(hunks)


def build_patched(tmp_path):
    src = tmp_path / "rabbit2.c"
    src.write_bytes(open(REF_SRC, "rb").read())
    subprocess.run(["patch", "-s", str(src), PATCH], check=True)
    exe = tmp_path / "rabbit2_hip"
    res = subprocess.run(["gcc", "-O2", "-std=c99", "-Wall", "-Wextra", "-Werror", "-DRABBIT2_HIP",
                          "-I", os.path.join(ROOT, "include"), str(src), "-L", os.path.join(ROOT, "rabbitm2_amd"),
                          "-lrbt2_hip", "-Wl,-rpath," + os.path.join(ROOT, "rabbitm2_amd"), "-lm", "-o", str(exe)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return str(exe)


def have_device():
    try:
        hip = C.CDLL("libamdhip64.so")
        n = C.c_int(0)
        return hip.hipGetDeviceCount(C.byref(n)) == 0 and n.value > 0
    except OSError:
        return False


@need_ref
def test_patched_engine_builds_and_keeps_the_cpu_path(tmp_path):
    exe = build_patched(tmp_path)
    cfg = po.Config(vocab=96, dim=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, n_experts=6, top_k=2,
                    expert_hidden=48, max_seq=32, dtype=po.DT_BF16, qk_norm=1, norm_topk=0)
    model = tmp_path / "m.rbt2"
    po.write_model(str(model), cfg, po.ref_style(5))
    for args in (["--info"], ["--info", "--kernel", "auto"]):
        a = subprocess.run([exe, str(model)] + args, capture_output=True, text=True)
        b = subprocess.run([po.REF_BIN, str(model)] + args, capture_output=True, text=True)
        assert (a.returncode, a.stdout, a.stderr) == (b.returncode, b.stdout, b.stderr), args
    toks = [str(t) for t in po.prompt_tokens(5, 7, cfg.vocab)]
    for kernel in ([], ["--kernel", "avx2"], ["--kernel", "scalar"]):
        outs = []
        for binary in (exe, po.REF_BIN):
            lp, rp = tmp_path / "l.bin", tmp_path / "r.bin"
            res = subprocess.run([binary, str(model), "--dump", str(lp), str(rp)] + kernel + toks, capture_output=True,
                                 text=True)
            assert res.returncode == 0, res.stderr
            gen = subprocess.run([binary, str(model), "--gen", "5"] + kernel + toks, capture_output=True, text=True)
            outs.append((lp.read_bytes(), rp.read_bytes(), gen.stdout))
        assert outs[0] == outs[1], kernel
    if not have_device():
        res = subprocess.run([exe, str(model), "--gen", "2", "--kernel", "hip"] + toks, capture_output=True, text=True)
        assert res.returncode == 1 and "rbt2_hip: init: no HIP device" in res.stderr, res.stderr
        assert res.stdout == ""
