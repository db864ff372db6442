"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU (every report is
fatal: -fno-sanitize-recover=all):

  * the library's host side (every .hip source compiled with the sanitizers on its host pass only; the
    kernels are built as usual and never launched here): header parsing and layout of valid, truncated and crafted .rbt2 files, argument
    checks, and the expert-cache replay, driven through
  * the engine's command line (rabbitm2_amd/host/rabbit2_main.c) built with the same sanitizers: every
    path that runs without a GPU, with the exit codes and messages of the normal build;
  * a small C driver of rbt_hip_expert_cache_replay on the reference engine's routing (golden fixtures);
  * the oracle (oracle/rbt2_oracle.c) built with gcc's sanitizers and loaded into a child Python:
    layout, full forward passes against the reference's fixtures, the MoE layer, the sampler.

Device code has no sanitizer on this GPU pool; the kernels are held to the oracle by the GPU tests.
"""
import concurrent.futures as cf
import glob
import json
import os
import shutil
import struct
import subprocess
import sys

import numpy as np
import pytest

from oracle import pyoracle as po

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
GOLDEN = os.path.join(ROOT, "tests", "golden")
HIPCC = "/opt/rocm/bin/hipcc"
CLANG = "/opt/rocm/llvm/bin/clang"
SAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined", "-Xarch_host",
            "-fno-sanitize-recover=all"]
SAN_C = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:exitcode=99",
           UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=98")

pytestmark = [pytest.mark.slow,
              pytest.mark.skipif(not (os.path.exists(HIPCC) and os.path.exists(CLANG)), reason="ROCm clang not found")]


@pytest.fixture(scope="module")
def san(tmp_path_factory):
    """Sanitized host-only library, command line and replay driver in a temporary directory."""
    d = tmp_path_factory.mktemp("san")
    srcs = sorted(glob.glob(os.path.join(ROOT, "rabbitm2_amd", "csrc", "*.hip")))

    def compile_one(src):
        obj = str(d / (os.path.basename(src) + ".o"))
        cmd = [HIPCC, "--offload-arch=gfx950", "-std=c++17", "-O1", "-g", "-fPIC", "-fno-omit-frame-pointer",
               "-Wno-inline-asm", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", INCLUDE] + \
            SAN_HOST + ["-c", src, "-o", obj]
        res = subprocess.run(cmd, capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-3000:]
        return obj

    with cf.ThreadPoolExecutor(min(8, len(srcs))) as ex:
        objs = list(ex.map(compile_one, srcs))
    lib = str(d / "librbt2_hip.so")
    res = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-shared-libsan"] + SAN_HOST +
                         ["-o", lib] + objs, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    rt = subprocess.run([CLANG, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                        text=True).stdout.strip()
    rt_dir = os.path.dirname(rt) if os.path.isabs(rt) else None
    if rt_dir is None or not os.path.exists(rt):
        cands = glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")
        assert cands, "clang ASan runtime not found"
        rt_dir = os.path.dirname(cands[0])
    link = ["-L", str(d), "-lrbt2_hip", "-Wl,-rpath," + str(d), "-Wl,-rpath," + rt_dir, "-shared-libsan"]
    cli = str(d / "rabbit2")
    res = subprocess.run([CLANG, "-std=c99", "-I", INCLUDE] + SAN_C +
                         [os.path.join(ROOT, "rabbitm2_amd", "host", "rabbit2_main.c"), "-o", cli] + link,
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    drv_src = d / "replay.c"
    drv_src.write_text(REPLAY_DRIVER)
    drv = str(d / "replay")
    res = subprocess.run([CLANG, "-std=c99", "-I", INCLUDE] + SAN_C + [str(drv_src), "-o", drv] + link,
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    return {"dir": d, "cli": cli, "replay": drv}


REPLAY_DRIVER = r"""
#include <stdio.h>
#include <stdlib.h>
#include "rbt2_hip.h"
/* replay <routing.bin> <n_tokens> <n_layers> <top_k> <n_experts> <stride> <budget> */
int main(int argc, char **argv) {
    if (argc != 8) return 2;
    const unsigned long long T = strtoull(argv[2], NULL, 10);
    const int L = atoi(argv[3]), K = atoi(argv[4]), E = atoi(argv[5]);
    const unsigned long long stride = strtoull(argv[6], NULL, 10), budget = strtoull(argv[7], NULL, 10);
    int32_t *r = (int32_t *)malloc(sizeof(int32_t) * (T * L * K + 1));
    FILE *f = fopen(argv[1], "rb");
    if (!f || !r || fread(r, sizeof(int32_t), T * L * K, f) != T * L * K) return 3;
    fclose(f);
    uint64_t s[6];
    const int ok = rbt_hip_expert_cache_replay(budget, stride, L, E, K, r, T, s);
    free(r);
    if (!ok) return 1;
    printf("%llu %llu %llu %llu %llu %llu\n", (unsigned long long)s[0], (unsigned long long)s[1],
           (unsigned long long)s[2], (unsigned long long)s[3], (unsigned long long)s[4], (unsigned long long)s[5]);
    return 0;
}
"""


def run(cmd):
    res = subprocess.run([str(c) for c in cmd], capture_output=True, text=True, env=ENV, timeout=120)
    assert "ERROR: AddressSanitizer" not in res.stderr and "runtime error:" not in res.stderr, res.stderr[-4000:]
    assert res.returncode not in (98, 99), res.stderr[-4000:]
    return res.returncode, res.stdout, res.stderr


def header(path, size, **over):
    kw = dict(vocab=8, dim=8, n_layers=1, n_heads=2, n_kv_heads=2, head_dim=4, n_experts=2, top_k=1,
              expert_hidden=8, max_seq=4, dtype=0, qk_norm=0, norm_topk=0)
    kw.update(over)
    fields = ("vocab", "dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "n_experts", "top_k", "expert_hidden",
              "max_seq", "dtype", "qk_norm", "norm_topk")
    with open(path, "wb") as f:
        f.write(b"RBT2" + struct.pack("<I13i2f", 2, *[kw[k] for k in fields], 1e4, 1e-5))
        f.truncate(size)


def test_command_line_paths_without_a_device(san, tmp_path):
    normal = os.path.join(ROOT, "rabbitm2_amd", "rabbit2")
    cfg = po.Config(vocab=64, dim=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, n_experts=4, top_k=2,
                    expert_hidden=32, max_seq=16, dtype=po.DT_BF16, qk_norm=1, norm_topk=0)
    good = tmp_path / "m.rbt2"
    po.write_model(str(good), cfg, po.GenParams(seed=3))
    blob = good.read_bytes()
    files = {"good": good}
    for name, data in (("short", blob[:len(blob) // 2]), ("magic", b"XBT2" + blob[4:]),
                       ("version", blob[:4] + struct.pack("<I", 3) + blob[8:]), ("tiny", blob[:40])):
        (tmp_path / name).write_bytes(data)
        files[name] = tmp_path / name
    for name, over in (("layers", dict(n_layers=2**31 - 1)), ("vocab", dict(vocab=2**31 - 1, dim=2**31 - 1)),
                       ("experts", dict(n_experts=2**31 - 1, expert_hidden=2**31 - 1, dim=2**31 - 1)),
                       ("topk", dict(top_k=5))):
        header(tmp_path / name, 1 << 20, **over)
        files[name] = tmp_path / name
    cases = [[], [good]]
    cases += [[files[k], "--info"] for k in files] + [[tmp_path / "missing", "--info"]]
    cases += [[good, "--info", "--kernel", k] for k in ("auto", "scalar", "avx2", "hip", "bad")]
    cases += [[good, "--gen", "1", "--expert-cache-mib", v, "1"] for v in ("0", "-1", "x", "18446744073709551616")]
    cases += [[good, "--gen", "1", "--nope", "1"], [good, "--gen", "2", "--ctx", "2", "1", "2", "3"],
              [good, "--gen", "2", "999"], [good, "--dump", "a"], [good, "--gen", "2", "1", "2"]]
    for args in cases:
        got = run([san["cli"]] + args)
        want = subprocess.run([normal] + [str(a) for a in args], capture_output=True, text=True, timeout=120)
        assert got[0] == want.returncode, (args, got, want.stderr)
        norm = lambda text, exe: text.replace(exe, "rabbit2")  # usage lines name argv[0]
        assert got[1] == want.stdout, (args, got, want.stdout)
        assert norm(got[2], san["cli"]) == norm(want.stderr, normal), (args, got[2], want.stderr)


def test_cache_replay_driver(san, tmp_path):
    fix = json.load(open(os.path.join(GOLDEN, "cache_stats.json")))
    manifest = json.load(open(os.path.join(GOLDEN, "manifest.json")))["cases"]
    for r in fix["runs"]:
        cfg = po.Config(**manifest[r["case"]]["config"])
        routing = np.load(os.path.join(GOLDEN, r["case"] + ".npz"))[f"routing_{r['order']}"]
        path = tmp_path / "routing.bin"
        routing.astype("<i4").tofile(path)
        stride = po.layout(cfg)["expert_stride"]
        rc, out, err = run([san["replay"], path, routing.shape[0], cfg.n_layers, cfg.top_k, cfg.n_experts, stride,
                            r["budget_mib"] << 20])
        assert rc == 0, err
        keys = ("hits", "misses", "evictions", "bytes_read", "resident_bytes", "capacity_bytes")
        assert dict(zip(keys, map(int, out.split()))) == r["dump"]
    rc, _, err = run([san["replay"], path, routing.shape[0], cfg.n_layers, cfg.top_k, cfg.n_experts, stride, 1])
    assert rc == 1 and "budget too small" in err


ORACLE_CHILD = r"""
import json, os, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from oracle import pyoracle as po
golden = os.path.join(sys.argv[1], "tests", "golden")
manifest = json.load(open(os.path.join(golden, "manifest.json")))["cases"]
for case in ("tiny_olmoe_f32", "ref_bf16", "ref_odd_shape", "ref_tail_dim8", "ref_top1"):
    spec = manifest[case]
    cfg = po.Config(**spec["config"])
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    fx = np.load(os.path.join(golden, case + ".npz"))
    for tag, order in (("scalar", po.ORDER_SCALAR), ("avx2", po.ORDER_AVX2)):
        lg, rt, gen = po.run(model, fx["tokens"], order=order, gen=spec["n_gen"])
        assert lg.tobytes() == fx[f"logits_{tag}"].tobytes(), (case, tag)
        assert np.array_equal(rt, fx[f"routing_{tag}"]) and gen == fx[f"gen_{tag}"].tolist(), (case, tag)
    lg, _, _ = po.run(model, fx["tokens"], order=po.ORDER_AVX2, gen=3, temperature=0.8, top_k=5, top_p=0.9, seed=7)
    lay = po.layout(cfg)
    st = np.uint16 if cfg.dtype == po.DT_BF16 else np.float32
    esz = po.ELEM[cfg.dtype]
    ly = lay["layers"][0]
    router = model[ly["router"]: ly["router"] + cfg.n_experts * cfg.dim * esz].view(st).reshape(cfg.n_experts, cfg.dim)
    experts = model[ly["experts"]: ly["experts"] + cfg.n_experts * lay["expert_stride"]]
    xb = np.random.default_rng(1).standard_normal((3, cfg.dim)).astype(np.float32)
    po.moe_layer(cfg.dim, cfg.n_experts, cfg.top_k, cfg.expert_hidden, cfg.dtype, cfg.norm_topk, router, experts,
                 lay["expert_stride"], xb, order=po.ORDER_SCALAR)
print("ORACLE OK", flush=True)
"""


def test_oracle_under_sanitizers(tmp_path):
    lib = tmp_path / "liboracle_san.so"
    res = subprocess.run(["gcc", "-std=c99", "-ffp-contract=off", "-fPIC", "-shared"] + SAN_C +
                         [os.path.join(ROOT, "oracle", "rbt2_oracle.c"), "-o", str(lib), "-lm"],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    pre = ":".join(subprocess.run(["gcc", f"-print-file-name={n}"], capture_output=True, text=True).stdout.strip()
                   for n in ("libasan.so", "libubsan.so"))
    env = dict(ENV, LD_PRELOAD=pre, RBT_ORACLE_LIB=str(lib))
    res = subprocess.run([sys.executable, "-c", ORACLE_CHILD, ROOT], capture_output=True, text=True, env=env,
                         timeout=600)
    assert "ERROR: AddressSanitizer" not in res.stderr and "runtime error:" not in res.stderr, res.stderr[-4000:]
    assert res.returncode == 0 and "ORACLE OK" in res.stdout, res.stderr[-4000:]
