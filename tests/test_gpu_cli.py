"""The engine's command line over the C ABI (rabbitm2_amd/rabbit2) on the GPU, run exactly as the
reference's own tests run the engine binary (rabbit2/tests/test_forward.py:53-66,
test_engine_cache.py:33-58): --dump files and --gen ids against the reference engine's outputs for the
same arguments (the golden fixtures, tests/golden/make_golden.py and make_sampled.py).

Bar: the routing file identical, logits normwise max error <= 1e-3 per position, ids identical (greedy
and sampled); the expert-cache line keeps the engine's bytes_read == misses * expert_stride."""
import json
import os
import re
import subprocess

import numpy as np
import pytest

from oracle import pyoracle as po
from tests.common import normwise_err

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "rabbitm2_amd", "rabbit2")
GOLDEN = os.path.join(ROOT, "tests", "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))["cases"]
SAMPLED = json.load(open(os.path.join(GOLDEN, "sampled.json")))
KERNEL_FLAGS = {"scalar": [], "avx2": ["--kernel", "avx2"]}  # the orders the fixtures were written in
CACHE = json.load(open(os.path.join(GOLDEN, "cache_stats.json")))
STATS_RE = re.compile(r"(hits|misses|evictions|bytes_read|resident_bytes|capacity_bytes)=(\d+)")
LOGIT_RTOL = 1e-3


def write_case(case, tmp_path):
    spec = MANIFEST[case]
    cfg = po.Config(**spec["config"])
    g = spec["gen_params"]
    path = tmp_path / f"{case}.rbt2"
    po.write_model(str(path), cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                                emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    return spec, cfg, path


def run(*args):
    print("rabbit2", " ".join(str(a) for a in args[1:]), flush=True)
    res = subprocess.run([CLI] + [str(a) for a in args], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    return res.stdout, res.stderr


@pytest.mark.parametrize("case", sorted(MANIFEST))
def test_cli_dump_and_gen_match_reference(tmp_path, case):
    spec, cfg, path = write_case(case, tmp_path)
    fx = np.load(os.path.join(GOLDEN, case + ".npz"))
    tokens = [int(t) for t in fx["tokens"]]
    for tag, flags in KERNEL_FLAGS.items():
        lp, rp = tmp_path / "logits.bin", tmp_path / "routing.bin"
        out, err = run(path, "--dump", lp, rp, *flags, *tokens)
        assert "prompt: %d tokens" % len(tokens) in err
        logits = np.fromfile(lp, dtype="<f4").reshape(len(tokens), cfg.vocab)
        routing = np.fromfile(rp, dtype="<i4").reshape(len(tokens), cfg.n_layers, cfg.top_k)
        assert np.array_equal(routing, fx[f"routing_{tag}"]), f"{case} {tag}"
        for pos in range(len(tokens)):
            assert normwise_err(logits[pos], fx[f"logits_{tag}"][pos]) <= LOGIT_RTOL, f"{case} {tag} pos {pos}"
        out, err = run(path, "--gen", spec["n_gen"], *flags, *tokens)
        assert [int(t) for t in out.split()] == fx[f"gen_{tag}"].tolist(), f"{case} {tag}"
        assert "generated %d in" % spec["n_gen"] in err


@pytest.mark.parametrize("case", sorted(SAMPLED["cases"]))
def test_cli_sampled_gen_matches_reference(tmp_path, case):
    spec, cfg, path = write_case(case, tmp_path)
    fx = np.load(os.path.join(GOLDEN, "sampled.npz"))
    tokens = po.prompt_tokens(spec["gen_params"]["seed"], spec["n_prompt"], cfg.vocab)
    n_gen = SAMPLED["cases"][case]["n_gen"]
    for j, (t, k, p, seed) in enumerate(SAMPLED["settings"]):
        for tag, flags in KERNEL_FLAGS.items():
            out, _ = run(path, "--gen", n_gen, "--temperature", t, "--top-k", k, "--top-p", p, "--seed", seed, *flags,
                         *tokens)
            assert [int(v) for v in out.split()] == fx[f"{case}_s{j}_{tag}"].tolist(), f"{case} setting {j} {tag}"


def test_cli_eos_ctx_and_expert_cache_line(tmp_path):
    spec, cfg, path = write_case("ref_bf16", tmp_path)
    fx = np.load(os.path.join(GOLDEN, "ref_bf16.npz"))
    tokens = [int(t) for t in fx["tokens"]]
    full = fx["gen_scalar"].tolist()
    eos = full[2]
    out, _ = run(path, "--gen", spec["n_gen"], "--eos", eos, *tokens)
    assert [int(v) for v in out.split()] == full[:full.index(eos) + 1]  # eos printed, then stop
    out, _ = run(path, "--gen", 50, "--ctx", len(tokens) + 3, *tokens)  # clamped to ctx - prompt
    assert [int(v) for v in out.split()] == full[:3]
    # --dump and --gen together: both outputs as separate runs give them
    lp, rp = tmp_path / "l.bin", tmp_path / "r.bin"
    out, err = run(path, "--dump", lp, rp, "--gen", spec["n_gen"], "--expert-cache-mib", 64, *tokens)
    assert [int(v) for v in out.split()] == full
    assert np.array_equal(np.fromfile(rp, dtype="<i4").reshape(fx["routing_scalar"].shape), fx["routing_scalar"])
    stats = {k: int(v) for k, v in STATS_RE.findall(err)}
    stride = po.layout(cfg)["expert_stride"]
    assert stats["evictions"] == 0 and stats["bytes_read"] == stats["misses"] * stride
    assert stats["hits"] + stats["misses"] == (len(tokens) + len(full) - 1) * cfg.n_layers * cfg.top_k
    # the moe line: the --dump pass's blocks (one per prompt token and layer; the --gen loop is not timed)
    esz = 2 if cfg.dtype == po.DT_BF16 else 4
    moe = re.findall(r"^moe: bytes=(\d+) GB/s=([\d.]+) %peak=([\d.]+)$", err, re.M)
    assert len(moe) == 1 and float(moe[0][1]) > 0, err
    assert int(moe[0][0]) == len(tokens) * cfg.n_layers * esz * (cfg.n_experts * cfg.dim +
                                                                 3 * cfg.top_k * cfg.expert_hidden * cfg.dim)
    out, err = run(path, "--gen", 2, "--kernel", "hip", *tokens)
    assert "matvec kernel: hip-gfx950" in err and len(out.split()) == 2


@pytest.mark.parametrize("case", sorted({r["case"] for r in CACHE["runs"]}))
def test_cli_expert_cache_line_matches_engine(tmp_path, case):
    """--expert-cache-mib as the reference's cache test runs it (rabbit2/tests/test_engine_cache.py:23-57):
    the dump files identical with and without a budget, and the stats line equal to the reference
    engine's own for the same arguments (tests/golden/cache_stats.json) -- evictions at small budgets,
    resident_bytes within the budget, bytes_read == misses * expert_stride."""
    spec, cfg, path = write_case(case, tmp_path)
    stride = po.layout(cfg)["expert_stride"]
    runs = [r for r in CACHE["runs"] if r["case"] == case]
    lp, rp = tmp_path / "l.bin", tmp_path / "r.bin"
    plain = {}
    for tag, flags in KERNEL_FLAGS.items():
        run(path, "--dump", lp, rp, *flags, *runs[0]["tokens"])
        plain[tag] = (lp.read_bytes(), rp.read_bytes())
    for r in runs:
        flags = KERNEL_FLAGS[r["order"]]
        _, err = run(path, "--dump", lp, rp, "--expert-cache-mib", r["budget_mib"], *flags, *r["tokens"])
        assert rp.read_bytes() == plain[r["order"]][1]
        assert np.array_equal(np.fromfile(lp, "<f4"), np.frombuffer(plain[r["order"]][0], "<f4"))
        stats = {k: int(v) for k, v in STATS_RE.findall(err)}
        assert stats == r["dump"], (r["order"], r["budget_mib"], stats)
        assert stats["resident_bytes"] <= r["budget_mib"] * 1024 * 1024
        assert stats["bytes_read"] == stats["misses"] * stride
        out, err = run(path, "--gen", r["n_gen"], "--expert-cache-mib", r["budget_mib"], *flags, *r["tokens"])
        assert [int(t) for t in out.split()] == r["gen_ids"]
        stats = {k: int(v) for k, v in STATS_RE.findall(err)}
        assert stats == r["gen"], (r["order"], r["budget_mib"], "gen", stats)
    small = min(r["budget_mib"] for r in runs)
    if any(r["dump"]["evictions"] for r in runs if r["budget_mib"] == small):
        print(f"{case}: evictions at {small} MiB as the engine's", flush=True)


def test_cli_gen_prints_each_id_on_its_own_line(tmp_path):
    """--gen writes one id per line as the engine does (rabbit2.c:728-729), read here line by line from
    the pipe as the reference's server does (rabbit2/tools/serve.py:45-60)."""
    spec, cfg, path = write_case("tiny_olmoe_bf16", tmp_path)
    fx = np.load(os.path.join(GOLDEN, "tiny_olmoe_bf16.npz"))
    tokens = [str(int(t)) for t in fx["tokens"]]
    proc = subprocess.Popen([CLI, str(path), "--gen", str(spec["n_gen"]), "--kernel", "avx2"] + tokens,
                            stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, bufsize=1)
    ids = []
    for line in proc.stdout:
        assert line.endswith("\n") and line.strip().lstrip("-").isdigit(), repr(line)
        ids.append(int(line))
    err = proc.stderr.read()
    assert proc.wait(timeout=120) == 0, err
    assert ids == fx["gen_avx2"].tolist()


def test_generate_stream_reports_ids_in_order(dev):
    """rbt_hip_generate_stream: the callback sees the device loop's ids in order; the eos id is reported
    and ends the output; a callback returning 0 stops it; out and n_out as rbt_hip_generate."""
    spec, cfg, _ = MANIFEST["tiny_olmoe_f32"], po.Config(**MANIFEST["tiny_olmoe_f32"]["config"]), None
    g = spec["gen_params"]
    model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                             emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    fx = np.load(os.path.join(GOLDEN, "tiny_olmoe_f32.npz"))
    dev.upload(model)
    dev.set_router_order(po.ORDER_AVX2)
    dev.state_init(0)
    want = fx["gen_avx2"].tolist()
    seen, out, ms = dev.generate_stream(fx["tokens"], spec["n_gen"])
    assert seen == want and out == want and ms[1] > 0
    eos = want[20]
    seen, out, _ = dev.generate_stream(fx["tokens"], spec["n_gen"], eos=eos)
    assert seen == want[:want.index(eos) + 1] and out == seen
    seen, out, _ = dev.generate_stream(fx["tokens"], spec["n_gen"], stop_after=5)
    assert seen == want[:5] and out == want[:5]
    ids, _ = dev.generate(fx["tokens"], spec["n_gen"])  # the plain loop after a stopped stream
    assert ids == want


PATCHED = os.path.join(ROOT, "oracle", "_ref", "rabbit2_hip")


def host_has_avx2():
    try:
        return any("avx2" in ln.split() for ln in open("/proc/cpuinfo") if ln.startswith("flags"))
    except OSError:
        return False


@pytest.mark.skipif(not os.path.exists(PATCHED), reason="patched reference engine not built (oracle/Makefile ref_hip)")
@pytest.mark.parametrize("case", ["tiny_olmoe_bf16", "ref_bf16", "ref_odd_shape", "olmoe_layer_bf16"])
def test_reference_engine_with_the_hip_seam(tmp_path, case):
    """The reference engine itself with the integration patch (rabbitm2_amd/host/rabbit2_hip.patch):
    --kernel hip sends every layer's MoE block to rbt_hip_moe (host pointers) while attention, the dense
    matvecs and sampling stay on the CPU in the engine's own code. Against the reference's fixtures in the
    order --kernel hip picks on this host (auto): routing identical, logits normwise within 1e-3, --gen
    ids identical."""
    spec, cfg, path = write_case(case, tmp_path)
    fx = np.load(os.path.join(GOLDEN, case + ".npz"))
    tag = "avx2" if host_has_avx2() else "scalar"
    tokens = [str(int(t)) for t in fx["tokens"]]
    lp, rp = tmp_path / "logits.bin", tmp_path / "routing.bin"
    print(f"rabbit2_hip {case} --dump --kernel hip", flush=True)
    res = subprocess.run([PATCHED, str(path), "--dump", str(lp), str(rp), "--kernel", "hip"] + tokens,
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr
    assert "matvec kernel: hip-gfx950" in res.stderr
    routing = np.fromfile(rp, dtype="<i4").reshape(len(tokens), cfg.n_layers, cfg.top_k)
    logits = np.fromfile(lp, dtype="<f4").reshape(len(tokens), cfg.vocab)
    assert np.array_equal(routing, fx[f"routing_{tag}"])
    worst = max(normwise_err(logits[p], fx[f"logits_{tag}"][p]) for p in range(len(tokens)))
    assert worst <= LOGIT_RTOL, worst
    res = subprocess.run([PATCHED, str(path), "--gen", str(spec["n_gen"]), "--kernel", "hip"] + tokens,
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr
    assert [int(t) for t in res.stdout.split()] == fx[f"gen_{tag}"].tolist()
    print(f"{case}: routing identical, worst logits error {worst:.2e}", flush=True)


def write_sparse_header(path, **kw):
    """A .rbt2 header of these config fields (the reference's Config defaults for the rest,
    rabbit2/ref/rbt2.py:28-44) in a sparse file exactly as long as its layout: zero weights."""
    import struct
    d = dict(vocab=256, dim=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, n_experts=8, top_k=2,
             expert_hidden=128, max_seq=64, dtype=po.DT_F32, qk_norm=0, norm_topk=1)
    d.update(kw)
    cfg = po.Config(**d)
    with open(path, "wb") as f:
        f.write(b"RBT2" + struct.pack("<I", 2) + bytes(cfg))
        f.truncate(po.layout(cfg)["end"])
    return cfg


@pytest.mark.parametrize("binary", ["cli", "patched"])
def test_expert_read_beyond_4gib(tmp_path, binary):
    """The reference's sparse-file case (rabbit2/tests/test_engine_cache.py:80-97): 1,048,576 zero
    experts per layer, so layer 1's experts start past 4 GiB (an 8 GiB image uploaded to HBM), top-1,
    --expert-cache-mib 1: the stats line reports misses=2 and the routing file holds (0, 0) -- every
    logit is 0, and the lowest index wins the tie. Also its 'budget too small' exit (:72-78)."""
    exe = CLI if binary == "cli" else PATCHED
    if not os.path.exists(exe):
        pytest.skip("patched reference engine not built (oracle/Makefile ref_hip)")
    path = tmp_path / "sparse.rbt2"
    cfg = write_sparse_header(path, vocab=8, dim=2, n_layers=2, n_heads=1, n_kv_heads=1, head_dim=2,
                              n_experts=1048576, top_k=1, expert_hidden=1, max_seq=2)
    assert po.layout(cfg)["layers"][1]["experts"] > 2**32
    kernel = ["--kernel", "hip"] if binary == "patched" else []
    print(f"{binary}: 8 GiB sparse image, --dump --expert-cache-mib 1", flush=True)
    res = subprocess.run([exe, str(path), "--dump", str(tmp_path / "logits"), str(tmp_path / "routing"),
                          "--expert-cache-mib", "1"] + kernel + ["1"], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr
    assert "misses=2" in res.stderr
    assert np.fromfile(tmp_path / "routing", dtype="<i4").tolist() == [0, 0]
    small = tmp_path / "small.rbt2"
    write_sparse_header(small, vocab=8, dim=1024, n_layers=1, n_heads=1, n_kv_heads=1, head_dim=2, n_experts=1,
                        top_k=1, expert_hidden=512, max_seq=2)  # one expert is 6 MiB: more than the 1 MiB budget
    res = subprocess.run([exe, str(small), "--gen", "1", "--expert-cache-mib", "1"] + kernel + ["1"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode != 0 and "budget too small" in res.stderr, res.stderr


TIMING_RE = re.compile(r"prompt: (\d+) tokens in [\d.]+s \(([\d.]+) tok/s\)(?: \| generated (\d+) in [\d.]+s \(([\d.]+) tok/s\))?")
MOE_RE = re.compile(r"^moe: bytes=(\d+) GB/s=([\d.]+) %peak=([\d.]+)$", re.M)


@pytest.mark.skipif(not os.path.exists(PATCHED), reason="patched reference engine not built (oracle/Makefile ref_hip)")
@pytest.mark.parametrize("case,n_gen", [("tiny_olmoe_f32", 32), ("olmoe_layer_bf16", 12)])
def test_engine_drop_in_timing(tmp_path, case, n_gen):
    """The drop-in timed as the engine times itself (its stderr line, rabbit2.c:742-744): the reference
    engine with --kernel hip (the MoE block through rbt_hip_moe, the rest on the CPU) against the same
    engine on the CPU alone (--kernel auto) on the same prompt: identical ids, and the moe line the
    patch adds after the timing line (bytes as the engine's block reads them, GB/s from the library's
    device times). Prints both rates."""
    spec, cfg, path = write_case(case, tmp_path)
    fx = np.load(os.path.join(GOLDEN, case + ".npz"))
    tokens = [str(int(t)) for t in fx["tokens"]]
    n_gen = min(n_gen, cfg.max_seq - len(tokens))
    runs = {}
    for name, exe, kernel in (("hip", PATCHED, "hip"), ("cpu", po.REF_BIN, "auto")):
        res = subprocess.run([exe, str(path), "--gen", str(n_gen), "--kernel", kernel] + tokens, capture_output=True,
                             text=True, timeout=300)
        assert res.returncode == 0, res.stderr
        m = TIMING_RE.search(res.stderr)
        assert m and int(m.group(1)) == len(tokens) and int(m.group(3)) == n_gen, res.stderr
        runs[name] = (res.stdout.split(), float(m.group(2)), float(m.group(4)), res.stderr)
    assert runs["hip"][0] == runs["cpu"][0]
    moe = MOE_RE.findall(runs["hip"][3])
    assert len(moe) == 1, runs["hip"][3]
    blocks = (len(tokens) + n_gen - 1) * cfg.n_layers
    esz = 2 if cfg.dtype == po.DT_BF16 else 4
    assert int(moe[0][0]) == blocks * esz * (cfg.n_experts * cfg.dim + 3 * cfg.top_k * cfg.expert_hidden * cfg.dim)
    assert float(moe[0][1]) > 0
    print(f"{case}: prompt {len(tokens)} + {n_gen} generated | engine --kernel hip: prompt {runs['hip'][1]:.1f} tok/s, "
          f"gen {runs['hip'][2]:.1f} tok/s, moe {moe[0][1]} GB/s ({moe[0][2]}% of peak) | engine on the CPU: prompt "
          f"{runs['cpu'][1]:.1f} tok/s, gen {runs['cpu'][2]:.1f} tok/s", flush=True)
