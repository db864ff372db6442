"""Benchmark of the MI355X MoE-layer path at the OLMoE-1B-7B shape, batch-1 decode.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]

Workload: one step = one decode token through the 16 MoE layers of an OLMoE-1B-7B-shaped model
(each layer: hidden 2048, 64 experts, top-8, SwiGLU intermediate 1024, bf16 weights ~N(0, 0.02),
renormalised top-8 weights). All 16 layers' routers and experts (12.9 GB) are resident in HBM in
the .rbt2 storage format; every layer reads its own weights, so a step streams ~1.6 GB and the
256 MB last-level cache cannot hold a step's working set. Inputs are bf16-valued N(0,1)
activations already in HBM; each (step, layer) takes one of 64 pre-generated vectors, so the
selected experts change from step to step. Only the MoE blocks are timed (the attention half of
the model is not part of this path).

Prints one JSON line: tok/s of the 16-layer MoE stack; the roofline of the dominant kernel
(expert gate/up GEMV) from HIP events on the stream it runs on; the whole-layer HBM rate; the
512-token prefill of layer 0 ("prefill": uniform and skewed routing, tokens-per-expert histogram,
HBM rate and matrix-core utilisation of the grouped GEMMs); the whole OLMoE-1B-7B-shaped model
("full_model": 16 layers with attention, vocab 50304, a 128-token prompt and 256 greedy tokens
through the device-side generate loop, and "batched_decode": 32 sequences with 2048-token contexts, 64
greedy tokens each); and the CPU baselines (the oracle, the engine's own
arithmetic in its AVX2 order, on one host core).
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s (OLMoE-1B-7B shape, bs=1); MoE-layer HBM GB/s & % of peak"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published

D, E, K, H, LAYERS = 2048, 64, 8, 1024, 16
SEED = 1
W_SCALE = 0.02
NX = 64  # distinct input vectors cycled through
TRAFFIC_KEY = {"gateup": "gateup_fast"}
KERNEL_DESC = {"gateup": "gateup_fast (softmax + top-k, expert gate+up projections, SwiGLU)"}


def hip_events():
    """hipEvent API from libamdhip64 (events recorded on the library's own stream)."""
    hip = C.CDLL("libamdhip64.so")
    hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
    hip.hipEventSynchronize.argtypes = [C.c_void_p]
    hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
    hip.hipEventDestroy.argtypes = [C.c_void_p]
    hip.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    hip.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    hip.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
    hip.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
    hip.hipGraphExecDestroy.argtypes = [C.c_void_p]
    hip.hipGraphDestroy.argtypes = [C.c_void_p]

    def make():
        e = C.c_void_p()
        assert hip.hipEventCreate(C.byref(e)) == 0
        return e

    def elapsed(a, b):
        assert hip.hipEventSynchronize(b) == 0
        ms = C.c_float()
        assert hip.hipEventElapsedTime(C.byref(ms), a, b) == 0
        return ms.value

    return hip, make, elapsed


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-fused", action="store_true", help="separate top-k launch (four launches per layer) "
                    "instead of the top-k inside the gate/up kernel")
    ap.add_argument("--eager", action="store_true", help="launch every layer from Python instead of replaying a "
                    "captured HIP graph of the steps")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target length of the CPU baseline sample")
    ap.add_argument("--no-prefill", action="store_true", help="skip the 512-token prefill leg")
    ap.add_argument("--prefill-reps", type=int, default=20, help="timed calls per prefill workload")
    ap.add_argument("--no-full-model", action="store_true", help="skip the whole-model generate leg")
    ap.add_argument("--no-batched", action="store_true", help="skip the 32-sequence batched decode leg")
    ap.add_argument("--profile-forward", type=int, default=0, metavar="N",
                    help="only run N eager forward() steps of the whole model (for kernel traces) and exit")
    ap.add_argument("--profile-decode", type=int, default=0, metavar="N",
                    help="only run N eager decode steps of the 16-layer MoE stack (one weight fill per layer) for "
                         "kernel traces and exit")
    ap.add_argument("--profile-prefill", type=int, default=0, metavar="N",
                    help="only run N eager 512-token calls of layer 0 (uniform, then skewed routing) for kernel "
                         "traces and exit")
    ap.add_argument("--profile-batch", type=int, default=0, metavar="B",
                    help="with --profile-forward: B sequences per step at the batched leg's context length")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="also run one device-to-device copy of this size (a known-size kernel for scaling "
                         "FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: the MoE-layer path runs on one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "multi-GPU sharding of the MoE layer is a design note, not a measured path.", file=sys.stderr)
        sys.exit(2)

    if args.profile_forward > 0:
        profile_forward(args.profile_forward, args.profile_batch)
        return
    if args.profile_prefill > 0:
        profile_prefill(args.profile_prefill)
        return
    if args.profile_decode > 0:
        profile_decode(args.profile_decode)
        return

    from rabbitm2_amd import hip as rh

    dev = rh.Device(0)
    esz = 2
    stride = (3 * H * D * esz + 4095) // 4096 * 4096
    layer_bytes = E * stride
    routers = dev.malloc(LAYERS * E * D * esz)
    experts = dev.malloc(LAYERS * layer_bytes)
    t0 = time.time()
    mat = H * D
    for l in range(LAYERS):
        # stream ids follow the oracle writer's numbering for layer l (router 16+16l+8, experts 1<<32 | ...)
        dev.fill_normal(routers, rh.DT_BF16, E * D, SEED, 16 + 16 * l + 8, scale=W_SCALE, byte_offset=l * E * D * esz)
        for e in range(E):
            base = l * layer_bytes + e * stride
            for w in range(3):
                st = (1 << 32) | ((l * E + e) * 3 + w)
                dev.fill_normal(experts, rh.DT_BF16, mat, SEED, st, scale=W_SCALE, byte_offset=base + w * mat * esz)
    xb = dev.malloc(NX * D * 4)
    xraw = dev.malloc(NX * D * 2)
    dev.fill_normal(xraw, rh.DT_BF16, NX * D, SEED, 0x5EED)
    xs_host = (dev.d2h(xraw, (NX * D,), np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(NX, D)
    dev.h2d(xb, xs_host)
    dev.synchronize()
    fill_s = time.time() - t0

    layers = [rh.moe_layer_desc(D, E, K, H, rh.DT_BF16, 1, routers.offset(l * E * D * esz),
                                experts.offset(l * layer_bytes), stride) for l in range(LAYERS)]
    moe_out = dev.malloc(LAYERS * D * 4)
    routing = dev.malloc(LAYERS * K * 4)
    dev.reserve(layers[0], 1)
    dev.set_router_order(rh.ORDER_AVX2)
    dev.set_option("fused_decode", 0 if args.no_fused else 1)

    def step(s):
        for l in range(LAYERS):
            i = (s * LAYERS + l) % NX
            dev.moe_dev(layers[l], xb.offset(i * D * 4), 1, moe=moe_out.offset(l * D * 4),
                        routing=routing.offset(l * K * 4))

    hipapi, mk, elapsed = hip_events()
    stream = C.c_void_p(dev.stream)
    if args.copy_calib_mib:
        # one device-to-device copy of known size (the runtime's blit kernel reads and writes exactly
        # this many bytes), for scaling the FETCH_SIZE / WRITE_SIZE counters of a --pmc run
        nb = args.copy_calib_mib << 20
        src, dst = dev.malloc(nb), dev.malloc(nb)
        dev.memset(src, 1)
        hipapi.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        assert hipapi.hipMemcpyAsync(dst.p, src.p, nb, 3, stream) == 0  # hipMemcpyDeviceToDevice
        dev.synchronize()
        dev.free(src)
        dev.free(dst)
    # A decode engine replays a captured graph per token; one graph here holds GRAPH_STEPS steps so
    # the 64 input vectors are all cycled through (kernels only: no memset/copy nodes).
    GRAPH_STEPS = NX // LAYERS
    for s in range(args.warmup):
        step(s)
    step(GRAPH_STEPS - 1)
    dev.synchronize()
    eager_ref = dev.d2h(moe_out, (LAYERS, D), np.float32)  # eager output of the graph's last step
    gexec = None
    if not args.eager:
        graph, gexec = C.c_void_p(), C.c_void_p()
        assert hipapi.hipStreamBeginCapture(stream, 2) == 0  # hipStreamCaptureModeRelaxed
        for s in range(GRAPH_STEPS):
            step(s)
        assert hipapi.hipStreamEndCapture(stream, C.byref(graph)) == 0
        assert hipapi.hipGraphInstantiate(C.byref(gexec), graph, None, None, 0) == 0
        # every replay must reproduce the eager result of the same step
        for r in range(3):
            assert hipapi.hipGraphLaunch(gexec, stream) == 0
            dev.synchronize()
            got = dev.d2h(moe_out, (LAYERS, D), np.float32)
            assert got.tobytes() == eager_ref.tobytes(), "graph replay differs from eager launch"

    steps = args.steps
    if gexec is not None:
        steps = (args.steps + GRAPH_STEPS - 1) // GRAPH_STEPS * GRAPH_STEPS
    ev0, ev1 = mk(), mk()
    w0 = time.perf_counter()
    hipapi.hipEventRecord(ev0, stream)
    if gexec is not None:
        for _ in range(steps // GRAPH_STEPS):
            hipapi.hipGraphLaunch(gexec, stream)
    else:
        for s in range(steps):
            step(args.warmup + s)
    hipapi.hipEventRecord(ev1, stream)
    dev.synchronize()
    wall = time.perf_counter() - w0
    gpu_ms = elapsed(ev0, ev1)
    ms_per_step = gpu_ms / steps
    args.steps = steps

    # ---- per-kernel durations: HIP events around every launch on the library stream, taken in a
    # pass of eager steps that run back to back (deferred profiling: no wait between calls)
    kern = {}
    dev.profile(2)
    nprof = max(10, min(args.steps, 50))
    for s in range(nprof):
        step(s)
    for name in ("router", "topk", "gateup", "down_combine"):
        tot, n = dev.profile_get(name)
        if n:
            kern[name] = {"avg_us": 1000.0 * tot / n, "launches": n}
    dev.profile(0)

    w_experts = K * 3 * H * D * esz  # the 8 selected experts' w1, w3, w2
    alg_bytes = {
        "router": E * D * esz + D * 4,
        "topk": E * 4 * 2 + K * 8,  # logits in, probabilities out, routing + weights out
        "gateup": K * 2 * H * D * esz + D * 4 + K * H * 4,  # weights + x read + h written
        "down_combine": K * D * H * esz + K * H * 4 + D * 4,
    }
    layer_alg = E * D * esz + w_experts  # 100,925,440: router + 8 experts
    for name in kern:
        kern[name]["alg_bytes"] = alg_bytes[name]
        kern[name]["GBps"] = alg_bytes[name] / (kern[name]["avg_us"] * 1e-6) / 1e9
    dom_name = "gateup"
    dom = kern[dom_name]
    layer_us = 1000.0 * ms_per_step / LAYERS
    layer_gbs = layer_alg / (layer_us * 1e-6) / 1e9

    # routing histogram sanity (the last step's selections)
    last_routing = dev.d2h(routing, (LAYERS, K), np.int32)
    assert np.all((last_routing >= 0) & (last_routing < E))

    # HBM bytes per launch of the dominant kernel, from the calibrated rocprofv3 --pmc runs kept
    # under profiles/ (counters cannot be read from inside this process)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "olmoe_moe_layer_traffic.json")
    if os.path.exists(tpath):
        try:
            traffic = json.load(open(tpath))["per_launch"][TRAFFIC_KEY[dom_name]]["bytes"]
        except (KeyError, ValueError):
            traffic = None

    value = 1000.0 / ms_per_step
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "OLMoE-1B-7B MoE stack decode, bs=1: 16 MoE layers (hidden 2048, 64 experts, top-8, "
                        "SwiGLU 1024, bf16 weights ~N(0,0.02), renormalised top-8), one token per step, "
                        "all experts HBM-resident",
            "layers": LAYERS, "dim": D, "n_experts": E, "top_k": K, "expert_hidden": H, "weights": "bf16",
            "activations": "f32 (bf16-valued N(0,1))", "router_order": "avx2 (bit-exact engine order)",
            "global_batch": 1,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": KERNEL_DESC[dom_name],
            "achieved": round(dom["GBps"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": "profiles/olmoe_moe_layer_traffic.json" if traffic else None,
            "alg_bytes_per_launch": alg_bytes[dom_name],
            "avg_launch_us": round(dom["avg_us"], 3),
        },
        "layer": {
            "alg_bytes": layer_alg,
            "us": round(layer_us, 3),
            "GBps": round(layer_gbs, 1),
            "frac_of_hbm_peak": round(layer_gbs / HBM_PEAK_GBS, 4),
        },
        "kernels": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kern.items()},
        "launch": "eager" if gexec is None else f"hip graph ({GRAPH_STEPS} steps per graph)",
        "wall_s": round(wall, 3),
        "setup_s": round(fill_s, 2),
    }

    if not args.no_prefill:
        out["prefill"] = prefill_leg(dev, routers, experts, stride, args.prefill_reps, not args.no_cpu)

    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(dev, routers, experts, stride, xs_host, args.cpu_seconds)

    if not args.no_full_model:
        out["full_model"] = full_model_leg(not args.no_cpu, args.cpu_seconds, not args.no_batched)

    print(json.dumps(out), flush=True)
    dev.close()


# The whole model at the OLMoE-1B-7B shape (16 layers, 16 heads x 128 with QK-norm and RoPE, 64
# experts top-8, SwiGLU 1024, vocab 50304, bf16 weights ~N(0, 0.02), norm weights 1.0, OLMoE's
# un-renormalised top-8).
FULL_CFG = dict(vocab=50304, dim=2048, n_layers=16, n_heads=16, n_kv_heads=16, head_dim=128, n_experts=64, top_k=8,
                expert_hidden=1024, max_seq=4096, dtype=1, qk_norm=1, norm_topk=0, rope_theta=10000.0, rms_eps=1e-5)
N_PROMPT, N_GEN = 128, 256
FULL_MATS = ("wq", "wk", "wv", "wo", "router", "experts")
FULL_NORMS = ("attn_norm", "q_norm", "k_norm", "ffn_norm")


def make_full_model(dev):
    """The random-init model of FULL_CFG in a fresh device image; returns (cfg, seconds)."""
    from rabbitm2_amd import hip as rh
    cfg = rh.Config(**FULL_CFG)
    t0 = time.time()
    base = dev.model_create(cfg)
    fill = dev.L.rbt_hip_fill_normal
    sid = [0x4D00]

    def fill_tensor(name, layer, dtype, scale, offset):
        off, nbytes = dev.tensor(name, layer)
        sid[0] += 1
        dev._check(fill(dev.h, C.c_void_p(base.value + off), dtype, nbytes // (2 if dtype == rh.DT_BF16 else 4),
                        SEED, sid[0], 0, scale, offset))

    fill_tensor("tok_emb", 0, rh.DT_BF16, W_SCALE, 0.0)
    for l in range(cfg.n_layers):
        for name in FULL_MATS:
            fill_tensor(name, l, rh.DT_BF16, W_SCALE, 0.0)  # the expert blobs' alignment padding is filled too
        for name in FULL_NORMS:
            fill_tensor(name, l, rh.DT_F32, 0.0, 1.0)
    fill_tensor("final_norm", 0, rh.DT_F32, 0.0, 1.0)
    fill_tensor("lm_head", 0, rh.DT_BF16, W_SCALE, 0.0)
    dev.synchronize()
    return cfg, time.time() - t0


def full_model_leg(with_cpu, cpu_seconds, batched=True):
    """128 random prompt ids, then 256 greedy tokens through rbt_hip_generate (one HIP graph replay
    per token, the argmax feeding the next step on the device). Reports generated tok/s, prompt tok/s
    and the weight bytes streamed per generated token."""
    from rabbitm2_amd import hip as rh
    dev = rh.Device(0)
    cfg, setup_s = make_full_model(dev)
    dev.set_router_order(rh.ORDER_AVX2)
    dev.state_init(N_PROMPT + N_GEN)
    prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, N_PROMPT).astype(np.int32)
    ids0, _ = dev.generate(prompt, N_GEN)  # warm-up (graph capture, first touch)
    ids, (p_ms, g_ms) = dev.generate(prompt, N_GEN)
    assert ids == ids0, "generate is not deterministic"
    assert len(ids) == N_GEN and all(0 <= t < cfg.vocab for t in ids)
    D_, hd = cfg.dim, cfg.head_dim
    qd, kvd = cfg.n_heads * hd, cfg.n_kv_heads * hd
    esz = 2
    per_layer = (qd + 2 * kvd) * D_ * esz + D_ * qd * esz + cfg.n_experts * D_ * esz + \
        cfg.top_k * 3 * cfg.expert_hidden * D_ * esz
    w_bytes = cfg.n_layers * per_layer + cfg.vocab * D_ * esz + D_ * esz
    mean_pos = N_PROMPT + (N_GEN - 1) / 2.0
    kv_bytes = cfg.n_layers * 2 * kvd * 4 * mean_pos
    gen_tok_s = (N_GEN - 1) / (g_ms * 1e-3)
    tok_bytes = w_bytes + kv_bytes
    res = {
        "workload": "OLMoE-1B-7B-shaped model (16 layers, hidden 2048, 16 heads x 128, QK-norm, RoPE, 64 experts "
                    "top-8, SwiGLU 1024, vocab 50304, bf16 ~N(0,0.02)), 128-token random prompt, greedy decode of "
                    "256 tokens at batch 1 with the KV cache in HBM",
        "gen_tok_per_s": round(gen_tok_s, 2),
        "ms_per_token": round(g_ms / (N_GEN - 1), 4),
        "prompt_tok_per_s": round(N_PROMPT / (p_ms * 1e-3), 2),
        "bytes_per_token": int(tok_bytes),
        "hbm_GBps_alg": round(tok_bytes * gen_tok_s / 1e9, 1),
        "hbm_frac_alg": round(tok_bytes * gen_tok_s / 1e9 / HBM_PEAK_GBS, 4),
        "launch": "one HIP graph per token (embedding .. argmax, 7 launches per layer + 3)",
        "setup_s": round(setup_s, 2),
    }
    if with_cpu:
        res["cpu_baseline"] = cpu_full_model(dev, cfg, prompt, cpu_seconds)
    if batched:
        res["batched_decode"] = batched_leg(dev, cfg)
    dev.close()
    return res


def profile_forward(steps, batch):
    """`steps` eager forward steps of the whole model over random ids, for kernel traces (no HIP graphs,
    no bench line). batch 0: rbt_hip_forward at positions 0 .. steps-1; batch B > 0: rbt_hip_forward_batch
    of B sequences at positions B_CTX .. B_CTX + steps - 1 of the batched leg's context (the caches
    below hold the zeros of batch_init instead of a filled context; the kernels read the same bytes)."""
    from rabbitm2_amd import hip as rh
    dev = rh.Device(0)
    cfg, _ = make_full_model(dev)
    dev.set_router_order(rh.ORDER_AVX2)
    rng = np.random.default_rng(SEED)
    t0 = time.perf_counter()
    if batch <= 0:
        dev.state_init(max(steps, 1))
        prompt = rng.integers(0, cfg.vocab, steps).astype(np.int32)
        for p in range(steps):
            dev.forward(int(prompt[p]), p, cfg.vocab, cfg.n_layers, cfg.top_k)
    else:
        dev.batch_init(batch, B_CTX + steps)
        for p in range(steps):
            toks = rng.integers(0, cfg.vocab, batch).astype(np.int32)
            dev.forward_batch(toks, np.full(batch, B_CTX + p, np.int32), cfg.vocab, cfg.n_layers, cfg.top_k)
    dev.synchronize()
    print(f"profile-forward: {steps} eager steps of the 16-layer model (batch {max(batch, 1)}) in "
          f"{time.perf_counter() - t0:.3f} s", file=sys.stderr, flush=True)
    dev.close()


def profile_decode(steps):
    """`steps` eager decode steps (one token through the 16 MoE layers, the decode leg's kernels and
    shapes) for kernel traces: no HIP graphs, no bench line. Each layer's router and expert block is
    filled by one launch (other values than the decode leg's per-expert streams, same sizes)."""
    from rabbitm2_amd import hip as rh
    dev = rh.Device(0)
    esz = 2
    stride = (3 * H * D * esz + 4095) // 4096 * 4096
    layer_bytes = E * stride
    routers = dev.malloc(LAYERS * E * D * esz)
    experts = dev.malloc(LAYERS * layer_bytes)
    for l in range(LAYERS):
        dev.fill_normal(routers, rh.DT_BF16, E * D, SEED, 16 + 16 * l + 8, scale=W_SCALE, byte_offset=l * E * D * esz)
        dev.fill_normal(experts, rh.DT_BF16, layer_bytes // esz, SEED, (1 << 33) | l, scale=W_SCALE,
                        byte_offset=l * layer_bytes)
    xraw = dev.malloc(NX * D * 2)
    dev.fill_normal(xraw, rh.DT_BF16, NX * D, SEED, 0x5EED)
    xs = (dev.d2h(xraw, (NX * D,), np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(NX, D)
    xb = dev.upload_array(xs)
    layers = [rh.moe_layer_desc(D, E, K, H, rh.DT_BF16, 1, routers.offset(l * E * D * esz),
                                experts.offset(l * layer_bytes), stride) for l in range(LAYERS)]
    moe_out = dev.malloc(LAYERS * D * 4)
    dev.reserve(layers[0], 1)
    dev.set_router_order(rh.ORDER_AVX2)
    t0 = time.perf_counter()
    for s in range(steps):
        for l in range(LAYERS):
            i = (s * LAYERS + l) % NX
            dev.moe_dev(layers[l], xb.offset(i * D * 4), 1, moe=moe_out.offset(l * D * 4))
    dev.synchronize()
    print(f"profile-decode: {steps} eager steps of the 16-layer MoE stack in {time.perf_counter() - t0:.3f} s",
          file=sys.stderr, flush=True)
    dev.close()


def profile_prefill(calls):
    """`calls` eager calls of the prefill leg's workload (512 tokens through layer 0 of the decode
    stack, same weights and inputs), uniform and then skewed routing, for kernel traces (no HIP
    graphs, no bench line). Only layer 0's router and experts are filled."""
    from rabbitm2_amd import hip as rh
    dev = rh.Device(0)
    esz = 2
    stride = (3 * H * D * esz + 4095) // 4096 * 4096
    routers = dev.malloc(E * D * esz)
    experts = dev.malloc(E * stride)
    mat = H * D
    dev.fill_normal(routers, rh.DT_BF16, E * D, SEED, 16 + 8, scale=W_SCALE)  # layer 0's stream ids
    for e in range(E):
        for w in range(3):
            dev.fill_normal(experts, rh.DT_BF16, mat, SEED, (1 << 32) | (e * 3 + w), scale=W_SCALE,
                            byte_offset=e * stride + w * mat * esz)
    T = PREFILL_T
    xraw = dev.malloc(T * D * 2)
    dev.fill_normal(xraw, rh.DT_BF16, T * D, SEED, 0x5EED + 1)
    xs = (dev.d2h(xraw, (T * D,), np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(T, D)
    xb = dev.upload_array(xs)
    moe = dev.malloc(T * D * 4)
    bias_dev = dev.upload_array(np.array([2.0] * 8 + [0.0] * (E - 8), np.float32))
    dev.set_router_order(rh.ORDER_AVX2)
    t0 = time.perf_counter()
    for bias in (None, bias_dev):
        L = rh.moe_layer_desc(D, E, K, H, rh.DT_BF16, 1, routers, experts, stride, bias)
        dev.reserve(L, T)
        for _ in range(calls):
            dev.moe_dev(L, xb, T, moe=moe)
        dev.synchronize()
    print(f"profile-prefill: {calls} eager 512-token calls each with uniform and skewed routing in "
          f"{time.perf_counter() - t0:.3f} s", file=sys.stderr, flush=True)
    dev.close()


B_SEQ, B_CTX, B_GEN = 32, 2048, 64


def batched_leg(dev, cfg):
    """32 independent sequences on the same model, each with a 2048-token random-id context run through
    the model into its own KV cache (the prompt phase of rbt_hip_generate_batch), then 64 greedy tokens
    each, all sequences in one step (every expert is touched every step)."""
    dev.batch_init(B_SEQ, B_CTX + B_GEN)
    prompts = np.random.default_rng(SEED + 5).integers(0, cfg.vocab, (B_SEQ, B_CTX)).astype(np.int32)
    ids, (p_ms, g_ms) = dev.generate_batch(prompts, B_GEN)
    assert ids.shape == (B_SEQ, B_GEN) and ids.min() >= 0 and ids.max() < cfg.vocab
    steps = B_GEN - 1
    D_, hd = cfg.dim, cfg.head_dim
    qd, kvd = cfg.n_heads * hd, cfg.n_kv_heads * hd
    esz = 2
    dense = cfg.n_layers * ((qd + 2 * kvd) * D_ + D_ * qd + cfg.n_experts * D_) * esz + cfg.vocab * D_ * esz
    experts = cfg.n_layers * cfg.n_experts * 3 * cfg.expert_hidden * D_ * esz  # every expert, every step
    mean_pos = B_CTX + B_GEN / 2.0
    kv = B_SEQ * cfg.n_layers * 2 * kvd * 4 * mean_pos
    step_bytes = dense + experts + kv
    ms_step = g_ms / steps
    return {
        "workload": f"{B_SEQ} sequences x {B_CTX}-token random-id context in the KV cache, {B_GEN} greedy tokens "
                    "each, one step for all sequences (OLMoE-1B-7B shape, f32 KV cache)",
        "tok_per_s": round(B_SEQ * steps / (g_ms * 1e-3), 1),
        "ms_per_step": round(ms_step, 3),
        "context_fill_s": round(p_ms * 1e-3, 2),
        "bytes_per_step": int(step_bytes),
        "hbm_GBps_alg": round(step_bytes / (ms_step * 1e-3) / 1e9, 1),
        "hbm_frac_alg": round(step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "note": "bytes per step: dense weights once, all 64 experts of every layer, the 32 KV caches at the mean "
                "position",
    }


def cpu_full_model(dev, cfg, prompt, seconds):
    """The engine's forward() (the oracle's orc_run, AVX2 order, bitwise the reference) on one host
    core over a prefix of the prompt, on the same weights read back from HBM."""
    from oracle import pyoracle as po
    size = dev.tensor("lm_head")[0] + dev.tensor("lm_head")[1]
    img = np.empty(size, np.uint8)
    dev._check(dev.L.rbt_hip_d2h(dev.h, img.ctypes.data_as(C.c_void_p), dev.model_base, size))
    hdr = np.frombuffer(b"RBT2" + np.uint32(2).tobytes() + bytes(cfg), np.uint8)  # the .rbt2 header (68 bytes)
    img[:hdr.size] = hdr
    try:
        old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {sorted(old)[0]})
    except (AttributeError, OSError):
        old = None
    try:
        t0 = time.perf_counter()
        po.run(img, prompt[:1], order=po.ORDER_AVX2, ctx=len(prompt))
        t1 = time.perf_counter() - t0
        n = int(max(2, min(len(prompt), seconds / max(t1, 1e-6))))
        t0 = time.perf_counter()
        po.run(img, prompt[:n], order=po.ORDER_AVX2, ctx=len(prompt))
        dt = time.perf_counter() - t0
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"forward() over the first {n} prompt tokens ({dt:.1f} s, one token per call as the engine's "
                      f"loop); host {cpu_model()}"}



PREFILL_T = 512
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix peak, published
PREFILL_KERNELS = ("router", "topk", "dispatch", "gateup", "down_combine", "combine")
PREFILL_GRAPH_CALLS = 8  # calls per captured graph in the prefill leg


def prefill_leg(dev, routers, experts, stride, reps, with_cpu):
    """512 tokens through one OLMoE-shaped MoE layer (layer 0 of the decode stack): once with the
    plain router and once with +2.0 on the router logits of experts 0-7 (skewed load). Reports the
    per-call time, per-kernel times (HIP events), the tokens-per-expert histogram of the dispatch,
    the layer's algorithmic HBM rate and the grouped GEMMs' matrix-core utilisation."""
    from rabbitm2_amd import hip as rh
    T = PREFILL_T
    P = T * K
    xraw = dev.malloc(T * D * 2)
    dev.fill_normal(xraw, rh.DT_BF16, T * D, SEED, 0x5EED + 1)
    xs = (dev.d2h(xraw, (T * D,), np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(T, D)
    dev.free(xraw)
    xb = dev.upload_array(xs)
    moe = dev.malloc(T * D * 4)
    bias_dev = dev.upload_array(np.array([2.0] * 8 + [0.0] * (E - 8), np.float32))
    # algorithmic totals of the layer (every expert touched once, router, x in, moe out)
    esz = 2
    alg_bytes = E * 3 * H * D * esz + E * D * esz + T * D * 2 + T * D * 4
    alg_flops = T * 2 * E * D + P * 6 * H * D
    gemm_flops = {"gateup": P * 4 * H * D, "down_combine": P * 2 * H * D}
    res = {}
    for name, bias in (("uniform", None), ("skewed", bias_dev)):
        L = rh.moe_layer_desc(D, E, K, H, rh.DT_BF16, 1, routers, experts, stride, bias)  # layer 0
        dev.reserve(L, T)
        for _ in range(3):
            dev.moe_dev(L, xb, T, moe=moe)
        dev.synchronize()
        hipapi, mk, elapsed = hip_events()
        stream = C.c_void_p(dev.stream)
        e0, e1 = mk(), mk()
        hipapi.hipEventRecord(e0, stream)
        for _ in range(reps):
            dev.moe_dev(L, xb, T, moe=moe)
        hipapi.hipEventRecord(e1, stream)
        us_eager = 1000.0 * elapsed(e0, e1) / reps
        # the same call captured PREFILL_GRAPH_CALLS times into a HIP graph (kernels only), checked
        # against the eager output; one graph launch per PREFILL_GRAPH_CALLS calls
        dev.synchronize()
        eager_out = dev.d2h(moe, (T, D), np.float32)
        graph, gexec = C.c_void_p(), C.c_void_p()
        assert hipapi.hipStreamBeginCapture(stream, 2) == 0
        for _ in range(PREFILL_GRAPH_CALLS):
            dev.moe_dev(L, xb, T, moe=moe)
        assert hipapi.hipStreamEndCapture(stream, C.byref(graph)) == 0
        assert hipapi.hipGraphInstantiate(C.byref(gexec), graph, None, None, 0) == 0
        for _ in range(3):
            dev.memset(moe, 0)
            assert hipapi.hipGraphLaunch(gexec, stream) == 0
            dev.synchronize()
            assert dev.d2h(moe, (T, D), np.float32).tobytes() == eager_out.tobytes(), "prefill graph replay differs"
        greps = max(1, reps // PREFILL_GRAPH_CALLS)
        hipapi.hipEventRecord(e0, stream)
        for _ in range(greps):
            hipapi.hipGraphLaunch(gexec, stream)
        hipapi.hipEventRecord(e1, stream)
        us = 1000.0 * elapsed(e0, e1) / (greps * PREFILL_GRAPH_CALLS)
        hipapi.hipGraphExecDestroy(gexec)
        hipapi.hipGraphDestroy(graph)
        dev.profile(2)  # per-kernel events, calls back to back
        for _ in range(reps):
            dev.moe_dev(L, xb, T, moe=moe)
        kern = {}
        for kname in PREFILL_KERNELS:
            tot, n = dev.profile_get(kname)
            if n:
                kern[kname] = {"avg_us": round(1000.0 * tot / n, 2)}
        dev.profile(0)
        counts = dev.expert_counts(E)
        tiles = int(sum((c + 63) // 64 for c in counts))  # the GEMMs' 64-row tiles
        issued_rows = int(sum((c + 15) // 16 * 16 for c in counts))
        for kname, fl in gemm_flops.items():
            if kname in kern:
                t = kern[kname]["avg_us"] * 1e-6
                # issued: the MFMAs run per block of 16 list rows (a block past an expert's list is
                # skipped, a partly filled one runs in full), two bf16 MFMAs per product (hi + lo part)
                issued = 2 * fl * issued_rows / P
                kern[kname]["mfma_util_alg"] = round(fl / t / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)
                kern[kname]["mfma_util_issued"] = round(issued / t / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)
                wbytes = E * (2 if kname == "gateup" else 1) * H * D * esz
                kern[kname]["weight_GBps"] = round(wbytes / t / 1e9, 1)
        res[name] = {
            "us_per_call": round(us, 2),
            "us_per_call_eager": round(us_eager, 2),
            "tok_per_s": round(T / (us * 1e-6), 1),
            "hbm_GBps_alg": round(alg_bytes / (us * 1e-6) / 1e9, 1),
            "hbm_frac_alg": round(alg_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "mfma_util_alg": round(alg_flops / (us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
            "kernels": kern,
            "tokens_per_expert": [int(c) for c in counts],
            "row_tiles": tiles,
        }
    out = {"tokens": T, "alg_bytes": alg_bytes, "alg_flops": alg_flops,
           "note": f"per-call time of the whole MoE block (router .. combine), HIP graph of {PREFILL_GRAPH_CALLS} "
                   "calls replayed (us_per_call_eager: back-to-back eager calls), inputs in HBM",
           **res}
    if with_cpu:
        out["cpu_baseline"] = cpu_prefill(dev, routers, experts, stride, xs, 64)
    for b in (xb, moe, bias_dev):
        dev.free(b)
    return out


def cpu_prefill(dev, routers, experts, stride, xs, n):
    """The engine evaluates a prompt token by token (rabbit2.c:703-714): the oracle's AVX2-order MoE
    layer on one host core over n of the prefill tokens, as tok/s."""
    from oracle import pyoracle as po
    router = dev.d2h(routers, (E, D), np.uint16)  # layer 0
    ex = dev.d2h(experts, (E * stride,), np.uint8)
    try:
        old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {sorted(old)[0]})
    except (AttributeError, OSError):
        old = None
    try:
        t0 = time.perf_counter()
        po.moe_layer(D, E, K, H, po.DT_BF16, 1, router, ex, stride, xs[:n], order=po.ORDER_AVX2)
        dt = time.perf_counter() - t0
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)
    return {"value": round(n / dt, 2), "unit": "tok/s", "cores": 1, "kind": "port",
            "sample": f"{n} of the 512 prefill tokens through the layer ({dt:.2f} s)"}


def cpu_baseline(dev, routers, experts, stride, xs, seconds):
    """The engine's own arithmetic (the oracle, AVX2 order, bitwise the reference's --kernel avx2
    path) on one host core, on layer 0's weights read back from HBM: a bounded sample of
    token-layers, scaled to tok/s of the 16-layer stack."""
    from oracle import pyoracle as po
    router = dev.d2h(routers, (E, D), np.uint16)
    ex = dev.d2h(experts, (E * stride,), np.uint8)
    try:
        old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {sorted(old)[0]})
    except (AttributeError, OSError):
        old = None
    try:
        t0 = time.perf_counter()
        po.moe_layer(D, E, K, H, po.DT_BF16, 1, router, ex, stride, xs[:1], order=po.ORDER_AVX2)
        t1 = time.perf_counter() - t0
        n = int(max(3, min(20000, seconds / max(t1, 1e-6))))  # about `seconds` of CPU work
        xin = np.stack([xs[i % len(xs)] for i in range(n)])
        t0 = time.perf_counter()
        po.moe_layer(D, E, K, H, po.DT_BF16, 1, router, ex, stride, xin, order=po.ORDER_AVX2)
        dt = time.perf_counter() - t0
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)
    per_layer = dt / n
    return {
        "value": round(1.0 / (LAYERS * per_layer), 3),
        "unit": "tok/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{n} token-layers through layer 0 (1 token each, {dt:.1f} s), scaled to the 16-layer stack; "
                  f"per layer-token {1000 * per_layer:.2f} ms; host {cpu_model()}",
    }


if __name__ == "__main__":
    main()
