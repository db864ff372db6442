"""Benchmark of the MI355X path for the RABBIT2 engine at the OLMoE-1B-7B shape.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]

Headline ("value"): batch-1 greedy decode of the whole OLMoE-1B-7B-shaped random-init model -- 16
layers, hidden 2048, 16 heads x 128 with QK-norm and RoPE, 64 experts top-8, SwiGLU 1024, vocab 50304,
bf16 weights ~N(0, 0.02), f32 KV cache in HBM -- on a 128-token random prompt, through the device-side
--gen loop (one HIP graph replay per token, the argmax on the device feeding the next step). One step =
one token's forward() + final norm + lm_head + argmax. W untimed steps, then a fresh run of the prompt
and the workload's 256 generated tokens (K + 1 if K > 255), whose last K steps are timed with HIP
events on the library's stream (default K = 255: every step after the first token). value = K / their
time.

The same JSON line carries:
  roofline  the dominant kernel of that step (the MoE gate/up kernel: softmax + top-k, the 8 selected
            experts' w1/w3 rows, SwiGLU): algorithmic bytes / its average duration, from HIP events
            around every launch in eager forward() steps at the timed positions; traffic from the
            calibrated rocprofv3 counter runs kept under profiles/. --profile-forward 383 runs the same
            eager steps for a kernel trace.
  layer     the MoE layer alone (the metric's "MoE-layer HBM GB/s & % of peak"): 16 OLMoE-shaped MoE
            layers with renormalised top-8, one token per step, each layer reading its own 100.9 MB,
            replayed from a HIP graph; per-layer time, HBM rate, per-kernel times; the host-pointer
            seam rbt_hip_moe's per-call cost.
  full_model  per-kernel times of the decode step, prompt rate, bytes per token; batched_decode (32
            sequences with 2048-token contexts, 64 greedy tokens each).
  prefill   512 tokens through one layer, uniform and skewed routing (histogram, HBM rate, MFMA use).
  cpu_baseline  the oracle's forward() (the engine's own arithmetic, AVX2 order, bitwise the
            reference binary) on one host core over a bounded prefix of the same prompt.
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
NX = 64  # distinct input vectors cycled through by the MoE-layer leg
TRAFFIC_KEY = {"gateup": "gateup_fast"}
KERNEL_DESC = {"gateup": "gateup_fast (softmax + top-k, expert gate+up projections, SwiGLU)"}
STEP_KERNELS = ("embed", "qkv", "attention", "attn_merge", "wo", "router", "gateup", "down_combine", "lm_head",
                "argmax")


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


def step_bytes(cfg, pos):
    """Algorithmic HBM bytes of one decode step at position pos: every dense weight once, the router and
    the 8 selected experts of every layer, the lm_head, and the f32 K/V rows of positions 0..pos."""
    D_, hd = cfg.dim, cfg.head_dim
    qd, kvd = cfg.n_heads * hd, cfg.n_kv_heads * hd
    esz = 2
    per_layer = (qd + 2 * kvd) * D_ * esz + D_ * qd * esz + cfg.n_experts * D_ * esz + \
        cfg.top_k * 3 * cfg.expert_hidden * D_ * esz
    return cfg.n_layers * per_layer + cfg.vocab * D_ * esz + D_ * esz + cfg.n_layers * 2 * kvd * 4 * (pos + 1)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=N_GEN - 1, help="timed decode steps (default: the 255 steps "
                    "after the first of the workload's 256 generated tokens)")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target length of each CPU baseline sample")
    ap.add_argument("--layer-steps", type=int, default=200, help="timed steps of the MoE-layer leg")
    ap.add_argument("--no-layer", action="store_true", help="skip the MoE-layer (and prefill) legs")
    ap.add_argument("--no-fused", action="store_true", help="MoE-layer leg: separate top-k launch (four launches "
                    "per layer) instead of the top-k inside the gate/up kernel")
    ap.add_argument("--no-prefill", action="store_true", help="skip the 512-token prefill leg")
    ap.add_argument("--prefill-reps", type=int, default=20, help="timed calls per prefill workload")
    ap.add_argument("--no-batched", action="store_true", help="skip the 32-sequence batched decode leg")
    ap.add_argument("--profile-forward", type=int, default=0, metavar="N",
                    help="only run N eager forward() steps of the whole model (for kernel traces) and exit")
    ap.add_argument("--profile-decode", type=int, default=0, metavar="N",
                    help="only run N eager decode steps of the 16-layer MoE stack (one weight fill per layer) for "
                         "kernel traces and exit")
    ap.add_argument("--profile-prefill", type=int, default=0, metavar="N",
                    help="only run N eager 512-token calls of layer 0 (uniform, then skewed routing) for kernel "
                         "traces and exit")
    ap.add_argument("--profile-layout", choices=("blobs", "tiled"), default="blobs",
                    help="with --profile-prefill: experts read in the .rbt2 storage format (default) or through the "
                         "opt-in tiled copy")
    ap.add_argument("--profile-batch", type=int, default=0, metavar="B",
                    help="with --profile-forward: B sequences per step at the batched leg's context length")
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="also run one device-to-device copy of this size (a known-size kernel for scaling "
                         "FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this path runs on one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "sharding the MoE layer over GPUs is a design note, not a measured path.", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        sys.exit("bench.py: --steps must be >= 1 and --warmup >= 0")

    if args.profile_forward > 0:
        profile_forward(args.profile_forward, args.profile_batch)
        return
    if args.profile_prefill > 0:
        profile_prefill(args.profile_prefill, args.profile_layout == "tiled")
        return
    if args.profile_decode > 0:
        profile_decode(args.profile_decode)
        return

    from rabbitm2_amd import hip as rh

    if rh.profiler_attached() and not args.copy_calib_mib:
        print("bench.py: a profiler tool is attached to this process, and the bench's legs replay HIP graphs, "
              "which are off under a profiler (traced replays have crashed the host process). Trace the eager "
              "modes instead: --profile-forward N, --profile-decode N, --profile-prefill N.", file=sys.stderr)
        sys.exit(2)
    dev = rh.Device(0)
    hipapi, mk, elapsed = hip_events()
    if args.copy_calib_mib:
        # one device-to-device copy of known size (the runtime's blit kernel reads and writes exactly
        # this many bytes), for scaling the FETCH_SIZE / WRITE_SIZE counters of a --pmc run
        nb = args.copy_calib_mib << 20
        src, dst = dev.malloc(nb), dev.malloc(nb)
        dev.memset(src, 1)
        hipapi.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
        assert hipapi.hipMemcpyAsync(dst.p, src.p, nb, 3, C.c_void_p(dev.stream)) == 0  # hipMemcpyDeviceToDevice
        dev.synchronize()
        dev.free(src)
        dev.free(dst)
        # calibration only: nothing else runs under the counters (and no HIP graph under the profiler)
        print(f"copy-calib: {args.copy_calib_mib} MiB device-to-device copy", file=sys.stderr, flush=True)
        dev.close()
        return

    # ---- headline: whole-model bs=1 greedy decode
    cfg, setup_s = make_full_model(dev)
    dev.set_router_order(rh.ORDER_AVX2)
    # every run decodes the workload's whole 256 tokens (more if K asks for more) and times the last K
    # steps of it; generated step g forwards token g - 1 at position N_PROMPT + g - 1
    K_steps = args.steps
    n_gen = max(N_GEN, K_steps + 1)
    first_timed = n_gen - K_steps
    pos_first, pos_last = N_PROMPT + first_timed - 1, N_PROMPT + n_gen - 2
    ctx = N_PROMPT + max(n_gen, args.warmup + 1)
    dev.state_init(ctx)
    prompt = np.random.default_rng(SEED).integers(0, cfg.vocab, N_PROMPT).astype(np.int32)
    warm = []
    if args.warmup > 0:
        warm, _ = dev.generate(prompt, args.warmup + 1)  # graph capture and first touch; untimed
    dev.set_option("generate_timed_from", first_timed)
    w0 = time.perf_counter()
    ids, (p_ms, g_ms) = dev.generate(prompt, n_gen)  # g_ms: the last K steps
    wall = time.perf_counter() - w0
    dev.set_option("generate_timed_from", 1)
    assert len(ids) == n_gen and all(0 <= t < cfg.vocab for t in ids)
    assert ids[:len(warm)] == warm, "generate is not deterministic"
    ms_per_step = g_ms / K_steps
    value = K_steps / (g_ms * 1e-3)
    tok_bytes = np.mean([step_bytes(cfg, p) for p in range(pos_first, pos_last + 1)])

    # ---- per-kernel durations of the step: HIP events around every launch (deferred profiling: no wait
    # between launches inside a step) in eager forward() steps at the timed positions, over the KV cache
    # the timed run left (each re-run writes its position's K/V row again with the same values)
    seq = prompt.tolist() + ids
    prof_pos = profile_positions(pos_first, pos_last)
    kern = eager_step_kernels(dev, cfg, seq, prof_pos)
    esz = 2
    alg = {"gateup": K * 2 * H * D * esz + D * 4 + K * H * 4,  # the 8 experts' w1/w3 rows, x, h written
           "down_combine": K * D * H * esz + K * H * 4 + D * 4,
           "router": E * D * esz + D * 4 * 2,
           "lm_head": cfg.vocab * D * esz + D * 4}
    for name, b in alg.items():
        if name in kern:
            kern[name]["alg_bytes"] = b
            kern[name]["GBps"] = round(b / (kern[name]["avg_us"] * 1e-6) / 1e9, 1)
    dom = kern["gateup"]
    dom_gbs = alg["gateup"] / (dom["avg_us"] * 1e-6) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "olmoe_moe_layer_traffic.json")
    if os.path.exists(tpath):
        try:
            traffic = json.load(open(tpath))["per_launch"][TRAFFIC_KEY["gateup"]]["bytes"]
        except (KeyError, ValueError):
            traffic = None

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K_steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"OLMoE-1B-7B-shaped random-init model, batch-1 greedy decode: {cfg.n_layers} layers, hidden "
                        f"{cfg.dim}, {cfg.n_heads} heads x {cfg.head_dim} (QK-norm, RoPE), {cfg.n_experts} experts "
                        f"top-{cfg.top_k}, SwiGLU {cfg.expert_hidden}, vocab {cfg.vocab}, bf16 weights ~N(0,0.02), "
                        f"f32 KV cache in HBM; {N_PROMPT}-token random prompt, then {len(ids)} generated tokens, "
                        f"the last {K_steps} steps timed (positions {pos_first}..{pos_last}), one HIP graph replay "
                        "per token",
            "model": "OLMoE-1B-7B shape", "layers": cfg.n_layers, "dim": cfg.dim, "n_experts": cfg.n_experts,
            "top_k": cfg.top_k, "expert_hidden": cfg.expert_hidden, "vocab": cfg.vocab, "weights": "bf16",
            "activations": "f32", "router_order": "avx2 (bit-exact engine order)", "global_batch": 1,
            "prompt_tokens": N_PROMPT, "generated_tokens": len(ids), "timed_steps": K_steps,
            "timed_positions": [pos_first, pos_last],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": KERNEL_DESC["gateup"],
            "achieved": round(dom_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dom_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": "profiles/olmoe_moe_layer_traffic.json" if traffic else None,
            "alg_bytes_per_launch": alg["gateup"],
            "avg_launch_us": dom["avg_us"],
            "timing": f"HIP events around each launch in eager forward() steps at {len(prof_pos)} of the timed "
                      f"positions ({prof_pos[0]}..{prof_pos[-1]}) x {cfg.n_layers} layers",
            "launches": dom["launches"],
            "trace_check": "profiles/olmoe_forward_decode_kernels.md: these HIP event timings from a bench run "
                           "beside a rocprofv3 kernel trace of the same eager steps (bench.py --profile-forward 383)",
        },
        "full_model": {
            "bytes_per_token": int(tok_bytes),
            "hbm_GBps_alg": round(tok_bytes * value / 1e9, 1),
            "hbm_frac_alg": round(tok_bytes * value / 1e9 / HBM_PEAK_GBS, 4),
            "prompt_tok_per_s": round(N_PROMPT / (p_ms * 1e-3), 2),
            "step_kernels": kern,
            "launch": "one HIP graph per token (embedding .. argmax)",
            "wall_s": round(wall, 3),
            "setup_s": round(setup_s, 2),
        },
    }

    if not args.no_batched:
        out["full_model"]["batched_decode"] = batched_leg(dev, cfg)
    out["full_model"]["host_pointer_moe"] = host_pointer_moe(dev, cfg)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_full_model(dev, cfg, prompt, args.cpu_seconds)
    dev.state_init(1)  # release the decode state before the layer legs
    if not args.no_layer:
        out["layer"] = moe_layer_leg(dev, args)
    print(json.dumps(out), flush=True)
    dev.close()


PROFILE_MAX_STEPS = 255  # eager steps timed per kernel at most (the workload has 255 timed steps)


def profile_positions(pos_first, pos_last):
    """At most PROFILE_MAX_STEPS positions spread evenly over [pos_first, pos_last], in order."""
    n = pos_last - pos_first + 1
    if n <= PROFILE_MAX_STEPS:
        return list(range(pos_first, pos_last + 1))
    return sorted({pos_first + (i * (n - 1)) // (PROFILE_MAX_STEPS - 1) for i in range(PROFILE_MAX_STEPS)})


def eager_step_kernels(dev, cfg, seq, positions):
    """Per-kernel durations from HIP events around every launch (profiling mode 2) in eager forward()
    steps of token seq[p] at each position p; the KV cache must already hold the positions before
    each p. Returns {kernel: {avg_us, launches, launches_per_step}}."""
    dev.profile(2)
    for pos in positions:
        dev.forward(seq[pos], pos, cfg.vocab, cfg.n_layers, cfg.top_k)
    kern = {}
    for name in STEP_KERNELS:
        tot, n = dev.profile_get(name)
        if n:
            kern[name] = {"avg_us": round(1000.0 * tot / n, 3), "launches": int(n),
                          "launches_per_step": n // len(positions)}
    dev.profile(0)
    return kern


def host_pointer_moe(dev, cfg, reps=200):
    """Per-call cost of the host-pointer MoE seam rbt_hip_moe (the call an engine patch puts into
    forward(): xb and x copied in, x and the routing copied back, one wait) on layer 0 of the model."""
    rng = np.random.default_rng(SEED + 3)
    res = {}
    for T in (1, 512):
        xb = rng.standard_normal((T, cfg.dim)).astype(np.float32)
        x = rng.standard_normal((T, cfg.dim)).astype(np.float32)
        n = reps if T == 1 else max(5, reps // 20)
        for _ in range(3):
            dev.moe(0, xb, x=x)
        t0 = time.perf_counter()
        for _ in range(n):
            dev.moe(0, xb, x=x)
        res[f"T{T}_us_per_call"] = round(1e6 * (time.perf_counter() - t0) / n, 1)
    res["note"] = "wall time per call through ctypes (a few us of Python included), host buffers pageable"
    return res


def moe_layer_leg(dev, args):
    """The MoE layer alone: 16 OLMoE-shaped MoE layers (router + 64 experts each, renormalised top-8),
    one token per step, every layer reading its own weights; a HIP graph of steps replayed."""
    from rabbitm2_amd import hip as rh
    hipapi, mk, elapsed = hip_events()
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

    stream = C.c_void_p(dev.stream)
    # A decode engine replays a captured graph per token; one graph here holds GRAPH_STEPS steps so
    # the 64 input vectors are all cycled through (kernels only: no memset/copy nodes).
    GRAPH_STEPS = NX // LAYERS
    for s in range(20):
        step(s)
    step(GRAPH_STEPS - 1)
    dev.synchronize()
    eager_ref = dev.d2h(moe_out, (LAYERS, D), np.float32)  # eager output of the graph's last step
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
    steps = (args.layer_steps + GRAPH_STEPS - 1) // GRAPH_STEPS * GRAPH_STEPS
    ev0, ev1 = mk(), mk()
    hipapi.hipEventRecord(ev0, stream)
    for _ in range(steps // GRAPH_STEPS):
        hipapi.hipGraphLaunch(gexec, stream)
    hipapi.hipEventRecord(ev1, stream)
    dev.synchronize()
    ms_per_step = elapsed(ev0, ev1) / steps
    hipapi.hipGraphExecDestroy(gexec)
    hipapi.hipGraphDestroy(graph)

    # per-kernel durations: HIP events around every launch on the library stream, in a pass of eager
    # steps that run back to back (deferred profiling: no wait between calls)
    kern = {}
    dev.profile(2)
    for s in range(50):
        step(s)
    for name in ("router", "topk", "gateup", "down_combine"):
        tot, n = dev.profile_get(name)
        if n:
            kern[name] = {"avg_us": 1000.0 * tot / n, "launches": n}
    dev.profile(0)
    alg_bytes = {
        "router": E * D * esz + D * 4,
        "topk": E * 4 * 2 + K * 8,  # logits in, probabilities out, routing + weights out
        "gateup": K * 2 * H * D * esz + D * 4 + K * H * 4,  # weights + x read + h written
        "down_combine": K * D * H * esz + K * H * 4 + D * 4,
    }
    layer_alg = E * D * esz + K * 3 * H * D * esz  # 100,925,440: router + 8 experts
    for name in kern:
        kern[name]["alg_bytes"] = alg_bytes[name]
        kern[name]["GBps"] = alg_bytes[name] / (kern[name]["avg_us"] * 1e-6) / 1e9
    layer_us = 1000.0 * ms_per_step / LAYERS
    layer_gbs = layer_alg / (layer_us * 1e-6) / 1e9
    last_routing = dev.d2h(routing, (LAYERS, K), np.int32)
    assert np.all((last_routing >= 0) & (last_routing < E))
    res = {
        "workload": "OLMoE-1B-7B MoE layer decode, bs=1: 16 MoE layers (hidden 2048, 64 experts, top-8, SwiGLU "
                    "1024, bf16 weights ~N(0,0.02), renormalised top-8), one bf16-valued N(0,1) token per step, "
                    "all experts HBM-resident, HIP graph of 4 steps replayed",
        "alg_bytes": layer_alg,
        "us": round(layer_us, 3),
        "GBps": round(layer_gbs, 1),
        "frac_of_hbm_peak": round(layer_gbs / HBM_PEAK_GBS, 4),
        "moe_stack_tok_per_s": round(1000.0 / ms_per_step, 2),
        "steps": steps,
        "kernels": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in kern.items()},
        "setup_s": round(fill_s, 2),
    }
    if not args.no_prefill:
        res["prefill"] = prefill_leg(dev, routers, experts, stride, args.prefill_reps, not args.no_cpu)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(dev, routers, experts, stride, xs_host, args.cpu_seconds)
    for b in (routers, experts, xb, xraw, moe_out, routing):
        dev.free(b)
    return res


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


def profile_forward(steps, batch):
    """`steps` eager forward steps of the whole model over random ids, for kernel traces (no HIP graphs,
    no bench line). batch 0: rbt_hip_forward at positions 0 .. steps-1 (383 steps are the bench's prompt
    and its 255 timed positions, the eager steps whose HIP event timings the bench reports; HIP events
    taken under a profiler tool are not a check on its trace, the tool's instrumentation stretches
    them). batch B > 0: rbt_hip_forward_batch of B
    sequences at positions B_CTX .. B_CTX + steps - 1 of the batched leg's context (the caches below
    hold the zeros of batch_init instead of a filled context; the kernels read the same bytes)."""
    from rabbitm2_amd import hip as rh
    dev = rh.Device(0)
    cfg, _ = make_full_model(dev)
    dev.set_router_order(rh.ORDER_AVX2)
    rng = np.random.default_rng(SEED)
    t0 = time.perf_counter()
    if batch <= 0:
        dev.state_init(max(steps, 1))
        seq = rng.integers(0, cfg.vocab, steps).astype(np.int32).tolist()
        for p in range(steps):
            dev.forward(seq[p], p, cfg.vocab, cfg.n_layers, cfg.top_k)
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


def profile_prefill(calls, tiled=False):
    """`calls` eager calls of the prefill leg's workload (512 tokens through layer 0 of the decode
    stack, same weights and inputs), uniform and then skewed routing, for kernel traces (no HIP
    graphs, no bench line). Only layer 0's router and experts are filled. tiled: the grouped GEMMs
    read the opt-in tiled copy of the experts, else the .rbt2 blobs."""
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
    if tiled:
        dev.prefill_layout(rh.moe_layer_desc(D, E, K, H, rh.DT_BF16, 1, routers, experts, stride))
    t0 = time.perf_counter()
    for bias in (None, bias_dev):
        L = rh.moe_layer_desc(D, E, K, H, rh.DT_BF16, 1, routers, experts, stride, bias)
        dev.reserve(L, T)
        for _ in range(calls):
            dev.moe_dev(L, xb, T, moe=moe)
        dev.synchronize()
    print(f"profile-prefill: {calls} eager 512-token calls each with uniform and skewed routing "
          f"({'tiled copy' if tiled else 'blobs'}) in {time.perf_counter() - t0:.3f} s", file=sys.stderr, flush=True)
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


def read_model_image(dev, cfg):
    """The device model image as the bytes of a .rbt2 file (the 68-byte header written in front)."""
    size = dev.tensor("lm_head")[0] + dev.tensor("lm_head")[1]
    img = np.empty(size, np.uint8)
    dev._check(dev.L.rbt_hip_d2h(dev.h, img.ctypes.data_as(C.c_void_p), dev.model_base, size))
    hdr = np.frombuffer(b"RBT2" + np.uint32(2).tobytes() + bytes(cfg), np.uint8)  # the .rbt2 header (68 bytes)
    img[:hdr.size] = hdr
    return img


def cpu_full_model(dev, cfg, prompt, seconds):
    """The CPU baseline of the headline: the reference engine itself (oracle/_ref/rabbit2, built from
    rabbit2/src/rabbit2.c by oracle/Makefile) with its AVX2 matvec (--kernel avx2) on one host core, over
    a prefix of the same prompt on the same weights (the device image written to a .rbt2 file in memory),
    as its own stderr timing line reports it (rabbit2.c:742-744). Beside it, the oracle's forward() (the
    C restatement, bitwise the same arithmetic) on the same prefix. Without the reference binary the
    oracle's rate is the baseline (kind "port")."""
    import re
    import subprocess
    import tempfile
    from oracle import pyoracle as po
    img = read_model_image(dev, cfg)
    try:
        old = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {sorted(old)[0]})  # one core, inherited by the engine's process
    except (AttributeError, OSError):
        old = None
    ref = None
    try:
        t0 = time.perf_counter()
        po.run(img, prompt[:1], order=po.ORDER_AVX2, ctx=len(prompt))
        t1 = time.perf_counter() - t0
        n = int(max(2, min(len(prompt), seconds / max(t1, 1e-6))))
        t0 = time.perf_counter()
        po.run(img, prompt[:n], order=po.ORDER_AVX2, ctx=len(prompt))
        dt = time.perf_counter() - t0
        port = {"value": round(n / dt, 3), "unit": "tok/s", "cores": 1, "kind": "port",
                "sample": f"the oracle's forward() over the first {n} prompt tokens ({dt:.1f} s, one token per call "
                          f"as the engine's loop); host {cpu_model()}"}
        if po.have_ref():
            shm = "/dev/shm" if os.path.isdir("/dev/shm") else None
            with tempfile.TemporaryDirectory(dir=shm) as td:
                path = os.path.join(td, "olmoe.rbt2")
                img.tofile(path)
                del img
                cmd = [po.REF_BIN, path, "--dump", os.devnull, os.devnull, "--ctx", str(len(prompt)), "--kernel", "avx2"]
                res = subprocess.run(cmd + [str(int(t)) for t in prompt[:n]], capture_output=True, text=True,
                                     timeout=max(120.0, 10 * seconds))
                m = re.search(r"prompt: (\d+) tokens in ([\d.]+)s \(([\d.]+) tok/s\)", res.stderr)
                if res.returncode == 0 and m and "matvec kernel: avx2" in res.stderr:
                    ref = {"value": float(m.group(3)), "unit": "tok/s", "cores": 1, "kind": "reference",
                           "sample": f"the reference engine (oracle/_ref/rabbit2 --kernel avx2, built from "
                                     f"rabbit2/src/rabbit2.c) over the first {m.group(1)} prompt tokens of the same "
                                     f"prompt and weights, its own timing line ({m.group(2)} s); host {cpu_model()}",
                           "port_cross_check": port}
    finally:
        if old is not None:
            os.sched_setaffinity(0, old)
    return ref if ref is not None else port



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
    layer0 = rh.moe_layer_desc(D, E, K, H, rh.DT_BF16, 1, routers, experts, stride)
    res = {}
    # first the experts as the converter stores them (the .rbt2 blobs, the default), then with the
    # opt-in tiled copy (rbt_hip_prefill_layout) that the 128-row grouped GEMMs read where it exists
    for layout_name in ("blobs", "tiled_copy"):
        if layout_name == "tiled_copy":
            dev.prefill_layout(layer0)
        res[layout_name] = prefill_workloads(dev, routers, experts, stride, xb, moe, bias_dev, reps, alg_bytes,
                                             alg_flops, gemm_flops)
    dev.prefill_layout_drop(layer0)
    out = {"tokens": T, "alg_bytes": alg_bytes, "alg_flops": alg_flops,
           "expert_layout": "uniform / skewed: the experts read in the .rbt2 storage format (the default); tiled_copy: "
                            "the same calls with the opt-in tiled copy of layer 0 (rbt_hip_prefill_layout)",
           "note": f"per-call time of the whole MoE block (router .. combine), HIP graph of {PREFILL_GRAPH_CALLS} "
                   "calls replayed (us_per_call_eager: back-to-back eager calls), inputs in HBM",
           **res["blobs"], "tiled_copy": res["tiled_copy"]}
    if with_cpu:
        out["cpu_baseline"] = cpu_prefill(dev, routers, experts, stride, xs, 64)
    for b in (xb, moe, bias_dev):
        dev.free(b)
    return out


def prefill_workloads(dev, routers, experts, stride, xb, moe, bias_dev, reps, alg_bytes, alg_flops, gemm_flops):
    """The 512-token call with uniform and with skewed routing (+2.0 on experts 0-7): graph-replayed and
    eager per-call times, per-kernel event times, histogram, HBM rate and matrix-core use."""
    from rabbitm2_amd import hip as rh
    T, P, esz = PREFILL_T, PREFILL_T * K, 2
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
        # the GEMMs' row tiles, by the device's rule: 32 rows while the experts average at most 16, else
        # 128 rows (512 weight rows wide at this shape), their slots column-major where some list is
        # longer than 4x the mean
        tile_rows = 32 if P <= 16 * E else 128
        tile_weight_rows = 512 if tile_rows == 128 and H % 256 == 0 and D % 512 == 0 else 256
        tiles = int(sum((c + tile_rows - 1) // tile_rows for c in counts))
        slot_order = "column-major" if tile_rows == 128 and int(counts.max()) * E > 4 * P else "expert-major"
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
            "tile_rows": tile_rows,
            "tile_weight_rows": tile_weight_rows,
            "row_tiles": tiles,
            "slot_order": slot_order,
        }
    return res


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
