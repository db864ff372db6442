"""ORACLE -- test infrastructure, not product code.

ctypes view of liboracle.so (the CPU restatement of the RABBIT2 engine arithmetic, see
rbt2_oracle.h). Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg import this,
only to check results or to time the CPU baseline; the product library never does.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# RBT_ORACLE_LIB: another build of the same source (the sanitizer test loads an instrumented one)
LIB_PATH = os.environ.get("RBT_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_BIN = os.path.join(HERE, "_ref", "rabbit2")

DT_F32, DT_BF16 = 0, 1
ORDER_SCALAR, ORDER_AVX2, ORDER_LANE16 = 0, 1, 2
ELEM = {DT_F32: 4, DT_BF16: 2}


class Config(C.Structure):
    """Bytes 8..67 of a .rbt2 header (rabbit2/src/rabbit2.c:63-69)."""
    _fields_ = [(n, C.c_int32) for n in ("vocab", "dim", "n_layers", "n_heads", "n_kv_heads", "head_dim",
                                         "n_experts", "top_k", "expert_hidden", "max_seq", "dtype", "qk_norm",
                                         "norm_topk")] + [("rope_theta", C.c_float), ("rms_eps", C.c_float)]

    def __init__(self, **kw):
        d = dict(vocab=256, dim=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16, n_experts=8, top_k=2,
                 expert_hidden=128, max_seq=64, dtype=DT_F32, qk_norm=0, norm_topk=1, rope_theta=10000.0,
                 rms_eps=1e-5)
        d.update(kw)
        super().__init__(**d)

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


class LayerOff(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("attn_norm", "wq", "wk", "wv", "wo", "q_norm", "k_norm", "ffn_norm",
                                          "router", "experts")]


class ModelOff(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("tok_emb", "final_norm", "lm_head", "expert_stride", "end")]


class MoeDesc(C.Structure):
    _fields_ = [("dim", C.c_int32), ("n_experts", C.c_int32), ("top_k", C.c_int32), ("expert_hidden", C.c_int32),
                ("dtype", C.c_int32), ("norm_topk", C.c_int32), ("router", C.c_void_p), ("experts", C.c_void_p),
                ("expert_stride", C.c_uint64), ("router_bias", C.c_void_p)]


class GenParams(C.Structure):
    _fields_ = [("seed", C.c_uint64), ("w_scale", C.c_float), ("fan_in_scale", C.c_int32),
                ("emb_scale", C.c_float), ("norm_jitter", C.c_float)]

    def __init__(self, seed=0, w_scale=0.02, fan_in_scale=0, emb_scale=None, norm_jitter=0.0):
        super().__init__(seed, w_scale, fan_in_scale, w_scale if emb_scale is None else emb_scale, norm_jitter)


# Reference-test-style weights: matrices N(0,1)/sqrt(cols), embeddings 0.5*N(0,1), norms 1+0.1*N(0,1)
# (the scales of rabbit2/ref/reference.py:24-31; the random stream is this repository's own).
def ref_style(seed):
    return GenParams(seed=seed, w_scale=1.0, fan_in_scale=1, emb_scale=0.5, norm_jitter=0.1)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (run `make -C oracle`)")
        L = C.CDLL(LIB_PATH)
        vp, i32, u64, f32 = C.c_void_p, C.c_int, C.c_uint64, C.c_float
        L.orc_layout.argtypes = [C.POINTER(Config), C.POINTER(ModelOff), C.POINTER(LayerOff)]
        L.orc_bf16_to_f32.argtypes, L.orc_bf16_to_f32.restype = [C.c_uint16], f32
        L.orc_f32_to_bf16.argtypes, L.orc_f32_to_bf16.restype = [f32], C.c_uint16
        L.orc_f32_to_bf16_n.argtypes = [vp, vp, C.c_size_t]
        L.orc_matvec.argtypes = [vp, vp, i32, vp, i32, i32, i32]
        L.orc_rmsnorm.argtypes = [vp, vp, vp, i32, f32]
        L.orc_softmax.argtypes = [vp, i32]
        L.orc_silu.argtypes, L.orc_silu.restype = [f32], f32
        L.orc_topk.argtypes = [vp, i32, i32, vp, vp, vp, vp]
        L.orc_moe_layer.argtypes = [C.POINTER(MoeDesc), vp, i32, i32, vp, vp, vp, vp, vp]
        L.orc_run.argtypes = [vp, u64, vp, i32, i32, i32, vp, vp, i32, C.c_int32, vp, C.POINTER(C.c_int)]
        L.orc_run_sampled.argtypes = [vp, u64, vp, i32, i32, i32, vp, vp, i32, C.c_int32, vp, C.POINTER(C.c_int),
                                      C.c_float, i32, C.c_float, u64]
        L.orc_rng_next.argtypes, L.orc_rng_next.restype = [C.POINTER(C.c_uint64)], u64
        L.orc_rng_uniform.argtypes, L.orc_rng_uniform.restype = [C.POINTER(C.c_uint64)], C.c_double
        L.orc_sample.argtypes = [vp, i32, C.c_float, i32, C.c_float, C.POINTER(C.c_uint64), vp, vp]
        L.orc_last_error.restype = C.c_char_p
        L.orc_parse_header.argtypes = [vp, u64, C.POINTER(Config)]
        L.orc_splitmix64_next.argtypes, L.orc_splitmix64_next.restype = [C.POINTER(C.c_uint64)], u64
        L.orc_normal.argtypes, L.orc_normal.restype = [u64, u64, u64], C.c_double
        L.orc_fill_normal.argtypes = [vp, i32, u64, u64, u64, u64, f32, f32]
        L.orc_expert_stream.argtypes, L.orc_expert_stream.restype = [C.POINTER(Config), i32, i32, i32], u64
        L.orc_layer_stream.argtypes, L.orc_layer_stream.restype = [i32, i32], u64
        L.orc_model_file_size.argtypes, L.orc_model_file_size.restype = [C.POINTER(Config)], u64
        L.orc_build_model.argtypes = [vp, u64, C.POINTER(Config), C.POINTER(GenParams)]
        L.orc_write_model.argtypes = [C.c_char_p, C.POINTER(Config), C.POINTER(GenParams)]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def layout(cfg):
    m, ly = ModelOff(), (LayerOff * max(cfg.n_layers, 1))()
    lib().orc_layout(C.byref(cfg), C.byref(m), ly)
    out = {f: getattr(m, f) for f, _ in ModelOff._fields_}
    out["layers"] = [{f: getattr(ly[i], f) for f, _ in LayerOff._fields_} for i in range(cfg.n_layers)]
    return out


def f32_to_bf16(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_n(_p(a), _p(out), a.size)
    return out


def bf16_to_f32(u):
    return (np.asarray(u, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def matvec(W, dtype, x, order):
    W = np.ascontiguousarray(W)
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = W.shape
    out = np.empty(rows, dtype=np.float32)
    lib().orc_matvec(_p(out), _p(W), dtype, _p(x), rows, cols, order)
    return out


def softmax(v):
    v = np.array(v, dtype=np.float32)
    lib().orc_softmax(_p(v), v.size)
    return v


def topk(probs, k):
    probs = np.ascontiguousarray(probs, dtype=np.float32)
    used = np.zeros(probs.size, dtype=np.uint8)
    idx, wt, ws = np.zeros(k, np.int32), np.zeros(k, np.float32), np.zeros(1, np.float32)
    lib().orc_topk(_p(probs), probs.size, k, _p(used), _p(idx), _p(wt), _p(ws))
    return idx, wt, float(ws[0])


def moe_layer(dim, n_experts, top_k, hidden, dtype, norm_topk, router, experts, stride, xb, order=ORDER_AVX2,
              bias=None, x=None):
    """router: array [E][D] in dtype storage; experts: uint8 buffer holding the expert blobs.
    Returns dict(moe, routing, weights, probs[, x])."""
    xb = np.ascontiguousarray(xb, dtype=np.float32).reshape(-1, dim)
    T = xb.shape[0]
    router = np.ascontiguousarray(router)
    experts = np.ascontiguousarray(experts)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    d = MoeDesc(dim, n_experts, top_k, hidden, dtype, norm_topk, router.ctypes.data, experts.ctypes.data, stride,
                None if bias is None else bias.ctypes.data)
    moe = np.zeros((T, dim), np.float32)
    routing = np.zeros((T, top_k), np.int32)
    weights = np.zeros((T, top_k), np.float32)
    probs = np.zeros((T, n_experts), np.float32)
    xo = None if x is None else np.array(x, dtype=np.float32).reshape(T, dim)
    if not lib().orc_moe_layer(C.byref(d), _p(xb), T, order, _p(xo), _p(moe), _p(routing), _p(weights), _p(probs)):
        raise RuntimeError(lib().orc_last_error().decode())
    out = dict(moe=moe, routing=routing, weights=weights, probs=probs)
    if xo is not None:
        out["x"] = xo
    return out


def parse_header(buf):
    cfg = Config()
    b = np.frombuffer(buf, dtype=np.uint8) if not isinstance(buf, np.ndarray) else buf
    if not lib().orc_parse_header(_p(b), b.size, C.byref(cfg)):
        raise ValueError(lib().orc_last_error().decode())
    return cfg


def run(model, tokens, order=ORDER_SCALAR, ctx=0, gen=0, eos=-1, temperature=0.0, top_k=0, top_p=1.0, seed=0):
    """The --dump/--gen behaviour of the engine. model: uint8 array of the .rbt2 bytes. temperature > 0
    samples the generated tokens like --temperature/--top-k/--top-p/--seed."""
    cfg = parse_header(model)
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    nt = tok.size
    logits = np.zeros((nt, cfg.vocab), np.float32)
    routing = np.zeros((nt, cfg.n_layers, cfg.top_k), np.int32)
    gen_out = np.zeros(max(gen, 1), np.int32)
    ng = C.c_int(0)
    if not lib().orc_run_sampled(_p(model), model.size, _p(tok), nt, ctx, order, _p(logits), _p(routing), gen, eos,
                         _p(gen_out), C.byref(ng), temperature, top_k, top_p, seed):
        raise RuntimeError(lib().orc_last_error().decode())
    return logits, routing, gen_out[:ng.value].tolist()


def sample(logits, temperature, top_k, top_p, rng_state):
    """sample_logits on one logits row; returns (token, new rng state)."""
    v = np.ascontiguousarray(logits, dtype=np.float32)
    st = C.c_uint64(rng_state)
    idx = np.zeros(v.size, np.int32)
    prob = np.zeros(v.size, np.float32)
    t = lib().orc_sample(_p(v), v.size, temperature, top_k, top_p, C.byref(st), _p(idx), _p(prob))
    return t, st.value


def rng_next(state):
    st = C.c_uint64(state)
    v = lib().orc_rng_next(C.byref(st))
    return v, st.value


def splitmix64(state, n):
    s = C.c_uint64(state)
    return [lib().orc_splitmix64_next(C.byref(s)) for _ in range(n)]


def normal(seed, stream, i):
    return lib().orc_normal(seed, stream, i)


def fill_normal(n, dtype, seed, stream, first=0, scale=1.0, offset=0.0):
    out = np.empty(n, dtype=np.float32 if dtype == DT_F32 else np.uint16)
    lib().orc_fill_normal(_p(out), dtype, n, seed, stream, first, scale, offset)
    return out


def expert_stream(cfg, layer, e, which):
    return lib().orc_expert_stream(C.byref(cfg), layer, e, which)


def layer_stream(layer, which):
    return lib().orc_layer_stream(layer, which)


def model_file_size(cfg):
    return lib().orc_model_file_size(C.byref(cfg))


def build_model(cfg, gp):
    size = model_file_size(cfg)
    buf = np.zeros(size, dtype=np.uint8)
    if not lib().orc_build_model(_p(buf), size, C.byref(cfg), C.byref(gp)):
        raise RuntimeError(lib().orc_last_error().decode())
    return buf


def write_model(path, cfg, gp):
    if not lib().orc_write_model(os.fsencode(path), C.byref(cfg), C.byref(gp)):
        raise RuntimeError(lib().orc_last_error().decode())


def prompt_tokens(seed, n, vocab):
    """Uniform prompt ids: SplitMix64 outputs of state 1000+seed, reduced mod vocab."""
    return [int(v % vocab) for v in splitmix64(1000 + seed, n)]


# ---------------------------------------------------------------- the reference binary (oracle/_ref)

def have_ref():
    return os.path.exists(REF_BIN)


def ref_dump(model_path, tokens, tmpdir, kernel=None, extra=()):
    """Runs the compiled reference engine with --dump; returns (logits bytes, routing bytes, stderr)."""
    lp, rp = os.path.join(tmpdir, "ref_logits.bin"), os.path.join(tmpdir, "ref_routing.bin")
    cmd = [REF_BIN, str(model_path), "--dump", lp, rp]
    if kernel:
        cmd += ["--kernel", kernel]
    cmd += list(extra) + [str(t) for t in tokens]
    res = subprocess.run(cmd, capture_output=True, text=True, check=True)
    with open(lp, "rb") as f:
        lb = f.read()
    with open(rp, "rb") as f:
        rb = f.read()
    return lb, rb, res.stderr


def ref_gen(model_path, tokens, n, kernel=None, extra=()):
    cmd = [REF_BIN, str(model_path), "--gen", str(n)]
    if kernel:
        cmd += ["--kernel", kernel]
    cmd += list(extra) + [str(t) for t in tokens]
    res = subprocess.run(cmd, capture_output=True, text=True, check=True)
    return [int(t) for t in res.stdout.split()]
