"""Python view of the C ABI in include/rbt2_hip.h (ctypes over librbt2_hip.so).

This is plumbing for Python hosts (tests, benchmark): every call goes straight to the HIP library.
There is no CPU code path: if the library is missing or no GPU is present, calls raise.
"""
import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "librbt2_hip.so")

DT_F32, DT_BF16 = 0, 1
ORDER_SCALAR, ORDER_AVX2 = 0, 1

# Every symbol include/rbt2_hip.h declares (checked by the CPU test suite).
EXPORTS = (
    "rbt_hip_init", "rbt_hip_free", "rbt_hip_last_error", "rbt_hip_set_router_order", "rbt_hip_upload",
    "rbt_hip_layer", "rbt_hip_moe", "rbt_hip_moe_dev", "rbt_hip_reserve", "rbt_hip_expert_counts_dev",
    "rbt_hip_matvec", "rbt_hip_matvec_dev", "rbt_hip_malloc", "rbt_hip_free_dev", "rbt_hip_h2d", "rbt_hip_d2h",
    "rbt_hip_memset_dev", "rbt_hip_synchronize", "rbt_hip_stream", "rbt_hip_fill_normal", "rbt_hip_profile_enable",
    "rbt_hip_profile_get", "rbt_hip_set_option", "rbt_hip_state_init", "rbt_hip_forward", "rbt_hip_generate",
    "rbt_hip_model_create", "rbt_hip_tensor", "rbt_hip_upload_file", "rbt_hip_expert_stats", "rbt_hip_batch_init",
    "rbt_hip_forward_batch", "rbt_hip_generate_batch", "rbt_hip_set_sampling", "rbt_hip_file_info",
    "rbt_hip_generate_stream", "rbt_hip_routing_history", "rbt_hip_expert_cache_replay",
    "rbt_hip_moe_dev_noalloc", "rbt_hip_prefill_layout", "rbt_hip_prefill_layout_drop", "rbt_hip_profiler_attached",
)

TOKEN_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int32)


class Config(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("vocab", "dim", "n_layers", "n_heads", "n_kv_heads", "head_dim",
                                         "n_experts", "top_k", "expert_hidden", "max_seq", "dtype", "qk_norm",
                                         "norm_topk")] + [("rope_theta", C.c_float), ("rms_eps", C.c_float)]


class MoeLayer(C.Structure):
    """rbt_moe_layer: device pointers to one layer in the .rbt2 storage format."""
    _fields_ = [("dim", C.c_int32), ("n_experts", C.c_int32), ("top_k", C.c_int32), ("expert_hidden", C.c_int32),
                ("dtype", C.c_int32), ("norm_topk", C.c_int32), ("router", C.c_void_p), ("experts", C.c_void_p),
                ("expert_stride", C.c_uint64), ("router_bias", C.c_void_p)]


class HipError(RuntimeError):
    pass


_lib = None


def lib():
    """Loads librbt2_hip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipError(f"{LIB_PATH} is missing: build it with `python -m rabbitm2_amd.build`")
        L = C.CDLL(LIB_PATH)
        vp, i32, u64, f32 = C.c_void_p, C.c_int, C.c_uint64, C.c_float
        L.rbt_hip_init.argtypes = [C.POINTER(vp), i32]
        L.rbt_hip_free.argtypes, L.rbt_hip_free.restype = [vp], None
        L.rbt_hip_last_error.argtypes, L.rbt_hip_last_error.restype = [vp], C.c_char_p
        L.rbt_hip_set_router_order.argtypes = [vp, i32]
        L.rbt_hip_upload.argtypes = [vp, vp, u64, C.POINTER(Config)]
        L.rbt_hip_layer.argtypes = [vp, i32, C.POINTER(MoeLayer)]
        L.rbt_hip_moe.argtypes = [vp, i32, vp, i32, vp, vp]
        L.rbt_hip_moe_dev.argtypes = [vp, C.POINTER(MoeLayer), vp, i32, vp, vp, vp, vp]
        L.rbt_hip_moe_dev_noalloc.argtypes = [vp, C.POINTER(MoeLayer), vp, i32, vp, vp, vp, vp]
        L.rbt_hip_reserve.argtypes = [vp, C.POINTER(MoeLayer), i32]
        L.rbt_hip_prefill_layout.argtypes = [vp, C.POINTER(MoeLayer)]
        L.rbt_hip_prefill_layout_drop.argtypes = [vp, C.POINTER(MoeLayer)]
        L.rbt_hip_expert_counts_dev.argtypes, L.rbt_hip_expert_counts_dev.restype = [vp], vp
        L.rbt_hip_matvec.argtypes = [vp, vp, u64, vp, i32, i32]
        L.rbt_hip_matvec_dev.argtypes = [vp, vp, vp, i32, vp, i32, i32]
        L.rbt_hip_malloc.argtypes = [vp, C.POINTER(vp), u64]
        L.rbt_hip_free_dev.argtypes = [vp, vp]
        L.rbt_hip_h2d.argtypes = [vp, vp, vp, u64]
        L.rbt_hip_d2h.argtypes = [vp, vp, vp, u64]
        L.rbt_hip_memset_dev.argtypes = [vp, vp, i32, u64]
        L.rbt_hip_synchronize.argtypes = [vp]
        L.rbt_hip_stream.argtypes, L.rbt_hip_stream.restype = [vp], vp
        L.rbt_hip_fill_normal.argtypes = [vp, vp, i32, u64, u64, u64, u64, f32, f32]
        L.rbt_hip_profile_enable.argtypes = [vp, i32]
        L.rbt_hip_set_option.argtypes = [vp, C.c_char_p, C.c_int64]
        L.rbt_hip_profile_get.argtypes = [vp, C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_uint64)]
        L.rbt_hip_state_init.argtypes = [vp, i32]
        L.rbt_hip_forward.argtypes = [vp, i32, i32, vp, vp]
        L.rbt_hip_generate.argtypes = [vp, vp, i32, i32, C.c_int32, vp, C.POINTER(C.c_int), C.POINTER(C.c_double)]
        L.rbt_hip_model_create.argtypes = [vp, C.POINTER(Config), C.POINTER(vp)]
        L.rbt_hip_tensor.argtypes = [vp, C.c_char_p, i32, C.POINTER(u64), C.POINTER(u64)]
        L.rbt_hip_upload_file.argtypes = [vp, C.c_char_p, C.POINTER(Config)]
        L.rbt_hip_expert_stats.argtypes = [vp, C.POINTER(C.c_uint64)]
        L.rbt_hip_batch_init.argtypes = [vp, i32, i32]
        L.rbt_hip_set_sampling.argtypes = [vp, f32, i32, f32, u64]
        L.rbt_hip_forward_batch.argtypes = [vp, vp, vp, vp, vp]
        L.rbt_hip_generate_batch.argtypes = [vp, vp, i32, i32, vp, C.POINTER(C.c_double)]
        L.rbt_hip_generate_stream.argtypes = [vp, vp, i32, i32, C.c_int32, TOKEN_FN, vp, vp, C.POINTER(C.c_int),
                                              C.POINTER(C.c_double)]
        L.rbt_hip_routing_history.argtypes = [vp, i32, i32, i32, vp]
        L.rbt_hip_expert_cache_replay.argtypes = [u64, u64, i32, i32, i32, vp, u64, C.POINTER(C.c_uint64)]
        L.rbt_hip_file_info.argtypes = [C.c_char_p, C.POINTER(Config), C.POINTER(C.c_uint64)]
        L.rbt_hip_profiler_attached.argtypes = []
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class DevBuf:
    """A device allocation owned by a Device (freed with it or by free())."""

    def __init__(self, dev, ptr, nbytes):
        self.dev, self.ptr, self.nbytes = dev, ptr, nbytes

    @property
    def p(self):
        return C.c_void_p(self.ptr)

    def offset(self, nbytes):
        return C.c_void_p(self.ptr + nbytes)


class Device:
    """One rbt_hip handle: a GPU, its stream, its device memory."""

    def __init__(self, device=0):
        self.L = lib()
        h = C.c_void_p()
        if not self.L.rbt_hip_init(C.byref(h), device):
            raise HipError(self.L.rbt_hip_last_error(None).decode())
        self.h = h
        self._bufs = []

    def _check(self, ok):
        if not ok:
            raise HipError(self.L.rbt_hip_last_error(self.h).decode())

    def close(self):
        if self.h:
            for b in self._bufs:
                self.L.rbt_hip_free_dev(self.h, C.c_void_p(b.ptr))
            self._bufs = []
            self.L.rbt_hip_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def stream(self):
        return self.L.rbt_hip_stream(self.h)

    def set_router_order(self, order):
        self._check(self.L.rbt_hip_set_router_order(self.h, order))

    def set_option(self, name, value):
        self._check(self.L.rbt_hip_set_option(self.h, name.encode(), int(value)))

    # ---- memory
    def malloc(self, nbytes):
        p = C.c_void_p()
        self._check(self.L.rbt_hip_malloc(self.h, C.byref(p), nbytes))
        b = DevBuf(self, p.value, nbytes)
        self._bufs.append(b)
        return b

    def free(self, b):
        self._bufs.remove(b)
        self._check(self.L.rbt_hip_free_dev(self.h, C.c_void_p(b.ptr)))

    def upload_array(self, a):
        a = np.ascontiguousarray(a)
        b = self.malloc(a.nbytes)
        self.h2d(b, a)
        return b

    def h2d(self, b, a, offset=0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= b.nbytes
        self._check(self.L.rbt_hip_h2d(self.h, b.offset(offset), _p(a), a.nbytes))

    def d2h(self, b, shape, dtype, offset=0):
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= b.nbytes
        self._check(self.L.rbt_hip_d2h(self.h, _p(out), b.offset(offset), out.nbytes))
        return out

    def memset(self, b, value=0):
        self._check(self.L.rbt_hip_memset_dev(self.h, b.p, value, b.nbytes))

    def synchronize(self):
        self._check(self.L.rbt_hip_synchronize(self.h))

    def fill_normal(self, b, dtype, n, seed, stream, first=0, scale=1.0, offset=0.0, byte_offset=0):
        esz = 4 if dtype == DT_F32 else 2
        assert byte_offset + n * esz <= b.nbytes
        self._check(self.L.rbt_hip_fill_normal(self.h, b.offset(byte_offset), dtype, n, seed, stream, first, scale,
                                               offset))

    def profile(self, on):
        """on: False/0 off, True/1 per call (each call waits), 2 deferred (nothing waits)."""
        self._check(self.L.rbt_hip_profile_enable(self.h, int(on)))

    def profile_get(self, kernel):
        ms, n = C.c_double(), C.c_uint64()
        self._check(self.L.rbt_hip_profile_get(self.h, kernel.encode(), C.byref(ms), C.byref(n)))
        return ms.value, n.value

    # ---- model level
    def upload(self, model):
        model = np.ascontiguousarray(model, dtype=np.uint8)
        cfg = Config()
        self._check(self.L.rbt_hip_upload(self.h, _p(model), model.size, C.byref(cfg)))
        return cfg

    def upload_file(self, path):
        cfg = Config()
        self._check(self.L.rbt_hip_upload_file(self.h, os.fsencode(path), C.byref(cfg)))
        return cfg

    def expert_stats(self):
        """{hits, misses, evictions, bytes_read, resident_bytes, capacity_bytes}"""
        a = (C.c_uint64 * 6)()
        self._check(self.L.rbt_hip_expert_stats(self.h, a))
        return dict(zip(("hits", "misses", "evictions", "bytes_read", "resident_bytes", "capacity_bytes"), a))

    def layer(self, l):
        L = MoeLayer()
        self._check(self.L.rbt_hip_layer(self.h, l, C.byref(L)))
        return L

    def moe(self, layer, xb, x=None):
        """Host-pointer MoE block of an uploaded model. Returns (x_out or None, routing)."""
        cfg_layer = self.layer(layer)
        xb = np.ascontiguousarray(xb, dtype=np.float32).reshape(-1, cfg_layer.dim)
        T = xb.shape[0]
        xo = None if x is None else np.array(x, dtype=np.float32).reshape(T, cfg_layer.dim)
        routing = np.zeros((T, cfg_layer.top_k), np.int32)
        self._check(self.L.rbt_hip_moe(self.h, layer, _p(xb), T, _p(xo), _p(routing)))
        return xo, routing

    def matvec(self, w_offset, x, rows):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(rows, np.float32)
        self._check(self.L.rbt_hip_matvec(self.h, _p(out), w_offset, _p(x), rows, x.size))
        return out

    # ---- full forward pass
    def model_create(self, cfg):
        """Allocates a model image of cfg's layout on the device; returns its base (c_void_p)."""
        p = C.c_void_p()
        self._check(self.L.rbt_hip_model_create(self.h, C.byref(cfg), C.byref(p)))
        self.model_base = p
        return p

    def tensor(self, name, layer=0):
        """(byte offset, bytes) of a tensor of the model image."""
        off, n = C.c_uint64(), C.c_uint64()
        self._check(self.L.rbt_hip_tensor(self.h, name.encode(), layer, C.byref(off), C.byref(n)))
        return off.value, n.value

    def state_init(self, ctx=0):
        self._check(self.L.rbt_hip_state_init(self.h, ctx))

    def forward(self, token, pos, vocab, n_layers, top_k):
        """forward(token, pos): (logits [vocab], routing [n_layers][top_k])."""
        logits = np.zeros(vocab, np.float32)
        routing = np.zeros((n_layers, top_k), np.int32)
        self._check(self.L.rbt_hip_forward(self.h, int(token), int(pos), _p(logits), _p(routing)))
        return logits, routing

    def set_sampling(self, temperature=0.0, top_k=0, top_p=1.0, seed=0):
        self._check(self.L.rbt_hip_set_sampling(self.h, temperature, top_k, top_p, seed))

    def batch_init(self, n_seq, ctx=0):
        self._check(self.L.rbt_hip_batch_init(self.h, n_seq, ctx))

    def forward_batch(self, tokens, pos, vocab, n_layers, top_k):
        """One step for every sequence: (logits [B][vocab], routing [n_layers][B][top_k])."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        pos = np.ascontiguousarray(pos, dtype=np.int32)
        B = tokens.size
        logits = np.zeros((B, vocab), np.float32)
        routing = np.zeros((n_layers, B, top_k), np.int32)
        self._check(self.L.rbt_hip_forward_batch(self.h, _p(tokens), _p(pos), _p(logits), _p(routing)))
        return logits, routing

    def generate_batch(self, prompts, n_gen):
        """Greedy --gen of every sequence: (ids [B][n_gen], [prompt ms, generation ms])."""
        prompts = np.ascontiguousarray(prompts, dtype=np.int32)
        B, n_prompt = prompts.shape
        out = np.zeros((B, max(n_gen, 1)), np.int32)
        ms = (C.c_double * 2)()
        self._check(self.L.rbt_hip_generate_batch(self.h, _p(prompts), n_prompt, int(n_gen), _p(out), ms))
        return out[:, :n_gen], (ms[0], ms[1])

    def generate(self, prompt, n_gen, eos=-1):
        """Greedy --gen loop on the device: (generated ids, [prompt ms, generation ms])."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(n_gen, 1), np.int32)
        n = C.c_int(0)
        ms = (C.c_double * 2)()
        self._check(self.L.rbt_hip_generate(self.h, _p(prompt), prompt.size, int(n_gen), int(eos), _p(out),
                                            C.byref(n), ms))
        return out[:n.value].tolist(), (ms[0], ms[1])

    def generate_stream(self, prompt, n_gen, eos=-1, stop_after=None):
        """The streaming --gen loop: (ids reported one by one through the callback, the ids of out,
        [prompt ms, generation ms]). stop_after: the callback returns 0 after that many ids."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(n_gen, 1), np.int32)
        n = C.c_int(0)
        ms = (C.c_double * 2)()
        seen = []

        def on_token(_user, tok):
            seen.append(int(tok))
            return 0 if stop_after is not None and len(seen) >= stop_after else 1

        fn = TOKEN_FN(on_token)
        self._check(self.L.rbt_hip_generate_stream(self.h, _p(prompt), prompt.size, int(n_gen), int(eos), fn, None,
                                                   _p(out), C.byref(n), ms))
        return seen, out[:n.value].tolist(), (ms[0], ms[1])

    def routing_history(self, seq, first_pos, n_pos, n_layers, top_k):
        out = np.zeros((max(n_pos, 1), n_layers, top_k), np.int32)
        self._check(self.L.rbt_hip_routing_history(self.h, seq, first_pos, n_pos, _p(out)))
        return out[:n_pos]

    # ---- device level
    def moe_dev(self, layer, xb, T, x=None, moe=None, routing=None, weights=None):
        vp = lambda b: None if b is None else (b if isinstance(b, C.c_void_p) else b.p)
        self._check(self.L.rbt_hip_moe_dev(self.h, C.byref(layer), vp(xb), T, vp(x), vp(moe), vp(routing),
                                           vp(weights)))

    def moe_dev_noalloc(self, layer, xb, T, x=None, moe=None, routing=None, weights=None):
        vp = lambda b: None if b is None else (b if isinstance(b, C.c_void_p) else b.p)
        self._check(self.L.rbt_hip_moe_dev_noalloc(self.h, C.byref(layer), vp(xb), T, vp(x), vp(moe), vp(routing),
                                                   vp(weights)))

    def reserve(self, layer, max_tokens):
        self._check(self.L.rbt_hip_reserve(self.h, C.byref(layer), max_tokens))

    def prefill_layout(self, layer=None):
        """The tiled copy of `layer`'s experts for the grouped GEMMs (None: every layer of the model)."""
        self._check(self.L.rbt_hip_prefill_layout(self.h, None if layer is None else C.byref(layer)))

    def prefill_layout_drop(self, layer=None):
        self._check(self.L.rbt_hip_prefill_layout_drop(self.h, None if layer is None else C.byref(layer)))

    def expert_counts(self, n_experts):
        p = self.L.rbt_hip_expert_counts_dev(self.h)
        if not p:
            return None
        out = np.empty(n_experts, np.int32)
        self._check(self.L.rbt_hip_d2h(self.h, _p(out), C.c_void_p(p), out.nbytes))
        return out

    def matvec_dev(self, out, W, dtype, x, rows, cols):
        self._check(self.L.rbt_hip_matvec_dev(self.h, out.p, W if isinstance(W, C.c_void_p) else W.p, dtype, x.p,
                                              rows, cols))


def profiler_attached():
    """True while a ROCm profiler tool is attached to this process (rbt_hip_profiler_attached): the
    library then refuses HIP graph replay, and so should a host that captures graphs of its own."""
    return bool(lib().rbt_hip_profiler_attached())


def expert_cache_replay(budget_bytes, expert_stride, routing, n_experts):
    """The engine's expert LRU replayed over routing [T][n_layers][top_k] (host only): the stats dict."""
    routing = np.ascontiguousarray(routing, dtype=np.int32)
    T, n_layers, top_k = routing.shape
    a = (C.c_uint64 * 6)()
    if not lib().rbt_hip_expert_cache_replay(budget_bytes, expert_stride, n_layers, n_experts, top_k, _p(routing), T, a):
        raise HipError(lib().rbt_hip_last_error(None).decode())
    return dict(zip(("hits", "misses", "evictions", "bytes_read", "resident_bytes", "capacity_bytes"), a))


def moe_layer_desc(dim, n_experts, top_k, hidden, dtype, norm_topk, router, experts, stride, bias=None):
    ptr = lambda b: None if b is None else (b.value if isinstance(b, C.c_void_p) else b.ptr)
    return MoeLayer(dim, n_experts, top_k, hidden, dtype, norm_topk, ptr(router), ptr(experts), stride, ptr(bias))
