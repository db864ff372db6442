"""Shared helpers for the parity tests: synthetic MoE layers and the comparison rules.

Comparison rules (the bar the HIP path is held to against the oracle, i.e. the engine's own fp32
CPU path, rabbit2/src/rabbit2.c:511-542):
  * routing: identical, except where the CPU's own probabilities of the two swapped experts are
    exactly equal (an exact tie; the engine then picks the lower index);
  * layer output: normwise max|gpu - cpu| / max|cpu| <= 1e-3 (MOE_RTOL).
"""
import numpy as np

from oracle import pyoracle as po

MOE_RTOL = 1e-3
X_STREAM = 0x5EED  # stream id of synthetic activations


def normwise_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    scale = np.max(np.abs(want))
    if scale == 0:
        return float(np.max(np.abs(got)))
    return float(np.max(np.abs(got - want)) / scale)


def routing_check(got, want, probs):
    """Returns (mismatched tokens, mismatches not explained by an exact CPU tie)."""
    got, want = np.asarray(got).reshape(want.shape), np.asarray(want)
    probs = np.asarray(probs).reshape(want.shape[0], -1)
    bad_tokens, unexplained = 0, 0
    for t in range(want.shape[0]):
        if np.array_equal(got[t], want[t]):
            continue
        bad_tokens += 1
        for g, w in zip(got[t], want[t]):
            if g != w and not (0 <= g < probs.shape[1] and probs[t, g] == probs[t, w]):
                unexplained += 1
    return bad_tokens, unexplained


class SynthLayer:
    """One MoE layer in .rbt2 storage format generated on the device (weights ~ N(0, w_scale) in
    dtype, expert e's streams as the oracle writer's layer 0), plus a host copy for the oracle."""

    def __init__(self, dev, dim, n_experts, top_k, hidden, dtype, norm_topk, seed, w_scale=0.02, fan_in=False,
                 bias=None, layer=0):
        self.dev = dev
        self.D, self.E, self.K, self.H = dim, n_experts, top_k, hidden
        self.dtype, self.norm_topk, self.seed = dtype, norm_topk, seed
        esz = po.ELEM[dtype]
        self.esz = esz
        self.stride = (3 * hidden * dim * esz + 4095) // 4096 * 4096
        cfg = po.Config(dim=dim, n_experts=n_experts, top_k=top_k, expert_hidden=hidden, dtype=dtype)
        self.router_dev = dev.malloc(n_experts * dim * esz)
        self.experts_dev = dev.malloc(n_experts * self.stride)
        dev.memset(self.experts_dev, 0)
        sc_d = w_scale / np.sqrt(dim) if fan_in else w_scale
        sc_h = w_scale / np.sqrt(hidden) if fan_in else w_scale
        dev.fill_normal(self.router_dev, dtype, n_experts * dim, seed, po.layer_stream(layer, 8), scale=sc_d)
        mat = hidden * dim
        for e in range(n_experts):
            base = e * self.stride
            dev.fill_normal(self.experts_dev, dtype, mat, seed, po.expert_stream(cfg, layer, e, 0), scale=sc_d,
                            byte_offset=base)
            dev.fill_normal(self.experts_dev, dtype, mat, seed, po.expert_stream(cfg, layer, e, 1), scale=sc_d,
                            byte_offset=base + mat * esz)
            dev.fill_normal(self.experts_dev, dtype, mat, seed, po.expert_stream(cfg, layer, e, 2), scale=sc_h,
                            byte_offset=base + 2 * mat * esz)
        self.scales = (sc_d, sc_d, sc_h)
        st = np.uint16 if dtype == po.DT_BF16 else np.float32
        self.router = dev.d2h(self.router_dev, (n_experts, dim), st)
        self.experts = dev.d2h(self.experts_dev, (n_experts * self.stride,), np.uint8)
        self.bias = None if bias is None else np.asarray(bias, np.float32)
        self.bias_dev = None if bias is None else dev.upload_array(self.bias)

    def reseed_experts(self, experts, seed):
        """Rewrites the blobs of the given experts with weights of another seed (device and host copy)."""
        cfg = po.Config(dim=self.D, n_experts=self.E, top_k=self.K, expert_hidden=self.H, dtype=self.dtype)
        mat = self.H * self.D
        for e in experts:
            for w in range(3):
                self.dev.fill_normal(self.experts_dev, self.dtype, mat, seed, po.expert_stream(cfg, 0, e, w),
                                     scale=self.scales[w], byte_offset=e * self.stride + w * mat * self.esz)
        self.experts = self.dev.d2h(self.experts_dev, (self.E * self.stride,), np.uint8)

    def desc(self):
        from rabbitm2_amd.hip import moe_layer_desc
        return moe_layer_desc(self.D, self.E, self.K, self.H, self.dtype, self.norm_topk, self.router_dev,
                              self.experts_dev, self.stride, self.bias_dev)

    def make_x(self, T, seed, bf16=True):
        """T activations ~N(0,1); bf16-representable values stored as f32 when bf16 is set."""
        dt = po.DT_BF16 if bf16 else po.DT_F32
        raw = po.fill_normal(T * self.D, dt, seed, X_STREAM)
        x = po.bf16_to_f32(raw) if bf16 else raw
        return x.reshape(T, self.D).astype(np.float32)

    def oracle(self, xb, order, x=None):
        return po.moe_layer(self.D, self.E, self.K, self.H, self.dtype, self.norm_topk, self.router, self.experts,
                            self.stride, xb, order=order, bias=self.bias, x=x)

    def run_gpu(self, xb, x=None):
        """HIP path through rbt_hip_moe_dev. Returns dict(moe, routing, weights[, x])."""
        dev = self.dev
        xb = np.ascontiguousarray(xb, np.float32)
        T = xb.shape[0]
        xb_d = dev.upload_array(xb) if T else dev.malloc(4)
        moe_d = dev.malloc(max(T * self.D * 4, 4))
        rt_d = dev.malloc(max(T * self.K * 4, 4))
        wt_d = dev.malloc(max(T * self.K * 4, 4))
        x_d = None if x is None else dev.upload_array(np.asarray(x, np.float32))
        dev.moe_dev(self.desc(), xb_d, T, x=x_d, moe=moe_d, routing=rt_d, weights=wt_d)
        dev.synchronize()
        out = dict(moe=dev.d2h(moe_d, (T, self.D), np.float32), routing=dev.d2h(rt_d, (T, self.K), np.int32),
                   weights=dev.d2h(wt_d, (T, self.K), np.float32))
        if x_d is not None:
            out["x"] = dev.d2h(x_d, (T, self.D), np.float32)
            dev.free(x_d)
        for b in (xb_d, moe_d, rt_d, wt_d):
            dev.free(b)
        return out

    def close(self):
        for b in (self.router_dev, self.experts_dev, self.bias_dev):
            if b is not None:
                self.dev.free(b)
