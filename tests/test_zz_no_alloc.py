"""rbt_hip_moe_dev_noalloc: the MoE block on the library's per-GPU scratch array instead of the handle's
workspace. Against rbt_hip_moe_dev on the same inputs, through the C ABI: outputs, routing, combine
weights and the tokens-per-expert histogram bit for bit (same kernels), and the oracle's bar (routing
identical except at exact ties, normwise error <= 1e-3). Two calls in a row, the second smaller than
the first; a call whose workspace exceeds the array fails with a message; device memory in use does not
change across the calls.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import pyoracle as po
from tests.common import MOE_RTOL, SynthLayer, normwise_err, routing_check

pytestmark = pytest.mark.gpu

D, E, K, H = 2048, 64, 8, 1024  # the OLMoE layer


def mem_in_use():
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return total.value - free.value


def run(dev, layer, xb, x, noalloc):
    T = xb.shape[0]
    xb_d, x_d = dev.upload_array(xb), dev.upload_array(x)
    moe_d, rt_d, wt_d = dev.malloc(T * D * 4), dev.malloc(T * K * 4), dev.malloc(T * K * 4)
    before = mem_in_use()
    call = dev.moe_dev_noalloc if noalloc else dev.moe_dev
    call(layer.desc(), xb_d, T, x=x_d, moe=moe_d, routing=rt_d, weights=wt_d)
    dev.synchronize()
    grew = mem_in_use() - before
    out = dict(moe=dev.d2h(moe_d, (T, D), np.float32), x=dev.d2h(x_d, (T, D), np.float32),
               routing=dev.d2h(rt_d, (T, K), np.int32), weights=dev.d2h(wt_d, (T, K), np.float32))
    counts = dev.expert_counts(E)
    out["counts"] = None if counts is None else counts.copy()
    for b in (xb_d, x_d, moe_d, rt_d, wt_d):
        dev.free(b)
    return out, grew


def test_noalloc_matches_the_workspace_path(dev):
    """The workspace path first (it also takes each kernel's first launch, when the runtime may set memory
    aside), then the no-alloc calls back to back, largest first: each must leave the device memory in use
    unchanged and reproduce the workspace path bit for bit."""
    dev.set_router_order(po.ORDER_AVX2)
    layer = SynthLayer(dev, D, E, K, H, po.DT_BF16, 1, seed=5)
    rng = np.random.default_rng(3)
    cases = []
    for T in (300, 1, 5):  # grouped GEMMs, then the batch-1 kernels, then the per-pair GEMVs
        xb = layer.make_x(T, seed=10 + T)
        x = rng.standard_normal((T, D)).astype(np.float32)
        want, _ = run(dev, layer, xb, x, noalloc=False)
        cases.append((T, xb, x, want))
    for T, xb, x, want in cases:
        print(f"noalloc: T = {T}", flush=True)
        got, grew = run(dev, layer, xb, x, noalloc=True)
        assert grew == 0, f"T = {T}: device memory in use grew by {grew} bytes"
        for k in ("moe", "x", "routing", "weights"):
            assert got[k].tobytes() == want[k].tobytes(), (T, k)
        if T == 300:
            assert got["counts"] is not None and np.array_equal(got["counts"], want["counts"])
            assert int(got["counts"].sum()) == T * K
        ref = layer.oracle(xb, po.ORDER_AVX2, x=x)
        bad, unexplained = routing_check(got["routing"], ref["routing"], ref["probs"])
        assert unexplained == 0, (T, bad)
        assert normwise_err(got["moe"], ref["moe"]) <= MOE_RTOL
        assert normwise_err(got["x"] - x, ref["x"] - x) <= MOE_RTOL
    layer.close()


def test_noalloc_rejects_calls_beyond_its_scratch(dev):
    from rabbitm2_amd.hip import HipError
    layer = SynthLayer(dev, D, E, K, H, po.DT_BF16, 1, seed=6)
    T = 1024  # 104 MiB of workspace at this shape
    xb_d, moe_d = dev.malloc(T * D * 4), dev.malloc(T * D * 4)
    with pytest.raises(HipError, match="bytes of scratch"):
        dev.moe_dev_noalloc(layer.desc(), xb_d, T, moe=moe_d)
    dev.moe_dev_noalloc(layer.desc(), xb_d, 0, moe=moe_d)  # an empty batch is a no-op
    for b in (xb_d, moe_d):
        dev.free(b)
    layer.close()
