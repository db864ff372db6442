"""Failure paths of the C ABI, forced from the host: with RBT_HIP_FAULT="<kind>:<n>" the library reports
its n-th HIP call of that kind (device allocation, kernel launch, copy, wait) as failed without making
it, so no kernel ever faults. Every entry point must then keep the engine's convention (int 0 + a
message on stderr, rabbit2/src/rabbit2.c:199-228, :533, :705-709 -> exit code 1) and leave the handle
usable: a failed upload leaves no model, a failed step leaves the model and state to run again.

Each case runs in a child process (the plan is read once per process), one at a time.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

from oracle import pyoracle as po

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "rabbitm2_amd", "rabbit2")
GOLDEN = os.path.join(ROOT, "tests", "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))["cases"]

CHILD = r"""
import json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from oracle import pyoracle as po
from rabbitm2_amd.hip import Device, HipError
spec = json.loads(sys.argv[2])
cfg = po.Config(**spec["config"])
g = spec["gen_params"]
model = po.build_model(cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                         emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
tokens = [int(t) for t in json.loads(sys.argv[3])]
res = {}
def attempt(name, fn):
    try:
        res[name] = ["ok", fn()]
    except HipError as e:
        res[name] = ["error", str(e)]
    return res[name][0] == "ok"
with Device(0) as dev:
    dev.set_router_order(po.ORDER_AVX2)
    def fwd0():
        logits, routing = dev.forward(tokens[0], 0, cfg.vocab, cfg.n_layers, cfg.top_k)
        return routing.tolist()
    steps = [("upload", lambda: dev.upload(model) and None), ("state_init", lambda: dev.state_init(0)),
             ("forward0", fwd0), ("generate", lambda: dev.generate(np.array(tokens, np.int32), spec["n_gen"])[0])]
    for name, fn in steps:  # every step that failed once is run again
        if not attempt(name, fn):
            if name == "upload":
                attempt("forward_without_model", fwd0)
            attempt(name + "_retry", fn)
print("RESULT " + json.dumps(res), flush=True)
"""


def run_child(fault, case="ref_bf16"):
    spec = MANIFEST[case]
    fx = np.load(os.path.join(GOLDEN, case + ".npz"))
    env = dict(os.environ, RBT_HIP_FAULT=fault)
    print(f"child with RBT_HIP_FAULT={fault}", flush=True)
    res = subprocess.run([sys.executable, "-c", CHILD, ROOT, json.dumps(spec), json.dumps(fx["tokens"].tolist())],
                         capture_output=True, text=True, env=env, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    line = [ln for ln in res.stdout.splitlines() if ln.startswith("RESULT ")][-1]
    return json.loads(line[7:]), res.stderr, fx


def check_recovered(res, fx, failed_step, text):
    """Exactly `failed_step` failed, naming `text`; its retry and every later step match the reference."""
    failed = [k for k, v in res.items() if v[0] == "error" and k != "forward_without_model"]
    assert failed == [failed_step], res
    assert text in res[failed_step][1], res[failed_step]
    want = {"upload": None, "state_init": None, "forward0": fx["routing_avx2"][0].tolist(),
            "generate": fx["gen_avx2"].tolist()}
    for name, value in want.items():
        key = name + "_retry" if name == failed_step else name
        assert res[key] == ["ok", value], (key, res[key])


def test_failed_device_allocation_at_upload():
    res, err, fx = run_child("malloc:1")
    check_recovered(res, fx, "upload", "out of memory")
    assert "hipMalloc" in res["upload"][1]
    assert "RBT_HIP_FAULT" in err and "rbt2_hip: hipMalloc" in err  # the message also goes to stderr
    assert res["forward_without_model"][0] == "error"  # no model, no state: a clean refusal


def test_failed_copy_at_upload():
    res, err, fx = run_child("copy:1")
    check_recovered(res, fx, "upload", "hipMemcpy")
    assert res["forward_without_model"][0] == "error"


@pytest.mark.parametrize("nth", [1, 7])
def test_failed_launch_in_a_forward_step(nth):
    """The n-th kernel launch of the process fails inside the first forward() (the embedding, a layer's
    attention): that call returns 0 with the launch named; the next call at the same position runs the
    whole step and matches the reference."""
    res, err, fx = run_child(f"launch:{nth}")
    check_recovered(res, fx, "forward0", "launch_")


@pytest.mark.parametrize("nth", [1, 2, 3, 5])
def test_failed_wait(nth):
    """The n-th stream or event wait of the process fails (during the upload, the state set-up, a
    forward or the generate loop): that call alone fails with the wait named, and running it again
    succeeds."""
    res, err, fx = run_child(f"sync:{nth}")
    failed = [k for k, v in res.items() if v[0] == "error" and k != "forward_without_model"]
    assert len(failed) == 1, res
    check_recovered(res, fx, failed[0], "Synchronize")


def test_cli_exits_1_with_the_message(tmp_path):
    spec = MANIFEST["ref_bf16"]
    cfg = po.Config(**spec["config"])
    g = spec["gen_params"]
    path = tmp_path / "m.rbt2"
    po.write_model(str(path), cfg, po.GenParams(seed=g["seed"], w_scale=g["w_scale"], fan_in_scale=g["fan_in_scale"],
                                                emb_scale=g["emb_scale"], norm_jitter=g["norm_jitter"]))
    fx = np.load(os.path.join(GOLDEN, "ref_bf16.npz"))
    toks = [str(int(t)) for t in fx["tokens"]]
    for fault, what in (("malloc:1", "hipMalloc"), ("launch:3", "launch_"), ("copy:2", "hipMemcpy")):
        res = subprocess.run([CLI, str(path), "--gen", "4"] + toks, capture_output=True, text=True, timeout=120,
                             env=dict(os.environ, RBT_HIP_FAULT=fault))
        assert res.returncode == 1 and what in res.stderr, (fault, res.returncode, res.stderr)
    res = subprocess.run([CLI, str(path), "--gen", "4"] + toks, capture_output=True, text=True, timeout=120)
    assert res.returncode == 0 and [int(t) for t in res.stdout.split()] == fx["gen_scalar"][:4].tolist()
