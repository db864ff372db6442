"""The C ABI library itself, on the CPU: it is built, it loads, and it exports every entry point
include/rbt2_hip.h declares. No device work is started here."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

from rabbitm2_amd import hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "rbt2_hip.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rbt_hip_\w+)\s*\(", text)))


def test_header_declarations_match_python_view():
    assert declared() == sorted(hip.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = hip.lib()
    for name in declared():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", hip.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\bT (rbt_hip_\w+)", out.stdout))
    assert set(declared()) <= exported


def test_header_compiles_as_c99():
    src = '#include "rbt2_hip.h"\nint main(void){ rbt_hip *h = 0; (void)h; return 0; }\n'
    res = subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
                          "-fsyntax-only", "-x", "c", "-"], input=src, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr


def test_null_handle_calls_fail_cleanly():
    lib = hip.lib()
    assert lib.rbt_hip_synchronize(None) == 0
    assert b"NULL" in lib.rbt_hip_last_error(None)
    assert lib.rbt_hip_moe_dev(None, None, None, 1, None, None, None, None) == 0
    assert lib.rbt_hip_stream(None) is None


def test_init_without_a_device_reports_an_error():
    import torch  # device count only; does not initialise HIP on this image
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present")
    h = ctypes.c_void_p()
    assert hip.lib().rbt_hip_init(ctypes.byref(h), 0) == 0
    assert b"no HIP device" in hip.lib().rbt_hip_last_error(None) or b"init" in hip.lib().rbt_hip_last_error(None)


PROFILER_VARS = ("ROCPROFILER_LIBRARY_CTOR", "ROCPROF_OUTPUT_PATH", "HSA_TOOLS_LIB", "ROCP_TOOL_LIB")


def _attached_in_child(extra_env):
    """rbt_hip_profiler_attached() in a fresh process whose environment is ours without any profiler
    variable, plus extra_env (the library reads the variables when asked, no device is touched)."""
    env = {k: v for k, v in os.environ.items() if k not in PROFILER_VARS}
    env.update(extra_env)
    code = ("import ctypes, sys; L = ctypes.CDLL(sys.argv[1]); print(L.rbt_hip_profiler_attached())")
    out = subprocess.run([sys.executable, "-c", code, hip.LIB_PATH], env=env, capture_output=True, text=True,
                         check=True)
    return int(out.stdout.strip())


@pytest.mark.parametrize("var", PROFILER_VARS)
def test_profiler_detection(var):
    assert _attached_in_child({}) == 0
    assert _attached_in_child({var: "1"}) == 1
    assert _attached_in_child({var: ""}) == 0  # set but empty: no tool


def test_bench_refuses_graph_replay_under_a_profiler():
    """bench.py's graph-replayed legs exit non-zero with a message when a profiler tool is attached,
    before anything touches a device."""
    env = {k: v for k, v in os.environ.items() if k not in PROFILER_VARS}
    env["ROCPROF_OUTPUT_PATH"] = "/tmp/unused"
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--no-cpu"], env=env, capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 2
    assert "profiler" in res.stderr and "--profile-" in res.stderr


@pytest.mark.parametrize("args,msg", [(["--gpus", "2"], "one GPU only"), (["--steps", "0"], "--steps must be")])
def test_bench_refuses_what_it_does_not_measure(args, msg):
    """More than one GPU (the sharded layer is a design note) and a non-positive step count end the bench
    with a message before anything touches a device."""
    env = {k: v for k, v in os.environ.items() if k not in PROFILER_VARS}
    res = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + args, env=env, capture_output=True,
                         text=True, timeout=120)
    assert res.returncode != 0
    assert msg in res.stderr
