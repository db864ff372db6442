"""The C ABI library itself, on the CPU: it is built, it loads, and it exports every entry point
include/rbt2_hip.h declares. No device work is started here."""
import ctypes
import os
import re
import subprocess

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
