"""Builds librbt2_hip.so (the C-ABI of include/rbt2_hip.h) for gfx950 with hipcc, in-tree, and the
engine's command line over it (rabbitm2_amd/rabbit2, C99, from host/rabbit2_main.c).

    python -m rabbitm2_amd.build          # or rabbitm2_amd.build.build()

Every .hip under csrc/ is compiled to an object in _build/ (in parallel) and linked into
rabbitm2_amd/librbt2_hip.so. Always recompiles: the driver uses this as its "does it build" check.
"""
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "librbt2_hip.so")
CLI = os.path.join(PKG, "rabbit2")
CLI_SRC = os.path.join(PKG, "host", "rabbit2_main.c")
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-Wall", "-Wno-unused-result",
    # m0 is set inside the one asm block that uses it (direct-to-LDS copies in prefill.hip)
    "-Wno-inline-asm",
    # Packed fp32 arithmetic stays off: hipcc would otherwise emit v_pk_* f32 forms by itself.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(os.path.basename(src))[0] + ".o")
    cmd = [hipcc()] + HIPCC_FLAGS + ["-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    return obj, "\n".join(noise)


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_compile, srcs))
    for obj, noise in results:
        if noise and verbose:
            print(noise, file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + [o for o, _ in results]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    build_cli()
    return LIB


def build_cli():
    """The engine's CLI: plain C99 linked against the library (found next to it at run time)."""
    cc = os.environ.get("CC") or shutil.which("gcc") or shutil.which("cc")
    if not cc:
        raise RuntimeError("no C compiler found for the rabbit2 command line")
    tmp = CLI + ".tmp"
    cmd = [cc, "-O2", "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"), CLI_SRC,
           "-L", PKG, "-lrbt2_hip", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building the rabbit2 command line failed:\n{res.stderr}")
    os.replace(tmp, CLI)
    return CLI


if __name__ == "__main__":
    print(build(verbose=True))
