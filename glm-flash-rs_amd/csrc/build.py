"""Build libgfr_moe.so (gfx950) in-tree with hipcc: every kernel family plus the C ABI in one shared library."""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
SOURCES = ["grouping.hip", "exl3_decode.hip", "exl3_prefill.hip", "router.hip", "gfr_moe_api.hip", "prepared.hip", "prefetch.hip",
           "shared_fp8.hip"]
LIB = os.path.join(PKG, "libgfr_moe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _obj(src):
    return os.path.join(PKG, "_build", src.replace(".hip", ".o"))


def _compile(src):
    out = _obj(src)
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(HERE, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{errs}")
    return errs


def build(verbose=False):
    os.makedirs(os.path.join(PKG, "_build"), exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        logs = list(ex.map(_compile, SOURCES))
    if verbose:
        for l in logs:
            if l:
                print(l)
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", LIB, *[_obj(s) for s in SOURCES],
           "-L/opt/rocm/lib", "-lrocblas"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
