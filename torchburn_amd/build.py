"""Build libtbhip.so (all HIP sources under csrc/) for gfx950 with hipcc.

Run as ``python -m torchburn_amd.build``.  Objects go to csrc/_build/ and the
library to torchburn_amd/libtbhip.so, in-tree, so it travels with the source
tree to the GPU box.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(CSRC, "_build")
LIB = os.path.join(PKG, "libtbhip.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-fvisibility=hidden", "-Wall", "-Wno-unused-function",
    # Packed FP32 VALU forms stay off in every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libtbhip.so)")


# Host-side sanitizer build (tests/run_sanitized.sh): AddressSanitizer and
# UndefinedBehaviorSanitizer on the host code only -- each flag behind
# -Xarch_host, so the gfx950 device code is built exactly as in the product.
HOST_SANITIZE_FLAGS = [
    "-g", "-Xarch_host", "-fno-omit-frame-pointer",
    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
]


# Per-source extra flags.  w4_limb: MFMA results in VGPRs (the kernel scales
# every result with VALU; accumulators in AGPRs would cost a copy each).
EXTRA_FLAGS = {
    "w4_limb.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: str, build_dir: str = BUILD, host_sanitize: bool = False) -> str:
    obj = os.path.join(build_dir, os.path.basename(src) + ".o")
    extra = EXTRA_FLAGS.get(os.path.basename(src), [])
    if host_sanitize:
        extra = extra + HOST_SANITIZE_FLAGS
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, "-I", os.path.join(PKG, ".."), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False, out: str = LIB, host_sanitize: bool = False) -> str:
    """Builds the library into `out`.  host_sanitize: the sanitizer build of the
    host code (objects in csrc/_build_san/; load it with the sanitizer runtime
    preloaded, as tests/run_sanitized.sh does)."""
    build_dir = BUILD + "_san" if host_sanitize else BUILD
    os.makedirs(build_dir, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, build_dir, host_sanitize), srcs))
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(srcs)} sources")
    return out


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "--host-sanitize":
        build(verbose=True, out=os.path.abspath(sys.argv[2]), host_sanitize=True)
    else:
        build(verbose=True)
    sys.exit(0)
