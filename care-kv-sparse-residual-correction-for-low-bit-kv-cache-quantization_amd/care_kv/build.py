"""Build libcarekv_hip.so (HIP kernels for gfx950) in-tree with hipcc.

    python -m care_kv.build          (from the package directory)

The library is a plain C-ABI shared object loaded with ctypes; it links the
HIP runtime by SONAME, so inside a torch process it binds to the runtime
torch already loaded.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(ROOT, "csrc")
REPO = os.path.dirname(ROOT)
INCLUDE = os.path.join(REPO, "include")
LIB_NAME = "libcarekv_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["capi.cpp", "store.hip", "decode.hip", "decode_stream.hip", "decode_stream4.hip", "decode_proxy.hip", "decode_select.hip", "decode_apply.hip", "decode_apply4.hip", "prefill.hip", "prefill_rows.hip", "ops.hip"]
ARCH = os.environ.get("CAREKV_OFFLOAD_ARCH", "gfx950")
# Per-source options.  The apply pass's window loop waits on memory at four
# waves per SIMD; LLVM's iterative ILP scheduler interleaves its independent
# loads and arithmetic better (config 3 apply 158-162 -> 151-157 us, config 2
# 41.5 -> 37 us, no spill).  The other kernels measured the same or slower
# with it (the streaming kernel spills 16 B and loses 3%).
EXTRA_FLAGS = {"decode_apply4.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]}


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (set HIPCC)")


def common_flags():
    return ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-I", INCLUDE, "-I", CSRC,
            "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-fast-math", "-ffp-contract=off",
            "-mcode-object-version=5",
            # MFMA accumulators in VGPRs: avoids AGPR<->VGPR copies of the
            # loop-carried output tiles
            "-mllvm", "-amdgpu-mfma-vgpr-form=1",
            # packed FP32 ops disabled on purpose
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wno-unused-command-line-argument"]


def build(verbose: bool = False, jobs: int = 4) -> str:
    cc = hipcc()
    out_dir = os.path.join(ROOT, "_build")
    os.makedirs(out_dir, exist_ok=True)

    def compile_one(src):
        obj = os.path.join(out_dir, src + ".o")
        cmd = [cc, *common_flags(), *EXTRA_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
        if src.endswith(".hip"):
            cmd[1:1] = ["-x", "hip"]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [cc, "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
