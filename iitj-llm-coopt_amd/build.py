"""Build recipe for libcoopt_amd.so: hipcc, gfx950 only, one object per csrc/*.hip.

    python -m iitj_llm_coopt_amd.build        (or __graft_entry__.build())

The library is written in-tree next to this file so that it travels with the repository
snapshot; it is loaded with ctypes after `import torch`, which makes it bind to the HIP
runtime torch already loaded.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libcoopt_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

SOURCES = ["abi.hip", "kv_cache.hip", "kv_blocks.hip", "accept.hip", "verify_attn.hip", "fused.hip",
           "linear.hip", "spec_step.hip"]

ARCH = "gfx950"
# -packed-fp32-ops: keep hipcc from forming packed fp32 VALU ops (the pool's known hazard).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the first 16 dwords of a kernel's scalar arguments arrive in SGPRs, so a kernel's first
    # loads do not wait for a kernel-argument load (a compatibility prologue loads them where
    # the firmware does not preload)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libcoopt_amd.so)")


def _compile(src: str, extra) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected.
    noise = ("packed-fp32-ops", "is not a recognized feature")
    lines = [ln for ln in res.stderr.splitlines() if ln.strip() and not any(n in ln for n in noise)]
    if lines:
        sys.stderr.write(f"[build] {src}:\n" + "\n".join(lines) + "\n")
    return obj


def build(verbose: bool = False, extra_flags=()) -> str:
    """Compile every csrc/*.hip for gfx950 and link LIB_PATH. Always recompiles."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    jobs = min(len(SOURCES), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, list(extra_flags)), SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[build] {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
