"""Compile the hi-rocm HIP library in-tree (``hi_amd/libhi_rocm.so``) for gfx950."""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libhi_rocm.so")
SOURCES = ["sampler_rows.hip", "sampler_select.hip", "sampler_fused.hip", "sampler_chunked.hip", "lm_head.hip", "sampler_debug.hip",
           "index_select.hip", "sampler_api.hip", "sampler_host.hip", "decode_step.hip",
           "moe_router.hip", "spec_verify.hip"]

# -ffp-contract=off: every f32/f64 operation that decides a token is a
# separate IEEE rounding (fused operations are written out explicitly).
# -packed-fp32-ops off: no v_pk_*_f32 instructions.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # leading scalar kernel arguments arrive in SGPRs at wave launch
    "-mllvm", "-amdgpu-kernarg-preload-count=8",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the hi-rocm HIP library cannot be built")


def build(verbose: bool = False, only=None) -> str:
    """Compile every HIP source and link libhi_rocm.so; returns its path.

    `only` (a list of source names) recompiles just those and links them with
    the objects of an earlier build of the others."""
    cc = hipcc()
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    def compile_one(src):
        obj = os.path.join(build_dir, src.replace(".hip", ".o"))
        cmd = [cc, *HIPCC_FLAGS, "-I", os.path.join(ROOT, "include"), "-I", CSRC, "-c",
               os.path.join(CSRC, src), "-o", obj]
        return src, obj, subprocess.run(cmd, capture_output=True, text=True)

    # the sources compile independently: one hipcc process each, at once
    todo = SOURCES if only is None else [s for s in SOURCES if s in only]
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(SOURCES)) as pool:
        results = list(pool.map(compile_one, todo))
    for src, obj, res in results:
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
        if verbose and res.stderr.strip():
            print(res.stderr)
    objs = [os.path.join(build_dir, src.replace(".hip", ".o")) for src in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
