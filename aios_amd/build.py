"""Build recipe for libaios_attn.so (gfx950 HIP kernels + C ABI).

Run ``python -m aios_amd.build`` (or ``__graft_entry__.build()``).  Every
``csrc/*.hip`` file is compiled with hipcc for gfx950 into an object file in
``aios_amd/_build/`` and the objects are linked into ``aios_amd/libaios_attn.so``.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libaios_attn.so"
LIB_PATH = PKG_DIR / LIB_NAME
INCLUDE_DIR = PKG_DIR.parent / "include"

ARCH = os.environ.get("AIOS_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Keep the compiler from forming packed-fp32 (v_pk_*_f32) instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast",
    "-Wall",
    "-Wno-unused-variable",
    "-Wno-unused-function",
    # Kernel-argument preloading: the leading scalar arguments of a kernel
    # arrive in SGPRs at wave start instead of through a load from the
    # kernel-argument segment (the code object keeps a prologue that loads
    # them for firmware without the feature).
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 HIP backend cannot be built")


# Per-source flags: LLVM's max-ILP machine scheduler instead of the default
# occupancy-driven one for the short, latency-bound kernels.  The decode
# combine: graph-replayed long-context decode step 429.4-431.1 -> 422.8-423.6
# us (three alternating rounds on one box).  The model-side ops, depth mixer,
# sampler, step preparation and KV append: every CandidateGroup leg's
# replayed step 0.1-1.1% shorter (two rounds, both orders).  The decode main
# kernel (8.50 -> 8.61 us) and the prefill measured slower with it and keep
# the default.
_MAX_ILP = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
SOURCE_FLAGS = {
    name: _MAX_ILP
    for name in ("attn_combine.hip", "gemm_skinny.hip", "model_ops.hip", "attnres.hip",
                 "sampling.hip", "cg_state.hip", "kv_append.hip")
}


def _compile(hipcc: str, src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), f"-I{INCLUDE_DIR}", "-c",
           str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    # The host pass warns that it does not know the packed-fp32 feature.
    noise = "is not a recognized feature for this target"
    rest = [ln for ln in proc.stderr.splitlines() if noise not in ln and ln.strip()]
    if rest:
        sys.stderr.write("\n".join(rest) + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libaios_attn.so."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources for {ARCH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
