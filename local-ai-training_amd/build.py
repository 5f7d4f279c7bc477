"""Build libratchet_hip.so (gfx950) from csrc/*.hip, and libratchet_torch.so (the
torch.ops.ratchet operators over it) from csrc/ratchet_torch_ops.cpp.

    python local-ai-training_amd/build.py [--jobs N]

Every HIP source is compiled with hipcc for gfx950 only. Flags that matter for
numerics: -ffp-contract=off (no fused multiply-add contraction: every fp32 op is
separately rounded, as the bit-exact parity contract requires) and no fast-math
(hipcc's default correctly rounded fp32 divide and square root stay on).
Packed-fp32 instruction selection is disabled for the device code.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = REPO / "include"
BUILD_DIR = HERE / "_build"
LIB = HERE / "local_ai_training" / "libratchet_hip.so"
OPS_LIB = HERE / "local_ai_training" / "libratchet_torch.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libratchet_hip.so)")


# Per-source flags. rk_attention.hip: MFMA results in VGPRs (the attention's softmax and
# output rescale read every accumulator with VALU instructions; in AGPRs each read and write
# back is an extra copy, about as many instructions as the softmax itself).
SOURCE_FLAGS = {
    "rk_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o",
           str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{proc.stdout}\n{proc.stderr}")
    return obj


def _torch_paths() -> tuple[list[str], str]:
    """Include directories and the library directory of the installed torch (ROCm build)."""
    from torch.utils import cpp_extension

    return cpp_extension.include_paths(), cpp_extension.library_paths()[0]


def build_torch_ops(verbose: bool = False) -> Path:
    """libratchet_torch.so: the torch.ops.ratchet.* registrations (host C++ only, compiled
    with g++ against torch's headers) over libratchet_hip.so, found next to it at run time."""
    includes, torch_lib = _torch_paths()
    rocm = Path(hipcc()).resolve().parent.parent
    tmp = OPS_LIB.with_suffix(".so.tmp")
    cmd = [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-Wall", "-Wno-unused-function",
        *[f"-I{p}" for p in includes], f"-I{rocm / 'include'}", f"-I{INCLUDE}",
        str(CSRC / "ratchet_torch_ops.cpp"), "-o", str(tmp),
        f"-L{LIB.parent}", "-lratchet_hip", "-Wl,-rpath,$ORIGIN",
        f"-L{torch_lib}", "-lc10", "-ltorch_cpu", "-lc10_hip", "-ltorch_hip",
        f"-Wl,-rpath,{torch_lib}",
    ]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"torch op library failed\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, OPS_LIB)
    if verbose:
        print(f"built {OPS_LIB}", flush=True)
    return OPS_LIB


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), os.cpu_count() or 4, 16)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources", flush=True)
    build_torch_ops(verbose)
    return LIB


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--jobs", type=int, default=None)
    args = parser.parse_args()
    try:
        build(args.jobs, verbose=True)
    except RuntimeError as error:
        print(error, file=sys.stderr)
        sys.exit(1)
