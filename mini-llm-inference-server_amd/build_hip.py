"""Builds libminillm_hip.so (the gfx950 HIP kernels behind include/minillm_hip.h) in-tree.

    python build_hip.py            # from this directory, or
    python -c "import build_hip; build_hip.build()"

Each csrc/*.hip is compiled by hipcc for --offload-arch=gfx950 in parallel, then linked into
minillm/_lib/libminillm_hip.so.  The packed-FP32 feature is switched off for device code.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
OUT_DIR = HERE / "minillm" / "_lib"
LIB_NAME = "libminillm_hip.so"
ARCH = os.environ.get("MLLM_OFFLOAD_ARCH", "gfx950")

# no packed FP32 in any kernel
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# MFMA accumulators in VGPRs (the unified register file) rather than AGPRs keeps the attention loops
# free of accumulator copies between the two register halves
FILE_FLAGS = {name: ["-mllvm", "-amdgpu-mfma-vgpr-form=1"] for name in ("decode.hip", "prefill.hip")}
# inline-asm diagnostics (e.g. a clobber of a reserved register such as m0) fail the build
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", f"-I{INCLUDE}", f"-I{CSRC}", "-Wall",
                "-Wno-unused-function", "-Werror=inline-asm"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in res.stderr.splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip and link the shared library; returns its path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    obj_dir = HERE / "_build"
    obj_dir.mkdir(exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    objs = [obj_dir / (s.stem + ".o") for s in sources]
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(sources))) as ex:
        list(ex.map(_compile, sources, objs))
    out = OUT_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build())
