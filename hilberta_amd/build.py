"""Build libhilberta_hip.so (gfx950) in-tree with hipcc.

    python -m hilberta_amd.build          # compile every csrc/*.hip, link the shared library

Objects go to hilberta_amd/_build/, the library to hilberta_amd/libhilberta_hip.so; both are
git-ignored and travel with the source tree to the GPU box.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "_build"
LIB = PKG / "libhilberta_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    "-Wno-unused-lambda-capture",
    # packed fp32 VALU ops stay off: the compiler must not emit v_pk_{add,mul,fma}_f32
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build")


# Per-file flags.  attention.hip: no atomic optimizer.  Its atomics are single-lane work-queue
# claims; the optimizer turns each into a wave-aggregated atomic that reads its result back (and
# so waits for the round trip) right after issue, where the kernel means to overlap it with a step.
FILE_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]}


def _compile(src: Path) -> Path:
    obj = OUT / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    OUT.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    # a kernel whose host-side launch stub was not emitted links fine but cannot be loaded
    undefined = subprocess.run(["nm", "-D", "--undefined-only", str(tmp)], capture_output=True,
                               text=True).stdout
    stubs = [line.split()[-1] for line in undefined.splitlines() if "__device_stub__" in line]
    if stubs:
        raise RuntimeError(f"link left {len(stubs)} kernel launch stubs undefined, e.g. {stubs[0]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build()
