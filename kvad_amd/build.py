"""Build libkvad_hip.so for gfx950 in-tree (kvad_amd/libkvad_hip.so).

The library is plain hipcc output: every .hip under kvad_amd/csrc is compiled
to an object and linked with -shared.  No torch extension machinery is used;
the ABI is include/kvad_hip.h.

Flags that matter for parity:
  -ffp-contract=off                  products are rounded before they are
                                     added, as the reference (Rust) does
  -fhip-fp32-correctly-rounded-divide-sqrt
                                     amax/127 and 1/scale round as on the CPU
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                     no packed-FP32 instructions (they have
                                     given wrong results on these boxes)
  -mllvm -amdgpu-mfma-vgpr-form      matrix-core results land in VGPRs, where
                                     the scaling epilogues read them (the
                                     default parks them in AGPRs and copies
                                     every value out: one more VALU op each)
  -mllvm -amdgpu-kernarg-preload-count=14
                                     a kernel's first fourteen argument
                                     words arrive in scalar registers (the
                                     GEMV's job index and its first job's
                                     pointers and sizes), no load round trip;
                                     code objects keep a preamble that loads
                                     them where the firmware does not preload
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OBJ = HERE / "_obj"
LIB = HERE / "libkvad_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("KVAD_HIP_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
    "-Wall",
    "-Wno-unused-function",
]


def _compile(src: Path) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass warns that packed-fp32-ops is unknown to it; drop that.
    noise = "is not a recognized feature for this target"
    rest = "\n".join(l for l in res.stderr.splitlines() if noise not in l and l.strip())
    if rest:
        print(f"[{src.name}] {rest}", file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build()
