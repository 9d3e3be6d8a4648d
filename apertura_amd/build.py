"""Build libesda.so (HIP, gfx950) in-tree with hipcc.

Every HIP source is compiled with packed-FP32 instructions disabled (the compiler
would otherwise form v_pk_*_f32 from ordinary float code) and the AMDGPU iterative-ILP
instruction scheduler.  The host pass prints a
harmless warning that it does not know that feature.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libesda.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", os.path.join(ROCM, "bin", "hipcc"))
CXX = os.environ.get("CXX", "g++")

SOURCES = [
    "esda_decode.hip",
    "esda_prefill.hip",
    "es/ESKVCache.cpp",
    "es/ESDecodeAttn.cpp",
    "es/ESSnapshot.cpp",
    "es/safetensors.cpp",
    "es/ESPrefillAttn.cpp",
    "es/es_capi.cpp",
]

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # The default scheduler serialises the attend loop's LDS reads behind their uses when
    # the loop is nested (the balanced split's segment walk); the iterative ILP strategy
    # keeps them overlapped in every copy.
    "-mllvm", "-amdgpu-sched-strategy=iterative-ilp",
    "-Wno-unused-command-line-argument",
]

# Per-source additions.  The raw-K ring kernel multiplies each row by diag(kw) with MFMAs whose
# results feed VALU work; the default heuristic gives every MFMA of a kernel that uses the
# accumulation registers an AGPR result, which would cost four copies per product.
EXTRA_FLAGS = {
    "esda_decode.hip": ["-mllvm", "--amdgpu-mfma-vgpr-form"],
}


def sources() -> list[str]:
    return [os.path.join(CSRC, s) for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]


def build(verbose: bool = False) -> str:
    """Compile every source and link libesda.so; always recompiles."""
    objs = []
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    for src in sources():
        obj = os.path.join(CSRC, os.path.basename(src) + ".o")
        # ES* C++ layer: host code only (HIP runtime API and the esda C ABI), built by
        # the host compiler so no device code is generated for it.
        cmd = [HIPCC] + HIP_FLAGS + EXTRA_FLAGS.get(os.path.basename(src), []) + inc + ["-c", src, "-o", obj]
        if src.endswith(".cpp"):
            cmd = [CXX, "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
                   "-I", os.path.join(ROCM, "include")] + inc + ["-c", src, "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objs.append(obj)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    for o in objs:
        os.remove(o)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB)
