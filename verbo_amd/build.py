"""Build recipe of libvsmp.so: hipcc for gfx950, in-tree.

    python -m verbo_amd.build        # or verbo_amd.build.build()

The library holds the HIP kernels, the C ABI (include/vsmp.h) and the drop-in verbo::Sampler. The
drop-in verbo::generate (csrc/generate.cpp, plain C++) calls verbo's Session and Model, so it is
compiled with the program that provides them: verbo's own build, or the test double.
"""
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libvsmp.so"
SOURCES = ["vsmp_kernels.hip", "vsmp_head.hip", "vsmp_api.cpp", "sampler.cpp", "decode.cpp"]
ARCH = os.environ.get("VSMP_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in the device code.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", str(ROOT / "include"), "-I", str(CSRC),
]


def hipcc():
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build libvsmp.so)")
    return exe


def build(verbose=False):
    """Compile every source and link libvsmp.so (always rebuilds)."""
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    objs = []
    for src in SOURCES:
        obj = objdir / (Path(src).stem + ".o")
        cmd = [hipcc(), *HIPCC_FLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objs.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB)
