"""Builds libqvkv.so (HIP kernels + C ABI + host pool manager) for gfx950, in-tree.

hipcc cross-compiles without a GPU.  All HIP code is built with packed-fp32 code
generation turned off (-packed-fp32-ops), and with the default IEEE float semantics
(correctly rounded f32 division, no fast-math): the append path must be bit-exact.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(OUT_DIR, "libqvkv.so")
ARCH = os.environ.get("QVKV_ARCH", "gfx950")

HIP_SOURCES = ["kernels.hip", "prefill.hip", "prelude.hip", "abi.hip"]
# Per-file code generation: the prefill kernels keep MFMA accumulators in VGPRs (their
# online-softmax rescale and P split are VALU work on them); decode attention is faster
# with the compiler's default (accumulators in AGPRs).
HIP_FLAGS = {"prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
CXX_SOURCES = ["pool.cpp", "prefix.cpp"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def hip_command(src: str, mode: list, out: str) -> list:
    """The hipcc command for one HIP source of the library (mode: ["-c", ...] for an object,
    ["--cuda-device-only", "-S"] for the device assembly)."""
    return ["hipcc", f"--offload-arch={ARCH}", *mode, "-O3", "-std=c++17", "-Wall",
            "-Wno-unused-function", "-I", os.path.join(ROOT, "include"), "-I", CSRC,
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            *HIP_FLAGS.get(src, []), *os.environ.get("QVKV_EXTRA_HIPFLAGS", "").split(),
            os.path.join(CSRC, src), "-o", out]


def build(verbose: bool = False, jobs: int = 4) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    obj_dir = os.path.join(OUT_DIR, "obj")
    os.makedirs(obj_dir, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    common = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function"]
    procs, objs = [], []
    for src in HIP_SOURCES:
        obj = os.path.join(obj_dir, src + ".o")
        objs.append(obj)
        cmd = hip_command(src, ["-c", "-fPIC", "-fno-gpu-rdc"], obj)
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append(subprocess.Popen(cmd))
    for src in CXX_SOURCES:
        obj = os.path.join(obj_dir, src + ".o")
        objs.append(obj)
        cmd = ["hipcc", "-c", *common, *inc, "-I", "/opt/rocm/include", "-D__HIP_PLATFORM_AMD__", "-x", "c++", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append(subprocess.Popen(cmd))
    failed = [p.args for p in procs if p.wait() != 0]
    if failed:
        raise RuntimeError(f"build failed: {failed[0]}")
    tmp = LIB + ".tmp"
    _run(["hipcc", f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    _check_stubs(tmp)
    os.replace(tmp, LIB)
    return LIB


def _check_stubs(path: str) -> None:
    """Fails the build when a kernel's host launch stub is referenced but not defined: the
    host pass of hipcc can drop one without a diagnostic, and the library would then fail
    only when loaded."""
    out = subprocess.run(["nm", "-D", "--undefined-only", path], check=True,
                         capture_output=True, text=True).stdout
    missing = [ln.split()[-1] for ln in out.splitlines() if "__device_stub__" in ln]
    if missing:
        os.remove(path)
        raise RuntimeError(f"build failed: undefined kernel launch stubs {missing}")


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
