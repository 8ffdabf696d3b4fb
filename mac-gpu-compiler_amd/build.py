"""Build recipe for libqe.so (the HIP engine + C ABI) for gfx950.

Run as `python mac-gpu-compiler_amd/build.py` or through __graft_entry__.build(). The library is
built in-tree (mac-gpu-compiler_amd/libqe.so) so it travels with the source tree.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libqe.so")

# every source in csrc/ except the profiling programs' own mains
TOOL_SOURCES = {"qe_decode_cli.cpp", "qe_stage_pmc.hip"}
SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")) and f not in TOOL_SOURCES)

HIPCC_FLAGS = [
    "-O3",
    "--offload-arch=gfx950",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # loadable by the HIP runtime that PyTorch ships (ROCm 7.0) as well as /opt/rocm's
    "-mcode-object-version=5",
    # packed f32 ops stay off: only scalar f32 VALU ops are emitted
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libqe.so)")


# Per-source additions. batch.hip: matrix-core results go to ordinary VGPRs, where the MFMAs
# accumulate in place; with the default accumulation registers the compiler moves the GEMM
# accumulators between register files on every k stage.
SOURCE_FLAGS = {"batch.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
                # fused.hip: the leading pointer arguments of the two-launch layer's kernels go
                # into scalar registers at wave launch (up to 14 dwords), so their first loads do
                # not wait for a load of the argument block
                "fused.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=14"],
                "fused_timed.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=14"],
                # kernels.hip: the same for k_matvec (the lm_head) and k_argmax
                "kernels.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=14"]}

OBJ_DIR = os.path.join(PKG, "_build")
# the host pass warns that it does not know the packed-fp32 feature; that is expected
NOISE = "is not a recognized feature for this target"


def _run(cmd, what: str, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if NOISE not in l)
    if res.returncode != 0:
        raise RuntimeError(f"{what} build failed:\n" + out)
    if verbose and out.strip():
        print(out)


def build(verbose: bool = False) -> str:
    """libqe.so: every source compiled in parallel, then linked."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]

    def compile_one(src):
        obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
        _run([hipcc(), *flags, *SOURCE_FLAGS.get(src, []), "-I", os.path.join(ROOT, "include"), "-c", "-o", obj,
              os.path.join(CSRC, src)], src, verbose)
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"], "libqe.so link",
         verbose)
    os.replace(tmp, LIB)
    return LIB


def build_tools(verbose: bool = False) -> list:
    """The profiling programs beside the library (qe_decode, qe_stage_pmc). They are not part of
    libqe.so: a failure here leaves the library as built."""
    return [build_cli(verbose), build_stage_pmc(verbose)]


CLI_SRC = os.path.join(CSRC, "qe_decode_cli.cpp")
CLI = os.path.join(PKG, "qe_decode")


def build_cli(verbose: bool = False) -> str:
    """qe_decode: the command-line decode loop over libqe.so (rpath $ORIGIN)."""
    tmp = CLI + ".tmp"
    cmd = [hipcc(), "-O2", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall",
           "-I", os.path.join(ROOT, "include"), "-o", tmp, CLI_SRC, "-L", PKG, "-lqe", "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError("qe_decode build failed:\n" + out)
    os.replace(tmp, CLI)
    return CLI



PMC_SRCS = ["qe_stage_pmc.hip", "kernels.hip", "attention.hip", "batch.hip", "fused.hip"]
PMC = os.path.join(PKG, "qe_stage_pmc")


def build_stage_pmc(verbose: bool = False) -> str:
    """qe_stage_pmc: each decode-step kernel (or, with --gemm, the prefill GEMM) on synthetic
    inputs, for counter collection."""
    tmp = PMC + ".tmp"
    flags = [f for f in HIPCC_FLAGS if f not in ("-fPIC", "-shared")]
    # the same code generation as the library's (one flag set for all four sources)
    extra = [f for src in PMC_SRCS for f in SOURCE_FLAGS.get(src, [])]
    cmd = [hipcc(), *flags, *extra, "-I", os.path.join(ROOT, "include"), "-o", tmp,
           *[os.path.join(CSRC, f) for f in PMC_SRCS]]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError("qe_stage_pmc build failed:\n" + out)
    os.replace(tmp, PMC)
    return PMC

if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    if "--tools" in sys.argv:
        print(build_tools(verbose="-v" in sys.argv))
