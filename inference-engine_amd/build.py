"""In-tree build of the native libraries (runs on a CPU-only host: hipcc cross-compiles gfx950).

  lib/libie_attn.so     HIP kernels + the C ABI of include/ie_attn.h (no torch dependency)
  lib/_ie_torch_ops.so  torch.ops.ie.* registration, a thin C++ shim over the C ABI

Usage: python -m <package>.build   or   build.build()
"""

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
BUILD = PKG / "_build"
INCLUDE = REPO / "include"

HIP_SOURCES = ["runtime.hip", "kv_write.hip", "decode_attention.hip", "prefill_attention.hip",
               "sampling.hip", "norm_act.hip", "skinny_gemm.hip"]
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # keep the compiler from emitting packed-fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    "-Wno-unused-parameter",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return str(Path(rocm) / "bin" / "hipcc")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    r = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(map(str, cmd))}\n"
                           f"{r.stdout}\n{r.stderr}")
    return r


def _torch_paths():
    import torch
    from torch.utils import cpp_extension as ce

    return ce.include_paths(), ce.library_paths(), Path(torch.__file__).parent


def build_hip(extra_flags=(), verbose=False, out_dir=None) -> Path:
    """Compile every HIP source for gfx950 and link libie_attn.so into `out_dir` (lib/)."""
    lib = Path(out_dir) if out_dir else LIB
    obj_dir = lib / "_obj" if out_dir else BUILD
    obj_dir.mkdir(parents=True, exist_ok=True)
    lib.mkdir(parents=True, exist_ok=True)
    hipcc = _hipcc()
    flags = HIPCC_FLAGS + [f"-I{INCLUDE}"] + list(extra_flags)
    objs = [obj_dir / (Path(s).stem + ".o") for s in HIP_SOURCES]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(HIP_SOURCES))) as ex:
        futs = [ex.submit(_run, [hipcc, *flags, "-c", CSRC / s, "-o", o], verbose)
                for s, o in zip(HIP_SOURCES, objs)]
        for f in futs:
            f.result()
    out = lib / "libie_attn.so"
    tmp = lib / "libie_attn.so.tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", tmp],
         verbose)
    os.replace(tmp, out)
    return out


def build_torch_ops(verbose=False) -> Path:
    """Compile the torch.ops.ie registration shim with g++ against libie_attn.so."""
    incs, libdirs, _ = _torch_paths()
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    out = LIB / "_ie_torch_ops.so"
    tmp = LIB / "_ie_torch_ops.so.tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__",
           "-DUSE_ROCM", "-D_GLIBCXX_USE_CXX11_ABI=1", f"-I{INCLUDE}", f"-I{rocm}/include"]
    cmd += [f"-I{p}" for p in incs]
    cmd += [CSRC / "torch_ops.cpp", "-o", tmp, f"-L{LIB}", "-lie_attn"]
    cmd += [f"-L{p}" for p in libdirs]
    cmd += ["-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
            f"-L{rocm}/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN"]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(extra_hip_flags=(), verbose=False) -> None:
    build_hip(extra_hip_flags, verbose)
    build_torch_ops(verbose)


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)


if __name__ == "__main__":
    if "--stamps" in sys.argv:
        # the prefill kernel with its phase stamps compiled in (bench.py --prefill-stamps)
        out = build_hip(["-DIE_PREFILL_PHASE_STAMPS"], verbose="-v" in sys.argv,
                        out_dir=LIB / "stamps")
        shutil.rmtree(LIB / "stamps" / "_obj", ignore_errors=True)
        print("built", out)
    else:
        build(verbose="-v" in sys.argv)
        print("built", LIB / "libie_attn.so", LIB / "_ie_torch_ops.so")
