"""Build recipe of ``libmtl_hip.so``: every ``csrc/*.hip`` compiled for gfx950.

The library exposes only the plain C ABI declared in ``include/mtl_gptq.h`` and
``include/mtl_decode.h`` (raw device pointers, sizes, a ``hipStream_t``), so it
links against whichever HIP runtime the process already has loaded (torch's).
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
LIB_NAME = "libmtl_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 HIP library cannot be built")


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(PKG_DIR, "csrc", "*.hip")))


FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # Packed fp32 VALU ops stay off: write plain float code only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", os.path.join(PKG_DIR, "csrc"),
]


def command(out: str = LIB_PATH) -> list[str]:
    """One-invocation form of the build (every source, then link)."""
    return [hipcc(), *FLAGS, "-shared", *sources(), "-o", out]


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    return err


TORCH_OPS_SRC = os.path.join(PKG_DIR, "torch_ops", "mtl_torch_ops.cpp")
TORCH_OPS_PATH = os.path.join(PKG_DIR, "libmtl_torch_ops.so")


def torch_ops_command(out: str = TORCH_OPS_PATH) -> list[str]:
    """g++ line of the torch dispatcher operators (host code over the C ABI), linked
    against libmtl_hip.so beside it and torch's own libraries."""
    import torch
    import torch.utils.cpp_extension as ce

    tdir = os.path.dirname(torch.__file__)
    incs = [p for p in ce.include_paths() if os.path.isdir(p)]
    abi = int(torch.compiled_with_cxx11_abi())
    return ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
            "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
            *[f"-I{p}" for p in incs], "-I/opt/rocm/include", f"-I{os.path.join(ROOT, 'include')}",
            TORCH_OPS_SRC, f"-L{os.path.join(tdir, 'lib')}", f"-L{PKG_DIR}",
            "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{os.path.join(tdir, 'lib')}",
            "-lmtl_hip", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch", "-o", out]


def build_torch_ops() -> str:
    """Compile the torch operator library in-tree (after libmtl_hip.so) and return its path."""
    tmp = TORCH_OPS_PATH + ".tmp"
    _run(torch_ops_command(tmp))
    os.replace(tmp, TORCH_OPS_PATH)
    return TORCH_OPS_PATH


def build(verbose: bool = False) -> str:
    """Compile the library in-tree (always recompiles; one hipcc per source, in
    parallel), then the torch operator library over it, and return the library's path."""
    from concurrent.futures import ThreadPoolExecutor

    with tempfile.TemporaryDirectory(prefix="mtl_build_") as tmpdir:
        objs = [os.path.join(tmpdir, os.path.basename(src) + ".o") for src in sources()]
        cmds = [[hipcc(), *FLAGS, "-c", src, "-o", obj] for src, obj in zip(sources(), objs)]
        with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as pool:
            errs = list(pool.map(_run, cmds))
        tmp = LIB_PATH + ".tmp"
        errs.append(_run([hipcc(), f"--offload-arch={ARCH}", "-shared", *objs, "-o", tmp]))
    err = "\n".join(e for e in errs if e.strip())
    if verbose and err:
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    build_torch_ops()
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
