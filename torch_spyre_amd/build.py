"""Builds libspyre_hip.so in-tree for gfx950 with hipcc.

    python torch_spyre_amd/build.py

(Run it by path: importing the package loads the library this builds.)

Objects go to torch_spyre_amd/_build/ (compiled in parallel), the shared
library to torch_spyre_amd/libspyre_hip.so, and the PyTorch kernels of the
attention and KV ops (csrc/torch_ops.cpp, against torch's headers, calling
that library) to torch_spyre_amd/libspyre_torch.so.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "libspyre_hip.so")
TORCH_OUT = os.path.join(HERE, "libspyre_torch.so")
SOURCES = ["layout.cpp", "dma.hip", "decode_attn.hip", "kv_append.hip", "sdpa_fwd.hip"]
TORCH_SOURCE = "torch_ops.cpp"
ARCH = os.environ.get("SPYRE_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall"]
# Packed-fp32 VALU ops are turned off for all device code.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _torch_dirs():
    """(include dirs, library dir) of the installed torch."""
    import torch

    root = os.path.dirname(os.path.abspath(torch.__file__))
    return [os.path.join(root, "include"), os.path.join(root, "include", "torch", "csrc", "api", "include")], \
        os.path.join(root, "lib")


def _compile(src: str, build_dir: str = BUILD, defines=()) -> str:
    obj = os.path.join(build_dir, os.path.splitext(src)[0] + ".o")
    path = os.path.join(CSRC, src)
    if src.endswith(".hip"):
        cmd = [HIPCC, *COMMON, *DEVICE, *[f"-D{d}" for d in defines], "-c", path, "-o", obj]
    elif src == TORCH_SOURCE:
        import torch

        incs, _ = _torch_dirs()
        abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
        rocm_inc = os.path.join(os.path.dirname(os.path.dirname(os.path.realpath(HIPCC))), "include")
        cmd = [HIPCC, *COMMON, "-x", "c++", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
               f"-D_GLIBCXX_USE_CXX11_ABI={abi}", *[f"-I{d}" for d in incs], f"-I{rocm_inc}", "-c", path, "-o", obj]
    else:
        cmd = [HIPCC, *COMMON, "-x", "c++", "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False, out: str = OUT, build_dir: str = BUILD, defines=()) -> str:
    """Compiles every source and links ``out``; ``defines`` are extra -D
    macros for the device sources (kernel variants)."""
    os.makedirs(build_dir, exist_ok=True)
    with_torch = out == OUT
    srcs = SOURCES + ([TORCH_SOURCE] if with_torch else [])
    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda f: _compile(f, build_dir, defines), srcs))
    torch_obj = objs.pop() if with_torch else None
    tmp = out + ".tmp"
    # --no-undefined: a kernel whose host stub was not emitted fails here,
    # not at the first dlopen.
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-Wl,--no-undefined", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    if with_torch:
        # the torch kernels, linked against the library just built (found
        # beside them at run time) and torch's own libraries
        _, tlib = _torch_dirs()
        tmp = TORCH_OUT + ".tmp"
        cmd = [HIPCC, "-shared", "-Wl,--no-undefined", torch_obj, f"-L{HERE}", "-lspyre_hip", f"-L{tlib}",
               "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-Wl,-rpath,$ORIGIN",
               f"-Wl,-rpath,{tlib}", "-o", tmp]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
        os.replace(tmp, TORCH_OUT)
        if verbose:
            print(f"built {TORCH_OUT}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
