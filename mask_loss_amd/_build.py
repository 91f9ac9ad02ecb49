"""In-tree build of the HIP kernels and the `mask_loss` extension module.

* ``libmask_loss_hip.so``: every ``csrc/*.hip`` file compiled by hipcc for
  gfx950 and linked into one shared library exposing the C ABI of
  ``include/mask_loss_hip.h``.
* ``mask_loss<ext-suffix>.so``: ``csrc/bindings.cpp`` (PyTorch C++ extension,
  pybind11) compiled by g++ against the installed PyTorch-ROCm headers and
  linked to ``libmask_loss_hip.so`` (rpath $ORIGIN).

Both land next to this file, so they travel with the repository tree.
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
ROOT = os.path.dirname(HERE)
HIP_LIB = os.path.join(HERE, "libmask_loss_hip.so")
EXT_SUFFIX = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
EXT = os.path.join(HERE, "mask_loss" + EXT_SUFFIX)
ARCH = os.environ.get("ML_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # no packed fp32 instructions anywhere in this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}")
    return r.stdout


def _hip_sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _headers():
    hs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    hs.append(os.path.join(ROOT, "include", "mask_loss_hip.h"))
    return hs


def _newer(target, deps):
    if not os.path.exists(target):
        return False
    t = os.path.getmtime(target)
    return all(os.path.getmtime(d) <= t for d in deps)


def build_hip(force=True, jobs=8, verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = _hip_sources()
    hdrs = _headers()
    objs = []
    todo = []
    for s in srcs:
        o = os.path.join(BUILD, os.path.basename(s)[:-4] + ".o")
        objs.append(o)
        if force or not _newer(o, [s] + hdrs):
            todo.append((s, o))

    def one(so):
        s, o = so
        out = _run(["hipcc", *HIPCC_FLAGS, "-c", s, "-o", o])
        if verbose and out.strip():
            print(out)

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(one, todo))
    if force or todo or not _newer(HIP_LIB, objs):
        _run(["hipcc", "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", HIP_LIB])
    return HIP_LIB


def build_ext(force=True):
    import torch.utils.cpp_extension as ce  # only for include / library paths
    import pybind11

    src = os.path.join(CSRC, "bindings.cpp")
    if not force and _newer(EXT, [src, HIP_LIB] + _headers()):
        return EXT
    inc = ce.include_paths()
    libdir = ce.library_paths()[0]
    pyinc = sysconfig.get_paths()["include"]
    abi = "1"
    try:
        import torch
        abi = "1" if torch._C._GLIBCXX_USE_CXX11_ABI else "0"
    except Exception:
        pass
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=mask_loss", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *[f"-I{p}" for p in inc], f"-I{pybind11.get_include()}", f"-I{pyinc}",
        "-I/opt/rocm/include",
        src, "-o", EXT,
        f"-L{HERE}", "-lmask_loss_hip", "-Wl,-rpath,$ORIGIN",
        f"-L{libdir}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip",
        "-ltorch_hip", f"-Wl,-rpath,{libdir}", "-L/opt/rocm/lib", "-lamdhip64",
    ]
    _run(cmd)
    return EXT


def build(force=True, verbose=False):
    build_hip(force=force, verbose=verbose)
    build_ext(force=force)
    return HIP_LIB, EXT


if __name__ == "__main__":
    force = "--incremental" not in sys.argv
    print(build(force=force, verbose=True))
