"""Builds the dot_amd native libraries in-tree.

    python -m dot_amd._build            # or __graft_entry__.build()

Produces, next to this file:

* ``libdot_amd.so`` — the HIP kernels and the C ABI declared in
  ``include/dot_amd.h`` (hipcc, ``--offload-arch=gfx950``, no torch).
* ``_C.so`` — the PyTorch operator library (``torch.ops.dot.*`` and
  ``torch.ops.dot_amd.*``), linked against ``libdot_amd.so``.

Object files go to ``<repo>/_build/``.  The ``packed-fp32-ops`` target feature
is disabled for all device code.
"""

from __future__ import annotations

import os
import shlex
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(ROOT, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = os.environ.get("DOT_AMD_ARCH", "gfx950")

HIP_SOURCES = ["sinkhorn.hip", "bidi.hip", "preflight.hip", "methods.hip", "capi.hip", "noalloc.hip"]
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def _run(cmd):
    print("+", " ".join(shlex.quote(c) for c in cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in res.stdout.splitlines() if "packed-fp32-ops" not in line)
    if out.strip():
        print(out, flush=True)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {cmd[0]} ... {cmd[-1]}")


def _stale(src, obj):
    """True when obj is missing or older than src or any header of csrc/
    (used by --changed; a plain build compiles everything)."""
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [src] + [os.path.join(CSRC, h) for h in os.listdir(CSRC) if h.endswith((".cuh", ".hpp", ".h"))]
    deps.append(os.path.join(ROOT, "include", "dot_amd.h"))
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


def _hip_object(src, changed_only=False):
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    if changed_only and not _stale(os.path.join(CSRC, src), obj):
        return obj
    _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_capi(changed_only=False):
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(HIP_SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda s: _hip_object(s, changed_only), HIP_SOURCES))
    out = os.path.join(PKG, "libdot_amd.so")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", out, *objs,
          "-Wl,-soname,libdot_amd.so"])
    return out


def build_torch_ops():
    import torch
    from torch.utils import cpp_extension as ce

    os.makedirs(OBJ, exist_ok=True)
    incs = ce.include_paths(device_type="cuda")
    libdirs = ce.library_paths(device_type="cuda")
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    obj = os.path.join(OBJ, "torch_ops.o")
    cxx = os.environ.get("CXX", "g++")
    _run([cxx, "-O2", "-std=c++17", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
          "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-Wno-deprecated-declarations",
          *[f"-I{p}" for p in incs], f"-I{sysconfig.get_paths()['include']}",
          "-c", os.path.join(CSRC, "torch_ops.cpp"), "-o", obj])
    objs = [obj]
    if os.path.exists(os.path.join(CSRC, "cpu_ops.cpp")):
        cobj = os.path.join(OBJ, "cpu_ops.o")
        _run([cxx, "-O3", "-std=c++17", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
              "-Wno-deprecated-declarations", *[f"-I{p}" for p in incs],
              "-c", os.path.join(CSRC, "cpu_ops.cpp"), "-o", cobj])
        objs.append(cobj)
    out = os.path.join(PKG, "_C.so")
    _run([cxx, "-shared", "-o", out, *objs, f"-L{PKG}", "-ldot_amd",
          *[f"-L{p}" for p in libdirs], "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"])
    return out


def build(changed_only=False):
    """Compile both libraries.  ``changed_only`` (``--changed`` on the command
    line) skips HIP objects newer than their source and every header."""
    build_capi(changed_only)
    build_torch_ops()


if __name__ == "__main__":
    build(changed_only="--changed" in sys.argv)
    sys.exit(0)
