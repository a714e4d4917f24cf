"""In-tree build of tvdcn_amd's native code (no cmake, no setuptools).

Two shared objects are produced next to this file:

* ``libtvdcn_hip.so`` -- the gfx950 HIP kernels behind the C ABI declared in
  ``include/tvdcn_hip.h`` (hipcc, one object per ``csrc/hip/*.hip``).
* ``_C.so`` -- the PyTorch operator layer (``csrc/torch/ops.cpp``) that registers
  the ``tvdcn`` ops and calls the C ABI (links against ``libtvdcn_hip.so``), with the
  host-tensor (CPU key) kernels of ``csrc/torch/cpu_kernels.cpp`` and the C++ API of
  ``include/tvdcn_ops.h`` (``csrc/torch/cpp_api.cpp``).

Run ``python -m tvdcn_amd._build`` (or ``__graft_entry__.build()``). Objects go to
``tvdcn_amd/_build/`` and are rebuilt when their sources (or shared headers) change.
"""
import concurrent.futures
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIP_DIR = os.path.join(HERE, "csrc", "hip")
TORCH_SRC = os.path.join(HERE, "csrc", "torch", "ops.cpp")
CPU_SRC = os.path.join(HERE, "csrc", "torch", "cpu_kernels.cpp")
CPP_API_SRC = os.path.join(HERE, "csrc", "torch", "cpp_api.cpp")
INCLUDE = os.path.join(ROOT, "include")
OBJ_DIR = os.path.join(HERE, "_build")
HIP_LIB = os.path.join(HERE, "libtvdcn_hip.so")
TORCH_LIB = os.path.join(HERE, "_C.so")

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 VALU forms are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wno-pass-failed", "-I", INCLUDE,
]


def _hip_sources():
    return sorted(os.path.join(HIP_DIR, f) for f in os.listdir(HIP_DIR) if f.endswith(".hip"))


def _headers():
    return [os.path.join(HIP_DIR, f) for f in os.listdir(HIP_DIR) if f.endswith(".h")] + \
        [os.path.join(INCLUDE, f) for f in os.listdir(INCLUDE) if f.endswith(".h")]


def _torch_headers():
    d = os.path.join(HERE, "csrc", "torch")
    return [os.path.join(d, f) for f in os.listdir(d) if f.endswith(".h")]


def _stale(target, deps):
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(d) > t for d in deps)


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build_hip(force=False, jobs=None, verbose=False):
    os.makedirs(OBJ_DIR, exist_ok=True)
    headers = _headers()
    srcs = _hip_sources()
    objs = [os.path.join(OBJ_DIR, os.path.basename(s)[:-4] + ".o") for s in srcs]
    todo = [(s, o) for s, o in zip(srcs, objs) if force or _stale(o, [s] + headers)]

    def compile_one(so):
        s, o = so
        _run([HIPCC] + HIP_FLAGS + ["-c", s, "-o", o])
        return s

    if todo:
        jobs = jobs or min(len(todo), max(1, os.cpu_count() or 1))
        with concurrent.futures.ThreadPoolExecutor(jobs) as ex:
            for s in ex.map(compile_one, todo):
                if verbose:
                    print("compiled", os.path.relpath(s, ROOT), flush=True)
    if force or todo or _stale(HIP_LIB, objs):
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", HIP_LIB] + objs +
             [f"-Wl,-rpath,{ROCM}/lib"])
    return HIP_LIB


def _torch_paths():
    import torch
    tdir = os.path.dirname(torch.__file__)
    return tdir, [os.path.join(tdir, "include"), os.path.join(tdir, "include", "torch", "csrc", "api", "include")]


def build_torch(force=False, verbose=False):
    import torch
    tdir, incs = _torch_paths()
    os.makedirs(OBJ_DIR, exist_ok=True)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    objs = []
    for src, extra in ((TORCH_SRC, []), (CPU_SRC, ["-O3", "-fopenmp"]), (CPP_API_SRC, [])):
        obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + "_torch.o")
        objs.append(obj)
        if force or _stale(obj, [src] + _headers() + _torch_headers()):
            cmd = ["g++", "-O2", "-std=c++17", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
                   "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-Wno-deprecated-declarations",
                   "-I", INCLUDE, "-I", os.path.join(ROCM, "include")] + extra
            for i in incs:
                cmd += ["-isystem", i]
            cmd += ["-c", src, "-o", obj]
            _run(cmd)
            if verbose:
                print("compiled", os.path.relpath(src, ROOT), flush=True)
    if force or _stale(TORCH_LIB, objs + [HIP_LIB]):
        libdir = os.path.join(tdir, "lib")
        # OpenMP from torch's own libgomp (the runtime ATen's parallel_for already uses)
        _run(["g++", "-shared", "-o", TORCH_LIB] + objs + ["-L", libdir, "-lc10", "-lc10_hip", "-ltorch",
              "-ltorch_cpu", "-ltorch_hip", "-lgomp", "-L", HERE, "-ltvdcn_hip",
              "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}"])
    return TORCH_LIB


def build(force=False, verbose=False):
    build_hip(force=force, verbose=verbose)
    build_torch(force=force, verbose=verbose)


if __name__ == "__main__":
    build(force="--force" in sys.argv, verbose=True)
    print("built", HIP_LIB, TORCH_LIB)
