"""Build libqlin.so (the HIP kernels + C ABI) for gfx950 with hipcc, in-tree.

    python mac-kernels-public_amd/build_lib.py [--jobs N]

Each .hip translation unit is compiled to an object in parallel, then linked into
mac-kernels-public_amd/qlin/libqlin.so.  The hardware-floor probes of the measurement suite
(probe/floors.hip) go into a library of their own, qlin/libqlin_floors.so, and the eager PyTorch
entry points (csrc/torch_ops.cpp) into the module qlin/_qlin_torch.so.  Packed-FP32 VALU
instructions are disabled for all device code (-Xclang -target-feature -Xclang -packed-fp32-ops).
"""
import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "qlin", "libqlin.so")
FLOORS_OUT = os.path.join(HERE, "qlin", "libqlin_floors.so")
BUILD = os.path.join(HERE, "_build")
ARCH = os.environ.get("QLIN_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]


def _stale(src, obj):
    if not os.path.exists(obj):
        return True
    deps = [src] + glob.glob(os.path.join(CSRC, "*.h")) + [os.path.join(HERE, "..", "include", "qlin.h"), __file__]
    return max(os.path.getmtime(d) for d in deps) > os.path.getmtime(obj)


def _compile(src, force=True):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if not force and not _stale(src, obj):
        return src, obj, 0, ""
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that noise.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in r.stderr.splitlines() if noise not in line)
    return src, obj, r.returncode, err


def build(jobs=None, verbose=False, force=True):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    objs = []
    with cf.ThreadPoolExecutor(jobs) as ex:
        for src, obj, rc, err in ex.map(lambda s: _compile(s, force), srcs):
            if err.strip() and (verbose or rc):
                print(err, file=sys.stderr)
            if rc:
                raise RuntimeError(f"hipcc failed on {os.path.basename(src)}")
            objs.append(obj)
    tmp = OUT + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs],
                       capture_output=True, text=True)
    if r.returncode:
        print(r.stderr, file=sys.stderr)
        raise RuntimeError("link failed")
    os.replace(tmp, OUT)
    build_floors()
    build_torch_ops()
    return OUT


def build_torch_ops():
    """qlin/_qlin_torch.so: the eager PyTorch entry points (csrc/torch_ops.cpp), a host-only C++
    module linked against libqlin.so and torch; built with the system C++ compiler."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension as ce
    src = os.path.join(CSRC, "torch_ops.cpp")
    out = os.path.join(HERE, "qlin", "_qlin_torch.so")
    tmp = out + ".tmp"
    tlib = ce.library_paths()[0]
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w", src, "-o", tmp,
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_qlin_torch",
           "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           "-I", os.path.join(HERE, "..", "include"), "-I", "/opt/rocm/include", "-I", sysconfig.get_paths()["include"],
           *[a for p in ce.include_paths() for a in ("-I", p)],
           "-L", os.path.dirname(OUT), "-lqlin", "-L", tlib, "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_python", "-L", "/opt/rocm/lib", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{tlib}", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        print(r.stderr, file=sys.stderr)
        raise RuntimeError("g++ failed on torch_ops.cpp")
    os.replace(tmp, out)
    return out


def build_floors():
    """libqlin_floors.so: the hardware-floor probes of the measurement suite (probe/floors.hip);
    a separate library that nothing in libqlin uses."""
    src = os.path.join(HERE, "probe", "floors.hip")
    tmp = FLOORS_OUT + ".tmp"
    r = subprocess.run([HIPCC, *FLAGS, "-shared", "-o", tmp, src], capture_output=True, text=True)
    if r.returncode:
        print(r.stderr, file=sys.stderr)
        raise RuntimeError("hipcc failed on probe/floors.hip")
    os.replace(tmp, FLOORS_OUT)
    return FLOORS_OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--incremental", action="store_true", help="recompile only stale objects")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose, force=not a.incremental))
