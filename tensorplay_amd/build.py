"""Build the native parts of tensorplay_amd in-tree for gfx950.

  libtpr_rocm.so   HIP kernels + the C-ABI launch layer (include/tpr_rocm.h)
  libtpr_rocm_dev.so  the same with the plan-override hook tpr_debug_set
                   (-DTPR_DEBUG_KNOBS): the test build, loaded by the tests
                   that force plans; the shipped library has no mutable plan state
  _C<ext>          host core (tensor, dispatcher with the ROCm key, caching
                   allocator, reduction adapters) + Python bindings; links
                   libtpr_rocm.so

Usage: python tensorplay_amd/build.py  (or tensorplay_amd.build.build_all()).
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: never emit packed fp32 (v_pk_*_f32) instructions.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]

ROCM_SOURCES = ["rocm/capi.cpp", "rocm/reduce.hip", "rocm/topk.hip", "rocm/copy.hip",
                "rocm/softmax.hip", "rocm/loss.hip", "rocm/reduce_bwd.hip"]
LIB_TPR = os.path.join(PKG, "libtpr_rocm.so")
LIB_TPR_DEV = os.path.join(PKG, "libtpr_rocm_dev.so")


def _run(cmd):
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def _run_all(cmds):
    """Independent compiles in parallel (at most 8 jobs)."""
    if not cmds:
        return
    with ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
        for f in [ex.submit(_run, c) for c in cmds]:
            f.result()


def _newer(target, deps):
    if not os.path.exists(target):
        return True
    t = os.path.getmtime(target)
    return any(os.path.getmtime(d) > t for d in deps)


def _tpr_compiles(force, dev):
    """(compile commands, objects) of one flavour of libtpr_rocm."""
    bdir = os.path.join(BUILD, "dev") if dev else BUILD
    os.makedirs(bdir, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(CSRC, "rocm")]
    headers = [os.path.join(ROOT, "include", "tpr_rocm.h"), os.path.join(CSRC, "rocm", "common.h")]
    extra = ["-DTPR_DEBUG_KNOBS"] if dev else []
    objs, cmds = [], []
    for src in ROCM_SOURCES:
        s = os.path.join(CSRC, src)
        o = os.path.join(bdir, os.path.basename(src) + ".o")
        if force or _newer(o, [s] + headers):
            lang = ["-x", "hip"] if src.endswith(".cpp") else []
            cmds.append([HIPCC] + HIP_FLAGS + extra + inc + lang + ["-c", s, "-o", o])
        objs.append(o)
    return cmds, objs


def build_tpr(force=True, dev=True):
    """libtpr_rocm.so and (dev=True) the test build libtpr_rocm_dev.so, compiled together."""
    cmds, objs = _tpr_compiles(force, False)
    dcmds, dobjs = _tpr_compiles(force, True) if dev else ([], [])
    # the longest compiles first, so the pool drains evenly
    _run_all(sorted(cmds + dcmds, key=lambda c: ("topk" not in c[-3], "reduce.hip" not in c[-3])))
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", LIB_TPR] + objs)
    if dev:
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", LIB_TPR_DEV] + dobjs)
    return LIB_TPR


CORE_SOURCES = ["core/Dispatcher.cpp", "core/Allocator.cpp", "core/Tensor.cpp",
                "core/ROCmReductionKernels.cpp", "core/CopyKernels.cpp", "core/ROCmSoftmaxLossKernels.cpp",
                "core/bindings.cpp"]
CXX = os.environ.get("CXX", "g++")


def build_core(force=True):
    import sysconfig
    import pybind11
    os.makedirs(BUILD, exist_ok=True)
    ext = sysconfig.get_config_var("EXT_SUFFIX")
    out = os.path.join(PKG, "_C" + ext)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(CSRC, "core"),
           "-I", "/opt/rocm/include", "-I", pybind11.get_include(),
           "-I", sysconfig.get_paths()["include"]]
    flags = ["-O2", "-std=c++17", "-fPIC", "-D__HIP_PLATFORM_AMD__", "-fvisibility=hidden", "-Wall"]
    headers = [os.path.join(CSRC, "core", h) for h in os.listdir(os.path.join(CSRC, "core")) if h.endswith(".h")]
    headers.append(os.path.join(ROOT, "include", "tpr_rocm.h"))
    objs, cmds = [], []
    for src in CORE_SOURCES:
        s = os.path.join(CSRC, src)
        o = os.path.join(BUILD, os.path.basename(src) + ".o")
        if force or _newer(o, [s] + headers):
            cmds.append([CXX] + flags + inc + ["-c", s, "-o", o])
        objs.append(o)
    _run_all(cmds)
    _run([CXX, "-shared", "-o", out] + objs +
         ["-L", PKG, "-ltpr_rocm", "-L", "/opt/rocm/lib", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,/opt/rocm/lib"])
    return out


def build_all(force=True):
    build_tpr(force)
    build_core(force)


if __name__ == "__main__":
    build_all(force="--incremental" not in sys.argv)
