"""Builds librepro_gemm.so (HIP, gfx950) and its PyTorch binding in-tree.

The library is compiled with hipcc from the sources under csrc/ into
bit_reproducible_training_amd/librepro_gemm.so, next to this file, so it travels with
the repository. Flags that affect results: no fast-math, no denormal flushing,
correctly rounded fp32 division (hipcc's default), no FP contraction.

The binding (csrc/rg_torch.cpp -> _backend<python suffix>.so) is host C++ compiled with g++
against PyTorch's headers; it calls the library through its C ABI and carries the CPU
implementation (include/repro_*_cpu.h) for CPU tensors.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
BUILD_DIR = os.path.join(CSRC, "_build")
LIB_PATH = os.path.join(PKG_DIR, "librepro_gemm.so")

SOURCES = ["rg_slice.hip", "rg_contract.hip", "rg_probe.hip", "rg_sum.hip", "rg_conv.hip", "rg_api.cpp"]
BINDING_SOURCE = "rg_torch.cpp"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    # Keep the compiler from emitting packed fp32 VALU instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    "-I", INCLUDE,
    "-I", CSRC,
]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "packed-fp32-ops" not in line and "not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError("command failed (%d): %s\n%s" % (proc.returncode, " ".join(cmd), out))
    return out


def binding_path():
    import sysconfig

    return os.path.join(PKG_DIR, "_backend" + sysconfig.get_config_var("EXT_SUFFIX"))


def _binding_compile_cmd(obj):
    import sysconfig

    import torch

    tdir = os.path.dirname(torch.__file__)
    return ["g++", "-O2", "-std=c++17", "-fPIC", "-fno-fast-math", "-ffp-contract=off", "-pthread",
            "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM", "-DTORCH_EXTENSION_NAME=_backend",
            "-DTORCH_API_INCLUDE_EXTENSION_H",
            "-D_GLIBCXX_USE_CXX11_ABI=%d" % int(torch._C._GLIBCXX_USE_CXX11_ABI),
            "-I", INCLUDE, "-I", os.path.join(tdir, "include"),
            "-I", os.path.join(tdir, "include", "torch", "csrc", "api", "include"),
            "-I", "/opt/rocm/include", "-I", sysconfig.get_paths()["include"],
            "-c", os.path.join(CSRC, BINDING_SOURCE), "-o", obj]


def _binding_link_cmd(obj, out):
    import torch

    tlib = os.path.join(os.path.dirname(torch.__file__), "lib")
    return ["g++", "-shared", "-pthread", obj, "-o", out, "-L", PKG_DIR, "-l:librepro_gemm.so",
            "-L", tlib, "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
            "-Wl,-rpath,$ORIGIN", "-Wl,-rpath," + tlib]


def build(verbose=False):
    """Compiles every source, links the shared library and the PyTorch binding. Always
    recompiles."""
    os.makedirs(BUILD_DIR, exist_ok=True)

    def compile_one(src):
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        cmd = [HIPCC] + COMMON_FLAGS + ["-c", os.path.join(CSRC, src), "-o", obj]
        if src.endswith(".cpp"):
            cmd[1:1] = ["-x", "hip"]
        out = _run(cmd)
        if verbose and out.strip():
            print(out, file=sys.stderr)
        return obj

    binding_obj = os.path.join(BUILD_DIR, "rg_torch.o")
    with ThreadPoolExecutor(max_workers=len(SOURCES) + 1) as ex:
        binding = ex.submit(_run, _binding_compile_cmd(binding_obj))
        objs = list(ex.map(compile_one, SOURCES))
        binding.result()
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs)
    os.replace(tmp, LIB_PATH)
    out = binding_path()
    _run(_binding_link_cmd(binding_obj, out + ".tmp"))
    os.replace(out + ".tmp", out)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
