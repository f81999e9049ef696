"""Python mirror of the exact-sum interface and of the non-finite scan.

Names, fields and error behaviour follow repro_sum_cuda/repro_sum.cuh:27-45 (SumConfig,
SumPlan, make_sum_plan, repro_sum_fp32_ws, repro_sum_fp32) and the PyTorch bindings
repro_torch/src/bindings.cpp:69-91 (exact_sum) and :286-297 (scan_finite). GPU work runs
through the C ABI of librepro_gemm.so (include/repro_sum.h); the tensor operations go through the
compiled binding _backend, which runs CPU tensors on the CPU implementation
(include/repro_sum_cpu.h) with the same bits.
"""
import ctypes
from dataclasses import dataclass

from . import _lib
from ._lib import _backend, lib
from .repro_gemm import ReproGemmError, _check


@dataclass
class SumConfig:
    chunks: int = 0     # 0: chosen for the shape and device
    mean: bool = False

    def to_c(self):
        return _lib.rg_sum_config(int(self.chunks), int(bool(self.mean)))


@dataclass
class SumPlan:
    chunks: int
    workspace_bytes: int


def make_sum_plan(A, B, C, cfg=None):
    """Chunking and workspace for x = [A][B][C] on the current device (repro_sum.cuh:37)."""
    c = (cfg or SumConfig()).to_c()
    p = _lib.rg_sum_plan()
    _check(lib.rg_make_sum_plan(int(A), int(B), int(C), ctypes.byref(c), ctypes.byref(p)),
           "make_sum_plan")
    return SumPlan(p.chunks, p.workspace_bytes)


def sum_plan_for_device(A, B, C, cfg=None, num_cus=256):
    """The planner with an explicit compute-unit count (no GPU needed)."""
    c = (cfg or SumConfig()).to_c()
    p = _lib.rg_sum_plan()
    _check(lib.rg_sum_plan_for_device(int(A), int(B), int(C), ctypes.byref(c), int(num_cus),
                                      ctypes.byref(p)), "sum_plan_for_device")
    return SumPlan(p.chunks, p.workspace_bytes)


def repro_sum_fp32_ws(x, out, A, B, C, cfg, workspace, workspace_bytes, stream=None):
    """Raw-pointer entry point (repro_sum.cuh:39-41): x, out, workspace are device addresses
    (ints), stream a hipStream_t handle or None. Returns the hipError_t code."""
    c = cfg.to_c()
    return lib.rg_sum_fp32_ws(x, out, int(A), int(B), int(C), ctypes.byref(c), workspace,
                              int(workspace_bytes), stream)


def repro_sum_fp32(x, out, A, B, C, cfg=None, stream=None):
    """Convenience entry point (repro_sum.cuh:43-45): allocates, runs, synchronises, frees."""
    c = (cfg or SumConfig()).to_c()
    return lib.rg_sum_fp32(x, out, int(A), int(B), int(C), ctypes.byref(c), stream)


def exact_sum(x, A, B, C, mean=False):
    """out[b] = exact sum over a, c of x[a, b, c] rounded once (divided exactly by A*C when
    mean), for a float32 tensor x viewed as [A][B][C]: on its GPU on the current stream, or on
    the CPU (same bits). Same arguments and checks as the reference binding
    (bindings.cpp:69-91)."""
    return _backend.exact_sum(x, int(A), int(B), int(C), bool(mean))


def scan_finite(x, flag, op_id):
    """Lowers flag[0] (an int32 tensor on x's device) to op_id if x holds a NaN or infinity;
    on the GPU it is queued on the current stream without synchronising (bindings.cpp:286-297,
    kernels.cu:8-20)."""
    _backend.scan_finite(x, flag, int(op_id))


__all__ = ["SumConfig", "SumPlan", "make_sum_plan", "sum_plan_for_device", "repro_sum_fp32_ws",
           "repro_sum_fp32", "exact_sum", "scan_finite", "ReproGemmError"]
