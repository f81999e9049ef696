"""Python mirror of the exact-sum interface and of the non-finite scan.

Names, fields and error behaviour follow repro_sum_cuda/repro_sum.cuh:27-45 (SumConfig,
SumPlan, make_sum_plan, repro_sum_fp32_ws, repro_sum_fp32) and the PyTorch bindings
repro_torch/src/bindings.cpp:69-91 (exact_sum) and :286-297 (scan_finite). Everything runs
through the C ABI of librepro_gemm.so (include/repro_sum.h) on the GPU; there is no CPU path.
"""
import ctypes
from dataclasses import dataclass

from . import _lib
from ._lib import lib
from .repro_gemm import ReproGemmError, _check, _workspace


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
    mean), for a float32 GPU tensor x viewed as [A][B][C]; on the current stream.

    Same arguments and checks as the reference binding (bindings.cpp:69-91); CPU tensors
    raise (no CPU path in this library).
    """
    import torch

    if x.dtype != torch.float32:
        raise ValueError("x must be float32")
    if not x.is_cuda:
        raise ValueError("exact_sum: x must be a GPU tensor (no CPU path in this library)")
    x = x.contiguous()
    if x.numel() != A * B * C:
        raise ValueError("sum: shape mismatch")
    cfg = SumConfig(mean=bool(mean))
    plan = make_sum_plan(A, B, C, cfg)
    out = torch.empty((B,), dtype=torch.float32, device=x.device)
    ws = _workspace(torch, plan.workspace_bytes, x.device)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    code = repro_sum_fp32_ws(x.data_ptr(), out.data_ptr(), A, B, C, cfg, ws.data_ptr(),
                             ws.numel(), stream)
    _check(code, "sum")
    return out


def scan_finite(x, flag, op_id):
    """Lowers flag[0] (an int32 GPU tensor) to op_id if x holds a NaN or infinity, on the
    current stream, without synchronising (bindings.cpp:286-297, kernels.cu:8-20)."""
    import torch

    if x.dtype != torch.float32:
        raise ValueError("x must be float32")
    if not (x.is_cuda and flag.is_cuda) or flag.dtype != torch.int32:
        raise ValueError("scan_finite: x and an int32 flag must be GPU tensors")
    x = x.contiguous()
    stream = torch.cuda.current_stream(x.device).cuda_stream
    code = lib.rg_scan_finite(x.data_ptr(), flag.data_ptr(), x.numel(), int(op_id), stream)
    _check(code, "finite scan")


__all__ = ["SumConfig", "SumPlan", "make_sum_plan", "sum_plan_for_device", "repro_sum_fp32_ws",
           "repro_sum_fp32", "exact_sum", "scan_finite", "ReproGemmError"]
