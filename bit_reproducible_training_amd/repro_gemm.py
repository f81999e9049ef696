"""Python mirror of the reproducible GEMM interface.

Names, fields and error behaviour follow repro_gemm_cuda/repro_gemm.cuh:25-75 (Algo,
Config, Plan, make_plan, repro_gemm_fp32_ws, repro_gemm_fp32, algo_name) and the
PyTorch binding repro_torch/src/bindings.cpp:43-66 (gemm). Everything runs through the
C ABI of librepro_gemm.so on the GPU; there is no CPU path. Device memory and streams
come from PyTorch (torch.cuda = HIP on ROCm).
"""
import ctypes
import enum
from dataclasses import dataclass

from . import _lib
from ._lib import lib

MAX_SLICES = 3


class ReproGemmError(RuntimeError):
    """A non-zero hipError_t from the library; .code holds it."""

    def __init__(self, code, what):
        self.code = int(code)
        super().__init__("%s: %s (hip error %d)" % (what, _lib.error_string(code), code))


class Algo(enum.IntEnum):
    Auto = 0        # MFMA contraction, block tile chosen for the shape
    Reference = 1   # one thread per output, int64 (verification)
    Tiled = 2       # MFMA contraction, 64x64 block tile
    TensorCore = 3  # MFMA contraction, block tile chosen for the shape


@dataclass
class Config:
    split_k: int = 1
    tile_m: int = 16
    tile_n: int = 16
    tile_k: int = 32
    algo: Algo = Algo.Auto
    slices: int = 3
    trans_a: bool = False
    trans_b: bool = False

    def to_c(self):
        return _lib.rg_config(int(self.split_k), int(self.tile_m), int(self.tile_n),
                              int(self.tile_k), int(self.algo), int(self.slices),
                              int(bool(self.trans_a)), int(bool(self.trans_b)))


@dataclass
class Plan:
    algo: Algo
    split_k: int
    workspace_bytes: int
    tile_m: int = 0
    tile_n: int = 0


def _check(code, what):
    if code != _lib.HIP_SUCCESS:
        raise ReproGemmError(code, what)


def make_plan(M, N, K, cfg=None):
    """What will run for this problem on the current device (repro_gemm.cuh:53)."""
    cfg = cfg or Config()
    c = cfg.to_c()
    p = _lib.rg_plan()
    _check(lib.rg_make_plan(int(M), int(N), int(K), ctypes.byref(c), ctypes.byref(p)), "make_plan")
    return Plan(Algo(p.algo), p.split_k, p.workspace_bytes, p.tile_m, p.tile_n)


def plan_for_device(M, N, K, cfg=None, is_gfx950=True, num_cus=256):
    """The planner with an explicit device description (no GPU needed)."""
    cfg = cfg or Config()
    c = cfg.to_c()
    p = _lib.rg_plan()
    info = _lib.rg_layout_info()
    _check(lib.rg_plan_for_device(int(M), int(N), int(K), ctypes.byref(c), int(bool(is_gfx950)),
                                  int(num_cus), ctypes.byref(p), ctypes.byref(info)),
           "plan_for_device")
    return Plan(Algo(p.algo), p.split_k, p.workspace_bytes, p.tile_m, p.tile_n), info


def workspace_layout(M, N, K, cfg=None):
    """Offsets of the internal workspace regions on the current device."""
    cfg = cfg or Config()
    c = cfg.to_c()
    info = _lib.rg_layout_info()
    _check(lib.rg_workspace_layout(int(M), int(N), int(K), ctypes.byref(c), ctypes.byref(info)),
           "workspace_layout")
    return info


def repro_gemm_fp32_ws(A, B, C, M, N, K, cfg, workspace, workspace_bytes, stream=None,
                       stage_events=None):
    """Raw-pointer entry point (repro_gemm.cuh:60-66). A, B, C, workspace are device
    addresses (ints), stream a hipStream_t handle (int) or None, stage_events a sequence
    of 4 hipEvent_t handles or None. Returns the hipError_t code."""
    c = cfg.to_c()
    ev = None
    if stage_events is not None:
        arr = (ctypes.c_void_p * 4)(*[int(e) for e in stage_events])
        ev = ctypes.cast(arr, ctypes.c_void_p)
    return lib.rg_gemm_fp32_ws(A, B, C, int(M), int(N), int(K), ctypes.byref(c), workspace,
                               int(workspace_bytes), stream, ev)


def repro_gemm_fp32(A, B, C, M, N, K, cfg=None, stream=None):
    """Convenience entry point (repro_gemm.cuh:69-73): allocates, runs, synchronises, frees."""
    cfg = cfg or Config()
    c = cfg.to_c()
    return lib.rg_gemm_fp32(A, B, C, int(M), int(N), int(K), ctypes.byref(c), stream)


def measure_mfma_int8_rate(dense=True):
    """Sustained int8 MFMA TOP/s of the current device with register operands (dense random
    bytes or zeros); the practical ceiling of the contraction under the power limit."""
    out = ctypes.c_double()
    _check(lib.rg_measure_mfma_int8_rate(int(bool(dense)), ctypes.byref(out)), "measure_mfma_int8_rate")
    return out.value


def algo_name(a):
    return lib.rg_algo_name(int(a)).decode()


# --------------------------------------------------------------------------------------
# PyTorch-facing operation (repro_torch/src/bindings.cpp:43-66)
# --------------------------------------------------------------------------------------

_ws_cache = {}


def _workspace(torch, nbytes, device):
    """A cached uint8 device buffer of at least nbytes per device (grown on demand)."""
    key = (device.type, device.index)
    buf = _ws_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
        _ws_cache[key] = buf
    return buf


def gemm(A, B, M, N, K, ta=False, tb=False, S=3, cfg=None, out=None):
    """C[M, N] = op(A) op(B) for float32 GPU tensors, on the current stream.

    Same argument meaning and checks as the reference binding: A holds M*K values
    (K x M if ta), B holds N*K values (N x K if tb); both float32. Unlike the
    reference there is no CPU fallback: CPU tensors raise.
    """
    import torch

    if A.dtype != torch.float32:
        raise ValueError("A must be float32")
    if B.dtype != torch.float32:
        raise ValueError("B must be float32")
    if not (A.is_cuda and B.is_cuda):
        raise ValueError("gemm: A and B must be GPU tensors (no CPU path in this library)")
    A = A.contiguous()
    B = B.contiguous()
    if A.numel() != M * K or B.numel() != N * K:
        raise ValueError("gemm: shape mismatch")
    if cfg is None:
        cfg = Config(slices=S, trans_a=bool(ta), trans_b=bool(tb))
    plan = make_plan(M, N, K, cfg)
    C = out if out is not None else torch.empty((M, N), dtype=torch.float32, device=A.device)
    ws = _workspace(torch, plan.workspace_bytes, A.device)
    stream = torch.cuda.current_stream(A.device).cuda_stream
    code = repro_gemm_fp32_ws(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, cfg,
                              ws.data_ptr(), ws.numel(), stream)
    _check(code, "gemm")
    return C
