"""Python mirror of the reproducible GEMM interface.

Names, fields and error behaviour follow repro_gemm_cuda/repro_gemm.cuh:25-75 (Algo,
Config, Plan, make_plan, repro_gemm_fp32_ws, repro_gemm_fp32, algo_name) and the
PyTorch binding repro_torch/src/bindings.cpp:43-66 (gemm). The strided-batched form (bmm,
repro_gemm_strided_batched_fp32_ws) has no counterpart in the reference, which lists batched
GEMM for attention as still needed (README.md:29). GPU work runs through the C ABI of
librepro_gemm.so (ctypes for the raw-pointer entry points, the compiled binding _backend for
tensors); CPU tensors run the CPU implementation (include/repro_gemm_cpu.h) inside _backend.
Device memory and streams come from PyTorch (torch.cuda = HIP on ROCm).
"""
import ctypes
import enum
from dataclasses import dataclass

from . import _lib
from ._lib import _backend, lib

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


def make_plan_strided_batched(M, N, K, batch, cfg=None):
    """Plan of `batch` independent GEMMs of one shape on the current device."""
    cfg = cfg or Config()
    c = cfg.to_c()
    p = _lib.rg_plan()
    _check(lib.rg_make_plan_strided_batched(int(M), int(N), int(K), int(batch), ctypes.byref(c),
                                            ctypes.byref(p)), "make_plan_strided_batched")
    return Plan(Algo(p.algo), p.split_k, p.workspace_bytes, p.tile_m, p.tile_n)


def repro_gemm_strided_batched_fp32_ws(A, lda, stride_a, B, ldb, stride_b, C, ldc, stride_c,
                                       M, N, K, batch, cfg, workspace, workspace_bytes,
                                       stream=None):
    """Raw-pointer strided-batched entry point (include/repro_gemm.h). Returns the code."""
    c = cfg.to_c()
    return lib.rg_gemm_strided_batched_fp32_ws(A, int(lda), int(stride_a), B, int(ldb),
                                               int(stride_b), C, int(ldc), int(stride_c), int(M),
                                               int(N), int(K), int(batch), ctypes.byref(c),
                                               workspace, int(workspace_bytes), stream)


def measure_mfma_int8_rate(dense=True, low7=False):
    """Sustained int8 MFMA TOP/s of the current device with register operands: dense random
    bytes, random bytes in [0, 127] (low7; the data of the lower digit planes) or zeros; the
    practical ceiling of the contraction under the power limit."""
    out = ctypes.c_double()
    mode = 2 if low7 else int(bool(dense))
    _check(lib.rg_measure_mfma_int8_rate(mode, ctypes.byref(out)), "measure_mfma_int8_rate")
    return out.value


def algo_name(a):
    return lib.rg_algo_name(int(a)).decode()


# --------------------------------------------------------------------------------------
# PyTorch-facing operations (repro_torch/src/bindings.cpp:43-66): the compiled binding
# (_backend, csrc/rg_torch.cpp) runs GPU tensors on the library and CPU tensors on the CPU
# implementation of the same definition.
# --------------------------------------------------------------------------------------
_backend.set_error_class(ReproGemmError)


def workspace(torch, nbytes, device):
    """A uint8 device buffer of nbytes for one call, from PyTorch's caching allocator on the
    current stream: the allocator gives it to no other stream's work while this call's kernels
    may still use it, so calls on different streams (or overlapping a graph replay) never share
    a workspace."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def gemm(A, B, M, N, K, ta=False, tb=False, S=3, cfg=None, out=None):
    """C[M, N] = op(A) op(B) for float32 tensors, both on one GPU (on the current stream) or
    both on the CPU (the CPU implementation; the same bits).

    Same argument meaning and checks as the reference binding: A holds M*K values (K x M if
    ta), B holds N*K values (N x K if tb). cfg (a Config) replaces ta, tb and S and adds the
    planner's options (split_k, block tile, algorithm), which never change a bit. out, if
    given, must be a contiguous float32 tensor of M*N elements on the inputs' device.
    """
    if cfg is None:
        return _backend.gemm_ex(A, B, int(M), int(N), int(K), bool(ta), bool(tb), int(S), 1, 16, 16,
                                int(Algo.Auto), out)
    return _backend.gemm_ex(A, B, int(M), int(N), int(K), bool(cfg.trans_a), bool(cfg.trans_b),
                            int(cfg.slices), int(cfg.split_k), int(cfg.tile_m), int(cfg.tile_n),
                            int(cfg.algo), out)


def bmm(A, B, ta=False, tb=False, S=3, cfg=None, out=None):
    """C[b] = op(A[b]) op(B[b]) for 3-D float32 GPU tensors, each item bit-identical to gemm()
    on that item alone (its own row and column scales); on the current stream.

    A is [batch, M, K] ([batch, K, M] if ta) and B is [batch, K, N] ([batch, N, K] if tb). They
    may be strided views whose last dimension is contiguous (for example one attention head per
    item of a [T, H * D] activation): the library reads them in place through leading
    dimensions and batch strides. A batch dimension of size 1 broadcasts. C is [batch, M, N];
    out, if given, must be a float32 [batch, M, N] tensor on A's device with a contiguous last
    dimension. CPU tensors run gemm() item by item. cfg (a Config), if given, replaces ta, tb and
    S as in gemm(): the shapes are read with cfg's transposes.
    """
    import torch

    if cfg is not None:
        ta, tb = bool(cfg.trans_a), bool(cfg.trans_b)
    if A.dim() != 3 or B.dim() != 3:
        raise ValueError("bmm: A and B must be 3-D")
    if A.dtype != torch.float32 or B.dtype != torch.float32:
        raise ValueError("bmm: A and B must be float32")
    if A.device != B.device:
        raise ValueError("bmm: A and B must be on the same device")
    batch = max(A.shape[0], B.shape[0])
    if A.shape[0] not in (1, batch) or B.shape[0] not in (1, batch):
        raise ValueError("bmm: batch sizes differ")
    M, K = (A.shape[2], A.shape[1]) if ta else (A.shape[1], A.shape[2])
    Kb, N = (B.shape[2], B.shape[1]) if tb else (B.shape[1], B.shape[2])
    if Kb != K:
        raise ValueError("bmm: shape mismatch")
    if cfg is None:
        cfg = Config(slices=S, trans_a=bool(ta), trans_b=bool(tb))
    if out is not None:
        if out.dtype != torch.float32 or out.device != A.device:
            raise ValueError("bmm: out must be float32 on the inputs' device")
        if tuple(out.shape) != (batch, M, N) or out.stride(2) != 1:
            raise ValueError("bmm: out must be [batch, M, N] with a contiguous last dimension")
    if not A.is_cuda:
        C = out if out is not None else torch.empty((batch, M, N), dtype=torch.float32)
        for b in range(batch):
            a = A[b if A.shape[0] > 1 else 0]
            bb = B[b if B.shape[0] > 1 else 0]
            C[b] = gemm(a, bb, M, N, K, cfg=cfg)
        return C
    if A.stride(2) != 1:
        A = A.contiguous()
    if B.stride(2) != 1:
        B = B.contiguous()
    stride_a = A.stride(0) if A.shape[0] > 1 else 0
    stride_b = B.stride(0) if B.shape[0] > 1 else 0
    plan = make_plan_strided_batched(M, N, K, batch, cfg)
    C = out if out is not None else torch.empty((batch, M, N), dtype=torch.float32, device=A.device)
    ws = workspace(torch, plan.workspace_bytes, A.device)
    stream = torch.cuda.current_stream(A.device).cuda_stream
    code = repro_gemm_strided_batched_fp32_ws(A.data_ptr(), A.stride(1), stride_a, B.data_ptr(),
                                              B.stride(1), stride_b, C.data_ptr(), C.stride(1),
                                              C.stride(0), M, N, K, batch, cfg, ws.data_ptr(),
                                              ws.numel(), stream)
    _check(code, "bmm")
    return C
