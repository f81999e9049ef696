"""Python mirror of the reproducible convolution.

Names and argument meaning follow repro_conv_cuda/repro_conv.cuh:19-31 (ConvShape,
conv2d_workspace, conv2d_grad_weight_workspace, conv2d_grad_input_workspace, repro_conv2d_ws,
repro_conv2d_grad_weight_ws, repro_conv2d_grad_input_ws) and the PyTorch bindings
repro_torch/src/bindings.cpp:97-175 (conv2d, conv2d_grad_weight, conv2d_grad_input).
GPU work runs through the C ABI of librepro_gemm.so (include/repro_conv.h); the tensor
operations go through the compiled binding _backend, which runs CPU tensors on the CPU
implementation (include/repro_conv_cpu.h) with the same bits.
"""
import ctypes
from dataclasses import dataclass

from . import _lib
from ._lib import _backend, lib
from .repro_gemm import _check


@dataclass
class ConvShape:
    """repro_conv_math.cuh:29-42: input [N][C][H][W], weight [F][C][KH][KW]."""
    N: int
    C: int
    H: int
    W: int
    F: int
    KH: int
    KW: int
    SY: int = 1
    SX: int = 1
    PY: int = 0
    PX: int = 0

    @property
    def OH(self):
        return (self.H + 2 * self.PY - self.KH) // self.SY + 1

    @property
    def OW(self):
        return (self.W + 2 * self.PX - self.KW) // self.SX + 1

    def to_c(self):
        return _lib.rg_conv_shape(self.N, self.C, self.H, self.W, self.F, self.KH, self.KW,
                                  self.SY, self.SX, self.PY, self.PX)

    def astuple(self):
        return (self.N, self.C, self.H, self.W, self.F, self.KH, self.KW, self.SY, self.SX,
                self.PY, self.PX)


def _ws_query(fn, g, S, what):
    n = ctypes.c_size_t()
    c = g.to_c()
    _check(fn(ctypes.byref(c), int(S), ctypes.byref(n)), what)
    return n.value


def conv2d_workspace(g, S=3):
    return _ws_query(lib.rg_conv2d_workspace, g, S, "conv plan")


def conv2d_grad_weight_workspace(g, S=3):
    return _ws_query(lib.rg_conv2d_grad_weight_workspace, g, S, "conv plan")


def conv2d_grad_input_workspace(g, S=3):
    return _ws_query(lib.rg_conv2d_grad_input_workspace, g, S, "conv plan")


def _run(fn, a, b, out, g, S, workspace, workspace_bytes, stream):
    c = g.to_c()
    return fn(a, b, out, ctypes.byref(c), int(S), workspace, int(workspace_bytes), stream)


def repro_conv2d_ws(x, weight, out, g, S, workspace, workspace_bytes, stream=None):
    """Raw-pointer entry points (repro_conv.cuh:26-31): device addresses as ints, stream a
    hipStream_t handle or None. Return the hipError_t code."""
    return _run(lib.rg_conv2d_ws, x, weight, out, g, S, workspace, workspace_bytes, stream)


def repro_conv2d_grad_weight_ws(dy, x, dw, g, S, workspace, workspace_bytes, stream=None):
    return _run(lib.rg_conv2d_grad_weight_ws, dy, x, dw, g, S, workspace, workspace_bytes, stream)


def repro_conv2d_grad_input_ws(dy, weight, dx, g, S, workspace, workspace_bytes, stream=None):
    return _run(lib.rg_conv2d_grad_input_ws, dy, weight, dx, g, S, workspace, workspace_bytes,
                stream)


# Passes and algorithms of the diagnostic hooks (include/repro_conv.h): AUTO is what the entry
# points above choose, GEMM the im2col + MFMA GEMM pipeline, DIRECT the one-launch kernels for
# small filters (forward and input gradient).
FORWARD, GRAD_WEIGHT, GRAD_INPUT = 0, 1, 2
ALGO_AUTO, ALGO_GEMM, ALGO_DIRECT = 0, 1, 2


def conv2d_algo(pass_, g, S=3):
    """The algorithm AUTO resolves to for this pass and shape (ALGO_GEMM or ALGO_DIRECT)."""
    a = ctypes.c_int()
    c = g.to_c()
    _check(lib.rg_conv2d_algo(int(pass_), ctypes.byref(c), int(S), ctypes.byref(a)), "conv algo")
    return a.value


def conv2d_algo_workspace(pass_, g, S=3, algo=ALGO_AUTO):
    n = ctypes.c_size_t()
    c = g.to_c()
    _check(lib.rg_conv2d_algo_workspace(int(pass_), ctypes.byref(c), int(S), int(algo),
                                        ctypes.byref(n)), "conv plan")
    return n.value


def repro_conv2d_algo_ws(pass_, a, b, out, g, S, algo, workspace, workspace_bytes, stream=None):
    """A pass with its algorithm forced (raw pointers as the entry points above)."""
    c = g.to_c()
    return lib.rg_conv2d_algo_ws(int(pass_), a, b, out, ctypes.byref(c), int(S), int(algo),
                                 workspace, int(workspace_bytes), stream)


def conv2d(x, w, SY, SX, PY, PX, S=3):
    """out[N][F][OH][OW] from x[N][C][H][W] and w[F][C][KH][KW] (bindings.cpp:112-131), on the
    tensors' GPU (current stream) or on the CPU (same bits)."""
    return _backend.conv2d(x, w, int(SY), int(SX), int(PY), int(PX), int(S))


def conv2d_grad_weight(dy, x, KH, KW, SY, SX, PY, PX, S=3):
    """dW[F][C][KH][KW] from dY[N][F][OH][OW] and x (bindings.cpp:133-152)."""
    return _backend.conv2d_grad_weight(dy, x, int(KH), int(KW), int(SY), int(SX), int(PY),
                                       int(PX), int(S))


def conv2d_grad_input(dy, w, x_shape, SY, SX, PY, PX, S=3):
    """dX[N][C][H][W] (x_shape) from dY[N][F][OH][OW] and w (bindings.cpp:154-175)."""
    return _backend.conv2d_grad_input(dy, w, [int(v) for v in x_shape], int(SY), int(SX),
                                      int(PY), int(PX), int(S))


__all__ = ["ALGO_AUTO", "ALGO_DIRECT", "ALGO_GEMM", "FORWARD", "GRAD_INPUT", "GRAD_WEIGHT",
           "conv2d_algo", "conv2d_algo_workspace", "repro_conv2d_algo_ws",
           "ConvShape", "conv2d", "conv2d_grad_input", "conv2d_grad_weight",
           "conv2d_grad_input_workspace", "conv2d_grad_weight_workspace", "conv2d_workspace",
           "repro_conv2d_grad_input_ws", "repro_conv2d_grad_weight_ws", "repro_conv2d_ws"]
