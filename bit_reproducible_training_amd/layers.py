"""Reproducible layers as custom autograd functions, on the MI355X kernels.

Mirrors repro_torch/repro_torch/layers.py:1-136 (set_slices, get_slices, FiniteGuard, guard,
name_layers, Linear, Conv2d): same names, argument meaning, results and errors. Every product
goes through the reproducible GEMM or convolution (one rounding of an exact sum of 7*S-bit
products; S = 3 by default), every bias gradient through the exact sum, so a training step
gives the same bits on every run and every GPU that runs these kernels, and the same bits as
the reference. GPU tensors only: the kernels have no CPU path.
"""
import torch

from .repro_conv import conv2d, conv2d_grad_input, conv2d_grad_weight
from .repro_gemm import gemm
from .repro_sum import exact_sum, scan_finite

_slices = 3


def set_slices(s):
    """Sets S for every GEMM: 7*S-bit inputs (21 bits at the default S = 3)."""
    global _slices
    if s not in (1, 2, 3):
        raise ValueError("slices must be 1, 2 or 3")
    _slices = s


def get_slices():
    return _slices


class FiniteGuard:
    """Stops training with a clear error once a NaN or infinity reaches a GEMM or convolution.

    The integer conversion inside the GEMM is undefined for such values, so results past that
    point could differ between machines (layers.py:21-27). Scans are queued on the stream with
    the operation and need no synchronisation; check() reads the flag once per step, so the
    error arrives at the same step everywhere.
    """

    _NONE = 2 ** 31 - 1

    def __init__(self):
        self._names = []
        self._ids = {}
        self._flag = None

    def _id(self, name):
        if name not in self._ids:
            self._ids[name] = len(self._names)
            self._names.append(name)
        return self._ids[name]

    def scan(self, x, name):
        if self._flag is None or self._flag.device != x.device:
            self._flag = torch.full((1,), self._NONE, dtype=torch.int32, device=x.device)
        scan_finite(x, self._flag, self._id(name))

    def check(self, step=None):
        """Raises FloatingPointError naming the first operation (in order of first use) that
        saw a NaN or infinity since the guard was created or reset."""
        if self._flag is None:
            return
        found = int(self._flag.item())
        if found != self._NONE:
            where = "" if step is None else " at step %d" % step
            raise FloatingPointError("non-finite value reached %s%s" % (self._names[found], where))

    def reset(self):
        """Clears the flag (a fill kernel on the flag's stream), keeping the names."""
        if self._flag is not None:
            self._flag.fill_(self._NONE)


_guard = FiniteGuard()


def guard():
    return _guard


def name_layers(model, prefix=""):
    """Names layers after their place in the model, for error messages."""
    for name, m in model.named_modules():
        if isinstance(m, (Linear, Conv2d)):
            m.repro_name = prefix + name
    return model


class _LinearFn(torch.autograd.Function):
    """y = x W^T + b; dX = dY W, dW = dY^T X (reproducible GEMMs), db = exact column sum of
    dY (layers.py:70-93)."""

    @staticmethod
    def forward(ctx, x, weight, bias, name):
        ctx.save_for_backward(x, weight)
        ctx.name = name
        _guard.scan(x, name + " input")
        _guard.scan(weight, name + " weight")
        m, k, n = x.shape[0], weight.shape[1], weight.shape[0]
        y = gemm(x, weight, m, n, k, False, True, _slices)
        return y + bias if bias is not None else y

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        _guard.scan(dy, ctx.name + " gradient")
        m, k, n = x.shape[0], weight.shape[1], weight.shape[0]
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = gemm(dy, weight, m, k, n, False, False, _slices)
        if ctx.needs_input_grad[1]:
            dw = gemm(dy, x, n, k, m, True, False, _slices)
        if ctx.needs_input_grad[2]:
            db = exact_sum(dy, m, n, 1, False)
        return dx, dw, db, None


class Linear(torch.nn.Linear):
    """torch.nn.Linear with reproducible forward and backward (layers.py:96-100). Input is
    [batch, in_features] float32 on the GPU."""

    repro_name = "linear"

    def forward(self, x):
        return _LinearFn.apply(x, self.weight, self.bias, self.repro_name)


class _ConvFn(torch.autograd.Function):
    """y = conv(x, W) (+ b); dX, dW by the reproducible convolution gradients, db = exact sum
    of dY over images and pixels (layers.py:103-126)."""

    @staticmethod
    def forward(ctx, x, weight, bias, stride, padding, name):
        ctx.save_for_backward(x, weight)
        ctx.stride, ctx.padding, ctx.name = stride, padding, name
        _guard.scan(x, name + " input")
        _guard.scan(weight, name + " weight")
        y = conv2d(x, weight, stride[0], stride[1], padding[0], padding[1], _slices)
        return y + bias[None, :, None, None] if bias is not None else y

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        sy, sx = ctx.stride
        py, px = ctx.padding
        _guard.scan(dy, ctx.name + " gradient")
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = conv2d_grad_input(dy, weight, list(x.shape), sy, sx, py, px, _slices)
        if ctx.needs_input_grad[1]:
            dw = conv2d_grad_weight(dy, x, weight.shape[2], weight.shape[3], sy, sx, py, px, _slices)
        if ctx.needs_input_grad[2]:
            db = exact_sum(dy, dy.shape[0], dy.shape[1], dy.shape[2] * dy.shape[3], False)
        return dx, dw, db, None, None, None


class Conv2d(torch.nn.Conv2d):
    """torch.nn.Conv2d with reproducible forward and backward (layers.py:129-136): stride and
    zero padding; groups, dilation and other padding modes raise NotImplementedError."""

    repro_name = "conv2d"

    def forward(self, x):
        if self.groups != 1 or self.dilation != (1, 1) or isinstance(self.padding, str) or \
                self.padding_mode != "zeros":
            raise NotImplementedError("Conv2d supports stride and zero padding only")
        return _ConvFn.apply(x, self.weight, self.bias, self.stride, self.padding, self.repro_name)


__all__ = ["Conv2d", "FiniteGuard", "Linear", "get_slices", "guard", "name_layers", "set_slices"]
