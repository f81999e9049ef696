"""Reproducible Linear and Conv2d layers for PyTorch autograd, and a NaN/infinity watchdog.

Public names and meaning follow repro_torch/repro_torch/layers.py (set_slices, get_slices,
FiniteGuard, guard, name_layers, Linear, Conv2d), so a model written against the reference
switches by changing its import. The implementation is this package's own.

Gradient mathematics (the definition of the layers' results, shared with the reference):
  Linear   y = x W^T (+ b)      dX = dY W      dW = dY^T x      db = exact sum of dY over rows
  Conv2d   y = conv(x, W) (+ b) dX, dW by the reproducible convolution gradients,
           db = exact sum of dY over images and pixels
Every product is a reproducible GEMM or convolution (one rounding of an exact sum of 7*S-bit
fixed-point products), every bias gradient an exact sum, the bias itself one IEEE addition per
output; so a training step gives the same bits on every run, on the GPU and on the CPU.

Design:
  - Each layer call carries its settings in a small record (_CallInfo: the layer's name, the
    slice count S in force when the forward pass ran, the guard). The backward pass uses that
    record, so changing set_slices() between forward and backward cannot mix slice counts
    inside one step.
  - Inputs and weights are checked for NaN/Inf by the module before the autograd function
    runs, incoming gradients inside backward; the checks are queued kernels (GPU) or a loop
    (CPU) that never synchronise.
  - Linear accepts any number of leading dimensions ([..., in_features]), flattened into the
    GEMM's rows.
"""
from dataclasses import dataclass

import torch

from .repro_conv import conv2d, conv2d_grad_input, conv2d_grad_weight
from .repro_gemm import gemm
from .repro_sum import exact_sum, scan_finite

__all__ = ["Conv2d", "FiniteGuard", "Linear", "get_slices", "guard", "name_layers", "set_slices"]

_state = {"slices": 3}


def set_slices(s):
    """Chooses S for every later layer call: inputs are rounded to 7*S-bit integers (21 bits at
    the default S = 3)."""
    if s not in (1, 2, 3):
        raise ValueError("slices must be 1, 2 or 3")
    _state["slices"] = int(s)


def get_slices():
    return _state["slices"]


class FiniteGuard:
    """Records which watched operation first met a NaN or infinity, and raises on check().

    A NaN or infinity has no fixed-point value, so any result computed from one would not be
    reproducible across machines; training should stop at the step where it appears. Labels
    ("<layer> input", "<layer> weight", "<layer> gradient") are numbered in the order they are
    first watched. Each device gets an int32 cell holding the smallest label number seen
    non-finite there; watching lowers it without any synchronisation, and check() reads the
    cells once, so every machine raises at the same step with the same label.
    """

    CLEAN = 2 ** 31 - 1

    def __init__(self):
        self._numbers = {}   # label -> number, in order of first use
        self._cells = {}     # device -> int32 tensor of one element

    def _number(self, label):
        return self._numbers.setdefault(label, len(self._numbers))

    def _cell(self, device):
        cell = self._cells.get(device)
        if cell is None:
            cell = torch.full((1,), self.CLEAN, dtype=torch.int32, device=device)
            self._cells[device] = cell
        return cell

    def scan(self, tensor, label):
        """Queues a check of `tensor` under `label`."""
        scan_finite(tensor.detach(), self._cell(tensor.device), self._number(label))

    def first_offender(self):
        """The first label (in order of first use) that met a NaN or infinity, or None."""
        worst = min((int(c.item()) for c in self._cells.values()), default=self.CLEAN)
        if worst == self.CLEAN:
            return None
        return next(label for label, n in self._numbers.items() if n == worst)

    def check(self, step=None):
        """Raises FloatingPointError naming the first watched operation that met a NaN or
        infinity since the guard was created or reset; reads the device cells once."""
        label = self.first_offender()
        if label is not None:
            when = "" if step is None else " at step %d" % step
            raise FloatingPointError("NaN or infinity first reached %s%s; results from here on "
                                     "would not be reproducible" % (label, when))

    def reset(self):
        """Marks every device clean again (a fill on each cell's stream), keeping the labels."""
        for cell in self._cells.values():
            cell.fill_(self.CLEAN)


_default_guard = FiniteGuard()


def guard():
    """The guard every layer reports to."""
    return _default_guard


def name_layers(model, prefix=""):
    """Gives every reproducible layer of `model` its path in the model (prefix + the name from
    named_modules()) as repro_name, which the guard's messages use. Returns the model."""
    for path, module in model.named_modules():
        if isinstance(module, (Linear, Conv2d)):
            module.repro_name = prefix + path
    return model


@dataclass(frozen=True)
class _CallInfo:
    name: str
    slices: int
    guard: FiniteGuard


def _watch_operands(info, x, weight):
    info.guard.scan(x, info.name + " input")
    info.guard.scan(weight, info.name + " weight")


class _LinearOp(torch.autograd.Function):
    """x2d [m, in], weight [out, in], bias [out] or None -> y [m, out]."""

    @staticmethod
    def forward(x2d, weight, bias, info):
        m, k = x2d.shape
        y = gemm(x2d, weight, m, weight.shape[0], k, False, True, info.slices)
        return y if bias is None else y + bias

    @staticmethod
    def setup_context(ctx, inputs, output):
        x2d, weight, _, info = inputs
        ctx.save_for_backward(x2d, weight)
        ctx.info = info

    @staticmethod
    def backward(ctx, dy):
        x2d, weight = ctx.saved_tensors
        info = ctx.info
        info.guard.scan(dy, info.name + " gradient")
        dy = dy.contiguous()
        m, k = x2d.shape
        n = weight.shape[0]
        want_x, want_w, want_b, _ = ctx.needs_input_grad
        dx = gemm(dy, weight, m, k, n, False, False, info.slices) if want_x else None
        dw = gemm(dy, x2d, n, k, m, True, False, info.slices) if want_w else None
        db = exact_sum(dy, m, n, 1, False) if want_b else None
        return dx, dw, db, None


class Linear(torch.nn.Linear):
    """torch.nn.Linear whose forward and backward are reproducible. Input [..., in_features]
    float32, on a GPU or on the CPU (the same bits either way)."""

    repro_name = "linear"

    def forward(self, x):
        info = _CallInfo(self.repro_name, get_slices(), _default_guard)
        _watch_operands(info, x, self.weight)
        lead = x.shape[:-1]
        y = _LinearOp.apply(x.reshape(-1, self.in_features), self.weight, self.bias, info)
        return y.reshape(*lead, self.out_features)


class _ConvOp(torch.autograd.Function):
    """x [N, C, H, W], weight [F, C, KH, KW], bias [F] or None -> y [N, F, OH, OW]."""

    @staticmethod
    def forward(x, weight, bias, stride, padding, info):
        y = conv2d(x, weight, stride[0], stride[1], padding[0], padding[1], info.slices)
        return y if bias is None else y + bias.view(1, -1, 1, 1)

    @staticmethod
    def setup_context(ctx, inputs, output):
        x, weight, _, stride, padding, info = inputs
        ctx.save_for_backward(x, weight)
        ctx.geometry = (tuple(stride), tuple(padding))
        ctx.info = info

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        (sy, sx), (py, px) = ctx.geometry
        info = ctx.info
        info.guard.scan(dy, info.name + " gradient")
        dy = dy.contiguous()
        want_x, want_w, want_b = ctx.needs_input_grad[:3]
        dx = dw = db = None
        if want_x:
            dx = conv2d_grad_input(dy, weight, list(x.shape), sy, sx, py, px, info.slices)
        if want_w:
            dw = conv2d_grad_weight(dy, x, weight.shape[2], weight.shape[3], sy, sx, py, px,
                                    info.slices)
        if want_b:
            n, f, oh, ow = dy.shape
            db = exact_sum(dy, n, f, oh * ow, False)
        return dx, dw, db, None, None, None


class Conv2d(torch.nn.Conv2d):
    """torch.nn.Conv2d whose forward and backward are reproducible, for 4-D float32 input on a
    GPU or on the CPU. Supports stride and zero padding (numbers, or "valid"; "same" when the
    stride is 1 and every kernel side is odd); groups, dilation and other padding modes raise
    NotImplementedError."""

    repro_name = "conv2d"

    def _zero_padding(self):
        if self.groups != 1 or tuple(self.dilation) != (1, 1) or self.padding_mode != "zeros":
            raise NotImplementedError("Conv2d supports stride and zero padding only")
        if self.padding == "valid":
            return (0, 0)
        if self.padding == "same":
            kh, kw = self.kernel_size
            if tuple(self.stride) != (1, 1) or kh % 2 == 0 or kw % 2 == 0:
                raise NotImplementedError('padding="same" needs stride 1 and odd kernel sides')
            return ((kh - 1) // 2, (kw - 1) // 2)
        return tuple(self.padding)

    def forward(self, x):
        padding = self._zero_padding()
        if x.dim() != 4:
            raise ValueError("Conv2d expects input [N, C, H, W]")
        info = _CallInfo(self.repro_name, get_slices(), _default_guard)
        _watch_operands(info, x, self.weight)
        return _ConvOp.apply(x, self.weight, self.bias, tuple(self.stride), padding, info)
