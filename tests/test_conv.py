"""The reproducible convolution on the CPU: the oracle's restatement
(oracle_conv2d, oracle_conv2d_grad_weight, oracle_conv2d_grad_input) against the five LeNet
hashes the reference records, against the GEMM definition on the im2col matrix (forward and
weight gradient; repro_conv_cuda/README.md:5-7), against brute force with Python integers
(input gradient), and against the reference's own repro_conv_cpu.h (oracle/_ref); plus the
shape validation of the C ABI (no kernel launched).
"""
import ctypes
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# The suite's LeNet convolutions (gpt2_ops_suite/gpt2_ops_suite.cu:513-521): seeds follow
# seed += 10 from the suite's start; inputs per make_conv (:432-436).
LENET = {
    "lenet conv1": ((100, 1, 28, 28, 6, 5, 5, 1, 1, 2, 2), {"fwd": 1340, "dW": 1350}),
    "lenet conv2": ((100, 6, 14, 14, 16, 5, 5, 1, 1, 0, 0), {"fwd": 1360, "dW": 1370, "dX": 1380}),
}


def suite_conv_cases():
    with open(os.path.join(GOLDEN, "suite_gemm_s3.json")) as f:
        golden = json.load(f)["conv"]
    cases = []
    for name, (shape, seeds) in LENET.items():
        N, C, H, W, F, KH, KW = shape[:7]
        OH, OW = O.conv_out_hw(shape)
        for kind, seed in seeds.items():
            x = O.gen_normal(N * C * H * W, 1.0, seed)
            w = O.gen_normal(F * C * KH * KW, 0.1, seed + 1)
            dy = O.gen_normal(N * F * OH * OW, 1e-3, seed + 2)
            inputs = {"fwd": (x, w), "dW": (dy, x), "dX": (dy, w)}[kind]
            cases.append(dict(name="%s.%s" % (name, kind), kind=kind, shape=shape, inputs=inputs,
                              golden=golden["%s.%s" % (name, kind)]))
    return cases


def _oracle(kind, a, b, shape, S=3):
    return {"fwd": O.conv2d, "dW": O.conv2d_grad_weight, "dX": O.conv2d_grad_input}[kind](
        a, b, shape, S)


def test_suite_conv_hashes():
    """conv1.fwd, conv1.dW, conv2.fwd, conv2.dW, conv2.dX (cpu.txt:35-39)."""
    for case in suite_conv_cases():
        assert "%016x" % O.fnv_chain(*case["inputs"]) == case["golden"]["in_hash"], case["name"]
        out = _oracle(case["kind"], *case["inputs"], case["shape"])
        assert "%016x" % O.fnv1a64(out) == case["golden"]["out_hash"], case["name"]


def im2col(x, shape):
    """[N*OH*OW][C*KH*KW] windows, zero in the padding (independent of the oracle)."""
    N, C, H, W, F, KH, KW, SY, SX, PY, PX = shape
    OH, OW = O.conv_out_hw(shape)
    xp = np.zeros((N, C, H + 2 * PY, W + 2 * PX), np.float32)
    xp[:, :, PY:PY + H, PX:PX + W] = x.reshape(N, C, H, W)
    cols = np.empty((N, OH, OW, C, KH, KW), np.float32)
    for ky in range(KH):
        for kx in range(KW):
            cols[:, :, :, :, ky, kx] = xp[:, :, ky:ky + SY * OH:SY, kx:kx + SX * OW:SX] \
                .transpose(0, 2, 3, 1)
    return cols.reshape(N * OH * OW, C * KH * KW)


SHAPES = [
    (2, 1, 8, 8, 3, 3, 3, 1, 1, 0, 0),
    (3, 2, 9, 7, 4, 3, 2, 2, 1, 1, 0),
    (2, 3, 10, 10, 5, 5, 5, 2, 2, 2, 2),
    (1, 4, 6, 5, 2, 1, 1, 1, 1, 0, 0),
    (2, 2, 7, 7, 3, 4, 4, 3, 3, 3, 1),
    (4, 5, 12, 12, 7, 3, 3, 1, 2, 1, 1),
]


@pytest.mark.parametrize("S", [1, 2, 3])
@pytest.mark.parametrize("shape", SHAPES)
def test_forward_and_weight_grad_are_gemm_on_im2col(shape, S):
    rng = np.random.default_rng(sum(shape) + S)
    N, C, H, W, F, KH, KW = shape[:7]
    OH, OW = O.conv_out_hw(shape)
    x = rng.standard_normal(N * C * H * W).astype(np.float32)
    w = (rng.standard_normal(F * C * KH * KW) * 0.1).astype(np.float32)
    dy = (rng.standard_normal(N * F * OH * OW) * 1e-3).astype(np.float32)
    cols = im2col(x, shape)
    Wn, K = cols.shape
    y = O.cpu_gemm(cols, w, Wn, F, K, False, True, S).reshape(N, OH, OW, F).transpose(0, 3, 1, 2)
    assert np.array_equal(O.conv2d(x, w, shape, S).view(np.uint32),
                          np.ascontiguousarray(y).view(np.uint32))
    D = np.ascontiguousarray(dy.reshape(N, F, OH * OW).transpose(0, 2, 1).reshape(Wn, F))
    dw = O.cpu_gemm(D, cols, F, K, Wn, True, False, S)
    assert np.array_equal(O.conv2d_grad_weight(dy, x, shape, S).reshape(F, K).view(np.uint32),
                          dw.view(np.uint32))


def _brute_grad_input(dy, w, shape, S):
    """dX by its definition with Python integers: per-image scale of dY, one weight scale,
    exact sums over every (window, filter) touching each pixel."""
    N, C, H, W, F, KH, KW, SY, SX, PY, PX = shape
    OH, OW = O.conv_out_hw(shape)
    dy = dy.reshape(N, F, OH, OW)
    w = w.reshape(F, C, KH, KW)
    eW = int(O.scale_exponent_n(np.array([np.abs(w).max()], np.float32))[0])
    Wq = O.fixed_point_n(w.reshape(-1), eW, S).reshape(F, C, KH, KW).astype(object)
    out = np.empty((N, C, H, W), np.float32)
    for n in range(N):
        eI = int(O.scale_exponent_n(np.array([np.abs(dy[n]).max()], np.float32))[0])
        D = O.fixed_point_n(dy[n].reshape(-1), eI, S).reshape(F, OH, OW).astype(object)
        T = np.zeros((C, H + 2 * PY, W + 2 * PX), object)
        for oy in range(OH):
            for ox in range(OW):
                for f in range(F):
                    T[:, oy * SY:oy * SY + KH, ox * SX:ox * SX + KW] += D[f, oy, ox] * Wq[f]
        T = T[:, PY:PY + H, PX:PX + W]
        E = eI + eW - 14 * (S - 1)
        flat = np.array([int(v) for v in T.reshape(-1)], np.int64)
        out[n] = O.round_to_float_n(flat, E).reshape(C, H, W)
    return out


@pytest.mark.parametrize("S", [1, 3])
@pytest.mark.parametrize("shape", SHAPES[:5])
def test_grad_input_brute_force(shape, S):
    rng = np.random.default_rng(7 * sum(shape) + S)
    N, C, H, W, F, KH, KW = shape[:7]
    OH, OW = O.conv_out_hw(shape)
    w = (rng.standard_normal(F * C * KH * KW) * 0.1).astype(np.float32)
    dy = (rng.standard_normal(N * F * OH * OW) * np.float32(2.0) ** rng.integers(-20, 20)).astype(np.float32)
    got = O.conv2d_grad_input(dy, w, shape, S)
    want = _brute_grad_input(dy, w, shape, S)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("S", [1, 2, 3])
def test_oracle_matches_reference_conv(S):
    if O.ref is None:
        pytest.skip("oracle/_ref not built (reference headers absent)")
    rng = np.random.default_rng(40 + S)
    for shape in SHAPES + [(8, 6, 14, 14, 16, 5, 5, 1, 1, 0, 0)]:
        N, C, H, W, F, KH, KW = shape[:7]
        OH, OW = O.conv_out_hw(shape)
        x = rng.standard_normal(N * C * H * W).astype(np.float32)
        w = (rng.standard_normal(F * C * KH * KW) * 0.1).astype(np.float32)
        dy = (rng.standard_normal(N * F * OH * OW) * 1e-3).astype(np.float32)
        for kind, a, b in (("fwd", x, w), ("dW", dy, x), ("dX", dy, w)):
            want = O.ref_conv(kind, a, b, shape, S)
            got = _oracle(kind, a, b, shape, S)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (shape, kind, S)


# ---------------------------------------------------------------------------------------
# C ABI shape validation (repro_conv_cuda/repro_conv.cu:138-149); no device needed, since
# invalid shapes are rejected before the device is queried.
# ---------------------------------------------------------------------------------------

def test_conv_abi_rejects_invalid_shapes():
    import bit_reproducible_training_amd as rg
    from bit_reproducible_training_amd import _lib

    g = _lib.rg_conv_shape()
    _lib.lib.rg_conv_shape_init(ctypes.byref(g))
    assert (g.SY, g.SX, g.PY, g.PX, g.N) == (1, 1, 0, 0, 0)
    good = (2, 3, 8, 8, 4, 3, 3, 1, 1, 1, 1)
    bad = [
        (0,) + good[1:],                                   # N <= 0
        good[:4] + (0,) + good[5:],                        # F <= 0
        good[:7] + (0,) + good[8:],                        # stride 0
        good[:9] + (-1,) + good[10:],                      # negative padding
        (2, 3, 2, 2, 4, 5, 5, 1, 1, 1, 1),                 # kernel larger than padded image
        (70000, 1, 100, 100, 64, 1, 1, 1, 1, 0, 0),        # output of 2^31 elements or more
        (1000, 1, 46, 46, 1, 1, 1, 1, 1, 0, 0),            # 2,116,000 windows: above the S=3 bound
    ]
    for shape in bad:
        for fn in (rg.conv2d_workspace, rg.conv2d_grad_weight_workspace,
                   rg.conv2d_grad_input_workspace):
            with pytest.raises(rg.ReproGemmError) as e:
                fn(rg.ConvShape(*shape), 3)
            assert e.value.code == 1, (shape, fn.__name__)
    for S in (0, 4):
        with pytest.raises(rg.ReproGemmError):
            rg.conv2d_workspace(rg.ConvShape(*good), S)
    c = rg.ConvShape(*good).to_c()
    assert _lib.lib.rg_conv2d_ws(None, None, None, ctypes.byref(c), 3, None, 0, None) == 1
