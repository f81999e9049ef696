"""GEMM inputs holding NaN or infinities, on the CPU.

The definition is meant for finite inputs (the reference's hash tool refuses others,
hash_repro_gemm.cu:96-98), but the reference's CPU path still gives a result, and that result is
what every path here reproduces: the row and column maxima skip NaN (std::fmax,
repro_gemm_cpu.h:30-31, 36-37) and keep infinities, and fixed_point's (int)nearbyintf turns a
NaN or an infinity into INT_MIN on x86, clamped to -127 * 2^(7(S-1)) (repro_gemm_math.cuh:71-83).
The oracle is pinned against the reference's own CPU path compiled from its sources
(oracle/_ref, when built) and against two cases worked out by hand; the library's CPU path
(the compiled binding over include/repro_gemm_cpu.h) must give the same bits.
"""
import numpy as np
import pytest

from oracle import oracle as O


def nonfinite_inputs(M, N, K, seed):
    """N(0,1) operands with NaN and infinities planted in a few rows of A and columns of B:
    a lone +inf, a lone -inf, a lone NaN, a whole NaN row, NaN and +inf in one row, and in B a
    NaN and a -inf. A is M x K and B is N x K in memory; with transposes the same values land
    in other rows and columns, which the tests also run."""
    rng = np.random.default_rng(seed)
    A = rng.standard_normal(M * K).astype(np.float32)
    B = rng.standard_normal(N * K).astype(np.float32)
    A[3 * K + 5] = np.inf
    A[4 * K + 7] = -np.inf
    A[5 * K + 1] = np.nan
    A[6 * K:7 * K] = np.nan
    A[8 * K + 2] = np.nan
    A[8 * K + 9] = np.inf
    B[2 * K + 4] = np.nan
    B[11 * K + 3] = -np.inf
    return A, B


TRANSPOSES = [(0, 0), (1, 0), (0, 1), (1, 1)]


@pytest.mark.parametrize("S", [1, 2, 3])
def test_oracle_matches_reference_cpu_path_on_nonfinite_inputs(S):
    if O.ref is None:
        pytest.skip("oracle/_ref (the reference's CPU path) is not built here")
    M, N, K = 37, 29, 53
    A, B = nonfinite_inputs(M, N, K, 5)
    for ta, tb in TRANSPOSES:
        want = np.asarray(O.ref_cpu_gemm(A, B, M, N, K, ta, tb, S)).view(np.uint32).ravel()
        got = O.cpu_gemm(A, B, M, N, K, ta, tb, S).view(np.uint32).ravel()
        assert np.array_equal(got, want), (ta, tb)


def test_oracle_nonfinite_hand_cases():
    """Two GEMMs worked out by hand at S = 3 (lim = 127 * 2^14).
    A = [inf], B = [1]: e_A = scale_exponent(inf) = 128, X = -lim; e_B = -6 (1/127 <= 2^-6),
    Y = 2^20; T = -127 * 2^34 and E = 128 - 6 - 28 = 94, so C = -127 * 2^128 = -inf.
    A = [NaN, 2], B = [1, 0]: the maximum skips NaN, e_A = -5 (2/127 <= 2^-5), X = [-lim, 2^20];
    T = -127 * 2^34 and E = -5 - 6 - 28 = -39, so C = -127 / 32."""
    C = O.cpu_gemm(np.array([np.inf], np.float32), np.array([1.0], np.float32), 1, 1, 1, 0, 0, 3)
    assert np.isneginf(np.asarray(C).ravel()[0])
    C = O.cpu_gemm(np.array([np.nan, 2.0], np.float32), np.array([1.0, 0.0], np.float32), 1, 1, 2, 0, 0, 3)
    assert np.asarray(C).ravel()[0] == np.float32(-127.0 / 32.0)


@pytest.mark.parametrize("S", [1, 2, 3])
def test_cpu_path_matches_oracle_on_nonfinite_inputs(S):
    import torch

    import bit_reproducible_training_amd as rg

    for M, N, K in [(37, 29, 53), (70, 90, 1100)]:
        A, B = nonfinite_inputs(M, N, K, 6 + S)
        tA, tB = torch.from_numpy(A), torch.from_numpy(B)
        for ta, tb in TRANSPOSES:
            want = O.cpu_gemm(A, B, M, N, K, ta, tb, S).view(np.uint32).ravel()
            got = rg.gemm(tA, tB, M, N, K, ta=bool(ta), tb=bool(tb), S=S).numpy().view(np.uint32).ravel()
            assert np.array_equal(got, want), (M, N, K, ta, tb)


CONV_SHAPE = (2, 3, 9, 9, 4, 3, 3, 1, 1, 1, 1)


def conv_nonfinite_inputs(shape, seed, nan=True):
    """x, w and dy of a convolution with infinities (and, if nan, NaN) planted in each."""
    rng = np.random.default_rng(seed)
    N, C, H, W, F, KH, KW = shape[:7]
    OH, OW = O.conv_out_hw(shape)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = rng.standard_normal((F, C, KH, KW)).astype(np.float32)
    dy = rng.standard_normal((N, F, OH, OW)).astype(np.float32)
    x[1, 0, 2, 7] = np.inf
    x[1, C - 1, H - 1, 0] = -np.inf
    dy[N - 1, 0, 1, 1] = np.inf
    if nan:
        x[0, 1, 4, 4] = np.nan
        w[F // 2, 1, 0, KW - 1] = np.nan
        dy[0, F - 1, OH // 2, OW // 2] = np.nan
    return x, w, dy


def _conv_cpu(kind, x, w, dy, shape, S):
    import torch

    import bit_reproducible_training_amd as rg

    N, C, H, W, F, KH, KW, SY, SX, PY, PX = shape
    t = torch.from_numpy
    if kind == "fwd":
        return rg.conv2d(t(x), t(w), SY, SX, PY, PX, S).numpy()
    if kind == "dW":
        return rg.conv2d_grad_weight(t(dy), t(x), KH, KW, SY, SX, PY, PX, S).numpy()
    return rg.conv2d_grad_input(t(dy), t(w), (N, C, H, W), SY, SX, PY, PX, S).numpy()


def conv_oracle(kind, x, w, dy, shape, S):
    if kind == "fwd":
        return O.conv2d(x, w, shape, S)
    if kind == "dW":
        return O.conv2d_grad_weight(dy, x, shape, S)
    return O.conv2d_grad_input(dy, w, shape, S)


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32).ravel()


@pytest.mark.parametrize("S", [1, 3])
def test_conv_cpu_path_matches_oracle_on_nonfinite_inputs(S):
    """The window maxima (forward) and position maxima (weight gradient) compare magnitude
    bits, so a NaN wins them and that window or position takes exponent 0; the filter, dY and
    weight maxima skip NaN; infinities and the -127 * 2^(7(S-1)) of a non-finite value are as
    in the GEMM."""
    x, w, dy = conv_nonfinite_inputs(CONV_SHAPE, 20 + S)
    for kind in ("fwd", "dW", "dX"):
        assert np.array_equal(_bits(_conv_cpu(kind, x, w, dy, CONV_SHAPE, S)),
                              _bits(conv_oracle(kind, x, w, dy, CONV_SHAPE, S))), kind


@pytest.mark.parametrize("nan", [False, True])
@pytest.mark.parametrize("S", [1, 2, 3])
def test_conv_oracle_matches_reference_on_nonfinite_inputs(S, nan):
    """The oracle's convolution gives the reference convolution's own bits (oracle/_ref) with
    infinities, and with NaN in x, the weights and dY."""
    if O.ref is None:
        pytest.skip("oracle/_ref (the reference's CPU path) is not built here")
    for seed in range(3):
        x, w, dy = conv_nonfinite_inputs(CONV_SHAPE, 30 + 4 * S + seed, nan=nan)
        for kind, a, b in (("fwd", x, w), ("dW", dy, x), ("dX", dy, w)):
            assert np.array_equal(_bits(O.ref_conv(kind, a, b, CONV_SHAPE, S)),
                                  _bits(conv_oracle(kind, x, w, dy, CONV_SHAPE, S))), (kind, seed)


def test_conv_oracle_nan_window_takes_exponent_zero():
    """Hand case: 1x1 image row [NaN, 2, 1, 0.5] (N=1, C=1, H=1, W=4), one 1x2 filter [1, 1],
    stride 1, no padding, S=1. Windows [NaN, 2] and [2, 1], [1, 0.5]. The first window's maximum
    is the NaN, exponent 0: X = [-127, 2 * 2^0 -> 2], so y0 = round((-127 + 2) * 2^(e_f)) with
    the filter's e_f = -6 (1/127 <= 2^-6), Wq = [64, 64], sum = -125 * 64 = -8000, times
    2^(0 - 6) = -125. The second window: max 2, e = -5, X = [64, 32], sum = 96 * 64 = 6144,
    times 2^(-11) = 3.0. The third: max 1, e = -6, X = [64, 32], sum 6144 * 2^-12 = 1.5.
    Skipping the NaN instead would give the first window e = -5 and y0 = (-127 + 64) * 64 * 2^-11
    = -1.96875."""
    x = np.array([np.nan, 2.0, 1.0, 0.5], np.float32).reshape(1, 1, 1, 4)
    w = np.ones((1, 1, 1, 2), np.float32)
    shape = (1, 1, 1, 4, 1, 1, 2, 1, 1, 0, 0)
    y = np.asarray(O.conv2d(x, w, shape, 1), np.float32).ravel()
    assert y.tolist() == [-125.0, 3.0, 1.5]
