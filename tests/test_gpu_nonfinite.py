"""GEMM inputs holding NaN or infinities on the GPU: every device route must give the bits of
the reference's CPU path (the oracle), which maps a NaN or an infinity to -127 * 2^(7(S-1)) and
skips NaN in the maxima (see tests/test_nonfinite.py). Routes: the one-launch small kernel, the
one-pass slicing by rows and by columns with 64x64 and 128x128 tiles and split-K, the two-pass
slicing past the one-pass K limit, the one-thread-per-output algorithm, and a strided batch."""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import note, run, to_dev
from oracle import oracle as O
from test_nonfinite import TRANSPOSES, conv_oracle, nonfinite_inputs

pytestmark = pytest.mark.gpu

CASES = [  # M, N, K, S, Config keyword arguments
    (37, 29, 53, 3, {}),
    (37, 29, 53, 1, {}),
    (200, 150, 300, 3, dict(tile_m=64, tile_n=64)),
    (200, 150, 300, 2, dict(tile_m=64, tile_n=64, split_k=3)),
    (600, 520, 900, 3, dict(tile_m=128, tile_n=128)),
    (300, 260, 5000, 3, dict(split_k=2)),
    (90, 70, 400, 3, dict(algo=rg.Algo.Reference)),
]


@pytest.mark.parametrize("M,N,K,S,kw", CASES)
def test_nonfinite_inputs_match_oracle(torch_gpu, M, N, K, S, kw):
    torch = torch_gpu
    A, B = nonfinite_inputs(M, N, K, 11 + K)
    dA, dB = to_dev(torch, A), to_dev(torch, B)
    ws = None
    for ta, tb in TRANSPOSES:
        want = O.cpu_gemm(A, B, M, N, K, ta, tb, S).view(np.uint32).ravel()
        cfg = rg.Config(slices=S, trans_a=ta, trans_b=tb, **kw)
        note("nonfinite", M, N, K, S, ta, tb, kw)
        C, _, ws = run(torch, dA, dB, M, N, K, cfg, ws=ws)
        assert np.array_equal(C.cpu().numpy().view(np.uint32).ravel(), want), (ta, tb)


def test_nonfinite_batched_matches_oracle(torch_gpu):
    torch = torch_gpu
    batch, M, N, K = 3, 70, 50, 200
    items = [nonfinite_inputs(M, N, K, 40 + b) for b in range(batch)]
    A = torch.from_numpy(np.stack([a.reshape(M, K) for a, _ in items])).cuda()
    B = torch.from_numpy(np.stack([b.reshape(N, K) for _, b in items])).cuda()
    note("nonfinite batched", batch, M, N, K)
    C = rg.bmm(A, B, tb=True).cpu().numpy()
    for b, (a, bb) in enumerate(items):
        want = O.cpu_gemm(a, bb, M, N, K, 0, 1, 3).view(np.uint32).ravel()
        assert np.array_equal(C[b].view(np.uint32).ravel(), want), b


@pytest.mark.parametrize("S", [1, 3])
def test_nonfinite_convolution_matches_oracle(torch_gpu, S):
    """Convolutions with NaN and infinities in x, w and dY, by the direct kernels, by the GEMM
    pipeline and by the automatic choice: the oracle's bits (a NaN wins the window and position
    maxima and is skipped by the filter, dY and weight maxima; a non-finite value counts as
    -127 * 2^(7(S-1)))."""
    from test_gpu_conv import RC, _run_algo
    from test_nonfinite import CONV_SHAPE, conv_nonfinite_inputs, conv_oracle

    torch = torch_gpu
    for shape in (CONV_SHAPE, (4, 6, 14, 14, 16, 5, 5, 1, 1, 0, 0)):
        x, w, dy = conv_nonfinite_inputs(shape, 50 + S + shape[1])
        for kind, a, b in (("fwd", x, w), ("dX", dy, w), ("dW", dy, x)):
            want = conv_oracle(kind, x, w, dy, shape, S).view(np.uint32).ravel()
            algos = (RC.ALGO_GEMM, RC.ALGO_AUTO) if kind == "dW" else (RC.ALGO_DIRECT, RC.ALGO_GEMM, RC.ALGO_AUTO)
            for algo in algos:
                note("nonfinite conv", kind, shape, "S=%d algo=%d" % (S, algo))
                got = _run_algo(torch, kind, a.ravel(), b.ravel(), shape, S, algo)
                assert np.array_equal(got.view(np.uint32).ravel(), want), (kind, shape, algo)


# Shapes whose window maxima (forward) and position maxima (weight gradient) go through each
# route: forward gathered in one pass with K = 288 (one wavefront per strip past K = 256), with
# K = 27 and 9 (wave strips), packed with K = 4608 (one read in two parts per 8-row strip) and
# K = 147456 (two passes: 36 parts would be too many); weight gradient over 200 windows (one
# pass), 5000 (one read in parts along the windows) and 40000 (two passes).
NAN_ROUTE_SHAPES = [
    (2, 32, 10, 10, 8, 3, 3, 1, 1, 1, 1), (1, 512, 6, 6, 4, 3, 3, 1, 1, 1, 1),
    (1, 16384, 3, 3, 2, 3, 3, 1, 1, 0, 0), (2, 2, 50, 50, 4, 3, 3, 1, 1, 1, 1),
    (4, 1, 100, 100, 2, 3, 3, 1, 1, 1, 1),
]
DIRECT_FORWARD = {0, 3, 4}  # indices of the shapes the direct forward kernel takes


def _plant_nonfinite(rng, t, count):
    """count NaN and one +inf at random places of t (in place)."""
    flat = t.reshape(-1)
    idx = rng.choice(flat.size, count + 1, replace=False)
    flat[idx[:-1]] = np.nan
    flat[idx[-1]] = np.inf


@pytest.mark.parametrize("S", [1, 3])
@pytest.mark.parametrize("si", range(len(NAN_ROUTE_SHAPES)))
def test_nonfinite_convolution_routes_match_oracle(torch_gpu, S, si):
    """A NaN in x wins the maxima of the windows (forward) and positions (weight gradient) it
    falls in, which then take exponent 0, on every slicing route of both passes, as in the
    reference's convolution (repro_conv_math.cuh:73-86, 121-130); the oracle's convolution is
    pinned to the reference's CPU path on such inputs by the CPU tests."""
    from test_gpu_conv import RC, _run_algo

    torch = torch_gpu
    shape = NAN_ROUTE_SHAPES[si]
    N, C, H, W, F, KH, KW = shape[:7]
    OH, OW = O.conv_out_hw(shape)
    rng = np.random.default_rng(70 + 7 * S + si)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = rng.standard_normal((F, C, KH, KW)).astype(np.float32)
    dy = rng.standard_normal((N, F, OH, OW)).astype(np.float32)
    _plant_nonfinite(rng, x, 3)
    for kind, a, b in (("fwd", x, w), ("dW", dy, x)):
        want = conv_oracle(kind, x, w, dy, shape, S).view(np.uint32).ravel()
        algos = [RC.ALGO_GEMM, RC.ALGO_AUTO]
        if kind == "fwd" and si in DIRECT_FORWARD:
            algos.append(RC.ALGO_DIRECT)
        for algo in algos:
            note("nonfinite conv route", kind, shape, "S=%d algo=%d" % (S, algo))
            got = _run_algo(torch, kind, a.ravel(), b.ravel(), shape, S, algo)
            assert np.array_equal(got.view(np.uint32).ravel(), want), (kind, shape, algo)


@pytest.mark.parametrize("chunk", range(2))
def test_random_shapes_and_plans_with_nonfinite_values(torch_gpu, chunk):
    """The seeded random sweep of shapes and plans (tests/test_gpu_random_shapes.py) on inputs
    with NaN, +inf and -inf sprinkled at random (about 1 in 200 values, and now and then a whole
    row of A or column of B)."""
    from test_gpu_random_shapes import _cases
    from gpu_util import bits

    torch = torch_gpu
    for M, N, K, ta, tb, S, plan, _, seed in _cases(48, 2000 + chunk):
        rng = np.random.default_rng(seed)
        A, B = O.gen_hash_inputs(M, N, K, seed, "normal")
        specials = np.array([np.nan, np.inf, -np.inf], np.float32)
        for X in (A, B):
            hit = rng.random(X.size) < 0.005
            X.reshape(-1)[hit] = rng.choice(specials, int(hit.sum()))
        if rng.random() < 0.3:
            A.reshape(M, K)[int(rng.integers(0, M))] = rng.choice(specials)
        if rng.random() < 0.3:
            B.reshape(K, N)[:, int(rng.integers(0, N))] = rng.choice(specials)
        want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
        As = np.ascontiguousarray(A.reshape(M, K).T) if ta else A
        Bs = np.ascontiguousarray(B.reshape(K, N).T) if tb else B
        cfg = rg.Config(slices=S, trans_a=bool(ta), trans_b=bool(tb), **plan)
        note("random nonfinite M=%d N=%d K=%d ta=%d tb=%d S=%d %s seed=%d" % (M, N, K, ta, tb, S, plan, seed))
        C, got_plan, _ = run(torch, As.ravel(), Bs.ravel(), M, N, K, cfg)
        assert np.array_equal(bits(C), want), (M, N, K, ta, tb, S, plan, seed, got_plan)
