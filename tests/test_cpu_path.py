"""The product's CPU implementation (include/repro_gemm_cpu.h, repro_sum_cpu.h,
repro_conv_cpu.h) against the oracle, bit for bit, and the PyTorch binding's CPU branch
(rg.gemm, rg.exact_sum, rg.conv2d*, the layers) on CPU tensors.

The headers are compiled here with g++ alone (tests/cpu_header_shim.cpp: no torch, no HIP),
so they are shown to stand on their own as the drop-in for repro_gemm_cpu.h. The oracle they
are compared with is pinned by the reference's recorded hashes (tests/test_oracle.py); the
GEMM CPU path also reproduces some of those hashes directly here.
"""
import ctypes
import json
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
GOLDEN = os.path.join(HERE, "golden")


@pytest.fixture(scope="module")
def ch(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("ch") / "libch.so")
    subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-pthread", "-ffp-contract=off",
                    "-fno-fast-math", "-Wall", "-Werror", "-I", os.path.join(REPO, "include"),
                    os.path.join(HERE, "cpu_header_shim.cpp"), "-o", out], check=True)
    lib = ctypes.CDLL(out)
    vp, i = ctypes.c_void_p, ctypes.c_int
    lib.ch_threads.restype = i
    lib.ch_for_visits.argtypes = [i, vp]
    lib.ch_gemm.argtypes = [vp, vp, vp, i, i, i, i, i, i]
    lib.ch_gemm.restype = i
    lib.ch_sum.argtypes = [vp, vp, i, i, i, i]
    lib.ch_sum.restype = i
    lib.ch_conv.argtypes = [i, vp, vp, vp, vp, i]
    lib.ch_conv.restype = i
    return lib


@pytest.fixture
def threads(monkeypatch):
    def set_threads(n):
        if n is None:
            monkeypatch.delenv("REPRO_CPU_THREADS", raising=False)
        else:
            monkeypatch.setenv("REPRO_CPU_THREADS", str(n))
    return set_threads


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def header_gemm(ch, A, B, M, N, K, ta, tb, S):
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    C = np.full((M, N), np.nan, np.float32)
    assert ch.ch_gemm(A.ctypes.data, B.ctypes.data, C.ctypes.data, M, N, K, int(ta), int(tb), S) == 0
    return C


# ---------------------------------------------------------------------------------------
# cpu_for
# ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("n", [0, 1, 7, 1000, 100003])
@pytest.mark.parametrize("nt", [None, 1, 3, 8, 64])
def test_cpu_for_calls_every_index_once(ch, threads, n, nt):
    threads(nt)
    visits = np.zeros(max(n, 1), np.int32)
    ch.ch_for_visits(n, visits.ctypes.data)
    assert (visits[:n] == 1).all()


def test_thread_count_override(ch, threads):
    threads(5)
    assert ch.ch_threads() == 5
    threads(None)
    hw = ch.ch_threads()
    assert hw == (os.cpu_count() or 1)
    for bad in ("0", "-3", "abc", "4x", ""):
        threads(bad)
        assert ch.ch_threads() == hw, bad


# ---------------------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------------------

SHAPES = [(1, 1, 1), (7, 5, 3), (33, 17, 65), (64, 64, 64), (130, 67, 301), (5, 300, 1000)]


def operands(M, N, K, ta, tb, seed, dist):
    a_shape = (K, M) if ta else (M, K)
    b_shape = (N, K) if tb else (K, N)
    if dist == "normal":
        A = O.gen_normal(M * K, 1.0, seed).reshape(a_shape)
        B = O.gen_normal(N * K, 0.02, seed + 1).reshape(b_shape)
    else:  # wide magnitudes, zeros, subnormals and near-cancelling pairs
        A = O.gen_adversarial(*a_shape, seed)
        B = O.gen_adversarial(*b_shape, seed + 1, pair_rows=True)
    return A, B


@pytest.mark.parametrize("S", [1, 2, 3])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("dist", ["normal", "adversarial"])
def test_cpu_gemm_matches_oracle(ch, S, ta, tb, dist):
    for i, (M, N, K) in enumerate(SHAPES):
        A, B = operands(M, N, K, ta, tb, 900 + 10 * i, dist)
        got = header_gemm(ch, A, B, M, N, K, ta, tb, S)
        want = O.cpu_gemm(A, B, M, N, K, ta, tb, S)
        assert np.array_equal(bits(got), bits(want)), (M, N, K, ta, tb, S, dist)


def test_cpu_gemm_extreme_rows(ch):
    """Zero rows, rows of 1e30 (results overflow to +-inf), subnormal rows, signed zeros and a
    1e6 outlier, at every S."""
    M, N, K = 9, 11, 37
    rng = np.random.default_rng(3)
    A = rng.standard_normal((M, K)).astype(np.float32)
    A[0] = 0.0
    A[1] = -0.0
    A[2] *= np.float32(1e30)
    mag = rng.integers(1, 1 << 23, K).astype(np.uint32)
    A[3] = (mag | ((rng.random(K) < 0.5).astype(np.uint32) << np.uint32(31))).view(np.float32)
    A[4, 5] = 1e6
    B = rng.standard_normal((K, N)).astype(np.float32)
    B[:, 0] = 0.0
    B[:, 1] *= np.float32(1e30)
    B[:, 2] = np.float32(1e-40)
    for S in (1, 2, 3):
        got = header_gemm(ch, A, B, M, N, K, 0, 0, S)
        want = O.cpu_gemm(A, B, M, N, K, 0, 0, S)
        assert np.array_equal(bits(got), bits(want)), S
    assert np.isinf(got[2, 1])


@pytest.mark.parametrize("nt", [1, 2, 7])
def test_cpu_gemm_thread_count_invariance(ch, threads, nt):
    M, N, K = 97, 83, 211
    A, B = operands(M, N, K, 0, 1, 77, "normal")
    threads(None)
    base = header_gemm(ch, A, B, M, N, K, 0, 1, 3)
    threads(nt)
    assert np.array_equal(bits(header_gemm(ch, A, B, M, N, K, 0, 1, 3)), bits(base))


def suite_ops():
    with open(os.path.join(GOLDEN, "suite_gemm_s3.json")) as f:
        ops = json.load(f)["gemm"]
    # Ops of at most 2.5e9 multiply-adds keep this file within seconds on the CPU; the oracle
    # reproduces all 21 in tests/test_oracle.py.
    return [op for op in ops if op["M"] * op["N"] * op["K"] <= 2.5e9]


@pytest.mark.parametrize("op", suite_ops(), ids=lambda op: op["name"])
def test_cpu_gemm_reproduces_recorded_suite_hashes(ch, op):
    """The reference's GPT-2 suite outputs (gpt2_ops_suite/results/mac/cpu.txt:2-22)."""
    M, N, K = op["M"], op["N"], op["K"]
    A = O.gen_normal(M * K, op["sa"], op["seed"])
    B = O.gen_normal(K * N, op["sb"], op["seed"] + 1)
    assert "%016x" % O.fnv_chain(A, B) == op["in_hash"]
    C = header_gemm(ch, A, B, M, N, K, op["ta"], op["tb"], 3)
    assert "%016x" % O.fnv1a64(C) == op["out_hash"]


def test_cpu_gemm_rejects_bad_arguments(ch):
    A = np.ones(4, np.float32)
    C = np.empty(4, np.float32)
    p = A.ctypes.data
    for M, N, K, S in ((0, 1, 1, 3), (1, -1, 1, 3), (1, 1, 0, 3), (1, 1, 1, 0), (1, 1, 1, 4)):
        assert ch.ch_gemm(p, p, C.ctypes.data, M, N, K, 0, 0, S) == 1
    assert ch.ch_gemm(None, p, C.ctypes.data, 1, 1, 1, 0, 0, 3) == 1
    # K beyond the exact-int64 bound at S = 3 (K * 2089024^2 > 2^62 from K = 1056752).
    K = 1056752
    big = np.zeros(K, np.float32)
    assert ch.ch_gemm(big.ctypes.data, big.ctypes.data, C.ctypes.data, 1, 1, K, 0, 0, 3) == 1
    assert ch.ch_gemm(big.ctypes.data, big.ctypes.data, C.ctypes.data, 1, 1, K - 1, 0, 0, 3) == 0


# ---------------------------------------------------------------------------------------
# Exact sum
# ---------------------------------------------------------------------------------------

def header_sum(ch, x, A, B, C, mean):
    x = np.ascontiguousarray(x, np.float32)
    out = np.full(B, np.nan, np.float32)
    assert ch.ch_sum(x.ctypes.data, out.ctypes.data, A, B, C, int(mean)) == 0
    return out


@pytest.mark.parametrize("mean", [False, True])
def test_cpu_sum_matches_oracle(ch, mean):
    rng = np.random.default_rng(11)
    for A, B, C in ((1, 1, 1), (3, 5, 7), (1, 4, 5000), (300, 3, 1), (17, 6, 49), (2, 1, 70000)):
        x = (rng.standard_normal(A * B * C) * np.exp2(rng.integers(-100, 100, A * B * C))).astype(np.float32)
        assert np.array_equal(bits(header_sum(ch, x, A, B, C, mean)), bits(O.exact_sum(x, A, B, C, mean)))


def test_cpu_sum_special_values(ch):
    cases = [
        [1e30, 1.0, -1e30],                       # exactly 1
        [0.0, -0.0],                              # +0.0
        [-0.0, -0.0],                             # +0.0 (exact zero)
        [np.float32(1e-45), np.float32(1e-45)],   # subnormals
        [3.4e38, 3.4e38],                         # overflow to +inf
        [-3.4e38, -3.4e38],                       # -inf
        [1.0, np.nan],                            # NaN
        [np.inf, -np.inf],                        # NaN
        [1.0, 2.0 ** -24, 2.0 ** -24],            # 1 + 2^-23 (tie broken by the exact sum)
    ]
    for vals in cases:
        x = np.array(vals, np.float32)
        assert np.array_equal(bits(header_sum(ch, x, 1, 1, len(vals), False)),
                              bits(O.exact_sum(x, 1, 1, len(vals), False))), vals
    # Many large terms: carries resolved every 252 additions.
    x = np.full(100001, np.float32(3.0e38))
    x[1::2] = -3.0e38
    x[-1] = 1.0
    assert header_sum(ch, x, 1, 1, x.size, False)[0] == 1.0


def test_cpu_sum_rejects_bad_arguments(ch):
    x = np.ones(4, np.float32)
    out = np.empty(4, np.float32)
    for A, B, C in ((0, 1, 1), (1, 0, 1), (1, 1, -2), (65536, 1, 32768)):
        assert ch.ch_sum(x.ctypes.data, out.ctypes.data, A, B, C, 0) == 1


# ---------------------------------------------------------------------------------------
# Convolution
# ---------------------------------------------------------------------------------------

CONV_SHAPES = [
    (2, 1, 8, 8, 3, 3, 3, 1, 1, 0, 0),
    (3, 2, 9, 7, 4, 3, 2, 2, 1, 1, 0),
    (2, 3, 10, 10, 5, 5, 5, 2, 2, 2, 2),
    (1, 4, 6, 5, 2, 1, 1, 1, 1, 0, 0),
    (2, 2, 7, 7, 3, 4, 4, 3, 3, 3, 1),
    (4, 5, 12, 12, 7, 3, 3, 1, 2, 1, 1),
]
KINDS = {"fwd": 0, "dW": 1, "dX": 2}


def header_conv(ch, kind, a, b, shape, S):
    N, C, H, W, F, KH, KW = shape[:7]
    OH, OW = O.conv_out_hw(shape)
    out_shape = {"fwd": (N, F, OH, OW), "dW": (F, C, KH, KW), "dX": (N, C, H, W)}[kind]
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.full(out_shape, np.nan, np.float32)
    s = np.ascontiguousarray(shape, np.int32)
    assert ch.ch_conv(KINDS[kind], a.ctypes.data, b.ctypes.data, out.ctypes.data, s.ctypes.data, S) == 0
    return out


def conv_inputs(shape, seed):
    N, C, H, W, F, KH, KW = shape[:7]
    OH, OW = O.conv_out_hw(shape)
    x = O.gen_normal(N * C * H * W, 1.0, seed)
    w = O.gen_normal(F * C * KH * KW, 0.1, seed + 1)
    dy = O.gen_normal(N * F * OH * OW, 1e-3, seed + 2)
    return {"fwd": (x, w), "dW": (dy, x), "dX": (dy, w)}


@pytest.mark.parametrize("S", [1, 2, 3])
def test_cpu_conv_matches_oracle(ch, S):
    oracle = {"fwd": O.conv2d, "dW": O.conv2d_grad_weight, "dX": O.conv2d_grad_input}
    for i, shape in enumerate(CONV_SHAPES):
        for kind, (a, b) in conv_inputs(shape, 500 + 10 * i).items():
            got = header_conv(ch, kind, a, b, shape, S)
            want = oracle[kind](a, b, shape, S)
            assert np.array_equal(bits(got), bits(want)), (shape, kind, S)


def test_cpu_conv_reproduces_recorded_lenet_hashes(ch):
    """conv1.fwd, conv1.dW, conv2.fwd, conv2.dW, conv2.dX (gpt2_ops_suite/results/mac/cpu.txt:35-39)."""
    from test_conv import suite_conv_cases

    for case in suite_conv_cases():
        out = header_conv(ch, case["kind"], *case["inputs"], case["shape"], 3)
        assert "%016x" % O.fnv1a64(out) == case["golden"]["out_hash"], case["name"]


def test_cpu_conv_rejects_bad_shapes(ch):
    a = np.ones(4096, np.float32)
    out = np.empty(4096, np.float32)
    for shape in ((0, 1, 4, 4, 1, 3, 3, 1, 1, 0, 0), (1, 1, 2, 2, 1, 3, 3, 1, 1, 0, 0),
                  (1, 1, 4, 4, 1, 3, 3, 0, 1, 0, 0), (1, 1, 4, 4, 1, 3, 3, 1, 1, -1, 0)):
        s = np.ascontiguousarray(shape, np.int32)
        for kind in range(3):
            assert ch.ch_conv(kind, a.ctypes.data, a.ctypes.data, out.ctypes.data, s.ctypes.data, 3) == 1
    s = np.ascontiguousarray(CONV_SHAPES[0], np.int32)
    assert ch.ch_conv(0, a.ctypes.data, a.ctypes.data, out.ctypes.data, s.ctypes.data, 4) == 1


# ---------------------------------------------------------------------------------------
# The PyTorch binding's CPU branch
# ---------------------------------------------------------------------------------------

def test_binding_cpu_gemm_and_checks(ch):
    import torch

    import bit_reproducible_training_amd as rg

    for ta, tb in ((0, 0), (0, 1), (1, 0), (1, 1)):
        M, N, K = 19, 23, 41
        A, B = operands(M, N, K, ta, tb, 1234, "normal")
        got = rg.gemm(torch.from_numpy(A), torch.from_numpy(B), M, N, K, ta, tb, 3)
        assert got.shape == (M, N) and got.dtype == torch.float32
        assert np.array_equal(bits(got.numpy()), bits(O.cpu_gemm(A, B, M, N, K, ta, tb, 3)))
    A = torch.randn(6, 5)
    B = torch.randn(5, 4)
    out = torch.empty(6, 4)
    assert rg.gemm(A, B, 6, 4, 5, out=out) is out
    assert np.array_equal(bits(out.numpy()), bits(O.cpu_gemm(A.numpy(), B.numpy(), 6, 4, 5)))
    # non-contiguous inputs are read as their contiguous copies, as the reference binding does
    At = torch.randn(5, 6).t()
    assert np.array_equal(bits(rg.gemm(At, B, 6, 4, 5).numpy()),
                          bits(O.cpu_gemm(At.contiguous().numpy(), B.numpy(), 6, 4, 5)))
    with pytest.raises(ValueError):
        rg.gemm(A.double(), B, 6, 4, 5)
    with pytest.raises(ValueError):
        rg.gemm(A, B, 6, 4, 6)
    with pytest.raises(ValueError):
        rg.gemm(A, B, 6, 4, 5, out=torch.empty(6, 5))
    with pytest.raises(ValueError):
        rg.gemm(A, B, 6, 4, 5, out=torch.empty(6, 4, dtype=torch.float16))
    with pytest.raises(ValueError):
        rg.gemm(A, B, 6, 4, 5, out=torch.empty(4, 6).t())
    with pytest.raises(ValueError):
        rg.gemm(A, B, 6, 4, 5, S=4)


def test_bmm_cpu_takes_transposes_from_cfg():
    """bmm(..., cfg=Config(trans_b=True)) reads B as [batch, N, K], as gemm() takes cfg's
    transposes; a layout that does not match cfg is refused rather than read out of bounds."""
    import torch

    import bit_reproducible_training_amd as rg

    batch, M, N, K = 2, 5, 7, 9
    for ta, tb in ((0, 1), (1, 0), (1, 1)):
        A = torch.randn(batch, K, M) if ta else torch.randn(batch, M, K)
        B = torch.randn(batch, N, K) if tb else torch.randn(batch, K, N)
        cfg = rg.Config(trans_a=bool(ta), trans_b=bool(tb))
        C = rg.bmm(A, B, cfg=cfg)  # ta, tb left at their defaults: cfg decides
        assert tuple(C.shape) == (batch, M, N)
        for i in range(batch):
            want = O.cpu_gemm(A[i].numpy(), B[i].numpy(), M, N, K, ta, tb, 3)
            assert np.array_equal(bits(C[i].numpy()), bits(want))
    # A [1, 2, 8] with cfg.trans_a: op(A) is 8 x 2, so K = 2 and B [1, 8, 4] does not match
    with pytest.raises(ValueError):
        rg.bmm(torch.randn(1, 2, 8), torch.randn(1, 8, 4), cfg=rg.Config(trans_a=True))


def test_binding_cpu_sum_conv_scan():
    import torch

    import bit_reproducible_training_amd as rg

    x = torch.randn(4, 3, 5)
    for mean in (False, True):
        assert np.array_equal(bits(rg.exact_sum(x, 4, 3, 5, mean).numpy()),
                              bits(O.exact_sum(x.numpy(), 4, 3, 5, mean)))
    shape = CONV_SHAPES[1]
    ins = conv_inputs(shape, 42)
    N, C, H, W, F, KH, KW, SY, SX, PY, PX = shape
    t = {k: (torch.from_numpy(a.copy()), torch.from_numpy(b.copy())) for k, (a, b) in ins.items()}
    OH, OW = O.conv_out_hw(shape)
    y = rg.conv2d(t["fwd"][0].view(N, C, H, W), t["fwd"][1].view(F, C, KH, KW), SY, SX, PY, PX, 3)
    dw = rg.conv2d_grad_weight(t["dW"][0].view(N, F, OH, OW), t["dW"][1].view(N, C, H, W), KH, KW,
                               SY, SX, PY, PX, 3)
    dx = rg.conv2d_grad_input(t["dX"][0].view(N, F, OH, OW), t["dX"][1].view(F, C, KH, KW),
                              [N, C, H, W], SY, SX, PY, PX, 3)
    assert np.array_equal(bits(y.numpy()), bits(O.conv2d(*ins["fwd"], shape)))
    assert np.array_equal(bits(dw.numpy()), bits(O.conv2d_grad_weight(*ins["dW"], shape)))
    assert np.array_equal(bits(dx.numpy()), bits(O.conv2d_grad_input(*ins["dX"], shape)))
    flag = torch.full((1,), 2 ** 31 - 1, dtype=torch.int32)
    rg.scan_finite(torch.ones(10), flag, 3)
    assert int(flag) == 2 ** 31 - 1
    v = torch.ones(10)
    v[7] = float("inf")
    rg.scan_finite(v, flag, 5)
    rg.scan_finite(v, flag, 9)
    assert int(flag) == 5
    with pytest.raises(ValueError):
        rg.conv2d(torch.randn(1, 2, 5, 5), torch.randn(3, 1, 3, 3), 1, 1, 0, 0, 3)
    with pytest.raises(ValueError):
        rg.exact_sum(x, 4, 3, 4, False)
