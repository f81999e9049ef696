"""GPU parity: the HIP path (through the C ABI) against the CPU oracle, bit for bit.

Mirrors the reference's correctness suite (repro_gemm_cuda/test_repro_gemm.cu:17-81),
hash tool checks (hash_repro_gemm.cu:79-204) and recorded suite hashes
(gpt2_ops_suite/results/mac/cpu.txt), plus stage-level checks of the slicing kernel
(digits and exponents) and of the contraction (exact int64 products).
"""
import json
import os

import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import bits, decode_digits, hip_events, note, run, to_dev
from oracle import oracle as O

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ALGOS = [rg.Algo.Reference, rg.Algo.Tiled, rg.Algo.TensorCore, rg.Algo.Auto]


def _transposed(A, B, M, N, K, ta, tb):
    At = np.ascontiguousarray(A.reshape(M, K).T) if ta else A
    Bt = np.ascontiguousarray(B.reshape(K, N).T) if tb else B
    return At, Bt


def test_config1_all_algorithms(torch_gpu):
    torch = torch_gpu
    with open(os.path.join(GOLDEN, "baseline_configs.json")) as f:
        fx = {c["name"]: c for c in json.load(f)["cases"]}
    n = 256 * 256
    A = O.gen_normal(n, 1.0, 12345, 0)
    B = O.gen_normal(n, 1.0, 12345, n)
    want = O.cpu_gemm(A, B, 256, 256, 256, 0, 0, 3)
    assert "%016x" % O.fnv1a64(want) == fx["c1.256cube"]["out_hash"]
    for algo in ALGOS:
        note("config1 algo", algo.name)
        C, plan, _ = run(torch, A, B, 256, 256, 256, rg.Config(algo=algo))
        assert np.array_equal(bits(C), want.view(np.uint32)), algo.name


@pytest.mark.parametrize("S", [1, 2, 3])
def test_reference_correctness_suite(torch_gpu, S):
    """test_repro_gemm.cu restated: 133x77x301 (not tile multiples), N(0,1) with one 1e6
    outlier; every algorithm x split_k {1,2,3,7,64} x transposes, plus a repeat run,
    each compared bit for bit with the CPU definition, output poisoned before each run."""
    torch = torch_gpu
    M, N, K = 133, 77, 301
    A = O.gen_normal(M * K, 1.0, 2024, 0)
    B = O.gen_normal(K * N, 1.0, 2024, M * K)
    A[5] = 1e6
    want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
    At, _ = _transposed(A, B, M, N, K, 1, 0)
    _, Bt = _transposed(A, B, M, N, K, 0, 1)
    dA, dB, dAt, dBt = (to_dev(torch, x) for x in (A, B, At, Bt))
    ws = None
    for algo in ALGOS[:3]:
        for split in (1, 2, 3, 7, 64):
            for ta, tb in ((0, 0), (0, 0), (1, 0), (1, 1), (0, 1)):
                note("suite S=%d algo=%s split=%d ta=%d tb=%d" % (S, algo.name, split, ta, tb))
                cfg = rg.Config(algo=algo, slices=S, split_k=split, trans_a=ta, trans_b=tb)
                C, _, ws = run(torch, dAt if ta else dA, dBt if tb else dB, M, N, K, cfg, ws=ws)
                assert np.array_equal(bits(C), want), (algo.name, split, ta, tb)


def test_tile_and_split_invariance(torch_gpu):
    torch = torch_gpu
    M, N, K = 600, 520, 2100
    A = O.gen_normal(M * K, 1.0, 31)
    B = O.gen_normal(N * K, 0.02, 32)
    want = O.cpu_gemm(A, B, M, N, K, 0, 1, 3).view(np.uint32)
    dA, dB = to_dev(torch, A), to_dev(torch, B)
    ws = None
    for tm, tn in ((128, 128), (128, 64), (64, 128), (64, 64), (64, 192), (192, 64)):
        for split in (1, 2, 5, 16, 33):
            note("tiles %dx%d split %d" % (tm, tn, split))
            cfg = rg.Config(tile_m=tm, tile_n=tn, split_k=split, trans_b=True)
            C, plan, ws = run(torch, dA, dB, M, N, K, cfg, ws=ws)
            assert (plan.tile_m, plan.tile_n) == (tm, tn)
            assert np.array_equal(bits(C), want), (tm, tn, split)


@pytest.mark.parametrize("S", [1, 2])
def test_eight_wave_half_tiles_low_slices(torch_gpu, S):
    """The eight-wavefront 128x64 and 64x128 tiles pinned at S = 1 and 2 (the planner offers them
    at S = 3 only), on ragged shapes, every transpose and splits 1 and 3."""
    torch = torch_gpu
    M, N, K = 333, 197, 1500
    A = O.gen_normal(M * K, 1.0, 71 + S)
    B = O.gen_normal(N * K, 0.3, 72 + S)
    dA, dB = to_dev(torch, A), to_dev(torch, B)
    ws = None
    for ta, tb in ((0, 0), (1, 0), (0, 1), (1, 1)):
        want = O.cpu_gemm(A, B, M, N, K, ta, tb, S).view(np.uint32)
        for tm, tn in ((128, 64), (64, 128)):
            for split in (1, 3):
                note("half tiles S=%d %dx%d split %d ta=%d tb=%d" % (S, tm, tn, split, ta, tb))
                cfg = rg.Config(tile_m=tm, tile_n=tn, split_k=split, slices=S, trans_a=ta, trans_b=tb)
                C, plan, ws = run(torch, dA, dB, M, N, K, cfg, ws=ws)
                assert (plan.tile_m, plan.tile_n) == (tm, tn)
                assert np.array_equal(bits(C), want), (ta, tb, tm, tn, split)


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_twelve_wave_tiles_ragged(torch_gpu, ta, tb):
    """The 64x192 and 192x64 tiles (S = 3) on shapes that are no multiple of 192 in either
    direction, with the stress values of the hash tool, every transpose and several splits."""
    from test_oracle import _stress_inputs

    torch = torch_gpu
    rng = np.random.default_rng(50 + 2 * ta + tb)
    for M, N, K in ((200, 391, 777), (450, 70, 1290), (64, 192, 64)):
        A, B = _stress_inputs(M, N, K, rng)
        want = O.cpu_gemm(A.ravel(), B.ravel(), M, N, K, 0, 0, 3).view(np.uint32)
        As = np.ascontiguousarray(A.T) if ta else A
        Bs = np.ascontiguousarray(B.T) if tb else B
        dA, dB = to_dev(torch, As), to_dev(torch, Bs)
        for tm, tn in ((64, 192), (192, 64)):
            for split in (1, 3, 7):
                note("12-wave tiles %dx%d M=%d N=%d K=%d ta=%d tb=%d split=%d" % (tm, tn, M, N, K, ta, tb, split))
                cfg = rg.Config(tile_m=tm, tile_n=tn, split_k=split, trans_a=bool(ta), trans_b=bool(tb))
                C, plan, _ = run(torch, dA, dB, M, N, K, cfg)
                assert (plan.tile_m, plan.tile_n) == (tm, tn)
                assert np.array_equal(bits(C), want), (M, N, K, tm, tn, split)


def _suite():
    with open(os.path.join(GOLDEN, "suite_gemm_s3.json")) as f:
        return json.load(f)


@pytest.mark.parametrize("op", _suite()["gemm"], ids=lambda o: o["name"])
def test_reference_suite_hashes_gpu(torch_gpu, op):
    """The 21 GEMMs of the reference's GPT-2 suite at 1024 tokens, S=3: the GPU output
    hash equals the hash the reference recorded on every CPU and GPU it ran on."""
    torch = torch_gpu
    M, N, K = op["M"], op["N"], op["K"]
    A = O.gen_normal(M * K, op["sa"], op["seed"])
    B = O.gen_normal(K * N, op["sb"], op["seed"] + 1)
    assert "%016x" % O.fnv_chain(A, B) == op["in_hash"]
    note("suite op", op["name"])
    C, _, _ = run(torch, A, B, M, N, K, rg.Config(trans_a=op["ta"], trans_b=op["tb"]))
    assert "%016x" % O.fnv1a64(C.cpu().numpy()) == op["out_hash"]


def test_reference_conv_hashes_gpu(torch_gpu):
    """LeNet conv forward / weight gradient of the suite as GEMMs on im2col (K up to 78400)."""
    from test_oracle import conv_gemm_cases, conv_post

    torch = torch_gpu
    for case in conv_gemm_cases():
        note("conv", case["name"])
        cfg = rg.Config(trans_a=case["ta"], trans_b=case["tb"])
        C, _, _ = run(torch, case["A"], case["B"], case["M"], case["N"], case["K"], cfg)
        out = conv_post(C.cpu().numpy(), case["post"])
        assert "%016x" % O.fnv1a64(out) == case["golden"]["out_hash"], case["name"]


@pytest.mark.parametrize("S", [1, 2, 3])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_slicing_kernel_digits_and_exponents(torch_gpu, S, ta, tb):
    """Stage check of the slice split: the digit panels in the workspace recombine to the
    oracle's fixed-point integers, digits stay in range, exponents equal the oracle's,
    and padding is zero."""
    torch = torch_gpu
    M, N, K = 97, 70, 203
    rng = np.random.default_rng(S * 4 + ta * 2 + tb)
    A = (rng.standard_normal(M * K) * 2.0 ** rng.integers(-30, 30, M * K)).astype(np.float32)
    B = rng.standard_normal(N * K).astype(np.float32)
    A[:K] = 0.0                        # a zero row (or part of a column when ta)
    A[K:2 * K] *= np.float32(2.0 ** -130)  # subnormal values
    X, Y, eA, eB = O.quantize(A, B, M, N, K, ta, tb, S)
    cfg = rg.Config(slices=S, trans_a=ta, trans_b=tb, split_k=2)
    note("slice S=%d ta=%d tb=%d" % (S, ta, tb))
    C, plan, ws = run(torch, A, B, M, N, K, cfg)
    info = rg.workspace_layout(M, N, K, cfg)
    w = ws.cpu().numpy()
    for off, R, Xo, eo, eoff in ((info.qa, info.Mp, X, eA, info.ea), (info.qb, info.Np, Y, eB, info.eb)):
        d, Xg = decode_digits(w, off, R, info.Kp, S)
        assert np.abs(d[0]).max() <= 127
        if S > 1:
            assert d[1:].min() >= 0  # lower digits are the bit fields of X
        assert np.array_equal(Xg[:Xo.shape[0], :K], Xo)
        assert not Xg[Xo.shape[0]:].any() and not Xg[:, K:].any()
        e = w[eoff:eoff + 4 * R].view(np.int32)
        assert np.array_equal(e[:Xo.shape[0]], eo)
        assert not e[Xo.shape[0]:].any()


# Shapes that route the slicing through each of its paths: one pass for rows (padded K <=
# 4096) and columns (padded K <= 3072), with 16-byte or scalar loads, in the wave-strip form
# for padded K <= 256; the fused one-pass + maxima launch when only one operand qualifies (with
# row or column maxima for the other); and two passes.
SLICE_ROUTES = [(96, 68, 1000), (100, 64, 2052), (64, 100, 3076), (68, 96, 4100),
                (96, 64, 1001), (97, 70, 1536), (128, 64, 4096), (96, 68, 200), (97, 70, 61),
                (64, 100, 128), (33, 9, 25),
                # long K, up to the padded K of the reference's tall-skinny case (two passes
                # with several maxima chunks per row), and a K that is no multiple of 4
                (40, 36, 9000), (33, 20, 17000), (9, 40, 40000), (24, 8, 65536), (20, 12, 9001),
                # column access over rows that are not 16-byte aligned (R % 4 != 0), more than 32
                # columns, padded K past the one-pass limits (XCD-paired maxima and split blocks)
                (45, 70, 3500), (301, 203, 5001)]


@pytest.mark.parametrize("M,N,K", SLICE_ROUTES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_slicing_routes_digits_exponents_and_result(torch_gpu, M, N, K, ta, tb):
    """Digits, exponents and padding of both operands, and the GEMM's bits, against the
    oracle on every route of the slicing (S = 3; S = 1 and 2 on the one-pass shapes)."""
    torch = torch_gpu
    rng = np.random.default_rng(M * 7 + N * 3 + K + ta * 2 + tb)
    A = (rng.standard_normal(M * K) * 2.0 ** rng.integers(-20, 20, M * K)).astype(np.float32)
    B = rng.standard_normal(N * K).astype(np.float32)
    A[:K] = 0.0
    for S in ((1, 2, 3) if K in (1000, 2052, 200) else (3,)):
        X, Y, eA, eB = O.quantize(A, B, M, N, K, ta, tb, S)
        # the pipeline's tile pinned: short K would otherwise take the one-launch kernel, which
        # leaves the workspace unused
        cfg = rg.Config(slices=S, trans_a=ta, trans_b=tb, tile_m=64, tile_n=64)
        note("slice route M=%d N=%d K=%d ta=%d tb=%d S=%d" % (M, N, K, ta, tb, S))
        C, plan, ws = run(torch, A, B, M, N, K, cfg)
        info = rg.workspace_layout(M, N, K, cfg)
        w = ws.cpu().numpy()
        for off, R, Xo, eo, eoff in ((info.qa, info.Mp, X, eA, info.ea), (info.qb, info.Np, Y, eB, info.eb)):
            d, Xg = decode_digits(w, off, R, info.Kp, S)
            assert np.abs(d[0]).max() <= 127
            if S > 1:
                assert d[1:].min() >= 0  # lower digits are the bit fields of X
            assert np.array_equal(Xg[:Xo.shape[0], :K], Xo)
            assert not Xg[Xo.shape[0]:].any() and not Xg[:, K:].any()
            e = w[eoff:eoff + 4 * R].view(np.int32)
            assert np.array_equal(e[:Xo.shape[0]], eo)
            assert not e[Xo.shape[0]:].any()
        assert np.array_equal(bits(C), O.cpu_gemm(A, B, M, N, K, ta, tb, S).view(np.uint32))


# Narrow column-access operands (at most 32 columns per item, whose maxima pass reads whole
# rows) over a K too long for the one-pass slicing, with split counts up to one part per
# pipeline stage: the split-K reduction then gives each of the few outputs several threads.
NARROW = [(6, 25, 20000), (1, 3, 9000), (2, 32, 5000), (17, 5, 12345), (32, 32, 8192)]


@pytest.mark.parametrize("M,N,K", NARROW)
@pytest.mark.parametrize("ta,tb", [(1, 0), (0, 0), (1, 1)])
def test_narrow_operands_long_k(torch_gpu, M, N, K, ta, tb):
    torch = torch_gpu
    rng = np.random.default_rng(M * 5 + N * 11 + K + ta * 2 + tb)
    A = (rng.standard_normal(M * K) * 2.0 ** rng.integers(-30, 30, M * K)).astype(np.float32)
    B = rng.standard_normal(N * K).astype(np.float32)
    B[rng.integers(0, N * K, 5)] = 1e20
    X, Y, eA, eB = O.quantize(A, B, M, N, K, ta, tb, 3)
    want = O.cpu_gemm(A, B, M, N, K, ta, tb, 3).view(np.uint32)
    dA, dB = to_dev(torch, A), to_dev(torch, B)
    nsteps = (K + 63) // 64
    for split in (1, 7, 64, nsteps):
        cfg = rg.Config(split_k=split, trans_a=ta, trans_b=tb)
        note("narrow M=%d N=%d K=%d ta=%d tb=%d split=%d" % (M, N, K, ta, tb, split))
        C, plan, ws = run(torch, dA, dB, M, N, K, cfg)
        assert split == 1 or plan.split_k == split
        info = rg.workspace_layout(M, N, K, cfg)
        w = ws.cpu().numpy()
        for R, eo, eoff in ((info.Mp, eA, info.ea), (info.Np, eB, info.eb)):
            assert np.array_equal(w[eoff:eoff + 4 * R].view(np.int32)[:eo.shape[0]], eo)
        _, Xg = decode_digits(w, info.qa, info.Mp, info.Kp, 3)
        assert np.array_equal(Xg[:M, :K], X)
        assert np.array_equal(bits(C), want), (split, plan.split_k)


# Row-access operands of 33-132 values a row through the two-pass slicing (the reference
# algorithm's int32 digits always take it): the maxima pass gives a 16-byte row 16 or 32 lanes
# (several rows per wavefront), and a row of K % 4 != 0 values a whole wavefront. Row scales
# spread over 2^-20 .. 2^20 so every row's own maximum matters.
SHORT_ROWS = [36, 64, 66, 68, 100, 128, 132]


@pytest.mark.parametrize("K", SHORT_ROWS)
def test_row_maxima_short_rows(torch_gpu, K):
    torch = torch_gpu
    M, N = 300, 77
    rng = np.random.default_rng(K)
    A = (rng.standard_normal((M, K)) * 2.0 ** rng.integers(-20, 20, (M, 1))).astype(np.float32).ravel()
    B = (rng.standard_normal((N, K)) * 2.0 ** rng.integers(-20, 20, (N, 1))).astype(np.float32).ravel()
    X, Y, eA, eB = O.quantize(A, B, M, N, K, 0, 1, 3)
    want = O.cpu_gemm(A, B, M, N, K, 0, 1, 3).view(np.uint32)
    dA, dB = to_dev(torch, A), to_dev(torch, B)
    for algo in (rg.Algo.Reference, rg.Algo.TensorCore):
        cfg = rg.Config(algo=algo, trans_b=True, tile_m=64, tile_n=64)  # the pipeline's slicing
        note("short rows K=%d algo=%s" % (K, algo.name))
        C, plan, ws = run(torch, dA, dB, M, N, K, cfg)
        info = rg.workspace_layout(M, N, K, cfg)
        w = ws.cpu().numpy()
        for R, eo, eoff in ((info.Mp, eA, info.ea), (info.Np, eB, info.eb)):
            assert np.array_equal(w[eoff:eoff + 4 * R].view(np.int32)[:eo.shape[0]], eo), algo
        assert np.array_equal(bits(C), want), algo


@pytest.mark.parametrize("split", [2, 3])
def test_contraction_exact_products(torch_gpu, split):
    """Stage check of the contraction: the int64 split-K partials sum to the exact
    integer products T = X Y^T of the oracle."""
    torch = torch_gpu
    M, N, K = 130, 66, 1000
    A = O.gen_normal(M * K, 1.0, 77)
    B = O.gen_normal(N * K, 1.0, 78)
    X, Y, _, _ = O.quantize(A, B, M, N, K, 0, 1, 3)
    T = O.exact_products(X, Y)
    for algo in (rg.Algo.TensorCore, rg.Algo.Tiled, rg.Algo.Reference):
        cfg = rg.Config(algo=algo, split_k=split, trans_b=True)
        note("products algo=%s split=%d" % (algo.name, split))
        C, plan, ws = run(torch, A, B, M, N, K, cfg)
        info = rg.workspace_layout(M, N, K, cfg)
        part = ws.cpu().numpy()[info.part:info.part + 8 * plan.split_k * M * N].view(np.int64)
        assert np.array_equal(part.reshape(plan.split_k, M, N).sum(axis=0), T)


def test_stress_and_extreme_values(torch_gpu):
    """hash_repro_gemm's stress pattern (zero, subnormal, 1e30, outlier and signed-zero
    rows; zero, wide and tiny columns) plus results that overflow to +-inf and round to -0."""
    from test_oracle import _stress_inputs

    torch = torch_gpu
    rng = np.random.default_rng(9)
    M, N, K = 96, 60, 257
    A, B = _stress_inputs(M, N, K, rng)
    A[7] = np.float32(3e38)
    B[:, 5] = np.float32(2e38)     # row 7 x column 5 overflows
    A[11] = np.float32(-1e-45)
    B[:, 8] = np.float32(1e-45)    # tiny negative products round to -0.0
    for S in (1, 2, 3):
        want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
        for algo in ALGOS[:3]:
            note("stress S=%d %s" % (S, algo.name))
            C, _, _ = run(torch, A, B, M, N, K, rg.Config(algo=algo, slices=S))
            assert np.array_equal(bits(C), want)
    assert np.isinf(O.cpu_gemm(A, B, M, N, K, 0, 0, 3)[7, 5])


def test_stage_events_and_streams(torch_gpu):
    torch = torch_gpu
    M, N, K = 512, 512, 1024
    A = O.gen_normal(M * K, 1.0, 5)
    B = O.gen_normal(K * N, 1.0, 6)
    want = O.cpu_gemm(A, B, M, N, K, 0, 0, 3).view(np.uint32)
    s = torch.cuda.Stream()
    ev = hip_events(torch, 4, s)
    with torch.cuda.stream(s):
        dA, dB = to_dev(torch, A), to_dev(torch, B)
        C, _, _ = run(torch, dA, dB, M, N, K, rg.Config(split_k=3),
                      events=[e.cuda_event for e in ev], stream=s.cuda_stream)
    s.synchronize()
    times = [ev[0].elapsed_time(ev[i]) for i in (1, 2, 3)]
    assert 0 <= times[0] <= times[1] <= times[2]
    assert np.array_equal(bits(C), want)


def test_error_codes_on_device(torch_gpu):
    torch = torch_gpu
    M = N = K = 64
    dA = torch.zeros(M * K, device="cuda")
    dC = torch.zeros(M * N, device="cuda")
    plan = rg.make_plan(M, N, K, rg.Config())
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    cfg = rg.Config()
    assert rg.repro_gemm_fp32_ws(dA.data_ptr(), dA.data_ptr(), dC.data_ptr(), M, N, K, cfg,
                                 ws.data_ptr(), plan.workspace_bytes - 1) == 1
    assert rg.repro_gemm_fp32_ws(dA.data_ptr(), dA.data_ptr(), dC.data_ptr(), M, N, K,
                                 rg.Config(slices=4), ws.data_ptr(), ws.numel()) == 1
    assert rg.repro_gemm_fp32(dA.data_ptr(), dA.data_ptr(), dC.data_ptr(), M, N, K, cfg) == 0
    assert rg.repro_gemm_fp32(dA.data_ptr(), dA.data_ptr(), dC.data_ptr(), 0, N, K, cfg) == 1


def test_torch_gemm_binding(torch_gpu):
    """rg.gemm mirrors repro_torch's _backend.gemm: Linear forward, dX and dW."""
    torch = torch_gpu
    B_, fin, fout = 64, 400, 120
    X = O.gen_normal(B_ * fin, 1.0, 1)
    W = O.gen_normal(fout * fin, 0.05, 2)
    dY = O.gen_normal(B_ * fout, 1.0, 3)
    tX, tW, tdY = (torch.from_numpy(v).cuda() for v in (X, W, dY))
    Y = rg.gemm(tX.view(B_, fin), tW.view(fout, fin), B_, fout, fin, False, True, 3)
    dX = rg.gemm(tdY, tW, B_, fin, fout, False, False, 3)
    dW = rg.gemm(tdY, tX, fout, fin, B_, True, False, 3)
    torch.cuda.synchronize()
    assert np.array_equal(bits(Y), O.cpu_gemm(X, W, B_, fout, fin, 0, 1, 3).view(np.uint32))
    assert np.array_equal(bits(dX), O.cpu_gemm(dY, W, B_, fin, fout, 0, 0, 3).view(np.uint32))
    assert np.array_equal(bits(dW), O.cpu_gemm(dY, X, fout, fin, B_, 1, 0, 3).view(np.uint32))
    # non-contiguous input is made contiguous, like the reference binding
    Wt = torch.from_numpy(W.reshape(fout, fin).T.copy()).cuda().t()
    Y2 = rg.gemm(tX, Wt, B_, fout, fin, False, True, 3)
    assert torch.equal(Y2.view(torch.int32), Y.view(torch.int32))
    # CPU tensors run the CPU implementation: the same bits
    Yc = rg.gemm(torch.from_numpy(X), torch.from_numpy(W), B_, fout, fin, False, True, 3)
    assert torch.equal(Yc.view(torch.int32), Y.cpu().view(torch.int32))
    with pytest.raises(ValueError):
        rg.gemm(torch.from_numpy(X), tW, B_, fout, fin, False, True, 3)
