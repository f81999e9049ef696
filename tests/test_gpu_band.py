"""The band kernel (contract_band: a block slices 32 rows of op(A) into LDS and contracts them
with every column tile of its column group, op(B)'s digits streamed from the caches) against the
oracle, bit for bit.

A pinned 32 x W tile (W >= 64, a multiple of 32) asks for it when op(A) is read along rows and
K <= 1024. Covered: the GPT-2 layer shapes of BASELINE configuration 3 that take it (forward and
input gradient at K = 768, both transposes of op(B)); ragged rows, columns and K (no multiple of
32, 16 or 4), several column groups and a W that does not divide N; rows that are not 16-byte
aligned; S = 1, 2, 3; the hash tool's input distributions; NaN and infinities in both operands;
the stress pattern (overflow to infinity, -0.0); equality with the 64x64 pipeline's bits on the
same inputs; and a second call on a workspace holding the first call's data.
"""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import bits, decode_digits, note, run, to_dev
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _band_cfg(W, S=3, tb=False):
    return rg.Config(slices=S, trans_b=bool(tb), tile_m=32, tile_n=W)


def _inputs(M, N, K, tb, seed):
    rng = np.random.default_rng(seed)
    A = rng.standard_normal(M * K).astype(np.float32)
    B = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    return A, B


# (M, N, K, W): GPT-2 shapes at 8192 tokens, then ragged ones
SHAPES = [(8192, 768, 768, 768), (8192, 768, 768, 384), (4096, 2304, 768, 1152),
          (1000, 300, 100, 128), (97, 70, 203, 64), (33, 65, 1024, 96), (64, 64, 1, 64),
          (2048, 130, 767, 160), (300, 1000, 513, 512), (31, 200, 64, 224)]


@pytest.mark.parametrize("M,N,K,W", SHAPES)
@pytest.mark.parametrize("tb", [0, 1])
def test_band_shapes_against_the_oracle(torch_gpu, M, N, K, W, tb):
    torch = torch_gpu
    A, B = _inputs(M, N, K, tb, M * 3 + N * 5 + K + tb)
    want = O.cpu_gemm(A, B, M, N, K, 0, tb, 3).view(np.uint32)
    note("band M=%d N=%d K=%d W=%d tb=%d" % (M, N, K, W, tb))
    C, plan, ws = run(torch, A, B, M, N, K, _band_cfg(W, 3, tb))
    assert (plan.tile_m, plan.tile_n, plan.split_k) == (32, W, 1)
    assert np.array_equal(bits(C), want), (M, N, K, W, tb)
    # op(B)'s digit panels and exponents, sliced into the workspace by the launch before
    info = rg.workspace_layout(M, N, K, _band_cfg(W, 3, tb))
    _, Y, _, eB = O.quantize(A, B, M, N, K, 0, tb, 3)
    w = ws.cpu().numpy()
    _, Yg = decode_digits(w, info.qb, info.Np, info.Kp, 3)
    assert np.array_equal(Yg[:N, :K], Y) and not Yg[N:, :K].any()
    assert np.array_equal(w[info.eb:info.eb + 4 * info.Np].view(np.int32)[:N], eB)


@pytest.mark.parametrize("S", [1, 2])
@pytest.mark.parametrize("tb", [0, 1])
def test_band_fewer_slices(torch_gpu, S, tb):
    torch = torch_gpu
    for M, N, K, W in ((1000, 300, 100, 128), (4096, 768, 768, 768), (65, 96, 1024, 64)):
        A, B = _inputs(M, N, K, tb, 11 * S + M + K)
        want = O.cpu_gemm(A, B, M, N, K, 0, tb, S).view(np.uint32)
        note("band S=%d M=%d N=%d K=%d W=%d tb=%d" % (S, M, N, K, W, tb))
        C, plan, _ = run(torch, A, B, M, N, K, _band_cfg(W, S, tb))
        assert (plan.tile_m, plan.tile_n) == (32, W)
        assert np.array_equal(bits(C), want), (S, M, N, K, W, tb)


@pytest.mark.parametrize("dist", O.HASH_DISTS)
def test_band_hash_tool_distributions(torch_gpu, dist):
    torch = torch_gpu
    M, N, K = 1024, 256, 768
    for S in (1, 2, 3):
        A, B = O.gen_hash_inputs(M, N, K, 4242, dist)
        want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
        note("band dist=%s S=%d" % (dist, S))
        C, plan, _ = run(torch, A, B, M, N, K, _band_cfg(128, S))
        assert (plan.tile_m, plan.tile_n) == (32, 128)
        assert np.array_equal(bits(C), want), (dist, S)


def test_band_unaligned_rows_and_base(torch_gpu):
    """Rows of op(A) that do not start 16-byte aligned take scalar loads: K % 4 != 0, and a
    base pointer 4 bytes past an aligned one."""
    torch = torch_gpu
    for M, N, K in ((512, 192, 765), (300, 64, 1022), (256, 96, 768)):
        A, B = _inputs(M, N, K, 1, M + N + K)
        want = O.cpu_gemm(A, B, M, N, K, 0, 1, 3).view(np.uint32)
        cfg = _band_cfg(96 if N % 96 == 0 else 64, 3, True)
        note("band unaligned M=%d N=%d K=%d" % (M, N, K))
        C, plan, _ = run(torch, A, B, M, N, K, cfg)
        assert np.array_equal(bits(C), want), (M, N, K)
        store = torch.zeros(M * K + 1, dtype=torch.float32, device="cuda")
        store[1:] = to_dev(torch, A)
        dA = store[1:]  # 4 bytes past the allocation's aligned start
        assert dA.data_ptr() % 16 == 4
        C2, _, _ = run(torch, dA, B, M, N, K, cfg)
        assert np.array_equal(bits(C2), want), ("base+4", M, N, K)


def test_band_nonfinite_inputs(torch_gpu):
    """NaN and infinities in both operands: the maxima skip NaN, a non-finite value rounds to
    -127 * 128^(S-1) (the reference CPU path's bits)."""
    torch = torch_gpu
    M, N, K = 640, 160, 700
    rng = np.random.default_rng(77)
    for S in (1, 2, 3):
        A, B = _inputs(M, N, K, 0, 90 + S)
        A[rng.integers(0, M * K, 40)] = np.nan
        A[rng.integers(0, M * K, 10)] = np.inf
        A[3 * K + 5] = -np.inf
        A[5 * K:6 * K] = np.nan  # a whole row of NaN
        B[rng.integers(0, N * K, 20)] = np.nan
        B[rng.integers(0, N * K, 5)] = -np.inf
        want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
        note("band nonfinite S=%d" % S)
        C, _, _ = run(torch, A, B, M, N, K, _band_cfg(160, S))
        assert np.array_equal(bits(C), want), S


def test_band_stress_overflow_and_negative_zero(torch_gpu):
    from test_oracle import _stress_inputs

    torch = torch_gpu
    rng = np.random.default_rng(23)
    M, N, K = 200, 96, 257
    A, B = _stress_inputs(M, N, K, rng)
    A[7] = np.float32(3e38)
    B[:, 5] = np.float32(2e38)     # row 7 x column 5 overflows
    A[11] = np.float32(-1e-45)
    B[:, 8] = np.float32(1e-45)    # tiny negative products round to -0.0
    for S in (1, 2, 3):
        want = O.cpu_gemm(A.ravel(), B.ravel(), M, N, K, 0, 0, S).view(np.uint32)
        note("band stress S=%d" % S)
        C, _, _ = run(torch, A.ravel(), B.ravel(), M, N, K, _band_cfg(96, S))
        assert np.array_equal(bits(C), want), S


def test_band_equals_pipeline_and_reuses_workspace(torch_gpu):
    """The same bits as the 64x64 pipeline on the same device inputs, and a second band call on
    a workspace (and output) holding the first call's data."""
    torch = torch_gpu
    M, N, K = 4096, 768, 768
    A, B = _inputs(M, N, K, 1, 5)
    dA, dB = to_dev(torch, A), to_dev(torch, B)
    note("band vs pipeline")
    C1, _, ws = run(torch, dA, dB, M, N, K, _band_cfg(768, 3, True))
    C2, p2, _ = run(torch, dA, dB, M, N, K, rg.Config(trans_b=True, tile_m=64, tile_n=64))
    assert (p2.tile_m, p2.tile_n) == (64, 64)
    assert np.array_equal(bits(C1), bits(C2))
    A2, B2 = _inputs(M, N, K, 1, 6)
    want = O.cpu_gemm(A2, B2, M, N, K, 0, 1, 3).view(np.uint32)
    C3, _, _ = run(torch, A2, B2, M, N, K, _band_cfg(768, 3, True), ws=ws, C=C1, poison=False)
    assert np.array_equal(bits(C3), want)
