"""Row-access operands whose rows are not 16-byte aligned, on every slicing route that reads
rows: the one pass with eight strips per block (K <= 256), the one pass with a strip per block
(K <= 4096), which read such rows by scalar loads, and the one read in parts along K (past 4096),
which reads them by aligned 16-byte loads, each lane taking the values it lacks from the next
lane of its row (the last lane of a row from the first lane's vector of the next k panel), the
loads that would cross either end of a row reading only the values inside it (the first wave of
a row's first part, the last part). The misalignment comes from K (K % 4 = 1, 2, 3, so
consecutive rows start at every offset), from the base pointer (1 to 3 floats past a 16-byte
boundary, K a multiple of 4) and from a leading dimension padded past K whose padding holds NaN
(a value read past the end of a row would show as a NaN output). Bits against the oracle, with
ragged row counts (the last strip of 8 rows part dead)."""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import bits, note, run
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ROUTE_K = [1, 2, 3, 5, 33, 63, 130, 255,   # one pass, eight strips per block
           257, 771, 2305, 4094,           # one pass, a strip per block
           4097, 6147, 20001, 50257]       # one read in parts along K


def _inputs(M, N, K, seed):
    rng = np.random.default_rng(seed)
    A = (rng.standard_normal(M * K) * 2.0 ** rng.integers(-12, 12, M * K)).astype(np.float32)
    B = rng.standard_normal(N * K).astype(np.float32)
    # each row's maximum at its first or its last value, where the realigned loads cross
    A.reshape(M, K)[0, 0] = 7e4
    A.reshape(M, K)[-1, -1] = -9e4
    return A, B


@pytest.mark.parametrize("K", ROUTE_K)
@pytest.mark.parametrize("S", [1, 3])
def test_rows_with_k_not_a_multiple_of_four(torch_gpu, K, S):
    torch = torch_gpu
    M, N = (37, 29) if K < 20000 else (21, 13)
    A, B = _inputs(M, N, K, K * 5 + S)
    ws = None
    for ta, tb in [(0, 0), (0, 1), (1, 1)]:  # op(A) row access when ta = 0, op(B) when tb = 1
        As = np.ascontiguousarray(A.reshape(M, K).T) if ta else A
        Bs = np.ascontiguousarray(B.reshape(K, N).T) if tb else B
        note("unaligned rows K=%d S=%d ta=%d tb=%d" % (K, S, ta, tb))
        C, _, ws = run(torch, As, Bs, M, N, K, rg.Config(slices=S, trans_a=bool(ta), trans_b=bool(tb)), ws=ws)
        want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
        assert np.array_equal(bits(C), want), (K, S, ta, tb)


@pytest.mark.parametrize("K", [64, 1000, 4096, 8192, 20000])
@pytest.mark.parametrize("shift", [1, 2, 3])
def test_rows_of_an_unaligned_base_pointer(torch_gpu, K, shift):
    """K a multiple of 4, the operands start 1 to 3 floats past a 16-byte boundary: every row has
    the same misalignment."""
    torch = torch_gpu
    M, N = 45, 30
    A, B = _inputs(M, N, K, 300 + K + shift)
    bufA = torch.full((M * K + 4,), float("nan"), dtype=torch.float32, device="cuda")
    bufB = torch.full((N * K + 4,), float("nan"), dtype=torch.float32, device="cuda")
    dA, dB = bufA[shift:shift + M * K], bufB[shift:shift + N * K]
    dA.copy_(torch.from_numpy(A))
    dB.copy_(torch.from_numpy(np.ascontiguousarray(B.reshape(K, N).T).reshape(-1)))
    note("unaligned base K=%d shift=%d" % (K, shift))
    C, _, _ = run(torch, dA, dB, M, N, K, rg.Config(slices=3, trans_b=True))
    assert np.array_equal(bits(C), O.cpu_gemm(A, B, M, N, K, 0, 0, 3).view(np.uint32)), (K, shift)


@pytest.mark.parametrize("K,pad", [(200, 1), (1001, 2), (3000, 3), (9000, 1), (9001, 5)])
def test_rows_padded_with_nan_past_k(torch_gpu, K, pad):
    """Leading dimension K + pad (rows start at every offset), the padding NaN, a batch of two
    items with a gap between them: nothing past a row's K values may be read."""
    torch = torch_gpu
    M, N, batch = 27, 19, 2
    lda, ldc = K + pad, N
    sa = M * lda + 3
    items = [_inputs(M, N, K, 40 + K + b) for b in range(batch)]
    hA = np.full(sa * batch, np.nan, np.float32)
    hB = np.stack([b.reshape(K, N) for _, b in items]).reshape(-1)
    for b, (a, _) in enumerate(items):
        hA[b * sa:b * sa + M * lda].reshape(M, lda)[:, :K] = a.reshape(M, K)
    dA, dB = torch.from_numpy(hA).cuda(), torch.from_numpy(hB).cuda()
    C = torch.full((M * N * batch,), float("nan"), dtype=torch.float32, device="cuda")
    cfg = rg.Config(slices=3)
    pl = rg.make_plan_strided_batched(M, N, K, batch, cfg)
    ws = torch.empty(max(pl.workspace_bytes, 1), dtype=torch.uint8, device="cuda")
    note("unaligned padded K=%d pad=%d" % (K, pad))
    code = rg.repro_gemm_strided_batched_fp32_ws(
        dA.data_ptr(), lda, sa, dB.data_ptr(), N, K * N, C.data_ptr(), ldc, M * N, M, N, K, batch,
        cfg, ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert code == 0, code
    torch.cuda.synchronize()
    hc = C.cpu().numpy().reshape(batch, M * N)
    for b, (a, bb) in enumerate(items):
        want = O.cpu_gemm(a, bb, M, N, K, 0, 0, 3).view(np.uint32).ravel()
        assert np.array_equal(hc[b].view(np.uint32), want), (K, pad, b)
