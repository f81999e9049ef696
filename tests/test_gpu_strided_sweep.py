"""Seeded random sweep of the strided-batched entry point against the oracle, bit for bit:
leading dimensions padded past the matrix (so rows are often not 16-byte aligned), item strides
with gaps, batches of 1 to 3, every transpose, S = 1, 2, 3, the planner's automatic choice and
pinned tiles and splits, the hash tool's input distributions, and K from 1 to 20000 (one-pass and
two-pass slicing, the unaligned routes of both). Every element outside the matrices is NaN, so
a read or write past a leading dimension or an item would show as a wrong or non-finite output.
"""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import note
from oracle import oracle as O

pytestmark = pytest.mark.gpu

PLANS = [dict(), dict(), dict(tile_m=64, tile_n=64), dict(tile_m=128, tile_n=128),
         dict(split_k=3), dict(split_k=5, tile_m=64, tile_n=64), dict(algo=rg.Algo.Tiled)]
PADS = (0, 1, 2, 3, 5, 7)


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        M = int(np.exp(rng.uniform(0, np.log(1500))))
        N = int(np.exp(rng.uniform(0, np.log(1500))))
        K = int(np.exp(rng.uniform(0, np.log(20000))))
        while M * K > 4_000_000 or N * K > 4_000_000 or M * N * K > 4e8:
            K = max(1, K // 2)
        batch = int(rng.integers(1, 4))
        pads = [PADS[int(i)] for i in rng.integers(0, len(PADS), 3)]
        gaps = [int(rng.integers(0, 5)) for _ in range(3)]
        out.append((M, N, K, int(rng.integers(0, 2)), int(rng.integers(0, 2)), int(rng.integers(1, 4)),
                    PLANS[int(rng.integers(0, len(PLANS)))], O.HASH_DISTS[int(rng.integers(0, len(O.HASH_DISTS)))],
                    int(rng.integers(1, 1 << 30)), batch, pads, gaps))
    return out


@pytest.mark.parametrize("chunk", range(4))
def test_strided_batched_padded_leading_dimensions(torch_gpu, chunk):
    torch = torch_gpu
    for M, N, K, ta, tb, S, plan, dist, seed, batch, pads, gaps in _cases(50, 2000 + chunk):
        items = [O.gen_hash_inputs(M, N, K, seed + b, dist) for b in range(batch)]
        items = [(a.reshape(M, K), b.reshape(K, N)) for a, b in items]
        ra, ca = (K, M) if ta else (M, K)   # stored item of A: ra rows of lda values
        rb, cb = (N, K) if tb else (K, N)
        lda, ldb, ldc = ca + pads[0], cb + pads[1], N + pads[2]
        sa, sb, sc = ra * lda + gaps[0], rb * ldb + gaps[1], M * ldc + gaps[2]
        hA = np.full(sa * batch, np.nan, np.float32)
        hB = np.full(sb * batch, np.nan, np.float32)
        for b, (a, bb) in enumerate(items):
            hA[b * sa:b * sa + ra * lda].reshape(ra, lda)[:, :ca] = a.T if ta else a
            hB[b * sb:b * sb + rb * ldb].reshape(rb, ldb)[:, :cb] = bb.T if tb else bb
        cfg = rg.Config(slices=S, trans_a=bool(ta), trans_b=bool(tb), **plan)
        note("strided M=%d N=%d K=%d ta=%d tb=%d S=%d %s %s seed=%d batch=%d lda=%d ldb=%d ldc=%d"
             % (M, N, K, ta, tb, S, plan, dist, seed, batch, lda, ldb, ldc))
        dA = torch.from_numpy(hA).cuda()
        dB = torch.from_numpy(hB).cuda()
        C = torch.full((sc * batch,), float("nan"), dtype=torch.float32, device="cuda")
        pl = rg.make_plan_strided_batched(M, N, K, batch, cfg)
        ws = torch.empty(max(pl.workspace_bytes, 1), dtype=torch.uint8, device="cuda")
        code = rg.repro_gemm_strided_batched_fp32_ws(
            dA.data_ptr(), lda, sa, dB.data_ptr(), ldb, sb, C.data_ptr(), ldc, sc, M, N, K, batch,
            cfg, ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
        assert code == 0, code
        torch.cuda.synchronize()
        hc = C.cpu().numpy()
        for b, (a, bb) in enumerate(items):
            want = O.cpu_gemm(a, bb, M, N, K, 0, 0, S).view(np.uint32).reshape(M, N)
            out = hc[b * sc:b * sc + M * ldc].reshape(M, ldc)
            assert np.array_equal(out[:, :N].view(np.uint32), want), (M, N, K, ta, tb, S, plan, dist, seed, b)
            # nothing written past the matrix: the padding columns and the gap after the item
            assert np.isnan(out[:, N:]).all() and np.isnan(hc[b * sc + M * ldc:(b + 1) * sc]).all()
