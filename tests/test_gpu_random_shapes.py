"""Seeded random sweep of shapes and plans against the oracle, bit for bit: sizes from 1 to a few
hundred (ragged in every direction), every transpose, S = 1, 2, 3, and every way the planner
can be steered (automatic, the one-launch 32x32 kernel, each pinned block tile including the
twelve-wavefront ones, the Tiled and Reference algorithms, explicit splits), with the hash
tool's input distributions. The cases are drawn from a fixed seed, so a failure names a case
that reproduces.
"""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import bits, note, run
from oracle import oracle as O

pytestmark = pytest.mark.gpu

PLANS = [dict(), dict(tile_m=32, tile_n=32), dict(tile_m=64, tile_n=64), dict(tile_m=128, tile_n=128),
         dict(tile_m=128, tile_n=64), dict(tile_m=64, tile_n=128), dict(tile_m=64, tile_n=192),
         dict(tile_m=192, tile_n=64), dict(algo=rg.Algo.Tiled), dict(algo=rg.Algo.Reference),
         dict(split_k=3), dict(split_k=7, tile_m=64, tile_n=192)]


def _cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M = int(rng.integers(1, 400))
        N = int(rng.integers(1, 400))
        K = int(rng.choice([rng.integers(1, 96), rng.integers(96, 600), rng.integers(600, 2500)]))
        while M * N * K > 30_000_000:
            K = max(1, K // 2)
        out.append((M, N, K, int(rng.integers(0, 2)), int(rng.integers(0, 2)), int(rng.integers(1, 4)),
                    PLANS[i % len(PLANS)], rng.choice(O.HASH_DISTS), int(rng.integers(1, 1 << 30))))
    return out


@pytest.mark.parametrize("chunk", range(6))
def test_random_shapes_and_plans(torch_gpu, chunk):
    torch = torch_gpu
    for M, N, K, ta, tb, S, plan, dist, seed in _cases(64, 1000 + chunk):
        A, B = O.gen_hash_inputs(M, N, K, seed, dist)
        want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
        As = np.ascontiguousarray(A.T) if ta else A
        Bs = np.ascontiguousarray(B.T) if tb else B
        cfg = rg.Config(slices=S, trans_a=bool(ta), trans_b=bool(tb), **plan)
        note("random M=%d N=%d K=%d ta=%d tb=%d S=%d %s %s seed=%d" % (M, N, K, ta, tb, S, plan, dist, seed))
        C, got_plan, _ = run(torch, As.ravel(), Bs.ravel(), M, N, K, cfg)
        assert np.array_equal(bits(C), want), (M, N, K, ta, tb, S, plan, dist, seed, got_plan)


# The band kernel pinned (32 x W): ragged rows, columns and K up to its 1024, every slice count,
# both transposes of op(B) (a transposed op(A) falls back to the planner's choice).
BAND_PLANS = [dict(tile_m=32, tile_n=64), dict(tile_m=32, tile_n=96), dict(tile_m=32, tile_n=256),
              dict(tile_m=32, tile_n=160)]


def _band_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M = int(rng.integers(1, 700))
        N = int(rng.integers(1, 500))
        K = int(rng.choice([rng.integers(1, 64), rng.integers(64, 1025)]))
        out.append((M, N, K, int(rng.integers(0, 8) == 0), int(rng.integers(0, 2)),
                    int(rng.integers(1, 4)), BAND_PLANS[i % len(BAND_PLANS)],
                    rng.choice(O.HASH_DISTS), int(rng.integers(1, 1 << 30))))
    return out


@pytest.mark.parametrize("chunk", range(2))
def test_random_shapes_band_plans(torch_gpu, chunk):
    torch = torch_gpu
    for M, N, K, ta, tb, S, plan, dist, seed in _band_cases(48, 2000 + chunk):
        A, B = O.gen_hash_inputs(M, N, K, seed, dist)
        want = O.cpu_gemm(A, B, M, N, K, 0, 0, S).view(np.uint32)
        As = np.ascontiguousarray(A.T) if ta else A
        Bs = np.ascontiguousarray(B.T) if tb else B
        cfg = rg.Config(slices=S, trans_a=bool(ta), trans_b=bool(tb), **plan)
        note("random band M=%d N=%d K=%d ta=%d tb=%d S=%d %s %s seed=%d" % (M, N, K, ta, tb, S, plan, dist, seed))
        C, got_plan, _ = run(torch, As.ravel(), Bs.ravel(), M, N, K, cfg)
        if not ta:
            assert (got_plan.tile_m, got_plan.tile_n) == (32, plan["tile_n"])
        assert np.array_equal(bits(C), want), (M, N, K, ta, tb, S, plan, dist, seed, got_plan)
