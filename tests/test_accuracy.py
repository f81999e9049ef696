"""Accuracy of the reproducible GEMM against FP64, the report of the reference's hash tool
(repro_gemm_cuda/hash_repro_gemm.cu:171-188: relative Frobenius error over the finite outputs and
the worst row), for every input distribution of the tool and S = 1, 2, 3.

The outputs here are the oracle's, which the GPU tests show are the GPU's bit for bit
(test_gpu_hash_dists.py), so these are the product's accuracy figures. Each slice adds 7 bits to
every input, so the error must shrink by about 2^7 per slice; the bounds below are about 4x the
values measured for these inputs, and S = 3 stays within a few times plain FP32 GEMM.
"""
import numpy as np
import pytest

from oracle import oracle as O

M, N, K = 256, 256, 1024
# (relative Frobenius error bound at S = 1, 2, 3) per distribution; weights carry 0.1% outliers
# x100, which set the row scales, so the typical entry keeps fewer bits.
BOUNDS = {"uniform": (4e-2, 4e-4, 3e-6), "normal": (5e-2, 4e-4, 4e-6), "weights": (5e-1, 4e-3, 4e-5),
          "wide": (6e-2, 6e-4, 6e-6), "stress": (6e-2, 5e-4, 4e-6)}


def accuracy(C, A, B):
    """(relative Frobenius error, worst row's relative error) of C against the FP64 product, over
    the outputs whose error is finite (the tool's rule for outputs that overflow FP32)."""
    ref = A.astype(np.float64) @ B.astype(np.float64)
    d = C.astype(np.float64) - ref
    ok = np.isfinite(d)
    d2 = np.where(ok, d * d, 0.0)
    r2 = np.where(ok, ref * ref, 0.0)
    row_e, row_r = d2.sum(axis=1), r2.sum(axis=1)
    live = row_r > 0
    worst = float(np.sqrt(row_e[live] / row_r[live]).max()) if live.any() else 0.0
    total = float(np.sqrt(d2.sum() / r2.sum())) if r2.sum() > 0 else 0.0
    return total, worst


@pytest.mark.parametrize("dist", O.HASH_DISTS)
def test_accuracy_against_fp64(dist):
    A, B = O.gen_hash_inputs(M, N, K, 12345, dist)
    errs = []
    for S in (1, 2, 3):
        with np.errstate(over="ignore", invalid="ignore"):
            total, worst = accuracy(O.cpu_gemm(A, B, M, N, K, 0, 0, S), A, B)
        assert 0.0 < total <= BOUNDS[dist][S - 1], (dist, S, total)
        assert total <= worst
        errs.append(total)
    assert errs[0] / errs[1] > 50 and errs[1] / errs[2] > 50, errs   # ~2^7 per slice
