"""The GPU epilogue's final rounding against the oracle's round_to_float, through the
rg_test_round hook, which runs the same device functions as the contraction's epilogue
(level sums combined and rounded through binary64, with the exact int64 path for what that
cannot take) and the split-K reduction (int64 sums through binary64). Inputs cover every bit
length of T, exact ties and their neighbours at every binade, the subnormal range, overflow,
signed zeros, |T| around 2^53 (the binary64 handover) and extreme level values."""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from bit_reproducible_training_amd import _lib
from gpu_util import note
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _device_round(torch, E, levels=None, T=None, S=3):
    dE = torch.from_numpy(np.ascontiguousarray(E, np.int32)).cuda()
    out = torch.full((E.size,), float("nan"), dtype=torch.float32, device="cuda")
    dl = dT = None
    if levels is not None:
        dl = torch.from_numpy(np.ascontiguousarray(levels, np.int32)).cuda()
    else:
        dT = torch.from_numpy(np.ascontiguousarray(T, np.int64)).cuda()
    code = _lib.lib.rg_test_round(dl.data_ptr() if dl is not None else None,
                                  dT.data_ptr() if dT is not None else None, dE.data_ptr(),
                                  out.data_ptr(), E.size, S,
                                  torch.cuda.current_stream().cuda_stream)
    assert code == 0
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint32)


def _combine(levels):
    L = levels.shape[1]
    T = np.zeros(levels.shape[0], np.int64)
    for l in range(L):
        T += levels[:, l].astype(np.int64) << (7 * (L - 1 - l))
    return T


def _tie_values():
    """|T| values at and around round-to-nearest ties, binade edges and 2^53."""
    vals = []
    rng = np.random.default_rng(5)
    for p in range(24, 59):   # |T| < 2^59: the top level T >> 28 fits int32
        sh = p - 23
        for top in (1 << 23, (1 << 23) + 1, (1 << 24) - 1, int(rng.integers(1 << 23, 1 << 24))):
            for d in ((1 << (sh - 1)) - 1, 1 << (sh - 1), (1 << (sh - 1)) + 1, 0, (1 << sh) - 1):
                vals.append((top << sh) + d)
    vals += [2 ** 53 - 1, 2 ** 53, 2 ** 53 + 1, 2 ** 53 + 2, 2 ** 52 + 1, 2 ** 54 - 1, 1, 3, 0]
    return np.array(vals, np.int64)


def _exponents_for(T, targets):
    """Exponents that put |T|'s leading bit at each target binade."""
    p = np.floor(np.log2(np.maximum(np.abs(T), 1).astype(np.float64))).astype(np.int64)
    T2 = np.repeat(T, len(targets))
    E = (np.tile(np.array(targets, np.int64), T.size) - np.repeat(p, len(targets)))
    return T2, E.astype(np.int32)


TARGETS = (-200, -151, -150, -149, -148, -127, -126, -125, -1, 0, 1, 126, 127, 128)


@pytest.mark.parametrize("S", [1, 2, 3])
def test_level_rounding_random(torch_gpu, S):
    torch = torch_gpu
    L = 2 * S - 1
    rng = np.random.default_rng(40 + S)
    n = 1 << 20
    mag = rng.integers(0, 32, (n, 1))
    levels = (rng.integers(-(2 ** 31), 2 ** 31, (n, L), dtype=np.int64) >> mag).astype(np.int32)
    levels[:64] = np.int32(2 ** 31 - 1)
    levels[64:128] = np.int32(-(2 ** 31))
    levels[128:192] = 0
    E = rng.integers(-330, 250, n).astype(np.int32)
    E[192:256] = rng.integers(-1200, 1100, 64)
    note("level rounding random S=%d" % S)
    got = _device_round(torch, E, levels=levels, S=S)
    want = O.round_to_float_n(_combine(levels), E).view(np.uint32)
    assert np.array_equal(got, want)


def test_level_rounding_ties_and_edges(torch_gpu):
    """T at ties and binade edges (split into 5 levels: top level T >> 28, then 7-bit digits),
    placed at every interesting output binade, both signs."""
    torch = torch_gpu
    T, E = _exponents_for(_tie_values(), TARGETS)
    T = np.concatenate([T, -T])
    E = np.concatenate([E, E])
    levels = np.stack([(T >> 28)] + [(T >> (7 * (4 - l))) & 127 for l in range(1, 5)],
                      axis=1).astype(np.int32)
    assert np.array_equal(_combine(levels), T)
    note("level rounding ties", T.size)
    got = _device_round(torch, E, levels=levels, S=3)
    assert np.array_equal(got, O.round_to_float_n(T, E).view(np.uint32))


def test_int64_rounding(torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(44)
    n = 1 << 20
    mag = rng.integers(0, 64, n)
    T = (rng.integers(0, 2 ** 63 - 1, n, dtype=np.int64) >> mag) * rng.choice([-1, 1], n)
    E = rng.integers(-340, 240, n).astype(np.int32)
    E[:1000] = rng.integers(-1200, 1100, 1000)
    t2, e2 = _exponents_for(_tie_values(), TARGETS)
    T = np.concatenate([T, t2, -t2, [0, -(2 ** 63), 2 ** 63 - 1]]).astype(np.int64)
    E = np.concatenate([E, e2, e2, [0, 0, 0]]).astype(np.int32)
    note("int64 rounding", T.size)
    got = _device_round(torch, E, T=T)
    assert np.array_equal(got, O.round_to_float_n(T, E).view(np.uint32))


def test_rounding_hook_arguments(torch_gpu):
    torch = torch_gpu
    x = torch.zeros(8, dtype=torch.int32, device="cuda")
    out = torch.zeros(8, device="cuda")
    f = _lib.lib.rg_test_round
    assert f(x.data_ptr(), x.data_ptr(), x.data_ptr(), out.data_ptr(), 1, 3, None) == 1
    assert f(None, None, x.data_ptr(), out.data_ptr(), 1, 3, None) == 1
    assert f(x.data_ptr(), None, x.data_ptr(), out.data_ptr(), 1, 4, None) == 1
    assert f(x.data_ptr(), None, x.data_ptr(), out.data_ptr(), 0, 3, None) == 0
