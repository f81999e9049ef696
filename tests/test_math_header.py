"""The product's scalar header (include/repro_gemm_math.h, integer formulations of
fixed_point and round_to_float) against the oracle, on the host. The device build of the
same header is compared with the oracle by the GPU tests."""
import ctypes
import os
import random
import subprocess
import threading

import numpy as np
import pytest

import exact
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)


@pytest.fixture(scope="module")
def hm(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("hm") / "libhm.so")
    subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
                    "-fno-fast-math", "-I", os.path.join(REPO, "include"), "-I",
                    os.path.join(REPO, "bit_reproducible_training_amd", "csrc"),
                    os.path.join(HERE, "host_math_shim.cpp"), "-o", out], check=True)
    lib = ctypes.CDLL(out)
    vp, ll = ctypes.c_void_p, ctypes.c_longlong
    lib.hm_scale_exponent_n.argtypes = [vp, vp, ll]
    lib.hm_fixed_point_n.argtypes = [vp, vp, ctypes.c_int, vp, ll]
    lib.hm_round_to_float_n.argtypes = [vp, vp, vp, ll]
    lib.hm_round_to_float_fast_n.argtypes = [vp, vp, vp, ll]
    lib.hm_round_to_float_f64_n.argtypes = [vp, vp, vp, ll]
    lib.hm_scale_exponent_count_range.argtypes = [ctypes.c_uint32, ctypes.c_uint32, vp]
    lib.hm_scale_exponent_count_range.restype = ll
    lib.hm_fastdiv_mismatches.argtypes = [vp, ll, vp, ll]
    lib.hm_fastdiv_mismatches.restype = ll
    lib.hm_fastdiv_range.argtypes = [ctypes.c_uint32] * 3
    lib.hm_fastdiv_range.restype = ll
    return lib


def test_fastdiv_matches_integer_division(hm):
    """The packing kernels' multiply-high divider (bit_reproducible_training_amd/csrc/
    rg_fastdiv.h) against C's unsigned division: every n below 2^31 for two divisors, and
    divisors 1..4096, powers of two and their neighbours and random ones against edge and
    random dividends."""
    assert hm.hm_fastdiv_range(7, 0, 1 << 31) == 0
    assert hm.hm_fastdiv_range(784, 0, 1 << 31) == 0
    rng = np.random.default_rng(5)
    d = np.concatenate([np.arange(1, 4097), [2 ** k + j for k in range(12, 31) for j in (-1, 0, 1)],
                        rng.integers(1, 2 ** 31, 3000)]).astype(np.uint32)
    n = np.concatenate([np.arange(0, 70000), 2 ** 31 - 1 - np.arange(0, 1000),
                        rng.integers(0, 2 ** 31, 20000)]).astype(np.uint32)
    assert hm.hm_fastdiv_mismatches(d.ctypes.data, d.size, n.ctypes.data, n.size) == 0


def test_scale_exponent_exhaustive_vs_oracle(hm):
    """All 2^31 non-negative finite floats (and their negatives' sign handling below)."""
    want = ctypes.cast(O.lib.oracle_scale_exponent, ctypes.c_void_p)
    bad = [0] * 8
    span = 0x7F800000

    def run(i):
        lo, hi = span * i // 8, span * (i + 1) // 8
        bad[i] = hm.hm_scale_exponent_count_range(lo, hi, want)

    ts = [threading.Thread(target=run, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert sum(bad) == 0
    neg = np.array([-1.0, -0.0, -1e-45, -3e38], np.float32)
    e = np.empty(4, np.int32)
    hm.hm_scale_exponent_n(neg.ctypes.data, e.ctypes.data, 4)
    assert list(e) == [0, 0, 0, 0]


@pytest.mark.parametrize("S", [1, 2, 3])
def test_fixed_point_vs_oracle(hm, S):
    rng = np.random.default_rng(S)
    n = 2_000_000
    bits = rng.integers(0, 0x7F800000, n, dtype=np.uint32) | (rng.integers(0, 2, n, dtype=np.uint32) << 31)
    x = bits.view(np.float32)
    # Reachable domain: in a GEMM the row exponent is that of the row max m >= |x|, so
    # se >= scale_exponent(|x|) and |x * 2^(7(S-1)-se)| stays below 2^31. (Outside it the
    # float-to-int conversion of the C definition is undefined behaviour.)
    se_min = O.scale_exponent_n(np.abs(x))
    se = np.clip(se_min + rng.integers(0, 30, n), -149, 127).astype(np.int32)
    got = np.empty(n, np.int32)
    hm.hm_fixed_point_n(x.ctypes.data, se.ctypes.data, S, got.ctypes.data, n)
    assert np.array_equal(got, O.fixed_point_n(x, se, S))
    # exact ties and clamp edges against the rational definition
    r = random.Random(S)
    xs, ses = [], []
    for _ in range(400):
        s2 = r.randint(-140, 110)
        xs.append(np.float32((r.randint(-2 ** 21, 2 ** 21) + 0.5) * 2.0 ** (s2 - 7 * (S - 1))))
        ses.append(s2)
        xs.append(np.float32(r.uniform(126.9, 128.5) * 2.0 ** s2))
        ses.append(s2)  # the clamp: fl(m/127) rounded down below m/127
    xs = np.array(xs, np.float32)
    ses = np.array(ses, np.int32)
    keep = np.isfinite(xs)
    xs, ses = xs[keep], ses[keep]
    got = np.empty(len(xs), np.int32)
    hm.hm_fixed_point_n(xs.ctypes.data, ses.ctypes.data, S, got.ctypes.data, len(xs))
    assert list(got) == [exact.fixed_point(a, b, S) for a, b in zip(xs, ses)]


def test_round_to_float_vs_oracle(hm):
    rng = np.random.default_rng(11)
    n = 2_000_000
    mag = rng.integers(0, 63, n)
    T = (rng.integers(0, 2 ** 62, n, dtype=np.int64) >> mag) * rng.choice([-1, 1], n)
    E = rng.integers(-330, 220, n).astype(np.int32)
    got = np.empty(n, np.float32)
    hm.hm_round_to_float_n(T.ctypes.data, E.ctypes.data, got.ctypes.data, n)
    assert np.array_equal(got.view(np.uint32), O.round_to_float_n(T, E).view(np.uint32))


def _fast_vs_general(hm, T, E, fn="hm_round_to_float_fast_n"):
    T = np.ascontiguousarray(T, np.int64)
    E = np.ascontiguousarray(E, np.int32)
    n = T.size
    fast = np.empty(n, np.float32)
    gen = np.empty(n, np.float32)
    getattr(hm, fn)(T.ctypes.data, E.ctypes.data, fast.ctypes.data, n)
    hm.hm_round_to_float_n(T.ctypes.data, E.ctypes.data, gen.ctypes.data, n)
    return fast.view(np.uint32), gen.view(np.uint32)


FAST = ["hm_round_to_float_fast_n", "hm_round_to_float_f64_n"]


@pytest.mark.parametrize("fn", FAST)
def test_round_to_float_fast_equals_general_and_oracle(hm, fn):
    """The epilogue roundings (round_to_float_fast: branch-free integer; round_to_float_f64:
    through binary64) against round_to_float and the oracle on every bit length of T and
    exponents across the whole range, including the boundaries where they hand over to the
    general path (zero, subnormal, overflow; |T| > 2^53 and exponents beyond binary64's)."""
    rng = np.random.default_rng(12)
    n = 3_000_000
    mag = rng.integers(0, 64, n)
    T = (rng.integers(0, 2 ** 63 - 1, n, dtype=np.int64) >> mag) * rng.choice([-1, 1], n)
    E = rng.integers(-340, 240, n).astype(np.int32)
    E[:1000] = rng.integers(-1200, 1100, 1000)
    fast, gen = _fast_vs_general(hm, T, E, fn)
    assert np.array_equal(fast, gen)
    assert np.array_equal(fast, O.round_to_float_n(T, E).view(np.uint32))


def _tie_cases():
    T, E = [], []
    rng = np.random.default_rng(13)
    for p in range(24, 63):
        sh = p - 23
        for top in (1 << 23, (1 << 23) + 1, (1 << 24) - 1, int(rng.integers(1 << 23, 1 << 24))):
            base = top << sh
            for d in ((1 << (sh - 1)) - 1, 1 << (sh - 1), (1 << (sh - 1)) + 1, 0, (1 << sh) - 1):
                v = base + d
                if v >= 2 ** 63:
                    continue
                for e_target in (-200, -150, -149, -127, -126, -125, -1, 0, 1, 100, 126, 127, 128):
                    T += [v, -v]
                    E += [e_target - p, e_target - p]
    # around the binary64 handover: |T| = 2^53 +- small, and T = -2^53 exactly
    for v in (2 ** 53 - 1, 2 ** 53, 2 ** 53 + 1, 2 ** 53 + 2, 2 ** 52 + 1, 2 ** 54 - 1):
        for e in (-1100, -1023, -1022, -160, -100, 0, 70, 74, 75, 970, 971):
            T += [v, -v]
            E += [e, e]
    T += [0, 1, -1, 2 ** 62, -(2 ** 62), 2 ** 63 - 1, -(2 ** 63)]
    E += [0, -149, -150, 65, 65, 64, 64]
    return np.array(T, np.int64), np.array(E, np.int32)


@pytest.mark.parametrize("fn", FAST)
def test_round_to_float_fast_ties_and_binade_edges(hm, fn):
    """Exact ties (even and odd), one above/below a tie, carries into the next binade, the
    carry out of the largest binade (+-inf), the smallest normal and the subnormal handover,
    and |T| around 2^53 with exponents at the edges of binary64's exact scaling."""
    T, E = _tie_cases()
    fast, gen = _fast_vs_general(hm, T, E, fn)
    assert np.array_equal(fast, gen)
    assert np.array_equal(fast, O.round_to_float_n(T, E).view(np.uint32))
