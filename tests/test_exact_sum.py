"""The exact sum (superaccumulator) on the CPU: the oracle against exact rational arithmetic
and against the reference's own header (oracle/_ref); the product header
(include/repro_sum_math.h, host build) against the oracle, including a replay of the GPU
kernels' accumulation schedule; and the host planner of the C ABI (no kernel launched).

Definition (repro_sum_cuda/repro_sum.cuh:8-25, repro_sum_math.cuh:102-109): out[b] is the
exact sum over a, c of x[a][b][c] (or that sum / (A*C)) rounded once to binary32,
nearest-even; an exactly zero result is +0.0; NaN or infinity among the summands gives NaN.
"""
import ctypes
import os
import subprocess
from fractions import Fraction

import numpy as np
import pytest

import exact
from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
QNAN = 0x7FC00000


def exact_bits(values, divisor=1):
    """Binary32 bits of the exactly rounded sum / divisor, in Python rationals."""
    vals = np.asarray(values, np.float32).reshape(-1)
    if not np.all(np.isfinite(vals)):
        return QNAN
    total = sum((exact.f32_to_fraction(v) for v in vals), Fraction(0))
    return exact.round_to_f32_bits(total / divisor)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def f32_from_bits(b):
    return np.array(b, np.uint32).view(np.float32)


# ---------------------------------------------------------------------------------------
# Input families
# ---------------------------------------------------------------------------------------

def wide_range(rng, n):
    """Random signs and biased exponents over the whole finite range, subnormals included."""
    e = rng.integers(0, 255, n, dtype=np.uint32)
    f = rng.integers(0, 1 << 23, n, dtype=np.uint32)
    s = rng.integers(0, 2, n, dtype=np.uint32)
    return f32_from_bits((s << 31) | (e << 23) | f)


def cancelling(rng, n):
    """Pairs x, -x of wide range plus a few tiny residues: the exact sum is tiny."""
    pairs = (n - max(1, n // 64)) // 2
    x = wide_range(rng, pairs)
    tiny = f32_from_bits(rng.integers(1, 1 << 20, n - 2 * pairs, dtype=np.uint32))
    out = np.concatenate([x, -x, tiny])
    rng.shuffle(out)
    return out


def families(rng, n):
    return {
        "normal": rng.standard_normal(n).astype(np.float32),
        "wide": wide_range(rng, n),
        "cancel": cancelling(rng, n),
        "small_exp": (rng.standard_normal(n) * 2.0 ** rng.integers(-140, -120, n)).astype(np.float32),
        "big": (rng.standard_normal(n) * 1e37).astype(np.float32),
    }


TWO24 = float(2 ** 24)
FLT_MAX = float(np.finfo(np.float32).max)
KNOWN = [
    # (values, divisor, expected float or "nan"/"+0"/"-0"/"inf"/"-inf")
    ([1e30, 1.0, -1e30], 1, 1.0),
    ([TWO24, 1.0], 1, TWO24),                          # tie, rounds to even
    ([TWO24 + 2, 1.0], 1, TWO24 + 4),                  # tie, rounds up to even
    ([TWO24, 1.0, 2.0 ** -100], 1, TWO24 + 2),         # just above the tie
    ([-TWO24, -1.0], 1, -TWO24),
    ([-0.0, -0.0], 1, "+0"),                           # exact zero is +0
    ([2.0 ** -149, -(2.0 ** -149)], 1, "+0"),
    ([2.0 ** -149, 2.0 ** -149], 1, 2.0 ** -148),
    ([FLT_MAX, FLT_MAX], 1, "inf"),
    ([-FLT_MAX, -FLT_MAX], 1, "-inf"),
    ([FLT_MAX, FLT_MAX, -FLT_MAX], 1, FLT_MAX),
    ([FLT_MAX, 2.0 ** 103], 1, "inf"),                 # half an ulp above FLT_MAX: tie to 2^128
    ([FLT_MAX, 2.0 ** 102], 1, FLT_MAX),
    ([1.0, 2.0], 2, 1.5),
    ([1.0, 1.0, 0.0], 3, float(np.float32(2.0 / 3.0))),
    ([2.0 ** -149, 0.0], 2, "+0"),                     # 2^-150: tie between 0 and 2^-149
    ([3 * 2.0 ** -149, 0.0], 2, 2.0 ** -148),          # 1.5 * 2^-149: tie, to even 2 * 2^-149
    ([-(2.0 ** -149), 0.0, 0.0], 3, "-0"),             # nonzero, rounds to a signed zero
    ([1.0, float("nan")], 1, "nan"),
    ([1.0, float("inf"), float("-inf")], 1, "nan"),
    ([float("inf")], 1, "nan"),
]


def _expected_bits(exp):
    return {"+0": 0, "-0": 0x80000000, "inf": 0x7F800000, "-inf": 0xFF800000,
            "nan": QNAN}.get(exp) if isinstance(exp, str) else int(bits(np.float32(exp)))


@pytest.mark.parametrize("case", range(len(KNOWN)))
def test_known_answers(case):
    values, divisor, expected = KNOWN[case]
    x = np.array(values, np.float32)
    want = _expected_bits(expected)
    if want != QNAN:
        assert exact_bits(x, divisor) == want      # the rational reference agrees
    assert divisor in (1, len(x))                  # a mean divides by the count
    got = O.exact_sum(x, len(x), 1, 1, mean=divisor != 1)
    assert int(bits(got)[0]) == want, (values, divisor, hex(int(bits(got)[0])), hex(want))


@pytest.mark.parametrize("seed", range(6))
def test_oracle_matches_exact_rationals(seed):
    rng = np.random.default_rng(100 + seed)
    for name, x in families(rng, 64).items():
        for mean in (False, True):
            n = x.size
            want = exact_bits(x, n if mean else 1)
            got = O.exact_sum(x, n, 1, 1, mean)
            assert int(bits(got)[0]) == want, (name, mean)


def test_oracle_rational_ties_and_random_means():
    """Sums built to land exactly on, just above and just below rounding ties, with divisors
    that make the quotient non-terminating in binary."""
    rng = np.random.default_rng(7)
    for _ in range(200):
        e = int(rng.integers(-120, 100))
        base = float(np.float32(1.0 + rng.integers(0, 1 << 23) * 2.0 ** -23)) * 2.0 ** e
        ulp = 2.0 ** (e - 23)
        for extra in ([ulp / 2], [ulp / 2, ulp * 2.0 ** -30], [ulp / 2, -ulp * 2.0 ** -30]):
            x = np.array([base] + extra, np.float32)
            if not np.all(np.isfinite(x)) or np.any((x != 0) & (np.abs(x) < 2.0 ** -149)):
                continue
            want = exact_bits(x)
            assert int(bits(O.exact_sum(x, len(x), 1, 1))[0]) == want
        d = int(rng.integers(2, 1000))
        x = rng.standard_normal(d).astype(np.float32) * np.float32(2.0 ** int(rng.integers(-60, 60)))
        assert int(bits(O.exact_sum(x, d, 1, 1, True))[0]) == exact_bits(x, d)


def test_oracle_layouts_and_order_independence():
    rng = np.random.default_rng(3)
    A, B, C = 5, 7, 3
    x = wide_range(rng, A * B * C).reshape(A, B, C)
    got = O.exact_sum(x, A, B, C)
    for b in range(B):
        assert int(bits(got)[b]) == exact_bits(x[:, b, :])
    perm = rng.permutation(A)
    assert np.array_equal(bits(O.exact_sum(x[perm], A, B, C)), bits(got))
    got_mean = O.exact_sum(x, A, B, C, True)
    for b in range(B):
        assert int(bits(got_mean)[b]) == exact_bits(x[:, b, :], A * C)


def test_oracle_matches_reference_header():
    """oracle/_ref compiles the reference's repro_sum_math.cuh itself."""
    if O.ref is None:
        pytest.skip("oracle/_ref not built (reference headers absent)")
    rng = np.random.default_rng(11)
    shapes = [(1, 1, 5000), (300, 17, 1), (9, 6, 784), (1, 33, 100), (64, 120, 1)]
    for A, B, C in shapes:
        for name, x in families(rng, A * B * C).items():
            for mean in (False, True):
                want = O.ref_exact_sum(x, A, B, C, mean)
                got = O.exact_sum(x, A, B, C, mean)
                assert np.array_equal(bits(got), bits(want)), (A, B, C, name, mean)
    for values, divisor, _ in KNOWN:
        x = np.array(values, np.float32)
        mean = divisor != 1
        assert np.array_equal(bits(O.exact_sum(x, 1, 1, len(x), mean)),
                              bits(O.ref_exact_sum(x, 1, 1, len(x), mean)))


def test_has_nonfinite():
    x = np.zeros(100, np.float32)
    assert not O.has_nonfinite(x)
    for v in (np.inf, -np.inf, np.nan):
        y = x.copy()
        y[57] = v
        assert O.has_nonfinite(y)
    assert not O.has_nonfinite(np.array([np.finfo(np.float32).max, 1e-45], np.float32))


# ---------------------------------------------------------------------------------------
# The product header on the host
# ---------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def hs(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("hs") / "libhs.so")
    subprocess.run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
                    "-fno-fast-math", "-I", os.path.join(REPO, "include"),
                    os.path.join(HERE, "host_sum_shim.cpp"), "-o", out], check=True)
    lib = ctypes.CDLL(out)
    vp, i = ctypes.c_void_p, ctypes.c_int
    lib.hs_exact_sum.argtypes = [vp, vp, i, i, i, i]
    lib.hs_wide_schedule.argtypes = [vp, vp, i, i, i, i, ctypes.c_uint32]
    lib.hs_wide_schedule.restype = ctypes.c_float
    return lib


def _hs_sum(hs, x, A, B, C, mean=False):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(B, np.float32)
    hs.hs_exact_sum(x.ctypes.data, out.ctypes.data, A, B, C, int(mean))
    return out


def test_product_header_matches_oracle(hs):
    rng = np.random.default_rng(21)
    for A, B, C in [(1, 1, 3000), (200, 9, 1), (7, 5, 130)]:
        for name, x in families(rng, A * B * C).items():
            for mean in (False, True):
                assert np.array_equal(bits(_hs_sum(hs, x, A, B, C, mean)),
                                      bits(O.exact_sum(x, A, B, C, mean))), (A, B, C, name, mean)
    for values, divisor, expected in KNOWN:
        x = np.array(values, np.float32)
        got = _hs_sum(hs, x, 1, 1, len(x), divisor != 1)
        assert int(bits(got)[0]) == _expected_bits(expected), values


@pytest.mark.parametrize("flush", [1, 7, 252])
def test_gpu_schedule_replay_matches_oracle(hs, flush):
    """Wide 64-bit adds, carries every `flush` adds, any lane count, order and chunking: the
    same bits as the oracle (the GPU kernels use flush <= 252)."""
    rng = np.random.default_rng(flush)
    for name, x in families(rng, 4000).items():
        want = int(bits(O.exact_sum(x, x.size, 1, 1))[0])
        want_mean = int(bits(O.exact_sum(x, x.size, 1, 1, True))[0])
        for lanes, groups in [(1, 1), (64, 1), (256, 7), (1000, 13)]:
            order = rng.permutation(x.size).astype(np.int32)
            for divisor, w in ((1, want), (x.size, want_mean)):
                got = hs.hs_wide_schedule(x.ctypes.data, order.ctypes.data, x.size, lanes, flush,
                                          groups, divisor)
                assert int(bits(np.float32(got))) == w, (name, lanes, groups, divisor)


def test_gpu_schedule_worst_case_magnitudes(hs):
    """252 adds of the largest wide term into one limb, in both signs, then merges."""
    big = np.full(252 * 64, np.finfo(np.float32).max, np.float32)
    order = np.arange(big.size, dtype=np.int32)
    for sign in (1, -1):
        x = (sign * big).astype(np.float32)
        got = hs.hs_wide_schedule(x.ctypes.data, order.ctypes.data, x.size, 64, 252, 3, 1)
        assert np.isinf(got) and np.sign(got) == sign
        got = hs.hs_wide_schedule(x.ctypes.data, order.ctypes.data, x.size, 64, 252, 3, x.size)
        assert int(bits(np.float32(got))) == int(bits(x[:1])[0])


# ---------------------------------------------------------------------------------------
# Host planner of the C ABI (repro_sum_cuda/repro_sum.cu:183-230 validation)
# ---------------------------------------------------------------------------------------

def test_sum_planner():
    import bit_reproducible_training_amd as rg

    ok = rg.sum_plan_for_device(8192, 768, 1, num_cus=256)
    assert ok.chunks > 1 and ok.workspace_bytes > 0
    one = rg.sum_plan_for_device(64, 10, 1, num_cus=256)
    assert one.chunks == 1 and one.workspace_bytes == 0
    forced = rg.sum_plan_for_device(1000, 3, 1, rg.SumConfig(chunks=7), num_cus=256)
    assert forced.chunks == 7
    capped = rg.sum_plan_for_device(5, 3, 1, rg.SumConfig(chunks=100), num_cus=256)
    assert capped.chunks == 5                       # at most one row per chunk
    seg = rg.sum_plan_for_device(100, 6, 784, num_cus=256)
    assert seg.chunks >= 1
    for bad in [(0, 1, 1), (1, 0, 1), (1, 1, 0), (-1, 1, 1), (2 ** 16, 1, 2 ** 16)]:
        with pytest.raises(rg.ReproGemmError) as e:
            rg.sum_plan_for_device(*bad, num_cus=256)
        assert e.value.code == 1
    with pytest.raises(rg.ReproGemmError):
        rg.sum_plan_for_device(4, 4, 4, rg.SumConfig(chunks=-1), num_cus=256)


def test_config_defaults_match_reference():
    from bit_reproducible_training_amd import _lib

    c = _lib.rg_sum_config(5, 5)
    _lib.lib.rg_sum_config_init(ctypes.byref(c))
    assert (c.chunks, c.mean) == (0, 0)             # repro_sum.cuh:27-30


def test_scan_finite_rejects_null_arguments():
    from bit_reproducible_training_amd import _lib

    assert _lib.lib.rg_scan_finite(None, None, 0, 0, None) == 0        # n == 0: nothing to do
    assert _lib.lib.rg_scan_finite(None, None, 10, 0, None) == 1
