"""Exact rational restatement of the scalar definition, in Python integers/fractions.

Independent of the C oracle and of the product header: it never uses binary32 division,
frexp or float multiplication, so it pins them. Small inputs only (pure Python).
"""
from fractions import Fraction

import numpy as np


def f32_bits(x):
    return int(np.array([x], np.float32).view(np.uint32)[0])


def bits_f32(b):
    return np.array([b], np.uint32).view(np.float32)[0]


def f32_to_fraction(x):
    """Exact value of a finite float32."""
    b = f32_bits(x)
    sign = -1 if b >> 31 else 1
    e = (b >> 23) & 0xFF
    f = b & 0x7FFFFF
    if e == 0xFF:
        raise ValueError("not finite")
    if e == 0:
        return sign * Fraction(f, 1 << 149)
    m = f | 0x800000
    p = e - 150
    return sign * (Fraction(m) * (Fraction(2) ** p))


def _floor_log2(a):
    """Largest e with 2^e <= a, for a positive Fraction."""
    e = a.numerator.bit_length() - a.denominator.bit_length()
    two = Fraction(2)
    while two ** e > a:
        e -= 1
    while two ** (e + 1) <= a:
        e += 1
    return e


def _rne(q):
    """Round a non-negative Fraction to the nearest integer, ties to even."""
    n, d = q.numerator, q.denominator
    i, r = divmod(n, d)
    if 2 * r > d or (2 * r == d and (i & 1)):
        i += 1
    return i


def round_to_f32_bits(q, negative_zero=False):
    """Bits of the binary32 value nearest to the rational q (ties to even), with
    subnormals and overflow to infinity. q == 0 gives +0, or -0 if negative_zero."""
    if q == 0:
        return 0x80000000 if negative_zero else 0
    sign = 0x80000000 if q < 0 else 0
    a = abs(q)
    e = _floor_log2(a)
    qexp = max(e - 23, -149)
    m = _rne(a / (Fraction(2) ** qexp))
    if m == 0:
        return sign
    value = Fraction(m) * Fraction(2) ** qexp
    if value >= Fraction(2) ** 128:
        return sign | 0x7F800000
    return sign | f32_bits(np.float32(float(m) * 2.0 ** qexp))


def scale_exponent(m):
    """Smallest e with 2^e >= fl32(m / 127); 0 if m <= 0 or the quotient rounds to 0."""
    mq = f32_to_fraction(np.float32(m))
    if mq <= 0:
        return 0
    vb = round_to_f32_bits(mq / 127)
    if vb & 0x7FFFFFFF == 0:
        return 0
    v = f32_to_fraction(bits_f32(vb))
    e = _floor_log2(v)
    return e if Fraction(2) ** e == v else e + 1


def fixed_point(x, se, S):
    """RNE(x * 2^(7(S-1) - se)) clamped to |X| <= 127 * 2^(7(S-1))."""
    se, S = int(se), int(S)
    q = f32_to_fraction(np.float32(x)) * Fraction(2) ** (7 * (S - 1) - se)
    X = _rne(abs(q))
    if q < 0:
        X = -X
    lim = 127 << (7 * (S - 1))
    return max(-lim, min(lim, X))


def round_to_float_bits(T, E):
    """Bits of the correctly rounded binary32 value of T * 2^E; -0.0 when T < 0 rounds to 0."""
    T, E = int(T), int(E)
    if T == 0:
        return 0
    return round_to_f32_bits(Fraction(T) * Fraction(2) ** E, negative_zero=T < 0)


def gemm_bits(A, B, M, N, K, ta, tb, S):
    """The whole definition with Python integers; returns uint32 bits [M, N]."""
    A = np.asarray(A, np.float32).reshape(-1)
    B = np.asarray(B, np.float32).reshape(-1)

    def a_at(r, k):
        return A[k * M + r] if ta else A[r * K + k]

    def b_at(k, c):
        return B[c * K + k] if tb else B[k * N + c]

    eA = []
    X = []
    for r in range(M):
        row = [a_at(r, k) for k in range(K)]
        m = max(abs(f32_to_fraction(v)) for v in row)
        e = scale_exponent(np.float32(float(m))) if m > 0 else 0
        eA.append(e)
        X.append([fixed_point(v, e, S) for v in row])
    eB = []
    Y = []
    for c in range(N):
        col = [b_at(k, c) for k in range(K)]
        m = max(abs(f32_to_fraction(v)) for v in col)
        e = scale_exponent(np.float32(float(m))) if m > 0 else 0
        eB.append(e)
        Y.append([fixed_point(v, e, S) for v in col])
    out = np.zeros((M, N), np.uint32)
    for r in range(M):
        for c in range(N):
            t = sum(X[r][k] * Y[c][k] for k in range(K))
            out[r, c] = round_to_float_bits(t, eA[r] + eB[c] - 14 * (S - 1))
    return out
