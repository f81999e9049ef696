"""ctypes bindings of the CPU checkers (liboracle.so and, when built, _ref/libref_cpu.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker or the timed CPU baseline. The product never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_cpu.so")
FNV_OFFSET = 0xCBF29CE484222325

_vp, _sz, _u64, _i, _f, _d = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_int,
                              ctypes.c_float, ctypes.c_double)

_SIG = {
    "oracle_scale_exponent": (_i, [_f]),
    "oracle_scale_by_pow2": (_f, [_f, _i]),
    "oracle_fixed_point": (_i, [_f, _i, _i]),
    "oracle_round_to_float": (_f, [ctypes.c_int64, _i]),
    "oracle_scale_exponent_n": (None, [_vp, _vp, _sz]),
    "oracle_fixed_point_n": (None, [_vp, _vp, _i, _vp, _sz]),
    "oracle_round_to_float_n": (None, [_vp, _vp, _vp, _sz]),
    "oracle_check_scale_exponent_range": (_u64, [ctypes.c_uint32, ctypes.c_uint32, _vp]),
    "oracle_quantize": (None, [_vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _i]),
    "oracle_exact_products": (None, [_vp, _vp, _vp, _i, _i, _i, _i]),
    "oracle_cpu_gemm": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i]),
    "oracle_cpu_gemm_rows": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _i]),
    "oracle_gen_normal": (None, [_vp, _sz, _d, _u64]),
    "oracle_gen_normal_at": (None, [_vp, _sz, _d, _u64, _u64]),
    "oracle_gen_uniform": (None, [_vp, _sz, _d, _u64]),
    "oracle_gen_uniform_pm": (None, [_vp, _sz, _f, _u64, _u64]),
    "oracle_gen_adversarial": (None, [_vp, _i, _i, _u64, _i, _i]),
    "oracle_gen_hash_inputs": (_i, [_vp, _vp, _i, _i, _i, _u64, _i]),
    "oracle_splitmix64": (None, [_vp, _sz, _u64]),
    "oracle_fnv1a64": (_u64, [_vp, _sz, _u64]),
    "oracle_exact_sum": (None, [_vp, _vp, _i, _i, _i, _i]),
    "oracle_has_nonfinite": (_i, [_vp, _sz]),
    "oracle_conv2d": (None, [_vp, _vp, _vp, _vp, _i]),
    "oracle_conv2d_grad_weight": (None, [_vp, _vp, _vp, _vp, _i]),
    "oracle_conv2d_grad_input": (None, [_vp, _vp, _vp, _vp, _i]),
}

_REF_SIG = {
    "ref_scale_exponent": (_i, [_f]),
    "ref_fixed_point": (_i, [_f, _i, _i]),
    "ref_round_to_float": (_f, [ctypes.c_int64, _i]),
    "ref_cpu_gemm": (None, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i]),
    "ref_exact_sum": (None, [_vp, _vp, _i, _i, _i, _i]),
    "ref_conv2d": (None, [_vp, _vp, _vp, _vp, _i]),
    "ref_conv2d_grad_weight": (None, [_vp, _vp, _vp, _vp, _i]),
    "ref_conv2d_grad_input": (None, [_vp, _vp, _vp, _vp, _i]),
}


def build_oracle(with_ref=True):
    """Runs the committed recipe (oracle/Makefile)."""
    targets = ["oracle"] + (["ref"] if with_ref else [])
    subprocess.run(["make", "-s", "-C", HERE] + targets, check=True)


def _load(path, sig):
    lib = ctypes.CDLL(path)
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


if not os.path.exists(LIB_PATH):
    build_oracle(with_ref=False)
lib = _load(LIB_PATH, _SIG)
ref = _load(REF_PATH, _REF_SIG) if os.path.exists(REF_PATH) else None


def _ptr(a):
    return a.ctypes.data


def fnv1a64(arr, h=FNV_OFFSET):
    a = np.ascontiguousarray(arr)
    return lib.oracle_fnv1a64(_ptr(a), a.nbytes, h)


def fnv_chain(*arrays):
    h = FNV_OFFSET
    for a in arrays:
        h = fnv1a64(a, h)
    return h


def gen_normal(n, scale, seed, first=0):
    out = np.empty(int(n), np.float32)
    lib.oracle_gen_normal_at(_ptr(out), out.size, float(scale), int(seed), int(first))
    return out


def gen_uniform(n, scale, seed):
    out = np.empty(int(n), np.float32)
    lib.oracle_gen_uniform(_ptr(out), out.size, float(scale), int(seed))
    return out


def gen_uniform_pm(n, bound, seed, first=0):
    out = np.empty(int(n), np.float32)
    lib.oracle_gen_uniform_pm(_ptr(out), out.size, float(bound), int(seed), int(first))
    return out


HASH_DISTS = ("uniform", "normal", "weights", "wide", "stress")


def gen_hash_inputs(M, N, K, seed, dist):
    """A [M][K], B [K][N] as the reference's hash tool draws them for `dist` (one of HASH_DISTS,
    hash_repro_gemm.cu:20-56)."""
    A = np.empty((int(M), int(K)), np.float32)
    B = np.empty((int(K), int(N)), np.float32)
    assert lib.oracle_gen_hash_inputs(_ptr(A), _ptr(B), int(M), int(N), int(K), int(seed),
                                      HASH_DISTS.index(dist)) == 0
    return A, B


def gen_adversarial(rows, cols, seed, pair_rows=False, negate=False):
    out = np.empty((int(rows), int(cols)), np.float32)
    lib.oracle_gen_adversarial(_ptr(out), int(rows), int(cols), int(seed), int(bool(pair_rows)),
                               int(bool(negate)))
    return out


def splitmix64(n, seed):
    out = np.empty(int(n), np.uint64)
    lib.oracle_splitmix64(_ptr(out), out.size, int(seed))
    return out


def cpu_gemm(A, B, M, N, K, ta=False, tb=False, S=3, nthreads=0):
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    assert A.size == M * K and B.size == N * K
    C = np.empty((M, N), np.float32)
    lib.oracle_cpu_gemm(_ptr(A), _ptr(B), _ptr(C), M, N, K, int(bool(ta)), int(bool(tb)), S,
                        int(nthreads))
    return C


def cpu_gemm_rows(A, B, M, N, K, r0, r1, ta=False, tb=False, S=3, nthreads=0):
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    C = np.empty((r1 - r0, N), np.float32)
    used = lib.oracle_cpu_gemm_rows(_ptr(A), _ptr(B), _ptr(C), M, N, K, int(bool(ta)),
                                    int(bool(tb)), S, int(r0), int(r1), int(nthreads))
    return C, used


def quantize(A, B, M, N, K, ta=False, tb=False, S=3, nthreads=0):
    """Returns X[M,K], Y[N,K] (int32) and eA[M], eB[N] (int32)."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    X = np.empty((M, K), np.int32)
    Y = np.empty((N, K), np.int32)
    eA = np.empty(M, np.int32)
    eB = np.empty(N, np.int32)
    lib.oracle_quantize(_ptr(A), _ptr(B), M, N, K, int(bool(ta)), int(bool(tb)), S, _ptr(X),
                        _ptr(Y), _ptr(eA), _ptr(eB), int(nthreads))
    return X, Y, eA, eB


def exact_products(X, Y, nthreads=0):
    X = np.ascontiguousarray(X, np.int32)
    Y = np.ascontiguousarray(Y, np.int32)
    M, K = X.shape
    N = Y.shape[0]
    T = np.empty((M, N), np.int64)
    lib.oracle_exact_products(_ptr(X), _ptr(Y), _ptr(T), M, N, K, int(nthreads))
    return T


def scale_exponent_n(m):
    m = np.ascontiguousarray(m, np.float32)
    e = np.empty(m.size, np.int32)
    lib.oracle_scale_exponent_n(_ptr(m), _ptr(e), m.size)
    return e


def fixed_point_n(x, se, S):
    x = np.ascontiguousarray(x, np.float32)
    se = np.ascontiguousarray(np.broadcast_to(se, x.shape), np.int32)
    out = np.empty(x.size, np.int32)
    lib.oracle_fixed_point_n(_ptr(x), _ptr(se), int(S), _ptr(out), x.size)
    return out


def round_to_float_n(T, E):
    T = np.ascontiguousarray(T, np.int64)
    E = np.ascontiguousarray(np.broadcast_to(E, T.shape), np.int32)
    out = np.empty(T.size, np.float32)
    lib.oracle_round_to_float_n(_ptr(T), _ptr(E), _ptr(out), T.size)
    return out


def check_scale_exponent_range(lo, hi):
    first = ctypes.c_uint32()
    bad = lib.oracle_check_scale_exponent_range(int(lo), int(hi), ctypes.byref(first))
    return bad, first.value


def ref_cpu_gemm(A, B, M, N, K, ta=False, tb=False, S=3):
    """The reference's own cpu_gemm (oracle/_ref), or None when it was not built."""
    if ref is None:
        return None
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    C = np.empty((M, N), np.float32)
    ref.ref_cpu_gemm(_ptr(A), _ptr(B), _ptr(C), M, N, K, int(bool(ta)), int(bool(tb)), S)
    return C


def exact_sum(x, A, B, C, mean=False):
    """out[b] = exact sum over a, c of x[a][b][c] rounded once (or the mean)."""
    x = np.ascontiguousarray(x, np.float32)
    assert x.size == A * B * C
    out = np.empty(int(B), np.float32)
    lib.oracle_exact_sum(_ptr(x), _ptr(out), int(A), int(B), int(C), int(bool(mean)))
    return out


def has_nonfinite(x):
    x = np.ascontiguousarray(x, np.float32)
    return bool(lib.oracle_has_nonfinite(_ptr(x), x.size))


def ref_exact_sum(x, A, B, C, mean=False):
    """The reference's own accumulator (oracle/_ref), or None when it was not built."""
    if ref is None:
        return None
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(int(B), np.float32)
    ref.ref_exact_sum(_ptr(x), _ptr(out), int(A), int(B), int(C), int(bool(mean)))
    return out


# ---------------------------------------------------------------------------------------
# Convolution. shape = (N, C, H, W, F, KH, KW, SY, SX, PY, PX).
# ---------------------------------------------------------------------------------------

def conv_out_hw(shape):
    N, C, H, W, F, KH, KW, SY, SX, PY, PX = shape
    return (H + 2 * PY - KH) // SY + 1, (W + 2 * PX - KW) // SX + 1


def _shape_arr(shape):
    assert len(shape) == 11
    return np.ascontiguousarray(shape, np.int32)


def _conv_call(fn, a, b, out_shape, shape, S):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty(out_shape, np.float32)
    s = _shape_arr(shape)
    fn(_ptr(a), _ptr(b), _ptr(out), _ptr(s), int(S))
    return out


def conv2d(x, w, shape, S=3):
    N, C, H, W, F = shape[:5]
    OH, OW = conv_out_hw(shape)
    return _conv_call(lib.oracle_conv2d, x, w, (N, F, OH, OW), shape, S)


def conv2d_grad_weight(dy, x, shape, S=3):
    N, C, H, W, F, KH, KW = shape[:7]
    return _conv_call(lib.oracle_conv2d_grad_weight, dy, x, (F, C, KH, KW), shape, S)


def conv2d_grad_input(dy, w, shape, S=3):
    N, C, H, W = shape[:4]
    return _conv_call(lib.oracle_conv2d_grad_input, dy, w, (N, C, H, W), shape, S)


def ref_conv(kind, a, b, shape, S=3):
    """The reference's own repro_conv_cpu.h (oracle/_ref): kind in fwd, dW, dX; None when
    _ref was not built."""
    if ref is None:
        return None
    N, C, H, W, F, KH, KW = shape[:7]
    OH, OW = conv_out_hw(shape)
    fn, out_shape = {"fwd": (ref.ref_conv2d, (N, F, OH, OW)),
                     "dW": (ref.ref_conv2d_grad_weight, (F, C, KH, KW)),
                     "dX": (ref.ref_conv2d_grad_input, (N, C, H, W))}[kind]
    return _conv_call(fn, a, b, out_shape, shape, S)
