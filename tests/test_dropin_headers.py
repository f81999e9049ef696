"""The reference's own CPU callers of the GEMM's scalar header, built on this repository's
include/repro_gemm_math.h instead of repro_gemm_cuda/repro_gemm_math.cuh, with only their one
`#include "repro_gemm_math.cuh"` line changed (repro_conv_cuda/repro_conv_math.cuh:20,
repro_gemm_cuda/repro_gemm_cpu.h:5): the header is a drop-in for them under g++ (the
reference's CPU build, gpt2_ops_suite/run_suite.sh:17-18), and their outputs equal the
oracle's bit for bit. The edited headers are written to a temporary directory outside the
repository at test time and compiled from there (a quoted include searches the including
file's own directory first); runs only where /root/reference exists."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O

REF = "/root/reference"
REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
pytestmark = pytest.mark.skipif(not os.path.isdir(REF), reason="reference sources not present")

DRIVER = r"""
#include <cstdint>
#include "repro_gemm_cpu.h"
#include "repro_conv_cpu.h"
extern "C" {
void dc_gemm(const float* A, const float* B, float* C, int M, int N, int K, int ta, int tb, int S) {
    repro_gemm::cpu_gemm(A, B, C, M, N, K, ta != 0, tb != 0, S);
}
void dc_conv(int kind, const float* a, const float* b, float* out, const int* s, int S) {
    repro_conv::ConvShape g;
    g.N = s[0]; g.C = s[1]; g.H = s[2]; g.W = s[3]; g.F = s[4]; g.KH = s[5]; g.KW = s[6];
    g.SY = s[7]; g.SX = s[8]; g.PY = s[9]; g.PX = s[10];
    if (kind == 0) repro_conv::cpu_conv2d(a, b, out, g, S);
    else if (kind == 1) repro_conv::cpu_conv2d_grad_weight(a, b, out, g, S);
    else repro_conv::cpu_conv2d_grad_input(a, b, out, g, S);
}
}
"""


def _edited(path, tmp):
    text = open(path).read()
    line = '#include "repro_gemm_math.cuh"'
    assert text.count(line) == 1, path
    out = os.path.join(tmp, os.path.basename(path))
    with open(out, "w") as f:
        f.write(text.replace(line, '#include "repro_gemm_math.h"'))


@pytest.fixture(scope="module")
def dc(tmp_path_factory):
    tmp = str(tmp_path_factory.mktemp("dropin"))
    _edited(os.path.join(REF, "repro_gemm_cuda", "repro_gemm_cpu.h"), tmp)
    _edited(os.path.join(REF, "repro_conv_cuda", "repro_conv_math.cuh"), tmp)
    with open(os.path.join(REF, "repro_conv_cuda", "repro_conv_cpu.h")) as f:  # unchanged
        text = f.read()
    with open(os.path.join(tmp, "repro_conv_cpu.h"), "w") as f:
        f.write(text)
    with open(os.path.join(tmp, "driver.cpp"), "w") as f:
        f.write(DRIVER)
    lib = os.path.join(tmp, "libdropin.so")
    # No reference directory on the include path: repro_gemm_math.cuh cannot be found.
    subprocess.run(["g++", "-O2", "-std=c++17", "-pthread", "-fno-fast-math", "-ffp-contract=off",
                    "-fPIC", "-shared", "-I", tmp, "-I", os.path.join(REPO, "include"),
                    os.path.join(tmp, "driver.cpp"), "-o", lib], check=True)
    L = ctypes.CDLL(lib)
    vp = ctypes.c_void_p
    L.dc_gemm.argtypes = [vp, vp, vp] + [ctypes.c_int] * 6
    L.dc_conv.argtypes = [ctypes.c_int, vp, vp, vp, vp, ctypes.c_int]
    return L


@pytest.mark.parametrize("S", [1, 2, 3])
def test_reference_cpu_gemm_on_this_header(dc, S):
    rng = np.random.default_rng(S)
    for M, N, K, ta, tb in ((33, 17, 91, 0, 0), (20, 45, 300, 1, 0), (64, 8, 1000, 0, 1),
                            (5, 7, 129, 1, 1)):
        A = (rng.standard_normal(M * K) * 2.0 ** rng.integers(-40, 40, M * K)).astype(np.float32)
        B = rng.standard_normal(K * N).astype(np.float32)
        A[:K] = 0.0
        C = np.empty(M * N, np.float32)
        dc.dc_gemm(A.ctypes.data, B.ctypes.data, C.ctypes.data, M, N, K, ta, tb, S)
        want = O.cpu_gemm(A, B, M, N, K, ta, tb, S)
        assert np.array_equal(C.view(np.uint32), want.reshape(-1).view(np.uint32)), (M, N, K, ta, tb)


@pytest.mark.parametrize("S", [1, 3])
def test_reference_cpu_conv_on_this_header(dc, S):
    rng = np.random.default_rng(10 + S)
    for shape in ((2, 3, 9, 8, 4, 3, 3, 1, 1, 1, 1), (3, 2, 11, 10, 5, 5, 3, 2, 1, 2, 0)):
        N, C, H, W, F, KH, KW = shape[:7]
        OH, OW = O.conv_out_hw(shape)
        x = rng.standard_normal(N * C * H * W).astype(np.float32)
        w = (rng.standard_normal(F * C * KH * KW) * 0.1).astype(np.float32)
        dy = (rng.standard_normal(N * F * OH * OW) * 1e-3).astype(np.float32)
        s = np.array(shape, np.int32)
        for kind, a, b, n_out, fn in ((0, x, w, N * F * OH * OW, O.conv2d),
                                      (1, dy, x, F * C * KH * KW, O.conv2d_grad_weight),
                                      (2, dy, w, N * C * H * W, O.conv2d_grad_input)):
            out = np.empty(n_out, np.float32)
            dc.dc_conv(kind, a.ctypes.data, b.ctypes.data, out.ctypes.data, s.ctypes.data, S)
            want = fn(a, b, shape, S).reshape(-1)
            assert np.array_equal(out.view(np.uint32), want.view(np.uint32)), (kind, shape)
