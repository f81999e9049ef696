"""The C++ interface, include/repro_gemm.hpp (the reference's names and signatures,
repro_gemm_cuda/repro_gemm.cuh:25-75, on HIP types), through the test driver
tests/cxx_api_driver.cpp (built by __graft_entry__.build() into tests/_build/libcxxapi.so):
Config's defaults (repro_gemm.cuh:32-41), MAX_SLICES, algo_name, make_plan's plans and error
codes (no device needed for the Reference algorithm), and on the GPU both run paths,
repro_gemm_fp32_ws with stage events and repro_gemm_fp32, against the oracle bit for bit."""
import ctypes
import os

import numpy as np
import pytest

import bit_reproducible_training_amd as rg  # binds the HIP runtime before the driver loads
from gpu_util import bits, note, to_dev
from oracle import oracle as O

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_build", "libcxxapi.so")
AUTO, REFERENCE, TILED, TENSOR_CORE = 0, 1, 2, 3


@pytest.fixture(scope="module")
def cx():
    if not os.path.exists(LIB):
        raise RuntimeError("%s is not built: run __graft_entry__.build()" % LIB)
    L = ctypes.CDLL(LIB)
    vp, i = ctypes.c_void_p, ctypes.c_int
    L.cx_config_defaults.argtypes = [vp]
    L.cx_algo_name.restype = ctypes.c_char_p
    L.cx_algo_name.argtypes = [i]
    L.cx_make_plan.argtypes = [i] * 9 + [vp, vp, vp]
    L.cx_gemm_ws.argtypes = [vp, vp, vp] + [i] * 9 + [vp, ctypes.c_ulonglong, vp, vp]
    L.cx_gemm.argtypes = [vp, vp, vp] + [i] * 6 + [vp]
    return L


def _plan(cx, M, N, K, algo=AUTO, S=3, ta=0, tb=0, split=1, tile=0):
    a, s, w = ctypes.c_int(), ctypes.c_int(), ctypes.c_ulonglong()
    e = cx.cx_make_plan(M, N, K, algo, S, ta, tb, split, tile, ctypes.byref(a), ctypes.byref(s),
                        ctypes.byref(w))
    return e, a.value, s.value, w.value


def test_config_defaults_and_names(cx):
    d = (ctypes.c_int * 8)()
    cx.cx_config_defaults(d)
    # split_k 1, tile 16x16x32, Algo::Auto, 3 slices, no transposes (repro_gemm.cuh:32-41)
    assert list(d) == [1, 16, 16, 32, AUTO, 3, 0, 0]
    assert cx.cx_max_slices() == 3
    names = [cx.cx_algo_name(a).decode() for a in (AUTO, REFERENCE, TILED, TENSOR_CORE)]
    assert names == [rg.algo_name(a) for a in (rg.Algo.Auto, rg.Algo.Reference, rg.Algo.Tiled,
                                               rg.Algo.TensorCore)]


def test_make_plan_reference_and_errors(cx):
    e, algo, split, ws = _plan(cx, 133, 77, 301, algo=REFERENCE, split=7)
    assert (e, algo, split) == (0, REFERENCE, 7) and ws > 0
    assert ws == rg.make_plan(133, 77, 301, rg.Config(algo=rg.Algo.Reference, split_k=7)).workspace_bytes
    for args in ((0, 4, 4), (4, 0, 4), (4, 4, 0), (-1, 4, 4)):
        assert _plan(cx, *args, algo=REFERENCE)[0] == 1, args        # hipErrorInvalidValue
    assert _plan(cx, 8, 8, 8, algo=REFERENCE, S=4)[0] == 1
    assert _plan(cx, 8, 8, 8, algo=REFERENCE, S=0)[0] == 1
    assert _plan(cx, 8, 8, 8, algo=REFERENCE, split=0)[0] == 1


@pytest.mark.gpu
def test_cxx_interface_runs_match_oracle(cx, torch_gpu):
    torch = torch_gpu
    stream = torch.cuda.current_stream().cuda_stream
    for M, N, K, ta, tb, S in ((133, 77, 301, 0, 0, 3), (96, 200, 1000, 1, 0, 2),
                               (64, 50, 130, 0, 1, 1), (40, 33, 5000, 1, 1, 3)):
        rng = np.random.default_rng(M + N + K)
        A = rng.standard_normal(M * K).astype(np.float32)
        B = (rng.standard_normal(K * N) * 2.0 ** rng.integers(-20, 20, K * N)).astype(np.float32)
        want = O.cpu_gemm(A, B, M, N, K, ta, tb, S).view(np.uint32)
        dA, dB = to_dev(torch, A), to_dev(torch, B)
        C = torch.empty(M, N, device="cuda")
        for algo, split, tile in ((AUTO, 1, 0), (TENSOR_CORE, 3, 64), (TILED, 1, 0), (REFERENCE, 2, 0)):
            e, _, _, nbytes = _plan(cx, M, N, K, algo, S, ta, tb, split, tile)
            assert e == 0
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
            C.fill_(float("nan"))
            stage = (ctypes.c_float * 3)()
            note("c++ ws", M, N, K, ta, tb, S, algo, split)
            code = cx.cx_gemm_ws(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K, algo, S, ta,
                                 tb, split, tile, ws.data_ptr(), ws.numel(), stream, stage)
            assert code == 0
            assert min(stage) >= 0.0
            assert np.array_equal(bits(C), want), (algo, split)
        C.fill_(float("nan"))
        note("c++ convenience", M, N, K)
        assert cx.cx_gemm(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K, S, ta, tb, stream) == 0
        assert np.array_equal(bits(C), want)
