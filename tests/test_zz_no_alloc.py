"""rg_gemm_fp32_noalloc (include/repro_gemm.h): the GEMM with the library's fixed device
scratch array as its workspace, for callers that cannot allocate. It has no counterpart in the
reference. Through the C ABI, two calls in a row (the second smaller, so it runs on the
scratch the first left behind) must give exactly the bits of rg_gemm_fp32_ws with a workspace
of its own; a plan larger than the scratch is refused before any launch.
"""
import ctypes

import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from bit_reproducible_training_amd import _lib
from gpu_util import note, to_dev
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _noalloc(torch, dA, dB, M, N, K, cfg):
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    C.view(torch.int32).fill_(-1)
    c = cfg.to_c()
    code = _lib.lib.rg_gemm_fp32_noalloc(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K,
                                         ctypes.byref(c), torch.cuda.current_stream().cuda_stream)
    assert code == 0, _lib.error_string(code)
    return C


def _with_workspace(torch, dA, dB, M, N, K, cfg):
    plan = rg.make_plan(M, N, K, cfg)
    ws = torch.empty(max(plan.workspace_bytes, 1), dtype=torch.uint8, device="cuda")
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    C.view(torch.int32).fill_(-1)
    code = rg.repro_gemm_fp32_ws(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K, cfg,
                                 ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert code == 0
    return C


@pytest.mark.parametrize("first,second", [
    ((1024, 1536, 2048, 0, 1, 3), (200, 130, 300, 1, 0, 3)),
    ((4096, 4096, 4096, 0, 0, 3), (64, 10, 84, 0, 1, 2)),
    ((256, 192, 40000, 0, 0, 3), (513, 257, 1000, 1, 1, 1)),    # split-K partials in scratch
])
def test_noalloc_matches_workspace_entry_point(torch_gpu, first, second):
    torch = torch_gpu
    for seed, (M, N, K, ta, tb, S) in ((31, first), (37, second)):
        note("noalloc", M, N, K, ta, tb, S)
        A = O.gen_normal(M * K, 1.0, seed)
        B = O.gen_normal(K * N, 0.1, seed + 1)
        dA, dB = to_dev(torch, A), to_dev(torch, B)
        cfg = rg.Config(slices=S, trans_a=bool(ta), trans_b=bool(tb))
        assert rg.make_plan(M, N, K, cfg).workspace_bytes <= _lib.NOALLOC_SCRATCH_BYTES
        got = _noalloc(torch, dA, dB, M, N, K, cfg)
        want = _with_workspace(torch, dA, dB, M, N, K, cfg)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int32), want.view(torch.int32)), (M, N, K, ta, tb, S)
        if M * N * K <= 1 << 27:
            ref = O.cpu_gemm(A, B, M, N, K, ta, tb, S)
            assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_noalloc_first_call_under_graph_capture(torch_gpu):
    """The entry point's first call in a process, made inside torch.cuda.graph capture (the
    scratch address is looked up then), replayed three times against eager rg_gemm_fp32_ws."""
    import os
    import subprocess
    import sys

    worker = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_capture_worker.py")
    note("noalloc first call under capture (worker process)")
    r = subprocess.run([sys.executable, worker], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True, timeout=300)
    assert r.returncode == 0 and "noalloc capture ok" in r.stdout, r.stdout[-2000:]


def test_noalloc_scratch_is_reserved_at_its_first_use(torch_gpu):
    """The 128 MiB scratch array is reserved on a GPU when the entry point is first called
    there, not when the library is loaded or a plain GEMM runs (fresh worker process; measured
    with torch.cuda.mem_get_info)."""
    import os
    import subprocess
    import sys

    worker = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_reserve_worker.py")
    note("noalloc scratch reservation (worker process)")
    r = subprocess.run([sys.executable, worker], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True, timeout=300)
    assert r.returncode == 0 and "noalloc reserve ok" in r.stdout, r.stdout[-2000:]


def test_noalloc_refuses_plans_beyond_the_scratch(torch_gpu):
    torch = torch_gpu
    M = N = K = 8192                     # digit panels alone: 2 * 8192 * 8192 * 3 B = 384 MiB
    cfg = rg.Config(slices=3)
    assert rg.make_plan(M, N, K, cfg).workspace_bytes > _lib.NOALLOC_SCRATCH_BYTES
    d = torch.empty(16, device="cuda")
    c = cfg.to_c()
    code = _lib.lib.rg_gemm_fp32_noalloc(d.data_ptr(), d.data_ptr(), d.data_ptr(), M, N, K,
                                         ctypes.byref(c), torch.cuda.current_stream().cuda_stream)
    assert code == _lib.HIP_ERROR_INVALID_VALUE
    code = _lib.lib.rg_gemm_fp32_noalloc(None, d.data_ptr(), d.data_ptr(), 4, 4, 4,
                                         ctypes.byref(c), None)
    assert code == _lib.HIP_ERROR_INVALID_VALUE
