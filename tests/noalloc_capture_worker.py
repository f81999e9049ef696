"""Worker of tests/test_zz_no_alloc.py: in a fresh process, the first rg_gemm_fp32_noalloc call
on the device is made while a HIP graph is being captured (so the scratch array's address is
looked up during capture). The graph is replayed three times with eager work and
synchronisations between the replays; every replay must give exactly the bits of eager
rg_gemm_fp32_ws. Prints "noalloc capture ok" on success.
"""
import ctypes
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))

import torch  # noqa: E402

import bit_reproducible_training_amd as rg  # noqa: E402
from bit_reproducible_training_amd import _lib  # noqa: E402


def main():
    M, N, K = 1000, 700, 5000  # the one-read slicing of op(B) and a two-pass route in one plan
    cfg = rg.Config(slices=3)
    c = cfg.to_c()
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    A = torch.randn(M * K, device="cuda", generator=g)
    B = torch.randn(K * N, device="cuda", generator=g)
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        code = _lib.lib.rg_gemm_fp32_noalloc(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K,
                                             ctypes.byref(c), torch.cuda.current_stream().cuda_stream)
    assert code == 0, "noalloc under capture: %s" % _lib.error_string(code)

    plan = rg.make_plan(M, N, K, cfg)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    want = torch.empty_like(C)
    for rep in range(3):
        C.view(torch.int32).fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        code = rg.repro_gemm_fp32_ws(A.data_ptr(), B.data_ptr(), want.data_ptr(), M, N, K, cfg,
                                     ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
        assert code == 0
        torch.cuda.synchronize()
        assert torch.equal(C.view(torch.int32), want.view(torch.int32)), "replay %d differs" % rep
        A.mul_(-0.5)  # new inputs in place for the next replay (eager work between replays)
        torch.cuda.synchronize()
    print("noalloc capture ok", flush=True)


if __name__ == "__main__":
    main()
