"""Worker of test_zz_no_alloc.py::test_noalloc_scratch_is_reserved_at_its_first_use, run in a
fresh process: the device memory the library reserves when it is loaded, when a plain GEMM
runs and when rg_gemm_fp32_noalloc runs for the first time (torch.cuda.mem_get_info, MiB).
The scratch array lives in a code object that holds nothing else, which the runtime loads on
its first use: a process that never calls the entry point never holds the array."""
import ctypes
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import torch  # noqa: E402


def free_mib():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info()[0] / 2 ** 20


def main():
    n = 256
    A = torch.randn(n * n, device="cuda")
    B = torch.randn(n * n, device="cuda")
    C = torch.empty(n * n, device="cuda")
    f0 = free_mib()
    import bit_reproducible_training_amd as rg
    from bit_reproducible_training_amd import _lib

    f1 = free_mib()
    rg.gemm(A, B, n, n, n)
    f2 = free_mib()
    cfg = rg.Config().to_c()
    code = _lib.lib.rg_gemm_fp32_noalloc(A.data_ptr(), B.data_ptr(), C.data_ptr(), n, n, n,
                                         ctypes.byref(cfg), torch.cuda.current_stream().cuda_stream)
    f3 = free_mib()
    print("reserved MiB: import %.1f, plain gemm %.1f, first noalloc call %.1f (code %d)"
          % (f0 - f1, f1 - f2, f2 - f3, code), flush=True)
    scratch = _lib.NOALLOC_SCRATCH_BYTES / 2 ** 20
    ok = code == 0 and f0 - f1 < 16 and f1 - f2 < 64 and f2 - f3 >= scratch - 1
    print("noalloc reserve ok" if ok else "noalloc reserve FAILED", flush=True)
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
