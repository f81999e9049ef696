"""One process of the cross-process determinism check (restates repro_gemm_cuda/run_repro.sh:
87-112 with hash_repro_gemm's loops, hash_repro_gemm.cu:115-143): for every (shape, input
distribution, S) it runs every algorithm x split_k x run on the GPU, requires all of them to give
the same output bits, and prints one line

    RESULT M=.. N=.. K=.. S=.. dist=.. hash=<fnv1a64 of the output bits>

Run by tests/test_gpu_cross_process.py as a separate Python process, several times; not a test
module itself.
"""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, HERE)

import numpy as np  # noqa: E402

# Shapes and split lists of run_repro.sh:23-28 (ragged 129x77x1000; K = 7 clamps split_k > K).
SHAPES = [(256, 256, 1024, (1, 2, 3, 4, 7, 8, 16, 64)), (129, 77, 1000, (1, 2, 3, 5, 7, 13, 64)),
          (64, 64, 7, (1, 2, 3, 7, 16)), (1024, 1024, 4096, (1, 2, 7))]
SLICES = (1, 3)       # run_repro.sh:16 default
RUNS = 2
SEED = 12345


def main():
    import torch

    import bit_reproducible_training_amd as rg
    from oracle import oracle as O

    algos = [rg.Algo.Reference, rg.Algo.Tiled, rg.Algo.TensorCore]
    for M, N, K, splits in SHAPES:
        for dist in O.HASH_DISTS:
            A, B = O.gen_hash_inputs(M, N, K, SEED, dist)
            dA = torch.from_numpy(A.reshape(-1)).cuda()
            dB = torch.from_numpy(B.reshape(-1)).cuda()
            C = torch.empty((M, N), dtype=torch.float32, device="cuda")
            for S in SLICES:
                first = None
                for algo in algos:
                    for split in splits:
                        cfg = rg.Config(algo=algo, slices=S, split_k=split)
                        plan = rg.make_plan(M, N, K, cfg)
                        ws = torch.empty(max(plan.workspace_bytes, 1), dtype=torch.uint8, device="cuda")
                        for _ in range(RUNS):
                            C.view(torch.int32).fill_(-1)    # poisoned, as the tool does
                            code = rg.repro_gemm_fp32_ws(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K,
                                                         cfg, ws.data_ptr(), ws.numel(),
                                                         torch.cuda.current_stream().cuda_stream)
                            if code != 0:
                                print("ERROR code %d M=%d N=%d K=%d S=%d %s split %d" % (code, M, N, K, S, algo.name, split))
                                return 1
                            torch.cuda.synchronize()
                            bits = C.cpu().numpy().view(np.uint32)
                            if first is None:
                                first = bits.copy()
                            elif not np.array_equal(first, bits):
                                print("MISMATCH M=%d N=%d K=%d S=%d dist=%s %s split %d" % (M, N, K, S, dist, algo.name, split))
                                return 1
                print("RESULT M=%d N=%d K=%d S=%d dist=%s hash=%016x" % (M, N, K, S, dist,
                                                                        O.fnv1a64(first.view(np.float32))),
                      flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
