"""Split-K plans on a workspace full of random bytes: every part's int64 partials, the exponents
and the digit panels must be written by the call itself before anything reads them. The
workspace is refilled with random bytes before every call and between graph replays, so a
region the call relied on without writing (or read before the writing launch) would show as a
wrong bit against the oracle. Tiles 64x64, 128x128, 128x64, 64x192, 192x64; S = 1..3; splits
2..64; all transposes; a strided batch."""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import note, run, to_dev
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().numpy().view(np.uint32)


def _garbage(torch, ws, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    ws.copy_(torch.randint(0, 256, (ws.numel(),), dtype=torch.uint8, device="cuda", generator=g))


CASES = [  # M, N, K, ta, tb, S, split, tile
    (300, 200, 3000, 0, 0, 3, 2, 16), (300, 200, 3000, 1, 0, 3, 5, 16),
    (257, 129, 4100, 0, 1, 3, 7, (64, 64)), (128, 128, 8192, 1, 1, 3, 16, (128, 128)),
    (700, 500, 2000, 1, 0, 3, 3, (64, 192)), (500, 700, 2000, 0, 0, 3, 4, (192, 64)),
    (400, 300, 2500, 0, 1, 2, 3, 16), (400, 300, 2500, 1, 0, 1, 6, (128, 64)),
    (33, 65, 9000, 0, 0, 3, 64, (64, 64)), (768, 768, 8192, 1, 0, 3, 1, 16),
]


@pytest.mark.parametrize("M,N,K,ta,tb,S,split,tile", CASES)
def test_split_k_matches_oracle_on_garbage_workspace(torch_gpu, M, N, K, ta, tb, S, split, tile):
    torch = torch_gpu
    tm, tn = tile if isinstance(tile, tuple) else (tile, tile)
    cfg = rg.Config(trans_a=ta, trans_b=tb, slices=S, split_k=split, tile_m=tm, tile_n=tn)
    plan = rg.make_plan(M, N, K, cfg)
    assert plan.split_k >= split
    A = O.gen_normal(M * K, 1.0, 4242 + M)
    B = O.gen_normal(K * N, 0.5, 4243 + N)
    want = O.cpu_gemm(A, B, M, N, K, ta, tb, S).view(np.uint32)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    dA, dB = to_dev(torch, A), to_dev(torch, B)
    for rep in range(3):
        note("split-K garbage ws", M, N, K, ta, tb, S, plan.split_k, plan.tile_m, plan.tile_n, rep)
        _garbage(torch, ws, 17 * rep + M)
        C, _, _ = run(torch, dA, dB, M, N, K, cfg, ws=ws)
        assert np.array_equal(_bits(C), want), rep


def test_split_k_graph_replays_on_garbage_workspace(torch_gpu):
    torch = torch_gpu
    M, N, K = 640, 384, 6000
    cfg = rg.Config(trans_a=True, split_k=5)
    plan = rg.make_plan(M, N, K, cfg)
    assert plan.split_k == 5
    torch.manual_seed(11)
    A = torch.randn(M * K, device="cuda")
    B = torch.randn(K * N, device="cuda") * 0.1
    C = torch.empty(M, N, device="cuda")
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")

    def call():
        code = rg.repro_gemm_fp32_ws(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, cfg,
                                     ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
        assert code == 0

    note("split-K graph", M, N, K)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    torch.cuda.synchronize()
    want = O.cpu_gemm(A.cpu().numpy(), B.cpu().numpy(), M, N, K, 1, 0, 3).view(np.uint32)
    for rep in range(4):
        C.fill_(float("nan"))
        _garbage(torch, ws, 99 + rep)      # eager work on the workspace between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(C), want), rep


def test_split_k_batched_items(torch_gpu):
    """A strided batch with split-K: each item's partials follow the previous item's."""
    torch = torch_gpu
    batch, M, N, K = 3, 96, 160, 5000
    torch.manual_seed(5)
    A = torch.randn(batch, M, K, device="cuda")
    B = torch.randn(batch, K, N, device="cuda")
    cfg = rg.Config(split_k=4)
    note("split-K batch", batch, M, N, K)
    C = rg.bmm(A, B, cfg=cfg)
    torch.cuda.synchronize()
    for b in range(batch):
        want = O.cpu_gemm(A[b].cpu().numpy(), B[b].cpu().numpy(), M, N, K, 0, 0, 3).view(np.uint32)
        assert np.array_equal(_bits(C[b]), want.reshape(M, N)), b
