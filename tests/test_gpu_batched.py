"""Strided-batched GEMM (rg_gemm_strided_batched_fp32_ws, bmm) on the GPU.

The reference has no batched GEMM (README.md:29 lists it as still needed; its suite runs the
attention-head GEMMs one head at a time, gpt2_ops_suite.cu:477-483). The definition of a batch
is therefore the plain GEMM of every item: each item must be bit-identical to the oracle's GEMM
of that item alone, with its own row and column scales, whatever the batch, the leading
dimensions, the tile or the split. Pinned by the oracle per item and by the suite's recorded
attention-head hashes (every item of a broadcast batch must reproduce them).
"""
import json
import os

import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import note
from oracle import oracle as O

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _bits(t):
    return t.detach().cpu().numpy().view(np.uint32)


def _oracle_item(a, b, ta, tb, S):
    """a, b: one item's stored matrices (numpy, 2-D)."""
    M, K = (a.shape[1], a.shape[0]) if ta else a.shape
    N = b.shape[0] if tb else b.shape[1]
    return O.cpu_gemm(np.ascontiguousarray(a), np.ascontiguousarray(b), M, N, K, ta, tb, S)


@pytest.mark.parametrize("S", [1, 2, 3])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_batched_items_equal_single_gemms(torch_gpu, S, ta, tb):
    torch = torch_gpu
    rng = np.random.default_rng(10 * S + 2 * ta + tb)
    for batch, M, N, K in [(3, 37, 45, 70), (5, 128, 64, 256), (2, 200, 130, 1000), (3, 20, 12, 9000),
                           (2, 45, 70, 3500)]:
        a_shape = (batch, K, M) if ta else (batch, M, K)
        b_shape = (batch, N, K) if tb else (batch, K, N)
        # Items with very different magnitudes: scales are per item, per row and column.
        A = (rng.standard_normal(a_shape) *
             2.0 ** rng.integers(-20, 20, (batch, 1, 1))).astype(np.float32)
        B = rng.standard_normal(b_shape).astype(np.float32)
        note("batched", batch, M, N, K, "ta=%d tb=%d S=%d" % (ta, tb, S))
        C = rg.bmm(torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda(), ta, tb, S)
        torch.cuda.synchronize()
        for i in range(batch):
            want = _oracle_item(A[i], B[i], ta, tb, S)
            assert np.array_equal(_bits(C[i]), want.view(np.uint32)), (batch, M, N, K, i)


def test_attention_heads_in_place(torch_gpu):
    """Q, K of shape [T, H*D]: head h is the column block h*D..(h+1)*D, read in place with
    lda = H*D and a batch stride of D. scores[h] = Q_h K_h^T and out[h] = P_h V_h."""
    torch = torch_gpu
    T, H, D = 192, 6, 64
    rng = np.random.default_rng(3)
    q = rng.standard_normal((T, H * D)).astype(np.float32)
    k = rng.standard_normal((T, H * D)).astype(np.float32)
    v = rng.standard_normal((T, H * D)).astype(np.float32)
    p = (rng.random((H, T, T)) / T).astype(np.float32)
    dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
    heads = lambda t: t.view(T, H, D).permute(1, 0, 2)          # [H, T, D], strides (D, H*D, 1)
    note("attention scores in place")
    scores = rg.bmm(heads(dq), heads(dk), False, True)
    note("attention PV in place")
    out = rg.bmm(torch.from_numpy(p).cuda(), heads(dv), False, False)
    torch.cuda.synchronize()
    for h in range(H):
        sl = slice(h * D, (h + 1) * D)
        want_s = O.cpu_gemm(np.ascontiguousarray(q[:, sl]), np.ascontiguousarray(k[:, sl]),
                            T, T, D, False, True, 3)
        want_o = O.cpu_gemm(p[h], np.ascontiguousarray(v[:, sl]), T, D, T, False, False, 3)
        assert np.array_equal(_bits(scores[h]), want_s.view(np.uint32)), h
        assert np.array_equal(_bits(out[h]), want_o.view(np.uint32)), h
    # Output written in place too: [T, H*D] with ldc = H*D and item stride D.
    o2 = torch.full((T, H * D), float("nan"), device="cuda")
    rg.bmm(torch.from_numpy(p).cuda(), heads(dv), False, False, out=heads(o2))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(heads(o2).contiguous()), _bits(out))


def test_suite_attention_head_hashes_in_broadcast_batches(torch_gpu):
    """Each recorded attention-head GEMM (cpu.txt:17-22) run as a batch of 4 identical items
    (batch stride 0 for the inputs): every item reproduces the recorded hash."""
    torch = torch_gpu
    with open(os.path.join(GOLDEN, "suite_gemm_s3.json")) as f:
        ops = [op for op in json.load(f)["gemm"] if op["name"].startswith("attn_head")]
    assert len(ops) == 6
    for op in ops:
        M, N, K, ta, tb = op["M"], op["N"], op["K"], op["ta"], op["tb"]
        A = O.gen_normal(M * K, op["sa"], op["seed"])
        B = O.gen_normal(K * N, op["sb"], op["seed"] + 1)
        dA = torch.from_numpy(A).cuda().reshape(1, *((K, M) if ta else (M, K))).expand(4, -1, -1)
        dB = torch.from_numpy(B).cuda().reshape(1, *((N, K) if tb else (K, N))).expand(4, -1, -1)
        note("suite head batch", op["name"])
        C = rg.bmm(dA, dB, ta, tb, 3)
        torch.cuda.synchronize()
        for i in range(4):
            assert "%016x" % O.fnv1a64(C[i].cpu().numpy()) == op["out_hash"], (op["name"], i)


def test_batched_tile_and_split_invariance(torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(8)
    batch, M, N, K = 4, 150, 260, 3000
    A = torch.from_numpy(rng.standard_normal((batch, M, K)).astype(np.float32)).cuda()
    B = torch.from_numpy(rng.standard_normal((batch, K, N)).astype(np.float32)).cuda()
    ref = None
    for tm, tn in [(16, 16), (128, 128), (128, 64), (64, 128), (64, 64)]:
        for split in (1, 3, 7):
            cfg = rg.Config(split_k=split, tile_m=tm, tile_n=tn)
            note("batched tiles", tm, tn, split)
            C = rg.bmm(A, B, cfg=cfg)
            torch.cuda.synchronize()
            if ref is None:
                ref = _bits(C)
                for i in range(batch):
                    want = O.cpu_gemm(A[i].cpu().numpy(), B[i].cpu().numpy(), M, N, K, 0, 0, 3)
                    assert np.array_equal(ref[i], want.view(np.uint32)), i
            else:
                assert np.array_equal(_bits(C), ref), (tm, tn, split)
    cfg = rg.Config(algo=rg.Algo.Reference)
    assert np.array_equal(_bits(rg.bmm(A, B, cfg=cfg)), ref)


def test_batched_argument_errors(torch_gpu):
    torch = torch_gpu
    A = torch.zeros((2, 8, 16), device="cuda")
    B = torch.zeros((2, 16, 4), device="cuda")
    C = torch.zeros((2, 8, 4), device="cuda")
    cfg = rg.Config()
    plan = rg.make_plan_strided_batched(8, 4, 16, 2, cfg)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    call = lambda lda, ldb, ldc, batch, sa=128: rg.repro_gemm_strided_batched_fp32_ws(
        A.data_ptr(), lda, sa, B.data_ptr(), ldb, 64, C.data_ptr(), ldc, 32, 8, 4, 16, batch, cfg,
        ws.data_ptr(), ws.numel())
    assert call(16, 4, 4, 2) == 0
    torch.cuda.synchronize()
    assert call(15, 4, 4, 2) == 1       # lda < K
    assert call(16, 3, 4, 2) == 1       # ldb < N
    assert call(16, 4, 3, 2) == 1       # ldc < N
    assert call(16, 4, 4, 0) == 1       # batch < 1
    assert call(16, 4, 4, 2, sa=-1) == 1
    with pytest.raises(rg.ReproGemmError):
        rg.make_plan_strided_batched(8, 4, 16, 65536, cfg)
    with pytest.raises(ValueError):
        rg.bmm(A, torch.zeros((3, 16, 4), device="cuda"))
