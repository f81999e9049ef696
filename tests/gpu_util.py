"""Shared helpers of the GPU tests: run one GEMM through the C ABI on torch device memory."""
import sys

import numpy as np

import bit_reproducible_training_amd as rg


def note(*args):
    """Names the case on stdout before it touches the GPU."""
    print(*args, flush=True)
    sys.stdout.flush()


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32).reshape(-1)).cuda()


def run(torch, A, B, M, N, K, cfg, ws=None, poison=True, events=None, stream=None, C=None):
    """Runs C = op(A) op(B) with cfg on the current stream; returns (C tensor, plan, ws).
    A and B may be numpy arrays or device tensors. C is poisoned with NaN bytes first."""
    dA = A if hasattr(A, "is_cuda") else to_dev(torch, A)
    dB = B if hasattr(B, "is_cuda") else to_dev(torch, B)
    assert dA.numel() == M * K and dB.numel() == N * K
    plan = rg.make_plan(M, N, K, cfg)
    if ws is None or ws.numel() < plan.workspace_bytes:
        ws = torch.empty(max(plan.workspace_bytes, 1), dtype=torch.uint8, device="cuda")
    if C is None:
        C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    if poison:
        C.view(torch.int32).fill_(-1)
    s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
    code = rg.repro_gemm_fp32_ws(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K, cfg,
                                 ws.data_ptr(), ws.numel(), s, events)
    if code != 0:
        raise rg.ReproGemmError(code, "repro_gemm_fp32_ws")
    torch.cuda.synchronize()
    return C, plan, ws


def hip_events(torch, n, stream=None):
    """n timing events whose HIP handles exist (torch creates them on first record)."""
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    for e in evs:
        e.record(stream) if stream is not None else e.record()
    torch.cuda.synchronize()
    return evs


def bits(C):
    return C.cpu().numpy().view(np.uint32)


def decode_digits(ws_np, off, Rp, Kp, S):
    """Digit panels [Rp/32][Kp/32][S][1024] -> (digits [S, Rp, Kp] int8, X [Rp, Kp] int64)."""
    q = ws_np[off:off + S * Rp * Kp].view(np.int8).reshape(Rp // 32, Kp // 32, S, 2, 32, 16)
    d = q.transpose(2, 0, 4, 1, 3, 5).reshape(S, Rp, Kp)
    X = np.zeros((Rp, Kp), np.int64)
    for p in range(S):
        X = X * 128 + d[p].astype(np.int64)
    return d, X
