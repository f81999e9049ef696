"""GPU parity of the exact sum and the non-finite scan (include/repro_sum.h) against the
oracle, through the C ABI.

Mirrors the reference's repro_sum suite (repro_sum_cuda/test_repro_sum.cu:1-6): GPU equals
CPU bit for bit for every layout kind, sum and mean; output identical for many chunk counts
and after shuffling the summation order; special cases (cancellation, overflow, NaN,
subnormals, zeros). Shapes include the reductions of LeNet-5 training at batch 100 and the
Linear bias gradients of the GPT-2 layers at 8192 tokens.
"""
import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from gpu_util import note, to_dev
from oracle import oracle as O
from test_exact_sum import KNOWN, _expected_bits, families

pytestmark = pytest.mark.gpu


def gpu_sum(torch, x, A, B, C, mean=False, chunks=0, ws=None):
    dx = x if hasattr(x, "is_cuda") else to_dev(torch, x)
    cfg = rg.SumConfig(chunks=chunks, mean=mean)
    plan = rg.make_sum_plan(A, B, C, cfg)
    if ws is None or ws.numel() < plan.workspace_bytes:
        ws = torch.empty(max(plan.workspace_bytes, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty(B, dtype=torch.float32, device="cuda")
    out.view(torch.int32).fill_(-1)
    code = rg.repro_sum_fp32_ws(dx.data_ptr(), out.data_ptr(), A, B, C, cfg, ws.data_ptr(),
                                ws.numel(), torch.cuda.current_stream().cuda_stream)
    if code != 0:
        raise rg.ReproGemmError(code, "repro_sum_fp32_ws")
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint32), plan


SHAPES = [
    # (A, B, C, what)
    (100, 120, 1, "LeNet fc1 bias grad"),
    (100, 10, 1, "LeNet fc3 bias grad"),
    (100, 6, 784, "LeNet conv1 bias grad"),
    (100, 16, 100, "LeNet conv2 bias grad"),
    (1, 1, 100, "loss mean"),
    (1, 1000, 10, "softmax row sums"),
    (1, 300, 5000, "long rows"),
    (8192, 768, 1, "GPT-2 proj bias grad"),
    (8192, 3072, 1, "GPT-2 fc bias grad"),
    (3, 5, 7, "tiny"),
    (1, 1, 1, "single"),
    (70000, 3, 1, "tall"),
    (2, 1, 300000, "one long output"),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: s[3])
def test_sum_matches_oracle(torch_gpu, shape):
    torch = torch_gpu
    A, B, C, what = shape
    rng = np.random.default_rng(A * 7 + B * 3 + C)
    fams = families(rng, A * B * C)
    if A * B * C > 2_000_000:
        fams = {k: fams[k] for k in ("normal", "wide")}
    for name, x in fams.items():
        for mean in (False, True):
            note("sum", what, A, B, C, name, "mean" if mean else "sum")
            got, _ = gpu_sum(torch, x, A, B, C, mean)
            want = O.exact_sum(x, A, B, C, mean).view(np.uint32)
            assert np.array_equal(got, want), (what, name, mean)


def test_chunk_and_order_invariance(torch_gpu):
    torch = torch_gpu
    rng = np.random.default_rng(5)
    for A, B, C in [(4096, 70, 1), (64, 9, 1000)]:
        x = families(rng, A * B * C)["wide"].reshape(A, B, C)
        want = O.exact_sum(x, A, B, C).view(np.uint32)
        ws = None
        for chunks in (1, 2, 3, 7, 64, 0):
            note("chunks", A, B, C, chunks)
            got, plan = gpu_sum(torch, x, A, B, C, chunks=chunks, ws=ws)
            assert np.array_equal(got, want), (A, B, C, chunks, plan)
        note("shuffled", A, B, C)
        perm = rng.permutation(A)
        got, _ = gpu_sum(torch, np.ascontiguousarray(x[perm]), A, B, C)
        assert np.array_equal(got, want)


def test_known_answers_on_gpu(torch_gpu):
    torch = torch_gpu
    for values, divisor, expected in KNOWN:
        x = np.array(values, np.float32)
        note("known", values, divisor)
        got, _ = gpu_sum(torch, x, 1, 1, len(x), mean=divisor != 1)
        assert int(got[0]) == _expected_bits(expected), (values, divisor, hex(int(got[0])))
        # The same values as one column of a [len, 1] matrix (columns kernel).
        got, _ = gpu_sum(torch, x, len(x), 1, 1, mean=divisor != 1)
        assert int(got[0]) == _expected_bits(expected), (values, divisor, "columns")


def test_nonfinite_in_one_output_only(torch_gpu):
    torch = torch_gpu
    A, B = 1000, 130
    x = np.random.default_rng(9).standard_normal((A, B)).astype(np.float32)
    x[517, 3] = np.nan
    x[999, 129] = np.inf
    got, _ = gpu_sum(torch, x, A, B, 1, chunks=5)
    want = O.exact_sum(x, A, B, 1).view(np.uint32)
    assert np.array_equal(got, want)
    assert got[3] == 0x7FC00000 and got[129] == 0x7FC00000
    assert np.isfinite(got.view(np.float32)[[0, 1, 2, 4, 128]]).all()


def test_torch_exact_sum_binding(torch_gpu):
    torch = torch_gpu
    x = torch.from_numpy(np.random.default_rng(1).standard_normal((512, 96)).astype(np.float32))
    out = rg.exact_sum(x.cuda(), 512, 96, 1)
    want = O.exact_sum(x.numpy(), 512, 96, 1)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    cpu = rg.exact_sum(x, 512, 96, 1)          # CPU tensor: the CPU implementation, same bits
    assert np.array_equal(cpu.numpy().view(np.uint32), want.view(np.uint32))
    with pytest.raises(ValueError):
        rg.exact_sum(x.cuda(), 512, 95, 1)     # shape mismatch


def test_scan_finite_flags_smallest_op(torch_gpu):
    torch = torch_gpu
    NONE = 2 ** 31 - 1
    flag = torch.full((1,), NONE, dtype=torch.int32, device="cuda")
    clean = torch.randn(100003, device="cuda")
    rg.scan_finite(clean, flag, 3)
    assert int(flag.item()) == NONE
    for n, pos, off in [(1, 0, 0), (100003, 100002, 0), (4096, 17, 1), (100003, 50000, 3)]:
        for value in (float("nan"), float("inf"), float("-inf")):
            base = torch.randn(n + off, device="cuda")
            base[off + pos] = value
            x = base[off:]                      # off != 0: not 16-byte aligned
            note("scan", n, pos, off, value)
            flag.fill_(NONE)
            rg.scan_finite(x, flag, 9)
            rg.scan_finite(clean, flag, 2)
            assert int(flag.item()) == 9
            rg.scan_finite(x, flag, 4)
            assert int(flag.item()) == 4
            rg.scan_finite(x, flag, 6)
            assert int(flag.item()) == 4        # the smallest id wins
