"""The five BASELINE configurations on the GPU: every case's output hash equals the CPU
oracle's (tests/golden/baseline_configs.json, written by tests/golden/make_golden.py),
and for configurations 4 and 5 the bits are identical across split-K values and MFMA
block tiles (compared on the device against the first run)."""
import gc
import json
import os

import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from golden import configs
from gpu_util import note, run, to_dev
from oracle import oracle as O

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SPLITS = (1, 2, 3, 7, 16, 64)
TILES = ((128, 128), (128, 64), (64, 128), (64, 64), (64, 192), (192, 64))
MAX_WS_BYTES = 24 << 30


def _fixtures():
    with open(os.path.join(GOLDEN, "baseline_configs.json")) as f:
        return {c["name"]: c for c in json.load(f)["cases"]}


FX = _fixtures()


def _check_case(torch, case, sweep):
    M, N, K, ta, tb, S = case["M"], case["N"], case["K"], case["ta"], case["tb"], case["S"]
    row = FX[case["name"]]
    A, B = case["make"]()
    assert "%016x" % O.fnv_chain(A, B) == row["in_hash"], case["name"]
    dA, dB = to_dev(torch, A), to_dev(torch, B)
    del A, B
    note("config case", case["name"])
    C0, _, ws = run(torch, dA, dB, M, N, K, rg.Config(slices=S, trans_a=ta, trans_b=tb))
    assert "%016x" % O.fnv1a64(C0.cpu().numpy()) == row["out_hash"], case["name"]
    if sweep:
        ref_bits = C0.view(torch.int32)
        C = torch.empty_like(C0)
        for tm, tn in TILES:
            for split in SPLITS:
                cfg = rg.Config(slices=S, trans_a=ta, trans_b=tb, tile_m=tm, tile_n=tn, split_k=split)
                if rg.make_plan(M, N, K, cfg).workspace_bytes > MAX_WS_BYTES:
                    continue
                note("  sweep %s tiles %dx%d split %d" % (case["name"], tm, tn, split))
                C, _, ws = run(torch, dA, dB, M, N, K, cfg, ws=ws, C=C)
                assert torch.equal(C.view(torch.int32), ref_bits), (tm, tn, split)
    del dA, dB, C0, ws
    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("cfg_id", [1, 2, 3])
def test_baseline_config(torch_gpu, cfg_id):
    for case in configs.ALL[cfg_id]():
        _check_case(torch_gpu, case, sweep=False)


@pytest.mark.parametrize("case", configs.config4() + configs.config5(), ids=lambda c: c["name"])
def test_baseline_large_config_with_sweep(torch_gpu, case):
    _check_case(torch_gpu, case, sweep=True)
