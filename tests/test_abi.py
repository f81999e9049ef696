"""The C ABI library on the host: it loads, exports every symbol include/*.h declares, and its planner behaves as the reference's make_plan does
(repro_gemm_cuda/repro_gemm.cu:390-439, 503-509). No kernel is launched here."""
import ctypes
import math
import os
import re

import pytest

import bit_reproducible_training_amd as rg
from bit_reproducible_training_amd import _lib

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_symbols():
    names = set()
    for header in ("repro_gemm.h", "repro_sum.h", "repro_conv.h"):
        with open(os.path.join(REPO, "include", header)) as f:
            names |= set(re.findall(r"\b(rg_[a-z0-9_]+)\s*\(", f.read()))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    declared = _declared_symbols()
    assert declared, "no declarations found"
    for name in declared:
        assert hasattr(_lib.lib, name), name
    assert set(declared) == set(_lib.EXPORTED)


def test_single_hip_runtime_in_process():
    """The library and torch share one HIP runtime (two in one process crash)."""
    import torch  # noqa: F401

    assert len(_lib.hip_runtimes_mapped()) == 1, _lib.hip_runtimes_mapped()


def test_config_defaults_match_reference():
    c = _lib.rg_config()
    _lib.lib.rg_config_init(ctypes.byref(c))
    assert (c.split_k, c.tile_m, c.tile_n, c.tile_k, c.algo, c.slices, c.trans_a, c.trans_b) == \
        (1, 16, 16, 32, 0, 3, 0, 0)
    d = rg.Config()
    assert (d.split_k, d.tile_m, d.tile_n, d.tile_k, int(d.algo), d.slices) == (1, 16, 16, 32, 0, 3)


def test_algo_names():
    assert [rg.algo_name(a) for a in (0, 1, 2, 3)] == ["auto", "ref", "tiled", "tc"]
    assert rg.algo_name(9) == "?"


def _plan(M, N, K, **kw):
    return rg.plan_for_device(M, N, K, rg.Config(**kw), is_gfx950=True, num_cus=256)


@pytest.mark.parametrize("args", [(0, 4, 4), (4, 0, 4), (4, 4, 0), (-1, 4, 4)])
def test_invalid_sizes(args):
    with pytest.raises(rg.ReproGemmError) as e:
        _plan(*args)
    assert e.value.code == _lib.HIP_ERROR_INVALID_VALUE


@pytest.mark.parametrize("kw", [dict(split_k=0), dict(slices=0), dict(slices=4), dict(algo=7)])
def test_invalid_config(kw):
    with pytest.raises(rg.ReproGemmError) as e:
        _plan(64, 64, 64, **kw)
    assert e.value.code == _lib.HIP_ERROR_INVALID_VALUE


@pytest.mark.parametrize("S", [1, 2, 3])
def test_k_bound_for_exact_int64(S):
    # K * maxX^2 <= 2^62 with maxX = 127*128^(S-1) + 64*sum_{t<S-1} 128^t
    d = 127 * 128 ** (S - 1) + sum(64 * 128 ** t for t in range(S - 1))
    kmax = (2 ** 62) // (d * d)
    kmax = min(kmax, 2 ** 31 - 1)
    if kmax < 2 ** 31 - 1:
        _plan(1, 1, kmax, slices=S)
        with pytest.raises(rg.ReproGemmError):
            _plan(1, 1, kmax + 1, slices=S)
    if S == 3:
        assert 1_000_000 < kmax < 1_100_000  # "S=3 allows K up to about 1,000,000"


def test_not_supported_off_gfx950():
    with pytest.raises(rg.ReproGemmError) as e:
        rg.plan_for_device(64, 64, 64, rg.Config(), is_gfx950=False, num_cus=256)
    assert e.value.code == _lib.HIP_ERROR_NOT_SUPPORTED
    p, _ = rg.plan_for_device(64, 64, 64, rg.Config(algo=rg.Algo.Reference), is_gfx950=False,
                              num_cus=256)
    assert p.algo == rg.Algo.Reference


def test_auto_resolves_to_mfma():
    p, _ = _plan(4096, 4096, 4096)
    assert p.algo == rg.Algo.TensorCore and (p.tile_m, p.tile_n) == (128, 128)
    p, _ = _plan(64, 10, 84)              # small: the one-launch kernel's 32x32 tiles
    assert p.algo == rg.Algo.TensorCore and (p.tile_m, p.tile_n) == (32, 32)
    p, _ = _plan(64, 10, 84, tile_m=64, tile_n=64)
    assert p.algo == rg.Algo.TensorCore and (p.tile_m, p.tile_n) == (64, 64)
    p, _ = _plan(256, 256, 256, algo=rg.Algo.Tiled)
    assert p.algo == rg.Algo.Tiled and (p.tile_m, p.tile_n) == (64, 64)


@pytest.mark.parametrize("tm,tn", [(128, 128), (128, 64), (64, 128), (64, 64), (64, 192), (192, 64)])
def test_tile_hints(tm, tn):
    p, info = _plan(300, 200, 100, tile_m=tm, tile_n=tn)
    assert (p.tile_m, p.tile_n) == (tm, tn)
    assert info.Mp % tm == 0 and info.Np % tn == 0 and info.Mp >= 300 and info.Np >= 200
    if tm == 192 or tn == 192:  # twelve-wavefront tiles: S = 3 only, else the planner's choice
        p, _ = _plan(300, 200, 100, tile_m=tm, tile_n=tn, slices=2)
        assert (p.tile_m, p.tile_n) != (tm, tn)


@pytest.mark.parametrize("S,limit", [(1, 133120), (2, 66560), (3, 44352)])
def test_split_raised_for_exact_int32(S, limit):
    """Each part spans at most floor((2^31-1) / level_bound / 64) * 64 values of k."""
    big = 4096  # enough output tiles to occupy 256 compute units: no occupancy split
    p, _ = _plan(big, big, limit, slices=S)
    assert p.split_k == 1
    p, _ = _plan(big, big, limit + 64, slices=S)
    assert p.split_k == 2
    p, _ = _plan(big, big, 3 * limit, slices=S, split_k=1)
    assert p.split_k == 3


def test_default_plan_follows_the_cost_model():
    """With the default split_k = 1 and tile hints, the planner picks the block tile (128x128,
    64x64, at S = 3 the twelve-wavefront 192x64 / 64x192, in that order on a tie, then the
    eight-wavefront 128x64 / 64x128) and split with the lowest
    estimated time: waves of blocks over the GPU's block slots times the stages of a part, plus
    the int64 partials of a split. The cases below were measured on MI355X over every block tile
    x split, and the chosen plan was the fastest (512x512x8192 within 10.5%). An explicit split_k
    is honoured; one-stage K is never split."""
    p, _ = _plan(64, 64, 65536)           # 1 tile, 1024 stages: one wave of 512 parts
    assert (p.tile_m, p.tile_n, p.split_k) == (64, 64, 512)
    p, _ = _plan(1024, 64, 1024)          # 16 tiles of 64x64, 16 stages: split to fill a wave
    assert (p.tile_m, p.tile_n) == (64, 64) and p.split_k >= 8
    p, _ = _plan(3072, 768, 8192, trans_a=True)   # 192 tiles of 192x64 = one wave, no partials
    assert (p.tile_m, p.tile_n, p.split_k) == (192, 64, 1)  # (64x192 ties: 192x64 measured faster)
    p, _ = _plan(768, 3072, 8192, trans_a=True)
    assert (p.tile_m, p.tile_n, p.split_k) == (192, 64, 1)
    p, _ = _plan(768, 768, 8192, trans_a=True)    # 48 tiles of 192x64 x 5 parts
    assert (p.tile_m, p.tile_n, p.split_k) == (192, 64, 5)
    p, _ = _plan(2304, 768, 8192, trans_a=True)   # 216 tiles of 128x64 (8 wavefronts), no parts
    assert (p.tile_m, p.tile_n, p.split_k) == (128, 64, 1)
    p, _ = _plan(8192, 768, 3072)         # 512 tiles of 64x192 = two waves of 48 stages
    assert (p.tile_m, p.tile_n, p.split_k) == (64, 192, 1)
    p, _ = _plan(1024, 1024, 65536)       # 64 tiles of 128x128, 1024 stages
    assert (p.tile_m, p.tile_n, p.split_k) == (128, 128, 4)
    p, _ = _plan(8192, 768, 768, trans_b=True, tile_m=64, tile_n=64)  # 3 waves of 512 tiles
    assert (p.tile_m, p.tile_n, p.split_k) == (64, 64, 1)
    p, _ = _plan(1024, 768, 768, trans_b=True)    # one wave either way: no split traffic
    assert p.split_k == 1
    p, _ = _plan(8192, 768, 3072, tile_m=64, tile_n=64)   # a pinned tile is kept
    assert (p.tile_m, p.tile_n, p.split_k) == (64, 64, 1)
    p, _ = _plan(50257, 768, 8192, trans_a=True)  # LM-head weight gradient
    assert (p.tile_m, p.tile_n, p.split_k) == (128, 128, 1)
    p, _ = _plan(1024, 1024, 64)          # one stage only
    assert p.split_k == 1
    p, _ = _plan(1024, 64, 1024, split_k=2)
    assert p.split_k == 2
    p, _ = _plan(4096, 4096, 4096)        # 1024 tiles of 128x128 = 4 full waves
    assert (p.tile_m, p.tile_n, p.split_k) == (128, 128, 1)
    p, _ = _plan(8192, 768, 3072, slices=2)   # the twelve-wavefront tiles exist at S = 3 only
    assert (p.tile_m, p.tile_n) in ((128, 128), (64, 64))


def test_band_kernel_plans():
    """op(A) read along rows with K <= 1024 over many rows takes the band kernel (plan 32 x W:
    blocks of 32 rows of op(A) by W columns) where its cost model beats the best tile plan plus
    op(A)'s slicing: the GPT-2 forward and input-gradient GEMMs at N = 768 and 2304 (measured on
    MI355X: 3-18% faster than the 64x64 tiles), not N = 3072 (the 128x128 tiles 2% faster), not
    a transposed op(A), K past 1024, a batch, a pinned tile or split. A pinned 32 x W tile (W >= 64,
    a multiple of 32) asks for it; the workspace then holds op(B)'s regions only."""
    for tb in (True, False):
        p, _ = _plan(8192, 768, 768, trans_b=tb)      # attn_proj forward (NT) and dX (NN)
        assert (p.tile_m, p.tile_n, p.split_k) == (32, 768, 1)
    p, _ = _plan(8192, 2304, 768, trans_b=True)       # qkv forward
    assert (p.tile_m, p.tile_n, p.split_k) == (32, 2304, 1)
    p, _ = _plan(8192, 3072, 768, trans_b=True)       # mlp_fc forward
    assert (p.tile_m, p.tile_n) == (128, 128)
    for kw in (dict(trans_a=True), dict(split_k=2), dict(tile_m=64, tile_n=64),
               dict(algo=rg.Algo.Tiled)):
        p, _ = _plan(8192, 768, 768, **kw)
        assert p.tile_m != 32, kw
    p, _ = _plan(8192, 768, 1056)                     # K past the band's LDS panels
    assert p.tile_m != 32
    p, info = _plan(97, 70, 203, tile_m=32, tile_n=64)
    assert (p.tile_m, p.tile_n, p.split_k) == (32, 64, 1)
    assert info.Np == 128 and info.qa == info.qb == 0   # two column groups; no op(A) regions
    p, _ = _plan(97, 70, 203, tile_m=32, tile_n=64, trans_a=True)   # not for a transposed op(A)
    assert (p.tile_m, p.tile_n) != (32, 64)
    p, _ = _plan(97, 70, 203, tile_m=32, tile_n=48)   # W must be a multiple of 32
    assert (p.tile_m, p.tile_n) != (32, 48)


def test_small_shapes_take_the_one_launch_kernel():
    """Plain GEMMs with K <= 512 and at most one 32x32 tile per compute unit run as one launch
    (nothing of the workspace used); a pinned 64/128 tile, Tiled, an explicit split or a longer K
    keep the pipeline, and a pinned 32x32 tile asks for the one-launch kernel whenever K allows."""
    for M, N, K in ((256, 256, 256), (64, 120, 400), (64, 400, 120), (120, 400, 64), (64, 10, 84),
                    (10, 84, 64), (1, 1, 1), (33, 47, 512)):
        for S in (1, 2, 3):
            p, info = _plan(M, N, K, slices=S)
            assert (p.tile_m, p.tile_n, p.split_k) == (32, 32, 1), (M, N, K, S)
            assert p.algo == rg.Algo.TensorCore and info.part == -1
            assert 0 < p.workspace_bytes <= 256
    for kw in (dict(tile_m=64, tile_n=64), dict(algo=rg.Algo.Tiled), dict(split_k=2),
               dict(algo=rg.Algo.Reference)):
        p, _ = _plan(64, 120, 400, **kw)
        assert (p.tile_m, p.tile_n) != (32, 32), kw
    p, _ = _plan(64, 120, 513)            # K past the kernel's LDS panels
    assert (p.tile_m, p.tile_n) == (64, 64)
    p, _ = _plan(512, 512, 512)           # 256 tiles: one per compute unit
    assert (p.tile_m, p.tile_n) == (32, 32)
    p, _ = _plan(512, 544, 512)           # 272 tiles
    assert (p.tile_m, p.tile_n) != (32, 32)
    p, _ = rg.plan_for_device(512, 544, 512, rg.Config(), is_gfx950=True, num_cus=304)
    assert (p.tile_m, p.tile_n) == (32, 32)
    p, _ = _plan(4096, 4096, 256)         # too many tiles: the pipeline
    assert (p.tile_m, p.tile_n) != (32, 32)
    p, _ = _plan(4096, 4096, 256, tile_m=32, tile_n=32)   # pinned
    assert (p.tile_m, p.tile_n) == (32, 32)
    p, _ = _plan(64, 64, 1024, tile_m=32, tile_n=32)      # pinned, but K too long: planner's choice
    assert (p.tile_m, p.tile_n) != (32, 32)
    # pinned, but 2^22 tiles of 1024 threads would not fit one launch dimension (2^32 work-items):
    # the pipeline, whose grid fits
    p, _ = _plan(65536, 65536, 256, tile_m=32, tile_n=32)
    assert (p.tile_m, p.tile_n) != (32, 32) and p.algo == rg.Algo.TensorCore
    p, _ = _plan(65536, 65504, 256, tile_m=32, tile_n=32)  # one tile column fewer: still fits
    assert (p.tile_m, p.tile_n) == (32, 32)


def test_split_clamped_to_k_steps():
    p, _ = _plan(4096, 4096, 100, split_k=64)
    assert p.split_k == 2  # Kp = 128 -> two stages of 64
    p, _ = _plan(64, 64, 7, split_k=64, algo=rg.Algo.Reference)
    assert p.split_k == 7  # the reference path clamps split to K


def test_workspace_layout_regions():
    for kw in (dict(tile_m=64, tile_n=64), dict(split_k=4), dict(algo=rg.Algo.Reference, split_k=3),
               dict(slices=1, tile_m=128, tile_n=64)):
        p, info = _plan(133, 77, 301, **kw)
        S = kw.get("slices", 3)
        elem = 4 if kw.get("algo") == rg.Algo.Reference else S
        assert info.qa % 256 == 0 and info.qb % 256 == 0 and info.ea % 256 == 0
        assert info.qb >= info.qa + info.Mp * info.Kp * elem
        assert info.ea >= info.qb + info.Np * info.Kp * elem
        assert info.Kp % 64 == 0 and info.Kp >= 301
        if p.split_k > 1:
            assert info.part >= 0
            assert p.workspace_bytes >= info.part + p.split_k * 133 * 77 * 8
        else:
            assert info.part == -1
        assert p.workspace_bytes % 256 == 0


def test_workspace_depends_only_on_shape_and_config():
    a, _ = _plan(1000, 1000, 1000)
    b, _ = _plan(1000, 1000, 1000)
    assert a == b


def test_reference_plan_needs_no_device():
    """The Reference algorithm never queries the device (like the reference, which queries
    only for Auto/TensorCore): make_plan works on a host without a GPU."""
    p = rg.make_plan(133, 77, 301, rg.Config(algo=rg.Algo.Reference))
    assert p.algo == rg.Algo.Reference and p.split_k == 1


def test_null_pointers_rejected_before_any_launch():
    c = rg.Config(algo=rg.Algo.Reference)
    assert rg.repro_gemm_fp32_ws(None, 1, 1, 4, 4, 4, c, 1, 1 << 20) == _lib.HIP_ERROR_INVALID_VALUE
    assert rg.repro_gemm_fp32_ws(1, 1, 1, 4, 4, 4, c, None, 1 << 20) == _lib.HIP_ERROR_INVALID_VALUE
    assert rg.repro_gemm_fp32_ws(1, 1, 1, 4, 4, 4, c, 1, 1) == _lib.HIP_ERROR_INVALID_VALUE


def test_max_fixed_point_constant():
    assert math.isclose(127 * 128 ** 2 + 64 * 129, 2089024)


def test_mfma_probe_rejects_unknown_operand_modes():
    """rg_measure_mfma_int8_rate checks its arguments before touching a device."""
    out = ctypes.c_double()
    for mode in (-1, 3):
        assert _lib.lib.rg_measure_mfma_int8_rate(mode, ctypes.byref(out)) == 1
    assert _lib.lib.rg_measure_mfma_int8_rate(1, None) == 1
