"""The contraction's XCD-aware block order (rg_test_block_order, host only): every workgroup of a
plan computes a distinct (item, split part, tile) and together they cover all of them, for
single GEMMs, splits, batches and ragged grids; and the blocks one XCD holds at once touch no
more digit panels than the plain row-major order gives them. The order only decides which block
computes which tile, so it cannot change a bit; the GPU tests compare results with the oracle."""
import ctypes

import numpy as np
import pytest

import bit_reproducible_training_amd as rg
from bit_reproducible_training_amd import _lib

lib = _lib.lib
CUS = 256


def _order(M, N, K, batch=1, num_cus=CUS, **kw):
    cfg = rg.Config(**kw).to_c()
    blocks = ctypes.c_longlong()
    code = lib.rg_test_block_order(M, N, K, ctypes.byref(cfg), 1, num_cus, batch, None, 0,
                                   ctypes.byref(blocks))
    assert code == 0
    n = blocks.value
    coords = np.zeros(4 * max(n, 1), dtype=np.int32)
    code = lib.rg_test_block_order(M, N, K, ctypes.byref(cfg), 1, num_cus, batch,
                                   coords.ctypes.data, coords.size, ctypes.byref(blocks))
    assert code == 0
    plan, _ = rg.plan_for_device(M, N, K, rg.Config(**kw), True, num_cus)
    return coords[: 4 * n].reshape(n, 4), plan


SHAPES = [
    (4096, 4096, 4096, {}),
    # (the GPT-2 K = 768 forward shapes take the band kernel by default, which has no tile
    # order: their 64x64 tile plans pinned)
    (8192, 768, 768, {"trans_b": True, "tile_m": 64, "tile_n": 64}),
    (8192, 768, 3072, {}),
    (8192, 2304, 768, {"trans_b": True, "tile_m": 64, "tile_n": 64}),
    (2304, 768, 8192, {"trans_a": True}),
    (768, 768, 8192, {"trans_a": True}),
    (1024, 1024, 65536, {}),
    (8192, 50257, 768, {"trans_b": True}),
    (3001, 1003, 4001, {}),
    (4096, 4096, 4096, {"tile_m": 64, "tile_n": 64}),
    (4096, 4096, 4096, {"tile_m": 64, "tile_n": 192}),
    (4096, 4096, 4096, {"tile_m": 192, "tile_n": 64}),
    (4096, 4096, 4096, {"split_k": 3}),
    (1000, 700, 5000, {"split_k": 7}),
    (640, 832, 1024, {"slices": 2}),
    (640, 832, 1024, {"slices": 1, "split_k": 2}),
]


@pytest.mark.parametrize("M,N,K,kw", SHAPES)
@pytest.mark.parametrize("batch", [1, 3])
def test_every_tile_part_and_item_exactly_once(M, N, K, kw, batch):
    coords, plan = _order(M, N, K, batch=batch, **kw)
    item, part, tm, tn = coords.T
    if batch == 1:
        tiles_m, tiles_n, split = -(-M // plan.tile_m), -(-N // plan.tile_n), plan.split_k
    else:  # a batch may plan another tile or split: take the grid the hook reports
        tiles_m, tiles_n, split = tm.max() + 1, tn.max() + 1, part.max() + 1
        assert any(-(-M // t) == tiles_m and -(-N // u) == tiles_n
                   for t in (64, 128, 192) for u in (64, 128, 192))
    assert len(coords) == tiles_m * tiles_n * split * batch
    assert item.min() >= 0 and item.max() < batch
    assert part.min() >= 0 and part.max() < split
    assert tm.min() >= 0 and tm.max() < tiles_m
    assert tn.min() >= 0 and tn.max() < tiles_n
    key = ((item.astype(np.int64) * split + part) * tiles_m + tm) * tiles_n + tn
    assert len(np.unique(key)) == len(key)


@pytest.mark.parametrize("cus", [8, 40, 104, 240, 304])
def test_bijection_for_other_device_sizes(cus):
    for M, N, K, kw in SHAPES[:8]:
        coords, plan = _order(M, N, K, num_cus=cus, **kw)
        tiles_m = -(-M // plan.tile_m)
        tiles_n = -(-N // plan.tile_n)
        key = (coords[:, 1].astype(np.int64) * tiles_m + coords[:, 2]) * tiles_n + coords[:, 3]
        assert sorted(key.tolist()) == list(range(tiles_m * tiles_n * plan.split_k))


def _panels_per_xcd_window(coords, plan, per_xcd):
    """Distinct row and column panels (in 64-row units) among the first `per_xcd` blocks each
    XCD receives (workgroup i goes to XCD i mod 8), summed over the 8 XCDs."""
    total = 0
    for x in range(8):
        mine = coords[x::8][:per_xcd]
        rows = {(int(i), int(p), int(r)) for i, p, r in mine[:, :3]}
        cols = {(int(i), int(p), int(c)) for i, p, c in mine[:, [0, 1, 3]]}
        total += len(rows) * plan.tile_m // 64 + len(cols) * plan.tile_n // 64
    return total


@pytest.mark.parametrize("M,N,K,kw", SHAPES[:9])
def test_resident_blocks_share_panels(M, N, K, kw):
    """The first round of blocks on each XCD touches no more panel rows than the row-major
    order (workgroup i -> tile i) would give it, and at least a third fewer where the tile
    columns are few (N = 768: every XCD would otherwise read most row panels)."""
    coords, plan = _order(M, N, K, **kw)
    per_cu = 2 if (plan.tile_m, plan.tile_n) == (64, 64) else 1
    per_xcd = CUS // 8 * per_cu
    tiles_m = -(-M // plan.tile_m)
    tiles_n = -(-N // plan.tile_n)
    n = len(coords)
    lin = np.arange(n)
    tiles = tiles_m * tiles_n
    plain = np.stack([lin // (tiles * plan.split_k), (lin // tiles) % plan.split_k,
                      (lin % tiles) // tiles_n, lin % tiles_n], axis=1)
    ours = _panels_per_xcd_window(coords, plan, per_xcd)
    base = _panels_per_xcd_window(plain, plan, per_xcd)
    assert ours <= base
    if tiles_n % 8 == 0:  # the plain order already keeps each XCD on fixed tile columns
        assert np.array_equal(coords, plain)
    if N == 768 and K <= 3072:
        assert ours * 3 <= base * 2


# Shapes whose long operands take the one-read slicing (padded K past the one-pass limit), with
# panel counts that are and are not multiples of 8: the headline, the GPT-2 weight gradients,
# the LM head's (1571 column panels of 8 parts), a ragged batch, and the convolution weight
# gradients of the widened benchmark (LeNet conv2: 10000 windows, 150 and 16 columns; ResNet-like
# 100352 windows is past the one-read limit and keeps two passes), and column-access operands
# past K = 32768, whose parts are 2.5 times as long (at most 26 per panel).
PSLICE_SHAPES = [
    (4096, 4096, 4096, 1, {}),
    (768, 768, 8192, 1, {"trans_a": True}),
    (2304, 768, 8192, 1, {"trans_a": True}),
    (50257, 768, 8192, 1, {"trans_a": True}),
    (1024, 1024, 65536, 1, {}),
    (1024, 1024, 65536, 1, {"trans_a": True}),
    (300, 40, 40000, 1, {"trans_a": True, "trans_b": True}),
    (16, 150, 10000, 1, {"trans_a": True}),
    (6, 150, 5000, 1, {"trans_a": True}),
    (96, 40, 6000, 3, {"trans_b": True}),
    (200, 70, 20000, 1, {}),
]


@pytest.mark.parametrize("M,N,K,batch,kw", PSLICE_SHAPES)
@pytest.mark.parametrize("num_cus", [256, 304, 80])
def test_one_read_slicing_keeps_each_panel_on_one_xcd(M, N, K, batch, kw, num_cus):
    """The parts of a panel exchange their partial maxima through their XCD's L2, so the
    one-read slicing must run all of them on one XCD (workgroup i on XCD i mod 8): with a panel
    split between two XCDs each part waits out its bound and re-reads the panel's whole K (the
    same bits, about 1 ms later; LeNet conv2's weight gradient took 3.2 ms instead of 0.04)."""
    cfg = rg.Config(**kw).to_c()
    blocks, split = ctypes.c_longlong(), ctypes.c_longlong()
    code = lib.rg_test_pslice_placement(M, N, K, ctypes.byref(cfg), num_cus, batch,
                                        ctypes.byref(blocks), ctypes.byref(split))
    assert code == 0
    assert blocks.value % 8 == 0
    assert split.value == 0, (blocks.value, split.value)


def test_one_read_slicing_placement_hook_sees_the_routes():
    """The hook reports blocks exactly when an operand takes the one-read route: none at K = 1024
    (one pass), some at 4096^3 NN (B, column access) and for a transposed A over K = 8192."""
    def blocks(M, N, K, **kw):
        cfg = rg.Config(**kw).to_c()
        b, s = ctypes.c_longlong(), ctypes.c_longlong()
        assert lib.rg_test_pslice_placement(M, N, K, ctypes.byref(cfg), 256, 1, ctypes.byref(b),
                                            ctypes.byref(s)) == 0
        return b.value
    assert blocks(1024, 1024, 1024) == 0
    assert blocks(4096, 4096, 4096) > 0
    assert blocks(768, 768, 8192, trans_a=True) > 0
    # both operands column-access (TN): the wide parts (2560 k, at most 26 per 32-column panel)
    # reach K = 66560; one more k takes the two passes for both
    assert blocks(64, 64, 66560, trans_a=True) == 2 * 8 * 26
    assert blocks(64, 64, 66561, trans_a=True) == 0
    # at K = 32768 the common parts (1024 k, 32 per panel), one k more the wide ones (13)
    assert blocks(64, 64, 32768, trans_a=True) == 2 * 8 * 32
    assert blocks(64, 64, 32769, trans_a=True) == 2 * 8 * 13
