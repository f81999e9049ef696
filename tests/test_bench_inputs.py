"""bench.py regenerates configuration 4's inputs without the oracle; they must be the
same bits as the recipe the fixtures were computed from (tests/golden/configs.py)."""
import numpy as np

import bench
from oracle import oracle as O


def test_bench_adversarial_inputs_match_recipe():
    for rows, cols, seed, pr, neg in ((64, 48, 4001, False, True), (50, 64, 4002, True, False)):
        got = bench._adversarial(rows, cols, seed, pr, neg)
        want = O.gen_adversarial(rows, cols, seed, pr, neg)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
