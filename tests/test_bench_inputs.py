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


def test_bench_normal_inputs_match_oracle_stream():
    n = 64
    A, B = bench.make_normal(n)
    assert np.array_equal(A.reshape(-1).view(np.uint32), O.gen_normal(n * n, 1.0, 12345, 0).view(np.uint32))
    assert np.array_equal(B.reshape(-1).view(np.uint32), O.gen_normal(n * n, 1.0, 12345, n * n).view(np.uint32))
    # chunk boundaries of the threaded generator do not change bits
    x = bench.normal_stream(5000, 7, 3, chunk=1000)
    assert np.array_equal(x.view(np.uint32), O.gen_normal(5000, 1.0, 7, 3).view(np.uint32))


def test_traffic_reported_only_for_the_measured_contraction_source(tmp_path, monkeypatch):
    """roofline.traffic is a rocprofv3 figure measured outside the run; bench.py gives it only
    while the contraction source hashes to the one it was measured on."""
    import hashlib

    src = tmp_path / "rg_contract.hip"
    src.write_bytes(b"kernel v1")
    monkeypatch.setattr(bench, "TRAFFIC_SOURCE", str(src))
    monkeypatch.setattr(bench, "TRAFFIC_SOURCE_SHA256", hashlib.sha256(b"kernel v1").hexdigest())
    assert bench.measured_traffic() == bench.TRAFFIC_BYTES
    src.write_bytes(b"kernel v2")
    assert bench.measured_traffic() is None
    monkeypatch.setattr(bench, "TRAFFIC_SOURCE", str(tmp_path / "missing.hip"))
    assert bench.measured_traffic() is None
