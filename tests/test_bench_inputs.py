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


def test_traffic_reported_only_for_the_measured_sources(tmp_path, monkeypatch):
    """roofline.traffic and slicing_roofline.traffic are rocprofv3 figures measured outside the
    run; bench.py gives each only while its sources hash to the ones it was measured on (a
    change to either file, or a missing file, gives None)."""
    (tmp_path / "k.hip").write_bytes(b"kernel v1")
    (tmp_path / "h.h").write_bytes(b"helpers v1")
    monkeypatch.setattr(bench, "CSRC", str(tmp_path))
    digest = bench.sources_digest(("k.hip", "h.h"))
    monkeypatch.setattr(bench, "TRAFFIC", {"contract": (123, ("k.hip", "h.h"), digest)})
    assert bench.measured_traffic("contract") == 123
    (tmp_path / "h.h").write_bytes(b"helpers v2")
    assert bench.measured_traffic("contract") is None
    (tmp_path / "h.h").write_bytes(b"helpers v1")
    (tmp_path / "k.hip").write_bytes(b"kernel v2")
    assert bench.measured_traffic("contract") is None
    (tmp_path / "k.hip").unlink()
    assert bench.measured_traffic("contract") is None
    # the names are part of the digest: the same bytes under other names do not match
    (tmp_path / "k2.hip").write_bytes(b"kernel v1")
    assert bench.sources_digest(("k2.hip", "h.h")) != digest

