"""The hash tool (bit_reproducible_training_amd.hash_repro_gemm, hash_repro_gemm.cu restated): its
input generator against the oracle's independent C restatement of the reference's tool for
every distribution (hash_repro_gemm.cu:20-56), FNV-1a-64 against published test vectors, the
file: input, argument errors; and on the GPU, the tool end to end with its RESULT line."""
import os
import subprocess
import sys

import numpy as np
import pytest

from bit_reproducible_training_amd import hash_repro_gemm as H
from oracle import oracle as O

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("dist", H.DISTS)
@pytest.mark.parametrize("M,N,K,seed", [(16, 12, 40, 12345), (33, 7, 9, 7), (8, 18, 64, 2 ** 64 - 5)])
def test_inputs_match_oracle_generator(dist, M, N, K, seed):
    A, B = H.fill(dist, seed, M, N, K)
    Ao, Bo = O.gen_hash_inputs(M, N, K, seed, dist)
    assert np.array_equal(A.view(np.uint32), Ao.reshape(-1).view(np.uint32)), dist
    assert np.array_equal(B.view(np.uint32), Bo.reshape(-1).view(np.uint32)), dist


def test_normal_inputs_match_the_reference_bench_recipe():
    """dist=normal is the reference bench's input (one stream, A then B): the same bits as the
    oracle's Irwin-Hall generator at offsets 0 and M*K."""
    M, N, K = 9, 5, 13
    A, B = H.fill("normal", 12345, M, N, K)
    assert np.array_equal(A, O.gen_normal(M * K, 1.0, 12345, 0))
    assert np.array_equal(B, O.gen_normal(K * N, 1.0, 12345, M * K))


def test_fnv1a64_published_vectors():
    import torch

    from bit_reproducible_training_amd.repro_gemm import _backend

    # FNV-1a 64-bit test vectors (Fowler/Noll/Vo): "", "a", "foobar"
    for text, want in ((b"", 0xcbf29ce484222325), (b"a", 0xaf63dc4c8601ec8c),
                       (b"foobar", 0x85944171f73967e8)):
        t = torch.frombuffer(bytearray(text), dtype=torch.uint8) if text else torch.empty(0, dtype=torch.uint8)
        assert _backend.fnv1a64(t) == want
    x = torch.from_numpy(np.arange(100, dtype=np.float32))
    assert _backend.fnv1a64(x) == O.fnv1a64(x.numpy())
    h = _backend.fnv1a64(x[:50].contiguous())
    assert _backend.fnv1a64(x[50:].contiguous(), h) == O.fnv1a64(x.numpy())


def test_file_inputs_and_errors(tmp_path):
    M, N, K = 3, 4, 5
    A = np.arange(M * K, dtype=np.float32)
    B = -np.arange(K * N, dtype=np.float32)
    pa, pb = tmp_path / "a.bin", tmp_path / "b.bin"
    A.astype("<f4").tofile(pa)
    B.astype("<f4").tofile(pb)
    a, b = H.fill("file:%s,%s" % (pa, pb), 0, M, N, K)
    assert np.array_equal(a, A) and np.array_equal(b, B)
    with pytest.raises(ValueError):
        H.fill("file:%s,%s" % (pa, pb), 0, M, N, K + 1)   # wrong size
    with pytest.raises(ValueError):
        H.fill("file:%s" % pa, 0, M, N, K)                # needs two files
    with pytest.raises(ValueError):
        H.fill("gauss", 0, M, N, K)
    assert H.main(["4", "4", "4", "1", "1", "1", "gauss"]) == 1
    bad = tmp_path / "nan.bin"
    np.full(M * K, np.nan, np.float32).tofile(bad)
    assert H.main([str(M), str(N), str(K), "1", "1", "0", "file:%s,%s" % (bad, pb)]) == 1


@pytest.mark.gpu
def test_tool_end_to_end_on_gpu(torch_gpu, tmp_path):
    """The tool as a program: every distribution at S = 1 and 3 passes, its RESULT line carries
    the oracle's hash of the definition's output, and file: inputs give the same line as the
    generated ones they were written from."""
    for dist in H.DISTS:
        for S in (1, 3):
            M, N, K = 67, 45, 301
            r = subprocess.run([sys.executable, "-m", "bit_reproducible_training_amd.hash_repro_gemm",
                                str(M), str(N), str(K), "2", "1,3,7", "99", dist, "ref,tiled,tc,auto", str(S)],
                               cwd=REPO, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                               timeout=300)
            assert r.returncode == 0, r.stdout[-3000:]
            A, B = O.gen_hash_inputs(M, N, K, 99, dist)
            want = O.fnv1a64(O.cpu_gemm(A.reshape(-1), B.reshape(-1), M, N, K, 0, 0, S))
            line = [l for l in r.stdout.splitlines() if l.startswith("RESULT")]
            assert line == ["RESULT M=%d N=%d K=%d S=%d seed=99 dist=%s hash=%016x status=PASS" % (
                M, N, K, S, dist, want)], r.stdout[-3000:]
            assert "exact vs CPU definition: MATCH" in r.stdout
    A, B = O.gen_hash_inputs(64, 64, 64, 5, "wide")
    pa, pb = tmp_path / "a.bin", tmp_path / "b.bin"
    A.astype("<f4").tofile(pa)
    B.astype("<f4").tofile(pb)
    r = subprocess.run([sys.executable, "-m", "bit_reproducible_training_amd.hash_repro_gemm", "64", "64",
                        "64", "1", "1,2", "5", "file:%s,%s" % (pa, pb)], cwd=REPO, stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-3000:]
    want = O.fnv1a64(O.cpu_gemm(A.reshape(-1), B.reshape(-1), 64, 64, 64, 0, 0, 3))
    assert "hash=%016x status=PASS" % want in r.stdout


def test_committed_suite_result_file_carries_the_recorded_hashes():
    """profiles/suite_gemm_1024tok_result_file.txt (bench.py --suite --suite-out, on MI355X) is in
    the reference suite's result-file format; each of its 21 GEMM lines must carry the input and
    output hashes the reference recorded for that operation (gpt2_ops_suite/results/mac/cpu.txt)."""
    import json

    with open(os.path.join(REPO, "tests", "golden", "suite_gemm_s3.json")) as f:
        want = {op["name"]: op for op in json.load(f)["gemm"]}
    with open(os.path.join(REPO, "profiles", "suite_gemm_1024tok_result_file.txt")) as f:
        lines = f.read().splitlines()
    assert lines[0].startswith("# ") and "tokens=1024 S=3" in lines[0]
    seen = set()
    for line in lines[1:]:
        tag, name, shape, hin, hout = line.split("\t")[:5]
        assert tag == "OP" and shape == want[name]["shape"]
        assert hin == "in=" + want[name]["in_hash"] and hout == "out=" + want[name]["out_hash"], name
        seen.add(name)
    assert seen == set(want)
