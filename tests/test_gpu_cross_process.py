"""Cross-process determinism, as the reference's run_repro.sh checks it (run_repro.sh:87-112):
three separate processes each hash every (shape, distribution, S) of the reference's list, every
algorithm x split_k x run inside a process must agree (tests/cross_process_worker.py), the three
processes must print identical RESULT lines, and those hashes must equal the CPU oracle's for the
shapes with M*N*K <= 2^28 (the reference's own limit for the CPU check, hash_repro_gemm.cu:161).
"""
import os
import re
import subprocess
import sys

import numpy as np
import pytest

from gpu_util import note
from oracle import oracle as O

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
PROCESSES = 3


def _run_worker(i):
    note("cross-process worker", i)
    r = subprocess.run([sys.executable, os.path.join(HERE, "cross_process_worker.py")],
                       capture_output=True, text=True, timeout=150)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
    lines = [l for l in r.stdout.splitlines() if l.startswith("RESULT")]
    assert lines, r.stdout[-2000:]
    return lines


@pytest.mark.timeout(500)
def test_three_processes_print_identical_hashes(torch_gpu):
    runs = [_run_worker(i) for i in range(PROCESSES)]
    assert all(r == runs[0] for r in runs[1:]), "processes disagree"
    assert len(runs[0]) == 4 * len(O.HASH_DISTS) * 2
    checked = 0
    for line in runs[0]:
        m = re.match(r"RESULT M=(\d+) N=(\d+) K=(\d+) S=(\d+) dist=(\w+) hash=([0-9a-f]{16})$", line)
        assert m, line
        M, N, K, S = (int(m.group(i)) for i in range(1, 5))
        if M * N * K > 1 << 28:
            continue
        A, B = O.gen_hash_inputs(M, N, K, 12345, m.group(5))
        want = O.cpu_gemm(A, B, M, N, K, 0, 0, S)
        assert "%016x" % O.fnv1a64(want) == m.group(6), line
        checked += 1
    assert checked == 3 * len(O.HASH_DISTS) * 2
