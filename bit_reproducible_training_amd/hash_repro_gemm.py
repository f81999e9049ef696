"""Hash tool: the output bits of the reproducible GEMM across repeated runs, split-K values and
algorithms, compared with each other and with the CPU implementation of the definition.

    python -m bit_reproducible_training_amd.hash_repro_gemm [M] [N] [K] [runs] [splits] [seed]
                                                            [dist] [algos] [slices]

The arguments, their defaults, the input distributions and the printed lines are those of the
reference's tool (repro_gemm_cuda/hash_repro_gemm.cu:8-16, 57-77, 79-89, 115-204), so the
`RESULT` line it ends with can be diffed against the reference's CUDA runs
(repro_gemm_cuda/run_repro.sh:125-132) and across processes and hosts:

    RESULT M=.. N=.. K=.. S=.. seed=.. dist=.. hash=<FNV-1a-64 of C's bits> status=PASS|FAIL

  splits  comma-separated split_k values (default 1,2,3,4,7,8,16,64)
  algos   comma-separated from ref, tiled, tc, auto (default ref,tiled,tc)
  dist    uniform  U[-1, 1)
          normal   N(0, 1) (Irwin-Hall)
          weights  N(0, 0.02), 0.1% outliers x100
          wide     random sign * 2^U[-40, 40] * [1, 2)
          stress   normal plus zero rows and columns, subnormal, 1e30 and mixed-scale rows and
                   columns, an outlier per fourth row, signed zeros
          file:A.bin,B.bin   raw little-endian float32, row-major A[M,K] and B[K,N]

Every run writes a C poisoned with NaN bytes first. For M*N*K <= 2^28 every output bit is also
compared with the CPU implementation of the definition (include/repro_gemm_cpu.h, through the
package's CPU path), and the error against an FP64 product is reported. Exit status 0 (PASS),
1 (bad arguments or inputs), 2 (FAIL).

The inputs are drawn from the reference's portable generator (repro_test_util.h:26-48:
SplitMix64, exact integer-to-double conversions, Irwin-Hall normals, ldexp), restated here with
numpy: SplitMix64 is a counter generator (draw i of seed s is mix(s + (i + 1) * gamma)), so every
element's draws are computed from their position in the stream.
"""
import ctypes
import sys

import numpy as np

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
DISTS = ("uniform", "normal", "weights", "wide", "stress")
DEFAULT_SPLITS = "1,2,3,4,7,8,16,64"
DEFAULT_ALGOS = "ref,tiled,tc"


def _mix(seed, idx):
    """SplitMix64 draw idx (0-based) of the stream seeded `seed` (repro_test_util.h:31-36)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (np.asarray(idx, dtype=np.uint64) + np.uint64(1)) * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


class Stream:
    """The reference's Rng as a position in one SplitMix64 stream; each method draws the values
    of n elements, element after element, exactly as n calls of the reference's method would."""

    def __init__(self, seed):
        self.seed = int(seed) & (2 ** 64 - 1)
        self.pos = 0

    def _take(self, count):
        idx = np.arange(self.pos, self.pos + count, dtype=np.uint64)
        self.pos += count
        return _mix(self.seed, idx)

    @staticmethod
    def _u01(draws):
        return (draws >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)

    def uniform_pm1(self, n):
        return (2.0 * self._u01(self._take(n)) - 1.0).astype(np.float32)

    def _normal_from(self, u):
        t = np.zeros(u.shape[0])
        for j in range(12):  # summed in the reference's order (exact in double)
            t += u[:, j]
        return t - 6.0

    def normal(self, n):
        """n Irwin-Hall N(0,1) values as doubles (12 draws each)."""
        return self._normal_from(self._u01(self._take(12 * n)).reshape(n, 12))

    def weights(self, n):
        d = self._take(13 * n).reshape(n, 13)
        v = 0.02 * self._normal_from(self._u01(d[:, :12]))
        return np.where(d[:, 12] % np.uint64(1000) == 0, v * 100.0, v).astype(np.float32)

    def range(self, lo, hi, n):
        return lo + (self._take(n) % np.uint64(hi - lo + 1)).astype(np.int64)

    def wide(self, elo, ehi, n):
        d = self._take(3 * n).reshape(n, 3)
        mant = 1.0 + self._u01(d[:, 0])
        e = elo + (d[:, 1] % np.uint64(ehi - elo + 1)).astype(np.int64)
        v = np.ldexp(mant, e)
        return np.where((d[:, 2] & np.uint64(1)) == 1, -v, v).astype(np.float32)


def _load(path, count):
    with open(path, "rb") as f:
        data = f.read()
    if len(data) != 4 * count:
        raise ValueError("%s: expected exactly %d float32 values" % (path, count))
    return np.frombuffer(data, dtype="<f4").astype(np.float32)


def fill(dist, seed, M, N, K):
    """A [M*K] and B [K*N] float32 as the reference's tool fills them
    (hash_repro_gemm.cu:20-77)."""
    if dist.startswith("file:"):
        spec = dist[5:]
        if "," not in spec:
            raise ValueError("file: needs A.bin,B.bin")
        pa, pb = spec.split(",", 1)
        return _load(pa, M * K), _load(pb, K * N)
    g = Stream(seed)
    nA, nB = M * K, K * N
    if dist == "uniform":
        return g.uniform_pm1(nA), g.uniform_pm1(nB)
    if dist == "normal":
        return g.normal(nA).astype(np.float32), g.normal(nB).astype(np.float32)
    if dist == "weights":
        return g.weights(nA), g.weights(nB)
    if dist == "wide":
        return g.wide(-40, 40, nA), g.wide(-40, 40, nB)
    if dist != "stress":
        raise ValueError("unknown dist '%s'" % dist)
    A = g.normal(nA).astype(np.float32).reshape(M, K)
    B = g.normal(nB).astype(np.float32).reshape(K, N)
    for r in range(M):
        case = r % 8
        if case == 1:
            A[r] = 0.0
        elif case == 2:
            A[r] = np.ldexp(g.normal(K), -140).astype(np.float32)
        elif case == 3:
            A[r] = (1e30 * g.normal(K)).astype(np.float32)
        elif case == 4:
            A[r, int(g.range(0, K - 1, 1)[0])] = np.float32(1e6)
        elif case == 5:
            A[r] = np.where(np.arange(K) & 1, np.float32(-0.0), np.float32(0.0))
    for c in range(N):
        case = c % 6
        if case == 1:
            B[:, c] = 0.0
        elif case == 2:
            B[:, c] = g.wide(-60, 60, K)
        elif case == 3:
            B[:, c] = np.ldexp(g.normal(K), -120).astype(np.float32)
    return A.reshape(-1), B.reshape(-1)


def _algo(name, rg):
    table = {"ref": rg.Algo.Reference, "tiled": rg.Algo.Tiled, "tc": rg.Algo.TensorCore,
             "auto": rg.Algo.Auto}
    if name not in table:
        raise ValueError("unknown algo '%s' (use ref, tiled, tc, auto)" % name)
    return table[name]


def _fp64_error(A, B, C, M, N, K):
    """Relative Frobenius error of C against the FP64 product, and the worst row's (finite
    differences only, as the reference reports them)."""
    a = A.reshape(M, K).astype(np.float64)
    b = B.reshape(K, N).astype(np.float64)
    exact = a @ b
    d = C.reshape(M, N).astype(np.float64) - exact
    fin = np.isfinite(d)
    d = np.where(fin, d, 0.0)
    ref = np.where(fin, exact, 0.0)
    row_err, row_ref = (d * d).sum(1), (ref * ref).sum(1)
    tot = row_ref.sum()
    worst = np.sqrt(row_err[row_ref > 0] / row_ref[row_ref > 0]).max() if (row_ref > 0).any() else 0.0
    return (np.sqrt(row_err.sum() / tot) if tot > 0 else 0.0), worst


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    try:
        M = int(argv[0]) if len(argv) > 0 else 256
        N = int(argv[1]) if len(argv) > 1 else 256
        K = int(argv[2]) if len(argv) > 2 else 1024
        runs = int(argv[3]) if len(argv) > 3 else 5
        splits = [int(t) for t in (argv[4] if len(argv) > 4 else DEFAULT_SPLITS).split(",") if t]
        seed = int(argv[5]) if len(argv) > 5 else 12345
        dist = argv[6] if len(argv) > 6 else "normal"
        algos = [t for t in (argv[7] if len(argv) > 7 else DEFAULT_ALGOS).split(",") if t]
        S = int(argv[8]) if len(argv) > 8 else 3
        A, B = fill(dist, seed, M, N, K)
    except (ValueError, OSError) as e:
        print(e, file=sys.stderr)
        return 1
    if not np.isfinite(A).all():
        print("A contains NaN/Inf (unsupported)", file=sys.stderr)
        return 1
    if not np.isfinite(B).all():
        print("B contains NaN/Inf (unsupported)", file=sys.stderr)
        return 1

    import torch

    import bit_reproducible_training_amd as rg
    from bit_reproducible_training_amd import _lib
    from bit_reproducible_training_amd.repro_gemm import _backend

    try:
        algo_list = [(a, _algo(a, rg)) for a in algos]
    except ValueError as e:
        print(e, file=sys.stderr)
        return 1
    if not torch.cuda.is_available():
        print("no GPU: the tool hashes the GPU path", file=sys.stderr)
        return 1
    prop = torch.cuda.get_device_properties(0)
    print("device: %s (%s)  runtime %s" % (prop.name, getattr(prop, "gcnArchName", "?"),
                                          torch.version.hip))
    print("M=%d N=%d K=%d S=%d runs=%d seed=%d dist=%s" % (M, N, K, S, runs, seed, dist))
    tA, tB = torch.from_numpy(A), torch.from_numpy(B)
    print("input hash A=%016x B=%016x" % (_backend.fnv1a64(tA), _backend.fnv1a64(tB)))
    dA, dB = tA.cuda(), tB.cuda()
    C = torch.empty(M * N, dtype=torch.float32, device="cuda")
    ref_bits, ref_hash, all_match = None, None, True
    for name, algo in algo_list:
        for split in splits:
            cfg = rg.Config(slices=S, split_k=split, algo=algo)
            try:
                plan = rg.make_plan(M, N, K, cfg)
            except rg.ReproGemmError as e:
                if e.code == _lib.HIP_ERROR_NOT_SUPPORTED:
                    print("%-5s skipped: not supported on this GPU" % name)
                    break
                print("plan: %s" % e, file=sys.stderr)
                return 1
            line = "%-5s split_k=%-4d" % (name, split)
            if plan.split_k != split:
                line += "(ran %-3d)" % plan.split_k
            for _ in range(runs):
                C.view(torch.int32).fill_(-1)  # NaN bytes: an unwritten output cannot pass
                code = _lib.lib.rg_gemm_fp32(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K,
                                             ctypes.byref(cfg.to_c()),
                                             torch.cuda.current_stream().cuda_stream)
                if code != 0:
                    print("GEMM: %s" % _lib.error_string(code), file=sys.stderr)
                    return 1
                out = C.cpu()
                h = _backend.fnv1a64(out)
                line += " %016x" % h
                if ref_bits is None:
                    ref_bits, ref_hash = out.numpy().view(np.uint32).copy(), h
                    continue
                if h != ref_hash:
                    all_match = False
                    got = out.numpy().view(np.uint32)
                    diff = np.flatnonzero(got != ref_bits)
                    i = int(diff[0])
                    line += " [MISMATCH: %d elems differ, first idx=%d (r=%d,c=%d) %.9g vs ref %.9g]" % (
                        diff.size, i, i // N, i % N, got.view(np.float32)[i], ref_bits.view(np.float32)[i])
            print(line, flush=True)
    if ref_bits is None:
        print("no algorithm ran", file=sys.stderr)
        return 1
    Cref = ref_bits.view(np.float32)
    nonfinite = int((~np.isfinite(Cref)).sum())
    if nonfinite:
        print("note: %d output elements are non-finite (FP32 overflow of the true result)" % nonfinite)
    exact_ok = True
    if float(M) * N * K <= float(1 << 28):
        cpu = rg.gemm(tA, tB, M, N, K, False, False, S).numpy().reshape(-1).view(np.uint32)
        diff = np.flatnonzero(cpu != ref_bits)
        exact_ok = diff.size == 0
        if exact_ok:
            print("exact vs CPU definition: MATCH (all %d elements)" % (M * N))
        else:
            i = int(diff[0])
            print("exact vs CPU definition: MISMATCH %d elements, first (r=%d,c=%d) gpu %s cpu %s" % (
                diff.size, i // N, i % N, float(Cref[i]).hex(), float(cpu.view(np.float32)[i]).hex()))
        rel, worst = _fp64_error(A, B, Cref, M, N, K)
        print("accuracy vs FP64: relative Frobenius error %.3e, worst row %.3e" % (rel, worst))
    else:
        print("exact vs CPU definition: skipped (M*N*K > 2^28)")
        print("accuracy vs FP64: skipped (M*N*K > 2^28)")
    print("output hash: %016x" % ref_hash)
    ok = all_match and exact_ok
    print("RESULT M=%d N=%d K=%d S=%d seed=%d dist=%s hash=%016x status=%s" % (
        M, N, K, S, seed, dist, ref_hash, "PASS" if ok else "FAIL"), flush=True)
    if not all_match:
        print("FAIL: outputs are not bit-identical across runs/splits/algos")
        return 2
    if not exact_ok:
        print("FAIL: output differs from the exact CPU definition")
        return 2
    print("PASS: all runs, split_k values, and algos bit-identical")
    return 0


if __name__ == "__main__":
    sys.exit(main())
