"""Benchmark of the reproducible FP32 GEMM on one MI355X.

Headline workload: C = A B, M = N = K = 4096, S = 3 slices, no transposes, A then B drawn
N(0,1) from one SplitMix64/Irwin-Hall stream seeded 12345 -- the recipe of the reference's
own benchmark (repro_gemm_cuda/bench_repro_gemm.cu:28-49), at the 4096^3 size of BASELINE
configuration 4. Configuration 4's adversarial inputs (random signs, |x| = 2^e with
e ~ U[-60, 60], 5% zeros, 1% subnormals, near-negative pairs along k) are timed as well and
reported beside it: their digits are mostly zero, which lets the GPU clock higher, so the
dense inputs give the lower (headline) number.

A "step" is one full reproducible GEMM: slice split of both operands, int8 MFMA
contraction, exact recombination and rounding, with inputs resident in HBM.

Prints one JSON line: effective FP32 TFLOP/s = 2 M N K / time (the reference's definition,
repro_gemm_cuda/bench_repro_gemm.cu:72-75), the contraction kernel's int8 rate against the
MI355X dense int8 MFMA peak (measured with HIP events on the launch stream), whether the
output bits equal the reference CPU path's and the committed fixture, and the reference
CPU path timed on this host on the same inputs.

  python bench.py [--steps K] [--warmup W] [--no-cpu] [--size N] [--calibrate]
"""
import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 MFMA, TOP/s
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E, GB/s
# The steady-state side measurement of the headline GEMM: GEMMs run first, then GEMMs timed.
STEADY_WARM = 200
STEADY_STEPS = 50
# HBM bytes per GEMM at 4096^3 S=3 (fetch + write) of the contraction launch and of the
# slicing launches (the slot marking and the one-read slicing), from rocprofv3 FETCH_SIZE /
# WRITE_SIZE scaled by the same counters on a
# 256 MiB device copy (profiles/contract_mfma_4096cube_traffic.md), each measured on the sources
# whose SHA-256 (sources_digest) is given: the kernel file and rg_internal.h, which holds the
# block order and the rounding helpers. A counter value cannot be read from inside this process,
# so a figure is reported only while its sources are unchanged; otherwise it is null.
CSRC = os.path.join(REPO, "bit_reproducible_training_amd", "csrc")
TRAFFIC = {
    "contract": (671606784, ("rg_contract.hip", "rg_internal.h"),
                 "aad6c405111935b53b5551a3876ec8e399399485b748e7b6e9606e5651ad0bf0"),
    "slicing": (235601510, ("rg_slice.hip", "rg_internal.h"),
                "a762ab26f759129cac13e138d0c181325da016b9360adccd2312f5678f9aaeb8"),
}
FIXTURE = os.path.join(REPO, "tests", "golden", "baseline_configs.json")

# --------------------------------------------------------------------------------------
# Synthetic input (same recipe and bits as tests/golden/configs.py config 4), vectorised
# SplitMix64 in numpy: draw i of seed s is mix(s + (i + 1) * gamma).
# --------------------------------------------------------------------------------------
_G = np.uint64(0x9E3779B97F4A7C15)


def sources_digest(names):
    """SHA-256 over the named files of csrc/, each as its name, a NUL byte and its bytes."""
    import hashlib

    h = hashlib.sha256()
    for name in names:
        with open(os.path.join(CSRC, name), "rb") as f:
            h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()


def measured_traffic(stage="contract"):
    """The measured HBM bytes per GEMM of a stage ("contract" or "slicing") if its sources are
    the ones it was measured on, else None."""
    nbytes, names, digest = TRAFFIC[stage]
    try:
        return nbytes if sources_digest(names) == digest else None
    except OSError:
        return None


def _draw(seed, idx):
    z = np.uint64(seed) + (idx + np.uint64(1)) * _G
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _adversarial(rows, cols, seed, pair_rows, negate):
    r = np.arange(rows, dtype=np.uint64)[:, None]
    c = np.arange(cols, dtype=np.uint64)[None, :]
    one = np.uint64(1)
    if pair_rows:
        base = (r & ~one) * np.uint64(cols) + c
        second = np.broadcast_to((r & one) == one, (rows, cols))
    else:
        base = r * np.uint64(cols) + (c & ~one)
        second = np.broadcast_to((c & one) == one, (rows, cols))
    u = _draw(seed, np.uint64(2) * base)
    v = _draw(seed, np.uint64(2) * base + one)
    pct = u % np.uint64(100)
    sign = ((v >> np.uint64(63)) & one).astype(np.uint32) << np.uint32(31)
    f = ((v >> np.uint64(8)) & np.uint64(0x7FFFFF)).astype(np.uint32)
    f = np.where(f == 0, np.uint32(1), f)
    e = ((v >> np.uint64(16)) % np.uint64(121)).astype(np.int64) - 60
    normal = ((e + 127).astype(np.uint32)) << np.uint32(23)
    b = np.where(pct < 5, np.uint32(0), np.where(pct < 6, f, normal)) | sign
    x = b.astype(np.uint32).view(np.float32)
    w = _draw(np.uint64(seed) ^ np.uint64(0x5BD1E995), base)
    t = (w % np.uint64(3)).astype(np.int64) - 1
    fac = (np.float32(1.0) + t.astype(np.float32) * np.float32(1.0 / 1048576.0)).astype(np.float32)
    y = (x * fac).astype(np.float32)
    if negate:
        y = -y
    return np.where(second, y, x).astype(np.float32)


def make_adversarial(n):
    A = _adversarial(n, n, 4001, pair_rows=False, negate=True)
    B = _adversarial(n, n, 4002, pair_rows=True, negate=False)
    return np.ascontiguousarray(A), np.ascontiguousarray(B)


def _normal_chunk(out, a, b, seed, first, scale=1.0):
    """Elements [a, b): Irwin-Hall sum of 12 draws (element i uses draws 12 i .. 12 i + 11),
    summed in the same order as the reference's Rng::normal (repro_test_util.h:41)."""
    j = np.arange(12, dtype=np.uint64)
    idx = np.arange(a + first, b + first, dtype=np.uint64)[:, None] * np.uint64(12) + j[None, :]
    u = (_draw(seed, idx) >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)
    t = np.zeros(b - a)
    for k in range(12):
        t += u[:, k]
    out[a:b] = (scale * (t - 6.0)).astype(np.float32)


def normal_stream(n, seed, first=0, chunk=1 << 20, scale=1.0):
    from concurrent.futures import ThreadPoolExecutor

    out = np.empty(n, np.float32)
    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        list(ex.map(lambda a: _normal_chunk(out, a, min(n, a + chunk), seed, first, scale),
                    range(0, n, chunk)))
    return out


def make_normal(n):
    """A then B from one N(0,1) stream seeded 12345 (bench_repro_gemm.cu:47-49)."""
    A = normal_stream(n * n, 12345, 0).reshape(n, n)
    B = normal_stream(n * n, 12345, n * n).reshape(n, n)
    return A, B


def host_cpus():
    """What the host offers the CPU baseline: nproc (os.cpu_count()), the CPUs this process may
    run on (sched_getaffinity), the cgroup CPU quota if one is set, and the CPU model."""
    info = {"nproc": os.cpu_count()}
    try:
        info["affinity"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        info["affinity"] = os.cpu_count()
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            info["cgroup_quota_cpus"] = round(int(quota) / int(period), 2)
    except (OSError, ValueError):
        pass
    try:
        info["model"] = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo")
                             if l.startswith("model name"))
    except (OSError, StopIteration):
        info["model"] = "unknown"
    return info


def default_cpu_threads(info):
    """REPRO_CPU_THREADS if set (the reference's override, repro_gemm_cpu.h:14-23), else every
    CPU the process may run on (hardware_concurrency() as the reference uses it, bounded by the
    affinity mask)."""
    env = os.environ.get("REPRO_CPU_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return max(1, int(info.get("affinity") or info.get("nproc") or 1))


# --------------------------------------------------------------------------------------
# CPU baseline and bit-exactness check: this repository's C port of the reference's CPU path
# (oracle/repro_oracle.c: the same three passes and thread pool, pinned bit for bit to the
# reference's own CPU path in this container), or the reference's path itself where
# oracle/_ref was built (never on the GPU box). Used here as the timed baseline and as the
# checker only.
# --------------------------------------------------------------------------------------
def cpu_baseline(A, B, n, gpu_C, threads, reps, fixtures, gpu_adv=None):
    from oracle import oracle as O

    info = host_cpus()
    kind = "reference" if O.ref is not None else "port"
    os.environ["REPRO_CPU_THREADS"] = str(threads)
    times = []
    C = None
    for _ in range(reps):
        t0 = time.perf_counter()
        if kind == "reference":
            C = O.ref_cpu_gemm(A, B, n, n, n, 0, 0, 3)
        else:
            C = O.cpu_gemm(A, B, n, n, n, 0, 0, 3, threads)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    match = bool(np.array_equal(C.view(np.uint32), gpu_C.view(np.uint32)))
    out_hash = "%016x" % O.fnv1a64(C)
    checks = {"gpu_bits_equal_cpu": match}
    if "bench.4096cube.normal" in fixtures and n == 4096:
        checks["cpu_hash_equals_fixture"] = out_hash == fixtures["bench.4096cube.normal"]
    if gpu_adv is not None and "c4.adversarial4096" in fixtures and n == 4096:
        checks["adversarial_gpu_hash_equals_fixture"] = (
            "%016x" % O.fnv1a64(gpu_adv)) == fixtures["c4.adversarial4096"]
    base = {
        "value": round(2.0 * n * n * n / t / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": kind,
        "sample": "the full %d^3 S=3 GEMM on the headline inputs, wall clock incl. quantisation, "
                  "median of %d runs, %d threads" % (n, reps, threads),
        "ms": round(t * 1e3, 2),
        "host": info,
    }
    return base, checks, out_hash


def time_workload(torch, rg, A, B, n, steps, warmup, calibrate=False, steady=False):
    M = N = K = n
    dA = torch.from_numpy(A).cuda()
    dB = torch.from_numpy(B).cuda()
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")
    cfg = rg.Config(slices=3)
    plan = rg.make_plan(M, N, K, cfg)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    sp = torch.cuda.current_stream().cuda_stream

    def step(events=None):
        code = rg.repro_gemm_fp32_ws(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K, cfg,
                                     ws.data_ptr(), ws.numel(), sp, events)
        if code != 0:
            raise rg.ReproGemmError(code, "bench step")

    for _ in range(warmup):
        step()
    # Timed region: exactly `steps` GEMMs as a caller runs them (no instrumentation).
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # Stage breakdown from a second pass of `steps` GEMMs with the stage events on the launch
    # stream: event 1 -> event 2 brackets only the contraction kernel's launch.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for e in (x for row in evs for x in row):
        e.record()  # torch creates the HIP event on first record
    torch.cuda.synchronize()
    for i in range(steps):
        step([e.cuda_event for e in evs[i]])
    torch.cuda.synchronize()
    steady_ms = None
    if steady:
        # The same GEMM once the GPU's clock has settled: STEADY_WARM more back-to-back GEMMs
        # (past the power-management transient that the timed loop above, started from an idle
        # GPU, runs inside), then STEADY_STEPS timed like the loop above. Reported beside the
        # headline, never as it.
        for _ in range(STEADY_WARM):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(STEADY_STEPS):
            step()
        torch.cuda.synchronize()
        steady_ms = (time.perf_counter() - t0) * 1e3 / STEADY_STEPS
    if calibrate:
        calibration_copies(torch)
    out = {
        "ms_per_step": wall * 1e3 / steps,
        "slice_ms": statistics.mean(e[0].elapsed_time(e[1]) for e in evs),
        "contract_ms": statistics.mean(e[1].elapsed_time(e[2]) for e in evs),
        "final_ms": statistics.mean(e[2].elapsed_time(e[3]) for e in evs),
        "plan": "%s %dx%d split %d" % (rg.algo_name(plan.algo), plan.tile_m, plan.tile_n, plan.split_k),
        "steady_ms": steady_ms,
        "C": C.cpu().numpy(),
    }
    del dA, dB, C, ws
    torch.cuda.empty_cache()
    return out


def suite(torch, rg, reps=10, warmup=2, out_path=None):
    """The 21 GEMMs of the reference's GPT-2 operation suite at 1024 tokens, S=3, with its
    input recipe (gpt2_ops_suite.cu:193-233, 463-483) and its timing method (median of `reps`
    event-timed calls after `warmup`, gpt2_ops_suite.cu:622-640), next to the times it recorded
    on three NVIDIA GPUs and an FP32 torch.matmul baseline on this GPU (not reproducible).
    Output bits of these ops are checked against the recorded hashes by
    tests/test_gpu_parity.py::test_reference_suite_hashes_gpu."""
    with open(os.path.join(REPO, "tests", "golden", "suite_gemm_s3.json")) as f:
        ops = json.load(f)["gemm"]
    torch.backends.cuda.matmul.allow_tf32 = False
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    rows = []
    # The reference suite's result-file format (gpt2_ops_suite.cu:591, 654-655), GEMM lines only,
    # so compare_suite.sh can set these hashes beside the reference's recorded runs.
    out_file = open(out_path, "w") if out_path else None
    if out_file is not None:
        out_file.write("# %s (this library) tokens=1024 S=3\n" % torch.cuda.get_device_name(0))
    for op in ops:
        M, N, K, ta, tb = op["M"], op["N"], op["K"], op["ta"], op["tb"]
        A = torch.from_numpy(normal_stream(M * K, op["seed"], scale=op["sa"])).cuda()
        B = torch.from_numpy(normal_stream(K * N, op["seed"] + 1, scale=op["sb"])).cuda()
        C = torch.empty((M, N), dtype=torch.float32, device="cuda")
        cfg = rg.Config(slices=3, trans_a=ta, trans_b=tb)
        plan = rg.make_plan(M, N, K, cfg)
        ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
        sp = torch.cuda.current_stream().cuda_stream

        def run():
            code = rg.repro_gemm_fp32_ws(A.data_ptr(), B.data_ptr(), C.data_ptr(), M, N, K, cfg,
                                         ws.data_ptr(), ws.numel(), sp)
            if code != 0:
                raise rg.ReproGemmError(code, op["name"])

        opA = A.view(K, M).t() if ta else A.view(M, K)
        opB = B.view(N, K).t() if tb else B.view(K, N)

        def base():
            torch.matmul(opA, opB)

        def timed(fn):
            for _ in range(warmup):
                fn()
            torch.cuda.synchronize()
            t = []
            for _ in range(reps):
                e0.record()
                fn()
                e1.record()
                e1.synchronize()
                t.append(e0.elapsed_time(e1))
            return statistics.median(t)

        ms, base_ms = timed(run), timed(base)
        if out_file is not None:
            from bit_reproducible_training_amd.repro_gemm import _backend

            C.view(torch.int32).fill_(-1)  # poisoned, then one more run, as the reference's suite
            run()
            hin = _backend.fnv1a64(B.cpu(), _backend.fnv1a64(A.cpu()))  # A then B
            hout = _backend.fnv1a64(C.cpu())
            out_file.write("OP\t%s\t%s\tin=%016x\tout=%016x\tms=%.4f\tbase_ms=%.4f\n" % (
                op["name"], op["shape"], hin, hout, ms, base_ms))
            out_file.flush()
        ref = op.get("reference_gpu_ms", {})
        best_ref = min((v["ms"] for v in ref.values()), default=None)
        rows.append({"op": op["name"], "shape": op["shape"], "ms": round(ms, 4),
                     "tflops": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 2),
                     "torch_fp32_ms": round(base_ms, 4),
                     "plan": "%dx%d split %d" % (plan.tile_m, plan.tile_n, plan.split_k),
                     "reference_best_gpu_ms": best_ref,
                     "speedup_vs_reference_best": round(best_ref / ms, 1) if best_ref else None})
        del A, B, C, ws
    if out_file is not None:
        out_file.close()
    total = sum(r["ms"] for r in rows)
    ref_total = sum(r["reference_best_gpu_ms"] for r in rows if r["reference_best_gpu_ms"])
    print(json.dumps({"mode": "suite", "tokens": 1024, "slices": 3, "ops": rows,
                      "total_ms": round(total, 3), "reference_best_gpu_total_ms": round(ref_total, 3)}),
          flush=True)


# --------------------------------------------------------------------------------------
# Beyond the GEMM: the exact sum, the convolution, the batched GEMM and the Linear layer, each
# against its roofline and next to the times the reference recorded for its own benchmarks.
# --------------------------------------------------------------------------------------
# Fastest time the reference recorded per benchmark case (median ms per call, RTX 2080 Ti,
# TITAN V, RTX 4070): repro_sum_cuda/results/*/sum.log (bench_repro_sum.cu:60-67 shapes) and
# repro_conv_cuda/results/*/conv.log (bench_repro_conv.cu, LeNet-5, batch 100, S=3).
REF_SUM_MS = {"vector 16M": 0.157, "conv bias grad 256x64x56x56": 0.373,
              "linear bias grad 8192x4096": 0.313, "row sums 8192x4096": 0.253,
              "LayerNorm-like rows 16384x1024": 0.144, "softmax-like rows 65536x128": 0.102,
              "LeNet conv1 bias 100x6x28x28": 0.019, "LeNet softmax rows 100x10": 0.008}
SUM_SHAPES = [("vector 16M", 1, 1, 1 << 24), ("conv bias grad 256x64x56x56", 256, 64, 3136),
              ("linear bias grad 8192x4096", 8192, 4096, 1), ("row sums 8192x4096", 1, 8192, 4096),
              ("LayerNorm-like rows 16384x1024", 1, 16384, 1024),
              ("softmax-like rows 65536x128", 1, 65536, 128),
              ("LeNet conv1 bias 100x6x28x28", 100, 6, 784), ("LeNet softmax rows 100x10", 1, 100, 10)]
REF_CONV_MS = {("conv1", "fwd"): 0.059, ("conv1", "dW"): 0.454, ("conv1", "dX"): 0.067,
               ("conv2", "fwd"): 0.121, ("conv2", "dW"): 0.337, ("conv2", "dX"): 0.077}


def _gpu_ms(torch, fn, reps=20, warmup=3):
    """GPU time per call: `reps` calls enqueued back to back between two events."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / reps


def _wall_ms(torch, fn, reps=20, warmup=3):
    """Median wall time per call including the launch and a device synchronisation: the
    reference benchmarks' method (bench_repro_conv.cu:45-57)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        t.append((time.perf_counter() - t0) * 1e3)
    return statistics.median(t)


def _cpu_widened(x_sums, convs, threads):
    """CPU baseline leg: the reference's own exact sum and convolution (oracle/_ref, built from
    repro_sum_cuda and repro_conv_cuda) or this repository's port, timed on the host, and the
    GPU results checked against them bit for bit."""
    from oracle import oracle as O

    os.environ["REPRO_CPU_THREADS"] = str(threads)
    kind = "reference" if O.ref is not None else "port"
    res = {"kind": kind, "sums": [], "conv": []}
    for name, A, B, C, x, gpu in x_sums:
        t0 = time.perf_counter()
        want = O.ref_exact_sum(x, A, B, C) if kind == "reference" else O.exact_sum(x, A, B, C)
        res["sums"].append({"case": name, "ms": round((time.perf_counter() - t0) * 1e3, 3),
                            "bits_equal": bool(np.array_equal(want.view(np.uint32), gpu.view(np.uint32)))})
    for name, shape, ins, gpu in convs:
        row = {"case": name}
        for kind_, a, b in ins:
            t0 = time.perf_counter()
            if kind == "reference":
                want = O.ref_conv(kind_, a, b, shape, 3)
            else:
                want = {"fwd": O.conv2d, "dW": O.conv2d_grad_weight, "dX": O.conv2d_grad_input}[kind_](a, b, shape, 3)
            row[kind_ + "_ms"] = round((time.perf_counter() - t0) * 1e3, 3)
            row[kind_ + "_bits_equal"] = bool(np.array_equal(np.asarray(want, np.float32).view(np.uint32).ravel(),
                                                             gpu[kind_].view(np.uint32).ravel()))
        res["conv"].append(row)
    res["cores"] = threads
    return res


def widened(torch, rg, cpu=True, threads=16):
    """One JSON line: exact sum (GB/s against HBM), LeNet convolutions, batched attention-head
    GEMMs and a GPT-2 Linear layer step (effective TFLOP/s), with the reference's recorded
    times where it has them."""
    line = {"mode": "widened", "slices": 3, "data": "synthetic N(0,1) (torch.randn, seed 0)"}
    torch.manual_seed(0)
    stream = lambda: torch.cuda.current_stream().cuda_stream
    # Exact sums: x = [A][B][C], out[b] = sum over a, c (bench_repro_sum.cu's shapes).
    sums, x_sums = [], []
    for name, A, B, C in SUM_SHAPES:
        x = torch.randn(A * B * C, device="cuda")
        out = torch.empty(B, device="cuda")
        cfg = rg.SumConfig()
        plan = rg.make_sum_plan(A, B, C, cfg)
        ws = torch.empty(max(plan.workspace_bytes, 1), dtype=torch.uint8, device="cuda")

        def run():
            code = rg.repro_sum_fp32_ws(x.data_ptr(), out.data_ptr(), A, B, C, cfg, ws.data_ptr(),
                                        ws.numel(), stream())
            if code != 0:
                raise rg.ReproGemmError(code, "exact sum")

        ms = _gpu_ms(torch, run)
        first = out.cpu().numpy().copy()
        run()
        same = bool(np.array_equal(first.view(np.uint32), out.cpu().numpy().view(np.uint32)))
        gbs = 4.0 * A * B * C / (ms * 1e-3) / 1e9
        sums.append({"case": name, "A": A, "B": B, "C": C, "gpu_ms": round(ms, 4),
                     "wall_ms": round(_wall_ms(torch, run), 4), "GB/s": round(gbs, 1),
                     "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "same_bits_every_run": same,
                     "reference_best_gpu_ms": REF_SUM_MS.get(name)})
        if A * B * C <= (1 << 22):
            x_sums.append((name, A, B, C, x.cpu().numpy(), first))
        del x, out, ws
    line["exact_sum"] = sums
    # LeNet-5 convolutions, batch 100 (bench_repro_conv.cu's shapes and input scales).
    RC = rg.repro_conv
    shapes = [("conv1", rg.ConvShape(100, 1, 28, 28, 6, 5, 5, 1, 1, 2, 2)),
              ("conv2", rg.ConvShape(100, 6, 14, 14, 16, 5, 5))]
    convs, conv_cpu = [], []
    for name, g in shapes:
        x = torch.randn(g.N, g.C, g.H, g.W, device="cuda")
        w = 0.1 * torch.randn(g.F, g.C, g.KH, g.KW, device="cuda")
        dy = 1e-3 * torch.randn(g.N, g.F, g.OH, g.OW, device="cuda")
        y = torch.empty_like(dy)
        dw = torch.empty_like(w)
        dx = torch.empty_like(x)
        row = {"case": name, "shape": list(g.astuple())}
        outs = {}
        for kind, fn, ws_fn, a, b, o in (("fwd", rg.repro_conv2d_ws, rg.conv2d_workspace, x, w, y),
                                          ("dW", rg.repro_conv2d_grad_weight_ws, rg.conv2d_grad_weight_workspace, dy, x, dw),
                                          ("dX", rg.repro_conv2d_grad_input_ws, rg.conv2d_grad_input_workspace, dy, w, dx)):
            ws = torch.empty(max(ws_fn(g, 3), 1), dtype=torch.uint8, device="cuda")

            def run():
                code = fn(a.data_ptr(), b.data_ptr(), o.data_ptr(), g, 3, ws.data_ptr(), ws.numel(), stream())
                if code != 0:
                    raise rg.ReproGemmError(code, "conv " + kind)

            row[kind + "_gpu_ms"] = round(_gpu_ms(torch, run), 4)
            row[kind + "_wall_ms"] = round(_wall_ms(torch, run), 4)
            row[kind + "_reference_best_gpu_ms"] = REF_CONV_MS[(name, kind)]
            outs[kind] = o.cpu().numpy().copy()
            pass_ = {"fwd": RC.FORWARD, "dW": RC.GRAD_WEIGHT, "dX": RC.GRAD_INPUT}[kind]
            algo = RC.conv2d_algo(pass_, g)
            row[kind + "_algo"] = "direct" if algo == RC.ALGO_DIRECT else "gemm"
            if algo == RC.ALGO_DIRECT:  # the GEMM pipeline on the same inputs, for comparison
                gws = torch.empty(max(RC.conv2d_algo_workspace(pass_, g, 3, RC.ALGO_GEMM), 1),
                                  dtype=torch.uint8, device="cuda")
                o2 = torch.empty_like(o)

                def run_gemm():
                    code = RC.repro_conv2d_algo_ws(pass_, a.data_ptr(), b.data_ptr(), o2.data_ptr(), g,
                                                   3, RC.ALGO_GEMM, gws.data_ptr(), gws.numel(), stream())
                    if code != 0:
                        raise rg.ReproGemmError(code, "conv gemm " + kind)

                row[kind + "_gemm_gpu_ms"] = round(_gpu_ms(torch, run_gemm), 4)
                row[kind + "_gemm_same_bits"] = bool(torch.equal(o2.view(torch.int32), o.view(torch.int32)))
        convs.append(row)
        conv_cpu.append((name, g.astuple(), [("fwd", x.cpu().numpy(), w.cpu().numpy()),
                                             ("dW", dy.cpu().numpy(), x.cpu().numpy()),
                                             ("dX", dy.cpu().numpy(), w.cpu().numpy())], outs))
    line["conv"] = convs
    # A ResNet-sized layer (batch 32, 64 -> 64 channels, 56 x 56, 3 x 3, padding 1): all three
    # passes take the GEMM pipeline (forward on the implicit im2col matrix). GPU time and the
    # same bits on a repeat; no CPU check at this size.
    g = rg.ConvShape(32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1)
    x = torch.randn(g.N, g.C, g.H, g.W, device="cuda")
    w = 0.1 * torch.randn(g.F, g.C, g.KH, g.KW, device="cuda")
    dy = 1e-3 * torch.randn(g.N, g.F, g.OH, g.OW, device="cuda")
    big = {"case": "resnet-like 32x64x56x56, 64 filters 3x3", "shape": list(g.astuple())}
    for kind, fn, ws_fn, a, b, o in (("fwd", rg.repro_conv2d_ws, rg.conv2d_workspace, x, w, torch.empty_like(dy)),
                                      ("dW", rg.repro_conv2d_grad_weight_ws, rg.conv2d_grad_weight_workspace, dy, x, torch.empty_like(w)),
                                      ("dX", rg.repro_conv2d_grad_input_ws, rg.conv2d_grad_input_workspace, dy, w, torch.empty_like(x))):
        ws = torch.empty(max(ws_fn(g, 3), 1), dtype=torch.uint8, device="cuda")

        def run():
            code = fn(a.data_ptr(), b.data_ptr(), o.data_ptr(), g, 3, ws.data_ptr(), ws.numel(), stream())
            if code != 0:
                raise rg.ReproGemmError(code, "conv " + kind)

        big[kind + "_gpu_ms"] = round(_gpu_ms(torch, run, reps=10), 4)
        first = o.clone()
        run()
        torch.cuda.synchronize()
        big[kind + "_same_bits"] = bool(torch.equal(first.view(torch.int32), o.view(torch.int32)))
        big[kind + "_algo"] = "gemm"
        del ws
    line["conv_large"] = big
    # Attention heads as one strided-batched GEMM vs one GEMM per head (GPT-2 small: 12 heads,
    # 1024 tokens, head size 64): scores = Q_h K_h^T and out = P_h V_h, read in place.
    T, H, D = 1024, 12, 64
    q, k, v = (torch.randn(T, H * D, device="cuda") for _ in range(3))
    p = torch.rand(H, T, T, device="cuda") / T
    heads = lambda z: z.view(T, H, D).permute(1, 0, 2)
    att = {}
    for name, fn_b, fn_l, flops in (
            ("scores QK^T", lambda: rg.bmm(heads(q), heads(k), False, True),
             lambda: [rg.gemm(q[:, h * D:(h + 1) * D].contiguous(), k[:, h * D:(h + 1) * D].contiguous(), T, T, D, False, True) for h in range(H)],
             2.0 * H * T * T * D),
            ("PV", lambda: rg.bmm(p, heads(v), False, False),
             lambda: [rg.gemm(p[h], v[:, h * D:(h + 1) * D].contiguous(), T, D, T, False, False) for h in range(H)],
             2.0 * H * T * T * D)):
        mb, ml = _gpu_ms(torch, fn_b, reps=10), _gpu_ms(torch, fn_l, reps=10)
        att[name] = {"batched_ms": round(mb, 4), "per_head_loop_ms": round(ml, 4),
                     "batched_tflops": round(flops / (mb * 1e-3) / 1e12, 2)}
    line["attention_heads"] = dict(att, heads=H, tokens=T, head_dim=D)
    del q, k, v, p
    # GPT-2 MLP up-projection as a reproducible Linear layer: forward + backward (dX, dW, db).
    tok, fin, fout = 8192, 768, 3072
    layer = rg.Linear(fin, fout).cuda()
    xin = torch.randn(tok, fin, device="cuda", requires_grad=True)
    gy = torch.randn(tok, fout, device="cuda")

    def step():
        y = layer(xin)
        y.backward(gy)

    ms = _gpu_ms(torch, step, reps=10)
    line["linear_step"] = {"layer": "Linear(768, 3072), 8192 tokens, forward + backward", "ms": round(ms, 4),
                           "effective_tflops": round(3 * 2.0 * tok * fin * fout / (ms * 1e-3) / 1e12, 2)}
    if cpu:
        line["cpu_baseline"] = _cpu_widened(x_sums, conv_cpu, threads)
    print(json.dumps(line), flush=True)


# BASELINE configurations 2, 3 and 5 (configuration 1 is 256^3 and 4 the default line's
# adversarial run): shapes, transposes, slices and value scales of tests/golden/configs.py,
# which the GPU tests check against the CPU oracle's hashes. Here: (name, M, N, K, ta, tb, S,
# scale of A, scale of B) with inputs drawn on the GPU (torch.randn, uniform for LeNet weights).
def _config_cases():
    cases = [("c1.256cube", 256, 256, 256, 0, 0, 3, 1.0, 1.0)]
    for li, (fin, fout) in enumerate([(400, 120), (120, 84), (84, 10)]):
        u = 1.0 / (fin ** 0.5)
        for S in (1, 2, 3):
            tag = "c2.fc%d.%dx%d" % (li + 1, fin, fout)
            cases += [(tag + ".fwd.S%d" % S, 64, fout, fin, 0, 1, S, 1.0, -u),
                      (tag + ".dX.S%d" % S, 64, fin, fout, 0, 0, S, 1.0, -u),
                      (tag + ".dW.S%d" % S, fout, fin, 64, 1, 0, S, 1.0, 1.0)]
    for nm, fin, fout in [("qkv", 768, 2304), ("attn_proj", 768, 768), ("mlp_fc", 768, 3072),
                          ("mlp_proj", 3072, 768)]:
        tag = "c3." + nm
        cases += [(tag + ".fwd", 8192, fout, fin, 0, 1, 3, 1.0, 0.02),
                  (tag + ".dX", 8192, fin, fout, 0, 0, 3, 1.0, 0.02),
                  (tag + ".dW", fout, fin, 8192, 1, 0, 3, 1.0, 1.0)]
    cases += [("c5.lm_head.fwd", 8192, 50257, 768, 0, 1, 3, 1.0, 1.0),
              ("c5.lm_head.dW", 50257, 768, 8192, 1, 0, 3, 1.0, 1.0),
              ("c5.tall_skinny", 1024, 1024, 65536, 0, 0, 3, 1.0, 1.0)]
    return cases


def _graph_ms(torch, step, reps=20):
    """GPU time per call of `step`: `reps` calls captured in one HIP graph and replayed, so the
    host's launch cost (a ctypes call and the launches, about 8 us) is not in the figure."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(stream=side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            step(stream=torch.cuda.current_stream().cuda_stream)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    del g
    return e0.elapsed_time(e1) / (5 * reps)


def calibration_copies(torch):
    """Three device-to-device copies of 256 MiB: a plain copy kernel of known size, whose
    rocprofv3 FETCH_SIZE / WRITE_SIZE readings scale those of the library's kernels."""
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def configs_mode(torch, rg, warm_ms=40.0, timed_ms=20.0, only=None, warm_gpu_ms=400.0,
                 calibrate=False):
    """One JSON line: every GEMM of BASELINE configurations 1, 2, 3 and 5 timed on the GPU in
    steady state: back-to-back GEMMs for about `warm_ms` of GPU time (past the GPU's
    power-management transient after a change of load), then HIP events around about `timed_ms`
    of back-to-back GEMMs (at least 10), the GPU brought out of idle first (warm_gpu). Reports
    effective FP32 TFLOP/s, the stage times (median of
    5 runs with stage events: slicing, contraction, final rounding), the contraction's share of the
    dense int8 MFMA peak, the plan, and whether the runs gave identical bits. GEMMs of less than
    0.1 ms also get `graph_ms`, the GPU time per GEMM without the host's launch cost.
    `only`: names of the cases to run (all if None); warm_gpu_ms = 0 skips bringing the GPU out
    of idle (for profiler runs, where the timings are not the point)."""
    if calibrate:
        calibration_copies(torch)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2024)
    sp = torch.cuda.current_stream().cuda_stream
    rows = []
    if warm_gpu_ms > 0:
        warm_gpu(torch, rg, warm_gpu_ms)
    # What two stage events recorded back to back measure with no launch between them: taken off
    # the stage times before the HBM rates below are computed.
    fe = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    floor = []
    for _ in range(20):
        fe[0].record()
        fe[1].record()
        torch.cuda.synchronize()
        floor.append(fe[0].elapsed_time(fe[1]))
    event_floor_ms = statistics.median(floor)
    cases = _config_cases()
    if only:
        unknown = set(only) - {c[0] for c in cases}
        if unknown:
            raise SystemExit("bench.py --case: unknown case(s) %s" % ", ".join(sorted(unknown)))
        cases = [c for c in cases if c[0] in only]
    for name, M, N, K, ta, tb, S, sa, sb in cases:
        if name == "c3.qkv.fwd" and warm_gpu_ms > 0:  # after the tiny LeNet GEMMs, which leave the GPU almost idle
            warm_gpu(torch, rg, warm_gpu_ms)
        def draw(n, scale):
            if scale < 0:  # U(-|scale|, |scale|)
                return (torch.rand(n, device="cuda", generator=gen) * 2 - 1) * -scale
            return torch.randn(n, device="cuda", generator=gen) * scale
        dA, dB = draw(M * K, sa), draw(K * N, sb)
        cfg = rg.Config(slices=S, trans_a=ta, trans_b=tb)
        plan = rg.make_plan(M, N, K, cfg)
        ws = torch.empty(max(plan.workspace_bytes, 1), dtype=torch.uint8, device="cuda")
        C = torch.empty((M, N), dtype=torch.float32, device="cuda")

        def step(events=None, stream=sp):
            code = rg.repro_gemm_fp32_ws(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K, cfg,
                                         ws.data_ptr(), ws.numel(), stream, events)
            if code != 0:
                raise rg.ReproGemmError(code, name)

        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        step()
        e1.record()
        torch.cuda.synchronize()
        once = max(e0.elapsed_time(e1), 1e-3)
        first = C.clone()
        for _ in range(max(3, int(warm_ms / once))):
            step()
        reps = max(10, int(timed_ms / once))
        e0.record()
        for _ in range(reps):
            step()
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        for e in evs:
            e.record()
        torch.cuda.synchronize()
        stages = []
        for _ in range(5):
            step([e.cuda_event for e in evs])
            torch.cuda.synchronize()
            stages.append([evs[i].elapsed_time(evs[i + 1]) for i in range(3)])
        slice_ms, contract_ms, final_ms = (statistics.median(x[i] for x in stages) for i in range(3))
        graph_ms = round(_graph_ms(torch, step), 4) if ms < 0.1 else None
        flops = 2.0 * M * N * K
        # Achieved HBM rates of the HBM-bound stages on their algorithmic bytes: the slicing
        # reads 4(MK + KN) and writes S(MK + NK) digit bytes + 4(M + N) exponent bytes; the
        # split-K reduction (plans with split > 1) reads 8 * split * MN int64 partials and writes
        # 4MN bytes of C (at split 1 the rounding is fused into the contraction).
        slice_bytes = 4 * (M * K + K * N) + S * (M * K + N * K) + 4 * (M + N)
        final_bytes = 8 * plan.split_k * M * N + 4 * M * N if plan.split_k > 1 else None
        small = (plan.tile_m, plan.tile_n) == (32, 32)  # one launch: no slicing or reduction
        if plan.tile_m == 32 and plan.tile_n > 32:
            # band kernel: the slicing stage is op(B)'s one pass (op(A) is sliced inside the
            # contraction launch)
            slice_bytes = 4 * K * N + S * N * K + 4 * N
        rows.append({"case": name, "M": M, "N": N, "K": K, "ta": ta, "tb": tb, "S": S,
                     "ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 2), "reps": reps,
                     "graph_ms": graph_ms,
                     "slice_ms": round(slice_ms, 4), "contract_ms": round(contract_ms, 4),
                     "final_ms": round(final_ms, 4),
                     "slice_gbs": (None if small else
                                   round(slice_bytes / (max(slice_ms - event_floor_ms, 1e-4) * 1e-3) / 1e9, 1)),
                     "final_gbs": (round(final_bytes / (max(final_ms - event_floor_ms, 1e-4) * 1e-3) / 1e9, 1)
                                   if final_bytes and not small else None),
                     "contract_int8_frac": round(S * S * flops / (contract_ms * 1e-3) / (PEAK_INT8_TOPS * 1e12), 4),
                     "plan": "%dx%d split %d" % (plan.tile_m, plan.tile_n, plan.split_k),
                     "repeat_bits_equal": bool(torch.equal(first.view(torch.int32), C.view(torch.int32)))})
        del dA, dB, ws, C, first
        torch.cuda.empty_cache()
    print(json.dumps({"mode": "configs", "data": "synthetic (torch.randn / uniform on the GPU, seed 2024)",
                      "event_floor_ms": round(event_floor_ms, 4),
                      "hbm_rates": "slice_gbs / final_gbs: algorithmic bytes over the stage time less "
                                   "event_floor_ms, against 8000 GB/s",
                      "cases": rows}))


SWEEP_SHAPES = [("sq4096", 4096, 4096, 4096, 0, 0), ("sq2048", 2048, 2048, 2048, 0, 0),
                ("sq1024", 1024, 1024, 1024, 0, 0), ("r512x512x8192", 512, 512, 8192, 0, 0),
                ("r4096x1024x1024", 4096, 1024, 1024, 0, 1), ("r16384x1024x4096", 16384, 1024, 4096, 0, 0),
                ("r2048x8192x1024", 2048, 8192, 1024, 0, 0)]


def warm_gpu(torch, rg, ms=400.0):
    """About `ms` of back-to-back 4096^3 GEMMs: takes the GPU past the power-management
    transient that follows idle, so that the first timings are not slowed by it."""
    n = 4096
    A = torch.randn(n * n, device="cuda")
    B = torch.randn(n * n, device="cuda")
    C = torch.empty(n * n, device="cuda")
    cfg = rg.Config()
    plan = rg.make_plan(n, n, n, cfg)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device="cuda")
    sp = torch.cuda.current_stream().cuda_stream
    for _ in range(int(ms / 0.5)):
        code = rg.repro_gemm_fp32_ws(A.data_ptr(), B.data_ptr(), C.data_ptr(), n, n, n, cfg,
                                     ws.data_ptr(), ws.numel(), sp, None)
        if code != 0:
            raise rg.ReproGemmError(code, "warm_gpu")
    torch.cuda.synchronize()
    del A, B, C, ws
    torch.cuda.empty_cache()


SWEEP_TILES = ((128, 128), (128, 64), (64, 128), (64, 64), (64, 192), (192, 64))


def sweep_plans(torch, rg, warm_ms=15.0, timed_ms=15.0):
    """One JSON line per shape: every block tile (SWEEP_TILES) x split_k in {1, 2, 3, 4, 6, 8,
    12, 16} forced through Config, each timed over about `timed_ms` of back-to-back GEMMs after
    about `warm_ms` (S = 3; the GPU warmed first), next to the plan the planner picks. The data
    the planner's cost model (rg_api.cpp::plan_cost) is fitted to."""
    cases = [(c[0], c[1], c[2], c[3], c[4], c[5]) for c in _config_cases() if c[0].startswith(("c3", "c5"))]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2024)
    sp = torch.cuda.current_stream().cuda_stream
    warm_gpu(torch, rg)
    for name, M, N, K, ta, tb in cases + SWEEP_SHAPES:
        dA = torch.randn(M * K, device="cuda", generator=gen)
        dB = torch.randn(K * N, device="cuda", generator=gen)
        C = torch.empty((M, N), device="cuda")
        auto = rg.make_plan(M, N, K, rg.Config(trans_a=ta, trans_b=tb))
        res, seen = [], set()
        for tm, tn in SWEEP_TILES:
            for split in (1, 2, 3, 4, 6, 8, 12, 16):
                cfg = rg.Config(trans_a=ta, trans_b=tb, tile_m=tm, tile_n=tn, split_k=split)
                plan = rg.make_plan(M, N, K, cfg)
                if (tm, tn, plan.split_k) in seen:
                    continue
                seen.add((tm, tn, plan.split_k))
                ws = torch.empty(max(plan.workspace_bytes, 1), dtype=torch.uint8, device="cuda")

                def step():
                    code = rg.repro_gemm_fp32_ws(dA.data_ptr(), dB.data_ptr(), C.data_ptr(), M, N, K,
                                                 cfg, ws.data_ptr(), ws.numel(), sp, None)
                    if code != 0:
                        raise rg.ReproGemmError(code, name)

                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                step()
                e1.record()
                torch.cuda.synchronize()
                once = max(e0.elapsed_time(e1), 1e-3)
                for _ in range(max(5, int(warm_ms / once))):
                    step()
                n = max(10, int(timed_ms / once))
                e0.record()
                for _ in range(n):
                    step()
                e1.record()
                torch.cuda.synchronize()
                res.append([tm, tn, plan.split_k, round(e0.elapsed_time(e1) / n, 4)])
                del ws
        print(json.dumps({"mode": "sweep_plans", "case": name, "M": M, "N": N, "K": K, "ta": ta,
                          "tb": tb, "auto": [auto.tile_m, auto.tile_n, auto.split_k], "res": res}),
              flush=True)
        del dA, dB, C
        torch.cuda.empty_cache()


def _rel_error(C, ref):
    """(relative Frobenius error, worst row) of C against ref over the finite differences, as
    the reference's hash tool reports them (hash_repro_gemm.cu:171-188)."""
    d = C.astype(np.float64) - ref
    ok = np.isfinite(d)
    d2 = np.where(ok, d * d, 0.0)
    r2 = np.where(ok, ref * ref, 0.0)
    row_e, row_r = d2.sum(axis=1), r2.sum(axis=1)
    live = row_r > 0
    worst = float(np.sqrt(row_e[live] / row_r[live]).max()) if live.any() else 0.0
    return (float(np.sqrt(d2.sum() / r2.sum())) if r2.sum() > 0 else 0.0), worst


def accuracy_mode(torch, rg):
    """One JSON line: accuracy against FP64 of the GPU results for every input distribution of
    the reference's hash tool at its default shape (256 x 256 x 1024) and S = 1, 2, 3 (bits
    checked against the oracle), and of the 4096^3 headline GEMM, next to FP32 torch.matmul."""
    from oracle import oracle as O

    torch.backends.cuda.matmul.allow_tf32 = False
    rows = []
    M, N, K = 256, 256, 1024
    for dist in O.HASH_DISTS:
        A, B = O.gen_hash_inputs(M, N, K, 12345, dist)
        with np.errstate(over="ignore", invalid="ignore"):
            ref = A.astype(np.float64) @ B.astype(np.float64)
        dA, dB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
        row = {"dist": dist, "M": M, "N": N, "K": K}
        for S in (1, 2, 3):
            C = rg.gemm(dA, dB, M, N, K, False, False, S).cpu().numpy()
            want = O.cpu_gemm(A, B, M, N, K, 0, 0, S)
            with np.errstate(over="ignore", invalid="ignore"):
                tot, worst = _rel_error(C, ref)
            row["S%d" % S] = {"rel_frobenius": tot, "worst_row": worst,
                              "bits_equal_oracle": bool(np.array_equal(C.view(np.uint32), want.view(np.uint32)))}
        with np.errstate(over="ignore", invalid="ignore"):
            row["torch_fp32"] = _rel_error(torch.matmul(dA, dB).cpu().numpy(), ref)[0]
        rows.append(row)
    n = 4096
    A, B = make_normal(n)
    dA, dB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
    ref64 = torch.matmul(dA.double(), dB.double())
    head = {"shape": "4096^3 N(0,1), bench inputs"}

    def rel(C):
        d = (C.double() - ref64)
        return float(torch.sqrt((d * d).sum() / (ref64 * ref64).sum()))

    for S in (1, 2, 3):
        head["S%d" % S] = rel(rg.gemm(dA, dB, n, n, n, False, False, S))
    head["torch_fp32"] = rel(torch.matmul(dA, dB))
    print(json.dumps({"mode": "accuracy", "reference": "FP64 product", "hash_tool_dists": rows,
                      "headline": head}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-adversarial", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=None,
                    help="threads of the CPU baseline (default: REPRO_CPU_THREADS, else every CPU "
                         "this process may run on)")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--widened", action="store_true",
                    help="time the exact sum, convolutions, batched GEMM and Linear layer instead")
    ap.add_argument("--suite", action="store_true",
                    help="time the reference GPT-2 suite's 21 GEMMs (1024 tokens) instead")
    ap.add_argument("--suite-out", default=None,
                    help="with --suite: also write the reference suite's result file (OP lines "
                         "with input and output hashes) to this path")
    ap.add_argument("--configs", action="store_true",
                    help="time every GEMM of BASELINE configurations 1, 2, 3 and 5 instead")
    ap.add_argument("--case", default=None,
                    help="with --configs: comma-separated case names to run (e.g. "
                         "c5.tall_skinny,c3.attn_proj.dW)")
    ap.add_argument("--warm-ms", type=float, default=400.0,
                    help="with --configs: ms of 4096^3 GEMMs that bring the GPU out of idle "
                         "first (0 skips them, for profiler runs)")
    ap.add_argument("--sweep-plans", action="store_true",
                    help="time every block tile x split on the planner's fitting shapes instead")
    ap.add_argument("--accuracy", action="store_true",
                    help="report accuracy against FP64 (the reference hash tool's distributions "
                         "and the headline GEMM) instead")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run 3 device-to-device copies of 256 MiB (a plain copy kernel of "
                         "known size, to scale rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (the "
              "reproducible GEMM would shard along M or N with no exchange, or along K with "
              "one exact int64 all-reduce, without changing bits).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import bit_reproducible_training_amd as rg

    if args.suite:
        suite(torch, rg, out_path=args.suite_out)
        return
    if args.configs:
        configs_mode(torch, rg, only=args.case.split(",") if args.case else None,
                     warm_gpu_ms=args.warm_ms, calibrate=args.calibrate)
        return
    if args.accuracy:
        accuracy_mode(torch, rg)
        return
    if args.sweep_plans:
        sweep_plans(torch, rg)
        return
    if args.cpu_threads is None:
        args.cpu_threads = default_cpu_threads(host_cpus())
    if args.widened:
        widened(torch, rg, cpu=not args.no_cpu, threads=args.cpu_threads)
        return

    n = args.size
    S = 3
    A, B = make_normal(n)
    head = time_workload(torch, rg, A, B, n, args.steps, args.warmup, args.calibrate, steady=True)
    adv = None
    if not args.no_adversarial:
        Aa, Ba = make_adversarial(n)
        adv = time_workload(torch, rg, Aa, Ba, n, args.steps, args.warmup)
        del Aa, Ba

    fixtures = {}
    for name in ("baseline_configs.json", "bench_fixtures.json"):
        path = os.path.join(REPO, "tests", "golden", name)
        if os.path.exists(path):
            with open(path) as f:
                fixtures.update({c["name"]: c["out_hash"] for c in json.load(f)["cases"]})

    cpu, checks = None, {}
    if not args.no_cpu:
        cpu, checks, _ = cpu_baseline(A, B, n, head["C"], args.cpu_threads, args.cpu_reps, fixtures,
                                      adv["C"] if adv else None)
    bit_exact = all(checks.values()) if checks else None

    # The practical ceiling: sustained int8 MFMA rate with register operands (no memory), on
    # random bytes, on random bytes in [0, 127] (the lower digit planes' data) and on zeros; the
    # matrix cores' power draw depends on the operands.
    ceiling = {"dense_tops": round(rg.measure_mfma_int8_rate(True), 1),
               "low7_tops": round(rg.measure_mfma_int8_rate(low7=True), 1),
               "zero_tops": round(rg.measure_mfma_int8_rate(False), 1)}

    M = N = K = n
    ms = head["ms_per_step"]
    eff = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    int8_ops = S * S * 2.0 * M * N * K
    slice_bytes = 4 * (M * K + K * N) + S * (M * K + N * K) + 4 * (M + N)
    # The measured traffic figures hold for the workload they were measured on only.
    measured_shape = (M, N, K, S) == (4096, 4096, 4096, 3)
    contract_traffic = measured_traffic("contract") if measured_shape else None
    slice_traffic = measured_traffic("slicing") if measured_shape else None
    contract_tops = int8_ops / (head["contract_ms"] * 1e-3) / 1e12
    line = {
        "metric": "effective FP32 TFLOP/s, S=3 repro GEMM 4096^3; % int8 MFMA peak; bit-exact",
        "value": round(eff, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "reproducible GEMM M=N=K=%d, S=3, NN, N(0,1) inputs from one "
                               "SplitMix64 stream seeded 12345 (the reference bench's recipe; "
                               "BASELINE config 4 size); plan %s" % (n, head["plan"]),
                   "M": M, "N": N, "K": K, "slices": S},
        "int8_peak_frac_end_to_end": round(S * S * eff / PEAK_INT8_TOPS, 4),
        "stages_ms": {"slice": round(head["slice_ms"], 4), "contract": round(head["contract_ms"], 4),
                      "final": round(head["final_ms"], 4)},
        "roofline": {"bound": "mfma", "achieved": round(contract_tops, 2), "peak": PEAK_INT8_TOPS,
                     "unit": "TFLOP/s", "frac": round(contract_tops / PEAK_INT8_TOPS, 4),
                     "traffic": contract_traffic,
                     "traffic_source": "rocprofv3 FETCH_SIZE + WRITE_SIZE per launch, scaled by a "
                                       "256 MiB copy (profiles/contract_mfma_4096cube_traffic.md); "
                                       "null when rg_contract.hip or rg_internal.h differs from the "
                                       "measured sources",
                     "kernel": "contract_mfma<3,2,1,2,4>: int8 ops = 9 * 2MNK per launch, one "
                               "launch per step; achieved = ops / HIP-event duration"},
        # The slicing stage against the HBM roofline: algorithmic bytes = fp32 inputs read once
        # (4(MK + KN)) + S digit planes written (S(MK + NK)) + the int32 exponents (4(M + N)),
        # over the stage's HIP-event duration (the slot-marking launch, the one-read slicing
        # launch and the gap between them). traffic: the launches' measured HBM bytes (each
        # input read once at this shape), and the rate they move them at.
        "slicing_roofline": {"bound": "hbm", "achieved": round(slice_bytes / (head["slice_ms"] * 1e-3) / 1e9, 1),
                             "peak": PEAK_HBM_GBS, "unit": "GB/s",
                             "frac": round(slice_bytes / (head["slice_ms"] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                             "bytes": slice_bytes, "traffic": slice_traffic,
                             "traffic_rate": (round(slice_traffic / (head["slice_ms"] * 1e-3) / 1e9, 1)
                                              if slice_traffic else None)},
        "mfma_ceiling_measured": dict(
            ceiling,
            contract_frac_of_dense=round(contract_tops / ceiling["dense_tops"], 4) if ceiling["dense_tops"] else None,
            contract_frac_of_low7=round(contract_tops / ceiling["low7_tops"], 4) if ceiling["low7_tops"] else None),
        "cpu_baseline": cpu,
        "bit_exact": bit_exact,
        "checks": checks,
    }
    if head["steady_ms"]:
        line["steady_state"] = {
            "value": round(2.0 * M * N * K / (head["steady_ms"] * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
            "ms_per_step": round(head["steady_ms"], 4), "steps": STEADY_STEPS,
            "after_gemms": args.warmup + 2 * args.steps + STEADY_WARM,
            "note": "the headline GEMM in the same process once the GPU's clock has settled after the "
                    "power-management transient the timed steps run in; not the headline value"}
    if adv:
        ams = adv["ms_per_step"]
        line["config4_adversarial"] = {
            "value": round(2.0 * M * N * K / (ams * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
            "ms_per_step": round(ams, 4), "contract_ms": round(adv["contract_ms"], 4),
            "contract_int8_frac": round(int8_ops / (adv["contract_ms"] * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4)}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
