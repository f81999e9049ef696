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
# HBM bytes per launch of the contraction at 4096^3 S=3 (fetch + write), from rocprofv3
# FETCH_SIZE / WRITE_SIZE scaled by the same counters on a 256 MiB device copy; see
# profiles/contract_mfma_4096cube_traffic.md. Updated when the kernel changes.
TRAFFIC_BYTES = 671529779
FIXTURE = os.path.join(REPO, "tests", "golden", "baseline_configs.json")

# --------------------------------------------------------------------------------------
# Synthetic input (same recipe and bits as tests/golden/configs.py config 4), vectorised
# SplitMix64 in numpy: draw i of seed s is mix(s + (i + 1) * gamma).
# --------------------------------------------------------------------------------------
_G = np.uint64(0x9E3779B97F4A7C15)


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


# --------------------------------------------------------------------------------------
# CPU baseline and bit-exactness check: the reference's own CPU path (oracle/_ref) or this
# repository's port, used here as the timed baseline and as the checker only.
# --------------------------------------------------------------------------------------
def cpu_baseline(A, B, n, gpu_C, threads, reps, fixtures, gpu_adv=None):
    from oracle import oracle as O

    os.environ["REPRO_CPU_THREADS"] = str(threads)
    kind = "reference" if O.ref is not None else "port"
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
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:  # noqa: BLE001
        model = "unknown"
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
                  "median of %d runs; host cpu %s" % (n, reps, model),
        "ms": round(t * 1e3, 2),
    }
    return base, checks, out_hash


def time_workload(torch, rg, A, B, n, steps, warmup, calibrate=False):
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
    # Timed region: exactly `steps` GEMMs; stage events on the launch stream give the
    # contraction kernel's own duration (event 1 -> event 2 brackets only that launch).
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for e in (x for row in evs for x in row):
        e.record()  # torch creates the HIP event on first record
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step([e.cuda_event for e in evs[i]])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if calibrate:
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    out = {
        "ms_per_step": wall * 1e3 / steps,
        "slice_ms": statistics.mean(e[0].elapsed_time(e[1]) for e in evs),
        "contract_ms": statistics.mean(e[1].elapsed_time(e[2]) for e in evs),
        "final_ms": statistics.mean(e[2].elapsed_time(e[3]) for e in evs),
        "plan": "%s %dx%d split %d" % (rg.algo_name(plan.algo), plan.tile_m, plan.tile_n, plan.split_k),
        "C": C.cpu().numpy(),
    }
    del dA, dB, C, ws
    torch.cuda.empty_cache()
    return out


def suite(torch, rg, reps=10, warmup=2):
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
        ref = op.get("reference_gpu_ms", {})
        best_ref = min((v["ms"] for v in ref.values()), default=None)
        rows.append({"op": op["name"], "shape": op["shape"], "ms": round(ms, 4),
                     "tflops": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 2),
                     "torch_fp32_ms": round(base_ms, 4),
                     "plan": "%dx%d split %d" % (plan.tile_m, plan.tile_n, plan.split_k),
                     "reference_best_gpu_ms": best_ref,
                     "speedup_vs_reference_best": round(best_ref / ms, 1) if best_ref else None})
        del A, B, C, ws
    total = sum(r["ms"] for r in rows)
    ref_total = sum(r["reference_best_gpu_ms"] for r in rows if r["reference_best_gpu_ms"])
    print(json.dumps({"mode": "suite", "tokens": 1024, "slices": 3, "ops": rows,
                      "total_ms": round(total, 3), "reference_best_gpu_total_ms": round(ref_total, 3)}),
          flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-adversarial", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--suite", action="store_true",
                    help="time the reference GPT-2 suite's 21 GEMMs (1024 tokens) instead")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run 3 device-to-device copies of 256 MiB (a plain copy kernel of "
                         "known size, to scale rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the reproducible GEMM shards without changing bits; see DESIGN.md).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import bit_reproducible_training_amd as rg

    if args.suite:
        suite(torch, rg)
        return

    n = args.size
    S = 3
    A, B = make_normal(n)
    head = time_workload(torch, rg, A, B, n, args.steps, args.warmup, args.calibrate)
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

    # The practical ceiling: sustained int8 MFMA rate with register operands (no memory),
    # dense random bytes and zeros; the matrix cores' power draw depends on the operands.
    ceiling = {"dense_tops": round(rg.measure_mfma_int8_rate(True), 1),
               "zero_tops": round(rg.measure_mfma_int8_rate(False), 1)}

    M = N = K = n
    ms = head["ms_per_step"]
    eff = 2.0 * M * N * K / (ms * 1e-3) / 1e12
    int8_ops = S * S * 2.0 * M * N * K
    slice_bytes = 4 * (M * K + K * N) + S * (M * K + N * K) + 4 * (M + N)
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
                     "traffic": TRAFFIC_BYTES,
                     "kernel": "contract_mfma<3,2,1,2,4>: int8 ops = 9 * 2MNK per launch, one "
                               "launch per step; achieved = ops / HIP-event duration"},
        # The slicing stage against the HBM roofline: algorithmic bytes = fp32 inputs read once
        # (4(MK + KN)) + S digit planes written (S(MK + NK)) + the int32 exponents (4(M + N)),
        # over the stage's HIP-event duration (both slicing launches and the gap between them).
        "slicing_roofline": {"bound": "hbm", "achieved": round(slice_bytes / (head["slice_ms"] * 1e-3) / 1e9, 1),
                             "peak": PEAK_HBM_GBS, "unit": "GB/s",
                             "frac": round(slice_bytes / (head["slice_ms"] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                             "bytes": slice_bytes},
        "mfma_ceiling_measured": dict(ceiling, contract_frac_of_dense=round(
            contract_tops / ceiling["dense_tops"], 4) if ceiling["dense_tops"] else None),
        "cpu_baseline": cpu,
        "bit_exact": bit_exact,
        "checks": checks,
    }
    if adv:
        ams = adv["ms_per_step"]
        line["config4_adversarial"] = {
            "value": round(2.0 * M * N * K / (ams * 1e-3) / 1e12, 3), "unit": "TFLOP/s",
            "ms_per_step": round(ams, 4), "contract_ms": round(adv["contract_ms"], 4),
            "contract_int8_frac": round(int8_ops / (adv["contract_ms"] * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4)}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
