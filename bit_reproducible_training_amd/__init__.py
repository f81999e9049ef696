"""MI355X (gfx950) reproducible FP32 GEMM: int8 slice split, int8 MFMA contraction,
exact recombination. Bit-identical to the CPU definition on every input. Around it: the
exact (superaccumulator) sum and non-finite scan its layers need, and the reproducible
Linear layer (autograd) built on both.

The compute path is librepro_gemm.so (HIP kernels + C ABI, include/repro_gemm.h and
include/repro_sum.h); this package is its Python host mirror. Importing it fails if the
library is not built.
"""
from .repro_gemm import (  # noqa: F401
    MAX_SLICES,
    Algo,
    Config,
    Plan,
    ReproGemmError,
    algo_name,
    gemm,
    make_plan,
    measure_mfma_int8_rate,
    plan_for_device,
    repro_gemm_fp32,
    repro_gemm_fp32_ws,
    workspace_layout,
)
from .repro_sum import (  # noqa: F401
    SumConfig,
    SumPlan,
    exact_sum,
    make_sum_plan,
    repro_sum_fp32,
    repro_sum_fp32_ws,
    scan_finite,
    sum_plan_for_device,
)
from .layers import FiniteGuard, Linear, get_slices, guard, name_layers, set_slices  # noqa: F401
