"""MI355X (gfx950) reproducible FP32 GEMM: int8 slice split, int8 MFMA contraction,
exact recombination. Bit-identical to the CPU definition on every input.

The compute path is librepro_gemm.so (HIP kernels + C ABI, include/repro_gemm.h);
this package is its Python host mirror. Importing it fails if the library is not built.
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
