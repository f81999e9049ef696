"""MI355X (gfx950) reproducible FP32 GEMM: int8 slice split, int8 MFMA contraction,
exact recombination. Bit-identical to the CPU definition on every input. Around it: the
reproducible convolution (forward and both gradients) on the same contraction, the exact
(superaccumulator) sum and non-finite scan the layers need, and the reproducible Linear and
Conv2d layers (autograd) built on them.

The compute path is librepro_gemm.so (HIP kernels + C ABI, include/repro_gemm.h,
include/repro_sum.h, include/repro_conv.h); this package is its Python host mirror. Importing it fails if the
library is not built.
"""
from .repro_gemm import (  # noqa: F401
    MAX_SLICES,
    Algo,
    Config,
    Plan,
    ReproGemmError,
    algo_name,
    bmm,
    gemm,
    make_plan,
    make_plan_strided_batched,
    measure_mfma_int8_rate,
    plan_for_device,
    repro_gemm_fp32,
    repro_gemm_fp32_ws,
    repro_gemm_strided_batched_fp32_ws,
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
from .repro_conv import (  # noqa: F401
    ConvShape,
    conv2d,
    conv2d_grad_input,
    conv2d_grad_input_workspace,
    conv2d_grad_weight,
    conv2d_grad_weight_workspace,
    conv2d_workspace,
    repro_conv2d_grad_input_ws,
    repro_conv2d_grad_weight_ws,
    repro_conv2d_ws,
)
from .layers import (  # noqa: F401
    Conv2d,
    FiniteGuard,
    Linear,
    get_slices,
    guard,
    name_layers,
    set_slices,
)
