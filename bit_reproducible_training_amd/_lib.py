"""Loads librepro_gemm.so (the C ABI in include/repro_gemm.h, include/repro_sum.h and
include/repro_conv.h) through ctypes, and the compiled PyTorch binding (_backend) that calls the
same library for tensors.

Both must have been built (bit_reproducible_training_amd._build.build(), or
__graft_entry__.build()). There is no fallback: if either is missing or does not load,
importing this module raises.
"""
import ctypes
import os

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "librepro_gemm.so")

# hipError_t codes returned by the C ABI.
HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1
HIP_ERROR_NOT_SUPPORTED = 801

# Size of the fixed device workspace of rg_gemm_fp32_noalloc (include/repro_gemm.h).
NOALLOC_SCRATCH_BYTES = 128 << 20


class rg_config(ctypes.Structure):
    _fields_ = [
        ("split_k", ctypes.c_int),
        ("tile_m", ctypes.c_int),
        ("tile_n", ctypes.c_int),
        ("tile_k", ctypes.c_int),
        ("algo", ctypes.c_int),
        ("slices", ctypes.c_int),
        ("trans_a", ctypes.c_int),
        ("trans_b", ctypes.c_int),
    ]


class rg_plan(ctypes.Structure):
    _fields_ = [
        ("algo", ctypes.c_int),
        ("split_k", ctypes.c_int),
        ("workspace_bytes", ctypes.c_size_t),
        ("tile_m", ctypes.c_int),
        ("tile_n", ctypes.c_int),
    ]


class rg_layout_info(ctypes.Structure):
    _fields_ = [
        ("qa", ctypes.c_size_t),
        ("qb", ctypes.c_size_t),
        ("ea", ctypes.c_size_t),
        ("eb", ctypes.c_size_t),
        ("part", ctypes.c_longlong),
        ("Mp", ctypes.c_int),
        ("Np", ctypes.c_int),
        ("Kp", ctypes.c_int),
        ("split_k", ctypes.c_int),
    ]


class rg_sum_config(ctypes.Structure):
    _fields_ = [("chunks", ctypes.c_int), ("mean", ctypes.c_int)]


class rg_sum_plan(ctypes.Structure):
    _fields_ = [("chunks", ctypes.c_int), ("workspace_bytes", ctypes.c_size_t)]


class rg_conv_shape(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int) for name in
                ("N", "C", "H", "W", "F", "KH", "KW", "SY", "SX", "PY", "PX")]


_CONV_WS = (ctypes.c_int, [ctypes.POINTER(rg_conv_shape), ctypes.c_int,
                           ctypes.POINTER(ctypes.c_size_t)])
_CONV_RUN = (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                            ctypes.POINTER(rg_conv_shape), ctypes.c_int, ctypes.c_void_p,
                            ctypes.c_size_t, ctypes.c_void_p])

# Every symbol declared in include/repro_gemm.h, include/repro_sum.h and include/repro_conv.h,
# with its ctypes signature.
_SIGNATURES = {
    "rg_config_init": (None, [ctypes.POINTER(rg_config)]),
    "rg_make_plan": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.POINTER(rg_config), ctypes.POINTER(rg_plan)]),
    "rg_gemm_fp32_ws": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.POINTER(rg_config), ctypes.c_void_p, ctypes.c_size_t,
                                       ctypes.c_void_p, ctypes.c_void_p]),
    "rg_gemm_fp32_noalloc": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                            ctypes.POINTER(rg_config), ctypes.c_void_p]),
    "rg_gemm_fp32": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    ctypes.POINTER(rg_config), ctypes.c_void_p]),
    "rg_algo_name": (ctypes.c_char_p, [ctypes.c_int]),
    "rg_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "rg_workspace_layout": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.POINTER(rg_config),
                                           ctypes.POINTER(rg_layout_info)]),
    "rg_measure_mfma_int8_rate": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_double)]),
    "rg_test_round": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_longlong, ctypes.c_int,
                                     ctypes.c_void_p]),
    "rg_test_set_spin_limit": (ctypes.c_int, [ctypes.c_int]),
    "rg_test_pslice_placement": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                ctypes.POINTER(rg_config), ctypes.c_int,
                                                ctypes.c_int, ctypes.POINTER(ctypes.c_longlong),
                                                ctypes.POINTER(ctypes.c_longlong)]),
    "rg_plan_for_device": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.POINTER(rg_config), ctypes.c_int, ctypes.c_int,
                                          ctypes.POINTER(rg_plan),
                                          ctypes.POINTER(rg_layout_info)]),
    "rg_test_block_order": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                           ctypes.POINTER(rg_config), ctypes.c_int, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_void_p, ctypes.c_longlong,
                                           ctypes.POINTER(ctypes.c_longlong)]),
    "rg_make_plan_strided_batched": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                    ctypes.c_int, ctypes.POINTER(rg_config),
                                                    ctypes.POINTER(rg_plan)]),
    "rg_gemm_strided_batched_fp32_ws": (ctypes.c_int, [
        ctypes.c_void_p, ctypes.c_longlong, ctypes.c_longlong,
        ctypes.c_void_p, ctypes.c_longlong, ctypes.c_longlong,
        ctypes.c_void_p, ctypes.c_longlong, ctypes.c_longlong,
        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(rg_config),
        ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "rg_sum_config_init": (None, [ctypes.POINTER(rg_sum_config)]),
    "rg_make_sum_plan": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.POINTER(rg_sum_config), ctypes.POINTER(rg_sum_plan)]),
    "rg_sum_plan_for_device": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                              ctypes.POINTER(rg_sum_config), ctypes.c_int,
                                              ctypes.POINTER(rg_sum_plan)]),
    "rg_sum_fp32_ws": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.POINTER(rg_sum_config),
                                      ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "rg_sum_fp32": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_int, ctypes.POINTER(rg_sum_config), ctypes.c_void_p]),
    "rg_scan_finite": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                      ctypes.c_int, ctypes.c_void_p]),
    "rg_conv_shape_init": (None, [ctypes.POINTER(rg_conv_shape)]),
    "rg_conv2d_workspace": _CONV_WS,
    "rg_conv2d_grad_weight_workspace": _CONV_WS,
    "rg_conv2d_grad_input_workspace": _CONV_WS,
    "rg_conv2d_ws": _CONV_RUN,
    "rg_conv2d_grad_weight_ws": _CONV_RUN,
    "rg_conv2d_grad_input_ws": _CONV_RUN,
    "rg_conv2d_algo": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(rg_conv_shape), ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_int)]),
    "rg_conv2d_algo_workspace": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(rg_conv_shape),
                                                ctypes.c_int, ctypes.c_int,
                                                ctypes.POINTER(ctypes.c_size_t)]),
    "rg_conv2d_algo_ws": (ctypes.c_int, [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.POINTER(rg_conv_shape),
                                         ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                         ctypes.c_size_t, ctypes.c_void_p]),
}

EXPORTED = tuple(_SIGNATURES)


def _bind_after_torch():
    """Makes the library use the same HIP runtime as PyTorch.

    torch bundles its own libamdhip64 (SONAME libamdhip64.so.7, requested by libtorch_hip
    as plain "libamdhip64.so" from torch/lib). If librepro_gemm.so were loaded first, the
    dynamic loader would bind the system runtime, and a later `import torch` would map a
    second HIP runtime into the process, which breaks both. Importing torch first lets the
    loader resolve this library's libamdhip64.so.7 to torch's already-loaded copy.
    The compiled binding links libtorch as well.
    """
    import torch  # noqa: F401


def hip_runtimes_mapped():
    """Paths of every libamdhip64 mapped into this process (should be exactly one)."""
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and "libamdhip64" in os.path.basename(parts[5]):
                paths.add(os.path.realpath(parts[5]))
    return sorted(paths)


def _load():
    _bind_after_torch()
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            "librepro_gemm.so is not built (%s); run __graft_entry__.build() or "
            "python -m bit_reproducible_training_amd._build" % LIB_PATH)
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _load_backend():
    """The compiled binding, after torch (it links libtorch) and after librepro_gemm.so, which
    it uses through the same mapping."""
    import importlib

    try:
        return importlib.import_module(__package__ + "._backend")
    except ImportError as e:
        raise ImportError("the PyTorch binding _backend is not built (%s); run "
                          "__graft_entry__.build()" % e) from e


_backend = _load_backend()


def error_string(code):
    s = lib.rg_error_string(int(code))
    return s.decode() if s else "hip error %d" % code
