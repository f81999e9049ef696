// PyTorch binding of the reproducible operations: the compiled counterpart of the reference's
// repro_torch/src/bindings.cpp:43-175,286-297 (_backend.gemm, exact_sum, conv2d,
// conv2d_grad_weight, conv2d_grad_input, scan_finite), with the same names, arguments, checks
// and results.
//
// A GPU tensor runs on the MI355X library (librepro_gemm.so, through its C ABI) on PyTorch's
// current HIP stream of the tensor's device, with the workspace taken from PyTorch's caching
// allocator on that stream: each call has its own workspace, which the allocator hands to no
// other stream's work while this call's kernels may still use it. A CPU tensor runs the CPU
// implementation of the same definition (include/repro_*_cpu.h), which gives the same bits.
// Errors from the library raise the package's ReproGemmError (its .code is the hipError_t);
// argument errors raise ValueError.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "repro_conv.h"
#include "repro_conv_cpu.h"
#include "repro_gemm.h"
#include "repro_gemm_cpu.h"
#include "repro_sum.h"
#include "repro_sum_cpu.h"

namespace {

using torch::Tensor;

// A non-zero hipError_t from the library, raised in Python as error_class(code, what).
struct LibraryError {
    int code;
    std::string what;
};
PyObject* g_error_class = nullptr;  // set once by the package (set_error_class)

void check(int code, const char* what) {
    if (code != 0) throw LibraryError{code, what};
}

void need(bool ok, const std::string& what) {
    if (!ok) throw std::invalid_argument(what);
}

void require_f32(const Tensor& t, const char* name) {
    need(t.scalar_type() == torch::kFloat32, std::string(name) + " must be float32");
}

// Both tensors on the GPU (true), both on the CPU (false), anything else is an error.
bool on_gpu(const Tensor& a, const Tensor& b, const char* op) {
    need(a.device() == b.device(), std::string(op) + ": tensors must be on the same device");
    need(a.is_cuda() || a.is_cpu(), std::string(op) + ": tensors must be on the CPU or a GPU");
    return a.is_cuda();
}

void* stream_of(const Tensor& t) { return c10::hip::getCurrentHIPStream(t.get_device()).stream(); }

Tensor workspace_like(size_t bytes, const Tensor& t) {
    return torch::empty({(int64_t)std::max<size_t>(bytes, 1)}, t.options().dtype(torch::kUInt8));
}

// C[M, N] = op(A) op(B) (bindings.cpp:43-66), with the planner's options exposed: split_k,
// the block tile and the algorithm change the speed, never a bit; they apply to GPU tensors.
// out, when given, must be a contiguous float32 tensor of M*N elements on A's device.
Tensor gemm_ex(Tensor A, Tensor B, int M, int N, int K, bool ta, bool tb, int S, int split_k,
               int tile_m, int tile_n, int algo, c10::optional<Tensor> out) {
    require_f32(A, "A");
    require_f32(B, "B");
    const bool gpu = on_gpu(A, B, "gemm");
    A = A.contiguous();
    B = B.contiguous();
    need(M > 0 && N > 0 && K > 0, "gemm: sizes must be positive");
    need(A.numel() == (int64_t)M * K && B.numel() == (int64_t)N * K, "gemm: shape mismatch");
    Tensor C;
    if (out.has_value()) {
        C = *out;
        need(C.scalar_type() == torch::kFloat32, "gemm: out must be float32");
        need(C.device() == A.device(), "gemm: out must be on the inputs' device");
        need(C.is_contiguous() && C.numel() == (int64_t)M * N, "gemm: out must be contiguous with M*N elements");
    } else {
        C = torch::empty({M, N}, A.options());
    }
    if (gpu) {
        c10::DeviceGuard guard(A.device());
        rg_config cfg;
        rg_config_init(&cfg);
        cfg.slices = S;
        cfg.trans_a = ta ? 1 : 0;
        cfg.trans_b = tb ? 1 : 0;
        cfg.split_k = split_k;
        cfg.tile_m = tile_m;
        cfg.tile_n = tile_n;
        cfg.algo = algo;
        rg_plan plan;
        check(rg_make_plan(M, N, K, &cfg, &plan), "gemm plan");
        Tensor ws = workspace_like(plan.workspace_bytes, A);
        check(rg_gemm_fp32_ws(A.data_ptr<float>(), B.data_ptr<float>(), C.data_ptr<float>(), M, N, K,
                              &cfg, ws.data_ptr(), (size_t)ws.numel(), stream_of(A), nullptr),
              "gemm");
        return C;
    }
    need(S >= 1 && S <= 3, "gemm: slices must be 1..3");
    const float* a = A.data_ptr<float>();
    const float* b = B.data_ptr<float>();
    float* c = C.data_ptr<float>();
    py::gil_scoped_release nogil;
    repro_gemm::cpu_gemm(a, b, c, M, N, K, ta, tb, S);
    return C;
}

Tensor gemm(Tensor A, Tensor B, int M, int N, int K, bool ta, bool tb, int S) {
    return gemm_ex(A, B, M, N, K, ta, tb, S, 1, 16, 16, RG_ALGO_AUTO, c10::nullopt);
}

// out[b] = exact sum over a, c of x[a, b, c], rounded once; divided by A * C if mean
// (bindings.cpp:69-91).
Tensor exact_sum(Tensor x, int A, int B, int C, bool mean) {
    require_f32(x, "x");
    need(x.is_cuda() || x.is_cpu(), "sum: x must be on the CPU or a GPU");
    x = x.contiguous();
    need(A > 0 && B > 0 && C > 0, "sum: sizes must be positive");
    need(x.numel() == (int64_t)A * B * C, "sum: shape mismatch");
    Tensor out = torch::empty({B}, x.options());
    if (x.is_cuda()) {
        c10::DeviceGuard guard(x.device());
        rg_sum_config cfg;
        rg_sum_config_init(&cfg);
        cfg.mean = mean ? 1 : 0;
        rg_sum_plan plan;
        check(rg_make_sum_plan(A, B, C, &cfg, &plan), "sum plan");
        Tensor ws = workspace_like(plan.workspace_bytes, x);
        check(rg_sum_fp32_ws(x.data_ptr<float>(), out.data_ptr<float>(), A, B, C, &cfg, ws.data_ptr(),
                             (size_t)ws.numel(), stream_of(x)),
              "sum");
        return out;
    }
    const float* p = x.data_ptr<float>();
    float* o = out.data_ptr<float>();
    py::gil_scoped_release nogil;
    repro_sum::cpu_sum(p, o, A, B, C, mean);
    return out;
}

repro_conv::ConvShape shape_of(const std::vector<int64_t>& x_shape, int F, int KH, int KW, int SY,
                               int SX, int PY, int PX) {
    need(x_shape.size() == 4, "conv: the input must be [N][C][H][W]");
    repro_conv::ConvShape g;
    g.N = (int)x_shape[0];
    g.C = (int)x_shape[1];
    g.H = (int)x_shape[2];
    g.W = (int)x_shape[3];
    g.F = F;
    g.KH = KH;
    g.KW = KW;
    g.SY = SY;
    g.SX = SX;
    g.PY = PY;
    g.PX = PX;
    return g;
}

typedef int (*ConvWorkspaceFn)(const rg_conv_shape*, int, size_t*);
typedef int (*ConvRunFn)(const float*, const float*, float*, const rg_conv_shape*, int, void*, size_t, void*);

// One convolution pass on the GPU: plan, per-call workspace, launch on the current stream.
void conv_gpu(ConvWorkspaceFn ws_fn, ConvRunFn run, const Tensor& a, const Tensor& b, Tensor& out,
              const repro_conv::ConvShape& g, int S, const char* what) {
    c10::DeviceGuard guard(a.device());
    const rg_conv_shape s = g.to_c();
    size_t bytes = 0;
    check(ws_fn(&s, S, &bytes), "conv plan");
    Tensor ws = workspace_like(bytes, a);
    check(run(a.data_ptr<float>(), b.data_ptr<float>(), out.data_ptr<float>(), &s, S, ws.data_ptr(),
              (size_t)ws.numel(), stream_of(a)),
          what);
}

// out[N][F][OH][OW] from x[N][C][H][W] and w[F][C][KH][KW] (bindings.cpp:112-131).
Tensor conv2d(Tensor x, Tensor w, int SY, int SX, int PY, int PX, int S) {
    require_f32(x, "x");
    require_f32(w, "weight");
    const bool gpu = on_gpu(x, w, "conv2d");
    x = x.contiguous();
    w = w.contiguous();
    need(x.dim() == 4 && w.dim() == 4, "conv2d: x and weight must be 4-D");
    need(w.size(1) == x.size(1), "conv2d: weight channels do not match the input");
    auto g = shape_of(x.sizes().vec(), (int)w.size(0), (int)w.size(2), (int)w.size(3), SY, SX, PY, PX);
    need(repro_conv::cpu_shape_valid(g, S), "conv2d: invalid shape");
    Tensor out = torch::empty({g.N, g.F, g.OH(), g.OW()}, x.options());
    if (gpu) {
        conv_gpu(rg_conv2d_workspace, rg_conv2d_ws, x, w, out, g, S, "conv");
        return out;
    }
    const float *px = x.data_ptr<float>(), *pw = w.data_ptr<float>();
    float* po = out.data_ptr<float>();
    py::gil_scoped_release nogil;
    repro_conv::cpu_conv2d(px, pw, po, g, S);
    return out;
}

// dW[F][C][KH][KW] from dY[N][F][OH][OW] and x (bindings.cpp:133-152).
Tensor conv2d_grad_weight(Tensor dy, Tensor x, int KH, int KW, int SY, int SX, int PY, int PX, int S) {
    require_f32(dy, "dy");
    require_f32(x, "x");
    const bool gpu = on_gpu(dy, x, "conv2d_grad_weight");
    dy = dy.contiguous();
    x = x.contiguous();
    need(x.dim() == 4 && dy.dim() == 4, "conv2d_grad_weight: dy and x must be 4-D");
    auto g = shape_of(x.sizes().vec(), (int)dy.size(1), KH, KW, SY, SX, PY, PX);
    need(repro_conv::cpu_shape_valid(g, S), "conv2d_grad_weight: invalid shape");
    need(dy.size(0) == g.N && dy.size(2) == g.OH() && dy.size(3) == g.OW(),
         "conv2d_grad_weight: dy shape does not match the convolution");
    Tensor dw = torch::empty({g.F, g.C, KH, KW}, x.options());
    if (gpu) {
        conv_gpu(rg_conv2d_grad_weight_workspace, rg_conv2d_grad_weight_ws, dy, x, dw, g, S, "conv weight grad");
        return dw;
    }
    const float *pd = dy.data_ptr<float>(), *px = x.data_ptr<float>();
    float* po = dw.data_ptr<float>();
    py::gil_scoped_release nogil;
    repro_conv::cpu_conv2d_grad_weight(pd, px, po, g, S);
    return dw;
}

// dX[N][C][H][W] (x_shape) from dY[N][F][OH][OW] and w (bindings.cpp:154-175).
Tensor conv2d_grad_input(Tensor dy, Tensor w, std::vector<int64_t> x_shape, int SY, int SX, int PY,
                         int PX, int S) {
    require_f32(dy, "dy");
    require_f32(w, "weight");
    const bool gpu = on_gpu(dy, w, "conv2d_grad_input");
    dy = dy.contiguous();
    w = w.contiguous();
    need(dy.dim() == 4 && w.dim() == 4, "conv2d_grad_input: dy and weight must be 4-D");
    auto g = shape_of(x_shape, (int)w.size(0), (int)w.size(2), (int)w.size(3), SY, SX, PY, PX);
    need(repro_conv::cpu_shape_valid(g, S), "conv2d_grad_input: invalid shape");
    need(w.size(1) == g.C && dy.size(0) == g.N && dy.size(1) == g.F && dy.size(2) == g.OH() &&
             dy.size(3) == g.OW(),
         "conv2d_grad_input: shapes do not match the convolution");
    Tensor dx = torch::empty(x_shape, dy.options());
    if (gpu) {
        conv_gpu(rg_conv2d_grad_input_workspace, rg_conv2d_grad_input_ws, dy, w, dx, g, S, "conv input grad");
        return dx;
    }
    const float *pd = dy.data_ptr<float>(), *pw = w.data_ptr<float>();
    float* po = dx.data_ptr<float>();
    py::gil_scoped_release nogil;
    repro_conv::cpu_conv2d_grad_input(pd, pw, po, g, S);
    return dx;
}

// Lowers flag[0] to op_id if x holds a NaN or infinity, without synchronising
// (bindings.cpp:286-297).
void scan_finite(Tensor x, Tensor flag, int op_id) {
    require_f32(x, "x");
    need(flag.scalar_type() == torch::kInt32 && flag.numel() >= 1, "scan_finite: flag must be an int32 tensor");
    const bool gpu = on_gpu(x, flag, "scan_finite");
    x = x.contiguous();
    if (gpu) {
        c10::DeviceGuard guard(x.device());
        check(rg_scan_finite(x.data_ptr<float>(), flag.data_ptr<int>(), (size_t)x.numel(), op_id, stream_of(x)),
              "finite scan");
        return;
    }
    const float* p = x.data_ptr<float>();
    int* f = flag.data_ptr<int>();
    const int64_t n = x.numel();
    for (int64_t i = 0; i < n; ++i) {
        if ((repro_gemm::float_to_bits(p[i]) & 0x7F800000u) == 0x7F800000u) {
            if (op_id < *f) *f = op_id;
            return;
        }
    }
}

}  // namespace

// 64-bit FNV-1a over the raw bytes of a contiguous CPU tensor, continuing from h: the hash the
// reference's tools print for inputs and outputs (repro_test_util.h:20-24,
// gpt2_ops_suite.cu:80-88), so hashes printed here can be compared with theirs.
uint64_t fnv1a64(const at::Tensor& t, uint64_t h) {
    TORCH_CHECK(!t.is_cuda() && t.is_contiguous(), "fnv1a64: a contiguous CPU tensor");
    const unsigned char* p = static_cast<const unsigned char*>(t.data_ptr());
    const size_t n = (size_t)t.numel() * t.element_size();
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 0x100000001b3ull;
    }
    return h;
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "Reproducible GEMM, exact sum and convolution on PyTorch tensors (MI355X or CPU)";
    m.def("fnv1a64", &fnv1a64, py::arg("tensor"), py::arg("h") = 0xcbf29ce484222325ull);
    m.def("gemm", &gemm);
    m.def("gemm_ex", &gemm_ex);
    m.def("exact_sum", &exact_sum);
    m.def("conv2d", &conv2d);
    m.def("conv2d_grad_weight", &conv2d_grad_weight);
    m.def("conv2d_grad_input", &conv2d_grad_input);
    m.def("scan_finite", &scan_finite);
    m.def("cpu_threads", &repro_gemm::cpu_thread_count);
    m.def("set_error_class", [](py::object cls) {
        Py_XINCREF(cls.ptr());
        Py_XDECREF(g_error_class);
        g_error_class = cls.ptr();
    });
    py::register_exception_translator([](std::exception_ptr p) {
        try {
            if (p) std::rethrow_exception(p);
        } catch (const LibraryError& e) {
            if (!g_error_class) {
                PyErr_SetString(PyExc_RuntimeError, (e.what + ": hip error " + std::to_string(e.code)).c_str());
                return;
            }
            PyObject* err = PyObject_CallFunction(g_error_class, "is", e.code, e.what.c_str());
            if (err) {
                PyErr_SetObject(g_error_class, err);
                Py_DECREF(err);
            }
        }
    });
    m.attr("has_cuda") = true;
}
