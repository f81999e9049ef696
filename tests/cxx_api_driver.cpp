// Test driver of include/repro_gemm.hpp, the C++ interface with the reference's names and
// signatures (repro_gemm_cuda/repro_gemm.cuh:25-75): C-linkage entry points that go through
// the header's inline wrappers, so the Python tests exercise the C++ interface itself
// (Config defaults and fields, Plan, make_plan, repro_gemm_fp32_ws with stage events,
// repro_gemm_fp32, algo_name, MAX_SLICES). TEST INFRASTRUCTURE: built by
// __graft_entry__.build() into tests/_build/libcxxapi.so, linked against librepro_gemm.so.
#include "repro_gemm.hpp"

namespace {
repro_gemm::Config config(int algo, int slices, int ta, int tb, int split, int tile) {
    repro_gemm::Config c;  // the reference's defaults, then the test's fields
    c.algo = static_cast<repro_gemm::Algo>(algo);
    c.slices = slices;
    c.trans_a = ta != 0;
    c.trans_b = tb != 0;
    c.split_k = split;
    if (tile > 0) c.tile_m = c.tile_n = tile;
    return c;
}
}  // namespace

extern "C" {

// The defaults of a value-initialised Config, in field order.
void cx_config_defaults(int* out) {
    const repro_gemm::Config c;
    out[0] = c.split_k;
    out[1] = c.tile_m;
    out[2] = c.tile_n;
    out[3] = c.tile_k;
    out[4] = static_cast<int>(c.algo);
    out[5] = c.slices;
    out[6] = c.trans_a;
    out[7] = c.trans_b;
}

int cx_max_slices() { return repro_gemm::MAX_SLICES; }

const char* cx_algo_name(int algo) { return repro_gemm::algo_name(static_cast<repro_gemm::Algo>(algo)); }

int cx_make_plan(int M, int N, int K, int algo, int slices, int ta, int tb, int split, int tile,
                 int* out_algo, int* out_split, unsigned long long* out_ws) {
    repro_gemm::Plan p;
    const hipError_t e = repro_gemm::make_plan(M, N, K, config(algo, slices, ta, tb, split, tile), &p);
    if (e == hipSuccess) {
        *out_algo = static_cast<int>(p.algo);
        *out_split = p.split_k;
        *out_ws = p.workspace_bytes;
    }
    return static_cast<int>(e);
}

// repro_gemm_fp32_ws on `stream` with four stage events; waits for the last and writes the
// three stage times (ms) to stage_ms when it is not null.
int cx_gemm_ws(const float* A, const float* B, float* C, int M, int N, int K, int algo, int slices,
               int ta, int tb, int split, int tile, void* ws, unsigned long long ws_bytes,
               void* stream, float* stage_ms) {
    hipEvent_t ev[4];
    for (auto& e : ev)
        if (hipEventCreate(&e) != hipSuccess) return static_cast<int>(hipErrorUnknown);
    hipError_t e = repro_gemm::repro_gemm_fp32_ws(A, B, C, M, N, K,
                                                  config(algo, slices, ta, tb, split, tile), ws,
                                                  ws_bytes, static_cast<hipStream_t>(stream), ev);
    if (e == hipSuccess) e = hipEventSynchronize(ev[3]);
    if (e == hipSuccess && stage_ms)
        for (int i = 0; i < 3 && e == hipSuccess; ++i) e = hipEventElapsedTime(&stage_ms[i], ev[i], ev[i + 1]);
    for (auto& x : ev) (void)hipEventDestroy(x);
    return static_cast<int>(e);
}

// repro_gemm_fp32: allocates its workspace, runs on `stream` and synchronises.
int cx_gemm(const float* A, const float* B, float* C, int M, int N, int K, int slices, int ta,
            int tb, void* stream) {
    return static_cast<int>(repro_gemm::repro_gemm_fp32(
        A, B, C, M, N, K, config(0, slices, ta, tb, 1, 0), static_cast<hipStream_t>(stream)));
}

}  // extern "C"
