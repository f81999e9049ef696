#pragma once
// repro_conv_shape.h -- the convolution's geometry as a C++ value type, shared by the CPU
// convolution (repro_conv_cpu.h) and C++ callers of the GPU convolution (repro_conv.h).
// Fields, defaults and derived sizes follow repro_conv_cuda/repro_conv_math.cuh:29-42, so code
// written against the reference's ConvShape (repro_torch/src/bindings.cpp:97-110) compiles
// unchanged. Layouts are PyTorch's: input [N][C][H][W], weight [F][C][KH][KW], output and its
// gradient [N][F][OH][OW]; a window is one (n, oy, ox), and its K = C*KH*KW values are
// numbered k = (c * KH + ky) * KW + kx.
#include <cstddef>

#include "repro_conv.h"

namespace repro_conv {

struct ConvShape {
    int N = 0, C = 0, H = 0, W = 0;  // input
    int F = 0, KH = 0, KW = 0;       // filters and their size
    int SY = 1, SX = 1;              // stride
    int PY = 0, PX = 0;              // zero padding on each side

    int K() const { return C * KH * KW; }
    int OH() const { return (H + 2 * PY - KH) / SY + 1; }
    int OW() const { return (W + 2 * PX - KW) / SX + 1; }
    int windows() const { return N * OH() * OW(); }
    size_t input_size() const { return (size_t)N * C * H * W; }
    size_t weight_size() const { return (size_t)F * K(); }
    size_t output_size() const { return (size_t)N * F * OH() * OW(); }

    rg_conv_shape to_c() const {
        rg_conv_shape s;
        s.N = N; s.C = C; s.H = H; s.W = W;
        s.F = F; s.KH = KH; s.KW = KW;
        s.SY = SY; s.SX = SX; s.PY = PY; s.PX = PX;
        return s;
    }
};

}  // namespace repro_conv
