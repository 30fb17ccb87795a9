// gemv.hpp -- host interface of the decode expert-product kernels.
#pragma once

#include "common.hpp"

namespace grim {

struct GemvArgs {
    WView w;                 // routed experts (gate_up or down)
    WView ws;                // shared expert (same role), valid when shared
    bool shared;
    const int32_t* rex;      // [M][K]
    const float* rwt;        // [M][K] (down)
    const float* x;          // [M][H] (gate_up)
    float* h;                // [M][KS][I]
    const uint16_t* gate_w;  // bf16 [H] or null (gate_up)
    float* gate_out;         // [M] (gate_up)
    const float* gate_in;    // [M] or null (down)
    float* y;                // [M][H] (down)
    int H, I, K, M, E;
};

hipError_t gemv_launch(hipStream_t st, int fmt, const GemvArgs& a, bool down);
size_t gemv_lds_bytes(int fmt, int H, int I, int KS, bool down);
int chunk_elems(int fmt);

}  // namespace grim
