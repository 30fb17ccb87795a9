// tiered.hpp -- NVFP4 experts behind a table of block pointers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace grim {

struct TmoeArgs {
    const uint8_t* const* eptr;  // device array [E] of expert blocks (VRAM or pinned host)
    int64_t gu_p, gu_s, dn_p, dn_s, gsc;   // byte offsets inside a block
    int H, I, K, E, M;
    const int32_t* expert;       // [M][K]
    const float* weight;         // [M][K] (down)
    const float* x;              // [M][H] (gate_up)
    float* h;                    // [M][K*I]
    float* y;                    // [M][H] (down)
};

hipError_t tmoe_gate_up(hipStream_t st, const TmoeArgs& a);
hipError_t tmoe_down(hipStream_t st, const TmoeArgs& a);
hipError_t tmoe_decode_bf16(hipStream_t st, const uint8_t* pay, const uint8_t* sc, int N, int K,
                            uint16_t* out);
hipError_t tmoe_scale_cols(hipStream_t st, float* out, int M, int N, int split, float s0, float s1);
hipError_t tmoe_swiglu(hipStream_t st, const float* gu, int M, int I, float sg, float su,
                       uint16_t* h);
hipError_t tmoe_set_rows(hipStream_t st, int32_t* cnt_off, int M);
hipError_t tmoe_store(hipStream_t st, const uint8_t** table, int e, const uint8_t* p);

}  // namespace grim
