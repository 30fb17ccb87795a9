// elementwise.hpp -- small launchers around the MoE path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace grim {

hipError_t permute_rows_bf16_launch(hipStream_t st, const float* src, const int32_t* perm,
                                    uint16_t* dst, int rows, int width);
hipError_t swiglu_bf16_launch(hipStream_t st, const uint16_t* gu, uint16_t* out, int tokens,
                              int inter);
// hidden == 0: every element scaled by gate[0]; else x[t][*] by gate[t]
hipError_t scale_by_sigmoid_launch(hipStream_t st, float* x, const float* gate, int64_t n,
                                   int hidden);

}  // namespace grim
