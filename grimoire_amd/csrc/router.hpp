// router.hpp -- host interface of the router kernels.
#pragma once

#include "common.hpp"

namespace grim {

struct TopkArgs {
    const float* logits;     // [T][E]
    int T, E, K;
    int mode;                // 0 softmax, 1 softmax batched, 2 sigmoid, 3 group
    int normalize;
    float scaling;
    const uint16_t* bias16;  // mode 2
    const float* bias32;     // mode 3
    int n_group, topk_group; // mode 3
    int32_t* out_e;
    float* out_w;
};

hipError_t topk_launch(hipStream_t st, const TopkArgs& a);
hipError_t topk_bf16_launch(hipStream_t st, const uint16_t* logits, int T, int E, int K,
                            int normalize, int32_t* out_e, float* out_w);
hipError_t router_logits_launch(hipStream_t st, const float* W, const float* x,
                                const float* bias, float* logits, int T, int E, int H);
hipError_t rowdot_sigmoid_launch(hipStream_t st, const float* x, const uint16_t* w, float* gate,
                                 int T, int H);

}  // namespace grim
