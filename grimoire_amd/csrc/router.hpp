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
    // split-K router partials (topk_launch only): logits holds a, part1 b;
    // the top-k forms (a + b) + lbias, writes it back to logits, and picks
    const float* part1 = nullptr;
    const float* lbias = nullptr;
};

hipError_t topk_launch(hipStream_t st, const TopkArgs& a);
hipError_t topk_bf16_launch(hipStream_t st, const uint16_t* logits, int T, int E, int K,
                            int normalize, int32_t* out_e, float* out_w);
// logits = x W^T + bias.  With part1 ([T][E] scratch) and deferred, a
// split-K launch may leave the two partials in logits and part1 and set
// *deferred: the caller then finishes (topk_launch with part1 / lbias, or
// router_finish_launch).  wimg (optional, router_wimg_bytes(T, E, H) bytes,
// 16-byte aligned): scratch for W's limb planes, split once per call
// instead of once per token block.
hipError_t router_logits_launch(hipStream_t st, const float* W, const float* x,
                                const float* bias, float* logits, int T, int E, int H,
                                float* part1 = nullptr, int* deferred = nullptr, void* wimg = nullptr);
// Bytes of the split router's W limb image for this shape (0: that path is
// not taken).
size_t router_wimg_bytes(int T, int E, int H);
// logits = (logits + part1) + bias (bias may be null)
hipError_t router_finish_launch(hipStream_t st, float* logits, const float* part1, const float* bias, int T,
                                int E);
hipError_t rowdot_sigmoid_launch(hipStream_t st, const float* x, const uint16_t* w, float* gate,
                                 int T, int H);

}  // namespace grim
