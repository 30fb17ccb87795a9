// gemv.hpp -- host interface of the decode (slot form) expert products.
#pragma once

#include "common.hpp"

namespace grim {

// One launch of moe_decode_kernel.  Blocks take roles in this order:
// NR router blocks (fp32 router GEMV, then top-k by the last of them),
// NG gate_up blocks (token, slot, row block), ND down blocks (token, row
// block).  `fused` = the roles of this launch depend on each other and
// hand off through ctr[] (8 int32, zero before the launch, zero after).
struct DecodeArgs {
    WView gu, sgu, dn, sdn;
    bool shared;
    // routing (router role)
    const float* router;
    const float* rbias;       // softmax router bias fp32 [E] or null
    int mode, normalize;
    float scaling;
    const uint16_t* bias16;
    const float* bias32;
    int n_group, topk_group;
    float* logits;            // [M][E]
    // data
    const float* x;           // [M][H]
    int32_t* rex;             // [M][K]
    float* rwt;               // [M][K]
    const uint16_t* gate_w;   // bf16 [H] or null: gate[t] = sigmoid(x_t . gate_w)
    float* gate;              // [M]
    const float* gate_in;     // down: shared-expert weight per token or null (= 1)
    float* h;                 // [M][KS][I]
    float* y;                 // [M][H]
    int H, I, K, E, M;
    // plan (decode_plan)
    int lpr_gu, lpr_dn, gu_rb, dn_rb;
    int NR, NG, ND;
    int fused;
    int32_t* ctr;
};

constexpr int kRoleRouter = 1, kRoleGateUp = 2, kRoleDown = 4;

// int32 words of the fused launch's hand-off counters (zero at rest):
// router_done [0], routes_ready [32], timeout [64], h_done and dn_done each
// 64 cache lines of 32 words from [128].
constexpr int kDecodeCounterWords = 128 + 2 * 64 * 32;

void decode_plan(int fmt, DecodeArgs& a, int roles);
size_t decode_lds_bytes(int fmt, const DecodeArgs& a);
hipError_t decode_launch(hipStream_t st, int fmt, const DecodeArgs& a);
int chunk_elems(int fmt);

}  // namespace grim
