// dispatch.hpp -- host interface of dispatch and combine kernels.
#pragma once

#include "common.hpp"

namespace grim {

struct DispatchArgs {
    const int32_t* ids;     // [T*K]
    int T, K, E, H;
    const void* hidden;     // fp32 or bf16 [T][H] (null: no permute pass)
    int hidden_bf16;
    uint16_t* xperm;        // bf16 [T*K][H] or null
    uint16_t* xrow;         // bf16 [T][H] or null
    int32_t* counts;        // [E]
    int32_t* offsets;       // [E]
    int32_t* inverse;       // [T*K]
    int32_t* perm_token;    // [T*K] or null
    int32_t* tile_e;        // [tmax] or null
    int32_t* tile_mb;
    int tmax, mc;
    void* workspace;        // dispatch_workspace_bytes
};

struct CombineArgs {
    const void* src;        // [R][H] fp32 or bf16
    int src_bf16;
    const int32_t* inverse; // [T*K]
    const float* rw;        // [T*K]
    const void* shared_src; // [T][H] or null
    int shared_bf16;
    const float* gate;      // [T] or null
    float* dst;             // [T][H]
    int T, K, H;
    int p0 = 0, p1 = 0x7FFFFFFF;  // routes with inverse in [p0, p1) read src row p - p0
    int accumulate = 0;           // dst += instead of dst =
};

// Fused combine + residual + RMSNorm (src/prefill.cpp:1004-1045); K == 0 is
// the residual RMSNorm without experts (src/prefill.cpp:627-700).
struct NormArgs {
    float* h;                // [T][H] residual stream, updated in place
    const uint16_t* routed;  // [R][H] bf16 expert outputs, dispatch order
    const int32_t* inverse;  // [T*K]
    const float* rw;         // [T*K]
    const float* shared;     // [T][H] or null
    const float* shared2;    // [T][H] or null, added after shared
    const uint16_t* weight;  // [H] bf16 norm weight
    float offset;            // added to every norm weight
    float* out;              // [T][H] or null
    uint16_t* out_bf;        // [T][H] or null
    int T, K, H;
    float eps;
};

size_t dispatch_workspace_bytes(int T, int K, int E);
// Where the dispatch leaves the live m-tile count inside its workspace.
int32_t* dispatch_live_tiles(void* workspace, int T, int K, int E);
hipError_t dispatch_launch(hipStream_t st, const DispatchArgs& a);
hipError_t combine_launch(hipStream_t st, const CombineArgs& a);
// Global routes -> one shard's local routes (expert - begin, or -1 / 0).
hipError_t route_local_launch(hipStream_t st, const int32_t* ids, const float* w, int32_t* lids, float* lw,
                              int R, int begin, int count);
hipError_t combine_norm_launch(hipStream_t st, const NormArgs& a);

}  // namespace grim
