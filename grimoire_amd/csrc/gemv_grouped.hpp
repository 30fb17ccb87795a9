// gemv_grouped.hpp -- host interface of the expert-grouped GEMV kernels
// (gemv_grouped.hip): the expert products for batches whose routes spread
// over many experts with few rows each.
#pragma once

#include "common.hpp"

namespace grim {

// Rows per group: an expert's rows are taken MT at a time; each group
// streams the expert's weights once.
constexpr int kGvMT = 4;

struct GvArgs {
    WView w, w_sh;               // routed experts, shared expert
    int N;                       // gate_up: I (row pairs); down: H (rows)
    int K;                       // reduction length: gate_up H, down I
    const float* x;              // gate_up: activations per token [T][H] (fp32; the slow path)
    const uint32_t* af;          // formatted activations: gate_up per token, down per route row
    const uint32_t* af_sh;       // down: formatted shared-expert rows (gate_up: unused)
    const int32_t* perm_token;   // gate_up: route row -> token
    float* h;                    // gate_up out / down in: per route [R][I]
    float* h_sh;                 // shared expert [T_sh][I]
    uint8_t* hf;                 // gate_up, matrix-core kernel: when set, h is written in the
    uint8_t* hf_sh;              // down's limb format (rows of gvm_row_bytes(I)) instead of fp32
    float* y;                    // down out: per route [R][H]
    float* y_sh;                 // shared expert [T_sh][H]
    const int32_t* counts;       // [E]
    const int32_t* offsets;      // [E]
    const int32_t* tile_e;       // [tmax] (expert, MT-row block) table, -1 padded
    const int32_t* tile_mb;
    const int32_t* n_live;       // live entries of the table (device, written by the dispatch)
    int T_sh;                    // shared-expert rows (0 = none)
    unsigned long long* ts;      // phase timestamps (GRIM_TIMING builds only), else null
};

bool gv_shape_ok(int fmt, int H, int I);
// Bytes of one formatted activation row of K elements.
size_t gv_act_bytes(int K);
// Format rows0 rows of src0 into dst0 and rows1 rows of src1 into dst1.
hipError_t gv_format_launch(hipStream_t st, int fmt, const float* src0, int rows0, uint32_t* dst0,
                            const float* src1, int rows1, uint32_t* dst1, int K);
hipError_t gv_launch(hipStream_t st, int fmt, const GvArgs& g, bool gate_up);

}  // namespace grim
