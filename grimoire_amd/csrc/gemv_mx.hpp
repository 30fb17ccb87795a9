// gemv_mx.hpp -- host interface of the MXFP4 expert-grouped GEMV on the
// scaled fp4 x fp8 matrix core (gemv_mx.hip).
#pragma once

#include "gemv_grouped.hpp"
#include "router.hpp"

namespace grim {

// MXFP4 experts whose reduction lengths are multiples of 128 (one MFMA K step).
bool gvm_shape_ok(int H, int I);
// K rounded up to whole 256-element stages: the row length a weight padded
// for this kernel holds (payload K'/2 bytes, K'/32 scale bytes per row,
// zero codes under scale byte 127 past K).  Rows of 128-byte multiples
// stream whole memory lines; with K' % 512 == 0 the scale rows are
// 16-byte aligned too.
int gvm_padded_k(int K);
// Bytes of one activation row of K elements in the limb format.
size_t gvm_act_bytes(int K);
// Format rows0 rows of src0 into dst0 and rows1 rows of src1 into dst1.
hipError_t gvm_format_launch(hipStream_t st, const float* src0, int rows0, uint8_t* dst0, const float* src1,
                             int rows1, uint8_t* dst1, int K);
// Routing for a batch of at most kGvmRouteMax routes in two launches: the
// top-k of tk (picks into tk.out_e, weights into tk.out_w), then expert
// counts, offsets, the (expert, kGvMT-row group) table, each route's row
// (inverse) and token (perm_token by row), and the x rows [T][H] in the
// limb format.
constexpr int kGvmRouteMax = 1024;
struct GvmRouteArgs {
    int32_t *counts, *offsets, *tile_e, *tile_mb;
    int tmax;
    int32_t* n_live;
    int32_t *inverse, *perm_token;
    const float* x;
    uint8_t* af;
    int H;
};
hipError_t gvm_route_launch(hipStream_t st, const TopkArgs& tk, const GvmRouteArgs& ra);
// The product: GvArgs with af / af_sh pointing at limb-format rows.
hipError_t gvm_launch(hipStream_t st, const GvArgs& g, bool gate_up);

}  // namespace grim
