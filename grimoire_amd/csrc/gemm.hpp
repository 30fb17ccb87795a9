// gemm.hpp -- host interface of the grouped MFMA GEMM.
#pragma once

#include "common.hpp"

namespace grim {

struct GemmArgs {
    WView w;                    // routed experts [E*N][K]
    WView w_sh;                 // shared expert [N][K] (T_sh > 0)
    int N, K, I;                // N = 2I for SwiGLU
    int swiglu, a_pair, out_bf16;
    const uint16_t* A;          // bf16 [R][K] (or pair [R][2][K])
    const uint16_t* A_sh;       // bf16 [T_sh][K] (or pair)
    void* out;                  // [R][N] fp32/bf16, or SwiGLU pair [R][2][I]
    void* out_sh;               // same for the shared rows
    const int32_t* offsets;     // [E]
    const int32_t* counts;      // [E]
    const int32_t* tile_e;      // [tmax], -1 padded
    const int32_t* tile_mb;
    int tmax;                   // capacity of the tile table
    const int32_t* n_tiles_dev; // live routed tile count (device) or null = tmax
    int T_sh;                   // shared-expert rows (0 = none)
    // rows mode: rows_per_expert[ne] in place of counts and the tile table;
    // every work-group forms the tile order (and, without offsets, the
    // offsets) in LDS, so the caller supplies no scratch
    const int* rows;
    int ne;
};

constexpr int kGemmRowsMaxExperts = 1024;

constexpr int kGemmBM = 128;
// Bridge-only weight format of the grouped GEMM: signed 4-bit codes
// [N][K/2] (low nibble = even K), bf16 group scales [N][K/G] with G a
// multiple of 64 (row_scales = K / G).  src/xe2_grouped_bridge.hpp:22.
constexpr int kGemmFmtS4 = 100;

bool gemm_format_ok(int fmt);
hipError_t gemm_launch(hipStream_t st, int fmt, const GemmArgs& g);

}  // namespace grim
