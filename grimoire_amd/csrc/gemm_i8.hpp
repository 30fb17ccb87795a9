// gemm_i8.hpp -- host interface of the INT8 grouped GEMM (int8 MFMA on
// activation limbs) and its quantisers.
#pragma once

#include "common.hpp"

namespace grim {

struct GemmI8Args {
    const uint8_t* w;           // routed experts' int8 codes [E*N][row_bytes]
    const float* ws;            // per-output-channel scales [E*N]
    int64_t row_bytes;
    const uint8_t* w_sh;        // shared expert [N][row_bytes_sh] (T_sh > 0)
    const float* ws_sh;
    int64_t row_bytes_sh;
    int N, K, I;                // N = 2I for SwiGLU
    int swiglu;
    const int8_t* A;            // limbs, row r = [K/64][2][64] bytes: per 64-K block the hi
                                // limb's 64 codes, then the lo limb's
    const float* sa;            // row scales [R]: a = s * (hi + lo / 254)
    const int8_t* A_sh;         // shared rows [T_sh], same layout
    const float* sa_sh;
    float* out;                 // SwiGLU: h [R][I]; else [R][N]
    float* out_sh;              // same for the shared rows
    const int32_t* offsets;     // [E]
    const int32_t* counts;      // [E]
    const int32_t* tile_e;      // [tmax], -1 padded (128-row m-tiles)
    const int32_t* tile_mb;
    int tmax;
    const int32_t* n_tiles_dev; // live routed tile count (device) or null = tmax
    int T_sh;                   // shared-expert rows (0 = none)
    // split > 0: rows mode -- the table is not read; each kernel forms its
    // tile list from counts (num_experts <= 1024): experts of more than
    // split rows in 128-row tiles, the others in 32-row tiles on the
    // narrow kernel.  0: the tile table, all on 128-row tiles.
    int split;
    int num_experts;
    int list_lo;                // set by the launcher: the 128-row list takes counts > list_lo
    // gather mode (gather != null): the routed rows are not stored permuted;
    // routed row r reads row gather[r] of A (gather_rows rows), the row
    // scales stay per routed row (sa[r])
    const int32_t* gather;
    int gather_rows;
    unsigned long long* ts;     // item timestamps (GRIM_TIMING builds only), else null
};

constexpr int kI8MaxListExperts = 1024;
// rows mode: experts of at most this many rows run on 32-row tiles
constexpr int kI8DefaultSplit = 64;

bool gemm_i8_shape_ok(int N, int K, int I, int swiglu);
// gather mode needs K tiles enough for a row map requested with an item's
// first tile to land before the item streams its successor's first tiles
bool gemm_i8_gather_ok(int K, int rows);
hipError_t gemm_i8_launch(hipStream_t st, const GemmI8Args& g);
// src fp32 [rows][n] -> limb rows [rows][n/64][2][64] + scale [rows]
// (n % 64 == 0, n <= 4096)
// (src2, rows2, dst2, scale2: a second row set in the same launch)
hipError_t quant_rows_launch(hipStream_t st, const float* src, int rows, int n, int8_t* dst,
                             float* scale, const float* src2 = nullptr, int rows2 = 0,
                             int8_t* dst2 = nullptr, float* scale2 = nullptr);
// token rows of x fp32 [T][n] -> limbs at their K permuted rows (inverse
// [T][K]) when xq is given, at their own row when xrowq is given; the row
// scale at every permuted row (sq) and own row (srow); perm, when given,
// gets the token of every permuted row (the gather map of gather mode);
// gate_w (bf16 [n], 16-byte aligned, or null): gate[t] = sigmoid(x_t . w)
hipError_t quant_permute_launch(hipStream_t st, const float* x, int T, int n, int K,
                                const int32_t* inverse, int8_t* xq, float* sq, int8_t* xrowq,
                                float* srow, int32_t* perm, const uint16_t* gate_w = nullptr,
                                float* gate = nullptr);

}  // namespace grim
