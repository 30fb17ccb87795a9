// tiered.hip -- NVFP4 routed experts read through a per-layer table of
// block pointers (include/b70/tiered_moe.hpp, src/tiered_moe.cpp).
//
// Every expert is one self-contained block (gate|up payload [2I][H/2],
// their E4M3 scales [2I][H/16], down payload [H][I/2] and scales [H][I/16],
// then the three fp32 projection scales {gate, up, down, 0}); the table
// entry eptr[e] points into device memory or into pinned host memory, and
// the kernels read both the same way (host blocks over PCIe).  Moving an
// expert between tiers is one block copy plus one table store.
//
// NVFP4 chunk: 16 payload bytes = 32 elements = two 16-element blocks, each
// with its own E4M3 scale.  Per lane and chunk the two block sums are formed
// as fma chains over their 16 elements and scaled once each (the scale is a
// power-of-two-times-small-integer, the same value as scaling every element);
// the projection's fp32 scale is applied once per row at the end, as in
// src/tiered_moe.cpp:45-61.  e2m1 pairs decode through the CDNA4 fp4
// converter (exact in fp32); E4M3 scales by their bit fields.
//
// Lane layout: LPR lanes share one weight row, each walking the row's
// 32-element chunks LPR apart, summed by group_sum<LPR>; a wave holds 64/LPR
// rows at once.  LPR = the chunk count rounded up to a power of two, at most
// 64, so a 2048-wide row is one chunk per lane.
#include "common.hpp"
#include "tiered.hpp"

namespace grim {

constexpr int kTmThreads = 256;

// E4M3 (OCP, no infinities; 0x7F / 0xFF NaN) -> fp32 (include/b70/formats.hpp:157-169)
__device__ __forceinline__ float e4m3_f32(uint32_t b) {
    const uint32_t s = (b & 0x80u) << 24, e = (b >> 3) & 0xFu, m = b & 7u;
    if (e == 0xFu && m == 7u) return bits_f(0x7FC00000u | s);
    if (e == 0u) {
        const float v = float(m) * 0.001953125f;   // m * 2^-9
        return s ? -v : v;
    }
    return bits_f(s | ((e + 120u) << 23) | (m << 20));
}

// 32 elements (payload words p0..p3, low nibble = even element) against
// x[0..31]; s2 holds the two block scales (low byte = elements 0..15).
__device__ __forceinline__ float nv_dot32(uint4 p, uint32_t s2, const float* x) {
    const uint32_t w[4] = {p.x, p.y, p.z, p.w};
    float a[2] = {0.0f, 0.0f};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const f32x2 v[4] = {__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 0),
                            __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 1),
                            __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 2),
                            __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 3)};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            a[d >> 1] = __builtin_fmaf(v[b].x, x[8 * d + 2 * b], a[d >> 1]);
            a[d >> 1] = __builtin_fmaf(v[b].y, x[8 * d + 2 * b + 1], a[d >> 1]);
        }
    }
    return a[0] * e4m3_f32(s2 & 0xFFu) + a[1] * e4m3_f32((s2 >> 8) & 0xFFu);
}

__device__ __forceinline__ void load_x32(const float* p, float* x) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float4 v = reinterpret_cast<const float4*>(p)[j];
        x[4 * j] = v.x; x[4 * j + 1] = v.y; x[4 * j + 2] = v.z; x[4 * j + 3] = v.w;
    }
}

__device__ __forceinline__ uint32_t load_s2(const uint8_t* p) {
    return uint32_t(*reinterpret_cast<const uint16_t*>(p));
}

// gate + up: each lane group owns 2 (gate row, up row) pairs of one
// (token, slot); h[t][slot*I + i] = silu(g * s_gate) * (u * s_up), 0 for a
// slot routed to no expert of this table (id < 0 or >= E).
template <int LPR>
__global__ __launch_bounds__(kTmThreads) void tmoe_gate_up_kernel(TmoeArgs a) {
    constexpr int kGroups = kWave / LPR;            // row groups per wave
    constexpr int kPairs = 2;                       // row pairs per group
    constexpr int kPerBlock = (kTmThreads / kWave) * kGroups * kPairs;
    const int H = a.H, I = a.I, K = a.K;
    const int per_token = (K * I + kPerBlock - 1) / kPerBlock;
    const int t = blockIdx.x / per_token;
    const int lane = threadIdx.x & (kWave - 1), sub = lane % LPR;
    const int group = (threadIdx.x / kWave) * kGroups + lane / LPR;
    const int r0 = (blockIdx.x % per_token) * kPerBlock + group * kPairs;
    const uint8_t* gp[kPairs];
    const uint8_t* gs[kPairs];
    float sgf[kPairs], suf[kPairs], ga[kPairs], ua[kPairs];
    bool on[kPairs];
#pragma unroll
    for (int r = 0; r < kPairs; ++r) {
        const int sr = r0 + r;
        const int slot = sr / I, i = sr % I;
        const int e = sr < K * I ? a.expert[int64_t(t) * K + slot] : -1;
        on[r] = e >= 0 && e < a.E;
        const uint8_t* blk = on[r] ? a.eptr[e] : nullptr;
        gp[r] = on[r] ? blk + a.gu_p + int64_t(i) * (H / 2) : nullptr;
        gs[r] = on[r] ? blk + a.gu_s + int64_t(i) * (H / 16) : nullptr;
        sgf[r] = on[r] ? reinterpret_cast<const float*>(blk + a.gsc)[0] : 0.0f;
        suf[r] = on[r] ? reinterpret_cast<const float*>(blk + a.gsc)[1] : 0.0f;
        ga[r] = 0.0f;
        ua[r] = 0.0f;
    }
    const float* xt = a.x + int64_t(t) * H;
    const int64_t up_p = int64_t(I) * (H / 2), up_s = int64_t(I) * (H / 16);
    for (int c = sub; c < H / 32; c += LPR) {
        uint4 pg[kPairs], pu[kPairs];
        uint32_t sg[kPairs], su[kPairs];
#pragma unroll
        for (int r = 0; r < kPairs; ++r) {
            if (!on[r]) continue;
            pg[r] = *reinterpret_cast<const uint4*>(gp[r] + c * 16);
            pu[r] = *reinterpret_cast<const uint4*>(gp[r] + up_p + c * 16);
            sg[r] = load_s2(gs[r] + c * 2);
            su[r] = load_s2(gs[r] + up_s + c * 2);
        }
        float x[32];
        load_x32(xt + c * 32, x);
#pragma unroll
        for (int r = 0; r < kPairs; ++r) {
            if (!on[r]) continue;
            ga[r] += nv_dot32(pg[r], sg[r], x);
            ua[r] += nv_dot32(pu[r], su[r], x);
        }
    }
#pragma unroll
    for (int r = 0; r < kPairs; ++r) {
        const float g = group_sum<LPR>(ga[r]);
        const float u = group_sum<LPR>(ua[r]);
        const int sr = r0 + r;
        if (sub == 0 && sr < K * I)
            a.h[int64_t(t) * K * I + sr] = on[r] ? silu(g * sgf[r]) * (u * suf[r]) : 0.0f;
    }
}

// down + routing-weighted sum over the K slots in slot order.  The four
// waves of a work-group share its output rows and split the slots (wave w
// takes slots w, w+4, ...), so a wave waits on K/4 rounds of weight loads,
// not K; each (slot, row) dot lands in LDS and one thread per row forms
// y[t][o] = fma chain over slots of (w_s * s_down) * dot, skipping a slot
// with id < 0 (or >= E) or weight 0.
constexpr int kTmMaxK = 32;

template <int LPR, int KW>
__global__ __launch_bounds__(kTmThreads) void tmoe_down_kernel(TmoeArgs a) {
    constexpr int kWaves = kTmThreads / kWave;
    constexpr int kGroups = kWave / LPR;
    constexpr int kRows = 2;
    constexpr int kPerBlock = kGroups * kRows;      // output rows of a work-group
    __shared__ float part[kTmMaxK][kPerBlock];
    const int H = a.H, I = a.I, K = a.K;
    const int per_token = (H + kPerBlock - 1) / kPerBlock;
    const int t = blockIdx.x / per_token;
    const int obase = (blockIdx.x % per_token) * kPerBlock;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1), sub = lane % LPR;
    const int g = lane / LPR;
    const int o0 = obase + g * kRows;
    __shared__ float coef[kTmMaxK];       // w_s * s_down
    __shared__ int on_slot[kTmMaxK];      // 0: slot skipped
    const float* ht = a.h + int64_t(t) * K * I;
    // this wave's slots: ids, weights, block pointers and down scales all
    // requested before any of them is used (three short dependent rounds
    // for every slot at once instead of one chain per slot)
    constexpr int kSlots = KW;             // slots per wave: ceil(K / 4)
    int ev[kSlots];
    float rv[kSlots], sdv[kSlots];
    const uint8_t* bv[kSlots];
    bool onv[kSlots];
    // unconditional loads at clamped indices, masked afterwards: no branch
    // (and no wait) between the requests
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int s = wave + j * kWaves;
        const int64_t sc = int64_t(t) * K + (s < K ? s : K - 1);
        ev[j] = a.expert[sc];
        rv[j] = a.weight[sc];
    }
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int s = wave + j * kWaves;
        onv[j] = s < K && ev[j] >= 0 && ev[j] < a.E && rv[j] != 0.0f;
        bv[j] = a.eptr[onv[j] ? ev[j] : 0];
    }
#pragma unroll
    for (int j = 0; j < kSlots; ++j) sdv[j] = reinterpret_cast<const float*>(bv[j] + a.gsc)[2];
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int s = wave + j * kWaves;
        if (s < K && lane == 0) {
            coef[s] = onv[j] ? rv[j] * sdv[j] : 0.0f;
            on_slot[s] = onv[j] ? 1 : 0;
        }
    }
    // the dots: two slots at a time, every weight and h load of both issued
    // before either is used (a skipped slot reads a valid block, masked)
    float acc[kSlots][kRows];
#pragma unroll
    for (int j = 0; j < kSlots; ++j)
#pragma unroll
        for (int r = 0; r < kRows; ++r) acc[j][r] = 0.0f;
    constexpr int kPair = kSlots < 2 ? 1 : 2;
    for (int c = sub; c < I / 32; c += LPR) {
#pragma unroll
        for (int j0 = 0; j0 < kSlots; j0 += kPair) {
            uint4 pv[kPair][kRows];
            uint32_t s2[kPair][kRows];
            float hx[kPair][32];
#pragma unroll
            for (int jj = 0; jj < kPair; ++jj) {
                const int j = j0 + jj;
                const int s = wave + j * kWaves;
                const int sc = s < K ? s : K - 1;
#pragma unroll
                for (int r = 0; r < kRows; ++r) {
                    const int o = o0 + r < H ? o0 + r : H - 1;
                    pv[jj][r] = *reinterpret_cast<const uint4*>(bv[j] + a.dn_p + int64_t(o) * (I / 2) + c * 16);
                    s2[jj][r] = load_s2(bv[j] + a.dn_s + int64_t(o) * (I / 16) + c * 2);
                }
                load_x32(ht + sc * I + c * 32, hx[jj]);
            }
#pragma unroll
            for (int jj = 0; jj < kPair; ++jj)
#pragma unroll
                for (int r = 0; r < kRows; ++r) {
                    const float d = nv_dot32(pv[jj][r], s2[jj][r], hx[jj]);
                    acc[j0 + jj][r] += onv[j0 + jj] ? d : 0.0f;
                }
        }
    }
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
        const int s = wave + j * kWaves;
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const float d = group_sum<LPR>(acc[j][r]);
            if (onv[j] && sub == 0) part[s][g * kRows + r] = d;
        }
    }
    __syncthreads();
    const int row = threadIdx.x;
    if (row < kPerBlock && obase + row < H) {
        float total = 0.0f;
        for (int s = 0; s < K; ++s) {
            if (on_slot[s]) total = __builtin_fmaf(coef[s], part[s][row], total);
        }
        a.y[int64_t(t) * H + obase + row] = total;
    }
}

// Prefill on one expert block: the block's NVFP4 rows decoded into bf16
// scratch rows (exact: an e2m1 value times an E4M3 scale has at most 6
// significant bits), which the grouped bf16 GEMM then reads; the fp32
// projection scales are applied to the GEMM's fp32 output, as the
// reference's launch_nvfp4_expert_gemm does (tiered_moe.hpp:83-93).
__global__ __launch_bounds__(kTmThreads) void nvfp4_to_bf16(const uint8_t* __restrict__ pay,
                                                            const uint8_t* __restrict__ sc,
                                                            int N, int K,
                                                            uint16_t* __restrict__ out) {
    // one thread per 32-element chunk: 16 payload bytes, two scale bytes
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int cpr = K / 32;
    if (i >= int64_t(N) * cpr) return;
    const int n = int(i / cpr), c = int(i % cpr);
    const uint4 p = *reinterpret_cast<const uint4*>(pay + int64_t(n) * (K / 2) + c * 16);
    const uint32_t s2 = load_s2(sc + int64_t(n) * (K / 16) + c * 2);
    const float b0 = e4m3_f32(s2 & 0xFFu), b1 = e4m3_f32((s2 >> 8) & 0xFFu);
    const uint32_t w[4] = {p.x, p.y, p.z, p.w};
    uint32_t o[16];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const f32x2 v[4] = {__builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 0),
                            __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 1),
                            __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 2),
                            __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w[d], 1.0f, 3)};
        const float bs = d < 2 ? b0 : b1;
#pragma unroll
        for (int b = 0; b < 4; ++b)
            o[4 * d + b] = uint32_t(f32_to_bf16(v[b].x * bs)) |
                           (uint32_t(f32_to_bf16(v[b].y * bs)) << 16);
    }
    uint4* dst = reinterpret_cast<uint4*>(out + int64_t(n) * K + c * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) dst[q] = make_uint4(o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]);
}

// out[m][n] *= (n < split ? s0 : s1) over [M][N]
__global__ __launch_bounds__(kTmThreads) void scale_cols(float* __restrict__ out, int64_t total,
                                                         int N, int split, float s0, float s1) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += int64_t(gridDim.x) * blockDim.x)
        out[i] *= (int(i % N) < split ? s0 : s1);
}

// h[m][i] = bf16(silu(s_g * gu[m][i]) * (s_u * gu[m][I + i]))
__global__ __launch_bounds__(kTmThreads) void swiglu_bf16(const float* __restrict__ gu, int M,
                                                          int I, float sg, float su,
                                                          uint16_t* __restrict__ h) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < int64_t(M) * I;
         i += int64_t(gridDim.x) * blockDim.x) {
        const int64_t m = i / I, c = i % I;
        const float g = gu[m * 2 * I + c] * sg, u = gu[m * 2 * I + I + c] * su;
        h[i] = f32_to_bf16(silu(g) * u);
    }
}

__global__ void set_rows(int32_t* cnt_off, int M) {
    if (threadIdx.x == 0) { cnt_off[0] = M; cnt_off[1] = 0; }
}

static unsigned ew_blocks(int64_t n) {
    const int64_t b = (n + kTmThreads - 1) / kTmThreads;
    return unsigned(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

hipError_t tmoe_decode_bf16(hipStream_t st, const uint8_t* pay, const uint8_t* sc, int N, int K,
                            uint16_t* out) {
    const int64_t items = int64_t(N) * (K / 32);
    hipLaunchKernelGGL(nvfp4_to_bf16, dim3(unsigned((items + kTmThreads - 1) / kTmThreads)),
                       dim3(kTmThreads), 0, st, pay, sc, N, K, out);
    return hipGetLastError();
}

hipError_t tmoe_scale_cols(hipStream_t st, float* out, int M, int N, int split, float s0, float s1) {
    hipLaunchKernelGGL(scale_cols, dim3(ew_blocks(int64_t(M) * N)), dim3(kTmThreads), 0, st, out,
                       int64_t(M) * N, N, split, s0, s1);
    return hipGetLastError();
}

hipError_t tmoe_swiglu(hipStream_t st, const float* gu, int M, int I, float sg, float su,
                       uint16_t* h) {
    hipLaunchKernelGGL(swiglu_bf16, dim3(ew_blocks(int64_t(M) * I)), dim3(kTmThreads), 0, st, gu,
                       M, I, sg, su, h);
    return hipGetLastError();
}

hipError_t tmoe_set_rows(hipStream_t st, int32_t* cnt_off, int M) {
    hipLaunchKernelGGL(set_rows, dim3(1), dim3(kWave), 0, st, cnt_off, M);
    return hipGetLastError();
}

__global__ void tmoe_store_ptr(const uint8_t** table, int e, const uint8_t* p) {
    if (threadIdx.x == 0) table[e] = p;
}

static int lanes_for(int chunks) {
    int l = 1;
    while (l < chunks && l < kWave) l *= 2;
    return l;
}

#define GRIM_TM_LAUNCH(KERNEL, LPR_VAL, GRID)                                                      \
    hipLaunchKernelGGL((KERNEL<LPR_VAL>), GRID, dim3(kTmThreads), 0, st, a)

#define GRIM_TM_SWITCH(KERNEL, LPR, GRID)                                                          \
    switch (LPR) {                                                                                 \
        case 1: GRIM_TM_LAUNCH(KERNEL, 1, GRID); break;                                            \
        case 2: GRIM_TM_LAUNCH(KERNEL, 2, GRID); break;                                            \
        case 4: GRIM_TM_LAUNCH(KERNEL, 4, GRID); break;                                            \
        case 8: GRIM_TM_LAUNCH(KERNEL, 8, GRID); break;                                            \
        case 16: GRIM_TM_LAUNCH(KERNEL, 16, GRID); break;                                          \
        case 32: GRIM_TM_LAUNCH(KERNEL, 32, GRID); break;                                          \
        default: GRIM_TM_LAUNCH(KERNEL, 64, GRID); break;                                          \
    }

hipError_t tmoe_gate_up(hipStream_t st, const TmoeArgs& a) {
    if (a.M <= 0) return hipSuccess;
    const int lpr = lanes_for(a.H / 32);
    const int per_block = (kTmThreads / kWave) * (kWave / lpr) * 2;
    const dim3 grid(unsigned(int64_t(a.M) * ((a.K * a.I + per_block - 1) / per_block)));
    GRIM_TM_SWITCH(tmoe_gate_up_kernel, lpr, grid);
    return hipGetLastError();
}

#define GRIM_TMD_LAUNCH(LPR_VAL, KW_VAL)                                                            \
    hipLaunchKernelGGL((tmoe_down_kernel<LPR_VAL, KW_VAL>), grid, dim3(kTmThreads), 0, st, a)
#define GRIM_TMD_KW(LPR_VAL)                                                                        \
    switch (kw) {                                                                                  \
        case 1: GRIM_TMD_LAUNCH(LPR_VAL, 1); break;                                                \
        case 2: GRIM_TMD_LAUNCH(LPR_VAL, 2); break;                                                \
        case 4: GRIM_TMD_LAUNCH(LPR_VAL, 4); break;                                                \
        default: GRIM_TMD_LAUNCH(LPR_VAL, 8); break;                                               \
    }

hipError_t tmoe_down(hipStream_t st, const TmoeArgs& a) {
    if (a.M <= 0) return hipSuccess;
    if (a.K > kTmMaxK) return hipErrorInvalidValue;
    const int lpr = lanes_for(a.I / 32);
    const int per_block = (kWave / lpr) * 2;
    const dim3 grid(unsigned(int64_t(a.M) * ((a.H + per_block - 1) / per_block)));
    const int need = (a.K + kTmThreads / kWave - 1) / (kTmThreads / kWave);
    const int kw = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8;
    switch (lpr) {
        case 1: GRIM_TMD_KW(1); break;
        case 2: GRIM_TMD_KW(2); break;
        case 4: GRIM_TMD_KW(4); break;
        case 8: GRIM_TMD_KW(8); break;
        case 16: GRIM_TMD_KW(16); break;
        case 32: GRIM_TMD_KW(32); break;
        default: GRIM_TMD_KW(64); break;
    }
    return hipGetLastError();
}

hipError_t tmoe_store(hipStream_t st, const uint8_t** table, int e, const uint8_t* p) {
    hipLaunchKernelGGL(tmoe_store_ptr, dim3(1), dim3(kWave), 0, st, table, e, p);
    return hipGetLastError();
}

}  // namespace grim
