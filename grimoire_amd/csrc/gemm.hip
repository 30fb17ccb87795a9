// gemm.hip -- grouped expert GEMM on CDNA4 MFMA (prefill regime).
//
// One launch per projection for all experts (the reference's design,
// src/gemm_fast.cpp:1603-1800, src/prefill.cpp:2726-2808), written for
// gfx950:
//   - block tile 128 rows x 128 columns x 64 K, 256 threads (4 waves), each
//     wave a 64x64 quadrant as 2x2 v_mfma_f32_32x32x16_bf16 tiles;
//   - weight tiles are dequantised ONCE per block into LDS as bf16 that
//     equals the stored weight exactly (int8 codes; e2m1 x e8m0 through the
//     CDNA4 fp4 converter; bf16 copies); per-output-channel scales (int8)
//     are applied to the fp32 accumulators in the epilogue, so the MFMA
//     operands are exact;
//   - two LDS stages: the next K tile's global loads are in flight while
//     the current one is multiplied; one barrier per K tile;
//   - rows come from the dispatch's (expert, m-tile) table (padding entries
//     -1 exit at once), the shared expert as extra tiles after it.
// Epilogues: SwiGLU (gate and up columns of the same h column live in the
// same lane) writing h as a bf16 pair hi + lo (|lo| <= 2^-9 |h|, so h is
// kept to ~2^-17 relative), or plain fp32 / bf16 output.  The down
// projection consumes the pair as two MFMA passes against the same B.
#include "common.hpp"
#include "gemm.hpp"

namespace grim {

typedef __bf16 bf16x8 __attribute__((__vector_size__(8 * sizeof(__bf16))));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDK = BK + 8;         // LDS row stride in bf16 (144 bytes)
constexpr int kGemmThreads = 256;

template <int F> struct BTile;
template <> struct BTile<GRIM_FMT_INT8> { static constexpr int CPR = 4; };   // 16B chunks per row
template <> struct BTile<GRIM_FMT_MXFP4> { static constexpr int CPR = 2; };
template <> struct BTile<GRIM_FMT_BF16> { static constexpr int CPR = 8; };

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    // exact conversions only (values representable in bf16): truncate
    return (f_bits(a) >> 16) | (f_bits(b) & 0xFFFF0000u);
}

// Dequantise one 16-byte chunk of B into LDS row `dst` (bf16 elements).
template <int F>
__device__ __forceinline__ void store_b_chunk(const u32x4 raw, uint8_t sc, uint16_t* dst);

template <>
__device__ __forceinline__ void store_b_chunk<GRIM_FMT_INT8>(const u32x4 raw, uint8_t,
                                                             uint16_t* dst) {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    uint32_t o[8];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const float f0 = float(int8_t(w[d] & 0xFF)), f1 = float(int8_t((w[d] >> 8) & 0xFF));
        const float f2 = float(int8_t((w[d] >> 16) & 0xFF)), f3 = float(int8_t(w[d] >> 24));
        o[2 * d] = pack_bf16(f0, f1);
        o[2 * d + 1] = pack_bf16(f2, f3);
    }
    u32x4* p = reinterpret_cast<u32x4*>(dst);
    p[0] = u32x4{o[0], o[1], o[2], o[3]};
    p[1] = u32x4{o[4], o[5], o[6], o[7]};
}

template <>
__device__ __forceinline__ void store_b_chunk<GRIM_FMT_MXFP4>(const u32x4 raw, uint8_t sc,
                                                              uint16_t* dst) {
    const float s = e8m0_to_f32(sc);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    uint32_t o[16];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const bf16x2v v0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], s, 0);
        const bf16x2v v1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], s, 1);
        const bf16x2v v2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], s, 2);
        const bf16x2v v3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], s, 3);
        __builtin_memcpy(&o[4 * d + 0], &v0, 4);
        __builtin_memcpy(&o[4 * d + 1], &v1, 4);
        __builtin_memcpy(&o[4 * d + 2], &v2, 4);
        __builtin_memcpy(&o[4 * d + 3], &v3, 4);
    }
    u32x4* p = reinterpret_cast<u32x4*>(dst);
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
}

template <>
__device__ __forceinline__ void store_b_chunk<GRIM_FMT_BF16>(const u32x4 raw, uint8_t,
                                                             uint16_t* dst) {
    *reinterpret_cast<u32x4*>(dst) = raw;
}

template <int F>
__device__ __forceinline__ float col_scale(const WView& w, int64_t row) {
    if constexpr (F == GRIM_FMT_INT8) return static_cast<const float*>(w.scales)[row];
    return 1.0f;
}

// One (m-tile, column-tile) of the grouped product.
template <int F, bool SWIGLU, bool APAIR, bool OUT_BF16>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, int ty, int n_routed,
                                          uint16_t (*As)[APAIR ? 2 : 1][BM * LDK],
                                          uint16_t (*Bs)[BN * LDK]) {
    constexpr int CPR = BTile<F>::CPR;
    constexpr int CH = BK / CPR;              // elements per B chunk
    constexpr int NBCH = BN * CPR / kGemmThreads;   // B chunks per thread (>= 1)
    static_assert(BN * CPR % kGemmThreads == 0, "B chunk split");

    // ---- which rows / weights
    int e, rows_valid;
    int64_t arow0;
    const uint16_t* A;
    WView w;
    void* out;
    int64_t wrow0;
    if (ty < n_routed) {
        e = g.tile_e[ty];
        if (e < 0) return;
        const int mb = g.tile_mb[ty];
        rows_valid = min(BM, g.counts[e] - mb * BM);
        arow0 = int64_t(g.offsets[e]) + int64_t(mb) * BM;
        A = g.A;
        w = g.w;
        out = g.out;
        wrow0 = int64_t(e) * g.N;
    } else {
        const int mb = ty - n_routed;
        rows_valid = min(BM, g.T_sh - mb * BM);
        arow0 = int64_t(mb) * BM;
        A = g.A_sh;
        w = g.w_sh;
        out = g.out_sh;
        wrow0 = 0;
    }
    if (rows_valid <= 0) return;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int K = g.K;
    const int64_t a_stride = APAIR ? 2 * int64_t(K) : int64_t(K);

    // B rows of this tile: SwiGLU: 64 gate cols then the 64 matching up cols
    const int nt = blockIdx.x;
    auto b_row = [&](int n) -> int64_t {
        int c;
        if (SWIGLU) {
            const int hc = min(nt * 64 + (n & 63), g.I - 1);
            c = n < 64 ? hc : g.I + hc;
        } else {
            c = min(nt * BN + n, g.N - 1);
        }
        return wrow0 + c;
    };

    // ---- global -> register staging
    u32x4 ra[APAIR ? 2 : 1][4];
    u32x4 rb[NBCH];
    uint8_t rs[NBCH];
    int64_t browv[NBCH];
#pragma unroll
    for (int i = 0; i < NBCH; ++i) browv[i] = b_row((tid + i * kGemmThreads) / CPR);

    auto load_tile = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + i * kGemmThreads;   // 1024 chunks of 8 bf16
            const int r = c >> 3, kc = (c & 7) * 8;
            const int rr = r < rows_valid ? r : rows_valid - 1;
            const uint16_t* p = A + (arow0 + rr) * a_stride + k0 + kc;
            ra[0][i] = *reinterpret_cast<const u32x4*>(p);
            if constexpr (APAIR) ra[1][i] = *reinterpret_cast<const u32x4*>(p + K);
        }
#pragma unroll
        for (int i = 0; i < NBCH; ++i) {
            const int c = tid + i * kGemmThreads;
            const int kc = (c % CPR) * CH;
            const int64_t byte_off =
                F == GRIM_FMT_MXFP4 ? (k0 + kc) / 2 : (F == GRIM_FMT_BF16 ? (k0 + kc) * 2 : k0 + kc);
            rb[i] = load16(w.payload + browv[i] * w.row_bytes + byte_off);
            if constexpr (F == GRIM_FMT_MXFP4)
                rs[i] = static_cast<const uint8_t*>(w.scales)[browv[i] * w.row_scales + (k0 + kc) / 32];
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + i * kGemmThreads;
            const int r = c >> 3, kc = (c & 7) * 8;
            const bool ok = r < rows_valid;
            const u32x4 z = {0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4*>(&As[buf][0][r * LDK + kc]) = ok ? ra[0][i] : z;
            if constexpr (APAIR)
                *reinterpret_cast<u32x4*>(&As[buf][1][r * LDK + kc]) = ok ? ra[1][i] : z;
        }
#pragma unroll
        for (int i = 0; i < NBCH; ++i) {
            const int c = tid + i * kGemmThreads;
            const int n = c / CPR, kc = (c % CPR) * CH;
            store_b_chunk<F>(rb[i], F == GRIM_FMT_MXFP4 ? rs[i] : 0, &Bs[buf][n * LDK + kc]);
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[mi][ni][v] = 0.0f;

    // column offsets (tile-local) of this wave's two 32-column B fragments
    const int ncol0 = SWIGLU ? wn * 32 : wn * 64;
    const int ncol1 = SWIGLU ? 64 + wn * 32 : wn * 64 + 32;

    const int nk = K / BK;
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_tile((kt + 1) * BK);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int kk = ks * 16 + 8 * (lane >> 5);
            bf16x8 a[APAIR ? 2 : 1][2], b[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                const int r = wm * 64 + mi * 32 + (lane & 31);
                a[0][mi] = *reinterpret_cast<const bf16x8*>(&As[buf][0][r * LDK + kk]);
                if constexpr (APAIR) a[1][mi] = *reinterpret_cast<const bf16x8*>(&As[buf][1][r * LDK + kk]);
            }
            b[0] = *reinterpret_cast<const bf16x8*>(&Bs[buf][(ncol0 + (lane & 31)) * LDK + kk]);
            b[1] = *reinterpret_cast<const bf16x8*>(&Bs[buf][(ncol1 + (lane & 31)) * LDK + kk]);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni) {
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0][mi], b[ni], acc[mi][ni], 0, 0, 0);
                    if constexpr (APAIR)
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1][mi], b[ni], acc[mi][ni], 0, 0, 0);
                }
        }
        if (kt + 1 < nk) store_tile(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue.  acc[mi][ni][v]: row = wm*64 + mi*32 + (v&3) + 4*(lane>>5)
    // + 8*(v>>2), column = ncol(ni) + (lane&31).
    const int lc = lane & 31;
    if constexpr (SWIGLU) {
        const int hc = nt * 64 + wn * 32 + lc;
        if (hc < g.I) {
            const float sg = col_scale<F>(w, wrow0 + hc);
            const float su = col_scale<F>(w, wrow0 + g.I + hc);
            uint16_t* o = static_cast<uint16_t*>(out);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = wm * 64 + mi * 32 + (v & 3) + 4 * (lane >> 5) + 8 * (v >> 2);
                    if (r < rows_valid) {
                        const float hv = silu(acc[mi][0][v] * sg) * (acc[mi][1][v] * su);
                        const uint16_t hi = f32_to_bf16(hv);
                        const uint16_t lo = f32_to_bf16(hv - bf16_to_f32(hi));
                        const int64_t base = (arow0 + r) * 2 * int64_t(g.I);
                        o[base + hc] = hi;
                        o[base + g.I + hc] = lo;
                    }
                }
        }
    } else {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const int c = nt * BN + (ni ? ncol1 : ncol0) + lc;
            if (c >= g.N) continue;
            const float sc = col_scale<F>(w, wrow0 + c);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = wm * 64 + mi * 32 + (v & 3) + 4 * (lane >> 5) + 8 * (v >> 2);
                    if (r < rows_valid) {
                        const float val = acc[mi][ni][v] * sc;
                        const int64_t idx = (arow0 + r) * int64_t(g.N) + c;
                        if constexpr (OUT_BF16) static_cast<uint16_t*>(out)[idx] = f32_to_bf16(val);
                        else static_cast<float*>(out)[idx] = val;
                    }
                }
        }
    }
}

// Grid: x = column tile; y strides over the m-tile entries: the routed
// table (its live length read from the device), then the shared expert's.
template <int F, bool SWIGLU, bool APAIR, bool OUT_BF16>
__global__ __launch_bounds__(kGemmThreads, 2) void grouped_gemm_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(16))) uint16_t As[2][APAIR ? 2 : 1][BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDK];
    int n_routed = g.n_tiles_dev ? *g.n_tiles_dev : g.tmax;
    n_routed = n_routed < g.tmax ? n_routed : g.tmax;
    const int total = n_routed + (g.T_sh > 0 ? (g.T_sh + BM - 1) / BM : 0);
    for (int ty = blockIdx.y; ty < total; ty += gridDim.y) {
        gemm_tile<F, SWIGLU, APAIR, OUT_BF16>(g, ty, n_routed, As, Bs);
        __syncthreads();
    }
}

template <int F>
static hipError_t launch_fmt(hipStream_t st, const GemmArgs& g) {
    const int ntiles = g.swiglu ? (g.I + 63) / 64 : (g.N + BN - 1) / BN;
    const int my_max = g.tmax + (g.T_sh > 0 ? (g.T_sh + BM - 1) / BM : 0);
    if (my_max <= 0 || ntiles <= 0) return hipSuccess;
    // about four resident blocks per CU over the whole grid
    int my = (4 * 256 + ntiles - 1) / ntiles;
    my = my < my_max ? my : my_max;
    dim3 grid(ntiles, my);
    if (g.swiglu) {
        hipLaunchKernelGGL((grouped_gemm_kernel<F, true, false, false>), grid, dim3(kGemmThreads), 0,
                           st, g);
    } else if (g.a_pair) {
        if (g.out_bf16)
            hipLaunchKernelGGL((grouped_gemm_kernel<F, false, true, true>), grid, dim3(kGemmThreads),
                               0, st, g);
        else
            hipLaunchKernelGGL((grouped_gemm_kernel<F, false, true, false>), grid, dim3(kGemmThreads),
                               0, st, g);
    } else {
        if (g.out_bf16)
            hipLaunchKernelGGL((grouped_gemm_kernel<F, false, false, true>), grid, dim3(kGemmThreads),
                               0, st, g);
        else
            hipLaunchKernelGGL((grouped_gemm_kernel<F, false, false, false>), grid,
                               dim3(kGemmThreads), 0, st, g);
    }
    return hipGetLastError();
}

bool gemm_format_ok(int fmt) {
    return fmt == GRIM_FMT_INT8 || fmt == GRIM_FMT_MXFP4 || fmt == GRIM_FMT_BF16;
}

hipError_t gemm_launch(hipStream_t st, int fmt, const GemmArgs& g) {
    switch (fmt) {
    case GRIM_FMT_INT8: return launch_fmt<GRIM_FMT_INT8>(st, g);
    case GRIM_FMT_MXFP4: return launch_fmt<GRIM_FMT_MXFP4>(st, g);
    case GRIM_FMT_BF16: return launch_fmt<GRIM_FMT_BF16>(st, g);
    }
    return hipErrorInvalidValue;
}

}  // namespace grim
