// gemm.hip -- grouped expert GEMM on CDNA4 MFMA (prefill regime).
//
// One launch per projection for all experts (the reference's design,
// src/gemm_fast.cpp:1603-1800, src/prefill.cpp:2726-2808), written for
// gfx950:
//   - block tile 128 rows x 256 columns x 64 K, 256 threads (4 waves), each
//     wave all 128 rows of its own 64 columns as 4x2
//     v_mfma_f32_32x32x16_bf16 tiles (each weight column is dequantised by
//     one wave only; 0.5 KB of LDS reads per MFMA);
//   - A (activation rows) is staged through LDS (double buffer, register
//     prefetch two K tiles deep); B (weights) never touches LDS: each lane
//     loads the 32 K-values of the weight column it multiplies straight into
//     registers and dequantises them there to bf16 that equals the stored
//     weight exactly (int8 codes; e2m1 x e8m0 through the CDNA4 fp4
//     converter; bf16 copies).  LDS traffic is A alone, which is what bounds
//     this loop.  Per-output-channel scales (int8) are applied to the fp32
//     accumulators in the epilogue, so the MFMA operands are exact;
//   - K loop barriers wait for LDS only, never for the prefetched loads;
//   - persistent XCD-aware grid over (m-tile, column tile) items, rows from
//     the dispatch's (expert, m-tile) table (padding entries -1 skip), the
//     shared expert's tiles after it.
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

constexpr int BM = 128, BN = 256, BK = 64;
constexpr int LDK = BK + 8;         // LDS row stride in bf16 (144 bytes)
constexpr int kGemmThreads = 256;
#ifndef GRIM_GEMM_OCC
#define GRIM_GEMM_OCC 1
#endif


// Work-group barrier for LDS hand-offs only: waits for this wave's LDS
// accesses, not for its global loads (a __syncthreads() fence would also
// wait for the prefetched tiles still in flight).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    // exact conversions only (values representable in bf16): truncate
    return (f_bits(a) >> 16) | (f_bits(b) & 0xFFFF0000u);
}

// MFMA B fragment (8 bf16, exact) for step ks from a lane's 32 K-values of
// one weight column: INT8 bytes 8ks..8ks+7; MXFP4 nibbles 8ks..8ks+7
// (low nibble = even K) times the group's e8m0 scale; BF16 elements
// 8ks..8ks+7.
template <int F, int BQ>
__device__ __forceinline__ bf16x8 b_frag(const u32x4 (&raw)[BQ], uint32_t sc, int ks);

template <>
__device__ __forceinline__ bf16x8 b_frag<GRIM_FMT_INT8, 2>(const u32x4 (&raw)[2], uint32_t, int ks) {
    const u32x4 q = raw[ks >> 1];
    const uint32_t w0 = (ks & 1) ? q.z : q.x, w1 = (ks & 1) ? q.w : q.y;
    uint32_t o[4];
    const uint32_t w[2] = {w0, w1};
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const float f0 = float(int8_t(w[d] & 0xFF)), f1 = float(int8_t((w[d] >> 8) & 0xFF));
        const float f2 = float(int8_t((w[d] >> 16) & 0xFF)), f3 = float(int8_t(w[d] >> 24));
        o[2 * d] = pack_bf16(f0, f1);
        o[2 * d + 1] = pack_bf16(f2, f3);
    }
    bf16x8 r;
    __builtin_memcpy(&r, o, 16);
    return r;
}

template <>
__device__ __forceinline__ bf16x8 b_frag<GRIM_FMT_MXFP4, 1>(const u32x4 (&raw)[1], uint32_t sc, int ks) {
    const float s = e8m0_to_f32(uint8_t(sc));
    const uint32_t wd = ks == 0 ? raw[0].x : ks == 1 ? raw[0].y : ks == 2 ? raw[0].z : raw[0].w;
    const bf16x2v v0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 0);
    const bf16x2v v1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 1);
    const bf16x2v v2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 2);
    const bf16x2v v3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd, s, 3);
    uint32_t o[4];
    __builtin_memcpy(&o[0], &v0, 4);
    __builtin_memcpy(&o[1], &v1, 4);
    __builtin_memcpy(&o[2], &v2, 4);
    __builtin_memcpy(&o[3], &v3, 4);
    bf16x8 r;
    __builtin_memcpy(&r, o, 16);
    return r;
}

template <>
__device__ __forceinline__ bf16x8 b_frag<GRIM_FMT_BF16, 4>(const u32x4 (&raw)[4], uint32_t, int ks) {
    bf16x8 r;
    __builtin_memcpy(&r, &raw[ks], 16);
    return r;
}

template <>
__device__ __forceinline__ bf16x8 b_frag<kGemmFmtS4, 1>(const u32x4 (&raw)[1], uint32_t, int ks) {
    const uint32_t wd = ks == 0 ? raw[0].x : ks == 1 ? raw[0].y : ks == 2 ? raw[0].z : raw[0].w;
    uint32_t o[4];
    // (the sbfe builtin is typed unsigned: convert its sign-extended result as int)
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const float f0 = float(int(__builtin_amdgcn_sbfe(int(wd), 8 * d, 4)));       // even K
        const float f1 = float(int(__builtin_amdgcn_sbfe(int(wd), 8 * d + 4, 4)));   // odd K
        o[d] = pack_bf16(f0, f1);
    }
    bf16x8 r;
    __builtin_memcpy(&r, o, 16);
    return r;
}

// The operands of one launch (routed experts, or the shared expert): chosen
// once per launch so that only one set of pointers is live.
struct GemmSrc {
    const uint8_t* payload;
    const void* scales;
    int64_t row_bytes;
    int row_scales;
    const uint16_t* A;
    void* out;
};

template <int F>
__device__ __forceinline__ float col_scale(const GemmSrc& w, int64_t row) {
    if constexpr (F == GRIM_FMT_INT8) return static_cast<const float*>(w.scales)[row];
    return 1.0f;
}

// One (m-tile, column-tile) of the grouped product.
// Rows mode: tp[e] = m-tiles of the experts before e, rp[e] = their rows
// (tp[ne], rp[ne] the totals), from rows_per_expert (negative = 0).
__device__ __forceinline__ int rows_tables(const int* __restrict__ rows, int ne, int* tp, int* rp) {
    constexpr int PER = kGemmRowsMaxExperts / kGemmThreads;
    __shared__ int st[kGemmThreads], sr[kGemmThreads];
    const int tid = threadIdx.x;
    int c[PER], ts = 0, rs = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = tid * PER + j;
        const int v = e < ne ? rows[e] : 0;
        c[j] = v > 0 ? v : 0;
        ts += (c[j] + BM - 1) / BM;
        rs += c[j];
    }
    st[tid] = ts;
    sr[tid] = rs;
    __syncthreads();
    for (int d = 1; d < kGemmThreads; d <<= 1) {   // inclusive scan
        const int a = tid >= d ? st[tid - d] : 0, b = tid >= d ? sr[tid - d] : 0;
        __syncthreads();
        st[tid] += a;
        sr[tid] += b;
        __syncthreads();
    }
    int t0 = st[tid] - ts, r0 = sr[tid] - rs;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = tid * PER + j;
        if (e <= ne) { tp[e] = t0; rp[e] = r0; }
        t0 += (c[j] + BM - 1) / BM;
        r0 += c[j];
    }
    const int total = st[kGemmThreads - 1];
    if (tid == kGemmThreads - 1) { tp[ne] = total; rp[ne] = sr[kGemmThreads - 1]; }
    __syncthreads();
    return total;
}

template <int F, bool SWIGLU, bool APAIR, bool OUT_BF16>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, const GemmSrc& w, bool routed, int ty,
                                          int nt, uint16_t (*As)[APAIR ? 2 : 1][BM * LDK],
                                          const int* tp, const int* rp) {
    // ---- which rows / weights
    int rows_valid;
    int64_t arow0, wrow0;
    if (routed && g.rows) {
        // the expert whose m-tiles hold tile ty: last e with tp[e] <= ty
        int lo = 0, hi = g.ne - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (tp[mid] <= ty) lo = mid; else hi = mid - 1;
        }
        const int e = __builtin_amdgcn_readfirstlane(lo);
        const int mb = ty - tp[e];
        rows_valid = min(BM, (rp[e + 1] - rp[e]) - mb * BM);
        const int off = g.offsets ? __builtin_amdgcn_readfirstlane(g.offsets[e]) : rp[e];
        arow0 = int64_t(off) + int64_t(mb) * BM;
        wrow0 = int64_t(e) * g.N;
    } else if (routed) {
        // table values are the same for the whole work-group: keep them in
        // scalar registers (buffer descriptors built from them must be)
        const int e = __builtin_amdgcn_readfirstlane(g.tile_e[ty]);
        if (e < 0) return;
        const int mb = __builtin_amdgcn_readfirstlane(g.tile_mb[ty]);
        rows_valid = min(BM, __builtin_amdgcn_readfirstlane(g.counts[e]) - mb * BM);
        arow0 = int64_t(__builtin_amdgcn_readfirstlane(g.offsets[e])) + int64_t(mb) * BM;
        wrow0 = int64_t(e) * g.N;
    } else {
        const int mb = ty;
        rows_valid = min(BM, g.T_sh - mb * BM);
        arow0 = int64_t(mb) * BM;
        wrow0 = 0;
    }
    // uniform per work-group: make that explicit, so descriptors and
    // offsets built from them stay in scalar registers
    rows_valid = __builtin_amdgcn_readfirstlane(rows_valid);
    arow0 = int64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(arow0)))) |
            (int64_t(__builtin_amdgcn_readfirstlane(int(arow0 >> 32))) << 32);
    wrow0 = int64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(wrow0)))) |
            (int64_t(__builtin_amdgcn_readfirstlane(int(wrow0 >> 32))) << 32);
    const uint16_t* A = w.A;
    void* out = w.out;
    if (rows_valid <= 0) return;

    // the thread id is laundered so that per-lane offsets are recomputed in
    // each tile instead of being hoisted out of the persistent loop (which
    // keeps dozens of them live across it and spills)
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, wave = tid >> 6;
    const int K = g.K;
    const int64_t a_stride = APAIR ? 2 * int64_t(K) : int64_t(K);

    // Each wave owns 64 output columns of the 256 (two 32-column MFMA
    // fragments) for all 128 rows: SwiGLU: the gate and the up column of
    // 32 h columns; else 64 consecutive columns.  Column of fragment ni for
    // this lane, and its weight row within the expert's slab:
    auto out_col = [&](int ni) -> int {
        if (SWIGLU) return nt * (BN / 2) + wave * 32 + (lane & 31);   // h column
        return nt * BN + wave * 64 + ni * 32 + (lane & 31);
    };
    auto b_row = [&](int ni) -> int {
        if (SWIGLU) {
            const int hc = min(out_col(ni), g.I - 1);
            return ni == 0 ? hc : g.I + hc;
        }
        return min(out_col(ni), g.N - 1);
    };

    // ---- A (activations) goes through LDS; B (weights) never does: each
    // lane loads the 32 K-values of its own weight column it multiplies and
    // dequantises them in registers, so LDS carries A only.  The K order
    // inside a 64-wide K tile is permuted consistently for A and B: in MFMA
    // step ks, lane half h supplies K = 32 h + 8 ks + [0, 8).
    //
    // Buffer loads off per-tile bases; A rows past rows_valid read as zero
    // (outside the buffer's range).
    const int a_row_bytes = int(a_stride) * 2;
    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(A + arow0 * a_stride), 0, rows_valid * a_row_bytes, 0x00020000);
    const int n_slab = SWIGLU ? 2 * g.I : g.N;
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(w.payload + wrow0 * w.row_bytes), 0, int(n_slab * w.row_bytes),
        0x00020000);
    // side scales: MXFP4 e8m0 bytes [N][K/32]; S4 bf16 [N][K/G]
    constexpr int SB = F == GRIM_FMT_MXFP4 ? 1 : (F == kGemmFmtS4 ? 2 : 0);   // bytes per scale
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(static_cast<const void*>(static_cast<const uint8_t*>(w.scales) +
                                                   wrow0 * w.row_scales * SB)),
        0, n_slab * w.row_scales * SB, 0x00020000);
    constexpr bool kGroupScaled = F == kGemmFmtS4;
    const int group = kGroupScaled ? K / w.row_scales : 64;   // K per scale group
    const int gk = group / BK;                                 // K tiles per group
    const int a_off0 = (tid >> 3) * a_row_bytes + (tid & 7) * 16;   // + 32 rows per chunk
    const int h = lane >> 5;
    constexpr int BQ = F == GRIM_FMT_BF16 ? 4 : (F == GRIM_FMT_INT8 ? 2 : 1);   // 16-B loads per lane per column
    int b_off[2], s_off[2];
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
        const int n = b_row(ni);
        const int kb = 32 * h;   // first K of this lane inside a K tile
        b_off[ni] = n * int(w.row_bytes) +
                    (F == GRIM_FMT_MXFP4 || F == kGemmFmtS4 ? kb / 2 : (F == GRIM_FMT_BF16 ? kb * 2 : kb));
        s_off[ni] = F == kGemmFmtS4 ? n * w.row_scales * 2 : n * w.row_scales + h;
    }

    struct StageA { u32x4 a[APAIR ? 2 : 1][4]; };
    struct StageB { u32x4 b[2][BQ]; uint32_t s[2]; };
#define GRIM_LOAD_A(R, k0)                                                                      \
    do {                                                                                        \
        const int kb_ = (k0) * 2;                                                               \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                         \
            (R).a[0][i] = __builtin_amdgcn_raw_buffer_load_b128(rA, a_off0 + 32 * i * a_row_bytes, kb_, 0); \
            if constexpr (APAIR)                                                                \
                (R).a[1][i] = __builtin_amdgcn_raw_buffer_load_b128(rA, a_off0 + 32 * i * a_row_bytes, \
                                                                    kb_ + 2 * K, 0);            \
        }                                                                                       \
    } while (0)
#define GRIM_LOAD_B(R, k0)                                                                      \
    do {                                                                                        \
        const int kw_ = F == GRIM_FMT_MXFP4 || F == kGemmFmtS4 ? (k0) / 2                      \
                        : (F == GRIM_FMT_BF16 ? (k0) * 2 : (k0));                               \
        _Pragma("unroll") for (int ni = 0; ni < 2; ++ni) {                                      \
            _Pragma("unroll") for (int q = 0; q < BQ; ++q)                                      \
                (R).b[ni][q] = __builtin_amdgcn_raw_buffer_load_b128(rB, b_off[ni] + 16 * q, kw_, 0); \
            if constexpr (F == GRIM_FMT_MXFP4)                                                  \
                (R).s[ni] = __builtin_amdgcn_raw_buffer_load_b8(rS, s_off[ni], (k0) / 32, 0);    \
            if constexpr (F == kGemmFmtS4)                                                      \
                (R).s[ni] = __builtin_amdgcn_raw_buffer_load_b16(rS, s_off[ni], ((k0) / group) * 2, 0); \
        }                                                                                       \
    } while (0)
#define GRIM_STORE_A(R, buf)                                                                    \
    do {                                                                                        \
        _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                         \
            const int c_ = tid + i * kGemmThreads;                                              \
            const int r_ = c_ >> 3, kc_ = (c_ & 7) * 8;                                         \
            *reinterpret_cast<u32x4*>(&As[buf][0][r_ * LDK + kc_]) = (R).a[0][i];               \
            if constexpr (APAIR) *reinterpret_cast<u32x4*>(&As[buf][1][r_ * LDK + kc_]) = (R).a[1][i]; \
        }                                                                                       \
    } while (0)

    // acc: the tile's sums.  Group-scaled formats multiply codes in gacc and
    // fold gacc x the group's per-column scale into acc after each group
    // (each lane's accumulators all belong to the two columns it owns).
    f32x16 acc[4][2], gacc[4][2];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                acc[mi][ni][v] = 0.0f;
                gacc[mi][ni][v] = 0.0f;
            }
    f32x16 (&mt)[4][2] = kGroupScaled ? gacc : acc;   // the MFMA target

// A fragments of step ks are read from LDS while step ks - 1 multiplies
// (two fragment sets), so LDS latency hides behind the MFMAs.
#define GRIM_READ_A(dst, buf, ks)                                                               \
    _Pragma("unroll") for (int mi = 0; mi < 4; ++mi) {                                          \
        const int r_ = mi * 32 + (lane & 31), kk_ = 32 * h + 8 * (ks);                          \
        dst[0][mi] = *reinterpret_cast<const bf16x8*>(&As[buf][0][r_ * LDK + kk_]);             \
        if constexpr (APAIR) dst[1][mi] = *reinterpret_cast<const bf16x8*>(&As[buf][1][r_ * LDK + kk_]); \
    }
#define GRIM_MMA_TILE(buf, RB)                                                                  \
    do {                                                                                        \
        bf16x8 fa0[APAIR ? 2 : 1][4], fa1[APAIR ? 2 : 1][4], fb0[2], fb1[2];                    \
        GRIM_READ_A(fa0, buf, 0);                                                               \
        _Pragma("unroll") for (int ni = 0; ni < 2; ++ni) fb0[ni] = b_frag<F>((RB).b[ni], (RB).s[ni], 0); \
        _Pragma("unroll") for (int ks = 0; ks < BK / 16; ++ks) {                                \
            if (ks + 1 < BK / 16) {                                                             \
                if (ks & 1) {                                                                   \
                    GRIM_READ_A(fa0, buf, ks + 1);                                              \
                    _Pragma("unroll") for (int ni = 0; ni < 2; ++ni)                            \
                        fb0[ni] = b_frag<F>((RB).b[ni], (RB).s[ni], ks + 1);                    \
                } else {                                                                        \
                    GRIM_READ_A(fa1, buf, ks + 1);                                              \
                    _Pragma("unroll") for (int ni = 0; ni < 2; ++ni)                            \
                        fb1[ni] = b_frag<F>((RB).b[ni], (RB).s[ni], ks + 1);                    \
                }                                                                               \
            }                                                                                   \
            _Pragma("unroll") for (int mi = 0; mi < 4; ++mi)                                    \
            _Pragma("unroll") for (int ni = 0; ni < 2; ++ni) {                                  \
                const bf16x8 bb = (ks & 1) ? fb1[ni] : fb0[ni];                                 \
                const bf16x8 ah = (ks & 1) ? fa1[0][mi] : fa0[0][mi];                           \
                mt[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bb, mt[mi][ni], 0, 0, 0);    \
                if constexpr (APAIR) {                                                          \
                    const bf16x8 al = (ks & 1) ? fa1[1][mi] : fa0[1][mi];                       \
                    mt[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bb, mt[mi][ni], 0, 0, 0); \
                }                                                                               \
            }                                                                                   \
            /* interleave: the next step's LDS reads and conversions between   */               \
            /* this step's MFMAs                                                */              \
            _Pragma("unroll") for (int j = 0; j < 8; ++j) {                                     \
                __builtin_amdgcn_sched_group_barrier(0x008, APAIR ? 2 : 1, 0);                  \
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                              \
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);                              \
            }                                                                                   \
        }                                                                                       \
    } while (0)

#define GRIM_FOLD(RB, t)                                                                        \
    do {                                                                                        \
        if constexpr (kGroupScaled) {                                                           \
            if (((t) + 1) % gk == 0) {                                                          \
                _Pragma("unroll") for (int ni = 0; ni < 2; ++ni) {                              \
                    const float sc_ = bf16_to_f32(uint16_t((RB).s[ni]));                        \
                    _Pragma("unroll") for (int mi = 0; mi < 4; ++mi)                            \
                    _Pragma("unroll") for (int v = 0; v < 16; ++v) {                            \
                        acc[mi][ni][v] = __builtin_fmaf(sc_, gacc[mi][ni][v], acc[mi][ni][v]);   \
                        gacc[mi][ni][v] = 0.0f;                                                 \
                    }                                                                           \
                }                                                                               \
            }                                                                                   \
        }                                                                                       \
    } while (0)

    // Iteration t multiplies LDS A buffer t & 1 with B register set t & 1.
    // Afterwards B(t + 2) is requested into that set, A(t + 1) moves from
    // its register set into the other LDS buffer and A(t + 3) is requested
    // into the freed set, so about two K tiles stay in flight.
    const int nk = K / BK;
    StageA RA0, RA1;
    StageB RB0, RB1;
    GRIM_LOAD_A(RA0, 0);
    GRIM_LOAD_B(RB0, 0);
    if (nk > 1) { GRIM_LOAD_A(RA1, BK); GRIM_LOAD_B(RB1, BK); }
    GRIM_STORE_A(RA0, 0);
    if (nk > 2) GRIM_LOAD_A(RA0, 2 * BK);
    lds_barrier();
    // pairs of K tiles, then an odd last tile: no exit from the middle of
    // the unrolled pair, so the accumulators stay in one register set
    int kt = 0;
    // MXFP4: requests past the last tile fetch the last again into a set
    // that is never consumed (requests under a branch make the compiler wait
    // for every load in flight at the loop head, which ends the look-ahead):
    // 10% faster on MXFP4 (16 experts x 512 rows, N 4096, K 7168: 670 -> 600
    // us); bf16 B tiles run 5% slower that way and keep the branches.
    constexpr bool kAhead = F == GRIM_FMT_MXFP4;
    for (; kt + 2 <= nk; kt += 2) {
        GRIM_MMA_TILE(0, RB0);
        GRIM_FOLD(RB0, kt);
        if (kAhead || kt + 2 < nk) GRIM_LOAD_B(RB0, min(kt + 2, nk - 1) * BK);
        GRIM_STORE_A(RA1, 1);
        if (kAhead || kt + 3 < nk) GRIM_LOAD_A(RA1, min(kt + 3, nk - 1) * BK);
        lds_barrier();
        GRIM_MMA_TILE(1, RB1);
        GRIM_FOLD(RB1, kt + 1);
        if (kAhead || kt + 3 < nk) GRIM_LOAD_B(RB1, min(kt + 3, nk - 1) * BK);
        if (kt + 2 < nk) GRIM_STORE_A(RA0, 0);
        if (kAhead || kt + 4 < nk) GRIM_LOAD_A(RA0, min(kt + 4, nk - 1) * BK);
        lds_barrier();
    }
    if (kt < nk) {
        GRIM_MMA_TILE(0, RB0);
        GRIM_FOLD(RB0, kt);
    }
#undef GRIM_LOAD_A
#undef GRIM_LOAD_B
#undef GRIM_STORE_A
#undef GRIM_MMA_TILE
#undef GRIM_FOLD
#undef GRIM_READ_A

    // ---- epilogue.  acc[mi][ni][v]: row = mi*32 + (v&3) + 4*(lane>>5) +
    // 8*(v>>2), column = out_col(ni).  Results go through LDS (the A
    // buffers, free once every wave has left the K loop) so that global
    // stores are whole 16-byte row segments.
    lds_barrier();
    constexpr int SP16 = 128 + 8;   // staging row stride, 16-bit results
    constexpr int SP32 = 64 + 4;    // staging row stride, 32-bit results
    uint16_t* st16 = &As[0][0][0];
    float* st32 = reinterpret_cast<float*>(&As[0][0][0]);
    static_assert(BM * SP16 * 2 <= 2 * BM * LDK * 2 && BM * SP32 * 4 <= 2 * BM * LDK * 2,
                  "epilogue staging fits the A buffers");
    if constexpr (SWIGLU) {
        // h columns [hc0, hc0 + 128): hi plane, then lo plane
        const int hc0 = nt * (BN / 2);
        const int hcl = wave * 32 + (lane & 31);
        const int hc = hc0 + hcl;
        const float sg = hc < g.I ? col_scale<F>(w, wrow0 + hc) : 0.0f;
        const float su = hc < g.I ? col_scale<F>(w, wrow0 + g.I + hc) : 0.0f;
        uint16_t lo_v[4][16];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = mi * 32 + (v & 3) + 4 * (lane >> 5) + 8 * (v >> 2);
                const float hv = fast_silu(acc[mi][0][v] * sg) * (acc[mi][1][v] * su);
                const uint16_t hi = f32_to_bf16(hv);
                lo_v[mi][v] = f32_to_bf16(hv - bf16_to_f32(hi));
                st16[r * SP16 + hcl] = hi;
            }
        // h as a bf16 pair plane by plane [R][2][I], or (OUT_BF16) plain
        // bf16 [R][I] (the hi plane alone)
        constexpr int kPlanes = OUT_BF16 ? 1 : 2;
        const int ostride = kPlanes * g.I;
        uint16_t* o = static_cast<uint16_t*>(out) + arow0 * int64_t(ostride);
#pragma unroll
        for (int plane = 0; plane < kPlanes; ++plane) {
            if (plane == 1) {
                lds_barrier();
#pragma unroll
                for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int r = mi * 32 + (v & 3) + 4 * (lane >> 5) + 8 * (v >> 2);
                        st16[r * SP16 + hcl] = lo_v[mi][v];
                    }
            }
            lds_barrier();
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int c = tid + k * kGemmThreads;   // 16-byte chunk: row c/16, part c%16
                const int r = c >> 4, part = c & 15;
                const int col = hc0 + part * 8;
                if (r < rows_valid && col < g.I)
                    *reinterpret_cast<u32x4*>(o + r * ostride + plane * g.I + col) =
                        *reinterpret_cast<const u32x4*>(&st16[r * SP16 + part * 8]);
            }
        }
    } else {
        // four passes, one per wave's 64 columns
#pragma unroll
        for (int pw = 0; pw < 4; ++pw) {
            if (pw) lds_barrier();
            if (wave == pw) {
#pragma unroll
                for (int ni = 0; ni < 2; ++ni) {
                    const int c = out_col(ni);
                    const float sc = c < g.N ? col_scale<F>(w, wrow0 + c) : 0.0f;
#pragma unroll
                    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                        for (int v = 0; v < 16; ++v) {
                            const int r = mi * 32 + (v & 3) + 4 * (lane >> 5) + 8 * (v >> 2);
                            st32[r * SP32 + ni * 32 + (lane & 31)] = acc[mi][ni][v] * sc;
                        }
                }
            }
            lds_barrier();
            const int c0 = nt * BN + pw * 64;
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int c = tid + k * kGemmThreads;   // 16-byte fp32 chunk: row c/16, part c%16
                const int r = c >> 4, part = c & 15;
                const int col = c0 + part * 4;
                if (r < rows_valid && col < g.N) {
                    const float4 v4 = *reinterpret_cast<const float4*>(&st32[r * SP32 + part * 4]);
                    if constexpr (OUT_BF16) {
                        uint16_t* o = static_cast<uint16_t*>(out) + arow0 * int64_t(g.N);
                        const uint32_t w0 = uint32_t(f32_to_bf16(v4.x)) | (uint32_t(f32_to_bf16(v4.y)) << 16);
                        const uint32_t w1 = uint32_t(f32_to_bf16(v4.z)) | (uint32_t(f32_to_bf16(v4.w)) << 16);
                        *reinterpret_cast<uint2*>(o + r * g.N + col) = make_uint2(w0, w1);
                    } else {
                        float* o = static_cast<float*>(out) + arow0 * int64_t(g.N);
                        *reinterpret_cast<float4*>(o + r * g.N + col) = v4;
                    }
                }
            }
        }
    }
}

// Persistent 1-D grid, XCD-aware.  Work-group b runs on XCD b % 8
// (work-groups are dealt round-robin over the eight XCDs, each with its own
// L2).  The m-tile list (routed table, expert-major, its live length read
// from the device; or the shared expert's tiles) is cut into eight
// contiguous ranges, one per XCD, and an XCD's work-groups walk the
// (m-tile, column tile) items of its range column-fastest.  So every
// column tile of an m-tile, and every m-tile of most experts, is computed
// under one L2: each A row block and each expert's weights are fetched
// from HBM about once instead of once per XCD.
constexpr int kXcds = 8;
template <int F, bool SWIGLU, bool APAIR, bool OUT_BF16>
__global__ __launch_bounds__(kGemmThreads, GRIM_GEMM_OCC) void grouped_gemm_kernel(GemmArgs g, int n_col_tiles,
                                                                              int shared_part) {
    __shared__ __attribute__((aligned(16))) uint16_t As[2][APAIR ? 2 : 1][BM * LDK];
    const bool routed = shared_part == 0;
    const GemmSrc w{routed ? g.w.payload : g.w_sh.payload, routed ? g.w.scales : g.w_sh.scales,
                    routed ? g.w.row_bytes : g.w_sh.row_bytes, routed ? g.w.row_scales : g.w_sh.row_scales,
                    routed ? g.A : g.A_sh, routed ? g.out : g.out_sh};
    __shared__ int tp[kGemmRowsMaxExperts + 1], rp[kGemmRowsMaxExperts + 1];
    int total;
    if (routed && g.rows) {
        total = rows_tables(g.rows, g.ne, tp, rp);
    } else if (routed) {
        total = g.n_tiles_dev ? __builtin_amdgcn_readfirstlane(*g.n_tiles_dev) : g.tmax;
        total = total < g.tmax ? total : g.tmax;
    } else {
        total = (g.T_sh + BM - 1) / BM;
    }
    const int xcd = blockIdx.x % kXcds, per_xcd = gridDim.x / kXcds;
    const int lo = int(int64_t(total) * xcd / kXcds), hi = int(int64_t(total) * (xcd + 1) / kXcds);
    const int items = (hi - lo) * n_col_tiles;
    for (int i = blockIdx.x / kXcds; i < items; i += per_xcd) {
        gemm_tile<F, SWIGLU, APAIR, OUT_BF16>(g, w, routed, lo + i / n_col_tiles, i % n_col_tiles, As,
                                              tp, rp);
        __syncthreads();
    }
}

template <int F, bool SWIGLU, bool APAIR, bool OUT_BF16>
static hipError_t launch_kernel(hipStream_t st, const GemmArgs& g, int ntiles) {
    // routed tiles, then (one more launch) the shared expert's
    // persistent: the resident capacity, a multiple of the XCD count
    static int grid = 0;
    if (grid == 0) {
        int per_cu = 0, dev = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu, grouped_gemm_kernel<F, SWIGLU, APAIR, OUT_BF16>, kGemmThreads, 0) != hipSuccess ||
            hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return hipErrorInvalidConfiguration;
        grid = (per_cu > 0 ? per_cu : 1) * cus;
        grid = (grid + kXcds - 1) / kXcds * kXcds;
    }
    if (g.tmax > 0 || g.rows)
        hipLaunchKernelGGL((grouped_gemm_kernel<F, SWIGLU, APAIR, OUT_BF16>), dim3(grid),
                           dim3(kGemmThreads), 0, st, g, ntiles, 0);
    if (g.T_sh > 0) {
        const int items = (g.T_sh + BM - 1) / BM * ntiles;
        const int gs = min(grid, (items + kXcds - 1) / kXcds * kXcds);
        hipLaunchKernelGGL((grouped_gemm_kernel<F, SWIGLU, APAIR, OUT_BF16>), dim3(gs),
                           dim3(kGemmThreads), 0, st, g, ntiles, 1);
    }
    return hipGetLastError();
}

template <int F>
static hipError_t launch_fmt(hipStream_t st, const GemmArgs& g) {
    const int ntiles = g.swiglu ? (g.I + BN / 2 - 1) / (BN / 2) : (g.N + BN - 1) / BN;
    const int my_max = g.tmax + (g.T_sh > 0 ? (g.T_sh + BM - 1) / BM : 0);
    if ((my_max <= 0 && !g.rows) || ntiles <= 0) return hipSuccess;
    if (g.swiglu)
        return g.out_bf16 ? launch_kernel<F, true, false, true>(st, g, ntiles)
                          : launch_kernel<F, true, false, false>(st, g, ntiles);
    if (g.a_pair)
        return g.out_bf16 ? launch_kernel<F, false, true, true>(st, g, ntiles)
                          : launch_kernel<F, false, true, false>(st, g, ntiles);
    return g.out_bf16 ? launch_kernel<F, false, false, true>(st, g, ntiles)
                      : launch_kernel<F, false, false, false>(st, g, ntiles);
}

bool gemm_format_ok(int fmt) {
    return fmt == GRIM_FMT_INT8 || fmt == GRIM_FMT_MXFP4 || fmt == GRIM_FMT_BF16 || fmt == kGemmFmtS4;
}

hipError_t gemm_launch(hipStream_t st, int fmt, const GemmArgs& g) {
    switch (fmt) {
    case GRIM_FMT_INT8: return launch_fmt<GRIM_FMT_INT8>(st, g);
    case GRIM_FMT_MXFP4: return launch_fmt<GRIM_FMT_MXFP4>(st, g);
    case GRIM_FMT_BF16: return launch_fmt<GRIM_FMT_BF16>(st, g);
    case kGemmFmtS4: return launch_fmt<kGemmFmtS4>(st, g);
    }
    return hipErrorInvalidValue;
}

}  // namespace grim
