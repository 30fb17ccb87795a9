// gemv_grouped.hip -- the expert products for few rows per expert, grouped
// by expert: each expert's weights are streamed once per group of up to
// kGvMT of its rows, instead of once per (token, slot) or once per 128-row
// MFMA tile.  For batches whose routes spread over many experts (C3: 32
// routes over ~20 experts; C5: 256 routes over ~170 experts) the weight
// stream is the whole cost, and a GEMV-shaped kernel streams it at HBM rate
// where the MFMA tile kernel spends its time on empty tile rows.
//
// Rows arrive grouped by expert (the dispatch's counts / offsets) and the
// dispatch's tile table, built with an m-block of kGvMT rows, names each
// group (expert, block); the shared expert's T rows follow as extra groups.
// A kernel with MT < kGvMT rows per pass takes each group in kGvMT / MT
// parts.
//
// Persistent work-groups walk items (group part, chunk of weight rows):
//   * every lane multiplies 32-element chunks c = lane, lane + 64, ...
//     (CI of them) of the reduction dimension.  At the start of an item it
//     reads the group's activation rows at its chunks from global memory
//     (L2: they are small and shared) and keeps them in registers for the
//     whole item, formatted as bf16 pair words (the hi halves of the exact
//     split x = hi + lo, in the weight decoder's pair order) with the
//     chunk's sum; the activations cost no LDS traffic;
//   * each wave owns RU rows (gate_up: (gate, up) pairs) of every
//     sub-block and streams exactly those rows -- payload, scales, zero
//     points -- through its own LDS ring, ST sub-blocks deep, filled by
//     buffer_load ... lds (straight into LDS, no registers).  A wave reads
//     only what it loaded, so its own vmcnt is its only wait: the kernel
//     has no barrier, and the waves of a work-group drift freely;
//   * each weight chunk is decoded once and multiplied with every row of
//     the group; a (row, group row) pair costs one cross-lane sum;
//   * activations with a non-zero lo half (fp32 values that are not bf16)
//     add a second product per sub-block with the lo halves, formed from
//     global memory as they are used: the two halves are exact, so the sum
//     is the product with the fp32 activations to within 2^-17 relative.
//     bf16 activations, the usual case, never take it.
// LDS holds only the rings: as many waves as fit, at most eight.
#include <algorithm>

#include "gemv_grouped.hpp"

#include "gemv_impl.hpp"

namespace grim {

#ifdef GRIM_TIMING
#define GV_TS(i)                                                                              \
    do {                                                                                      \
        if (a.ts && threadIdx.x == 0 && first_item && (i) < 16)                               \
            a.ts[blockIdx.x * 16 + (i)] = __builtin_amdgcn_s_memrealtime();                   \
    } while (0)
#else
#define GV_TS(i) do {} while (0)
#endif

constexpr int kGvMaxWaves = 8;
constexpr size_t kGvLds = 160u << 10;          // LDS per work-group

typedef __attribute__((address_space(3))) void* gv_lds_ptr_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t*)(p)));
}

// LDS reads hidden from the compiler: it would otherwise wait for every
// load in flight before each LDS read, as it cannot tell them apart from
// the ring the DMA writes.  The caller waits on lgkmcnt itself, tied to
// the registers read.
__device__ __forceinline__ u32x4 lds_u32x4(uint32_t addr) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}

// One activation chunk (32 elements) in the weight decoder's pair order:
// four quads of bf16 pair words (quad q: elements [8q, 8q + 8)) of the hi
// halves and (LO) of the lo halves, and the sum of the staged values.
template <bool LO> struct GvAct {
    u32x4 h[4];
    u32x4 l[LO ? 4 : 1];
    float s;
};

// The 32 fp32 values of chunk c of row src.
struct GvRaw {
    float4 v[8];
};

__device__ __forceinline__ GvRaw gv_raw(const float* src, int c) {
    const float4* s4 = reinterpret_cast<const float4*>(src) + c * 8;
    GvRaw r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r.v[i] = s4[i];
    return r;
}

// The chunk formatted.  LO: both planes; else the hi plane, and any_lo is
// set when a value has a non-zero lo half.
template <int F, bool LO>
__device__ __forceinline__ GvAct<LO> gv_format(const GvRaw& r, int& any_lo) {
    GvAct<LO> x;
    float part[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4 p = r.v[2 * g], q = r.v[2 * g + 1];
        const float vals[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
        uint32_t hw[4], lw[4];
        part[g] = format_group<F>(vals, hw, lw, any_lo);   // sum of hi + lo
        x.h[g] = u32x4{hw[0], hw[1], hw[2], hw[3]};
        if constexpr (LO) {
            x.l[g] = u32x4{lw[0], lw[1], lw[2], lw[3]};
        } else {
            float sh = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) sh += bits_f(hw[j] << 16) + bits_f(hw[j] & 0xFFFF0000u);
            part[g] = sh;
        }
    }
    x.s = (part[0] + part[1]) + (part[2] + part[3]);
    // the packed words are formed here, not next to their uses: sunk to
    // the streaming loop, the unpacked halves would hold twice the registers
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        asm volatile("" : "+v"(x.h[g]));
        if constexpr (LO) asm volatile("" : "+v"(x.l[g]));
    }
    asm volatile("" : "+v"(x.s));
    return x;
}

template <int F, bool LO>
__device__ __forceinline__ GvAct<LO> gv_act(const float* src, int c, int& any_lo) {
    return gv_format<F, LO>(gv_raw(src, c), any_lo);
}

// Words of one formatted activation row of K elements: hi plane (K / 2
// pair words), lo plane (K / 2), then per chunk (sum of hi + lo, lo flag),
// rounded to 16 bytes.
__host__ __device__ inline int gv_act_words(int K) { return (K + K / 16 + 3) & ~3; }

// Formats rows [0, rows0) of src0 into dst0 and [0, rows1) of src1 into
// dst1 (K elements a row): one thread per group of eight elements, the
// four threads of a chunk aligned lanes.
template <int F>
__global__ __launch_bounds__(256) void gv_format_kernel(const float* src0, int rows0, uint32_t* dst0,
                                                        const float* src1, int rows1, uint32_t* dst1, int K) {
    const int ng = K / 8, AW = gv_act_words(K);
    const int64_t gi = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t n0 = int64_t(rows0) * ng, n1 = int64_t(rows1) * ng;
    const bool ok = gi < n0 + n1;
    const bool second = gi >= n0;
    const int64_t li = ok ? (second ? gi - n0 : gi) : 0;
    const int row = int(li / ng), g = int(li % ng);
    const float* src = (second ? src1 : src0) + int64_t(row) * K;
    uint32_t* dst = (second ? dst1 : dst0) + int64_t(row) * AW;
    float4 p = make_float4(0.f, 0.f, 0.f, 0.f), q = p;
    if (ok) {
        p = reinterpret_cast<const float4*>(src)[2 * g];
        q = reinterpret_cast<const float4*>(src)[2 * g + 1];
    }
    const float vals[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
    uint32_t hw[4], lw[4];
    int lo = 0;
    float part = format_group<F>(vals, hw, lw, lo);
    part += dpp_f<kDppXor1>(part);
    part += dpp_f<kDppXor2>(part);
    uint32_t fl = uint32_t(lo);
    fl |= dpp_u<kDppXor1>(fl);
    fl |= dpp_u<kDppXor2>(fl);
    if (!ok) return;
    reinterpret_cast<u32x4*>(dst)[g] = u32x4{hw[0], hw[1], hw[2], hw[3]};
    reinterpret_cast<u32x4*>(dst + K / 2)[g] = u32x4{lw[0], lw[1], lw[2], lw[3]};
    if ((g & 3) == 0) reinterpret_cast<uint2*>(dst + K)[g / 4] = make_uint2(f_bits(part), fl);
}

// One weight chunk decoded once for several activation rows: 16 bf16 pair
// words in the activation pair order, the chunk's scale and (INT4) the
// offset 128 + zero point that the pair words carry.
struct GvW {
    uint32_t q[16];
    float s, zc;
};

template <int F>
__device__ __forceinline__ GvW gv_decode(const Pre& p) {
    GvW d;
    const uint32_t w[4] = {p.raw.x, p.raw.y, p.raw.z, p.raw.w};
    d.s = pre_scale<F>(p);
    if constexpr (F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16) {
        int z = int(p.zb);
        uint32_t xm = 0;
        if (z == 0xFF) { xm = 0x88888888u; z = 8; }   // signed s4 -> offset binary
        d.zc = 128.0f + float(z);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t ww = w[i] ^ xm;
#pragma unroll
            for (int j = 0; j < 4; ++j) d.q[4 * i + j] = ((ww >> (4 * j)) & 0x000F000Fu) | 0x43004300u;   // 128 + q
        }
    } else {
        static_assert(F == GRIM_FMT_MXFP4, "int4 or mxfp4");
        d.zc = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bf16x2_t v0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[i], 1.0f, 0);
            const bf16x2_t v1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[i], 1.0f, 1);
            const bf16x2_t v2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[i], 1.0f, 2);
            const bf16x2_t v3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[i], 1.0f, 3);
            __builtin_memcpy(&d.q[4 * i + 0], &v0, 4);
            __builtin_memcpy(&d.q[4 * i + 1], &v1, 4);
            __builtin_memcpy(&d.q[4 * i + 2], &v2, 4);
            __builtin_memcpy(&d.q[4 * i + 3], &v3, 4);
        }
    }
    return d;
}

// The decoded chunk times one activation chunk (both planes with LO).
template <int F, bool LO>
__device__ __forceinline__ float gv_dot(const GvW& d, const GvAct<LO>& x) {
    float a = 0.0f, b = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a = dot2(d.q[4 * i + 0], x.h[i].x, a);
        a = dot2(d.q[4 * i + 1], x.h[i].y, a);
        a = dot2(d.q[4 * i + 2], x.h[i].z, a);
        a = dot2(d.q[4 * i + 3], x.h[i].w, a);
        if constexpr (LO) {
            b = dot2(d.q[4 * i + 0], x.l[i].x, b);
            b = dot2(d.q[4 * i + 1], x.l[i].y, b);
            b = dot2(d.q[4 * i + 2], x.l[i].z, b);
            b = dot2(d.q[4 * i + 3], x.l[i].w, b);
        }
    }
    if constexpr (F == GRIM_FMT_MXFP4) return (a + b) * d.s;
    else return d.s * ((a + b) - d.zc * x.s);
}

__device__ __forceinline__ WRsrc gv_rsrc(const WView& w, int64_t row0, uint32_t nrows, int sb) {
    const bool hz = w.zeros != nullptr;
    WRsrc rs;
    rs.p = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(w.payload + row0 * w.row_bytes), 0,
                                             int(nrows * uint32_t(w.row_bytes)), 0x00020000);
    rs.s = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(static_cast<const uint8_t*>(w.scales) + row0 * w.row_scales * sb), 0,
        int(nrows * uint32_t(w.row_scales) * sb), 0x00020000);
    // without zero points the zero-point loads read scale bytes (never
    // used), so that the count of loads per stage stays fixed
    rs.z = hz ? __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(w.zeros + row0 * w.row_scales), 0,
                                                  int(nrows * uint32_t(w.row_scales)), 0x00020000)
              : rs.s;
    return rs;
}

// Item resolution: the part's first row, row count and weight block.
// Groups [0, n_live) are the dispatch table's (expert, kGvMT-row block);
// the shared expert's groups follow.  Part p of a group: rows
// [p * MT, p * MT + MT) of it.
struct GvItem {
    int64_t wrow0;   // first weight row of the expert block
    int r0, mc;      // first input / output row, rows in the part (<= 0: none)
    bool sh;
};

template <int MT>
__device__ __forceinline__ GvItem gv_item(const GvArgs& a, int grp, int part, int n_live, int rows_per_expert) {
    GvItem it{0, 0, 0, false};
    int r0, cnt;
    if (grp < n_live) {
        const int e = __builtin_amdgcn_readfirstlane(a.tile_e[grp]);
        if (e < 0) return it;
        const int mb = __builtin_amdgcn_readfirstlane(a.tile_mb[grp]);
        r0 = __builtin_amdgcn_readfirstlane(a.offsets[e]) + mb * kGvMT;
        cnt = min(kGvMT, __builtin_amdgcn_readfirstlane(a.counts[e]) - mb * kGvMT);
        it.wrow0 = int64_t(e) * rows_per_expert;
    } else {
        r0 = (grp - n_live) * kGvMT;
        cnt = min(kGvMT, a.T_sh - r0);
        it.sh = true;
    }
    it.r0 = r0 + part * MT;
    it.mc = min(MT, cnt - part * MT);
    return it;
}

// Shape of a reduction length K <= 2048 * CI: MT group rows per pass (the
// activations of MT rows at CI chunks stay in registers: 17 * MT * CI of
// them, twice that with both planes), RU rows (gate_up: pairs) per wave and sub-block, ST ring stages;
// per weight row CI payload loads of 1 KiB (16 bytes a lane) and NSS + NSZ
// side loads of 256 bytes (4 bytes a lane): scales (INT4 groups of >= 32
// give at most K / 16 bytes a row; MXFP4 K / 32) and zero points, each
// copied from its 4-byte-aligned start.
template <int F, int CI, bool GU> struct GvShape {
    static constexpr bool kInt4 = F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16;
    static constexpr int KMAX = 2048 * CI;
    // down multiplies h, fp32 values: both activation planes, always
    static constexpr bool LO = !GU;
    static constexpr int MT = GU ? (CI <= 2 ? kGvMT : 2) : (CI == 1 ? kGvMT : CI == 2 ? 2 : 1);
    static constexpr int RU = GU ? 1 : (CI <= 2 ? 2 : 1);
    static constexpr int RW = GU ? 2 * RU : RU;             // weight rows per wave and sub-block
    static constexpr int RI = GU ? 256 : 512;               // rows (pairs) per item, about
    static constexpr int NSS = (KMAX / (kInt4 ? 16 : 32) + 3 + 255) / 256;
    static constexpr int NSZ = kInt4 ? (KMAX / 32 + 3 + 255) / 256 : 0;
    static constexpr int NT = RW * (CI + NSS + NSZ);        // loads per wave and stage
    static constexpr int SA = CI >= 3 ? 2 : 4;             // stages ahead, at most (long rows: more waves)
    static constexpr int ST = 1 + (63 / NT < SA ? 63 / NT : SA);
    static_assert((ST - 1) * NT <= 63, "vmcnt holds 63");
    static_assert(kGvMT % MT == 0, "parts of a group");
};

// Bytes of one wave's ring stage for reduction length K.
template <int F, int CI, bool GU>
__host__ __device__ inline uint32_t gv_wave_stage_bytes(int K) {
    using S = GvShape<F, CI, GU>;
    return uint32_t(S::RW) * (uint32_t(K / 2) + uint32_t(S::NSS + S::NSZ) * 256u);
}

// An item of gate_up whose activations are fp32 values that are not all
// bf16 (rare: the layer input is usually bf16-valued): both planes, formed
// from global memory, and the weights read straight from global memory.
// The calling wave computes the rows it would have streamed: i0 + sb * SB
// + [0, RU) for sb < nsb.  A function of its own, so that its registers do
// not weigh on the streaming loop.
template <int F, bool GU>
__device__ __forceinline__ void gv_item_slow(const GvArgs& a, const GvItem& it, int i0, int SB, int nsb,
                                                       int RU) {
    const int lane = threadIdx.x & (kWave - 1);
    const int N = a.N, Kd = a.K, C = Kd / 32;
    const WView& w = it.sh ? a.w_sh : a.w;
    for (int k = 0; k < nsb * RU; ++k) {
        const int i = i0 + (k / RU) * SB + k % RU;
        if (i >= N) continue;
        for (int m = 0; m < it.mc; ++m) {
            const int rr = it.r0 + m;
            const float* sm = GU ? a.x + int64_t(it.sh ? rr : a.perm_token[rr]) * Kd
                                 : (it.sh ? a.h_sh : a.h) + int64_t(rr) * Kd;
            float g = 0.0f, u = 0.0f;
            for (int c = lane; c < C; c += kWave) {
                int dummy = 0;
                const GvAct<true> x = gv_act<F, true>(sm, c, dummy);
                Pre p;
                prefetch<F>(w, it.wrow0 + i, c, p);
                g += gv_dot<F, true>(gv_decode<F>(p), x);
                if constexpr (GU) {
                    prefetch<F>(w, it.wrow0 + N + i, c, p);
                    u += gv_dot<F, true>(gv_decode<F>(p), x);
                }
            }
            g = wave_sum(g);
            if constexpr (GU) {
                u = wave_sum(u);
                if (lane == 0) (it.sh ? a.h_sh : a.h)[int64_t(rr) * N + i] = fast_silu(g) * u;
            } else {
                if (lane == 0) (it.sh ? a.y_sh : a.y)[int64_t(rr) * N + i] = g;
            }
        }
    }
}

// One persistent kernel for both products.  GU: gate_up + SwiGLU, rows are
// (gate, up) pairs, out h; else down, out y.  Work-group b walks items
// b, b + gridDim.x, ... over (group part, chunk of rows), with
// blockDim.x / 64 waves.  Per sub-block each wave issues its NT loads for
// the sub-block ST - 1 ahead, then waits until only those are in flight.
template <int F, int CI, bool GU>
__global__ __launch_bounds__(kGvMaxWaves * kWave) void gv_kernel(GvArgs a) {
    using S = GvShape<F, CI, GU>;
    constexpr int MT = S::MT, RU = S::RU, RW = S::RW, NT = S::NT, NSS = S::NSS, NSZ = S::NSZ;
    constexpr int ST = S::ST, WAIT = (ST - 1) * NT, PARTS = kGvMT / MT;
    constexpr bool kInt4 = S::kInt4, LO = S::LO;
    extern __shared__ __attribute__((aligned(1024))) uint8_t gv_ring[];
    const int W = blockDim.x / kWave;
    const int N = a.N, Kd = a.K, C = Kd / 32;
    const uint32_t lrow = uint32_t(Kd / 2);                  // payload row bytes, global and LDS
    const int rows_per_expert = GU ? 2 * N : N;
    const int SB = W * RU;                                   // rows (pairs) per sub-block
    const int NSB = max(1, S::RI / SB);                      // sub-blocks per item
    const int n_chunks = (N + SB * NSB - 1) / (SB * NSB);
    const int n_live = __builtin_amdgcn_readfirstlane(*a.n_live);
    const int groups = n_live + (a.T_sh + kGvMT - 1) / kGvMT;
    const int n_items = groups * PARTS * n_chunks;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const uint32_t WS = gv_wave_stage_bytes<F, CI, GU>(Kd);
    uint8_t* ring = gv_ring + size_t(wave) * ST * WS;
    const uint32_t ring_base = lds_addr(ring);
    const uint32_t side0 = uint32_t(RW) * lrow;              // side slots inside a wave stage

    for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
        const bool first_item = item == int(blockIdx.x);
        (void)first_item;
        GV_TS(0);
        const int gp = item / n_chunks, chunk = item % n_chunks;
        const GvItem it = gv_item<MT>(a, gp / PARTS, gp % PARTS, n_live, rows_per_expert);
        if (it.mc <= 0) continue;   // uniform
        const WView& w = it.sh ? a.w_sh : a.w;
        const bool hz = kInt4 && w.zeros != nullptr;
        const int srb = kInt4 ? 2 * w.row_scales : w.row_scales;     // scale bytes per row
        const WRsrc rs = gv_rsrc(w, it.wrow0, uint32_t(rows_per_expert), kInt4 ? 2 : 1);
        const int row0 = chunk * SB * NSB;                   // first row (pair) of the item
        const int nsb = min(NSB, (N - row0 + SB - 1) / SB);  // sub-blocks with rows
        // weight row of this wave's row r in sub-block sb (rows past N
        // repeat the last: loaded, never written out)
        auto wrow = [&](int sb, int r) {
            const int g = (GU && r >= RU) ? 1 : 0;
            const int i = min(row0 + sb * SB + wave * RU + (r < RU ? r : r - RU), N - 1);
            return (g ? N : 0) + i;
        };
        // this wave's loads of sub-block sb into its ring stage sb % ST:
        // exactly NT instructions, each with lane 0 active
        auto issue = [&](int sb) {
            uint8_t* st = ring + (sb % ST) * WS;
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const uint32_t row = uint32_t(wrow(sb, r));
#pragma unroll
                for (int j = 0; j < CI; ++j) {
                    const int ch = j * kWave + lane;
                    // (CI - 1) * 64 < C: lane 0 always loads
                    if (ch < C)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            rs.p, (gv_lds_ptr_t)(st + r * lrow + j * kWave * 16), 16,
                            int(uint32_t(ch) * 16u), int(row * lrow), 0, 2);
                }
#pragma unroll
                for (int k = 0; k < NSS + NSZ; ++k) {
                    const bool z = k >= NSS;
                    const uint32_t rb = uint32_t(z ? w.row_scales : srb);
                    const uint32_t b0 = row * rb, a0 = b0 & ~3u;
                    const uint32_t len = b0 - a0 + rb;
                    const uint32_t off = uint32_t((z ? k - NSS : k) * 256 + lane * 4);
                    if (off < len || lane == 0)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            z ? rs.z : rs.s, (gv_lds_ptr_t)(st + side0 + (r * (NSS + NSZ) + k) * 256), 4,
                            int(off < len ? off : 0u), int(a0), 0, 0);
                }
            }
        };

        // the ring's first stages, then this lane's chunks of the part's
        // activation rows (formatted rows: hi plane, lo plane, then (sum,
        // lo flag) per chunk), in registers for the whole item; rows past
        // mc repeat row 0 and are never used.  The activations are waited
        // for here (with the ring's first stages: they are older), so
        // that the streaming loop holds no compiler-tracked load.
#pragma unroll
        for (int u = 0; u < ST - 1; ++u)
            if (u < nsb) issue(u);
        const int AW = gv_act_words(Kd);
        GvAct<LO> xr[CI][MT];
        uint32_t any_lo = 0;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int r = it.r0 + (m < it.mc ? m : 0);
            const uint32_t* row = GU ? a.af + int64_t(it.sh ? r : a.perm_token[r]) * AW
                                     : (it.sh ? a.af_sh : a.af) + int64_t(r) * AW;
#pragma unroll
            for (int ci = 0; ci < CI; ++ci) {
                const int cc = min(ci * kWave + lane, C - 1);
                const u32x4* hq = reinterpret_cast<const u32x4*>(row) + cc * 4;
#pragma unroll
                for (int q = 0; q < 4; ++q) xr[ci][m].h[q] = hq[q];
                if constexpr (LO) {
                    const u32x4* lq = reinterpret_cast<const u32x4*>(row + Kd / 2) + cc * 4;
#pragma unroll
                    for (int q = 0; q < 4; ++q) xr[ci][m].l[q] = lq[q];
                }
                const uint2 sf = reinterpret_cast<const uint2*>(row + Kd)[cc];
                xr[ci][m].s = bits_f(sf.x);
                any_lo |= sf.y;
            }
        }
#pragma unroll
        for (int ci = 0; ci < CI; ++ci)
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                asm volatile("" : "+v"(xr[ci][m].h[0]), "+v"(xr[ci][m].h[1]), "+v"(xr[ci][m].h[2]),
                             "+v"(xr[ci][m].h[3]), "+v"(xr[ci][m].s));
                if constexpr (LO)
                    asm volatile("" : "+v"(xr[ci][m].l[0]), "+v"(xr[ci][m].l[1]), "+v"(xr[ci][m].l[2]),
                                 "+v"(xr[ci][m].l[3]));
            }
        if constexpr (!LO) {
            // a lo half somewhere: this wave takes its rows the slow way
            if (__builtin_amdgcn_ballot_w64(any_lo != 0) != 0) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the ring's loads, unused
                gv_item_slow<F, GU>(a, it, row0 + wave * RU, SB, nsb, RU);
                continue;
            }
        }
        GV_TS(1);

        // sub-block sb's loads complete (this wave's), the next ones issued
        auto wait_stage = [&](int sb) {
            const int ahead = sb + ST - 1;
            if (ahead < nsb) {
                issue(ahead);
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAIT) : "memory");
            } else if (ahead == nsb) {
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NT) : "memory");
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
        };
        // this lane's weights of sub-block sb at chunk iteration ci
        auto weights = [&](int sb, int ci, Pre (&pw)[RW], uint32_t dep) {
            const uint32_t stb = ring_base + uint32_t(sb % ST) * WS + dep;
            const uint32_t cc = uint32_t(min(ci * kWave + lane, C - 1));
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const uint32_t row = uint32_t(wrow(sb, r));
                pw[r].raw = lds_u32x4(stb + uint32_t(r) * lrow + cc * 16u);
                const uint32_t slot = stb + side0 + uint32_t(r * (NSS + NSZ)) * 256u;
                uint32_t v;
                if constexpr (kInt4) {
                    const uint32_t gi = (cc * 32u) >> w.gshift;
                    asm volatile("ds_read_u16 %0, %1"
                                 : "=v"(v) : "v"(slot + ((row * uint32_t(srb)) & 3u) + gi * 2u));
                    pw[r].sb = v;
                    if (hz) {
                        asm volatile("ds_read_u8 %0, %1"
                                     : "=v"(v)
                                     : "v"(slot + uint32_t(NSS) * 256u + ((row * uint32_t(w.row_scales)) & 3u) + gi));
                        pw[r].zb = v;
                    } else {
                        pw[r].zb = uint32_t(w.default_zero);
                    }
                } else {
                    asm volatile("ds_read_u8 %0, %1" : "=v"(v) : "v"(slot + ((row * uint32_t(srb)) & 3u) + cc));
                    pw[r].sb = v;
                    pw[r].zb = 0;
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int r = 0; r < RW; ++r) asm volatile("" : "+v"(pw[r].raw), "+v"(pw[r].sb), "+v"(pw[r].zb));
        };
        // one cross-lane sum per (row, group row); lane 0 writes
        auto store = [&](int sb, float (&acc)[RW][MT]) {
            const int ib = row0 + sb * SB + wave * RU;
#pragma unroll
            for (int r = 0; r < RU; ++r) {
                const int i = ib + r;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    if (m >= it.mc) break;   // uniform
                    if constexpr (GU) {
                        const float g = wave_sum(acc[r][m]);
                        const float u = wave_sum(acc[RU + r][m]);
                        if (lane == 0 && i < N)
                            (it.sh ? a.h_sh : a.h)[int64_t(it.r0 + m) * N + i] = fast_silu(g) * u;
                    } else {
                        const float v = wave_sum(acc[r][m]);
                        if (lane == 0 && i < N) (it.sh ? a.y_sh : a.y)[int64_t(it.r0 + m) * N + i] = v;
                    }
                }
            }
        };

        // the streaming loop: no global load inside it, so the only waits
        // on the ring are the ones above
#pragma unroll 1
        for (int sb = 0; sb < nsb; ++sb) {
            wait_stage(sb);
            GV_TS(2 + 2 * sb);
            float acc[RW][MT];
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
            uint32_t dep = 0;
#pragma unroll
            for (int ci = 0; ci < CI; ++ci) {
                const bool cok = ci * kWave + lane < C;
                Pre pw[RW];
                weights(sb, ci, pw, dep);
#pragma unroll
                for (int r = 0; r < RW; ++r) {
                    const GvW wd = gv_decode<F>(pw[r]);
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        if (m >= it.mc) break;   // uniform
                        const float d = gv_dot<F, LO>(wd, xr[ci][m]);
                        acc[r][m] += cok ? d : 0.0f;
                    }
                }
                // the next chunk's reads wait for this chunk's last product:
                // left to itself the compiler interleaves chunks and runs
                // out of registers
                asm volatile("v_mov_b32 %0, 0" : "=v"(dep) : "v"(acc[RW - 1][0]));
            }
            GV_TS(3 + 2 * sb);
            store(sb, acc);
        }
    }
}

// Launch plan: waves, as many as fit in LDS, at most eight, at least four.
struct GvPlan {
    int waves;        // 0: no fit
    size_t lds;       // dynamic LDS bytes
};

template <int F, int CI, bool GU>
static GvPlan gv_plan_t(int K) {
    const size_t ws = size_t(GvShape<F, CI, GU>::ST) * gv_wave_stage_bytes<F, CI, GU>(K);
    const int wv = int(std::min<size_t>(kGvMaxWaves, kGvLds / ws));
    return wv >= 4 ? GvPlan{wv, size_t(wv) * ws} : GvPlan{0, 0};
}

template <int F, bool GU>
static GvPlan gv_plan(int K) {
    switch ((K / 32 + kWave - 1) / kWave) {
    case 1: return gv_plan_t<F, 1, GU>(K);
    case 2: return gv_plan_t<F, 2, GU>(K);
    case 3: return gv_plan_t<F, 3, GU>(K);
    case 4: return gv_plan_t<F, 4, GU>(K);
    }
    return GvPlan{0, 0};
}

static GvPlan gv_plan_fmt(int fmt, int K, bool gate_up) {
    switch (fmt) {
    case GRIM_FMT_INT4: return gate_up ? gv_plan<GRIM_FMT_INT4, true>(K) : gv_plan<GRIM_FMT_INT4, false>(K);
    case GRIM_FMT_INT4_F16:
        return gate_up ? gv_plan<GRIM_FMT_INT4_F16, true>(K) : gv_plan<GRIM_FMT_INT4_F16, false>(K);
    case GRIM_FMT_MXFP4: return gate_up ? gv_plan<GRIM_FMT_MXFP4, true>(K) : gv_plan<GRIM_FMT_MXFP4, false>(K);
    }
    return GvPlan{0, 0};
}

template <int F, bool GU>
static hipError_t gv_launch_fmt(hipStream_t st, const GvArgs& a) {
    const GvPlan p = gv_plan<F, GU>(a.K);
    if (!p.waves) return hipErrorInvalidValue;
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return hipErrorInvalidConfiguration;
    }
    const dim3 grid(cus), block(p.waves * kWave);
    switch ((a.K / 32 + kWave - 1) / kWave) {
    case 1: hipLaunchKernelGGL((gv_kernel<F, 1, GU>), grid, block, p.lds, st, a); break;
    case 2: hipLaunchKernelGGL((gv_kernel<F, 2, GU>), grid, block, p.lds, st, a); break;
    case 3: hipLaunchKernelGGL((gv_kernel<F, 3, GU>), grid, block, p.lds, st, a); break;
    case 4: hipLaunchKernelGGL((gv_kernel<F, 4, GU>), grid, block, p.lds, st, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t gv_format_launch(hipStream_t st, int fmt, const float* src0, int rows0, uint32_t* dst0,
                            const float* src1, int rows1, uint32_t* dst1, int K) {
    const int64_t n = int64_t(rows0 + rows1) * (K / 8);
    if (n == 0) return hipSuccess;
    const dim3 grid(unsigned((n + 255) / 256)), block(256);
    switch (fmt) {
    case GRIM_FMT_INT4:
        hipLaunchKernelGGL(gv_format_kernel<GRIM_FMT_INT4>, grid, block, 0, st, src0, rows0, dst0, src1, rows1, dst1, K);
        break;
    case GRIM_FMT_INT4_F16:
        hipLaunchKernelGGL(gv_format_kernel<GRIM_FMT_INT4_F16>, grid, block, 0, st, src0, rows0, dst0, src1, rows1,
                           dst1, K);
        break;
    case GRIM_FMT_MXFP4:
        hipLaunchKernelGGL(gv_format_kernel<GRIM_FMT_MXFP4>, grid, block, 0, st, src0, rows0, dst0, src1, rows1, dst1, K);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

size_t gv_act_bytes(int K) { return size_t(gv_act_words(K)) * 4; }

bool gv_shape_ok(int fmt, int H, int I) {
    const bool f = fmt == GRIM_FMT_INT4 || fmt == GRIM_FMT_INT4_F16 || fmt == GRIM_FMT_MXFP4;
    return f && H % 32 == 0 && I % 32 == 0 && gv_plan_fmt(fmt, H, true).waves && gv_plan_fmt(fmt, I, false).waves;
}

hipError_t gv_launch(hipStream_t st, int fmt, const GvArgs& g, bool gate_up) {
    switch (fmt) {
    case GRIM_FMT_INT4: return gate_up ? gv_launch_fmt<GRIM_FMT_INT4, true>(st, g)
                                       : gv_launch_fmt<GRIM_FMT_INT4, false>(st, g);
    case GRIM_FMT_INT4_F16: return gate_up ? gv_launch_fmt<GRIM_FMT_INT4_F16, true>(st, g)
                                           : gv_launch_fmt<GRIM_FMT_INT4_F16, false>(st, g);
    case GRIM_FMT_MXFP4: return gate_up ? gv_launch_fmt<GRIM_FMT_MXFP4, true>(st, g)
                                        : gv_launch_fmt<GRIM_FMT_MXFP4, false>(st, g);
    }
    return hipErrorInvalidValue;
}

}  // namespace grim
