// gemm_i8.hip -- grouped expert GEMM for INT8 weights on the CDNA4 int8
// MFMA (prefill regime), and the activation limb quantisers it reads.
//
// The weights are int8 codes with one scale per output channel
// (include/b70/weights.hpp:46-126); the activations are bf16 / fp32.  A bf16
// MFMA would need every weight byte converted to bf16 in registers (about
// seven VALU instructions per MFMA, which with one wave per SIMD keeps the
// matrix core idle most of the time).  Here the activations are split
// instead, once per row, into two int8 limbs under one fp32 scale,
//     a = s * (hi + lo / 254),   s = max|row| / 127,  |hi|, |lo| <= 127,
// (error <= s / 508 per element, ~2^-16 of the row's largest value), and
// both limbs multiply the raw weight codes on v_mfma_i32_32x32x32_i8 into
// exact int32 sums; the epilogue forms s_row * s_col * (hi + lo / 254).
// Two int8 passes cost what one bf16 pass costs, with no conversion at all.
//
// Tile: 128 rows x 256 columns x 64 K, 256 threads; wave w owns columns
// [64w, 64w + 64) of the tile for all 128 rows (4 x 2 MFMA tiles per limb).
// A (limbs) and B (codes) both stream into a 4-stage LDS ring through
// buffer_load ... lds (16 bytes per lane, no registers involved).  A limb
// rows are stored [K/64][2][64] so that one K tile of a row is one 128-byte
// line; every DMA instruction moves whole row segments (A 8 x 128 bytes, B
// 16 x 64 bytes) into XOR-swizzled slots that keep the fragment reads free
// of bank conflicts.  Three K tiles are in flight while one is multiplied.
// Persistent XCD-aware grid over (m-tile, column tile) items, rows from the
// dispatch's tile table.
#include "common.hpp"
#include "gemm.hpp"
#include "gemm_i8.hpp"

#include <type_traits>

namespace grim {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int QBM = 128, QBN = 256, QBK = 64;
constexpr int kQStages = 4;
constexpr int kQStageBytes = 32768;          // A 16 KiB (2 limbs x 4 x 2 fragments), B 16 KiB
constexpr int kQThreads = 256;
constexpr int kQXcds = 8;
constexpr float kLoScale = 1.0f / 254.0f;

typedef __attribute__((address_space(3))) void* lds_ptr_t;

#ifdef GRIM_I8_TIMING
__device__ uint64_t g_i8_wait[4096], g_i8_issue[4096], g_i8_total[4096], g_i8_epi[4096];
#endif

template <int AUX>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, voff, soff, 0, AUX);
}

struct I8Src {
    const uint8_t* w;
    const float* ws;
    int64_t row_bytes;
    const int8_t* A;
    const float* sa;
    float* out;
};

template <bool SWIGLU>
__device__ __forceinline__ void i8_tile(const GemmI8Args& g, const I8Src& src, bool routed, int ty,
                                        int nt, uint8_t (*smem)[kQStageBytes]) {
    int rows_valid;
    int64_t arow0, wrow0;
    if (routed) {
        const int e = __builtin_amdgcn_readfirstlane(g.tile_e[ty]);
        if (e < 0) return;
        const int mb = __builtin_amdgcn_readfirstlane(g.tile_mb[ty]);
        rows_valid = min(QBM, __builtin_amdgcn_readfirstlane(g.counts[e]) - mb * QBM);
        arow0 = int64_t(__builtin_amdgcn_readfirstlane(g.offsets[e])) + int64_t(mb) * QBM;
        wrow0 = int64_t(e) * g.N;
    } else {
        rows_valid = min(QBM, g.T_sh - ty * QBM);
        arow0 = int64_t(ty) * QBM;
        wrow0 = 0;
    }
    rows_valid = __builtin_amdgcn_readfirstlane(rows_valid);
    arow0 = int64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(arow0)))) |
            (int64_t(__builtin_amdgcn_readfirstlane(int(arow0 >> 32))) << 32);
    wrow0 = int64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(wrow0)))) |
            (int64_t(__builtin_amdgcn_readfirstlane(int(wrow0 >> 32))) << 32);
    if (rows_valid <= 0) return;

    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, wave = tid >> 6;
    const int K = g.K;
    const int a_row_bytes = 2 * K;
    const int n_slab = SWIGLU ? 2 * g.I : g.N;
    // rows past rows_valid and columns past the slab read as zero
    const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(src.A + arow0 * a_row_bytes), 0, rows_valid * a_row_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(src.w + wrow0 * src.row_bytes), 0, int(n_slab * src.row_bytes), 0x00020000);

    // Stage layout (one K tile of 64):
    //   A 16 KiB: row r's 128 bytes (limb hi K 0..63, limb lo K 0..63 as
    //     eight 16-byte chunks c = 4 limb + K/16) at r * 128, chunk c at
    //     physical slot c ^ ((r >> 1) & 7);
    //   B 16 KiB: tile column n's 64 bytes (four chunks c = K/16) at
    //     16384 + n * 64, chunk c at slot c ^ ((n >> 2) & 3).
    // The swizzles make every fragment read (32 rows or columns at one
    // chunk, 16 lanes per LDS cycle) hit 16 distinct 16-byte slots of the
    // bank window.  Each DMA instruction covers whole row segments: A 8 rows
    // x 128 bytes, B 16 columns x 64 bytes (lane i: 16 bytes at slot i).
    // In global memory A rows are [K/64][2][64] bytes (the quantisers write
    // that layout), B rows are the weight rows as stored.
    int a_off[4], b_off[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int ja = 4 * wave + j;
        const int r = 8 * ja + (lane >> 3), pc = lane & 7;
        a_off[j] = r * a_row_bytes + ((pc ^ ((r >> 1) & 7)) << 4);
        const int jb = 4 * wave + j;
        const int col = 16 * jb + (lane >> 2), pcb = lane & 3;
        const int nsub = col >> 5, x = col & 31;
        int row;
        if (SWIGLU) {
            // h columns [32 w', +32) of wave w' = nsub / 2: gate rows for
            // nsub even, up rows for nsub odd
            const int hc = min(nt * (QBN / 2) + (nsub >> 1) * 32 + x, g.I - 1);
            row = (nsub & 1) ? g.I + hc : hc;
        } else {
            row = min(nt * QBN + col, g.N - 1);
        }
        b_off[j] = row * int(src.row_bytes) + ((pcb ^ ((col >> 2) & 3)) << 4);
    }
    auto issue = [&](int t) {
        uint8_t* st = smem[t % kQStages];
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16<0>(rA, st + (4 * wave + j) * 1024, a_off[j], t * 128);
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16<2>(rB, st + 16384 + (4 * wave + j) * 1024, b_off[j], t * QBK);
    };
    // fragment read addresses inside a stage
    int fa_off[2][2][4], fb_off[2][2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int ch = 2 * ks + (lane >> 5);
#pragma unroll
        for (int l = 0; l < 2; ++l)
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) {
                const int r = mi * 32 + (lane & 31);
                fa_off[ks][l][mi] = r * 128 + (((4 * l + ch) ^ ((r >> 1) & 7)) << 4);
            }
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const int n = (2 * wave + ni) * 32 + (lane & 31);
            fb_off[ks][ni] = 16384 + n * 64 + ((ch ^ ((n >> 2) & 3)) << 4);
        }
    }

    i32x16 acc[2][4][2];
#pragma unroll
    for (int l = 0; l < 2; ++l)
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[l][mi][ni][v] = 0;

    const int nk = K / QBK;   // >= 3
    // Iteration t: tile t complete (this wave's loads are counted in order,
    // 8 per tile; then the barrier covers every wave's), which also retires
    // every wave's reads of tile t - 1, whose stage then takes tile t + 3;
    // tile t's 20 fragments are read at once (LDS latency paid once per
    // tile), then its 32 MFMAs run.
#pragma unroll
    for (int p = 0; p < kQStages - 1; ++p)
        if (p < nk) issue(p);
    for (int t = 0; t < nk; ++t) {
#ifdef GRIM_I8_TIMING
        const uint64_t tw0 = __builtin_amdgcn_s_memtime();
#endif
        const int later = min(kQStages - 2, nk - 1 - t);
        if (later >= 2) asm volatile("s_waitcnt vmcnt(16)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else if (later == 1) asm volatile("s_waitcnt vmcnt(8)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#ifdef GRIM_I8_TIMING
        const uint64_t tw1 = __builtin_amdgcn_s_memtime();
        g_i8_wait[blockIdx.x * 4 + wave] += tw1 - tw0;
#endif
        if (t + kQStages - 1 < nk) issue(t + kQStages - 1);
#ifdef GRIM_I8_TIMING
        g_i8_issue[blockIdx.x * 4 + wave] += __builtin_amdgcn_s_memtime() - tw1;
#endif
        const uint8_t* st = smem[t % kQStages];
        i32x4 fb[2][2], fa[2][2][4];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
                fb[ks][ni] = *reinterpret_cast<const i32x4*>(st + fb_off[ks][ni]);
#pragma unroll
            for (int l = 0; l < 2; ++l)
#pragma unroll
                for (int mi = 0; mi < 4; ++mi)
                    fa[ks][l][mi] = *reinterpret_cast<const i32x4*>(st + fa_off[ks][l][mi]);
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                    for (int l = 0; l < 2; ++l)
                        acc[l][mi][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[ks][l][mi], fb[ks][ni], acc[l][mi][ni], 0, 0, 0);
    }

#ifdef GRIM_I8_TIMING
    const uint64_t te0 = __builtin_amdgcn_s_memtime();
#endif
    // ---- epilogue.  acc[l][mi][ni][v] is row 32 mi + 8 (v/4) + 4 (l/32) +
    // v%4, column 32 (2 w + ni) + l%32 of the tile.  The tile goes through
    // LDS (the ring is idle now) so that global stores are whole rows, 16
    // bytes per lane; row scales through LDS too.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    float* srow = reinterpret_cast<float*>(smem[3] + 32768 - QBM * 4);
    if (tid < QBM) srow[tid] = tid < rows_valid ? src.sa[arow0 + tid] : 0.0f;
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    float* stg = reinterpret_cast<float*>(smem[0]);
    if constexpr (SWIGLU) {
        // h [128 rows][128 columns] fp32, row pitch 132 floats
        constexpr int P = QBN / 2 + 4;
        const int hcl = wave * 32 + (lane & 31);
        const int hc = nt * (QBN / 2) + hcl;
        const float sg = hc < g.I ? src.ws[wrow0 + hc] : 0.0f;
        const float su = hc < g.I ? src.ws[wrow0 + g.I + hc] : 0.0f;
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = mi * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                const float sr = srow[r];
                const float gv = sr * sg * __builtin_fmaf(float(acc[1][mi][0][v]), kLoScale, float(acc[0][mi][0][v]));
                const float uv = sr * su * __builtin_fmaf(float(acc[1][mi][1][v]), kLoScale, float(acc[0][mi][1][v]));
                stg[r * P + hcl] = fast_silu(gv) * uv;
            }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        // 128 rows x 32 chunks of 16 bytes: 16 per thread, a row per half-wave
        const int c0 = nt * (QBN / 2);
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int c = tid + k * kQThreads;
            const int r = c >> 5, part = c & 31;
            const int col = c0 + part * 4;
            if (r < rows_valid && col < g.I)
                *reinterpret_cast<float4*>(src.out + (arow0 + r) * g.I + col) =
                    *reinterpret_cast<const float4*>(&stg[r * P + part * 4]);
        }
    } else {
        // [128 rows][256 columns] fp32 in two halves of 64 rows, pitch 260
        constexpr int P = QBN + 4;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            if (half) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const int cl = wave * 64 + ni * 32 + (lane & 31);
                const int n = nt * QBN + cl;
                const float sc = n < g.N ? src.ws[wrow0 + n] : 0.0f;
#pragma unroll
                for (int mh = 0; mh < 2; ++mh) {
                    const int mi = 2 * half + mh;
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int r = mi * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                        stg[(r - 64 * half) * P + cl] =
                            srow[r] * sc * __builtin_fmaf(float(acc[1][mi][ni][v]), kLoScale, float(acc[0][mi][ni][v]));
                    }
                }
            }
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            // 64 rows x 64 chunks of 16 bytes: 16 per thread, a row per wave
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const int c = tid + k * kQThreads;
                const int rl = c >> 6, part = c & 63;
                const int r = 64 * half + rl;
                const int col = nt * QBN + part * 4;
                if (r < rows_valid && col < g.N)
                    *reinterpret_cast<float4*>(src.out + (arow0 + r) * g.N + col) =
                        *reinterpret_cast<const float4*>(&stg[rl * P + part * 4]);
            }
        }
    }
    // the ring is refilled by the next tile only after every wave's LDS
    // reads; its first wait also covers these stores (one in-order counter)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#ifdef GRIM_I8_TIMING
    g_i8_epi[blockIdx.x * 4 + wave] += __builtin_amdgcn_s_memtime() - te0;
#endif
}

template <bool SWIGLU>
__global__ __launch_bounds__(kQThreads, 1) void grouped_gemm_i8_kernel(GemmI8Args g, int n_col_tiles,
                                                                      int shared_part) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kQStages][kQStageBytes];
    const bool routed = shared_part == 0;
    const I8Src src{routed ? g.w : g.w_sh, routed ? g.ws : g.ws_sh,
                    routed ? g.row_bytes : g.row_bytes_sh, routed ? g.A : g.A_sh,
                    routed ? g.sa : g.sa_sh, routed ? g.out : g.out_sh};
    int total;
    if (routed) {
        total = g.n_tiles_dev ? __builtin_amdgcn_readfirstlane(*g.n_tiles_dev) : g.tmax;
        total = total < g.tmax ? total : g.tmax;
    } else {
        total = (g.T_sh + QBM - 1) / QBM;
    }
    // work-group b runs on XCD b % 8: each XCD walks a contiguous range of
    // the m-tile list, column tiles fastest, so an expert's weights and an
    // A row block stay under one L2
    const int xcd = blockIdx.x % kQXcds, per_xcd = gridDim.x / kQXcds;
    const int lo = int(int64_t(total) * xcd / kQXcds), hi = int(int64_t(total) * (xcd + 1) / kQXcds);
    const int items = (hi - lo) * n_col_tiles;
#ifdef GRIM_I8_TIMING
    const uint64_t t0 = __builtin_amdgcn_s_memtime();
#endif
    for (int i = blockIdx.x / kQXcds; i < items; i += per_xcd)
        i8_tile<SWIGLU>(g, src, routed, lo + i / n_col_tiles, i % n_col_tiles, smem);
#ifdef GRIM_I8_TIMING
    g_i8_total[blockIdx.x * 4 + threadIdx.x / 64] += __builtin_amdgcn_s_memtime() - t0;
#endif
}

// ------------------------------------------------------------ quantisers

// Row max, limbs, scale: one wave per row of n <= 4096 elements (8 per lane
// per step).  src fp32 [rows][n] -> dst limb rows [rows][n/64][2][64],
// scale [rows].
__device__ __forceinline__ void limbs8(const float (&v)[8], float inv, uint32_t& h0, uint32_t& h1,
                                       uint32_t& l0, uint32_t& l1) {
    uint32_t hb[8], lb[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float y = v[i] * inv;
        const float hq = __builtin_rintf(y);
        const float lq = __builtin_rintf((y - hq) * 254.0f);
        hb[i] = uint32_t(int(hq)) & 0xFF;
        lb[i] = uint32_t(int(fminf(fmaxf(lq, -127.0f), 127.0f))) & 0xFF;
    }
    h0 = hb[0] | (hb[1] << 8) | (hb[2] << 16) | (hb[3] << 24);
    h1 = hb[4] | (hb[5] << 8) | (hb[6] << 16) | (hb[7] << 24);
    l0 = lb[0] | (lb[1] << 8) | (lb[2] << 16) | (lb[3] << 24);
    l1 = lb[4] | (lb[5] << 8) | (lb[6] << 16) | (lb[7] << 24);
}

// Byte offset of element k's hi limb in a limb row [K/64][2][64] (the lo
// limb is 64 bytes further).
__device__ __forceinline__ int limb_block(int k) { return (k >> 6) * 128 + (k & 63); }

__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

constexpr int kQuantRowsPerBlock = 4;

__global__ __launch_bounds__(256) void quant_rows_kernel(const float* __restrict__ src, int rows,
                                                         int n, int8_t* __restrict__ dst,
                                                         float* __restrict__ scale) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * kQuantRowsPerBlock + threadIdx.x / 64;
    if (r >= rows) return;
    const float* s = src + int64_t(r) * n;
    float m = 0.0f;
    for (int c = lane * 8; c < n; c += 512) {
        const float4 a = *reinterpret_cast<const float4*>(s + c);
        const float4 b = *reinterpret_cast<const float4*>(s + c + 4);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        m = fmaxf(m, fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
    }
    m = wave_max_f(m);
    const float sc = m > 0.0f ? m / 127.0f : 1.0f;
    const float inv = m > 0.0f ? 127.0f / m : 0.0f;
    int8_t* d = dst + int64_t(r) * 2 * n;
    for (int c = lane * 8; c < n; c += 512) {
        const float4 a = *reinterpret_cast<const float4*>(s + c);
        const float4 b = *reinterpret_cast<const float4*>(s + c + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t h0, h1, l0, l1;
        limbs8(v, inv, h0, h1, l0, l1);
        int8_t* blk = d + limb_block(c);
        *reinterpret_cast<uint2*>(blk) = make_uint2(h0, h1);
        *reinterpret_cast<uint2*>(blk + 64) = make_uint2(l0, l1);
    }
    if (lane == 0) scale[r] = sc;
}

// The activations of every token as limbs, written to each of its K
// permuted rows (inverse) and to its own row (xrow, the shared expert's
// input) when given.  One work-group of 256 threads per token, n <= 8192.
__global__ __launch_bounds__(256) void quant_permute_kernel(const float* __restrict__ x, int n, int K,
                                                            const int32_t* __restrict__ inverse,
                                                            int8_t* __restrict__ xq, float* __restrict__ sq,
                                                            int8_t* __restrict__ xrowq,
                                                            float* __restrict__ srow) {
    __shared__ float red[4];
    const int t = blockIdx.x;
    const float* s = x + int64_t(t) * n;
    float4 va[4], vb[4];
    float m = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int c = threadIdx.x * 8 + q * 2048;
        if (c < n) {
            va[q] = *reinterpret_cast<const float4*>(s + c);
            vb[q] = *reinterpret_cast<const float4*>(s + c + 4);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(va[q].x), fabsf(va[q].y)), fmaxf(fabsf(va[q].z), fabsf(va[q].w))));
            m = fmaxf(m, fmaxf(fmaxf(fabsf(vb[q].x), fabsf(vb[q].y)), fmaxf(fabsf(vb[q].z), fabsf(vb[q].w))));
        }
    }
    m = wave_max_f(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x / 64] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = m > 0.0f ? m / 127.0f : 1.0f;
    const float inv = m > 0.0f ? 127.0f / m : 0.0f;
    int dst[16];
    for (int k = 0; k < K; ++k) dst[k] = inverse[int64_t(t) * K + k];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int c = threadIdx.x * 8 + q * 2048;
        if (c < n) {
            const float v[8] = {va[q].x, va[q].y, va[q].z, va[q].w, vb[q].x, vb[q].y, vb[q].z, vb[q].w};
            uint32_t h0, h1, l0, l1;
            limbs8(v, inv, h0, h1, l0, l1);
            for (int k = 0; k < K; ++k) {
                if (dst[k] < 0) continue;
                int8_t* d = xq + int64_t(dst[k]) * 2 * n + limb_block(c);
                *reinterpret_cast<uint2*>(d) = make_uint2(h0, h1);
                *reinterpret_cast<uint2*>(d + 64) = make_uint2(l0, l1);
            }
            if (xrowq) {
                int8_t* d = xrowq + int64_t(t) * 2 * n + limb_block(c);
                *reinterpret_cast<uint2*>(d) = make_uint2(h0, h1);
                *reinterpret_cast<uint2*>(d + 64) = make_uint2(l0, l1);
            }
        }
    }
    if (int(threadIdx.x) < K) {
        const int dk = inverse[int64_t(t) * K + threadIdx.x];
        if (dk >= 0) sq[dk] = sc;
    }
    if (srow && threadIdx.x == 0) srow[t] = sc;
}

// ----------------------------------------------------------------- host

template <bool SWIGLU>
static hipError_t launch_i8(hipStream_t st, const GemmI8Args& g, int ntiles) {
    static int grid = 0;
    if (grid == 0) {
        int per_cu = 0, dev = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, grouped_gemm_i8_kernel<SWIGLU>,
                                                         kQThreads, 0) != hipSuccess ||
            hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return hipErrorInvalidConfiguration;
        grid = (per_cu > 0 ? per_cu : 1) * cus;
        grid = (grid + kQXcds - 1) / kQXcds * kQXcds;
    }
    if (g.tmax > 0)
        hipLaunchKernelGGL(grouped_gemm_i8_kernel<SWIGLU>, dim3(grid), dim3(kQThreads), 0, st, g,
                           ntiles, 0);
    if (g.T_sh > 0) {
        const int items = (g.T_sh + QBM - 1) / QBM * ntiles;
        const int gs = min(grid, (items + kQXcds - 1) / kQXcds * kQXcds);
        hipLaunchKernelGGL(grouped_gemm_i8_kernel<SWIGLU>, dim3(gs), dim3(kQThreads), 0, st, g,
                           ntiles, 1);
    }
    return hipGetLastError();
}

bool gemm_i8_shape_ok(int N, int K, int I, int swiglu) {
    if (K % QBK || K < 3 * QBK || K > 8192) return false;
    if (swiglu) return I > 0 && N == 2 * I;
    return N > 0;
}

hipError_t gemm_i8_launch(hipStream_t st, const GemmI8Args& g) {
    if (!gemm_i8_shape_ok(g.N, g.K, g.I, g.swiglu)) return hipErrorInvalidValue;
    const int ntiles = g.swiglu ? (g.I + QBN / 2 - 1) / (QBN / 2) : (g.N + QBN - 1) / QBN;
    if (ntiles <= 0) return hipSuccess;
    return g.swiglu ? launch_i8<true>(st, g, ntiles) : launch_i8<false>(st, g, ntiles);
}

hipError_t quant_rows_launch(hipStream_t st, const float* src, int rows, int n, int8_t* dst,
                             float* scale) {
    if (rows <= 0) return hipSuccess;
    if (n % 64 || n > 4096) return hipErrorInvalidValue;
    hipLaunchKernelGGL(quant_rows_kernel, dim3((rows + kQuantRowsPerBlock - 1) / kQuantRowsPerBlock),
                       dim3(256), 0, st, src, rows, n, dst, scale);
    return hipGetLastError();
}

hipError_t quant_permute_launch(hipStream_t st, const float* x, int T, int n, int K,
                                const int32_t* inverse, int8_t* xq, float* sq, int8_t* xrowq,
                                float* srow) {
    if (T <= 0) return hipSuccess;
    if (n % 64 || n > 8192 || K > 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(quant_permute_kernel, dim3(T), dim3(256), 0, st, x, n, K, inverse, xq, sq,
                       xrowq, srow);
    return hipGetLastError();
}

}  // namespace grim
