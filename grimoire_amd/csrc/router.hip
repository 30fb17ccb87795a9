// router.hip -- router projection and top-k selection.
//
// The per-wave top-k itself lives in topk.hpp (shared with the fused decode
// kernel).
#include "common.hpp"
#include "router.hpp"
#include "topk.hpp"

#include <algorithm>
#include <type_traits>

namespace grim {

constexpr int kTopkWaves = 4;
typedef float f32x4n __attribute__((ext_vector_type(4)));   // native vector (HIP's float4 is a struct)
typedef uint32_t u32x4n __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kTopkWaves * kWave) void topk_kernel(
    const float* __restrict__ logits, int T, int E, int K, int mode, int normalize,
    float scaling, const uint16_t* __restrict__ bias16, const float* __restrict__ bias32,
    int n_group, int topk_group, int32_t* __restrict__ out_e, float* __restrict__ out_w) {
    __shared__ float gsel[kTopkWaves][512];
    __shared__ float gscore[kTopkWaves][64];
    const int wv = threadIdx.x / kWave;
    const int t = blockIdx.x * kTopkWaves + wv;
    if (t >= T) return;   // whole wave exits together
    topk_wave(logits + int64_t(t) * E, E, K, mode, normalize, scaling, bias16, bias32, n_group,
              topk_group, out_e + int64_t(t) * K, out_w + int64_t(t) * K, gsel[wv], gscore[wv]);
}

// The same on split-K router partials: logits = (a + b) + bias formed as
// they are loaded (the arithmetic of the router's own finishing pass, so
// the same bits), then the top-k.  The finished logits are not stored:
// nothing after the top-k reads them.
__global__ __launch_bounds__(kTopkWaves * kWave) void topk_split_kernel(
    const float* __restrict__ logits, const float* __restrict__ part1, const float* __restrict__ lbias,
    int T, int E, int K, int mode, int normalize,
    float scaling, const uint16_t* __restrict__ bias16, const float* __restrict__ bias32,
    int n_group, int topk_group, int32_t* __restrict__ out_e, float* __restrict__ out_w) {
    __shared__ float gsel[kTopkWaves][512];
    __shared__ float gscore[kTopkWaves][64];
    const int wv = threadIdx.x / kWave;
    const int t = blockIdx.x * kTopkWaves + wv;
    if (t >= T) return;   // whole wave exits together
    const int lane = threadIdx.x & (kWave - 1);
    const int V = (E + kWave - 1) / kWave;
    const float* row = logits + int64_t(t) * E;
    const float* row1 = part1 + int64_t(t) * E;
    float lv[kMaxV];
    if (E == kWave * kMaxV) {
        // every lane's kMaxV logits are contiguous: 16-byte loads and stores
#pragma unroll
        for (int j = 0; j < kMaxV; j += 4) {
            const int e = lane * kMaxV + j;
            f32x4n v = *reinterpret_cast<const f32x4n*>(row + e);
            const f32x4n q = *reinterpret_cast<const f32x4n*>(row1 + e);
            v = f32x4n{v.x + q.x, v.y + q.y, v.z + q.z, v.w + q.w};
            if (lbias) {
                const f32x4n b = *reinterpret_cast<const f32x4n*>(lbias + e);
                v = f32x4n{v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w};
            }
            lv[j] = v.x; lv[j + 1] = v.y; lv[j + 2] = v.z; lv[j + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < kMaxV; ++j) {
            const int e = lane * V + j;
            const int ec = (j < V && e < E) ? e : 0;
            float v = row[ec] + row1[ec];
            if (lbias) v += lbias[ec];
            lv[j] = v;
        }
    }
    topk_wave_regs(lv, E, K, mode, normalize, scaling, bias16, bias32, n_group, topk_group,
                   out_e + int64_t(t) * K, out_w + int64_t(t) * K, gsel[wv], gscore[wv]);
}

// launch_router_topk_bf16_batched (src/ops.cpp:1425-1480): the batched
// softmax top-k (mode 1) on bf16 logits
__global__ __launch_bounds__(kTopkWaves * kWave) void topk_bf16_kernel(
    const uint16_t* __restrict__ logits, int T, int E, int K, int normalize,
    int32_t* __restrict__ out_e, float* __restrict__ out_w) {
    __shared__ float gsel[kTopkWaves][512];
    __shared__ float gscore[kTopkWaves][64];
    const int wv = threadIdx.x / kWave;
    const int t = blockIdx.x * kTopkWaves + wv;
    if (t >= T) return;   // whole wave exits together
    float lv[kMaxV];
    topk_load(logits + int64_t(t) * E, E, lv);
    topk_wave_regs(lv, E, K, 1, normalize, 1.0f, nullptr, nullptr, 0, 0,
                   out_e + int64_t(t) * K, out_w + int64_t(t) * K, gsel[wv], gscore[wv]);
}

hipError_t topk_bf16_launch(hipStream_t st, const uint16_t* logits, int T, int E, int K,
                            int normalize, int32_t* out_e, float* out_w) {
    dim3 grid((T + kTopkWaves - 1) / kTopkWaves);
    hipLaunchKernelGGL(topk_bf16_kernel, grid, dim3(kTopkWaves * kWave), 0, st, logits, T, E, K,
                       normalize, out_e, out_w);
    return hipGetLastError();
}

hipError_t topk_launch(hipStream_t st, const TopkArgs& a) {
    dim3 grid((a.T + kTopkWaves - 1) / kTopkWaves);
    if (a.part1) {
        hipLaunchKernelGGL(topk_split_kernel, grid, dim3(kTopkWaves * kWave), 0, st,
                           a.logits, a.part1, a.lbias, a.T, a.E, a.K, a.mode,
                           a.normalize, a.scaling, a.bias16, a.bias32, a.n_group, a.topk_group, a.out_e,
                           a.out_w);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(topk_kernel, grid, dim3(kTopkWaves * kWave), 0, st, a.logits, a.T, a.E,
                       a.K, a.mode, a.normalize, a.scaling, a.bias16, a.bias32, a.n_group,
                       a.topk_group, a.out_e, a.out_w);
    return hipGetLastError();
}

// ---------------------------------------------------------- router logits

// Small T: one work-group per (expert row, kRouterTok tokens), the row
// streamed once with 16-byte loads (router_row); x read through the cache.
__global__ __launch_bounds__(256) void router_gemv(const float* __restrict__ W,
                                                   const float* __restrict__ x,
                                                   const float* __restrict__ bias,
                                                   float* __restrict__ logits, int T, int E,
                                                   int H) {
    __shared__ float red[4 * kRouterTok];
    const int e = blockIdx.x;
    const int t0 = blockIdx.y * kRouterTok;
    const int nt = T - t0 < kRouterTok ? T - t0 : kRouterTok;
    const float s = router_row(W + int64_t(e) * H, x + int64_t(t0) * H, nt, H, red);
    if (int(threadIdx.x) < nt) logits[int64_t(t0 + threadIdx.x) * E + e] = bias ? s + bias[e] : s;
}

// Small T, H <= 1024 NK: the arithmetic of router_row (thread i's chain over
// elements 4i + 1024m in m order, DPP wave sums, the four waves added in
// order), so the same bits, for EB experts x TT tokens per work-group: every
// load of the work-group's rows and tokens is issued before the products
// (addresses past H clamped to 0, their products not added), and x is read
// E / EB times instead of E times.
template <int NK, int EB, int TT>
__global__ __launch_bounds__(256) void router_gemv_nk(const float* __restrict__ W,
                                                      const float* __restrict__ x,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ logits, int T, int E, int H) {
    __shared__ float red[4 * EB * TT];
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int e0 = blockIdx.x * EB, t0 = blockIdx.y * TT;
    const int ne = min(EB, E - e0), nt = min(TT, T - t0);
    float4 wv[NK][EB], xv[NK][TT];
#pragma unroll
    for (int m = 0; m < NK; ++m) {
        const int k = int(threadIdx.x) * 4 + 1024 * m;
        const int kk = k < H ? k : 0;
#pragma unroll
        for (int j = 0; j < EB; ++j)
            wv[m][j] = *reinterpret_cast<const float4*>(W + int64_t(e0 + min(j, ne - 1)) * H + kk);
#pragma unroll
        for (int i = 0; i < TT; ++i)
            xv[m][i] = *reinterpret_cast<const float4*>(x + int64_t(t0 + min(i, nt - 1)) * H + kk);
    }
#pragma unroll
    for (int j = 0; j < EB; ++j) {
#pragma unroll
        for (int i = 0; i < TT; ++i) {
            float acc = 0.0f;
#pragma unroll
            for (int m = 0; m < NK; ++m) {
                const int k = int(threadIdx.x) * 4 + 1024 * m;
                float a2 = __builtin_fmaf(wv[m][j].x, xv[m][i].x, acc);
                a2 = __builtin_fmaf(wv[m][j].y, xv[m][i].y, a2);
                a2 = __builtin_fmaf(wv[m][j].z, xv[m][i].z, a2);
                a2 = __builtin_fmaf(wv[m][j].w, xv[m][i].w, a2);
                acc = k < H ? a2 : acc;
            }
            const float v = group_sum<kWave>(acc);
            if (lane == 0) red[(wave * EB + j) * TT + i] = v;
        }
    }
    __syncthreads();
    const int j = int(threadIdx.x) / TT, i = int(threadIdx.x) % TT;
    if (j < ne && i < nt) {
        const int q = j * TT + i, st = EB * TT;
        const float r = (red[q] + red[st + q]) + (red[2 * st + q] + red[3 * st + q]);
        const int e = e0 + j;
        logits[int64_t(t0 + i) * E + e] = bias ? r + bias[e] : r;
    }
}

template <int NK, int EB, int TT>
static void router_nk_go(hipStream_t st, const float* W, const float* x, const float* bias, float* logits, int T,
                         int E, int H) {
    const dim3 grid((E + EB - 1) / EB, (T + TT - 1) / TT);
    hipLaunchKernelGGL((router_gemv_nk<NK, EB, TT>), grid, dim3(256), 0, st, W, x, bias, logits, T, E, H);
}

// EB x TT per work-group, measured (rocprof, one MI355X): 2 x 4 for rows up
// to 5K (T=8, H=2880, E=128: 3.6 us; 2 x 8: 5.3; 1 x 8: 4.1), 4 x 4 for
// longer ones (T=32, H=7168, E=256: 9.0 us; 1 x 4: 12.8; 2 x 4: 10.2;
// 8 x 4: 11.7; 4 x 2: 10.2).
template <int NK>
static void router_nk_pick(hipStream_t st, const float* W, const float* x, const float* bias, float* logits, int T,
                           int E, int H) {
    if constexpr (NK <= 5) router_nk_go<NK, 2, 4>(st, W, x, bias, logits, T, E, H);
    else router_nk_go<NK, 4, 4>(st, W, x, bias, logits, T, E, H);
}

static bool router_nk_launch(hipStream_t st, const float* W, const float* x, const float* bias, float* logits,
                             int T, int E, int H) {
    switch ((H + 1023) / 1024) {
    case 1: router_nk_pick<1>(st, W, x, bias, logits, T, E, H); return true;
    case 2: router_nk_pick<2>(st, W, x, bias, logits, T, E, H); return true;
    case 3: router_nk_pick<3>(st, W, x, bias, logits, T, E, H); return true;
    case 4: router_nk_pick<4>(st, W, x, bias, logits, T, E, H); return true;
    case 5: router_nk_pick<5>(st, W, x, bias, logits, T, E, H); return true;
    case 6: router_nk_pick<6>(st, W, x, bias, logits, T, E, H); return true;
    case 7: router_nk_pick<7>(st, W, x, bias, logits, T, E, H); return true;
    case 8: router_nk_pick<8>(st, W, x, bias, logits, T, E, H); return true;
    default: return false;
    }
}

// Large T: LDS-tiled fp32 GEMM, 64 tokens x 64 experts per block, each
// thread a 4x4 register tile, K in steps of 16.
__global__ __launch_bounds__(256) void router_gemm(const float* __restrict__ W,
                                                   const float* __restrict__ x,
                                                   const float* __restrict__ bias,
                                                   float* __restrict__ logits, int T, int E,
                                                   int H) {
    __shared__ float xs[16][64 + 4];
    __shared__ float ws[16][64 + 4];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int t0 = blockIdx.y * 64, e0 = blockIdx.x * 64;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < H; k0 += 16) {
        for (int i = threadIdx.x; i < 64 * 16; i += 256) {
            const int r = i / 16, kk = i % 16;
            const int t = t0 + r, e = e0 + r;
            xs[kk][r] = (t < T && k0 + kk < H) ? x[int64_t(t) * H + k0 + kk] : 0.0f;
            ws[kk][r] = (e < E && k0 + kk < H) ? W[int64_t(e) * H + k0 + kk] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) { a[i] = xs[kk][ty * 4 + i]; b[i] = ws[kk][tx * 4 + i]; }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = t0 + ty * 4 + i, e = e0 + tx * 4 + j;
            if (t < T && e < E) logits[int64_t(t) * E + e] = bias ? acc[i][j] + bias[e] : acc[i][j];
        }
}

// Large T on MFMA: fp32 v_mfma_f32_32x32x2f32 (fp32 products and sums, no
// reduced-precision operands).  Block tile (64 MI) tokens x (64 NI) experts x
// 32 K, 4 waves of (32 MI) x (32 NI) (MI x NI MFMA tiles), LDS double buffer
// with a register prefetch of the next K tile.  Inside a 32-wide K tile lane
// half h supplies K = 16 h + s in MFMA step s (the same order for x and W),
// so each lane reads 16 consecutive floats per row with 16-byte LDS loads.
// MI = NI = 1 (64 x 64) is the default: T = 4096, E = 512 then gives 512
// blocks, two per CU, where 128 x 128 tiles would leave half the CUs idle.
constexpr int kRtBK = 32, kRtLD = kRtBK + 4;
typedef float f32x16r __attribute__((__vector_size__(16 * sizeof(float))));

// staging of one K tile: ROWS/32 f32x4n per thread from `src` (row c/8,
// K offset 4 (c % 8)); rows past `n` repeat the last one
template <int ROWS>
__device__ __forceinline__ void rt_load(const float* __restrict__ src, int n, int H, int r0,
                                        int k0, f32x4n (&reg)[ROWS / 32]) {
#pragma unroll
    for (int i = 0; i < ROWS / 32; ++i) {
        const int c = threadIdx.x + i * 256, r = c >> 3, kc = (c & 7) * 4;
        const int rr = min(r0 + r, n - 1);
        reg[i] = *reinterpret_cast<const f32x4n*>(src + int64_t(rr) * H + k0 + kc);
    }
}
template <int ROWS>
__device__ __forceinline__ void rt_store(float* dst, const f32x4n (&reg)[ROWS / 32]) {
#pragma unroll
    for (int i = 0; i < ROWS / 32; ++i) {
        const int c = threadIdx.x + i * 256, r = c >> 3, kc = (c & 7) * 4;
        *reinterpret_cast<f32x4n*>(&dst[r * kRtLD + kc]) = reg[i];
    }
}
template <int MI, int NI>
__global__ __launch_bounds__(256) void router_mfma(const float* __restrict__ W,
                                                   const float* __restrict__ x,
                                                   const float* __restrict__ bias,
                                                   float* __restrict__ logits, int T, int E, int H) {
    constexpr int BM = 64 * MI, BN = 64 * NI;
    __shared__ __attribute__((aligned(16))) float Xs[2][BM * kRtLD];
    __shared__ __attribute__((aligned(16))) float Ws[2][BN * kRtLD];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, h = lane >> 5;
    const int t0 = blockIdx.y * BM, e0 = blockIdx.x * BN;
    f32x4n rx[BM / 32], rw[BN / 32];
    f32x16r acc[MI][NI];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[mi][ni][v] = 0.0f;
    const int nk = H / kRtBK;
    rt_load<BM>(x, T, H, t0, 0, rx);
    rt_load<BN>(W, E, H, e0, 0, rw);
    rt_store<BM>(Xs[0], rx);
    rt_store<BN>(Ws[0], rw);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) {
            rt_load<BM>(x, T, H, t0, (kt + 1) * kRtBK, rx);
            rt_load<BN>(W, E, H, e0, (kt + 1) * kRtBK, rw);
        }
        float av[MI][16], bv[NI][16];
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
            const float* p = &Xs[buf][(wm * 32 * MI + mi * 32 + (lane & 31)) * kRtLD + 16 * h];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4n v4 = *reinterpret_cast<const f32x4n*>(p + 4 * q);
                av[mi][4 * q] = v4.x; av[mi][4 * q + 1] = v4.y; av[mi][4 * q + 2] = v4.z; av[mi][4 * q + 3] = v4.w;
            }
        }
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
            const float* p = &Ws[buf][(wn * 32 * NI + ni * 32 + (lane & 31)) * kRtLD + 16 * h];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4n v4 = *reinterpret_cast<const f32x4n*>(p + 4 * q);
                bv[ni][4 * q] = v4.x; bv[ni][4 * q + 1] = v4.y; bv[ni][4 * q + 2] = v4.z; bv[ni][4 * q + 3] = v4.w;
            }
        }
#pragma unroll
        for (int st = 0; st < 16; ++st)
#pragma unroll
            for (int mi = 0; mi < MI; ++mi)
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[mi][st], bv[ni][st], acc[mi][ni], 0, 0, 0);
        if (kt + 1 < nk) {
            rt_store<BM>(Xs[buf ^ 1], rx);
            rt_store<BN>(Ws[buf ^ 1], rw);
        }
        __syncthreads();
    }
    // acc[mi][ni][v]: token row (v&3) + 4*(lane>>5) + 8*(v>>2), expert lane&31
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
        const int e = e0 + wn * 32 * NI + ni * 32 + (lane & 31);
        if (e >= E) continue;
        const float b = bias ? bias[e] : 0.0f;
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int t = t0 + wm * 32 * MI + mi * 32 + (v & 3) + 4 * (lane >> 5) + 8 * (v >> 2);
                if (t < T) logits[int64_t(t) * E + e] = bias ? acc[mi][ni][v] + b : acc[mi][ni][v];
            }
    }
}

// Large T in three bf16 limbs: each fp32 value v splits exactly into
// hi + mid + lo (hi = bf16(v), mid = bf16(v - hi), lo = bf16(v - hi - mid):
// 24 significant bits in three 8-bit pieces), and
//     x . w = sum of xh.wh + xh.wm + xm.wh + xh.wl + xl.wh + xm.wm
// up to the three products below 2^-23 of the leading one (the size of an
// fp32 rounding), each product exact in fp32 and accumulated in fp32 by
// v_mfma_f32_32x32x16_bf16 -- 16x the fp32 MFMA's rate per product, 2.7x
// for the six.  Tile 64 tokens x 64 experts x 32 K, 4 waves of 32 x 32;
// the fp32 tiles are split while staged into LDS (three bf16 planes).
constexpr int kR3BK = 32, kR3LD = kR3BK + 8;   // LDS row pitch in bf16
typedef __bf16 bf16x8r __attribute__((__vector_size__(8 * sizeof(__bf16))));

// three limbs of 4 values as packed bf16 pairs: limb p -> out[p] (2 words);
// the bf16 conversions round to nearest even (one instruction per pair)
typedef __bf16 bf16x2r __attribute__((ext_vector_type(2)));
typedef float f32x2r __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bits(bf16x2r v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ f32x2r widen(bf16x2r v) {
    const uint32_t b = pk_bits(v);
    return f32x2r{__uint_as_float(b << 16), __uint_as_float(b & 0xFFFF0000u)};
}
__device__ __forceinline__ void split3(const f32x4n v, uint32_t (&out)[3][2]) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const f32x2r x = q ? f32x2r{v.z, v.w} : f32x2r{v.x, v.y};
        const bf16x2r h = __builtin_convertvector(x, bf16x2r);
        const f32x2r r1 = x - widen(h);
        const bf16x2r m = __builtin_convertvector(r1, bf16x2r);
        const f32x2r r2 = r1 - widen(m);
        const bf16x2r l = __builtin_convertvector(r2, bf16x2r);
        out[0][q] = pk_bits(h);
        out[1][q] = pk_bits(m);
        out[2][q] = pk_bits(l);
    }
}
__device__ __forceinline__ void r3_store(uint16_t* dst, int plane_stride, const f32x4n (&reg)[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = threadIdx.x + i * 256, r = c >> 3, kc = (c & 7) * 4;
        uint32_t w[3][2];
        split3(reg[i], w);
#pragma unroll
        for (int p = 0; p < 3; ++p)
            *reinterpret_cast<uint2*>(&dst[p * plane_stride + r * kR3LD + kc]) = make_uint2(w[p][0], w[p][1]);
    }
}

constexpr int kR3Pre = 4;   // K tiles in flight (register sets)

__global__ __launch_bounds__(256) void router_bf16x3(const float* __restrict__ W,
                                                     const float* __restrict__ x,
                                                     const float* __restrict__ bias,
                                                     float* __restrict__ logits, int T, int E, int H) {
    constexpr int PS = 64 * kR3LD;                    // one plane of one operand
    __shared__ __attribute__((aligned(16))) uint16_t Xs[2][3 * PS];
    __shared__ __attribute__((aligned(16))) uint16_t Ws[2][3 * PS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1, h = lane >> 5;
    // blockIdx.x = token block: work-group b runs on XCD b % 8, so the
    // column blocks of one token block share an XCD (and its L2 copy of x)
    const int t0 = blockIdx.x * 64, e0 = blockIdx.y * 64;
    // K tile j is loaded into register set j % kR3Pre, kR3Pre - 1 tiles
    // ahead of the one being multiplied (the latency of a tile's loads is
    // several tiles' worth of MFMA time)
    f32x4n rx[kR3Pre][2], rw[kR3Pre][2];
    f32x16r acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    const int nk = H / kR3BK;                         // a multiple of kR3Pre
#pragma unroll
    for (int j = 0; j < kR3Pre; ++j) {
        rt_load<64>(x, T, H, t0, j * kR3BK, rx[j]);
        rt_load<64>(W, E, H, e0, j * kR3BK, rw[j]);
    }
    r3_store(Xs[0], PS, rx[0]);
    r3_store(Ws[0], PS, rw[0]);
    __syncthreads();
    for (int k0 = 0; k0 < nk; k0 += kR3Pre) {
#pragma unroll
        for (int u = 0; u < kR3Pre; ++u) {
            const int kt = k0 + u, buf = kt & 1;
            // tile kt's set is free once it is in LDS: request tile kt + kR3Pre
            // (past the last tile the last again, never stored: loads under a
            // branch would make the compiler wait for every load in flight,
            // the ones just issued included, before each LDS store)
            const int kn = min(kt + kR3Pre, nk - 1) * kR3BK;
            rt_load<64>(x, T, H, t0, kn, rx[u]);
            rt_load<64>(W, E, H, e0, kn, rw[u]);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                // lane half h supplies K = 16 h + 8 ks .. + 7 (the same for x and W)
                const int kk = 16 * h + 8 * ks;
                bf16x8r a[3], b[3];
#pragma unroll
                for (int p = 0; p < 3; ++p) {
                    a[p] = *reinterpret_cast<const bf16x8r*>(&Xs[buf][p * PS + (wm * 32 + (lane & 31)) * kR3LD + kk]);
                    b[p] = *reinterpret_cast<const bf16x8r*>(&Ws[buf][p * PS + (wn * 32 + (lane & 31)) * kR3LD + kk]);
                }
                // smallest products first
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
            }
            if (kt + 1 < nk) {
                const int un = (u + 1) % kR3Pre;
                r3_store(Xs[buf ^ 1], PS, rx[un]);
                r3_store(Ws[buf ^ 1], PS, rw[un]);
            }
            __syncthreads();
        }
    }
    // acc[v]: token row (v&3) + 4*(lane>>5) + 8*(v>>2), expert lane&31
    const int e = e0 + wn * 32 + (lane & 31);
    if (e < E) {
        const float bb = bias ? bias[e] : 0.0f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int t = t0 + wm * 32 + (v & 3) + 4 * (lane >> 5) + 8 * (v >> 2);
            if (t < T) logits[int64_t(t) * E + e] = bias ? acc[v] + bb : acc[v];
        }
    }
}

// The same three-limb products on 128 x 128 tiles with K split in two
// halves (grid z).  At T = 4096, E = 512 a 64 x 64 tile per work-group reads
// its 64 x rows and 64 W rows over the whole K (2 MB per CU); a 128 x 128
// tile over half of K reads 1 MB.  The halves store their partial sums a
// (logits) and b (part1) for the caller to finish as (a + b) + bias, or,
// without part1, add them into zeroed logits by two float atomics
// (0 + a + b = a + b whichever lands first).
//
// The work is divided by wave, not by phase: loading a K tile, splitting
// it into limbs and storing the limb planes in LDS is vector-ALU and load
// work that one wave per SIMD cannot issue fast enough, and run in the same
// waves as the matrix products their times add.  Waves 4..11 (producers)
// load K tile kt + 3 into registers and store tile kt + 1 into the other LDS
// buffer while waves 0..3 (consumers, one per SIMD) run tile kt's products,
// one barrier per tile.  Consumer c owns tokens 64 (c / 2) .. + 64 and
// experts 64 (c % 2) .. + 64 of the tile (2 x 2 blocks of 32 x 32).
// IMG: W's limb planes come from router_wimg_kernel's image (split once per
// call, in K-tile order), so the producers only copy them; else the
// producers split W as they split x.  x is split only where it is not a
// bf16 value: a producer wave whose x pieces are all bf16 values stores the
// hi plane only and flags the tile clean; if some wave flags it, the
// consumers run the six products of router_bf16x3 in its order (mm, lh, hl,
// mh, hm, hh), else the three of x's one limb (hl, hm, hh) -- the skipped
// products are exact zeros.  x's mid / lo planes start at zero in both
// buffers; a wave clears its mid / lo pieces again only after a tile that
// had them.
constexpr int kRsBM = 128, kRsBN = 128, kRsPre = 3;
// producer waves: 4 copy the W image and handle x; 8 split W and x
template <bool IMG> constexpr int rs_prod() { return 8; }
template <bool IMG> constexpr int rs_threads() { return 64 * (4 + rs_prod<IMG>()); }
constexpr int kRsPlane = kRsBM * kR3LD;                       // bf16 per limb plane of one operand
constexpr size_t kRsLds = size_t(2) * 6 * kRsPlane * sizeof(uint16_t) + 2 * 8 * sizeof(int);
// W image: per (128-row expert block, K tile of 32), the three limb planes
// [plane][row][32] bf16 (24 KiB); rows past E repeat the last
constexpr int kRsImgPieces = 3 * kRsBN * kR3BK / 8;          // 16-byte pieces per block (1536)

size_t router_wimg_bytes(int T, int E, int H) {
    if (!(H % (2 * kR3BK) == 0 && H >= 2 * kR3BK * kRsPre && T >= 256)) return 0;
    return size_t((E + kRsBN - 1) / kRsBN) * (H / kR3BK) * kRsImgPieces * 16;
}

// One thread per 8 consecutive weights of a row: their three limbs, 16
// bytes per plane (split3, the split the GEMM would do).
__global__ __launch_bounds__(256) void router_wimg_kernel(const float* __restrict__ W, int E, int H,
                                                          uint4* __restrict__ img) {
    const int nkt = H / kR3BK, neb = (E + kRsBN - 1) / kRsBN;
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(neb) * nkt * (kRsBN * kR3BK / 8)) return;
    const int q = int(i % (kRsBN * kR3BK / 8));                  // row * 4 + 8-column group
    const int64_t blk = i / (kRsBN * kR3BK / 8);                 // eb * nkt + kt
    const int eb = int(blk / nkt), kt = int(blk % nkt);
    const int e = min(eb * kRsBN + (q >> 2), E - 1);
    const float* src = W + int64_t(e) * H + kt * kR3BK + (q & 3) * 8;
    uint32_t w0[3][2], w1[3][2];
    split3(*reinterpret_cast<const f32x4n*>(src), w0);
    split3(*reinterpret_cast<const f32x4n*>(src + 4), w1);
#pragma unroll
    for (int p = 0; p < 3; ++p)
        img[blk * kRsImgPieces + p * (kRsImgPieces / 3) + q] = make_uint4(w0[p][0], w0[p][1], w1[p][0], w1[p][1]);
}

// Barrier for LDS hand-offs: waits for the wave's own LDS accesses, not for
// its global loads in flight (a __syncthreads() fence would wait for those too).
__device__ __forceinline__ void rs_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <bool IMG>
__global__ __launch_bounds__(rs_threads<IMG>()) void router_bf16x3_ws(const float* __restrict__ W,
                                                               const uint4* __restrict__ wimg,
                                                               const float* __restrict__ x,
                                                               float* __restrict__ logits,
                                                               float* __restrict__ part1, int T, int E, int H) {
    constexpr int kRsProd = rs_prod<IMG>();
    constexpr int PS = kRsPlane, NP = 64 * kRsProd;
    extern __shared__ __attribute__((aligned(16))) uint16_t rs_lds[];
    uint16_t* Xs0 = rs_lds;                                   // [buf][plane][128][kR3LD]
    uint16_t* Ws0 = rs_lds + 2 * 3 * PS;
    int* wflag = reinterpret_cast<int*>(rs_lds + 4 * 3 * PS); // [buf][producer wave]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // blockIdx.x = token block (the expert blocks and K halves of one token
    // block share an XCD and its copy of x)
    const int t0 = blockIdx.x * kRsBM, e0 = blockIdx.y * kRsBN;
    const int nk = H / kR3BK / 2, kb = blockIdx.z * nk;
    if (wave >= 4) {
        // ---------------- producers: thread p's x pieces (and W pieces
        // without the image) are c = p + NP i: row c / 8, K 4 (c % 8) .. + 4
        const int p = tid - 256, pw = wave - 4;
        for (int i = p; i < 2 * 2 * PS / 4; i += NP) {
            const int b = i / (2 * PS / 4), o = i % (2 * PS / 4);
            reinterpret_cast<uint2*>(Xs0 + b * 3 * PS + PS)[o] = make_uint2(0u, 0u);
        }
        constexpr int NX = kRsBM * kR3BK / 4 / NP;                 // x pieces per thread (2)
        constexpr int NW = IMG ? kRsImgPieces / NP : NX;           // W pieces (3 image / 2 fp32)
        static_assert(NX * NP * 4 == kRsBM * kR3BK && (!IMG || NW * NP == kRsImgPieces), "pieces");
        typedef typename std::conditional<IMG, u32x4n, f32x4n>::type WPiece;
        f32x4n rx[kRsPre][NX];
        WPiece rv[kRsPre][NW];
        const u32x4n* wblk = IMG ? reinterpret_cast<const u32x4n*>(wimg) + int64_t(blockIdx.y) * (H / kR3BK) * kRsImgPieces
                                  : nullptr;
        auto load = [&](int kt, f32x4n (&ax)[NX], WPiece (&aw)[NW]) {
            const int k0 = (kb + kt) * kR3BK;
#pragma unroll
            for (int i = 0; i < NX; ++i) {
                const int c = p + NP * i, r = c >> 3, kc = (c & 7) * 4;
                ax[i] = *reinterpret_cast<const f32x4n*>(x + int64_t(min(t0 + r, T - 1)) * H + k0 + kc);
            }
#pragma unroll
            for (int i = 0; i < NW; ++i) {
                if constexpr (IMG) {
                    aw[i] = wblk[int64_t(kb + kt) * kRsImgPieces + p + NP * i];
                } else {
                    const int c = p + NP * i, r = c >> 3, kc = (c & 7) * 4;
                    aw[i] = *reinterpret_cast<const f32x4n*>(W + int64_t(min(e0 + r, E - 1)) * H + k0 + kc);
                }
            }
        };
        int dirty = 0;   // bit b: this wave left x mid / lo pieces in buffer b
        auto store = [&](int buf, const f32x4n (&ax)[NX], const WPiece (&aw)[NW]) {
            uint16_t* xs = Xs0 + buf * 3 * PS;
            uint16_t* ws = Ws0 + buf * 3 * PS;
            uint32_t any = 0;
#pragma unroll
            for (int i = 0; i < NX; ++i)
                any |= (__float_as_uint(ax[i].x) | __float_as_uint(ax[i].y) | __float_as_uint(ax[i].z) |
                        __float_as_uint(ax[i].w)) & 0xFFFFu;
            const bool full = __ballot(any != 0u) != 0;   // uniform
#pragma unroll
            for (int i = 0; i < NX; ++i) {
                const int c = p + NP * i, o = (c >> 3) * kR3LD + (c & 7) * 4;
                if (full) {
                    uint32_t w[3][2];
                    split3(ax[i], w);
#pragma unroll
                    for (int q = 0; q < 3; ++q)
                        *reinterpret_cast<uint2*>(&xs[q * PS + o]) = make_uint2(w[q][0], w[q][1]);
                } else {
                    // bf16 values: the hi limb is the upper half of each word
                    const uint32_t h0 = __builtin_amdgcn_perm(__float_as_uint(ax[i].y), __float_as_uint(ax[i].x),
                                                              0x07060302u);
                    const uint32_t h1 = __builtin_amdgcn_perm(__float_as_uint(ax[i].w), __float_as_uint(ax[i].z),
                                                              0x07060302u);
                    *reinterpret_cast<uint2*>(&xs[o]) = make_uint2(h0, h1);
                    if (dirty & (1 << buf)) {
                        *reinterpret_cast<uint2*>(&xs[PS + o]) = make_uint2(0u, 0u);
                        *reinterpret_cast<uint2*>(&xs[2 * PS + o]) = make_uint2(0u, 0u);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < NW; ++i) {
                if constexpr (IMG) {
                    // image piece q: plane q / 512, row (q % 512) / 4, columns 8 (q % 4) .. + 8
                    const int q = p + NP * i;
                    *reinterpret_cast<u32x4n*>(&ws[(q >> 9) * PS + ((q & 511) >> 2) * kR3LD + (q & 3) * 8]) = aw[i];
                } else {
                    const int c = p + NP * i, o = (c >> 3) * kR3LD + (c & 7) * 4;
                    uint32_t w[3][2];
                    split3(aw[i], w);
#pragma unroll
                    for (int q = 0; q < 3; ++q)
                        *reinterpret_cast<uint2*>(&ws[q * PS + o]) = make_uint2(w[q][0], w[q][1]);
                }
            }
            dirty = full ? (dirty | (1 << buf)) : (dirty & ~(1 << buf));
            if (lane == 0) wflag[buf * kRsProd + pw] = full ? 1 : 0;
        };
#pragma unroll
        for (int j = 0; j < kRsPre; ++j) load(min(j, nk - 1), rx[j], rv[j]);
        store(0, rx[0], rv[0]);
        rs_barrier();
        for (int k0 = 0; k0 < nk; k0 += kRsPre) {
#pragma unroll
            for (int u = 0; u < kRsPre; ++u) {
                const int kt = k0 + u;
                if (kt >= nk) break;
                // set u held tile kt (stored already): request tile kt + kRsPre
                // (past the end the last again, never stored: loads under a
                // branch would make the compiler wait for every load in flight)
                load(min(kt + kRsPre, nk - 1), rx[u], rv[u]);
                if (kt + 1 < nk) store((kt + 1) & 1, rx[(u + 1) % kRsPre], rv[(u + 1) % kRsPre]);
                rs_barrier();
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }
    // ---------------- consumers
    const int wm = wave >> 1, wn = wave & 1, h = lane >> 5;
    f32x16r acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[mi][ni][v] = 0.0f;
    rs_barrier();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        const uint16_t* xs = Xs0 + buf * 3 * PS;
        const uint16_t* ws = Ws0 + buf * 3 * PS;
        // both K steps' fragments of the planes every tile uses, and the
        // flags, issued together (lane half h supplies K = 16 h + 8 ks .. + 7,
        // the same for x and W); x's mid / lo planes after, when flagged
        bf16x8r a[2][2], b[2][2][3];   // [ks][mi] hi plane, [ks][ni][plane]
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int kk = 16 * h + 8 * ks;
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
                a[ks][mi] = *reinterpret_cast<const bf16x8r*>(&xs[(wm * 64 + mi * 32 + (lane & 31)) * kR3LD + kk]);
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                for (int q = 0; q < 3; ++q)
                    b[ks][ni][q] = *reinterpret_cast<const bf16x8r*>(
                        &ws[q * PS + (wn * 64 + ni * 32 + (lane & 31)) * kR3LD + kk]);
        }
        int fl = 0;
#pragma unroll
        for (int w = 0; w < kRsProd; ++w) fl |= wflag[buf * kRsProd + w];
        const bool full = fl != 0;   // uniform
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            // per accumulator: mm, lh, hl, mh, hm, hh (router_bf16x3's order)
            bf16x8r am[2], al[2];   // x's mid / lo planes (full tiles only)
            if (full) {
#pragma unroll
                for (int mi = 0; mi < 2; ++mi) {
                    const uint16_t* xa = &xs[(wm * 64 + mi * 32 + (lane & 31)) * kR3LD + 16 * h + 8 * ks];
                    am[mi] = *reinterpret_cast<const bf16x8r*>(xa + PS);
                    al[mi] = *reinterpret_cast<const bf16x8r*>(xa + 2 * PS);
                }
#pragma unroll
                for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                    for (int ni = 0; ni < 2; ++ni) {
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am[mi], b[ks][ni][1], acc[mi][ni], 0, 0, 0);
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[mi], b[ks][ni][0], acc[mi][ni], 0, 0, 0);
                    }
            }
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks][mi], b[ks][ni][2], acc[mi][ni], 0, 0, 0);
            if (full) {
#pragma unroll
                for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                    for (int ni = 0; ni < 2; ++ni)
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am[mi], b[ks][ni][0], acc[mi][ni], 0, 0, 0);
            }
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks][mi], b[ks][ni][1], acc[mi][ni], 0, 0, 0);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks][mi], b[ks][ni][0], acc[mi][ni], 0, 0, 0);
        }
        rs_barrier();
    }
    // acc[mi][ni][v]: token row (v&3) + 4*(lane>>5) + 8*(v>>2), expert lane&31
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const int e = e0 + wn * 64 + ni * 32 + (lane & 31);
            if (e >= E) continue;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int t = t0 + wm * 64 + mi * 32 + (v & 3) + 4 * (lane >> 5) + 8 * (v >> 2);
                if (t >= T) continue;
                if (part1) (blockIdx.z == 0 ? logits : part1)[int64_t(t) * E + e] = acc[mi][ni][v];
                else unsafeAtomicAdd(&logits[int64_t(t) * E + e], acc[mi][ni][v]);
            }
        }
}

// logits = 0 (bias null) or logits += bias, four values per thread when E
// is a multiple of 4
__global__ __launch_bounds__(256) void router_fill_kernel(float* __restrict__ logits, const float* __restrict__ bias,
                                                          int64_t n, int E, const float* __restrict__ part1) {
    const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    if (E % 4 == 0) {
        f32x4n v = f32x4n{0.0f, 0.0f, 0.0f, 0.0f};
        if (bias || part1) v = *reinterpret_cast<const f32x4n*>(logits + i);
        if (part1) {
            const f32x4n q = *reinterpret_cast<const f32x4n*>(part1 + i);
            v = f32x4n{v.x + q.x, v.y + q.y, v.z + q.z, v.w + q.w};
        }
        if (bias) {
            const f32x4n b = *reinterpret_cast<const f32x4n*>(bias + i % E);
            v = f32x4n{v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w};
        }
        *reinterpret_cast<f32x4n*>(logits + i) = v;
    } else {
        for (int64_t k = i; k < min(n, i + 4); ++k) {
            float v = (bias || part1) ? logits[k] : 0.0f;
            if (part1) v += part1[k];
            if (bias) v += bias[k % E];
            logits[k] = v;
        }
    }
}

hipError_t router_logits_launch(hipStream_t st, const float* W, const float* x,
                                const float* bias, float* logits, int T, int E, int H, float* part1,
                                int* deferred, void* wimg) {
    if (deferred) *deferred = 0;
    if (T <= 32 && H % 4 == 0 && router_nk_launch(st, W, x, bias, logits, T, E, H)) {
    } else if (T <= 32 && H % 4 == 0) {
        dim3 grid(E, (T + kRouterTok - 1) / kRouterTok);
        hipLaunchKernelGGL(router_gemv, grid, dim3(256), 0, st, W, x, bias, logits, T, E, H);
    } else if (H % (2 * kR3BK) == 0 && H >= 2 * kR3BK * kRsPre && T >= 256) {
        // split K.  With part1 and deferred: the halves store a (logits) and
        // b (part1), and the caller finishes (a + b) + bias (the top-k's
        // loads do it).  Otherwise: zero the logits, both halves add into
        // them (0 + a + b = a + b in either order), then the bias.
        const int64_t n = int64_t(T) * E;
        const unsigned fb = unsigned((n + 1023) / 1024);
        // (wimg: W's limb planes split once here by router_wimg_kernel,
        // router_wimg_bytes(T, E, H) bytes, 16-byte aligned)
        dim3 grid((T + kRsBM - 1) / kRsBM, (E + kRsBN - 1) / kRsBN, 2);
        const uint4* img = static_cast<const uint4*>(wimg);
        if (img && (reinterpret_cast<uintptr_t>(img) & 15)) return hipErrorInvalidValue;
        if (img) {
            const int64_t nt = int64_t((E + kRsBN - 1) / kRsBN) * (H / kR3BK) * (kRsBN * kR3BK / 8);
            hipLaunchKernelGGL(router_wimg_kernel, dim3(unsigned((nt + 255) / 256)), dim3(256), 0, st, W, E, H,
                               static_cast<uint4*>(wimg));
        }
        auto gemm = [&](float* p1) {
            if (img)
                hipLaunchKernelGGL(router_bf16x3_ws<true>, grid, dim3(rs_threads<true>()), kRsLds, st, W, img, x, logits,
                                   p1, T, E, H);
            else
                hipLaunchKernelGGL(router_bf16x3_ws<false>, grid, dim3(rs_threads<false>()), kRsLds, st, W, img, x, logits,
                                   p1, T, E, H);
        };
        if (part1 && deferred) {
            gemm(part1);
            *deferred = 1;
            return hipGetLastError();
        }
        hipLaunchKernelGGL(router_fill_kernel, dim3(fb), dim3(256), 0, st, logits, nullptr, n, E,
                           static_cast<const float*>(nullptr));
        gemm(nullptr);
        if (bias)
            hipLaunchKernelGGL(router_fill_kernel, dim3(fb), dim3(256), 0, st, logits, bias, n, E,
                               static_cast<const float*>(nullptr));
    } else if (H % (kR3BK * kR3Pre) == 0) {
        dim3 grid((T + 63) / 64, (E + 63) / 64);
        hipLaunchKernelGGL(router_bf16x3, grid, dim3(256), 0, st, W, x, bias, logits, T, E, H);
    } else if (H % kRtBK == 0) {
        dim3 grid((E + 63) / 64, (T + 63) / 64);
        hipLaunchKernelGGL((router_mfma<1, 1>), grid, dim3(256), 0, st, W, x, bias, logits, T, E, H);
    } else {
        dim3 grid((E + 63) / 64, (T + 63) / 64);
        hipLaunchKernelGGL(router_gemm, grid, dim3(256), 0, st, W, x, bias, logits, T, E, H);
    }
    return hipGetLastError();
}

hipError_t router_finish_launch(hipStream_t st, float* logits, const float* part1, const float* bias, int T,
                                int E) {
    const int64_t n = int64_t(T) * E;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(router_fill_kernel, dim3(unsigned((n + 1023) / 1024)), dim3(256), 0, st, logits, bias, n, E,
                       part1);
    return hipGetLastError();
}

}  // namespace grim

namespace grim {

// gate[t] = sigmoid(x_t . w) with w bf16 [H]; one wave per token
// (launch_rowdot_sigmoid, src/kernels.hpp:580; formula of
// src/moe_kernels.cpp:162-172).
__global__ __launch_bounds__(256) void rowdot_sigmoid(const float* __restrict__ x,
                                                      const uint16_t* __restrict__ w,
                                                      float* __restrict__ gate, int T, int H) {
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * 4 + threadIdx.x / kWave;
    if (t >= T) return;
    float a = 0.0f;
    for (int c = lane; c < H; c += kWave) a = __builtin_fmaf(bf16_to_f32(w[c]), x[int64_t(t) * H + c], a);
    a = group_sum<kWave>(a);
    if (lane == 0) gate[t] = det_sigmoid(a);
}

// The same with 4 columns per lane per step (float4 of x, four bf16 of w)
// and the row's loads unrolled 8 deep, so a wave has a whole 2048-wide row
// in flight instead of one dependent 4-byte load per step.  H % 4 == 0,
// x rows 16-byte and w 8-byte aligned.
__global__ __launch_bounds__(256) void rowdot_sigmoid4(const float* __restrict__ x,
                                                       const uint16_t* __restrict__ w,
                                                       float* __restrict__ gate, int T, int H) {
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * 4 + threadIdx.x / kWave;
    if (t >= T) return;
    const float* xr = x + int64_t(t) * H;
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll 8
    for (int c = lane * 4; c < H; c += kWave * 4) {
        const float4 v = *reinterpret_cast<const float4*>(xr + c);
        const uint2 u = *reinterpret_cast<const uint2*>(w + c);
        a0 = __builtin_fmaf(bits_f(u.x << 16), v.x, a0);
        a1 = __builtin_fmaf(bits_f(u.x & 0xFFFF0000u), v.y, a1);
        a2 = __builtin_fmaf(bits_f(u.y << 16), v.z, a2);
        a3 = __builtin_fmaf(bits_f(u.y & 0xFFFF0000u), v.w, a3);
    }
    float a = (a0 + a1) + (a2 + a3);
    a = group_sum<kWave>(a);
    if (lane == 0) gate[t] = det_sigmoid(a);
}

hipError_t rowdot_sigmoid_launch(hipStream_t st, const float* x, const uint16_t* w, float* gate,
                                 int T, int H) {
    if (H % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(w) & 7) == 0)
        hipLaunchKernelGGL(rowdot_sigmoid4, dim3((T + 3) / 4), dim3(256), 0, st, x, w, gate, T, H);
    else
        hipLaunchKernelGGL(rowdot_sigmoid, dim3((T + 3) / 4), dim3(256), 0, st, x, w, gate, T, H);
    return hipGetLastError();
}

}  // namespace grim
