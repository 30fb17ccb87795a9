// gemv.hip -- decode / batched-decode MoE expert products (slot form).
//
// Two launches per layer, as the reference's fused decode design
// (include/b70/moe.hpp:26-45, src/moe_kernels.cpp:82-445), re-laid out for
// CDNA4 wave64:
//
//   gate_up  grid (KS*row_blocks [+1 gate block], M).  A work-group stages
//            its token's x (fp32) and per-chunk sums of x in LDS.  Each
//            lane owns 16-byte chunks of LPR-lane row groups; a lane holds
//            RU (gate, up) row pairs, so 2*RU independent 16-byte loads are
//            in flight per chunk.  h = silu(g) * u.
//   down     grid (row_blocks over H, M).  h[t] (KS*I fp32) is staged in
//            LDS once per work-group; each lane group walks the slots in
//            slot order and keeps w_s * partial in registers, reducing
//            across the LPR lanes once at the end (linear, like
//            src/moe_kernels.cpp:415-423).
//
// The routing table is read on the device (src/moe_kernels.cpp:32-40), so
// per-token routing needs no host round trip.
#include "common.hpp"
#include "gemv.hpp"

namespace grim {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;

template <int F>
__device__ __forceinline__ void load_chunk_x(const float* __restrict__ xl, int c, float* xv) {
    constexpr int CH = Chunk<F>::CH;
    const float4* p = reinterpret_cast<const float4*>(xl + c * CH);
#pragma unroll
    for (int i = 0; i < CH / 4; ++i) {
        const float4 v = p[i];
        xv[4 * i + 0] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
    }
}

// Stage n floats of src and the per-chunk sums into LDS.
template <int F>
__device__ __forceinline__ void stage_vec(const float* __restrict__ src, int n, float* xl, float* xs) {
    constexpr int CH = Chunk<F>::CH;
    for (int i = threadIdx.x; i < n; i += blockDim.x) xl[i] = src[i];
    __syncthreads();
    if constexpr (Chunk<F>::kOffset) {
        const int nc = n / CH;
        for (int c = threadIdx.x; c < nc; c += blockDim.x) {
            float s = 0.0f;
            for (int i = 0; i < CH; ++i) s += xl[c * CH + i];
            xs[c] = s;
        }
        __syncthreads();
    }
}

template <int F, int LPR, int RU, bool SH>
__global__ __launch_bounds__(kGemvThreads) void moe_gate_up_slots(
    WView w, WView ws, const int32_t* __restrict__ rex, const float* __restrict__ x,
    float* __restrict__ h, const uint16_t* __restrict__ gate_w, float* __restrict__ gate_out,
    int H, int I, int K, int E, int row_blocks) {
    extern __shared__ float lds[];
    constexpr int CH = Chunk<F>::CH;
    constexpr int GPW = kWave / LPR;                 // row groups per wave
    constexpr int RB = kGemvWaves * GPW * RU;        // row pairs per block
    const int KS = K + (SH ? 1 : 0);
    const int C = H / CH;
    const int t = blockIdx.y;
    const float* xt = x + int64_t(t) * H;

    float* xl = lds;
    float* xs = lds + H;
    stage_vec<F>(xt, H, xl, xs);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int b = blockIdx.x;

    if (b == KS * row_blocks) {
        // shared_expert_gate: sigmoid(x . gate_w)  (src/moe_kernels.cpp:162-172)
        if (wave == 0) {
            float a = 0.0f;
            for (int c = lane; c < H; c += kWave) a = __builtin_fmaf(bf16_to_f32(gate_w[c]), xl[c], a);
            a = group_sum<kWave>(a);
            if (lane == 0) gate_out[t] = det_sigmoid(a);
        }
        return;
    }
    const int slot = b / row_blocks;
    const int i0 = (b % row_blocks) * RB + (wave * GPW + lane / LPR) * RU;
    const bool shr = SH && slot >= K;
    const WView& wv = w;
    int64_t gbase = 0;
    if (!shr) {
        const int e = rex[int64_t(t) * K + slot];
        if (e < 0 || e >= E) {
            // a route not computed here (expert-parallel remap uses -1): h = 0
            if ((lane % LPR) == 0)
                for (int r = 0; r < RU; ++r)
                    if (i0 + r < I) h[(int64_t(t) * KS + slot) * I + i0 + r] = 0.0f;
            return;
        }
        gbase = int64_t(e) * 2 * I;
    }

    float ga[RU], ua[RU];
#pragma unroll
    for (int r = 0; r < RU; ++r) { ga[r] = 0.0f; ua[r] = 0.0f; }

    auto run = [&](const WView& v) {
        for (int c = lane % LPR; c < C; c += LPR) {
            float xv[CH];
            load_chunk_x<F>(xl, c, xv);
            const float xsum = Chunk<F>::kOffset ? xs[c] : 0.0f;
            u32x4 rg[RU], ru[RU];
#pragma unroll
            for (int r = 0; r < RU; ++r) {
                const int i = i0 + r < I ? i0 + r : I - 1;
                rg[r] = load16(v.payload + (gbase + i) * v.row_bytes + int64_t(c) * 16);
                ru[r] = load16(v.payload + (gbase + I + i) * v.row_bytes + int64_t(c) * 16);
            }
#pragma unroll
            for (int r = 0; r < RU; ++r) {
                const int i = i0 + r < I ? i0 + r : I - 1;
                ga[r] += chunk_scaled<F>(v, gbase + i, c, rg[r], xv, xsum);
                ua[r] += chunk_scaled<F>(v, gbase + I + i, c, ru[r], xv, xsum);
            }
        }
#pragma unroll
        for (int r = 0; r < RU; ++r) {
            const int i = i0 + r < I ? i0 + r : I - 1;
            ga[r] *= row_scale<F>(v, gbase + i);
            ua[r] *= row_scale<F>(v, gbase + I + i);
        }
    };
    if (SH && shr) run(ws);
    else run(wv);

#pragma unroll
    for (int r = 0; r < RU; ++r) {
        const float g = group_sum<LPR>(ga[r]);
        const float u = group_sum<LPR>(ua[r]);
        const int i = i0 + r;
        if ((lane % LPR) == 0 && i < I) h[(int64_t(t) * KS + slot) * I + i] = silu(g) * u;
    }
}

template <int F, int LPR, int RU, bool SH>
__global__ __launch_bounds__(kGemvThreads) void moe_down_slots(
    WView w, WView wd, const int32_t* __restrict__ rex, const float* __restrict__ rwt,
    const float* __restrict__ gate_in, const float* __restrict__ h, float* __restrict__ y,
    int H, int I, int K, int E) {
    extern __shared__ float lds[];
    constexpr int CH = Chunk<F>::CH;
    constexpr int GPW = kWave / LPR;
    const int KS = K + (SH ? 1 : 0);
    const int C = I / CH;
    const int t = blockIdx.y;

    float* hl = lds;
    float* hs = lds + KS * I;
    {
        const float* ht = h + int64_t(t) * KS * I;
        for (int i = threadIdx.x; i < KS * I; i += blockDim.x) hl[i] = ht[i];
        __syncthreads();
        if constexpr (Chunk<F>::kOffset) {
            for (int c = threadIdx.x; c < KS * C; c += blockDim.x) {
                float s = 0.0f;
                for (int i = 0; i < CH; ++i) s += hl[c * CH + i];
                hs[c] = s;
            }
            __syncthreads();
        }
    }
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    constexpr int RB = kGemvWaves * GPW * RU;
    const int o0 = blockIdx.x * RB + (wave * GPW + lane / LPR) * RU;

    float total[RU];
#pragma unroll
    for (int r = 0; r < RU; ++r) total[r] = 0.0f;

    auto slot_dot = [&](const WView& v, int64_t ebase, int s, float rw) {
        float acc[RU];
#pragma unroll
        for (int r = 0; r < RU; ++r) acc[r] = 0.0f;
        const float* hv_s = hl + s * I;
        for (int c = lane % LPR; c < C; c += LPR) {
            float hv[CH];
            load_chunk_x<F>(hv_s, c, hv);
            const float hsum = Chunk<F>::kOffset ? hs[s * C + c] : 0.0f;
            u32x4 raw[RU];
#pragma unroll
            for (int r = 0; r < RU; ++r) {
                const int o = o0 + r < H ? o0 + r : H - 1;
                raw[r] = load16(v.payload + (ebase + o) * v.row_bytes + int64_t(c) * 16);
            }
#pragma unroll
            for (int r = 0; r < RU; ++r) {
                const int o = o0 + r < H ? o0 + r : H - 1;
                acc[r] += chunk_scaled<F>(v, ebase + o, c, raw[r], hv, hsum);
            }
        }
#pragma unroll
        for (int r = 0; r < RU; ++r) {
            const int o = o0 + r < H ? o0 + r : H - 1;
            total[r] = __builtin_fmaf(rw, acc[r] * row_scale<F>(v, ebase + o), total[r]);
        }
    };
    for (int s = 0; s < K; ++s) {
        const int64_t route = int64_t(t) * K + s;
        const int e = rex[route];
        const float rw = rwt[route];
        if (e < 0 || e >= E || rw == 0.0f) continue;
        slot_dot(w, int64_t(e) * H, s, rw);
    }
    if constexpr (SH) slot_dot(wd, 0, K, gate_in ? gate_in[t] : 1.0f);

#pragma unroll
    for (int r = 0; r < RU; ++r) {
        const float v = group_sum<LPR>(total[r]);
        const int o = o0 + r;
        if ((lane % LPR) == 0 && o < H) y[int64_t(t) * H + o] = v;
    }
}

// ------------------------------------------------------------------ host

static int pick_lpr(int chunks) {
    int l = 8;
    while (l < 64 && l < chunks) l <<= 1;
    return l;
}

int chunk_elems(int fmt) {
    switch (fmt) {
    case GRIM_FMT_BF16: return Chunk<GRIM_FMT_BF16>::CH;
    case GRIM_FMT_INT8: return Chunk<GRIM_FMT_INT8>::CH;
    case GRIM_FMT_INT4:
    case GRIM_FMT_INT4_F16: return Chunk<GRIM_FMT_INT4>::CH;
    case GRIM_FMT_MXFP4: return Chunk<GRIM_FMT_MXFP4>::CH;
    }
    return 0;
}

constexpr int kRuGU = 2;
constexpr int kRuDN = 2;

template <int F, int LPR, bool SH>
static hipError_t launch_gu_t(hipStream_t st, const GemvArgs& a) {
    constexpr int RB = kGemvWaves * (kWave / LPR) * kRuGU;
    const int KS = a.K + (SH ? 1 : 0);
    const int row_blocks = (a.I + RB - 1) / RB;
    const int C = a.H / Chunk<F>::CH;
    dim3 grid(KS * row_blocks + (a.gate_w ? 1 : 0), a.M);
    const size_t lds = size_t(a.H + C) * sizeof(float);
    hipLaunchKernelGGL((moe_gate_up_slots<F, LPR, kRuGU, SH>), grid, dim3(kGemvThreads), lds, st,
                       a.w, a.ws, a.rex, a.x, a.h, a.gate_w, a.gate_out, a.H, a.I, a.K, a.E,
                       row_blocks);
    return hipGetLastError();
}

template <int F, int LPR, bool SH>
static hipError_t launch_dn_t(hipStream_t st, const GemvArgs& a) {
    constexpr int RB = kGemvWaves * (kWave / LPR) * kRuDN;
    const int KS = a.K + (SH ? 1 : 0);
    const int C = a.I / Chunk<F>::CH;
    dim3 grid((a.H + RB - 1) / RB, a.M);
    const size_t lds = size_t(KS) * (a.I + C) * sizeof(float);
    hipLaunchKernelGGL((moe_down_slots<F, LPR, kRuDN, SH>), grid, dim3(kGemvThreads), lds, st,
                       a.w, a.ws, a.rex, a.rwt, a.gate_in, a.h, a.y, a.H, a.I, a.K, a.E);
    return hipGetLastError();
}

template <int F, bool SH>
static hipError_t dispatch_lpr(hipStream_t st, const GemvArgs& a, bool down) {
    const int chunks = (down ? a.I : a.H) / Chunk<F>::CH;
    switch (pick_lpr(chunks)) {
    case 8: return down ? launch_dn_t<F, 8, SH>(st, a) : launch_gu_t<F, 8, SH>(st, a);
    case 16: return down ? launch_dn_t<F, 16, SH>(st, a) : launch_gu_t<F, 16, SH>(st, a);
    case 32: return down ? launch_dn_t<F, 32, SH>(st, a) : launch_gu_t<F, 32, SH>(st, a);
    default: return down ? launch_dn_t<F, 64, SH>(st, a) : launch_gu_t<F, 64, SH>(st, a);
    }
}

template <int F>
static hipError_t dispatch_sh(hipStream_t st, const GemvArgs& a, bool down) {
    return a.shared ? dispatch_lpr<F, true>(st, a, down) : dispatch_lpr<F, false>(st, a, down);
}

hipError_t gemv_launch(hipStream_t st, int fmt, const GemvArgs& a, bool down) {
    switch (fmt) {
    case GRIM_FMT_BF16: return dispatch_sh<GRIM_FMT_BF16>(st, a, down);
    case GRIM_FMT_INT8: return dispatch_sh<GRIM_FMT_INT8>(st, a, down);
    case GRIM_FMT_INT4: return dispatch_sh<GRIM_FMT_INT4>(st, a, down);
    case GRIM_FMT_INT4_F16: return dispatch_sh<GRIM_FMT_INT4_F16>(st, a, down);
    case GRIM_FMT_MXFP4: return dispatch_sh<GRIM_FMT_MXFP4>(st, a, down);
    }
    return hipErrorInvalidValue;
}

size_t gemv_lds_bytes(int fmt, int H, int I, int KS, bool down) {
    const int CH = chunk_elems(fmt);
    if (!CH) return 0;
    return down ? size_t(KS) * (I + I / CH) * sizeof(float) : size_t(H + H / CH) * sizeof(float);
}

}  // namespace grim
