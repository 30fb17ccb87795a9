// gemv_wave.hpp -- the decode forward's router formatting step and its
// wave-centric gate_up kernel (INT4 / GPTQ INT4 / MXFP4 weights).
//
// Measured on MI355X, the decode layer is bound by VALU issue, not by HBM:
// a work-group that stages x into LDS, runs a top-k and addresses each
// weight chunk with 64-bit arithmetic spends ~1,100 VALU instructions per
// wave for 4 KiB of weights.  This kernel keeps the VALU work per weight
// byte near the dot products themselves:
//   * the router kernel formats the activations once per token (bf16 pair
//     words hi / lo, chunk sums and a lo-nonzero flag per 32-element
//     chunk); gate_up lanes read the 16 words of their chunk straight from
//     L2, with no LDS staging and no barrier;
//   * weights are addressed through buffer descriptors on the expert's block
//     (scalar base, 32-bit per-lane offsets);
//   * one wave runs the top-k from logits already in registers;
//   * each lane multiplies one chunk of RU gate rows and RU up rows per
//     chunk iteration; rows are summed over the wave by DPP and readlane.
#pragma once

namespace grim {

// ------------------------------------------------------ router formatting

// Chunk c of token t in the formatted activations (xf_words(H) words per
// token): hi words [16c, 16c+16), lo words [H/2 + 16c, +16), then at
// H + 2c the chunk's sum (of hi + lo, element order by pairs of lanes) and
// a flag that its lo words are not all zero.  Work-group b of the router
// launch formats chunks [b*CPB, (b+1)*CPB) of all tokens, four threads per
// chunk (one group of eight elements each).
template <int F>
__device__ __forceinline__ void xf_format(const DecodeArgs& a, int b) {
    const int C = a.H / 32;
    const int total = a.M * C;
    const int cpb = (total + a.NR - 1) / a.NR;
    const int tid = threadIdx.x;
    if (tid >= 4 * cpb) return;          // whole quads of lanes leave together
    const int ck = b * cpb + tid / 4;
    const bool ok = ck < total;
    const int t = ok ? ck / C : 0, c = ok ? ck % C : 0;
    const int g = 4 * c + (tid & 3);     // group of eight inside the token
    const float4* s4 = reinterpret_cast<const float4*>(a.x + int64_t(t) * a.H);
    const float4 p = s4[2 * g], q = s4[2 * g + 1];
    const float v[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
    uint32_t hw[4], lw[4];
    int any_lo = 0;
    float part = format_group<F>(v, hw, lw, any_lo);
    part += dpp_f<kDppXor1>(part);
    part += dpp_f<kDppXor2>(part);
    uint32_t fl = uint32_t(any_lo);
    fl |= dpp_u<kDppXor1>(fl);
    fl |= dpp_u<kDppXor2>(fl);
    if (!ok) return;
    uint32_t* xt = a.xf + int64_t(t) * a.xf_words;
    reinterpret_cast<u32x4*>(xt)[g] = u32x4{hw[0], hw[1], hw[2], hw[3]};
    reinterpret_cast<u32x4*>(xt + a.H / 2)[g] = u32x4{lw[0], lw[1], lw[2], lw[3]};
    if ((tid & 3) == 0) {
        xt[a.H + 2 * c] = f_bits(part);
        xt[a.H + 2 * c + 1] = fl;
    }
}

// ------------------------------------------------------------- gate_up

// Sum of v over the 64 lanes of a wave (uniform result): DPP inside each
// row of 16, then the four row sums in row order.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<kDppXor1>(v);
    v += dpp_f<kDppXor2>(v);
    v += dpp_f<kDppHalfMirror>(v);
    v += dpp_f<kDppMirror>(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

// wave_sum of N independent values with the same operations and order per
// value, step by step across the values: a lone DPP chain waits on each
// step (the compiler pads it with s_nop), N chains fill each other's gaps.
template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
#pragma unroll
    for (int r = 0; r < N; ++r) v[r] += dpp_f<kDppXor1>(v[r]);
#pragma unroll
    for (int r = 0; r < N; ++r) v[r] += dpp_f<kDppXor2>(v[r]);
#pragma unroll
    for (int r = 0; r < N; ++r) v[r] += dpp_f<kDppHalfMirror>(v[r]);
#pragma unroll
    for (int r = 0; r < N; ++r) v[r] += dpp_f<kDppMirror>(v[r]);
#pragma unroll
    for (int r = 0; r < N; ++r) v[r] = (lane_f(v[r], 0) + lane_f(v[r], 16)) + (lane_f(v[r], 32) + lane_f(v[r], 48));
}

// The two half-wave sums of N values (lanes 0-31 and 32-63), interleaved
// as wave_sum_n: after the four DPP steps h0 = lane 0 + lane 16, h1 =
// lane 32 + lane 48.
template <int N>
__device__ __forceinline__ void half_sums_n(float (&v)[N], float (&h0)[N], float (&h1)[N]) {
#pragma unroll
    for (int r = 0; r < N; ++r) v[r] += dpp_f<kDppXor1>(v[r]);
#pragma unroll
    for (int r = 0; r < N; ++r) v[r] += dpp_f<kDppXor2>(v[r]);
#pragma unroll
    for (int r = 0; r < N; ++r) v[r] += dpp_f<kDppHalfMirror>(v[r]);
#pragma unroll
    for (int r = 0; r < N; ++r) v[r] += dpp_f<kDppMirror>(v[r]);
#pragma unroll
    for (int r = 0; r < N; ++r) {
        h0[r] = lane_f(v[r], 0) + lane_f(v[r], 16);
        h1[r] = lane_f(v[r], 32) + lane_f(v[r], 48);
    }
}

// One weight chunk requested through buffer descriptors: the payload, and
// the raw scale / zero the chunk needs (decoded where it is used).
struct WRsrc {
    __amdgpu_buffer_rsrc_t p, s, z;
};

template <int F>
__device__ __forceinline__ void wprefetch(const WRsrc& r, const WView& w, bool hz, uint32_t row,
                                          uint32_t c, Pre& out) {
    out.raw = __builtin_amdgcn_raw_buffer_load_b128(r.p, row * uint32_t(w.row_bytes) + c * 16u, 0, 2);
    if constexpr (F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16) {
        const uint32_t si = row * uint32_t(w.row_scales) + ((c * 32u) >> w.gshift);
        out.sb = __builtin_amdgcn_raw_buffer_load_b16(r.s, si * 2u, 0, 0);
        // without zeros the descriptor covers nothing and the load returns 0
        const uint32_t zl = __builtin_amdgcn_raw_buffer_load_b8(r.z, si, 0, 0);
        out.zb = hz ? zl : uint32_t(w.default_zero);
    } else {   // MXFP4
        out.sb = __builtin_amdgcn_raw_buffer_load_b8(r.s, row * uint32_t(w.row_scales) + c, 0, 0);
        out.zb = 0;
    }
}

// Lanes 0..R-1 of a wave (R a multiple of 8) each hold element i0 + lane
// of a formatted vector of n elements (layout of put_group_fmt); lanes at
// or past `valid` hold padding and store nothing.  Each group of eight
// lanes forms its group: bf16 hi / lo halves per lane, pair words through
// lane shuffles, the group sum (of hi + lo) by DPP.
template <int F>
__device__ __forceinline__ void put_rows_fmt(uint32_t* dst, int n, int i0, int valid, float v) {
    const int lane = threadIdx.x & (kWave - 1);
    const int k = lane & 7;
    uint32_t lo16;
    const uint32_t hi16 = split_hi_lo(v, lo16);
    float part = bits_f(hi16 << 16) + bits_f(lo16 << 16);
    part += dpp_f<kDppXor1>(part);
    part += dpp_f<kDppXor2>(part);
    part += dpp_f<kDppHalfMirror>(part);
    constexpr int D = Act<F>::kInterleave ? 4 : 1;   // pair partner distance
    const uint32_t hp = uint32_t(__shfl_down(int(hi16), D, 8));
    const uint32_t lp = uint32_t(__shfl_down(int(lo16), D, 8));
    const int g = (i0 + lane) / 8;
    const int nch = n / Chunk<F>::CH;
    const int qp = quad_pos<F>(g, nch);
    const bool ok = lane - (lane & 7) < valid;      // the group holds real rows
    const bool owner = Act<F>::kInterleave ? k < 4 : (k & 1) == 0;
    const int word = Act<F>::kInterleave ? k : k / 2;
    if (ok && owner) {
        dst[4 * qp + word] = hi16 | (hp << 16);
        dst[n / 2 + 4 * qp + word] = lo16 | (lp << 16);
    }
    if (ok && k == 0) reinterpret_cast<float*>(dst)[n + g] = part;
}

// Work item j = (token, slot, row block of 4 * RU (gate, up) row pairs);
// wave w owns pairs [4 * RU * rb + RU * w, + RU); lane l multiplies chunks
// l, l + 64, ... (NCI of them) of each of its rows.
template <int F, int RU, int NCI, bool SH>
__global__ __launch_bounds__(kGemvThreads) void moe_gate_up_wave_kernel(DecodeArgs a) {
    constexpr int RB = kGemvWaves * RU;
    const int H = a.H, I = a.I, K = a.K, E = a.E;
    const int KS = K + (SH ? 1 : 0);
    const int C = H / 32;
    const int j = blockIdx.x;
    const int t = j / (KS * a.gu_rb);
    const int slot = (j / a.gu_rb) % KS;
    const int rb = j % a.gu_rb;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const bool shr = SH && slot >= K;   // block-uniform
    GRIM_TS(a, 1, 0);

    // (1) everything that does not depend on the routing: this lane's
    // activation chunks with their sums and flags
    const uint32_t* xt = a.xf + int64_t(t) * a.xf_words;
    XChunk<F, false> xc[NCI];
    uint32_t xflag = 0;
#pragma unroll
    for (int ci = 0; ci < NCI; ++ci) {
        const int c = lane + ci * kWave;
        const int cc = c < C ? c : C - 1;
        const u32x4* h4 = reinterpret_cast<const u32x4*>(xt + 16 * cc);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = h4[q];
            xc[ci].hi[4 * q] = v.x; xc[ci].hi[4 * q + 1] = v.y;
            xc[ci].hi[4 * q + 2] = v.z; xc[ci].hi[4 * q + 3] = v.w;
        }
        const uint2 sf = *reinterpret_cast<const uint2*>(xt + H + 2 * cc);
        xc[ci].xs = bits_f(sf.x);
        xflag |= c < C ? sf.y : 0u;
    }

    // (2) routing: the token's picks from the logits (parallel ranks; the
    // group-limited mode by one wave).  The weights of the picks are formed
    // after this item's weight loads are issued (only down needs them).
    __shared__ int sel_e[16];
    __shared__ float sel_w[16];
    __shared__ RankLds rl;
    int e = 0;
    bool active = true;
    const bool rank_path = !shr && a.mode <= 2;
    const bool first = slot == 0 && rb == 0;   // stores the token's routes
    if (!shr) {
        const float* lrow = a.logits + int64_t(t) * E;
        if (rank_path) {
            topk_rank_block<kGemvThreads>(lrow, E, K, a.mode, a.bias16, rl,
                                          a.ts && blockIdx.x < 2048 ? a.ts + (2048 + blockIdx.x) * 8 : nullptr);
            e = __builtin_amdgcn_readfirstlane(rl.sel_e[slot]);
        } else {
            __shared__ float tk_scratch[512 + 64];
            if (wave == 0) {
                float lv[kMaxV];
                topk_load(lrow, E, lv);
                topk_wave_regs(lv, E, K, a.mode, a.normalize, a.scaling, a.bias16, a.bias32,
                               a.n_group, a.topk_group, sel_e, sel_w, tk_scratch, tk_scratch + 512);
            }
            __syncthreads();
            if (first && int(threadIdx.x) < K) {
                a.rex[int64_t(t) * K + threadIdx.x] = sel_e[threadIdx.x];
                a.rwt[int64_t(t) * K + threadIdx.x] = sel_w[threadIdx.x];
            }
            e = __builtin_amdgcn_readfirstlane(sel_e[slot]);
        }
        if (e < 0 || e >= E) { active = false; e = 0; }
    }
    GRIM_TS(a, 1, 1);

    // (3) this wave's weights, all requested before anything waits on them
    const WView& w = shr ? a.sgu : a.gu;
    const bool hz = w.zeros != nullptr;
    const int64_t rows0 = int64_t(e) * 2 * I;
    const uint32_t nrows = 2u * uint32_t(I);
    constexpr int SB = (F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16) ? 2 : 1;
    WRsrc rs;
    rs.p = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(w.payload + rows0 * w.row_bytes), 0,
                                             int(nrows * uint32_t(w.row_bytes)), 0x00020000);
    rs.s = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(static_cast<const uint8_t*>(w.scales) + rows0 * w.row_scales * SB), 0,
        int(nrows * uint32_t(w.row_scales) * SB), 0x00020000);
    rs.z = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(hz ? w.zeros + rows0 * w.row_scales : w.payload), 0,
        hz ? int(nrows * uint32_t(w.row_scales)) : 0, 0x00020000);
    const int i0 = rb * RB + wave * RU;
    Pre pg[RU][NCI], pu[RU][NCI];
#pragma unroll
    for (int r = 0; r < RU; ++r) {
        const uint32_t i = uint32_t(i0 + r < I ? i0 + r : I - 1);
#pragma unroll
        for (int ci = 0; ci < NCI; ++ci) {
            const int c = lane + ci * kWave;
            const uint32_t cc = uint32_t(c < C ? c : C - 1);
            wprefetch<F>(rs, w, hz, i, cc, pg[r][ci]);
            wprefetch<F>(rs, w, hz, uint32_t(I) + i, cc, pu[r][ci]);
        }
    }
    GRIM_TS(a, 1, 2);
    // the routing weights, while the loads fly (first item of the token)
    if (rank_path && first && wave == 0) {
        topk_rank_weights(rl, K, a.mode, a.normalize, a.scaling, a.rex + int64_t(t) * K,
                          a.rwt + int64_t(t) * K);
    }

    // (4) the dots; the lo plane only when some chunk of this wave has one
    float ga[RU], ua[RU];
#pragma unroll
    for (int r = 0; r < RU; ++r) { ga[r] = 0.0f; ua[r] = 0.0f; }
    const bool lo_pass = __ballot(xflag != 0) != 0;   // wave-uniform
    if (!lo_pass) {
#pragma unroll
        for (int ci = 0; ci < NCI; ++ci) {
            const bool ok = lane + ci * kWave < C;
#pragma unroll
            for (int r = 0; r < RU; ++r) {
                const float dg = dot_chunk<F, false>(pg[r][ci], xc[ci]);
                const float du = dot_chunk<F, false>(pu[r][ci], xc[ci]);
                ga[r] += ok ? dg : 0.0f;
                ua[r] += ok ? du : 0.0f;
            }
        }
    } else {
#pragma unroll
        for (int ci = 0; ci < NCI; ++ci) {
            const int c = lane + ci * kWave;
            const int cc = c < C ? c : C - 1;
            XChunk<F, true> x2;
            const u32x4* l4 = reinterpret_cast<const u32x4*>(xt + H / 2 + 16 * cc);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u32x4 v = l4[q];
                x2.lo[4 * q] = v.x; x2.lo[4 * q + 1] = v.y;
                x2.lo[4 * q + 2] = v.z; x2.lo[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int k = 0; k < 16; ++k) x2.hi[k] = xc[ci].hi[k];
            x2.xs = xc[ci].xs;
            const bool ok = c < C;
#pragma unroll
            for (int r = 0; r < RU; ++r) {
                const float dg = dot_chunk<F, true>(pg[r][ci], x2);
                const float du = dot_chunk<F, true>(pu[r][ci], x2);
                ga[r] += ok ? dg : 0.0f;
                ua[r] += ok ? du : 0.0f;
            }
        }
    }
    GRIM_TS(a, 1, 3);

    // (5) h = silu(gate) * up for the wave's RU rows, then the block's RB
    // rows as formatted groups of eight (the down kernel's staging layout),
    // one row per lane of wave 0
    __shared__ float hrow[RB];
    {
        float gu[2 * RU];
#pragma unroll
        for (int r = 0; r < RU; ++r) { gu[r] = ga[r]; gu[RU + r] = ua[r]; }
        wave_sum_n(gu);
        // lane r < RU stores row r: a select chain, no branch per row
        float hv = 0.0f;
#pragma unroll
        for (int r = 0; r < RU; ++r) {
            const float v = (active && i0 + r < I) ? fast_silu(gu[r]) * gu[RU + r] : 0.0f;
            hv = lane == r ? v : hv;
        }
        if (lane < RU) hrow[wave * RU + lane] = hv;
    }
    __syncthreads();
    if (wave == 0 && lane < RB) put_rows_fmt<F>(a.hf + int64_t(t) * fmt_words(KS * I), KS * I,
                                                 slot * I + rb * RB, I - rb * RB, hrow[lane]);
    // shared_expert_gate: sigmoid(x . gate_w) (src/moe_kernels.cpp:162-172),
    // by the first item of each token
    if (a.gate_w && slot == 0 && rb == 0 && wave == 0) {
        const float* xr = a.x + int64_t(t) * H;
        float acc = 0.0f;
        for (int c = lane; c < H; c += kWave) acc = __builtin_fmaf(bf16_to_f32(a.gate_w[c]), xr[c], acc);
        acc = group_sum<kWave>(acc);
        if (lane == 0) a.gate[t] = det_sigmoid(acc);
    }
    GRIM_TS(a, 1, 4);
}

// ---------------------------------------------------------------- down

// Work item j = (token, block of 2 * RH output rows).  Wave s owns slot s
// (its expert is wave-uniform, so its weights go through one buffer
// descriptor); half-wave hw of it owns rows [2 * RH * ob + RH * hw, + RH);
// lane cl of the half multiplies chunks cl, cl + 32, ... (NCI of them) of
// those rows against the same chunks of h_s, held in registers (read from
// the formatted h written by gate_up).  Rows are summed over the half-wave
// by DPP; the slots are combined in slot order as in
// src/moe_kernels.cpp:273-445.
template <int F, int RH, int NCI, bool SH>
__global__ __launch_bounds__(512) void moe_down_wave_kernel(DecodeArgs a) {
    constexpr int RB = 2 * RH;
    const int H = a.H, I = a.I, K = a.K, E = a.E;
    const int KS = K + (SH ? 1 : 0);
    const int C = I / 32;
    const int nb = (H + RB - 1) / RB;
    const int t = blockIdx.x / nb;
    const int ob = blockIdx.x % nb;
    const int lane = threadIdx.x & (kWave - 1);
    const int s = threadIdx.x / kWave;          // slot of this wave
    const int hw = lane / 32, cl = lane & 31;
    const bool shared_slot = SH && s == K;
    const int n = KS * I;
    const int nch = n / 32;
    GRIM_TS(a, 2, 0);

    // (1) the slot's route and this lane's chunks of h_s, requested together
    const int sr = s < K ? s : 0;
    const int e_raw = a.rex[int64_t(t) * K + sr];
    const float w_raw = a.rwt[int64_t(t) * K + sr];
    const uint32_t* hsrc = a.hf + int64_t(t) * fmt_words(n);
    XChunk<F, true> hx[NCI];
#pragma unroll
    for (int ci = 0; ci < NCI; ++ci) {
        const int c = cl + 32 * ci;
        const int gc = s * C + (c < C ? c : C - 1);
        const u32x4* h4 = reinterpret_cast<const u32x4*>(hsrc);
        const u32x4* l4 = reinterpret_cast<const u32x4*>(hsrc + n / 2);
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const u32x4 v = h4[d * nch + gc];
            const u32x4 l = l4[d * nch + gc];
            hx[ci].hi[4 * d] = v.x; hx[ci].hi[4 * d + 1] = v.y;
            hx[ci].hi[4 * d + 2] = v.z; hx[ci].hi[4 * d + 3] = v.w;
            hx[ci].lo[4 * d] = l.x; hx[ci].lo[4 * d + 1] = l.y;
            hx[ci].lo[4 * d + 2] = l.z; hx[ci].lo[4 * d + 3] = l.w;
        }
        const float4 gs = reinterpret_cast<const float4*>(hsrc + n)[gc];
        hx[ci].xs = (gs.x + gs.y) + (gs.z + gs.w);
    }
    int e = __builtin_amdgcn_readfirstlane(e_raw);
    const float rw = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(w_raw)));
    bool valid = s < KS && (shared_slot || (e >= 0 && e < E && rw != 0.0f));
    if (!valid || shared_slot) e = 0;
    GRIM_TS(a, 2, 1);

    // (2) the weights of this half-wave's rows
    const WView& w = shared_slot ? a.sdn : a.dn;
    const bool hz = w.zeros != nullptr;
    constexpr int SB = (F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16) ? 2 : 1;
    const int64_t rows0 = int64_t(e) * H;
    WRsrc rs;
    rs.p = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(w.payload + rows0 * w.row_bytes), 0,
                                             int(uint32_t(H) * uint32_t(w.row_bytes)), 0x00020000);
    rs.s = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(static_cast<const uint8_t*>(w.scales) + rows0 * w.row_scales * SB), 0,
        int(uint32_t(H) * uint32_t(w.row_scales) * SB), 0x00020000);
    rs.z = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(hz ? w.zeros + rows0 * w.row_scales : w.payload), 0,
        hz ? int(uint32_t(H) * uint32_t(w.row_scales)) : 0, 0x00020000);
    const int o0 = ob * RB + hw * RH;
    Pre pw[RH][NCI];
#pragma unroll
    for (int r = 0; r < RH; ++r) {
        const uint32_t o = uint32_t(o0 + r < H ? o0 + r : H - 1);
#pragma unroll
        for (int ci = 0; ci < NCI; ++ci) {
            const int c = cl + 32 * ci;
            wprefetch<F>(rs, w, hz, o, uint32_t(c < C ? c : C - 1), pw[r][ci]);
        }
    }
    GRIM_TS(a, 2, 2);

    // (3) dots and the per-row sums over the half-wave
    float acc[RH];
#pragma unroll
    for (int r = 0; r < RH; ++r) {
        acc[r] = 0.0f;
#pragma unroll
        for (int ci = 0; ci < NCI; ++ci) {
            const float d = dot_chunk<F, true>(pw[r][ci], hx[ci]);
            acc[r] += cl + 32 * ci < C ? d : 0.0f;
        }
    }
    __shared__ float part[16][RB];
    __shared__ float slot_w[16];
    {
        float h0[RH], h1[RH];
        half_sums_n(acc, h0, h1);
        // lane r < 2 RH stores part row r: a select chain
        float pv = 0.0f;
#pragma unroll
        for (int r = 0; r < RH; ++r) {
            pv = lane == r ? h0[r] : pv;
            pv = lane == RH + r ? h1[r] : pv;
        }
        if (lane < 2 * RH && s < KS) part[s][lane] = valid ? pv : 0.0f;
    }
    if (lane == 0 && s < K) slot_w[s] = valid ? rw : 0.0f;
    GRIM_TS(a, 2, 3);
    __syncthreads();
    // (4) slot-order combine, + gate * shared expert last
    if (int(threadIdx.x) < RB) {
        const int r = threadIdx.x;
        const int o = ob * RB + r;
        if (o < H) {
            // part rows: half-wave 0 holds rows [0, RH), half 1 [RH, 2RH)
            // every slot's weight and part read before the fma chain (one
            // LDS round trip instead of K); slots past K or of weight 0
            // leave the total as the skipping loop does
            float wv[8], pv[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                wv[q] = q < K ? slot_w[q] : 0.0f;
                pv[q] = q < K ? part[q][r] : 0.0f;
            }
            float total = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; ++q) total = wv[q] != 0.0f ? __builtin_fmaf(wv[q], pv[q], total) : total;
            if (SH) {
                const float g = a.gate_in ? a.gate_in[t] : 1.0f;
                total = __builtin_fmaf(g, part[K][r], total);
            }
            a.y[int64_t(t) * H + o] = total;
        }
    }
    GRIM_TS(a, 2, 4);
}

}  // namespace grim
