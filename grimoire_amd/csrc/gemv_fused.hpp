// gemv_fused.hpp -- the one-launch decode layer: router, top-k, gate_up +
// SwiGLU and down + combine for one token in a single kernel.
//
// Behaviour follows the three-launch decode (src/moe_kernels.cpp:82-445,
// src/ops.cpp:1100-1148): logits = router . x (+ bias), the top-k of the
// token, h = silu(gate) * up per picked expert, y = sum over slots in slot
// order of w_s * (down_s . h_s).
//
// On MI355X a dependent kernel boundary inside a graph costs ~1.6 us and a
// grid-wide counter barrier 4-15 us (every arrival is an atomic on one
// address).  This kernel therefore has no barrier and no counter.  Each
// value another work-group needs is published as data that carries the
// call's epoch:
//   * router logits: one 64-bit store of (fp32 dot, epoch) per row;
//   * h: fp32 values stored write-through (sc1), then one 32-bit epoch flag
//     per work-group after its stores have completed.
// A reader polls those words with sc1 loads (they miss the XCD's L2, which
// is not coherent with the other XCDs') until every tag equals the epoch.
// Every such word is written in kSyncCopies copies and work-group b reads
// copy b % kSyncCopies: reads that miss L2 are served by the memory
// channel that holds the line, and 256 work-groups reading one copy of
// 24 KB of h measured ~6 us (a few channels serving every request).
// The epoch is the epoch word plus one (skipping 0, the value of cleared
// words).  Every work-group reads the word before it publishes its flag
// (the flag holds the epoch), and work-group 0 advances the word only after
// it has seen every work-group's flag, so all work-groups of a call agree on
// the epoch.  Tags are compared for equality: every word a call reads is
// also written by that call, so a stale value is the one an earlier call
// left, and it is taken for current only if exactly a multiple of 2^32
// calls separate the two (the 32-bit epoch wraps).  The sync words must be
// zero before a workspace's first use.
// Polls are bounded by the real-time counter (DecodeArgs::spin_ticks).  A
// work-group that runs out of time sets the error word, writes NaN to the
// outputs it owns (and, work-group 0, expert -1 / weight NaN routes) and
// carries on, so every wave exits.  A set error word poisons the
// workspace: work-group 0 does not advance the epoch after a time-out, and
// every later call reads the error word first and only writes NaN outputs,
// until the caller clears the sync words (grimoire_moe_decode_sync_reset).
// Late work-groups of a timed-out call therefore never feed the next one.
// All work-groups must be resident at once (a poll waits on work-groups
// that have not started otherwise): the host keeps the grid at or below one
// work-group of 512 threads per CU.
//
// Work per work-group b (8 waves):
//   router    rows e = b, b + G, ... (256 threads, router_row1's order);
//   gate_up   wave unit u = 8b + w: RU row pairs of one slot;
//   down      output rows [RB b, RB b + RB), RB = 2 RH, wave s = slot s,
//             half-wave = RH rows, lane = one 32-element chunk of I.
// Down weights are requested with the gate_up weights, before h exists, so
// the two streams share the memory system's queue and down waits only for
// h.
#pragma once

namespace grim {

constexpr int kFzThreads = 512;
constexpr int kFzWaves = kFzThreads / kWave;

__device__ __forceinline__ uint32_t sync_ld(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t sync_ld64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sync_st(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sync_st64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void sync_stf(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Formats n fp32 values (n % 32 == 0, n <= 32 * kFzChunks) into LDS once
// per work-group: chunk c at 36 c words, hi pair words at +0, lo at +16, the
// chunk sum at +32 (xf_format's arithmetic: four threads per chunk, one
// group of eight each, group sums combined by DPP in quad order).  ld(i)
// returns the float4 at value offset 4 i.  Returns whether any lo word is
// nonzero (block-uniform; ends with a barrier).
constexpr int kFzChunks = 256;
template <int F, typename LD>
__device__ __forceinline__ bool format_to_lds(uint32_t* lds, int n, LD ld) {
    const int groups = n / 8;
    int any_lo = 0;
    for (int g0 = 0; g0 < groups; g0 += kFzThreads) {
        const int g = g0 + int(threadIdx.x);
        const bool ok = g < groups;
        const int gg = ok ? g : groups - 1;
        const float4 p = ld(2 * gg), q = ld(2 * gg + 1);
        const float v[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
        uint32_t hw[4], lw[4];
        int lo = 0;
        float part = format_group<F>(v, hw, lw, lo);
        part += dpp_f<kDppXor1>(part);
        part += dpp_f<kDppXor2>(part);
        if (ok) {
            any_lo |= lo;
            uint32_t* c = lds + 36 * (g / 4);
            reinterpret_cast<u32x4*>(c)[g & 3] = u32x4{hw[0], hw[1], hw[2], hw[3]};
            reinterpret_cast<u32x4*>(c + 16)[g & 3] = u32x4{lw[0], lw[1], lw[2], lw[3]};
            if ((g & 3) == 0) c[32] = f_bits(part);
        }
    }
    return __syncthreads_or(any_lo) != 0;
}

template <int F, bool LO>
__device__ __forceinline__ void chunk_from_lds(const uint32_t* lds, int c, XChunk<F, LO>& x) {
    const u32x4* h4 = reinterpret_cast<const u32x4*>(lds + 36 * c);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const u32x4 v = h4[q];
        x.hi[4 * q] = v.x; x.hi[4 * q + 1] = v.y; x.hi[4 * q + 2] = v.z; x.hi[4 * q + 3] = v.w;
        if constexpr (LO) {
            const u32x4 l = h4[4 + q];
            x.lo[4 * q] = l.x; x.lo[4 * q + 1] = l.y; x.lo[4 * q + 2] = l.z; x.lo[4 * q + 3] = l.w;
        }
    }
    x.xs = bits_f(lds[36 * c + 32]);
}

template <int F>
__device__ __forceinline__ WRsrc expert_rsrc(const WView& w, int64_t rows0, uint32_t nrows) {
    constexpr int SB = (F == GRIM_FMT_INT4 || F == GRIM_FMT_INT4_F16) ? 2 : 1;
    const bool hz = w.zeros != nullptr;
    WRsrc rs;
    rs.p = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(w.payload + rows0 * w.row_bytes), 0,
                                             int(nrows * uint32_t(w.row_bytes)), 0x00020000);
    rs.s = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(static_cast<const uint8_t*>(w.scales) + rows0 * w.row_scales * SB), 0,
        int(nrows * uint32_t(w.row_scales) * SB), 0x00020000);
    rs.z = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(hz ? w.zeros + rows0 * w.row_scales : w.payload), 0,
        hz ? int(nrows * uint32_t(w.row_scales)) : 0, 0x00020000);
    return rs;
}

// Polls until pred() holds for the whole wave or the time bound passes;
// returns false on a time-out.
template <typename P>
__device__ __forceinline__ bool wave_poll(uint64_t ticks, P pred) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (true) {
        if (__ballot(!pred()) == 0) return true;
        if (__builtin_amdgcn_s_memrealtime() - t0 > ticks) return false;
        __builtin_amdgcn_s_sleep(1);
    }
}

template <int F, int RU, int RH>
__global__ __launch_bounds__(kFzThreads) void moe_decode_fused_kernel(DecodeArgs a) {
    const int H = a.H, I = a.I, K = a.K, E = a.E;
    const int G = gridDim.x;
    const int b = blockIdx.x;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    const int C = H / 32, CI = I / 32;
    uint32_t* epoch_word = a.sync;
    uint32_t* err = a.sync + 1;
    uint32_t* flags = a.sync + kSyncFlagOff;                             // [copy][G]
    uint64_t* rtags = reinterpret_cast<uint64_t*>(a.sync + kSyncRtagOff);  // [copy][E]
    const int hst = fused_h_stride(K, I);
    // the copies this work-group reads
    const int mine = b % kSyncCopies;
    const uint32_t* my_flags = flags + mine * kSyncFlagStride;
    const uint64_t* my_rtags = rtags + mine * kSyncRtagStride;

    __shared__ uint32_t s_epoch, s_err, s_bad;
    __shared__ float red[4];
    __shared__ int sel_e[16];
    __shared__ float sel_w[16];
    __shared__ float tk_scratch[512 + 64];
    __shared__ RankLds rl;
    __shared__ __align__(16) float hs[kFzWaves * 4];   // this work-group's h values
    __shared__ float part[8][2 * RH];
    __shared__ uint32_t fl[kFzChunks * 36];   // formatted x, later h (format_to_lds)

    GRIM_TS(a, 0, 0);
#ifdef GRIM_TIMING
    if (a.ts && threadIdx.x == 0) a.ts[(2048 + b) * 8 + 1] = __builtin_amdgcn_s_memtime();
#endif
    // (1) the epoch, the router row's loads, this lane's x chunk
    if (threadIdx.x == 0) {
        const uint32_t e = sync_ld(epoch_word) + 1u;
        s_epoch = e == 0u ? 1u : e;
        s_err = sync_ld(err);
        s_bad = 0u;
    }
    // router rows e = b, b + G, ...: threads 0..255 hold router_row1's
    // elements (k = 4t + 1024m) and follow its FMA order and reduction, so
    // the logits equal grimoire_moe_router_logits' bit for bit
    const bool rt = threadIdx.x < 256;
    RouterRegs<2> rr;
    if (rt && b < E) router_row1_load(a.router + int64_t(b) * H, a.x, H, rr);
    const int cx = lane < C ? lane : C - 1;
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    const bool x_lo = format_to_lds<F>(fl, H, [&](int i) { return x4[i]; });
    const uint32_t epoch = s_epoch;
    constexpr int RB = 2 * RH;
    if (s_err != 0u) {
        // poisoned workspace (an earlier call timed out): NaN outputs only
        const float qnan = __builtin_nanf("");
        for (int o = b * RB + int(threadIdx.x); o < min(H, (b + 1) * RB); o += kFzThreads) a.y[o] = qnan;
        if (b == 0 && int(threadIdx.x) < K) {
            a.rex[threadIdx.x] = -1;
            a.rwt[threadIdx.x] = qnan;
        }
        return;
    }
    for (int e = b; e < E; e += G) {
        if (e != b && rt) router_row1_load(a.router + int64_t(e) * H, a.x, H, rr);
        float acc = 0.0f;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int k = int(threadIdx.x) * 4 + 1024 * m;
            float a2 = __builtin_fmaf(rr.w[m].x, rr.x[m].x, acc);
            a2 = __builtin_fmaf(rr.w[m].y, rr.x[m].y, a2);
            a2 = __builtin_fmaf(rr.w[m].z, rr.x[m].z, a2);
            a2 = __builtin_fmaf(rr.w[m].w, rr.x[m].w, a2);
            acc = k < H ? a2 : acc;
        }
        const float v = group_sum<kWave>(acc);
        if (lane == 0 && wave < 4) red[wave] = v;
        __syncthreads();
        if (wave == 0 && lane < kSyncCopies) {
            const float t = (red[0] + red[1]) + (red[2] + red[3]);
            sync_st64(rtags + lane * kSyncRtagStride + e, uint64_t(f_bits(t)) | (uint64_t(epoch) << 32));
        }
        __syncthreads();
    }
    GRIM_TS(a, 0, 1);

    // (2) every work-group forms the token's picks from all router pieces
    if (wave == 0) {
        const int V = (E + kWave - 1) / kWave;
        float lv[kMaxV], rb[kMaxV];
#pragma unroll
        for (int j = 0; j < kMaxV; ++j) {
            const int e = lane * V + j;
            rb[j] = (a.rbias && j < V && e < E) ? a.rbias[e] : 0.0f;
        }
        // every tag requested before any is compared
        const bool ok = wave_poll(a.spin_ticks, [&]() {
            uint64_t v[kMaxV];
#pragma unroll
            for (int j = 0; j < kMaxV; ++j) {
                const int e = lane * V + j;
                v[j] = (j < V && e < E) ? sync_ld64(my_rtags + e) : uint64_t(epoch) << 32;
            }
            bool all = true;
#pragma unroll
            for (int j = 0; j < kMaxV; ++j) {
                all &= uint32_t(v[j] >> 32) == epoch;
                lv[j] = a.rbias ? bits_f(uint32_t(v[j])) + rb[j] : bits_f(uint32_t(v[j]));
            }
            return all;
        });
        if (!ok && lane == 0) {
            sync_st(err, 1u);
            s_bad = 1u;
        }
        GRIM_TS(a, 0, 2);
        if (b == 0) {
#pragma unroll
            for (int j = 0; j < kMaxV; ++j)
                if (j < V && lane * V + j < E) a.logits[lane * V + j] = lv[j];
        }
        if (a.mode <= 2) {
            // the logits to LDS for the work-group's parallel-rank top-k
#pragma unroll
            for (int j = 0; j < kMaxV; ++j)
                if (j < V && lane * V + j < E) tk_scratch[lane * V + j] = lv[j];
        } else {
            topk_wave_regs(lv, E, K, a.mode, a.normalize, a.scaling, a.bias16, a.bias32, a.n_group,
                           a.topk_group, sel_e, sel_w, tk_scratch, tk_scratch + 512);
        }
    }
    __syncthreads();
    if (a.mode <= 2) {
        // every rank at once over the 512 threads (topk_rank_block), the
        // weights of the picks by one wave: the picks and weights of
        // topk_wave_regs
        topk_rank_block<kFzThreads>(tk_scratch, E, K, a.mode, a.bias16, rl);
        if (wave == 0) topk_rank_weights(rl, K, a.mode, a.normalize, a.scaling, sel_e, sel_w);
        __syncthreads();
    }
    GRIM_TS(a, 0, 7);
    if (b == 0 && int(threadIdx.x) < K) {
        a.rex[threadIdx.x] = s_bad ? -1 : sel_e[threadIdx.x];
        a.rwt[threadIdx.x] = s_bad ? __builtin_nanf("") : sel_w[threadIdx.x];
    }

    // (3) gate_up weights of this wave's unit, then down weights of this
    // work-group's rows, all requested before anything waits on them
    const int upe = I / RU;                 // units per slot
    const int u = b * kFzWaves + wave;
    const bool has_gu = u < K * upe;
    const int gslot = has_gu ? u / upe : 0;
    const int i0 = has_gu ? (u % upe) * RU : 0;
    int ge = __builtin_amdgcn_readfirstlane(sel_e[gslot]);
    const bool gactive = has_gu && ge >= 0 && ge < E;
    if (!gactive) ge = 0;
    const bool ghz = a.gu.zeros != nullptr;
    const WRsrc grs = expert_rsrc<F>(a.gu, int64_t(ge) * 2 * I, 2u * uint32_t(I));
    Pre pg[RU], pu[RU];
#pragma unroll
    for (int r = 0; r < RU; ++r) {
        wprefetch<F>(grs, a.gu, ghz, uint32_t(i0 + r), uint32_t(cx), pg[r]);
        wprefetch<F>(grs, a.gu, ghz, uint32_t(I + i0 + r), uint32_t(cx), pu[r]);
    }
    const int nb = (H + RB - 1) / RB;
    const bool has_dn = b < nb;
    const int s = wave;                      // down: wave s = slot s
    const int hw = lane / 32, cl = lane & 31;
    const int ccl = cl < CI ? cl : CI - 1;
    int de = __builtin_amdgcn_readfirstlane(sel_e[s < K ? s : 0]);
    const float rw = sel_w[s < K ? s : 0];
    const bool dvalid = has_dn && s < K && de >= 0 && de < E && rw != 0.0f;
    if (!(de >= 0 && de < E)) de = 0;
    const bool dhz = a.dn.zeros != nullptr;
    const WRsrc drs = expert_rsrc<F>(a.dn, int64_t(de) * H, uint32_t(H));
    const int o0 = b * RB + hw * RH;
    Pre pw[RH];
#pragma unroll
    for (int r = 0; r < RH; ++r) {
        const uint32_t o = uint32_t(o0 + r < H ? o0 + r : H - 1);
        wprefetch<F>(drs, a.dn, dhz, o, uint32_t(ccl), pw[r]);
    }

    GRIM_TS(a, 0, 3);
    // (4) gate_up dots, h = silu(gate) * up, published write-through
    if (has_gu) {
        float ga[RU], ua[RU];
        const bool okc = lane < C;
        if (!x_lo) {
            XChunk<F, false> x1;
            chunk_from_lds<F, false>(fl, cx, x1);
#pragma unroll
            for (int r = 0; r < RU; ++r) {
                const float dg = dot_chunk<F, false>(pg[r], x1);
                const float du = dot_chunk<F, false>(pu[r], x1);
                ga[r] = okc ? dg : 0.0f;
                ua[r] = okc ? du : 0.0f;
            }
        } else {
            XChunk<F, true> xc;
            chunk_from_lds<F, true>(fl, cx, xc);
#pragma unroll
            for (int r = 0; r < RU; ++r) {
                const float dg = dot_chunk<F, true>(pg[r], xc);
                const float du = dot_chunk<F, true>(pu[r], xc);
                ga[r] = okc ? dg : 0.0f;
                ua[r] = okc ? du : 0.0f;
            }
        }
#ifdef GRIM_TIMING
        if (a.ts && threadIdx.x == 0) a.ts[(2048 + b) * 8] = __builtin_amdgcn_s_memrealtime();
#endif
        float gu[2 * RU];
#pragma unroll
        for (int r = 0; r < RU; ++r) { gu[r] = ga[r]; gu[RU + r] = ua[r]; }
        wave_sum_n(gu);
        float hv = 0.0f;
#pragma unroll
        for (int r = 0; r < RU; ++r) hv = lane == r ? (gactive ? fast_silu(gu[r]) * gu[RU + r] : 0.0f) : hv;
        if (lane < RU) hs[wave * RU + lane] = hv;
    }
    __syncthreads();
    // the work-group's units are consecutive, so its h values are one
    // span [8 RU b, + nv) of the flat h: nv / 4 16-byte write-through
    // stores per copy (one 4-byte store per value and copy measured
    // ~3 us slower: ~200 K partial-line writes per layer)
    {
        const int v0 = kFzWaves * RU * b;
        const int nv = min(kFzWaves * RU, K * I - v0);
        const int n4 = nv > 0 ? nv / 4 : 0;
        const int t = threadIdx.x;
        if (t < kSyncCopies * n4) {
            const int c = t / n4, q = t % n4;
            const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
                a.hrep, 0, kSyncCopies * hst * 4, 0x00020000);
            const float4 v = *reinterpret_cast<const float4*>(hs + 4 * q);
            __builtin_amdgcn_raw_buffer_store_b128(u32x4{f_bits(v.x), f_bits(v.y), f_bits(v.z), f_bits(v.w)},
                                                   hr, uint32_t(4 * (c * hst + v0 + 4 * q)), 0, 16);
        }
    }
    // every h store complete (and, with them, this wave's weight loads)
    // before the work-group's flag
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (wave == 0 && lane < kSyncCopies) sync_st(flags + lane * kSyncFlagStride + b, epoch);
    GRIM_TS(a, 0, 4);
    if (!has_dn && b != 0) return;

    // (5) wait for every work-group's flag (its h, and its read of the
    // epoch word), then the down dots
    if (wave == 0) {
        const bool ok = wave_poll(a.spin_ticks, [&]() {
            bool all = true;
            for (int q = lane; q < G; q += kWave) all = all && sync_ld(my_flags + q) == epoch;
            return all;
        });
        if (!ok && lane == 0) {
            sync_st(err, 1u);
            s_bad = 1u;
        }
        // every work-group has read the epoch word: the next call's epoch
        // (not after a time-out: the workspace is poisoned then)
        if (b == 0 && lane == 0 && ok) sync_st(epoch_word, epoch);
    }
    __syncthreads();
    GRIM_TS(a, 0, 5);
    if (!has_dn) return;
    // this work-group's copy of h (whole-line requests), formatted once into
    // LDS; chunk c of slot q is chunk q CI + c there
    {
        const __amdgpu_buffer_rsrc_t hr = __builtin_amdgcn_make_buffer_rsrc(
            a.hrep + mine * hst, 0, K * I * 4, 0x00020000);
        __syncthreads();   // every wave is done with the formatted x
        format_to_lds<F>(fl, K * I, [&](int i) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(hr, uint32_t(16 * i), 0, 16);
            return make_float4(bits_f(v.x), bits_f(v.y), bits_f(v.z), bits_f(v.w));
        });
    }
#ifdef GRIM_TIMING
    if (a.ts && threadIdx.x == 0) a.ts[(2048 + b) * 8 + 3] = __builtin_amdgcn_s_memrealtime();
#endif
    XChunk<F, true> hx;
    chunk_from_lds<F, true>(fl, (s < K ? s : 0) * CI + ccl, hx);
    float acc[RH];
#pragma unroll
    for (int r = 0; r < RH; ++r) {
        const float d = dot_chunk<F, true>(pw[r], hx);
        acc[r] = cl < CI ? d : 0.0f;
    }
    {
        float h0[RH], h1[RH];
        half_sums_n(acc, h0, h1);
        float pv = 0.0f;
#pragma unroll
        for (int r = 0; r < RH; ++r) {
            pv = lane == r ? h0[r] : pv;
            pv = lane == RH + r ? h1[r] : pv;
        }
        if (lane < 2 * RH) part[s][lane] = dvalid ? pv : 0.0f;
    }
    __syncthreads();
#ifdef GRIM_TIMING
    if (a.ts && threadIdx.x == 0) a.ts[(2048 + b) * 8 + 4] = __builtin_amdgcn_s_memrealtime();
#endif
    // (6) slot-order combine
    if (int(threadIdx.x) < RB) {
        const int r = threadIdx.x;
        const int o = b * RB + r;
        if (o < H) {
            float wv[8], pv[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int eq = q < K ? sel_e[q] : -1;
                wv[q] = (eq >= 0 && eq < E) ? sel_w[q] : 0.0f;
                pv[q] = q < K ? part[q][r] : 0.0f;
            }
            float total = 0.0f;
#pragma unroll
            for (int q = 0; q < 8; ++q) total = wv[q] != 0.0f ? __builtin_fmaf(wv[q], pv[q], total) : total;
            a.y[o] = s_bad ? __builtin_nanf("") : total;
        }
    }
    GRIM_TS(a, 0, 6);
#ifdef GRIM_TIMING
    if (a.ts && threadIdx.x == 0) a.ts[(2048 + b) * 8 + 2] = __builtin_amdgcn_s_memtime();
#endif
}

}  // namespace grim
