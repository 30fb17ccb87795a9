// dispatch.hip -- expert histogram, scan, stable permutation, and combine.
//
// The permutation is deterministic: expert-major, ascending route index,
// i.e. the order of the reference's host counting sort
// (src/grimoire.cpp:23162-23170), produced on the device without global
// atomics:
//   1. count   each block counts its chunk of routes per expert in LDS and
//              writes the row bcount[b][E];
//   2. scan    a column scan turns bcount into per-(block, expert) bases
//              inside the expert and per-expert counts; one block then
//              forms the exclusive offsets and the m-tile table
//              (src/prefill.cpp:2770-2782);
//   3. rank    each block ranks its routes inside their expert by counting
//              earlier routes of the same expert in the block (stable);
//              row = offsets[e] + block base + rank;
//   4. permute one block per token writes bf16(x[t]) to its K rows
//              (src/prefill.cpp:2784-2806).
#include "common.hpp"
#include "dispatch.hpp"

namespace grim {

constexpr int kDispThreads = 256;
constexpr int kRoutesPerBlock = 256;

__global__ __launch_bounds__(kDispThreads) void disp_count(const int32_t* __restrict__ ids, int R,
                                                           int E, int32_t* __restrict__ bcount) {
    extern __shared__ int32_t hist[];
    for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
    __syncthreads();
    const int r0 = blockIdx.x * kRoutesPerBlock;
    for (int i = threadIdx.x; i < kRoutesPerBlock; i += blockDim.x) {
        const int r = r0 + i;
        if (r < R) {
            const int e = ids[r];
            if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) bcount[int64_t(blockIdx.x) * E + e] = hist[e];
}

// Per-block bases inside each expert: one block per 64 experts, 16 threads
// per expert each summing a contiguous slice of the count blocks (all its
// loads in flight together), slices combined in LDS; writes the exclusive
// bases back into bcount and the expert's total into counts.
constexpr int kColExperts = 64, kColSlices = 16;
__global__ __launch_bounds__(kColExperts * kColSlices) void disp_colscan(int32_t* __restrict__ bcount,
                                                                       int nb, int E,
                                                                       int32_t* __restrict__ counts) {
    __shared__ int32_t ssum[kColSlices][kColExperts];
    const int el = threadIdx.x % kColExperts, sl = threadIdx.x / kColExperts;
    const int e = blockIdx.x * kColExperts + el;
    const int per = (nb + kColSlices - 1) / kColSlices;
    const int b0 = sl * per, b1 = min(nb, b0 + per);
    int tot = 0;
    if (e < E)
        for (int b = b0; b < b1; ++b) tot += bcount[int64_t(b) * E + e];
    ssum[sl][el] = tot;
    __syncthreads();
    int base = 0;
    for (int k = 0; k < sl; ++k) base += ssum[k][el];
    if (e < E) {
        for (int b = b0; b < b1; ++b) {
            const int v = bcount[int64_t(b) * E + e];
            bcount[int64_t(b) * E + e] = base;
            base += v;
        }
        if (sl == kColSlices - 1) counts[e] = base;
    }
}

// One block of 1024 threads over the expert totals: exclusive offsets, the
// m-tile table and the live tile count.
__global__ __launch_bounds__(1024) void disp_scan(int E, int32_t* __restrict__ counts,
                                                  int32_t* __restrict__ offsets,
                                                  int32_t* __restrict__ tile_e,
                                                  int32_t* __restrict__ tile_mb, int tmax, int mc,
                                                  int32_t* __restrict__ n_tiles_out) {
    // per 1024-expert chunk: inclusive scans of counts and tiles within each
    // wave by lane shifts, then over the 16 waves' totals (two barriers)
    __shared__ int32_t wsum[16][2];
    __shared__ int32_t carry[2];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    if (threadIdx.x == 0) { carry[0] = 0; carry[1] = 0; }
    __syncthreads();
    for (int e0 = 0; e0 < E; e0 += 1024) {
        const int e = e0 + threadIdx.x;
        const int c = e < E ? counts[e] : 0;
        const int nt = (mc > 0 && e < E) ? (c + mc - 1) / mc : 0;
        int ic = c, it = nt;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int a = __shfl_up(ic, off, 64), b = __shfl_up(it, off, 64);
            if (lane >= off) { ic += a; it += b; }
        }
        if (lane == 63) { wsum[wv][0] = ic; wsum[wv][1] = it; }
        __syncthreads();
        int bc = carry[0], bt = carry[1], totc = 0, tott = 0;
        for (int w = 0; w < 16; ++w) {
            const int tc = wsum[w][0], tt = wsum[w][1];
            bc += w < wv ? tc : 0;
            bt += w < wv ? tt : 0;
            totc += tc;
            tott += tt;
        }
        const int rbase = bc + ic - c;
        const int tbase = bt + it - nt;
        if (e < E) {
            offsets[e] = rbase;
            if (tile_e)
                for (int i = 0; i < nt; ++i)
                    if (tbase + i < tmax) { tile_e[tbase + i] = e; tile_mb[tbase + i] = i; }
        }
        __syncthreads();
        if (threadIdx.x == 0) { carry[0] += totc; carry[1] += tott; }
        __syncthreads();
    }
    if (tile_e)
        for (int t = carry[1] + threadIdx.x; t < tmax; t += 1024) { tile_e[t] = -1; tile_mb[t] = 0; }
    if (threadIdx.x == 0 && n_tiles_out) *n_tiles_out = carry[1];
}

__global__ __launch_bounds__(kDispThreads) void disp_rank(const int32_t* __restrict__ ids, int R,
                                                          int E, int K,
                                                          const int32_t* __restrict__ bbase,
                                                          const int32_t* __restrict__ offsets,
                                                          int32_t* __restrict__ inverse,
                                                          int32_t* __restrict__ perm_token) {
    static_assert(kRoutesPerBlock == kDispThreads, "one route per thread");
    __shared__ __attribute__((aligned(16))) int32_t le[kRoutesPerBlock];
    const int r0 = blockIdx.x * kRoutesPerBlock;
    const int n = R - r0 < kRoutesPerBlock ? R - r0 : kRoutesPerBlock;
    const int i = threadIdx.x;
    le[i] = i < n ? ids[r0 + i] : -1;
    __syncthreads();
    const int my_e = le[i];
    // count earlier routes of the same expert (uniform loop: LDS broadcast)
    int rank = 0;
#pragma unroll 4
    for (int j = 0; j < kRoutesPerBlock; j += 4) {
        const int4 q = *reinterpret_cast<const int4*>(&le[j]);
        rank += (j < i && q.x == my_e) ? 1 : 0;
        rank += (j + 1 < i && q.y == my_e) ? 1 : 0;
        rank += (j + 2 < i && q.z == my_e) ? 1 : 0;
        rank += (j + 3 < i && q.w == my_e) ? 1 : 0;
    }
    if (i >= n) return;
    const int r = r0 + i;
    if (my_e < 0 || my_e >= E) { inverse[r] = -1; return; }
    const int p = offsets[my_e] + bbase[int64_t(blockIdx.x) * E + my_e] + rank;
    inverse[r] = p;
    if (perm_token) perm_token[p] = r / K;
}

// disp_rank for calls without a tile table: every block forms the
// exclusive expert offsets itself (a block-wide scan of the E counts, the
// same sums as disp_scan's), so the single-block scan launch drops out;
// block 0 publishes them (and the m-tile count when mc > 0).
constexpr int kRankScanMaxE = 2048;
__global__ __launch_bounds__(kDispThreads) void disp_rank_scan(const int32_t* __restrict__ ids, int R, int E,
                                                               int K, const int32_t* __restrict__ bbase,
                                                               const int32_t* __restrict__ counts,
                                                               int32_t* __restrict__ offsets,
                                                               int32_t* __restrict__ inverse,
                                                               int32_t* __restrict__ perm_token, int mc,
                                                               int32_t* __restrict__ n_tiles_out) {
    static_assert(kRoutesPerBlock == kDispThreads, "one route per thread");
    constexpr int PER = kRankScanMaxE / kDispThreads;
    __shared__ __attribute__((aligned(16))) int32_t le[kRoutesPerBlock];
    __shared__ int32_t off_s[kRankScanMaxE];
    __shared__ int32_t wsum[kDispThreads / 64][2];
    const int i = threadIdx.x, lane = i & 63, wv = i >> 6;
    const int r0 = blockIdx.x * kRoutesPerBlock;
    const int n = R - r0 < kRoutesPerBlock ? R - r0 : kRoutesPerBlock;
    le[i] = i < n ? ids[r0 + i] : -1;
    // thread i's experts [i * per, +per): counts, their sum and tile count
    const int per = (E + kDispThreads - 1) / kDispThreads;
    int loc[PER];
    int sum = 0, tiles = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = i * per + j;
        loc[j] = (j < per && e < E) ? counts[e] : 0;
        sum += loc[j];
        tiles += mc > 0 ? (loc[j] + mc - 1) / mc : 0;
    }
    int incl = sum, tinc = tiles;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int a = __shfl_up(incl, off, 64), b = __shfl_up(tinc, off, 64);
        if (lane >= off) { incl += a; tinc += b; }
    }
    if (lane == 63) { wsum[wv][0] = incl; wsum[wv][1] = tinc; }
    __syncthreads();
    int base = incl - sum, ttot = 0;
    for (int w = 0; w < kDispThreads / 64; ++w) {
        base += w < wv ? wsum[w][0] : 0;
        ttot += wsum[w][1];
    }
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = i * per + j;
        if (j < per && e < E) {
            off_s[e] = base;
            if (blockIdx.x == 0) offsets[e] = base;
        }
        base += loc[j];
    }
    if (blockIdx.x == 0 && i == 0 && n_tiles_out) *n_tiles_out = ttot;
    __syncthreads();
    const int my_e = le[i];
    int rank = 0;
#pragma unroll 4
    for (int j = 0; j < kRoutesPerBlock; j += 4) {
        const int4 q = *reinterpret_cast<const int4*>(&le[j]);
        rank += (j < i && q.x == my_e) ? 1 : 0;
        rank += (j + 1 < i && q.y == my_e) ? 1 : 0;
        rank += (j + 2 < i && q.z == my_e) ? 1 : 0;
        rank += (j + 3 < i && q.w == my_e) ? 1 : 0;
    }
    if (i >= n) return;
    const int r = r0 + i;
    if (my_e < 0 || my_e >= E) { inverse[r] = -1; return; }
    const int p = off_s[my_e] + bbase[int64_t(blockIdx.x) * E + my_e] + rank;
    inverse[r] = p;
    if (perm_token) perm_token[p] = r / K;
}

// One block per token: bf16 row written to each of its K permuted rows.
template <bool SRC_BF16>
__global__ __launch_bounds__(kDispThreads) void disp_permute(const void* __restrict__ hidden,
                                                             const int32_t* __restrict__ inverse,
                                                             uint16_t* __restrict__ xperm,
                                                             uint16_t* __restrict__ xrow, int H,
                                                             int K) {
    const int t = blockIdx.x;
    int dst[16];
    for (int s = 0; s < K; ++s) dst[s] = inverse[int64_t(t) * K + s];
    for (int d = threadIdx.x * 4; d < H; d += blockDim.x * 4) {
        uint32_t lo, hi;
        if constexpr (SRC_BF16) {
            const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(hidden) +
                                                            int64_t(t) * H + d);
            lo = v.x; hi = v.y;
        } else {
            const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(hidden) +
                                                              int64_t(t) * H + d);
            lo = uint32_t(f32_to_bf16(f.x)) | (uint32_t(f32_to_bf16(f.y)) << 16);
            hi = uint32_t(f32_to_bf16(f.z)) | (uint32_t(f32_to_bf16(f.w)) << 16);
        }
        const uint2 v = make_uint2(lo, hi);
        for (int s = 0; s < K; ++s)
            if (dst[s] >= 0) *reinterpret_cast<uint2*>(xperm + int64_t(dst[s]) * H + d) = v;
        if (xrow) *reinterpret_cast<uint2*>(xrow + int64_t(t) * H + d) = v;
    }
}

size_t dispatch_workspace_bytes(int T, int K, int E) {
    const int64_t R = int64_t(T) * K;
    const int64_t nb = (R + kRoutesPerBlock - 1) / kRoutesPerBlock;
    return size_t((nb > 0 ? nb : 1) * E + 16) * sizeof(int32_t);
}

int32_t* dispatch_live_tiles(void* workspace, int T, int K, int E) {
    const int64_t R = int64_t(T) * K;
    const int64_t nb = (R + kRoutesPerBlock - 1) / kRoutesPerBlock;
    return static_cast<int32_t*>(workspace) + (nb > 0 ? nb : 1) * E;
}

hipError_t dispatch_launch(hipStream_t st, const DispatchArgs& a) {
    const int R = a.T * a.K;
    const int nb = (R + kRoutesPerBlock - 1) / kRoutesPerBlock;
    int32_t* bcount = static_cast<int32_t*>(a.workspace);
    int32_t* ntiles = bcount + int64_t(nb > 0 ? nb : 1) * a.E;
    if (nb > 0)
        hipLaunchKernelGGL(disp_count, dim3(nb), dim3(kDispThreads), size_t(a.E) * 4, st, a.ids, R,
                           a.E, bcount);
    // T > 0 here (the callers return before), so nb >= 1
    hipLaunchKernelGGL(disp_colscan, dim3((a.E + kColExperts - 1) / kColExperts),
                       dim3(kColExperts * kColSlices), 0, st, bcount, nb, a.E, a.counts);
    if (!a.tile_e && a.E <= kRankScanMaxE && nb > 0) {
        // no tile table: the rank blocks form the offsets themselves
        hipLaunchKernelGGL(disp_rank_scan, dim3(nb), dim3(kDispThreads), 0, st, a.ids, R, a.E, a.K, bcount,
                           a.counts, a.offsets, a.inverse, a.perm_token, a.mc, ntiles);
    } else {
        hipLaunchKernelGGL(disp_scan, dim3(1), dim3(1024), 0, st, a.E, a.counts, a.offsets, a.tile_e,
                           a.tile_mb, a.tmax, a.mc, ntiles);
        if (nb > 0)
            hipLaunchKernelGGL(disp_rank, dim3(nb), dim3(kDispThreads), 0, st, a.ids, R, a.E, a.K,
                               bcount, a.offsets, a.inverse, a.perm_token);
    }
    if (a.xperm && a.T > 0) {
        if (a.hidden_bf16)
            hipLaunchKernelGGL(disp_permute<true>, dim3(a.T), dim3(kDispThreads), 0, st, a.hidden,
                               a.inverse, a.xperm, a.xrow, a.H, a.K);
        else
            hipLaunchKernelGGL(disp_permute<false>, dim3(a.T), dim3(kDispThreads), 0, st, a.hidden,
                               a.inverse, a.xperm, a.xrow, a.H, a.K);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------- combine

// dst[t][d] = fma chain over slots of w * src[inverse][d] (+ gate * shared).
// One block per token, 4 columns per thread.  KT is the slot count the loops
// are unrolled for (KT == K, or 16 with the slots past K masked), so the
// slot tables stay in registers and all KT row loads are issued before the
// first use.  A skipped slot (p < 0, or s >= K) reads row 0 and is masked
// after the load, not branched around.
template <bool SRC_BF16, bool NT = false>
__device__ __forceinline__ float4 combine_load(const void* src, int64_t row, int H, int d) {
    if constexpr (SRC_BF16) {
        const uint2 u =
            *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(src) + row * H + d);
        return make_float4(bits_f(u.x << 16), bits_f(u.x & 0xFFFF0000u), bits_f(u.y << 16),
                           bits_f(u.y & 0xFFFF0000u));
    } else {
        const float* p = static_cast<const float*>(src) + row * H + d;
        if constexpr (NT) {
            typedef float f4nt __attribute__((ext_vector_type(4)));
            const f4nt v = __builtin_nontemporal_load(reinterpret_cast<const f4nt*>(p));
            return make_float4(v.x, v.y, v.z, v.w);
        } else {
            return *reinterpret_cast<const float4*>(p);
        }
    }
}

template <bool SRC_BF16, int KT, bool NT>
__global__ __launch_bounds__(kDispThreads) void combine_kernel(
    const void* __restrict__ src, const int32_t* __restrict__ inverse,
    const float* __restrict__ rw, const void* __restrict__ shared_src, int shared_bf16,
    const float* __restrict__ gate, float* __restrict__ dst, int H, int K, int p0, int p1,
    int accumulate) {
    const int t = blockIdx.x;
    int p[KT];
    float w[KT];
#pragma unroll
    for (int s = 0; s < KT; ++s) {
        const int sc = s < K ? s : K - 1;
        const int q = s < K ? inverse[int64_t(t) * K + sc] : -1;
        p[s] = (q >= p0 && q < p1) ? q - p0 : -1;   // a route of another range: skipped
        w[s] = rw[int64_t(t) * K + sc];
    }
    const float g = gate ? gate[t] : 1.0f;
    const int step = blockDim.x * 4;
    // two column blocks per pass: 2*KT row loads in flight per lane (the
    // second block is clamped to the first when it falls past H)
    for (int d0 = threadIdx.x * 4; d0 < H; d0 += 2 * step) {
        const bool two = d0 + step < H;
        const int d1 = two ? d0 + step : d0;
        float4 a0[KT], a1[KT];
#pragma unroll
        for (int s = 0; s < KT; ++s) {
            const int64_t row = p[s] < 0 ? 0 : p[s];
            a0[s] = combine_load<SRC_BF16, NT>(src, row, H, d0);
            a1[s] = combine_load<SRC_BF16, NT>(src, row, H, d1);
        }
        float4 v0 = make_float4(0.f, 0.f, 0.f, 0.f), v1 = v0;
        if (accumulate) {
            v0 = *reinterpret_cast<const float4*>(dst + int64_t(t) * H + d0);
            v1 = *reinterpret_cast<const float4*>(dst + int64_t(t) * H + d1);
        }
#pragma unroll
        for (int s = 0; s < KT; ++s) {
            const bool on = p[s] >= 0;
            v0.x = on ? __builtin_fmaf(w[s], a0[s].x, v0.x) : v0.x;
            v0.y = on ? __builtin_fmaf(w[s], a0[s].y, v0.y) : v0.y;
            v0.z = on ? __builtin_fmaf(w[s], a0[s].z, v0.z) : v0.z;
            v0.w = on ? __builtin_fmaf(w[s], a0[s].w, v0.w) : v0.w;
            v1.x = on ? __builtin_fmaf(w[s], a1[s].x, v1.x) : v1.x;
            v1.y = on ? __builtin_fmaf(w[s], a1[s].y, v1.y) : v1.y;
            v1.z = on ? __builtin_fmaf(w[s], a1[s].z, v1.z) : v1.z;
            v1.w = on ? __builtin_fmaf(w[s], a1[s].w, v1.w) : v1.w;
        }
        if (shared_src) {
            const float4 b0 = shared_bf16 ? combine_load<true>(shared_src, t, H, d0)
                                          : combine_load<false>(shared_src, t, H, d0);
            const float4 b1 = shared_bf16 ? combine_load<true>(shared_src, t, H, d1)
                                          : combine_load<false>(shared_src, t, H, d1);
            v0.x = __builtin_fmaf(g, b0.x, v0.x); v0.y = __builtin_fmaf(g, b0.y, v0.y);
            v0.z = __builtin_fmaf(g, b0.z, v0.z); v0.w = __builtin_fmaf(g, b0.w, v0.w);
            v1.x = __builtin_fmaf(g, b1.x, v1.x); v1.y = __builtin_fmaf(g, b1.y, v1.y);
            v1.z = __builtin_fmaf(g, b1.z, v1.z); v1.w = __builtin_fmaf(g, b1.w, v1.w);
        }
        *reinterpret_cast<float4*>(dst + int64_t(t) * H + d0) = v0;
        if (two) *reinterpret_cast<float4*>(dst + int64_t(t) * H + d1) = v1;
    }
}

// Expert rows larger than the last-level cache (256 MiB) stream through
// with non-temporal loads; smaller ones (a few tokens' rows, just written by
// the down projection) are still cached and load normally.
constexpr int64_t kCombineStreamBytes = int64_t(256) << 20;

template <bool SRC_BF16, bool NT>
static void combine_k(hipStream_t st, const CombineArgs& a) {
#define GRIM_COMBINE(KT)                                                                          \
    hipLaunchKernelGGL((combine_kernel<SRC_BF16, KT, NT>), dim3(a.T), dim3(kDispThreads), 0, st,  \
                       a.src, a.inverse, a.rw, a.shared_src, a.shared_bf16, a.gate, a.dst, a.H,   \
                       a.K, a.p0, a.p1, a.accumulate)
    switch (a.K) {
        case 1: GRIM_COMBINE(1); break;
        case 2: GRIM_COMBINE(2); break;
        case 4: GRIM_COMBINE(4); break;
        case 6: GRIM_COMBINE(6); break;
        case 8: GRIM_COMBINE(8); break;
        case 10: GRIM_COMBINE(10); break;
        default: GRIM_COMBINE(16); break;
    }
#undef GRIM_COMBINE
}

// Routes of one expert shard: an expert in [begin, begin + count) becomes
// its local index, any other route expert -1 with weight 0
// (src/grimoire.cpp:15392-15399, :23231-23240).
__global__ __launch_bounds__(256) void route_local_kernel(const int32_t* __restrict__ ids,
                                                          const float* __restrict__ w,
                                                          int32_t* __restrict__ lids, float* __restrict__ lw,
                                                          int R, int begin, int count) {
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= R) return;
    const int e = ids[r];
    const bool own = e >= begin && e - begin < count;
    lids[r] = own ? e - begin : -1;
    lw[r] = own ? w[r] : 0.0f;
}

hipError_t route_local_launch(hipStream_t st, const int32_t* ids, const float* w, int32_t* lids, float* lw,
                              int R, int begin, int count) {
    if (R <= 0) return hipSuccess;
    route_local_kernel<<<(R + 255) / 256, 256, 0, st>>>(ids, w, lids, lw, R, begin, count);
    return hipGetLastError();
}

hipError_t combine_launch(hipStream_t st, const CombineArgs& a) {
    if (a.T <= 0) return hipSuccess;
    if (a.K <= 0 || a.K > 16) return hipErrorInvalidValue;
    const bool nt = int64_t(a.T) * a.K * a.H * (a.src_bf16 ? 2 : 4) > kCombineStreamBytes;
    if (a.src_bf16) nt ? combine_k<true, true>(st, a) : combine_k<true, false>(st, a);
    else nt ? combine_k<false, true>(st, a) : combine_k<false, false>(st, a);
    return hipGetLastError();
}

// ------------------------------------------------ combine + residual + RMSNorm

// launch_rmsnorm_moe_residual_batched (src/prefill.cpp:1004-1045): per token
//   v = h + shared, then v = fma(w_s, bf16 routed[inverse[s]], v) in slot
//   order; h = v; out = v * rsqrt(sum v^2 / H + eps) * (offset + bf16 w).
// KT == 0 is launch_rmsnorm_residual_batched (src/prefill.cpp:627-700):
//   v = (h + r0) + r1, h written back only when a residual was added.
// One block per token, 4 columns per thread.  The first kNormRegChunks
// chunks of v stay in registers between the two passes, so H <= 8192 reads
// h, shared and the routed rows once and writes h and out once; wider rows
// re-read their tail of h, which this thread itself wrote.
constexpr int kNormRegChunks = 8;

template <int KT>
__device__ __forceinline__ float4 norm_chunk(const float* __restrict__ h,
                                             const float* __restrict__ sh,
                                             const float* __restrict__ sh2,
                                             const uint16_t* __restrict__ routed, const int* p,
                                             const float* w, int H, int d) {
    float4 v = *reinterpret_cast<const float4*>(h + d);
    if (sh) {
        const float4 a = *reinterpret_cast<const float4*>(sh + d);
        v.x += a.x; v.y += a.y; v.z += a.z; v.w += a.w;
    }
    if (sh2) {
        const float4 a = *reinterpret_cast<const float4*>(sh2 + d);
        v.x += a.x; v.y += a.y; v.z += a.z; v.w += a.w;
    }
    uint2 u[KT > 0 ? KT : 1];
#pragma unroll
    for (int s = 0; s < KT; ++s) {
        const int64_t row = p[s] < 0 ? 0 : p[s];
        u[s] = *reinterpret_cast<const uint2*>(routed + row * H + d);
    }
#pragma unroll
    for (int s = 0; s < KT; ++s) {
        const bool on = p[s] >= 0;
        v.x = on ? __builtin_fmaf(w[s], bits_f(u[s].x << 16), v.x) : v.x;
        v.y = on ? __builtin_fmaf(w[s], bits_f(u[s].x & 0xFFFF0000u), v.y) : v.y;
        v.z = on ? __builtin_fmaf(w[s], bits_f(u[s].y << 16), v.z) : v.z;
        v.w = on ? __builtin_fmaf(w[s], bits_f(u[s].y & 0xFFFF0000u), v.w) : v.w;
    }
    return v;
}

__device__ __forceinline__ void norm_store(const NormArgs& a, int64_t base, int d, float4 v,
                                           float scale) {
    const uint2 wb = *reinterpret_cast<const uint2*>(a.weight + d);
    float4 o;
    o.x = v.x * scale * (a.offset + bits_f(wb.x << 16));
    o.y = v.y * scale * (a.offset + bits_f(wb.x & 0xFFFF0000u));
    o.z = v.z * scale * (a.offset + bits_f(wb.y << 16));
    o.w = v.w * scale * (a.offset + bits_f(wb.y & 0xFFFF0000u));
    if (a.out) *reinterpret_cast<float4*>(a.out + base + d) = o;
    if (a.out_bf) {
        uint2 b;
        b.x = uint32_t(f32_to_bf16(o.x)) | (uint32_t(f32_to_bf16(o.y)) << 16);
        b.y = uint32_t(f32_to_bf16(o.z)) | (uint32_t(f32_to_bf16(o.w)) << 16);
        *reinterpret_cast<uint2*>(a.out_bf + base + d) = b;
    }
}

template <int KT>
__global__ __launch_bounds__(kDispThreads) void combine_norm_kernel(NormArgs a) {
    const int t = blockIdx.x, H = a.H, K = a.K;
    const int64_t base = int64_t(t) * H;
    int p[KT > 0 ? KT : 1];
    float w[KT > 0 ? KT : 1];
#pragma unroll
    for (int s = 0; s < KT; ++s) {
        const int sc = s < K ? s : K - 1;
        p[s] = s < K ? a.inverse[int64_t(t) * K + sc] : -1;
        w[s] = a.rw[int64_t(t) * K + sc];
    }
    float* ht = a.h + base;
    const float* sh = a.shared ? a.shared + base : nullptr;
    const float* sh2 = a.shared2 ? a.shared2 + base : nullptr;
    const bool write_h = KT > 0 || sh || sh2;
    const int step = kDispThreads * 4;
    float4 keep[kNormRegChunks];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < kNormRegChunks; ++c) {
        const int d = threadIdx.x * 4 + c * step;
        if (d < H) {
            keep[c] = norm_chunk<KT>(ht, sh, sh2, a.routed, p, w, H, d);
            if (write_h) *reinterpret_cast<float4*>(ht + d) = keep[c];
            ss = __builtin_fmaf(keep[c].x, keep[c].x, ss);
            ss = __builtin_fmaf(keep[c].y, keep[c].y, ss);
            ss = __builtin_fmaf(keep[c].z, keep[c].z, ss);
            ss = __builtin_fmaf(keep[c].w, keep[c].w, ss);
        }
    }
    for (int d = threadIdx.x * 4 + kNormRegChunks * step; d < H; d += step) {
        const float4 v = norm_chunk<KT>(ht, sh, sh2, a.routed, p, w, H, d);
        if (write_h) *reinterpret_cast<float4*>(ht + d) = v;
        ss = __builtin_fmaf(v.x, v.x, ss);
        ss = __builtin_fmaf(v.y, v.y, ss);
        ss = __builtin_fmaf(v.z, v.z, ss);
        ss = __builtin_fmaf(v.w, v.w, ss);
    }
    __shared__ float part[kDispThreads / kWave];
    ss = group_sum<kWave>(ss);
    if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = ss;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < kDispThreads / kWave; ++i) total += part[i];
    const float scale = rsqrtf(total / float(H) + a.eps);
#pragma unroll
    for (int c = 0; c < kNormRegChunks; ++c) {
        const int d = threadIdx.x * 4 + c * step;
        if (d < H) norm_store(a, base, d, keep[c], scale);
    }
    for (int d = threadIdx.x * 4 + kNormRegChunks * step; d < H; d += step)
        norm_store(a, base, d, *reinterpret_cast<const float4*>(ht + d), scale);
}

hipError_t combine_norm_launch(hipStream_t st, const NormArgs& a) {
    if (a.T <= 0) return hipSuccess;
    if (a.K < 0 || a.K > 16 || a.H % 4) return hipErrorInvalidValue;
#define GRIM_NORM(KT) \
    hipLaunchKernelGGL((combine_norm_kernel<KT>), dim3(a.T), dim3(kDispThreads), 0, st, a)
    switch (a.K) {
        case 0: GRIM_NORM(0); break;
        case 1: GRIM_NORM(1); break;
        case 2: GRIM_NORM(2); break;
        case 4: GRIM_NORM(4); break;
        case 6: GRIM_NORM(6); break;
        case 8: GRIM_NORM(8); break;
        case 10: GRIM_NORM(10); break;
        default: GRIM_NORM(16); break;
    }
#undef GRIM_NORM
    return hipGetLastError();
}

}  // namespace grim
