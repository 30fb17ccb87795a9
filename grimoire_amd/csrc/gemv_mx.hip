// gemv_mx.hip -- the expert-grouped GEMV for MXFP4 experts on the scaled
// fp4 x fp8 matrix core (v_mfma_scale_f32_16x16x128_f8f6f4).
//
// Same work as gemv_grouped.hip (each touched expert's weights streamed once
// per group of up to kGvMT of its rows), with the arithmetic moved off the
// vector ALU: the e2m1 weight codes and their e8m0 block scales go to the
// matrix core exactly as stored, and the activations are split into three
// e4m3 limbs under one e8m0 scale per 32-element block,
//     x = 2^s (hi + mid + lo),   s = floor(log2 max|block|) - 7,
// each limb the round-to-nearest e4m3 of what the previous ones left: the
// three cover 12 significant bits of every value within 2^9 of its block's
// largest one (bf16 values, 8 bits, exactly).  One MFMA per limb
// accumulates 16 weight rows x 16 activation rows x 128 K in fp32; the
// group's <= 4 rows use 4 of the 16 columns and the others are never
// stored.  The vector ALU is left with the SwiGLU and the stores.
//
// Operand layout of the instruction with A = e2m1 and B = e4m3 (measured
// with one-hot operands): lane l of A holds row l % 16 and the 32-element
// K block g = l / 16 of the 128 (16 bytes, element p at nibble p, low
// nibble first: a weight row's stored bytes), with that block's scale; lane
// l of B holds column l % 16 and, in its 32 bytes, elements [16 (g & 1),
// +16) of blocks (g >> 1) and (g >> 1) + 2, with the scale of block g; D
// holds column l % 16, rows 4 (l / 16) + [0, 4).
//
// Each wave owns 64 weight rows of an item (gate_up: 32 gate and the
// matching 32 up rows) and walks K in stages of 256 (two MFMA steps): per
// stage its rows' 8 KiB of codes and their scale bytes, and the group's
// limb rows at the stage with their scales, stream through its own
// three-stage LDS ring by buffer_load ... lds (code slots XOR-swizzled so
// that the 16-row operand reads are free of bank conflicts), and 4 row
// blocks x 3 limbs of MFMAs per step accumulate.  K is padded to whole
// stages: the activation limbs past K are zero and the weight tail is
// masked.  One continuous stage stream runs across a wave's items, so an
// item starts with its data in flight.  Like gemv_grouped.hip: one
// work-group per CU, no barrier, every wave waits on its own vmcnt only.
// Scale rows that are 16-byte aligned (K % 512 == 0) come in a 16-byte lane
// per row for two stages at a time (gvm_kernel<., true>); weight rows that
// straddle memory lines are loaded without the non-temporal hint.
//
// Also here: the formatting of activation rows into limbs, and for small
// batches the dispatch (counts, offsets, group table, stable ranks) in one
// launch beside that formatting (gvm_route_kernel).
#include "gemv_mx.hpp"

#include "gemv_impl.hpp"

namespace grim {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* gvm_lds_ptr_t;

// Wave timestamps for kernel studies, compiled in only with GRIM_TIMING: 16
// per wave of the grid (wave 4 b + w), lane 0: 0 start, 1 first stage in,
// 2 + k end of the wave's item k (k < 13), 15 exit.
#ifdef GRIM_TIMING
#define GVM_TS(i)                                                                                 \
    do {                                                                                          \
        if (a.ts && lane == 0 && (i) < 16)                                                        \
            a.ts[(blockIdx.x * kGvmWaves + wave) * 16 + (i)] = __builtin_amdgcn_s_memrealtime();   \
    } while (0)
#else
#define GVM_TS(i) do {} while (0)
#endif

constexpr int kGvmWaves = 4;
constexpr int kGvmRows = 64;                    // weight rows per wave and item
constexpr int kGvmKS = 256;                     // K per ring stage (two MFMA steps)
constexpr int kGvmStages = 3;                   // ring stages per wave
constexpr int kGvmLimbs = 3;
// stage: codes 64 rows x 128 B, their scales 64 x 8 B, the group's limb rows
// 4 x 3 x 256 B, their scales 4 x 8 B
constexpr int kGvmOS = kGvmRows * kGvmKS / 2;                       // 8192
// (each row's 8 scale bytes come in the 12 from their 4-byte-aligned start)
constexpr int kGvmOA = kGvmOS + kGvmRows * 12;                      // 8960
constexpr int kGvmOAS = kGvmOA + 4 * kGvmLimbs * kGvmKS;            // 12032
constexpr int kGvmStage = kGvmOAS + 256;                            // 12288
// a buffer offset past every activation descriptor's range
constexpr int kGvmNoLoad = int(0x80000000u);

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gvm_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

// Scalar load of one int from a wave-uniform address.  It waits on
// lgkmcnt, not vmcnt: the item descriptors read between stages do not wait
// for the DMA ring in flight (a compiler-visible vector load there would
// bring an s_waitcnt vmcnt(0) that drains it).
__device__ __forceinline__ int gvm_sload(const int32_t* p) {
    int v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
    return v;
}

__device__ __forceinline__ uint32_t gvm_lds_addr(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t*)(p)));
}

// K padded to whole stages.
__host__ __device__ inline int gvm_kpad(int K) { return (K + kGvmKS - 1) / kGvmKS * kGvmKS; }

// Activation row in the limb format, K padded to Kp = gvm_kpad(K) with
// zeros: limb L's Kp bytes at L * Kp, then one e8m0 scale per 32-element
// block at 3 Kp; rounded to 16 bytes.
__host__ __device__ inline int gvm_row_bytes(int K) {
    const int kp = gvm_kpad(K);
    return (3 * kp + kp / 32 + 15) & ~15;
}

size_t gvm_act_bytes(int K) { return size_t(gvm_row_bytes(K)); }

// Block scale exponent s (e8m0 byte s + 127) of a 32-element block whose
// largest magnitude is mx, and inv = 2^-s: the largest value lands in
// [128, 256), inside e4m3's range of 448.
__device__ __forceinline__ int gvm_block_scale(float mx, float& inv) {
    const int ex = mx > 0.0f ? int((f_bits(mx) >> 23) & 0xFF) - 127 : -127;
    const int s = max(-127, min(127, ex - 7));
    inv = bits_f(uint32_t(127 - s) << 23);   // 2^-s (s >= -127: 2^127 at most)
    return s;
}

// Four consecutive values times inv as three e4m3 limbs (each the
// remainder of the ones before), one packed word per limb.
__device__ __forceinline__ void gvm_limbs4(const float* v, float inv, uint32_t (&q)[kGvmLimbs]) {
    float r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = v[j] * inv;
#pragma unroll
    for (int L = 0; L < kGvmLimbs; ++L) {
        int p = __builtin_amdgcn_cvt_pk_fp8_f32(r[0], r[1], 0, false);
        p = __builtin_amdgcn_cvt_pk_fp8_f32(r[2], r[3], p, true);
        q[L] = uint32_t(p);
        r[0] -= __builtin_amdgcn_cvt_f32_fp8(p, 0);
        r[1] -= __builtin_amdgcn_cvt_f32_fp8(p, 1);
        r[2] -= __builtin_amdgcn_cvt_f32_fp8(p, 2);
        r[3] -= __builtin_amdgcn_cvt_f32_fp8(p, 3);
    }
}

// Block b (32 elements) of one row: src the row (K floats), dst its limb
// row (gvm_row_bytes(K)); blocks past K give zero limbs (scale byte 0).
__device__ __forceinline__ void gvm_format_block(const float* __restrict__ src, uint8_t* __restrict__ dst, int K,
                                                 int kp, int b) {
    const float4* s4 = reinterpret_cast<const float4*>(src + b * 32);
    float v[32];
    const bool in = b * 32 < K;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 q = in ? s4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        v[4 * i] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) mx = fmaxf(mx, fabsf(v[i]));
    float inv;
    const int s = gvm_block_scale(mx, inv);
    uint32_t w[3][8];
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        uint32_t q[kGvmLimbs];
        gvm_limbs4(v + i, inv, q);
#pragma unroll
        for (int L = 0; L < kGvmLimbs; ++L) w[L][i / 4] = q[L];
    }
#pragma unroll
    for (int L = 0; L < kGvmLimbs; ++L) {
        uint4* d4 = reinterpret_cast<uint4*>(dst + int64_t(L) * kp + b * 32);
        d4[0] = make_uint4(w[L][0], w[L][1], w[L][2], w[L][3]);
        d4[1] = make_uint4(w[L][4], w[L][5], w[L][6], w[L][7]);
    }
    dst[3 * kp + b] = uint8_t(s + 127);
}

// One thread per 32-element block of the padded row.
__global__ __launch_bounds__(256) void gvm_format_kernel(const float* src0, int rows0, uint8_t* dst0,
                                                         const float* src1, int rows1, uint8_t* dst1, int K) {
    const int kp = gvm_kpad(K), nb = kp / 32;
    const int64_t gi = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t n0 = int64_t(rows0) * nb;
    if (gi >= n0 + int64_t(rows1) * nb) return;
    const bool second = gi >= n0;
    const int64_t li = second ? gi - n0 : gi;
    const int row = int(li / nb), b = int(li % nb);
    gvm_format_block((second ? src1 : src0) + int64_t(row) * K, (second ? dst1 : dst0) + int64_t(row) * gvm_row_bytes(K),
                     K, kp, b);
}

hipError_t gvm_format_launch(hipStream_t st, const float* src0, int rows0, uint8_t* dst0, const float* src1,
                             int rows1, uint8_t* dst1, int K) {
    const int64_t n = int64_t(rows0 + rows1) * (gvm_kpad(K) / 32);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(gvm_format_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st, src0, rows0, dst0, src1,
                       rows1, dst1, K);
    return hipGetLastError();
}

// ------------------------------------------------- small-batch routing
//
// Everything between the top-k and the grouped GEMV for a batch of at most
// kGvmRouteMax routes in one launch instead of five (the dispatch's count /
// column scan / scan / rank and the activation formatting).  Work-group 0:
// the expert counts come from LDS atomics (counts only: order-free), one
// scan forms the offsets and the (expert, group of kGvMT rows) table, and
// each route's row is its expert's offset plus the number of earlier
// routes of that expert -- the dispatch's stable order
// (src/grimoire.cpp:23162-23170).  Up to 16 tokens the top-k runs in
// work-group 0 first, one wave per token; more tokens take a launch of their
// own (all their top-k in one work-group would share one CU).  The x rows are
// formatted as limbs by the same code as gvm_format_kernel, one block of
// 32 elements per thread of the launch's other work-groups.
constexpr int kGvmRouteThreads = 1024;

__global__ __launch_bounds__(kGvmRouteThreads) void gvm_route_kernel(TopkArgs tk, GvmRouteArgs ra, int fused_topk) {
    if (blockIdx.x > 0) {
        // work-groups 1..: the x rows in the limb format, in parallel with
        // the routing in work-group 0
        const int kp = gvm_kpad(ra.H), nb = kp / 32;
        const int ab = gvm_row_bytes(ra.H);
        const int i = (int(blockIdx.x) - 1) * kGvmRouteThreads + int(threadIdx.x);
        if (i < tk.T * nb)
            gvm_format_block(ra.x + int64_t(i / nb) * ra.H, ra.af + int64_t(i / nb) * ab, ra.H, kp, i % nb);
        return;
    }
    __shared__ __attribute__((aligned(16))) int32_t ids[kGvmRouteMax];
    __shared__ int32_t cnt[kGvmRouteThreads], wsum[kGvmRouteThreads / kWave][2];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid / kWave;
    const int T = tk.T, E = tk.E, K = tk.K, R = T * K;
    cnt[tid] = 0;
    if (fused_topk) {
        // T <= 16: wave t selects token t's experts (topk_kernel's code,
        // so the same bits) into LDS; the picks are stored from there
        __shared__ float gsel[kGvmRouteThreads / kWave][512];
        __shared__ float gscore[kGvmRouteThreads / kWave][64];
        __shared__ int32_t pick_e[kGvmRouteThreads / kWave][16];
        __shared__ float pick_w[kGvmRouteThreads / kWave][16];
        if (wv < T)
            topk_wave(tk.logits + int64_t(wv) * E, E, K, tk.mode, tk.normalize, tk.scaling, tk.bias16, tk.bias32,
                      tk.n_group, tk.topk_group, pick_e[wv], pick_w[wv], gsel[wv], gscore[wv]);
        __syncthreads();
        if (tid < R) {
            const int32_t pe = pick_e[tid / K][tid % K];
            ids[tid] = pe;
            tk.out_e[tid] = pe;
            tk.out_w[tid] = pick_w[tid / K][tid % K];
        }
    } else {
        if (tid < R) ids[tid] = tk.out_e[tid];
    }
    __syncthreads();
    const int my_id = tid < R ? ids[tid] : -1;
    if (my_id >= 0 && my_id < E) atomicAdd(&cnt[my_id], 1);
    __syncthreads();
    // inclusive scans of the counts and of the groups per expert: within
    // each wave by lane shifts, then the waves' totals (two barriers in
    // place of a block-wide scan's twenty)
    const int c = tid < E ? cnt[tid] : 0;
    const int ng = (c + kGvMT - 1) / kGvMT;
    int ic = c, ig = ng;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int a = __shfl_up(ic, off, kWave), b = __shfl_up(ig, off, kWave);
        if (lane >= off) { ic += a; ig += b; }
    }
    if (lane == kWave - 1) { wsum[wv][0] = ic; wsum[wv][1] = ig; }
    __syncthreads();
    int bc = 0, bg = 0, groups = 0;
    for (int w = 0; w < kGvmRouteThreads / kWave; ++w) {
        const int tc = wsum[w][0], tg = wsum[w][1];
        bc += w < wv ? tc : 0;
        bg += w < wv ? tg : 0;
        groups += tg;
    }
    const int off_e = bc + ic - c, g0 = bg + ig - ng;
    if (tid < E) {
        ra.counts[tid] = c;
        ra.offsets[tid] = off_e;
        for (int i = 0; i < ng; ++i)
            if (g0 + i < ra.tmax) {
                ra.tile_e[g0 + i] = tid;
                ra.tile_mb[g0 + i] = i;
            }
    }
    for (int g = groups + tid; g < ra.tmax; g += kGvmRouteThreads) {
        ra.tile_e[g] = -1;
        ra.tile_mb[g] = 0;
    }
    if (tid == 0) *ra.n_live = groups < ra.tmax ? groups : ra.tmax;
    __syncthreads();
    cnt[tid] = off_e;   // the offsets, for the ranks
    __syncthreads();
    if (tid < R) {
        int dest = -1;
        if (my_id >= 0 && my_id < E) {
            // earlier routes of the same expert: four ids per 16-byte read,
            // four reads in flight (the same count as a route-by-route loop)
            int rank = 0;
            const int4* ids4 = reinterpret_cast<const int4*>(ids);
            const int n4 = (tid + 3) / 4;
#pragma unroll 4
            for (int j = 0; j < n4; ++j) {
                const int4 v = ids4[j];
                rank += (v.x == my_id && 4 * j < tid) ? 1 : 0;
                rank += (v.y == my_id && 4 * j + 1 < tid) ? 1 : 0;
                rank += (v.z == my_id && 4 * j + 2 < tid) ? 1 : 0;
                rank += (v.w == my_id && 4 * j + 3 < tid) ? 1 : 0;
            }
            dest = cnt[my_id] + rank;
            ra.perm_token[dest] = tid / K;
        }
        ra.inverse[tid] = dest;
    }
}

hipError_t gvm_route_launch(hipStream_t st, const TopkArgs& tk, const GvmRouteArgs& ra) {
    if (int64_t(tk.T) * tk.K > kGvmRouteMax || tk.E > 512 || tk.E <= 0) return hipErrorInvalidValue;
    // up to one token per wave of work-group 0: the top-k in this launch
    const int fused = tk.T <= kGvmRouteThreads / kWave;
    if (!fused) {
        hipError_t e = topk_launch(st, tk);
        if (e != hipSuccess) return e;
    }
    const int64_t blocks = int64_t(tk.T) * (gvm_kpad(ra.H) / 32);
    const int fmt_groups = int((blocks + kGvmRouteThreads - 1) / kGvmRouteThreads);
    hipLaunchKernelGGL(gvm_route_kernel, dim3(1 + fmt_groups), dim3(kGvmRouteThreads), 0, st, tk, ra, fused);
    return hipGetLastError();
}

// Stage s of an item into the ring stage at st: exactly 13 instructions,
// every lane active (the stage loop's vmcnt wait counts 13 per stage: a
// lane-masked load whose lanes are all off would be branched around and
// not counted).  Lanes with nothing to load read past the buffer
// (kGvmNoLoad): zeros, into LDS that no MFMA of theirs reads.  Codes: instruction j covers the wave's rows
// 8 j + lane / 8, slot lane % 8 holding 16-byte piece (lane % 8) ^
// ((row >> 1) & 7).  Scales: row lane's 16 bytes at sup + 16 lane (S16:
// two stages' 8 bytes every other stage; else the stage's 8 bytes inside
// the 16 from their 4-byte-aligned start).  Activations: piece p = 64 ja + lane of [row m][limb L]
// [16 x 16 B] (192 pieces; rows past mc are not loaded: their columns are
// never stored), then the 4 rows' 8 block scales (lane = 2 m + half).
template <bool S16>
__device__ __forceinline__ void gvm_issue(uint8_t* st, uint8_t* sup, __amdgpu_buffer_rsrc_t rp,
                                          __amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t ra, const int (&pofs)[8],
                                          const int (&sofs)[3], const int (&aofs)[3], int asofs, int mc, int lane,
                                          int s, bool nt) {
    static_assert(kGvmStages <= 3, "a stage's scale window buffer: one of the wave's three 1 KiB areas");
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        // non-temporal when a row's 128 bytes of a stage are whole memory
        // lines; rows that straddle lines (K/2 % 128 != 0) keep them cached,
        // for the next stage reads the rest of each line
        if (nt) __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, (gvm_lds_ptr_t)(st + j * 1024), 16, pofs[j], s * 128, 0, 2);
        else __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, (gvm_lds_ptr_t)(st + j * 1024), 16, pofs[j], s * 128, 0, 0);
    }
    if constexpr (S16) {
        // even stages: the next two stages' scales of the wave's 64 rows,
        // 16 bytes a lane (row = lane), into the super-stage buffer sup;
        // odd stages: the same instruction past the buffer, into a dummy
        // area (one load per stage either way)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (gvm_lds_ptr_t)sup, 16, (s & 1) ? kGvmNoLoad : sofs[0],
                                                 (s >> 1) * 16, 0, 0);
    } else {
        // the stage's 8 scale bytes of each of the wave's 64 rows inside a
        // 16-byte window from their 4-byte-aligned start (row = lane; the
        // 8 bytes start 0 or 2 bytes in), into the stage's own 1 KiB of sup:
        // one instruction, where three 4-byte-lane ones (each reaching 21
        // rows' lines) cost ~10% of a C3 layer
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (gvm_lds_ptr_t)sup, 16, sofs[0], s * 8, 0, 0);
    }
#pragma unroll
    for (int ja = 0; ja < 3; ++ja) {
        const int vo = (64 * ja + lane) / 48 < mc ? aofs[ja] : kGvmNoLoad;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (gvm_lds_ptr_t)(st + kGvmOA + ja * 1024), 16, vo, s * 256, 0, 0);
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (gvm_lds_ptr_t)(st + kGvmOAS), 4, lane < 8 ? asofs : kGvmNoLoad,
                                             s * 8, 0, 0);
}

// One persistent kernel for both products (GU: gate_up + SwiGLU, rows are
// (gate, up) pairs, out h; else down, out y).  Items are per wave: (group,
// chunk of 32 pairs / 64 rows); wave w of work-group b walks 4 b + w,
// + 4 gridDim.x, ...
// A wave's ring stage s (K [256 s, +256)) holds its 64 rows' codes (one
// 128-byte line per row), their scales, and the group's limb rows at those
// K with their block scales: everything a stage's MFMAs read comes with the
// stage, so one vmcnt wait per stage covers it.
// S16: scale rows 16-byte aligned (K % 512 == 0): a row's scales for two
// stages come as one 16-byte lane of one instruction every other stage
// (instead of three 4-byte-lane instructions per stage, each reaching 64
// rows' lines), into a double-buffered per-wave super-stage area.
template <bool GU, bool S16>
__global__ __launch_bounds__(kGvmWaves * kWave) void gvm_kernel(GvArgs a) {
    constexpr int NT = 13;                                   // DMA instructions per stage
    constexpr int ST = kGvmStages;
    constexpr int WAIT = NT * (ST - 1);
    static_assert(WAIT <= 63, "vmcnt holds 63");
    extern __shared__ __attribute__((aligned(1024))) uint8_t gvm_ring[];
    const int N = a.N, Kd = a.K, Kp = gvm_kpad(Kd), S = Kp / kGvmKS;
    const int lrow = Kd / 2, srb = Kd / 32;                  // code / scale bytes per weight row
    const int AB = gvm_row_bytes(Kd);
    const bool nt = lrow % 128 == 0;
    constexpr int PW = GU ? kGvmRows / 2 : kGvmRows;         // rows (pairs) per wave
    constexpr int NRB = kGvmRows / 16;                       // 16-row blocks per wave
    const int rows_per_expert = GU ? 2 * N : N;
    // items are per wave: (group, chunk of PW rows / pairs); wave w of
    // work-group b takes items 4 b + w, + 4 gridDim.x, ... (the waves of a
    // work-group share nothing, so a wave needs no partner: an expert whose
    // rows end mid-work-group leaves no wave idle on padding, and the last
    // round spreads over the waves of every work-group)
    const int n_chunks = (N + PW - 1) / PW;
    const int wstride = int(gridDim.x) * kGvmWaves;
    const int n_live = __builtin_amdgcn_readfirstlane(*a.n_live);
    const int groups = n_live + (a.T_sh + kGvMT - 1) / kGvMT;
    const int n_items = groups * n_chunks;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) / kWave);
    uint8_t* ring = gvm_ring + wave * (ST * kGvmStage);
    // per wave: two 1 KiB super-stage scale buffers and a 1 KiB dummy area
    uint8_t* supw = gvm_ring + kGvmWaves * ST * kGvmStage + wave * 3 * 1024;
    const uint32_t sup_base = gvm_lds_addr(supw);
    const uint32_t ring_base = gvm_lds_addr(ring);
    const int col = lane & 15, grp = lane >> 4;              // B / D column, lane group

    // One item's addressing: its weight and activation descriptors and the
    // per-lane DMA offsets (see issue below), its rows and outputs.
    struct Desc {
        const uint8_t* pb;     // the expert's codes, scales; the activation rows
        const uint8_t* sbp;
        const uint32_t* ab;
        int pofs[8], sofs[3], aofs[3], asofs;
        int r0, mc, i0;
        bool sh;
    };
    // The item with index >= item0 that has rows, in this work-group's
    // order (mc = 0: none left).
    auto make = [&](int item0, int& item) {
        Desc d;
        d.mc = 0;
        for (item = item0; item < n_items; item += wstride) {
            const int g = item / n_chunks, chunk = item % n_chunks;
            int64_t wrow0 = 0;
            if (g < n_live) {
                const int e = gvm_sload(a.tile_e + g);
                if (e < 0) continue;   // uniform
                const int mb = gvm_sload(a.tile_mb + g);
                d.r0 = gvm_sload(a.offsets + e) + mb * kGvMT;
                d.mc = min(kGvMT, gvm_sload(a.counts + e) - mb * kGvMT);
                wrow0 = int64_t(e) * rows_per_expert;
                d.sh = false;
            } else {
                d.r0 = (g - n_live) * kGvMT;
                d.mc = min(kGvMT, a.T_sh - d.r0);
                d.sh = true;
            }
            if (d.mc <= 0) continue;   // uniform
            const WView& w = d.sh ? a.w_sh : a.w;
            d.pb = w.payload + wrow0 * lrow;
            d.sbp = static_cast<const uint8_t*>(w.scales) + wrow0 * srb;
            d.ab = d.sh ? a.af_sh : a.af;
            d.i0 = chunk * PW;                               // this wave's first row (pair)
            // weight row of the wave's row r (GU: r < 32 gate, else up); rows
            // past N repeat the last (loaded, never stored)
            auto wrow = [&](int r) {
                if constexpr (GU) return (r >= PW ? N : 0) + min(d.i0 + (r & (PW - 1)), N - 1);
                else return min(d.i0 + r, N - 1);
            };
            // activation row of group row m (rows past mc: row 0, never used)
            // (four named values selected per lane: an indexed array here
            // goes to scratch memory, whose loads wait like the ring's)
            static_assert(kGvMT == 4, "four group rows");
            auto trow = [&](int m) {
                const int rr = d.r0 + (m < d.mc ? m : 0);
                return (GU && !d.sh) ? gvm_sload(a.perm_token + rr) : rr;
            };
            const int ar0 = trow(0), ar1 = trow(1), ar2 = trow(2), ar3 = trow(3);
            auto arow = [&](int m) {
                // per-lane select in the vector ALU (the optimiser turns a
                // plain select chain back into an indexed table)
                int v = ar0;
                asm volatile("v_cmp_eq_u32_e32 vcc, 1, %1\n\t"
                             "v_cndmask_b32_e32 %0, %0, %2, vcc\n\t"
                             "v_cmp_eq_u32_e32 vcc, 2, %1\n\t"
                             "v_cndmask_b32_e32 %0, %0, %3, vcc\n\t"
                             "v_cmp_eq_u32_e32 vcc, 3, %1\n\t"
                             "v_cndmask_b32_e32 %0, %0, %4, vcc"
                             : "+v"(v) : "v"(m), "v"(ar1), "v"(ar2), "v"(ar3) : "vcc");
                return v;
            };
            // Codes: instruction j covers rows 8 j + lane / 8, slot lane % 8
            // holding 16-byte piece (lane % 8) ^ ((row >> 1) & 7).  Scales:
            // instruction jj covers rows 32 jj + lane / 2, 4 bytes each.
            // Activations: piece p = 64 ja + lane of [row m][limb L][16 x 16 B]
            // (192 pieces), then the 4 rows' 8 block scales (lane = 2 m + half).
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int r = 8 * j + (lane >> 3);
                d.pofs[j] = wrow(r) * lrow + (((lane & 7) ^ ((r >> 1) & 7)) << 4);
            }
            // row lane's scales (S16: 16-byte aligned; else from the 4-byte-
            // aligned start of its first byte)
            d.sofs[0] = S16 ? wrow(lane) * srb : (wrow(lane) * srb) & ~3;
            d.sofs[1] = d.sofs[2] = 0;
#pragma unroll
            for (int ja = 0; ja < 3; ++ja) {
                const int pc = 64 * ja + lane;
                d.aofs[ja] = arow(pc / 48) * AB + ((pc / 16) % 3) * Kp + (pc % 16) * 16;
            }
            d.asofs = arow((lane >> 1) & 3) * AB + 3 * Kp + (lane & 1) * 4;
            break;
        }
        return d;
    };
    // buffer descriptors of the current and the next item (codes, scales,
    // activation rows)
    __amdgpu_buffer_rsrc_t cp, cs, ca, np, ns, na;
    Desc cur, nxt;
    // Stage s of the current item (the next one when nx) into ring slot
    // q % ST (gvm_issue)
    // (S16: global stage q's super-stage buffer is (q / 2) % 2; items hold
    // an even number of stages, so q and s have the same parity; else the
    // stage's scale window buffer q % 3, reused with its ring slot)
    auto issue = [&](bool nx, int s, int q) {
        uint8_t* sup = S16 ? supw + ((q & 1) ? 2048 : ((q >> 1) & 1) * 1024) : supw + (q % ST) * 1024;
        if (nx)
            gvm_issue<S16>(ring + (q % ST) * kGvmStage, sup, np, ns, na, nxt.pofs, nxt.sofs, nxt.aofs, nxt.asofs,
                           nxt.mc, lane, s, nt);
        else
            gvm_issue<S16>(ring + (q % ST) * kGvmStage, sup, cp, cs, ca, cur.pofs, cur.sofs, cur.aofs, cur.asofs,
                           cur.mc, lane, s, nt);
    };

    // One continuous stream of stages over this wave's items: the last
    // ST - 1 iterations of an item issue the next item's first stages (or,
    // past the last item, repeats of the current one's last stage, never
    // read), so an item starts with its data in flight.
    // (the descriptors are built here, not in the lambdas: a buffer
    // descriptor formed inside a lambda keeps the host pass from emitting
    // the kernel)
    int item_c = 0, item_n = 0, n_done = 0;
    GVM_TS(0);
    cur = make(int(blockIdx.x) * kGvmWaves + wave, item_c);
    if (cur.mc <= 0) return;
    nxt = make(item_c + wstride, item_n);
    cp = gvm_rsrc(cur.pb, rows_per_expert * lrow);
    cs = gvm_rsrc(cur.sbp, rows_per_expert * srb);
    ca = gvm_rsrc(cur.ab, 0x7FFFFFFF);
    np = gvm_rsrc(nxt.pb, rows_per_expert * lrow);
    ns = gvm_rsrc(nxt.sbp, rows_per_expert * srb);
    na = gvm_rsrc(nxt.ab, 0x7FFFFFFF);
    int q = 0;                                               // stages consumed by this wave
#pragma unroll
    for (int u = 0; u < ST - 1; ++u) issue(false, min(u, S - 1), u);
    while (true) {
        f32x4 acc[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int mcol = col < cur.mc ? col : 0;
        // byte offset of each of this lane's rows' scales from its 4-byte-aligned start
        int soff[NRB];
#pragma unroll
        for (int rb = 0; rb < NRB; ++rb) {
            const int r = 16 * rb + col;
            const int wr = GU ? (r >= PW ? N : 0) + min(cur.i0 + (r & (PW - 1)), N - 1) : min(cur.i0 + r, N - 1);
            soff[rb] = wr * srb;
        }
        // B operand of MFMA step t of a stage: limb L's bytes at
        // [m][L][256]: K 128 t + 32 (g >> 1) + 16 (g & 1), and + 64
        const uint32_t boff = uint32_t(mcol * kGvmLimbs * kGvmKS + 32 * (grp >> 1) + 16 * (grp & 1));

#pragma unroll 1
        for (int s = 0; s < S; ++s, ++q) {
            // stage s + ST - 1 in, then stage s complete: NT (ST - 1) younger loads
            const int ahead = s + ST - 1;
            if (ahead < S) issue(false, ahead, q + ST - 1);
            else if (nxt.mc > 0) issue(true, ahead - S, q + ST - 1);
            else issue(false, S - 1, q + ST - 1);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(WAIT) : "memory");
            if (q == 0) GVM_TS(1);
            const uint32_t stb = ring_base + uint32_t(q % ST) * kGvmStage;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                u32x4 bq[kGvmLimbs][2];
                uint32_t sb, sa[NRB];
                u32x4 aq[NRB];
#pragma unroll
                for (int L = 0; L < kGvmLimbs; ++L) {
                    const uint32_t pb = stb + kGvmOA + boff + L * kGvmKS + t * 128;
                    asm volatile("ds_read_b128 %0, %1" : "=v"(bq[L][0]) : "v"(pb));
                    asm volatile("ds_read_b128 %0, %1" : "=v"(bq[L][1]) : "v"(pb + 64));
                }
                asm volatile("ds_read_u8 %0, %1" : "=v"(sb) : "v"(stb + kGvmOAS + mcol * 8 + 4 * t + grp));
#pragma unroll
                for (int rb = 0; rb < NRB; ++rb) {
                    const int r = 16 * rb + col;
                    const int pc = 4 * t + grp;                      // 16-byte piece of the row's 128
                    asm volatile("ds_read_b128 %0, %1"
                                 : "=v"(aq[rb]) : "v"(stb + r * 128 + ((pc ^ ((r >> 1) & 7)) << 4)));
                    const uint32_t sadr = S16 ? sup_base + uint32_t(((q >> 1) & 1) * 1024 + r * 16 + (s & 1) * 8 + pc)
                                              : sup_base + uint32_t((q % ST) * 1024 + r * 16 + (soff[rb] & 3) + pc);
                    asm volatile("ds_read_u8 %0, %1" : "=v"(sa[rb]) : "v"(sadr));
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int L = 0; L < kGvmLimbs; ++L) asm volatile("" : "+v"(bq[L][0]), "+v"(bq[L][1]));
                asm volatile("" : "+v"(sb));
#pragma unroll
                for (int rb = 0; rb < NRB; ++rb) asm volatile("" : "+v"(aq[rb]), "+v"(sa[rb]));
                if (Kp != Kd && s == S - 1) {
                    // blocks past K (the codes of the next row, or zero past
                    // the buffer; the activations there are zero): zero
                    // codes under scale 1, so that no scale byte read there
                    // can turn the zero products into NaN
                    if ((8 * s + 4 * t + grp) * 32 >= Kd) {
#pragma unroll
                        for (int rb = 0; rb < NRB; ++rb) {
                            aq[rb] = u32x4{0u, 0u, 0u, 0u};
                            sa[rb] = 127u;
                        }
                    }
                }
                // limbs outer: consecutive MFMAs update different accumulators
#pragma unroll
                for (int L = 0; L < kGvmLimbs; ++L) {
                    const i32x8 B{int(bq[L][0].x), int(bq[L][0].y), int(bq[L][0].z), int(bq[L][0].w),
                                  int(bq[L][1].x), int(bq[L][1].y), int(bq[L][1].z), int(bq[L][1].w)};
#pragma unroll
                    for (int rb = 0; rb < NRB; ++rb) {
                        const i32x8 A{int(aq[rb].x), int(aq[rb].y), int(aq[rb].z), int(aq[rb].w), 0, 0, 0, 0};
                        acc[rb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, B, acc[rb], 4, 0, 0,
                                                                                  int(sa[rb]), 0, int(sb));
                    }
                }
            }
        }

        // D: column col = group row, weight rows 4 grp + [0, 4) of each block
        if constexpr (GU) {
            if (a.hf && cur.i0 < N) {
                // h straight into the down's limb format: the wave's 32 pairs
                // are one 32-element block b of each group row, 8 values per
                // lane (positions 4 grp + [0, 4) and 16 + 4 grp + [0, 4)), the
                // column's 4 lanes at lanes col + 16 grp.  Same arithmetic as
                // gvm_format_block.  (N % 32 == 0: the block is whole.)
                float hv[8];
                float mx = 0.0f;
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        hv[4 * rb + qq] = fast_silu(acc[rb][qq]) * acc[NRB / 2 + rb][qq];
                        mx = fmaxf(mx, fabsf(hv[4 * rb + qq]));
                    }
                mx = fmaxf(mx, __shfl_xor(mx, 16));
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                if (col < cur.mc) {
                    const int hkp = gvm_kpad(N), b = cur.i0 / 32;
                    uint8_t* dst = (cur.sh ? a.hf_sh : a.hf) + int64_t(cur.r0 + col) * gvm_row_bytes(N);
                    float inv;
                    const int s = gvm_block_scale(mx, inv);
                    uint32_t q0[kGvmLimbs], q1[kGvmLimbs];
                    gvm_limbs4(hv, inv, q0);
                    gvm_limbs4(hv + 4, inv, q1);
#pragma unroll
                    for (int L = 0; L < kGvmLimbs; ++L) {
                        uint32_t* d = reinterpret_cast<uint32_t*>(dst + int64_t(L) * hkp + b * 32) + grp;
                        d[0] = q0[L];
                        d[4] = q1[L];
                    }
                    if (grp == 0) dst[3 * hkp + b] = uint8_t(s + 127);
                    if (cur.i0 + 32 == N) {
                        // the last block also writes the pad blocks: zero
                        // limbs, scale byte 0 (a zero block's)
                        for (int pb = N / 32; pb < hkp / 32; ++pb) {
#pragma unroll
                            for (int L = 0; L < kGvmLimbs; ++L)
                                *reinterpret_cast<uint2*>(dst + int64_t(L) * hkp + pb * 32 + 8 * grp) =
                                    make_uint2(0u, 0u);
                            if (grp == 0) dst[3 * hkp + pb] = 0;
                        }
                    }
                }
            }
        }
        if (col < cur.mc && !(GU && a.hf)) {
            const int64_t orow = int64_t(cur.r0 + col) * N;
            if constexpr (GU) {
                float* h = cur.sh ? a.h_sh : a.h;
#pragma unroll
                for (int rb = 0; rb < NRB / 2; ++rb) {
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        const int i = cur.i0 + 16 * rb + 4 * grp + qq;
                        if (i < N) h[orow + i] = fast_silu(acc[rb][qq]) * acc[NRB / 2 + rb][qq];
                    }
                }
            } else {
                float* y = cur.sh ? a.y_sh : a.y;
#pragma unroll
                for (int rb = 0; rb < NRB; ++rb) {
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) {
                        const int i = cur.i0 + 16 * rb + 4 * grp + qq;
                        if (i < N) y[orow + i] = acc[rb][qq];
                    }
                }
            }
        }
        if (n_done < 13) GVM_TS(2 + n_done);
        ++n_done;
        if (nxt.mc <= 0) break;
        cur = nxt;
        cp = np;
        cs = ns;
        ca = na;
        nxt = make(item_n + wstride, item_n);
        np = gvm_rsrc(nxt.pb, rows_per_expert * lrow);
        ns = gvm_rsrc(nxt.sbp, rows_per_expert * srb);
        na = gvm_rsrc(nxt.ab, 0x7FFFFFFF);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the repeats past the last item
    GVM_TS(15);
    (void)n_done;
}

// K a multiple of 64 (2-byte aligned scale rows) with at least ST - 1
// stages per item (the stream's look-ahead reaches at most into the next
// item).
int gvm_padded_k(int K) { return gvm_kpad(K); }

bool gvm_shape_ok(int H, int I) {
    const int kmin = (kGvmStages - 1) * kGvmKS;
    return H % 64 == 0 && I % 64 == 0 && gvm_kpad(H) >= kmin && gvm_kpad(I) >= kmin;
}

hipError_t gvm_launch(hipStream_t st, const GvArgs& a, bool gate_up) {
    if (a.K % 64 || gvm_kpad(a.K) < (kGvmStages - 1) * kGvmKS) return hipErrorInvalidValue;
    if (gate_up && a.hf && a.N % 32) return hipErrorInvalidValue;   // whole h blocks
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return hipErrorInvalidConfiguration;
    }
    const size_t lds = size_t(kGvmWaves) * kGvmStages * kGvmStage + kGvmWaves * 3 * 1024;
    const dim3 grid(cus), blk(kGvmWaves * kWave);
    if (a.K % 512 == 0) {
        if (gate_up) hipLaunchKernelGGL((gvm_kernel<true, true>), grid, blk, lds, st, a);
        else hipLaunchKernelGGL((gvm_kernel<false, true>), grid, blk, lds, st, a);
    } else {
        if (gate_up) hipLaunchKernelGGL((gvm_kernel<true, false>), grid, blk, lds, st, a);
        else hipLaunchKernelGGL((gvm_kernel<false, false>), grid, blk, lds, st, a);
    }
    return hipGetLastError();
}

}  // namespace grim
