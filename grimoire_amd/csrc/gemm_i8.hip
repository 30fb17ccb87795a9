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
// Tile: 128 rows x 256 columns x 64 K, 512 threads; wave w owns columns
// [64 (w % 4), +64) for rows [64 (w / 4), +64) (2 x 2 MFMA tiles per limb).
// A (limbs) and B (codes) both stream into a 4-stage LDS ring through
// buffer_load ... lds (16 bytes per lane, no registers involved).  A limb
// rows are stored [K/64][2][64] so that one K tile of a row is one 128-byte
// line; every DMA instruction moves whole row segments (A 8 x 128 bytes, B
// 16 x 64 bytes) into XOR-swizzled slots that keep the fragment reads free
// of bank conflicts.  Three K tiles are in flight while one is multiplied,
// and the stream runs on across items: a work-group's next item has its
// first tiles and its scales in LDS before the current one's epilogue,
// which stores straight from the accumulators.  Persistent XCD-aware grid
// over (m-tile, column tile) items, rows from the dispatch's tile table.
//
// Rows mode (the forward's): no tile table; every work-group lists the
// tiles itself from the per-expert row counts.  Experts above `split` rows
// take the 128-row tiles; the rest (the tail of a skewed routing, where a
// 128-row tile would be mostly empty rows and the expert's weights read
// once from memory are the real work) take 32-row x 256-column tiles whose
// stages span 128 K, so every weight DMA lane moves a whole 128-byte line.
// One launch walks the 128-row items, then the narrow ones.
#include "common.hpp"
#include "gemm.hpp"
#include "gemm_i8.hpp"

#include <type_traits>

namespace grim {

// Item timestamps for kernel studies, compiled in only with GRIM_TIMING:
// per work-group b < 256, 128 (time, info) pairs; the 128-row items at
// pairs 0..61 (start, end alternating), the narrow ones at 64..125.
#ifdef GRIM_TIMING
#define GRIM_ITEM_TS(base, ev, info)                                                              \
    do {                                                                                          \
        if (g.ts && threadIdx.x == 0 && blockIdx.x < 256 && (ev) < 62) {                          \
            g.ts[(blockIdx.x * 128 + (base) + (ev)) * 2] = __builtin_amdgcn_s_memrealtime();      \
            g.ts[(blockIdx.x * 128 + (base) + (ev)) * 2 + 1] = (info);                            \
        }                                                                                         \
    } while (0)
#else
#define GRIM_ITEM_TS(base, ev, info) do {} while (0)
#endif

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));

constexpr int QBM = 128, QBN = 256, QBK = 64;
constexpr int kQThreads = 512;
constexpr int kQStages = 4;
constexpr int kQStageBytes = 32768;          // A 16 KiB (2 limbs x 4 x 2 fragments), B 16 KiB
constexpr int kQXcds = 8;
constexpr float kLoScale = 1.0f / 254.0f;
// gather mode: the A offset of a row past an item's count (beyond every
// gather buffer, which the host keeps below it: the load returns zeros)
constexpr int kI8FarOffset = 0x70000000;

typedef __attribute__((address_space(3))) void* lds_ptr_t;


// AUX: the buffer load's cache policy bits (0 everywhere here: the weight
// tiles are read again -- the other half of a line by the next K tile, the
// same lines by an expert's next m-tile -- so they stay cacheable)
template <int AUX>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, voff, soff, 0, AUX);
}

typedef float f32x4v __attribute__((ext_vector_type(4)));

// LDS reads the compiler does not see as such (no wait is inserted for
// them; the caller waits on lgkmcnt itself)
__device__ __forceinline__ float lds_f32(int addr) {
    float v;
    asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}
__device__ __forceinline__ f32x4v lds_f32x4(int addr) {
    f32x4v v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}

// Lane index from mbcnt: formed where it is needed, so no register holds
// it (and no spill reload, with its wait on every outstanding load) across
// the item loop.
// The value is opaque to the optimiser, so what is derived from it is
// formed at each call and not hoisted out of the loops.
__device__ __forceinline__ int lane_id() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// Scalar load of one int (lgkmcnt, not vmcnt: it does not wait on the
// vector loads and stores in flight); p must be wave-uniform.
__device__ __forceinline__ int sload_i32(const int32_t* p) {
    int v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
    return v;
}

__device__ __forceinline__ int lds_i32(int addr) {
    int v;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
    return v;
}

// Rows mode: the tile list of a kernel from the per-expert row counts.
// Expert e takes ceil(count / BM) tiles when lo < count <= hi; tp[e] is
// the inclusive prefix of those tile counts (tile ty belongs to the first
// e with tp[e] > ty).  All threads of the work-group call it, before any
// LDS-DMA is in flight; tmp holds 2 KiB.  Returns the list's length.
template <int BM, int NT>
__device__ int i8_list_scan(const int32_t* __restrict__ counts, int E, int lo, int hi, int32_t* tp,
                            int32_t* tmp) {
    constexpr int PER = kI8MaxListExperts / NT;   // experts per thread
    const int t = threadIdx.x;
    int v[PER], sum = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = PER * t + j;
        const int c = e < E ? counts[e] : 0;
        v[j] = (c > lo && c <= hi) ? (c + BM - 1) / BM : 0;
        sum += v[j];
    }
    tmp[t] = sum;
    __syncthreads();
    for (int off = 1; off < NT; off <<= 1) {
        const int a = t >= off ? tmp[t - off] : 0;
        __syncthreads();
        tmp[t] += a;
        __syncthreads();
    }
    int run = tmp[t] - sum;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        run += v[j];
        if (PER * t + j < E) tp[PER * t + j] = run;
    }
    const int total = tmp[NT - 1];
    __syncthreads();
    return total;
}

// The expert of list tile ty (wave-uniform, ty < the list's length) and
// the end of its tiles, tend = tp[e]: two ballots over 16-expert blocks.
__device__ __forceinline__ int i8_list_find(int tp_addr, int E, int ty, int& tend) {
    const int ln = lane_id();
    const int i0 = min(E - 1, 16 * ln + 15);
    const uint64_t b0 = __ballot(lds_i32(tp_addr + 4 * i0) > ty);
    const int f = __builtin_amdgcn_readfirstlane(int(__builtin_ctzll(b0)));
    const int i1 = min(E - 1, 16 * f + (ln & 15));
    const int v1 = lds_i32(tp_addr + 4 * i1);
    const uint64_t b1 = __ballot(v1 > ty) & 0xFFFFull;
    const int j = __builtin_amdgcn_readfirstlane(int(__builtin_ctzll(b1)));
    tend = __builtin_amdgcn_readlane(v1, j);
    return 16 * f + j;
}

struct I8Src {
    const uint8_t* w;
    const float* ws;
    int64_t row_bytes;
    const int8_t* A;
    const float* sa;
    float* out;
};

// One (m-tile, column tile) work item, wave-uniform: its first A row, row
// count, first weight row and first output column (h column for SwiGLU).
// The buffer resources built from it bound everything: rows past the
// expert's count and columns past the slab read as zero, and stores past
// them are dropped by the hardware.
struct I8Item {
    int64_t arow0, wrow;   // wrow: first weight row of the tile (expert base + col0)
    int rows, col0;
    int sh;                // 1: a shared-expert item (its own A rows, weights, output)
};

// Item (list tile ty, column tile nt) of a kernel with BM x BN tiles.  The
// routed tiles come from the dispatch's table, or in rows mode (tp_addr >=
// 0) from the kernel's own list; tiles past n_routed are the shared
// expert's.
template <bool SWIGLU, int BM, int BN>
__device__ __forceinline__ I8Item i8_item(const GemmI8Args& g, int n_routed, int ty, int nt,
                                          int tp_addr) {
    int rows_valid;
    int64_t arow0, wrow0;
    ty = __builtin_amdgcn_readfirstlane(ty);
    const bool routed = ty < n_routed;
    if (!routed) ty -= n_routed;
    if (routed && tp_addr >= 0) {
        int tend;
        const int e = i8_list_find(tp_addr, g.num_experts, ty, tend);
        const int c = sload_i32(g.counts + e);
        const int mb = ty - (tend - (c + BM - 1) / BM);
        rows_valid = min(BM, c - mb * BM);
        arow0 = int64_t(sload_i32(g.offsets + e)) + int64_t(mb) * BM;
        wrow0 = int64_t(e) * g.N;
    } else if (routed) {
        const int e = sload_i32(g.tile_e + ty);
        const int ec = e < 0 ? 0 : e;
        const int mb = sload_i32(g.tile_mb + ty);
        rows_valid = e < 0 ? 0 : min(BM, sload_i32(g.counts + ec) - mb * BM);
        arow0 = int64_t(sload_i32(g.offsets + ec)) + int64_t(mb) * BM;
        wrow0 = int64_t(ec) * g.N;
    } else {
        rows_valid = min(BM, g.T_sh - ty * BM);
        arow0 = int64_t(ty) * BM;
        wrow0 = 0;
    }
    I8Item it;
    it.sh = routed ? 0 : 1;
    it.col0 = nt * (SWIGLU ? BN / 2 : BN);
    it.rows = max(0, __builtin_amdgcn_readfirstlane(rows_valid));
    it.arow0 = int64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(arow0)))) |
               (int64_t(__builtin_amdgcn_readfirstlane(int(arow0 >> 32))) << 32);
    const int64_t wr = wrow0 + it.col0;
    it.wrow = int64_t(uint32_t(__builtin_amdgcn_readfirstlane(int(wr)))) |
              (int64_t(__builtin_amdgcn_readfirstlane(int(wr >> 32))) << 32);
    return it;
}

// The share of an XCD's list of n items that a run walks: part 0 all of
// it, part 1 the first half, part 2 the second half.
__device__ __forceinline__ int i8_part_begin(int n, int part) { return part == 2 ? n / 2 : 0; }
__device__ __forceinline__ int i8_part_end(int n, int part) { return part == 1 ? n / 2 : n; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t i8_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

// Persistent XCD-aware walk over (m-tile, column tile) items with one
// continuous stream of K tiles through the 4-stage LDS ring: the last three
// iterations of an item request the next item's first three tiles (and,
// ahead of them, its row and column scales), so an item starts with its
// data already in LDS, and the epilogue stores straight from the
// accumulators (no LDS, no barrier) while those tiles land.
//
// Iteration t of an item: tile t complete -- this wave's loads and stores
// complete in issue order, so waiting until at most Y operations younger
// than tile t's last load are outstanding suffices (Y = 16: the two tiles
// requested after it; plus the previous item's epilogue stores for t < 3;
// capped at 63, the counter's limit); the barrier then covers every
// wave's loads and retires every wave's reads of tile t - 1, whose stage
// takes stream tile t + 3.  Tile t's 20 fragments are read at once, and its
// 32 MFMAs run with the 8 DMA instructions for tile t + 3 interleaved, one
// per 4 MFMAs (issued together, the 4 waves' 32 instructions would queue
// at the texture unit, 16 cycles each, and hold the MFMAs back).  Past the
// last item the stream requests tiles from an empty buffer (num_records 0:
// no memory traffic), which keeps every iteration alike.
// The body of the 128-row kernel for one work-group: it takes the items
// slot, slot + per_xcd, ... of its XCD's range; n_routed routed tiles (from
// the table, or from the list at tp_addr >= 0) then, for parts & 2, the
// shared expert's.  smem / meta: the kernel's LDS.  Returns where the
// work-group's sequence continues past the last item (its first index in
// a list that follows).
template <bool SWIGLU>
__device__ __forceinline__ int i8_big_run(const GemmI8Args& g, int n_col_tiles, int parts,
                                           int n_routed, int tp_addr, int part, int slot, int per_xcd,
                                           uint8_t (*smem)[kQStageBytes], float (*meta)[512],
                                           int32_t (*rmap)[256]) {
    // 8 waves, two per SIMD: wave w owns tile columns [64 (w % 4), +64) for
    // rows [64 (w / 4), +64)
    constexpr int MIW = 2;                   // 32-row MFMA tiles per wave
    constexpr int NJ = 2;                    // DMA instructions per wave per K tile, for A and for B
    // meta, per item parity: row scales [128] at 0, column scales at 1024
    // (plain: [256]; SwiGLU: gate [128] then up [128]).
    // parts: 1 = routed m-tiles, 2 = the shared expert's, 3 = both in one
    // list (routed first; the host fuses them only when the two weight sets
    // share a row length, which the per-lane weight offsets assume)
    const I8Src src_r{g.w, g.ws, g.row_bytes, g.A, g.sa, g.out};
    const I8Src src_s{g.w_sh, g.ws_sh, g.row_bytes_sh, g.A_sh, g.sa_sh, g.out_sh};
    const int64_t wrb = parts == 2 ? g.row_bytes_sh : g.row_bytes;
    const int total = n_routed + ((parts & 2) ? (g.T_sh + QBM - 1) / QBM : 0);
    // work-group b runs on XCD b % 8: each XCD walks a contiguous range of
    // the m-tile list, column tiles fastest, so an expert's weights and an
    // A row block stay under one L2
    const int xcd = blockIdx.x % kQXcds;
    const int lo = int(int64_t(total) * xcd / kQXcds), hi = int(int64_t(total) * (xcd + 1) / kQXcds);
    const int items = i8_part_end((hi - lo) * n_col_tiles, part);
    int i = i8_part_begin((hi - lo) * n_col_tiles, part) + slot;
    if (i >= items) return i - items;

    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
    const int wn = wave & 3, wm = wave >> 2;
    const int K = g.K;
    const int a_row_bytes = 2 * K;

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
    // Per-lane offsets, formed from an opaque copy of the lane index: once
    // here and again at every item's start, so that they are not kept live
    // (and spilled) across the epilogue, whose reloads would make the
    // compiler wait for every outstanding load before each fragment read.
    int a_off[NJ], a_offn[NJ], b_off[NJ], fa_off[2][2][MIW], fb_off[2][2];
#define GRIM_I8_OFFSETS()                                                                         \
    do {                                                                                          \
        const int ln = lane_id();                                                                 \
        _Pragma("unroll") for (int j = 0; j < NJ; ++j) {                                          \
            const int ja = NJ * wave + j;                                                         \
            const int col = 16 * ja + (ln >> 2), pcb = ln & 3;                                    \
            const int nsub = col >> 5, x = col & 31;                                              \
            /* SwiGLU: h columns [32 w', +32) of wave w' = nsub / 2: gate rows */                 \
            /* for nsub even, up rows for nsub odd; otherwise the tile's columns */               \
            const int row = SWIGLU ? ((nsub & 1) ? g.I : 0) + (nsub >> 1) * 32 + x : col;         \
            b_off[j] = row * int(wrb) + ((pcb ^ ((col >> 2) & 3)) << 4);                          \
        }                                                                                         \
        /* fragment read addresses inside a stage */                                              \
        _Pragma("unroll") for (int ks = 0; ks < 2; ++ks) {                                        \
            const int ch = 2 * ks + (ln >> 5);                                                    \
            _Pragma("unroll") for (int l = 0; l < 2; ++l)                                         \
                _Pragma("unroll") for (int mi = 0; mi < MIW; ++mi) {                              \
                    const int r = (wm * MIW + mi) * 32 + (ln & 31);                               \
                    fa_off[ks][l][mi] = r * 128 + (((4 * l + ch) ^ ((r >> 1) & 7)) << 4);         \
                }                                                                                 \
            _Pragma("unroll") for (int ni = 0; ni < 2; ++ni) {                                    \
                const int n = (2 * wn + ni) * 32 + (ln & 31);                                     \
                fb_off[ks][ni] = 16384 + n * 64 + ((ch ^ ((n >> 2) & 3)) << 4);                   \
            }                                                                                     \
        }                                                                                         \
    } while (0)
    GRIM_I8_OFFSETS();
    // A rows: lane (j, ln) moves tile row 8 (NJ wave + j) + ln / 8, chunk
    // ln % 8.  Contiguous items read row r of their base; gather-mode
    // routed items read the row the map names (from the map's LDS copy at
    // rm_addr), and rows past the item's count an address past the buffer
    // (zeros).
    const bool gat = g.gather != nullptr;
    const int rmap_base = int(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int32_t*)(&rmap[0][0])));
    auto a_offsets = [&](const I8Item& it, int rm_addr, int (&o)[NJ]) {
        const int ln = lane_id();
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int r = 8 * (NJ * wave + j) + (ln >> 3), pc = ln & 7;
            const int sw = (pc ^ ((r >> 1) & 7)) << 4;
            if (gat && !it.sh) {
                const int src = lds_i32(rm_addr + 4 * r);
                o[j] = r < it.rows ? src * a_row_bytes + sw : kI8FarOffset;
            } else {
                o[j] = r * a_row_bytes + sw;
            }
        }
    };

    auto tile_of = [&](int ii) { return lo + ii / n_col_tiles; };
    auto col_of = [&](int ii) { return ii % n_col_tiles; };
    const int n_slab = SWIGLU ? 2 * g.I : g.N;
    const int ldo = SWIGLU ? g.I : g.N;
    // weight rows from the tile's first one; for SwiGLU the up rows follow
    // I rows later (gate rows past I read up rows: their columns are never
    // stored).  rows == 0 (past the last item) gives empty buffers.
    auto rsrc_a = [&](const I8Item& it) {
        if (gat && !it.sh) return i8_rsrc(src_r.A, it.rows > 0 ? g.gather_rows * a_row_bytes : 0);
        const int8_t* A = it.sh ? src_s.A : src_r.A;
        return i8_rsrc(A + it.arow0 * a_row_bytes, it.rows * a_row_bytes);
    };
    auto rsrc_b = [&](const I8Item& it) {
        const uint8_t* w = it.sh ? src_s.w : src_r.w;
        return i8_rsrc(w + it.wrow * wrb, it.rows > 0 ? int((n_slab - it.col0) * wrb) : 0);
    };
    // scale requests: wave 0 the 128 row scales (lanes 32..63 past the end
    // read zero into padding), wave 1 the 256 column scales; in gather mode
    // wave 2 the item's row map
    auto request_meta = [&](const I8Item& it, int par) {
        const int ln = lane_id();
        if (wave == 0) {
            dma16<0>(i8_rsrc((it.sh ? src_s.sa : src_r.sa) + it.arow0, it.rows * 4),
                     reinterpret_cast<uint8_t*>(&meta[par][0]),
                     ln * 16, 0);
        } else if (wave == 2 && gat) {
            dma16<0>(i8_rsrc(g.gather + it.arow0, it.sh ? 0 : it.rows * 4),
                     reinterpret_cast<uint8_t*>(&rmap[par][0]), ln * 16, 0);
        } else if (wave == 1) {
            const int m_off = (SWIGLU && ln >= 32) ? g.I * 4 + (ln - 32) * 16 : ln * 16;
            dma16<0>(i8_rsrc((it.sh ? src_s.ws : src_r.ws) + it.wrow, it.rows > 0 ? (n_slab - it.col0) * 4 : 0),
                     reinterpret_cast<uint8_t*>(&meta[par][256]), m_off, 0);
        }
    };
    auto request = [&](const I8Item& it, int stage, int t) {
        uint8_t* st = smem[stage];
        const __amdgpu_buffer_rsrc_t ra = rsrc_a(it), rb = rsrc_b(it);
#pragma unroll
        for (int j = 0; j < NJ; ++j) dma16<0>(ra, st + (NJ * wave + j) * 1024, a_off[j], t * 128);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            dma16<0>(rb, st + 16384 + (NJ * wave + j) * 1024, b_off[j], t * QBK);
    };

    const int nk = K / QBK;   // >= 3 (gather mode: >= 6)
    I8Item cur = i8_item<SWIGLU, QBM, QBN>(g, n_routed, tile_of(i), col_of(i), tp_addr);
    I8Item none;
    none.arow0 = 0; none.wrow = 0; none.rows = 0; none.col0 = 0; none.sh = 0;
    request_meta(cur, 0);
    if (gat) {
        // the first item's map, before its first tiles
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    a_offsets(cur, rmap_base, a_off);
#pragma unroll
    for (int p = 0; p < kQStages - 1; ++p) request(cur, p, p);

    // LDS byte address of the ring (a C-style cast is the address-space cast)
    const int smem_base = int(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)(&smem[0][0])));
    const int meta_base = int(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) float*)(&meta[0][0])));
    int gs = 0, par = 0;
    bool first = true;
    i32x16 acc[2][MIW][2];
    i32x4 fb[2][2], fa[2][2][MIW];
    int nev = 0;
    (void)nev;
    for (; i < items; i += per_xcd) {
        GRIM_ITEM_TS(0, 2 * nev, (unsigned long long)(cur.rows) | ((unsigned long long)cur.sh << 16));
        GRIM_I8_OFFSETS();
        a_offsets(cur, rmap_base + par * 1024, a_off);
#pragma unroll
        for (int j = 0; j < NJ; ++j) a_offn[j] = a_off[j];
        const bool more = i + per_xcd < items;
        const I8Item nxt = more ? i8_item<SWIGLU, QBM, QBN>(g, n_routed, tile_of(i + per_xcd), col_of(i + per_xcd), tp_addr)
                                : none;
#pragma unroll
        for (int l = 0; l < 2; ++l)
#pragma unroll
            for (int mi = 0; mi < MIW; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[l][mi][ni][v] = 0;
        // The wait before tile t: the operations younger than tile t's last
        // load are the two later tiles' loads (YT), and right after an
        // epilogue (t < 3) also its stores (ES per lane); waiting until at
        // most min(63, that many) are outstanding (63: the counter's limit)
        // completes tile t.  One asm block, so that the loop body is not
        // duplicated per case.
        constexpr int YT = 4 * NJ;
        constexpr int ES = (SWIGLU ? 1 : 2) * MIW * 16;
        constexpr int YE = YT + ES < 63 ? YT + ES : 63;
#define GRIM_I8_WAIT(after_epi)                                                                   \
        asm volatile("s_cmp_eq_u32 %0, 0\n\t"                                                    \
                     "s_cbranch_scc1 .Lgrim_w16_%=\n\t"                                           \
                     "s_waitcnt vmcnt(%2)\n\t"                                                   \
                     "s_branch .Lgrim_wdone_%=\n"                                                 \
                     ".Lgrim_w16_%=:\n\t"                                                        \
                     "s_waitcnt vmcnt(%1)\n"                                                      \
                     ".Lgrim_wdone_%=:\n\t"                                                      \
                     "s_waitcnt lgkmcnt(0)\n\t"                                                  \
                     "s_barrier" ::"s"(__builtin_amdgcn_readfirstlane(after_epi)), "n"(YT), "n"(YE) \
                     : "memory", "scc")
        // Fragment reads are inline asm with explicit lgkmcnt waits tied to
        // the fragment registers: the compiler cannot tell that they and the
        // in-flight DMA writes touch different ring stages, and guards a
        // compiler-visible LDS read with a wait for every outstanding load.
        // Reads in MFMA order (ks, mi; B then the two limbs): 12 outstanding
        // (lgkmcnt holds 15).
#define GRIM_I8_DSR(dst, addr)                                                                    \
        asm volatile("ds_read_b128 %0, %1" : "=v"(dst) : "v"(addr))
#define GRIM_I8_LGKM(n, ks_, mi_)                                                                 \
        asm volatile("s_waitcnt lgkmcnt(" #n ")"                                                   \
                     : "+v"(fb[ks_][0]), "+v"(fb[ks_][1]), "+v"(fa[ks_][0][mi_]), "+v"(fa[ks_][1][mi_]))
#define GRIM_I8_MMA_MI(ks_, mi_)                                                                  \
        _Pragma("unroll") for (int ni = 0; ni < 2; ++ni)                                          \
            _Pragma("unroll") for (int l = 0; l < 2; ++l)                                         \
                acc[l][mi_][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[ks_][l][mi_], fb[ks_][ni], \
                                                                        acc[l][mi_][ni], 0, 0, 0)
#define GRIM_I8_READS(ks_)                                                                        \
        do {                                                                                      \
            GRIM_I8_DSR(fb[ks_][0], sb + fb_off[ks_][0]);                                         \
            GRIM_I8_DSR(fb[ks_][1], sb + fb_off[ks_][1]);                                         \
            _Pragma("unroll") for (int mi = 0; mi < MIW; ++mi) {                                  \
                GRIM_I8_DSR(fa[ks_][0][mi], sb + fa_off[ks_][0][mi]);                             \
                GRIM_I8_DSR(fa[ks_][1][mi], sb + fa_off[ks_][1][mi]);                             \
            }                                                                                     \
        } while (0)
#define GRIM_I8_DMA(q)                                                                            \
        do {                                                                                      \
            if ((q) < NJ) dma16<0>(qa, nx + (NJ * wave + (q)) * 1024, own ? a_off[(q) % NJ] : a_offn[(q) % NJ], tu * 128); \
            else dma16<0>(qb, nx + 16384 + (NJ * wave + (q) - NJ) * 1024, b_off[(q) % NJ], tu * QBK); \
        } while (0)
#define GRIM_I8_ITER(t_, META)                                                                    \
        do {                                                                                      \
            const int t = (t_);                                                                   \
            GRIM_I8_WAIT((t < 3 && !first) ? 1 : 0);                                              \
            /* the next item's row map (requested at t = 0, landed by t = 3) */                   \
            if (gat && t == nk - (kQStages - 1)) a_offsets(nxt, rmap_base + (par ^ 1) * 1024, a_offn); \
            const int sb = ((gs + t) & 3) * kQStageBytes + smem_base;                             \
            GRIM_I8_READS(0);                                                                     \
            if (META) request_meta(nxt, par ^ 1);                                                 \
            /* stream tile t + 3: this item's, or the next item's 0, 1, 2 */                      \
            const int u = t + kQStages - 1;                                                       \
            const bool own = u < nk;                                                              \
            const __amdgpu_buffer_rsrc_t qa = rsrc_a(own ? cur : nxt);                            \
            const __amdgpu_buffer_rsrc_t qb = rsrc_b(own ? cur : nxt);                            \
            const int tu = own ? u : u - nk;                                                      \
            uint8_t* nx = smem[(gs + u) & 3];                                                     \
            /* K half 0's 6 reads in flight: (0, 0) needs the first 4; K half 1's 6 */          \
            /* are issued behind (0, 0)'s products, so the LDS serves them while the */          \
            /* matrix core works: (0, 1) needs 6 of the 8 then in flight, (1, 0) 4 of */          \
            /* the last 6 */                                                                      \
            GRIM_I8_LGKM(2, 0, 0); GRIM_I8_MMA_MI(0, 0); GRIM_I8_DMA(0);                          \
            __builtin_amdgcn_sched_barrier(0);                                                    \
            GRIM_I8_READS(1);                                                                     \
            GRIM_I8_LGKM(6, 0, 1); GRIM_I8_MMA_MI(0, 1); GRIM_I8_DMA(1);                          \
            GRIM_I8_LGKM(2, 1, 0); GRIM_I8_MMA_MI(1, 0); GRIM_I8_DMA(2);                          \
            GRIM_I8_LGKM(0, 1, 1); GRIM_I8_MMA_MI(1, 1); GRIM_I8_DMA(3);                          \
        } while (0)
        // iteration 0 also requests the next item's scales: after its
        // barrier (every wave is past the epilogue that read that parity)
        // and before any of the next item's tiles
        GRIM_I8_ITER(0, true);
        for (int t1 = 1; t1 < nk; ++t1) GRIM_I8_ITER(t1, false);
#undef GRIM_I8_ITER
#undef GRIM_I8_WAIT
#undef GRIM_I8_DSR
#undef GRIM_I8_LGKM
#undef GRIM_I8_MMA_MI
#undef GRIM_I8_DMA
#undef GRIM_I8_READS

        // ---- epilogue.  acc[l][mi][ni][v] is row 32 mi + 8 (v/4) + 4 (l/32)
        // + v%4, column 32 (2 w + ni) + l%32 of the tile.  Scales from LDS
        // (landed with tile 0, behind this item's barriers); each store
        // writes two 128-byte row segments.
        const __amdgpu_buffer_rsrc_t ro =
            i8_rsrc((cur.sh ? src_s.out : src_r.out) + cur.arow0 * ldo, cur.rows * ldo * 4);
        // the scales are read by inline asm too (a compiler-visible LDS read
        // here would wait for the next item's tiles already in flight)
        const int mb = meta_base + par * 2048;
        const int ln = lane_id();
        const int hrow = 4 * (ln >> 5);
        const int row0 = wm * MIW * 32;       // this wave's first tile row
        if constexpr (SWIGLU) {
            const int hcl = wn * 32 + (ln & 31);
            float sg = lds_f32(mb + 1024 + hcl * 4), su = lds_f32(mb + 1024 + (128 + hcl) * 4);
            // per-lane byte offset of (row row0 + hrow, this column), opaque so
            // the row offsets below are formed here and not kept live
            int base = cur.col0 + hcl < g.I ? ((row0 + hrow) * g.I + cur.col0 + hcl) * 4 : 0x40000000;
            asm volatile("" : "+v"(base));
#pragma unroll
            for (int mi = 0; mi < MIW; ++mi) {
                f32x4v s4[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) s4[q] = lds_f32x4(mb + (row0 + mi * 32 + 8 * q + hrow) * 4);
                asm volatile("s_waitcnt lgkmcnt(0)"
                             : "+v"(s4[0]), "+v"(s4[1]), "+v"(s4[2]), "+v"(s4[3]), "+v"(sg), "+v"(su));
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int v = 4 * q + j;
                        const float gv = s4[q][j] * sg * __builtin_fmaf(float(acc[1][mi][0][v]), kLoScale, float(acc[0][mi][0][v]));
                        const float uv = s4[q][j] * su * __builtin_fmaf(float(acc[1][mi][1][v]), kLoScale, float(acc[0][mi][1][v]));
                        const int off = base + (mi * 32 + 8 * q + j) * g.I * 4;
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, fast_silu(gv) * uv),
                                                              ro, off, 0, 0);
                    }
            }
        } else {
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const int cl = wn * 64 + ni * 32 + (ln & 31);
                float sc = lds_f32(mb + 1024 + cl * 4);
                int base = cur.col0 + cl < g.N ? ((row0 + hrow) * g.N + cur.col0 + cl) * 4 : 0x40000000;
                asm volatile("" : "+v"(base));
#pragma unroll
                for (int mi = 0; mi < MIW; ++mi) {
                    f32x4v s4[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) s4[q] = lds_f32x4(mb + (row0 + mi * 32 + 8 * q + hrow) * 4);
                    asm volatile("s_waitcnt lgkmcnt(0)"
                                 : "+v"(s4[0]), "+v"(s4[1]), "+v"(s4[2]), "+v"(s4[3]), "+v"(sc));
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int v = 4 * q + j;
                            const float y = s4[q][j] * sc * __builtin_fmaf(float(acc[1][mi][ni][v]), kLoScale, float(acc[0][mi][ni][v]));
                            const int off = base + (mi * 32 + 8 * q + j) * g.N * 4;
                            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), ro, off, 0, 0);
                        }
                }
            }
        }
        GRIM_ITEM_TS(0, 2 * nev + 1, 0ull);
        ++nev;
        gs += nk;
        par ^= 1;
        cur = nxt;
        first = false;
    }
#undef GRIM_I8_OFFSETS
    // drain: the last iterations requested tiles from the empty buffer
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return i - items;
}

// Table mode: the dispatch's tile table (parts & 1) and / or the shared
// expert's tiles (parts & 2) over the whole grid.
template <bool SWIGLU>
__global__ __launch_bounds__(kQThreads) void grouped_gemm_i8_kernel(GemmI8Args g, int n_col_tiles,
                                                                   int parts) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[kQStages][kQStageBytes];
    __shared__ __attribute__((aligned(16))) float meta[2][512];
    __shared__ __attribute__((aligned(16))) int32_t rmap[2][256];
    int n_routed = 0;
    if (parts & 1) {
        n_routed = g.n_tiles_dev ? __builtin_amdgcn_readfirstlane(*g.n_tiles_dev) : g.tmax;
        n_routed = n_routed < g.tmax ? n_routed : g.tmax;
    }
    i8_big_run<SWIGLU>(g, n_col_tiles, parts, n_routed, -1, 0, blockIdx.x / kQXcds, gridDim.x / kQXcds,
                       smem, meta, rmap);
}

// ------------------------------------------------------- narrow tiles
//
// Experts with few rows (the long tail of a skewed routing: most of C4's
// 512 experts hold fewer than 32 of its 40960 rows) on the 128-row tiles
// above cost a whole tile's A feed and MFMAs for a handful of rows, and
// their weights -- read once, from memory -- are the real work.  This
// kernel runs them in 32-row x 256-column tiles whose ring stages span
// 128 K: each weight row's 128 bytes of a stage are one whole memory line,
// and every DMA instruction moves whole lines (B: 8 rows x 128 bytes; A: 4
// limb rows x 256 bytes), which streams weights markedly faster than the
// half-line segments of 64-K stages.  Four waves, three stages of 40 KiB
// (two in flight while one is multiplied); wave w owns tile columns
// [64 w, +64) (SwiGLU: h columns [32 w, +32), gate and up) for all 32
// rows.  Same wait accounting and continuous stage stream across items as
// the 128-row kernel.
constexpr int NBM = 32, NBN = 256, NBK = 128;
constexpr int kNThreads = 256;
constexpr int kNStages = 3;
constexpr int kNA = NBM * 2 * NBK;                 // 8 KiB of limbs
constexpr int kNStageBytes = kNA + NBN * NBK;      // + 32 KiB of codes

bool gemm_i8_narrow_ok(int K) { return K % NBK == 0 && K >= (kNStages - 1) * NBK; }

// The body of the narrow kernel for one work-group (its first kNThreads
// threads): slot / per_xcd as for i8_big_run, total tiles in the list at
// tp_addr.  smem / meta: the kernel's LDS.
template <bool SWIGLU>
__device__ __forceinline__ void i8_narrow_run(const GemmI8Args& g, int n_col_tiles, int total,
                                              int tp_addr, int part, int slot, int per_xcd,
                                              uint8_t (*smem)[kNStageBytes], float (*meta)[512],
                                              int32_t (*rmap)[256]) {
    constexpr int NJA = 2, NJB = 8;          // A / B instructions per wave per stage
    constexpr int OPS = NJA + NJB;
    // meta, per item parity: row scales [32] at 0 (the DMA pads to 256),
    // column scales at 256 (plain: [256]; SwiGLU: gate [128] then up [128])
    const int xcd = blockIdx.x % kQXcds;
    const int lo = int(int64_t(total) * xcd / kQXcds), hi = int(int64_t(total) * (xcd + 1) / kQXcds);
    const int items = i8_part_end((hi - lo) * n_col_tiles, part);
    int i = i8_part_begin((hi - lo) * n_col_tiles, part) + slot;
    if (i >= items) return;

    const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
    const int K = g.K;
    const int a_row_bytes = 2 * K;
    const int64_t wrb = g.row_bytes;

    // Stage layout (K [128 s, +128)):
    //   A 8 KiB: limb row r's 256 bytes (two 64-K blocks of hi then lo
    //     codes: chunk c = 8 block + 4 limb + K%64/16) at r * 256, chunk c
    //     at slot c ^ (r & 15);
    //   B 32 KiB: tile column n's 128 bytes (chunk c = K/16) at 8192 +
    //     n * 128, chunk c at slot c ^ ((n >> 1) & 7).
    // A fragment read (32 rows, one chunk) and a B fragment read (32
    // columns, one chunk) each hit 16 distinct 16-byte slots per 16 lanes.
    int a_off[NJA], a_offn[NJA], b_off[NJB], fa_off[2][2][2], fb_off[2][2][2];
#define GRIM_N8_OFFSETS()                                                                         \
    do {                                                                                          \
        const int ln = lane_id();                                                                 \
        _Pragma("unroll") for (int j = 0; j < NJB; ++j) {                                         \
            const int col = 8 * (NJB * wave + j) + (ln >> 3), sl = ln & 7;                        \
            const int nsub = col >> 5, x = col & 31;                                              \
            const int row = SWIGLU ? ((nsub & 1) ? g.I : 0) + (nsub >> 1) * 32 + x : col;         \
            b_off[j] = row * int(wrb) + ((sl ^ ((col >> 1) & 7)) << 4);                           \
        }                                                                                         \
        _Pragma("unroll") for (int kk = 0; kk < 2; ++kk)                                          \
            _Pragma("unroll") for (int ks = 0; ks < 2; ++ks) {                                    \
                const int ch = 2 * ks + (ln >> 5);                                                \
                const int r = ln & 31;                                                            \
                _Pragma("unroll") for (int l = 0; l < 2; ++l)                                     \
                    fa_off[kk][ks][l] = r * 256 + (((8 * kk + 4 * l + ch) ^ (r & 15)) << 4);      \
                _Pragma("unroll") for (int ni = 0; ni < 2; ++ni) {                                \
                    const int n = (2 * wave + ni) * 32 + (ln & 31);                               \
                    fb_off[kk][ks][ni] = kNA + n * 128 + (((4 * kk + ch) ^ ((n >> 1) & 7)) << 4); \
                }                                                                                 \
            }                                                                                     \
    } while (0)
    GRIM_N8_OFFSETS();
    // A rows: lane (j, ln) moves tile row 4 (NJA wave + j) + ln / 16,
    // chunk ln % 16; gather mode as in the 128-row kernel
    const bool gat = g.gather != nullptr;
    const int rmap_base = int(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int32_t*)(&rmap[0][0])));
    auto a_offsets = [&](const I8Item& it, int rm_addr, int (&o)[NJA]) {
        const int ln = lane_id();
#pragma unroll
        for (int j = 0; j < NJA; ++j) {
            const int r = 4 * (NJA * wave + j) + (ln >> 4), sl = ln & 15;
            const int sw = (sl ^ (r & 15)) << 4;
            if (gat) {
                const int src = lds_i32(rm_addr + 4 * r);
                o[j] = r < it.rows ? src * a_row_bytes + sw : kI8FarOffset;
            } else {
                o[j] = r * a_row_bytes + sw;
            }
        }
    };

    auto tile_of = [&](int ii) { return lo + ii / n_col_tiles; };
    auto col_of = [&](int ii) { return ii % n_col_tiles; };
    const int n_slab = SWIGLU ? 2 * g.I : g.N;
    const int ldo = SWIGLU ? g.I : g.N;
    auto rsrc_a = [&](const I8Item& it) {
        if (gat) return i8_rsrc(g.A, it.rows > 0 ? g.gather_rows * a_row_bytes : 0);
        return i8_rsrc(g.A + it.arow0 * a_row_bytes, it.rows * a_row_bytes);
    };
    auto rsrc_b = [&](const I8Item& it) {
        return i8_rsrc(g.w + it.wrow * wrb, it.rows > 0 ? int((n_slab - it.col0) * wrb) : 0);
    };
    // scale requests: wave 0 the 32 row scales, wave 1 the 256 column
    // scales (SwiGLU: lanes 0..31 gate, 32..63 up)
    auto request_meta = [&](const I8Item& it, int par) {
        const int ln = lane_id();
        if (wave == 0) {
            dma16<0>(i8_rsrc(g.sa + it.arow0, it.rows * 4), reinterpret_cast<uint8_t*>(&meta[par][0]),
                     ln * 16, 0);
        } else if (wave == 2 && gat) {
            dma16<0>(i8_rsrc(g.gather + it.arow0, it.rows * 4), reinterpret_cast<uint8_t*>(&rmap[par][0]),
                     ln * 16, 0);
        } else if (wave == 1) {
            const int m_off = (SWIGLU && ln >= 32) ? g.I * 4 + (ln - 32) * 16 : ln * 16;
            dma16<0>(i8_rsrc(g.ws + it.wrow, it.rows > 0 ? (n_slab - it.col0) * 4 : 0),
                     reinterpret_cast<uint8_t*>(&meta[par][256]), m_off, 0);
        }
    };
    auto request = [&](const I8Item& it, int stage, int t) {
        uint8_t* st = smem[stage];
        const __amdgpu_buffer_rsrc_t ra = rsrc_a(it), rb = rsrc_b(it);
#pragma unroll
        for (int j = 0; j < NJA; ++j) dma16<0>(ra, st + (NJA * wave + j) * 1024, a_off[j], t * 256);
#pragma unroll
        for (int j = 0; j < NJB; ++j) dma16<0>(rb, st + kNA + (NJB * wave + j) * 1024, b_off[j], t * NBK);
    };

    const int nk = K / NBK;   // >= kNStages - 1 (gather mode: >= 4)
    I8Item cur = i8_item<SWIGLU, NBM, NBN>(g, total, tile_of(i), col_of(i), tp_addr);
    I8Item none;
    none.arow0 = 0; none.wrow = 0; none.rows = 0; none.col0 = 0; none.sh = 0;
    request_meta(cur, 0);
    if (gat) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    a_offsets(cur, rmap_base, a_off);
#pragma unroll
    for (int p = 0; p < kNStages - 1; ++p) request(cur, p, p);

    const int smem_base = int(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)(&smem[0][0])));
    const int meta_base = int(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) float*)(&meta[0][0])));
    int gs = 0, par = 0;       // gs: ring slot of the item's stage 0
    bool first = true;
    i32x16 acc[2][2];
    i32x4 fb[2][2], fa[2][2];
    int nev = 0;
    (void)nev;
    for (; i < items; i += per_xcd) {
        GRIM_ITEM_TS(64, 2 * nev, (unsigned long long)(cur.rows) | (2ull << 16));
        GRIM_N8_OFFSETS();
        a_offsets(cur, rmap_base + par * 1024, a_off);
#pragma unroll
        for (int j = 0; j < NJA; ++j) a_offn[j] = a_off[j];
        const bool more = i + per_xcd < items;
        const I8Item nxt = more ? i8_item<SWIGLU, NBM, NBN>(g, total, tile_of(i + per_xcd), col_of(i + per_xcd), tp_addr)
                                : none;
#pragma unroll
        for (int l = 0; l < 2; ++l)
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[l][ni][v] = 0;
        // the wait before stage t: the next stage's loads (YT) are younger,
        // and right after an epilogue (t < 2) also its stores (ES per lane)
        constexpr int YT = OPS;
        constexpr int ES = (SWIGLU ? 1 : 2) * 16;
        constexpr int YE = YT + ES < 63 ? YT + ES : 63;
#define GRIM_N8_WAIT(after_epi)                                                                   \
        asm volatile("s_cmp_eq_u32 %0, 0\n\t"                                                    \
                     "s_cbranch_scc1 .Lgrim_n16_%=\n\t"                                           \
                     "s_waitcnt vmcnt(%2)\n\t"                                                   \
                     "s_branch .Lgrim_ndone_%=\n"                                                 \
                     ".Lgrim_n16_%=:\n\t"                                                        \
                     "s_waitcnt vmcnt(%1)\n"                                                      \
                     ".Lgrim_ndone_%=:\n\t"                                                      \
                     "s_waitcnt lgkmcnt(0)\n\t"                                                  \
                     "s_barrier" ::"s"(__builtin_amdgcn_readfirstlane(after_epi)), "n"(YT), "n"(YE) \
                     : "memory", "scc")
#define GRIM_N8_DSR(dst, addr)                                                                    \
        asm volatile("ds_read_b128 %0, %1" : "=v"(dst) : "v"(addr))
#define GRIM_N8_LGKM(n, ks_)                                                                      \
        asm volatile("s_waitcnt lgkmcnt(" #n ")"                                                   \
                     : "+v"(fb[ks_][0]), "+v"(fb[ks_][1]), "+v"(fa[ks_][0]), "+v"(fa[ks_][1]))
#define GRIM_N8_MMA(ks_)                                                                          \
        _Pragma("unroll") for (int ni = 0; ni < 2; ++ni)                                          \
            _Pragma("unroll") for (int l = 0; l < 2; ++l)                                         \
                acc[l][ni] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[ks_][l], fb[ks_][ni], acc[l][ni], 0, 0, 0)
#define GRIM_N8_READS(kk_)                                                                        \
        _Pragma("unroll") for (int ks = 0; ks < 2; ++ks) {                                        \
            GRIM_N8_DSR(fb[ks][0], sb + fb_off[kk_][ks][0]);                                      \
            GRIM_N8_DSR(fb[ks][1], sb + fb_off[kk_][ks][1]);                                      \
            GRIM_N8_DSR(fa[ks][0], sb + fa_off[kk_][ks][0]);                                      \
            GRIM_N8_DSR(fa[ks][1], sb + fa_off[kk_][ks][1]);                                      \
        }
#define GRIM_N8_DMA(q)                                                                            \
        do {                                                                                      \
            if ((q) < NJA) dma16<0>(qa, nx + (NJA * wave + (q)) * 1024, own ? a_off[(q) % NJA] : a_offn[(q) % NJA], tu * 256); \
            else dma16<0>(qb, nx + kNA + (NJB * wave + (q) - NJA) * 1024, b_off[((q) + NJB - NJA) % NJB], tu * NBK); \
        } while (0)
#define GRIM_N8_ITER(t_, META)                                                                    \
        do {                                                                                      \
            const int t = (t_);                                                                   \
            GRIM_N8_WAIT((t < kNStages - 1 && !first) ? 1 : 0);                                   \
            /* the next item's row map (requested at t = 0, landed by t = 2) */                   \
            if (gat && t == nk - (kNStages - 1)) a_offsets(nxt, rmap_base + (par ^ 1) * 1024, a_offn); \
            const int slot = (gs + t) % kNStages;                                                 \
            const int sb = slot * kNStageBytes + smem_base;                                       \
            GRIM_N8_READS(0);                                                                     \
            if (META) request_meta(nxt, par ^ 1);                                                 \
            /* stream stage t + 2: this item's, or the next item's 0, 1 */                        \
            const int u = t + kNStages - 1;                                                       \
            const bool own = u < nk;                                                              \
            const __amdgpu_buffer_rsrc_t qa = rsrc_a(own ? cur : nxt);                            \
            const __amdgpu_buffer_rsrc_t qb = rsrc_b(own ? cur : nxt);                            \
            const int tu = own ? u : u - nk;                                                      \
            uint8_t* nx = smem[(gs + u) % kNStages];                                              \
            GRIM_N8_LGKM(4, 0); GRIM_N8_MMA(0); GRIM_N8_DMA(0); GRIM_N8_DMA(1);                   \
            GRIM_N8_LGKM(0, 1); GRIM_N8_MMA(1); GRIM_N8_DMA(2); GRIM_N8_DMA(3); GRIM_N8_DMA(4);   \
            GRIM_N8_READS(1);                                                                     \
            GRIM_N8_DMA(5); GRIM_N8_DMA(6);                                                       \
            GRIM_N8_LGKM(4, 0); GRIM_N8_MMA(0); GRIM_N8_DMA(7); GRIM_N8_DMA(8);                   \
            GRIM_N8_LGKM(0, 1); GRIM_N8_MMA(1); GRIM_N8_DMA(9);                                   \
        } while (0)
        GRIM_N8_ITER(0, true);
        for (int t1 = 1; t1 < nk; ++t1) GRIM_N8_ITER(t1, false);
#undef GRIM_N8_ITER
#undef GRIM_N8_WAIT
#undef GRIM_N8_DSR
#undef GRIM_N8_LGKM
#undef GRIM_N8_MMA
#undef GRIM_N8_READS
#undef GRIM_N8_DMA

        // ---- epilogue.  acc[l][ni][v] is row 8 (v/4) + 4 (lane/32) + v%4,
        // column 32 (2 w + ni) + lane%32 of the tile.
        const __amdgpu_buffer_rsrc_t ro = i8_rsrc(g.out + cur.arow0 * ldo, cur.rows * ldo * 4);
        const int mb = meta_base + par * 2048;
        const int ln = lane_id();
        const int hrow = 4 * (ln >> 5);
        f32x4v s4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) s4[q] = lds_f32x4(mb + (8 * q + hrow) * 4);
        if constexpr (SWIGLU) {
            const int hcl = wave * 32 + (ln & 31);
            float sg = lds_f32(mb + 1024 + hcl * 4), su = lds_f32(mb + 1024 + (128 + hcl) * 4);
            int base = cur.col0 + hcl < g.I ? (hrow * g.I + cur.col0 + hcl) * 4 : 0x40000000;
            asm volatile("" : "+v"(base));
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(s4[0]), "+v"(s4[1]), "+v"(s4[2]), "+v"(s4[3]), "+v"(sg), "+v"(su));
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int v = 4 * q + j;
                    const float gv = s4[q][j] * sg * __builtin_fmaf(float(acc[1][0][v]), kLoScale, float(acc[0][0][v]));
                    const float uv = s4[q][j] * su * __builtin_fmaf(float(acc[1][1][v]), kLoScale, float(acc[0][1][v]));
                    const int off = base + (8 * q + j) * g.I * 4;
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, fast_silu(gv) * uv), ro, off, 0, 0);
                }
        } else {
            float sc[2];
            int base[2];
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const int cl = wave * 64 + ni * 32 + (ln & 31);
                sc[ni] = lds_f32(mb + 1024 + cl * 4);
                base[ni] = cur.col0 + cl < g.N ? (hrow * g.N + cur.col0 + cl) * 4 : 0x40000000;
            }
            asm volatile("" : "+v"(base[0]), "+v"(base[1]));
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(s4[0]), "+v"(s4[1]), "+v"(s4[2]), "+v"(s4[3]), "+v"(sc[0]), "+v"(sc[1]));
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int v = 4 * q + j;
                        const float y = s4[q][j] * sc[ni] * __builtin_fmaf(float(acc[1][ni][v]), kLoScale, float(acc[0][ni][v]));
                        const int off = base[ni] + (8 * q + j) * g.N * 4;
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), ro, off, 0, 0);
                    }
        }
        GRIM_ITEM_TS(64, 2 * nev + 1, 0ull);
        ++nev;
        gs = (gs + nk) % kNStages;
        par ^= 1;
        cur = nxt;
        first = false;
    }
#undef GRIM_N8_OFFSETS
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// The number of s_barrier instructions i8_narrow_run executes for the
// same arguments (its gather prologue, then one per K stage of each of its
// items): what the waves that sit the narrow run out execute instead, so
// that every barrier of the work-group still pairs up.
__device__ __forceinline__ int i8_narrow_barriers(const GemmI8Args& g, int n_col_tiles, int total, int part,
                                                  int slot, int per_xcd) {
    const int xcd = blockIdx.x % kQXcds;
    const int lo = int(int64_t(total) * xcd / kQXcds), hi = int(int64_t(total) * (xcd + 1) / kQXcds);
    const int items = i8_part_end((hi - lo) * n_col_tiles, part);
    const int i = i8_part_begin((hi - lo) * n_col_tiles, part) + slot;
    if (i >= items) return 0;
    const int mine = (items - i + per_xcd - 1) / per_xcd;
    return (g.gather ? 1 : 0) + mine * (g.K / NBK);
}

// Rows mode, one launch: every work-group forms both tile lists (experts
// above list_lo rows in 128-row tiles, then the shared expert's for parts &
// 2; experts of 1..split rows in 32-row tiles when list_lo > 0).
//
// With both lists non-empty the work-groups of an XCD form two halves that
// take the lists in opposite orders: even slots walk the first half of the
// 128-row items and then the second half of the narrow ones, odd slots the
// first half of the narrow items and then the second half of the 128-row
// ones.  The 128-row items are bound by the matrix core and the LDS (their
// operands come mostly from the L2), the narrow ones by the memory stream
// (each expert's weights read once for a few rows): run side by side on
// different CUs they overlap, where run one after the other on every CU
// the narrow phase had all 256 CUs contending for memory (a narrow item
// took 1.5x as long as with half of them).  The narrow run uses the first
// four waves; the other four end after it, or (odd slots, which run the
// 128-row items afterwards) execute as many barriers as it does and wait.
//
// With one list only: every work-group walks its share of the 128-row
// items, then -- continuing the same round robin over its XCD's work-groups
// -- its share of the narrow ones.
template <bool SWIGLU>
__global__ __launch_bounds__(kQThreads) void grouped_gemm_i8_rows_kernel(GemmI8Args g, int nct_big,
                                                                        int nct_nar, int parts) {
    __shared__ __attribute__((aligned(1024))) uint8_t ring[kQStages * kQStageBytes];
    __shared__ __attribute__((aligned(16))) float meta[2][512];
    __shared__ int32_t tpb[kI8MaxListExperts], tpn[kI8MaxListExperts];
    __shared__ __attribute__((aligned(16))) int32_t rmap[2][256];
    static_assert(kNStages * kNStageBytes <= kQStages * kQStageBytes, "narrow ring fits");
    int32_t* tmp = reinterpret_cast<int32_t*>(ring);
    const int E = g.num_experts;
    const int nb = (parts & 1) ? i8_list_scan<QBM, kQThreads>(g.counts, E, g.list_lo, 0x7FFFFFFF, tpb, tmp) : 0;
    const int nn = ((parts & 1) && g.list_lo > 0) ? i8_list_scan<NBM, kQThreads>(g.counts, E, 0, g.split, tpn, tmp) : 0;
    const int S = gridDim.x / kQXcds;            // work-group slots per XCD
    const int q = blockIdx.x / kQXcds;           // this work-group's slot
    const int tpa_b = int(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int32_t*)(&tpb[0])));
    const int tpa_n = int(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) int32_t*)(&tpn[0])));
    const int nb_total = nb + ((parts & 2) ? (g.T_sh + QBM - 1) / QBM : 0);
    auto big = reinterpret_cast<uint8_t (*)[kQStageBytes]>(ring);
    auto nar = reinterpret_cast<uint8_t (*)[kNStageBytes]>(ring);
    if (nn > 0 && nb_total > 0 && S >= 2 && S % 2 == 0) {
        const int h = S / 2, p = q >> 1;
        if ((q & 1) == 0) {
            i8_big_run<SWIGLU>(g, nct_big, parts, nb, tpa_b, 1, p, h, big, meta, rmap);
            __syncthreads();                     // every wave is past the 128-row ring
            if (threadIdx.x >= kNThreads) return;
            i8_narrow_run<SWIGLU>(g, nct_nar, nn, tpa_n, 2, p, h, nar, meta, rmap);
        } else {
            if (threadIdx.x < kNThreads) {
                i8_narrow_run<SWIGLU>(g, nct_nar, nn, tpa_n, 1, p, h, nar, meta, rmap);
            } else {
                const int nbar = i8_narrow_barriers(g, nct_nar, nn, 1, p, h);
                for (int b = 0; b < nbar; ++b) __builtin_amdgcn_s_barrier();
            }
            __syncthreads();                     // every wave is past the narrow ring
            i8_big_run<SWIGLU>(g, nct_big, parts, nb, tpa_b, 2, p, h, big, meta, rmap);
        }
        return;
    }
    const int next = i8_big_run<SWIGLU>(g, nct_big, parts, nb, tpa_b, 0, q, S, big, meta, rmap);
    if (nn == 0) return;
    __syncthreads();                             // every wave is past the 128-row ring
    if (threadIdx.x >= kNThreads) return;
    i8_narrow_run<SWIGLU>(g, nct_nar, nn, tpa_n, 0, next, S, nar, meta, rmap);
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

// Rows of n <= 512 (h of C4-like layers): one wave per kQuantRowsPerWave
// rows, each lane holding its 8 elements of every row in registers, all
// loads issued before the first reduction; the same arithmetic as
// quant_rows_kernel (limbs8), so the same limbs and scales.
constexpr int kQuantRowsPerWave = 4;

// Two row sets in one launch: the waves of the first cover rows / 4 of
// them, the rest the second set's (src2, may be empty).
__global__ __launch_bounds__(256) void quant_rows_short_kernel(const float* __restrict__ src, int rows,
                                                               int n, int8_t* __restrict__ dst,
                                                               float* __restrict__ scale,
                                                               const float* __restrict__ src2, int rows2,
                                                               int8_t* __restrict__ dst2,
                                                               float* __restrict__ scale2) {
    const int lane = threadIdx.x & 63;
    const int wv = blockIdx.x * 4 + int(threadIdx.x) / 64;
    const int nw1 = (rows + kQuantRowsPerWave - 1) / kQuantRowsPerWave;
    if (wv >= nw1) {
        src = src2;
        rows = rows2;
        dst = dst2;
        scale = scale2;
    }
    const int r0 = (wv >= nw1 ? wv - nw1 : wv) * kQuantRowsPerWave;
    if (r0 >= rows) return;
    const int c = lane * 8;
    const bool in = c < n;
    float v[kQuantRowsPerWave][8];
#pragma unroll
    for (int q = 0; q < kQuantRowsPerWave; ++q) {
        const int r = r0 + q < rows ? r0 + q : r0;
        const float* s = src + int64_t(r) * n + (in ? c : 0);
        const float4 a = *reinterpret_cast<const float4*>(s);
        const float4 b = *reinterpret_cast<const float4*>(s + 4);
        v[q][0] = a.x; v[q][1] = a.y; v[q][2] = a.z; v[q][3] = a.w;
        v[q][4] = b.x; v[q][5] = b.y; v[q][6] = b.z; v[q][7] = b.w;
    }
#pragma unroll
    for (int q = 0; q < kQuantRowsPerWave; ++q) {
        const int r = r0 + q;
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[q][i]));
        m = wave_max_f(in ? m : 0.0f);
        const float sc = m > 0.0f ? m / 127.0f : 1.0f;
        const float inv = m > 0.0f ? 127.0f / m : 0.0f;
        uint32_t h0, h1, l0, l1;
        limbs8(v[q], inv, h0, h1, l0, l1);
        if (r < rows) {
            if (in) {
                int8_t* blk = dst + int64_t(r) * 2 * n + limb_block(c);
                *reinterpret_cast<uint2*>(blk) = make_uint2(h0, h1);
                *reinterpret_cast<uint2*>(blk + 64) = make_uint2(l0, l1);
            }
            if (lane == 0) scale[r] = sc;
        }
    }
}

// The activations of every token as limbs, written to each of its K
// permuted rows (inverse) when xq is given and to its own row (xrowq: the
// shared expert's input, and the gather source of gather mode) when given;
// the scale to every permuted row, and the token to perm[permuted row];
// with gate_w (bf16 [n], 16-byte aligned) also gate[t] = sigmoid(x_t . w),
// the shared expert's gate, from the same loads.
// One work-group of 256 threads per token, n <= 8192.
__global__ __launch_bounds__(256) void quant_permute_kernel(const float* __restrict__ x, int n, int K,
                                                            const int32_t* __restrict__ inverse,
                                                            int8_t* __restrict__ xq, float* __restrict__ sq,
                                                            int8_t* __restrict__ xrowq,
                                                            float* __restrict__ srow,
                                                            int32_t* __restrict__ perm,
                                                            const uint16_t* __restrict__ gate_w,
                                                            float* __restrict__ gate) {
    __shared__ float red[4], gred[4];
    const int t = blockIdx.x;
    const float* s = x + int64_t(t) * n;
    // this thread's route row (threads < K), requested with the row's loads
    // instead of after the reduction's barrier
    const int dk_own = int(threadIdx.x) < K ? inverse[int64_t(t) * K + threadIdx.x] : -1;
    float4 va[4], vb[4];
    float m = 0.0f, d = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int c = threadIdx.x * 8 + q * 2048;
        if (c < n) {
            va[q] = *reinterpret_cast<const float4*>(s + c);
            vb[q] = *reinterpret_cast<const float4*>(s + c + 4);
            m = fmaxf(m, fmaxf(fmaxf(fabsf(va[q].x), fabsf(va[q].y)), fmaxf(fabsf(va[q].z), fabsf(va[q].w))));
            m = fmaxf(m, fmaxf(fmaxf(fabsf(vb[q].x), fabsf(vb[q].y)), fmaxf(fabsf(vb[q].z), fabsf(vb[q].w))));
            if (gate_w) {
                // the shared expert's gate: x . w in one fixed order (the
                // thread's 8 elements per 2048, then the waves' DPP sums,
                // then the four waves in order)
                const uint4 u = *reinterpret_cast<const uint4*>(gate_w + c);
                d = __builtin_fmaf(bits_f(u.x << 16), va[q].x, d);
                d = __builtin_fmaf(bits_f(u.x & 0xFFFF0000u), va[q].y, d);
                d = __builtin_fmaf(bits_f(u.y << 16), va[q].z, d);
                d = __builtin_fmaf(bits_f(u.y & 0xFFFF0000u), va[q].w, d);
                d = __builtin_fmaf(bits_f(u.z << 16), vb[q].x, d);
                d = __builtin_fmaf(bits_f(u.z & 0xFFFF0000u), vb[q].y, d);
                d = __builtin_fmaf(bits_f(u.w << 16), vb[q].z, d);
                d = __builtin_fmaf(bits_f(u.w & 0xFFFF0000u), vb[q].w, d);
            }
        }
    }
    m = wave_max_f(m);
    if (gate_w) d = group_sum<kWave>(d);
    if ((threadIdx.x & 63) == 0) {
        red[threadIdx.x / 64] = m;
        gred[threadIdx.x / 64] = d;
    }
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    if (gate_w && threadIdx.x == 0) gate[t] = det_sigmoid((gred[0] + gred[1]) + (gred[2] + gred[3]));
    const float sc = m > 0.0f ? m / 127.0f : 1.0f;
    const float inv = m > 0.0f ? 127.0f / m : 0.0f;
    int dst[16];
    if (xq)
        for (int k = 0; k < K; ++k) dst[k] = inverse[int64_t(t) * K + k];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int c = threadIdx.x * 8 + q * 2048;
        if (c < n) {
            const float v[8] = {va[q].x, va[q].y, va[q].z, va[q].w, vb[q].x, vb[q].y, vb[q].z, vb[q].w};
            uint32_t h0, h1, l0, l1;
            limbs8(v, inv, h0, h1, l0, l1);
            for (int k = 0; k < K && xq; ++k) {
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
    if (dk_own >= 0) {
        sq[dk_own] = sc;
        if (perm) perm[dk_own] = t;
    }
    if (srow && threadIdx.x == 0) srow[t] = sc;
}

// ----------------------------------------------------------------- host

template <typename Kern>
static int i8_grid(Kern k, int threads = kQThreads) {
    int per_cu = 0, dev = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, threads, 0) != hipSuccess ||
        hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    const int grid = (per_cu > 0 ? per_cu : 1) * cus;
    return (grid + kQXcds - 1) / kQXcds * kQXcds;
}

template <bool SWIGLU>
static hipError_t launch_i8(hipStream_t st, const GemmI8Args& g, int ntiles) {
    static int grid = 0, grid_r = 0;
    if (grid == 0) {
        grid = i8_grid(grouped_gemm_i8_kernel<SWIGLU>);
        grid_r = i8_grid(grouped_gemm_i8_rows_kernel<SWIGLU>);
        if (grid == 0 || grid_r == 0) {
            grid = 0;
            return hipErrorInvalidConfiguration;
        }
    }
    const bool rows_mode = g.split > 0;
    const bool routed = rows_mode || g.tmax > 0;
    const bool fuse = routed && g.T_sh > 0 && g.row_bytes == g.row_bytes_sh;
    if (rows_mode) {
        const int nct = SWIGLU ? (g.I + NBN / 2 - 1) / (NBN / 2) : (g.N + NBN - 1) / NBN;
        hipLaunchKernelGGL(grouped_gemm_i8_rows_kernel<SWIGLU>, dim3(grid_r), dim3(kQThreads), 0, st, g,
                           ntiles, nct, fuse ? 3 : 1);
    } else if (fuse) {
        // the shared expert's m-tiles follow the routed ones in one launch
        hipLaunchKernelGGL(grouped_gemm_i8_kernel<SWIGLU>, dim3(grid), dim3(kQThreads), 0, st, g,
                           ntiles, 3);
    } else if (routed) {
        hipLaunchKernelGGL(grouped_gemm_i8_kernel<SWIGLU>, dim3(grid), dim3(kQThreads), 0, st, g,
                           ntiles, 1);
    }
    if (g.T_sh > 0 && !fuse) {
        const int items = (g.T_sh + QBM - 1) / QBM * ntiles;
        const int gs = min(grid, (items + kQXcds - 1) / kQXcds * kQXcds);
        hipLaunchKernelGGL(grouped_gemm_i8_kernel<SWIGLU>, dim3(gs), dim3(kQThreads), 0, st, g,
                           ntiles, 2);
    }
    return hipGetLastError();
}

bool gemm_i8_shape_ok(int N, int K, int I, int swiglu) {
    if (K % QBK || K < 3 * QBK || K > 8192) return false;
    if (swiglu) return I > 0 && N == 2 * I;
    return N > 0;
}

bool gemm_i8_gather_ok(int K, int rows) {
    // the next item's row map is read at its first streamed tile: 128-row
    // kernel nk - 3 >= 3, narrow kernel (when it runs) nk - 2 >= 2
    const bool big = K % QBK == 0 && K / QBK >= 6;
    const bool nar = !gemm_i8_narrow_ok(K) || K / NBK >= 4;
    return big && nar && rows > 0 && int64_t(rows) * 2 * K < kI8FarOffset;
}

hipError_t gemm_i8_launch(hipStream_t st, const GemmI8Args& g) {
    if (!gemm_i8_shape_ok(g.N, g.K, g.I, g.swiglu)) return hipErrorInvalidValue;
    if (g.gather && !gemm_i8_gather_ok(g.K, g.gather_rows)) return hipErrorInvalidValue;
    if (g.split > 0 && (g.num_experts <= 0 || g.num_experts > kI8MaxListExperts))
        return hipErrorInvalidValue;
    if (g.split > 0) {
        // rows mode: the 128-row kernel takes the experts above list_lo rows,
        // the narrow one the rest (all on the 128-row kernel when K does not
        // fit the narrow kernel's 128-K stages)
        GemmI8Args r = g;
        r.list_lo = gemm_i8_narrow_ok(g.K) ? g.split : 0;
        const int nt = r.swiglu ? (r.I + QBN / 2 - 1) / (QBN / 2) : (r.N + QBN - 1) / QBN;
        return r.swiglu ? launch_i8<true>(st, r, nt) : launch_i8<false>(st, r, nt);
    }
    const int ntiles = g.swiglu ? (g.I + QBN / 2 - 1) / (QBN / 2) : (g.N + QBN - 1) / QBN;
    if (ntiles <= 0) return hipSuccess;
    return g.swiglu ? launch_i8<true>(st, g, ntiles) : launch_i8<false>(st, g, ntiles);
}

hipError_t quant_rows_launch(hipStream_t st, const float* src, int rows, int n, int8_t* dst,
                             float* scale, const float* src2, int rows2, int8_t* dst2, float* scale2) {
    if (n % 64 || n > 4096) return hipErrorInvalidValue;
    if (!src2) rows2 = 0;
    if (rows <= 0 && rows2 <= 0) return hipSuccess;
    if (n <= 512) {
        const int waves = (rows + kQuantRowsPerWave - 1) / kQuantRowsPerWave +
                          (rows2 + kQuantRowsPerWave - 1) / kQuantRowsPerWave;
        hipLaunchKernelGGL(quant_rows_short_kernel, dim3((waves + 3) / 4), dim3(256), 0, st,
                           src, rows, n, dst, scale, src2, rows2, dst2, scale2);
        return hipGetLastError();
    }
    if (rows2 > 0) {
        hipError_t e = quant_rows_launch(st, src2, rows2, n, dst2, scale2);
        if (e != hipSuccess) return e;
    }
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(quant_rows_kernel, dim3((rows + kQuantRowsPerBlock - 1) / kQuantRowsPerBlock),
                       dim3(256), 0, st, src, rows, n, dst, scale);
    return hipGetLastError();
}

hipError_t quant_permute_launch(hipStream_t st, const float* x, int T, int n, int K,
                                const int32_t* inverse, int8_t* xq, float* sq, int8_t* xrowq,
                                float* srow, int32_t* perm, const uint16_t* gate_w, float* gate) {
    if (T <= 0) return hipSuccess;
    if (n % 64 || n > 8192 || K > 16) return hipErrorInvalidValue;
    if (gate_w && (reinterpret_cast<uintptr_t>(gate_w) & 15)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(quant_permute_kernel, dim3(T), dim3(256), 0, st, x, n, K, inverse, xq, sq,
                       xrowq, srow, perm, gate_w, gate);
    return hipGetLastError();
}

}  // namespace grim
