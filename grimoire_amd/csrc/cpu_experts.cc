// cpu_experts.cc -- NVFP4 routed experts computed by host threads.
//
// The CPU side of the tiered experts (behaviour of src/cpu_experts.cpp:242-363
// and include/b70/cpu_experts.hpp): an expert block that lives in host memory
// is read by the host cores at DRAM speed instead of by the GPU over PCIe; the
// caller adds the host partial sum to the device one.  Same block layout as
// the GPU tiered kernels (grim_nv_expert_layout).
//
// Arithmetic.  Every weight is exact in fp32: an e2m1 value (at most two
// significant bits) times its block's E4M3 scale (at most four) needs six
// bits.  One (weight row, activation vector) dot product is a fixed chain:
// 16 lane accumulators, block b of 16 elements adds w[16b + l] * x[16b + l]
// into lane l by one fma (blocks in order), and the lanes are summed by
// halving (l + 8, + 4, + 2, + 1).  The AVX-512, AVX2 and scalar kernels all
// perform exactly this chain for every (row, vector) pair, whatever number
// of rows and vectors they block together, so the instruction set, the
// blocking and the thread count never change a bit.
//
// Decoding: a 16-element block is 8 payload bytes.  The bytes are doubled
// (each byte twice, so lane l holds byte l / 2), widened to 32-bit lanes and
// shifted right by 4 on odd lanes; the low four bits of each lane are then
// the element's e2m1 code, which indexes a 16-entry float table by a
// register permute (AVX-512: vpermps over all 16 codes; AVX2: the 8
// magnitudes by vpermps and the sign from bit 3).
//
// Work.  One call is one job of items on a pool: first the gate/up items
// (a group of slots that share one expert block x 16 intermediate rows),
// then the down items (64 outputs x one group).  Slots are grouped by
// sorting (block pointer, slot) pairs, so each distinct block's rows are
// decoded once and multiplied with every vector routed to it.  A down item
// starts when its group's gate/up items have all finished (a per-group
// countdown), writes per-slot partial dots, and the thread that finishes the
// last group of an output tile sums the tile's partials in slot order for
// every row.  No step waits for the whole of a pass.
//
// Host-only code (built by the C++ compiler, not the HIP one).
#include "grimoire_moe.h"

#include <immintrin.h>
#include <pthread.h>
#include <sched.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <new>
#include <thread>
#include <utility>
#include <vector>

namespace {

// ------------------------------------------------------------ formats

// e2m1 code -> value; code 8 is -0
alignas(64) constexpr float kE2m1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                         -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

// E4M3 (OCP: no infinities, 0x7F / 0xFF NaN) -> fp32
float e4m3_value(uint8_t b) {
    const int e = (b >> 3) & 15, m = b & 7;
    float v;
    if (e == 15 && m == 7) return std::nanf("");
    if (e == 0) v = std::ldexp(float(m), -9);
    else v = std::ldexp(float(8 + m), e - 10);
    return (b & 0x80) ? -v : v;
}

const float* e4m3_table() {
    static const struct T {
        float v[256];
        T() {
            for (int i = 0; i < 256; ++i) v[i] = e4m3_value(uint8_t(i));
        }
    } t;
    return t.v;
}

// the lane tree every kernel ends with
float lanes_sum(float (&v)[16]) {
    for (int w = 8; w >= 1; w >>= 1)
        for (int l = 0; l < w; ++l) v[l] = v[l] + v[l + w];
    return v[0];
}

// One call: R weight rows (payload, scales) x G activation vectors, K
// elements; out[r * G + g] = the chain for (row r, vector g).
struct RowSet {
    const uint8_t* pay[4];
    const uint8_t* scl[4];
};
constexpr int kMaxR = 4, kMaxG = 4;

// ------------------------------------------------------------ scalar

template <int R, int G>
void rows_scalar(const RowSet& rs, const float* const* xs, int K, float* out) {
    const float* sc = e4m3_table();
    float acc[R][G][16] = {};
    for (int b = 0; b < K / 16; ++b)
        for (int r = 0; r < R; ++r) {
            const float s = sc[rs.scl[r][b]];
            float w[16];
            for (int l = 0; l < 16; ++l) {
                const uint8_t byte = rs.pay[r][8 * b + l / 2];
                w[l] = kE2m1[(byte >> (4 * (l & 1))) & 15] * s;
            }
            for (int g = 0; g < G; ++g)
                for (int l = 0; l < 16; ++l) acc[r][g][l] = std::fma(w[l], xs[g][16 * b + l], acc[r][g][l]);
        }
    for (int r = 0; r < R; ++r)
        for (int g = 0; g < G; ++g) out[r * G + g] = lanes_sum(acc[r][g]);
}

// ------------------------------------------------------------ AVX2

template <int R, int G>
__attribute__((target("avx2,fma"))) void rows_avx2(const RowSet& rs, const float* const* xs, int K, float* out) {
    const float* sc = e4m3_table();
    const __m256 mag = _mm256_loadu_ps(kE2m1);      // codes 0-7
    const __m256i odd4 = _mm256_setr_epi32(0, 4, 0, 4, 0, 4, 0, 4);
    const __m256i sign = _mm256_set1_epi32(int(0x80000000u));
    __m256 acc[R][G][2];
    for (int r = 0; r < R; ++r)
        for (int g = 0; g < G; ++g) acc[r][g][0] = acc[r][g][1] = _mm256_setzero_ps();
    for (int b = 0; b < K / 16; ++b) {
        for (int r = 0; r < R; ++r) {
            const __m128i v = _mm_loadl_epi64(reinterpret_cast<const __m128i*>(rs.pay[r] + 8 * b));
            const __m128i d = _mm_unpacklo_epi8(v, v);    // byte i at positions 2i, 2i + 1
            const __m256 s = _mm256_set1_ps(sc[rs.scl[r][b]]);
            __m256 w[2];
            for (int h = 0; h < 2; ++h) {
                const __m256i c = _mm256_srlv_epi32(_mm256_cvtepu8_epi32(h ? _mm_srli_si128(d, 8) : d), odd4);
                const __m256 m = _mm256_permutevar8x32_ps(mag, c);
                const __m256 sg = _mm256_castsi256_ps(_mm256_and_si256(_mm256_slli_epi32(c, 28), sign));
                w[h] = _mm256_mul_ps(_mm256_xor_ps(m, sg), s);
            }
            for (int g = 0; g < G; ++g) {
                const float* xp = xs[g] + 16 * b;
                acc[r][g][0] = _mm256_fmadd_ps(w[0], _mm256_loadu_ps(xp), acc[r][g][0]);
                acc[r][g][1] = _mm256_fmadd_ps(w[1], _mm256_loadu_ps(xp + 8), acc[r][g][1]);
            }
        }
    }
    for (int r = 0; r < R; ++r)
        for (int g = 0; g < G; ++g) {
            float v[16];
            _mm256_storeu_ps(v, acc[r][g][0]);
            _mm256_storeu_ps(v + 8, acc[r][g][1]);
            out[r * G + g] = lanes_sum(v);
        }
}

// ------------------------------------------------------------ AVX-512

template <int R, int G>
__attribute__((target("avx512f,avx512bw,avx2,fma"))) void rows_avx512(const RowSet& rs, const float* const* xs,
                                                                       int K, float* out) {
    const float* sc = e4m3_table();
    const __m512 table = _mm512_loadu_ps(kE2m1);
    const __m512i odd4 = _mm512_setr_epi32(0, 4, 0, 4, 0, 4, 0, 4, 0, 4, 0, 4, 0, 4, 0, 4);
    __m512 acc[R][G];
    for (int r = 0; r < R; ++r)
        for (int g = 0; g < G; ++g) acc[r][g] = _mm512_setzero_ps();
    for (int b = 0; b < K / 16; ++b) {
        __m512 xv[G];
        for (int g = 0; g < G; ++g) xv[g] = _mm512_loadu_ps(xs[g] + 16 * b);
        for (int r = 0; r < R; ++r) {
            const __m128i v = _mm_loadl_epi64(reinterpret_cast<const __m128i*>(rs.pay[r] + 8 * b));
            const __m512i c = _mm512_srlv_epi32(_mm512_cvtepu8_epi32(_mm_unpacklo_epi8(v, v)), odd4);
            const __m512 w = _mm512_mul_ps(_mm512_permutexvar_ps(c, table), _mm512_set1_ps(sc[rs.scl[r][b]]));
            for (int g = 0; g < G; ++g) acc[r][g] = _mm512_fmadd_ps(w, xv[g], acc[r][g]);
        }
    }
    for (int r = 0; r < R; ++r)
        for (int g = 0; g < G; ++g) {
            float v[16];
            _mm512_storeu_ps(v, acc[r][g]);
            out[r * G + g] = lanes_sum(v);
        }
}

// ------------------------------------------------------------ dispatch

using RowsFn = void (*)(const RowSet&, const float* const*, int, float*);

#define GRIM_ROWS_TABLE(NAME, FN)                                              \
    const RowsFn NAME[kMaxR][kMaxG] = {                                        \
        {FN<1, 1>, FN<1, 2>, FN<1, 3>, FN<1, 4>}, {FN<2, 1>, FN<2, 2>, FN<2, 3>, FN<2, 4>}, \
        {FN<3, 1>, FN<3, 2>, FN<3, 3>, FN<3, 4>}, {FN<4, 1>, FN<4, 2>, FN<4, 3>, FN<4, 4>}};
GRIM_ROWS_TABLE(kScalar, rows_scalar)
GRIM_ROWS_TABLE(kAvx2, rows_avx2)
GRIM_ROWS_TABLE(kAvx512, rows_avx512)
#undef GRIM_ROWS_TABLE

std::atomic<int> g_isa{-1};   // 0 scalar, 1 AVX2, 2 AVX-512; -1 = not chosen yet

int best_isa() {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw")) return 2;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return 1;
    return 0;
}

const RowsFn (*rows_table())[kMaxG] {
    int isa = g_isa.load(std::memory_order_relaxed);
    if (isa < 0) {
        isa = best_isa();
        g_isa.store(isa, std::memory_order_relaxed);
    }
    return isa == 2 ? kAvx512 : isa == 1 ? kAvx2 : kScalar;
}

float silu_mul(float g, float u) { return g / (1.0f + std::exp(-g)) * u; }

constexpr uint64_t kIdxBits = 20, kIdxMask = (uint64_t(1) << kIdxBits) - 1;
constexpr int kMaxItems = 1 << 19;   // leaves room for late claims in the index field

}  // namespace

// ------------------------------------------------------------ pool
//
// A job is n items numbered 0 .. n-1, run as fn(ctx, item).  It is published
// in one 64-bit claim word: generation (bits 40+), item count (20-39) and the
// next unclaimed item (0-19).  Every participant, the caller included, takes
// items by fetch_add on that word; the value returned names the generation
// and count it belongs to, so an index below the count is a real item of the
// current job and an index at or above it means the job has no items left.
// The caller then waits until the job's finished-item count reaches n.  A
// thread that arrives late only adds to the index field (bounded by the
// thread count) and takes nothing; fn and ctx cannot change while a claimed
// item runs, because the job cannot finish before it.  Idle threads spin on
// the claim word for a while and then sleep on a bell the caller rings when
// it publishes.

struct grim_cpu_experts {
    int nthreads = 1;
    std::vector<std::thread> threads;
    std::atomic<uint64_t> claim{0};
    std::atomic<int> finished{0};
    std::atomic<uint32_t> bell{0};
    std::atomic<int> sleepers{0};
    std::atomic<bool> quit{false};
    void (*fn)(void*, int) = nullptr;
    void* ctx = nullptr;
    double wait_us = 0.0;

    // per-call state of an FFN (owned by the pool so calls allocate only to grow)
    std::vector<std::pair<uintptr_t, int>> order;   // (block, slot) sorted
    std::vector<int> group_begin;                     // groups: runs of one block in `order`
    std::vector<int> slot_row;
    std::vector<float> h, part;
    std::unique_ptr<std::atomic<int>[]> gu_left, tile_left;
    size_t gu_cap = 0, tile_cap = 0;

    static uint64_t gen_of(uint64_t w) { return w >> 40; }
    static int count_of(uint64_t w) { return int((w >> kIdxBits) & kIdxMask); }
    static int index_of(uint64_t w) { return int(w & kIdxMask); }

    // take and run items until the claimed index is past the count
    void drain() {
        for (;;) {
            const uint64_t w = claim.fetch_add(1, std::memory_order_acq_rel);
            const int i = index_of(w);
            if (i >= count_of(w)) return;
            fn(ctx, i);
            finished.fetch_add(1, std::memory_order_release);
        }
    }

    void loop(int cpu) {
        if (cpu >= 0) {
            cpu_set_t s;
            CPU_ZERO(&s);
            CPU_SET(cpu, &s);
            pthread_setaffinity_np(pthread_self(), sizeof s, &s);
        }
        uint64_t seen = gen_of(claim.load(std::memory_order_acquire));
        int idle = 0;
        while (!quit.load(std::memory_order_acquire)) {
            const uint32_t b = bell.load(std::memory_order_acquire);
            const uint64_t w = claim.load(std::memory_order_acquire);
            if (gen_of(w) != seen) {
                seen = gen_of(w);
                if (index_of(w) < count_of(w)) drain();
                idle = 0;
                continue;
            }
            if (++idle < 30000) {
                _mm_pause();
                continue;
            }
            // seq_cst with run()'s store of the claim word and its load of
            // `sleepers`: one of the two sides sees the other
            sleepers.fetch_add(1, std::memory_order_seq_cst);
            if (gen_of(claim.load(std::memory_order_seq_cst)) == seen && !quit.load()) bell.wait(b);
            sleepers.fetch_sub(1, std::memory_order_acq_rel);
            idle = 0;
        }
    }

    void run(int n, void (*f)(void*, int), void* c) {
        if (n <= 0) return;
        fn = f;
        ctx = c;
        finished.store(0, std::memory_order_relaxed);
        const uint64_t g = gen_of(claim.load(std::memory_order_relaxed)) + 1;
        claim.store((g << 40) | (uint64_t(n) << kIdxBits), std::memory_order_seq_cst);
        if (sleepers.load(std::memory_order_seq_cst) > 0) {
            bell.fetch_add(1, std::memory_order_release);
            bell.notify_all();
        }
        drain();
        const auto t0 = std::chrono::steady_clock::now();
        while (finished.load(std::memory_order_acquire) < n) _mm_pause();
        wait_us += std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    }

    void grow_counters(size_t groups, size_t tiles) {
        if (groups > gu_cap) {
            gu_left.reset(new std::atomic<int>[groups]);
            gu_cap = groups;
        }
        if (tiles > tile_cap) {
            tile_left.reset(new std::atomic<int>[tiles]);
            tile_cap = tiles;
        }
    }

    ~grim_cpu_experts() {
        quit.store(true, std::memory_order_release);
        bell.fetch_add(1, std::memory_order_release);
        bell.notify_all();
        for (auto& t : threads) t.join();
    }
};

namespace {

constexpr int kGuRows = 16;    // gate/up item: 16 intermediate rows of one group
constexpr int kDnOuts = 64;    // down item: 64 outputs of one group

int check_layout(const grim_nv_expert_layout* L) {
    if (!L || L->H <= 0 || L->I <= 0 || L->H % 128 || L->I % 128) return GRIM_ERR_SHAPE;
    return GRIM_OK;
}

// One FFN call over `rows` rows and their slots.
struct Ffn {
    grim_cpu_experts* p;
    grim_nv_expert_layout L;
    const uint8_t* const* blocks;
    const float* w;
    const int32_t* off;
    int rows, slots, groups, gu_items, tiles;
    const float* x;
    float* y;
    const RowsFn (*kern)[kMaxG];

    const uint8_t* block_of(int grp) const {
        return reinterpret_cast<const uint8_t*>(p->order[size_t(p->group_begin[size_t(grp)])].first);
    }

    // gate/up of one group: rows i0 .. i0 + 15 against every slot of the group
    void gate_up(int grp, int i0) {
        const int H = L.H, I = L.I;
        const uint8_t* b = block_of(grp);
        const float* s3 = reinterpret_cast<const float*>(b + L.gsc);
        const int q0 = p->group_begin[size_t(grp)], q1 = p->group_begin[size_t(grp) + 1];
        for (int i = i0; i < i0 + kGuRows; i += 2) {
            RowSet rs;
            for (int k = 0; k < 4; ++k) {
                const int row = (k & 1 ? I : 0) + i + (k >> 1);   // gate i, up i, gate i+1, up i+1
                rs.pay[k] = b + L.gu_p + size_t(row) * (H / 2);
                rs.scl[k] = b + L.gu_s + size_t(row) * (H / 16);
            }
            for (int q = q0; q < q1; q += kMaxG) {
                const int G = std::min(kMaxG, q1 - q);
                const float* xs[kMaxG];
                for (int g = 0; g < G; ++g) xs[g] = x + size_t(p->slot_row[size_t(p->order[size_t(q + g)].second)]) * H;
                float d[4 * kMaxG];
                kern[3][G - 1](rs, xs, H, d);
                for (int g = 0; g < G; ++g) {
                    float* hs = p->h.data() + size_t(p->order[size_t(q + g)].second) * I;
                    hs[i] = silu_mul(s3[0] * d[0 * G + g], s3[1] * d[1 * G + g]);
                    hs[i + 1] = silu_mul(s3[0] * d[2 * G + g], s3[1] * d[3 * G + g]);
                }
            }
        }
        p->gu_left[size_t(grp)].fetch_sub(1, std::memory_order_release);
    }

    // down of one group on one output tile: per-slot partial dots
    void down(int tile, int grp) {
        const int H = L.H, I = L.I;
        while (p->gu_left[size_t(grp)].load(std::memory_order_acquire) != 0) _mm_pause();
        const uint8_t* b = block_of(grp);
        const int q0 = p->group_begin[size_t(grp)], q1 = p->group_begin[size_t(grp) + 1];
        const int o0 = tile * kDnOuts, o1 = std::min(H, o0 + kDnOuts);
        for (int o = o0; o < o1; o += 4) {
            const int R = std::min(4, o1 - o);
            RowSet rs;
            for (int k = 0; k < R; ++k) {
                rs.pay[k] = b + L.dn_p + size_t(o + k) * (I / 2);
                rs.scl[k] = b + L.dn_s + size_t(o + k) * (I / 16);
            }
            for (int q = q0; q < q1; q += kMaxG) {
                const int G = std::min(kMaxG, q1 - q);
                const float* hs[kMaxG];
                for (int g = 0; g < G; ++g) hs[g] = p->h.data() + size_t(p->order[size_t(q + g)].second) * I;
                float d[4 * kMaxG];
                kern[R - 1][G - 1](rs, hs, I, d);
                for (int g = 0; g < G; ++g) {
                    float* ps = p->part.data() + size_t(p->order[size_t(q + g)].second) * H;
                    for (int k = 0; k < R; ++k) ps[o + k] = d[k * G + g];
                }
            }
        }
        if (p->tile_left[size_t(tile)].fetch_sub(1, std::memory_order_acq_rel) == 1) reduce(tile);
    }

    // y[r][o] = sum over r's slots in slot order of (w s_down) * partial
    void reduce(int tile) {
        const int H = L.H;
        const int o0 = tile * kDnOuts, o1 = std::min(H, o0 + kDnOuts);
        for (int r = 0; r < rows; ++r) {
            float acc[kDnOuts] = {};
            for (int s = off[r]; s < off[r + 1]; ++s) {
                const float f = w[s] * reinterpret_cast<const float*>(blocks[s] + L.gsc)[2];
                const float* ps = p->part.data() + size_t(s) * H;
                for (int o = o0; o < o1; ++o) acc[o - o0] = std::fma(f, ps[o], acc[o - o0]);
            }
            std::memcpy(y + size_t(r) * H + o0, acc, sizeof(float) * size_t(o1 - o0));
        }
    }

    static void item(void* c, int i) {
        Ffn& f = *static_cast<Ffn*>(c);
        const int per = f.L.I / kGuRows;
        if (i < f.gu_items) f.gate_up(i / per, (i % per) * kGuRows);
        else {
            i -= f.gu_items;
            f.down(i / f.groups, i % f.groups);
        }
    }
};

int ffn_call(grim_cpu_experts* p, const grim_nv_expert_layout* L, int rows, const uint8_t* const* blocks,
             const float* w, const int32_t* off, const float* x, float* y) {
    const int H = L->H, I = L->I;
    const int S = off[rows];
    if (S == 0) {
        std::fill(y, y + size_t(rows) * H, 0.0f);
        return GRIM_OK;
    }
    // slots grouped by block: one sort of (block, slot), runs of equal blocks
    p->order.resize(size_t(S));
    p->slot_row.resize(size_t(S));
    for (int r = 0; r < rows; ++r)
        for (int s = off[r]; s < off[r + 1]; ++s) {
            p->slot_row[size_t(s)] = r;
            p->order[size_t(s)] = {reinterpret_cast<uintptr_t>(blocks[s]), s};
        }
    std::sort(p->order.begin(), p->order.end());
    p->group_begin.clear();
    for (int q = 0; q < S; ++q)
        if (q == 0 || p->order[size_t(q)].first != p->order[size_t(q) - 1].first) p->group_begin.push_back(q);
    const int groups = int(p->group_begin.size());
    p->group_begin.push_back(S);
    const int tiles = (H + kDnOuts - 1) / kDnOuts;
    const long items = long(groups) * (I / kGuRows) + long(groups) * tiles;
    if (items >= kMaxItems) return GRIM_ERR_SHAPE;
    p->h.resize(size_t(S) * I);
    p->part.resize(size_t(S) * H);
    p->grow_counters(size_t(groups), size_t(tiles));
    for (int g = 0; g < groups; ++g) p->gu_left[size_t(g)].store(I / kGuRows, std::memory_order_relaxed);
    for (int t = 0; t < tiles; ++t) p->tile_left[size_t(t)].store(groups, std::memory_order_relaxed);
    Ffn f{p, *L, blocks, w, off, rows, S, groups, groups * (I / kGuRows), tiles, x, y, rows_table()};
    p->run(int(items), &Ffn::item, &f);
    return GRIM_OK;
}

}  // namespace

extern "C" {

grim_cpu_experts* grimoire_cpu_experts_create(int threads, const int32_t* cpus, int ncpus) {
    if (threads <= 0) threads = std::max(1, int(std::thread::hardware_concurrency()) - 1);
    auto* p = new (std::nothrow) grim_cpu_experts();
    if (!p) return nullptr;
    p->nthreads = threads;
    for (int t = 1; t < threads; ++t) {
        const int cpu = (cpus && t < ncpus) ? int(cpus[t]) : -1;
        p->threads.emplace_back([p, cpu] { p->loop(cpu); });
    }
    return p;
}

void grimoire_cpu_experts_destroy(grim_cpu_experts* p) { delete p; }

int grimoire_cpu_experts_threads(const grim_cpu_experts* p) { return p ? p->nthreads : 0; }

double grimoire_cpu_experts_wait_us(const grim_cpu_experts* p) { return p ? p->wait_us : 0.0; }

float grimoire_cpu_nvfp4_dot(const uint8_t* pay, const uint8_t* scl, const float* x, int K) {
    if (K <= 0 || K % 64) return std::nanf("");
    RowSet rs{};
    rs.pay[0] = pay;
    rs.scl[0] = scl;
    float d;
    rows_table()[0][0](rs, &x, K, &d);
    return d;
}

int grimoire_cpu_set_isa(int isa) {
    const int best = best_isa();
    if (isa < 0) isa = best;
    if (isa > best) return GRIM_ERR_ARG;
    g_isa.store(isa);
    return GRIM_OK;
}

int grimoire_cpu_experts_ffn(grim_cpu_experts* p, const grim_nv_expert_layout* L,
                             const uint8_t* const* blocks, const float* w, int n, const float* x,
                             float* y) {
    if (!p || !x || !y || n < 0 || (n > 0 && (!blocks || !w))) return GRIM_ERR_ARG;
    if (int r = check_layout(L)) return r;
    const int32_t off[2] = {0, n};
    return ffn_call(p, L, 1, blocks, w, off, x, y);
}

int grimoire_cpu_experts_ffn_rows(grim_cpu_experts* p, const grim_nv_expert_layout* L, int rows,
                                  const uint8_t* const* blocks, const float* w, const int32_t* off,
                                  const float* x, float* y) {
    if (!p || rows < 0 || (rows > 0 && (!off || !x || !y))) return GRIM_ERR_ARG;
    if (int r = check_layout(L)) return r;
    if (rows == 0) return GRIM_OK;
    if (off[0] != 0) return GRIM_ERR_ARG;
    for (int r = 0; r < rows; ++r)
        if (off[r + 1] < off[r]) return GRIM_ERR_ARG;
    if (off[rows] > 0 && (!blocks || !w)) return GRIM_ERR_ARG;
    return ffn_call(p, L, rows, blocks, w, off, x, y);
}

int grimoire_cpu_pool_cpus(int ranks, int rank, int32_t* out, int cap) {
    if (ranks < 1 || rank < 0 || rank >= ranks || (cap > 0 && !out)) return GRIM_ERR_ARG;
    cpu_set_t s;
    if (sched_getaffinity(0, sizeof s, &s) != 0) return 0;
    const int n = CPU_COUNT(&s);
    // rank's share: positions [n rank / ranks, n (rank + 1) / ranks) of the allowed CPUs in order
    const long lo = long(n) * rank / ranks, hi = long(n) * (rank + 1) / ranks;
    int pos = 0, k = 0;
    for (int c = 0; c < CPU_SETSIZE && pos < hi; ++c) {
        if (!CPU_ISSET(c, &s)) continue;
        if (pos++ < lo) continue;
        if (k < cap) out[k] = c;
        ++k;
    }
    return k;
}

}  // extern "C"
