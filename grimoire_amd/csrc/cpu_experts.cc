// cpu_experts.cc -- NVFP4 routed experts computed by host threads.
//
// The CPU side of the tiered experts (src/cpu_experts.cpp:242-363,
// include/b70/cpu_experts.hpp): an expert block that lives in host memory
// is read by the host cores at DRAM speed instead of by the GPU over PCIe;
// the caller adds the host partial sum to the device one.  Same block
// layout as the GPU tiered kernels (grim_nv_expert_layout).
//
// Arithmetic (fp32, no activation quantisation): every weight is exact in
// fp32 -- an e2m1 code times two is an integer in [-12, 12], times half its
// block's E4M3 scale is the dequantised value with at most 6 significant
// bits.  A row dot product keeps 4 x 16 lane accumulators: block b of 16
// elements goes to accumulator b % 4, lane l takes element 16 b + l by one
// fma; the accumulators are added as (a0 + a1) + (a2 + a3) and the 16
// lanes by halving (l + 8, + 4, + 2, + 1).  The AVX-512, AVX2 and scalar
// paths all perform exactly these operations, so they give the same bits,
// and every output element is formed by one work item from start to end,
// so the result does not depend on the thread count.
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
#include <new>
#include <thread>
#include <vector>

namespace {

// ------------------------------------------------------------ formats

// e2m1 code -> 2x its value (an exact int8)
constexpr int8_t kE2m1x2[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

// E4M3 (OCP: no infinities, 0x7F / 0xFF NaN) -> fp32, times 0.5 (the other
// half of the e2m1 doubling)
float e4m3_half(uint8_t b) {
    const int s = b >> 7, e = (b >> 3) & 15, m = b & 7;
    float v;
    if (e == 15 && m == 7) v = std::nanf("");
    else if (e == 0) v = std::ldexp(float(m), -9);
    else v = std::ldexp(float(8 + m), e - 10);
    return 0.5f * (s ? -v : v);
}

struct ScaleTable {
    float v[256];
    ScaleTable() {
        for (int i = 0; i < 256; ++i) v[i] = e4m3_half(uint8_t(i));
    }
};
const float* scale_table() {
    static const ScaleTable t;
    return t.v;
}

// Lanes -> one float: (a0 + a1) + (a2 + a3) per lane, then halving.
float finish(const float (&a)[4][16]) {
    float v[16];
    for (int l = 0; l < 16; ++l) v[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
    for (int w = 8; w >= 1; w >>= 1)
        for (int l = 0; l < w; ++l) v[l] = v[l] + v[l + w];
    return v[0];
}

// ------------------------------------------------------------ dot paths

float dot_scalar(const uint8_t* pay, const uint8_t* scl, const float* x, int K) {
    const float* st = scale_table();
    float a[4][16] = {};
    for (int b = 0; b < K / 16; ++b) {
        const float hs = st[scl[b]];
        float* acc = a[b & 3];
        for (int l = 0; l < 16; ++l) {
            const uint8_t byte = pay[8 * b + (l >> 1)];
            const int code = (l & 1) ? byte >> 4 : byte & 15;
            const float w = float(kE2m1x2[code]) * hs;
            acc[l] = std::fma(w, x[16 * b + l], acc[l]);
        }
    }
    return finish(a);
}

// 64 elements (32 payload bytes) as four 16-byte blocks of int8 codes x 2
// in element order: bytes i of a 128-bit half hold elements 2i (low nibble)
// and 2i + 1 (high), so unpacking low / high nibbles per half gives
// [blocks 0 | 2] and [1 | 3].
__attribute__((target("avx2")))
inline void codes64(const uint8_t* p, __m128i (&blk)[4]) {
    const __m256i lut = _mm256_setr_epi8(0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12,
                                         0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12);
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    const __m256i v = _mm256_loadu_si256(reinterpret_cast<const __m256i*>(p));
    const __m256i lo = _mm256_shuffle_epi8(lut, _mm256_and_si256(v, m4));
    const __m256i hi = _mm256_shuffle_epi8(lut, _mm256_and_si256(_mm256_srli_epi16(v, 4), m4));
    const __m256i e0 = _mm256_unpacklo_epi8(lo, hi), e1 = _mm256_unpackhi_epi8(lo, hi);
    blk[0] = _mm256_castsi256_si128(e0);
    blk[1] = _mm256_castsi256_si128(e1);
    blk[2] = _mm256_extracti128_si256(e0, 1);
    blk[3] = _mm256_extracti128_si256(e1, 1);
}

__attribute__((target("avx2,fma")))
float dot_avx2(const uint8_t* pay, const uint8_t* scl, const float* x, int K) {
    const float* st = scale_table();
    __m256 lo[4], hi[4];
    for (int j = 0; j < 4; ++j) lo[j] = hi[j] = _mm256_setzero_ps();
    for (int k = 0; k < K; k += 64) {
        __m128i blk[4];
        codes64(pay + k / 2, blk);
        for (int j = 0; j < 4; ++j) {
            const __m256 hs = _mm256_set1_ps(st[scl[k / 16 + j]]);
            const __m256 w0 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(blk[j])), hs);
            const __m256 w1 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(blk[j], 8))), hs);
            lo[j] = _mm256_fmadd_ps(w0, _mm256_loadu_ps(x + k + 16 * j), lo[j]);
            hi[j] = _mm256_fmadd_ps(w1, _mm256_loadu_ps(x + k + 16 * j + 8), hi[j]);
        }
    }
    float a[4][16];
    for (int j = 0; j < 4; ++j) {
        _mm256_storeu_ps(a[j], lo[j]);
        _mm256_storeu_ps(a[j] + 8, hi[j]);
    }
    return finish(a);
}

__attribute__((target("avx512f,avx512bw,avx2,fma")))
float dot_avx512(const uint8_t* pay, const uint8_t* scl, const float* x, int K) {
    const float* st = scale_table();
    __m512 acc[4];
    for (int j = 0; j < 4; ++j) acc[j] = _mm512_setzero_ps();
    for (int k = 0; k < K; k += 64) {
        __m128i blk[4];
        codes64(pay + k / 2, blk);
        for (int j = 0; j < 4; ++j) {
            const __m512 w = _mm512_mul_ps(_mm512_cvtepi32_ps(_mm512_cvtepi8_epi32(blk[j])),
                                           _mm512_set1_ps(st[scl[k / 16 + j]]));
            acc[j] = _mm512_fmadd_ps(w, _mm512_loadu_ps(x + k + 16 * j), acc[j]);
        }
    }
    float a[4][16];
    for (int j = 0; j < 4; ++j) _mm512_storeu_ps(a[j], acc[j]);
    return finish(a);
}

using DotFn = float (*)(const uint8_t*, const uint8_t*, const float*, int);

int g_isa = -1;   // 0 scalar, 1 AVX2, 2 AVX-512; -1 = not chosen yet

int best_isa() {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw")) return 2;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return 1;
    return 0;
}

DotFn dot_fn() {
    if (g_isa < 0) g_isa = best_isa();
    return g_isa == 2 ? dot_avx512 : g_isa == 1 ? dot_avx2 : dot_scalar;
}

float silu_mul(float g, float u) { return g / (1.0f + std::exp(-g)) * u; }

}  // namespace

// ------------------------------------------------------------ pool
//
// Persistent workers wake on a new epoch, enter the job only while it is
// open (counted in `inside`, checked after entering), and claim work items
// from the job's own counter.  The caller works through items too, closes
// the job when none are left and waits only for the workers inside; a
// worker that is descheduled misses the job and nothing waits for it.

struct grim_cpu_experts {
    struct Job {
        void (*fn)(void*, int);
        void* ctx;
    };
    int nthreads = 1;
    std::vector<std::thread> workers;
    std::atomic<uint32_t> epoch{0};
    std::atomic<bool> open{false};
    std::atomic<int> inside{0};
    std::atomic<bool> quit{false};
    Job job{};
    double wait_us = 0.0;
    std::vector<float> h;                    // per-call scratch
    std::vector<const uint8_t*> uniq;        // ffn_rows: distinct blocks
    std::vector<int> slot_row, slot_uniq, uniq_off, uniq_slots;

    void worker(int tid, uint32_t seen, int cpu) {
        if (cpu >= 0) {
            cpu_set_t s;
            CPU_ZERO(&s);
            CPU_SET(cpu, &s);
            pthread_setaffinity_np(pthread_self(), sizeof s, &s);
        }
        for (;;) {
            uint32_t e = epoch.load(std::memory_order_acquire);
            for (int spin = 0; e == seen && spin < 20000; ++spin) {
                _mm_pause();
                e = epoch.load(std::memory_order_acquire);
            }
            if (e == seen) {
                if (quit.load()) return;
                epoch.wait(seen);
                continue;
            }
            seen = e;
            if (quit.load()) return;
            inside.fetch_add(1);
            if (open.load()) job.fn(job.ctx, tid);
            inside.fetch_sub(1);
        }
    }

    void run(void (*fn)(void*, int), void* ctx) {
        job = Job{fn, ctx};
        if (nthreads > 1) {
            open.store(true);
            epoch.fetch_add(1, std::memory_order_release);
            epoch.notify_all();
        }
        fn(ctx, 0);
        if (nthreads > 1) {
            open.store(false);
            const auto t0 = std::chrono::steady_clock::now();
            while (inside.load() != 0) _mm_pause();
            wait_us += std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
        }
    }

    // fn(i) for i in [0, n) over the pool, items claimed one at a time
    template <class F>
    void parallel(int n, F&& f) {
        struct Ctx {
            F* f;
            int n;
            std::atomic<int> next{0};
        } c{&f, n};
        run([](void* p, int) {
                Ctx& c = *static_cast<Ctx*>(p);
                for (int i; (i = c.next.fetch_add(1, std::memory_order_relaxed)) < c.n;) (*c.f)(i);
            },
            &c);
    }

    ~grim_cpu_experts() {
        quit.store(true);
        epoch.fetch_add(1);
        epoch.notify_all();
        for (auto& t : workers) t.join();
    }
};

namespace {

constexpr int kPairs = 16;    // pass 1 item: 16 (gate, up) row pairs of one expert
constexpr int kOuts = 32;     // pass 2 item: 32 outputs

int check_layout(const grim_nv_expert_layout* L) {
    if (!L || L->H <= 0 || L->I <= 0 || L->H % 128 || L->I % 128) return GRIM_ERR_SHAPE;
    return GRIM_OK;
}

}  // namespace

extern "C" {

grim_cpu_experts* grimoire_cpu_experts_create(int threads, const int32_t* cpus, int ncpus) {
    if (threads <= 0) threads = std::max(1, int(std::thread::hardware_concurrency()) - 1);
    auto* p = new (std::nothrow) grim_cpu_experts();
    if (!p) return nullptr;
    p->nthreads = threads;
    // the epoch every worker starts from is read here, before any job
    const uint32_t e0 = p->epoch.load();
    for (int t = 1; t < threads; ++t)
        p->workers.emplace_back(&grim_cpu_experts::worker, p, t, e0, (cpus && t < ncpus) ? int(cpus[t]) : -1);
    return p;
}

void grimoire_cpu_experts_destroy(grim_cpu_experts* p) { delete p; }

int grimoire_cpu_experts_threads(const grim_cpu_experts* p) { return p ? p->nthreads : 0; }

double grimoire_cpu_experts_wait_us(const grim_cpu_experts* p) { return p ? p->wait_us : 0.0; }

float grimoire_cpu_nvfp4_dot(const uint8_t* pay, const uint8_t* scl, const float* x, int K) {
    if (K <= 0 || K % 64) return std::nanf("");
    return dot_fn()(pay, scl, x, K);
}

int grimoire_cpu_set_isa(int isa) {
    const int best = best_isa();
    if (isa < 0) isa = best;
    if (isa > best) return GRIM_ERR_ARG;
    g_isa = isa;
    return GRIM_OK;
}

int grimoire_cpu_experts_ffn(grim_cpu_experts* p, const grim_nv_expert_layout* L,
                             const uint8_t* const* blocks, const float* w, int n, const float* x,
                             float* y) {
    if (!p || !x || !y || n < 0 || (n > 0 && (!blocks || !w))) return GRIM_ERR_ARG;
    if (int r = check_layout(L)) return r;
    const int H = L->H, I = L->I;
    if (n == 0) {
        std::fill(y, y + H, 0.0f);
        return GRIM_OK;
    }
    const DotFn dot = dot_fn();
    p->h.resize(size_t(n) * I);
    float* h = p->h.data();
    const grim_nv_expert_layout lay = *L;
    // pass 1: h[j][i] = silu(s_g gate_i . x) * (s_u up_i . x)
    p->parallel(n * (I / kPairs), [&](int c) {
        const int j = c / (I / kPairs), i0 = (c % (I / kPairs)) * kPairs;
        const uint8_t* b = blocks[j];
        const float* g3 = reinterpret_cast<const float*>(b + lay.gsc);
        for (int i = i0; i < i0 + kPairs; ++i) {
            const float g = g3[0] * dot(b + lay.gu_p + size_t(i) * (H / 2), b + lay.gu_s + size_t(i) * (H / 16), x, H);
            const float u = g3[1] * dot(b + lay.gu_p + size_t(I + i) * (H / 2),
                                        b + lay.gu_s + size_t(I + i) * (H / 16), x, H);
            h[size_t(j) * I + i] = silu_mul(g, u);
        }
    });
    // pass 2: y[o] = sum over j in order of (w_j s_d) (down_o . h_j)
    p->parallel((H + kOuts - 1) / kOuts, [&](int c) {
        const int o0 = c * kOuts, o1 = std::min(H, o0 + kOuts);
        for (int o = o0; o < o1; ++o) {
            float acc = 0.0f;
            for (int j = 0; j < n; ++j) {
                const uint8_t* b = blocks[j];
                const float f = w[j] * reinterpret_cast<const float*>(b + lay.gsc)[2];
                acc = std::fma(f, dot(b + lay.dn_p + size_t(o) * (I / 2), b + lay.dn_s + size_t(o) * (I / 16),
                                      h + size_t(j) * I, I),
                               acc);
            }
            y[o] = acc;
        }
    });
    return GRIM_OK;
}

int grimoire_cpu_experts_ffn_rows(grim_cpu_experts* p, const grim_nv_expert_layout* L, int rows,
                                  const uint8_t* const* blocks, const float* w, const int32_t* off,
                                  const float* x, float* y) {
    if (!p || rows < 0 || (rows > 0 && (!off || !x || !y))) return GRIM_ERR_ARG;
    if (int r = check_layout(L)) return r;
    if (rows == 0) return GRIM_OK;
    const int H = L->H, I = L->I;
    const int total = off[rows];
    if (off[0] != 0 || total < 0) return GRIM_ERR_ARG;
    for (int r = 0; r < rows; ++r)
        if (off[r + 1] < off[r]) return GRIM_ERR_ARG;
    if (total == 0) {
        std::fill(y, y + size_t(rows) * H, 0.0f);
        return GRIM_OK;
    }
    if (!blocks || !w) return GRIM_ERR_ARG;
    const DotFn dot = dot_fn();
    const grim_nv_expert_layout lay = *L;
    // distinct blocks, and each one's slots in slot order
    p->slot_row.resize(size_t(total));
    p->slot_uniq.resize(size_t(total));
    p->uniq.clear();
    for (int r = 0; r < rows; ++r)
        for (int s = off[r]; s < off[r + 1]; ++s) {
            p->slot_row[size_t(s)] = r;
            const auto it = std::find(p->uniq.begin(), p->uniq.end(), blocks[s]);
            p->slot_uniq[size_t(s)] = int(it - p->uniq.begin());
            if (it == p->uniq.end()) p->uniq.push_back(blocks[s]);
        }
    const int nu = int(p->uniq.size());
    p->uniq_off.assign(size_t(nu) + 1, 0);
    for (int s = 0; s < total; ++s) ++p->uniq_off[size_t(p->slot_uniq[size_t(s)]) + 1];
    for (int u = 0; u < nu; ++u) p->uniq_off[size_t(u) + 1] += p->uniq_off[size_t(u)];
    p->uniq_slots.resize(size_t(total));
    {
        std::vector<int> fill(p->uniq_off.begin(), p->uniq_off.end() - 1);
        for (int s = 0; s < total; ++s) p->uniq_slots[size_t(fill[size_t(p->slot_uniq[size_t(s)])]++)] = s;
    }
    p->h.resize(size_t(total) * I);
    float* h = p->h.data();
    const int* srow = p->slot_row.data();
    const int* uoff = p->uniq_off.data();
    const int* uslots = p->uniq_slots.data();
    const uint8_t* const* uniq = p->uniq.data();
    // pass 1 over distinct blocks: each gate / up row dotted with the input
    // of every slot that routes to the block while the row is in cache
    p->parallel(nu * (I / kPairs), [&](int c) {
        const int u = c / (I / kPairs), i0 = (c % (I / kPairs)) * kPairs;
        const uint8_t* b = uniq[u];
        const float* g3 = reinterpret_cast<const float*>(b + lay.gsc);
        for (int i = i0; i < i0 + kPairs; ++i)
            for (int q = uoff[u]; q < uoff[u + 1]; ++q) {
                const int s = uslots[q];
                const float* xr = x + size_t(srow[s]) * H;
                const float g = g3[0] * dot(b + lay.gu_p + size_t(i) * (H / 2), b + lay.gu_s + size_t(i) * (H / 16), xr, H);
                const float uu = g3[1] * dot(b + lay.gu_p + size_t(I + i) * (H / 2),
                                             b + lay.gu_s + size_t(I + i) * (H / 16), xr, H);
                h[size_t(s) * I + i] = silu_mul(g, uu);
            }
    });
    // pass 2: per row, grimoire_cpu_experts_ffn's sum in its order
    p->parallel((H + kOuts - 1) / kOuts, [&](int c) {
        const int o0 = c * kOuts, o1 = std::min(H, o0 + kOuts);
        for (int r = 0; r < rows; ++r)
            for (int o = o0; o < o1; ++o) {
                float acc = 0.0f;
                for (int s = off[r]; s < off[r + 1]; ++s) {
                    const uint8_t* b = blocks[s];
                    const float f = w[s] * reinterpret_cast<const float*>(b + lay.gsc)[2];
                    acc = std::fma(f, dot(b + lay.dn_p + size_t(o) * (I / 2), b + lay.dn_s + size_t(o) * (I / 16),
                                          h + size_t(s) * I, I),
                                   acc);
                }
                y[size_t(r) * H + o] = acc;
            }
    });
    return GRIM_OK;
}

int grimoire_cpu_pool_cpus(int ranks, int rank, int32_t* out, int cap) {
    if (ranks < 1 || rank < 0 || rank >= ranks || (cap > 0 && !out)) return GRIM_ERR_ARG;
    cpu_set_t s;
    if (sched_getaffinity(0, sizeof s, &s) != 0) return 0;
    std::vector<int> all;
    for (int c = 0; c < CPU_SETSIZE; ++c)
        if (CPU_ISSET(c, &s)) all.push_back(c);
    const size_t b = all.size() * size_t(rank) / size_t(ranks), e = all.size() * size_t(rank + 1) / size_t(ranks);
    int n = 0;
    for (size_t i = b; i < e; ++i, ++n)
        if (n < cap) out[n] = all[i];
    return n;
}

}  // extern "C"
