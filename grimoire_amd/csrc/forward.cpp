// forward.cpp -- grimoire_moe_forward: the whole MoE block of one layer.
//
// The engine's per-layer sequence (src/grimoire.cpp:15362-15500 decode,
// :22743-23300 prefill) behind one call, all on one stream, no host sync:
//
//   GEMV regime (decode, T*K small):
//     router GEMV -> top-k -> gate_up(+shared, +gate) -> down(+shared)
//   GEMM regime (prefill / verify):
//     router GEMM -> top-k -> dispatch (counts, scan, stable permutation,
//     bf16 rows) -> [shared gate] -> grouped gate_up+SwiGLU (MFMA, shared
//     expert as extra tiles) -> grouped down (MFMA, fp32 rows) -> combine
//     (slot-order fma chain + gate * shared)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <atomic>
#include <mutex>

#include "../../include/grimoire_moe.h"
#include "common.hpp"
#include "dispatch.hpp"
#include "gemm.hpp"
#include "gemm_i8.hpp"
#include "gemv_grouped.hpp"
#include "gemv_mx.hpp"
#include "gemv.hpp"
#include "router.hpp"

using namespace grim;

extern "C" int grimoire_moe_gate_up_shared(void*, const grim_moe_layer*, const grim_quant_weight*,
                                           const uint16_t*, const int32_t*, const float*, float*,
                                           float*);

namespace {

struct Carve {
    char* base;
    size_t off = 0;
    template <class T>
    T* take(size_t n) {
        off = (off + 255) & ~size_t(255);
        T* p = reinterpret_cast<T*>(base ? base + off : nullptr);
        off += n * sizeof(T);
        return p;
    }
};

// Poll bound of the one-launch decode, in real-time counter ticks; the
// default unless a test lowers it (grimoire_moe_debug_spin_ticks).
std::atomic<uint64_t> g_spin_ticks{kSpinTicksDefault};

__global__ void zero_words_kernel(uint32_t* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// The decode path with device-side routing covers up to this many tokens.
constexpr int kDecodeMaxTokens = 8;

bool gv_ok(const grim_moe_layer* L);

// MXFP4 experts that the matrix-core grouped GEMV takes: from 16 routes
// per call on, one stream per expert group beats the per-route decode
// kernels (C3: 8 tokens x top-4, 204 -> ~120 us measured).
bool prefer_grouped_mx(const grim_moe_layer* L, int T) {
    const int64_t R = int64_t(T) * L->cfg.top_k;
    return L->gate_up.fmt == GRIM_FMT_MXFP4 && R >= 16 && R <= 2 * int64_t(L->cfg.num_experts) &&
           gvm_shape_ok(L->cfg.hidden, L->cfg.inter) && gv_ok(L);
}

bool use_gemv(const grim_moe_layer* L, int T, int regime) {
    if (regime == 1 || regime == 3 || regime == 7) return true;
    if (regime == 2 || regime == 4 || regime == 5) return false;
    return int64_t(T) * L->cfg.top_k <= 64 && !prefer_grouped_mx(L, T);
}

static_assert(kSyncBytes == GRIM_SYNC_BYTES, "sync words of the header");

struct Plan {
    uint32_t* sync;   // fused decode: epoch-tagged words, zero before first use
    float* logits;
    int32_t* rex;
    float* rwt;
    int32_t* lrex;  // one shard's local routes (grimoire_moe_forward_shard)
    float* lrwt;
    float* gate;
    // GEMV
    float* h;
    uint32_t* hf;   // decode: h in the staged layout
    uint32_t* xf;   // decode: x formatted for the wave-centric gate_up
    float* hrep;    // fused decode: copies of h
    // GEMM
    float* logits2;   // the split-K router's second partial
    void* wimg;       // the split-K router's W limb image
    void* disp_ws;
    int32_t *counts, *offsets, *inverse, *tile_e, *tile_mb;
    int tmax;
    uint16_t *xperm, *xrow, *hp, *hp_sh;
    float *yperm, *ysh;
    // INT8 weights: activation limbs for the int8 MFMA
    int8_t *xq, *xrowq, *hq, *hshq;
    float *sx, *sxrow, *sh, *shsh, *h32, *h32sh;
    int32_t* qperm;   // token of every routed row (the gate_up GEMM's gather map)
    // expert-grouped GEMV (gemv_grouped.hip): its own tile table (MT-row
    // blocks), the route -> token map and fp32 h rows
    int32_t *gv_te, *gv_tm, *gv_perm;
    int gv_tmax;
    float *gv_h, *gv_hsh;
    uint32_t *gv_xf, *gv_hf, *gv_hfsh;   // formatted activation rows
};

// MXFP4 rows of the matrix-core grouped GEMV's length (gvm_padded_k):
// payload K'/2, K'/32 scale bytes per row, K' = gvm_padded_k(K) >= K.
static bool mx_rows_kp(const grim_quant_weight& w, int K) {
    const int kp = gvm_padded_k(K);
    return w.fmt == GRIM_FMT_MXFP4 && w.row_bytes == int64_t(kp / 2) && w.row_scales == kp / 32;
}

// ... and longer than K: padded rows.
static bool mx_padded(const grim_quant_weight& w, int K) {
    return gvm_padded_k(K) != K && mx_rows_kp(w, K);
}

// Some weight of the layer holds padded MXFP4 rows: of the grouped GEMVs
// only the matrix-core one reads them (as rows of K' elements).
static bool layer_mx_padded(const grim_moe_layer* L) {
    const int H = L->cfg.hidden, I = L->cfg.inter;
    return mx_padded(L->gate_up, H) || mx_padded(L->down, I) ||
           (L->has_shared && (mx_padded(L->shared_gate_up, H) || mx_padded(L->shared_down, I)));
}

// The expert-grouped GEMV covers these shapes and formats.
bool gv_ok(const grim_moe_layer* L) {
    const int f = L->gate_up.fmt;
    const int H = L->cfg.hidden, I = L->cfg.inter;
    // payload rows packed (K / 2 bytes): a sub-block's rows are one span
    // (or MXFP4 rows padded for the matrix-core kernel, all alike)
    const bool pad = layer_mx_padded(L);
    auto packed = [pad](const grim_quant_weight& w, int K) {
        if (pad) return mx_rows_kp(w, K);   // (K' = K where K is whole stages already)
        // INT4 scale groups of >= 32 elements: at most K / 16 scale bytes per row
        return w.row_bytes == int64_t(K / 2) && int64_t(w.row_scales) * 32 <= K;
    };
    return f == L->down.fmt && gv_shape_ok(f, H, I) && packed(L->gate_up, H) && packed(L->down, I) &&
           (!L->has_shared || (L->shared_gate_up.fmt == f && L->shared_down.fmt == f &&
                               packed(L->shared_gate_up, H) && packed(L->shared_down, I))) &&
           (!pad || gvm_shape_ok(H, I));
}

size_t carve(const grim_moe_layer* L, int T, bool gemv, char* base, Plan& p) {
    const auto& c = L->cfg;
    const int E = c.num_experts, K = c.top_k, H = c.hidden, I = c.inter;
    const int64_t R = int64_t(T) * K;
    const bool sh = L->has_shared;
    Carve cv{base};
    // every plan keeps the fused decode's sync words at the head, so no
    // other regime's data ever lands on them
    p.sync = cv.take<uint32_t>(kSyncBytes / 4);
    p.logits = cv.take<float>(size_t(T) * E);
    p.rex = cv.take<int32_t>(R);
    p.rwt = cv.take<float>(R);
    p.lrex = cv.take<int32_t>(R);
    p.lrwt = cv.take<float>(R);
    p.gate = cv.take<float>(T);
    if (gemv) {
        p.h = cv.take<float>(size_t(T) * (K + (sh ? 1 : 0)) * I);
        p.hf = cv.take<uint32_t>(size_t(T) * fmt_words((K + (sh ? 1 : 0)) * I));
        p.xf = cv.take<uint32_t>(size_t(T) * xf_words(H));
        p.hrep = T == 1 ? cv.take<float>(size_t(kSyncCopies) * fused_h_stride(K, I)) : nullptr;
    } else {
        const size_t dws = dispatch_workspace_bytes(T, K, E);
        p.disp_ws = cv.take<char>(dws);
        p.logits2 = cv.take<float>(size_t(T) * E);
        const size_t wib = router_wimg_bytes(T, E, H);
        p.wimg = wib ? static_cast<void*>(cv.take<char>(wib)) : nullptr;
        p.counts = cv.take<int32_t>(E);
        p.offsets = cv.take<int32_t>(E);
        p.inverse = cv.take<int32_t>(R);
        p.tmax = int(E + (R + kGemmBM - 1) / kGemmBM);
        p.tile_e = cv.take<int32_t>(p.tmax + 4);
        p.tile_mb = cv.take<int32_t>(p.tmax);
        p.xperm = cv.take<uint16_t>(R * H);
        p.xrow = sh ? cv.take<uint16_t>(size_t(T) * H) : nullptr;
        p.hp = cv.take<uint16_t>(R * 2 * I);
        p.hp_sh = sh ? cv.take<uint16_t>(size_t(T) * 2 * I) : nullptr;
        p.yperm = cv.take<float>(R * H);
        p.ysh = sh ? cv.take<float>(size_t(T) * H) : nullptr;
        if (gv_ok(L)) {
            p.gv_tmax = int(E + (R + kGvMT - 1) / kGvMT);
            p.gv_te = cv.take<int32_t>(p.gv_tmax + 4);
            p.gv_tm = cv.take<int32_t>(p.gv_tmax);
            p.gv_perm = cv.take<int32_t>(R);
            p.gv_h = cv.take<float>(R * I);
            p.gv_hsh = sh ? cv.take<float>(size_t(T) * I) : nullptr;
            // formatted activation rows: either kernel's format fits
            const size_t ax = std::max(gv_act_bytes(H), gvm_act_bytes(H)) / 4;
            const size_t ai = std::max(gv_act_bytes(I), gvm_act_bytes(I)) / 4;
            p.gv_xf = cv.take<uint32_t>(size_t(T) * ax);
            p.gv_hf = cv.take<uint32_t>(R * ai);
            p.gv_hfsh = sh ? cv.take<uint32_t>(size_t(T) * ai) : nullptr;
        }
        if (L->gate_up.fmt == GRIM_FMT_INT8 && L->down.fmt == GRIM_FMT_INT8) {
            p.xq = cv.take<int8_t>(R * 2 * H);
            p.sx = cv.take<float>(R);
            p.h32 = cv.take<float>(R * I);
            p.hq = cv.take<int8_t>(R * 2 * I);
            p.sh = cv.take<float>(R);
            p.xrowq = cv.take<int8_t>(size_t(T) * 2 * H);
            p.sxrow = cv.take<float>(T);
            p.qperm = cv.take<int32_t>(R);
            if (sh) {
                p.h32sh = cv.take<float>(size_t(T) * I);
                p.hshq = cv.take<int8_t>(size_t(T) * 2 * I);
                p.shsh = cv.take<float>(T);
            }
        }
    }
    return cv.off + 256;
}

}  // namespace

extern "C" size_t grimoire_moe_forward_workspace_bytes(const grim_moe_layer* L, int tokens) {
    if (!L || tokens <= 0) return 0;
    Plan p{};
    const size_t a = carve(L, tokens, true, nullptr, p);
    const size_t b = carve(L, tokens, false, nullptr, p);
    return a > b ? a : b;
}

extern "C" int grimoire_moe_router_logits(void*, const float*, const float*, float*, int, int, int);
extern "C" int grimoire_moe_router_topk_batched(void*, const float*, int, int, int, int32_t*,
                                                float*, int);
extern "C" int grimoire_moe_router_topk_sigmoid(void*, const float*, const uint16_t*, int, int,
                                                int, int32_t*, float*, int, float);
extern "C" int grimoire_moe_router_topk_group(void*, const float*, const float*, int, int, int,
                                              int, int, int32_t*, float*, int, float);
extern "C" int grimoire_moe_shared_rows(void*, const grim_moe_layer*, const grim_quant_weight*,
                                        const grim_quant_weight*, const uint16_t*, const int32_t*,
                                        const float*, const float*, float*, float*, float*, int);
extern "C" int grimoire_moe_gate_up_batched(void*, const grim_moe_layer*, const int32_t*,
                                            const float*, float*, int);
extern "C" int grimoire_moe_down_batched(void*, const grim_moe_layer*, const int32_t*,
                                         const float*, const float*, float*, int);
extern "C" int grimoire_moe_route_grouped(void*, const float*, const int32_t*, uint16_t*,
                                          uint16_t*, int32_t*, int32_t*, int32_t*, int32_t*,
                                          int32_t*, int, int, int, int, int, int, int32_t*, void*,
                                          size_t);
extern "C" const char* grimoire_moe_last_error(void);

static int ferr(int code, const char* msg);

#ifdef GRIM_TIMING
static unsigned long long* g_timing = nullptr;
extern "C" __attribute__((visibility("default"))) void grim_timing_set(void* p) {
    g_timing = static_cast<unsigned long long*>(p);
}
#endif

// GEMM regime for INT8 weights: the activations go to the int8 MFMA as
// two limbs per row (gemm_i8.hip): routes -> limbs of x (once per token,
// gathered by the GEMM through the route -> token map; at every permuted
// row when K is too short for the gather) -> gate_up + SwiGLU (h fp32) ->
// limbs of h -> down -> combine.
static int forward_gemm_i8(hipStream_t st, const grim_moe_layer* L, const Plan& p, const float* x,
                           float* y, int tokens, const uint16_t* shared_gate_w) {
    const auto& c = L->cfg;
    const int E = c.num_experts, K = c.top_k, H = c.hidden, I = c.inter;
    const bool sh = L->has_shared;
    const int64_t R = int64_t(tokens) * K;
    // rows mode (E <= kI8MaxListExperts): the GEMM lists its tiles from the
    // counts itself, so the dispatch forms no tile table
    const bool rows_mode = E <= kI8MaxListExperts;
    int r = grimoire_moe_route_grouped(st, x, p.rex, nullptr, nullptr, p.counts, p.offsets,
                                       p.inverse, rows_mode ? nullptr : p.tile_e,
                                       rows_mode ? nullptr : p.tile_mb, p.tmax, tokens, H, E,
                                       kGemmBM, K, nullptr, p.disp_ws,
                                       dispatch_workspace_bytes(tokens, K, E));
    if (r) return r;
    // gather mode: x limbs once per token, the gate_up GEMM reads each
    // routed row's token row through qperm; otherwise limbs at every
    // routed row
    const bool gather = gemm_i8_gather_ok(H, tokens) && E <= kI8MaxListExperts;
    // the shared expert's gate from the same loads of x when its weights
    // are 16-byte aligned
    const bool gate_fused = sh && shared_gate_w && (reinterpret_cast<uintptr_t>(shared_gate_w) & 15) == 0;
    hipError_t e = quant_permute_launch(st, x, tokens, H, K, p.inverse, gather ? nullptr : p.xq, p.sx,
                                        (sh || gather) ? p.xrowq : nullptr,
                                        (sh || gather) ? p.sxrow : nullptr, gather ? p.qperm : nullptr,
                                        gate_fused ? shared_gate_w : nullptr, gate_fused ? p.gate : nullptr);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    if (sh && shared_gate_w && !gate_fused) {
        e = rowdot_sigmoid_launch(st, x, shared_gate_w, p.gate, tokens, H);
        if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    }
    GemmI8Args g{};
    g.w = L->gate_up.payload;
    g.ws = static_cast<const float*>(L->gate_up.scales);
    g.row_bytes = L->gate_up.row_bytes;
    if (sh) {
        g.w_sh = L->shared_gate_up.payload;
        g.ws_sh = static_cast<const float*>(L->shared_gate_up.scales);
        g.row_bytes_sh = L->shared_gate_up.row_bytes;
    }
    g.N = 2 * I;
    g.K = H;
    g.I = I;
    g.swiglu = 1;
    g.A = gather ? p.xrowq : p.xq;
    g.sa = p.sx;
    g.gather = gather ? p.qperm : nullptr;
    g.gather_rows = tokens;
    g.A_sh = p.xrowq;
    g.sa_sh = p.sxrow;
    g.out = p.h32;
    g.out_sh = p.h32sh;
    g.offsets = p.offsets;
    g.counts = p.counts;
    g.tile_e = p.tile_e;
    g.tile_mb = p.tile_mb;
    g.tmax = p.tmax;
    g.n_tiles_dev = dispatch_live_tiles(p.disp_ws, tokens, K, E);
    g.T_sh = sh ? tokens : 0;
    // experts with few rows on 32-row tiles (tile lists formed in the kernels)
    if (rows_mode) {
        g.split = kI8DefaultSplit;
        g.num_experts = E;
    }
#ifdef GRIM_TIMING
    g.ts = g_timing;
#endif
    e = gemm_i8_launch(st, g);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    // h limbs (rows beyond the routed count are never read)
    e = quant_rows_launch(st, p.h32, int(R), I, p.hq, p.sh, sh ? p.h32sh : nullptr, sh ? tokens : 0,
                          p.hshq, p.shsh);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    GemmI8Args d = g;
    d.w = L->down.payload;
    d.ws = static_cast<const float*>(L->down.scales);
    d.row_bytes = L->down.row_bytes;
    if (sh) {
        d.w_sh = L->shared_down.payload;
        d.ws_sh = static_cast<const float*>(L->shared_down.scales);
        d.row_bytes_sh = L->shared_down.row_bytes;
    }
    d.N = H;
    d.K = I;
    d.I = 0;
    d.swiglu = 0;
    d.A = p.hq;
    d.sa = p.sh;
    d.gather = nullptr;
#ifdef GRIM_TIMING
    d.ts = g_timing ? g_timing + 256 * 128 * 2 : nullptr;
#endif
    d.A_sh = p.hshq;
    d.sa_sh = p.shsh;
    d.out = p.yperm;
    d.out_sh = p.ysh;
    e = gemm_i8_launch(st, d);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    CombineArgs cb{p.yperm, 0, p.inverse, p.rwt, p.ysh, 0, (sh && shared_gate_w) ? p.gate : nullptr,
                   y, tokens, K, H};
    e = combine_launch(st, cb);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    return GRIM_OK;
}

// Expert-grouped GEMV regime (few rows per expert): routes -> counts,
// offsets and an (expert, MT-row block) table -> [shared gate] -> gate_up
// + SwiGLU per group (fp32 h per route) -> down per group (fp32 rows per
// route) -> combine (slot-order fma chain + gate * shared).
static int forward_gv(hipStream_t st, const grim_moe_layer* L, const Plan& p, const float* x,
                      float* y, int tokens, const uint16_t* shared_gate_w, bool mx, const TopkArgs* route) {
    const auto& c = L->cfg;
    const int E = c.num_experts, K = c.top_k, H = c.hidden, I = c.inter;
    const bool sh = L->has_shared;
    if (route) {
        // top-k, dispatch and the x limbs in one launch (small batches)
        GvmRouteArgs ra{p.counts, p.offsets, p.gv_te, p.gv_tm, p.gv_tmax,
                        dispatch_live_tiles(p.disp_ws, tokens, K, E), p.inverse, p.gv_perm, x,
                        reinterpret_cast<uint8_t*>(p.gv_xf), H};
        hipError_t e = gvm_route_launch(st, *route, ra);
        if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    } else {
        int r = grimoire_moe_route_grouped(st, x, p.rex, nullptr, nullptr, p.counts, p.offsets,
                                           p.inverse, p.gv_te, p.gv_tm, p.gv_tmax, tokens, H, E, kGvMT,
                                           K, p.gv_perm, p.disp_ws,
                                           dispatch_workspace_bytes(tokens, K, E));
        if (r) return r;
    }
    if (sh && shared_gate_w) {
        hipError_t e = rowdot_sigmoid_launch(st, x, shared_gate_w, p.gate, tokens, H);
        if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    }
    if (!route) {
        // (the limb format of the matrix-core kernel is smaller than the
        // vector-ALU format the buffers are sized for)
        hipError_t e = mx ? gvm_format_launch(st, x, tokens, reinterpret_cast<uint8_t*>(p.gv_xf), nullptr, 0,
                                              nullptr, H)
                          : gv_format_launch(st, L->gate_up.fmt, x, tokens, p.gv_xf, nullptr, 0, nullptr, H);
        if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    }
    GvArgs g{};
    g.w = make_view(L->gate_up);
    g.af = p.gv_xf;
    g.af_sh = p.gv_xf;
    g.w_sh = sh ? make_view(L->shared_gate_up) : g.w;
    // padded MXFP4 rows: the weights' K' (the activation rows are formatted
    // for K and padded with zeros to the same K')
    const bool pad = mx && layer_mx_padded(L);
    g.N = I;
    g.K = pad ? gvm_padded_k(H) : H;
    g.x = x;
    g.perm_token = p.gv_perm;
    g.h = p.gv_h;
    g.h_sh = p.gv_hsh;
    g.counts = p.counts;
    g.offsets = p.offsets;
    g.tile_e = p.gv_te;
    g.tile_mb = p.gv_tm;
    g.n_live = dispatch_live_tiles(p.disp_ws, tokens, K, E);
    g.T_sh = sh ? tokens : 0;
#ifdef GRIM_TIMING
    g.ts = g_timing;
#endif
    if (mx) {
        // the matrix-core gate_up writes h in the down's limb format itself
        g.hf = reinterpret_cast<uint8_t*>(p.gv_hf);
        g.hf_sh = reinterpret_cast<uint8_t*>(p.gv_hfsh);
    }
    hipError_t e = mx ? gvm_launch(st, g, true) : gv_launch(st, L->gate_up.fmt, g, true);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    if (!mx) {
        e = gv_format_launch(st, L->down.fmt, p.gv_h, tokens * K, p.gv_hf, p.gv_hsh, sh ? tokens : 0, p.gv_hfsh, I);
        if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    }
    g.hf = g.hf_sh = nullptr;
    GvArgs d = g;
    d.af = p.gv_hf;
    d.af_sh = p.gv_hfsh;
    d.w = make_view(L->down);
    d.w_sh = sh ? make_view(L->shared_down) : d.w;
    d.N = H;
    d.K = pad ? gvm_padded_k(I) : I;
    d.y = p.yperm;
    d.y_sh = p.ysh;
#ifdef GRIM_TIMING
    d.ts = g_timing ? g_timing + 4096 * 16 : nullptr;
#endif
    e = mx ? gvm_launch(st, d, false) : gv_launch(st, L->down.fmt, d, false);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    CombineArgs cb{p.yperm, 0, p.inverse, p.rwt, p.ysh, 0, (sh && shared_gate_w) ? p.gate : nullptr,
                   y, tokens, K, H};
    e = combine_launch(st, cb);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    return GRIM_OK;
}

static int forward_impl(void* stream, const grim_moe_layer* L, const grim_route_params* rp,
                        const uint16_t* shared_gate_w, const float* x, float* y, int tokens,
                        int32_t* out_expert, float* out_weight, int regime, void* workspace,
                        size_t workspace_bytes, int roles, int shard_begin = 0, int shard_count = 0);

extern "C" int grimoire_moe_forward(void* stream, const grim_moe_layer* L,
                                    const grim_route_params* rp, const uint16_t* shared_gate_w,
                                    const float* x, float* y, int tokens, int32_t* out_expert,
                                    float* out_weight, int regime, void* workspace,
                                    size_t workspace_bytes) {
    return forward_impl(stream, L, rp, shared_gate_w, x, y, tokens, out_expert, out_weight, regime,
                        workspace, workspace_bytes, kRoleRouter | kRoleGateUp | kRoleDown);
}

// ---- the one-launch decode's sync words: status and reset
//
// workspace == NULL addresses the current device's array of
// grimoire_moe_forward_noalloc.

static int sync_words(void* workspace, size_t bytes, uint32_t** out);

extern "C" int grimoire_moe_decode_sync_status(void* stream, const void* workspace, size_t workspace_bytes,
                                               int* status) {
    if (!status) return ferr(GRIM_ERR_ARG, "decode_sync_status: null status");
    uint32_t* w = nullptr;
    if (int r = sync_words(const_cast<void*>(workspace), workspace_bytes, &w)) return r;
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint32_t v = 0;
    hipError_t e = hipMemcpyAsync(&v, w + 1, sizeof v, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    *status = v ? 1 : 0;
    return GRIM_OK;
}

extern "C" int grimoire_moe_decode_sync_reset(void* stream, void* workspace, size_t workspace_bytes) {
    uint32_t* w = nullptr;
    if (int r = sync_words(workspace, workspace_bytes, &w)) return r;
    const int n = int(kSyncBytes / 4);
    zero_words_kernel<<<(n + 1023) / 1024, 256, 0, static_cast<hipStream_t>(stream)>>>(w, n);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    return GRIM_OK;
}

extern "C" uint64_t grimoire_moe_debug_spin_ticks(int64_t ticks) {
    return g_spin_ticks.exchange(ticks < 0 ? kSpinTicksDefault : uint64_t(ticks));
}

// ---- the allocation-free variant
//
// Its workspace is one file-scope device array per GPU (the module's copy
// on each device), addressed through the pointer hipGetSymbolAddress gives
// for that device: the array's name is a host-side stand-in and is never
// passed to a kernel.  Every call on a GPU shares that GPU's array and
// finds the previous call's contents in it.  The forward writes every word
// it reads except the fused decode's sync words at the head of the
// workspace, which start zero (the array is zero-initialised storage) and
// which every call leaves consistent, so nothing is cleared.  Calls that
// overlap on one GPU race.
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// The current device's address of `scratch`, looked up on the first call
// on that device (with it current) and kept.
int scratch_ptr(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return int(e);
    if (dev < 0 || dev >= kMaxDevices) return GRIM_ERR_ARG;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return e != hipSuccess ? int(e) : GRIM_ERR_WORKSPACE;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return GRIM_OK;
}
}  // namespace

static int sync_words(void* workspace, size_t bytes, uint32_t** out) {
    if (workspace) {
        if (bytes < kSyncBytes) return ferr(GRIM_ERR_WORKSPACE, "workspace smaller than its sync words");
        *out = static_cast<uint32_t*>(workspace);
        return GRIM_OK;
    }
    void* ws = nullptr;
    if (int r = scratch_ptr(&ws)) return ferr(r, "no device address for the scratch array");
    *out = static_cast<uint32_t*>(ws);
    return GRIM_OK;
}

extern "C" size_t grimoire_moe_forward_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int grimoire_moe_forward_noalloc(void* stream, const grim_moe_layer* L,
                                            const grim_route_params* rp,
                                            const uint16_t* shared_gate_w, const float* x, float* y,
                                            int tokens, int32_t* out_expert, float* out_weight,
                                            int regime) {
    if (!L || !x || !y) return ferr(GRIM_ERR_ARG, "null layer/x/y");
    if (tokens <= 0) return GRIM_OK;
    Plan p{};
    const size_t need = carve(L, tokens, use_gemv(L, tokens, regime), nullptr, p);
    if (need > kNoAllocScratchBytes) {
        static thread_local char msg[160];
        std::snprintf(msg, sizeof msg,
                      "forward_noalloc: this call needs %zu bytes of workspace, above the %zu-byte "
                      "scratch limit (use grimoire_moe_forward with a workspace)",
                      need, kNoAllocScratchBytes);
        return ferr(GRIM_ERR_WORKSPACE, msg);
    }
    void* ws = nullptr;
    const int r = scratch_ptr(&ws);
    if (r) return ferr(r, "forward_noalloc: no device address for the scratch array");
    return forward_impl(stream, L, rp, shared_gate_w, x, y, tokens, out_expert, out_weight, regime,
                        ws, kNoAllocScratchBytes, kRoleRouter | kRoleGateUp | kRoleDown);
}

extern "C" int grimoire_moe_forward_shard(void* stream, const grim_moe_layer* L, const grim_route_params* rp,
                                          const uint16_t* shared_gate_w, const float* x, float* y, int tokens,
                                          int32_t* out_expert, float* out_weight, int regime, int expert_begin,
                                          int expert_count, void* workspace, size_t workspace_bytes) {
    if (expert_count <= 0) return ferr(GRIM_ERR_ARG, "expert_count must be > 0");
    if (regime == 1 || regime == 7) regime = 3;   // the in-kernel top-k decode has no shard form
    return forward_impl(stream, L, rp, shared_gate_w, x, y, tokens, out_expert, out_weight, regime,
                        workspace, workspace_bytes, kRoleRouter | kRoleGateUp | kRoleDown, expert_begin,
                        expert_count);
}

extern "C" int grimoire_moe_decode_stage(void* stream, const grim_moe_layer* L,
                                         const grim_route_params* rp,
                                         const uint16_t* shared_gate_w, const float* x, float* y,
                                         int tokens, int stage, void* workspace,
                                         size_t workspace_bytes) {
    if (stage != kRoleRouter && stage != kRoleGateUp && stage != kRoleDown)
        return ferr(GRIM_ERR_ARG, "stage: 1 router, 2 gate_up, 4 down");
    if (!L || tokens <= 0 || !use_gemv(L, tokens, 1) || tokens > kDecodeMaxTokens)
        return ferr(GRIM_ERR_SHAPE, "decode stages cover the single-launch-per-stage decode only");
    return forward_impl(stream, L, rp, shared_gate_w, x, y, tokens, nullptr, nullptr, 1, workspace,
                        workspace_bytes, stage);
}

static int forward_impl(void* stream, const grim_moe_layer* L, const grim_route_params* rp,
                        const uint16_t* shared_gate_w, const float* x, float* y, int tokens,
                        int32_t* out_expert, float* out_weight, int regime, void* workspace,
                        size_t workspace_bytes, int roles, int shard_begin, int shard_count) {
    if (!L || !x || !y) return ferr(GRIM_ERR_ARG, "null layer/x/y");
    if (tokens <= 0) return GRIM_OK;
    if (!L->router) return ferr(GRIM_ERR_ARG, "layer has no router");
    const auto& c = L->cfg;
    if (L->has_shared && c.shared_inter != c.inter)
        return ferr(GRIM_ERR_SHAPE, "shared_inter must equal inter");
    const bool gemv = use_gemv(L, tokens, regime);
    Plan p{};
    const size_t need = carve(L, tokens, gemv, nullptr, p);
    if (!workspace || workspace_bytes < need) return ferr(GRIM_ERR_WORKSPACE, "workspace too small");
    carve(L, tokens, gemv, static_cast<char*>(workspace), p);
    if (out_expert) p.rex = out_expert;
    if (out_weight) p.rwt = out_weight;
    hipStream_t st = static_cast<hipStream_t>(stream);

    int E = c.num_experts;
    const int K = c.top_k, H = c.hidden, I = c.inter;
    const bool shard = shard_count > 0;
    if (shard && (shard_begin < 0 || int64_t(shard_begin) + shard_count > E))
        return ferr(GRIM_ERR_ARG, "expert shard outside [0, num_experts)");
    const int mode = rp ? rp->mode : GRIM_ROUTE_SOFTMAX;
    if (H % 4) return ferr(GRIM_ERR_SHAPE, "hidden must be a multiple of 4");
    if (mode < GRIM_ROUTE_SOFTMAX || mode > GRIM_ROUTE_GROUP) return ferr(GRIM_ERR_ARG, "unknown route mode");
    if (mode == GRIM_ROUTE_GROUP &&
        (!rp || rp->n_group <= 0 || rp->n_group > 64 || E % rp->n_group || rp->topk_group <= 0 ||
         rp->topk_group > rp->n_group || K > rp->topk_group * (E / rp->n_group)))
        return ferr(GRIM_ERR_SHAPE, "group-limited routing parameters");
    if (E > 512 || K > 16 || K > E) return ferr(GRIM_ERR_SHAPE, "E <= 512 and top_k <= min(16, E)");
    const float* rbias = (mode == GRIM_ROUTE_SOFTMAX && rp) ? static_cast<const float*>(rp->bias) : nullptr;
    const int topk_mode = mode == GRIM_ROUTE_SOFTMAX ? 0 : (mode == GRIM_ROUTE_SIGMOID ? 2 : 3);
    const uint16_t* b16 = mode == GRIM_ROUTE_SIGMOID ? static_cast<const uint16_t*>(rp->bias) : nullptr;
    const float* b32 = mode == GRIM_ROUTE_GROUP ? static_cast<const float*>(rp->bias) : nullptr;
    const float scaling = (rp && mode != GRIM_ROUTE_SOFTMAX) ? rp->scaling : 1.0f;
    const bool sh = L->has_shared;

    if (gemv && regime != 3 && tokens <= kDecodeMaxTokens && !shard) {
        // three launches: router GEMV, gate_up (each item runs its token's
        // top-k; h written in the staged layout), down
        if (sh && (L->shared_gate_up.fmt != L->gate_up.fmt || L->shared_down.fmt != L->down.fmt))
            return ferr(GRIM_ERR_FORMAT, "shared expert format must match routed experts");
        DecodeArgs a{};
        a.gu = make_view(L->gate_up);
        a.dn = make_view(L->down);
        a.sgu = sh ? make_view(L->shared_gate_up) : a.gu;
        a.sdn = sh ? make_view(L->shared_down) : a.dn;
        a.shared = sh;
        a.router = L->router;
        a.rbias = rbias;
        a.mode = topk_mode;
        a.normalize = c.norm_topk;
        a.scaling = scaling;
        a.bias16 = b16;
        a.bias32 = b32;
        a.n_group = rp ? rp->n_group : 0;
        a.topk_group = rp ? rp->topk_group : 0;
        a.logits = p.logits;
        a.x = x;
        a.rex = p.rex;
        a.rwt = p.rwt;
        a.gate_w = sh ? shared_gate_w : nullptr;
        a.gate = p.gate;
        a.gate_in = (sh && shared_gate_w) ? p.gate : nullptr;
        a.h = p.h;
        a.hf = p.hf;
        a.y = y;
        a.H = H;
        a.I = I;
        a.K = K;
        a.E = E;
        a.M = tokens;
        a.fmt_h = 1;
        a.route_topk = 1;
#ifdef GRIM_TIMING
        a.ts = g_timing;
#endif
        if (L->gate_up.fmt != L->down.fmt) {
            // two formats: the roles need one kernel instantiation each
            return ferr(GRIM_ERR_FORMAT, "decode needs gate_up and down in one format");
        }
        {
            const int f = L->gate_up.fmt;
            const bool wave_fmt = f == GRIM_FMT_INT4 || f == GRIM_FMT_INT4_F16 || f == GRIM_FMT_MXFP4;
            // formatting runs in the router launch: a quad of threads per
            // chunk, at most 64 chunks per router work-group
            const int chunks = tokens * (H / 32);
            if (wave_fmt && H % 32 == 0 && H <= 8192 && I % 8 == 0 && (chunks + E - 1) / E <= 64) {
                a.xf = p.xf;
                a.xf_words = xf_words(H);
            }
        }
        decode_plan(L->gate_up.fmt, a, roles);
        // one token through all three roles: the one-launch kernel
        a.sync = p.sync;
        a.hrep = p.hrep;
        a.spin_ticks = g_spin_ticks.load(std::memory_order_relaxed);
        if (roles == (kRoleRouter | kRoleGateUp | kRoleDown) && regime == 7 &&
            decode_plan_fused(L->gate_up.fmt, a)) {
            hipError_t e = decode_launch(st, L->gate_up.fmt, a);
            if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
            return GRIM_OK;
        }
        if (decode_lds_bytes(L->gate_up.fmt, a) > 160 * 1024)
            return ferr(GRIM_ERR_SHAPE, "layer too large for the decode kernels");
        hipError_t e = decode_launch(st, L->gate_up.fmt, a);
        if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
        return GRIM_OK;
    }

    int deferred = 0;
    {
        hipError_t e = router_logits_launch(st, L->router, x, rbias, p.logits, tokens, E, H,
                                            gemv ? nullptr : p.logits2, &deferred,
                                            gemv ? nullptr : p.wimg);
        if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    }
    int r = GRIM_OK;
    TopkArgs tka{p.logits, tokens, E, K, topk_mode, c.norm_topk, scaling, b16, b32,
                 rp ? rp->n_group : 0, rp ? rp->topk_group : 0, p.rex, p.rwt};
    // few rows per expert (on average at most 2): stream each expert once
    // per group of rows instead of once per 128-row MFMA tile
    const bool gv = !gemv && p.gv_te &&
                    (regime == 4 || regime == 5 || (regime == 0 && int64_t(tokens) * K <= 2 * int64_t(E))) &&
                    !(regime == 5 && layer_mx_padded(L));   // the vector-ALU one reads packed rows only
    const bool gv_mx = gv && regime != 5 && L->gate_up.fmt == GRIM_FMT_MXFP4 && gvm_shape_ok(H, I);
    if (gv_mx && int64_t(tokens) * K <= kGvmRouteMax && !shard) {
        if (deferred) {
            hipError_t e = router_finish_launch(st, p.logits, p.logits2, rbias, tokens, E);
            if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
        }
        return forward_gv(st, L, p, x, y, tokens, shared_gate_w, true, &tka);
    }
    if (deferred) {
        // the top-k finishes the split router's sum as it loads
        tka.part1 = p.logits2;
        tka.lbias = rbias;
    }
    {
        hipError_t e = topk_launch(st, tka);
        if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    }
    // one expert shard: the routes it owns become local indices, the rest
    // expert -1 / weight 0, and everything after the top-k sees a layer of
    // shard_count experts (the routing itself stays global)
    grim_moe_layer local;
    if (shard) {
        hipError_t e = route_local_launch(st, p.rex, p.rwt, p.lrex, p.lrwt, tokens * K, shard_begin, shard_count);
        if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
        p.rex = p.lrex;
        p.rwt = p.lrwt;
        local = *L;
        local.cfg.num_experts = shard_count;
        L = &local;
        E = shard_count;
    }

    if (gemv) {
        if (sh)
            return grimoire_moe_shared_rows(stream, L, &L->shared_gate_up, &L->shared_down,
                                            shared_gate_w, p.rex, p.rwt, x, p.h,
                                            shared_gate_w ? p.gate : nullptr, y, tokens);
        r = grimoire_moe_gate_up_batched(stream, L, p.rex, x, p.h, tokens);
        if (r) return r;
        return grimoire_moe_down_batched(stream, L, p.rex, p.rwt, p.h, y, tokens);
    }

    if (gv) return forward_gv(st, L, p, x, y, tokens, shared_gate_w, gv_mx, nullptr);
    if (regime == 5 && layer_mx_padded(L))
        return ferr(GRIM_ERR_FORMAT, "regime 5 reads packed MXFP4 rows (K/2 bytes); these are padded");
    if (regime == 4 || regime == 5)
        return ferr(GRIM_ERR_FORMAT, "regimes 4, 5: int4 / mxfp4 experts, hidden and inter % 32");

    // ---- GEMM regime
    const int fu = L->gate_up.fmt, fd = L->down.fmt;
    if (!gemm_format_ok(fu) || !gemm_format_ok(fd))
        return ferr(GRIM_ERR_FORMAT, "grouped GEMM supports int8, mxfp4 and bf16 weights");
    if (H % 64 || I % 64) return ferr(GRIM_ERR_SHAPE, "hidden and inter must be multiples of 64");
    const bool i8 = fu == GRIM_FMT_INT8 && fd == GRIM_FMT_INT8 && p.xq &&
                    (!sh || (L->shared_gate_up.fmt == fu && L->shared_down.fmt == fd)) &&
                    gemm_i8_shape_ok(2 * I, H, I, 1) && gemm_i8_shape_ok(H, I, 0, 0) && I <= 4096;
    if (i8) return forward_gemm_i8(st, L, p, x, y, tokens, shared_gate_w);

    r = grimoire_moe_route_grouped(stream, x, p.rex, p.xperm, p.xrow, p.counts, p.offsets,
                                   p.inverse, p.tile_e, p.tile_mb, p.tmax, tokens, H, E, kGemmBM, K,
                                   nullptr, p.disp_ws, dispatch_workspace_bytes(tokens, K, E));
    if (r) return r;
    if (sh && shared_gate_w) {
        hipError_t e = rowdot_sigmoid_launch(st, x, shared_gate_w, p.gate, tokens, H);
        if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    }
    int32_t* live = dispatch_live_tiles(p.disp_ws, tokens, K, E);

    GemmArgs g{};
    g.w = make_view(L->gate_up);
    if (sh)
        g.w_sh = make_view(L->shared_gate_up);
    g.N = 2 * I;
    g.K = H;
    g.I = I;
    g.swiglu = 1;
    g.A = p.xperm;
    g.A_sh = p.xrow;
    g.out = p.hp;
    g.out_sh = p.hp_sh;
    g.offsets = p.offsets;
    g.counts = p.counts;
    g.tile_e = p.tile_e;
    g.tile_mb = p.tile_mb;
    g.tmax = p.tmax;
    g.n_tiles_dev = live;
    g.T_sh = sh ? tokens : 0;
    if (sh && L->shared_gate_up.fmt != fu) return ferr(GRIM_ERR_FORMAT, "shared format mismatch");
    hipError_t e = gemm_launch(st, fu, g);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));

    GemmArgs d = g;
    d.w = make_view(L->down);
    if (sh)
        d.w_sh = make_view(L->shared_down);
    d.N = H;
    d.K = I;
    d.I = 0;
    d.swiglu = 0;
    d.a_pair = 1;
    d.out_bf16 = 0;
    d.A = p.hp;
    d.A_sh = p.hp_sh;
    d.out = p.yperm;
    d.out_sh = p.ysh;
    if (sh && L->shared_down.fmt != fd) return ferr(GRIM_ERR_FORMAT, "shared format mismatch");
    e = gemm_launch(st, fd, d);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));

    CombineArgs cb{p.yperm, 0, p.inverse, p.rwt, p.ysh, 0, (sh && shared_gate_w) ? p.gate : nullptr,
                   y, tokens, K, H};
    e = combine_launch(st, cb);
    if (e != hipSuccess) return ferr(int(e), hipGetErrorString(e));
    return GRIM_OK;
}

// forward.cpp shares api.cpp's thread-local message through this setter.
extern "C" __attribute__((visibility("hidden"))) void grimoire_moe_set_error_(const char* msg);
static int ferr(int code, const char* msg) {
    grimoire_moe_set_error_(msg);
    return code;
}
