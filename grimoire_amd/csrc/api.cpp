// api.cpp -- the extern "C" entry points of libgrimoire_moe.so.
//
// Argument checks happen here, on the host, before any launch: a shape the
// kernels do not support is rejected with a negative status and a message
// (grimoire_moe_last_error), never launched.  Each entry point cites the
// reference launcher it replaces in include/grimoire_moe.h.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/grimoire_moe.h"
#include "common.hpp"
#include "dispatch.hpp"
#include "gemm.hpp"
#include "gemm_i8.hpp"
#include "gemv.hpp"
#include "elementwise.hpp"
#include "ingest.hpp"
#include "tiered.hpp"
#include "router.hpp"
#include "gemv_mx.hpp"

using namespace grim;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int status(hipError_t e) {
    if (e == hipSuccess) return GRIM_OK;
    std::snprintf(g_err, sizeof g_err, "HIP error: %s", hipGetErrorString(e));
    return int(e);
}

hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

bool fmt_known(int f) {
    return f == GRIM_FMT_BF16 || f == GRIM_FMT_INT8 || f == GRIM_FMT_INT4 ||
           f == GRIM_FMT_INT4_F16 || f == GRIM_FMT_MXFP4;
}

// Check a weight view against the rows/cols the kernels will touch.
int check_weight(const grim_quant_weight* w, const char* name, int64_t rows, int K) {
    if (!w) return fail(GRIM_ERR_ARG, "%s: null weight", name);
    if (!fmt_known(w->fmt)) return fail(GRIM_ERR_FORMAT, "%s: format %d not supported", name, w->fmt);
    if (!w->payload) return fail(GRIM_ERR_ARG, "%s: null payload", name);
    if (w->K != K) return fail(GRIM_ERR_SHAPE, "%s: K=%d, expected %d", name, w->K, K);
    if (int64_t(w->N) < rows) return fail(GRIM_ERR_SHAPE, "%s: N=%d < %lld rows", name, w->N, (long long)rows);
    const int CH = chunk_elems(w->fmt);
    if (K % CH) return fail(GRIM_ERR_SHAPE, "%s: K=%d not a multiple of %d", name, K, CH);
    int64_t need = 0;
    switch (w->fmt) {
    case GRIM_FMT_BF16: need = int64_t(K) * 2; break;
    case GRIM_FMT_INT8: need = K; break;
    default: need = K / 2; break;
    }
    if (w->row_bytes < need || (w->row_bytes % 16))
        return fail(GRIM_ERR_SHAPE, "%s: row_bytes=%lld (need >= %lld, multiple of 16)", name,
                    (long long)w->row_bytes, (long long)need);
    if (reinterpret_cast<uintptr_t>(w->payload) % 16)
        return fail(GRIM_ERR_ARG, "%s: payload not 16-byte aligned", name);
    if (w->fmt != GRIM_FMT_BF16 && !w->scales) return fail(GRIM_ERR_ARG, "%s: null scales", name);
    if (w->fmt == GRIM_FMT_MXFP4 && w->row_scales < K / 32)
        return fail(GRIM_ERR_SHAPE, "%s: row_scales=%d < K/32", name, w->row_scales);
    if (w->fmt == GRIM_FMT_INT4 || w->fmt == GRIM_FMT_INT4_F16) {
        const int gs = 1 << int4_gshift(w->row_scales, K);
        if (K % gs || w->row_scales * gs != K)
            return fail(GRIM_ERR_SHAPE, "%s: INT4 group layout (row_scales=%d, K=%d)", name,
                        w->row_scales, K);
        if (gs < 32) return fail(GRIM_ERR_SHAPE, "%s: INT4 group < 32", name);
    }
    return GRIM_OK;
}

WView view(const grim_quant_weight& w) { return make_view(w); }

int check_layer(const grim_moe_layer* L) {
    if (!L) return fail(GRIM_ERR_ARG, "null layer");
    const auto& c = L->cfg;
    if (c.hidden <= 0 || c.inter <= 0 || c.num_experts <= 0 || c.top_k <= 0)
        return fail(GRIM_ERR_SHAPE, "bad config");
    // top_k may exceed num_experts on an expert shard (most slots then -1)
    if (c.top_k > 16) return fail(GRIM_ERR_SHAPE, "top_k=%d", c.top_k);
    if (c.num_experts > 512) return fail(GRIM_ERR_SHAPE, "num_experts=%d > 512", c.num_experts);
    int r = check_weight(&L->gate_up, "gate_up", int64_t(c.num_experts) * 2 * c.inter, c.hidden);
    if (r) return r;
    return check_weight(&L->down, "down", int64_t(c.num_experts) * c.hidden, c.inter);
}

// LDS ceiling of one work-group on gfx950 (160 KiB).
constexpr size_t kMaxLds = 160 * 1024;

int gemv_common(void* stream, const grim_moe_layer* L, const grim_quant_weight* wsh,
                const uint16_t* gate_w, const int32_t* rex, const float* x, float* h,
                float* gate_out, int M) {
    int r = check_layer(L);
    if (r) return r;
    if (M <= 0) return GRIM_OK;
    if (!rex || !x || !h) return fail(GRIM_ERR_ARG, "null routing/x/h");
    const auto& c = L->cfg;
    if (wsh) {
        r = check_weight(wsh, "shared gate_up", 2 * int64_t(c.inter), c.hidden);
        if (r) return r;
        if (wsh->fmt != L->gate_up.fmt)
            return fail(GRIM_ERR_FORMAT, "shared expert format must match routed experts");
    }
    if (gate_w && !gate_out) return fail(GRIM_ERR_ARG, "gate_w without gate_out");
    DecodeArgs a{};
    a.gu = view(L->gate_up);
    a.sgu = wsh ? view(*wsh) : a.gu;
    a.dn = a.sdn = view(L->down);
    a.shared = wsh != nullptr;
    a.rex = const_cast<int32_t*>(rex);
    a.x = x;
    a.h = h;
    a.gate_w = gate_w;
    a.gate = gate_out;
    a.H = c.hidden;
    a.I = c.inter;
    a.K = c.top_k;
    a.E = c.num_experts;
    a.M = M;
    decode_plan(L->gate_up.fmt, a, kRoleGateUp);
    if (decode_lds_bytes(L->gate_up.fmt, a) > kMaxLds)
        return fail(GRIM_ERR_SHAPE, "hidden=%d too large for the decode kernel", c.hidden);
    return status(decode_launch(S(stream), L->gate_up.fmt, a));
}

int down_common(void* stream, const grim_moe_layer* L, const grim_quant_weight* wd,
                const int32_t* rex, const float* rwt, const float* gate_in, const float* h,
                float* y, int M) {
    int r = check_layer(L);
    if (r) return r;
    if (M <= 0) return GRIM_OK;
    if (!rex || !rwt || !h || !y) return fail(GRIM_ERR_ARG, "null routing/h/y");
    const auto& c = L->cfg;
    if (wd) {
        r = check_weight(wd, "shared down", c.hidden, c.inter);
        if (r) return r;
        if (wd->fmt != L->down.fmt)
            return fail(GRIM_ERR_FORMAT, "shared expert format must match routed experts");
    }
    DecodeArgs a{};
    a.gu = a.sgu = view(L->gate_up);
    a.dn = view(L->down);
    a.sdn = wd ? view(*wd) : a.dn;
    a.shared = wd != nullptr;
    a.rex = const_cast<int32_t*>(rex);
    a.rwt = const_cast<float*>(rwt);
    a.gate_in = gate_in;
    a.h = const_cast<float*>(h);
    a.y = y;
    a.H = c.hidden;
    a.I = c.inter;
    a.K = c.top_k;
    a.E = c.num_experts;
    a.M = M;
    decode_plan(L->down.fmt, a, kRoleDown);
    if (decode_lds_bytes(L->down.fmt, a) > kMaxLds)
        return fail(GRIM_ERR_SHAPE, "(top_k+shared)*inter too large for the decode kernel");
    return status(decode_launch(S(stream), L->down.fmt, a));
}

// Shared body of the three bridges: one grouped GEMM over [ne][n (x2 for
// swiglu)][k] packed experts in rows mode (each work-group forms the
// expert offsets and tile order from rows_per_expert in LDS), so a bridge
// call allocates nothing and shares nothing with other calls.
int bridge_common(void* stream, const grim_quant_weight& w, int N, int I, int swiglu,
                  const void* a, void* d, const int* rows, int ne) {
    if (ne > kGemmRowsMaxExperts)
        return fail(GRIM_ERR_SHAPE, "bridge: num_experts %d > %d", ne, kGemmRowsMaxExperts);
    GemmArgs g{};
    g.w = view(w);
    g.N = N;
    g.K = w.K;
    g.I = I;
    g.swiglu = swiglu;
    g.a_pair = 0;
    g.out_bf16 = 1;
    g.A = static_cast<const uint16_t*>(a);
    g.out = d;
    g.rows = rows;
    g.ne = ne;
    g.tmax = 0;
    g.T_sh = 0;
    return status(gemm_launch(S(stream), w.fmt, g));
}

}  // namespace

extern "C" {

__attribute__((visibility("hidden"))) void grimoire_moe_set_error_(const char* msg) {
    std::snprintf(g_err, sizeof g_err, "%s", msg);
}

const char* grimoire_moe_last_error(void) { return g_err; }
const char* grimoire_moe_version(void) { return "grimoire_amd 0.1 (gfx950)"; }

int grimoire_moe_router_logits(void* stream, const float* router, const float* x, float* logits,
                               int tokens, int n_experts, int hidden) {
    if (tokens <= 0) return GRIM_OK;
    if (!router || !x || !logits) return fail(GRIM_ERR_ARG, "null pointer");
    if (n_experts <= 0 || hidden <= 0 || hidden % 4) return fail(GRIM_ERR_SHAPE, "hidden %% 4");
    return status(router_logits_launch(S(stream), router, x, nullptr, logits, tokens, n_experts, hidden));
}

static int topk_common(void* stream, const TopkArgs& a) {
    if (a.T <= 0) return GRIM_OK;
    if (!a.logits || !a.out_e || !a.out_w) return fail(GRIM_ERR_ARG, "null pointer");
    if (a.E <= 0 || a.E > 512) return fail(GRIM_ERR_SHAPE, "n_experts=%d (1..512)", a.E);
    if (a.K <= 0 || a.K > 16 || a.K > a.E) return fail(GRIM_ERR_SHAPE, "top_k=%d (1..16)", a.K);
    return status(topk_launch(S(stream), a));
}

int grimoire_moe_router_topk(void* stream, const float* logits, int n_experts, int top_k,
                             int32_t* out_expert, float* out_weight, int normalize) {
    TopkArgs a{logits, 1, n_experts, top_k, 0, normalize, 1.0f, nullptr, nullptr, 0, 0,
               out_expert, out_weight};
    return topk_common(stream, a);
}

int grimoire_moe_router_topk_batched(void* stream, const float* logits, int tokens, int n_experts,
                                     int top_k, int32_t* out_expert, float* out_weight,
                                     int normalize) {
    TopkArgs a{logits, tokens, n_experts, top_k, 1, normalize, 1.0f, nullptr, nullptr, 0, 0,
               out_expert, out_weight};
    return topk_common(stream, a);
}

int grimoire_moe_router_topk_bf16_batched(void* stream, const uint16_t* logits, int tokens,
                                          int n_experts, int top_k, int32_t* out_expert,
                                          float* out_weight, int normalize) {
    if (tokens <= 0) return GRIM_OK;
    if (!logits || !out_expert || !out_weight) return fail(GRIM_ERR_ARG, "null pointer");
    if (n_experts <= 0 || n_experts > 512)
        return fail(GRIM_ERR_SHAPE, "n_experts=%d (1..512)", n_experts);
    if (top_k <= 0 || top_k > 16 || top_k > n_experts)
        return fail(GRIM_ERR_SHAPE, "top_k=%d (1..16)", top_k);
    return status(topk_bf16_launch(S(stream), logits, tokens, n_experts, top_k, normalize,
                                   out_expert, out_weight));
}

int grimoire_moe_router_topk_sigmoid(void* stream, const float* logits, const uint16_t* bias_bf16,
                                     int tokens, int n_experts, int top_k, int32_t* out_expert,
                                     float* out_weight, int normalize, float scaling) {
    TopkArgs a{logits, tokens, n_experts, top_k, 2, normalize, scaling, bias_bf16, nullptr, 0, 0,
               out_expert, out_weight};
    return topk_common(stream, a);
}

int grimoire_moe_router_topk_group(void* stream, const float* logits, const float* bias,
                                   int tokens, int n_experts, int top_k, int n_group,
                                   int topk_group, int32_t* out_expert, float* out_weight,
                                   int normalize, float scaling) {
    if (n_group <= 0 || n_group > 64 || n_experts % n_group)
        return fail(GRIM_ERR_SHAPE, "n_group=%d must divide n_experts=%d (<= 64 groups)", n_group,
                    n_experts);
    if (topk_group <= 0 || topk_group > n_group) return fail(GRIM_ERR_SHAPE, "topk_group=%d", topk_group);
    if (top_k > topk_group * (n_experts / n_group))
        return fail(GRIM_ERR_SHAPE, "top_k exceeds the experts of the kept groups");
    TopkArgs a{logits, tokens, n_experts, top_k, 3, normalize, scaling, nullptr, bias, n_group,
               topk_group, out_expert, out_weight};
    return topk_common(stream, a);
}

int grimoire_moe_gate_up(void* stream, const grim_moe_layer* L, const int32_t* d_expert,
                         const float* x, float* h) {
    return gemv_common(stream, L, nullptr, nullptr, d_expert, x, h, nullptr, 1);
}

int grimoire_moe_down(void* stream, const grim_moe_layer* L, const int32_t* d_expert,
                      const float* d_weight, const float* h, float* y) {
    return down_common(stream, L, nullptr, d_expert, d_weight, nullptr, h, y, 1);
}

int grimoire_moe_gate_up_shared(void* stream, const grim_moe_layer* L, const grim_quant_weight* ws,
                                const uint16_t* gate_w, const int32_t* d_expert, const float* x,
                                float* h, float* gate_out) {
    if (!ws) return fail(GRIM_ERR_ARG, "null shared weight");
    return gemv_common(stream, L, ws, gate_w, d_expert, x, h, gate_out, 1);
}

int grimoire_moe_down_shared(void* stream, const grim_moe_layer* L, const grim_quant_weight* wd,
                             const int32_t* d_expert, const float* d_weight, const float* gate_in,
                             const float* h, float* y) {
    if (!wd) return fail(GRIM_ERR_ARG, "null shared weight");
    return down_common(stream, L, wd, d_expert, d_weight, gate_in, h, y, 1);
}

int grimoire_moe_gate_up_batched(void* stream, const grim_moe_layer* L, const int32_t* d_expert,
                                 const float* x, float* h, int tokens) {
    return gemv_common(stream, L, nullptr, nullptr, d_expert, x, h, nullptr, tokens);
}

int grimoire_moe_down_batched(void* stream, const grim_moe_layer* L, const int32_t* d_expert,
                              const float* d_weight, const float* h, float* y, int tokens) {
    return down_common(stream, L, nullptr, d_expert, d_weight, nullptr, h, y, tokens);
}

int grimoire_moe_shared_rows(void* stream, const grim_moe_layer* L, const grim_quant_weight* ws,
                             const grim_quant_weight* wd, const uint16_t* gate_w,
                             const int32_t* rex, const float* rwt, const float* x, float* h,
                             float* gate_out, float* y, int M) {
    if (!ws || !wd) return fail(GRIM_ERR_ARG, "null shared weight");
    int r = gemv_common(stream, L, ws, gate_w, rex, x, h, gate_out, M);
    if (r) return r;
    return down_common(stream, L, wd, rex, rwt, gate_w ? gate_out : nullptr, h, y, M);
}

size_t grimoire_moe_route_workspace_bytes(int tokens, int top_k, int num_experts) {
    return dispatch_workspace_bytes(tokens, top_k, num_experts);
}

static int dispatch_common(void* stream, const DispatchArgs& a, size_t ws_bytes) {
    if (a.T <= 0) return GRIM_OK;
    if (!a.ids || !a.counts || !a.offsets || !a.inverse) return fail(GRIM_ERR_ARG, "null pointer");
    if (a.E <= 0 || a.K <= 0 || a.K > 16) return fail(GRIM_ERR_SHAPE, "E/top_k");
    if (a.xperm && (a.H % 4 || !a.hidden)) return fail(GRIM_ERR_SHAPE, "hidden_size %% 4 / null hidden");
    if (!a.workspace || ws_bytes < dispatch_workspace_bytes(a.T, a.K, a.E))
        return fail(GRIM_ERR_WORKSPACE, "dispatch workspace too small (need %zu)",
                    dispatch_workspace_bytes(a.T, a.K, a.E));
    return status(dispatch_launch(S(stream), a));
}

int grimoire_moe_route_grouped(void* stream, const float* hidden, const int32_t* topk_ids,
                               uint16_t* xperm, uint16_t* xrow, int32_t* counts, int32_t* offsets,
                               int32_t* inverse, int32_t* tile_e, int32_t* tile_mb, int tmax,
                               int tokens, int hidden_size, int num_experts, int mc, int top_k,
                               int32_t* perm_token, void* workspace, size_t workspace_bytes) {
    if ((tile_e == nullptr) != (tile_mb == nullptr)) return fail(GRIM_ERR_ARG, "tile_e/tile_mb");
    if (tile_e && mc <= 0) return fail(GRIM_ERR_ARG, "mc must be > 0");
    DispatchArgs a{};
    a.ids = topk_ids; a.T = tokens; a.K = top_k; a.E = num_experts; a.H = hidden_size;
    a.hidden = hidden; a.hidden_bf16 = 0; a.xperm = xperm; a.xrow = xrow;
    a.counts = counts; a.offsets = offsets; a.inverse = inverse; a.perm_token = perm_token;
    a.tile_e = tile_e; a.tile_mb = tile_mb; a.tmax = tile_e ? tmax : 0; a.mc = mc;
    a.workspace = workspace;
    return dispatch_common(stream, a, workspace_bytes);
}

int grimoire_moe_remap_bf16(void* stream, const uint16_t* hidden, const int32_t* topk_ids,
                            uint16_t* remapped, int32_t* rows_per_expert, int32_t* expert_offsets,
                            int32_t* inverse, int tokens, int hidden_size, int num_experts,
                            int top_k, void* workspace, size_t workspace_bytes) {
    DispatchArgs a{};
    a.ids = topk_ids; a.T = tokens; a.K = top_k; a.E = num_experts; a.H = hidden_size;
    a.hidden = hidden; a.hidden_bf16 = 1; a.xperm = remapped; a.xrow = nullptr;
    a.counts = rows_per_expert; a.offsets = expert_offsets; a.inverse = inverse;
    a.perm_token = nullptr; a.tile_e = nullptr; a.tile_mb = nullptr; a.tmax = 0; a.mc = 0;
    a.workspace = workspace;
    return dispatch_common(stream, a, workspace_bytes);
}

int grimoire_moe_route_local(void* stream, const int32_t* topk_ids, const float* topk_w, int32_t* local_ids,
                             float* local_w, int routes, int expert_begin, int expert_count) {
    if (routes <= 0) return GRIM_OK;
    if (!topk_ids || !topk_w || !local_ids || !local_w) return fail(GRIM_ERR_ARG, "null pointer");
    if (expert_begin < 0 || expert_count <= 0) return fail(GRIM_ERR_ARG, "expert range");
    return status(route_local_launch(S(stream), topk_ids, topk_w, local_ids, local_w, routes, expert_begin,
                                     expert_count));
}

static int combine_common(void* stream, const CombineArgs& a) {
    if (a.T <= 0) return GRIM_OK;
    if (!a.src || !a.inverse || !a.rw || !a.dst) return fail(GRIM_ERR_ARG, "null pointer");
    if (a.K <= 0 || a.K > 16) return fail(GRIM_ERR_SHAPE, "top_k=%d", a.K);
    if (a.H % 4) return fail(GRIM_ERR_SHAPE, "hidden %% 4");
    return status(combine_launch(S(stream), a));
}

int grimoire_moe_unpermute(void* stream, const float* src, const int32_t* inverse,
                           const float* route_weight, float* dst, int tokens, int top_k,
                           int hidden) {
    CombineArgs a{src, 0, inverse, route_weight, nullptr, 0, nullptr, dst, tokens, top_k, hidden};
    return combine_common(stream, a);
}

int grimoire_moe_unpermute_bf16(void* stream, const uint16_t* src, const int32_t* inverse,
                                const float* route_weight, float* dst, int tokens, int top_k,
                                int hidden) {
    CombineArgs a{src, 1, inverse, route_weight, nullptr, 0, nullptr, dst, tokens, top_k, hidden};
    return combine_common(stream, a);
}

int grimoire_moe_combine(void* stream, const uint16_t* src, const int32_t* inverse,
                         const float* route_weight, const uint16_t* shared_src, const float* gate,
                         float* dst, int tokens, int top_k, int hidden) {
    CombineArgs a{src, 1, inverse, route_weight, shared_src, 1, gate, dst, tokens, top_k, hidden};
    return combine_common(stream, a);
}

int grimoire_moe_rmsnorm_residual(void* stream, float* h, const uint16_t* routed,
                                  const int32_t* inverse, const float* route_weight,
                                  const float* shared, const uint16_t* weight,
                                  float weight_offset, float* out, uint16_t* out_bf,
                                  int tokens, int top_k, int hidden, float eps) {
    if (tokens <= 0) return GRIM_OK;
    if (!h || !routed || !inverse || !route_weight || !weight)
        return fail(GRIM_ERR_ARG, "null pointer");
    if (top_k <= 0 || top_k > 16) return fail(GRIM_ERR_SHAPE, "top_k=%d", top_k);
    if (hidden <= 0 || hidden % 4) return fail(GRIM_ERR_SHAPE, "hidden=%d (need %% 4)", hidden);
    NormArgs a{h, routed, inverse, route_weight, shared, nullptr, weight, weight_offset, out,
               out_bf, tokens, top_k, hidden, eps};
    return status(combine_norm_launch(S(stream), a));
}

int grimoire_rmsnorm_residual(void* stream, float* h, const float* r0, const float* r1,
                              const uint16_t* weight, float weight_offset, float* out,
                              uint16_t* out_bf, int tokens, int hidden, float eps) {
    if (tokens <= 0) return GRIM_OK;
    if (!h || !weight) return fail(GRIM_ERR_ARG, "null pointer");
    if (hidden <= 0 || hidden % 4) return fail(GRIM_ERR_SHAPE, "hidden=%d (need %% 4)", hidden);
    NormArgs a{h, nullptr, nullptr, nullptr, r0, r1, weight, weight_offset, out, out_bf,
               tokens, 0, hidden, eps};
    return status(combine_norm_launch(S(stream), a));
}

static int ingest_common(void* stream, const grim_expert_src* srcs, const int32_t* row0s, int n,
                         const grim_quant_weight* dst) {
    if (n <= 0) return GRIM_OK;
    if (!srcs || !row0s || !dst) return fail(GRIM_ERR_ARG, "null srcs/row0/dst");
    if (!dst->payload || !dst->scales) return fail(GRIM_ERR_ARG, "null dst tensor");
    const grim_expert_src& s0 = srcs[0];
    const int in = s0.in, out = s0.out, g = s0.group;
    if (in <= 0 || out <= 0 || in % 32) return fail(GRIM_ERR_SHAPE, "in=%d out=%d", in, out);
    if (dst->K != in) return fail(GRIM_ERR_SHAPE, "dst K=%d, source in=%d", dst->K, in);
    if (dst->row_bytes != in / 2)
        return fail(GRIM_ERR_SHAPE, "dst row_bytes=%lld, need %d", (long long)dst->row_bytes, in / 2);
    for (int i = 0; i < n; ++i) {
        const grim_expert_src& s = srcs[i];
        if (s.kind != s0.kind || s.in != in || s.out != out || s.group != g)
            return fail(GRIM_ERR_SHAPE, "projection %d: kind or shape differs from projection 0", i);
        if (!s.weight || !s.scales) return fail(GRIM_ERR_ARG, "projection %d: null tensor", i);
        if (row0s[i] < 0 || int64_t(row0s[i]) + out > dst->N)
            return fail(GRIM_ERR_SHAPE, "projection %d: rows [%d, %d) outside dst N=%d", i,
                        row0s[i], row0s[i] + out, dst->N);
    }
    hipStream_t st = S(stream);
    uint8_t* pay0 = const_cast<uint8_t*>(dst->payload);
    if (s0.kind == GRIM_SRC_MXFP4_PACKED) {
        if (dst->fmt != GRIM_FMT_MXFP4) return fail(GRIM_ERR_FORMAT, "MXFP4 source needs MXFP4 dst");
        if (dst->row_scales != in / 32) return fail(GRIM_ERR_SHAPE, "dst row_scales != in/32");
        uint8_t* sc0 = static_cast<uint8_t*>(const_cast<void*>(dst->scales));
        for (int i = 0; i < n; ++i) {
            hipError_t e = hipMemcpyAsync(pay0 + int64_t(row0s[i]) * dst->row_bytes, srcs[i].weight,
                                          size_t(out) * (in / 2), hipMemcpyDefault, st);
            if (e == hipSuccess)
                e = hipMemcpyAsync(sc0 + int64_t(row0s[i]) * dst->row_scales, srcs[i].scales,
                                   size_t(out) * (in / 32), hipMemcpyDefault, st);
            if (e != hipSuccess) return status(e);
        }
        return GRIM_OK;
    }
    if (s0.kind != GRIM_SRC_GPTQ && s0.kind != GRIM_SRC_INT4_PACKED)
        return fail(GRIM_ERR_FORMAT, "source kind %d", s0.kind);
    if (g <= 0 || in % g || in % 8) return fail(GRIM_ERR_SHAPE, "group=%d in=%d", g, in);
    if (dst->row_scales != in / g) return fail(GRIM_ERR_SHAPE, "dst row_scales != in/group");
    if (!dst->zeros) return fail(GRIM_ERR_ARG, "dst zeros required");
    uint16_t* sc0 = static_cast<uint16_t*>(const_cast<void*>(dst->scales));
    uint8_t* zr0 = const_cast<uint8_t*>(dst->zeros);
    if (s0.kind == GRIM_SRC_GPTQ) {
        if (dst->fmt != GRIM_FMT_INT4 && dst->fmt != GRIM_FMT_INT4_F16)
            return fail(GRIM_ERR_FORMAT, "GPTQ source needs INT4 or INT4_F16 dst");
        if (out % 8) return fail(GRIM_ERR_SHAPE, "out=%d not a multiple of 8", out);
        if (reinterpret_cast<uintptr_t>(pay0) & 3) return fail(GRIM_ERR_ARG, "payload not 4-byte aligned");
        for (int i = 0; i < n; ++i) {
            if (!srcs[i].zeros) return fail(GRIM_ERR_ARG, "projection %d: GPTQ qzeros required", i);
            if ((reinterpret_cast<uintptr_t>(srcs[i].weight) |
                 reinterpret_cast<uintptr_t>(srcs[i].zeros)) & 3)
                return fail(GRIM_ERR_ARG, "projection %d: qweight/qzeros not 4-byte aligned", i);
        }
        for (int b = 0; b < n; b += kIngBatch) {
            IngestGptq a{};
            a.n = n - b < kIngBatch ? n - b : kIngBatch;
            for (int i = 0; i < a.n; ++i) {
                a.qweight[i] = static_cast<const uint32_t*>(srcs[b + i].weight);
                a.qzeros[i] = static_cast<const uint32_t*>(srcs[b + i].zeros);
                a.scales[i] = static_cast<const uint16_t*>(srcs[b + i].scales);
                a.row0[i] = row0s[b + i];
            }
            a.in = in; a.out = out; a.group = g;
            a.dst_payload = pay0; a.dst_row_bytes = dst->row_bytes;
            a.dst_scales = sc0; a.dst_zeros = zr0; a.dst_rs = dst->row_scales;
            a.keep_f16 = dst->fmt == GRIM_FMT_INT4_F16 ? 1 : 0;
            const hipError_t e = ingest_gptq(st, a);
            if (e != hipSuccess) return status(e);
        }
        return GRIM_OK;
    }
    if (dst->fmt != GRIM_FMT_INT4) return fail(GRIM_ERR_FORMAT, "INT4 source needs INT4 dst");
    if (out % 8) return fail(GRIM_ERR_SHAPE, "out=%d not a multiple of 8", out);
    for (int i = 0; i < n; ++i) {
        const grim_expert_src& s = srcs[i];
        if (s.zeros && (reinterpret_cast<uintptr_t>(s.zeros) & 3))
            return fail(GRIM_ERR_ARG, "projection %d: zero points not 4-byte aligned", i);
        const int64_t r0 = row0s[i];
        hipError_t e = hipMemcpyAsync(pay0 + r0 * dst->row_bytes, s.weight, size_t(out) * (in / 2),
                                      hipMemcpyDefault, st);
        if (e == hipSuccess)
            e = hipMemcpyAsync(sc0 + r0 * dst->row_scales, s.scales, size_t(out) * (in / g) * 2,
                               hipMemcpyDefault, st);
        if (e == hipSuccess)
            e = ingest_int4_zeros(st, static_cast<const uint32_t*>(s.zeros), out, in / g,
                                  zr0 + r0 * dst->row_scales, dst->row_scales);
        if (e != hipSuccess) return status(e);
    }
    return GRIM_OK;
}

int grimoire_moe_ingest_projection(void* stream, const grim_expert_src* src,
                                   const grim_quant_weight* dst, int row0) {
    if (!src) return fail(GRIM_ERR_ARG, "null src");
    const int32_t r = row0;
    return ingest_common(stream, src, &r, 1, dst);
}

int grimoire_moe_ingest_projections(void* stream, const grim_expert_src* srcs,
                                    const int32_t* row0, int n, const grim_quant_weight* dst) {
    return ingest_common(stream, srcs, row0, n, dst);
}

int grimoire_moe_int4_to_signed(void* stream, uint8_t* gu_payload, size_t gu_bytes,
                                uint8_t* gu_zeros, size_t gu_zero_bytes, uint8_t* dn_payload,
                                size_t dn_bytes, uint8_t* dn_zeros, size_t dn_zero_bytes,
                                int32_t* converted) {
    if (!converted) return fail(GRIM_ERR_ARG, "null converted flag");
    if ((gu_bytes && !gu_payload) || (gu_zero_bytes && !gu_zeros) || (dn_bytes && !dn_payload) ||
        (dn_zero_bytes && !dn_zeros))
        return fail(GRIM_ERR_ARG, "null region with a nonzero size");
    SignedRegion r[2] = {{gu_payload, int64_t(gu_bytes), gu_zeros, int64_t(gu_zero_bytes)},
                         {dn_payload, int64_t(dn_bytes), dn_zeros, int64_t(dn_zero_bytes)}};
    return status(int4_signed(S(stream), r, 2, converted));
}

int grimoire_tmoe_layout(int H, int I, grim_nv_expert_layout* out) {
    if (!out) return fail(GRIM_ERR_ARG, "null layout");
    if (H <= 0 || I <= 0 || H % 128 || I % 128)
        return fail(GRIM_ERR_SHAPE, "H=%d I=%d (need multiples of 128)", H, I);
    int64_t o = 0;
    out->H = H; out->I = I;
    out->gu_p = o; o += int64_t(2) * I * (H / 2);
    out->gu_s = o; o += int64_t(2) * I * (H / 16);
    out->dn_p = o; o += int64_t(H) * (I / 2);
    out->dn_s = o; o += int64_t(H) * (I / 16);
    out->gsc = o; o += 16;
    out->bytes = (o + 4095) & ~int64_t(4095);
    return GRIM_OK;
}

static int tmoe_args(const grim_tiered_moe_view* v, int M, TmoeArgs& a) {
    if (!v || !v->eptr) return fail(GRIM_ERR_ARG, "null view / block table");
    const grim_nv_expert_layout& L = v->lay;
    grim_nv_expert_layout want;
    if (grimoire_tmoe_layout(L.H, L.I, &want) != GRIM_OK) return GRIM_ERR_SHAPE;
    if (want.gu_p != L.gu_p || want.gu_s != L.gu_s || want.dn_p != L.dn_p ||
        want.dn_s != L.dn_s || want.gsc != L.gsc)
        return fail(GRIM_ERR_ARG, "block layout differs from grimoire_tmoe_layout(H, I)");
    if (v->E <= 0 || v->top_k <= 0 || v->top_k > 32)
        return fail(GRIM_ERR_SHAPE, "E=%d top_k=%d", v->E, v->top_k);
    if (M < 0) return fail(GRIM_ERR_SHAPE, "M=%d", M);
    a = TmoeArgs{};
    a.eptr = v->eptr;
    a.gu_p = L.gu_p; a.gu_s = L.gu_s; a.dn_p = L.dn_p; a.dn_s = L.dn_s; a.gsc = L.gsc;
    a.H = L.H; a.I = L.I; a.K = v->top_k; a.E = v->E; a.M = M;
    return GRIM_OK;
}

int grimoire_tmoe_gate_up(void* stream, const grim_tiered_moe_view* v, const int32_t* d_expert,
                          const float* x, float* h, int M) {
    TmoeArgs a;
    if (int st = tmoe_args(v, M, a)) return st;
    if (M == 0) return GRIM_OK;
    if (!d_expert || !x || !h) return fail(GRIM_ERR_ARG, "null pointer");
    a.expert = d_expert; a.x = x; a.h = h;
    return status(tmoe_gate_up(S(stream), a));
}

int grimoire_tmoe_down(void* stream, const grim_tiered_moe_view* v, const int32_t* d_expert,
                       const float* d_weight, const float* h, float* y, int M) {
    TmoeArgs a;
    if (int st = tmoe_args(v, M, a)) return st;
    if (M == 0) return GRIM_OK;
    if (!d_expert || !d_weight || !h || !y) return fail(GRIM_ERR_ARG, "null pointer");
    a.expert = d_expert; a.weight = d_weight; a.h = const_cast<float*>(h); a.y = y;  // read only
    return status(tmoe_down(S(stream), a));
}

size_t grimoire_tmoe_scratch_bytes(const grim_nv_expert_layout* L, int M) {
    if (!L || M < 0) return 0;
    const size_t w = size_t(2) * L->I * L->H * 2;            // decoded gate|up (>= down)
    return w + size_t(M) * 2 * L->I * 4 + 256;
}

static int tmoe_prefill_check(const uint8_t* block, const grim_nv_expert_layout* L, int M,
                              const void* A, const void* out, const void* scratch,
                              size_t scratch_bytes) {
    if (!block || !L || !A || !out || !scratch) return fail(GRIM_ERR_ARG, "null pointer");
    grim_nv_expert_layout want;
    if (grimoire_tmoe_layout(L->H, L->I, &want) != GRIM_OK) return GRIM_ERR_SHAPE;
    if (want.gu_p != L->gu_p || want.dn_s != L->dn_s || want.gsc != L->gsc)
        return fail(GRIM_ERR_ARG, "block layout differs from grimoire_tmoe_layout(H, I)");
    if (M < 0) return fail(GRIM_ERR_SHAPE, "M=%d", M);
    if (scratch_bytes < grimoire_tmoe_scratch_bytes(L, M))
        return fail(GRIM_ERR_WORKSPACE, "scratch %zu < %zu bytes", scratch_bytes,
                    grimoire_tmoe_scratch_bytes(L, M));
    return GRIM_OK;
}

// one expert's rows through the grouped bf16 GEMM: counts/offsets at the
// scratch tail
static int tmoe_gemm(hipStream_t st, const uint16_t* Wb, int N, int K, const uint16_t* A, float* out,
                     int M, int32_t* cnt_off) {
    hipError_t e = tmoe_set_rows(st, cnt_off, M);
    if (e != hipSuccess) return status(e);
    grim_quant_weight w{GRIM_FMT_BF16, N, K, 0, int64_t(K) * 2,
                        reinterpret_cast<const uint8_t*>(Wb), nullptr, nullptr};
    return grimoire_moe_grouped_gemm(st, &w, N, 0, A, 0, out, 0, cnt_off + 1, cnt_off, 1, M);
}

int grimoire_tmoe_expert_gemm(void* stream, const uint8_t* block, const grim_nv_expert_layout* L,
                              int gate_up, float s0, float s1, const uint16_t* A, float* out,
                              int M, void* scratch, size_t scratch_bytes) {
    if (int r = tmoe_prefill_check(block, L, M, A, out, scratch, scratch_bytes)) return r;
    if (M == 0) return GRIM_OK;
    hipStream_t st = S(stream);
    const int H = L->H, I = L->I;
    const int N = gate_up ? 2 * I : H, K = gate_up ? H : I;
    uint16_t* Wb = static_cast<uint16_t*>(scratch);
    int32_t* cnt_off = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(scratch) +
                                                  grimoire_tmoe_scratch_bytes(L, M) - 256);
    hipError_t e = tmoe_decode_bf16(st, block + (gate_up ? L->gu_p : L->dn_p),
                                    block + (gate_up ? L->gu_s : L->dn_s), N, K, Wb);
    if (e != hipSuccess) return status(e);
    if (int r = tmoe_gemm(st, Wb, N, K, A, out, M, cnt_off)) return r;
    return status(tmoe_scale_cols(st, out, M, N, gate_up ? I : N, s0, gate_up ? s1 : s0));
}

int grimoire_tmoe_expert_ffn(void* stream, const uint8_t* block, const grim_nv_expert_layout* L,
                             float sg, float su, float sd, const uint16_t* A, uint16_t* hbuf,
                             float* out, int M, void* scratch, size_t scratch_bytes) {
    if (int r = tmoe_prefill_check(block, L, M, A, out, scratch, scratch_bytes)) return r;
    if (!hbuf) return fail(GRIM_ERR_ARG, "null hbuf");
    if (M == 0) return GRIM_OK;
    hipStream_t st = S(stream);
    const int H = L->H, I = L->I;
    uint8_t* sb = static_cast<uint8_t*>(scratch);
    uint16_t* Wb = reinterpret_cast<uint16_t*>(sb);
    float* gu = reinterpret_cast<float*>(sb + size_t(2) * I * H * 2);
    int32_t* cnt_off = reinterpret_cast<int32_t*>(sb + grimoire_tmoe_scratch_bytes(L, M) - 256);
    hipError_t e = tmoe_decode_bf16(st, block + L->gu_p, block + L->gu_s, 2 * I, H, Wb);
    if (e != hipSuccess) return status(e);
    if (int r = tmoe_gemm(st, Wb, 2 * I, H, A, gu, M, cnt_off)) return r;
    e = tmoe_swiglu(st, gu, M, I, sg, su, hbuf);
    if (e == hipSuccess) e = tmoe_decode_bf16(st, block + L->dn_p, block + L->dn_s, H, I, Wb);
    if (e != hipSuccess) return status(e);
    if (int r = tmoe_gemm(st, Wb, H, I, hbuf, out, M, cnt_off)) return r;
    return status(tmoe_scale_cols(st, out, M, H, H, sd, sd));
}

int grimoire_tmoe_place(void* stream, const uint8_t** eptr, int e, uint8_t* dst_block,
                        const uint8_t* src_block, size_t bytes) {
    if (!eptr || !dst_block || e < 0) return fail(GRIM_ERR_ARG, "null table/block or e < 0");
    hipStream_t st = S(stream);
    if (src_block && bytes) {
        const hipError_t c = hipMemcpyAsync(dst_block, src_block, bytes, hipMemcpyDefault, st);
        if (c != hipSuccess) return status(c);
    }
    return status(tmoe_store(st, eptr, e, dst_block));
}

int grimoire_moe_unpermute_range(void* stream, const float* src, const int32_t* inverse,
                                 const float* route_weight, float* dst, int tokens, int top_k,
                                 int hidden, int p0, int p1, int accumulate) {
    if (p0 < 0 || p1 < p0) return fail(GRIM_ERR_ARG, "route range [%d, %d)", p0, p1);
    CombineArgs a{src, 0, inverse, route_weight, nullptr, 0, nullptr, dst, tokens, top_k, hidden};
    a.p0 = p0;
    a.p1 = p1;
    a.accumulate = accumulate ? 1 : 0;
    return combine_common(stream, a);
}

int grimoire_moe_permute_rows_bf16(void* stream, const float* src, const int32_t* perm_token,
                                   uint16_t* dst, int rows, int width) {
    if (rows <= 0) return GRIM_OK;
    if (!src || !perm_token || !dst) return fail(GRIM_ERR_ARG, "null pointer");
    if (width <= 0) return fail(GRIM_ERR_SHAPE, "width=%d", width);
    if ((width & 3) == 0 && ((reinterpret_cast<uintptr_t>(src) & 15) ||
                             (reinterpret_cast<uintptr_t>(dst) & 7)))
        return fail(GRIM_ERR_ARG, "src 16-byte / dst 8-byte alignment");
    return status(permute_rows_bf16_launch(S(stream), src, perm_token, dst, rows, width));
}

int grimoire_moe_swiglu_bf16(void* stream, const uint16_t* gu, uint16_t* out, int tokens,
                             int inter) {
    if (tokens <= 0) return GRIM_OK;
    if (!gu || !out) return fail(GRIM_ERR_ARG, "null pointer");
    if (inter <= 0) return fail(GRIM_ERR_SHAPE, "inter=%d", inter);
    return status(swiglu_bf16_launch(S(stream), gu, out, tokens, inter));
}

int grimoire_moe_scale_by_sigmoid(void* stream, float* x, const float* g, int n) {
    if (n <= 0) return GRIM_OK;
    if (!x || !g) return fail(GRIM_ERR_ARG, "null pointer");
    return status(scale_by_sigmoid_launch(S(stream), x, g, n, 0));
}

int grimoire_moe_scale_by_sigmoid_batched(void* stream, float* x, const float* gate, int tokens,
                                          int hidden) {
    if (tokens <= 0) return GRIM_OK;
    if (!x || !gate) return fail(GRIM_ERR_ARG, "null pointer");
    if (hidden <= 0) return fail(GRIM_ERR_SHAPE, "hidden=%d", hidden);
    return status(scale_by_sigmoid_launch(S(stream), x, gate, int64_t(tokens) * hidden, hidden));
}

int grimoire_moe_mxfp4_padded_k(int K) {
    if (K <= 0 || K % 32) return 0;
    return gvm_padded_k(K);
}

int grimoire_moe_pad_mxfp4_rows(void* stream, const grim_quant_weight* src, const grim_quant_weight* dst) {
    if (!src || !dst || !src->payload || !src->scales || !dst->payload || !dst->scales)
        return fail(GRIM_ERR_ARG, "null pointer");
    if (src->fmt != GRIM_FMT_MXFP4 || dst->fmt != GRIM_FMT_MXFP4) return fail(GRIM_ERR_FORMAT, "MXFP4 only");
    const int N = src->N, K = src->K;
    if (dst->N != N || dst->K != K || K <= 0 || K % 32 || N <= 0) return fail(GRIM_ERR_SHAPE, "N, K");
    const int64_t kb = K / 2, ks = K / 32;
    if (src->row_bytes < kb || src->row_scales < ks || dst->row_bytes < kb || dst->row_scales < ks)
        return fail(GRIM_ERR_SHAPE, "rows shorter than K");
    hipStream_t st = S(stream);
    const uint8_t* ss = static_cast<const uint8_t*>(src->scales);
    uint8_t* dp = const_cast<uint8_t*>(dst->payload);
    uint8_t* ds = static_cast<uint8_t*>(const_cast<void*>(dst->scales));
    hipError_t e = hipMemcpy2DAsync(dp, size_t(dst->row_bytes), src->payload, size_t(src->row_bytes), size_t(kb),
                                    size_t(N), hipMemcpyDefault, st);
    if (e == hipSuccess && dst->row_bytes > kb)
        e = hipMemset2DAsync(dp + kb, size_t(dst->row_bytes), 0, size_t(dst->row_bytes - kb), size_t(N), st);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync(ds, size_t(dst->row_scales), ss, size_t(src->row_scales), size_t(ks), size_t(N),
                             hipMemcpyDefault, st);
    // padding blocks: zero codes under scale byte 127 (2^0), so every
    // product there is an exact zero
    if (e == hipSuccess && dst->row_scales > ks)
        e = hipMemset2DAsync(ds + ks, size_t(dst->row_scales), 127, size_t(dst->row_scales - ks), size_t(N), st);
    return status(e);
}

int grimoire_moe_quant_limbs(void* stream, const float* src, int rows, int n, int8_t* dst,
                             float* scale) {
    if (rows <= 0) return GRIM_OK;
    if (!src || !dst || !scale) return fail(GRIM_ERR_ARG, "null pointer");
    if (n <= 0 || n % 64 || n > 4096) return fail(GRIM_ERR_SHAPE, "n=%d: a multiple of 64, <= 4096", n);
    return status(quant_rows_launch(S(stream), src, rows, n, dst, scale));
}

int grimoire_moe_grouped_gemm_i8(void* stream, const grim_quant_weight* w, int N, int swiglu,
                                 const int8_t* A, const float* a_scale, float* out,
                                 const int32_t* offsets, const int32_t* counts,
                                 const int32_t* tile_e, const int32_t* tile_mb, int tmax,
                                 int num_experts) {
    if (!w || !A || !a_scale || !out || !offsets || !counts || !tile_e || !tile_mb)
        return fail(GRIM_ERR_ARG, "null pointer");
    if (w->fmt != GRIM_FMT_INT8) return fail(GRIM_ERR_FORMAT, "INT8 weights only");
    int r = check_weight(w, "grouped weight", int64_t(num_experts) * N, w->K);
    if (r) return r;
    if (swiglu && N % 2) return fail(GRIM_ERR_SHAPE, "swiglu needs even N");
    if (!gemm_i8_shape_ok(N, w->K, swiglu ? N / 2 : 0, swiglu))
        return fail(GRIM_ERR_SHAPE, "K=%d: a multiple of 64 in [192, 8192]", w->K);
    if (tmax <= 0) return GRIM_OK;
    GemmI8Args g{};
    g.w = w->payload;
    g.ws = static_cast<const float*>(w->scales);
    g.row_bytes = w->row_bytes;
    g.N = N;
    g.K = w->K;
    g.I = swiglu ? N / 2 : 0;
    g.swiglu = swiglu;
    g.A = A;
    g.sa = a_scale;
    g.out = out;
    g.offsets = offsets;
    g.counts = counts;
    g.tile_e = tile_e;
    g.tile_mb = tile_mb;
    g.tmax = tmax;
    g.n_tiles_dev = nullptr;   // the table is -1 padded to tmax
    return status(gemm_i8_launch(S(stream), g));
}

int grimoire_moe_grouped_gemm_i8_rows(void* stream, const grim_quant_weight* w, int N, int swiglu,
                                      const int8_t* A, const float* a_scale, float* out,
                                      const int32_t* offsets, const int32_t* counts, int num_experts,
                                      int split) {
    if (!w || !A || !a_scale || !out || !offsets || !counts) return fail(GRIM_ERR_ARG, "null pointer");
    if (w->fmt != GRIM_FMT_INT8) return fail(GRIM_ERR_FORMAT, "INT8 weights only");
    if (num_experts <= 0 || num_experts > kI8MaxListExperts)
        return fail(GRIM_ERR_SHAPE, "num_experts=%d: 1..%d", num_experts, kI8MaxListExperts);
    int r = check_weight(w, "grouped weight", int64_t(num_experts) * N, w->K);
    if (r) return r;
    if (swiglu && N % 2) return fail(GRIM_ERR_SHAPE, "swiglu needs even N");
    if (!gemm_i8_shape_ok(N, w->K, swiglu ? N / 2 : 0, swiglu))
        return fail(GRIM_ERR_SHAPE, "K=%d: a multiple of 64 in [192, 8192]", w->K);
    GemmI8Args g{};
    g.w = w->payload;
    g.ws = static_cast<const float*>(w->scales);
    g.row_bytes = w->row_bytes;
    g.N = N;
    g.K = w->K;
    g.I = swiglu ? N / 2 : 0;
    g.swiglu = swiglu;
    g.A = A;
    g.sa = a_scale;
    g.out = out;
    g.offsets = offsets;
    g.counts = counts;
    g.split = split > 0 ? split : kI8DefaultSplit;
    g.num_experts = num_experts;
    return status(gemm_i8_launch(S(stream), g));
}

int grimoire_moe_grouped_gemm_i8_rows_gather(void* stream, const grim_quant_weight* w, int N, int swiglu,
                                             const int8_t* A, int a_rows, const int32_t* row_map,
                                             const float* a_scale, float* out, const int32_t* offsets,
                                             const int32_t* counts, int num_experts, int split) {
    if (!w || !A || !row_map || !a_scale || !out || !offsets || !counts)
        return fail(GRIM_ERR_ARG, "null pointer");
    if (w->fmt != GRIM_FMT_INT8) return fail(GRIM_ERR_FORMAT, "INT8 weights only");
    if (num_experts <= 0 || num_experts > kI8MaxListExperts)
        return fail(GRIM_ERR_SHAPE, "num_experts=%d: 1..%d", num_experts, kI8MaxListExperts);
    int r = check_weight(w, "grouped weight", int64_t(num_experts) * N, w->K);
    if (r) return r;
    if (swiglu && N % 2) return fail(GRIM_ERR_SHAPE, "swiglu needs even N");
    if (!gemm_i8_shape_ok(N, w->K, swiglu ? N / 2 : 0, swiglu))
        return fail(GRIM_ERR_SHAPE, "K=%d: a multiple of 64 in [192, 8192]", w->K);
    if (!gemm_i8_gather_ok(w->K, a_rows))
        return fail(GRIM_ERR_SHAPE, "gather: K=%d needs >= 6 K tiles of 64 (>= 4 of 128 when K %% 128 == 0), "
                    "a_rows=%d rows of 2K bytes below 1.75 GiB", w->K, a_rows);
    GemmI8Args g{};
    g.w = w->payload;
    g.ws = static_cast<const float*>(w->scales);
    g.row_bytes = w->row_bytes;
    g.N = N;
    g.K = w->K;
    g.I = swiglu ? N / 2 : 0;
    g.swiglu = swiglu;
    g.A = A;
    g.sa = a_scale;
    g.out = out;
    g.offsets = offsets;
    g.counts = counts;
    g.split = split > 0 ? split : kI8DefaultSplit;
    g.num_experts = num_experts;
    g.gather = row_map;
    g.gather_rows = a_rows;
    return status(gemm_i8_launch(S(stream), g));
}

int grimoire_moe_grouped_gemm(void* stream, const grim_quant_weight* w, int N, int swiglu,
                              const uint16_t* A, int a_pair, void* out, int out_bf16,
                              const int32_t* offsets, const int32_t* counts, int num_experts,
                              int total_rows) {
    if (!w || !A || !out || !offsets || !counts) return fail(GRIM_ERR_ARG, "null pointer");
    if (!gemm_format_ok(w->fmt))
        return fail(GRIM_ERR_FORMAT, "grouped GEMM supports int8, mxfp4 and bf16 weights");
    int r = check_weight(w, "grouped weight", int64_t(num_experts) * N, w->K);
    if (r) return r;
    if (w->K % 64) return fail(GRIM_ERR_SHAPE, "K=%d not a multiple of 64", w->K);
    if (swiglu && (N % 2 || a_pair)) return fail(GRIM_ERR_SHAPE, "swiglu needs even N, bf16 A");
    if (total_rows <= 0) return GRIM_OK;
    if (num_experts > kGemmRowsMaxExperts)
        return fail(GRIM_ERR_SHAPE, "num_experts %d > %d", num_experts, kGemmRowsMaxExperts);
    GemmArgs g{};
    g.w = view(*w);
    g.N = N;
    g.K = w->K;
    g.I = swiglu ? N / 2 : 0;
    g.swiglu = swiglu;
    g.a_pair = a_pair;
    g.out_bf16 = swiglu ? 0 : out_bf16;   // SwiGLU: h as bf16 pairs
    g.A = A;
    g.out = out;
    g.offsets = offsets;   // rows mode on the device counts
    g.rows = counts;
    g.ne = num_experts;
    return status(gemm_launch(S(stream), w->fmt, g));
}

void grimoire_xe2_grouped_mxfp4_bf16(void* stream, const void* a, const unsigned char* b,
                                     const unsigned char* scales, void* d, int n, int k,
                                     const int* rows_per_expert, const int* expert_ids,
                                     int num_experts, int* atomic_buffer) {
    (void)expert_ids;      // rows are grouped in expert order, as the reference
    (void)atomic_buffer;   // no work counter: each work-group forms the tile order
    if (!a || !b || !scales || !d || !rows_per_expert) {
        fail(GRIM_ERR_ARG, "xe2 mxfp4: null pointer");
        return;
    }
    if (n <= 0 || k <= 0 || num_experts <= 0 || k % 64) {
        fail(GRIM_ERR_SHAPE, "xe2 mxfp4: n=%d k=%d num_experts=%d (k a multiple of 64)", n, k,
             num_experts);
        return;
    }
    grim_quant_weight w{GRIM_FMT_MXFP4, num_experts * n, k, k / 32, k / 2, b, scales, nullptr};
    if (check_weight(&w, "xe2 mxfp4", int64_t(num_experts) * n, k)) return;
    bridge_common(stream, w, n, 0, 0, a, d, rows_per_expert, num_experts);
}

void grimoire_xe2_grouped_mxfp4_bf16_full(void* stream, const void* a, const unsigned char* b,
                                          const unsigned char* scales, void* d, int n, int k,
                                          const int* rows_per_expert, const int* expert_ids,
                                          int num_experts, int* atomic_buffer) {
    grimoire_xe2_grouped_mxfp4_bf16(stream, a, b, scales, d, n, k, rows_per_expert, expert_ids,
                                    num_experts, atomic_buffer);
}

void grimoire_xe2_grouped_mxfp4_bf16_m8(void* stream, const void* a, const unsigned char* b,
                                        const unsigned char* scales, void* d, int n, int k,
                                        const int* rows_per_expert, const int* expert_ids,
                                        int num_experts, int* atomic_buffer) {
    grimoire_xe2_grouped_mxfp4_bf16(stream, a, b, scales, d, n, k, rows_per_expert, expert_ids,
                                    num_experts, atomic_buffer);
}

void grimoire_xe2_grouped_mxfp4_bf16_m16(void* stream, const void* a, const unsigned char* b,
                                         const unsigned char* scales, void* d, int n, int k,
                                         const int* rows_per_expert, const int* expert_ids,
                                         int num_experts, int* atomic_buffer) {
    grimoire_xe2_grouped_mxfp4_bf16(stream, a, b, scales, d, n, k, rows_per_expert, expert_ids,
                                    num_experts, atomic_buffer);
}

void grimoire_xe2_grouped_w4a16(void* stream, const void* activations_bf16,
                                const unsigned char* weights_int4, const void* scales_bf16,
                                void* outputs_bf16, int n, int k, const int* rows_per_expert,
                                const int* expert_ids, int num_experts, int group_size,
                                int* atomic_buffer) {
    (void)expert_ids;      // rows are grouped in expert order, as the reference
    (void)atomic_buffer;   // no work counter: each work-group forms the tile order
    if (!activations_bf16 || !weights_int4 || !scales_bf16 || !outputs_bf16 || !rows_per_expert) {
        fail(GRIM_ERR_ARG, "xe2 w4a16: null pointer");
        return;
    }
    if (n <= 0 || k <= 0 || num_experts <= 0 || group_size <= 0 || group_size % 64 || k % group_size) {
        fail(GRIM_ERR_SHAPE, "xe2 w4a16: n=%d k=%d group=%d (group a multiple of 64 dividing k)", n,
             k, group_size);
        return;
    }
    grim_quant_weight w{kGemmFmtS4, num_experts * n, k, k / group_size, k / 2, weights_int4,
                        scales_bf16, nullptr};
    bridge_common(stream, w, n, 0, 0, activations_bf16, outputs_bf16, rows_per_expert, num_experts);
}

void grimoire_xe2_fused_moe_gate_up_mxfp4_silu_bf16(void* stream, const void* activations,
                                                    const unsigned char* weights,
                                                    const unsigned char* scales, void* outputs,
                                                    int n, int k, const int* rows_per_expert,
                                                    int num_experts, int32_t* atomic_buffer) {
    (void)atomic_buffer;   // no work counter: each work-group forms the tile order
    if (!activations || !weights || !scales || !outputs || !rows_per_expert) {
        fail(GRIM_ERR_ARG, "xe2 fused gate_up: null pointer");
        return;
    }
    if (n <= 0 || k <= 0 || num_experts <= 0 || k % 64 || n % 8) {
        fail(GRIM_ERR_SHAPE, "xe2 fused gate_up: n=%d k=%d num_experts=%d (k %% 64, n %% 8)", n, k,
             num_experts);
        return;
    }
    grim_quant_weight w{GRIM_FMT_MXFP4, num_experts * 2 * n, k, k / 32, k / 2, weights, scales, nullptr};
    if (check_weight(&w, "xe2 fused gate_up", int64_t(num_experts) * 2 * n, k)) return;
    bridge_common(stream, w, 2 * n, n, 1, activations, outputs, rows_per_expert, num_experts);
}

}  // extern "C"
