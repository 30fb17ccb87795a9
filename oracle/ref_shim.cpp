// ref_shim.cpp -- extern "C" wrapper around the reference's own CPU MoE
// oracle (src/moe_ref.cpp) and GPTQ decode (include/b70/gptq.hpp), compiled
// from the reference sources where they lie by oracle/Makefile into
// oracle/_ref/libmoe_ref.so.
//
// TEST INFRASTRUCTURE ONLY: used to pin oracle/moe_oracle.c and as the
// "reference" CPU baseline of bench.py.  Nothing here is product code.
#include <cstring>

#include "b70/moe.hpp"
#include "b70/gptq.hpp"
#include "b70/nvfp4.hpp"
#include "b70/expert_heat.hpp"
#include "../include/grimoire_moe.h"

using namespace b70;

static QuantWeight to_ref(const grim_quant_weight& w) {
    QuantWeight q;
    q.fmt = Fmt(uint8_t(w.fmt));
    q.N = w.N;
    q.K = w.K;
    q.payload = w.payload;
    q.scales = w.scales;
    q.zeros = w.zeros;
    q.row_bytes = w.row_bytes;
    q.row_scales = w.row_scales;
    return q;
}

extern "C" {

// QuantWeight::at (include/b70/weights.hpp:102-121).  Formats 0..6 only.
float ref_qw_at(const grim_quant_weight* w, int n, int k) { return to_ref(*w).at(n, k); }

// gptq_at (include/b70/gptq.hpp:80-91)
float ref_gptq_at(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                  int in, int out, int group, int o, int k) {
    GptqTensor t;
    t.qweight = qweight; t.qzeros = qzeros; t.scales = scales;
    t.in = in; t.out = out; t.group = group;
    return gptq_at(t, o, k);
}

// gptq_repack_int4 (src/gptq.cpp:56-83); returns 0 when it refused the tensor.
int ref_gptq_repack_int4(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                         int in, int out, int group, uint8_t* payload, uint16_t* scales_out,
                         uint8_t* zeros_out) {
    GptqTensor t;
    t.qweight = qweight; t.qzeros = qzeros; t.scales = scales;
    t.in = in; t.out = out; t.group = group;
    PackedWeight p = gptq_repack_int4(t);
    if (p.payload.empty()) return 0;
    std::memcpy(payload, p.payload.data(), p.payload.size());
    std::memcpy(scales_out, p.scales_raw.data(), p.scales_raw.size());
    std::memcpy(zeros_out, p.zeros.data(), p.zeros.size());
    return 1;
}

// e4m3_to_f32 (include/b70/formats.hpp:157-169)
float ref_e4m3_to_f32(uint8_t b) { return e4m3_to_f32(b); }

// nvfp4_dequant_row (include/b70/nvfp4.hpp)
void ref_nvfp4_dequant_row(const uint8_t* packed, const uint8_t* scales, float gscale, int K,
                           float* out, int mul) {
    nvfp4_dequant_row(packed, scales, gscale, K, out, mul != 0);
}

// ExpertHeat (include/b70/expert_heat.hpp)
void* ref_heat_create(int layers, int experts, float decay, float hysteresis, float min_gain,
                      float credit_cap, int moves) {
    ExpertHeatParams p;
    p.decay = decay; p.hysteresis = hysteresis; p.min_gain = min_gain;
    p.credit_cap = credit_cap; p.moves_per_step = moves;
    ExpertHeat* h = new ExpertHeat;
    h->init(layers, experts, p);
    return h;
}
void ref_heat_destroy(void* h) { delete static_cast<ExpertHeat*>(h); }
void ref_heat_credit(void* h, int l, const int32_t* ids, size_t n) {
    static_cast<ExpertHeat*>(h)->credit(l, ids, n);
}
float ref_heat_get(void* h, int l, int e) { return static_cast<ExpertHeat*>(h)->heat(l, e); }
int ref_heat_propose(void* hp, int experts, const uint8_t* resident, const uint8_t* movable,
                     int32_t* out4, int max_out) {
    ExpertHeat* h = static_cast<ExpertHeat*>(hp);
    std::vector<ExpertSwap> sw;
    h->propose([&](int l, int e) { return resident[size_t(l) * experts + e] != 0; },
               [&](int l, int e) { return !movable || movable[size_t(l) * experts + e] != 0; }, sw);
    int n = 0;
    for (const ExpertSwap& s : sw) {
        if (n >= max_out) break;
        out4[4 * n] = s.promote_layer; out4[4 * n + 1] = s.promote_expert;
        out4[4 * n + 2] = s.demote_layer; out4[4 * n + 3] = s.demote_expert;
        ++n;
    }
    return n;
}

// route_ref (src/moe_ref.cpp:30-63)
void ref_route_ref(const float* logits, int n_experts, int top_k, int norm_topk,
                   int32_t* out_expert, float* out_weight) {
    Routing r;
    route_ref(logits, n_experts, top_k, norm_topk != 0, r);
    for (int j = 0; j < r.k; ++j) { out_expert[j] = r.expert[j]; out_weight[j] = r.weight[j]; }
}

// moe_forward_ref (src/moe_ref.cpp:88-105), one token at a time, shared
// expert (if any) with weight 1.
void ref_moe_forward(const grim_moe_layer* L, const int32_t* rex, const float* rwt,
                     const float* x, float* y, int tokens) {
    MoeLayer m;
    m.cfg.hidden = L->cfg.hidden; m.cfg.inter = L->cfg.inter;
    m.cfg.num_experts = L->cfg.num_experts; m.cfg.top_k = L->cfg.top_k;
    m.cfg.shared_inter = L->cfg.shared_inter; m.cfg.norm_topk = L->cfg.norm_topk != 0;
    m.gate_up = to_ref(L->gate_up);
    m.down = to_ref(L->down);
    m.has_shared = L->has_shared != 0;
    if (m.has_shared) {
        m.shared_gate_up = to_ref(L->shared_gate_up);
        m.shared_down = to_ref(L->shared_down);
    }
    const int H = L->cfg.hidden, K = L->cfg.top_k;
    for (int t = 0; t < tokens; ++t) {
        Routing r;
        r.k = K;
        for (int j = 0; j < K; ++j) {
            r.expert[j] = rex[int64_t(t) * K + j];
            r.weight[j] = rwt[int64_t(t) * K + j];
        }
        moe_forward_ref(m, r, x + int64_t(t) * H, y + int64_t(t) * H);
    }
}

}  // extern "C"
