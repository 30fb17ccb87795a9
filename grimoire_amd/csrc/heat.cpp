// heat.cpp -- which experts of a tiered layer live in VRAM.
//
// Per (layer, expert) a decayed count of how often the router picked it
// (include/b70/expert_heat.hpp): every call of a layer multiplies that
// layer's heats by `decay` and adds one per route, or credit_cap / n per
// route when a call routes more than credit_cap rows (a long prompt would
// otherwise take over the resident set).  A step proposes up to
// moves_per_step swaps: the hottest non-resident candidates against the
// coldest resident ones, in order, while hot >= cold * hysteresis +
// min_gain; ties go to the lower (layer, expert).  Host code: placement
// decisions are a few thousand floats per step.
#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <new>
#include <vector>

#include "../../include/grimoire_moe.h"

// the guard hot >= cold * hysteresis + min_gain rounds the product before
// the sum, as the reference's build does: no fused multiply-add here
#pragma clang fp contract(off)

struct grim_heat {
    int L = 0, E = 0;
    grim_heat_params p{};
    std::vector<float> h;
};

namespace {

struct Cand {
    float h;
    int l, e;
};

bool hotter(const Cand& a, const Cand& b) {
    if (a.h != b.h) return a.h > b.h;
    return a.l != b.l ? a.l < b.l : a.e < b.e;
}

bool colder(const Cand& a, const Cand& b) {
    if (a.h != b.h) return a.h < b.h;
    return a.l != b.l ? a.l < b.l : a.e < b.e;
}

}  // namespace

extern "C" {

void grimoire_heat_default_params(grim_heat_params* p) {
    if (!p) return;
    p->decay = 0.95f;
    p->hysteresis = 1.25f;
    p->min_gain = 1.5f;
    p->credit_cap = 512.0f;
    p->moves_per_step = 32;
}

grim_heat* grimoire_heat_create(int layers, int experts, const grim_heat_params* params) {
    if (layers <= 0 || experts <= 0) return nullptr;
    grim_heat* s = new (std::nothrow) grim_heat;
    if (!s) return nullptr;
    s->L = layers;
    s->E = experts;
    if (params) s->p = *params;
    else grimoire_heat_default_params(&s->p);
    s->h.assign(size_t(layers) * size_t(experts), 0.0f);
    return s;
}

void grimoire_heat_destroy(grim_heat* s) { delete s; }

void grimoire_heat_credit(grim_heat* s, int layer, const int32_t* ids, size_t n) {
    if (!s || layer < 0 || layer >= s->L || !ids) return;
    float* row = s->h.data() + size_t(layer) * size_t(s->E);
    for (int e = 0; e < s->E; ++e) row[e] *= s->p.decay;
    const float w = float(n) > s->p.credit_cap ? s->p.credit_cap / float(n) : 1.0f;
    for (size_t i = 0; i < n; ++i)
        if (ids[i] >= 0 && ids[i] < s->E) row[ids[i]] += w;
}

float grimoire_heat_get(const grim_heat* s, int layer, int expert) {
    if (!s || layer < 0 || layer >= s->L || expert < 0 || expert >= s->E) return 0.0f;
    return s->h[size_t(layer) * size_t(s->E) + size_t(expert)];
}

int grimoire_heat_propose(const grim_heat* s, const uint8_t* resident, const uint8_t* movable,
                          grim_expert_swap* out, int max_out) {
    if (!s || !resident || (!out && max_out > 0)) return GRIM_ERR_ARG;
    std::vector<Cand> hot, cold;
    for (int l = 0; l < s->L; ++l)
        for (int e = 0; e < s->E; ++e) {
            const size_t i = size_t(l) * size_t(s->E) + size_t(e);
            if (movable && !movable[i]) continue;
            const float x = s->h[i];
            if (resident[i]) cold.push_back({x, l, e});
            else if (x > 0.0f) hot.push_back({x, l, e});
        }
    const size_t S = size_t(std::max(0, std::min(s->p.moves_per_step, max_out)));
    const size_t nh = std::min(S, hot.size()), nc = std::min(S, cold.size());
    std::partial_sort(hot.begin(), hot.begin() + std::ptrdiff_t(nh), hot.end(), hotter);
    std::partial_sort(cold.begin(), cold.begin() + std::ptrdiff_t(nc), cold.end(), colder);
    int n = 0;
    for (size_t i = 0; i < nh && i < nc; ++i) {
        if (!(hot[i].h >= cold[i].h * s->p.hysteresis + s->p.min_gain)) break;
        out[n++] = grim_expert_swap{hot[i].l, hot[i].e, cold[i].l, cold[i].e};
    }
    return n;
}

}  // extern "C"
