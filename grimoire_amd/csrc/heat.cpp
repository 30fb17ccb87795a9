// heat.cpp -- which experts of a tiered layer live in VRAM.
//
// State: one fp32 heat per (layer, expert), flat index i = layer * E +
// expert.  Crediting a call of layer l ages that layer's heats by `decay`
// and adds a weight per route (1, or credit_cap / n when the call routes
// more than credit_cap rows, so that a long prompt does not take over the
// resident set).  A step proposes swaps: the k-th hottest non-resident
// expert against the k-th coldest resident one, k = 0, 1, ..., while
// hot >= cold * hysteresis + min_gain, at most moves_per_step of them.
// Behaviour of include/b70/expert_heat.hpp:62-97 (decay, cap, guard and the
// lower-(layer, expert) tie rule); the implementation is this file's own:
//
//   * credit histograms the route ids first and then walks the layer's
//     row once: each heat is aged and then receives its own routes' weight
//     one addition at a time (the per-expert operation sequence, and so
//     the rounding, of aging then adding route by route);
//   * the ranking works on one 64-bit integer key per candidate: the heat's
//     bit pattern (heats are never negative, so bit order is value order)
//     above the flat index, complemented for the "hottest first" key so
//     that the lower index wins ties either way; a bounded max-heap keeps
//     the moves_per_step best keys of each side in one pass over the
//     model, and the kept keys are then sorted.
// Host code: placement decisions are a few thousand floats per step.
#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <new>
#include <queue>
#include <vector>

#include "../../include/grimoire_moe.h"

// the guard rounds the product before the sum: no fused multiply-add
#pragma clang fp contract(off)

struct grim_heat {
    int layers = 0, experts = 0;
    grim_heat_params prm{};
    std::vector<float> heat;        // [layers * experts]
    std::vector<uint32_t> hist;     // credit scratch [experts]
};

namespace {

uint32_t float_bits(float v) {
    uint32_t b;
    std::memcpy(&b, &v, sizeof b);
    return b;
}

float bits_float(uint32_t b) {
    float v;
    std::memcpy(&v, &b, sizeof v);
    return v;
}

// Larger key = hotter: heat first, then the lower flat index.
uint64_t hot_key(float h, uint32_t i) { return (uint64_t(float_bits(h)) << 32) | (0xFFFFFFFFu - i); }
// Smaller key = colder: heat first, then the lower flat index.
uint64_t cold_key(float h, uint32_t i) { return (uint64_t(float_bits(h)) << 32) | i; }

// Keeps the `cap` smallest keys seen (a max-heap of them).
class SmallestK {
public:
    explicit SmallestK(size_t cap) : cap_(cap) {}
    void offer(uint64_t k) {
        if (cap_ == 0) return;
        if (q_.size() < cap_) q_.push(k);
        else if (k < q_.top()) { q_.pop(); q_.push(k); }
    }
    std::vector<uint64_t> ascending() {
        std::vector<uint64_t> v;
        v.reserve(q_.size());
        while (!q_.empty()) { v.push_back(q_.top()); q_.pop(); }
        std::reverse(v.begin(), v.end());
        return v;
    }
private:
    size_t cap_;
    std::priority_queue<uint64_t> q_;
};

}  // namespace

extern "C" {

void grimoire_heat_default_params(grim_heat_params* p) {
    if (!p) return;
    *p = grim_heat_params{};
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
    s->layers = layers;
    s->experts = experts;
    if (params) s->prm = *params;
    else grimoire_heat_default_params(&s->prm);
    s->heat.assign(size_t(layers) * size_t(experts), 0.0f);
    s->hist.assign(size_t(experts), 0u);
    return s;
}

void grimoire_heat_destroy(grim_heat* s) { delete s; }

void grimoire_heat_credit(grim_heat* s, int layer, const int32_t* ids, size_t n) {
    if (!s || layer < 0 || layer >= s->layers || !ids) return;
    const int E = s->experts;
    std::fill(s->hist.begin(), s->hist.end(), 0u);
    for (size_t r = 0; r < n; ++r)
        if (ids[r] >= 0 && ids[r] < E) ++s->hist[size_t(ids[r])];
    const float cap = s->prm.credit_cap;
    const float w = float(n) > cap ? cap / float(n) : 1.0f;
    float* h = s->heat.data() + size_t(layer) * size_t(E);
    for (int e = 0; e < E; ++e) {
        float v = h[e] * s->prm.decay;
        for (uint32_t k = s->hist[size_t(e)]; k > 0; --k) v += w;
        h[e] = v;
    }
}

float grimoire_heat_get(const grim_heat* s, int layer, int expert) {
    if (!s || layer < 0 || layer >= s->layers || expert < 0 || expert >= s->experts) return 0.0f;
    return s->heat[size_t(layer) * size_t(s->experts) + size_t(expert)];
}

int grimoire_heat_propose(const grim_heat* s, const uint8_t* resident, const uint8_t* movable,
                          grim_expert_swap* out, int max_out) {
    if (!s || !resident || (!out && max_out > 0)) return GRIM_ERR_ARG;
    const int budget = std::min(s->prm.moves_per_step, max_out);
    const size_t cap = size_t(budget > 0 ? budget : 0);
    // hottest first == smallest complemented hot key
    SmallestK hot(cap), cold(cap);
    const size_t total = s->heat.size();
    for (size_t i = 0; i < total; ++i) {
        if (movable && !movable[i]) continue;
        const float h = s->heat[i];
        if (resident[i]) cold.offer(cold_key(h, uint32_t(i)));
        else if (h > 0.0f) hot.offer(~hot_key(h, uint32_t(i)));
    }
    const std::vector<uint64_t> hk = hot.ascending(), ck = cold.ascending();
    const size_t pairs = std::min(hk.size(), ck.size());
    const int E = s->experts;
    int n = 0;
    for (size_t k = 0; k < pairs; ++k) {
        const uint64_t up = ~hk[k];
        const float h_up = bits_float(uint32_t(up >> 32));
        const uint32_t i_up = 0xFFFFFFFFu - uint32_t(up);
        const float h_dn = bits_float(uint32_t(ck[k] >> 32));
        const uint32_t i_dn = uint32_t(ck[k]);
        if (!(h_up >= h_dn * s->prm.hysteresis + s->prm.min_gain)) break;
        out[n++] = grim_expert_swap{int(i_up / uint32_t(E)), int(i_up % uint32_t(E)),
                                    int(i_dn / uint32_t(E)), int(i_dn % uint32_t(E))};
    }
    return n;
}

}  // extern "C"
