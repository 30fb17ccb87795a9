/*
 * moe_oracle.c -- CPU restatement of GRIMOIRE's MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY (see moe_oracle.h).  Not linked into, called by,
 * or shipped with the product library.
 *
 * Parity pinning (what checks each function, tests/test_oracle.py):
 *   orc_f16_to_f32      exhaustive closed form over 65536 codes
 *   orc_bf16/e8m0/e2m1  closed forms + tables of tests/test_formats.cpp:45-83
 *   orc_gptq_at         16 golden probes of tests/test_gptq.cpp:50-56
 *   orc_qw_at           reference QuantWeight::at via oracle/_ref + brute force
 *   orc_route_ref       reference route_ref via oracle/_ref + properties
 *   orc_topk_*          brute-force full sort on the same scores
 *   orc_topk_group      brute force over every group subset (no reference)
 *   orc_moe_forward     reference moe_forward_ref via oracle/_ref; loose
 *                       per-expert tensors (tests/test_moe.cpp:54-74 idea)
 *   orc_dispatch        invariants of src/grimoire.cpp:23047-23097
 *   orc_unpermute       closed form on one-hot routes
 *   orc_rmsnorm_moe_residual  orc_unpermute (h = 0, no shared), exact
 *                       h + shared (all slots skipped), float64 RMSNorm
 *   orc_rmsnorm_residual  exact (h + r0) + r1, float64 RMSNorm, torch
 *                       rms_norm
 *   orc_gptq_repack     reference gptq_repack_int4 via oracle/_ref, golden
 *                       GPTQ probes through orc_qw_at, orc_gptq_at
 *   orc_int4_zero_unpack  brute-force nibble extraction
 *   orc_e4m3_to_f32     reference e4m3_to_f32 over all 256 codes via oracle/_ref
 *   orc_nvfp4_dequant_row  reference nvfp4_dequant_row via oracle/_ref
 *   orc_tmoe_*          float64 products of the reference-dequantised blocks
 *   orc_int4_to_signed  dequantised values unchanged (orc_qw_at before and
 *                       after), untouched when one zero point is not 8
 *   orc_grouped_gemm    numpy matmul of the dequantised weights
 *   orc_expf            libm expf to within 2 ulp
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static float bits_f(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t f_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* include/b70/formats.hpp:72-86 */
float orc_f16_to_f32(uint16_t h) {
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return bits_f(s);
        /* subnormal: value m * 2^-24 exactly */
        float v = (float)m * 5.9604644775390625e-08f;
        return s ? -v : v;
    }
    if (e == 0x1F) return bits_f(s | 0x7F800000u | (m << 13));
    return bits_f(s | ((e - 15 + 127) << 23) | (m << 13));
}

/* include/b70/formats.hpp:68 */
float orc_bf16_to_f32(uint16_t b) { return bits_f((uint32_t)b << 16); }

/* include/b70/formats.hpp:88-97, round to nearest even, NaN kept NaN */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f_bits(f);
    if (((u >> 23) & 0xFFu) == 0xFFu)
        return (uint16_t)((u >> 16) | ((u & 0x7FFFFFu) ? 0x40u : 0u));
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* include/b70/formats.hpp:105-109 */
float orc_e8m0_to_f32(uint8_t x) {
    if (x == 0xFF) return bits_f(0x7FC00000u);
    if (x == 0x00) return bits_f(0x00400000u);
    return bits_f((uint32_t)x << 23);
}

/* include/b70/formats.hpp:122-126 */
float orc_e2m1_to_f32(uint8_t nib) {
    static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    float v = mag[nib & 7];
    return (nib & 8) ? -v : v;
}

/* exp(x) by Cody-Waite reduction x = k ln2 + r, |r| <= ln2/2, and the
 * degree-7 Taylor polynomial of e^r in Horner form (truncation < 6e-9
 * relative), scaled by 2^k as two exact power-of-two factors so that the
 * only rounding of a subnormal result is the last multiply.  Every step is
 * an explicit IEEE operation, so the device restatement of this function
 * returns the same bits. */
float orc_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.972084045410156f) return 0.0f;
    const float kf = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(kf, -0.693145751953125f, x);
    r = fmaf(kf, -1.428606765330187045e-06f, r);
    float p = 1.98412698412698413e-04f;          /* 1/5040 */
    p = fmaf(p, r, 1.38888888888888889e-03f);    /* 1/720  */
    p = fmaf(p, r, 8.33333333333333333e-03f);    /* 1/120  */
    p = fmaf(p, r, 4.16666666666666667e-02f);    /* 1/24   */
    p = fmaf(p, r, 1.66666666666666667e-01f);    /* 1/6    */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int k = (int)kf;
    const int k1 = k / 2, k2 = k - k1;
    const float s1 = bits_f((uint32_t)(k1 + 127) << 23);
    const float s2 = bits_f((uint32_t)(k2 + 127) << 23);
    return (p * s1) * s2;
}

float orc_sigmoid(float x) { return 1.0f / (1.0f + orc_expf(-x)); }

/* INT4 group size from the shape, as include/b70/weights.hpp:80-84. */
static int int4_gshift(const grim_quant_weight* w) {
    const int64_t rs = w->row_scales, k = w->K;
    return rs * 32 == k ? 5 : rs * 64 == k ? 6 : rs * 256 == k ? 8 : 7;
}

/* include/b70/weights.hpp:58-121 + formats.hpp:456-491 */
float orc_qw_at(const grim_quant_weight* w, int n, int k) {
    const uint8_t* row = w->payload + (int64_t)n * w->row_bytes;
    switch (w->fmt) {
    case GRIM_FMT_BF16:
        return orc_bf16_to_f32((uint16_t)(row[2 * k] | (row[2 * k + 1] << 8)));
    case GRIM_FMT_INT8:
        return (float)(int8_t)row[k] * ((const float*)w->scales)[n];
    case GRIM_FMT_MXFP4: {
        const uint8_t byte = row[k >> 1];
        const uint8_t nib = (k & 1) ? (byte >> 4) : (byte & 0x0F);
        const uint8_t e = ((const uint8_t*)w->scales)[(int64_t)n * w->row_scales + k / 32];
        return orc_e2m1_to_f32(nib) * orc_e8m0_to_f32(e);
    }
    case GRIM_FMT_INT4:
    case GRIM_FMT_INT4_F16: {
        const int gi = k >> int4_gshift(w);
        const int64_t si = (int64_t)n * w->row_scales + gi;
        const uint16_t sraw = ((const uint16_t*)w->scales)[si];
        const float s = w->fmt == GRIM_FMT_INT4 ? orc_bf16_to_f32(sraw) : orc_f16_to_f32(sraw);
        const uint8_t byte = row[k >> 1];
        const int q = (k & 1) ? (byte >> 4) : (byte & 0x0F);
        uint8_t z;
        if (w->zeros) z = w->zeros[si];
        else z = w->fmt == GRIM_FMT_INT4_F16 ? 8 : 0;
        if (z == 0xFF) return (float)((q & 8) ? q - 16 : q) * s;
        return ((float)q - (float)z) * s;
    }
    }
    return 0.0f;
}

/* include/b70/gptq.hpp:80-91 */
float orc_gptq_at(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                  int in, int out, int group, int o, int k) {
    (void)in;
    const int grp = k / group;
    const uint32_t wword = (uint32_t)qweight[(int64_t)(k >> 3) * out + o];
    const uint32_t nib = (wword >> ((k & 7) * 4)) & 0xFu;
    const uint32_t zword = (uint32_t)qzeros[(int64_t)grp * (out >> 3) + (o >> 3)];
    const uint32_t znib = (zword >> ((o & 7) * 4)) & 0xFu;
    const float scale = orc_f16_to_f32(scales[(int64_t)grp * out + o]);
    return ((float)nib - (float)(znib + 1u)) * scale;
}

/* ---------------------------------------------------------------- router */

/* src/moe_ref.cpp:30-63 */
void orc_route_ref(const float* logits, int n_experts, int top_k, int norm_topk,
                   int32_t* out_expert, float* out_weight) {
    float m = logits[0];
    for (int e = 1; e < n_experts; ++e) m = logits[e] > m ? logits[e] : m;
    float* p = (float*)malloc(sizeof(float) * (size_t)n_experts);
    unsigned char* taken = (unsigned char*)calloc((size_t)n_experts, 1);
    double z = 0.0;
    for (int e = 0; e < n_experts; ++e) {
        p[e] = expf(logits[e] - m);
        z += p[e];
    }
    for (int e = 0; e < n_experts; ++e) p[e] = (float)(p[e] / z);
    /* selection: probability descending, lower index first on ties */
    for (int j = 0; j < top_k; ++j) {
        int best = -1;
        for (int e = 0; e < n_experts; ++e) {
            if (taken[e]) continue;
            if (best < 0 || p[e] > p[best]) best = e;
        }
        taken[best] = 1;
        out_expert[j] = best;
        out_weight[j] = p[best];
    }
    double s = 0.0;
    for (int j = 0; j < top_k; ++j) s += out_weight[j];
    if (norm_topk && s > 0.0)
        for (int j = 0; j < top_k; ++j) out_weight[j] = (float)(out_weight[j] / s);
    free(p);
    free(taken);
}

/* src/ops.cpp:1100-1148 (register kernel) and :1347-1422 (batched). */
void orc_topk_softmax(const float* logits, int tokens, int n_experts, int top_k, int normalize,
                      int batched, int32_t* out_expert, float* out_weight) {
    unsigned char* taken = (unsigned char*)malloc((size_t)n_experts);
    for (int t = 0; t < tokens; ++t) {
        const float* row = logits + (int64_t)t * n_experts;
        int32_t* oe = out_expert + (int64_t)t * top_k;
        float* ow = out_weight + (int64_t)t * top_k;
        memset(taken, 0, (size_t)n_experts);
        float v[16];
        for (int s = 0; s < top_k; ++s) {
            int best = -1;
            for (int e = 0; e < n_experts; ++e) {
                if (taken[e]) continue;
                if (best < 0 || row[e] > row[best]) best = e;   /* strict >: lowest index */
            }
            taken[best] = 1;
            oe[s] = best;
            v[s] = row[best];
        }
        if (batched && !normalize) {
            for (int s = 0; s < top_k; ++s) ow[s] = v[s];
            continue;
        }
        float m = v[0];
        for (int s = 1; s < top_k; ++s) m = fmaxf(m, v[s]);
        float sum = 0.0f;
        float ev[16];
        for (int s = 0; s < top_k; ++s) {
            ev[s] = orc_expf(v[s] - m);
            sum += ev[s];
        }
        for (int s = 0; s < top_k; ++s) ow[s] = (normalize && sum > 0.0f) ? ev[s] / sum : ev[s];
    }
    free(taken);
}

static void finish_weights(float* ow, int top_k, int normalize, float scaling) {
    if (normalize) {
        float sum = 0.0f;
        for (int s = 0; s < top_k; ++s) sum += ow[s];
        if (sum > 0.0f)
            for (int s = 0; s < top_k; ++s) ow[s] /= sum;
    }
    if (scaling != 1.0f)
        for (int s = 0; s < top_k; ++s) ow[s] *= scaling;
}

/* src/ops.cpp:2059-2170 */
void orc_topk_sigmoid(const float* logits, const uint16_t* bias_bf16, int tokens, int n_experts,
                      int top_k, int normalize, float scaling, int32_t* out_expert,
                      float* out_weight) {
    float* sc = (float*)malloc(sizeof(float) * (size_t)n_experts);
    float* sel = (float*)malloc(sizeof(float) * (size_t)n_experts);
    unsigned char* taken = (unsigned char*)malloc((size_t)n_experts);
    for (int t = 0; t < tokens; ++t) {
        const float* row = logits + (int64_t)t * n_experts;
        int32_t* oe = out_expert + (int64_t)t * top_k;
        float* ow = out_weight + (int64_t)t * top_k;
        memset(taken, 0, (size_t)n_experts);
        for (int e = 0; e < n_experts; ++e) {
            sc[e] = orc_sigmoid(row[e]);
            sel[e] = sc[e] + (bias_bf16 ? orc_bf16_to_f32(bias_bf16[e]) : 0.0f);
        }
        for (int s = 0; s < top_k; ++s) {
            int best = -1;
            for (int e = 0; e < n_experts; ++e) {
                if (taken[e]) continue;
                if (best < 0 || sel[e] > sel[best]) best = e;
            }
            taken[best] = 1;
            oe[s] = best;
            ow[s] = sc[best];
        }
        finish_weights(ow, top_k, normalize, scaling);
    }
    free(sc);
    free(sel);
    free(taken);
}

/* DeepSeek-V3 group-limited routing, from its published definition. */
void orc_topk_group(const float* logits, const float* bias, int tokens, int n_experts, int top_k,
                    int n_group, int topk_group, int normalize, float scaling,
                    int32_t* out_expert, float* out_weight) {
    const int gs = n_experts / n_group;
    float* sc = (float*)malloc(sizeof(float) * (size_t)n_experts);
    float* sel = (float*)malloc(sizeof(float) * (size_t)n_experts);
    unsigned char* taken = (unsigned char*)malloc((size_t)n_experts);
    unsigned char* gkeep = (unsigned char*)malloc((size_t)n_group);
    float* gscore = (float*)malloc(sizeof(float) * (size_t)n_group);
    for (int t = 0; t < tokens; ++t) {
        const float* row = logits + (int64_t)t * n_experts;
        int32_t* oe = out_expert + (int64_t)t * top_k;
        float* ow = out_weight + (int64_t)t * top_k;
        for (int e = 0; e < n_experts; ++e) {
            sc[e] = orc_sigmoid(row[e]);
            sel[e] = sc[e] + (bias ? bias[e] : 0.0f);
        }
        for (int g = 0; g < n_group; ++g) {
            /* two largest of the group (lower index first among equals) */
            int b1 = -1, b2 = -1;
            for (int e = g * gs; e < (g + 1) * gs; ++e) {
                if (b1 < 0 || sel[e] > sel[b1]) { b2 = b1; b1 = e; }
                else if (b2 < 0 || sel[e] > sel[b2]) b2 = e;
            }
            gscore[g] = gs > 1 ? sel[b1] + sel[b2] : sel[b1];
        }
        memset(gkeep, 0, (size_t)n_group);
        for (int j = 0; j < topk_group; ++j) {
            int best = -1;
            for (int g = 0; g < n_group; ++g) {
                if (gkeep[g]) continue;
                if (best < 0 || gscore[g] > gscore[best]) best = g;
            }
            gkeep[best] = 1;
        }
        for (int e = 0; e < n_experts; ++e) taken[e] = gkeep[e / gs] ? 0 : 1;
        for (int s = 0; s < top_k; ++s) {
            int best = -1;
            for (int e = 0; e < n_experts; ++e) {
                if (taken[e]) continue;
                if (best < 0 || sel[e] > sel[best]) best = e;
            }
            taken[best] = 1;
            oe[s] = best;
            ow[s] = sc[best];
        }
        finish_weights(ow, top_k, normalize, scaling);
    }
    free(sc);
    free(sel);
    free(taken);
    free(gkeep);
    free(gscore);
}

/* src/grimoire.cpp:15364 (router GEMV), double accumulation */
void orc_router_logits(const float* router, const float* x, float* logits, int tokens,
                       int n_experts, int hidden) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < tokens; ++t)
        for (int e = 0; e < n_experts; ++e) {
            double a = 0.0;
            const float* w = router + (int64_t)e * hidden;
            const float* xt = x + (int64_t)t * hidden;
            for (int k = 0; k < hidden; ++k) a += (double)w[k] * xt[k];
            logits[(int64_t)t * n_experts + e] = (float)a;
        }
}

/* --------------------------------------------------------------- experts */

static float silu_f(float v) { return v / (1.0f + expf(-v)); }

/* one (gate,up) row pair: src/moe_ref.cpp:72-79 */
static float swiglu_row(const grim_quant_weight* w, int64_t g_row, int64_t u_row, int H,
                        const float* x) {
    double g = 0.0, u = 0.0;
    for (int c = 0; c < H; ++c) {
        g += (double)orc_qw_at(w, (int)g_row, c) * x[c];
        u += (double)orc_qw_at(w, (int)u_row, c) * x[c];
    }
    return silu_f((float)g) * (float)u;
}

/* src/moe_kernels.cpp:82-257 semantics */
void orc_gate_up(const grim_moe_layer* L, const grim_quant_weight* ws, const uint16_t* gate_w,
                 const int32_t* rex, const float* x, float* h, float* gate_out, int tokens) {
    const int H = L->cfg.hidden, I = L->cfg.inter, K = L->cfg.top_k;
    const int KS = K + (ws ? 1 : 0);
#pragma omp parallel for schedule(dynamic)
    for (int t = 0; t < tokens; ++t) {
        const float* xt = x + (int64_t)t * H;
        for (int s = 0; s < KS; ++s) {
            const grim_quant_weight* w = s < K ? &L->gate_up : ws;
            const int64_t base = s < K ? (int64_t)rex[(int64_t)t * K + s] * 2 * I : 0;
            for (int i = 0; i < I; ++i)
                h[((int64_t)t * KS + s) * I + i] = swiglu_row(w, base + i, base + I + i, H, xt);
        }
        if (gate_w && gate_out) {
            float a = 0.0f;
            for (int c = 0; c < H; ++c) a = fmaf(orc_bf16_to_f32(gate_w[c]), xt[c], a);
            gate_out[t] = 1.0f / (1.0f + expf(-a));
        }
    }
}

/* src/moe_kernels.cpp:273-445 semantics */
void orc_down(const grim_moe_layer* L, const grim_quant_weight* wd, const int32_t* rex,
              const float* rwt, const float* gate_in, const float* h, float* y, int tokens) {
    const int H = L->cfg.hidden, I = L->cfg.inter, K = L->cfg.top_k;
    const int KS = K + (wd ? 1 : 0);
#pragma omp parallel for schedule(dynamic)
    for (int t = 0; t < tokens; ++t) {
        const float* ht = h + (int64_t)t * KS * I;
        for (int o = 0; o < H; ++o) {
            float total = 0.0f;
            for (int s = 0; s < KS; ++s) {
                const grim_quant_weight* w;
                int64_t row;
                float rw;
                if (s < K) {
                    const int e = rex[(int64_t)t * K + s];
                    rw = rwt[(int64_t)t * K + s];
                    if (e < 0 || rw == 0.0f) continue;
                    w = &L->down;
                    row = (int64_t)e * H + o;
                } else {
                    w = wd;
                    row = o;
                    rw = gate_in ? gate_in[t] : 1.0f;
                }
                double a = 0.0;
                for (int i = 0; i < I; ++i) a += (double)orc_qw_at(w, (int)row, i) * ht[s * I + i];
                total += rw * (float)a;
            }
            y[(int64_t)t * H + o] = total;
        }
    }
}

/* src/moe_ref.cpp:68-105 for T tokens */
void orc_moe_forward(const grim_moe_layer* L, const int32_t* rex, const float* rwt,
                     const float* gate, const float* x, float* y, int tokens) {
    const int H = L->cfg.hidden, I = L->cfg.inter, K = L->cfg.top_k;
    const int SI = L->cfg.shared_inter;
#pragma omp parallel
    {
        const int IM = I > SI ? I : SI;
        float* hb = (float*)malloc(sizeof(float) * (size_t)IM);
#pragma omp for schedule(dynamic)
        for (int t = 0; t < tokens; ++t) {
            const float* xt = x + (int64_t)t * H;
            float* yt = y + (int64_t)t * H;
            for (int o = 0; o < H; ++o) yt[o] = 0.0f;
            const int nslot = K + (L->has_shared ? 1 : 0);
            for (int s = 0; s < nslot; ++s) {
                const grim_quant_weight *gu, *dn;
                int64_t g0, u0, d0;
                int II;
                float scale;
                if (s < K) {
                    const int e = rex[(int64_t)t * K + s];
                    if (e < 0) continue;
                    gu = &L->gate_up; dn = &L->down;
                    g0 = (int64_t)e * 2 * I; u0 = g0 + I; d0 = (int64_t)e * H;
                    II = I;
                    scale = rwt[(int64_t)t * K + s];
                } else {
                    gu = &L->shared_gate_up; dn = &L->shared_down;
                    g0 = 0; u0 = SI; d0 = 0;
                    II = SI;
                    scale = gate ? gate[t] : 1.0f;
                }
                for (int i = 0; i < II; ++i) hb[i] = swiglu_row(gu, g0 + i, u0 + i, H, xt);
                for (int o = 0; o < H; ++o) {
                    double a = 0.0;
                    for (int i = 0; i < II; ++i) a += (double)orc_qw_at(dn, (int)(d0 + o), i) * hb[i];
                    yt[o] += scale * (float)a;
                }
            }
        }
        free(hb);
    }
}

/* -------------------------------------------------------------- dispatch */

/* src/grimoire.cpp:23162-23170 (stable counting sort) and the tile table
 * of src/prefill.cpp:2770-2782 */
int orc_dispatch(const int32_t* topk_ids, int tokens, int top_k, int n_experts, int mc,
                 int32_t* counts, int32_t* offsets, int32_t* inverse, int32_t* perm_token,
                 int32_t* tile_e, int32_t* tile_mb, int tmax) {
    const int R = tokens * top_k;
    for (int e = 0; e < n_experts; ++e) counts[e] = 0;
    for (int r = 0; r < R; ++r) {
        const int e = topk_ids[r];
        if (e >= 0 && e < n_experts) ++counts[e];
    }
    int acc = 0;
    for (int e = 0; e < n_experts; ++e) { offsets[e] = acc; acc += counts[e]; }
    int32_t* cur = (int32_t*)malloc(sizeof(int32_t) * (size_t)(n_experts > 0 ? n_experts : 1));
    for (int e = 0; e < n_experts; ++e) cur[e] = offsets[e];
    for (int r = 0; r < R; ++r) {
        const int e = topk_ids[r];
        if (e < 0 || e >= n_experts) { inverse[r] = -1; continue; }
        const int p = cur[e]++;
        inverse[r] = p;
        if (perm_token) perm_token[p] = r / top_k;
    }
    free(cur);
    int nt = 0;
    if (tile_e && tile_mb && mc > 0) {
        for (int e = 0; e < n_experts; ++e)
            for (int mb = 0; mb * mc < counts[e]; ++mb) {
                if (nt < tmax) { tile_e[nt] = e; tile_mb[nt] = mb; }
                ++nt;
            }
        for (int t = nt; t < tmax; ++t) { tile_e[t] = -1; tile_mb[t] = 0; }
    }
    return nt;
}

/* src/prefill.cpp:2654-2668 */
void orc_unpermute(const float* src, const int32_t* inverse, const float* route_weight,
                   float* dst, int tokens, int top_k, int hidden) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < tokens; ++t)
        for (int d = 0; d < hidden; ++d) {
            float v = 0.0f;
            for (int s = 0; s < top_k; ++s) {
                const int64_t r = (int64_t)t * top_k + s;
                const int32_t p = inverse[r];
                if (p >= 0) v = fmaf(route_weight[r], src[(int64_t)p * hidden + d], v);
            }
            dst[(int64_t)t * hidden + d] = v;
        }
}

/* src/prefill.cpp:1004-1045 (launch_rmsnorm_moe_residual_batched); the
 * weight offset is g_norm_weight_offset (include/b70/prefill_qk_math.hpp:14).
 * ss accumulates as an fma chain in column order (the reference splits it
 * over work-items; the order only moves the last bits of the scale). */
void orc_rmsnorm_moe_residual(float* h, const uint16_t* routed, const int32_t* inverse,
                              const float* route_weight, const float* shared,
                              const uint16_t* weight, float weight_offset, float* out,
                              uint16_t* out_bf, int tokens, int top_k, int hidden, float eps) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < tokens; ++t) {
        float* ht = h + (int64_t)t * hidden;
        float ss = 0.0f;
        for (int d = 0; d < hidden; ++d) {
            float v = ht[d] + (shared ? shared[(int64_t)t * hidden + d] : 0.0f);
            for (int s = 0; s < top_k; ++s) {
                const int64_t r = (int64_t)t * top_k + s;
                const int32_t p = inverse[r];
                if (p >= 0)
                    v = fmaf(route_weight[r], orc_bf16_to_f32(routed[(int64_t)p * hidden + d]), v);
            }
            ht[d] = v;
            ss = fmaf(v, v, ss);
        }
        const float scale = 1.0f / sqrtf(ss / (float)hidden + eps);
        for (int d = 0; d < hidden; ++d) {
            const float o = ht[d] * scale * (weight_offset + orc_bf16_to_f32(weight[d]));
            if (out) out[(int64_t)t * hidden + d] = o;
            if (out_bf) out_bf[(int64_t)t * hidden + d] = orc_f32_to_bf16(o);
        }
    }
}

/* src/prefill.cpp:627-700 (launch_rmsnorm_residual_batched, ungrouped). */
void orc_rmsnorm_residual(float* h, const float* r0, const float* r1, const uint16_t* weight,
                          float weight_offset, float* out, uint16_t* out_bf, int tokens,
                          int hidden, float eps) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < tokens; ++t) {
        float* ht = h + (int64_t)t * hidden;
        float ss = 0.0f;
        for (int d = 0; d < hidden; ++d) {
            float v = ht[d];
            if (r0) v += r0[(int64_t)t * hidden + d];
            if (r1) v += r1[(int64_t)t * hidden + d];
            if (r0 || r1) ht[d] = v;
            ss = fmaf(v, v, ss);
        }
        const float scale = 1.0f / sqrtf(ss / (float)hidden + eps);
        for (int d = 0; d < hidden; ++d) {
            const float o = ht[d] * scale * (weight_offset + orc_bf16_to_f32(weight[d]));
            if (out) out[(int64_t)t * hidden + d] = o;
            if (out_bf) out_bf[(int64_t)t * hidden + d] = orc_f32_to_bf16(o);
        }
    }
}

/* gptq_repack_int4 (src/gptq.cpp:56-83): payload [out][in/2] (even k in the
 * low nibble), zeros [out][in/g] = stored + 1, scales [out][in/g] rounded to
 * bf16, or the fp16 bits kept when keep_f16. */
void orc_gptq_repack(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                     int in, int out, int group, int keep_f16, uint8_t* payload,
                     uint16_t* scales_out, uint8_t* zeros_out) {
    const int ng = in / group;
    for (int o = 0; o < out; ++o) {
        for (int g = 0; g < ng; ++g) {
            const uint32_t zw = (uint32_t)qzeros[(int64_t)g * (out / 8) + o / 8];
            zeros_out[(int64_t)o * ng + g] = (uint8_t)(((zw >> ((o & 7) * 4)) & 0xFu) + 1u);
            const uint16_t s = scales[(int64_t)g * out + o];
            scales_out[(int64_t)o * ng + g] = keep_f16 ? s : orc_f32_to_bf16(orc_f16_to_f32(s));
        }
        uint8_t* row = payload + (int64_t)o * (in / 2);
        for (int k = 0; k < in; ++k) {
            const uint32_t w = (uint32_t)qweight[(int64_t)(k / 8) * out + o];
            const uint8_t q = (uint8_t)((w >> ((k & 7) * 4)) & 0xFu);
            if (k & 1) row[k / 2] = (uint8_t)(row[k / 2] | (q << 4));
            else row[k / 2] = q;
        }
    }
}

/* Compressed-tensors INT4 zero points (src/grimoire.cpp:1418-1434):
 * [out/8][groups] int32, row n in nibble n % 8; NULL = 8 for every group. */
void orc_int4_zero_unpack(const int32_t* zp, int out, int groups, uint8_t* zeros_out) {
    for (int n = 0; n < out; ++n)
        for (int g = 0; g < groups; ++g)
            zeros_out[(int64_t)n * groups + g] =
                zp ? (uint8_t)(((uint32_t)zp[(int64_t)(n / 8) * groups + g] >> (4 * (n % 8))) & 0xFu)
                   : (uint8_t)8;
}

/* src/grimoire.cpp:8386-8397: all zero points 8 -> payload ^= 0x88,
 * zeros = 0xFF.  Returns 1 when converted. */
int orc_int4_to_signed(uint8_t* gu, int64_t gu_bytes, uint8_t* gz, int64_t gz_bytes, uint8_t* dn,
                       int64_t dn_bytes, uint8_t* dz, int64_t dz_bytes) {
    for (int64_t i = 0; i < gz_bytes; ++i) if (gz[i] != 8) return 0;
    for (int64_t i = 0; i < dz_bytes; ++i) if (dz[i] != 8) return 0;
    for (int64_t i = 0; i < gu_bytes; ++i) gu[i] ^= 0x88;
    for (int64_t i = 0; i < dn_bytes; ++i) dn[i] ^= 0x88;
    memset(gz, 0xFF, (size_t)gz_bytes);
    memset(dz, 0xFF, (size_t)dz_bytes);
    return 1;
}

/* include/b70/formats.hpp:157-169 */
float orc_e4m3_to_f32(uint8_t b) {
    const uint32_t s = (uint32_t)(b & 0x80u) << 24;
    const int e = (b >> 3) & 0xF, m = b & 7;
    if (e == 0xF && m == 7) return bits_f(0x7FC00000u | s);
    if (e == 0) {
        const float v = (float)m * (1.0f / 8.0f) * 0.015625f;
        return s ? -v : v;
    }
    return bits_f(s | ((uint32_t)(e - 7 + 127) << 23) | ((uint32_t)m << 20));
}

/* nvfp4_dequant_row (include/b70/nvfp4.hpp): mul = 1 multiplies by gscale. */
void orc_nvfp4_dequant_row(const uint8_t* packed, const uint8_t* scales, float gscale, int K,
                           float* out, int mul) {
    for (int k = 0; k < K; ++k) {
        const uint8_t byte = packed[k >> 1];
        const uint8_t nib = (k & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0x0F);
        const float blk = orc_e4m3_to_f32(scales[k / 16]);
        out[k] = mul ? orc_e2m1_to_f32(nib) * blk * gscale : orc_e2m1_to_f32(nib) * blk / gscale;
    }
}

/* NvExpertLayout::make (include/b70/tiered_moe.hpp:40-60) */
void orc_tmoe_layout(int H, int I, int64_t* off /* gu_p gu_s dn_p dn_s gsc bytes */) {
    int64_t o = 0;
    off[0] = o; o += (int64_t)2 * I * (H / 2);
    off[1] = o; o += (int64_t)2 * I * (H / 16);
    off[2] = o; o += (int64_t)H * (I / 2);
    off[3] = o; o += (int64_t)H * (I / 16);
    off[4] = o; o += 16;
    off[5] = (o + 4095) & ~(int64_t)4095;
}

/* nv_dot32 (src/tiered_moe.cpp:45-61): two 16-element fma chains, each
 * scaled by its E4M3 block scale. */
static float orc_nv_dot32(const uint8_t* p, const uint8_t* s, const float* x) {
    float a0 = 0.0f, a1 = 0.0f;
    for (int k = 0; k < 16; ++k) {
        const uint8_t nib = (k & 1) ? (uint8_t)(p[k >> 1] >> 4) : (uint8_t)(p[k >> 1] & 15);
        a0 = fmaf(orc_e2m1_to_f32(nib), x[k], a0);
    }
    for (int k = 16; k < 32; ++k) {
        const uint8_t nib = (k & 1) ? (uint8_t)(p[k >> 1] >> 4) : (uint8_t)(p[k >> 1] & 15);
        a1 = fmaf(orc_e2m1_to_f32(nib), x[k], a1);
    }
    return a0 * orc_e4m3_to_f32(s[0]) + a1 * orc_e4m3_to_f32(s[1]);
}

static float orc_nv_row(const uint8_t* p, const uint8_t* s, const float* x, int K) {
    float acc = 0.0f;
    for (int c = 0; c < K / 32; ++c) acc += orc_nv_dot32(p + c * 16, s + c * 2, x + c * 32);
    return acc;
}

/* launch_tmoe_gate_up (src/tiered_moe.cpp:88-176): blocks[e] host copies. */
void orc_tmoe_gate_up(const uint8_t* const* blocks, int H, int I, int K, int E,
                      const int32_t* expert, const float* x, float* h, int M) {
    int64_t off[6];
    orc_tmoe_layout(H, I, off);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < M; ++t)
        for (int sr = 0; sr < K * I; ++sr) {
            const int slot = sr / I, i = sr % I;
            const int e = expert[(int64_t)t * K + slot];
            float v = 0.0f;
            if (e >= 0 && e < E) {
                const uint8_t* b = blocks[e];
                const float* g3 = (const float*)(b + off[4]);
                const float g = orc_nv_row(b + off[0] + (int64_t)i * (H / 2),
                                           b + off[1] + (int64_t)i * (H / 16), x + (int64_t)t * H, H);
                const float u = orc_nv_row(b + off[0] + (int64_t)(I + i) * (H / 2),
                                           b + off[1] + (int64_t)(I + i) * (H / 16),
                                           x + (int64_t)t * H, H);
                v = silu_f(g * g3[0]) * (u * g3[1]);
            }
            h[(int64_t)t * K * I + sr] = v;
        }
}

/* launch_tmoe_down (src/tiered_moe.cpp:187-278) */
void orc_tmoe_down(const uint8_t* const* blocks, int H, int I, int K, int E,
                   const int32_t* expert, const float* weight, const float* h, float* y, int M) {
    int64_t off[6];
    orc_tmoe_layout(H, I, off);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < M; ++t)
        for (int o = 0; o < H; ++o) {
            float total = 0.0f;
            for (int s = 0; s < K; ++s) {
                const int e = expert[(int64_t)t * K + s];
                const float rw = weight[(int64_t)t * K + s];
                if (e < 0 || e >= E || rw == 0.0f) continue;
                const uint8_t* b = blocks[e];
                const float sd = ((const float*)(b + off[4]))[2];
                const float acc = orc_nv_row(b + off[2] + (int64_t)o * (I / 2),
                                             b + off[3] + (int64_t)o * (I / 16),
                                             h + (int64_t)t * K * I + (int64_t)s * I, I);
                total = fmaf(rw * sd, acc, total);
            }
            y[(int64_t)t * H + o] = total;
        }
}

/* src/gemm_fast.cpp:1603-1800 contract (EPI 0 / EPI 1) */
void orc_grouped_gemm(const grim_quant_weight* w, int N, int swiglu, const float* A,
                      float* out, const int32_t* offsets, const int32_t* counts,
                      int n_experts) {
    const int K = w->K;
    const int NO = swiglu ? N / 2 : N;
    for (int e = 0; e < n_experts; ++e) {
        const int r0 = offsets[e], nr = counts[e];
#pragma omp parallel for schedule(dynamic)
        for (int j = 0; j < nr; ++j) {
            const float* a = A + (int64_t)(r0 + j) * K;
            float* o = out + (int64_t)(r0 + j) * NO;
            for (int n = 0; n < NO; ++n) {
                if (swiglu) {
                    o[n] = swiglu_row(w, (int64_t)e * N + n, (int64_t)e * N + NO + n, K, a);
                } else {
                    double acc = 0.0;
                    for (int k = 0; k < K; ++k)
                        acc += (double)orc_qw_at(w, (int)((int64_t)e * N + n), k) * a[k];
                    o[n] = (float)acc;
                }
            }
        }
    }
}
