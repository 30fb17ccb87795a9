/*
 * moe_oracle.h -- CPU restatement of GRIMOIRE's MoE layer.
 *
 * TEST INFRASTRUCTURE ONLY.  This code is the checker the HIP path is
 * compared against: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product library never links it and
 * has no CPU fallback.
 *
 * Every function cites the reference file:line whose semantics it restates
 * (paths relative to the reference tree).  Arithmetic is scalar C with
 * double accumulation where the reference's oracle uses it
 * (src/moe_ref.cpp), compiled with -ffp-contract=off so that what is
 * written is what is computed.
 */
#ifndef GRIMOIRE_MOE_ORACLE_H
#define GRIMOIRE_MOE_ORACLE_H

#include <stdint.h>
#include "../include/grimoire_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Scalar decodes (include/b70/formats.hpp:72-126). */
float orc_f16_to_f32(uint16_t h);
float orc_bf16_to_f32(uint16_t b);
uint16_t orc_f32_to_bf16(float f);
float orc_e8m0_to_f32(uint8_t x);
float orc_e2m1_to_f32(uint8_t nib);

/* Deterministic exp and sigmoid shared (as an algorithm, restated in each
 * code base) by the oracle and the device kernels, so that router scores
 * and weights can be compared bit for bit. */
float orc_expf(float x);
float orc_sigmoid(float x);

/* Dequantised weight element w[n][k] (include/b70/weights.hpp:102-121). */
float orc_qw_at(const grim_quant_weight* w, int n, int k);

/* GPTQ element (include/b70/gptq.hpp:80-91): qweight [in/8][out],
 * qzeros [in/group][out/8], scales fp16 [in/group][out]. */
float orc_gptq_at(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                  int in, int out, int group, int o, int k);

/* route_ref (src/moe_ref.cpp:30-63): softmax over all experts, top-k by
 * probability (lower index on ties), renormalise in double. */
void orc_route_ref(const float* logits, int n_experts, int top_k, int norm_topk,
                   int32_t* out_expert, float* out_weight);

/* Device top-k semantics (src/ops.cpp:1100-1201, :1347-1422): rank on raw
 * logits, lowest index among equals; softmax over the picks. batched != 0
 * with normalize == 0 returns raw pick logits (ops.cpp:1395-1409). */
void orc_topk_softmax(const float* logits, int tokens, int n_experts, int top_k, int normalize,
                      int batched, int32_t* out_expert, float* out_weight);

/* Sigmoid + selection-only bias (src/ops.cpp:2059-2170). bias bf16 or NULL. */
void orc_topk_sigmoid(const float* logits, const uint16_t* bias_bf16, int tokens, int n_experts,
                      int top_k, int normalize, float scaling, int32_t* out_expert,
                      float* out_weight);

/* Group-limited sigmoid top-k (DeepSeek-V3 definition; no reference code). */
void orc_topk_group(const float* logits, const float* bias, int tokens, int n_experts, int top_k,
                    int n_group, int topk_group, int normalize, float scaling,
                    int32_t* out_expert, float* out_weight);

/* Router GEMV (src/grimoire.cpp:15364), double accumulation. */
void orc_router_logits(const float* router, const float* x, float* logits, int tokens,
                       int n_experts, int hidden);

/* Fused decode gate_up (src/moe_kernels.cpp:82-257): h [T][KS][I] with the
 * shared expert (ws, may be NULL) as slot K; gate_out[t] = sigmoid(x.gate_w)
 * when gate_w != NULL.  Double dots as src/moe_ref.cpp:68-86. */
void orc_gate_up(const grim_moe_layer* L, const grim_quant_weight* ws, const uint16_t* gate_w,
                 const int32_t* rex, const float* x, float* h, float* gate_out, int tokens);

/* Fused decode down (src/moe_kernels.cpp:273-445): y[t][o] =
 * sum_s w*(down_e[o].h_s) (+ g * shared). Skips e < 0 or w == 0. */
void orc_down(const grim_moe_layer* L, const grim_quant_weight* wd, const int32_t* rex,
              const float* rwt, const float* gate_in, const float* h, float* y, int tokens);

/* moe_forward_ref (src/moe_ref.cpp:88-105) for T tokens with the routing
 * given; the shared expert (L->has_shared) is weighted by gate[t] when
 * gate != NULL (moe_kernels.cpp:1278 form), else 1. OpenMP over tokens. */
void orc_moe_forward(const grim_moe_layer* L, const int32_t* rex, const float* rwt,
                     const float* gate, const float* x, float* y, int tokens);

/* Stable counting-sort dispatch (src/grimoire.cpp:23162-23170) plus the
 * tile table of src/prefill.cpp:2770-2782.  Routes with an id outside
 * [0, E) get inverse -1 and are not counted.  Returns the tile count. */
int orc_dispatch(const int32_t* topk_ids, int tokens, int top_k, int n_experts, int mc,
                 int32_t* counts, int32_t* offsets, int32_t* inverse, int32_t* perm_token,
                 int32_t* tile_e, int32_t* tile_mb, int tmax);

/* launch_moe_unpermute (src/prefill.cpp:2654-2668): fma chain, slot order. */
void orc_unpermute(const float* src, const int32_t* inverse, const float* route_weight,
                   float* dst, int tokens, int top_k, int hidden);

/* launch_rmsnorm_moe_residual_batched (src/prefill.cpp:1004-1045): h +=
 * shared + fma chain over slots of w * bf16 routed[inverse]; out (fp32
 * and/or bf16, either may be NULL) = h * rsqrt(mean h^2 + eps) *
 * (weight_offset + bf16 weight). */
void orc_rmsnorm_moe_residual(float* h, const uint16_t* routed, const int32_t* inverse,
                              const float* route_weight, const float* shared,
                              const uint16_t* weight, float weight_offset, float* out,
                              uint16_t* out_bf, int tokens, int top_k, int hidden, float eps);

/* launch_rmsnorm_residual_batched (src/prefill.cpp:627-700), ungrouped:
 * h = (h + r0) + r1 (NULL addends skipped), out = rmsnorm(h) *
 * (weight_offset + bf16 weight). */
void orc_rmsnorm_residual(float* h, const float* r0, const float* r1, const uint16_t* weight,
                          float weight_offset, float* out, uint16_t* out_bf, int tokens,
                          int hidden, float eps);

/* gptq_repack_int4 (src/gptq.cpp:56-83); keep_f16 keeps the fp16 scale bits. */
void orc_gptq_repack(const int32_t* qweight, const int32_t* qzeros, const uint16_t* scales,
                     int in, int out, int group, int keep_f16, uint8_t* payload,
                     uint16_t* scales_out, uint8_t* zeros_out);
/* compressed-tensors INT4 zero points (src/grimoire.cpp:1418-1434). */
void orc_int4_zero_unpack(const int32_t* zp, int out, int groups, uint8_t* zeros_out);
/* signed-s4 conversion (src/grimoire.cpp:8386-8397); 1 when converted. */
int orc_int4_to_signed(uint8_t* gu, int64_t gu_bytes, uint8_t* gz, int64_t gz_bytes, uint8_t* dn,
                       int64_t dn_bytes, uint8_t* dz, int64_t dz_bytes);

/* Tiered NVFP4 experts (include/b70/nvfp4.hpp, tiered_moe.hpp,
 * src/tiered_moe.cpp); blocks[e] are host copies of the expert blocks. */
float orc_e4m3_to_f32(uint8_t b);
void orc_nvfp4_dequant_row(const uint8_t* packed, const uint8_t* scales, float gscale, int K,
                           float* out, int mul);
void orc_tmoe_layout(int H, int I, int64_t* off);
void orc_tmoe_gate_up(const uint8_t* const* blocks, int H, int I, int K, int E,
                      const int32_t* expert, const float* x, float* h, int M);
void orc_tmoe_down(const uint8_t* const* blocks, int H, int I, int K, int E,
                   const int32_t* expert, const float* weight, const float* h, float* y, int M);

/* Grouped GEMM (src/gemm_fast.cpp:1603-1800 contract): rows [off_e,
 * off_e+cnt_e) of A (fp32 values) times W_e^T; swiglu gives silu(g)*u over
 * N = 2I. out fp32 [R][N or I]. Double accumulation. */
void orc_grouped_gemm(const grim_quant_weight* w, int N, int swiglu, const float* A,
                      float* out, const int32_t* offsets, const int32_t* counts,
                      int n_experts);

#ifdef __cplusplus
}
#endif
#endif
