/*
 * grimoire_moe.h -- C ABI of the MI355X (gfx950) mixture-of-experts layer.
 *
 * Drop-in for the MoE launchers and bridges of doopeworld/GRIMOIRE.  Every
 * entry point below names the reference interface it replaces (file:line in
 * the reference tree).  Differences that apply to all of them:
 *
 *   - `sycl::queue&` / `sycl::queue*` becomes `void* stream` (a hipStream_t;
 *     NULL = the default stream).  Work is ordered by the stream.
 *   - the returned `sycl::event` becomes an int status: 0 on success, a
 *     positive hipError_t when a launch failed, GRIM_ERR_* (negative) when
 *     the arguments were rejected before anything was launched.  The
 *     reference returns an empty event for an unknown format
 *     (src/moe_kernels.cpp:1243) and throws std::runtime_error for an
 *     unsupported grouped shape (src/gemm_fast.cpp:2312); both map to a
 *     negative status here, with the reason in grimoire_moe_last_error().
 *   - `const std::vector<sycl::event>& deps` disappears: stream order.
 *   - No entry point allocates device memory except where stated; scratch
 *     (h, xperm, tables) is caller-owned exactly as in the reference
 *     (include/b70/weights.hpp:22-25).
 *
 * All pointers are device pointers unless stated otherwise.  Layouts are the
 * reference's: expert-major packed experts, gate_up [E*2I][H] (gate rows
 * [e*2I, e*2I+I), up rows [e*2I+I, (e+1)*2I)), down [E*H][I]
 * (include/b70/moe.hpp:47-56, :100-102).
 */
#ifndef GRIMOIRE_MOE_H
#define GRIMOIRE_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

/* ------------------------------------------------------------------------
 * Weight formats.  Codes 0..6 keep the numbering of the reference's
 * `enum class Fmt` (include/b70/formats.hpp:237-239).  GRIM_FMT_INT4_F16 is
 * new: GPTQ int4 with the checkpoint's IEEE fp16 group scales kept exactly
 * (the reference rounds them to bf16 at repack, src/gptq.cpp:65-66).
 *
 *   BF16       payload [N][2K]                     scales unused
 *   INT8       payload [N][K] int8                 scales float [N]
 *   INT4       payload [N][K/2] (low nibble = even k)
 *              scales bf16 [N][K/G], zeros u8 [N][K/G]; value (q - z) * s,
 *              or signed s4 * s when z == 0xff (formats.hpp:483-491);
 *              zeros == NULL means z = 0.  G = 128 (or 32/64/256, derived
 *              from row_scales as weights.hpp:80-84 does).
 *   INT4_F16   as INT4 with fp16 scales; zeros == NULL means the symmetric
 *              GPTQ zero point 8 (AutoGPTQ's stored 7, plus its +1).
 *   MXFP4      payload [N][K/2] e2m1 (low nibble = even k),
 *              scales e8m0 u8 [N][K/32] (formats.hpp:105-126).
 * ---------------------------------------------------------------------- */
enum grim_fmt {
    GRIM_FMT_BF16 = 0,
    GRIM_FMT_INT8 = 3,
    GRIM_FMT_INT4 = 4,
    GRIM_FMT_MXFP4 = 6,
    GRIM_FMT_INT4_F16 = 64
};

/* Error codes (negative; positive values are hipError_t). */
enum grim_status {
    GRIM_OK = 0,
    GRIM_ERR_FORMAT = -1,      /* weight format not supported here        */
    GRIM_ERR_SHAPE = -2,       /* shape outside what the kernels support  */
    GRIM_ERR_ARG = -3,         /* null pointer or inconsistent argument   */
    GRIM_ERR_WORKSPACE = -4    /* workspace too small                     */
};

/* Flat weight view, no ownership: mirrors b70::QuantWeight
 * (include/b70/weights.hpp:46-126) field for field. */
typedef struct grim_quant_weight {
    int32_t fmt;               /* enum grim_fmt                            */
    int32_t N;                 /* output features                          */
    int32_t K;                 /* input features                           */
    int32_t row_scales;        /* scales per row                           */
    int64_t row_bytes;         /* payload bytes per row                    */
    const uint8_t* payload;
    const void* scales;
    const uint8_t* zeros;
} grim_quant_weight;

/* b70::MoeConfig (include/b70/moe.hpp:70-77). */
typedef struct grim_moe_config {
    int32_t hidden;            /* H */
    int32_t inter;             /* I */
    int32_t num_experts;       /* E */
    int32_t top_k;             /* K <= 16 */
    int32_t shared_inter;      /* SI, 0 if none */
    int32_t norm_topk;         /* renormalise the picked weights */
} grim_moe_config;

/* b70::MoeLayer (include/b70/moe.hpp:85-117). */
typedef struct grim_moe_layer {
    grim_moe_config cfg;
    grim_quant_weight gate_up;          /* [E*2I][H] */
    grim_quant_weight down;             /* [E*H][I]  */
    int32_t has_shared;
    int32_t _pad;
    grim_quant_weight shared_gate_up;   /* [2*SI][H] */
    grim_quant_weight shared_down;      /* [H][SI]   */
    const float* router;                /* fp32 [E][H] */
} grim_moe_layer;

/* Text of the last argument rejection on this thread ("" if none). */
const char* grimoire_moe_last_error(void);
/* Library version string. */
const char* grimoire_moe_version(void);

/* ------------------------------------------------------------------------
 * Router
 * ---------------------------------------------------------------------- */

/* logits[t][e] = sum_k router[e][k] * x[t][k], fp32.  Replaces the router
 * GEMV gemv_any(d.router, s.h2, s.rlogits) (src/grimoire.cpp:15364) and the
 * prefill router GEMM (src/grimoire.cpp:22774). */
int grimoire_moe_router_logits(void* stream, const float* router, const float* x,
                               float* logits, int tokens, int n_experts, int hidden);

/* Softmax top-k on raw logits for one token: picks = max logit, lowest index
 * among equals; weights = softmax over the picks in pick order, divided by
 * their sum when `normalize`, else the unnormalised exp(l - max).
 * Replaces launch_router_topk (src/ops.cpp:1205-1344). */
int grimoire_moe_router_topk(void* stream, const float* logits, int n_experts, int top_k,
                             int32_t* out_expert, float* out_weight, int normalize);

/* The same for `tokens` rows, [T][E] -> [T][K].  As the reference's batched
 * kernel (src/ops.cpp:1347-1422), normalize == 0 returns the raw logits of
 * the picks. */
int grimoire_moe_router_topk_batched(void* stream, const float* logits, int tokens,
                                     int n_experts, int top_k, int32_t* out_expert,
                                     float* out_weight, int normalize);

/* The batched top-k on bf16 logits [T][E] (widened exactly to fp32; same
 * picks, ties and weights as grimoire_moe_router_topk_batched).  Replaces
 * launch_router_topk_bf16_batched (src/ops.cpp:1425). */
int grimoire_moe_router_topk_bf16_batched(void* stream, const uint16_t* logits, int tokens,
                                          int n_experts, int top_k, int32_t* out_expert,
                                          float* out_weight, int normalize);

/* Sigmoid scoring with a selection-only bf16 bias (may be NULL): rank on
 * sigmoid(l) + bias[e], weight = unbiased sigmoid(l), divided by the sum of
 * the picks when `normalize`, then multiplied by `scaling`.
 * Replaces launch_router_topk_k2 (src/ops.cpp:2059-2170). */
int grimoire_moe_router_topk_sigmoid(void* stream, const float* logits,
                                     const uint16_t* bias_bf16, int tokens, int n_experts,
                                     int top_k, int32_t* out_expert, float* out_weight,
                                     int normalize, float scaling);

/* Group-limited sigmoid top-k (DeepSeek-V3 routing; no counterpart in the
 * reference).  bias is fp32 [E] (may be NULL).  s = sigmoid(l), s' = s + b;
 * group score = sum of the two largest s' in each of n_group contiguous
 * groups; keep the topk_group best groups (lower group index wins ties);
 * pick top_k over s' of the kept experts (lower index wins ties); weight =
 * s, divided by the sum when `normalize`, times `scaling`. */
int grimoire_moe_router_topk_group(void* stream, const float* logits, const float* bias,
                                   int tokens, int n_experts, int top_k, int n_group,
                                   int topk_group, int32_t* out_expert, float* out_weight,
                                   int normalize, float scaling);

/* ------------------------------------------------------------------------
 * Decode / batched-decode expert products (slot form).  h holds
 * [M][KS][I] fp32, KS = top_k (+1 with the shared expert, whose
 * intermediate must equal I).  d_expert/d_weight are [M][top_k]; a route
 * with expert < 0 or weight == 0 is skipped by down.
 * ---------------------------------------------------------------------- */

/* h[t][s][i] = silu(gate_e[i] . x_t) * (up_e[i] . x_t), e = d_expert[t][s].
 * Replaces launch_moe_gate_up (src/moe_kernels.cpp:1225). */
int grimoire_moe_gate_up(void* stream, const grim_moe_layer* L, const int32_t* d_expert,
                         const float* x, float* h);

/* y[t][o] = sum_s w[t][s] * (down_e[o] . h[t][s]).
 * Replaces launch_moe_down (src/moe_kernels.cpp:1350). */
int grimoire_moe_down(void* stream, const grim_moe_layer* L, const int32_t* d_expert,
                      const float* d_weight, const float* h, float* y);

/* gate_up with the shared expert as slot top_k (ws = [2I][H], same format
 * as the routed experts); gate_w (bf16 [H], may be NULL) gives
 * gate_out[t] = sigmoid(x_t . gate_w).
 * Replaces launch_moe_gate_up_shared (src/moe_kernels.cpp:1246). */
int grimoire_moe_gate_up_shared(void* stream, const grim_moe_layer* L,
                                const grim_quant_weight* ws, const uint16_t* gate_w,
                                const int32_t* d_expert, const float* x, float* h,
                                float* gate_out);

/* down with the shared expert (wd = [H][I]) weighted by gate_in[t] (1 when
 * NULL).  Replaces launch_moe_down_shared (src/moe_kernels.cpp:1278). */
int grimoire_moe_down_shared(void* stream, const grim_moe_layer* L,
                             const grim_quant_weight* wd, const int32_t* d_expert,
                             const float* d_weight, const float* gate_in, const float* h,
                             float* y);

/* M-token forms.  Replace launch_moe_gate_up_batched / launch_moe_down_batched
 * (src/moe_kernels.cpp:1372, :1394). */
int grimoire_moe_gate_up_batched(void* stream, const grim_moe_layer* L,
                                 const int32_t* d_expert, const float* x, float* h,
                                 int tokens);
int grimoire_moe_down_batched(void* stream, const grim_moe_layer* L, const int32_t* d_expert,
                              const float* d_weight, const float* h, float* y, int tokens);

/* Both products for M tokens with the shared expert fused (gate_w may be
 * NULL).  Replaces launch_moe_shared_rows (src/moe_kernels.cpp:1316). */
int grimoire_moe_shared_rows(void* stream, const grim_moe_layer* L,
                             const grim_quant_weight* ws, const grim_quant_weight* wd,
                             const uint16_t* gate_w, const int32_t* rex, const float* rwt,
                             const float* x, float* h, float* gate_out, float* y, int M);

/* ------------------------------------------------------------------------
 * Dispatch (prefill / verify).  The permutation is deterministic and
 * stable: expert-major, ascending route index r = t*top_k + s, the order
 * of the reference's host counting sort (src/grimoire.cpp:23162-23170).
 * The reference's device kernels use atomic arrival order instead
 * (src/prefill.cpp:2721-2725).
 * ---------------------------------------------------------------------- */

/* Bytes of device workspace grimoire_moe_route_grouped needs. */
size_t grimoire_moe_route_workspace_bytes(int tokens, int top_k, int num_experts);

/* counts[E], offsets[E] (exclusive scan), inverse[T*K] = absolute permuted
 * row of route r, xperm bf16 [T*K][H] = bf16(hidden[t]) at each permuted
 * row, xrow bf16 [T][H] (may be NULL) = the unpermuted bf16 copy, and the
 * m-tile table tile_e/tile_mb [tmax] (expert, tile index) padded with -1.
 * Replaces launch_moe_route_grouped (src/prefill.cpp:2726-2808), whose
 * TOPK is fixed at 8; here top_k is the trailing argument.  perm_token
 * (may be NULL) receives the token of each permuted row. */
int grimoire_moe_route_grouped(void* stream, const float* hidden, const int32_t* topk_ids,
                               uint16_t* xperm, uint16_t* xrow, int32_t* counts,
                               int32_t* offsets, int32_t* inverse, int32_t* tile_e,
                               int32_t* tile_mb, int tmax, int tokens, int hidden_size,
                               int num_experts, int mc, int top_k, int32_t* perm_token,
                               void* workspace, size_t workspace_bytes);

/* The same without tile table from bf16 hidden states (vLLM
 * RowsPerExpertCount / RemapHiddenStates form).  Replaces
 * launch_moe_remap_bf16_top8 (src/prefill.cpp:2810-2890). */
int grimoire_moe_remap_bf16(void* stream, const uint16_t* hidden, const int32_t* topk_ids,
                            uint16_t* remapped, int32_t* rows_per_expert,
                            int32_t* expert_offsets, int32_t* inverse, int tokens,
                            int hidden_size, int num_experts, int top_k, void* workspace,
                            size_t workspace_bytes);

/* dst[t][d] = sum_s w[t,s] * src[inverse[t,s]][d] as an fma chain in slot
 * order; inverse -1 = route not computed here.  Replaces
 * launch_moe_unpermute (src/prefill.cpp:2654). */
int grimoire_moe_unpermute(void* stream, const float* src, const int32_t* inverse,
                           const float* route_weight, float* dst, int tokens, int top_k,
                           int hidden);
/* bf16 source rows.  Replaces launch_moe_unpermute_bf16 (src/prefill.cpp:2690). */
int grimoire_moe_unpermute_bf16(void* stream, const uint16_t* src, const int32_t* inverse,
                                const float* route_weight, float* dst, int tokens,
                                int top_k, int hidden);

/* One route range of a grouped expert pass: a route whose dispatch row p
 * lies in [p0, p1) reads src row p - p0; dst = the fma chain over slots in
 * slot order, starting from 0, or from dst when accumulate != 0.  Replaces
 * launch_moe_unpermute_range (src/prefill.cpp:2674-2688). */
int grimoire_moe_unpermute_range(void* stream, const float* src, const int32_t* inverse,
                                 const float* route_weight, float* dst, int tokens, int top_k,
                                 int hidden, int p0, int p1, int accumulate);

/* dst[r] = bf16(src[perm_token[r]]) (round to nearest even) over `width`
 * columns.  Replaces launch_permute_rows_bf16 (src/prefill.cpp:2644). */
int grimoire_moe_permute_rows_bf16(void* stream, const float* src, const int32_t* perm_token,
                                   uint16_t* dst, int rows, int width);

/* out[t][d] = bf16(silu(g) * u), g = gu[t][d], u = gu[t][inter + d], all
 * bf16.  Replaces launch_swiglu_bf16 (src/prefill.cpp:2541). */
int grimoire_moe_swiglu_bf16(void* stream, const uint16_t* gu, uint16_t* out, int tokens,
                             int inter);

/* x[i] *= sigmoid(g[0]) over n elements (launch_scale_by_sigmoid,
 * src/ops.cpp:1491); the batched form scales row t by sigmoid(gate[t])
 * (launch_scale_by_sigmoid_batched, src/prefill.cpp:2610). */
int grimoire_moe_scale_by_sigmoid(void* stream, float* x, const float* g, int n);
int grimoire_moe_scale_by_sigmoid_batched(void* stream, float* x, const float* gate, int tokens,
                                          int hidden);

/* Combine with the gated shared expert: dst[t] = unpermute(...)[t] +
 * gate[t] * shared_src[t] (gate NULL = 1).  Replaces the unpermute plus the
 * shared-expert add of src/grimoire.cpp:23118 and :23247-23283. */
int grimoire_moe_combine(void* stream, const uint16_t* src, const int32_t* inverse,
                         const float* route_weight, const uint16_t* shared_src,
                         const float* gate, float* dst, int tokens, int top_k, int hidden);

/* Combine fused with the residual add and the next RMSNorm.  Per token t:
 * v = h[t] + shared[t] (shared NULL = 0), then v = fma(route_weight[t,s],
 * routed[inverse[t,s]], v) in slot order (inverse -1 skips the slot);
 * h[t] = v; out[t] = v * rsqrt(sum(v^2)/hidden + eps) * (weight_offset +
 * weight) in fp32 and/or bf16 (either output may be NULL).  routed and
 * weight are bf16; top_k <= 16; hidden % 4 == 0.  Replaces
 * launch_rmsnorm_moe_residual_batched (src/prefill.cpp:1004-1045), whose
 * weight offset is the global g_norm_weight_offset
 * (include/b70/prefill_qk_math.hpp:9-15): pass its value. */
int grimoire_moe_rmsnorm_residual(void* stream, float* h, const uint16_t* routed,
                                  const int32_t* inverse, const float* route_weight,
                                  const float* shared, const uint16_t* weight,
                                  float weight_offset, float* out, uint16_t* out_bf,
                                  int tokens, int top_k, int hidden, float eps);

/* The residual RMSNorm that feeds the router: v = (h[t] + r0[t]) + r1[t]
 * (either addend may be NULL; h is written back only when one is given);
 * out[t] = v * rsqrt(sum(v^2)/hidden + eps) * (weight_offset + weight), fp32
 * and/or bf16.  hidden % 4 == 0.  Replaces launch_rmsnorm_residual_batched
 * (src/prefill.cpp:627-700) for ungrouped norms (its grouped-norm branch,
 * launch_rmsnorm_grouped, is not covered). */
int grimoire_rmsnorm_residual(void* stream, float* h, const float* r0, const float* r1,
                              const uint16_t* weight, float weight_offset, float* out,
                              uint16_t* out_bf, int tokens, int hidden, float eps);

/* ------------------------------------------------------------------------
 * Expert-weight ingestion: one checkpoint projection [out][in] of one expert
 * into rows [row0, row0 + out) of a stacked weight, the per-expert staging
 * of src/grimoire.cpp:8340-8383 (gate at expert*2I, up at expert*2I + I in
 * gate_up; down at expert*H).
 *
 *   GRIM_SRC_GPTQ           weight = qweight int32 [in/8][out] (8 nibbles
 *                           along in), zeros = qzeros int32 [in/g][out/8]
 *                           (8 nibbles along out), scales = fp16 [in/g][out]
 *                           (include/b70/gptq.hpp:21-55).  dst INT4: the
 *                           repack of gptq_repack_int4 (src/gptq.cpp:56-83),
 *                           scales rounded to bf16, zeros = stored + 1.
 *                           dst INT4_F16: the same with the fp16 scales kept.
 *                           dst->zeros required.
 *   GRIM_SRC_MXFP4_PACKED   compressed-tensors weight_packed u8 [out][in/2]
 *                           and weight_scale e8m0 u8 [out][in/32], copied as
 *                           stored (src/grimoire.cpp:8355-8367).  dst MXFP4.
 *   GRIM_SRC_INT4_PACKED    compressed-tensors pack-quantized INT4: weight
 *                           u8 [out][in/2] (offset binary, +8), scales bf16
 *                           [out][in/g], zeros = weight_zero_point int32
 *                           [out/8][in/g] (row n in nibble n % 8) or NULL for
 *                           8 (read_compressed_int4_ref, src/grimoire.cpp:
 *                           1396-1434).  dst INT4 with dst->zeros.
 *
 * GPTQ and INT4 zero-point sources are read by kernels: device memory or
 * hipHostMalloc'd host memory.  Copied parts go through hipMemcpyAsync and
 * may be any host or device memory; every source must stay valid until the
 * stream has passed the call (synchronise before freeing or reusing it).  dst->row_bytes must be in/2 and
 * dst->row_scales in/g (in/32 for MXFP4).
 * ---------------------------------------------------------------------- */
enum grim_src_kind {
    GRIM_SRC_GPTQ = 1,
    GRIM_SRC_MXFP4_PACKED = 2,
    GRIM_SRC_INT4_PACKED = 3
};

typedef struct grim_expert_src {
    int32_t kind;              /* enum grim_src_kind                        */
    int32_t in;                /* input features (K)                        */
    int32_t out;               /* output features (N)                       */
    int32_t group;             /* quantisation group along in (GPTQ, INT4)  */
    const void* weight;
    const void* zeros;
    const void* scales;
} grim_expert_src;

int grimoire_moe_ingest_projection(void* stream, const grim_expert_src* src,
                                   const grim_quant_weight* dst, int row0);
/* n projections of one kind and shape (host arrays src[n], row0[n]) into
 * the same stacked weight, e.g. every expert's gate and up of a layer:
 * GPTQ sources go 64 per launch.  Same conversions and rules as above. */
int grimoire_moe_ingest_projections(void* stream, const grim_expert_src* srcs,
                                    const int32_t* row0, int n, const grim_quant_weight* dst);

/* MXFP4 rows padded for the matrix-core expert-grouped GEMV.  No
 * counterpart in the reference, whose MXFP4 rows are K/2 payload bytes and
 * K/32 scale bytes (formats.hpp:105-126); a layout of this library's own,
 * for callers that pad their MXFP4 experts once at load.  At K = 2880 a
 * row is 1440 bytes and every 128-byte piece the kernel streams straddles
 * two memory lines; padded to K' = grimoire_moe_mxfp4_padded_k(K) (K
 * rounded up to 256; 3072 there) every piece is one line and, with
 * K' % 512 == 0, the scale rows are 16-byte aligned.  The padded elements
 * hold zero codes under scale byte 127 (2^0): every product there is an
 * exact zero, so the layer's results are those of the unpadded rows.
 * grimoire_moe_forward takes a layer whose MXFP4 weights are all padded
 * (row_bytes = K'/2, row_scales = K'/32) on every regime but 5: the
 * expert-grouped GEMV on the vector ALU reads packed rows only, and regime
 * 5 returns GRIM_ERR_FORMAT for such a layer.
 *
 * grimoire_moe_mxfp4_padded_k returns K' (0 when K is not a positive
 * multiple of 32).  grimoire_moe_pad_mxfp4_rows copies src (any row
 * strides of at least K/2 and K/32) into dst (same fmt, N, K; dst->payload
 * and dst->scales device memory of dst->N rows of dst->row_bytes and
 * dst->row_scales bytes) and fills dst's elements past K as above;
 * stream-ordered, no allocation. */
int grimoire_moe_mxfp4_padded_k(int K);
int grimoire_moe_pad_mxfp4_rows(void* stream, const grim_quant_weight* src, const grim_quant_weight* dst);

/* Signed-s4 conversion of a layer's INT4 experts (src/grimoire.cpp:
 * 8386-8397): when every zero point in gu_zeros and dn_zeros is 8, XOR
 * every payload byte with 0x88 (offset binary -> two's complement) and set
 * every zero point to 0xFF, the "signed s4" marker; otherwise change
 * nothing.  *converted (device int32) receives 1 or 0.  Either region may
 * be empty (NULL, 0). */
int grimoire_moe_int4_to_signed(void* stream, uint8_t* gu_payload, size_t gu_bytes,
                                uint8_t* gu_zeros, size_t gu_zero_bytes, uint8_t* dn_payload,
                                size_t dn_bytes, uint8_t* dn_zeros, size_t dn_zero_bytes,
                                int32_t* converted);

/* ------------------------------------------------------------------------
 * Tiered experts (include/b70/tiered_moe.hpp): every routed expert of a
 * layer is one self-contained NVFP4 block, and a device array of block
 * pointers (one per expert) is all the kernels need, so a block may sit in
 * device memory or in pinned host memory (hipHostMalloc; read over PCIe).
 * Block layout, NvExpertLayout::make (tiered_moe.hpp:40-60):
 *   gu_p  gate|up payload [2I][H/2] (e2m1, low nibble = even element)
 *   gu_s  gate|up E4M3 scales [2I][H/16]
 *   dn_p  down payload [H][I/2];  dn_s  down E4M3 scales [H][I/16]
 *   gsc   four fp32 {gate, up, down, 0} projection scales (multipliers)
 *   bytes the block size rounded up to 4096.
 * ---------------------------------------------------------------------- */
typedef struct grim_nv_expert_layout {
    int32_t H, I;
    int64_t gu_p, gu_s, dn_p, dn_s, gsc, bytes;
} grim_nv_expert_layout;

/* b70::TieredMoeView (tiered_moe.hpp:63-67). */
typedef struct grim_tiered_moe_view {
    grim_nv_expert_layout lay;
    const uint8_t* const* eptr;  /* device array [E] of block pointers   */
    int32_t E;
    int32_t top_k;
} grim_tiered_moe_view;

/* NvExpertLayout::make; returns GRIM_ERR_SHAPE unless H and I are
 * multiples of 128 (NvExpertLayout::supported). */
int grimoire_tmoe_layout(int H, int I, grim_nv_expert_layout* out);

/* h[M][K*I] = silu(x W_gate^T * s_gate) * (x W_up^T * s_up) for each routed
 * slot; 0 for a slot whose id is < 0 or >= E (another tier's or rank's).
 * Replaces launch_tmoe_gate_up (src/tiered_moe.cpp:88-176, :292). */
int grimoire_tmoe_gate_up(void* stream, const grim_tiered_moe_view* v, const int32_t* d_expert,
                          const float* x, float* h, int M);
/* y[M][H] = sum over slots in slot order of (w * s_down) * (h_slot W_down^T),
 * slots with id < 0 or >= E or weight 0 skipped.  Replaces launch_tmoe_down
 * (src/tiered_moe.cpp:187-278, :300). */
int grimoire_tmoe_down(void* stream, const grim_tiered_moe_view* v, const int32_t* d_expert,
                       const float* d_weight, const float* h, float* y, int M);

/* Moves expert e of a layer to another tier: copies `bytes` from src_block
 * to dst_block (hipMemcpyAsync, any memory) and then stores dst_block into
 * eptr[e] on the device, in stream order (tiered_moe.hpp:21-22: "one block
 * copy plus one pointer store").  src_block NULL: pointer store only. */
int grimoire_tmoe_place(void* stream, const uint8_t** eptr, int e, uint8_t* dst_block,
                        const uint8_t* src_block, size_t bytes);

/* Prefill on one expert block (tiered_moe.hpp:83-107).  The caller's
 * device scratch holds grimoire_tmoe_scratch_bytes(L, M) bytes (the block
 * decoded to bf16, the fp32 gate|up rows of the FFN, two counters).
 *   expert_gemm: out[M][N] fp32 = A[M][K] (bf16 rows) x W^T, W = gate|up
 *     (gate_up = 1: N = 2I, K = H; columns [0, I) x s0, [I, 2I) x s1) or
 *     down (N = H, K = I; x s0).  Replaces launch_nvfp4_expert_gemm.
 *   expert_ffn: hbuf[M][I] = bf16(silu(s_g A W_g^T) * (s_u A W_u^T)),
 *     out[M][H] = s_d hbuf W_d^T.  Replaces launch_nvfp4_expert_ffn.
 * The block may be in device or pinned host memory; it is read once, by
 * the decode into the scratch. */
size_t grimoire_tmoe_scratch_bytes(const grim_nv_expert_layout* L, int M);
int grimoire_tmoe_expert_gemm(void* stream, const uint8_t* block, const grim_nv_expert_layout* L,
                              int gate_up, float s0, float s1, const uint16_t* A, float* out,
                              int M, void* scratch, size_t scratch_bytes);
int grimoire_tmoe_expert_ffn(void* stream, const uint8_t* block, const grim_nv_expert_layout* L,
                             float sg, float su, float sd, const uint16_t* A, uint16_t* hbuf,
                             float* out, int M, void* scratch, size_t scratch_bytes);

/* ------------------------------------------------------------------------
 * Host expert pool (include/b70/cpu_experts.hpp, src/cpu_experts.cpp):
 * NVFP4 expert blocks in host memory computed by host threads while the
 * GPU runs the resident ones; the caller adds the two partial sums.  Plain
 * fp32 on the exact dequantised weights; results do not depend on the
 * thread count.  A pool is used by one calling thread at a time.
 * ---------------------------------------------------------------------- */
typedef struct grim_cpu_experts grim_cpu_experts;

/* CpuExperts::start (cpu_experts.hpp:49-52): threads <= 0 = the hardware
 * threads - 1; the calling thread is worker 0.  cpus[t] (t >= 1, t <
 * ncpus) pins pool thread t; NULL = not pinned.  NULL on failure. */
grim_cpu_experts* grimoire_cpu_experts_create(int threads, const int32_t* cpus, int ncpus);
/* CpuExperts::stop / ~CpuExperts */
void grimoire_cpu_experts_destroy(grim_cpu_experts* p);
/* CpuExperts::threads, CpuExperts::wait_us (microseconds the caller spent
 * waiting for workers after its own share, summed over calls) */
int grimoire_cpu_experts_threads(const grim_cpu_experts* p);
double grimoire_cpu_experts_wait_us(const grim_cpu_experts* p);
/* CpuExperts::ffn (cpu_experts.hpp:58-61): y[H] = sum over j < n in order
 * of (w[j] s_down_j) down_j(silu(s_gate_j gate_j x) * (s_up_j up_j x)),
 * blocks[j] host pointers (layout grim_nv_expert_layout).  Overwrites y;
 * n = 0 gives zeros. */
int grimoire_cpu_experts_ffn(grim_cpu_experts* p, const grim_nv_expert_layout* L,
                             const uint8_t* const* blocks, const float* w, int n, const float* x,
                             float* y);
/* CpuExperts::ffn_rows (cpu_experts.hpp:62-66): row r's experts are
 * blocks[off[r] .. off[r + 1]) with weights w[same], input x + r H, output
 * y + r H; each row bit-identical to grimoire_cpu_experts_ffn on it, and a
 * block several rows route to is read once.  off[0] = 0, rows + 1 entries. */
int grimoire_cpu_experts_ffn_rows(grim_cpu_experts* p, const grim_nv_expert_layout* L, int rows,
                                  const uint8_t* const* blocks, const float* w, const int32_t* off,
                                  const float* x, float* y);
/* cpu_nvfp4_dot (cpu_experts.hpp:90): one NVFP4 row of K elements (K % 64
 * == 0; else NaN) dotted with x. */
float grimoire_cpu_nvfp4_dot(const uint8_t* pay, const uint8_t* scl, const float* x, int K);
/* Instruction set of the host dot product: 0 scalar, 1 AVX2, 2 AVX-512, -1
 * the best this CPU has (the default).  All give the same bits; for tests.
 * GRIM_ERR_ARG if the CPU lacks it.  No reference counterpart. */
int grimoire_cpu_set_isa(int isa);
/* hybrid_pool_cpus (cpu_experts.hpp:93-97), for a CPU that is not hybrid:
 * rank's contiguous share of the CPUs this process may run on, written to
 * out (at most cap); returns how many are in the share. */
int grimoire_cpu_pool_cpus(int ranks, int rank, int32_t* out, int cap);

/* Expert heat and tier placement (include/b70/expert_heat.hpp). */
typedef struct grim_heat_params {
    float decay;               /* per call of a layer, 0.95              */
    float hysteresis;          /* promote if hot >= cold * h + min_gain  */
    float min_gain;
    float credit_cap;          /* most credited selections per call      */
    int32_t moves_per_step;
} grim_heat_params;

typedef struct grim_expert_swap {
    int32_t promote_layer, promote_expert;   /* to device memory */
    int32_t demote_layer, demote_expert;     /* to pinned host   */
} grim_expert_swap;

typedef struct grim_heat grim_heat;

void grimoire_heat_default_params(grim_heat_params* p);
grim_heat* grimoire_heat_create(int layers, int experts, const grim_heat_params* params);
void grimoire_heat_destroy(grim_heat* s);
/* ExpertHeat::credit: one call of `layer` with its n routes (host ids). */
void grimoire_heat_credit(grim_heat* s, int layer, const int32_t* ids, size_t n);
float grimoire_heat_get(const grim_heat* s, int layer, int expert);
/* ExpertHeat::propose over host flags resident[L*E] and movable[L*E]
 * (NULL = all movable); writes at most min(moves_per_step, max_out) swaps,
 * returns their count. */
int grimoire_heat_propose(const grim_heat* s, const uint8_t* resident, const uint8_t* movable,
                          grim_expert_swap* out, int max_out);

/* ------------------------------------------------------------------------
 * Grouped GEMM on MFMA (prefill).  One launch per projection for all
 * experts.  A bf16 [R][K] rows grouped by expert (offsets/counts from the
 * dispatch), W the packed expert weight [E*N][K].
 *   swiglu != 0: N = 2I; out[r][i] = silu(A_r . gate_e[i]) * (A_r . up_e[i])
 *                 written as a bf16 pair (hi, lo) with hi + lo = h to
 *                 within 2^-17 relative: out is uint16_t [R][2][I]
 *                 (hi row then lo row).
 *   swiglu == 0: out[r][n] = A_r . W_e[n]; A may be a bf16 pair [R][2][K]
 *                 (a_pair != 0), out is bf16 [R][N] (out_bf16 != 0) or
 *                 fp32 [R][N].
 * Replaces launch_moe_mxfp4_grouped (src/gemm_fast.cpp:2343-2365) and, with
 * the tile table, gemm_mxfp4_fused_grouped (src/gemm_fast.cpp:1603).  The
 * work-groups form the tile order from counts themselves (num_experts <=
 * 1024); nothing is allocated. */
int grimoire_moe_grouped_gemm(void* stream, const grim_quant_weight* w, int N, int swiglu,
                              const uint16_t* A, int a_pair, void* out, int out_bf16,
                              const int32_t* offsets, const int32_t* counts,
                              int num_experts, int total_rows);

/* INT8 weights on the int8 MFMA.  Activation rows are first split into
 * two int8 limbs under one fp32 scale per row, a = s * (hi + lo / 254),
 * s = max|row| / 127 (grimoire_moe_quant_limbs); each limb row is stored
 * [n/64][2][64] bytes (per 64 elements: the hi codes, then the lo codes).
 * src fp32 [rows][n] (n % 64 == 0, n <= 4096) -> dst [rows][2n], scale [rows].
 * No reference counterpart: the activation format of the kernel below. */
int grimoire_moe_quant_limbs(void* stream, const float* src, int rows, int n, int8_t* dst,
                             float* scale);

/* Grouped GEMM for INT8 weights (w->fmt GRIM_FMT_INT8, fp32 per-row scales)
 * on limb rows A [R][2K] with scales a_scale [R], grouped by expert
 * (offsets / counts [num_experts]) and walked through the caller's
 * (expert, 128-row m-block) tile table tile_e / tile_mb [tmax], -1 padded
 * (as the dispatch writes it); out fp32: swiglu != 0 -> h [R][N/2] =
 * silu(A_r . gate_e) * (A_r . up_e), else [R][N].  The computation of
 * launch_moe_mxfp4_grouped (src/gemm_fast.cpp:2343-2365, which takes the
 * same tile table) for the INT8 experts that the reference runs one expert
 * at a time (src/grimoire.cpp:23214-23229).  Allocates nothing. */
int grimoire_moe_grouped_gemm_i8(void* stream, const grim_quant_weight* w, int N, int swiglu,
                                 const int8_t* A, const float* a_scale, float* out,
                                 const int32_t* offsets, const int32_t* counts,
                                 const int32_t* tile_e, const int32_t* tile_mb, int tmax,
                                 int num_experts);

/* grimoire_moe_grouped_gemm_i8 without a tile table: the library forms its
 * own tile lists from counts (num_experts <= 1024) -- experts of more than
 * `split` rows (<= 0: the library's default, 64) in 128-row tiles, the
 * others in 32-row tiles, so that the long tail of a skewed routing does
 * not pay for empty tile rows.  Same products, bit for bit, as the tiled
 * call.  No reference counterpart (the reference's INT8 experts run one
 * expert at a time, src/grimoire.cpp:23214-23229); the forward's INT8
 * prefill uses it.  Allocates nothing. */
int grimoire_moe_grouped_gemm_i8_rows(void* stream, const grim_quant_weight* w, int N, int swiglu,
                                      const int8_t* A, const float* a_scale, float* out,
                                      const int32_t* offsets, const int32_t* counts, int num_experts,
                                      int split);

/* grimoire_moe_grouped_gemm_i8_rows on rows that are not stored in expert
 * order: routed row r (the order offsets / counts describe) reads row
 * row_map[r] of A [a_rows][2K] limb rows (e.g. the token rows, each read
 * once per route instead of copied K times); a_scale stays per routed row
 * [R].  Needs K / 64 >= 6 and, when K % 128 == 0, K / 128 >= 4, and
 * a_rows * 2K below 0x70000000 bytes (GRIM_ERR_SHAPE otherwise).  Same
 * products, bit for bit, as the call on the rows copied into routed order.
 * No reference counterpart (the reference materialises permuted rows,
 * src/prefill.cpp:2784-2806); the forward's INT8 gate_up uses it.
 * Allocates nothing. */
int grimoire_moe_grouped_gemm_i8_rows_gather(void* stream, const grim_quant_weight* w, int N, int swiglu,
                                             const int8_t* A, int a_rows, const int32_t* row_map,
                                             const float* a_scale, float* out, const int32_t* offsets,
                                             const int32_t* counts, int num_experts, int split);

/* ------------------------------------------------------------------------
 * Bridges (the vLLM-XPU grouped GEMMs the reference dlopens).  Same
 * argument lists apart from the queue.  rows_per_expert [ne] gives the
 * contiguous row blocks of `a`; expert_ids may be NULL (expert i = block
 * i).  atomic_buffer is accepted and ignored (no persistent tile counter is
 * needed here).  A bridge call allocates nothing and keeps no state between
 * calls: every work-group of its one launch forms the expert offsets and
 * the tile order from rows_per_expert itself (num_experts <= 1024), so
 * calls on different streams may run concurrently.  Errors (null pointers,
 * k not a multiple of 64, ...) launch nothing and leave the message in
 * grimoire_moe_last_error().
 * ---------------------------------------------------------------------- */

/* d[r][n] = a[r] . dequant(b_e)[n], b u8 [E][n][k/2] MXFP4, scales e8m0
 * [E][n][k/32], a/d bf16.  Replaces grimoire_xe2_grouped_mxfp4_bf16
 * (src/xe2_grouped_bridge.cpp:135). */
void grimoire_xe2_grouped_mxfp4_bf16(void* stream, const void* a, const unsigned char* b,
                                     const unsigned char* scales, void* d, int n, int k,
                                     const int* rows_per_expert, const int* expert_ids,
                                     int num_experts, int* atomic_buffer);

/* The reference's tile-policy variants of the same product
 * (src/xe2_grouped_bridge.cpp:149 full-tile, :163 8-row, :171 16-row
 * tiles), bound by name at src/grimoire.cpp:20638-20642.  Same arguments
 * and results; this library picks its tiles itself, so all three run the
 * kernel above. */
void grimoire_xe2_grouped_mxfp4_bf16_full(void* stream, const void* a, const unsigned char* b,
                                          const unsigned char* scales, void* d, int n, int k,
                                          const int* rows_per_expert, const int* expert_ids,
                                          int num_experts, int* atomic_buffer);
void grimoire_xe2_grouped_mxfp4_bf16_m8(void* stream, const void* a, const unsigned char* b,
                                        const unsigned char* scales, void* d, int n, int k,
                                        const int* rows_per_expert, const int* expert_ids,
                                        int num_experts, int* atomic_buffer);
void grimoire_xe2_grouped_mxfp4_bf16_m16(void* stream, const void* a, const unsigned char* b,
                                         const unsigned char* scales, void* d, int n, int k,
                                         const int* rows_per_expert, const int* expert_ids,
                                         int num_experts, int* atomic_buffer);

/* Signed-s4 weights [E][n][k/2] with bf16 group scales [E][n][k/group].
 * Declared, never defined, in the reference (src/xe2_grouped_bridge.hpp:22). */
void grimoire_xe2_grouped_w4a16(void* stream, const void* activations_bf16,
                                const unsigned char* weights_int4, const void* scales_bf16,
                                void* outputs_bf16, int n, int k, const int* rows_per_expert,
                                const int* expert_ids, int num_experts, int group_size,
                                int* atomic_buffer);

/* Grouped gate_up with SiLU(gate)*up epilogue: weights [E][2n][k/2] MXFP4
 * (gate rows then up rows), out bf16 [R][n].  Replaces
 * grimoire_xe2_fused_moe_gate_up_mxfp4_silu_bf16 (src/xe2_fused_moe_bridge.cpp:32-43). */
void grimoire_xe2_fused_moe_gate_up_mxfp4_silu_bf16(void* stream, const void* activations,
                                                    const unsigned char* weights,
                                                    const unsigned char* scales, void* outputs,
                                                    int n, int k, const int* rows_per_expert,
                                                    int num_experts, int32_t* atomic_buffer);

/* ------------------------------------------------------------------------
 * Whole MoE block, the sequence the engine runs per layer
 * (src/grimoire.cpp:15362-15500 decode, :22743-23300 prefill):
 * router GEMV -> top-k -> expert products -> combine (+ gated shared).
 * ---------------------------------------------------------------------- */
enum grim_route_mode {
    GRIM_ROUTE_SOFTMAX = 0,    /* softmax top-k (+ renormalise per cfg)   */
    GRIM_ROUTE_SIGMOID = 1,    /* sigmoid + selection bias (bf16)         */
    GRIM_ROUTE_GROUP = 2       /* group-limited sigmoid (bias fp32)       */
};

typedef struct grim_route_params {
    int32_t mode;              /* enum grim_route_mode                     */
    int32_t n_group;           /* GROUP only                               */
    int32_t topk_group;        /* GROUP only                               */
    float scaling;             /* routed scaling factor (1 = none)         */
    const void* bias;          /* SOFTMAX: router bias fp32 [E] added to the
                                  logits (logits = W x + b); SIGMOID: bf16
                                  [E] selection bias; GROUP: fp32 [E]
                                  selection bias; or NULL */
} grim_route_params;

/* Workspace bytes for grimoire_moe_forward at `tokens`.  Its first
 * GRIM_SYNC_BYTES hold the one-launch decode's (regime 7) epoch-tagged sync
 * words: they must be zero before the workspace's first regime-7 call
 * (hipMemset once after allocating it, or grimoire_moe_decode_sync_reset);
 * no other regime writes them, and a call that completes leaves them ready
 * for the next.  A regime-7 call whose polls time out sets the error word
 * and poisons the workspace (see grimoire_moe_decode_sync_status).
 * Otherwise no initial contents are needed.  Calls that share one
 * workspace must not overlap. */
#define GRIM_SYNC_BYTES 180480
size_t grimoire_moe_forward_workspace_bytes(const grim_moe_layer* L, int tokens);

/* y fp32 [T][H] = MoE(x fp32 [T][H]).  shared_gate_w bf16 [H] (may be NULL:
 * shared expert weight 1, as src/moe_ref.cpp:100-104).  Routing is written
 * to out_expert/out_weight [T][K] when not NULL.  regime: 0 = choose
 * (the expert-grouped GEMV on the matrix core for MXFP4 batches of
 * 16 <= T*K <= 2E whose shapes it takes; else slot GEMV for T*K <= 64;
 * else the expert-grouped GEMV for T*K <= 2E on INT4 / MXFP4 experts;
 * else the grouped MFMA GEMM), 1 = GEMV,
 * 2 = grouped GEMM, 3 = GEMV with one launch per stage, 7 = GEMV in one
 * launch for one token with no shared expert (INT4 / MXFP4 experts,
 * K <= 8, H <= 2048, I <= 1024, K * I <= 8192: router, top-k, gate_up and
 * down in one kernel whose work-groups exchange epoch-tagged words; other
 * shapes take regime 1.  Its work-groups (at most one per CU) must all be
 * resident at once: kernels of other streams that hold CUs can make its
 * bounded polls (20 ms) time out; that call and every later regime-7 call
 * on the workspace then write NaN outputs (routes: expert -1, weight NaN)
 * until grimoire_moe_decode_sync_reset, and
 * grimoire_moe_decode_sync_status reports it), 4 = expert-grouped
 * GEMV (MXFP4 with hidden and inter multiples of 64 above 256: on the
 * scaled fp4 matrix core, K padded to 256; otherwise on the vector ALU), 5 = expert-grouped GEMV on
 * the vector ALU.  No reference counterpart for 3-5 (regimes of this
 * build; the reference picks its kernels per batch size the same way). */
int grimoire_moe_forward(void* stream, const grim_moe_layer* L, const grim_route_params* rp,
                         const uint16_t* shared_gate_w, const float* x, float* y, int tokens,
                         int32_t* out_expert, float* out_weight, int regime, void* workspace,
                         size_t workspace_bytes);

/* One expert shard of the layer (expert parallelism on one GPU's share;
 * src/grimoire.cpp:15392-15399 decode, :23231-23240 batched): the router
 * (L->router, [num_experts][H]) and the top-k are global, while
 * L->gate_up / L->down hold only experts [expert_begin, expert_begin +
 * expert_count) (local index e - expert_begin).  Routes to other experts
 * become expert -1 / weight 0 and are skipped, so y is this shard's
 * partial sum; a shared expert in L is added as usual (give it to one
 * shard).  out_expert / out_weight receive the global routing.  regime as
 * grimoire_moe_forward, except that 1 and 7 run as 3 (their top-k lives
 * inside the expert kernels).  The workspace is
 * grimoire_moe_forward_workspace_bytes(L, tokens).  The sum over shards is
 * the caller's collective. */
int grimoire_moe_forward_shard(void* stream, const grim_moe_layer* L, const grim_route_params* rp,
                               const uint16_t* shared_gate_w, const float* x, float* y, int tokens,
                               int32_t* out_expert, float* out_weight, int regime, int expert_begin,
                               int expert_count, void* workspace, size_t workspace_bytes);
/* The shard remap alone: local_ids[r] = topk_ids[r] - expert_begin and
 * local_w[r] = topk_w[r] when the expert is in [expert_begin, expert_begin
 * + expert_count), else -1 and 0 (src/grimoire.cpp:23231-23240). */
int grimoire_moe_route_local(void* stream, const int32_t* topk_ids, const float* topk_w, int32_t* local_ids,
                             float* local_w, int routes, int expert_begin, int expert_count);

/* grimoire_moe_forward without a workspace argument and without any
 * allocation: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No reference counterpart.  The workspace is a fixed device
 * array of grimoire_moe_forward_noalloc_max_bytes() (8 MiB) per GPU inside
 * the library; a call whose workspace (grimoire_moe_forward_workspace_bytes
 * for its regime) exceeds it returns GRIM_ERR_WORKSPACE and launches
 * nothing (single-token and small-batch decode fit; large prefills do not).
 * All calls on one GPU share that array: calls that overlap on one GPU
 * (other streams, other threads) race and must be serialised by the
 * caller. */
size_t grimoire_moe_forward_noalloc_max_bytes(void);

/* Status of the one-launch decode (regime 7) on a workspace: *status = 1
 * when a call's bounded polls timed out (the workspace is poisoned: every
 * regime-7 call on it writes NaN outputs), else 0.  Reads the error word
 * in stream order and waits for the stream (a host synchronisation; not
 * for capture).  workspace NULL = the current device's array of
 * grimoire_moe_forward_noalloc.  No reference counterpart (the reference
 * has no one-launch decode). */
int grimoire_moe_decode_sync_status(void* stream, const void* workspace, size_t workspace_bytes,
                                    int* status);
/* Clears the sync words (epoch, error word, flags, router tags) of a
 * workspace in stream order with a fill kernel, so a poisoned workspace is
 * usable again; also the first-use initialisation.  workspace NULL = the
 * noalloc array of the current device.  No reference counterpart. */
int grimoire_moe_decode_sync_reset(void* stream, void* workspace, size_t workspace_bytes);
/* Test hook: sets the poll bound of the one-launch decode in real-time
 * counter ticks (100 MHz; a negative value restores the 20 ms default) and
 * returns the previous one.  A tiny bound makes the polls give up at once
 * while every kernel still exits normally.  No reference counterpart. */
uint64_t grimoire_moe_debug_spin_ticks(int64_t ticks);
int grimoire_moe_forward_noalloc(void* stream, const grim_moe_layer* L, const grim_route_params* rp,
                                 const uint16_t* shared_gate_w, const float* x, float* y,
                                 int tokens, int32_t* out_expert, float* out_weight, int regime);

/* One stage of the decode path of grimoire_moe_forward (regime 1, tokens
 * <= 8): stage 1 = router logits (and the formatted activations), 2 =
 * top-k + gate_up + SwiGLU, 4 = down + combine, each reading what the
 * earlier stages (or an earlier grimoire_moe_forward call on the same
 * workspace and inputs) left in the workspace.  For timing and tests of a
 * single launch; the three stages in order equal one forward call.  No
 * reference counterpart (the reference's launchers are per stage already:
 * launch_moe_gate_up_shared / launch_moe_down_shared,
 * include/b70/moe.hpp:133-185). */
int grimoire_moe_decode_stage(void* stream, const grim_moe_layer* L, const grim_route_params* rp,
                              const uint16_t* shared_gate_w, const float* x, float* y, int tokens,
                              int stage, void* workspace, size_t workspace_bytes);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif
#endif /* GRIMOIRE_MOE_H */
