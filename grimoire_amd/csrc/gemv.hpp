// gemv.hpp -- host interface of the decode (slot form) expert products.
#pragma once

#include "common.hpp"

namespace grim {

// Arguments of the decode kernels.  Work items: NR router items (fp32
// router GEMV), NG gate_up items (token, slot, row block), ND down items
// (token, row block); each role is one kernel launch, in that order.
struct DecodeArgs {
    WView gu, sgu, dn, sdn;
    bool shared;
    // routing (router role)
    const float* router;
    const float* rbias;       // softmax router bias fp32 [E] or null
    int mode, normalize;
    float scaling;
    const uint16_t* bias16;
    const float* bias32;
    int n_group, topk_group;
    float* logits;            // [M][E]
    // data
    const float* x;           // [M][H]
    int32_t* rex;             // [M][K]
    float* rwt;               // [M][K]
    const uint16_t* gate_w;   // bf16 [H] or null: gate[t] = sigmoid(x_t . gate_w)
    float* gate;              // [M]
    const float* gate_in;     // down: shared-expert weight per token or null (= 1)
    float* h;                 // [M][KS][I] (single-role launches)
    uint32_t* hf;             // fmt_h: h formatted for staging, fmt_words(KS*I) words per token
    float* y;                 // [M][H]
    int H, I, K, E, M;
    // plan (decode_plan)
    int lpr_gu, lpr_dn, gu_rb, dn_rb;
    int NR, NG, ND;
    int fmt_h;                // gate_up writes hf, down stages hf (else plain h)
    int route_topk;           // gate_up items compute the top-k from logits (and store rex/rwt)
    unsigned long long* ts;   // phase timestamps (GRIM_TIMING builds only), else null
    // wave-centric gate_up (INT4 / MXFP4): the router kernel writes the
    // activations formatted once (xf, xf_words per token), gate_up lanes read
    // their chunks from it directly
    uint32_t* xf;
    int xf_words;
    int dn_wave;              // wave-centric down (one wave per slot)
    int gu_ru;                // wave-centric gate_up: row pairs per wave
    // one-launch decode (gemv_fused.hpp): one token, no shared expert
    int fused;                // launch the fused kernel instead of the roles
    uint32_t* sync;           // kSyncBytes of epoch-tagged words, zero before first use
    float* hrep;              // kSyncCopies copies of h, fused_h_stride(K, I) floats apart
    int fz_G, fz_ru, fz_rh;   // grid, row pairs per wave, rows per half-wave
    uint64_t spin_ticks;      // bound of each poll, real-time counter ticks (100 MHz)
};

// Default poll bound of the one-launch decode: 20 ms.
constexpr uint64_t kSpinTicksDefault = 2000000;

// Sync words at the head of every forward workspace (32-bit word offsets):
// [0] the epoch word, [1] the error word; from kSyncFlagOff, kSyncCopies
// copies of the per-work-group flags (kSyncFlagStride words apart); from
// kSyncRtagOff, kSyncCopies copies of the 64-bit router rows
// (kSyncRtagStride 64-bit words apart).  Work-group b reads copy
// b % kSyncCopies, so no memory channel serves every work-group's polls.
constexpr int kSyncCopies = 32;
constexpr int kSyncMaxGrid = 256;
constexpr int kSyncMaxE = 512;
constexpr int kSyncFlagStride = kSyncMaxGrid + 64;
constexpr int kSyncRtagStride = kSyncMaxE + 32;
constexpr size_t kSyncFlagOff = 64;
constexpr size_t kSyncRtagOff = kSyncFlagOff + size_t(kSyncCopies) * kSyncFlagStride;
constexpr size_t kSyncBytes = (kSyncRtagOff + size_t(kSyncCopies) * kSyncRtagStride * 2) * 4;
// h copies of the fused decode: kSyncCopies rows of K * I fp32 padded to this
__host__ __device__ constexpr int fused_h_stride(int K, int I) { return ((K * I + 63) & ~63) + 64; }

// Words per token of the formatted h (n = KS * I elements):
// the staged planes, one fp32 sum per group of eight, padded to 16 bytes.
__host__ __device__ constexpr int fmt_words(int n) { return (n + n / 8 + 3) & ~3; }

// Words per token of the formatted activations for the wave-centric gate_up
// (32-element chunks, H = 32 * C): hi plane [H/2], lo plane [H/2], then
// (sum, lo-nonzero flag) per chunk, padded to 16 bytes.
__host__ __device__ constexpr int xf_words(int H) { return (H + 2 * (H / 32) + 3) & ~3; }

constexpr int kRoleRouter = 1, kRoleGateUp = 2, kRoleDown = 4;


void decode_plan(int fmt, DecodeArgs& a, int roles);
// Plans the fused kernel (sets fused and the fz_* fields) when the shape
// fits it; returns whether it does.
bool decode_plan_fused(int fmt, DecodeArgs& a);
size_t decode_lds_bytes(int fmt, const DecodeArgs& a);
hipError_t decode_launch(hipStream_t st, int fmt, const DecodeArgs& a);
int chunk_elems(int fmt);

}  // namespace grim
