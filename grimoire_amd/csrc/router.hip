// router.hip -- router projection and top-k selection.
//
// Top-k runs one wavefront per token with every score in VGPRs (lane l owns
// experts [l*V, l*V+V), V = ceil(E/64) <= 8).  Each round packs
// (order-preserving score bits, ~expert) into one 64-bit key, so a single
// wave max gives the largest score and, among equal scores, the lowest
// expert index -- the tie rule of src/ops.cpp:1125-1131.  The weights are
// then formed serially in pick order with the same operations as the
// reference kernels (src/ops.cpp:1133-1147, :2126-2135), using det_expf so
// that the oracle reproduces them bit for bit.
#include "common.hpp"
#include "router.hpp"

namespace grim {

constexpr int kMaxV = 8;          // E <= 512
constexpr int kTopkWaves = 4;

__device__ __forceinline__ uint64_t score_key(float v, int e) {
    if (v != v) return (uint64_t(1) << 32) | uint32_t(~e);   // NaN ranks below everything
    uint32_t u = f_bits(v + 0.0f);                           // -0 -> +0
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (uint64_t(u) << 32) | uint32_t(~e);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
        const uint64_t o = __shfl_xor(k, m, kWave);
        k = o > k ? o : k;
    }
    return k;
}

// K rounds of wave argmax over sel[V] (lane-owned), skipping masked
// entries.  Returns the picks in pick order (uniform across the wave).
__device__ __forceinline__ void wave_select(const float* sel, bool* taken, int V, int E, int K,
                                            int lane, int* picks) {
    for (int s = 0; s < K; ++s) {
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < kMaxV; ++j) {
            const int e = lane * V + j;
            if (j < V && e < E && !taken[j]) {
                const uint64_t k = score_key(sel[j], e);
                best = k > best ? k : best;
            }
        }
        best = wave_max_u64(best);
        const int e = int(~uint32_t(best));
        picks[s] = e;
        const int owner = e / V, j = e - owner * V;
        if (lane == owner) {
#pragma unroll
            for (int jj = 0; jj < kMaxV; ++jj)
                if (jj == j) taken[jj] = true;
        }
    }
}

// mode 0: softmax (decode semantics); 1: softmax batched semantics
// (normalize == 0 -> raw logits); 2: sigmoid + bf16 bias; 3: group-limited
// sigmoid + fp32 bias.
__global__ __launch_bounds__(kTopkWaves * kWave) void topk_kernel(
    const float* __restrict__ logits, int T, int E, int K, int mode, int normalize,
    float scaling, const uint16_t* __restrict__ bias16, const float* __restrict__ bias32,
    int n_group, int topk_group, int32_t* __restrict__ out_e, float* __restrict__ out_w) {
    __shared__ float gsel[kTopkWaves][512];
    __shared__ float gscore[kTopkWaves][64];
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x / kWave;
    const int t = blockIdx.x * kTopkWaves + wv;
    if (t >= T) return;   // whole wave exits together
    const int V = (E + kWave - 1) / kWave;
    const float* row = logits + int64_t(t) * E;

    float sc[kMaxV], sel[kMaxV];
    bool taken[kMaxV];
#pragma unroll
    for (int j = 0; j < kMaxV; ++j) {
        const int e = lane * V + j;
        taken[j] = false;
        sc[j] = 0.0f;
        sel[j] = 0.0f;
        if (j < V && e < E) {
            const float l = row[e];
            if (mode <= 1) {
                sel[j] = l;
            } else {
                sc[j] = det_sigmoid(l);
                const float b = mode == 2 ? (bias16 ? bf16_to_f32(bias16[e]) : 0.0f)
                                          : (bias32 ? bias32[e] : 0.0f);
                sel[j] = sc[j] + b;
            }
        }
    }

    if (mode == 3) {
        // group scores: sum of the two largest biased scores per group
        for (int j = 0; j < V; ++j) {
            const int e = lane * V + j;
            if (e < E) gsel[wv][e] = sel[j];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int gs = E / n_group;
        if (lane < n_group) {
            int b1 = -1, b2 = -1;
            for (int e = lane * gs; e < (lane + 1) * gs; ++e) {
                const float v = gsel[wv][e];
                if (b1 < 0 || v > gsel[wv][b1]) { b2 = b1; b1 = e; }
                else if (b2 < 0 || v > gsel[wv][b2]) b2 = e;
            }
            gscore[wv][lane] = gs > 1 ? gsel[wv][b1] + gsel[wv][b2] : gsel[wv][b1];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        uint64_t keep = 0;
        for (int j = 0; j < topk_group; ++j) {
            int best = -1;
            for (int g = 0; g < n_group; ++g) {
                if (keep & (uint64_t(1) << g)) continue;
                if (best < 0 || gscore[wv][g] > gscore[wv][best]) best = g;
            }
            keep |= uint64_t(1) << best;
        }
#pragma unroll
        for (int j = 0; j < kMaxV; ++j) {
            const int e = lane * V + j;
            if (j < V && e < E) taken[j] = !((keep >> (e / gs)) & 1);
        }
    }

    int picks[16];
    wave_select(sel, taken, V, E, K, lane, picks);

    // gather the picked values (uniform): raw score for softmax, unbiased
    // sigmoid for the sigmoid modes
    float v[16];
    for (int s = 0; s < K; ++s) {
        const int e = picks[s];
        const int owner = e / V, j = e - owner * V;
        float mine = 0.0f;
#pragma unroll
        for (int jj = 0; jj < kMaxV; ++jj)
            if (jj == j) mine = mode <= 1 ? sel[jj] : sc[jj];
        v[s] = __shfl(mine, owner, kWave);
    }

    if (lane == 0) {
        int32_t* oe = out_e + int64_t(t) * K;
        float* ow = out_w + int64_t(t) * K;
        if (mode <= 1) {
            if (mode == 1 && !normalize) {
                for (int s = 0; s < K; ++s) { oe[s] = picks[s]; ow[s] = v[s]; }
            } else {
                float m = v[0];
                for (int s = 1; s < K; ++s) m = fmaxf(m, v[s]);
                float sum = 0.0f;
                float ev[16];
                for (int s = 0; s < K; ++s) {
                    ev[s] = det_expf(v[s] - m);
                    sum += ev[s];
                }
                for (int s = 0; s < K; ++s) {
                    oe[s] = picks[s];
                    ow[s] = (normalize && sum > 0.0f) ? ev[s] / sum : ev[s];
                }
            }
        } else {
            float w[16];
            for (int s = 0; s < K; ++s) w[s] = v[s];
            if (normalize) {
                float sum = 0.0f;
                for (int s = 0; s < K; ++s) sum += w[s];
                if (sum > 0.0f)
                    for (int s = 0; s < K; ++s) w[s] /= sum;
            }
            if (scaling != 1.0f)
                for (int s = 0; s < K; ++s) w[s] *= scaling;
            for (int s = 0; s < K; ++s) { oe[s] = picks[s]; ow[s] = w[s]; }
        }
    }
}

hipError_t topk_launch(hipStream_t st, const TopkArgs& a) {
    dim3 grid((a.T + kTopkWaves - 1) / kTopkWaves);
    hipLaunchKernelGGL(topk_kernel, grid, dim3(kTopkWaves * kWave), 0, st, a.logits, a.T, a.E,
                       a.K, a.mode, a.normalize, a.scaling, a.bias16, a.bias32, a.n_group,
                       a.topk_group, a.out_e, a.out_w);
    return hipGetLastError();
}

// ---------------------------------------------------------- router logits

// Small T: one wave per expert row, fp32 row chunks streamed with 16-byte
// loads, up to kRT tokens per block; x read through the cache.
constexpr int kRT = 8;
__global__ __launch_bounds__(256) void router_gemv(const float* __restrict__ W,
                                                   const float* __restrict__ x,
                                                   const float* __restrict__ bias,
                                                   float* __restrict__ logits, int T, int E,
                                                   int H) {
    const int lane = threadIdx.x & (kWave - 1);
    const int e = blockIdx.x * 4 + threadIdx.x / kWave;
    const int t0 = blockIdx.y * kRT;
    if (e >= E) return;
    const int nt = T - t0 < kRT ? T - t0 : kRT;
    float acc[kRT];
#pragma unroll
    for (int i = 0; i < kRT; ++i) acc[i] = 0.0f;
    const float* wr = W + int64_t(e) * H;
    for (int k = lane * 4; k < H; k += kWave * 4) {
        const float4 wv = *reinterpret_cast<const float4*>(wr + k);
#pragma unroll
        for (int i = 0; i < kRT; ++i) {
            if (i < nt) {
                const float4 xv = *reinterpret_cast<const float4*>(x + int64_t(t0 + i) * H + k);
                acc[i] = __builtin_fmaf(wv.x, xv.x, acc[i]);
                acc[i] = __builtin_fmaf(wv.y, xv.y, acc[i]);
                acc[i] = __builtin_fmaf(wv.z, xv.z, acc[i]);
                acc[i] = __builtin_fmaf(wv.w, xv.w, acc[i]);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < kRT; ++i) {
        if (i < nt) {
            const float s = group_sum<kWave>(acc[i]);
            if (lane == 0) logits[int64_t(t0 + i) * E + e] = bias ? s + bias[e] : s;
        }
    }
}

// Large T: LDS-tiled fp32 GEMM, 64 tokens x 64 experts per block, each
// thread a 4x4 register tile, K in steps of 16.
__global__ __launch_bounds__(256) void router_gemm(const float* __restrict__ W,
                                                   const float* __restrict__ x,
                                                   const float* __restrict__ bias,
                                                   float* __restrict__ logits, int T, int E,
                                                   int H) {
    __shared__ float xs[16][64 + 4];
    __shared__ float ws[16][64 + 4];
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int t0 = blockIdx.y * 64, e0 = blockIdx.x * 64;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < H; k0 += 16) {
        for (int i = threadIdx.x; i < 64 * 16; i += 256) {
            const int r = i / 16, kk = i % 16;
            const int t = t0 + r, e = e0 + r;
            xs[kk][r] = (t < T && k0 + kk < H) ? x[int64_t(t) * H + k0 + kk] : 0.0f;
            ws[kk][r] = (e < E && k0 + kk < H) ? W[int64_t(e) * H + k0 + kk] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 16; ++kk) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) { a[i] = xs[kk][ty * 4 + i]; b[i] = ws[kk][tx * 4 + i]; }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int t = t0 + ty * 4 + i, e = e0 + tx * 4 + j;
            if (t < T && e < E) logits[int64_t(t) * E + e] = bias ? acc[i][j] + bias[e] : acc[i][j];
        }
}

hipError_t router_logits_launch(hipStream_t st, const float* W, const float* x,
                                const float* bias, float* logits, int T, int E, int H) {
    if (T <= 32 && H % 4 == 0) {
        dim3 grid((E + 3) / 4, (T + kRT - 1) / kRT);
        hipLaunchKernelGGL(router_gemv, grid, dim3(256), 0, st, W, x, bias, logits, T, E, H);
    } else {
        dim3 grid((E + 63) / 64, (T + 63) / 64);
        hipLaunchKernelGGL(router_gemm, grid, dim3(256), 0, st, W, x, bias, logits, T, E, H);
    }
    return hipGetLastError();
}

}  // namespace grim

namespace grim {

// gate[t] = sigmoid(x_t . w) with w bf16 [H]; one wave per token
// (launch_rowdot_sigmoid, src/kernels.hpp:580; formula of
// src/moe_kernels.cpp:162-172).
__global__ __launch_bounds__(256) void rowdot_sigmoid(const float* __restrict__ x,
                                                      const uint16_t* __restrict__ w,
                                                      float* __restrict__ gate, int T, int H) {
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * 4 + threadIdx.x / kWave;
    if (t >= T) return;
    float a = 0.0f;
    for (int c = lane; c < H; c += kWave) a = __builtin_fmaf(bf16_to_f32(w[c]), x[int64_t(t) * H + c], a);
    a = group_sum<kWave>(a);
    if (lane == 0) gate[t] = det_sigmoid(a);
}

hipError_t rowdot_sigmoid_launch(hipStream_t st, const float* x, const uint16_t* w, float* gate,
                                 int T, int H) {
    hipLaunchKernelGGL(rowdot_sigmoid, dim3((T + 3) / 4), dim3(256), 0, st, x, w, gate, T, H);
    return hipGetLastError();
}

}  // namespace grim
