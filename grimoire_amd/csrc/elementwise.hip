// elementwise.hip -- the small launchers around the MoE path:
//   permute_rows_bf16   dst[r] = bf16(src[perm_token[r]])   (src/prefill.cpp:2644-2652)
//   swiglu_bf16         out = bf16(silu(g) * u) on bf16 gate|up rows (src/prefill.cpp:2541-2558)
//   scale_by_sigmoid    x *= sigmoid(g[0]) / x[t] *= sigmoid(gate[t])
//                       (src/ops.cpp:1491-1499, src/prefill.cpp:2610-2622)
// All HBM-bound streams: 4 (permute: 4 fp32 -> 4 bf16; swiglu: 4 outputs)
// elements per thread with 16/8-byte accesses where the widths allow.
#include "common.hpp"
#include "elementwise.hpp"

namespace grim {

constexpr int kEwThreads = 256;

__global__ __launch_bounds__(kEwThreads) void permute_rows_bf16_kernel(
    const float* __restrict__ src, const int32_t* __restrict__ perm, uint16_t* __restrict__ dst,
    int rows, int width) {
    const int r = blockIdx.x;
    const float* s = src + int64_t(perm[r]) * width;
    uint16_t* d = dst + int64_t(r) * width;
    if ((width & 3) == 0) {
        for (int c = threadIdx.x * 4; c < width; c += kEwThreads * 4) {
            const float4 v = *reinterpret_cast<const float4*>(s + c);
            uint2 o;
            o.x = uint32_t(f32_to_bf16(v.x)) | (uint32_t(f32_to_bf16(v.y)) << 16);
            o.y = uint32_t(f32_to_bf16(v.z)) | (uint32_t(f32_to_bf16(v.w)) << 16);
            *reinterpret_cast<uint2*>(d + c) = o;
        }
    } else {
        for (int c = threadIdx.x; c < width; c += kEwThreads) d[c] = f32_to_bf16(s[c]);
    }
}

__global__ __launch_bounds__(kEwThreads) void swiglu_bf16_kernel(const uint16_t* __restrict__ gu,
                                                                 uint16_t* __restrict__ out,
                                                                 int inter) {
    const int t = blockIdx.x;
    const uint16_t* g = gu + int64_t(t) * 2 * inter;
    for (int d = threadIdx.x; d < inter; d += kEwThreads) {
        const float gv = bf16_to_f32(g[d]);
        out[int64_t(t) * inter + d] = f32_to_bf16(silu(gv) * bf16_to_f32(g[inter + d]));
    }
}

__global__ __launch_bounds__(kEwThreads) void scale_by_sigmoid_kernel(float* __restrict__ x,
                                                                      const float* __restrict__ gate,
                                                                      int64_t n, int hidden) {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * blockDim.x) {
        const float g = gate[hidden > 0 ? i / hidden : 0];
        x[i] *= 1.0f / (1.0f + det_expf(-g));
    }
}

hipError_t permute_rows_bf16_launch(hipStream_t st, const float* src, const int32_t* perm,
                                    uint16_t* dst, int rows, int width) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(permute_rows_bf16_kernel, dim3(rows), dim3(kEwThreads), 0, st, src, perm, dst,
                       rows, width);
    return hipGetLastError();
}

hipError_t swiglu_bf16_launch(hipStream_t st, const uint16_t* gu, uint16_t* out, int tokens,
                              int inter) {
    if (tokens <= 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_bf16_kernel, dim3(tokens), dim3(kEwThreads), 0, st, gu, out, inter);
    return hipGetLastError();
}

hipError_t scale_by_sigmoid_launch(hipStream_t st, float* x, const float* gate, int64_t n,
                                   int hidden) {
    if (n <= 0) return hipSuccess;
    int64_t b = (n + kEwThreads - 1) / kEwThreads;
    if (b > 8192) b = 8192;
    hipLaunchKernelGGL(scale_by_sigmoid_kernel, dim3(unsigned(b)), dim3(kEwThreads), 0, st, x, gate,
                       n, hidden);
    return hipGetLastError();
}

}  // namespace grim
