// ingest.hip -- expert-weight ingestion into the expert-major layout.
//
// Checkpoint tensors arrive in their on-disk layouts; the MoE kernels read
// [N][K/2] nibble rows with [N][K/G] scales and zero points (the layout of
// grim_quant_weight).  The conversions are byte work, so every kernel here
// is bound by HBM bandwidth:
//
//   GPTQ qweight int32 [in/8][out]  ->  payload [out][in/2]
//     word qweight[k/8][o] holds the nibbles of k = 8(k/8)..8(k/8)+7 of
//     output o, nibble j at bits 4j; the payload row stores k in byte k/2,
//     even k in the low nibble.  Both orders put nibble j of the word in
//     byte j/2 of the same four bytes, so the repack of src/gptq.cpp:56-83
//     is a plain 32-bit transpose: payload32[o][k/8] = qweight[k/8][o].
//     It runs as 64x64-word tiles through LDS: coalesced reads of qweight
//     rows, coalesced writes of payload rows.
//   GPTQ scales fp16 [in/g][out], qzeros [in/g][out/8] -> [out][in/g]
//     scale (bf16 rounded, or the fp16 bits kept), zero = nibble + 1
//     (AutoGPTQ stores the zero point minus one, src/gptq.cpp:67-70).
//   compressed-tensors INT4 zero points int32 [out/8][in/g], row n in
//     nibble n % 8 (src/grimoire.cpp:1418-1434), or 8 when absent.
//   signed s4 conversion (src/grimoire.cpp:8386-8397): when every zero
//     point of the layer is 8, payload ^= 0x88 turns offset-binary nibbles
//     into two's-complement ones and the zeros become 0xFF ("signed").
#include "common.hpp"
#include "ingest.hpp"

namespace grim {

constexpr int kTile = 64;        // words per tile side
constexpr int kIngThreads = 256;

// Projection z of the batch: out32[o * out_stride + r] = in32[r * C + o]
// for r < R, o < C, out32 = the payload rows from row0[z].
__global__ __launch_bounds__(kIngThreads) void transpose_u32(const IngestGptq a) {
    __shared__ uint32_t tile[kTile][kTile + 1];
    const int z = blockIdx.z;
    const int R = a.in / 8, C = a.out;
    const uint32_t* __restrict__ in = a.qweight[z];
    uint32_t* __restrict__ out =
        reinterpret_cast<uint32_t*>(a.dst_payload + int64_t(a.row0[z]) * a.dst_row_bytes);
    const int64_t out_stride = a.dst_row_bytes / 4;
    const int c0 = blockIdx.x * kTile, r0 = blockIdx.y * kTile;
    const int tx = threadIdx.x & (kTile - 1), ty = threadIdx.x / kTile;   // ty in 0..3
    constexpr int kRows = kTile / (kIngThreads / kTile);   // 16 loads per thread, all in flight
    uint32_t v[kRows];
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
        const int r = r0 + ty + j * (kIngThreads / kTile), c = c0 + tx;
        v[j] = (r < R && c < C) ? in[int64_t(r) * C + c] : 0u;
    }
#pragma unroll
    for (int j = 0; j < kRows; ++j) tile[ty + j * (kIngThreads / kTile)][tx] = v[j];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kTile; i += kIngThreads / kTile) {
        const int o = c0 + ty + i, r = r0 + tx;
        if (o < C && r < R) out[int64_t(o) * out_stride + r] = tile[tx][ty + i];
    }
}

// One thread per (group g, output o) of projection blockIdx.y, o fastest:
// reads of the checkpoint rows are coalesced; the [out][groups] writes are
// short rows.
__global__ __launch_bounds__(kIngThreads) void gptq_meta(const IngestGptq a) {
    const int z = blockIdx.y;
    const int out = a.out, groups = a.in / a.group;
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= int64_t(out) * groups) return;
    const int g = int(i / out), o = int(i % out);
    const uint16_t s = a.scales[z][int64_t(g) * out + o];
    const uint32_t zw = a.qzeros[z][int64_t(g) * (out >> 3) + (o >> 3)];
    const int64_t d = int64_t(a.row0[z] + o) * a.dst_rs + g;
    a.dst_scales[d] = a.keep_f16 ? s : f32_to_bf16(f16_to_f32(s));
    a.dst_zeros[d] = uint8_t(((zw >> ((o & 7) * 4)) & 0xFu) + 1u);
}

// compressed-tensors INT4 zero points, or the symmetric 8 when zp == NULL.
__global__ __launch_bounds__(kIngThreads) void int4_zero_unpack(const uint32_t* __restrict__ zp,
                                                                int out, int groups,
                                                                uint8_t* __restrict__ dst_zeros,
                                                                int dst_rs) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= int64_t(out) * groups) return;
    const int n = int(i / groups), g = int(i % groups);
    const uint8_t z =
        zp ? uint8_t((zp[int64_t(n >> 3) * groups + g] >> (4 * (n & 7))) & 0xFu) : uint8_t(8);
    dst_zeros[int64_t(n) * dst_rs + g] = z;
}

__global__ void flag_set(int32_t* flag, int32_t v) {
    if (threadIdx.x == 0) *flag = v;
}

// Clears *flag when any byte of z is not 8.  Every writer stores the same 0.
__global__ __launch_bounds__(kIngThreads) void zeros_all8(const uint8_t* __restrict__ z,
                                                          int64_t n, int32_t* flag) {
    bool bad = false;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += int64_t(gridDim.x) * blockDim.x)
        bad |= z[i] != 8;
    if (__any(bad) && (threadIdx.x & (kWave - 1)) == 0) *flag = 0;
}

// When *flag is set: p ^= pattern (set_to < 0) or p = set_to, over n bytes:
// an unaligned head and tail bytewise, the 16-byte aligned body as uint4.
__device__ __forceinline__ uint32_t xor_or_set(uint32_t v, uint32_t pattern, int set_to) {
    return set_to >= 0 ? uint32_t(set_to) * 0x01010101u : v ^ pattern;
}

__global__ __launch_bounds__(kIngThreads) void xor_bytes(uint8_t* __restrict__ p, int64_t n,
                                                         uint32_t pattern, int set_to,
                                                         const int32_t* flag) {
    if (*flag == 0) return;
    const int64_t stride = int64_t(gridDim.x) * blockDim.x;
    const int64_t t0 = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    int64_t head = int64_t((16 - (reinterpret_cast<uintptr_t>(p) & 15)) & 15);
    if (head > n) head = n;
    const int64_t n16 = (n - head) / 16;
    const int64_t tail0 = head + n16 * 16;
    uint4* p16 = reinterpret_cast<uint4*>(p + head);
    for (int64_t i = t0; i < n16; i += stride) {
        uint4 v = p16[i];
        v.x = xor_or_set(v.x, pattern, set_to);
        v.y = xor_or_set(v.y, pattern, set_to);
        v.z = xor_or_set(v.z, pattern, set_to);
        v.w = xor_or_set(v.w, pattern, set_to);
        p16[i] = v;
    }
    if (t0 < head) p[t0] = uint8_t(xor_or_set(p[t0], pattern, set_to));
    if (t0 < n - tail0) p[tail0 + t0] = uint8_t(xor_or_set(p[tail0 + t0], pattern, set_to));
}

static dim3 grid_for(int64_t items, int per_block) {
    return dim3(unsigned((items + per_block - 1) / per_block));
}

static unsigned stream_blocks(int64_t bytes) {
    const int64_t b = (bytes / 16 + kIngThreads - 1) / kIngThreads;
    return unsigned(b < 1 ? 1 : (b > 4096 ? 4096 : b));
}

hipError_t ingest_gptq(hipStream_t st, const IngestGptq& a) {
    if (a.n <= 0 || a.n > kIngBatch) return hipErrorInvalidValue;
    const int words_r = a.in / 8;   // qweight rows
    dim3 g1((a.out + kTile - 1) / kTile, (words_r + kTile - 1) / kTile, a.n);
    hipLaunchKernelGGL(transpose_u32, g1, dim3(kIngThreads), 0, st, a);
    const int64_t items = int64_t(a.out) * (a.in / a.group);
    dim3 g2(unsigned((items + kIngThreads - 1) / kIngThreads), a.n);
    hipLaunchKernelGGL(gptq_meta, g2, dim3(kIngThreads), 0, st, a);
    return hipGetLastError();
}

hipError_t ingest_int4_zeros(hipStream_t st, const uint32_t* zp, int out, int groups,
                             uint8_t* dst_zeros, int dst_rs) {
    hipLaunchKernelGGL(int4_zero_unpack, grid_for(int64_t(out) * groups, kIngThreads),
                       dim3(kIngThreads), 0, st, zp, out, groups, dst_zeros, dst_rs);
    return hipGetLastError();
}

hipError_t int4_signed(hipStream_t st, const SignedRegion* r, int n, int32_t* flag) {
    hipLaunchKernelGGL(flag_set, dim3(1), dim3(kWave), 0, st, flag, 1);
    for (int i = 0; i < n; ++i)
        if (r[i].zbytes > 0)
            hipLaunchKernelGGL(zeros_all8, dim3(stream_blocks(r[i].zbytes * 16)),
                               dim3(kIngThreads), 0, st, r[i].zeros, r[i].zbytes, flag);
    for (int i = 0; i < n; ++i) {
        if (r[i].bytes > 0)
            hipLaunchKernelGGL(xor_bytes, dim3(stream_blocks(r[i].bytes)), dim3(kIngThreads), 0,
                               st, r[i].payload, r[i].bytes, 0x88888888u, -1, flag);
        if (r[i].zbytes > 0)
            hipLaunchKernelGGL(xor_bytes, dim3(stream_blocks(r[i].zbytes)), dim3(kIngThreads), 0,
                               st, r[i].zeros, r[i].zbytes, 0u, 0xFF, flag);
    }
    return hipGetLastError();
}

}  // namespace grim
