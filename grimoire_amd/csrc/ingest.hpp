// ingest.hpp -- checkpoint tensors -> expert-major weight rows.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace grim {

// GPTQ triples of up to kIngBatch projections of one shape into rows
// [row0[i], row0[i] + out) of one stacked INT4 / INT4_F16 weight
// (src/gptq.cpp:56-83).  The table travels in the kernel arguments.
constexpr int kIngBatch = 64;

struct IngestGptq {
    const uint32_t* qweight[kIngBatch];  // [in/8][out]
    const uint32_t* qzeros[kIngBatch];   // [in/group][out/8]
    const uint16_t* scales[kIngBatch];   // fp16 [in/group][out]
    int32_t row0[kIngBatch];
    int n, in, out, group;
    uint8_t* dst_payload;     // [N][dst_row_bytes]
    int64_t dst_row_bytes;    // in / 2
    uint16_t* dst_scales;     // [N][dst_rs]
    uint8_t* dst_zeros;       // [N][dst_rs]
    int dst_rs;               // in / group
    int keep_f16;             // 1: fp16 bits kept (INT4_F16); 0: bf16 (INT4)
};

struct SignedRegion {
    uint8_t* payload;
    int64_t bytes;
    uint8_t* zeros;
    int64_t zbytes;
};

hipError_t ingest_gptq(hipStream_t st, const IngestGptq& a);
hipError_t ingest_int4_zeros(hipStream_t st, const uint32_t* zp, int out, int groups,
                             uint8_t* dst_zeros, int dst_rs);
// src/grimoire.cpp:8386-8397 over n regions; *flag = 1 if converted.
hipError_t int4_signed(hipStream_t st, const SignedRegion* r, int n, int32_t* flag);

}  // namespace grim
