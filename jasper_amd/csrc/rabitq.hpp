// rabitq.hpp -- one-bit RaBitQ quantizer (reference rabitq/quantize.cuh).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jasper_amd {

// ceil(dim / 8) rounded up to 4 (rabitq_data_store::code_bytes, 1 bit/dim).
uint32_t rabitq_code_bytes(uint32_t dim);

// nodes[n][code_bytes + 8] <- codes, f_add, f_rescale of rows x (fp16 when
// f16, else fp32; row stride `stride` elements) with rotation P (device,
// column-major fp32 [dim*dim]) and centroid (device fp32 [dim], or null for
// zero). metric: kL2 or kIP. All pointers are device memory.
void rabitq_quantize(const void* x, bool f16, int64_t n, uint32_t dim, uint32_t stride, const float* P,
                     const float* centroid, int metric, void* out, hipStream_t s);

}  // namespace jasper_amd
