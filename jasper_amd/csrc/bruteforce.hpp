// bruteforce.hpp -- exact k-NN by brute force on the matrix cores.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace jasper_amd {

// base [n][dp] and queries [nq][dp]: device fp16 rows (dp a multiple of 8,
// entries past dim zero, 16-byte aligned). Writes the k nearest per query
// (distance ascending, then id) to device out_ids / out_d; fewer than k
// vectors pad with (-1, FLT_MAX). Supports k <= 128, dp <= 4096.
void bruteforce_knn(const void* base, int64_t n, uint32_t dim, uint32_t dp, const void* queries, int64_t nq,
                    uint32_t k, int metric, int32_t* out_ids, float* out_d, hipStream_t s);

}  // namespace jasper_amd
