// sort.hip -- device radix sort of u64 keys for the reverse-edge grouping.
//
// The reference groups reverse edges with thrust::sort by source
// (index/construct.cuh:846-879). Here the pairs are packed as (target <<
// shift | source) and sorted as integers with rocPRIM's radix sort over bits
// [begin_bit, end_bit). The sort is stable, so a caller whose pairs are
// already in source order sorts the target bits only and still gets the
// sources of each target ascending -- the deterministic arrival order the
// reverse merge relies on.
#include <rocprim/device/device_radix_sort.hpp>

#include "build.hpp"

namespace jasper_amd {

size_t sort_u64_temp_bytes(size_t max_items) {
  size_t bytes = 0;
  hip_check(rocprim::radix_sort_keys(nullptr, bytes, (const uint64_t*)nullptr, (uint64_t*)nullptr, max_items, 0, 64),
            "radix sort temp size");
  return bytes;
}

void sort_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, size_t n, int begin_bit,
              int end_bit, hipStream_t stream) {
  if (n == 0) return;
  hip_check(rocprim::radix_sort_keys(temp, temp_bytes, in, out, n, (unsigned)begin_bit, (unsigned)end_bit, stream),
            "radix sort");
}

}  // namespace jasper_amd
