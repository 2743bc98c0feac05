// sort.hip -- device radix sort of u64 keys for the reverse-edge grouping.
//
// The reference groups reverse edges with thrust::sort by source
// (index/construct.cuh:846-879). Here the pairs are packed as
// (target << 32 | source) and sorted as plain integers with rocPRIM's radix
// sort, which also orders the sources of each target ascending -- the
// deterministic arrival order the reverse merge relies on.
#include <rocprim/device/device_radix_sort.hpp>

#include "build.hpp"

namespace jasper_amd {

size_t sort_u64_temp_bytes(size_t max_items) {
  size_t bytes = 0;
  hip_check(rocprim::radix_sort_keys(nullptr, bytes, (const uint64_t*)nullptr, (uint64_t*)nullptr, max_items, 0, 64),
            "radix sort temp size");
  return bytes;
}

void sort_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, size_t n, int end_bit,
              hipStream_t stream) {
  if (n == 0) return;
  hip_check(rocprim::radix_sort_keys(temp, temp_bytes, in, out, n, 0, (unsigned)end_bit, stream),
            "radix sort");
}

}  // namespace jasper_amd
