// build.hpp -- Vamana construction on the device (host driver).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "graph.hpp"

namespace jasper_amd {

struct BuildStats {
  double search_ms = 0, prune_ms = 0, sort_ms = 0, reverse_ms = 0, total_ms = 0;
  int64_t batches = 0;
  int64_t max_batch = 0;
};

// Maximum batch size of the reference for a workspace budget
// (graph_construct_workspace::max_batch_size_for_budget, index/construct.cuh:
// 238-262, capped at n/50 by ffi/jasper_ffi_common.cuh:245-248).
int64_t reference_max_batch(int64_t n, uint32_t R, int64_t budget_bytes);

// Builds the edges of `g` (vectors already resident) with the reference's
// batch schedule: batches of 1, 2, 4, ... up to max_batch over ids in order.
// `time_stages` records per-stage HIP-event times (adds stream syncs).
void build_graph(Graph& g, float alpha, int64_t max_batch, hipStream_t stream, bool time_stages,
                 BuildStats* stats);

// Radix sort of u64 keys (defined in sort.hip).
size_t sort_u64_temp_bytes(size_t max_items);
void sort_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, size_t n, int end_bit,
              hipStream_t stream);

}  // namespace jasper_amd
