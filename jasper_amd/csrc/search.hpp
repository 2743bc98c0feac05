// search.hpp -- batched plain beam search (host entry points).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "graph.hpp"

namespace jasper_amd {

struct SearchRequest {
  const void* queries = nullptr;   // fp16 [nq, dp] device rows (ignored when use_range)
  uint32_t nq = 0;
  bool use_range = false;          // queries are graph rows [q_start, q_start + nq)
  uint32_t q_start = 0;
  uint32_t medoid = 0;
  uint32_t k = 10, beam_width = 64, limit = 128, max_result = 2048;
  int32_t* out_ids = nullptr;      // [nq, k] (may be null)
  float* out_dists = nullptr;      // [nq, k]
  uint64_t* visited = nullptr;     // [nq, max_result] popped keys in pop order (may be null)
  uint32_t* visited_counts = nullptr;
  uint32_t hash_bits = 0;          // 0 = choose from beam width
  // id window: neighbours outside [id_lo, id_lo + id_n) are dropped as the
  // reference drops ids past a graph's range (beam_search/device_kernels.cuh:
  // 95-129); id_n < 0 = the whole graph. The partitioned build's merge
  // searches one partition of the full graph this way.
  uint32_t id_lo = 0;
  int64_t id_n = -1;
  // measurement mode (exact seen set, work counters); both or neither
  uint32_t* seen_bits = nullptr;   // [nq, ceil(n/32)], zeroed by the caller
  uint32_t* stats = nullptr;       // [nq, 4]: hops, sum of degrees, vectors scored,
                                   // hops whose adjacency was read one hop ahead
};

// Launches the search kernel on `stream`; asynchronous.
void launch_beam_search(const Graph& g, const SearchRequest& r, hipStream_t stream);

// LDS bytes one query (one wave) uses for the given request.
size_t beam_search_lds_bytes(const Graph& g, const SearchRequest& r);

// log2 of the seen-cache entries for a graph of n vertices (queries and build).
uint32_t seen_cache_hash_bits(int64_t n);

}  // namespace jasper_amd
