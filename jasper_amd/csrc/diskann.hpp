// diskann.hpp -- the DiskANN build (reference index/construct_diskann.cuh).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "graph.hpp"

namespace jasper_amd {

struct DiskannStats {
  double assign_ms = 0, build_ms = 0, merge_ms = 0, total_ms = 0;
  int64_t shards = 0, max_shard = 0;
};

// Shard assignment of g's rows (assign_shards, construct_diskann.cuh:104-276):
// writes shard_of [n, n_dup] (0xFFFFFFFF where a rank repeats a shard) and
// the fp16 mean [dim] to host memory (either may be null).
void diskann_assign(const Graph& g, int64_t n_parts, int64_t n_dup, uint64_t seed, uint32_t* shard_of_host,
                    uint16_t* mean_host, hipStream_t s);

// The DiskANN build into g (rows uploaded, no edges; g.R = R_final):
// shards by cross-polytope LSH with n_dup copies, one graph of degree R_int
// per shard (batches doubling to min(batch_cap, shard size)), then the
// distance-only merge into g's rows, largest first (equal sizes by shard
// index, then sub-shard). A shard of more than max_shard rows (max_shard >
// 0) is built as equal sub-shards of its ascending ids, each at most
// max_shard rows (construct_diskann.cuh:386-417), so the shard graph never
// outgrows the device memory the caller gives it. medoid 0.
void build_diskann(Graph& g, uint32_t R_int, float alpha, int64_t n_parts, int64_t n_dup, uint64_t seed,
                   int64_t batch_cap, int64_t max_shard, hipStream_t s, DiskannStats* stats);

// Rows of the largest shard graph that fits the device's free memory after
// the construction workspace and 4 GB of slack (construct_diskann.cuh:
// 386-397), for rows of dim values and degree R_int.
int64_t diskann_max_shard_for_device(uint32_t dim, uint32_t R_int, int64_t workspace_budget);

}  // namespace jasper_amd
