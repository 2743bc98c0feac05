// build.hpp -- Vamana construction on the device (host driver).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>
#include <vector>

#include "graph.hpp"

namespace jasper_amd {

// Work counters of one build (filled only while work counting is on, see
// set_build_work_counting), indices of BuildStats::work:
enum BuildWork : int {
  kWorkSearchQueries = 0,   // rows searched by the search stage
  kWorkSearchHops,          // pops (one adjacency row each)
  kWorkSearchAdjacency,     // adjacency entries read (sum of degrees)
  kWorkSearchScored,        // distinct vectors scored, per query
  kWorkSearchVisited,       // popped keys written to the visited list
  kWorkForwardRows,         // vertices through the forward prune
  kWorkForwardExisting,     // existing edges read (ids + bf16 distances)
  kWorkForwardVisited,      // visited keys read
  kWorkForwardCandidates,   // candidate rows the prune reads (existing + visited, self excluded)
  kWorkForwardSelected,     // edges written (= reverse pairs)
  kWorkReverseTargets,      // targets through the reverse prune
  kWorkReverseExisting,     // their existing edges read
  kWorkReverseSources,      // reverse pairs read (sources taken)
  kWorkReverseSelected,     // edges written
  kWorkCount = 16
};

struct BuildStats {
  double search_ms = 0, prune_ms = 0, sort_ms = 0, reverse_ms = 0, total_ms = 0;
  int64_t batches = 0;
  int64_t max_batch = 0;
  uint64_t work[kWorkCount] = {};
};

// While on, builds count their work (BuildStats::work): the search stage
// runs the plain search's exact-counter instance (a per-query seen bitmap of
// n bits, so this mode is for measurement at moderate n; it refuses more than
// 8 GiB of bitmap) and the prune kernels add their counts. The graph built is
// the same. Process-wide; not for concurrent builds.
void set_build_work_counting(bool on);
bool build_work_counting();

// Maximum batch size of the reference for a workspace budget
// (graph_construct_workspace::max_batch_size_for_budget, index/construct.cuh:
// 238-262, capped at n/50 by ffi/jasper_ffi_common.cuh:245-248).
int64_t reference_max_batch(int64_t n, uint32_t R, int64_t budget_bytes);
// The same without the n/50 cap (the partitioned build's merges use it).
int64_t budget_max_batch(uint32_t R, int64_t budget_bytes);

// Builds the edges of `g` (vectors already resident) with the reference's
// batch schedule: batches of 1, 2, 4, ... up to max_batch over ids in order.
// `time_stages` records per-stage HIP-event times (adds stream syncs).
// rabitq_search: the search stage pops by the RaBitQ estimate (the graph's
// RaBitQ codes must exist; rabitq_build_search) instead of running the plain
// search; the rest of each batch is unchanged.
void build_graph(Graph& g, float alpha, int64_t max_batch, hipStream_t stream, bool time_stages,
                 BuildStats* stats, bool rabitq_search = false);

// The same per-batch steps over the vertices [first, last) only, in batches
// of 1, 2, 4, ... up to max_batch (doubling) or of max_batch; the rows of
// [first, last) must hold no edges yet.
void build_range(Graph& g, float alpha, int64_t first, int64_t last, int64_t max_batch, bool doubling,
                 hipStream_t stream, bool time_stages, BuildStats* stats, bool rabitq_search = false);

// The partitioned build (reference index/construct_scale.cuh:68-446, driven
// by cmd/create_scale_index.cu:57-98): the n rows of g (no edges yet) split
// into n_parts contiguous partitions of ceil(n / n_parts) rows, each built
// on its own (batches doubling to part_batch, search from its first row),
// then every pair merged once in scale_merge_order: B1 in batches of up to
// merge_batch searched in B2 alone (from B2's first row, edges leaving B2
// dropped), the forward merge prune into B1 and the reverse merge prune into
// B2, where a vector outside B1 and B2 is kept untested and prunes nothing
// (construct_scale_kernels.cuh:22-310). The whole graph stays in HBM: the
// reference stages partitions through host memory two at a time, which
// changes where rows live, not the result.
struct ScaleStats {
  double partition_ms = 0, merge_ms = 0, total_ms = 0;
  int64_t merges = 0, merge_batches = 0, part_batch = 0, merge_batch = 0;
};
std::vector<std::pair<int64_t, int64_t>> scale_merge_order(int64_t n_parts);
void build_scale(Graph& g, float alpha, int64_t n_parts, int64_t part_batch, int64_t merge_batch,
                 hipStream_t stream, ScaleStats* stats);
// The same build with the graph in pinned host memory (g.on_host, rows
// uploaded): each partition is built on the device and written back, and
// every merge runs with its two partitions in two device slots of ceil(n /
// n_parts) rows (the reference's staging, construct_scale.cuh:121-124,
// 398-445), so the device holds two partitions and the workspace, not the
// index. The graph is the in-HBM build's, edge for edge.
void build_scale_staged(Graph& g, float alpha, int64_t n_parts, int64_t part_batch, int64_t merge_batch,
                        hipStream_t stream, ScaleStats* stats);

// Live updates (reference construct.cuh:1169-1265, graph_ops.cuh:94-258).
// append_rows: copies `count` rows (host or device fp16 [count, dim]) into
// new slots, wires them in with build_range in batches of min(count, 100000),
// assigns fresh stable ids from next_id and writes them to out_ids (host or
// device int32 [count]).
void append_rows(Graph& g, const void* rows, int64_t count, float alpha, int32_t* out_ids, hipStream_t stream);
// mark_deleted: tombstones the given ids (slot == id; out-of-range ignored),
// replacing a deleted medoid. Returns the number newly deleted.
int64_t mark_deleted(Graph& g, const int32_t* ids, int64_t n_ids, hipStream_t stream);
// consolidate: repairs the edges of live vertices through deleted ones and
// clears the tombstones. Returns the number of repair candidates.
int64_t consolidate(Graph& g, float alpha, hipStream_t stream);

// Radix sort of u64 keys (defined in sort.hip).
size_t sort_u64_temp_bytes(size_t max_items);
// Stable: keys equal in bits [begin_bit, end_bit) keep their input order.
// in and out must differ; in is not written.
void sort_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, size_t n, int begin_bit,
              int end_bit, hipStream_t stream);
// Exclusive prefix sums of n u64 values (defined in sort.hip).
size_t scan_u64_temp_bytes(size_t max_items);
void exclusive_scan_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, size_t n,
                        hipStream_t stream);

}  // namespace jasper_amd
