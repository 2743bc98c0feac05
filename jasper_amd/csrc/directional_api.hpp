// directional_api.hpp -- host entry points of the directional path
// (reference DEFINE_DIRECTIONAL_OPS, ffi/jasper_ffi_common.cuh:442-775).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <memory>
#include <string>

#include "build.hpp"
#include "graph.hpp"

namespace jasper_amd {

// The directional configs come in two dim buckets (reference
// python/jasper/__init__.py:66-84): packed_t = u8 for dim <= 128, u16 above.
void check_directional_dim(bool small_dim, int64_t dim);

// options of construct_directional (jasperx_construct_directional_ex)
constexpr uint32_t kBuildRabitqSearch = 1u;  // RaBitQ codes first, then the RaBitQ build search
constexpr uint32_t kBuildOptionsKnown = kBuildRabitqSearch;
std::unique_ptr<Graph> construct_directional(uint32_t R, int metric, uint32_t k_ranks, bool small_dim,
                                             const void* vectors, int64_t n, int64_t dim, double alpha,
                                             int64_t budget, bool on_host, bool prerotate, uint64_t seed,
                                             hipStream_t stream, BuildStats* stats, uint32_t options = 0);
void build_lsh(Graph& g, int64_t n_samples, uint64_t seed);
// m = number of subspaces (0: the config's k_ranks, as the reference, whose
// pq_m equals k_ranks); any m dividing the padded dim, up to kPqMaxM.
void build_pq(Graph& g, int64_t n_train, int64_t iters, uint64_t seed, uint32_t m = 0);
// RaBitQ one-bit codes of the stored rows (the reference's quantizer,
// rabitq/quantize.cuh:322-354, on the rows as stored) against their mean.
void build_rabitq(Graph& g);
// The construction's search stage with the RaBitQ estimator (an extension;
// the reference's is the plain search, construct.cuh:778-794): the
// directional traversal of rows [q_start, q_start + nq) as queries, popped
// by estimate, each visit scored with the plain search's distance and
// recorded as a key in visited[i * max_result + j] (count in
// visited_counts[i]), the record build_range's forward prune reads.
void rabitq_build_search(const Graph& g, uint32_t q_start, uint32_t nq, uint32_t bw, uint32_t limit,
                         uint32_t max_result, uint64_t* visited, uint32_t* visited_counts, hipStream_t stream);
// directional estimators (jasperx_directional_search_ex's estimator id)
constexpr int kEstLsh = 0, kEstPq = 1, kEstRabitq = 2;
// option flags of jasperx_directional_search_ex
constexpr uint32_t kDirUnique = 1u;
constexpr uint32_t kDirFlagsKnown = kDirUnique;

// stats (optional, device [nq * 3]): per query visits, hops expanded and
// adjacency entries read. unique: skip pops of ids already in the frontier,
// so the k results are distinct (an extension; the reference re-visits them).
void directional_search(Graph& g, int est, const void* queries, int64_t nq, int64_t dim, int32_t* out_ids,
                        float* out_dists, int64_t k, int64_t bw, int64_t limit, bool print, hipStream_t stream,
                        uint32_t* stats = nullptr, bool unique = false);
// The plain (exact-distance) beam search over any graph's stored rows, the
// queries padded and, for a prerotated graph, rotated as the directional
// search does: what the graph itself allows, without an estimator.
void exact_search(Graph& g, const void* queries, int64_t nq, int64_t dim, int32_t* out_ids, float* out_dists,
                  int64_t k, int64_t bw, int64_t limit, hipStream_t stream);
// Device scratch bytes a directional search of nq queries takes (query
// rows, their rotation, PQ tables).
size_t directional_scratch_bytes(const Graph& g, int est, int64_t nq);
// The same search with its scratch carved from [scratch_base,
// scratch_base + scratch_bytes): it allocates nothing and throws before
// launching anything when the call needs more. Queries must be device
// memory; there is no print_throughput and no work counters.
void directional_search_fixed(Graph& g, int est, const void* queries, int64_t nq, int64_t dim, int32_t* out_ids,
                              float* out_dists, int64_t k, int64_t bw, int64_t limit, bool unique, hipStream_t stream,
                              void* scratch_base, size_t scratch_bytes);
// directional_search_fixed on a static device scratch of
// directional_noalloc_scratch_bytes() per GPU (no allocation at all). Calls
// that overlap on one GPU share that scratch and race.
size_t directional_noalloc_scratch_bytes();
void directional_search_noalloc(Graph& g, int est, const void* queries, int64_t nq, int64_t dim,
                                int32_t* out_ids, float* out_dists, int64_t k, int64_t bw, int64_t limit,
                                bool unique, hipStream_t stream);
// The query rows the directional kernels read (padded, rotated when the
// graph was prerotated), copied to host memory [nq, padded_dim].
void directional_query_rows_to_host(const Graph& g, const void* queries, int64_t nq, int64_t dim, uint16_t* out,
                                    hipStream_t stream);
// A graph's PQ codes as the reference's subspace-major rows, host
// out[n][m][R] (the file and export layout).
void pq_codes_to_file_layout(const Graph& g, uint8_t* out);
void save_directional_file(const Graph& g, const std::string& path);
std::unique_ptr<Graph> load_directional_file(const std::string& path, uint32_t dim, uint32_t R, int metric,
                                             uint32_t k_ranks, bool small_dim, bool on_host, bool prerotate,
                                             uint64_t seed);

}  // namespace jasper_amd
