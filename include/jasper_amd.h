/* jasper_amd.h -- C ABI of the MI355X Jasper hot path (libjasper_amd.so).
 *
 * Drop-in boundary for the reference's TVM-FFI exports
 * (reference ffi/jasper_ffi_common.cuh:208-807, ffi/jasper_ffi_plain.cu:19-131):
 * the same symbol names `jasper_<op>_<config>`, the same argument order and
 * meaning. Tensor arguments of the reference become a raw pointer plus the
 * sizes the reference read from the tensor; every call that launches device
 * work also takes the HIP stream to run on (NULL = the default stream).
 *
 * Conventions
 *   - Every function returns int64_t. A negative value is an error; the
 *     message is available from jasper_last_error() (thread-local). The
 *     reference raised TVM_FFI_ICHECK failures and C++ exceptions as Python
 *     exceptions (ffi/jasper_ffi_common.cuh:226, beam_search/api.cuh:70-72);
 *     the Python package turns a negative return into the same exceptions.
 *   - Handles are non-negative int64 ids into a process-wide table
 *     (ffi/jasper_ffi_plain.cu:11-13).
 *   - Vectors and queries are contiguous [n, dim] fp16 rows (device or
 *     host memory for construction; device memory for queries). Rows need no
 *     padding: dim need not be a multiple of 8 (fixes the reference's
 *     stride assumption, vector.cuh:20-22).
 *   - Search outputs are device int32 [n_queries, k] ids and fp32
 *     [n_queries, k] distances.
 *
 * Plain configs (reference _CONFIGS, python/jasper/__init__.py:29-38):
 *   f16_r{8,16,32,64}_{l2,ip}
 * Directional configs (reference _DIRECTIONAL_CONFIGS, __init__.py:66-84):
 *   f16_r{32,64}_{l2,ip}_k{4,16}_d{128,32678}
 */
#ifndef JASPER_AMD_H
#define JASPER_AMD_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JASPER_PLAIN_CONFIGS(X) \
  X(f16_r8_l2) X(f16_r16_l2) X(f16_r32_l2) X(f16_r64_l2) \
  X(f16_r8_ip) X(f16_r16_ip) X(f16_r32_ip) X(f16_r64_ip)

#define JASPER_DIRECTIONAL_CONFIGS(X) \
  X(f16_r32_l2_k4_d128) X(f16_r32_l2_k4_d32678) X(f16_r64_l2_k4_d128) X(f16_r64_l2_k4_d32678) \
  X(f16_r32_l2_k16_d128) X(f16_r32_l2_k16_d32678) X(f16_r64_l2_k16_d128) X(f16_r64_l2_k16_d32678) \
  X(f16_r32_ip_k4_d128) X(f16_r32_ip_k4_d32678) X(f16_r64_ip_k4_d128) X(f16_r64_ip_k4_d32678) \
  X(f16_r32_ip_k16_d128) X(f16_r32_ip_k16_d32678) X(f16_r64_ip_k16_d128) X(f16_r64_ip_k16_d32678)

/* ---- per plain config (DEFINE_OPS, ffi/jasper_ffi_common.cuh:208-431) ---- */
#define JASPER_DECLARE_PLAIN(id)                                                              \
  /* LoadGraph_ :210-219 -> handle */                                                         \
  int64_t jasper_load_##id(const char* path, int64_t dim, bool on_host);                      \
  /* ConstructGraph_ :232-261 -> handle; vectors [n_vectors, dim] fp16 */                     \
  int64_t jasper_construct_##id(const void* vectors, int64_t n_vectors, int64_t dim,          \
                                double alpha, int64_t workspace_budget_bytes, bool on_host,   \
                                void* stream);                                                \
  /* Search_ :302-369; queries [n_queries, dim] fp16 on device */                             \
  int64_t jasper_search_##id(int64_t handle, const void* queries, int64_t n_queries,          \
                             int64_t dim, int32_t* out_indices, float* out_distances,         \
                             int64_t k, int64_t beam_width, int64_t limit,                    \
                             bool print_throughput, void* stream);                            \
  /* SaveGraph_ :221-230 */                                                                   \
  int64_t jasper_save_##id(int64_t handle, const char* path);                                 \
  /* GetVector_ :263-300; out: [dim] fp16 device */                                           \
  int64_t jasper_get_vector_##id(int64_t handle, int64_t stable_id, void* out, void* stream); \
  /* MarkDeleted_ :371-386; ids: host int32 [n_ids] */                                        \
  int64_t jasper_mark_deleted_##id(int64_t handle, const int32_t* ids, int64_t n_ids);        \
  /* Consolidate_ :388-397 */                                                                 \
  int64_t jasper_consolidate_##id(int64_t handle, double alpha);                              \
  /* Compact_ :399-408: returns an error, as the reference's default build                  \
   * (graph_ops.cuh:265-270, JASPER_ENABLE_COMPACT off) */                                    \
  int64_t jasper_compact_##id(int64_t handle);                                                \
  /* Append_ :412-430; out_ids: host int32 [n_vectors] */                                     \
  int64_t jasper_append_##id(int64_t handle, const void* vectors, int64_t n_vectors,          \
                             double alpha, int32_t* out_ids, void* stream);

/* ---- per directional config (DEFINE_DIRECTIONAL_OPS, :442-775) ---- */
#define JASPER_DECLARE_DIRECTIONAL(id)                                                        \
  /* ConstructDirectionalGraph_ :444-486 -> handle */                                         \
  int64_t jasper_construct_directional_##id(const void* vectors, int64_t n_vectors,           \
                                            int64_t dim, double alpha,                        \
                                            int64_t workspace_budget_bytes, bool on_host,     \
                                            bool prerotate, int64_t prerotate_seed,           \
                                            void* stream);                                    \
  /* BuildLsh_ :488-505 */                                                                    \
  int64_t jasper_build_lsh_##id(int64_t handle, int64_t n_samples, int64_t seed);             \
  /* BuildPq_ :507-528 */                                                                     \
  int64_t jasper_build_pq_##id(int64_t handle, int64_t n_train, int64_t kmeans_iter,          \
                               int64_t seed);                                                 \
  /* DirectionalSearch_ :530-608 */                                                           \
  int64_t jasper_directional_search_##id(int64_t handle, const void* queries,                 \
                                         int64_t n_queries, int64_t dim,                      \
                                         int32_t* out_indices, float* out_distances,          \
                                         int64_t k, int64_t beam_width, int64_t limit,        \
                                         bool print_throughput, void* stream);                \
  /* PqSearch_ :610-688 */                                                                    \
  int64_t jasper_pq_search_##id(int64_t handle, const void* queries, int64_t n_queries,       \
                                int64_t dim, int32_t* out_indices, float* out_distances,      \
                                int64_t k, int64_t beam_width, int64_t limit,                 \
                                bool print_throughput, void* stream);                         \
  /* SaveDirectionalGraph_ :690-710 */                                                        \
  int64_t jasper_save_directional_##id(int64_t handle, const char* path);                     \
  /* LoadDirectionalGraph_ :712-733 -> handle */                                              \
  int64_t jasper_load_directional_##id(const char* path, int64_t dim, bool on_host,           \
                                       bool prerotate, int64_t prerotate_seed);               \
  /* GetVectorDirectional_ :735-763 */                                                        \
  int64_t jasper_get_vector_directional_##id(int64_t handle, int64_t index, void* out,        \
                                             void* stream);                                   \
  /* GetDirectionalFlags_ :765-775: bit 0 = LSH, bit 1 = PQ; bit 3 = prerotated rows,        \
   * bit 4 = RaBitQ codes (both extensions) */                                                \
  int64_t jasper_get_directional_flags_##id(int64_t handle);

JASPER_PLAIN_CONFIGS(JASPER_DECLARE_PLAIN)
JASPER_DIRECTIONAL_CONFIGS(JASPER_DECLARE_DIRECTIONAL)

/* ---- config-agnostic (ffi/jasper_ffi_plain.cu:19-131) ---- */
int64_t jasper_free_graph(int64_t handle);            /* FreeGraph :19-47 */
int64_t jasper_get_n_vectors(int64_t handle);         /* GetNumVectors :50-61 */
int64_t jasper_get_n_tombstoned(int64_t handle);      /* GetNumTombstoned :63-74 */
int64_t jasper_get_n_live(int64_t handle);            /* GetNumLive :96-107 */
int64_t jasper_reserve_ids(int64_t handle, int32_t* out_ids, int64_t count); /* ReserveIds :78-94 */
int64_t jasper_get_dim(int64_t handle);               /* GetDim :109-120 */

/* Error message of the last failed call on this thread (no reference
 * counterpart: TVM-FFI carried the message in the raised exception). */
const char* jasper_last_error(void);

/* ---- extensions without a reference counterpart ----
 * For parity tests and measurement: copy a graph's columns to host buffers
 * (edges [n, R] u32, edge distances [n, R] bf16 bits, counts [n] u8; any
 * pointer may be NULL), and the per-stage timing of the last construction
 * (ms: search, forward prune, reverse grouping, reverse prune, total;
 * plus batches and max batch size) when JASPER_BUILD_TIMING=1 was set. */
int64_t jasperx_export_graph(int64_t handle, uint32_t* edges, uint16_t* edge_dist, uint8_t* counts);
int64_t jasperx_last_build_stats(double* out7);
/* Build work counting (measurement; no reference counterpart): while on != 0,
 * constructions count their work and jasperx_last_build_work copies the 16
 * counters of the last one: rows searched, search pops, adjacency entries,
 * distinct vectors scored, visited keys written, forward-prune rows, their
 * existing edges, visited keys read, candidate rows, edges written, reverse
 * targets, their existing edges, reverse pairs read, edges written (the rest
 * zero). The search stage then runs with an exact per-query seen bitmap
 * (n bits per row of a batch; refused above 8 GiB); the graph is the same. */
int64_t jasperx_build_work_counting(int64_t on);
int64_t jasperx_last_build_work(uint64_t* out16);
/* Measurement run of the plain search: same traversal with an exact
 * per-query seen set, writing per-query work counters to host memory
 * out_stats[n_queries * 4] = {hops, sum of degrees read, vectors scored,
 * hops whose adjacency row was read one hop ahead}.
 * Used to compute algorithmic bytes per launch; not a search entry point. */
int64_t jasperx_search_stats(int64_t handle, const void* queries, int64_t n_queries, int64_t dim,
                             int64_t k, int64_t beam_width, int64_t limit, uint32_t* out_stats,
                             void* stream);
/* Host copies of a graph's device columns for parity tests: vectors
 * [n, padded_dim] fp16 bits (after prerotation when enabled; returns
 * padded_dim); LSH calibration (k_ranks floats, norm_denom) and per-edge
 * rows [n, row_bytes] (returns row_bytes); PQ centroids [M*256*dsub] f32,
 * codes [n, M*R] and vector norms [n] (returns dsub). NULL skips a part. */
int64_t jasperx_export_vectors(int64_t handle, uint16_t* out);
int64_t jasperx_export_lsh(int64_t handle, float* c_per_rank, float* norm_denom, uint8_t* rows);
int64_t jasperx_export_pq(int64_t handle, float* centroids, uint8_t* codes, float* norms);
/* The query rows a directional search reads (padded to padded_dim, and
 * rotated when the graph was prerotated), written to host memory
 * out[n_queries * padded_dim] as fp16 bits; returns padded_dim. */
int64_t jasperx_directional_query_rows(int64_t handle, const void* queries, int64_t n_queries, int64_t dim,
                                       uint16_t* out, void* stream);
/* The prerotation matrix for (dim, seed), column-major f32 [dim*dim], as
 * set_rotation_matrix returns it before the fp16 cast (reference
 * include/jasper/rotation/rotation.cuh:71-111). Host-only. */
int64_t jasperx_rotation_matrix(int64_t dim, int64_t seed, float* out);
/* Rotate fp16 rows by that matrix on the GPU: out[r][i] = fp16(sum_k
 * P[k + i*dim] * x[r][k]) with fp32 accumulation (the prerotation of
 * include/jasper/index/construct.cuh:1068-1090 as an operator). x: n rows of
 * stride x_stride elements (device or host memory); out: device, stride
 * out_stride. Asynchronous on `stream` (matrices are cached per device, dim
 * and seed). */
int64_t jasperx_rotate_rows(int64_t dim, int64_t seed, const void* x, int64_t n, int64_t x_stride, void* out,
                            int64_t out_stride, void* stream);
/* One-bit RaBitQ quantizer (include/jasper/rabitq/quantize.cuh:322-354,
 * rabitq_quantize<1>; the reference has no FFI binding for it). vectors:
 * device rows, dtype 0 = fp16 (stride a multiple of 8, 16-byte aligned) or
 * 1 = fp32, row stride `stride` elements; rotation: device fp32 [dim*dim]
 * column-major; centroid: device fp32 [dim] or NULL (zero); metric 0 = L2,
 * 1 = IP; out: device [n * node_bytes], node = code bytes (ceil(dim/8)
 * rounded up to 4, bits LSB-first) + f_add + f_rescale (fp32). Returns
 * node_bytes; supports dim <= 256. Asynchronous on `stream`. */
int64_t jasperx_rabitq_node_bytes(int64_t dim);
int64_t jasperx_rabitq_quantize(const void* vectors, int32_t dtype, int64_t n, int64_t dim, int64_t stride,
                                const float* rotation, const float* centroid, int32_t metric, void* out,
                                void* stream);
/* Exact k-NN by brute force on the matrix cores (the ground-truth utility
 * generate_groundtruth, python/jasper/__init__.py:828-926, which the
 * reference runs in torch): L2 = (||q||^2 + ||v||^2) - 2 q.v in fp32 clamped
 * at 0; IP = -(fp16(q.v)). base [n][stride] and queries [nq][stride] are
 * device fp16 rows padded with zeros to stride = the next multiple of 8 of
 * dim, 16-byte aligned. Results (device) ordered by (distance, id); k <= 128,
 * padded dim <= 4096. Asynchronous on `stream`. */
int64_t jasperx_bruteforce_knn(const void* base, int64_t n, int64_t dim, int64_t base_stride, const void* queries,
                               int64_t n_queries, int64_t query_stride, int64_t k, int32_t metric,
                               int32_t* out_ids, float* out_dists, void* stream);
/* build_pq with m subspaces instead of the config's k_ranks (the
 * reference's pq_m is k_ranks, graph.cuh:89, so it offers 4 or 16): any m
 * that divides the padded dim, up to 128 (one subspace per 8 dims at
 * d = 960 is m = 120). The file trailer records m; this library's loader
 * reads it back. Otherwise as jasper_build_pq_<cfg> (BuildPq_,
 * ffi/jasper_ffi_common.cuh:507-528). No reference counterpart. */
int64_t jasperx_build_pq_m(int64_t handle, int64_t m, int64_t n_train, int64_t kmeans_iter, int64_t seed);
/* The plain beam search (Search_, ffi/jasper_ffi_common.cuh:302-369) on any
 * graph, directional ones included: exact distances over the stored rows,
 * the queries padded and, on a prerotated graph, rotated as the directional
 * search rotates them. It shows what a directional graph allows without an
 * estimator; the reference offers no search() on directional graphs
 * (python/jasper/__init__.py:469-475). Outputs as jasper_search_<cfg>. */
int64_t jasperx_exact_search(int64_t handle, const void* queries, int64_t n_queries, int64_t dim, int32_t* out_ids,
                             float* out_dists, int64_t k, int64_t beam_width, int64_t limit, void* stream);
/* jasper_construct_directional_<config> (ConstructDirectionalGraph_,
 * ffi/jasper_ffi_common.cuh:444-486) with the config named by its id (e.g.
 * "f16_r64_l2_k16_d128") and option bits; no reference counterpart.
 * JASPERX_BUILD_RABITQ_SEARCH computes the RaBitQ codes of the stored rows
 * first (jasperx_build_rabitq) and lets the construction's search stage pop
 * by the RaBitQ estimate (each popped row is scored exactly, as the plain
 * build search does); forward prune, grouping and reverse prune are
 * unchanged. options = 0 is the reference construction. */
#define JASPERX_BUILD_RABITQ_SEARCH 1u
int64_t jasperx_construct_directional_ex(const char* config, const void* vectors, int64_t n_vectors, int64_t dim,
                                         double alpha, int64_t workspace_budget_bytes, bool on_host,
                                         bool prerotate, int64_t prerotate_seed, uint32_t options, void* stream);
/* The partitioned build of cmd/create_scale_index.cu:57-98 (the reference
 * exposes it only as that command; no FFI binding): include/jasper/index/
 * construct_scale.cuh intermediate_graph::allocate_and_construct (:83-128)
 * with n_parts partitions of ceil(n / n_parts) rows, then merge() (:378-446).
 * config: a plain config id (e.g. "f16_r64_l2"); vectors [n_vectors, dim]
 * fp16 (host or device); partitions are built in batches of up to
 * min(budget batch, max_batch_size), max_batch_size <= 0 meaning the
 * command's n / n_parts / 20; merges in batches of the budget batch.
 * on_host = false: the graph is resident in device memory. on_host = true:
 * the graph lives in pinned host memory and the build stages partitions
 * through it, two on the device at a time (the reference's staging,
 * construct_scale.cuh:121-124, 398-445), for indexes larger than HBM; the
 * graph is the same edge for edge. Returns a plain-config handle (search /
 * save / updates as for jasper_construct_<config>; an on_host graph as a
 * graph loaded with on_host). Errors: a partition would be empty, a budget
 * below one batch item. */
int64_t jasperx_construct_scale(const char* config, const void* vectors, int64_t n_vectors, int64_t dim,
                                double alpha, int64_t n_parts, int64_t workspace_budget_bytes,
                                int64_t max_batch_size, bool on_host, void* stream);
/* Times of the last partitioned build: {partition builds ms, merges ms,
 * total ms, merges, merge batches, partition batch size, merge batch
 * size}. */
int64_t jasperx_last_scale_stats(double* out7);
/* The DiskANN build of cmd/create_diskann_index.cu:59-103 (no FFI binding in
 * the reference): include/jasper/index/construct_diskann.cuh
 * diskann_intermediate_graph::build (:328-613). Rows go to n_dup shards by
 * cross-polytope LSH (centred on the sampled mean, rotated by the seed's
 * orthogonal matrix; the reference uses seed 42), each shard is built as its
 * own graph of degree r_int (batches doubling to min(budget batch,
 * max_batch_size); max_batch_size <= 0 takes the command's n / n_parts / 20),
 * and the shards' rows are merged by stored distance into rows of the
 * config's R (the reference's configs: r_int 32 with R 32 or 64). config: a
 * plain config id; vectors [n_vectors, dim] fp16 (host or device), dim <=
 * 1024; n_dup <= 16. A shard of more than max_shard rows is built as equal
 * sub-shards (construct_diskann.cuh:386-417); max_shard <= 0 takes the
 * largest shard graph the free device memory holds after the workspace and
 * 4 GB. Returns a plain-config handle. Tasks of equal size are merged in
 * (shard, sub-shard) order (the reference leaves that order unspecified). */
int64_t jasperx_construct_diskann(const char* config, const void* vectors, int64_t n_vectors, int64_t dim,
                                  double alpha, int64_t r_int, int64_t n_parts, int64_t n_dup,
                                  int64_t workspace_budget_bytes, int64_t max_batch_size, int64_t seed,
                                  int64_t max_shard, void* stream);
/* The shard assignment alone (assign_shards, construct_diskann.cuh:104-276)
 * for tests: out_shard_of [n_vectors * n_dup] (0xFFFFFFFF where a rank
 * repeats a shard) and out_mean [dim] fp16 bits, host memory, either NULL. */
int64_t jasperx_diskann_assign(const void* vectors, int64_t n_vectors, int64_t dim, int64_t n_parts, int64_t n_dup,
                               int64_t seed, uint32_t* out_shard_of, uint16_t* out_mean, void* stream);
/* Times of the last DiskANN build: {assignment ms, shard builds ms, merges
 * ms, total ms, shards, largest shard}. */
int64_t jasperx_last_diskann_stats(double* out6);
/* One-bit RaBitQ codes of a directional graph's stored rows (rotated rows
 * when prerotated): the reference's quantizer (rabitq/quantize.cuh:322-354)
 * on the rows as stored, against their mean; they feed the RaBitQ estimator
 * (estimator 2 below) and are saved in the trailer (flag 16). No reference
 * counterpart (the reference has no RaBitQ estimator: rabitq/distance.cuh
 * holds only the metric enum). */
int64_t jasperx_build_rabitq(int64_t handle);
/* Host copies of the RaBitQ codes: centroid [dim] f32 and nodes
 * [n, node_bytes] (code bytes, f_add, f_rescale); returns node_bytes. NULL
 * skips a part. */
int64_t jasperx_export_rabitq(int64_t handle, float* centroid, uint8_t* nodes);
/* The directional search with estimator 0 = LSH (directional_search),
 * 1 = PQ (pq_search) or 2 = RaBitQ (an extension: the one-bit estimator
 * est = f_add + g_add + f_rescale * <b - 1/2, q'> over the neighbour's
 * code b and the query quantized to 4 bits, inner product by popcounts),
 * with option flags; no reference counterpart. JASPERX_DIR_UNIQUE skips every pop of a
 * node already in the exact top-k list: the reference's traversal
 * (graph_beam_search.cuh:160-206) re-visits such nodes and inserts them
 * into that list again, so one node can fill several of the k slots. With
 * the flag the k results are distinct ids. flags = 0 is the reference's
 * traversal, identical to jasper_directional_search_<cfg>. Queries, outputs
 * and stream as for jasper_directional_search_<cfg>. */
#define JASPERX_DIR_UNIQUE 1u
int64_t jasperx_directional_search_ex(int64_t handle, int32_t estimator, const void* queries, int64_t n_queries,
                                      int64_t dim, int32_t* out_ids, float* out_dists, int64_t k,
                                      int64_t beam_width, int64_t limit, uint32_t flags, void* stream);
/* No reference counterpart; for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The same search as jasperx_directional_search_ex (same
 * arguments, flags and results) with its scratch -- the padded query rows,
 * their rotation for prerotated graphs and pq_search's per-query tables --
 * in a static 64 MiB device buffer per GPU instead of stream-ordered
 * allocations; nothing is allocated or freed. A call takes 2 * padded_dim
 * bytes per query for the rows (twice that on a prerotated graph) plus
 * m * 1 KB per query for pq_search, each part rounded up to 256 bytes; one
 * that needs more than 64 MiB is rejected before anything runs (split such
 * batches: e.g. at most ~4,000 queries for pq_search with m = 16 at d = 128,
 * ~540 with m = 120 at d = 960). Queries must be device memory.
 * Every call on a GPU shares that GPU's buffer, so calls that overlap on one
 * GPU (other streams, other threads) race. */
int64_t jasperx_directional_search_noalloc(int64_t handle, int32_t estimator, const void* queries,
                                           int64_t n_queries, int64_t dim, int32_t* out_ids, float* out_dists,
                                           int64_t k, int64_t beam_width, int64_t limit, uint32_t flags,
                                           void* stream);
/* Measurement run of the directional search with an estimator as above
 * (0 LSH, 1 PQ, 2 RaBitQ), flags as above: the same traversal, writing per-query work
 * counters to host memory out_stats[n_queries * 3] = {visits, hops
 * expanded, adjacency entries read}. Not a search entry point. */
int64_t jasperx_directional_stats(int64_t handle, int32_t estimator, const void* queries, int64_t n_queries,
                                  int64_t dim, int64_t k, int64_t beam_width, int64_t limit, uint32_t flags,
                                  uint32_t* out_stats, void* stream);
/* The prerotation seed of a directional graph (-1 when its rows are not
 * prerotated). Directional files written by this build record the
 * prerotation in the trailer (flag 8, a u64 seed after the other sections;
 * readers of flags 1, 2 and 4 stop before it), and loading them restores it
 * whatever prerotate/seed the caller passed. No reference counterpart. */
int64_t jasperx_prerotate_seed(int64_t handle);
/* The row formats the graph keeps: out4 = {value state (0 no rows, 1 all
 * values integers in [lo, hi], 2 otherwise), lo, hi, byte rows (1 when the
 * search reads the rows as bytes value - lo: L2, integers spanning at most
 * 255 values, dim 112 or 128; JASPER_SEARCH_BYTES=0 turns them off)}. No
 * reference counterpart (an inspection call for tests and tooling). */
int64_t jasperx_row_format(int64_t handle, int64_t* out4);
/* Library build identifier (git-independent), for load checks. */
const char* jasperx_version(void);

#ifdef __cplusplus
}
#endif

#endif /* JASPER_AMD_H */
