// graph.hpp -- device-resident Vamana graph, flat structure-of-arrays.
//
// The reference keeps 2^20-vector segments behind a device array of segment
// structs (reference include/jasper/index/graph.cuh:92-496, 498-1066), which
// costs a dependent pointer load on every access. On MI355X the whole index
// fits one allocation per column (config 5, 100M x 128 with R = 64, is
// ~65 GB of the 288 GB of HBM), so every column here is one flat array
// indexed by vertex id:
//   vecs      fp16 [n, dp]   rows padded to dp = pad(dim) (16-byte rows)
//   edges     u32  [n, R]    adjacency rows (4R bytes: 256 B at R = 64)
//   edist     bf16 [n, R]    stored edge distances (construction only)
//   counts    u8   [n]       valid prefix length of each row
//   deleted   u32  [(n+31)/32] tombstone bits
//   slot_to_id u32 [n]       stable id of each slot (identity after build)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "directional.hpp"
#include "rotation.hpp"

namespace jasper_amd {

void hip_check(hipError_t e, const char* what);

inline uint32_t pad_dim(uint32_t d) { return (d + 7u) / 8u * 8u; }

struct Graph {
  uint32_t dim = 0, dp = 0, R = 0;
  int metric = 0;  // 0 = L2, 1 = IP
  int64_t n = 0;
  uint32_t medoid = 0;
  uint64_t next_id = 0;
  uint64_t n_deleted = 0;
  bool on_host = false;
  // directional configuration (0 for plain graphs)
  uint32_t k_ranks = 0;
  uint32_t packed_bytes = 0;

  void* vecs = nullptr;        // fp16
  // value range of vecs, written by scan_int_range wherever rows are
  // written: 0 = no rows, 1 = all values integers in [int_lo, int_hi],
  // 2 = some value is not an integer (or the scan is off)
  int int_state = 0;
  int32_t int_lo = 0, int_hi = -1;
  // byte rows for the search: value - vecs8_lo per value, u8 [vecs8_cap,
  // dim], kept by scan_int_range while the rows are integers spanning at
  // most 255 values (update_byte_rows); null otherwise
  uint8_t* vecs8 = nullptr;
  int64_t vecs8_cap = 0;
  int32_t vecs8_lo = 0;
  uint32_t* edges = nullptr;
  uint16_t* edist = nullptr;
  uint8_t* counts = nullptr;
  uint32_t* deleted = nullptr;
  uint32_t* slot_to_id = nullptr;

  // directional state (owned; null when absent)
  bool prerotate = false;
  uint64_t prerotate_seed = 42;
  std::unique_ptr<RotationMatrix> rotation;  // prerotation (MFMA layout)
  std::unique_ptr<LshArtifacts> lsh;
  std::unique_ptr<PqArtifacts> pq;
  std::unique_ptr<RabitqArtifacts> rabitq;
  float* vector_norms = nullptr;  // [n] ||x||^2

  Graph();
  Graph(const Graph&) = delete;
  Graph& operator=(const Graph&) = delete;
  ~Graph();

  void allocate(int64_t n_, uint32_t dim_, uint32_t R_, int metric_, bool on_host_);
  void release();
  // Grows the device arrays to hold at least `rows` vertices, keeping their
  // contents; new slots start empty (no edges, not deleted, no stable id).
  void reserve(int64_t rows, hipStream_t stream);
  int64_t capacity = 0;  // rows allocated (>= n)

  size_t vec_bytes() const { return (size_t)n * dp * 2; }
};

// File I/O, byte-compatible with the reference format
// (save_graph_to_file / load_graph_from_file, graph.cuh:1425-1788).
void save_graph_file(const Graph& g, const std::string& path);
std::unique_ptr<Graph> load_graph_file(const std::string& path, uint32_t dim, uint32_t R, int metric,
                                       bool on_host, uint64_t* trailer_offset);

// Host copies of the graph columns (for export and file writing).
struct HostGraph {
  std::vector<uint16_t> vecs;   // [n, dp]
  std::vector<uint32_t> edges;  // [n, R]
  std::vector<uint16_t> edist;  // [n, R]
  std::vector<uint8_t> counts;
  std::vector<uint32_t> deleted;
  std::vector<uint32_t> slot_to_id;
};
void download_graph(const Graph& g, HostGraph& h, bool with_vectors = true);

// Largest span S of integer values for which L2 sums over `dim` values are
// exact in any order: S <= 2,048 (exact fp16 differences) and dim * S^2 <
// 2^24 (exact fp32 partial sums).
int32_t int_exact_span(uint32_t dim);

// Scans device rows [row0, row0 + n) (synchronising `stream`) and records on
// the graph whether all stored values (padding included) are integers, and
// their range; with row0 > 0 the result is merged with what rows [0, row0)
// gave. Every path that writes rows (upload, load, prerotation) calls it
// there, so searches only read the result. JASPER_INT_EXACT=0 (measurement)
// records "not integers".
void scan_int_range(Graph& g, int64_t row0, int64_t n, hipStream_t stream);
// Whether the graph's rows qualify for byte rows: L2, device-resident,
// integers spanning at most 255 values, dim 112 or 128 (16-value byte
// chunks, four fp16 chunks per quad lane), and lo - 1024 an fp16 value (the
// search's query shift).
bool byte_rows_eligible(const Graph& g);
// Rewrites the byte rows of rows [0, rows) (or drops them) from the value
// range already recorded in g, for rows written without a range scan whose
// values lie in that range (the DiskANN build's shard graphs).
void refresh_byte_rows(Graph& g, int64_t rows, hipStream_t stream);

// The recorded result: true when every stored value is an integer in
// [int_lo, int_hi].
bool int_range(const Graph& g);

// True when L2 distances between stored rows are exact integers in any
// summation order (int_range holds and the span is within int_exact_span).
// lo_out receives the smallest value when the test passes.
bool int_exact_l2(const Graph& g, hipStream_t stream, int32_t* lo_out = nullptr);

// Uploads a contiguous host or device fp16 matrix [n, dim] into rows padded
// to dp on the device graph (vecs must be allocated).
void upload_vectors(Graph& g, const void* src, int64_t n, uint32_t dim, hipStream_t stream);

// Same into rows [row0, row0 + n) (within capacity).
void upload_rows(Graph& g, const void* src, int64_t row0, int64_t n, uint32_t dim, hipStream_t stream);

}  // namespace jasper_amd
