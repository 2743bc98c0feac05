// directional.hpp -- per-graph artifacts of the directional estimators.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <vector>

namespace jasper_amd {

// Cross-polytope LSH calibration and per-edge words
// (reference lsh/lsh_globals.cuh:11-15, lsh/edge_lsh.cuh:9-27).
struct LshArtifacts {
  uint32_t k_ranks = 0;
  uint32_t packed_bytes = 0;         // 1 (dim <= 128) or 2
  std::vector<float> c_per_rank;     // [k_ranks]
  float norm_denom = 0.0f;
  void* rows = nullptr;              // device [n, R*k_ranks*packed_bytes + 2R (bf16 mag^2)]
  size_t row_bytes = 0;
  ~LshArtifacts();
};

// Product-quantization codebooks and per-edge codes
// (reference pq/pq_codebooks.cuh:20-66, pq/edge_pq.cuh:23-50).
//
// Device codes are edge-interleaved: a vertex's row is [G][R][W] with W
// codes per group (W = 4, 8 or 16 by m) and G = ceil(m / W) groups, so the
// codes of subspaces W*g .. W*g + W - 1 for edge e are W consecutive bytes
// and one lane reads its edge's codes with G loads of W bytes. Bytes of
// subspaces >= m in the last group are zero. The file trailer and
// jasperx_export_pq use the reference's subspace-major rows [m][R]
// (code[j * R + e]).
struct PqArtifacts {
  uint32_t m = 0, k = 256, dsub = 0;
  float* centroids = nullptr;        // device [m*256*dsub]
  uint8_t* codes = nullptr;          // device [n][G][R][W] (above)
  ~PqArtifacts();
};

// RaBitQ one-bit codes of the stored rows, in the reference's node layout
// (rabitq_data_store<float>, rabitq/layout.cuh:43-143: code bytes =
// ceil(dim/8) rounded up to 4, bits LSB-first, then f_add and f_rescale),
// taken against `centroid` (the mean of the stored rows) with no further
// rotation: on a prerotated graph the rows already went through P^T.
struct RabitqArtifacts {
  uint32_t dim = 0, code_bytes = 0;
  void* nodes = nullptr;             // device [n, code_bytes + 8]
  float* centroid = nullptr;         // device [dim]
  ~RabitqArtifacts();
};

// (constexpr: usable in host and device code)
constexpr uint32_t pq_group_width(uint32_t m) { return m <= 4 ? 4u : m <= 8 ? 8u : 16u; }
constexpr uint32_t pq_groups(uint32_t m) { return (m + pq_group_width(m) - 1) / pq_group_width(m); }
// device bytes of one vertex's codes
constexpr size_t pq_row_bytes(uint32_t m, uint32_t R) { return (size_t)pq_groups(m) * R * pq_group_width(m); }
// subspaces a graph's PQ may have: the search keeps 8 groups of 16 codes per
// edge in registers and the query's table (m KB) in LDS
constexpr uint32_t kPqMaxM = 128;

}  // namespace jasper_amd
