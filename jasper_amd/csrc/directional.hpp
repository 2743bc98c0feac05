// directional.hpp -- per-graph artifacts of the directional estimators.
#pragma once

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
struct PqArtifacts {
  uint32_t m = 0, k = 256, dsub = 0;
  float* centroids = nullptr;        // device [m*256*dsub]
  uint8_t* codes = nullptr;          // device [n, m*R] subspace-major per row
  ~PqArtifacts();
};

}  // namespace jasper_amd
