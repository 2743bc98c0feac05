// directional.hip -- directional (estimator-driven) path: prerotation, LSH
// and PQ artifacts, the directional beam search, and the file trailer.
//
// References: graph_beam_search.cuh:55-347 (skeleton), beam_search_common.cuh:
// 87-185 (exact visit, frontier list), directional_beam_search.cuh:31-192
// (LSH estimator), pq_beam_search.cuh:32-201 (PQ estimator),
// lsh/lsh_globals.cuh + lsh/lsh_kernels.cuh (LSH artifacts),
// pq/pq_kernels.cuh (PQ artifacts), rotation/rotation.cuh (rotation),
// index/graph.cuh:1790-2093 (trailer), ffi/jasper_ffi_common.cuh:442-775.
//
// Reductions reproduce the reference's 128-thread trees exactly: a query is
// one wave64 whose lane l plays virtual threads l and l + 64; each 32-lane
// half runs the warp's xor butterfly (16, 8, 4, 2, 1) and the four warp sums
// w0..w3 combine as (w0 + w2) + (w1 + w3), which is what the second-stage
// butterfly over {w0, w1, w2, w3, 0, ...} computes.
#include "build.hpp"
#include "common.hpp"
#include "directional.hpp"
#include "directional_api.hpp"
#include "rabitq.hpp"
#include "rotation.hpp"
#include "search.hpp"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <mutex>
#include <stdexcept>
#include <vector>

namespace jasper_amd {

LshArtifacts::~LshArtifacts() {
  if (rows) (void)hipFree(rows);
}

PqArtifacts::~PqArtifacts() {
  if (centroids) (void)hipFree(centroids);
  if (codes) (void)hipFree(codes);
}

RabitqArtifacts::~RabitqArtifacts() {
  if (nodes) (void)hipFree(nodes);
  if (centroid) (void)hipFree(centroid);
}

constexpr uint32_t kInv31 = 0x7FFFFFFFu;
constexpr uint32_t kTrailerMagic = 0x484C5344u;   // graph.cuh:1815
constexpr uint32_t kTrailerVersion = 1u;

void check_directional_dim(bool small_dim, int64_t dim) {
  if (small_dim ? dim > 128 : dim <= 128)
    throw std::invalid_argument("dim " + std::to_string(dim) + " does not match the config's dim bucket");
}

// ------------------------------------------------------------- fp16 ops --

__device__ __forceinline__ uint32_t hsub2_bits(uint32_t a, uint32_t b) {
  __half2 x = *reinterpret_cast<__half2*>(&a), y = *reinterpret_cast<__half2*>(&b);
  __half2 r = __hsub2(x, y);
  return *reinterpret_cast<uint32_t*>(&r);
}

__device__ __forceinline__ uint32_t hmul2_bits(uint32_t a, uint32_t b) {
  __half2 x = *reinterpret_cast<__half2*>(&a), y = *reinterpret_cast<__half2*>(&b);
  __half2 r = __hmul2(x, y);
  return *reinterpret_cast<uint32_t*>(&r);
}

__device__ __forceinline__ uint16_t hsub_bits(uint16_t a, uint16_t b) {
  __half r = __hsub(__ushort_as_half(a), __ushort_as_half(b));
  return __half_as_ushort(r);
}

__device__ __forceinline__ float h2f16(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// 32-lane xor butterfly inside each half of the wave.
__device__ __forceinline__ float warp32_sum(float v) {
  v = v + xor_lane_f<16>(v);
  v = v + xor_lane_f<8>(v);
  v = v + xor_lane_f<4>(v);
  v = v + xor_lane_f<2>(v);
  v = v + xor_lane_f<1>(v);
  return v;
}

__device__ __forceinline__ float readlane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// The reference 128-thread reduction, p0 = virtual thread lane, p1 =
// virtual thread lane + 64. Every lane receives the result (the four warp
// sums are read from lanes 0 and 32 without the LDS crossbar).
__device__ __forceinline__ float block128_sum(float p0, float p1) {
  p0 = warp32_sum(p0);
  p1 = warp32_sum(p1);
  const float w0 = readlane_f(p0, 0), w1 = readlane_f(p0, 32);
  const float w2 = readlane_f(p1, 0), w3 = readlane_f(p1, 32);
  return (w0 + w2) + (w1 + w3);
}

// Lane 0 of each row of 16 lanes receives the row's butterfly sum (xor 8,
// 4, 2, 1): lane l adds lane l + j by a DPP row shift, and since a + b and
// b + a are the same float, lane 0 holds exactly the butterfly's value. The
// other lanes hold partial sums.
template <int J>
__device__ __forceinline__ float row_shl_f(float v) {
  // lanes past the row's end read 0 (bound_ctrl), which lets the shift fold
  // into the add as one DPP instruction
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + J, 0xF, 0xF, true));
}

__device__ __forceinline__ float row_sum_first(float v) {
  v = v + row_shl_f<8>(v);
  v = v + row_shl_f<4>(v);
  v = v + row_shl_f<2>(v);
  v = v + row_shl_f<1>(v);
  return v;
}

// Lanes 0 and 32 receive the butterfly sums of lanes 0..31 and 32..63
// (warp32_sum's values there): rows 0 and 2 first add the row above them.
__device__ __forceinline__ float warp32_sum_first(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return row_sum_first(v + __uint_as_float(r[1]));
}

// block128_sum for the visit, by rows: with at most 16 virtual threads
// holding values the other three warp sums are +0.0 and the tree reduces to
// (row 0's sum + 0) + 0, which is row 0's sum + 0 (a sum tree whose leaves
// differ only in the signs of zeros gives the same value or a zero, and
// adding +0.0 makes either zero +0.0).
__device__ __forceinline__ float block128_sum_rows(float p0, float p1, uint32_t nthreads) {
  if (nthreads <= 16) return readlane_f(row_sum_first(p0), 0) + 0.0f;
  p0 = warp32_sum_first(p0);
  const float w0 = readlane_f(p0, 0), w1 = readlane_f(p0, 32);
  if (nthreads <= 64) return (w0 + 0.0f) + (w1 + 0.0f);
  p1 = warp32_sum_first(p1);
  const float w2 = readlane_f(p1, 0), w3 = readlane_f(p1, 32);
  return (w0 + w2) + (w1 + w3);
}

// Sums of an fp16 pair with one rounding, the halves read by v_fma_mix_f32.
// h2_sq_sum: f0^2 + f1^2 (each square of an fp16 value is exact in fp32, 22
// significant bits, so fma(f1, f1, f0 * f0) is the rounded sum of squares);
// h2_sum: f0 + f1 as fma(f0, 1, f1).
__device__ __forceinline__ float h2_sq_sum(uint32_t w) {
  const float f0 = h2f_lo(w), f1 = h2f_hi(w);
  return __builtin_fmaf(f1, f1, __builtin_fmaf(f0, f0, 0.0f));
}

__device__ __forceinline__ float h2_sum(uint32_t w) {
  float r;
  asm("v_fma_mix_f32 %0, %1, %2, %1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(w), "s"(1.0f));
  return r;
}

// Square root of a bf16 value through a 256-entry table in LDS: for sign 0
// and exponent field E in 1..254 the value is (1 + m / 128) * 2^e, e = E -
// 127, and its root is sqrt((1 + m / 128) * 2^p) * 2^((e - p) / 2) with p =
// e mod 2. tab[(p << 7) | m] holds the correctly rounded first factor (in
// [1, 2)), and the power of two scales it exactly (the result is normal).
// Index bit 7 is p = 1 - (E mod 2), i.e. bit 7 of the bf16 bits inverted.
// Zeros, subnormals, infinities, NaNs and negative values take sqrt_rn.
__device__ __forceinline__ float bf16_sqrt(const float* tab, uint32_t bits) {
  if (bits - 0x80u < 0x7F00u) {
    const int e = (int)((bits >> 7) & 0xFFu) - 127;
    return __builtin_ldexpf(tab[(bits & 0xFFu) ^ 0x80u], e >> 1);
  }
  return sqrt_rn(bf2f((uint16_t)bits));
}

__device__ __forceinline__ void fill_sqrt_table(float* tab, uint32_t lane) {
  for (uint32_t i = lane; i < 256; i += 64) {
    const uint32_t p = i >> 7, m = i & 127u;
    tab[i] = sqrt_rn(bf2f((uint16_t)(((127u + p) << 7) | m)));
  }
}

// splitmix64 counter sampler, identical to the oracle's
// (oracle/directional_oracle.cpp, sample_edge).
__host__ __device__ __forceinline__ uint64_t splitmix(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// pq_hash, pq_kernels.cuh:19-24
__host__ __device__ __forceinline__ uint64_t pq_hash(uint64_t x, uint64_t seed) {
  x += seed + 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Offset of subspace j's code for edge e inside a vertex's device code row
// (the edge-interleaved layout [G][R][W] of PqArtifacts).
__host__ __device__ __forceinline__ size_t pq_code_at(uint32_t j, uint32_t e, uint32_t R, uint32_t W) {
  return ((size_t)(j / W) * R + e) * W + (j % W);
}

// A random valid edge (u -> nb) for sample s, up to 8 attempts
// (lsh_globals.cuh:46-67, pq_kernels.cuh:77-93).
__device__ bool sample_edge(const uint32_t* edges, const uint8_t* counts, int64_t n, uint32_t R, uint64_t seed,
                            uint64_t s, uint32_t* u_out, uint32_t* nb_out) {
  uint64_t state = splitmix(seed ^ splitmix(s + 1));
  for (int attempt = 0; attempt < 8; ++attempt) {
    state = splitmix(state);
    const uint32_t r1 = (uint32_t)(state >> 32);
    state = splitmix(state);
    const uint32_t r2 = (uint32_t)(state >> 32);
    const uint32_t qlid = (uint32_t)((uint64_t)r1 % (uint64_t)n);
    const uint32_t cnt = counts[qlid];
    if (cnt == 0) continue;
    const uint32_t e = r2 % cnt;
    const uint32_t nb = edges[(size_t)qlid * R + e];
    if (nb == kInvalid32) continue;
    *u_out = qlid;
    *nb_out = nb;
    return true;
  }
  return false;
}

// ------------------------------------------------------------ LSH build --

// accumulate_rank_sums (lsh_globals.cuh:17-158): one wave per sample;
// per-sample contributions are written out and summed in sample order by
// lsh_finalize_kernel (the reference sums with float atomics).
__global__ __launch_bounds__(64) void lsh_calib_kernel(const uint16_t* __restrict__ vecs, int64_t n, uint32_t dp,
                                                       const uint32_t* __restrict__ edges,
                                                       const uint8_t* __restrict__ counts, uint32_t R, uint32_t K,
                                                       uint64_t seed, float* __restrict__ contrib,
                                                       uint8_t* __restrict__ valid) {
  extern __shared__ uint32_t keys[];
  const uint32_t lane = threadIdx.x;
  const uint64_t s = blockIdx.x;
  uint32_t u = 0, nb = 0;
  const bool ok = sample_edge(edges, counts, n, R, seed, s, &u, &nb);
  if (!ok) {
    if (lane == 0) valid[s] = 0;
    return;
  }
  const uint16_t* uv = vecs + (size_t)u * dp;
  const uint16_t* nv = vecs + (size_t)nb * dp;
  float p0 = 0.0f, p1 = 0.0f;
  for (uint32_t i = lane; i < dp; i += 128) {
    const uint16_t d = hsub_bits(nv[i], uv[i]);
    keys[i] = ((uint32_t)(d & 0x7FFFu) << 16) | ((uint32_t)(d >> 15) << 15) | (i & 0x7FFFu);
    const float f = h2f16(d);
    p0 = __builtin_fmaf(f, f, p0);
  }
  for (uint32_t i = lane + 64; i < dp; i += 128) {
    const uint16_t d = hsub_bits(nv[i], uv[i]);
    keys[i] = ((uint32_t)(d & 0x7FFFu) << 16) | ((uint32_t)(d >> 15) << 15) | (i & 0x7FFFu);
    const float f = h2f16(d);
    p1 = __builtin_fmaf(f, f, p1);
  }
  const float inv_norm = div_rn(1.0f, sqrt_rn(block128_sum(p0, p1) + 1e-20f));
  wave_sync();
  if (inv_norm > 1e9f) {
    if (lane == 0) valid[s] = 0;
    return;
  }
  for (uint32_t r = 0; r < K; ++r) {
    uint32_t m = 0;
    for (uint32_t i = lane; i < dp; i += 64) m = max(m, keys[i]);
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, d, 64));
    if (lane == 0) {
      contrib[s * K + r] = h2f16((uint16_t)(m >> 16)) * inv_norm;
      keys[m & 0x7FFFu] = 0;
    }
    wave_sync();
  }
  if (lane == 0) valid[s] = 1;
}

// finalize_lsh_globals (lsh_globals.cuh:160-178), sums in sample order:
// lane r < K of one wave keeps rank r's running sum, over tiles of 256
// samples staged in LDS (a sample's K values are contiguous, so the tile
// loads are coalesced).
__global__ __launch_bounds__(64) void lsh_finalize_kernel(const float* __restrict__ contrib,
                                                          const uint8_t* __restrict__ valid, int64_t n_samples,
                                                          uint32_t K, float* __restrict__ out /* K + 2 */) {
  constexpr uint32_t kTile = 256;
  __shared__ float tile[kTile * 16];
  __shared__ uint8_t ok[kTile];
  const uint32_t lane = threadIdx.x;
  float sum = 0.0f;
  int64_t nv = 0;
  const uint32_t rk = min(lane, K - 1u);  // lanes past K repeat rank K - 1's reads
  for (int64_t s0 = 0; s0 < n_samples; s0 += kTile) {
    const uint32_t ns = (uint32_t)min<int64_t>(kTile, n_samples - s0);
    wave_sync();
    for (uint32_t i = lane; i < ns * K; i += 64) tile[i] = contrib[s0 * K + i];
    for (uint32_t i = lane; i < ns; i += 64) ok[i] = valid[s0 + i];
    wave_sync();
    // 64 samples at a time: their validity as one mask, each add kept or
    // dropped by a select, so the reads do not wait on a branch
    for (uint32_t b = 0; b < ns; b += 64) {
      const uint64_t vm = ballot(b + lane < ns && ok[b + lane] != 0u);
      nv += __builtin_popcountll(vm);
      const uint32_t nb = min(ns - b, 64u);
      for (uint32_t j = 0; j < nb; j += 8) {
        // eight reads in flight (slots past the tile's samples are inside
        // the array and dropped by the mask), then the adds in order
        float x[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) x[u] = tile[(b + j + u) * K + rk];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
          const float y = sum + x[u];
          sum = ((vm >> (j + u)) & 1ull) ? y : sum;
        }
      }
    }
  }
  const float inv_n = div_rn(1.0f, (float)nv);
  const float c = sum * inv_n;
  if (lane < K) out[lane] = c;
  float denom = 0.0f;
  for (uint32_t r = 0; r < K; ++r) {
    const float cr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), (int)r));
    denom = __builtin_fmaf(cr, cr, denom);
  }
  if (lane == 0) {
    out[K] = denom;
    out[K + 1] = (float)nv;
  }
}

// populate_lsh (lsh/lsh_kernels.cuh:9-132): one wave per vertex, edges
// e < count (slots past the count stay zero). The row is staged in LDS and
// written out once.
__global__ __launch_bounds__(64) void lsh_populate_kernel(const uint16_t* __restrict__ vecs, int64_t n, uint32_t dp,
                                                          const uint32_t* __restrict__ edges,
                                                          const uint8_t* __restrict__ counts, uint32_t R, uint32_t K,
                                                          uint32_t pbytes, uint8_t* __restrict__ rows,
                                                          uint32_t row_bytes) {
  extern __shared__ uint32_t keys[];           // [dp] then the staged row
  uint8_t* stage = reinterpret_cast<uint8_t*>(keys + dp);
  const uint32_t lane = threadIdx.x;
  const uint32_t coord_bits = pbytes * 8 - 1;
  const uint32_t coord_mask = (1u << coord_bits) - 1u;
  const uint32_t word_mask = (1u << (coord_bits + 1)) - 1u;
  for (int64_t u = blockIdx.x; u < n; u += gridDim.x) {
    for (uint32_t b = lane; b < row_bytes; b += 64) stage[b] = 0;
    const uint16_t* uv = vecs + (size_t)u * dp;
    const uint32_t cnt = min((uint32_t)counts[u], R);
    for (uint32_t e = 0; e < cnt; ++e) {
      const uint32_t nb = edges[(size_t)u * R + e];
      const uint16_t* nv = vecs + (size_t)nb * dp;
      wave_sync();
      float p[2] = {0.0f, 0.0f};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        for (uint32_t i = lane + 64u * h; i < dp; i += 128) {
          const uint16_t d = hsub_bits(nv[i], uv[i]);
          keys[i] = ((uint32_t)(d & 0x7FFFu) << (coord_bits + 1)) | ((uint32_t)(d >> 15) << coord_bits) |
                    (i & coord_mask);
          const float f = h2f16(d);
          p[h] = __builtin_fmaf(f, f, p[h]);
        }
      }
      const float mag_sq = block128_sum(p[0], p[1]);
      wave_sync();
      for (uint32_t r = 0; r < K; ++r) {
        uint32_t m = 0;
        for (uint32_t i = lane; i < dp; i += 64) m = max(m, keys[i]);
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, d, 64));
        if (lane == 0) {
          const uint32_t word = m & word_mask;
          const size_t at = ((size_t)e * K + r) * pbytes;
          stage[at] = (uint8_t)word;
          if (pbytes == 2) stage[at + 1] = (uint8_t)(word >> 8);
          keys[m & coord_mask] = 0;
        }
        wave_sync();
      }
      if (lane == 0) {
        const uint16_t mb = f2bf(mag_sq);
        const size_t at = (size_t)R * K * pbytes + 2 * (size_t)e;
        stage[at] = (uint8_t)mb;
        stage[at + 1] = (uint8_t)(mb >> 8);
      }
    }
    wave_sync();
    uint8_t* row = rows + (size_t)u * row_bytes;
    for (uint32_t b = lane; b < row_bytes; b += 64) row[b] = stage[b];
    wave_sync();
  }
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ void cx_desc(uint32_t& a, uint32_t& b) {
  const uint32_t hi = max(a, b), lo = min(a, b);
  a = hi;
  b = lo;
}

// populate_lsh for rows of at most 128 coordinates and at most 64 edges
// (the same words and magnitudes as lsh_populate_kernel). Each row of 16
// lanes takes one edge, four edges per wave at a time; lane j holds
// coordinates 8j..8j+7 of the edge's difference vector.
//  - Keys: the key of coordinate i is (|d| bits, sign, i), unique for
//    nonzero keys. The K largest, in descending order, are the words the
//    repeated wave-max extracts. Each lane sorts its eight keys (a
//    19-comparator network), then each of the K rounds takes the row's
//    largest head by four DPP max steps (xor 1, xor 2 in the quad, half-row
//    and row mirrors), and the lane holding it shifts its list up. Lane r
//    keeps round r's word. A round whose largest head is 0 outputs word 0,
//    as the wave-max does when only zero keys remain.
//  - Magnitude: the 128-thread reduction of the squares, virtual thread t
//    holding coordinate t. Warp w's butterfly tree (strides 16, 8, 4, 2, 1
//    over its 32 coordinates) has lanes 4w..4w+3 of the row: stride 16 is
//    lane xor 2, stride 8 lane xor 1, and strides 4, 2, 1 stay inside the
//    lane. Lane 0 then forms (W0 + W2) + (W1 + W3) by row shifts of 8 and
//    4.
//  - Edges past the vertex's count (and slots of a partial group) take
//    zero keys and squares, which give the zero words and magnitude that
//    the row holds there.
__global__ __launch_bounds__(256) void lsh_populate_rows_kernel(const uint16_t* __restrict__ vecs, int64_t n,
                                                                uint32_t dp, const uint32_t* __restrict__ edges,
                                                                const uint8_t* __restrict__ counts, uint32_t R,
                                                                uint32_t K, uint32_t pbytes,
                                                                uint8_t* __restrict__ rows, uint32_t row_bytes) {
  const uint32_t lane = threadIdx.x & 63u, j = lane & 15u, g = lane >> 4;
  const uint32_t coord_bits = pbytes * 8 - 1;
  const uint32_t word_mask = (1u << (coord_bits + 1)) - 1u;
  const bool has = 8u * j < dp;
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x >> 6);
  for (int64_t u = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); u < n; u += waves) {
    const uint32_t cnt = min((uint32_t)counts[u], R);
    const uint32_t my_edge = lane < cnt ? edges[(size_t)u * R + lane] : 0u;
    uint4 uw = make_uint4(0, 0, 0, 0);
    if (has) uw = *reinterpret_cast<const uint4*>(vecs + (size_t)u * dp + 8u * j);
    uint8_t* row = rows + (size_t)u * row_bytes;
    for (uint32_t e0 = 0; e0 < R; e0 += 4) {
      const uint32_t e = e0 + g;
      const uint32_t nb = (uint32_t)__shfl((int)my_edge, (int)min(e, 63u), 64);
      uint32_t word = 0;
      float mag = 0.0f;
      if (e0 < cnt) {
        uint4 nw = make_uint4(0, 0, 0, 0);
        if (has && e < cnt) nw = *reinterpret_cast<const uint4*>(vecs + (size_t)nb * dp + 8u * j);
        const uint32_t dw[4] = {hsub2_bits(nw.x, uw.x), hsub2_bits(nw.y, uw.y), hsub2_bits(nw.z, uw.z),
                                hsub2_bits(nw.w, uw.w)};
        uint32_t k[8];
        float x[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          const uint32_t d = (m & 1) ? dw[m >> 1] >> 16 : dw[m >> 1] & 0xFFFFu;
          const uint32_t i = 8u * j + (uint32_t)m;
          k[m] = has && e < cnt ? ((d & 0x7FFFu) << (coord_bits + 1)) | ((d >> 15) << coord_bits) | i : 0u;
          const float f = h2f16((uint16_t)d);
          x[m] = has && e < cnt ? __builtin_fmaf(f, f, 0.0f) : 0.0f;
        }
        // the squares' tree: strides 16 and 8 across the quad, 4, 2, 1 in the lane
#pragma unroll
        for (int m = 0; m < 8; ++m) x[m] = x[m] + dpp_f<0x4E>(x[m]);
#pragma unroll
        for (int m = 0; m < 8; ++m) x[m] = x[m] + dpp_f<0xB1>(x[m]);
        const float w = ((x[0] + x[4]) + (x[2] + x[6])) + ((x[1] + x[5]) + (x[3] + x[7]));
        const float s = w + row_shl_f<8>(w);
        mag = s + row_shl_f<4>(s);
        cx_desc(k[0], k[2]); cx_desc(k[1], k[3]); cx_desc(k[4], k[6]); cx_desc(k[5], k[7]);
        cx_desc(k[0], k[4]); cx_desc(k[1], k[5]); cx_desc(k[2], k[6]); cx_desc(k[3], k[7]);
        cx_desc(k[0], k[1]); cx_desc(k[2], k[3]); cx_desc(k[4], k[5]); cx_desc(k[6], k[7]);
        cx_desc(k[2], k[4]); cx_desc(k[3], k[5]);
        cx_desc(k[1], k[4]); cx_desc(k[3], k[6]);
        cx_desc(k[1], k[2]); cx_desc(k[3], k[4]); cx_desc(k[5], k[6]);
        for (uint32_t r = 0; r < K; ++r) {
          uint32_t m = k[0];
          m = max(m, dpp_u32<0xB1>(m));
          m = max(m, dpp_u32<0x4E>(m));
          m = max(m, dpp_u32<0x141>(m));
          m = max(m, dpp_u32<0x140>(m));
          if (j == r) word = m & word_mask;
          if (k[0] == m) {
#pragma unroll
            for (int q = 0; q < 7; ++q) k[q] = k[q + 1];
            k[7] = 0;
          }
        }
      }
      if (e < R) {
        if (j < K) {
          const size_t at = ((size_t)e * K + j) * pbytes;
          if (pbytes == 2)
            *reinterpret_cast<uint16_t*>(row + at) = (uint16_t)word;
          else
            row[at] = (uint8_t)word;
        }
        if (j == 0) *reinterpret_cast<uint16_t*>(row + (size_t)R * K * pbytes + 2 * (size_t)e) = f2bf(mag);
      }
    }
  }
}

// ------------------------------------------------------------- PQ build --

// pq_sample_residuals (pq_kernels.cuh:64-106): residual nb - u (fp16) of a
// sampled edge per training row, zeros when no edge was found.
__global__ void pq_sample_kernel(const uint16_t* __restrict__ vecs, int64_t n, uint32_t dp,
                                 const uint32_t* __restrict__ edges, const uint8_t* __restrict__ counts, uint32_t R,
                                 int64_t n_train, uint64_t seed, uint16_t* __restrict__ X) {
  const int64_t p = blockIdx.x;
  if (p >= n_train) return;
  __shared__ uint32_t s_u, s_nb, s_ok;
  if (threadIdx.x == 0) {
    uint32_t u = 0, nb = 0;
    s_ok = sample_edge(edges, counts, n, R, seed, (uint64_t)p, &u, &nb) ? 1u : 0u;
    s_u = u;
    s_nb = nb;
  }
  __syncthreads();
  uint16_t* row = X + (size_t)p * dp;
  for (uint32_t i = threadIdx.x; i < dp; i += blockDim.x)
    row[i] = s_ok ? hsub_bits(vecs[(size_t)s_nb * dp + i], vecs[(size_t)s_u * dp + i]) : (uint16_t)0;
}

// pq_kmeans_init (pq_kernels.cuh:110-125)
__global__ void pq_init_kernel(const uint16_t* __restrict__ X, int64_t n_train, uint32_t dp, uint32_t M, uint32_t dsub,
                               uint64_t init_seed, float* __restrict__ C) {
  const uint32_t jc = blockIdx.x;
  const uint32_t j = jc / 256;
  const uint64_t r = pq_hash(jc, init_seed) % (uint64_t)n_train;
  for (uint32_t t = threadIdx.x; t < dsub; t += blockDim.x)
    C[(size_t)jc * dsub + t] = h2f16(X[(size_t)r * dp + (size_t)j * dsub + t]);
}

// pq_kmeans_assign (pq_kernels.cuh:127-160): nearest centroid per
// (point, subspace), sequential fma distance, ties -> smaller index.
__global__ void pq_assign_kernel(const uint16_t* __restrict__ X, int64_t n_train, uint32_t dp, uint32_t M,
                                 uint32_t dsub, const float* __restrict__ C, uint8_t* __restrict__ labels,
                                 bool stage) {
  extern __shared__ float sc_lds[];  // [256 * dsub] centroids of subspace j when staged
  const uint32_t j = blockIdx.y;
  const float* sc = C + (size_t)j * 256 * dsub;
  if (stage) {
    for (uint32_t i = threadIdx.x; i < 256 * dsub; i += blockDim.x) sc_lds[i] = sc[i];
    __syncthreads();
    sc = sc_lds;
  }
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= n_train) return;
  const uint16_t* x = X + (size_t)p * dp + (size_t)j * dsub;
  float best = FLT_MAX;
  uint32_t bi = 0;
  for (uint32_t c = 0; c < 256; ++c) {
    const float* cc = sc + (size_t)c * dsub;
    float d = 0.0f;
    for (uint32_t t = 0; t < dsub; ++t) {
      const float df = h2f16(x[t]) - cc[t];
      d = __builtin_fmaf(df, df, d);
    }
    if (d < best) { best = d; bi = c; }
  }
  labels[(size_t)p * M + j] = (uint8_t)bi;
}

// pq_kmeans_accumulate + pq_kmeans_finalize (pq_kernels.cuh:162-211): one
// thread per (subspace, centroid, coordinate); sums in sample order; empty
// clusters reseeded from a pq_hash pick.
__global__ void pq_update_kernel(const uint16_t* __restrict__ X, int64_t n_train, uint32_t dp, uint32_t M,
                                 uint32_t dsub, const uint8_t* __restrict__ labels, uint64_t init_seed, uint32_t iter,
                                 float* __restrict__ C) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= (int64_t)M * 256 * dsub) return;
  const uint32_t jc = (uint32_t)(tid / dsub), t = (uint32_t)(tid % dsub);
  const uint32_t j = jc / 256, c = jc % 256;
  float s = 0.0f;
  uint32_t cnt = 0;
  for (int64_t p = 0; p < n_train; ++p) {
    if (labels[(size_t)p * M + j] == c) {
      ++cnt;
      s = s + h2f16(X[(size_t)p * dp + (size_t)j * dsub + t]);
    }
  }
  if (cnt > 0) {
    C[(size_t)jc * dsub + t] = s * div_rn(1.0f, (float)cnt);
  } else {
    const uint64_t r = pq_hash((uint64_t)jc ^ ((uint64_t)iter * 0x9E3779B9u), init_seed) % (uint64_t)n_train;
    C[(size_t)jc * dsub + t] = h2f16(X[(size_t)r * dp + (size_t)j * dsub + t]);
  }
}

// pq_populate (pq_kernels.cuh:249-295): one wave per vertex; for each edge
// the fp16 residual goes to LDS and each lane scores centroids c = lane + 64m
// (argmin, ties to the smaller index). Codes are staged in LDS.
__global__ __launch_bounds__(64) void pq_encode_kernel(const uint16_t* __restrict__ vecs, int64_t n, uint32_t dp,
                                                       const uint32_t* __restrict__ edges,
                                                       const uint8_t* __restrict__ counts, uint32_t R, uint32_t M,
                                                       uint32_t dsub, const float* __restrict__ C,
                                                       uint8_t* __restrict__ codes) {
  extern __shared__ float res[];  // [dp] then the vertex's staged code row
  uint8_t* stage = reinterpret_cast<uint8_t*>(res + dp);
  const uint32_t lane = threadIdx.x;
  const uint32_t W = pq_group_width(M);
  const uint32_t row_bytes = (uint32_t)pq_row_bytes(M, R);
  for (int64_t u = blockIdx.x; u < n; u += gridDim.x) {
    for (uint32_t b = lane; b < row_bytes; b += 64) stage[b] = 0;
    const uint32_t cnt = min((uint32_t)counts[u], R);
    for (uint32_t e = 0; e < cnt; ++e) {
      const uint32_t nb = edges[(size_t)u * R + e];
      wave_sync();
      for (uint32_t i = lane; i < dp; i += 64)
        res[i] = h2f16(hsub_bits(vecs[(size_t)nb * dp + i], vecs[(size_t)u * dp + i]));
      wave_sync();
      for (uint32_t j = 0; j < M; ++j) {
        float best = FLT_MAX;
        uint32_t bi = 0;
        const float* rj = res + (size_t)j * dsub;
        for (uint32_t c = lane; c < 256; c += 64) {
          const float* cc = C + ((size_t)j * 256 + c) * dsub;
          float d = 0.0f;
          for (uint32_t t = 0; t < dsub; ++t) {
            const float df = rj[t] - cc[t];
            d = __builtin_fmaf(df, df, d);
          }
          if (d < best) { best = d; bi = c; }
        }
#pragma unroll
        for (int dd = 32; dd > 0; dd >>= 1) {
          const float ob = __shfl_xor(best, dd, 64);
          const uint32_t oi = (uint32_t)__shfl_xor((int)bi, dd, 64);
          if (ob < best || (ob == best && oi < bi)) { best = ob; bi = oi; }
        }
        if (lane == 0) stage[pq_code_at(j, e, R, W)] = (uint8_t)bi;
      }
    }
    wave_sync();
    uint8_t* code = codes + (size_t)u * row_bytes;
    for (uint32_t b = lane; b < row_bytes; b += 64) code[b] = stage[b];
    wave_sync();
  }
}

// The same codes with the work turned around for subspaces of at most 64
// dims: a 256-thread block holds the 256 centroids of one subspace j in LDS
// (rows padded with zeros to DS floats), each wave takes one vertex at a
// time and each lane one edge, with its residual slice in registers; the
// centroids are read as wave-wide LDS broadcasts. Per centroid the distance
// is the same ordered fma sum (padding adds exact zeros) and the argmin
// keeps the first minimum, as a scan over c = 0..255 does.
template <int DS>
__global__ __launch_bounds__(256) void pq_encode_lds_kernel(const uint16_t* __restrict__ vecs, int64_t n,
                                                            uint32_t dp, const uint32_t* __restrict__ edges,
                                                            const uint8_t* __restrict__ counts, uint32_t R,
                                                            uint32_t M, uint32_t dsub, const float* __restrict__ C,
                                                            uint8_t* __restrict__ codes) {
  __shared__ float4 sc4[256 * DS / 4];
  float* sc = reinterpret_cast<float*>(sc4);
  const uint32_t j = blockIdx.y;
  const float* cj = C + (size_t)j * 256 * dsub;
  for (uint32_t i = threadIdx.x; i < 256u * DS; i += 256) {
    const uint32_t c = i / DS, t = i % DS;
    sc[i] = t < dsub ? cj[(size_t)c * dsub + t] : 0.0f;
  }
  __syncthreads();
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t W = pq_group_width(M);
  const size_t row_bytes = pq_row_bytes(M, R);
  for (int64_t u = (int64_t)blockIdx.x * 4 + wave; u < n; u += (int64_t)gridDim.x * 4) {
    const uint32_t cnt = min((uint32_t)counts[u], R);
    const bool act = lane < cnt;
    const uint32_t nb = act ? edges[(size_t)u * R + lane] : (uint32_t)u;
    const uint16_t* vrow = vecs + (size_t)nb * dp + (size_t)j * dsub;
    const uint16_t* urow = vecs + (size_t)u * dp + (size_t)j * dsub;
    float r[DS];
#pragma unroll
    for (int t = 0; t < DS; ++t) r[t] = (uint32_t)t < dsub ? h2f16(hsub_bits(vrow[t], urow[t])) : 0.0f;
    float best = FLT_MAX;
    uint32_t bi = 0;
    for (uint32_t c = 0; c < 256; ++c) {
      const float4* cc = sc4 + c * (DS / 4);
      float d = 0.0f;
#pragma unroll
      for (int q = 0; q < DS / 4; ++q) {
        const float4 w = cc[q];
        const float wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float df = r[4 * q + k] - wv[k];
          d = __builtin_fmaf(df, df, d);
        }
      }
      if (d < best) {
        best = d;
        bi = c;
      }
    }
    if (lane < R) codes[(size_t)u * row_bytes + pq_code_at(j, lane, R, W)] = act ? (uint8_t)bi : (uint8_t)0;
  }
}

// pq_compute_vector_norms (pq_kernels.cuh:218-247)
__global__ __launch_bounds__(64) void norms_kernel(const uint16_t* __restrict__ vecs, int64_t n, uint32_t dp,
                                                   float* __restrict__ out) {
  const uint32_t lane = threadIdx.x;
  for (int64_t u = blockIdx.x; u < n; u += gridDim.x) {
    const uint16_t* x = vecs + (size_t)u * dp;
    float p0 = 0.0f, p1 = 0.0f;
    for (uint32_t i = lane; i < dp; i += 128) {
      const float v = h2f16(x[i]);
      p0 = __builtin_fmaf(v, v, p0);
    }
    for (uint32_t i = lane + 64; i < dp; i += 128) {
      const float v = h2f16(x[i]);
      p1 = __builtin_fmaf(v, v, p1);
    }
    const float s = block128_sum(p0, p1);
    if (lane == 0) out[u] = s;
  }
}

// Codes between the device layout and the file's subspace-major rows
// [M][R] for vertices [u0, u0 + count): one thread per (vertex, edge).
// to_file: dev -> file; otherwise file -> dev (the padding bytes of dev's
// last group must already be zero).
__global__ void pq_layout_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t count,
                                 uint32_t R, uint32_t M, bool to_file) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= count * R) return;
  const int64_t u = t / R;
  const uint32_t e = (uint32_t)(t % R), W = pq_group_width(M);
  const size_t dev_row = pq_row_bytes(M, R), file_row = (size_t)M * R;
  for (uint32_t j = 0; j < M; ++j) {
    const size_t di = (size_t)u * dev_row + pq_code_at(j, e, R, W), fi = (size_t)u * file_row + (size_t)j * R + e;
    if (to_file) dst[fi] = src[di];
    else dst[di] = src[fi];
  }
}

// ---------------------------------------------------- directional search --

// LUT entries [e_begin, e_end) of one query (pq_build_lut: entry e =
// <q_j, C_e> with j = e / 256, pq_beam_search.cuh:32-60): one 32-lane half
// per entry, lanes stride dsub with an fma chain, then the 32-lane
// butterfly sum. At dsub <= 64 a lane holds at most two elements (hl,
// hl + 32) and the centroid values of kLutBatch entry pairs are loaded
// together before their products; each entry keeps the same chain.
__device__ __forceinline__ void pq_lut_range(const uint16_t* q16, const float* centroids, uint32_t dsub,
                                             uint32_t e_begin, uint32_t e_end, float* lut) {
  const uint32_t lane = lane_id();
  const uint32_t half = lane >> 5, hl = lane & 31u;
  if (dsub <= 64) {
    constexpr uint32_t kLutBatch = 8;
    const bool v0 = hl < dsub, v1 = hl + 32u < dsub;
    for (uint32_t e0 = e_begin; e0 < e_end; e0 += 2 * kLutBatch) {
      float c0[kLutBatch], c1[kLutBatch];
#pragma unroll
      for (uint32_t u = 0; u < kLutBatch; ++u) {
        const uint32_t e = e0 + 2u * u + half;
        const float* C = centroids + (size_t)(e < e_end ? e : e_begin) * dsub;
        c0[u] = (e < e_end && v0) ? C[hl] : 0.0f;
        c1[u] = (e < e_end && v1) ? C[hl + 32u] : 0.0f;
      }
#pragma unroll
      for (uint32_t u = 0; u < kLutBatch; ++u) {
        const uint32_t e = e0 + 2u * u + half;
        const uint16_t* qj = q16 + (size_t)(min(e, e_end - 1u) / 256u) * dsub;
        float acc = 0.0f;
        if (e < e_end && v0) acc = __builtin_fmaf(h2f16(qj[hl]), c0[u], acc);
        if (e < e_end && v1) acc = __builtin_fmaf(h2f16(qj[hl + 32u]), c1[u], acc);
        acc = warp32_sum(acc);
        if (hl == 0 && e < e_end) lut[e] = acc;
      }
    }
  } else {
    for (uint32_t e0 = e_begin; e0 < e_end; e0 += 2) {
      const uint32_t e = e0 + half;
      float acc = 0.0f;
      if (e < e_end) {
        const float* C = centroids + (size_t)e * dsub;
        const uint16_t* qj = q16 + (size_t)(e / 256u) * dsub;
        for (uint32_t t = hl; t < dsub; t += 32) acc = __builtin_fmaf(h2f16(qj[t]), C[t], acc);
      }
      acc = warp32_sum(acc);
      if (hl == 0 && e < e_end) lut[e] = acc;
    }
  }
}

// Rows of 256 entries per query in the tables the search reads: M rows,
// then rows of -0.0f up to a multiple of 4 (the search adds the last
// group of subspaces 4 rows at a time; x + (-0.0f) == x for every x under
// round to nearest).
__host__ __device__ constexpr uint32_t pq_lut_rows(uint32_t m) { return (m + 3u) / 4u * 4u; }

// Every query's LUT [nq, pq_lut_rows(M) * 256] in one launch,
// kLutWaveEntries entries per wave, so the whole GPU builds them instead of
// one wave per query.
constexpr uint32_t kLutWaveEntries = 64;
__global__ __launch_bounds__(64) void pq_lut_kernel(const uint16_t* __restrict__ queries, uint32_t dp, uint32_t M,
                                                    uint32_t dsub, const float* __restrict__ centroids,
                                                    float* __restrict__ lut) {
  const uint32_t total = M * 256, stride = pq_lut_rows(M) * 256;
  const uint32_t e_begin = blockIdx.y * kLutWaveEntries;
  float* out = lut + (size_t)blockIdx.x * stride;
  if (e_begin >= total) {  // a pad row
    for (uint32_t e = e_begin + threadIdx.x; e < min(stride, e_begin + kLutWaveEntries); e += 64) out[e] = -0.0f;
    return;
  }
  const uint32_t e_end = min(total, e_begin + kLutWaveEntries);
  pq_lut_range(queries + (size_t)blockIdx.x * dp, centroids, dsub, e_begin, e_end, out);
}

// dsub <= 32: one table entry per thread. Block (b, j) holds the 256
// centroids of subspace j in registers, one per thread, and builds their
// entries for queries b * kLutQueries ... (the queries' slices are the same
// address across the block, so they are broadcast reads); each query's 256
// entries are one coalesced 1 KB store. In the 32-lane form above, lane t
// holds the leaf v_t = fma(q_t, C_t, +0.0) for t < dsub and +0.0 beyond, and
// the butterfly leaves the writing lane with the tree v_l + v_(l+16), then
// + the partner 8 lanes away, 4, 2, 1. The thread sums its own leaves in
// that tree. Leaves past DS are left out, which is exact: no leaf is -0.0
// (fma(a, b, +0.0) of a zero product is +0.0) and x + 0.0 == x for every
// other x.
constexpr uint32_t kLutQueries = 32;
template <int DS>
__global__ __launch_bounds__(256) void pq_lut_small_kernel(const uint16_t* __restrict__ queries, int64_t nq,
                                                           uint32_t dp, uint32_t M, uint32_t dsub,
                                                           const float* __restrict__ centroids,
                                                           float* __restrict__ lut) {
  const uint32_t j = blockIdx.y;
  const uint32_t e = j * 256 + threadIdx.x;
  const size_t stride = (size_t)pq_lut_rows(M) * 256;
  const int64_t q0 = (int64_t)blockIdx.x * kLutQueries;
  const int64_t q1 = min(nq, q0 + (int64_t)kLutQueries);
  if (j >= M) {  // a pad row
    for (int64_t qi = q0; qi < q1; ++qi) lut[(size_t)qi * stride + e] = -0.0f;
    return;
  }
  const float* C = centroids + (size_t)e * dsub;
  float c[DS];
#pragma unroll
  for (int t = 0; t < DS; ++t) c[t] = (uint32_t)t < dsub ? C[t] : 0.0f;
  for (int64_t qi = q0; qi < q1; ++qi) {
    const uint16_t* qj = queries + (size_t)qi * dp + (size_t)j * dsub;
    float v[DS];
#pragma unroll
    for (int t = 0; t < DS; ++t) v[t] = (uint32_t)t < dsub ? __builtin_fmaf(h2f16(qj[t]), c[t], 0.0f) : 0.0f;
#pragma unroll
    for (int h = 16; h >= 1; h >>= 1) {
#pragma unroll
      for (int t = 0; t < h; ++t)
        if (t + h < DS) v[t] = v[t] + v[t + h];
    }
    lut[(size_t)qi * stride + e] = v[0];
  }
}

struct DirArgs {
  const uint16_t* vecs;
  int64_t n;
  uint32_t dp, R;
  const uint32_t* edges;
  const uint8_t* counts;
  const uint32_t* deleted;
  const uint16_t* queries;  // [nq, dp]
  uint32_t medoid, k, bw, limit, max_result;
  int32_t* out_ids;
  float* out_dists;
  // LSH
  uint32_t K, pbytes;
  const uint8_t* lsh_rows;
  uint32_t row_bytes;
  float c[16];
  float inv_norm_denom;
  // 1: the bf16 square-root table sits in LDS; 0: each root is computed
  uint32_t sqrt_lds;
  // PQ
  uint32_t M, dsub;
  const float* centroids;
  const uint8_t* codes;  // edge-interleaved rows of code_row_bytes
  uint32_t code_row_bytes, pq_w, pq_groups;
  const float* norms;
  const float* luts;  // [nq, pq_lut_rows(M) * 256] from pq_lut_kernel
  // RaBitQ
  const uint8_t* rq_nodes;     // [n, rq_node_bytes]: code dwords, f_add, f_rescale
  const float* rq_centroid;    // [rq_dim]
  uint32_t rq_node_bytes, rq_words, rq_dim;
  // optional work counters per query: {visits, hops expanded, adjacency entries}
  uint32_t* stats;
  // build mode (RaBitQ only): queries are the graph's rows [q_start,
  // q_start + nq); each visit is scored with the plain search's distance and
  // recorded as a key in visited[qid * max_result + i], with the count in
  // visited_counts[qid]
  uint64_t* visited;
  uint32_t* visited_counts;
  uint32_t q_start;
  // skip pops of ids already in the frontier (distinct results; an extension)
  uint32_t unique;
};

// One thread's share of the visit for one chunk of 8 fp16 values, summed
// in order from 0 (L2 also stores the fp16 differences to *d).
template <bool L2>
__device__ __forceinline__ float chunk_sum(uint4 q, uint4 u, uint4* d, float local) {
  const uint32_t qw[4] = {q.x, q.y, q.z, q.w}, uw[4] = {u.x, u.y, u.z, u.w};
  uint32_t dw[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (L2) {
      dw[j] = hsub2_bits(qw[j], uw[j]);
      local = local + h2_sq_sum(dw[j]);
    } else {
      local = local + h2_sum(hmul2_bits(qw[j], uw[j]));
    }
  }
  if constexpr (L2) *d = make_uint4(dw[0], dw[1], dw[2], dw[3]);
  return local;
}

// Exact distance of the popped node (compute_qu_diff_and_exact,
// beam_search_common.cuh:87-154). L2: fp16 q - u, stored to diff, sum of
// f0^2 + f1^2 per half2; IP: sum of fp16 products per half2.
// qreg: the query's chunks lane and lane + 64 in registers, used when the
// row has at most 128 chunks (longer rows read qrow).
// ureg: u's chunks lane and lane + 64, loaded by the caller, when the row
// has at most 128 chunks.
// kMaxChunks: a bound on nchunks known to the caller at compile time.
template <bool L2, uint32_t kMaxChunks>
__device__ __forceinline__ float visit_exact(const uint4* qrow, const uint4 (&qreg)[2], const uint4* urow,
                                             const uint4 (&ureg)[2], uint32_t nchunks, uint4* diff) {
  const uint32_t lane = lane_id();
  float p[2] = {0.0f, 0.0f};
  if (kMaxChunks <= 16) {
    if (lane < nchunks) p[0] = chunk_sum<L2>(qreg[0], ureg[0], diff + lane, 0.0f);
    return readlane_f(row_sum_first(p[0]), 0) + 0.0f;  // block128_sum_rows with nthreads <= 16
  }
  if (nchunks <= 128) {
    // at most one chunk per virtual thread: lane and lane + 64
    if (lane < nchunks) p[0] = chunk_sum<L2>(qreg[0], ureg[0], diff + lane, 0.0f);
    if (kMaxChunks > 64 && nchunks > 64 && lane + 64u < nchunks)
      p[1] = chunk_sum<L2>(qreg[1], ureg[1], diff + lane + 64u, 0.0f);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float local = 0.0f;
      for (uint32_t i = lane + 64u * h; i < nchunks; i += 128) local = chunk_sum<L2>(qrow[i], urow[i], diff + i, local);
      p[h] = local;
    }
  }
  return block128_sum_rows(p[0], p[1], nchunks);
}

// The build mode's L2 visit for rows of at most C chunks (RaBitQ graphs:
// ceil(dim / 8) chunks, at most 4 per code dword): the lane's chunks ql,
// ql + 4, ... of u's row are loaded together, then summed in that order,
// the chain stream_partial_l2 forms.
template <uint32_t C>
__device__ __forceinline__ float visit_partial_l2(const uint4* q, const uint4* row, uint32_t ql, uint32_t nchunks) {
  uint4 xb[C / 4];
#pragma unroll
  for (uint32_t u = 0; u < C / 4; ++u) {
    const uint32_t c = ql + 4u * u;
    xb[u] = c < nchunks ? row[c] : make_uint4(0u, 0u, 0u, 0u);
  }
  float acc = 0.0f;
#pragma unroll
  for (uint32_t u = 0; u < C / 4; ++u) {
    const uint32_t c = ql + 4u * u;
    if (c < nchunks) l2_chunk(q[c], xb[u], acc);
  }
  return acc;
}

// One LSH word (sign in the MSB, coordinate below) of rank r from the
// edge's K * P bytes held in registers.
template <int P>
__device__ __forceinline__ uint32_t lsh_word(const uint32_t* w, int r) {
  if constexpr (P == 1) return (w[r >> 2] >> (8 * (r & 3))) & 0xFFu;
  else return (w[r >> 1] >> (16 * (r & 1))) & 0xFFFFu;
}

// Largest number of new keys a hop merges by counting (larger ones take
// the binary searches).
constexpr uint32_t kCountMerge = 16;
// Largest number of 64-entry rows the general merge moves with marks in LDS
// (more rows take masks built in scalar registers).
constexpr uint32_t kMarkRows = 8;

// 8-byte words of the merge's position marks (one bit per slot of the
// candidate buffer, rounded to 128 slots so that what follows stays 16-byte
// aligned).
__host__ __device__ __forceinline__ uint32_t dir_mark_words(uint32_t cap) { return ((cap + 127u) & ~127u) / 64u; }

// PQ table layouts in LDS (the last argument of directional_kernel): the
// whole table; the first 4 groups of 16 subspaces and the last, partly
// filled group, with the other groups' entries gathered from the table in
// global memory; the first 4 groups, the rest gathered. The split layouts
// (P = 8, more than 64 subspaces) let two queries' waves share a CU.
constexpr int kLutWhole = 0, kLutSplitLast = 1, kLutSplit = 2;

// K = 0: the PQ estimator, with up to 16 * P subspaces (the edge's codes are
// P groups of 16 bytes in registers); K = 1: the RaBitQ estimator with codes
// of up to 32 * P dims; K in {4, 16} with P-byte words: the LSH estimator.
template <int METRIC, int K, int P, int LUT = kLutWhole>
__global__ __launch_bounds__(64) void directional_kernel(DirArgs a) {
  extern __shared__ uint64_t smem[];
  constexpr bool L2 = METRIC == kL2;
  constexpr bool PQ = K == 0;
  constexpr bool RQ = K == 1;
  constexpr int KW = (PQ || RQ) ? 1 : K * P / 4;  // dwords of LSH words per edge
  const uint32_t lane = threadIdx.x;
  const uint32_t qid = blockIdx.x;
  const uint32_t nchunks = a.dp / 8;
  const uint32_t cap = a.bw + a.R;
  // PQ: the query's table at the start of LDS, so that a table row's offset
  // is a constant of the read instruction; the search state after it
  // (rows: the whole padded table, or 64 and, with kLutSplitLast, the last
  // group's)
  const uint32_t lut_tail_rows = LUT == kLutSplitLast ? pq_lut_rows(a.M & 15u) : 0u;
  const uint32_t lut_words = PQ ? ((LUT == kLutWhole ? pq_lut_rows(a.M) : 64u) + lut_tail_rows) * 128u : 0u;
  uint64_t* sm = smem + lut_words;
  uint64_t* buf0 = sm;
  uint64_t* T = buf0 + cap;
  float* Fd = reinterpret_cast<float*>(T + 64);  // frontier distances (exact bits)
  uint32_t* Fi = reinterpret_cast<uint32_t*>(Fd + a.k);
  // marks of the new keys' positions in the general merge (bit o of the
  // array set = position o holds a new key)
  uint32_t* MK = reinterpret_cast<uint32_t*>(sm + ((cap + 64 + a.k + 1) & ~1u));
  // LSH with 1-byte words (dp <= 128): q and q - u take 16 chunks each,
  // zero past dp, so any 7-bit coordinate reads inside them
  constexpr bool LSH8 = !PQ && !RQ && P == 1;
  // split PQ layouts: groups 4 .. 7 may be gathered
  constexpr int kGlobGroups = (PQ && P == 8 && LUT != kLutWhole) ? 4 : 0;
  static_assert(LUT == kLutWhole || (PQ && P == 8), "split tables need 8 groups");
  const uint32_t qchunks = LSH8 ? 16u : nchunks;
  uint4* qv = reinterpret_cast<uint4*>(sm + ((cap + 64 + a.k + 1) & ~1u) + dir_mark_words(cap));  // 16-byte aligned
  for (uint32_t i = lane; i < dir_mark_words(cap) * 2u; i += 64) MK[i] = 0u;
  uint4* xv = qv + qchunks;  // L2 LSH: fp16 q - u
  // PQ: the query's LUT; LSH: the bf16 sqrt table
  float* lut = PQ ? reinterpret_cast<float*>(smem) : reinterpret_cast<float*>(xv + qchunks);

  const uint4* qsrc = a.visited ? reinterpret_cast<const uint4*>(a.vecs) + (size_t)(a.q_start + qid) * nchunks
                               : reinterpret_cast<const uint4*>(a.queries) + (size_t)qid * nchunks;
  for (uint32_t i = lane; i < nchunks; i += 64) qv[i] = qsrc[i];
  if constexpr (LSH8) {
    for (uint32_t i = nchunks + lane; i < 16u; i += 64) {
      qv[i] = make_uint4(0u, 0u, 0u, 0u);
      xv[i] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  if constexpr (!PQ && !RQ) {
    if (a.sqrt_lds) fill_sqrt_table(lut, lane);
  }
  uint4 qreg[2];
  qreg[0] = lane < nchunks ? qsrc[lane] : make_uint4(0u, 0u, 0u, 0u);
  qreg[1] = lane + 64u < nchunks ? qsrc[lane + 64u] : make_uint4(0u, 0u, 0u, 0u);
  lds_wave_sync();
  const uint16_t* q16 = reinterpret_cast<const uint16_t*>(qv);

  float q_sq = 0.0f;
  if constexpr (PQ) {
    // the query's LUT, built by pq_lut_kernel, into LDS: every row, pad
    // rows included, or the first 64 rows, then the last group's rows with
    // kLutSplitLast
    const float4* src = reinterpret_cast<const float4*>(a.luts + (size_t)qid * pq_lut_rows(a.M) * 256);
    float4* dst = reinterpret_cast<float4*>(lut);
    const uint32_t head4 = lut_words / 2u - lut_tail_rows * 64u;  // 16-byte chunks: rows * 64
    for (uint32_t i = lane; i < head4; i += 64) dst[i] = src[i];
    const uint32_t tail4 = lut_tail_rows * 64u, from4 = (a.M >> 4) * 16u * 64u;
    for (uint32_t i = lane; i < tail4; i += 64) dst[head4 + i] = src[from4 + i];
    if constexpr (L2) {
      float p0 = 0.0f, p1 = 0.0f;
      for (uint32_t i = lane; i < a.dp; i += 128) {
        const float v = h2f16(q16[i]);
        p0 = __builtin_fmaf(v, v, p0);
      }
      for (uint32_t i = lane + 64; i < a.dp; i += 128) {
        const float v = h2f16(q16[i]);
        p1 = __builtin_fmaf(v, v, p1);
      }
      q_sq = block128_sum(p0, p1);
    }
    lds_wave_sync();
  }

  // RaBitQ query factors (the estimator of directional_oracle.cpp,
  // rq_prepare): the query quantized to 4 bits over its first rq_dim values,
  // as bit planes (uniform: plane j, dword w at rq_planes[j * P + w]), the
  // sum of the 4-bit values, delta / 2, lo / 2 and g_add
  uint32_t rq_planes[RQ ? 4 * P : 1];
  int32_t rq_sumq = 0;
  float rq_hd = 0.0f, rq_hl = 0.0f, rq_gadd = 0.0f;
  if constexpr (RQ) {
    float lo = FLT_MAX, hi = -FLT_MAX;
    for (uint32_t i = lane; i < a.rq_dim; i += 64) {
      const float v = h2f16(q16[i]);
      lo = fminf(lo, v);
      hi = fmaxf(hi, v);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      lo = fminf(lo, __shfl_xor(lo, m, 64));
      hi = fmaxf(hi, __shfl_xor(hi, m, 64));
    }
    lo = lo + 0.0f;  // one zero for -0.0 and +0.0
    hi = hi + 0.0f;
    const float delta = div_rn(hi - lo, 15.0f);
    int32_t sq = 0;
    float g = 0.0f;
#pragma unroll
    for (int m = 0; m < P / 2; ++m) {
      const uint32_t i = 64u * m + lane;
      uint32_t qb = 0;
      if (i < a.rq_dim) {
        const float qi = h2f16(q16[i]), ci = a.rq_centroid[i];
        if (delta > 0.0f) {
          const float t = rintf(div_rn(qi - lo, delta));
          qb = (uint32_t)fminf(15.0f, fmaxf(0.0f, t));
        }
        if constexpr (L2) {
          const float d = qi - ci;
          g = __builtin_fmaf(d, d, g);
        } else {
          g = __builtin_fmaf(qi, ci, g);
        }
      }
      sq += (int32_t)qb;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint64_t bits = ballot(((qb >> j) & 1u) != 0u);
        rq_planes[j * P + 2 * m] = (uint32_t)bits;
        rq_planes[j * P + 2 * m + 1] = (uint32_t)(bits >> 32);
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      sq += __shfl_xor(sq, m, 64);
      g = g + __shfl_xor(g, m, 64);
    }
    rq_sumq = sq;
    rq_hd = 0.5f * delta;
    rq_hl = 0.5f * lo;
    rq_gadd = L2 ? g : -1.0f - g;
  }

  // B = [(medoid, est 0.0, unvisited)], F empty (graph_beam_search.cuh:141-149)
  uint64_t* B = buf0;
  if (lane == 0) B[0] = make_key(0.0f, a.medoid);
  uint32_t cnt = 1, fc = 0, vc = 0, loop = 0, n_hops = 0, n_adj = 0;
  float fdr = FLT_MAX;     // F's distances and ids in registers when k <= 64
  uint32_t fir = kInv31;
  uint32_t hint = 0;  // every entry of B before `hint` is visited
  // degree of the predicted next pop (the next unvisited entry of B after
  // the pop), read one hop ahead: when the pop matches, the adjacency and
  // estimator rows are read only up to the degree
  uint32_t spec_u = kInvalid32, spec_c = 0;
  lds_wave_sync();
  while (loop <= a.limit) {
    loop += 1;
    int p = -1;
    uint64_t pk = 0;
    uint32_t next_u = kInvalid32;
    for (uint32_t base = hint; base < cnt; base += 64) {
      const uint32_t i = base + lane;
      const uint64_t bv = i < cnt ? B[i] : 1ull;
      const uint64_t m = ballot(!key_visited(bv));
      if (m) {
        const int l = __builtin_ctzll(m);
        p = (int)base + l;
        pk = readlane64(bv, l);
        const uint64_t m2 = m & (m - 1u);
        if (m2) next_u = key_id(readlane64(bv, __builtin_ctzll(m2)));
        break;
      }
    }
    next_u = uniform(next_u);
    if (p < 0) break;
    lds_wave_sync();
    if (lane == 0) B[p] = pk | 1ull;
    hint = (uint32_t)p + 1u;
    const uint32_t u = uniform(key_id(pk));
    if (a.unique) {
      // u already in F: its exact distance and its neighbours' estimates are
      // those of its first visit, so the hop would only duplicate F entries
      bool in_f = false;
      if (a.k <= 64) {
        in_f = ballot(lane < fc && fir == u) != 0;
      } else {
        for (uint32_t base = 0; base < fc && !in_f; base += 64) {
          const uint32_t i = base + lane;
          in_f = ballot(i < fc && Fi[i] == u) != 0;
        }
      }
      if (in_f) {
        lds_wave_sync();
        continue;
      }
    }
    // every read that depends only on u, issued before the visit: the edge
    // count, the adjacency row, and u's estimator data for edge slot `lane`
    // (slots past the count are read and ignored; they lie inside u's rows)
    // u's row first (rows of at most 128 chunks): the visit's arithmetic
    // then overlaps the gathers below
    const uint4* urow = reinterpret_cast<const uint4*>(a.vecs) + (size_t)u * nchunks;
    // Loads below are issued by every lane, at clamped indexes, so that the
    // wait for the visited row does not also wait for later loads; lanes
    // past the row or the degree ignore what they read.
    // a compile-time bound on the row's chunks: 1-byte LSH words address at
    // most 128 dims, RaBitQ codes at most 256
    constexpr uint32_t kMaxChunks = LSH8 ? 16u : RQ ? 32u : 0xFFFFFFFFu;
    const bool short_row = nchunks <= 128 && !(RQ && a.visited);
    uint4 ureg[2] = {make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
    // adjacency slot `lane` (slots past R read slot R - 1 and are never used:
    // only lanes below the degree are); with the degree read ahead, slots
    // past it read the last live one, so only the lines the degree covers
    // are fetched
    const bool known = u == spec_u;
    const uint32_t el = known ? min(lane, max(min(spec_c, a.R), 1u) - 1u) : min(lane, a.R - 1u);
    const uint32_t deg_raw = known ? spec_c : (uint32_t)a.counts[u];
    spec_u = next_u;
    spec_c = next_u != kInvalid32 ? (uint32_t)a.counts[next_u] : 0u;
    const uint32_t* erow = a.edges + (size_t)u * a.R;
    const uint32_t v_raw = erow[el];
    uint32_t wl[KW];
    uint32_t mag_bits = 0;
    uint4 cw[PQ ? P : 1];  // PQ: codes of subspaces 16g .. 16g + 15 in cw[g]
    if constexpr (RQ) {
      // nothing of u's row: the estimator reads the neighbours' codes below
    } else if constexpr (!PQ) {
      const uint8_t* row = a.lsh_rows + (size_t)u * a.row_bytes;
      if constexpr (KW == 1) wl[0] = reinterpret_cast<const uint32_t*>(row)[el];
      else if constexpr (KW == 2) {
        const uint2 t2 = reinterpret_cast<const uint2*>(row)[el];
        wl[0] = t2.x; wl[1] = t2.y;
      } else {
#pragma unroll
        for (int c = 0; c < KW / 4; ++c) {
          const uint4 t4 = reinterpret_cast<const uint4*>(row)[el * (KW / 4) + c];
          wl[4 * c] = t4.x; wl[4 * c + 1] = t4.y; wl[4 * c + 2] = t4.z; wl[4 * c + 3] = t4.w;
        }
      }
      mag_bits = reinterpret_cast<const uint16_t*>(row + (size_t)a.R * (K * P))[el];
    } else {
      const uint8_t* crow = a.codes + (size_t)u * a.code_row_bytes + (size_t)el * a.pq_w;
#pragma unroll
      for (int g = 0; g < (PQ ? P : 1); ++g) {
        cw[g] = make_uint4(0u, 0u, 0u, 0u);
        if ((uint32_t)g < a.pq_groups) {
          const uint8_t* cp = crow + (size_t)g * a.R * a.pq_w;
          if (P > 1 || a.pq_w == 16) {  // more than one group: M > 16, groups of 16
            cw[g] = *reinterpret_cast<const uint4*>(cp);
          } else if (a.pq_w == 8) {
            const uint2 t2 = *reinterpret_cast<const uint2*>(cp);
            cw[g].x = t2.x;
            cw[g].y = t2.y;
          } else {
            cw[g].x = *reinterpret_cast<const uint32_t*>(cp);
          }
        }
      }
    }
    if (short_row) ureg[0] = urow[min(lane, nchunks - 1u)];
    if (kMaxChunks > 64 && short_row && nchunks > 64) ureg[1] = urow[min(lane + 64u, nchunks - 1u)];
    // the degree and edge validity: before the visit where gathers depend
    // on them (PQ norms, RaBitQ codes), after it for LSH
    uint32_t deg = 0;
    bool has = false, valid_v = false;
    if constexpr (PQ || RQ) {
      deg = uniform(min(deg_raw, a.R));
      has = lane < deg;
      valid_v = has && (int64_t)v_raw < a.n;
    }
    float vnorm = 0.0f;
    if constexpr (PQ && L2) vnorm = valid_v ? a.norms[v_raw] : 0.0f;
    // PQ: the table's group counts, re-read every hop so that the compiler
    // tests them where they are used rather than holding every test's
    // result in scalar registers across the loop. pq_q4: the last group's
    // 4-row chunks (the rows past M hold -0.0f)
    uint32_t pq_full = a.M >> 4, pq_q4 = ((a.M & 15u) + 3u) >> 2;
    if constexpr (PQ) asm volatile("" : "+s"(pq_full), "+s"(pq_q4));
    // split layouts, groups 4 .. 7: their entries from the query's LUT in
    // global memory (the last group's, with kLutSplit, in 4-row chunks),
    // issued here so that the gathers overlap the visit; group g lands in
    // gv[(g - 4) * 16 + i]
    float gv[kGlobGroups > 0 ? kGlobGroups * 16 : 1];
    if constexpr (kGlobGroups > 0) {
      if (valid_v) {
        const float* gl = a.luts + (size_t)qid * pq_lut_rows(a.M) * 256;
#pragma unroll
        for (int h = 0; h < kGlobGroups; ++h) {
          const int g = P - kGlobGroups + h;
          {
            const uint32_t w4[4] = {cw[g].x, cw[g].y, cw[g].z, cw[g].w};
            // rows 4c .. 4c + 3: byte offset of entry (16g + 4c + j, code),
            // below 512 KB, kept opaque so the load adds it to the table's
            // base as a 32-bit offset
            const auto gather = [&](int c) {
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                uint32_t off = (((uint32_t)g * 16u + 4u * c + j) << 10) + (((w4[c] >> (8 * j)) & 0xFFu) << 2);
                asm volatile("" : "+v"(off));
                gv[h * 16 + 4 * c + j] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(gl) + off);
              }
            };
            // 4 chunks in a full group, pq_q4 in the last
            if ((uint32_t)g < pq_full) {
#pragma unroll
              for (int c = 0; c < 4; ++c) gather(c);
            } else if (LUT == kLutSplit && (uint32_t)g == pq_full) {
#pragma unroll
              for (int c = 0; c < 4; ++c)
                if ((uint32_t)c < pq_q4) gather(c);
            }
          }
        }
      }
    }
    // RaBitQ: the neighbour's code dwords and factors (a gather per edge,
    // issued before the visit so the two overlap)
    uint32_t rq_code[RQ ? P : 1];
    float rq_fadd = 0.0f, rq_fres = 0.0f;
    if constexpr (RQ) {
      const uint32_t* node = reinterpret_cast<const uint32_t*>(a.rq_nodes + (size_t)(valid_v ? v_raw : 0u) *
                                                                                 a.rq_node_bytes);
#pragma unroll
      for (int w = 0; w < P; ++w) rq_code[w] = (valid_v && (uint32_t)w < a.rq_words) ? node[w] : 0u;
      if (valid_v) {
        rq_fadd = __uint_as_float(node[a.rq_words]);
        rq_fres = __uint_as_float(node[a.rq_words + 1]);
      }
    }

    // visit: exact distance of u (the one vector fetch per hop)
    float exact_u = 0.0f, qu_dot = 0.0f, stored;
    if constexpr (PQ) {
      qu_dot = visit_exact<false, kMaxChunks>(qv, qreg, urow, ureg, nchunks, nullptr);
      stored = L2 ? (q_sq - 2.0f * qu_dot) + a.norms[u] : -qu_dot;
    } else if (RQ && a.visited) {
      // build mode: the plain search's distance (distance.cuh's 4-lane
      // order), so visits carry the values the plain build search records
      const float part = L2 ? visit_partial_l2<4u * P>(qv, urow, lane & 3u, nchunks)
                            : stream_partial_ip(qv, urow, lane & 3u, nchunks, a.dp);
      stored = __shfl(quad_finish<METRIC>(part), 0, 64);
      if (lane == 0) a.visited[(size_t)qid * a.max_result + vc] = make_key(stored, u);
    } else {
      exact_u = visit_exact<L2, kMaxChunks>(qv, qreg, urow, ureg, nchunks, xv);
      stored = L2 ? exact_u : -exact_u;
    }
    // frontier_insert_sorted (beam_search_common.cuh:156-185): the new entry
    // goes after the last entry that is not greater (its insertion loop runs
    // from the end while F[j - 1] > stored); when F is full it enters only
    // below the last entry, which drops out
    if (a.k > 0) {
      if (a.k <= 64) {
        // F in registers (lane i holds entry i): entries pos .. lim - 1 move
        // up one lane (DPP wave shift), the new one lands at pos
        const bool full = fc == a.k;
        const uint32_t lim = full ? a.k - 1 : fc;
        const bool enter = !full || stored < readlane_f(fdr, (int)(a.k - 1));
        if (enter) {
          const uint64_t le = ballot(lane < lim && !(fdr > stored));
          const uint32_t pos = le ? 64u - (uint32_t)__builtin_clzll(le) : 0u;
          const float sd = __int_as_float(
              __builtin_amdgcn_update_dpp(__float_as_int(fdr), __float_as_int(fdr), 0x138, 0xF, 0xF, false));
          const uint32_t si = (uint32_t)__builtin_amdgcn_update_dpp((int)fir, (int)fir, 0x138, 0xF, 0xF, false);
          if (lane > pos && lane <= lim) {
            fdr = sd;
            fir = si;
          }
          if (lane == pos) {
            fdr = stored;
            fir = u;
          }
          if (!full) fc += 1;
        }
      } else if (lane == 0) {
        int j = -1;
        if (fc < a.k) {
          j = (int)fc;
          fc += 1;
        } else if (stored < Fd[a.k - 1]) {
          j = (int)a.k - 1;
        }
        if (j >= 0) {
          while (j > 0 && Fd[j - 1] > stored) {
            Fd[j] = Fd[j - 1];
            Fi[j] = Fi[j - 1];
            --j;
          }
          Fd[j] = stored;
          Fi[j] = u;
        }
      }
      if (a.k > 64) fc = (uint32_t)__shfl((int)fc, 0, 64);
      fc = uniform(fc);
    }
    if constexpr (!PQ && !RQ) {
      deg = uniform(min(deg_raw, a.R));
      has = lane < deg;
      valid_v = has && (int64_t)v_raw < a.n;
    }
    vc += 1;
    if (vc == a.max_result) break;
    lds_wave_sync();

    // estimate u's neighbours from the data read above (no neighbour vector fetches)
    n_hops += 1;
    n_adj += deg;
    // every lane takes the gathered words here, on every path, so no load of
    // this hop is still in flight when the next hop reuses its registers
    if constexpr (!PQ && !RQ) {
#pragma unroll
      for (int c = 0; c < KW; ++c) asm volatile("" ::"v"(wl[c]));
      asm volatile("" ::"v"(mag_bits));
    }
    asm volatile("" ::"v"(v_raw));
    uint64_t t = kEmptyKey;
    if (has) {
      if (valid_v) {
        float est;
        if constexpr (RQ) {
          // one count per bit plane (v_bcnt accumulates), weighted once
          int32_t dj[4] = {0, 0, 0, 0}, pc = 0;
#pragma unroll
          for (int w = 0; w < P; ++w) {
            const uint32_t c = rq_code[w];
            pc += __builtin_popcount(c);
#pragma unroll
            for (int j = 0; j < 4; ++j) dj[j] += __builtin_popcount(c & rq_planes[j * P + w]);
          }
          const int32_t dot = dj[0] + 2 * dj[1] + 4 * dj[2] + 8 * dj[3];
          const float t1 = (float)(2 * dot - rq_sumq), t2 = (float)(2 * pc - (int32_t)a.rq_dim);
          const float ipq = __builtin_fmaf(rq_hd, t1, rq_hl * t2);
          est = __builtin_fmaf(rq_fres, ipq, rq_fadd + rq_gadd);
        } else if constexpr (PQ) {
          // acc = <q,u> + sum over j = 0, 1, ..., M - 1 of LUT[j][code_j], in
          // that order (pq_beam_search.cuh:97-100): the full groups of 16
          // subspaces, then the last group's subspaces, each group from LDS
          // or from the gathers as the layout places it
          float acc = qu_dot;
#pragma unroll
          for (int g = 0; g < (PQ ? P : 1); ++g) {
            const uint32_t w4[4] = {cw[g].x, cw[g].y, cw[g].z, cw[g].w};
            const bool past_lds = kGlobGroups > 0 && g >= P - kGlobGroups;
            // a group past the first 4, but the last group with kLutSplitLast,
            // comes from the gathers
            const bool from_global = past_lds && (LUT == kLutSplit || (uint32_t)g < pq_full);
            // with kLutSplitLast the last group's rows follow the first 64
            const float* lg = lut + (past_lds ? 64u : (uint32_t)g * 16u) * 256u;
            // rows 4c .. 4c + 3 of the group
            const auto add4 = [&](int c) {
              if (from_global) {
                const int h = kGlobGroups > 0 ? g - (P - kGlobGroups) : 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) acc = acc + gv[h * 16 + 4 * c + j];
              } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) acc = acc + lg[(4 * c + j) * 256 + ((w4[c] >> (8 * j)) & 0xFFu)];
              }
            };
            // 4 chunks in a full group, pq_q4 in the last
            if ((uint32_t)g < pq_full) {
#pragma unroll
              for (int c = 0; c < 4; ++c) add4(c);
            } else if ((uint32_t)g == pq_full) {
#pragma unroll
              for (int c = 0; c < 4; ++c)
                if ((uint32_t)c < pq_q4) add4(c);
            }
          }
          est = L2 ? (q_sq - 2.0f * acc) + vnorm : -acc;
        } else {
          const uint16_t* x16 = L2 ? reinterpret_cast<const uint16_t*>(xv) : q16;
          constexpr uint32_t kSign = P == 1 ? 0x80u : 0x8000u;
          float dot_acc = 0.0f;
#pragma unroll
          for (int r = 0; r < K; ++r) {
            const uint32_t w = lsh_word<P>(wl, r);
            const uint32_t coord = w & (kSign - 1u);
            // -c_r when the sign bit is set: the bit moved to the float's sign
            const float cs = __uint_as_float(__float_as_uint(a.c[r]) ^ ((w & kSign) << (P == 1 ? 24 : 16)));
            // 1-byte words: coord < 128 and x16 is zero past dp; 2-byte
            // words: the bound guards a corrupt row
            const float xc = (P == 1 || coord < a.dp) ? h2f16(x16[coord]) : 0.0f;
            dot_acc = __builtin_fmaf(cs, xc, dot_acc);
          }
          const float mag_sq = bf2f((uint16_t)mag_bits);
          const float dot_est = dot_acc * a.inv_norm_denom;
          const float mag = a.sqrt_lds ? bf16_sqrt(lut, mag_bits) : sqrt_rn(bf2f((uint16_t)mag_bits));
          est = L2 ? __builtin_fmaf(-(2.0f * mag), dot_est, exact_u + mag_sq)
                   : -__builtin_fmaf(mag, dot_est, exact_u);
        }
        t = make_key(est, v_raw);
      } else {
        t = make_key(FLT_MAX, kInv31) | 1ull;  // INVALID, visited (device_kernels.cuh:115-122)
      }
    }
    // merge_sort_tail: sort the tail, merge with the head (head first on
    // ties), drop entries whose id equals the previous one, clip to bw.
    // Once B is full, a key ranked at or above B's last entry cannot enter:
    // the merged order puts B's bw entries before it, and each of those the
    // dedup drops heads no run of equal ids (B holds no two adjacent equal
    // ids, so a run holds at most one member of B) -- the run is headed by a
    // kept new key that also precedes it. Only keys ranked below B's last
    // are merged (nt of them); a hop that keeps none leaves B as it is.
    const uint64_t thr = cnt == a.bw ? key_rank(B[a.bw - 1u]) : ~0ull;
    const bool kt = lane < deg && key_rank(t) < thr;
    const uint64_t km = ballot(kt);
    const uint32_t nt = (uint32_t)__builtin_popcountll(km);
    if (nt == 0) {
      lds_wave_sync();
      continue;
    }
    if (kt) T[mbcnt(km)] = t;
    lds_wave_sync();
    t = lane < nt ? T[lane] : kEmptyKey;
    t = wave_sort_upto(t, nt);
    if (lane < nt) T[lane] = t;
    lds_wave_sync();
    // Merge by rank: new key t_i (sorted, lane i) lands at lo_i + i, where
    // lo_i = the number of head entries ranked <= t_i (head first on ties),
    // and head entry j moves to j + #{i : lo_i <= j}. Positions below the
    // smallest key's insertion point lo0 keep their entries; the merge and
    // the dedup start there.
    uint32_t lo0;
    uint32_t lo_v = 0;       // lane i < nt holds lo_i
    if (nt <= kCountMerge && cnt <= 128) {
      // few new keys and a head of at most two rows: the head is held in
      // registers, so the merge writes B in place. Key i is counted against
      // the head with ballots: g0 / g1 mark the head entries ranked after
      // it, lo_i = the rest, and each marked entry moves up one slot (the
      // head is sorted, so lo_i <= j exactly when entry j is marked).
      const uint64_t h0 = lane < cnt ? B[lane] : ~0ull;
      const uint64_t h1 = lane + 64u < cnt ? B[lane + 64u] : ~0ull;
      uint32_t s0 = 0, s1 = 0;
      // rank(h) <= rank(t) <=> h <= t | 1
      if ((uint32_t)__builtin_amdgcn_readfirstlane(cnt) > 64u) {
        for (uint32_t i = 0; i < nt; ++i) {
          const uint64_t ti = readlane64(t, (int)i) | 1ull;
          const bool g0 = h0 > ti, g1 = h1 > ti;
          s0 += g0 ? 1u : 0u;
          s1 += g1 ? 1u : 0u;
          lo_v = writelane(lo_v, 128u - (uint32_t)__builtin_popcountll(ballot(g0)) -
                                     (uint32_t)__builtin_popcountll(ballot(g1)), i);
        }
      } else {
        for (uint32_t i = 0; i < nt; ++i) {
          const uint64_t ti = readlane64(t, (int)i) | 1ull;
          const bool g0 = h0 > ti;
          s0 += g0 ? 1u : 0u;
          lo_v = writelane(lo_v, 64u - (uint32_t)__builtin_popcountll(ballot(g0)), i);
        }
      }
      lo0 = (uint32_t)__builtin_amdgcn_readlane((int)lo_v, 0);
      if (lane < nt) B[lane + lo_v] = t;
      if (lane >= lo0 && lane < cnt) B[lane + s0] = h0;
      if (lane + 64u >= lo0 && lane + 64u < cnt) B[lane + 64u + s1] = h1;
    } else {
      // wider heads or more keys: each key finds lo_i by a binary search,
      // and its position is lo_i + i; every other position o >= lo0 takes
      // head entry o - (new keys below o), counted per 64-entry row from a
      // mask of the row's new positions. The rows run from the top down, so
      // each reads only entries not yet overwritten (a source lies at most
      // nt <= 64 slots below its position), and the keys are written last,
      // into B itself.
      const uint32_t top = pow2_ceil(cnt);
      uint32_t lo = 0;
      if (lane < nt) {
        // upper bound: head entries with rank <= rank(t) precede t
        for (uint32_t step = top; step > 0; step >>= 1) {
          const uint32_t probe = lo + step;
          if (probe <= cnt && key_rank(B[probe - 1]) <= key_rank(t)) lo = probe;
        }
      }
      lo0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)lo);
      lo_v = lo;
      const uint32_t tot = cnt + nt;
      const uint32_t rows = (tot - lo0 + 63u) / 64u;
      uint32_t above = 0;  // new keys at positions past the current row
      if (rows <= kMarkRows) {
        // a few rows: the masks come from marks in LDS, one bit per slot
        if (lane < nt) atomicOr(&MK[(lane + lo) >> 5], 1u << ((lane + lo) & 31u));
        lds_wave_sync();
        for (uint32_t r = rows; r-- > 0;) {
          const uint32_t o = lo0 + 64u * r + lane;
          const bool valid = o < tot;
          const bool isnew = valid && ((MK[o >> 5] >> (o & 31u)) & 1u) != 0u;
          const uint64_t m = ballot(isnew);
          if (valid && !isnew) {
            const uint32_t below = nt - above - (uint32_t)__builtin_popcountll(m >> lane);
            const uint64_t v = B[o - below];
            B[o] = v;
          }
          above = uniform(above + (uint32_t)__builtin_popcountll(m));
        }
        if (lane < nt) MK[(lane + lo) >> 5] = 0u;  // every set bit is a new key's
      } else {
        // many rows (a wide head): each row's mask is folded in scalar
        // registers from the keys whose positions fall in it (a run of
        // lanes, the keys being sorted), which takes an LDS round trip off
        // every row
        const uint32_t pos_v = lane < nt ? lo + lane : 0xFFFFFFFFu;  // key `lane`'s position
        for (uint32_t r = rows; r-- > 0;) {
          const uint32_t o0 = lo0 + 64u * r, o = o0 + lane;
          uint64_t in_row = ballot(pos_v >= o0 && pos_v < o0 + 64u);
          uint64_t m = 0;  // bit l: position o0 + l holds a new key
          while (in_row) {
            const int i = __builtin_ctzll(in_row);
            in_row &= in_row - 1u;
            m |= 1ull << ((uint32_t)__builtin_amdgcn_readlane((int)pos_v, i) - o0);
          }
          if (o < tot && ((m >> lane) & 1ull) == 0u) {
            const uint32_t below = nt - above - (uint32_t)__builtin_popcountll(m >> lane);
            const uint64_t v = B[o - below];
            B[o] = v;
          }
          above = uniform(above + (uint32_t)__builtin_popcountll(m));
        }
      }
      if (lane < nt) B[lane + lo] = t;
    }
    lds_wave_sync();
    const uint32_t total = cnt + nt;
    // Dedup: drop each entry whose id equals the previous entry's. Merging
    // never makes two head entries adjacent that were not, and B holds no
    // adjacent equal ids, so an entry can only be dropped at a new key or
    // right after one. The merge checks those two places and is done when
    // neither drops anything (the usual case).
    bool dedup;
    {
      bool d = false;
      if (lane < nt) {
        const uint32_t pos = lane + lo_v, id = key_id(t);
        const uint32_t prev_id = pos == 0 ? kInv31 : key_id(B[pos - 1u]);
        d = prev_id == id || (pos + 1u < total && key_id(B[pos + 1u]) == id);
      }
      dedup = ballot(d) != 0;
    }
    uint32_t kept = total;
    if (dedup) {
      // in order from lo0, reading the merged entries in B itself: each row
      // is read before any of its slots is written, and writes only go to
      // slots at or below the ones read
      const uint64_t* src = B;
      // the previous entry's id: the lane below (DPP wave shift), or for
      // lane 0 the last id of the previous row (the head's entry below lo0
      // at first)
      uint32_t carry = lo0 == 0 ? kInv31 : key_id(B[lo0 - 1u]);
      kept = lo0;
      for (uint32_t base = lo0; base < total; base += 64) {
        const uint32_t m = base + lane;
        const uint64_t cur = m < total ? src[m] : 0ull;
        const uint32_t cid = key_id(cur);
        const uint32_t prev_id = (uint32_t)__builtin_amdgcn_update_dpp((int)carry, (int)cid, 0x138, 0xF, 0xF, false);
        const bool keep = m < total && cid != prev_id;
        const uint64_t kmask = ballot(keep);
        const uint32_t pos = kept + mbcnt(kmask);
        if (keep && pos < a.bw) B[pos] = cur;
        kept += (uint32_t)__builtin_popcountll(kmask);
        carry = (uint32_t)__builtin_amdgcn_readlane((int)cid, 63);
      }
    }
    cnt = uniform(min(kept, a.bw));
    hint = uniform(min(hint, lo0));
    lds_wave_sync();
  }

  if (a.visited_counts && lane == 0) a.visited_counts[qid] = vc;
  if (a.stats && lane == 0) {
    a.stats[(size_t)qid * 3] = vc;
    a.stats[(size_t)qid * 3 + 1] = n_hops;
    a.stats[(size_t)qid * 3 + 2] = n_adj;
  }
  // output: F in order, skipping invalid / deleted, pad (0x7FFFFFFF, FLT_MAX)
  // (graph_beam_search.cuh:246-266)
  lds_wave_sync();
  uint32_t out = 0;
  for (uint32_t base = 0; base < fc && out < a.k; base += 64) {
    const uint32_t i = base + lane;
    bool ok = i < fc;
    float dist = 0.0f;
    uint32_t id = 0;
    if (ok) {
      dist = a.k <= 64 ? fdr : Fd[i];
      id = a.k <= 64 ? fir : Fi[i];
      ok = (int64_t)id < a.n && ((a.deleted[id >> 5] >> (id & 31u)) & 1u) == 0u;
    }
    const uint64_t m = ballot(ok);
    const uint32_t pos = out + mbcnt(m);
    if (ok && pos < a.k) {
      a.out_ids[(size_t)qid * a.k + pos] = (int32_t)id;
      a.out_dists[(size_t)qid * a.k + pos] = dist;
    }
    out += (uint32_t)__builtin_popcountll(m);
  }
  for (uint32_t i = out + lane; i < a.k; i += 64) {
    a.out_ids[(size_t)qid * a.k + i] = (int32_t)kInv31;
    a.out_dists[(size_t)qid * a.k + i] = FLT_MAX;
  }
}

// ------------------------------------------------------------ host side --

std::unique_ptr<Graph> construct_directional(uint32_t R, int metric, uint32_t k_ranks, bool small_dim,
                                             const void* vectors, int64_t n, int64_t dim, double alpha,
                                             int64_t budget, bool on_host, bool prerotate, uint64_t seed,
                                             hipStream_t stream, BuildStats* stats, uint32_t options) {
  if (n <= 0) throw std::invalid_argument("vectors must contain at least one row");
  if (n > 0x7FFFFFFF) throw std::invalid_argument("too many vectors for 31-bit ids");
  auto g = std::make_unique<Graph>();
  g->allocate(n, (uint32_t)dim, R, metric, on_host);
  g->k_ranks = k_ranks;
  g->packed_bytes = small_dim ? 1 : 2;
  upload_vectors(*g, vectors, n, (uint32_t)dim, stream);
  g->prerotate = prerotate;
  g->prerotate_seed = seed;
  if (prerotate) {
    // The reference rotates the caller's buffer in place (E.4,
    // construct.cuh:1104-1107); here the graph's own copy is rotated.
    g->rotation = make_rotation(rotation_matrix((uint32_t)dim, seed), (uint32_t)dim);
    void* tmp = nullptr;
    hip_check(hipMalloc(&tmp, (size_t)n * g->dp * 2), "alloc rotation output");
    rotate_rows(*g->rotation, g->vecs, n, g->dp, tmp, g->dp, stream);
    hip_check(hipMemcpyAsync(g->vecs, tmp, (size_t)n * g->dp * 2, hipMemcpyDeviceToDevice, stream), "copy rotated");
    scan_int_range(*g, 0, n, stream);  // synchronises the stream
    (void)hipFree(tmp);
  }
  const int64_t mbs = reference_max_batch(n, R, budget);
  const char* timing = std::getenv("JASPER_BUILD_TIMING");
  const bool time_stages = timing && timing[0] == '1';
  BuildStats local;
  BuildStats* st = stats ? stats : &local;
  const bool rq_search = (options & kBuildRabitqSearch) != 0;
  if (rq_search) build_rabitq(*g);  // codes of the stored (prerotated) rows, before any edge exists
  build_graph(*g, (float)alpha, mbs, stream, time_stages, st, rq_search);
  if (time_stages) {
    std::fprintf(stderr, "[construct] n=%lld batches=%lld max_batch=%lld search=%.1fms prune=%.1fms group=%.1fms "
                "reverse=%.1fms total=%.1fms\n",
                (long long)n, (long long)st->batches, (long long)st->max_batch, st->search_ms, st->prune_ms,
                st->sort_ms, st->reverse_ms, st->total_ms);
    std::fflush(stderr);
  }
  g->next_id = (uint64_t)n;
  return g;
}

void build_lsh(Graph& g, int64_t n_samples, uint64_t seed) {
  if (g.n <= 0) throw std::runtime_error("generate_lsh_globals: graph is empty");
  const uint32_t K = g.k_ranks, P = g.packed_bytes;
  if (K == 0 || K > 16) throw std::invalid_argument("k_ranks must be in 1..16");
  if (n_samples <= 0 || n_samples > 0xFFFFFFFFll) throw std::invalid_argument("n_samples must be in 1..2^32-1");
  if (P == 1 && g.dp > 128) throw std::invalid_argument("dim too large for 7-bit LSH coordinates");
  hipStream_t s = nullptr;
  float* contrib = nullptr;
  uint8_t* valid = nullptr;
  float* out = nullptr;
  hip_check(hipMalloc(&contrib, (size_t)std::max<int64_t>(n_samples, 1) * K * 4), "alloc lsh contrib");
  hip_check(hipMalloc(&valid, (size_t)std::max<int64_t>(n_samples, 1)), "alloc lsh valid");
  hip_check(hipMalloc(&out, (K + 2) * 4), "alloc lsh globals");
  auto art = std::make_unique<LshArtifacts>();
  art->k_ranks = K;
  art->packed_bytes = P;
  art->row_bytes = (size_t)g.R * K * P + 2 * (size_t)g.R;
  try {
    const size_t plds = (size_t)g.dp * 4 + ((art->row_bytes + 3) & ~(size_t)3);
    if (plds > 160 * 1024) throw std::invalid_argument("dim too large for the LSH kernels");
    if (plds > 64 * 1024) {
      hip_check(hipFuncSetAttribute((const void*)lsh_calib_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)plds), "LDS size");
      hip_check(hipFuncSetAttribute((const void*)lsh_populate_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)plds), "LDS size");
    }
    if (n_samples > 0)
      hipLaunchKernelGGL(lsh_calib_kernel, dim3((uint32_t)n_samples), dim3(64), g.dp * 4, s, (const uint16_t*)g.vecs,
                         g.n, g.dp, g.edges, g.counts, g.R, K, seed, contrib, valid);
    hip_check(hipGetLastError(), "launch lsh_calib_kernel");
    hipLaunchKernelGGL(lsh_finalize_kernel, dim3(1), dim3(64), 0, s, contrib, valid, n_samples, K, out);
    hip_check(hipGetLastError(), "launch lsh_finalize_kernel");
    std::vector<float> h(K + 2);
    hip_check(hipMemcpy(h.data(), out, (K + 2) * 4, hipMemcpyDeviceToHost), "download lsh globals");
    art->c_per_rank.assign(h.begin(), h.begin() + K);
    art->norm_denom = h[K];
    hip_check(hipMalloc(&art->rows, (size_t)g.n * art->row_bytes), "alloc edge lsh rows");
    if (g.dp <= 128 && g.R <= 64) {
      const uint32_t grid = (uint32_t)std::min<int64_t>((g.n + 3) / 4, 65536);
      hipLaunchKernelGGL(lsh_populate_rows_kernel, dim3(grid), dim3(256), 0, s, (const uint16_t*)g.vecs, g.n, g.dp,
                         g.edges, g.counts, g.R, K, P, (uint8_t*)art->rows, (uint32_t)art->row_bytes);
      hip_check(hipGetLastError(), "launch lsh_populate_rows_kernel");
    } else {
      const uint32_t grid = (uint32_t)std::min<int64_t>(g.n, 65536);
      hipLaunchKernelGGL(lsh_populate_kernel, dim3(grid), dim3(64), plds, s, (const uint16_t*)g.vecs, g.n, g.dp,
                         g.edges, g.counts, g.R, K, P, (uint8_t*)art->rows, (uint32_t)art->row_bytes);
      hip_check(hipGetLastError(), "launch lsh_populate_kernel");
    }
    hip_check(hipDeviceSynchronize(), "lsh build");
  } catch (...) {
    (void)hipFree(contrib);
    (void)hipFree(valid);
    (void)hipFree(out);
    throw;
  }
  (void)hipFree(contrib);
  (void)hipFree(valid);
  (void)hipFree(out);
  g.lsh = std::move(art);
}

static void compute_norms(Graph& g) {
  if (!g.vector_norms) hip_check(hipMalloc(&g.vector_norms, (size_t)g.n * 4), "alloc vector norms");
  const uint32_t grid = (uint32_t)std::min<int64_t>(g.n, 65536);
  hipLaunchKernelGGL(norms_kernel, dim3(grid), dim3(64), 0, nullptr, (const uint16_t*)g.vecs, g.n, g.dp,
                     g.vector_norms);
  hip_check(hipGetLastError(), "launch norms_kernel");
}

void build_pq(Graph& g, int64_t n_train, int64_t iters, uint64_t seed, uint32_t m) {
  if (g.n <= 0) throw std::runtime_error("generate_pq_codebooks: graph is empty");
  const uint32_t M = m ? m : g.k_ranks;
  if (M == 0 || g.dp % M != 0)
    throw std::runtime_error("generate_pq_codebooks: padded_dim (" + std::to_string(g.dp) +
                             ") must be divisible by M=" + std::to_string(M));
  if (M > kPqMaxM) throw std::invalid_argument("PQ supports at most " + std::to_string(kPqMaxM) + " subspaces");
  const uint32_t dsub = g.dp / M;
  if (n_train < 256) n_train = 256;
  uint16_t* X = nullptr;
  uint8_t* labels = nullptr;
  auto art = std::make_unique<PqArtifacts>();
  art->m = M;
  art->dsub = dsub;
  try {
    hip_check(hipMalloc(&X, (size_t)n_train * g.dp * 2), "alloc pq training rows");
    hip_check(hipMalloc(&labels, (size_t)n_train * M), "alloc pq labels");
    hip_check(hipMalloc(&art->centroids, (size_t)M * 256 * dsub * 4), "alloc pq centroids");
    hipLaunchKernelGGL(pq_sample_kernel, dim3((uint32_t)n_train), dim3(128), 0, nullptr, (const uint16_t*)g.vecs, g.n,
                       g.dp, g.edges, g.counts, g.R, n_train, seed, X);
    const uint64_t init_seed = seed ^ 0xA5A5A5A5ull;
    hipLaunchKernelGGL(pq_init_kernel, dim3(M * 256), dim3(64), 0, nullptr, X, n_train, g.dp, M, dsub, init_seed,
                       art->centroids);
    const size_t lds_want = (size_t)256 * dsub * 4;
    const bool stage = lds_want <= 64 * 1024;
    const size_t lds = stage ? lds_want : 0;
    const int64_t upd = (int64_t)M * 256 * dsub;
    for (int64_t it = 0; it < iters; ++it) {
      hipLaunchKernelGGL(pq_assign_kernel, dim3((uint32_t)((n_train + 255) / 256), M), dim3(256), lds, nullptr, X,
                         n_train, g.dp, M, dsub, art->centroids, labels, stage);
      hipLaunchKernelGGL(pq_update_kernel, dim3((uint32_t)((upd + 255) / 256)), dim3(256), 0, nullptr, X, n_train,
                         g.dp, M, dsub, labels, init_seed, (uint32_t)it, art->centroids);
    }
    hip_check(hipGetLastError(), "launch pq training");
    const size_t code_bytes = (size_t)g.n * pq_row_bytes(M, g.R);
    hip_check(hipMalloc(&art->codes, code_bytes), "alloc pq codes");
    hip_check(hipMemset(art->codes, 0, code_bytes), "clear pq codes");
    if (dsub <= 64) {
      // subspace centroids in LDS, one edge per lane
      const uint32_t gx = (uint32_t)std::max<int64_t>(1, std::min<int64_t>((g.n + 3) / 4, 2048 / M + 1));
      const dim3 egrid(gx, M);
      const auto launch = [&](auto kern) {
        hipLaunchKernelGGL(kern, egrid, dim3(256), 0, nullptr, (const uint16_t*)g.vecs, g.n, g.dp, g.edges,
                           g.counts, g.R, M, dsub, art->centroids, art->codes);
      };
      if (dsub <= 8) launch(pq_encode_lds_kernel<8>);
      else if (dsub <= 16) launch(pq_encode_lds_kernel<16>);
      else if (dsub <= 24) launch(pq_encode_lds_kernel<24>);
      else if (dsub <= 32) launch(pq_encode_lds_kernel<32>);
      else if (dsub <= 48) launch(pq_encode_lds_kernel<48>);
      else launch(pq_encode_lds_kernel<64>);
      hip_check(hipGetLastError(), "launch pq_encode_lds_kernel");
    } else {
      const uint32_t grid = (uint32_t)std::min<int64_t>(g.n, 65536);
      const size_t elds = (size_t)g.dp * 4 + pq_row_bytes(M, g.R);
      if (elds > 160 * 1024) throw std::invalid_argument("dim too large for the PQ encoder");
      if (elds > 64 * 1024)
        hip_check(hipFuncSetAttribute((const void*)pq_encode_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)elds), "LDS size");
      hipLaunchKernelGGL(pq_encode_kernel, dim3(grid), dim3(64), elds, nullptr, (const uint16_t*)g.vecs, g.n, g.dp,
                         g.edges, g.counts, g.R, M, dsub, art->centroids, art->codes);
      hip_check(hipGetLastError(), "launch pq_encode_kernel");
    }
    compute_norms(g);
    hip_check(hipDeviceSynchronize(), "pq build");
  } catch (...) {
    (void)hipFree(X);
    (void)hipFree(labels);
    throw;
  }
  (void)hipFree(X);
  (void)hipFree(labels);
  g.pq = std::move(art);
}

// ----------------------------------------------------------- RaBitQ build --

// Column sums of the stored rows in a fixed order (so the centroid is the
// same on every run): block b adds rows [b * chunk, (b + 1) * chunk) of each
// column (thread = column, four rows per step), then rabitq_mean_kernel adds
// the block sums in block order and divides by n.
__global__ __launch_bounds__(256) void column_partial_kernel(const uint16_t* __restrict__ vecs, int64_t n,
                                                             uint32_t dp, uint32_t dim, int64_t chunk,
                                                             float* __restrict__ partial) {
  const int64_t r0 = (int64_t)blockIdx.x * chunk, r1 = min(n, r0 + chunk);
  for (uint32_t c = threadIdx.x; c < dim; c += blockDim.x) {
    float s = 0.0f;
    int64_t r = r0;
    for (; r + 4 <= r1; r += 4) {
      const float v0 = h2f16(vecs[(size_t)r * dp + c]), v1 = h2f16(vecs[(size_t)(r + 1) * dp + c]);
      const float v2 = h2f16(vecs[(size_t)(r + 2) * dp + c]), v3 = h2f16(vecs[(size_t)(r + 3) * dp + c]);
      s = s + v0;
      s = s + v1;
      s = s + v2;
      s = s + v3;
    }
    for (; r < r1; ++r) s = s + h2f16(vecs[(size_t)r * dp + c]);
    partial[(size_t)blockIdx.x * dim + c] = s;
  }
}

__global__ void rabitq_mean_kernel(const float* __restrict__ partial, uint32_t blocks, uint32_t dim, int64_t n,
                                   float* __restrict__ out) {
  for (uint32_t c = threadIdx.x; c < dim; c += blockDim.x) {
    float s = 0.0f;
    for (uint32_t b = 0; b < blocks; ++b) s = s + partial[(size_t)b * dim + c];
    out[c] = div_rn(s, (float)n);
  }
}

__global__ void identity_kernel(float* __restrict__ P, uint32_t dim) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < (uint64_t)dim * dim) P[t] = (t % (dim + 1u) == 0) ? 1.0f : 0.0f;
}

void build_rabitq(Graph& g) {
  if (g.n <= 0) throw std::runtime_error("build_rabitq: graph is empty");
  if (g.dim == 0 || g.dim > 256) throw std::invalid_argument("RaBitQ codes support 1 <= dim <= 256");
  if (g.on_host) throw std::invalid_argument("build_rabitq requires the graph on device");
  auto art = std::make_unique<RabitqArtifacts>();
  art->dim = g.dim;
  art->code_bytes = rabitq_code_bytes(g.dim);
  const size_t node = art->code_bytes + 8;
  const uint32_t blocks = (uint32_t)std::max<int64_t>(1, std::min<int64_t>(8192, (g.n + 255) / 256));
  const int64_t chunk = (g.n + blocks - 1) / blocks;
  float* partial = nullptr;
  float* eye = nullptr;
  hip_check(hipMalloc(&art->nodes, (size_t)g.n * node), "alloc rabitq nodes");
  hip_check(hipMalloc((void**)&art->centroid, (size_t)g.dim * 4), "alloc rabitq centroid");
  try {
    hip_check(hipMalloc((void**)&partial, (size_t)blocks * g.dim * 4), "alloc column sums");
    hip_check(hipMalloc((void**)&eye, (size_t)g.dim * g.dim * 4), "alloc identity");
    hipLaunchKernelGGL(column_partial_kernel, dim3(blocks), dim3(256), 0, nullptr, (const uint16_t*)g.vecs, g.n, g.dp,
                       g.dim, chunk, partial);
    hipLaunchKernelGGL(rabitq_mean_kernel, dim3(1), dim3(256), 0, nullptr, (const float*)partial, blocks, g.dim, g.n,
                       art->centroid);
    const uint64_t pe = (uint64_t)g.dim * g.dim;
    hipLaunchKernelGGL(identity_kernel, dim3((uint32_t)((pe + 255) / 256)), dim3(256), 0, nullptr, eye, g.dim);
    hip_check(hipGetLastError(), "launch rabitq centroid");
    // the rows are already rotated when the graph was prerotated: quantize
    // them as stored (identity rotation: one product per output, exact)
    rabitq_quantize(g.vecs, true, g.n, g.dim, g.dp, eye, art->centroid, g.metric, art->nodes, nullptr);
    hip_check(hipDeviceSynchronize(), "rabitq build");
  } catch (...) {
    (void)hipFree(partial);
    (void)hipFree(eye);
    throw;
  }
  (void)hipFree(partial);
  (void)hipFree(eye);
  g.rabitq = std::move(art);
}

// Query rows [nq, dim] (device memory) into rows of stride dp, zero padded.
__global__ void pad_rows_kernel(const uint16_t* __restrict__ src, int64_t nq, uint32_t dim, uint32_t dp,
                                uint16_t* __restrict__ dst) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= nq * dp) return;
  const int64_t r = t / dp;
  const uint32_t i = (uint32_t)(t % dp);
  dst[t] = i < dim ? src[(size_t)r * dim + i] : (uint16_t)0;
}

namespace {

size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// Device scratch of one directional search: either stream-ordered
// allocations that are freed (stream-ordered) when the search returns or
// throws, or slices of a caller-provided buffer, which allocate nothing.
class SearchScratch {
 public:
  explicit SearchScratch(hipStream_t s) : s_(s) {}
  SearchScratch(hipStream_t s, void* base, size_t cap) : s_(s), base_((char*)base), cap_(cap) {}
  SearchScratch(const SearchScratch&) = delete;
  SearchScratch& operator=(const SearchScratch&) = delete;
  ~SearchScratch() {
    for (void* p : owned_) (void)hipFreeAsync(p, s_);
  }
  bool fixed() const { return base_ != nullptr; }
  void* take(size_t bytes) {
    bytes = round256(bytes);
    if (base_) {
      if (used_ + bytes > cap_) throw std::logic_error("directional search scratch overrun");
      void* p = base_ + used_;
      used_ += bytes;
      return p;
    }
    void* p = nullptr;
    hip_check(hipMallocAsync(&p, bytes, s_), "alloc directional search scratch");
    owned_.push_back(p);
    return p;
  }

 private:
  hipStream_t s_;
  char* base_ = nullptr;
  size_t cap_ = 0, used_ = 0;
  std::vector<void*> owned_;
};

// Timing events of print_throughput, destroyed on every exit.
struct EventPair {
  hipEvent_t e0 = nullptr, e1 = nullptr;
  ~EventPair() {
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
  }
};

bool device_rows(const void* p) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

// Padded and, when the graph was prerotated, rotated query rows [nq, dp]
// in scratch. Device queries are padded by a kernel; host queries (only
// with allocating scratch) by a copy.
const uint16_t* directional_query_rows(const Graph& g, const void* queries, int64_t nq, int64_t dim,
                                       hipStream_t stream, SearchScratch& scratch) {
  if (g.prerotate && !g.rotation) throw std::runtime_error("prerotated graph has no rotation matrix");
  uint16_t* rows = (uint16_t*)scratch.take((size_t)nq * g.dp * 2);
  if (device_rows(queries)) {
    const int64_t total = nq * (int64_t)g.dp;
    hipLaunchKernelGGL(pad_rows_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, stream,
                       (const uint16_t*)queries, nq, (uint32_t)dim, g.dp, rows);
    hip_check(hipGetLastError(), "launch pad_rows_kernel");
  } else {
    if (scratch.fixed()) throw std::invalid_argument("queries must be device memory");
    hip_check(hipMemsetAsync(rows, 0, (size_t)nq * g.dp * 2, stream), "clear query rows");
    hip_check(hipMemcpy2DAsync(rows, (size_t)g.dp * 2, queries, (size_t)dim * 2, (size_t)dim * 2, (size_t)nq,
                               hipMemcpyDefault, stream),
              "copy queries");
  }
  if (!g.prerotate) return rows;
  uint16_t* rot = (uint16_t*)scratch.take((size_t)nq * g.dp * 2);
  rotate_rows(*g.rotation, rows, nq, g.dp, rot, g.dp, stream);
  return rot;
}

// The LSH estimate's bf16 square-root table (1 KB) stays in LDS unless LDS
// bounds how many queries share a CU and dropping it lets one more in (wide
// beams); the kernel then computes each root with sqrt_rn, whose values the
// table holds. lds: the query's LDS without the table.
bool lsh_sqrt_in_lds(size_t lds) {
  const size_t cu = 160 * 1024, with = lds + 256 * 4;
  return cu / with >= 32 || cu / lds == cu / with;
}

// LDS of one query's wave, less the PQ table; *sqrt_lds (LSH) tells whether
// the square-root table is part of it.
size_t directional_base_lds_bytes(const Graph& g, int est, int64_t k, int64_t bw, bool* sqrt_lds = nullptr) {
  size_t lds = ((size_t)(((bw + g.R) + 64 + k + 1) & ~(int64_t)1) + dir_mark_words((uint32_t)(bw + g.R))) * 8;
  if (sqrt_lds) *sqrt_lds = false;
  if (est == kEstLsh) {
    // q and q - u (16 chunks each with 1-byte words), the sqrt table
    const size_t chunks = g.lsh->packed_bytes == 1 ? 16 : g.dp / 8;
    lds += 2 * chunks * 16;
    const bool tab = lsh_sqrt_in_lds(lds);
    if (tab) lds += 256 * 4;
    if (sqrt_lds) *sqrt_lds = tab;
  } else {
    lds += (size_t)2 * g.dp * 2;
  }
  return lds;
}

// PQ: the table layout in LDS. A table of more than 64 subspaces leaves
// room for one query per CU; when a launch has more queries than CUs, the
// kernel keeps the first 4 groups of 16 subspaces in LDS, which lets two
// queries share a CU (5 groups would be 80 KB alone), and gathers the
// entries of the other groups from the table in global memory -- all but
// the last group's when its rows fit in LDS beside the 4 (a full group and
// the last group's rows save the same gathers per KB). The sum runs over
// the subspaces in the same order in every layout.
int pq_lut_layout(const Graph& g, int64_t k, int64_t bw, int64_t nq) {
  const uint32_t m = g.pq->m;
  if (m <= 64) return kLutWhole;
  static const int cus = [] {
    int dev = 0, c = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
      c = 256;
    return c;
  }();
  const size_t base = directional_base_lds_bytes(g, kEstPq, k, bw);
  const size_t half_cu = 80 * 1024, four = 64 * 1024;
  if (nq <= cus || base + (size_t)pq_lut_rows(m) * 1024 <= half_cu || base + four > half_cu) return kLutWhole;
  return m % 16 != 0 && base + four + (size_t)pq_lut_rows(m % 16) * 1024 <= half_cu ? kLutSplitLast : kLutSplit;
}

// LDS of one query's wave, with the PQ table in the given layout.
size_t directional_lds_bytes(const Graph& g, int est, int64_t k, int64_t bw, int lut_layout = kLutWhole,
                             bool* sqrt_lds = nullptr) {
  size_t lds = directional_base_lds_bytes(g, est, k, bw, sqrt_lds);
  if (est == kEstPq) {
    const uint32_t m = g.pq->m;
    const uint32_t rows = lut_layout == kLutWhole ? pq_lut_rows(m)
                        : lut_layout == kLutSplitLast ? 64 + pq_lut_rows(m % 16)
                                                      : 64;
    lds += (size_t)rows * 1024;
  }
  return lds;
}

// Every argument check of directional_search, before anything is allocated
// or launched.
void check_directional_search(const Graph& g, int est, int64_t nq, int64_t dim, int64_t k, int64_t bw,
                              int64_t limit) {
  if (est < kEstLsh || est > kEstRabitq) throw std::invalid_argument("unknown directional estimator");
  const bool use_pq = est == kEstPq;
  if (use_pq && !g.pq) throw std::runtime_error("graph has no PQ artifacts built — call build_pq() first");
  if (est == kEstLsh && !g.lsh) throw std::runtime_error("graph has no LSH artifacts built — call build_lsh() first");
  if (est == kEstRabitq && !g.rabitq)
    throw std::runtime_error("graph has no RaBitQ codes built — call build_rabitq() first");
  if (dim != (int64_t)g.dim)
    throw std::invalid_argument("query dim (" + std::to_string(dim) + ") != graph dim (" + std::to_string(g.dim) + ")");
  if (nq < 0 || k < 0 || bw <= 0 || limit < 0) throw std::invalid_argument("negative size argument");
  if (nq > 0x7FFFFFFF) throw std::invalid_argument("too many queries");
  if (bw + 64 >= 2048)
    throw std::invalid_argument("beam_width " + std::to_string(bw) + " is too large (beam_width + 64 must be < 2048)");
  if (g.R > 64) throw std::invalid_argument("R must be <= 64");
  if (g.n <= 0) throw std::runtime_error("graph is empty");
  if ((int64_t)g.medoid >= g.n) throw std::runtime_error("graph medoid is out of range");
  if (use_pq) {
    if (g.metric == kL2 && !g.vector_norms) throw std::runtime_error("graph has no vector norms");
    if (g.pq->m == 0 || g.pq->m > kPqMaxM)
      throw std::invalid_argument("pq_search supports at most " + std::to_string(kPqMaxM) + " subspaces");
  } else if (est == kEstLsh && !((g.lsh->k_ranks == 4 || g.lsh->k_ranks == 16) &&
                                  (g.lsh->packed_bytes == 1 || g.lsh->packed_bytes == 2))) {
    throw std::invalid_argument("k_ranks must be 4 or 16 with 1- or 2-byte words");
  } else if (est == kEstLsh && g.lsh->packed_bytes == 1 && g.dp > 128) {
    throw std::invalid_argument("1-byte LSH words address at most 128 dims");
  } else if (est == kEstRabitq && (g.rabitq->dim != g.dim || g.rabitq->code_bytes > 32)) {
    throw std::invalid_argument("RaBitQ codes do not match the graph");
  }
  if (directional_lds_bytes(g, est, k, bw, use_pq ? pq_lut_layout(g, k, bw, nq) : kLutWhole) > 160 * 1024)
    throw std::invalid_argument("beam_width, k and dim need more than 160 KB of LDS");
}

template <int METRIC, int K, int P, int LUT = kLutWhole>
void launch_directional(const DirArgs& a, uint32_t nq, size_t lds, hipStream_t stream) {
  auto kern = directional_kernel<METRIC, K, P, LUT>;
  if (lds > 64 * 1024)
    hip_check(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
              "LDS size");
  hipLaunchKernelGGL(kern, dim3(nq), dim3(64), lds, stream, a);
}

// The search after check_directional_search, with its device buffers taken
// from `scratch`.
void directional_search_run(Graph& g, int est, const void* queries, int64_t nq, int64_t dim, int32_t* out_ids,
                            float* out_dists, int64_t k, int64_t bw, int64_t limit, bool print, hipStream_t stream,
                            uint32_t* stats, bool unique, SearchScratch& scratch) {
  const bool use_pq = est == kEstPq;
  EventPair ev;
  if (print) {
    hip_check(hipEventCreate(&ev.e0), "event");
    hip_check(hipEventCreate(&ev.e1), "event");
    hip_check(hipEventRecord(ev.e0, stream), "event record");
  }
  const uint16_t* qsrc = directional_query_rows(g, queries, nq, dim, stream, scratch);
  DirArgs a{};
  a.vecs = (const uint16_t*)g.vecs;
  a.n = g.n;
  a.dp = g.dp;
  a.R = g.R;
  a.edges = g.edges;
  a.counts = g.counts;
  a.deleted = g.deleted;
  a.queries = qsrc;
  a.medoid = g.medoid;
  a.k = (uint32_t)k;
  a.bw = (uint32_t)bw;
  a.limit = (uint32_t)limit;
  a.max_result = 2048;
  a.out_ids = out_ids;
  a.out_dists = out_dists;
  a.stats = stats;
  a.unique = unique ? 1u : 0u;
  const int lut_layout = use_pq ? pq_lut_layout(g, k, bw, nq) : kLutWhole;
  bool sqrt_lds = false;
  const size_t lds = directional_lds_bytes(g, est, k, bw, lut_layout, &sqrt_lds);
  a.sqrt_lds = sqrt_lds ? 1u : 0u;
  const bool l2 = g.metric == kL2;
  if (est == kEstRabitq) {
    const RabitqArtifacts& rq = *g.rabitq;
    a.rq_nodes = (const uint8_t*)rq.nodes;
    a.rq_centroid = rq.centroid;
    a.rq_node_bytes = rq.code_bytes + 8;
    a.rq_words = rq.code_bytes / 4;
    a.rq_dim = rq.dim;
    if (a.rq_words <= 4) {
      if (l2) launch_directional<kL2, 1, 4>(a, (uint32_t)nq, lds, stream);
      else launch_directional<kIP, 1, 4>(a, (uint32_t)nq, lds, stream);
    } else {
      if (l2) launch_directional<kL2, 1, 8>(a, (uint32_t)nq, lds, stream);
      else launch_directional<kIP, 1, 8>(a, (uint32_t)nq, lds, stream);
    }
  } else if (use_pq) {
    a.M = g.pq->m;
    a.dsub = g.pq->dsub;
    a.centroids = g.pq->centroids;
    a.codes = g.pq->codes;
    a.code_row_bytes = (uint32_t)pq_row_bytes(a.M, g.R);
    a.pq_w = pq_group_width(a.M);
    a.pq_groups = pq_groups(a.M);
    a.norms = g.vector_norms;
    float* luts = (float*)scratch.take((size_t)nq * pq_lut_rows(a.M) * 256 * 4);
    const auto small_lut = [&](auto kern) {
      const dim3 lgrid((uint32_t)((nq + kLutQueries - 1) / kLutQueries), pq_lut_rows(a.M));
      hipLaunchKernelGGL(kern, lgrid, dim3(256), 0, stream, qsrc, nq, a.dp, a.M, a.dsub, a.centroids, luts);
    };
    if (a.dsub <= 8) small_lut(pq_lut_small_kernel<8>);
    else if (a.dsub <= 16) small_lut(pq_lut_small_kernel<16>);
    else if (a.dsub <= 32) small_lut(pq_lut_small_kernel<32>);
    else {
      const dim3 lgrid((uint32_t)nq, (pq_lut_rows(a.M) * 256 + kLutWaveEntries - 1) / kLutWaveEntries);
      hipLaunchKernelGGL(pq_lut_kernel, lgrid, dim3(64), 0, stream, qsrc, a.dp, a.M, a.dsub, a.centroids, luts);
    }
    hip_check(hipGetLastError(), "launch PQ table kernel");
    a.luts = luts;
    const uint32_t n32 = (uint32_t)nq;
    if (a.M <= 16) {
      if (l2) launch_directional<kL2, 0, 1>(a, n32, lds, stream);
      else launch_directional<kIP, 0, 1>(a, n32, lds, stream);
    } else if (lut_layout == kLutSplitLast) {
      if (l2) launch_directional<kL2, 0, 8, kLutSplitLast>(a, n32, lds, stream);
      else launch_directional<kIP, 0, 8, kLutSplitLast>(a, n32, lds, stream);
    } else if (lut_layout == kLutSplit) {
      if (l2) launch_directional<kL2, 0, 8, kLutSplit>(a, n32, lds, stream);
      else launch_directional<kIP, 0, 8, kLutSplit>(a, n32, lds, stream);
    } else {
      if (l2) launch_directional<kL2, 0, 8>(a, n32, lds, stream);
      else launch_directional<kIP, 0, 8>(a, n32, lds, stream);
    }
  } else {
    a.K = g.lsh->k_ranks;
    a.pbytes = g.lsh->packed_bytes;
    a.lsh_rows = (const uint8_t*)g.lsh->rows;
    a.row_bytes = (uint32_t)g.lsh->row_bytes;
    for (uint32_t r = 0; r < a.K; ++r) a.c[r] = g.lsh->c_per_rank[r];
    a.inv_norm_denom = 1.0f / g.lsh->norm_denom;
    const uint32_t n32 = (uint32_t)nq;
    if (a.K == 4 && a.pbytes == 1) {
      if (l2) launch_directional<kL2, 4, 1>(a, n32, lds, stream);
      else launch_directional<kIP, 4, 1>(a, n32, lds, stream);
    } else if (a.K == 16 && a.pbytes == 1) {
      if (l2) launch_directional<kL2, 16, 1>(a, n32, lds, stream);
      else launch_directional<kIP, 16, 1>(a, n32, lds, stream);
    } else if (a.K == 4) {
      if (l2) launch_directional<kL2, 4, 2>(a, n32, lds, stream);
      else launch_directional<kIP, 4, 2>(a, n32, lds, stream);
    } else {
      if (l2) launch_directional<kL2, 16, 2>(a, n32, lds, stream);
      else launch_directional<kIP, 16, 2>(a, n32, lds, stream);
    }
  }
  hip_check(hipGetLastError(), "launch directional_kernel");
  if (print) {
    hip_check(hipEventRecord(ev.e1, stream), "event record");
    hip_check(hipEventSynchronize(ev.e1), "event sync");
    float ms = 0;
    (void)hipEventElapsedTime(&ms, ev.e0, ev.e1);
    std::printf("[%s] duration=%gms, throughput=%g\n",
                use_pq ? "pq_search" : (est == kEstRabitq ? "rabitq_search" : "directional_search"), ms,
                nq * 1000.0 / ms);
    std::fflush(stdout);
  }
}

}  // namespace

void rabitq_build_search(const Graph& g, uint32_t q_start, uint32_t nq, uint32_t bw, uint32_t limit,
                         uint32_t max_result, uint64_t* visited, uint32_t* visited_counts, hipStream_t stream) {
  if (!g.rabitq) throw std::runtime_error("RaBitQ build search needs the RaBitQ codes");
  if (nq == 0) return;
  if ((int64_t)q_start + nq > g.n) throw std::invalid_argument("query range out of bounds");
  if (g.R > 64) throw std::invalid_argument("R must be <= 64");
  DirArgs a{};
  a.vecs = (const uint16_t*)g.vecs;
  a.n = g.n;
  a.dp = g.dp;
  a.R = g.R;
  a.edges = g.edges;
  a.counts = g.counts;
  a.deleted = g.deleted;
  a.medoid = g.medoid;
  a.k = 0;
  a.bw = bw;
  a.limit = limit;
  a.max_result = max_result;
  a.visited = visited;
  a.visited_counts = visited_counts;
  a.q_start = q_start;
  const RabitqArtifacts& rq = *g.rabitq;
  a.rq_nodes = (const uint8_t*)rq.nodes;
  a.rq_centroid = rq.centroid;
  a.rq_node_bytes = rq.code_bytes + 8;
  a.rq_words = rq.code_bytes / 4;
  a.rq_dim = rq.dim;
  const size_t lds = directional_lds_bytes(g, kEstRabitq, 0, bw);
  const bool l2 = g.metric == kL2;
  if (a.rq_words <= 4) {
    if (l2) launch_directional<kL2, 1, 4>(a, nq, lds, stream);
    else launch_directional<kIP, 1, 4>(a, nq, lds, stream);
  } else {
    if (l2) launch_directional<kL2, 1, 8>(a, nq, lds, stream);
    else launch_directional<kIP, 1, 8>(a, nq, lds, stream);
  }
  hip_check(hipGetLastError(), "launch directional_kernel (build search)");
}

size_t directional_scratch_bytes(const Graph& g, int est, int64_t nq) {
  if (nq <= 0) return 0;
  const size_t rows = round256((size_t)nq * g.dp * 2);
  size_t b = rows + (g.prerotate ? rows : 0);
  if (est == kEstPq && g.pq) b += round256((size_t)nq * pq_lut_rows(g.pq->m) * 256 * 4);
  return b;
}

void directional_query_rows_to_host(const Graph& g, const void* queries, int64_t nq, int64_t dim, uint16_t* out,
                                    hipStream_t stream) {
  if (dim != (int64_t)g.dim) throw std::invalid_argument("query dim does not match the graph");
  if (nq <= 0) return;
  SearchScratch scratch(stream);
  const uint16_t* rows = directional_query_rows(g, queries, nq, dim, stream, scratch);
  hip_check(hipMemcpyAsync(out, rows, (size_t)nq * g.dp * 2, hipMemcpyDefault, stream), "download query rows");
  hip_check(hipStreamSynchronize(stream), "sync query rows");
}

void directional_search(Graph& g, int est, const void* queries, int64_t nq, int64_t dim, int32_t* out_ids,
                        float* out_dists, int64_t k, int64_t bw, int64_t limit, bool print, hipStream_t stream,
                        uint32_t* stats, bool unique) {
  check_directional_search(g, est, nq, dim, k, bw, limit);
  if (nq == 0 || k == 0) return;
  SearchScratch scratch(stream);
  directional_search_run(g, est, queries, nq, dim, out_ids, out_dists, k, bw, limit, print, stream, stats, unique,
                         scratch);
}

void exact_search(Graph& g, const void* queries, int64_t nq, int64_t dim, int32_t* out_ids, float* out_dists,
                  int64_t k, int64_t bw, int64_t limit, hipStream_t stream) {
  if (dim != (int64_t)g.dim)
    throw std::invalid_argument("query dim (" + std::to_string(dim) + ") != graph dim (" + std::to_string(g.dim) + ")");
  if (nq < 0 || k < 0 || bw <= 0 || limit < 0) throw std::invalid_argument("negative size argument");
  if (nq > 0x7FFFFFFF) throw std::invalid_argument("too many queries");
  if (nq == 0 || k == 0) return;
  if (bw + 64 >= 2048)
    throw std::invalid_argument("beam_width " + std::to_string(bw) + " is too large (beam_width + 64 must be < 2048)");
  SearchScratch scratch(stream);
  const uint16_t* rows = directional_query_rows(g, queries, nq, dim, stream, scratch);
  SearchRequest r;
  r.queries = rows;
  r.nq = (uint32_t)nq;
  r.medoid = g.medoid;
  r.k = (uint32_t)k;
  r.beam_width = (uint32_t)bw;
  r.limit = (uint32_t)limit;
  r.max_result = 2048;
  r.out_ids = out_ids;
  r.out_dists = out_dists;
  launch_beam_search(g, r, stream);
}

void directional_search_fixed(Graph& g, int est, const void* queries, int64_t nq, int64_t dim, int32_t* out_ids,
                              float* out_dists, int64_t k, int64_t bw, int64_t limit, bool unique, hipStream_t stream,
                              void* scratch_base, size_t scratch_bytes) {
  check_directional_search(g, est, nq, dim, k, bw, limit);
  if (nq == 0 || k == 0) return;
  const size_t need = directional_scratch_bytes(g, est, nq);
  if (need > scratch_bytes)
    throw std::invalid_argument("directional search of " + std::to_string(nq) + " queries needs " +
                                std::to_string(need) + " bytes of scratch; at most " + std::to_string(scratch_bytes) +
                                " are available (search fewer queries per call)");
  if (!device_rows(queries)) throw std::invalid_argument("queries must be device memory");
  SearchScratch scratch(stream, scratch_base, scratch_bytes);
  directional_search_run(g, est, queries, nq, dim, out_ids, out_dists, k, bw, limit, false, stream, nullptr, unique,
                         scratch);
}

// ------------------------------------------------- allocation-free search --
// Scratch of directional_search_noalloc: a file-scope device array, so each
// GPU the library runs on holds one copy from module load until the process
// ends. Host code never passes the array's name to a kernel or copy (on the
// host it is only a stand-in for the symbol): the device address comes from
// hipGetSymbolAddress, taken once per device with that device current.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

void* scratch_address() {
  int dev = 0;
  hip_check(hipGetDevice(&dev), "current device");
  if (dev < 0 || dev >= kMaxDevices) throw std::runtime_error("device index out of range for the static scratch");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "address of the static search scratch");
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}
}  // namespace

size_t directional_noalloc_scratch_bytes() { return kNoAllocScratchBytes; }

void directional_search_noalloc(Graph& g, int est, const void* queries, int64_t nq, int64_t dim,
                                int32_t* out_ids, float* out_dists, int64_t k, int64_t bw, int64_t limit,
                                bool unique, hipStream_t stream) {
  // every byte a call reads from the scratch it has written first (the
  // padded query rows, their rotation, the PQ tables), so nothing is cleared
  directional_search_fixed(g, est, queries, nq, dim, out_ids, out_dists, k, bw, limit, unique, stream,
                           scratch_address(), kNoAllocScratchBytes);
}

// ---------------------------------------------------------------- files --
// Trailer after the base section (graph.cuh:1790-1937): u32 magic, u32
// version, u8 flags (1 LSH, 2 PQ, 4 norms); LSH: u8 K, u8 sizeof(packed_t),
// K floats c_per_rank + float norm_denom, N rows; PQ: u32 M, u32 256,
// u32 dsub, centroids, N code rows; norms: N floats. This build adds flag 8
// (prerotated rows) with a u64 seed after the other sections, then flag 16
// (RaBitQ codes: u32 dim, u32 code bytes, dim floats of centroid, N nodes):
// readers that know flags 1, 2 and 4 only stop before them. Read back at the end of
// the base section (total_file_size), where the saver puts it; the
// reference loader looks elsewhere (graph.cuh:1959-1964) and never finds it.

// Vertices per pass of the code layout conversion (bounds its device buffer).
constexpr int64_t kPqLayoutChunk = 1 << 18;

void pq_codes_to_file_layout(const Graph& g, uint8_t* out) {
  const uint32_t M = g.pq->m, R = g.R;
  const size_t dev_row = pq_row_bytes(M, R), file_row = (size_t)M * R;
  const int64_t chunk = std::min<int64_t>(g.n, kPqLayoutChunk);
  void* tmp = nullptr;
  hip_check(hipMalloc(&tmp, (size_t)chunk * file_row), "alloc code layout buffer");
  try {
    for (int64_t u0 = 0; u0 < g.n; u0 += chunk) {
      const int64_t cnt = std::min<int64_t>(chunk, g.n - u0);
      const int64_t threads = cnt * R;
      hipLaunchKernelGGL(pq_layout_kernel, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, nullptr,
                         g.pq->codes + (size_t)u0 * dev_row, (uint8_t*)tmp, cnt, R, M, true);
      hip_check(hipGetLastError(), "launch pq_layout_kernel");
      hip_check(hipMemcpy(out + (size_t)u0 * file_row, tmp, (size_t)cnt * file_row, hipMemcpyDeviceToHost),
                "download codes");
    }
  } catch (...) {
    (void)hipFree(tmp);
    throw;
  }
  (void)hipFree(tmp);
}

// Device codes (allocated here) of n vertices from subspace-major rows.
static void pq_codes_from_file_layout(PqArtifacts& art, int64_t n, uint32_t R, const uint8_t* in) {
  const uint32_t M = art.m;
  const size_t dev_row = pq_row_bytes(M, R), file_row = (size_t)M * R;
  hip_check(hipMalloc(&art.codes, (size_t)n * dev_row), "alloc codes");
  hip_check(hipMemset(art.codes, 0, (size_t)n * dev_row), "clear codes");
  const int64_t chunk = std::min<int64_t>(n, kPqLayoutChunk);
  void* tmp = nullptr;
  hip_check(hipMalloc(&tmp, (size_t)chunk * file_row), "alloc code layout buffer");
  try {
    for (int64_t u0 = 0; u0 < n; u0 += chunk) {
      const int64_t cnt = std::min<int64_t>(chunk, n - u0);
      hip_check(hipMemcpy(tmp, in + (size_t)u0 * file_row, (size_t)cnt * file_row, hipMemcpyHostToDevice),
                "upload codes");
      const int64_t threads = cnt * R;
      hipLaunchKernelGGL(pq_layout_kernel, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, nullptr,
                         (const uint8_t*)tmp, art.codes + (size_t)u0 * dev_row, cnt, R, M, false);
      hip_check(hipGetLastError(), "launch pq_layout_kernel");
    }
    hip_check(hipDeviceSynchronize(), "code layout");
  } catch (...) {
    (void)hipFree(tmp);
    throw;
  }
  (void)hipFree(tmp);
}

void save_directional_file(const Graph& g, const std::string& path) {
  save_graph_file(g, path);
  if (g.n == 0) return;
  const bool has_lsh = (bool)g.lsh, has_pq = (bool)g.pq, has_norms = g.vector_norms != nullptr;
  const bool has_rq = (bool)g.rabitq;
  if (!has_lsh && !has_pq && !has_norms && !g.prerotate && !has_rq) return;
  std::ofstream f(path, std::ios::binary | std::ios::app);
  if (!f.is_open()) throw std::runtime_error("save_directional_graph_to_file: cannot reopen " + path);
  const uint8_t flags = (has_lsh ? 1u : 0u) | (has_pq ? 2u : 0u) | (has_norms ? 4u : 0u) | (g.prerotate ? 8u : 0u) |
                        (has_rq ? 16u : 0u);
  f.write((const char*)&kTrailerMagic, 4);
  f.write((const char*)&kTrailerVersion, 4);
  f.write((const char*)&flags, 1);
  hip_check(hipDeviceSynchronize(), "sync before save");
  if (has_lsh) {
    const uint8_t K = (uint8_t)g.lsh->k_ranks, P = (uint8_t)g.lsh->packed_bytes;
    f.write((const char*)&K, 1);
    f.write((const char*)&P, 1);
    f.write((const char*)g.lsh->c_per_rank.data(), (std::streamsize)K * 4);
    f.write((const char*)&g.lsh->norm_denom, 4);
    std::vector<uint8_t> h((size_t)g.n * g.lsh->row_bytes);
    hip_check(hipMemcpy(h.data(), g.lsh->rows, h.size(), hipMemcpyDeviceToHost), "download lsh rows");
    f.write((const char*)h.data(), (std::streamsize)h.size());
  }
  if (has_pq) {
    const uint32_t M = g.pq->m, K = 256, dsub = g.pq->dsub;
    f.write((const char*)&M, 4);
    f.write((const char*)&K, 4);
    f.write((const char*)&dsub, 4);
    std::vector<float> c((size_t)M * K * dsub);
    hip_check(hipMemcpy(c.data(), g.pq->centroids, c.size() * 4, hipMemcpyDeviceToHost), "download centroids");
    f.write((const char*)c.data(), (std::streamsize)c.size() * 4);
    std::vector<uint8_t> codes((size_t)g.n * M * g.R);
    pq_codes_to_file_layout(g, codes.data());
    f.write((const char*)codes.data(), (std::streamsize)codes.size());
  }
  if (has_norms) {
    std::vector<float> nrm((size_t)g.n);
    hip_check(hipMemcpy(nrm.data(), g.vector_norms, nrm.size() * 4, hipMemcpyDeviceToHost), "download norms");
    f.write((const char*)nrm.data(), (std::streamsize)nrm.size() * 4);
  }
  if (g.prerotate) {
    const uint64_t seed = g.prerotate_seed;
    f.write((const char*)&seed, 8);
  }
  if (has_rq) {
    const RabitqArtifacts& rq = *g.rabitq;
    f.write((const char*)&rq.dim, 4);
    f.write((const char*)&rq.code_bytes, 4);
    std::vector<float> c(rq.dim);
    hip_check(hipMemcpy(c.data(), rq.centroid, (size_t)rq.dim * 4, hipMemcpyDeviceToHost), "download centroid");
    f.write((const char*)c.data(), (std::streamsize)c.size() * 4);
    std::vector<uint8_t> h((size_t)g.n * (rq.code_bytes + 8));
    hip_check(hipMemcpy(h.data(), rq.nodes, h.size(), hipMemcpyDeviceToHost), "download rabitq nodes");
    f.write((const char*)h.data(), (std::streamsize)h.size());
  }
  if (!f.good()) throw std::runtime_error("short write while saving " + path);
}

// The trailer of a directional file from byte `off` (absent or foreign
// trailers leave the graph as loaded).
static void read_directional_trailer(Graph& gr, const std::string& path, uint64_t off) {
  Graph* g = &gr;
  const uint32_t k_ranks = g->k_ranks, R = g->R;
  if (g->n == 0) return;
  std::ifstream f(path, std::ios::binary | std::ios::ate);
  if (!f.is_open()) throw std::runtime_error("load_directional_graph_from_file: cannot reopen " + path);
  const uint64_t size = (uint64_t)f.tellg();
  if (size < off + 9) return;
  f.seekg((std::streamoff)off);
  uint32_t magic = 0, version = 0;
  uint8_t flags = 0;
  f.read((char*)&magic, 4);
  f.read((char*)&version, 4);
  f.read((char*)&flags, 1);
  if (magic != kTrailerMagic || version != kTrailerVersion) return;
  if (flags & 1u) {
    uint8_t K = 0, P = 0;
    f.read((char*)&K, 1);
    f.read((char*)&P, 1);
    if (K != k_ranks || P != g->packed_bytes)
      throw std::runtime_error("load_directional_graph_from_file: LSH trailer k_ranks/packed_t mismatch — file was "
                               "written with a different graph_cfg");
    auto art = std::make_unique<LshArtifacts>();
    art->k_ranks = K;
    art->packed_bytes = P;
    art->row_bytes = (size_t)R * K * P + 2 * (size_t)R;
    art->c_per_rank.resize(K);
    f.read((char*)art->c_per_rank.data(), (std::streamsize)K * 4);
    f.read((char*)&art->norm_denom, 4);
    std::vector<uint8_t> h((size_t)g->n * art->row_bytes);
    f.read((char*)h.data(), (std::streamsize)h.size());
    if ((size_t)f.gcount() != h.size()) throw std::runtime_error("truncated LSH trailer in " + path);
    hip_check(hipMalloc(&art->rows, h.size()), "alloc lsh rows");
    hip_check(hipMemcpy(art->rows, h.data(), h.size(), hipMemcpyHostToDevice), "upload lsh rows");
    g->lsh = std::move(art);
  }
  if (flags & 2u) {
    uint32_t M = 0, K = 0, dsub = 0;
    f.read((char*)&M, 4);
    f.read((char*)&K, 4);
    f.read((char*)&dsub, 4);
    // the reference requires M == k_ranks; this build also reads the other
    // subspace counts it writes (build_pq with m)
    if (M == 0 || M > kPqMaxM || K != 256 || g->dp % M != 0 || dsub != g->dp / M)
      throw std::runtime_error("load_directional_graph_from_file: PQ trailer M/K mismatch — file was written with a "
                               "different graph_cfg");
    auto art = std::make_unique<PqArtifacts>();
    art->m = M;
    art->dsub = dsub;
    std::vector<float> c((size_t)M * K * dsub);
    f.read((char*)c.data(), (std::streamsize)c.size() * 4);
    std::vector<uint8_t> codes((size_t)g->n * M * R);
    f.read((char*)codes.data(), (std::streamsize)codes.size());
    if ((size_t)f.gcount() != codes.size()) throw std::runtime_error("truncated PQ trailer in " + path);
    hip_check(hipMalloc(&art->centroids, c.size() * 4), "alloc centroids");
    hip_check(hipMemcpy(art->centroids, c.data(), c.size() * 4, hipMemcpyHostToDevice), "upload centroids");
    pq_codes_from_file_layout(*art, g->n, R, codes.data());
    g->pq = std::move(art);
  }
  if (flags & 4u) {
    std::vector<float> nrm((size_t)g->n);
    f.read((char*)nrm.data(), (std::streamsize)nrm.size() * 4);
    if ((size_t)f.gcount() != nrm.size() * 4) throw std::runtime_error("truncated norms in " + path);
    hip_check(hipMalloc(&g->vector_norms, nrm.size() * 4), "alloc norms");
    hip_check(hipMemcpy(g->vector_norms, nrm.data(), nrm.size() * 4, hipMemcpyHostToDevice), "upload norms");
  }
  if (flags & 8u) {
    uint64_t s = 0;
    f.read((char*)&s, 8);
    if (f.gcount() != 8) throw std::runtime_error("truncated prerotation record in " + path);
    g->prerotate = true;
    g->prerotate_seed = s;
  }
  if (flags & 16u) {
    auto art = std::make_unique<RabitqArtifacts>();
    f.read((char*)&art->dim, 4);
    f.read((char*)&art->code_bytes, 4);
    if (art->dim != g->dim || art->code_bytes != rabitq_code_bytes(g->dim))
      throw std::runtime_error("RaBitQ trailer does not match the graph in " + path);
    std::vector<float> c(art->dim);
    f.read((char*)c.data(), (std::streamsize)c.size() * 4);
    std::vector<uint8_t> h((size_t)g->n * (art->code_bytes + 8));
    f.read((char*)h.data(), (std::streamsize)h.size());
    if ((size_t)f.gcount() != h.size()) throw std::runtime_error("truncated RaBitQ trailer in " + path);
    hip_check(hipMalloc((void**)&art->centroid, c.size() * 4), "alloc rabitq centroid");
    hip_check(hipMemcpy(art->centroid, c.data(), c.size() * 4, hipMemcpyHostToDevice), "upload rabitq centroid");
    hip_check(hipMalloc(&art->nodes, h.size()), "alloc rabitq nodes");
    hip_check(hipMemcpy(art->nodes, h.data(), h.size(), hipMemcpyHostToDevice), "upload rabitq nodes");
    g->rabitq = std::move(art);
  }
  return;
}

std::unique_ptr<Graph> load_directional_file(const std::string& path, uint32_t dim, uint32_t R, int metric,
                                             uint32_t k_ranks, bool small_dim, bool on_host, bool prerotate,
                                             uint64_t seed) {
  uint64_t off = 0;
  auto g = load_graph_file(path, dim, R, metric, on_host, &off);
  g->k_ranks = k_ranks;
  g->packed_bytes = small_dim ? 1 : 2;
  g->prerotate = prerotate;
  g->prerotate_seed = seed;
  read_directional_trailer(*g, path, off);
  // a prerotation recorded in the file (flag 8) wins over the arguments
  if (g->prerotate) g->rotation = make_rotation(rotation_matrix(dim, g->prerotate_seed), dim);
  return g;
}

}  // namespace jasper_amd

// The prerotation matrix (column-major fp32, before the fp16 cast), for
// callers that rotate on their own and for tests.
extern "C" int64_t jasperx_rotation_matrix(int64_t dim, int64_t seed, float* out) {
  if (dim <= 0 || dim > 65536 || out == nullptr) return -1;
  const std::vector<float> m = jasper_amd::rotation_matrix((uint32_t)dim, (uint64_t)seed);
  std::memcpy(out, m.data(), m.size() * sizeof(float));
  return 0;
}
