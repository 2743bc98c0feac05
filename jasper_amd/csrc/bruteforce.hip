// bruteforce.hip -- exact k-NN by brute force on the matrix cores
// (the reference's ground-truth utility, python/jasper/__init__.py:828-926).
//
// Arithmetic as the reference computes it: L2 = (||q||^2 + ||v||^2) - 2 q.v in
// fp32, clamped at 0; IP = -(q.v) where the fp16 matmul's result is rounded to
// fp16 before the negation. q.v comes from v_mfma_f32_32x32x16_f16 (fp16
// products are exact in fp32, accumulation in fp32); the squared norms are
// fp32 sums in element order. Ties are ordered by (distance, id).
//
// Phase 1 (bf_scan_kernel): one wave owns 32 queries and one chunk of the
// base. It holds the A fragments of its queries in registers and walks the
// chunk 32 vectors at a time (one 32x32 output tile, K over the padded dim),
// loading the next 32 vectors while the current ones are on the matrix cores.
// Work-groups of one chunk run side by side (query tile is the fast grid
// index), so the chunk is read from HBM about once and served from L2 to the
// other query tiles. A score enters a per-query candidate buffer in LDS only
// if it beats the query's current k-th best; a buffer that could overflow in
// the next step is compacted (sorted, cut to k), which also lowers the
// threshold. At the end each (query, chunk) writes its best k, sorted.
// Phase 2 (bf_merge_kernel): one wave per query merges the chunk lists.
#include "bruteforce.hpp"
#include "common.hpp"
#include "graph.hpp"

#include <algorithm>
#include <cfloat>
#include <stdexcept>

namespace jasper_amd {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kBfMaxK = 64;          // k the fused scan supports
constexpr int kBfStep = 32;          // vectors per step = most keys a query can gain per step

__device__ __forceinline__ half8 u4_as_h8(uint4 v) {
  half8 h;
  __builtin_memcpy(&h, &v, 16);
  return h;
}

// ||x||^2 per row, fp32 fma in element order.
__global__ void row_sqnorm_kernel(const uint16_t* __restrict__ x, int64_t n, uint32_t dp, uint32_t dim,
                                  float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint16_t* r = x + (size_t)i * dp;
  float s = 0.0f;
  for (uint32_t t = 0; t < dim; ++t) {
    const float v = __half2float(__ushort_as_half(r[t]));
    s = __builtin_fmaf(v, v, s);
  }
  out[i] = s;
}

// Sort key: order-preserving distance bits (high) and id (low).
__device__ __forceinline__ uint64_t bf_key(float d, uint32_t id) { return ((uint64_t)dist_to_ord(d) << 32) | id; }

// Compact one query's buffer through the wave's 128-entry scratch: sort the
// cnt (<= 128) keys, keep min(cnt, k) in buf; returns that count and the k-th
// key (~0 when fewer than k remain). Wave-wide.
__device__ uint32_t bf_compact(uint64_t* buf, uint32_t cnt, uint32_t k, uint64_t* scratch, uint64_t* kth) {
  const uint32_t lane = lane_id();
  scratch[lane] = lane < cnt ? buf[lane] : ~0ull;
  scratch[lane + 64] = lane + 64 < cnt ? buf[lane + 64] : ~0ull;
  wave_sync();
  lds_bitonic_sort(scratch, 128);
  const uint32_t keep = min(cnt, k);
  if (lane < keep) buf[lane] = scratch[lane];
  *kth = keep == k ? scratch[k - 1] : ~0ull;
  wave_sync();
  return keep;
}

template <int KS, int METRIC>
__global__ __launch_bounds__(64) void bf_scan_kernel(const uint16_t* __restrict__ base, int64_t n, uint32_t dp,
                                                     const uint16_t* __restrict__ queries, int64_t nq,
                                                     const float* __restrict__ vsq, const float* __restrict__ qsq,
                                                     uint32_t k, uint32_t cap, int64_t chunk, uint32_t n_chunks,
                                                     uint64_t* __restrict__ out /* [nq][n_chunks][k] */) {
  // cap = k + kBfStep rounded up to 8: candidate slots per query
  extern __shared__ uint64_t bf_lds[];
  uint64_t* cand = bf_lds;                 // [32][cap]
  uint64_t* scratch = bf_lds + 32 * cap;   // [128]
  __shared__ uint32_t cnt[32];
  __shared__ uint64_t thr[32];
  const uint32_t lane = threadIdx.x;
  const int64_t q0 = (int64_t)blockIdx.x * 32;
  const uint32_t ci = blockIdx.y;
  const int64_t v_begin = (int64_t)ci * chunk;
  const int64_t v_end = min(n, v_begin + chunk);
  const uint32_t nck = dp / 8;  // 16-byte chunks per row

  if (lane < 32) {
    cnt[lane] = 0;
    thr[lane] = ~0ull;
  }
  wave_sync();

  // A fragments: lane holds query q0 + (lane % 32), K slice 8 * (lane / 32).
  const uint32_t am = lane & 31u, ah = lane >> 5;
  const int64_t aq = q0 + am;
  uint4 af[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const uint32_t c = (uint32_t)s * 2 + ah;
    af[s] = (aq < nq && c < nck) ? reinterpret_cast<const uint4*>(queries + (size_t)aq * dp)[c]
                                 : make_uint4(0, 0, 0, 0);
  }
  // the query rows of this lane's accumulators: m = 8g + 4*(lane/32) + j.
  // thd[r] is the distance of row r's current k-th key (+inf until known);
  // a score passes the cheap test d <= thd[r] and then the exact key test.
  float qs[16], thd[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t q = q0 + 8 * (r >> 2) + 4 * ah + (r & 3);
    qs[r] = (METRIC == kL2 && q < nq) ? qsq[q] : 0.0f;
    thd[r] = __builtin_inff();
  }

  // one 32-vector tile per step; the next tile's rows load while this one
  // is on the matrix cores
  uint4 nb[KS];
  auto load_step = [&](int64_t v0) {
    const int64_t v = v0 + am;
    const uint4* rv = reinterpret_cast<const uint4*>(base + (size_t)(v < v_end ? v : v_begin) * dp);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint32_t c = (uint32_t)s * 2 + ah;
      nb[s] = (v < v_end && c < nck) ? rv[c] : make_uint4(0, 0, 0, 0);
    }
  };
  if (v_begin < v_end) load_step(v_begin);

  for (int64_t v0 = v_begin; v0 < v_end; v0 += 32) {
    uint4 cb[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) cb[s] = nb[s];
    if (v0 + 32 < v_end) load_step(v0 + 32);
    float16v acc = {};
#pragma unroll
    for (int s = 0; s < KS; ++s)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(u4_as_h8(af[s]), u4_as_h8(cb[s]), acc, 0, 0, 0);
    // lane holds column n = lane % 32 (vector) and rows 8g + 4*(lane/32) + j
    const int64_t v = v0 + am;
    if (v < v_end) {
      const float vs = METRIC == kL2 ? vsq[v] : 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float d;
        if constexpr (METRIC == kL2) {
          d = __builtin_fmaf(-2.0f, acc[r], qs[r] + vs);  // == (qs + vs) - 2 dot: 2 dot is exact
        } else {
          d = -__half2float(__float2half_rn(acc[r]));
        }
        if (d <= thd[r]) {
          if constexpr (METRIC == kL2) d = d < 0.0f ? 0.0f : d;
          const uint32_t m = 8u * (r >> 2) + 4u * ah + (r & 3);
          const uint64_t key = bf_key(d, (uint32_t)v);
          if (key < thr[m]) {
            const uint32_t slot = atomicAdd(&cnt[m], 1u);
            cand[m * cap + slot] = key;
          }
        }
      }
    }
    wave_sync();
    // compact the buffers that could overflow in the next step (32 new keys at most)
    uint64_t full = ballot(lane < 32 && cnt[lane] > cap - kBfStep);
    if (full) {
      while (full) {
        const uint32_t m = (uint32_t)__builtin_ctzll(full);
        full &= full - 1;
        uint64_t kth;
        const uint32_t keep = bf_compact(cand + m * cap, cnt[m], k, scratch, &kth);
        if (lane == 0) {
          cnt[m] = keep;
          thr[m] = kth;
        }
        wave_sync();
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint64_t t = thr[8u * (r >> 2) + 4u * ah + (r & 3)];
        thd[r] = t == ~0ull ? __builtin_inff() : ord_to_dist((uint32_t)(t >> 32));
      }
    }
  }
  // final: best k of each query, sorted, padded with ~0
  for (uint32_t m = 0; m < 32; ++m) {
    const int64_t q = q0 + m;
    if (q >= nq) break;
    uint64_t kth;
    const uint32_t keep = bf_compact(cand + m * cap, cnt[m], k, scratch, &kth);
    uint64_t* dst = out + ((size_t)q * n_chunks + ci) * k;
    for (uint32_t i = lane; i < k; i += 64) dst[i] = i < keep ? cand[m * cap + i] : ~0ull;
    wave_sync();
  }
}

// Merge the n_chunks sorted lists of one query (one wave per query).
__global__ __launch_bounds__(64) void bf_merge_kernel(const uint64_t* __restrict__ lists, int64_t nq,
                                                      uint32_t n_chunks, uint32_t k, int32_t* __restrict__ out_ids,
                                                      float* __restrict__ out_d) {
  __shared__ uint64_t buf[256];
  const int64_t q = blockIdx.x;
  if (q >= nq) return;
  const uint32_t lane = threadIdx.x;
  const uint64_t* src = lists + (size_t)q * n_chunks * k;
  const size_t total = (size_t)n_chunks * k;
  // running best: buf[0, k) sorted; fill buf[k, 256) with the next keys
  for (uint32_t i = lane; i < 256; i += 64) buf[i] = ~0ull;
  wave_sync();
  const uint32_t room = 256 - k;
  for (size_t off = 0; off < total; off += room) {
    for (uint32_t i = lane; i < room; i += 64) buf[k + i] = off + i < total ? src[off + i] : ~0ull;
    wave_sync();
    lds_bitonic_sort(buf, 256);
  }
  for (uint32_t i = lane; i < k; i += 64) {
    const uint64_t key = buf[i];
    out_ids[(size_t)q * k + i] = key == ~0ull ? -1 : (int32_t)(uint32_t)key;
    out_d[(size_t)q * k + i] = key == ~0ull ? FLT_MAX : ord_to_dist((uint32_t)(key >> 32));
  }
}

void bruteforce_knn(const void* base, int64_t n, uint32_t dim, uint32_t dp, const void* queries, int64_t nq,
                    uint32_t k, int metric, int32_t* out_ids, float* out_d, hipStream_t s) {
  if (k == 0 || nq <= 0) return;
  if (k > (uint32_t)kBfMaxK) throw std::invalid_argument("bruteforce_knn supports k <= 64");
  if (dp % 8 != 0 || dp > 512) throw std::invalid_argument("bruteforce_knn supports padded dim <= 512");
  if (n <= 0) throw std::invalid_argument("empty base");
  if (n > 0x7FFFFFFFll) throw std::invalid_argument("too many base vectors");
  const uint32_t ks = (dp + 15) / 16;  // 16-wide K steps (the last may be half empty)
  float* vsq = nullptr;
  float* qsq = nullptr;
  if (metric == kL2) {
    hip_check(hipMallocAsync((void**)&vsq, (size_t)n * 4, s), "alloc base norms");
    hip_check(hipMallocAsync((void**)&qsq, (size_t)nq * 4, s), "alloc query norms");
    hipLaunchKernelGGL(row_sqnorm_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, s, (const uint16_t*)base,
                       n, dp, dim, vsq);
    hipLaunchKernelGGL(row_sqnorm_kernel, dim3((uint32_t)((nq + 255) / 256)), dim3(256), 0, s,
                       (const uint16_t*)queries, nq, dp, dim, qsq);
  }
  // chunks: about 8192 work-groups (single waves) in all, each chunk a
  // multiple of 64 vectors (a whole number of 32-vector steps)
  const int64_t qtiles = (nq + 31) / 32;
  int64_t want = std::max<int64_t>(1, 8192 / qtiles);
  want = std::min<int64_t>(want, (n + 63) / 64);
  int64_t chunk = ((n + want - 1) / want + 63) / 64 * 64;
  const uint32_t n_chunks = (uint32_t)((n + chunk - 1) / chunk);
  uint64_t* lists = nullptr;
  hip_check(hipMallocAsync((void**)&lists, (size_t)nq * n_chunks * k * 8, s), "alloc chunk lists");
  const dim3 grid((uint32_t)qtiles, n_chunks);
  const uint32_t cap = (k + kBfStep + 7u) & ~7u;
  const size_t lds = ((size_t)32 * cap + 128) * 8;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(64), lds, s, (const uint16_t*)base, n, dp, (const uint16_t*)queries, nq,
                       (const float*)vsq, (const float*)qsq, k, cap, chunk, n_chunks, lists);
  };
#define JA_BF_CASE(K)                                              \
  case K:                                                          \
    if (metric == kL2) go(bf_scan_kernel<K, kL2>);                 \
    else go(bf_scan_kernel<K, kIP>);                               \
    break;
  switch (ks) {
    JA_BF_CASE(1) JA_BF_CASE(2) JA_BF_CASE(3) JA_BF_CASE(4) JA_BF_CASE(5) JA_BF_CASE(6) JA_BF_CASE(7)
    JA_BF_CASE(8) JA_BF_CASE(9) JA_BF_CASE(10) JA_BF_CASE(11) JA_BF_CASE(12) JA_BF_CASE(13) JA_BF_CASE(14)
    JA_BF_CASE(15) JA_BF_CASE(16) JA_BF_CASE(17) JA_BF_CASE(18) JA_BF_CASE(19) JA_BF_CASE(20) JA_BF_CASE(21)
    JA_BF_CASE(22) JA_BF_CASE(23) JA_BF_CASE(24) JA_BF_CASE(25) JA_BF_CASE(26) JA_BF_CASE(27) JA_BF_CASE(28)
    JA_BF_CASE(29) JA_BF_CASE(30) JA_BF_CASE(31) JA_BF_CASE(32)
    default: throw std::invalid_argument("bruteforce_knn: unsupported dim");
  }
#undef JA_BF_CASE
  hip_check(hipGetLastError(), "launch bf_scan_kernel");
  hipLaunchKernelGGL(bf_merge_kernel, dim3((uint32_t)nq), dim3(64), 0, s, (const uint64_t*)lists, nq, n_chunks, k,
                     out_ids, out_d);
  hip_check(hipGetLastError(), "launch bf_merge_kernel");
  (void)hipFreeAsync(lists, s);
  if (vsq) (void)hipFreeAsync(vsq, s);
  if (qsq) (void)hipFreeAsync(qsq, s);
}

}  // namespace jasper_amd
