// bruteforce.hip -- exact k-NN by brute force on the matrix cores
// (the reference's ground-truth utility, python/jasper/__init__.py:828-926).
//
// Arithmetic as the reference computes it: L2 = (||q||^2 + ||v||^2) - 2 q.v in
// fp32, clamped at 0; IP = -(q.v) where the fp16 matmul's result is rounded to
// fp16 before the negation. q.v comes from v_mfma_f32_32x32x16_f16 (fp16
// products are exact in fp32, accumulation in fp32); the squared norms are
// fp32 sums in element order. Ties are ordered by (distance, id).
//
// One-pass path, used for bases under four samples (262,144 rows at k = 10),
// for rows longer than 512 values, for the threshold sample of the two-pass
// path and for queries that overflow it:
// bf_scan_kernel: one wave owns 32 queries and one chunk of the base. It
// holds the A fragments of its queries in registers and walks the chunk 32
// vectors at a time (one 32x32 output tile, K over the padded dim), loading
// the next 32 vectors while the current ones are on the matrix cores. A
// score enters a per-query candidate buffer in LDS only if it beats the
// query's current k-th best; a buffer that could overflow in the next step
// is compacted (sorted, cut to k), which also lowers the threshold. At the
// end each (query, chunk) writes its best k, sorted. bf_merge_kernel: one
// wave per query merges the chunk lists. Rows longer than 32 K steps (512
// values, config 4's 960) take the same kernel with the query and base
// fragments read per slice of 8 K steps.
// The two-pass path for large bases is described before bf_filter_kernel.
#include "bruteforce.hpp"
#include "common.hpp"
#include "graph.hpp"

#include <algorithm>
#include <cfloat>
#include <cstdlib>
#include <stdexcept>

namespace jasper_amd {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int kBfMaxK = 128;         // k the fused scan supports
constexpr int kBfStep = 32;          // vectors per step = most keys a query can gain per step
constexpr int kBfScratch = 256;      // compaction scratch: holds a full buffer (k + kBfStep <= 160)
constexpr uint32_t kBfMaxDp = 4096;  // longest padded row
constexpr int kBfSlice = 8;          // K steps per slice of the long-row scan (KS = 0)

__device__ uint4 kBfZeroChunk = {0u, 0u, 0u, 0u};  // never written

__device__ __forceinline__ half8 u4_as_h8(uint4 v) {
  half8 h;
  __builtin_memcpy(&h, &v, 16);
  return h;
}

// ||x||^2 per row, fp32 fma in element order. A block of 256 rows stages
// them 64 values at a time in LDS with coalesced loads (eight threads per
// 128-byte row segment), and each thread continues its own row's fma chain
// from there: the per-row order of the one-thread-per-row loop, with the
// memory access of a stream (the strided per-thread reads had run at about
// a sixth of the bandwidth). Row stride in LDS 136 bytes (34 words): at most
// two rows of a wave share a bank when they read the same column.
constexpr uint32_t kSqnRows = 256, kSqnChunk = 64, kSqnStride = kSqnChunk * 2 + 8;  // bytes
__global__ __launch_bounds__(kSqnRows) void row_sqnorm_kernel(const uint16_t* __restrict__ x, int64_t n,
                                                              uint32_t dp, uint32_t dim, float* __restrict__ out) {
  __shared__ __align__(16) uint8_t tile[kSqnRows * kSqnStride];  // 34,816 bytes
  const uint32_t t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * kSqnRows;
  const int64_t i = r0 + t;
  float s = 0.0f;
  for (uint32_t c0 = 0; c0 < dim; c0 += kSqnChunk) {
    // 256 rows x 8 segments of 16 bytes: each thread loads 8 of them
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k) {
      const uint32_t e = k * kSqnRows + t;    // segment index in the tile
      const uint32_t rr = e >> 3, seg = e & 7u;
      const int64_t row = r0 + rr;
      const uint32_t col = c0 + seg * 8u;   // first value of the segment
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (row < n && col < dp) v = *reinterpret_cast<const uint4*>(x + (size_t)row * dp + col);
      uint2* dst = reinterpret_cast<uint2*>(tile + rr * kSqnStride + seg * 16u);  // 8-byte aligned
      dst[0] = make_uint2(v.x, v.y);
      dst[1] = make_uint2(v.z, v.w);
    }
    __syncthreads();
    const uint8_t* mine = tile + t * kSqnStride;
#pragma unroll
    for (uint32_t j = 0; j < kSqnChunk; ++j) {
      if (c0 + j < dim) {
        _Float16 hv;
        __builtin_memcpy(&hv, mine + 2u * j, 2);
        const float f = (float)hv;
        s = __builtin_fmaf(f, f, s);
      }
    }
    __syncthreads();
  }
  if (i < n) out[i] = s;
}

// Sort key: order-preserving distance bits (high) and id (low).
__device__ __forceinline__ uint64_t bf_key(float d, uint32_t id) { return ((uint64_t)dist_to_ord(d) << 32) | id; }

// Compact one query's buffer through the wave's kBfScratch-entry scratch:
// sort the cnt (<= kBfScratch) keys, keep min(cnt, k) in buf; returns that
// count and the k-th key (~0 when fewer than k remain). Wave-wide.
__device__ uint32_t bf_compact(uint64_t* buf, uint32_t cnt, uint32_t k, uint64_t* scratch, uint64_t* kth) {
  const uint32_t lane = lane_id();
  if (cnt <= 64) {
    // one key per lane, sorted in registers
    uint64_t x = lane < cnt ? buf[lane] : ~0ull;
    x = wave_bitonic_sort<64>(x);
    const uint32_t keep = min(cnt, k);
    const uint64_t kk = (uint64_t)__shfl((long long)x, (int)(k - 1), 64);
    if (lane < keep) buf[lane] = x;
    *kth = keep == k ? kk : ~0ull;
    lds_wave_sync();
    return keep;
  }
  const uint32_t N = pow2_ceil(cnt);
  for (uint32_t i = lane; i < N; i += 64) scratch[i] = i < cnt ? buf[i] : ~0ull;
  wave_sync();
  lds_bitonic_sort(scratch, N);
  const uint32_t keep = min(cnt, k);
  for (uint32_t i = lane; i < keep; i += 64) buf[i] = scratch[i];
  *kth = keep == k ? scratch[k - 1] : ~0ull;
  wave_sync();
  return keep;
}

template <int KS, int METRIC>
__global__ __launch_bounds__(64) void bf_scan_kernel(const uint16_t* __restrict__ base, int64_t n, uint32_t dp,
                                                     const uint16_t* __restrict__ queries, int64_t nq,
                                                     const float* __restrict__ vsq, const float* __restrict__ qsq,
                                                     uint32_t k, uint32_t cap, int64_t chunk, uint32_t n_chunks,
                                                     uint64_t* __restrict__ out /* [nq][n_chunks][k] */,
                                                     const uint8_t* __restrict__ tile_flags) {
  // cap >= k + kBfStep (a multiple of 8): candidate slots per query.
  // KS = 0: rows longer than 32 K steps; the query and base fragments are
  // read per slice of kBfSlice steps instead of held in registers.
  extern __shared__ uint64_t bf_lds[];
  uint64_t* cand = bf_lds;                 // [32][cap]
  uint64_t* scratch = bf_lds + 32 * cap;   // [kBfScratch]
  __shared__ uint32_t cnt[32];
  __shared__ uint64_t thr[32];
  const uint32_t lane = threadIdx.x;
  const int64_t q0 = (int64_t)blockIdx.x * 32;
  const uint32_t ci = blockIdx.y;
  const int64_t v_begin = (int64_t)ci * chunk;
  const int64_t v_end = min(n, v_begin + chunk);
  const uint32_t nck = dp / 8;  // 16-byte chunks per row
  if (tile_flags && !tile_flags[blockIdx.x]) return;  // only the flagged query tiles

  if (lane < 32) {
    cnt[lane] = 0;
    thr[lane] = ~0ull;
  }
  wave_sync();

  // A fragments: lane holds query q0 + (lane % 32), K slice 8 * (lane / 32).
  const uint32_t am = lane & 31u, ah = lane >> 5;
  const int64_t aq = q0 + am;
  constexpr int KR = KS > 0 ? KS : 1;  // K steps held in registers
  uint4 af[KR];
  if constexpr (KS > 0) {
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint32_t c = (uint32_t)s * 2 + ah;
      af[s] = (aq < nq && c < nck) ? reinterpret_cast<const uint4*>(queries + (size_t)aq * dp)[c]
                                   : make_uint4(0, 0, 0, 0);
    }
  }
  // long rows: this lane's query row (a row of zeros past nq)
  const uint4* qrow = aq < nq ? reinterpret_cast<const uint4*>(queries + (size_t)aq * dp) : nullptr;
  const uint32_t nks = (dp + 15) / 16;  // K steps (the last may be half empty)
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

  // one 32-vector tile per step, double-buffered by hand so that a step's
  // MFMAs wait only for its own rows: the next tile's rows (and squared
  // norms) load while this one is on the matrix cores
  // a K slot past the row (dp % 16 == 8) reads the zero chunk: no per-lane
  // branch in the loop, and the product stays an exact 0 (the query side is
  // zero there too)
  auto load_step = [&](int64_t v0, uint4 (&nb)[KR], float& nvs) {
    const int64_t v = v0 + am;
    const int64_t vr = v < v_end ? v : v_begin;
    if constexpr (METRIC == kL2) nvs = vsq[vr];
    if constexpr (KS > 0) {
      const uint4* rv = reinterpret_cast<const uint4*>(base + (size_t)vr * dp);
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const uint32_t c = (uint32_t)s * 2 + ah;
        nb[s] = *(c < nck ? rv + c : &kBfZeroChunk);
      }
    }
  };
  auto step = [&](int64_t v0, const uint4 (&cb)[KR], float vs) {
    float16v acc = {};
    if constexpr (KS > 0) {
#pragma unroll
      for (int s = 0; s < KS; ++s)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(u4_as_h8(af[s]), u4_as_h8(cb[s]), acc, 0, 0, 0);
    } else {
      // K in slices: both fragments of a slice read together, then its
      // chain of kBfSlice matrix-core steps (the query rows stay in cache)
      const int64_t v = v0 + am;
      const uint4* rv = reinterpret_cast<const uint4*>(base + (size_t)(v < v_end ? v : v_begin) * dp);
      for (uint32_t s0 = 0; s0 < nks; s0 += kBfSlice) {
        uint4 a8[kBfSlice], b8[kBfSlice];
#pragma unroll
        for (int t = 0; t < kBfSlice; ++t) {
          const uint32_t c = (s0 + (uint32_t)t) * 2 + ah;
          a8[t] = qrow && c < nck ? qrow[c] : make_uint4(0u, 0u, 0u, 0u);
          b8[t] = *(c < nck ? rv + c : &kBfZeroChunk);
        }
#pragma unroll
        for (int t = 0; t < kBfSlice; ++t)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(u4_as_h8(a8[t]), u4_as_h8(b8[t]), acc, 0, 0, 0);
      }
    }
    // lane holds column n = lane % 32 (vector) and rows 8g + 4*(lane/32) + j
    const int64_t v = v0 + am;
    if (v < v_end) {
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
    lds_wave_sync();
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
        lds_wave_sync();
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint64_t t = thr[8u * (r >> 2) + 4u * ah + (r & 3)];
        thd[r] = t == ~0ull ? __builtin_inff() : ord_to_dist((uint32_t)(t >> 32));
      }
    }
  };
  // two tiles per iteration; tiles past v_end load a clamped row and add no
  // candidates (v < v_end fails), so the loop needs no mid-iteration exit
  uint4 ba[KR], bb[KR];
  float vsa = 0.0f, vsb = 0.0f;
  if (v_begin < v_end) load_step(v_begin, ba, vsa);
  for (int64_t v0 = v_begin; v0 < v_end; v0 += 64) {
    load_step(v0 + 32, bb, vsb);
    step(v0, ba, vsa);
    load_step(v0 + 64, ba, vsa);
    step(v0 + 32, bb, vsb);
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
                                                      float* __restrict__ out_d, const uint8_t* __restrict__ q_flags) {
  __shared__ uint64_t buf[256];
  const int64_t q = blockIdx.x;
  if (q >= nq) return;
  if (q_flags && !q_flags[q]) return;
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

// ----------------------------------------------------------- two-pass path
// For large bases the exact top-k is found in two passes over a GEMM:
//  1. the one-pass kernels above on a sample (the first rows of the base:
//     kBfSample, or more when k * n is large) give
//     each query the k-th smallest distance T_q of that sample. The true
//     k-th smallest over the whole base is <= T_q (the sample's k nearest are
//     k base rows), so every true neighbour has d <= T_q;
//  2. bf_filter_kernel computes every distance (same arithmetic) and appends
//     the keys with d <= T_q to a per-query list in HBM (about k * n / sample
//     entries per query), with no per-query state in the loop, so its
//     work-groups share one base tile in LDS across 256 (or 128) queries;
//  3. bf_select_kernel sorts each list by (distance, id) and writes the top k.
// A query whose list would exceed kBfCandCap is flagged and redone with the
// one-pass kernels (only its 32-query tile runs). Results are identical to
// the one-pass path: the same distances, the same (distance, id) order.
constexpr int64_t kBfSample = 65536;  // smallest sample (larger for large k * n)
constexpr uint32_t kBfCandCap = 1024;
constexpr uint32_t kBfLocal = 16;  // candidates a filter work-group stages per query before appending to HBM

// Appends a candidate key to query q's list (a rare path, kept out of line
// so that its address arithmetic does not occupy registers in the loop).
__device__ __noinline__ void bf_append(uint32_t* qcount, uint64_t* qcand, uint32_t q, uint64_t key) {
  const uint32_t slot = atomicAdd(&qcount[q], 1u);
  if (slot < kBfCandCap) qcand[(size_t)q * kBfCandCap + slot] = key;
}

// Cooperative base-tile staging of bf_filter_kernel: thread element i is
// (row srow[i], chunk scol[i]) of the ROWS-row tile starting at v0.
// (native vector registers: a uint4 struct copied under a condition stays in
// private memory)
// offb[i]: the element's byte offset in a whole tile (srow[i] * nck +
// scol[i] chunks), so a whole tile's loads add a per-thread constant to a
// uniform base and need no address arithmetic; the chunk's last, partial
// tile clamps its rows to the chunk.
template <int PER, int ROWS, int METRIC>
__device__ __forceinline__ void bf_gload(const uint4* base4, const float* vsq, int64_t v0, int64_t v_begin,
                                         int64_t v_end, uint32_t nck, uint32_t nel, uint32_t tid,
                                         const uint32_t (&srow)[PER], const uint32_t (&scol)[PER],
                                         const uint32_t (&offb)[PER], u32x4 (&stage)[PER], float& svs) {
  if (v0 + ROWS <= v_end) {
    const char* tb = reinterpret_cast<const char*>(base4 + (size_t)v0 * nck);
#pragma unroll
    for (int i = 0; i < PER; ++i) stage[i] = *reinterpret_cast<const u32x4*>(tb + offb[i]);
    if constexpr (METRIC == kL2) svs = vsq[v0 + (tid & (uint32_t)(ROWS - 1))];
    return;
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    // elements past the tile re-read chunk 0 of the first row and are not stored
    const bool in = tid + 256u * (uint32_t)i < nel;
    const int64_t vv = v0 + (in ? srow[i] : 0u);
    stage[i] = *reinterpret_cast<const u32x4*>(base4 + (size_t)(vv < v_end ? vv : v_begin) * nck + (in ? scol[i] : 0u));
  }
  if constexpr (METRIC == kL2) {
    const int64_t vv = v0 + (tid & (uint32_t)(ROWS - 1));
    svs = vsq[vv < v_end ? vv : v_begin];
  }
}

// The filter's cheap test reads ||v||^2 shrunk by 2^-20 (see bf_filter_kernel).
constexpr float kBfVsShrink = 1.0f - 0x1p-20f;

template <int PER, int ROWS>
__device__ __forceinline__ void bf_sstore(uint4* tile, float* tvs, uint32_t buf, uint32_t rs, uint32_t nel,
                                          uint32_t tid, const uint32_t (&srow)[PER], const uint32_t (&scol)[PER],
                                          const u32x4 (&stage)[PER], float svs) {
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (tid + 256u * (uint32_t)i < nel)
      *reinterpret_cast<u32x4*>(tile + buf * ROWS * rs + srow[i] * rs + scol[i]) = stage[i];
  if (tid < (uint32_t)ROWS) {
    tvs[buf * ROWS + tid] = svs;
    tvs[2 * ROWS + buf * ROWS + tid] = svs * kBfVsShrink;
  }
}

// TILES: 32-query tiles per wave; SUB: 32-row base tiles per step (one
// barrier per SUB tiles, SUB independent matrix-core chains per query tile).
// Two waves per SIMD up to 128 values per row (the pipelined loop's two
// accumulator sets then fit 256 registers: config 2, 1M x 128, 5.38 ms ->
// 4.98 ms against one wave); wider rows keep one (two spill: 1M x 256,
// 12.9 ms at one wave, 18.2 ms at two).
template <int KS, int TILES, int SUB, int METRIC>
__global__ __launch_bounds__(256, (KS <= 8 ? 2 : 1)) void bf_filter_kernel(const uint16_t* __restrict__ base, int64_t n, uint32_t dp,
                                                        const uint16_t* __restrict__ queries, int64_t nq,
                                                        const float* __restrict__ vsq, const float* __restrict__ qsq,
                                                        const float* __restrict__ qthr, uint32_t thr_stride,
                                                        int64_t chunk, uint32_t qblocks,
                                                        uint32_t* __restrict__ qcount,
                                                        uint64_t* __restrict__ qcand) {
  // XCD-aware work order: work-groups are dealt to the 8 XCDs round-robin
  // by id, so work-group p runs on XCD p % 8. Logical item L = (the items of
  // the XCDs before it) + p / 8, with query block L % qblocks and base chunk
  // L / qblocks: the query blocks of one chunk run on one XCD together and
  // read its base tiles through that XCD's L2 (dealt round-robin they would
  // fetch every tile into all eight L2s).
  const uint32_t G = gridDim.x, p = blockIdx.x, xcd = p & 7u, per = G >> 3, extra = G & 7u;
  const uint32_t L = xcd * per + min(xcd, extra) + (p >> 3);
  const uint32_t qblock = L % qblocks, cblock = L / qblocks;
  // LDS: two base tiles of ROWS rows, row stride nck + 1 chunks (the extra
  // chunk is zero: it is the K slot past the row when dp % 16 == 8, and it
  // staggers the rows across banks); two sets of ROWS squared norms (and
  // their shrunk copies); per wave and query tile the 32 query norms,
  // thresholds and cheap-test bounds.
  //
  // L2 scores first take a cheap conservative test: y = fl(2 q.v - vs')
  // >= c_q, with vs' = fl(||v||^2 (1 - 2^-20)) and c_q <= (||q||^2 - T_q) -
  // 2^-19 (||q||^2 + T_q). Whenever the exact score d = fl(fl(||q||^2 +
  // ||v||^2) - 2 q.v) satisfies d <= T_q (T_q >= 0), y passes: with u =
  // 2^-24 and |2 q.v| <= (||q||^2 + ||v||^2)(1 + 128u), d <= T_q gives
  // 2 q.v - ||v||^2 >= ||q||^2 - T_q - (||q||^2 + ||v||^2 + 2 T_q) u, and y
  // exceeds 2 q.v - ||v||^2 by at least 11.9 u ||v||^2 - 2.1 u ||q||^2. Only
  // a 32 x 32 block in which some lane's test passes computes the exact
  // scores and their appends; the others cost one fma and one compare per
  // score.
  constexpr int ROWS = 32 * SUB;
  extern __shared__ uint4 bf_tile[];
  const uint32_t nck = dp / 8, rs = nck + 1;
  float* tvs = reinterpret_cast<float*>(bf_tile + 2 * ROWS * rs);  // [2][ROWS] norms, then [2][ROWS] shrunk
  float* sqs = tvs + 4 * ROWS;         // [4 waves][TILES][32]
  float* sth = sqs + 4 * TILES * 32;   // [4 waves][TILES][32]
  float* scr = sth + 4 * TILES * 32;   // [4 waves][TILES][32] c_q of the cheap test
  // per wave and query row: a count and kBfLocal staged candidate keys
  // (wave-private; flushed to the query's HBM list once, at the end)
  uint32_t* lcnt = reinterpret_cast<uint32_t*>(scr + 4 * TILES * 32);  // [4 waves][TILES * 32]
  uint64_t* lbuf = reinterpret_cast<uint64_t*>(lcnt + 4 * TILES * 32); // [4 waves][TILES * 32][kBfLocal]
  const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63u, am = lane & 31u, ah = lane >> 5;
  const int64_t qbase = (int64_t)qblock * (128 * TILES) + (int64_t)w * (32 * TILES);
  for (uint32_t r = lane; r < 32u * TILES; r += 64) lcnt[w * TILES * 32 + r] = 0u;
  const int64_t v_begin = (int64_t)cblock * chunk;
  const int64_t v_end = min(n, v_begin + chunk);
  const uint4* base4 = reinterpret_cast<const uint4*>(base);

  for (uint32_t r = tid; r < 2u * ROWS; r += 256) bf_tile[(r / ROWS) * ROWS * rs + (r % ROWS) * rs + nck] =
      make_uint4(0, 0, 0, 0);
  uint4 af[TILES][KS];
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    const int64_t aq = qbase + 32 * t + am;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint32_t c = (uint32_t)s * 2 + ah;
      af[t][s] = (aq < nq && c < nck) ? reinterpret_cast<const uint4*>(queries + (size_t)aq * dp)[c]
                                      : make_uint4(0, 0, 0, 0);
    }
    if (ah == 0) {
      // a NaN threshold passes nothing (rows past the last query)
      const float qn = (METRIC == kL2 && aq < nq) ? qsq[aq] : 0.0f;
      const float th = aq < nq ? qthr[(size_t)aq * thr_stride] : __builtin_nanf("");
      sqs[(w * TILES + t) * 32 + am] = qn;
      sth[(w * TILES + t) * 32 + am] = th;
      // c_q in double, pushed below its own rounding to fp32
      const double c = ((double)qn - (double)th) - ((double)qn + fabs((double)th)) * 0x1p-19;
      scr[(w * TILES + t) * 32 + am] = (float)(c - fabs(c) * 0x1p-22);
    }
  }

  // cooperative tile loads: thread element i is (row srow[i], chunk scol[i])
  constexpr int kPer = (ROWS * 2 * KS + 255) / 256;
  const uint32_t nel = ROWS * nck;
  uint32_t srow[kPer], scol[kPer], offb[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const uint32_t e = tid + 256u * (uint32_t)i;
    srow[i] = e / nck;
    scol[i] = e % nck;
    offb[i] = e < nel ? e * 16u : 0u;  // srow * nck + scol chunks; past the tile: chunk 0 of the first row
  }
  // base tiles: tile i is in LDS buffer i % 2 while tile i + 1 waits in
  // registers and tile i + 2 is loading, so a load has two steps of work to
  // hide behind
  u32x4 sta[kPer], stb[kPer];
  float sva = 0.0f, svb = 0.0f;
  if (v_begin < v_end) {
    bf_gload<kPer, ROWS, METRIC>(base4, vsq, v_begin, v_begin, v_end, nck, nel, tid, srow, scol, offb, sta, sva);
    bf_sstore<kPer, ROWS>(bf_tile, tvs, 0u, rs, nel, tid, srow, scol, sta, sva);
    bf_gload<kPer, ROWS, METRIC>(base4, vsq, v_begin + ROWS, v_begin, v_end, nck, nel, tid, srow, scol, offb, stb, svb);
  }
  __syncthreads();
  // every load issued so far (query fragments, first tiles) completes here:
  // otherwise the loop's first MFMA waits for all outstanding loads on every
  // iteration, the prefetched tile included
  __builtin_amdgcn_s_waitcnt(0);
  // the cheap test's c_q of this lane's 16 rows per query tile (rows 8g +
  // 4ah + j), held in registers for the whole loop
  float cq[TILES][16];
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j) cq[t][4 * g + j] = scr[(w * TILES + t) * 32 + 8 * g + 4 * ah + j];
  // One tile's products: the chains of every (query tile, base sub-tile)
  // interleaved; each accumulates over s in order, as bf_scan_kernel does
  // (the distances must match it bit for bit). The tile's norms are taken
  // into registers with it, so its LDS buffer is free once the MFMAs are
  // issued.
  auto mma = [&](uint32_t buf, float16v (&accs)[TILES][SUB], float (&vs)[SUB], float (&vsm)[SUB]) {
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int u = 0; u < SUB; ++u) accs[t][u] = float16v{};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      uint4 b[SUB];
#pragma unroll
      for (int u = 0; u < SUB; ++u) b[u] = bf_tile[buf * ROWS * rs + (32u * u + am) * rs + (uint32_t)s * 2 + ah];
#pragma unroll
      for (int t = 0; t < TILES; ++t)
#pragma unroll
        for (int u = 0; u < SUB; ++u)
          accs[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(u4_as_h8(af[t][s]), u4_as_h8(b[u]), accs[t][u], 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < SUB; ++u) {
      vs[u] = tvs[buf * ROWS + 32u * u + am];
      vsm[u] = tvs[2 * ROWS + buf * ROWS + 32u * u + am];
    }
  };
  // One tile's tests and appends.
  auto epi = [&](int64_t v0, const float16v (&accs)[TILES][SUB], const float (&vs)[SUB], const float (&vsm)[SUB]) {
#pragma unroll
    for (int u = 0; u < SUB; ++u) {
      const int64_t v = v0 + 32 * u + am;
      const bool vok = v < v_end;
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        const float16v acc = accs[t][u];
        if constexpr (METRIC == kL2) {
          uint64_t any = 0;  // lanes with a passing score, one compare mask per score
#pragma unroll
          for (int i = 0; i < 16; ++i) any |= ballot(__builtin_fmaf(2.0f, acc[i], -vsm[u]) >= cq[t][i]);
          if (any == 0) continue;
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          // rows 8g + 4ah + j, j = 0..3
          const uint32_t row0 = 8u * (uint32_t)g + 4u * ah;
          const float4 q4 = *reinterpret_cast<const float4*>(sqs + (w * TILES + t) * 32 + row0);
          const float4 t4 = *reinterpret_cast<const float4*>(sth + (w * TILES + t) * 32 + row0);
          const float qsv[4] = {q4.x, q4.y, q4.z, q4.w}, thv[4] = {t4.x, t4.y, t4.z, t4.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float d;
            if constexpr (METRIC == kL2) d = __builtin_fmaf(-2.0f, acc[4 * g + j], qsv[j] + vs[u]);
            else d = -__half2float(__float2half_rn(acc[4 * g + j]));
            if (vok && d <= thv[j]) {
              if constexpr (METRIC == kL2) d = d < 0.0f ? 0.0f : d;
              // staged in LDS (an LDS atomic); a full stage appends to HBM
              const uint32_t r = (uint32_t)(32 * t + j) + row0;
              const uint64_t key = bf_key(d, (uint32_t)v);
              const uint32_t slot = atomicAdd(&lcnt[w * TILES * 32 + r], 1u);
              if (slot < kBfLocal) lbuf[(size_t)(w * TILES * 32 + r) * kBfLocal + slot] = key;
              else bf_append(qcount, qcand, (uint32_t)qbase + r, key);
            }
          }
        }
      }
    }
  };
  // Software pipeline over tiles of ROWS rows: tile i + 1's MFMAs are
  // issued before tile i's tests, so the matrix cores work while the VALU
  // runs the tests. Invariant at the loop head: tile v0's products are in
  // accA, tile v0 + ROWS is in LDS buffer 1 and tile v0 + 2 ROWS is loading
  // into sta. A tile's LDS buffer is overwritten only after the barrier
  // that follows its MFMAs' reads. Loads and stores are unconditional
  // inside the loop (rows past the chunk are clamped reads, stored but
  // never scored): with a conditional store the compiler cannot prove the
  // staging registers free at the loop head and waits there for every load
  // in flight, the prefetch included.
  float16v accA[TILES][SUB], accB[TILES][SUB];
  float vsA[SUB], vsmA[SUB], vsB[SUB], vsmB[SUB];
  if (v_begin < v_end) {
    mma(0u, accA, vsA, vsmA);
    bf_sstore<kPer, ROWS>(bf_tile, tvs, 1u, rs, nel, tid, srow, scol, stb, svb);
    bf_gload<kPer, ROWS, METRIC>(base4, vsq, v_begin + 2 * ROWS, v_begin, v_end, nck, nel, tid, srow, scol, offb, sta,
                                 sva);
  }
  __syncthreads();
  for (int64_t v0 = v_begin; v0 < v_end; v0 += 2 * ROWS) {
    const bool more1 = v0 + ROWS < v_end;
    if (more1) mma(1u, accB, vsB, vsmB);
    epi(v0, accA, vsA, vsmA);
    if (!more1) break;
    // tile v0 + 2 ROWS into buffer 0, tile v0 + 3 ROWS loads into stb
    bf_sstore<kPer, ROWS>(bf_tile, tvs, 0u, rs, nel, tid, srow, scol, sta, sva);
    bf_gload<kPer, ROWS, METRIC>(base4, vsq, v0 + 3 * ROWS, v_begin, v_end, nck, nel, tid, srow, scol, offb, stb, svb);
    __syncthreads();
    const bool more2 = v0 + 2 * ROWS < v_end;
    if (more2) mma(0u, accA, vsA, vsmA);
    epi(v0 + ROWS, accB, vsB, vsmB);
    if (!more2) break;
    // tile v0 + 3 ROWS into buffer 1, tile v0 + 4 ROWS loads into sta
    bf_sstore<kPer, ROWS>(bf_tile, tvs, 1u, rs, nel, tid, srow, scol, stb, svb);
    bf_gload<kPer, ROWS, METRIC>(base4, vsq, v0 + 4 * ROWS, v_begin, v_end, nck, nel, tid, srow, scol, offb, sta, sva);
    __syncthreads();
  }
  // flush the staged candidates: one HBM slot reservation per query row
  lds_wave_sync();
  for (uint32_t r = lane; r < 32u * TILES; r += 64) {
    const int64_t q = qbase + r;
    const uint32_t c = min(lcnt[w * TILES * 32 + r], kBfLocal);
    if (q >= nq || c == 0) continue;
    const uint32_t at = atomicAdd(&qcount[q], c);
    for (uint32_t i = 0; i < c && at + i < kBfCandCap; ++i)
      qcand[(size_t)q * kBfCandCap + at + i] = lbuf[(size_t)(w * TILES * 32 + r) * kBfLocal + i];
  }
}

// Per query: sort the candidate list by (distance, id) and write the best k;
// a list that overflowed flags the query (and its 32-query tile) for the
// one-pass kernels.
__global__ __launch_bounds__(64) void bf_select_kernel(const uint32_t* __restrict__ qcount,
                                                       const uint64_t* __restrict__ qcand, int64_t nq, uint32_t k,
                                                       int32_t* __restrict__ out_ids, float* __restrict__ out_d,
                                                       uint8_t* __restrict__ q_flags, uint8_t* __restrict__ tile_flags) {
  __shared__ uint64_t buf[kBfCandCap];
  const int64_t q = blockIdx.x;
  const uint32_t lane = threadIdx.x;
  const uint32_t cnt = qcount[q];
  if (cnt > kBfCandCap) {
    if (lane == 0) {
      q_flags[q] = 1;
      tile_flags[q >> 5] = 1;
    }
    return;
  }
  const uint32_t N = max(pow2_ceil(cnt), 2u);
  const uint64_t* src = qcand + (size_t)q * kBfCandCap;
  for (uint32_t i = lane; i < N; i += 64) buf[i] = i < cnt ? src[i] : ~0ull;
  wave_sync();
  lds_bitonic_sort(buf, N);
  for (uint32_t i = lane; i < k; i += 64) {
    const uint64_t key = i < N ? buf[i] : ~0ull;
    out_ids[(size_t)q * k + i] = key == ~0ull ? -1 : (int32_t)(uint32_t)key;
    out_d[(size_t)q * k + i] = key == ~0ull ? FLT_MAX : ord_to_dist((uint32_t)(key >> 32));
  }
}

// The one-pass path (scan + merge) over base rows [0, n), for all queries or
// only the flagged ones.
static void bf_one_pass(const void* base, int64_t n, uint32_t dp, const void* queries, int64_t nq, uint32_t k,
                        int metric, const float* vsq, const float* qsq, int32_t* out_ids, float* out_d,
                        const uint8_t* tile_flags, const uint8_t* q_flags, hipStream_t s) {
  const uint32_t ks = (dp + 15) / 16;  // 16-wide K steps (the last may be half empty)
  // chunks: each a multiple of 64 vectors (a whole number of 32-vector steps)
  // about 2,048 work-groups (single waves): longer chunks spend fewer of
  // their steps filling and compacting the buffers before the threshold
  // settles (config 2's 65,536-row sample: 8,192 work-groups 6.24 ms per
  // ground-truth call, 4,096 5.62, 2,048 5.44, 1,024 5.77);
  // JASPER_BF_SCAN_WGS overrides it (tuning)
  const int64_t qtiles = (nq + 31) / 32;
  static const int64_t target = [] {
    const char* e = std::getenv("JASPER_BF_SCAN_WGS");
    return e ? std::max<int64_t>(1, std::atoll(e)) : 2048;
  }();
  int64_t want = std::max<int64_t>(1, target / qtiles);
  want = std::min<int64_t>(want, (n + 63) / 64);
  int64_t chunk = ((n + want - 1) / want + 63) / 64 * 64;
  const uint32_t n_chunks = (uint32_t)((n + chunk - 1) / chunk);
  uint64_t* lists = nullptr;
  hip_check(hipMallocAsync((void**)&lists, (size_t)nq * n_chunks * k * 8, s), "alloc chunk lists");
  const dim3 grid((uint32_t)qtiles, n_chunks);
  // at least 64 slots: a buffer is compacted (a 64-key register sort, then
  // every row's threshold reloaded) once it holds more than cap - kBfStep
  // keys, so at k = 10 the 48 slots of k + kBfStep compacted each query
  // after every 6 or so new candidates; 64 allow 22 between compactions
  // and keep all of config 2's 1,878 work-groups resident (18.4 KB of LDS
  // each): its 65,536-row sample scan 0.90 -> 0.77 ms
  const uint32_t cap = std::max<uint32_t>((k + kBfStep + 7u) & ~7u, 64u);
  const size_t lds = ((size_t)32 * cap + kBfScratch) * 8;
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(64), lds, s, (const uint16_t*)base, n, dp, (const uint16_t*)queries, nq,
                       vsq, qsq, k, cap, chunk, n_chunks, lists, tile_flags);
  };
#define JA_BF_CASE(K)                                              \
  case K:                                                          \
    if (metric == kL2) go(bf_scan_kernel<K, kL2>);                 \
    else go(bf_scan_kernel<K, kIP>);                               \
    break;
  switch (ks > 32 ? 0u : ks) {
    JA_BF_CASE(0)
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
                     out_ids, out_d, q_flags);
  hip_check(hipGetLastError(), "launch bf_merge_kernel");
  (void)hipFreeAsync(lists, s);
}

template <int KS, int SUB, int METRIC>
static void launch_filter_sub(const void* base, int64_t n, uint32_t dp, const void* queries, int64_t nq,
                              const float* vsq, const float* qsq, const float* qthr, uint32_t thr_stride,
                              uint32_t* qcount, uint64_t* qcand, hipStream_t s) {
  // one 32-query tile per wave: two (208 VGPRs) and three (272) measured
  // 7.48 and 11.7 ms against 7.15 ms on config 2's 10k x 1M ground truth
  constexpr int TILES = 1;
  const int64_t qblocks = (nq + 128 * TILES - 1) / (128 * TILES);
  // about 2,500 work-groups in a 1-D grid that the kernel maps to (query
  // block, chunk) so that one chunk's query blocks share an XCD
  int64_t want = std::max<int64_t>(1, 2560 / qblocks);
  want = std::min<int64_t>(want, (n + 31) / 32);
  const int64_t chunk = ((n + want - 1) / want + 31) / 32 * 32;
  const uint32_t n_chunks = (uint32_t)((n + chunk - 1) / chunk);
  const uint32_t rs = dp / 8 + 1;
  const size_t lds = (size_t)2 * 32 * SUB * rs * 16 + 4 * 32 * SUB * 4 + (size_t)3 * 4 * TILES * 32 * 4 +
                     (size_t)4 * TILES * 32 * (4 + 8 * kBfLocal);
  auto kern = bf_filter_kernel<KS, TILES, SUB, METRIC>;
  if (lds > 64 * 1024)
    hip_check(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds), "LDS");
  hipLaunchKernelGGL(kern, dim3((uint32_t)qblocks * n_chunks), dim3(256), lds, s, (const uint16_t*)base, n, dp,
                     (const uint16_t*)queries, nq, vsq, qsq, qthr, thr_stride, chunk, (uint32_t)qblocks, qcount,
                     qcand);
  hip_check(hipGetLastError(), "launch bf_filter_kernel");
}

template <int KS, int METRIC>
static void launch_filter(const void* base, int64_t n, uint32_t dp, const void* queries, int64_t nq,
                          const float* vsq, const float* qsq, const float* qthr, uint32_t thr_stride,
                          uint32_t* qcount, uint64_t* qcand, hipStream_t s) {
  // 64-row steps (two 32-row tiles, two chains per wave): 6.25 ms against
  // 6.73 ms with 32-row steps on config 2's ground truth; JASPER_BF_SUB=1
  // selects the latter (tuning)
  static const int sub = [] {
    const char* e = std::getenv("JASPER_BF_SUB");
    return e ? std::atoi(e) : 2;
  }();
  if (sub == 1 || KS > 16)
    launch_filter_sub<KS, 1, METRIC>(base, n, dp, queries, nq, vsq, qsq, qthr, thr_stride, qcount, qcand, s);
  else
    launch_filter_sub<KS, 2, METRIC>(base, n, dp, queries, nq, vsq, qsq, qthr, thr_stride, qcount, qcand, s);
}

template <int METRIC>
static void dispatch_filter(uint32_t ks, const void* base, int64_t n, uint32_t dp, const void* queries, int64_t nq,
                            const float* vsq, const float* qsq, const float* qthr, uint32_t thr_stride,
                            uint32_t* qcount, uint64_t* qcand, hipStream_t s) {
  switch (ks) {
#define JA_F(K) \
  case K: launch_filter<K, METRIC>(base, n, dp, queries, nq, vsq, qsq, qthr, thr_stride, qcount, qcand, s); break;
    JA_F(1) JA_F(2) JA_F(3) JA_F(4) JA_F(5) JA_F(6) JA_F(7) JA_F(8) JA_F(9) JA_F(10) JA_F(11) JA_F(12) JA_F(13)
    JA_F(14) JA_F(15) JA_F(16) JA_F(17) JA_F(18) JA_F(19) JA_F(20) JA_F(21) JA_F(22) JA_F(23) JA_F(24) JA_F(25)
    JA_F(26) JA_F(27) JA_F(28) JA_F(29) JA_F(30) JA_F(31) JA_F(32)
#undef JA_F
    default: throw std::invalid_argument("bruteforce_knn: unsupported dim");
  }
}

void bruteforce_knn(const void* base, int64_t n, uint32_t dim, uint32_t dp, const void* queries, int64_t nq,
                    uint32_t k, int metric, int32_t* out_ids, float* out_d, hipStream_t s) {
  if (k == 0 || nq <= 0) return;
  if (k > (uint32_t)kBfMaxK) throw std::invalid_argument("bruteforce_knn supports k <= 128");
  if (dp % 8 != 0 || dp > kBfMaxDp) throw std::invalid_argument("bruteforce_knn supports padded dim <= 4096");
  if (n <= 0) throw std::invalid_argument("empty base");
  if (n > 0x7FFFFFFFll) throw std::invalid_argument("too many base vectors");
  if (nq > 0x7FFFFFFFll) throw std::invalid_argument("too many queries");
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
  // the two-pass path: rows of up to 32 K steps (512 values), and a sample
  // large enough that a query's filtered list (about k * n / sample keys)
  // stays near half of kBfCandCap
  const int64_t sample = std::max<int64_t>(kBfSample, ((int64_t)2 * k * n / kBfCandCap + 63) / 64 * 64);
  if (n < 4 * sample || dp > 512) {
    bf_one_pass(base, n, dp, queries, nq, k, metric, vsq, qsq, out_ids, out_d, nullptr, nullptr, s);
  } else {
    // 1. thresholds from the sample rows [0, sample)
    int32_t* sid = nullptr;
    float* sd = nullptr;
    uint32_t* qcount = nullptr;
    uint64_t* qcand = nullptr;
    uint8_t* flags = nullptr;  // [nq] query flags, then [ceil(nq / 32)] tile flags
    const int64_t ntiles = (nq + 31) / 32;
    hip_check(hipMallocAsync((void**)&sid, (size_t)nq * k * 4, s), "alloc sample ids");
    hip_check(hipMallocAsync((void**)&sd, (size_t)nq * k * 4, s), "alloc sample dists");
    hip_check(hipMallocAsync((void**)&qcount, (size_t)nq * 4, s), "alloc candidate counts");
    hip_check(hipMallocAsync((void**)&qcand, (size_t)nq * kBfCandCap * 8, s), "alloc candidate lists");
    hip_check(hipMallocAsync((void**)&flags, (size_t)(nq + ntiles), s), "alloc overflow flags");
    hip_check(hipMemsetAsync(qcount, 0, (size_t)nq * 4, s), "clear candidate counts");
    hip_check(hipMemsetAsync(flags, 0, (size_t)(nq + ntiles), s), "clear overflow flags");
    bf_one_pass(base, sample, dp, queries, nq, k, metric, vsq, qsq, sid, sd, nullptr, nullptr, s);
    // 2. every distance against the thresholds (the k-th sample distance)
    const uint32_t ks = (dp + 15) / 16;
    if (metric == kL2) dispatch_filter<kL2>(ks, base, n, dp, queries, nq, vsq, qsq, sd + (k - 1), k, qcount, qcand, s);
    else dispatch_filter<kIP>(ks, base, n, dp, queries, nq, vsq, qsq, sd + (k - 1), k, qcount, qcand, s);
    // 3. select, and redo overflowed queries in one pass
    hipLaunchKernelGGL(bf_select_kernel, dim3((uint32_t)nq), dim3(64), 0, s, (const uint32_t*)qcount,
                       (const uint64_t*)qcand, nq, k, out_ids, out_d, flags, flags + nq);
    hip_check(hipGetLastError(), "launch bf_select_kernel");
    bf_one_pass(base, n, dp, queries, nq, k, metric, vsq, qsq, out_ids, out_d, flags + nq, flags, s);
    (void)hipFreeAsync(sid, s);
    (void)hipFreeAsync(sd, s);
    (void)hipFreeAsync(qcount, s);
    (void)hipFreeAsync(qcand, s);
    (void)hipFreeAsync(flags, s);
  }
  if (vsq) (void)hipFreeAsync(vsq, s);
  if (qsq) (void)hipFreeAsync(qsq, s);
}

}  // namespace jasper_amd
