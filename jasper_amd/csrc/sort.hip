// sort.hip -- stable LSD radix sort of u64 keys and an exclusive scan of u64
// counts: the reverse-edge grouping of the build, the repair grouping of
// consolidate and the shard grouping of the DiskANN build.
//
// The reference groups reverse edges with thrust::sort by source
// (index/construct.cuh:846-879). Here the pairs are packed as (target <<
// shift | source) and sorted as integers over bits [begin_bit, end_bit),
// eight bits per pass. Every pass is stable, so a caller whose pairs are
// already in source order sorts the target bits only and still gets the
// sources of each target ascending -- the deterministic arrival order the
// reverse merge relies on.
//
// One pass over n keys in tiles of 4,096 (a work-group of four waves, 16
// keys per lane; wave w of a tile holds keys [w * 1024, (w + 1) * 1024) in
// lane-fastest order, so every load is one coalesced 512-byte read):
//   1. count   -- each work-group counts the digits of its contiguous run of
//                 tiles (at most 2,048 work-groups);
//   2. scan    -- one work-group per digit turns its row of per-group counts
//                 into exclusive offsets and the digit's total;
//   3. scatter -- each work-group ranks a tile's keys stably (lanes with the
//                 same digit found by one ballot per digit bit; per-wave
//                 running counts in LDS), places the tile in LDS in digit
//                 order and writes each digit's run to consecutive
//                 addresses.
// Inputs of at most one tile are sorted by one work-group in LDS over all
// passes. Nothing spins or waits on another work-group.
#include <algorithm>
#include <cstdlib>
#include <stdexcept>

#include "build.hpp"
#include "common.hpp"

namespace jasper_amd {
namespace {

constexpr uint32_t kSortThreads = 256;  // four waves
constexpr uint32_t kSortWaves = kSortThreads / 64;
constexpr uint32_t kSortJ = 16;  // keys per lane per tile
constexpr uint32_t kSortTile = kSortThreads * kSortJ;
constexpr uint32_t kWaveKeys = 64 * kSortJ;
constexpr uint32_t kBins = 256;
constexpr uint32_t kMaxGroups = 2048;
constexpr uint32_t kScanJ = 16;  // u64 counts per thread per scan tile
constexpr uint32_t kScanTile = kSortThreads * kScanJ;
constexpr uint32_t kMaxScanGroups = 1024;
static_assert(kBins == kSortThreads, "one digit per thread");
static_assert(kMaxGroups % kSortThreads == 0, "scan rows split evenly");

struct PassArgs {
  const uint64_t* src;
  uint64_t* dst;
  uint32_t n;
  uint32_t shift;
  uint32_t nbits;   // digit bits of this pass, 1..8
  uint32_t tiles;   // ceil(n / kSortTile)
  uint32_t groups;  // work-groups of the count and scatter kernels
  uint32_t* counts;  // [kBins][groups]: counts, then exclusive offsets within a digit
  uint32_t* totals;  // [kBins]
};

__device__ __forceinline__ uint64_t lanes_below() {
  const uint32_t l = lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// tiles of work-group b: [b * tiles / groups, (b + 1) * tiles / groups)
__device__ __forceinline__ void group_range(uint32_t b, uint32_t tiles, uint32_t groups, uint32_t& t0,
                                            uint32_t& t1) {
  t0 = (uint32_t)((uint64_t)b * tiles / groups);
  t1 = (uint32_t)((uint64_t)(b + 1) * tiles / groups);
}

// the lanes of `live` whose digit equals this lane's (nbits uniform)
__device__ __forceinline__ uint64_t digit_peers(uint32_t d, uint32_t nbits, uint64_t live) {
  uint64_t m = live;
#pragma unroll
  for (uint32_t i = 0; i < 8; ++i) {
    if (i < nbits) {
      const bool bit = (d >> i) & 1u;
      const uint64_t b = ballot(bit);
      m &= bit ? b : ~b;
    }
  }
  return m;
}

// exclusive prefix of v over the work-group's threads in thread order, and
// the sum over all of them
template <typename T>
__device__ __forceinline__ T group_exclusive_scan(T v, T& total) {
  __shared__ T wsum[kSortWaves];
  const uint32_t lane = lane_id(), w = threadIdx.x >> 6;
  T x = v;
#pragma unroll
  for (uint32_t o = 1; o < 64; o <<= 1) {
    const T y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  T before = 0, all = 0;
#pragma unroll
  for (uint32_t k = 0; k < kSortWaves; ++k) {
    const T s = wsum[k];
    if (k < w) before += s;
    all += s;
  }
  __syncthreads();
  total = all;
  return before + x - v;
}

// Stable ranks of a wave's kSortJ x 64 keys: r[j] = earlier keys of the wave
// with the same digit. wc (this wave's row) ends holding the wave's counts.
__device__ __forceinline__ void rank_wave(const uint64_t (&k)[kSortJ], uint32_t (&r)[kSortJ], uint32_t base,
                                          uint32_t n, uint32_t shift, uint32_t nbits, uint32_t* wc) {
  const uint32_t lane = lane_id(), mask = (1u << nbits) - 1u;
  const uint64_t below = lanes_below();
#pragma unroll
  for (uint32_t j = 0; j < kSortJ; ++j) {
    const bool ok = base + j * 64 + lane < n;
    const uint64_t live = ballot(ok);
    const uint32_t d = (uint32_t)(k[j] >> shift) & mask;
    const uint64_t m = digit_peers(d, nbits, live);
    const uint32_t c = ok ? wc[d] : 0u;
    if (ok && (m & below) == 0) wc[d] = c + (uint32_t)__popcll(m);
    r[j] = c + (uint32_t)__popcll(m & below);
  }
}

// After rank_wave by every wave: wc[w][d] becomes the count of digit d in
// earlier waves, and the return value (thread d) is the tile's count of d.
__device__ __forceinline__ uint32_t wave_prefix(uint32_t (*wc)[kBins]) {
  const uint32_t d = threadIdx.x;
  uint32_t run = 0;
#pragma unroll
  for (uint32_t w = 0; w < kSortWaves; ++w) {
    const uint32_t c = wc[w][d];
    wc[w][d] = run;
    run += c;
  }
  return run;
}

__global__ __launch_bounds__(kSortThreads) void radix_count_kernel(PassArgs a) {
  __shared__ uint32_t wc[kSortWaves][kBins];
  const uint32_t tid = threadIdx.x, w = tid >> 6, lane = lane_id();
#pragma unroll
  for (uint32_t k = 0; k < kSortWaves; ++k) wc[k][tid] = 0;
  __syncthreads();
  const uint32_t mask = (1u << a.nbits) - 1u;
  const uint64_t below = lanes_below();
  uint32_t t0, t1;
  group_range(blockIdx.x, a.tiles, a.groups, t0, t1);
  for (uint32_t t = t0; t < t1; ++t) {
    const uint32_t base = t * kSortTile + w * kWaveKeys;
    uint64_t k[kSortJ];
#pragma unroll
    for (uint32_t j = 0; j < kSortJ; ++j) {
      const uint32_t i = base + j * 64 + lane;
      k[j] = i < a.n ? a.src[i] : 0ull;
    }
#pragma unroll
    for (uint32_t j = 0; j < kSortJ; ++j) {
      const bool ok = base + j * 64 + lane < a.n;
      const uint64_t live = ballot(ok);
      const uint32_t d = (uint32_t)(k[j] >> a.shift) & mask;
      const uint64_t m = digit_peers(d, a.nbits, live);
      if (ok && (m & below) == 0) wc[w][d] += (uint32_t)__popcll(m);
    }
  }
  __syncthreads();
  uint32_t s = 0;
#pragma unroll
  for (uint32_t k = 0; k < kSortWaves; ++k) s += wc[k][tid];
  a.counts[(size_t)tid * a.groups + blockIdx.x] = s;
}

// work-group d: row d of the counts to exclusive offsets, totals[d]
__global__ __launch_bounds__(kSortThreads) void radix_scan_kernel(PassArgs a) {
  constexpr uint32_t E = kMaxGroups / kSortThreads;
  uint32_t* row = a.counts + (size_t)blockIdx.x * a.groups;
  const uint32_t tid = threadIdx.x;
  uint32_t v[E], s = 0;
#pragma unroll
  for (uint32_t e = 0; e < E; ++e) {
    const uint32_t i = tid * E + e;
    v[e] = i < a.groups ? row[i] : 0u;
    s += v[e];
  }
  uint32_t total;
  uint32_t run = group_exclusive_scan<uint32_t>(s, total);
#pragma unroll
  for (uint32_t e = 0; e < E; ++e) {
    const uint32_t i = tid * E + e;
    if (i < a.groups) row[i] = run;
    run += v[e];
  }
  if (tid == 0) a.totals[blockIdx.x] = total;
}

__global__ __launch_bounds__(kSortThreads) void radix_scatter_kernel(PassArgs a) {
  __shared__ uint64_t stage[kSortTile];
  __shared__ uint32_t wc[kSortWaves][kBins];
  __shared__ uint32_t lstart[kBins];
  __shared__ uint32_t goff[kBins];
  const uint32_t tid = threadIdx.x, w = tid >> 6, lane = lane_id();
  const uint32_t mask = (1u << a.nbits) - 1u;
  uint32_t all;
  // thread tid owns digit tid: where this work-group's keys of it start
  uint32_t off = group_exclusive_scan<uint32_t>(a.totals[tid], all) + a.counts[(size_t)tid * a.groups + blockIdx.x];
  uint32_t t0, t1;
  group_range(blockIdx.x, a.tiles, a.groups, t0, t1);
  for (uint32_t t = t0; t < t1; ++t) {
#pragma unroll
    for (uint32_t k = 0; k < kSortWaves; ++k) wc[k][tid] = 0;
    goff[tid] = off;
    __syncthreads();
    const uint32_t base = t * kSortTile + w * kWaveKeys;
    uint64_t k[kSortJ];
    uint32_t r[kSortJ];
#pragma unroll
    for (uint32_t j = 0; j < kSortJ; ++j) {
      const uint32_t i = base + j * 64 + lane;
      k[j] = i < a.n ? a.src[i] : 0ull;
    }
    rank_wave(k, r, base, a.n, a.shift, a.nbits, wc[w]);
    __syncthreads();
    const uint32_t tile_count = wave_prefix(wc);
    uint32_t tile_all;
    lstart[tid] = group_exclusive_scan<uint32_t>(tile_count, tile_all);
    __syncthreads();
#pragma unroll
    for (uint32_t j = 0; j < kSortJ; ++j) {
      if (base + j * 64 + lane < a.n) {
        const uint32_t d = (uint32_t)(k[j] >> a.shift) & mask;
        stage[lstart[d] + wc[w][d] + r[j]] = k[j];
      }
    }
    __syncthreads();
    const uint32_t cnt = min(kSortTile, a.n - t * kSortTile);
    for (uint32_t i = tid; i < cnt; i += kSortThreads) {
      const uint64_t key = stage[i];
      const uint32_t d = (uint32_t)(key >> a.shift) & mask;
      const uint32_t pos = goff[d] + (i - lstart[d]);
      if (pos < a.n) a.dst[pos] = key;  // always true when the counts agree
    }
    off += tile_count;
    __syncthreads();
  }
}

// n <= kSortTile: every pass in LDS by one work-group
__global__ __launch_bounds__(kSortThreads) void radix_small_kernel(const uint64_t* in, uint64_t* out, uint32_t n,
                                                                   uint32_t begin_bit, uint32_t end_bit) {
  __shared__ uint64_t stage[kSortTile];
  __shared__ uint32_t wc[kSortWaves][kBins];
  __shared__ uint32_t lstart[kBins];
  const uint32_t tid = threadIdx.x, w = tid >> 6, lane = lane_id();
  const uint32_t base = w * kWaveKeys;
  uint64_t k[kSortJ];
  uint32_t r[kSortJ];
#pragma unroll
  for (uint32_t j = 0; j < kSortJ; ++j) {
    const uint32_t i = base + j * 64 + lane;
    k[j] = i < n ? in[i] : 0ull;
  }
  for (uint32_t shift = begin_bit; shift < end_bit; shift += 8) {
    const uint32_t nbits = min(8u, end_bit - shift), mask = (1u << nbits) - 1u;
#pragma unroll
    for (uint32_t q = 0; q < kSortWaves; ++q) wc[q][tid] = 0;
    __syncthreads();
    rank_wave(k, r, base, n, shift, nbits, wc[w]);
    __syncthreads();
    const uint32_t tile_count = wave_prefix(wc);
    uint32_t tile_all;
    lstart[tid] = group_exclusive_scan<uint32_t>(tile_count, tile_all);
    __syncthreads();
#pragma unroll
    for (uint32_t j = 0; j < kSortJ; ++j) {
      if (base + j * 64 + lane < n) {
        const uint32_t d = (uint32_t)(k[j] >> shift) & mask;
        stage[lstart[d] + wc[w][d] + r[j]] = k[j];
      }
    }
    __syncthreads();
#pragma unroll
    for (uint32_t j = 0; j < kSortJ; ++j) {
      const uint32_t i = base + j * 64 + lane;
      k[j] = i < n ? stage[i] : 0ull;
    }
    __syncthreads();
  }
#pragma unroll
  for (uint32_t j = 0; j < kSortJ; ++j) {
    const uint32_t i = base + j * 64 + lane;
    if (i < n) out[i] = k[j];
  }
}

// ---- exclusive scan of u64 counts

__global__ __launch_bounds__(kSortThreads) void scan_reduce_kernel(const uint64_t* in, uint64_t n, uint32_t tiles,
                                                                   uint32_t groups, uint64_t* partial) {
  uint32_t t0, t1;
  group_range(blockIdx.x, tiles, groups, t0, t1);
  const uint64_t lo = (uint64_t)t0 * kScanTile, hi = std::min<uint64_t>(n, (uint64_t)t1 * kScanTile);
  uint64_t s = 0;
  for (uint64_t i = lo + threadIdx.x; i < hi; i += kSortThreads) s += in[i];
  uint64_t total;
  (void)group_exclusive_scan<uint64_t>(s, total);
  if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

__global__ __launch_bounds__(kSortThreads) void scan_down_kernel(const uint64_t* in, uint64_t* out, uint64_t n,
                                                                 uint32_t tiles, uint32_t groups,
                                                                 const uint64_t* partial) {
  uint64_t s = 0;
  for (uint32_t i = threadIdx.x; i < blockIdx.x; i += kSortThreads) s += partial[i];
  uint64_t carry;
  (void)group_exclusive_scan<uint64_t>(s, carry);
  uint32_t t0, t1;
  group_range(blockIdx.x, tiles, groups, t0, t1);
  for (uint32_t t = t0; t < t1; ++t) {
    const uint64_t lo = (uint64_t)t * kScanTile + (uint64_t)threadIdx.x * kScanJ;
    uint64_t v[kScanJ], sum = 0;
#pragma unroll
    for (uint32_t e = 0; e < kScanJ; ++e) {
      v[e] = lo + e < n ? in[lo + e] : 0ull;
      sum += v[e];
    }
    uint64_t tile_total;
    uint64_t run = carry + group_exclusive_scan<uint64_t>(sum, tile_total);
#pragma unroll
    for (uint32_t e = 0; e < kScanJ; ++e) {
      if (lo + e < n) out[lo + e] = run;
      run += v[e];
    }
    carry += tile_total;
  }
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// work-groups of a pass: one per tile up to kMaxGroups. JASPER_SORT_GROUPS
// lowers the cap (read on every call; tests use it to give each work-group
// several tiles at small sizes).
uint32_t sort_groups(uint32_t tiles) {
  uint32_t cap = kMaxGroups;
  if (const char* e = std::getenv("JASPER_SORT_GROUPS")) {
    const long v = std::atol(e);
    if (v >= 1 && v < (long)kMaxGroups) cap = (uint32_t)v;
  }
  return std::min(tiles, cap);
}

}  // namespace

size_t sort_u64_temp_bytes(size_t max_items) {
  return align256(max_items * 8) + align256((size_t)kBins * kMaxGroups * 4) + align256((size_t)kBins * 4);
}

void sort_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, size_t n, int begin_bit,
              int end_bit, hipStream_t stream) {
  if (n == 0) return;
  if (begin_bit < 0 || end_bit > 64 || begin_bit > end_bit) throw std::invalid_argument("radix sort: bad bit range");
  if (n > (size_t)0xFFFFFFFFu - kSortTile) throw std::invalid_argument("radix sort: more than 2^32 - 4097 keys");
  if (in == out) throw std::invalid_argument("radix sort: input and output must differ");
  const uint32_t n32 = (uint32_t)n;
  if (n32 <= kSortTile) {
    hipLaunchKernelGGL(radix_small_kernel, dim3(1), dim3(kSortThreads), 0, stream, in, out, n32, (uint32_t)begin_bit,
                       (uint32_t)end_bit);
    hip_check(hipGetLastError(), "launch radix_small_kernel");
    return;
  }
  const uint32_t passes = (uint32_t)(end_bit - begin_bit + 7) / 8;
  if (passes == 0) {
    hip_check(hipMemcpyAsync(out, in, n * 8, hipMemcpyDeviceToDevice, stream), "radix sort copy");
    return;
  }
  if (temp_bytes < sort_u64_temp_bytes(n)) throw std::invalid_argument("radix sort: temporary storage too small");
  char* p = (char*)temp;
  uint64_t* tmp = (uint64_t*)p;
  p += align256(n * 8);
  uint32_t* counts = (uint32_t*)p;
  p += align256((size_t)kBins * kMaxGroups * 4);
  uint32_t* totals = (uint32_t*)p;
  PassArgs a{};
  a.n = n32;
  a.tiles = (n32 + kSortTile - 1) / kSortTile;
  a.groups = sort_groups(a.tiles);
  a.counts = counts;
  a.totals = totals;
  const uint64_t* src = in;
  for (uint32_t q = 0; q < passes; ++q) {
    uint64_t* dst = (passes - 1 - q) % 2 == 0 ? out : tmp;  // the last pass writes out
    a.src = src;
    a.dst = dst;
    a.shift = (uint32_t)begin_bit + 8 * q;
    a.nbits = std::min<uint32_t>(8, (uint32_t)end_bit - a.shift);
    hipLaunchKernelGGL(radix_count_kernel, dim3(a.groups), dim3(kSortThreads), 0, stream, a);
    hip_check(hipGetLastError(), "launch radix_count_kernel");
    hipLaunchKernelGGL(radix_scan_kernel, dim3(kBins), dim3(kSortThreads), 0, stream, a);
    hip_check(hipGetLastError(), "launch radix_scan_kernel");
    hipLaunchKernelGGL(radix_scatter_kernel, dim3(a.groups), dim3(kSortThreads), 0, stream, a);
    hip_check(hipGetLastError(), "launch radix_scatter_kernel");
    src = dst;
  }
}

size_t scan_u64_temp_bytes(size_t /*max_items*/) { return (size_t)kMaxScanGroups * 8; }

void exclusive_scan_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, size_t n,
                        hipStream_t stream) {
  if (n == 0) return;
  if (temp_bytes < scan_u64_temp_bytes(n)) throw std::invalid_argument("scan: temporary storage too small");
  if (n > ((size_t)1 << 40)) throw std::invalid_argument("scan: too many items");
  const uint32_t tiles = (uint32_t)((n + kScanTile - 1) / kScanTile);
  const uint32_t groups = std::min(tiles, kMaxScanGroups);
  uint64_t* partial = (uint64_t*)temp;
  hipLaunchKernelGGL(scan_reduce_kernel, dim3(groups), dim3(kSortThreads), 0, stream, in, (uint64_t)n, tiles, groups,
                     partial);
  hip_check(hipGetLastError(), "launch scan_reduce_kernel");
  hipLaunchKernelGGL(scan_down_kernel, dim3(groups), dim3(kSortThreads), 0, stream, in, out, (uint64_t)n, tiles,
                     groups, (const uint64_t*)partial);
  hip_check(hipGetLastError(), "launch scan_down_kernel");
}

}  // namespace jasper_amd
