// diskann.hip -- the DiskANN build (reference index/construct_diskann.cuh,
// construct_diskann_kernels.cuh; driven by cmd/create_diskann_index.cu).
//
//   1. Shards by cross-polytope LSH (assign_shards, :104-276): each row,
//      centred on the sampled mean and rotated by the seed's orthogonal
//      matrix, goes to the shards of its n_dup largest |coordinates| (bucket
//      2 coord + sign, shard bucket mod n_parts). One wave per row: each
//      lane holds the centred coordinates lane, lane + 64, ... and
//      accumulates the rotated ones with the same indexes in fp32 (k
//      ascending, coordinate k broadcast by v_readlane, one fma per term;
//      cuBLAS's order in the reference is unspecified), and n_dup wave
//      max-reductions over the packed keys (|bits| << 16 | coord) pick the
//      ranks. The (shard, row) pairs are radix-sorted, which lists every
//      shard's rows in ascending order; shard sizes come from the run
//      boundaries.
//   2. Each shard, largest first, is gathered into a shard graph of degree
//      R_int and built with the plain construction (build_graph: batches
//      doubling to min(batch cap, shard size), search from its first row).
//   3. Distance-only merge (merge_row, :278-325), one wave per shard row:
//      the final row's entries and the shard row's (ids mapped to global),
//      the shard's duplicates of ids already in the final row dropped (the
//      same id carries the same stored distance: distances are symmetric
//      bit for bit), a 128-key bitonic sort by (distance, position), and the
//      first R_fin kept.
// The reference stages shards through host memory and merges on the CPU in
// a worker thread, one shard after another; here the whole graph stays in
// HBM and the merges run as kernels on the build stream in the same order.
#include "build.hpp"
#include "common.hpp"
#include "diskann.hpp"
#include "rotation.hpp"

#include <algorithm>
#include <numeric>
#include <vector>

namespace jasper_amd {

namespace {

constexpr uint32_t kMaxDup = 16;

__device__ __forceinline__ float h2f_bits(uint16_t b) { return __half2float(__ushort_as_half(b)); }

// binary64 -> binary16 bits, round to nearest even (one rounding).
__device__ uint16_t d2h_rn(double x) {
  const uint64_t b = (uint64_t)__double_as_longlong(x);
  const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
  const double a = fabs(x);
  if (a != a) return (uint16_t)(sign | 0x7E00u);
  if (a >= 65520.0) return (uint16_t)(sign | 0x7C00u);  // rounds to infinity
  if (a < 6.103515625e-05) {                            // below 2^-14: subnormal step 2^-24
    const double q = rint(a * 16777216.0);               // exact scaling, rint = RNE
    return (uint16_t)(sign | (uint16_t)q);
  }
  int e = 0;
  const double m = frexp(a, &e);  // a = m 2^e, m in [0.5, 1)
  double q = rint((m * 2.0 - 1.0) * 1024.0);
  int E = e - 1;
  if (q >= 1024.0) {
    q = 0.0;
    E += 1;
  }
  if (E + 15 >= 31) return (uint16_t)(sign | 0x7C00u);
  return (uint16_t)(sign | (uint16_t)((E + 15) << 10) | (uint16_t)q);
}

__global__ void mean_partial_kernel(const uint16_t* vecs, uint32_t dp, uint32_t dim, int64_t stride,
                                    int64_t sampled, int64_t per_block, double* partial) {
  const int64_t s0 = (int64_t)blockIdx.x * per_block;
  const int64_t s1 = min(sampled, s0 + per_block);
  for (uint32_t d = threadIdx.x; d < dim; d += blockDim.x) {
    double acc = 0.0;
    for (int64_t s = s0; s < s1; ++s) acc += (double)h2f_bits(vecs[(size_t)(s * stride) * dp + d]);
    partial[(size_t)blockIdx.x * dim + d] = acc;
  }
}

// One block per coordinate: the partial sums in any order (they are exact),
// a tree in LDS, one rounding to fp16.
__global__ __launch_bounds__(256) void mean_final_kernel(const double* partial, uint32_t blocks, uint32_t dim,
                                                         int64_t sampled, uint16_t* mean) {
  __shared__ double red[256];
  const uint32_t d = blockIdx.x;
  double acc = 0.0;
  for (uint32_t b = threadIdx.x; b < blocks; b += 256) acc += partial[(size_t)b * dim + d];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (uint32_t w = 128; w > 0; w >>= 1) {
    if (threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) mean[d] = d2h_rn(red[0] / (double)(sampled > 0 ? sampled : 1));
}

struct AssignArgs {
  const uint16_t* vecs;
  int64_t n;
  uint32_t dp, dim;
  const uint16_t* mean;  // [dim] fp16
  const float* pt;       // [dim][dim]: pt[k * dim + i] = fp16(P[k + i * dim]) as f32
  uint32_t n_parts, n_dup;
  uint32_t* shard_of;    // [n, n_dup]
  uint64_t* pairs;       // [n, n_dup]: shard << 32 | row, empty for repeats
};

// Shard sizes from the sorted pairs: each shard's run [start, end) is
// found at its boundaries (no atomics: one shard's counter would be hit by
// every row that lands in it).
__global__ void shard_bounds_kernel(const uint64_t* sorted, int64_t np, uint32_t* start, uint32_t* end) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= np) return;
  const uint64_t k = sorted[i];
  if (k == kEmptyKey) return;
  const uint32_t sh = (uint32_t)(k >> 32);
  if (i == 0 || (uint32_t)(sorted[i - 1] >> 32) != sh) start[sh] = (uint32_t)i;
  if (i + 1 == np || sorted[i + 1] == kEmptyKey || (uint32_t)(sorted[i + 1] >> 32) != sh) end[sh] = (uint32_t)(i + 1);
}

// Four waves per block, one row per wave at a time (grid-stride). The
// rotation (f32 values of the fp16 matrix, pt[k * dim + i]) is staged in LDS
// when it fits (dim <= 128: 64 KB); lane l owns output coordinates l, l + 64,
// ... and input coordinates likewise, and coordinate k of the centred row
// reaches every lane by v_readlane, k ascending.
constexpr uint32_t kAssignWaves = 4;

template <int T, bool LDS_P>
__global__ __launch_bounds__(64 * kAssignWaves) void assign_kernel(AssignArgs a) {
  extern __shared__ float pt_l[];
  const uint32_t lane = lane_id();
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t dim = a.dim;
  if constexpr (LDS_P) {
    for (uint32_t j = threadIdx.x; j < dim * dim; j += 64 * kAssignWaves) pt_l[j] = a.pt[j];
    __syncthreads();
  }
  const int64_t step = (int64_t)gridDim.x * kAssignWaves;
  for (int64_t row = (int64_t)blockIdx.x * kAssignWaves + wave; row < a.n; row += step) {
    const uint16_t* x = a.vecs + (size_t)row * a.dp;
    float c[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t k = lane + 64u * (uint32_t)t;
      // subtract_mean_kernel: v - mean in fp16, one rounding
      c[t] = k < dim ? (float)(_Float16)(__builtin_bit_cast(_Float16, x[k]) -
                                         __builtin_bit_cast(_Float16, a.mean[k]))
                     : 0.0f;
    }
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.0f;
#pragma unroll
    for (int tk = 0; tk < T; ++tk) {
      const uint32_t k0 = 64u * (uint32_t)tk;
      const uint32_t kend = dim > k0 ? min(64u, dim - k0) : 0u;
      for (uint32_t kk = 0; kk < kend; ++kk) {
        const float ck = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c[tk]), (int)kk));
        const size_t base = (size_t)(k0 + kk) * dim;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          const uint32_t i = lane + 64u * (uint32_t)t;
          float pk = 0.0f;
          if (i < dim) pk = LDS_P ? pt_l[base + i] : a.pt[base + i];
          acc[t] = __builtin_fmaf(pk, ck, acc[t]);
        }
      }
    }
    uint32_t rbits[T], key[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const uint32_t i = lane + 64u * (uint32_t)t;
      const _Float16 h = (_Float16)acc[t];
      rbits[t] = (uint32_t)__builtin_bit_cast(uint16_t, h);
      key[t] = i < dim ? (((rbits[t] & 0x7FFFu) << 16) | i) : 0u;
    }
    uint32_t prev[kMaxDup];
    for (uint32_t r = 0; r < a.n_dup; ++r) {
      uint32_t m = 0;
#pragma unroll
      for (int t = 0; t < T; ++t) m = max(m, key[t]);
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off, 64));
      const uint32_t win = uniform(m);
      const uint32_t coord = win & 0xFFFFu;
      const uint32_t owner = coord & 63u, slot = coord >> 6;
      uint32_t rb = 0;
#pragma unroll
      for (int t = 0; t < T; ++t)
        if ((uint32_t)t == slot) rb = rbits[t];
      const uint32_t sign = (uniform((uint32_t)__shfl((int)rb, (int)owner, 64)) >> 15) & 1u;
      const uint32_t shard = (2u * coord + sign) % a.n_parts;
      bool dup = false;
      for (uint32_t t = 0; t < r; ++t) dup = dup || prev[t] == shard;
      prev[r] = dup ? kInvalid32 : shard;
      if (lane == 0) {
        a.shard_of[(size_t)row * a.n_dup + r] = dup ? kInvalid32 : shard;
        a.pairs[(size_t)row * a.n_dup + r] = dup ? kEmptyKey : (((uint64_t)shard << 32) | (uint64_t)row);
      }
      if (lane == owner) {
#pragma unroll
        for (int t = 0; t < T; ++t)
          if ((uint32_t)t == slot) key[t] = 0u;
      }
    }
  }
}

// Shard rows from the graph: row i of the shard is graph row ids[i] (the low
// 32 bits of the sorted pairs).
__global__ void gather_rows_kernel(const uint4* src, const uint64_t* ids, int64_t count, uint32_t words, uint4* dst) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= count * words) return;
  const int64_t i = t / words, w = t % words;
  dst[t] = src[(size_t)(uint32_t)ids[i] * words + w];
}

struct MergeArgs {
  const uint64_t* ids;  // shard row -> global id (low 32 bits)
  int64_t count;
  const uint32_t* s_edges;
  const uint16_t* s_edist;
  const uint8_t* s_counts;
  uint32_t R_int;
  uint32_t* f_edges;
  uint16_t* f_edist;
  uint8_t* f_counts;
  uint32_t R_fin;
};

// Order of a bf16 distance as the float comparison sees it (-0 = +0).
__device__ __forceinline__ uint32_t bf16_order(uint32_t b) {
  if ((b & 0x7FFFu) == 0u) b = 0u;
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}

__global__ __launch_bounds__(64) void merge_rows_kernel(MergeArgs a) {
  __shared__ uint32_t ids_l[128];
  __shared__ uint16_t bits_l[128];
  const uint32_t lane = lane_id();
  for (int64_t i = blockIdx.x; i < a.count; i += gridDim.x) {
    const uint32_t gid = (uint32_t)a.ids[i];
    const uint32_t cf = uniform(a.f_counts[gid]);
    const uint32_t cs = uniform(a.s_counts[i]);
    const uint32_t el = min(lane, a.R_fin - 1u), sl = min(lane, a.R_int - 1u);
    const uint32_t e_id = a.f_edges[(size_t)gid * a.R_fin + el];
    const uint16_t e_bits = a.f_edist[(size_t)gid * a.R_fin + el];
    const uint32_t s_loc = a.s_edges[(size_t)i * a.R_int + sl];
    const uint16_t s_bits = a.s_edist[(size_t)i * a.R_int + sl];
    const bool ve = lane < cf && lane < a.R_fin && e_id != kInvalid32;
    bool vs = lane < cs && lane < a.R_int && s_loc != kInvalid32;
    const uint32_t s_id = vs ? (uint32_t)a.ids[s_loc] : kInvalid32;
    ids_l[lane] = ve ? e_id : kInvalid32;
    bits_l[lane] = e_bits;
    ids_l[64 + lane] = s_id;
    bits_l[64 + lane] = s_bits;
    wave_sync();
    // a shard entry whose id the final row holds already: the final row's
    // copy (same distance, earlier position) is the one kept
    for (uint32_t j = 0; j < cf && j < 64; ++j) vs = vs && ids_l[j] != s_id;
    uint64_t x0 = ve ? (((uint64_t)bf16_order(e_bits) << 32) | lane) : kEmptyKey;
    uint64_t x1 = vs ? (((uint64_t)bf16_order(s_bits) << 32) | (64u + lane)) : kEmptyKey;
    const uint32_t nv = (uint32_t)__builtin_popcountll(ballot(ve)) + (uint32_t)__builtin_popcountll(ballot(vs));
    wave_bitonic_sort128(x0, x1);
    const uint32_t keep = min(nv, a.R_fin);
    if (lane < keep) {
      const uint32_t pos = (uint32_t)x0 & 0xFFu;
      a.f_edges[(size_t)gid * a.R_fin + lane] = ids_l[pos];
      a.f_edist[(size_t)gid * a.R_fin + lane] = bits_l[pos];
    }
    if (lane == 0) a.f_counts[gid] = (uint8_t)keep;
    wave_sync();
  }
}

template <int T>
void launch_assign(const AssignArgs& a, hipStream_t s) {
  const uint32_t grid = (uint32_t)std::min<int64_t>((a.n + kAssignWaves - 1) / kAssignWaves, 2048);
  if ((size_t)a.dim * a.dim * 4 <= 64 * 1024) {
    auto k = assign_kernel<T, true>;
    hip_check(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024), "LDS");
    hipLaunchKernelGGL(k, dim3(grid), dim3(64 * kAssignWaves), (size_t)a.dim * a.dim * 4, s, a);
  } else {
    hipLaunchKernelGGL((assign_kernel<T, false>), dim3(grid), dim3(64 * kAssignWaves), 0, s, a);
  }
}

struct DeviceBuf {
  void* p = nullptr;
  explicit DeviceBuf(size_t bytes, const char* what) { hip_check(hipMalloc(&p, std::max<size_t>(bytes, 16)), what); }
  ~DeviceBuf() { (void)hipFree(p); }
  DeviceBuf(const DeviceBuf&) = delete;
  DeviceBuf& operator=(const DeviceBuf&) = delete;
  template <typename X>
  X* as() const { return static_cast<X*>(p); }
};

// Steps of assign_shards on the device rows of g. Leaves the sorted pairs in
// sorted[0, n * n_dup) and the shard sizes in counts_out.
void assign_device(const Graph& g, uint32_t n_parts, uint32_t n_dup, uint64_t seed, uint32_t* shard_of,
                   uint64_t* pairs, uint64_t* sorted, uint16_t* mean, std::vector<uint32_t>& counts_out,
                   hipStream_t s) {
  const int64_t n = g.n;
  const uint32_t dim = g.dim;
  // mean over rows 0, stride, 2 stride, ...
  const int64_t target = std::min<int64_t>(n, 2000000);
  const int64_t stride = std::max<int64_t>(1, n / target);
  const int64_t sampled = (n + stride - 1) / stride;
  const uint32_t blocks = (uint32_t)std::min<int64_t>(sampled, 4096);
  const int64_t per_block = (sampled + blocks - 1) / blocks;
  DeviceBuf partial((size_t)blocks * dim * 8, "alloc mean partials");
  hipLaunchKernelGGL(mean_partial_kernel, dim3(blocks), dim3(256), 0, s, (const uint16_t*)g.vecs, g.dp, dim, stride,
                     sampled, per_block, partial.as<double>());
  hip_check(hipGetLastError(), "launch mean_partial_kernel");
  hipLaunchKernelGGL(mean_final_kernel, dim3(dim), dim3(256), 0, s, partial.as<const double>(), blocks, dim, sampled,
                     mean);
  hip_check(hipGetLastError(), "launch mean_final_kernel");
  // the rotation matrix rounded to fp16, transposed for coalesced reads
  const std::vector<float> P = rotation_matrix(dim, seed);
  std::vector<float> pt((size_t)dim * dim);
  for (uint32_t i = 0; i < dim; ++i)
    for (uint32_t k = 0; k < dim; ++k) {
      const uint16_t h = f2h_rn(P[(size_t)k + (size_t)i * dim]);
      _Float16 hv;
      std::memcpy(&hv, &h, 2);
      pt[(size_t)k * dim + i] = (float)hv;
    }
  DeviceBuf dpt(pt.size() * 4, "alloc rotation");
  DeviceBuf bounds((size_t)n_parts * 8, "alloc shard bounds");
  hip_check(hipMemcpyAsync(dpt.p, pt.data(), pt.size() * 4, hipMemcpyHostToDevice, s), "upload rotation");
  hip_check(hipMemsetAsync(bounds.p, 0, (size_t)n_parts * 8, s), "clear shard bounds");
  AssignArgs a{};
  a.vecs = (const uint16_t*)g.vecs;
  a.n = n;
  a.dp = g.dp;
  a.dim = dim;
  a.mean = mean;
  a.pt = dpt.as<const float>();
  a.n_parts = n_parts;
  a.n_dup = n_dup;
  a.shard_of = shard_of;
  a.pairs = pairs;
  const uint32_t T = (dim + 63) / 64;
  if (T <= 1) launch_assign<1>(a, s);
  else if (T <= 2) launch_assign<2>(a, s);
  else if (T <= 4) launch_assign<4>(a, s);
  else if (T <= 8) launch_assign<8>(a, s);
  else if (T <= 16) launch_assign<16>(a, s);
  else throw std::invalid_argument("DiskANN shard assignment supports dim <= 1024");
  hip_check(hipGetLastError(), "launch assign_kernel");
  // group by shard, rows ascending within a shard
  const size_t np = (size_t)n * n_dup;
  // shard bits: an empty key's field (all ones) must not be a shard number
  int sbits = 1;
  while ((1u << sbits) <= n_parts) ++sbits;
  const size_t tb = sort_u64_temp_bytes(np);
  DeviceBuf temp(tb, "alloc sort temp");
  // pairs are written in row order: a stable sort of the shard bits keeps
  // each shard's rows ascending
  sort_u64(temp.p, tb, pairs, sorted, np, 32, 32 + sbits, s);
  uint32_t* start = bounds.as<uint32_t>();
  uint32_t* end = start + n_parts;
  hipLaunchKernelGGL(shard_bounds_kernel, dim3((uint32_t)((np + 255) / 256)), dim3(256), 0, s, sorted, (int64_t)np,
                     start, end);
  hip_check(hipGetLastError(), "launch shard_bounds_kernel");
  std::vector<uint32_t> be((size_t)n_parts * 2);
  hip_check(hipMemcpyAsync(be.data(), bounds.p, (size_t)n_parts * 8, hipMemcpyDeviceToHost, s), "read shard bounds");
  hip_check(hipStreamSynchronize(s), "shard assignment");
  counts_out.assign(n_parts, 0);
  uint64_t total = 0, expect = 0;
  for (uint32_t p = 0; p < n_parts; ++p) {
    counts_out[p] = be[(size_t)n_parts + p] - be[p];
    if (be[(size_t)n_parts + p] < be[p] || counts_out[p] > (uint64_t)n)
      throw std::logic_error("shard assignment: inconsistent shard runs");
    if (counts_out[p] && be[p] != expect) throw std::logic_error("shard assignment: shard runs out of order");
    expect += counts_out[p];
    total += counts_out[p];
  }
  if (total > np) throw std::logic_error("shard assignment: more shard rows than pairs");
}

void check_assign_args(const Graph& g, int64_t n_parts, int64_t n_dup) {
  if (g.n <= 0) throw std::invalid_argument("graph is empty");
  if (n_parts < 1 || n_parts > 0x7FFFFFFF) throw std::invalid_argument("n_parts must be positive");
  if (n_dup < 1 || n_dup > (int64_t)kMaxDup)
    throw std::invalid_argument("n_dup must be between 1 and " + std::to_string(kMaxDup));
  if (g.dim > 1024) throw std::invalid_argument("DiskANN shard assignment supports dim <= 1024");
}

}  // namespace

void diskann_assign(const Graph& g, int64_t n_parts, int64_t n_dup, uint64_t seed, uint32_t* shard_of_host,
                    uint16_t* mean_host, hipStream_t s) {
  check_assign_args(g, n_parts, n_dup);
  const size_t np = (size_t)g.n * n_dup;
  DeviceBuf shard_of(np * 4, "alloc shard ids");
  DeviceBuf pairs(np * 8, "alloc shard pairs");
  DeviceBuf sorted(np * 8, "alloc sorted shard pairs");
  DeviceBuf mean((size_t)g.dim * 2, "alloc mean");
  std::vector<uint32_t> counts;
  assign_device(g, (uint32_t)n_parts, (uint32_t)n_dup, seed, shard_of.as<uint32_t>(), pairs.as<uint64_t>(),
                sorted.as<uint64_t>(), mean.as<uint16_t>(), counts, s);
  if (shard_of_host)
    hip_check(hipMemcpy(shard_of_host, shard_of.p, np * 4, hipMemcpyDeviceToHost), "read shard ids");
  if (mean_host) hip_check(hipMemcpy(mean_host, mean.p, (size_t)g.dim * 2, hipMemcpyDeviceToHost), "read mean");
}

int64_t diskann_max_shard_for_device(uint32_t dim, uint32_t R_int, int64_t workspace_budget) {
  size_t free_b = 0, total_b = 0;
  hip_check(hipMemGetInfo(&free_b, &total_b), "device memory info");
  // a shard graph row: fp16 vector, R_int ids and bf16 distances, degree,
  // slot id, deletion bit, and its byte row when the rows qualify
  const size_t per_vec = (size_t)pad_dim(dim) * 2 + (size_t)R_int * 6 + 1 + 4 + 1 + dim;
  const size_t reserve = (size_t)std::max<int64_t>(workspace_budget, 0) + ((size_t)4 << 30);
  const size_t avail = free_b > reserve ? free_b - reserve : free_b / 2;
  return (int64_t)std::min<size_t>(std::max<size_t>(avail / per_vec, 1), 0x7FFFFFFF);
}

void build_diskann(Graph& g, uint32_t R_int, float alpha, int64_t n_parts, int64_t n_dup, uint64_t seed,
                   int64_t batch_cap, int64_t max_shard, hipStream_t s, DiskannStats* stats) {
  check_assign_args(g, n_parts, n_dup);
  if (R_int < 1 || R_int > 64) throw std::invalid_argument("R_int must be between 1 and 64");
  if (g.R > 64) throw std::invalid_argument("R must be <= 64");
  if (batch_cap < 1) batch_cap = 1;
  DiskannStats st;
  // events: 0 start, 1 shards assigned, 2 a shard's gather, 3 its build
  // done, 4 its merge done
  hipEvent_t e[5];
  for (hipEvent_t& x : e) hip_check(hipEventCreate(&x), "event");
  struct Events {
    hipEvent_t* e;
    ~Events() { for (int i = 0; i < 5; ++i) (void)hipEventDestroy(e[i]); }
  } ev{e};
  hip_check(hipEventRecord(e[0], s), "event record");

  const size_t np = (size_t)g.n * n_dup;
  DeviceBuf shard_of(np * 4, "alloc shard ids");
  DeviceBuf pairs(np * 8, "alloc shard pairs");
  DeviceBuf sorted(np * 8, "alloc sorted shard pairs");
  DeviceBuf mean((size_t)g.dim * 2, "alloc mean");
  std::vector<uint32_t> counts;
  assign_device(g, (uint32_t)n_parts, (uint32_t)n_dup, seed, shard_of.as<uint32_t>(), pairs.as<uint64_t>(),
                sorted.as<uint64_t>(), mean.as<uint16_t>(), counts, s);
  hip_check(hipEventRecord(e[1], s), "event record");

  // tasks: non-empty shards, each split into equal sub-shards of at most
  // max_shard rows (max_shard > 0); largest first, equal sizes by shard
  // index, then sub-shard
  std::vector<int64_t> offset((size_t)n_parts + 1, 0);
  for (int64_t p = 0; p < n_parts; ++p) offset[(size_t)p + 1] = offset[(size_t)p] + counts[(size_t)p];
  struct Task {
    int64_t begin, len;  // a run of the sorted (shard, row) pairs
  };
  std::vector<Task> tasks;
  for (int64_t p = 0; p < n_parts; ++p) {
    const int64_t total = counts[(size_t)p];
    if (total == 0) continue;
    const int64_t n_sub = max_shard > 0 ? (total + max_shard - 1) / max_shard : 1;
    const int64_t sub = (total + n_sub - 1) / n_sub;
    for (int64_t b = 0; b < total; b += sub) tasks.push_back({offset[(size_t)p] + b, std::min(sub, total - b)});
  }
  std::stable_sort(tasks.begin(), tasks.end(), [](const Task& a, const Task& b) { return a.len > b.len; });
  st.shards = (int64_t)tasks.size();
  int64_t max_count = 0;
  for (const Task& t : tasks) max_count = std::max<int64_t>(max_count, t.len);
  st.max_shard = max_count;

  Graph sg;
  sg.allocate(max_count, g.dim, R_int, g.metric, false);
  const uint32_t words = g.dp / 8;
  double build_ms = 0, merge_ms = 0;
  for (const Task& task : tasks) {
    const int64_t c = task.len;
    const uint64_t* ids = sorted.as<uint64_t>() + task.begin;
    hip_check(hipEventRecord(e[2], s), "event record");
    const int64_t threads = c * words;
    hipLaunchKernelGGL(gather_rows_kernel, dim3((uint32_t)((threads + 255) / 256)), dim3(256), 0, s,
                       (const uint4*)g.vecs, ids, c, words, (uint4*)sg.vecs);
    hip_check(hipGetLastError(), "launch gather_rows_kernel");
    hip_check(hipMemsetAsync(sg.counts, 0, (size_t)c, s), "clear shard degrees");
    sg.n = c;
    sg.medoid = 0;
    // the shard's values lie in the graph's recorded range
    sg.int_state = g.int_state;
    sg.int_lo = g.int_lo;
    sg.int_hi = g.int_hi;
    refresh_byte_rows(sg, c, s);  // the shard's byte rows, when the graph's rows qualify
    build_graph(sg, alpha, std::max<int64_t>(1, std::min<int64_t>(batch_cap, c)), s, false, nullptr);
    hip_check(hipEventRecord(e[3], s), "event record");
    MergeArgs m{};
    m.ids = ids;
    m.count = c;
    m.s_edges = sg.edges;
    m.s_edist = sg.edist;
    m.s_counts = sg.counts;
    m.R_int = R_int;
    m.f_edges = g.edges;
    m.f_edist = g.edist;
    m.f_counts = g.counts;
    m.R_fin = g.R;
    hipLaunchKernelGGL(merge_rows_kernel, dim3((uint32_t)std::min<int64_t>(c, 1 << 20)), dim3(64), 0, s, m);
    hip_check(hipGetLastError(), "launch merge_rows_kernel");
    hip_check(hipEventRecord(e[4], s), "event record");
    hip_check(hipEventSynchronize(e[4]), "diskann shard");
    float b = 0, mm = 0;
    hip_check(hipEventElapsedTime(&b, e[2], e[3]), "event elapsed");
    hip_check(hipEventElapsedTime(&mm, e[3], e[4]), "event elapsed");
    build_ms += b;
    merge_ms += mm;
  }
  hip_check(hipEventRecord(e[4], s), "event record");
  hip_check(hipStreamSynchronize(s), "diskann build");
  float assign = 0, total = 0;
  hip_check(hipEventElapsedTime(&assign, e[0], e[1]), "event elapsed");
  hip_check(hipEventElapsedTime(&total, e[0], e[4]), "event elapsed");
  st.assign_ms = assign;
  st.build_ms = build_ms;
  st.merge_ms = merge_ms;
  st.total_ms = total;
  g.medoid = 0;
  if (stats) *stats = st;
}

}  // namespace jasper_amd
