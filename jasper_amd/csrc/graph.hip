// graph.hip -- allocation, host transfer and the on-disk format.
//
// The base file layout is the reference's current format
// (include/jasper/index/graph.cuh:1653-1788):
//   u64 total_file_size | u64 N | u64 medoid | u64 bytes_per_node
//   N records: fp16[dim] | u8 edge_count | u32 edges[R] | bf16 dist[R] | u32 slot_to_id
//   ceil(N/8) bytes of deletion bits (bit g&7 of byte g>>3 is slot g)
//   u64 next_id
// and the loader accepts the three older per-node layouts the reference
// loader accepts (graph.cuh:1460-1479).
#include "graph.hpp"
#include "directional.hpp"

#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>

namespace jasper_amd {

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    (void)hipGetLastError();
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
  }
}

static void* alloc_bytes(size_t bytes, bool on_host, const char* what) {
  if (bytes == 0) bytes = 16;
  void* p = nullptr;
  if (on_host) {
    // pinned host memory that kernels read in place: its device address must
    // be the host address, since the graph keeps one pointer for both
    hip_check(hipHostMalloc(&p, bytes, hipHostMallocMapped | hipHostMallocPortable), what);
    void* dp = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&dp, p, 0);
    if (e != hipSuccess || dp != p) {
      (void)hipHostFree(p);
      throw std::runtime_error(std::string(what) + ": host memory is not addressable by the device at its host address");
    }
  } else {
    hip_check(hipMalloc(&p, bytes), what);
  }
  return p;
}

static void free_bytes(void* p, bool on_host) {
  if (!p) return;
  if (on_host) (void)hipHostFree(p);
  else (void)hipFree(p);
}

Graph::Graph() = default;
Graph::~Graph() { release(); }

void Graph::allocate(int64_t n_, uint32_t dim_, uint32_t R_, int metric_, bool on_host_) {
  release();
  int_state = 0;
  n = n_;
  dim = dim_;
  dp = pad_dim(dim_);
  R = R_;
  metric = metric_;
  on_host = on_host_;
  medoid = 0;
  next_id = (uint64_t)n_;
  n_deleted = 0;
  const size_t nn = (size_t)std::max<int64_t>(n_, 1);
  capacity = (int64_t)nn;
  try {
    vecs = alloc_bytes(nn * dp * 2, on_host, "alloc vectors");
    edges = (uint32_t*)alloc_bytes(nn * R * 4, on_host, "alloc edges");
    edist = (uint16_t*)alloc_bytes(nn * R * 2, on_host, "alloc edge distances");
    counts = (uint8_t*)alloc_bytes(nn, on_host, "alloc edge counts");
    deleted = (uint32_t*)alloc_bytes(((nn + 31) / 32) * 4, on_host, "alloc deletion bits");
    slot_to_id = (uint32_t*)alloc_bytes(nn * 4, on_host, "alloc slot ids");
  } catch (...) {
    release();
    throw;
  }
  if (on_host) {
    std::memset(vecs, 0, nn * dp * 2);
    std::memset(edges, 0xFF, nn * R * 4);
    std::memset(edist, 0, nn * R * 2);
    std::memset(counts, 0, nn);
    std::memset(deleted, 0, ((nn + 31) / 32) * 4);
    for (size_t i = 0; i < nn; ++i) slot_to_id[i] = (uint32_t)i;
  } else {
    hip_check(hipMemset(vecs, 0, nn * dp * 2), "memset vectors");
    hip_check(hipMemset(edges, 0xFF, nn * R * 4), "memset edges");
    hip_check(hipMemset(edist, 0, nn * R * 2), "memset edge distances");
    hip_check(hipMemset(counts, 0, nn), "memset counts");
    hip_check(hipMemset(deleted, 0, ((nn + 31) / 32) * 4), "memset deletion bits");
    std::vector<uint32_t> ids(nn);
    for (size_t i = 0; i < nn; ++i) ids[i] = (uint32_t)i;
    hip_check(hipMemcpy(slot_to_id, ids.data(), nn * 4, hipMemcpyHostToDevice), "init slot ids");
  }
}

void Graph::reserve(int64_t rows, hipStream_t stream) {
  if (rows <= capacity) return;
  if (on_host) throw std::runtime_error("growing a graph requires it on the device");
  const size_t oc = (size_t)capacity, nc = (size_t)rows;
  const size_t ow = (oc + 31) / 32, nw = (nc + 31) / 32;
  void* v2 = nullptr;
  uint32_t *e2 = nullptr, *d2 = nullptr, *s2 = nullptr;
  uint16_t* w2 = nullptr;
  uint8_t* c2 = nullptr;
  try {
    v2 = alloc_bytes(nc * dp * 2, false, "grow vectors");
    e2 = (uint32_t*)alloc_bytes(nc * R * 4, false, "grow edges");
    w2 = (uint16_t*)alloc_bytes(nc * R * 2, false, "grow edge distances");
    c2 = (uint8_t*)alloc_bytes(nc, false, "grow edge counts");
    d2 = (uint32_t*)alloc_bytes(nw * 4, false, "grow deletion bits");
    s2 = (uint32_t*)alloc_bytes(nc * 4, false, "grow slot ids");
    hip_check(hipMemcpyAsync(v2, vecs, oc * dp * 2, hipMemcpyDeviceToDevice, stream), "copy vectors");
    hip_check(hipMemsetAsync((char*)v2 + oc * dp * 2, 0, (nc - oc) * dp * 2, stream), "clear vectors");
    hip_check(hipMemcpyAsync(e2, edges, oc * R * 4, hipMemcpyDeviceToDevice, stream), "copy edges");
    hip_check(hipMemsetAsync(e2 + oc * R, 0xFF, (nc - oc) * R * 4, stream), "clear edges");
    hip_check(hipMemcpyAsync(w2, edist, oc * R * 2, hipMemcpyDeviceToDevice, stream), "copy edge distances");
    hip_check(hipMemsetAsync(w2 + oc * R, 0, (nc - oc) * R * 2, stream), "clear edge distances");
    hip_check(hipMemcpyAsync(c2, counts, oc, hipMemcpyDeviceToDevice, stream), "copy edge counts");
    hip_check(hipMemsetAsync(c2 + oc, 0, nc - oc, stream), "clear edge counts");
    hip_check(hipMemcpyAsync(d2, deleted, ow * 4, hipMemcpyDeviceToDevice, stream), "copy deletion bits");
    hip_check(hipMemsetAsync(d2 + ow, 0, (nw - ow) * 4, stream), "clear deletion bits");
    hip_check(hipMemcpyAsync(s2, slot_to_id, oc * 4, hipMemcpyDeviceToDevice, stream), "copy slot ids");
    hip_check(hipMemsetAsync(s2 + oc, 0xFF, (nc - oc) * 4, stream), "clear slot ids");
    hip_check(hipStreamSynchronize(stream), "grow graph");
  } catch (...) {
    free_bytes(v2, false);
    free_bytes(e2, false);
    free_bytes(w2, false);
    free_bytes(c2, false);
    free_bytes(d2, false);
    free_bytes(s2, false);
    throw;
  }
  free_bytes(vecs, false);
  free_bytes(edges, false);
  free_bytes(edist, false);
  free_bytes(counts, false);
  free_bytes(deleted, false);
  free_bytes(slot_to_id, false);
  vecs = v2;
  edges = e2;
  edist = w2;
  counts = c2;
  deleted = d2;
  slot_to_id = s2;
  capacity = rows;
}

void Graph::release() {
  free_bytes(vecs, on_host);
  free_bytes(edges, on_host);
  free_bytes(edist, on_host);
  free_bytes(counts, on_host);
  free_bytes(deleted, on_host);
  free_bytes(slot_to_id, on_host);
  vecs = nullptr;
  edges = nullptr;
  edist = nullptr;
  counts = nullptr;
  deleted = nullptr;
  slot_to_id = nullptr;
  if (vecs8) (void)hipFree(vecs8);
  vecs8 = nullptr;
  vecs8_cap = 0;
  rotation.reset();
  if (vector_norms) (void)hipFree(vector_norms);
  vector_norms = nullptr;
  lsh.reset();
  pq.reset();
  rabitq.reset();
}

// out = {non-integer flag, min, max} over fp16 values (infinities and NaN
// count as non-integer); count8 = values / 8, read as 16-byte chunks
__global__ void int_range_kernel(const uint4* __restrict__ v, size_t count8, int32_t* __restrict__ out) {
  float lo = 65504.0f, hi = -65504.0f;
  bool bad = false;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count8; i += (size_t)gridDim.x * blockDim.x) {
    const uint4 c = v[i];
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      _Float16 hv;
      const uint16_t bits = (uint16_t)(w[k >> 1] >> (16 * (k & 1)));
      __builtin_memcpy(&hv, &bits, 2);
      const float h = (float)hv;
      bad = bad || !(fabsf(h) <= 65504.0f) || h != rintf(h);
      const float hc = fminf(fmaxf(h, -65504.0f), 65504.0f);  // NaN -> -65504
      lo = fminf(lo, hc);
      hi = fmaxf(hi, hc);
    }
  }
  for (int d = 32; d > 0; d >>= 1) {
    lo = fminf(lo, __shfl_xor(lo, d, 64));
    hi = fmaxf(hi, __shfl_xor(hi, d, 64));
  }
  const bool any_bad = __ballot(bad) != 0;
  // one set of atomics per block (each on one of three words: the launch's
  // thousands of waves contending for them had cost more than the scan)
  __shared__ float s_lo[4], s_hi[4];
  __shared__ int s_bad[4];
  const uint32_t wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63u) == 0) {
    s_lo[wv] = lo;
    s_hi[wv] = hi;
    s_bad[wv] = any_bad ? 1 : 0;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t nw = blockDim.x >> 6;
    for (uint32_t i = 1; i < nw; ++i) {
      lo = fminf(lo, s_lo[i]);
      hi = fmaxf(hi, s_hi[i]);
    }
    int b = 0;
    for (uint32_t i = 0; i < nw; ++i) b |= s_bad[i];
    if (b) atomicMax(&out[0], 1);
    atomicMin(&out[1], (int32_t)lo);
    atomicMax(&out[2], (int32_t)hi);
  }
}

int32_t int_exact_span(uint32_t dim) {
  int32_t S = 2048;
  while (S > 0 && (double)dim * (double)S * (double)S >= 16777216.0) --S;
  return S;
}

static bool int_exact_enabled() {
  static const bool enabled = [] {
    const char* e = std::getenv("JASPER_INT_EXACT");
    return !(e && std::atoi(e) == 0);
  }();
  return enabled;
}

// rows [row0, row0 + rows) to bytes: value - lo, one thread per 8 values
__global__ void byte_rows_kernel(const uint4* __restrict__ vecs, uint32_t dp8, uint32_t dim8, int64_t row0,
                                 int64_t rows, int32_t lo, uint2* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= rows * (int64_t)dim8) return;
  const int64_t r = row0 + t / dim8;
  const uint32_t c = (uint32_t)(t % dim8);
  const uint4 v = vecs[(size_t)r * dp8 + c];
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t b[2] = {0u, 0u};
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    _Float16 hv;
    const uint16_t bits = (uint16_t)(w[k >> 1] >> (16 * (k & 1)));
    __builtin_memcpy(&hv, &bits, 2);
    const int32_t x = (int32_t)(float)hv;  // an integer in [lo, lo + 255]
    b[k >> 2] |= (uint32_t)(x - lo) << (8 * (k & 3));
  }
  out[(size_t)r * dim8 + c] = make_uint2(b[0], b[1]);
}

static bool byte_rows_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("JASPER_SEARCH_BYTES");
    return !(e && std::atoi(e) == 0);
  }();
  return on;
}

// an integer s is an fp16 value when |s| <= 2048, or |s| <= 65504 and s is
// a multiple of the fp16 spacing at |s|
static bool fp16_integer(int64_t s) {
  const int64_t m = s < 0 ? -s : s;
  if (m <= 2048) return true;
  if (m > 65504) return false;
  int64_t spacing = 1;
  while ((int64_t)2048 * spacing <= m) spacing *= 2;
  return m % spacing == 0;
}

bool byte_rows_eligible(const Graph& g) {
  if (!byte_rows_enabled() || g.on_host || g.metric != 0 || g.int_state != 1) return false;
  if ((int64_t)g.int_hi - (int64_t)g.int_lo > 255) return false;
  if (g.dim % 16 != 0 || g.dim < 112 || g.dim > 128 || g.dp != g.dim) return false;
  return fp16_integer((int64_t)g.int_lo - 1024);
}

// After rows [row0, end) were written and scanned: keep the byte rows of
// [0, end) current, or drop them when the rows no longer qualify.
static void update_byte_rows(Graph& g, int64_t row0, int64_t end, hipStream_t stream) {
  if (!byte_rows_eligible(g)) {
    if (g.vecs8) (void)hipFree(g.vecs8);
    g.vecs8 = nullptr;
    g.vecs8_cap = 0;
    return;
  }
  if (end <= 0) return;
  int64_t from = row0;
  if (!g.vecs8 || g.vecs8_lo != g.int_lo || g.vecs8_cap < end) {
    if (g.vecs8) (void)hipFree(g.vecs8);
    g.vecs8 = nullptr;
    const int64_t cap = std::max<int64_t>(g.capacity, end);
    hip_check(hipMalloc((void**)&g.vecs8, (size_t)cap * g.dim), "alloc byte rows");
    g.vecs8_cap = cap;
    g.vecs8_lo = g.int_lo;
    from = 0;
  }
  const int64_t rows = end - from;
  if (rows <= 0) return;
  const uint32_t dim8 = g.dim / 8;
  const int64_t total = rows * dim8;
  hipLaunchKernelGGL(byte_rows_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, stream,
                     (const uint4*)g.vecs, g.dp / 8, dim8, from, rows, g.int_lo, (uint2*)g.vecs8);
  hip_check(hipGetLastError(), "launch byte_rows_kernel");
}

void refresh_byte_rows(Graph& g, int64_t rows, hipStream_t stream) { update_byte_rows(g, 0, rows, stream); }

static void scan_int_range_only(Graph& g, int64_t row0, int64_t n, hipStream_t stream);

void scan_int_range(Graph& g, int64_t row0, int64_t n, hipStream_t stream) {
  scan_int_range_only(g, row0, n, stream);
  update_byte_rows(g, row0, row0 + n, stream);
}

static void scan_int_range_only(Graph& g, int64_t row0, int64_t n, hipStream_t stream) {
  if (!int_exact_enabled() || !g.vecs || g.on_host) {
    g.int_state = 2;
    return;
  }
  if (row0 > 0 && g.int_state == 0) {  // rows before row0 were never scanned
    n += row0;
    row0 = 0;
  }
  if (row0 > 0 && g.int_state == 2) return;  // already known not to be integers
  if (n <= 0) {
    if (row0 == 0) g.int_state = 0;
    return;
  }
  int32_t* d = nullptr;
  hip_check(hipMallocAsync((void**)&d, 12, stream), "alloc range");
  const int32_t init[3] = {0, INT32_MAX, INT32_MIN};
  hip_check(hipMemcpyAsync(d, init, 12, hipMemcpyHostToDevice, stream), "init range");
  const size_t count8 = (size_t)n * g.dp / 8;  // dp is a multiple of 8
  const uint4* first = (const uint4*)g.vecs + (size_t)row0 * g.dp / 8;
  const uint32_t grid = (uint32_t)std::min<size_t>((count8 + 255) / 256, 1024);  // 4 blocks per CU
  hipLaunchKernelGGL(int_range_kernel, dim3(grid), dim3(256), 0, stream, first, count8, d);
  hip_check(hipGetLastError(), "launch int_range_kernel");
  int32_t h[3];
  hip_check(hipMemcpyAsync(h, d, 12, hipMemcpyDeviceToHost, stream), "read range");
  hip_check(hipStreamSynchronize(stream), "sync range");
  hip_check(hipFreeAsync(d, stream), "free range");
  const bool ok = h[0] == 0 && h[1] <= h[2];
  if (!ok) {
    g.int_state = 2;
  } else if (row0 > 0) {  // state 1: merge with the range of rows [0, row0)
    g.int_lo = std::min(g.int_lo, h[1]);
    g.int_hi = std::max(g.int_hi, h[2]);
  } else {
    g.int_lo = h[1];
    g.int_hi = h[2];
    g.int_state = 1;
  }
}

bool int_range(const Graph& g) { return g.int_state == 1; }

bool int_exact_l2(const Graph& g, hipStream_t stream, int32_t* lo_out) {
  (void)stream;
  if (g.metric != 0 || !int_range(g)) return false;
  if ((int64_t)g.int_hi - (int64_t)g.int_lo > (int64_t)int_exact_span(g.dim)) return false;
  if (lo_out) *lo_out = g.int_lo;
  return true;
}

void upload_vectors(Graph& g, const void* src, int64_t n, uint32_t dim, hipStream_t stream) {
  upload_rows(g, src, 0, n, dim, stream);
}

void upload_rows(Graph& g, const void* src, int64_t row0, int64_t n, uint32_t dim, hipStream_t stream) {
  if (n <= 0) return;
  if (row0 < 0 || row0 + n > g.capacity) throw std::out_of_range("rows outside the graph's storage");
  const hipMemcpyKind kind = hipMemcpyDefault;
  hip_check(hipMemcpy2DAsync((char*)g.vecs + (size_t)row0 * g.dp * 2, (size_t)g.dp * 2, src, (size_t)dim * 2,
                             (size_t)dim * 2, (size_t)n, kind, stream),
            "upload vectors");
  scan_int_range(g, row0, n, stream);
}

void download_graph(const Graph& g, HostGraph& h, bool with_vectors) {
  const size_t n = (size_t)g.n;
  h.edges.resize(n * g.R);
  h.edist.resize(n * g.R);
  h.counts.resize(n);
  h.deleted.resize((n + 31) / 32);
  h.slot_to_id.resize(n);
  if (n == 0) return;
  hip_check(hipDeviceSynchronize(), "sync before download");
  hip_check(hipMemcpy(h.edges.data(), g.edges, n * g.R * 4, hipMemcpyDefault), "download edges");
  hip_check(hipMemcpy(h.edist.data(), g.edist, n * g.R * 2, hipMemcpyDefault), "download edge distances");
  hip_check(hipMemcpy(h.counts.data(), g.counts, n, hipMemcpyDefault), "download counts");
  hip_check(hipMemcpy(h.deleted.data(), g.deleted, h.deleted.size() * 4, hipMemcpyDefault), "download deleted");
  hip_check(hipMemcpy(h.slot_to_id.data(), g.slot_to_id, n * 4, hipMemcpyDefault), "download slot ids");
  if (with_vectors) {
    h.vecs.resize(n * g.dp);
    hip_check(hipMemcpy(h.vecs.data(), g.vecs, n * g.dp * 2, hipMemcpyDefault), "download vectors");
  }
}

void save_graph_file(const Graph& g, const std::string& path) {
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  if (!f.is_open()) throw std::runtime_error("failed to open " + path + " for graph save");
  const uint64_t n = (uint64_t)g.n;
  const uint64_t bpn = 2ull * g.dim + 1 + 6ull * g.R + 4;
  const uint64_t del_bytes = (n + 7) / 8;
  const uint64_t total = 32 + n * bpn + del_bytes + 8;
  const uint64_t medoid = g.medoid;
  f.write((const char*)&total, 8);
  f.write((const char*)&n, 8);
  f.write((const char*)&medoid, 8);
  f.write((const char*)&bpn, 8);

  HostGraph h;
  download_graph(g, h, true);
  std::vector<uint8_t> packed(del_bytes, 0);
  const size_t chunk = 1u << 16;
  std::vector<uint8_t> buf;
  for (size_t s = 0; s < n; s += chunk) {
    const size_t e = std::min<size_t>(n, s + chunk);
    buf.resize((e - s) * bpn);
    uint8_t* p = buf.data();
    for (size_t i = s; i < e; ++i) {
      std::memcpy(p, &h.vecs[i * g.dp], 2ull * g.dim);
      p += 2ull * g.dim;
      *p++ = h.counts[i];
      std::memcpy(p, &h.edges[i * g.R], 4ull * g.R);
      p += 4ull * g.R;
      std::memcpy(p, &h.edist[i * g.R], 2ull * g.R);
      p += 2ull * g.R;
      std::memcpy(p, &h.slot_to_id[i], 4);
      p += 4;
      if ((h.deleted[i >> 5] >> (i & 31)) & 1u) packed[i >> 3] |= (uint8_t)(1u << (i & 7));
    }
    f.write((const char*)buf.data(), (std::streamsize)buf.size());
  }
  f.write((const char*)packed.data(), (std::streamsize)packed.size());
  const uint64_t next_id = g.next_id;
  f.write((const char*)&next_id, 8);
  if (!f.good()) throw std::runtime_error("short write while saving " + path);
}

std::unique_ptr<Graph> load_graph_file(const std::string& path, uint32_t dim, uint32_t R, int metric,
                                       bool on_host, uint64_t* trailer_offset) {
  std::ifstream f(path, std::ios::binary);
  if (!f.is_open()) throw std::runtime_error("failed to open " + path + " for graph load");
  uint64_t hdr[4];
  f.read((char*)hdr, 32);
  if (f.gcount() != 32) throw std::runtime_error("truncated graph header in " + path);
  const uint64_t total = hdr[0], n = hdr[1], medoid = hdr[2], bpn = hdr[3];
  const uint64_t base = 2ull * dim + 1 + 6ull * R;
  const bool bitpacked = bpn == base + 4;
  const bool has_id = bitpacked || bpn == base + 5;
  const bool inline_del = bpn == base + 5 || bpn == base + 1;
  if (!bitpacked && !inline_del && bpn != base)
    throw std::runtime_error("bytes_per_node " + std::to_string(bpn) + " matches no known layout for dim " +
                             std::to_string(dim) + ", R " + std::to_string(R));
  if (n > 0x7FFFFFFFull) throw std::runtime_error("graph too large for 31-bit ids");

  auto g = std::make_unique<Graph>();
  g->allocate((int64_t)n, dim, R, metric, on_host);
  g->medoid = (uint32_t)medoid;
  const uint32_t dp = g->dp;
  HostGraph h;
  h.vecs.assign((size_t)n * dp, 0);
  h.edges.assign((size_t)n * R, 0);
  h.edist.assign((size_t)n * R, 0);
  h.counts.assign((size_t)n, 0);
  h.deleted.assign(((size_t)n + 31) / 32, 0);
  h.slot_to_id.assign((size_t)n, 0);
  const size_t chunk = 1u << 16;
  std::vector<uint8_t> buf;
  uint64_t n_del = 0;
  for (size_t s = 0; s < n; s += chunk) {
    const size_t e = std::min<size_t>(n, s + chunk);
    buf.resize((e - s) * bpn);
    f.read((char*)buf.data(), (std::streamsize)buf.size());
    if ((size_t)f.gcount() != buf.size())
      throw std::runtime_error("short read at record " + std::to_string(s) + " of " + path);
    const uint8_t* p = buf.data();
    for (size_t i = s; i < e; ++i) {
      std::memcpy(&h.vecs[i * dp], p, 2ull * dim);
      p += 2ull * dim;
      h.counts[i] = *p++;
      std::memcpy(&h.edges[i * R], p, 4ull * R);
      p += 4ull * R;
      std::memcpy(&h.edist[i * R], p, 2ull * R);
      p += 2ull * R;
      if (inline_del) {
        if (*p) { h.deleted[i >> 5] |= 1u << (i & 31); ++n_del; }
        ++p;
      }
      if (has_id) { std::memcpy(&h.slot_to_id[i], p, 4); p += 4; }
      else h.slot_to_id[i] = (uint32_t)i;
    }
  }
  uint64_t pos = 32 + n * bpn;
  if (bitpacked) {
    std::vector<uint8_t> packed((size_t)((n + 7) / 8));
    f.read((char*)packed.data(), (std::streamsize)packed.size());
    if ((size_t)f.gcount() != packed.size()) throw std::runtime_error("short read of deletion bits in " + path);
    for (size_t i = 0; i < n; ++i)
      if ((packed[i >> 3] >> (i & 7)) & 1u) { h.deleted[i >> 5] |= 1u << (i & 31); ++n_del; }
    pos += packed.size();
  }
  uint64_t next_id = n;
  if (has_id) {
    f.read((char*)&next_id, 8);
    if (f.gcount() != 8) throw std::runtime_error("missing next_id in " + path);
    pos += 8;
  }
  (void)total;
  if (trailer_offset) *trailer_offset = pos;
  g->next_id = next_id;
  g->n_deleted = n_del;
  if (n > 0) {
    hip_check(hipMemcpy(g->vecs, h.vecs.data(), (size_t)n * dp * 2, hipMemcpyDefault), "upload vectors");
    hip_check(hipMemcpy(g->edges, h.edges.data(), (size_t)n * R * 4, hipMemcpyDefault), "upload edges");
    hip_check(hipMemcpy(g->edist, h.edist.data(), (size_t)n * R * 2, hipMemcpyDefault), "upload edge dists");
    hip_check(hipMemcpy(g->counts, h.counts.data(), (size_t)n, hipMemcpyDefault), "upload counts");
    hip_check(hipMemcpy(g->deleted, h.deleted.data(), h.deleted.size() * 4, hipMemcpyDefault), "upload deleted");
    hip_check(hipMemcpy(g->slot_to_id, h.slot_to_id.data(), (size_t)n * 4, hipMemcpyDefault), "upload slot ids");
    scan_int_range(*g, 0, n, nullptr);
  }
  return g;
}

}  // namespace jasper_amd
