// capi.hip -- the C ABI (include/jasper_amd.h): handle table, argument
// checks, and the per-config entry points named like the reference's
// TVM-FFI exports (ffi/jasper_ffi_common.cuh:787-807, ffi/jasper_ffi_plain.cu).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstring>
#include <map>
#include <tuple>
#include <exception>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>

#include "../../include/jasper_amd.h"
#include "bruteforce.hpp"
#include "build.hpp"
#include "diskann.hpp"
#include "common.hpp"
#include "directional.hpp"
#include "directional_api.hpp"
#include "graph.hpp"
#include "rabitq.hpp"
#include "search.hpp"

namespace jasper_amd {

namespace {

thread_local std::string g_last_error;

struct Entry {
  std::unique_ptr<Graph> g;
  bool directional = false;
};

std::unordered_map<int64_t, Entry> g_table;
std::mutex g_mutex;
int64_t g_next_handle = 0;
BuildStats g_last_build;
ScaleStats g_last_scale;
DiskannStats g_last_diskann;

struct Config {
  uint32_t R;
  int metric;
  bool directional;
  uint32_t k_ranks;
  bool small_dim;  // dim <= 128 (packed_t = u8)
};

int64_t fail(const std::string& msg) {
  g_last_error = msg;
  return -1;
}

template <typename F>
int64_t guarded(F&& f) {
  try {
    return f();
  } catch (const std::exception& e) {
    return fail(e.what());
  } catch (...) {
    return fail("unknown error");
  }
}

int64_t insert(std::unique_ptr<Graph> g, bool directional) {
  std::lock_guard<std::mutex> lock(g_mutex);
  const int64_t h = g_next_handle++;
  g_table[h] = Entry{std::move(g), directional};
  return h;
}

// Handle lookup under the table lock; operations run outside the lock, as
// in the reference (ffi/jasper_ffi_common.cuh:308-314).
Graph& lookup(int64_t handle, const Config* cfg) {
  std::lock_guard<std::mutex> lock(g_mutex);
  auto it = g_table.find(handle);
  if (it == g_table.end()) throw std::invalid_argument("Invalid handle: " + std::to_string(handle));
  Graph& g = *it->second.g;
  if (cfg) {
    if (cfg->directional != it->second.directional || g.R != cfg->R || g.metric != cfg->metric ||
        (cfg->directional && g.k_ranks != cfg->k_ranks))
      throw std::invalid_argument("handle " + std::to_string(handle) + " was created with a different config");
  }
  return g;
}

bool is_device_ptr(const void* p) {
  if (!p) return false;
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

// Queries as device rows of padded length g.dp (copying when the caller's
// rows are unpadded, misaligned or in host memory).
struct QueryRows {
  const void* ptr = nullptr;
  void* owned = nullptr;
  hipStream_t stream = nullptr;
  ~QueryRows() {
    if (owned) (void)hipFreeAsync(owned, stream);
  }
};

void prepare_queries(const Graph& g, const void* q, int64_t nq, int64_t dim, hipStream_t s, QueryRows& out) {
  if (dim != (int64_t)g.dim)
    throw std::invalid_argument("query dim (" + std::to_string(dim) + ") != graph dim (" + std::to_string(g.dim) + ")");
  out.stream = s;
  const bool aligned = ((uintptr_t)q % 16) == 0;
  if (g.dp == g.dim && aligned && is_device_ptr(q)) {
    out.ptr = q;
    return;
  }
  hip_check(hipMallocAsync(&out.owned, (size_t)nq * g.dp * 2 + 16, s), "alloc padded queries");
  hip_check(hipMemsetAsync(out.owned, 0, (size_t)nq * g.dp * 2, s), "clear padded queries");
  hip_check(hipMemcpy2DAsync(out.owned, (size_t)g.dp * 2, q, (size_t)dim * 2, (size_t)dim * 2, (size_t)nq,
                             hipMemcpyDefault, s),
            "copy queries");
  out.ptr = out.owned;
}

int64_t do_search(const Config& cfg, int64_t handle, const void* queries, int64_t nq, int64_t dim, int32_t* out_idx,
                  float* out_dist, int64_t k, int64_t bw, int64_t limit, bool print, void* stream) {
  Graph& g = lookup(handle, &cfg);
  if (nq < 0 || k < 0 || bw <= 0 || limit < 0) throw std::invalid_argument("negative size argument");
  if (nq == 0 || k == 0) return 0;
  if (!is_device_ptr(out_idx) || !is_device_ptr(out_dist))
    throw std::invalid_argument("search outputs must be device memory");
  if (nq > 0x7FFFFFFF) throw std::invalid_argument("too many queries");
  hipStream_t s = (hipStream_t)stream;
  QueryRows rows;
  prepare_queries(g, queries, nq, dim, s, rows);
  SearchRequest r;
  r.queries = rows.ptr;
  r.nq = (uint32_t)nq;
  r.medoid = g.medoid;
  r.k = (uint32_t)k;
  r.beam_width = (uint32_t)bw;
  r.limit = (uint32_t)limit;
  r.max_result = 2048;  // search_params default (beam_search/api.cuh:17)
  r.out_ids = out_idx;
  r.out_dists = out_dist;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (print) {
    hip_check(hipEventCreate(&e0), "event");
    hip_check(hipEventCreate(&e1), "event");
    hip_check(hipEventRecord(e0, s), "event record");
  }
  launch_beam_search(g, r, s);
  if (print) {
    hip_check(hipEventRecord(e1, s), "event record");
    hip_check(hipEventSynchronize(e1), "event sync");
    float ms = 0;
    (void)hipEventElapsedTime(&ms, e0, e1);
    std::printf("[beam_search] duration=%gms, throughput=%g\n", ms, nq * 1000.0 / ms);
    std::fflush(stdout);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
  }
  return 0;
}

std::unique_ptr<Graph> construct(const Config& cfg, const void* vectors, int64_t n, int64_t dim, double alpha,
                                 int64_t budget, bool on_host, hipStream_t s) {
  if (n <= 0) throw std::invalid_argument("vectors must contain at least one row");
  if (n > 0x7FFFFFFF) throw std::invalid_argument("too many vectors for 31-bit ids");
  if (dim <= 0) throw std::invalid_argument("dim must be positive");
  auto g = std::make_unique<Graph>();
  g->allocate(n, (uint32_t)dim, cfg.R, cfg.metric, on_host);
  upload_vectors(*g, vectors, n, (uint32_t)dim, s);
  const int64_t mbs = reference_max_batch(n, cfg.R, budget);
  const char* timing = std::getenv("JASPER_BUILD_TIMING");
  const bool time_stages = timing && timing[0] == '1';
  BuildStats st;
  build_graph(*g, (float)alpha, mbs, s, time_stages, &st);
  g->next_id = (uint64_t)n;  // identity stable ids (id_map.cuh:260-281)
  {
    std::lock_guard<std::mutex> lock(g_mutex);
    g_last_build = st;
  }
  if (time_stages) {
    std::fprintf(stderr, "[construct] n=%lld batches=%lld max_batch=%lld search=%.1fms prune=%.1fms group=%.1fms "
                "reverse=%.1fms total=%.1fms\n",
                (long long)n, (long long)st.batches, (long long)st.max_batch, st.search_ms, st.prune_ms, st.sort_ms,
                st.reverse_ms, st.total_ms);
    std::fflush(stderr);
  }
  return g;
}

int64_t get_vector(Graph& g, int64_t index, void* out, hipStream_t s) {
  if (index < 0 || index >= g.n) throw std::out_of_range("Stable id " + std::to_string(index) + " not found");
  hip_check(hipMemcpyAsync(out, (const char*)g.vecs + (size_t)index * g.dp * 2, (size_t)g.dim * 2, hipMemcpyDefault, s),
            "copy vector");
  hip_check(hipStreamSynchronize(s), "sync");
  return 0;
}

}  // namespace
}  // namespace jasper_amd

using namespace jasper_amd;

#define JA_DEFINE_PLAIN(id)                                                                                    \
  extern "C" int64_t jasper_load_##id(const char* path, int64_t dim, bool on_host) {                           \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      if (!path) throw std::invalid_argument("null path");                                                     \
      auto g = load_graph_file(path, (uint32_t)dim, c.R, c.metric, on_host, nullptr);                          \
      return insert(std::move(g), false);                                                                      \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_construct_##id(const void* vectors, int64_t n, int64_t dim, double alpha,          \
                                           int64_t budget, bool on_host, void* stream) {                       \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      auto g = construct(c, vectors, n, dim, alpha, budget, on_host, (hipStream_t)stream);                     \
      return insert(std::move(g), false);                                                                      \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_search_##id(int64_t h, const void* q, int64_t nq, int64_t dim, int32_t* oi,        \
                                        float* od, int64_t k, int64_t bw, int64_t limit, bool print,           \
                                        void* stream) {                                                        \
    return guarded([&]() -> int64_t {                                                                          \
      return do_search(config_of(#id), h, q, nq, dim, oi, od, k, bw, limit, print, stream);                    \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_save_##id(int64_t h, const char* path) {                                           \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      save_graph_file(lookup(h, &c), path);                                                                    \
      return 0;                                                                                                \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_get_vector_##id(int64_t h, int64_t index, void* out, void* stream) {               \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      return get_vector(lookup(h, &c), index, out, (hipStream_t)stream);                                       \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_mark_deleted_##id(int64_t h, const int32_t* ids, int64_t n_ids) {                  \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      if (n_ids < 0) throw std::invalid_argument("negative id count");                                       \
      Graph& g = lookup(h, &c);                                                                                \
      mark_deleted(g, ids, n_ids, nullptr);                                                                    \
      return 0;                                                                                                \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_consolidate_##id(int64_t h, double alpha) {                                        \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      Graph& g = lookup(h, &c);                                                                                \
      consolidate(g, (float)alpha, nullptr);                                                                   \
      return 0;                                                                                                \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_compact_##id(int64_t h) {                                                          \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      lookup(h, &c);                                                                                           \
      throw std::runtime_error(                                                                                \
          "compact() is disabled in this build (deletion path is mark_deleted + consolidate only)");          \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_append_##id(int64_t h, const void* v, int64_t n, double alpha, int32_t* out_ids,   \
                                        void* stream) {                                                        \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      if (n < 0) throw std::invalid_argument("negative vector count");                                       \
      Graph& g = lookup(h, &c);                                                                                \
      append_rows(g, v, n, (float)alpha, out_ids, (hipStream_t)stream);                                        \
      return 0;                                                                                                \
    });                                                                                                        \
  }

namespace jasper_amd {
namespace {
// Parses a config id such as "f16_r64_l2" or "f16_r64_ip_k16_d128".
Config config_of(const char* id) {
  Config c{};
  const std::string s(id);
  const size_t r = s.find("_r");
  c.R = (uint32_t)std::atoi(s.c_str() + r + 2);
  c.metric = s.find("_ip") != std::string::npos ? kIP : kL2;
  const size_t k = s.find("_k");
  c.directional = k != std::string::npos;
  c.k_ranks = c.directional ? (uint32_t)std::atoi(s.c_str() + k + 2) : 0;
  c.small_dim = s.find("_d128") != std::string::npos;
  return c;
}
}  // namespace
}  // namespace jasper_amd

JASPER_PLAIN_CONFIGS(JA_DEFINE_PLAIN)

#define JA_DEFINE_DIRECTIONAL(id)                                                                              \
  extern "C" int64_t jasper_construct_directional_##id(const void* vectors, int64_t n, int64_t dim,            \
                                                       double alpha, int64_t budget, bool on_host,             \
                                                       bool prerotate, int64_t seed, void* stream) {           \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      check_directional_dim(c.small_dim, dim);                                                                 \
      auto g = construct_directional(c.R, c.metric, c.k_ranks, c.small_dim, vectors, n, dim, alpha, budget,    \
                                     on_host, prerotate, (uint64_t)seed, (hipStream_t)stream, &g_last_build);  \
      return insert(std::move(g), true);                                                                       \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_build_lsh_##id(int64_t h, int64_t n_samples, int64_t seed) {                       \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      build_lsh(lookup(h, &c), n_samples, (uint64_t)seed);                                                     \
      return 0;                                                                                                \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_build_pq_##id(int64_t h, int64_t n_train, int64_t iters, int64_t seed) {           \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      build_pq(lookup(h, &c), n_train, iters, (uint64_t)seed);                                                 \
      return 0;                                                                                                \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_directional_search_##id(int64_t h, const void* q, int64_t nq, int64_t dim,         \
                                                    int32_t* oi, float* od, int64_t k, int64_t bw,             \
                                                    int64_t limit, bool print, void* stream) {                 \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      directional_search(lookup(h, &c), false, q, nq, dim, oi, od, k, bw, limit, print, (hipStream_t)stream);  \
      return 0;                                                                                                \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_pq_search_##id(int64_t h, const void* q, int64_t nq, int64_t dim, int32_t* oi,     \
                                           float* od, int64_t k, int64_t bw, int64_t limit, bool print,        \
                                           void* stream) {                                                     \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      directional_search(lookup(h, &c), true, q, nq, dim, oi, od, k, bw, limit, print, (hipStream_t)stream);   \
      return 0;                                                                                                \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_save_directional_##id(int64_t h, const char* path) {                               \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      if (!path) throw std::invalid_argument("null path");                                                     \
      save_directional_file(lookup(h, &c), path);                                                              \
      return 0;                                                                                                \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_load_directional_##id(const char* path, int64_t dim, bool on_host, bool prerotate, \
                                                  int64_t seed) {                                              \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      if (!path) throw std::invalid_argument("null path");                                                     \
      check_directional_dim(c.small_dim, dim);                                                                 \
      auto g = load_directional_file(path, (uint32_t)dim, c.R, c.metric, c.k_ranks, c.small_dim, on_host,      \
                                     prerotate, (uint64_t)seed);                                               \
      return insert(std::move(g), true);                                                                       \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_get_vector_directional_##id(int64_t h, int64_t index, void* out, void* stream) {   \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      return get_vector(lookup(h, &c), index, out, (hipStream_t)stream);                                       \
    });                                                                                                        \
  }                                                                                                            \
  extern "C" int64_t jasper_get_directional_flags_##id(int64_t h) {                                            \
    return guarded([&]() -> int64_t {                                                                          \
      const Config c = config_of(#id);                                                                         \
      Graph& g = lookup(h, &c);                                                                                \
      return (int64_t)((g.lsh ? 1 : 0) | (g.pq ? 2 : 0) | (g.prerotate ? 8 : 0) | (g.rabitq ? 16 : 0));                             \
    });                                                                                                        \
  }

JASPER_DIRECTIONAL_CONFIGS(JA_DEFINE_DIRECTIONAL)

extern "C" int64_t jasperx_prerotate_seed(int64_t h) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    return g.prerotate ? (int64_t)(g.prerotate_seed & 0x7FFFFFFFFFFFFFFFull) : -1;
  });
}

extern "C" int64_t jasperx_row_format(int64_t h, int64_t* out4) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    if (!out4) throw std::invalid_argument("null output");
    out4[0] = g.int_state;
    out4[1] = g.int_lo;
    out4[2] = g.int_hi;
    out4[3] = g.vecs8 && g.vecs8_lo == g.int_lo && g.vecs8_cap >= g.n && byte_rows_eligible(g) ? 1 : 0;
    return 0;
  });
}

extern "C" int64_t jasper_free_graph(int64_t h) {
  return guarded([&]() -> int64_t {
    std::unique_ptr<Graph> victim;
    {
      std::lock_guard<std::mutex> lock(g_mutex);
      auto it = g_table.find(h);
      if (it == g_table.end()) throw std::invalid_argument("Invalid handle: " + std::to_string(h));
      victim = std::move(it->second.g);
      g_table.erase(it);
    }
    (void)hipDeviceSynchronize();
    victim.reset();
    return 0;
  });
}

extern "C" int64_t jasper_get_n_vectors(int64_t h) {
  return guarded([&]() -> int64_t { return lookup(h, nullptr).n; });
}

extern "C" int64_t jasper_get_n_tombstoned(int64_t h) {
  return guarded([&]() -> int64_t { return (int64_t)lookup(h, nullptr).n_deleted; });
}

extern "C" int64_t jasper_get_n_live(int64_t h) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    return g.n - (int64_t)g.n_deleted;
  });
}

extern "C" int64_t jasper_reserve_ids(int64_t h, int32_t* out_ids, int64_t count) {
  return guarded([&]() -> int64_t {
    if (count < 0) throw std::invalid_argument("negative count");
    std::lock_guard<std::mutex> lock(g_mutex);
    auto it = g_table.find(h);
    if (it == g_table.end()) throw std::invalid_argument("Invalid handle: " + std::to_string(h));
    Graph& g = *it->second.g;
    const uint64_t start = g.next_id;
    g.next_id += (uint64_t)count;
    for (int64_t i = 0; i < count; ++i) out_ids[i] = (int32_t)(start + (uint64_t)i);
    return 0;
  });
}

extern "C" int64_t jasper_get_dim(int64_t h) {
  return guarded([&]() -> int64_t { return (int64_t)lookup(h, nullptr).dim; });
}

extern "C" const char* jasper_last_error(void) { return g_last_error.c_str(); }

extern "C" int64_t jasperx_export_graph(int64_t h, uint32_t* edges, uint16_t* edge_dist, uint8_t* counts) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    HostGraph hg;
    download_graph(g, hg, false);
    if (edges) std::memcpy(edges, hg.edges.data(), hg.edges.size() * 4);
    if (edge_dist) std::memcpy(edge_dist, hg.edist.data(), hg.edist.size() * 2);
    if (counts) std::memcpy(counts, hg.counts.data(), hg.counts.size());
    return g.n;
  });
}

extern "C" int64_t jasperx_export_vectors(int64_t h, uint16_t* out) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    if (out && g.n > 0)
      hip_check(hipMemcpy(out, g.vecs, (size_t)g.n * g.dp * 2, hipMemcpyDefault), "download vectors");
    return (int64_t)g.dp;
  });
}

extern "C" int64_t jasperx_export_lsh(int64_t h, float* c_per_rank, float* norm_denom, uint8_t* rows) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    if (!g.lsh) throw std::runtime_error("graph has no LSH artifacts");
    const LshArtifacts& a = *g.lsh;
    if (c_per_rank) std::memcpy(c_per_rank, a.c_per_rank.data(), a.c_per_rank.size() * 4);
    if (norm_denom) *norm_denom = a.norm_denom;
    if (rows && g.n > 0) hip_check(hipMemcpy(rows, a.rows, (size_t)g.n * a.row_bytes, hipMemcpyDefault), "download lsh rows");
    return (int64_t)a.row_bytes;
  });
}

extern "C" int64_t jasperx_export_pq(int64_t h, float* centroids, uint8_t* codes, float* norms) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    if (!g.pq) throw std::runtime_error("graph has no PQ artifacts");
    const PqArtifacts& a = *g.pq;
    if (centroids)
      hip_check(hipMemcpy(centroids, a.centroids, (size_t)a.m * 256 * a.dsub * 4, hipMemcpyDefault), "download centroids");
    if (codes && g.n > 0) pq_codes_to_file_layout(g, codes);
    if (norms && g.n > 0 && g.vector_norms)
      hip_check(hipMemcpy(norms, g.vector_norms, (size_t)g.n * 4, hipMemcpyDefault), "download norms");
    return (int64_t)a.dsub;
  });
}

extern "C" int64_t jasperx_directional_query_rows(int64_t h, const void* queries, int64_t nq, int64_t dim,
                                                  uint16_t* out, void* stream) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    directional_query_rows_to_host(g, queries, nq, dim, out, (hipStream_t)stream);
    return (int64_t)g.dp;
  });
}

extern "C" int64_t jasperx_rotate_rows(int64_t dim, int64_t seed, const void* x, int64_t n, int64_t x_stride,
                                       void* out, int64_t out_stride, void* stream) {
  return guarded([&]() -> int64_t {
    if (dim <= 0 || dim > 65536) throw std::invalid_argument("dim must be in 1..65536");
    if (n < 0 || x_stride < dim || out_stride < dim) throw std::invalid_argument("bad row counts or strides");
    // matrices are cached per (device, dim, seed): the Householder QR runs on the host
    static std::mutex cache_mutex;
    static std::map<std::tuple<int, int64_t, int64_t>, std::unique_ptr<RotationMatrix>> cache;
    int device = 0;
    hip_check(hipGetDevice(&device), "get device");
    const RotationMatrix* r = nullptr;
    {
      std::lock_guard<std::mutex> lock(cache_mutex);
      auto& slot = cache[std::make_tuple(device, dim, seed)];
      if (!slot) slot = make_rotation(rotation_matrix((uint32_t)dim, (uint64_t)seed), (uint32_t)dim);
      r = slot.get();
    }
    hipStream_t s = (hipStream_t)stream;
    rotate_rows_any(*r, x, n, x_stride, out, out_stride, s);
    return 0;
  });
}

extern "C" int64_t jasperx_rabitq_node_bytes(int64_t dim) {
  return guarded([&]() -> int64_t {
    if (dim <= 0 || dim > 65536) throw std::invalid_argument("dim must be in 1..65536");
    return (int64_t)rabitq_code_bytes((uint32_t)dim) + 8;
  });
}

extern "C" int64_t jasperx_rabitq_quantize(const void* vectors, int32_t dtype, int64_t n, int64_t dim, int64_t stride,
                                           const float* rotation, const float* centroid, int32_t metric, void* out,
                                           void* stream) {
  return guarded([&]() -> int64_t {
    if (dtype != 0 && dtype != 1) throw std::invalid_argument("dtype must be 0 (fp16) or 1 (fp32)");
    if (metric != kL2 && metric != kIP) throw std::invalid_argument("metric must be 0 (L2) or 1 (IP)");
    if (n < 0 || dim <= 0 || stride < dim) throw std::invalid_argument("bad sizes");
    if (!rotation) throw std::invalid_argument("rotation matrix is required");
    rabitq_quantize(vectors, dtype == 0, n, (uint32_t)dim, (uint32_t)stride, rotation, centroid, metric, out,
                    (hipStream_t)stream);
    return (int64_t)rabitq_code_bytes((uint32_t)dim) + 8;
  });
}

extern "C" int64_t jasperx_bruteforce_knn(const void* base, int64_t n, int64_t dim, int64_t base_stride,
                                          const void* queries, int64_t nq, int64_t query_stride, int64_t k,
                                          int32_t metric, int32_t* out_ids, float* out_dists, void* stream) {
  return guarded([&]() -> int64_t {
    if (metric != kL2 && metric != kIP) throw std::invalid_argument("metric must be 0 (L2) or 1 (IP)");
    if (dim <= 0 || n <= 0 || nq < 0 || k <= 0) throw std::invalid_argument("bad sizes");
    if (base_stride != query_stride || base_stride % 8 != 0 || base_stride < dim || base_stride - dim >= 8)
      throw std::invalid_argument("rows must be padded to the next multiple of 8 (same stride for both)");
    if (((uintptr_t)base & 15u) || ((uintptr_t)queries & 15u)) throw std::invalid_argument("rows must be 16-byte aligned");
    bruteforce_knn(base, n, (uint32_t)dim, (uint32_t)base_stride, queries, nq, (uint32_t)k, metric, out_ids,
                   out_dists, (hipStream_t)stream);
    return 0;
  });
}

extern "C" int64_t jasperx_build_pq_m(int64_t h, int64_t m, int64_t n_train, int64_t iters, int64_t seed) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    if (g.k_ranks == 0) throw std::invalid_argument("build_pq needs a directional graph");
    if (m <= 0 || m > (int64_t)kPqMaxM)
      throw std::invalid_argument("m must be in 1.." + std::to_string(kPqMaxM));
    build_pq(g, n_train, iters, (uint64_t)seed, (uint32_t)m);
    return 0;
  });
}

extern "C" int64_t jasperx_construct_directional_ex(const char* config, const void* vectors, int64_t n, int64_t dim,
                                                    double alpha, int64_t budget, bool on_host, bool prerotate,
                                                    int64_t seed, uint32_t options, void* stream) {
  return guarded([&]() -> int64_t {
    if (!config) throw std::invalid_argument("null config id");
    static const char* const kNames[] = {
#define JA_DIR_NAME(id) #id,
        JASPER_DIRECTIONAL_CONFIGS(JA_DIR_NAME)
#undef JA_DIR_NAME
    };
    bool known = false;
    for (const char* name : kNames) known = known || std::strcmp(name, config) == 0;
    if (!known) throw std::invalid_argument(std::string("unknown directional config ") + config);
    if (options & ~kBuildOptionsKnown) throw std::invalid_argument("unknown construction options");
    const Config c = config_of(config);
    check_directional_dim(c.small_dim, dim);
    auto g = construct_directional(c.R, c.metric, c.k_ranks, c.small_dim, vectors, n, dim, alpha, budget, on_host,
                                   prerotate, (uint64_t)seed, (hipStream_t)stream, &g_last_build, options);
    return insert(std::move(g), true);
  });
}

extern "C" int64_t jasperx_construct_scale(const char* config, const void* vectors, int64_t n, int64_t dim,
                                           double alpha, int64_t n_parts, int64_t budget, int64_t max_batch_size,
                                           bool on_host, void* stream) {
  return guarded([&]() -> int64_t {
    if (!config) throw std::invalid_argument("null config id");
    static const char* const kNames[] = {
#define JA_PLAIN_NAME(id) #id,
        JASPER_PLAIN_CONFIGS(JA_PLAIN_NAME)
#undef JA_PLAIN_NAME
    };
    bool known = false;
    for (const char* name : kNames) known = known || std::strcmp(name, config) == 0;
    if (!known) throw std::invalid_argument(std::string("unknown plain config ") + config);
    if (n <= 0) throw std::invalid_argument("vectors must contain at least one row");
    if (n > 0x7FFFFFFF) throw std::invalid_argument("too many vectors for 31-bit ids");
    if (dim <= 0) throw std::invalid_argument("dim must be positive");
    if (n_parts < 1) throw std::invalid_argument("n_parts must be positive");
    const Config c = config_of(config);
    hipStream_t s = (hipStream_t)stream;
    // partitions: min(budget batch, max_batch_size), the caller's cap
    // defaulting to n / n_parts / 20 (cmd/create_scale_index.cu:84,
    // construct_scale.cuh:96-99); merges: the budget batch (:383-385)
    const int64_t budget_batch = budget_max_batch(c.R, budget);
    if (budget_batch < 1) throw std::invalid_argument("workspace budget below one batch item");
    const int64_t cap = max_batch_size > 0 ? max_batch_size : std::max<int64_t>(1, n / n_parts / 20);
    const int64_t part_batch = std::min(budget_batch, cap);
    auto g = std::make_unique<Graph>();
    g->allocate(n, (uint32_t)dim, c.R, c.metric, on_host);
    upload_vectors(*g, vectors, n, (uint32_t)dim, s);
    ScaleStats st;
    if (on_host) build_scale_staged(*g, (float)alpha, n_parts, part_batch, budget_batch, s, &st);
    else build_scale(*g, (float)alpha, n_parts, part_batch, budget_batch, s, &st);
    g->next_id = (uint64_t)n;
    {
      std::lock_guard<std::mutex> lock(g_mutex);
      g_last_scale = st;
    }
    return insert(std::move(g), false);
  });
}

extern "C" int64_t jasperx_construct_diskann(const char* config, const void* vectors, int64_t n, int64_t dim,
                                             double alpha, int64_t r_int, int64_t n_parts, int64_t n_dup,
                                             int64_t budget, int64_t max_batch_size, int64_t seed,
                                             int64_t max_shard, void* stream) {
  return guarded([&]() -> int64_t {
    if (!config) throw std::invalid_argument("null config id");
    static const char* const kNames[] = {
#define JA_PLAIN_NAME(id) #id,
        JASPER_PLAIN_CONFIGS(JA_PLAIN_NAME)
#undef JA_PLAIN_NAME
    };
    bool known = false;
    for (const char* name : kNames) known = known || std::strcmp(name, config) == 0;
    if (!known) throw std::invalid_argument(std::string("unknown plain config ") + config);
    if (n <= 0) throw std::invalid_argument("vectors must contain at least one row");
    if (n > 0x7FFFFFFF) throw std::invalid_argument("too many vectors for 31-bit ids");
    if (dim <= 0) throw std::invalid_argument("dim must be positive");
    if (n_parts < 1) throw std::invalid_argument("n_parts must be positive");
    if (r_int < 1 || r_int > 64) throw std::invalid_argument("r_int must be between 1 and 64");
    const Config c = config_of(config);
    hipStream_t s = (hipStream_t)stream;
    // min(budget batch at R_int, the command's n / n_parts / 20)
    // (construct_diskann.cuh:373-375, cmd/create_diskann_index.cu:84)
    const int64_t budget_batch = budget_max_batch((uint32_t)r_int, budget);
    if (budget_batch < 1) throw std::invalid_argument("workspace budget below one batch item");
    const int64_t cap = max_batch_size > 0 ? max_batch_size : std::max<int64_t>(1, n / n_parts / 20);
    auto g = std::make_unique<Graph>();
    g->allocate(n, (uint32_t)dim, c.R, c.metric, false);
    upload_vectors(*g, vectors, n, (uint32_t)dim, s);
    DiskannStats st;
    // shards larger than the device can build are split (max_shard <= 0:
    // from the free device memory, as construct_diskann.cuh:386-397)
    const int64_t shard_cap =
        max_shard > 0 ? max_shard : diskann_max_shard_for_device((uint32_t)dim, (uint32_t)r_int, budget);
    build_diskann(*g, (uint32_t)r_int, (float)alpha, n_parts, n_dup, (uint64_t)seed, std::min(budget_batch, cap),
                  shard_cap, s, &st);
    g->next_id = (uint64_t)n;
    {
      std::lock_guard<std::mutex> lock(g_mutex);
      g_last_diskann = st;
    }
    return insert(std::move(g), false);
  });
}

extern "C" int64_t jasperx_diskann_assign(const void* vectors, int64_t n, int64_t dim, int64_t n_parts,
                                          int64_t n_dup, int64_t seed, uint32_t* out_shard_of, uint16_t* out_mean,
                                          void* stream) {
  return guarded([&]() -> int64_t {
    if (n <= 0) throw std::invalid_argument("vectors must contain at least one row");
    if (n > 0x7FFFFFFF) throw std::invalid_argument("too many vectors for 31-bit ids");
    if (dim <= 0) throw std::invalid_argument("dim must be positive");
    hipStream_t s = (hipStream_t)stream;
    Graph g;
    g.allocate(n, (uint32_t)dim, 1, kL2, false);
    upload_vectors(g, vectors, n, (uint32_t)dim, s);
    diskann_assign(g, n_parts, n_dup, (uint64_t)seed, out_shard_of, out_mean, s);
    return 0;
  });
}

extern "C" int64_t jasperx_last_diskann_stats(double* out6) {
  return guarded([&]() -> int64_t {
    std::lock_guard<std::mutex> lock(g_mutex);
    const DiskannStats& s = g_last_diskann;
    const double v[6] = {s.assign_ms, s.build_ms, s.merge_ms, s.total_ms, (double)s.shards, (double)s.max_shard};
    std::memcpy(out6, v, sizeof(v));
    return 0;
  });
}

extern "C" int64_t jasperx_last_scale_stats(double* out7) {
  return guarded([&]() -> int64_t {
    std::lock_guard<std::mutex> lock(g_mutex);
    const ScaleStats& s = g_last_scale;
    const double v[7] = {s.partition_ms, s.merge_ms, s.total_ms, (double)s.merges, (double)s.merge_batches,
                         (double)s.part_batch, (double)s.merge_batch};
    std::memcpy(out7, v, sizeof(v));
    return 0;
  });
}

extern "C" int64_t jasperx_exact_search(int64_t h, const void* q, int64_t nq, int64_t dim, int32_t* out_ids,
                                        float* out_dists, int64_t k, int64_t bw, int64_t limit, void* stream) {
  return guarded([&]() -> int64_t {
    exact_search(lookup(h, nullptr), q, nq, dim, out_ids, out_dists, k, bw, limit, (hipStream_t)stream);
    return 0;
  });
}

extern "C" int64_t jasperx_build_rabitq(int64_t h) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    if (g.k_ranks == 0) throw std::invalid_argument("build_rabitq needs a directional graph");
    build_rabitq(g);
    return 0;
  });
}

extern "C" int64_t jasperx_export_rabitq(int64_t h, float* centroid, uint8_t* nodes) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    if (!g.rabitq) throw std::runtime_error("graph has no RaBitQ codes");
    const RabitqArtifacts& a = *g.rabitq;
    if (centroid) hip_check(hipMemcpy(centroid, a.centroid, (size_t)a.dim * 4, hipMemcpyDefault), "download centroid");
    if (nodes && g.n > 0)
      hip_check(hipMemcpy(nodes, a.nodes, (size_t)g.n * (a.code_bytes + 8), hipMemcpyDefault), "download nodes");
    return (int64_t)(a.code_bytes + 8);
  });
}

extern "C" int64_t jasperx_directional_search_ex(int64_t h, int32_t estimator, const void* q, int64_t nq, int64_t dim,
                                                 int32_t* out_ids, float* out_dists, int64_t k, int64_t bw,
                                                 int64_t limit, uint32_t flags, void* stream) {
  return guarded([&]() -> int64_t {
    if (flags & ~kDirFlagsKnown) throw std::invalid_argument("unknown directional search flags");
    directional_search(lookup(h, nullptr), estimator, q, nq, dim, out_ids, out_dists, k, bw, limit, false,
                       (hipStream_t)stream, nullptr, (flags & kDirUnique) != 0);
    return 0;
  });
}

extern "C" int64_t jasperx_directional_search_noalloc(int64_t h, int32_t estimator, const void* q, int64_t nq,
                                                      int64_t dim, int32_t* out_ids, float* out_dists, int64_t k,
                                                      int64_t bw, int64_t limit, uint32_t flags, void* stream) {
  return guarded([&]() -> int64_t {
    if (flags & ~kDirFlagsKnown) throw std::invalid_argument("unknown directional search flags");
    directional_search_noalloc(lookup(h, nullptr), estimator, q, nq, dim, out_ids, out_dists, k, bw, limit,
                               (flags & kDirUnique) != 0, (hipStream_t)stream);
    return 0;
  });
}

extern "C" int64_t jasperx_directional_stats(int64_t h, int32_t estimator, const void* q, int64_t nq, int64_t dim,
                                             int64_t k, int64_t bw, int64_t limit, uint32_t flags,
                                             uint32_t* out_stats, void* stream) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    if (nq <= 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    int32_t* ids = nullptr;
    float* d = nullptr;
    uint32_t* st = nullptr;
    hip_check(hipMalloc(&ids, (size_t)nq * k * 4), "alloc ids");
    hip_check(hipMalloc(&d, (size_t)nq * k * 4), "alloc dists");
    hip_check(hipMalloc(&st, (size_t)nq * 12), "alloc stats");
    try {
      if (flags & ~kDirFlagsKnown) throw std::invalid_argument("unknown directional search flags");
      directional_search(g, estimator, q, nq, dim, ids, d, k, bw, limit, false, s, st, (flags & kDirUnique) != 0);
      hip_check(hipMemcpyAsync(out_stats, st, (size_t)nq * 12, hipMemcpyDeviceToHost, s), "download stats");
      hip_check(hipStreamSynchronize(s), "sync stats");
    } catch (...) {
      (void)hipFree(ids);
      (void)hipFree(d);
      (void)hipFree(st);
      throw;
    }
    (void)hipFree(ids);
    (void)hipFree(d);
    (void)hipFree(st);
    return 0;
  });
}

extern "C" int64_t jasperx_last_build_stats(double* out7) {
  return guarded([&]() -> int64_t {
    std::lock_guard<std::mutex> lock(g_mutex);
    const BuildStats& s = g_last_build;
    const double v[7] = {s.search_ms, s.prune_ms, s.sort_ms, s.reverse_ms, s.total_ms, (double)s.batches,
                         (double)s.max_batch};
    std::memcpy(out7, v, sizeof(v));
    return 0;
  });
}

extern "C" int64_t jasperx_build_work_counting(int64_t on) {
  return guarded([&]() -> int64_t {
    set_build_work_counting(on != 0);
    return 0;
  });
}

extern "C" int64_t jasperx_last_build_work(uint64_t* out16) {
  return guarded([&]() -> int64_t {
    std::lock_guard<std::mutex> lock(g_mutex);
    std::memcpy(out16, g_last_build.work, sizeof(g_last_build.work));
    return 0;
  });
}

extern "C" int64_t jasperx_search_stats(int64_t h, const void* q, int64_t nq, int64_t dim, int64_t k, int64_t bw,
                                        int64_t limit, uint32_t* out_stats, void* stream) {
  return guarded([&]() -> int64_t {
    Graph& g = lookup(h, nullptr);
    if (nq <= 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    QueryRows rows;
    prepare_queries(g, q, nq, dim, s, rows);
    const size_t words = (size_t)((g.n + 31) / 32);
    const size_t chunk = std::max<size_t>(1, std::min<size_t>((size_t)nq, ((size_t)1 << 31) / (words * 4)));
    uint32_t* bits = nullptr;
    uint32_t* st = nullptr;
    hip_check(hipMalloc(&bits, chunk * words * 4), "alloc seen bitmap");
    hip_check(hipMalloc(&st, chunk * 16), "alloc stats");
    try {
      for (size_t b = 0; b < (size_t)nq; b += chunk) {
        const size_t m = std::min(chunk, (size_t)nq - b);
        hip_check(hipMemsetAsync(bits, 0, m * words * 4, s), "clear seen bitmap");
        SearchRequest r;
        r.queries = (const char*)rows.ptr + b * g.dp * 2;
        r.nq = (uint32_t)m;
        r.medoid = g.medoid;
        r.k = (uint32_t)k;
        r.beam_width = (uint32_t)bw;
        r.limit = (uint32_t)limit;
        r.max_result = 2048;
        r.seen_bits = bits;
        r.stats = st;
        launch_beam_search(g, r, s);
        hip_check(hipMemcpyAsync(out_stats + b * 4, st, m * 16, hipMemcpyDeviceToHost, s), "copy stats");
        hip_check(hipStreamSynchronize(s), "sync stats");
      }
    } catch (...) {
      (void)hipFree(bits);
      (void)hipFree(st);
      throw;
    }
    (void)hipFree(bits);
    (void)hipFree(st);
    return 0;
  });
}

extern "C" const char* jasperx_version(void) { return "jasper_amd 0.1 gfx950"; }
