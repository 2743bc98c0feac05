// jasper_oracle.cpp -- TEST INFRASTRUCTURE ONLY.
//
// CPU restatement of the reference's query/build hot path, used as the parity
// checker for the HIP implementation. Nothing in the product (jasper_amd/)
// links, loads or calls this file; only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg do, and only as the checker / the reported CPU
// baseline.
//
// Every function cites the reference source it restates (paths relative to
// the reference tree, saltsystemslab/Jasper). The restatement is written from
// the algorithm, not translated from the CUDA: the device-side parallel
// decomposition (tiles, CUB sorts, atomics) is replaced by the sequential
// order it is equivalent to, and every arithmetic step that decides a result
// bit (accumulation order, fma, bf16 rounding) is spelled out.
//
// Build: oracle/Makefile (g++ -O3 -fopenmp -ffp-contract=off). fp contraction
// is off so that the only fused multiply-adds are the explicit fmaf() calls.

#include <algorithm>
#include <numeric>
#include <atomic>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>
#include <vector>

#include <omp.h>

namespace {

constexpr uint32_t kInvalid31 = 0x7FFFFFFFu;   // beam_search/entry.cuh:24-29 (31-bit masked id)
constexpr uint32_t kInvalid32 = 0xFFFFFFFFu;   // index/construct.cuh:303 (numeric_limits<index_t>::max)

// ---------------------------------------------------------------- numerics --

// IEEE binary16 -> binary32, exact.
inline float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {  // subnormal: normalise
      int e = -1;
      do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
      man &= 0x3FFu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// binary32 -> bfloat16 bits, round to nearest even (the conversion
// `(__nv_bfloat16)float` performs; index/graph.cuh:494).
inline uint16_t f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
  const uint32_t bias = 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)((u + bias) >> 16);
}

inline float bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Squared L2 distance, distance/distance.cuh:33-92 (l2_distance::compute)
// with DATA_T = __half, TILE_SIZE = 4, loads_per_round = 2.
// Lane l of the 4-lane tile owns the 16-byte chunks w = l + 4j + 8i, i.e. the
// chunks congruent to l mod 4 in ascending order, and accumulates
// acc = fma(d, d, acc) with d = f32(a) - f32(b) over the 8 halves of each
// chunk in order (nvcc contracts `local_sum += diff * diff`). The four lane
// sums are combined by cg::reduce as a xor butterfly (offset 2, then 1):
// (l0 + l2) + (l1 + l3).
float l2_dist(const uint16_t* a, const uint16_t* b, int dim) {
  const int total_loads = dim / 8;
  float lane[4];
  for (int l = 0; l < 4; ++l) {
    float acc = 0.0f;
    for (int c = l; c < total_loads; c += 4) {
      for (int k = 0; k < 8; ++k) {
        const float d = h2f(a[c * 8 + k]) - h2f(b[c * 8 + k]);
        acc = std::fmaf(d, d, acc);
      }
    }
    lane[l] = acc;
  }
  return (lane[0] + lane[2]) + (lane[1] + lane[3]);
}

// Negated inner product, distance/distance.cuh:94-106. Lane l sums elements
// i = l, l+4, ... (products of two halves are exact in fp32, so fma and
// mul+add agree); same butterfly; negated.
float ip_dist(const uint16_t* a, const uint16_t* b, int dim) {
  float lane[4];
  for (int l = 0; l < 4; ++l) {
    float acc = 0.0f;
    for (int i = l; i < dim; i += 4) acc = std::fmaf(h2f(a[i]), h2f(b[i]), acc);
    lane[l] = acc;
  }
  return -((lane[0] + lane[2]) + (lane[1] + lane[3]));
}

inline float dist(int metric, const uint16_t* a, const uint16_t* b, int dim) {
  return metric == 0 ? l2_dist(a, b, dim) : ip_dist(a, b, dim);
}

// ------------------------------------------------------------ plain search --

struct Entry {
  uint32_t id;   // 31-bit masked index (entry.cuh:18)
  float dist;
  bool visited;  // bit 63 (entry.cuh:31-38)
};

// CustomPairLess, beam_search/device_kernels.cuh:132-151: distance ascending,
// then 31-bit index ascending; the visited bit is ignored.
inline bool pair_less(const Entry& a, const Entry& b) {
  return (a.dist < b.dist) || (a.dist == b.dist && a.id < b.id);
}

struct Graph {
  const uint16_t* vecs;  // [n, dp] fp16 bits, zero padded rows
  int64_t n;
  int dp;                // padded dim (row stride, multiple of 8)
  const uint32_t* edges; // [n, R]
  const uint8_t* counts; // [n]
  int R;
  const uint32_t* deleted_bits;  // [(n+31)/32] or null
  int metric;            // 0 = L2, 1 = IP
};

struct SearchStats {
  uint64_t hops = 0;        // expansions (frontier nodes whose edges were read)
  uint64_t edges_read = 0;  // sum of degrees over expansions
  uint64_t dist_calls = 0;  // distances computed, reference-equivalent (all appended)
  uint64_t distinct = 0;    // distinct vertices whose distance was computed
};

// One query of beam_search_kernel, beam_search/beam_search.cuh:27-225, with
// the device helpers of device_kernels.cuh restated sequentially:
//   populate_distances :23-57, choose_new_frontier :60-92,
//   add_frontier_out :95-129, merge_sort :154-185 (CUB BlockMergeSort, taken
//   as stable), dedup_results :197-288, clip_k :188-193.
// Returns the final candidate buffer; appends (id, dist) of every popped
// node to `visited` when get_visited is set (beam_search.cuh:157-166).
std::vector<Entry> search_one(const Graph& g, const uint16_t* q, uint32_t medoid,
                              uint32_t bw, uint32_t limit, uint32_t max_result,
                              bool get_visited, std::vector<Entry>* visited,
                              SearchStats* st, std::vector<uint32_t>* seen_scratch) {
  std::vector<Entry> B;
  B.reserve(bw + 64 + 8);
  B.push_back({medoid & kInvalid31, FLT_MAX, false});
  auto compute = [&](Entry& e) {
    e.dist = dist(g.metric, q, g.vecs + (size_t)e.id * g.dp, g.dp);
    if (st) {
      st->dist_calls++;
      if (seen_scratch) seen_scratch->push_back(e.id);
    }
  };
  if (B[0].id != kInvalid31) compute(B[0]);

  uint32_t vc = 0, loop = 0;
  std::vector<Entry> merged;
  while (loop <= limit) {
    loop += 1;
    size_t p = B.size();
    for (size_t i = 0; i < B.size(); ++i)
      if (!B[i].visited) { p = i; break; }
    if (p == B.size()) break;
    B[p].visited = true;
    if (get_visited && visited) visited->push_back(B[p]);
    vc += 1;
    if (vc == max_result) break;

    const uint32_t u = B[p].id;
    const uint32_t deg = g.counts[u];
    const size_t offset = B.size();
    for (uint32_t e = 0; e < deg; ++e) {
      const uint32_t nb = g.edges[(size_t)u * g.R + e];
      if ((int64_t)nb < g.n) B.push_back({nb & kInvalid31, FLT_MAX, false});
      else B.push_back({kInvalid31, FLT_MAX, true});
    }
    if (st) { st->hops++; st->edges_read += deg; }
    for (size_t i = offset; i < B.size(); ++i)
      if (B[i].id != kInvalid31) compute(B[i]);

    std::stable_sort(B.begin(), B.end(), pair_less);
    merged.clear();
    uint32_t prev = kInvalid31;  // thread 0 compares against INVALID
    for (const Entry& e : B) {
      if (e.id != prev) merged.push_back(e);
      prev = e.id;
    }
    if (merged.size() > bw) merged.resize(bw);
    B.swap(merged);
  }
  return B;
}

// beam_search.cuh:207-222 (output of the first k valid, non-deleted entries;
// padding (0xFFFFFFFF, 1e30)) followed by translate_slots_to_ids_kernel
// (index/id_map.cuh:49-56) and unpack_results_kernel
// (ffi/jasper_ffi_common.cuh:193-203).
void write_output(const Graph& g, const std::vector<Entry>& B, uint32_t k,
                  const uint32_t* slot_to_id, int32_t* out_ids, float* out_dists) {
  uint32_t out = 0;
  for (size_t i = 0; i < B.size() && out < k; ++i) {
    const uint32_t idx = B[i].id;
    if ((int64_t)idx >= g.n) continue;
    if (g.deleted_bits && ((g.deleted_bits[idx >> 5] >> (idx & 31u)) & 1u)) continue;
    out_ids[out] = (int32_t)(slot_to_id ? slot_to_id[idx] : idx);
    out_dists[out] = B[i].dist;
    ++out;
  }
  for (; out < k; ++out) {
    out_ids[out] = (int32_t)0xFFFFFFFFu;
    out_dists[out] = 1e30f;
  }
}

// ------------------------------------------------------------------ build --

struct Cand {
  uint32_t id;
  float dist;
};

// EntryLess, index/construct.cuh:334-340 / :583-589.
inline bool cand_less(const Cand& a, const Cand& b) {
  if (a.dist != b.dist) return a.dist < b.dist;
  return a.id < b.id;
}

// RobustPrune, index/construct.cuh:419-472 (forward) and :680-729 (reverse):
// walk the sorted candidates; stop once R are selected; skip the node itself
// and INVALID; drop c if some already selected s has d(c, s) * alpha < d_c.
int robust_prune(const Graph& g, int dim_for_prune, uint32_t self,
                 const std::vector<Cand>& C, float alpha, int R, Cand* sel) {
  int ns = 0;
  for (const Cand& c : C) {
    if (ns >= R) break;
    if (c.id == self || c.id == kInvalid32) continue;
    const uint16_t* cv = g.vecs + (size_t)c.id * g.dp;
    bool pruned = false;
    for (int j = 0; j < ns; ++j) {
      const float d = dist(g.metric, cv, g.vecs + (size_t)sel[j].id * g.dp, dim_for_prune);
      const float lhs = d * alpha;
      if (lhs < c.dist) { pruned = true; break; }
    }
    if (!pruned) sel[ns++] = c;
  }
  return ns;
}

}  // namespace

// ================================================================ C ABI ====
extern "C" {

float jo_l2(const uint16_t* a, const uint16_t* b, int dim) { return l2_dist(a, b, dim); }
float jo_ip(const uint16_t* a, const uint16_t* b, int dim) { return ip_dist(a, b, dim); }

uint16_t jo_f2bf(float f) { return f2bf(f); }

// Pairwise distances for n pairs (rows of a and b, stride dp).
void jo_distance_pairs(int metric, const uint16_t* a, const uint16_t* b, int64_t n,
                       int dp, float* out, int nthreads) {
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i)
    out[i] = dist(metric, a + (size_t)i * dp, b + (size_t)i * dp, dp);
}

// Batched plain beam search (Appendix A of the contract; reference
// beam_search/beam_search.cuh + api.cuh). Queries are [nq, dp] fp16 bits.
// visited_* may be null; when given they are [nq, max_result].
// stats (may be null) receives per-query [hops, edges_read, dist_calls, distinct].
int jo_beam_search(const uint16_t* vecs, int64_t n, int dp,
                   const uint32_t* edges, const uint8_t* counts, int R,
                   const uint32_t* deleted_bits, const uint32_t* slot_to_id,
                   int metric, const uint16_t* queries, int64_t nq, uint32_t medoid,
                   int k, int bw, int limit, int max_result,
                   int32_t* out_ids, float* out_dists,
                   uint32_t* visited_ids, float* visited_dists, uint32_t* visited_counts,
                   uint64_t* stats, int nthreads) {
  Graph g{vecs, n, dp, edges, counts, R, deleted_bits, metric};
  if (nthreads > 0) omp_set_num_threads(nthreads);
  const bool get_visited = visited_ids != nullptr;
#pragma omp parallel
  {
    std::vector<Entry> vis;
    std::vector<uint32_t> seen;
#pragma omp for schedule(dynamic, 4)
    for (int64_t qi = 0; qi < nq; ++qi) {
      vis.clear();
      seen.clear();
      SearchStats st;
      std::vector<Entry> B = search_one(g, queries + (size_t)qi * dp, medoid, (uint32_t)bw,
                                        (uint32_t)limit, (uint32_t)max_result, get_visited,
                                        &vis, stats ? &st : nullptr, stats ? &seen : nullptr);
      if (out_ids) write_output(g, B, (uint32_t)k, slot_to_id, out_ids + qi * k, out_dists + qi * k);
      if (get_visited) {
        for (size_t i = 0; i < vis.size(); ++i) {
          visited_ids[qi * max_result + i] = vis[i].id;
          visited_dists[qi * max_result + i] = vis[i].dist;
        }
        visited_counts[qi] = (uint32_t)vis.size();
      }
      if (stats) {
        std::sort(seen.begin(), seen.end());
        st.distinct = (uint64_t)(std::unique(seen.begin(), seen.end()) - seen.begin());
        stats[qi * 4 + 0] = st.hops;
        stats[qi * 4 + 1] = st.edges_read;
        stats[qi * 4 + 2] = st.dist_calls;
        stats[qi * 4 + 3] = st.distinct;
      }
    }
  }
  return 0;
}

// Reference maximum batch size for a construction workspace budget:
// graph_construct_workspace::max_batch_size_for_budget (index/construct.cuh:238-262)
// capped at n/50 (ffi/jasper_ffi_common.cuh:245-248).
int64_t jo_max_batch_size(int64_t n, int R, int64_t budget_bytes) {
  const int64_t L = 64, max_result = 256, max_cands = max_result + R;
  const int64_t per_item = 8 * L + 8 * max_result + 4 + 8 * max_cands + 4 + 8 * R + 4 * R + 4 * R;
  const int64_t fixed = 4;
  int64_t b = budget_bytes <= fixed ? 0 : (budget_bytes - fixed) / per_item;
  b = std::min<int64_t>(b, 0xFFFFFFFFll);
  return std::min<int64_t>(b, n / 50);
}

// Vamana construction (Appendix D of the contract; reference
// index/construct.cuh construct_graph :992-1160, construction_round :913-958,
// process_batch :743-911). Input vectors [n, dp]; outputs edges [n, R] (u32),
// edge_dist [n, R] (bf16 bits), counts [n]. medoid = 0. max_batch must be >= 1.
// The beam search of each batch is the plain search above with k = L = 64,
// beam width 64, limit 256, max_result 256 (construct.cuh:57-62, :778-794).
//
// Candidate caps (256 + R) never bind in the forward step. In the reverse
// step the reference keeps an arrival-order subset when a target receives
// more than 256 + R candidates (atomicAdd, construct.cuh:642-658); this
// restatement fixes that order as: the target's existing edges in slot order,
// then the new sources in ascending id order.
namespace {

// process_reverse_edges_kernel (construct.cuh:560-741) over pairs
// (target << 32 | source) sorted ascending: per target, its existing edges in
// slot order, then the sources in ascending id order (capped at 256 + R),
// sorted by (distance, id), then RobustPrune. Also the repair step of
// consolidate (graph_ops.cuh:151-258), whose pairs are (live vertex, repair
// candidate).
// Target groups whose candidate list reached the 256 + R cap with sources
// left over, since the last jo_build (read by jo_last_capped_groups; a
// test counter, so tests can show the cap was exercised).
std::atomic<int64_t> g_capped_groups{0};

// Work counters of the last build's process_batches while jo_build_work is
// on (the device build's BuildWork indices): rows searched, pops, adjacency
// entries, distinct vectors scored, popped keys recorded; forward rows,
// existing edges, visited keys, candidates, edges written; reverse targets,
// existing edges, sources taken, edges written. Test infrastructure: the
// device counts of the same build must equal these.
std::atomic<bool> g_count_work{false};
std::atomic<uint64_t> g_work[16];


void reverse_step(const Graph& g, int dim_for_prune, float alpha, const std::vector<uint64_t>& pairs,
                  uint32_t* edges, uint16_t* edge_dist, uint8_t* counts) {
  const int R = g.R, max_cands = 256 + R;
  std::vector<size_t> heads;
  for (size_t p = 0; p < pairs.size(); ++p)
    if (p == 0 || (pairs[p] >> 32) != (pairs[p - 1] >> 32)) heads.push_back(p);
  heads.push_back(pairs.size());
#pragma omp parallel
  {
    std::vector<Cand> C;
    std::vector<Cand> sel((size_t)R);
    const int64_t n_groups = (int64_t)heads.size() - 1;
#pragma omp for schedule(dynamic, 1)
    for (int64_t h = 0; h < n_groups; ++h) {
      const uint32_t w = (uint32_t)(pairs[heads[(size_t)h]] >> 32);
      C.clear();
      for (uint32_t e = 0; e < counts[w]; ++e) {
        const uint32_t x = edges[(size_t)w * R + e];
        if (x == kInvalid32) continue;
        C.push_back({x, bf2f(edge_dist[(size_t)w * R + e])});
      }
      const size_t n_existing = C.size();
      const uint16_t* wv = g.vecs + (size_t)w * g.dp;
      for (size_t p = heads[(size_t)h]; p < heads[(size_t)h + 1]; ++p) {
        if ((int)C.size() >= max_cands) {
          g_capped_groups.fetch_add(1, std::memory_order_relaxed);
          break;
        }
        const uint32_t v = (uint32_t)(pairs[p] & 0xFFFFFFFFu);
        if (v == kInvalid32 || v == w) continue;
        C.push_back({v, dist(g.metric, wv, g.vecs + (size_t)v * g.dp, dim_for_prune)});
      }
      const size_t n_cands = C.size();
      std::sort(C.begin(), C.end(), cand_less);
      const int ns = robust_prune(g, dim_for_prune, w, C, alpha, R, sel.data());
      if (g_count_work.load()) {
        g_work[10] += 1;
        g_work[11] += n_existing;
        g_work[12] += n_cands - n_existing;
        g_work[13] += (uint64_t)ns;
      }
      for (int j = 0; j < ns; ++j) {
        edges[(size_t)w * R + j] = sel[(size_t)j].id;
        edge_dist[(size_t)w * R + j] = f2bf(sel[(size_t)j].dist);
      }
      counts[w] = (uint8_t)ns;
    }
  }
}

// process_batch (construct.cuh:743-911) over the vertices [first, last), in
// batches of 1, 2, 4, ... up to max_batch (construction) or of max_batch
// (append_batch, construct.cuh:1226-1241), searching from `medoid`.
int jo_rq_visit(const uint16_t* vecs, int64_t n, int dp, const uint32_t* edges, const uint8_t* counts, int R,
                int metric, int rq_dim, const uint8_t* rq_nodes, const float* rq_centroid, const uint16_t* q,
                uint32_t medoid, int bw, int limit, int max_result, uint32_t* vis_ids,
                float* vis_d);  // directional_oracle.cpp

// RaBitQ codes for the build search (jo_build_rq); null: the plain search.
struct RqBuild {
  int dim;
  const uint8_t* nodes;
  const float* centroid;
};

int64_t process_batches(const Graph& g, int dim_for_prune, float alpha, int64_t first, int64_t last,
                        int64_t max_batch, bool doubling, uint32_t medoid, uint32_t* edges,
                        uint16_t* edge_dist, uint8_t* counts, const RqBuild* rqb = nullptr) {
  const uint16_t* vecs = g.vecs;
  const int dp = g.dp, R = g.R;
  const int L = 64, LIMIT = 256, MAX_RESULT = 256;
  const int max_cands = MAX_RESULT + R;
  int64_t count = first, bs = doubling ? 1 : max_batch, nb = 0;
  std::vector<std::vector<Entry>> visited;
  std::vector<uint64_t> pairs;
  while (count < last) {
    bs = std::min<int64_t>(bs, last - count);
    bs = std::min<int64_t>(bs, max_batch);
    const int64_t s = count;
    visited.assign((size_t)bs, {});
    const bool cw = g_count_work.load();
    if (cw) g_work[0] += (uint64_t)bs;
    // (i) beam search of every batch vector against the pre-batch graph
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t i = 0; i < bs; ++i) {
      if (cw && !rqb) {
        SearchStats st;
        std::vector<uint32_t> seen;
        search_one(g, vecs + (size_t)(s + i) * dp, medoid, (uint32_t)L, (uint32_t)LIMIT,
                   (uint32_t)MAX_RESULT, true, &visited[(size_t)i], &st, &seen);
        std::sort(seen.begin(), seen.end());
        g_work[1] += st.hops;
        g_work[2] += st.edges_read;
        g_work[3] += (uint64_t)(std::unique(seen.begin(), seen.end()) - seen.begin());
        g_work[4] += visited[(size_t)i].size();
      } else if (rqb) {
        // the RaBitQ build search (directional_oracle.cpp, jo_rq_visit)
        uint32_t ids[MAX_RESULT];
        float ds[MAX_RESULT];
        const int nv = jo_rq_visit(vecs, g.n, dp, g.edges, g.counts, R, g.metric, rqb->dim, rqb->nodes,
                                   rqb->centroid, vecs + (size_t)(s + i) * dp, medoid, L, LIMIT, MAX_RESULT, ids, ds);
        for (int j = 0; j < nv; ++j) visited[(size_t)i].push_back({ids[j], ds[j], true});
      } else {
        search_one(g, vecs + (size_t)(s + i) * dp, medoid, (uint32_t)L, (uint32_t)LIMIT,
                   (uint32_t)MAX_RESULT, true, &visited[(size_t)i], nullptr, nullptr);
      }
    }
    // (ii)+(iii) merge_candidates_kernel + robust_prune_kernel
#pragma omp parallel
    {
      std::vector<Cand> C;
      std::vector<Cand> sel((size_t)R);
#pragma omp for schedule(dynamic, 1)
      for (int64_t i = 0; i < bs; ++i) {
        const uint32_t v = (uint32_t)(s + i);
        C.clear();
        for (uint32_t e = 0; e < counts[v]; ++e) {
          const uint32_t w = edges[(size_t)v * R + e];
          if (w == kInvalid32) continue;
          C.push_back({w, bf2f(edge_dist[(size_t)v * R + e])});
        }
        const size_t n_existing = C.size();
        for (const Entry& x : visited[(size_t)i])
          if (x.id != v && x.id != kInvalid32) C.push_back({x.id, x.dist});
        if ((int)C.size() > max_cands) C.resize((size_t)max_cands);
        std::sort(C.begin(), C.end(), cand_less);
        const int ns = robust_prune(g, dim_for_prune, v, C, alpha, R, sel.data());
        if (cw) {
          g_work[5] += 1;
          g_work[6] += n_existing;
          g_work[7] += visited[(size_t)i].size();
          g_work[8] += C.size();
          g_work[9] += (uint64_t)ns;
        }
        for (int j = 0; j < ns; ++j) {
          edges[(size_t)v * R + j] = sel[(size_t)j].id;
          edge_dist[(size_t)v * R + j] = f2bf(sel[(size_t)j].dist);
        }
        counts[v] = (uint8_t)ns;
      }
    }
    // (iv)+(v) reverse pairs (target << 32 | source), grouped by target
    pairs.clear();
    for (int64_t i = 0; i < bs; ++i) {
      const uint32_t v = (uint32_t)(s + i);
      for (uint32_t e = 0; e < counts[v]; ++e)
        pairs.push_back(((uint64_t)edges[(size_t)v * R + e] << 32) | v);
    }
    std::sort(pairs.begin(), pairs.end());
    // (vi) process_reverse_edges_kernel
    reverse_step(g, dim_for_prune, alpha, pairs, edges, edge_dist, counts);
    count += bs;
    ++nb;
    if (doubling && bs < max_batch) bs = std::min<int64_t>(max_batch, bs * 2);
  }
  return nb;
}

}  // namespace

int jo_build(const uint16_t* vecs, int64_t n, int dp, int dim_for_prune, int R, int metric,
             float alpha, int64_t max_batch, uint32_t* edges, uint16_t* edge_dist,
             uint8_t* counts, int nthreads, int64_t* n_batches_out) {
  if (n <= 0) return 0;
  if (max_batch < 1) return -1;
  if (nthreads > 0) omp_set_num_threads(nthreads);
  g_capped_groups.store(0);
  std::fill(counts, counts + n, (uint8_t)0);
  std::fill(edges, edges + (size_t)n * R, kInvalid32);
  std::fill(edge_dist, edge_dist + (size_t)n * R, (uint16_t)0);
  Graph g{vecs, n, dp, edges, counts, R, nullptr, metric};
  const int64_t nb = process_batches(g, dim_for_prune, alpha, 0, n, max_batch, true, 0u, edges, edge_dist, counts);
  if (n_batches_out) *n_batches_out = nb;
  return 0;
}

int64_t jo_last_capped_groups() { return g_capped_groups.load(); }

// Work counting of the following builds (see g_work): on != 0 clears the
// counters and turns counting on, 0 turns it off.
void jo_build_work(int on) {
  if (on)
    for (auto& w : g_work) w.store(0);
  g_count_work.store(on != 0);
}

void jo_last_build_work(uint64_t* out16) {
  for (int i = 0; i < 16; ++i) out16[i] = g_work[i].load();
}

// jo_build with the RaBitQ build search (rabitq_build_search): the search
// stage pops by the RaBitQ estimate of the given codes (nodes [n,
// code_bytes + 8] of the rows as stored, centroid [rq_dim]).
int jo_build_rq(const uint16_t* vecs, int64_t n, int dp, int dim_for_prune, int R, int metric, float alpha,
                int64_t max_batch, int rq_dim, const uint8_t* rq_nodes, const float* rq_centroid, uint32_t* edges,
                uint16_t* edge_dist, uint8_t* counts, int nthreads, int64_t* n_batches_out) {
  if (n <= 0) return 0;
  if (max_batch < 1 || rq_dim <= 0 || rq_dim > 256) return -1;
  if (nthreads > 0) omp_set_num_threads(nthreads);
  g_capped_groups.store(0);
  std::fill(counts, counts + n, (uint8_t)0);
  std::fill(edges, edges + (size_t)n * R, kInvalid32);
  std::fill(edge_dist, edge_dist + (size_t)n * R, (uint16_t)0);
  Graph g{vecs, n, dp, edges, counts, R, nullptr, metric};
  const RqBuild rqb{rq_dim, rq_nodes, rq_centroid};
  const int64_t nb =
      process_batches(g, dim_for_prune, alpha, 0, n, max_batch, true, 0u, edges, edge_dist, counts, &rqb);
  if (n_batches_out) *n_batches_out = nb;
  return 0;
}

// ------------------------------------------------------- partitioned build --
// intermediate_graph (reference index/construct_scale.cuh:68-330 with
// construct_scale_kernels.cuh:23-330): the rows are cut into n_parts
// contiguous partitions of ceil(n / n_parts) rows, each built on its own
// (construct_graph with batches doubling up to part_batch), its edge ids
// shifted to global ids; then every unordered pair of partitions is merged
// once, in the reference's cyclic order (merge(), :391-450). A merge (B1,
// B2) walks B1 in batches of merge_batch (not crossing a 2^20-row segment
// boundary of B1, :358-365) and per batch:
//   (i)   searches B2's graph with each batch row (k = L = 64, beam width
//         64, limit 256, 256 visits kept); B2's edges to other partitions
//         are out of its range and skipped;
//   (ii)  per batch row: its edges and the visits (as global ids), sorted by
//         (distance, id), then the merge prune below, into B1;
//   (iii) reverse pairs (neighbour, row) of the batch's new rows whose
//         neighbour is in B2, grouped by neighbour; per B2 target: its
//         edges, then the sources (distances computed; this restatement
//         takes them in ascending id), capped at 256 + R, sorted, then the
//         merge prune, into B2.
// The merge prune (robust_prune_kernel_scale, :23-139) keeps a candidate
// whose vector is in neither partition without testing it, and tests
// candidates only against selected members whose vectors are in B1 or B2.
namespace {

struct ScaleRange {
  const uint16_t* vecs;
  int dp;
  int64_t b1s, n1, b2s, n2;
  const uint16_t* row(uint32_t id) const {
    if ((int64_t)id >= b1s && (int64_t)id < b1s + n1) return vecs + (size_t)id * dp;
    if ((int64_t)id >= b2s && (int64_t)id < b2s + n2) return vecs + (size_t)id * dp;
    return nullptr;
  }
};

int robust_prune_scale(const ScaleRange& sr, int metric, int dim_for_prune, uint32_t self,
                       const std::vector<Cand>& C, float alpha, int R, Cand* sel) {
  int ns = 0;
  for (const Cand& c : C) {
    if (ns >= R) break;
    if (c.id == self || c.id == kInvalid32) continue;
    const uint16_t* cv = sr.row(c.id);
    if (!cv) {  // "we cant prune this, but we need to keep it"
      sel[ns++] = c;
      continue;
    }
    bool pruned = false;
    for (int j = 0; j < ns && !pruned; ++j) {
      const uint16_t* sv = sr.row(sel[j].id);
      if (!sv) continue;
      if (dist(metric, cv, sv, dim_for_prune) * alpha < c.dist) pruned = true;
    }
    if (!pruned) sel[ns++] = c;
  }
  return ns;
}

void scale_merge(const uint16_t* vecs, int dp, int dim_for_prune, int R, int metric, float alpha, int64_t b1s,
                 int64_t n1, int64_t b2s, int64_t n2, int64_t merge_batch, uint32_t* edges, uint16_t* edge_dist,
                 uint8_t* counts) {
  const int L = 64, LIMIT = 256, MAX_RESULT = 256, max_cands = MAX_RESULT + R;
  const int64_t kSegment = (int64_t)1 << 20;
  const ScaleRange sr{vecs, dp, b1s, n1, b2s, n2};
  std::vector<uint32_t> local((size_t)n2 * R);
  std::vector<std::vector<Entry>> visited;
  std::vector<uint64_t> pairs;
  int64_t count = 0;
  while (count < n1) {
    const int64_t bs = std::min({merge_batch, n1 - count, kSegment - count % kSegment});
    // B2's adjacency with ids local to B2 (others past its range)
    for (int64_t w = 0; w < n2; ++w)
      for (int e = 0; e < R; ++e) {
        const uint32_t x = edges[(size_t)(b2s + w) * R + e];
        local[(size_t)w * R + e] = ((int64_t)x >= b2s && (int64_t)x < b2s + n2) ? (uint32_t)(x - b2s) : kInvalid32;
      }
    const Graph g2{vecs + (size_t)b2s * dp, n2, dp, local.data(), counts + b2s, R, nullptr, metric};
    visited.assign((size_t)bs, {});
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t i = 0; i < bs; ++i)
      search_one(g2, vecs + (size_t)(b1s + count + i) * dp, 0u, (uint32_t)L, (uint32_t)LIMIT, (uint32_t)MAX_RESULT,
                 true, &visited[(size_t)i], nullptr, nullptr);
#pragma omp parallel
    {
      std::vector<Cand> C;
      std::vector<Cand> sel((size_t)R);
#pragma omp for schedule(dynamic, 1)
      for (int64_t i = 0; i < bs; ++i) {
        const uint32_t v = (uint32_t)(b1s + count + i);
        C.clear();
        for (uint32_t e = 0; e < counts[v]; ++e) {
          const uint32_t w = edges[(size_t)v * R + e];
          if (w == kInvalid32) continue;
          C.push_back({w, bf2f(edge_dist[(size_t)v * R + e])});
        }
        for (const Entry& x : visited[(size_t)i]) {
          const uint32_t gid = x.id == kInvalid31 ? kInvalid32 : (uint32_t)(b2s + x.id);
          if (gid != v && gid != kInvalid32) C.push_back({gid, x.dist});
        }
        if ((int)C.size() > max_cands) C.resize((size_t)max_cands);
        std::sort(C.begin(), C.end(), cand_less);
        const int ns = robust_prune_scale(sr, metric, dim_for_prune, v, C, alpha, R, sel.data());
        for (int j = 0; j < ns; ++j) {
          edges[(size_t)v * R + j] = sel[(size_t)j].id;
          edge_dist[(size_t)v * R + j] = f2bf(sel[(size_t)j].dist);
        }
        counts[v] = (uint8_t)ns;
      }
    }
    pairs.clear();
    for (int64_t i = 0; i < bs; ++i) {
      const uint32_t v = (uint32_t)(b1s + count + i);
      for (uint32_t e = 0; e < counts[v]; ++e) {
        const uint32_t w = edges[(size_t)v * R + e];
        if ((int64_t)w >= b2s && (int64_t)w < b2s + n2) pairs.push_back(((uint64_t)w << 32) | v);
      }
    }
    std::sort(pairs.begin(), pairs.end());
    std::vector<size_t> heads;
    for (size_t q = 0; q < pairs.size(); ++q)
      if (q == 0 || (pairs[q] >> 32) != (pairs[q - 1] >> 32)) heads.push_back(q);
    heads.push_back(pairs.size());
#pragma omp parallel
    {
      std::vector<Cand> C;
      std::vector<Cand> sel((size_t)R);
      const int64_t n_groups = (int64_t)heads.size() - 1;
#pragma omp for schedule(dynamic, 1)
      for (int64_t h = 0; h < n_groups; ++h) {
        const uint32_t w = (uint32_t)(pairs[heads[(size_t)h]] >> 32);
        C.clear();
        for (uint32_t e = 0; e < counts[w]; ++e) {
          const uint32_t x = edges[(size_t)w * R + e];
          if (x == kInvalid32) continue;
          C.push_back({x, bf2f(edge_dist[(size_t)w * R + e])});
        }
        const uint16_t* wv = vecs + (size_t)w * dp;
        for (size_t q = heads[(size_t)h]; q < heads[(size_t)h + 1]; ++q) {
          if ((int)C.size() >= max_cands) break;
          const uint32_t v = (uint32_t)(pairs[q] & 0xFFFFFFFFu);
          if (v == w) continue;
          const uint16_t* vv = sr.row(v);
          if (!vv) continue;
          C.push_back({v, dist(metric, wv, vv, dim_for_prune)});
        }
        std::sort(C.begin(), C.end(), cand_less);
        const int ns = robust_prune_scale(sr, metric, dim_for_prune, w, C, alpha, R, sel.data());
        for (int j = 0; j < ns; ++j) {
          edges[(size_t)w * R + j] = sel[(size_t)j].id;
          edge_dist[(size_t)w * R + j] = f2bf(sel[(size_t)j].dist);
        }
        counts[w] = (uint8_t)ns;
      }
    }
    count += bs;
  }
}

}  // namespace

// The merge order of intermediate_graph::merge (construct_scale.cuh:386-445):
// for each interval itv = 1 .. P/2 the pairs (B1, B1 + itv mod P) walk
// cycles of P / gcd(itv, P) calls (one call when the cycle has length 2), B1
// taking the previous call's B2, and the next cycle starting one partition
// further on. Writes (B1, B2) pairs to out; returns the number of merges.
int64_t jo_scale_merge_order(int64_t P, int64_t* out) {
  int64_t B1 = 0, m = 0;
  for (int64_t itv = 1; itv <= P / 2; ++itv) {
    const int64_t gg = std::gcd(itv, P), cycle_len = P / gg;
    const int64_t calls = cycle_len == 2 ? 1 : cycle_len;
    for (int64_t cyc = 0; cyc < gg; ++cyc) {
      if (cyc > 0) B1 = (B1 + 1) % P;
      for (int64_t step = 0; step < calls; ++step) {
        const int64_t B2 = (B1 + itv) % P;
        out[2 * m] = B1;
        out[2 * m + 1] = B2;
        ++m;
        B1 = B2;
      }
    }
  }
  return m;
}

// The partitioned build above. Outputs as jo_build (global ids); medoid = 0.
// Returns -1 on bad arguments (a partition would be empty).
int jo_build_scale(const uint16_t* vecs, int64_t n, int dp, int dim_for_prune, int R, int metric, float alpha,
                   int64_t n_parts, int64_t part_batch, int64_t merge_batch, uint32_t* edges, uint16_t* edge_dist,
                   uint8_t* counts, int nthreads) {
  if (n <= 0) return 0;
  if (n_parts < 1 || part_batch < 1 || merge_batch < 1) return -1;
  const int64_t part = (n + n_parts - 1) / n_parts;
  if (part * (n_parts - 1) >= n) return -1;
  if (nthreads > 0) omp_set_num_threads(nthreads);
  g_capped_groups.store(0);
  std::fill(counts, counts + n, (uint8_t)0);
  std::fill(edges, edges + (size_t)n * R, kInvalid32);
  std::fill(edge_dist, edge_dist + (size_t)n * R, (uint16_t)0);
  for (int64_t p = 0; p < n_parts; ++p) {
    const int64_t s = p * part, c = std::min(part, n - s);
    uint32_t* e = edges + (size_t)s * R;
    Graph g{vecs + (size_t)s * dp, c, dp, e, counts + s, R, nullptr, metric};
    process_batches(g, dim_for_prune, alpha, 0, c, part_batch, true, 0u, e, edge_dist + (size_t)s * R, counts + s);
    for (int64_t i = 0; i < c; ++i)
      for (uint32_t j = 0; j < counts[s + i]; ++j) e[(size_t)i * R + j] += (uint32_t)s;
  }
  std::vector<int64_t> order((size_t)(n_parts * (n_parts - 1)));
  const int64_t n_merges = jo_scale_merge_order(n_parts, order.data());
  for (int64_t m = 0; m < n_merges; ++m) {
    const int64_t b1s = order[(size_t)(2 * m)] * part, b2s = order[(size_t)(2 * m + 1)] * part;
    scale_merge(vecs, dp, dim_for_prune, R, metric, alpha, b1s, std::min(part, n - b1s), b2s,
                std::min(part, n - b2s), merge_batch, edges, edge_dist, counts);
  }
  return 0;
}

// The merge prune on one hand-made candidate list (test hook): B1 = rows
// [b1s, b1s + n1), B2 = rows [b2s, b2s + n2) of vecs; candidates already
// sorted. Returns the number selected.
int jo_prune_scale(const uint16_t* vecs, int dp, int dim_for_prune, int metric, float alpha, int R, int64_t b1s,
                   int64_t n1, int64_t b2s, int64_t n2, uint32_t self, const uint32_t* cand_ids,
                   const float* cand_dists, int n_cands, uint32_t* out_ids, float* out_dists) {
  const ScaleRange sr{vecs, dp, b1s, n1, b2s, n2};
  std::vector<Cand> C((size_t)n_cands);
  for (int i = 0; i < n_cands; ++i) C[(size_t)i] = {cand_ids[i], cand_dists[i]};
  std::vector<Cand> sel((size_t)R);
  const int ns = robust_prune_scale(sr, metric, dim_for_prune, self, C, alpha, R, sel.data());
  for (int j = 0; j < ns; ++j) {
    out_ids[j] = sel[(size_t)j].id;
    out_dists[j] = sel[(size_t)j].dist;
  }
  return ns;
}

// append_batch (construct.cuh:1169-1265): the rows [first, n) were appended
// to a graph of `first` vertices (their counts must be 0); wires them in with
// process_batch in batches of max_batch (the reference's default is
// min(count, 100000)), searching from `medoid`. Deleted vertices stay in the
// graph and are traversed like the reference's construction search does.
int jo_append(const uint16_t* vecs, int64_t n, int dp, int dim_for_prune, int R, int metric, float alpha,
              int64_t first, int64_t max_batch, uint32_t medoid, const uint32_t* deleted_bits, uint32_t* edges,
              uint16_t* edge_dist, uint8_t* counts, int nthreads, int64_t* n_batches_out) {
  if (first < 0 || first > n || max_batch < 1) return -1;
  if (nthreads > 0) omp_set_num_threads(nthreads);
  Graph g{vecs, n, dp, edges, counts, R, deleted_bits, metric};
  const int64_t nb =
      process_batches(g, dim_for_prune, alpha, first, n, max_batch, false, medoid, edges, edge_dist, counts);
  if (n_batches_out) *n_batches_out = nb;
  return 0;
}

// consolidate (graph_ops.cuh:151-258, deletion.cuh:45-174): for every live
// vertex N, each live neighbour M != N of each deleted neighbour D of N is a
// repair candidate (N, M) (count/fill_repair_candidates_kernel, in N's edge
// order, then D's); deleted neighbours are dropped from the live lists
// (compact_deleted_neighbors_kernel, order kept, distances moved along); the
// candidates are grouped by N with M ascending and merged and pruned as the
// reverse step of construction; then the deleted vertices' lists are cleared
// and every tombstone is reset. Returns the number of repair candidates.
int64_t jo_consolidate(const uint16_t* vecs, int64_t n, int dp, int dim_for_prune, int R, int metric, float alpha,
                       uint32_t* deleted_bits, uint32_t* edges, uint16_t* edge_dist, uint8_t* counts,
                       int nthreads) {
  if (nthreads > 0) omp_set_num_threads(nthreads);
  auto is_del = [&](uint32_t v) { return ((deleted_bits[v >> 5] >> (v & 31u)) & 1u) != 0u; };
  std::vector<uint64_t> pairs;
  for (int64_t N = 0; N < n; ++N) {
    if (is_del((uint32_t)N)) continue;
    for (uint32_t j = 0; j < counts[N]; ++j) {
      const uint32_t D = edges[(size_t)N * R + j];
      if (D == kInvalid32 || (int64_t)D >= n || !is_del(D)) continue;
      for (uint32_t k = 0; k < counts[D]; ++k) {
        const uint32_t M = edges[(size_t)D * R + k];
        if (M == kInvalid32 || (int64_t)M >= n) continue;
        if (is_del(M) || M == (uint32_t)N) continue;
        pairs.push_back(((uint64_t)N << 32) | M);
      }
    }
  }
  for (int64_t N = 0; N < n; ++N) {
    if (is_del((uint32_t)N)) continue;
    uint32_t nc = 0;
    for (uint32_t j = 0; j < counts[N]; ++j) {
      const uint32_t nb = edges[(size_t)N * R + j];
      if (nb == kInvalid32 || (int64_t)nb >= n || is_del(nb)) continue;
      edges[(size_t)N * R + nc] = nb;
      edge_dist[(size_t)N * R + nc] = edge_dist[(size_t)N * R + j];
      ++nc;
    }
    counts[N] = (uint8_t)nc;
  }
  std::sort(pairs.begin(), pairs.end());
  Graph g{vecs, n, dp, edges, counts, R, nullptr, metric};
  reverse_step(g, dim_for_prune, alpha, pairs, edges, edge_dist, counts);
  for (int64_t D = 0; D < n; ++D) {
    if (!is_del((uint32_t)D)) continue;
    std::fill(edges + (size_t)D * R, edges + (size_t)(D + 1) * R, kInvalid32);
    counts[D] = 0;
  }
  std::fill(deleted_bits, deleted_bits + (n + 31) / 32, 0u);
  return (int64_t)pairs.size();
}

// Exact kNN by the contract's distance (l2_dist / ip_dist), top-k by
// (dist, id). Used as ground truth on small configs.
void jo_bruteforce_exact(int metric, const uint16_t* vecs, int64_t n, const uint16_t* queries,
                         int64_t nq, int dp, int k, int32_t* out_ids, float* out_dists,
                         int nthreads) {
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
  {
    std::vector<Cand> all((size_t)n);
#pragma omp for schedule(dynamic, 1)
    for (int64_t qi = 0; qi < nq; ++qi) {
      const uint16_t* q = queries + (size_t)qi * dp;
      for (int64_t i = 0; i < n; ++i)
        all[(size_t)i] = {(uint32_t)i, dist(metric, q, vecs + (size_t)i * dp, dp)};
      const int kk = (int)std::min<int64_t>(k, n);
      std::partial_sort(all.begin(), all.begin() + kk, all.end(), cand_less);
      for (int j = 0; j < k; ++j) {
        out_ids[qi * k + j] = j < kk ? (int32_t)all[(size_t)j].id : -1;
        out_dists[qi * k + j] = j < kk ? all[(size_t)j].dist : FLT_MAX;
      }
    }
  }
}

// The reference's ground-truth arithmetic, python/jasper/__init__.py:828-926:
// L2 = ||q||^2 + ||v||^2 - 2 q.v in fp32, clamped at 0; IP = -(q.v), where
// with fp16 inputs the matmul result is fp16 (ip_round_fp16 != 0 rounds q.v
// to fp16 before the negation). Dot products accumulate sequentially in fp32
// (torch's order is unspecified). Also the CPU baseline "exact kNN scan".
// Vectors are pre-converted to fp32.
extern "C" uint16_t jo_d2h(double x);  // directional_oracle.cpp: double -> fp16, RNE

static float round_to_fp16(float x) {
  const uint16_t h = jo_d2h((double)x);
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  float v;
  if (e == 0) v = std::ldexp((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = std::ldexp((float)(m | 0x400u), (int)e - 25);
  return sign ? -v : v;
}

void jo_bruteforce_ref(int metric, const float* vecs, int64_t n, const float* queries,
                       int64_t nq, int dim, int k, int32_t* out_ids, float* out_dists,
                       int nthreads, int ip_round_fp16) {
  if (nthreads > 0) omp_set_num_threads(nthreads);
  std::vector<float> vsq((size_t)n, 0.0f);
  if (metric == 0) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
      float s = 0.0f;
      const float* v = vecs + (size_t)i * dim;
      for (int t = 0; t < dim; ++t) s += v[t] * v[t];
      vsq[(size_t)i] = s;
    }
  }
#pragma omp parallel
  {
    std::vector<Cand> heap;
#pragma omp for schedule(dynamic, 1)
    for (int64_t qi = 0; qi < nq; ++qi) {
      const float* q = queries + (size_t)qi * dim;
      float qsq = 0.0f;
      for (int t = 0; t < dim; ++t) qsq += q[t] * q[t];
      heap.clear();
      auto worse = [](const Cand& a, const Cand& b) { return cand_less(a, b); };
      for (int64_t i = 0; i < n; ++i) {
        const float* v = vecs + (size_t)i * dim;
        float dot = 0.0f;
        for (int t = 0; t < dim; ++t) dot += q[t] * v[t];
        float d;
        if (metric == 0) {
          d = qsq + vsq[(size_t)i] - 2.0f * dot;
          if (d < 0.0f) d = 0.0f;
        } else {
          d = ip_round_fp16 ? -round_to_fp16(dot) : -dot;
        }
        const Cand c{(uint32_t)i, d};
        if ((int)heap.size() < k) {
          heap.push_back(c);
          std::push_heap(heap.begin(), heap.end(), worse);
        } else if (cand_less(c, heap.front())) {
          std::pop_heap(heap.begin(), heap.end(), worse);
          heap.back() = c;
          std::push_heap(heap.begin(), heap.end(), worse);
        }
      }
      std::sort(heap.begin(), heap.end(), cand_less);
      for (int j = 0; j < k; ++j) {
        out_ids[qi * k + j] = j < (int)heap.size() ? (int32_t)heap[(size_t)j].id : -1;
        out_dists[qi * k + j] = j < (int)heap.size() ? heap[(size_t)j].dist : FLT_MAX;
      }
    }
  }
}

// The Gaussian matrix set_rotation_matrix factorises (rotation.cuh:81-88),
// column-major; exposed so tests can check Q against an independent QR.
void jo_gaussian_matrix(int d, uint64_t seed, float* A) {
  std::mt19937_64 rng(seed);
  std::normal_distribution<float> N(0, 1);
  for (int j = 0; j < d; j++)
    for (int i = 0; i < d; i++) A[(size_t)i + (size_t)j * d] = N(rng);
}

// Random orthogonal matrix, rotation/rotation.cuh:28-111 (householder_qr +
// set_rotation_matrix): A ~ N(0,1) column-major from std::mt19937_64(seed)
// and std::normal_distribution<float>; Householder QR in float; columns of Q
// flipped where diag(R) < 0. Outputs m = Q and mt = Q^T, both column-major.
void jo_rotation_matrix(int d, uint64_t seed, float* m, float* mt) {
  std::mt19937_64 rng(seed);
  std::normal_distribution<float> N(0, 1);
  std::vector<float> A((size_t)d * d);
  for (int j = 0; j < d; j++)
    for (int i = 0; i < d; i++) A[(size_t)i + (size_t)j * d] = N(rng);

  std::vector<float> Q((size_t)d * d, 0.0f);
  for (int i = 0; i < d; i++) Q[(size_t)i + (size_t)i * d] = 1.0f;
  std::vector<float> v((size_t)d);
  for (int k = 0; k < d; k++) {
    float norm_sq = 0;
    for (int i = k; i < d; i++) {
      v[i] = A[(size_t)i + (size_t)k * d];
      norm_sq += v[i] * v[i];
    }
    float norm = std::sqrt(norm_sq);
    if (norm < 1e-12f) continue;
    float sign = (A[(size_t)k + (size_t)k * d] >= 0) ? 1.0f : -1.0f;
    v[k] += sign * norm;
    float v_norm_sq = 0;
    for (int i = k; i < d; i++) v_norm_sq += v[i] * v[i];
    float tau = 2.0f / v_norm_sq;
    for (int j = k; j < d; j++) {
      float dot = 0;
      for (int i = k; i < d; i++) dot += v[i] * A[(size_t)i + (size_t)j * d];
      for (int i = k; i < d; i++) A[(size_t)i + (size_t)j * d] -= tau * v[i] * dot;
    }
    for (int j = 0; j < d; j++) {
      float dot = 0;
      for (int i = k; i < d; i++) dot += v[i] * Q[(size_t)i + (size_t)j * d];
      for (int i = k; i < d; i++) Q[(size_t)i + (size_t)j * d] -= tau * v[i] * dot;
    }
  }
  for (int i = 0; i < d; i++) {
    if (A[(size_t)i + (size_t)i * d] < 0.0f) {
      for (int j = 0; j < d; j++) Q[(size_t)j + (size_t)i * d] *= -1.0f;
    }
  }
  for (int j = 0; j < d; j++) {
    for (int i = 0; i < d; i++) {
      m[(size_t)i + (size_t)j * d] = Q[(size_t)i + (size_t)j * d];
      mt[(size_t)i + (size_t)j * d] = Q[(size_t)j + (size_t)i * d];
    }
  }
}

// --------------------------------------------------------- DiskANN build --
// construct_diskann.cuh (driven by cmd/create_diskann_index.cu:59-103).
//
// assign_shards (:104-276, kernels construct_diskann_kernels.cuh:15-139):
//   mean: rows 0, s, 2s, ... with s = max(1, n / min(n, 2,000,000)), summed
//     per coordinate in double, divided by the row count, rounded to fp16;
//   each row centred in fp16 (v - mean, one rounding), rotated by P (the
//     rotation matrix for `seed` rounded to fp16): r_i = fp16(sum_k
//     P[k + i*dim] * c_k) with fp32 accumulation (cublasGemmEx, op T; its
//     summation order is unspecified: here k ascending, one fma per term);
//   keys (|bits(r_i)| << 16) | i; n_dup times: the largest key wins, its
//     coordinate and sign give bucket 2 coord + sign and shard bucket mod
//     n_parts (INVALID when an earlier rank chose the same shard), then the
//     winner's key is cleared.
// Shard lists hold global ids in ascending order.
static uint16_t hsub16(uint16_t a, uint16_t b) { return jo_d2h((double)h2f(a) - (double)h2f(b)); }

int jo_diskann_assign(const uint16_t* vecs, int64_t n, int dp, int dim, int n_parts, int n_dup, uint64_t seed,
                      uint32_t* shard_of, uint16_t* mean_out) {
  if (n <= 0 || dim <= 0 || n_parts < 1 || n_dup < 1 || dp < dim || dp > 65536) return -1;
  const int64_t target = std::min<int64_t>(n, 2000000);
  const int64_t stride = std::max<int64_t>(1, n / target);
  std::vector<double> acc((size_t)dim, 0.0);
  int64_t sampled = 0;
  for (int64_t i = 0; i < n; i += stride) {
    for (int d = 0; d < dim; ++d) acc[(size_t)d] += (double)h2f(vecs[(size_t)i * dp + d]);
    ++sampled;
  }
  std::vector<uint16_t> mean((size_t)dim);
  for (int d = 0; d < dim; ++d) mean[(size_t)d] = jo_d2h(acc[(size_t)d] / (double)std::max<int64_t>(1, sampled));
  if (mean_out) std::copy(mean.begin(), mean.end(), mean_out);
  std::vector<float> P((size_t)dim * dim), Pt((size_t)dim * dim);
  jo_rotation_matrix(dim, seed, P.data(), Pt.data());
  std::vector<float> P16((size_t)dim * dim);
  for (size_t i = 0; i < P.size(); ++i) P16[i] = h2f(jo_d2h((double)P[i]));
#pragma omp parallel
  {
    std::vector<float> c((size_t)dim);
    std::vector<uint16_t> rot((size_t)dim);
    std::vector<uint32_t> keys((size_t)dp);
#pragma omp for schedule(static)
    for (int64_t v = 0; v < n; ++v) {
      const uint16_t* x = vecs + (size_t)v * dp;
      for (int k = 0; k < dim; ++k) c[(size_t)k] = h2f(hsub16(x[k], mean[(size_t)k]));
      for (int i = 0; i < dim; ++i) {
        float a = 0.0f;
        const float* col = P16.data() + (size_t)i * dim;
        for (int k = 0; k < dim; ++k) a = std::fmaf(col[k], c[(size_t)k], a);
        rot[(size_t)i] = jo_d2h((double)a);
      }
      for (int i = 0; i < dp; ++i)
        keys[(size_t)i] = i < dim ? ((uint32_t)(rot[(size_t)i] & 0x7FFFu) << 16) | (uint32_t)i : 0u;
      uint32_t* out = shard_of + (size_t)v * n_dup;
      for (int r = 0; r < n_dup; ++r) {
        uint32_t win = 0;
        for (int i = 0; i < dp; ++i) win = std::max(win, keys[(size_t)i]);
        const uint32_t coord = win & 0xFFFFu;
        const uint32_t sign = (rot[coord] >> 15) & 1u;
        const uint32_t shard = (2u * coord + sign) % (uint32_t)n_parts;
        bool dup = false;
        for (int t = 0; t < r; ++t) dup = dup || out[t] == shard;
        out[r] = dup ? kInvalid32 : shard;
        keys[coord] = 0;
      }
    }
  }
  return 0;
}

// diskann_intermediate_graph::build (:328-613): shards that are not empty
// become tasks, largest first (the reference's std::sort leaves equal sizes
// in an unspecified order: here ascending shard index). Each task: its rows
// (ascending global id) built as their own graph of degree R_int (the plain
// construction, batches doubling to max(1, min(batch_cap, count)), search
// from its first row), neighbour ids mapped to global ids, then merge_row
// (:278-325) for every row: the final row's entries then the shard row's,
// stably sorted by stored (bf16) distance, the first R_fin distinct ids
// kept. Merges run one task after another. medoid = 0.
int jo_build_diskann(const uint16_t* vecs, int64_t n, int dp, int dim_for_prune, int R_int, int R_fin, int metric,
                     float alpha, int n_parts, int n_dup, uint64_t seed, int64_t batch_cap, int64_t max_shard,
                     uint32_t* edges, uint16_t* edge_dist, uint8_t* counts, uint32_t* shard_of_out, int nthreads) {
  if (n <= 0 || R_int < 1 || R_fin < 1 || R_int > 255 || R_fin > 255 || batch_cap < 1) return -1;
  if (nthreads > 0) omp_set_num_threads(nthreads);
  std::vector<uint32_t> shard_of((size_t)n * n_dup);
  if (jo_diskann_assign(vecs, n, dp, dim_for_prune, n_parts, n_dup, seed, shard_of.data(), nullptr) != 0)
    return -1;
  if (shard_of_out) std::copy(shard_of.begin(), shard_of.end(), shard_of_out);
  std::vector<std::vector<uint32_t>> shard_ids((size_t)n_parts);
  for (int64_t v = 0; v < n; ++v)
    for (int r = 0; r < n_dup; ++r) {
      const uint32_t s = shard_of[(size_t)v * n_dup + r];
      if (s != kInvalid32) shard_ids[s].push_back((uint32_t)v);
    }
  // build tasks (construct_diskann.cuh:386-417): a shard above max_shard
  // rows (max_shard > 0) splits into equal sub-shards of its ascending ids;
  // largest first, ties in (shard, sub-shard) order
  struct Task {
    int part;
    int64_t begin, len;
  };
  std::vector<Task> tasks;
  for (int p = 0; p < n_parts; ++p) {
    const int64_t total = (int64_t)shard_ids[(size_t)p].size();
    if (total == 0) continue;
    const int64_t n_sub = max_shard > 0 ? (total + max_shard - 1) / max_shard : 1;
    const int64_t sub = (total + n_sub - 1) / n_sub;
    for (int64_t b = 0; b < total; b += sub) tasks.push_back({p, b, std::min(sub, total - b)});
  }
  std::stable_sort(tasks.begin(), tasks.end(), [](const Task& a, const Task& b) { return a.len > b.len; });
  std::fill(counts, counts + n, (uint8_t)0);
  std::fill(edges, edges + (size_t)n * R_fin, kInvalid32);
  std::fill(edge_dist, edge_dist + (size_t)n * R_fin, (uint16_t)0);
  g_capped_groups.store(0);
  for (const Task& task : tasks) {
    const std::vector<uint32_t> ids(shard_ids[(size_t)task.part].begin() + task.begin,
                                    shard_ids[(size_t)task.part].begin() + task.begin + task.len);
    const int64_t c = (int64_t)ids.size();
    std::vector<uint16_t> sv((size_t)c * dp);
    for (int64_t i = 0; i < c; ++i)
      std::copy(vecs + (size_t)ids[(size_t)i] * dp, vecs + (size_t)(ids[(size_t)i] + 1) * dp, sv.begin() + i * dp);
    std::vector<uint32_t> se((size_t)c * R_int, kInvalid32);
    std::vector<uint16_t> sd((size_t)c * R_int, 0);
    std::vector<uint8_t> sc((size_t)c, 0);
    Graph g{sv.data(), c, dp, se.data(), sc.data(), R_int, nullptr, metric};
    process_batches(g, dim_for_prune, alpha, 0, c, std::max<int64_t>(1, std::min<int64_t>(batch_cap, c)), true, 0u,
                    se.data(), sd.data(), sc.data());
#pragma omp parallel
    {
      std::vector<std::pair<float, uint32_t>> C;  // (distance, slot in ids/bits)
      std::vector<uint32_t> cid;
      std::vector<uint16_t> cbits;
#pragma omp for schedule(static)
      for (int64_t i = 0; i < c; ++i) {
        const uint32_t gid = ids[(size_t)i];
        uint32_t* fe = edges + (size_t)gid * R_fin;
        uint16_t* fd = edge_dist + (size_t)gid * R_fin;
        cid.clear();
        cbits.clear();
        for (int j = 0; j < counts[gid]; ++j)
          if (fe[j] != kInvalid32) { cid.push_back(fe[j]); cbits.push_back(fd[j]); }
        for (int j = 0; j < sc[(size_t)i]; ++j) {
          const uint32_t nb = se[(size_t)i * R_int + j];
          if (nb == kInvalid32) continue;
          cid.push_back(ids[nb]);
          cbits.push_back(sd[(size_t)i * R_int + j]);
        }
        C.clear();
        for (size_t t = 0; t < cid.size(); ++t) C.push_back({bf2f(cbits[t]), (uint32_t)t});
        std::stable_sort(C.begin(), C.end(), [](const std::pair<float, uint32_t>& a,
                                                const std::pair<float, uint32_t>& b) { return a.first < b.first; });
        int sel = 0;
        for (size_t t = 0; t < C.size() && sel < R_fin; ++t) {
          const uint32_t id = cid[C[t].second];
          bool dup = false;
          for (int u = 0; u < sel && !dup; ++u) dup = fe[u] == id;
          if (dup) continue;
          fe[sel] = id;
          fd[sel] = f2bf(C[t].first);
          ++sel;
        }
        counts[gid] = (uint8_t)sel;
      }
    }
  }
  return 0;
}

}  // extern "C"
