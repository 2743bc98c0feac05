// build.hip -- batched Vamana construction (reference index/construct.cuh).
//
// Per batch [s, s + b) of vertex ids (reference process_batch, :743-911):
//   1. beam search of every batch vector against the pre-batch graph
//      (the plain search kernel in "visited" mode: k = bw = 64, limit 256,
//      at most 256 pops recorded);
//   2. forward merge + RobustPrune, one wave per batch vertex: candidates are
//      the vertex's existing edges (stored bf16 distances) and its popped
//      nodes; the new edges and the reverse pairs (target << sb | source -
//      batch start, sb = bits of the largest batch)
//      are written in the same kernel (merge_candidates_kernel,
//      robust_prune_kernel and fill_reverse_edges, :280-501);
//   3. a stable radix sort of the reverse pairs on their target bits (they
//      are written in source order) and a head-marking pass, which groups
//      them by target with sources ascending (:846-879);
//   4. reverse merge + RobustPrune, one wave per target
//      (process_reverse_edges_kernel, :560-741).
// Batches grow 1, 2, 4, ... up to the maximum batch size (:913-958).
//
// The reference keeps an arbitrary arrival-order subset when one target gets
// more than 256 + R candidates in a batch (atomicAdd slots, :642-658). This
// implementation fixes that order: existing edges in slot order, then new
// sources in ascending id order. It is one of the orders the reference can
// produce, and it makes the build deterministic.
#include "build.hpp"
#include "directional_api.hpp"
#include "common.hpp"
#include "prune.hpp"
#include "search.hpp"


#include <algorithm>
#include <numeric>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace jasper_amd {

constexpr uint32_t kBuildL = 64;          // graph_construct_config L (ffi/jasper_ffi_common.cuh:58-59)
constexpr uint32_t kBuildLimit = 256;     // BEAM_SEARCH_LIMIT (construct.cuh:57)
constexpr uint32_t kBuildMaxResult = 256; // beam_search_max_result_size (construct.cuh:62)
constexpr uint32_t kCandBuf = 512;        // >= 256 + R, power of two

int64_t budget_max_batch(uint32_t R, int64_t budget_bytes) {
  const int64_t L = kBuildL, max_result = kBuildMaxResult, max_cands = max_result + R;
  const int64_t per_item = 8 * L + 8 * max_result + 4 + 8 * max_cands + 4 + 8 * (int64_t)R + 4 * (int64_t)R +
                           4 * (int64_t)R;
  const int64_t fixed = 4;
  const int64_t b = budget_bytes <= fixed ? 0 : (budget_bytes - fixed) / per_item;
  return std::min<int64_t>(b, 0xFFFFFFFFll);
}

int64_t reference_max_batch(int64_t n, uint32_t R, int64_t budget_bytes) {
  return std::min<int64_t>(budget_max_batch(R, budget_bytes), n / 50);
}

struct PruneKernelArgs {
  PruneCtx pc;
  uint32_t* edges;
  uint16_t* edist;
  uint8_t* counts;
  // forward
  const uint64_t* visited;
  const uint32_t* visited_counts;
  uint32_t batch_offset;
  uint32_t pair_shift;  // reverse pair keys: target << pair_shift | (source - batch_offset)
  uint32_t pair_mask;   // (1 << pair_shift) - 1, all ones at a shift of 32
  uint64_t* pairs;
  // reverse
  const uint64_t* sorted_pairs;
  uint32_t n_pairs;
  const uint32_t* heads;
  const uint32_t* n_heads;
  // work counters (BuildWork indices) or null
  unsigned long long* work;
};

static bool g_build_work = false;
void set_build_work_counting(bool on) { g_build_work = on; }
bool build_work_counting() { return g_build_work; }

// Work counters are kept in kWorkCopies copies (counter i, copy c at
// i * kWorkCopies + c), a block adding to copy blockIdx % kWorkCopies, so
// that a million waves do not serialise on one address; the host sums them.
constexpr int kWorkCopies = 64;
__device__ __forceinline__ void add_work(unsigned long long* w, int i, uint64_t v) {
  if (v) atomicAdd(&w[i * kWorkCopies + (blockIdx.x & (kWorkCopies - 1))], (unsigned long long)v);
}

// Sums the search stage's per-query counters (hops, degrees, scored) and
// visited counts of a batch into the work counters.
__global__ __launch_bounds__(256) void search_work_kernel(const uint32_t* st, const uint32_t* vcounts, uint32_t nq,
                                                          unsigned long long* work) {
  unsigned long long h = 0, d = 0, s = 0, v = 0;
  for (uint32_t q = blockIdx.x * 256 + threadIdx.x; q < nq; q += gridDim.x * 256) {
    h += st[(size_t)q * 4 + 0];
    d += st[(size_t)q * 4 + 1];
    s += st[(size_t)q * 4 + 2];
    v += vcounts[q];
  }
  for (int o = 32; o > 0; o >>= 1) {
    h += __shfl_xor(h, o, 64);
    d += __shfl_xor(d, o, 64);
    s += __shfl_xor(s, o, 64);
    v += __shfl_xor(v, o, 64);
  }
  if (lane_id() == 0) {
    add_work(work, kWorkSearchHops, h);
    add_work(work, kWorkSearchAdjacency, d);
    add_work(work, kWorkSearchScored, s);
    add_work(work, kWorkSearchVisited, v);
  }
}

// The adjacency row of v as loaded: degree, and per lane one slot (lanes
// past R read slot R - 1), issued together with no dependence on the degree.
struct ExistingRow {
  uint32_t cnt, id;
  uint16_t ed;
};

__device__ __forceinline__ ExistingRow load_existing(const PruneKernelArgs& a, uint32_t v) {
  const uint32_t R = a.pc.R;
  const size_t o = (size_t)v * R + min(lane_id(), R - 1u);
  ExistingRow e;
  e.cnt = a.counts[v];
  e.id = a.edges[o];
  e.ed = a.edist[o];
  return e;
}

// Appends the loaded existing edges to C (keys with their stored bf16
// distances); returns how many were appended.
__device__ __forceinline__ uint32_t append_existing(const ExistingRow& e, uint32_t R, uint64_t* C) {
  const uint32_t lane = lane_id();
  const bool ok = lane < e.cnt && lane < R && e.id != kInvalid32;
  const uint64_t m = ballot(ok);
  if (ok) C[mbcnt(m)] = make_key(bf2f(e.ed), e.id);
  return (uint32_t)__builtin_popcountll(m);
}

// Sort candidates C[0, nc) ascending (empty keys sort last). Up to 128
// keys are sorted in registers, one or two per lane; longer lists in LDS.
__device__ __forceinline__ void sort_candidates(uint64_t* C, uint32_t nc) {
  const uint32_t lane = lane_id();
  if (nc <= 64) {
    uint64_t x = lane < nc ? C[lane] : kEmptyKey;
    x = wave_bitonic_sort<64>(x);
    C[lane] = x;
    wave_sync();
    return;
  }
  if (nc <= 128) {
    uint64_t x0 = C[lane], x1 = lane + 64 < nc ? C[lane + 64] : kEmptyKey;
    wave_bitonic_sort128(x0, x1);
    C[lane] = x0;
    C[lane + 64] = x1;
    wave_sync();
    return;
  }
  const uint32_t N = pow2_ceil(nc);
  for (uint32_t i = nc + lane; i < N; i += 64) C[i] = kEmptyKey;
  wave_sync();
  lds_bitonic_sort(C, N);
}

// Sorts a reverse target's candidates: C[0, nE) its existing edges in slot
// order (stored bf16 distances), C[nE, nE + taken) its new sources. A stored
// row is the output of an earlier prune, so its keys are usually ascending
// already; ties of the rounded distances can break the id order (on config
// 2 one row in six, almost all of them one or two odd-even transposition
// passes from sorted). The existing keys take such passes while a lane
// finds its predecessor larger (the full bitonic sort after four). Up to
// kInsertSources sources are then placed by counting: existing key e_i goes
// to i + #{t_k <= e_i}, source t_j to #{t_k before t_j} + #{e_i < t_j}, with
// one broadcast per source. More sources are sorted apart and the two lists
// meet in one bitonic merge (64 wide when they fit, else 128 wide over two
// registers). The keys are distinct or identical 64-bit values, so the
// result is the full sort's.
constexpr uint32_t kInsertSources = 8;
constexpr int kOddEvenPasses = 4;

__device__ __forceinline__ void sort_reverse_candidates(uint64_t* C, uint32_t nE, uint32_t taken) {
  const uint32_t nc = nE + taken;
  if (nE > 64u || taken > 64u) {
    sort_candidates(C, nc);
    return;
  }
  const uint32_t lane = lane_id();
  uint64_t e = lane < nE ? C[lane] : kEmptyKey;
  uint64_t t = lane < taken ? C[nE + lane] : kEmptyKey;
  // lanes past nE hold the largest key, so they never start a descent (the
  // shuffles run in every lane: a lane reading an inactive one gets 0)
  uint64_t prev = __shfl_up(e, 1, 64);
  uint64_t desc = ballot(lane > 0u && e < prev);
  if (desc) {
    // odd phase partners (2i + 1, 2i + 2); lanes 0 and 63 pair with themselves
    const int podd = (lane & 1u) ? (int)min(lane + 1u, 63u) : (int)(lane == 0u ? 0u : lane - 1u);
    for (int pass = 0; desc != 0 && pass < kOddEvenPasses; ++pass) {
      e = bitonic_stage<64, 1>(e, lane);  // even phase: pairs (2i, 2i + 1)
      const uint64_t o = __shfl(e, podd, 64);
      const bool lower = (lane & 1u) != 0u;  // the odd lane keeps the smaller key
      e = lower ? (o < e ? o : e) : (o < e ? e : o);
      prev = __shfl_up(e, 1, 64);
      desc = ballot(lane > 0u && e < prev);
    }
    if (desc) e = wave_bitonic_sort<64>(e);
  }
  if (taken <= kInsertSources) {
    uint32_t pe = lane, pt = 0;
    for (uint32_t k = 0; k < taken; ++k) {
      const uint64_t tk = readlane64(t, (int)k);
      const bool e_lt = e < tk;
      const uint32_t below = (uint32_t)__builtin_popcountll(ballot(lane < nE && e_lt));
      pe += e_lt ? 0u : 1u;                                    // t_k <= e_i: t_k goes first
      pt += (tk < t || (tk == t && k < lane)) ? 1u : 0u;       // t_k before t_j
      pt += lane == k ? below : 0u;                            // e_i < t_j
    }
    wave_sync();  // every read of C precedes the writes below
    if (lane < nE) C[pe] = e;
    if (lane < taken) C[pt] = t;
    wave_sync();
    return;
  }
  t = wave_sort_upto(t, taken);
  wave_sync();  // every read of C precedes the writes below
  // e ascending then the sources descending: a bitonic sequence of 128
  const uint64_t tr = reverse_lanes64(t);
  const bool lt = e < tr;
  uint64_t x0 = lt ? e : tr;
  if (nc <= 64u) {
    x0 = bitonic_merge_steps<64, 32>(x0, lane);
    C[lane] = x0;
  } else {
    uint64_t x1 = lt ? tr : e;
    bitonic_stage128<128, 32>(x0, x1);
    C[lane] = x0;
    C[lane + 64] = x1;
  }
  wave_sync();
}

__device__ __forceinline__ void write_selection(const PruneKernelArgs& a, uint32_t v, uint32_t ns,
                                                const uint32_t* S_ids, const float* S_dist) {
  const uint32_t lane = lane_id();
  const uint32_t R = a.pc.R;
  if (lane < ns) {
    a.edges[(size_t)v * R + lane] = S_ids[lane];
    a.edist[(size_t)v * R + lane] = f2bf(S_dist[lane]);
  }
  if (lane == 0) a.counts[v] = (uint8_t)ns;
}

struct PruneLds {
  uint64_t* C;
  uint32_t* S_ids;
  float* S_dist;
  uint32_t* srcs;
};

__device__ __forceinline__ PruneLds carve_prune_lds(uint64_t* smem, uint32_t R) {
  PruneLds l;
  l.C = smem;
  l.S_ids = reinterpret_cast<uint32_t*>(smem + kCandBuf);
  l.S_dist = reinterpret_cast<float*>(l.S_ids + 64);
  l.srcs = reinterpret_cast<uint32_t*>(l.S_dist + 64);
  (void)R;
  return l;
}

// JASPER_GRAM_MARGIN (>= 1, default 1) widens the proof margin of the Gram
// prune on non-integer rows, sending more pairs to the exact chain; the
// results do not change (used by the tests to exercise that path).
static float gram_margin_scale() {
  static const float v = [] {
    const char* e = std::getenv("JASPER_GRAM_MARGIN");
    const float f = e ? (float)std::atof(e) : 1.0f;
    return f >= 1.0f ? f : 1.0f;
  }();
  return v;
}

#ifndef JASPER_GRAM_WAVES
#define JASPER_GRAM_WAVES 2
#endif
#ifndef JASPER_GRAM8_WAVES
#define JASPER_GRAM8_WAVES 4
#endif
// The forward prune on byte rows takes the Gram form for up to 96 candidates.
#ifndef JASPER_RQ_BUILD_L
#define JASPER_RQ_BUILD_L kBuildL
#endif
#ifndef JASPER_FWD_GRAM
#define JASPER_FWD_GRAM 1
#endif

static size_t prune_lds_bytes() { return kCandBuf * 8 + 64 * 4 + 64 * 4 + kCandBuf * 4; }
static_assert(kGramLdsWords <= kCandBuf, "the Gram prune's scratch reuses the source list");

// SCALE: a merge of the partitioned build (B1 batch against B2): the merge
// prune, and reverse pairs only for targets in B2 (r2 of the prune context;
// process_reverse_edges_kernel_scale skips the others,
// index/construct_scale_kernels.cuh:193-194).
// BYTES: the graph keeps byte rows (CPL 4, L2, integer rows): the prune
// works on them (robust_prune_wave_u8)
// The forward prune takes the Gram prune wherever the reverse prune does
// (rows of up to 128 values, at most 96 candidates): on byte rows the
// integer form at four waves per SIMD, on other rows the fp16 integer form
// or the form with proof at two.
template <int CPL, int METRIC, bool INTX, bool SCALE, bool BYTES>
constexpr int forward_waves_per_simd() {
  return !SCALE && JASPER_FWD_GRAM ? (BYTES ? JASPER_GRAM8_WAVES : CPL >= 1 && CPL <= 4 ? JASPER_GRAM_WAVES : 1) : 1;
}

template <int CPL, int METRIC, bool INTX, bool SCALE, bool BYTES = false>
__global__ __launch_bounds__(64, (forward_waves_per_simd<CPL, METRIC, INTX, SCALE, BYTES>())) void
forward_prune_kernel(PruneKernelArgs a) {
  static_assert(!BYTES || (CPL == 4 && METRIC == kL2 && INTX), "byte rows: integer L2 rows of 112/128");
  extern __shared__ uint64_t smem[];
  const PruneLds l = carve_prune_lds(smem, a.pc.R);
  const uint32_t lane = lane_id();
  const uint32_t bid = blockIdx.x;
  const uint32_t v = a.batch_offset + bid;
  const uint32_t R = a.pc.R;

  const ExistingRow er = load_existing(a, v);
  const uint32_t nv = a.visited_counts[bid];
  uint32_t nc = append_existing(er, R, l.C);
  const uint32_t n_existing = nc;
  for (uint32_t base = 0; base < nv; base += 64) {
    const uint32_t i = base + lane;
    bool ok = i < nv;
    uint64_t key = 0;
    if (ok) {
      key = a.visited[(size_t)bid * kBuildMaxResult + i] & ~1ull;
      ok = key_id(key) != v;
    }
    const uint64_t m = ballot(ok);
    if (ok) l.C[nc + mbcnt(m)] = key;
    nc += (uint32_t)__builtin_popcountll(m);
  }
  wave_sync();
  sort_candidates(l.C, nc);
  uint32_t ns;
  if constexpr (BYTES && !SCALE && JASPER_FWD_GRAM) {
    // up to 96 candidates: the byte-row Gram prune (all candidate rows read
    // at once, pair distances on the matrix cores); longer lists the wave prune
    float* gn = reinterpret_cast<float*>(l.srcs);
    if (nc <= 32 && a.pc.alpha >= 0.0f) ns = robust_prune_gram<1, 2>(a.pc, l.C, nc, v, l.S_ids, l.S_dist, gn);
    else if (nc <= 64 && a.pc.alpha >= 0.0f) ns = robust_prune_gram<2, 2>(a.pc, l.C, nc, v, l.S_ids, l.S_dist, gn);
    else if (nc <= kGramMaxCands && a.pc.alpha >= 0.0f)
      ns = robust_prune_gram<3, 2>(a.pc, l.C, nc, v, l.S_ids, l.S_dist, gn);
    else ns = robust_prune_wave_u8<SCALE>(a.pc, l.C, nc, v, l.S_ids, l.S_dist);
  } else if constexpr (BYTES) {
    ns = robust_prune_wave_u8<SCALE>(a.pc, l.C, nc, v, l.S_ids, l.S_dist);
  } else if constexpr (!SCALE && JASPER_FWD_GRAM && CPL >= 1 && CPL <= 4) {
    // the reverse prune's choice: pair distances on the matrix cores, exact
    // for integer rows (alpha >= 0), proved otherwise
    const uint32_t climit = METRIC == kL2 ? a.pc.nlimit : (a.pc.nlimit + 7u) / 8u;
    float* gn = reinterpret_cast<float*>(l.srcs);
    if (nc <= kGramMaxCands && climit <= kGramMaxChunks && (!INTX || a.pc.alpha >= 0.0f)) {
      if constexpr (INTX) {
        if (nc <= 32) ns = robust_prune_gram<1, 0>(a.pc, l.C, nc, v, l.S_ids, l.S_dist, gn);
        else if (nc <= 64) ns = robust_prune_gram<2, 0>(a.pc, l.C, nc, v, l.S_ids, l.S_dist, gn);
        else ns = robust_prune_gram<3, 0>(a.pc, l.C, nc, v, l.S_ids, l.S_dist, gn);
      } else {
        if (nc <= 32) ns = robust_prune_gram_f<1, CPL, METRIC>(a.pc, l.C, nc, v, l.S_ids, l.S_dist, gn);
        else if (nc <= 64) ns = robust_prune_gram_f<2, CPL, METRIC>(a.pc, l.C, nc, v, l.S_ids, l.S_dist, gn);
        else ns = robust_prune_gram_f<3, CPL, METRIC>(a.pc, l.C, nc, v, l.S_ids, l.S_dist, gn);
      }
    } else {
      ns = robust_prune_wave<CPL, METRIC, INTX, SCALE>(a.pc, l.C, nc, v, l.S_ids, l.S_dist);
    }
  } else {
    ns = robust_prune_wave<CPL, METRIC, INTX, SCALE>(a.pc, l.C, nc, v, l.S_ids, l.S_dist);
  }
  write_selection(a, v, ns, l.S_ids, l.S_dist);
  if (a.work && lane == 0) {
    add_work(a.work, kWorkForwardRows, 1u);
    add_work(a.work, kWorkForwardExisting, n_existing);
    add_work(a.work, kWorkForwardVisited, nv);
    add_work(a.work, kWorkForwardCandidates, nc);
    add_work(a.work, kWorkForwardSelected, ns);
  }
  if (lane < R) {
    const uint32_t t = lane < ns ? l.S_ids[lane] : 0u;
    const bool pair = lane < ns && (!SCALE || t - a.pc.r2_lo < a.pc.r2_n);
    a.pairs[(size_t)bid * R + lane] = pair ? (((uint64_t)t << a.pair_shift) | bid) : kEmptyKey;
  }
}

// Records the first position of every target group; one counter atomic
// per block of kMarkHeadsBlock threads, its waves' counts summed in LDS (one
// atomic per wave measured 108 us per batch of 1.28M pairs, bound by the
// atomics on the one counter). The order of heads does not matter: each
// target is pruned on its own.
constexpr uint32_t kMarkHeadsBlock = 1024;
__global__ __launch_bounds__(kMarkHeadsBlock) void mark_heads_kernel(const uint64_t* sorted, uint32_t n,
                                                                     uint32_t shift, uint32_t* heads,
                                                                     uint32_t* n_heads) {
  __shared__ uint32_t wave_base[kMarkHeadsBlock / 64];
  __shared__ uint32_t block_base;
  const uint32_t i = blockIdx.x * kMarkHeadsBlock + threadIdx.x;
  const uint32_t wv = threadIdx.x >> 6;
  bool head = false;
  if (i < n) {
    const uint64_t k = sorted[i];
    head = k != kEmptyKey && (i == 0 || (sorted[i - 1] >> shift) != (k >> shift));
  }
  const uint64_t m = ballot(head);
  if (lane_id() == 0) wave_base[wv] = (uint32_t)__builtin_popcountll(m);
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t total = 0;
    for (uint32_t j = 0; j < kMarkHeadsBlock / 64; ++j) {
      const uint32_t c = wave_base[j];
      wave_base[j] = total;
      total += c;
    }
    block_base = total ? atomicAdd(n_heads, total) : 0u;
  }
  __syncthreads();
  if (head) heads[block_base + wave_base[wv] + mbcnt(m)] = i;
}

// The Gram prune holds 96 candidate rows of up to 128 values in registers
// (96 VGPRs as fp16) beside its accumulators; two waves per SIMD keep it
// unspilled (three spill, and measured slower). As bytes (I8) the rows take
// 48 VGPRs.
template <int CPL, bool INTX, int I8>
constexpr int reverse_waves_per_simd() {
  return I8 ? JASPER_GRAM8_WAVES : CPL >= 1 && CPL <= 4 ? JASPER_GRAM_WAVES : 1;
}

// I8 (integer rows spanning at most 255 values, CPL 1..4, L2): the Gram
// prune on bytes, converted from the fp16 rows (1) or read from the graph's
// byte rows (2, CPL 4), which then also give the sources' distances to the
// target; the rest of the kernel is the INTX kernel's.
template <int CPL, int METRIC, bool INTX, bool SCALE, int I8 = 0>
__global__ __launch_bounds__(64, (reverse_waves_per_simd<CPL, INTX, I8>())) void reverse_prune_kernel(
    PruneKernelArgs a) {
  static_assert(!I8 || (INTX && METRIC == kL2 && CPL >= 1 && CPL <= 4 && !SCALE), "byte rows: integer L2 only");
  static_assert(I8 != 2 || CPL == 4, "byte rows hold rows of 112 or 128 values");
  extern __shared__ uint64_t smem[];
  const PruneLds l = carve_prune_lds(smem, a.pc.R);
  const uint32_t lane = lane_id();
  const uint32_t ql = lane & 3u, qg = lane >> 2;
  const uint32_t R = a.pc.R;
  const uint32_t nh = *a.n_heads;
  const uint32_t max_cands = kBuildMaxResult + R;
  uint32_t h = blockIdx.x;
  if (h >= nh) return;
  uint64_t wk_targets = 0, wk_existing = 0, wk_sources = 0, wk_selected = 0;  // work counters (a.work)
  // the first pair of the next head is read one target ahead
  uint32_t start = a.heads[h];
  uint32_t w = (uint32_t)(a.sorted_pairs[start] >> a.pair_shift);
  for (; h < nh; h += gridDim.x) {
    // this target's reads, issued together: its adjacency row, its row of
    // values, the first 64 pairs of its group, and the next head
    const ExistingRow er = load_existing(a, w);
    RowFrag<CPL> xw;
    if constexpr (I8 == 2) load_query_bytes(a.pc.vecs + (size_t)w * a.pc.nchunks, a.pc.nb8, a.pc.qsh2, ql, xw.x);
    else load_row_frag<CPL>(vec_row(a.pc, w), ql, a.pc.nchunks, true, xw);
    uint64_t key = a.sorted_pairs[min(start + lane, a.n_pairs - 1u)];
    if (start + lane >= a.n_pairs) key = kEmptyKey;
    const uint32_t start_next = a.heads[min(h + gridDim.x, nh - 1u)];
    const uint32_t nE = append_existing(er, R, l.C);
    // sources of w in ascending id order, self skipped, capped at 256 + R
    const uint32_t cap = max_cands - nE;
    uint32_t taken = 0;
    for (uint32_t pos = start;;) {
      const bool same = key != kEmptyKey && (uint32_t)(key >> a.pair_shift) == w;
      const uint32_t src = a.batch_offset + ((uint32_t)key & a.pair_mask);
      const bool ok = same && src != w;
      const uint64_t m = ballot(ok);
      const uint32_t rank = mbcnt(m);
      if (ok && taken + rank < cap) l.srcs[taken + rank] = src;
      taken = min(cap, taken + (uint32_t)__builtin_popcountll(m));
      if (taken >= cap || ballot(!same)) break;
      pos += 64;
      const uint32_t i = pos + lane;
      key = i < a.n_pairs ? a.sorted_pairs[i] : kEmptyKey;
    }
    const uint32_t w_next = (uint32_t)(a.sorted_pairs[start_next] >> a.pair_shift);
    wave_sync();
    // d(w, v) for every source (compute_distance(src_vec = w, sink_vec = v))
    if constexpr (I8 == 2) {
      // xw holds w shifted in byte-chunk order; a graph row's values lie in
      // the byte range, so w becomes bytes and the sources' byte rows are
      // scored with v_dot4_u32_u8
      uint4 wb[2];
      uint32_t wn;
      (void)left_bytes_u8(a.pc.nb8, xw.x, ql, wb, wn);
      for (uint32_t base = 0; base < taken; base += 16) {
        const uint32_t j = base + qg;
        const bool act = j < taken;
        const uint32_t sid = act ? l.srcs[j] : 0u;
        RowBytes xs;
        load_row_bytes(a.pc.vecs8, a.pc.nb8, sid, ql, xs);
        const float d = score_bytes_u8(a.pc.nb8, wb[0], wb[1], wn, xs, ql);
        if (act && ql == 0) l.C[nE + j] = make_key(d, sid);
      }
    } else {
      LeftFrag<CPL, METRIC> wf;
      left_from_row<CPL, METRIC>(xw, ql, wf);
      for (uint32_t base = 0; base < taken; base += 16) {
        const uint32_t j = base + qg;
        const bool act = j < taken;
        const uint32_t sid = act ? l.srcs[j] : a.pc.r1_lo;
        RowFrag<CPL> xs;
        load_row_frag<CPL>(vec_row(a.pc, sid), ql, a.pc.nchunks, act, xs);
        const float d = left_distance<CPL, METRIC, INTX>(wf, xs, ql, a.pc.nchunks, a.pc.nlimit);
        if (act && ql == 0) l.C[nE + j] = make_key(d, sid);
      }
    }
    wave_sync();
    const uint32_t nc = nE + taken;
    sort_reverse_candidates(l.C, nE, taken);
    uint32_t ns;
    if constexpr (SCALE) {
      if constexpr (CPL == 4 && METRIC == kL2 && INTX) {
        if (a.pc.vecs8) ns = robust_prune_wave_u8<true>(a.pc, l.C, nc, w, l.S_ids, l.S_dist);
        else ns = robust_prune_wave<CPL, METRIC, INTX, true>(a.pc, l.C, nc, w, l.S_ids, l.S_dist);
      } else {
        ns = robust_prune_wave<CPL, METRIC, INTX, true>(a.pc, l.C, nc, w, l.S_ids, l.S_dist);
      }
    } else if constexpr (CPL >= 1 && CPL <= 4) {
      // up to 96 candidates of rows of up to 128 values: pair distances on
      // the matrix cores, exact for integer rows, proved otherwise
      const uint32_t climit = METRIC == kL2 ? a.pc.nlimit : (a.pc.nlimit + 7u) / 8u;
      // (the integer Gram prune's thresholds need alpha >= 0)
      if (nc <= kGramMaxCands && climit <= kGramMaxChunks && (!INTX || a.pc.alpha >= 0.0f)) {
        float* gn = reinterpret_cast<float*>(l.srcs);
        if constexpr (INTX) {
          if (nc <= 32) ns = robust_prune_gram<1, I8>(a.pc, l.C, nc, w, l.S_ids, l.S_dist, gn);
          else if (nc <= 64) ns = robust_prune_gram<2, I8>(a.pc, l.C, nc, w, l.S_ids, l.S_dist, gn);
          else ns = robust_prune_gram<3, I8>(a.pc, l.C, nc, w, l.S_ids, l.S_dist, gn);
        } else {
          if (nc <= 32) ns = robust_prune_gram_f<1, CPL, METRIC>(a.pc, l.C, nc, w, l.S_ids, l.S_dist, gn);
          else if (nc <= 64) ns = robust_prune_gram_f<2, CPL, METRIC>(a.pc, l.C, nc, w, l.S_ids, l.S_dist, gn);
          else ns = robust_prune_gram_f<3, CPL, METRIC>(a.pc, l.C, nc, w, l.S_ids, l.S_dist, gn);
        }
      } else if constexpr (I8 == 2) {
        ns = robust_prune_wave_u8(a.pc, l.C, nc, w, l.S_ids, l.S_dist);  // more than 96 candidates
      } else {
        ns = robust_prune_wave<CPL, METRIC, INTX>(a.pc, l.C, nc, w, l.S_ids, l.S_dist);
      }
    } else {
      ns = robust_prune_wave<CPL, METRIC, INTX>(a.pc, l.C, nc, w, l.S_ids, l.S_dist);
    }
    write_selection(a, w, ns, l.S_ids, l.S_dist);
    wk_targets += 1;
    wk_existing += nE;
    wk_sources += taken;
    wk_selected += ns;
    wave_sync();
    start = start_next;
    w = w_next;
  }
  if (a.work && lane == 0) {
    add_work(a.work, kWorkReverseTargets, wk_targets);
    add_work(a.work, kWorkReverseExisting, wk_existing);
    add_work(a.work, kWorkReverseSources, wk_sources);
    add_work(a.work, kWorkReverseSelected, wk_selected);
  }
}

template <int CPL, int METRIC, bool INTX, bool SCALE, bool BYTES = false>
static void launch_forward(const PruneKernelArgs& a, uint32_t bs, size_t lds, hipStream_t s) {
  auto k = forward_prune_kernel<CPL, METRIC, INTX, SCALE, BYTES>;
  if (lds > 64 * 1024)
    hip_check(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds), "LDS");
  hipLaunchKernelGGL(k, dim3(bs), dim3(64), lds, s, a);
}

template <int CPL, int METRIC, bool INTX, bool SCALE, int I8 = 0>
static void launch_reverse(const PruneKernelArgs& a, uint32_t grid, size_t lds, hipStream_t s) {
  auto k = reverse_prune_kernel<CPL, METRIC, INTX, SCALE, I8>;
  if (lds > 64 * 1024)
    hip_check(hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds), "LDS");
  hipLaunchKernelGGL(k, dim3(grid), dim3(64), lds, s, a);
}

template <int METRIC, bool INTX, bool SCALE = false>
static void dispatch_prune(bool reverse, uint32_t cpl, const PruneKernelArgs& a, uint32_t grid, size_t lds,
                           hipStream_t s) {
  switch (cpl) {
#define JA_CASE(C)                                                                  \
  case C:                                                                           \
    if (reverse) launch_reverse<C, METRIC, INTX && C != 0, SCALE>(a, grid, lds, s); \
    else launch_forward<C, METRIC, INTX && C != 0, SCALE>(a, grid, lds, s);         \
    break;
    JA_CASE(0)
    JA_CASE(1)
    JA_CASE(2)
    JA_CASE(3)
    JA_CASE(4)
    JA_CASE(5)
    JA_CASE(6)
    JA_CASE(7)
    JA_CASE(8)
#undef JA_CASE
    default:
      throw std::logic_error("unreachable chunks-per-lane case");
  }
}

// The graph's byte rows, when it keeps them current, for the reverse
// prune's byte mode (null otherwise).
static void set_byte_rows(PruneCtx& pc, const Graph& g) {
  pc.vecs8 = nullptr;
  pc.nb8 = 0;
  pc.qsh2 = 0;
  if (g.vecs8 && g.vecs8_lo == g.int_lo && g.vecs8_cap >= g.n && byte_rows_eligible(g)) {
    pc.vecs8 = (const uint4*)g.vecs8;
    pc.nb8 = g.dim / 16;
    const uint32_t h = f2h_rn((float)g.int_lo - 1024.0f);  // exact (byte_rows_eligible)
    pc.qsh2 = h | (h << 16);
  }
}

// Integer rows (int_exact_l2 holds) whose values span at most 255: the
// reverse prune's Gram step can take them as bytes. JASPER_GRAM8=0 turns
// that off (the fp16 Gram kernel then runs; the results are the same).
static bool int8_rows(const Graph& g) {
  static const bool on = [] {
    const char* e = std::getenv("JASPER_GRAM8");
    return !(e && std::atoi(e) == 0);
  }();
  return on && g.int_state == 1 && (int64_t)g.int_hi - (int64_t)g.int_lo <= 255;
}

// The reverse prune on integer rows spanning at most 255 values: rows of up
// to 128 values take the byte Gram kernel, longer ones the INTX kernel.
static void dispatch_reverse_i8(uint32_t cpl, const PruneKernelArgs& a, uint32_t grid, size_t lds, hipStream_t s) {
  switch (cpl) {
    case 1: launch_reverse<1, kL2, true, false, 1>(a, grid, lds, s); break;
    case 2: launch_reverse<2, kL2, true, false, 1>(a, grid, lds, s); break;
    case 3: launch_reverse<3, kL2, true, false, 1>(a, grid, lds, s); break;
    case 4:
      if (a.pc.vecs8) launch_reverse<4, kL2, true, false, 2>(a, grid, lds, s);
      else launch_reverse<4, kL2, true, false, 1>(a, grid, lds, s);
      break;
    default: dispatch_prune<kL2, true>(true, cpl, a, grid, lds, s); break;
  }
}

struct EventTimer {
  bool on;
  hipStream_t s;
  hipEvent_t e0, e1;
  EventTimer(bool on_, hipStream_t s_) : on(on_), s(s_) {
    if (on) { (void)hipEventCreate(&e0); (void)hipEventCreate(&e1); }
  }
  ~EventTimer() {
    if (on) { (void)hipEventDestroy(e0); (void)hipEventDestroy(e1); }
  }
  void start() { if (on) (void)hipEventRecord(e0, s); }
  void stop(double& acc) {
    if (!on) return;
    (void)hipEventRecord(e1, s);
    (void)hipEventSynchronize(e1);
    float ms = 0;
    (void)hipEventElapsedTime(&ms, e0, e1);
    acc += ms;
  }
};

void build_graph(Graph& g, float alpha, int64_t max_batch, hipStream_t stream, bool time_stages,
                 BuildStats* stats, bool rabitq_search) {
  build_range(g, alpha, 0, g.n, max_batch, true, stream, time_stages, stats, rabitq_search);
}

// Device workspace of one build pass for batches of up to mb vertices:
// the search's popped keys, reverse pairs (unsorted and sorted), group
// heads and the radix sort's temporary storage. Freed on destruction.
struct BuildWorkspace {
  uint64_t* visited = nullptr;
  uint32_t* vcounts = nullptr;
  uint64_t* pairs = nullptr;
  uint64_t* sorted = nullptr;
  uint32_t* heads = nullptr;
  uint32_t* nheads = nullptr;
  void* temp = nullptr;
  size_t temp_bytes = 0;

  BuildWorkspace(int64_t mb, uint32_t R) {
    const size_t max_pairs = (size_t)mb * R;
    temp_bytes = sort_u64_temp_bytes(max_pairs);
    try {
      hip_check(hipMalloc(&visited, (size_t)mb * kBuildMaxResult * 8), "alloc build visited");
      hip_check(hipMalloc(&vcounts, (size_t)mb * 4), "alloc build visited counts");
      hip_check(hipMalloc(&pairs, max_pairs * 8), "alloc reverse pairs");
      hip_check(hipMalloc(&sorted, max_pairs * 8), "alloc sorted pairs");
      hip_check(hipMalloc(&heads, max_pairs * 4), "alloc heads");
      hip_check(hipMalloc(&nheads, 4), "alloc head count");
      hip_check(hipMalloc(&temp, std::max<size_t>(temp_bytes, 16)), "alloc sort temp");
    } catch (...) {
      release();
      throw;
    }
  }
  ~BuildWorkspace() { release(); }
  BuildWorkspace(const BuildWorkspace&) = delete;
  BuildWorkspace& operator=(const BuildWorkspace&) = delete;
  void release() {
    (void)hipFree(visited);
    (void)hipFree(vcounts);
    (void)hipFree(pairs);
    (void)hipFree(sorted);
    (void)hipFree(heads);
    (void)hipFree(nheads);
    (void)hipFree(temp);
    visited = nullptr;
    vcounts = nullptr;
    pairs = sorted = nullptr;
    heads = nheads = nullptr;
    temp = nullptr;
  }
};

// Reverse pair keys are target << sb | (source - batch start) with sb the
// bits of the largest batch; the radix sort covers the bits of both.
struct PairBits {
  uint32_t sb;
  int end_bit;
};
static PairBits pair_bits(int64_t mb, int64_t n) {
  PairBits b;
  b.sb = 1;
  while (((uint64_t)1 << b.sb) < (uint64_t)mb) ++b.sb;
  b.end_bit = (int)b.sb;
  while (b.end_bit < 64 && ((uint64_t)1 << (b.end_bit - b.sb)) <= (uint64_t)n) ++b.end_bit;
  return b;
}

// Kernel arguments of the prune passes over g with workspace ws. *intx
// tells whether the rows are integers in the exact range (int_exact_l2:
// packed-difference distances, the same bits as the fp32 chain).
static PruneKernelArgs prune_args(Graph& g, float alpha, const BuildWorkspace& ws, uint32_t sb, hipStream_t stream,
                                  bool* intx) {
  PruneKernelArgs pa{};
  pa.pair_shift = sb;
  pa.pair_mask = (1u << sb) - 1u;
  pa.pc.vecs = (const uint4*)g.vecs;
  pa.pc.nchunks = g.dp / 8;
  pa.pc.nlimit = g.metric == kL2 ? g.dim / 8 : g.dim;  // the reference prunes with `dim`
  pa.pc.R = g.R;
  pa.pc.alpha = alpha;
  pa.pc.margin_scale = gram_margin_scale();
  pa.edges = g.edges;
  pa.edist = g.edist;
  pa.counts = g.counts;
  pa.visited = ws.visited;
  pa.visited_counts = ws.vcounts;
  pa.pairs = ws.pairs;
  pa.sorted_pairs = ws.sorted;
  pa.heads = ws.heads;
  pa.n_heads = ws.nheads;
  int32_t int_lo = 0;
  *intx = int_exact_l2(g, stream, &int_lo);
  const _Float16 lo = (_Float16)int_lo;  // exact: an fp16 value of the rows
  uint16_t bits;
  std::memcpy(&bits, &lo, 2);
  pa.pc.lo2 = (uint32_t)bits * 0x10001u;
  set_byte_rows(pa.pc, g);
  return pa;
}

// chunks per quad lane held in registers; 0 streams rows longer than 32 chunks
static uint32_t prune_cpl(const Graph& g) {
  const uint32_t nchunks = g.dp / 8;
  return (nchunks + 3) / 4 > 8 ? 0u : (nchunks + 3) / 4;
}

// Steps 3 and 4 of a batch: group the reverse pairs of its bs vertices by
// target, then the reverse merge + prune (SCALE: the merge prune).
template <bool SCALE>
static void reverse_step(const Graph& g, PruneKernelArgs& pa, const BuildWorkspace& ws, const PairBits& pb,
                         int64_t bs, bool intx, uint32_t cpl, EventTimer& timer, BuildStats& st,
                         hipStream_t stream) {
  const size_t plds = prune_lds_bytes();
  const uint32_t np = (uint32_t)(bs * g.R);
  timer.start();
  // the pairs are written in source order (pair index = source * R + slot),
  // so a stable sort of the target bits groups them with sources ascending
  sort_u64(ws.temp, ws.temp_bytes, ws.pairs, ws.sorted, np, (int)pb.sb, pb.end_bit, stream);
  hip_check(hipMemsetAsync(ws.nheads, 0, 4, stream), "clear head count");
  hipLaunchKernelGGL(mark_heads_kernel, dim3((np + kMarkHeadsBlock - 1) / kMarkHeadsBlock), dim3(kMarkHeadsBlock), 0,
                     stream, ws.sorted, np, pb.sb, ws.heads, ws.nheads);
  hip_check(hipGetLastError(), "launch mark_heads_kernel");
  timer.stop(st.sort_ms);
  pa.n_pairs = np;
  const uint32_t grid = (uint32_t)std::min<int64_t>(std::max<int64_t>(np, 1), 16384);
  timer.start();
  if (SCALE) {
    if (intx) dispatch_prune<kL2, true, true>(true, cpl, pa, grid, plds, stream);
    else if (g.metric == kL2) dispatch_prune<kL2, false, true>(true, cpl, pa, grid, plds, stream);
    else dispatch_prune<kIP, false, true>(true, cpl, pa, grid, plds, stream);
  } else {
    if (intx && int8_rows(g)) dispatch_reverse_i8(cpl, pa, grid, plds, stream);
    else if (intx) dispatch_prune<kL2, true>(true, cpl, pa, grid, plds, stream);
    else if (g.metric == kL2) dispatch_prune<kL2, false>(true, cpl, pa, grid, plds, stream);
    else dispatch_prune<kIP, false>(true, cpl, pa, grid, plds, stream);
  }
  hip_check(hipGetLastError(), "launch reverse_prune_kernel");
  timer.stop(st.reverse_ms);
}

void build_range(Graph& g, float alpha, int64_t first, int64_t last, int64_t max_batch, bool doubling,
                 hipStream_t stream, bool time_stages, BuildStats* stats, bool rabitq_search) {
  if (rabitq_search && !g.rabitq) throw std::invalid_argument("RaBitQ build search needs the RaBitQ codes");
  if (last <= first) return;
  if (first < 0 || last > g.n) throw std::invalid_argument("vertex range outside the graph");
  if (max_batch < 1) max_batch = 1;  // the reference loops forever here (n < 50); clamp instead
  if (g.R > 64) throw std::invalid_argument("R must be <= 64");
  const uint32_t cpl = prune_cpl(g);
  const int64_t mb = std::min<int64_t>(max_batch, last - first);

  BuildWorkspace ws(mb, g.R);
  const PairBits pb = pair_bits(mb, g.n);
  bool intx = false;
  PruneKernelArgs pa = prune_args(g, alpha, ws, pb.sb, stream, &intx);
  const size_t plds = prune_lds_bytes();

  BuildStats st;
  st.max_batch = mb;
  // work counting: counters, the search stage's per-query counters and its
  // exact seen bitmap (freed when the build returns or throws)
  struct WorkBuffers {
    unsigned long long* work = nullptr;
    uint32_t* qstats = nullptr;
    uint32_t* seen = nullptr;
    ~WorkBuffers() {
      (void)hipFree(work);
      (void)hipFree(qstats);
      (void)hipFree(seen);
    }
  } wb;
  const size_t seen_words = (size_t)((g.n + 31) / 32);
  if (g_build_work) {
    const size_t seen_bytes = (size_t)mb * seen_words * 4;
    if (seen_bytes > ((size_t)8 << 30))
      throw std::invalid_argument("build work counting needs " + std::to_string(seen_bytes >> 20) +
                                  " MiB of seen bitmap (limit 8 GiB): count a smaller build");
    hip_check(hipMalloc(&wb.work, kWorkCount * kWorkCopies * 8), "alloc build work counters");
    hip_check(hipMemsetAsync(wb.work, 0, kWorkCount * kWorkCopies * 8, stream), "clear build work counters");
    hip_check(hipMalloc(&wb.qstats, (size_t)mb * 16), "alloc search counters");
    hip_check(hipMalloc(&wb.seen, std::max<size_t>(seen_bytes, 4)), "alloc seen bitmap");
    pa.work = wb.work;
  }
  EventTimer timer(time_stages, stream);
  hipEvent_t t0, t1;
  hip_check(hipEventCreate(&t0), "event");
  hip_check(hipEventCreate(&t1), "event");
  hip_check(hipEventRecord(t0, stream), "event record");
  try {
    int64_t count = first, bs = doubling ? 1 : mb;
    while (count < last) {
      bs = std::min<int64_t>(bs, last - count);
      bs = std::min<int64_t>(bs, mb);
      // 1. beam search of the batch against the pre-batch graph
      SearchRequest r;
      r.use_range = true;
      r.q_start = (uint32_t)count;
      r.nq = (uint32_t)bs;
      r.medoid = g.medoid;
      r.k = kBuildL;
      r.beam_width = kBuildL;
      r.limit = kBuildLimit;
      r.max_result = kBuildMaxResult;
      r.visited = ws.visited;
      r.visited_counts = ws.vcounts;
      // the queries' seen-cache size (at 100M vectors the 8 KB 16-bit form
      // took the search stage from 11.4 s to 10.6 s)
      r.hash_bits = seen_cache_hash_bits(g.n);
      if (wb.work && !rabitq_search) {
        hip_check(hipMemsetAsync(wb.seen, 0, (size_t)bs * seen_words * 4, stream), "clear seen bitmap");
        r.stats = wb.qstats;
        r.seen_bits = wb.seen;
      }
      timer.start();
      if (rabitq_search)
        rabitq_build_search(g, (uint32_t)count, (uint32_t)bs, JASPER_RQ_BUILD_L, kBuildLimit, kBuildMaxResult, ws.visited,
                            ws.vcounts, stream);
      else
        launch_beam_search(g, r, stream);
      timer.stop(st.search_ms);
      if (wb.work) {
        st.work[kWorkSearchQueries] += (uint64_t)bs;
        if (!rabitq_search) {
          const uint32_t blocks = (uint32_t)std::min<int64_t>((bs + 255) / 256, 1024);
          hipLaunchKernelGGL(search_work_kernel, dim3(blocks), dim3(256), 0, stream, wb.qstats, ws.vcounts,
                             (uint32_t)bs, wb.work);
          hip_check(hipGetLastError(), "launch search_work_kernel");
        }
      }
      // 2. forward merge + prune + reverse pairs
      pa.batch_offset = (uint32_t)count;
      timer.start();
      if (intx && pa.pc.vecs8 && cpl == 4) launch_forward<4, kL2, true, false, true>(pa, (uint32_t)bs, plds, stream);
      else if (intx) dispatch_prune<kL2, true>(false, cpl, pa, (uint32_t)bs, plds, stream);
      else if (g.metric == kL2) dispatch_prune<kL2, false>(false, cpl, pa, (uint32_t)bs, plds, stream);
      else dispatch_prune<kIP, false>(false, cpl, pa, (uint32_t)bs, plds, stream);
      hip_check(hipGetLastError(), "launch forward_prune_kernel");
      timer.stop(st.prune_ms);
      // 3-4. group reverse pairs by target, reverse merge + prune
      reverse_step<false>(g, pa, ws, pb, bs, intx, cpl, timer, st, stream);
      count += bs;
      st.batches += 1;
      if (doubling && bs < mb) bs = std::min<int64_t>(mb, bs * 2);
    }
    hip_check(hipEventRecord(t1, stream), "event record");
    hip_check(hipStreamSynchronize(stream), "build synchronize");
    float total = 0;
    hip_check(hipEventElapsedTime(&total, t0, t1), "event elapsed");
    st.total_ms = total;
    if (wb.work) {
      std::vector<uint64_t> w((size_t)kWorkCount * kWorkCopies);
      hip_check(hipMemcpy(w.data(), wb.work, w.size() * 8, hipMemcpyDeviceToHost), "read build work counters");
      for (int i = 0; i < kWorkCount; ++i) {
        if (i == kWorkSearchQueries) continue;
        uint64_t sum = 0;
        for (int c = 0; c < kWorkCopies; ++c) sum += w[(size_t)i * kWorkCopies + c];
        st.work[i] = sum;
      }
    }
  } catch (...) {
    (void)hipStreamSynchronize(stream);
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    throw;
  }
  (void)hipEventDestroy(t0);
  (void)hipEventDestroy(t1);
  if (stats) *stats = st;
}

// ------------------------------------------------------ partitioned build

std::vector<std::pair<int64_t, int64_t>> scale_merge_order(int64_t P) {
  std::vector<std::pair<int64_t, int64_t>> order;
  int64_t B1 = 0;
  for (int64_t itv = 1; itv <= P / 2; ++itv) {
    const int64_t gg = std::gcd(itv, P), cycle_len = P / gg;
    const int64_t calls = cycle_len == 2 ? 1 : cycle_len;
    for (int64_t cyc = 0; cyc < gg; ++cyc) {
      if (cyc > 0) B1 = (B1 + 1) % P;
      for (int64_t step = 0; step < calls; ++step) {
        const int64_t B2 = (B1 + itv) % P;
        order.emplace_back(B1, B2);
        B1 = B2;
      }
    }
  }
  return order;
}

void build_scale(Graph& g, float alpha, int64_t n_parts, int64_t part_batch, int64_t merge_batch,
                 hipStream_t stream, ScaleStats* stats) {
  const int64_t n = g.n;
  if (n <= 0) throw std::invalid_argument("graph is empty");
  if (n_parts < 1) throw std::invalid_argument("n_parts must be positive");
  if (g.R > 64) throw std::invalid_argument("R must be <= 64");
  const int64_t part = (n + n_parts - 1) / n_parts;
  if (part * (n_parts - 1) >= n)
    throw std::invalid_argument("n_parts must be smaller: " + std::to_string(n_parts) +
                                " partitions of " + std::to_string(n) + " vectors leave one empty");
  if (part_batch < 1) part_batch = 1;
  if (merge_batch < 1) merge_batch = 1;
  ScaleStats st;
  st.part_batch = part_batch;
  hipEvent_t t0, t1, t2;
  hip_check(hipEventCreate(&t0), "event");
  hip_check(hipEventCreate(&t1), "event");
  hip_check(hipEventCreate(&t2), "event");
  struct Events {
    hipEvent_t* e[3];
    ~Events() { for (hipEvent_t* x : e) (void)hipEventDestroy(*x); }
  } ev{{&t0, &t1, &t2}};
  hip_check(hipEventRecord(t0, stream), "event record");

  // 1. each partition on its own: its rows start without edges and its
  //    search starts at its first row, so no edge leaves the partition --
  //    the reference's separate construct_graph plus apply_global_offset
  //    (construct_scale.cuh:107-124, graph.cuh:804-827), in place
  const uint32_t medoid = g.medoid;
  try {
    for (int64_t p = 0; p < n_parts; ++p) {
      const int64_t s = p * part, c = std::min(part, n - s);
      g.medoid = (uint32_t)s;
      build_range(g, alpha, s, s + c, part_batch, true, stream, false, nullptr);
    }
  } catch (...) {
    g.medoid = medoid;
    throw;
  }
  g.medoid = medoid;
  hip_check(hipEventRecord(t1, stream), "event record");

  // 2. merge every pair once (construct_scale.cuh:378-446), B1 in batches
  //    cut at 2^20-row segment boundaries (:362-364)
  const auto order = scale_merge_order(n_parts);
  if (!order.empty()) {
    const int64_t mb = std::min<int64_t>(merge_batch, part);
    st.merge_batch = mb;
    const uint32_t cpl = prune_cpl(g);
    BuildWorkspace ws(mb, g.R);
    const PairBits pb = pair_bits(mb, n);
    bool intx = false;
    PruneKernelArgs pa = prune_args(g, alpha, ws, pb.sb, stream, &intx);
    const size_t plds = prune_lds_bytes();
    EventTimer timer(false, stream);
    BuildStats bst;
    constexpr int64_t kSegment = (int64_t)1 << 20;
    for (const auto& m : order) {
      const int64_t b1s = m.first * part, n1 = std::min(part, n - b1s);
      const int64_t b2s = m.second * part, n2 = std::min(part, n - b2s);
      pa.pc.r1_lo = (uint32_t)b1s;
      pa.pc.r1_n = (uint32_t)n1;
      pa.pc.r2_lo = (uint32_t)b2s;
      pa.pc.r2_n = (uint32_t)n2;
      int64_t count = 0;
      while (count < n1) {
        const int64_t bs = std::min({mb, n1 - count, kSegment - count % kSegment});
        // 1. B1's batch searched in B2 alone, from B2's first row
        //    (construct_scale.cuh:190-213): edges leaving B2 are dropped
        SearchRequest r;
        r.use_range = true;
        r.q_start = (uint32_t)(b1s + count);
        r.nq = (uint32_t)bs;
        r.medoid = (uint32_t)b2s;
        r.id_lo = (uint32_t)b2s;
        r.id_n = n2;
        r.k = kBuildL;
        r.beam_width = kBuildL;
        r.limit = kBuildLimit;
        r.max_result = kBuildMaxResult;
        r.visited = ws.visited;
        r.visited_counts = ws.vcounts;
        r.hash_bits = seen_cache_hash_bits(n);
        launch_beam_search(g, r, stream);
        // 2. forward merge + merge prune into B1, pairs for B2 targets
        pa.batch_offset = (uint32_t)(b1s + count);
        if (intx && pa.pc.vecs8 && cpl == 4) launch_forward<4, kL2, true, true, true>(pa, (uint32_t)bs, plds, stream);
        else if (intx) dispatch_prune<kL2, true, true>(false, cpl, pa, (uint32_t)bs, plds, stream);
        else if (g.metric == kL2) dispatch_prune<kL2, false, true>(false, cpl, pa, (uint32_t)bs, plds, stream);
        else dispatch_prune<kIP, false, true>(false, cpl, pa, (uint32_t)bs, plds, stream);
        hip_check(hipGetLastError(), "launch forward_prune_kernel (merge)");
        // 3-4. reverse edges into B2 (process_reverse_edges_kernel_scale)
        reverse_step<true>(g, pa, ws, pb, bs, intx, cpl, timer, bst, stream);
        count += bs;
        st.merge_batches += 1;
      }
      st.merges += 1;
    }
  }
  hip_check(hipEventRecord(t2, stream), "event record");
  hip_check(hipStreamSynchronize(stream), "scale build synchronize");
  float a = 0, b = 0;
  hip_check(hipEventElapsedTime(&a, t0, t1), "event elapsed");
  hip_check(hipEventElapsedTime(&b, t1, t2), "event elapsed");
  st.partition_ms = a;
  st.merge_ms = b;
  st.total_ms = (double)a + b;
  if (stats) *stats = st;
}

// ------------------------------------------- staged (out-of-core) scale build

// Adds `off` to the valid edge ids of rows [0, n): a partition built with
// local ids (its first row is id 0) moves to its global ids (the reference's
// apply_global_offset, graph.cuh:804-827).
__global__ void offset_edges_kernel(uint32_t* edges, const uint8_t* counts, int64_t n, uint32_t R, uint32_t off) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n * (int64_t)R) return;
  const int64_t row = t / R;
  if ((uint32_t)(t % R) < counts[row]) edges[t] += off;
}

namespace {

// A Graph whose columns point into memory it does not own (a device slot,
// shifted so that global ids index it): the pointers are dropped before the
// Graph's destructor could free them.
struct GraphView {
  Graph g;
  ~GraphView() {
    g.vecs = nullptr;
    g.vecs8 = nullptr;
    g.edges = nullptr;
    g.edist = nullptr;
    g.counts = nullptr;
    g.deleted = nullptr;
    g.slot_to_id = nullptr;
  }
};

// One device slot of the staged merge: the columns of one partition.
struct StageSlot {
  Graph d;              // device columns for up to `part` rows (ids local)
  int64_t part_id = -1;
  int64_t lo = 0, rows = 0;
  bool dirty = false;   // adjacency changed since it was loaded
};

}  // namespace

void build_scale_staged(Graph& g, float alpha, int64_t n_parts, int64_t part_batch, int64_t merge_batch,
                        hipStream_t stream, ScaleStats* stats) {
  if (!g.on_host) throw std::invalid_argument("the staged build keeps the graph in host memory (on_host)");
  const int64_t n = g.n;
  if (n <= 0) throw std::invalid_argument("graph is empty");
  if (n_parts < 1) throw std::invalid_argument("n_parts must be positive");
  if (g.R > 64) throw std::invalid_argument("R must be <= 64");
  const int64_t part = (n + n_parts - 1) / n_parts;
  if (part * (n_parts - 1) >= n)
    throw std::invalid_argument("n_parts must be smaller: " + std::to_string(n_parts) + " partitions of " +
                                std::to_string(n) + " vectors leave one empty");
  if (part_batch < 1) part_batch = 1;
  if (merge_batch < 1) merge_batch = 1;
  const uint32_t R = g.R, dp = g.dp;
  ScaleStats st;
  st.part_batch = part_batch;
  hipEvent_t t0, t1, t2;
  hip_check(hipEventCreate(&t0), "event");
  hip_check(hipEventCreate(&t1), "event");
  hip_check(hipEventCreate(&t2), "event");
  struct Events {
    hipEvent_t* e[3];
    ~Events() { for (hipEvent_t* x : e) (void)hipEventDestroy(*x); }
  } ev{{&t0, &t1, &t2}};
  hip_check(hipEventRecord(t0, stream), "event record");

  // two device slots of `part` rows; the graph's columns stay in pinned host
  // memory (construct_scale.cuh:121-124, 398-445)
  StageSlot slot[2];
  for (StageSlot& x : slot) x.d.allocate(part, g.dim, R, g.metric, false);
  auto upload = [&](StageSlot& x, int64_t p) {
    x.part_id = p;
    x.lo = p * part;
    x.rows = std::min(part, n - x.lo);
    x.dirty = false;
    const size_t r = (size_t)x.rows;
    hip_check(hipMemcpyAsync(x.d.vecs, (const char*)g.vecs + (size_t)x.lo * dp * 2, r * dp * 2,
                             hipMemcpyHostToDevice, stream), "stage vectors in");
    hip_check(hipMemcpyAsync(x.d.edges, g.edges + (size_t)x.lo * R, r * R * 4, hipMemcpyHostToDevice, stream),
              "stage edges in");
    hip_check(hipMemcpyAsync(x.d.edist, g.edist + (size_t)x.lo * R, r * R * 2, hipMemcpyHostToDevice, stream),
              "stage edge distances in");
    hip_check(hipMemcpyAsync(x.d.counts, g.counts + x.lo, r, hipMemcpyHostToDevice, stream), "stage counts in");
  };
  auto write_back = [&](StageSlot& x) {
    if (x.part_id < 0 || !x.dirty) return;
    const size_t r = (size_t)x.rows;
    hip_check(hipMemcpyAsync(g.edges + (size_t)x.lo * R, x.d.edges, r * R * 4, hipMemcpyDeviceToHost, stream),
              "stage edges out");
    hip_check(hipMemcpyAsync(g.edist + (size_t)x.lo * R, x.d.edist, r * R * 2, hipMemcpyDeviceToHost, stream),
              "stage edge distances out");
    hip_check(hipMemcpyAsync(g.counts + x.lo, x.d.counts, r, hipMemcpyDeviceToHost, stream), "stage counts out");
    hip_check(hipStreamSynchronize(stream), "stage out");
    x.dirty = false;
  };

  // 1. each partition on its own in slot 0, with local ids (search from its
  //    first row), then shifted to global ids; the value ranges of all
  //    partitions together give the merges' integer test
  int32_t lo = 0, hi = -1;
  bool all_int = true;
  for (int64_t p = 0; p < n_parts; ++p) {
    StageSlot& x = slot[0];
    upload(x, p);
    Graph& d = x.d;
    d.n = x.rows;
    d.medoid = 0;
    scan_int_range(d, 0, x.rows, stream);
    if (int_range(d)) {
      lo = hi < lo ? d.int_lo : std::min(lo, d.int_lo);
      hi = hi < lo ? d.int_hi : std::max(hi, d.int_hi);
    } else {
      all_int = false;
    }
    build_range(d, alpha, 0, x.rows, part_batch, true, stream, false, nullptr);
    const int64_t total = x.rows * (int64_t)R;
    hipLaunchKernelGGL(offset_edges_kernel, dim3((uint32_t)((total + 255) / 256)), dim3(256), 0, stream, d.edges,
                       (const uint8_t*)d.counts, x.rows, R, (uint32_t)x.lo);
    hip_check(hipGetLastError(), "launch offset_edges_kernel");
    x.dirty = true;
    write_back(x);
    x.part_id = -1;
  }
  hip_check(hipEventRecord(t1, stream), "event record");

  // 2. merge every pair once in scale_merge_order: B1's batches searched in
  //    B2 alone, the forward prune into B1, the reverse prune into B2, with
  //    the two partitions in the slots (a partition shared with the previous
  //    pair stays on the device)
  const auto order = scale_merge_order(n_parts);
  if (!order.empty()) {
    const int64_t mb = std::min<int64_t>(merge_batch, part);
    st.merge_batch = mb;
    const uint32_t cpl = prune_cpl(g);
    BuildWorkspace ws(mb, R);
    const PairBits pb = pair_bits(mb, n);
    const bool intx = g.metric == kL2 && all_int && hi >= lo &&
                      (int64_t)hi - (int64_t)lo <= (int64_t)int_exact_span(g.dim);
    PruneKernelArgs pa{};
    pa.pair_shift = pb.sb;
    pa.pair_mask = (1u << pb.sb) - 1u;
    pa.pc.nchunks = dp / 8;
    pa.pc.nlimit = g.metric == kL2 ? g.dim / 8 : g.dim;  // the reference prunes with `dim`
    pa.pc.R = R;
    pa.pc.alpha = alpha;
    pa.pc.margin_scale = gram_margin_scale();
    pa.pc.staged = 1;
    pa.visited = ws.visited;
    pa.visited_counts = ws.vcounts;
    pa.pairs = ws.pairs;
    pa.sorted_pairs = ws.sorted;
    pa.heads = ws.heads;
    pa.n_heads = ws.nheads;
    {
      const _Float16 h = (_Float16)(intx ? lo : 0);  // exact: an fp16 value of the rows
      uint16_t bits;
      std::memcpy(&bits, &h, 2);
      pa.pc.lo2 = (uint32_t)bits * 0x10001u;
    }
    const size_t plds = prune_lds_bytes();
    EventTimer timer(false, stream);
    BuildStats bst;
    constexpr int64_t kSegment = (int64_t)1 << 20;
    for (const auto& m : order) {
      // slots for B1 and B2: keep whichever is already resident
      StageSlot* s1 = slot[0].part_id == m.first ? &slot[0] : slot[1].part_id == m.first ? &slot[1] : nullptr;
      StageSlot* s2 = slot[0].part_id == m.second ? &slot[0] : slot[1].part_id == m.second ? &slot[1] : nullptr;
      if (!s1) {
        s1 = s2 == &slot[0] ? &slot[1] : &slot[0];
        write_back(*s1);
        upload(*s1, m.first);
      }
      if (!s2) {
        s2 = s1 == &slot[0] ? &slot[1] : &slot[0];
        write_back(*s2);
        upload(*s2, m.second);
      }
      const int64_t b1s = s1->lo, n1 = s1->rows, b2s = s2->lo, n2 = s2->rows;
      // B2 as a graph over global ids (only its window is read)
      GraphView v2;
      Graph& gv = v2.g;
      gv.dim = g.dim;
      gv.dp = dp;
      gv.R = R;
      gv.metric = g.metric;
      gv.n = n;
      gv.capacity = n;
      gv.medoid = (uint32_t)b2s;
      gv.int_state = intx ? 1 : 2;
      gv.int_lo = lo;
      gv.int_hi = hi;
      gv.vecs = (char*)s2->d.vecs - (size_t)b2s * dp * 2;
      gv.edges = s2->d.edges - (size_t)b2s * R;
      gv.counts = s2->d.counts - b2s;
      pa.pc.vecs = (const uint4*)s1->d.vecs;
      pa.pc.vecs_b = (const uint4*)s2->d.vecs;
      pa.pc.r1_lo = (uint32_t)b1s;
      pa.pc.r1_n = (uint32_t)n1;
      pa.pc.r2_lo = (uint32_t)b2s;
      pa.pc.r2_n = (uint32_t)n2;
      int64_t count = 0;
      while (count < n1) {
        const int64_t bs = std::min({mb, n1 - count, kSegment - count % kSegment});
        SearchRequest r;
        r.queries = (const char*)s1->d.vecs + (size_t)count * dp * 2;
        r.nq = (uint32_t)bs;
        r.medoid = (uint32_t)b2s;
        r.id_lo = (uint32_t)b2s;
        r.id_n = n2;
        r.k = kBuildL;
        r.beam_width = kBuildL;
        r.limit = kBuildLimit;
        r.max_result = kBuildMaxResult;
        r.visited = ws.visited;
        r.visited_counts = ws.vcounts;
        r.hash_bits = seen_cache_hash_bits(n);
        launch_beam_search(gv, r, stream);
        // forward merge prune into B1 (its adjacency indexed by global id)
        pa.batch_offset = (uint32_t)(b1s + count);
        pa.edges = s1->d.edges - (size_t)b1s * R;
        pa.edist = s1->d.edist - (size_t)b1s * R;
        pa.counts = s1->d.counts - b1s;
        if (intx) dispatch_prune<kL2, true, true>(false, cpl, pa, (uint32_t)bs, plds, stream);
        else if (g.metric == kL2) dispatch_prune<kL2, false, true>(false, cpl, pa, (uint32_t)bs, plds, stream);
        else dispatch_prune<kIP, false, true>(false, cpl, pa, (uint32_t)bs, plds, stream);
        hip_check(hipGetLastError(), "launch forward_prune_kernel (staged merge)");
        // reverse merge prune into B2
        pa.edges = s2->d.edges - (size_t)b2s * R;
        pa.edist = s2->d.edist - (size_t)b2s * R;
        pa.counts = s2->d.counts - b2s;
        reverse_step<true>(g, pa, ws, pb, bs, intx, cpl, timer, bst, stream);
        count += bs;
        st.merge_batches += 1;
      }
      s1->dirty = s2->dirty = true;
      st.merges += 1;
    }
    for (StageSlot& x : slot) write_back(x);
  }
  hip_check(hipEventRecord(t2, stream), "event record");
  hip_check(hipStreamSynchronize(stream), "staged scale build synchronize");
  scan_int_range(g, 0, n, stream);
  float a = 0, b = 0;
  hip_check(hipEventElapsedTime(&a, t0, t1), "event elapsed");
  hip_check(hipEventElapsedTime(&b, t1, t2), "event elapsed");
  st.partition_ms = a;
  st.merge_ms = b;
  st.total_ms = (double)a + b;
  if (stats) *stats = st;
}

// ------------------------------------------------------------ live updates

void append_rows(Graph& g, const void* rows, int64_t count, float alpha, int32_t* out_ids, hipStream_t stream) {
  if (count <= 0) return;
  if (g.on_host) throw std::runtime_error("append_batch requires graph on device");
  const int64_t old_n = g.n, new_n = old_n + count;
  if (new_n > 0x7FFFFFFF) throw std::invalid_argument("too many vectors for 31-bit ids");
  // storage grows geometrically, so repeated appends are amortized
  if (new_n > g.capacity) g.reserve(std::max<int64_t>(new_n, g.capacity + g.capacity / 2), stream);
  upload_rows(g, rows, old_n, count, g.dim, stream);
  g.n = new_n;
  build_range(g, alpha, old_n, new_n, std::min<int64_t>(count, 100000), false, stream, false, nullptr);
  // fresh monotonic ids (id_map.cuh assign_ids, set_id_range_kernel)
  std::vector<uint32_t> ids((size_t)count);
  for (int64_t i = 0; i < count; ++i) ids[(size_t)i] = (uint32_t)(g.next_id + (uint64_t)i);
  g.next_id += (uint64_t)count;
  hip_check(hipMemcpyAsync(g.slot_to_id + old_n, ids.data(), (size_t)count * 4, hipMemcpyHostToDevice, stream),
            "write slot ids");
  hip_check(hipMemcpyAsync(out_ids, ids.data(), (size_t)count * 4, hipMemcpyDefault, stream), "write ids");
  hip_check(hipStreamSynchronize(stream), "append");
}

// mark_deleted_batch_kernel (deletion.cuh:21-42): one thread per id; the old
// word tells whether the id was newly deleted.
__global__ void mark_deleted_kernel(const int32_t* ids, int64_t n_ids, int64_t n, uint32_t* bits, uint32_t* newly) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_ids) return;
  const uint32_t v = (uint32_t)ids[i];
  if ((int64_t)v >= n) return;
  const uint32_t m = 1u << (v & 31u);
  if ((atomicOr(&bits[v >> 5], m) & m) == 0u) atomicAdd(newly, 1u);
}

// Lowest vertex whose tombstone bit is clear (out = n when none).
__global__ void first_live_kernel(const uint32_t* bits, int64_t n, uint32_t* out) {
  const int64_t words = (n + 31) / 32;
  for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < words; w += (int64_t)gridDim.x * blockDim.x) {
    uint32_t free_bits = ~bits[w];
    const int64_t base = w * 32;
    if (base + 32 > n) free_bits &= (1u << (uint32_t)(n - base)) - 1u;
    if (free_bits) atomicMin(out, (uint32_t)(base + __builtin_ctz(free_bits)));
  }
}

int64_t mark_deleted(Graph& g, const int32_t* ids, int64_t n_ids, hipStream_t stream) {
  if (n_ids <= 0 || g.n <= 0) return 0;
  if (g.on_host) throw std::runtime_error("mark_deleted requires graph on device");
  int32_t* d_ids = nullptr;
  uint32_t* d_cnt = nullptr;
  int64_t newly = 0;
  try {
    hip_check(hipMalloc(&d_ids, (size_t)n_ids * 4), "alloc ids");
    hip_check(hipMalloc(&d_cnt, 8), "alloc count");
    hip_check(hipMemcpyAsync(d_ids, ids, (size_t)n_ids * 4, hipMemcpyDefault, stream), "upload ids");
    hip_check(hipMemsetAsync(d_cnt, 0, 8, stream), "clear count");
    hipLaunchKernelGGL(mark_deleted_kernel, dim3((uint32_t)((n_ids + 255) / 256)), dim3(256), 0, stream, d_ids, n_ids,
                       g.n, g.deleted, d_cnt);
    hip_check(hipGetLastError(), "launch mark_deleted_kernel");
    uint32_t h = 0;
    hip_check(hipMemcpyAsync(&h, d_cnt, 4, hipMemcpyDeviceToHost, stream), "read count");
    hip_check(hipStreamSynchronize(stream), "mark deleted");
    newly = h;
    g.n_deleted += h;
    // update_medoid_if_deleted (graph_ops.cuh:50-88) with find_new_medoid_kernel
    // (deletion.cuh:245-266): the first live neighbour in edge order, else the
    // lowest live vertex
    uint32_t mw = 0;
    hip_check(hipMemcpy(&mw, g.deleted + (g.medoid >> 5), 4, hipMemcpyDeviceToHost), "read medoid bit");
    if ((mw >> (g.medoid & 31u)) & 1u) {
      uint8_t deg = 0;
      std::vector<uint32_t> row(g.R);
      hip_check(hipMemcpy(&deg, g.counts + g.medoid, 1, hipMemcpyDeviceToHost), "read medoid degree");
      hip_check(hipMemcpy(row.data(), g.edges + (size_t)g.medoid * g.R, (size_t)g.R * 4, hipMemcpyDeviceToHost),
                "read medoid edges");
      int64_t pick = -1;
      for (uint32_t j = 0; j < deg && j < g.R && pick < 0; ++j) {
        const uint32_t nb = row[j];
        if (nb == kInvalid32 || (int64_t)nb >= g.n) continue;
        uint32_t w = 0;
        hip_check(hipMemcpy(&w, g.deleted + (nb >> 5), 4, hipMemcpyDeviceToHost), "read bit");
        if (!((w >> (nb & 31u)) & 1u)) pick = nb;
      }
      if (pick < 0) {
        const uint32_t init = 0xFFFFFFFFu;
        hip_check(hipMemcpy(d_cnt, &init, 4, hipMemcpyHostToDevice), "init first live");
        const int64_t words = (g.n + 31) / 32;
        hipLaunchKernelGGL(first_live_kernel, dim3((uint32_t)std::min<int64_t>((words + 255) / 256, 4096)), dim3(256), 0,
                           stream, g.deleted, g.n, d_cnt);
        hip_check(hipGetLastError(), "launch first_live_kernel");
        uint32_t f = 0;
        hip_check(hipMemcpyAsync(&f, d_cnt, 4, hipMemcpyDeviceToHost, stream), "read first live");
        hip_check(hipStreamSynchronize(stream), "first live");
        if ((int64_t)f < g.n) pick = f;
      }
      if (pick >= 0) g.medoid = (uint32_t)pick;
      else std::fprintf(stderr, "Warning: update_medoid_if_deleted found no live vertex\n");
    }
  } catch (...) {
    (void)hipFree(d_ids);
    (void)hipFree(d_cnt);
    throw;
  }
  (void)hipFree(d_ids);
  (void)hipFree(d_cnt);
  return newly;
}

__device__ __forceinline__ bool is_deleted_bit(const uint32_t* bits, uint32_t v) {
  return ((bits[v >> 5] >> (v & 31u)) & 1u) != 0u;
}

// count / fill_repair_candidates_kernel (deletion.cuh:45-109), one wave per
// live vertex N of [n_min, n_max): the live neighbours M != N of each deleted
// neighbour D of N, in N's edge order and then D's. FILL writes the pairs
// (N << 32 | M) from offsets[N - n_min]; otherwise counts go to offsets.
template <bool FILL>
__global__ __launch_bounds__(256) void repair_candidates_kernel(const uint32_t* edges, const uint8_t* counts,
                                                                const uint32_t* bits, int64_t n, uint32_t R,
                                                                int64_t n_min, int64_t n_max, uint64_t* offsets,
                                                                uint64_t* pairs) {
  const uint32_t lane = lane_id();
  const int64_t N = n_min + (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (N >= n_max) return;
  if (is_deleted_bit(bits, (uint32_t)N)) {
    if constexpr (!FILL) {
      if (lane == 0) offsets[N - n_min] = 0;
    }
    return;
  }
  const uint32_t degN = min((uint32_t)counts[N], R);
  const uint32_t D = lane < degN ? edges[(size_t)N * R + lane] : kInvalid32;
  uint64_t dm = ballot(D != kInvalid32 && (int64_t)D < n && is_deleted_bit(bits, D));
  uint64_t pos = FILL ? offsets[N - n_min] : 0;
  while (dm) {
    const uint32_t j = (uint32_t)__builtin_ctzll(dm);
    dm &= dm - 1u;
    const uint32_t d = (uint32_t)__shfl((int)D, (int)j, 64);
    const uint32_t degD = min((uint32_t)counts[d], R);
    const uint32_t M = lane < degD ? edges[(size_t)d * R + lane] : kInvalid32;
    const bool ok = M != kInvalid32 && (int64_t)M < n && !is_deleted_bit(bits, M) && M != (uint32_t)N;
    const uint64_t m = ballot(ok);
    if constexpr (FILL) {
      if (ok) pairs[pos + mbcnt(m)] = ((uint64_t)N << 32) | M;
    }
    pos += (uint64_t)__builtin_popcountll(m);
  }
  if constexpr (!FILL) {
    if (lane == 0) offsets[N - n_min] = pos;
  }
}

// compact_deleted_neighbors_kernel (deletion.cuh:111-143): drops deleted
// neighbours from the lists of the live vertices of [n_min, n_max), keeping
// order and moving each distance with its edge.
__global__ __launch_bounds__(256) void drop_deleted_neighbors_kernel(uint32_t* edges, uint16_t* edist,
                                                                     uint8_t* counts, const uint32_t* bits,
                                                                     int64_t n, uint32_t R, int64_t n_min,
                                                                     int64_t n_max) {
  const uint32_t lane = lane_id();
  const int64_t N = n_min + (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (N >= n_max || is_deleted_bit(bits, (uint32_t)N)) return;
  const uint32_t deg = min((uint32_t)counts[N], R);
  const uint32_t e = lane < deg ? edges[(size_t)N * R + lane] : kInvalid32;
  const uint16_t w = lane < deg ? edist[(size_t)N * R + lane] : (uint16_t)0;
  const bool keep = e != kInvalid32 && (int64_t)e < n && !is_deleted_bit(bits, e);
  const uint64_t m = ballot(keep);
  if (keep) {
    const uint32_t k = mbcnt(m);
    edges[(size_t)N * R + k] = e;
    edist[(size_t)N * R + k] = w;
  }
  if (lane == 0) counts[N] = (uint8_t)__builtin_popcountll(m);
}

// clear_deleted_nodes_kernel (deletion.cuh:145-160)
__global__ void clear_deleted_nodes_kernel(uint32_t* edges, uint8_t* counts, const uint32_t* bits, int64_t n,
                                           uint32_t R) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t v = i / R;
  if (v >= n || !is_deleted_bit(bits, (uint32_t)v)) return;
  edges[i] = kInvalid32;
  if (i % R == 0) counts[v] = 0;
}

int64_t consolidate(Graph& g, float alpha, hipStream_t stream) {
  if (g.n_deleted == 0) return 0;
  if (g.on_host) throw std::runtime_error("consolidate requires graph on device");
  if (g.R > 64) throw std::invalid_argument("R must be <= 64");
  const int64_t n = g.n;
  const uint32_t R = g.R;
  const uint32_t nchunks = g.dp / 8;
  const uint32_t cpl = (nchunks + 3) / 4 > 8 ? 0u : (nchunks + 3) / 4;
  int32_t int_lo = 0;
  const bool intx = int_exact_l2(g, stream, &int_lo);
  // vertices per chunk, so that one chunk's candidates stay within bounds
  // (the reference splits the source range the same way, graph_ops.cuh:175-185)
  const int64_t chunk = std::min<int64_t>(n, (int64_t)1 << 20);
  uint64_t* per_vertex = nullptr;
  uint64_t* offsets = nullptr;
  uint64_t* pairs = nullptr;
  uint64_t* sorted = nullptr;
  uint32_t* heads = nullptr;
  uint32_t* nheads = nullptr;
  void* temp = nullptr;
  void* scan_temp = nullptr;
  size_t cap_pairs = 0, temp_bytes = 0, scan_bytes = 0;
  int64_t total_pairs = 0;
  auto cleanup = [&]() {
    (void)hipFree(per_vertex);
    (void)hipFree(offsets);
    (void)hipFree(pairs);
    (void)hipFree(sorted);
    (void)hipFree(heads);
    (void)hipFree(nheads);
    (void)hipFree(temp);
    (void)hipFree(scan_temp);
  };
  try {
    hip_check(hipMalloc(&per_vertex, (size_t)(chunk + 1) * 8), "alloc repair counts");
    hip_check(hipMalloc(&offsets, (size_t)(chunk + 1) * 8), "alloc repair offsets");
    hip_check(hipMalloc(&nheads, 4), "alloc head count");
    scan_bytes = scan_u64_temp_bytes((size_t)chunk + 1);
    hip_check(hipMalloc(&scan_temp, std::max<size_t>(scan_bytes, 16)), "alloc scan temp");
    int end_bit = 32;
    while (end_bit < 64 && ((uint64_t)1 << (end_bit - 32)) <= (uint64_t)n) ++end_bit;

    PruneKernelArgs pa{};
    pa.pc.vecs = (const uint4*)g.vecs;
    pa.pc.nchunks = nchunks;
    pa.pc.nlimit = g.metric == kL2 ? g.dim / 8 : g.dim;
    pa.pc.R = R;
    pa.pc.alpha = alpha;
    pa.pc.margin_scale = gram_margin_scale();
    {
      const _Float16 lo = (_Float16)int_lo;
      uint16_t bits;
      std::memcpy(&bits, &lo, 2);
      pa.pc.lo2 = (uint32_t)bits * 0x10001u;
    }
    set_byte_rows(pa.pc, g);
    pa.edges = g.edges;
    pa.edist = g.edist;
    pa.counts = g.counts;
    pa.batch_offset = 0;
    pa.pair_shift = 32;
    pa.pair_mask = 0xFFFFFFFFu;
    const size_t plds = prune_lds_bytes();

    for (int64_t n_min = 0; n_min < n; n_min += chunk) {
      const int64_t n_max = std::min<int64_t>(n, n_min + chunk), cn = n_max - n_min;
      const dim3 wgrid((uint32_t)((cn + 3) / 4));
      hipLaunchKernelGGL(repair_candidates_kernel<false>, wgrid, dim3(256), 0, stream, g.edges, g.counts, g.deleted,
                         n, R, n_min, n_max, per_vertex, (uint64_t*)nullptr);
      hip_check(hipGetLastError(), "launch repair_candidates_kernel");
      hip_check(hipMemsetAsync(per_vertex + cn, 0, 8, stream), "clear scan tail");
      exclusive_scan_u64(scan_temp, scan_bytes, per_vertex, offsets, (size_t)cn + 1, stream);
      uint64_t np = 0;
      hip_check(hipMemcpyAsync(&np, offsets + cn, 8, hipMemcpyDeviceToHost, stream), "read repair count");
      hip_check(hipStreamSynchronize(stream), "repair count");
      if (np > 0xFFFFFFFFull) throw std::runtime_error("too many repair candidates in one chunk");
      if (np > cap_pairs) {
        (void)hipFree(pairs);
        (void)hipFree(sorted);
        (void)hipFree(heads);
        (void)hipFree(temp);
        pairs = sorted = nullptr;
        heads = nullptr;
        temp = nullptr;
        cap_pairs = np;
        temp_bytes = sort_u64_temp_bytes(cap_pairs);
        hip_check(hipMalloc(&pairs, cap_pairs * 8), "alloc repair pairs");
        hip_check(hipMalloc(&sorted, cap_pairs * 8), "alloc sorted repair pairs");
        hip_check(hipMalloc(&heads, cap_pairs * 4), "alloc repair heads");
        hip_check(hipMalloc(&temp, std::max<size_t>(temp_bytes, 16)), "alloc sort temp");
      }
      if (np > 0) {
        hipLaunchKernelGGL(repair_candidates_kernel<true>, wgrid, dim3(256), 0, stream, g.edges, g.counts, g.deleted, n,
                           R, n_min, n_max, offsets, pairs);
        hip_check(hipGetLastError(), "launch repair_candidates_kernel");
      }
      hipLaunchKernelGGL(drop_deleted_neighbors_kernel, wgrid, dim3(256), 0, stream, g.edges, g.edist, g.counts,
                         g.deleted, n, R, n_min, n_max);
      hip_check(hipGetLastError(), "launch drop_deleted_neighbors_kernel");
      if (np == 0) continue;
      total_pairs += (int64_t)np;
      const uint32_t np32 = (uint32_t)np;
      sort_u64(temp, temp_bytes, pairs, sorted, np32, 0, end_bit, stream);
      hip_check(hipMemsetAsync(nheads, 0, 4, stream), "clear head count");
      hipLaunchKernelGGL(mark_heads_kernel, dim3((np32 + kMarkHeadsBlock - 1) / kMarkHeadsBlock),
                         dim3(kMarkHeadsBlock), 0, stream, sorted, np32, 32u, heads, nheads);
      hip_check(hipGetLastError(), "launch mark_heads_kernel");
      pa.sorted_pairs = sorted;
      pa.n_pairs = np32;
      pa.heads = heads;
      pa.n_heads = nheads;
      const uint32_t grid = (uint32_t)std::min<uint64_t>(np, 16384);
      if (intx && int8_rows(g)) dispatch_reverse_i8(cpl, pa, grid, plds, stream);
      else if (intx) dispatch_prune<kL2, true>(true, cpl, pa, grid, plds, stream);
      else if (g.metric == kL2) dispatch_prune<kL2, false>(true, cpl, pa, grid, plds, stream);
      else dispatch_prune<kIP, false>(true, cpl, pa, grid, plds, stream);
      hip_check(hipGetLastError(), "launch reverse_prune_kernel");
    }
    const int64_t slots = n * (int64_t)R;
    hipLaunchKernelGGL(clear_deleted_nodes_kernel, dim3((uint32_t)((slots + 255) / 256)), dim3(256), 0, stream,
                       g.edges, g.counts, g.deleted, n, R);
    hip_check(hipGetLastError(), "launch clear_deleted_nodes_kernel");
    hip_check(hipMemsetAsync(g.deleted, 0, (size_t)((n + 31) / 32) * 4, stream), "clear tombstones");
    hip_check(hipStreamSynchronize(stream), "consolidate");
  } catch (...) {
    (void)hipStreamSynchronize(stream);
    cleanup();
    throw;
  }
  cleanup();
  g.n_deleted = 0;
  return total_pairs;
}

}  // namespace jasper_amd
