// search.hip -- batched plain beam search, one wave64 per query.
//
// Reference: beam_search_kernel (include/jasper/beam_search/beam_search.cuh:
// 27-259) with the helpers of beam_search/device_kernels.cuh. The result is
// the reference's, bit for bit; the mechanics are redesigned for CDNA4:
//
//  * One 64-lane wave owns a query; no block barriers beyond the wave.
//  * The candidate list B (<= beam width) lives in LDS as sorted u64 keys
//    (order-preserving distance | 31-bit id | visited bit).
//  * A direct-mapped LDS cache of vertex ids skips re-fetching vectors that
//    were already scored by this query. This cannot change the result: a
//    vertex still in B would be removed by the reference's dedup (its key is
//    identical), and a vertex that was clipped out of B can never re-enter,
//    because the bw-th smallest key of B never increases once B is full.
//    The cache may forget ids (it is lossy); exactness does not depend on
//    it, because every new key is also checked for membership in B during
//    the merge (equal keys <=> same vertex).
//  * Adjacency rows are read as one coalesced 4R-byte load; each quad of
//    lanes scores one new neighbour with the reference's accumulation order
//    (lane l: chunks l, l+4, ...; quad sum (l0+l2)+(l1+l3)).
//  * New keys are sorted with a register bitonic network, deduplicated and
//    merged into B (in registers at bw <= 64, else in place in LDS), then
//    clipped to bw.
#include "common.hpp"
#include "search.hpp"

#include <algorithm>
#include <cstdlib>

namespace jasper_amd {

struct SearchArgs {
  const uint4* vecs;
  int64_t n;
  // neighbours are followed only when their id is in [id_lo, id_lo + id_n)
  // (the whole graph unless the request narrows it)
  uint32_t id_lo, id_n;
  uint32_t dp, nchunks, R;
  const uint32_t* edges;
  const uint8_t* counts;
  const uint32_t* deleted;
  const uint32_t* slot_to_id;
  const uint4* queries;
  uint32_t use_range, q_start, medoid;
  uint32_t k, bw, limit, max_result;
  int32_t* out_ids;
  float* out_dists;
  uint64_t* visited;
  uint32_t* visited_counts;
  uint32_t hash_bits;
  // seen-cache entry format: tag_bits = 0 stores full 32-bit ids; otherwise
  // 16-bit tags (see seen_test_insert) with dom_mask = 2^b - 1, b = hash_bits
  // + tag_bits >= log2(n)
  uint32_t tag_bits, dom_mask;
  uint32_t two_way;  // 16-bit entries as 2-way sets (one 32-bit word per set)
  // measurement mode: exact per-query seen bitmap in HBM and work counters
  uint32_t* seen_bits;      // [nq, seen_words]
  uint32_t seen_words;
  uint32_t* stats;          // [nq, 4]: hops, sum of degrees, vectors scored, predicted hops
  // byte rows (value - glo, 16 * nb8 bytes per row) when the graph keeps
  // them, and the query shift glo - 1024 as two fp16 (qsh2)
  const uint4* vecs8;
  uint32_t nb8, qsh2;
  // the graph's rows are integers in [glo, ghi] (gint); queries that are
  // integers too, with the union spanning at most smax, take the packed form
  uint32_t gint;
  int32_t glo, ghi, smax;
};

// Seen cache: returns true when v is recorded, else records it (replacing
// the slot's previous id). A hit is exact (never a false positive), a miss
// may be an id that was replaced, which only costs a re-score. With 16-bit
// entries the id is first mapped through h = v * K mod 2^b (K odd: a
// bijection of [0, 2^b), which holds every id below n); the top hash_bits
// bits of h pick the slot and the low tag_bits bits (+1, 0 = empty) are
// stored, so (slot, tag) still identifies v uniquely.
__device__ __forceinline__ bool seen_test_insert(const SearchArgs& a, uint32_t* H, uint32_t v) {
  const uint32_t hm = v * 0x9E3779B1u;
  if (a.tag_bits) {
    const uint32_t hd = hm & a.dom_mask;
    const uint32_t slot = hd >> a.tag_bits;
    const uint32_t tag = (hd & ((1u << a.tag_bits) - 1u)) + 1u;
    if (a.two_way) {
      // set of two tags, newest in the low half; a miss evicts the older
      const uint32_t w = H[slot];
      if ((w & 0xFFFFu) == tag || (w >> 16) == tag) return true;
      H[slot] = (w << 16) | tag;
      return false;
    }
    uint16_t* H16 = reinterpret_cast<uint16_t*>(H);
    if (H16[slot] == tag) return true;
    H16[slot] = (uint16_t)tag;
    return false;
  }
  const uint32_t slot = hm >> (32u - a.hash_bits);
  if (H[slot] == v) return true;
  H[slot] = v;
  return false;
}

// The query as a left operand: fp16 chunks for L2 (converted inside
// v_fma_mix_f32), fp32 elements for IP (quad_partial's broadcast layout),
// or for rows longer than 32 chunks (CPL = 0) its address.
template <int CPL, int METRIC>
using QueryFrag = LeftFrag<CPL, METRIC>;

// True (wave-uniform) when every value of the query is an integer and the
// query's values together with the graph's span at most smax: then every
// difference to a row is exact in fp16 and every partial sum of squares an
// exact fp32 integer, whatever the order.
template <int CPL>
__device__ __forceinline__ bool query_int_exact(const SearchArgs& a, const RowFrag<CPL>& qh) {
  bool ok = true;
  float lo = 65504.0f, hi = -65504.0f;
#pragma unroll
  for (int t = 0; t < CPL; ++t) {
    const uint32_t w[4] = {qh.x[t].x, qh.x[t].y, qh.x[t].z, qh.x[t].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        _Float16 hv;
        const uint16_t bits = (uint16_t)(w[k] >> (16 * e));
        __builtin_memcpy(&hv, &bits, 2);
        const float v = (float)hv;
        ok = ok && fabsf(v) <= 65504.0f && v == rintf(v);
        lo = fminf(lo, v);
        hi = fmaxf(hi, v);
      }
    }
  }
  if (ballot(!ok)) return false;
#pragma unroll
  for (int j = 1; j < 64; j <<= 1) {
    lo = fminf(lo, __shfl_xor(lo, j, 64));
    hi = fmaxf(hi, __shfl_xor(hi, j, 64));
  }
  const float ulo = fminf(lo, (float)a.glo), uhi = fmaxf(hi, (float)a.ghi);
  return uhi - ulo <= (float)a.smax;
}

// intx (wave-uniform): the query and the rows are integer-valued within
// the exact span (query_int_exact), so the packed-difference form gives the
// same bits.
template <int CPL, int METRIC>
__device__ __forceinline__ float score(const SearchArgs& a, const QueryFrag<CPL, METRIC>& q, const RowFrag<CPL>& x,
                                       uint32_t ql, uint32_t nlimit, bool intx) {
  if constexpr (METRIC == kL2 && CPL > 0) {
    if (intx) return left_distance<CPL, METRIC, true>(q, x, ql, a.nchunks, nlimit);
  }
  return left_distance<CPL, METRIC, false>(q, x, ql, a.nchunks, nlimit);
}

// ---- byte rows (common.hpp: load_query_bytes, load_row_bytes, score_bytes)
__device__ __forceinline__ void load_query_bytes(const SearchArgs& a, const uint4* qrow, uint32_t ql,
                                                 uint4 (&q)[4]) {
  load_query_bytes(qrow, a.nb8, a.qsh2, ql, q);
}
__device__ __forceinline__ void load_row_bytes(const SearchArgs& a, uint32_t v, uint32_t ql, RowBytes& r) {
  load_row_bytes(a.vecs8, a.nb8, v, ql, r);
}
__device__ __forceinline__ float score_bytes(const SearchArgs& a, const uint4 (&q)[4], const RowBytes& r,
                                             uint32_t ql) {
  return score_bytes(a.nb8, q, r, ql);
}

// Appends the key of a scored row to T[nt..) when its rank is below thr
// (the quad's first lane writes); returns the new count (wave-uniform).
__device__ __forceinline__ uint32_t append_key(uint64_t* T, uint32_t nt, bool act, uint32_t ql, float d, uint32_t v,
                                               uint64_t thr) {
  const uint64_t key = make_key(d, v);
  const bool w = ql == 0 && act && key_rank(key) < thr;
  const uint64_t m = ballot(w);
  if (w) T[nt + mbcnt(m)] = key;
  return nt + (uint32_t)__builtin_popcountll(m);
}

// Scores up to 16 (or 32 with TWO) candidate rows listed in cand[base..)
// and appends the keys that rank below thr to T[nt..); returns the count.
template <int CPL, int METRIC, bool TWO>
__device__ __forceinline__ uint32_t score_pass(const SearchArgs& a, const QueryFrag<CPL, METRIC>& qf,
                                               const uint32_t* cand, uint64_t* T, uint32_t base, uint32_t nm,
                                               uint32_t ql, uint32_t qg, bool intx, uint64_t thr, uint32_t nt) {
  const uint32_t nlimit = METRIC == kL2 ? a.nchunks : a.dp;
  const uint32_t j0 = base + qg;
  const bool act0 = j0 < nm;
  const uint32_t v0 = act0 ? cand[j0] : a.id_lo;  // inactive lanes read the window's first row
  RowFrag<CPL> x0;
  load_row_frag<CPL>(a.vecs + (size_t)v0 * a.nchunks, ql, a.nchunks, act0, x0);
  if constexpr (TWO) {
    const uint32_t j1 = base + 16u + qg;
    const bool act1 = j1 < nm;
    const uint32_t v1 = act1 ? cand[j1] : a.id_lo;
    RowFrag<CPL> x1;
    load_row_frag<CPL>(a.vecs + (size_t)v1 * a.nchunks, ql, a.nchunks, act1, x1);
    const float d0 = score<CPL, METRIC>(a, qf, x0, ql, nlimit, intx);
    const float d1 = score<CPL, METRIC>(a, qf, x1, ql, nlimit, intx);
    nt = append_key(T, nt, act0, ql, d0, v0, thr);
    return append_key(T, nt, act1, ql, d1, v1, thr);
  } else {
    const float d0 = score<CPL, METRIC>(a, qf, x0, ql, nlimit, intx);
    return append_key(T, nt, act0, ql, d0, v0, thr);
  }
}

// score_pass on the byte rows (U8: the query held as bytes, left_bytes_u8).
// Inactive lanes read row 0 (a constant: measured 1.5 % faster at config 2's
// bw 44 than a row id from the arguments); byte rows are only read through
// the graph's own arrays, where row 0 exists (the staged merge's shifted
// views carry no byte rows).
template <bool TWO, bool U8 = false>
__device__ __forceinline__ uint32_t score_pass_bytes(const SearchArgs& a, const uint4 (&q8)[4], const uint32_t* cand,
                                                     uint64_t* T, uint32_t base, uint32_t nm, uint32_t ql,
                                                     uint32_t qg, uint64_t thr, uint32_t nt) {
  const uint32_t j0 = base + qg;
  const bool act0 = j0 < nm;
  const uint32_t v0 = act0 ? cand[j0] : 0u;
  RowBytes x0;
  load_row_bytes(a, v0, ql, x0);
  if constexpr (TWO) {
    const uint32_t j1 = base + 16u + qg;
    const bool act1 = j1 < nm;
    const uint32_t v1 = act1 ? cand[j1] : 0u;
    RowBytes x1;
    load_row_bytes(a, v1, ql, x1);
    const float d0 = (U8 ? score_bytes_u8(a.nb8, q8[0], q8[1], q8[2].x, x0, ql) : score_bytes(a, q8, x0, ql));
    const float d1 = (U8 ? score_bytes_u8(a.nb8, q8[0], q8[1], q8[2].x, x1, ql) : score_bytes(a, q8, x1, ql));
    nt = append_key(T, nt, act0, ql, d0, v0, thr);
    return append_key(T, nt, act1, ql, d1, v1, thr);
  } else {
    const float d0 = (U8 ? score_bytes_u8(a.nb8, q8[0], q8[1], q8[2].x, x0, ql) : score_bytes(a, q8, x0, ql));
    return append_key(T, nt, act0, ql, d0, v0, thr);
  }
}

// At dim <= 128 with L2 the registers fit six waves per SIMD (the LDS of a
// query at bw <= 64 is about 5.6 KB, so registers decide the occupancy).
// Streamed long rows hold no row in registers.
// two rows per quad in flight in the score passes (tuning)
#ifndef JASPER_SEARCH_TWO_ROWS
#define JASPER_SEARCH_TWO_ROWS 1
#endif
#ifndef JASPER_SEARCH_WAVES_L2
#define JASPER_SEARCH_WAVES_L2 6
#endif
// graphs with byte rows: two byte rows (16 VGPRs) in flight, the fp16 rows of
// the few queries outside the exact span one at a time (72 VGPRs: seven waves
// fit, but measured 0.445 ms against 0.436 ms at six on config 2, bw 44: the
// hop's chain of dependent reads, not residency, sets the pace)
#ifndef JASPER_SEARCH_WAVES_BYTES
#define JASPER_SEARCH_WAVES_BYTES 6
#endif
template <int CPL, int METRIC, bool BYTES>
constexpr int search_waves_per_simd() {
  return BYTES ? JASPER_SEARCH_WAVES_BYTES
               : CPL == 0 ? 4 : (CPL <= 4 && METRIC == kL2) ? JASPER_SEARCH_WAVES_L2 : 1;
}

// Merge of the sorted new keys t (nt of them, one per lane) into B held one
// key per lane (b, cnt entries, bw <= 64): B ascending against the new keys
// reversed, the lane-wise minima are a bitonic sequence holding the 64
// smallest keys, sorted by six more stages. Equal ranks (a re-scored member
// of B, an id scored twice) sit side by side in the merged order, or across
// its 64th key: then nothing changes and false is returned (the general
// path takes the hop).
__device__ __forceinline__ bool merge_regs(uint64_t& b, uint64_t t, uint32_t nt, uint32_t& cnt, uint32_t bw,
                                           uint32_t lane) {
  const uint64_t tr = reverse_lanes64(t);
  const bool lt = b < tr;
  uint64_t x0 = lt ? b : tr;
  const uint64_t x1 = lt ? tr : b;
  x0 = bitonic_merge_steps<64, 32>(x0, lane);
  const uint64_t nx = __shfl_down(x0, 1, 64);
  const uint64_t last = readlane64(x0, 63);
  const bool dup = (lane < 63u && x0 != kEmptyKey && key_rank(x0) == key_rank(nx)) ||
                   (last != kEmptyKey && key_rank(x1) == key_rank(last));
  if (ballot(dup) != 0) return false;
  cnt = uniform(min(cnt + nt, bw));
  b = lane < cnt ? x0 : kEmptyKey;
  return true;
}

// General merge of the sorted new keys t (nt of them) into B[0, cnt) in LDS:
// equal neighbours are dropped, and so is any key already in B (a binary
// search in LDS); the rest are merged in place, clipped to bw. Kept key i
// (compacted to T[i]) lands at p_i = lb_i + i, and that position is marked
// in TAG with i (cleared again after the merge); entries of B below the
// smallest kept key's position lb0 keep their places, and every other output
// position o >= lb0 takes B[o - (placed keys below o)]. The 64-entry chunks
// of [lb0, ncnt) run from the top down, so a chunk reads only entries that
// are not yet overwritten (its own reads precede its writes). Returns false
// when every new key was a repeat or a member of B (B unchanged).
__device__ __forceinline__ bool merge_general(uint64_t* B, uint64_t* T, uint32_t* TAG, uint64_t t, uint32_t nt,
                                              uint32_t& cnt, uint32_t& hint, uint32_t bw, uint32_t lane) {
  const uint64_t prev = __shfl_up(t, 1, 64);
  bool keep = lane < nt && !(lane > 0 && key_rank(prev) == key_rank(t));
  uint32_t lb = 0;
  const uint32_t top = pow2_ceil(cnt);
  if (lane < nt) {
    lb = lds_lower_bound(B, cnt, top, key_rank(t));
    if (lb < cnt && key_rank(B[lb]) == key_rank(t)) keep = false;
  }
  const uint64_t km = ballot(keep);
  const uint32_t nk = (uint32_t)__builtin_popcountll(km);
  if (nk == 0) return false;
  const uint32_t ti = mbcnt(km);
  wave_sync();
  if (keep) T[ti] = t;
  wave_sync();
  const uint32_t lb0 = uniform((uint32_t)__shfl((int)lb, (int)__builtin_ctzll(km), 64));
  const uint32_t ncnt = min(cnt + nk, bw);
  const bool placed = keep && ti + lb < ncnt;
  if (placed) TAG[ti + lb] = 0x100u | ti;
  // kept keys that land inside the clipped list (the others fall past it)
  const uint32_t np = (uint32_t)__builtin_popcountll(ballot(placed));
  wave_sync();
  uint32_t above = 0;  // kept keys above the current chunk
  for (int32_t o0 = (int32_t)(lb0 + ((ncnt - 1u - lb0) & ~63u)); o0 >= (int32_t)lb0; o0 -= 64) {
    const uint32_t o = (uint32_t)o0 + lane;
    const bool valid = o < ncnt;
    const uint32_t tg = valid ? TAG[o] : 0u;
    const bool isnew = tg != 0u;
    const uint64_t m = ballot(isnew);
    // kept keys at positions >= o: above, plus this chunk's from lane on
    const uint32_t ge = above + (uint32_t)__builtin_popcountll(m >> lane);
    uint64_t v = 0;
    if (isnew) v = T[tg & 0xFFu];
    else if (valid) v = B[o - (np - ge)];
    if (valid) B[o] = v;
    above = uniform(above + (uint32_t)__builtin_popcountll(m));
  }
  if (placed) TAG[ti + lb] = 0u;
  hint = uniform(min(hint, lb0));
  cnt = uniform(ncnt);
  wave_sync();
  return true;
}

// BYTES: the graph keeps byte rows (CPL 4, L2, no measurement mode)
template <int CPL, int METRIC, bool STATS, bool BYTES = false>
__global__ __launch_bounds__(64, (search_waves_per_simd<CPL, METRIC, BYTES>())) void beam_search_kernel(
    SearchArgs a) {
  static_assert(!BYTES || (CPL == 4 && METRIC == kL2 && !STATS), "byte rows: L2 rows of 112 or 128 values");
  extern __shared__ uint64_t smem[];
  const uint32_t lane = threadIdx.x;
  const uint32_t qid = blockIdx.x;
  const uint32_t bw = a.bw;
  uint64_t* B = smem;                                     // [bw] the candidate list
  uint64_t* T = smem + bw;                                // [64] new keys
  uint32_t* cand = reinterpret_cast<uint32_t*>(T + 64);   // [64] new neighbour ids
  uint32_t* TAG = cand + 64;                              // [bw] merge position tags
  uint32_t* H = TAG + bw;                                 // seen cache
  {
    // 32-bit words of the cache: empty = all ones (ids) or zero (tags)
    const uint32_t words = a.tag_bits ? (1u << a.hash_bits) / 2u : 1u << a.hash_bits;
    const uint32_t fill = a.tag_bits ? 0u : kInvalid32;
    for (uint32_t i = lane; i < words; i += 64) H[i] = fill;
    for (uint32_t i = lane; i < bw; i += 64) TAG[i] = 0u;  // no position marked
  }

  const uint32_t ql = lane & 3u, qg = lane >> 2;
  const uint4* qrow = a.use_range ? a.vecs + (size_t)(a.q_start + qid) * a.nchunks
                                  : a.queries + (size_t)qid * a.nchunks;
  QueryFrag<CPL, METRIC> qf;
  load_left<CPL, METRIC>(qrow, ql, a.nchunks, qf);
  const uint32_t nlimit = METRIC == kL2 ? a.nchunks : a.dp;
  bool intx = false;
  if constexpr (METRIC == kL2 && CPL > 0 && !STATS) {
    if (a.gint) intx = uniform(query_int_exact<CPL>(a, qf.h) ? 1u : 0u) != 0u;
  }
  // byte rows for this query (wave-uniform; rows of 112 or 128 values).
  // From here on such a query is held shifted, in byte-chunk order, in the
  // registers of its fp16 fragment, which it no longer uses.
  // A query whose values also lie in [glo, glo + 255] then moves on to its
  // bytes (u8q): qf.h.x[0..1] its byte chunks, qf.h.x[2].x the lane's sum of
  // their squares (left_bytes_u8).
  bool bytes = false, u8q = false;
  if constexpr (BYTES) {
    bytes = intx;
    if (bytes) {
      load_query_bytes(a, qrow, ql, qf.h.x);
      uint4 qb[2];
      uint32_t qn;
      u8q = left_bytes_u8(a.nb8, qf.h.x, ql, qb, qn);
      if (u8q) {
        qf.h.x[0] = qb[0];
        qf.h.x[1] = qb[1];
        qf.h.x[2].x = qn;
      }
    }
  }

  // B = [(medoid, d(q, medoid))]; at bw <= 64 B lives in registers, one key
  // per lane (`b`), and is written to LDS only for the merge's general path
  // and the epilogue
  const bool regb = bw <= 64u;
  uint32_t cnt = 1;
  uint64_t b = kEmptyKey;
  {
    float d = 0.0f;
    if (bytes) {
      if constexpr (BYTES) {
        RowBytes xb;
        load_row_bytes(a, a.medoid, ql, xb);
        d = u8q ? score_bytes_u8(a.nb8, qf.h.x[0], qf.h.x[1], qf.h.x[2].x, xb, ql) : score_bytes(a, qf.h.x, xb, ql);
      }
    } else {
      RowFrag<CPL> x;
      load_row_frag<CPL>(a.vecs + (size_t)a.medoid * a.nchunks, ql, a.nchunks, true, x);
      d = score<CPL, METRIC>(a, qf, x, ql, nlimit, intx);
    }
    if (lane == 0) b = make_key(d, a.medoid);
    wave_sync();  // hash table initialised
    if (lane == 0) {
      B[0] = make_key(d, a.medoid);
      seen_test_insert(a, H, a.medoid);
      if constexpr (STATS) atomicOr(&a.seen_bits[(size_t)qid * a.seen_words + (a.medoid >> 5)], 1u << (a.medoid & 31u));
    }
  }
  wave_sync();
  uint32_t st_hops = 0, st_deg = 0, st_scored = 1, st_pred = 0;

  uint32_t hint = 0, vc = 0, loop = 0;
  // adjacency (degree, row) of the predicted next pop, loaded one hop ahead
  // so that a correct prediction takes the adjacency read off the hop's
  // chain of dependent memory reads; the prediction is the next unvisited
  // entry of B, which is the next pop unless a new neighbour displaces it
  const uint32_t elane = min(lane, a.R - 1u);
  uint32_t spec_u = kInvalid32, spec_c = 0, spec_v = kInvalid32;
  while (loop <= a.limit) {
    loop += 1;
    // ---- pop: first unvisited entry (all entries before `hint` are visited)
    uint64_t pk;
    uint32_t next_u;
    if (regb) {
      const uint64_t m = ballot(lane < cnt && !key_visited(b));
      if (m == 0) break;
      const uint32_t p = (uint32_t)__builtin_ctzll(m);
      const uint64_t m2 = m & (m - 1u);
      pk = readlane64(b, (int)p) | 1ull;
      next_u = uniform(m2 ? key_id(readlane64(b, (int)__builtin_ctzll(m2))) : kInvalid32);
      if (lane == p) b = pk;
      if (a.visited && lane == 0) a.visited[(size_t)qid * a.max_result + vc] = pk;
    } else {
      int p = -1, p2 = -1;
      for (uint32_t base = hint; base < cnt; base += 64) {
        const uint32_t i = base + lane;
        const bool unv = i < cnt && !key_visited(B[i]);
        const uint64_t m = ballot(unv);
        if (m) {
          p = (int)(base + (uint32_t)__builtin_ctzll(m));
          const uint64_t m2 = m & (m - 1u);
          if (m2) p2 = (int)(base + (uint32_t)__builtin_ctzll(m2));
          break;
        }
      }
      if (p < 0) break;
      pk = B[p] | 1ull;
      next_u = uniform(p2 >= 0 ? key_id(B[p2]) : kInvalid32);
      wave_sync();
      if (lane == 0) {
        B[p] = pk;
        if (a.visited) a.visited[(size_t)qid * a.max_result + vc] = pk;
      }
      hint = uniform((uint32_t)p + 1);
    }
    vc = uniform(vc + 1u);
    if (vc == a.max_result) break;

    // ---- expand: one coalesced row read (degree and row issued together,
    //      or taken from the prediction), filter through the seen cache
    const uint32_t u = uniform(key_id(pk));
    uint32_t cu, v;
    if (u == spec_u) {
      cu = spec_c;
      v = spec_v;
      if constexpr (STATS) st_pred += 1;
    } else {
      cu = a.counts[u];
      v = a.edges[(size_t)u * a.R + elane];
    }
    // the next prediction's reads, unconditional (a valid id either way)
    {
      const uint32_t su = next_u != kInvalid32 ? next_u : u;
      spec_u = next_u;
      spec_c = a.counts[su];
      spec_v = a.edges[(size_t)su * a.R + elane];
    }
    const uint32_t deg = min(cu, a.R);
    bool isnew = lane < deg && v - a.id_lo < a.id_n;
    if constexpr (STATS) {
      // exact filter: first time this query sees v
      if (isnew) {
        const uint32_t bit = 1u << (v & 31u);
        isnew = (atomicOr(&a.seen_bits[(size_t)qid * a.seen_words + (v >> 5)], bit) & bit) == 0u;
      }
    } else if (isnew) {
      isnew = !seen_test_insert(a, H, v);
    }
    const uint64_t newm = ballot(isnew);
    const uint32_t nm = (uint32_t)__builtin_popcountll(newm);
    if constexpr (STATS) {
      st_hops += 1;
      st_deg += deg;
      st_scored += nm;
    }
    if (isnew) cand[mbcnt(newm)] = v;
    wave_sync();

    // ---- score the new neighbours (4 lanes per vector). Once B is full,
    //      a key ranked above B's last cannot enter: B's bw distinct ranks
    //      all survive the dedup and precede it, so after the clip it is
    //      gone; a key equal to B's last is that member again. Only keys
    //      ranked below B's last are kept (nt of them), and a hop that
    //      keeps none leaves B as it is.
    uint64_t thr = ~0ull;
    if (cnt == bw) thr = key_rank(regb ? readlane64(b, (int)(bw - 1u)) : B[bw - 1u]);
    uint32_t nt = 0, base = 0;
    if (bytes) {
      if constexpr (BYTES) {
        if (u8q) {
          for (; base + 16 < nm; base += 32)
            nt = score_pass_bytes<true, true>(a, qf.h.x, cand, T, base, nm, ql, qg, thr, nt);
          if (base < nm) nt = score_pass_bytes<false, true>(a, qf.h.x, cand, T, base, nm, ql, qg, thr, nt);
        } else {
          for (; base + 16 < nm; base += 32)
            nt = score_pass_bytes<true>(a, qf.h.x, cand, T, base, nm, ql, qg, thr, nt);
          if (base < nm) nt = score_pass_bytes<false>(a, qf.h.x, cand, T, base, nm, ql, qg, thr, nt);
        }
      }
    } else {
#if JASPER_SEARCH_TWO_ROWS
      if constexpr (!BYTES) {
        for (; base + 16 < nm; base += 32)
          nt = score_pass<CPL, METRIC, true>(a, qf, cand, T, base, nm, ql, qg, intx, thr, nt);
      }
#endif
      for (; base + 16 < nm; base += 16)
        nt = score_pass<CPL, METRIC, false>(a, qf, cand, T, base, nm, ql, qg, intx, thr, nt);
      if (base < nm) nt = score_pass<CPL, METRIC, false>(a, qf, cand, T, base, nm, ql, qg, intx, thr, nt);
    }
    if (nt == 0) {
      lds_wave_sync();
      continue;
    }
    wave_sync();

    // ---- sort the new keys, merge them into B
    uint64_t t = lane < nt ? T[lane] : kEmptyKey;
    t = wave_sort_upto(t, nt);
    if (regb && merge_regs(b, t, nt, cnt, bw, lane)) {
      lds_wave_sync();
      continue;
    }
    if (regb) {
      // B to LDS for the general path
      if (lane < cnt) B[lane] = b;
      hint = 0;
      wave_sync();
    }
    if (!merge_general(B, T, TAG, t, nt, cnt, hint, bw, lane)) {
      lds_wave_sync();
      continue;
    }
    if (regb) b = lane < cnt ? B[lane] : kEmptyKey;
  }
  if (regb) {
    if (lane < cnt) B[lane] = b;
    wave_sync();
  }

  // ---- output: first k valid, non-deleted entries, then padding
  //      (beam_search.cuh:206-222, id translation id_map.cuh:49-56,
  //       unpacking ffi/jasper_ffi_common.cuh:193-203)
  if (a.out_ids) {
    uint32_t out = 0;
    for (uint32_t base = 0; base < cnt && out < a.k; base += 64) {
      const uint32_t i = base + lane;
      bool ok = i < cnt;
      uint64_t key = 0;
      uint32_t id = 0;
      if (ok) {
        key = B[i];
        id = key_id(key);
        ok = (a.deleted[id >> 5] >> (id & 31u) & 1u) == 0u;
      }
      const uint64_t m = ballot(ok);
      const uint32_t pos = out + mbcnt(m);
      if (ok && pos < a.k) {
        a.out_ids[(size_t)qid * a.k + pos] = (int32_t)(a.slot_to_id ? a.slot_to_id[id] : id);
        a.out_dists[(size_t)qid * a.k + pos] = key_dist(key);
      }
      out += (uint32_t)__builtin_popcountll(m);
    }
    for (uint32_t i = out + lane; i < a.k; i += 64) {
      a.out_ids[(size_t)qid * a.k + i] = -1;
      a.out_dists[(size_t)qid * a.k + i] = 1e30f;
    }
  }
  if (a.visited_counts && lane == 0) a.visited_counts[qid] = vc;
  if constexpr (STATS) {
    if (lane == 0) {
      a.stats[(size_t)qid * 4 + 0] = st_hops;
      a.stats[(size_t)qid * 4 + 1] = st_deg;
      a.stats[(size_t)qid * 4 + 2] = st_scored;
      a.stats[(size_t)qid * 4 + 3] = st_pred;
    }
  }
}

// Tag width of 16-bit seen-cache entries for a graph of n vertices, or 0
// when the ids need full 32-bit entries (more than 15 tag bits).
static uint32_t seen_tag_bits(int64_t n, uint32_t hash_bits) {
  uint32_t b = 1;
  while (b < 32 && ((int64_t)1 << b) < n) ++b;
  b = std::max(b, hash_bits + 1);
  return b - hash_bits <= 15 ? b - hash_bits : 0u;
}

// Size of the per-query seen cache (2^hash_bits entries) for a graph of n
// vertices, shared by queries and the build's searches. Up to 2^25 ids the
// entries are 15-bit tags in two-way sets, 2^11 of them (4 KB): on config 2
// (1M) this beat 2^10 (more re-scoring) and 2^12 or 2^13 (fewer resident
// waves) at bw 32..384. Up to 2^27 ids, 2^12 direct-mapped 16-bit tags (8 KB):
// at 100M vectors they beat 2^10 and 2^11 full 32-bit ids by 9-18 % at bw
// 32..128. Beyond, 2^11 32-bit ids (8 KB).
uint32_t seen_cache_hash_bits(int64_t n) {
  if (n <= ((int64_t)1 << 25)) return 11;
  if (n <= ((int64_t)1 << 27)) return 12;
  return 11;
}

static uint32_t default_hash_bits(uint32_t bw, int64_t n) {
  // JASPER_SEARCH_HASH_BITS (8..15) overrides the size of the per-query seen
  // cache for tuning; the results do not depend on it.
  static const int override_bits = [] {
    const char* e = std::getenv("JASPER_SEARCH_HASH_BITS");
    const int v = e ? std::atoi(e) : 0;
    return (v >= 8 && v <= 15) ? v : 0;
  }();
  if (override_bits) return (uint32_t)override_bits;
  (void)bw;
  return seen_cache_hash_bits(n);
}

size_t beam_search_lds_bytes(const Graph& g, const SearchRequest& r) {
  const uint32_t hb = r.hash_bits ? r.hash_bits : default_hash_bits(r.beam_width, g.n);
  const size_t entry = seen_tag_bits(g.n, hb) ? 2 : 4;
  return (size_t)r.beam_width * 8 + 64 * 8 + 64 * 4 + (size_t)r.beam_width * 4 +
         std::max<size_t>(((size_t)1 << hb) * entry, 4);
}

template <int CPL, int METRIC, bool STATS, bool BYTES = false>
static void launch_one(const SearchArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
  auto kern = beam_search_kernel<CPL, METRIC, STATS, BYTES>;
  if (lds > 64 * 1024)
    hip_check(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
              "set LDS size");
  hipLaunchKernelGGL(kern, grid, dim3(64), lds, stream, a);
}

void launch_beam_search(const Graph& g, const SearchRequest& r, hipStream_t stream) {
  if (r.nq == 0) return;
  if (r.beam_width == 0) throw std::invalid_argument("beam_width must be positive");
  if (r.beam_width + 64 >= 2048)
    throw std::invalid_argument("beam_width " + std::to_string(r.beam_width) +
                                " is too large (beam_width + 64 must be < 2048)");
  if (g.R > 64) throw std::invalid_argument("R must be <= 64");
  if (g.n <= 0) throw std::invalid_argument("graph is empty");
  if ((int64_t)r.medoid >= g.n) throw std::invalid_argument("medoid out of range");
  if (r.use_range && (int64_t)r.q_start + r.nq > g.n) throw std::invalid_argument("query range out of bounds");
  const int64_t win_n = r.id_n < 0 ? g.n : r.id_n;
  if ((int64_t)r.id_lo + win_n > g.n || win_n == 0) throw std::invalid_argument("id window outside the graph");
  if (r.medoid < r.id_lo || (int64_t)r.medoid >= (int64_t)r.id_lo + win_n)
    throw std::invalid_argument("medoid outside the id window");
  SearchArgs a{};
  a.vecs = (const uint4*)g.vecs;
  a.n = g.n;
  a.id_lo = r.id_lo;
  a.id_n = (uint32_t)win_n;
  a.dp = g.dp;
  a.nchunks = g.dp / 8;
  a.R = g.R;
  a.edges = g.edges;
  a.counts = g.counts;
  a.deleted = g.deleted;
  a.slot_to_id = g.slot_to_id;
  a.queries = (const uint4*)r.queries;
  a.use_range = r.use_range ? 1u : 0u;
  a.q_start = r.q_start;
  a.medoid = r.medoid;
  a.k = r.k;
  a.bw = r.beam_width;
  a.limit = r.limit;
  a.max_result = r.max_result;
  a.out_ids = r.out_ids;
  a.out_dists = r.out_dists;
  a.visited = r.visited;
  a.visited_counts = r.visited_counts;
  a.hash_bits = r.hash_bits ? r.hash_bits : default_hash_bits(r.beam_width, g.n);
  {
    // JASPER_SEARCH_SEEN_WAYS=1 keeps direct-mapped 16-bit entries (tuning)
    static const bool direct = [] {
      const char* e = std::getenv("JASPER_SEARCH_SEEN_WAYS");
      return e && std::atoi(e) == 1;
    }();
    const uint32_t set_bits = a.hash_bits - 1;  // 2^hash_bits entries in 2-way sets
    const uint32_t tb2 = a.hash_bits >= 2 ? seen_tag_bits(g.n, set_bits) : 0u;
    if (!direct && tb2) {
      a.two_way = 1;
      a.tag_bits = tb2;
      a.dom_mask = (uint32_t)(((uint64_t)1 << (set_bits + tb2)) - 1u);
    } else {
      a.tag_bits = seen_tag_bits(g.n, a.hash_bits);
      a.dom_mask = a.tag_bits ? (uint32_t)(((uint64_t)1 << (a.hash_bits + a.tag_bits)) - 1u) : 0u;
    }
  }
  {
    // the graph's value range, recorded when its rows were written
    a.gint = 0;
    if (g.metric == kL2 && int_range(g)) {
      a.gint = 1;
      a.glo = g.int_lo;
      a.ghi = g.int_hi;
      a.smax = int_exact_span(g.dim);
    }
  }
  a.vecs8 = nullptr;
  a.nb8 = 0;
  a.qsh2 = 0;
  if (a.gint && g.vecs8 && g.vecs8_lo == g.int_lo && g.vecs8_cap >= g.n && byte_rows_eligible(g)) {
    a.vecs8 = (const uint4*)g.vecs8;
    a.nb8 = g.dim / 16;
    const uint32_t h = f2h_rn((float)g.int_lo - 1024.0f);  // exact (byte_rows_eligible)
    a.qsh2 = h | (h << 16);
  }
  a.seen_bits = r.seen_bits;
  a.seen_words = (uint32_t)((g.n + 31) / 32);
  a.stats = r.stats;
  const bool stats = r.stats != nullptr;
  if (stats && !r.seen_bits) throw std::invalid_argument("stats mode needs a seen bitmap");
  const size_t lds = beam_search_lds_bytes(g, r);
  const uint32_t cpl = (a.nchunks + 3) / 4;
  const dim3 grid(r.nq);
  if (a.vecs8 && !stats && g.metric == kL2 && cpl == 4) {
    launch_one<4, kL2, false, true>(a, grid, lds, stream);
    hip_check(hipGetLastError(), "launch beam_search_kernel");
    return;
  }
#define JA_LAUNCH(C)                                                                                   \
  case C: {                                                                                            \
    if (g.metric == kL2) {                                                                             \
      if (stats) launch_one<C, kL2, true>(a, grid, lds, stream);                                       \
      else launch_one<C, kL2, false>(a, grid, lds, stream);                                            \
    } else {                                                                                           \
      if (stats) launch_one<C, kIP, true>(a, grid, lds, stream);                                       \
      else launch_one<C, kIP, false>(a, grid, lds, stream);                                            \
    }                                                                                                  \
    break;                                                                                             \
  }
  switch (cpl > 8 ? 0u : cpl) {
    JA_LAUNCH(0)
    JA_LAUNCH(1)
    JA_LAUNCH(2)
    JA_LAUNCH(3)
    JA_LAUNCH(4)
    JA_LAUNCH(5)
    JA_LAUNCH(6)
    JA_LAUNCH(7)
    JA_LAUNCH(8)
    default:
      throw std::logic_error("unreachable chunks-per-lane case");
  }
#undef JA_LAUNCH
  hip_check(hipGetLastError(), "launch beam_search_kernel");
}

}  // namespace jasper_amd
