// directional_oracle.cpp -- TEST INFRASTRUCTURE ONLY.
//
// CPU restatement of the directional (estimator-driven) traversal and its
// artifacts, reference include/jasper/beam_search/graph_beam_search.cuh,
// beam_search_common.cuh, directional_beam_search.cuh, pq_beam_search.cuh,
// lsh/lsh_globals.cuh, lsh/lsh_kernels.cuh, pq/pq_kernels.cuh.
//
// Device reductions are restated as the exact trees the reference executes:
//   * block128: per-thread partials of a 128-thread block -> xor butterfly
//     (16, 8, 4, 2, 1) inside each 32-lane warp -> the 4 warp partials in
//     lanes 0..3 of warp 0 (other lanes 0) -> the same butterfly
//     (beam_search_common.cuh:133-153, pq_kernels.cuh:230-246,
//     lsh_globals.cuh:92-110);
//   * warp32: one 32-lane xor butterfly (pq_beam_search.cuh:52-57).
// fp16 arithmetic (__hsub2, __hmul2, __half operator-) is exact-then-round
// to nearest even through double.
//
// Where the reference leaves an order to hardware (float atomics, curand
// Philox sampling) this restatement fixes one: samples come from a
// splitmix64 counter generator, and sums run in sample order. These only
// feed calibration constants and codebooks, which are saved with the graph;
// search parity is checked on fixed artifacts.

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include <omp.h>

namespace {

constexpr uint32_t kInv31 = 0x7FFFFFFFu;
constexpr uint32_t kInv32 = 0xFFFFFFFFu;

inline float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
  if (exp == 0) {
    if (man == 0) bits = sign;
    else {
      int e = -1;
      do { man <<= 1; ++e; } while ((man & 0x400u) == 0);
      man &= 0x3FFu;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) bits = sign | 0x7F800000u | (man << 13);
  else bits = sign | ((exp + 112u) << 23) | (man << 13);
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// double -> binary16, round to nearest even (used for exact fp16 sums and
// products: the double holds the exact result before rounding).
inline uint16_t d2h(double x) {
  uint64_t b;
  std::memcpy(&b, &x, 8);
  const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
  const double ax = std::fabs(x);
  if (std::isnan(x)) return (uint16_t)(sign | 0x7E00u);
  if (ax >= 65520.0) return (uint16_t)(sign | 0x7C00u);  // rounds to infinity
  if (ax < std::ldexp(1.0, -25)) {
    // below half the smallest subnormal: rounds to zero, except exactly
    // half rounds to even (zero)
    return sign;
  }
  int e;
  std::frexp(ax, &e);  // ax = m * 2^e, m in [0.5, 1)
  int exp16 = e - 1;   // ax in [2^exp16, 2^(exp16+1))
  double scaled;
  uint32_t mant;
  if (exp16 < -14) {  // subnormal: units of 2^-24
    scaled = ax * std::ldexp(1.0, 24);
  } else {
    scaled = ax * std::ldexp(1.0, 10 - exp16);  // in [1024, 2048)
  }
  double fl = std::floor(scaled);
  double rem = scaled - fl;
  mant = (uint32_t)fl;
  if (rem > 0.5 || (rem == 0.5 && (mant & 1u))) mant += 1;
  if (exp16 < -14) {
    // mant is the subnormal significand (may carry into the first normal)
    return (uint16_t)(sign | mant);
  }
  if (mant == 2048) {  // carry into the next binade
    mant = 1024;
    exp16 += 1;
    if (exp16 > 15) return (uint16_t)(sign | 0x7C00u);
  }
  return (uint16_t)(sign | ((uint32_t)(exp16 + 15) << 10) | (mant - 1024));
}

inline uint16_t hsub(uint16_t a, uint16_t b) { return d2h((double)h2f(a) - (double)h2f(b)); }
inline uint16_t hmul(uint16_t a, uint16_t b) { return d2h((double)h2f(a) * (double)h2f(b)); }

inline uint16_t f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
inline float bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// 32-lane xor butterfly, result of lane 0.
float warp32(const float* v_in) {
  float v[32], nv[32];
  std::memcpy(v, v_in, sizeof(v));
  for (int d = 16; d > 0; d >>= 1) {
    for (int l = 0; l < 32; ++l) nv[l] = v[l] + v[l ^ d];
    std::memcpy(v, nv, sizeof(v));
  }
  return v[0];
}

// 128-thread block reduction tree (see header).
float block128(const float* p) {
  float w[32] = {0};
  for (int wi = 0; wi < 4; ++wi) w[wi] = warp32(p + 32 * wi);
  return warp32(w);
}

// compute_qu_diff_and_exact, beam_search_common.cuh:87-154 (BLOCK_SIZE 128).
// L2: returns sum of f0^2 + f1^2 over fp16 dh = q - u (stored to diff);
// IP: returns sum of fp16 products q*u.
float visit_exact(const uint16_t* q, const uint16_t* u, int dp, bool l2, uint16_t* diff) {
  float part[128] = {0};
  const int n4 = dp / 8;
  for (int t = 0; t < 128; ++t) {
    float local = 0.0f;
    for (int i = t; i < n4; i += 128) {
      for (int j = 0; j < 4; ++j) {
        const int e0 = i * 8 + 2 * j, e1 = e0 + 1;
        if (l2) {
          const uint16_t d0 = hsub(q[e0], u[e0]), d1 = hsub(q[e1], u[e1]);
          if (diff) { diff[e0] = d0; diff[e1] = d1; }
          const float f0 = h2f(d0), f1 = h2f(d1);
          local = local + (f0 * f0 + f1 * f1);  // both squares exact in fp32
        } else {
          const uint16_t p0 = hmul(q[e0], u[e0]), p1 = hmul(q[e1], u[e1]);
          local = local + (h2f(p0) + h2f(p1));
        }
      }
    }
    part[t] = local;
  }
  return block128(part);
}

// per-vector ||x||^2, pq_compute_vector_norms (pq_kernels.cuh:218-247);
// also the query's ||q||^2 in pq_estimator (pq_beam_search.cuh:151-175).
float norm_sq(const uint16_t* x, int dp) {
  float part[128] = {0};
  for (int t = 0; t < 128; ++t) {
    float local = 0.0f;
    for (int i = t; i < dp; i += 128) {
      const float v = h2f(x[i]);
      local = std::fmaf(v, v, local);
    }
    part[t] = local;
  }
  return block128(part);
}

struct DEntry {
  uint32_t id;
  float dist;
  bool visited;
};

inline bool pair_less(const DEntry& a, const DEntry& b) {
  return (a.dist < b.dist) || (a.dist == b.dist && a.id < b.id);
}

struct DGraph {
  const uint16_t* vecs;
  int64_t n;
  int dp;
  const uint32_t* edges;
  const uint8_t* counts;
  int R;
  const uint32_t* deleted;
  int metric;  // 0 L2, 1 IP
};

struct Lsh {
  int K;
  int pbytes;            // 1 or 2
  const float* c;        // [K]
  float norm_denom;
  const uint8_t* rows;   // [n, row_bytes]: packed[R*K] (pbytes each) then bf16 mag[R]
  size_t row_bytes;
};

struct Pq {
  int M;
  int dsub;
  const float* centroids;  // [M*256*dsub]
  const uint8_t* codes;    // [n, M*R] subspace-major
  const float* norms;      // [n]
};

// RaBitQ one-bit codes of the stored rows, as rabitq_quantize<1> writes them
// (rabitq/layout.cuh:43-143): per vertex code bytes (bit i = [r_i >= 0],
// LSB-first, rounded up to 4 bytes) then f_add and f_rescale (fp32), taken
// against the centroid c (the codes' residuals are r = x - c).
struct Rq {
  int dim;
  uint32_t code_bytes;
  const uint8_t* nodes;    // [n, code_bytes + 8]
  const float* centroid;   // [dim]
};

// The RaBitQ estimator (this build's; the reference stops at the quantizer:
// rabitq/distance.cuh:1-10 is only the metric enum and RabitqQueryFactor,
// layout.cuh:146-150, is unused). It is the published one-bit estimator
// (Gao and Long, SIGMOD 2024) in the factor form the quantizer's f_add and
// f_rescale encode:
//   est = f_add + g_add + f_rescale * <b - 1/2, q'>
// with b the code bits and q' the query row, g_add = ||q' - c||^2 (L2) or
// -1 - <c, q'> (IP: the estimate is then of -<x, q'>, the IP distance).
// <b - 1/2, q'> uses the query quantized to 4 bits: lo = min q'_i, delta =
// (max - lo) / 15, qbar_i = rint((q'_i - lo) / delta) in [0, 15], so that
//   <b - 1/2, q'> ~ (delta / 2) (2 <b, qbar> - sum qbar) + (lo / 2) (2 |b| - dim)
// where <b, qbar> = sum_j 2^j popcount(b & plane_j) over the qbar bit planes.
struct RqQuery {
  uint32_t planes[4][8];   // plane j, dword w: bit i of dword w is bit j of qbar_(32w + i)
  int32_t sumq;
  float hd, hl, g_add;
};

// g_add's sum runs in the device's order: lane l accumulates i = l, l + 64,
// ... with an fma chain, then the 64 lane sums meet in the xor butterfly
// 32, 16, 8, 4, 2, 1 (lane 0's tree).
RqQuery rq_prepare(const uint16_t* q, const Rq& rq, bool l2) {
  RqQuery Q{};
  const int dim = rq.dim;
  float lo = h2f(q[0]), hi = lo;
  for (int i = 1; i < dim; ++i) {
    lo = std::min(lo, h2f(q[i]));
    hi = std::max(hi, h2f(q[i]));
  }
  lo = lo + 0.0f;  // one zero for -0.0 and +0.0
  hi = hi + 0.0f;
  const float delta = (hi - lo) / 15.0f;
  int32_t sumq = 0;
  for (int i = 0; i < dim; ++i) {
    uint32_t qb = 0;
    if (delta > 0.0f) {
      const float t = std::rint((h2f(q[i]) - lo) / delta);
      qb = (uint32_t)std::min(15.0f, std::max(0.0f, t));
    }
    sumq += (int32_t)qb;
    for (int j = 0; j < 4; ++j)
      if ((qb >> j) & 1u) Q.planes[j][i >> 5] |= 1u << (i & 31);
  }
  Q.sumq = sumq;
  Q.hd = 0.5f * delta;
  Q.hl = 0.5f * lo;
  float lanes[64];
  for (int l = 0; l < 64; ++l) {
    float acc = 0.0f;
    for (int i = l; i < dim; i += 64) {
      const float qi = h2f(q[i]), ci = rq.centroid[i];
      if (l2) {
        const float d = qi - ci;
        acc = std::fmaf(d, d, acc);
      } else {
        acc = std::fmaf(qi, ci, acc);
      }
    }
    lanes[l] = acc;
  }
  float half[32];
  for (int l = 0; l < 32; ++l) half[l] = lanes[l] + lanes[l + 32];
  const float s = warp32(half);
  Q.g_add = l2 ? s : -1.0f - s;
  return Q;
}

float rq_estimate(const uint8_t* node, const RqQuery& Q, const Rq& rq) {
  const uint32_t words = rq.code_bytes / 4;
  int32_t dot = 0, pc = 0;
  for (uint32_t w = 0; w < words && w < 8; ++w) {
    uint32_t c;
    std::memcpy(&c, node + 4 * w, 4);
    pc += __builtin_popcount(c);
    for (int j = 0; j < 4; ++j) dot += __builtin_popcount(c & Q.planes[j][w]) << j;
  }
  float f_add, f_rescale;
  std::memcpy(&f_add, node + rq.code_bytes, 4);
  std::memcpy(&f_rescale, node + rq.code_bytes + 4, 4);
  const float t1 = (float)(2 * dot - Q.sumq), t2 = (float)(2 * pc - rq.dim);
  const float ipq = std::fmaf(Q.hd, t1, Q.hl * t2);
  return std::fmaf(f_rescale, ipq, f_add + Q.g_add);
}

// frontier_insert_sorted, beam_search_common.cuh:156-185.
void frontier_insert(std::vector<DEntry>& F, DEntry e, uint32_t k) {
  if (k == 0) return;
  if (F.size() < k) {
    F.push_back(e);
    size_t j = F.size() - 1;
    while (j > 0 && F[j - 1].dist > e.dist) { F[j] = F[j - 1]; --j; }
    F[j] = e;
    return;
  }
  if (e.dist >= F[k - 1].dist) return;
  size_t j = k - 1;
  while (j > 0 && F[j - 1].dist > e.dist) { F[j] = F[j - 1]; --j; }
  F[j] = e;
}

// graph_beam_search_kernel, graph_beam_search.cuh:55-270, with the LSH
// (directional_beam_search.cuh:31-192) or PQ (pq_beam_search.cuh:32-201)
// estimator.
//
// unique != 0 is this build's extension (no reference counterpart): a popped
// node whose id is already in the frontier F is skipped (no visit, no
// expansion; the hop still counts against `limit`), so the results hold
// distinct ids. The reference re-visits such nodes and re-inserts them into
// F, which lets one node fill several of the k result slots.
extern "C" float jo_l2(const uint16_t* a, const uint16_t* b, int dim);  // jasper_oracle.cpp (distance.cuh)
extern "C" float jo_ip(const uint16_t* a, const uint16_t* b, int dim);

// plain_visit (the RaBitQ build search, this build's extension): a visit is
// scored with the plain search's distance (distance.cuh's lane order over
// the padded row) instead of compute_qu_diff_and_exact.
void directional_one(const DGraph& g, const Lsh* lsh, const Pq* pq, const Rq* rq, const uint16_t* q,
                     uint32_t medoid,
                     uint32_t k, uint32_t bw, uint32_t limit, uint32_t max_result, int32_t* out_ids,
                     float* out_d, uint32_t* vis_ids, float* vis_d, uint32_t* vis_count, uint64_t* stats,
                     bool unique, bool plain_visit = false) {
  const bool l2 = g.metric == 0;
  std::vector<DEntry> B, tail, merged;
  std::vector<DEntry> F;
  B.push_back({medoid & kInv31, 0.0f, false});
  std::vector<uint16_t> diff((size_t)g.dp, 0);
  float inv_norm_denom = 0.0f;
  std::vector<float> lut;
  float q_sq = 0.0f;
  if (lsh) inv_norm_denom = 1.0f / lsh->norm_denom;
  if (pq) {
    // pq_build_lut: one 32-lane warp per centroid, lanes stride the dsub coords
    lut.assign((size_t)pq->M * 256, 0.0f);
    for (int j = 0; j < pq->M; ++j) {
      for (int c = 0; c < 256; ++c) {
        const float* C = pq->centroids + ((size_t)j * 256 + c) * pq->dsub;
        const uint16_t* qj = q + (size_t)j * pq->dsub;
        float lanes[32];
        for (int l = 0; l < 32; ++l) {
          float acc = 0.0f;
          for (int t = l; t < pq->dsub; t += 32) acc = std::fmaf(h2f(qj[t]), C[t], acc);
          lanes[l] = acc;
        }
        lut[(size_t)j * 256 + c] = warp32(lanes);
      }
    }
    if (l2) q_sq = norm_sq(q, g.dp);
  }
  RqQuery rqq{};
  if (rq) rqq = rq_prepare(q, *rq, l2);
  uint32_t vc = 0, loop = 0;
  uint64_t hops = 0, visits = 0;
  while (loop <= limit) {
    loop += 1;
    size_t p = B.size();
    for (size_t i = 0; i < B.size(); ++i)
      if (!B[i].visited) { p = i; break; }
    if (p == B.size()) break;
    B[p].visited = true;
    const uint32_t u = B[p].id;
    if (unique) {
      bool in_f = false;
      for (const DEntry& f : F) in_f = in_f || f.id == u;
      if (in_f) continue;
    }
    const uint16_t* uv = g.vecs + (size_t)u * g.dp;
    float stored, exact_u = 0.0f, qu_dot = 0.0f;
    if (rq && plain_visit) {
      stored = l2 ? jo_l2(q, uv, g.dp) : jo_ip(q, uv, g.dp);
    } else if (lsh || rq) {
      exact_u = visit_exact(q, uv, g.dp, l2, l2 ? diff.data() : nullptr);
      stored = l2 ? exact_u : -exact_u;
    } else {
      qu_dot = visit_exact(q, uv, g.dp, false, nullptr);
      stored = l2 ? (q_sq - 2.0f * qu_dot) + pq->norms[u] : -qu_dot;
    }
    ++visits;
    frontier_insert(F, {u, stored, false}, k);
    if (vis_ids) { vis_ids[vc] = u; vis_d[vc] = stored; }
    vc += 1;
    if (vc == max_result) break;

    const size_t offset = B.size();
    const uint32_t deg = g.counts[u];
    for (uint32_t e = 0; e < deg; ++e) {
      const uint32_t nb = g.edges[(size_t)u * g.R + e];
      if ((int64_t)nb < g.n) B.push_back({nb & kInv31, FLT_MAX, false});
      else B.push_back({kInv31, FLT_MAX, true});
    }
    ++hops;
    for (uint32_t e = 0; e < deg; ++e) {
      DEntry& x = B[offset + e];
      if (x.id == kInv31) continue;
      if (lsh) {
        const uint8_t* row = lsh->rows + (size_t)u * lsh->row_bytes;
        const uint16_t* xv = l2 ? diff.data() : q;
        float dot_acc = 0.0f;
        for (int r = 0; r < lsh->K; ++r) {
          uint32_t word, coord;
          bool neg;
          if (lsh->pbytes == 1) {
            word = row[(size_t)e * lsh->K + r];
            neg = (word & 0x80u) != 0;
            coord = word & 0x7Fu;
          } else {
            uint16_t w16;
            std::memcpy(&w16, row + 2 * ((size_t)e * lsh->K + r), 2);
            word = w16;
            neg = (word & 0x8000u) != 0;
            coord = word & 0x7FFFu;
          }
          const float cs = neg ? -lsh->c[r] : lsh->c[r];
          dot_acc = std::fmaf(cs, h2f(xv[coord]), dot_acc);
        }
        uint16_t magb;
        std::memcpy(&magb, row + (size_t)g.R * lsh->K * lsh->pbytes + 2 * (size_t)e, 2);
        const float mag_sq = bf2f(magb);
        const float dot_est = dot_acc * inv_norm_denom;
        const float mag = std::sqrt(mag_sq);
        if (l2) x.dist = std::fmaf(-(2.0f * mag), dot_est, exact_u + mag_sq);
        else x.dist = -std::fmaf(mag, dot_est, exact_u);
      } else if (rq) {
        x.dist = rq_estimate(rq->nodes + (size_t)x.id * (rq->code_bytes + 8), rqq, *rq);
      } else {
        const uint8_t* code = pq->codes + (size_t)u * pq->M * g.R;
        float acc = qu_dot;
        for (int j = 0; j < pq->M; ++j) acc = acc + lut[(size_t)j * 256 + code[(size_t)j * g.R + e]];
        x.dist = l2 ? (q_sq - 2.0f * acc) + pq->norms[x.id] : -acc;
      }
    }
    // merge_sort_tail (device_kernels.cuh:319-408): stable sort of the tail,
    // then a merge that takes the head on ties
    if (B.size() > offset) {
      tail.assign(B.begin() + (long)offset, B.end());
      std::stable_sort(tail.begin(), tail.end(), pair_less);
      merged.clear();
      size_t ia = 0, ib = 0;
      while (ia < offset || ib < tail.size()) {
        if (ia >= offset) merged.push_back(tail[ib++]);
        else if (ib >= tail.size()) merged.push_back(B[ia++]);
        else if (!pair_less(tail[ib], B[ia])) merged.push_back(B[ia++]);
        else merged.push_back(tail[ib++]);
      }
      B.swap(merged);
    }
    // dedup_results + clip_k
    merged.clear();
    uint32_t prev = kInv31;
    for (const DEntry& e : B) {
      if (e.id != prev) merged.push_back(e);
      prev = e.id;
    }
    if (merged.size() > bw) merged.resize(bw);
    B.swap(merged);
  }
  if (vis_count) *vis_count = vc;
  if (stats) { stats[0] = hops; stats[1] = visits; }
  uint32_t out = 0;
  for (size_t i = 0; i < F.size() && out < k; ++i) {
    const uint32_t idx = F[i].id;
    if ((int64_t)idx >= g.n) continue;
    if (g.deleted && ((g.deleted[idx >> 5] >> (idx & 31u)) & 1u)) continue;
    out_ids[out] = (int32_t)idx;
    out_d[out] = F[i].dist;
    ++out;
  }
  for (; out < k; ++out) {
    out_ids[out] = (int32_t)kInv31;
    out_d[out] = FLT_MAX;
  }
}

// splitmix64 counter generator (the sampler of this restatement)
inline uint64_t splitmix(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// pq_hash, pq_kernels.cuh:19-24
inline uint64_t pq_hash(uint64_t x, uint64_t seed) {
  x += seed + 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Picks a random valid directed edge (u -> nb) for sample s, up to 8
// attempts (lsh_globals.cuh:46-67, pq_kernels.cuh:77-93).
bool sample_edge(const DGraph& g, uint64_t seed, uint64_t s, uint32_t* u_out, uint32_t* nb_out) {
  uint64_t state = splitmix(seed ^ splitmix(s + 1));
  for (int attempt = 0; attempt < 8; ++attempt) {
    state = splitmix(state);
    const uint32_t r1 = (uint32_t)(state >> 32);
    state = splitmix(state);
    const uint32_t r2 = (uint32_t)(state >> 32);
    const uint32_t qlid = (uint32_t)((uint64_t)r1 % (uint64_t)g.n);
    const uint32_t cnt = g.counts[qlid];
    if (cnt == 0) continue;
    const uint32_t e = r2 % cnt;
    const uint32_t nb = g.edges[(size_t)qlid * g.R + e];
    if (nb == kInv32) continue;
    *u_out = qlid;
    *nb_out = nb;
    return true;
  }
  return false;
}

}  // namespace

extern "C" {

uint16_t jo_d2h(double x) { return d2h(x); }
uint64_t jo_pq_hash(uint64_t x, uint64_t seed) { return pq_hash(x, seed); }
uint64_t jo_splitmix(uint64_t x) { return splitmix(x); }
int jo_sample_edge(const uint32_t* edges, const uint8_t* counts, int64_t n, int R, uint64_t seed, uint64_t s,
                   uint32_t* u, uint32_t* nb) {
  DGraph g{nullptr, n, 0, edges, counts, R, nullptr, 0};
  return sample_edge(g, seed, s, u, nb) ? 1 : 0;
}
void jo_frontier_insert_seq(const float* d, const uint32_t* ids, int m, int k, float* out_d, uint32_t* out_ids,
                            int* out_count) {
  std::vector<DEntry> F;
  for (int i = 0; i < m; ++i) frontier_insert(F, {ids[i], d[i], false}, (uint32_t)k);
  for (size_t i = 0; i < F.size(); ++i) { out_d[i] = F[i].dist; out_ids[i] = F[i].id; }
  *out_count = (int)F.size();
}
// The RaBitQ build search of one row (rabitq_build_search): directional
// traversal from the medoid with k = 0, visits scored by the plain distance;
// writes the visits (ids, distances) and returns their count.
int jo_rq_visit(const uint16_t* vecs, int64_t n, int dp, const uint32_t* edges, const uint8_t* counts, int R,
                int metric, int rq_dim, const uint8_t* rq_nodes, const float* rq_centroid, const uint16_t* q,
                uint32_t medoid, int bw, int limit, int max_result, uint32_t* vis_ids, float* vis_d) {
  DGraph g{vecs, n, dp, edges, counts, R, nullptr, metric};
  Rq rq{rq_dim, (((uint32_t)rq_dim + 7u) / 8u + 3u) / 4u * 4u, rq_nodes, rq_centroid};
  uint32_t vc = 0;
  directional_one(g, nullptr, nullptr, &rq, q, medoid, 0, (uint32_t)bw, (uint32_t)limit, (uint32_t)max_result,
                  nullptr, nullptr, vis_ids, vis_d, &vc, nullptr, false, true);
  return (int)vc;
}

// RaBitQ estimates of every node for every query row (test access to the
// estimator): out[nq, n]; also each query's prepared factors when asked
// (q_sumq [nq], q_hd_hl_g [nq, 3], q_planes [nq, 4, 8]).
void jo_rq_estimates(const uint8_t* nodes, int64_t n, int dim, const float* centroid, int metric,
                     const uint16_t* queries, int64_t nq, int dp, float* out, int32_t* q_sumq, float* q_hd_hl_g,
                     uint32_t* q_planes) {
  Rq rq{dim, (((uint32_t)dim + 7u) / 8u + 3u) / 4u * 4u, nodes, centroid};
  for (int64_t i = 0; i < nq; ++i) {
    const RqQuery Q = rq_prepare(queries + (size_t)i * dp, rq, metric == 0);
    if (q_sumq) q_sumq[i] = Q.sumq;
    if (q_hd_hl_g) { q_hd_hl_g[3 * i] = Q.hd; q_hd_hl_g[3 * i + 1] = Q.hl; q_hd_hl_g[3 * i + 2] = Q.g_add; }
    if (q_planes) std::memcpy(q_planes + (size_t)i * 32, Q.planes, sizeof(Q.planes));
    for (int64_t v = 0; v < n; ++v) out[(size_t)i * n + v] = rq_estimate(nodes + (size_t)v * (rq.code_bytes + 8), Q, rq);
  }
}

uint16_t jo_hsub(uint16_t a, uint16_t b) { return hsub(a, b); }
uint16_t jo_hmul(uint16_t a, uint16_t b) { return hmul(a, b); }

float jo_visit_exact(const uint16_t* q, const uint16_t* u, int dp, int l2, uint16_t* diff) {
  return visit_exact(q, u, dp, l2 != 0, diff);
}

void jo_vector_norms(const uint16_t* vecs, int64_t n, int dp, float* out, int nthreads) {
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = norm_sq(vecs + (size_t)i * dp, dp);
}

// Batched directional search. mode 0 = LSH, 1 = PQ, 2 = RaBitQ.
int jo_directional_search(int mode, const uint16_t* vecs, int64_t n, int dp, const uint32_t* edges,
                          const uint8_t* counts, int R, const uint32_t* deleted, int metric,
                          // LSH
                          int K, int pbytes, const float* c_per_rank, float norm_denom, const uint8_t* lsh_rows,
                          // PQ
                          int M, int dsub, const float* centroids, const uint8_t* codes, const float* norms,
                          // RaBitQ
                          int rq_dim, const uint8_t* rq_nodes, const float* rq_centroid,
                          const uint16_t* queries, int64_t nq, uint32_t medoid, int k, int bw, int limit,
                          int max_result, int32_t* out_ids, float* out_d, uint32_t* vis_ids, float* vis_d,
                          uint32_t* vis_counts, uint64_t* stats, int unique, int nthreads) {
  DGraph g{vecs, n, dp, edges, counts, R, deleted, metric};
  Lsh lsh{K, pbytes, c_per_rank, norm_denom, lsh_rows, (size_t)R * K * pbytes + 2 * (size_t)R};
  Pq pq{M, dsub, centroids, codes, norms};
  Rq rq{rq_dim, rq_dim > 0 ? (((uint32_t)rq_dim + 7u) / 8u + 3u) / 4u * 4u : 0u, rq_nodes, rq_centroid};
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 2)
  for (int64_t i = 0; i < nq; ++i) {
    directional_one(g, mode == 0 ? &lsh : nullptr, mode == 1 ? &pq : nullptr, mode == 2 ? &rq : nullptr,
                    queries + (size_t)i * dp, medoid,
                    (uint32_t)k, (uint32_t)bw, (uint32_t)limit, (uint32_t)max_result, out_ids + i * k,
                    out_d + i * k, vis_ids ? vis_ids + i * max_result : nullptr,
                    vis_d ? vis_d + i * max_result : nullptr, vis_counts ? vis_counts + i : nullptr,
                    stats ? stats + i * 2 : nullptr, unique != 0);
  }
  return 0;
}

// populate_lsh, lsh/lsh_kernels.cuh:9-132, for every vertex and edge slot
// e < count (the reference walks all R slots; slots past the count read
// unspecified neighbour ids there and are left zero here). rows:
// [n, R*K*pbytes + 2R].
void jo_populate_lsh(const uint16_t* vecs, int64_t n, int dp, const uint32_t* edges, const uint8_t* counts, int R,
                     int K, int pbytes, uint8_t* rows, int nthreads) {
  const size_t row_bytes = (size_t)R * K * pbytes + 2 * (size_t)R;
  const uint32_t coord_bits = pbytes * 8 - 1;
  const uint32_t coord_mask = (1u << coord_bits) - 1u;
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
  {
    std::vector<uint32_t> keys((size_t)dp);
    std::vector<float> part(128);
#pragma omp for schedule(dynamic, 64)
    for (int64_t u = 0; u < n; ++u) {
      uint8_t* row = rows + (size_t)u * row_bytes;
      std::memset(row, 0, row_bytes);
      const uint16_t* uv = vecs + (size_t)u * dp;
      for (uint32_t e = 0; e < counts[u]; ++e) {
        const uint32_t nb = edges[(size_t)u * R + e];
        const uint16_t* nv = vecs + (size_t)nb * dp;
        std::fill(part.begin(), part.end(), 0.0f);
        for (int t = 0; t < 128; ++t) {
          float local = 0.0f;
          for (int i = t; i < dp; i += 128) {
            const uint16_t d = hsub(nv[i], uv[i]);
            keys[(size_t)i] = ((uint32_t)(d & 0x7FFFu) << (coord_bits + 1)) | ((uint32_t)(d >> 15) << coord_bits) |
                              ((uint32_t)i & coord_mask);
            const float f = h2f(d);
            local = std::fmaf(f, f, local);
          }
          part[(size_t)t] = local;
        }
        const float mag_sq = block128(part.data());
        for (int r = 0; r < K; ++r) {
          uint32_t best = 0;
          for (int i = 0; i < dp; ++i) best = std::max(best, keys[(size_t)i]);
          const uint32_t word = best & ((1u << (coord_bits + 1)) - 1u);
          if (pbytes == 1) row[(size_t)e * K + r] = (uint8_t)word;
          else {
            const uint16_t w16 = (uint16_t)word;
            std::memcpy(row + 2 * ((size_t)e * K + r), &w16, 2);
          }
          keys[best & coord_mask] = 0;
        }
        const uint16_t mb = f2bf(mag_sq);
        std::memcpy(row + (size_t)R * K * pbytes + 2 * (size_t)e, &mb, 2);
      }
    }
  }
}

// LSH calibration, lsh/lsh_globals.cuh:17-178, with this restatement's
// sampler and sample-order sums. Returns the number of valid samples.
int64_t jo_lsh_globals(const uint16_t* vecs, int64_t n, int dp, const uint32_t* edges, const uint8_t* counts, int R,
                       int K, int64_t n_samples, uint64_t seed, float* c_out, float* norm_denom_out) {
  DGraph g{vecs, n, dp, edges, counts, R, nullptr, 0};
  std::vector<float> contrib((size_t)n_samples * K, 0.0f);
  std::vector<uint8_t> valid((size_t)n_samples, 0);
#pragma omp parallel
  {
    std::vector<uint32_t> keys((size_t)dp);
    std::vector<float> part(128);
#pragma omp for schedule(dynamic, 64)
    for (int64_t s = 0; s < n_samples; ++s) {
      uint32_t u, nb;
      if (!sample_edge(g, seed, (uint64_t)s, &u, &nb)) continue;
      const uint16_t* uv = vecs + (size_t)u * dp;
      const uint16_t* nv = vecs + (size_t)nb * dp;
      for (int t = 0; t < 128; ++t) {
        float local = 0.0f;
        for (int i = t; i < dp; i += 128) {
          const uint16_t d = hsub(nv[i], uv[i]);
          keys[(size_t)i] = ((uint32_t)(d & 0x7FFFu) << 16) | ((uint32_t)(d >> 15) << 15) | ((uint32_t)i & 0x7FFFu);
          const float f = h2f(d);
          local = std::fmaf(f, f, local);
        }
        part[(size_t)t] = local;
      }
      const float inv_norm = 1.0f / std::sqrt(block128(part.data()) + 1e-20f);
      if (inv_norm > 1e9f) continue;
      for (int r = 0; r < K; ++r) {
        uint32_t best = 0;
        for (int i = 0; i < dp; ++i) best = std::max(best, keys[(size_t)i]);
        contrib[(size_t)s * K + r] = h2f((uint16_t)(best >> 16)) * inv_norm;
        keys[best & 0x7FFFu] = 0;
      }
      valid[(size_t)s] = 1;
    }
  }
  std::vector<float> sum((size_t)K, 0.0f);
  int64_t nv = 0;
  for (int64_t s = 0; s < n_samples; ++s) {
    if (!valid[(size_t)s]) continue;
    ++nv;
    for (int r = 0; r < K; ++r) sum[(size_t)r] += contrib[(size_t)s * K + r];
  }
  const float inv_n = 1.0f / (float)nv;
  float denom = 0.0f;
  for (int r = 0; r < K; ++r) {
    const float c = sum[(size_t)r] * inv_n;
    c_out[r] = c;
    denom = std::fmaf(c, c, denom);
  }
  *norm_denom_out = denom;
  return nv;
}

// PQ codebook training, graph.cuh:1206-1273 with pq/pq_kernels.cuh:65-212:
// residual samples (this restatement's sampler), init from pq_hash picks,
// Lloyd iterations (argmin ties -> smaller index), means summed in sample
// order, empty clusters reseeded. centroids: [M*256*dsub].
void jo_pq_train(const uint16_t* vecs, int64_t n, int dp, const uint32_t* edges, const uint8_t* counts, int R, int M,
                 int64_t n_train, int iters, uint64_t seed, float* centroids, uint16_t* train_out, int nthreads) {
  DGraph g{vecs, n, dp, edges, counts, R, nullptr, 0};
  const int dsub = dp / M;
  if (n_train < 256) n_train = 256;
  if (nthreads > 0) omp_set_num_threads(nthreads);
  std::vector<uint16_t> X((size_t)n_train * dp, 0);
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < n_train; ++p) {
    uint32_t u, nb;
    if (!sample_edge(g, seed, (uint64_t)p, &u, &nb)) continue;
    for (int i = 0; i < dp; ++i) X[(size_t)p * dp + i] = hsub(vecs[(size_t)nb * dp + i], vecs[(size_t)u * dp + i]);
  }
  if (train_out) std::memcpy(train_out, X.data(), X.size() * 2);
  const uint64_t init_seed = seed ^ 0xA5A5A5A5ull;
  for (int jc = 0; jc < M * 256; ++jc) {
    const int j = jc / 256;
    const uint64_t r = pq_hash((uint64_t)jc, init_seed) % (uint64_t)n_train;
    for (int t = 0; t < dsub; ++t) centroids[(size_t)jc * dsub + t] = h2f(X[(size_t)r * dp + (size_t)j * dsub + t]);
  }
  std::vector<uint8_t> labels((size_t)n_train * M);
  std::vector<float> sum((size_t)M * 256 * dsub);
  std::vector<uint32_t> cnt((size_t)M * 256);
  for (int it = 0; it < iters; ++it) {
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < n_train; ++p) {
      for (int j = 0; j < M; ++j) {
        float best = FLT_MAX;
        int bi = 0;
        for (int c = 0; c < 256; ++c) {
          const float* C = centroids + ((size_t)j * 256 + c) * dsub;
          float d = 0.0f;
          for (int t = 0; t < dsub; ++t) {
            const float df = h2f(X[(size_t)p * dp + (size_t)j * dsub + t]) - C[t];
            d = std::fmaf(df, df, d);
          }
          if (d < best) { best = d; bi = c; }
        }
        labels[(size_t)p * M + j] = (uint8_t)bi;
      }
    }
    std::fill(sum.begin(), sum.end(), 0.0f);
    std::fill(cnt.begin(), cnt.end(), 0u);
    for (int64_t p = 0; p < n_train; ++p) {
      for (int j = 0; j < M; ++j) {
        const size_t jc = (size_t)j * 256 + labels[(size_t)p * M + j];
        cnt[jc] += 1;
        for (int t = 0; t < dsub; ++t) sum[jc * dsub + t] += h2f(X[(size_t)p * dp + (size_t)j * dsub + t]);
      }
    }
    for (int jc = 0; jc < M * 256; ++jc) {
      const int j = jc / 256;
      if (cnt[(size_t)jc] > 0) {
        const float inv = 1.0f / (float)cnt[(size_t)jc];
        for (int t = 0; t < dsub; ++t) centroids[(size_t)jc * dsub + t] = sum[(size_t)jc * dsub + t] * inv;
      } else {
        const uint64_t r = pq_hash((uint64_t)jc ^ ((uint64_t)it * 0x9E3779B9u), init_seed) % (uint64_t)n_train;
        for (int t = 0; t < dsub; ++t)
          centroids[(size_t)jc * dsub + t] = h2f(X[(size_t)r * dp + (size_t)j * dsub + t]);
      }
    }
  }
}

// pq_populate, pq_kernels.cuh:249-295: code of every edge e < count.
// codes: [n, M*R], subspace-major (code[j*R + e]).
void jo_pq_encode(const uint16_t* vecs, int64_t n, int dp, const uint32_t* edges, const uint8_t* counts, int R, int M,
                  const float* centroids, uint8_t* codes, int nthreads) {
  const int dsub = dp / M;
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
  {
    std::vector<float> res((size_t)dp);
#pragma omp for schedule(dynamic, 64)
    for (int64_t u = 0; u < n; ++u) {
      uint8_t* code = codes + (size_t)u * M * R;
      std::memset(code, 0, (size_t)M * R);
      for (uint32_t e = 0; e < counts[u]; ++e) {
        const uint32_t nb = edges[(size_t)u * R + e];
        for (int i = 0; i < dp; ++i) res[(size_t)i] = h2f(hsub(vecs[(size_t)nb * dp + i], vecs[(size_t)u * dp + i]));
        for (int j = 0; j < M; ++j) {
          float best = FLT_MAX;
          int bi = 0;
          for (int c = 0; c < 256; ++c) {
            const float* C = centroids + ((size_t)j * 256 + c) * dsub;
            float d = 0.0f;
            for (int t = 0; t < dsub; ++t) {
              const float df = res[(size_t)j * dsub + t] - C[t];
              d = std::fmaf(df, df, d);
            }
            if (d < best) { best = d; bi = c; }
          }
          code[(size_t)j * R + e] = (uint8_t)bi;
        }
      }
    }
  }
}

// Prerotation reference: rows x' = P^T x with P column-major (fp16 entries),
// fp32 accumulation in k order, fp16 output (construct.cuh:1077-1089). The
// device GEMM's accumulation order differs, so parity is a tolerance.
void jo_rotate_rows(const uint16_t* x, int64_t n, int dim, int dp, const uint16_t* P16, uint16_t* out, int nthreads) {
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n; ++r) {
    for (int i = 0; i < dp; ++i) {
      if (i >= dim) { out[(size_t)r * dp + i] = 0; continue; }
      float acc = 0.0f;
      for (int k = 0; k < dim; ++k) acc = std::fmaf(h2f(P16[(size_t)k + (size_t)i * dim]), h2f(x[(size_t)r * dp + k]), acc);
      out[(size_t)r * dp + i] = d2h((double)acc);
    }
  }
}

}  // extern "C"
