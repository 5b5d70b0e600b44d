// One AR step of the reference chain for one row, decided in one pass over
// the row (k_rows_step).
//
// The chain is the reference's (text2semantic.cpp:142-166, sampling.cpp:14-76):
// penalty -> greedy ? argmax : temperature -> top_k -> top_p -> draw. Thread t of
// the step workgroup owns the ids [t*P, t*P + P) (P odd) and keeps their values in
// registers (the row is staged in LDS with coalesced 16-byte loads). After the
// row maximum m:
//
//  * masses exp(t), t = fl(z - m), are first taken in fp32 (mass32, with an
//    error bound per term); every value falls in a bucket of (m - z) (four
//    buckets per unit, the last one unbounded), and one histogram pass (per-wave
//    counters in LDS, masses in 2^-32 fixed point) locates the bucket of the k-th largest
//    value (top_k) or the nucleus boundary (top_p: a window of +-1e-3 relative
//    around the kept mass p * S, far wider than the fp32 errors);
//  * only the entries of the boundary buckets (every bucket up to the k-th
//    value for top_k) are sorted, by (value desc, id asc): up to 64 by a
//    bitonic network on lane shuffles, up to 256 by rank counting, more by a
//    bitonic network across waves, and their masses
//    are the reference's exp((double)t) (sampling.cpp:55);
//  * the cut is taken on the sorted entries with sums formed in parallel, each
//    decision with the margin rel_eps(V) * S plus the fp32 error bounds; a
//    decision inside it is taken again with every mass in double;
//  * the kept set is then every id whose key (value, then lower id first) is
//    at or above the last kept key; the draw is one workgroup scan of the
//    kept fp32 masses in id order (thread order) and a walk of the one thread
//    whose range holds r = u * K, accepted when r is farther than the error
//    bounds from both ends of the chosen id's interval. Otherwise that
//    thread's wave recomputes the whole draw in double from the row
//    (text2semantic.cpp:150-165; sequentially when even that is too close).
//
// Rows the one pass cannot settle (an all -inf row or one below the draw's
// -1e30 floor, p <= 0, a boundary of more than 1024 entries or in the
// unbounded bucket, a cut inside the margin even in double, subnormal kept
// masses) return false before the RNG or any output changes; the kernel then
// runs the multi-pass chain (run_chain) on the row staged in LDS.

#pragma once

#include "c4s_chain.hpp"

namespace c4s {
namespace {

constexpr int kNB = 256;                 // buckets of (m - z) * kBucketScale; the last is unbounded
constexpr float kBucketScale = 4.0f;
// Threads of the workgroup that owns a row in the one-pass step.
constexpr int kStepThreads = 512;
constexpr int kStepWaves = kStepThreads / kWave;
static_assert(kStepThreads >= kNB && kStepThreads <= NT, "one bucket per thread in the merge");
constexpr int kSortCap = kStepThreads;   // boundary entries one sort handles (one per thread)
// Work area of the one-pass step (aliases the mass cache of the fallback
// chain): per-wave bucket counters and masses (64-bit fixed point, 2^-31
// units: integer LDS atomics), two sort exchange buffers, the boundary
// entries, then the fp32 mass of every id (top_p and p = 1 rows).
constexpr size_t kHistBytes = (size_t)kStepWaves * kNB * 4;
// top_p rows count entries in the same 64-bit atomic as their masses: a mass
// is at most 2^31 units and a wave's bucket sum stays below 2^44 (at most
// 64 x 65 entries), so bits 48.. hold the count.
constexpr unsigned long long kHistOne = 1ull << 48;
constexpr size_t kStepWorkBytes = 3 * kHistBytes + 3 * (size_t)kSortCap * 8;

__host__ __device__ __forceinline__ size_t step_work_bytes(int V) {
  const size_t e = 8 * (size_t)vpad(V), o = kStepWorkBytes + 4 * (size_t)vpad(V);
  return e > o ? e : o;
}

using StepScratch = ScratchT<kStepWaves>;

// Coalesced fetch of an f32 row (V <= kLdsVocabMax) by the step workgroup into
// registers, then into LDS (the layout of fetch_row / store_row).
constexpr int kStepQuads = (kLdsVocabMax / 4 + kStepThreads - 1) / kStepThreads;
struct StepFetch {
  float4 body[kStepQuads];
  float edge;
};
__device__ __forceinline__ void step_fetch(const float* p, int V, StepFetch& f) {
  const RowShape r = row_shape(p, V);
  const float4* p4 = reinterpret_cast<const float4*>(p + r.head);
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < kStepQuads; ++j) {
    const int q = t + kStepThreads * j;
    f.body[j] = (q < r.nq) ? p4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  f.edge = (t < r.head) ? p[t] : ((t < r.head + r.tail) ? p[r.head + 4 * r.nq + (t - r.head)] : 0.f);
}
__device__ __forceinline__ float* step_store(const float* p, int V, const StepFetch& f, float* buf) {
  const RowShape r = row_shape(p, V);
  float* val = buf + ((4 - r.head) & 3);
  const int t = threadIdx.x;
  float4* body = reinterpret_cast<float4*>(val + r.head);
#pragma unroll
  for (int j = 0; j < kStepQuads; ++j) {
    const int q = t + kStepThreads * j;
    if (q < r.nq) body[q] = f.body[j];
  }
  if (t < r.head) val[t] = f.edge;
  else if (t < r.head + r.tail) val[r.head + 4 * r.nq + (t - r.head)] = f.edge;
  return val;
}

struct StepSh {
  float wmax[NW];
  // per-wave partials of the workgroup scans; each set is written again only
  // after a barrier that follows every read of its previous contents
  double wa[NW], wb[NW], wc[NW], wd[NW], we[NW], wf[NW];
  uint32_t wu[NW], wv[NW], ww[NW];
  int bsel[3];       // first boundary bucket, last boundary bucket, entries above the first
  int sub[2];        // the same in the refined histogram over the boundary buckets
  float wmin[NW];    // per-wave minimum (the boundary's tie test)
  uint32_t thru;     // entries up to and including the last boundary bucket
  double mab;        // mass of the entries above the first boundary bucket
  double mabx;       // mass of the entries above X (the boundary (sub-)buckets), from the histogram
  uint32_t nabx;     // their count
  uint32_t nx;       // boundary entries (compaction counter)
  float zx;          // the largest value among them (after their sort)
  uint64_t kthr;     // kept iff key64 >= kthr
  int verdict;       // 1 decided, 2 decide again with every mass in double, 0 multi-pass chain
};

constexpr float kStepLog2e = 1.44269502162933349609375f;   // fp32(log2 e)
constexpr float kStepLog2eLo = 1.925963033500011e-8f;       // log2 e - kStepLog2e
constexpr float kStepLn2 = 0.693147180559945309f;

// exp(t) for a finite t <= 0 in fp32, as 2^th * 2^tl with th + tl = t log2 e
// carried in two parts. Its error against exp((double)t) is below
// mass32_err(e) (v_exp_f32 to about an ulp, the rest below 2^-24 relative;
// fp32 underflow below 2^-126 absolute).
__device__ __forceinline__ float mass32(float t) {
  const float th = t * kStepLog2e;
  const float tl = fmaf(t, kStepLog2e, -th) + t * kStepLog2eLo;
  const float e = __builtin_amdgcn_exp2f(th);
  return fmaf(e * kStepLn2, tl, e);
}
__device__ __forceinline__ double mass32_err(float e) { return (double)e * 0x1p-20 + 0x1p-125; }

__device__ __forceinline__ int bucket_of(float z, float m) {
  const float q = (m - z) * kBucketScale;   // monotone in z; +inf for z = -inf
  return q < (float)(kNB - 1) ? (int)q : kNB - 1;
}
// out[j] = row[lo + j] for j < n and row[V - 1] past it: every read in bounds
// and issued together. A thread whose ids all lie in the row (all but the last
// few) reads at immediate offsets from one address instead of clamping each
// index.
template <int PT>
__device__ __forceinline__ void read_row(const float* row, int lo, int n, int V, float (&out)[PT]) {
  if (n == PT) {
    const float* p = row + lo;
#pragma unroll
    for (int j = 0; j < PT; ++j) out[j] = p[j];
  } else {
#pragma unroll
    for (int j = 0; j < PT; ++j) out[j] = row[min(lo + j, V - 1)];
  }
}

// The same bucket from d = fl(m - z) (= -fl(z - m): IEEE subtraction is
// symmetric in sign).
__device__ __forceinline__ int bucket_of_diff(float d) {
  const float q = d * kBucketScale;
  return q < (float)(kNB - 1) ? (int)q : kNB - 1;
}

// The refined histogram: kNB sub-buckets over buckets lo2 .. lo2 + kNB / sc2 - 1
// (an entry of those buckets; monotone in z like bucket_of).
__device__ __forceinline__ int sub_bucket_of(float z, float m, int lo2, float sc2) {
  const float v = ((m - z) * kBucketScale - (float)lo2) * sc2;
  return v < (float)(kNB - 1) ? (int)fmaxf(v, 0.0f) : kNB - 1;
}

// Which side of the boundary entries X an entry of value z lies on: -1 above
// (kept without sorting), 0 in X, 1 below (removed); monotone in z. X is the
// buckets xlo .. xhi and, when refined, within buckets lo2 .. xhi only the
// sub-buckets slo .. shi.
struct SideRule {
  float m, sc2;
  int xlo, xhi, lo2, slo, shi;
  bool refine;
  // Every test evaluated and combined by selects: per-value code without
  // branches (a branch a value costs the wave an exec-mask round trip).
  __device__ __forceinline__ int side(float z) const {
    const int b = bucket_of(z, m);
    const int sb = sub_bucket_of(z, m, lo2, sc2);
    const int in_sub = sb < slo ? -1 : (sb > shi ? 1 : 0);
    const int in_x = ((int)refine & (int)(b >= lo2)) ? in_sub : 0;
    return b < xlo ? -1 : (b > xhi ? 1 : in_x);
  }
};

// Wave 0: where the kept set's boundary falls in a histogram of kNB buckets in
// descending value order (cnt entries and mass ms each; c0 entries of mass m0
// come before bucket 0). top_k: the bucket of the k-th entry (lo == hi);
// top_p: the first bucket whose running mass reaches Blo, and the first that
// reaches Bhi. Lane l takes buckets 4l .. 4l + 3. -1 where none does.
struct Boundary {
  int lo, hi;
  uint32_t above;   // entries before bucket lo
  double mabove;    // their mass
  uint32_t thru;    // entries up to and including bucket hi
};
__device__ Boundary boundary_scan(const uint32_t* cnt, const double* ms, bool topk, uint32_t k, double Blo,
                                  double Bhi, uint32_t c0, double m0) {
  const int lane = lane_id();
  uint32_t c4[4], lc = 0;
  double m4[4], lmass = 0.0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    c4[q] = cnt[4 * lane + q];
    m4[q] = ms[4 * lane + q];
    lc += c4[q];
    lmass += m4[q];
  }
  const uint32_t ci = wave_scan_u32(lc);
  const double mi = wave_scan_f64(lmass);
  uint32_t crun = c0 + ci - lc;
  double mrun = m0 + (mi - lmass);
  int blo = -1, bhi = -1;
  uint32_t above = 0, thru = 0;
  double mab = 0.0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int b = 4 * lane + q;
    const double nx = mrun + m4[q];
    const uint32_t cx = crun + c4[q];
    if (topk) {
      if (blo < 0 && cx >= k) { blo = b; bhi = b; above = crun; thru = cx; }
    } else {
      if (blo < 0 && nx >= Blo) { blo = b; above = crun; mab = mrun; }
      if (bhi < 0 && nx >= Bhi) { bhi = b; thru = cx; }
    }
    mrun = nx;
    crun = cx;
  }
  Boundary r{-1, -1, 0u, 0.0, 0u};
  const uint64_t hl = __ballot(blo >= 0), hh = __ballot(bhi >= 0);
  if (hl) {
    const int f = __ffsll((unsigned long long)hl) - 1;
    r.lo = (int)readlane_u32((uint32_t)blo, f);
    r.above = readlane_u32(above, f);
    r.mabove = readlane_f64(mab, f);
  }
  if (hh) {
    const int f = __ffsll((unsigned long long)hh) - 1;
    r.hi = (int)readlane_u32((uint32_t)bhi, f);
    r.thru = readlane_u32(thru, f);
  }
  return r;
}

// Strict total order of the chain: value descending, then lower id first
// (the declared top_p tie order).
__device__ __forceinline__ uint64_t key64(float z, int id) {
  return ((uint64_t)fkey(z) << 32) | (uint64_t)(~(uint32_t)id);
}
__device__ __forceinline__ float key_value(uint64_t k) { return kfloat((uint32_t)(k >> 32)); }

// Workgroup scan (thread order) of a double v: exclusive and inclusive prefix
// and total, with a second double summed and a u32 scanned (exclusive prefix,
// total) over the workgroup, one barrier. The inclusive prefix of thread t is
// bitwise the exclusive prefix of thread t + 1 and the last thread's is the
// total, so the intervals (ex, in] tile (0, total].
struct Scan2 {
  double ex, in, tot, tot2;
  uint32_t utot, uex;
};
__device__ __forceinline__ Scan2 block_scan2(double v, double v2, uint32_t u, double* wa, double* wb,
                                             uint32_t* wu) {
  const int lane = lane_id(), w = wave_id();
  const double inc = wave_scan_f64(v);
  const double exc = wave_shr1_f64(inc, 0.0);
  const double s2 = wave_sum_dpp(v2);
  const uint32_t uinc = wave_scan_u32(u);
  if (lane == kWave - 1) { wa[w] = inc; wu[w] = uinc; }
  if (lane == 0) wb[w] = s2;
  __syncthreads();
  Scan2 r;
  double base = 0.0, run = 0.0, t2 = 0.0;
  uint32_t ut = 0, ubase = 0;
#pragma unroll
  for (int i = 0; i < kStepWaves; ++i) {
    if (i == w) { base = run; ubase = ut; }
    run += wa[i];
    t2 += wb[i];
    ut += wu[i];
  }
  r.ex = base + exc;
  r.in = base + inc;
  r.tot = run;
  r.tot2 = t2;
  r.utot = ut;
  r.uex = ubase + uinc - u;
  return r;
}

// Descending bitonic sort of P2 (a power of two, <= kSortCap) distinct keys,
// one per thread t < P2 (threads at or above P2 carry padding among
// themselves). Stages across waves exchange through `buf` (two halves of
// kSortCap keys, one barrier each), stages inside a wave through DPP lane
// moves (partners 1-8 lanes apart) or lane permutes (16, 32). Fully unrolled
// per P2.
template <int K, int J>
__device__ __forceinline__ uint64_t bitonic_step(uint64_t v, int t, uint64_t* buf, int& half) {
  uint64_t p;
  if constexpr (J >= kWave) {
    buf[half * kSortCap + t] = v;
    __syncthreads();
    p = buf[half * kSortCap + (t ^ J)];
    half ^= 1;
  } else {
    p = xor_lane_u64<J>(v);
  }
  const bool take_max = ((t & J) == 0) == ((t & K) == 0);
  return take_max ? (v > p ? v : p) : (v < p ? v : p);
}
template <int K, int J>
__device__ __forceinline__ uint64_t bitonic_merge(uint64_t v, int t, uint64_t* buf, int& half) {
  v = bitonic_step<K, J>(v, t, buf, half);
  if constexpr (J > 1) v = bitonic_merge<K, J / 2>(v, t, buf, half);
  return v;
}
template <int P2, int K = 2>
__device__ __forceinline__ uint64_t bitonic_sort(uint64_t v, int t, uint64_t* buf, int& half) {
  v = bitonic_merge<K, K / 2>(v, t, buf, half);
  if constexpr (K < P2) v = bitonic_sort<P2, 2 * K>(v, t, buf, half);
  return v;
}
// Wave 0 alone (P2 <= 64): no barrier.
__device__ __forceinline__ uint64_t sort_desc_wave(uint64_t v, int P2) {
  const int t = threadIdx.x;
  int half = 0;
  switch (P2) {
    case 2: return bitonic_sort<2>(v, t, nullptr, half);
    case 4: return bitonic_sort<4>(v, t, nullptr, half);
    case 8: return bitonic_sort<8>(v, t, nullptr, half);
    case 16: return bitonic_sort<16>(v, t, nullptr, half);
    case 32: return bitonic_sort<32>(v, t, nullptr, half);
    case 64: return bitonic_sort<64>(v, t, nullptr, half);
    default: return v;
  }
}
// The whole workgroup (64 < P2 <= kSortCap).
__device__ __forceinline__ uint64_t sort_desc_block(uint64_t v, int P2, uint64_t* buf) {
  static_assert(kSortCap == 512, "sort sizes up to 512");
  const int t = threadIdx.x;
  int half = 0;
  if (P2 == 128) return bitonic_sort<128>(v, t, buf, half);
  if (P2 == 256) return bitonic_sort<256>(v, t, buf, half);
  return bitonic_sort<512>(v, t, buf, half);
}

// Descending order of list[0 .. nX), nX <= E, distinct keys, in place, by rank
// counting: kStepThreads / E threads per key, each counting the keys above it
// in its share of the list (16 broadcast reads in flight a round), the shares'
// counts meeting in `part` (E * kStepThreads / E words). Returns the t-th
// largest key (0 for t >= nX). The whole workgroup enters with the list
// complete and visible; two barriers inside.
template <int E>
__device__ __forceinline__ uint64_t rank_sort_desc(uint64_t* list, int nX, uint32_t* part) {
  constexpr int G = kStepThreads / E;
  static_assert(G * E == kStepThreads && E % kWave == 0 && (E / G) % 16 == 0, "whole waves and rounds per share");
  const int t = threadIdx.x;
  // the share and the bounds are the same on every lane of a wave: scalar
  // loop control and bound tests (a vector loop costs several times as much)
  const int nXs = __builtin_amdgcn_readfirstlane(nX);
  const int i = t % E, q = __builtin_amdgcn_readfirstlane(t / E);
  const int chunk = ((nXs + G - 1) / G + 15) & ~15;   // <= E / G: every read below E
  const int j0 = q * chunk, j1 = min(nXs, j0 + chunk);
  const uint64_t mine = list[i];
  uint32_t r = 0;
  if (__builtin_amdgcn_readfirstlane(i & ~(kWave - 1)) < nXs)   // waves whose keys all lie past nX skip the count
    for (int j = j0; j < j1; j += 16) {
      uint64_t o[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) o[u] = list[j + u];   // in bounds: j + u < G * chunk
#pragma unroll
      for (int u = 0; u < 16; ++u) r += ((int)(j + u < j1) & (int)(o[u] > mine)) ? 1u : 0u;
    }
  C4S_PHASE(24);
  part[q * E + i] = r;
  __syncthreads();
  C4S_PHASE(25);
  if (t < nX) {
    uint32_t rank = 0;
#pragma unroll
    for (int g = 0; g < G; ++g) rank += part[g * E + t];
    list[rank] = mine;
  }
  __syncthreads();
  return t < nX ? list[t] : 0ull;
}

// Where one row's inputs and outputs are (the kernel's view of c4s_rows).
struct StepIO {
  const float* xf;           // f32 row or null
  const uint16_t* xb;        // bf16 row or null
  const uint32_t* bitmap;    // penalised ids: LDS bitmap (CSR history) or null
  const uint32_t* hbits;     // penalised ids: the caller's history set or null
  int32_t* out_tok;          // this row's token
  uint64_t* rng;             // this row's state
  float* masked;             // row or null
  uint32_t* stats;           // 4 words or null
  uint32_t* join;            // the history set that the token joins, or null
  int stop_token;
};

// The value of id i as the chain sees it before the temperature (penalty applied).
__device__ __forceinline__ float step_value(const StepIO& io, const RowCfg& c, int i) {
  float x = io.xf ? io.xf[i] : __uint_as_float((uint32_t)io.xb[i] << 16);
  if (c.pen_on) {
    const uint32_t wd = io.bitmap ? io.bitmap[i >> 5] : io.hbits[i >> 5];
    if ((wd >> (i & 31)) & 1u) x = (x < 0) ? x * c.pen : x / c.pen;   // sampling.cpp:26
  }
  return x;
}

// The kept set of the draw, as the one pass decided it.
struct KeptRule {
  bool dense;      // every id with a positive mass (thr == 0) or every id (thr < 0)
  bool all;        // thr < 0
  uint64_t kthr;   // otherwise: key64 >= kthr
};
__device__ __forceinline__ bool kept_by(const KeptRule& kr, float z, float m, int id) {
  if (kr.dense) return kr.all || (z != neg_inf() && exp((double)(z - m)) > 0.0);
  return key64(z, id) >= kr.kthr;
}
// The same test in the one pass (dense rows whose t = fl(z - m) lies within
// [-745.25, -745] leave it, so `t > -745` decides there), and the fp32 mass.
__device__ __forceinline__ bool kept_in(const KeptRule& kr, float z, float m, int id) {
  return kr.dense ? (kr.all || (z != neg_inf() && z - m > -745.0f)) : key64(z, id) >= kr.kthr;
}
__device__ __forceinline__ float kept_mass32(const KeptRule& kr, float z, float m, int id, bool& kept) {
  kept = kept_in(kr, z, m, id);
  return (kept && z != neg_inf()) ? mass32(z - m) : 0.0f;
}

// The draw recomputed in double by one wave from the row (text2semantic.cpp:
// 150-165): the kept masses exp((double)fl(z - m)) summed in parallel and the
// first id whose prefix reaches r = u * sum taken when both ends of its
// interval are farther than rel_eps from r; otherwise the reference's
// sequential sums in id order.
__device__ __noinline__ int draw_replay(const StepIO& io, const RowCfg& c, const KeptRule kr, float m, double u) {
  const int lane = lane_id();
  const int V = c.V;
  auto mass_at = [&](int i) -> double {
    if (i >= V) return 0.0;
    const float y = step_value(io, c, i);
    const float z = c.temp_on ? y / c.temp : y;
    return (z != neg_inf() && kept_by(kr, z, m, i)) ? exp((double)(z - m)) : 0.0;
  };
  double tot = 0.0;
  for (int base = 0; base < V; base += kWave) tot += wave_sum_dpp(mass_at(base + lane));
  const double r = u * tot;
  const double eps = rel_eps(V);
  if (!(r > 0.0)) return 0;
  double carry = 0.0;
  for (int base = 0; base < V; base += kWave) {
    const double e = mass_at(base + lane);
    const double inc = wave_scan_f64(e) + carry;
    const uint64_t hit = __ballot(e > 0.0 && inc >= r);
    if (hit) {
      const int f = __ffsll((unsigned long long)hit) - 1;
      const double af = readlane_f64(inc, f), pf = af - readlane_f64(e, f);
      if ((af - r > eps * af) && (r - pf > eps * r)) return base + f;
      break;
    }
    carry = readlane_f64(inc, kWave - 1);
  }
  // sequential, in id order, as the reference sums
  double total = 0.0;
  for (int base = 0; base < V; base += kWave) {
    const double e = mass_at(base + lane);
    total = seq_sum_lanes(total, e, min(kWave, V - base));
  }
  const double rr = u * total;
  if (!(rr > 0.0)) return 0;
  double acc = 0.0;
  for (int base = 0; base < V; base += kWave) {
    const double e = mass_at(base + lane);
    const int q = seq_find_lanes(acc, e, min(kWave, V - base), rr);
    if (q >= 0) return base + q;
  }
  return V - 1;
}

// The nucleus / top-k cut on the sorted boundary entries, by the whole
// workgroup (kBlock, more than 64 entries) or by wave 0. v: this thread's
// sorted entry (valid below nX). S, errS: the sum of all masses and its error
// bound (rows without top-k); Ma, errMa: the mass above the boundary buckets
// and its bound. Writes sh.kthr and sh.verdict (1; 2 when a decision falls
// inside the margin while fp32 errors remain; 4 when it does with none, on a
// row without top-k; 0).
template <bool kBlock>
__device__ __noinline__ void decide_cut(const RowCfg& c, uint64_t v, int nX, float m, double thr, double S, double errS,
                           double Ma, double errMa, uint32_t n_above, const uint64_t* list, StepSh& sh) {
  const int t = threadIdx.x;
  const bool topk = c.topk_on;
  const bool valid = t < nX;
  const float ninf = neg_inf();
  const float zt = valid ? key_value(v) : ninf;
  // top_k (sampling.cpp:30-40): survivors are the entries >= the k-th largest value
  uint32_t kkey = 0;
  if (topk) kkey = kBlock ? (uint32_t)(list[c.k - 1] >> 32) : readlane_u32((uint32_t)(v >> 32), c.k - 1);
  const bool surv = valid && (!topk || (uint32_t)(v >> 32) >= kkey);
  const double et = (surv && zt != ninf) ? exp((double)(zt - m)) : 0.0;
  double ex, tot;
  if (kBlock) {
    const Scan2 sc = block_scan2(et, 0.0, 0u, sh.we, sh.wf, sh.wv);
    ex = sc.ex;
    tot = sc.tot;
  } else {
    const double inc = wave_scan_f64(et);
    ex = wave_shr1_f64(inc, 0.0);
    tot = readlane_f64(inc, kWave - 1);
  }
  // entry removed iff the mass at or below it in ascending order,
  // M = S - (mass above it), is <= (1 - p) S (sampling.cpp:60-65)
  const double Sx = topk ? tot : S;   // after top_k only the survivors carry mass
  const double err = topk ? 0.0 : 2.0 * errS + errMa;
  const double above = topk ? ex : Ma + ex;
  const double A = thr * Sx;
  const double M = Sx - above;
  bool kept, unsure;
  if (thr <= 0.0) {   // p >= 1 (top_k rows only here): only zero-mass positions can go
    kept = surv && (thr < 0.0 || et > 0.0);
    unsure = false;
  } else {
    kept = surv && M > A;
    unsure = surv && !(fabs(M - A) > rel_eps(c.V) * Sx + err);
  }
  uint32_t nk, ns, nuns;
  if (kBlock) {
    const Scan2 cn = block_scan2(0.0, 0.0, (kept ? 1u : 0u) | (surv ? 1u << 11 : 0u) | (unsure ? 1u << 22 : 0u),
                                 sh.wc, sh.wd, sh.ww);
    nk = cn.utot & 2047u;
    ns = (cn.utot >> 11) & 2047u;
    nuns = cn.utot >> 22;
  } else {
    nk = (uint32_t)__popcll(__ballot(kept));
    ns = (uint32_t)__popcll(__ballot(surv));
    nuns = (uint32_t)__popcll(__ballot(unsure));
  }
  // min_tokens_to_keep (sampling.cpp:67-68): the top min_keep positions stay
  const uint32_t mk = (uint32_t)max(0, c.min_keep);
  int verdict = 1;
  if (nuns) {
    verdict = err > 0.0 ? 2 : (topk ? 0 : 4);
  } else if (topk) {
    if (nk < mk) nk = min(mk, ns);
  } else if (n_above + nk < mk) {
    if (mk > n_above + (uint32_t)nX) verdict = 0;
    else nk = mk - n_above;
  }
  if (t == 0) sh.verdict = verdict;
  // the last kept entry; with none kept here, everything above the boundary buckets
  if (verdict == 1 && t == (nk > 0 ? (int)nk - 1 : 0)) sh.kthr = nk > 0 ? v : v + 1ull;
}

}  // namespace
}  // namespace c4s

namespace c4s {
namespace {

// Stages a bf16 row in LDS as fp32 with 16-byte loads (eight ids each): the
// 0-7 ids before the first 16-byte boundary and the 0-7 after the last one go
// one per thread. Returns where the row starts (buf + 0..3, the body 16-byte
// aligned). V <= kLdsVocabMax.
constexpr int kStepOcts = (kLdsVocabMax / 8 + kStepThreads - 1) / kStepThreads;
__device__ __forceinline__ float* stage_row_bf16(const uint16_t* p, int V, float* buf) {
  const int head = min(V, (int)(((16u - ((uint32_t)(uintptr_t)p & 15u)) & 15u) >> 1));
  const int nq = (V - head) >> 3;
  const int tail = V - head - 8 * nq;
  float* val = buf + ((4 - (head & 3)) & 3);
  const uint4* p8 = reinterpret_cast<const uint4*>(p + head);
  const int t = threadIdx.x;
  uint4 q[kStepOcts];
#pragma unroll
  for (int j = 0; j < kStepOcts; ++j) {
    const int i = t + kStepThreads * j;
    q[j] = (i < nq) ? p8[i] : make_uint4(0u, 0u, 0u, 0u);
  }
  const int eidx = (t < head) ? t : ((t < head + tail) ? head + 8 * nq + (t - head) : -1);
  const uint16_t ev = (eidx >= 0) ? p[eidx] : (uint16_t)0;
  auto lo16 = [](uint32_t x) { return __uint_as_float(x << 16); };
  auto hi16 = [](uint32_t x) { return __uint_as_float(x & 0xFFFF0000u); };
#pragma unroll
  for (int j = 0; j < kStepOcts; ++j) {
    const int i = t + kStepThreads * j;
    if (i < nq) {
      float4* d = reinterpret_cast<float4*>(val + head + 8 * i);
      d[0] = make_float4(lo16(q[j].x), hi16(q[j].x), lo16(q[j].y), hi16(q[j].y));
      d[1] = make_float4(lo16(q[j].z), hi16(q[j].z), lo16(q[j].w), hi16(q[j].w));
    }
  }
  if (eidx >= 0) val[eidx] = __uint_as_float((uint32_t)ev << 16);
  return val;
}

}  // namespace
}  // namespace c4s
