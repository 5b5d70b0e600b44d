// Device code shared by the gfx950 sampling kernels: row configuration, element
// sources, radix selections, the exact sequential emulations, the top-k fast
// path, the processor chain, and row staging in LDS.
//
// One workgroup (1024 threads = 16 wave64) owns one row. The chain follows the
// reference order (src/t2s/text2semantic.cpp:142-166):
//   repetition penalty -> greedy ? argmax : temperature -> top_k -> top_p -> draw
// with the per-processor semantics of src/t2s/sampling.cpp:14-76 and the
// xorshift64 inverse-CDF draw of text2semantic.cpp:150-165.
//
// Exactness. Penalty, temperature and top-k are single IEEE fp32 operations or
// comparisons and are reproduced bit for bit. top_p and the draw accumulate
// double sums sequentially in the reference (ascending value order, resp. id
// order). Here those sums are formed in parallel; every decision taken from
// them (does the nucleus cut remove this position, does r <= acc hold at this
// id) is accepted only when its margin exceeds a bound on the difference
// between any sequential and any parallel evaluation (relative
// (4n+64)*2^-53 + 2^-48, which also covers a few ulp of exp(double) between
// libm implementations). Otherwise the row re-runs that step as an exact
// sequential emulation in reference order. Selections use radix passes over
// order-preserving 32-bit keys (no sort); the top_p tie order is the declared
// one: within a tie group cut by the nucleus the lower ids survive.
//
// Rows with vocab <= kLdsVocabMax are staged in LDS (values + cached double
// masses); larger rows are re-read from HBM on every pass (penalty via an LDS
// bitmap, temperature re-applied on the fly).

#pragma once

#include <limits.h>
#include <math.h>

#include "c4s_device.hpp"
#include "c4s_internal.h"

namespace c4s {
namespace {

constexpr int NT = kThreads;
constexpr int NW = NT / kWave;

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

// Workgroup scratch of the chain for NWX wavefronts (the chain functions take
// their workgroup size from it).
template <int NWX>
struct ScratchT {
  static constexpr int kWaves = NWX;
  uint32_t hcnt[256];
  double hmass[256];
  double redd[NWX];
  float redf[NWX];
  float redf2[NWX];
  float redf3[NWX];
  int redi[NWX];
  uint32_t redu[NWX];
  double wmass[NWX];
  uint32_t wcnt[NWX];
  uint32_t bu[8];
  double bd[8];
  int bi[8];
  uint32_t counter;
  uint32_t step_stats[4];
};
using Scratch = ScratchT<NW>;

// Bound on |sequential - parallel| for non-negative double sums over n terms,
// relative to the compared quantities (see file header).
__device__ __forceinline__ double rel_eps(int n) {
  return (4.0 * (double)n + 64.0) * 0x1p-53 + 0x1p-48;
}

struct RowCfg {
  int V;
  bool pen_on;
  float pen;
  bool greedy;
  bool draw;
  bool temp_on;
  float temp;
  bool topk_on;
  int k;
  bool topp_on;
  float p;
  int min_keep;
};

// The processor configuration from one row's parameter values.
__device__ __forceinline__ RowCfg make_cfg_vals(const uint32_t mode, int V, float pen, float temp, int32_t k, float p,
                                                int32_t min_keep, bool sample) {
  RowCfg c;
  c.V = V;
  c.pen = pen;
  c.temp = temp;
  c.k = k;
  c.p = p;
  c.min_keep = min_keep;
  if (!(mode & kCustom)) {
    c.pen_on = c.pen != 1.0f;                      // sampling.cpp:21
    c.greedy = !sample;                            // text2semantic.cpp:144-145
    c.draw = sample;
    c.temp_on = sample && !(c.temp == 1.0f || c.temp <= 0.0f);  // sampling.cpp:15
    c.topk_on = sample && c.k > 0 && c.k < V;      // sampling.cpp:32
    c.topp_on = sample;                            // sampling.cpp:42 has no early return
  } else {
    c.pen_on = (mode & kPenalty) && c.pen != 1.0f;
    c.greedy = (mode & kArgmax) != 0;
    c.draw = !c.greedy && (mode & kDraw) != 0;
    c.temp_on = !c.greedy && (mode & kTemperature) && !(c.temp == 1.0f || c.temp <= 0.0f);
    c.topk_on = !c.greedy && (mode & kTopK) && c.k > 0 && c.k < V;
    c.topp_on = !c.greedy && (mode & kTopP);
  }
  return c;
}

__device__ __forceinline__ RowCfg make_cfg(const uint32_t mode, int V, int row, const float* temp,
                           const int32_t* top_k, const float* top_p, const float* pen,
                           const int32_t* min_keep, const uint8_t* do_sample) {
  return make_cfg_vals(mode, V, pen ? pen[row] : 1.0f, temp ? temp[row] : 1.0f, top_k ? top_k[row] : 0,
                       top_p ? top_p[row] : 1.0f, min_keep ? min_keep[row] : 1,
                       (mode & kCustom) || (do_sample ? (do_sample[row] != 0) : true));
}

// ---- element sources ---------------------------------------------------------

// Row staged in LDS. `val` holds the penalised logits, then (after
// apply_temperature) the divided ones. `E` caches double masses by id and
// doubles as the key buffer of the exact top_p pass.
struct LdsRow {
  float* val;
  double* E;
  int V;
  uint32_t thr_key;
  bool topk_on;
  static constexpr bool kCache = true;

  __device__ float zraw(int i) const { return val[i]; }
  __device__ float z(int i) const {
    const float v = val[i];
    return (topk_on && fkey(v) < thr_key) ? neg_inf() : v;
  }
  __device__ double cached(int i) const { return E[i]; }
  __device__ void cache(int i, double e) { E[i] = e; }
  __device__ void apply_temperature(float t, int lo, int hi) {
    const double r = 1.0 / (double)t;
    for (int i = lo + lane_id(); i < hi; i += kWave) val[i] = div_rcp(val[i], r);
    __syncthreads();
  }
  __device__ uint32_t* sort_buf() const { return reinterpret_cast<uint32_t*>(E); }
  __device__ size_t sort_bytes() const { return 8 * (size_t)V; }
};

// Row staged in LDS without a mass cache (kernels whose LDS holds several rows):
// masses are recomputed per pass and the exact top_p pass sorts in a global
// key buffer.
struct LdsRowNC {
  float* val;
  int V;
  uint32_t thr_key;
  bool topk_on;
  uint32_t* sortbuf;
  uint32_t sortcap = 0;   // bytes of sortbuf (0: the keys only)
  static constexpr bool kCache = false;

  __device__ float zraw(int i) const { return val[i]; }
  __device__ float z(int i) const {
    const float v = val[i];
    return (topk_on && fkey(v) < thr_key) ? neg_inf() : v;
  }
  __device__ double cached(int) const { return 0.0; }
  __device__ void cache(int, double) {}
  __device__ void apply_temperature(float t, int lo, int hi) {
    const double r = 1.0 / (double)t;
    for (int i = lo + lane_id(); i < hi; i += kWave) val[i] = div_rcp(val[i], r);
    __syncthreads();
  }
  __device__ uint32_t* sort_buf() const { return sortbuf; }
  __device__ size_t sort_bytes() const { return sortcap; }
};

// Row re-read from HBM on every pass.
struct GlobalRow {
  const float* xf;
  const uint16_t* xb;
  int V;
  const uint32_t* bitmap;  // LDS, penalised ids
  bool pen_on;
  float pen;
  bool temp_on;
  float temp;
  uint32_t thr_key;
  bool topk_on;
  uint32_t* sortbuf;       // global workspace for the exact top_p pass
  uint32_t sortcap;        // its bytes
  static constexpr bool kCache = false;

  __device__ float y(int i) const {
    float x = xf ? xf[i] : __uint_as_float(static_cast<uint32_t>(xb[i]) << 16);
    if (pen_on && ((bitmap[i >> 5] >> (i & 31)) & 1u)) x = (x < 0) ? x * pen : x / pen;
    return x;
  }
  __device__ float zraw(int i) const {
    const float v = y(i);
    return temp_on ? v / temp : v;
  }
  __device__ float z(int i) const {
    const float v = zraw(i);
    return (topk_on && fkey(v) < thr_key) ? neg_inf() : v;
  }
  __device__ double cached(int) const { return 0.0; }
  __device__ void cache(int, double) {}
  __device__ void apply_temperature(float t, int, int) { temp_on = true; temp = t; }
  __device__ uint32_t* sort_buf() const { return sortbuf; }
  __device__ size_t sort_bytes() const { return sortcap; }
};

// Wave w owns ids [w*seg, min(V, (w+1)*seg)), visited in slices of 64.
struct Seg {
  int lo, hi;
};
template <int NWX = NW>
__device__ __forceinline__ Seg my_seg(int V) {
  const int seg = (V + NWX - 1) / NWX;
  const int lo = min(V, wave_id() * seg);
  return Seg{lo, min(V, lo + seg)};
}

// ---- count-based radix select (descending) -----------------------------------
// Key of the m-th largest element (1-based, with multiplicity) among keyfn(i)
// for i in [0, V); also the number of keys strictly greater (`gt`) and equal
// (`eq`) to it.
template <int NWX, class KeyFn>
__device__ uint32_t select_desc(KeyFn keyfn, Seg sg, ScratchT<NWX>& sh, uint32_t m, uint32_t& gt,
                                uint32_t& eq) {
  constexpr int NTX = NWX * kWave;
  uint32_t prefix = 0, mask = 0, rem = m;
  gt = 0;
  eq = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = threadIdx.x; b < 256; b += NTX) sh.hcnt[b] = 0;
    __syncthreads();
    for (int i = sg.lo + lane_id(); i < sg.hi; i += kWave) {
      const uint32_t k = keyfn(i);
      if ((k & mask) == prefix) atomicAdd(&sh.hcnt[(k >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (wave_id() == 0) {
      const int l = lane_id();
      uint32_t c[4], lc = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) { c[j] = sh.hcnt[255 - (4 * l + j)]; lc += c[j]; }
      const uint32_t incl = wave_incl_scan_u32(lc);
      uint32_t run = incl - lc;
      int hitb = -1;
      uint32_t above = 0, ceq = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (hitb < 0 && run + c[j] >= rem) { hitb = 255 - (4 * l + j); above = run; ceq = c[j]; }
        run += c[j];
      }
      const uint64_t hit = __ballot(hitb >= 0);
      const int first = __ffsll((unsigned long long)hit) - 1;
      if (l == first) { sh.bu[0] = (uint32_t)hitb; sh.bu[1] = above; sh.bu[2] = ceq; }
    }
    __syncthreads();
    const uint32_t b = sh.bu[0];
    rem -= sh.bu[1];
    gt += sh.bu[1];
    eq = sh.bu[2];
    prefix |= b << shift;
    mask |= 0xFFu << shift;
    __syncthreads();
  }
  return prefix;
}

// ---- nucleus cut from the bottom, by mass (top_p) -----------------------------
// Finds the first value group, in ascending order, whose cumulative mass exceeds
// A = (1 - p) * S. Returns false when a decision falls inside the error bound.
// On success: R = positions (ascending, all V ids) the reference removes by
// `cum <= 1 - p`, wkey/eq = the crossing group, nkeep = how many of that group
// stay (its lowest ids).
template <int NWX, class Src>
__device__ bool cut_by_mass(const Src& src, Seg sg, ScratchT<NWX>& sh, float maxv, double A, double eps,
                            int V, long long& R, uint32_t& wkey, uint32_t& eq, uint32_t& nkeep) {
  constexpr int NTX = NWX * kWave;
  uint32_t prefix = 0, mask = 0;
  double blow = 0.0;
  uint32_t cnt_low = 0;
  bool ok = true;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int b = threadIdx.x; b < 256; b += NTX) { sh.hcnt[b] = 0; sh.hmass[b] = 0.0; }
    __syncthreads();
    for (int i = sg.lo + lane_id(); i < sg.hi; i += kWave) {
      const float zi = src.z(i);
      const uint32_t k = fkey(zi);
      if ((k & mask) == prefix) {
        const uint32_t b = (k >> shift) & 255u;
        atomicAdd(&sh.hcnt[b], 1u);
        const double e = Src::kCache ? src.cached(i)
                                     : (zi == neg_inf() ? 0.0 : exp((double)(zi - maxv)));
        if (e != 0.0) atomicAdd(&sh.hmass[b], e);
      }
    }
    __syncthreads();
    if (wave_id() == 0) {
      const int l = lane_id();
      uint32_t c[4], lc = 0;
      double m[4], lm = 0.0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = sh.hcnt[4 * l + j];
        m[j] = sh.hmass[4 * l + j];
        lc += c[j];
        lm += m[j];
      }
      const double mincl = wave_incl_scan_f64(lm);
      const double mexcl = wave_shr1_f64(mincl, 0.0);
      const uint32_t cincl = wave_incl_scan_u32(lc);
      uint32_t crun = cincl - lc;
      double run = blow + mexcl;
      int hitb = -1;
      double before = 0.0, end = 0.0;
      uint32_t cbefore = 0, ceq = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const double e2 = run + m[j];
        if (hitb < 0 && e2 > A) { hitb = 4 * l + j; before = run; end = e2; cbefore = crun; ceq = c[j]; }
        run = e2;
        crun += c[j];
      }
      const uint64_t hit = __ballot(hitb >= 0);
      const int first = hit ? __ffsll((unsigned long long)hit) - 1 : -1;
      if (first < 0) {
        if (l == 63) { sh.bu[0] = 0xFFFFFFFFu; sh.bd[0] = run; }
      } else if (l == first) {
        sh.bu[0] = (uint32_t)hitb;
        sh.bu[1] = cbefore;
        sh.bu[2] = ceq;
        sh.bd[0] = before;
        sh.bd[1] = end;
      }
    }
    __syncthreads();
    const uint32_t b = sh.bu[0];
    if (b == 0xFFFFFFFFu) {
      // Nothing in range ends above A: every position has cum <= 1 - p.
      const double tot = sh.bd[0];
      __syncthreads();
      if (!(A - tot > eps * A)) return false;
      R = V;
      wkey = 0;
      eq = 0;
      nkeep = 0;
      return true;
    }
    const double before = sh.bd[0], end = sh.bd[1];
    const uint32_t cb = sh.bu[1], ceq = sh.bu[2];
    __syncthreads();
    if (!(end - A > eps * end)) ok = false;
    if (before > 0.0 && !(A - before > eps * A)) ok = false;
    if (!ok) return false;
    blow = before;
    cnt_low += cb;
    prefix |= b << shift;
    mask |= 0xFFu << shift;
    eq = ceq;
  }
  // Positions inside the crossing group: position j (1-based, ascending order)
  // is removed iff blow + j*q <= A.
  wkey = prefix;
  const double q = (wkey == kKeyNegInf) ? 0.0 : exp((double)(kfloat(wkey) - maxv));
  long long j = 0;
  if (q > 0.0) {
    double jf = floor((A - blow) / q);
    j = (long long)fmax(0.0, fmin(jf, (double)eq - 1.0));
    while (j > 0 && blow + (double)j * q > A) --j;
    while (j + 1 < (long long)eq && blow + (double)(j + 1) * q <= A) ++j;
    if (j >= 1) {
      const double bj = blow + (double)j * q;
      if (!(A - bj > eps * A)) return false;
    }
    if (j + 1 <= (long long)eq) {
      const double bj1 = blow + (double)(j + 1) * q;
      if (!(bj1 - A > eps * bj1)) return false;
    }
  }
  R = (long long)cnt_low + j;
  nkeep = eq - (uint32_t)j;
  return true;
}

// ---- exact sequential emulations -----------------------------------------------

// In-buffer ascending bitonic sort of P (a power of two) keys by the NTX
// threads of the workgroup.
template <int NTX>
__device__ void bitonic_sort_u32(uint32_t* buf, int P) {
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int t = threadIdx.x; t < (P >> 1); t += NTX) {
        const int i = (t / j) * 2 * j + (t % j);
        const int pi = i + j;
        const uint32_t a = buf[i], b = buf[pi];
        const bool up = (i & k) == 0;
        if ((a > b) == up) { buf[i] = b; buf[pi] = a; }
      }
      __syncthreads();
    }
  }
}

// Ascending sort of n <= 31 * NTX keys, buf -> buf + tmp_off -> buf ...: every
// thread owns one chunk of K keys (K odd, so that lanes K words apart hit
// distinct LDS banks): its run, sorted in registers by a 32-wide bitonic
// network, then merge-path rounds that double the run length, a thread
// writing the K outputs of its chunk's place in a pair of runs: a binary
// search over the pair's diagonal gives where they start in each run, then a
// sequential merge (equal keys from the first run first, in the search and
// the merge alike). Ends in buf.
template <int NWX>
__device__ void merge_sort_asc_u32(uint32_t* buf, int tmp_off, int n) {
  constexpr int NTX = NWX * kWave, R = 32;
  const int t = threadIdx.x;
  const int K = max(15, ((n + NTX - 1) / NTX) | 1);
  {
    const int b = t * K;
    const int cnt = max(0, min(K, n - b));
    uint32_t r[R];
#pragma unroll
    for (int i = 0; i < R; ++i) r[i] = i < cnt ? buf[b + i] : 0xFFFFFFFFu;   // the fill sorts last
#pragma unroll
    for (int k = 2; k <= R; k <<= 1)
#pragma unroll
      for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
        for (int i = 0; i < R; ++i) {
          const int l = i ^ j;
          if (l > i) {
            const uint32_t lo = min(r[i], r[l]), hi = max(r[i], r[l]);
            r[i] = (i & k) ? hi : lo;
            r[l] = (i & k) ? lo : hi;
          }
        }
#pragma unroll
    for (int i = 0; i < R; ++i)
      if (i < cnt) buf[b + i] = r[i];
  }
  __syncthreads();
  C4S_PHASE(9);
  // the source and destination as offsets from buf (a select between two
  // pointers would hide from the compiler that they are LDS addresses)
  int so = 0, dso = tmp_off;
  for (int L = K; L < n; L <<= 1) {
    const uint32_t* src = buf + so;
    uint32_t* dst = buf + dso;
    const int o = t * K;
    if (o < n) {
      const int base = o / (2 * L) * (2 * L);
      const int na = min(L, n - base), nb = min(L, n - base - na);   // na >= 1
      const uint32_t* A = src + base;
      const uint32_t* B = A + na;
      const int d = o - base;
      int lo = max(0, d - nb), hi = min(d, na);
      while (lo < hi) {   // the first i whose A[i] comes after B[d - i - 1]
        const int mid = (lo + hi) >> 1;
        if (A[mid] <= B[d - mid - 1]) lo = mid + 1;
        else hi = mid;
      }
      int i = lo, j = d - lo;
      const int cnt = min(K, n - o);
      // the heads of both runs in registers; past a run's end its last key is
      // read again and never taken
      uint32_t av = A[min(i, na - 1)], bv = nb > 0 ? B[min(j, nb - 1)] : 0u;
#pragma unroll
      for (int q = 0; q < R; ++q) {
        if (q < cnt) {
          const bool ta = j >= nb || (i < na && av <= bv);
          dst[o + q] = ta ? av : bv;
          i += ta ? 1 : 0;
          j += ta ? 0 : 1;
          const uint32_t nv = ta ? A[min(i, na - 1)] : B[min(j, nb - 1)];
          av = ta ? nv : av;
          bv = ta ? bv : nv;
        }
      }
    }
    __syncthreads();
    if (L == 512) C4S_PHASE(10);
    const int x = so;
    so = dso;
    dso = x;
  }
  if (so != 0) {
    for (int i = t; i < n; i += NTX) buf[i] = buf[so + i];
    __syncthreads();
  }
}

// exact_top_p (below) in the form for a workgroup of eight waves whose row and work area
// are in LDS and whose registers are its own (the one-AR-step kernel's
// fallback): one slot claim per wave and 64 keys; the merge sort when the
// work area holds the keys twice (else the bitonic network); the masses in two
// alternating windows, waves 1.. computing the next while wave 0 adds the
// current one in unguarded blocks.
template <int NWX, class Src>
__device__ long long exact_top_p_fast(const Src& src, Seg sg, ScratchT<NWX>& sh, float maxv, double thr, int V,
                                      uint32_t* buf) {
  constexpr int NTX = NWX * kWave;
  const int lane = lane_id(), w = wave_id();
  if (threadIdx.x == 0) sh.counter = 0;
  __syncthreads();
  // the finite keys
  for (int b0 = sg.lo; b0 < sg.hi; b0 += kWave) {
    const int i = b0 + lane;
    const float zi = i < sg.hi ? src.z(i) : neg_inf();
    const bool fin = zi != neg_inf();
    const uint64_t m = __ballot(fin);
    uint32_t slot = 0u;
    if (lane == 0 && m != 0ull) slot = atomicAdd(&sh.counter, (uint32_t)__popcll(m));
    slot = (uint32_t)__shfl((int)slot, 0, kWave);
    if (fin) buf[slot + __popcll(m & lanemask_lt())] = fkey(zi);
  }
  __syncthreads();
  const int nf = __builtin_amdgcn_readfirstlane((int)sh.counter);
  C4S_PHASE(11);
  const size_t cap = src.sort_bytes();
  if (cap >= 8 * (size_t)nf && nf <= 31 * NTX) {
    merge_sort_asc_u32<NWX>(buf, nf, nf);   // the second half of the work area
  } else {
    int P = 1;
    while (P < nf) P <<= 1;
    for (int i = nf + threadIdx.x; i < P; i += NTX) buf[i] = 0xFFFFFFFFu;
    __syncthreads();
    bitonic_sort_u32<NTX>(buf, P);
  }
  C4S_PHASE(12);
  const size_t kb = ((size_t)nf * 4 + 15) & ~(size_t)15;
  const int W2 = cap > kb ? (int)min((size_t)2048, (cap - kb) / 16) & ~(kWave - 1) : 0;
  if (W2 >= kWave) {
    // window k of the masses (divided by div unless it is 0) and zeros up to
    // the next multiple of 32 terms, by threads t0, t0 + nt, ...
    auto fill = [&](double* dst, int k, double div, int t0, int nt) {
      const int w0 = k * W2, wn = min(W2, nf - w0), wn32 = (wn + 31) & ~31;
      for (int j = t0; j < wn32; j += nt) {
        double e = 0.0;
        if (j < wn) {
          e = exp((double)(kfloat(buf[w0 + j]) - maxv));
          if (div != 0.0) e = e / div;
        }
        dst[j] = e;
      }
    };
    const int nwin = (nf + W2 - 1) / W2;
    double* const ew = reinterpret_cast<double*>(reinterpret_cast<unsigned char*>(buf) + kb);
    // window k's buffer: offsets from one base (a select between two pointers
    // would hide from the compiler that they are LDS addresses)
    auto win = [&](int k) { return ew + (k & 1) * W2; };
    fill(win(0), 0, 0.0, threadIdx.x, NTX);
    __syncthreads();
    double total = 0.0;
    for (int k = 0; k < nwin; ++k) {
      if (w == 0) total = seq_sum_blk(total, win(k), min(W2, nf - k * W2));
      else if (k + 1 < nwin) fill(win(k + 1), k + 1, 0.0, threadIdx.x - kWave, NTX - kWave);
      __syncthreads();
    }
    if (threadIdx.x == 0) sh.bd[7] = total;
    __syncthreads();
    total = sh.bd[7];
    C4S_PHASE(13);
    fill(win(0), 0, total, threadIdx.x, NTX);
    __syncthreads();
    double cum = 0.0;
    for (int k = 0; k < nwin; ++k) {
      // the stop flag alternates between bu[6] and bu[7]: wave 0 sets the next
      // one while the other waves may still read this one
      if (w == 0) {
        bool stop = false;
        const uint32_t removed = k * W2 + seq_cut_blk(cum, win(k), min(W2, nf - k * W2), thr, stop);
        if (lane == 0) {
          sh.bu[4] = removed;
          sh.bu[6 + (k & 1)] = stop ? 1u : 0u;
        }
      } else if (k + 1 < nwin) {
        fill(win(k + 1), k + 1, total, threadIdx.x - kWave, NTX - kWave);
      }
      __syncthreads();
      if (sh.bu[6 + (k & 1)]) break;
    }
  } else if (w == 0) {
    double total = 0.0;
    for (int base = 0; base < nf; base += kWave) {
      const int j = base + lane;
      const double e = (j < nf) ? exp((double)(kfloat(buf[j]) - maxv)) : 0.0;
      total = seq_sum_lanes(total, e, min(kWave, nf - base));
    }
    double cum = 0.0;
    uint32_t removed = 0;
    bool stop = false;
    for (int base = 0; base < nf && !stop; base += kWave) {
      const int j = base + lane;
      const double q = (j < nf) ? exp((double)(kfloat(buf[j]) - maxv)) / total : 0.0;
      removed = base + seq_cut_lanes(cum, q, min(kWave, nf - base), thr, stop);
    }
    if (lane == 0) sh.bu[4] = removed;
  }
  __syncthreads();
  C4S_PHASE(15);
  const uint32_t rfin = sh.bu[4];
  __syncthreads();
  return (long long)(V - nf) + rfin;
}

// Exact top_p removal count: sorts the finite keys ascending, then wave 0 runs
// sampling.cpp:52-65 literally (sequential double sum, then sequential
// cum += prob/sum against 1 - p). Returns R over all V positions (the -inf
// positions come first in ascending order with probability 0). The form
// for kernels that inline the chain beside live registers of their own: a
// claim per key, the bitonic network, one window at a time.
template <int NWX, class Src>
__device__ long long exact_top_p(const Src& src, Seg sg, ScratchT<NWX>& sh, float maxv, double thr,
                                 int V, uint32_t* buf, uint32_t& n_fin_out) {
  constexpr int NTX = NWX * kWave;
  if (threadIdx.x == 0) sh.counter = 0;
  __syncthreads();
  for (int i = sg.lo + lane_id(); i < sg.hi; i += kWave) {
    const float zi = src.z(i);
    if (zi != neg_inf()) {
      const uint32_t slot = atomicAdd(&sh.counter, 1u);
      buf[slot] = fkey(zi);
    }
  }
  __syncthreads();
  const uint32_t n_fin = sh.counter;
  int P = 1;
  while (P < (int)n_fin) P <<= 1;
  for (int i = n_fin + threadIdx.x; i < P; i += NTX) buf[i] = 0xFFFFFFFFu;
  __syncthreads();
  bitonic_sort_u32<NTX>(buf, P);
  C4S_SPEC_EV(0, 0);
  // The masses in windows of the buffer's free space after the keys: every
  // wave computes a window's exp (and quotients), wave 0 adds them one after
  // the other; without room for a window, wave 0 computes them itself.
  const size_t kb = ((size_t)n_fin * 4 + 15) & ~(size_t)15;
  const size_t cap = src.sort_bytes();
  int W = cap > kb ? (int)min((size_t)2048, (cap - kb) / 8) : 0;
  W &= ~(kWave - 1);
  if (W >= kWave) {
    double* ew = reinterpret_cast<double*>(reinterpret_cast<unsigned char*>(buf) + kb);
    double total = 0.0;
    for (int w0 = 0; w0 < (int)n_fin; w0 += W) {
      const int wn = min(W, (int)n_fin - w0);
      for (int j = threadIdx.x; j < wn; j += NTX) ew[j] = exp((double)(kfloat(buf[w0 + j]) - maxv));
      __syncthreads();
      if (wave_id() == 0) total = seq_sum_mem(total, ew, wn);
      __syncthreads();
    }
    if (threadIdx.x == 0) sh.bd[7] = total;
    __syncthreads();
    total = sh.bd[7];
    C4S_SPEC_EV(0, 1);
    double cum = 0.0;
    uint32_t removed = 0;
    for (int w0 = 0; w0 < (int)n_fin; w0 += W) {
      const int wn = min(W, (int)n_fin - w0);
      for (int j = threadIdx.x; j < wn; j += NTX) ew[j] = exp((double)(kfloat(buf[w0 + j]) - maxv)) / total;
      __syncthreads();
      if (wave_id() == 0) {
        bool stop = false;
        removed = w0 + seq_cut_mem(cum, ew, wn, thr, stop);
        if (lane_id() == 0) {
          sh.bu[4] = removed;
          sh.bu[7] = stop ? 1u : 0u;
        }
      }
      __syncthreads();
      if (sh.bu[7]) break;
    }
    C4S_SPEC_EV(0, 2);
  } else if (wave_id() == 0) {
    const int l = lane_id();
    double total = 0.0;
    for (int base = 0; base < (int)n_fin; base += kWave) {
      const int j = base + l;
      const double e = (j < (int)n_fin) ? exp((double)(kfloat(buf[j]) - maxv)) : 0.0;
      total = seq_sum_lanes(total, e, min(kWave, (int)n_fin - base));
    }
    double cum = 0.0;
    uint32_t removed = 0;
    bool stop = false;
    for (int base = 0; base < (int)n_fin && !stop; base += kWave) {
      const int j = base + l;
      const double q = (j < (int)n_fin) ? exp((double)(kfloat(buf[j]) - maxv)) / total : 0.0;
      removed = base + seq_cut_lanes(cum, q, min(kWave, (int)n_fin - base), thr, stop);
    }
    if (l == 0) sh.bu[4] = removed;
  }
  C4S_SPEC_EV(0, 3);
  __syncthreads();
  const uint32_t rfin = sh.bu[4];
  __syncthreads();
  n_fin_out = n_fin;
  return (long long)(V - (int)n_fin) + rfin;
}

// ---- keep predicate after top_p ------------------------------------------------
enum KeepMode { kKeepAll = 0, kKeepMassPos = 1, kKeepBoundary = 2, kKeepNone = 3 };

struct Keep {
  int mode;
  uint32_t wkey;
  uint32_t nkeep;   // how many of the wkey group stay (lowest ids first)
  bool ranked;      // nkeep < group size: needs tie ranks in id order
};

// Does position i survive, given its value, the mass w.r.t. the top_p maximum
// and its rank among the wkey group in id order.
__device__ __forceinline__ bool keep_test(const Keep& kp, uint32_t key, double e_tp, uint32_t rank) {
  switch (kp.mode) {
    case kKeepAll: return true;
    case kKeepMassPos: return e_tp > 0.0;
    case kKeepBoundary:
      return key > kp.wkey || (key == kp.wkey && (!kp.ranked || rank < kp.nkeep));
    default: return false;
  }
}

// ---- fast path for top-k rows (row staged in LDS) ------------------------------
//
// For 0 < k <= 64 the chain is decided on a few dozen candidates instead of the
// whole row. Layout: wave w owns ids [w*S, (w+1)*S), S = 64 * slots; lane l of
// slot j holds id w*S + 64*j + l (LDS reads are bank-conflict free and a wave's
// slot-major order is id order).
//  P1 (all waves)  per-lane maximum; per wave the j-th largest lane maximum L_w
//                  (j = ceil(k/10)): wave w holds j distinct ids >= L_w.
//  P2 (wave 0)     L0 = the ceil(k/j)-th largest L_w, a lower bound of the k-th
//                  largest value (ceil(k/j) * j >= k distinct ids are >= L0).
//  P3 (all)        ids with value >= L0 are compacted per wave, in id order.
//  P4 (all)        each wave copies its candidates into one id-ordered list at
//                  its prefix and adds them to a 256-bucket histogram of
//                  [L0, max].
//  P5 (wave 0)     the bucket holding the k-th largest value, the k-th value
//                  itself (ties counted with multiplicity), survivors of top_k
//                  (divided value >= threshold; a non-candidate can not reach it
//                  because fl(pred(L0)/t) < threshold is checked), exact
//                  masses exp(double(z - max)).
//  P6 (all)        for each survivor, mass and count at or below it in the
//                  ascending order (value asc, id desc), summed over survivors.
//  P7 (wave 0)     nucleus cut (cum <= 1 - p, with the error bound), min_keep,
//                  inverse-CDF draw in id order; a draw inside the bound is
//                  replayed sequentially in this wave.
// Anything undecidable returns false before the RNG or any output changes.
constexpr int kFastCap = 128;     // candidates handled by wave 0 (two per lane)
constexpr int kRegionCap = 64;    // candidates one wave may contribute
constexpr int kMaxSlots = kLdsVocabMax / (NW * kWave);
static_assert(kMaxSlots * NW * kWave == kLdsVocabMax, "slots cover the LDS-staged rows");

template <int NTX = NT>
__device__ __forceinline__ int odd_chunk(int V) { return ((V + NTX - 1) / NTX) | 1; }

struct FastBuf {
  float* ry;       // [NW][kRegionCap]
  int* rid;        // [NW][kRegionCap]
  float* fy;       // [kFastCap] id-ordered candidate values
  int* fid;        // [kFastCap]
  uint32_t* fb;    // [kFastCap] histogram bucket
  float* sz;       // [kFastCap] divided value (survivors)
  double* sE;      // [kFastCap] mass (0 for non-survivors)
  double* M;       // [kFastCap] mass at or below, over survivors
  uint32_t* Mc;    // [kFastCap] count at or below
};
constexpr size_t kFastBytes = (size_t)NW * kRegionCap * 8 + (size_t)kFastCap * (4 + 4 + 4 + 4 + 8 + 8 + 4);

__device__ __forceinline__ FastBuf fast_buf(unsigned char* work) {
  FastBuf f;
  f.sE = reinterpret_cast<double*>(work);
  f.M = f.sE + kFastCap;
  f.ry = reinterpret_cast<float*>(f.M + kFastCap);
  f.rid = reinterpret_cast<int*>(f.ry + NW * kRegionCap);
  f.fy = reinterpret_cast<float*>(f.rid + NW * kRegionCap);
  f.fid = reinterpret_cast<int*>(f.fy + kFastCap);
  f.fb = reinterpret_cast<uint32_t*>(f.fid + kFastCap);
  f.sz = reinterpret_cast<float*>(f.fb + kFastCap);
  f.Mc = reinterpret_cast<uint32_t*>(f.sz + kFastCap);
  return f;
}

__device__ __forceinline__ bool fast_topk_applies(const RowCfg& c, int V) {
  return c.draw && c.topk_on && c.k <= 64 && V <= kLdsVocabMax &&
         (size_t)8 * ((V + 3) & ~3) >= kFastBytes;
}

__device__ __forceinline__ uint32_t near_top_bucket(float maxY, float y, float inv) {
  return (uint32_t)min(255, (int)((maxY - y) * inv));
}

template <int NS>
__device__ bool fast_topk(const float* val, int V, const RowCfg& c, Scratch& sh,
                          unsigned char* work, uint64_t& rng, int& tok_out, float* masked,
                          uint32_t* stats) {
  constexpr int S = NS * kWave;
  const int t = threadIdx.x, lane = lane_id(), w = wave_id();
  const float ninf = neg_inf();
  const FastBuf fb = fast_buf(work);
  const int jj = min(8, max(1, (c.k + 9) / 10));
  const int need_w = (c.k + jj - 1) / jj;

  // P1: values, lane maxima, per-wave bound
  const int base = w * S;
  float yv[NS];
  float tmax = ninf;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int i = base + kWave * j + lane;
    yv[j] = (i < V) ? val[i] : ninf;
    tmax = fmaxf(tmax, yv[j]);
  }
  if (t < 256) sh.hcnt[t] = 0u;
  if (t < kFastCap) { fb.M[t] = 0.0; fb.Mc[t] = 0u; }
  const float wmax = wave_max_dpp(tmax);
  float cur = tmax, lw = wmax;
  for (int r = 1; r < jj; ++r) {
    const uint64_t m = __ballot(cur == lw);
    if (lane == __ffsll((unsigned long long)m) - 1) cur = ninf;
    lw = wave_max_dpp(cur);
  }
  if (lane == 0) { sh.redf[w] = wmax; sh.redf2[w] = lw; }
  if (masked)
    for (int i = t; i < V; i += NT) masked[i] = ninf;
  __syncthreads();
  C4S_PHASE(2);

  // P2: L0 (wave 0)
  if (w == 0) {
    const float lwl = lane < NW ? sh.redf2[lane] : ninf;
    const float maxY = wave_max_dpp(lane < NW ? sh.redf[lane] : ninf);
    uint32_t ge = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) ge += (readlane_f32(lwl, i) >= lwl) ? 1u : 0u;
    const float L0 = wave_max_dpp((lane < NW && ge >= (uint32_t)need_w) ? lwl : ninf);
    if (lane == 0) { sh.bd[0] = (double)maxY; sh.bd[1] = (double)L0; }
  }
  __syncthreads();
  C4S_PHASE(3);
  const float maxY = (float)sh.bd[0], L0 = (float)sh.bd[1];
  const float R = maxY - L0;
  if (!(L0 > ninf) || !(R < __builtin_inff())) { __syncthreads(); return false; }
  const float inv = (R > 0.0f) ? 256.0f / R : 0.0f;

  // P3: per-wave compaction, id order within the wave
  uint32_t wcount = 0;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const bool f = yv[j] >= L0;
    const uint64_t m = __ballot(f);
    if (m) {
      const uint32_t pos = wcount + (uint32_t)__popcll(m & lanemask_lt());
      if (f && pos < (uint32_t)kRegionCap) {
        fb.ry[w * kRegionCap + pos] = yv[j];
        fb.rid[w * kRegionCap + pos] = base + kWave * j + lane;
      }
      wcount += (uint32_t)__popcll(m);
    }
  }
  if (lane == 0) sh.wcnt[w] = wcount;
  __syncthreads();
  C4S_PHASE(4);

  // P4: one id-ordered list + histogram
  uint32_t C = 0, pre = 0;
  bool over = false;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const uint32_t ci = sh.wcnt[i];
    over = over || ci > (uint32_t)kRegionCap;
    if (i < w) pre += ci;
    C += ci;
  }
  if (over || C > (uint32_t)kFastCap) { __syncthreads(); return false; }
  if (lane < (int)wcount) {
    const float y = fb.ry[w * kRegionCap + lane];
    const uint32_t bk = near_top_bucket(maxY, y, inv);
    fb.fy[pre + lane] = y;
    fb.fid[pre + lane] = fb.rid[w * kRegionCap + lane];
    fb.fb[pre + lane] = bk;
    atomicAdd(&sh.hcnt[bk], 1u);
  }
  __syncthreads();
  C4S_PHASE(5);

  // P5: k-th value, survivors, masses (wave 0; entries lane and lane + 64)
  const float maxv = c.temp_on ? maxY / c.temp : maxY;
  if (w == 0) {
    uint32_t c4[4], lc = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) { c4[j] = sh.hcnt[4 * lane + j]; lc += c4[j]; }
    const uint32_t incl = wave_scan_u32(lc);
    uint32_t run = incl - lc, above_b = 0;
    int hit = -1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (hit < 0 && run + c4[j] >= (uint32_t)c.k) { hit = 4 * lane + j; above_b = run; }
      run += c4[j];
    }
    const uint64_t hm = __ballot(hit >= 0);
    bool bail = hm == 0ull;
    float zthr = ninf;
    uint32_t nsurv = 0;
    if (!bail) {
      const int fl = __ffsll((unsigned long long)hm) - 1;
      const uint32_t bstar = readlane_u32((uint32_t)hit, fl);
      const uint32_t need = (uint32_t)c.k - readlane_u32(above_b, fl);
      const bool v0 = lane < (int)C, v1 = lane + kWave < (int)C;
      const float y0 = v0 ? fb.fy[lane] : ninf, y1 = v1 ? fb.fy[lane + kWave] : ninf;
      const bool in0 = v0 && fb.fb[lane] == bstar, in1 = v1 && fb.fb[lane + kWave] == bstar;
      // need-th largest value among the boundary bucket (multiplicity counted)
      float yk = ninf;
      uint64_t m0 = __ballot(in0), m1 = __ballot(in1);
      while (m0 | m1) {
        float yq;
        if (m0) { const int q = __ffsll((unsigned long long)m0) - 1; m0 &= m0 - 1; yq = readlane_f32(y0, q); }
        else { const int q = __ffsll((unsigned long long)m1) - 1; m1 &= m1 - 1; yq = readlane_f32(y1, q); }
        const uint32_t gt = (uint32_t)(__popcll(__ballot(in0 && y0 > yq)) + __popcll(__ballot(in1 && y1 > yq)));
        const uint32_t ge = (uint32_t)(__popcll(__ballot(in0 && y0 >= yq)) + __popcll(__ballot(in1 && y1 >= yq)));
        if (gt < need && need <= ge) { yk = yq; break; }
      }
      zthr = c.temp_on ? yk / c.temp : yk;
      // every id left out is <= pred(L0); after the division it must stay below the threshold
      const float l0m = nextafterf(L0, ninf);
      bail = !(yk > ninf) || (c.temp_on ? !(l0m / c.temp < zthr) : !(l0m < zthr));
      const float z0 = c.temp_on ? y0 / c.temp : y0, z1 = c.temp_on ? y1 / c.temp : y1;
      const bool s0 = v0 && z0 >= zthr, s1 = v1 && z1 >= zthr;
      fb.sz[lane] = z0;
      fb.sz[lane + kWave] = z1;
      fb.sE[lane] = s0 ? exp((double)(z0 - maxv)) : -1.0;
      fb.sE[lane + kWave] = s1 ? exp((double)(z1 - maxv)) : -1.0;
      nsurv = (uint32_t)(__popcll(__ballot(s0)) + __popcll(__ballot(s1)));
    }
    if (lane == 0) { sh.bi[0] = bail ? 1 : 0; sh.bu[0] = nsurv; sh.bd[2] = (double)zthr; }
  }
  __syncthreads();
  C4S_PHASE(6);
  if (sh.bi[0]) { __syncthreads(); return false; }
  const uint32_t nsurv = sh.bu[0];

  // P6: survivor pairs; wave w takes partner entries [8w, 8w + 8)
  {
    constexpr int kPer = kFastCap / NW;
    const float zq0 = fb.sz[lane], zq1 = fb.sz[lane + kWave];
    const bool sq0 = fb.sE[lane] >= 0.0, sq1 = fb.sE[lane + kWave] >= 0.0;
    double m0 = 0.0, m1 = 0.0;
    uint32_t c0 = 0, c1 = 0;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int j = w * kPer + i;
      const double Ej = fb.sE[j];
      if (Ej >= 0.0) {
        const float zj = fb.sz[j];
        // j is at or below q in ascending order: z_j < z_q, or equal and id_j >= id_q
        if (sq0 && ((zj < zq0) || (zj == zq0 && j >= lane))) { m0 += Ej; ++c0; }
        if (sq1 && ((zj < zq1) || (zj == zq1 && j >= lane + kWave))) { m1 += Ej; ++c1; }
      }
    }
    if (c0) { atomicAdd(&fb.M[lane], m0); atomicAdd(&fb.Mc[lane], c0); }
    if (c1) { atomicAdd(&fb.M[lane + kWave], m1); atomicAdd(&fb.Mc[lane + kWave], c1); }
  }
  __syncthreads();
  C4S_PHASE(7);

  // P7: nucleus cut, min_keep, draw (wave 0)
  if (w == 0) {
    const double e0r = fb.sE[lane], e1r = fb.sE[lane + kWave];
    const bool s0 = e0r >= 0.0, s1 = e1r >= 0.0;
    const double E0 = s0 ? e0r : 0.0, E1 = s1 ? e1r : 0.0;
    const double M0 = fb.M[lane], M1 = fb.M[lane + kWave];
    const uint32_t q0 = fb.Mc[lane], q1 = fb.Mc[lane + kWave];
    const int id0 = (lane < (int)C) ? fb.fid[lane] : 0;
    const int id1 = (lane + kWave < (int)C) ? fb.fid[lane + kWave] : 0;
    const double S = wave_sum_dpp(E0 + E1);
    const double thr = 1.0 - (double)c.p;
    const double eps = rel_eps(V);
    bool r0 = false, r1 = false, unsure = false;
    if (c.topp_on && thr >= 0.0) {
      if (thr == 0.0) {
        r0 = s0 && M0 == 0.0;
        r1 = s1 && M1 == 0.0;
      } else {
        const double A = thr * S;
        r0 = s0 && M0 <= A;
        r1 = s1 && M1 <= A;
        unsure = (s0 && !(fabs(M0 - A) > eps * fmax(M0, A))) || (s1 && !(fabs(M1 - A) > eps * fmax(M1, A)));
      }
    }
    // subnormal masses may differ between libm implementations: let the general path decide
    unsure = unsure || (s0 && E0 < 0x1p-1000) || (s1 && E1 < 0x1p-1000);
    const bool bail = __ballot(unsure) != 0ull;
    const long long R = (c.topp_on && thr >= 0.0)
                            ? (long long)(V - (int)nsurv) + (long long)(__popcll(__ballot(r0)) + __popcll(__ballot(r1)))
                            : 0ll;
    const long long lim = (long long)V - (long long)c.min_keep < 0 ? 0 : (long long)V - (long long)c.min_keep;
    const long long m = (long long)V - (R < lim ? R : lim);
    const bool k0 = s0 && (long long)(nsurv - q0) < m;
    const bool k1 = s1 && (long long)(nsurv - q1) < m;
    const double K0 = k0 ? E0 : 0.0, K1 = k1 ? E1 : 0.0;
    const double a0 = wave_scan_f64(K0);
    const double h0 = readlane_f64(a0, kWave - 1);
    const double a1 = wave_scan_f64(K1) + h0;
    const double Sd = readlane_f64(a1, kWave - 1);
    const uint64_t st = xorshift64(rng);
    const double u = unit_from_state(st);
    const double r = u * Sd;
    int tok = 0;
    bool sure = false;
    const uint64_t hm0 = __ballot(k0 && a0 >= r), hm1 = __ballot(k1 && a1 >= r);
    if (r > 0.0 && (hm0 | hm1)) {
      double af, pf;
      if (hm0) {
        const int f = __ffsll((unsigned long long)hm0) - 1;
        af = readlane_f64(a0, f); pf = af - readlane_f64(K0, f); tok = (int)readlane_u32((uint32_t)id0, f);
      } else {
        const int f = __ffsll((unsigned long long)hm1) - 1;
        af = readlane_f64(a1, f); pf = af - readlane_f64(K1, f); tok = (int)readlane_u32((uint32_t)id1, f);
      }
      sure = (af - r > eps * af) && (r - pf > eps * r);
    }
    uint32_t draw_exact = 0;
    if (!sure) {
      // text2semantic.cpp:152-164 in id order; ids outside the list weigh 0
      draw_exact = 1;
      double tot = 0.0;
      for (int q = 0; q < kWave; ++q) tot += readlane_f64(K0, q);
      for (int q = 0; q < kWave; ++q) tot += readlane_f64(K1, q);
      const double rr = u * tot;
      double acc = 0.0;
      tok = V - 1;
      if (rr <= 0.0) {
        tok = 0;
      } else {
        bool fnd = false;
        for (int q = 0; q < 2 * kWave && !fnd; ++q) {
          acc += (q < kWave) ? readlane_f64(K0, q) : readlane_f64(K1, q - kWave);
          if (rr <= acc) {
            tok = (int)((q < kWave) ? readlane_u32((uint32_t)id0, q) : readlane_u32((uint32_t)id1, q - kWave));
            fnd = true;
          }
        }
      }
    }
    if (masked) {
      if (k0) masked[id0] = fb.sz[lane];
      if (k1) masked[id1] = fb.sz[lane + kWave];
    }
    if (lane == 0) {
      sh.bi[0] = tok;
      sh.bi[1] = bail ? 1 : 0;
      sh.bu[3] = (uint32_t)(__popcll(__ballot(k0)) + __popcll(__ballot(k1)));
      sh.bu[4] = draw_exact;
    }
  }
  __syncthreads();
  C4S_PHASE(8);
  const bool bail = sh.bi[1] != 0;
  const int tok = sh.bi[0];
  const uint32_t nk = sh.bu[3], dex = sh.bu[4];
  __syncthreads();
  if (bail) return false;
  rng = xorshift64(rng);
  tok_out = tok;
  if (stats && t == 0) {
    stats[0] = 1u | 2u | (c.topp_on ? 4u : 0u) | 16u;
    stats[1] = 0u;
    stats[2] = dex;
    stats[3] = nk;
  }
  return true;
}

// Dispatch on the slot count (9 slots cover 9216 ids, 12 cover 12288).
__device__ __forceinline__ bool fast_topk_any(const float* val, int V, const RowCfg& c, Scratch& sh,
                                              unsigned char* work, uint64_t& rng, int& tok,
                                              float* masked, uint32_t* stats) {
  if (V <= 9 * NW * kWave) return fast_topk<9>(val, V, c, sh, work, rng, tok, masked, stats);
  return fast_topk<12>(val, V, c, sh, work, rng, tok, masked, stats);
}

// ---- the chain ------------------------------------------------------------------
template <int NWX, class Src, bool kFastExact = false>
__device__ __forceinline__ int run_chain(Src& src, ScratchT<NWX>& sh, const RowCfg& c, uint64_t& rng,
                                         float* masked, uint32_t* stats, bool tp_exact_first = false) {
  constexpr int NTX = NWX * kWave;
  const int V = c.V;
  const Seg sg = my_seg<NWX>(V);
  const int lane = lane_id();
  uint32_t st_path = 0, st_tp_exact = 0, st_draw_exact = 0, st_kept = 0;

  if (c.greedy) {
    float bv = neg_inf();
    int bi = INT_MAX;
    for (int i = sg.lo + lane; i < sg.hi; i += kWave) argmax_merge(bv, bi, src.z(i), i);
    block_argmax<NTX>(bv, bi, sh.redf, sh.redi);
    if (masked)
      for (int i = sg.lo + lane; i < sg.hi; i += kWave) masked[i] = src.z(i);
    if (stats && threadIdx.x == 0) { stats[0] = 8u; stats[1] = 0; stats[2] = 0; stats[3] = V; }
    return bi;
  }

  if (c.temp_on) src.apply_temperature(c.temp, sg.lo, sg.hi);

  if (c.topk_on) {
    uint32_t gt, eq;
    const uint32_t tk = select_desc([&](int i) { return fkey(src.zraw(i)); }, sg, sh,
                                    (uint32_t)c.k, gt, eq);
    src.thr_key = tk;
    src.topk_on = true;
    st_path |= 2u;
  }

  float maxv = neg_inf();
  if (c.topp_on || c.draw) {
    float lm = neg_inf();
    for (int i = sg.lo + lane; i < sg.hi; i += kWave) lm = fmaxf(lm, src.z(i));
    maxv = block_max_f32<NTX>(lm, sh.redf);
  }

  Keep kp{kKeepAll, 0u, 0u, false};
  bool cache_ok = false;   // E[] holds exp(z - maxv) for every id (LDS rows)
  bool any_kept = true;
  if (c.topp_on && maxv != neg_inf()) {
    st_path |= 4u;
    // tp_exact_first: the caller's own mass test missed its margin with double
    // sums, so the one below would too; the exact emulation decides at once
    // (p < 1 is 1 - p > 0)
    const bool direct = tp_exact_first && c.p < 1.0f;
    double sl = 0.0;
    uint32_t zl = 0;
    if (!direct)
      for (int i = sg.lo + lane; i < sg.hi; i += kWave) {
        const float zi = src.z(i);
        const double e = (zi == neg_inf()) ? 0.0 : exp((double)(zi - maxv));
        if (Src::kCache) src.cache(i, e);
        sl += e;
        zl += (e == 0.0) ? 1u : 0u;
      }
    const double S = direct ? 0.0 : block_sum_f64<NTX>(sl, sh.redd);
    cache_ok = Src::kCache && !direct;
    const double thr = 1.0 - (double)c.p;   // sampling.cpp:64 compares cum <= (1.0 - p)
    long long R = 0;
    bool have_cross = false;
    uint32_t cwkey = 0, ceq = 0, cnkeep = 0;
    if (thr < 0.0) {
      R = 0;
    } else if (thr == 0.0) {
      R = block_sum_u32<NTX>(zl, sh.redu);  // only zero-probability positions have cum == 0
    } else {
      const double eps = rel_eps(V);
      if (!direct && cut_by_mass(src, sg, sh, maxv, thr * S, eps, V, R, cwkey, ceq, cnkeep)) {
        have_cross = (R < V);
      } else {
        if constexpr (kFastExact) {
          R = exact_top_p_fast<NWX>(src, sg, sh, maxv, thr, V, src.sort_buf());
        } else {
          uint32_t nfin;
          R = exact_top_p(src, sg, sh, maxv, thr, V, src.sort_buf(), nfin);
        }
        cache_ok = false;
        st_tp_exact = 1;
      }
    }
    // min_tokens_to_keep: the last min_keep ascending positions are never removed.
    const long long mk = c.min_keep;
    const long long lim = (long long)V - mk < 0 ? 0 : (long long)V - mk;
    const long long Rf = R < lim ? R : lim;
    if (Rf <= 0) {
      kp.mode = kKeepAll;
    } else if (Rf >= V) {
      kp.mode = kKeepNone;
      any_kept = false;
    } else if (have_cross && Rf == R) {
      kp.mode = kKeepBoundary;
      kp.wkey = cwkey;
      kp.nkeep = cnkeep;
      kp.ranked = cnkeep < ceq;
    } else if (thr == 0.0 && Rf == R) {
      kp.mode = kKeepMassPos;
    } else {
      // Keep exactly the top m = V - Rf positions in (value desc, id asc) order.
      uint32_t gt, eq;
      const uint32_t wk = select_desc([&](int i) { return fkey(src.z(i)); }, sg, sh,
                                      (uint32_t)((long long)V - Rf), gt, eq);
      kp.mode = kKeepBoundary;
      kp.wkey = wk;
      kp.nkeep = (uint32_t)((long long)V - Rf) - gt;
      kp.ranked = kp.nkeep < eq;
    }
  }

  // Tie-rank bases: how many wkey-group members precede each wave's segment.
  uint32_t tie_base = 0;
  if (kp.mode == kKeepBoundary && kp.ranked) {
    uint32_t cl = 0;
    for (int i = sg.lo + lane; i < sg.hi; i += kWave) cl += (fkey(src.z(i)) == kp.wkey) ? 1u : 0u;
    cl = wave_sum_u32(cl);
    if (lane == 0) sh.wcnt[wave_id()] = cl;
    __syncthreads();
    for (int w = 0; w < wave_id(); ++w) tie_base += sh.wcnt[w];
    __syncthreads();
  }

  // Draw maximum (text2semantic.cpp:150-151): max over surviving values, from -1e30f.
  const float maxv_d = fmaxf(-1e30f, any_kept ? maxv : neg_inf());
  const bool reuse = cache_ok && (maxv_d == maxv);

  // Finalize: survivors in id order, masked output, draw masses per wave.
  double wm = 0.0;
  uint32_t kl = 0;
  {
    uint32_t carry = tie_base;
    for (int base = sg.lo; base < sg.hi; base += kWave) {
      const int i = base + lane;
      const bool valid = i < sg.hi;
      const float zi = valid ? src.z(i) : neg_inf();
      const uint32_t key = fkey(zi);
      const bool is_w = valid && kp.mode == kKeepBoundary && key == kp.wkey;
      const uint64_t bal = __ballot(is_w);
      const uint32_t rank = carry + (uint32_t)__popcll(bal & lanemask_lt());
      carry += (uint32_t)__popcll(bal);
      double e_tp = 0.0;
      if (kp.mode == kKeepMassPos)
        e_tp = cache_ok ? (valid ? src.cached(i) : 0.0)
                        : (zi == neg_inf() ? 0.0 : exp((double)(zi - maxv)));
      const bool kept = valid && keep_test(kp, key, e_tp, rank);
      const float out = kept ? zi : neg_inf();
      if (masked && valid) masked[i] = out;
      if (kept && zi != neg_inf()) ++kl;
      if (c.draw && valid) {
        double e = 0.0;
        if (kept && zi != neg_inf())   // +inf/NaN are outside the input contract
          e = reuse ? src.cached(i) : exp((double)(out - maxv_d));
        wm += e;
        if (Src::kCache) src.cache(i, e);
      }
    }
  }
  st_kept = block_sum_u32<NTX>(kl, sh.redu);

  int tok = 0;
  if (c.draw) {
    wm = wave_sum_f64(wm);
    if (lane == 0) sh.wmass[wave_id()] = wm;
    __syncthreads();
    // Per-wave exclusive prefixes and the total, summed in a fixed order.
    double tot = 0.0;
    for (int w = 0; w < NWX; ++w) tot += sh.wmass[w];
    rng = xorshift64(rng);
    const double u = unit_from_state(rng);
    const double r = u * tot;
    int owner = NWX - 1;
    double xown = 0.0;
    {
      double x = 0.0;
      for (int w = 0; w < NWX; ++w) {
        const double nx = x + sh.wmass[w];
        if (nx >= r) { owner = w; xown = x; break; }
        x = nx;
      }
    }
    __syncthreads();
    const double eps = rel_eps(V);
    if (wave_id() == owner) {
      double carry_m = xown;
      int found = -1;
      double acc = 0.0, prev = 0.0;
      uint32_t carry = tie_base;
      for (int base = sg.lo; base < sg.hi && found < 0; base += kWave) {
        const int i = base + lane;
        const bool valid = i < sg.hi;
        double e = 0.0;
        if (Src::kCache) {
          e = valid ? src.cached(i) : 0.0;
        } else {
          const float zi = valid ? src.z(i) : neg_inf();
          const uint32_t key = fkey(zi);
          const bool is_w = valid && kp.mode == kKeepBoundary && key == kp.wkey;
          const uint64_t bal = __ballot(is_w);
          const uint32_t rank = carry + (uint32_t)__popcll(bal & lanemask_lt());
          carry += (uint32_t)__popcll(bal);
          const double e_tp = (kp.mode == kKeepMassPos && zi != neg_inf())
                                  ? exp((double)(zi - maxv)) : 0.0;
          if (valid && zi != neg_inf() && keep_test(kp, key, e_tp, rank))
            e = exp((double)(zi - maxv_d));
        }
        const double inc = wave_incl_scan_f64(e) + carry_m;
        const uint64_t hit = __ballot(valid && inc >= r);
        if (hit) {
          const int L = __ffsll((unsigned long long)hit) - 1;
          found = base + L;
          acc = __shfl(inc, L, kWave);
          const double before = wave_shr1_f64(inc, 0.0);
          const double pb = __shfl(before, L, kWave);
          prev = (L == 0) ? carry_m : pb;
        }
        carry_m = __shfl(inc, kWave - 1, kWave);
      }
      const bool certain = found >= 0 && (acc - r > eps * acc) && (r - prev > eps * r);
      if (lane == 0) { sh.bi[0] = found; sh.bi[1] = certain ? 1 : 0; }
    }
    __syncthreads();
    tok = sh.bi[0];
    const bool certain = sh.bi[1] != 0;
    __syncthreads();
    if (!certain) {
      // text2semantic.cpp:152-165 literally: sequential sums in id order.
      st_draw_exact = 1;
      if (wave_id() == 0) {
        double total = 0.0;
        for (int pass = 0; pass < 2; ++pass) {
          double acc = 0.0, rr = 0.0;
          if (pass == 1) rr = u * total;
          int t = V - 1;
          bool done = false;
          uint32_t carry = 0;
          for (int base = 0; base < V && !done; base += kWave) {
            const int i = base + lane;
            const bool valid = i < V;
            double e = 0.0;
            if (Src::kCache) {
              e = valid ? src.cached(i) : 0.0;
            } else {
              const float zi = valid ? src.z(i) : neg_inf();
              const uint32_t key = fkey(zi);
              const bool is_w = valid && kp.mode == kKeepBoundary && key == kp.wkey;
              const uint64_t bal = __ballot(is_w);
              const uint32_t rank = carry + (uint32_t)__popcll(bal & lanemask_lt());
              carry += (uint32_t)__popcll(bal);
              const double e_tp = (kp.mode == kKeepMassPos && zi != neg_inf())
                                      ? exp((double)(zi - maxv)) : 0.0;
              if (valid && zi != neg_inf() && keep_test(kp, key, e_tp, rank))
                e = exp((double)(zi - maxv_d));
            }
            const int cnt = min(kWave, V - base);
            if (pass == 0) {
              total = seq_sum_lanes(total, e, cnt);
            } else {
              const int q = seq_find_lanes(acc, e, cnt, rr);
              if (q >= 0) { t = base + q; done = true; }
            }
          }
          if (pass == 1 && lane == 0) sh.bi[2] = t;
        }
      }
      __syncthreads();
      tok = sh.bi[2];
      __syncthreads();
    }
  }
  if (stats && threadIdx.x == 0) {
    stats[0] = st_path | (c.draw ? 1u : 0u);
    stats[1] = st_tp_exact;
    stats[2] = st_draw_exact;
    stats[3] = st_kept;
  }
  return tok;
}

__device__ __forceinline__ float load_logit(const void* base, int dtype, int64_t off) {
  if (dtype == 1) {
    const uint16_t b = static_cast<const uint16_t*>(base)[off];
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
  }
  return static_cast<const float*>(base)[off];
}

struct LdsLayout {
  double* E;
  float* val;
  uint32_t* bitmap;
};

__host__ __device__ __forceinline__ int vpad(int V) { return (V + 3) & ~3; }
__host__ __device__ __forceinline__ int bitmap_words(int V) { return ((V + 31) / 32 + 1 + 3) & ~3; }
// Words of a caller's per-row history set (c4s_rows.hist_bits).
__host__ __device__ __forceinline__ int hist_words(int V) { return (V + 31) / 32; }

// `val` is the row buffer base (vpad(V) + 4 floats); a row is stored at
// val + shift so that its float4 body is 16-byte aligned in LDS.
__device__ __forceinline__ LdsLayout lds_layout(unsigned char* smem, int V) {
  LdsLayout L;
  L.E = reinterpret_cast<double*>(smem);
  L.val = reinterpret_cast<float*>(smem + 8 * (size_t)vpad(V));
  L.bitmap = reinterpret_cast<uint32_t*>(L.val + vpad(V) + 4);
  return L;
}

// Coalesced fetch of one f32 row of at most kLdsVocabMax ids into registers:
// the 0-3 ids before the first 16-byte boundary and the 0-3 ids after the
// last one go one per thread, the rest as float4 (at most 3 per thread).
struct RowFetch {
  float4 body[3];
  float edge;
};

struct RowShape {
  int head, nq, tail;
};
__device__ __forceinline__ RowShape row_shape(const float* p, int V) {
  RowShape r;
  r.head = min(V, (int)(((16u - ((uint32_t)(uintptr_t)p & 15u)) & 15u) >> 2));
  r.nq = (V - r.head) >> 2;
  r.tail = V - r.head - 4 * r.nq;
  return r;
}

__device__ __forceinline__ void fetch_row(const float* p, int V, RowFetch& f) {
  const RowShape r = row_shape(p, V);
  const float4* p4 = reinterpret_cast<const float4*>(p + r.head);
  const int t = threadIdx.x;
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int q = t + NT * j;
    f.body[j] = (q < r.nq) ? p4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  f.edge = (t < r.head) ? p[t] : ((t < r.head + r.tail) ? p[r.head + 4 * r.nq + (t - r.head)] : 0.f);
}

// Writes the fetched row into LDS and returns where it starts (buf + 0..3).
__device__ __forceinline__ float* store_row(const float* p, int V, const RowFetch& f, float* buf) {
  const RowShape r = row_shape(p, V);
  float* val = buf + ((4 - r.head) & 3);
  const int t = threadIdx.x;
  float4* body = reinterpret_cast<float4*>(val + r.head);
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int q = t + NT * j;
    if (q < r.nq) body[q] = f.body[j];
  }
  if (t < r.head) val[t] = f.edge;
  else if (t < r.head + r.tail) val[r.head + 4 * r.nq + (t - r.head)] = f.edge;
  return val;
}

// Repetition penalty on the LDS row (sampling.cpp:19-28): every id whose bit is
// set in `bitmap` is penalised once. Thread t of NTX handles its own id chunk.
template <int NTX = NT>
__device__ __forceinline__ void penalise_chunk(float* val, const uint32_t* bitmap, int V, float pen) {
  const double rp = 1.0 / (double)pen;
  const int ch = odd_chunk<NTX>(V);
  const int lo = min(V, (int)threadIdx.x * ch);
  const int hi = min(V, lo + ch);
  // the chunk's bits, 32 ids at a time (a chunk may span several words)
  for (int b0 = lo; b0 < hi; b0 += 32) {
    const int w0 = b0 >> 5;
    uint64_t bits = (uint64_t)bitmap[w0] | ((uint64_t)bitmap[w0 + 1] << 32);
    bits >>= (b0 - 32 * w0);
    const int len = min(32, hi - b0);
    bits &= (1ull << len) - 1ull;
    while (bits) {
      const int i = b0 + __ffsll((unsigned long long)bits) - 1;
      bits &= bits - 1;
      const float s = val[i];
      val[i] = (s < 0) ? s * pen : div_rcp(s, rp);   // sampling.cpp:26
    }
  }
}


// ---- draw over one candidate per lane ------------------------------------------

// Inverse-CDF draw (text2semantic.cpp:150-165) over at most one kept entry per
// lane: id, mass e, and slot = its rank in id order among some superset of the
// kept entries (distinct, below 2^kBits). The entries move to lanes in id order
// (rank by ballots over the slot bits, then a lane permute) and one prefix
// scan forms the id-order sums. The reference sums sequentially, so the first
// lane reaching r = u * total decides only with the margin rel_eps (plus
// eps_add, the relative error of masses that are approximations); otherwise
// the id-order sums are replayed sequentially (ids outside the kept set weigh
// 0), or, when replay is false (approximate masses), -1 is returned.
template <int kBits = 10>
__device__ __forceinline__ int lane_draw(bool kept, int id, int slot, double e, double u, int V, uint32_t& exact,
                                         double eps_add = 0.0, bool replay = true) {
  const int lane = lane_id();
  const double eps = rel_eps(V) + eps_add;
  const uint64_t km = __ballot(kept);
  const int nk = __popcll(km);
  // position among the kept entries in id order
  uint64_t same = km;
  int pos = 0;
#pragma unroll
  for (int b = kBits - 1; b >= 0; --b) {
    const bool bit = kept && ((slot >> b) & 1);
    const uint64_t one = __ballot(bit);
    pos += bit ? __popcll(same & ~one) : 0;
    same &= bit ? one : ~one;
  }
  const int a4 = (kept ? pos : kWave - 1) << 2;   // lanes past nk are ignored
  const uint64_t eb = (uint64_t)__double_as_longlong(e);
  const uint32_t plo = (uint32_t)__builtin_amdgcn_ds_permute(a4, (int)(uint32_t)eb);
  const uint32_t phi = (uint32_t)__builtin_amdgcn_ds_permute(a4, (int)(uint32_t)(eb >> 32));
  const int pid = __builtin_amdgcn_ds_permute(a4, id);
  const bool in = lane < nk;
  const double es = in ? __longlong_as_double((long long)(((uint64_t)phi << 32) | plo)) : 0.0;
  const int ids = in ? pid : 0;
  const double acc = wave_scan_f64(es);
  const double r = u * readlane_f64(acc, kWave - 1);
  const uint64_t hit = __ballot(in && es > 0.0 && acc >= r);
  if (r > 0.0 && hit) {
    const int f = __ffsll((unsigned long long)hit) - 1;
    const double af = readlane_f64(acc, f), pf = af - readlane_f64(es, f);
    if ((af - r > eps * af) && (r - pf > eps * r)) {
      exact = 0;
      return (int)readlane_u32((uint32_t)ids, f);
    }
  }
  if (!replay) return -1;
  // text2semantic.cpp:152-164 sequentially in id order
  exact = 1;
  double total = 0.0;
  for (int j = 0; j < nk; ++j) total += readlane_f64(es, j);
  const double rr = u * total;
  if (rr <= 0.0) return 0;
  double run = 0.0;
  for (int j = 0; j < nk; ++j) {
    const double ej = readlane_f64(es, j);
    run += ej;
    if (ej > 0.0 && rr <= run) return (int)readlane_u32((uint32_t)ids, j);
  }
  return V - 1;
}

}  // namespace
}  // namespace c4s
