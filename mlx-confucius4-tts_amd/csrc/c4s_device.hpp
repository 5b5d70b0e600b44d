// Device primitives for the gfx950 token-sampling kernels: order-preserving
// float keys, the xorshift64 step, and wave64 / workgroup reductions and scans.
//
// Everything here is written for CDNA wave64: a workgroup of NT threads is
// NT/64 waves, wave-level steps use cross-lane shuffles, workgroup-level steps
// combine one value per wave through LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Phase marker for cycle accounting. Expands to nothing here; an instrumented
// build may define it before including this header.
#ifndef C4S_PHASE
#define C4S_PHASE(n) ((void)0)
#endif
#ifndef C4S_PHASE_IF
#define C4S_PHASE_IF(cond, n) ((void)0)
#endif
#ifndef C4S_PHASE_VAL
#define C4S_PHASE_VAL(n, v) ((void)0)
#endif
#ifndef C4S_SCAN_PHASE
#define C4S_SCAN_PHASE(n) ((void)0)
#endif
#ifndef C4S_LIST_PHASE
#define C4S_LIST_PHASE(n) ((void)0)
#endif
#ifndef C4S_HELPER_PHASE
#define C4S_HELPER_PHASE(n) ((void)0)
#endif
#ifndef C4S_ROW_TIME
#define C4S_ROW_TIME(n) ((void)0)
#endif
#ifndef C4S_SPEC_T
#define C4S_SPEC_T(n) ((void)0)
#define C4S_SPEC_DECL ((void)0)
#define C4S_SPEC_END(w) ((void)0)
#define C4S_SPEC_EV(step, ev) ((void)0)
#endif

namespace c4s {

constexpr int kWave = 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / kWave; }

// Order-preserving map float -> uint32 (a < b as floats <=> key(a) < key(b)),
// with -0.0 folded onto +0.0 because the reference compares with `<`, under
// which the two are equal. NaN is outside the input contract.
__device__ __forceinline__ uint32_t fkey(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float kfloat(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

constexpr uint32_t kKeyNegInf = 0x007fffffu;  // fkey(-inf)

// Reference RNG step, src/t2s/text2semantic.cpp:158.
__device__ __forceinline__ uint64_t xorshift64(uint64_t s) {
  s ^= s << 13;
  s ^= s >> 7;
  s ^= s << 17;
  return s;
}

// Uniform in [0,1) from the top 53 bits, as text2semantic.cpp:159 forms it.
__device__ __forceinline__ double unit_from_state(uint64_t s) {
  return static_cast<double>(s >> 11) / static_cast<double>(1ull << 53);
}

// ---- wave64 reductions ------------------------------------------------------
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, o, kWave));
  return v;
}
__device__ __forceinline__ int wave_min_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, kWave));
  return v;
}

// (value, index) pair: larger value wins, equal values -> smaller index
// (std::max_element keeps the first maximum).
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o, kWave);
    const int oi = __shfl_xor(i, o, kWave);
    argmax_merge(v, i, ov, oi);
  }
}

// Inclusive prefix sums across the wave (lane order).
__device__ __forceinline__ double wave_incl_scan_f64(double v) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const double t = __shfl_up(v, o, kWave);
    if (l >= o) v += t;
  }
  return v;
}
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t t = (uint32_t)__shfl_up((int)v, o, kWave);
    if (l >= o) v += t;
  }
  return v;
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// ---- DPP (data-parallel primitives, no LDS traffic) ------------------------------
// gfx9 DPP controls: row_shr:n = 0x110+n (lane i reads lane i-n of its 16-lane
// row), row_bcast:15 = 0x142 (lane 15 of row r-1 to row r), row_bcast:31 =
// 0x143 (lane 31 to rows 2 and 3). Lanes without a source read `fill`.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v, uint32_t fill) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)fill, (int)v, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_f64(double v, double fill) {
  const uint64_t b = __double_as_longlong(v), f = __double_as_longlong(fill);
  const uint32_t lo = dpp_u32<CTRL, ROW_MASK>((uint32_t)b, (uint32_t)f);
  const uint32_t hi = dpp_u32<CTRL, ROW_MASK>((uint32_t)(b >> 32), (uint32_t)(f >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Lane i's value from lane i - 1 across the whole wave (wave_shr:1 = 0x138,
// a gfx9 DPP control), `fill` in lane 0: the exclusive prefix from an
// inclusive one without the LDS crossbar.
__device__ __forceinline__ double wave_shr1_f64(double v, double fill) { return dpp_f64<0x138>(v, fill); }

// Lane i's value from lane i ^ J. J = 1, 2: quad permutes; J = 4, 8: row shifts
// by J inside the lane's 16-lane row (lane i reads i + J where bit J of i is
// clear, i - J where it is set); wider: a cross-lane permute through LDS.
template <int J>
__device__ __forceinline__ uint32_t xor_lane_u32(uint32_t v) {
  if constexpr (J == 1) {
    return dpp_u32<0xB1>(v, v);   // quad_perm [1, 0, 3, 2]
  } else if constexpr (J == 2) {
    return dpp_u32<0x4E>(v, v);   // quad_perm [2, 3, 0, 1]
  } else if constexpr (J == 4 || J == 8) {
    const uint32_t up = dpp_u32<0x100 + J>(v, v), dn = dpp_u32<0x110 + J>(v, v);
    return (lane_id() & J) ? dn : up;
  } else {
    return (uint32_t)__shfl_xor((int)v, J, kWave);
  }
}
template <int J>
__device__ __forceinline__ uint64_t xor_lane_u64(uint64_t v) {
  return ((uint64_t)xor_lane_u32<J>((uint32_t)(v >> 32)) << 32) | xor_lane_u32<J>((uint32_t)v);
}

// fl32(x / d) for floats x and d, given r = fl64(1 / d): fl32(fl64(x * r)).
// Exact for every x (+-0 and +-inf included): fl64(x * r) lies within
// 2^-52 (1 + 2^-54) relative of x / d, while a quotient of two floats lies
// farther than 2^-49 relative from every float and every midpoint between
// floats that it does not equal (x - d M is a nonzero integer multiple of
// 2^min(e_x, e_d + e_M), so |x / d - M| >= 2^e_M / 2^24 for a midpoint M of
// 25-bit odd significand, normal or subnormal), so both round to one float.
// One multiply and two conversions instead of the IEEE divide's ten steps.
__device__ __forceinline__ float div_rcp(float x, double r) { return (float)((double)x * r); }

// x_{i+1} = fl(x_i + q) for i < m (q > 0 and x_0 > 0 finite, below 2^53):
// the final x_m and the number of i <= m with x_i <= thr (a prefix: x does
// not decrease). Stepping a binade at a time: with x = C ulp (C in [2^52,
// 2^53), ulp of x's binade) and q = Q ulp + r (0 <= r < ulp), every add that
// stays in the binade adds exactly D ulp, D = Q + (r > ulp / 2) (r = ulp / 2,
// a tie resolved by parity, and the add that leaves the binade are taken one
// at a time), so C grows by D per step while C + D < 2^53. Every count is an
// integer below 2^53, held in a double (exact; the GPU has no 64-bit integer
// divide, and double arithmetic beats emulated 64-bit integers).
// floor(a / b) for integers 0 <= a < 2^53 and 0 < b < 2^53 held in doubles:
// the rounded quotient lies within 1 of a / b and not below floor(a / b) (an
// integer below 2^53, representable), so it is floor(a / b) or one more, and
// the remainder a - s b, an integer of magnitude below b, is exact in one fma.
__host__ __device__ __forceinline__ double floor_div(double a, double b) {
  double s = floor(a / b);
  if (fma(-s, b, a) < 0.0) s -= 1.0;
  return s;
}
struct RepAdd {
  double x;
  int le;
};
__host__ __device__ __noinline__ inline RepAdd repeat_add(double x, double q, int m, double thr, bool need_x) {
  int i = 0, le = 0;
  bool counting = true;
  while (true) {
    if (counting) {
      if (x <= thr) le = i + 1;
      else counting = false;
    }
    if (i == m || (!counting && !need_x)) break;
    const int ex = ilogb(x) + 1;   // x in [2^(ex-1), 2^ex) (no address-taken local: frexp's would live in scratch)
    const double ulp = ldexp(1.0, ex - 53);
    const double Qd = floor(ldexp(q, 53 - ex));   // q / ulp (scalings by powers of 2 are exact)
    const double r = q - Qd * ulp;   // exact: the bits of q below ulp
    if (r == 0.5 * ulp || Qd >= 0x1p52) {
      x = x + q;
      ++i;
      continue;
    }
    const double D = Qd + (r > 0.5 * ulp ? 1.0 : 0.0);
    if (D == 0.0) {   // every add rounds back to x
      if (counting) le = m + 1;
      break;
    }
    const double C = ldexp(x, 53 - ex);   // an integer in [2^52, 2^53)
    double sb = floor_div(0x1p53 - 1.0 - C, D);   // adds that keep C below 2^53
    if (sb > (double)(m - i)) sb = (double)(m - i);
    if (counting) {
      // x_k <= thr iff C_k <= T = floor(thr / ulp) (T >= C here); the binade's
      // adds all stay at or below thr when T - C >= sb D
      const double T = floor(ldexp(thr, 53 - ex));
      if (T - C < sb * D) {   // T - C below 2^53
        const double st = floor_div(T - C, D);
        le = i + (int)st + 1;
        counting = false;
        if (!need_x) break;
      } else {
        le = i + (int)sb + 1;
      }
    }
    x = (C + sb * D) * ulp;   // exact: below 2^53 units of ulp
    i += (int)sb;
    if (i == m) break;
    x = x + q;   // the add that leaves the binade
    ++i;
  }
  return RepAdd{x, le};
}

// Inclusive scans in lane order (Hillis-Steele inside 16-lane rows, then the
// row totals through row_bcast:15 / row_bcast:31).
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t v) {
  v += dpp_u32<0x111>(v, 0u);
  v += dpp_u32<0x112>(v, 0u);
  v += dpp_u32<0x114>(v, 0u);
  v += dpp_u32<0x118>(v, 0u);
  v += dpp_u32<0x142, 0xA>(v, 0u);
  v += dpp_u32<0x143, 0xC>(v, 0u);
  return v;
}
__device__ __forceinline__ double wave_scan_f64(double v) {
  v += dpp_f64<0x111>(v, 0.0);
  v += dpp_f64<0x112>(v, 0.0);
  v += dpp_f64<0x114>(v, 0.0);
  v += dpp_f64<0x118>(v, 0.0);
  v += dpp_f64<0x142, 0xA>(v, 0.0);
  v += dpp_f64<0x143, 0xC>(v, 0.0);
  return v;
}
// Max over the wave, valid in lane 63 after the scan pattern; broadcast.
__device__ __forceinline__ float wave_max_dpp(float v) {
  uint32_t u = __float_as_uint(v);
  v = fmaxf(v, __uint_as_float(dpp_u32<0x111>(u, u))); u = __float_as_uint(v);
  v = fmaxf(v, __uint_as_float(dpp_u32<0x112>(u, u))); u = __float_as_uint(v);
  v = fmaxf(v, __uint_as_float(dpp_u32<0x114>(u, u))); u = __float_as_uint(v);
  v = fmaxf(v, __uint_as_float(dpp_u32<0x118>(u, u))); u = __float_as_uint(v);
  v = fmaxf(v, __uint_as_float(dpp_u32<0x142, 0xA>(u, u))); u = __float_as_uint(v);
  v = fmaxf(v, __uint_as_float(dpp_u32<0x143, 0xC>(u, u)));
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 63));
}
__device__ __forceinline__ uint32_t wave_max_u32_dpp(uint32_t v) {
  v = max(v, dpp_u32<0x111>(v, v));
  v = max(v, dpp_u32<0x112>(v, v));
  v = max(v, dpp_u32<0x114>(v, v));
  v = max(v, dpp_u32<0x118>(v, v));
  v = max(v, dpp_u32<0x142, 0xA>(v, v));
  v = max(v, dpp_u32<0x143, 0xC>(v, v));
  return __builtin_amdgcn_readlane(v, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32_dpp(uint32_t v) {
  v = min(v, dpp_u32<0x111>(v, v));
  v = min(v, dpp_u32<0x112>(v, v));
  v = min(v, dpp_u32<0x114>(v, v));
  v = min(v, dpp_u32<0x118>(v, v));
  v = min(v, dpp_u32<0x142, 0xA>(v, v));
  v = min(v, dpp_u32<0x143, 0xC>(v, v));
  return __builtin_amdgcn_readlane(v, 63);
}
// Max of 64-bit keys over the wave (the same pattern on (hi, lo) pairs).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint64_t dpp_max_u64_step(uint64_t v) {
  const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  const uint32_t olo = dpp_u32<CTRL, ROW_MASK>(lo, lo), ohi = dpp_u32<CTRL, ROW_MASK>(hi, hi);
  const uint64_t o = ((uint64_t)ohi << 32) | olo;
  return o > v ? o : v;
}
__device__ __forceinline__ uint64_t wave_max_u64_dpp(uint64_t v) {
  v = dpp_max_u64_step<0x111>(v);
  v = dpp_max_u64_step<0x112>(v);
  v = dpp_max_u64_step<0x114>(v);
  v = dpp_max_u64_step<0x118>(v);
  v = dpp_max_u64_step<0x142, 0xA>(v);
  v = dpp_max_u64_step<0x143, 0xC>(v);
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), 63);
  return ((uint64_t)hi << 32) | lo;
}
// Lane i receives lane i + 1 (wave_shl:1); lane 63 receives `fill`.
__device__ __forceinline__ uint32_t wave_next_u32(uint32_t v, uint32_t fill) {
  return dpp_u32<0x130>(v, fill);
}
__device__ __forceinline__ double wave_sum_dpp(double v) {
  v = wave_scan_f64(v);
  const uint64_t b = __double_as_longlong(v);
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)b, 63);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(b >> 32), 63);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int l) {
  return __builtin_amdgcn_readlane(v, l);
}
__device__ __forceinline__ float readlane_f32(float v, int l) {
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), l));
}
__device__ __forceinline__ double readlane_f64(double v, int l) {
  const uint64_t b = __double_as_longlong(v);
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)b, l);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(b >> 32), l);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// Sequential double sums over the lanes (the reference's loops add one term
// after the other): the lane index is a scalar loop counter, so each term
// costs two scalar reads and the dependent chain is the adds alone. The loops
// stay rolled: unrolled over 64 lanes they raised the scalar register pressure
// of the kernels that inline them into spills (a 1024-thread kernel into
// scratch, 2.7x its time).
// seq_sum_lanes: total + e[0] + e[1] + ... + e[n-1] in that order (n <= 64,
// wave-uniform).
__device__ __forceinline__ double seq_sum_lanes(double total, double e, int n) {
#pragma unroll 1
  for (int t = 0; t < n; ++t) total += readlane_f64(e, t);
  return total;
}
// seq_find_lanes: the same running sum continued from acc; returns the first
// t < n after whose term r <= acc (acc then the sum through t), else -1 (acc
// the sum of all n terms).
__device__ __forceinline__ int seq_find_lanes(double& acc, double e, int n, double r) {
#pragma unroll 1
  for (int t = 0; t < n; ++t) {
    acc += readlane_f64(e, t);
    if (r <= acc) return t;
  }
  return -1;
}
// seq_sum_mem / seq_cut_mem: the same over n terms in memory (LDS or global),
// every lane reading the same addresses and computing the same sum, 16 terms
// loaded at a time, so the chain is plain FP64 adds on vector registers.
__device__ __forceinline__ double seq_sum_mem(double total, const double* p, int n) {
  for (int j = 0; j < n; j += 16) {
    double v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = p[min(j + i, n - 1)];
#pragma unroll
    for (int i = 0; i < 16; ++i) total += (j + i < n) ? v[i] : 0.0;   // + 0.0 leaves a sum >= 0 unchanged
  }
  return total;
}
// top_p's removal loop over n terms from cum: returns how many leading terms
// leave cum <= thr; sets stop (and cum to the sum through the first term past
// thr) when one takes it above.
__device__ __forceinline__ int seq_cut_mem(double& cum, const double* p, int n, double thr, bool& stop) {
  for (int j = 0; j < n; j += 16) {
    double v[16], cs[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = p[min(j + i, n - 1)];
    double x = cum;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      x += (j + i < n) ? v[i] : 0.0;
      cs[i] = x;
    }
    int first = 16;
#pragma unroll
    for (int i = 15; i >= 0; --i)
      if (j + i < n && !(cs[i] <= thr)) first = i;
    if (first < 16) {
      stop = true;
      cum = cs[first];
      return j + first;
    }
    cum = x;
  }
  return n;
}
// seq_sum_blk / seq_cut_blk: seq_sum_mem / seq_cut_mem over terms padded with
// +0.0 to a multiple of 32, for callers whose n is uniform: blocks of 32 terms
// need no bounds, so the loop is 32 loads (the adds start as the first ones
// arrive) and 32 dependent FP64 adds. An added +0.0 leaves a sum >= 0
// unchanged and never takes cum above thr. The terms are >= 0, so cum only
// grows: a block whose last sum is <= thr has every sum <= thr, and only the
// block that ends above thr is added again, term by term, to find the first.
__device__ __forceinline__ double seq_sum_blk(double total, const double* p, int n) {
  n = __builtin_amdgcn_readfirstlane(n);
#pragma unroll 1
  for (int j = 0; j < n; j += 32) {
    double v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = p[j + i];
#pragma unroll
    for (int i = 0; i < 32; ++i) total += v[i];
  }
  return total;
}
__device__ __forceinline__ int seq_cut_blk(double& cum, const double* p, int n, double thr, bool& stop) {
  n = __builtin_amdgcn_readfirstlane(n);
  double x = cum;
#pragma unroll 1
  for (int j = 0; j < n; j += 32) {
    double v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) v[i] = p[j + i];
    double y = x;
#pragma unroll
    for (int i = 0; i < 32; ++i) y += v[i];
    if (__builtin_amdgcn_readfirstlane(y <= thr ? 0 : 1)) {   // every lane holds the same sums
      int i = 0;
      x += p[j];
#pragma unroll 1
      while (i < 31 && x <= thr) x += p[j + ++i];
      stop = true;
      cum = x;
      return j + i;
    }
    x = y;
  }
  cum = x;
  return n;
}
// seq_cut_lanes: top_p's removal loop (sampling.cpp:60-65) over n terms from
// cum: the number of leading terms after which cum <= thr still holds; sets
// stop when a term took cum above thr (cum only grows).
__device__ __forceinline__ int seq_cut_lanes(double& cum, double q, int n, double thr, bool& stop) {
#pragma unroll 1
  for (int t = 0; t < n; ++t) {
    cum += readlane_f64(q, t);
    if (!(cum <= thr)) {
      stop = true;
      return t;
    }
  }
  return n;
}

// ---- workgroup reductions ------------------------------------------------------
// `red` is LDS scratch with room for one entry per wave (typed views of the same
// bytes are fine). Every thread returns the result. Two barriers: the trailing
// one lets the caller reuse `red` immediately.
template <int NT>
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = wave_sum_f64(v);
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  double r = 0.0;
#pragma unroll
  for (int w = 0; w < NT / kWave; ++w) r += red[w];
  __syncthreads();
  return r;
}

template <int NT>
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* red) {
  v = wave_sum_u32(v);
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  uint32_t r = 0;
#pragma unroll
  for (int w = 0; w < NT / kWave; ++w) r += red[w];
  __syncthreads();
  return r;
}

template <int NT>
__device__ __forceinline__ float block_max_f32(float v, float* red) {
  v = wave_max_f32(v);
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < NT / kWave; ++w) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}

template <int NT>
__device__ __forceinline__ int block_min_i32(int v, int* red) {
  v = wave_min_i32(v);
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  int r = red[0];
#pragma unroll
  for (int w = 1; w < NT / kWave; ++w) r = min(r, red[w]);
  __syncthreads();
  return r;
}

template <int NT>
__device__ __forceinline__ void block_argmax(float& v, int& i, float* redv, int* redi) {
  wave_argmax(v, i);
  if (lane_id() == 0) { redv[wave_id()] = v; redi[wave_id()] = i; }
  __syncthreads();
  v = redv[0];
  i = redi[0];
#pragma unroll
  for (int w = 1; w < NT / kWave; ++w) argmax_merge(v, i, redv[w], redi[w]);
  __syncthreads();
}

}  // namespace c4s
