// gfx950 kernels for the c4tts Text2Semantic token-sampling path.
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


#include "c4s_list.hpp"
#include "c4s_step.hpp"

namespace c4s {
namespace {

// ---- kernels -------------------------------------------------------------------

// The drawn token joins the row's kept history set unless it is the stop token
// (text2semantic.cpp:333-334: a finished row appends nothing).
__device__ __forceinline__ void join_history(const RowsArgs& a, int row, int tok) {
  if (a.hist_bits && tok >= 0 && tok < a.vocab && tok != a.stop_token)
    atomicOr(&a.hist_bits[(int64_t)row * hist_words(a.vocab) + (tok >> 5)], 1u << (tok & 31));
}

__global__ __launch_bounds__(NT) void k_rows_lds(RowsArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ Scratch sh;
  const int row = blockIdx.x;
  const int V = a.vocab;
  if (a.row_active && !a.row_active[row]) {
    if (threadIdx.x == 0) a.out_tok[row] = -1;
    return;
  }
  const RowCfg c = make_cfg(a.mode, V, row, a.temp, a.top_k, a.top_p, a.pen, a.min_keep,
                            a.do_sample);
  LdsLayout L = lds_layout(smem, V);
  const int64_t roff = (int64_t)row * a.ld;
  if (a.dtype == 0) {
    RowFetch f;
    const float* p = static_cast<const float*>(a.logits) + roff;
    fetch_row(p, V, f);
    L.val = store_row(p, V, f, L.val);
  } else {
    for (int i = threadIdx.x; i < V; i += NT) L.val[i] = load_logit(a.logits, a.dtype, roff + i);
  }
  if (c.pen_on) {
    const int nw = bitmap_words(V);
    if (a.hist_bits) {   // the history set kept across steps
      const uint32_t* hb = a.hist_bits + (int64_t)row * hist_words(V);
      for (int w = threadIdx.x; w < nw; w += NT) L.bitmap[w] = w < hist_words(V) ? hb[w] : 0u;
    } else {
      for (int w = threadIdx.x; w < nw; w += NT) L.bitmap[w] = 0u;
      __syncthreads();
      const int64_t h0 = a.hist_off[row], h1 = a.hist_off[row + 1];
      for (int64_t j = h0 + threadIdx.x; j < h1; j += NT) {
        const int id = a.hist_ids[j];
        if (id < 0 || id >= V) continue;   // sampling.cpp:24
        atomicOr(&L.bitmap[id >> 5], 1u << (id & 31));
      }
    }
    __syncthreads();
    penalise_chunk(L.val, L.bitmap, V, c.pen);
  }
  __syncthreads();
  LdsRow src{L.val, L.E, V, 0u, false};
  uint64_t rng = a.rng ? a.rng[row] : 0ull;
  float* masked = a.out_masked ? a.out_masked + (int64_t)row * V : nullptr;
  uint32_t* st = a.stats ? a.stats + 4 * (int64_t)row : nullptr;
  int tok = 0;
  if (!(fast_topk_applies(c, V) &&
        fast_topk_any(L.val, V, c, sh, reinterpret_cast<unsigned char*>(L.E), rng, tok, masked, st)))
    tok = run_chain(src, sh, c, rng, masked, st);
  if (threadIdx.x == 0) {
    a.out_tok[row] = tok;
    if (c.draw && a.rng) a.rng[row] = rng;
    join_history(a, row, tok);
  }
}

// Writes one row's result: token, RNG state, history set (text2semantic.cpp:
// 333-334: the stop token does not join), statistics.
__device__ __forceinline__ void step_out(const StepIO& io, int V, int tok, uint64_t rng, bool draw,
                                         uint32_t s0, uint32_t s1, uint32_t s2, uint32_t s3) {
  *io.out_tok = tok;
  if (draw && io.rng) *io.rng = rng;
  if (io.join && tok >= 0 && tok < V && tok != io.stop_token) atomicOr(&io.join[tok >> 5], 1u << (tok & 31));
  if (io.stats) { io.stats[0] = s0; io.stats[1] = s1; io.stats[2] = s2; io.stats[3] = s3; }
}

// The draw of the one-pass step (text2semantic.cpp:150-165) once the kept set
// is known: the kept fp32 masses of each thread and ds, the workgroup scan of
// their sums with the error bound in tot2. The thread whose interval holds r
// decides. When it cannot (r within the bound of one end of its entry: on a
// flat row of thousands of kept entries a few percent of rows a call), the
// masses are taken again in double: at most 64 kept ids go in id order (kl, by
// the scan's kept counts) to one wave, which draws on them and replays the
// sums sequentially if that is too close (lane_draw); otherwise every thread
// recomputes its kept masses, the workgroup scans them (bound rel_eps, about
// 1e-11 relative) and the owner's wave walks the owner's ids, one a lane; only
// if that still does not decide does one wave replay the draw sequentially
// over the row (draw_replay).
// The row's configuration and I/O as one LDS copy for the workgroup: the
// out-of-line helpers take them by reference, and a reference to a copy in
// registers would make the compiler keep that copy in per-lane scratch memory
// for the whole kernel (about 120 bytes a lane written at entry).
struct StepRowSh {
  RowCfg cfg;
  StepIO io;
  uint32_t tp_exact_first;   // 1: the one pass's top_p test missed its margin in double
};

template <int PT, bool kCached>
__device__ __forceinline__ void draw_finish(const StepIO& io, const RowCfg& c, const KeptRule& kr, const float (&z)[PT],
                                            int lo, int n, float m, const Scan2& ds, uint32_t n_kept,
                                            uint32_t st_path, uint32_t st_exact, StepSh& ss, const StepRowSh& rs,
                                            const float* em, uint64_t* kl) {
  const int t = threadIdx.x;
  const uint64_t st2 = xorshift64(*io.rng);
  const double u = unit_from_state(st2);
  const double K = ds.tot;
  const double r = u * K;
  const double margin = 2.0 * ds.tot2 + rel_eps(c.V) * K;
  if (!(r > 0.0)) {   // r == 0: the first id satisfies r <= acc (text2semantic.cpp:161-162)
    if (t == 0) step_out(io, c.V, 0, st2, true, st_path, st_exact, 0u, n_kept);
    return;
  }
  const bool owner = (ds.ex < r && r <= ds.in) || (t == kStepThreads - 1 && r > ds.in);
  int found = -1;
  bool certain = false;
  C4S_PHASE_IF(owner, 18);
  const uint64_t obw = __ballot(owner);
  if (obw) {
    // the owner's wave: lane j takes the owner's id lo + j and its kept fp32
    // mass (independent loads and tests, one a lane), the running sums in id
    // order by a wave scan in double from the owner's exclusive prefix (its
    // rounding, about 2^-53 relative a step, lies far inside the margin), then
    // the first kept id whose sum reaches r and the sums on both sides of it
    const int ol = __ffsll((unsigned long long)obw) - 1, l = lane_id();
    float zl = neg_inf();
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const float zj = readlane_f32(z[j], ol);
      zl = (l == j) ? zj : zl;
    }
    const int lo_o = (int)readlane_u32((uint32_t)lo, ol);
    const double ex_o = readlane_f64(ds.ex, ol);
    float el;   // lanes past the owner's ids hold -inf: not kept
    if constexpr (kCached) {
      const float ec = em[min(lo_o + l, c.V - 1)];
      el = ((int)(zl != neg_inf()) & (int)kept_in(kr, zl, m, lo_o + l)) ? ec : 0.0f;
    } else {
      bool kp;
      el = kept_mass32(kr, zl, m, lo_o + l, kp);
    }
    const double al = ex_o + wave_scan_f64((double)el);
    const uint64_t hit = __ballot(el > 0.0f && al >= r);
    if (hit) {
      const int f = __ffsll((unsigned long long)hit) - 1;
      const double af = readlane_f64(al, f);
      const double pf = f > 0 ? readlane_f64(al, max(f - 1, 0)) : ex_o;
      found = lo_o + f;
      certain = (af - r > margin) && (r - pf > margin);
    }
  }
  C4S_PHASE_IF(owner, 19);
  if (!__syncthreads_or(owner && !certain)) {
    if (owner) step_out(io, c.V, found, st2, true, st_path, st_exact, 0u, n_kept);
    return;
  }
  // the kept masses in double. The kept test is the one pass's (kept_in): a
  // dense row reaches this draw only without values whose double mass lies
  // near underflow, so `z - m > -745` there is exactly `exp((double)(z - m)) > 0`.
  C4S_PHASE(24);
  if (n_kept <= (uint32_t)kWave) {
    // at most 64 kept ids: in id order (thread order, then the thread's own)
    // to one wave, which draws on them in double and replays the sums
    // sequentially when that is too close (lane_draw)
    uint32_t km = 0;
#pragma unroll
    for (int j = 0; j < PT; ++j)
      km |= ((int)(j < n) & (int)(z[j] != neg_inf()) & (int)kept_in(kr, z[j], m, lo + j)) ? 1u << j : 0u;
#pragma unroll
    for (int j = 0; j < PT; ++j)
      if ((km >> j) & 1u)
        kl[ds.uex + (uint32_t)__popc(km & ((1u << j) - 1u))] = ((uint64_t)__float_as_uint(z[j]) << 32) | (uint32_t)(lo + j);
    __syncthreads();
    if (wave_id() == 0) {
      const int l = lane_id();
      const bool in = l < (int)n_kept;
      const uint64_t ent = kl[in ? l : 0];
      const double e = in ? exp((double)(__uint_as_float((uint32_t)(ent >> 32)) - m)) : 0.0;
      uint32_t ex2 = 0;
      const int tk = lane_draw<6>(in, (int)(uint32_t)ent, l, e, u, c.V, ex2);
      if (l == 0) step_out(io, c.V, tk, st2, true, st_path, st_exact, 1u + ex2, n_kept);
    }
    return;
  }
  double dk = 0.0;
#pragma unroll
  for (int j = 0; j < PT; ++j)
    if (j < n && z[j] != neg_inf() && kept_in(kr, z[j], m, lo + j)) dk += exp((double)(z[j] - m));
  const Scan2 d2 = block_scan2(dk, 0.0, 0u, ss.wa, ss.wb, ss.wu);
  C4S_PHASE(25);
  const double r2 = u * d2.tot;
  const double m2 = 2.0 * rel_eps(c.V) * d2.tot;
  const bool own2 = (d2.ex < r2 && r2 <= d2.in) || (t == kStepThreads - 1 && r2 > d2.in);
  found = -1;
  certain = false;
  const uint64_t ob = __ballot(own2);
  if (ob) {   // the owner's wave: lane j takes the owner's id lo + j, the prefix by a wave scan
    const int ol = __ffsll((unsigned long long)ob) - 1, l = lane_id();
    float zl = neg_inf();
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const float zj = readlane_f32(z[j], ol);
      zl = (l == j) ? zj : zl;
    }
    const int lo_o = readlane_u32((uint32_t)lo, ol), n_o = readlane_u32((uint32_t)n, ol);
    const double ex_o = readlane_f64(d2.ex, ol);
    const bool kp = ((int)(l < n_o) & (int)(zl != neg_inf()) & (int)kept_in(kr, zl, m, lo_o + l)) != 0;
    const double el = kp ? exp((double)(zl - m)) : 0.0;
    const double al = ex_o + wave_scan_f64(el);
    const uint64_t hit = __ballot(el > 0.0 && al >= r2);
    if (r2 > 0.0 && hit) {
      const int f = __ffsll((unsigned long long)hit) - 1;
      const double af = readlane_f64(al, f), pf = af - readlane_f64(el, f);
      found = lo_o + f;
      certain = (af - r2 > m2) && (r2 - pf > m2);
    }
  }
  C4S_PHASE(26);
  if (!__syncthreads_or(own2 && !certain)) {
    if (own2) step_out(io, c.V, found, st2, true, st_path, st_exact, 1u, n_kept);
    return;
  }
  if (wave_id() == 0) {   // the reference's sequential sums, one wave
    const int tk = draw_replay(rs.io, rs.cfg, kr, m, u);
    if (lane_id() == 0) step_out(io, c.V, tk, st2, true, st_path, st_exact, 2u, n_kept);
  }
}

// sampling.cpp:52-65 replayed for a row whose top group X (nX entries at the
// maximum, mass 1 each) is preceded in ascending order by entries of total
// mass B (known within relative `re` of the reference's sequential sum):
// total = B + 1 + ... + 1 and cum = sum of prob / total, both sequential. The
// sums over the entries below X reach the sequence only through B and B /
// total; each enters one add (B + 1, then B / total + 1 / total), which rounds
// every value of its interval to one double, or the replay gives up (-1).
// Returns the members of X kept (cum > thr), the rest removed in order.
__device__ __forceinline__ int tie_top_exact(double B, int nX, double thr, double re) {
  const double t_lo = B * (1.0 - 2.0 * re) + 1.0, t_hi = B * (1.0 + 2.0 * re) + 1.0;
  if (t_lo != t_hi) return -1;
  const double tot = repeat_add(t_lo, 1.0, nX - 1, -1.0, true).x;
  const double q = 1.0 / tot;
  const double cb = B / tot, cb_hi = cb * (1.0 + 3.0 * re);
  if (!(cb_hi <= thr)) return -1;   // some entry below X could be kept
  const double c_lo = cb * (1.0 - 3.0 * re) + q, c_hi = cb_hi + q;
  if (c_lo != c_hi) return -1;
  return nX - repeat_add(c_lo, q, nX - 1, thr, false).le;
}

// The cut when the boundary entries X (more than one sort takes) all hold one
// value z*: each has the mass e = exp(z* - m), and in the chain's order (value
// descending, lower id first) X is ordered by id, which is thread order here,
// so a member's rank is a prefix count. Member i is kept iff the mass at or
// below it, M_i = S - (mass above X) - i e, exceeds thr S (sampling.cpp:60-65;
// top_k rows: every member survives top_k, S = the survivors' mass); kept
// members are ranks 0 .. k-1. A decision within the margin is taken again with
// S and the mass above X summed in double, and, when X holds the maximum, by
// replaying the reference's sums over X (tie_top_exact). Sets ss.kthr;
// returns 1 decided, 3 decided with the double sums or the replay, 4 neither
// settles it (the multi-pass chain decides, by the exact emulation), 0 the
// multi-pass chain decides (X holds more than one value; top-k rows;
// min_tokens_to_keep).
template <int PT>
__device__ __noinline__ int tie_cut(const RowCfg& c, const float* val, int lo, int n, const SideRule sr, int nX,
                                    double thr, double S, double errS, double Ma, double eMa, uint32_t n_above,
                                    StepSh& ss) {
  const int lane = lane_id(), w = wave_id();
  const float ninf = neg_inf();
  const bool topk = c.topk_on;
  // z = fl(y / T) by the exact reciprocal division; every read unconditional
  // (index clamped); the loops rolled (code size: this path is rare)
  const double rt = 1.0 / (double)c.temp;
  float zmax = ninf, zmin = -ninf;
  uint32_t cnt = 0;
#pragma unroll 1
  for (int j = 0; j < PT; ++j) {
    const float y = val[min(lo + j, c.V - 1)];
    const float z = c.temp_on ? div_rcp(y, rt) : y;
    const bool inx = ((int)(j < n) & (int)(sr.side(z) == 0)) != 0;
    zmax = inx ? fmaxf(zmax, z) : zmax;
    zmin = inx ? fminf(zmin, z) : zmin;
    cnt += inx ? 1u : 0u;
  }
  zmax = wave_max_dpp(zmax);
  zmin = -wave_max_dpp(-zmin);
  if (lane == 0) { ss.wmax[w] = zmax; ss.wmin[w] = zmin; }
  const Scan2 rk = block_scan2((double)cnt, 0.0, 0u, ss.we, ss.wf, ss.ww);   // includes a barrier
  float zs = ninf, zl = -ninf;
#pragma unroll
  for (int i = 0; i < kStepWaves; ++i) { zs = fmaxf(zs, ss.wmax[i]); zl = fminf(zl, ss.wmin[i]); }
  if (!(zs == zl) || zs == ninf) return 0;   // not one value (or nothing finite)
  C4S_PHASE(24);
  const double e = exp((double)(zs - sr.m));
  const double N = (double)nX;
  const uint32_t mk = (uint32_t)max(0, c.min_keep);
  double Sx = topk ? N * e : S, base = topk ? 0.0 : Ma, err = topk ? 0.0 : 2.0 * errS + eMa;
  double nB = 0.0;   // the mass below X, in double (pass 1)
  int k = 0, verdict = 1;
  for (int pass = 0; pass < 2; ++pass) {
    if (thr <= 0.0) {   // p >= 1: only zero-mass positions can go
      k = (thr < 0.0 || e > 0.0) ? nX : 0;
      break;
    }
    const double A = thr * Sx;
    // k = the members with M_i > A, M_i = Sx - base - i e decreasing in i
    const double q = (Sx - base - A) / e;
    k = q <= 0.0 ? 0 : (q >= N ? nX : (int)ceil(q));
    while (k > 0 && !(Sx - base - (double)(k - 1) * e > A)) --k;
    while (k < nX && Sx - base - (double)k * e > A) ++k;
    const double mg = rel_eps(c.V) * Sx + err;
    const bool sure = (k == 0 || fabs(Sx - base - (double)(k - 1) * e - A) > mg) &&
                      (k == nX || fabs(Sx - base - (double)k * e - A) > mg);
    if (sure) break;
    if (topk) return 0;
    if (pass == 1) {
      // X holds the maximum and nothing lies above it: the reference's sums
      // in ascending order are the entries below X, then X's nX masses of 1.
      // The entries below enter only through their sums, known within
      // rel_eps, which the first add of a mass of 1 (or of 1 / total) rounds
      // to one double unless the interval straddles a rounding boundary; from
      // there the sums over X are replayed exactly.
      if (n_above != 0u || zs != sr.m) return 4;
      C4S_PHASE(25);
      if (threadIdx.x == 0) ss.bsel[0] = tie_top_exact(nB, nX, thr, rel_eps(c.V));   // one thread; the rest wait
      __syncthreads();
      k = ss.bsel[0];
      C4S_PHASE(26);
      if (k < 0) return 4;
      break;
    }
    // decide again with S and the mass above X in double (and the mass below
    // X). X holds the one value zs and side() is monotone in z, so the entries
    // above X are those above zs and the entries below X those below it; z is
    // -inf past the thread's ids (exp(-inf) = 0)
    double se = 0.0, sa = 0.0, sb = 0.0;
#pragma unroll 1
    for (int j = 0; j < PT; ++j) {
      const float y = val[min(lo + j, c.V - 1)];
      const float z = (j < n) ? (c.temp_on ? div_rcp(y, rt) : y) : ninf;
      const double ed = exp((double)(z - sr.m));
      se += ed;
      sa += z > zs ? ed : 0.0;
      sb += z < zs ? ed : 0.0;
    }
    se = wave_sum_dpp(se);
    sa = wave_sum_dpp(sa);
    sb = wave_sum_dpp(sb);
    if (lane == 0) { ss.wc[w] = se; ss.wd[w] = sa; ss.wa[w] = sb; }
    __syncthreads();
    Sx = 0.0;
    base = 0.0;
#pragma unroll
    for (int i = 0; i < kStepWaves; ++i) { Sx += ss.wc[i]; base += ss.wd[i]; nB += ss.wa[i]; }
    err = 0.0;
    verdict = 3;
  }
  // min_tokens_to_keep (sampling.cpp:67-68): the top min_keep positions stay
  if (topk) {
    if ((uint32_t)k < mk) k = (int)min(mk, (uint32_t)nX);
  } else if (n_above + (uint32_t)k < mk) {
    if (mk > n_above + (uint32_t)nX) return 0;
    k = (int)(mk - n_above);
  }
  // the last kept member's key (rank k - 1), or with none kept, one above
  // every member (the lowest id's key + 1)
  C4S_PHASE(27);
  const int want = k > 0 ? k - 1 : 0;
  const int r0 = (int)rk.ex;
  if (cnt > 0 && want >= r0 && want < r0 + (int)cnt) {
    int rank = r0;
    for (int j = 0; j < n; ++j) {
      const float y = val[lo + j];
      const float z = c.temp_on ? y / c.temp : y;
      if (sr.side(z) == 0) {
        if (rank == want) ss.kthr = key64(zs, lo + j) + (k > 0 ? 0ull : 1ull);
        ++rank;
      }
    }
  }
  __syncthreads();
  return verdict;
}

// The multi-pass chain (c4s_chain.hpp) on the penalised row staged in LDS
// (`val`), for the rows the one pass leaves; kept out of line so that its
// registers do not weigh on the one-pass path.
__device__ __noinline__ void chain_fallback(const StepIO& io, const RowCfg& c, unsigned char* work, float* val,
                                            StepScratch& sh, bool tp_exact_first) {
  const int V = c.V, t = threadIdx.x;
  uint64_t rng = *io.rng;
  LdsRow src{val, reinterpret_cast<double*>(work), V, 0u, false};
  const int tok = run_chain<kStepWaves, LdsRow, true>(src, sh, c, rng, io.masked, sh.step_stats, tp_exact_first);
  if (t == 0) {
    const uint32_t* sp = sh.step_stats;
    step_out(io, V, tok, rng, true, sp[0], sp[1], sp[2], sp[3]);
  }
}

// ---- top-k rows on a candidate list --------------------------------------------------
//
// A sampled row with top_k in [1, 64] is decided by its largest values alone
// (sampling.cpp:30-40 keeps the k largest and their ties; top_p and the draw,
// :42-71 and text2semantic.cpp:150-165, then read the kept entries only). So
// the step takes a candidate list as the AR stream's scan makes it, from the
// penalised values y each thread holds (ids [lo, lo + n), thread order is id
// order): a key L0 at or below the 112th largest of the threads' top-2 keys
// (two 11-bit histogram passes), every value with key(y) >= L0 in id order
// (one workgroup scan), the temperature on those alone (fl(y / T) is monotone
// in y), their sort by (z desc, id asc), and a bound on every value outside.
// One wave then decides the step on the first 128 entries (list_step). When
// the list cannot settle it (a boundary tie group past the list, a cut inside
// the error bound, ...), nothing has been written but the work area, and the
// row takes the one-pass step.
constexpr int kFastList = kListSmall;           // list entries the decision sees
constexpr int kFastSel = kListSmall - 16;       // thread-top keys at or above L0
constexpr int kFastCands = 256;                 // candidates the list step sorts
constexpr int kFastOneBin = 64;                 // thread-top keys from the first pass's bin up: no second pass
static_assert(kStepThreads * 4 == 2048, "four histogram bins a thread");

struct NoHit {   // no id drawn since the list was made
  __device__ __forceinline__ bool hit(int) const { return false; }
};

struct FastSh {
  uint32_t hist[2][2048];      // the two histogram passes; the first then holds the sorted head (uint64)
  uint64_t cand[kFastCands];   // candidates as entries (key of z, id, candidate position)
  uint32_t red[4][kStepWaves];   // one set per workgroup scan (no barrier between reuses)
  uint32_t redm[kStepWaves];
  uint32_t bu[8];
  LSpecCS cs;
};
static_assert(sizeof(FastSh) <= kStepWorkBytes, "the list step's area lies in the one pass's work area");
static_assert(offsetof(FastSh, hist) == 0 && sizeof(FastSh::hist) <= 3 * kHistBytes,
              "the list step's histograms lie in the area the step clears before staging");

// Exclusive scan of v over the workgroup (thread order); total in `tot`. One
// barrier: each call uses its own `red`.
__device__ __forceinline__ uint32_t fast_scan(uint32_t v, uint32_t* red, uint32_t& tot) {
  const uint32_t inc = wave_scan_u32(v);
  if (lane_id() == kWave - 1) red[wave_id()] = inc;
  __syncthreads();
  uint32_t pre = 0;
  tot = 0;
#pragma unroll
  for (int w = 0; w < kStepWaves; ++w) {
    const uint32_t x = red[w];
    pre += (w < wave_id()) ? x : 0u;
    tot += x;
  }
  return pre + inc - v;
}

// Bin of hist (2048 bins, scanned from the top) holding the m-th largest
// counted key, and the count above it, through bu[0..1] of this pick; false
// when fewer than m keys were counted.
__device__ __forceinline__ bool fast_pick(const uint32_t* hist, uint32_t* red, uint32_t* bu, uint32_t m,
                                          uint32_t& bin, uint32_t& above) {
  const int t = threadIdx.x;
  uint32_t cb[4], loc = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) { cb[i] = hist[2047 - 4 * t - i]; loc += cb[i]; }
  uint32_t total;
  const uint32_t ex = fast_scan(loc, red, total);
  if (total < m) return false;   // uniform
  if (ex < m && ex + loc >= m) {
    uint32_t run = ex;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (run < m && run + cb[i] >= m) { bu[0] = 2047 - 4 * t - i; bu[1] = run; }
      run += cb[i];
    }
  }
  __syncthreads();
  bin = bu[0];
  above = bu[1];
  return true;
}

template <int PT>
__device__ __forceinline__ bool list_fast(const StepIO& io, const RowCfg& c, int V, const float (&y)[PT], int lo,
                                          int n, const float* val, FastSh& fs) {
  const int t = threadIdx.x, lane = lane_id(), wv = wave_id();
  const double rt = 1.0 / (double)c.temp;   // used only when the temperature applies
  uint32_t ky[PT];
#pragma unroll
  for (int j = 0; j < PT; ++j) ky[j] = fkey(y[j]);
  if (n < PT) {   // the last threads: 0 past the row, below every key of a value
#pragma unroll
    for (int j = 0; j < PT; ++j) ky[j] = j < n ? ky[j] : 0u;
  }
  uint32_t t1 = 0, t2 = 0;
#pragma unroll
  for (int j = 0; j < PT; ++j) {
    t2 = max(t2, min(t1, ky[j]));
    t1 = max(t1, ky[j]);
  }
  // L0: two 11-bit passes over the threads' top-2 keys, on histograms that are
  // zero on entry (the caller clears the one-pass histogram area, which they lie in)
  C4S_PHASE(20);
  C4S_PHASE(21);
  if (t1) atomicAdd(&fs.hist[0][t1 >> 21], 1u);
  if (t2) atomicAdd(&fs.hist[0][t2 >> 21], 1u);
  __syncthreads();
  // L0 lies at or below the msel-th largest of those keys, so at least msel
  // values are candidates: for k < kFastSel the k-th largest and the next one
  const uint32_t msel = min((uint32_t)kFastSel, (uint32_t)c.k + 1u);
  uint32_t L0 = 0;
  {
    uint32_t b1, ab1;
    C4S_PHASE(22);
    if (fast_pick(fs.hist[0], fs.red[0], fs.bu, msel, b1, ab1)) {
      C4S_PHASE(23);
      if (ab1 + fs.hist[0][b1] <= (uint32_t)kFastOneBin) {
        L0 = b1 << 21;   // few keys from b1 up: its floor bounds them closely enough (uniform)
      } else {
        if (t1 && (t1 >> 21) == b1) atomicAdd(&fs.hist[1][(t1 >> 10) & 2047u], 1u);
        if (t2 && (t2 >> 21) == b1) atomicAdd(&fs.hist[1][(t2 >> 10) & 2047u], 1u);
        __syncthreads();
        uint32_t b2, ab2;
        fast_pick(fs.hist[1], fs.red[1], fs.bu + 2, msel - ab1, b2, ab2);
        L0 = (b1 << 21) | (b2 << 10);
      }
    }
  }
  L0 = max(L0, 1u);   // the same values; excludes the zero keys past the row
  C4S_PHASE(11);
  // candidates in id order; the largest key under L0 bounds everything else
  uint32_t cnt = 0, below = 0;
#pragma unroll
  for (int j = 0; j < PT; ++j) {
    cnt += (ky[j] >= L0) ? 1u : 0u;
    below = max(below, ky[j] < L0 ? ky[j] : 0u);
  }
  {
    const uint32_t bm = wave_max_u32_dpp(below);   // every lane of the workgroup is here
    if (lane == 0) fs.redm[wv] = bm;
  }
  uint32_t C;
  const uint32_t pos = fast_scan(cnt, fs.red[2], C);   // its barrier also publishes redm
  C4S_PHASE(26);
  uint32_t tout = 0;
#pragma unroll
  for (int w = 0; w < kStepWaves; ++w) tout = max(tout, fs.redm[w]);
  if (tout != 0u && c.temp_on) tout = fkey(div_rcp(kfloat(tout), rt));   // the quotient is monotone in y
  // uniform; past kFastCands the rank sort costs more than the one pass
  // (a tie group of hundreds at the k-th value, which the list cannot take anyway)
  if (C > (uint32_t)kFastCands || C == 0u) return false;
  {
    // this thread's candidates as entries: z = fl(y / T) (sampling.cpp:16), the
    // id, and the candidate's position (pos + the candidates before it), which
    // is the id order: the draw's order key
    // (the set bits only: a wave takes as many rounds as its lane with the
    // most candidates, each value read again from the row in LDS)
    uint32_t cm = 0;
#pragma unroll
    for (int j = 0; j < PT; ++j) cm |= (ky[j] >= L0) ? 1u << j : 0u;
    uint32_t i = pos;
    for (uint32_t bits = cm; bits != 0u; bits &= bits - 1u, ++i) {
      const int j = __ffs(bits) - 1;
      const float yv = val[lo + j];
      fs.cand[i] = make_entry(c.temp_on ? div_rcp(yv, rt) : yv, lo + j, (int)i);
    }
  }
  static_assert(kFastCands % 16 == 0 && kFastCands <= 1024, "padding to 16 entries stays in the candidate array; "
                "positions fit the entry's rank field");
  const int C16 = __builtin_amdgcn_readfirstlane(((int)C + 15) & ~15);   // uniform: scalar loop control below
  if (t < C16 - (int)C) fs.cand[C + t] = 0ull;   // every entry is positive
  C4S_PHASE(27);
  __syncthreads();
  C4S_PHASE(12);
  // sort by rank counting (entries are distinct: their ids are); the first
  // kFastList + 1 places are kept
  uint64_t* srt = reinterpret_cast<uint64_t*>(fs.hist[0]);
  static_assert(sizeof(FastSh::hist[0]) >= (kFastList + 1) * sizeof(uint64_t), "the sorted head fits");
  const int Cs = __builtin_amdgcn_readfirstlane((int)C);
  for (int base = 0; base < Cs; base += kStepThreads) {
    const int i = base + t;
    const uint64_t mine = (i < Cs) ? fs.cand[i] : ~0ull;
    uint32_t r = 0;
    if (base + __builtin_amdgcn_readfirstlane(wv) * kWave < Cs)   // waves without an entry skip the count
      for (int j = 0; j < C16; j += 16) {   // 16 broadcast reads in flight a round
        uint64_t o[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) o[q] = fs.cand[j + q];
#pragma unroll
        for (int q = 0; q < 16; ++q) r += (o[q] > mine) ? 1u : 0u;
      }
    if (i < Cs && r < (uint32_t)(kFastList + 1)) srt[r] = mine;
  }
  __syncthreads();
  C4S_PHASE(13);
  if (wv == 0) {
    // the list: the leading entries above the bound (a prefix), at most kFastList
    const int nl = min((int)C, kFastList + 1);
    const bool a0 = lane < nl, a1 = lane + kWave < nl;
    uint64_t e0 = srt[a0 ? lane : 0], e1 = srt[a1 ? lane + kWave : 0];
    const uint64_t e2 = srt[nl > 2 * kWave ? 2 * kWave : 0];
    const int n_all = __popcll(__ballot(a0 && ent_key(e0) > tout)) + __popcll(__ballot(a1 && ent_key(e1) > tout)) +
                      ((nl > 2 * kWave && ent_key(e2) > tout) ? 1 : 0);
    const int nlist = min(n_all, kFastList);
    if (n_all > kFastList) tout = max(tout, ent_key(e2));
    const float ztop = kfloat(ent_key(srt[0]));   // C >= 1
    // the draw starts its maximum at -1e30 (text2semantic.cpp:150): below it the one pass decides
    bool ok = nlist > 0 && ztop >= -1e30f;
    C4S_PHASE(24);
    if (ok) {
      // each entry keeps its candidate position as its id-order key (8 bits)
      e0 = lane < nlist ? e0 : 0ull;
      e1 = lane + kWave < nlist ? e1 : 0ull;
      SumHdr h{};
      h.n = nlist;
      h.tout = tout;
      h.flags = 0u;
      uint64_t r = io.rng ? *io.rng : 0ull;
      StepOut o{0, 0u, 0u, 0u, 0u};
      static_assert(kFastCands <= 256, "candidate positions in 8 bits");
      ok = list_step<8, true>(h, e0, e1, 0.0f, 0.0f, c, V, NoHit{}, r, fs.cs, o);
      C4S_PHASE(25);
      if (ok && lane == 0) step_out(io, V, o.tok, r, true, 1u | 2u | 4u | 16u | 32u, 0u, o.dex, o.kept);
    }
    if (lane == 0) fs.bu[4] = ok ? 1u : 0u;
  }
  __syncthreads();
  C4S_PHASE(15);
  return fs.bu[4] != 0u;
}

// The one pass of a sampled row, specialised by the row's kind (top_k on; top_p
// with p < 1; p >= 1, a dense draw) so that the per-value loops carry no tests
// of the kind. Returns true when the row is finished; false leaves the row to
// the multi-pass chain (nothing written but the work area).
constexpr int kKindTopK = 0, kKindTopP = 1, kKindDense = 2;

template <int PT, int kKind>
__device__ __forceinline__ bool sampled_step(const StepIO& io, const RowCfg& c, const float (&y)[PT], int lo, int n,
                                             float* val, uint32_t* hc, unsigned long long* hm, uint64_t* sbuf,
                                             uint64_t* list, float* em, StepSh& ss, StepRowSh& rs) {
  const int t = threadIdx.x, lane = lane_id(), w = wave_id();
  const float ninf = neg_inf();
  // ---- sampled rows: temperature (sampling.cpp:14-17) and the maximum ----
  float z[PT];
  const double rt = 1.0 / (double)c.temp;   // used only when the temperature applies
#pragma unroll
  for (int j = 0; j < PT; ++j) z[j] = c.temp_on ? div_rcp(y[j], rt) : y[j];
  if (n < PT) {   // the last threads: the padding past the row stays -inf whatever the temperature
#pragma unroll
    for (int j = 0; j < PT; ++j) z[j] = j < n ? z[j] : ninf;
  }
  {
    float lm = ninf;
#pragma unroll
    for (int j = 0; j < PT; ++j) lm = fmaxf(lm, z[j]);
    lm = wave_max_dpp(lm);
    if (lane == 0) ss.wmax[w] = lm;
  }
  C4S_PHASE(2);
  __syncthreads();
  C4S_PHASE(3);
  float m = ninf;
#pragma unroll
  for (int i = 0; i < kStepWaves; ++i) m = fmaxf(m, ss.wmax[i]);
  const double thr = 1.0 - (double)c.p;   // sampling.cpp:64 removes while cum <= 1 - p
  constexpr bool topk = kKind == kKindTopK;
  constexpr bool dense = kKind == kKindDense;
  // The draw's maximum starts from -1e30f (text2semantic.cpp:150): below it, or
  // for an all -inf row, or with p <= 0, the multi-pass chain decides.
  bool one_pass = !(m < -1e30f) && thr < 1.0;
  int verdict = 0;
  bool tp_exact = false;
  if (one_pass) {
    // fp32 masses; the dense rows' kept set; the histogram (counts for top_k,
    // masses for top_p). Sums per thread in fp32: bound (2^-20 + PT 2^-24)
    // relative (terms and summation) + 2^-125 a term (underflow).
    // Every value goes through the same instructions (no branch a value): z is
    // -inf past the thread's ids, and an entry of the unbounded last bucket
    // adds to a word of its own thread instead (in the boundary list, unused
    // until the compaction): on a wide row most values lie there, and lanes
    // adding to one LDS word take turns.
    // The error bound counts every id of the thread (at least its finite ones).
    float s32 = 0.0f;
    uint32_t flags = 0, kc = 0;
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const float tt = z[j] - m;
      if (topk) {
        const int b = bucket_of_diff(-tt);   // the last bucket for -inf
        atomicAdd(b < kNB - 1 ? &hc[w * kNB + b] : reinterpret_cast<uint32_t*>(list) + t, 1u);
      } else {
        // 0 for -inf without a select: below about -150 the fp32 exp2 is 0
        // and mass32 returns +0, so clamping at -1000 changes no mass
        float ej = mass32(fmaxf(tt, -1000.0f));
        if (j < n) em[lo + j] = ej;   // read again by the kept sums and the draw
        if (dense) {
          // p == 1 removes the zero-mass positions: exp((double)tt) == 0 below
          // about -745.13; near that, and for subnormal kept masses, the chain decides
          const bool fin = z[j] != ninf;
          const bool kp = fin && (thr < 0.0 || tt > -745.0f);
          if (fin && ((thr == 0.0 && tt <= -745.0f && tt >= -745.25f) || (kp && tt < -690.0f))) flags = 1u;
          ej = kp ? ej : 0.0f;
          kc += kp ? 1u : 0u;
        } else {
          // 2^-31 fixed point, truncated (ej <= 1)
          const int b = bucket_of_diff(-tt);
          const uint32_t q = (uint32_t)(ej * 0x1p31f);
          atomicAdd(b < kNB - 1 ? &hm[w * kNB + b] : reinterpret_cast<unsigned long long*>(list) + t,
                    (unsigned long long)q + kHistOne);
        }
        s32 += ej;
      }
    }
    const double s = (double)s32;
    const double er = s * (0x1p-20 + PT * 0x1p-24) + (double)max(n, 0) * 0x1p-125;
    C4S_PHASE(4);
    const Scan2 sc = block_scan2(s, er, kc | (flags << 16), ss.wa, ss.wb, ss.wu);
    C4S_PHASE(5);
    const uint32_t n_pos = sc.utot & 0xFFFFu;   // dense rows: kept ids with a finite value
    // p == 1 with min_keep above the positive-mass count keeps zero-mass values
    // unmasked (sampling.cpp:67-68): the multi-pass chain handles that
    if ((sc.utot >> 16) || (dense && thr == 0.0 && n_pos < (uint32_t)max(0, c.min_keep))) {
      one_pass = false;
    } else if (dense) {
      // nothing to cut: the draw over the fp32 masses scanned above
      const KeptRule kr{true, thr < 0.0, 0ull};
      if (io.masked)
#pragma unroll
        for (int j = 0; j < PT; ++j)
          if (j < n) io.masked[lo + j] = (thr < 0.0 || (z[j] != ninf && z[j] - m > -745.0f)) ? z[j] : ninf;
      C4S_PHASE(10);
      draw_finish<PT, true>(io, c, kr, z, lo, n, m, sc, n_pos, 1u | 4u | 16u, 0u, ss, rs, em, list);
      C4S_PHASE(15);
      return true;
    } else {
      const double S = sc.tot, errS = sc.tot2;
      // boundary buckets: threads 0..255 merge one bucket each over the waves,
      // then wave 0 scans them (lane l holds buckets 4l .. 4l+3)
      uint32_t* bcnt = reinterpret_cast<uint32_t*>(sbuf);           // sort buffers are free here
      double* bmass = reinterpret_cast<double*>(sbuf) + kNB;
      if (t < kNB) {
        uint32_t cn = 0;
        unsigned long long ms = 0ull;
#pragma unroll
        for (int i = 0; i < kStepWaves; ++i) {
          const unsigned long long h = hm[i * kNB + t];
          cn += hc[i * kNB + t] + (uint32_t)(h >> 48);
          ms += h & (kHistOne - 1ull);
        }
        bcnt[t] = cn;
        bmass[t] = (double)ms * 0x1p-31;
      }
      __syncthreads();
      const double B = S - thr * S;   // the mass the kept entries hold
      const double Blo = B * (1.0 - 1e-3) - errS, Bhi = B * (1.0 + 1e-3) + errS;
      if (w == 0) {
        const Boundary bd = boundary_scan(bcnt, bmass, topk, (uint32_t)c.k, Blo, Bhi, 0u, 0.0);
        if (lane == 0) {
          ss.bsel[0] = bd.lo;
          ss.bsel[1] = bd.hi;
          ss.bsel[2] = (int)bd.above;
          ss.thru = bd.thru;
          ss.mab = bd.mabove;
          ss.mabx = topk ? 0.0 : bd.mabove;   // top_k: nothing lies above X
          ss.nabx = topk ? 0u : bd.above;
          ss.nx = 0u;
        }
      }
      __syncthreads();
      C4S_PHASE(6);
      const int blo = ss.bsel[0], bhi = ss.bsel[1];
      // the sub-window of the boundary buckets (all of them unless refined)
      int slo = 0, shi = kNB - 1, lo2 = 0;
      float sc2 = 0.0f;
      bool refine = false;
      if (blo >= 0 && bhi >= 0) {
        // More boundary entries than one sort takes (flat rows): histogram the
        // boundary buckets again, kNB sub-buckets over them (top_k: over the
        // k-th entry's bucket), and keep the sub-buckets where the boundary
        // falls. Not for the unbounded last bucket.
        const uint32_t nest = topk ? ss.thru : ss.thru - (uint32_t)ss.bsel[2];
        refine = nest > (uint32_t)kSortCap && bhi < kNB - 1;
        if (refine) {
          lo2 = topk ? bhi : blo;
          sc2 = (float)kNB / (float)(bhi + 1 - lo2);
          for (int i = t; i < (int)(3 * kHistBytes / 4); i += kStepThreads) hc[i] = 0u;
          __syncthreads();
          // Per value: no branch, and the fp32 mass the first pass cached (the
          // same mass32), read unconditionally (index clamped). -inf and the
          // padding past the thread's ids lie in the last bucket, never in the
          // window (bhi < kNB - 1); entries outside it add to a word of the
          // thread's own (the boundary list, unused until the compaction).
#pragma unroll
          for (int j = 0; j < PT; ++j) {
            const int b = bucket_of(z[j], m);
            const bool inw = ((int)(b >= lo2) & (int)(b <= bhi)) != 0;
            const int sb = sub_bucket_of(z[j], m, lo2, sc2);
            if (topk) {
              atomicAdd(inw ? &hc[w * kNB + sb] : reinterpret_cast<uint32_t*>(list) + t, 1u);
            } else {
              const float ec = em[min(lo + j, c.V - 1)];
              atomicAdd(inw ? &hm[w * kNB + sb] : reinterpret_cast<unsigned long long*>(list) + t,
                        (unsigned long long)(uint32_t)(ec * 0x1p31f) + kHistOne);
            }
          }
          __syncthreads();
          if (t < kNB) {
            uint32_t cn = 0;
            unsigned long long ms = 0ull;
#pragma unroll
            for (int i = 0; i < kStepWaves; ++i) {
              const unsigned long long h = hm[i * kNB + t];
              cn += hc[i * kNB + t] + (uint32_t)(h >> 48);
              ms += h & (kHistOne - 1ull);
            }
            bcnt[t] = cn;
            bmass[t] = (double)ms * 0x1p-31;
          }
          __syncthreads();
          if (w == 0) {
            const Boundary b2 = boundary_scan(bcnt, bmass, topk, (uint32_t)c.k, Blo, Bhi, (uint32_t)ss.bsel[2],
                                              ss.mab);
            if (lane == 0) {
              ss.sub[0] = topk ? 0 : b2.lo;   // top_k: every entry above the k-th stays in the sort
              ss.sub[1] = b2.hi;
              if (!topk) {
                ss.mabx = b2.mabove;
                ss.nabx = b2.above;
              }
            }
          }
          __syncthreads();
          slo = ss.sub[0];
          shi = ss.sub[1];
        }
      }
      C4S_PHASE(16);
      C4S_PHASE_VAL(21, refine ? 1 : 0);
      if (blo < 0 || bhi < 0 || slo < 0 || shi < 0) {
        one_pass = false;
      } else {
        // X: the entries to sort. top_k: every entry up to the k-th value's
        // (sub-)bucket (the survivors then are a prefix of X). top_p: the
        // boundary (sub-)buckets; every entry above them is kept, every entry
        // below removed. side(): -1 above X, 0 in X, 1 below (monotone in z).
        const int xlo = topk ? 0 : blo, xhi = bhi;
        const SideRule sr{m, sc2, xlo, xhi, lo2, slo, shi, refine};
        auto side = [&](float zj) { return sr.side(zj); };
        // X's entries go to `list`, each wave taking one block of slots with
        // one atomic (slot order is arbitrary: the sort orders them)
        static_assert(PT < 32, "a thread's X entries as one bit mask");
        uint32_t xm = 0;   // this thread's X entries (its ids only: the -inf padding may lie in the last bucket)
        if (!refine) {
          // uniform: X is whole buckets xlo .. xhi. With q = (m - z) 4 (exact:
          // a power of two; q >= 0, +inf for -inf) bucket_of is trunc(q) below
          // 255, else 255: b >= xlo iff !(q < xlo) (NaN in the last bucket), and
          // b <= xhi iff q < xhi + 1 unless xhi is the last bucket
          const float qlo = (float)xlo, qhi = xhi >= kNB - 1 ? __builtin_inff() : (float)(xhi + 1);
          const bool last = xhi >= kNB - 1;
#pragma unroll
          for (int j = 0; j < PT; ++j) {
            const float q = (m - z[j]) * kBucketScale;
            xm |= ((int)!(q < qlo) & (int)(last || q < qhi)) ? 1u << j : 0u;
          }
        } else {
#pragma unroll
          for (int j = 0; j < PT; ++j) xm |= (side(z[j]) == 0) ? 1u << j : 0u;
        }
        xm &= (1u << n) - 1u;
        {
          const uint32_t cx = (uint32_t)__popc(xm);
          const uint32_t inc = wave_scan_u32(cx);
          uint32_t wb = 0;
          if (lane == kWave - 1 && inc > 0u) wb = atomicAdd(&ss.nx, inc);
          const uint32_t base = readlane_u32(wb, kWave - 1) + inc - cx;
          // the set bits only, in id order (a wave takes as many rounds as its
          // lane with the most X entries: usually one or two), each value read
          // again from the row in LDS (z = fl(y / T), the same division)
          uint32_t slot = base;
          for (uint32_t bits = xm; bits != 0u; bits &= bits - 1u, ++slot) {
            const int j = __ffs(bits) - 1;
            const float yv = val[lo + j];
            if (slot < (uint32_t)kSortCap) list[slot] = key64(c.temp_on ? div_rcp(yv, rt) : yv, lo + j);
          }
        }
        C4S_PHASE(17);
        __syncthreads();
        C4S_PHASE(7);
        const int nX = (int)ss.nx;
        C4S_PHASE_VAL(20, nX);
        // The mass above X and its count, from the histogram: the fixed-point
        // masses of the (sub-)buckets above X. Against the exact masses each
        // entry is off by its fp32 mass error (2^-20 relative + 2^-125) and
        // the truncation (below 2^-31); the bucket sums are exact integers and
        // the scan's double prefix adds a few 2^-53 relative.
        const double Ma = ss.mabx;
        const uint32_t n_above = ss.nabx;
        const double eMa = Ma * (0x1p-20 + 0x1p-40) + (double)n_above * 0x1p-30;
        if (nX > kSortCap) {
          // more boundary entries than one sort takes: one_pass only if they
          // all hold one value (ties), which needs no sort
          verdict = tie_cut<PT>(rs.cfg, val, lo, n, sr, nX, thr, S, errS, Ma, eMa, n_above, ss);
          C4S_PHASE(28);
          tp_exact = verdict == 3;
          if (verdict != 1 && verdict != 3) one_pass = false;
          if (verdict == 4 && t == 0) rs.tp_exact_first = 1u;
        } else {
          int P2 = 1;
          while (P2 < nX) P2 <<= 1;
          const bool block = P2 > kWave;
          uint64_t v = 0ull;
          if (block) {
            // up to 256 entries by rank counting (two to four threads a key,
            // two barriers); more by the bitonic network (six barriers)
            if (nX <= 128) {
              v = rank_sort_desc<128>(list, nX, reinterpret_cast<uint32_t*>(sbuf));
            } else if (nX <= 256) {
              v = rank_sort_desc<256>(list, nX, reinterpret_cast<uint32_t*>(sbuf));
            } else {
              v = t < nX ? list[t] : 0ull;
              v = sort_desc_block(v, P2, sbuf);
              if (t < nX) list[t] = v;
              __syncthreads();
            }
            C4S_PHASE(8);
            if (t == 0) ss.zx = key_value(v);   // X's largest value (read after the barriers below)
            decide_cut<true>(rs.cfg, v, nX, m, thr, S, errS, Ma, eMa, n_above, list, ss);
          } else if (w == 0) {
            v = lane < nX ? list[lane] : 0ull;
            v = sort_desc_wave(v, P2);
            C4S_PHASE(8);
            if (t == 0) ss.zx = key_value(v);
            decide_cut<false>(rs.cfg, v, nX, m, thr, S, errS, Ma, eMa, n_above, list, ss);
          }
          __syncthreads();
          verdict = ss.verdict;
          if (verdict == 2) {
            // decide again with every mass in double (S and the mass above the boundary)
            tp_exact = true;
            // every value through the same instructions, so that the exps
            // interleave: z is -inf past the thread's ids and exp(-inf) = 0.
            // side() is monotone in z and equal values share a side, so the
            // entries above X are exactly those above X's largest value.
            double se = 0.0, sa = 0.0;
            if (nX > 0) {
              const float zx = ss.zx;
#pragma unroll
              for (int j = 0; j < PT; ++j) {
                const double ed = exp((double)(z[j] - m));
                se += ed;
                sa += z[j] > zx ? ed : 0.0;
              }
            } else {
#pragma unroll
              for (int j = 0; j < PT; ++j) {
                const double ed = exp((double)(z[j] - m));
                se += ed;
                sa += side(z[j]) < 0 ? ed : 0.0;
              }
            }
            se = wave_sum_dpp(se);
            sa = wave_sum_dpp(sa);
            if (lane == 0) { ss.wc[w] = se; ss.wd[w] = sa; }
            __syncthreads();
            double Se = 0.0, Mae = 0.0;
#pragma unroll
            for (int i = 0; i < kStepWaves; ++i) { Se += ss.wc[i]; Mae += ss.wd[i]; }
            if (block) decide_cut<true>(rs.cfg, v, nX, m, thr, Se, 0.0, Mae, 0.0, n_above, list, ss);
            else if (w == 0) decide_cut<false>(rs.cfg, v, nX, m, thr, Se, 0.0, Mae, 0.0, n_above, list, ss);
            __syncthreads();
            verdict = ss.verdict;
          }
          C4S_PHASE(9);
          C4S_PHASE_VAL(22, verdict);
          if (verdict != 1) one_pass = false;
          if (verdict == 4 && t == 0) rs.tp_exact_first = 1u;
        }
      }
    }
  }
  if (one_pass) {
    // the draw over the kept set: key >= the last kept key
    const uint64_t kthr = ss.kthr;
    const KeptRule kr{false, false, kthr};
    float ks32 = 0.0f;
    uint32_t kc = 0, flags = 0;
    float ecs[PT];   // top_p: the masses cached by the histogram pass (0 for -inf)
    if (!topk) read_row(em, lo, n, c.V, ecs);
#pragma unroll
    for (int j = 0; j < PT; ++j) {   // z is -inf past the thread's ids: never kept with a mass
      bool kp;
      float ej;
      if (topk) {
        ej = kept_mass32(kr, z[j], m, lo + j, kp);
      } else {
        const float ec = ecs[j];
        kp = ((int)(z[j] != ninf) & (int)kept_in(kr, z[j], m, lo + j)) != 0;   // z is -inf past the thread's ids
        ej = kp ? ec : 0.0f;
      }
      const bool kf = kp && z[j] != ninf;
      kc += kf ? 1u : 0u;
      ks32 += ej;
    }
    // subnormal kept masses (libm implementations may disagree): the smallest
    // kept value is the last kept key's (a -inf there also sends the row on)
    flags = (t == 0 && key_value(kthr) - m < -690.0f) ? 1u : 0u;
    if (io.masked)
#pragma unroll
      for (int j = 0; j < PT; ++j) {
        bool kp;
        kept_mass32(kr, z[j], m, lo + j, kp);
        if (j < n) io.masked[lo + j] = kp ? z[j] : ninf;
      }
    C4S_PHASE(27);
    const double ks = (double)ks32;
    const double ek = ks * (0x1p-20 + PT * 0x1p-24) + (double)kc * 0x1p-125;
    const Scan2 ds = block_scan2(ks, ek, kc | (flags << 16), ss.wa, ss.wb, ss.wu);
    C4S_PHASE(10);
    if ((ds.utot >> 16) == 0u) {
      draw_finish<PT, !topk>(io, c, kr, z, lo, n, m, ds, ds.utot & 0xFFFFu, 1u | (topk ? 2u : 0u) | 4u | 16u,
                             tp_exact ? 1u : 0u, ss, rs, em, list);
      C4S_PHASE(15);
      return true;
    }
  }
  return false;
}

// One AR step of the reference chain (C4S_MODE_CHAIN) for one row per
// workgroup, in one pass where it can (c4s_step.hpp), else the multi-pass
// chain on the row staged in LDS. PT >= the ids a thread owns.
// Byte i of a per-row flag array, nonzero or not, read through the aligned
// dword that holds it: a scalar load (the flags are the same for the whole
// workgroup), where a byte load would go through the vector memory path and be
// waited for at once. The dword never leaves the allocation's 256-byte granule.
__device__ __forceinline__ bool flag_byte(const uint8_t* __restrict__ p, int i) {
  const uint8_t* b = p + i;
  const int sh = (int)(reinterpret_cast<uintptr_t>(b) & 3);
  const uint32_t wd = *reinterpret_cast<const uint32_t*>(b - sh);
  return ((wd >> (8 * sh)) & 0xFFu) != 0u;
}

template <int PT>
__global__ __launch_bounds__(kStepThreads) void k_rows_step(RowsArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ StepScratch sh;
  __shared__ StepSh ss;
  __shared__ StepRowSh rs;
  const int row = blockIdx.x;
  const int V = a.vocab;
  const int t = threadIdx.x;
  // Every read that depends on no other goes out first: the row's flags and
  // parameters, its history offsets, then the row itself (fp32 rows into
  // registers here, stored to LDS below); nothing waits on them before the
  // row's loads are in flight, so the step pays one memory round trip up front
  // instead of one per dependent read.
  const int64_t roff = (int64_t)row * a.ld;
  const float* xf_row = a.dtype == 0 ? static_cast<const float*>(a.logits) + roff : nullptr;
  StepFetch f;
  if (xf_row) step_fetch(xf_row, V, f);
  const bool act = a.row_active ? flag_byte(a.row_active, row) : true;
  const bool sample = a.do_sample ? flag_byte(a.do_sample, row) : true;
  const float pv = a.pen ? a.pen[row] : 1.0f, tv = a.temp ? a.temp[row] : 1.0f;
  const int32_t kv = a.top_k ? a.top_k[row] : 0, mv = a.min_keep ? a.min_keep[row] : 1;
  const float ppv = a.top_p ? a.top_p[row] : 1.0f;
  const bool csr_arg = a.hist_off && !a.hist_bits;
  int64_t h0 = 0, h1 = 0;
  if (csr_arg) {
    h0 = a.hist_off[row];
    h1 = a.hist_off[row + 1];
  }
  if (!act) {
    if (t == 0) a.out_tok[row] = -1;
    return;
  }
  const RowCfg c = make_cfg_vals(0u, V, pv, tv, kv, ppv, mv, sample);
  C4S_PHASE(0);
  unsigned char* work = smem;
  float* vbuf = reinterpret_cast<float*>(smem + step_work_bytes(V));
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(vbuf + vpad(V) + 4);
  uint32_t* hc = reinterpret_cast<uint32_t*>(work);   // [waves][kNB] bucket counts
  unsigned long long* hm = reinterpret_cast<unsigned long long*>(work + kHistBytes);   // [waves][kNB] masses, 2^-32 units
  uint64_t* sbuf = reinterpret_cast<uint64_t*>(work + 3 * kHistBytes);
  uint64_t* list = sbuf + 2 * kSortCap;
  const int P = odd_chunk<kStepThreads>(V);
  const int lo = min(V, t * P), n = min(V, lo + P) - lo;
  const bool csr = c.pen_on && !a.hist_bits;
  StepIO io;
  io.xf = xf_row;
  io.xb = a.dtype == 1 ? static_cast<const uint16_t*>(a.logits) + roff : nullptr;
  io.bitmap = csr ? bitmap : nullptr;
  io.hbits = (c.pen_on && a.hist_bits) ? a.hist_bits + (int64_t)row * hist_words(V) : nullptr;
  io.out_tok = a.out_tok + row;
  io.rng = a.rng ? a.rng + row : nullptr;
  io.masked = a.out_masked ? a.out_masked + (int64_t)row * V : nullptr;
  io.stats = a.stats ? a.stats + 4 * (int64_t)row : nullptr;
  io.join = a.hist_bits ? a.hist_bits + (int64_t)row * hist_words(V) : nullptr;
  io.stop_token = a.stop_token;
  if (t == 0) {   // read only after the barrier below
    rs.cfg = c;
    rs.io = io;
    rs.tp_exact_first = 0u;
  }
  const float ninf = neg_inf();

  // The history's first two ids of this thread (or this thread's words of the
  // history set) go out behind the row's loads, before anything waits for the
  // row: storing the row to LDS waits for the row alone.
  if (!csr) h0 = h1 = 0;
  const int hid = (csr && h0 + t < h1) ? a.hist_ids[h0 + t] : -1;
  const int hid2 = (csr && h0 + t + kStepThreads < h1) ? a.hist_ids[h0 + t + kStepThreads] : -1;
  // penalty bits of this thread's ids: words lo/32 and lo/32 + 1 (up to 33 ids
  // from bit lo % 32 span at most two words)
  static_assert(PT <= 33, "a thread's ids span at most two bitmap words");
  uint32_t pw[2] = {0u, 0u};
  if (io.hbits) {
    // every load unconditional (index clamped), so nothing waits for them here:
    // the penalty below keeps only the bits of ids lo .. lo + n - 1, and a
    // clamped word past the set would stand for ids at or above V
    const int w0 = lo >> 5, hwn = hist_words(V);
#pragma unroll
    for (int q = 0; q < 2; ++q) pw[q] = io.hbits[min(w0 + q, hwn - 1)];
  }
  // the row into LDS (fp32: its loads went out above)
  float* val;
  if (io.xf) {
    val = step_store(io.xf, V, f, vbuf);
  } else {
    val = stage_row_bf16(io.xb, V, vbuf);
  }
  // LDS: the history bitmap and the histograms start at zero
  const int nw = bitmap_words(V);
  if (csr)
    for (int i = t; i < nw; i += kStepThreads) bitmap[i] = 0u;
  if (!c.greedy)
    for (int i = t; i < (int)(3 * kHistBytes / 4); i += kStepThreads) hc[i] = 0u;
  __syncthreads();
  if (csr) {
    if (hid >= 0 && hid < V) atomicOr(&bitmap[hid >> 5], 1u << (hid & 31));   // sampling.cpp:24
    if (hid2 >= 0 && hid2 < V) atomicOr(&bitmap[hid2 >> 5], 1u << (hid2 & 31));
    for (int64_t j = h0 + t + 2 * kStepThreads; j < h1; j += kStepThreads) {
      const int id = a.hist_ids[j];
      if (id >= 0 && id < V) atomicOr(&bitmap[id >> 5], 1u << (id & 31));
    }
    __syncthreads();
    // unconditional reads (index clamped, as for the caller's set above)
    const int w0 = lo >> 5;
#pragma unroll
    for (int q = 0; q < 2; ++q) pw[q] = bitmap[min(w0 + q, nw - 1)];
  }
  C4S_PHASE(1);
  if (c.pen_on) {
    // sampling.cpp:19-28 on this thread's ids in LDS, one set bit at a time
    // (each distinct id once); the row in LDS is the penalised row from here on
    // (dividing only the set bits: every value of the thread through the
    // double reciprocal costs more than this loop)
    const double rp = 1.0 / (double)c.pen;
    uint32_t pm = (uint32_t)(((((uint64_t)pw[1] << 32) | pw[0]) >> (lo & 31))) & ((1u << n) - 1u);
    while (pm) {
      const int i = lo + __ffs(pm) - 1;
      pm &= pm - 1;
      const float x = val[i];
      val[i] = (x < 0) ? x * c.pen : div_rcp(x, rp);   // sampling.cpp:26
    }
  }
  C4S_PHASE(14);
  // this thread's ids (odd stride: no LDS bank conflicts), every read
  // unconditional (index clamped) and the padding selected afterwards
  float y[PT];
  read_row(val, lo, n, V, y);
  if (n < PT) {
#pragma unroll
    for (int j = 0; j < PT; ++j) y[j] = j < n ? y[j] : ninf;
  }
  C4S_PHASE(29);

  if (c.greedy) {   // text2semantic.cpp:144-145: argmax of the penalised row, first maximum
    float bv = ninf;
    int bi = INT_MAX;
#pragma unroll
    for (int j = 0; j < PT; ++j)
      if (j < n) argmax_merge(bv, bi, y[j], lo + j);
    block_argmax<kStepThreads>(bv, bi, sh.redf, sh.redi);
    if (io.masked)
#pragma unroll
      for (int j = 0; j < PT; ++j)
        if (j < n) io.masked[lo + j] = y[j];
    if (t == 0) step_out(io, V, bi, 0ull, false, 8u | 16u, 0u, 0u, (uint32_t)V);
    return;
  }

  // top-k rows with k <= 64: on a candidate list when it settles the step
  if (c.draw && c.topk_on && c.k <= kWave && c.p > 0.0f && !io.masked) {
    if (list_fast<PT>(io, c, V, y, lo, n, val, *reinterpret_cast<FastSh*>(work))) return;
    for (int i = t; i < (int)(3 * kHistBytes / 4); i += kStepThreads) hc[i] = 0u;
    __syncthreads();
  }

  bool done;
  float* em = reinterpret_cast<float*>(work + kStepWorkBytes);   // per-id fp32 masses
  if (c.topk_on) done = sampled_step<PT, kKindTopK>(io, c, y, lo, n, val, hc, hm, sbuf, list, em, ss, rs);
  else if (c.p >= 1.0f) done = sampled_step<PT, kKindDense>(io, c, y, lo, n, val, hc, hm, sbuf, list, em, ss, rs);
  else done = sampled_step<PT, kKindTopP>(io, c, y, lo, n, val, hc, hm, sbuf, list, em, ss, rs);
  if (done) return;
  // ---- the multi-pass chain on the row staged in LDS (c4s_chain.hpp) ----
  __syncthreads();   // every thread is done with the work area
  chain_fallback(rs.io, rs.cfg, work, val, sh, rs.tp_exact_first != 0u);
}

// ---- large vocabularies: top_k in two passes -----------------------------------------
//
// A sampled row with top_k in [1, kT2MaxK] (e.g. 256 rows x V = 151936, k = 50)
// does not need the whole row after top_k: every entry below the k-th largest
// value is -inf from there on (sampling.cpp:30-40), so top_p (sampling.cpp:
// 42-71) and the draw (text2semantic.cpp:150-165) only see the survivors.
// Pass 1 reads the row once (penalty, temperature) for its maximum and a
// histogram of the top kT2Bits bits of the order-preserving value keys, which
// locates the bucket b* of the k-th largest value; pass 2 reads it again and
// collects every entry of b* and above (at most kT2Cap) with its id. Sorted,
// their first k give the threshold (ties kept). Wave 0 then replays top_p and
// the draw on the survivors sequentially in double, in the reference's order
// (top_p ascending by value, equal values higher id first; the draw in id
// order), so the sums are the reference's own: the -inf positions add 0.
constexpr int kT2Bits = 11;
constexpr int kT2Buckets = 1 << kT2Bits;
constexpr int kT2Copies = 4;        // histogram copies (by wave) to spread the LDS atomics
constexpr int kT2Cap = 2 * NT;      // candidates the sort takes
constexpr int kT2MaxK = NT;
constexpr int kT2MaxV = 1 << 19;    // above: the LDS holds the history bitmap only

struct T2Sh {
  uint32_t hist[kT2Copies][kT2Buckets];
  uint64_t list[kT2Cap];
  double e[kT2Cap];                 // the draw's masses in id order
  uint32_t wsum[NW];
  float wmax[NW];
  uint32_t wm4[NW];                 // one read: per-wave largest candidate key
  uint32_t n;
  int bstar;
  uint32_t nge, nkeep;
  int tok;
  uint32_t dex;                     // the draw replayed sequentially (1) or not
  uint32_t pick[2];                 // one read: the picked candidate's bin and the candidates above it
  uint32_t nq;                      // one read: gathered entries whose penalised key reaches the bound
};

__host__ __device__ __forceinline__ size_t t2_offset(int V) { return ((size_t)4 * ((V + 31) / 32) + 15) & ~(size_t)15; }

// Descending sort of n <= NT distinct 64-bit keys by rank counting (each key's
// place is the count of keys above it), through tmp; two barriers.
__device__ __forceinline__ void rank_sort_desc_u64(uint64_t* buf, uint64_t* tmp, int n) {
  const int t = threadIdx.x;
  if (t < n) {
    const uint64_t mine = buf[t];
    int r = 0;
    for (int j = 0; j < n; ++j) r += (buf[j] > mine) ? 1 : 0;
    tmp[r] = mine;
  }
  __syncthreads();
  if (t < n) buf[t] = tmp[t];
  __syncthreads();
}
constexpr int kRankSortMax = 256;   // above: the bitonic network

// In-buffer descending bitonic sort of P (a power of two) 64-bit keys by the
// NT threads of the workgroup.
__device__ void bitonic_desc_u64(uint64_t* buf, int P) {
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int t = threadIdx.x; t < (P >> 1); t += NT) {
        const int i = (t / j) * 2 * j + (t % j);
        const int pi = i + j;
        const uint64_t x = buf[i], y = buf[pi];
        const bool down = (i & k) == 0;
        if ((x < y) == down) { buf[i] = y; buf[pi] = x; }
      }
      __syncthreads();
    }
  }
}

// The row's value at id i after penalty and temperature (sampling.cpp:19-28,
// 14-17), as the multi-pass chain computes it.
struct T2Row {
  const float* xf;
  const uint16_t* xb;
  const uint32_t* bitmap;
  bool pen_on, temp_on;
  float pen, temp;
  double rpen, rtemp;   // fl64(1 / pen), fl64(1 / temp)
  __device__ __forceinline__ float z(int i, float x) const {
    if (pen_on && ((bitmap[i >> 5] >> (i & 31)) & 1u)) x = (x < 0) ? x * pen : div_rcp(x, rpen);
    return temp_on ? div_rcp(x, rtemp) : x;
  }
  // f(i, z) for every id, each by one thread: 16-byte loads over the aligned body
  template <class F>
  __device__ __forceinline__ void each(int V, F&& f) const {
    const int t = threadIdx.x;
    if (xf) {
      const RowShape rs = row_shape(xf, V);
      const float4* p4 = reinterpret_cast<const float4*>(xf + rs.head);
      for (int q = t; q < rs.nq; q += NT) {
        const float4 v = p4[q];
        const int i = rs.head + 4 * q;
        f(i, z(i, v.x));
        f(i + 1, z(i + 1, v.y));
        f(i + 2, z(i + 2, v.z));
        f(i + 3, z(i + 3, v.w));
      }
      if (t < rs.head) f(t, z(t, xf[t]));
      else if (t < rs.head + rs.tail) {
        const int i = rs.head + 4 * rs.nq + (t - rs.head);
        f(i, z(i, xf[i]));
      }
    } else {
      for (int i = t; i < V; i += NT) f(i, z(i, __uint_as_float((uint32_t)xb[i] << 16)));
    }
  }
};

// ---- one read of the row (fp32 rows, penalty >= 1) ----
//
// Each thread streams its ids once (16-byte loads, U of them in flight) and
// keeps its four largest entries as packed keys: the top 23 bits of the
// order-preserving key of the raw value x, then a 9-bit index of the entry
// in the thread's stream (3 v_med3 and 1 v_max a value, no LDS atomics). The
// penalty only lowers a value (penalty >= 1, sampling.cpp:26) and fl(y / T) is
// monotone in y, so the raw keys bound the penalised and divided ones from
// above. One pick over the 4 NT candidates, binned by their distance below
// the largest, gives Q, the 23-bit prefix of the lowest key in the bin of the
// (k + kOneSlack)-th largest candidate (the slack leaves room for entries the
// penalty takes below Q). Every entry whose raw prefix reaches Q is gathered:
// from the four of a thread whose fourth lies below Q, else from its stream
// read again by its wave; each is read again (a few cache lines), penalised
// and divided exactly, and goes to ts.list. The rest of the row stays out of
// the top k when at least k gathered entries still reach Q after their
// penalty (then the k-th largest value is at or above Q's smallest key, and
// every entry at or above it was gathered; otherwise the pick is taken again
// deeper down) and no value below Q can tie the k-th quotient (checked once
// the list is sorted). Returns false, with nothing but the work area written,
// when a check fails: the two passes over the row decide then.
constexpr int kOneIdxBits = 9;
constexpr uint32_t kOneEdge = (1u << kOneIdxBits) - 1;   // index of the thread's unaligned head / tail entry
constexpr int kOneUnroll = 8;
constexpr uint32_t kOneSlack = 16;
constexpr int kOneBinShift = 15;   // candidate bins of 2^15 packed keys: 1/256 of a binade
// 16-byte loads a thread; the unrolled loop rounds them up to kOneUnroll, and
// every index it makes (padding past the row included) stays below kOneEdge
constexpr int kOneMaxIters = 120;
static_assert(kOneMaxIters % kOneUnroll == 0 && 4 * kOneMaxIters - 1 < (int)kOneEdge, "indices below the edge's");
constexpr int kOneMaxV = 4 * NT * kOneMaxIters;

__device__ __forceinline__ uint32_t one_pack(float x, uint32_t idx) {
  return (fkey(x) & ~kOneEdge) | idx;
}
// The median of three (v_med3_u32): max(lo, min(hi, e)) when lo <= hi, which
// the compiler cannot know here.
__device__ __forceinline__ uint32_t med3_u32(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// t0 >= t1 >= t2 >= t3 keeps the four largest (the order holds from the start, all zero)
__device__ __forceinline__ void one_insert(uint32_t& t0, uint32_t& t1, uint32_t& t2, uint32_t& t3, uint32_t e) {
  t3 = med3_u32(t3, t2, e);
  t2 = med3_u32(t2, t1, e);
  t1 = med3_u32(t1, t0, e);
  t0 = max(t0, e);
}

// Bin of `hist` (nb bins scanned from the top, nb / NT a thread) holding the
// m-th largest counted key, and the count above it, into ts.pick; false when
// fewer than m keys were counted. Two barriers.
template <int NB>
__device__ __forceinline__ bool one_pick(const uint32_t* hist, uint32_t m, T2Sh& ts) {
  constexpr int PB = NB / NT;
  const int t = threadIdx.x, lane = lane_id(), w = wave_id();
  uint32_t cb[PB], loc = 0;
#pragma unroll
  for (int i = 0; i < PB; ++i) { cb[i] = hist[NB - 1 - PB * t - i]; loc += cb[i]; }
  const uint32_t inc = wave_scan_u32(loc);
  if (lane == kWave - 1) ts.wsum[w] = inc;
  __syncthreads();
  uint32_t ex = inc - loc, total = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const uint32_t x = ts.wsum[i];
    ex += (i < w) ? x : 0u;
    total += x;
  }
  if (total < m) return false;   // uniform
  if (ex < m && ex + loc >= m) {
    uint32_t run = ex;
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      if (run < m && run + cb[i] >= m) { ts.pick[0] = (uint32_t)(NB - 1 - PB * t - i); ts.pick[1] = run; }
      run += cb[i];
    }
  }
  __syncthreads();
  return true;
}

// Buffer resource of `bytes` bytes from p (raw: byte offsets; a load past
// the end returns zeros without an access). Loads through one issue on every
// path, so that the waits of later loads count them exactly.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ float4 rsrc_load16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// The first kOneUnroll 16-byte loads of this thread's stream of an f32 row
// (the layout of topk_one_read), issued before the row's set-up so that they
// are in flight meanwhile; with `on` false nothing is read (xf need only be
// a pointer).
struct OneFirst {
  float4 v[kOneUnroll];
};
__device__ __forceinline__ void one_first(const float* xf, int V, bool on, OneFirst& f) {
  const RowShape rs = row_shape(xf, V);
  const __amdgpu_buffer_rsrc_t r = raw_rsrc(xf + rs.head, on ? 16 * rs.nq : 0);
  const float ninf = neg_inf();
#pragma unroll
  for (int u = 0; u < kOneUnroll; ++u) {
    const int q = threadIdx.x + NT * u;
    const float4 v = rsrc_load16(r, 16 * q);
    f.v[u] = (q < rs.nq) ? v : make_float4(ninf, ninf, ninf, ninf);
  }
}

__device__ __forceinline__ bool topk_one_read(const RowsArgs& a, const RowCfg& c, const float* xf, const uint32_t* bitmap,
                              T2Sh& ts, uint32_t& qkey, const OneFirst& first) {
  const int V = c.V, t = threadIdx.x, w = wave_id(), lane = lane_id();
  const RowShape rs = row_shape(xf, V);
  const float4* p4 = reinterpret_cast<const float4*>(xf + rs.head);
  const float ninf = neg_inf();
  uint32_t t0 = 0u, t1 = 0u, t2 = 0u, t3 = 0u;   // 0: below every packed key
  const int iters = (rs.nq + NT - 1) / NT;
  auto take = [&](const float4 (&v)[kOneUnroll], int j0) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kOneUnroll; ++u) {
      const uint32_t i0 = 4u * (uint32_t)(j0 + u);
      one_insert(t0, t1, t2, t3, one_pack(v[u].x, i0));
      one_insert(t0, t1, t2, t3, one_pack(v[u].y, i0 + 1u));
      one_insert(t0, t1, t2, t3, one_pack(v[u].z, i0 + 2u));
      one_insert(t0, t1, t2, t3, one_pack(v[u].w, i0 + 3u));
    }
  };
  take(first.v, 0);   // loads 0 .. kOneUnroll - 1 (past the row: -inf)
  for (int j0 = kOneUnroll; j0 < iters; j0 += kOneUnroll) {
    float4 v[kOneUnroll];
#pragma unroll
    for (int u = 0; u < kOneUnroll; ++u) {
      const int q = t + NT * (j0 + u);
      v[u] = (q < rs.nq) ? p4[q] : make_float4(ninf, ninf, ninf, ninf);
    }
    take(v, j0);
  }
  const int edge = (t < rs.head) ? t : ((t < rs.head + rs.tail) ? rs.head + 4 * rs.nq + (t - rs.head) : -1);
  if (edge >= 0) one_insert(t0, t1, t2, t3, one_pack(xf[edge], kOneEdge));
  C4S_PHASE(8);
  auto id_of = [&](uint32_t e) -> int {
    const uint32_t ix = e & kOneEdge;
    if (ix == kOneEdge) return edge;
    return rs.head + 4 * (t + NT * (int)(ix >> 2)) + (int)(ix & 3u);
  };
  auto valid = [&](uint32_t e) {   // a real entry of the row (not padding past it)
    const uint32_t ix = e & kOneEdge;
    return e != 0u && (ix == kOneEdge ? edge >= 0 : t + NT * (int)(ix >> 2) < rs.nq);
  };
  // The candidates by their distance below the largest, M: bin b (from the
  // top) holds the packed keys in (M - (b + 1) 2^S, M - b 2^S], 1/256 of a
  // binade, the last bin everything farther down (the LDS atomics spread over
  // many bins where a histogram of the keys' top bits had a few).
  for (int i = t; i < kT2Buckets; i += NT) ts.hist[0][i] = 0u;
  {
    const uint32_t m0 = wave_max_u32(t0);
    if (lane == 0) ts.wm4[w] = m0;
    if (t == 0) { ts.n = 0u; ts.nq = 0u; }
  }
  __syncthreads();
  uint32_t M = 0u;
#pragma unroll
  for (int i = 0; i < NW; ++i) M = max(M, ts.wm4[i]);
  const uint32_t tk[4] = {t0, t1, t2, t3};
  uint32_t* h1 = ts.hist[0];
#pragma unroll
  for (int i = 0; i < 4; ++i)   // one_pick scans from the highest bin: the bins nearest M
    if (tk[i]) atomicAdd(&h1[(kT2Buckets - 1) - min((uint32_t)(kT2Buckets - 1), (M - tk[i]) >> kOneBinShift)], 1u);
  __syncthreads();
  C4S_PHASE(1);
  const uint32_t k = (uint32_t)c.k;
  uint32_t kb = k + kOneSlack;
  for (int attempt = 0;; ++attempt) {
    if (!one_pick<kT2Buckets>(h1, kb, ts)) return false;   // fewer candidates than that (uniform)
    const uint32_t bfar = (kT2Buckets - 1) - ts.pick[0];   // bins below M
    const int64_t lo = (int64_t)M - ((int64_t)(bfar + 1) << kOneBinShift) + 1;
    // the bound: the prefix of the lowest key of that bin, above -inf's
    if (bfar >= (uint32_t)(kT2Buckets - 1) || lo <= (int64_t)kKeyNegInf) return false;
    const uint32_t Q = (uint32_t)lo >> kOneIdxBits;
    const uint32_t kq = Q << kOneIdxBits;   // smallest key with prefix Q
    C4S_PHASE(2);
    // every entry whose raw prefix reaches Q, with its penalised
    // (sampling.cpp:26) and divided (:16) value
    uint32_t reach = 0u;
    auto push = [&](int id, float x) {
      float y = x;
      if (c.pen_on && ((bitmap[id >> 5] >> (id & 31)) & 1u)) y = (y < 0) ? y * c.pen : y / c.pen;
      reach += fkey(y) >= kq ? 1u : 0u;
      const float z = c.temp_on ? y / c.temp : y;
      const uint32_t slot = atomicAdd(&ts.n, 1u);
      if (slot < (uint32_t)kT2Cap) ts.list[slot] = ((uint64_t)fkey(z) << 32) | (uint32_t)~(uint32_t)id;
    };
    // A thread whose fourth candidate lies below Q holds every such entry of
    // its stream among its four; another may hold more: its wave reads that
    // thread's stream again (16-byte loads, one a lane).
    const bool redo = (t3 >> kOneIdxBits) >= Q;
    if (!redo) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (valid(tk[i]) && (tk[i] >> kOneIdxBits) >= Q) {
          const int id = id_of(tk[i]);
          push(id, xf[id]);
        }
    }
    for (uint64_t rm = __ballot(redo); rm; rm &= rm - 1) {
      const int tf = w * kWave + (__ffsll((unsigned long long)rm) - 1);
      for (int j = lane; j < iters; j += kWave) {
        const int q = tf + NT * j;
        if (q < rs.nq) {
          const float4 v = p4[q];
          const int i0 = rs.head + 4 * q;
          if ((fkey(v.x) >> kOneIdxBits) >= Q) push(i0, v.x);
          if ((fkey(v.y) >> kOneIdxBits) >= Q) push(i0 + 1, v.y);
          if ((fkey(v.z) >> kOneIdxBits) >= Q) push(i0 + 2, v.z);
          if ((fkey(v.w) >> kOneIdxBits) >= Q) push(i0 + 3, v.w);
        }
      }
      const int ef = (tf < rs.head) ? tf : ((tf < rs.head + rs.tail) ? rs.head + 4 * rs.nq + (tf - rs.head) : -1);
      if (lane == 0 && ef >= 0 && (fkey(xf[ef]) >> kOneIdxBits) >= Q) push(ef, xf[ef]);
    }
    reach = wave_sum_u32(reach);
    if (lane == 0 && reach) atomicAdd(&ts.nq, reach);
    __syncthreads();
    C4S_PHASE(3);
    const uint32_t n = ts.n, nq = ts.nq;
    if (n > (uint32_t)kT2Cap) return false;   // uniform
    if (nq >= k) {
      qkey = kq;
      return true;
    }
    // fewer than k reach Q after their penalty: a bound further down
    if (attempt == 2) return false;
    __syncthreads();   // every thread has read ts.n and ts.nq
    if (t == 0) { ts.n = 0u; ts.nq = 0u; }
    __syncthreads();
    kb *= 4u;
  }
}

// top_k, top_p and the draw on the sorted candidates ts.list[0, ts.n) (every
// entry at or above the k-th largest value among them); returns true.
__device__ __forceinline__ bool topk_finish(const RowsArgs& a, int row, const RowCfg& c, const T2Row& src, T2Sh& ts,
                            uint32_t stat_bits) {
  const int V = c.V, t = threadIdx.x, w = wave_id(), lane = lane_id();
  const float ninf = neg_inf();
  const uint32_t k = (uint32_t)c.k;
  const int n = (int)ts.n;
  // top_k: every entry with the k-th largest value or above survives
  const uint32_t kkey = (uint32_t)(ts.list[k - 1] >> 32);
  if (w == 0) {
    int ns = (int)k;
    while (ns < n && (uint32_t)(ts.list[ns] >> 32) >= kkey) ++ns;
    const float vmax = kfloat((uint32_t)(ts.list[0] >> 32));
    int nkeep = ns, tok = -2;   // -2: not decided here
    uint32_t dex = 0u;
    if (ns <= kWave) {
      // At most 64 survivors, one a lane in value order: top_p and the draw
      // with sums formed in parallel, each decision farther than rel_eps from
      // its boundary or taken by the sequential sums below (top_p) or the
      // sequential replay of lane_draw (the draw), as the candidate-list step
      // does. Survivor j's mass is exp(z_j - vmax), vmax the first survivor's.
      const bool sv = lane < ns;
      const uint64_t ent = ts.list[sv ? lane : 0];
      const float zs = sv ? kfloat((uint32_t)(ent >> 32)) : ninf;
      const int ids = (int)~(uint32_t)ent;
      const double e = sv ? exp((double)(zs - vmax)) : 0.0;
      // the sequential path for subnormal masses and below the draw's -1e30 floor
      bool ok = !__ballot(sv && e < 0x1p-1000) && !(vmax < -1e30f);
      const double thr = 1.0 - (double)c.p;
      if (ok && c.topp_on && thr >= 0.0) {
        // entry j removed iff the mass at or below it in ascending order,
        // M = S - (mass above it), is <= thr S (sampling.cpp:60-65)
        const double S = wave_sum_dpp(e);
        const double M = S - (wave_scan_f64(e) - e);
        bool rem, unsure = false;
        if (thr == 0.0) {
          rem = sv && M == 0.0;
        } else {
          const double A = thr * S;
          rem = sv && M <= A;
          unsure = sv && lane >= c.min_keep && !(fabs(M - A) > rel_eps(V) * fmax(M, A));
        }
        if (__ballot(unsure)) {
          ok = false;
        } else {
          nkeep = ns - __popcll(__ballot(rem));
          const int mk = min(max(0, c.min_keep), ns);   // sampling.cpp:67-68
          if (nkeep < mk) nkeep = mk;
        }
      }
      if (ok) {   // text2semantic.cpp:150-165 over the kept survivors in id order
        const uint64_t st2 = xorshift64(a.rng[row]);
        tok = lane_draw<19>(sv && lane < nkeep, ids, ids, e, unit_from_state(st2), V, dex);
      } else {
        nkeep = ns;
      }
    }
    if (tok == -2 && c.topp_on) {
      // sampling.cpp:52-65 in ascending order (list position ns - 1 - j)
      double total = 0.0;
      for (int base = 0; base < ns; base += kWave) {
        const int j = base + lane;
        const double e = j < ns ? exp((double)(kfloat((uint32_t)(ts.list[ns - 1 - j] >> 32)) - vmax)) : 0.0;
        total = seq_sum_lanes(total, e, min(kWave, ns - base));
      }
      const double thr = 1.0 - (double)c.p;
      double cum = 0.0;
      int removed = 0;
      bool stop = false;
      for (int base = 0; base < ns && !stop; base += kWave) {
        const int j = base + lane;
        const double q = j < ns ? exp((double)(kfloat((uint32_t)(ts.list[ns - 1 - j] >> 32)) - vmax)) / total : 0.0;
        removed = base + seq_cut_lanes(cum, q, min(kWave, ns - base), thr, stop);
      }
      nkeep = ns - removed;
      const int mk = min(max(0, c.min_keep), ns);   // sampling.cpp:67-68
      if (nkeep < mk) nkeep = mk;
    }
    if (lane == 0) {
      ts.nkeep = (uint32_t)nkeep;
      ts.tok = tok;
      ts.dex = dex;
    }
  }
  __syncthreads();
  const int nkeep = (int)ts.nkeep;
  C4S_PHASE(5);
  // the state before the draw: kept values, -inf elsewhere
  if (a.out_masked) {
    float* mrow = a.out_masked + (int64_t)row * V;
    for (int i = t; i < V; i += NT) mrow[i] = ninf;
    __syncthreads();
    for (int j = t; j < nkeep; j += NT) {   // the row's own value (the key folds -0 onto +0)
      const int i = (int)~(uint32_t)ts.list[j];
      mrow[i] = src.z(i, src.xf ? src.xf[i] : __uint_as_float((uint32_t)src.xb[i] << 16));
    }
  }
  if (ts.tok != -2) {   // drawn above
    if (t == 0) {
      const int tok = ts.tok;
      a.out_tok[row] = tok;
      a.rng[row] = xorshift64(a.rng[row]);
      join_history(a, row, tok);
      if (a.stats) {
        uint32_t* st = a.stats + 4 * (int64_t)row;
        st[0] = 1u | 2u | 4u | 32u | stat_bits;
        st[1] = 0u;
        st[2] = ts.dex;
        st[3] = (uint32_t)nkeep;
      }
    }
    return true;
  }
  // the kept entries in id order: (~id) as the high half sorts descending by it
  int Pk = 1;
  while (Pk < nkeep) Pk <<= 1;
  __syncthreads();
  const int Ps = nkeep <= kRankSortMax ? nkeep : Pk;
  for (int j = t; j < Ps; j += NT) {
    const uint64_t v = j < nkeep ? ts.list[j] : 0ull;
    ts.list[j] = j < nkeep ? (((uint64_t)(uint32_t)v << 32) | (v >> 32)) : 0ull;
  }
  __syncthreads();
  if (nkeep <= kRankSortMax) rank_sort_desc_u64(ts.list, reinterpret_cast<uint64_t*>(ts.e), nkeep);
  else bitonic_desc_u64(ts.list, Pk);
  C4S_PHASE(6);
  if (w == 0) {
    // text2semantic.cpp:150-165 over the kept entries in id order (the maximum
    // starts from -1e30f; -inf positions add 0)
    float m = -1e30f;
    for (int j = lane; j < nkeep; j += kWave) m = fmaxf(m, kfloat((uint32_t)ts.list[j]));
    m = wave_max_f32(m);
    double total = 0.0;
    for (int base = 0; base < nkeep; base += kWave) {
      const int j = base + lane;
      const float zj = j < nkeep ? kfloat((uint32_t)ts.list[j]) : ninf;
      const double e = (j < nkeep && zj != ninf) ? exp((double)(zj - m)) : 0.0;
      if (j < nkeep) ts.e[j] = e;
      total = seq_sum_lanes(total, e, min(kWave, nkeep - base));
    }
    const uint64_t st2 = xorshift64(a.rng[row]);
    const double r = unit_from_state(st2) * total;
    int tok = V - 1;   // no id reached r (text2semantic.cpp:160)
    double acc = 0.0;
    bool done = false;
    for (int base = 0; base < nkeep && !done; base += kWave) {
      const int j = base + lane;
      const double e = j < nkeep ? ts.e[j] : 0.0;
      const int q = seq_find_lanes(acc, e, min(kWave, nkeep - base), r);
      if (q >= 0) {
        tok = (int)~(uint32_t)(ts.list[base + q] >> 32);
        done = true;
      }
    }
    if (lane == 0) {
      a.out_tok[row] = tok;
      a.rng[row] = st2;
      join_history(a, row, tok);
      if (a.stats) {
        uint32_t* st = a.stats + 4 * (int64_t)row;
        st[0] = 1u | 2u | 4u | 32u | stat_bits;
        st[1] = 0u;
        st[2] = 0u;
        st[3] = (uint32_t)nkeep;
      }
    }
  }
  C4S_PHASE(7);
  return true;
}

// Returns false (nothing written) when the survivors' bucket holds more than
// the sort takes; the multi-pass chain decides the row then.
__device__ __forceinline__ bool topk_two_pass(const RowsArgs& a, int row, const RowCfg& c, const T2Row& src, T2Sh& ts,
                                              const OneFirst& first) {
  const int V = c.V, t = threadIdx.x, w = wave_id(), lane = lane_id();
  const float ninf = neg_inf();
  const uint32_t k = (uint32_t)c.k;
  // one read of the row when its checks pass
  uint32_t qkey = 0u;
  bool one = src.xf && V <= kOneMaxV && (!c.pen_on || c.pen >= 1.0f) &&
             topk_one_read(a, c, src.xf, src.bitmap, ts, qkey, first);
  if (one) {
    const int n = (int)ts.n;
    if (n <= kRankSortMax) {
      rank_sort_desc_u64(ts.list, reinterpret_cast<uint64_t*>(ts.e), n);   // the draw's masses come later
    } else {
      int P = 1;
      while (P < n) P <<= 1;
      for (int i = n + t; i < P; i += NT) ts.list[i] = 0ull;
      __syncthreads();
      bitonic_desc_u64(ts.list, P);
    }
    C4S_PHASE(4);
    // no value below the bound ties the k-th quotient (the largest of them, divided)
    if (c.temp_on && !(fkey(kfloat(qkey - 1u) / c.temp) < (uint32_t)(ts.list[k - 1] >> 32))) one = false;
  }
  if (one) return topk_finish(a, row, c, src, ts, 64u);
  __syncthreads();   // the work area is free again
  for (int i = t; i < kT2Copies * kT2Buckets; i += NT) (&ts.hist[0][0])[i] = 0u;
  if (t == 0) ts.n = 0u;
  __syncthreads();
  // pass 1: maximum and histogram
  uint32_t* hist = ts.hist[w % kT2Copies];
  float lmax = ninf;
  src.each(V, [&](int, float zi) {
    lmax = fmaxf(lmax, zi);
    atomicAdd(&hist[fkey(zi) >> (32 - kT2Bits)], 1u);
  });
  lmax = wave_max_f32(lmax);
  if (lane == 0) ts.wmax[w] = lmax;
  __syncthreads();
  // b*: thread t takes buckets 2047 - 2t (higher) and 2046 - 2t; counts from the top
  const int bh = kT2Buckets - 1 - 2 * t, bl = bh - 1;
  uint32_t ch = 0, cl = 0;
#pragma unroll
  for (int q = 0; q < kT2Copies; ++q) { ch += ts.hist[q][bh]; cl += ts.hist[q][bl]; }
  const uint32_t inc = wave_scan_u32(ch + cl);
  if (lane == kWave - 1) ts.wsum[w] = inc;
  __syncthreads();
  uint32_t ex = inc - (ch + cl);
  for (int i = 0; i < w; ++i) ex += ts.wsum[i];
  if (ex < k && k <= ex + ch) { ts.bstar = bh; ts.nge = ex + ch; }
  else if (ex + ch < k && k <= ex + ch + cl) { ts.bstar = bl; ts.nge = ex + ch + cl; }
  __syncthreads();
  const int bstar = ts.bstar;
  const uint32_t nge = ts.nge;
  if (nge > (uint32_t)kT2Cap) return false;   // uniform
  // pass 2: the candidates (bucket >= b*)
  src.each(V, [&](int i, float zi) {
    const uint32_t key = fkey(zi);
    if ((int)(key >> (32 - kT2Bits)) >= bstar) {
      const uint32_t slot = atomicAdd(&ts.n, 1u);
      ts.list[slot] = ((uint64_t)key << 32) | (uint32_t)~(uint32_t)i;
    }
  });
  __syncthreads();
  const int n = (int)ts.n;   // == nge
  int P = 1;
  while (P < n) P <<= 1;
  for (int i = n + t; i < P; i += NT) ts.list[i] = 0ull;
  __syncthreads();
  bitonic_desc_u64(ts.list, P);
  return topk_finish(a, row, c, src, ts, 0u);
}

__global__ __launch_bounds__(NT) void k_rows_global(RowsArgs a) {
  C4S_PHASE(14);
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ Scratch sh;
  const int row = blockIdx.x;
  const int V = a.vocab;
  // the row's flags and parameters by scalar loads, all issued before any
  // waits for them (a byte flag read as its aligned word: flag_byte)
  const bool act = a.row_active ? flag_byte(a.row_active, row) : true;
  const bool sample = a.do_sample ? flag_byte(a.do_sample, row) : true;
  const float pv = a.pen ? a.pen[row] : 1.0f, tv = a.temp ? a.temp[row] : 1.0f;
  const int32_t kv = a.top_k ? a.top_k[row] : 0, mv = a.min_keep ? a.min_keep[row] : 1;
  const float ppv = a.top_p ? a.top_p[row] : 1.0f;
  if (!act) {
    if (threadIdx.x == 0) a.out_tok[row] = -1;
    return;
  }
  const RowCfg c = make_cfg_vals(a.mode, V, pv, tv, kv, ppv, mv, (a.mode & kCustom) || sample);
  const int64_t roff = (int64_t)row * a.ld;
  // The history's first ids (four a thread), then, for a row that the top-k
  // read takes, that read's first loads: in flight during the set-up (loads
  // complete in issue order, so the ids come first)
  constexpr int kPreIds = 4;
  const bool csr = c.pen_on && !a.hist_bits;
  const int64_t h0 = csr ? a.hist_off[row] : 0, h1 = csr ? a.hist_off[row + 1] : 0;
  int hid[kPreIds];
  {
    const int nb = (int)min(h1 - h0, (int64_t)NT * kPreIds) * 4;   // the first ids' bytes
    const __amdgpu_buffer_rsrc_t r = raw_rsrc(csr ? a.hist_ids + h0 : a.out_tok, nb);
#pragma unroll
    for (int i = 0; i < kPreIds; ++i) {
      const int jo = threadIdx.x + NT * i;
      const int id = __builtin_amdgcn_raw_buffer_load_b32(r, 4 * jo, 0, 0);
      hid[i] = 4 * jo < nb ? id : -1;
    }
  }
  const bool one_row = c.draw && c.topk_on && c.k <= kT2MaxK && V <= kT2MaxV && a.rng && a.dtype == 0 &&
                       V <= kOneMaxV && (!c.pen_on || c.pen >= 1.0f);
  OneFirst first;
  one_first(static_cast<const float*>(a.logits) + (one_row ? roff : 0), V, one_row, first);
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(smem);
  const int nw = (V + 31) / 32;
  for (int w = threadIdx.x; w < nw; w += NT) bitmap[w] = 0u;
  __syncthreads();
  if (c.pen_on) {
    if (a.hist_bits) {   // the history set kept across steps
      const uint32_t* hb = a.hist_bits + (int64_t)row * hist_words(V);
      for (int w = threadIdx.x; w < nw; w += NT) bitmap[w] = hb[w];
    } else {
#pragma unroll
      for (int i = 0; i < kPreIds; ++i)
        if (hid[i] >= 0 && hid[i] < V) atomicOr(&bitmap[hid[i] >> 5], 1u << (hid[i] & 31));
      for (int64_t j = h0 + threadIdx.x + (int64_t)NT * kPreIds; j < h1; j += NT) {
        const int id = a.hist_ids[j];
        if (id < 0 || id >= V) continue;
        atomicOr(&bitmap[id >> 5], 1u << (id & 31));
      }
    }
    __syncthreads();
  }
  C4S_PHASE(0);
  if (c.draw && c.topk_on && c.k <= kT2MaxK && V <= kT2MaxV && a.rng) {
    T2Row tr;
    tr.xf = a.dtype == 0 ? static_cast<const float*>(a.logits) + roff : nullptr;
    tr.xb = a.dtype == 1 ? static_cast<const uint16_t*>(a.logits) + roff : nullptr;
    tr.bitmap = bitmap;
    tr.pen_on = c.pen_on;
    tr.pen = c.pen;
    tr.temp_on = c.temp_on;
    tr.temp = c.temp;
    tr.rpen = 1.0 / (double)c.pen;
    tr.rtemp = 1.0 / (double)c.temp;
    if (topk_two_pass(a, row, c, tr, *reinterpret_cast<T2Sh*>(smem + t2_offset(V)), first)) return;
    __syncthreads();
  }
  GlobalRow src;
  src.xf = a.dtype == 0 ? static_cast<const float*>(a.logits) + roff : nullptr;
  src.xb = a.dtype == 1 ? static_cast<const uint16_t*>(a.logits) + roff : nullptr;
  src.V = V;
  src.bitmap = bitmap;
  src.pen_on = c.pen_on;
  src.pen = c.pen;
  src.temp_on = false;
  src.temp = 1.0f;
  src.thr_key = 0u;
  src.topk_on = false;
  src.sortbuf = a.sort_ws + (int64_t)row * a.sort_ws_stride;
  src.sortcap = (uint32_t)(a.sort_ws_stride * 4);
  uint64_t rng = a.rng ? a.rng[row] : 0ull;
  float* masked = a.out_masked ? a.out_masked + (int64_t)row * V : nullptr;
  uint32_t* st = a.stats ? a.stats + 4 * (int64_t)row : nullptr;
  const int tok = run_chain(src, sh, c, rng, masked, st);
  if (threadIdx.x == 0) {
    a.out_tok[row] = tok;
    if (c.draw && a.rng) a.rng[row] = rng;
    join_history(a, row, tok);
  }
}

// hist_bits[b] = the ids in [0, V) of row b's CSR history (sampling.cpp:24).
__global__ __launch_bounds__(NT) void k_hist_bits_init(const int32_t* ids, const int64_t* off, int V,
                                                       uint32_t* bits) {
  const int row = blockIdx.x;
  const int W = hist_words(V);
  uint32_t* b = bits + (int64_t)row * W;
  for (int w = threadIdx.x; w < W; w += NT) b[w] = 0u;
  __syncthreads();
  if (!ids) return;
  for (int64_t j = off[row] + threadIdx.x; j < off[row + 1]; j += NT) {
    const int id = ids[j];
    if (id >= 0 && id < V) atomicOr(&b[id >> 5], 1u << (id & 31));
  }
}

// Multi-step AR stream for rows staged in LDS: one persistent workgroup per
// row walks all steps. The row's distinct penalised ids live in an LDS bitmap
// that gains every sampled token that is not the stop token
// (text2semantic.cpp:333-334). While step s runs, the logits of step s+1 are
// already in flight into registers. A stopped row reports -1 afterwards and its
// RNG stays frozen.
__global__ __launch_bounds__(NT) void k_stream_lds(StreamArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ Scratch sh;
  const int row = blockIdx.x;
  const int V = a.vocab;
  const RowCfg c = make_cfg(0u, V, row, a.temp, a.top_k, a.top_p, a.pen, nullptr, a.do_sample);
  LdsLayout L = lds_layout(smem, V);
  const int nw = bitmap_words(V);
  for (int w = threadIdx.x; w < nw; w += NT) L.bitmap[w] = 0u;
  __syncthreads();
  {
    const int64_t h0 = a.hist_off[row], h1 = a.hist_off[row + 1];
    for (int64_t j = h0 + threadIdx.x; j < h1; j += NT) {
      const int id = a.hist_ids[j];
      if (id < 0 || id >= V) continue;
      atomicOr(&L.bitmap[id >> 5], 1u << (id & 31));
    }
  }
  uint64_t rng = a.rng[row];
  bool done = false;
  uint32_t acc_stats[4] = {0, 0, 0, 0};
  const float* base = a.logits + (int64_t)row * a.ld;
  RowFetch pf;
  fetch_row(base, V, pf);
  for (int s = 0; s < a.n_steps; ++s) {
    int32_t* outp = a.out_tok + (int64_t)s * a.n_rows + row;
    if (done) {
      if (threadIdx.x == 0) *outp = -1;
      continue;
    }
    C4S_PHASE(0);
    const float* cur = base + (int64_t)s * a.step_stride;
    float* val = store_row(cur, V, pf, L.val);
    if (s + 1 < a.n_steps) fetch_row(cur + a.step_stride, V, pf);
    __syncthreads();
    if (c.pen_on) {
      penalise_chunk(val, L.bitmap, V, c.pen);
      __syncthreads();
    }
    C4S_PHASE(1);
    LdsRow src{val, L.E, V, 0u, false};
    uint32_t* st = a.stats ? sh.step_stats : nullptr;   // written and read by thread 0 only
    int tok = 0;
    if (!(fast_topk_applies(c, V) &&
          fast_topk_any(val, V, c, sh, reinterpret_cast<unsigned char*>(L.E), rng, tok, nullptr, st)))
      tok = run_chain(src, sh, c, rng, nullptr, st);
    C4S_PHASE(8);
    if (threadIdx.x == 0) {
      *outp = tok;
      if (a.stats) {
        acc_stats[0] |= st[0];
        acc_stats[1] += st[1];
        acc_stats[2] += st[2];
        acc_stats[3] += st[3];
      }
      // Appending a token already in the history changes nothing: the penalty
      // applies once per distinct id (sampling.cpp:22).
      if (tok != a.stop_token && tok >= 0 && tok < V) L.bitmap[tok >> 5] |= 1u << (tok & 31);
    }
    if (tok == a.stop_token) done = true;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    a.rng[row] = rng;
    if (a.stats) {
      uint32_t* o = a.stats + 4 * (int64_t)row;
      o[0] = acc_stats[0]; o[1] = acc_stats[1]; o[2] = acc_stats[2]; o[3] = acc_stats[3];
    }
  }
}

}  // namespace

size_t rows_lds_bytes(int V) {
  const size_t vp = (size_t)((V + 3) & ~3);
  return 8 * vp + 4 * (vp + 4) + 4 * (size_t)bitmap_words(V);
}

size_t stream_lds_bytes(int V, int) { return rows_lds_bytes(V); }

size_t rows_global_lds_bytes(int V) {
  return V <= kT2MaxV ? t2_offset(V) + sizeof(T2Sh) : 4 * (size_t)((V + 31) / 32);
}

size_t rows_step_lds_bytes(int V) {
  return step_work_bytes(V) + 4 * ((size_t)vpad(V) + 4) + 4 * (size_t)bitmap_words(V);
}

hipError_t launch_hist_bits_init(const int32_t* ids, const int64_t* off, int n_rows, int V, uint32_t* bits,
                                 hipStream_t s) {
  if (n_rows <= 0) return hipSuccess;
  (void)hipGetLastError();
  hipLaunchKernelGGL(k_hist_bits_init, dim3(n_rows), dim3(NT), 0, s, ids, off, V, bits);
  return hipGetLastError();
}

hipError_t launch_rows(const RowsArgs& a, hipStream_t s) {
  if (a.n_rows <= 0) return hipSuccess;
  (void)hipGetLastError();  // report only this launch's status
  if (a.vocab <= kLdsVocabMax && a.mode == 0u) {
    const size_t lds = rows_step_lds_bytes(a.vocab);
    const int P = ((a.vocab + kStepThreads - 1) / kStepThreads) | 1;   // ids a thread owns (odd_chunk)
    const dim3 g(a.n_rows), b(kStepThreads);
    if (P <= 9) hipLaunchKernelGGL(k_rows_step<9>, g, b, lds, s, a);
    else if (P <= 17) hipLaunchKernelGGL(k_rows_step<17>, g, b, lds, s, a);
    else hipLaunchKernelGGL(k_rows_step<25>, g, b, lds, s, a);
  } else if (a.vocab <= kLdsVocabMax) {
    const size_t lds = rows_lds_bytes(a.vocab);
    hipLaunchKernelGGL(k_rows_lds, dim3(a.n_rows), dim3(NT), lds, s, a);
  } else {
    const size_t lds = rows_global_lds_bytes(a.vocab);
    hipLaunchKernelGGL(k_rows_global, dim3(a.n_rows), dim3(NT), lds, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_stream(const StreamArgs& a, hipStream_t s) {
  if (a.n_rows <= 0 || a.n_steps <= 0) return hipSuccess;
  (void)hipGetLastError();
  const size_t lds = stream_lds_bytes(a.vocab, 0);
  hipLaunchKernelGGL(k_stream_lds, dim3(a.n_rows), dim3(NT), lds, s, a);
  return hipGetLastError();
}

}  // namespace c4s
