// Candidate lists of the token-sampling step: the list entry format, the
// summary header, and the decision of a greedy or top-k step on its list
// (list_step), shared by the AR stream (every step of a call) and the
// per-call step (one step, no ids drawn since the list was made).
#pragma once

#include "c4s_chain.hpp"

namespace c4s {
namespace {

// LDS writes of this wave visible to its own later reads (all lanes).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bool bit_of(const uint32_t* bm, int id) {
  return (bm[id >> 5] >> (id & 31)) & 1u;
}

__device__ __forceinline__ float pen_exact(float s, float pen) {
  return (s < 0) ? s * pen : s / pen;   // sampling.cpp:26
}

struct SumHdr {
  int n;            // list entries
  uint32_t tout;    // key bound on every value outside the list (0: nothing outside)
  uint32_t flags;   // bit 0: unusable (candidate overflow or empty list)
  float m0;         // chunk masses are exp(z - m0)
  int nchunk;
  int head;         // ids before the first 16-byte boundary of the row
  double err;       // absolute error bound of the chunk masses, summed over the row
  double s0;        // sum of the chunk masses
  int qhint;        // nucleus rows: kLanesHint (or 256) when the cut without hits and corrections
                    // lies within that many first entries, else kListLarge (a hint)
  int pad[5];
};
static_assert(sizeof(SumHdr) == kSumHdrBytes, "summary header size");

// List entry: key of z = fl(y / T) (y itself on the greedy path), then the id
// and an id-order rank (while the scan sorts: the candidate's position; in a
// summary: the rank among the list's entries); larger entries come first
// (z desc, id asc), which is the declared top_p order of equal values.
__device__ __forceinline__ uint64_t make_entry(float y, int id, int rank) {
  return ((uint64_t)fkey(y) << 32) | ((uint32_t)(16383 - id) << 10) | (uint32_t)rank;
}
__device__ __forceinline__ uint32_t ent_key(uint64_t e) { return (uint32_t)(e >> 32); }
__device__ __forceinline__ int ent_id(uint64_t e) { return 16383 - (int)(((uint32_t)e >> 10) & 16383u); }
__device__ __forceinline__ int ent_rank(uint64_t e) { return (int)((uint32_t)e & 1023u); }

constexpr int kSlotBits = 9;   // summary slots are below kListLarge
static_assert((1 << kSlotBits) == kListLarge, "slot bits cover the list");

struct StepOut {
  int tok;
  uint32_t kept;
  uint32_t dex;
  uint32_t why;     // reason of a fallback to the exact step (bit index, see kWhy*)
  uint32_t nsurv;   // list_step: top-k survivors (their ids in cs.lid)
};

// Fallback reasons, reported as bit 20 + reason in the per-row path statistics.
enum : uint32_t {
  kWhySummary = 0,    // summary unusable (candidate overflow, empty list)
  kWhyBound = 1,      // a value outside the list may reach the decision
  kWhyShort = 2,      // too few candidates left after the penalty
  kWhyHit = 3,        // a penalised candidate stays above the threshold
  kWhyTies = 4,       // equal values out of id order, or ties at a boundary
  kWhyMargin = 5,     // top_p decision inside the error bound
  kWhyDeep = 6,       // nucleus cut below the candidate list
  kWhyDraw = 7,       // dense draw inside the error bound
  kWhyTiny = 8,       // subnormal masses
};

struct LSpecCS {   // list_step's survivor arrays
  float lz[kWave + 1];
  int lid[kWave + 1];
  int lslot[kWave + 1];
};

// Drawn-id set as a bitmap (hit test of list_step).
struct BitsHit {
  const uint32_t* bm;
  __device__ __forceinline__ bool hit(int id) const { return bit_of(bm, id); }
};

// Candidate-list step for greedy and top-k rows (one wave; two entries per
// lane: keys e0, e1 and their values before the temperature yb0, yb1).
// Returns false (nothing changed) when a decision needs the exact step. The
// entries' rank fields order them by id (kSB bits); kNoHits: the hit test is
// never true (no id drawn since the list was made).
template <int kSB = kSlotBits, bool kNoHits = false, class Hit, class CS>
__device__ __forceinline__ bool list_step(const SumHdr& h, uint64_t e0, uint64_t e1, float yb0, float yb1,
                          const RowCfg& c, int V, const Hit& hs, uint64_t& rng, CS& cs,
                          StepOut& o) {
  const int lane = lane_id();
  o.why = kWhySummary;
  if (h.flags & 1u) return false;
  const int n = h.n;
  const float ninf = neg_inf();
  const bool v0 = lane < n, v1 = lane + kWave < n;
  const int id0 = ent_id(e0), id1 = ent_id(e1);
  const bool h0 = c.pen_on && v0 && hs.hit(id0);
  const bool h1 = c.pen_on && v1 && hs.hit(id1);
  // z of an unhit entry is its key; a hit is penalised (sampling.cpp:26) and divided again
  float z0 = v0 ? kfloat(ent_key(e0)) : ninf, z1 = v1 ? kfloat(ent_key(e1)) : ninf;
  if (h0) { const float y = pen_exact(yb0, c.pen); z0 = c.temp_on ? y / c.temp : y; }
  if (h1) { const float y = pen_exact(yb1, c.pen); z1 = c.temp_on ? y / c.temp : y; }
  C4S_LIST_PHASE(2);

  if (c.greedy) {   // text2semantic.cpp:144-145, argmax of the penalised row, first max wins
    const uint64_t k0 = v0 ? ((uint64_t)fkey(z0) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)id0) : 0ull;
    const uint64_t k1 = v1 ? ((uint64_t)fkey(z1) << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)id1) : 0ull;
    const uint64_t kb = wave_max_u64_dpp(k0 > k1 ? k0 : k1);
    o.why = kWhyBound;
    if (kb == 0ull || !((uint32_t)(kb >> 32) > h.tout)) return false;
    o.tok = (int)(0xFFFFFFFFu - (uint32_t)kb);
    o.kept = 1;
    o.dex = 0;
    return true;
  }

  // top-k on the unhit entries (sorted by z desc, id asc); hits must fall below the k-th
  const bool u0 = v0 && !h0, u1 = v1 && !h1;
  const uint64_t b0 = __ballot(u0), b1 = __ballot(u1);
  const int r0 = __popcll(b0 & lanemask_lt());
  const int r1 = __popcll(b0) + __popcll(b1 & lanemask_lt());
  const int nu = __popcll(b0) + __popcll(b1);
  const int k = c.k;
  o.why = kWhyShort;
  if (nu < k) return false;
  const uint64_t mk0 = __ballot(u0 && r0 == k - 1), mk1 = __ballot(u1 && r1 == k - 1);
  const float zk = mk0 ? readlane_f32(z0, __ffsll((unsigned long long)mk0) - 1)
                       : readlane_f32(z1, __ffsll((unsigned long long)mk1) - 1);
  if constexpr (!kNoHits) {
    float zh = ninf;
    if (h0) zh = z0;
    if (h1) zh = fmaxf(zh, z1);
    zh = wave_max_dpp(zh);
    o.why = kWhyHit;
    if (!(zh < zk) && zh != ninf) return false;
  }
  o.why = kWhyBound;
  if (!(zk > ninf)) return false;
  if (h.tout != 0u && !(kfloat(h.tout) < zk)) return false;   // everything outside stays below
  const bool s0 = u0 && z0 >= zk, s1 = u1 && z1 >= zk;
  C4S_LIST_PHASE(3);
  const int nsurv = __popcll(__ballot(s0)) + __popcll(__ballot(s1));
  o.why = kWhyTies;
  if (nsurv > kWave) return false;
  o.nsurv = (uint32_t)nsurv;
  // survivors are the unhit ranks [0, nsurv): one per lane in rank order
  const bool sv = lane < nsurv;
  float zs;
  int ids, slot;
  if constexpr (kNoHits) {   // every entry unhit: the survivors are lanes [0, nsurv) of e0 already
    zs = sv ? z0 : ninf;
    ids = sv ? id0 : 0;
    slot = sv ? ent_rank(e0) : 0;
  } else {
    if (s0) { cs.lz[r0] = z0; cs.lid[r0] = id0; cs.lslot[r0] = ent_rank(e0); }
    if (s1) { cs.lz[r1] = z1; cs.lid[r1] = id1; cs.lslot[r1] = ent_rank(e1); }
    wave_sync();
    zs = sv ? cs.lz[lane] : ninf;
    ids = sv ? cs.lid[lane] : 0;
    slot = sv ? cs.lslot[lane] : 0;
  }
  C4S_LIST_PHASE(4);
  // masses, top_p (sampling.cpp:52-65), min_keep (:67-68)
  const float zmax = readlane_f32(zs, 0);
  const double e = sv ? exp((double)(zs - zmax)) : 0.0;
  const double S = wave_sum_dpp(e);
  const double above = wave_scan_f64(e) - e;
  const double M = S - above;
  const double thr = 1.0 - (double)c.p;
  const double eps = rel_eps(V);
  bool rem = false, unsure = false;
  if (c.topp_on && thr >= 0.0) {
    if (thr == 0.0) {
      rem = sv && M == 0.0;
    } else {
      const double A = thr * S;
      rem = sv && M <= A;
      unsure = sv && !(fabs(M - A) > eps * fmax(M, A));
    }
  }
  o.why = __ballot(sv && e < 0x1p-1000) ? kWhyTiny : kWhyMargin;
  unsure = (unsure && lane >= c.min_keep) || (sv && e < 0x1p-1000);
  if (__ballot(unsure)) return false;
  const long long R = (long long)(V - nsurv) + (long long)__popcll(__ballot(rem));
  const long long lim = (long long)V - (long long)c.min_keep < 0 ? 0 : (long long)V - (long long)c.min_keep;
  const long long m = (long long)V - (R < lim ? R : lim);
  const bool kept = sv && (long long)lane < m;
  const uint64_t st = xorshift64(rng);
  C4S_LIST_PHASE(5);
  o.tok = lane_draw<kSB>(kept, ids, slot, e, unit_from_state(st), V, o.dex);
  C4S_LIST_PHASE(6);
  o.kept = (uint32_t)__popcll(__ballot(kept));
  rng = st;
  return true;
}

}  // namespace
}  // namespace c4s
