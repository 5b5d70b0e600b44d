// Two-phase AR token stream for rows staged in LDS (vocab <= 12288).
//
// The stream of text2semantic.cpp:296-337 is sequential only through the
// generated history: step s penalises H0 + {tokens of steps < s}
// (sampling.cpp:19-28, text2semantic.cpp:333-334), while its logits are given
// and its RNG advances once per sampled step whatever was drawn
// (text2semantic.cpp:158). So the bulk of the work is split off:
//
//  scan  (k_stream_scan, every (step, row) independently)
//        reads the row once from HBM, applies the initial history H0 and writes
//        a summary: the top of the row sorted by (value desc, id asc), a key
//        bound on everything left out, and, for rows without top-k, the chunk
//        masses exp((double)fl(z - m0)) of the whole row in 64-id chunks, their
//        sum, the list entries' fp32 masses, a cut hint and the first 256
//        entries' id-order places.
//  chains (one per row, steps in order) apply the penalty of ids drawn during
//        the stream to the summary (only those ids change), then decide top-k /
//        top-p / the draw on the candidates: k_stream_list (greedy and top-k
//        rows, one wave), k_stream_rowp (full-vocabulary rows, a CU each,
//        pipelined with helper waves; rows without penalty in step segments
//        settled by k_stream_segfix), k_stream_chain (the exact chain, for
//        rows the fast chains do not take). Every decision is accepted only
//        with a margin larger than the error bounds; otherwise the step runs
//        the exact chain on the full row staged in LDS. Vocabularies whose
//        pipelined chain does not fit in LDS take the single-kernel stream.
//
// Row modes (stream_mode): greedy rows and top-k rows with k <= 64 use the
// candidate list alone; full-vocabulary rows (top-k off) also use the chunk
// masses and stream their raw row into LDS for the few corrections; rows whose
// penalty can raise values (penalty < 1) take the exact chain every step.

#include "c4s_list.hpp"

namespace c4s {
namespace {


constexpr int NTA = 256;
constexpr int kLanesHint = 48;   // nucleus cuts within this many entries take the chain's register path
constexpr int NWA = NTA / kWave;
constexpr float kLog2e = 1.44269504088896340736f;

enum : int { kModeExact = 0, kModeList = 1, kModeRow = 2 };

__device__ __forceinline__ int stream_mode(const RowCfg& c, int V) {
  if (!(c.pen >= 1.0f) || V > kLdsVocabMax) return kModeExact;   // pen < 1 raises values
  if (c.greedy) return kModeList;
  if (!c.draw) return kModeExact;
  if (c.topk_on) return c.k <= 64 ? kModeList : kModeExact;
  return kModeRow;
}

__device__ __forceinline__ int list_cap(const RowCfg& c) {
  return (!c.greedy && !c.topk_on && c.p > 0.0f && c.p < 1.0f) ? kListLarge : kListSmall;
}


// Summary words: list entries [0, kListLarge); from kYW one float per entry:
// its value before the temperature (greedy and top-k rows) or its mass
// exp((double)fl(z - m0)) rounded to fp32 (full-vocabulary rows); header
// [kHdrW, kHdrW + 8); chunk masses from kChunkW; from kPlaceW (full-vocabulary
// rows) one byte per entry of the list's first NTA: its id-order place among
// them. List entry i sits in lane i % 64 of a wave's i / 64-th load, so list
// rows read their entries straight into registers.
constexpr int kYW = kListLarge;
constexpr int kHdrW = kYW + kListLarge / 2;
constexpr int kChunkW = kHdrW + kSumHdrBytes / 8;
constexpr int kPlaceW = kChunkW + kMaxChunks;
constexpr int kSumWords = kPlaceW + NTA / 8;
static_assert(NTA <= 256, "places fit a byte");
static_assert((size_t)kSumWords * 8 <= kSumStride, "summary fits its stride");

__device__ __forceinline__ const uint64_t* sum_words(const StreamWs& w, int n_rows, int s, int row) {
  return reinterpret_cast<const uint64_t*>(w.sum + ((size_t)(s - w.s_begin) * n_rows + row) * kSumStride);
}

// Approximate masses: exp(fl(y/T) - m0) as exp2(y*a - b) (v_exp_f32). Against
// the reference's exp((double)fl(fl(y/T) - m0)) its relative error is below
// (4|m0| + 4|t| + 8) * 2^-23: rounding of the quotient and of the difference
// (<= 2^-24 (|z| + |d|) each), of a, b and the fma, and a few ulp of v_exp_f32.
struct MassCoef {
  float a, b, relc;
};
__device__ __forceinline__ MassCoef mass_coef(const RowCfg& c, float m0) {
  MassCoef k;
  k.a = c.temp_on ? kLog2e / c.temp : kLog2e;
  k.b = m0 * kLog2e;
  k.relc = 4.0f * fabsf(m0) + 8.0f;
  return k;
}
__device__ __forceinline__ float mass_approx(float y, const MassCoef& k, float& err) {
  const float t = fmaf(y, k.a, -k.b);
  const float e = __builtin_amdgcn_exp2f(t);
  err = e * (k.relc + 4.0f * fabsf(t)) * 0x1p-23f;
  return e;
}
// The reference's mass of value y: exp((double)fl(fl(y/T) - m0)) (sampling.cpp:55).
__device__ __forceinline__ double mass_exact(float y, const RowCfg& c, float m0) {
  const float z = c.temp_on ? y / c.temp : y;
  return exp((double)(z - m0));
}
// Penalised value for a mass only (x / pen within 2 ulp).
__device__ __forceinline__ float pen_approx(float x, float pen, float rpen) {
  return (x < 0) ? x * pen : x * rpen;
}

__device__ __forceinline__ int chunk_of(int id, int head, int nchunk) {
  return id < head ? 0 : min(nchunk - 1, (id - head) >> 6);
}


// ---- scan (all CUs) -----------------------------------------------------------------

constexpr int kIdWords = (kLdsVocabMax / 32 + 1 + 3) & ~3;   // bitmap_words(kLdsVocabMax)
static_assert(kIdWords <= 2 * NTA, "two id-bitmap words a thread");

struct ScanSh {
  uint32_t hist[2048];
  uint64_t cand[kCandCap];
  float candy[kCandCap];   // value before the temperature, by candidate position
  uint32_t bm[kStateWords];
  uint32_t red[NWA];
  uint32_t redm[NWA];
  double redd[NWA];
  double chunk[kMaxChunks];
  double edge[8];
  uint32_t bu[4];
  double redh[NWA];                // per wave: mass of its list positions below NTA
  uint32_t lmark[kIdWords];        // ids of the list entries
  uint32_t fmark[kIdWords];        // ids of the list's first NTA entries
  uint32_t pre2[kIdWords];         // marks before each word: lmark's (low half), fmark's (high half)
  uint32_t place4[NTA / 4];        // their id-order places, a byte each, stored as words
};

// Block exclusive scan over the NTA threads (thread order).
__device__ __forceinline__ uint32_t scan_excl_nta(uint32_t v, uint32_t* red, uint32_t& total) {
  const uint32_t inc = wave_scan_u32(v);
  if (lane_id() == kWave - 1) red[wave_id()] = inc;
  __syncthreads();
  uint32_t pre = 0;
  total = 0;
#pragma unroll
  for (int w = 0; w < NWA; ++w) {
    const uint32_t x = red[w];
    pre += (w < wave_id()) ? x : 0u;
    total += x;
  }
  __syncthreads();
  return pre + inc - v;
}

// Bin (of 2048, scanned from the top) holding the m-th largest counted key.
// Returns false when fewer than m keys were counted.
__device__ bool hist_pick(ScanSh& sh, uint32_t m, uint32_t& bin, uint32_t& above) {
  const int t = threadIdx.x;
  uint32_t c[8], loc = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) { c[i] = sh.hist[2047 - 8 * t - i]; loc += c[i]; }
  uint32_t total;
  const uint32_t ex = scan_excl_nta(loc, sh.red, total);
  if (total < m) return false;
  if (ex < m && ex + loc >= m) {
    uint32_t run = ex;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (run < m && run + c[i] >= m) { sh.bu[0] = 2047 - 8 * t - i; sh.bu[1] = run; }
      run += c[i];
    }
  }
  __syncthreads();
  bin = sh.bu[0];
  above = sh.bu[1];
  __syncthreads();
  return true;
}

// Descending block bitonic sort of P (power of two) 64-bit entries in LDS.
// Descending bitonic sort of v[0, P), P a power of two >= 2 NWA. A stage
// whose pairs lie within 2 j <= P / NWA consecutive elements is run by each
// wave on its own quarter of v, wave-synchronous; only the longer stages
// need the workgroup barrier.
__device__ void bitonic_desc_u64(uint64_t* v, int P) {
  const int per_wave = P / NWA;
  const int wpairs = per_wave >> 1;
  const int lane = lane_id(), wv = wave_id();
  auto cmpswap = [&](int i, int j, int k) __attribute__((always_inline)) {
    const int lo = ((i & ~(j - 1)) << 1) | (i & (j - 1));
    const int hi = lo + j;
    const uint64_t x = v[lo], y = v[hi];
    if ((x < y) == ((lo & k) == 0)) { v[lo] = y; v[hi] = x; }
  };
  bool wave_stage = false;   // the last stage ran wave-locally
  for (int k = 2; k <= P; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (2 * j <= per_wave) {
        for (int i = lane; i < wpairs; i += kWave) cmpswap(wv * wpairs + i, j, k);
        wave_sync();
        wave_stage = true;
      } else {
        if (wave_stage) __syncthreads();
        for (int i = threadIdx.x; i < (P >> 1); i += NTA) cmpswap(i, j, k);
        __syncthreads();
        wave_stage = false;
      }
    }
  if (wave_stage) __syncthreads();
}


// One workgroup scans steps [s0, s1) of one row (ONE: exactly one step, so
// that nothing is hoisted out of a loop that runs once). Thread t holds the
// float4 quads t + 256 j of the 16-byte aligned body and one head or tail id.
template <int NQ, bool ONE>
__global__ __launch_bounds__(NTA, 3) void k_stream_scan(StreamArgs a, StreamWs w) {
  __shared__ ScanSh sh;
  const int row = blockIdx.y;
  const int V = a.vocab;
  const RowCfg c = make_cfg(0u, V, row, a.temp, a.top_k, a.top_p, a.pen, nullptr, a.do_sample);
  if (w.s_begin == 0 && blockIdx.x == 0) {   // the chain kernels' per-row state starts clear
    uint32_t* stw = w.state + (size_t)row * kStateWords;
    for (int i = threadIdx.x; i < kStateWords; i += NTA) stw[i] = 0u;
  }
  const int mode = stream_mode(c, V);
  if (mode == kModeExact) return;
  const int s0 = w.s_begin + (int)blockIdx.x * w.steps_per_group;
  const int s1 = ONE ? s0 + 1 : min(w.s_end, s0 + w.steps_per_group);
  if (s0 >= s1) return;
  const int t = threadIdx.x, lane = lane_id(), wv = wave_id();
  const int cap = list_cap(c);
  const bool large = cap == kListLarge;
  const uint32_t msel = (uint32_t)cap - 16u;
  const bool masses = mode == kModeRow;

  const int nwords = bitmap_words(V);
  for (int i = t; i < nwords; i += NTA) sh.bm[i] = 0u;
  __syncthreads();
  {
    const int64_t h0 = a.hist_off[row], h1 = a.hist_off[row + 1];
    for (int64_t j = h0 + t; j < h1; j += NTA) {
      const int id = a.hist_ids[j];
      if (id >= 0 && id < V) atomicOr(&sh.bm[id >> 5], 1u << (id & 31));   // sampling.cpp:24
    }
  }
  __syncthreads();
  const float pen = c.pen;

  for (int s = s0; s < s1; ++s) {
    C4S_SCAN_PHASE(0);
    const float* p = a.logits + (int64_t)s * a.step_stride + (int64_t)row * a.ld;
    const RowShape rs = row_shape(p, V);
    const float4* p4 = reinterpret_cast<const float4*>(p + rs.head);
    // The thread's values as keys (0 past the row: below every key of a value).
    uint32_t kq[NQ][4];
    {
      float4 xv[NQ];
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int q = t + NTA * j;
        xv[j] = (q < rs.nq) ? p4[q] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const bool in = t + NTA * j < rs.nq;
        kq[j][0] = in ? fkey(xv[j].x) : 0u;
        kq[j][1] = in ? fkey(xv[j].y) : 0u;
        kq[j][2] = in ? fkey(xv[j].z) : 0u;
        kq[j][3] = in ? fkey(xv[j].w) : 0u;
      }
    }
    const bool eh = t < rs.head;
    const bool et = !eh && t < rs.head + rs.tail;
    const int eid = eh ? t : rs.head + 4 * rs.nq + (t - rs.head);
    const uint32_t ke = (eh || et) ? fkey(p[eid]) : 0u;

    // Per-thread top-2 (top-4 for large lists) keys.
    uint32_t t1 = 0, t2 = 0, t3 = 0, t4 = 0;
    if (large) {
      auto ins4 = [&](uint32_t k) {
        t4 = max(t4, min(t3, k));
        t3 = max(t3, min(t2, k));
        t2 = max(t2, min(t1, k));
        t1 = max(t1, k);
      };
#pragma unroll
      for (int j = 0; j < NQ; ++j) { ins4(kq[j][0]); ins4(kq[j][1]); ins4(kq[j][2]); ins4(kq[j][3]); }
      ins4(ke);
    } else {
      auto ins2 = [&](uint32_t k) {
        t2 = max(t2, min(t1, k));
        t1 = max(t1, k);
      };
#pragma unroll
      for (int j = 0; j < NQ; ++j) { ins2(kq[j][0]); ins2(kq[j][1]); ins2(kq[j][2]); ins2(kq[j][3]); }
      ins2(ke);
    }
    C4S_SCAN_PHASE(1);

    // L0: a key at or below the msel-th largest of those keys (two 11-bit passes).
    for (int i = t; i < 2048; i += NTA) sh.hist[i] = 0u;
    for (int i = t; i < kIdWords; i += NTA) { sh.lmark[i] = 0u; sh.fmark[i] = 0u; }
    __syncthreads();
    if (t1) atomicAdd(&sh.hist[t1 >> 21], 1u);
    if (t2) atomicAdd(&sh.hist[t2 >> 21], 1u);
    if (t3) atomicAdd(&sh.hist[t3 >> 21], 1u);
    if (t4) atomicAdd(&sh.hist[t4 >> 21], 1u);
    __syncthreads();
    uint32_t L0 = 0;
    {
      uint32_t b1, ab1;
      if (hist_pick(sh, msel, b1, ab1)) {
        for (int i = t; i < 2048; i += NTA) sh.hist[i] = 0u;
        __syncthreads();
        if (t1 && (t1 >> 21) == b1) atomicAdd(&sh.hist[(t1 >> 10) & 2047u], 1u);
        if (t2 && (t2 >> 21) == b1) atomicAdd(&sh.hist[(t2 >> 10) & 2047u], 1u);
        if (t3 && (t3 >> 21) == b1) atomicAdd(&sh.hist[(t3 >> 10) & 2047u], 1u);
        if (t4 && (t4 >> 21) == b1) atomicAdd(&sh.hist[(t4 >> 10) & 2047u], 1u);
        __syncthreads();
        uint32_t b2, ab2;
        hist_pick(sh, msel - ab1, b2, ab2);
        L0 = (b1 << 21) | (b2 << 10);
      }
    }
    L0 = max(L0, 1u);   // the same set of values; excludes the zero keys past the row
    C4S_SCAN_PHASE(2);

    // Candidates (key >= L0) in thread order: one scan of the per-thread
    // counts places them (their id order comes from id bitmaps below).
    uint32_t cnt = 0;
    uint32_t below = 0;   // largest key under L0 (raw value: bounds the penalised one)
    if (ke >= L0) ++cnt; else below = ke;
#pragma unroll
    for (int j = 0; j < NQ; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t k = kq[j][i];
        cnt += (k >= L0) ? 1u : 0u;
        below = max(below, k < L0 ? k : 0u);
      }
    {
      const uint32_t bm = wave_max_u32(below);
      if (lane == 0) sh.redm[wv] = bm;
    }
    uint32_t C;
    uint32_t pos = scan_excl_nta(cnt, sh.red, C);   // its barriers also publish redm
    uint32_t tout = 0;
#pragma unroll
    for (int ww = 0; ww < NWA; ++ww) tout = max(tout, sh.redm[ww]);
    // raw values bound the penalised ones; the quotient is monotone in them
    if (tout != 0u && c.temp_on) tout = fkey(kfloat(tout) / c.temp);
    const bool overflow = C > (uint32_t)kCandCap;
    C4S_SCAN_PHASE(3);
    if (!overflow && cnt) {
      // key and id of each candidate
      auto put = [&](uint32_t k, int id) { sh.cand[pos++] = ((uint64_t)k << 32) | (uint32_t)id; };
      if (ke >= L0) put(ke, eid);
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int id = rs.head + 4 * (t + NTA * j);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kq[j][i] >= L0) put(kq[j][i], id + i);
      }
    }
    __syncthreads();
    // Each candidate, one thread each: the penalty of H0 (sampling.cpp:26), the
    // temperature (:16), its entry.
    if (!overflow)
      for (int i = t; i < (int)C; i += NTA) {
        const uint64_t cw = sh.cand[i];
        const int id = (int)(uint32_t)cw;
        const float x = kfloat((uint32_t)(cw >> 32));
        const float y = (c.pen_on && bit_of(sh.bm, id)) ? pen_exact(x, pen) : x;
        sh.cand[i] = make_entry(c.temp_on ? y / c.temp : y, id, i);
        sh.candy[i] = y;
      }
    // Sorted entries (descending). Up to 256 of them by rank counting into the
    // free histogram: entries are distinct (ids are), so an entry's rank is the
    // number of larger ones; the list is padded with zero entries (every entry
    // is positive) to a multiple of eight. More by a bitonic sort in place.
    const bool small = C <= (uint32_t)NTA;
    uint64_t* srt = small ? reinterpret_cast<uint64_t*>(sh.hist) : sh.cand;
    static_assert(sizeof(sh.hist) >= NTA * sizeof(uint64_t), "the histogram holds a small sorted list");
    const int C8 = ((int)C + 7) & ~7;
    int P = 2;
    while (P < (int)C) P <<= 1;
    if (!overflow) {
      if (small) {
        if (t < C8 - (int)C) sh.cand[C + t] = 0ull;
      } else {
        for (int i = (int)C + t; i < P; i += NTA) sh.cand[i] = 0ull;
      }
    }
    __syncthreads();
    C4S_SCAN_PHASE(4);
    if (!overflow) {
      if (small) {
        const uint64_t mine = (t < (int)C) ? sh.cand[t] : ~0ull;
        uint32_t r = 0;
        if (wv * kWave < (int)C)   // waves without an entry skip the count
          for (int j = 0; j < C8; j += 8) {
            uint64_t o[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = sh.cand[j + i];
#pragma unroll
            for (int i = 0; i < 8; ++i) r += (o[i] > mine) ? 1u : 0u;
          }
        if (t < (int)C) srt[r] = mine;
        __syncthreads();
      } else {
        bitonic_desc_u64(sh.cand, P);
      }
    }
    C4S_SCAN_PHASE(5);

    // Leading entries above the bound, at most cap of them.
    uint32_t nabove = 0;
    if (!overflow)
      for (int i = t; i < (int)C; i += NTA) nabove += (ent_key(srt[i]) > tout) ? 1u : 0u;
    uint32_t n_all;
    (void)scan_excl_nta(nabove, sh.red, n_all);
    int n = min((int)n_all, cap);
    if (!overflow && (int)n_all > cap) tout = max(tout, ent_key(srt[cap]));
    const bool bad = overflow || n == 0;

    uint64_t* sw = reinterpret_cast<uint64_t*>(w.sum + ((size_t)(s - w.s_begin) * a.n_rows + row) * kSumStride);
    double top_mass = 0.0;   // wave 0: mass of the list's first kLanesHint entries
    double first_mass = 0.0; // the thread's list position below NTA
    uint64_t* lst = sw;
    SumHdr* hdr = reinterpret_cast<SumHdr*>(sw + kHdrW);
    double* chk = reinterpret_cast<double*>(sw + kChunkW);
    if (!bad) {
      // greedy / top-k rows: the value before the temperature (their hits are
      // penalised again from it); full-vocabulary rows: the entry's mass
      // exp((double)fl(z - z_max)) as the reference computes it, in fp32.
      float* ly = reinterpret_cast<float*>(sw + kYW);
      const float zmax = kfloat(ent_key(srt[0]));
      // The stored rank is the id-order rank among the list entries: the
      // list's ids below the entry's own, counted in an id bitmap of the
      // list. Full-vocabulary rows also get each of the first NTA entries'
      // id-order place among those NTA (a bitmap of their ids).
      for (int i = t; i < n; i += NTA) {
        const int id = ent_id(srt[i]);
        atomicOr(&sh.lmark[id >> 5], 1u << (id & 31));
        if (i < NTA) atomicOr(&sh.fmark[id >> 5], 1u << (id & 31));
      }
      __syncthreads();
      {
        // marks before each word, both bitmaps in one scan (16-bit halves: at
        // most kListLarge marks); thread t takes words 2t and 2t + 1
        const int wa = 2 * t, wb = 2 * t + 1;
        const uint32_t pa = wa < kIdWords ? (uint32_t)__popc(sh.lmark[wa]) | ((uint32_t)__popc(sh.fmark[wa]) << 16) : 0u;
        const uint32_t pb = wb < kIdWords ? (uint32_t)__popc(sh.lmark[wb]) | ((uint32_t)__popc(sh.fmark[wb]) << 16) : 0u;
        uint32_t tot;
        const uint32_t ex = scan_excl_nta(pa + pb, sh.red, tot);
        if (wa < kIdWords) sh.pre2[wa] = ex;
        if (wb < kIdWords) sh.pre2[wb] = ex + pa;
      }
      __syncthreads();
      // Entries t and t + NTA (n <= 2 NTA): every LDS read first, at clamped
      // positions, so that each dependent group goes out together.
      static_assert(kListLarge <= 2 * NTA, "two list entries a thread");
      const bool v0 = t < n, v1 = t + NTA < n;
      const uint64_t e0 = srt[v0 ? t : 0], e1 = srt[v1 ? t + NTA : 0];
      const int c0 = ent_rank(e0), c1 = ent_rank(e1);   // candidate positions
      const int i0 = ent_id(e0), i1 = ent_id(e1);
      const uint32_t below0 = (1u << (i0 & 31)) - 1u, below1 = (1u << (i1 & 31)) - 1u;
      const uint32_t pr0 = sh.pre2[i0 >> 5], lk0 = sh.lmark[i0 >> 5], fk0 = sh.fmark[i0 >> 5];
      const uint32_t pr1 = sh.pre2[i1 >> 5], lk1 = sh.lmark[i1 >> 5];
      const uint32_t lp0 = pr0 & 0xFFFFu, lp1 = pr1 & 0xFFFFu, fp0 = pr0 >> 16;
      const float y0 = sh.candy[c0], y1 = sh.candy[c1];
      if (masses && v0)   // the place among the first NTA, to the summary as words below
        reinterpret_cast<uint8_t*>(sh.place4)[t] = (uint8_t)(fp0 + (uint32_t)__popc(fk0 & below0));
      if (v0) {
        lst[t] = (e0 & ~1023ull) | (lp0 + (uint32_t)__popc(lk0 & below0));
        if (masses) {
          const float m = (float)exp((double)(kfloat(ent_key(e0)) - zmax));
          ly[t] = m;
          if (t < kLanesHint) top_mass += (double)m;   // wave 0
          first_mass = (double)m;
        } else {
          ly[t] = y0;
        }
      }
      if (v1) {
        lst[t + NTA] = (e1 & ~1023ull) | (lp1 + (uint32_t)__popc(lk1 & below1));
        ly[t + NTA] = masses ? (float)exp((double)(kfloat(ent_key(e1)) - zmax)) : y1;
      }
      if (masses) {
        if (wv == 0) top_mass = wave_sum_f64(top_mass);
        const double fm = wave_sum_f64(first_mass);
        if (lane == 0) sh.redh[wv] = fm;   // read after the barriers of the chunk masses
      }
    }

    C4S_SCAN_PHASE(6);
    // Chunk masses of the whole row (rows without top-k).
    float m0 = 0.f;
    int nchunk = 0, qhint = kListLarge;   // qhint: read by thread 0 (wave 0 holds top_mass)
    double err = 0.0, s0 = 0.0;
    if (masses && !bad) {
      // Chunk masses as the reference computes them, exp((double)fl(fl(y/T) - m0)):
      // the nucleus cut and the full-vocabulary draw are then decided with
      // margins of a few ulp, and the masses carry no error term (err = 0).
      m0 = kfloat(ent_key(srt[0]));
      nchunk = max(1, (rs.nq + 15) >> 4);
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int q = t + NTA * j;
        double qd = 0.0;
        if (q < rs.nq) {
          const int qid = rs.head + 4 * q;   // the quad's H0 bits
          const uint32_t hb =
              (uint32_t)(((uint64_t)sh.bm[qid >> 5] | ((uint64_t)sh.bm[(qid >> 5) + 1] << 32)) >> (qid & 31)) & 15u;
          const bool pon = c.pen_on;
          const float x0 = kfloat(kq[j][0]), x1 = kfloat(kq[j][1]), x2 = kfloat(kq[j][2]), x3 = kfloat(kq[j][3]);
          qd = mass_exact((pon && (hb & 1u)) ? pen_exact(x0, pen) : x0, c, m0) +
               mass_exact((pon && (hb & 2u)) ? pen_exact(x1, pen) : x1, c, m0) +
               mass_exact((pon && (hb & 4u)) ? pen_exact(x2, pen) : x2, c, m0) +
               mass_exact((pon && (hb & 8u)) ? pen_exact(x3, pen) : x3, c, m0);
        }
        // 16 consecutive lanes hold the 16 quads of one chunk
        double d = qd;
        d += dpp_f64<0x111>(d, 0.0);
        d += dpp_f64<0x112>(d, 0.0);
        d += dpp_f64<0x114>(d, 0.0);
        d += dpp_f64<0x118>(d, 0.0);
        const int ci = q >> 4;
        if ((lane & 15) == 15 && ci < nchunk) sh.chunk[ci] = d;
      }
      if (t < 8) sh.edge[t] = 0.0;
      __syncthreads();
      if (eh || et) {
        const bool pb = c.pen_on && bit_of(sh.bm, eid);
        const float xe = kfloat(ke);
        sh.edge[t] = mass_exact(pb ? pen_exact(xe, pen) : xe, c, m0);   // t < 6
      }
      if (t == 0) {
        double hs = 0.0, ts = 0.0;
        for (int i = 0; i < rs.head; ++i) hs += sh.edge[i];
        for (int i = rs.head; i < rs.head + rs.tail; ++i) ts += sh.edge[i];
        sh.chunk[0] += hs;
        sh.chunk[nchunk - 1] += ts;
      }
      __syncthreads();
      double cl = 0.0;
      for (int i = t; i < nchunk; i += NTA) { chk[i] = sh.chunk[i]; cl += sh.chunk[i]; }
      s0 = block_sum_f64<NTA>(cl, sh.redd);
      // Cut hint for the chains (nucleus rows): the list's first kLanesHint
      // (or NTA) entries hold p * s0 of the mass, so the cut lies among them
      // unless hits or corrections move it.
      if (1.0 - (double)c.p > 0.0) {
        double top_nta = 0.0;
#pragma unroll
        for (int ww = 0; ww < NWA; ++ww) top_nta += sh.redh[ww];
        const double pS0 = (double)c.p * s0;
        qhint = top_mass >= pS0 ? kLanesHint : (top_nta >= pS0 ? NTA : kListLarge);
      }
    }
    C4S_SCAN_PHASE(7);
    if (masses && !bad && t < NTA / 4) reinterpret_cast<uint32_t*>(sw + kPlaceW)[t] = sh.place4[t];   // places (above)
    if (t == 0) {
      SumHdr h{};
      h.n = bad ? 0 : n;
      h.tout = tout;
      h.flags = bad ? 1u : 0u;
      h.m0 = m0;
      h.nchunk = nchunk;
      h.head = rs.head;
      h.err = err + 0x1p-100;
      h.s0 = s0;
      h.qhint = qhint;
      *hdr = h;
    }
    __syncthreads();
    C4S_SCAN_PHASE(8);
  }
}

// ---- chain (one workgroup per row) ----------------------------------------------------


struct ChainSh {
  uint64_t sum[kSumWords];   // this step's summary: header words, list, chunks
  double cdelta[kMaxChunks];
  uint32_t inv[kListLarge + 1];   // id-order slot -> (generation << 10) | unhit rank; + a trash word
  uint32_t gen;             // generation of the last row step
  float lz[kListLarge + 1];   // by unhit rank; + a trash entry
  float lm[kListLarge + 1];
  int lid[kListLarge + 1];
  int lslot[kListLarge];
  double wd[NW];
  double we[NW];
  uint64_t rng;
  int bi[4];
};

// Per-row state carried across the chain kernels and across chunks of steps
// (kStateWords words): done flag, statistics, next step, pending exact step,
// then the bitmap of ids drawn during the stream.
enum : int { kStDone = 0, kStStats = 1, kStNext = 5, kStBits = 8 };


// Slot s (an id-order rank among the list entries) lives at position
// slot_pos(s): lane l's eight slots [8 l, 8 l + 8) are the l-th word of eight
// 64-word rows, so a wave reads them without bank conflicts.
constexpr int kSlotsPerLane = kListLarge / kWave;
static_assert(kSlotsPerLane == 8, "slot_pos assumes eight slots a lane");
__device__ __forceinline__ int slot_pos(int s) { return ((s & 7) << 6) | (s >> 3); }

__device__ __forceinline__ SumHdr hdr_words(uint64_t w0, uint64_t w1, uint64_t w2, uint64_t w3,
                                            uint64_t w4) {
  SumHdr h{};
  h.s0 = __longlong_as_double((long long)w4);
  h.n = (int)(uint32_t)w0;
  h.tout = (uint32_t)(w0 >> 32);
  h.flags = (uint32_t)w1;
  h.m0 = __uint_as_float((uint32_t)(w1 >> 32));
  h.nchunk = (int)(uint32_t)w2;
  h.head = (int)(uint32_t)(w2 >> 32);
  h.err = __longlong_as_double((long long)w3);
  return h;
}
__device__ __forceinline__ SumHdr hdr_from(const uint64_t* sw) {   // sw: summary words (LDS)
  return hdr_words(sw[kHdrW], sw[kHdrW + 1], sw[kHdrW + 2], sw[kHdrW + 3], sw[kHdrW + 4]);
}
// Header held in lanes 0..3 of a wave's register `hw` (word kHdrW + lane).
__device__ __forceinline__ SumHdr hdr_lanes(uint64_t hw) {
  auto rl = [&](int l) -> uint64_t {
    return (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)hw, l) |
           ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(hw >> 32), l) << 32);
  };
  return hdr_words(rl(0), rl(1), rl(2), rl(3), rl(4));
}



// Where a step reads raw values and the set of ids drawn during the stream.
// RowAcc: the raw row and the drawn-id bitmap staged in LDS.
//   hit(id)  id was drawn during the stream (it is then penalised again)
//   hval(id) raw value of a drawn id
//   raw(id)  raw value of any id (the dense draw's chunk)
//   pen(id)  id is penalised (H0 or drawn)
struct RowAcc {
  const float* v;
  const uint32_t* bmN;
  const uint32_t* bmH0;
  __device__ __forceinline__ bool hit(int id) const { return (bmN[id >> 5] >> (id & 31)) & 1u; }
  __device__ __forceinline__ float hval(int id) const { return v[id]; }
  __device__ __forceinline__ float raw(int id) const { return v[id]; }
  __device__ __forceinline__ bool pen(int id) const { return ((bmH0[id >> 5] | bmN[id >> 5]) >> (id & 31)) & 1u; }
};

// What a decided step rests on, so that it can be checked later against ids
// drawn after the set it was decided with: kind 1, a nucleus cut (the kept
// ranks [0, q), the masses above ranks q - 1 and q, the cut value); kind 2,
// the dense draw (the prefixes through and before the token, the uniform);
// kind 0, nothing to check against (the step is redone).
struct SpecInfo {
  int kind;
  int q;
  int chk1;    // rank q - 1 is at or past min_keep (its margin is checked)
  float zcut;  // z of rank q - 1
  float mt;    // the maximum
  double S, rho, err, eps, dmass, p;
  double A1, A2;
  double af, pf, u;
};

// Dense draw (top_p keeps every id of nonzero mass; zero masses never win),
// text2semantic.cpp:150-165: r = u * S, the chunk prefixes (summary chunk
// masses less the corrections, times rho) locate r, the chunk's masses are
// recomputed exactly from the staged row. False when r is not inside its
// chunk by the error margin.
template <class Acc>
__device__ __forceinline__ bool dense_draw(const SumHdr& h, const RowCfg& c, int V, const Acc& acc,
                                           const uint64_t* sum,
                                           const double* cdelta, double u, double S, double rho, double err,
                                           float mt, StepOut& o, SpecInfo* si) {
  const int lane = lane_id();
  const float ninf = neg_inf();
  const double eps = rel_eps(V);
  o.why = kWhyDraw;
  const int nchunk = h.nchunk;
  double cv[4];
  double cs_l = 0.0;
  // chunk words read unconditionally (in bounds: index clamped), then selected
  uint64_t cw[4];
  double cd[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int cr = min(4 * lane + i, kMaxChunks - 1);
    cw[i] = sum[kChunkW + cr];
    cd[i] = cdelta[cr];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ci = 4 * lane + i;
    cv[i] = (ci < nchunk) ? __longlong_as_double((long long)cw[i]) - cd[i] : 0.0;
    cs_l += cv[i];
  }
  const double r = u * S;
  const double inc = wave_scan_f64(cs_l);
  double run = (inc - cs_l) * rho;
  int cstar = -1;
  double pstar = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ci = 4 * lane + i;
    const double nx = run + cv[i] * rho;
    if (cstar < 0 && ci < nchunk && nx >= r) { cstar = ci; pstar = run; }
    run = nx;
  }
  const uint64_t hmk = __ballot(cstar >= 0);
  if (!hmk || !(r > 0.0)) return false;
  const int fl = __ffsll((unsigned long long)hmk) - 1;
  cstar = (int)readlane_u32((uint32_t)cstar, fl);
  pstar = readlane_f64(pstar, fl);
  C4S_PHASE(13);
  const int lo = cstar == 0 ? 0 : h.head + kChunkIds * cstar;
  const int hi = (cstar == nchunk - 1) ? V : h.head + kChunkIds * (cstar + 1);
  const int ia = lo + lane, ib = lo + kWave + lane;
  // the chunk's values and bitmap words read unconditionally (ids clamped into
  // the chunk), so that both reads of each id go out together
  const int ja = min(ia, hi - 1), jb = min(ib, hi - 1);
  const float xa = acc.raw(ja), xb = acc.raw(jb);
  const bool ha = acc.pen(ja), hb = acc.pen(jb);
  auto mass_of = [&](float x, bool pn) -> double {
    const float y = (c.pen_on && pn) ? pen_exact(x, c.pen) : x;
    const float z = c.temp_on ? y / c.temp : y;
    return (z == ninf) ? 0.0 : exp((double)(z - mt));
  };
  const double ea = ia < hi ? mass_of(xa, ha) : 0.0;
  const double eb = ib < hi ? mass_of(xb, hb) : 0.0;
  C4S_PHASE(14);
  const double sa = wave_scan_f64(ea) + pstar;
  const double ta = readlane_f64(sa, kWave - 1);
  const double sb = wave_scan_f64(eb) + ta;
  const double mg = 2.0 * err;
  const uint64_t fa = __ballot(ia < hi && ea > 0.0 && sa >= r);
  const uint64_t fb = __ballot(ib < hi && eb > 0.0 && sb >= r);
  double af, pf;
  int tok;
  if (fa) {
    const int f = __ffsll((unsigned long long)fa) - 1;
    af = readlane_f64(sa, f);
    pf = af - readlane_f64(ea, f);
    tok = lo + f;
  } else if (fb) {
    const int f = __ffsll((unsigned long long)fb) - 1;
    af = readlane_f64(sb, f);
    pf = af - readlane_f64(eb, f);
    tok = lo + kWave + f;
  } else {
    return false;
  }
  if (!((af - r > mg + eps * af) && (r - pf > mg + eps * r))) return false;
  o.tok = tok;
  o.kept = (uint32_t)V;
  o.dex = 0;
  if (si) {
    si->kind = 2;
    si->mt = mt;
    si->S = S;
    si->rho = rho;
    si->err = err;
    si->eps = eps;
    si->af = af;
    si->pf = pf;
    si->u = u;
  }
  return true;
}

// row_step in registers for a step decided within the first 64 list entries
// (one per lane): a nucleus of at most 64 unhit ranks, or the dense draw. The
// unhit entries move to lanes 0..nu-1 in rank order by one lane permute; the
// cut is one prefix scan, the draw the lane draw. Same decisions and margins
// as row_step; false, with rng and o unchanged, when the step needs row_step.
template <class Acc>
__device__ __forceinline__ bool row_step_lanes(const SumHdr& h, const RowCfg& c, int V, const Acc& acc,
                                               double dsum, double derr,
                                               const uint64_t* sum, const double* cdelta, uint64_t& rng,
                                               StepOut& o, SpecInfo* si = nullptr) {
  const int lane = lane_id();
  if (h.flags & 1u) return false;
  const int n = h.n;
  const float ninf = neg_inf();
  const bool v = lane < n;
  // reads unconditional and in bounds (entry and bitmap word, raw value, issued together)
  const uint64_t e = sum[lane];
  const float m32 = reinterpret_cast<const float*>(sum + kYW)[lane];
  const int id = v ? ent_id(e) : 0;
  const bool drawn = acc.hit(id);
  const float xr = acc.hval(id);
  const bool hit = c.pen_on && v && drawn;
  // a drawn id is never in H0: its value is the raw one (the penalty and the
  // temperature are monotone, so the largest penalised hit comes from the largest raw one)
  const float hraw = hit ? xr : ninf;
  const bool un = v && !hit;
  const uint64_t ub = __ballot(un);
  const int nu = __popcll(ub);
  if (nu == 0) return false;
  // lane permutation: unhit entries to their ranks, the others after them
  const int dst = (un ? __popcll(ub & lanemask_lt()) : nu + __popcll(~ub & lanemask_lt())) << 2;
  const uint32_t pk = (uint32_t)__builtin_amdgcn_ds_permute(dst, (int)ent_key(e));
  const float pm = __int_as_float(__builtin_amdgcn_ds_permute(dst, __float_as_int(m32)));
  const int pid = __builtin_amdgcn_ds_permute(dst, id);
  const int pslot = __builtin_amdgcn_ds_permute(dst, ent_rank(e));
  C4S_PHASE(4);
  const bool in = lane < nu;
  const float z = in ? kfloat(pk) : ninf;
  const float mt = readlane_f32(z, 0);
  const float zo = (h.tout != 0u) ? kfloat(h.tout) : ninf;
  if (!(mt > ninf) || !(zo < mt)) return false;
  // entries past the first 64 are at or below entry 63
  const float zend = (n > kWave) ? kfloat(readlane_u32(ent_key(e), kWave - 1)) : ninf;
  if (!(zend < mt)) return false;
  const float hx = wave_max_dpp(hraw);
  const float hy = pen_exact(hx, c.pen);   // sampling.cpp:26, then :16
  const float hm = c.temp_on ? hy / c.temp : hy;
  if (!(hm < mt)) return false;
  C4S_PHASE(5);

  const double eps = rel_eps(V);
  const double dm = (double)h.m0 - (double)mt;
  const double rho = (dm == 0.0) ? 1.0 : exp(dm);
  const double S = (h.s0 - dsum) * rho;
  const double err = (h.err + derr + fabs(dsum) * 0x1p-50) * rho +
                     (dm > 0.0 ? 0x1p-23 * ((40.0 + dm) * S + (double)V * 0x1p-50) : 0.0) + eps * S;
  const double thr = 1.0 - (double)c.p;
  const uint64_t st = xorshift64(rng);
  const double u = unit_from_state(st);
  C4S_PHASE(6);
  if (!(thr > 0.0)) {
    if (!dense_draw(h, c, V, acc, sum, cdelta, u, S, rho, err, mt, o, si)) return false;
    rng = st;
    return true;
  }
  // nucleus cut on the unhit ranks: removed iff above >= p * S (as row_step)
  const double pS = (double)c.p * S;
  const double marg = (double)c.p * err + eps * S;
  const bool approx = dm == 0.0;
  const double dmass = approx ? 0x1p-23 : 0.0;
  const bool stored = approx && pm >= 0x1p-100f;
  double em = (in && stored) ? (double)pm : 0.0;
  if (__ballot(in && !stored)) em = (in && !stored) ? exp((double)(z - mt)) : em;
  const double inc = wave_scan_f64(em);
  const double above = inc - em;
  const double D = above - pS;
  if (__ballot(in && lane >= c.min_keep && !(fabs(D) > marg + (eps + dmass) * above))) return false;
  if (__ballot(in && D < 0.0 && em < 0x1p-1000)) return false;   // subnormal kept masses
  const uint64_t qm = __ballot(in && D >= 0.0);
  if (!qm) return false;   // the cut lies past these ranks
  const int q = max(__ffsll((unsigned long long)qm) - 1, c.min_keep);
  if (q > nu) return false;
  const float zq1 = readlane_f32(z, q - 1);
  if (!(zo < zq1) || !(zend < zq1) || !(hm < zq1)) return false;
  if (si) {
    si->kind = 1;
    si->q = q;
    si->chk1 = q - 1 >= c.min_keep;
    si->zcut = zq1;
    si->mt = mt;
    si->S = S;
    si->rho = rho;
    si->err = err;
    si->eps = eps;
    si->dmass = dmass;
    si->p = (double)c.p;
    si->A1 = readlane_f64(above, q - 1);
    si->A2 = readlane_f64(inc, q - 1);
  }
  C4S_PHASE(7);
  // the draw on the kept ranks [0, q): first with the masses above, then exact
  const bool kept = lane < q;
  uint32_t dex = 0;
  int tok = -1;
  if (approx) tok = lane_draw<kSlotBits>(kept, pid, pslot, kept ? em : 0.0, u, V, dex, 0x1p-22, false);
  if (tok < 0) {
    const double ex = kept ? exp((double)(z - mt)) : 0.0;
    tok = lane_draw<kSlotBits>(kept, pid, pslot, ex, u, V, dex);
  }
  o.tok = tok;
  o.kept = (uint32_t)q;
  o.dex = dex;
  rng = st;
  return true;
}

// Draw over the kept unhit ranks [0, q) in id order (text2semantic.cpp:150-165):
// cs.inv maps the id-order slots to the ranks tagged with generation gen,
// cs.lz/lm/lid hold the ranks' values, stored fp32 masses and ids. Sets o.dex.
template <class CS>
__device__ __forceinline__ int inv_draw(CS& cs, uint32_t gen, int q, bool approx, float mt, double u, int V,
                                        StepOut& o) {
  const int lane = lane_id();
  // Kept ranks [0, q) in id order: lane l reads the id-order slots
  // [8 l, 8 l + 8); a slot tagged with this call's generation names its
  // unhit rank, every other slot (no candidate, a hit, a rank past the cut)
  // weighs 0. First with the masses above, then with exact masses.
  constexpr int kPer = kSlotsPerLane;
  int rks[kPer];
  uint32_t vb = 0u;   // bit i: slot 8 lane + i is kept
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const uint32_t x = cs.inv[(i << 6) | lane];
    rks[i] = (int)(x & 1023u);
    vb |= (((x >> 10) == gen && rks[i] < q) ? 1u : 0u) << i;
  }
  float mf[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) mf[i] = cs.lm[rks[i]];   // tagged ranks are below kListLarge
  C4S_PHASE(13);
  auto draw = [&](bool exact_only, double eps_add) __attribute__((always_inline)) -> int {
    // in-lane inclusive prefix p[i], then one scan over the lanes
    double e[kPer], p[kPer];
    bool need = false;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const bool v = (vb >> i) & 1u;
      const bool st = approx && !exact_only && mf[i] >= 0x1p-100f;
      e[i] = (v && st) ? (double)mf[i] : 0.0;
      need |= v && !st;
    }
    if (__ballot(need)) {   // exp for every slot (no per-slot branches), kept where needed
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const double x = exp((double)(cs.lz[rks[i]] - mt));
        const bool st = approx && !exact_only && mf[i] >= 0x1p-100f;
        e[i] = (((vb >> i) & 1u) && !st) ? x : e[i];
      }
    }
    p[0] = e[0];
#pragma unroll
    for (int i = 1; i < kPer; ++i) p[i] = p[i - 1] + e[i];
    const double inc = wave_scan_f64(p[kPer - 1]);
    const double r = u * readlane_f64(inc, kWave - 1);
    const double base = inc - p[kPer - 1];
    double ha = 0.0, hp = 0.0;
    int hrk = -1;
#pragma unroll
    for (int i = kPer - 1; i >= 0; --i) {   // the first slot reaching r wins
      const double nx = base + p[i];
      if (e[i] > 0.0 && nx >= r) { hrk = rks[i]; ha = nx; hp = i ? base + p[i - 1] : base; }
    }
    const uint64_t hb = __ballot(hrk >= 0);
    if (!hb) return -1;
    const int f = __ffsll((unsigned long long)hb) - 1;
    const double af = readlane_f64(ha, f), pf = readlane_f64(hp, f);
    const double eps = rel_eps(V) + eps_add;
    if (!(r > 0.0 && (af - r > eps * af) && (r - pf > eps * r))) return -1;
    return cs.lid[readlane_u32((uint32_t)hrk, f)];
  };
  int tok = -1;
  o.dex = 0;
  if (approx) tok = draw(false, 0x1p-22);
  C4S_PHASE(14);
  if (tok < 0) tok = draw(true, 0.0);
  if (tok < 0) {
    // text2semantic.cpp:152-164 sequentially in id order with exact masses
    o.dex = 1;
    int res = 0;
    if (lane == 0) {
      auto kept_mass = [&](int sl, int& rk) -> double {
        const uint32_t x = cs.inv[slot_pos(sl)];
        rk = (int)(x & 1023u);
        return ((x >> 10) == gen && rk < q) ? exp((double)(cs.lz[rk] - mt)) : 0.0;
      };
      double total = 0.0;
      for (int sl = 0; sl < kListLarge; ++sl) {
        int rk;
        total += kept_mass(sl, rk);
      }
      const double rr = u * total;
      res = V - 1;
      if (rr <= 0.0) {
        res = 0;
      } else {
        double acc = 0.0;
        for (int sl = 0; sl < kListLarge; ++sl) {
          int rk;
          const double ei = kept_mass(sl, rk);
          acc += ei;
          if (ei > 0.0 && rr <= acc) { res = cs.lid[rk]; break; }
        }
      }
    }
    tok = (int)readlane_u32((uint32_t)res, 0);
  }
  return tok;
}

// row_step in registers for a nucleus within the first 256 list entries, four
// consecutive ones per lane: unhit ranks from one scan of the lane counts, the
// cut from one prefix scan of the lane masses, no list compaction; the kept
// ranks then go to LDS for the id-order draw (inv_draw). Same decisions and
// margins as row_step; false, with rng and o unchanged, when the step needs
// row_step (its generation counter may have moved, which is harmless).
template <class CS, class Acc>
__device__ __forceinline__ bool row_step_lanes4(const SumHdr& h, const RowCfg& c, int V, const Acc& acc,
                                                double dsum, double derr, const uint64_t* sum,
                                                uint64_t& rng, CS& cs, StepOut& o, SpecInfo* si = nullptr) {
  constexpr int K = 4;
  const int lane = lane_id();
  if (h.flags & 1u) return false;
  const int n = h.n;
  const float ninf = neg_inf();
  const int p0 = K * lane;
  const float* ly = reinterpret_cast<const float*>(sum + kYW);
  // id-order places of this lane's entries among the list's first K * 64, one byte each
  const uint32_t pl = reinterpret_cast<const uint32_t*>(sum + kPlaceW)[lane];
  uint64_t e[K];
  float mk[K], z[K];
  bool un[K];
  uint32_t cnt = 0;
  float hraw = ninf;
  // All reads unconditional, from addresses that are always in bounds (list
  // positions below K * 64 <= kListLarge; id 0 for positions past n), so that
  // the four entries' reads go out together: entries, then bitmap words and
  // raw values. A drawn id is never in H0: its value is the raw one.
  int id[K];
  bool dr[K];
  float xr[K];
#pragma unroll
  for (int i = 0; i < K; ++i) {
    e[i] = sum[p0 + i];
    mk[i] = ly[p0 + i];
  }
#pragma unroll
  for (int i = 0; i < K; ++i) id[i] = (p0 + i < n) ? ent_id(e[i]) : 0;
#pragma unroll
  for (int i = 0; i < K; ++i) {
    dr[i] = acc.hit(id[i]);
    xr[i] = acc.hval(id[i]);
  }
#pragma unroll
  for (int i = 0; i < K; ++i) {
    const bool v = p0 + i < n;
    const bool hit = c.pen_on & v & dr[i];
    hraw = hit ? fmaxf(hraw, xr[i]) : hraw;
    un[i] = v & !hit;
    z[i] = un[i] ? kfloat(ent_key(e[i])) : ninf;
    cnt += un[i] ? 1u : 0u;
  }
  C4S_PHASE(4);
  const uint32_t cinc = wave_scan_u32(cnt);
  const int nu = (int)readlane_u32(cinc, kWave - 1);
  if (nu == 0) return false;
  int rk[K];
  {
    int r = (int)(cinc - cnt);
#pragma unroll
    for (int i = 0; i < K; ++i) { rk[i] = r; r += un[i] ? 1 : 0; }
  }
  // the largest unhit value is rank 0: the first lane with an unhit entry
  float zf = ninf;
#pragma unroll
  for (int i = K - 1; i >= 0; --i) zf = un[i] ? z[i] : zf;
  const float mt = readlane_f32(zf, __ffsll((unsigned long long)__ballot(cnt != 0u)) - 1);
  const float zo = (h.tout != 0u) ? kfloat(h.tout) : ninf;
  if (!(mt > ninf) || !(zo < mt)) return false;
  const float zend = (n > K * kWave) ? kfloat(readlane_u32(ent_key(e[K - 1]), kWave - 1)) : ninf;
  if (!(zend < mt)) return false;
  float hm = ninf;   // the largest penalised hit: sampling.cpp:26, then :16
  if (__ballot(hraw > ninf)) {
    const float hy = pen_exact(wave_max_dpp(hraw), c.pen);
    hm = c.temp_on ? hy / c.temp : hy;
  }
  if (!(hm < mt)) return false;

  C4S_PHASE(5);
  const double eps = rel_eps(V);
  const double dm = (double)h.m0 - (double)mt;
  const double rho = (dm == 0.0) ? 1.0 : exp(dm);
  const double S = (h.s0 - dsum) * rho;
  const double err = (h.err + derr + fabs(dsum) * 0x1p-50) * rho +
                     (dm > 0.0 ? 0x1p-23 * ((40.0 + dm) * S + (double)V * 0x1p-50) : 0.0) + eps * S;
  if (!(1.0 - (double)c.p > 0.0)) return false;   // dense rows take the other paths
  const uint64_t st = xorshift64(rng);
  const double u = unit_from_state(st);
  const double pS = (double)c.p * S;
  const double marg = (double)c.p * err + eps * S;
  const bool approx = dm == 0.0;
  const double dmass = approx ? 0x1p-23 : 0.0;
  C4S_PHASE(6);
  double em[K];
  bool need = false;
#pragma unroll
  for (int i = 0; i < K; ++i) {
    const bool stored = approx && mk[i] >= 0x1p-100f;
    em[i] = (un[i] && stored) ? (double)mk[i] : 0.0;
    need |= un[i] && !stored;
  }
  if (__ballot(need)) {
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const double x = exp((double)(z[i] - mt));
      const bool stored = approx && mk[i] >= 0x1p-100f;
      em[i] = (un[i] && !stored) ? x : em[i];
    }
  }
  double ls = 0.0;
#pragma unroll
  for (int i = 0; i < K; ++i) ls += em[i];
  const double inc = wave_scan_f64(ls);
  double ab = inc - ls;
  double abv[K];
  bool unsure = false, tiny = false;
  int qloc = 0x7fffffff;
#pragma unroll
  for (int i = 0; i < K; ++i) {
    abv[i] = ab;
    const double D = ab - pS;
    unsure |= un[i] && rk[i] >= c.min_keep && !(fabs(D) > marg + (eps + dmass) * ab);
    tiny |= un[i] && D < 0.0 && em[i] < 0x1p-1000;
    if (un[i] && D >= 0.0) qloc = min(qloc, rk[i]);
    ab += em[i];
  }
  C4S_PHASE(7);
  if (__ballot(unsure) || __ballot(tiny)) return false;
  const uint64_t qb = __ballot(qloc != 0x7fffffff);
  if (!qb) return false;   // the cut lies past these ranks
  const int q = max((int)readlane_u32((uint32_t)qloc, __ffsll((unsigned long long)qb) - 1), c.min_keep);
  if (q > nu) return false;
  float zs = ninf;
  bool has = false;
#pragma unroll
  for (int i = 0; i < K; ++i) {
    const bool m = un[i] && rk[i] == q - 1;
    zs = m ? z[i] : zs;
    has |= m;
  }
  const int lq = __ffsll((unsigned long long)__ballot(has)) - 1;
  const float zq1 = readlane_f32(zs, lq);
  if (!(zo < zq1) || !(zend < zq1) || !(hm < zq1)) return false;
  if (si) {
    double a1 = 0.0, a2 = 0.0;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const bool m = un[i] && rk[i] == q - 1;
      a1 = m ? abv[i] : a1;
      a2 = m ? abv[i] + em[i] : a2;
    }
    si->kind = 1;
    si->q = q;
    si->chk1 = q - 1 >= c.min_keep;
    si->zcut = zq1;
    si->mt = mt;
    si->S = S;
    si->rho = rho;
    si->err = err;
    si->eps = eps;
    si->dmass = dmass;
    si->p = (double)c.p;
    si->A1 = readlane_f64(a1, lq);
    si->A2 = readlane_f64(a2, lq);
  }
  // Id-order draw (text2semantic.cpp:150-165) over the kept ranks: every entry
  // of the list's first np writes its stored mass, value and id (-1 unless
  // kept) at its id-order place among them (the scan's place bytes); four
  // places a lane, one prefix scan, decide. First with the masses above, then
  // exact, then replayed.
  const int np = min(n, K * kWave);
#pragma unroll
  for (int i = 0; i < K; ++i) {   // positions past np write the trash entry
    const int pp = (p0 + i < np) ? (int)((pl >> (8 * i)) & 255u) : kListLarge;
    cs.lm[pp] = mk[i];
    cs.lz[pp] = z[i];
    cs.lid[pp] = (un[i] && rk[i] < q) ? ent_id(e[i]) : -1;
  }
  wave_sync();
  C4S_PHASE(11);
  float pm[K], pz[K];
  int pid[K];
#pragma unroll
  for (int i = 0; i < K; ++i) {
    const int pp = K * lane + i;
    pm[i] = cs.lm[pp];
    pz[i] = cs.lz[pp];
    const int rid = cs.lid[pp];
    pid[i] = pp < np ? rid : -1;
  }
  C4S_PHASE(8);
  auto draw = [&](bool exact_only, double eps_add) __attribute__((always_inline)) -> int {
    double ed[K], pr[K];
    bool need2 = false;
#pragma unroll
    for (int i = 0; i < K; ++i) {
      const bool v = pid[i] >= 0;
      const bool stp = approx && !exact_only && pm[i] >= 0x1p-100f;
      ed[i] = (v && stp) ? (double)pm[i] : 0.0;
      need2 |= v && !stp;
    }
    if (__ballot(need2)) {
#pragma unroll
      for (int i = 0; i < K; ++i) {
        const bool v = pid[i] >= 0;
        const bool stp = approx && !exact_only && pm[i] >= 0x1p-100f;
        const double x = exp((double)(pz[i] - mt));
        ed[i] = (v && !stp) ? x : ed[i];
      }
    }
    pr[0] = ed[0];
#pragma unroll
    for (int i = 1; i < K; ++i) pr[i] = pr[i - 1] + ed[i];
    const double sinc = wave_scan_f64(pr[K - 1]);
    const double r = u * readlane_f64(sinc, kWave - 1);
    const double base = sinc - pr[K - 1];
    double ha = 0.0, hp = 0.0;
    int hpos = -1;
#pragma unroll
    for (int i = K - 1; i >= 0; --i) {   // the first place reaching r wins
      const double nx = base + pr[i];
      if (ed[i] > 0.0 && nx >= r) { hpos = K * lane + i; ha = nx; hp = i ? base + pr[i - 1] : base; }
    }
    const uint64_t hb = __ballot(hpos >= 0);
    if (!hb) return -1;
    const int f = __ffsll((unsigned long long)hb) - 1;
    const double af = readlane_f64(ha, f), pf = readlane_f64(hp, f);
    const double eps2 = rel_eps(V) + eps_add;
    if (!(r > 0.0 && (af - r > eps2 * af) && (r - pf > eps2 * r))) return -1;
    int hid = -1;
#pragma unroll
    for (int i = 0; i < K; ++i) hid = (hpos == K * lane + i) ? pid[i] : hid;
    return (int)readlane_u32((uint32_t)hid, f);
  };
  int tok = -1;
  o.dex = 0;
  if (approx) tok = draw(false, 0x1p-22);
  if (tok < 0) tok = draw(true, 0.0);
  if (tok < 0) {   // text2semantic.cpp:152-164 sequentially in id order with exact masses
    o.dex = 1;
    int res = 0;
    if (lane == 0) {
      double total = 0.0;
      for (int pp = 0; pp < np; ++pp)
        if (cs.lid[pp] >= 0) total += exp((double)(cs.lz[pp] - mt));
      const double rr = u * total;
      res = V - 1;
      if (rr <= 0.0) {
        res = 0;
      } else {
        double acc = 0.0;
        for (int pp = 0; pp < np; ++pp) {
          if (cs.lid[pp] < 0) continue;
          const double ei = exp((double)(cs.lz[pp] - mt));
          acc += ei;
          if (ei > 0.0 && rr <= acc) { res = cs.lid[pp]; break; }
        }
      }
    }
    tok = (int)readlane_u32((uint32_t)res, 0);
  }
  o.tok = tok;
  o.kept = (uint32_t)q;
  rng = st;
  return true;
}

// Full-vocabulary step (wave 0). The summary words are in LDS at `sum`; also
// needs the correction of the masses for ids drawn during the stream (dsum,
// its error derr; per chunk in `cdelta`) and the raw row in LDS (`val`). The
// list is compacted lazily, 256 entries at a time, only as deep as the decision
// needs; cs provides the compaction and slot arrays.
template <class CS, class Acc>
__device__ __forceinline__ bool row_step(const SumHdr& h, const RowCfg& c, int V, const Acc& acc,
                         double dsum, double derr,
                         const uint64_t* sum, const double* cdelta, uint64_t& rng, CS& cs,
                         StepOut& o, SpecInfo* si = nullptr) {
  const int lane = lane_id();
  o.why = kWhySummary;
  if (h.flags & 1u) return false;
  const int n = h.n;
  const float ninf = neg_inf();
  const uint64_t* lst = sum;
  const float* ly = reinterpret_cast<const float*>(sum + kYW);
  // This call's generation tags the id-order slots it fills (a kernel starts
  // with generation 0; the slots are cleared at the first call and on wrap).
  uint32_t gen = cs.gen + 1u;
  if (gen == 1u || gen >= (1u << 22)) {
#pragma unroll
    for (int i = 0; i < kSlotsPerLane; ++i) cs.inv[(i << 6) | lane] = 0u;
    gen = 1u;
  }
  if (lane == 0) cs.gen = gen;
  int nb = 0, nu = 0;
  float hm = ninf;
  // list block [nb, nb + 256): unhit entries to their ranks, penalised hits into
  // hm (four consecutive entries per lane)
  auto compact = [&]() __attribute__((always_inline)) {
    const int p0 = nb + 4 * lane;
    uint64_t e[4];
    bool hit[4], un[4];
    uint32_t cu = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = (p0 + i < n) ? lst[p0 + i] : 0ull;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool v = p0 + i < n;
      // every lane reads its bitmap word (no branch around the load)
      const bool drawn = acc.hit(v ? ent_id(e[i]) : 0);
      hit[i] = c.pen_on & v & drawn;
      un[i] = v & !hit[i];
      cu += un[i] ? 1u : 0u;
    }
    const uint32_t inc = wave_scan_u32(cu);
    int rk = nu + (int)(inc - cu);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int id = ent_id(e[i]);
      if (un[i]) {
        cs.lz[rk] = kfloat(ent_key(e[i]));
        cs.lm[rk] = ly[p0 + i];
        cs.lid[rk] = id;
        cs.lslot[rk] = ent_rank(e[i]);
        cs.inv[slot_pos(ent_rank(e[i]))] = (gen << 10) | (uint32_t)rk;
        ++rk;
      }
      if (hit[i]) {   // sampling.cpp:26, then :16; a drawn id is never in H0, so its value is the raw one
        const float y = pen_exact(acc.hval(id), c.pen);
        hm = fmaxf(hm, c.temp_on ? y / c.temp : y);
      }
    }
    nu += (int)readlane_u32(inc, kWave - 1);
    nb = min(n, nb + 4 * kWave);
  };
  // every list entry past the compacted ones is at or below this value
  auto zend = [&]() -> float { return nb >= n ? ninf : kfloat(ent_key(lst[nb - 1])); };
  compact();
  while (nu == 0 && nb < n) compact();
  C4S_PHASE(8);
  o.why = kWhyShort;
  if (nu == 0) return false;
  wave_sync();
  const float mt = cs.lz[0];
  const float zo = (h.tout != 0u) ? kfloat(h.tout) : ninf;
  o.why = kWhyBound;
  if (!(mt > ninf) || !(zo < mt)) return false;
  while (nb < n && !(zend() < mt)) compact();
  o.why = kWhyHit;
  if (!(wave_max_dpp(hm) < mt)) return false;   // the maximum is an unhit entry

  const double eps = rel_eps(V);
  // S = (chunk masses - corrections) * exp(m0 - mt). When the maximum moved,
  // fl(z - mt) against fl(z - m0) + (m0 - mt): relative 2^-23 (|d| + m0 - mt)
  // per mass, with sum(e |d|) <= 40 S + V 2^-50 (e |d| < 2^-50 once |d| > 40).
  const double dm = (double)h.m0 - (double)mt;
  const double rho = (dm == 0.0) ? 1.0 : exp(dm);
  const double S = (h.s0 - dsum) * rho;
  const double err = (h.err + derr + fabs(dsum) * 0x1p-50) * rho +
                     (dm > 0.0 ? 0x1p-23 * ((40.0 + dm) * S + (double)V * 0x1p-50) : 0.0) + eps * S;
  const double thr = 1.0 - (double)c.p;
  const uint64_t st = xorshift64(rng);
  const double u = unit_from_state(st);
  C4S_PHASE(9);

  if (thr > 0.0) {
    // nucleus cut on the unhit entries in rank order: removed iff above >= p * S
    const double pS = (double)c.p * S;
    const double marg = (double)c.p * err + eps * S;
    // While the maximum did not move, the entries' masses come from the summary
    // (the reference's mass rounded to fp32: relative error below 2^-23 when
    // at least 2^-100); otherwise, and for tinier ones, exp is evaluated.
    const bool approx = dm == 0.0;
    const double dmass = approx ? 0x1p-23 : 0.0;
    auto mass_of = [&](int rk, bool exact_only) __attribute__((always_inline)) -> double {
      const float m = cs.lm[rk];
      return (approx && !exact_only && m >= 0x1p-100f) ? (double)m : exp((double)(cs.lz[rk] - mt));
    };
    // Masses of up to R ranks per lane: the stored ones are read first; exp runs
    // only if some lane needs it (the maximum moved, a tiny mass, or exact_only).
    auto masses_of = [&](const int* rks, const bool* vs, double* out, int R, bool exact_only)
        __attribute__((always_inline)) {
      bool need = false;
      for (int j = 0; j < R; ++j) {
        const float m = vs[j] ? cs.lm[rks[j]] : 0.0f;
        out[j] = (double)m;
        need |= vs[j] & !(approx & !exact_only & (m >= 0x1p-100f));
      }
      if (__ballot(need))
        for (int j = 0; j < R; ++j)
          if (vs[j] && !(approx && !exact_only && out[j] >= 0x1p-100)) out[j] = exp((double)(cs.lz[rks[j]] - mt));
    };
    // Up to 256 ranks per iteration, four per lane, one prefix scan; the list
    // is compacted further only once the compacted ranks are used up.
    double carry = 0.0;
    int q = -1, rdone = 0;
    while (q < 0) {
      C4S_PHASE(4);
      while (rdone >= nu && nb < n) compact();
      if (rdone >= nu) break;
      wave_sync();
      C4S_PHASE(5);
      double e4[4], ls = 0.0;
      int rk4[4];
      bool v4[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        rk4[i] = rdone + 4 * lane + i;
        v4[i] = rk4[i] < nu;
      }
      masses_of(rk4, v4, e4, 4, false);
#pragma unroll
      for (int i = 0; i < 4; ++i) ls += e4[i];
      const double inc = wave_scan_f64(ls);
      double ab = carry + inc - ls;
      bool unsure = false, tiny = false;
      int qloc = -1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rk = rdone + 4 * lane + i;
        const bool v = rk < nu;
        const double D = ab - pS;
        unsure |= v && rk >= c.min_keep && !(fabs(D) > marg + (eps + dmass) * ab);
        tiny |= v && D < 0.0 && e4[i] < 0x1p-1000;
        if (v && D >= 0.0 && qloc < 0) qloc = rk;
        ab += e4[i];
      }
      o.why = kWhyMargin;
      if (__ballot(unsure)) return false;
      o.why = kWhyTiny;   // subnormal kept masses may differ between libm implementations
      if (__ballot(tiny)) return false;
      const uint64_t rm = __ballot(qloc >= 0);
      if (rm) q = max((int)readlane_u32((uint32_t)qloc, __ffsll((unsigned long long)rm) - 1), c.min_keep);
      carry = readlane_f64(carry + inc, kWave - 1);
      rdone = min(nu, rdone + 4 * kWave);
      C4S_PHASE(6);
    }
    C4S_PHASE(10);
    o.why = kWhyDeep;
    if (q < 0 || q > nu) return false;   // the cut lies below the list
    const float zq1 = cs.lz[q - 1];
    while (nb < n && !(zend() < zq1)) compact();
    C4S_PHASE(15);
    o.why = kWhyBound;
    if (!(zo < zq1)) return false;
    o.why = kWhyHit;
    if (!(wave_max_dpp(hm) < zq1)) return false;
    if (si) {   // the masses above ranks q - 1 and q, summed again over the kept ranks
      double a1 = 0.0;
      for (int r0 = 0; r0 < q - 1; r0 += kWave) a1 += (r0 + lane < q - 1) ? mass_of(r0 + lane, false) : 0.0;
      a1 = wave_sum_dpp(a1);
      si->kind = 1;
      si->q = q;
      si->chk1 = q - 1 >= c.min_keep;
      si->zcut = zq1;
      si->mt = mt;
      si->S = S;
      si->rho = rho;
      si->err = err;
      si->eps = eps;
      si->dmass = dmass;
      si->p = (double)c.p;
      si->A1 = a1;
      si->A2 = a1 + mass_of(q - 1, false);
    }
    // The draw on the kept ranks [0, q): first with the masses above (a decision
    // inside their error is not replayed), then, if needed, with exact masses.
    if (q <= kWave) {   // kept ranks are the first chunk: lane = rank
      const bool kept = lane < q;
      const int kid = kept ? cs.lid[lane] : 0, ks = kept ? cs.lslot[lane] : 0;
      int tok = -1;
      if (approx)
        tok = lane_draw<kSlotBits>(kept, kid, ks, kept ? mass_of(lane, false) : 0.0, u, V, o.dex, 0x1p-22, false);
      if (tok < 0) tok = lane_draw<kSlotBits>(kept, kid, ks, kept ? mass_of(lane, true) : 0.0, u, V, o.dex);
      o.tok = tok;
    } else {
      o.tok = inv_draw(cs, gen, q, approx, mt, u, V, o);
    }
    C4S_PHASE(12);
    o.kept = (uint32_t)q;
    rng = st;
    return true;
  }

  if (!dense_draw(h, c, V, acc, sum, cdelta, u, S, rho, err, mt, o, si)) return false;
  rng = st;
  return true;
}

// Exact step on the row in LDS (raw values at `val`): penalty of H0 and the
// stream's ids, then the chain of the single-kernel path.
__device__ __forceinline__ int exact_step(float* val, double* E, const uint32_t* bmAll, const RowCfg& c,
                                       int V, Scratch& sh, uint64_t& rng, uint32_t* stp) {
  if (c.pen_on) {
    penalise_chunk(val, bmAll, V, c.pen);
    __syncthreads();
  }
  int tok = 0;
  if (!(fast_topk_applies(c, V) &&
        fast_topk_any(val, V, c, sh, reinterpret_cast<unsigned char*>(E), rng, tok, nullptr, stp))) {
    LdsRow src{val, E, V, 0u, false};
    tok = run_chain(src, sh, c, rng, nullptr, stp);
  }
  return tok;
}


// ---- fast chain kernels ------------------------------------------------------------------
//
// Greedy and top-k rows need only their candidate list: one wavefront per
// row, no barriers, summaries four steps ahead in registers. Full-vocabulary
// rows also stream their raw row for the corrections: four wavefronts per
// row. A step the summary cannot settle runs the exact chain inside the
// kernel, on the row read into LDS.

// State load shared by both: returns false when the row has nothing to do in
// this chunk (finished, or stopped; a stopped row reports -1 for the rest of
// the chunk, text2semantic.cpp:304).
__device__ __forceinline__ bool fast_begin(const StreamArgs& a, const StreamWs& w, int row, int nthr,
                                           int& s_first) {
  uint32_t* stw = w.state + (size_t)row * kStateWords;
  s_first = (int)stw[kStNext];
  if (stw[kStDone] != 0u || s_first >= w.s_end) {
    if (stw[kStDone] != 0u) {
      for (int s = s_first + (int)threadIdx.x; s < w.s_end; s += nthr) a.out_tok[(int64_t)s * a.n_rows + row] = -1;
      if (threadIdx.x == 0) stw[kStNext] = (uint32_t)w.s_end;
    }
    if (threadIdx.x == 0 && a.stats && w.s_end == a.n_steps)   // nothing left: the final statistics
      for (int i = 0; i < 4; ++i) a.stats[4 * (int64_t)row + i] = stw[kStStats + i];
    return false;
  }
  return true;
}

// H0 bitmap from the history and the bitmap of ids drawn during the stream
// (kept in the state without H0 ids).
__device__ __forceinline__ void fast_bitmaps(const StreamArgs& a, const uint32_t* stw, int row, int V,
                                             int nthr, uint32_t* bmH0, uint32_t* bmN, bool block) {
  const int nwords = bitmap_words(V);
  for (int i = threadIdx.x; i < nwords; i += nthr) bmH0[i] = 0u;
  if (block) __syncthreads(); else wave_sync();
  const int64_t h0 = a.hist_off[row], h1 = a.hist_off[row + 1];
  for (int64_t j = h0 + threadIdx.x; j < h1; j += nthr) {
    const int id = a.hist_ids[j];
    if (id >= 0 && id < V) atomicOr(&bmH0[id >> 5], 1u << (id & 31));   // sampling.cpp:24
  }
  if (block) __syncthreads(); else wave_sync();
  for (int i = threadIdx.x; i < nwords; i += nthr) bmN[i] = stw[kStBits + i] & ~bmH0[i];
  if (block) __syncthreads(); else wave_sync();
}

__device__ __forceinline__ void fast_end(const StreamArgs& a, const StreamWs& w, int row, int V, int nthr,
                                         int s, bool done, uint64_t rng, const uint32_t* acc,
                                         const uint32_t* bmN) {
  uint32_t* stw = w.state + (size_t)row * kStateWords;
  if (threadIdx.x == 0) {
    a.rng[row] = rng;
    stw[kStDone] = done ? 1u : 0u;
    stw[1] = acc[0]; stw[2] = acc[1]; stw[3] = acc[2]; stw[4] = acc[3];
    stw[kStNext] = (uint32_t)s;
    if (a.stats && s >= a.n_steps) {   // the row's last step: its statistics
      uint32_t* o = a.stats + 4 * (int64_t)row;
      o[0] = acc[0]; o[1] = acc[1]; o[2] = acc[2]; o[3] = acc[3];
    }
  }
  const int nwords = bitmap_words(V);
  for (int i = threadIdx.x; i < nwords; i += nthr) stw[kStBits + i] = bmN[i];
}

struct ListRegs {
  uint64_t e0, e1, hw;   // entries lane and lane + 64, header word lane (lanes < 8)
  float y0, y1;          // their values before the temperature
};

// Penalises the ids set in bm (text2semantic.cpp:142 via sampling.cpp:26),
// one wave: lane l takes the bitmap words l + 64 j.
__device__ __forceinline__ void penalise_wave(float* val, const uint32_t* bm, int V, float pen) {
  const int nwords = bitmap_words(V);
  for (int wi = lane_id(); wi < nwords; wi += kWave) {
    uint32_t b = bm[wi];
    while (b) {
      const int i = 32 * wi + __ffs(b) - 1;
      b &= b - 1;
      if (i < V) val[i] = pen_exact(val[i], pen);
    }
  }
}

// Candidate-list rows, one wave per row. A step the list cannot decide runs
// exactly in the kernel: the row read into LDS, the penalty of H0 and the
// stream's ids, the whole chain (its top_p exact pass sorts in the per-row
// key buffer).
__global__ __launch_bounds__(kWave) void k_stream_list(StreamArgs a, StreamWs w) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ ChainSh cs;
  __shared__ ScratchT<1> xs;   // exact steps
  __shared__ uint32_t bmH0[kStateWords], bmN[kStateWords];
  const int row = blockIdx.x;
  const int V = a.vocab;
  const int lane = lane_id();
  const RowCfg c = make_cfg(0u, V, row, a.temp, a.top_k, a.top_p, a.pen, nullptr, a.do_sample);
  if (stream_mode(c, V) != kModeList) return;
  int s_first;
  if (!fast_begin(a, w, row, kWave, s_first)) return;
  const uint32_t* stw = w.state + (size_t)row * kStateWords;
  fast_bitmaps(a, stw, row, V, kWave, bmH0, bmN, false);
  uint64_t rng = a.rng[row];
  uint32_t acc[4] = {stw[1], stw[2], stw[3], stw[4]};
  bool done = false;

  auto load = [&](int s, ListRegs& r) __attribute__((always_inline)) {
    const uint64_t* sw = sum_words(w, a.n_rows, s, row);
    r.e0 = sw[lane];
    r.e1 = sw[lane + kWave];
    r.hw = sw[kHdrW + (lane & 7)];   // lanes 0..3 are read
    const float* sy = reinterpret_cast<const float*>(sw + kYW);
    r.y0 = sy[lane];
    r.y1 = sy[lane + kWave];
  };
  float* xrow = reinterpret_cast<float*>(smem);   // exact steps (with the sort buffer)
  auto exact = [&](int s) -> int {
    const float* p = a.logits + (int64_t)row * a.ld + (int64_t)s * a.step_stride;
    for (int i = lane; i < V; i += kWave) xrow[i] = p[i];
    wave_sync();
    if (c.pen_on) {   // H0 and the stream's ids are disjoint: each id once
      penalise_wave(xrow, bmH0, V, c.pen);
      penalise_wave(xrow, bmN, V, c.pen);
    }
    __syncthreads();
    LdsRowNC src{xrow, V, 0u, false, w.sortbuf + (int64_t)row * w.sort_stride, (uint32_t)(w.sort_stride * 4)};
    const int tok = run_chain(src, xs, c, rng, nullptr, xs.step_stats);
    __syncthreads();
    if (lane == 0) {
      acc[0] |= xs.step_stats[0];
      acc[1] += 1u;
      acc[2] += xs.step_stats[2];
      acc[3] += xs.step_stats[3];
    }
    return tok;
  };
  auto step = [&](int s, ListRegs& r) __attribute__((always_inline)) {
    int32_t* outp = a.out_tok + (int64_t)s * a.n_rows + row;
    C4S_LIST_PHASE(0);
    const SumHdr h = hdr_lanes(r.hw);
    const uint64_t e0 = (lane < h.n) ? r.e0 : 0ull;
    const uint64_t e1 = (lane + kWave < h.n) ? r.e1 : 0ull;
    const float yb0 = r.y0, yb1 = r.y1;
    if (s + 4 < w.s_end) load(s + 4, r);
    C4S_LIST_PHASE(1);
    StepOut o{0, 0u, 0u, 0u};
    const bool ok = list_step(h, e0, e1, yb0, yb1, c, V, BitsHit{bmN}, rng, cs, o);
    if (!ok && lane == 0) acc[0] |= 1u << (20 + o.why);
    const int tok = ok ? o.tok : exact(s);
    if (lane == 0) {
      *outp = tok;
      if (ok) {
        acc[0] |= 32u | 1u;
        acc[2] += o.dex;
        acc[3] += o.kept;
      }
      // text2semantic.cpp:333-334: the stop token is not appended
      if (c.pen_on && tok != a.stop_token && tok >= 0 && tok < V && !bit_of(bmH0, tok))
        bmN[tok >> 5] |= 1u << (tok & 31);
    }
    wave_sync();
    C4S_LIST_PHASE(7);
    if (tok == a.stop_token) done = true;
  };

  ListRegs P0{}, P1{}, P2{}, P3{};
  load(s_first, P0);
  if (s_first + 1 < w.s_end) load(s_first + 1, P1);
  if (s_first + 2 < w.s_end) load(s_first + 2, P2);
  if (s_first + 3 < w.s_end) load(s_first + 3, P3);
  // A stopped row leaves the loop (no step path skips its prefetch) and
  // reports -1 afterwards.
  int s = s_first;
  while (s < w.s_end) {
    step(s, P0);
    if (++s >= w.s_end || done) break;
    step(s, P1);
    if (++s >= w.s_end || done) break;
    step(s, P2);
    if (++s >= w.s_end || done) break;
    step(s, P3);
    if (++s >= w.s_end || done) break;
  }
  if (done) {
    for (int s2 = s + lane; s2 < w.s_end; s2 += kWave) a.out_tok[(int64_t)s2 * a.n_rows + row] = -1;
    s = w.s_end;
  }
  fast_end(a, w, row, V, kWave, s, done, rng, acc, bmN);
}

constexpr int NTC = 256;
constexpr int NWC = NTC / kWave;

// ---- pipelined full-vocabulary chain ------------------------------------------------
//
// Wave 0 decides step s while waves 1-3 prepare step s+1: each helper wave
// owns a third of the ids, loads that third of the raw row and of the summary
// straight into LDS (global_load_lds, three slots in rotation, two steps
// ahead) and computes the mass corrections of step s+1 for the ids drawn
// during the stream up to step s-1 (fp32 masses with their error bounds).
// Wave 0 then adds the exact correction of the one token it drew at step s-1
// and decides; a decision inside the error bound is retried once with exact
// corrections computed by all four wavefronts. The drawn-id bitmap is kept twice (by
// step parity) so that wave 0 can record step s's token while the helpers read
// the set of step s. Barriers only wait for LDS traffic; the helpers wait for
// their own loads before reading them. A step the summary cannot settle runs
// the exact chain with all four wavefronts on the staged row.

constexpr int kSumQuads = (kSumWords + 1) / 2;          // 16-byte units of a summary
constexpr int kSumWordsP = 2 * kSumQuads;               // summary slot in LDS (words)
constexpr int kSumQPerWave = (kSumQuads + 2) / 3;       // per helper wave
constexpr int kDrawnList = 512;                         // drawn ids listed per helper wave
static_assert((size_t)kSumWordsP * 8 <= kSumStride, "whole quads stay inside a summary");
static_assert(kHdrW % 2 == 0, "header words start a quad");

// Segment results of the pipelined row chain, word 0.
constexpr uint64_t kSegIdle = 0;                   // the row did not run in this chunk
constexpr uint64_t kSegRan = 1ull << 62;           // ran to the segment's end
constexpr uint64_t kSegStop = 1ull << 63;          // | stop step: ended by the stop token
constexpr uint64_t kSegEmpty = 3ull << 60;         // no steps in this segment

struct RowPSh {
  double cdelta[2][kMaxChunks];   // corrections per chunk, by step parity
  double cdx[kMaxChunks];         // exact corrections of a retried step
  double wd[2][4];                // helper waves' correction sums, by step parity
  double we[2][4];                // and their error bounds
  double xd[NWC];                 // exact corrections of a retried step, per wave
  uint32_t inv[kListLarge + 1];   // id-order slot -> (generation << 10) | unhit rank; + a trash word
  uint32_t gen;                   // generation of the last row step
  float lz[kListLarge + 1];   // by unhit rank; + a trash entry
  float lm[kListLarge + 1];
  int lid[kListLarge + 1];
  int lslot[kListLarge];
  alignas(16) uint64_t hdr[2][3][8];   // per parity and helper wave: header copy
  int dlist[3][kDrawnList];       // per helper wave: drawn ids of its range (while they fit)
  int nt[2];                      // token of step s when it joined bmN, else -1, at [s & 1]
  uint64_t rng;
  int tok[2];                     // token of step s at [s & 1]
  int flag[2];                    // 1: wave 0 decided step s, at [s & 1]
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef const __attribute__((address_space(1))) void* glb_ptr_t;

// Workgroup barrier for LDS traffic only: this wave's LDS operations are
// complete, global loads in flight stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// Waits for every global load (and LDS load) this wave has in flight.
__device__ __forceinline__ void wait_loads() {
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
}

// Ids of helper wave h (0..2): [lo, hi), fixed for the row (multiples of 64
// apart from the ends), and the body quads holding any of them (a quad that
// straddles a boundary is loaded by both neighbours).
struct Third {
  int q0, q1;    // body quads
  int lo, hi;    // ids
};
__device__ __forceinline__ int third_bound(int V, int h) {
  return h <= 0 ? 0 : (h >= 3 ? V : ((h * V / 3) & ~63));
}
__device__ __forceinline__ Third third_of(const RowShape& r, int V, int h) {
  Third th;
  th.lo = third_bound(V, h);
  th.hi = third_bound(V, h + 1);
  th.q0 = 0;
  th.q1 = 0;
  if (th.hi > th.lo && r.nq > 0) {
    th.q0 = max(0, (th.lo - r.head) >> 2);
    const int last = th.hi - 1 - r.head;   // id offset of the last id from the body start
    th.q1 = last < 0 ? 0 : min(r.nq, (last >> 2) + 1);
    th.q0 = min(th.q0, th.q1);
  }
  return th;
}

// Loads of step s issued by helper wave h into its LDS slot: its third of the
// row, its share of the summary quads, and its own copy of the header.
__device__ __forceinline__ void dma_step(const float* p, int V, const uint64_t* sg, float* rowslot,
                                         uint64_t* sumslot, uint64_t* hdrcopy, int h) {
  const int lane = lane_id();
  const RowShape r = row_shape(p, V);
  float* val = rowslot + ((4 - r.head) & 3);   // val + head is 16-byte aligned
  const Third th = third_of(r, V, h);
  for (int q0 = th.q0; q0 < th.q1; q0 += kWave) {
    const int q = q0 + lane;
    if (q < th.q1)
      __builtin_amdgcn_global_load_lds((glb_ptr_t)(p + r.head + 4 * q), (lds_ptr_t)(val + r.head + 4 * q0),
                                       16, 0, 0);
  }
  if (lane < r.head && lane >= th.lo && lane < th.hi)
    __builtin_amdgcn_global_load_lds((glb_ptr_t)(p + lane), (lds_ptr_t)(val), 4, 0, 0);
  const int e0 = r.head + 4 * r.nq;
  if (lane < r.tail && e0 + lane >= th.lo && e0 + lane < th.hi)
    __builtin_amdgcn_global_load_lds((glb_ptr_t)(p + e0 + lane), (lds_ptr_t)(val + e0), 4, 0, 0);
  const int s0 = h * kSumQPerWave, s1 = min(kSumQuads, s0 + kSumQPerWave);
  for (int q0 = s0; q0 < s1; q0 += kWave) {
    const int q = q0 + lane;
    if (q < s1)
      __builtin_amdgcn_global_load_lds((glb_ptr_t)(sg + 2 * q), (lds_ptr_t)(sumslot + 2 * q0), 16, 0, 0);
  }
  if (lane < 4)
    __builtin_amdgcn_global_load_lds((glb_ptr_t)(sg + kHdrW + 2 * lane), (lds_ptr_t)(hdrcopy), 16, 0, 0);
}

// Corrections of one step over ids [lo, hi) drawn during the stream (bmN,
// never in H0): the mass of the raw value minus that of the penalised value,
// added to its chunk (unless cdelta is null: only the full-vocabulary draw
// reads chunks). fp32 masses with their error bound (el), or exact ones.
__device__ __forceinline__ double corrections_range(const float* val, int lo, int hi, const uint32_t* bmN,
                                                    const SumHdr& hh, const RowCfg& c, double* cdelta,
                                                    bool exact, double& el) {
  double dl = 0.0;
  el = 0.0;
  if (hh.flags & 1u) return 0.0;
  const MassCoef mk = mass_coef(c, hh.m0);
  const float rpen = 1.0f / c.pen;
  for (int wb = lo >> 5; wb < ((hi + 31) >> 5); ++wb) {
    uint32_t bits = bmN[wb];
    const int b0 = 32 * wb;
    if (b0 < lo) bits &= ~0u << (lo - b0);
    if (b0 + 32 > hi) bits &= (hi - b0 >= 32) ? ~0u : ((1u << (hi - b0)) - 1u);
    while (bits) {
      const int id = b0 + __ffs(bits) - 1;
      bits &= bits - 1;
      const float x = val[id];
      double d;
      if (exact) {
        d = mass_exact(x, c, hh.m0) - mass_exact(pen_exact(x, c.pen), c, hh.m0);
      } else {
        float er0, er1;
        const float m_raw = mass_approx(x, mk, er0);
        const float m_pen = mass_approx(pen_approx(x, c.pen, rpen), mk, er1);
        d = (double)m_raw - (double)m_pen;
        el += (double)er0 + (double)er1;
      }
      if (cdelta) atomicAdd(&cdelta[chunk_of(id, hh.head, hh.nchunk)], d);
      dl += d;
    }
  }
  return dl;
}

// Lists the ids of [lo, hi) set in bmN into list (at most kDrawnList of them,
// in id order); returns how many there are (wave-uniform).
__device__ __forceinline__ int list_drawn(const uint32_t* bmN, int lo, int hi, int* list) {
  const int lane = lane_id();
  const int wa = lo >> 5, wz = (hi + 31) >> 5;
  auto word = [&](int wb) __attribute__((always_inline)) -> uint32_t {
    uint32_t bits = bmN[wb];
    const int b0 = 32 * wb;
    if (b0 < lo) bits &= ~0u << (lo - b0);
    if (b0 + 32 > hi) bits &= (hi - b0 >= 32) ? ~0u : ((1u << (hi - b0)) - 1u);
    return bits;
  };
  int n = 0;
  for (int w0 = wa; w0 < wz; w0 += kWave) {
    const int wb = w0 + lane;
    uint32_t bits = wb < wz ? word(wb) : 0u;
    const uint32_t cnt = (uint32_t)__popc(bits);
    const uint32_t incl = wave_scan_u32(cnt);
    int p = n + (int)(incl - cnt);
    while (bits) {
      if (p < kDrawnList) list[p] = 32 * wb + __ffs(bits) - 1;
      bits &= bits - 1;
      ++p;
    }
    n += (int)readlane_u32(incl, kWave - 1);
  }
  wave_sync();
  return n;
}

// fp32 corrections of one step by helper wave h over the listed drawn ids of
// its range (n of them, all listed); returns the wave's total and (in el) its
// error bound, in all lanes, and adds to the chunks unless cdelta is null.
// Two ids per lane at a time.
__device__ __forceinline__ double listed_corrections(const float* val, const int* list, int n, const SumHdr& hh,
                                                     const RowCfg& c, double* cdelta, double& el) {
  const int lane = lane_id();
  el = 0.0;
  if (hh.flags & 1u) return 0.0;
  const MassCoef mk = mass_coef(c, hh.m0);
  const float rpen = 1.0f / c.pen;
  double dl = 0.0, ell = 0.0;
  for (int j = lane; j < n; j += 2 * kWave) {
    const bool v1 = j + kWave < n;
    const int i0 = list[j], i1r = list[min(j + kWave, kDrawnList - 1)];   // both reads together
    const int i1 = v1 ? i1r : i0;
    const float x0 = val[i0], x1 = val[i1];
    float e00, e01, e10, e11;
    const float a0 = mass_approx(x0, mk, e00), b0 = mass_approx(pen_approx(x0, c.pen, rpen), mk, e01);
    const float a1 = mass_approx(x1, mk, e10), b1 = mass_approx(pen_approx(x1, c.pen, rpen), mk, e11);
    const double d0 = (double)a0 - (double)b0;
    if (cdelta) atomicAdd(&cdelta[chunk_of(i0, hh.head, hh.nchunk)], d0);
    dl += d0;
    ell += (double)e00 + (double)e01;
    if (v1) {
      const double d1 = (double)a1 - (double)b1;
      if (cdelta) atomicAdd(&cdelta[chunk_of(i1, hh.head, hh.nchunk)], d1);
      dl += d1;
      ell += (double)e10 + (double)e11;
    }
  }
  el = wave_sum_dpp(ell);
  return wave_sum_dpp(dl);
}

// fp32 corrections of one step by helper wave h over its range: from its list
// while the drawn ids fit, else per lane from the bitmap.
__device__ __forceinline__ double helper_corrections(const float* val, int V, int h, const uint32_t* bmN,
                                                     const SumHdr& hh, const RowCfg& c, double* cdelta,
                                                     const int* list, int n, double& el) {
  if (n <= kDrawnList) return listed_corrections(val, list, n, hh, c, cdelta, el);
  const int lane = lane_id();
  const int lo_h = third_bound(V, h), hi_h = third_bound(V, h + 1);
  const int ch = (hi_h - lo_h + kWave - 1) / kWave;
  const int lo = min(hi_h, lo_h + lane * ch), hi = min(hi_h, lo + ch);
  const double dl = corrections_range(val, lo, hi, bmN, hh, c, cdelta, false, el);
  el = wave_sum_dpp(el);
  return wave_sum_dpp(dl);
}

__global__ __launch_bounds__(NTC) void k_stream_rowp(StreamArgs a, StreamWs w) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ RowPSh ps;
  __shared__ ScratchT<NWC> xs;   // exact steps
  __shared__ uint32_t bmH0[kStateWords], bmNb[2][kStateWords];
  const int row = blockIdx.x;
  const int V = a.vocab;
  const int t = threadIdx.x, lane = lane_id(), wv = wave_id(), hw = wv - 1;
  const RowCfg c = make_cfg(0u, V, row, a.temp, a.top_k, a.top_p, a.pen, nullptr, a.do_sample);
  if (stream_mode(c, V) != kModeRow) return;
  // A row without penalty has independent steps but for the RNG, which every
  // step advances once: workgroup (row, g) takes the g-th of nseg segments
  // of the steps, from the RNG state jumped ahead, and k_stream_segfix
  // settles the stop token and the carried state. A penalty makes the steps
  // depend on the tokens drawn: one segment.
  const int nseg = c.pen_on ? 1 : w.nseg;
  const int g = blockIdx.y;
  if (g >= nseg) return;
  uint64_t* segres = nseg > 1 ? w.segres + ((size_t)row * w.nseg + g) * 4 : nullptr;
  int s_first;
  if (!fast_begin(a, w, row, NTC, s_first)) {
    if (nseg > 1 && t == 0) segres[0] = kSegIdle;
    return;
  }
  int s_end = w.s_end;
  uint64_t rng0 = a.rng[row];
  if (nseg > 1) {
    const int L = (s_end - s_first + nseg - 1) / nseg;
    const int lo = min(s_end, s_first + g * L), hi = min(s_end, lo + L);
    if (lo >= hi) {
      if (t == 0) segres[0] = kSegEmpty;
      return;
    }
    for (int i = s_first; i < lo; ++i) rng0 = xorshift64(rng0);
    s_first = lo;
    s_end = hi;
  }
  C4S_ROW_TIME(0);
  // Per-chunk corrections feed only the full-vocabulary draw (top_p >= 1);
  // nucleus rows use their totals.
  const bool dense = !(1.0 - (double)c.p > 0.0);
  const uint32_t* stw = w.state + (size_t)row * kStateWords;
  uint64_t* sumslots = reinterpret_cast<uint64_t*>(smem);
  float* rowslots = reinterpret_cast<float*>(smem + 3 * (size_t)kSumWordsP * 8);
  const int RS = vpad(V) + 4;
  auto sumslot = [&](int s) { return sumslots + (size_t)(s % 3) * kSumWordsP; };
  auto rowslot = [&](int s) { return rowslots + (size_t)(s % 3) * RS; };
  const float* base = a.logits + (int64_t)row * a.ld;
  auto rowp = [&](int s) { return base + (int64_t)s * a.step_stride; };
  auto rowval = [&](int s) { return rowslot(s) + ((4 - row_shape(rowp(s), V).head) & 3); };
  uint32_t* sortbuf = w.sortbuf + (int64_t)row * w.sort_stride;

  // prologue: bitmaps, the first two steps in flight, corrections of the first
  fast_bitmaps(a, stw, row, V, NTC, bmH0, bmNb[s_first & 1], true);
  const int nwords = bitmap_words(V);
  for (int i = t; i < nwords; i += NTC) bmNb[(s_first + 1) & 1][i] = bmNb[s_first & 1][i];
  for (int i = t; i < 2 * kMaxChunks; i += NTC) (&ps.cdelta[0][0])[i] = 0.0;
  if (t == 0) ps.gen = 0u;
  if (wv > 0) {
    dma_step(rowp(s_first), V, sum_words(w, a.n_rows, s_first, row), rowslot(s_first), sumslot(s_first),
             ps.hdr[s_first & 1][hw], hw);
    if (s_first + 1 < s_end)
      dma_step(rowp(s_first + 1), V, sum_words(w, a.n_rows, s_first + 1, row), rowslot(s_first + 1),
               sumslot(s_first + 1), ps.hdr[(s_first + 1) & 1][hw], hw);
  }
  __syncthreads();   // cdelta cleared, bitmaps in place (also drains the loads)
  int ndrawn = 0;    // helper wave: drawn ids of its range (listed while they fit)
  if (wv > 0) {
    const uint64_t* hc = ps.hdr[s_first & 1][hw];
    const SumHdr hh = hdr_words(hc[0], hc[1], hc[2], hc[3], hc[4]);
    ndrawn = list_drawn(bmNb[s_first & 1], third_bound(V, hw), third_bound(V, hw + 1), ps.dlist[hw]);
    double d = 0.0, e = 0.0;
    if (c.pen_on)
      d = helper_corrections(rowval(s_first), V, hw, bmNb[s_first & 1], hh, c,
                             dense ? ps.cdelta[s_first & 1] : nullptr,
                             ps.dlist[hw], ndrawn, e);
    if (lane == 0) { ps.wd[s_first & 1][hw] = d; ps.we[s_first & 1][hw] = e; }
  }
  if (t == 0) ps.rng = rng0;
  uint64_t rng = rng0;
  uint32_t acc[4] = {0u, 0u, 0u, 0u};   // a segment's statistics start at zero
  if (t == 0 && nseg == 1) { acc[0] = stw[1]; acc[1] = stw[2]; acc[2] = stw[3]; acc[3] = stw[4]; }
  int tprev = -1;        // wave 0: token of the previous step when it joined bmN
  bool done = false;
  __syncthreads();

  int s = s_first;
  for (; s < s_end; ++s) {
    const int par = s & 1;
    const uint32_t* bmN = bmNb[par];
    int sflag = 0, stok = -1;   // the step's outcome, read after its barrier
    // Attempt 0: wave 0 decides with the fp32 corrections while the helpers
    // prepare step s+1. Attempt 1 (a decision inside their error bound): all
    // four wavefronts compute the exact corrections of step s, wave 0 decides
    // again. One call site of row_step keeps it inlined.
    for (int attempt = 0;; ++attempt) {
      if (attempt == 1) {
        const int ch = (V + NTC - 1) / NTC;
        const int lo = min(V, t * ch), hi = min(V, lo + ch);
        if (dense)
          for (int i = t; i < kMaxChunks; i += NTC) ps.cdx[i] = 0.0;
        __syncthreads();
        double el;
        double d = corrections_range(rowval(s), lo, hi, bmN, hdr_from(sumslot(s)), c, dense ? ps.cdx : nullptr,
                                     true, el);
        d = wave_sum_dpp(d);
        if (lane == 0) ps.xd[wv] = d;
        __syncthreads();
      }
      if (wv == 0) {
        C4S_PHASE(0);
        const uint64_t* sw = sumslot(s);
        const float* val = rowval(s);
        const SumHdr h = hdr_from(sw);
        double ds, de;
        double* cd;
        const float xprev = val[tprev >= 0 ? tprev : 0];   // read with the header words
        if (attempt == 0) {
          cd = ps.cdelta[par];
          ds = ps.wd[par][0] + ps.wd[par][1] + ps.wd[par][2];
          de = ps.we[par][0] + ps.we[par][1] + ps.we[par][2];
          if (tprev >= 0 && !(h.flags & 1u)) {   // step s-1's token, not in the helpers' sums
            const float x = xprev;
            const MassCoef mk = mass_coef(c, h.m0);
            float e0, e1;
            const float m1 = mass_approx(x, mk, e0);
            const float m2 = mass_approx(pen_approx(x, c.pen, 1.0f / c.pen), mk, e1);
            const double d = (double)m1 - (double)m2;
            if (dense) {
              if (lane == 0) cd[chunk_of(tprev, h.head, h.nchunk)] += d;
              wave_sync();
            }
            ds += d;
            de += (double)e0 + (double)e1;
          }
        } else {   // the exact sums cover bmN(s), step s-1's token included
          cd = ps.cdx;
          ds = ps.xd[0] + ps.xd[1] + ps.xd[2] + ps.xd[3];
          de = 0.0;
        }
        C4S_PHASE(1);
        StepOut o{0, 0u, 0u, 0u};
        // the register path when the scan's cut hint leaves room for hits within 64 ranks
        const int hint = (int)(uint32_t)sw[kHdrW + 5];
        const RowAcc rac{val, bmN, bmH0};
        const bool ok = ((dense || hint <= kLanesHint) && row_step_lanes(h, c, V, rac, ds, de, sw, cd, rng, o)) ||
                        (!dense && hint <= 4 * kWave && row_step_lanes4(h, c, V, rac, ds, de, sw, rng, ps, o)) ||
                        row_step(h, c, V, rac, ds, de, sw, cd, rng, ps, o);
        const bool retry = attempt == 0 && !ok && c.pen_on && (o.why == kWhyDraw || o.why == kWhyMargin);
        C4S_PHASE(2);
        if (attempt == 0 && dense)
          for (int i = lane; i < kMaxChunks; i += kWave) ps.cdelta[par][i] = 0.0;
        // The token joins bmN of step s+1 unless it is the stop token
        // (text2semantic.cpp:333-334) or already penalised; both bitmap words
        // are read by every lane at once (tok is wave-uniform).
        const int tok = o.tok;
        const int tc = (tok >= 0 && tok < V) ? tok : 0;
        const uint32_t wh = bmH0[tc >> 5], wn = bmN[tc >> 5];
        const bool fresh = ok && c.pen_on && tok != a.stop_token && tok == tc && !(((wh | wn) >> (tc & 31)) & 1u);
        if (lane == 0) {
          ps.flag[par] = ok ? 1 : (retry ? 2 : 0);
          ps.rng = rng;
          if (ok) {
            ps.tok[par] = tok;
            acc[0] |= 64u | 1u;
            acc[2] += o.dex;
            acc[3] += o.kept;
            uint32_t* nb = bmNb[par ^ 1];   // becomes the set of step s+1
            if (tprev >= 0) atomicOr(&nb[tprev >> 5], 1u << (tprev & 31));
            if (fresh) atomicOr(&nb[tok >> 5], 1u << (tok & 31));
            ps.nt[par] = fresh ? tok : -1;
          } else if (!retry) {
            acc[0] |= 1u << (20 + o.why);
          }
        }
        if (ok) tprev = fresh ? tok : -1;
      } else if (attempt == 0) {
        C4S_HELPER_PHASE(0);
        wait_loads();   // step s+1 is in LDS (this wave's range)
        C4S_HELPER_PHASE(1);
        if (s > s_first) {   // the previous step's token joined bmN: list it if it is ours
          const int nt = ps.nt[par ^ 1];
          if (nt >= third_bound(V, hw) && nt < third_bound(V, hw + 1)) {
            if (lane == 0 && ndrawn < kDrawnList) ps.dlist[hw][ndrawn] = nt;
            ++ndrawn;
            wave_sync();
          }
        }
        if (s + 1 < s_end) {
          const int sn = s + 1;
          const uint64_t* hc = ps.hdr[sn & 1][hw];
          const SumHdr hh = hdr_words(hc[0], hc[1], hc[2], hc[3], hc[4]);
          double d = 0.0, e = 0.0;
          if (c.pen_on)
            d = helper_corrections(rowval(sn), V, hw, bmN, hh, c, dense ? ps.cdelta[sn & 1] : nullptr,
                                   ps.dlist[hw], ndrawn, e);
          if (lane == 0) { ps.wd[sn & 1][hw] = d; ps.we[sn & 1][hw] = e; }
        }
        C4S_HELPER_PHASE(2);
        if (s + 2 < s_end)
          dma_step(rowp(s + 2), V, sum_words(w, a.n_rows, s + 2, row), rowslot(s + 2), sumslot(s + 2),
                   ps.hdr[s & 1][hw], hw);
        C4S_HELPER_PHASE(3);
        if (hw == 0 && lane == 0 && s > s_first) a.out_tok[(int64_t)(s - 1) * a.n_rows + row] = ps.tok[par ^ 1];
      }
      lds_barrier();
      C4S_PHASE(3);
      C4S_HELPER_PHASE(4);
      sflag = ps.flag[par];   // read together with the token
      stok = ps.tok[par];
      if (sflag != 2) break;
    }
    if (!sflag) {
      // text2semantic.cpp:142-166 on the whole staged row: penalty over H0 and
      // the stream's ids (disjoint sets, so each id once), then the chain.
      rng = ps.rng;
      float* val = rowval(s);
      if (c.pen_on) {
        penalise_chunk<NTC>(val, bmH0, V, c.pen);
        penalise_chunk<NTC>(val, bmN, V, c.pen);
      }
      __syncthreads();
      LdsRowNC src{val, V, 0u, false, sortbuf, (uint32_t)(w.sort_stride * 4)};
      const int tok = run_chain(src, xs, c, rng, nullptr, xs.step_stats);
      if (t == 0) {
        const uint32_t* stp = xs.step_stats;
        ps.rng = rng;
        ps.tok[par] = tok;
        acc[0] |= stp[0];
        acc[1] += 1u;
        acc[2] += stp[2];
        acc[3] += stp[3];
        uint32_t* nb = bmNb[par ^ 1];
        if (tprev >= 0) nb[tprev >> 5] |= 1u << (tprev & 31);
        tprev = -1;
        if (c.pen_on && tok != a.stop_token && tok >= 0 && tok < V && !bit_of(bmH0, tok) && !bit_of(bmN, tok)) {
          nb[tok >> 5] |= 1u << (tok & 31);
          tprev = tok;
        }
        ps.nt[par] = tprev;
      }
      tprev = (int)readlane_u32((uint32_t)tprev, 0);
      __syncthreads();
      stok = ps.tok[par];
    }
    if (stok == a.stop_token) {
      done = true;
      ++s;
      break;
    }
  }
  // s: first step not decided here. The last decided token, and -1 after a stop.
  wait_loads();
  __syncthreads();
  if (t == 0 && s > s_first) a.out_tok[(int64_t)(s - 1) * a.n_rows + row] = ps.tok[(s - 1) & 1];
  for (int s2 = s + t; s2 < s_end; s2 += NTC) a.out_tok[(int64_t)s2 * a.n_rows + row] = -1;
  if (nseg > 1) {
    if (t == 0) {
      segres[0] = done ? (kSegStop | (uint64_t)(uint32_t)(s - 1)) : kSegRan;
      segres[1] = ps.rng;
      segres[2] = (uint64_t)acc[0] | ((uint64_t)acc[1] << 32);
      segres[3] = (uint64_t)acc[2] | ((uint64_t)acc[3] << 32);
    }
  } else {
    fast_end(a, w, row, V, NTC, s_end, done, ps.rng, acc, bmNb[s & 1]);
  }
  C4S_ROW_TIME(1);
}

// Settles the step segments of rows without penalty: the first stop token
// ends the row (later segments' tokens become -1), the RNG state is the one
// after the last step decided, the statistics add up.
__global__ __launch_bounds__(kWave) void k_stream_segfix(StreamArgs a, StreamWs w) {
  const int row = blockIdx.x;
  const int t = threadIdx.x;
  const RowCfg c = make_cfg(0u, a.vocab, row, a.temp, a.top_k, a.top_p, a.pen, nullptr, a.do_sample);
  if (stream_mode(c, a.vocab) != kModeRow || c.pen_on || w.nseg <= 1) return;
  const uint64_t* sr = w.segres + (size_t)row * w.nseg * 4;
  if (sr[0] == kSegIdle) return;   // nothing ran: the row was done or had no steps here
  uint32_t* stw = w.state + (size_t)row * kStateWords;
  uint32_t acc[4] = {stw[1], stw[2], stw[3], stw[4]};
  uint64_t rng = a.rng[row];
  int stop = -1;
  for (int g = 0; g < w.nseg && stop < 0; ++g) {
    const uint64_t st = sr[4 * g];
    if (st == kSegEmpty) continue;
    rng = sr[4 * g + 1];
    acc[0] |= (uint32_t)sr[4 * g + 2];
    acc[1] += (uint32_t)(sr[4 * g + 2] >> 32);
    acc[2] += (uint32_t)sr[4 * g + 3];
    acc[3] += (uint32_t)(sr[4 * g + 3] >> 32);
    if ((st & kSegStop) != 0u) stop = (int)(uint32_t)st;
  }
  if (stop >= 0)
    for (int s = stop + 1 + t; s < w.s_end; s += kWave) a.out_tok[(int64_t)s * a.n_rows + row] = -1;
  if (t == 0) {
    a.rng[row] = rng;
    stw[kStDone] = stop >= 0 ? 1u : 0u;
    stw[1] = acc[0]; stw[2] = acc[1]; stw[3] = acc[2]; stw[4] = acc[3];
    stw[kStNext] = (uint32_t)w.s_end;
    if (a.stats && w.s_end == a.n_steps) {
      uint32_t* o = a.stats + 4 * (int64_t)row;
      o[0] = acc[0]; o[1] = acc[1]; o[2] = acc[2]; o[3] = acc[3];
    }
  }
}

// ---- finisher: every remaining step, exact steps inline -------------------------------
__global__ __launch_bounds__(NT) void k_stream_chain(StreamArgs a, StreamWs w) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ Scratch sh;
  __shared__ ChainSh cs;
  const int row = blockIdx.x;
  const int V = a.vocab;
  const int t = threadIdx.x, lane = lane_id(), wv = wave_id();
  const RowCfg c = make_cfg(0u, V, row, a.temp, a.top_k, a.top_p, a.pen, nullptr, a.do_sample);
  const int mode = stream_mode(c, V);
  if (mode != kModeExact) return;   // the fast chains finish these rows
  LdsLayout L = lds_layout(smem, V);
  const int nwords = bitmap_words(V);
  uint32_t* bmH0 = L.bitmap + nwords;
  uint32_t* bmN = bmH0 + nwords;   // ids drawn during the stream, not in H0
  uint32_t* stw = w.state + (size_t)row * kStateWords;
  // The fast rounds initialised the state; rows they finished have nothing left.
  const int s_first = (int)stw[kStNext];
  if (s_first >= w.s_end) {
    if (t == 0 && a.stats && w.s_end == a.n_steps)
      for (int i = 0; i < 4; ++i) a.stats[4 * (int64_t)row + i] = stw[kStStats + i];
    return;
  }
  for (int i = t; i < nwords; i += NT) bmH0[i] = 0u;
  for (int i = t; i < kMaxChunks; i += NT) cs.cdelta[i] = 0.0;
  if (t == 0) cs.gen = 0u;
  __syncthreads();
  {
    const int64_t h0 = a.hist_off[row], h1 = a.hist_off[row + 1];
    for (int64_t j = h0 + t; j < h1; j += NT) {
      const int id = a.hist_ids[j];
      if (id >= 0 && id < V) atomicOr(&bmH0[id >> 5], 1u << (id & 31));   // sampling.cpp:24
    }
  }
  __syncthreads();
  for (int i = t; i < nwords; i += NT) {
    bmN[i] = stw[kStBits + i] & ~bmH0[i];
    L.bitmap[i] = bmH0[i] | bmN[i];
  }
  uint64_t rng = a.rng[row];
  bool done = stw[kStDone] != 0u;
  uint32_t acc[4] = {0u, 0u, 0u, 0u};
  if (t == 0) { acc[0] = stw[1]; acc[1] = stw[2]; acc[2] = stw[3]; acc[3] = stw[4]; }
  __syncthreads();
  const float* base = a.logits + (int64_t)row * a.ld;
  const float rpen = 1.0f / c.pen;
  // Summary of the next step in flight as vector loads (barriers do not wait
  // for them): list rows, wave 0, three words per lane of the header and the
  // small list; full-vocabulary rows, one word per thread of the whole summary.
  uint64_t pw0 = 0, pw1 = 0, pw2 = 0, pw3 = 0;
  auto load_sum = [&](int s) {
    const uint64_t* sw = sum_words(w, a.n_rows, s, row);
    if (mode == kModeList) {
      if (wv == 0) {
        pw0 = sw[lane];
        pw1 = sw[lane + kWave];
        pw2 = (lane < 8) ? sw[kHdrW + lane] : 0ull;
        pw3 = sw[kYW + lane];   // values of entries 2 lane, 2 lane + 1
      }
    } else if (t < kSumWords) {
      pw0 = sw[t];
    }
  };
  auto stage_sum = [&]() {
    if (mode == kModeList) {
      if (wv == 0) {
        cs.sum[lane] = pw0;
        cs.sum[lane + kWave] = pw1;
        if (lane < 8) cs.sum[kHdrW + lane] = pw2;
        cs.sum[kYW + lane] = pw3;
        wave_sync();
      }
    } else if (t < kSumWords) {
      cs.sum[t] = pw0;
    }
  };
  const bool summaries = mode != kModeExact;
  if (summaries) load_sum(s_first);

  // fetch of the raw row of step s (full-vocabulary and exact rows)
  RowFetch pf;
  const bool stream_rows = mode != kModeList;
  if (stream_rows && !done) fetch_row(base + (int64_t)s_first * a.step_stride, V, pf);

  for (int s = s_first; s < w.s_end; ++s) {
    int32_t* outp = a.out_tok + (int64_t)s * a.n_rows + row;
    if (done) {
      if (t == 0) *outp = -1;
      continue;
    }
    const float* cur = base + (int64_t)s * a.step_stride;
    float* val = L.val;
    if (stream_rows) {
      val = store_row(cur, V, pf, L.val);
      if (mode == kModeRow && s + 1 < w.s_end) fetch_row(cur + a.step_stride, V, pf);
    }
    if (summaries) stage_sum();
    uint32_t pbits = 0;
    StepOut o{0, 0u, 0u, 0u};
    if (mode == kModeList) {
      if (wv == 0) {
        const SumHdr h = hdr_from(cs.sum);
        const uint64_t* lst = cs.sum;
        const uint64_t e0 = (lane < h.n) ? lst[lane] : 0ull;
        const uint64_t e1 = (lane + kWave < h.n) ? lst[lane + kWave] : 0ull;
        const float* ly = reinterpret_cast<const float*>(cs.sum + kYW);
        const bool ok = list_step(h, e0, e1, ly[lane], ly[lane + kWave], c, V, BitsHit{bmN}, rng, cs, o);
        if (lane == 0) { cs.bi[0] = ok ? 1 : 0; cs.bi[1] = o.tok; cs.bi[2] = ok ? (int)o.kept : (int)o.why; cs.bi[3] = (int)o.dex; cs.rng = rng; }
      }
      pbits = 32u;
      __syncthreads();
    } else if (mode == kModeRow) {
      __syncthreads();   // row and summary in LDS
      const SumHdr h = hdr_from(cs.sum);
      const uint32_t hflags = h.flags;
      const float hm0 = h.m0;
      const int hhead = h.head, hnch = h.nchunk;
      // corrections for ids drawn during the stream (never in H0)
      double dl = 0.0, el = 0.0;
      if (!(hflags & 1u) && c.pen_on) {
        const MassCoef mk = mass_coef(c, hm0);
        const int ch = odd_chunk(V);
        const int lo = min(V, t * ch), hi = min(V, lo + ch);
        if (lo < hi) {
          const int w0 = lo >> 5;
          uint64_t bits = ((uint64_t)(L.bitmap[w0] & ~bmH0[w0])) |
                          ((uint64_t)(L.bitmap[w0 + 1] & ~bmH0[w0 + 1]) << 32);
          bits >>= (lo - 32 * w0);
          bits &= (hi - lo >= 64) ? ~0ull : ((1ull << (hi - lo)) - 1ull);
          while (bits) {
            const int id = lo + __ffsll((unsigned long long)bits) - 1;
            bits &= bits - 1;
            const float x = val[id];
            double d;
            {   // fp32 masses: their error bounds join the decision margins
              float er0, er1;
              const float m_raw = mass_approx(x, mk, er0);
              const float m_pen = mass_approx(pen_approx(x, c.pen, rpen), mk, er1);
              d = (double)m_raw - (double)m_pen;
              el += (double)er0 + (double)er1;
            }
            atomicAdd(&cs.cdelta[chunk_of(id, hhead, hnch)], d);
            dl += d;
          }
        }
      }
      dl = wave_sum_f64(dl);
      el = wave_sum_f64(el);
      if (lane == 0) { cs.wd[wv] = dl; cs.we[wv] = el; }
      __syncthreads();
      if (wv == 0) {
        double ds = 0.0, de = 0.0;
        for (int i = 0; i < NW; ++i) { ds += cs.wd[i]; de += cs.we[i]; }
        const bool ok = row_step(h, c, V, RowAcc{val, bmN, bmH0}, ds, de, cs.sum, cs.cdelta, rng, cs, o);
        for (int i = lane; i < kMaxChunks; i += kWave) cs.cdelta[i] = 0.0;
        if (lane == 0) { cs.bi[0] = ok ? 1 : 0; cs.bi[1] = o.tok; cs.bi[2] = ok ? (int)o.kept : (int)o.why; cs.bi[3] = (int)o.dex; cs.rng = rng; }
      }
      pbits = 64u;
      __syncthreads();
    } else {
      if (t == 0) { cs.bi[0] = 0; cs.rng = rng; }
      __syncthreads();
    }
    const bool ok = cs.bi[0] != 0;
    rng = cs.rng;
    if (summaries && s + 1 < w.s_end) load_sum(s + 1);
    int tok = 0;
    uint32_t stq[4] = {0u, 0u, 0u, 0u};
    if (ok) {
      tok = cs.bi[1];
      stq[0] = pbits | 1u;
      stq[2] = (uint32_t)cs.bi[3];
      stq[3] = (uint32_t)cs.bi[2];
    } else {
      if (t == 0 && mode != kModeExact) acc[0] |= 1u << (20 + (uint32_t)cs.bi[2]);
      if (mode == kModeList) {   // the row was not staged: fetch it now
        RowFetch f1;
        fetch_row(cur, V, f1);
        val = store_row(cur, V, f1, L.val);
      }
      __syncthreads();
      uint32_t* stp = a.stats ? sh.step_stats : nullptr;
      tok = exact_step(val, L.E, L.bitmap, c, V, sh, rng, stp);
      if (t == 0) {
        if (stp) { stq[0] = stp[0]; stq[2] = stp[2]; stq[3] = stp[3]; }
        stq[1] = (mode == kModeExact) ? 0u : 1u;
      }
      // the prefetched row is not kept across the exact step (register pressure)
      if (stream_rows && s + 1 < w.s_end) fetch_row(cur + a.step_stride, V, pf);
    }
    if (t == 0) {
      *outp = tok;
      acc[0] |= stq[0];
      acc[1] += stq[1];
      acc[2] += stq[2];
      acc[3] += stq[3];
      // text2semantic.cpp:333-334: the stop token is not appended
      if (tok != a.stop_token && tok >= 0 && tok < V) {
        L.bitmap[tok >> 5] |= 1u << (tok & 31);
        if (!bit_of(bmH0, tok)) bmN[tok >> 5] |= 1u << (tok & 31);
      }
    }
    if (tok == a.stop_token) done = true;
    __syncthreads();
  }
  if (t == 0) {
    a.rng[row] = rng;
    stw[kStDone] = done ? 1u : 0u;
    stw[1] = acc[0]; stw[2] = acc[1]; stw[3] = acc[2]; stw[4] = acc[3];
    stw[kStNext] = (uint32_t)w.s_end;
    if (a.stats && w.s_end == a.n_steps) {
      uint32_t* o = a.stats + 4 * (int64_t)row;
      o[0] = acc[0]; o[1] = acc[1]; o[2] = acc[2]; o[3] = acc[3];
    }
  }
  for (int i = t; i < nwords; i += NT) stw[kStBits + i] = bmN[i];
}


// ---- speculative full-vocabulary chain --------------------------------------------
//
// One workgroup per row: wave kSpecVW validates, the others decide. A step
// depends on earlier steps only through the ids drawn before it (the
// penalty) and its RNG state, which is fixed. Decider k takes steps
// s_first + k, + kSpecND, ... and decides each against the ids drawn before
// the validated frontier when it starts (at most kSpecND - 1 steps behind).
// Wave 0 takes the steps in order and accepts a decision when the ids drawn
// since provably leave it as it is: none of them is kept by it (none reaches
// the cut value, or the maximum of a dense row, and none is its token), and
// the mass their penalty removes moves neither the nucleus cut (ranks q - 1
// and q keep their sides with the error margins) nor, for the dense draw,
// r = u * S out of the drawn id's prefix interval. Otherwise wave 0 decides
// the step again with every drawn id. Only summaries are staged: a decider
// gathers the drawn ids' raw values from the step's row in HBM, and wave 0
// gathers, for each decided token, its raw values in the next 64 steps, so
// that the check reads LDS only. A step no summary path settles stops every
// wave for the exact chain on the row read into LDS.

constexpr int kSpecND = 5;                 // decider waves
constexpr int NTS = (kSpecND + 1) * kWave;
constexpr int kSpecGv = 1024;              // ids a call can draw (its steps at most)
constexpr int kRing = 16;                  // per-token value rows kept by wave 0
constexpr int kSpecVW = 3;                 // the checking wave: alone on its SIMD (waves go to SIMDs in turn)
constexpr int kHist = 8;                   // steps of tokens the checking wave keeps in registers
static_assert(kHist >= kSpecND, "history covers the steps a decision can lag");
static_assert(kRing >= 2 * kSpecND, "ring covers the steps a check looks back");

struct SpecCS {   // a decider's rank and slot arrays (what row_step needs)
  uint32_t inv[kListLarge + 1];
  uint32_t gen;
  float lz[kListLarge + 1];
  float lm[kListLarge + 1];
  int lid[kListLarge + 1];
  int lslot[kListLarge];
};

struct SpecRec {
  int tag;   // step of this decision (written last), -1 none
  int tok;
  int nF;    // drawn ids the decision knew (a prefix of the drawn list)
  int F;     // ... those drawn before step F
  int fresh; // tok is none of them, nor in H0, nor the stop token
  int ok;
  int ring;  // the decider gathers tok's values of the next steps into ring row tag
  uint32_t why, dex, kept;
  double ds, de;
  // The check, with DL the mass the ids drawn since remove (sum of m(x) -
  // m(pen x)), Y its error bound plus |DL| 2^-50, Da the part of DL from ids
  // below tok. kind 1 (nucleus): no new id reaches zlim (the cut value),
  // w (DL + Y) < g1 (rank q - 1 stays kept) and w (DL - Y) > g2 (rank q stays
  // out). kind 2 (dense): no new id reaches zlim (the maximum) nor is tok,
  // w (u DL - ome Da - 2 Y) > g1 and w (Da - ome u DL - 2 Y) > g2 (r stays
  // inside tok's prefix interval). Any other kind: decide again.
  int kind;
  float zlim;
  double g1, g2, w, u, ome;
  float ma, mb, mrel;   // mass coefficients of the step (mass_coef of its m0)
  SpecInfo si;
};

struct SpecCtl {
  int ringtag[kRing];   // step whose token's values ring row r holds (landed), else -1
  int snap;   // (frontier << 16) | drawn ids before the frontier
  int halt;   // step of an exact chain run by every wave, else -1
  int done;
  int err;
  int qend;   // first step not decided
  int stopped;
  int tok;
  uint64_t rng;
  uint32_t acc[4];
};

// Drawn set of one decision: ids whose drawn index is below nF; raw values of
// drawn ids by drawn index in gv, any other raw value from the row in HBM.
struct SpecAcc {
  const uint16_t* didx;
  const float* gv;
  const uint32_t* bmH0;
  const float* grow;
  int nF;
  __device__ __forceinline__ bool hit(int id) const { return (int)didx[id] < nF; }
  __device__ __forceinline__ float hval(int id) const { return gv[min((int)didx[id], kSpecGv - 1)]; }
  __device__ __forceinline__ float raw(int id) const { return grow[id]; }
  __device__ __forceinline__ bool pen(int id) const { return bit_of(bmH0, id) || hit(id); }
};

struct SpecLayout {
  size_t didx, tok, tstep, ring, tout, dec, stride, o_gv, o_cd, o_cs, total;
};
__host__ __device__ inline size_t al16(size_t x) { return (x + 15) & ~(size_t)15; }
__host__ __device__ inline SpecLayout spec_layout(int V) {
  SpecLayout L;
  L.didx = 0;
  L.tok = al16(L.didx + 2 * (size_t)V);
  L.tstep = al16(L.tok + 4 * (size_t)kSpecGv);
  L.ring = al16(L.tstep + 2 * (size_t)kSpecGv);
  L.tout = al16(L.ring + 4 * (size_t)kRing * kWave);
  L.dec = al16(L.tout + 2 * (size_t)kSpecGv);
  L.o_gv = al16(8 * (size_t)kSumWordsP);
  L.o_cd = al16(L.o_gv + 4 * (size_t)kSpecGv);
  L.o_cs = al16(L.o_cd + 8 * (size_t)kMaxChunks);
  L.stride = al16(L.o_cs + sizeof(SpecCS));
  size_t dec = (size_t)kSpecND * L.stride;
  const size_t rowb = al16(4 * ((size_t)vpad(V) + 4));   // the exact chain's row over the deciders' areas
  L.total = L.dec + (dec > rowb ? dec : rowb);
  return L;
}

template <class CS, class Acc>
__device__ __forceinline__ bool spec_decide(const SumHdr& h, const RowCfg& c, int V, const Acc& acc, double ds,
                                            double de, const uint64_t* sw, double* cd, uint64_t& r, CS& cs,
                                            StepOut& o, SpecInfo* si, bool dense) {
  const int hint = (int)(uint32_t)sw[kHdrW + 5];
  return ((dense || hint <= kLanesHint) && row_step_lanes(h, c, V, acc, ds, de, sw, cd, r, o, si)) ||
         (!dense && hint <= 4 * kWave && row_step_lanes4(h, c, V, acc, ds, de, sw, r, cs, o, si)) ||
         row_step(h, c, V, acc, ds, de, sw, cd, r, cs, o, si);
}

// Corrections of one step over drawn indices [0, n): the mass of the raw value
// minus that of the penalised one (fp32 with the error bound el, or exact),
// added per chunk into cd for dense rows (cd cleared by the caller).
__device__ __forceinline__ double spec_corrections(const float* gv, const int* tokl, int n, const SumHdr& h,
                                                   const RowCfg& c, double* cd, bool exact, double& el) {
  const int lane = lane_id();
  double dl = 0.0, ell = 0.0;
  if (!(h.flags & 1u)) {
    const MassCoef mk = mass_coef(c, h.m0);
    const float rpen = 1.0f / c.pen;
    for (int j0 = 0; j0 < n; j0 += 4 * kWave) {
      float x[4];
      int id[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {   // reads in bounds, issued together
        const int j = min(j0 + i * kWave + lane, kSpecGv - 1);
        x[i] = gv[j];
        id[i] = cd ? tokl[j] : 0;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (j0 + i * kWave + lane >= n) continue;
        double d;
        if (exact) {
          d = mass_exact(x[i], c, h.m0) - mass_exact(pen_exact(x[i], c.pen), c, h.m0);
        } else {
          float e0, e1;
          const float m1 = mass_approx(x[i], mk, e0);
          const float m2 = mass_approx(pen_approx(x[i], c.pen, rpen), mk, e1);
          d = (double)m1 - (double)m2;
          ell += (double)e0 + (double)e1;
        }
        if (cd) atomicAdd(&cd[chunk_of(id[i], h.head, h.nchunk)], d);
        dl += d;
      }
    }
  }
  el = wave_sum_dpp(ell);
  return wave_sum_dpp(dl);
}

// Volatile LDS accesses (p points into LDS). Through an LDS pointer: a
// generic (flat) access would also wait for this wave's global loads.
template <typename T>
__device__ __forceinline__ T vload(const T* p) {
  typedef const volatile __attribute__((address_space(3))) T LT;
  return *(LT*)(const __attribute__((address_space(3))) T*)p;
}
template <typename T>
__device__ __forceinline__ void vstore(T* p, T v) {
  typedef volatile __attribute__((address_space(3))) T LT;
  *(LT*)(__attribute__((address_space(3))) T*)p = v;
}
// One LDS word or-ed in place (ds_or_b32: no read back).
__device__ __forceinline__ void lds_or(uint32_t* p, uint32_t v) {
  __hip_atomic_fetch_or((__attribute__((address_space(3))) uint32_t*)p, v, __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_WORKGROUP);
}
// The fields of a record the check reads, read after its tag (see the checking wave).
struct RecView {
  int tag, nF, tok, F, ok, fresh, kind;
  float zlim, ma, mb, mrel;
  double g1, g2, w, u, ome;
  uint32_t dex, kept;
};
__device__ __forceinline__ RecView rec_view(const SpecRec& rc) {
  RecView v;
  v.tag = vload(&rc.tag);
  v.nF = vload(&rc.nF);
  v.tok = vload(&rc.tok);
  v.F = vload(&rc.F);
  v.ok = vload(&rc.ok);
  v.fresh = vload(&rc.fresh);
  v.kind = vload(&rc.kind);
  v.zlim = vload(&rc.zlim);
  v.ma = vload(&rc.ma);
  v.mb = vload(&rc.mb);
  v.mrel = vload(&rc.mrel);
  v.g1 = vload(&rc.g1);
  v.g2 = vload(&rc.g2);
  v.w = vload(&rc.w);
  v.u = vload(&rc.u);
  v.ome = vload(&rc.ome);
  v.dex = vload(&rc.dex);
  v.kept = vload(&rc.kept);
  return v;
}
__device__ __forceinline__ void lgkm_wait() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Waits until at most n of this wave's vector memory operations are in flight.
__device__ __forceinline__ void wait_vm(int n) {
  switch (n < 0 ? 0 : (n > 15 ? 15 : n)) {
    case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
    case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
    case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
    case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
    case 5: __builtin_amdgcn_s_waitcnt(0x0F75); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
    case 7: __builtin_amdgcn_s_waitcnt(0x0F77); break;
    case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
    case 9: __builtin_amdgcn_s_waitcnt(0x0F79); break;
    case 10: __builtin_amdgcn_s_waitcnt(0x0F7A); break;
    case 11: __builtin_amdgcn_s_waitcnt(0x0F7B); break;
    case 12: __builtin_amdgcn_s_waitcnt(0x0F7C); break;
    case 13: __builtin_amdgcn_s_waitcnt(0x0F7D); break;
    case 14: __builtin_amdgcn_s_waitcnt(0x0F7E); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F7F); break;
  }
}

// kForcedLimit: the bounded waits poll a.spin_max times (a test's limit);
// otherwise the compile-time default, so that the production instance's
// checking loop is built with a constant bound. (The checking wave's loop is
// sensitive to its control flow: an extra exit in the middle of it made the
// 1000-step call about 7% slower, so a wait that gives up only marks the row
// and the loop's own test ends it.)
template <bool kForcedLimit>
__global__ __launch_bounds__(NTS) void k_stream_spec(StreamArgs a, StreamWs w) {
  const int spin_max = kForcedLimit ? a.spin_max : kSpinMaxDefault;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ SpecRec recs[kSpecND];
  __shared__ SpecCtl ctl;
  __shared__ ScratchT<kSpecND + 1> xs;   // exact steps
  __shared__ uint32_t bmH0[kStateWords], bmN[kStateWords];
  const int row = blockIdx.x;
  const int V = a.vocab;
  const int t = threadIdx.x, lane = lane_id(), wv = wave_id();
  const RowCfg c = make_cfg(0u, V, row, a.temp, a.top_k, a.top_p, a.pen, nullptr, a.do_sample);
  if (stream_mode(c, V) != kModeRow) return;
  int s_first;
  if (!fast_begin(a, w, row, NTS, s_first)) return;
  const int s_end = w.s_end;
  const uint64_t rng0 = a.rng[row];
  const uint32_t* stw = w.state + (size_t)row * kStateWords;
  const SpecLayout L = spec_layout(V);
  uint16_t* didx = reinterpret_cast<uint16_t*>(smem + L.didx);
  int* tokl = reinterpret_cast<int*>(smem + L.tok);
  uint16_t* tstep = reinterpret_cast<uint16_t*>(smem + L.tstep);
  float* ring = reinterpret_cast<float*>(smem + L.ring);
  int16_t* tout = reinterpret_cast<int16_t*>(smem + L.tout);
  auto dbase = [&](int k) { return smem + L.dec + (size_t)k * L.stride; };
  auto dsum = [&](int k) { return reinterpret_cast<uint64_t*>(dbase(k)); };
  auto dgv = [&](int k) { return reinterpret_cast<float*>(dbase(k) + L.o_gv); };
  auto dcd = [&](int k) { return reinterpret_cast<double*>(dbase(k) + L.o_cd); };
  auto dcs = [&](int k) -> SpecCS& { return *reinterpret_cast<SpecCS*>(dbase(k) + L.o_cs); };
  const float* base = a.logits + (int64_t)row * a.ld;
  auto rowp = [&](int s) { return base + (int64_t)s * a.step_stride; };
  const bool dense = !(1.0 - (double)c.p > 0.0);
  const int nwords = bitmap_words(V);
  C4S_SPEC_DECL;

  // Prologue: H0 and the ids drawn in earlier chunks, listed in id order.
  fast_bitmaps(a, stw, row, V, NTS, bmH0, bmN, true);
  for (int i = t; i < V; i += NTS) didx[i] = 0xFFFFu;
  if (t < kSpecND) recs[t].tag = -1;
  __syncthreads();
  if (wv == 0) {
    int n = 0;
    for (int w0 = 0; w0 < nwords; w0 += kWave) {
      const int wb = w0 + lane;
      uint32_t bits = wb < nwords ? bmN[wb] : 0u;
      const uint32_t cnt = (uint32_t)__popc(bits);
      const uint32_t incl = wave_scan_u32(cnt);
      int p = n + (int)(incl - cnt);
      while (bits) {
        const int id = 32 * wb + __ffs(bits) - 1;
        bits &= bits - 1;
        if (p < kSpecGv && id < V) {
          tokl[p] = id;
          tstep[p] = 0;
          didx[id] = (uint16_t)p;
        }
        ++p;
      }
      n += (int)readlane_u32(incl, kWave - 1);
    }
    if (lane == 0) {
      ctl.snap = (s_first << 16) | min(n, kSpecGv);
      ctl.halt = -1;
      ctl.done = 0;
      ctl.err = n > kSpecGv ? 1 : 0;
      ctl.qend = s_first;
      ctl.stopped = 0;
      for (int i = 0; i < kRing; ++i) ctl.ringtag[i] = -1;
      ctl.rng = rng0;
      for (int i = 0; i < 4; ++i) ctl.acc[i] = stw[1 + i];
    }
  }
  __syncthreads();

  // Every wave runs the exact chain of step hq on the raw row read into LDS
  // over the deciders' areas (text2semantic.cpp:142-166); ends at a barrier.
  auto exact_all = [&](int hq) __attribute__((always_inline)) {
    __syncthreads();
    float* X = reinterpret_cast<float*>(smem + L.dec);
    const float* src = rowp(hq);
    for (int i = t; i < V; i += NTS) X[i] = src[i];
    __syncthreads();
    if (c.pen_on) {   // H0 and the stream's ids are disjoint: each id once
      penalise_chunk<NTS>(X, bmH0, V, c.pen);
      penalise_chunk<NTS>(X, bmN, V, c.pen);
    }
    __syncthreads();
    uint64_t r = ctl.rng;
    LdsRowNC srow{X, V, 0u, false, w.sortbuf + (int64_t)row * w.sort_stride, (uint32_t)(w.sort_stride * 4)};
    const int tok = run_chain(srow, xs, c, r, nullptr, xs.step_stats);
    __syncthreads();
    if (t == 0) {
      ctl.tok = tok;
      ctl.rng = r;
    }
    __syncthreads();
  };

  if (wv == kSpecVW) {
    // ---- the checking wave: takes the decisions in step order ----
    int q = s_first;
    int n = ctl.snap & 0xFFFF;
    uint64_t rng = rng0;
    uint32_t acc[4] = {ctl.acc[0], ctl.acc[1], ctl.acc[2], ctl.acc[3]};
    bool stopped = false, bad = ctl.err != 0, expired = false;
    const float rpen = 1.0f / c.pen;
    const double rtemp = 1.0 / (double)c.temp;
    // the last kHist steps: lane (step % kHist) holds the step, its token and
    // whether the token joined the drawn ids
    int htok = -1, hstep = -1;
    bool hfresh = false;
    // the values of decided token tk in steps gs + 1 .. gs + 64, into ring row gs
    auto issue_ring = [&](int gs, int tk) __attribute__((always_inline)) {
      const int tc = (tk >= 0 && tk < V) ? tk : 0;
      const int sidx = min(gs + 1 + lane, a.n_steps - 1);
      __builtin_amdgcn_global_load_lds((glb_ptr_t)(rowp(sidx) + tc),
                                       (lds_ptr_t)(ring + (gs & (kRing - 1)) * kWave), 4, 0, 0);
    };
    while (q < s_end && !bad) {
      C4S_SPEC_T(0);
      const int k = (q - s_first) % kSpecND;
      SpecRec& rc = recs[k];
      // The tag, then the fields of the check, in one batch of LDS reads kept
      // in order (volatile): the decider stores the fields before the tag, so
      // when the tag read gives q the reads behind it see the decision.
      RecView rv = rec_view(rc);
      if (rv.tag != q) {
        int spins = 0;
        while (vload(&rc.tag) != q && ++spins <= spin_max) __builtin_amdgcn_s_sleep(1);
        if (spins > spin_max) {
          bad = true;
          expired = true;
          break;
        }
        rv = rec_view(rc);
      }
      int spins = 0;
      C4S_SPEC_T(1);
      C4S_SPEC_EV(q, 2);
      const int nFd = rv.nF, rtok = rv.tok, Fd = rv.F, rok = rv.ok, rfresh = rv.fresh, kind = rv.kind;
      const float zlim = rv.zlim;
      const MassCoef mk{rv.ma, rv.mb, rv.mrel};
      // The ids drawn since the decision (steps [Fd, q)) are in the history
      // lanes; their values at step q are in the ring rows of their steps.
      const bool isnew = lane < kHist && hfresh && hstep >= Fd && hstep < q;
      const uint64_t nm = __ballot(isnew);
      const int nn = __popcll(nm);
      const int rslot = hstep & (kRing - 1);
      const int ridx = rslot * kWave + ((q - hstep - 1) & (kWave - 1));
      // the ring row's tag, then its value, read together (valid when the tag is hstep)
      int rtag = vload(&ctl.ringtag[rslot]);
      float x = vload(&ring[ridx]);
      spins = 0;
      while (__ballot(isnew && rtag != hstep) && ++spins <= spin_max) {
        __builtin_amdgcn_s_sleep(1);
        rtag = vload(&ctl.ringtag[rslot]);
        x = vload(&ring[ridx]);
      }
      if (spins > spin_max) {
        bad = true;
        expired = true;
        break;
      }
      C4S_SPEC_T(2);
      const float z = c.temp_on ? div_rcp(x, rtemp) : x;
      float e0, e1;
      const float m1 = mass_approx(x, mk, e0);
      const float m2 = mass_approx(pen_approx(x, c.pen, rpen), mk, e1);
      const double d = isnew ? (double)m1 - (double)m2 : 0.0;
      const double e = isnew ? (double)e0 + (double)e1 : 0.0;
      // the history and the drawn list agree unless the decision is older than the history
      bool accept = rok != 0 && nn == n - nFd && q - Fd <= kHist;
      // sums over the new ids (d and e are 0 in the other lanes), by wave
      // reductions: any order of at most kHist non-negative terms stays within
      // the |DL| 2^-50 that Y allows for rounding
      const double DL = wave_sum_dpp(d), EL = wave_sum_dpp(e), Da = wave_sum_dpp(htok < rtok ? d : 0.0);
      if (accept && nn > 0) {
        const double Y = EL + fabs(DL) * 0x1p-50;
        if (kind == 1) {
          accept = !__ballot(isnew && !(z < zlim)) && rv.w * (DL + Y) < rv.g1 && rv.w * (DL - Y) > rv.g2;
        } else if (kind == 2) {
          accept = !__ballot(isnew && (!(z < zlim) || htok == rtok)) &&
                   rv.w * (rv.u * DL - rv.ome * Da - 2.0 * Y) > rv.g1 &&
                   rv.w * (Da - rv.ome * rv.u * DL - 2.0 * Y) > rv.g2;
        } else {
          accept = false;
        }
      }
      int tokq = rtok;
      uint32_t dex = rv.dex, kept = rv.kept;
      bool exact = false;
      C4S_SPEC_T(3);
      if (!accept) {
        // decide again with every drawn id: the ids drawn since the decision
        // (drawn list [nFd, n)) join the decider's list with their values
        const SumHdr h = hdr_from(dsum(k));
        const int nl = n - nFd;
        const bool hl = lane < nl;
        const int idx = min(nFd + lane, kSpecGv - 1);
        const int tl = tokl[idx];
        const int ts = tstep[idx];
        const float xl = ring[(ts & (kRing - 1)) * kWave + ((q - ts - 1) & (kWave - 1))];
        float f0, f1;
        const float l1 = mass_approx(xl, mk, f0);
        const float l2 = mass_approx(pen_approx(xl, c.pen, rpen), mk, f1);
        const double dl = hl ? (double)l1 - (double)l2 : 0.0;
        const double el = hl ? (double)f0 + (double)f1 : 0.0;
        float* gvk = dgv(k);
        double* cd = dcd(k);
        if (hl && nl <= kWave) gvk[idx] = xl;
        if (dense && hl && nl <= kWave) atomicAdd(&cd[chunk_of(tl, h.head, h.nchunk)], dl);
        wave_sync();
        double ds = rc.ds + wave_sum_dpp(dl), de = rc.de + wave_sum_dpp(el);
        StepOut o{0, 0u, 0u, 0u};
        uint64_t r = rng;
        const int nn = nl;
        bool ok = nn <= kWave &&
                  spec_decide(h, c, V, SpecAcc{didx, gvk, bmH0, rowp(q), n}, ds, de, dsum(k), cd, r, dcs(k), o,
                              (SpecInfo*)nullptr, dense);
        if (!ok && nn <= kWave && c.pen_on && (o.why == kWhyDraw || o.why == kWhyMargin)) {
          if (dense)
            for (int i = lane; i < kMaxChunks; i += kWave) cd[i] = 0.0;
          wave_sync();
          double el;
          ds = spec_corrections(gvk, tokl, n, h, c, dense ? cd : nullptr, true, el);
          wave_sync();
          r = rng;
          ok = spec_decide(h, c, V, SpecAcc{didx, gvk, bmH0, rowp(q), n}, ds, 0.0, dsum(k), cd, r, dcs(k), o,
                           (SpecInfo*)nullptr, dense);
        }
        if (ok) {
          tokq = o.tok;
          dex = o.dex;
          kept = o.kept;
        } else {
          if (lane == 0) acc[0] |= 1u << (20 + o.why);
          exact = true;
        }
      }
      C4S_SPEC_T(4);
      if (exact) {
        // every wave stops (the deciders' areas hold the row), then resumes at q + 1
        if (lane == 0) {
          ctl.rng = rng;
          lgkm_wait();
          vstore(&ctl.halt, q);
        }
        exact_all(q);
        tokq = ctl.tok;
        if (lane == 0) {
          const uint32_t* stp = xs.step_stats;
          acc[0] |= stp[0];
          acc[1] += 1u;
          acc[2] += stp[2];
          acc[3] += stp[3];
          for (int i = 0; i < kSpecND; ++i) recs[i].tag = -1;
        }
        // ring rows of dropped decisions (steps after q) are stale
        if (lane < kRing && ctl.ringtag[lane] > q) ctl.ringtag[lane] = -1;
      }
      if (!accept) {   // ring row q: the values of the token decided here
        spins = 0;
        while (!exact && rc.ring && vload(&ctl.ringtag[q & (kRing - 1)]) != q && ++spins <= spin_max)
          __builtin_amdgcn_s_sleep(1);   // the decider's gather lands first
        // A late gather could still overwrite this ring row: the row stops
        // after this step (its decision stands), at the loop's test.
        if (spins > spin_max) bad = expired = true;
        // the same token as the decider's: its gather (landed, tagged q) is this row
        if (exact || !rc.ring || tokq != rtok || spins > spin_max) {
          issue_ring(q, tokq);
          wait_vm(0);
          if (lane == 0) vstore(&ctl.ringtag[q & (kRing - 1)], q);
        }
      }
      C4S_SPEC_T(5);
      if (lane == 0) {
        tout[q - s_first] = (int16_t)tokq;
        if (!exact) {
          acc[0] |= 64u | 1u;
          acc[2] += dex;
          acc[3] += kept;
        }
      }
      rng = exact ? ctl.rng : xorshift64(rng);
      if (tokq == a.stop_token) {
        stopped = true;
        ++q;
        if (exact) {
          lgkm_wait();
          if (lane == 0) vstore(&ctl.halt, -1);
          __syncthreads();
        }
        break;
      }
      // text2semantic.cpp:333-334: the token joins the drawn ids unless it is
      // the stop token or already penalised (an accepted decision knows all
      // but the ids drawn since it)
      const bool fresh = accept ? (rfresh != 0 && !__ballot(isnew && htok == tokq))
                                : (c.pen_on && tokq >= 0 && tokq < V && !bit_of(bmH0, tokq) &&
                                   didx[tokq] == 0xFFFFu);
      if (lane == (q & (kHist - 1))) {
        htok = tokq;
        hstep = q;
        hfresh = fresh && n < kSpecGv;
      }
      if (fresh && n >= kSpecGv) bad = true;
      if (fresh && n < kSpecGv) {
        if (lane == 0) {
          tokl[n] = tokq;
          tstep[n] = (uint16_t)q;
          didx[tokq] = (uint16_t)n;
          lds_or(&bmN[tokq >> 5], 1u << (tokq & 31));
        }
        ++n;
      }
      ++q;
      lgkm_wait();
      if (lane == 0) vstore(&ctl.snap, (q << 16) | n);
      C4S_SPEC_T(6);
      C4S_SPEC_EV(q - 1, 3);
      if (exact) {
        lgkm_wait();
        if (lane == 0) vstore(&ctl.halt, -1);
        __syncthreads();   // the deciders resume from the new frontier
      }
    }
    wait_vm(0);
    if (lane == 0) {
      ctl.qend = q;
      ctl.stopped = (stopped || bad) ? 1 : 0;   // a row that gave up stops as at a stop token
      ctl.rng = rng;
      if (bad) acc[0] |= 1u << 30;
      // a row that gave up stops here: the call reports it (the status word)
      if (bad && a.status) *a.status = expired ? kStatusWaitExpired : kStatusDrawnOverflow;
      for (int i = 0; i < 4; ++i) ctl.acc[i] = acc[i];
      lgkm_wait();
      vstore(&ctl.done, 1);
    }
  } else {
    // ---- deciders ----
    const int k = wv < kSpecVW ? wv : wv - 1;
    auto start_at = [&](int from, int& q, uint64_t& rq) __attribute__((always_inline)) {
      q = from + (((k - (from - s_first)) % kSpecND) + kSpecND) % kSpecND;
      rq = rng0;
      for (int i = s_first; i < q; ++i) rq = xorshift64(rq);
    };
    int q;
    uint64_t rq;
    start_at(s_first, q, rq);
    SpecCS& cs = dcs(k);
    uint64_t* sw = dsum(k);
    float* gv = dgv(k);
    double* cd = dcd(k);
    if (lane == 0) cs.gen = 0u;
    int pend = -1;   // step whose token's ring gather this wave has in flight
    for (;;) {
      int snap = 0;
      bool halted = false, quit = false;
      if (pend >= 0) {   // the gather has landed: its ring row is usable
        wait_loads();
        if (lane == 0) vstore(&ctl.ringtag[pend & (kRing - 1)], pend);
        pend = -1;
      }
      C4S_SPEC_T(0);
      for (;;) {
        if (vload(&ctl.halt) >= 0) { halted = true; break; }
        if (vload(&ctl.done)) { quit = true; break; }
        snap = vload(&ctl.snap);
        if (q < s_end && (snap >> 16) > q - kSpecND) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (quit) break;
      if (halted) {
        exact_all(vload(&ctl.halt));
        __syncthreads();   // the checking wave has moved the frontier past the exact step
        start_at(vload(&ctl.snap) >> 16, q, rq);
        if (lane == 0) cs.gen = 0u;
        continue;
      }
      C4S_SPEC_T(1);
      C4S_SPEC_EV(q, 0);
      const int nF = snap & 0xFFFF;
      const float* grow = rowp(q);
      // the step's summary into this wave's slot, the drawn ids' raw values into gv
      const uint64_t* sg = sum_words(w, a.n_rows, q, row);
      for (int q0 = 0; q0 < kSumQuads; q0 += kWave)
        if (q0 + lane < kSumQuads)
          __builtin_amdgcn_global_load_lds((glb_ptr_t)(sg + 2 * (q0 + lane)), (lds_ptr_t)(sw + 2 * q0), 16, 0, 0);
      for (int j0 = 0; j0 < nF; j0 += 4 * kWave) {
        int id[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) id[i] = tokl[min(j0 + i * kWave + lane, kSpecGv - 1)];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (j0 + i * kWave + lane < nF)
            __builtin_amdgcn_global_load_lds((glb_ptr_t)(grow + id[i]), (lds_ptr_t)(gv + j0 + i * kWave), 4, 0,
                                             0);
      }
      if (dense)
        for (int i = lane; i < kMaxChunks; i += kWave) cd[i] = 0.0;
      C4S_SPEC_T(2);
      wait_loads();
      wave_sync();
      C4S_SPEC_T(3);
      const SumHdr h = hdr_from(sw);
      double de = 0.0, ds = 0.0;
      if (c.pen_on) ds = spec_corrections(gv, tokl, nF, h, c, dense ? cd : nullptr, false, de);
      wave_sync();
      C4S_SPEC_T(4);
      SpecRec& rc = recs[k];
      SpecInfo* si = &rc.si;   // the decision writes what it rests on straight into its record
      if (lane == 0) si->kind = 0;
      StepOut o{0, 0u, 0u, 0u};
      uint64_t r = rq;
      bool ok = spec_decide(h, c, V, SpecAcc{didx, gv, bmH0, grow, nF}, ds, de, sw, cd, r, cs, o, si, dense);
      if (!ok && c.pen_on && (o.why == kWhyDraw || o.why == kWhyMargin)) {
        if (dense)
          for (int i = lane; i < kMaxChunks; i += kWave) cd[i] = 0.0;
        wave_sync();
        ds = spec_corrections(gv, tokl, nF, h, c, dense ? cd : nullptr, true, de);
        de = 0.0;
        wave_sync();
        if (lane == 0) si->kind = 0;
        r = rq;
        ok = spec_decide(h, c, V, SpecAcc{didx, gv, bmH0, grow, nF}, ds, de, sw, cd, r, cs, o, si, dense);
      }
      C4S_SPEC_T(5);
      if (ok) {   // the token's values in the next 64 steps, for the checks of later steps
        const int tc = (o.tok >= 0 && o.tok < V) ? o.tok : 0;
        const int sidx = min(q + 1 + lane, a.n_steps - 1);
        __builtin_amdgcn_global_load_lds((glb_ptr_t)(rowp(sidx) + tc),
                                         (lds_ptr_t)(ring + (q & (kRing - 1)) * kWave), 4, 0, 0);
        pend = q;
      }
      if (lane == 0) {
        const int tk = o.tok;
        rc.tok = tk;
        rc.nF = nF;
        rc.F = snap >> 16;
        rc.fresh = (ok && c.pen_on && tk >= 0 && tk < V && tk != a.stop_token && !bit_of(bmH0, tk) &&
                    (int)didx[tk] >= nF) ? 1 : 0;
        rc.ok = ok ? 1 : 0;
        rc.ring = ok ? 1 : 0;
        const MassCoef mk = mass_coef(c, h.m0);
        rc.ma = mk.a;
        rc.mb = mk.b;
        rc.mrel = mk.relc;
        const int kd = ok ? si->kind : 0;
        rc.kind = kd;
        if (kd == 1) {
          const double c1 = si->eps + si->dmass;
          rc.w = si->p * si->rho;
          rc.g1 = si->chk1 ? si->p * si->S - si->A1 - si->p * si->err - si->eps * si->S - c1 * si->A1
                           : __builtin_inf();
          rc.g2 = si->p * si->S - si->A2 + si->p * si->err + si->eps * si->S + c1 * si->A2;
          rc.zlim = si->zcut;
        } else if (kd == 2) {
          rc.w = si->rho;
          rc.u = si->u;
          rc.ome = 1.0 - si->eps;
          rc.g1 = si->u * si->S - si->af + 2.0 * si->err + si->eps * si->af;
          rc.g2 = si->pf - si->u * si->S + 2.0 * si->err + si->eps * si->u * si->S;
          rc.zlim = si->mt;
        }
        rc.why = o.why;
        rc.dex = o.dex;
        rc.kept = o.kept;
        rc.ds = ds;
        rc.de = de;
        lgkm_wait();
        vstore(&rc.tag, q);
      }
      C4S_SPEC_EV(q, 1);
      q += kSpecND;
      for (int i = 0; i < kSpecND; ++i) rq = xorshift64(rq);
      C4S_SPEC_T(6);
    }
  }
  C4S_SPEC_END(wv);
  __syncthreads();
  // Epilogue: tokens of the chunk (-1 after a stop), the row state.
  const int qend = ctl.qend;
  for (int s2 = s_first + t; s2 < s_end; s2 += NTS)
    a.out_tok[(int64_t)s2 * a.n_rows + row] = s2 < qend ? (int)tout[s2 - s_first] : -1;
  uint32_t acc[4] = {ctl.acc[0], ctl.acc[1], ctl.acc[2], ctl.acc[3]};
  fast_end(a, w, row, V, NTS, s_end, ctl.stopped != 0, ctl.rng, acc, bmN);
}


// ---- speculative candidate-list chain -----------------------------------------------
//
// Greedy and top-k rows (k <= 64), one workgroup per row: wave kLND checks,
// the others decide, as in the full-vocabulary chain. A greedy or top-k
// decision depends on ids drawn before it only through its candidates: an id
// drawn since that is neither the greedy token nor one of the top-k survivors
// leaves the decision as it is (the penalty only lowers values, and top_p and
// the draw read the survivors alone). So the checking wave accepts a decision
// unless an id drawn since is one of its survivors; otherwise it decides the
// step again from the decider's stored candidate list with every drawn id,
// and a step the list cannot settle stops every wave for the exact chain on
// the row read into LDS.

constexpr int kLND = 4;                   // deciding waves
constexpr int NTL = (kLND + 1) * kWave;
constexpr int kLVW = kLND;                // the checking wave (the last)


struct LSpecRec {
  int tag;     // step of this decision (written last), -1 none
  int tok;
  int nF;      // drawn ids the decision knew (a prefix of the drawn list)
  int F;       // ... those drawn before step F
  int fresh;   // tok is none of them, nor in H0, nor the stop token
  int ok;
  int nsurv;   // survivors in the decider's lid (greedy: the token)
  uint32_t why, dex, kept;
};

struct LSpecCtl {
  int snap;   // (frontier << 16) | drawn ids before the frontier
  int halt;   // step of an exact chain run by every wave, else -1
  int done;
  int err;
  int qend;
  int stopped;
  int tok;
  uint64_t rng;
  uint32_t acc[4];
};

struct LSpecLayout {
  size_t didx, tok, tout, xrow, dec, stride, o_e1, o_hw, o_y0, o_y1, o_cs, total;
};
__host__ __device__ inline LSpecLayout lspec_layout(int V) {
  LSpecLayout L;
  L.didx = 0;
  L.tok = al16(2 * (size_t)V);
  L.tout = al16(L.tok + 4 * (size_t)kSpecGv);
  L.xrow = al16(L.tout + 2 * (size_t)kSpecGv);
  L.dec = al16(L.xrow + 4 * ((size_t)vpad(V) + 4));
  L.o_e1 = 8 * (size_t)kWave;          // candidate list of a decision: e0, e1, hw, y0, y1 by lane
  L.o_hw = L.o_e1 + 8 * (size_t)kWave;
  L.o_y0 = L.o_hw + 8 * (size_t)kWave;
  L.o_y1 = L.o_y0 + 4 * (size_t)kWave;
  L.o_cs = al16(L.o_y1 + 4 * (size_t)kWave);
  L.stride = al16(L.o_cs + sizeof(LSpecCS));
  L.total = L.dec + (size_t)kLND * L.stride;
  return L;
}

// Drawn set of one decision: ids whose drawn index is below nF.
struct IdxHit {
  const uint16_t* didx;
  int nF;
  __device__ __forceinline__ bool hit(int id) const { return (int)didx[id] < nF; }
};

// At most 128 VGPRs (four waves a SIMD): two workgroups of five waves share a CU.
template <bool kForcedLimit>
__global__ __launch_bounds__(NTL) __attribute__((amdgpu_waves_per_eu(4))) void k_stream_lspec(StreamArgs a,
                                                                                          StreamWs w) {
  const int spin_max = kForcedLimit ? a.spin_max : kSpinMaxDefault;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ LSpecRec recs[kLND];
  __shared__ LSpecCtl ctl;
  __shared__ ScratchT<kLND + 1> xs;   // exact steps
  __shared__ uint32_t bmH0[kStateWords], bmN[kStateWords];
  const int row = blockIdx.x;
  const int V = a.vocab;
  const int t = threadIdx.x, lane = lane_id(), wv = wave_id();
  const RowCfg c = make_cfg(0u, V, row, a.temp, a.top_k, a.top_p, a.pen, nullptr, a.do_sample);
  if (stream_mode(c, V) != kModeList) return;
  int s_first;
  if (!fast_begin(a, w, row, NTL, s_first)) return;
  const int s_end = w.s_end;
  const uint64_t rng0 = a.rng[row];
  const uint32_t* stw = w.state + (size_t)row * kStateWords;
  const LSpecLayout L = lspec_layout(V);
  uint16_t* didx = reinterpret_cast<uint16_t*>(smem + L.didx);
  int* tokl = reinterpret_cast<int*>(smem + L.tok);
  int16_t* tout = reinterpret_cast<int16_t*>(smem + L.tout);
  float* xrow = reinterpret_cast<float*>(smem + L.xrow);
  auto dbase = [&](int k) { return smem + L.dec + (size_t)k * L.stride; };
  auto dcs = [&](int k) -> LSpecCS& { return *reinterpret_cast<LSpecCS*>(dbase(k) + L.o_cs); };
  const float* base = a.logits + (int64_t)row * a.ld;
  auto rowp = [&](int s) { return base + (int64_t)s * a.step_stride; };
  const int nwords = bitmap_words(V);

  // Prologue: H0 and the ids drawn in earlier chunks, listed in id order.
  fast_bitmaps(a, stw, row, V, NTL, bmH0, bmN, true);
  for (int i = t; i < V; i += NTL) didx[i] = 0xFFFFu;
  if (t < kLND) recs[t].tag = -1;
  __syncthreads();
  if (wv == kLVW) {
    int n = 0;
    for (int w0 = 0; w0 < nwords; w0 += kWave) {
      const int wb = w0 + lane;
      uint32_t bits = wb < nwords ? bmN[wb] : 0u;
      const uint32_t cnt = (uint32_t)__popc(bits);
      const uint32_t incl = wave_scan_u32(cnt);
      int p = n + (int)(incl - cnt);
      while (bits) {
        const int id = 32 * wb + __ffs(bits) - 1;
        bits &= bits - 1;
        if (p < kSpecGv && id < V) {
          tokl[p] = id;
          didx[id] = (uint16_t)p;
        }
        ++p;
      }
      n += (int)readlane_u32(incl, kWave - 1);
    }
    if (lane == 0) {
      ctl.snap = (s_first << 16) | min(n, kSpecGv);
      ctl.halt = -1;
      ctl.done = 0;
      ctl.err = n > kSpecGv ? 1 : 0;
      ctl.qend = s_first;
      ctl.stopped = 0;
      ctl.rng = rng0;
      for (int i = 0; i < 4; ++i) ctl.acc[i] = stw[1 + i];
    }
  }
  __syncthreads();

  // Every wave runs the exact chain of step hq on the raw row read into LDS
  // (text2semantic.cpp:142-166); ends at a barrier.
  auto exact_all = [&](int hq) __attribute__((always_inline)) {
    __syncthreads();
    const float* src = rowp(hq);
    for (int i = t; i < V; i += NTL) xrow[i] = src[i];
    __syncthreads();
    if (c.pen_on) {   // H0 and the stream's ids are disjoint: each id once
      penalise_chunk<NTL>(xrow, bmH0, V, c.pen);
      penalise_chunk<NTL>(xrow, bmN, V, c.pen);
    }
    __syncthreads();
    uint64_t r = ctl.rng;
    LdsRowNC srow{xrow, V, 0u, false, w.sortbuf + (int64_t)row * w.sort_stride, (uint32_t)(w.sort_stride * 4)};
    const int tok = run_chain(srow, xs, c, r, nullptr, xs.step_stats);
    __syncthreads();
    if (t == 0) {
      ctl.tok = tok;
      ctl.rng = r;
    }
    __syncthreads();
  };

  if (wv == kLVW) {
    // ---- the checking wave: takes the decisions in step order ----
    int q = s_first;
    int n = ctl.snap & 0xFFFF;
    uint64_t rng = rng0;
    uint32_t acc[4] = {ctl.acc[0], ctl.acc[1], ctl.acc[2], ctl.acc[3]};
    bool stopped = false, bad = ctl.err != 0, expired = false;
    int htok = -1, hstep = -1;   // lane (step % kHist): a recent step, its token, whether it was drawn anew
    bool hfresh = false;
    while (q < s_end && !bad) {
      const int k = (q - s_first) % kLND;
      LSpecRec& rc = recs[k];
      int spins = 0;
      while (vload(&rc.tag) != q && ++spins <= spin_max) __builtin_amdgcn_s_sleep(1);
      if (spins > spin_max) {
        bad = true;
        expired = true;
        break;
      }
      C4S_SPEC_EV(q, 2);
      const int nFd = rc.nF, rtok = rc.tok, Fd = rc.F, rok = rc.ok, rfresh = rc.fresh, ns = rc.nsurv;
      LSpecCS& cs = dcs(k);
      // the ids drawn since the decision (steps [Fd, q)) against its survivors
      const bool isnew = lane < kHist && hfresh && hstep >= Fd && hstep < q;
      const uint64_t nm = __ballot(isnew);
      const int nn = __popcll(nm);
      bool accept = rok != 0 && nn == n - nFd && q - Fd <= kHist;
      if (accept && nn > 0) {
        const int sid = lane < ns ? cs.lid[lane] : -1;
        for (uint64_t b = nm; b && accept; b &= b - 1) {
          const int tj = (int)readlane_u32((uint32_t)htok, __ffsll((unsigned long long)b) - 1);
          accept = !__ballot(sid == tj);
        }
      }
      int tokq = rtok;
      uint32_t dex = rc.dex, kept = rc.kept;
      bool exact = false;
      uint64_t rnext = c.greedy ? rng : xorshift64(rng);
      if (!accept) {
        // decide again from the decider's candidate list with every drawn id
        unsigned char* db = dbase(k);
        const uint64_t e0r = reinterpret_cast<const uint64_t*>(db)[lane];
        const uint64_t e1r = reinterpret_cast<const uint64_t*>(db + L.o_e1)[lane];
        const uint64_t hwr = reinterpret_cast<const uint64_t*>(db + L.o_hw)[lane];
        const float y0 = reinterpret_cast<const float*>(db + L.o_y0)[lane];
        const float y1 = reinterpret_cast<const float*>(db + L.o_y1)[lane];
        const SumHdr h = hdr_lanes(hwr);
        const uint64_t e0 = (lane < h.n) ? e0r : 0ull;
        const uint64_t e1 = (lane + kWave < h.n) ? e1r : 0ull;
        StepOut o{0, 0u, 0u, 0u};
        uint64_t r = rng;
        const bool ok = list_step(h, e0, e1, y0, y1, c, V, IdxHit{didx, n}, r, cs, o);
        if (ok) {
          tokq = o.tok;
          dex = o.dex;
          kept = o.kept;
          rnext = r;
        } else {
          if (lane == 0) acc[0] |= 1u << (20 + o.why);
          exact = true;
        }
      }
      if (exact) {   // every wave stops, then resumes at q + 1
        if (lane == 0) {
          ctl.rng = rng;
          lgkm_wait();
          vstore(&ctl.halt, q);
        }
        exact_all(q);
        tokq = ctl.tok;
        rnext = ctl.rng;
        if (lane == 0) {
          const uint32_t* stp = xs.step_stats;
          acc[0] |= stp[0];
          acc[1] += 1u;
          acc[2] += stp[2];
          acc[3] += stp[3];
          for (int i = 0; i < kLND; ++i) recs[i].tag = -1;
        }
      }
      if (lane == 0) {
        tout[q - s_first] = (int16_t)tokq;
        if (!exact) {
          acc[0] |= 32u | 1u;
          acc[2] += dex;
          acc[3] += kept;
        }
      }
      rng = rnext;
      if (tokq == a.stop_token) {
        stopped = true;
        ++q;
        if (exact) {
          lgkm_wait();
          if (lane == 0) vstore(&ctl.halt, -1);
          __syncthreads();
        }
        break;
      }
      // text2semantic.cpp:333-334: the token joins the drawn ids unless it is
      // the stop token or already penalised
      const bool fresh = accept ? (rfresh != 0 && !__ballot(isnew && htok == tokq))
                                : (c.pen_on && tokq >= 0 && tokq < V && !bit_of(bmH0, tokq) &&
                                   didx[tokq] == 0xFFFFu);
      if (lane == (q & (kHist - 1))) {
        htok = tokq;
        hstep = q;
        hfresh = fresh && n < kSpecGv;
      }
      if (fresh && n >= kSpecGv) bad = true;
      if (fresh && n < kSpecGv) {
        if (lane == 0) {
          tokl[n] = tokq;
          didx[tokq] = (uint16_t)n;
          bmN[tokq >> 5] |= 1u << (tokq & 31);
        }
        ++n;
      }
      ++q;
      lgkm_wait();
      if (lane == 0) vstore(&ctl.snap, (q << 16) | n);
      C4S_SPEC_EV(q - 1, 3);
      if (exact) {
        lgkm_wait();
        if (lane == 0) vstore(&ctl.halt, -1);
        __syncthreads();   // the deciders resume from the new frontier
      }
    }
    if (lane == 0) {
      ctl.qend = q;
      ctl.stopped = (stopped || bad) ? 1 : 0;   // a row that gave up stops as at a stop token
      ctl.rng = rng;
      if (bad) acc[0] |= 1u << 30;
      // a row that gave up stops here: the call reports it (the status word)
      if (bad && a.status) *a.status = expired ? kStatusWaitExpired : kStatusDrawnOverflow;
      for (int i = 0; i < 4; ++i) ctl.acc[i] = acc[i];
      lgkm_wait();
      vstore(&ctl.done, 1);
    }
  } else {
    // ---- deciders ----
    const int k = wv;
    auto start_at = [&](int from, int& q, uint64_t& rq) __attribute__((always_inline)) {
      q = from + (((k - (from - s_first)) % kLND) + kLND) % kLND;
      rq = rng0;
      if (!c.greedy)
        for (int i = s_first; i < q; ++i) rq = xorshift64(rq);
    };
    auto load = [&](int s, ListRegs& r) __attribute__((always_inline)) {
      const uint64_t* sw = sum_words(w, a.n_rows, min(s, s_end - 1), row);
      r.e0 = sw[lane];
      r.e1 = sw[lane + kWave];
      r.hw = sw[kHdrW + (lane & 7)];
      const float* sy = reinterpret_cast<const float*>(sw + kYW);
      r.y0 = sy[lane];
      r.y1 = sy[lane + kWave];
    };
    int q;
    uint64_t rq;
    start_at(s_first, q, rq);
    LSpecCS& cs = dcs(k);
    unsigned char* db = dbase(k);
    LSpecRec& rc = recs[k];
    ListRegs P{};
    load(q, P);
    for (;;) {
      int snap = 0;
      bool halted = false, quit = false;
      for (;;) {
        if (vload(&ctl.halt) >= 0) { halted = true; break; }
        if (vload(&ctl.done)) { quit = true; break; }
        snap = vload(&ctl.snap);
        if (q < s_end && (snap >> 16) > q - kLND) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (quit) break;
      if (halted) {
        exact_all(vload(&ctl.halt));
        __syncthreads();   // the checking wave has moved the frontier past the exact step
        start_at(vload(&ctl.snap) >> 16, q, rq);
        load(q, P);
        continue;
      }
      C4S_SPEC_EV(q, 0);
      const int nF = snap & 0xFFFF;
      const ListRegs R = P;
      if (q + kLND < s_end) load(q + kLND, P);   // the next decision's list, in flight meanwhile
      const SumHdr h = hdr_lanes(R.hw);
      const uint64_t e0 = (lane < h.n) ? R.e0 : 0ull;
      const uint64_t e1 = (lane + kWave < h.n) ? R.e1 : 0ull;
      StepOut o{0, 0u, 0u, 0u};
      uint64_t r = rq;
      const bool ok = list_step(h, e0, e1, R.y0, R.y1, c, V, IdxHit{didx, nF}, r, cs, o);
      // the list, for the checking wave's second decision
      reinterpret_cast<uint64_t*>(db)[lane] = R.e0;
      reinterpret_cast<uint64_t*>(db + L.o_e1)[lane] = R.e1;
      reinterpret_cast<uint64_t*>(db + L.o_hw)[lane] = R.hw;
      reinterpret_cast<float*>(db + L.o_y0)[lane] = R.y0;
      reinterpret_cast<float*>(db + L.o_y1)[lane] = R.y1;
      if (lane == 0) {
        const int tk = o.tok;
        if (c.greedy) cs.lid[0] = tk;
        rc.tok = tk;
        rc.nF = nF;
        rc.F = snap >> 16;
        rc.fresh = (ok && c.pen_on && tk >= 0 && tk < V && tk != a.stop_token && !bit_of(bmH0, tk) &&
                    (int)didx[tk] >= nF) ? 1 : 0;
        rc.ok = ok ? 1 : 0;
        rc.nsurv = c.greedy ? 1 : (int)o.nsurv;
        rc.why = o.why;
        rc.dex = o.dex;
        rc.kept = o.kept;
        lgkm_wait();
        vstore(&rc.tag, q);
      }
      C4S_SPEC_EV(q, 1);
      q += kLND;
      if (!c.greedy)
        for (int i = 0; i < kLND; ++i) rq = xorshift64(rq);
    }
  }
  __syncthreads();
  // Epilogue: tokens of the chunk (-1 after a stop), the row state.
  const int qend = ctl.qend;
  for (int s2 = s_first + t; s2 < s_end; s2 += NTL)
    a.out_tok[(int64_t)s2 * a.n_rows + row] = s2 < qend ? (int)tout[s2 - s_first] : -1;
  uint32_t acc[4] = {ctl.acc[0], ctl.acc[1], ctl.acc[2], ctl.acc[3]};
  fast_end(a, w, row, V, NTL, s_end, ctl.stopped != 0, ctl.rng, acc, bmN);
}

}  // namespace

size_t stream_chain_lds_bytes(int V) {
  return rows_lds_bytes(V) + 8 * (size_t)bitmap_words(V);
}

hipError_t launch_stream_scan(const StreamArgs& a, const StreamWs& w, hipStream_t s) {
  if (a.n_rows <= 0 || w.s_end <= w.s_begin) return hipSuccess;
  (void)hipGetLastError();
  const int steps = w.s_end - w.s_begin;
  const dim3 grid((unsigned)((steps + w.steps_per_group - 1) / w.steps_per_group), (unsigned)a.n_rows);
  const int nq_max = a.vocab >> 2;
  const bool one = w.steps_per_group == 1;
  if (nq_max <= 2 * NTA) {
    if (one) hipLaunchKernelGGL((k_stream_scan<2, true>), grid, dim3(NTA), 0, s, a, w);
    else hipLaunchKernelGGL((k_stream_scan<2, false>), grid, dim3(NTA), 0, s, a, w);
  } else if (nq_max <= 8 * NTA) {
    if (one) hipLaunchKernelGGL((k_stream_scan<8, true>), grid, dim3(NTA), 0, s, a, w);
    else hipLaunchKernelGGL((k_stream_scan<8, false>), grid, dim3(NTA), 0, s, a, w);
  } else {
    if (one) hipLaunchKernelGGL((k_stream_scan<12, true>), grid, dim3(NTA), 0, s, a, w);
    else hipLaunchKernelGGL((k_stream_scan<12, false>), grid, dim3(NTA), 0, s, a, w);
  }
  return hipGetLastError();
}

size_t stream_list_lds_bytes(int V) { return 4 * ((size_t)vpad(V) + 4); }

hipError_t launch_stream_list(const StreamArgs& a, const StreamWs& w, hipStream_t s) {
  if (a.n_rows <= 0 || w.s_end <= w.s_begin) return hipSuccess;
  (void)hipGetLastError();
  hipLaunchKernelGGL(k_stream_list, dim3(a.n_rows), dim3(kWave), w.sortbuf ? stream_list_lds_bytes(a.vocab) : 0, s,
                     a, w);
  return hipGetLastError();
}

size_t stream_rowp_lds_bytes(int V) {
  return 3 * (size_t)kSumWordsP * 8 + 3 * 4 * ((size_t)vpad(V) + 4);
}

hipError_t launch_stream_rowp(const StreamArgs& a, const StreamWs& w, hipStream_t s) {
  if (a.n_rows <= 0 || w.s_end <= w.s_begin) return hipSuccess;
  (void)hipGetLastError();
  hipLaunchKernelGGL(k_stream_rowp, dim3(a.n_rows, max(1, w.nseg)), dim3(NTC), stream_rowp_lds_bytes(a.vocab), s, a,
                     w);
  return hipGetLastError();
}

size_t stream_spec_lds_bytes(int V) {
  if (V > kLdsVocabMax) return 0;
  return spec_layout(V).total;
}

int stream_spec_max_steps() { return kSpecGv; }

size_t stream_lspec_lds_bytes(int V) {
  if (V > kLdsVocabMax) return 0;
  return lspec_layout(V).total;
}

hipError_t launch_stream_lspec(const StreamArgs& a, const StreamWs& w, hipStream_t s) {
  if (a.n_rows <= 0 || w.s_end <= w.s_begin) return hipSuccess;
  (void)hipGetLastError();
  if (a.spin_max == kSpinMaxDefault)
    hipLaunchKernelGGL(k_stream_lspec<false>, dim3(a.n_rows), dim3(NTL), stream_lspec_lds_bytes(a.vocab), s, a, w);
  else
    hipLaunchKernelGGL(k_stream_lspec<true>, dim3(a.n_rows), dim3(NTL), stream_lspec_lds_bytes(a.vocab), s, a, w);
  return hipGetLastError();
}

hipError_t launch_stream_spec(const StreamArgs& a, const StreamWs& w, hipStream_t s) {
  if (a.n_rows <= 0 || w.s_end <= w.s_begin) return hipSuccess;
  (void)hipGetLastError();
  if (a.spin_max == kSpinMaxDefault)
    hipLaunchKernelGGL(k_stream_spec<false>, dim3(a.n_rows), dim3(NTS), stream_spec_lds_bytes(a.vocab), s, a, w);
  else
    hipLaunchKernelGGL(k_stream_spec<true>, dim3(a.n_rows), dim3(NTS), stream_spec_lds_bytes(a.vocab), s, a, w);
  return hipGetLastError();
}

hipError_t launch_stream_segfix(const StreamArgs& a, const StreamWs& w, hipStream_t s) {
  if (a.n_rows <= 0 || w.s_end <= w.s_begin || w.nseg <= 1) return hipSuccess;
  (void)hipGetLastError();
  hipLaunchKernelGGL(k_stream_segfix, dim3(a.n_rows), dim3(kWave), 0, s, a, w);
  return hipGetLastError();
}

hipError_t launch_stream_chain(const StreamArgs& a, const StreamWs& w, hipStream_t s) {
  if (a.n_rows <= 0 || w.s_end <= w.s_begin) return hipSuccess;
  (void)hipGetLastError();
  hipLaunchKernelGGL(k_stream_chain, dim3(a.n_rows), dim3(NT), stream_chain_lds_bytes(a.vocab), s, a, w);
  return hipGetLastError();
}

}  // namespace c4s
