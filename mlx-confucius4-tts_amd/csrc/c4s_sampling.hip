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


#include "c4s_chain.hpp"

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

__global__ __launch_bounds__(NT) void k_rows_global(RowsArgs a) {
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
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(smem);
  const int nw = (V + 31) / 32;
  for (int w = threadIdx.x; w < nw; w += NT) bitmap[w] = 0u;
  __syncthreads();
  if (c.pen_on) {
    if (a.hist_bits) {   // the history set kept across steps
      const uint32_t* hb = a.hist_bits + (int64_t)row * hist_words(V);
      for (int w = threadIdx.x; w < nw; w += NT) bitmap[w] = hb[w];
    } else {
      const int64_t h0 = a.hist_off[row], h1 = a.hist_off[row + 1];
      for (int64_t j = h0 + threadIdx.x; j < h1; j += NT) {
        const int id = a.hist_ids[j];
        if (id < 0 || id >= V) continue;
        atomicOr(&bitmap[id >> 5], 1u << (id & 31));
      }
    }
    __syncthreads();
  }
  const int64_t roff = (int64_t)row * a.ld;
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

size_t rows_global_lds_bytes(int V) { return 4 * (size_t)((V + 31) / 32); }

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
  if (a.vocab <= kLdsVocabMax) {
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
