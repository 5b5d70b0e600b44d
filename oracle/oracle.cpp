// CPU oracle for the c4tts Text2Semantic token-sampling path.
//
// TEST INFRASTRUCTURE ONLY. This file is the checker: tests/, the smoke check
// and the CPU-baseline leg of bench.py may load it; the product path
// (libc4s_sampling.so) never links, loads or falls back to it.
//
// It restates, in its own code, the reference's host algorithm with the same
// STL building blocks (std::nth_element, std::sort, std::unordered_set,
// std::exp(double)) so that it also serves as a faithful CPU baseline:
//   temperature          src/t2s/sampling.cpp:14-17
//   repetition_penalty   src/t2s/sampling.cpp:19-28
//   top_k                src/t2s/sampling.cpp:30-40
//   top_p                src/t2s/sampling.cpp:42-71
//   argmax               src/t2s/sampling.cpp:73-76
//   categorical draw     src/t2s/text2semantic.cpp:150-165 (single) / :315-331 (batch)
//   processor chain      src/t2s/text2semantic.cpp:142-149 (single) / :303-337 (batch)
//   RNG seeding          src/t2s/text2semantic.cpp:109 (single) / :292-294 (batch)
//   LayerNorm + linear   src/nn/nn.cpp:73-83, :11-16 (LM head, text2semantic.cpp:118-121)
//
// One deliberate difference, the declared tie order of top_p: the reference
// sorts with an unstable std::sort on value only (sampling.cpp:47-48), so the
// ids that survive inside a tie group cut by the nucleus are whatever the
// host's introsort permutation leaves. This restatement breaks those ties by
// id (ascending sort on (value asc, id desc), i.e. the lower id survives).
// orc_top_p_literal keeps the reference's value-only comparator for measuring
// how often the two differ.
//
// Pinning (what checks each function) is enforced by tests/test_oracle_pins.py
// (closed forms, invariants, exact rational top_p, the xorshift64 shift
// matrices) and tests/test_oracle_golden.py (HF processor goldens).

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <numeric>
#include <thread>
#include <unordered_set>
#include <vector>

namespace {

constexpr float kNegInf = -std::numeric_limits<float>::infinity();

// ---- processors (in place on one row) --------------------------------------

// sampling.cpp:14-17 -- IEEE fp32 division, skipped for temp==1 or temp<=0.
void temperature_row(float* v, int n, float temp) {
  if (temp == 1.0f || temp <= 0.0f) return;
  for (int i = 0; i < n; ++i) v[i] = v[i] / temp;
}

// sampling.cpp:19-28 -- every distinct id in [0, n) is penalised once:
// negative logits are multiplied, the others (0 and -0 included) divided.
void penalty_row(float* v, int n, const int32_t* ids, int64_t n_ids, float pen) {
  if (pen == 1.0f) return;
  std::unordered_set<int> distinct(ids, ids + n_ids);
  for (int id : distinct) {
    if (id < 0 || id >= n) continue;
    const float s = v[id];
    v[id] = (s < 0) ? s * pen : s / pen;
  }
}

// sampling.cpp:30-40 -- threshold = k-th largest value counted with
// multiplicity; everything strictly below it becomes -inf, so ties survive.
void top_k_row(float* v, int n, int k) {
  if (k <= 0 || k >= n) return;
  std::vector<float> tmp(v, v + n);
  std::nth_element(tmp.begin(), tmp.begin() + (k - 1), tmp.end(), std::greater<float>());
  const float thresh = tmp[k - 1];
  for (int i = 0; i < n; ++i)
    if (v[i] < thresh) v[i] = kNegInf;
}

// sampling.cpp:42-71 with the declared tie order (see file header).
// `literal` selects the reference's own value-only comparator instead.
void top_p_row(float* v, int n, float p, int min_keep, bool literal) {
  if (n <= 0) return;  // the reference dereferences max_element of an empty row (UB)
  std::vector<int> order(n);
  std::iota(order.begin(), order.end(), 0);
  if (literal) {
    std::sort(order.begin(), order.end(), [&](int a, int b) { return v[a] < v[b]; });
  } else {
    std::sort(order.begin(), order.end(), [&](int a, int b) {
      if (v[a] < v[b]) return true;
      if (v[b] < v[a]) return false;
      return a > b;  // equal values: higher id earlier in ascending order -> removed first
    });
  }
  const float vmax = *std::max_element(v, v + n);
  std::vector<double> prob(n);
  double total = 0.0;
  for (int j = 0; j < n; ++j) {
    prob[j] = std::exp(static_cast<double>(v[order[j]] - vmax));
    total += prob[j];
  }
  const double cut = 1.0 - p;
  std::vector<char> drop(n, 0);
  double cum = 0.0;
  for (int j = 0; j < n; ++j) {
    cum += prob[j] / total;
    if (cum <= cut) drop[j] = 1;
  }
  for (int j = n - min_keep; j < n; ++j)
    if (j >= 0) drop[j] = 0;
  for (int j = 0; j < n; ++j)
    if (drop[j]) v[order[j]] = kNegInf;
}

// sampling.cpp:73-76 -- first maximum (std::max_element).
int argmax_row(const float* v, int n) {
  return static_cast<int>(std::max_element(v, v + n) - v);
}

// text2semantic.cpp:158 -- xorshift64 with shifts (13, 7, 17).
inline uint64_t xorshift_step(uint64_t s) {
  s ^= s << 13;
  s ^= s >> 7;
  s ^= s << 17;
  return s;
}

// text2semantic.cpp:150-165 -- inverse-CDF draw in id order, double sums,
// -inf (and +inf) entries weigh 0; advances the RNG once.
int draw_row(const float* v, int n, uint64_t* rng) {
  float vmax = -1e30f;
  for (int i = 0; i < n; ++i) vmax = std::max(vmax, v[i]);
  std::vector<double> prob(n);
  double total = 0.0;
  for (int i = 0; i < n; ++i) {
    prob[i] = std::isinf(v[i]) ? 0.0 : std::exp(static_cast<double>(v[i] - vmax));
    total += prob[i];
  }
  *rng = xorshift_step(*rng);
  const double r = static_cast<double>(*rng >> 11) / static_cast<double>(1ull << 53) * total;
  double acc = 0.0;
  int tok = n - 1;
  for (int i = 0; i < n; ++i) {
    acc += prob[i];
    if (r <= acc) { tok = i; break; }
  }
  return tok;
}

// text2semantic.cpp:142-166 -- penalty, then argmax (greedy) or
// temperature -> top_k -> top_p -> draw. `v` holds the row state before the
// final argmax/draw on return (that is what the parity checks compare).
int chain_row(float* v, int n, const int32_t* hist, int64_t n_hist, float temp, int top_k,
              float top_p, float pen, int min_keep, int do_sample, uint64_t* rng) {
  penalty_row(v, n, hist, n_hist, pen);
  if (!do_sample) return argmax_row(v, n);
  temperature_row(v, n, temp);
  top_k_row(v, n, top_k);
  top_p_row(v, n, top_p, min_keep, false);
  return draw_row(v, n, rng);
}

inline float bf16_to_f32(uint16_t b) {
  uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

inline uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

template <class F>
void parallel_rows(int n_rows, int n_threads, F&& fn) {
  if (n_threads <= 1 || n_rows <= 1) {
    for (int b = 0; b < n_rows; ++b) fn(b);
    return;
  }
  n_threads = std::min(n_threads, n_rows);
  std::vector<std::thread> pool;
  for (int t = 0; t < n_threads; ++t)
    pool.emplace_back([&, t] {
      for (int b = t; b < n_rows; b += n_threads) fn(b);
    });
  for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

// ---- single-row processors, the five legacy entry points -------------------
void orc_temperature(float* v, int n, float temp) { temperature_row(v, n, temp); }
void orc_repetition_penalty(float* v, int n, const int32_t* ids, int64_t n_ids, float pen) {
  penalty_row(v, n, ids, n_ids, pen);
}
void orc_top_k(float* v, int n, int k) { top_k_row(v, n, k); }
void orc_top_p(float* v, int n, float p, int min_keep) { top_p_row(v, n, p, min_keep, false); }
void orc_top_p_literal(float* v, int n, float p, int min_keep) { top_p_row(v, n, p, min_keep, true); }
int orc_argmax(const float* v, int n) { return argmax_row(v, n); }

// ---- RNG and draw -----------------------------------------------------------
uint64_t orc_xorshift64(uint64_t s) { return xorshift_step(s); }
// text2semantic.cpp:109
uint64_t orc_seed_single(uint64_t seed) { return seed ? seed : 0x9E3779B97F4A7C15ull; }
// text2semantic.cpp:292-294
void orc_seed_batch(uint64_t seed, int n, uint64_t* out) {
  const uint64_t base = seed ? seed : 0x9E3779B97F4A7C15ull;
  for (int b = 0; b < n; ++b) out[b] = base + static_cast<uint64_t>(b) * 0x100000001b3ull;
}
int orc_draw(const float* v, int n, uint64_t* rng) { return draw_row(v, n, rng); }

// ---- batched chain: one AR step over n_rows rows ---------------------------
// logits: f32 rows (dtype 0) or bf16 bit patterns (dtype 1), row stride `ld`
// elements. History in CSR form (hist_off has n_rows+1 entries). Per-row
// parameters. out_masked (optional, n_rows x vocab f32) receives the row state
// just before argmax/draw. Inactive rows (row_active[b]==0) are skipped: no RNG
// advance, out_tok = -1, masked row untouched.
void orc_sample_rows(const void* logits, int dtype, int64_t ld, int n_rows, int vocab,
                     const int32_t* hist_ids, const int64_t* hist_off, const float* temp,
                     const int32_t* top_k, const float* top_p, const float* pen,
                     const int32_t* min_keep, const uint8_t* do_sample, const uint8_t* row_active,
                     uint64_t* rng, int32_t* out_tok, float* out_masked, int n_threads) {
  parallel_rows(n_rows, n_threads, [&](int b) {
    if (row_active && !row_active[b]) { out_tok[b] = -1; return; }
    std::vector<float> row(vocab);
    if (dtype == 1) {
      const uint16_t* src = static_cast<const uint16_t*>(logits) + static_cast<int64_t>(b) * ld;
      for (int i = 0; i < vocab; ++i) row[i] = bf16_to_f32(src[i]);
    } else {
      const float* src = static_cast<const float*>(logits) + static_cast<int64_t>(b) * ld;
      std::copy(src, src + vocab, row.begin());
    }
    const int64_t h0 = hist_off ? hist_off[b] : 0, h1 = hist_off ? hist_off[b + 1] : 0;
    out_tok[b] = chain_row(row.data(), vocab, hist_ids ? hist_ids + h0 : nullptr, h1 - h0, temp[b],
                           top_k[b], top_p[b], pen[b], min_keep ? min_keep[b] : 1, do_sample[b],
                           &rng[b]);
    if (out_masked) std::copy(row.begin(), row.end(), out_masked + static_cast<int64_t>(b) * vocab);
  });
}

// ---- multi-step AR stream (generate_batch inner loop, :296-337) ------------
// logits: [n_steps][n_rows][ld] f32. Each row starts from its CSR history and
// appends every sampled token that is not `stop_token` (stop_token < 0: never
// stop). A row that draws stop_token is done: its later steps report -1 and
// its RNG no longer advances. out_tok: [n_steps][n_rows].
void orc_sample_stream(const float* logits, int64_t ld, int n_steps, int n_rows, int vocab,
                       const int32_t* hist_ids, const int64_t* hist_off, const float* temp,
                       const int32_t* top_k, const float* top_p, const float* pen,
                       const uint8_t* do_sample, int stop_token, uint64_t* rng, int32_t* out_tok,
                       int n_threads) {
  parallel_rows(n_rows, n_threads, [&](int b) {
    std::vector<int32_t> hist(hist_ids + hist_off[b], hist_ids + hist_off[b + 1]);
    std::vector<float> row(vocab);
    bool done = false;
    for (int s = 0; s < n_steps; ++s) {
      int32_t& out = out_tok[static_cast<int64_t>(s) * n_rows + b];
      if (done) { out = -1; continue; }
      const float* src = logits + (static_cast<int64_t>(s) * n_rows + b) * ld;
      std::copy(src, src + vocab, row.begin());
      const int tok = chain_row(row.data(), vocab, hist.data(), static_cast<int64_t>(hist.size()),
                                temp[b], top_k[b], top_p[b], pen[b], 1, do_sample[b], &rng[b]);
      out = tok;
      if (tok == stop_token) { done = true; continue; }
      hist.push_back(tok);
    }
  });
}

// ---- LM head (config with the fused LN + linear) ---------------------------
// hidden: [M][D] bf16, gamma/beta: [D] f32, W: [V][D] (nn.cpp:11-16 takes the
// weight as (out, in)) in one of three kinds: bf16, f32, or 8-bit affine groups
// along D as the reference's quantized projections use them (gpt2.cpp:53-62,
// group 64: w = scale * q + bias per group; q one byte per element, scales and
// biases [V][D / group]); bias: [V] f32. LayerNorm over D with biased variance
// and eps (nn.cpp:73-83; eps default 1e-5, nn.h:49-50). Everything in double:
// the exact values that an fp32 LayerNorm + linear approximates. `y_out`
// (optional, [M][D]) receives the normalised rows as f32.
enum { ORC_W_BF16 = 0, ORC_W_F32 = 1, ORC_W_Q8 = 2 };

void orc_ln_lmhead(const uint16_t* hidden, int M, int D, const float* gamma, const float* beta, float eps,
                   const void* W, int wkind, const float* wscale, const float* wbias, int group,
                   const float* bias, int V, float* logits, float* y_out, int n_threads) {
  std::vector<double> y(static_cast<size_t>(M) * D);
  for (int m = 0; m < M; ++m) {
    const uint16_t* x = hidden + static_cast<int64_t>(m) * D;
    double mean = 0.0;
    for (int d = 0; d < D; ++d) mean += bf16_to_f32(x[d]);
    mean /= D;
    double var = 0.0;
    for (int d = 0; d < D; ++d) {
      const double c = bf16_to_f32(x[d]) - mean;
      var += c * c;
    }
    var /= D;
    const double inv = 1.0 / std::sqrt(var + static_cast<double>(eps));
    for (int d = 0; d < D; ++d)
      y[static_cast<size_t>(m) * D + d] = (bf16_to_f32(x[d]) - mean) * inv * gamma[d] + beta[d];
  }
  if (y_out)
    for (size_t i = 0; i < y.size(); ++i) y_out[i] = static_cast<float>(y[i]);
  parallel_rows(V, n_threads, [&](int v) {
    std::vector<double> w(D);
    for (int d = 0; d < D; ++d) {
      const int64_t i = static_cast<int64_t>(v) * D + d;
      if (wkind == ORC_W_BF16) {
        w[d] = bf16_to_f32(static_cast<const uint16_t*>(W)[i]);
      } else if (wkind == ORC_W_F32) {
        w[d] = static_cast<const float*>(W)[i];
      } else {
        const int64_t gi = static_cast<int64_t>(v) * (D / group) + d / group;
        w[d] = static_cast<double>(wscale[gi]) * static_cast<const uint8_t*>(W)[i] + wbias[gi];
      }
    }
    for (int m = 0; m < M; ++m) {
      double acc = 0.0;
      const double* h = y.data() + static_cast<size_t>(m) * D;
      for (int d = 0; d < D; ++d) acc += h[d] * w[d];
      logits[static_cast<int64_t>(m) * V + v] = static_cast<float>(acc + bias[v]);
    }
  });
}

}  // extern "C"
