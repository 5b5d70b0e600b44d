// Per-step time of the level-1 drop-in: the reference's AR loop body at B = 1
// (src/t2s/text2semantic.cpp:136-166) through c4::t2s::sampling
// (c4tts/t2s_sampling.h), which is what a c4tts build gets by swapping
// src/t2s/sampling.cpp for this library. Each step copies that step's logits
// into a std::vector (the loop's read-back, :137-140), then
//   sampled: repetition_penalty -> temperature -> top_k -> top_p -> draw
//   greedy:  repetition_penalty -> argmax
// with the pipeline's defaults (include/c4tts/pipeline.h:31-35: penalty 10,
// temperature 0.8, top_k 30, top_p 0.8) and a history that starts at 200 ids
// and grows by each token. Every call is synchronous (host vector in and out).
//
// Usage: bench_dropin [steps]   prints one JSON line.
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "c4tts/t2s_sampling.h"

namespace {

struct SplitMix {
  uint64_t s;
  uint64_t next() {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  double unit() { return (double)(next() >> 11) * 0x1p-53; }
  float normal() {   // Box-Muller
    const double u1 = unit() + 0x1p-60, u2 = unit();
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
  }
};

}  // namespace

int main(int argc, char** argv) {
  namespace S = c4::t2s::sampling;
  const int steps = argc > 1 ? std::atoi(argv[1]) : 1000;
  const int V = 8194, warm = 20;
  SplitMix g{20261202};
  // the steps' logits, made ahead: N(0, 3^2) with five spikes at +12
  std::vector<float> all((size_t)(steps + warm) * V);
  for (size_t i = 0; i < all.size(); ++i) all[i] = 3.0f * g.normal();
  for (int s = 0; s < steps + warm; ++s)
    for (int j = 0; j < 5; ++j) all[(size_t)s * V + g.next() % V] = 12.0f;
  std::vector<int> hist0(200);
  for (int& h : hist0) h = (int)(g.next() % V);

  std::vector<float> logits(V);
  double us[2] = {0.0, 0.0};
  int last[2] = {0, 0};
  for (int mode = 0; mode < 2; ++mode) {   // 0 sampled, 1 greedy
    std::vector<int> hist = hist0;
    uint64_t rng = S::seed_single(1234);
    std::chrono::steady_clock::time_point t0;
    for (int s = 0; s < steps + warm; ++s) {
      if (s == warm) t0 = std::chrono::steady_clock::now();
      const float* src = &all[(size_t)s * V];
      logits.assign(src, src + V);
      S::repetition_penalty(logits, hist, 10.0f);
      int tok;
      if (mode == 0) {
        S::temperature(logits, 0.8f);
        S::top_k(logits, 30);
        S::top_p(logits, 0.8f);
        tok = S::draw(logits, rng);
      } else {
        tok = S::argmax(logits);
      }
      if (tok != V - 1) hist.push_back(tok);
      last[mode] = tok;
    }
    const auto t1 = std::chrono::steady_clock::now();
    us[mode] = std::chrono::duration<double, std::micro>(t1 - t0).count() / steps;
  }
  std::printf("{\"steps\": %d, \"vocab\": %d, \"sampled_us_per_step\": %.3f, \"greedy_us_per_step\": %.3f, "
              "\"last_tokens\": [%d, %d]}\n",
              steps, V, us[0], us[1], last[0], last[1]);
  return 0;
}
