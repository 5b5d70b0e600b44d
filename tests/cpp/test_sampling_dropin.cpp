// Drop-in test for the c4::t2s::sampling C++ entry points running on the GPU.
//
// Mirrors the reference's tests/test_sampling.cpp:24-55: apply each processor
// once to a golden row and compare with the golden output (max-abs < 1e-5 over
// finite entries, identical -inf masks). Also checks argmax and the draw
// against values computed by the CPU oracle. Inputs are raw little-endian
// files written by tests/test_gpu_dropin_cpp.py into one directory per case:
//   logits.f32 ids.i32 params.txt (temp penalty top_k top_p seed)
//   temp.f32 rep.f32 topk.f32 topp.f32 expect.txt (argmax draw_token draw_state)
// Usage: test_sampling_dropin <case_dir>...

#include <cmath>
#include <cstring>
#include <algorithm>
#include <cstdio>
#include <fstream>
#include <iterator>
#include <string>
#include <vector>

#include "c4tts/t2s_sampling.h"

namespace S = c4::t2s::sampling;
static int failures = 0;

template <class T>
static std::vector<T> read_raw(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  std::vector<char> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  std::vector<T> out(bytes.size() / sizeof(T));
  if (!out.empty()) std::memcpy(out.data(), bytes.data(), out.size() * sizeof(T));
  return out;
}

static void check(const std::string& name, const std::vector<float>& got,
                  const std::vector<float>& ref) {
  double max_err = 0;
  bool ok = got.size() == ref.size();
  for (size_t i = 0; ok && i < got.size(); ++i) {
    const bool gi = std::isinf(got[i]) && got[i] < 0;
    const bool ri = std::isinf(ref[i]) && ref[i] < 0;
    if (gi != ri) { ok = false; break; }
    if (!gi) max_err = std::max(max_err, (double)std::fabs(got[i] - ref[i]));
  }
  const bool pass = ok && max_err < 1e-5;
  std::printf("  [%s] max_err=%.3e %s\n", name.c_str(), max_err, pass ? "" : "<-- FAIL");
  if (!pass) ++failures;
}

int main(int argc, char** argv) {
  std::printf("test_sampling_dropin:\n");
  for (int a = 1; a < argc; ++a) {
    const std::string d = std::string(argv[a]) + "/";
    std::printf(" case %s\n", argv[a]);
    const std::vector<float> base = read_raw<float>(d + "logits.f32");
    const std::vector<int> ids = read_raw<int>(d + "ids.i32");
    double temp = 1, pen = 1, p = 1;
    long long k = 0;
    unsigned long long seed = 0;
    {
      std::ifstream f(d + "params.txt");
      f >> temp >> pen >> k >> p >> seed;
    }
    { auto v = base; S::temperature(v, (float)temp); check("temperature", v, read_raw<float>(d + "temp.f32")); }
    { auto v = base; S::repetition_penalty(v, ids, (float)pen); check("repetition_penalty", v, read_raw<float>(d + "rep.f32")); }
    { auto v = base; S::top_k(v, (int)k); check("top_k", v, read_raw<float>(d + "topk.f32")); }
    { auto v = base; S::top_p(v, (float)p); check("top_p", v, read_raw<float>(d + "topp.f32")); }
    long long exp_arg = -1, exp_tok = -1;
    unsigned long long exp_state = 0;
    {
      std::ifstream f(d + "expect.txt");
      f >> exp_arg >> exp_tok >> exp_state;
    }
    const int got_arg = S::argmax(base);
    std::printf("  [argmax] got=%d want=%lld %s\n", got_arg, exp_arg, got_arg == exp_arg ? "" : "<-- FAIL");
    if (got_arg != exp_arg) ++failures;
    auto v = base;
    S::top_p(v, (float)p);
    uint64_t state = S::seed_single(seed);
    const int tok = S::draw(v, state);
    const bool ok = tok == exp_tok && state == exp_state;
    std::printf("  [draw] got=%d want=%lld state_ok=%d %s\n", tok, exp_tok, (int)(state == exp_state),
                ok ? "" : "<-- FAIL");
    if (!ok) ++failures;
  }
  std::printf("test_sampling_dropin: %s\n", failures == 0 ? "ALL PASSED" : "FAILED");
  return failures == 0 ? 0 : 1;
}
