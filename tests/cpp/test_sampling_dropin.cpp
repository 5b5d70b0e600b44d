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
#include <limits>
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

// Acceptance rule of the reference's sampling test: the -inf pattern must be
// identical, and every finite entry within 1e-5 of the golden value.
struct RowDiff {
  size_t mask_mismatches = 0;   // positions -inf on one side only
  double largest = 0.0;         // largest |difference| over positions finite on both sides
  bool same_length = true;
};

static bool is_neg_inf(float x) { return x == -std::numeric_limits<float>::infinity(); }

static RowDiff diff_rows(const std::vector<float>& a, const std::vector<float>& b) {
  RowDiff d;
  if (a.size() != b.size()) {
    d.same_length = false;
    return d;
  }
  for (size_t i = 0; i < a.size(); ++i) {
    if (is_neg_inf(a[i]) != is_neg_inf(b[i])) {
      ++d.mask_mismatches;
    } else if (!is_neg_inf(a[i])) {
      d.largest = std::max(d.largest, std::fabs((double)a[i] - (double)b[i]));
    }
  }
  return d;
}

static void expect_row(const char* what, const std::vector<float>& got, const std::vector<float>& golden) {
  const RowDiff d = diff_rows(got, golden);
  const bool pass = d.same_length && d.mask_mismatches == 0 && d.largest < 1e-5;
  if (!pass) ++failures;
  std::printf("  %-18s %s  |diff| <= %.2e, -inf mismatches %zu%s\n", what, pass ? "ok  " : "FAIL", d.largest,
              d.mask_mismatches, d.same_length ? "" : ", lengths differ");
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
    std::vector<float> row;
    row = base;
    S::temperature(row, (float)temp);
    expect_row("temperature", row, read_raw<float>(d + "temp.f32"));
    row = base;
    S::repetition_penalty(row, ids, (float)pen);
    expect_row("repetition_penalty", row, read_raw<float>(d + "rep.f32"));
    row = base;
    S::top_k(row, (int)k);
    expect_row("top_k", row, read_raw<float>(d + "topk.f32"));
    row = base;
    S::top_p(row, (float)p);
    expect_row("top_p", row, read_raw<float>(d + "topp.f32"));
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
