// Host check of c4s::repeat_add (the closed-form replay of n sequential
// double adds x <- fl(x + q) used by the exact top_p replay of a top tie
// group) against the literal loop, on seeded random inputs: every final sum
// and every count of sums at or below the threshold must agree bit for bit.
// Input families: repeated adds of 1 (the total over a tie group), of
// 1 / total from just above 1 / total (the cumulative probabilities), of
// arbitrary q across binades, and of q with few significand bits (adds whose
// rounding is a tie, resolved by parity); the last two put the threshold on
// one of the sums and just below it.
#include <cmath>
#include <cstdio>
#include <random>

#include "c4s_device.hpp"

namespace {
c4s::RepAdd literal(double x, double q, int m, double thr) {
  int le = 0;
  bool counting = true;
  for (int i = 0; i <= m; ++i) {
    if (i) x = x + q;
    if (counting) {
      if (x <= thr) le = i + 1;
      else counting = false;
    }
  }
  return c4s::RepAdd{x, le};
}
}  // namespace

int main() {
  std::mt19937_64 g(20261202);
  std::uniform_real_distribution<double> U(0.0, 1.0);
  long bad = 0, n = 0;
  for (int it = 0; it < 200000; ++it) {
    const int family = it % 6;
    const int m = 1 + (int)(U(g) * (family == 0 ? 20000 : 3000));
    double x, q, thr;
    if (family == 0) {
      x = 1.0 + (U(g) < 0.5 ? std::floor(U(g) * 4) * std::ldexp(1.0, -52 + (int)(U(g) * 3)) : 0.0);
      q = 1.0;
      thr = -1.0;
    } else if (family == 1) {
      q = 1.0 / (1.0 + U(g) * 1000.0);
      x = q + U(g) * 1e-12;
      thr = U(g);
    } else if (family == 2) {
      q = std::ldexp(U(g) + 0.5, -(int)(U(g) * 20));
      x = q * (1.0 + U(g));
      thr = 2.0 * U(g);
    } else if (family == 3) {
      q = std::ldexp(1.0 + std::floor(U(g) * 8) * 0x1p-52, -10);
      x = std::ldexp(1.0 + std::floor(U(g) * 16) * 0x1p-52, -(int)(U(g) * 9));
      thr = U(g);
    } else {
      q = 1.0 / (1.0 + U(g) * 1000.0);
      x = q * (1.0 + U(g));
      const int k = (int)(U(g) * (m + 1));
      thr = literal(x, q, k, -1.0).x;   // the k-th sum
      if (family == 5) thr = std::nextafter(thr, 0.0);
    }
    const c4s::RepAdd want = literal(x, q, m, thr);
    const c4s::RepAdd got = c4s::repeat_add(x, q, m, thr, true);
    const c4s::RepAdd cnt = c4s::repeat_add(x, q, m, thr, false);
    ++n;
    if (got.x != want.x || got.le != want.le || cnt.le != want.le) {
      if (bad < 5)
        std::printf("mismatch: family %d x %.17g q %.17g m %d thr %.17g: got %.17g / %d (%d), want %.17g / %d\n",
                    family, x, q, m, thr, got.x, got.le, cnt.le, want.x, want.le);
      ++bad;
    }
  }
  std::printf("repeat_add: %ld cases, %ld mismatches\n", n, bad);
  return bad != 0;
}
