// Helpers shared by the C++ test programs: failure counting, a seeded normal generator and the
// relative-error measure of the parity tests (element-wise with a floor of 1e-3 * max|ref|, and
// max|diff| / max|ref|).
#ifndef SQ8_TESTS_CPP_TEST_UTIL_H_
#define SQ8_TESTS_CPP_TEST_UTIL_H_
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <vector>

namespace sq8test {

inline int& failures() {
  static int n = 0;
  return n;
}

#define EXPECT(cond, msg)                                                  \
  do {                                                                     \
    if (!(cond)) {                                                         \
      std::printf("FAIL %s:%d %s (%s)\n", __FILE__, __LINE__, #cond, msg); \
      ++sq8test::failures();                                               \
    }                                                                      \
  } while (0)

// Deterministic N(0, sigma) values (Box-Muller over a 64-bit LCG).
struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed * 6364136223846793005ull + 1442695040888963407ull) {}
  double uni() {
    s = s * 6364136223846793005ull + 1442695040888963407ull;
    return ((s >> 11) + 0.5) / 9007199254740992.0;
  }
  float normal(float sigma) {
    return static_cast<float>(sigma * std::sqrt(-2.0 * std::log(uni())) *
                              std::cos(6.283185307179586 * uni()));
  }
};

inline double max_rel_err(const std::vector<float>& y, const std::vector<double>& r, double* norm) {
  double amax = 0, dmax = 0, elem = 0;
  for (double v : r) amax = std::fmax(amax, std::fabs(v));
  for (size_t i = 0; i < y.size(); ++i) {
    const double d = std::fabs(y[i] - r[i]);
    dmax = std::fmax(dmax, d);
    elem = std::fmax(elem, d / std::fmax(std::fabs(r[i]), 1e-3 * amax));
  }
  *norm = amax > 0 ? dmax / amax : dmax;
  return elem;
}

}  // namespace sq8test
#endif  // SQ8_TESTS_CPP_TEST_UTIL_H_
