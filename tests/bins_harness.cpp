// CPU harness for ace::bucket (ace-kernels_amd/csrc/ace_bins.hpp), the bin index
// the kernels use.  Built with g++ by tests/test_bins.py and called through
// ctypes; the reference answer is a binary search over the same float32 table
// (std::lower_bound / std::upper_bound == torch.bucketize semantics).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

#include "ace_bins.hpp"

namespace {

std::vector<float> padded(const float* table, int n) {
  std::vector<float> tab(n + 2);
  tab[0] = -std::numeric_limits<float>::infinity();
  for (int j = 0; j < n; ++j) tab[j + 1] = table[j];
  tab[n + 1] = std::numeric_limits<float>::infinity();
  return tab;
}

int expected(const float* table, int n, float p, bool right) {
  const float* end = table + n;
  const float* it = right ? std::upper_bound(table, end, p) : std::lower_bound(table, end, p);
  return (int)(it - table);  // number of entries < p (<= p if right)
}

float from_bits(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint32_t to_bits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

}  // namespace

extern "C" {

// Mismatches of ace::bucket against the binary search for `count` values.
long long check_values(const float* table, int n, int right, const float* ps, long long count) {
  const std::vector<float> tab = padded(table, n);
  long long bad = 0;
  for (long long i = 0; i < count; ++i) {
    const float p = ps[i];
    if (std::isnan(p)) continue;
    int want = expected(table, n, p, right != 0);
    if (want > n - 1) want = n - 1;  // p above the last edge: kernels clamp
    if ((right ? ace::bucket<true>(p, (float)n, n, tab.data()) : ace::bucket<false>(p, (float)n, n, tab.data())) != want) ++bad;
  }
  return bad;
}

// Every float32 within `ulps` of every table entry (and of 0 and 1).
long long check_near_edges(const float* table, int n, int right, int ulps) {
  const std::vector<float> tab = padded(table, n);
  long long bad = 0;
  std::vector<float> centres(table, table + n);
  centres.push_back(0.0f);
  centres.push_back(1.0f);
  for (float c : centres) {
    const int64_t b = (int64_t)to_bits(c);
    for (int64_t d = -ulps; d <= ulps; ++d) {
      const int64_t u = b + d;
      if (u < 0 || u > 0x7f7fffff) continue;
      const float p = from_bits((uint32_t)u);
      int want = expected(table, n, p, right != 0);
      if (want > n - 1) want = n - 1;
      if ((right ? ace::bucket<true>(p, (float)n, n, tab.data()) : ace::bucket<false>(p, (float)n, n, tab.data())) != want) ++bad;
    }
  }
  return bad;
}

// Every float32 in [lo, hi] (both >= 0): an exhaustive check of one table.
long long check_range(const float* table, int n, int right, float lo, float hi) {
  const std::vector<float> tab = padded(table, n);
  const uint32_t a = to_bits(lo), z = to_bits(hi);
  long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (int64_t u = a; u <= (int64_t)z; ++u) {
    const float p = from_bits((uint32_t)u);
    int want = expected(table, n, p, right != 0);
    if (want > n - 1) want = n - 1;
    if ((right ? ace::bucket<true>(p, (float)n, n, tab.data()) : ace::bucket<false>(p, (float)n, n, tab.data())) != want) ++bad;
  }
  return bad;
}

// bucket<RIGHT, false> (no input clamp, the softmax path) at every float32 in
// [lo, hi] within [0, 1], and at every float32 of [0, 1] within `ulps` of an
// edge when ulps > 0 (lo, hi then ignored).
long long check_unclamped(const float* table, int n, int right, float lo, float hi, int ulps) {
  const std::vector<float> tab = padded(table, n);
  auto one = [&](float p) -> long long {
    int want = expected(table, n, p, right != 0);
    if (want > n - 1) want = n - 1;
    const int k = right ? ace::bucket<true, false>(p, (float)n, n, tab.data())
                        : ace::bucket<false, false>(p, (float)n, n, tab.data());
    return k != want ? 1 : 0;
  };
  long long bad = 0;
  if (ulps > 0) {
    std::vector<float> centres(table, table + n);
    centres.push_back(0.0f);
    centres.push_back(1.0f);
    for (float c : centres) {
      const int64_t b = (int64_t)to_bits(c);
      for (int64_t d = -ulps; d <= ulps; ++d) {
        const int64_t u = b + d;
        if (u < 0 || u > (int64_t)to_bits(1.0f)) continue;
        bad += one(from_bits((uint32_t)u));
      }
    }
    return bad;
  }
  const uint32_t a = to_bits(lo), z = to_bits(hi);
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (int64_t u = a; u <= (int64_t)z; ++u) bad += one(from_bits((uint32_t)u));
  return bad;
}

// bucket<RIGHT, false> of a NaN (NaN logits) is 0, inside the histogram.
int check_unclamped_nan(const float* table, int n) {
  const std::vector<float> tab = padded(table, n);
  const float q = std::nanf("");
  return ace::bucket<false, false>(q, (float)n, n, tab.data()) == 0 &&
         ace::bucket<true, false>(q, (float)n, n, tab.data()) == 0;
}

// Planted mistake for the sensitivity test: the first guess floor(p * n)
// without the correction against the table.
long long check_near_edges_uncorrected(const float* table, int n, int right, int ulps) {
  long long bad = 0;
  for (int j = 0; j < n; ++j) {
    const int64_t b = (int64_t)to_bits(table[j]);
    for (int64_t d = -ulps; d <= ulps; ++d) {
      const float p = from_bits((uint32_t)(b + d));
      int want = expected(table, n, p, right != 0);
      if (want > n - 1) want = n - 1;
      float t = std::fmin(std::fmax(p * (float)n, 0.0f), (float)n);
      int g = (int)t;
      g = g > n - 1 ? n - 1 : g;
      if (g != want) ++bad;
    }
  }
  return bad;
}

// Out-of-domain inputs stay in [0, n - 1] (histogram indices never leave range).
int check_clamped(const float* table, int n) {
  const std::vector<float> tab = padded(table, n);
  const float odd[] = {std::nanf(""), -std::numeric_limits<float>::infinity(),
                       std::numeric_limits<float>::infinity(), -1.0f, -1e30f, 2.0f, 1e30f,
                       -0.0f, 1.0000002f};
  for (float p : odd)
    for (int r = 0; r < 2; ++r) {
      const int k = r ? ace::bucket<true>(p, (float)n, n, tab.data()) : ace::bucket<false>(p, (float)n, n, tab.data());
      if (k < 0 || k > n - 1) return 0;
    }
  return 1;
}

}  // extern "C"
