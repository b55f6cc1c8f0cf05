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

// bucket_unit<RIGHT> (probabilities in [0, 1], one correction: the softmax
// path) at every float32 in [lo, hi] within [0, 1], and at every float32 of
// [0, 1] within `ulps` of an edge when ulps > 0 (lo, hi then ignored).
// planted != 0 drops the correction (the first guess alone): the sweep must
// then find mismatches.
long long check_unit(const float* table, int n, int right, float lo, float hi, int ulps,
                     int planted) {
  const std::vector<float> tab = padded(table, n);
  auto one = [&](float p) -> long long {
    int want = expected(table, n, p, right != 0);
    if (want > n - 1) want = n - 1;
    int k;
    if (planted) {
      const float t = std::fmaf(p, (float)n, -0.25f);
      k = (int)t;
    } else {
      k = right ? ace::bucket_unit<true>(p, (float)n, tab.data())
                : ace::bucket_unit<false>(p, (float)n, tab.data());
    }
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

// ace::div_rn(a, b, 1 / b) against a / b: every float b with bits in
// [b_lo, b_hi) times `per_b` pseudo-random a of exponents in [ea, eb] (plus
// a = 1 and a = b / 2).  Returns the mismatches.  planted != 0 checks a * y
// instead (no residual correction): the check must then report mismatches.
long long check_div(uint32_t b_lo, uint32_t b_hi, int per_b, int ea, int eb, int planted) {
  long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (int64_t u = b_lo; u < (int64_t)b_hi; ++u) {
    const float b = from_bits((uint32_t)u);
    const float y = 1.0f / b;
    uint32_t h = (uint32_t)u * 2654435761u;
    for (int t = 0; t < per_b + 2; ++t) {
      h ^= h >> 15;
      h *= 0x2c1b3c6dU;
      h ^= h >> 12;
      h *= 0x297a2d39U;
      h ^= h >> 15;
      float a;
      if (t == 0) {
        a = 1.0f;
      } else if (t == 1) {
        a = b * 0.5f;
      } else {
        const int e = ea + (int)(h % (uint32_t)(eb - ea + 1));
        a = std::ldexp(1.0f + (float)(h >> 9) * (1.0f / 8388608.0f), e);
      }
      if ((planted ? a * y : ace::div_rn(a, b, y)) != a / b) ++bad;
    }
  }
  return bad;
}

// bucket_unit of a NaN (NaN logits) is 0, inside the histogram.
int check_unit_nan(const float* table, int n) {
  const std::vector<float> tab = padded(table, n);
  const float q = std::nanf("");
  return ace::bucket_unit<false>(q, (float)n, tab.data()) == 0 &&
         ace::bucket_unit<true>(q, (float)n, tab.data()) == 0;
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

// Soft moments fixed point (ace::moment_scale): for the 2K half boundaries
// `table` (torch.linspace(0, 1 + eps, 2K + 1)[1:]) every half-bin's
// smallest and largest quantised probability q = trunc(p 2^m) lies in
// [h w, h w + 2^24), w < 2^23 and h w fits 32 bits.  p ranges over
// (e_{h-1}, e_h] (right: [e_{h-1}, e_h)) with e_{-1} = 0 and p <= 1.
// planted 1: m one larger; planted 2: w = ceil(ws) (no margin below the
// boundaries).  Returns the violations.
long long check_moment_offsets(const float* table, int K, int planted) {
  ace::MomentScale s = ace::moment_scale(K);
  if (planted == 1) {
    s.m += 1;
    s.w = (int)((double)(1ll << s.m) / (2.0 * K) * (1.0 - 1.0 / 16384.0));
  } else if (planted == 2) {
    s.w = (int)std::ceil((double)(1ll << s.m) / (2.0 * K));
  }
  const int n = 2 * K;
  long long bad = s.w >= (1 << 23) ? 1 : 0;
  const float sc = std::ldexp(1.0f, s.m);
  for (int h = 0; h < n; ++h) {
    const uint32_t qlo = h == 0 ? 0u : (uint32_t)(table[h - 1] * sc);
    const uint32_t qhi = (uint32_t)(std::fmin(table[h], 1.0f) * sc);
    const long long base = (long long)h * s.w;
    if (base > 0x7fffffffLL) ++bad;
    if ((long long)qlo < base) ++bad;
    if ((long long)qhi - base >= (long long)ace::kMomentUMax) ++bad;
  }
  return bad;
}

// The offsets of every float32 p in [0, 1] (the softmax path: bucket_unit
// half-bin h): 0 <= u < 2^24, and base + u reproduces q = trunc(p 2^m),
// which equals p 2^m for p >= 2^(23 - m).  Returns the violations.
long long check_moment_all(const float* table, int K, int right) {
  const ace::MomentScale s = ace::moment_scale(K);
  const int n = 2 * K;
  const std::vector<float> tab = padded(table, n);
  const float sc = std::ldexp(1.0f, s.m);
  const float exact_from = std::ldexp(1.0f, 23 - s.m);
  long long bad = 0;
  const uint32_t z = to_bits(1.0f);
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (int64_t b = 0; b <= (int64_t)z; ++b) {
    const float p = from_bits((uint32_t)b);
    const int h = right ? ace::bucket_unit<true>(p, (float)n, tab.data())
                        : ace::bucket_unit<false>(p, (float)n, tab.data());
    const float ps = p * sc;
    const int64_t q = (int64_t)ps;
    const int64_t u = q - (int64_t)h * s.w;
    if (u < 0 || u >= (int64_t)ace::kMomentUMax) ++bad;
    if (p >= exact_from && (double)q != (double)ps) ++bad;
  }
  return bad;
}

// The fast bins' margin against their error bound: for every float32 p
// within `width` ulp of every entry of `table` (the n hard edges), and a
// sample of [0, 1] every 997 ulp, take the
// fast path's q at the two ends of the error window, trunc(p n 2^qs
// (1 -+ rel)); whenever fast_bin_index calls such a q not near an edge, its
// bin must equal torch.bucketize(p) (left and right).  margin_div > 1
// plants a margin that many times too small.  Returns the violations.
long long check_fast_margin(const float* table, int n, int channels, double rel, int width,
                            int margin_div) {
  ace::FastBinConsts f = ace::fast_bin_consts(n, channels);
  if (margin_div > 1) f.qmq = f.qmq / (uint32_t)margin_div;
  const double scale = std::ldexp((double)n, f.qs);
  const uint32_t one = to_bits(1.0f);
  long long bad = 0;
  auto check = [&](float p) -> long long {
    long long b = 0;
    for (int r = 0; r < 2; ++r) {
      int want = expected(table, n, p, r != 0);
      if (want > n - 1) want = n - 1;
      for (double s : {1.0 - rel, 1.0 + rel}) {
        double qd = std::floor((double)p * scale * s);
        if (qd < 0) qd = 0;
        if (qd > scale) qd = scale;
        uint32_t k;
        const bool near = ace::fast_bin_index((uint32_t)qd, f.qlo, f.qhi, f.qmq, f.qmask, f.qs, k);
        if (!near && (int)k != want) ++b;
      }
    }
    return b;
  };
#pragma omp parallel for reduction(+ : bad) schedule(dynamic)
  for (int j = 0; j < n; ++j) {
    const int64_t e = to_bits(table[j]);
    for (int64_t d = -width; d <= width; ++d) {
      const int64_t bits = e + d;
      if (bits < 0 || bits > (int64_t)one) continue;
      bad += check(from_bits((uint32_t)bits));
    }
  }
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (int64_t bits = 0; bits <= (int64_t)one; bits += 997) bad += check(from_bits((uint32_t)bits));
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
