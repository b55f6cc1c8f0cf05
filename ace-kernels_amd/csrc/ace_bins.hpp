// O(1) bin index, shared by the kernels and the CPU test harness
// (tests/bins_harness.cpp compiles this header with g++ and checks it against
// a binary search at every float32 near every boundary).
#pragma once

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define ACE_HD __host__ __device__ __forceinline__
#else
#include <algorithm>
#include <cmath>
#define ACE_HD inline
#endif

namespace ace {

// torch.bucketize(p, table, right) for a sorted table of n float32 values with
// entry j ~= (j + 1) / n (the reference's torch.linspace edges): the number of
// entries < p (right == false) or <= p (right == true).  floor(p * n) is within
// one of that count, so one up-check against table[g] and one down-check
// against table[g - 1] make it exact: count = g + (table[g] < p) -
// (table[g - 1] >= p) (<= and > for right); the two checks never both hold
// because the table is sorted.  `tab` is padded: tab[0] = -inf,
// tab[1 + j] = table[j], tab[n + 1] = +inf, so both neighbours of the first
// guess are read together.
// CLAMP = true clamps p * n to [0, n] and the result to [0, n - 1]: p > 1 + eps32
// and NaN are outside the reference's domain (its scatter raises for them), and
// the clamp keeps every histogram index in range.
// CLAMP = false is for probabilities known to lie in [0, 1] (softmax output):
// p * n is then in [0, n] and the result in [0, n - 1] (the last table entry,
// 1 + eps, exceeds p); a NaN p is mapped to g = 0 by fmaxf and fails both
// checks, so it lands in bin 0.
template <bool RIGHT, bool CLAMP = true>
ACE_HD int bucket(float p, float nf, int n, const float* tab) {
  const float t = CLAMP ? fminf(fmaxf(p * nf, 0.0f), nf) : fmaxf(p * nf, 0.0f);  // fmaxf(NaN, 0) = 0
  const int g = (int)t;                            // t >= 0: truncation is floor
  const float lo = tab[g];                         // table[g - 1]
  const float hi = tab[g + 1];                     // table[g]
  const bool up = RIGHT ? (hi <= p) : (hi < p);
  const bool down = RIGHT ? (lo > p) : (lo >= p);
  const int g2 = g + (up ? 1 : 0) - (down ? 1 : 0);
  if (!CLAMP) return g2;
  return g2 < 0 ? 0 : (g2 > n - 1 ? n - 1 : g2);
}

}  // namespace ace
