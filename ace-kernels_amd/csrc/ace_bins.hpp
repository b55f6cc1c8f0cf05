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
// one of that count, so one up-check and one down-check against the table make
// it exact.  `tab` is padded: tab[0] = -inf, tab[1 + j] = table[j],
// tab[n + 1] = +inf, so both neighbours of the first guess are read together.
// The result is clamped to [0, n - 1]: p > 1 + eps32 and NaN are outside the
// reference's domain (its scatter raises for them), and the clamp keeps every
// histogram index in range.
// CLAMP = false is for probabilities known to lie in [0, 1] (softmax output):
// p * n is then in [0, n] and needs no clamping; the final clamp stays so that
// NaN logits cannot produce an index out of range.
template <bool RIGHT, bool CLAMP = true>
ACE_HD int bucket(float p, float nf, int n, const float* tab) {
  const float t = CLAMP ? fminf(fmaxf(p * nf, 0.0f), nf) : p * nf;  // fmaxf(NaN, 0) = 0
  const int g = (int)t;                            // t >= 0: truncation is floor
  const float lo = tab[g];                         // table[g - 1]
  const float hi = tab[g + 1];                     // table[g]
  const bool up = RIGHT ? (hi <= p) : (hi < p);
  const int g1 = g + (up ? 1 : 0);
  const float lo1 = up ? hi : lo;                  // table[g1 - 1]
  const bool keep = RIGHT ? (lo1 <= p) : (lo1 < p);
  int g2 = g1 - (keep ? 0 : 1);
  g2 = g2 < 0 ? 0 : g2;
  return g2 > n - 1 ? n - 1 : g2;
}

}  // namespace ace
