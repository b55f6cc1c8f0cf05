// O(1) bin index, shared by the kernels and the CPU test harness
// (tests/bins_harness.cpp compiles this header with g++ and checks it against
// a binary search at every float32 near every boundary).
#pragma once

#include <stdint.h>

#include <cmath>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define ACE_HD __host__ __device__ __forceinline__
#else
#include <algorithm>
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
// p * n is clamped to [0, n] and the result to [0, n - 1]: p > 1 + eps32 and
// NaN are outside the reference's domain (its scatter raises for them), and
// the clamp keeps every histogram index in range.  Probabilities known to lie
// in [0, 1] (softmax output) take bucket_unit below, with one check.
template <bool RIGHT>
ACE_HD int bucket(float p, float nf, int n, const float* tab) {
  const float t = fminf(fmaxf(p * nf, 0.0f), nf);  // fmaxf(NaN, 0) = 0
  const int g = (int)t;                            // t >= 0: truncation is floor
  const float lo = tab[g];                         // table[g - 1]
  const float hi = tab[g + 1];                     // table[g]
  const bool up = RIGHT ? (hi <= p) : (hi < p);
  const bool down = RIGHT ? (lo > p) : (lo >= p);
  const int g2 = g + (up ? 1 : 0) - (down ? 1 : 0);
  return g2 < 0 ? 0 : (g2 > n - 1 ? n - 1 : g2);
}

// a / b correctly rounded from y = RN(1 / b) (Markstein): q = RN(a y) is
// within an ulp, the residual a - b q is exact, and RN(q + r y) is the IEEE
// quotient while a and a / b stay >= 2^-100 (the residual then does not
// underflow).  Three instructions.
ACE_HD float div_rn(float a, float b, float y) {
  const float q = a * y;
  const float r = fmaf(-b, q, a);
  return fmaf(r, y, q);
}

// Bin of a probability p in [0, 1] (or NaN -> 0) with a single correction:
// the first guess g = trunc(p * n - 1/4) is the bin k or k - 1, never more
// or less, so one comparison with the upper edge of bin g fixes it.  With
// the float32 edges e_j = linspace(0, 1 + eps, n + 1)[j + 1] = (j + 1) / n
// times (1 + d_j), |d_j| < 8 * 2^-24 (eps and torch's float32 rounding), and
// the fused p * n - 1/4 rounded once:
//   p <= e_k      gives p * n - 1/4 <= k + 3/4 + (k + 1) * 8 * 2^-24 < k + 1
//                 for n < 2^19, so g <= k;
//   p >  e_{k-1}  gives p * n - 1/4 > k - 1/4 - k * 8 * 2^-24 > k - 1, so
//                 g >= k - 1 (and g = 0 when k = 0).
// g <= n - 1 for p <= 1, and e_{n-1} = 1 + eps > 1, so no clamp is needed.
// tab is the padded table (tab[j + 1] = e_j).  NaN bins to 0: the device
// conversion is v_cvt_i32_f32, which maps NaN to 0.
ACE_HD int bucket_guess(float p, float nf) {
  const float t = fmaf(p, nf, -0.25f);
#if defined(__HIP_DEVICE_COMPILE__)
  int g;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(g) : "v"(t));
  return g;
#else
  return t == t ? (int)t : 0;
#endif
}
// e = tab[g + 1], the upper edge of bin g.
template <bool RIGHT>
ACE_HD int bucket_fix(int g, float e, float p) {
  return g + ((RIGHT ? (e <= p) : (e < p)) ? 1 : 0);
}
template <bool RIGHT>
ACE_HD int bucket_unit(float p, float nf, const float* tab) {
  const int g = bucket_guess(p, nf);
  return bucket_fix<RIGHT>(g, tab[g + 1], p);
}

// Fast bins (the hard forward kernels with class labels: ace_core.hpp,
// fast_exp / fast_bin): with n = K bins a probability is held as
// q = trunc(p n 2^qs), n 2^qs <= 2^30.  Its bin is k = z >> qs, z = q
// clamped to [2^(qs-1), (2n - 1) 2^(qs-1)] (t = p n clamped to [1/2, n - 1/2],
// away from the outer edges 0 and n), and it is "near" an interior edge
// when z lies within qmq of a multiple of 2^qs.  The margin qmq is n 2^-18
// of t (C <= 4 channels) or n 2^-17 (more), in units of 2^-qs: twice the
// fast probabilities' relative error bound (3e-6 at C = 16) plus the edges'
// offsets from (j + 1) / n (8 2^-24 relative, see bucket_unit).  Beyond 512
// bins the margin is half a bin: every value is near, and the kernels take
// the exact path throughout.
struct FastBinConsts {
  float qscale;      // n 2^qs
  uint32_t qlo, qhi; // 2^(qs-1), (2n - 1) 2^(qs-1)
  uint32_t qmq;      // margin
  uint32_t qmask;    // 2^qs - 1
  int qs;
  double pscale;     // 1 / (n 2^qs): the value of one unit of q
};

inline FastBinConsts fast_bin_consts(int n, long long channels) {
  int c = 0;
  while ((1ll << c) < n) ++c;  // ceil(log2 n)
  const int qs = 30 - c;
  FastBinConsts f;
  f.qs = qs;
  f.qscale = (float)std::ldexp((double)n, qs);
  f.qlo = 1u << (qs - 1);
  f.qhi = (uint32_t)(2 * n - 1) << (qs - 1);
  f.qmask = (1u << qs) - 1;
  unsigned long long mq = ((unsigned long long)n << qs) >> (channels <= 4 ? 18 : 17);
  if (mq < 1) mq = 1;
  if (n > 512) mq = 1ull << (qs - 1);
  f.qmq = (uint32_t)mq;
  f.pscale = 1.0 / std::ldexp((double)n, qs);
  return f;
}

// The bin of q and whether q is near an interior edge (see FastBinConsts).
ACE_HD uint32_t med3_u32(uint32_t a, uint32_t lo, uint32_t hi) {
#if defined(__HIP_DEVICE_COMPILE__)
  uint32_t r;
  asm("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(lo), "v"(hi));
  return r;
#else
  return a < lo ? lo : (a > hi ? hi : a);
#endif
}
ACE_HD bool fast_bin_index(uint32_t q, uint32_t qlo, uint32_t qhi, uint32_t qmq, uint32_t qmask,
                           int qs, uint32_t& k) {
  const uint32_t z = med3_u32(q, qlo, qhi);
  k = z >> qs;
  return ((z + qmq) & qmask) < 2 * qmq;
}

// Fixed point of the soft moments (per half-bin sums of p and p^2).  A
// probability in half-bin h is quantised to q = trunc(p 2^m) and stored as
// its offset u = q - h w from the integer base h w, so that u^2 is exact in
// 64 bits and the sums describe the quantised values exactly (the moment
// formulas subtract nearly equal sums, so a rounded p^2 would carry its
// rounding, amplified by 1 / S = 2K, into P).  q is exact (p 2^m is an
// integer) for p >= 2^(23-m): p >= 2^-5 at m = 28 (K = 16..31).  With the
// half boundaries e_h = h / 2K (1 + d_h), |d_h| < 8 2^-24 (see bucket_unit),
// and ws = 2^m / 2K <= 2^23:
//   w <= ws (1 - 2^-14) and h w < e_h 2^m for h >= 1, so u >= 0;
//   u <= e_{h+1} 2^m - h w < ws (1 + 2K (2^-14 + 2^-21)) + 2K
//     < 1.26 * 2^23 + 2^12 < 2^24 = kMomentUMax for 2K <= 2^12,
// so h w and u^2 are 24-bit multiplies (w < 2^23 fits a signed one).
// m = 23 + floor(log2 2K), at most 30 (2^22 < ws <= 2^23 while m < 30).
constexpr int kMomentMaxBins = 2048;
constexpr unsigned kMomentUMax = 1u << 24;

struct MomentScale {
  int m;  // q = trunc(p 2^m)
  int w;  // base of half-bin h: h w
};

ACE_HD MomentScale moment_scale(int num_bins) {
  int lg = 0;
  while ((2ll << lg) <= 2ll * num_bins) ++lg;  // floor(log2 2K)
  MomentScale s;
  s.m = 23 + lg < 30 ? 23 + lg : 30;
  const double ws = (double)(1ll << s.m) / (2.0 * num_bins);
  s.w = (int)(ws * (1.0 - 1.0 / 16384.0));
  return s;
}

// Right shift of the per-copy sums of u^2 before they are added into the
// final sums of a batch index of N voxels: u^2 < 2^48, one copy holds at
// most 4095 voxels (< 2^60), a block's tile fewer than 2^15 (below N unless
// N >= 2^14, where the shift is at least 1), and N 2^48 / 2^shift < 2^62.
ACE_HD int moment_shift(long long voxels) {
  int bits = 0;
  while (bits < 62 && (1ll << bits) <= voxels) ++bits;  // bit length of N
  return bits > 14 ? bits - 14 : 0;
}

}  // namespace ace
