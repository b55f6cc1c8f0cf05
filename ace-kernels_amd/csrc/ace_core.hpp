// mL1-ACE forward / backward kernels for CDNA4 (gfx950).
//
// Forward (one launch): every block streams a tile of voxels of one batch
// index, computes the channel softmax (or sigmoid) in registers, bins every
// loss channel (hard: one bin; soft: two neighbouring bins with interpolation
// weights) and accumulates the per-bin sums W, P, G into LDS histograms.  The
// sums are fixed-point integers (30 fraction bits) added with LDS integer
// atomics, so they are exact for the float32 terms >= 2^-7 (and within 2^-31
// per term below) and independent of the order of addition: the result is
// bitwise deterministic with no float atomics.  Lane l of a wave adds into
// copy (l % copies) of the histogram, copies laid out bin-major, so the lanes
// one LDS cycle serves hit distinct banks whatever their bins.  Each block
// then adds its sums into one of a few replicas of its batch index's final
// sums with integer atomics; ticket counters select the block that runs the
// epilogue of each batch index (d, coef, per-class error, jac) and the one
// that sums the loss.  Every call leaves counters and sums zero for the next.
//
// Backward (one launch): recompute the activation and the bins from the
// logits with the same device functions (identical bits), gather coef (and d
// for soft binning) from LDS, form dL/dp with g = jac * grad_output and apply
// the activation's Jacobian across channels in registers; write dx once.
//
// Reference semantics: hard/soft statistics src/ace_kernels/binning.py:54-116,
// soft assignment common.py:43-61, epilogue kernels/epilogue.py:23-82,
// backward impls/v2_autograd.py:88-118 and kernels/{hard,soft}_bwd.py.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_ext.h>
#include <stdint.h>

#include "ace_bins.hpp"
#include "ace_geometry.hpp"

namespace ace {

enum { kActNone = 0, kActSoftmax = 1, kActSigmoid = 2 };
enum { kRedMean = 0, kRedSum = 1, kRedNone = 2 };
enum { kTgtLabels = 0, kTgtOnehot = 1 };

// Packed hard-binning histogram word: count | label count | sum p.
//   bits [53, 64): voxels in the bin (<= 2047 per copy and block)
//   bits [42, 53): voxels of the bin whose label is this channel
//   bits [ 0, 42): sum of p in 30-bit fixed point (|sum| < 2^11)
constexpr int kShiftN = 53;
constexpr int kShiftG = 42;
// Soft moments' packed word: count | labelled count | sum u, with
// u < 2^24 per voxel (moment_scale), so 40 bits hold the sum of
// kMaxMomCopyCount voxels and the counts take 12 bits each.
//   bits [52, 64): voxels in the half-bin (<= 4095 per copy and block)
//   bits [40, 52): of them, voxels labelled with this channel
//   bits [ 0, 40): sum of u
constexpr int kMomShiftN = 52;
constexpr int kMomShiftG = 40;

struct FwdParams {
  const void* x;
  const void* tgt;
  int64_t N;
  int64_t tile_vox;
  int64_t tiles;
  int64_t gs;
  int64_t gpb;
  int B, C, off, K, act, tk, copies, vec_ok, ignore_empty, red;
  int reps;            // replicas of each batch index's final sums
  int lchunk;          // log2 of the copies one lane adds before unpacking
  int epi_all;         // one block runs every batch index's epilogue and the loss
  float empty_w;
  int packed;          // hard binning with labels: final sums W << 32 | G, then P
  int max_polls;       // bound of the loss block's wait for a partial word (kMaxPolls)
  int publish_delay;   // test knob: sleeps before a batch epilogue publishes its word (0)
  // fast hard kernels (softmax + class labels, fast_bin): with n = K bins, a
  // probability p is held as q = trunc(p n 2^qs), its bin as q >> qs (q
  // clamped to [qlo, qhi]), and it is "near" an edge when the clamped q lies
  // within qmq of a multiple of 2^qs (ace_bins.hpp: FastBinConsts)
  float qscale;        // n 2^qs
  uint32_t qlo, qhi;   // 2^(qs-1) and (2n - 1) 2^(qs-1): t = p n clamped to [1/2, n - 1/2]
  uint32_t qmq;        // the edge margin in units of 2^-qs of t
  uint32_t qmask;      // 2^qs - 1
  int qs;
  double pscale;       // value of one unit of the hard sums of p (fast: 1 / (K 2^qs), else 2^-30)
  float sfx;           // generic soft sums: fixed-point scale 2^f (soft_frac)
  double sscale;       // 2^-f
  float msc;           // soft moments: 2^m, the fixed-point scale of p (moment_scale)
  float misc;          // 2^-m
  int mw;              // soft moments: half-bin h has base h mw (in units of 2^-m)
  int mshift;          // soft moments: right shift of the per-copy sums of u^2
  const float* btab;   // bucket table (K or 2K upper boundaries)
  const float* rtab;   // soft centre table (2K + 2)
  const float* clsw;   // C' class weights or null
  unsigned long long* fin;  // [B][reps][3][CK] zeroed final sums (reset by the epilogues)
  int* ctr;            // zeroed ticket counters, kCtrStride ints apart:
                       // [B * gpb] groups, [B] batch indices, [1] loss
  unsigned long long* part;  // [B] zeroed loss partial words: 1 << 32 | float bits
  float* coef;
  float* d;
  float* jac;
  float* f;
  float* loss;
  double* stats;
  // timeline (ace_set_timeline; null otherwise): per block, 8 stamps of the
  // 100 MHz clock (s_memrealtime) at the phases of fast_stamp
  unsigned long long* tl;
};

// Phases a fast forward block stamps into FwdParams::tl (thread 0, vector
// stores): start, main loop done, block sums and their final-sum atomics
// done, ticket drawn, and in an epilogue block its float64 terms (soft
// moments), its bins, its end and the loss.
enum { kTlStart = 0, kTlLoop, kTlSums, kTlTicket, kTlEpiEnd, kTlLoss, kTlEpiTerms, kTlEpiBins };
__device__ __forceinline__ void fast_stamp(const FwdParams& P, int phase) {
  if (P.tl && threadIdx.x == 0)
    P.tl[(size_t)blockIdx.x * 8 + phase] = __builtin_amdgcn_s_memrealtime();
}

// Soft moments fixed point in the main loop: p scaled by sc = 2^m (isc =
// 2^-m); nw = -w (the half-bin base is h w).
struct MomentScaleArgs {
  float sc;
  float isc;
  int nw;
};

struct BwdParams {
  const void* x;
  const void* tgt;
  void* dx;
  int64_t N;
  int64_t tile_vox;
  int64_t tiles;
  int B, C, off, K, act, tk, vec_ok, go_per_class;
  const float* btab;
  const float* rtab;
  const float* coef;
  const float* d;
  const float* jac;
  const float* go;
  int stream;          // streaming (nontemporal) gradient stores: stream_problem
};

// ------------------------------------------------------------ conversions

template <typename T> __device__ __forceinline__ float to_f32(T v);
template <> __device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ float to_f32<__hip_bfloat16>(__hip_bfloat16 v) {
  return __bfloat162float(v);
}
template <> __device__ __forceinline__ float to_f32<__half>(__half v) { return __half2float(v); }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ __hip_bfloat16 from_f32<__hip_bfloat16>(float v) {
  return __float2bfloat16(v);  // round to nearest even
}
template <> __device__ __forceinline__ __half from_f32<__half>(float v) {
  return __float2half(v);  // round to nearest even
}

template <int BYTES> struct RawVec;
template <> struct RawVec<16> { using type = uint4; };
template <> struct RawVec<8> { using type = uint2; };
template <> struct RawVec<4> { using type = unsigned int; };
template <> struct RawVec<2> { using type = unsigned short; };

// The same widths as clang vector types, which the nontemporal store builtin
// takes (global_store with the nt bit).
typedef unsigned int xu32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int xu32x2 __attribute__((ext_vector_type(2)));
template <int BYTES> struct XVec { using type = typename RawVec<BYTES>::type; };
template <> struct XVec<16> { using type = xu32x4; };
template <> struct XVec<8> { using type = xu32x2; };
// VEC consecutive elements from an address aligned to VEC * sizeof(T).
template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, float (&out)[VEC]) {
  using R = typename RawVec<sizeof(T) * VEC>::type;
  const R raw = *reinterpret_cast<const R*>(p);
  T vals[VEC];
  __builtin_memcpy(vals, &raw, sizeof(R));
#pragma unroll
  for (int j = 0; j < VEC; ++j) out[j] = to_f32<T>(vals[j]);
}

template <typename T, int VEC>
__device__ __forceinline__ void store_vec(T* __restrict__ p, const float (&in)[VEC]) {
  using R = typename RawVec<sizeof(T) * VEC>::type;
  T vals[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) vals[j] = from_f32<T>(in[j]);
  R raw;
  __builtin_memcpy(&raw, vals, sizeof(R));
  *reinterpret_cast<R*>(p) = raw;
}

// store_vec with a nontemporal store (streamed past the caches).
template <typename T, int VEC>
__device__ __forceinline__ void store_vec_nt(T* __restrict__ p, const float (&in)[VEC]) {
  using R = typename XVec<sizeof(T) * VEC>::type;
  T vals[VEC];
#pragma unroll
  for (int j = 0; j < VEC; ++j) vals[j] = from_f32<T>(in[j]);
  R raw;
  __builtin_memcpy(&raw, vals, sizeof(R));
  __builtin_nontemporal_store(raw, reinterpret_cast<R*>(p));
}
// A gradient store: nontemporal for streaming problems (stream_problem).
template <typename T, int VEC, bool NT>
__device__ __forceinline__ void store_dx(T* __restrict__ p, const float (&in)[VEC]) {
  if constexpr (NT)
    store_vec_nt<T, VEC>(p, in);
  else
    store_vec<T, VEC>(p, in);
}

// Class index of an int64 label if it names a channel in [0, C), else -1.
__device__ __forceinline__ int label_channel(long long v, int C) {
  return (v >= 0 && v < (long long)C) ? (int)v : -1;
}

// VEC labels from an address aligned to 16 bytes (VEC even) or one label.
template <int VEC>
__device__ __forceinline__ void load_labels(const long long* __restrict__ p, int C,
                                            int (&lab)[VEC]) {
  if constexpr (VEC % 2 == 0) {
#pragma unroll
    for (int j = 0; j < VEC; j += 2) {
      const longlong2 t = *reinterpret_cast<const longlong2*>(p + j);
      lab[j] = label_channel(t.x, C);
      lab[j + 1] = label_channel(t.y, C);
    }
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) lab[j] = label_channel(p[j], C);
  }
}

// VEC consecutive elements, vector load when VEC > 1 (caller guarantees
// alignment) or one element.
template <typename T, int VEC>
__device__ __forceinline__ void load_row(const T* __restrict__ p, float (&out)[VEC]) {
  if constexpr (VEC > 1) {
    load_vec<T, VEC>(p, out);
  } else {
    out[0] = to_f32<T>(p[0]);
  }
}

// ------------------------------------------------------------ division

// Correctly rounded a / b with the reciprocal y = rcp_rn(b) shared by every
// numerator over b: y is v_rcp_f32 refined by one Newton step, which equals the
// IEEE quotient 1 / b for every float b in [2^-20, 2^20) (checked exhaustively
// on MI355X).  Given y = RN(1 / b) and q = RN(a y) within an ulp of a / b, the
// residual r = a - b q is exact and RN(q + r y) is the IEEE quotient
// (Markstein's theorem) as long as r does not underflow: checked against '/'
// for every float b in [2^-20, 2^14) with a of every exponent, no mismatch
// where a and a / b are >= 2^-100.  Below that (softmax terms e^-69 and
// smaller) the quotient may be an ulp off, far below any bin edge or
// tolerance.  Used where b is a softmax sum in [1, C] or a soft-bin span in
// [2^-20, 2^14]: three instructions per quotient.
__device__ __forceinline__ float rcp_rn(float b) {
  const float y = __builtin_amdgcn_rcpf(b);
  const float e = fmaf(-b, y, 1.0f);
  return fmaf(e, y, y);
}
// div_rn(a, b, y): ace_bins.hpp (shared with the CPU test harness).

// a * b + c with 24-bit signed a, b (v_mad_i32_i24; the compiler would
// otherwise sign-extend a it cannot bound first).
__device__ __forceinline__ uint32_t mad_i24(int a, int b, uint32_t c) {
  uint32_t r;
  asm("v_mad_i32_i24 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// u^2 for u < 2^24 as two 24-bit multiplies (low 32 and high 16 bits).
__device__ __forceinline__ unsigned long long square_u24(uint32_t u) {
  uint32_t lo, hi;
  asm("v_mul_u32_u24 %0, %1, %1" : "=v"(lo) : "v"(u));
  asm("v_mul_hi_u32_u24 %0, %1, %1" : "=v"(hi) : "v"(u));
  return ((unsigned long long)hi << 32) | lo;
}

// A probability already scaled by 2^m (p in [0, 2^m] or NaN; m = 30 for
// hard binning, the soft moments' scale otherwise) as m-bit fixed point,
// truncated: v_cvt_u32_f32 rounds toward zero and maps NaN to 0.  At most
// 2^-m below p.
__device__ __forceinline__ uint32_t cvt_u32(float p30) {
  uint32_t q;
  asm("v_cvt_u32_f32 %0, %1" : "=v"(q) : "v"(p30));
  return q;
}

// ------------------------------------------------------------ activation

// exp(x) for the softmax arguments x = logit - max <= 0: 2^(x log2 e) with
// e = rint(x log2 e) split off and the reduced argument a = x log2 e - e
// formed with one fma (exact product, one rounding: |a| <= 1/2, so its
// rounding error is ~2^-26) plus x times the remainder of log2 e
// (log2 e = L + Llo, L its float rounding).  v_exp_f32 then sees a in
// [-1/2, 1/2].  The rounding to an integer is t = fma(x, L, 1.5 2^23): t is
// 1.5 2^23 + e exactly (|x L| < 2^22), e = t - 1.5 2^23, and since the low 9
// bits of 1.5 2^23 are zero, (bits(t) << 23) mod 2^32 = e << 23, which one
// integer add puts into the exponent of v_exp_f32's result (instead of
// rint + cvt + ldexp: one instruction fewer).  That add needs a normal
// result: x is clamped at -87 (exp(-87) = 1.6e-38, e >= -126), which also
// keeps -inf logits finite (x <= 0 cannot overflow); below it the
// probability is ~1e-38 either way, bin 0 and 0 in fixed point.  Measured
// on MI355X against a float64 exp for every float x in [-87, 0]: max error
// 0.968 ulp, no result off by more than 1 ulp (ROCm's expf: 0.857 / none;
// its range reduction splits x log2 e into two terms first, two
// instructions more).
__device__ __forceinline__ float exp_neg(float x) {
  x = fmaxf(x, -87.0f);
  const float t = fmaf(x, 0x1.715476p+0f, 0x1.8p23f);
  const float e = t - 0x1.8p23f;
  float a = fmaf(x, 0x1.715476p+0f, -e);
  a = fmaf(x, 0x1.4ae0bep-26f, a);
  const float v = __builtin_amdgcn_exp2f(a);
  return __uint_as_float(__float_as_uint(v) + (__float_as_uint(t) << 23));
}

// In place: logits -> probabilities.  Softmax follows torch.softmax: max over
// channels, e_c = exp(x_c - max), s = sequential sum over c, p_c = e_c / s
// (IEEE quotient), with exp_neg.  Sigmoid: 1 / (1 + exp(-x)).
template <int CMAX, bool EXACT>
__device__ __forceinline__ void activate(float (&x)[CMAX], int nc, int act) {
  if (act == kActSoftmax) {
    float m = x[0];
#pragma unroll
    for (int c = 1; c < CMAX; ++c)
      if (EXACT || c < nc) m = fmaxf(m, x[c]);
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) {
        x[c] = exp_neg(x[c] - m);
        s += x[c];
      }
    const float y = rcp_rn(s);
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) x[c] = div_rn(x[c], s, y);
  } else if (act == kActSigmoid) {
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) x[c] = 1.0f / (1.0f + expf(-x[c]));
  }
}

// ------------------------------------------------------------ binning

struct SoftW {
  int l, r;
  float lw, rw, span, inv_span;
};

// Soft assignment of common.py:43-61: half-bin index h against the 2K upper
// half boundaries; bins l = max(h-1,0)/2, r = min(h+1,2K-1)/2; distances to
// the replicated centres (sentinels +-1e4); lw = rd/S, rw = ld/S and 1/S, all
// IEEE quotients (one shared reciprocal of S).
template <bool RIGHT>
__device__ __forceinline__ SoftW soft_assign(float p, int K, float n2f, const float* htab,
                                             const float* repl) {
  const int n2 = 2 * K;
  const int h = bucket<RIGHT>(p, n2f, n2, htab);
  SoftW w;
  w.l = max(h - 1, 0) >> 1;
  w.r = min(h + 1, n2 - 1) >> 1;
  const float ld = p - repl[h];
  const float rd = repl[h + 2] - p;
  w.span = ld + rd;
  w.inv_span = rcp_rn(w.span);
  w.lw = div_rn(rd, w.span, w.inv_span);
  w.rw = div_rn(ld, w.span, w.inv_span);
  return w;
}

// The same assignment with the exact-arithmetic weights of the moments
// kernels: ld, rd and S formed in float64 from the float32 p and centres,
// lw = rd / S and rw = ld / S rounded once in float64, where the float32 form
// rounds ld, rd, S and both quotients (each ~1e-7 relative).  The generic
// soft forward sums these: the soft gradient takes d = P/W - G/W amplified
// by 2K / W, and float32 weights move d by ~1e-7 there.
struct SoftW64 {
  int l, r;
  double lw, rw;
};
template <bool RIGHT>
__device__ __forceinline__ SoftW64 soft_assign64(float p, int K, float n2f, const float* htab,
                                                 const float* repl) {
  const int n2 = 2 * K;
  const int h = bucket<RIGHT>(p, n2f, n2, htab);
  SoftW64 w;
  w.l = max(h - 1, 0) >> 1;
  w.r = min(h + 1, n2 - 1) >> 1;
  const double ld = (double)p - (double)repl[h];
  const double rd = (double)repl[h + 2] - (double)p;
  const double inv = 1.0 / (ld + rd);
  w.lw = rd * inv;
  w.rw = ld * inv;
  return w;
}

// Fixed-point value of a float32 term with |v| < 2 (2^30 scale, rounded to
// nearest even): exact for |v| >= 2^-7.
__device__ __forceinline__ long long fx(float v) {
  return (long long)(int)rintf(v * 1073741824.0f);
}
// A float64 term |v| < 2 at scale sfx = 2^f (soft_frac: up to 2^40), rounded
// to nearest even: an error of at most 2^-(f+1) per term.  x = v sfx is exact
// (a power-of-two scale) and |x| < 2^41, so x + 1.5 2^52 lies in [2^52, 2^53),
// where the float64 spacing is 1: the add rounds x to the nearest even integer
// and the difference of the bit patterns is that integer (rint and a float64
// to int64 conversion, ~8 instructions, in 3).
__device__ __forceinline__ long long fx_soft(double v, float sfx) {
  constexpr double kMagic = 0x1.8p52;
  const double t = v * (double)sfx + kMagic;
  return __double_as_longlong(t) - __double_as_longlong(kMagic);
}

__device__ __forceinline__ void lds_add(unsigned long long* p, unsigned long long v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_add(long long* p, long long v) {
  lds_add(reinterpret_cast<unsigned long long*>(p), (unsigned long long)v);
}

// Cross-block communication without cache-wide fences.  An agent-scope
// fence on gfx950 writes back and invalidates the whole L2 (buffer_wbl2 sc1 /
// buffer_inv sc1), which thousands of blocks cannot afford.  Instead every
// value another block reads is written and read with device-coherent (sc1)
// accesses -- relaxed agent-scope atomic stores/loads -- or integer atomics; a
// block waits for its own writes to complete (s_waitcnt vmcnt(0)) before it
// increments a ticket, and the block that draws the last ticket reads the data
// with sc1 loads.  No dirty L2 line holds shared data, so no write-back is
// needed, and no stale line can be read.
//
// Device-scope atomics are serialised per cache line at the memory side
// (about 10-17 ns per wave request on MI355X, measured): 1024 blocks
// incrementing one counter take ~11 us, and counters sharing a line contend
// as if they were one.  So every ticket counter has its own 256-byte line and
// takes at most a few dozen arrivals (groups of <= 16 blocks, then the groups
// of a batch index).  The final sums take one request per block and line;
// blocks finish spread over several microseconds, and up to kMaxReps replicas
// (one per kRepTiles blocks) trade that contention against the epilogue's
// loads -- 2 replicas for 512 blocks per batch index measured fastest.
__device__ __forceinline__ void store_dev(long long* p, long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long load_dev(const unsigned long long* p) {
  return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this thread's global stores and atomics have completed.
__device__ __forceinline__ void wait_own_writes() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// Polls of another block's loss partial word before the loss gives up (NaN):
// far beyond the few microseconds the other epilogues take.
constexpr int kMaxPolls = 1 << 20;
// A partial word the loss block gave up on (no flag bit 32): the late block
// then finds it instead of zero and clears it, so the workspace is left zero.
constexpr unsigned long long kAbandoned = 1ull;
__device__ __forceinline__ unsigned long long cas_dev(unsigned long long* p, unsigned long long expected,
                                                      unsigned long long desired) {
  __hip_atomic_compare_exchange_strong(p, &expected, desired, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return expected;  // the word's value before the exchange
}
__device__ __forceinline__ unsigned long long xchg_dev(unsigned long long* p, unsigned long long v) {
  return __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ticket(int* ctr) {
  return __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Copies the bucket table (padded with -inf / +inf) and the centre table into
// LDS.
__device__ __forceinline__ void load_tables(float* lds, const float* btab, const float* rtab,
                                            int n, int nrepl) {
  for (int i = threadIdx.x; i < n + 2; i += kThreads) {
    float v;
    if (i == 0) v = -__builtin_inff();
    else if (i == n + 1) v = __builtin_inff();
    else v = btab[i - 1];
    lds[i] = v;
  }
  for (int i = threadIdx.x; i < nrepl; i += kThreads) lds[n + 2 + i] = rtab[i];
}

// A thread's share of the LDS tables -- entries tid and tid + nt (the block
// size) of the padded bucket table and of the centre table -- held in registers, so
// that a kernel can issue these loads, then its first tiles' loads, and only
// then wait for the tables (in-order vmcnt, a partial wait) and write them to
// LDS.  The loads are unconditional (clamped in-bounds indices, unused values
// discarded): a load under a branch would make the compiler wait for every
// outstanding load instead.
struct TableRegs {
  float b[2], r[2];  // raw table values; padding applied when stored
  // nt: the block size (a compile-time kThreads where the kernel has one)
  __device__ __forceinline__ void load(const float* btab, const float* rtab, int n, int nrepl,
                                       int nt) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = (int)threadIdx.x + u * nt;
      b[u] = btab[min(max(i - 1, 0), n - 1)];
      r[u] = nrepl > 0 ? rtab[min(i, nrepl - 1)] : 0.0f;
    }
  }
  // bscale: a power of two the bucket table is multiplied by (exact)
  __device__ __forceinline__ void store(float* lds, const float* btab, const float* rtab, int n,
                                        int nrepl, int nt, float bscale = 1.0f) const {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = (int)threadIdx.x + u * nt;
      if (i < n + 2) lds[i] = i == 0 ? -__builtin_inff() : (i <= n ? b[u] * bscale : __builtin_inff());
      if (i < nrepl) lds[n + 2 + i] = r[u];
    }
    // tables longer than 2 x nt entries
    for (int i = (int)threadIdx.x + 2 * nt; i < n + 2; i += nt)
      lds[i] = i == n + 1 ? __builtin_inff() : btab[i - 1] * bscale;
    for (int i = (int)threadIdx.x + 2 * nt; i < nrepl; i += nt) lds[n + 2 + i] = rtab[i];
  }
};

// ------------------------------------------------------------ tiles

// One thread's slice of a step: VEC voxels of every channel, their labels or
// per-channel targets.  `load` issues the vector loads only; the values are
// first used by the binning, so a load can be in flight while another tile is
// processed.
// Whether a generic kernel streams two tiles in rotation (software
// pipelining).  At one voxel per lane with 16 or more channels it does not:
// the per-voxel arrays leave no room for a second tile.
template <int CMAX, int VEC, bool SOFT>
constexpr bool generic_pipelined() {
  return !(VEC == 1 && CMAX >= 16);
}

template <int CMAX, int VEC>
struct Tile {
  float x[CMAX][VEC];
  int lab[VEC];
  float y[CMAX][VEC];

  template <typename T, bool EXACT>
  __device__ __forceinline__ void load(const T* xt, const long long* lt, const float* yt,
                                       int64_t N, int v, int nc, int off, bool labels) {
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) load_row<T, VEC>(xt + c * N + v, x[c]);
    if (labels) {
      load_labels<VEC>(lt + v, nc, lab);
    } else {
#pragma unroll
      for (int c = 0; c < CMAX; ++c)
        if ((EXACT || c < nc) && c >= off) load_row<float, VEC>(yt + c * N + v, y[c]);
    }
  }
};

// ------------------------------------------------------------ forward

// LDS views of one block's histogram copies.
struct Hist {
  unsigned long long* a;  // hard: packed count | label count | sum p   [CK][R]
                          // moments: the same per half-bin, with the
                          // offsets u of moment_scale for p           [2CK][R]
  long long* g1;          // hard + per-channel targets: sum y          [CK][R]
  long long* w;           // soft: sum of weights                       [CK][R]
  long long* p;           // soft: sum of weight * p                    [CK][R]
  long long* g;           // soft: sum of weight * y                    [CK][R]
  unsigned long long* m2; // moments: sum u^2                           [2CK][R]
  unsigned long long* mg; // moments: sum u over the labelled voxels    [2CK][R]
};

// Adds NV voxels (logits xv, labels lab or targets yv) into the histograms.
template <int CMAX, bool EXACT, int NV, bool SOFT, bool RIGHT>
__device__ __forceinline__ void fwd_accumulate(const FwdParams& P, const Hist& H, const float* btab,
                                               const float* repl, int nc, int copy,
                                               float (&xv)[CMAX][NV], const int (&lab)[NV],
                                               const float (&yv)[CMAX][NV], bool labels) {
  const int K = P.K;
  const int off = P.off;
  const int R = P.copies;
  const float nf = (float)(SOFT ? 2 * K : K);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    float p[CMAX];
#pragma unroll
    for (int c = 0; c < CMAX; ++c) p[c] = xv[c][j];
    activate<CMAX, EXACT>(p, nc, P.act);
    if constexpr (!SOFT) {
#pragma unroll
      for (int c = 0; c < CMAX; ++c) {
        if (!(EXACT || c < nc) || c < off) continue;
        const int k = bucket<RIGHT>(p[c], nf, K, btab);
        const int slot = ((c - off) * K + k) * R + copy;
        const unsigned long long hit = (labels && lab[j] == c) ? (1ull << kShiftG) : 0ull;
        lds_add(&H.a[slot], (1ull << kShiftN) + hit + (unsigned long long)fx(p[c]));
        if (!labels) {
          const float y = yv[c][j];
          if (y != 0.0f) lds_add(&H.g1[slot], fx(y));
        }
      }
    } else {
      int gl = 0, gr = 0;
      double glw = 0.0, grw = 0.0;
#pragma unroll
      for (int c = 0; c < CMAX; ++c) {
        if (!(EXACT || c < nc) || c < off) continue;
        const SoftW64 w = soft_assign64<RIGHT>(p[c], K, nf, btab, repl);
        const int sl = ((c - off) * K + w.l) * R + copy;
        const int sr = ((c - off) * K + w.r) * R + copy;
        lds_add(&H.w[sl], fx_soft(w.lw, P.sfx));
        lds_add(&H.w[sr], fx_soft(w.rw, P.sfx));
        lds_add(&H.p[sl], fx_soft(w.lw * (double)p[c], P.sfx));
        lds_add(&H.p[sr], fx_soft(w.rw * (double)p[c], P.sfx));
        if (labels) {
          const bool hit = lab[j] == c;
          gl = hit ? sl : gl;
          gr = hit ? sr : gr;
          glw = hit ? w.lw : glw;
          grw = hit ? w.rw : grw;
        } else {
          const float y = yv[c][j];
          if (y != 0.0f) {
            lds_add(&H.g[sl], fx_soft(w.lw * (double)y, P.sfx));
            lds_add(&H.g[sr], fx_soft(w.rw * (double)y, P.sfx));
          }
        }
      }
      if (labels && lab[j] >= off) {
        lds_add(&H.g[gl], fx_soft(glw, P.sfx));
        lds_add(&H.g[gr], fx_soft(grw, P.sfx));
      }
    }
  }
}

// Sum of v over the 64 lanes of a wave (every lane active), returned in every
// lane: DPP row shifts by 1, 2, 4 and 8 leave each row's 16-lane total in its
// lane 15, then the four row totals are read and added in row order -- a fixed
// order, so the result is bit-identical run to run.  No LDS round trips (a
// ds_bpermute butterfly costs six of them).
template <int N>
__device__ __forceinline__ int row_shr(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x110 + N, 0xf, 0xf, true);
}
__device__ __forceinline__ float wave_sum(float v) {
  v += __int_as_float(row_shr<1>(__float_as_int(v)));
  v += __int_as_float(row_shr<2>(__float_as_int(v)));
  v += __int_as_float(row_shr<4>(__float_as_int(v)));
  v += __int_as_float(row_shr<8>(__float_as_int(v)));
  const int b = __float_as_int(v);
  return ((__int_as_float(__builtin_amdgcn_readlane(b, 15)) +
           __int_as_float(__builtin_amdgcn_readlane(b, 31))) +
          __int_as_float(__builtin_amdgcn_readlane(b, 47))) +
         __int_as_float(__builtin_amdgcn_readlane(b, 63));
}
// Sum over the seg lanes (16, 32 or 64) of segment `sub` of a wave, every
// lane active: the DPP row totals of wave_sum, added per segment in row
// order (seg 64: exactly wave_sum's order).
__device__ __forceinline__ float seg_sum(float v, int sub, int seg) {
  v += __int_as_float(row_shr<1>(__float_as_int(v)));
  v += __int_as_float(row_shr<2>(__float_as_int(v)));
  v += __int_as_float(row_shr<4>(__float_as_int(v)));
  v += __int_as_float(row_shr<8>(__float_as_int(v)));
  const int b = __float_as_int(v);
  const float t0 = __int_as_float(__builtin_amdgcn_readlane(b, 15));
  const float t1 = __int_as_float(__builtin_amdgcn_readlane(b, 31));
  const float t2 = __int_as_float(__builtin_amdgcn_readlane(b, 47));
  const float t3 = __int_as_float(__builtin_amdgcn_readlane(b, 63));
  if (seg == 64) return ((t0 + t1) + t2) + t3;
  if (seg == 32) return sub == 0 ? t0 + t1 : t2 + t3;
  return sub == 0 ? t0 : (sub == 1 ? t1 : (sub == 2 ? t2 : t3));
}
__device__ __forceinline__ int wave_sum(int v) {
  v += row_shr<1>(v);
  v += row_shr<2>(v);
  v += row_shr<4>(v);
  v += row_shr<8>(v);
  return __builtin_amdgcn_readlane(v, 15) + __builtin_amdgcn_readlane(v, 31) +
         __builtin_amdgcn_readlane(v, 47) + __builtin_amdgcn_readlane(v, 63);
}

// Ticket counter i of the workspace (counters are kCtrStride ints apart).
__device__ __forceinline__ int* counter(const FwdParams& P, int64_t i) {
  return P.ctr + i * kCtrStride;
}

// Epilogue of batch index b (kernels/epilogue.py:23-82): final sums -> d, W,
// G per bin; per class row: K_ne, f, coef, jac.  Runs in the block that drew
// the last ticket of batch b; it also leaves b's final sums zero.
// Soft moments: the bin sums of half-bin h (interval of half boundaries
// between the replicated centres cl = repl[h] and cr = repl[h + 2]) follow
// from its moments, because both interpolation weights are linear in p there:
// lw = (cr - p) / S, rw = (p - cl) / S with S = cr - cl (common.py:43-61).
// The kernels store each p of half-bin h as L + v, L its base and v its
// offset (moment_scale: p quantised to 2^-m, v = u 2^-m), so with
// a = cr - L, b = L - cl (a + b = S), V1 = sum v, V2 = sum v^2, Vg = sum v
// over the labelled voxels, n = count and g = labelled count:
//   W_l += (n a - V1) / S,               W_r += (n b + V1) / S,
//   P_l += (n a L + (a - L) V1 - V2) / S, P_r += (n b L + (b + L) V1 + V2) / S,
//   G_l += (g a - Vg) / S,               G_r += (g b + Vg) / S;
// bins l = max(h-1,0)/2, r = min(h+1,2K-1)/2.  The sums are exact for the
// quantised p, and W, P and G describe the same values, so d = P/W - G/W
// keeps its precision in bins of one or two voxels with small weights
// (P_l cancels to p (cr - p) there).  The weights are the exact-arithmetic
// ones (the reference rounds ld, rd and S to float32 per voxel: a ~1e-7
// relative difference per voxel).
__device__ __forceinline__ void moment_terms(double n, double g, double v1, double v2, double vg,
                                             double L, double cl, double cr, double* out) {
  const double inv = 1.0 / (cr - cl);
  const double a = cr - L;
  const double b = L - cl;
  out[0] = (n * a - v1) * inv;
  out[1] = (n * b + v1) * inv;
  out[2] = (n * a * L + (a - L) * v1 - v2) * inv;
  out[3] = (n * b * L + (b + L) * v1 + v2) * inv;
  out[4] = (g * a - vg) * inv;
  out[5] = (g * b + vg) * inv;
}

// Sums over the `reps` replicas of NVAL final-sum words of one item (word j
// at fb + r * NV + j * stride + idx).  Every load is unconditional -- the
// replica index is clamped to reps - 1 and the extra replicas are dropped
// after loading -- so all of them are in flight at once and a caller can
// issue a second item's loads before it waits for the first's.
template <int NVAL>
__device__ __forceinline__ void load_sums(const unsigned long long* fb, int NV, int reps, int stride,
                                          int idx, long long (&out)[NVAL]) {
  unsigned long long v[kMaxReps][NVAL];
#pragma unroll
  for (int r = 0; r < kMaxReps; ++r) {
    const int rr = r < reps ? r : reps - 1;
#pragma unroll
    for (int j = 0; j < NVAL; ++j) v[r][j] = load_dev(fb + (int64_t)rr * NV + j * stride + idx);
  }
#pragma unroll
  for (int j = 0; j < NVAL; ++j) {
    long long acc = 0;
#pragma unroll
    for (int r = 0; r < kMaxReps; ++r)
      if (r < reps) acc += (long long)v[r][j];
    out[j] = acc;
  }
}
template <int NVAL>
__device__ __forceinline__ void zero_sums(unsigned long long* fb, int NV, int reps, int stride, int idx) {
  for (int r = 0; r < reps; ++r)
#pragma unroll
    for (int j = 0; j < NVAL; ++j) store_dev(fb + (int64_t)r * NV + j * stride + idx, 0ull);
}

// Epilogue of batch indices [b0, b0 + nb) in one block.  Final sums -> W, P,
// G per bin, d = P/W - G/W (kernels/epilogue.py:23-82); per class row: K_ne,
// f, coef, jac (one wave per row).  It leaves its final sums zero and returns
// (in wave 0, unless the reduction is "none") the sum of its rows'
// per-class errors, in wave_sum's fixed order.
template <bool SOFT, bool MOM>
__device__ __forceinline__ float epilogue(const FwdParams& P, unsigned char* hist,
                                          const float* repl, int CK, int CL, int b0, int nb) {
  const int tid = threadIdx.x;
  const int K = P.K;
  const int NV = fin_values(CK, MOM, P.packed != 0);
  const int reps = P.reps;
  const EpiLayout L = epi_layout(CK, CL, nb, MOM);
  const int NB = nb * CK;  // bins of this epilogue
  float* sd = reinterpret_cast<float*>(hist);
  float* sw = sd + NB;
  float* sg = sw + NB;
  unsigned char* se = reinterpret_cast<unsigned char*>(sg + NB);
  float* sf = reinterpret_cast<float*>(hist + L.sf);        // [nb * CL]
  double* terms = reinterpret_cast<double*>(hist + L.terms);  // [nb * 2CK][6]
  const int64_t BCK = (int64_t)P.B * CK;
  const double dscale = 1.0 / 1073741824.0;  // W and G of the unpacked sums
  const double pscale = P.pscale;             // the sums of p (hard)
  if constexpr (MOM) {
    // per half-bin: the five moments (every replica in flight at once), then
    // its six contributions
    const int H2 = 2 * CK;
    for (int t = tid; t < nb * H2; t += kThreads) {
      const int bb = nb == 1 ? 0 : t / H2;
      const int th = t - bb * H2;
      unsigned long long* fb = P.fin + (int64_t)(b0 + bb) * reps * NV;
      long long m[5];
      load_sums<5>(fb, NV, reps, H2, th, m);  // every replica's loads in flight at once
      zero_sums<5>(fb, NV, reps, H2, th);
      const int hh = th % (2 * K);
      const double mscale = (double)P.misc;
      const double L = (double)((long long)hh * P.mw) * mscale;
      moment_terms((double)m[0], (double)m[1], (double)m[2] * mscale,
                   (double)m[3] * (mscale * mscale * (double)(1ll << P.mshift)),
                   (double)m[4] * mscale, L, (double)repl[hh], (double)repl[hh + 2], terms + 6 * t);
    }
    __syncthreads();
    fast_stamp(P, kTlEpiTerms);
  }
  // per bin: W, P, G (final sums, or the half-bin terms of soft moments),
  // then d; without moments two bins per thread and pass, both bins' loads
  // in flight together
  auto fb_of = [&](int i) { return P.fin + (int64_t)(b0 + (nb == 1 ? 0 : i / CK)) * reps * NV; };
  auto bin = [&](int i, const long long (&sm)[3]) {
    const int bb = nb == 1 ? 0 : i / CK;
    const int t = i - bb * CK;
    double Wd, Pd, Gd;
    if constexpr (MOM) {
      // bin k of channel row cl: left share of half-bins l(h) = k, right share
      // of r(h) = k, h in [2k - 1, 2k + 2], in increasing h
      const int cl = t / K;
      const int k = t - cl * K;
      const double* tb = terms + 6 * ((size_t)bb * 2 * CK + (size_t)cl * 2 * K);
      Wd = Pd = Gd = 0.0;
      for (int hh = max(2 * k - 1, 0); hh <= min(2 * k + 2, 2 * K - 1); ++hh) {
        if ((max(hh - 1, 0) >> 1) == k) {
          Wd += tb[6 * hh];
          Pd += tb[6 * hh + 2];
          Gd += tb[6 * hh + 4];
        }
        if ((min(hh + 1, 2 * K - 1) >> 1) == k) {
          Wd += tb[6 * hh + 1];
          Pd += tb[6 * hh + 3];
          Gd += tb[6 * hh + 5];
        }
      }
    } else if (P.packed) {
      // W << 32 | G (unsigned: W may reach 2^31), then the sum of p
      zero_sums<2>(fb_of(i), NV, reps, CK, t);
      const unsigned long long wg = (unsigned long long)sm[0];
      Wd = (double)(wg >> 32);
      Gd = (double)(wg & 0xffffffffull);
      Pd = (double)sm[1] * pscale;
    } else {
      zero_sums<3>(fb_of(i), NV, reps, CK, t);
      // generic soft sums at 2^f (soft_frac), hard ones at 2^30
      const double ws = SOFT ? P.sscale : dscale;
      Wd = (double)sm[0] * ws;
      Pd = (double)sm[1] * (SOFT ? P.sscale : pscale);
      Gd = (double)sm[2] * ws;
    }
    const int64_t o = (int64_t)(b0 + bb) * CK + t;
    if (P.stats) {
      P.stats[o] = Wd;
      P.stats[BCK + o] = Pd;
      P.stats[2 * BCK + o] = Gd;
    }
    const float Wf = (float)Wd;
    const float Pf = (float)Pd;
    const float Gf = (float)Gd;
    const bool empty = SOFT ? !(Wf >= P.empty_w) : (Wf == 0.0f);
    // d = P/W - G/W (binning.py:136-141).  Hard: the reference's float32
    // order, two quotients rounded to float32, then their difference.  Soft:
    // (P - G) / W from the float64 sums, stored as its float32 rounding and
    // the remainder (diff[0] and diff[1]).  The soft gradient takes d
    // amplified by 2K / W through (p - y - d) / S, where a float32 d (a few
    // 1e-8 off wherever P/W and G/W nearly cancel) moves dL/dp by ~1e-7; the
    // backward adds both parts, so p - y - d keeps the precision of the sums,
    // and in a bin of one voxel (d = p - y exactly) it cancels to 0.  The loss
    // and sign(d) take the rounded value.
    float dd = 0.0f, dlo = 0.0f;
    if (!empty) {
      if constexpr (SOFT) {
        const double dx = (Pd - Gd) / Wd;
        dd = (float)dx;
        dlo = (float)(dx - (double)dd);
      } else {
        dd = Pf / Wf - Gf / Wf;
      }
    }
    sd[i] = dd;
    sw[i] = Wf;
    sg[i] = Gf;
    se[i] = empty ? 1 : 0;
    P.d[o] = dd;
    if constexpr (SOFT) P.d[BCK + o] = dlo;
  };
  if constexpr (MOM) {
    const long long none[3] = {0, 0, 0};
    for (int i = tid; i < NB; i += kThreads) bin(i, none);
  } else {
    for (int i0 = tid; i0 < NB; i0 += 2 * kThreads) {
      const int i1 = i0 + kThreads < NB ? i0 + kThreads : i0;
      long long s0[3] = {0, 0, 0}, s1[3] = {0, 0, 0};
      if (P.packed) {
        long long a0[2], a1[2];
        load_sums<2>(fb_of(i0), NV, reps, CK, i0 - (nb == 1 ? 0 : i0 / CK) * CK, a0);
        load_sums<2>(fb_of(i1), NV, reps, CK, i1 - (nb == 1 ? 0 : i1 / CK) * CK, a1);
        s0[0] = a0[0]; s0[1] = a0[1];
        s1[0] = a1[0]; s1[1] = a1[1];
      } else {
        load_sums<3>(fb_of(i0), NV, reps, CK, i0 - (nb == 1 ? 0 : i0 / CK) * CK, s0);
        load_sums<3>(fb_of(i1), NV, reps, CK, i1 - (nb == 1 ? 0 : i1 / CK) * CK, s1);
      }
      bin(i0, s0);
      if (i1 != i0) bin(i1, s1);
    }
  }
  __syncthreads();
  fast_stamp(P, kTlEpiBins);
  // class rows: K <= 64 bins per row take one lane each, 64 / seg rows per
  // wave (seg = 16, 32 or 64 lanes per row); longer rows loop over a wave
  const int lane = tid & 63;
  const int rows = P.B * CL;
  const int nrows = nb * CL;
  auto row_tail = [&](int row, float fcls, float present) {
    const int bb = nb == 1 ? 0 : row / CL;
    const int cl = row - bb * CL;
    const float w = P.clsw ? P.clsw[cl] : 1.0f;
    float fw = P.ignore_empty ? fcls * present : fcls;
    fw = fw * w;
    float jac = P.ignore_empty ? present * w : w;
    if (P.red == kRedMean) jac = jac / (float)rows;
    const int gi = (b0 + bb) * CL + cl;
    P.f[gi] = fw;
    sf[row] = fw;
    P.jac[gi] = jac;
  };
  if (K <= 64) {
    const int seg = K <= 16 ? 16 : (K <= 32 ? 32 : 64);
    const int per_wave = 64 / seg;
    const int sub = lane / seg;
    const int kl = lane & (seg - 1);
    const unsigned long long smask = (seg == 64 ? ~0ull : ((1ull << seg) - 1)) << (sub * seg);
    for (int r0 = (tid >> 6) * per_wave; r0 < nrows; r0 += (kThreads / 64) * per_wave) {
      const int row = r0 + sub;
      const bool rv = row < nrows;
      const bool in = rv && kl < K;
      const int rr = rv ? row : r0;  // an in-range row for idle lanes
      // one bin per lane: every LDS value read once, in one round trip
      const int i = rr * K + (in ? kl : 0);
      const float dd = sd[i];
      const float wv = sw[i];
      const float gv = sg[i];
      const bool emp = se[i] != 0;
      const bool ne = in && !emp;
      const int kne = __popcll(__ballot(ne) & smask);
      const float err = seg_sum(ne ? fabsf(dd) : 0.0f, sub, seg);
      const float gsum = seg_sum(in ? gv : 0.0f, sub, seg);
      // the row's serial tail: v_rcp_f32 (1 ulp) instead of IEEE quotients
      // for f = mean |d| and coef = sign(d) / (K_ne W), far inside the loss
      // and gradient tolerances
      const float fcls = kne > 0 ? err * __builtin_amdgcn_rcpf((float)kne) : __builtin_nanf("");
      const float present = gsum > 0.0f ? 1.0f : 0.0f;
      const float kf = (float)(kne > 0 ? kne : 1);
      if (in) {
        const int bb = nb == 1 ? 0 : rr / CL;
        const int cl = rr - bb * CL;
        const int64_t ob = (int64_t)(b0 + bb) * CK + cl * K;
        const float sgn = dd > 0.0f ? 1.0f : (dd < 0.0f ? -1.0f : 0.0f);
        P.coef[ob + kl] = emp ? 0.0f : sgn * __builtin_amdgcn_rcpf(kf * wv);
      }
      if (rv && kl == 0) row_tail(row, fcls, present);
    }
  } else {
    for (int row = tid >> 6; row < nrows; row += kThreads / 64) {
      const int base = row * K;  // == bb * CK + cl * K
      const int bb = nb == 1 ? 0 : row / CL;
      const int cl = row - bb * CL;
      const int64_t ob = (int64_t)(b0 + bb) * CK + cl * K;
      int kne = 0;
      float err = 0.0f, gsum = 0.0f;
      for (int k = lane; k < K; k += 64) {
        if (!se[base + k]) {
          ++kne;
          err += fabsf(sd[base + k]);
        }
        gsum += sg[base + k];
      }
      kne = wave_sum(kne);
      err = wave_sum(err);
      gsum = wave_sum(gsum);
      const float fcls = kne > 0 ? err / (float)kne : __builtin_nanf("");
      const float present = gsum > 0.0f ? 1.0f : 0.0f;
      const float kf = (float)(kne > 0 ? kne : 1);
      for (int k = lane; k < K; k += 64) {
        const float dd = sd[base + k];
        const float sgn = dd > 0.0f ? 1.0f : (dd < 0.0f ? -1.0f : 0.0f);
        P.coef[ob + k] = se[base + k] ? 0.0f : sgn / (kf * sw[base + k]);
      }
      if (lane == 0) row_tail(row, fcls, present);
    }
  }
  // the rows' errors summed by wave 0 (every lane active): lane-strided, then
  // wave_sum's fixed order, so the loss is bit-identical run to run (one LDS
  // read and a DPP reduction instead of one dependent read per row)
  float total = 0.0f;
  if (P.red != kRedNone) {
    __syncthreads();
    if (tid < 64) {
      float v = 0.0f;
      for (int r = tid; r < nb * CL; r += 64) v += sf[r];
      total = wave_sum(v);
    }
  }
  return total;
}

// Block sums: one lane per bin (half-bin for moments) loads the R copies of
// that bin, adds them -- packed words `chunk` at a time, decoded after each
// chunk (the geometry keeps chunk x per-copy counts within the 11-bit fields)
// -- and issues the atomics into `fin`, so one wave request covers 64
// consecutive final sums and no lanes combine.  R is a template argument so
// that the loads are unconditional and issue back to back; the copy index is
// skewed by the bin so that the lanes of a wave read distinct bank pairs.

// Adds the decoded fields of a sum of packed words (count | label count |
// sum p): counts unscaled, sum p signed (probabilities outside [0, 1] without
// an activation) -- the upper fields are rounded so that it decodes in
// [-2^41, 2^41).
template <int SN = kShiftN, int SG = kShiftG>
__device__ __forceinline__ void decode_packed(unsigned long long a, long long& n, long long& g,
                                              long long& sp) {
  const unsigned long long hi = (a + (1ull << (SG - 1))) >> SG;
  n += (long long)(hi >> (SN - SG));
  g += (long long)(hi & ((1ull << (SN - SG)) - 1));
  sp += (long long)(a - (hi << SG));
}

// Copies one lane loads before adding them: bounds the registers the block
// sums hold (the kernel's register count is that of its widest phase).
constexpr int kSumBatch = 8;

// Sum of the R packed copies starting at w0 (skew s), decoded every `chunk`;
// MOM: the soft moments' layout (kMomShiftN, kMomShiftG).
template <int R, int BATCH = kSumBatch, bool MOM = false>
__device__ __forceinline__ void sum_packed(const unsigned long long* a, int w0, int s, int chunk,
                                           long long& n, long long& g, long long& sp) {
  constexpr int NB = R < BATCH ? R : BATCH;
  unsigned long long acc = 0;
#pragma unroll 1
  for (int r0 = 0; r0 < R; r0 += NB) {
    unsigned long long v[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) v[j] = a[w0 + ((r0 + j + s) & (R - 1))];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      acc += v[j];
      if (((r0 + j + 1) & (chunk - 1)) == 0) {
        if constexpr (MOM)
          decode_packed<kMomShiftN, kMomShiftG>(acc, n, g, sp);
        else
          decode_packed(acc, n, g, sp);
        acc = 0;
      }
    }
  }
}

template <int R, int BATCH = kSumBatch, typename T>
__device__ __forceinline__ long long sum_copies(const T* a, int w0, int s) {
  constexpr int NB = R < BATCH ? R : BATCH;
  long long acc = 0;
#pragma unroll 1
  for (int r0 = 0; r0 < R; r0 += NB) {
    T v[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) v[j] = a[w0 + ((r0 + j + s) & (R - 1))];
#pragma unroll
    for (int j = 0; j < NB; ++j) acc += (long long)v[j];
  }
  return acc;
}

// Sum of the R copies, each rounded to a multiple of 2^sh first (the sums
// of u^2: one copy is below 2^59, a batch index's total after the shift
// below 2^62 -- moment_shift).
template <int R, int BATCH = kSumBatch>
__device__ __forceinline__ long long sum_copies_shifted(const unsigned long long* a, int w0, int s,
                                                        int sh) {
  constexpr int NB = R < BATCH ? R : BATCH;
  const unsigned long long half = sh > 0 ? 1ull << (sh - 1) : 0ull;
  long long acc = 0;
#pragma unroll 1
  for (int r0 = 0; r0 < R; r0 += NB) {
    unsigned long long v[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) v[j] = a[w0 + ((r0 + j + s) & (R - 1))];
#pragma unroll
    for (int j = 0; j < NB; ++j) acc += (long long)((v[j] + half) >> sh);
  }
  return acc;
}

// Moments variant: 5 values per half-bin (count, labelled count, sum u,
// sum u^2 >> mshift, labelled sum u of the offsets u of moment_scale;
// counts unscaled), fin layout [5][2CK].
template <int R>
__device__ __forceinline__ void block_moments_r(const FwdParams& P, const Hist& H, int CK,
                                                unsigned long long* fin) {
  const int chunk = 1 << P.lchunk;
  const int H2 = 2 * CK;
  for (int t = threadIdx.x; t < H2; t += kThreads) {
    long long m[5] = {0, 0, 0, 0, 0};
    // three arrays: half batches keep the registers of the main loop's
    sum_packed<R, kSumBatch / 2, true>(H.a, t * R, t, chunk, m[0], m[1], m[2]);
    m[3] = sum_copies_shifted<R, kSumBatch / 2>(H.m2, t * R, t, P.mshift);
    m[4] = sum_copies<R, kSumBatch / 2>(H.mg, t * R, t);
#pragma unroll
    for (int v = 0; v < 5; ++v)
      if (m[v]) atomicAdd(&fin[v * H2 + t], (unsigned long long)m[v]);
  }
}

template <int R, bool SOFT>
__device__ __forceinline__ void block_sums_r(const FwdParams& P, const Hist& H, int CK, bool labels,
                                             unsigned long long* fin) {
  const int chunk = 1 << P.lchunk;
  for (int t = threadIdx.x; t < CK; t += kThreads) {
    long long s0, s1 = 0, s2;
    if constexpr (!SOFT) {
      long long n = 0, g = 0;
      sum_packed<R>(H.a, t * R, t, chunk, n, g, s1);
      if (labels) {
        // fin layout [2][CK] (P.packed): the counts share one word, W << 32 | G
        // (a batch index has fewer than 2^32 voxels per channel row)
        const unsigned long long wg = ((unsigned long long)n << 32) | (unsigned long long)g;
        if (wg) atomicAdd(&fin[t], wg);
        if (s1) atomicAdd(&fin[CK + t], (unsigned long long)s1);
        continue;
      }
      s0 = n << kFrac;
      s2 = sum_copies<R>(H.g1, t * R, t);
    } else {
      s0 = sum_copies<R>(H.w, t * R, t);
      s1 = sum_copies<R>(H.p, t * R, t);
      s2 = sum_copies<R>(H.g, t * R, t);
    }
    if (s0) atomicAdd(&fin[t], (unsigned long long)s0);
    if (s1) atomicAdd(&fin[CK + t], (unsigned long long)s1);
    if (s2) atomicAdd(&fin[2 * CK + t], (unsigned long long)s2);
  }
}

// Copies per block are a power of two <= 64.
#define ACE_SWITCH_COPIES(R_, CALL) \
  switch (R_) {                     \
    case 1: CALL(1); break;         \
    case 2: CALL(2); break;         \
    case 4: CALL(4); break;         \
    case 8: CALL(8); break;         \
    case 16: CALL(16); break;       \
    case 32: CALL(32); break;       \
    default: CALL(64); break;       \
  }

__device__ __forceinline__ void block_moments(const FwdParams& P, const Hist& H, int CK,
                                              unsigned long long* fin) {
#define ACE_MOM(R) block_moments_r<R>(P, H, CK, fin)
  ACE_SWITCH_COPIES(P.copies, ACE_MOM)
#undef ACE_MOM
}

template <bool SOFT>
__device__ __forceinline__ void block_sums(const FwdParams& P, const Hist& H, int CK, bool labels,
                                           unsigned long long* fin) {
#define ACE_SUMS(R) block_sums_r<R, SOFT>(P, H, CK, labels, fin)
  ACE_SWITCH_COPIES(P.copies, ACE_SUMS)
#undef ACE_SUMS
}
#undef ACE_SWITCH_COPIES

// ---- end of a forward block.  Adds the block's sums into replica
// (tile % reps) of batch b's final sums (fixed point: exact and
// order-independent).  Ticket counters, each on its own 256-byte line, then
// pick the last block of each group of gs tiles, the last group of batch b
// (which runs b's epilogue; with one group per batch index the group's last
// block, one round trip sooner) and the last batch epilogue to start (which
// sums the per-class errors into the loss in a fixed order).  Runs in the
// block's first kThreads threads.
template <bool SOFT, bool MOM>
__device__ __forceinline__ void fwd_finish(const FwdParams& P, const Hist& H, unsigned char* hist,
                                           const float* repl, int CK, int CL, int b,
                                           int64_t tile, bool labels) {
  const int tid = threadIdx.x;
  unsigned long long* fin =
      P.fin + ((int64_t)b * P.reps + tile % P.reps) * fin_values(CK, MOM, P.packed != 0);
  if constexpr (MOM)
    block_moments(P, H, CK, fin);
  else
    block_sums<SOFT>(P, H, CK, labels, fin);
  __shared__ int s_last;
  wait_own_writes();
  __syncthreads();
  fast_stamp(P, kTlSums);
  if (tid == 0) {
    const int64_t g = tile / P.gs;
    const int64_t gsize = min(P.gs, P.tiles - g * P.gs);
    int last = 0;
    int* gc = counter(P, (int64_t)b * P.gpb + g);
    if (ticket(gc) == (int)gsize - 1) {
      __hip_atomic_store(gc, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (P.gpb == 1) {
        // one group per batch index (and epi_all implies one batch index)
        last = 1;
      } else {
        // the last group of batch b -- or, with one epilogue block for all
        // batch indices, the last group of all
        int* bc = counter(P, (int64_t)P.B * P.gpb + (P.epi_all ? 0 : b));
        const int arrivals = P.epi_all ? (int)(P.B * P.gpb) : (int)P.gpb;
        last = ticket(bc) == arrivals - 1;
        if (last) __hip_atomic_store(bc, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    s_last = last;
  }
  __syncthreads();
  fast_stamp(P, kTlTicket);
  if (!s_last) return;
  const int rows = P.B * CL;
  if (P.epi_all) {
    const float total = epilogue<SOFT, MOM>(P, hist, repl, CK, CL, 0, P.B);
    fast_stamp(P, kTlEpiEnd);
    if (tid == 0 && P.red != kRedNone)
      P.loss[0] = P.red == kRedMean ? total / (float)rows : total;
    fast_stamp(P, kTlLoss);
    return;
  }
  if (P.B == 2) {
    // ---- loss of two batch indices: each epilogue block swaps its partial
    // sum (flag bit 32 | float bits) into one word with a returning atomic
    // exchange.  The block that swaps second receives the other's partial,
    // writes the loss and clears the word; the first is done.  No ticket and
    // no wait: one device-scope round trip after the later epilogue.
    const float total = epilogue<SOFT, MOM>(P, hist, repl, CK, CL, b, 1);
    fast_stamp(P, kTlEpiEnd);
    if (P.red == kRedNone || tid != 0) return;
    for (int n = 0; n < P.publish_delay; ++n) __builtin_amdgcn_s_sleep(2);
    const unsigned long long w =
        xchg_dev(&P.part[0], (1ull << 32) | (unsigned long long)__float_as_uint(total));
    if (w >> 32) {
      store_dev(&P.part[0], 0ull);
      // the bits of wave_sum over the two partials and zero lanes: their sum
      // (either order), plus zero
      const float sum = (total + __uint_as_float((unsigned)w)) + 0.0f;
      P.loss[0] = P.red == kRedMean ? sum / (float)rows : sum;
      fast_stamp(P, kTlLoss);
    }
    return;
  }
  // ---- loss of three or more batch indices.  The loss ticket is drawn as
  // b's epilogue starts, so that its round trip overlaps the epilogue's
  // loads; the block that draws the last one sums the loss.  Every other batch epilogue publishes its partial sum
  // as one word (flag bit 32 | float bits) -- no wait for its own writes, no
  // second ticket -- and the last block polls those words.  The blocks it
  // waits for drew their tickets earlier and run epilogues that wait on
  // nothing, so the wait ends; it is bounded all the same (P.max_polls, then
  // the loss is NaN).  A word given up on is marked kAbandoned by a
  // compare-exchange, which the late block finds when it publishes (also a
  // compare-exchange) and clears: the workspace is left zero either way, and
  // the late block runs within the same launch, before any later call.
  int lt = 0;
  int* tc = counter(P, (int64_t)P.B * P.gpb + P.B);
  if (tid == 0 && P.red != kRedNone) lt = ticket(tc);
  const float total = epilogue<SOFT, MOM>(P, hist, repl, CK, CL, b, 1);
  fast_stamp(P, kTlEpiEnd);
  if (P.red == kRedNone || tid >= 64) return;
  // wave 0, every lane active: thread 0's ticket and partial sum
  const bool last = __builtin_amdgcn_readfirstlane(lt) == P.B - 1;
  const float own = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(total)));
  if (!last) {
    if (tid == 0) {
      for (int n = 0; n < P.publish_delay; ++n) __builtin_amdgcn_s_sleep(2);
      if (cas_dev(&P.part[b], 0ull, (1ull << 32) | (unsigned long long)__float_as_uint(own)) != 0ull)
        store_dev(&P.part[b], 0ull);  // the loss block gave up on this word
    }
    return;
  }
  if (tid == 0) __hip_atomic_store(tc, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float sum = 0.0f;
  for (int c0 = 0; c0 < P.B; c0 += 64) {
    const int bb = c0 + tid;
    float v = 0.0f;
    if (bb == b) {
      v = own;
    } else if (bb < P.B) {
      unsigned long long w = load_dev(&P.part[bb]);
      for (int n = 0; (w >> 32) == 0 && n < P.max_polls; ++n) {
        __builtin_amdgcn_s_sleep(2);
        w = load_dev(&P.part[bb]);
      }
      // give up: mark the word abandoned, unless it arrived meanwhile
      if ((w >> 32) == 0) w = cas_dev(&P.part[bb], 0ull, kAbandoned);
      if (w >> 32) {
        v = __uint_as_float((unsigned)w);
        store_dev(&P.part[bb], 0ull);
      } else {
        v = __builtin_nanf("");
      }
    }
    sum += wave_sum(v);
  }
  if (tid == 0) P.loss[0] = P.red == kRedMean ? sum / (float)rows : sum;
  fast_stamp(P, kTlLoss);
}

template <typename T, int CMAX, bool EXACT, int VEC, bool SOFT, bool RIGHT>
__global__ void __launch_bounds__(kThreads) fwd_kernel(const FwdParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* tabs = reinterpret_cast<float*>(smem);
  const int K = P.K;
  const int n = SOFT ? 2 * K : K;
  const int nc = EXACT ? CMAX : P.C;
  const int off = P.off;
  const int CL = nc - off;
  const int CK = CL * K;
  const int R = P.copies;
  const int tid = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int b = (int)(blk / P.tiles);
  const int64_t tile = blk - (int64_t)b * P.tiles;
  const bool labels = P.tk == kTgtLabels;

  const size_t tab_floats = (size_t)(((n + 2) + (SOFT ? 2 * K + 2 : 0) + 3) / 4 * 4);
  unsigned char* hist = smem + tab_floats * 4;
  Hist H;
  H.a = reinterpret_cast<unsigned long long*>(hist);
  H.g1 = reinterpret_cast<long long*>(hist) + (size_t)CK * R;
  H.w = reinterpret_cast<long long*>(hist);
  H.p = H.w + (size_t)CK * R;
  H.g = H.p + (size_t)CK * R;
  const size_t hist_words = (hist_bytes_per_copy(CK, SOFT, labels) * (size_t)R + 7) / 8;

  load_tables(tabs, P.btab, P.rtab, n, SOFT ? 2 * K + 2 : 0);
  {
    unsigned long long* h64 = reinterpret_cast<unsigned long long*>(hist);
    for (size_t i = tid; i < hist_words; i += kThreads) h64[i] = 0ull;
  }
  __syncthreads();
  const float* btab = tabs;
  const float* repl = tabs + n + 2;
  const int copy = tid & (R - 1);

  // this tile: voxels [t0, t0 + nvox) of batch index b
  const int64_t N = P.N;
  const int64_t t0 = tile * P.tile_vox;
  const int nvox = (int)min(P.tile_vox, N - t0);
  const T* xt = reinterpret_cast<const T*>(P.x) + (int64_t)b * nc * N + t0;
  const long long* lt = reinterpret_cast<const long long*>(P.tgt) + (int64_t)b * N + t0;
  const float* yt = reinterpret_cast<const float*>(P.tgt) + (int64_t)b * nc * N + t0;
  // generic kernels with one voxel per lane and 16 or more channels bin
  // every voxel in the single-voxel loop below: two tiles in flight held
  // their logits and targets twice (soft: 204 VGPRs at 32 channels, 2 waves
  // per SIMD); occupancy hides the loads instead
  constexpr bool kPipe = generic_pipelined<CMAX, VEC, SOFT>();
  const int nfull = (kPipe && P.vec_ok) ? nvox / VEC * VEC : 0;

  // full vector steps, software-pipelined: the next step's loads are in flight
  // while the current step is binned (two buffers, unrolled by two)
  if constexpr (kPipe) {
    Tile<CMAX, VEC> ta, tb;
    const int stride = kThreads * VEC;
    int v = tid * VEC;
    if (v < nfull) ta.template load<T, EXACT>(xt, lt, yt, N, v, nc, off, labels);
    for (; v < nfull; v += 2 * stride) {
      if (v + stride < nfull) tb.template load<T, EXACT>(xt, lt, yt, N, v + stride, nc, off, labels);
      fwd_accumulate<CMAX, EXACT, VEC, SOFT, RIGHT>(P, H, btab, repl, nc, copy, ta.x, ta.lab, ta.y, labels);
      if (v + 2 * stride < nfull) ta.template load<T, EXACT>(xt, lt, yt, N, v + 2 * stride, nc, off, labels);
      if (v + stride < nfull)
        fwd_accumulate<CMAX, EXACT, VEC, SOFT, RIGHT>(P, H, btab, repl, nc, copy, tb.x, tb.lab, tb.y, labels);
    }
  }
  // one voxel per iteration, not unrolled (the registers of one voxel's
  // channels; the generic soft kernels take every voxel here)
#pragma unroll 1
  for (int v = nfull + tid; v < nvox; v += kThreads) {
    float xv[CMAX][1];
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) load_row<T, 1>(xt + c * N + v, xv[c]);
    int lab[1];
    float yv[CMAX][1];
    if (labels) {
      load_labels<1>(lt + v, nc, lab);
    } else {
#pragma unroll
      for (int c = 0; c < CMAX; ++c)
        if ((EXACT || c < nc) && c >= off) load_row<float, 1>(yt + c * N + v, yv[c]);
    }
    fwd_accumulate<CMAX, EXACT, 1, SOFT, RIGHT>(P, H, btab, repl, nc, copy, xv, lab, yv, labels);
  }
  __syncthreads();
  fwd_finish<SOFT, false>(P, H, hist, repl, CK, CL, b, tile, labels);
}

// ------------------------------------------------------------ backward

// dL/dx of NV voxels, in place in xv (logits in, gradient out).
template <int CMAX, bool EXACT, int NV, bool SOFT, bool RIGHT>
__device__ __forceinline__ void bwd_voxels(const BwdParams& P, const float* btab, const float* repl,
                                           const float* scoef, const float* sdd, const float* sdl,
                                           const float* sg, int nc, float (&xv)[CMAX][NV],
                                           const int (&lab)[NV],
                                           const float (&yv)[CMAX][NV], bool labels) {
  const int K = P.K;
  const int off = P.off;
  const float nf = (float)(SOFT ? 2 * K : K);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    float p[CMAX];
#pragma unroll
    for (int c = 0; c < CMAX; ++c) p[c] = xv[c][j];
    activate<CMAX, EXACT>(p, nc, P.act);
    float gp[CMAX];
#pragma unroll
    for (int c = 0; c < CMAX; ++c) {
      gp[c] = 0.0f;
      if (!(EXACT || c < nc) || c < off) continue;
      const int cl = c - off;
      if constexpr (!SOFT) {
        const int k = bucket<RIGHT>(p[c], nf, K, btab);
        gp[c] = scoef[cl * K + k] * sg[cl];
      } else {
        const SoftW w = soft_assign<RIGHT>(p[c], K, nf, btab, repl);
        const float y = labels ? (lab[j] == c ? 1.0f : 0.0f) : yv[c][j];
        // p - y - d (v2_autograd.py:94-104) with p - y = s + e exactly
        // (TwoSum) and d = d_hi + d_lo: (s - d_hi) + (e - d_lo), so that the
        // residual carries neither the float32 rounding of p - y nor that of d
        const float s = p[c] - y;
        const float sp = s - p[c];
        const float e = (p[c] - (s - sp)) + (-y - sp);
        const int il = cl * K + w.l, ir = cl * K + w.r;
        const float rl = (s - sdd[il]) + (e - sdl[il]);
        const float rr = (s - sdd[ir]) + (e - sdl[ir]);
        const float left = scoef[il] * (w.lw - w.inv_span * rl);
        const float rght = scoef[ir] * (w.rw + w.inv_span * rr);
        gp[c] = sg[cl] * (left + rght);
      }
    }
    if (P.act == kActSoftmax) {
      float dot = 0.0f;
#pragma unroll
      for (int c = 0; c < CMAX; ++c)
        if (EXACT || c < nc) dot += gp[c] * p[c];
#pragma unroll
      for (int c = 0; c < CMAX; ++c)
        if (EXACT || c < nc) xv[c][j] = p[c] * (gp[c] - dot);
    } else if (P.act == kActSigmoid) {
#pragma unroll
      for (int c = 0; c < CMAX; ++c)
        if (EXACT || c < nc) xv[c][j] = gp[c] * p[c] * (1.0f - p[c]);
    } else {
#pragma unroll
      for (int c = 0; c < CMAX; ++c)
        if (EXACT || c < nc) xv[c][j] = gp[c];
    }
  }
}

template <typename T, bool EXACT, int CMAX, int VEC>
__device__ __forceinline__ void bwd_load(Tile<CMAX, VEC>& t, const T* xt, const long long* lt,
                                         const float* yt, int64_t N, int v, int nc, int off,
                                         bool labels, bool need_tgt) {
  if (need_tgt) {
    t.template load<T, EXACT>(xt, lt, yt, N, v, nc, off, labels);
  } else {
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) load_row<T, VEC>(xt + c * N + v, t.x[c]);
  }
}

template <typename T, int CMAX, bool EXACT, int VEC, bool SOFT, bool RIGHT>
__global__ void __launch_bounds__(kThreads)
    bwd_kernel(const BwdParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* tabs = reinterpret_cast<float*>(smem);
  const int K = P.K;
  const int n = SOFT ? 2 * K : K;
  const int nc = EXACT ? CMAX : P.C;
  const int off = P.off;
  const int CL = nc - off;
  const int CK = CL * K;
  const int tid = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int b = (int)(blk / P.tiles);
  const int64_t tile = blk - (int64_t)b * P.tiles;
  const bool labels = P.tk == kTgtLabels;

  const size_t tab_floats = (size_t)(((n + 2) + (SOFT ? 2 * K + 2 : 0) + 3) / 4 * 4);
  float* scoef = tabs + tab_floats;
  float* sdd = scoef + CK;          // soft: d rounded to float32 (diff[0])
  float* sdl = sdd + CK;            // soft: its remainder (diff[1])
  float* sg = sdd + (SOFT ? 2 * CK : 0);
  load_tables(tabs, P.btab, P.rtab, n, SOFT ? 2 * K + 2 : 0);
  const int64_t BCK = (int64_t)P.B * CK;
  for (int t = tid; t < CK; t += kThreads) {
    scoef[t] = P.coef[(int64_t)b * CK + t];
    if (SOFT) {
      sdd[t] = P.d[(int64_t)b * CK + t];
      sdl[t] = P.d[BCK + (int64_t)b * CK + t];
    }
  }
  for (int t = tid; t < CL; t += kThreads) {
    const float go = P.go_per_class ? P.go[b * CL + t] : P.go[0];
    sg[t] = P.jac[b * CL + t] * go;
  }
  __syncthreads();
  const float* btab = tabs;
  const float* repl = tabs + n + 2;

  const int64_t N = P.N;
  const int64_t t0 = tile * P.tile_vox;
  const int nvox = (int)min(P.tile_vox, N - t0);
  const T* xt = reinterpret_cast<const T*>(P.x) + (int64_t)b * nc * N + t0;
  T* dt = reinterpret_cast<T*>(P.dx) + (int64_t)b * nc * N + t0;
  const long long* lt = reinterpret_cast<const long long*>(P.tgt) + (int64_t)b * N + t0;
  const float* yt = reinterpret_cast<const float*>(P.tgt) + (int64_t)b * nc * N + t0;
  // as in the forward: the generic kernels at one voxel per lane with 16 or
  // more channels take every voxel through the single-voxel loop (soft: two
  // tiles plus the probabilities and dL/dp held 340 VGPRs at 32 channels)
  constexpr bool kPipe = generic_pipelined<CMAX, VEC, SOFT>();
  const int nfull = (kPipe && P.vec_ok) ? nvox / VEC * VEC : 0;

  // full vector steps, software-pipelined as in the forward
  if constexpr (kPipe) {
    Tile<CMAX, VEC> ta, tb;
    const int stride = kThreads * VEC;
    // the hard gradient needs no targets: only the logits are loaded
    const bool need_tgt = SOFT;
    int v = tid * VEC;
    if (v < nfull) bwd_load<T, EXACT, CMAX, VEC>(ta, xt, lt, yt, N, v, nc, off, labels, need_tgt);
    for (; v < nfull; v += 2 * stride) {
      if (v + stride < nfull)
        bwd_load<T, EXACT, CMAX, VEC>(tb, xt, lt, yt, N, v + stride, nc, off, labels, need_tgt);
      bwd_voxels<CMAX, EXACT, VEC, SOFT, RIGHT>(P, btab, repl, scoef, sdd, sdl, sg, nc, ta.x, ta.lab, ta.y, labels);
#pragma unroll
      for (int c = 0; c < CMAX; ++c)
        if (EXACT || c < nc) store_vec<T, VEC>(dt + c * N + v, ta.x[c]);
      if (v + 2 * stride < nfull)
        bwd_load<T, EXACT, CMAX, VEC>(ta, xt, lt, yt, N, v + 2 * stride, nc, off, labels, need_tgt);
      if (v + stride < nfull) {
        bwd_voxels<CMAX, EXACT, VEC, SOFT, RIGHT>(P, btab, repl, scoef, sdd, sdl, sg, nc, tb.x, tb.lab, tb.y, labels);
#pragma unroll
        for (int c = 0; c < CMAX; ++c)
          if (EXACT || c < nc) store_vec<T, VEC>(dt + c * N + v + stride, tb.x[c]);
      }
    }
  }
  // one voxel per iteration, not unrolled (the registers of one voxel's
  // channels; the generic soft kernels take every voxel here)
#pragma unroll 1
  for (int v = nfull + tid; v < nvox; v += kThreads) {
    float xv[CMAX][1];
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) load_row<T, 1>(xt + c * N + v, xv[c]);
    int lab[1];
    float yv[CMAX][1];
    if (SOFT) {
      if (labels) {
        load_labels<1>(lt + v, nc, lab);
      } else {
#pragma unroll
        for (int c = 0; c < CMAX; ++c)
          if ((EXACT || c < nc) && c >= off) load_row<float, 1>(yt + c * N + v, yv[c]);
      }
    }
    bwd_voxels<CMAX, EXACT, 1, SOFT, RIGHT>(P, btab, repl, scoef, sdd, sdl, sg, nc, xv, lab, yv, labels);
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) dt[c * N + v] = from_f32<T>(xv[c][0]);
  }
}


// ------------------------------------------------------------ fast path
//
// The benchmark configuration of the loss -- softmax over C channels with
// class-index targets -- as kernels with no runtime switches in the voxel
// loop.  Loads are issued unconditionally (past the last step they re-read the
// current step, a cache hit), so the compiler can wait for exactly one
// buffer's loads while the other buffer's are in flight.  Softmax outputs lie
// in [0, 1], so the bin index needs no float clamp and the fixed-point terms
// are non-negative.

// Word of bin k in a histogram copy whose bins are 1 << lsh bytes apart.
__device__ __forceinline__ unsigned long long* bin_at(unsigned long long* base, int k, int lsh) {
  return reinterpret_cast<unsigned long long*>(reinterpret_cast<unsigned char*>(base) +
                                               ((uint32_t)k << lsh));
}

// Load source of the pipelined kernels' first two steps when a tile has no
// full step: 64 bytes of zeros in device memory (read, never used), so that
// these loads can be issued unconditionally.
static __device__ __align__(16) unsigned char g_dummy_src[64];

template <int C, int VEC>
struct FastTile {
  float x[C][VEC];
  long long lab[VEC];  // raw int64 labels, converted when used
};

// One tile's logits and labels; NTL: nontemporal loads of the labels (the
// hard forward: no later kernel of the step reads them, stream_problem).
template <typename T, int C, int VEC, bool NTL = false>
__device__ __forceinline__ void fast_load(FastTile<C, VEC>& t, const T* const (&xr)[C],
                                          const long long* lr, uint32_t v, bool with_labels) {
#pragma unroll
  for (int c = 0; c < C; ++c) load_vec<T, VEC>(xr[c] + v, t.x[c]);
  if (with_labels) {
    if constexpr (VEC % 2 == 0) {
#pragma unroll
      for (int j = 0; j < VEC; j += 2) {
        if constexpr (NTL) {
          typedef long long xi64x2 __attribute__((ext_vector_type(2)));
          const xi64x2 q = __builtin_nontemporal_load(reinterpret_cast<const xi64x2*>(lr + v + j));
          t.lab[j] = q.x;
          t.lab[j + 1] = q.y;
        } else {
          const longlong2 q = *reinterpret_cast<const longlong2*>(lr + v + j);
          t.lab[j] = q.x;
          t.lab[j + 1] = q.y;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        if constexpr (NTL)
          t.lab[j] = __builtin_nontemporal_load(lr + v + j);
        else
          t.lab[j] = lr[v + j];
      }
    }
  }
}

// Channel index of a raw label, or 0xffffffff when it names no channel.
template <int C>
__device__ __forceinline__ uint32_t fast_label(long long v) {
  const uint32_t lo = (uint32_t)(unsigned long long)v;
  const uint32_t hi = (uint32_t)((unsigned long long)v >> 32);
  return (hi == 0u && lo < (uint32_t)C) ? lo : 0xffffffffu;
}

// max of raw logits with v_max3_f32 / v_max_f32 directly: fmaxf would first
// canonicalise each loaded value (one more instruction per operand)
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float vmax2(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
template <int C>
__device__ __forceinline__ float max_of(const float (&x)[C]) {
  if constexpr (C == 1) {
    return x[0];
  } else if constexpr (C == 2) {
    return vmax2(x[0], x[1]);
  } else {
    float m = vmax3(x[0], x[1], x[2]);
    int c = 3;
#pragma unroll
    for (; c + 1 < C; c += 2) m = vmax3(m, x[c], x[c + 1]);
    if (c < C) m = vmax2(m, x[c]);
    return m;
  }
}

template <int C>
__device__ __forceinline__ void softmax_fast(float (&x)[C]) {
  const float m = max_of<C>(x);
  x[0] = exp_neg(x[0] - m);
  float s = x[0];  // == 0 + x[0]: the sum starts from +0
#pragma unroll
  for (int c = 1; c < C; ++c) {
    x[c] = exp_neg(x[c] - m);
    s += x[c];
  }
  const float y = rcp_rn(s);
#pragma unroll
  for (int c = 0; c < C; ++c) x[c] = div_rn(x[c], s, y);
}

// Fast bins (softmax over C channels), for the hard forward kernels with
// class labels.  With n = K bins, each loss channel's probability is held as
// q = trunc(p~ n 2^qs), where
// p~ = e_c / s with e_c = exp2((x_c - max) log2 e) and s = e_0 + ... + e_{C-1}
// from the hardware's v_exp_f32 and v_rcp_f32 (three VALU instructions per
// channel for the exponential instead of the nine of exp_neg, no correctly
// rounded division).  The bin is k = z >> qs with z = q clamped to
// [2^(qs-1), (2n - 1) 2^(qs-1)] (t = p n clamped to [1/2, n - 1/2]).
//
// p~ is not the correctly rounded softmax: its relative error is below
// 3e-6 for C <= 16 and p >= 1 / (2n) (a, the exponent, rounded twice and
// times the float log2 e: 1.3e-7 |a|; v_exp_f32 and v_rcp_f32 1 ulp each; the
// sum's C - 1 roundings and the other terms' exponent errors), and measured
// on MI355X below 5.4e-7 over 2^24 random logit vectors at C = 4.  The bin
// edges lie within (j + 1) 8 2^-24 of the integers j + 1 in units of t
// (torch's float32 linspace, see bucket_unit).  So whenever z is at least the
// margin qmq (n 2^-18 of t for C <= 4, n 2^-17 above: twice the error bound
// plus the edge offsets) away from every multiple of 2^qs, k is the bin of
// the exact probability, on either side of `right`.  Otherwise -- or when
// the sum is NaN (NaN or infinite logits) -- the channel is "near" and takes
// the exact path (softmax_fast, bucket_unit), the path the backward kernels
// always take.  The largest logit's term is exactly 1 (x - max = 0), so a
// saturated voxel gets p~ = 1 exactly, as the exact path does.
template <int C>
__device__ __forceinline__ void fast_exp(const float (&x)[C], const FwdParams& P, float (&e)[C],
                                         float& rq, bool& nan) {
  constexpr float kLog2e = 0x1.715476p+0f;
  const float m = max_of<C>(x);
  e[0] = __builtin_amdgcn_exp2f((x[0] - m) * kLog2e);
  float s = e[0];
#pragma unroll
  for (int c = 1; c < C; ++c) {
    e[c] = __builtin_amdgcn_exp2f((x[c] - m) * kLog2e);
    s += e[c];
  }
  rq = __builtin_amdgcn_rcpf(s) * P.qscale;
  nan = !(s == s);
}
// q, the bin k and whether the channel is near an edge, from e_c and n 2^qs / s
// (ace_bins.hpp: fast_bin_index).
__device__ __forceinline__ bool fast_bin(float e, float rq, const FwdParams& P, uint32_t& q,
                                         uint32_t& k) {
  q = cvt_u32(e * rq);
  return fast_bin_index(q, P.qlo, P.qhi, P.qmq, P.qmask, P.qs, k);
}

// softmax_fast with every probability scaled by sc = 2^m (the fixed-point
// scale of the histograms, isc = 2^-m): q = e y sc, r = e - (s isc) q,
// p = q + r y sc are the steps of div_rn with both factors scaled by powers
// of two, so p is exactly 2^m times the correctly rounded quotient (tiny
// quotients below 2^-126 aside, which are bin 0 and 0 in fixed point either
// way) and one multiply per channel is saved.
template <int C>
__device__ __forceinline__ void softmax_fixed(float (&x)[C], float sc, float isc) {
  const float m = max_of<C>(x);
  x[0] = exp_neg(x[0] - m);
  float s = x[0];
#pragma unroll
  for (int c = 1; c < C; ++c) {
    x[c] = exp_neg(x[c] - m);
    s += x[c];
  }
  const float y = rcp_rn(s) * sc;
  const float s30 = s * isc;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const float q = x[c] * y;
    const float r = fmaf(-s30, q, x[c]);
    x[c] = fmaf(r, y, q);
  }
}

// Hard binning, C <= 4: the high word of a voxel's packed increment for
// channel c is 1 << 21 (count) | (label == c) << 10 (label count).  X holds
// 0x04 in byte `label` (0 for labels naming no channel); one v_perm_b32 per
// channel picks that byte into byte 1 and 0x20 from K into byte 2.
__device__ __forceinline__ uint32_t label_bytes(long long lab, int C) {
  const unsigned long long u = (unsigned long long)lab;
  const uint32_t lo = (uint32_t)u;
  return u < (unsigned long long)C ? (4u << ((lo << 3) & 31)) : 0u;
}
__device__ __forceinline__ uint32_t packed_high(uint32_t X, int c) {
  return __builtin_amdgcn_perm(X, 1u << (kShiftN - 32), 0x0c02040cu + ((uint32_t)c << 8));
}

// One (voxel, channel) into the hard histogram copies.  hb: this lane's
// copy of the channel's bin 0 (u64 words), bins R words = 1 << lsh bytes
// apart; k the bin, q = trunc(p K 2^qs), hi the high word of the packed
// increment (count | label count).
__device__ __forceinline__ void accumulate_hard(uint32_t k, uint32_t q, uint32_t hi, int lsh,
                                                unsigned long long* hb) {
  lds_add(bin_at(hb, (int)k, lsh), ((unsigned long long)hi << 32) | q);
}

// High word of a voxel's packed increment for channel c: 1 << 21 (count)
// | (label == c) << 10 (label count).  X = label_bytes(label) (C <= 4), lc =
// fast_label(label).
template <int C>
__device__ __forceinline__ uint32_t high_word(uint32_t X, uint32_t lc, int c) {
  if constexpr (C <= 4)
    return packed_high(X, c);
  else
    return lc == (uint32_t)c ? ((1u << (kShiftN - 32)) | (1u << (kShiftG - 32))) : (1u << (kShiftN - 32));
}

// Soft binning, one tile: the correctly rounded softmax computed directly
// scaled by 2^m (softmax_fixed, the moments' fixed-point scale; the bucket
// table in LDS is scaled the same way), the half-bin h by one table read and
// one comparison, and the moments of the offset u = trunc(p 2^m) - h w
// (moment_scale) -- exact for the quantised p, which the soft gradient needs
// in bins of a few voxels (d enters it amplified by 1 / S = 2K).  C <= 4: two
// voxels at a time, every table read issued before the atomics (the reads
// cannot pass an LDS atomic); C = 16: one voxel at a time.
template <int C, int VEC, bool RIGHT, bool SKIP0>
__device__ __forceinline__ void soft_accumulate(const FastTile<C, VEC>& t, const float* tab,
                                                const FwdParams& P, int K, int lsh,
                                                unsigned long long* const (&hb)[C],
                                                const size_t words) {
  const float sc = P.msc;
  const float isc = P.misc;
  const int nw = -P.mw;
  const float nf = (float)(2 * K) * isc;
  constexpr bool BATCH = C <= 4;
  constexpr int NJ = BATCH ? (VEC > 2 ? 2 : VEC) : 1;
#pragma unroll
  for (int j0 = 0; j0 < VEC; j0 += NJ) {
    float p[NJ][C];
    uint32_t lab[NJ];
    int g[NJ][C];
    float e[NJ][C];
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
#pragma unroll
      for (int c = 0; c < C; ++c) p[jj][c] = t.x[c][j0 + jj];
      softmax_fixed<C>(p[jj], sc, isc);
      lab[jj] = fast_label<C>(t.lab[j0 + jj]);
#pragma unroll
      for (int c = 0; c < C; ++c) g[jj][c] = bucket_guess(p[jj][c], nf);
    }
    if constexpr (BATCH) {
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int c = 0; c < C; ++c)
          if (!(c == 0 && SKIP0)) e[jj][c] = tab[g[jj][c] + 1];
    }
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      // moments of the voxel's half-bin h: count | labelled count | sum u
      // packed as in hard binning, sum u^2, labelled sum u; u < 2^24 (one
      // 24-bit multiply-add, u^2 two 24-bit multiplies)
      unsigned long long* ga = hb[0];
      uint32_t gq = 0u;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (c == 0 && SKIP0) continue;
        const int h = bucket_fix<RIGHT>(g[jj][c], BATCH ? e[jj][c] : tab[g[jj][c] + 1], p[jj][c]);
        const uint32_t u = mad_i24(h, nw, cvt_u32(p[jj][c]));
        const bool hit = lab[jj] == (uint32_t)c;
        const uint32_t hi = hit ? ((1u << (kMomShiftN - 32)) | (1u << (kMomShiftG - 32)))
                                : (1u << (kMomShiftN - 32));
        unsigned long long* a = bin_at(hb[c], h, lsh);
        lds_add(a, ((unsigned long long)hi << 32) | u);
        lds_add(a + words, square_u24(u));
        ga = hit ? a : ga;
        gq = hit ? u : gq;
      }
      // unconditional: without a labelled loss channel gq is 0 and ga the
      // first half-bin of channel 0's copy, so the add changes nothing
      lds_add(ga + 2 * words, (unsigned long long)gq);
    }
  }
}

// One tile into the histogram copies.  Hard binning: every (voxel, loss
// channel) through fast_bin; the few near an edge are added afterwards
// through the exact path (correctly rounded softmax, table lookup), so every
// bin is the exact bin of the reference's float32 probability semantics, and
// the sums of p carry p~ (the loss and the gradient's sign(d) are within
// their tolerances of the exact sums).  Soft binning: soft_accumulate.
// SKIP0: channel 0 (background) is not in the loss.
template <int C, int VEC, bool SOFT, bool RIGHT, bool SKIP0>
__device__ __forceinline__ void fast_accumulate(const FastTile<C, VEC>& t, const float* tab,
                                                const FwdParams& P, int K, int lsh,
                                                unsigned long long* const (&hb)[C],
                                                const size_t words) {
  static_assert(C * VEC <= 32, "near flags of a tile in one 32-bit word");
  if constexpr (SOFT) {
    soft_accumulate<C, VEC, RIGHT, SKIP0>(t, tab, P, K, lsh, hb, words);
    return;
  }
  uint32_t nearbits = 0;
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    float x[C], e[C], rq;
    bool nan;
#pragma unroll
    for (int c = 0; c < C; ++c) x[c] = t.x[c][j];
    fast_exp<C>(x, P, e, rq, nan);
    const uint32_t X = C <= 4 ? label_bytes(t.lab[j], C) : 0u;
    const uint32_t lc = fast_label<C>(t.lab[j]);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (c == 0 && SKIP0) continue;
      uint32_t q, k;
      const bool near = fast_bin(e[c], rq, P, q, k) || nan;
      // k is a valid bin either way (fast_bin clamps it): a near channel adds
      // 0 here, which keeps the atomics out of a branch, and its value below
      const uint32_t hi = near ? 0u : high_word<C>(X, lc, c);
      accumulate_hard(k, near ? 0u : q, hi, lsh, hb[c]);
      nearbits |= (near ? 1u : 0u) << (j * C + c);
    }
  }
  if (nearbits) {
    const float nf = (float)K;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const uint32_t bits = (nearbits >> (j * C)) & ((1u << C) - 1u);
      if (bits) {
        float p[C];
#pragma unroll
        for (int c = 0; c < C; ++c) p[c] = t.x[c][j];
        softmax_fast<C>(p);
        const uint32_t X = C <= 4 ? label_bytes(t.lab[j], C) : 0u;
        const uint32_t lc = fast_label<C>(t.lab[j]);
#pragma unroll
        for (int c = 0; c < C; ++c) {
          if ((c == 0 && SKIP0) || !(bits & (1u << c))) continue;
          const uint32_t k = (uint32_t)bucket_unit<RIGHT>(p[c], nf, tab);
          const uint32_t q = cvt_u32(p[c] * P.qscale);
          accumulate_hard(k, q, high_word<C>(X, lc, c), lsh, hb[c]);
        }
      }
    }
  }
}

// SKIP0: channel 0 (background) is not in the loss (P.off == 1).  blk is the
// block's index in P's own grid, smem the block's dynamic LDS.  Any block
// size that is a multiple of 256 up to 1024 (kFastThreads, the launch
// bound): every thread bins its share of the tile, then the first 256
// threads add the block's sums and run the cross-block protocol.
template <typename T, int C, int VEC, bool SOFT, bool RIGHT, bool SKIP0>
__device__ __forceinline__ void fwd_fast_body(const FwdParams& P, const int64_t blk,
                                              unsigned char* smem) {
  fast_stamp(P, kTlStart);
  float* tabs = reinterpret_cast<float*>(smem);
  const int K = P.K;
  const int n = SOFT ? 2 * K : K;
  constexpr int off = SKIP0 ? 1 : 0;
  const int CL = C - off;
  const int CK = CL * K;
  const int R = P.copies;
  const int lr = __builtin_ctz((unsigned)R);
  const int lsh = lr + 3;
  const int tid = threadIdx.x;
  const int b = (int)(blk / P.tiles);
  const int64_t tile = blk - (int64_t)b * P.tiles;

  const size_t tab_floats = (size_t)(((n + 2) + (SOFT ? 2 * K + 2 : 0) + 3) / 4 * 4);
  unsigned char* hist = smem + tab_floats * 4;
  // bins per channel: K (hard) or 2K half-bins (soft moments)
  const int NB = SOFT ? 2 * K : K;
  const size_t words = (size_t)CL * NB * R;  // u64 words of one histogram array
  Hist H;
  H.a = reinterpret_cast<unsigned long long*>(hist);
  H.m2 = H.a + words;
  H.mg = H.a + 2 * words;
  const size_t hist_words = (hist_bytes_per_copy(CK, SOFT, true, SOFT) * (size_t)R + 7) / 8;
  const int nrepl = SOFT ? 2 * K + 2 : 0;

  const int64_t N = P.N;
  const int64_t t0 = tile * P.tile_vox;
  const int nvox = (int)min(P.tile_vox, N - t0);
  const T* xr[C];
#pragma unroll
  for (int c = 0; c < C; ++c)
    xr[c] = reinterpret_cast<const T*>(P.x) + ((int64_t)b * C + c) * N + t0;
  const long long* lr_ = reinterpret_cast<const long long*>(P.tgt) + (int64_t)b * N + t0;
  const int nfull = P.vec_ok ? nvox / VEC * VEC : 0;
  const int nt = SOFT ? kThreads : (int)blockDim.x;  // soft: 256-thread blocks (fast_bound)
  const int stride = nt * VEC;
  const int nsteps = nfull / stride;  // steps in which every thread has a full vector

  // table loads, then the first tile's loads; the tables are written to LDS
  // and the histogram cleared while the tile is in flight
  TableRegs treg;
  treg.load(P.btab, P.rtab, n, nrepl, nt);
  FastTile<C, VEC> ta, tb;
  const uint32_t v0 = (uint32_t)(tid * VEC);
  // voxel offset of this lane in step j, clamped to the last step: a load
  // past the end (odd step counts only) re-reads the last step (L2 hit) so
  // that every load is unconditional and the waits stay partial
  auto at = [&](int j) -> uint32_t {
    return v0 + (uint32_t)((j < nsteps ? j : nsteps - 1) * stride);
  };
  {
    // unconditional (a load under a branch would turn the table wait below
    // into a wait for every load); without a full step they read g_dummy_src
    const bool pipe = nsteps > 0;
    const T* px[C];
#pragma unroll
    for (int c = 0; c < C; ++c) px[c] = pipe ? xr[c] : reinterpret_cast<const T*>(g_dummy_src);
    const long long* pl = pipe ? lr_ : reinterpret_cast<const long long*>(g_dummy_src);
    fast_load<T, C, VEC, !SOFT>(ta, px, pl, pipe ? at(0) : 0u, true);
    fast_load<T, C, VEC, !SOFT>(tb, px, pl, pipe ? at(1) : 0u, true);
  }
  // soft: the bucket table scaled by 2^m like softmax_fixed's probabilities;
  // hard: as given (the exact path's bucket_unit)
  treg.store(tabs, P.btab, P.rtab, n, nrepl, nt, SOFT ? P.msc : 1.0f);
  {
    unsigned long long* h64 = reinterpret_cast<unsigned long long*>(hist);
    for (size_t i = tid; i < hist_words; i += nt) h64[i] = 0ull;
  }
  __syncthreads();
  const float* tab = tabs;
  const float* repl = tabs + n + 2;
  const int copy = tid & (R - 1);
  unsigned long long* hb[C];
#pragma unroll
  for (int c = 0; c < C; ++c)
    hb[c] = H.a + ((size_t)((c < off ? 0 : c - off) * NB) << lr) + copy;

  // two tiles in rotation (steps i and i + 1 loaded before step i is
  // binned); the last pair is peeled so that no step is loaded twice
  if (nsteps > 0) {
    int i = 0;
    for (; i + 2 < nsteps; i += 2) {
      fast_accumulate<C, VEC, SOFT, RIGHT, SKIP0>(ta, tab, P, K, lsh, hb, words);
      fast_load<T, C, VEC, !SOFT>(ta, xr, lr_, at(i + 2), true);
      fast_accumulate<C, VEC, SOFT, RIGHT, SKIP0>(tb, tab, P, K, lsh, hb, words);
      fast_load<T, C, VEC, !SOFT>(tb, xr, lr_, at(i + 3), true);
    }
    fast_accumulate<C, VEC, SOFT, RIGHT, SKIP0>(ta, tab, P, K, lsh, hb, words);
    if (i + 1 < nsteps) fast_accumulate<C, VEC, SOFT, RIGHT, SKIP0>(tb, tab, P, K, lsh, hb, words);
  }
  // remaining full vectors (not every thread has one), then single voxels
  for (int v = nsteps * stride + tid * VEC; v < nfull; v += stride) {
    FastTile<C, VEC> t;
    fast_load<T, C, VEC, !SOFT>(t, xr, lr_, (uint32_t)v, true);
    fast_accumulate<C, VEC, SOFT, RIGHT, SKIP0>(t, tab, P, K, lsh, hb, words);
  }
  for (int v = nfull + tid; v < nvox; v += nt) {
    FastTile<C, 1> t;
    fast_load<T, C, 1>(t, xr, lr_, (uint32_t)v, true);
    fast_accumulate<C, 1, SOFT, RIGHT, SKIP0>(t, tab, P, K, lsh, hb, words);
  }
  __syncthreads();
  // the block's sums and the cross-block protocol take kThreads threads; the
  // other waves end here (a barrier waits only for waves that have not ended)
  if (tid >= kThreads) return;
  fast_stamp(P, kTlLoop);
  fwd_finish<SOFT, SOFT>(P, H, hist, repl, CK, CL, b, tile, true);
}

// Soft backward per half-bin: with the exact-arithmetic weights of the
// moments forward (lw = (cr - p) / S, rw = (p - cl) / S, S = cr - cl), the
// soft dL/dp of v2_autograd.py:94-104,
//   g (coef_l (lw - (p - y - d_l) / S) + coef_r (rw + (p - y - d_r) / S)),
// is linear in p and y: A + B (p - y/2) with A = g/S (coef_l (cr + d_l) -
// coef_r (cl + d_r)) and B = 2 g/S (coef_r - coef_l).  A and B are each of
// the order of 2K coef g, while dL/dp is a small residual wherever p - y - d
// is small (bins of a few well-calibrated voxels), so the form is evaluated
// from the half-bin's lower boundary e instead: A_y + B (p - e) with
// A_y = A + B (e - y/2) formed in float64 for y = 0 and y = 1, from
// d = d_hi + d_lo (sdd, sdl: the float64 d of the forward's sums).  p - e is
// exact in float32 (e <= p <= 2e for h >= 1, Sterbenz; e = 0 for h = 0) and
// at most 1/(2K).  A_y and B (p - e) can still be many times dL/dp, which
// they cancel to (bins whose weight is just above empty_weight, where coef
// is large), so A_0, A_1 and B are each held as a float32 pair, value and
// remainder: dL/dp = fma(B, p - e, A_y) + fma(B', p - e, A_y') is within an
// ulp or two of dL/dp itself.  Per half-bin h of every loss channel (index
// t = cl 2K + h): sab[8t + 4y .. 8t + 4y + 3] = (A_y, A_y', B, e) for y = 0
// and y = 1, read by one 16-byte load at the voxel's y, and sbl[t] = B'
// (sbl = sab + 8 C' 2K); tab is the padded half-boundary table (tab[h] = e
// for h >= 1).
__device__ __forceinline__ void soft_half_bin_coefficients(float* sab, const float* tab,
                                                           const float* repl, const float* scoef,
                                                           const float* sdd, const float* sdl,
                                                           const float* sg, int K, int CL) {
  const int H = 2 * K;
  for (int t = threadIdx.x; t < CL * H; t += kThreads) {
    const int cl = t / H;
    const int hh = t - cl * H;
    const int l = max(hh - 1, 0) >> 1;
    const int r = min(hh + 1, H - 1) >> 1;
    const double cL = repl[hh], cR = repl[hh + 2];
    const double gs = (double)sg[cl] / (cR - cL);
    const double kl = scoef[cl * K + l], kr = scoef[cl * K + r];
    const double dl = (double)sdd[cl * K + l] + (double)sdl[cl * K + l];
    const double dr = (double)sdd[cl * K + r] + (double)sdl[cl * K + r];
    const double A = gs * (kl * (cR + dl) - kr * (cL + dr));
    const double Bc = 2.0 * gs * (kr - kl);
    const float e = hh == 0 ? 0.0f : tab[hh];
    const double a0 = A + Bc * (double)e, a1 = A + Bc * ((double)e - 0.5);
    const float a0h = (float)a0, a1h = (float)a1, bh = (float)Bc;
    *reinterpret_cast<float4*>(sab + 8 * t) = make_float4(a0h, (float)(a0 - (double)a0h), bh, e);
    *reinterpret_cast<float4*>(sab + 8 * t + 4) = make_float4(a1h, (float)(a1 - (double)a1h), bh, e);
    sab[8 * CL * H + t] = (float)(Bc - (double)bh);
  }
}

// Backward of one tile, in place in t.x (logits in, gradient out).
template <int C, int VEC, bool SOFT, bool RIGHT, bool SKIP0>
__device__ __forceinline__ void fast_backward(FastTile<C, VEC>& t, const float* tab,
                                              const float* sab, const float* scoef,
                                              const float* sg, int K) {
  constexpr int off = SKIP0 ? 1 : 0;
  const float nf = (float)(SOFT ? 2 * K : K);
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    float p[C];
#pragma unroll
    for (int c = 0; c < C; ++c) p[c] = t.x[c][j];
    softmax_fast<C>(p);
    float gp[C];
    uint32_t lab = 0xffffffffu;
    if constexpr (SOFT) lab = fast_label<C>(t.lab[j]);
#pragma unroll
    for (int c = 0; c < C; ++c) {
      gp[c] = 0.0f;
      if (c == 0 && off != 0) continue;
      const int cl = c - off;
      if constexpr (!SOFT) {
        const int k = bucket_unit<RIGHT>(p[c], nf, tab);
        gp[c] = scoef[cl * K + k] * sg[cl];
      } else {
        const int h = bucket_unit<RIGHT>(p[c], nf, tab);
        const int hb = cl * 2 * K + h;
        const bool hit = lab == (uint32_t)c;
        const float4 ab = *reinterpret_cast<const float4*>(sab + 8 * hb + (hit ? 4 : 0));
        const float bl = sab[8 * (C - off) * 2 * K + hb];
        const float t = p[c] - ab.w;
        gp[c] = fmaf(ab.z, t, ab.x) + fmaf(bl, t, ab.y);
      }
    }
    float dot = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) dot += gp[c] * p[c];
#pragma unroll
    for (int c = 0; c < C; ++c) t.x[c][j] = p[c] * (gp[c] - dot);
  }
}

template <typename T, int C, int VEC, bool SOFT, bool RIGHT, bool SKIP0, bool STREAM>
__device__ __forceinline__ void bwd_fast_body(const BwdParams& P, const int64_t blk,
                                              unsigned char* smem) {
  float* tabs = reinterpret_cast<float*>(smem);
  const int K = P.K;
  const int n = SOFT ? 2 * K : K;
  constexpr int off = SKIP0 ? 1 : 0;
  const int CL = C - off;
  const int CK = CL * K;
  const int tid = threadIdx.x;
  const int b = (int)(blk / P.tiles);
  const int64_t tile = blk - (int64_t)b * P.tiles;

  const size_t tab_floats = (size_t)(((n + 2) + (SOFT ? 2 * K + 2 : 0) + 3) / 4 * 4);
  float* scoef = tabs + tab_floats;
  float* sdd = scoef + CK;  // soft: d rounded to float32 (diff[0])
  float* sdl = sdd + CK;    // soft: its remainder (diff[1])
  float* sg = sdd + (SOFT ? 2 * CK : 0);
  // soft: (A_0, A_1, B, e) and their remainders per half-bin, 16-byte
  // aligned after g (tab_floats is a multiple of 4; the host sizes the region
  // the same way)
  float* sab = tabs + (((size_t)tab_floats + (size_t)CK * (SOFT ? 3 : 1) + CL + 3) & ~(size_t)3);
  const int nrepl = SOFT ? 2 * K + 2 : 0;

  const int64_t N = P.N;
  const int64_t t0 = tile * P.tile_vox;
  const int nvox = (int)min(P.tile_vox, N - t0);
  const T* xr[C];
  T* dr[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    xr[c] = reinterpret_cast<const T*>(P.x) + ((int64_t)b * C + c) * N + t0;
    dr[c] = reinterpret_cast<T*>(P.dx) + ((int64_t)b * C + c) * N + t0;
  }
  const long long* lr_ = reinterpret_cast<const long long*>(P.tgt) + (int64_t)b * N + t0;
  const int nfull = P.vec_ok ? nvox / VEC * VEC : 0;
  const int stride = kThreads * VEC;
  const int nsteps = nfull / stride;

  // tables and this thread's first coefficients, then the first tile's loads;
  // LDS is filled while the tile is in flight
  TableRegs treg;
  treg.load(P.btab, P.rtab, n, nrepl, kThreads);
  const float* cb = P.coef + (int64_t)b * CK;
  const float* db = P.d + (int64_t)b * CK;
  const float* dlb = db + (int64_t)P.B * CK;
  // unconditional loads (clamped indices) so that the waits below stay partial
  const int tc_ = min(tid, CK - 1);
  const int tl_ = min(tid, CL - 1);
  const float c0 = cb[tc_];
  const float d0 = SOFT ? db[tc_] : 0.0f;
  const float dl0 = SOFT ? dlb[tc_] : 0.0f;
  const float g0 = P.jac[b * CL + tl_] * P.go[P.go_per_class ? b * CL + tl_ : 0];
  FastTile<C, VEC> ta, tb;
  const uint32_t v0 = (uint32_t)(tid * VEC);
  auto at = [&](int j) -> uint32_t {
    return v0 + (uint32_t)((j < nsteps ? j : nsteps - 1) * stride);
  };
  {
    const bool pipe = nsteps > 0;
    const T* px[C];
#pragma unroll
    for (int c = 0; c < C; ++c) px[c] = pipe ? xr[c] : reinterpret_cast<const T*>(g_dummy_src);
    const long long* pl = pipe ? lr_ : reinterpret_cast<const long long*>(g_dummy_src);
    fast_load<T, C, VEC>(ta, px, pl, pipe ? at(0) : 0u, SOFT);
    fast_load<T, C, VEC>(tb, px, pl, pipe ? at(1) : 0u, SOFT);
  }
  treg.store(tabs, P.btab, P.rtab, n, nrepl, kThreads);
  if (tid < CK) {
    scoef[tid] = c0;
    if (SOFT) {
      sdd[tid] = d0;
      sdl[tid] = dl0;
    }
  }
  if (tid < CL) sg[tid] = g0;
  for (int i = tid + kThreads; i < CK; i += kThreads) {
    scoef[i] = cb[i];
    if (SOFT) {
      sdd[i] = db[i];
      sdl[i] = dlb[i];
    }
  }
  for (int i = tid + kThreads; i < CL; i += kThreads)
    sg[i] = P.jac[b * CL + i] * (P.go_per_class ? P.go[b * CL + i] : P.go[0]);
  __syncthreads();
  const float* tab = tabs;
  const float* repl = tabs + n + 2;
  if constexpr (SOFT) {
    soft_half_bin_coefficients(sab, tab, repl, scoef, sdd, sdl, sg, K, CL);
    __syncthreads();
  }

  // two tiles in rotation (steps i and i + 1 loaded before step i is
  // processed); the last pair is peeled so that no step is loaded twice
  if (nsteps > 0) {
    int i = 0;
    for (; i + 2 < nsteps; i += 2) {
      fast_backward<C, VEC, SOFT, RIGHT, SKIP0>(ta, tab, sab, scoef, sg, K);
#pragma unroll
      for (int c = 0; c < C; ++c) store_dx<T, VEC, STREAM>(dr[c] + at(i), ta.x[c]);
      fast_load<T, C, VEC>(ta, xr, lr_, at(i + 2), SOFT);
      fast_backward<C, VEC, SOFT, RIGHT, SKIP0>(tb, tab, sab, scoef, sg, K);
#pragma unroll
      for (int c = 0; c < C; ++c) store_dx<T, VEC, STREAM>(dr[c] + at(i + 1), tb.x[c]);
      fast_load<T, C, VEC>(tb, xr, lr_, at(i + 3), SOFT);
    }
    fast_backward<C, VEC, SOFT, RIGHT, SKIP0>(ta, tab, sab, scoef, sg, K);
#pragma unroll
    for (int c = 0; c < C; ++c) store_dx<T, VEC, STREAM>(dr[c] + at(i), ta.x[c]);
    if (i + 1 < nsteps) {
      fast_backward<C, VEC, SOFT, RIGHT, SKIP0>(tb, tab, sab, scoef, sg, K);
#pragma unroll
      for (int c = 0; c < C; ++c) store_dx<T, VEC, STREAM>(dr[c] + at(i + 1), tb.x[c]);
    }
  }
  for (int v = nsteps * stride + tid * VEC; v < nfull; v += stride) {
    FastTile<C, VEC> t;
    fast_load<T, C, VEC>(t, xr, lr_, (uint32_t)v, SOFT);
    fast_backward<C, VEC, SOFT, RIGHT, SKIP0>(t, tab, sab, scoef, sg, K);
#pragma unroll
    for (int c = 0; c < C; ++c) store_dx<T, VEC, STREAM>(dr[c] + v, t.x[c]);
  }
  for (int v = nfull + tid; v < nvox; v += kThreads) {
    FastTile<C, 1> t;
    fast_load<T, C, 1>(t, xr, lr_, (uint32_t)v, SOFT);
    fast_backward<C, 1, SOFT, RIGHT, SKIP0>(t, tab, sab, scoef, sg, K);
#pragma unroll
    for (int c = 0; c < C; ++c) dr[c][v] = from_f32<T>(t.x[c][0]);
  }
}

// One problem per launch: block blockIdx.x of P's grid.
// Block size bound of the fast forward kernels (ace_geometry.hpp:
// fast_fwd_bound).
template <int C, bool SOFT>
constexpr int fast_bound() {
  return fast_fwd_bound(C, SOFT);
}
// Backward: at least 4 waves per SIMD (at most 128 VGPRs) for the
// 16-channel kernel with every channel in the loss, whose grid is sized for
// that occupancy (ace_abi.hip: bwd_steps).  At one voxel per lane it takes 81
// VGPRs and the bound holds by itself; at two it took ~134 without it.
template <int C, bool SKIP0>
constexpr int bwd_min_waves() {
  return (C > 4 && !SKIP0) ? 4 : 1;
}
template <typename T, int C, int VEC, bool SOFT, bool RIGHT, bool SKIP0>
__global__ void __launch_bounds__((fast_bound<C, SOFT>())) fwd_kernel_fast(const FwdParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  fwd_fast_body<T, C, VEC, SOFT, RIGHT, SKIP0>(P, blockIdx.x, smem);
}
// STREAM: the problem's logits, targets and gradient exceed the last-level
// cache (stream_problem): the gradient is written with nontemporal stores.
template <typename T, int C, int VEC, bool SOFT, bool RIGHT, bool SKIP0, bool STREAM>
__global__ void __launch_bounds__(kThreads, (bwd_min_waves<C, SKIP0>())) bwd_kernel_fast(const BwdParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  bwd_fast_body<T, C, VEC, SOFT, RIGHT, SKIP0, STREAM>(P, blockIdx.x, smem);
}

// Several problems of one configuration in one launch (the levels of a
// deep-supervision step): problem l owns blocks [start[l], start[l + 1]) of
// the grid and runs exactly as its own launch would, with its own workspace
// region, so each result is bit-identical to a separate call.
constexpr int kMaxLevels = 4;
struct FwdLevels {
  FwdParams lv[kMaxLevels];
  long long start[kMaxLevels];  // first block of each level, increasing
  int n;
  int nt;                       // threads per block, the same for every level
};
struct BwdLevels {
  BwdParams lv[kMaxLevels];
  long long start[kMaxLevels];
  int n;
};
__device__ __forceinline__ int level_of(const long long (&start)[kMaxLevels], int n, long long g) {
  int l = 0;
#pragma unroll
  for (int j = 1; j < kMaxLevels; ++j)
    if (j < n && g >= start[j]) l = j;
  return l;
}
template <typename T, int C, int VEC, bool SOFT, bool RIGHT, bool SKIP0>
__global__ void __launch_bounds__((fast_bound<C, SOFT>())) fwd_kernel_fast_levels(const FwdLevels L) {
  extern __shared__ __align__(16) unsigned char smem[];
  const long long g = blockIdx.x;
  const int l = level_of(L.start, L.n, g);
  fwd_fast_body<T, C, VEC, SOFT, RIGHT, SKIP0>(L.lv[l], g - L.start[l], smem);
}
template <typename T, int C, int VEC, bool SOFT, bool RIGHT, bool SKIP0>
__global__ void __launch_bounds__(kThreads, (bwd_min_waves<C, SKIP0>())) bwd_kernel_fast_levels(const BwdLevels L) {
  extern __shared__ __align__(16) unsigned char smem[];
  const long long g = blockIdx.x;
  const int l = level_of(L.start, L.n, g);
  bwd_fast_body<T, C, VEC, SOFT, RIGHT, SKIP0, false>(L.lv[l], g - L.start[l], smem);
}

// ------------------------------------------------------------ launchers

template <typename T, bool SOFT, bool RIGHT>
hipError_t launch_variant_fwd(const Geometry& g, const FwdParams& prm, hipStream_t s);
template <typename T, bool SOFT, bool RIGHT>
hipError_t launch_variant_bwd(const Geometry& g, const BwdParams& prm, hipStream_t s);
template <typename T, bool SOFT, bool RIGHT>
hipError_t launch_levels_fwd(int cmax, long long nblk, size_t lds, const FwdLevels& L,
                             hipStream_t s);
template <typename T, bool SOFT, bool RIGHT>
hipError_t launch_levels_bwd(int cmax, long long nblk, size_t lds, const BwdLevels& L,
                             hipStream_t s);

// The fast kernels serve softmax with class-index targets for C in {2, 3, 4, 16};
// soft binning only in the moments layout (g.moments: the host declines it
// when the bin count or its LDS size is too large, and the generic soft
// kernels then run with their own layout).
template <int CMAX, bool EXACT>
constexpr bool has_fast() {
  return EXACT && (CMAX == 2 || CMAX == 3 || CMAX == 4 || CMAX == 16);
}

// Events stamped by the kernels launched from the calling thread
// (ace_set_launch_events): start as the dispatch begins, stop as it ends.
struct LaunchEvents {
  hipEvent_t start = nullptr;
  hipEvent_t stop = nullptr;
};
inline LaunchEvents& launch_events() {
  static thread_local LaunchEvents ev;
  return ev;
}

// One launch of `kern` (one by-value parameter block) on nt-thread blocks.
template <typename Kern, typename Params>
hipError_t launch(Kern kern, long long nblk, size_t lds, hipStream_t s, const Params& prm,
                  int nt = kThreads) {
  const LaunchEvents& ev = launch_events();
  if (ev.start || ev.stop) {
    void* args[] = {const_cast<Params*>(&prm)};
    return hipExtLaunchKernel(reinterpret_cast<const void*>(kern), dim3((unsigned)nblk),
                              dim3((unsigned)nt), args, lds, s, ev.start, ev.stop, 0);
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3((unsigned)nt), lds, s, prm);
  return hipGetLastError();
}

template <typename T, int CMAX, bool EXACT, int VEC, bool SOFT, bool RIGHT>
hipError_t launch_fwd_t(const Geometry& g, const FwdParams& prm, hipStream_t s) {
  // the geometry's voxels per lane (tiles, the alignment test behind
  // vec_ok) must be the kernel's: a wider kernel would issue vector loads
  // the host never checked
  if (g.var.vec != VEC) return hipErrorInvalidConfiguration;
  auto kern = fwd_kernel<T, CMAX, EXACT, VEC, SOFT, RIGHT>;
  int nt = kThreads;
  if constexpr (has_fast<CMAX, EXACT>()) {
    // g.fast: softmax with class labels, soft binning in the moments layout
    // (the host's decision, ace_abi.hip: fast_forward)
    if (g.fast) {
      kern = prm.off ? fwd_kernel_fast<T, CMAX, VEC, SOFT, RIGHT, true>
                     : fwd_kernel_fast<T, CMAX, VEC, SOFT, RIGHT, false>;
      nt = g.nt;
      // never more threads per block than the kernel was compiled for
      if (nt > fast_bound<CMAX, SOFT>()) return hipErrorInvalidConfiguration;
    }
  }
  if (g.lds_fwd > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)g.lds_fwd);
    if (e != hipSuccess) return e;
  }
  return launch(kern, g.nblk, g.lds_fwd, s, prm, nt);
}

template <typename T, int CMAX, bool EXACT, int VEC, bool SOFT, bool RIGHT>
hipError_t launch_bwd_t(const Geometry& g, const BwdParams& prm, hipStream_t s) {
  if (g.var.vec != VEC) return hipErrorInvalidConfiguration;  // as in launch_fwd_t
  auto kern = bwd_kernel<T, CMAX, EXACT, VEC, SOFT, RIGHT>;
  if constexpr (has_fast<CMAX, EXACT>()) {
    // the hard gradient reads no targets: any target layout takes the fast path
    if (prm.act == kActSoftmax && (!SOFT || (prm.tk == kTgtLabels && g.moments))) {
      if (prm.stream)
        kern = prm.off ? bwd_kernel_fast<T, CMAX, VEC, SOFT, RIGHT, true, true>
                       : bwd_kernel_fast<T, CMAX, VEC, SOFT, RIGHT, false, true>;
      else
        kern = prm.off ? bwd_kernel_fast<T, CMAX, VEC, SOFT, RIGHT, true, false>
                       : bwd_kernel_fast<T, CMAX, VEC, SOFT, RIGHT, false, false>;
    }
  }
  if (g.lds_bwd > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)g.lds_bwd);
    if (e != hipSuccess) return e;
  }
  return launch(kern, g.nblk, g.lds_bwd, s, prm);
}

// Multi-level launches: the fast kernels only (softmax, class-index
// targets, C in {2, 3, 4, 16}, soft in the moments layout); every level
// has the same configuration, so one instantiation serves all of them.
template <typename T, int C, int VEC, bool SOFT, bool RIGHT>
hipError_t launch_fwd_levels_t(long long nblk, size_t lds, const FwdLevels& L, hipStream_t s) {
  if (L.nt > fast_bound<C, SOFT>()) return hipErrorInvalidConfiguration;
  auto kern = L.lv[0].off ? fwd_kernel_fast_levels<T, C, VEC, SOFT, RIGHT, true>
                          : fwd_kernel_fast_levels<T, C, VEC, SOFT, RIGHT, false>;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  return launch(kern, nblk, lds, s, L, L.nt);
}
template <typename T, int C, int VEC, bool SOFT, bool RIGHT>
hipError_t launch_bwd_levels_t(long long nblk, size_t lds, const BwdLevels& L, hipStream_t s) {
  auto kern = L.lv[0].off ? bwd_kernel_fast_levels<T, C, VEC, SOFT, RIGHT, true>
                          : bwd_kernel_fast_levels<T, C, VEC, SOFT, RIGHT, false>;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  return launch(kern, nblk, lds, s, L);
}

// VEC4: the vector width at C = 4 (the fast hard forward takes 2, make_geometry)
#define ACE_LEVELS_SWITCH(LAUNCH, T, SOFT, RIGHT, VEC4)               \
  switch (cmax) {                                                     \
    case 2: return LAUNCH<T, 2, 4, SOFT, RIGHT>(nblk, lds, L, s);       \
    case 3: return LAUNCH<T, 3, 4, SOFT, RIGHT>(nblk, lds, L, s);       \
    case 4: return LAUNCH<T, 4, (VEC4), SOFT, RIGHT>(nblk, lds, L, s);  \
    case 16: return LAUNCH<T, 16, 1, SOFT, RIGHT>(nblk, lds, L, s);     \
  }                                                                   \
  return hipErrorInvalidValue;

// Instantiates the per-variant switch for one (element type, binning, right).
#define ACE_VARIANT_SWITCH(LAUNCH, T, SOFT, RIGHT)                                   \
  const Variant v = g.var;                                                           \
  if (v.exact) {                                                                     \
    switch (v.cmax) {                                                                \
      case 1: return LAUNCH<T, 1, true, 4, SOFT, RIGHT>(g, p, s);                    \
      case 2: return LAUNCH<T, 2, true, 4, SOFT, RIGHT>(g, p, s);                    \
      case 3: return LAUNCH<T, 3, true, 4, SOFT, RIGHT>(g, p, s);                    \
      case 4: return LAUNCH<T, 4, true, 4, SOFT, RIGHT>(g, p, s);                    \
      case 16: return LAUNCH<T, 16, true, 1, SOFT, RIGHT>(g, p, s);                  \
    }                                                                                \
  } else {                                                                           \
    switch (v.cmax) {                                                                \
      case 8: return LAUNCH<T, 8, false, 1, SOFT, RIGHT>(g, p, s);                   \
      case 16: return LAUNCH<T, 16, false, 1, SOFT, RIGHT>(g, p, s);                 \
      case 32: return LAUNCH<T, 32, false, 1, SOFT, RIGHT>(g, p, s);                 \
      case 64: return LAUNCH<T, 64, false, 1, SOFT, RIGHT>(g, p, s);                 \
    }                                                                                \
  }                                                                                  \
  return hipErrorInvalidValue;

#define ACE_DEFINE_LAUNCHERS(T, SOFT, RIGHT)                                          \
  template <>                                                                        \
  hipError_t launch_variant_fwd<T, SOFT, RIGHT>(const Geometry& g, const FwdParams& p, \
                                                hipStream_t s) {                     \
    if constexpr (!SOFT)                                                             \
      if (g.var.exact && g.var.cmax == 4 && g.var.vec == 2)                          \
        return launch_fwd_t<T, 4, true, 2, SOFT, RIGHT>(g, p, s);                    \
    ACE_VARIANT_SWITCH(launch_fwd_t, T, SOFT, RIGHT)                                 \
  }                                                                                  \
  template <>                                                                        \
  hipError_t launch_variant_bwd<T, SOFT, RIGHT>(const Geometry& g, const BwdParams& p, \
                                                hipStream_t s) {                     \
    /* the generic backward for 9-15 channels runs the 32-channel kernel       \
       (soft 176 / hard 140 VGPRs against 272 / 253 for the 16-channel one) */  \
    if (!g.var.exact && g.var.cmax == 16)                                            \
      return launch_bwd_t<T, 32, false, 1, SOFT, RIGHT>(g, p, s);                    \
    /* the hard 5-8-channel backward: two voxels per lane (make_geometry) */      \
    if constexpr (!SOFT)                                                             \
      if (!g.var.exact && g.var.cmax == 8 && g.var.vec == 2)                         \
        return launch_bwd_t<T, 8, false, 2, SOFT, RIGHT>(g, p, s);                   \
    ACE_VARIANT_SWITCH(launch_bwd_t, T, SOFT, RIGHT)                                 \
  }                                                                                  \
  template <>                                                                        \
  hipError_t launch_levels_fwd<T, SOFT, RIGHT>(int cmax, long long nblk, size_t lds,   \
                                               const FwdLevels& L, hipStream_t s) {  \
    ACE_LEVELS_SWITCH(launch_fwd_levels_t, T, SOFT, RIGHT, (SOFT ? 4 : 2))           \
  }                                                                                  \
  template <>                                                                        \
  hipError_t launch_levels_bwd<T, SOFT, RIGHT>(int cmax, long long nblk, size_t lds,   \
                                               const BwdLevels& L, hipStream_t s) {  \
    ACE_LEVELS_SWITCH(launch_bwd_levels_t, T, SOFT, RIGHT, 4)                        \
  }

}  // namespace ace
