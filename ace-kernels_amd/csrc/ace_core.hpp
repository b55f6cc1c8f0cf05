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
// then publishes an integer partial; the last block of each group (ticket
// counter) sums its group into the final sums with integer atomics, and the
// last group's block runs the epilogue (d, coef, per-class error, jac, loss)
// and leaves counters and sums zero for the next call.
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
#include <stdint.h>

#include "ace_bins.hpp"
#include "ace_geometry.hpp"

namespace ace {

enum { kActNone = 0, kActSoftmax = 1, kActSigmoid = 2 };
enum { kRedMean = 0, kRedSum = 1, kRedNone = 2 };
enum { kTgtLabels = 0, kTgtOnehot = 1 };
enum { kReduceTree = 0, kReduceDirect = 1 };

// Packed hard-binning histogram word: count | label count | sum p.
//   bits [53, 64): voxels in the bin (<= 2047 per copy and block)
//   bits [42, 53): voxels of the bin whose label is this channel
//   bits [ 0, 42): sum of p in 30-bit fixed point (|sum| < 2^11)
constexpr int kShiftN = 53;
constexpr int kShiftG = 42;

struct FwdParams {
  const void* x;
  const void* tgt;
  int64_t N;
  int64_t tile_vox;
  int64_t tiles;
  int64_t gs;
  int64_t gpb;
  int B, C, off, K, act, tk, copies, vec_ok, ignore_empty, red;
  int mode;            // kReduceTree or kReduceDirect
  int epi_batch;       // batch indices per epilogue pass
  float empty_w;
  const float* btab;   // bucket table (K or 2K upper boundaries)
  const float* rtab;   // soft centre table (2K + 2)
  const float* clsw;   // C' class weights or null
  long long* part;     // [nblk][3][CK] block partials (tree mode)
  unsigned long long* fin;  // [B][3][CK] zeroed final sums (reset by the epilogue)
  int* ctr;            // [B * gpb + 1] zeroed ticket counters
  float* coef;
  float* d;
  float* jac;
  float* f;
  float* loss;
  double* stats;
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
// on MI355X); given y = RN(1 / b), two residual corrections of a * y give the
// IEEE quotient (Markstein's theorem), checked against '/' for 2e10 (a, b)
// pairs.  Used where b is a softmax sum in [1, C] or a soft-bin span in
// [2^-20, 2^14]; bit-identical to '/', at a quarter of its instructions.
__device__ __forceinline__ float rcp_rn(float b) {
  const float y = __builtin_amdgcn_rcpf(b);
  const float e = fmaf(-b, y, 1.0f);
  return fmaf(e, y, y);
}
__device__ __forceinline__ float div_rn(float a, float b, float y) {
  float q = a * y;
  float r = fmaf(-b, q, a);
  q = fmaf(r, y, q);
  r = fmaf(-b, q, a);
  return fmaf(r, y, q);
}

// ------------------------------------------------------------ activation

// In place: logits -> probabilities.  Softmax follows torch.softmax: max over
// channels, e_c = exp(x_c - max), s = sequential sum over c, p_c = e_c / s
// (IEEE quotient), with ROCm's accurate expf.  Sigmoid: 1 / (1 + exp(-x)).
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
        x[c] = expf(x[c] - m);
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
template <bool RIGHT, bool CLAMP = true>
__device__ __forceinline__ SoftW soft_assign(float p, int K, float n2f, const float* htab,
                                             const float* repl) {
  const int n2 = 2 * K;
  const int h = bucket<RIGHT, CLAMP>(p, n2f, n2, htab);
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

// Fixed-point value of a float32 term with |v| < 2 (2^30 scale, rounded to
// nearest even): exact for |v| >= 2^-7.
__device__ __forceinline__ long long fx(float v) {
  return (long long)(int)rintf(v * 1073741824.0f);
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
__device__ __forceinline__ void store_dev(long long* p, long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long load_dev(const unsigned long long* p) {
  return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this thread's global stores and atomics have completed.
__device__ __forceinline__ void wait_own_writes() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
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

// ------------------------------------------------------------ tiles

// One thread's slice of a step: VEC voxels of every channel, their labels or
// per-channel targets.  `load` issues the vector loads only; the values are
// first used by the binning, so a load can be in flight while another tile is
// processed.
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
  long long* g1;          // hard + per-channel targets: sum y          [CK][R]
  long long* w;           // soft: sum of weights                       [CK][R]
  long long* p;           // soft: sum of weight * p                    [CK][R]
  long long* g;           // soft: sum of weight * y                    [CK][R]
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
      float glw = 0.0f, grw = 0.0f;
#pragma unroll
      for (int c = 0; c < CMAX; ++c) {
        if (!(EXACT || c < nc) || c < off) continue;
        const SoftW w = soft_assign<RIGHT>(p[c], K, nf, btab, repl);
        const int sl = ((c - off) * K + w.l) * R + copy;
        const int sr = ((c - off) * K + w.r) * R + copy;
        lds_add(&H.w[sl], fx(w.lw));
        lds_add(&H.w[sr], fx(w.rw));
        lds_add(&H.p[sl], fx(w.lw * p[c]));
        lds_add(&H.p[sr], fx(w.rw * p[c]));
        if (labels) {
          const bool hit = lab[j] == c;
          gl = hit ? sl : gl;
          gr = hit ? sr : gr;
          glw = hit ? w.lw : glw;
          grw = hit ? w.rw : grw;
        } else {
          const float y = yv[c][j];
          if (y != 0.0f) {
            lds_add(&H.g[sl], fx(w.lw * y));
            lds_add(&H.g[sr], fx(w.rw * y));
          }
        }
      }
      if (labels && lab[j] >= off) {
        lds_add(&H.g[gl], fx(glw));
        lds_add(&H.g[gr], fx(grw));
      }
    }
  }
}

// ---- end of a forward block: publish the block's sums, and in the last
// block of a group / of the grid run the reductions and the epilogue
template <bool SOFT>
__device__ __forceinline__ void fwd_finish(const FwdParams& P, const Hist& H, unsigned char* hist,
                                           int CK, int CL, int b, int64_t tile, int64_t blk,
                                           bool labels) {
  const int tid = threadIdx.x;
  const int K = P.K;
  const int R = P.copies;
  // ---- block partial: sum the copies -> W3 = 3 x CK fixed-point values
  const int W3 = 3 * CK;
  const bool direct = P.mode == kReduceDirect;
  unsigned long long* fin_b = P.fin + (int64_t)b * W3;
  long long* part = P.part + blk * (int64_t)W3;
  for (int t = tid; t < CK; t += kThreads) {
    long long s0 = 0, s1 = 0, s2 = 0;
    for (int r = 0; r < R; ++r) {
      // skew the copy index by t: neighbouring threads read neighbouring banks
      const int slot = t * R + ((r + t) & (R - 1));
      if constexpr (!SOFT) {
        const unsigned long long a = H.a[slot];
        const unsigned long long hi = (a + (1ull << (kShiftG - 1))) >> kShiftG;
        s0 += (long long)((hi >> (kShiftN - kShiftG)) << kFrac);
        s1 += (long long)(a - (hi << kShiftG));
        s2 += labels ? (long long)((hi & ((1ull << (kShiftN - kShiftG)) - 1)) << kFrac)
                     : H.g1[slot];
      } else {
        s0 += H.w[slot];
        s1 += H.p[slot];
        s2 += H.g[slot];
      }
    }
    if (direct) {
      // integer atomics into the final sums: order-independent, deterministic
      if (s0) atomicAdd(&fin_b[t], (unsigned long long)s0);
      if (s1) atomicAdd(&fin_b[CK + t], (unsigned long long)s1);
      if (s2) atomicAdd(&fin_b[2 * CK + t], (unsigned long long)s2);
    } else {
      store_dev(&part[t], s0);
      store_dev(&part[CK + t], s1);
      store_dev(&part[2 * CK + t], s2);
    }
  }

  __shared__ int s_last;
  wait_own_writes();
  __syncthreads();
  const int64_t ngroups = (int64_t)P.B * P.gpb;  // index of the top counter
  int64_t arrivals = P.B * P.tiles;              // direct: every block reports
  if (!direct) {
    // ---- group ticket: the last block of the group sums the group's rows
    const int64_t g = tile / P.gs;
    const int64_t gidx = (int64_t)b * P.gpb + g;
    const int64_t gsize = min(P.gs, P.tiles - g * P.gs);
    if (tid == 0) {
      const int prev = ticket(&P.ctr[gidx]);
      s_last = (prev == (int)gsize - 1);
    }
    __syncthreads();
    if (!s_last) return;
    unsigned long long* acc = reinterpret_cast<unsigned long long*>(hist);
    for (int t = tid; t < W3; t += kThreads) acc[t] = 0ull;
    __syncthreads();
    // the group's partials are gsize contiguous rows of W3 values: read them
    // with every thread, four independent loads in flight per thread
    const unsigned long long* src = reinterpret_cast<const unsigned long long*>(
        P.part + ((int64_t)b * P.tiles + g * P.gs) * W3);
    const int total = (int)gsize * W3;
    for (int i0 = tid; i0 < total; i0 += 4 * kThreads) {
      unsigned long long v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * kThreads;
        v[u] = i < total ? load_dev(src + i) : 0ull;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (v[u]) lds_add(&acc[(i0 + u * kThreads) % W3], v[u]);
    }
    __syncthreads();
    for (int t = tid; t < W3; t += kThreads)
      if (acc[t]) atomicAdd(&fin_b[t], acc[t]);
    if (tid == 0) __hip_atomic_store(&P.ctr[gidx], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    wait_own_writes();
    __syncthreads();
    arrivals = ngroups;
  }
  // ---- top ticket: the last arrival runs the epilogue
  if (tid == 0) {
    const int prev = ticket(&P.ctr[ngroups]);
    s_last = (prev == (int)arrivals - 1);
  }
  __syncthreads();
  if (!s_last) return;

  // ---- epilogue (one block), `bc` batch indices at a time:
  // sums -> d, W, G per bin (LDS); per (b, c') row: K_ne, f, coef, jac
  const int bc = P.epi_batch;
  float* sd = reinterpret_cast<float*>(hist);
  float* sw = sd + (size_t)bc * CK;
  float* sg = sw + (size_t)bc * CK;
  float* sf = sg + (size_t)bc * CK;
  unsigned char* se = reinterpret_cast<unsigned char*>(sf + (size_t)bc * CK);
  const int64_t BCK = (int64_t)P.B * CK;
  const double dscale = 1.0 / 1073741824.0;
  const int rows = P.B * CL;
  float total = 0.0f;  // thread 0: sequential sum of the per-class errors
  for (int b0 = 0; b0 < P.B; b0 += bc) {
    const int nb = min(bc, P.B - b0);
    for (int i = tid; i < nb * CK; i += kThreads) {
      const int bb = b0 + i / CK;
      const int t = i - (i / CK) * CK;
      unsigned long long* fb = P.fin + (int64_t)bb * W3;
      const long long s0 = (long long)load_dev(&fb[t]);
      const long long s1 = (long long)load_dev(&fb[CK + t]);
      const long long s2 = (long long)load_dev(&fb[2 * CK + t]);
      // leave the accumulator zero for the next call
      __hip_atomic_store(&fb[t], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&fb[CK + t], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&fb[2 * CK + t], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const double Wd = (double)s0 * dscale;
      const double Pd = (double)s1 * dscale;
      const double Gd = (double)s2 * dscale;
      if (P.stats) {
        P.stats[(int64_t)bb * CK + t] = Wd;
        P.stats[BCK + (int64_t)bb * CK + t] = Pd;
        P.stats[2 * BCK + (int64_t)bb * CK + t] = Gd;
      }
      const float Wf = (float)Wd;
      const float Pf = (float)Pd;
      const float Gf = (float)Gd;
      const bool empty = SOFT ? !(Wf >= P.empty_w) : (Wf == 0.0f);
      const float dd = empty ? 0.0f : (Pf / Wf - Gf / Wf);
      sd[i] = dd;
      sw[i] = Wf;
      sg[i] = Gf;
      se[i] = empty ? 1 : 0;
      P.d[(int64_t)bb * CK + t] = dd;
    }
    __syncthreads();
    for (int r = tid; r < nb * CL; r += kThreads) {
      const int bb = b0 + r / CL;
      const int cl = r - (r / CL) * CL;
      const int base = (r / CL) * CK + cl * K;
      int kne = 0;
      float err = 0.0f, gsum = 0.0f;
      for (int k = 0; k < K; ++k) {
        if (!se[base + k]) {
          ++kne;
          err += fabsf(sd[base + k]);
        }
        gsum += sg[base + k];
      }
      const float fcls = kne > 0 ? err / (float)kne : __builtin_nanf("");
      const float present = gsum > 0.0f ? 1.0f : 0.0f;
      const float kf = (float)(kne > 0 ? kne : 1);
      for (int k = 0; k < K; ++k) {
        const float dd = sd[base + k];
        const float sgn = dd > 0.0f ? 1.0f : (dd < 0.0f ? -1.0f : 0.0f);
        P.coef[(int64_t)bb * CK + cl * K + k] = se[base + k] ? 0.0f : sgn / (kf * sw[base + k]);
      }
      const float w = P.clsw ? P.clsw[cl] : 1.0f;
      float fw = P.ignore_empty ? fcls * present : fcls;
      fw = fw * w;
      float jac = P.ignore_empty ? present * w : w;
      if (P.red == kRedMean) jac = jac / (float)rows;
      P.f[bb * CL + cl] = fw;
      P.jac[bb * CL + cl] = jac;
      sf[r] = fw;
    }
    __syncthreads();
    if (tid == 0)
      for (int r = 0; r < nb * CL; ++r) total += sf[r];
    __syncthreads();
  }
  if (tid == 0) {
    if (P.red == kRedMean) total = total / (float)rows;
    if (P.red != kRedNone) P.loss[0] = total;
    __hip_atomic_store(&P.ctr[ngroups], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
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
  const int nfull = P.vec_ok ? nvox / VEC * VEC : 0;

  // full vector steps, software-pipelined: the next step's loads are in flight
  // while the current step is binned (two buffers, unrolled by two)
  {
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
  fwd_finish<SOFT>(P, H, hist, CK, CL, b, tile, blk, labels);
}

// ------------------------------------------------------------ backward

// dL/dx of NV voxels, in place in xv (logits in, gradient out).
template <int CMAX, bool EXACT, int NV, bool SOFT, bool RIGHT>
__device__ __forceinline__ void bwd_voxels(const BwdParams& P, const float* btab, const float* repl,
                                           const float* scoef, const float* sdd, const float* sg,
                                           int nc, float (&xv)[CMAX][NV], const int (&lab)[NV],
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
        const float resid = p[c] - y;
        const float left = scoef[cl * K + w.l] * (w.lw - w.inv_span * (resid - sdd[cl * K + w.l]));
        const float rght = scoef[cl * K + w.r] * (w.rw + w.inv_span * (resid - sdd[cl * K + w.r]));
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
__global__ void __launch_bounds__(kThreads) bwd_kernel(const BwdParams P) {
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
  float* sdd = scoef + CK;
  float* sg = sdd + (SOFT ? CK : 0);
  load_tables(tabs, P.btab, P.rtab, n, SOFT ? 2 * K + 2 : 0);
  for (int t = tid; t < CK; t += kThreads) {
    scoef[t] = P.coef[(int64_t)b * CK + t];
    if (SOFT) sdd[t] = P.d[(int64_t)b * CK + t];
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
  const int nfull = P.vec_ok ? nvox / VEC * VEC : 0;

  // full vector steps, software-pipelined as in the forward
  {
    Tile<CMAX, VEC> ta, tb;
    const int stride = kThreads * VEC;
    // the hard gradient needs no targets: only the logits are loaded
    const bool need_tgt = SOFT;
    int v = tid * VEC;
    if (v < nfull) bwd_load<T, EXACT, CMAX, VEC>(ta, xt, lt, yt, N, v, nc, off, labels, need_tgt);
    for (; v < nfull; v += 2 * stride) {
      if (v + stride < nfull)
        bwd_load<T, EXACT, CMAX, VEC>(tb, xt, lt, yt, N, v + stride, nc, off, labels, need_tgt);
      bwd_voxels<CMAX, EXACT, VEC, SOFT, RIGHT>(P, btab, repl, scoef, sdd, sg, nc, ta.x, ta.lab, ta.y, labels);
#pragma unroll
      for (int c = 0; c < CMAX; ++c)
        if (EXACT || c < nc) store_vec<T, VEC>(dt + c * N + v, ta.x[c]);
      if (v + 2 * stride < nfull)
        bwd_load<T, EXACT, CMAX, VEC>(ta, xt, lt, yt, N, v + 2 * stride, nc, off, labels, need_tgt);
      if (v + stride < nfull) {
        bwd_voxels<CMAX, EXACT, VEC, SOFT, RIGHT>(P, btab, repl, scoef, sdd, sg, nc, tb.x, tb.lab, tb.y, labels);
#pragma unroll
        for (int c = 0; c < CMAX; ++c)
          if (EXACT || c < nc) store_vec<T, VEC>(dt + c * N + v + stride, tb.x[c]);
      }
    }
  }
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
    bwd_voxels<CMAX, EXACT, 1, SOFT, RIGHT>(P, btab, repl, scoef, sdd, sg, nc, xv, lab, yv, labels);
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

template <int C, int VEC>
struct FastTile {
  float x[C][VEC];
  long long lab[VEC];  // raw int64 labels, converted when used
};

template <typename T, int C, int VEC>
__device__ __forceinline__ void fast_load(FastTile<C, VEC>& t, const T* const (&xr)[C],
                                          const long long* lr, uint32_t v, bool with_labels) {
#pragma unroll
  for (int c = 0; c < C; ++c) load_vec<T, VEC>(xr[c] + v, t.x[c]);
  if (with_labels) {
    if constexpr (VEC % 2 == 0) {
#pragma unroll
      for (int j = 0; j < VEC; j += 2) {
        const longlong2 q = *reinterpret_cast<const longlong2*>(lr + v + j);
        t.lab[j] = q.x;
        t.lab[j + 1] = q.y;
      }
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) t.lab[j] = lr[v + j];
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

template <int C>
__device__ __forceinline__ void softmax_fast(float (&x)[C]) {
  float m = x[0];
#pragma unroll
  for (int c = 1; c < C; ++c) m = fmaxf(m, x[c]);
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    x[c] = expf(x[c] - m);
    s += x[c];
  }
  const float y = rcp_rn(s);
#pragma unroll
  for (int c = 0; c < C; ++c) x[c] = div_rn(x[c], s, y);
}

// One tile into the histogram copies.  hb[c]: this lane's copy of channel c's
// bin 0 (u64 words), bins `R` words apart (R = 1 << lr).
template <int C, int VEC, bool SOFT, bool RIGHT>
__device__ __forceinline__ void fast_accumulate(const FastTile<C, VEC>& t, const float* tab,
                                                const float* repl, int K, int off, int lr,
                                                unsigned long long* const (&hb)[C],
                                                const size_t words) {
  const float nf = (float)(SOFT ? 2 * K : K);
#pragma unroll
  for (int j = 0; j < VEC; ++j) {
    float p[C];
#pragma unroll
    for (int c = 0; c < C; ++c) p[c] = t.x[c][j];
    softmax_fast<C>(p);
    const uint32_t lab = fast_label<C>(t.lab[j]);
    if constexpr (!SOFT) {
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (c < off) continue;
        const int k = bucket<RIGHT, false>(p[c], nf, K, tab);
        const uint32_t q = (uint32_t)rintf(p[c] * 1073741824.0f);
        const uint32_t hi = (lab == (uint32_t)c) ? ((1u << (kShiftN - 32)) | (1u << (kShiftG - 32)))
                                                 : (1u << (kShiftN - 32));
        lds_add(hb[c] + ((size_t)k << lr), ((unsigned long long)hi << 32) | q);
      }
    } else {
      unsigned long long* gl = hb[0];
      unsigned long long* gr = hb[0];
      uint32_t glw = 0u, grw = 0u;
#pragma unroll
      for (int c = 0; c < C; ++c) {
        if (c < off) continue;
        const SoftW w = soft_assign<RIGHT, false>(p[c], K, nf, tab, repl);
        unsigned long long* sl = hb[c] + ((size_t)w.l << lr);
        unsigned long long* sr = hb[c] + ((size_t)w.r << lr);
        const uint32_t ql = (uint32_t)rintf(w.lw * 1073741824.0f);
        const uint32_t qr = (uint32_t)rintf(w.rw * 1073741824.0f);
        lds_add(sl, (unsigned long long)ql);
        lds_add(sr, (unsigned long long)qr);
        lds_add(sl + words, (unsigned long long)(uint32_t)rintf((w.lw * p[c]) * 1073741824.0f));
        lds_add(sr + words, (unsigned long long)(uint32_t)rintf((w.rw * p[c]) * 1073741824.0f));
        const bool hit = lab == (uint32_t)c;
        gl = hit ? sl : gl;
        gr = hit ? sr : gr;
        glw = hit ? ql : glw;
        grw = hit ? qr : grw;
      }
      if (lab != 0xffffffffu && lab >= (uint32_t)off) {
        lds_add(gl + 2 * words, (unsigned long long)glw);
        lds_add(gr + 2 * words, (unsigned long long)grw);
      }
    }
  }
}

template <typename T, int C, int VEC, bool SOFT, bool RIGHT>
__global__ void __launch_bounds__(kThreads) fwd_kernel_fast(const FwdParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* tabs = reinterpret_cast<float*>(smem);
  const int K = P.K;
  const int n = SOFT ? 2 * K : K;
  const int off = P.off;
  const int CL = C - off;
  const int CK = CL * K;
  const int R = P.copies;
  const int lr = __builtin_ctz((unsigned)R);
  const int tid = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int b = (int)(blk / P.tiles);
  const int64_t tile = blk - (int64_t)b * P.tiles;

  const size_t tab_floats = (size_t)(((n + 2) + (SOFT ? 2 * K + 2 : 0) + 3) / 4 * 4);
  unsigned char* hist = smem + tab_floats * 4;
  Hist H;
  H.a = reinterpret_cast<unsigned long long*>(hist);
  H.g1 = reinterpret_cast<long long*>(hist) + (size_t)CK * R;
  H.w = reinterpret_cast<long long*>(hist);
  H.p = H.w + (size_t)CK * R;
  H.g = H.p + (size_t)CK * R;
  const size_t hist_words = (hist_bytes_per_copy(CK, SOFT, true) * (size_t)R + 7) / 8;
  load_tables(tabs, P.btab, P.rtab, n, SOFT ? 2 * K + 2 : 0);
  {
    unsigned long long* h64 = reinterpret_cast<unsigned long long*>(hist);
    for (size_t i = tid; i < hist_words; i += kThreads) h64[i] = 0ull;
  }
  __syncthreads();
  const float* tab = tabs;
  const float* repl = tabs + n + 2;
  const int copy = tid & (R - 1);
  unsigned long long* hb[C];
#pragma unroll
  for (int c = 0; c < C; ++c)
    hb[c] = H.a + ((size_t)((c < off ? 0 : c - off) * K) << lr) + copy;

  const int64_t N = P.N;
  const int64_t t0 = tile * P.tile_vox;
  const int nvox = (int)min(P.tile_vox, N - t0);
  const T* xr[C];
#pragma unroll
  for (int c = 0; c < C; ++c)
    xr[c] = reinterpret_cast<const T*>(P.x) + ((int64_t)b * C + c) * N + t0;
  const long long* lr_ = reinterpret_cast<const long long*>(P.tgt) + (int64_t)b * N + t0;
  const size_t words = (size_t)CK * R;
  const int nfull = P.vec_ok ? nvox / VEC * VEC : 0;
  const int stride = kThreads * VEC;
  const int nsteps = nfull / stride;  // steps in which every thread has a full vector

  if (nsteps > 0) {
    FastTile<C, VEC> ta, tb;
    const uint32_t v0 = (uint32_t)(tid * VEC);
    fast_load<T, C, VEC>(ta, xr, lr_, v0, true);
    for (int i = 0; i < nsteps; i += 2) {
      const uint32_t va = v0 + (uint32_t)(i * stride);
      const uint32_t vb = (i + 1 < nsteps) ? va + (uint32_t)stride : va;
      fast_load<T, C, VEC>(tb, xr, lr_, vb, true);
      fast_accumulate<C, VEC, SOFT, RIGHT>(ta, tab, repl, K, off, lr, hb, words);
      const uint32_t vc = (i + 2 < nsteps) ? va + 2u * (uint32_t)stride : vb;
      fast_load<T, C, VEC>(ta, xr, lr_, vc, true);
      if (i + 1 < nsteps) fast_accumulate<C, VEC, SOFT, RIGHT>(tb, tab, repl, K, off, lr, hb, words);
    }
  }
  // remaining full vectors (not every thread has one), then single voxels
  for (int v = nsteps * stride + tid * VEC; v < nfull; v += stride) {
    FastTile<C, VEC> t;
    fast_load<T, C, VEC>(t, xr, lr_, (uint32_t)v, true);
    fast_accumulate<C, VEC, SOFT, RIGHT>(t, tab, repl, K, off, lr, hb, words);
  }
  for (int v = nfull + tid; v < nvox; v += kThreads) {
    FastTile<C, 1> t;
    fast_load<T, C, 1>(t, xr, lr_, (uint32_t)v, true);
    fast_accumulate<C, 1, SOFT, RIGHT>(t, tab, repl, K, off, lr, hb, words);
  }
  __syncthreads();
  fwd_finish<SOFT>(P, H, hist, CK, CL, b, tile, blk, true);
}

// Backward of one tile, in place in t.x (logits in, gradient out).
template <int C, int VEC, bool SOFT, bool RIGHT>
__device__ __forceinline__ void fast_backward(FastTile<C, VEC>& t, const float* tab,
                                              const float* repl, const float* scoef,
                                              const float* sdd, const float* sg, int K,
                                              int off) {
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
      if (c < off) continue;
      const int cl = c - off;
      if constexpr (!SOFT) {
        const int k = bucket<RIGHT, false>(p[c], nf, K, tab);
        gp[c] = scoef[cl * K + k] * sg[cl];
      } else {
        const SoftW w = soft_assign<RIGHT, false>(p[c], K, nf, tab, repl);
        const float y = lab == (uint32_t)c ? 1.0f : 0.0f;
        const float resid = p[c] - y;
        const float left = scoef[cl * K + w.l] * (w.lw - w.inv_span * (resid - sdd[cl * K + w.l]));
        const float rght = scoef[cl * K + w.r] * (w.rw + w.inv_span * (resid - sdd[cl * K + w.r]));
        gp[c] = sg[cl] * (left + rght);
      }
    }
    float dot = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) dot += gp[c] * p[c];
#pragma unroll
    for (int c = 0; c < C; ++c) t.x[c][j] = p[c] * (gp[c] - dot);
  }
}

template <typename T, int C, int VEC, bool SOFT, bool RIGHT>
__global__ void __launch_bounds__(kThreads) bwd_kernel_fast(const BwdParams P) {
  extern __shared__ __align__(16) unsigned char smem[];
  float* tabs = reinterpret_cast<float*>(smem);
  const int K = P.K;
  const int n = SOFT ? 2 * K : K;
  const int off = P.off;
  const int CL = C - off;
  const int CK = CL * K;
  const int tid = threadIdx.x;
  const int64_t blk = blockIdx.x;
  const int b = (int)(blk / P.tiles);
  const int64_t tile = blk - (int64_t)b * P.tiles;

  const size_t tab_floats = (size_t)(((n + 2) + (SOFT ? 2 * K + 2 : 0) + 3) / 4 * 4);
  float* scoef = tabs + tab_floats;
  float* sdd = scoef + CK;
  float* sg = sdd + (SOFT ? CK : 0);
  load_tables(tabs, P.btab, P.rtab, n, SOFT ? 2 * K + 2 : 0);
  for (int i = tid; i < CK; i += kThreads) {
    scoef[i] = P.coef[(int64_t)b * CK + i];
    if (SOFT) sdd[i] = P.d[(int64_t)b * CK + i];
  }
  for (int i = tid; i < CL; i += kThreads) {
    const float go = P.go_per_class ? P.go[b * CL + i] : P.go[0];
    sg[i] = P.jac[b * CL + i] * go;
  }
  __syncthreads();
  const float* tab = tabs;
  const float* repl = tabs + n + 2;

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

  if (nsteps > 0) {
    FastTile<C, VEC> ta, tb;
    const uint32_t v0 = (uint32_t)(tid * VEC);
    fast_load<T, C, VEC>(ta, xr, lr_, v0, SOFT);
    for (int i = 0; i < nsteps; i += 2) {
      const uint32_t va = v0 + (uint32_t)(i * stride);
      const uint32_t vb = (i + 1 < nsteps) ? va + (uint32_t)stride : va;
      fast_load<T, C, VEC>(tb, xr, lr_, vb, SOFT);
      fast_backward<C, VEC, SOFT, RIGHT>(ta, tab, repl, scoef, sdd, sg, K, off);
#pragma unroll
      for (int c = 0; c < C; ++c) store_vec<T, VEC>(dr[c] + va, ta.x[c]);
      const uint32_t vc = (i + 2 < nsteps) ? va + 2u * (uint32_t)stride : vb;
      fast_load<T, C, VEC>(ta, xr, lr_, vc, SOFT);
      if (i + 1 < nsteps) {
        fast_backward<C, VEC, SOFT, RIGHT>(tb, tab, repl, scoef, sdd, sg, K, off);
#pragma unroll
        for (int c = 0; c < C; ++c) store_vec<T, VEC>(dr[c] + vb, tb.x[c]);
      }
    }
  }
  for (int v = nsteps * stride + tid * VEC; v < nfull; v += stride) {
    FastTile<C, VEC> t;
    fast_load<T, C, VEC>(t, xr, lr_, (uint32_t)v, SOFT);
    fast_backward<C, VEC, SOFT, RIGHT>(t, tab, repl, scoef, sdd, sg, K, off);
#pragma unroll
    for (int c = 0; c < C; ++c) store_vec<T, VEC>(dr[c] + v, t.x[c]);
  }
  for (int v = nfull + tid; v < nvox; v += kThreads) {
    FastTile<C, 1> t;
    fast_load<T, C, 1>(t, xr, lr_, (uint32_t)v, SOFT);
    fast_backward<C, 1, SOFT, RIGHT>(t, tab, repl, scoef, sdd, sg, K, off);
#pragma unroll
    for (int c = 0; c < C; ++c) dr[c][v] = from_f32<T>(t.x[c][0]);
  }
}

// ------------------------------------------------------------ launchers

template <typename T, bool SOFT, bool RIGHT>
hipError_t launch_variant_fwd(const Geometry& g, const FwdParams& prm, hipStream_t s);
template <typename T, bool SOFT, bool RIGHT>
hipError_t launch_variant_bwd(const Geometry& g, const BwdParams& prm, hipStream_t s);

// The fast kernels serve softmax with class-index targets for C in {2, 3, 4, 16}.
template <int CMAX, bool EXACT>
constexpr bool has_fast() {
  return EXACT && (CMAX == 2 || CMAX == 3 || CMAX == 4 || CMAX == 16);
}

template <typename T, int CMAX, bool EXACT, int VEC, bool SOFT, bool RIGHT>
hipError_t launch_fwd_t(const Geometry& g, const FwdParams& prm, hipStream_t s) {
  auto kern = fwd_kernel<T, CMAX, EXACT, VEC, SOFT, RIGHT>;
  if constexpr (has_fast<CMAX, EXACT>()) {
    if (prm.act == kActSoftmax && prm.tk == kTgtLabels)
      kern = fwd_kernel_fast<T, CMAX, VEC, SOFT, RIGHT>;
  }
  if (g.lds_fwd > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)g.lds_fwd);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)g.nblk), dim3(kThreads), g.lds_fwd, s, prm);
  return hipGetLastError();
}

template <typename T, int CMAX, bool EXACT, int VEC, bool SOFT, bool RIGHT>
hipError_t launch_bwd_t(const Geometry& g, const BwdParams& prm, hipStream_t s) {
  auto kern = bwd_kernel<T, CMAX, EXACT, VEC, SOFT, RIGHT>;
  if constexpr (has_fast<CMAX, EXACT>()) {
    // the hard gradient reads no targets: any target layout takes the fast path
    if (prm.act == kActSoftmax && (!SOFT || prm.tk == kTgtLabels))
      kern = bwd_kernel_fast<T, CMAX, VEC, SOFT, RIGHT>;
  }
  if (g.lds_bwd > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)g.lds_bwd);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)g.nblk), dim3(kThreads), g.lds_bwd, s, prm);
  return hipGetLastError();
}

// Instantiates the per-variant switch for one (element type, binning, right).
#define ACE_VARIANT_SWITCH(LAUNCH, T, SOFT, RIGHT)                                   \
  const Variant v = g.var;                                                           \
  if (v.exact) {                                                                     \
    switch (v.cmax) {                                                                \
      case 1: return LAUNCH<T, 1, true, 4, SOFT, RIGHT>(g, p, s);                    \
      case 2: return LAUNCH<T, 2, true, 4, SOFT, RIGHT>(g, p, s);                    \
      case 3: return LAUNCH<T, 3, true, 4, SOFT, RIGHT>(g, p, s);                    \
      case 4: return LAUNCH<T, 4, true, 4, SOFT, RIGHT>(g, p, s);                    \
      case 16: return LAUNCH<T, 16, true, 2, SOFT, RIGHT>(g, p, s);                  \
    }                                                                                \
  } else {                                                                           \
    switch (v.cmax) {                                                                \
      case 8: return LAUNCH<T, 8, false, 4, SOFT, RIGHT>(g, p, s);                   \
      case 16: return LAUNCH<T, 16, false, 4, SOFT, RIGHT>(g, p, s);                 \
      case 32: return LAUNCH<T, 32, false, 1, SOFT, RIGHT>(g, p, s);                 \
      case 64: return LAUNCH<T, 64, false, 1, SOFT, RIGHT>(g, p, s);                 \
    }                                                                                \
  }                                                                                  \
  return hipErrorInvalidValue;

#define ACE_DEFINE_LAUNCHERS(T, SOFT, RIGHT)                                          \
  template <>                                                                        \
  hipError_t launch_variant_fwd<T, SOFT, RIGHT>(const Geometry& g, const FwdParams& p, \
                                                hipStream_t s) {                     \
    ACE_VARIANT_SWITCH(launch_fwd_t, T, SOFT, RIGHT)                                 \
  }                                                                                  \
  template <>                                                                        \
  hipError_t launch_variant_bwd<T, SOFT, RIGHT>(const Geometry& g, const BwdParams& p, \
                                                hipStream_t s) {                     \
    ACE_VARIANT_SWITCH(launch_bwd_t, T, SOFT, RIGHT)                                 \
  }

}  // namespace ace
