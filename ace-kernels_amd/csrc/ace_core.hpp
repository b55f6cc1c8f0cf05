// mL1-ACE forward / backward kernels for CDNA4 (gfx950).
//
// Forward (one launch): every block streams a tile of voxels of one batch
// index, computes the channel softmax (or sigmoid) in registers, bins every
// loss channel (hard: one bin; soft: two neighbouring bins with interpolation
// weights) and accumulates the per-bin sums W, P, G into LDS histograms.  The
// sums are fixed-point integers (30 fraction bits) added with LDS integer
// atomics, so they are exact for the float32 terms >= 2^-7 (and within 2^-31
// per term below) and independent of the order of addition: the result is
// bitwise deterministic with no float atomics.  Each wave lane adds into copy
// (lane % copies) of the histogram; with 16 copies laid out bin-major the 16
// lanes an LDS cycle serves always hit 16 distinct bank pairs, whatever their
// bins, so the atomics never conflict.  Blocks then write integer partials;
// the last block of each group (ticket counter) sums its group, and the last
// group's block sums the groups and runs the epilogue (d, coef, per-class
// error, jac, loss).  Counters are reset by the blocks that consume them.
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

struct FwdParams {
  const void* x;
  const void* tgt;
  int64_t N;
  int64_t tile_vox;
  int64_t tiles;
  int64_t gs;
  int64_t gpb;
  int B, C, off, K, act, tk, right, copies, vec_ok, ignore_empty, red;
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
  int B, C, off, K, act, tk, right, vec_ok, go_per_class;
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

template <int VEC>
__device__ __forceinline__ void load_labels(const long long* __restrict__ p, int C,
                                            bool aligned, int nv, int (&lab)[VEC]) {
  if (aligned && nv == VEC && (VEC % 2) == 0) {
#pragma unroll
    for (int j = 0; j < VEC; j += 2) {
      const longlong2 t = *reinterpret_cast<const longlong2*>(p + j);
      lab[j] = label_channel(t.x, C);
      lab[j + 1] = label_channel(t.y, C);
    }
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) lab[j] = j < nv ? label_channel(p[j], C) : -1;
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void load_row(const T* __restrict__ p, bool aligned, int nv,
                                         float (&out)[VEC]) {
  if (aligned && nv == VEC) {
    load_vec<T, VEC>(p, out);
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) out[j] = j < nv ? to_f32<T>(p[j]) : 0.0f;
  }
}

// ------------------------------------------------------------ activation

// In place: logits -> probabilities.  Softmax follows torch.softmax: max over
// channels, e_c = exp(x_c - max), s = sequential sum over c, p_c = e_c / s
// with IEEE division (hipcc's default for '/'), and ROCm's accurate expf.
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
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) x[c] = x[c] / s;
  } else if (act == kActSigmoid) {
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) x[c] = 1.0f / (1.0f + expf(-x[c]));
  }
}

// ------------------------------------------------------------ binning

struct SoftW {
  int l, r;
  float lw, rw, span;
};

// Soft assignment of common.py:43-61: half-bin index h against the 2K upper
// half boundaries; bins l = max(h-1,0)/2, r = min(h+1,2K-1)/2; distances to
// the replicated centres (sentinels +-1e4); lw = rd/S, rw = ld/S (IEEE).
__device__ __forceinline__ SoftW soft_assign(float p, int K, float n2f, const float* htab,
                                             const float* repl, bool right) {
  const int n2 = 2 * K;
  const int h = bucket(p, n2f, n2, htab, right);
  SoftW w;
  w.l = max(h - 1, 0) >> 1;
  w.r = min(h + 1, n2 - 1) >> 1;
  const float ld = p - repl[h];
  const float rd = repl[h + 2] - p;
  w.span = ld + rd;
  w.lw = rd / w.span;
  w.rw = ld / w.span;
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
__device__ __forceinline__ void lds_add(unsigned int* p, unsigned int v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
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
// LDS; returns pointers to both.
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

// ------------------------------------------------------------ forward

// Sums of a voxel's contribution into histogram copy `copy`.
//  hard: A[(c'K + k) * R + copy] += (1 << 48) + fx(p)   (count and sum p)
//        G: labels -> u32 count at the label channel's bin;
//           one-hot -> i64 fx(y) per channel with y != 0
//  soft: W, P, G i64 at bins l and r.
template <typename T, int CMAX, bool EXACT, int VEC, bool SOFT>
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
  const float nf = (float)n;
  const bool right = P.right != 0;
  const bool labels = P.tk == kTgtLabels;

  const size_t tab_floats = (size_t)(((n + 2) + (SOFT ? 2 * K + 2 : 0) + 3) / 4 * 4);
  unsigned char* hist = smem + tab_floats * 4;
  unsigned long long* histA = reinterpret_cast<unsigned long long*>(hist);       // hard
  unsigned int* histGc = reinterpret_cast<unsigned int*>(hist + (size_t)CK * R * 8);
  long long* histGf = reinterpret_cast<long long*>(hist + (size_t)CK * R * 8);
  long long* histW = reinterpret_cast<long long*>(hist);                         // soft
  long long* histP = histW + (size_t)CK * R;
  long long* histG = histP + (size_t)CK * R;
  const size_t hist_words =
      (hist_bytes_per_copy(CK, SOFT, labels) * (size_t)R + 7) / 8;

  load_tables(tabs, P.btab, P.rtab, n, SOFT ? 2 * K + 2 : 0);
  {
    unsigned long long* h64 = reinterpret_cast<unsigned long long*>(hist);
    for (size_t i = tid; i < hist_words; i += kThreads) h64[i] = 0ull;
  }
  __syncthreads();
  const float* btab = tabs;
  const float* repl = tabs + n + 2;
  const int copy = tid & (R - 1);

  const T* xb = reinterpret_cast<const T*>(P.x) + (int64_t)b * nc * P.N;
  const long long* lb = reinterpret_cast<const long long*>(P.tgt) + (int64_t)b * P.N;
  const float* yb = reinterpret_cast<const float*>(P.tgt) + (int64_t)b * nc * P.N;
  const int64_t v0 = tile * P.tile_vox;
  const int64_t v1 = min(v0 + P.tile_vox, P.N);
  const bool aligned = P.vec_ok != 0;

  for (int64_t v = v0 + (int64_t)tid * VEC; v < v1; v += (int64_t)kThreads * VEC) {
    const int nv = (int)min((int64_t)VEC, v1 - v);
    float xv[CMAX][VEC];
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) load_row<T, VEC>(xb + (int64_t)c * P.N + v, aligned, nv, xv[c]);
    int lab[VEC];
    float yv[CMAX][VEC];
    if (labels) {
      load_labels<VEC>(lb + v, nc, aligned, nv, lab);
    } else {
#pragma unroll
      for (int c = 0; c < CMAX; ++c)
        if ((EXACT || c < nc) && c >= off) load_row<float, VEC>(yb + (int64_t)c * P.N + v, aligned, nv, yv[c]);
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      if (j >= nv) break;
      float p[CMAX];
#pragma unroll
      for (int c = 0; c < CMAX; ++c) p[c] = xv[c][j];
      activate<CMAX, EXACT>(p, nc, P.act);
      if constexpr (!SOFT) {
        int kl = 0;
#pragma unroll
        for (int c = 0; c < CMAX; ++c) {
          if (!(EXACT || c < nc) || c < off) continue;
          const int k = bucket(p[c], nf, n, btab, right);
          const int slot = ((c - off) * K + k) * R + copy;
          const unsigned long long add =
              (1ull << 48) + (unsigned long long)fx(p[c]);
          lds_add(&histA[slot], add);
          if (labels) {
            kl = (lab[j] == c) ? k : kl;
          } else {
            const float y = yv[c][j];
            if (y != 0.0f) lds_add(reinterpret_cast<unsigned long long*>(&histGf[slot]),
                                   (unsigned long long)fx(y));
          }
        }
        if (labels && lab[j] >= off) {
          const int slot = ((lab[j] - off) * K + kl) * R + copy;
          lds_add(&histGc[slot], 1u);
        }
      } else {
        int gl = 0, gr = 0;
        float glw = 0.0f, grw = 0.0f;
#pragma unroll
        for (int c = 0; c < CMAX; ++c) {
          if (!(EXACT || c < nc) || c < off) continue;
          const SoftW w = soft_assign(p[c], K, nf, btab, repl, right);
          const int sl = ((c - off) * K + w.l) * R + copy;
          const int sr = ((c - off) * K + w.r) * R + copy;
          lds_add(reinterpret_cast<unsigned long long*>(&histW[sl]), (unsigned long long)fx(w.lw));
          lds_add(reinterpret_cast<unsigned long long*>(&histW[sr]), (unsigned long long)fx(w.rw));
          lds_add(reinterpret_cast<unsigned long long*>(&histP[sl]), (unsigned long long)fx(w.lw * p[c]));
          lds_add(reinterpret_cast<unsigned long long*>(&histP[sr]), (unsigned long long)fx(w.rw * p[c]));
          if (labels) {
            const bool hit = lab[j] == c;
            gl = hit ? sl : gl;
            gr = hit ? sr : gr;
            glw = hit ? w.lw : glw;
            grw = hit ? w.rw : grw;
          } else {
            const float y = yv[c][j];
            if (y != 0.0f) {
              lds_add(reinterpret_cast<unsigned long long*>(&histG[sl]), (unsigned long long)fx(w.lw * y));
              lds_add(reinterpret_cast<unsigned long long*>(&histG[sr]), (unsigned long long)fx(w.rw * y));
            }
          }
        }
        if (labels && lab[j] >= off) {
          lds_add(reinterpret_cast<unsigned long long*>(&histG[gl]), (unsigned long long)fx(glw));
          lds_add(reinterpret_cast<unsigned long long*>(&histG[gr]), (unsigned long long)fx(grw));
        }
      }
    }
  }
  __syncthreads();

  // ---- block partial: sum the copies -> W3 = 3 x CK fixed-point values
  const int W3 = 3 * CK;
  const bool direct = P.mode == kReduceDirect;
  unsigned long long* fin_b = P.fin + (int64_t)b * W3;
  long long* part = P.part + blk * (int64_t)W3;
  for (int t = tid; t < CK; t += kThreads) {
    long long s0 = 0, s1 = 0, s2 = 0;
    for (int r = 0; r < R; ++r) {
      const int slot = t * R + r;
      if constexpr (!SOFT) {
        const unsigned long long a = histA[slot];
        const unsigned long long cnt = (a + (1ull << 47)) >> 48;
        s0 += (long long)(cnt << kFrac);
        s1 += (long long)(a - (cnt << 48));
        s2 += labels ? ((long long)histGc[slot] << kFrac) : histGf[slot];
      } else {
        s0 += histW[slot];
        s1 += histP[slot];
        s2 += histG[slot];
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

// ------------------------------------------------------------ backward

template <typename T, int CMAX, bool EXACT, int VEC, bool SOFT>
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
  const float nf = (float)n;
  const bool right = P.right != 0;
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

  const T* xb = reinterpret_cast<const T*>(P.x) + (int64_t)b * nc * P.N;
  T* db = reinterpret_cast<T*>(P.dx) + (int64_t)b * nc * P.N;
  const long long* lb = reinterpret_cast<const long long*>(P.tgt) + (int64_t)b * P.N;
  const float* yb = reinterpret_cast<const float*>(P.tgt) + (int64_t)b * nc * P.N;
  const int64_t v0 = tile * P.tile_vox;
  const int64_t v1 = min(v0 + P.tile_vox, P.N);
  const bool aligned = P.vec_ok != 0;

  for (int64_t v = v0 + (int64_t)tid * VEC; v < v1; v += (int64_t)kThreads * VEC) {
    const int nv = (int)min((int64_t)VEC, v1 - v);
    float xv[CMAX][VEC];
#pragma unroll
    for (int c = 0; c < CMAX; ++c)
      if (EXACT || c < nc) load_row<T, VEC>(xb + (int64_t)c * P.N + v, aligned, nv, xv[c]);
    int lab[VEC];
    float yv[CMAX][VEC];
    if (SOFT) {
      if (labels) {
        load_labels<VEC>(lb + v, nc, aligned, nv, lab);
      } else {
#pragma unroll
        for (int c = 0; c < CMAX; ++c)
          if ((EXACT || c < nc) && c >= off) load_row<float, VEC>(yb + (int64_t)c * P.N + v, aligned, nv, yv[c]);
      }
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
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
          const int k = bucket(p[c], nf, n, btab, right);
          gp[c] = scoef[cl * K + k] * sg[cl];
        } else {
          const SoftW w = soft_assign(p[c], K, nf, btab, repl, right);
          const float y = labels ? (lab[j] == c ? 1.0f : 0.0f) : yv[c][j];
          const float inv = 1.0f / w.span;
          const float resid = p[c] - y;
          const float left = scoef[cl * K + w.l] * (w.lw - inv * (resid - sdd[cl * K + w.l]));
          const float rght = scoef[cl * K + w.r] * (w.rw + inv * (resid - sdd[cl * K + w.r]));
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
#pragma unroll
    for (int c = 0; c < CMAX; ++c) {
      if (!(EXACT || c < nc)) continue;
      T* dst = db + (int64_t)c * P.N + v;
      if (aligned && nv == VEC) {
        store_vec<T, VEC>(dst, xv[c]);
      } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          if (j < nv) dst[j] = from_f32<T>(xv[c][j]);
      }
    }
  }
}

// ------------------------------------------------------------ launchers

template <typename T, bool SOFT>
hipError_t launch_variant_fwd(const Geometry& g, const FwdParams& prm, hipStream_t s);
template <typename T, bool SOFT>
hipError_t launch_variant_bwd(const Geometry& g, const BwdParams& prm, hipStream_t s);

template <typename T, int CMAX, bool EXACT, int VEC, bool SOFT>
hipError_t launch_fwd_t(const Geometry& g, const FwdParams& prm, hipStream_t s) {
  auto kern = fwd_kernel<T, CMAX, EXACT, VEC, SOFT>;
  if (g.lds_fwd > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)g.lds_fwd);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)g.nblk), dim3(kThreads), g.lds_fwd, s, prm);
  return hipGetLastError();
}

template <typename T, int CMAX, bool EXACT, int VEC, bool SOFT>
hipError_t launch_bwd_t(const Geometry& g, const BwdParams& prm, hipStream_t s) {
  auto kern = bwd_kernel<T, CMAX, EXACT, VEC, SOFT>;
  if (g.lds_bwd > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)g.lds_bwd);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)g.nblk), dim3(kThreads), g.lds_bwd, s, prm);
  return hipGetLastError();
}

// Instantiates the per-variant switch for one (element type, binning).
#define ACE_DEFINE_LAUNCHERS(T, SOFT)                                                  \
  template <>                                                                        \
  hipError_t launch_variant_fwd<T, SOFT>(const Geometry& g, const FwdParams& p,      \
                                         hipStream_t s) {                            \
    const Variant v = g.var;                                                         \
    if (v.exact) {                                                                   \
      switch (v.cmax) {                                                              \
        case 1: return launch_fwd_t<T, 1, true, 4, SOFT>(g, p, s);                   \
        case 2: return launch_fwd_t<T, 2, true, 4, SOFT>(g, p, s);                   \
        case 3: return launch_fwd_t<T, 3, true, 4, SOFT>(g, p, s);                   \
        case 4: return launch_fwd_t<T, 4, true, 4, SOFT>(g, p, s);                   \
        case 16: return launch_fwd_t<T, 16, true, 4, SOFT>(g, p, s);                 \
      }                                                                              \
    } else {                                                                         \
      switch (v.cmax) {                                                              \
        case 8: return launch_fwd_t<T, 8, false, 4, SOFT>(g, p, s);                  \
        case 16: return launch_fwd_t<T, 16, false, 4, SOFT>(g, p, s);                \
        case 32: return launch_fwd_t<T, 32, false, 1, SOFT>(g, p, s);                \
        case 64: return launch_fwd_t<T, 64, false, 1, SOFT>(g, p, s);                \
      }                                                                              \
    }                                                                                \
    return hipErrorInvalidValue;                                                     \
  }                                                                                  \
  template <>                                                                        \
  hipError_t launch_variant_bwd<T, SOFT>(const Geometry& g, const BwdParams& p,      \
                                         hipStream_t s) {                            \
    const Variant v = g.var;                                                         \
    if (v.exact) {                                                                   \
      switch (v.cmax) {                                                              \
        case 1: return launch_bwd_t<T, 1, true, 4, SOFT>(g, p, s);                   \
        case 2: return launch_bwd_t<T, 2, true, 4, SOFT>(g, p, s);                   \
        case 3: return launch_bwd_t<T, 3, true, 4, SOFT>(g, p, s);                   \
        case 4: return launch_bwd_t<T, 4, true, 4, SOFT>(g, p, s);                   \
        case 16: return launch_bwd_t<T, 16, true, 4, SOFT>(g, p, s);                 \
      }                                                                              \
    } else {                                                                         \
      switch (v.cmax) {                                                              \
        case 8: return launch_bwd_t<T, 8, false, 4, SOFT>(g, p, s);                  \
        case 16: return launch_bwd_t<T, 16, false, 4, SOFT>(g, p, s);                \
        case 32: return launch_bwd_t<T, 32, false, 1, SOFT>(g, p, s);                \
        case 64: return launch_bwd_t<T, 64, false, 1, SOFT>(g, p, s);                \
      }                                                                              \
    }                                                                                \
    return hipErrorInvalidValue;                                                     \
  }

}  // namespace ace
