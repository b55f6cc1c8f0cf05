// Float64 path of the loss: float64 logits, every quantity computed in
// double, outputs in double (ace_forward_f64 / ace_backward_f64, declared in
// include/ace_hip.h).
//
// The reference sends float64 input to its handwritten "recompute" backward
// in torch (src/ace_kernels/impls/v6_triton.py:226-227 ->
// impls/v2_autograd.py:196-236): softmax / sigmoid in float64
// (common.py:85-140), bins by torch.bucketize against the float32 tables
// converted to float64 (common.py:17-25, 43-61; binning.py:54-116), the
// epilogue in float64 (binning.py:127-147, v2_autograd.py:66-76) and the
// gradient of v2_autograd.py:88-118.  These kernels compute the same
// quantities in the same precision; only the order of float64 additions
// differs (fixed here: results are bit-identical run to run).
//
// Forward: block (b, tile) of 64 x `waves` threads.  Every wave walks its
// own run of voxels one voxel per iteration with lane c holding channel c
// (C <= 64): the softmax is a wave max and a wave sum, and lane c adds its
// channel's (W, P, G) contributions into row c of the wave's own LDS
// histogram -- no two lanes write one word, so no atomics.  The block adds its
// waves' histograms in wave order, writes the block's partial sums with
// device-coherent stores, and takes a ticket; the last block of batch index b
// adds the partials in tile order, runs the epilogue, and the last batch
// epilogue (a second ticket) adds the per-class errors into the loss in
// (b, c') order.  Every read partial and counter is set back to zero, so the
// workspace is left zero like the float32 kernels' (ace_workspace_bytes).
//
// Backward: one thread per voxel, channels in three passes (softmax max and
// sum; sum of p * dL/dp; dx), recomputing p instead of holding C values.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ace_core.hpp"
#include "ace_hip.h"

namespace ace {
namespace f64 {

constexpr size_t kMaxLds64 = 160 * 1024;
// Static LDS of fwd64_kernel (s_rows: 64 doubles, s_last: one int, 16-byte
// aligned); its dynamic LDS must fit beside it.
constexpr size_t kFwdStaticLds64 = 64 * sizeof(double) + 16;
constexpr size_t kMaxFwdDynLds64 = kMaxLds64 - kFwdStaticLds64;
constexpr int kMaxTiles64 = 256;  // blocks per batch index: the last block reads them all

struct Geo64 {
  int C, CL, off, K, ck, nv;  // nv = 3 C'K values per histogram (W, P, G)
  int64_t B, N;
  int waves;          // waves per block: the LDS holds one histogram per wave
  int64_t wave_vox;   // voxels per wave
  int64_t tile_vox;   // voxels per block
  int64_t tiles;      // blocks per batch index
  int ntab;           // double table entries: K edges, or 2K half edges + 2K + 2 centres
  size_t tab_bytes;
  size_t lds;
  size_t off_part, off_lossp, ws_bytes;
};

inline Geo64 geometry(int64_t B, int64_t C, int64_t N, int K, bool soft, bool include_background) {
  Geo64 g{};
  g.C = (int)C;
  g.off = (!include_background && C > 1) ? 1 : 0;
  g.CL = g.C - g.off;
  g.K = K;
  g.ck = g.CL * K;
  g.nv = 3 * g.ck;
  g.B = B;
  g.N = N;
  g.ntab = soft ? 4 * K + 2 : K;
  g.tab_bytes = align_up((size_t)g.ntab * sizeof(double), 16);
  g.waves = 0;
  for (int w : {4, 2, 1}) {
    if (g.tab_bytes + (size_t)w * g.nv * sizeof(double) <= kMaxFwdDynLds64) {
      g.waves = w;
      break;
    }
  }
  g.lds = g.tab_bytes + (size_t)(g.waves > 0 ? g.waves : 1) * g.nv * sizeof(double);
  const int64_t n = N > 0 ? N : 1;
  g.wave_vox = cdiv(n, (int64_t)kMaxTiles64 * (g.waves > 0 ? g.waves : 1));
  g.tile_vox = g.wave_vox * (g.waves > 0 ? g.waves : 1);
  g.tiles = cdiv(n, g.tile_vox);
  const int64_t counters = B + 1;  // one per batch index, then the loss
  g.off_part = align_up((size_t)counters * kCtrStride * sizeof(int), 256);
  g.off_lossp = align_up(g.off_part + (size_t)(B * g.tiles * g.nv) * sizeof(double), 256);
  g.ws_bytes = align_up(g.off_lossp + (size_t)B * sizeof(double), 256);
  return g;
}

struct Fwd64Params {
  const double* x;
  const void* tgt;
  int tk;  // kTgtLabels (int64 class ids) or kTgtOnehot (float64 [B, C, N])
  int64_t N, wave_vox, tile_vox, tiles;
  int B, C, off, K, CL, ck, nv, act, right, ntab, ignore_empty, red;
  size_t tab_bytes;
  double empty_w;
  const float* btab;
  const float* rtab;
  const double* clsw;
  int* ctr;
  double* part;
  double* lossp;
  double *coef, *d, *jac, *f, *loss, *stats;
};

struct Bwd64Params {
  const double* x;
  const void* tgt;
  int tk;
  int64_t N, total;
  int B, C, off, K, CL, act, right, ntab, go_per_class;
  const float* btab;
  const float* rtab;
  const double *coef, *d, *jac, *go;
  double* dx;
};

__device__ __forceinline__ void store_dev64(double* p, double v) {
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p),
                     (unsigned long long)__double_as_longlong(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double load_dev64(const double* p) {
  return __longlong_as_double((long long)__hip_atomic_load(
      reinterpret_cast<unsigned long long*>(const_cast<double*>(p)), __ATOMIC_RELAXED,
      __HIP_MEMORY_SCOPE_AGENT));
}

// Butterfly reductions over the 64 lanes of a wave (every lane active).
__device__ __forceinline__ double wave_max64(double v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = fmax(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ double wave_sum64(double v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// torch.bucketize(p, e[0..n), right) clamped to [0, n - 1]: the number of
// entries < p (<= p for right); NaN -> 0 (every comparison is false).  The
// clamp keeps out-of-domain values (p > 1 + eps32 without an activation) in
// range, as the float32 kernels do.
__device__ __forceinline__ int bucket64(double p, const double* e, int n, bool right) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    const bool below = right ? (e[mid] <= p) : (e[mid] < p);
    if (below) lo = mid + 1;
    else hi = mid;
  }
  return lo < n ? lo : n - 1;
}

// Soft assignment of common.py:43-61: half bin h, the two bins l, r and their
// weights (lw = rd / span, rw = ld / span), span = ld + rd.
struct Soft64 {
  int l, r;
  double lw, rw, span;
};
__device__ __forceinline__ Soft64 soft_assign64(double p, const double* tab, int K, bool right) {
  const double* half = tab;        // 2K upper half boundaries
  const double* repl = tab + 2 * K;  // 2K + 2 replicated centres
  const int h = bucket64(p, half, 2 * K, right);
  Soft64 s;
  s.l = max(h - 1, 0) >> 1;
  s.r = min(h + 1, 2 * K - 1) >> 1;
  const double ld = p - repl[h];
  const double rd = repl[h + 2] - p;
  s.span = ld + rd;
  s.lw = rd / s.span;
  s.rw = ld / s.span;
  return s;
}

// The float32 tables as double (exact), into LDS: K edges, or the 2K half
// boundaries followed by the 2K + 2 replicated centres.
__device__ __forceinline__ void load_tables64(double* tab, const float* btab, const float* rtab,
                                              int ntab, int nedge) {
  for (int i = threadIdx.x; i < ntab; i += blockDim.x)
    tab[i] = i < nedge ? (double)btab[i] : (double)rtab[i - nedge];
}

__device__ __forceinline__ double target_of(const void* tgt, int tk, int64_t N, int b, int C, int c,
                                            int64_t v) {
  if (tk == kTgtLabels) {
    const long long lab = static_cast<const long long*>(tgt)[(int64_t)b * N + v];
    return lab == (long long)c ? 1.0 : 0.0;
  }
  return static_cast<const double*>(tgt)[((int64_t)b * C + c) * N + v];
}

// Epilogue of batch index b from its sums s[3][C'K] (LDS): d, coef, the
// per-class error f * present * w and the reduction's jacobian
// (binning.py:127-147, v2_autograd.py:66-76, 138-151, common.py:184-207);
// returns in thread 0 the sum of its rows' per-class errors in row order.
// sd: C'K doubles and emp: C'K bytes of LDS for d and the empty flags.
template <bool SOFT>
__device__ double epilogue64(const Fwd64Params& P, int b, const double* s, double* sd,
                             unsigned char* emp) {
  const int tid = threadIdx.x;
  const int K = P.K, ck = P.ck;
  for (int i = tid; i < ck; i += blockDim.x) {
    const double W = s[i], Pp = s[ck + i], G = s[2 * ck + i];
    const bool empty = SOFT ? (W < P.empty_w) : (W == 0.0);
    const double dd = empty ? 0.0 : (Pp / W - G / W);
    emp[i] = empty ? 1 : 0;
    sd[i] = dd;
    P.d[(int64_t)b * ck + i] = dd;
    if (P.stats) {
      const int64_t bck = (int64_t)P.B * ck;
      P.stats[(int64_t)b * ck + i] = W;
      P.stats[bck + (int64_t)b * ck + i] = Pp;
      P.stats[2 * bck + (int64_t)b * ck + i] = G;
    }
  }
  __syncthreads();
  __shared__ double s_rows[64];
  const int rows = P.B * P.CL;
  for (int cl = tid; cl < P.CL; cl += blockDim.x) {
    const double* W = s + cl * K;
    const double* G = s + 2 * ck + cl * K;
    int kne = 0;
    double err = 0.0, gsum = 0.0;
    for (int k = 0; k < K; ++k) {
      gsum += G[k];
      if (!emp[cl * K + k]) {
        ++kne;
        err += fabs(sd[cl * K + k]);
      }
    }
    const double f = kne > 0 ? err / (double)kne : __builtin_nan("");
    const double present = gsum > 0.0 ? 1.0 : 0.0;
    const double kf = (double)(kne > 0 ? kne : 1);
    for (int k = 0; k < K; ++k) {
      const int64_t o = (int64_t)b * ck + cl * K + k;
      const double dd = sd[cl * K + k];
      const double sgn = dd > 0.0 ? 1.0 : (dd < 0.0 ? -1.0 : 0.0);
      P.coef[o] = emp[cl * K + k] ? 0.0 : sgn / (kf * W[k]);
    }
    const double w = P.clsw ? P.clsw[cl] : 1.0;
    const double fw = (P.ignore_empty ? f * present : f) * w;
    double jac = P.ignore_empty ? present * w : w;
    if (P.red == kRedMean) jac = jac / (double)rows;
    P.f[b * P.CL + cl] = fw;
    P.jac[b * P.CL + cl] = jac;
    s_rows[cl] = fw;
  }
  __syncthreads();
  double total = 0.0;
  if (tid == 0)
    for (int cl = 0; cl < P.CL; ++cl) total += s_rows[cl];
  return total;
}

template <bool SOFT>
__global__ void __launch_bounds__(kThreads) fwd64_kernel(const Fwd64Params P) {
  extern __shared__ __align__(16) unsigned char smem[];
  double* tab = reinterpret_cast<double*>(smem);
  double* hist = reinterpret_cast<double*>(smem + P.tab_bytes);
  const int tid = threadIdx.x;
  const int nt = blockDim.x;
  const int waves = nt >> 6;
  const int K = P.K, ck = P.ck, nv = P.nv;
  const int b = (int)(blockIdx.x / P.tiles);
  const int64_t tile = blockIdx.x - (int64_t)b * P.tiles;
  load_tables64(tab, P.btab, P.rtab, P.ntab, SOFT ? 2 * K : K);
  for (int i = tid; i < waves * nv; i += nt) hist[i] = 0.0;
  __syncthreads();

  {
    const int w = tid >> 6;
    const int c = tid & 63;
    double* h = hist + (size_t)w * nv;
    const bool chan = c < P.C;
    const bool in_loss = chan && c >= P.off;
    const int cl = c - P.off;
    const int64_t v0 = tile * P.tile_vox + (int64_t)w * P.wave_vox;
    const int64_t v1 = min(v0 + P.wave_vox, P.N);
    const double* xc = P.x + ((int64_t)b * P.C + (chan ? c : 0)) * P.N;
    for (int64_t v = v0; v < v1; ++v) {  // wave-uniform bounds: every lane runs every iteration
      const double xv = chan ? xc[v] : 0.0;
      double p;
      if (P.act == kActSoftmax) {
        const double m = wave_max64(chan ? xv : -__builtin_inf());
        const double e = chan ? exp(xv - m) : 0.0;
        p = e / wave_sum64(e);
      } else if (P.act == kActSigmoid) {
        p = 1.0 / (1.0 + exp(-xv));
      } else {
        p = xv;
      }
      if (in_loss) {
        const double y = target_of(P.tgt, P.tk, P.N, b, P.C, c, v);
        double* W = h + cl * K;
        double* Ps = h + ck + cl * K;
        double* G = h + 2 * ck + cl * K;
        if constexpr (SOFT) {
          const Soft64 a = soft_assign64(p, tab, K, P.right != 0);
          W[a.l] += a.lw;
          W[a.r] += a.rw;
          Ps[a.l] += a.lw * p;
          Ps[a.r] += a.rw * p;
          G[a.l] += a.lw * y;
          G[a.r] += a.rw * y;
        } else {
          const int k = bucket64(p, tab, K, P.right != 0);
          W[k] += 1.0;
          Ps[k] += p;
          G[k] += y;
        }
      }
    }
  }
  __syncthreads();
  // the block's sums: its waves' histograms in wave order
  double* part = P.part + ((int64_t)b * P.tiles + tile) * nv;
  for (int i = tid; i < nv; i += nt) {
    double s = 0.0;
    for (int w = 0; w < waves; ++w) s += hist[(size_t)w * nv + i];
    store_dev64(part + i, s);
  }
  wait_own_writes();
  __syncthreads();
  __shared__ int s_last;
  if (tid == 0) {
    int* bc = P.ctr + (int64_t)b * kCtrStride;
    const int last = ticket(bc) == (int)P.tiles - 1;
    if (last) __hip_atomic_store(bc, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;

  // last block of batch index b: the partials in tile order (and zeroed)
  // (LDS: the nv sums, then d and the empty flags, over the histograms)
  double* sums = hist;
  double* pb = P.part + (int64_t)b * P.tiles * nv;
  constexpr int kBatch = 8;  // loads in flight per thread
  for (int i = tid; i < nv; i += nt) {
    double s = 0.0;
    for (int64_t t0 = 0; t0 < P.tiles; t0 += kBatch) {
      double v[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) v[j] = t0 + j < P.tiles ? load_dev64(pb + (t0 + j) * nv + i) : 0.0;
#pragma unroll
      for (int j = 0; j < kBatch; ++j)
        if (t0 + j < P.tiles) s += v[j];
    }
    for (int64_t t = 0; t < P.tiles; ++t) store_dev64(pb + t * nv + i, 0.0);
    sums[i] = s;
  }
  __syncthreads();
  double* sd = hist + nv;
  unsigned char* emp = reinterpret_cast<unsigned char*>(sd + ck);
  const double total = epilogue64<SOFT>(P, b, sums, sd, emp);
  if (P.red == kRedNone) return;
  const int rows = P.B * P.CL;
  if (P.B == 1) {
    if (tid == 0) P.loss[0] = P.red == kRedMean ? total / (double)rows : total;
    return;
  }
  // the last batch epilogue adds the batch totals in b order
  if (tid == 0) {
    store_dev64(P.lossp + b, total);
    wait_own_writes();
    int* lc = P.ctr + (int64_t)P.B * kCtrStride;
    if (ticket(lc) == P.B - 1) {
      __hip_atomic_store(lc, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      double sum = 0.0;
      for (int bb = 0; bb < P.B; ++bb) {
        sum += load_dev64(P.lossp + bb);
        store_dev64(P.lossp + bb, 0.0);
      }
      P.loss[0] = P.red == kRedMean ? sum / (double)rows : sum;
    }
  }
}

// dL/dp of loss channel c' at p (v2_autograd.py:88-104).
template <bool SOFT>
__device__ __forceinline__ double dfdp64(const Bwd64Params& P, const double* tab, int b, int cl,
                                         double p, double y) {
  const int K = P.K;
  const double* cf = P.coef + ((int64_t)b * P.CL + cl) * K;
  if constexpr (SOFT) {
    const double* dd = P.d + ((int64_t)b * P.CL + cl) * K;
    const Soft64 a = soft_assign64(p, tab, K, P.right != 0);
    const double inv_span = 1.0 / a.span;
    const double resid = p - y;
    return cf[a.l] * (a.lw - inv_span * (resid - dd[a.l])) +
           cf[a.r] * (a.rw + inv_span * (resid - dd[a.r]));
  } else {
    return cf[bucket64(p, tab, K, P.right != 0)];
  }
}

template <bool SOFT>
__global__ void __launch_bounds__(kThreads) bwd64_kernel(const Bwd64Params P) {
  extern __shared__ __align__(16) unsigned char smem[];
  double* tab = reinterpret_cast<double*>(smem);
  load_tables64(tab, P.btab, P.rtab, P.ntab, SOFT ? 2 * P.K : P.K);
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < P.total; idx += stride) {
    const int b = (int)(idx / P.N);
    const int64_t v = idx - (int64_t)b * P.N;
    const double* xb = P.x + (int64_t)b * P.C * P.N + v;
    double* db = P.dx + (int64_t)b * P.C * P.N + v;
    double m = 0.0, s = 1.0;
    if (P.act == kActSoftmax) {
      m = -__builtin_inf();
      for (int c = 0; c < P.C; ++c) m = fmax(m, xb[c * P.N]);
      s = 0.0;
      for (int c = 0; c < P.C; ++c) s += exp(xb[c * P.N] - m);
    }
    auto prob = [&](int c) -> double {
      const double xv = xb[c * P.N];
      if (P.act == kActSoftmax) return exp(xv - m) / s;
      if (P.act == kActSigmoid) return 1.0 / (1.0 + exp(-xv));
      return xv;
    };
    auto grad_p = [&](int c, double p) -> double {
      if (c < P.off) return 0.0;
      const int cl = c - P.off;
      const double g = P.jac[b * P.CL + cl] * P.go[P.go_per_class ? b * P.CL + cl : 0];
      const double y = SOFT ? target_of(P.tgt, P.tk, P.N, b, P.C, c, v) : 0.0;
      return g * dfdp64<SOFT>(P, tab, b, cl, p, y);
    };
    double dot = 0.0;
    if (P.act == kActSoftmax)
      for (int c = 0; c < P.C; ++c) {
        const double p = prob(c);
        dot += grad_p(c, p) * p;
      }
    for (int c = 0; c < P.C; ++c) {
      const double p = prob(c);
      const double gp = grad_p(c, p);
      double out;
      if (P.act == kActSoftmax) out = p * (gp - dot);
      else if (P.act == kActSigmoid) out = gp * p * (1.0 - p);
      else out = gp;
      db[c * P.N] = out;
    }
  }
}

}  // namespace f64
}  // namespace ace

using namespace ace;
using namespace ace::f64;

namespace {

int check64(const double* x, const void* target, int target_kind, int64_t batch, int64_t channels,
            int64_t voxels, int num_bins, int binning, int activation, const float* bin_table,
            const float* centre_table) {
  if (!x && batch * channels * voxels > 0) return ACE_EINVAL;
  if (target_kind != ACE_TARGET_LABELS_I64 && target_kind != ACE_TARGET_ONEHOT_F64)
    return ACE_EINVAL;
  if (binning != ACE_HARD && binning != ACE_SOFT) return ACE_EINVAL;
  if (activation != ACE_ACT_NONE && activation != ACE_ACT_SOFTMAX && activation != ACE_ACT_SIGMOID)
    return ACE_EINVAL;
  if (batch < 1 || channels < 1 || voxels < 0 || num_bins < 1) return ACE_EINVAL;
  if (channels > 64) return ACE_EUNSUPPORTED;
  if (num_bins > (1 << 20)) return ACE_EUNSUPPORTED;
  if (!bin_table || (binning == ACE_SOFT && !centre_table)) return ACE_EINVAL;
  if (channels == 1 && target_kind == ACE_TARGET_LABELS_I64) return ACE_EINVAL;
  if (!target && voxels > 0) return ACE_EINVAL;
  return ACE_OK;
}

int code_of(hipError_t e) { return e == hipSuccess ? ACE_OK : ACE_EHIP + (int)e; }

}  // namespace

namespace ace {
namespace f64 {
// Workspace bytes of ace_forward_f64 (ace_workspace_bytes with ACE_F64).
size_t workspace_bytes(int64_t batch, int64_t channels, int64_t voxels, int num_bins, int binning,
                       int include_background) {
  if (batch < 1 || channels < 1 || voxels < 0 || num_bins < 1) return 0;
  return geometry(batch, channels, voxels, num_bins, binning == ACE_SOFT, include_background != 0)
      .ws_bytes;
}
}  // namespace f64
}  // namespace ace

extern "C" {

int ace_forward_f64(const double* x, const void* target, int target_kind, int64_t batch,
                    int64_t channels, int64_t voxels, int num_bins, int binning, int activation,
                    int include_background, int ignore_empty_classes, int reduction, int right,
                    double empty_weight, const double* class_weight, const float* bin_table,
                    const float* centre_table, void* workspace, size_t workspace_bytes,
                    double* coef, double* diff, double* jac, double* per_class, double* loss,
                    double* stats, void* stream) {
  int rc = check64(x, target, target_kind, batch, channels, voxels, num_bins, binning, activation,
                   bin_table, centre_table);
  if (rc) return rc;
  if (reduction != ACE_RED_MEAN && reduction != ACE_RED_SUM && reduction != ACE_RED_NONE)
    return ACE_EINVAL;
  if (!workspace || !coef || !diff || !jac || !per_class) return ACE_EINVAL;
  if (reduction != ACE_RED_NONE && !loss) return ACE_EINVAL;
  const bool soft = binning == ACE_SOFT;
  const Geo64 g = geometry(batch, channels, voxels, num_bins, soft, include_background != 0);
  if (g.waves == 0) return ACE_EUNSUPPORTED;
  if (workspace_bytes < g.ws_bytes) return ACE_EWORKSPACE;
  if (batch * g.tiles > 0x7fffffffLL) return ACE_EUNSUPPORTED;

  Fwd64Params p{};
  p.x = x;
  p.tgt = target;
  p.tk = target_kind == ACE_TARGET_LABELS_I64 ? kTgtLabels : kTgtOnehot;
  p.N = voxels;
  p.wave_vox = g.wave_vox;
  p.tile_vox = g.tile_vox;
  p.tiles = g.tiles;
  p.B = (int)batch;
  p.C = (int)channels;
  p.off = g.off;
  p.K = num_bins;
  p.CL = g.CL;
  p.ck = g.ck;
  p.nv = g.nv;
  // softmax over one channel is the identity (common.py:93-101)
  p.act = (activation == ACE_ACT_SOFTMAX && channels == 1) ? kActNone : activation;
  p.right = right != 0;
  p.ntab = g.ntab;
  p.ignore_empty = ignore_empty_classes != 0;
  p.red = reduction;
  p.tab_bytes = g.tab_bytes;
  p.empty_w = empty_weight;
  p.btab = bin_table;
  p.rtab = centre_table;
  p.clsw = class_weight;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  p.ctr = reinterpret_cast<int*>(ws);
  p.part = reinterpret_cast<double*>(ws + g.off_part);
  p.lossp = reinterpret_cast<double*>(ws + g.off_lossp);
  p.coef = coef;
  p.d = diff;
  p.jac = jac;
  p.f = per_class;
  p.loss = loss;
  p.stats = stats;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const long long nblk = batch * g.tiles;
  const int nt = 64 * g.waves;
  // the epilogue reuses the histogram LDS: 3 C'K sums, C'K d, C'K empty flags
  const size_t epi = g.tab_bytes + (size_t)4 * g.ck * 8 + align_up((size_t)g.ck, 16);
  const size_t lds = g.lds > epi ? g.lds : epi;
  // refused before any HIP call: the dynamic LDS beside the kernel's static
  // arrays must fit the workgroup's
  if (lds > kMaxFwdDynLds64) return ACE_EUNSUPPORTED;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(soft ? fwd64_kernel<true> : fwd64_kernel<false>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return code_of(e);
  }
  return code_of(soft ? launch(fwd64_kernel<true>, nblk, lds, s, p, nt)
                      : launch(fwd64_kernel<false>, nblk, lds, s, p, nt));
}

int ace_backward_f64(const double* x, const void* target, int target_kind, int64_t batch,
                     int64_t channels, int64_t voxels, int num_bins, int binning, int activation,
                     int include_background, int right, const float* bin_table,
                     const float* centre_table, const double* coef, const double* diff,
                     const double* jac, const double* grad_output, int grad_output_per_class,
                     double* dx, void* stream) {
  const bool soft = binning == ACE_SOFT;
  int rc = check64(x, soft ? target : (target ? target : x), target_kind, batch, channels, voxels,
                   num_bins, binning, activation, bin_table, centre_table);
  if (rc) return rc;
  if (!coef || !jac || !grad_output || (!dx && voxels > 0)) return ACE_EINVAL;
  if (soft && !diff) return ACE_EINVAL;
  if (voxels == 0) return ACE_OK;
  const Geo64 g = geometry(batch, channels, voxels, num_bins, soft, include_background != 0);
  Bwd64Params p{};
  p.x = x;
  p.tgt = target;
  p.tk = target_kind == ACE_TARGET_LABELS_I64 ? kTgtLabels : kTgtOnehot;
  p.N = voxels;
  p.total = batch * voxels;
  p.B = (int)batch;
  p.C = (int)channels;
  p.off = g.off;
  p.K = num_bins;
  p.CL = g.CL;
  p.act = (activation == ACE_ACT_SOFTMAX && channels == 1) ? kActNone : activation;
  p.right = right != 0;
  p.ntab = g.ntab;
  p.go_per_class = grad_output_per_class != 0;
  p.btab = bin_table;
  p.rtab = centre_table;
  p.coef = coef;
  p.d = diff;
  p.jac = jac;
  p.go = grad_output;
  p.dx = dx;
  const int64_t blocks = cdiv(p.total, (int64_t)kThreads);
  const long long nblk = blocks < 4096 ? blocks : 4096;
  const size_t lds = g.tab_bytes;
  if (lds > kMaxLds64) return ACE_EUNSUPPORTED;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(soft ? bwd64_kernel<true> : bwd64_kernel<false>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return code_of(e);
  }
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return code_of(soft ? launch(bwd64_kernel<true>, nblk, lds, s, p, kThreads)
                      : launch(bwd64_kernel<false>, nblk, lds, s, p, kThreads));
}

}  // extern "C"
