// extern "C" entry points of libace_hip.so (declared in include/ace_hip.h).
//
// Host side of the boundary: argument validation, launch geometry, the
// alignment test that selects vector loads, and dispatch to the kernel
// instantiation for (element type, binning, channel variant).  No call
// allocates, copies or synchronises.
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stdlib.h>

#include <atomic>
#include <mutex>

#include "ace_core.hpp"
#include "ace_hip.h"

namespace ace {
#define ACE_DECLARE_LAUNCHERS(T, SOFT, RIGHT)                                                \
  template <> hipError_t launch_variant_fwd<T, SOFT, RIGHT>(const Geometry&, const FwdParams&, \
                                                            hipStream_t);                    \
  template <> hipError_t launch_variant_bwd<T, SOFT, RIGHT>(const Geometry&, const BwdParams&, \
                                                            hipStream_t);                    \
  template <> hipError_t launch_levels_fwd<T, SOFT, RIGHT>(int, long long, size_t,             \
                                                           const FwdLevels&, hipStream_t);   \
  template <> hipError_t launch_levels_bwd<T, SOFT, RIGHT>(int, long long, size_t,             \
                                                           const BwdLevels&, hipStream_t);
#define ACE_DECLARE_BOTH(T, SOFT) ACE_DECLARE_LAUNCHERS(T, SOFT, false) ACE_DECLARE_LAUNCHERS(T, SOFT, true)
ACE_DECLARE_BOTH(float, false)
ACE_DECLARE_BOTH(float, true)
ACE_DECLARE_BOTH(__hip_bfloat16, false)
ACE_DECLARE_BOTH(__hip_bfloat16, true)
ACE_DECLARE_BOTH(__half, false)
ACE_DECLARE_BOTH(__half, true)
#undef ACE_DECLARE_BOTH
#undef ACE_DECLARE_LAUNCHERS

// Dispatch on (element type, binning, right) to the instantiated launchers.
template <typename T>
hipError_t pick_fwd(bool soft, bool right, const Geometry& g, const FwdParams& p, hipStream_t s) {
  if (soft)
    return right ? launch_variant_fwd<T, true, true>(g, p, s) : launch_variant_fwd<T, true, false>(g, p, s);
  return right ? launch_variant_fwd<T, false, true>(g, p, s) : launch_variant_fwd<T, false, false>(g, p, s);
}
template <typename T>
hipError_t pick_bwd(bool soft, bool right, const Geometry& g, const BwdParams& p, hipStream_t s) {
  if (soft)
    return right ? launch_variant_bwd<T, true, true>(g, p, s) : launch_variant_bwd<T, true, false>(g, p, s);
  return right ? launch_variant_bwd<T, false, true>(g, p, s) : launch_variant_bwd<T, false, false>(g, p, s);
}
hipError_t dispatch_fwd(int dtype, bool soft, bool right, const Geometry& g, const FwdParams& p,
                        hipStream_t s) {
  switch (dtype) {
    case ACE_F32: return pick_fwd<float>(soft, right, g, p, s);
    case ACE_BF16: return pick_fwd<__hip_bfloat16>(soft, right, g, p, s);
    default: return pick_fwd<__half>(soft, right, g, p, s);
  }
}
hipError_t dispatch_bwd(int dtype, bool soft, bool right, const Geometry& g, const BwdParams& p,
                        hipStream_t s) {
  switch (dtype) {
    case ACE_F32: return pick_bwd<float>(soft, right, g, p, s);
    case ACE_BF16: return pick_bwd<__hip_bfloat16>(soft, right, g, p, s);
    default: return pick_bwd<__half>(soft, right, g, p, s);
  }
}

namespace {

constexpr size_t kMaxLds = 160 * 1024;  // gfx950 LDS per workgroup

size_t elem_size(int dtype) { return dtype == ACE_F32 ? 4 : 2; }

// Bytes of the targets: int64 class labels [B, N] or float32 one-hot [B, C, N].
size_t target_bytes(bool labels, int64_t batch, int64_t channels, int64_t voxels) {
  return labels ? 8 * (size_t)batch * (size_t)voxels
                : 4 * (size_t)batch * (size_t)channels * (size_t)voxels;
}

bool aligned_to(const void* p, size_t a) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

int check_common(const void* x, int x_dtype, const void* target, int target_kind,
                 int64_t batch, int64_t channels, int64_t voxels, int num_bins,
                 int binning, int activation, const float* bin_table,
                 const float* centre_table, bool need_target) {
  // with no voxels, input and target may be null (empty tensors): nothing
  // reads them
  if ((!x && voxels > 0) || !bin_table) return ACE_EINVAL;
  if (x_dtype != ACE_F32 && x_dtype != ACE_BF16 && x_dtype != ACE_F16) return ACE_EINVAL;
  if (target_kind != ACE_TARGET_LABELS_I64 && target_kind != ACE_TARGET_ONEHOT_F32)
    return ACE_EINVAL;
  if (binning != ACE_HARD && binning != ACE_SOFT) return ACE_EINVAL;
  if (activation != ACE_ACT_NONE && activation != ACE_ACT_SOFTMAX &&
      activation != ACE_ACT_SIGMOID)
    return ACE_EINVAL;
  if (batch < 1 || channels < 1 || voxels < 0 || num_bins < 1) return ACE_EINVAL;
  if (channels > kMaxChannels) return ACE_EUNSUPPORTED;
  if (num_bins > (1 << 20)) return ACE_EUNSUPPORTED;
  if (binning == ACE_SOFT && !centre_table) return ACE_EINVAL;
  if (need_target && !target && voxels > 0) return ACE_EINVAL;
  // one channel: to_onehot_y is ignored upstream, the target is per-channel
  if (channels == 1 && target_kind == ACE_TARGET_LABELS_I64 && target) return ACE_EINVAL;
  return ACE_OK;
}

int to_code(hipError_t e) { return e == hipSuccess ? ACE_OK : ACE_EHIP + (int)e; }

// Soft binning of softmax probabilities with label targets on a fast
// channel count bins through half-bin moments when the bin count and the
// moments' LDS layout (48 C'K bytes per copy, and the epilogue's terms)
// allow it; otherwise the generic soft kernels (per-voxel weights, 24 C'K
// bytes per copy).  Forward and backward take the same decision.
// The test uses the 256-thread layout (at most 32 KB of copies); a
// 1024-thread block then fits as well (fewer copies if need be, or 256
// threads, make_geometry), so the decision does not depend on the block size.
bool use_moments(bool soft, bool labels, int act, int64_t batch, int64_t channels, int64_t voxels,
                 int num_bins, int include_background) {
  if (!(soft && labels && act == kActSoftmax && fast_channels(channels) &&
        num_bins <= kMomentMaxBins))
    return false;
  const Geometry g = make_geometry(batch, channels, voxels, num_bins, true, include_background != 0,
                                   true, 0, 0, true, true, kThreads);
  return g.lds_fwd <= kMaxLds && g.lds_bwd <= kMaxLds;
}

// The forward runs a fast kernel (fast_bins, 1024-thread blocks where the
// histogram copies allow): softmax over a fast channel count with class
// labels, soft binning in the moments layout.
bool fast_forward(bool soft, bool labels, int act, int64_t channels, bool moments) {
  return act == kActSoftmax && labels && fast_channels(channels) && (!soft || moments);
}

// Test hooks (ace_set_test_hooks), process-wide: the bound of the loss
// block's wait for another batch epilogue's partial word (kMaxPolls; 0 makes
// the wait give up at once wherever the word has not arrived, the loss NaN,
// with every kernel still exiting normally), and sleeps (s_sleep 2 each)
// before a batch epilogue publishes its word (0), so that a test can make
// that wait give up.
std::atomic<int> g_max_polls{kMaxPolls};
// ace_set_timeline's buffer (null: no stamps), process-wide
std::atomic<unsigned long long*> g_timeline{nullptr};
std::atomic<int> g_publish_delay{0};

// Forward geometry of one problem (the kernel the launcher will pick).
Geometry forward_geometry(int64_t batch, int64_t channels, int64_t voxels, int num_bins, bool soft,
                          int include_background, bool labels, int act, bool moments,
                          int max_nt = kFastThreads) {
  return make_geometry(batch, channels, voxels, num_bins, soft, include_background != 0, labels, 0, 0,
                       moments, fast_forward(soft, labels, act, channels, moments), max_nt);
}

// The activation is not an argument here: the largest workspace of the
// layouts a call may use (generic, fast, soft moments).
size_t workspace_size(int64_t batch, int64_t channels, int64_t voxels, int num_bins, int binning,
                      int include_background, int target_kind) {
  const bool soft = binning == ACE_SOFT;
  const bool labels = target_kind == ACE_TARGET_LABELS_I64;
  size_t best = 0;
  for (int act : {(int)kActNone, (int)kActSoftmax}) {
    for (int max_nt : {kThreads, kFastThreads}) {
      const bool moments = use_moments(soft, labels, act, batch, channels, voxels, num_bins,
                                       include_background);
      const Geometry g = forward_geometry(batch, channels, voxels, num_bins, soft,
                                          include_background, labels, act, moments, max_nt);
      best = g.ws_bytes > best ? g.ws_bytes : best;
    }
  }
  return best;
}

// Vector steps per backward block: make_geometry's choice (~1024 blocks; 512 above 8 channels, where the forward's final-sum
// atomics set the count) -- except the fast 16-channel backward with every
// channel in the loss, which holds 4 or more waves per SIMD (ace_core.hpp:
// bwd_min_waves) and measured fastest with ~1024 blocks on MI355X (cfg 4,
// one voxel per lane: 49.7 us against 53.7 at 512 blocks and 55.2 at ~680;
// two voxels per lane: 50.8 against 57.2 at 512).
int bwd_steps(bool soft, bool labels, int act, int64_t batch, int64_t channels, int64_t voxels,
              int include_background, bool moments) {
  const bool fast = act == kActSoftmax && fast_channels(channels) && (!soft || (labels && moments));
  if (!(fast && channels > 8 && (include_background != 0 || channels == 1))) return 0;
  const int64_t step_vox = (int64_t)kThreads * variant_for(channels).vec;
  const int64_t steps = cdiv(batch * (voxels > 0 ? voxels : 1), step_vox * 1024);
  return (int)(steps < 1 ? 1 : (steps > 64 ? 64 : steps));
}

// The forward's launch plan and the checks it must pass before anything is
// launched: the geometry of the kernel the launcher will pick, within the
// LDS and the grid's limits.
struct ForwardPlan {
  int rc;
  int act;
  bool moments;
  Geometry g;
};
ForwardPlan plan_forward(int64_t batch, int64_t channels, int64_t voxels, int num_bins, int binning,
                         int activation, int include_background, int target_kind) {
  ForwardPlan fp{};
  const bool soft = binning == ACE_SOFT;
  const bool labels = target_kind == ACE_TARGET_LABELS_I64;
  fp.act = (activation == ACE_ACT_SOFTMAX && channels == 1) ? kActNone : activation;
  fp.moments = use_moments(soft, labels, fp.act, batch, channels, voxels, num_bins, include_background);
  fp.g = forward_geometry(batch, channels, voxels, num_bins, soft, include_background, labels, fp.act,
                          fp.moments);
  fp.rc = (fp.g.lds_fwd > kMaxLds || fp.g.nblk > 0x7fffffffLL) ? ACE_EUNSUPPORTED : ACE_OK;
  return fp;
}

// fast_bin's fixed point and edge margin for K bins (ace_bins.hpp:
// fast_bin_consts).
void set_fast_bins(FwdParams& p, int num_bins, int64_t channels) {
  const FastBinConsts f = fast_bin_consts(num_bins, channels);
  p.qscale = f.qscale;
  p.qlo = f.qlo;
  p.qhi = f.qhi;
  p.qmq = f.qmq;
  p.qmask = f.qmask;
  p.qs = f.qs;
  p.pscale = f.pscale;
}

// Kernel parameters of one forward problem (geometry g, workspace at ws).
FwdParams fwd_params(const void* x, int x_dtype, const void* target, bool labels, int64_t voxels,
                     int64_t batch, int64_t channels, int num_bins, int act,
                     int ignore_empty_classes, int reduction, float empty_weight, bool moments,
                     const float* class_weight, const float* bin_table, const float* centre_table,
                     void* workspace, const Geometry& g, float* coef, float* diff, float* jac,
                     float* per_class, float* loss, double* stats) {
  const int vec = g.var.vec;
  const size_t es = elem_size(x_dtype);
  const bool vec_ok = (voxels % vec) == 0 && aligned_to(x, es * vec) &&
                      (labels ? aligned_to(target, 16) : aligned_to(target, 4 * vec));

  FwdParams p{};
  p.x = x;
  p.tgt = target;
  p.N = voxels;
  p.tile_vox = g.tile_vox;
  p.tiles = g.tiles;
  p.gs = g.gs;
  p.gpb = g.gpb;
  p.B = (int)batch;
  p.C = (int)channels;
  p.off = g.off;
  p.K = num_bins;
  p.act = act;
  p.tk = labels ? kTgtLabels : kTgtOnehot;
  p.copies = g.copies;
  p.vec_ok = vec_ok ? 1 : 0;
  p.ignore_empty = ignore_empty_classes != 0;
  p.red = reduction;
  p.empty_w = empty_weight;
  p.packed = g.packed ? 1 : 0;
  p.tl = g_timeline.load(std::memory_order_relaxed);
  p.max_polls = g_max_polls.load(std::memory_order_relaxed);
  p.publish_delay = g_publish_delay.load(std::memory_order_relaxed);
  p.pscale = 1.0 / 1073741824.0;  // the generic kernels' sums: 30-bit fixed point
  const int sf = soft_frac(voxels);  // the generic soft sums: finer (soft_frac)
  p.sfx = ldexpf(1.0f, sf);
  p.sscale = ldexp(1.0, -sf);
  if (g.fast && !moments) set_fast_bins(p, num_bins, channels);
  if (moments) {
    const MomentScale ms = moment_scale(num_bins);
    p.msc = ldexpf(1.0f, ms.m);
    p.misc = ldexpf(1.0f, -ms.m);
    p.mw = ms.w;
    p.mshift = moment_shift(voxels);
  }
  p.btab = bin_table;
  p.rtab = centre_table;
  p.clsw = class_weight;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  p.ctr = reinterpret_cast<int*>(ws);
  p.part = reinterpret_cast<unsigned long long*>(ws + g.off_part);
  p.fin = reinterpret_cast<unsigned long long*>(ws + g.off_fin);
  p.reps = g.reps;
  p.lchunk = g.lchunk;
  p.epi_all = g.epi_all ? 1 : 0;
  p.coef = coef;
  p.d = diff;
  p.jac = jac;
  p.f = per_class;
  p.loss = loss;
  p.stats = stats;

  return p;
}

// Kernel parameters of one backward problem (geometry g).
BwdParams bwd_params(const void* x, int x_dtype, const void* target, bool labels, bool soft,
                     int64_t voxels, int64_t batch, int64_t channels, int num_bins, int act,
                     const float* bin_table, const float* centre_table, const float* coef,
                     const float* diff, const float* jac, const float* grad_output,
                     int grad_output_per_class, void* dx, const Geometry& g) {
  const int vec = g.var.vec;
  const size_t es = elem_size(x_dtype);
  bool vec_ok = (voxels % vec) == 0 && aligned_to(x, es * vec) && aligned_to(dx, es * vec);
  if (soft && target)
    vec_ok = vec_ok && (labels ? aligned_to(target, 16) : aligned_to(target, 4 * vec));

  BwdParams p{};
  p.x = x;
  p.tgt = target;
  p.dx = dx;
  p.N = voxels;
  p.tile_vox = g.tile_vox;
  p.tiles = g.tiles;
  p.B = (int)batch;
  p.C = (int)channels;
  p.off = g.off;
  p.K = num_bins;
  p.act = act;
  p.tk = labels ? kTgtLabels : kTgtOnehot;
  p.vec_ok = vec_ok ? 1 : 0;
  p.go_per_class = grad_output_per_class != 0;
  p.btab = bin_table;
  p.rtab = centre_table;
  p.coef = coef;
  p.d = diff;
  p.jac = jac;
  p.go = grad_output;
  p.stream = stream_problem(es * (size_t)batch * (size_t)channels * (size_t)voxels,
                            target_bytes(labels, batch, channels, voxels)) ? 1 : 0;

  return p;
}

// Bytes of one level's workspace region in a multi-level call.
size_t level_ws_bytes(int64_t batch, int64_t channels, int64_t voxels, int num_bins, int binning,
                      int include_background) {
  return align_up(workspace_size(batch, channels, voxels, num_bins, binning, include_background,
                                 ACE_TARGET_LABELS_I64),
                  256);
}

template <typename T>
hipError_t pick_levels_fwd(bool soft, bool right, int cmax, long long nblk, size_t lds,
                           const FwdLevels& L, hipStream_t s) {
  if (soft)
    return right ? launch_levels_fwd<T, true, true>(cmax, nblk, lds, L, s)
                 : launch_levels_fwd<T, true, false>(cmax, nblk, lds, L, s);
  return right ? launch_levels_fwd<T, false, true>(cmax, nblk, lds, L, s)
               : launch_levels_fwd<T, false, false>(cmax, nblk, lds, L, s);
}
template <typename T>
hipError_t pick_levels_bwd(bool soft, bool right, int cmax, long long nblk, size_t lds,
                           const BwdLevels& L, hipStream_t s) {
  if (soft)
    return right ? launch_levels_bwd<T, true, true>(cmax, nblk, lds, L, s)
                 : launch_levels_bwd<T, true, false>(cmax, nblk, lds, L, s);
  return right ? launch_levels_bwd<T, false, true>(cmax, nblk, lds, L, s)
               : launch_levels_bwd<T, false, false>(cmax, nblk, lds, L, s);
}

}  // namespace
}  // namespace ace

// ---------------------------------------------- allocation-free forward
// ace_forward_noalloc's workspace: one array per device, zero at load, held
// until the process ends.  Host code never passes the array's name to a
// kernel (on the host it is a stand-in, not a device address); it uses the
// device address that scratch_address() obtains once per device.
static __device__ __align__(256) unsigned char scratch[ACE_NOALLOC_SCRATCH_BYTES];

namespace ace {
namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch`, per device

// Device address of the current device's `scratch` (hipGetSymbolAddress on
// the first call on that device, with that device current).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return to_code(e);
  if (dev < 0 || dev >= kMaxScratchDevices) return ACE_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return to_code(e);
    if (!ptr) return ACE_EHIP + (int)hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return ACE_OK;
}

// Zero `words` 8-byte words at p (a fill kernel rather than hipMemsetAsync,
// so that a captured call records no memset node).
__global__ void __launch_bounds__(kThreads) clear_words(unsigned long long* p, size_t words) {
  const size_t stride = (size_t)gridDim.x * kThreads;
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < words; i += stride) p[i] = 0ull;
}

// ace_read_bytes: every 16-byte vector of a and b read once (grid-stride,
// four vectors in flight per lane) and folded into a per-lane xor.
// kFastThreads-thread blocks, the forward's widest.
constexpr int kReadBlocks = 512;
__global__ void __launch_bounds__(kFastThreads) read_bytes_kernel(const uint4* a, size_t na,
                                                                   const uint4* b, size_t nb,
                                                                   unsigned* out) {
  const size_t stride = (size_t)gridDim.x * kFastThreads;
  unsigned acc = 0;
  for (int buf = 0; buf < 2; ++buf) {
    const uint4* p = buf == 0 ? a : b;
    const size_t n = buf == 0 ? na : nb;
    size_t i = (size_t)blockIdx.x * kFastThreads + threadIdx.x;
    for (; i + 3 * stride < n; i += 4 * stride) {
      const uint4 v0 = p[i], v1 = p[i + stride], v2 = p[i + 2 * stride], v3 = p[i + 3 * stride];
      acc ^= v0.x ^ v0.y ^ v0.z ^ v0.w ^ v1.x ^ v1.y ^ v1.z ^ v1.w;
      acc ^= v2.x ^ v2.y ^ v2.z ^ v2.w ^ v3.x ^ v3.y ^ v3.z ^ v3.w;
    }
    for (; i < n; i += stride) {
      const uint4 v = p[i];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  // a store that depends on every lane's loads (and almost never happens), so
  // that no load is dead; the scratch word's value means nothing
  if (acc == 0x2545f491u) out[blockIdx.x] = acc;
}

// ace_probabilities: activate (the activation of every forward and backward
// kernel) of one voxel per lane, written as float32.
template <typename T>
__global__ void __launch_bounds__(kThreads) probabilities_kernel(const T* x, int64_t batch, int nc,
                                                                 int64_t n, int act, float* p) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= batch * n) return;
  const int64_t b = i / n;
  const int64_t off = b * nc * n + (i - b * n);
  float v[kMaxChannels];
#pragma unroll
  for (int c = 0; c < kMaxChannels; ++c) v[c] = c < nc ? to_f32<T>(x[off + c * n]) : 0.0f;
  activate<kMaxChannels, false>(v, nc, act);
#pragma unroll
  for (int c = 0; c < kMaxChannels; ++c)
    if (c < nc) p[off + c * n] = v[c];
}

}  // namespace
}  // namespace ace

namespace ace {
namespace f64 {
// ace_f64.hip: workspace bytes of ace_forward_f64
size_t workspace_bytes(int64_t batch, int64_t channels, int64_t voxels, int num_bins, int binning,
                       int include_background);
}  // namespace f64
}  // namespace ace

using namespace ace;

extern "C" {

int ace_abi_version(void) { return 9; }

const char* ace_error_string(int code) {
  switch (code) {
    case ACE_OK: return "success";
    case ACE_EINVAL: return "invalid argument";
    case ACE_EUNSUPPORTED: return "unsupported configuration (channels > 64 or LDS too large)";
    case ACE_EWORKSPACE: return "workspace smaller than ace_workspace_bytes()";
    case ACE_ESCRATCH:
      return "problem needs more workspace than ace_forward_noalloc's scratch "
             "(ACE_NOALLOC_SCRATCH_BYTES); use ace_forward with a workspace";
    default: break;
  }
  if (code >= ACE_EHIP) return hipGetErrorString((hipError_t)(code - ACE_EHIP));
  return "unknown error";
}

size_t ace_workspace_bytes(int64_t batch, int64_t channels, int64_t voxels, int num_bins,
                           int binning, int x_dtype, int include_background, int target_kind) {
  if (batch < 1 || channels < 1 || voxels < 0 || num_bins < 1) return 0;
  if (x_dtype == ACE_F64)
    return f64::workspace_bytes(batch, channels, voxels, num_bins, binning, include_background);
  return workspace_size(batch, channels, voxels, num_bins, binning, include_background,
                        target_kind);
}

size_t ace_workspace_reset_bytes(int64_t batch, int64_t channels, int64_t voxels,
                                 int num_bins, int binning, int x_dtype,
                                 int include_background, int target_kind) {
  return ace_workspace_bytes(batch, channels, voxels, num_bins, binning, x_dtype,
                             include_background, target_kind);
}

int ace_forward(const void* x, int x_dtype, const void* target, int target_kind,
                int64_t batch, int64_t channels, int64_t voxels, int num_bins, int binning,
                int activation, int include_background, int ignore_empty_classes,
                int reduction, int right, float empty_weight, const float* class_weight,
                const float* bin_table, const float* centre_table, void* workspace,
                size_t workspace_bytes, float* coef, float* diff, float* jac,
                float* per_class, float* loss, double* stats, void* stream) {
  int rc = check_common(x, x_dtype, target, target_kind, batch, channels, voxels, num_bins,
                        binning, activation, bin_table, centre_table, true);
  if (rc) return rc;
  if (reduction != ACE_RED_MEAN && reduction != ACE_RED_SUM && reduction != ACE_RED_NONE)
    return ACE_EINVAL;
  if (!workspace || !coef || !diff || !jac || !per_class) return ACE_EINVAL;
  if (reduction != ACE_RED_NONE && !loss) return ACE_EINVAL;
  const bool soft = binning == ACE_SOFT;
  const bool labels = target_kind == ACE_TARGET_LABELS_I64;
  const ForwardPlan fp = plan_forward(batch, channels, voxels, num_bins, binning, activation,
                                      include_background, target_kind);
  if (fp.rc) return fp.rc;
  const Geometry& g = fp.g;
  const int act = fp.act;
  const bool moments = fp.moments;
  if (workspace_bytes < g.ws_bytes) return ACE_EWORKSPACE;

  const FwdParams p = fwd_params(x, x_dtype, target, labels, voxels, batch, channels, num_bins, act,
                                  ignore_empty_classes, reduction, empty_weight, moments, class_weight,
                                  bin_table, centre_table, workspace, g, coef, diff, jac, per_class,
                                  loss, stats);
  return to_code(dispatch_fwd(x_dtype, soft, right != 0, g, p, static_cast<hipStream_t>(stream)));
}

int ace_backward(const void* x, int x_dtype, const void* target, int target_kind,
                 int64_t batch, int64_t channels, int64_t voxels, int num_bins, int binning,
                 int activation, int include_background, int right, const float* bin_table,
                 const float* centre_table, const float* coef, const float* diff,
                 const float* jac, const float* grad_output, int grad_output_per_class,
                 void* dx, void* stream) {
  const bool soft = binning == ACE_SOFT;
  int rc = check_common(x, x_dtype, target, target_kind, batch, channels, voxels, num_bins,
                        binning, activation, bin_table, centre_table, soft);
  if (rc) return rc;
  if (!coef || !jac || !grad_output || (!dx && voxels > 0)) return ACE_EINVAL;
  if (soft && !diff) return ACE_EINVAL;
  const bool labels = target_kind == ACE_TARGET_LABELS_I64;
  const int act = (activation == ACE_ACT_SOFTMAX && channels == 1) ? kActNone : activation;
  const bool moments =
      use_moments(soft, labels, act, batch, channels, voxels, num_bins, include_background);
  const Geometry g = make_geometry(
      batch, channels, voxels, num_bins, soft, include_background != 0, labels,
      bwd_steps(soft, labels, act, batch, channels, voxels, include_background, moments), 0,
      moments, false, kFastThreads, true);
  if (g.lds_bwd > kMaxLds) return ACE_EUNSUPPORTED;
  if (g.nblk > 0x7fffffffLL) return ACE_EUNSUPPORTED;
  if (voxels == 0) return ACE_OK;

  const BwdParams p = bwd_params(x, x_dtype, target, labels, soft, voxels, batch, channels, num_bins,
                                  act, bin_table, centre_table, coef, diff, jac, grad_output,
                                  grad_output_per_class, dx, g);
  return to_code(dispatch_bwd(x_dtype, soft, right != 0, g, p, static_cast<hipStream_t>(stream)));
}

size_t ace_workspace_bytes_levels(int levels, const int64_t* voxels, int64_t batch,
                                  int64_t channels, int num_bins, int binning, int x_dtype,
                                  int include_background) {
  (void)x_dtype;
  if (levels < 1 || levels > kMaxLevels || !voxels || batch < 1 || channels < 1 || num_bins < 1)
    return 0;
  size_t total = 0;
  for (int l = 0; l < levels; ++l) {
    if (voxels[l] < 0) return 0;
    total += level_ws_bytes(batch, channels, voxels[l], num_bins, binning, include_background);
  }
  return total;
}

int ace_forward_levels(int levels, const AceFwdLevel* lv, int x_dtype, int64_t batch,
                       int64_t channels, int num_bins, int binning, int include_background,
                       int ignore_empty_classes, int reduction, int right, float empty_weight,
                       const float* class_weight, const float* bin_table,
                       const float* centre_table, void* workspace, size_t workspace_bytes,
                       void* stream) {
  if (levels < 1 || levels > kMaxLevels || !lv || !workspace) return ACE_EINVAL;
  if (reduction != ACE_RED_MEAN && reduction != ACE_RED_SUM && reduction != ACE_RED_NONE)
    return ACE_EINVAL;
  if (!fast_channels(channels)) return ACE_EUNSUPPORTED;
  const bool soft = binning == ACE_SOFT;
  // every level in one launch, in 256-thread blocks: with the small levels'
  // many short blocks beside the large one, 1024-thread blocks measured
  // slower on MI355X (four SegResNetDS levels, hard, HIP graph: 61.6 vs
  // 57.7 us per step)
  const int max_nt = kThreads;
  for (int l = 0; l < levels; ++l)
    if (lv[l].voxels < 0) return ACE_EINVAL;
  FwdLevels L{};
  L.n = levels;
  L.nt = max_nt;
  long long nblk = 0;
  size_t lds = 0, off = 0;
  int cmax = 0;
  for (int l = 0; l < levels; ++l) {
    const AceFwdLevel& v = lv[l];
    int rc = check_common(v.x, x_dtype, v.target, ACE_TARGET_LABELS_I64, batch, channels, v.voxels,
                          num_bins, binning, ACE_ACT_SOFTMAX, bin_table, centre_table, true);
    if (rc) return rc;
    if (!v.coef || !v.diff || !v.jac || !v.per_class) return ACE_EINVAL;
    if (reduction != ACE_RED_NONE && !v.loss) return ACE_EINVAL;
    const bool moments = use_moments(soft, true, kActSoftmax, batch, channels, v.voxels, num_bins,
                                     include_background);
    if (soft && !moments) return ACE_EUNSUPPORTED;
    const Geometry g = forward_geometry(batch, channels, v.voxels, num_bins, soft,
                                        include_background, true, kActSoftmax, moments, max_nt);
    if (g.lds_fwd > kMaxLds) return ACE_EUNSUPPORTED;
    // one launch, one block size: every level's geometry must use it
    if (g.nt != L.nt) return ACE_EUNSUPPORTED;
    if (nblk + g.nblk > 0x7fffffffLL) return ACE_EUNSUPPORTED;
    L.lv[l] = fwd_params(v.x, x_dtype, v.target, true, v.voxels, batch, channels, num_bins,
                         kActSoftmax, ignore_empty_classes, reduction, empty_weight, moments,
                         class_weight, bin_table, centre_table,
                         static_cast<unsigned char*>(workspace) + off, g, v.coef, v.diff, v.jac,
                         v.per_class, v.loss, nullptr);
    L.start[l] = nblk;
    nblk += g.nblk;
    lds = g.lds_fwd > lds ? g.lds_fwd : lds;
    cmax = g.var.cmax;
    off += level_ws_bytes(batch, channels, v.voxels, num_bins, binning, include_background);
  }
  if (workspace_bytes < off) return ACE_EWORKSPACE;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (x_dtype) {
    case ACE_F32: e = pick_levels_fwd<float>(soft, right != 0, cmax, nblk, lds, L, s); break;
    case ACE_BF16: e = pick_levels_fwd<__hip_bfloat16>(soft, right != 0, cmax, nblk, lds, L, s); break;
    default: e = pick_levels_fwd<__half>(soft, right != 0, cmax, nblk, lds, L, s); break;
  }
  return to_code(e);
}

int ace_backward_levels(int levels, const AceBwdLevel* lv, int x_dtype, int64_t batch,
                        int64_t channels, int num_bins, int binning, int include_background,
                        int right, int grad_output_per_class, const float* bin_table,
                        const float* centre_table, void* stream) {
  if (levels < 1 || levels > kMaxLevels || !lv) return ACE_EINVAL;
  if (!fast_channels(channels)) return ACE_EUNSUPPORTED;
  const bool soft = binning == ACE_SOFT;
  BwdLevels L{};
  L.n = levels;
  long long nblk = 0;
  size_t lds = 0;
  int cmax = 0;
  for (int l = 0; l < levels; ++l) {
    const AceBwdLevel& v = lv[l];
    int rc = check_common(v.x, x_dtype, v.target, ACE_TARGET_LABELS_I64, batch, channels, v.voxels,
                          num_bins, binning, ACE_ACT_SOFTMAX, bin_table, centre_table, soft);
    if (rc) return rc;
    if (!v.coef || !v.jac || !v.grad_output || (!v.dx && v.voxels > 0)) return ACE_EINVAL;
    if (soft && !v.diff) return ACE_EINVAL;
    const bool moments = use_moments(soft, true, kActSoftmax, batch, channels, v.voxels, num_bins,
                                     include_background);
    if (soft && !moments) return ACE_EUNSUPPORTED;
    const Geometry g = make_geometry(
        batch, channels, v.voxels, num_bins, soft, include_background != 0, true,
        bwd_steps(soft, true, kActSoftmax, batch, channels, v.voxels, include_background, moments),
        0, moments);
    if (g.lds_bwd > kMaxLds) return ACE_EUNSUPPORTED;
    if (nblk + g.nblk > 0x7fffffffLL) return ACE_EUNSUPPORTED;
    L.lv[l] = bwd_params(v.x, x_dtype, v.target, true, soft, v.voxels, batch, channels, num_bins,
                         kActSoftmax, bin_table, centre_table, v.coef, v.diff, v.jac,
                         v.grad_output, grad_output_per_class, v.dx, g);
    L.start[l] = nblk;
    // a level with no voxels launches no blocks (ace_backward returns early)
    nblk += v.voxels > 0 ? g.nblk : 0;
    lds = g.lds_bwd > lds ? g.lds_bwd : lds;
    cmax = g.var.cmax;
  }
  if (nblk == 0) return ACE_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (x_dtype) {
    case ACE_F32: e = pick_levels_bwd<float>(soft, right != 0, cmax, nblk, lds, L, s); break;
    case ACE_BF16: e = pick_levels_bwd<__hip_bfloat16>(soft, right != 0, cmax, nblk, lds, L, s); break;
    default: e = pick_levels_bwd<__half>(soft, right != 0, cmax, nblk, lds, L, s); break;
  }
  return to_code(e);
}

int ace_forward_noalloc(const void* x, int x_dtype, const void* target, int target_kind,
                        int64_t batch, int64_t channels, int64_t voxels, int num_bins,
                        int binning, int activation, int include_background,
                        int ignore_empty_classes, int reduction, int right, float empty_weight,
                        const float* class_weight, const float* bin_table,
                        const float* centre_table, float* coef, float* diff, float* jac,
                        float* per_class, float* loss, double* stats, void* stream) {
  // the checks ace_forward makes before it looks at the workspace (arguments,
  // then the launch plan), so that an invalid or unsupported call launches
  // nothing
  int rc = check_common(x, x_dtype, target, target_kind, batch, channels, voxels, num_bins,
                        binning, activation, bin_table, centre_table, true);
  if (rc) return rc;
  if (reduction != ACE_RED_MEAN && reduction != ACE_RED_SUM && reduction != ACE_RED_NONE)
    return ACE_EINVAL;
  if (!coef || !diff || !jac || !per_class) return ACE_EINVAL;
  if (reduction != ACE_RED_NONE && !loss) return ACE_EINVAL;
  rc = plan_forward(batch, channels, voxels, num_bins, binning, activation, include_background,
                    target_kind).rc;
  if (rc) return rc;
  const size_t need = ace_workspace_reset_bytes(batch, channels, voxels, num_bins, binning, x_dtype,
                                                include_background, target_kind);
  if (need == 0) return ACE_EINVAL;
  if (need > ACE_NOALLOC_SCRATCH_BYTES) return ACE_ESCRATCH;
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc) return rc;
  // the scratch holds whatever the last call on this device left: clear the
  // bytes that must start zero, in stream order before the forward
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t words = need / sizeof(unsigned long long);
  const int64_t blocks = cdiv((int64_t)words, (int64_t)kThreads);
  hipLaunchKernelGGL(clear_words, dim3((unsigned)(blocks < 256 ? blocks : 256)), dim3(kThreads), 0,
                     s, static_cast<unsigned long long*>(ws), words);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return to_code(e);
  return ace_forward(x, x_dtype, target, target_kind, batch, channels, voxels, num_bins, binning,
                     activation, include_background, ignore_empty_classes, reduction, right,
                     empty_weight, class_weight, bin_table, centre_table, ws,
                     ACE_NOALLOC_SCRATCH_BYTES, coef, diff, jac, per_class, loss, stats, stream);
}

int ace_set_launch_events(void* start, void* stop) {
  launch_events() = LaunchEvents{static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)};
  return ACE_OK;
}

int ace_set_timeline(void* stamps) {
  g_timeline.store(static_cast<unsigned long long*>(stamps), std::memory_order_relaxed);
  return ACE_OK;
}

size_t ace_read_bytes_scratch(void) { return kReadBlocks * sizeof(unsigned); }

int ace_read_bytes(const void* a, size_t a_bytes, const void* b, size_t b_bytes, void* scratch,
                   void* stream) {
  if ((!a && a_bytes) || (!b && b_bytes) || !scratch) return ACE_EINVAL;
  if (!aligned_to(a, 16) || !aligned_to(b, 16) || (a_bytes % 16) || (b_bytes % 16)) return ACE_EINVAL;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const LaunchEvents& ev = launch_events();
  const uint4* pa = static_cast<const uint4*>(a);
  const uint4* pb = static_cast<const uint4*>(b);
  const size_t na = a_bytes / 16, nb = b_bytes / 16;
  unsigned* out = static_cast<unsigned*>(scratch);
  if (ev.start || ev.stop) {
    void* args[] = {&pa, const_cast<size_t*>(&na), &pb, const_cast<size_t*>(&nb), &out};
    return to_code(hipExtLaunchKernel(reinterpret_cast<const void*>(read_bytes_kernel),
                                      dim3(kReadBlocks), dim3(kFastThreads), args, 0, s, ev.start,
                                      ev.stop, 0));
  }
  hipLaunchKernelGGL(read_bytes_kernel, dim3(kReadBlocks), dim3(kFastThreads), 0, s, pa, na, pb, nb, out);
  return to_code(hipGetLastError());
}

int ace_probabilities(const void* x, int x_dtype, int64_t batch, int64_t channels, int64_t voxels,
                      int activation, float* p, void* stream) {
  if (batch < 0 || channels < 1 || voxels < 0) return ACE_EINVAL;
  if (activation < kActNone || activation > kActSigmoid) return ACE_EINVAL;
  if (channels > kMaxChannels) return ACE_EUNSUPPORTED;
  const int64_t n = batch * voxels;
  if (n == 0) return ACE_OK;
  if (!x || !p) return ACE_EINVAL;
  if ((n + kThreads - 1) / kThreads > INT32_MAX) return ACE_EUNSUPPORTED;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((n + kThreads - 1) / kThreads));
  const int nc = (int)channels;
  switch (x_dtype) {
    case ACE_F32:
      hipLaunchKernelGGL(probabilities_kernel<float>, grid, dim3(kThreads), 0, s,
                         static_cast<const float*>(x), batch, nc, voxels, activation, p);
      break;
    case ACE_BF16:
      hipLaunchKernelGGL(probabilities_kernel<__hip_bfloat16>, grid, dim3(kThreads), 0, s,
                         static_cast<const __hip_bfloat16*>(x), batch, nc, voxels, activation, p);
      break;
    case ACE_F16:
      hipLaunchKernelGGL(probabilities_kernel<__half>, grid, dim3(kThreads), 0, s,
                         static_cast<const __half*>(x), batch, nc, voxels, activation, p);
      break;
    default:
      return ACE_EINVAL;
  }
  return to_code(hipGetLastError());
}

int ace_set_test_hooks(int max_polls, int publish_delay) {
  if (max_polls > kMaxPolls || publish_delay > (1 << 16)) return ACE_EINVAL;
  g_max_polls.store(max_polls < 0 ? kMaxPolls : max_polls, std::memory_order_relaxed);
  g_publish_delay.store(publish_delay < 0 ? 0 : publish_delay, std::memory_order_relaxed);
  return ACE_OK;
}

}  // extern "C"
