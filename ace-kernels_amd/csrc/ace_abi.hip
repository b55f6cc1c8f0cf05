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

#include "ace_core.hpp"
#include "ace_hip.h"

namespace ace {
#define ACE_DECLARE_LAUNCHERS(T, SOFT)                                                          \
  template <> hipError_t launch_variant_fwd<T, SOFT>(const Geometry&, const FwdParams&, hipStream_t); \
  template <> hipError_t launch_variant_bwd<T, SOFT>(const Geometry&, const BwdParams&, hipStream_t);
ACE_DECLARE_LAUNCHERS(float, false)
ACE_DECLARE_LAUNCHERS(float, true)
ACE_DECLARE_LAUNCHERS(__hip_bfloat16, false)
ACE_DECLARE_LAUNCHERS(__hip_bfloat16, true)
ACE_DECLARE_LAUNCHERS(__half, false)
ACE_DECLARE_LAUNCHERS(__half, true)
#undef ACE_DECLARE_LAUNCHERS

namespace {

constexpr size_t kMaxLds = 160 * 1024;  // gfx950 LDS per workgroup

// Tuning knob for experiments: vector steps per block (0 = automatic).
int env_steps(const char* name) {
  const char* v = getenv(name);
  if (!v) return 0;
  const int s = atoi(v);
  return s > 0 && s <= 1024 ? s : 0;
}

// Cross-block reduction: "tree" (group tickets, default) or "direct"
// (every block adds its partial to the final sums with integer atomics).
int env_reduce_mode() {
  const char* v = getenv("ACE_FWD_REDUCE");
  return (v && v[0] == 'd') ? kReduceDirect : kReduceTree;
}

size_t elem_size(int dtype) { return dtype == ACE_F32 ? 4 : 2; }

bool aligned_to(const void* p, size_t a) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

int check_common(const void* x, int x_dtype, const void* target, int target_kind,
                 int64_t batch, int64_t channels, int64_t voxels, int num_bins,
                 int binning, int activation, const float* bin_table,
                 const float* centre_table, bool need_target) {
  if (!x || !bin_table) return ACE_EINVAL;
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
  if (need_target && !target) return ACE_EINVAL;
  // one channel: to_onehot_y is ignored upstream, the target is per-channel
  if (channels == 1 && target_kind == ACE_TARGET_LABELS_I64 && target) return ACE_EINVAL;
  return ACE_OK;
}

int to_code(hipError_t e) { return e == hipSuccess ? ACE_OK : ACE_EHIP + (int)e; }

}  // namespace
}  // namespace ace

using namespace ace;

extern "C" {

int ace_abi_version(void) { return 1; }

const char* ace_error_string(int code) {
  switch (code) {
    case ACE_OK: return "success";
    case ACE_EINVAL: return "invalid argument";
    case ACE_EUNSUPPORTED: return "unsupported configuration (channels > 64 or LDS too large)";
    case ACE_EWORKSPACE: return "workspace smaller than ace_workspace_bytes()";
    default: break;
  }
  if (code >= ACE_EHIP) return hipGetErrorString((hipError_t)(code - ACE_EHIP));
  return "unknown error";
}

size_t ace_workspace_bytes(int64_t batch, int64_t channels, int64_t voxels, int num_bins,
                           int binning, int x_dtype, int include_background) {
  (void)x_dtype;
  if (batch < 1 || channels < 1 || voxels < 0 || num_bins < 1) return 0;
  const Geometry g = make_geometry(batch, channels, voxels, num_bins, binning == ACE_SOFT,
                                   include_background != 0, true, env_steps("ACE_FWD_STEPS"));
  return g.ws_bytes;
}

size_t ace_workspace_reset_bytes(int64_t batch, int64_t channels, int64_t voxels,
                                 int num_bins, int binning, int x_dtype,
                                 int include_background) {
  (void)x_dtype;
  if (batch < 1 || channels < 1 || voxels < 0 || num_bins < 1) return 0;
  const Geometry g = make_geometry(batch, channels, voxels, num_bins, binning == ACE_SOFT,
                                   include_background != 0, true, env_steps("ACE_FWD_STEPS"));
  return g.ws_counters;
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
  const Geometry g = make_geometry(batch, channels, voxels, num_bins, soft,
                                   include_background != 0, labels, env_steps("ACE_FWD_STEPS"));
  if (workspace_bytes < g.ws_bytes) return ACE_EWORKSPACE;
  if (g.lds_fwd > kMaxLds) return ACE_EUNSUPPORTED;
  if (g.nblk > 0x7fffffffLL) return ACE_EUNSUPPORTED;

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
  p.act = (activation == ACE_ACT_SOFTMAX && channels == 1) ? kActNone : activation;
  p.tk = labels ? kTgtLabels : kTgtOnehot;
  p.right = right != 0;
  p.copies = g.copies;
  p.vec_ok = vec_ok ? 1 : 0;
  p.ignore_empty = ignore_empty_classes != 0;
  p.red = reduction;
  p.empty_w = empty_weight;
  p.btab = bin_table;
  p.rtab = centre_table;
  p.clsw = class_weight;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  p.ctr = reinterpret_cast<int*>(ws);
  p.fin = reinterpret_cast<unsigned long long*>(ws + g.off_fin);
  p.part = reinterpret_cast<long long*>(ws + g.off_part);
  p.mode = env_reduce_mode();
  p.epi_batch = g.epi_batch;
  p.coef = coef;
  p.d = diff;
  p.jac = jac;
  p.f = per_class;
  p.loss = loss;
  p.stats = stats;

  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (x_dtype) {
    case ACE_F32:
      e = soft ? launch_variant_fwd<float, true>(g, p, s) : launch_variant_fwd<float, false>(g, p, s);
      break;
    case ACE_BF16:
      e = soft ? launch_variant_fwd<__hip_bfloat16, true>(g, p, s)
               : launch_variant_fwd<__hip_bfloat16, false>(g, p, s);
      break;
    default:
      e = soft ? launch_variant_fwd<__half, true>(g, p, s) : launch_variant_fwd<__half, false>(g, p, s);
      break;
  }
  return to_code(e);
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
  if (!coef || !jac || !grad_output || !dx) return ACE_EINVAL;
  if (soft && !diff) return ACE_EINVAL;
  const bool labels = target_kind == ACE_TARGET_LABELS_I64;
  const Geometry g = make_geometry(batch, channels, voxels, num_bins, soft,
                                   include_background != 0, labels, env_steps("ACE_BWD_STEPS"));
  if (g.lds_bwd > kMaxLds) return ACE_EUNSUPPORTED;
  if (g.nblk > 0x7fffffffLL) return ACE_EUNSUPPORTED;
  if (voxels == 0) return ACE_OK;

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
  p.act = (activation == ACE_ACT_SOFTMAX && channels == 1) ? kActNone : activation;
  p.tk = labels ? kTgtLabels : kTgtOnehot;
  p.right = right != 0;
  p.vec_ok = vec_ok ? 1 : 0;
  p.go_per_class = grad_output_per_class != 0;
  p.btab = bin_table;
  p.rtab = centre_table;
  p.coef = coef;
  p.d = diff;
  p.jac = jac;
  p.go = grad_output;

  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  switch (x_dtype) {
    case ACE_F32:
      e = soft ? launch_variant_bwd<float, true>(g, p, s) : launch_variant_bwd<float, false>(g, p, s);
      break;
    case ACE_BF16:
      e = soft ? launch_variant_bwd<__hip_bfloat16, true>(g, p, s)
               : launch_variant_bwd<__hip_bfloat16, false>(g, p, s);
      break;
    default:
      e = soft ? launch_variant_bwd<__half, true>(g, p, s) : launch_variant_bwd<__half, false>(g, p, s);
      break;
  }
  return to_code(e);
}

}  // extern "C"
