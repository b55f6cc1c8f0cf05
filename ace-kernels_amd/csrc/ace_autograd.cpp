// The autograd node of hip_mi355x in C++: the host side of one loss call
// (output allocation, the ace_forward launch, the backward node and its
// ace_backward launch) without the Python autograd Function, for call
// signatures whose arguments are fixed (ace_kernels/impls/hip_mi355x.py:
// _Call); and the same for several levels in one launch per direction
// (ace_kernels/levels.py).  It mirrors the reference's `_V6Loss` autograd Function
// (src/ace_kernels/impls/v6_triton.py:93-111): saved for backward are the
// input, the target and coef / d / jac; the backward returns d input only.
//
// The kernels are reached through the C-ABI of libace_hip.so, by the entry
// points that the Python loader hands over (set_entry_points), so that this
// module and the ctypes binding drive the same loaded library.  Host code
// only: it builds with g++ against torch's headers.
#include <torch/csrc/autograd/function.h>
#include <torch/csrc/autograd/functions/utils.h>
#include <torch/csrc/autograd/saved_variable.h>
#include <torch/extension.h>

#include <c10/hip/HIPStream.h>

#include <atomic>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "ace_hip.h"

namespace {

using torch::autograd::Node;
using torch::autograd::SavedVariable;
using torch::autograd::variable_list;

using ForwardFn = decltype(&ace_forward);
using BackwardFn = decltype(&ace_backward);
using ErrorFn = decltype(&ace_error_string);

std::atomic<ForwardFn> g_forward{nullptr};
std::atomic<BackwardFn> g_backward{nullptr};
std::atomic<ErrorFn> g_error{nullptr};

// The arguments of ace_forward / ace_backward that a call signature fixes.
// Device pointers (tables, class weights, workspace) belong to buffers the
// Python side keeps for the life of the process.
struct Signature {
  int x_dtype = 0, target_kind = 0, num_bins = 0, binning = 0, activation = 0;
  int include_background = 0, ignore_empty = 0, reduction = 0, right = 0;
  int64_t batch = 0, channels = 0, voxels = 0;
  float empty_weight = 0.0f;
  const float* class_weight = nullptr;
  const float* bin_table = nullptr;
  const float* centre_table = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  // `saved` (float32): coef [B, C', K] at 0, d at o_d ([B, C', K], soft
  // [2, B, C', K]: its float32 rounding and remainder), jac [B, C'] at o_jac,
  // and the per-class errors at o_pc unless they are the returned loss
  int64_t n_saved = 0, o_d = 0, o_jac = 0, o_pc = 0;
  bool reduced = true, soft = false;
  std::vector<int64_t> loss_shape;
};

[[noreturn]] void fail(int rc, const char* what) {
  const ErrorFn err = g_error.load(std::memory_order_relaxed);
  throw std::runtime_error(std::string(what) + " failed with code " + std::to_string(rc) + ": " +
                           (err ? err(rc) : "unknown error"));
}

hipStream_t current_stream(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

float* at_offset(const at::Tensor& base, int64_t bytes) {
  return reinterpret_cast<float*>(static_cast<char*>(base.data_ptr()) + bytes);
}

struct AceLossBackward : public Node {
  explicit AceLossBackward(std::shared_ptr<const Signature> s) : sig(std::move(s)) {}

  std::string name() const override { return "AceLossBackward"; }

  variable_list apply(variable_list&& grads) override {
    const Signature& s = *sig;
    at::Tensor x = x_.unpack();
    at::Tensor saved = saved_.unpack();
    at::Tensor target = s.soft ? target_.unpack() : at::Tensor();
    const at::Tensor& g = grads[0];
    if (!g.defined()) return {at::Tensor()};
    at::Tensor go = g;
    if (go.scalar_type() != at::kFloat || !go.is_contiguous()) go = go.to(at::kFloat).contiguous();
    at::Tensor dx = at::empty_like(x, at::MemoryFormat::Contiguous);
    const BackwardFn bwd = g_backward.load(std::memory_order_relaxed);
    if (!bwd) throw std::runtime_error("ace_autograd: entry points not set");
    const int rc = bwd(x.data_ptr(), s.x_dtype, s.soft ? target.data_ptr() : nullptr, s.target_kind,
                       s.batch, s.channels, s.voxels, s.num_bins, s.binning, s.activation,
                       s.include_background, s.right, s.bin_table, s.centre_table,
                       at_offset(saved, 0), at_offset(saved, s.o_d), at_offset(saved, s.o_jac),
                       go.data_ptr<float>(), s.reduced ? 0 : 1, dx.data_ptr(), current_stream(x));
    if (rc) fail(rc, "ace_backward");
    return {dx};
  }

  void release_variables() override {
    x_.reset_data();
    target_.reset_data();
    saved_.reset_data();
  }

  std::shared_ptr<const Signature> sig;
  SavedVariable x_, target_, saved_;
};

// The loss of one call of signature `s` (input and target contiguous, of
// the signature's shapes and dtypes: the Python caller checks), with a
// backward node when the input needs a gradient.
at::Tensor ace_loss(const at::Tensor& x, const at::Tensor& target,
                    const std::shared_ptr<Signature>& sig) {
  const Signature& s = *sig;
  const ForwardFn fwd = g_forward.load(std::memory_order_relaxed);
  if (!fwd) throw std::runtime_error("ace_autograd: entry points not set");
  const c10::DeviceGuard guard(x.device());  // the C-ABI launches on the current device
  const auto opts = x.options().dtype(at::kFloat).requires_grad(false);
  at::Tensor saved = at::empty({s.n_saved}, opts);
  at::Tensor loss = at::empty(s.loss_shape, opts);
  float* lp = loss.data_ptr<float>();
  const int rc = fwd(x.data_ptr(), s.x_dtype, target.data_ptr(), s.target_kind, s.batch, s.channels,
                     s.voxels, s.num_bins, s.binning, s.activation, s.include_background,
                     s.ignore_empty, s.reduction, s.right, s.empty_weight, s.class_weight,
                     s.bin_table, s.centre_table, s.workspace, s.workspace_bytes,
                     at_offset(saved, 0), at_offset(saved, s.o_d), at_offset(saved, s.o_jac),
                     s.reduced ? at_offset(saved, s.o_pc) : lp, s.reduced ? lp : nullptr, nullptr,
                     current_stream(x));
  if (rc) fail(rc, "ace_forward");
  if (torch::autograd::compute_requires_grad(x)) {
    auto node = std::shared_ptr<AceLossBackward>(new AceLossBackward(sig),
                                                 torch::autograd::deleteNode);
    node->set_next_edges(torch::autograd::collect_next_edges(x));
    node->x_ = SavedVariable(x, false);
    if (s.soft) node->target_ = SavedVariable(target, false);
    node->saved_ = SavedVariable(saved, false);
    torch::autograd::set_history(loss, node);
  }
  return loss;
}

// ---------------------------------------------------------------- levels
// Several levels of one loss in one launch per direction (the Python
// counterpart is ace_kernels/levels.py: _HipLevelsLoss): the arguments of
// ace_forward_levels / ace_backward_levels that a levels signature fixes.
// Every level has the same batch, channels and configuration; `voxels`
// holds each level's count.  Each level's coef / d / jac (and per-class
// errors unless they are its loss) sit in one float32 allocation, `n_saved`
// floats per level at the same offsets as in Signature.
struct LevelSignature {
  int x_dtype = 0, num_bins = 0, binning = 0, include_background = 0, ignore_empty = 0;
  int reduction = 0, right = 0;
  int64_t batch = 0, channels = 0;
  float empty_weight = 0.0f;
  const float* class_weight = nullptr;
  const float* bin_table = nullptr;
  const float* centre_table = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  std::vector<int64_t> voxels;
  int64_t n_saved = 0, o_d = 0, o_jac = 0, o_pc = 0;
  bool reduced = true, soft = false;
  std::vector<int64_t> loss_shape;
};

using ForwardLevelsFn = decltype(&ace_forward_levels);
using BackwardLevelsFn = decltype(&ace_backward_levels);
std::atomic<ForwardLevelsFn> g_forward_levels{nullptr};
std::atomic<BackwardLevelsFn> g_backward_levels{nullptr};

struct AceLevelsBackward : public Node {
  explicit AceLevelsBackward(std::shared_ptr<const LevelSignature> s) : sig(std::move(s)) {}

  std::string name() const override { return "AceLevelsBackward"; }

  variable_list apply(variable_list&& grads) override {
    const LevelSignature& s = *sig;
    const size_t n = s.voxels.size();
    const BackwardLevelsFn bwd = g_backward_levels.load(std::memory_order_relaxed);
    if (!bwd) throw std::runtime_error("ace_autograd: entry points not set");
    at::Tensor saved = saved_.unpack();
    std::vector<at::Tensor> xs(n), keep(n);
    std::vector<AceBwdLevel> lv(n);
    variable_list out(n);
    const at::Tensor* ref = nullptr;  // a defined upstream gradient: the shape of any missing one
    for (const at::Tensor& g : grads)
      if (g.defined()) ref = &g;
    if (!ref) return out;
    for (size_t i = 0; i < n; ++i) {
      xs[i] = xs_[i].unpack();
      at::Tensor target = s.soft ? ts_[i].unpack() : at::Tensor();
      at::Tensor go = grads[i].defined() ? grads[i] : at::zeros_like(*ref);
      if (go.scalar_type() != at::kFloat || !go.is_contiguous()) go = go.to(at::kFloat).contiguous();
      keep[i] = go;
      out[i] = at::empty_like(xs[i], at::MemoryFormat::Contiguous);
      const int64_t base = (int64_t)i * s.n_saved * 4;
      lv[i] = AceBwdLevel{xs[i].data_ptr(), s.soft ? target.data_ptr() : nullptr, s.voxels[i],
                          at_offset(saved, base), at_offset(saved, base + s.o_d),
                          at_offset(saved, base + s.o_jac), go.data_ptr<float>(),
                          out[i].data_ptr()};
    }
    const int rc = bwd((int)n, lv.data(), s.x_dtype, s.batch, s.channels, s.num_bins, s.binning,
                       s.include_background, s.right, s.reduced ? 0 : 1, s.bin_table,
                       s.centre_table, current_stream(xs[0]));
    if (rc) fail(rc, "ace_backward_levels");
    for (size_t i = 0; i < n; ++i)
      if (!should_compute_output(i)) out[i] = at::Tensor();
    return out;
  }

  void release_variables() override {
    for (auto& v : xs_) v.reset_data();
    for (auto& v : ts_) v.reset_data();
    saved_.reset_data();
  }

  std::shared_ptr<const LevelSignature> sig;
  std::vector<SavedVariable> xs_, ts_;
  SavedVariable saved_;
};

// The loss of every level from one ace_forward_levels launch, with one
// backward node for all of them when an input needs a gradient.  Inputs and
// targets are contiguous, of the signature's shapes and dtypes (the Python
// caller checks).
std::vector<at::Tensor> ace_loss_levels(const std::vector<at::Tensor>& xs,
                                        const std::vector<at::Tensor>& targets,
                                        const std::shared_ptr<LevelSignature>& sig) {
  const LevelSignature& s = *sig;
  const size_t n = s.voxels.size();
  if (xs.size() != n || targets.size() != n)
    throw std::invalid_argument("ace_loss_levels: one input and one target per level");
  const ForwardLevelsFn fwd = g_forward_levels.load(std::memory_order_relaxed);
  if (!fwd) throw std::runtime_error("ace_autograd: entry points not set");
  const c10::DeviceGuard guard(xs[0].device());
  const auto opts = xs[0].options().dtype(at::kFloat).requires_grad(false);
  at::Tensor saved = at::empty({(int64_t)n * s.n_saved}, opts);
  std::vector<at::Tensor> losses(n);
  std::vector<AceFwdLevel> lv(n);
  for (size_t i = 0; i < n; ++i) {
    losses[i] = at::empty(s.loss_shape, opts);
    float* lp = losses[i].data_ptr<float>();
    const int64_t base = (int64_t)i * s.n_saved * 4;
    lv[i] = AceFwdLevel{xs[i].data_ptr(), targets[i].data_ptr(), s.voxels[i],
                        at_offset(saved, base), at_offset(saved, base + s.o_d),
                        at_offset(saved, base + s.o_jac),
                        s.reduced ? at_offset(saved, base + s.o_pc) : lp,
                        s.reduced ? lp : nullptr};
  }
  const int rc = fwd((int)n, lv.data(), s.x_dtype, s.batch, s.channels, s.num_bins, s.binning,
                     s.include_background, s.ignore_empty, s.reduction, s.right, s.empty_weight,
                     s.class_weight, s.bin_table, s.centre_table, s.workspace, s.workspace_bytes,
                     current_stream(xs[0]));
  if (rc) fail(rc, "ace_forward_levels");
  if (torch::autograd::compute_requires_grad(at::ArrayRef<at::Tensor>(xs))) {
    auto node = std::shared_ptr<AceLevelsBackward>(new AceLevelsBackward(sig),
                                                   torch::autograd::deleteNode);
    node->set_next_edges(torch::autograd::collect_next_edges(at::ArrayRef<at::Tensor>(xs)));
    for (size_t i = 0; i < n; ++i) {
      node->xs_.emplace_back(xs[i], false);
      node->ts_.emplace_back(s.soft ? targets[i] : at::Tensor(), false);
    }
    node->saved_ = SavedVariable(saved, false);
    torch::autograd::set_history(losses, node);
  }
  return losses;
}

std::shared_ptr<LevelSignature> make_level_signature(
    int x_dtype, int64_t batch, int64_t channels, int num_bins, int binning, int include_background,
    int ignore_empty, int reduction, int right, float empty_weight, uintptr_t class_weight,
    uintptr_t bin_table, uintptr_t centre_table, uintptr_t workspace, size_t workspace_bytes,
    std::vector<int64_t> voxels, int64_t n_saved, int64_t o_d, int64_t o_jac, int64_t o_pc,
    bool reduced, bool soft, std::vector<int64_t> loss_shape) {
  if (voxels.empty() || voxels.size() > 4)
    throw std::invalid_argument("make_level_signature: 1 to 4 levels");
  auto s = std::make_shared<LevelSignature>();
  s->x_dtype = x_dtype;
  s->batch = batch;
  s->channels = channels;
  s->num_bins = num_bins;
  s->binning = binning;
  s->include_background = include_background;
  s->ignore_empty = ignore_empty;
  s->reduction = reduction;
  s->right = right;
  s->empty_weight = empty_weight;
  s->class_weight = reinterpret_cast<const float*>(class_weight);
  s->bin_table = reinterpret_cast<const float*>(bin_table);
  s->centre_table = reinterpret_cast<const float*>(centre_table);
  s->workspace = reinterpret_cast<void*>(workspace);
  s->workspace_bytes = workspace_bytes;
  s->voxels = std::move(voxels);
  s->n_saved = n_saved;
  s->o_d = o_d;
  s->o_jac = o_jac;
  s->o_pc = o_pc;
  s->reduced = reduced;
  s->soft = soft;
  s->loss_shape = std::move(loss_shape);
  return s;
}

std::shared_ptr<Signature> make_signature(
    int x_dtype, int target_kind, int64_t batch, int64_t channels, int64_t voxels, int num_bins,
    int binning, int activation, int include_background, int ignore_empty, int reduction,
    int right, float empty_weight, uintptr_t class_weight, uintptr_t bin_table,
    uintptr_t centre_table, uintptr_t workspace, size_t workspace_bytes, int64_t n_saved,
    int64_t o_d, int64_t o_jac, int64_t o_pc, bool reduced, bool soft,
    std::vector<int64_t> loss_shape) {
  auto s = std::make_shared<Signature>();
  s->x_dtype = x_dtype;
  s->target_kind = target_kind;
  s->batch = batch;
  s->channels = channels;
  s->voxels = voxels;
  s->num_bins = num_bins;
  s->binning = binning;
  s->activation = activation;
  s->include_background = include_background;
  s->ignore_empty = ignore_empty;
  s->reduction = reduction;
  s->right = right;
  s->empty_weight = empty_weight;
  s->class_weight = reinterpret_cast<const float*>(class_weight);
  s->bin_table = reinterpret_cast<const float*>(bin_table);
  s->centre_table = reinterpret_cast<const float*>(centre_table);
  s->workspace = reinterpret_cast<void*>(workspace);
  s->workspace_bytes = workspace_bytes;
  s->n_saved = n_saved;
  s->o_d = o_d;
  s->o_jac = o_jac;
  s->o_pc = o_pc;
  s->reduced = reduced;
  s->soft = soft;
  s->loss_shape = std::move(loss_shape);
  return s;
}

void set_entry_points(uintptr_t forward, uintptr_t backward, uintptr_t forward_levels,
                      uintptr_t backward_levels, uintptr_t error_string) {
  g_forward.store(reinterpret_cast<ForwardFn>(forward));
  g_backward.store(reinterpret_cast<BackwardFn>(backward));
  g_forward_levels.store(reinterpret_cast<ForwardLevelsFn>(forward_levels));
  g_backward_levels.store(reinterpret_cast<BackwardLevelsFn>(backward_levels));
  g_error.store(reinterpret_cast<ErrorFn>(error_string));
}

}  // namespace

PYBIND11_MODULE(_ace_autograd, m) {
  m.doc() = "hip_mi355x's loss call and backward node in C++ over libace_hip.so";
  pybind11::class_<Signature, std::shared_ptr<Signature>>(m, "Signature");
  pybind11::class_<LevelSignature, std::shared_ptr<LevelSignature>>(m, "LevelSignature");
  m.def("make_signature", &make_signature);
  m.def("make_level_signature", &make_level_signature);
  m.def("set_entry_points", &set_entry_points);
  m.def("ace_loss", &ace_loss);
  m.def("ace_loss_levels", &ace_loss_levels);
}
