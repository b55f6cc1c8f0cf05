// The autograd node of hip_mi355x in C++: the host side of one loss call
// (output allocation, the ace_forward launch, the backward node and its
// ace_backward launch) without the Python autograd Function, for call
// signatures whose arguments are fixed (ace_kernels/impls/hip_mi355x.py:
// _Call).  It mirrors the reference's `_V6Loss` autograd Function
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
  // `saved` (float32): coef [B, C', K] at 0, d at o_d, jac [B, C'] at o_jac,
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

void set_entry_points(uintptr_t forward, uintptr_t backward, uintptr_t error_string) {
  g_forward.store(reinterpret_cast<ForwardFn>(forward));
  g_backward.store(reinterpret_cast<BackwardFn>(backward));
  g_error.store(reinterpret_cast<ErrorFn>(error_string));
}

}  // namespace

PYBIND11_MODULE(_ace_autograd, m) {
  m.doc() = "hip_mi355x's loss call and backward node in C++ over libace_hip.so";
  pybind11::class_<Signature, std::shared_ptr<Signature>>(m, "Signature");
  m.def("make_signature", &make_signature);
  m.def("set_entry_points", &set_entry_points);
  m.def("ace_loss", &ace_loss);
}
