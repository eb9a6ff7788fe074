// torch.ops.fbgemm.* drop-in registrations for the MI355X kernels.
//
// Boundary: the reference plugs a device implementation into its upstream
// project's own interface from a static initializer of a
// torch.ops.load_library()'d module (reference:
// packages/torchcodec-xpu/src/torchcodec_xpu/XpuDeviceInterface.cpp:33-35,
// __init__.py:25-56).  Here the upstream interface is fbgemm_gpu's `fbgemm`
// dispatcher namespace: schemas are defined with TORCH_LIBRARY_FRAGMENT and
// the implementations registered for the CUDA dispatch key, which is the key
// HIP tensors carry on PyTorch-ROCm, plus Autograd wrappers.  Each op
// validates its arguments (TORCH_CHECK -> RuntimeError), takes the current
// HIP stream and calls the C-ABI in libmx_fbgemm_kernels.so; a non-zero
// status becomes a RuntimeError carrying mx_last_error().  No CPU kernels
// are registered: CPU tensors raise the dispatcher's NotImplementedError.
#include <ATen/ATen.h>
#include <ATen/hip/HIPGeneratorImpl.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/csrc/autograd/custom_function.h>
#include <torch/library.h>

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <array>
#include <cstring>
#include <mutex>
#include <vector>

#include "mx_fbgemm.h"

using at::Tensor;
using torch::autograd::AutogradContext;
using torch::autograd::variable_list;

namespace mx_ops {

#define MX_CALL(expr)                                                                  \
  do {                                                                                 \
    const int mx_rc_ = (expr);                                                         \
    TORCH_CHECK(mx_rc_ == MX_OK, #expr " failed (", mx_rc_, "): ", mx_last_error()); \
  } while (0)

void* stream_of(const Tensor& t) {
  return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_gpu(const Tensor& t, const char* name) {
  TORCH_CHECK(t.defined(), name, " must be defined");
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU (HIP) tensor, got ", t.device());
}

void check_same_device(const Tensor& a, const Tensor& b, const char* name) {
  TORCH_CHECK(a.device() == b.device(), name, " is on ", b.device(), " but expected ", a.device());
}

// An argument the kernels read or write by pointer: on `like`'s device and,
// for the small metadata arrays (`dense`), contiguous -- a strided view would
// be read as if it were dense.  Indices, offsets and gradients are made
// contiguous by the callers instead.
void check_arg(const Tensor& t, const Tensor& like, const char* name, bool dense) {
  check_gpu(t, name);
  check_same_device(like, t, name);
  TORCH_CHECK(!dense || t.is_contiguous(), name, " must be contiguous");
}

// ---------------------------------------------------------------------------
// Look-back failures of the sort and scans
// ---------------------------------------------------------------------------
// The kernels report a look-back wait that exhausted its bound (never
// expected) by storing 1 in a host-visible word registered for the device;
// the call's later kernels then leave its outputs (run layout, weights,
// momentum) alone.  The nbit lookup reports a table it cannot serve (its
// columns written as zeros) in a second word.  The pinned words of a device
// are registered on the first backward, transpose or nbit lookup on that
// device outside graph capture; every such op reads them first (a host read,
// no synchronisation) and raises if an earlier call failed.

struct Mailboxes {
  std::mutex mu;
  std::array<Tensor, 64> word;  // int32 [MX_STATUS_WORDS], pinned host memory
};

Mailboxes& mailboxes() {
  static Mailboxes m;
  return m;
}

int32_t* mailbox_of(int dev) {
  auto& m = mailboxes();
  std::lock_guard<std::mutex> lock(m.mu);
  return m.word[dev].defined() ? m.word[dev].data_ptr<int32_t>() : nullptr;
}

// Raises if a look-back of an earlier call on `dev` gave up, or an earlier
// nbit lookup met a table it could not serve (the word is cleared, so each
// failure is reported once).
void raise_if_lookback_failed(int dev) {
  int32_t* p = mailbox_of(dev);
  if (p == nullptr) return;
  if (__atomic_load_n(p + MX_STATUS_LOOKBACK, __ATOMIC_ACQUIRE) != 0) {
    __atomic_store_n(p + MX_STATUS_LOOKBACK, 0, __ATOMIC_RELAXED);
    TORCH_CHECK(false, "an earlier TBE backward or transpose_embedding_input on cuda:", dev,
                " gave up a look-back wait in its sort or scan, so it left its outputs (sorted "
                "indices and run layout, or the weight and momentum update) unwritten; that "
                "step has to be run again");
  }
  if (__atomic_load_n(p + MX_STATUS_NBIT_TABLE, __ATOMIC_ACQUIRE) != 0) {
    __atomic_store_n(p + MX_STATUS_NBIT_TABLE, 0, __ATOMIC_RELAXED);
    TORCH_CHECK(false, "an earlier int_nbit_split_embedding_codegen_lookup_function on cuda:",
                dev, " met a table it cannot serve (a weights_tys byte naming no type whose "
                "max_*_D is positive, an INT4 table of odd D, an INT2 table of D not a "
                "multiple of 4, or rows not starting at 4-byte boundaries: weights_offsets[t] "
                "or the row stride after row_alignment not a multiple of 4; with PoolingMode "
                "NONE also a table whose D is not the largest max_*_D) and wrote that "
                "table's output (columns, or rows of its positions) as zeros");
  }
}

// Registers the device's mailbox (the caller holds a device guard for it).
void ensure_mailbox(int dev, void* stream) {
  TORCH_CHECK(dev >= 0 && dev < 64, "device index ", dev, " out of range");
  raise_if_lookback_failed(dev);
  if (mailbox_of(dev) != nullptr) return;
  // The pinned allocation is left to a call that is not being captured.
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(reinterpret_cast<hipStream_t>(stream), &cs) != hipSuccess ||
      cs != hipStreamCaptureStatusNone)
    return;
  Tensor w = at::zeros({MX_STATUS_WORDS}, at::TensorOptions().dtype(at::kInt).pinned_memory(true));
  auto& m = mailboxes();
  std::lock_guard<std::mutex> lock(m.mu);
  if (m.word[dev].defined()) return;
  MX_CALL(mx_set_status_mailbox(reinterpret_cast<unsigned int*>(w.data_ptr<int32_t>())));
  m.word[dev] = w;
}

// mx_fbgemm::pending_lookback_faults(device): waits for the device, then
// returns (and clears) its look-back failure word.
int64_t pending_lookback_faults(int64_t device) {
  TORCH_CHECK(device >= 0 && device < 64, "device index ", device, " out of range");
  c10::DeviceGuard guard(c10::Device(c10::DeviceType::CUDA, static_cast<int8_t>(device)));
  TORCH_CHECK(hipDeviceSynchronize() == hipSuccess, "hipDeviceSynchronize failed");
  int32_t* p = mailbox_of(static_cast<int>(device));
  if (p == nullptr) return 0;
  const int32_t v = __atomic_load_n(p + MX_STATUS_LOOKBACK, __ATOMIC_ACQUIRE);
  __atomic_store_n(p + MX_STATUS_LOOKBACK, 0, __ATOMIC_RELAXED);
  return v;
}

// mx_fbgemm::test_force_lookback_giveup(enable): failure-handling tests only --
// every look-back wait of later calls gives up at once.
void test_force_lookback_giveup(bool enable) {
  MX_CALL(mx_test_force_lookback_giveup(enable ? 1 : 0));
}

// mx_fbgemm::test_force_wide_sort_words(enable): tests only -- later sorts
// keep 64-bit look-back words (the form of sorts of 2^30 keys or more).
void test_force_wide_sort_words(bool enable) {
  MX_CALL(mx_test_force_wide_sort_words(enable ? 1 : 0));
}

// mx_fbgemm::test_force_workspace_counters(enable): tests only -- later eager
// backward calls clear their sort counters in the workspace (the form of
// graph-captured calls) instead of using the stream's zeroed region.
void test_force_workspace_counters(bool enable) {
  MX_CALL(mx_test_force_workspace_counters(enable ? 1 : 0));
}

int32_t index_bytes_of(const Tensor& t, const char* name) {
  TORCH_CHECK(t.scalar_type() == at::kLong || t.scalar_type() == at::kInt, name,
              " must be int32 or int64, got ", t.scalar_type());
  return t.scalar_type() == at::kLong ? 8 : 4;
}

// ---------------------------------------------------------------------------
// Jagged ops
// ---------------------------------------------------------------------------

int32_t mx_dtype_of(at::ScalarType st) {
  switch (st) {
    case at::kFloat: return MX_DTYPE_F32;
    case at::kHalf: return MX_DTYPE_F16;
    case at::kBFloat16: return MX_DTYPE_BF16;
    case at::kDouble: return MX_DTYPE_F64;
    default: return -1;
  }
}

uint64_t pad_bits_of(double pad, at::ScalarType st) {
  // The padding value's bits in the element type, converted by torch's own
  // scalar types (round to nearest even), with no tensor in between.
  uint64_t bits = 0;
  switch (st) {
    case at::kFloat: {
      const float f = static_cast<float>(pad);
      std::memcpy(&bits, &f, sizeof(f));
      break;
    }
    case at::kDouble:
      std::memcpy(&bits, &pad, sizeof(pad));
      break;
    case at::kHalf:
      bits = c10::Half(static_cast<float>(pad)).x;
      break;
    case at::kBFloat16:
      bits = c10::BFloat16(static_cast<float>(pad)).x;
      break;
    default: {
      Tensor p = at::scalar_tensor(pad, at::TensorOptions().dtype(st));
      std::memcpy(&bits, p.data_ptr(), p.element_size());
    }
  }
  return bits;
}

// The offsets of a jagged op as the C-ABI takes them, on the stack (no heap
// allocation per call); contiguous offsets are used in place, others through
// a contiguous copy kept here.
struct OffsetsPack {
  std::array<Tensor, MX_MAX_JAGGED_DIM> keep;
  std::array<const void*, MX_MAX_JAGGED_DIM> ptrs{};
  std::array<int64_t, MX_MAX_JAGGED_DIM> numel{};
  int32_t bytes = 8;
};

void pack_offsets(const std::vector<Tensor>& offsets, const Tensor& like, OffsetsPack& p) {
  TORCH_CHECK(!offsets.empty(), "offsets must hold at least one tensor");
  TORCH_CHECK(offsets.size() <= MX_MAX_JAGGED_DIM, "at most ", MX_MAX_JAGGED_DIM,
              " jagged dimensions are supported, got ", offsets.size());
  p.bytes = index_bytes_of(offsets[0], "offsets");
  for (size_t k = 0; k < offsets.size(); ++k) {
    const Tensor& o = offsets[k];
    check_gpu(o, "offsets");
    check_same_device(like, o, "offsets");
    TORCH_CHECK(o.dim() == 1, "offsets must be 1-D");
    TORCH_CHECK(index_bytes_of(o, "offsets") == p.bytes, "all offsets must share one dtype");
    TORCH_CHECK(o.numel() >= 1, "offsets must not be empty");
    if (o.is_contiguous()) {
      p.ptrs[k] = o.data_ptr();
    } else {
      p.keep[k] = o.contiguous();
      p.ptrs[k] = p.keep[k].data_ptr();
    }
    p.numel[k] = o.numel();
  }
}

Tensor jagged_to_padded_dense_forward(const Tensor& values, const std::vector<Tensor>& offsets,
                                      c10::SymIntArrayRef max_lengths_sym, double padding_value) {
  check_gpu(values, "values");
  c10::OptionalDeviceGuard guard(values.device());
  const auto max_lengths = C10_AS_INTARRAYREF_SLOW(max_lengths_sym);
  TORCH_CHECK(max_lengths.size() == offsets.size(), "max_lengths has ", max_lengths.size(),
              " entries but there are ", offsets.size(), " offsets");
  TORCH_CHECK(values.dim() >= 1, "values must have at least one dimension");
  OffsetsPack p;
  pack_offsets(offsets, values, p);
  const c10::MaybeOwned<Tensor> vm = values.expect_contiguous();
  const Tensor& v = *vm;
  const int64_t inner_elems = v.dim() == 1 ? 1 : c10::multiply_integers(v.sizes().slice(1));
  at::DimVector shape{p.numel[0] - 1};
  for (auto m : max_lengths) shape.push_back(m);
  for (int64_t d = 1; d < v.dim(); ++d) shape.push_back(v.size(d));
  Tensor out = at::empty(shape, v.options());
  MX_CALL(mx_jagged_to_padded_dense(v.data_ptr(), v.element_size(), inner_elems,
                                    static_cast<int32_t>(offsets.size()), p.ptrs.data(), p.bytes,
                                    p.numel.data(), max_lengths.data(),
                                    pad_bits_of(padding_value, v.scalar_type()), out.data_ptr(),
                                    stream_of(v)));
  return out;
}

int64_t last_offset(const Tensor& o) { return o.numel() == 0 ? 0 : o[-1].item<int64_t>(); }

Tensor dense_to_jagged_forward(const Tensor& dense, const std::vector<Tensor>& offsets,
                               std::optional<c10::SymInt> total_L_sym) {
  check_gpu(dense, "dense");
  c10::OptionalDeviceGuard guard(dense.device());
  const int64_t nd = static_cast<int64_t>(offsets.size());
  TORCH_CHECK(dense.dim() >= 1 + nd, "dense must have at least ", 1 + nd, " dimensions");
  OffsetsPack p;
  pack_offsets(offsets, dense, p);
  TORCH_CHECK(dense.size(0) == p.numel[0] - 1, "dense has ", dense.size(0),
              " rows but offsets describe ", p.numel[0] - 1);
  const c10::MaybeOwned<Tensor> dm = dense.expect_contiguous();
  const Tensor& d = *dm;
  std::array<int64_t, MX_MAX_JAGGED_DIM> max_lengths{};
  for (int64_t k = 0; k < nd; ++k) max_lengths[k] = d.size(1 + k);
  const int64_t total_L =
      total_L_sym.has_value() ? total_L_sym->expect_int() : last_offset(offsets.back());
  TORCH_CHECK(total_L >= 0, "total_L must be non-negative");
  at::DimVector shape{total_L};
  int64_t inner = 1;
  for (int64_t k = 1 + nd; k < d.dim(); ++k) {
    shape.push_back(d.size(k));
    inner *= d.size(k);
  }
  Tensor out = at::empty(shape, d.options());
  MX_CALL(mx_dense_to_jagged(d.data_ptr(), d.element_size(), inner, static_cast<int32_t>(nd),
                             p.ptrs.data(), p.bytes, p.numel.data(), max_lengths.data(), total_L,
                             out.data_ptr(), stream_of(d)));
  return out;
}

Tensor jagged_dense_add_forward(const Tensor& x_values, const std::vector<Tensor>& offsets,
                                const Tensor& y) {
  check_gpu(x_values, "x_values");
  check_gpu(y, "y");
  check_same_device(x_values, y, "y");
  c10::OptionalDeviceGuard guard(x_values.device());
  TORCH_CHECK(x_values.scalar_type() == y.scalar_type(), "x_values and y must share a dtype");
  const int32_t dt = mx_dtype_of(x_values.scalar_type());
  TORCH_CHECK(dt >= 0, "dtype ", x_values.scalar_type(), " is not supported");
  const int64_t nd = static_cast<int64_t>(offsets.size());
  TORCH_CHECK(y.dim() >= 1 + nd, "y must have at least ", 1 + nd, " dimensions");
  OffsetsPack p;
  pack_offsets(offsets, x_values, p);
  TORCH_CHECK(y.size(0) == p.numel[0] - 1, "y has ", y.size(0), " rows but offsets describe ",
              p.numel[0] - 1);
  const c10::MaybeOwned<Tensor> xm = x_values.expect_contiguous();
  const c10::MaybeOwned<Tensor> ym = y.expect_contiguous();
  const Tensor& x = *xm;
  const Tensor& yc = *ym;
  std::array<int64_t, MX_MAX_JAGGED_DIM> max_lengths{};
  for (int64_t k = 0; k < nd; ++k) max_lengths[k] = yc.size(1 + k);
  int64_t inner = 1;
  for (int64_t k = 1 + nd; k < yc.dim(); ++k) inner *= yc.size(k);
  const int64_t x_inner = x.dim() == 1 ? 1 : c10::multiply_integers(x.sizes().slice(1));
  TORCH_CHECK(x_inner == inner, "x_values inner size ", x_inner, " != y inner size ", inner);
  Tensor out = at::empty_like(x);
  MX_CALL(mx_jagged_dense_elementwise_add(x.data_ptr(), yc.data_ptr(), dt, inner,
                                          static_cast<int32_t>(nd), p.ptrs.data(), p.bytes,
                                          p.numel.data(), max_lengths.data(), x.size(0),
                                          out.data_ptr(), stream_of(x)));
  return out;
}

Tensor jagged_dense_mul_forward(const Tensor& x_values, const std::vector<Tensor>& offsets,
                                const Tensor& y) {
  check_gpu(x_values, "x_values");
  check_gpu(y, "y");
  check_same_device(x_values, y, "y");
  c10::OptionalDeviceGuard guard(x_values.device());
  TORCH_CHECK(x_values.scalar_type() == y.scalar_type(), "x_values and y must share a dtype");
  const int32_t dt = mx_dtype_of(x_values.scalar_type());
  TORCH_CHECK(dt >= 0, "dtype ", x_values.scalar_type(), " is not supported");
  const int64_t nd = static_cast<int64_t>(offsets.size());
  TORCH_CHECK(y.dim() >= 1 + nd, "y must have at least ", 1 + nd, " dimensions");
  OffsetsPack p;
  pack_offsets(offsets, x_values, p);
  TORCH_CHECK(y.size(0) == p.numel[0] - 1, "y has ", y.size(0), " rows but offsets describe ",
              p.numel[0] - 1);
  const c10::MaybeOwned<Tensor> xm = x_values.expect_contiguous();
  const c10::MaybeOwned<Tensor> ym = y.expect_contiguous();
  const Tensor& x = *xm;
  const Tensor& yc = *ym;
  std::array<int64_t, MX_MAX_JAGGED_DIM> max_lengths{};
  for (int64_t k = 0; k < nd; ++k) max_lengths[k] = yc.size(1 + k);
  int64_t inner = 1;
  for (int64_t k = 1 + nd; k < yc.dim(); ++k) inner *= yc.size(k);
  const int64_t x_inner = x.dim() == 1 ? 1 : c10::multiply_integers(x.sizes().slice(1));
  TORCH_CHECK(x_inner == inner, "x_values inner size ", x_inner, " != y inner size ", inner);
  Tensor out = at::empty_like(x);
  MX_CALL(mx_jagged_dense_elementwise_mul(x.data_ptr(), yc.data_ptr(), dt, inner,
                                          static_cast<int32_t>(nd), p.ptrs.data(), p.bytes,
                                          p.numel.data(), max_lengths.data(), x.size(0),
                                          out.data_ptr(), stream_of(x)));
  return out;
}

Tensor jagged_to_padded_dense_backward(const Tensor& grad_output,
                                       const std::vector<Tensor>& offsets,
                                       c10::SymInt total_L) {
  return dense_to_jagged_forward(grad_output, offsets, total_L);
}

std::vector<c10::SymInt> sym_lengths(const Tensor& dense, int64_t nd) {
  std::vector<c10::SymInt> v;
  for (int64_t k = 0; k < nd; ++k) v.emplace_back(dense.size(1 + k));
  return v;
}

class JaggedToPaddedDense : public torch::autograd::Function<JaggedToPaddedDense> {
 public:
  static Tensor forward(AutogradContext* ctx, const Tensor& values,
                        const std::vector<Tensor>& offsets, c10::SymIntArrayRef max_lengths,
                        double padding_value) {
    ctx->save_for_backward(offsets);
    ctx->saved_data["total_L"] = values.size(0);
    at::AutoDispatchBelowADInplaceOrView g;
    return jagged_to_padded_dense_forward(values, offsets, max_lengths, padding_value);
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const auto offsets = ctx->get_saved_variables();
    const int64_t total_L = ctx->saved_data["total_L"].toInt();
    // One slot per forward argument (the offsets list is one).
    variable_list out(4);  // values, offsets, max_lengths, padding_value
    out[0] = dense_to_jagged_forward(grads[0], offsets, c10::SymInt(total_L));
    return out;
  }
};

class DenseToJagged : public torch::autograd::Function<DenseToJagged> {
 public:
  static Tensor forward(AutogradContext* ctx, const Tensor& dense,
                        const std::vector<Tensor>& offsets, std::optional<c10::SymInt> total_L) {
    ctx->save_for_backward(offsets);
    std::vector<int64_t> ml;
    for (size_t k = 0; k < offsets.size(); ++k) ml.push_back(dense.size(1 + k));
    ctx->saved_data["max_lengths"] = ml;
    at::AutoDispatchBelowADInplaceOrView g;
    return dense_to_jagged_forward(dense, offsets, total_L);
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const auto offsets = ctx->get_saved_variables();
    const auto ml = ctx->saved_data["max_lengths"].toIntVector();
    std::vector<c10::SymInt> sml(ml.begin(), ml.end());
    variable_list out(3);  // dense, offsets, total_L
    out[0] = jagged_to_padded_dense_forward(grads[0], offsets, sml, 0.0);
    return out;
  }
};

class JaggedDenseAdd : public torch::autograd::Function<JaggedDenseAdd> {
 public:
  static Tensor forward(AutogradContext* ctx, const Tensor& x, const std::vector<Tensor>& offsets,
                        const Tensor& y) {
    ctx->save_for_backward(offsets);
    std::vector<int64_t> ml;
    for (size_t k = 0; k < offsets.size(); ++k) ml.push_back(y.size(1 + k));
    ctx->saved_data["max_lengths"] = ml;
    at::AutoDispatchBelowADInplaceOrView g;
    return jagged_dense_add_forward(x, offsets, y);
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    const auto offsets = ctx->get_saved_variables();
    const auto ml = ctx->saved_data["max_lengths"].toIntVector();
    std::vector<c10::SymInt> sml(ml.begin(), ml.end());
    variable_list out(3);  // x, offsets (one argument), y
    out[0] = grads[0];
    out[2] = jagged_to_padded_dense_forward(grads[0], offsets, sml, 0.0);
    return out;
  }
};

// d(x * y): grad_x = grad * y at the coordinates (the mul again), grad_y =
// the padded dense of grad * x (zero where no jagged element lies).
class JaggedDenseMul : public torch::autograd::Function<JaggedDenseMul> {
 public:
  static Tensor forward(AutogradContext* ctx, const Tensor& x, const std::vector<Tensor>& offsets,
                        const Tensor& y) {
    std::vector<Tensor> keep(offsets);
    keep.push_back(x);
    keep.push_back(y);
    ctx->save_for_backward(keep);
    ctx->saved_data["num_offsets"] = static_cast<int64_t>(offsets.size());
    at::AutoDispatchBelowADInplaceOrView g;
    return jagged_dense_mul_forward(x, offsets, y);
  }
  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    auto saved = ctx->get_saved_variables();
    const int64_t nd = ctx->saved_data["num_offsets"].toInt();
    const Tensor y = saved.back();
    saved.pop_back();
    const Tensor x = saved.back();
    saved.pop_back();
    std::vector<c10::SymInt> sml;
    for (int64_t k = 0; k < nd; ++k) sml.emplace_back(y.size(1 + k));
    const Tensor g = grads[0].contiguous();
    variable_list out(3);  // x, offsets (one argument), y
    out[0] = jagged_dense_mul_forward(g, saved, y);
    out[2] = jagged_to_padded_dense_forward(g * x, saved, sml, 0.0);
    return out;
  }
};

// The Autograd kernels build a graph node only when a gradient is wanted;
// otherwise they call the forward directly (no node, ~0.7 us less host time
// per call).
bool wants_grad(const Tensor& a, const Tensor& b = Tensor()) {
  return at::GradMode::is_enabled() &&
         (a.requires_grad() || (b.defined() && b.requires_grad()));
}

Tensor jagged_to_padded_dense_autograd(const Tensor& values, const std::vector<Tensor>& offsets,
                                       c10::SymIntArrayRef max_lengths, double padding_value) {
  if (!wants_grad(values))
    return jagged_to_padded_dense_forward(values, offsets, max_lengths, padding_value);
  return JaggedToPaddedDense::apply(values, offsets, max_lengths, padding_value);
}

std::tuple<Tensor, std::vector<Tensor>> dense_to_jagged_autograd(
    const Tensor& dense, const std::vector<Tensor>& offsets, std::optional<c10::SymInt> total_L) {
  if (!wants_grad(dense)) return {dense_to_jagged_forward(dense, offsets, total_L), offsets};
  return {DenseToJagged::apply(dense, offsets, total_L), offsets};
}

std::tuple<Tensor, std::vector<Tensor>> jagged_dense_add_autograd(
    const Tensor& x, const std::vector<Tensor>& offsets, const Tensor& y) {
  if (!wants_grad(x, y)) return {jagged_dense_add_forward(x, offsets, y), offsets};
  return {JaggedDenseAdd::apply(x, offsets, y), offsets};
}

Tensor jagged_dense_mul_autograd(const Tensor& x, const std::vector<Tensor>& offsets,
                                 const Tensor& y) {
  if (!wants_grad(x, y)) return jagged_dense_mul_forward(x, offsets, y);
  return JaggedDenseMul::apply(x, offsets, y);
}

// The older one-dim spellings: values [total_L, D] (2d) or [total_L] (1d).
Tensor jagged_2d_to_dense_autograd(const Tensor& values, const Tensor& offsets,
                                   c10::SymInt max_sequence_length) {
  TORCH_CHECK(values.dim() == 2, "jagged_2d_to_dense takes values [total_L, D]");
  const std::vector<c10::SymInt> ml{max_sequence_length};
  return jagged_to_padded_dense_autograd(values, {offsets}, ml, 0.0);
}

Tensor jagged_2d_to_dense_plain(const Tensor& values, const Tensor& offsets,
                                c10::SymInt max_sequence_length) {
  TORCH_CHECK(values.dim() == 2, "jagged_2d_to_dense takes values [total_L, D]");
  const std::vector<c10::SymInt> ml{max_sequence_length};
  return jagged_to_padded_dense_forward(values, {offsets}, ml, 0.0);
}

Tensor jagged_1d_to_dense(const Tensor& values, const Tensor& offsets,
                          c10::SymInt max_sequence_length, int64_t padding_value) {
  TORCH_CHECK(values.dim() == 1, "jagged_1d_to_dense takes values [total_L]");
  check_gpu(values, "values");
  c10::OptionalDeviceGuard guard(values.device());
  const int64_t max_L = max_sequence_length.expect_int();
  OffsetsPack p;
  pack_offsets({offsets}, values, p);
  const c10::MaybeOwned<Tensor> vm = values.expect_contiguous();
  const Tensor& v = *vm;
  Tensor out = at::empty({p.numel[0] - 1, max_L}, v.options());
  // An integer padding keeps every bit of its type (no trip through a double).
  const uint64_t pad = at::isIntegralType(v.scalar_type(), false)
                           ? static_cast<uint64_t>(padding_value)
                           : pad_bits_of(static_cast<double>(padding_value), v.scalar_type());
  MX_CALL(mx_jagged_to_padded_dense(v.data_ptr(), v.element_size(), 1, 1, p.ptrs.data(), p.bytes,
                                    p.numel.data(), &max_L, pad, out.data_ptr(), stream_of(v)));
  return out;
}

Tensor jagged_to_padded_dense_plain(const Tensor& values, const std::vector<Tensor>& offsets,
                                    c10::SymIntArrayRef max_lengths, double padding_value) {
  return jagged_to_padded_dense_forward(values, offsets, max_lengths, padding_value);
}

std::tuple<Tensor, std::vector<Tensor>> dense_to_jagged_plain(
    const Tensor& dense, const std::vector<Tensor>& offsets, std::optional<c10::SymInt> total_L) {
  return {dense_to_jagged_forward(dense, offsets, total_L), offsets};
}

std::tuple<Tensor, std::vector<Tensor>> jagged_dense_add_plain(
    const Tensor& x, const std::vector<Tensor>& offsets, const Tensor& y) {
  return {jagged_dense_add_forward(x, offsets, y), offsets};
}

// ---------------------------------------------------------------------------
// TBE training
// ---------------------------------------------------------------------------

// DEVICE-only build: a populated LXU cache is refused (the per-table
// placements are validated by the modules; reading them here would need a
// device-to-host copy on every call).
void check_no_cache(const Tensor& lxu_cache_weights) {
  TORCH_CHECK(!lxu_cache_weights.defined() || lxu_cache_weights.numel() == 0,
              "the LXU cache is not supported (DEVICE placement only)");
}

// Variable-batch-per-feature (VBE) metadata of one lookup; undefined tensors
// mean a fixed batch B per table.
struct VbeMeta {
  Tensor B_offsets;  // int32 [T+1]: first bag of each table
  Tensor row_out;    // int64 [total_B]: output (and gradient) row offset of each bag
  Tensor b_t_map;    // int32 [total_B]: (t << info_B_num_bits) | b of each bag
  int64_t output_size = 0;
  int64_t info_B_num_bits = 0;
  int64_t max_B = 0;
  bool on() const { return b_t_map.defined(); }
};

void check_vbe(const VbeMeta& v, int64_t total_B) {
  TORCH_CHECK(v.row_out.defined() && v.b_t_map.defined(), "VBE needs row offsets and a b_t map");
  check_gpu(v.row_out, "vbe_row_output_offsets");
  check_gpu(v.b_t_map, "vbe_b_t_map");
  TORCH_CHECK(v.row_out.scalar_type() == at::kLong && v.row_out.is_contiguous() &&
                  v.row_out.numel() == total_B,
              "vbe_row_output_offsets must be contiguous int64 with one entry per bag");
  TORCH_CHECK(v.b_t_map.scalar_type() == at::kInt && v.b_t_map.is_contiguous() &&
                  v.b_t_map.numel() == total_B,
              "vbe_b_t_map must be contiguous int32 with one entry per bag");
  TORCH_CHECK(v.info_B_num_bits >= 1 && v.info_B_num_bits <= 32, "info_B_num_bits invalid");
}

// Element type of TBE training weights: fp32 or fp16 rows.
int32_t weights_ty_of(const Tensor& w) {
  TORCH_CHECK(w.is_contiguous(), "dev_weights must be contiguous");
  if (w.scalar_type() == at::kFloat) return MX_SPARSE_FP32;
  if (w.scalar_type() == at::kHalf) return MX_SPARSE_FP16;
  TORCH_CHECK(false, "dev_weights must be fp32 or fp16, got ", w.scalar_type());
  return -1;
}

// Random state of one stochastic-rounding update: the device's default
// generator (so torch.manual_seed makes it reproducible), advanced per call.
// philox_cuda_state is torch's capture-safe form: values when eager, device
// pointers plus this call's offset under graph capture, which the kernel
// reads when it runs (each replay then draws new bits).
mx_rng_state next_rounding_state(const Tensor& on) {
  auto gen = at::cuda::detail::getDefaultCUDAGenerator(on.device().index());
  std::lock_guard<std::mutex> lock(gen.mutex());
  const at::PhiloxCudaState st =
      at::check_generator<at::CUDAGeneratorImpl>(gen)->philox_cuda_state(4);
  mx_rng_state r{};
  if (st.captured_) {
    r.seed_dev = st.seed_.ptr;
    r.offset_dev = st.offset_.ptr;
    r.offset = st.offset_intragraph_;
  } else {
    r.seed = st.seed_.val;
    r.offset = st.offset_.val;
  }
  return r;
}

Tensor tbe_forward(const Tensor& dev_weights, const Tensor& uvm_weights,
                   const Tensor& weights_placements, const Tensor& weights_offsets,
                   const Tensor& D_offsets, int64_t total_D, int64_t max_D, const Tensor& indices,
                   const Tensor& offsets, int64_t pooling_mode,
                   const std::optional<Tensor>& indice_weights, int64_t output_dtype,
                   const VbeMeta& vbe = VbeMeta()) {
  check_gpu(dev_weights, "dev_weights");
  c10::OptionalDeviceGuard guard(dev_weights.device());
  check_arg(weights_offsets, dev_weights, "weights_offsets", true);
  check_arg(D_offsets, dev_weights, "D_offsets", true);
  check_arg(indices, dev_weights, "indices", false);
  check_arg(offsets, dev_weights, "offsets", false);
  TORCH_CHECK(uvm_weights.numel() == 0, "UVM weights are not supported (DEVICE placement only)");
  (void)weights_placements;  // validated once by the module; avoided here (host sync)
  const int32_t wty = weights_ty_of(dev_weights);
  TORCH_CHECK(weights_offsets.scalar_type() == at::kLong, "weights_offsets must be int64");
  TORCH_CHECK(D_offsets.scalar_type() == at::kInt, "D_offsets must be int32");
  const int32_t ib = index_bytes_of(indices, "indices");
  TORCH_CHECK(index_bytes_of(offsets, "offsets") == ib, "indices and offsets must share a dtype");
  const int64_t T = D_offsets.numel() - 1;
  TORCH_CHECK(T >= 1, "D_offsets must have T+1 >= 2 entries");
  TORCH_CHECK(weights_offsets.numel() == T, "weights_offsets must have T entries");
  TORCH_CHECK(vbe.on() || (offsets.numel() - 1) % T == 0, "offsets must have T*B+1 entries");
  const int64_t B = vbe.on() ? 0 : (offsets.numel() - 1) / T;
  TORCH_CHECK(output_dtype == MX_SPARSE_FP32 || output_dtype == MX_SPARSE_FP16,
              "output_dtype must be FP32 (0) or FP16 (1)");
  const float* iw = nullptr;
  Tensor iwc;
  if (indice_weights.has_value() && indice_weights->defined()) {
    check_gpu(*indice_weights, "indice_weights");
    TORCH_CHECK(indice_weights->scalar_type() == at::kFloat, "indice_weights must be fp32");
    TORCH_CHECK(indice_weights->numel() == indices.numel(), "indice_weights must match indices");
    iwc = indice_weights->contiguous();
    iw = iwc.data_ptr<float>();
  }
  auto opts = dev_weights.options().dtype(output_dtype == MX_SPARSE_FP16 ? at::kHalf : at::kFloat);
  const Tensor idx = indices.contiguous(), off = offsets.contiguous();
  if (vbe.on()) {  // flat output, one row per bag at its row offset
    const int64_t total_B = offsets.numel() - 1;
    check_vbe(vbe, total_B);
    Tensor out = at::zeros({vbe.output_size}, opts);
    MX_CALL(mx_tbe_forward_vbe(
        dev_weights.data_ptr(), wty, weights_offsets.data_ptr<int64_t>(),
        D_offsets.data_ptr<int32_t>(), static_cast<int32_t>(T), total_B,
        static_cast<int32_t>(max_D), idx.data_ptr(), off.data_ptr(), ib,
        static_cast<int32_t>(pooling_mode), iw, vbe.row_out.data_ptr<int64_t>(),
        vbe.b_t_map.data_ptr<int32_t>(), static_cast<int32_t>(vbe.info_B_num_bits),
        out.data_ptr(), static_cast<int32_t>(output_dtype), stream_of(dev_weights)));
    return out;
  }
  Tensor out = at::empty({B, total_D}, opts);
  MX_CALL(mx_tbe_forward(dev_weights.data_ptr(), wty, weights_offsets.data_ptr<int64_t>(),
                         D_offsets.data_ptr<int32_t>(), static_cast<int32_t>(T), B,
                         static_cast<int32_t>(max_D), idx.data_ptr(), off.data_ptr(), ib,
                         static_cast<int32_t>(pooling_mode), iw, out.data_ptr(),
                         static_cast<int32_t>(output_dtype), total_D, stream_of(dev_weights)));
  return out;
}

// PoolingMode NONE: out [N, D], row l the row of position l.
Tensor tbe_forward_nobag(const Tensor& dev_weights, const Tensor& uvm_weights,
                         const Tensor& weights_offsets, int64_t D, const Tensor& indices,
                         const Tensor& offsets, int64_t output_dtype) {
  check_gpu(dev_weights, "dev_weights");
  c10::OptionalDeviceGuard guard(dev_weights.device());
  check_arg(weights_offsets, dev_weights, "weights_offsets", true);
  check_arg(indices, dev_weights, "indices", false);
  check_arg(offsets, dev_weights, "offsets", false);
  TORCH_CHECK(uvm_weights.numel() == 0, "UVM weights are not supported (DEVICE placement only)");
  const int32_t wty = weights_ty_of(dev_weights);
  TORCH_CHECK(weights_offsets.scalar_type() == at::kLong, "weights_offsets must be int64");
  const int32_t ib = index_bytes_of(indices, "indices");
  TORCH_CHECK(index_bytes_of(offsets, "offsets") == ib, "indices and offsets must share a dtype");
  const int64_t T = weights_offsets.numel();
  TORCH_CHECK(T >= 1 && (offsets.numel() - 1) % T == 0, "offsets must have T*B+1 entries");
  const int64_t B = (offsets.numel() - 1) / T;
  TORCH_CHECK(output_dtype == MX_SPARSE_FP32 || output_dtype == MX_SPARSE_FP16,
              "output_dtype must be FP32 (0) or FP16 (1)");
  const int64_t N = indices.numel();
  auto opts = dev_weights.options().dtype(output_dtype == MX_SPARSE_FP16 ? at::kHalf : at::kFloat);
  Tensor out = at::empty({N, D}, opts);
  const Tensor idx = indices.contiguous(), off = offsets.contiguous();
  MX_CALL(mx_tbe_forward_nobag(dev_weights.data_ptr(), wty, weights_offsets.data_ptr<int64_t>(),
                               static_cast<int32_t>(T), B, static_cast<int32_t>(D),
                               idx.data_ptr(), off.data_ptr(), ib, N, out.data_ptr(),
                               static_cast<int32_t>(output_dtype), stream_of(dev_weights)));
  return out;
}

Tensor forward_nobag_unweighted(const Tensor& dev_weights, const Tensor& uvm_weights,
                                const Tensor& lxu_cache_weights, const Tensor& weights_placements,
                                const Tensor& weights_offsets, c10::SymInt D,
                                const Tensor& indices, const Tensor& offsets,
                                const Tensor& lxu_cache_locations, const Tensor& uvm_cache_stats,
                                int64_t output_dtype, bool is_experimental) {
  check_no_cache(lxu_cache_weights);
  (void)weights_placements;
  (void)lxu_cache_locations;
  (void)uvm_cache_stats;
  (void)is_experimental;
  return tbe_forward_nobag(dev_weights, uvm_weights, weights_offsets, D.expect_int(), indices,
                           offsets, output_dtype);
}

Tensor forward_unweighted(const Tensor& dev_weights, const Tensor& uvm_weights,
                          const Tensor& lxu_cache_weights, const Tensor& weights_placements,
                          const Tensor& weights_offsets, const Tensor& D_offsets,
                          c10::SymInt total_D, c10::SymInt max_D, const Tensor& indices,
                          const Tensor& offsets, int64_t pooling_mode,
                          const Tensor& lxu_cache_locations, const Tensor& uvm_cache_stats,
                          int64_t output_dtype, bool is_experimental) {
  check_no_cache(lxu_cache_weights);
  (void)lxu_cache_locations;
  (void)uvm_cache_stats;
  (void)is_experimental;
  return tbe_forward(dev_weights, uvm_weights, weights_placements, weights_offsets, D_offsets,
                     total_D.expect_int(), max_D.expect_int(), indices, offsets, pooling_mode,
                     std::nullopt, output_dtype);
}

Tensor forward_weighted(const Tensor& dev_weights, const Tensor& uvm_weights,
                        const Tensor& lxu_cache_weights, const Tensor& weights_placements,
                        const Tensor& weights_offsets, const Tensor& D_offsets,
                        c10::SymInt total_D, c10::SymInt max_D, const Tensor& indices,
                        const Tensor& offsets, int64_t pooling_mode, const Tensor& indice_weights,
                        const Tensor& lxu_cache_locations, const Tensor& uvm_cache_stats,
                        int64_t output_dtype, bool is_experimental) {
  check_no_cache(lxu_cache_weights);
  (void)lxu_cache_locations;
  (void)uvm_cache_stats;
  (void)is_experimental;
  return tbe_forward(dev_weights, uvm_weights, weights_placements, weights_offsets, D_offsets,
                     total_D.expect_int(), max_D.expect_int(), indices, offsets, pooling_mode,
                     indice_weights, output_dtype);
}

// ---- variable batch size per feature (VBE) ----------------------------------

VbeMeta vbe_meta(const Tensor& row_out, const Tensor& b_t_map, int64_t output_size,
                 int64_t info_B_num_bits, const Tensor& B_offsets = Tensor(),
                 int64_t max_B = 0) {
  VbeMeta v;
  v.row_out = row_out.contiguous();
  v.b_t_map = b_t_map.contiguous();
  v.output_size = output_size;
  v.info_B_num_bits = info_B_num_bits;
  v.B_offsets = B_offsets;
  v.max_B = max_B;
  return v;
}

// (row_output_offsets int64 [total_B], b_t_map int32 [total_B]).
std::tuple<Tensor, Tensor> generate_vbe_metadata(
    const Tensor& B_offsets, const Tensor& B_offsets_rank_per_feature,
    const Tensor& output_offsets_feature_rank, const Tensor& D_offsets, int64_t D, bool nobag,
    c10::SymInt max_B_feature_rank, int64_t info_B_num_bits, c10::SymInt total_B_sym) {
  (void)max_B_feature_rank;
  check_gpu(B_offsets, "B_offsets");
  for (auto* t : {&B_offsets, &B_offsets_rank_per_feature, &output_offsets_feature_rank,
                  &D_offsets})
    check_arg(*t, B_offsets, "generate_vbe_metadata argument", true);
  c10::OptionalDeviceGuard guard(B_offsets.device());
  TORCH_CHECK(B_offsets.scalar_type() == at::kInt && B_offsets_rank_per_feature.scalar_type() ==
                  at::kInt && D_offsets.scalar_type() == at::kInt,
              "B_offsets, B_offsets_rank_per_feature and D_offsets must be int32");
  TORCH_CHECK(output_offsets_feature_rank.scalar_type() == at::kLong,
              "output_offsets_feature_rank must be int64");
  const int64_t T = B_offsets.numel() - 1;
  TORCH_CHECK(T >= 1 && B_offsets_rank_per_feature.dim() == 2 &&
                  B_offsets_rank_per_feature.size(0) == T,
              "B_offsets_rank_per_feature must be [T, R+1]");
  const int64_t R = B_offsets_rank_per_feature.size(1) - 1;
  TORCH_CHECK(R >= 1 && output_offsets_feature_rank.numel() == R * T + 1,
              "output_offsets_feature_rank must have R*T+1 entries");
  TORCH_CHECK(nobag ? D > 0 : D_offsets.numel() == T + 1, "D_offsets must have T+1 entries");
  const int64_t total_B = total_B_sym.expect_int();
  Tensor row_out = at::empty({total_B}, B_offsets.options().dtype(at::kLong));
  Tensor b_t_map = at::empty({total_B}, B_offsets.options().dtype(at::kInt));
  const Tensor bo = B_offsets.contiguous(), rpf = B_offsets_rank_per_feature.contiguous(),
               ofr = output_offsets_feature_rank.contiguous(), dof = D_offsets.contiguous();
  MX_CALL(mx_generate_vbe_metadata(bo.data_ptr<int32_t>(), rpf.data_ptr<int32_t>(),
                                   ofr.data_ptr<int64_t>(), dof.data_ptr<int32_t>(),
                                   nobag ? static_cast<int32_t>(D) : 0, static_cast<int32_t>(T),
                                   static_cast<int32_t>(R), static_cast<int32_t>(info_B_num_bits),
                                   total_B, row_out.data_ptr<int64_t>(),
                                   b_t_map.data_ptr<int32_t>(), stream_of(B_offsets)));
  return {row_out, b_t_map};
}

Tensor forward_unweighted_vbe(const Tensor& dev_weights, const Tensor& uvm_weights,
                              const Tensor& lxu_cache_weights, const Tensor& weights_placements,
                              const Tensor& weights_offsets, const Tensor& D_offsets,
                              c10::SymInt total_D, c10::SymInt max_D, const Tensor& indices,
                              const Tensor& offsets, int64_t pooling_mode,
                              const Tensor& lxu_cache_locations, const Tensor& uvm_cache_stats,
                              int64_t output_dtype, const Tensor& vbe_row_output_offsets,
                              const Tensor& vbe_b_t_map, c10::SymInt vbe_output_size,
                              int64_t info_B_num_bits, int64_t info_B_mask,
                              bool is_experimental) {
  check_no_cache(lxu_cache_weights);
  (void)lxu_cache_locations;
  (void)uvm_cache_stats;
  (void)info_B_mask;
  (void)is_experimental;
  return tbe_forward(dev_weights, uvm_weights, weights_placements, weights_offsets, D_offsets,
                     total_D.expect_int(), max_D.expect_int(), indices, offsets, pooling_mode,
                     std::nullopt, output_dtype,
                     vbe_meta(vbe_row_output_offsets, vbe_b_t_map, vbe_output_size.expect_int(),
                              info_B_num_bits));
}

Tensor forward_weighted_vbe(const Tensor& dev_weights, const Tensor& uvm_weights,
                            const Tensor& lxu_cache_weights, const Tensor& weights_placements,
                            const Tensor& weights_offsets, const Tensor& D_offsets,
                            c10::SymInt total_D, c10::SymInt max_D, const Tensor& indices,
                            const Tensor& offsets, int64_t pooling_mode,
                            const Tensor& indice_weights, const Tensor& lxu_cache_locations,
                            const Tensor& uvm_cache_stats, int64_t output_dtype,
                            const Tensor& vbe_row_output_offsets, const Tensor& vbe_b_t_map,
                            c10::SymInt vbe_output_size, int64_t info_B_num_bits,
                            int64_t info_B_mask, bool is_experimental) {
  check_no_cache(lxu_cache_weights);
  (void)lxu_cache_locations;
  (void)uvm_cache_stats;
  (void)info_B_mask;
  (void)is_experimental;
  return tbe_forward(dev_weights, uvm_weights, weights_placements, weights_offsets, D_offsets,
                     total_D.expect_int(), max_D.expect_int(), indices, offsets, pooling_mode,
                     indice_weights, output_dtype,
                     vbe_meta(vbe_row_output_offsets, vbe_b_t_map, vbe_output_size.expect_int(),
                              info_B_num_bits));
}

std::tuple<int64_t, int64_t> get_infos_metadata(const Tensor& unused, int64_t B, int64_t T) {
  (void)unused;
  const int32_t nb = mx_tbe_info_B_num_bits(static_cast<int32_t>(T), B);
  TORCH_CHECK(nb > 0, "T=", T, " and B=", B, " do not fit a 32-bit info word");
  const int64_t mask = nb >= 32 ? 0xffffffffll : ((int64_t(1) << nb) - 1);
  return {nb, mask};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> transpose_embedding_input(
    const Tensor& hash_size_cumsum, int64_t total_hash_size_bits, const Tensor& indices,
    const Tensor& offsets, bool nobag, const std::optional<Tensor>& vbe_b_t_map,
    int64_t info_B_num_bits, int64_t info_B_mask, int64_t total_unique_indices) {
  (void)info_B_mask;
  (void)total_unique_indices;
  const bool vbe = vbe_b_t_map.has_value() && vbe_b_t_map->defined();
  TORCH_CHECK(!(nobag && vbe), "nobag transpose takes no vbe_b_t_map");
  check_gpu(indices, "indices");
  c10::OptionalDeviceGuard guard(indices.device());
  check_arg(hash_size_cumsum, indices, "hash_size_cumsum", true);
  check_arg(offsets, indices, "offsets", false);
  TORCH_CHECK(hash_size_cumsum.scalar_type() == at::kLong, "hash_size_cumsum must be int64");
  const int32_t ib = index_bytes_of(indices, "indices");
  TORCH_CHECK(index_bytes_of(offsets, "offsets") == ib, "indices and offsets must share a dtype");
  ensure_mailbox(indices.device().index(), stream_of(indices));
  const int64_t T = hash_size_cumsum.numel() - 1;
  TORCH_CHECK(T >= 1 && (vbe || (offsets.numel() - 1) % T == 0),
              "offsets must have T*B+1 entries");
  const int64_t B = vbe ? 0 : (offsets.numel() - 1) / T;
  const int64_t N = indices.numel();
  auto o64 = indices.options().dtype(at::kLong);
  auto o32 = indices.options().dtype(at::kInt);
  const Tensor idx = indices.contiguous(), off = offsets.contiguous();
  if (nobag) {  // sequence lookups: int64 infos l * T + t
    Tensor linear = at::empty({N}, o64), sorted = at::empty({N}, o64);
    Tensor infos = at::empty({N}, o64), run = at::empty({N}, o64);
    Tensor lengths = at::empty({N}, o32), num_runs = at::zeros({1}, o32);
    Tensor cum = at::empty({N + 1}, o32);
    const size_t nb_bytes = mx_tbe_transpose_nobag_workspace_bytes(
        N, static_cast<int32_t>(T), static_cast<int32_t>(total_hash_size_bits));
    Tensor nws = at::empty({static_cast<int64_t>(nb_bytes)}, indices.options().dtype(at::kByte));
    MX_CALL(mx_tbe_transpose_embedding_input_nobag(
        hash_size_cumsum.data_ptr<int64_t>(), static_cast<int32_t>(T), B,
        static_cast<int32_t>(total_hash_size_bits), idx.data_ptr(), off.data_ptr(), ib, N,
        linear.data_ptr<int64_t>(), sorted.data_ptr<int64_t>(), infos.data_ptr<int64_t>(),
        run.data_ptr<int64_t>(), lengths.data_ptr<int32_t>(), num_runs.data_ptr<int32_t>(),
        cum.data_ptr<int32_t>(), nws.data_ptr(), nb_bytes, stream_of(indices)));
    return {linear, sorted, infos, run, lengths, num_runs, cum};
  }
  Tensor linear = at::empty({N}, o64), sorted = at::empty({N}, o64);
  Tensor infos = at::empty({N}, o32), run = at::empty({N}, o64);
  // Every entry of lengths and cum is written (past num_runs: 0 and N; all 0
  // when a look-back of the call gave up).
  Tensor lengths = at::empty({N}, o32), num_runs = at::zeros({1}, o32);
  Tensor cum = at::empty({N + 1}, o32);
  const size_t ws_bytes = mx_tbe_transpose_workspace_bytes(N, total_hash_size_bits);
  Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, indices.options().dtype(at::kByte));
  if (vbe) {
    const int64_t total_B = offsets.numel() - 1;
    check_gpu(*vbe_b_t_map, "vbe_b_t_map");
    TORCH_CHECK(vbe_b_t_map->scalar_type() == at::kInt && vbe_b_t_map->numel() == total_B,
                "vbe_b_t_map must be int32 with one entry per bag");
    const Tensor btm = vbe_b_t_map->contiguous();
    MX_CALL(mx_tbe_transpose_embedding_input_vbe(
        hash_size_cumsum.data_ptr<int64_t>(), static_cast<int32_t>(T), total_B,
        btm.data_ptr<int32_t>(), static_cast<int32_t>(total_hash_size_bits),
        static_cast<int32_t>(info_B_num_bits), idx.data_ptr(), off.data_ptr(), ib, N,
        linear.data_ptr<int64_t>(), sorted.data_ptr<int64_t>(), infos.data_ptr<int32_t>(),
        run.data_ptr<int64_t>(), lengths.data_ptr<int32_t>(), num_runs.data_ptr<int32_t>(),
        cum.data_ptr<int32_t>(), ws.data_ptr(), ws_bytes, stream_of(indices)));
    return {linear, sorted, infos, run, lengths, num_runs, cum};
  }
  MX_CALL(mx_tbe_transpose_embedding_input(
      hash_size_cumsum.data_ptr<int64_t>(), static_cast<int32_t>(T), B,
      static_cast<int32_t>(total_hash_size_bits), static_cast<int32_t>(info_B_num_bits),
      idx.data_ptr(), off.data_ptr(), ib, N, linear.data_ptr<int64_t>(),
      sorted.data_ptr<int64_t>(), infos.data_ptr<int32_t>(), run.data_ptr<int64_t>(),
      lengths.data_ptr<int32_t>(), num_runs.data_ptr<int32_t>(), cum.data_ptr<int32_t>(),
      ws.data_ptr(), ws_bytes, stream_of(indices)));
  return {linear, sorted, infos, run, lengths, num_runs, cum};
}

// Shared body of the unweighted and weighted backward ops; `indice_weights`
// undefined = unweighted.
Tensor backward_rowwise_adagrad_impl(
    const Tensor& grad_output, const Tensor& dev_weights, const Tensor& uvm_weights,
    const Tensor& lxu_cache_weights, const Tensor& weights_placements,
    const Tensor& weights_offsets, const Tensor& D_offsets, c10::SymInt max_D_sym,
    const Tensor& hash_size_cumsum, int64_t total_hash_size_bits, const Tensor& indices,
    const Tensor& offsets, int64_t pooling_mode, const Tensor& indice_weights,
    const Tensor& lxu_cache_locations, int64_t BT_block_size,
    int64_t max_segment_length_per_warp, bool stochastic_rounding,
    const Tensor& momentum1_dev, const Tensor& momentum1_uvm, const Tensor& momentum1_placements,
    const Tensor& momentum1_offsets, double eps, double learning_rate, double weight_decay,
    int64_t weight_decay_mode, double max_norm, const VbeMeta& vbe = VbeMeta()) {
  check_no_cache(lxu_cache_weights);
  (void)weights_placements;
  (void)lxu_cache_locations;
  (void)BT_block_size;
  (void)max_segment_length_per_warp;
  (void)momentum1_placements;
  check_gpu(dev_weights, "dev_weights");
  c10::OptionalDeviceGuard guard(dev_weights.device());
  for (auto* t : {&grad_output, &indices, &offsets})
    check_arg(*t, dev_weights, "TBE backward argument", false);
  for (auto* t : {&weights_offsets, &D_offsets, &hash_size_cumsum, &momentum1_dev,
                  &momentum1_offsets})
    check_arg(*t, dev_weights, "TBE backward argument", true);
  TORCH_CHECK(uvm_weights.numel() == 0 && momentum1_uvm.numel() == 0,
              "UVM storage is not supported (DEVICE placement only)");
  TORCH_CHECK(max_norm == 0.0, "max_norm is not supported");
  const int32_t wty = weights_ty_of(dev_weights);
  TORCH_CHECK(momentum1_dev.scalar_type() == at::kFloat && momentum1_dev.is_contiguous(),
              "momentum1_dev must be contiguous fp32");
  TORCH_CHECK(grad_output.scalar_type() == at::kFloat, "grad_output must be fp32");
  TORCH_CHECK(momentum1_offsets.scalar_type() == at::kLong, "momentum1_offsets must be int64");
  TORCH_CHECK(hash_size_cumsum.scalar_type() == at::kLong, "hash_size_cumsum must be int64");
  const int32_t ib = index_bytes_of(indices, "indices");
  TORCH_CHECK(index_bytes_of(offsets, "offsets") == ib, "indices and offsets must share a dtype");
  ensure_mailbox(dev_weights.device().index(), stream_of(dev_weights));
  const int64_t T = D_offsets.numel() - 1;
  TORCH_CHECK(T >= 1 && (vbe.on() || (offsets.numel() - 1) % T == 0),
              "offsets must have T*B+1 entries");
  const int64_t B = vbe.on() ? 0 : (offsets.numel() - 1) / T;
  const Tensor g = grad_output.contiguous();
  if (vbe.on()) {
    TORCH_CHECK(g.numel() == vbe.output_size, "grad_output must hold the flat VBE output");
  } else {
    TORCH_CHECK(g.dim() == 2 && g.size(0) == B, "grad_output must be [B, total_D]");
  }
  const int64_t max_D = max_D_sym.expect_int();
  const int64_t N = indices.numel();
  const size_t ws_bytes =
      mx_tbe_backward_workspace_bytes(N, static_cast<int32_t>(total_hash_size_bits),
                                      static_cast<int32_t>(max_D));
  Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, dev_weights.options().dtype(at::kByte));
  const Tensor idx = indices.contiguous(), off = offsets.contiguous();
  Tensor iwc;
  if (indice_weights.defined()) {
    check_gpu(indice_weights, "indice_weights");
    TORCH_CHECK(indice_weights.scalar_type() == at::kFloat, "indice_weights must be fp32");
    TORCH_CHECK(indice_weights.numel() == N, "indice_weights has ", indice_weights.numel(),
                " entries but there are ", N, " indices");
    iwc = indice_weights.contiguous();
  }
  // fp16 weights: the update rounds stochastically when asked (fp32: no rounding step).
  const bool sr = wty == MX_SPARSE_FP16 && stochastic_rounding;
  const mx_rng_state rng = sr ? next_rounding_state(dev_weights) : mx_rng_state{};
  if (vbe.on()) {
    const int64_t total_B = offsets.numel() - 1;
    check_vbe(vbe, total_B);
    check_gpu(vbe.B_offsets, "B_offsets");
    TORCH_CHECK(vbe.B_offsets.scalar_type() == at::kInt && vbe.B_offsets.numel() == T + 1,
                "B_offsets must be int32 [T+1]");
    const Tensor bo = vbe.B_offsets.contiguous();
    MX_CALL(mx_tbe_backward_rowwise_adagrad_vbe(
        dev_weights.data_ptr(), wty, weights_offsets.data_ptr<int64_t>(),
        D_offsets.data_ptr<int32_t>(), static_cast<int32_t>(T), vbe.max_B,
        static_cast<int32_t>(max_D), hash_size_cumsum.data_ptr<int64_t>(),
        static_cast<int32_t>(total_hash_size_bits), idx.data_ptr(), off.data_ptr(), ib, N,
        static_cast<int32_t>(pooling_mode), iwc.defined() ? iwc.data_ptr<float>() : nullptr,
        g.data_ptr<float>(), total_B, bo.data_ptr<int32_t>(), vbe.row_out.data_ptr<int64_t>(),
        vbe.b_t_map.data_ptr<int32_t>(), static_cast<int32_t>(vbe.info_B_num_bits),
        momentum1_dev.data_ptr<float>(), momentum1_offsets.data_ptr<int64_t>(),
        static_cast<float>(learning_rate), static_cast<float>(eps),
        static_cast<float>(weight_decay), static_cast<int32_t>(weight_decay_mode), sr ? 1 : 0,
        &rng, ws.data_ptr(), ws_bytes, stream_of(dev_weights)));
    return at::empty({0}, dev_weights.options());
  }
  MX_CALL(mx_tbe_backward_rowwise_adagrad(
      dev_weights.data_ptr(), wty, weights_offsets.data_ptr<int64_t>(),
      D_offsets.data_ptr<int32_t>(), static_cast<int32_t>(T), B, static_cast<int32_t>(max_D),
      hash_size_cumsum.data_ptr<int64_t>(), static_cast<int32_t>(total_hash_size_bits),
      idx.data_ptr(), off.data_ptr(), ib, N, static_cast<int32_t>(pooling_mode),
      iwc.defined() ? iwc.data_ptr<float>() : nullptr, g.data_ptr<float>(), g.size(1),
      momentum1_dev.data_ptr<float>(),
      momentum1_offsets.data_ptr<int64_t>(), static_cast<float>(learning_rate),
      static_cast<float>(eps), static_cast<float>(weight_decay),
      static_cast<int32_t>(weight_decay_mode), sr ? 1 : 0, &rng, ws.data_ptr(), ws_bytes,
      stream_of(dev_weights)));
  return at::empty({0}, dev_weights.options());
}

// PoolingMode NONE: grad_output [N, D], row l the gradient of position l.
Tensor backward_rowwise_adagrad_nobag(
    const Tensor& grad_output, const Tensor& dev_weights, const Tensor& uvm_weights,
    const Tensor& lxu_cache_weights, const Tensor& weights_placements,
    const Tensor& weights_offsets, c10::SymInt D_sym, const Tensor& hash_size_cumsum,
    int64_t total_hash_size_bits, const Tensor& indices, const Tensor& offsets,
    const Tensor& lxu_cache_locations, int64_t BT_block_size,
    int64_t max_segment_length_per_warp, bool stochastic_rounding,
    const Tensor& momentum1_dev, const Tensor& momentum1_uvm, const Tensor& momentum1_placements,
    const Tensor& momentum1_offsets, double eps, double learning_rate, double weight_decay,
    int64_t weight_decay_mode, double max_norm) {
  check_no_cache(lxu_cache_weights);
  (void)weights_placements;
  (void)lxu_cache_locations;
  (void)BT_block_size;
  (void)max_segment_length_per_warp;
  (void)momentum1_placements;
  check_gpu(dev_weights, "dev_weights");
  c10::OptionalDeviceGuard guard(dev_weights.device());
  for (auto* t : {&grad_output, &indices, &offsets})
    check_arg(*t, dev_weights, "TBE backward argument", false);
  for (auto* t : {&weights_offsets, &hash_size_cumsum, &momentum1_dev, &momentum1_offsets})
    check_arg(*t, dev_weights, "TBE backward argument", true);
  TORCH_CHECK(uvm_weights.numel() == 0 && momentum1_uvm.numel() == 0,
              "UVM storage is not supported (DEVICE placement only)");
  TORCH_CHECK(max_norm == 0.0, "max_norm is not supported");
  const int32_t wty = weights_ty_of(dev_weights);
  TORCH_CHECK(momentum1_dev.scalar_type() == at::kFloat && momentum1_dev.is_contiguous(),
              "momentum1_dev must be contiguous fp32");
  TORCH_CHECK(grad_output.scalar_type() == at::kFloat, "grad_output must be fp32");
  TORCH_CHECK(weights_offsets.scalar_type() == at::kLong, "weights_offsets must be int64");
  TORCH_CHECK(momentum1_offsets.scalar_type() == at::kLong, "momentum1_offsets must be int64");
  TORCH_CHECK(hash_size_cumsum.scalar_type() == at::kLong, "hash_size_cumsum must be int64");
  const int32_t ib = index_bytes_of(indices, "indices");
  TORCH_CHECK(index_bytes_of(offsets, "offsets") == ib, "indices and offsets must share a dtype");
  ensure_mailbox(dev_weights.device().index(), stream_of(dev_weights));
  const int64_t T = weights_offsets.numel();
  TORCH_CHECK(T >= 1 && hash_size_cumsum.numel() == T + 1 && momentum1_offsets.numel() == T,
              "hash_size_cumsum must have T+1 and momentum1_offsets T entries");
  TORCH_CHECK((offsets.numel() - 1) % T == 0, "offsets must have T*B+1 entries");
  const int64_t B = (offsets.numel() - 1) / T;
  const int64_t D = D_sym.expect_int();
  const int64_t N = indices.numel();
  const Tensor g = grad_output.contiguous();
  TORCH_CHECK(g.dim() == 2 && g.size(0) == N && g.size(1) == D, "grad_output must be [N, D] = [",
              N, ", ", D, "]");
  const size_t ws_bytes = mx_tbe_backward_nobag_workspace_bytes(
      N, static_cast<int32_t>(T), static_cast<int32_t>(total_hash_size_bits),
      static_cast<int32_t>(D));
  Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, dev_weights.options().dtype(at::kByte));
  const Tensor idx = indices.contiguous(), off = offsets.contiguous();
  const bool sr = wty == MX_SPARSE_FP16 && stochastic_rounding;
  const mx_rng_state rng = sr ? next_rounding_state(dev_weights) : mx_rng_state{};
  MX_CALL(mx_tbe_backward_rowwise_adagrad_nobag(
      dev_weights.data_ptr(), wty, weights_offsets.data_ptr<int64_t>(), static_cast<int32_t>(T), B,
      static_cast<int32_t>(D), hash_size_cumsum.data_ptr<int64_t>(),
      static_cast<int32_t>(total_hash_size_bits), idx.data_ptr(), off.data_ptr(), ib, N,
      g.data_ptr<float>(), momentum1_dev.data_ptr<float>(), momentum1_offsets.data_ptr<int64_t>(),
      static_cast<float>(learning_rate), static_cast<float>(eps),
      static_cast<float>(weight_decay), static_cast<int32_t>(weight_decay_mode), sr ? 1 : 0,
      &rng, ws.data_ptr(), ws_bytes, stream_of(dev_weights)));
  return at::empty({0}, dev_weights.options());
}

Tensor backward_rowwise_adagrad_exact(
    const Tensor& grad_output, const Tensor& dev_weights, const Tensor& uvm_weights,
    const Tensor& lxu_cache_weights, const Tensor& weights_placements,
    const Tensor& weights_offsets, const Tensor& D_offsets, c10::SymInt max_D,
    const Tensor& hash_size_cumsum, int64_t total_hash_size_bits, const Tensor& indices,
    const Tensor& offsets, int64_t pooling_mode, const Tensor& lxu_cache_locations,
    int64_t BT_block_size, int64_t max_segment_length_per_warp, bool stochastic_rounding,
    const Tensor& momentum1_dev, const Tensor& momentum1_uvm, const Tensor& momentum1_placements,
    const Tensor& momentum1_offsets, double eps, double learning_rate, double weight_decay,
    int64_t weight_decay_mode, double max_norm) {
  return backward_rowwise_adagrad_impl(
      grad_output, dev_weights, uvm_weights, lxu_cache_weights, weights_placements,
      weights_offsets, D_offsets, std::move(max_D), hash_size_cumsum, total_hash_size_bits,
      indices, offsets, pooling_mode, Tensor(), lxu_cache_locations, BT_block_size,
      max_segment_length_per_warp, stochastic_rounding, momentum1_dev, momentum1_uvm,
      momentum1_placements, momentum1_offsets, eps, learning_rate, weight_decay,
      weight_decay_mode, max_norm);
}

Tensor backward_rowwise_adagrad_weighted_exact(
    const Tensor& grad_output, const Tensor& dev_weights, const Tensor& uvm_weights,
    const Tensor& lxu_cache_weights, const Tensor& weights_placements,
    const Tensor& weights_offsets, const Tensor& D_offsets, c10::SymInt max_D,
    const Tensor& hash_size_cumsum, int64_t total_hash_size_bits, const Tensor& indices,
    const Tensor& offsets, int64_t pooling_mode, const Tensor& indice_weights,
    const Tensor& lxu_cache_locations, int64_t BT_block_size,
    int64_t max_segment_length_per_warp, bool stochastic_rounding,
    const Tensor& momentum1_dev, const Tensor& momentum1_uvm, const Tensor& momentum1_placements,
    const Tensor& momentum1_offsets, double eps, double learning_rate, double weight_decay,
    int64_t weight_decay_mode, double max_norm) {
  TORCH_CHECK(indice_weights.defined(), "the weighted backward needs indice_weights");
  return backward_rowwise_adagrad_impl(
      grad_output, dev_weights, uvm_weights, lxu_cache_weights, weights_placements,
      weights_offsets, D_offsets, std::move(max_D), hash_size_cumsum, total_hash_size_bits,
      indices, offsets, pooling_mode, indice_weights, lxu_cache_locations, BT_block_size,
      max_segment_length_per_warp, stochastic_rounding, momentum1_dev, momentum1_uvm,
      momentum1_placements, momentum1_offsets, eps, learning_rate, weight_decay,
      weight_decay_mode, max_norm);
}

Tensor backward_rowwise_adagrad_vbe_common(
    const Tensor& grad_output, const Tensor& dev_weights, const Tensor& uvm_weights,
    const Tensor& lxu_cache_weights, const Tensor& weights_placements,
    const Tensor& weights_offsets, const Tensor& D_offsets, c10::SymInt max_D,
    const Tensor& hash_size_cumsum, int64_t total_hash_size_bits, const Tensor& indices,
    const Tensor& offsets, int64_t pooling_mode, const Tensor& indice_weights,
    const Tensor& lxu_cache_locations, int64_t BT_block_size,
    int64_t max_segment_length_per_warp, bool stochastic_rounding, int64_t info_B_num_bits,
    const Tensor& B_offsets, const Tensor& vbe_row_output_offsets, const Tensor& vbe_b_t_map,
    const Tensor& momentum1_dev, const Tensor& momentum1_uvm, const Tensor& momentum1_placements,
    const Tensor& momentum1_offsets, double eps, double learning_rate, double weight_decay,
    int64_t weight_decay_mode, double max_norm) {
  // b < 2^info_B_num_bits by the encoding: the widest batch the info words allow.
  const int64_t max_B = info_B_num_bits >= 32 ? (int64_t(1) << 32) : (int64_t(1) << info_B_num_bits);
  return backward_rowwise_adagrad_impl(
      grad_output, dev_weights, uvm_weights, lxu_cache_weights, weights_placements,
      weights_offsets, D_offsets, std::move(max_D), hash_size_cumsum, total_hash_size_bits,
      indices, offsets, pooling_mode, indice_weights, lxu_cache_locations, BT_block_size,
      max_segment_length_per_warp, stochastic_rounding, momentum1_dev, momentum1_uvm,
      momentum1_placements, momentum1_offsets, eps, learning_rate, weight_decay,
      weight_decay_mode, max_norm,
      vbe_meta(vbe_row_output_offsets, vbe_b_t_map, grad_output.numel(), info_B_num_bits,
               B_offsets, max_B));
}

Tensor backward_rowwise_adagrad_exact_vbe(
    const Tensor& grad_output, const Tensor& dev_weights, const Tensor& uvm_weights,
    const Tensor& lxu_cache_weights, const Tensor& weights_placements,
    const Tensor& weights_offsets, const Tensor& D_offsets, c10::SymInt max_D,
    const Tensor& hash_size_cumsum, int64_t total_hash_size_bits, const Tensor& indices,
    const Tensor& offsets, int64_t pooling_mode, const Tensor& lxu_cache_locations,
    int64_t BT_block_size, int64_t max_segment_length_per_warp, bool stochastic_rounding,
    int64_t info_B_num_bits, int64_t info_B_mask, const Tensor& B_offsets,
    const Tensor& vbe_row_output_offsets, const Tensor& vbe_b_t_map,
    const Tensor& momentum1_dev, const Tensor& momentum1_uvm, const Tensor& momentum1_placements,
    const Tensor& momentum1_offsets, double eps, double learning_rate, double weight_decay,
    int64_t weight_decay_mode, double max_norm) {
  (void)info_B_mask;
  return backward_rowwise_adagrad_vbe_common(
      grad_output, dev_weights, uvm_weights, lxu_cache_weights, weights_placements,
      weights_offsets, D_offsets, std::move(max_D), hash_size_cumsum, total_hash_size_bits,
      indices, offsets, pooling_mode, Tensor(), lxu_cache_locations, BT_block_size,
      max_segment_length_per_warp, stochastic_rounding, info_B_num_bits, B_offsets,
      vbe_row_output_offsets, vbe_b_t_map, momentum1_dev, momentum1_uvm, momentum1_placements,
      momentum1_offsets, eps, learning_rate, weight_decay, weight_decay_mode, max_norm);
}

Tensor backward_rowwise_adagrad_weighted_exact_vbe(
    const Tensor& grad_output, const Tensor& dev_weights, const Tensor& uvm_weights,
    const Tensor& lxu_cache_weights, const Tensor& weights_placements,
    const Tensor& weights_offsets, const Tensor& D_offsets, c10::SymInt max_D,
    const Tensor& hash_size_cumsum, int64_t total_hash_size_bits, const Tensor& indices,
    const Tensor& offsets, int64_t pooling_mode, const Tensor& indice_weights,
    const Tensor& lxu_cache_locations, int64_t BT_block_size,
    int64_t max_segment_length_per_warp, bool stochastic_rounding, int64_t info_B_num_bits,
    int64_t info_B_mask, const Tensor& B_offsets, const Tensor& vbe_row_output_offsets,
    const Tensor& vbe_b_t_map, const Tensor& momentum1_dev, const Tensor& momentum1_uvm,
    const Tensor& momentum1_placements, const Tensor& momentum1_offsets, double eps,
    double learning_rate, double weight_decay, int64_t weight_decay_mode, double max_norm) {
  (void)info_B_mask;
  TORCH_CHECK(indice_weights.defined(), "the weighted backward needs indice_weights");
  return backward_rowwise_adagrad_vbe_common(
      grad_output, dev_weights, uvm_weights, lxu_cache_weights, weights_placements,
      weights_offsets, D_offsets, std::move(max_D), hash_size_cumsum, total_hash_size_bits,
      indices, offsets, pooling_mode, indice_weights, lxu_cache_locations, BT_block_size,
      max_segment_length_per_warp, stochastic_rounding, info_B_num_bits, B_offsets,
      vbe_row_output_offsets, vbe_b_t_map, momentum1_dev, momentum1_uvm, momentum1_placements,
      momentum1_offsets, eps, learning_rate, weight_decay, weight_decay_mode, max_norm);
}

// Gradient of the per-sample weights of a weighted SUM/MEAN lookup (fp32 [N]):
// grad_indice_weights[l] = <grad_output[b, D_t slice], W_t[indices[l]]>, times
// 1/L under MEAN; 0 for tables whose feature_requires_grad entry is 0.
Tensor grad_indice_weights_impl(const Tensor& grad_output, const Tensor& dev_weights,
                                const Tensor& uvm_weights, const Tensor& lxu_cache_weights,
                                const Tensor& weights_placements, const Tensor& weights_offsets,
                                const Tensor& D_offsets, c10::SymInt max_D_sym,
                                const Tensor& indices, const Tensor& offsets,
                                const Tensor& lxu_cache_locations,
                                const std::optional<Tensor>& feature_requires_grad,
                                int64_t pooling_mode, const VbeMeta& vbe) {
  check_no_cache(lxu_cache_weights);
  (void)weights_placements;
  (void)lxu_cache_locations;
  check_gpu(dev_weights, "dev_weights");
  c10::OptionalDeviceGuard guard(dev_weights.device());
  for (auto* t : {&grad_output, &indices, &offsets})
    check_arg(*t, dev_weights, "grad_indice_weights argument", false);
  for (auto* t : {&weights_offsets, &D_offsets})
    check_arg(*t, dev_weights, "grad_indice_weights argument", true);
  TORCH_CHECK(uvm_weights.numel() == 0, "UVM storage is not supported (DEVICE placement only)");
  const int32_t wty = weights_ty_of(dev_weights);
  TORCH_CHECK(grad_output.scalar_type() == at::kFloat, "grad_output must be fp32");
  TORCH_CHECK(weights_offsets.scalar_type() == at::kLong, "weights_offsets must be int64");
  TORCH_CHECK(D_offsets.scalar_type() == at::kInt, "D_offsets must be int32");
  const int32_t ib = index_bytes_of(indices, "indices");
  TORCH_CHECK(index_bytes_of(offsets, "offsets") == ib, "indices and offsets must share a dtype");
  const int64_t T = D_offsets.numel() - 1;
  TORCH_CHECK(T >= 1 && (vbe.on() || (offsets.numel() - 1) % T == 0),
              "offsets must have T*B+1 entries");
  const int64_t B = vbe.on() ? 0 : (offsets.numel() - 1) / T;
  const Tensor g = grad_output.contiguous();
  if (vbe.on()) {
    TORCH_CHECK(g.numel() == vbe.output_size, "grad_output must hold the flat VBE output");
  } else {
    TORCH_CHECK(g.dim() == 2 && g.size(0) == B, "grad_output must be [B, total_D]");
  }
  Tensor frg;
  if (feature_requires_grad.has_value() && feature_requires_grad->defined() &&
      feature_requires_grad->numel() > 0) {
    check_gpu(*feature_requires_grad, "feature_requires_grad");
    TORCH_CHECK(feature_requires_grad->numel() == T, "feature_requires_grad must have T entries");
    frg = feature_requires_grad->to(at::kInt).contiguous();
  }
  const Tensor idx = indices.contiguous(), off = offsets.contiguous();
  Tensor out = at::empty({indices.numel()}, dev_weights.options().dtype(at::kFloat));
  if (indices.numel() == 0) return out;  // one entry per index: nothing to compute
  if (vbe.on()) {
    const int64_t total_B = offsets.numel() - 1;
    check_vbe(vbe, total_B);
    MX_CALL(mx_tbe_grad_indice_weights_vbe(
        g.data_ptr<float>(), dev_weights.data_ptr(), wty, weights_offsets.data_ptr<int64_t>(),
        D_offsets.data_ptr<int32_t>(), static_cast<int32_t>(T), total_B,
        static_cast<int32_t>(max_D_sym.expect_int()), idx.data_ptr(), off.data_ptr(), ib,
        static_cast<int32_t>(pooling_mode), vbe.row_out.data_ptr<int64_t>(),
        vbe.b_t_map.data_ptr<int32_t>(), static_cast<int32_t>(vbe.info_B_num_bits),
        frg.defined() ? frg.data_ptr<int32_t>() : nullptr, out.data_ptr<float>(),
        stream_of(dev_weights)));
    return out;
  }
  MX_CALL(mx_tbe_grad_indice_weights(
      g.data_ptr<float>(), g.size(1), dev_weights.data_ptr(), wty,
      weights_offsets.data_ptr<int64_t>(), D_offsets.data_ptr<int32_t>(),
      static_cast<int32_t>(T), B, static_cast<int32_t>(max_D_sym.expect_int()), idx.data_ptr(),
      off.data_ptr(), ib, static_cast<int32_t>(pooling_mode),
      frg.defined() ? frg.data_ptr<int32_t>() : nullptr, out.data_ptr<float>(),
      stream_of(dev_weights)));
  return out;
}

Tensor grad_indice_weights(const Tensor& grad_output, const Tensor& dev_weights,
                           const Tensor& uvm_weights, const Tensor& lxu_cache_weights,
                           const Tensor& weights_placements, const Tensor& weights_offsets,
                           const Tensor& D_offsets, c10::SymInt max_D, const Tensor& indices,
                           const Tensor& offsets, const Tensor& lxu_cache_locations,
                           const std::optional<Tensor>& feature_requires_grad,
                           int64_t pooling_mode) {
  return grad_indice_weights_impl(grad_output, dev_weights, uvm_weights, lxu_cache_weights,
                                  weights_placements, weights_offsets, D_offsets,
                                  std::move(max_D), indices, offsets, lxu_cache_locations,
                                  feature_requires_grad, pooling_mode, VbeMeta());
}

Tensor grad_indice_weights_vbe(const Tensor& grad_output, const Tensor& dev_weights,
                               const Tensor& uvm_weights, const Tensor& lxu_cache_weights,
                               const Tensor& weights_placements, const Tensor& weights_offsets,
                               const Tensor& D_offsets, c10::SymInt max_D, const Tensor& indices,
                               const Tensor& offsets, const Tensor& lxu_cache_locations,
                               const std::optional<Tensor>& feature_requires_grad,
                               const Tensor& vbe_row_output_offsets, const Tensor& vbe_b_t_map,
                               int64_t info_B_num_bits, int64_t info_B_mask,
                               int64_t pooling_mode) {
  (void)info_B_mask;
  return grad_indice_weights_impl(grad_output, dev_weights, uvm_weights, lxu_cache_weights,
                                  weights_placements, weights_offsets, D_offsets,
                                  std::move(max_D), indices, offsets, lxu_cache_locations,
                                  feature_requires_grad, pooling_mode,
                                  vbe_meta(vbe_row_output_offsets, vbe_b_t_map,
                                           grad_output.numel(), info_B_num_bits));
}

class LookupRowwiseAdagrad : public torch::autograd::Function<LookupRowwiseAdagrad> {
 public:
  static Tensor forward(AutogradContext* ctx, const Tensor& placeholder,
                        const Tensor& dev_weights, const Tensor& uvm_weights,
                        const Tensor& weights_placements, const Tensor& weights_offsets,
                        const Tensor& D_offsets, int64_t total_D, int64_t max_D,
                        const Tensor& hash_size_cumsum, int64_t total_hash_size_bits,
                        const Tensor& indices, const Tensor& offsets, int64_t pooling_mode,
                        const std::optional<Tensor>& indice_weights,
                        const std::optional<Tensor>& feature_requires_grad,
                        const Tensor& momentum1_dev, const Tensor& momentum1_uvm,
                        const Tensor& momentum1_placements, const Tensor& momentum1_offsets,
                        double eps, double learning_rate, double weight_decay,
                        int64_t weight_decay_mode, double max_norm, int64_t output_dtype,
                        bool stochastic_rounding, const std::optional<Tensor>& vbe_B_offsets,
                        const std::optional<Tensor>& vbe_row_out,
                        const std::optional<Tensor>& vbe_b_t_map, int64_t vbe_output_size,
                        int64_t vbe_info_B_num_bits) {
    (void)placeholder;
    // Stored as IValues: the backward updates dev_weights/momentum1 in place.
    auto& s = ctx->saved_data;
    s["dev_weights"] = dev_weights;
    s["uvm_weights"] = uvm_weights;
    s["weights_placements"] = weights_placements;
    s["weights_offsets"] = weights_offsets;
    s["D_offsets"] = D_offsets;
    s["hash_size_cumsum"] = hash_size_cumsum;
    s["indices"] = indices;
    s["offsets"] = offsets;
    // Optional (not plain Tensor) arguments: an absent one is no autograd input.
    s["indice_weights"] = indice_weights.has_value() ? *indice_weights : Tensor();
    s["feature_requires_grad"] =
        feature_requires_grad.has_value() ? *feature_requires_grad : Tensor();
    s["momentum1_dev"] = momentum1_dev;
    s["momentum1_uvm"] = momentum1_uvm;
    s["momentum1_placements"] = momentum1_placements;
    s["momentum1_offsets"] = momentum1_offsets;
    s["max_D"] = max_D;
    s["total_hash_size_bits"] = total_hash_size_bits;
    s["pooling_mode"] = pooling_mode;
    s["eps"] = eps;
    s["learning_rate"] = learning_rate;
    s["weight_decay"] = weight_decay;
    s["weight_decay_mode"] = weight_decay_mode;
    s["max_norm"] = max_norm;
    s["stochastic_rounding"] = stochastic_rounding;
    const bool vbe = vbe_b_t_map.has_value() && vbe_b_t_map->defined();
    s["vbe_B_offsets"] = vbe ? *vbe_B_offsets : Tensor();
    s["vbe_row_out"] = vbe ? *vbe_row_out : Tensor();
    s["vbe_b_t_map"] = vbe ? *vbe_b_t_map : Tensor();
    s["vbe_output_size"] = vbe_output_size;
    s["vbe_info_B_num_bits"] = vbe_info_B_num_bits;
    at::AutoDispatchBelowADInplaceOrView g;
    if (pooling_mode == MX_POOL_NONE) {  // sequence lookups: [N, max_D]
      const int64_t T = D_offsets.numel() - 1;
      TORCH_CHECK(!vbe, "PoolingMode NONE takes no VBE metadata");
      TORCH_CHECK(!indice_weights.has_value() || !indice_weights->defined(),
                  "PoolingMode NONE takes no indice_weights");
      // Every D_t <= max_D, so total_D = T * max_D makes all of them max_D.
      TORCH_CHECK(T >= 1 && total_D == T * max_D,
                  "PoolingMode NONE needs every table of one width (total_D ", total_D,
                  " != T * max_D = ", T * max_D, ")");
      return tbe_forward_nobag(dev_weights, uvm_weights, weights_offsets, max_D, indices, offsets,
                               output_dtype);
    }
    return tbe_forward(dev_weights, uvm_weights, weights_placements, weights_offsets, D_offsets,
                       total_D, max_D, indices, offsets, pooling_mode, indice_weights,
                       output_dtype, vbe ? saved_vbe(s) : VbeMeta());
  }

  // The VBE metadata saved by forward (undefined tensors: fixed batch).
  static VbeMeta saved_vbe(const ska::flat_hash_map<std::string, at::IValue>& s) {
    const Tensor btm = s.at("vbe_b_t_map").toTensor();
    if (!btm.defined()) return VbeMeta();
    const int64_t nb = s.at("vbe_info_B_num_bits").toInt();
    return vbe_meta(s.at("vbe_row_out").toTensor(), btm, s.at("vbe_output_size").toInt(), nb,
                    s.at("vbe_B_offsets").toTensor(),
                    nb >= 32 ? (int64_t(1) << 32) : (int64_t(1) << nb));
  }

  // indice_weights is argument 13 of forward() (after ctx) and, when present,
  // the 10th Tensor argument, i.e. autograd edge 9; backward returns one slot
  // per argument.
  static constexpr size_t kIndiceWeightsArg = 13;
  static constexpr size_t kIndiceWeightsEdge = 9;
  static constexpr size_t kNumInputs = 31;

  static variable_list backward(AutogradContext* ctx, variable_list grads) {
    auto& s = ctx->saved_data;
    Tensor grad = grads[0];
    TORCH_CHECK(grad.scalar_type() == at::kFloat,
                "the rowwise-Adagrad backward needs an fp32 gradient (output_dtype FP32)");
    const Tensor empty;
    const Tensor g = grad.contiguous();
    const Tensor iw = s["indice_weights"].toTensor();
    variable_list out(kNumInputs);
    if (s["pooling_mode"].toInt() == MX_POOL_NONE) {
      backward_rowwise_adagrad_nobag(
          g, s["dev_weights"].toTensor(), s["uvm_weights"].toTensor(), empty,
          s["weights_placements"].toTensor(), s["weights_offsets"].toTensor(),
          c10::SymInt(s["max_D"].toInt()), s["hash_size_cumsum"].toTensor(),
          s["total_hash_size_bits"].toInt(), s["indices"].toTensor(), s["offsets"].toTensor(),
          empty, 0, 0, s["stochastic_rounding"].toBool(), s["momentum1_dev"].toTensor(),
          s["momentum1_uvm"].toTensor(), s["momentum1_placements"].toTensor(),
          s["momentum1_offsets"].toTensor(), s["eps"].toDouble(), s["learning_rate"].toDouble(),
          s["weight_decay"].toDouble(), s["weight_decay_mode"].toInt(), s["max_norm"].toDouble());
      return out;
    }
    // The weight gradient reads the rows before the fused update below
    // overwrites them (same stream, so ordered).
    if (iw.defined() && ctx->needs_input_grad(kIndiceWeightsEdge)) {
      const Tensor frg = s["feature_requires_grad"].toTensor();
      out[kIndiceWeightsArg] = grad_indice_weights_impl(
          g, s["dev_weights"].toTensor(), s["uvm_weights"].toTensor(), empty,
          s["weights_placements"].toTensor(), s["weights_offsets"].toTensor(),
          s["D_offsets"].toTensor(), c10::SymInt(s["max_D"].toInt()), s["indices"].toTensor(),
          s["offsets"].toTensor(), empty,
          frg.defined() ? std::optional<Tensor>(frg) : std::nullopt, s["pooling_mode"].toInt(),
          saved_vbe(s));
    }
    backward_rowwise_adagrad_impl(
        g, s["dev_weights"].toTensor(), s["uvm_weights"].toTensor(), empty,
        s["weights_placements"].toTensor(), s["weights_offsets"].toTensor(),
        s["D_offsets"].toTensor(), c10::SymInt(s["max_D"].toInt()),
        s["hash_size_cumsum"].toTensor(), s["total_hash_size_bits"].toInt(),
        s["indices"].toTensor(), s["offsets"].toTensor(), s["pooling_mode"].toInt(), iw, empty,
        0, 0, s["stochastic_rounding"].toBool(), s["momentum1_dev"].toTensor(),
        s["momentum1_uvm"].toTensor(),
        s["momentum1_placements"].toTensor(), s["momentum1_offsets"].toTensor(),
        s["eps"].toDouble(), s["learning_rate"].toDouble(), s["weight_decay"].toDouble(),
        s["weight_decay_mode"].toInt(), s["max_norm"].toDouble(), saved_vbe(s));
    return out;
  }
};

Tensor lookup_rowwise_adagrad(
    const Tensor& placeholder_autograd_tensor, const Tensor& dev_weights,
    const Tensor& uvm_weights, const Tensor& lxu_cache_weights, const Tensor& weights_placements,
    const Tensor& weights_offsets, const Tensor& D_offsets, c10::SymInt total_D,
    c10::SymInt max_D, const Tensor& hash_size_cumsum, int64_t total_hash_size_bits,
    const Tensor& indices, const Tensor& offsets, int64_t pooling_mode,
    const std::optional<Tensor>& indice_weights, const std::optional<Tensor>& feature_requires_grad,
    const Tensor& lxu_cache_locations, bool gradient_clipping, double max_gradient,
    bool stochastic_rounding, const Tensor& momentum1_dev, const Tensor& momentum1_uvm,
    const Tensor& momentum1_placements, const Tensor& momentum1_offsets, double eps,
    double learning_rate, double weight_decay, int64_t weight_decay_mode, double max_norm,
    int64_t output_dtype, const std::optional<Tensor>& B_offsets,
    const std::optional<Tensor>& vbe_output_offsets_feature_rank,
    const std::optional<Tensor>& vbe_B_offsets_rank_per_feature, c10::SymInt max_B,
    c10::SymInt max_B_feature_rank, c10::SymInt vbe_output_size) {
  check_no_cache(lxu_cache_weights);
  (void)lxu_cache_locations;
  TORCH_CHECK(!gradient_clipping || max_gradient <= 0.0, "gradient clipping is not supported");
  // Variable batch per feature: the per-bag metadata is built once here.
  std::optional<Tensor> vbe_row_out, vbe_b_t_map;
  int64_t vbe_size = 0, vbe_nb = 0;
  if (B_offsets.has_value() && B_offsets->defined()) {
    TORCH_CHECK(vbe_output_offsets_feature_rank.has_value() &&
                    vbe_B_offsets_rank_per_feature.has_value(),
                "VBE needs vbe_output_offsets_feature_rank and vbe_B_offsets_rank_per_feature");
    const int64_t T = D_offsets.numel() - 1;
    const int64_t mB = max_B.expect_int();
    vbe_size = vbe_output_size.expect_int();
    TORCH_CHECK(mB >= 1 && vbe_size >= 0, "VBE needs max_B >= 1 and vbe_output_size >= 0");
    vbe_nb = mx_tbe_info_B_num_bits(static_cast<int32_t>(T), mB);
    TORCH_CHECK(vbe_nb > 0, "T=", T, " and max_B=", mB, " do not fit a 32-bit info word");
    auto meta = generate_vbe_metadata(*B_offsets, *vbe_B_offsets_rank_per_feature,
                                      *vbe_output_offsets_feature_rank, D_offsets, -1, false,
                                      max_B_feature_rank, vbe_nb,
                                      c10::SymInt(offsets.numel() - 1));
    vbe_row_out = std::get<0>(meta);
    vbe_b_t_map = std::get<1>(meta);
  }
  return LookupRowwiseAdagrad::apply(
      placeholder_autograd_tensor, dev_weights, uvm_weights, weights_placements, weights_offsets,
      D_offsets, total_D.expect_int(), max_D.expect_int(), hash_size_cumsum, total_hash_size_bits,
      indices, offsets, pooling_mode, indice_weights, feature_requires_grad, momentum1_dev,
      momentum1_uvm, momentum1_placements,
      momentum1_offsets, eps, learning_rate, weight_decay, weight_decay_mode, max_norm,
      output_dtype, stochastic_rounding, B_offsets, vbe_row_out, vbe_b_t_map, vbe_size, vbe_nb);
}

// ---------------------------------------------------------------------------
// bounds_check_indices
// ---------------------------------------------------------------------------

void bounds_check_indices(const Tensor& rows_per_table, const Tensor& indices,
                          const Tensor& offsets, int64_t bounds_check_mode, const Tensor& warning,
                          const std::optional<Tensor>& weights,
                          const std::optional<Tensor>& B_offsets, c10::SymInt max_B,
                          const std::optional<Tensor>& b_t_map, int64_t info_B_num_bits,
                          int64_t info_B_mask, int64_t bounds_check_version) {
  (void)max_B;
  (void)b_t_map;  // the table of a bag comes from B_offsets
  (void)info_B_num_bits;
  (void)info_B_mask;
  (void)bounds_check_version;
  check_gpu(indices, "indices");
  c10::OptionalDeviceGuard guard(indices.device());
  check_arg(offsets, indices, "offsets", false);
  check_arg(rows_per_table, indices, "rows_per_table", true);
  check_arg(warning, indices, "warning", true);
  TORCH_CHECK(bounds_check_mode >= MX_BOUNDS_FATAL && bounds_check_mode <= MX_BOUNDS_NONE,
              "bounds_check_mode must be FATAL(0), WARNING(1), IGNORE(2) or NONE(3)");
  TORCH_CHECK(rows_per_table.scalar_type() == at::kLong, "rows_per_table must be int64");
  TORCH_CHECK(warning.scalar_type() == at::kLong && warning.numel() >= 1 &&
                  warning.is_contiguous(),
              "warning must be a contiguous int64 tensor");
  TORCH_CHECK(indices.is_contiguous() && offsets.is_contiguous(),
              "indices and offsets are repaired in place and must be contiguous");
  const int32_t ib = index_bytes_of(indices, "indices");
  TORCH_CHECK(index_bytes_of(offsets, "offsets") == ib, "indices and offsets must share a dtype");
  const int64_t T = rows_per_table.numel();
  // Variable batch per feature: bags B_offsets[t] .. B_offsets[t+1]-1 are table t's.
  const bool vbe = B_offsets.has_value() && B_offsets->defined();
  Tensor bo;
  if (vbe) {
    check_gpu(*B_offsets, "B_offsets");
    TORCH_CHECK(B_offsets->scalar_type() == at::kInt && B_offsets->numel() == T + 1,
                "B_offsets must be int32 [T+1]");
    bo = B_offsets->contiguous();
  }
  TORCH_CHECK(T >= 1 && (vbe || (offsets.numel() - 1) % T == 0),
              "offsets must have T*B+1 entries");
  const int64_t B = vbe ? 0 : (offsets.numel() - 1) / T;
  const int64_t total_B = offsets.numel() - 1;
  if (weights.has_value() && weights->defined())
    TORCH_CHECK(weights->numel() == indices.numel(), "per-sample weights have ",
                weights->numel(), " entries but there are ", indices.numel(), " indices");
  if (bounds_check_mode == MX_BOUNDS_NONE) return;
  const Tensor rows = rows_per_table.contiguous();
  const size_t ws_bytes = vbe ? mx_bounds_check_workspace_bytes_vbe(total_B)
                              : mx_bounds_check_workspace_bytes(static_cast<int32_t>(T), B);
  Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, indices.options().dtype(at::kByte));
  const bool fatal = bounds_check_mode == MX_BOUNDS_FATAL;
  Tensor count = fatal ? at::zeros({1}, warning.options()) : warning;
  if (vbe)
    MX_CALL(mx_bounds_check_indices_vbe(rows.data_ptr<int64_t>(), static_cast<int32_t>(T),
                                        total_B, bo.data_ptr<int32_t>(), indices.data_ptr(),
                                        offsets.data_ptr(), ib, indices.numel(),
                                        static_cast<int32_t>(bounds_check_mode),
                                        count.data_ptr<int64_t>(), ws.data_ptr(), ws_bytes,
                                        stream_of(indices)));
  else
    MX_CALL(mx_bounds_check_indices(rows.data_ptr<int64_t>(), static_cast<int32_t>(T), B,
                                    indices.data_ptr(), offsets.data_ptr(), ib, indices.numel(),
                                    static_cast<int32_t>(bounds_check_mode),
                                    count.data_ptr<int64_t>(), ws.data_ptr(), ws_bytes,
                                    stream_of(indices)));
  if (fatal) {
    const int64_t n = count.item<int64_t>();  // FATAL synchronises to report
    TORCH_CHECK(n == 0, "bounds_check_indices: ", n,
                " out-of-range indices/offsets (BoundsCheckMode.FATAL)");
  }
}

// ---------------------------------------------------------------------------
// Rowwise quantization codecs
// ---------------------------------------------------------------------------

Tensor rows_2d(const Tensor& t, const char* name) {
  check_gpu(t, name);
  TORCH_CHECK(t.dim() >= 1, name, " must have at least one dimension");
  return t.contiguous().view({-1, t.size(-1)});
}

std::vector<int64_t> with_last(const Tensor& t, int64_t last) {
  std::vector<int64_t> shape(t.sizes().begin(), t.sizes().end());
  shape.back() = last;
  return shape;
}

Tensor quantize_8bit(const Tensor& input) {
  const Tensor x = rows_2d(input, "input");
  c10::OptionalDeviceGuard guard(x.device());
  const int32_t dt = mx_dtype_of(x.scalar_type());
  TORCH_CHECK(dt == MX_DTYPE_F32 || dt == MX_DTYPE_F16, "input must be float32 or float16");
  const int64_t D = x.size(1);
  Tensor out = at::empty(with_last(input, D + 8), x.options().dtype(at::kByte));
  MX_CALL(mx_quantize_fused8bit_rowwise(x.data_ptr(), dt, x.size(0), D, out.data_ptr<uint8_t>(),
                                        stream_of(x)));
  return out;
}

Tensor dequantize_8bit(const Tensor& input, at::ScalarType st) {
  const Tensor q = rows_2d(input, "input");
  c10::OptionalDeviceGuard guard(q.device());
  TORCH_CHECK(q.scalar_type() == at::kByte, "input must be uint8");
  const int64_t D = q.size(1) - 8;
  TORCH_CHECK(D >= 0, "rows must hold at least the 8 bytes of scale and bias");
  Tensor out = at::empty(with_last(input, D), q.options().dtype(st));
  MX_CALL(mx_dequantize_fused8bit_rowwise(q.data_ptr<uint8_t>(), q.size(0), D, out.data_ptr(),
                                          mx_dtype_of(st), stream_of(q)));
  return out;
}

Tensor quantize_nbit(const Tensor& input, int64_t bit_rate) {
  const Tensor x = rows_2d(input, "input");
  c10::OptionalDeviceGuard guard(x.device());
  const int32_t dt = mx_dtype_of(x.scalar_type());
  TORCH_CHECK(dt == MX_DTYPE_F32 || dt == MX_DTYPE_F16, "input must be float32 or float16");
  TORCH_CHECK(bit_rate == 2 || bit_rate == 4 || bit_rate == 8, "bit_rate must be 2, 4 or 8");
  const int64_t D = x.size(1);
  const int64_t per = 8 / bit_rate;
  const int64_t nbytes = (D + per - 1) / per;
  Tensor out = at::empty(with_last(input, nbytes + 4), x.options().dtype(at::kByte));
  MX_CALL(mx_quantize_fused_nbit_rowwise(x.data_ptr(), dt, x.size(0), D,
                                         static_cast<int32_t>(bit_rate), out.data_ptr<uint8_t>(),
                                         stream_of(x)));
  return out;
}

Tensor dequantize_nbit(const Tensor& input, int64_t bit_rate, at::ScalarType st) {
  const Tensor q = rows_2d(input, "input");
  c10::OptionalDeviceGuard guard(q.device());
  TORCH_CHECK(q.scalar_type() == at::kByte, "input must be uint8");
  TORCH_CHECK(bit_rate == 2 || bit_rate == 4 || bit_rate == 8, "bit_rate must be 2, 4 or 8");
  const int64_t D = (q.size(1) - 4) * (8 / bit_rate);
  TORCH_CHECK(D >= 0, "rows must hold at least the 4 bytes of scale and bias");
  Tensor out = at::empty(with_last(input, D), q.options().dtype(st));
  MX_CALL(mx_dequantize_fused_nbit_rowwise(q.data_ptr<uint8_t>(), q.size(0), D,
                                           static_cast<int32_t>(bit_rate), out.data_ptr(),
                                           mx_dtype_of(st), stream_of(q)));
  return out;
}

Tensor float_to_hfp8(const Tensor& input, int64_t ebits, int64_t exponent_bias,
                     double max_pos) {
  check_gpu(input, "input");
  TORCH_CHECK(input.scalar_type() == at::kFloat, "input must be float32");
  c10::OptionalDeviceGuard guard(input.device());
  const Tensor x = input.contiguous();
  Tensor out = at::empty(x.sizes(), x.options().dtype(at::kByte));
  MX_CALL(mx_float_to_hfp8(x.data_ptr<float>(), x.numel(), static_cast<int32_t>(ebits),
                           static_cast<int32_t>(exponent_bias), static_cast<float>(max_pos),
                           out.data_ptr<uint8_t>(), stream_of(x)));
  return out;
}

Tensor hfp8_to_float(const Tensor& input, int64_t ebits, int64_t exponent_bias) {
  check_gpu(input, "input");
  TORCH_CHECK(input.scalar_type() == at::kByte, "input must be uint8");
  c10::OptionalDeviceGuard guard(input.device());
  const Tensor q = input.contiguous();
  Tensor out = at::empty(q.sizes(), q.options().dtype(at::kFloat));
  MX_CALL(mx_hfp8_to_float(q.data_ptr<uint8_t>(), q.numel(), static_cast<int32_t>(ebits),
                           static_cast<int32_t>(exponent_bias), out.data_ptr<float>(),
                           stream_of(q)));
  return out;
}

Tensor float_to_8bit(const Tensor& t) {
  TORCH_CHECK(t.scalar_type() == at::kFloat, "input must be float32");
  return quantize_8bit(t);
}
Tensor half_to_8bit(const Tensor& t) {
  TORCH_CHECK(t.scalar_type() == at::kHalf, "input must be float16");
  return quantize_8bit(t);
}
Tensor float_or_half_to_8bit(const Tensor& t) { return quantize_8bit(t); }
Tensor fused8bit_to_float(const Tensor& t) { return dequantize_8bit(t, at::kFloat); }
Tensor fused8bit_to_half(const Tensor& t) { return dequantize_8bit(t, at::kHalf); }
Tensor float_to_nbit(const Tensor& t, int64_t bit_rate) {
  TORCH_CHECK(t.scalar_type() == at::kFloat, "input must be float32");
  return quantize_nbit(t, bit_rate);
}
Tensor half_to_nbit(const Tensor& t, int64_t bit_rate) {
  TORCH_CHECK(t.scalar_type() == at::kHalf, "input must be float16");
  return quantize_nbit(t, bit_rate);
}
Tensor float_or_half_to_nbit(const Tensor& t, int64_t bit_rate) { return quantize_nbit(t, bit_rate); }
Tensor nbit_to_float(const Tensor& t, int64_t bit_rate) {
  return dequantize_nbit(t, bit_rate, at::kFloat);
}
Tensor nbit_to_half(const Tensor& t, int64_t bit_rate) {
  return dequantize_nbit(t, bit_rate, at::kHalf);
}

// ---------------------------------------------------------------------------
// nbit inference
// ---------------------------------------------------------------------------

Tensor int_nbit_lookup(const Tensor& dev_weights, const Tensor& uvm_weights,
                       const Tensor& weights_placements, const Tensor& weights_offsets,
                       const Tensor& weights_tys, const Tensor& D_offsets, c10::SymInt total_D_sym,
                       int64_t max_int2_D, int64_t max_int4_D, int64_t max_int8_D,
                       int64_t max_float16_D, int64_t max_float32_D, const Tensor& indices,
                       const Tensor& offsets, int64_t pooling_mode,
                       const std::optional<Tensor>& indice_weights, int64_t output_dtype,
                       const std::optional<Tensor>& lxu_cache_weights,
                       const std::optional<Tensor>& lxu_cache_locations,
                       std::optional<int64_t> row_alignment, std::optional<int64_t> max_float8_D,
                       std::optional<int64_t> fp8_exponent_bits,
                       std::optional<int64_t> fp8_exponent_bias) {
  (void)weights_placements;
  check_no_cache(lxu_cache_weights.value_or(Tensor()));
  (void)lxu_cache_locations;
  check_gpu(dev_weights, "dev_weights");
  c10::OptionalDeviceGuard guard(dev_weights.device());
  for (auto* t : {&indices, &offsets}) check_arg(*t, dev_weights, "nbit argument", false);
  for (auto* t : {&weights_offsets, &weights_tys, &D_offsets})
    check_arg(*t, dev_weights, "nbit argument", true);
  TORCH_CHECK(uvm_weights.numel() == 0, "UVM weights are not supported (DEVICE placement only)");
  TORCH_CHECK(dev_weights.scalar_type() == at::kByte && dev_weights.is_contiguous(),
              "dev_weights must be contiguous uint8");
  TORCH_CHECK(weights_offsets.scalar_type() == at::kLong, "weights_offsets must be int64");
  TORCH_CHECK(weights_tys.scalar_type() == at::kByte, "weights_tys must be uint8");
  TORCH_CHECK(D_offsets.scalar_type() == at::kInt, "D_offsets must be int32");
  const int32_t ib = index_bytes_of(indices, "indices");
  TORCH_CHECK(index_bytes_of(offsets, "offsets") == ib, "indices and offsets must share a dtype");
  const int64_t T = D_offsets.numel() - 1;
  TORCH_CHECK(T >= 1 && weights_tys.numel() == T && weights_offsets.numel() == T,
              "weights_tys/weights_offsets must have T entries");
  TORCH_CHECK((offsets.numel() - 1) % T == 0, "offsets must have T*B+1 entries");
  const int64_t B = (offsets.numel() - 1) / T;
  const int64_t total_D = total_D_sym.expect_int();
  TORCH_CHECK(output_dtype == MX_SPARSE_FP32 || output_dtype == MX_SPARSE_FP16 ||
                  output_dtype == MX_SPARSE_BF16,
              "output_dtype must be FP32 (0), FP16 (1) or BF16 (5)");
  const float* iw = nullptr;
  Tensor iwc;
  if (indice_weights.has_value() && indice_weights->defined()) {
    check_arg(*indice_weights, dev_weights, "indice_weights", false);
    TORCH_CHECK(indice_weights->scalar_type() == at::kFloat, "indice_weights must be fp32");
    TORCH_CHECK(indice_weights->numel() == indices.numel(),
                "indice_weights must have one entry per index (", indices.numel(), "), got ",
                indice_weights->numel());
    iwc = indice_weights->contiguous();
    iw = iwc.data_ptr<float>();
  }
  ensure_mailbox(dev_weights.device().index(), stream_of(dev_weights));
  auto opts = dev_weights.options().dtype(output_dtype == MX_SPARSE_FP16   ? at::kHalf
                                          : output_dtype == MX_SPARSE_BF16 ? at::kBFloat16
                                                                           : at::kFloat);
  const Tensor idx = indices.contiguous(), off = offsets.contiguous();
  if (pooling_mode == MX_POOL_NONE) {  // sequence lookups: [N, D], D the largest max_*_D
    TORCH_CHECK(iw == nullptr, "PoolingMode NONE takes no indice_weights");
    const int64_t D = std::max({max_int2_D, max_int4_D, max_int8_D, max_float16_D,
                                max_float32_D, max_float8_D.value_or(0)});
    Tensor out = at::empty({indices.numel(), D}, opts);
    MX_CALL(mx_nbit_forward_nobag(
        dev_weights.data_ptr<uint8_t>(), weights_offsets.data_ptr<int64_t>(),
        weights_tys.data_ptr<uint8_t>(), D_offsets.data_ptr<int32_t>(), static_cast<int32_t>(T),
        B, static_cast<int32_t>(max_int2_D), static_cast<int32_t>(max_int4_D),
        static_cast<int32_t>(max_int8_D), static_cast<int32_t>(max_float16_D),
        static_cast<int32_t>(max_float32_D), idx.data_ptr(), off.data_ptr(), ib, indices.numel(),
        static_cast<int32_t>(output_dtype), static_cast<int32_t>(row_alignment.value_or(16)),
        static_cast<int32_t>(max_float8_D.value_or(0)),
        static_cast<int32_t>(fp8_exponent_bits.value_or(-1)),
        static_cast<int32_t>(fp8_exponent_bias.value_or(-1)), out.data_ptr(),
        stream_of(dev_weights)));
    return out;
  }
  Tensor out = at::empty({B, total_D}, opts);
  MX_CALL(mx_nbit_forward(
      dev_weights.data_ptr<uint8_t>(), weights_offsets.data_ptr<int64_t>(),
      weights_tys.data_ptr<uint8_t>(), D_offsets.data_ptr<int32_t>(), static_cast<int32_t>(T), B,
      static_cast<int32_t>(max_int2_D), static_cast<int32_t>(max_int4_D),
      static_cast<int32_t>(max_int8_D), static_cast<int32_t>(max_float16_D),
      static_cast<int32_t>(max_float32_D), idx.data_ptr(), off.data_ptr(), ib,
      static_cast<int32_t>(pooling_mode), iw, static_cast<int32_t>(output_dtype),
      static_cast<int32_t>(row_alignment.value_or(16)),
      static_cast<int32_t>(max_float8_D.value_or(0)),
      static_cast<int32_t>(fp8_exponent_bits.value_or(-1)),
      static_cast<int32_t>(fp8_exponent_bias.value_or(-1)), out.data_ptr(), total_D,
      stream_of(dev_weights)));
  return out;
}

// ---------------------------------------------------------------------------
// Sparse-feature helpers: cumsums and permute_2D_sparse_data
// ---------------------------------------------------------------------------

// kind 0 exclusive, 1 inclusive, 2 complete.
Tensor cumsum_impl(const Tensor& t_in, int32_t kind) {
  check_gpu(t_in, "t_in");
  c10::OptionalDeviceGuard guard(t_in.device());
  TORCH_CHECK(t_in.scalar_type() == at::kInt || t_in.scalar_type() == at::kLong,
              "cumsum input must be int32 or int64, got ", t_in.scalar_type());
  TORCH_CHECK(t_in.dim() == 1 || (kind == 2 && t_in.dim() == 2),
              kind == 2 ? "complete cumsum input must be 1-D or 2-D" : "cumsum input must be 1-D");
  const Tensor x = t_in.contiguous();
  const int32_t eb = static_cast<int32_t>(x.element_size());
  const int64_t rows = x.dim() == 2 ? x.size(0) : 1;
  const int64_t n = x.dim() == 2 ? x.size(1) : x.numel();
  Tensor out = x.dim() == 2 ? at::empty({rows, n + 1}, x.options())
                            : at::empty({kind == 2 ? n + 1 : n}, x.options());
  if (rows == 0) return out;
  const size_t ws_bytes = rows == 1 ? mx_cumsum_workspace_bytes(n, eb) : 0;
  Tensor ws = at::empty({static_cast<int64_t>(ws_bytes)}, x.options().dtype(at::kByte));
  MX_CALL(mx_cumsum(x.data_ptr(), eb, rows, n, kind, out.data_ptr(), ws.data_ptr(), ws_bytes,
                    stream_of(x)));
  return out;
}

Tensor exclusive_cumsum(const Tensor& t_in) { return cumsum_impl(t_in, 0); }
Tensor inclusive_cumsum(const Tensor& t_in) { return cumsum_impl(t_in, 1); }
Tensor complete_cumsum(const Tensor& t_in) { return cumsum_impl(t_in, 2); }

std::tuple<Tensor, Tensor, std::optional<Tensor>> permute_2D_sparse_data(
    const Tensor& permute, const Tensor& lengths, const Tensor& indices,
    const std::optional<Tensor>& weights, std::optional<c10::SymInt> permuted_lengths_sum) {
  check_gpu(lengths, "lengths");
  c10::OptionalDeviceGuard guard(lengths.device());
  check_arg(permute, lengths, "permute", true);
  check_arg(indices, lengths, "indices", false);
  TORCH_CHECK(permute.scalar_type() == at::kInt && permute.dim() == 1, "permute must be 1-D int32");
  TORCH_CHECK(lengths.dim() == 2, "lengths must be [T, B]");
  TORCH_CHECK(lengths.scalar_type() == at::kInt || lengths.scalar_type() == at::kLong,
              "lengths must be int32 or int64");
  const int32_t ib = index_bytes_of(indices, "indices");
  const int64_t T = lengths.size(0), B = lengths.size(1), Tp = permute.numel();
  TORCH_CHECK(T <= 0x7fffffffll, "too many features");
  const Tensor perm = permute.contiguous(), len = lengths.contiguous(), idx = indices.contiguous();
  const int32_t lb = static_cast<int32_t>(len.element_size());
  Tensor plen = at::empty({Tp, B}, len.options());
  MX_CALL(mx_permute_2d_lengths(perm.data_ptr<int32_t>(), Tp, len.data_ptr(), lb,
                                static_cast<int32_t>(T), B, plen.data_ptr(), stream_of(len)));
  const Tensor in_off = cumsum_impl(len.view({-1}), 2);
  const Tensor out_off = cumsum_impl(plen.view({-1}), 2);
  const int64_t out_len = permuted_lengths_sum.has_value()
                              ? permuted_lengths_sum->expect_int()
                              : out_off[Tp * B].item<int64_t>();  // one host sync, as upstream
  Tensor pidx = at::empty({out_len}, idx.options());
  std::optional<Tensor> pw;
  Tensor wc;
  if (weights.has_value() && weights->defined()) {
    check_arg(*weights, lengths, "weights", false);
    TORCH_CHECK(weights->scalar_type() == at::kFloat && weights->numel() == indices.numel(),
                "weights must be fp32 with one entry per index");
    wc = weights->contiguous();
    pw = at::empty({out_len}, wc.options());
  }
  MX_CALL(mx_permute_2d_data(perm.data_ptr<int32_t>(), Tp, static_cast<int32_t>(T), B,
                             in_off.data_ptr(), out_off.data_ptr(), lb, idx.data_ptr(), ib,
                             idx.numel(), wc.defined() ? wc.data_ptr<float>() : nullptr, out_len,
                             pidx.data_ptr(), pw.has_value() ? pw->data_ptr<float>() : nullptr,
                             stream_of(len)));
  return {plen, pidx, pw};
}

std::tuple<Tensor, Tensor, std::optional<Tensor>> permute_1D_sparse_data(
    const Tensor& permute, const Tensor& lengths, const Tensor& indices,
    const std::optional<Tensor>& weights, std::optional<c10::SymInt> permuted_lengths_sum) {
  TORCH_CHECK(lengths.dim() == 1, "lengths must be 1-D [T]");
  auto r = permute_2D_sparse_data(permute, lengths.view({-1, 1}), indices, weights,
                                  permuted_lengths_sum);
  return {std::get<0>(r).view({-1}), std::get<1>(r), std::get<2>(r)};
}

Tensor offsets_range(const Tensor& offsets, c10::SymInt range_size_sym) {
  check_gpu(offsets, "offsets");
  c10::OptionalDeviceGuard guard(offsets.device());
  TORCH_CHECK(offsets.dim() == 1, "offsets must be 1-D");
  const int32_t ib = index_bytes_of(offsets, "offsets");
  const int64_t range_size = range_size_sym.expect_int();
  const Tensor off = offsets.contiguous();
  Tensor out = at::empty({range_size}, off.options());
  MX_CALL(mx_offsets_range(off.data_ptr(), ib, off.numel(), range_size, out.data_ptr(),
                           stream_of(off)));
  return out;
}

Tensor expand_into_jagged_permute(const Tensor& permute, const Tensor& input_offsets,
                                  const Tensor& output_offsets, c10::SymInt output_size_sym) {
  check_gpu(permute, "permute");
  c10::OptionalDeviceGuard guard(permute.device());
  check_arg(input_offsets, permute, "input_offsets", true);
  check_arg(output_offsets, permute, "output_offsets", true);
  TORCH_CHECK(permute.scalar_type() == at::kInt, "permute must be int32");
  const int32_t ib = index_bytes_of(input_offsets, "input_offsets");
  TORCH_CHECK(index_bytes_of(output_offsets, "output_offsets") == ib,
              "input_offsets and output_offsets must share a dtype");
  const int64_t output_size = output_size_sym.expect_int();
  const Tensor p = permute.contiguous(), io = input_offsets.contiguous(),
               oo = output_offsets.contiguous();
  Tensor out = at::empty({output_size}, io.options());
  MX_CALL(mx_expand_into_jagged_permute(p.data_ptr<int32_t>(), p.numel(), io.data_ptr(),
                                        io.numel(), oo.data_ptr(), oo.numel(), ib, output_size,
                                        out.data_ptr(), stream_of(p)));
  return out;
}

}  // namespace mx_ops

TORCH_LIBRARY_FRAGMENT(fbgemm, m) {
  m.def("permute_1D_sparse_data(Tensor permute, Tensor lengths, Tensor values, "
        "Tensor? weights=None, SymInt? permuted_lengths_sum=None) -> (Tensor, Tensor, Tensor?)");
  m.def("offsets_range(Tensor offsets, SymInt range_size) -> Tensor");
  m.def("expand_into_jagged_permute(Tensor permute, Tensor input_offset, Tensor output_offset, "
        "SymInt output_size) -> Tensor");
  m.def("asynchronous_exclusive_cumsum(Tensor t_in) -> Tensor");
  m.def("asynchronous_inclusive_cumsum(Tensor t_in) -> Tensor");
  m.def("asynchronous_complete_cumsum(Tensor t_in) -> Tensor");
  m.def("permute_2D_sparse_data(Tensor permute, Tensor lengths, Tensor values, "
        "Tensor? weights=None, SymInt? permuted_lengths_sum=None) -> (Tensor, Tensor, Tensor?)");
  m.def("jagged_to_padded_dense_forward(Tensor values, Tensor[] offsets, SymInt[] max_lengths, "
        "float padding_value=0) -> Tensor");
  m.def("jagged_to_padded_dense(Tensor values, Tensor[] offsets, SymInt[] max_lengths, "
        "float padding_value=0) -> Tensor");
  m.def("jagged_to_padded_dense_backward(Tensor grad_output, Tensor[] offsets, SymInt total_L) "
        "-> Tensor");
  m.def("dense_to_jagged_forward(Tensor dense, Tensor[] offsets, SymInt? total_L=None) -> Tensor");
  m.def("dense_to_jagged(Tensor dense, Tensor[] x_offsets, SymInt? total_L=None) "
        "-> (Tensor, Tensor[])");
  m.def("jagged_dense_elementwise_add_jagged_output(Tensor x_values, Tensor[] x_offsets, "
        "Tensor y) -> (Tensor, Tensor[])");
  m.def("jagged_dense_elementwise_mul(Tensor x_values, Tensor[] x_offsets, Tensor y) -> Tensor");
  m.def("jagged_2d_to_dense(Tensor values, Tensor offsets, SymInt max_sequence_length) -> Tensor");
  m.def("jagged_1d_to_dense(Tensor values, Tensor offsets, SymInt max_sequence_length, "
        "int padding_value) -> Tensor");
  m.def("split_embedding_codegen_forward_unweighted_cuda(Tensor dev_weights, Tensor uvm_weights, "
        "Tensor lxu_cache_weights, Tensor weights_placements, Tensor weights_offsets, "
        "Tensor D_offsets, SymInt total_D, SymInt max_D, Tensor indices, Tensor offsets, "
        "int pooling_mode, Tensor lxu_cache_locations, Tensor uvm_cache_stats, "
        "int output_dtype, bool is_experimental) -> Tensor");
  m.def("split_embedding_codegen_forward_weighted_cuda(Tensor dev_weights, Tensor uvm_weights, "
        "Tensor lxu_cache_weights, Tensor weights_placements, Tensor weights_offsets, "
        "Tensor D_offsets, SymInt total_D, SymInt max_D, Tensor indices, Tensor offsets, "
        "int pooling_mode, Tensor indice_weights, Tensor lxu_cache_locations, "
        "Tensor uvm_cache_stats, int output_dtype, bool is_experimental) -> Tensor");
  m.def("split_embedding_nobag_codegen_forward_unweighted_cuda(Tensor dev_weights, "
        "Tensor uvm_weights, Tensor lxu_cache_weights, Tensor weights_placements, "
        "Tensor weights_offsets, SymInt D, Tensor indices, Tensor offsets, "
        "Tensor lxu_cache_locations, Tensor uvm_cache_stats, int output_dtype, "
        "bool is_experimental) -> Tensor");
  m.def("split_embedding_nobag_backward_codegen_rowwise_adagrad_unweighted_exact_cuda("
        "Tensor grad_output, Tensor(a!) dev_weights, Tensor uvm_weights, "
        "Tensor lxu_cache_weights, Tensor weights_placements, Tensor weights_offsets, SymInt D, "
        "Tensor hash_size_cumsum, int total_hash_size_bits, Tensor indices, Tensor offsets, "
        "Tensor lxu_cache_locations, int BT_block_size, int max_segment_length_per_warp, "
        "bool stochastic_rounding, Tensor(b!) momentum1_dev, Tensor momentum1_uvm, "
        "Tensor momentum1_placements, Tensor momentum1_offsets, float eps=0, "
        "float learning_rate=0, float weight_decay=0.0, int weight_decay_mode=0, "
        "float max_norm=0.0) -> Tensor");
  m.def("get_infos_metadata(Tensor unused, int B, int T) -> (int, int)");
  m.def("transpose_embedding_input(Tensor hash_size_cumsum, int total_hash_size_bits, "
        "Tensor indices, Tensor offsets, bool nobag=False, Tensor? vbe_b_t_map=None, "
        "int info_B_num_bits=26, int info_B_mask=67108863, int total_unique_indices=-1) "
        "-> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda("
        "Tensor grad_output, Tensor(a!) dev_weights, Tensor uvm_weights, "
        "Tensor lxu_cache_weights, Tensor weights_placements, Tensor weights_offsets, "
        "Tensor D_offsets, SymInt max_D, Tensor hash_size_cumsum, int total_hash_size_bits, "
        "Tensor indices, Tensor offsets, int pooling_mode, Tensor lxu_cache_locations, "
        "int BT_block_size, int max_segment_length_per_warp, bool stochastic_rounding, "
        "Tensor(b!) momentum1_dev, Tensor momentum1_uvm, Tensor momentum1_placements, "
        "Tensor momentum1_offsets, float eps=0, float learning_rate=0, float weight_decay=0.0, "
        "int weight_decay_mode=0, float max_norm=0.0) -> Tensor");
  m.def("split_embedding_backward_codegen_rowwise_adagrad_weighted_exact_cuda("
        "Tensor grad_output, Tensor(a!) dev_weights, Tensor uvm_weights, "
        "Tensor lxu_cache_weights, Tensor weights_placements, Tensor weights_offsets, "
        "Tensor D_offsets, SymInt max_D, Tensor hash_size_cumsum, int total_hash_size_bits, "
        "Tensor indices, Tensor offsets, int pooling_mode, Tensor indice_weights, "
        "Tensor lxu_cache_locations, int BT_block_size, int max_segment_length_per_warp, "
        "bool stochastic_rounding, Tensor(b!) momentum1_dev, Tensor momentum1_uvm, "
        "Tensor momentum1_placements, Tensor momentum1_offsets, float eps=0, "
        "float learning_rate=0, float weight_decay=0.0, int weight_decay_mode=0, "
        "float max_norm=0.0) -> Tensor");
  m.def("split_embedding_codegen_grad_indice_weights_cuda(Tensor grad_output, "
        "Tensor dev_weights, Tensor uvm_weights, Tensor lxu_cache_weights, "
        "Tensor weights_placements, Tensor weights_offsets, Tensor D_offsets, SymInt max_D, "
        "Tensor indices, Tensor offsets, Tensor lxu_cache_locations, "
        "Tensor? feature_requires_grad, int pooling_mode=0) -> Tensor");
  m.def("split_embedding_codegen_lookup_rowwise_adagrad_function(Tensor placeholder_autograd_tensor, "
        "Tensor dev_weights, Tensor uvm_weights, Tensor lxu_cache_weights, "
        "Tensor weights_placements, Tensor weights_offsets, Tensor D_offsets, SymInt total_D, "
        "SymInt max_D, Tensor hash_size_cumsum, int total_hash_size_bits, Tensor indices, "
        "Tensor offsets, int pooling_mode, Tensor? indice_weights, Tensor? feature_requires_grad, "
        "Tensor lxu_cache_locations, bool gradient_clipping, float max_gradient, "
        "bool stochastic_rounding, Tensor momentum1_dev, Tensor momentum1_uvm, "
        "Tensor momentum1_placements, Tensor momentum1_offsets, float eps=0, "
        "float learning_rate=0, float weight_decay=0.0, int weight_decay_mode=0, "
        "float max_norm=0.0, int output_dtype=0, Tensor? B_offsets=None, "
        "Tensor? vbe_output_offsets_feature_rank=None, "
        "Tensor? vbe_B_offsets_rank_per_feature=None, SymInt max_B=-1, "
        "SymInt max_B_feature_rank=-1, SymInt vbe_output_size=-1) -> Tensor");
  m.def("generate_vbe_metadata(Tensor B_offsets, Tensor B_offsets_rank_per_feature, "
        "Tensor output_offsets_feature_rank, Tensor D_offsets, int D, bool nobag, "
        "SymInt max_B_feature_rank, int info_B_num_bits, SymInt total_B) -> (Tensor, Tensor)");
  m.def("split_embedding_codegen_forward_unweighted_vbe_cuda(Tensor dev_weights, "
        "Tensor uvm_weights, Tensor lxu_cache_weights, Tensor weights_placements, "
        "Tensor weights_offsets, Tensor D_offsets, SymInt total_D, SymInt max_D, Tensor indices, "
        "Tensor offsets, int pooling_mode, Tensor lxu_cache_locations, Tensor uvm_cache_stats, "
        "int output_dtype, Tensor vbe_row_output_offsets, Tensor vbe_b_t_map, "
        "SymInt vbe_output_size, int info_B_num_bits, int info_B_mask, bool is_experimental) "
        "-> Tensor");
  m.def("split_embedding_codegen_forward_weighted_vbe_cuda(Tensor dev_weights, "
        "Tensor uvm_weights, Tensor lxu_cache_weights, Tensor weights_placements, "
        "Tensor weights_offsets, Tensor D_offsets, SymInt total_D, SymInt max_D, Tensor indices, "
        "Tensor offsets, int pooling_mode, Tensor indice_weights, Tensor lxu_cache_locations, "
        "Tensor uvm_cache_stats, int output_dtype, Tensor vbe_row_output_offsets, "
        "Tensor vbe_b_t_map, SymInt vbe_output_size, int info_B_num_bits, int info_B_mask, "
        "bool is_experimental) -> Tensor");
  m.def("split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_vbe_cuda("
        "Tensor grad_output, Tensor(a!) dev_weights, Tensor uvm_weights, "
        "Tensor lxu_cache_weights, Tensor weights_placements, Tensor weights_offsets, "
        "Tensor D_offsets, SymInt max_D, Tensor hash_size_cumsum, int total_hash_size_bits, "
        "Tensor indices, Tensor offsets, int pooling_mode, Tensor lxu_cache_locations, "
        "int BT_block_size, int max_segment_length_per_warp, bool stochastic_rounding, "
        "int info_B_num_bits, int info_B_mask, Tensor B_offsets, Tensor vbe_row_output_offsets, "
        "Tensor vbe_b_t_map, Tensor(b!) momentum1_dev, Tensor momentum1_uvm, "
        "Tensor momentum1_placements, Tensor momentum1_offsets, float eps=0, "
        "float learning_rate=0, float weight_decay=0.0, int weight_decay_mode=0, "
        "float max_norm=0.0) -> Tensor");
  m.def("split_embedding_backward_codegen_rowwise_adagrad_weighted_exact_vbe_cuda("
        "Tensor grad_output, Tensor(a!) dev_weights, Tensor uvm_weights, "
        "Tensor lxu_cache_weights, Tensor weights_placements, Tensor weights_offsets, "
        "Tensor D_offsets, SymInt max_D, Tensor hash_size_cumsum, int total_hash_size_bits, "
        "Tensor indices, Tensor offsets, int pooling_mode, Tensor indice_weights, "
        "Tensor lxu_cache_locations, int BT_block_size, int max_segment_length_per_warp, "
        "bool stochastic_rounding, int info_B_num_bits, int info_B_mask, Tensor B_offsets, "
        "Tensor vbe_row_output_offsets, Tensor vbe_b_t_map, Tensor(b!) momentum1_dev, "
        "Tensor momentum1_uvm, Tensor momentum1_placements, Tensor momentum1_offsets, "
        "float eps=0, float learning_rate=0, float weight_decay=0.0, int weight_decay_mode=0, "
        "float max_norm=0.0) -> Tensor");
  m.def("split_embedding_codegen_grad_indice_weights_vbe_cuda(Tensor grad_output, "
        "Tensor dev_weights, Tensor uvm_weights, Tensor lxu_cache_weights, "
        "Tensor weights_placements, Tensor weights_offsets, Tensor D_offsets, SymInt max_D, "
        "Tensor indices, Tensor offsets, Tensor lxu_cache_locations, "
        "Tensor? feature_requires_grad, Tensor vbe_row_output_offsets, Tensor vbe_b_t_map, "
        "int info_B_num_bits, int info_B_mask, int pooling_mode=0) -> Tensor");
  m.def("FloatToFused8BitRowwiseQuantized(Tensor t) -> Tensor");
  m.def("HalfToFused8BitRowwiseQuantized(Tensor t) -> Tensor");
  m.def("FloatOrHalfToFused8BitRowwiseQuantized(Tensor t) -> Tensor");
  m.def("Fused8BitRowwiseQuantizedToFloat(Tensor input) -> Tensor");
  m.def("Fused8BitRowwiseQuantizedToHalf(Tensor input) -> Tensor");
  m.def("FloatToFusedNBitRowwiseQuantizedSBHalf(Tensor input, int bit_rate) -> Tensor");
  m.def("HalfToFusedNBitRowwiseQuantizedSBHalf(Tensor input, int bit_rate) -> Tensor");
  m.def("FloatOrHalfToFusedNBitRowwiseQuantizedSBHalf(Tensor input, int bit_rate) -> Tensor");
  m.def("FusedNBitRowwiseQuantizedSBHalfToFloat(Tensor input, int bit_rate) -> Tensor");
  m.def("FusedNBitRowwiseQuantizedSBHalfToHalf(Tensor input, int bit_rate) -> Tensor");
  m.def("FloatToHFP8Quantized(Tensor input, int ebits, int exponent_bias, float max_pos) -> Tensor");
  m.def("HFP8QuantizedToFloat(Tensor input, int ebits, int exponent_bias) -> Tensor");
  m.def("bounds_check_indices(Tensor rows_per_table, Tensor(a!) indices, Tensor(b!) offsets, "
        "int bounds_check_mode, Tensor(c!) warning, Tensor? weights=None, "
        "Tensor? B_offsets=None, SymInt max_B=-1, Tensor? b_t_map=None, int info_B_num_bits=-1, "
        "int info_B_mask=-1, int bounds_check_version=1) -> ()");
  m.def("int_nbit_split_embedding_codegen_lookup_function(Tensor dev_weights, "
        "Tensor uvm_weights, Tensor weights_placements, Tensor weights_offsets, "
        "Tensor weights_tys, Tensor D_offsets, SymInt total_D, int max_int2_D, int max_int4_D, "
        "int max_int8_D, int max_float16_D, int max_float32_D, Tensor indices, Tensor offsets, "
        "int pooling_mode, Tensor? indice_weights, int output_dtype, "
        "Tensor? lxu_cache_weights, Tensor? lxu_cache_locations, int? row_alignment=None, "
        "int? max_float8_D=0, int? fp8_exponent_bits=-1, int? fp8_exponent_bias=-1) -> Tensor");
}

TORCH_LIBRARY_IMPL(fbgemm, CUDA, m) {
  m.impl("jagged_to_padded_dense_forward", TORCH_FN(mx_ops::jagged_to_padded_dense_forward));
  m.impl("jagged_to_padded_dense", TORCH_FN(mx_ops::jagged_to_padded_dense_plain));
  m.impl("jagged_to_padded_dense_backward", TORCH_FN(mx_ops::jagged_to_padded_dense_backward));
  m.impl("dense_to_jagged_forward", TORCH_FN(mx_ops::dense_to_jagged_forward));
  m.impl("dense_to_jagged", TORCH_FN(mx_ops::dense_to_jagged_plain));
  m.impl("jagged_dense_elementwise_add_jagged_output", TORCH_FN(mx_ops::jagged_dense_add_plain));
  m.impl("jagged_dense_elementwise_mul", TORCH_FN(mx_ops::jagged_dense_mul_forward));
  m.impl("jagged_2d_to_dense", TORCH_FN(mx_ops::jagged_2d_to_dense_plain));
  m.impl("jagged_1d_to_dense", TORCH_FN(mx_ops::jagged_1d_to_dense));
  m.impl("split_embedding_codegen_forward_unweighted_cuda", TORCH_FN(mx_ops::forward_unweighted));
  m.impl("split_embedding_codegen_forward_weighted_cuda", TORCH_FN(mx_ops::forward_weighted));
  m.impl("transpose_embedding_input", TORCH_FN(mx_ops::transpose_embedding_input));
  m.impl("split_embedding_nobag_codegen_forward_unweighted_cuda",
         TORCH_FN(mx_ops::forward_nobag_unweighted));
  m.impl("split_embedding_nobag_backward_codegen_rowwise_adagrad_unweighted_exact_cuda",
         TORCH_FN(mx_ops::backward_rowwise_adagrad_nobag));
  m.impl("split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda",
         TORCH_FN(mx_ops::backward_rowwise_adagrad_exact));
  m.impl("split_embedding_codegen_lookup_rowwise_adagrad_function",
         TORCH_FN(mx_ops::lookup_rowwise_adagrad));
  m.impl("split_embedding_backward_codegen_rowwise_adagrad_weighted_exact_cuda",
         TORCH_FN(mx_ops::backward_rowwise_adagrad_weighted_exact));
  m.impl("split_embedding_codegen_grad_indice_weights_cuda",
         TORCH_FN(mx_ops::grad_indice_weights));
  m.impl("generate_vbe_metadata", TORCH_FN(mx_ops::generate_vbe_metadata));
  m.impl("split_embedding_codegen_forward_unweighted_vbe_cuda",
         TORCH_FN(mx_ops::forward_unweighted_vbe));
  m.impl("split_embedding_codegen_forward_weighted_vbe_cuda",
         TORCH_FN(mx_ops::forward_weighted_vbe));
  m.impl("split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_vbe_cuda",
         TORCH_FN(mx_ops::backward_rowwise_adagrad_exact_vbe));
  m.impl("split_embedding_backward_codegen_rowwise_adagrad_weighted_exact_vbe_cuda",
         TORCH_FN(mx_ops::backward_rowwise_adagrad_weighted_exact_vbe));
  m.impl("split_embedding_codegen_grad_indice_weights_vbe_cuda",
         TORCH_FN(mx_ops::grad_indice_weights_vbe));
  m.impl("int_nbit_split_embedding_codegen_lookup_function", TORCH_FN(mx_ops::int_nbit_lookup));
  m.impl("bounds_check_indices", TORCH_FN(mx_ops::bounds_check_indices));
  m.impl("asynchronous_exclusive_cumsum", TORCH_FN(mx_ops::exclusive_cumsum));
  m.impl("asynchronous_inclusive_cumsum", TORCH_FN(mx_ops::inclusive_cumsum));
  m.impl("asynchronous_complete_cumsum", TORCH_FN(mx_ops::complete_cumsum));
  m.impl("permute_2D_sparse_data", TORCH_FN(mx_ops::permute_2D_sparse_data));
  m.impl("permute_1D_sparse_data", TORCH_FN(mx_ops::permute_1D_sparse_data));
  m.impl("offsets_range", TORCH_FN(mx_ops::offsets_range));
  m.impl("expand_into_jagged_permute", TORCH_FN(mx_ops::expand_into_jagged_permute));
  m.impl("FloatToFused8BitRowwiseQuantized", TORCH_FN(mx_ops::float_to_8bit));
  m.impl("HalfToFused8BitRowwiseQuantized", TORCH_FN(mx_ops::half_to_8bit));
  m.impl("FloatOrHalfToFused8BitRowwiseQuantized", TORCH_FN(mx_ops::float_or_half_to_8bit));
  m.impl("Fused8BitRowwiseQuantizedToFloat", TORCH_FN(mx_ops::fused8bit_to_float));
  m.impl("Fused8BitRowwiseQuantizedToHalf", TORCH_FN(mx_ops::fused8bit_to_half));
  m.impl("FloatToFusedNBitRowwiseQuantizedSBHalf", TORCH_FN(mx_ops::float_to_nbit));
  m.impl("HalfToFusedNBitRowwiseQuantizedSBHalf", TORCH_FN(mx_ops::half_to_nbit));
  m.impl("FloatOrHalfToFusedNBitRowwiseQuantizedSBHalf", TORCH_FN(mx_ops::float_or_half_to_nbit));
  m.impl("FusedNBitRowwiseQuantizedSBHalfToFloat", TORCH_FN(mx_ops::nbit_to_float));
  m.impl("FusedNBitRowwiseQuantizedSBHalfToHalf", TORCH_FN(mx_ops::nbit_to_half));
  m.impl("FloatToHFP8Quantized", TORCH_FN(mx_ops::float_to_hfp8));
  m.impl("HFP8QuantizedToFloat", TORCH_FN(mx_ops::hfp8_to_float));
}

TORCH_LIBRARY_IMPL(fbgemm, Autograd, m) {
  m.impl("jagged_to_padded_dense", TORCH_FN(mx_ops::jagged_to_padded_dense_autograd));
  m.impl("dense_to_jagged", TORCH_FN(mx_ops::dense_to_jagged_autograd));
  m.impl("jagged_dense_elementwise_add_jagged_output", TORCH_FN(mx_ops::jagged_dense_add_autograd));
  m.impl("jagged_dense_elementwise_mul", TORCH_FN(mx_ops::jagged_dense_mul_autograd));
  m.impl("jagged_2d_to_dense", TORCH_FN(mx_ops::jagged_2d_to_dense_autograd));
  m.impl("split_embedding_codegen_lookup_rowwise_adagrad_function",
         TORCH_FN(mx_ops::lookup_rowwise_adagrad));
}

TORCH_LIBRARY_IMPL(fbgemm, CompositeExplicitAutograd, m) {
  m.impl("get_infos_metadata", TORCH_FN(mx_ops::get_infos_metadata));
}

// Ops of this build that have no fbgemm counterpart.
TORCH_LIBRARY(mx_fbgemm, m) {
  m.def("pending_lookback_faults(int device) -> int", &mx_ops::pending_lookback_faults);
  m.def("test_force_lookback_giveup(bool enable) -> ()", &mx_ops::test_force_lookback_giveup);
  m.def("test_force_wide_sort_words(bool enable) -> ()", &mx_ops::test_force_wide_sort_words);
  m.def("test_force_workspace_counters(bool enable) -> ()",
        &mx_ops::test_force_workspace_counters);
}
