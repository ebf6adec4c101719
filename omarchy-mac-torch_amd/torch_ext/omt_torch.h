// Shared declarations of the torch extension (_native): the "omarchy_mac_torch" PrivateUse1 device on MI355X.
//
// Device tensors live in HBM allocated by libomt_hip.so's caching allocator. The convolution hot path (conv, BN,
// pools, the omt:: fused ops and the stack plans) runs the library's HIP kernels through its C ABI. Every other aten
// op is delegated, by a boxed fallback, to torch's own HIP kernels on an alias of the same memory (hip_alias), so a
// training step never round-trips through the host.
#pragma once

#include <ATen/ATen.h>
#include <ATen/native/CPUFallback.h>
#include <torch/library.h>

#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <type_traits>

#include "omt_hip.h"

namespace omt {

using at::IntArrayRef;
using at::Tensor;
constexpr c10::DeviceType kDev = c10::DeviceType::PrivateUse1;

// ---- memory and tensors (device.cpp) -----------------------------------------------------------------------------

c10::Allocator* allocator();
inline bool is_dev(const Tensor& t) { return t.defined() && t.device().type() == kDev; }
inline bool f32(const Tensor& t) { return t.defined() && t.scalar_type() == at::kFloat; }
Tensor empty_dev(IntArrayRef size, at::ScalarType dt = at::kFloat);
// device tensor of a 4-D size in channels_last memory order
Tensor empty_dev_cl(IntArrayRef size, at::ScalarType dt = at::kFloat);
// 4-D tensor whose memory is channels-last (NHWC) and not also plain NCHW (with c == 1 or h * w == 1 the two orders
// are one and the NCHW kernels read it as it is)
inline bool is_cl(const Tensor& t) {
  return t.defined() && t.dim() == 4 && !t.is_contiguous() && t.is_contiguous(at::MemoryFormat::ChannelsLast);
}
// byte workspace for a C-ABI call (undefined tensor when bytes == 0)
Tensor workspace(size_t bytes);
inline void* wsptr(const Tensor& ws) { return ws.defined() ? ws.data_ptr() : nullptr; }
inline size_t wsbytes(const Tensor& ws) { return ws.defined() ? (size_t)ws.numel() : 0; }
// torch HIP-device ("cuda") tensor over the same memory and geometry as device tensor t (non-owning)
Tensor hip_alias(const Tensor& t);
// device tensor that owns torch HIP tensor h's storage (same memory and geometry)
Tensor dev_from_hip(const Tensor& h);
// torch's current HIP stream, the stream every device op runs on
void* cur_stream();
// raw float pointers (null for undefined tensors)
inline const float* fp(const Tensor& t) { return t.defined() ? t.data_ptr<float>() : nullptr; }
inline float* fpm(const Tensor& t) { return t.defined() ? t.mutable_data_ptr<float>() : nullptr; }
inline const float* fp(const std::optional<Tensor>& t) { return t && t->defined() ? t->data_ptr<float>() : nullptr; }
inline bool defined(const std::optional<Tensor>& t) { return t && t->defined(); }

// ---- coverage, and where uncovered calls go --------------------------------------------------------------------
//
// A hot-path wrapper states what its kernels cover with cover(ok, why) before it launches anything (an OMT_UNSUPPORTED
// status from the library means the same). A call outside that raises NotCovered, and the wrapper's registration
// (HotKernel) hands the untouched arguments to torch's HIP kernels over aliases of the same memory, counting
// "op (why)" in fallback_counts() (the reference's FALLBACKS, csrc/omt.h:161-220). With OMARCHY_MAC_TORCH_STRICT=1 such
// a call raises instead.

class NotCovered : public std::runtime_error {
 public:
  using std::runtime_error::runtime_error;
};
inline void cover(bool ok, const char* why) {
  if (!ok) throw NotCovered(why);
}

// Raises for a non-OK library status: OMT_UNSUPPORTED -> NotCovered, OMT_OOM -> torch.OutOfMemoryError (the library
// has already emptied its cache and retried once), anything else -> RuntimeError with the library's message.
void check(int status, const char* what);

std::recursive_mutex& big_lock();
#define OMT_LOCK std::lock_guard<std::recursive_mutex> omt_lock_(::omt::big_lock())

std::map<std::string, int64_t>& fallback_counts();   // hot-path ops that could not use the HIP kernels
std::map<std::string, int64_t>& delegated_counts();  // other ops, run on torch's HIP kernels (counted when enabled)
// The single exit of every uncovered call: raises in strict mode, else counts "op (why)".
void left_hot_path(const std::string& op, const char* why);
// Autotunes (direction, geometry) once when tuning is on and the plan cache has no entry (libomt_hip.so times the
// candidates on the current stream); no-op otherwise.
// Tunes grad input and grad weight together (for omt_conv_bwd) unless both already have cached plans.
void tune_conv_bwd(const omt_conv_geo& g);
void tune_conv(int dir, const omt_conv_geo& g);
bool strict_mode();
void set_strict_mode(bool on);
bool debug_mode();
void set_debug_mode(bool on);
void set_count_delegated(bool on);
// Failure-path tests: the next debug_point reports `msg` as if the stream had returned a device error.
void force_next_sync_error(const std::string& msg);
// Debug mode only: synchronizes the current stream and raises any asynchronous device error with the op's name.
void debug_point(const std::string& op);

void hip_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack);        // counted
void hip_fallback_quiet(const c10::OperatorHandle& op, torch::jit::Stack* stack);  // the exit of HotKernel

// "name.overload" of an aten operator, as FALLBACKS and the registrations spell it.
template <class Op>
const std::string& op_label() {
  static const std::string label = [] {
    std::string s(Op::name);
    s.erase(0, s.find("::") + 2);
    if (*Op::overload_name) (s += '.') += Op::overload_name;
    return s;
  }();
  return label;
}

// The device kernel of aten operator Op: Impl under the device lock; a call Impl does not cover continues on torch's
// HIP kernels. Specialized on Impl's own signature, which the registration checks against Op's schema.
template <class Op, auto Impl>
struct HotKernel;
template <class Op, class R, class... A, R (*Impl)(A...)>
struct HotKernel<Op, Impl> {
  static R run(A... a) {
    OMT_LOCK;
    try {
      if constexpr (std::is_void_v<R>) {
        Impl(a...);
        if (debug_mode()) debug_point(op_label<Op>());
      } else {
        R out = Impl(a...);
        if (debug_mode()) debug_point(op_label<Op>());
        return out;
      }
    } catch (const NotCovered& e) {
      left_hot_path(op_label<Op>(), e.what());
      return at::native::call_fallback_fn<&hip_fallback_quiet, Op>::call(a...);
    }
  }
};

// The device kernel of an aten op outside the convolution path (pointwise ops, reductions, the loss): Impl where it
// covers the call, else torch's HIP kernels like any op without a kernel here (counted with the delegated ops when
// counting is on; neither a FALLBACKS entry nor an error in strict mode).
template <class Op, auto Impl>
struct AuxKernel;
template <class Op, class R, class... A, R (*Impl)(A...)>
struct AuxKernel<Op, Impl> {
  static R run(A... a) {
    OMT_LOCK;
    try {
      if constexpr (std::is_void_v<R>) {
        Impl(a...);
        if (debug_mode()) debug_point(op_label<Op>());
      } else {
        R out = Impl(a...);
        if (debug_mode()) debug_point(op_label<Op>());
        return out;
      }
    } catch (const NotCovered&) {
      return at::native::call_fallback_fn<&hip_fallback, Op>::call(a...);
    }
  }
};

// Registers HotKernels into a TORCH_LIBRARY_IMPL block: HotOps(m).on<at::_ops::op, &impl>().on<...>(); aux<> for
// AuxKernels.
class HotOps {
 public:
  explicit HotOps(torch::Library& lib) : lib_(lib) {}
  template <class Op, auto Impl>
  HotOps& on() {
    lib_.impl(op_label<Op>().c_str(), &HotKernel<Op, Impl>::run);
    return *this;
  }
  template <class Op, auto Impl>
  HotOps& aux() {
    lib_.impl(op_label<Op>().c_str(), &AuxKernel<Op, Impl>::run);
    return *this;
  }

 private:
  torch::Library& lib_;
};

// For the omt:: fused ops, whose way out is their composite reference (plain aten ops, which in turn reach the device
// kernels or torch's): Dev(a...) if it covers the call, else Ref(a...).
template <auto Dev, auto Ref, class... A>
auto dev_or_ref(const char* op, A&&... a) {
  OMT_LOCK;
  try {
    return Dev(a...);
  } catch (const NotCovered& e) {
    left_hot_path(op, e.what());
    return Ref(a...);
  }
}

// ---- geometry helpers shared by ops.cpp and plans.cpp -------------------------------------------------------------

omt_conv_geo conv_geo(int64_t n, int64_t ci, int64_t co, int64_t ih, int64_t iw, int64_t ks, int64_t stride,
                      int64_t pad);
int64_t pool_out(int64_t size, int64_t k, int64_t s, int64_t p, int64_t d, bool ceil);

}  // namespace omt
