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
#include <string>

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

// ---- fallback by construction -------------------------------------------------------------------------------------
//
// A hot-path op checks what it covers with NEED(cond, why) before it launches anything; a failed NEED (or an
// OMT_UNSUPPORTED status from the library) throws Unsupported and Safe<> re-runs the call on torch's HIP kernels,
// recording "op (why)" in fallback_counts() (the reference's FALLBACKS, csrc/omt.h:161-220). With
// OMARCHY_MAC_TORCH_STRICT=1 that is an error instead.

struct Unsupported : std::exception {
  std::string why;
  explicit Unsupported(std::string w) : why(std::move(w)) {}
  const char* what() const noexcept override { return why.c_str(); }
};
#define NEED(cond, why)                          \
  do {                                           \
    if (!(cond)) throw ::omt::Unsupported(why);  \
  } while (0)

// Raises for a non-OK library status: OMT_UNSUPPORTED -> Unsupported, OMT_OOM -> torch.OutOfMemoryError (after
// emptying the cache, the library already retried once), anything else -> RuntimeError with the library's message.
void check(int status, const char* what);

std::recursive_mutex& big_lock();
#define OMT_LOCK std::lock_guard<std::recursive_mutex> omt_lock_(::omt::big_lock())

std::map<std::string, int64_t>& fallback_counts();   // hot-path ops that could not use the HIP kernels
std::map<std::string, int64_t>& delegated_counts();  // other ops, run on torch's HIP kernels (counted when enabled)
void note_fallback(const std::string& op, const std::string& why);
// Autotunes (direction, geometry) once when tuning is on and the plan cache has no entry (libomt_hip.so times the
// candidates on the current stream); no-op otherwise.
// Tunes grad input and grad weight together (for omt_conv_bwd) unless both already have cached plans.
void tune_conv_bwd(const omt_conv_geo& g);
void tune_conv(int dir, const omt_conv_geo& g);
bool strict_mode();
bool debug_mode();
void set_debug_mode(bool on);
void set_count_delegated(bool on);
void debug_after(const char* op);  // debug mode: synchronize and surface asynchronous errors with the op's name

void hip_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack);        // counted
void hip_fallback_quiet(const c10::OperatorHandle& op, torch::jit::Stack* stack);  // used by Safe<> after NEED

template <class Op, auto Fn, class Sig = typename Op::schema>
struct Safe;
template <class Op, auto Fn, class R, class... A>
struct Safe<Op, Fn, R(A...)> {
  static R call(typename c10::maybe_keep_symint<false, A>::type... a) {
    OMT_LOCK;
    try {
      if constexpr (std::is_void_v<R>) {
        Fn(a...);
        if (debug_mode()) debug_after(Op::name);
      } else {
        R r = Fn(a...);
        if (debug_mode()) debug_after(Op::name);
        return r;
      }
    } catch (const Unsupported& e) {
      std::string name = std::string(Op::name).substr(6);
      if (Op::overload_name[0]) name += std::string(".") + Op::overload_name;
      TORCH_CHECK(!strict_mode(), "omarchy-mac-torch (strict): ", name, " not supported by the HIP kernels: ", e.why);
      note_fallback(name, e.why);
      return at::native::call_fallback_fn<&hip_fallback_quiet, Op>::call(a...);
    }
  }
};
template <class Op, class F>
void impl_name(torch::Library& m, F f) {
  std::string name = std::string(Op::name).substr(6);
  if (Op::overload_name[0]) name += std::string(".") + Op::overload_name;
  m.impl(name.c_str(), f);
}
// register aten::<op> for the device through the fallback wrapper
#define OMT_IMPL(m, op, fn) ::omt::impl_name<at::_ops::op>(m, &::omt::Safe<at::_ops::op, fn>::call)

// ---- geometry helpers shared by ops.cpp and plans.cpp -------------------------------------------------------------

omt_conv_geo conv_geo(int64_t n, int64_t ci, int64_t co, int64_t ih, int64_t iw, int64_t ks, int64_t stride,
                      int64_t pad);
int64_t pool_out(int64_t size, int64_t k, int64_t s, int64_t p, int64_t d, bool ceil);

}  // namespace omt
