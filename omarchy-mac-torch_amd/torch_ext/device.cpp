// The "omarchy_mac_torch" PrivateUse1 device: allocator, tensor creation and copies, view ops, device guard with HIP
// events, hooks, and the boxed fallback that runs every op without a hot-path kernel on torch's HIP kernels.
// Reference counterpart: csrc/device.cpp:18-256 (allocator, guard, hooks, generator, CPU fallback, memory ops).
#include <ATen/EmptyTensor.h>
#include <ATen/detail/PrivateUse1HooksInterface.h>
#include <ATen/hip/HIPGeneratorImpl.h>
#include <ATen/native/Resize.h>
#include <c10/core/impl/DeviceGuardImplInterface.h>
#include <c10/hip/HIPCachingAllocator.h>
#include <c10/hip/HIPStream.h>

#include <cstdlib>
#include <mutex>

#include "omt_torch.h"

namespace omt {

// ------------------------------------------------------------------------------------------------------------------
// allocator (libomt_hip.so's caching allocator)
// ------------------------------------------------------------------------------------------------------------------

static void free_dev(void* p) {
  if (p) omt_free(p);
}

struct Allocator final : c10::Allocator {
  c10::DataPtr allocate(size_t n) override {
    void* p = nullptr;
    if (n) {
      void* s = cur_stream();
      int st = omt_malloc_on(&p, n, s);
      if (st == OMT_OOM) {
        omt_empty_cache();  // synchronizes the device: parked and pending blocks of every stream become free
        st = omt_malloc_on(&p, n, s);
      }
      TORCH_CHECK_WITH(OutOfMemoryError, st != OMT_OOM, "omarchy-mac-torch: out of device memory: ", omt_last_error());
      TORCH_CHECK(st == OMT_OK, "omarchy-mac-torch: allocation failed: ", omt_last_error());
    }
    return {p, p, &free_dev, c10::Device(kDev, 0)};
  }
  void copy_data(void* dst, const void* src, std::size_t count) const override {
    TORCH_CHECK(omt_memcpy(dst, src, count, 2, cur_stream()) == OMT_OK, "omarchy-mac-torch: copy failed: ",
                omt_last_error());
  }
  c10::DeleterFnPtr raw_deleter() const override { return &free_dev; }
};
static Allocator g_alloc;
REGISTER_ALLOCATOR(c10::DeviceType::PrivateUse1, &g_alloc);

c10::Allocator* allocator() { return &g_alloc; }

void* cur_stream() { return (void*)c10::hip::getCurrentHIPStream().stream(); }

Tensor empty_dev(IntArrayRef size, at::ScalarType dt) {
  return at::detail::empty_generic(size, &g_alloc, c10::DispatchKeySet(c10::DispatchKey::PrivateUse1), dt,
                                   std::nullopt);
}

Tensor empty_dev_cl(IntArrayRef size, at::ScalarType dt) {
  return at::detail::empty_generic(size, &g_alloc, c10::DispatchKeySet(c10::DispatchKey::PrivateUse1), dt,
                                   at::MemoryFormat::ChannelsLast);
}

Tensor workspace(size_t bytes) { return bytes ? empty_dev({(int64_t)bytes}, at::kByte) : Tensor(); }

// ------------------------------------------------------------------------------------------------------------------
// aliases between the device and torch's HIP device
// ------------------------------------------------------------------------------------------------------------------

// The alias storage is resizable through torch's HIP allocator: an op that grows an output argument (out= forms,
// resize_) reallocates the alias, and the fallback then adopts the new storage into the device tensor.
// torch's HIP context (its caching allocator above all) initializes lazily, on the first HIP tensor a program creates;
// a program that only uses this device reaches torch's HIP kernels through the aliases below, so they initialize it.
static void init_torch_hip() {
  static std::once_flag once;
  std::call_once(once, []() { at::globalContext().lazyInitDevice(c10::DeviceType::CUDA); });
}

Tensor hip_alias(const Tensor& t) {
  if (!is_dev(t)) return t;
  init_torch_hip();
  const c10::Storage& s = t.storage();
  c10::DataPtr dp(const_cast<void*>(s.data()), c10::Device(c10::DeviceType::CUDA, 0));  // non-owning
  c10::Storage hs(c10::Storage::use_byte_size_t(), s.nbytes(), std::move(dp),
                  c10::GetAllocator(c10::DeviceType::CUDA), true);
  auto impl = c10::make_intrusive<c10::TensorImpl>(std::move(hs), c10::DispatchKeySet(c10::DispatchKey::CUDA),
                                                   t.dtype());
  impl->set_sizes_and_strides(t.sizes(), t.strides(), t.storage_offset());
  return Tensor(std::move(impl));
}

namespace {
struct Keep {
  c10::Storage s;
};
void release_keep(void* ctx) { delete static_cast<Keep*>(ctx); }
}  // namespace

Tensor dev_from_hip(const Tensor& h) {
  const c10::Storage& s = h.storage();
  auto* keep = new Keep{s};
  c10::DataPtr dp(const_cast<void*>(s.data()), keep, &release_keep, c10::Device(kDev, 0));
  c10::Storage ds(c10::Storage::use_byte_size_t(), s.nbytes(), std::move(dp), &g_alloc, false);
  auto impl = c10::make_intrusive<c10::TensorImpl>(std::move(ds), c10::DispatchKeySet(c10::DispatchKey::PrivateUse1),
                                                   h.dtype());
  impl->set_sizes_and_strides(h.sizes(), h.strides(), h.storage_offset());
  return Tensor(std::move(impl));
}

// a device tensor sharing orig's storage with another geometry (a view produced by a delegated op)
static Tensor dev_view(const Tensor& orig, const Tensor& h) {
  auto impl = c10::make_intrusive<c10::TensorImpl>(c10::Storage(orig.storage()), orig.key_set(), h.dtype());
  impl->set_sizes_and_strides(h.sizes(), h.strides(), h.storage_offset());
  return Tensor(std::move(impl));
}

// ------------------------------------------------------------------------------------------------------------------
// status, locking, accounting
// ------------------------------------------------------------------------------------------------------------------

void check(int st, const char* what) {
  if (st == OMT_OK) return;
  if (st == OMT_UNSUPPORTED) throw NotCovered(omt_last_error());
  TORCH_CHECK_WITH(OutOfMemoryError, st != OMT_OOM, what, ": out of device memory: ", omt_last_error());
  TORCH_CHECK(false, what, ": ", omt_last_error());
}

std::recursive_mutex& big_lock() {
  static std::recursive_mutex m;
  return m;
}
std::map<std::string, int64_t>& fallback_counts() {
  static std::map<std::string, int64_t> m;
  return m;
}
std::map<std::string, int64_t>& delegated_counts() {
  static std::map<std::string, int64_t> m;
  return m;
}
static bool env_on(const char* name) {
  const char* e = std::getenv(name);
  return e && e[0] == '1';
}
static bool g_strict = env_on("OMARCHY_MAC_TORCH_STRICT");
static bool g_debug = env_on("OMARCHY_MAC_TORCH_DEBUG");
static bool g_count_delegated = false;
static std::string g_forced_sync_error;  // set by tests only: the next debug_point reports it as a device error
bool strict_mode() { return g_strict; }
void set_strict_mode(bool on) { g_strict = on; }
bool debug_mode() { return g_debug; }
void set_debug_mode(bool on) { g_debug = on; }
void set_count_delegated(bool on) { g_count_delegated = on; }
void force_next_sync_error(const std::string& msg) { g_forced_sync_error = msg; }
void debug_point(const std::string& op) {
  std::string err;
  if (!g_forced_sync_error.empty()) {
    err.swap(g_forced_sync_error);
  } else if (omt_stream_sync(cur_stream()) != OMT_OK) {
    err = omt_last_error();
  }
  TORCH_CHECK(err.empty(), "omarchy-mac-torch (debug): asynchronous error after ", op, ": ", err);
}
void left_hot_path(const std::string& op, const char* why) {
  TORCH_CHECK(!strict_mode(), "omarchy-mac-torch (strict): ", op, " is not covered by the HIP kernels: ", why);
  std::string key = op;
  ((key += " (") += why) += ')';
  ++fallback_counts()[key];
}

// ------------------------------------------------------------------------------------------------------------------
// boxed fallback: run the op on torch's HIP kernels over aliases of the device tensors
// ------------------------------------------------------------------------------------------------------------------

namespace {
struct AliasPair {
  Tensor orig, alias;
};

c10::IValue to_hip_ivalue(const c10::IValue& v, std::vector<AliasPair>& pairs) {
  auto conv = [&](const Tensor& t) -> Tensor {
    if (!is_dev(t)) return t;
    Tensor a = hip_alias(t);
    pairs.push_back({t, a});
    return a;
  };
  if (v.isTensor()) return c10::IValue(conv(v.toTensor()));
  if (v.isTensorList()) {
    c10::List<Tensor> out;
    for (const Tensor& t : v.toTensorList()) out.push_back(conv(t));
    return c10::IValue(out);
  }
  if (v.isOptionalTensorList()) {
    c10::List<std::optional<Tensor>> out;
    for (const std::optional<Tensor>& t : v.toOptionalTensorList())
      out.push_back(t && t->defined() ? std::optional<Tensor>(conv(*t)) : t);
    return c10::IValue(out);
  }
  if (v.isDevice() && v.toDevice().type() == kDev) return c10::IValue(c10::Device(c10::DeviceType::CUDA, 0));
  return v;
}

Tensor back_to_dev(const Tensor& h, const std::vector<AliasPair>& pairs) {
  if (!h.defined() || h.device().type() != c10::DeviceType::CUDA) return h;
  const void* base = h.storage().data();
  for (const AliasPair& p : pairs) {
    if (p.alias.storage().data() != base || !base) continue;
    if (h.sizes().equals(p.orig.sizes()) && h.strides().equals(p.orig.strides()) &&
        h.storage_offset() == p.orig.storage_offset() && h.dtype() == p.orig.dtype())
      return p.orig;          // in-place / out= result: the argument itself
    return dev_view(p.orig, h);  // a view of an argument
  }
  return dev_from_hip(h);
}

void run_on_hip(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
  const auto& schema = op.schema();
  const size_t nargs = schema.arguments().size();
  std::vector<AliasPair> pairs;
  const size_t first = stack->size() - nargs;
  for (size_t i = first; i < stack->size(); ++i) (*stack)[i] = to_hip_ivalue((*stack)[i], pairs);
  op.callBoxed(stack);
  // arguments whose storage or geometry the op changed (out= outputs that were resized, in-place metadata ops)
  for (const AliasPair& p : pairs) {
    c10::TensorImpl* impl = p.orig.unsafeGetTensorImpl();
    if (p.alias.storage().data() != p.orig.storage().data() || p.alias.storage().nbytes() != p.orig.storage().nbytes()) {
      impl->set_storage_keep_dtype(dev_from_hip(p.alias).storage());
      impl->set_sizes_and_strides(p.alias.sizes(), p.alias.strides(), p.alias.storage_offset());
    } else if (!p.alias.sizes().equals(p.orig.sizes()) || !p.alias.strides().equals(p.orig.strides()) ||
               p.alias.storage_offset() != p.orig.storage_offset()) {
      impl->set_sizes_and_strides(p.alias.sizes(), p.alias.strides(), p.alias.storage_offset());
    }
  }
  const size_t nret = schema.returns().size();
  for (size_t i = stack->size() - nret; i < stack->size(); ++i) {
    c10::IValue& v = (*stack)[i];
    if (v.isTensor()) {
      v = c10::IValue(back_to_dev(v.toTensor(), pairs));
    } else if (v.isTensorList()) {
      c10::List<Tensor> out;
      for (const Tensor& t : v.toTensorList()) out.push_back(back_to_dev(t, pairs));
      v = c10::IValue(out);
    }
  }
}
}  // namespace

void hip_fallback(const c10::OperatorHandle& op, torch::jit::Stack* stack) {
  if (g_count_delegated) {
    OMT_LOCK;
    const auto& s = op.schema();
    delegated_counts()[s.name().substr(6) + (s.overload_name().empty() ? "" : "." + s.overload_name())]++;
  }
  run_on_hip(op, stack);
}
void hip_fallback_quiet(const c10::OperatorHandle& op, torch::jit::Stack* stack) { run_on_hip(op, stack); }

// ------------------------------------------------------------------------------------------------------------------
// memory / copy ops
// ------------------------------------------------------------------------------------------------------------------

static Tensor empty_memory_format(IntArrayRef size, std::optional<at::ScalarType> dtype, std::optional<at::Layout>,
                                  std::optional<at::Device>, std::optional<bool>, std::optional<at::MemoryFormat> mf) {
  return at::detail::empty_generic(size, &g_alloc, c10::DispatchKeySet(c10::DispatchKey::PrivateUse1),
                                   dtype.value_or(c10::get_default_dtype_as_scalartype()), mf);
}
static Tensor empty_strided(IntArrayRef size, IntArrayRef stride, std::optional<at::ScalarType> dtype,
                            std::optional<at::Layout>, std::optional<at::Device>, std::optional<bool>) {
  return at::detail::empty_strided_generic(size, stride, &g_alloc, c10::DispatchKeySet(c10::DispatchKey::PrivateUse1),
                                           dtype.value_or(c10::get_default_dtype_as_scalartype()));
}

// copy self -> dst (host <-> device, device <-> device, any dtype, strides and broadcast): torch's HIP copy kernel
// over aliases. A device-to-device copy between two memory orders (a layout conversion, e.g. .contiguous() of a
// channels_last tensor) is counted with the delegated ops when they are counted, under its sizes.
static Tensor copy_from(const Tensor& self, const Tensor& dst, bool non_blocking) {
  if (g_count_delegated && is_dev(self) && is_dev(dst) && self.sizes().equals(dst.sizes()) &&
      !self.strides().equals(dst.strides())) {
    OMT_LOCK;
    delegated_counts()["copy_ (layout conversion) " + c10::str(self.sizes())]++;
  }
  Tensor d = hip_alias(dst);
  d.copy_(hip_alias(self), non_blocking);
  return dst;
}

// grows the storage on the device (copying the live bytes) when the new shape needs more
static const Tensor& resize_dev_(const Tensor& self, IntArrayRef size, std::optional<at::MemoryFormat> mf) {
  auto* impl = self.unsafeGetTensorImpl();
  int64_t numel = 1;
  for (int64_t s : size) numel *= s;
  const size_t need = (size_t)(self.storage_offset() + numel) * self.itemsize();
  c10::StorageImpl* st = impl->storage().unsafeGetStorageImpl();
  if (need > st->nbytes()) {
    TORCH_CHECK(st->resizable(), "omarchy-mac-torch: trying to resize storage that is not resizable");
    c10::DataPtr nd = g_alloc.allocate(need);
    if (st->nbytes() && st->data())
      TORCH_CHECK(omt_memcpy(nd.get(), st->data(), st->nbytes(), 2, cur_stream()) == OMT_OK, omt_last_error());
    st->set_data_ptr_noswap(std::move(nd));
    st->set_nbytes(need);
  }
  impl->set_sizes_contiguous(size);
  if (mf && *mf != at::MemoryFormat::Preserve) impl->empty_tensor_restride(*mf);
  return self;
}
static Tensor copy_from_and_resize(const Tensor& self, const Tensor& dst) {
  resize_dev_(dst, self.sizes(), std::nullopt);
  return copy_from(self, dst, false);
}
static at::Scalar local_scalar(const Tensor& self) { return hip_alias(self).item(); }
static Tensor& set_storage(Tensor& self, c10::Storage src, int64_t off, IntArrayRef size, IntArrayRef stride) {
  return at::native::set_storage_cpu_(self, src, off, size, stride);  // metadata only
}

// ------------------------------------------------------------------------------------------------------------------
// device guard: one device, torch's current HIP stream, HIP events
// ------------------------------------------------------------------------------------------------------------------

// The device's streams are torch's HIP streams under another device type: a device Stream carries the HIP stream's
// id, and making it current makes that HIP stream current. The autograd engine records the forward's stream and makes
// it current on its backward thread, so backward kernels follow the forward's stream (a capturing one included).
static c10::Stream as_dev_stream(const c10::hip::HIPStream& h) {
  return c10::Stream(c10::Stream::UNSAFE, c10::Device(kDev, 0), h.id());
}
static c10::hip::HIPStream as_hip_stream(const c10::Stream& s) {
  return c10::hip::HIPStream::unpack3(s.id(), 0, c10::DeviceType::HIP);
}

// The block behind `dp` is not reused before the work queued on `hs` so far has completed. Storage adopted from
// torch's HIP allocator (results of delegated ops) is that allocator's to track.
static void record_on_stream(const c10::DataPtr& dp, const c10::hip::HIPStream& hs) {
  if (!dp.get()) return;
  if (dp.get_deleter() == &release_keep) {
    const auto* keep = static_cast<const Keep*>(dp.get_context());
    c10::hip::HIPCachingAllocator::recordStream(keep->s.data_ptr(), hs);
    return;
  }
  TORCH_CHECK(omt_record_stream(dp.get(), hs.stream()) == OMT_OK, "omarchy-mac-torch: ", omt_last_error());
}

// aten::record_stream for device tensors; the stream may be one of this device's or the torch HIP stream it wraps.
static void record_stream_dev(at::Tensor& self, c10::Stream s) {
  const c10::hip::HIPStream hs = s.device_type() == kDev ? as_hip_stream(s)
                                                         : c10::hip::HIPStream(c10::hip::HIPStream::UNCHECKED, s);
  record_on_stream(self.storage().data_ptr(), hs);
}

struct Guard final : c10::impl::DeviceGuardImplInterface {
  c10::DeviceType type() const override { return kDev; }
  c10::Device exchangeDevice(c10::Device) const override { return {kDev, 0}; }
  c10::Device getDevice() const override { return {kDev, 0}; }
  void setDevice(c10::Device) const override {}
  void uncheckedSetDevice(c10::Device) const noexcept override {}
  c10::Stream getStream(c10::Device) const noexcept override { return as_dev_stream(c10::hip::getCurrentHIPStream(0)); }
  c10::Stream getDefaultStream(c10::Device) const override { return as_dev_stream(c10::hip::getDefaultHIPStream(0)); }
  // streams keep the default priority whatever is asked (mixed priorities are avoided on these GPUs)
  c10::Stream getNewStream(c10::Device, int) const override { return as_dev_stream(c10::hip::getStreamFromPool(false, 0)); }
  c10::Stream exchangeStream(c10::Stream s) const noexcept override {
    const c10::Stream prev = as_dev_stream(c10::hip::getCurrentHIPStream(0));
    c10::hip::setCurrentHIPStream(as_hip_stream(s));
    return prev;
  }
  c10::DeviceIndex deviceCount() const noexcept override { return 1; }
  void record(void** event, const c10::Stream& s, const c10::DeviceIndex, const c10::EventFlag) const override {
    if (!*event) TORCH_CHECK(omt_event_create(event) == OMT_OK, omt_last_error());
    TORCH_CHECK(omt_event_record(*event, as_hip_stream(s).stream()) == OMT_OK, omt_last_error());
  }
  void block(void* event, const c10::Stream& s) const override {
    if (event) TORCH_CHECK(hipStreamWaitEvent(as_hip_stream(s).stream(), (hipEvent_t)event, 0) == hipSuccess);
  }
  bool queryEvent(void* event) const override { return !event || omt_event_query(event) == 1; }
  void destroyEvent(void* event, const c10::DeviceIndex) const noexcept override {
    if (event) omt_event_destroy(event);
  }
  void synchronizeEvent(void* event) const override {
    if (event) TORCH_CHECK(omt_event_sync(event) == OMT_OK, omt_last_error());
  }
  bool queryStream(const c10::Stream& s) const override {
    return hipStreamQuery(as_hip_stream(s).stream()) == hipSuccess;
  }
  void synchronizeStream(const c10::Stream& s) const override {
    TORCH_CHECK(omt_stream_sync(as_hip_stream(s).stream()) == OMT_OK, omt_last_error());
  }
  void synchronizeDevice(const c10::DeviceIndex) const override {
    TORCH_CHECK(hipDeviceSynchronize() == hipSuccess, "hipDeviceSynchronize failed");
  }
  double elapsedTime(void* start, void* end, const c10::DeviceIndex) const override {
    float ms = 0.f;
    TORCH_CHECK(omt_event_elapsed_ms(start, end, &ms) == OMT_OK, omt_last_error());
    return ms;
  }
  // autograd's cross-stream uses of a gradient (and Tensor.record_stream, below): see record_on_stream
  void recordDataPtrOnStream(const c10::DataPtr& dp, const c10::Stream& s) const override {
    record_on_stream(dp, as_hip_stream(s));
  }
};
C10_REGISTER_GUARD_IMPL(PrivateUse1, Guard);

// ------------------------------------------------------------------------------------------------------------------
// hooks: random numbers come from torch's HIP generator (the delegated RNG ops run on torch's HIP kernels)
// ------------------------------------------------------------------------------------------------------------------

struct Hooks final : at::PrivateUse1HooksInterface {
  bool isBuilt() const override { return true; }
  bool isAvailable() const override { return true; }
  bool hasPrimaryContext(c10::DeviceIndex) const override { return true; }
  c10::DeviceIndex deviceCount() const override { return 1; }
  c10::DeviceIndex getCurrentDevice() const override { return 0; }
  void setCurrentDevice(c10::DeviceIndex) const override {}
  c10::DeviceIndex exchangeDevice(c10::DeviceIndex) const override { return 0; }
  c10::DeviceIndex maybeExchangeDevice(c10::DeviceIndex) const override { return 0; }
  const at::Generator& getDefaultGenerator(c10::DeviceIndex) const override {
    return at::cuda::detail::getDefaultCUDAGenerator(0);
  }
  at::Generator getNewGenerator(c10::DeviceIndex) const override { return at::cuda::detail::createCUDAGenerator(0); }
};
static struct HooksRegistrar {
  HooksRegistrar() {
    static Hooks hooks;
    at::RegisterPrivateUse1HooksInterface(&hooks);
  }
} g_hooks_registrar;

// ------------------------------------------------------------------------------------------------------------------
// registration
// ------------------------------------------------------------------------------------------------------------------

TORCH_LIBRARY_IMPL(_, PrivateUse1, m) { m.fallback(torch::CppFunction::makeFromBoxedFunction<&hip_fallback>()); }

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("empty.memory_format", &empty_memory_format);
  m.impl("empty_strided", &empty_strided);
  m.impl("_copy_from", &copy_from);
  m.impl("_copy_from_and_resize", &copy_from_and_resize);
  m.impl("_local_scalar_dense", &local_scalar);
  m.impl("set_.source_Storage_storage_offset", &set_storage);
  m.impl("set_.source_Storage", &at::native::set_);
  m.impl("resize_", &resize_dev_);
  m.impl("record_stream", &record_stream_dev);
  // views share the device storage: metadata-only kernels, never delegated
  m.impl("view", &at::native::view);
  m.impl("_unsafe_view", &at::native::_unsafe_view);
  m.impl("as_strided", &at::native::as_strided_tensorimpl);
  m.impl("_reshape_alias", &at::native::_reshape_alias);
  m.impl("unfold", &at::native::unfold);
  m.impl("view_as_real", &at::native::view_as_real);
  m.impl("view_as_complex", &at::native::view_as_complex);
  // torch's _foreach_* ops carry a CompositeExplicitAutograd kernel that loops over the list one tensor at a time;
  // for this key it would win over the boxed fallback and cost one delegated op per tensor. Registered here, each list
  // op goes to torch's HIP kernels whole (one multi-tensor launch). _foreach_add_.Scalar has a kernel of this library
  // (pointwise.cpp: step counts and batch counters), registered there instead.
  for (const c10::OperatorName& op : c10::Dispatcher::singleton().getAllOpNames()) {
    if (op.name.rfind("aten::_foreach_", 0) != 0) continue;
    if (op.name == "aten::_foreach_add_" && op.overload_name == "Scalar") continue;
    const std::string name = op.name.substr(6) + (op.overload_name.empty() ? "" : "." + op.overload_name);
    m.impl(name.c_str(), torch::CppFunction::makeFromBoxedFunction<&hip_fallback>());
  }
}

// ------------------------------------------------------------------------------------------------------------------
// geometry helpers
// ------------------------------------------------------------------------------------------------------------------

omt_conv_geo conv_geo(int64_t n, int64_t ci, int64_t co, int64_t ih, int64_t iw, int64_t ks, int64_t stride,
                      int64_t pad) {
  omt_conv_geo g;
  omt_conv_geo_init(&g, n, ci, co, ih, iw, ks, stride, pad);
  return g;
}

int64_t pool_out(int64_t size, int64_t k, int64_t s, int64_t p, int64_t d, bool ceil) {
  int64_t num = size + 2 * p - d * (k - 1) - 1 + (ceil ? s - 1 : 0);
  int64_t out = num / s + 1;  // num >= 0 for every valid pooling geometry
  if (ceil && (out - 1) * s >= size + p) --out;
  return out;
}

}  // namespace omt
