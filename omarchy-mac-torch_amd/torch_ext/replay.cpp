// Tensors that a replayed HIP graph rewrites in place, for the torch.compile backend's graph replay
// (omarchy_mac_torch/replay.py). No counterpart in the reference, whose compiled graphs run op by op
// (docs/roadmap.md:26-33 names graph capture and replay as the next step).
//
// A captured graph writes its outputs to the same memory on every replay. The caller hands out new tensor objects over
// that memory after each replay (aliases()), so that autograd and the user can own them (a saved activation, a
// parameter's .grad) without owning the graph's memory; and before the next replay it asks whether any of them is
// still alive (in_use()), in which case the replay would overwrite a value someone still reads, and the call runs
// eagerly instead. Both are counts on the storages' reference counts, done here in C++ because a step hands out
// dozens of tensors (Python-side set_() costs several microseconds each).
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>
#include <torch/extension.h>

#include <unordered_map>

#include "omt_torch.h"

namespace omt {

namespace {

class StaticTensors {
 public:
  explicit StaticTensors(const std::vector<Tensor>& ts) {
    for (const Tensor& t : ts) {
      TORCH_CHECK(t.defined(), "StaticTensors: undefined tensor");
      keep_.push_back({c10::Storage(t.storage()), t.key_set(), t.dtype(), t.sizes().vec(), t.strides().vec(),
                       t.storage_offset()});
    }
    for (const Entry& e : keep_) ++base_[e.storage.unsafeGetStorageImpl()];
  }

  // Takes the storages' present reference counts as the baseline: everything that holds them now (this object, the
  // caller's own bookkeeping) is not a use.
  void mark() {
    for (auto& [impl, n] : base_) n = c10::raw::intrusive_ptr::use_count(impl);
  }

  // One new tensor per kept tensor, over the same storage, sizes, strides and offset.
  std::vector<Tensor> aliases() const {
    std::vector<Tensor> out;
    out.reserve(keep_.size());
    for (const Entry& e : keep_) {
      auto impl = c10::make_intrusive<c10::TensorImpl>(c10::Storage(e.storage), e.keys, e.dtype);
      impl->set_sizes_and_strides(e.sizes, e.strides, e.offset);
      out.emplace_back(std::move(impl));
    }
    return out;
  }

  // True when one of the kept storages has more references than at the baseline (this object's own until mark()).
  bool in_use() const {
    for (const auto& [impl, n] : base_)
      if (c10::raw::intrusive_ptr::use_count(impl) > n) return true;
    return false;
  }

  size_t size() const { return keep_.size(); }

 private:
  struct Entry {
    c10::Storage storage;
    c10::DispatchKeySet keys;
    caffe2::TypeMeta dtype;
    std::vector<int64_t> sizes, strides;
    int64_t offset;
  };
  std::vector<Entry> keep_;
  std::unordered_map<c10::StorageImpl*, uint32_t> base_;  // baseline reference count, per storage
};

}  // namespace

void bind_replay(pybind11::module_& m) {
  namespace py = pybind11;
  // per tensor, the base address of its storage (0 for an undefined tensor)
  m.def("storage_ptrs", [](const std::vector<Tensor>& ts) {
    std::vector<int64_t> out;
    out.reserve(ts.size());
    for (const Tensor& t : ts) out.push_back(t.defined() ? (int64_t)(intptr_t)t.storage().data() : 0);
    return out;
  });
  // the indices i with expected[i] != 0 whose tensor's storage no longer starts at expected[i]: a replay's check
  // that the inputs it reads in place are where the capture found them
  m.def("moved_inputs", [](const std::vector<Tensor>& ts, const std::vector<int64_t>& expected) {
    TORCH_CHECK(ts.size() == expected.size(), "moved_inputs: ", ts.size(), " tensors, ", expected.size(), " addresses");
    std::vector<int64_t> out;
    for (size_t i = 0; i < ts.size(); ++i)
      if (expected[i] != 0 && (!ts[i].defined() || (int64_t)(intptr_t)ts[i].storage().data() != expected[i]))
        out.push_back((int64_t)i);
    return out;
  });
  py::class_<StaticTensors>(m, "StaticTensors")
      .def(py::init<const std::vector<Tensor>&>())
      .def("aliases", &StaticTensors::aliases)
      .def("in_use", &StaticTensors::in_use)
      .def("mark", &StaticTensors::mark)
      .def("__len__", &StaticTensors::size);
}

}  // namespace omt
