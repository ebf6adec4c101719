// Python bindings (omarchy_mac_torch._native). Reference counterpart: csrc/module.cpp:15-63.
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>
#include <torch/extension.h>

#include "omt_torch.h"

namespace omt {
void bind_plans(pybind11::module_& m);
void bind_tuning(pybind11::module_& m);
void bind_replay(pybind11::module_& m);
}

PYBIND11_MODULE(_native, m) {
  using namespace omt;
  m.def("sync", []() {
    TORCH_CHECK(omt_stream_sync(cur_stream()) == OMT_OK, "omarchy-mac-torch: ", omt_last_error());
  });
  m.def("empty_cache", []() {
    OMT_LOCK;
    TORCH_CHECK(omt_empty_cache() == OMT_OK, "omarchy-mac-torch: ", omt_last_error());
  });
  m.def("memory_allocated", []() { return (int64_t)omt_memory_allocated(); });
  m.def("memory_reserved", []() { return (int64_t)omt_memory_reserved(); });
  m.def("set_memory_limit", [](int64_t bytes) { omt_set_memory_limit((size_t)std::max<int64_t>(bytes, 0)); });
  m.def("fallback_counts", []() {
    OMT_LOCK;
    return fallback_counts();
  });
  m.def("reset_fallbacks", []() {
    OMT_LOCK;
    fallback_counts().clear();
  });
  m.def("delegated_counts", []() {
    OMT_LOCK;
    return delegated_counts();
  });
  m.def("count_delegated", [](bool on) {
    OMT_LOCK;
    set_count_delegated(on);
    if (!on) delegated_counts().clear();
  });
  m.def("graph_pool_create", []() { return omt_graph_pool_create(); });
  m.def("graph_pool_begin", [](int id) {
    TORCH_CHECK(omt_graph_pool_begin(id) == OMT_OK, "omarchy-mac-torch: ", omt_last_error());
  });
  m.def("graph_pool_end", []() { omt_graph_pool_end(); });
  m.def("graph_pool_release", [](int id) {
    TORCH_CHECK(omt_graph_pool_release(id) == OMT_OK, "omarchy-mac-torch: ", omt_last_error());
  });
  m.def("set_debug", [](bool on) { set_debug_mode(on); });
  m.def("strict", []() { return strict_mode(); });
  m.def("set_strict", [](bool on) {
    OMT_LOCK;
    set_strict_mode(on);
  });
  m.def("debug", []() { return debug_mode(); });
  m.def("force_next_sync_error", [](const std::string& msg) {
    OMT_LOCK;
    force_next_sync_error(msg);
  });
  // per-kernel launch counts and timings, as the reference's kernel_counts / kernel_times / debug_time_kernels
  // (csrc/module.cpp:30-33): {kernel name: launches} and {kernel name: ms}, each optionally reset after reading
  auto kernel_stats = [](int what, bool reset) {
    std::map<std::string, double> out;
    const int n = omt_kernel_stat_count();
    for (int i = 0; i < n; ++i) {
      const char* name = nullptr;
      int64_t launches = 0;
      double ms = 0;
      if (omt_kernel_stat_entry(i, &name, &launches, &ms) != OMT_OK) break;
      if (what == OMT_KSTAT_LAUNCHES ? launches > 0 : ms > 0) out[name] = what == OMT_KSTAT_LAUNCHES ? launches : ms;
    }
    if (reset) omt_kernel_stats_reset(what);
    return out;
  };
  m.def("kernel_counts", [kernel_stats](bool reset) {
    std::map<std::string, int64_t> out;
    for (const auto& [k, v] : kernel_stats(OMT_KSTAT_LAUNCHES, reset)) out[k] = (int64_t)v;
    return out;
  }, pybind11::arg("reset") = false);
  m.def("kernel_times", [kernel_stats](bool reset) { return kernel_stats(OMT_KSTAT_TIMES, reset); },
        pybind11::arg("reset") = false);
  m.def("debug_time_kernels", [](bool on) { omt_set_kernel_timing(on ? 1 : 0); });
  m.def("abi_version", []() { return omt_abi_version(); });
  m.def("hip_runtime_version", []() { return omt_hip_runtime_version(); });
  m.attr("built_with_torch") = TORCH_VERSION;
  bind_plans(m);
  bind_tuning(m);
  bind_replay(m);
}
