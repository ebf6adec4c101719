// Conv plan tuning for the device's operators and stack plans (reference: set_tuning / tune_dump / tune_load /
// tuned_plans and the autotune-on-first-use of conv_plan, csrc/conv.cpp:45-60, 116-155, 239-283). The plan cache
// itself lives in libomt_hip.so (omt_conv_get_plan / omt_conv_set_plan / omt_conv_autotune).
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <atomic>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "omt_torch.h"

namespace omt {

static std::atomic<bool> g_tune{false};
static std::atomic<int> g_num_tiles{0};

void tune_conv(int dir, const omt_conv_geo& g) {
  if (!g_tune.load(std::memory_order_relaxed)) return;
  omt_conv_plan p;
  int cached = 0;
  if (omt_conv_get_plan(dir, &g, &p, &cached) != OMT_OK || cached) return;
  // OMT_UNSUPPORTED while a graph is being captured: the call keeps the model's plan
  const int st = omt_conv_autotune(dir, &g, g_num_tiles.load(), cur_stream(), nullptr);
  if (st != OMT_OK && st != OMT_UNSUPPORTED) check(st, "conv autotune");
}

void tune_conv_bwd(const omt_conv_geo& g) {
  if (!g_tune.load(std::memory_order_relaxed)) return;
  omt_conv_plan p;
  int dc = 0, wc = 0;
  if (omt_conv_get_plan(OMT_DIR_DGRAD, &g, &p, &dc) != OMT_OK || omt_conv_get_plan(OMT_DIR_WGRAD, &g, &p, &wc) != OMT_OK ||
      (dc && wc))
    return;
  const int st = omt_conv_autotune_bwd(&g, g_num_tiles.load(), cur_stream(), nullptr, nullptr);
  if (st != OMT_OK && st != OMT_UNSUPPORTED) check(st, "conv autotune");
}

static std::string key_string(int dir, const omt_conv_geo& g) {
  std::ostringstream o;
  o << dir << ',' << g.n << ',' << g.ci << ',' << g.co << ',' << g.ih << ',' << g.iw << ',' << g.oh << ',' << g.ow
    << ',' << g.ks << ',' << g.stride << ',' << g.pad;
  return o.str();
}

void bind_tuning(pybind11::module_& m) {
  m.def("set_tuning", [](bool on, int num_tiles) {
    g_tune = on;
    g_num_tiles = num_tiles;
  });
  m.def("tuning", []() { return g_tune.load(); });
  // "dir,n,ci,co,ih,iw,oh,ow,ks,stride,pad" -> (tile, slices)
  m.def("tune_dump", []() {
    std::map<std::string, std::pair<int, int>> r;
    const int n = omt_conv_plan_count();
    for (int i = 0; i < n; ++i) {
      int dir = 0;
      omt_conv_geo g;
      omt_conv_plan p;
      if (omt_conv_plan_entry(i, &dir, &g, &p) == OMT_OK) r[key_string(dir, g)] = {p.tile, p.slices};
    }
    return r;
  });
  // loads entries of that form; malformed keys, geometries the kernels do not cover and out-of-range plans are
  // skipped. Returns the number loaded.
  m.def("tune_load", [](const std::map<std::string, std::pair<int, int>>& entries) {
    int loaded = 0;
    for (const auto& e : entries) {
      std::vector<int64_t> k;
      std::stringstream ss(e.first);
      std::string item;
      bool ok = true;
      while (std::getline(ss, item, ',')) {
        try {
          size_t used = 0;
          k.push_back(std::stoll(item, &used));
          ok = ok && used == item.size();
        } catch (...) {
          ok = false;
        }
      }
      if (!ok || k.size() != 11) continue;
      omt_conv_geo g{k[1], k[2], k[3], k[4], k[5], k[6], k[7], k[8], k[9], k[10]};
      omt_conv_plan p{e.second.first, e.second.second};
      if (omt_conv_set_plan((int)k[0], &g, &p) == OMT_OK) ++loaded;
    }
    return loaded;
  });
  m.def("tuned_plans", []() {
    std::map<std::string, std::string> r;
    static const char* names[] = {"fwd", "dgrad", "wgrad", "fwd_nhwc", "dgrad_nhwc", "wgrad_nhwc"};
    const int n = omt_conv_plan_count();
    for (int i = 0; i < n; ++i) {
      int dir = 0;
      omt_conv_geo g;
      omt_conv_plan p;
      if (omt_conv_plan_entry(i, &dir, &g, &p) != OMT_OK) continue;
      r[key_string(dir, g)] = std::string(names[dir]) + " tile " + std::to_string(p.tile) + " x" +
                              std::to_string(p.slices) + " slices";
    }
    return r;
  });
  m.def("clear_plans", []() { omt_conv_clear_plans(); });
}

}  // namespace omt
