// Fused Conv / BatchNorm+ReLU / pool stacks: an nn.Sequential compiled once per (input shape, train, input_grad) into
// fixed forward and backward step lists over plan-owned device buffers, driven from Python by an autograd Function
// (stacks.py). Every step is one libomt_hip.so call with its pointers and workspace fixed at build time, so running
// a plan is a straight sequence of kernel launches with no dispatcher, autograd or allocation work per layer.
// Reference counterpart: csrc/plans.cpp:9-362 (Plan, build_plan, run_steps, plan_forward, plan_backward, make_plan).
//
// Layer kinds (omarchy_mac_torch/stacks.py:41-94): conv (dense, odd ks, stride 1, "same" padding, no bias),
// dw (depthwise 3/5/7), bn (BatchNorm2d with its ReLU fused), pool (2x2 max), apool (2x2 avg), gap (global avg).
// Eval plans fold a BatchNorm+ReLU into the next conv's input loader: fold policy 0 never, 1 only 1x1 convs
// (the default), 2 every conv and depthwise conv (csrc/plans.cpp:162-170).
//
// Graph replay: after kPlanWarmup runs step by step, each step list is captured once as a HIP graph and every later
// run is one graph launch (the reference's plans replay their recorded dispatch list the same way,
// csrc/plans.cpp:280-294). The graph reads and writes plan-owned buffers and the module's tensors, which stay put
// (reassigning one drops the plans, stacks.py). The backward's parameter gradients then go to plan-owned buffers as
// well: a run finds them still held by someone (a gradient kept from the last backward) runs step by step into new
// tensors instead. Inside a capture of the caller's own the steps run one by one (into that capture).
// OMARCHY_MAC_TORCH_PLAN_GRAPHS=0 keeps every plan step by step.
#include <hip/hip_runtime_api.h>
#include <pybind11/functional.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>
#include <torch/extension.h>

#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>

#include "omt_torch.h"

namespace omt {

static int g_fold = 1;
constexpr int kPlanWarmup = 1;  // step-by-step runs of a step list before it is captured
static bool g_plan_graphs = [] {
  const char* e = std::getenv("OMARCHY_MAC_TORCH_PLAN_GRAPHS");
  return !(e && std::strcmp(e, "0") == 0);
}();

struct PlanLayer {
  std::string kind;
  int64_t ci = 0, co = 0, ks = 0;
  double momentum = 0.1;
};

struct Run {
  std::vector<Tensor> grads;  // per parameter, filled by the backward steps
};

using Steps = std::vector<std::function<void(Run&, void*)>>;

// One step list's graph: its step-by-step runs so far, and once captured, the executable graph.
struct StepGraph {
  int runs = 0;
  bool off = false;  // a step could not be captured: step by step from now on
  hipGraphExec_t exec = nullptr;
};

struct Plan {
  bool train = false, input_grad = false, busy = false;
  std::vector<int64_t> in_shape, out_shape;
  std::vector<Tensor> params, rms, rvs;  // the module's tensors (updated in place by optimizers)
  std::vector<Tensor> bufs;              // plan-owned activations, statistics, indices, workspaces
  Tensor xin, xout, gout, gin;
  Steps fwd, bwd;
  std::vector<std::vector<int64_t>> grad_shapes;  // per parameter
  StepGraph fgraph, bgraph;
  std::vector<Tensor> gbufs;  // parameter gradients of a backward that replays its graph
  Plan() = default;
  Plan(const Plan&) = delete;
  Plan& operator=(const Plan&) = delete;
  ~Plan() {
    // a launch still running keeps its resources until it completes; the buffers go back to the caching allocator,
    // whose later users on this stream run after it
    for (StepGraph* g : {&fgraph, &bgraph})
      if (g->exec) (void)hipGraphExecDestroy(g->exec);
  }
};

static bool stream_capturing(void* s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing((hipStream_t)s, &st) != hipSuccess || st != hipStreamCaptureStatusNone;
}

// Captures `steps` run with `run` on a private stream as a HIP graph; nullptr if a step cannot be captured (a call
// that synchronizes or allocates fails under capture, and its error ends the capture).
static hipGraphExec_t capture_steps(Steps& steps, Run& run) {
  hipStream_t cs = nullptr;
  if (hipStreamCreateWithFlags(&cs, hipStreamNonBlocking) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  bool ok = hipStreamBeginCapture(cs, hipStreamCaptureModeThreadLocal) == hipSuccess;
  if (ok) {
    try {
      for (auto& step : steps) step(run, cs);
    } catch (const std::exception&) {
      ok = false;
    }
    ok = hipStreamEndCapture(cs, &graph) == hipSuccess && ok && graph;
  }
  if (ok) ok = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
  if (graph) (void)hipGraphDestroy(graph);
  (void)hipStreamDestroy(cs);
  (void)hipGetLastError();
  return ok ? exec : nullptr;
}

// Whether this run of the list replays (capturing it first when its warm-up is over).
static bool replays(StepGraph& sg, Steps& steps, Run& run, void* s) {
  if (!g_plan_graphs || sg.off || stream_capturing(s)) return false;
  if (!sg.exec && sg.runs >= kPlanWarmup) {
    sg.exec = capture_steps(steps, run);
    sg.off = sg.exec == nullptr;
  }
  return sg.exec != nullptr;
}

static void run_list(StepGraph& sg, Steps& steps, Run& run, void* s, bool graph) {
  ++sg.runs;
  if (graph) {
    const hipError_t e = hipGraphLaunch(sg.exec, (hipStream_t)s);
    TORCH_CHECK(e == hipSuccess, "omarchy-mac-torch plan: graph launch failed: ", hipGetErrorString(e));
    return;
  }
  for (auto& step : steps) step(run, s);
}

static Tensor own(Plan& p, IntArrayRef shape, at::ScalarType dt = at::kFloat) {
  p.bufs.push_back(empty_dev(shape, dt));
  return p.bufs.back();
}
static Tensor own_ws(Plan& p, size_t bytes) {
  if (!bytes) return Tensor();
  return own(p, {(int64_t)bytes}, at::kByte);
}

namespace {
struct BackRec {
  std::string kind;
  Tensor x, y, sm, si, idx;
  int param = -1;
  int64_t n = 0, c = 0, co = 0, h = 0, w = 0, ks = 0;
};
}  // namespace

static std::shared_ptr<Plan> build_plan(const std::vector<PlanLayer>& layers, std::vector<int64_t> shape, bool train,
                                        bool input_grad, std::vector<Tensor> params, std::vector<Tensor> rms,
                                        std::vector<Tensor> rvs) {
  OMT_LOCK;
  cover(shape.size() == 4, "4-D input");
  for (auto& t : params) cover(is_dev(t) && f32(t) && t.is_contiguous(), "plan parameters must be contiguous float32 device tensors");
  for (auto& t : rms) cover(is_dev(t) && f32(t) && t.is_contiguous(), "running statistics on the device");
  for (auto& t : rvs) cover(is_dev(t) && f32(t) && t.is_contiguous(), "running statistics on the device");
  auto P = std::make_shared<Plan>();
  Plan& p = *P;
  p.train = train;
  p.input_grad = input_grad;
  p.params = params;
  p.rms = rms;
  p.rvs = rvs;
  p.in_shape = shape;
  for (auto& t : params) p.grad_shapes.push_back(t.sizes().vec());
  int64_t n = shape[0], c = shape[1], h = shape[2], w = shape[3];
  p.xin = own(p, {n, c, h, w});
  Tensor cur = p.xin;
  std::vector<BackRec> recs;
  int pi = 0, bi = 0;
  struct Pending {
    bool on = false;
    int bn = -1, gamma = -1;
  } pend;
  for (size_t li = 0; li < layers.size(); ++li) {
    const PlanLayer& L = layers[li];
    if (L.kind == "conv" || L.kind == "dw") {
      const bool dw = L.kind == "dw";
      const int64_t co = dw ? c : L.co, ks = L.ks;
      cover(L.ci == c && pi < (int)params.size(), "layer channels");
      Tensor out = own(p, {n, co, h, w});
      omt_conv_geo g = conv_geo(n, c, co, h, w, ks, 1, ks / 2);
      cover(g.oh == h && g.ow == w, "'same' convolution");
      Tensor wt = params[pi];
      const float *bm = nullptr, *bv = nullptr, *bg = nullptr, *bb = nullptr;
      if (pend.on) {  // eval: previous BatchNorm + ReLU applied by this conv's loader
        bm = fp(rms[pend.bn]);
        bv = fp(rvs[pend.bn]);
        bg = fp(params[pend.gamma]);
        bb = fp(params[pend.gamma + 1]);
        pend.on = false;
      }
      if (dw) {
        p.fwd.push_back([g, x = cur, wt, out, bm, bv, bg, bb](Run&, void* s) {
          check(omt_dw_fwd(&g, fp(x), fp(wt), nullptr, bm, bv, bg, bb, 1e-5f, fpm(out), s), "plan: depthwise conv");
        });
      } else {
        tune_conv(OMT_DIR_FWD, g);
        Tensor ws = own_ws(p, omt_conv_fwd_workspace(&g));
        p.fwd.push_back([g, x = cur, wt, out, bm, bv, bg, bb, ws](Run&, void* s) {
          check(omt_conv_fwd(&g, fp(x), fp(wt), nullptr, 0, bm, bv, bg, bb, 1e-5f, fpm(out), wsptr(ws), wsbytes(ws), s),
                "plan: conv");
        });
      }
      BackRec r;
      r.kind = L.kind;
      r.x = cur;
      r.param = pi;
      r.n = n;
      r.c = c;
      r.co = co;
      r.h = h;
      r.w = w;
      r.ks = ks;
      recs.push_back(r);
      cur = out;
      c = co;
      ++pi;
    } else if (L.kind == "bn") {
      cover(L.ci == c && pi + 1 < (int)params.size() && bi < (int)rms.size(), "layer channels");
      bool next_conv = false;
      if (li + 1 < layers.size() && g_fold > 0) {
        const PlanLayer& N = layers[li + 1];
        next_conv = g_fold >= 2 ? (N.kind == "conv" || N.kind == "dw") : (N.kind == "conv" && N.ks == 1);
      }
      if (!train && next_conv) {  // folded into the consumer's loader
        pend.on = true;
        pend.bn = bi;
        pend.gamma = pi;
        ++bi;
        pi += 2;
        continue;
      }
      const int64_t hw = h * w;
      Tensor y = own(p, {n, c, h, w});
      Tensor gamma = params[pi], beta = params[pi + 1], rm = rms[bi], rv = rvs[bi];
      BackRec r;
      // training: a following 2x2 max pool runs inside the BatchNorm's apply pass (one launch fewer, y not re-read)
      const bool fuse_pool = train && li + 1 < layers.size() && layers[li + 1].kind == "pool" && h >= 2 && w >= 2;
      Tensor pout, pidx;
      if (fuse_pool) {
        pout = own(p, {n, c, h / 2, w / 2});
        pidx = own(p, {n, c, h / 2, w / 2}, at::kLong);
      }
      if (train) {
        Tensor sm = own(p, {c}), si = own(p, {c});
        Tensor ws = own_ws(p, omt_bn_train_workspace(n, c, hw));
        const double mom = L.momentum;
        const int64_t h0 = h, w0 = w;
        p.fwd.push_back([=](Run&, void* s) {
          float* rmp = rm.mutable_data_ptr<float>();
          float* rvp = rv.mutable_data_ptr<float>();
          if (fuse_pool)
            check(omt_bn_train_fwd_pool(n, c, h0, w0, fp(cur), fp(gamma), fp(beta), rmp, rvp, mom, 1e-5, 1, fpm(y),
                                        fpm(sm), fpm(si), rmp, rvp, 2, 2, 2, 2, 0, 0, fpm(pout),
                                        pidx.mutable_data_ptr<int64_t>(), wsptr(ws), wsbytes(ws), s),
                  "plan: batch norm + max pool");
          else
            check(omt_bn_train_fwd(n, c, hw, fp(cur), fp(gamma), fp(beta), rmp, rvp, mom, 1e-5, 1, fpm(y), fpm(sm),
                                   fpm(si), rmp, rvp, wsptr(ws), wsbytes(ws), s),
                  "plan: batch norm");
        });
        r.sm = sm;
        r.si = si;
      } else {
        p.fwd.push_back([=](Run&, void* s) {
          check(omt_bn_eval_fwd(n, c, hw, fp(cur), fp(gamma), fp(beta), fp(rm), fp(rv), 1e-5, 1, fpm(y), s),
                "plan: batch norm (eval)");
        });
      }
      r.kind = "bn";
      r.x = cur;
      r.y = y;
      r.param = pi;
      r.n = n;
      r.c = c;
      r.h = h;
      r.w = w;
      recs.push_back(r);
      cur = y;
      ++bi;
      pi += 2;
      if (fuse_pool) {  // the pool layer's record (its backward step is unchanged); the layer itself is done
        BackRec pr;
        pr.kind = "pool";
        pr.idx = pidx;
        pr.n = n;
        pr.c = c;
        pr.h = h;
        pr.w = w;
        recs.push_back(pr);
        cur = pout;
        h /= 2;
        w /= 2;
        ++li;
      }
    } else if (L.kind == "pool" || L.kind == "apool") {
      cover(h >= 2 && w >= 2, "2x2 pool over an image smaller than 2x2");
      const int64_t oh = h / 2, ow = w / 2;
      Tensor out = own(p, {n, c, oh, ow});
      BackRec r;
      r.kind = L.kind;
      if (L.kind == "pool") {
        Tensor idx = own(p, {n, c, oh, ow}, at::kLong);
        p.fwd.push_back([=](Run&, void* s) {
          check(omt_maxpool_fwd(n * c, h, w, oh, ow, 2, 2, 2, 2, 0, 0, 1, 1, fp(cur), fpm(out),
                                idx.mutable_data_ptr<int64_t>(), s),
                "plan: max pool");
        });
        r.idx = idx;
      } else {
        p.fwd.push_back([=](Run&, void* s) {
          check(omt_avgpool_fwd(n * c, h, w, oh, ow, 2, 2, 2, 2, 0, 0, 1, 0, fp(cur), fpm(out), s), "plan: avg pool");
        });
      }
      r.n = n;
      r.c = c;
      r.h = h;
      r.w = w;
      recs.push_back(r);
      cur = out;
      h = oh;
      w = ow;
    } else if (L.kind == "gap") {
      Tensor out = own(p, {n, c, 1, 1});
      p.fwd.push_back([=](Run&, void* s) {
        check(omt_adapool_fwd(n * c, h, w, 1, 1, fp(cur), fpm(out), s), "plan: global average pool");
      });
      BackRec r;
      r.kind = "gap";
      r.n = n;
      r.c = c;
      r.h = h;
      r.w = w;
      recs.push_back(r);
      cur = out;
      h = w = 1;
    } else {
      throw NotCovered("unknown layer kind " + L.kind);
    }
  }
  cover(!pend.on, "a folded BatchNorm needs a following convolution");
  p.xout = cur;
  p.out_shape = {n, c, h, w};
  if (!train) return P;

  // ---- backward, in reverse ----
  p.gout = own(p, p.out_shape);
  Tensor g = p.gout;
  for (int ri = (int)recs.size() - 1; ri >= 0; --ri) {
    const BackRec r = recs[ri];
    const bool first = ri == 0;
    const int64_t n_ = r.n, c_ = r.c, h_ = r.h, w_ = r.w;
    if (r.kind == "pool" || r.kind == "apool" || r.kind == "gap") {
      Tensor gx = own(p, {n_, c_, h_, w_});
      if (r.kind == "pool") {
        Tensor idx = r.idx;
        p.bwd.push_back([=](Run&, void* s) {
          check(omt_maxpool_bwd(n_ * c_, h_, w_, h_ / 2, w_ / 2, 2, 2, 2, 2, 0, 0, 1, 1, fp(g), idx.data_ptr<int64_t>(),
                                fpm(gx), s),
                "plan: max pool backward");
        });
      } else if (r.kind == "apool") {
        p.bwd.push_back([=](Run&, void* s) {
          check(omt_avgpool_bwd(n_ * c_, h_, w_, h_ / 2, w_ / 2, 2, 2, 2, 2, 0, 0, 1, 0, fp(g), fpm(gx), s),
                "plan: avg pool backward");
        });
      } else {
        p.bwd.push_back([=](Run&, void* s) {
          check(omt_adapool_bwd(n_ * c_, h_, w_, 1, 1, fp(g), fpm(gx), s), "plan: global average pool backward");
        });
      }
      g = gx;
    } else if (r.kind == "bn") {
      Tensor gx = own(p, {n_, c_, h_, w_});
      Tensor ws = own_ws(p, omt_bn_bwd_workspace(n_, c_, h_ * w_));
      Tensor x = r.x, y = r.y, sm = r.sm, si = r.si, gamma = params[r.param];
      const int gi = r.param;
      p.bwd.push_back([=](Run& run, void* s) {
        check(omt_bn_bwd(n_, c_, h_ * w_, fp(g), fp(x), fp(y), fp(sm), fp(si), fp(gamma), fpm(gx), fpm(run.grads[gi]),
                         fpm(run.grads[gi + 1]), wsptr(ws), wsbytes(ws), s),
              "plan: batch norm backward");
      });
      g = gx;
    } else {  // conv / dw
      const bool dw = r.kind == "dw";
      omt_conv_geo geo = conv_geo(n_, c_, r.co, h_, w_, r.ks, 1, r.ks / 2);
      Tensor x = r.x, wt = params[r.param];
      const int gi = r.param;
      if (!dw && (!first || input_grad)) {
        // dense with both gradients: one call, the two GEMMs share a launch when their plans allow it
        tune_conv_bwd(geo);
        Tensor gx = own(p, {n_, c_, h_, w_});
        Tensor bws = own_ws(p, omt_conv_bwd_workspace(&geo));
        p.bwd.push_back([=](Run& run, void* s) {
          check(omt_conv_bwd(&geo, fp(x), fp(g), fp(wt), fpm(gx), fpm(run.grads[gi]), wsptr(bws), wsbytes(bws), s),
                "plan: input and weight gradients");
        });
        g = gx;
        continue;
      }
      if (!dw) tune_conv(OMT_DIR_WGRAD, geo);
      Tensor wws = own_ws(p, dw ? omt_dw_wgrad_workspace(&geo) : omt_conv_wgrad_workspace(&geo));
      p.bwd.push_back([=](Run& run, void* s) {
        if (dw)
          check(omt_dw_wgrad(&geo, fp(x), fp(g), fpm(run.grads[gi]), wsptr(wws), wsbytes(wws), s),
                "plan: depthwise weight gradient");
        else
          check(omt_conv_wgrad(&geo, fp(x), fp(g), fpm(run.grads[gi]), wsptr(wws), wsbytes(wws), s),
                "plan: weight gradient");
      });
      if (!first || input_grad) {
        Tensor gx = own(p, {n_, c_, h_, w_});
        if (!dw) tune_conv(OMT_DIR_DGRAD, geo);
        Tensor dws = dw ? Tensor() : own_ws(p, omt_conv_dgrad_workspace(&geo));
        p.bwd.push_back([=](Run&, void* s) {
          if (dw)
            check(omt_dw_dgrad(&geo, fp(g), fp(wt), fpm(gx), s), "plan: depthwise input gradient");
          else
            check(omt_conv_dgrad(&geo, fp(g), fp(wt), fpm(gx), wsptr(dws), wsbytes(dws), s), "plan: input gradient");
        });
        g = gx;
      }
    }
  }
  p.gin = g;
  return P;
}

static Tensor plan_forward(Plan& p, const Tensor& x) {
  OMT_LOCK;
  TORCH_CHECK(is_dev(x) && f32(x) && x.sizes().vec() == p.in_shape,
              "omarchy-mac-torch plan: expected a float32 device input of shape ", p.in_shape);
  void* s = cur_stream();
  Tensor xc = x.is_contiguous() ? x : x.contiguous();
  check(omt_memcpy(fpm(p.xin), fp(xc), (size_t)xc.numel() * 4, 2, s), "plan: input copy");
  Run run;
  run_list(p.fgraph, p.fwd, run, s, replays(p.fgraph, p.fwd, run, s));
  Tensor out = empty_dev(p.out_shape);
  check(omt_memcpy(fpm(out), fp(p.xout), (size_t)out.numel() * 4, 2, s), "plan: output copy");
  if (debug_mode()) debug_point("plan.forward");
  return out;
}

static std::pair<std::optional<Tensor>, std::vector<Tensor>> plan_backward(Plan& p, const Tensor& g) {
  OMT_LOCK;
  TORCH_CHECK(p.train, "omarchy-mac-torch plan: backward of an eval plan");
  TORCH_CHECK(is_dev(g) && f32(g) && g.sizes().vec() == p.out_shape, "omarchy-mac-torch plan: bad gradient");
  void* s = cur_stream();
  Tensor gc = g.is_contiguous() ? g : g.contiguous();
  check(omt_memcpy(fpm(p.gout), fp(gc), (size_t)gc.numel() * 4, 2, s), "plan: gradient copy");
  Run run;
  // the graph writes the gradients to the plan's buffers: only when nobody holds them from the last backward
  bool free = g_plan_graphs;
  for (const Tensor& t : p.gbufs) free = free && t.use_count() == 1;
  if (free && p.gbufs.empty() && !p.bgraph.off && p.bgraph.runs >= kPlanWarmup)
    for (auto& shape : p.grad_shapes) p.gbufs.push_back(empty_dev(shape));
  bool graph = false;
  if (free && !p.gbufs.empty()) {
    run.grads = p.gbufs;
    graph = replays(p.bgraph, p.bwd, run, s);
    if (!graph) run.grads.clear();
  }
  if (!graph)
    for (auto& shape : p.grad_shapes) run.grads.push_back(empty_dev(shape));
  run_list(p.bgraph, p.bwd, run, s, graph);
  std::optional<Tensor> gx;
  if (p.input_grad) {
    Tensor t = empty_dev(p.in_shape);
    check(omt_memcpy(fpm(t), fp(p.gin), (size_t)t.numel() * 4, 2, s), "plan: input gradient copy");
    gx = t;
  }
  if (debug_mode()) debug_point("plan.backward");
  return {gx, run.grads};
}

void bind_plans(pybind11::module_& m) {
  namespace py = pybind11;
  py::class_<Plan, std::shared_ptr<Plan>>(m, "Plan")
      .def_readwrite("busy", &Plan::busy)
      .def_readonly("out_shape", &Plan::out_shape)
      .def("num_steps", [](const Plan& p) { return py::make_tuple(p.fwd.size(), p.bwd.size()); })
      // whether the forward and backward step lists replay captured graphs
      .def("graphed", [](const Plan& p) { return py::make_tuple(p.fgraph.exec != nullptr, p.bgraph.exec != nullptr); })
      .def("forward", [](Plan& p, const Tensor& x) { return plan_forward(p, x); })
      .def("backward", [](Plan& p, const Tensor& g) {
        auto r = plan_backward(p, g);
        return py::make_tuple(r.first ? py::cast(*r.first) : py::none(), r.second);
      });
  m.def("make_plan", [](std::vector<std::tuple<std::string, int64_t, int64_t, int64_t, double>> layers,
                        std::vector<int64_t> shape, bool train, bool input_grad, std::vector<Tensor> params,
                        std::vector<Tensor> rms, std::vector<Tensor> rvs) {
    std::vector<PlanLayer> L;
    for (auto& t : layers) {
      PlanLayer l;
      l.kind = std::get<0>(t);
      l.ci = std::get<1>(t);
      l.co = std::get<2>(t);
      l.ks = std::get<3>(t);
      l.momentum = std::get<4>(t);
      L.push_back(l);
    }
    try {
      return build_plan(L, shape, train, input_grad, params, rms, rvs);
    } catch (const NotCovered& e) {
      throw std::runtime_error(std::string("omarchy-mac-torch: cannot build a fused stack: ") + e.what());
    }
  });
  m.def("set_fold", [](int f) { g_fold = f; });
  // turns graph replay of the plans' step lists on or off (plans already captured stop replaying when off); returns
  // the previous setting
  m.def("set_plan_graphs", [](bool on) {
    const bool prev = g_plan_graphs;
    g_plan_graphs = on;
    return prev;
  });
  m.def("get_fold", []() { return g_fold; });
}

}  // namespace omt
