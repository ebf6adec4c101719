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

// ---- plan construction: a fusion pass over the layer list, then one emitter per fused stage ----------------------
//
// fuse_stages groups the layers into stages (what runs as one library call): an eval BatchNorm + ReLU whose consumer
// can apply it in its input loader becomes part of that convolution's stage; a training BatchNorm + ReLU followed by a
// 2x2 max pool is one stage (the pool inside the BatchNorm's apply pass). The emitters then allocate each stage's
// buffers, append its forward steps and push onto a tape a closure that appends its backward steps; the tape runs in
// reverse, each closure taking the gradient of the stage's output and leaving the gradient of its input.

enum class StageOp { Conv, Depthwise, BatchNorm, BatchNormPool, MaxPool, AvgPool, GlobalPool };

struct Stage {
  StageOp op;
  int layer = 0;           // the stage's (first) layer
  int loader_bn = -1;      // eval: the BatchNorm layer the convolution applies in its input loader, or -1
};

// Whether an eval BatchNorm + ReLU may be applied by `consumer`'s input loader under the fold policy (0 never, 1 1x1
// convolutions only, 2 every convolution and depthwise convolution).
static bool loader_can_fold(const PlanLayer& consumer, int policy) {
  if (policy <= 0) return false;
  if (consumer.kind == "conv") return policy >= 2 || consumer.ks == 1;
  return policy >= 2 && consumer.kind == "dw";
}

static std::vector<Stage> fuse_stages(const std::vector<PlanLayer>& layers, bool train, int policy) {
  std::vector<Stage> out;
  const int nl = (int)layers.size();
  for (int li = 0; li < nl; ++li) {
    const std::string& k = layers[li].kind;
    const bool has_next = li + 1 < nl;
    if (k == "bn") {
      if (!train && has_next && loader_can_fold(layers[li + 1], policy)) {
        out.push_back({layers[li + 1].kind == "dw" ? StageOp::Depthwise : StageOp::Conv, li + 1, li});
        ++li;  // the consumer is this stage
      } else if (train && has_next && layers[li + 1].kind == "pool") {
        out.push_back({StageOp::BatchNormPool, li});
        ++li;
      } else {
        out.push_back({StageOp::BatchNorm, li});
      }
    } else if (k == "conv" || k == "dw") {
      out.push_back({k == "dw" ? StageOp::Depthwise : StageOp::Conv, li});
    } else if (k == "pool" || k == "apool") {
      out.push_back({k == "pool" ? StageOp::MaxPool : StageOp::AvgPool, li});
    } else if (k == "gap") {
      out.push_back({StageOp::GlobalPool, li});
    } else {
      throw NotCovered("unknown layer kind " + k);
    }
  }
  return out;
}

// Walks the stages, tracking the activation's shape and the next parameter / running-statistics slots.
struct PlanBuilder {
  Plan& p;
  const std::vector<PlanLayer>& layers;
  Tensor cur;                // the current activation
  int64_t n, c, h, w;        // its shape
  int pi = 0, bi = 0;        // next parameter, next running-statistics pair
  // each stage's backward emitter: (the gradient of its output -> the gradient of its input, and whether it is the
  // network's first stage)
  std::vector<std::function<void(Tensor&, bool)>> tape;

  const float* param_ptr(int i) const { return fp(p.params[i]); }

  void conv(const Stage& st) {
    const PlanLayer& L = layers[st.layer];
    const bool dw = st.op == StageOp::Depthwise;
    // an eval BatchNorm applied in this convolution's loader consumes its gamma, beta and running statistics first
    const float *bm = nullptr, *bv = nullptr, *bg = nullptr, *bb = nullptr;
    if (st.loader_bn >= 0) {
      cover(layers[st.loader_bn].ci == c && pi + 1 < (int)p.params.size() && bi < (int)p.rms.size(), "layer channels");
      bg = param_ptr(pi);
      bb = param_ptr(pi + 1);
      bm = fp(p.rms[bi]);
      bv = fp(p.rvs[bi]);
      pi += 2;
      ++bi;
    }
    const int64_t co = dw ? c : L.co, ks = L.ks;
    cover(L.ci == c && pi < (int)p.params.size(), "layer channels");
    const omt_conv_geo g = conv_geo(n, c, co, h, w, ks, 1, ks / 2);
    cover(g.oh == h && g.ow == w, "'same' convolution");
    const int wi = pi++;
    const Tensor x = cur, wt = p.params[wi], y = own(p, {n, co, h, w});
    if (dw) {
      p.fwd.push_back([g, x, wt, y, bm, bv, bg, bb](Run&, void* s) {
        check(omt_dw_fwd(&g, fp(x), fp(wt), nullptr, bm, bv, bg, bb, 1e-5f, fpm(y), s), "plan: depthwise conv");
      });
    } else {
      tune_conv(OMT_DIR_FWD, g);
      const Tensor ws = own_ws(p, omt_conv_fwd_workspace(&g));
      p.fwd.push_back([g, x, wt, y, bm, bv, bg, bb, ws](Run&, void* s) {
        check(omt_conv_fwd(&g, fp(x), fp(wt), nullptr, 0, bm, bv, bg, bb, 1e-5f, fpm(y), wsptr(ws), wsbytes(ws), s),
              "plan: conv");
      });
    }
    Plan& P = p;
    tape.push_back([&P, g, x, wt, wi, dw](Tensor& gy, bool first) {
      const bool gx_needed = !first || P.input_grad;
      const Tensor go = gy;
      if (!dw && gx_needed) {  // both gradients in one call: the two GEMMs share a launch when their plans allow it
        tune_conv_bwd(g);
        const Tensor gx = own(P, {g.n, g.ci, g.ih, g.iw}), ws = own_ws(P, omt_conv_bwd_workspace(&g));
        P.bwd.push_back([g, x, go, wt, gx, wi, ws](Run& run, void* s) {
          check(omt_conv_bwd(&g, fp(x), fp(go), fp(wt), fpm(gx), fpm(run.grads[wi]), wsptr(ws), wsbytes(ws), s),
                "plan: input and weight gradients");
        });
        gy = gx;
        return;
      }
      if (!dw) tune_conv(OMT_DIR_WGRAD, g);
      const Tensor wws = own_ws(P, dw ? omt_dw_wgrad_workspace(&g) : omt_conv_wgrad_workspace(&g));
      P.bwd.push_back([g, x, go, wi, wws, dw](Run& run, void* s) {
        if (dw)
          check(omt_dw_wgrad(&g, fp(x), fp(go), fpm(run.grads[wi]), wsptr(wws), wsbytes(wws), s),
                "plan: depthwise weight gradient");
        else
          check(omt_conv_wgrad(&g, fp(x), fp(go), fpm(run.grads[wi]), wsptr(wws), wsbytes(wws), s),
                "plan: weight gradient");
      });
      if (!gx_needed) return;
      if (!dw) tune_conv(OMT_DIR_DGRAD, g);
      const Tensor gx = own(P, {g.n, g.ci, g.ih, g.iw});
      const Tensor dws = dw ? Tensor() : own_ws(P, omt_conv_dgrad_workspace(&g));
      P.bwd.push_back([g, go, wt, gx, dws, dw](Run&, void* s) {
        if (dw)
          check(omt_dw_dgrad(&g, fp(go), fp(wt), fpm(gx), s), "plan: depthwise input gradient");
        else
          check(omt_conv_dgrad(&g, fp(go), fp(wt), fpm(gx), wsptr(dws), wsbytes(dws), s), "plan: input gradient");
      });
      gy = gx;
    });
    cur = y;
    c = co;
  }

  void batch_norm(const Stage& st) {
    const PlanLayer& L = layers[st.layer];
    cover(L.ci == c && pi + 1 < (int)p.params.size() && bi < (int)p.rms.size(), "layer channels");
    const bool pool = st.op == StageOp::BatchNormPool;
    if (pool) cover(h >= 2 && w >= 2, "2x2 pool over an image smaller than 2x2");
    const int gi = pi;
    pi += 2;
    const Tensor gamma = p.params[gi], beta = p.params[gi + 1], rm = p.rms[bi], rv = p.rvs[bi];
    ++bi;
    const int64_t n0 = n, c0 = c, h0 = h, w0 = w, hw = h * w;
    const Tensor x = cur, y = own(p, {n, c, h, w});
    if (!p.train) {
      p.fwd.push_back([=](Run&, void* s) {
        check(omt_bn_eval_fwd(n0, c0, hw, fp(x), fp(gamma), fp(beta), fp(rm), fp(rv), 1e-5, 1, fpm(y), s),
              "plan: batch norm (eval)");
      });
      cur = y;
      return;  // an eval plan has no backward
    }
    const Tensor sm = own(p, {c}), si = own(p, {c}), ws = own_ws(p, omt_bn_train_workspace(n, c, hw));
    const double mom = L.momentum;
    Tensor pooled, idx;
    if (pool) {
      pooled = own(p, {n, c, h / 2, w / 2});
      idx = own(p, {n, c, h / 2, w / 2}, at::kLong);
    }
    p.fwd.push_back([=](Run&, void* s) {
      float* rmp = rm.mutable_data_ptr<float>();
      float* rvp = rv.mutable_data_ptr<float>();
      if (pool)
        check(omt_bn_train_fwd_pool(n0, c0, h0, w0, fp(x), fp(gamma), fp(beta), rmp, rvp, mom, 1e-5, 1, fpm(y),
                                    fpm(sm), fpm(si), rmp, rvp, 2, 2, 2, 2, 0, 0, fpm(pooled),
                                    idx.mutable_data_ptr<int64_t>(), wsptr(ws), wsbytes(ws), s),
              "plan: batch norm + max pool");
      else
        check(omt_bn_train_fwd(n0, c0, hw, fp(x), fp(gamma), fp(beta), rmp, rvp, mom, 1e-5, 1, fpm(y), fpm(sm),
                               fpm(si), rmp, rvp, wsptr(ws), wsbytes(ws), s),
              "plan: batch norm");
    });
    Plan& P = p;
    tape.push_back([&P, n0, c0, h0, w0, x, y, sm, si, gamma, gi, pool, idx](Tensor& gy, bool) {
      if (pool) {  // the pool's gradient first: the fused forward's pooled output is this stage's output
        const Tensor go = gy, gp = own(P, {n0, c0, h0, w0});
        P.bwd.push_back([=](Run&, void* s) {
          check(omt_maxpool_bwd(n0 * c0, h0, w0, h0 / 2, w0 / 2, 2, 2, 2, 2, 0, 0, 1, 1, fp(go),
                                idx.data_ptr<int64_t>(), fpm(gp), s),
                "plan: max pool backward");
        });
        gy = gp;
      }
      const Tensor go = gy, gx = own(P, {n0, c0, h0, w0}), ws = own_ws(P, omt_bn_bwd_workspace(n0, c0, h0 * w0));
      P.bwd.push_back([=](Run& run, void* s) {
        check(omt_bn_bwd(n0, c0, h0 * w0, fp(go), fp(x), fp(y), fp(sm), fp(si), fp(gamma), fpm(gx),
                         fpm(run.grads[gi]), fpm(run.grads[gi + 1]), wsptr(ws), wsbytes(ws), s),
              "plan: batch norm backward");
      });
      gy = gx;
    });
    if (pool) {
      cur = pooled;
      h /= 2;
      w /= 2;
    } else {
      cur = y;
    }
  }

  void pool(const Stage& st) {
    const int64_t n0 = n, c0 = c, h0 = h, w0 = w;
    const Tensor x = cur;
    Plan& P = p;
    if (st.op == StageOp::GlobalPool) {
      const Tensor y = own(p, {n, c, 1, 1});
      p.fwd.push_back([=](Run&, void* s) {
        check(omt_adapool_fwd(n0 * c0, h0, w0, 1, 1, fp(x), fpm(y), s), "plan: global average pool");
      });
      tape.push_back([&P, n0, c0, h0, w0](Tensor& gy, bool) {
        const Tensor go = gy, gx = own(P, {n0, c0, h0, w0});
        P.bwd.push_back([=](Run&, void* s) {
          check(omt_adapool_bwd(n0 * c0, h0, w0, 1, 1, fp(go), fpm(gx), s), "plan: global average pool backward");
        });
        gy = gx;
      });
      cur = y;
      h = w = 1;
      return;
    }
    cover(h >= 2 && w >= 2, "2x2 pool over an image smaller than 2x2");
    const int64_t oh = h / 2, ow = w / 2;
    const Tensor y = own(p, {n, c, oh, ow});
    if (st.op == StageOp::MaxPool) {
      const Tensor idx = own(p, {n, c, oh, ow}, at::kLong);
      p.fwd.push_back([=](Run&, void* s) {
        check(omt_maxpool_fwd(n0 * c0, h0, w0, oh, ow, 2, 2, 2, 2, 0, 0, 1, 1, fp(x), fpm(y),
                              idx.mutable_data_ptr<int64_t>(), s),
              "plan: max pool");
      });
      tape.push_back([&P, n0, c0, h0, w0, idx](Tensor& gy, bool) {
        const Tensor go = gy, gx = own(P, {n0, c0, h0, w0});
        P.bwd.push_back([=](Run&, void* s) {
          check(omt_maxpool_bwd(n0 * c0, h0, w0, h0 / 2, w0 / 2, 2, 2, 2, 2, 0, 0, 1, 1, fp(go),
                                idx.data_ptr<int64_t>(), fpm(gx), s),
                "plan: max pool backward");
        });
        gy = gx;
      });
    } else {
      p.fwd.push_back([=](Run&, void* s) {
        check(omt_avgpool_fwd(n0 * c0, h0, w0, oh, ow, 2, 2, 2, 2, 0, 0, 1, 0, fp(x), fpm(y), s), "plan: avg pool");
      });
      tape.push_back([&P, n0, c0, h0, w0](Tensor& gy, bool) {
        const Tensor go = gy, gx = own(P, {n0, c0, h0, w0});
        P.bwd.push_back([=](Run&, void* s) {
          check(omt_avgpool_bwd(n0 * c0, h0, w0, h0 / 2, w0 / 2, 2, 2, 2, 2, 0, 0, 1, 0, fp(go), fpm(gx), s),
                "plan: avg pool backward");
        });
        gy = gx;
      });
    }
    cur = y;
    h = oh;
    w = ow;
  }
};

static std::shared_ptr<Plan> build_plan(const std::vector<PlanLayer>& layers, std::vector<int64_t> shape, bool train,
                                        bool input_grad, std::vector<Tensor> params, std::vector<Tensor> rms,
                                        std::vector<Tensor> rvs) {
  OMT_LOCK;
  cover(shape.size() == 4, "4-D input");
  for (auto& t : params) cover(is_dev(t) && f32(t) && t.is_contiguous(), "plan parameters must be contiguous float32 device tensors");
  for (auto& t : rms) cover(is_dev(t) && f32(t) && t.is_contiguous(), "running statistics on the device");
  for (auto& t : rvs) cover(is_dev(t) && f32(t) && t.is_contiguous(), "running statistics on the device");
  const std::vector<Stage> stages = fuse_stages(layers, train, g_fold);
  auto P = std::make_shared<Plan>();
  Plan& p = *P;
  p.train = train;
  p.input_grad = input_grad;
  p.params = std::move(params);
  p.rms = std::move(rms);
  p.rvs = std::move(rvs);
  p.in_shape = shape;
  for (auto& t : p.params) p.grad_shapes.push_back(t.sizes().vec());
  p.xin = own(p, {shape[0], shape[1], shape[2], shape[3]});
  PlanBuilder b{p, layers, p.xin, shape[0], shape[1], shape[2], shape[3]};
  for (const Stage& st : stages) {
    switch (st.op) {
      case StageOp::Conv:
      case StageOp::Depthwise: b.conv(st); break;
      case StageOp::BatchNorm:
      case StageOp::BatchNormPool: b.batch_norm(st); break;
      default: b.pool(st); break;
    }
  }
  p.xout = b.cur;
  p.out_shape = {b.n, b.c, b.h, b.w};
  if (!train) return P;
  p.gout = own(p, p.out_shape);
  Tensor g = p.gout;
  for (int i = (int)b.tape.size() - 1; i >= 0; --i) b.tape[i](g, i == 0);
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
