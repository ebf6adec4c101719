// Device kernels for the training steps' ops outside the convolution path, over libomt_hip.so's pointwise, reduction
// and loss entry points: residual add, ReLU / hardswish / hardsigmoid and their gradients, the squeeze-excite channel
// scale, plane means and sums (AdaptiveAvgPool2d(1) lowers to mean over the last two dims) and their gradients, a
// linear layer's bias gradient, log-softmax and the NLL loss. Reference counterparts: csrc/elementwise.cpp:702-817
// (registrations), csrc/reduce.cpp:128-202 (softmax, nll_loss); the scalar adds of the optimizers' step counts and
// BatchNorm's batch counters (the reference loops _foreach_ ops over its per-tensor kernels, csrc/device.cpp:220-225).
// The linear layers' matrix products are in linalg.cpp. Calls these kernels do not cover (other dtypes, broadcasts,
// layouts) run on torch's HIP kernels, like every op without a kernel here.
#include "omt_torch.h"

namespace omt {

namespace {

// contiguous NCHW float32 (the order-dependent ops: planes, rows, channel scales)
bool dense(const Tensor& t) { return is_dev(t) && f32(t) && t.is_contiguous(); }
bool same(const Tensor& a, const Tensor& b) { return dense(a) && dense(b) && a.sizes().equals(b.sizes()); }
// one dense block in NCHW or channels-last order (elementwise ops, which run over the memory in its own order)
bool flat(const Tensor& t) { return is_dev(t) && f32(t) && (t.is_contiguous() || is_cl(t)); }
Tensor empty_like_dev(const Tensor& t) { return is_cl(t) ? empty_dev_cl(t.sizes()) : empty_dev(t.sizes()); }
// both flat, one shape, one memory order
bool same_flat(const Tensor& a, const Tensor& b) {
  return flat(a) && flat(b) && a.sizes().equals(b.sizes()) && is_cl(a) == is_cl(b);
}
// one shape, 4-D, one operand NCHW and the other channels-last
bool mixed_flat(const Tensor& a, const Tensor& b) {
  return flat(a) && flat(b) && a.dim() == 4 && a.sizes().equals(b.sizes()) && is_cl(a) != is_cl(b);
}
// a 0-dim CPU tensor: a Python number the dispatcher wrapped, or a host scalar
bool host_scalar(const Tensor& t) { return t.defined() && t.dim() == 0 && t.device().is_cpu(); }

void pw(int op, const Tensor& a, const Tensor* b, float alpha, const Tensor& out) {
  check(omt_pointwise(op, out.numel(), a.defined() ? fp(a) : nullptr, b ? fp(*b) : nullptr, alpha, fpm(out),
                      cur_stream()),
        "pointwise");
}
Tensor unary(int op, const Tensor& x, float alpha = 0.f) {
  cover(flat(x), "contiguous float32");
  Tensor y = empty_like_dev(x);
  pw(op, x, nullptr, alpha, y);
  return y;
}
Tensor& unary_(int op, Tensor& x) {
  cover(flat(x), "contiguous float32");
  pw(op, x, nullptr, 0.f, x);
  return x;
}
// Operands in one memory order run over the memory as it is. An NCHW operand meeting a channels-last one (a
// channels-last model's global-average-pool gradient, broadcast over its planes, meeting the ReLU mask) runs the
// mixed-order kernel, its output channels-last, so the model stays channels-last without a conversion.
Tensor binary(int op, const Tensor& a, const Tensor& b, float alpha = 0.f) {
  if (mixed_flat(a, b)) {
    Tensor y = empty_dev_cl(a.sizes());
    check(omt_pointwise_layouts(op, a.size(0), a.size(1), a.size(2) * a.size(3), fp(a), is_cl(a) ? 1 : 0, fp(b),
                                is_cl(b) ? 1 : 0, alpha, fpm(y), 1, cur_stream()),
          "pointwise (mixed memory orders)");
    return y;
  }
  cover(same_flat(a, b), "contiguous float32 operands of one shape");
  Tensor y = empty_like_dev(a);
  pw(op, a, &b, alpha, y);
  return y;
}

// ---- pointwise ----

bool real(const at::Scalar& v) { return v.isFloatingPoint() || v.isIntegral(false); }

// t += v for contiguous int64 / float32 device tensors of at most OMT_FOREACH_MAX_NUMEL elements (counters, steps)
void add_small(at::TensorList ts, const at::Scalar& v) {
  cover(!ts.empty(), "non-empty list");
  const at::ScalarType dt = ts[0].scalar_type();
  cover((dt == at::kLong && v.isIntegral(false)) || (dt == at::kFloat && real(v)), "int64 or float32 tensors");
  std::vector<void*> ptrs;
  std::vector<int64_t> numels;
  for (const Tensor& t : ts) {
    cover(is_dev(t) && t.scalar_type() == dt && t.is_contiguous() && t.numel() <= OMT_FOREACH_MAX_NUMEL,
          "small contiguous device tensors of one dtype");
    ptrs.push_back(t.numel() ? t.data_ptr() : nullptr);
    numels.push_back(t.numel());
  }
  check(omt_foreach_add_scalar((int)ts.size(), ptrs.data(), numels.data(), dt == at::kLong ? OMT_DT_I64 : OMT_DT_F32,
                               dt == at::kLong ? v.toLong() : 0, dt == at::kFloat ? v.toFloat() : 0.f, cur_stream()),
        "add (scalar)");
}

Tensor add_t(const Tensor& a, const Tensor& b, const at::Scalar& alpha) {
  cover(real(alpha), "real alpha");
  if (host_scalar(b) && flat(a) && b.is_floating_point())  // a + alpha * b with b a number
    return unary(OMT_PW_ADD_SCALAR, a, (float)(alpha.toDouble() * b.item<double>()));
  return binary(OMT_PW_ADD, a, b, alpha.toFloat());
}
Tensor& add_t_(Tensor& a, const Tensor& b, const at::Scalar& alpha) {
  cover(real(alpha), "real alpha");
  if (host_scalar(b) && is_dev(a)) {  // a += alpha * b with b a number (BatchNorm's num_batches_tracked.add_(1))
    if (a.scalar_type() == at::kLong && alpha.isIntegral(false) && !b.is_floating_point()) {
      add_small({a}, b.item<int64_t>() * alpha.toLong());
      return a;
    }
    cover(flat(a), "contiguous float32");
    pw(OMT_PW_ADD_SCALAR, a, nullptr, (float)(alpha.toDouble() * b.item<double>()), a);
    return a;
  }
  if (mixed_flat(a, b)) {  // a += alpha * b with b in the other memory order (autograd's gradient accumulation)
    check(omt_pointwise_layouts(OMT_PW_ADD, a.size(0), a.size(1), a.size(2) * a.size(3), fp(a), is_cl(a) ? 1 : 0,
                                fp(b), is_cl(b) ? 1 : 0, alpha.toFloat(), fpm(a), is_cl(a) ? 1 : 0, cur_stream()),
          "add_ (mixed memory orders)");
    return a;
  }
  cover(same_flat(a, b), "contiguous float32, one shape");
  pw(OMT_PW_ADD, a, &b, alpha.toFloat(), a);
  return a;
}
Tensor& add_s_(Tensor& a, const at::Scalar& v, const at::Scalar& alpha) {
  cover(real(v) && real(alpha), "real operands");
  if (a.scalar_type() == at::kLong && v.isIntegral(false) && alpha.isIntegral(false)) {
    add_small({a}, v.toLong() * alpha.toLong());
    return a;
  }
  cover(flat(a), "contiguous float32");
  pw(OMT_PW_ADD_SCALAR, a, nullptr, (float)(v.toDouble() * alpha.toDouble()), a);
  return a;
}
// torch._foreach_add_(tensors, scalar): the optimizers' step counts, the compiled graph's merged batch counters
void foreach_add_s_(at::TensorList ts, const at::Scalar& v) { add_small(ts, v); }

// x [N, C, H, W] times s [N, C, 1, 1] (squeeze-excite, and the gradient of that product with respect to x)
bool channel_pair(const Tensor& big, const Tensor& s) {
  return dense(big) && dense(s) && big.dim() == 4 && s.dim() == 4 && s.size(0) == big.size(0) &&
         s.size(1) == big.size(1) && s.size(2) == 1 && s.size(3) == 1 && big.numel() > s.numel();
}
// x channels-last [N, C, H, W] times s [N, C, 1, 1]
bool channel_pair_cl(const Tensor& big, const Tensor& s) {
  return is_dev(big) && f32(big) && is_cl(big) && dense(s) && s.dim() == 4 && s.size(0) == big.size(0) &&
         s.size(1) == big.size(1) && s.size(2) == 1 && s.size(3) == 1;
}
Tensor mul_t(const Tensor& a, const Tensor& b) {
  if (host_scalar(b) && flat(a) && b.is_floating_point()) return unary(OMT_PW_SCALE, a, b.item<float>());
  const bool abl = channel_pair_cl(a, b), bal = channel_pair_cl(b, a);
  if (abl || bal) {
    const Tensor& big = abl ? a : b;
    const Tensor& s = abl ? b : a;
    Tensor y = empty_dev_cl(big.sizes());
    check(omt_channel_scale_nhwc(big.size(0), big.size(1), big.size(2) * big.size(3), fp(big), fp(s), fpm(y),
                                 cur_stream()),
          "mul (channel scale, channels last)");
    return y;
  }
  const bool ab = channel_pair(a, b), ba = channel_pair(b, a);
  if (ab || ba) {
    const Tensor& big = ab ? a : b;
    const Tensor& s = ab ? b : a;
    Tensor y = empty_dev(big.sizes());
    check(omt_channel_scale(big.size(0) * big.size(1), big.size(2) * big.size(3), fp(big), fp(s), fpm(y),
                            cur_stream()),
          "mul (channel scale)");
    return y;
  }
  return binary(OMT_PW_MUL, a, b);
}

// x / d with d a host scalar: x contiguous, or a per-plane value broadcast over H x W (strides (C, 1, 0, 0): the
// gradient of a plane mean, sum_backward's expand)
Tensor div_t(const Tensor& a, const Tensor& b) {
  cover(host_scalar(b) && (b.is_floating_point() || b.dtype() == at::kLong), "divisor on the host");
  const double d = b.item<double>();
  cover(d != 0.0, "non-zero divisor");
  const float inv = (float)(1.0 / d);
  if (flat(a)) return unary(OMT_PW_SCALE, a, inv);
  cover(is_dev(a) && f32(a) && a.dim() == 4 && a.stride(3) == 0 && a.stride(2) == 0 && a.stride(1) == 1 &&
            a.stride(0) == a.size(1),
        "contiguous, or an [N, C] tensor expanded over H x W");
  Tensor y = empty_dev(a.sizes());
  check(omt_plane_broadcast(a.size(0) * a.size(1), a.size(2) * a.size(3), fp(a), inv, fpm(y), cur_stream()),
        "div (plane broadcast)");
  return y;
}

Tensor relu_(const Tensor& x) { return unary(OMT_PW_RELU, x); }
Tensor& relu_ip(Tensor& x) { return unary_(OMT_PW_RELU, x); }
Tensor threshold_bwd(const Tensor& g, const Tensor& x, const at::Scalar& th) {
  cover(th.isFloatingPoint() || th.isIntegral(false), "real threshold");
  return binary(OMT_PW_THRESHOLD_BWD, g, x, th.toFloat());
}
Tensor hardswish_(const Tensor& x) { return unary(OMT_PW_HARDSWISH, x); }
Tensor& hardswish_ip(Tensor& x) { return unary_(OMT_PW_HARDSWISH, x); }
Tensor hardswish_bwd(const Tensor& g, const Tensor& x) { return binary(OMT_PW_HARDSWISH_BWD, g, x); }
Tensor hardsigmoid_(const Tensor& x) { return unary(OMT_PW_HARDSIGMOID, x); }
Tensor& hardsigmoid_ip(Tensor& x) { return unary_(OMT_PW_HARDSIGMOID, x); }
Tensor hardsigmoid_bwd(const Tensor& g, const Tensor& x) { return binary(OMT_PW_HARDSIGMOID_BWD, g, x); }
Tensor& fill_s(Tensor& x, const at::Scalar& v) {
  cover(flat(x) && (v.isFloatingPoint() || v.isIntegral(false)), "contiguous float32");
  pw(OMT_PW_FILL, Tensor(), nullptr, v.toFloat(), x);
  return x;
}

// any contiguous dtype: the bytes are zero (a fill kernel, not a memset node: safe inside a captured graph)
Tensor& zero_ip(Tensor& x) {
  cover(is_dev(x) && (x.is_contiguous() || is_cl(x)), "contiguous");
  check(omt_memset_zero(x.data_ptr(), (size_t)x.nbytes(), cur_stream()), "zero_");
  return x;
}

// ---- reductions ----

// The reduced dims of `dims` over a tensor of rank `nd`, sorted, or empty for "all" (not covered here).
std::vector<int64_t> reduced(at::OptionalIntArrayRef dims, int64_t nd) {
  std::vector<int64_t> r;
  if (!dims) return r;
  for (int64_t d : *dims) r.push_back(c10::maybe_wrap_dim(d, nd));
  std::sort(r.begin(), r.end());
  r.erase(std::unique(r.begin(), r.end()), r.end());
  return r;
}

// sum or mean over the last two dims of [N, C, H, W] (scale 1 or 1 / (H W)), or sum over dim 0 of [R, F]
Tensor plane_or_rows(const Tensor& x, at::OptionalIntArrayRef dims, bool keepdim, std::optional<at::ScalarType> dt,
                     bool mean) {
  cover((dense(x) || (is_dev(x) && f32(x) && is_cl(x))) && (!dt || *dt == at::kFloat), "contiguous float32");
  const std::vector<int64_t> r = reduced(dims, x.dim());
  if (is_cl(x)) {  // channels-last planes
    cover(r == std::vector<int64_t>{2, 3}, "sum / mean over the last two dims");
    const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
    cover(hw > 0 && n <= 65535, "non-empty planes, at most 65535 images");
    Tensor y = keepdim ? empty_dev({n, c, 1, 1}) : empty_dev({n, c});
    check(omt_plane_sum_nhwc(n, c, hw, fp(x), mean ? 1.f / (float)hw : 1.f, fpm(y), cur_stream()),
          "sum / mean (channels-last planes)");
    return y;
  }
  if (x.dim() == 4 && r == std::vector<int64_t>{2, 3}) {
    const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
    cover(hw > 0, "non-empty planes");
    Tensor y = keepdim ? empty_dev({n, c, 1, 1}) : empty_dev({n, c});
    check(omt_plane_sum(n * c, hw, fp(x), mean ? 1.f / (float)hw : 1.f, fpm(y), cur_stream()), "sum / mean (planes)");
    return y;
  }
  cover(!mean && x.dim() == 2 && r == std::vector<int64_t>{0}, "sum over the last two dims of 4-D or dim 0 of 2-D");
  const int64_t rows = x.size(0), cols = x.size(1);
  Tensor y = keepdim ? empty_dev({1, cols}) : empty_dev({cols});
  check(omt_bias_grad(rows, cols, 1, fp(x), fpm(y), cur_stream()), "sum (rows)");
  return y;
}
Tensor sum_dims(const Tensor& x, at::OptionalIntArrayRef dims, bool keepdim, std::optional<at::ScalarType> dt) {
  return plane_or_rows(x, dims, keepdim, dt, false);
}
Tensor mean_dims(const Tensor& x, at::OptionalIntArrayRef dims, bool keepdim, std::optional<at::ScalarType> dt) {
  return plane_or_rows(x, dims, keepdim, dt, true);
}

// ---- log-softmax and the NLL loss (F.cross_entropy decomposes into both) ----

Tensor log_softmax_(const Tensor& x, int64_t dim, bool half_to_float) {
  cover(dense(x) && !half_to_float && x.dim() >= 1 && c10::maybe_wrap_dim(dim, x.dim()) == x.dim() - 1 &&
            x.numel() > 0,
        "contiguous float32 over the last dim");
  const int64_t cols = x.size(-1);
  Tensor y = empty_dev(x.sizes());
  check(omt_log_softmax_fwd(x.numel() / cols, cols, fp(x), fpm(y), cur_stream()), "_log_softmax");
  return y;
}
Tensor log_softmax_bwd(const Tensor& g, const Tensor& y, int64_t dim, at::ScalarType input_dtype) {
  cover(same(g, y) && input_dtype == at::kFloat && y.dim() >= 1 && c10::maybe_wrap_dim(dim, y.dim()) == y.dim() - 1 &&
            y.numel() > 0,
        "contiguous float32 over the last dim");
  const int64_t cols = y.size(-1);
  Tensor gx = empty_dev(y.sizes());
  check(omt_log_softmax_bwd(y.numel() / cols, cols, fp(g), fp(y), fpm(gx), cur_stream()),
        "_log_softmax_backward_data");
  return gx;
}

bool targets_ok(const Tensor& x, const Tensor& t) {
  return dense(x) && x.dim() == 2 && x.size(0) > 0 && is_dev(t) && t.scalar_type() == at::kLong &&
         t.is_contiguous() && t.dim() == 1 && t.size(0) == x.size(0);
}
std::tuple<Tensor, Tensor> nll_fwd(const Tensor& x, const Tensor& t, const std::optional<Tensor>& w,
                                   int64_t reduction, int64_t ignore) {
  cover(targets_ok(x, t) && (!defined(w) || (dense(*w) && w->numel() == x.size(1))) && reduction >= 0 &&
            reduction <= 2,
        "(N, C) float32 log-probabilities and N int64 targets");
  Tensor out = reduction == 0 ? empty_dev({x.size(0)}) : empty_dev({});
  Tensor tw = empty_dev({});
  check(omt_nll_loss_fwd(x.size(0), x.size(1), fp(x), t.data_ptr<int64_t>(), defined(w) ? fp(*w) : nullptr, ignore,
                         (int)reduction, fpm(out), fpm(tw), cur_stream()),
        "nll_loss_forward");
  return {out, tw};
}
Tensor nll_bwd(const Tensor& g, const Tensor& x, const Tensor& t, const std::optional<Tensor>& w, int64_t reduction,
               int64_t ignore, const Tensor& tw) {
  cover(targets_ok(x, t) && dense(g) && (reduction == 0 ? g.numel() == x.size(0) : g.numel() == 1) &&
            (!defined(w) || (dense(*w) && w->numel() == x.size(1))) && dense(tw) && tw.numel() == 1 &&
            reduction >= 0 && reduction <= 2,
        "(N, C) float32 log-probabilities and N int64 targets");
  Tensor gx = empty_dev(x.sizes());
  check(omt_nll_loss_bwd(x.size(0), x.size(1), fp(g), t.data_ptr<int64_t>(), defined(w) ? fp(*w) : nullptr, ignore,
                         (int)reduction, fp(tw), fpm(gx), cur_stream()),
        "nll_loss_backward");
  return gx;
}

// ---- squeeze-excite backward (omt:: ops the compile backend rewrites to) ----

// g * s + v * scale, s and v [N, C, 1, 1] (or [N, C]): the gradient reaching a squeeze-excite input through the gate
// and through the plane mean (a multiply, the mean's broadcast and an add in the graph)
Tensor se_gate_backward_ref(const Tensor& g, const Tensor& s, const Tensor& v, double scale) {
  const int64_t n = g.size(0), c = g.size(1);
  return at::add(at::mul(g, s.reshape({n, c, 1, 1})), at::mul(v.reshape({n, c, 1, 1}), scale));
}
Tensor se_gate_backward_dev(const Tensor& g, const Tensor& s, const Tensor& v, double scale) {
  cover(g.dim() == 4 && s.numel() == g.size(0) * g.size(1) && v.numel() == s.numel(), "[N, C, H, W] with [N, C] gates");
  cover(dense(s) && dense(v), "contiguous float32 gates");
  if (is_cl(g) && f32(g)) {  // channels-last planes
    Tensor y = empty_dev_cl(g.sizes());
    check(omt_se_gate_bwd_nhwc(g.size(0), g.size(1), g.size(2) * g.size(3), fp(g), fp(s), fp(v), (float)scale, fpm(y),
                               cur_stream()),
          "omt::se_gate_backward (channels last)");
    return y;
  }
  cover(dense(g), "contiguous float32");
  Tensor y = empty_dev(g.sizes());
  check(omt_se_gate_bwd(g.size(0) * g.size(1), g.size(2) * g.size(3), fp(g), fp(s), fp(v), (float)scale, fpm(y),
                        cur_stream()),
        "omt::se_gate_backward");
  return y;
}
Tensor se_gate_backward_k(const Tensor& g, const Tensor& s, const Tensor& v, double scale) {
  return dev_or_ref<&se_gate_backward_dev, &se_gate_backward_ref>("omt::se_gate_backward", g, s, v, scale);
}

// sum over the last two dims of a * b, [N, C, 1, 1] (a multiply and a sum in the graph)
Tensor plane_dot_ref(const Tensor& a, const Tensor& b) { return at::sum(at::mul(a, b), {2, 3}, true); }
Tensor plane_dot_dev(const Tensor& a, const Tensor& b) {
  cover(a.dim() == 4 && a.sizes().equals(b.sizes()), "two [N, C, H, W] operands");
  if (is_cl(a) || is_cl(b)) return plane_dot_ref(a, b);  // channels-last: the elementwise and plane-sum kernels
  cover(dense(a) && dense(b), "contiguous float32");
  const int64_t n = a.size(0), c = a.size(1);
  Tensor y = empty_dev({n, c, 1, 1});
  check(omt_plane_dot(n * c, a.size(2) * a.size(3), fp(a), fp(b), 1.f, fpm(y), cur_stream()), "omt::plane_dot");
  return y;
}
Tensor plane_dot_k(const Tensor& a, const Tensor& b) {
  return dev_or_ref<&plane_dot_dev, &plane_dot_ref>("omt::plane_dot", a, b);
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(omt, m) {
  // g * s + v * scale (s, v: [N, C] gates of [N, C, H, W] planes); the sum of a * b over each plane, [N, C, 1, 1]
  m.def("se_gate_backward(Tensor g, Tensor s, Tensor v, float scale) -> Tensor");
  m.def("plane_dot(Tensor a, Tensor b) -> Tensor");
}
TORCH_LIBRARY_IMPL(omt, CompositeExplicitAutograd, m) {
  m.impl("se_gate_backward", &se_gate_backward_ref);
  m.impl("plane_dot", &plane_dot_ref);
}
TORCH_LIBRARY_IMPL(omt, PrivateUse1, m) {
  m.impl("se_gate_backward", &se_gate_backward_k);
  m.impl("plane_dot", &plane_dot_k);
}

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  HotOps(m)
      .aux<at::_ops::add_Tensor, &add_t>()
      .aux<at::_ops::add__Tensor, &add_t_>()
      .aux<at::_ops::add__Scalar, &add_s_>()
      .aux<at::_ops::_foreach_add__Scalar, &foreach_add_s_>()
      .aux<at::_ops::mul_Tensor, &mul_t>()
      .aux<at::_ops::div_Tensor, &div_t>()
      .aux<at::_ops::relu, &relu_>()
      .aux<at::_ops::relu_, &relu_ip>()
      .aux<at::_ops::threshold_backward, &threshold_bwd>()
      .aux<at::_ops::hardswish, &hardswish_>()
      .aux<at::_ops::hardswish_, &hardswish_ip>()
      .aux<at::_ops::hardswish_backward, &hardswish_bwd>()
      .aux<at::_ops::hardsigmoid, &hardsigmoid_>()
      .aux<at::_ops::hardsigmoid_, &hardsigmoid_ip>()
      .aux<at::_ops::hardsigmoid_backward, &hardsigmoid_bwd>()
      .aux<at::_ops::fill__Scalar, &fill_s>()
      .aux<at::_ops::zero_, &zero_ip>()
      .aux<at::_ops::sum_dim_IntList, &sum_dims>()
      .aux<at::_ops::mean_dim, &mean_dims>()
      .aux<at::_ops::_log_softmax, &log_softmax_>()
      .aux<at::_ops::_log_softmax_backward_data, &log_softmax_bwd>()
      .aux<at::_ops::nll_loss_forward, &nll_fwd>()
      .aux<at::_ops::nll_loss_backward, &nll_bwd>();
}

}  // namespace omt
