// Hot-path operators of the device, each a thin host wrapper over libomt_hip.so's C ABI:
//   aten::convolution / convolution_backward            reference csrc/conv.cpp:179-237
//   aten::native_batch_norm / native_batch_norm_backward reference csrc/nn.cpp:25-78
//   aten::_native_batch_norm_legit{,_no_training}       reference csrc/fused.cpp:173-181, 234-237
//   aten::max_pool2d_with_indices(_backward), avg_pool2d(_backward), _adaptive_avg_pool2d(_backward)
//                                                        reference csrc/nn.cpp:157-222, 275-285
//   omt::bn_relu_train, bn_relu_backward, conv_act, conv_bn_act_eval (composite references + device kernels)
//                                                        reference csrc/fused.cpp:19-136, 213-233
// Cases a kernel does not cover fail a cover() and run on torch's HIP kernels instead, recorded in FALLBACKS.
#include "omt_torch.h"

namespace omt {

static Tensor contig(const Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }
static Tensor contig_cl(const Tensor& t) {
  return t.is_contiguous(at::MemoryFormat::ChannelsLast) ? t : t.contiguous(at::MemoryFormat::ChannelsLast);
}
// A dense convolution runs channels-last when its input or filter is (torch's convolutions pick their output memory
// format the same way): the NHWC kernels read and write that order in place. The reference makes every operand
// contiguous NCHW instead (base0, csrc/device.cpp:60-66).
static bool channels_last(const Tensor& x, const Tensor& w) {
  return x.suggest_memory_format() == at::MemoryFormat::ChannelsLast ||
         w.suggest_memory_format() == at::MemoryFormat::ChannelsLast;
}
static bool whole(const Tensor& t) { return f32(t) && t.is_contiguous(); }

// ------------------------------------------------------------------------------------------------------------------
// convolution
// ------------------------------------------------------------------------------------------------------------------

static int kind_of(const Tensor& x, const Tensor& w, IntArrayRef stride, IntArrayRef padding, IntArrayRef dilation,
                   bool transposed, int64_t groups) {
  if (!f32(x) || !f32(w) || x.dim() != 4 || w.dim() != 4 || stride.size() != 2 || padding.size() != 2 ||
      dilation.size() != 2)
    return OMT_CONV_NONE;
  return omt_conv_kind(x.size(1), w.size(0), w.size(2), w.size(3), stride[0], stride[1], padding[0], padding[1],
                       dilation[0], dilation[1], transposed ? 1 : 0, groups);
}

// y = conv(x, w) (+ bias) (+ ReLU for dense convs); shared by convolution and omt::conv_act
static Tensor conv_forward(const Tensor& x_, const Tensor& w_, const std::optional<Tensor>& bias, IntArrayRef stride,
                           IntArrayRef padding, IntArrayRef dilation, bool transposed, int64_t groups, bool relu) {
  const int kind = kind_of(x_, w_, stride, padding, dilation, transposed, groups);
  cover(kind != OMT_CONV_NONE, "dilated, transposed, grouped or non-square convolution");
  cover(!defined(bias) || (f32(*bias) && bias->dim() == 1), "float32 bias");
  cover(!relu || kind == OMT_CONV_DENSE, "ReLU epilogue on a depthwise convolution");
  Tensor b = defined(bias) ? contig(*bias) : Tensor();
  const bool cl = kind == OMT_CONV_DENSE && channels_last(x_, w_);
  unsigned epi = (b.defined() ? OMT_EPI_BIAS : 0u) | (relu ? OMT_EPI_RELU : 0u);
  if (cl) {
    Tensor x = contig_cl(x_), w = contig_cl(w_);
    omt_conv_geo g = conv_geo(x.size(0), x.size(1), w.size(0), x.size(2), x.size(3), w.size(2), stride[0], padding[0]);
    cover(g.oh >= 1 && g.ow >= 1, "empty output");
    Tensor y = empty_dev_cl({g.n, g.co, g.oh, g.ow});
    // input channels not a multiple of 16 (the 3-channel stem) run one fixed element-by-element gather: nothing to tune
    if (g.ci % 16 == 0) tune_conv(OMT_DIR_FWD_NHWC, g);
    Tensor ws = workspace(omt_conv_fwd_nhwc_workspace(&g));
    check(omt_conv_fwd_nhwc(&g, fp(x), fp(w), fp(b), epi, fpm(y), wsptr(ws), wsbytes(ws), cur_stream()),
          "convolution (channels last)");
    return y;
  }
  if (kind != OMT_CONV_DENSE && is_cl(x_)) {  // channels-last depthwise: the NHWC kernel, a channels-last output
    Tensor w = contig(w_);  // [c][1][ks][ks]: the same memory in either order
    omt_conv_geo g = conv_geo(x_.size(0), x_.size(1), w.size(0), x_.size(2), x_.size(3), w.size(2), stride[0],
                              padding[0]);
    cover(g.oh >= 1 && g.ow >= 1, "empty output");
    Tensor y = empty_dev_cl({g.n, g.co, g.oh, g.ow});
    const int st = omt_dw_fwd_nhwc(&g, fp(x_), fp(w), fp(b), fpm(y), cur_stream());
    cover(st != OMT_UNSUPPORTED, "channels-last depthwise size");
    check(st, "convolution (depthwise, channels last)");
    return y;
  }
  Tensor x = contig(x_), w = contig(w_);
  omt_conv_geo g = conv_geo(x.size(0), x.size(1), w.size(0), x.size(2), x.size(3), w.size(2), stride[0], padding[0]);
  cover(g.oh >= 1 && g.ow >= 1, "empty output");
  Tensor y = empty_dev({g.n, g.co, g.oh, g.ow});
  if (kind == OMT_CONV_DENSE) {
    tune_conv(OMT_DIR_FWD, g);
    Tensor ws = workspace(omt_conv_fwd_workspace(&g));
    check(omt_conv_fwd(&g, fp(x), fp(w), fp(b), epi, nullptr, nullptr, nullptr, nullptr, 1e-5f, fpm(y), wsptr(ws),
                       wsbytes(ws), cur_stream()),
          "convolution");
  } else {
    check(omt_dw_fwd(&g, fp(x), fp(w), fp(b), nullptr, nullptr, nullptr, nullptr, 1e-5f, fpm(y), cur_stream()),
          "convolution (depthwise)");
  }
  return y;
}

static Tensor convolution_(const Tensor& x, const Tensor& w, const std::optional<Tensor>& bias, IntArrayRef stride,
                           IntArrayRef padding, IntArrayRef dilation, bool transposed, IntArrayRef, int64_t groups) {
  return conv_forward(x, w, bias, stride, padding, dilation, transposed, groups, false);
}

// Backward of a channels-last dense convolution: grads in channels-last order, from the NHWC kernels (grad weight of
// co not a multiple of 4: the NCHW kernel and its result converted).
static std::tuple<Tensor, Tensor, Tensor> conv_backward_cl(const Tensor& gy_, const Tensor& x_, const Tensor& w_,
                                                           IntArrayRef stride, IntArrayRef padding,
                                                           std::array<bool, 3> mask) {
  omt_conv_geo g = conv_geo(x_.size(0), x_.size(1), w_.size(0), x_.size(2), x_.size(3), w_.size(2), stride[0],
                            padding[0]);
  cover(gy_.size(0) == g.n && gy_.size(1) == g.co && gy_.size(2) == g.oh && gy_.size(3) == g.ow, "gradient shape");
  Tensor gy = contig_cl(gy_);
  Tensor gx, gw, gb;
  void* s = cur_stream();
  if (mask[0]) {
    Tensor w = contig_cl(w_);
    gx = empty_dev_cl(x_.sizes());
    // co not a multiple of 16: one fixed element-by-element gather, nothing to tune
    if (g.co % 16 == 0) tune_conv(OMT_DIR_DGRAD_NHWC, g);
    Tensor ws = workspace(omt_conv_dgrad_nhwc_workspace(&g));
    check(omt_conv_dgrad_nhwc(&g, fp(gy), fp(w), fpm(gx), wsptr(ws), wsbytes(ws), s),
          "convolution_backward (input, channels last)");
  }
  if (mask[1]) {
    if (g.co % 4 == 0) {
      Tensor x = contig_cl(x_);
      gw = empty_dev_cl(w_.sizes());
      tune_conv(OMT_DIR_WGRAD_NHWC, g);
      Tensor ws = workspace(omt_conv_wgrad_nhwc_workspace(&g));
      check(omt_conv_wgrad_nhwc(&g, fp(x), fp(gy), fpm(gw), wsptr(ws), wsbytes(ws), s),
            "convolution_backward (weight, channels last)");
    } else {
      Tensor x = contig(x_), gyc = contig(gy_);
      Tensor t = empty_dev(w_.sizes());
      tune_conv(OMT_DIR_WGRAD, g);
      Tensor ws = workspace(omt_conv_wgrad_workspace(&g));
      check(omt_conv_wgrad(&g, fp(x), fp(gyc), fpm(t), wsptr(ws), wsbytes(ws), s), "convolution_backward (weight)");
      gw = contig_cl(t);
    }
  }
  if (mask[2]) {  // channels-last gy is [n oh ow][co]: the column sums of those rows
    gb = empty_dev({g.co});
    check(omt_bias_grad(g.n * g.oh * g.ow, g.co, 1, fp(gy), fpm(gb), s), "convolution_backward (bias)");
  }
  return {gx, gw, gb};
}

static std::tuple<Tensor, Tensor, Tensor> convolution_backward_(const Tensor& gy_, const Tensor& x_, const Tensor& w_,
                                                                at::OptionalIntArrayRef, IntArrayRef stride,
                                                                IntArrayRef padding, IntArrayRef dilation,
                                                                bool transposed, IntArrayRef, int64_t groups,
                                                                std::array<bool, 3> mask) {
  const int kind = kind_of(x_, w_, stride, padding, dilation, transposed, groups);
  cover(kind != OMT_CONV_NONE && f32(gy_), "dilated, transposed, grouped or non-square convolution");
  if (kind == OMT_CONV_DENSE && channels_last(x_, w_)) return conv_backward_cl(gy_, x_, w_, stride, padding, mask);
  if (kind != OMT_CONV_DENSE && is_cl(x_)) {  // channels-last depthwise
    Tensor gy = contig_cl(gy_), w = contig(w_);
    omt_conv_geo g = conv_geo(x_.size(0), x_.size(1), w.size(0), x_.size(2), x_.size(3), w.size(2), stride[0],
                              padding[0]);
    cover(gy.size(0) == g.n && gy.size(1) == g.co && gy.size(2) == g.oh && gy.size(3) == g.ow, "gradient shape");
    Tensor gx, gw, gb;
    void* s = cur_stream();
    if (mask[0]) {
      gx = empty_dev_cl(x_.sizes());
      const int st = omt_dw_dgrad_nhwc(&g, fp(gy), fp(w), fpm(gx), s);
      cover(st != OMT_UNSUPPORTED, "channels-last depthwise size");
      check(st, "convolution_backward (depthwise input, channels last)");
    }
    if (mask[1]) {
      gw = empty_dev(w.sizes());
      Tensor ws = workspace(omt_dw_wgrad_nhwc_workspace(&g));
      const int st = omt_dw_wgrad_nhwc(&g, fp(x_), fp(gy), fpm(gw), wsptr(ws), wsbytes(ws), s);
      cover(st != OMT_UNSUPPORTED, "channels-last depthwise size");
      check(st, "convolution_backward (depthwise weight, channels last)");
    }
    if (mask[2]) {  // [n oh ow][c] rows: their column sums
      gb = empty_dev({g.co});
      check(omt_bias_grad(g.n * g.oh * g.ow, g.co, 1, fp(gy), fpm(gb), s), "convolution_backward (bias)");
    }
    return {gx, gw, gb};
  }
  Tensor gy = contig(gy_), x = contig(x_), w = contig(w_);
  omt_conv_geo g = conv_geo(x.size(0), x.size(1), w.size(0), x.size(2), x.size(3), w.size(2), stride[0], padding[0]);
  cover(gy.size(0) == g.n && gy.size(1) == g.co && gy.size(2) == g.oh && gy.size(3) == g.ow, "gradient shape");
  Tensor gx, gw, gb;
  void* s = cur_stream();
  if (kind == OMT_CONV_DENSE && mask[0] && mask[1]) {
    // both GEMMs in one call: they share a launch when their plans allow it
    gx = empty_dev(x.sizes());
    gw = empty_dev(w.sizes());
    tune_conv_bwd(g);
    Tensor ws = workspace(omt_conv_bwd_workspace(&g));
    check(omt_conv_bwd(&g, fp(x), fp(gy), fp(w), fpm(gx), fpm(gw), wsptr(ws), wsbytes(ws), s), "convolution_backward");
  } else if (kind == OMT_CONV_DENSE) {
    if (mask[0]) {
      gx = empty_dev(x.sizes());
      tune_conv(OMT_DIR_DGRAD, g);
      Tensor ws = workspace(omt_conv_dgrad_workspace(&g));
      check(omt_conv_dgrad(&g, fp(gy), fp(w), fpm(gx), wsptr(ws), wsbytes(ws), s), "convolution_backward (input)");
    }
    if (mask[1]) {
      gw = empty_dev(w.sizes());
      tune_conv(OMT_DIR_WGRAD, g);
      Tensor ws = workspace(omt_conv_wgrad_workspace(&g));
      check(omt_conv_wgrad(&g, fp(x), fp(gy), fpm(gw), wsptr(ws), wsbytes(ws), s), "convolution_backward (weight)");
    }
  } else {
    if (mask[0]) {
      gx = empty_dev(x.sizes());
      check(omt_dw_dgrad(&g, fp(gy), fp(w), fpm(gx), s), "convolution_backward (depthwise input)");
    }
    if (mask[1]) {
      gw = empty_dev(w.sizes());
      Tensor ws = workspace(omt_dw_wgrad_workspace(&g));
      check(omt_dw_wgrad(&g, fp(x), fp(gy), fpm(gw), wsptr(ws), wsbytes(ws), s), "convolution_backward (depthwise weight)");
    }
  }
  if (mask[2]) {
    gb = empty_dev({g.co});
    check(omt_bias_grad(g.n, g.co, g.oh * g.ow, fp(gy), fpm(gb), s), "convolution_backward (bias)");
  }
  return {gx, gw, gb};
}

// ------------------------------------------------------------------------------------------------------------------
// batch norm
// ------------------------------------------------------------------------------------------------------------------

// The channels-last BatchNorm backward (omt_bn_bwd_nhwc): gz = (g + g2) through the activation's gradient (act_in:
// the ReLU's output or the hardswish's input), the BatchNorm grads of gz, and gz itself when want_gz (a residual
// branch's gradient). Operands not already channels-last are converted (none are in a channels-last model).
static std::tuple<Tensor, Tensor, Tensor, Tensor> bn_backward_cl4(const Tensor& g_, const Tensor* g2_,
                                                                  const Tensor& x, int act, const Tensor* act_in_,
                                                                  const Tensor& w, const Tensor& mean,
                                                                  const Tensor& invstd, std::array<bool, 3> mask,
                                                                  bool want_gz, const char* what) {
  const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
  // an NCHW g (a global average pool's gradient broadcast over its planes) is read in place
  const bool g_nchw = hw > 1 && c > 1 && !is_cl(g_) && g_.is_contiguous();
  Tensor g = g_nchw ? g_ : contig_cl(g_);
  Tensor g2 = g2_ ? contig_cl(*g2_) : Tensor();
  Tensor r = act_in_ ? contig_cl(*act_in_) : Tensor();
  Tensor gx = mask[0] ? empty_dev_cl(x.sizes()) : Tensor();
  Tensor dg = mask[1] ? empty_dev({c}) : Tensor();
  Tensor db = mask[2] ? empty_dev({c}) : Tensor();
  Tensor gz = want_gz ? empty_dev_cl(x.sizes()) : Tensor();
  Tensor ws = workspace(omt_bn_nhwc_workspace(n, c, hw));
  check(omt_bn_bwd_nhwc(n, c, hw, fp(g), g_nchw ? 1 : 0, g2.defined() ? fp(g2) : nullptr, fp(x), act,
                        r.defined() ? fp(r) : nullptr,
                        fp(mean), fp(invstd), fp(w), fpm(gx), fpm(dg), fpm(db), fpm(gz), wsptr(ws), wsbytes(ws),
                        cur_stream()),
        what);
  return {gx, dg, db, gz};
}
static std::tuple<Tensor, Tensor, Tensor> bn_backward_cl(const Tensor& g, const Tensor* g2, const Tensor& x, int act,
                                                         const Tensor* act_in, const Tensor& w, const Tensor& mean,
                                                         const Tensor& invstd, std::array<bool, 3> mask, bool want_gz,
                                                         const char* what) {
  auto r = bn_backward_cl4(g, g2, x, act, act_in, w, mean, invstd, mask, want_gz, what);
  return {std::get<0>(r), std::get<1>(r), std::get<2>(r)};
}
// The channels-last training BatchNorm (omt_bn_train_fwd_nhwc): y = act(bn(x) + res), z = its activation's input
// when want_z; running statistics rm / rv updated into nrm / nrv (which may be them).
static std::tuple<Tensor, Tensor, Tensor, Tensor> bn_train_cl(const Tensor& x, const Tensor& w, const Tensor& b,
                                                              const Tensor& rm, const Tensor& rv, const Tensor& nrm,
                                                              const Tensor& nrv, double mom, double eps, int act,
                                                              const Tensor* res_, bool want_z, const char* what) {
  const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
  Tensor res = res_ ? contig_cl(*res_) : Tensor();
  Tensor y = empty_dev_cl(x.sizes()), sm = empty_dev({c}), si = empty_dev({c});
  Tensor z = want_z ? empty_dev_cl(x.sizes()) : Tensor();
  Tensor ws = workspace(omt_bn_nhwc_workspace(n, c, hw));
  check(omt_bn_train_fwd_nhwc(n, c, hw, fp(x), fp(w), fp(b), fp(rm), fp(rv), mom, eps, act,
                              res.defined() ? fp(res) : nullptr, fpm(y), fpm(z), fpm(sm), fpm(si), fpm(nrm), fpm(nrv),
                              wsptr(ws), wsbytes(ws), cur_stream()),
        what);
  return {y, sm, si, z};
}

static std::tuple<Tensor, Tensor, Tensor> batch_norm_(const Tensor& x_, const std::optional<Tensor>& weight,
                                                      const std::optional<Tensor>& bias,
                                                      const std::optional<Tensor>& rm,
                                                      const std::optional<Tensor>& rv, bool training,
                                                      double momentum, double eps) {
  cover(defined(weight) && defined(bias) && defined(rm) && defined(rv) && f32(x_) && x_.dim() == 4,
       "batch norm without affine parameters or running stats, or not 4-D float32");
  cover(whole(*weight) && whole(*bias) && whole(*rm) && whole(*rv), "batch norm parameters must be contiguous float32");
  if (is_cl(x_)) {  // channels-last input: the NHWC kernels, a channels-last output
    const int64_t n = x_.size(0), c = x_.size(1), hw = x_.size(2) * x_.size(3);
    Tensor y = empty_dev_cl(x_.sizes());
    if (!training) {
      check(omt_bn_eval_fwd_nhwc(n, c, hw, fp(x_), fp(weight), fp(bias), fp(rm), fp(rv), eps, 0, fpm(y), cur_stream()),
            "native_batch_norm (eval, channels last)");
      return {y, empty_dev({0}), empty_dev({0})};
    }
    Tensor sm = empty_dev({c}), si = empty_dev({c});
    Tensor ws = workspace(omt_bn_nhwc_workspace(n, c, hw));
    float* rmp = rm->mutable_data_ptr<float>();
    float* rvp = rv->mutable_data_ptr<float>();
    check(omt_bn_train_fwd_nhwc(n, c, hw, fp(x_), fp(weight), fp(bias), rmp, rvp, momentum, eps, 0, nullptr, fpm(y),
                                nullptr, fpm(sm), fpm(si), rmp, rvp, wsptr(ws), wsbytes(ws), cur_stream()),
          "native_batch_norm (channels last)");
    return {y, sm, si};
  }
  Tensor x = contig(x_);
  const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
  Tensor y = empty_dev(x.sizes());
  if (!training) {
    check(omt_bn_eval_fwd(n, c, hw, fp(x), fp(weight), fp(bias), fp(rm), fp(rv), eps, 0, fpm(y), cur_stream()),
          "native_batch_norm (eval)");
    return {y, empty_dev({0}), empty_dev({0})};
  }
  Tensor sm = empty_dev({c}), si = empty_dev({c});
  Tensor ws = workspace(omt_bn_train_workspace(n, c, hw));
  float* rmp = rm->mutable_data_ptr<float>();
  float* rvp = rv->mutable_data_ptr<float>();
  check(omt_bn_train_fwd(n, c, hw, fp(x), fp(weight), fp(bias), rmp, rvp, momentum, eps, 0, fpm(y), fpm(sm), fpm(si),
                         rmp, rvp, wsptr(ws), wsbytes(ws), cur_stream()),
        "native_batch_norm");
  return {y, sm, si};
}

static std::tuple<Tensor, Tensor, Tensor> batch_norm_backward_(const Tensor& gy_, const Tensor& x_,
                                                               const std::optional<Tensor>& weight,
                                                               const std::optional<Tensor>&,
                                                               const std::optional<Tensor>&,
                                                               const std::optional<Tensor>& sm,
                                                               const std::optional<Tensor>& si, bool train, double,
                                                               std::array<bool, 3> mask) {
  cover(train && defined(weight) && defined(sm) && defined(si) && f32(x_) && f32(gy_) && x_.dim() == 4,
       "eval-mode or non-affine batch norm backward");
  cover(whole(*weight) && whole(*sm) && whole(*si), "contiguous float32 parameters");
  if (is_cl(x_)) return bn_backward_cl(gy_, nullptr, x_, OMT_ACT_NONE, nullptr, *weight, *sm, *si, mask, false,
                                       "native_batch_norm_backward (channels last)");
  Tensor gy = contig(gy_), x = contig(x_);
  const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
  Tensor gx = mask[0] ? empty_dev(x.sizes()) : Tensor();
  Tensor dg = mask[1] ? empty_dev({c}) : Tensor();
  Tensor db = mask[2] ? empty_dev({c}) : Tensor();
  Tensor ws = workspace(omt_bn_bwd_workspace(n, c, hw));
  check(omt_bn_bwd(n, c, hw, fp(gy), fp(x), nullptr, fp(sm), fp(si), fp(weight), fpm(gx), fpm(dg), fpm(db), wsptr(ws),
                   wsbytes(ws), cur_stream()),
        "native_batch_norm_backward");
  return {gx, dg, db};
}

// eager entry points of the non-functional BatchNorm variants that traced / compiled graphs call
static std::tuple<Tensor, Tensor, Tensor> bn_legit(const Tensor& x, const std::optional<Tensor>& w,
                                                   const std::optional<Tensor>& b, Tensor& rm, Tensor& rv,
                                                   bool training, double mom, double eps) {
  return batch_norm_(x, w, b, rm, rv, training, mom, eps);
}
static std::tuple<Tensor, Tensor, Tensor> bn_legit_no_training(const Tensor& x, const std::optional<Tensor>& w,
                                                               const std::optional<Tensor>& b, const Tensor& rm,
                                                               const Tensor& rv, double mom, double eps) {
  return batch_norm_(x, w, b, rm, rv, false, mom, eps);
}

// ------------------------------------------------------------------------------------------------------------------
// pools
// ------------------------------------------------------------------------------------------------------------------

struct Pool2 {
  int64_t kh, kw, sh, sw, ph, pw, dh, dw;
};
static Pool2 pool_args(IntArrayRef k, IntArrayRef s, IntArrayRef p, IntArrayRef d) {
  cover(k.size() == 1 || k.size() == 2, "kernel size");
  Pool2 r;
  r.kh = k[0];
  r.kw = k.size() == 2 ? k[1] : k[0];
  r.sh = s.empty() ? r.kh : s[0];
  r.sw = s.empty() ? r.kw : (s.size() == 2 ? s[1] : s[0]);
  r.ph = p[0];
  r.pw = p.size() == 2 ? p[1] : p[0];
  r.dh = d.empty() ? 1 : d[0];
  r.dw = d.empty() ? 1 : (d.size() == 2 ? d[1] : d[0]);
  // PyTorch's own argument checks (and their messages) stay with its kernels
  cover(r.kh > 0 && r.kw > 0 && r.sh > 0 && r.sw > 0 && r.dh > 0 && r.dw > 0 && r.ph >= 0 && r.pw >= 0 &&
           r.ph <= ((r.kh - 1) * r.dh + 1) / 2 && r.pw <= ((r.kw - 1) * r.dw + 1) / 2,
       "pooling arguments");
  return r;
}

static std::tuple<Tensor, Tensor> max_pool2d_(const Tensor& x_, IntArrayRef k, IntArrayRef s, IntArrayRef p,
                                              IntArrayRef d, bool ceil) {
  cover(f32(x_) && x_.dim() == 4, "4-D float32");
  Pool2 a = pool_args(k, s, p, d);
  if (is_cl(x_)) {  // channels-last input and outputs
    const int64_t n = x_.size(0), c = x_.size(1), ih = x_.size(2), iw = x_.size(3);
    const int64_t oh = pool_out(ih, a.kh, a.sh, a.ph, a.dh, ceil), ow = pool_out(iw, a.kw, a.sw, a.pw, a.dw, ceil);
    cover(oh >= 1 && ow >= 1, "empty output");
    Tensor y = empty_dev_cl({n, c, oh, ow}), idx = empty_dev_cl({n, c, oh, ow}, at::kLong);
    const int st = omt_maxpool_fwd_nhwc(n, c, ih, iw, oh, ow, a.kh, a.kw, a.sh, a.sw, a.ph, a.pw, a.dh, a.dw, fp(x_),
                                        fpm(y), idx.mutable_data_ptr<int64_t>(), cur_stream());
    cover(st != OMT_UNSUPPORTED, "channels-last pool size");
    check(st, "max_pool2d_with_indices (channels last)");
    return {y, idx};
  }
  Tensor x = contig(x_);
  const int64_t n = x.size(0), c = x.size(1), ih = x.size(2), iw = x.size(3);
  const int64_t oh = pool_out(ih, a.kh, a.sh, a.ph, a.dh, ceil), ow = pool_out(iw, a.kw, a.sw, a.pw, a.dw, ceil);
  cover(oh >= 1 && ow >= 1, "empty output");
  Tensor y = empty_dev({n, c, oh, ow}), idx = empty_dev({n, c, oh, ow}, at::kLong);
  check(omt_maxpool_fwd(n * c, ih, iw, oh, ow, a.kh, a.kw, a.sh, a.sw, a.ph, a.pw, a.dh, a.dw, fp(x), fpm(y),
                        idx.mutable_data_ptr<int64_t>(), cur_stream()),
        "max_pool2d_with_indices");
  return {y, idx};
}

static Tensor max_pool2d_backward_(const Tensor& gy_, const Tensor& x, IntArrayRef k, IntArrayRef s, IntArrayRef p,
                                   IntArrayRef d, bool, const Tensor& idx_) {
  cover(f32(gy_) && x.dim() == 4 && idx_.scalar_type() == at::kLong, "4-D float32");
  Pool2 a = pool_args(k, s, p, d);
  const int64_t n = x.size(0), c = x.size(1), ih = x.size(2), iw = x.size(3);
  if (is_cl(x)) {
    Tensor gy = contig_cl(gy_), idx = idx_.is_contiguous(at::MemoryFormat::ChannelsLast)
                                          ? idx_
                                          : idx_.contiguous(at::MemoryFormat::ChannelsLast);
    Tensor gx = empty_dev_cl(x.sizes());
    const int st = omt_maxpool_bwd_nhwc(n, c, ih, iw, gy.size(2), gy.size(3), a.kh, a.kw, a.sh, a.sw, a.ph, a.pw, a.dh,
                                        a.dw, fp(gy), idx.data_ptr<int64_t>(), fpm(gx), cur_stream());
    cover(st != OMT_UNSUPPORTED, "channels-last pool size");
    check(st, "max_pool2d_with_indices_backward (channels last)");
    return gx;
  }
  Tensor gy = contig(gy_), idx = contig(idx_);
  Tensor gx = empty_dev(x.sizes());
  check(omt_maxpool_bwd(n * c, ih, iw, gy.size(2), gy.size(3), a.kh, a.kw, a.sh, a.sw, a.ph, a.pw, a.dh, a.dw, fp(gy),
                        idx.data_ptr<int64_t>(), fpm(gx), cur_stream()),
        "max_pool2d_with_indices_backward");
  return gx;
}

static Tensor avg_pool2d_(const Tensor& x_, IntArrayRef k, IntArrayRef s, IntArrayRef p, bool ceil, bool incl,
                          std::optional<int64_t> div) {
  cover(f32(x_) && x_.dim() == 4, "4-D float32");
  cover(!div || *div > 0, "divisor_override");
  Pool2 a = pool_args(k, s, p, {});
  cover(a.ph <= a.kh / 2 && a.pw <= a.kw / 2, "pooling arguments");
  if (is_cl(x_)) {
    const int64_t n = x_.size(0), c = x_.size(1), ih = x_.size(2), iw = x_.size(3);
    const int64_t oh = pool_out(ih, a.kh, a.sh, a.ph, 1, ceil), ow = pool_out(iw, a.kw, a.sw, a.pw, 1, ceil);
    cover(oh >= 1 && ow >= 1, "empty output");
    Tensor y = empty_dev_cl({n, c, oh, ow});
    const int st = omt_avgpool_fwd_nhwc(n, c, ih, iw, oh, ow, a.kh, a.kw, a.sh, a.sw, a.ph, a.pw, incl ? 1 : 0,
                                        div.value_or(0), fp(x_), fpm(y), cur_stream());
    cover(st != OMT_UNSUPPORTED, "channels-last pool size");
    check(st, "avg_pool2d (channels last)");
    return y;
  }
  Tensor x = contig(x_);
  const int64_t n = x.size(0), c = x.size(1), ih = x.size(2), iw = x.size(3);
  const int64_t oh = pool_out(ih, a.kh, a.sh, a.ph, 1, ceil), ow = pool_out(iw, a.kw, a.sw, a.pw, 1, ceil);
  cover(oh >= 1 && ow >= 1, "empty output");
  Tensor y = empty_dev({n, c, oh, ow});
  check(omt_avgpool_fwd(n * c, ih, iw, oh, ow, a.kh, a.kw, a.sh, a.sw, a.ph, a.pw, incl ? 1 : 0, div.value_or(0), fp(x),
                        fpm(y), cur_stream()),
        "avg_pool2d");
  return y;
}

static Tensor avg_pool2d_backward_(const Tensor& gy_, const Tensor& x, IntArrayRef k, IntArrayRef s, IntArrayRef p,
                                   bool, bool incl, std::optional<int64_t> div) {
  cover(f32(gy_) && x.dim() == 4, "4-D float32");
  cover(!div || *div > 0, "divisor_override");
  Pool2 a = pool_args(k, s, p, {});
  const int64_t n = x.size(0), c = x.size(1), ih = x.size(2), iw = x.size(3);
  if (is_cl(x)) {
    Tensor gy = contig_cl(gy_);
    Tensor gx = empty_dev_cl(x.sizes());
    const int st = omt_avgpool_bwd_nhwc(n, c, ih, iw, gy.size(2), gy.size(3), a.kh, a.kw, a.sh, a.sw, a.ph, a.pw,
                                        incl ? 1 : 0, div.value_or(0), fp(gy), fpm(gx), cur_stream());
    cover(st != OMT_UNSUPPORTED, "channels-last pool size");
    check(st, "avg_pool2d_backward (channels last)");
    return gx;
  }
  Tensor gy = contig(gy_);
  Tensor gx = empty_dev(x.sizes());
  check(omt_avgpool_bwd(n * c, ih, iw, gy.size(2), gy.size(3), a.kh, a.kw, a.sh, a.sw, a.ph, a.pw, incl ? 1 : 0,
                        div.value_or(0), fp(gy), fpm(gx), cur_stream()),
        "avg_pool2d_backward");
  return gx;
}

static Tensor adaptive_avg_pool2d_(const Tensor& x_, IntArrayRef out) {
  cover(f32(x_) && x_.dim() == 4 && out.size() == 2 && out[0] >= 1 && out[1] >= 1, "4-D float32");
  if (is_cl(x_)) {
    const int64_t n = x_.size(0), c = x_.size(1);
    Tensor y = empty_dev_cl({n, c, out[0], out[1]});
    const int st = omt_adapool_fwd_nhwc(n, c, x_.size(2), x_.size(3), out[0], out[1], fp(x_), fpm(y), cur_stream());
    cover(st != OMT_UNSUPPORTED, "channels-last pool size");
    check(st, "_adaptive_avg_pool2d (channels last)");
    return y;
  }
  Tensor x = contig(x_);
  const int64_t n = x.size(0), c = x.size(1);
  Tensor y = empty_dev({n, c, out[0], out[1]});
  check(omt_adapool_fwd(n * c, x.size(2), x.size(3), out[0], out[1], fp(x), fpm(y), cur_stream()),
        "_adaptive_avg_pool2d");
  return y;
}

static Tensor adaptive_avg_pool2d_backward_(const Tensor& gy_, const Tensor& x) {
  cover(f32(gy_) && x.dim() == 4, "4-D float32");
  if (is_cl(x)) {
    Tensor gy = contig_cl(gy_);
    Tensor gx = empty_dev_cl(x.sizes());
    const int st = omt_adapool_bwd_nhwc(x.size(0), x.size(1), x.size(2), x.size(3), gy.size(2), gy.size(3), fp(gy),
                                        fpm(gx), cur_stream());
    cover(st != OMT_UNSUPPORTED, "channels-last pool size");
    check(st, "_adaptive_avg_pool2d_backward (channels last)");
    return gx;
  }
  Tensor gy = contig(gy_);
  Tensor gx = empty_dev(x.sizes());
  check(omt_adapool_bwd(x.size(0) * x.size(1), x.size(2), x.size(3), gy.size(2), gy.size(3), fp(gy), fpm(gx),
                        cur_stream()),
        "_adaptive_avg_pool2d_backward");
  return gx;
}

// ------------------------------------------------------------------------------------------------------------------
// omt:: fused ops (the torch.compile backend rewrites graphs to them)
// ------------------------------------------------------------------------------------------------------------------

// composite references in plain aten ops (csrc/fused.cpp:19-46): any device, and the fallback of the fast paths
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> bn_relu_train_ref(const Tensor& x, const Tensor& w,
                                                                          const Tensor& b, const Tensor& rm,
                                                                          const Tensor& rv, double mom, double eps) {
  auto r = at::_native_batch_norm_legit_functional(x, w, b, rm, rv, true, mom, eps);
  return {at::relu(std::get<0>(r)), std::get<1>(r), std::get<2>(r), std::get<3>(r), std::get<4>(r)};
}
// act 1: ReLU, 2: hardswish (whose input z is also returned: its backward reads it), else none
static std::tuple<Tensor, Tensor, Tensor, Tensor> bn_train_inplace_ref(const Tensor& x, const Tensor& w,
                                                                       const Tensor& b, const Tensor& rm,
                                                                       const Tensor& rv, double mom, double eps,
                                                                       int64_t act, const std::optional<Tensor>& res) {
  Tensor rm_ = rm, rv_ = rv;  // _native_batch_norm_legit updates them in place
  auto r = at::_native_batch_norm_legit(x, w, b, rm_, rv_, true, mom, eps);
  Tensor z = std::get<0>(r);
  if (defined(res)) z = z + *res;
  Tensor y = act == OMT_ACT_RELU ? at::relu(z) : act == OMT_ACT_HARDSWISH ? at::hardswish(z) : z;
  return {y, std::get<1>(r), std::get<2>(r), act == OMT_ACT_HARDSWISH ? z : Tensor()};
}
// convolution (no bias) -> training BatchNorm (in place) [-> + residual] [-> activation]; also returns the
// convolution's output, which the BatchNorm backward reads
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> conv_bn_train_ref(const Tensor& x, const Tensor& cw,
                                                                            IntArrayRef stride, IntArrayRef padding,
                                                                            const Tensor& w, const Tensor& b,
                                                                            const Tensor& rm, const Tensor& rv,
                                                                            double mom, double eps, int64_t act,
                                                                            const std::optional<Tensor>& res) {
  Tensor conv = at::convolution(x, cw, std::nullopt, stride, padding, {1, 1}, false, {0, 0}, 1);
  auto r = bn_train_inplace_ref(conv, w, b, rm, rv, mom, eps, act, res);
  return {std::get<0>(r), std::get<1>(r), std::get<2>(r), std::get<3>(r), conv};
}
static std::tuple<Tensor, Tensor, Tensor> bn_relu_backward_ref(const Tensor& g, const Tensor& x, const Tensor& y,
                                                               const Tensor& w, const Tensor& mean,
                                                               const Tensor& invstd, std::array<bool, 3> mask) {
  Tensor gz = at::threshold_backward(g, y, 0);
  return at::native_batch_norm_backward(gz, x, w, std::nullopt, std::nullopt, mean, invstd, true, 0.0, mask);
}
// r: the ReLU's output (act 1) or the hardswish's input (act 2)
static std::tuple<Tensor, Tensor, Tensor> bn_act_backward_ref(const Tensor& g, const Tensor& x, const Tensor& r,
                                                              const Tensor& w, const Tensor& mean,
                                                              const Tensor& invstd, int64_t act,
                                                              std::array<bool, 3> mask) {
  Tensor gz = act == OMT_ACT_RELU ? at::threshold_backward(g, r, 0)
              : act == OMT_ACT_HARDSWISH ? at::hardswish_backward(g, r) : g;
  return at::native_batch_norm_backward(gz, x, w, std::nullopt, std::nullopt, mean, invstd, true, 0.0, mask);
}
static std::tuple<Tensor, Tensor, Tensor, Tensor> bn_relu_res_backward_ref(const Tensor& g,
                                                                           const std::optional<Tensor>& g2,
                                                                           const Tensor& x, const Tensor& y,
                                                                           const Tensor& w, const Tensor& mean,
                                                                           const Tensor& invstd,
                                                                           std::array<bool, 3> mask) {
  Tensor gz = at::threshold_backward(defined(g2) ? g + *g2 : g, y, 0);
  auto r = at::native_batch_norm_backward(gz, x, w, std::nullopt, std::nullopt, mean, invstd, true, 0.0, mask);
  return {std::get<0>(r), std::get<1>(r), std::get<2>(r), gz};
}
// A convolution backward whose grad input g is a BatchNorm backward's incoming gradient (BatchNorm -> activation ->
// convolution in the forward): the convolution's grad weight, then omt::bn_relu_res_backward(g, other, x, r, ...)
// (res) or omt::bn_act_backward(g, x, r, ..., act), as (grad weight, gx, dgamma, dbeta, gz; gz undefined unless res)
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> conv_bn_backward_ref(
    const Tensor& gy, const Tensor& cx, const Tensor& cw, IntArrayRef stride, IntArrayRef padding,
    const std::optional<Tensor>& other, const Tensor& x, const Tensor& r, const Tensor& w, const Tensor& mean,
    const Tensor& invstd, int64_t act, bool res, std::array<bool, 3> mask) {
  auto cb = at::convolution_backward(gy, cx, cw, std::nullopt, stride, padding, {1, 1}, false, {0, 0}, 1,
                                     {true, true, false});
  if (res) {
    auto b = bn_relu_res_backward_ref(std::get<0>(cb), other, x, r, w, mean, invstd, mask);
    return {std::get<1>(cb), std::get<0>(b), std::get<1>(b), std::get<2>(b), std::get<3>(b)};
  }
  TORCH_CHECK(!defined(other), "omt::conv_bn_backward: a second gradient needs res");
  auto b = bn_act_backward_ref(std::get<0>(cb), x, r, w, mean, invstd, act, mask);
  return {std::get<1>(cb), std::get<0>(b), std::get<1>(b), std::get<2>(b), Tensor()};
}
// omt::bn_train_ (no residual) followed by max_pool2d_with_indices of its output (no dilation, floor mode):
// (y, save_mean, save_invstd, pooled, indices)
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> bn_train_pool_ref(const Tensor& x, const Tensor& w,
                                                                            const Tensor& b, const Tensor& rm,
                                                                            const Tensor& rv, double mom, double eps,
                                                                            int64_t act, IntArrayRef kernel,
                                                                            IntArrayRef stride, IntArrayRef padding) {
  auto r = bn_train_inplace_ref(x, w, b, rm, rv, mom, eps, act, std::nullopt);
  auto mp = at::max_pool2d_with_indices(std::get<0>(r), kernel, stride, padding, {1, 1}, false);
  return {std::get<0>(r), std::get<1>(r), std::get<2>(r), std::get<0>(mp), std::get<1>(mp)};
}
static Tensor conv_act_ref(const Tensor& x, const Tensor& w, const std::optional<Tensor>& b, IntArrayRef stride,
                           IntArrayRef padding, int64_t act) {
  Tensor y = at::convolution(x, w, b, stride, padding, {1, 1}, false, {0, 0}, 1);
  return act == 1 ? at::relu(y) : y;
}
static std::pair<Tensor, Tensor> fold_bn_ref(const Tensor& cw, const std::optional<Tensor>& cb, const Tensor& w,
                                             const Tensor& b, const Tensor& rm, const Tensor& rv, double eps) {
  Tensor scale = w * at::rsqrt(rv + eps);
  Tensor fw = cw * scale.view({-1, 1, 1, 1});
  Tensor fb = (defined(cb) ? (*cb - rm) : -rm) * scale + b;
  return {fw, fb};
}
static Tensor conv_bn_act_eval_ref(const Tensor& x, const Tensor& cw, const std::optional<Tensor>& cb,
                                   const Tensor& w, const Tensor& b, const Tensor& rm, const Tensor& rv, double eps,
                                   IntArrayRef stride, IntArrayRef padding, int64_t act) {
  auto f = fold_bn_ref(cw, cb, w, b, rm, rv, eps);
  return conv_act_ref(x, f.first, f.second, stride, padding, act);
}

// device paths
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> bn_relu_train_dev(const Tensor& x_, const Tensor& w,
                                                                          const Tensor& b, const Tensor& rm,
                                                                          const Tensor& rv, double mom, double eps) {
  cover(f32(x_) && x_.dim() == 4 && whole(w) && whole(b) && whole(rm) && whole(rv),
       "4-D float32 with contiguous parameters");
  if (is_cl(x_)) {
    const int64_t c = x_.size(1);
    Tensor nrm = empty_dev({c}), nrv = empty_dev({c});
    auto r = bn_train_cl(x_, w, b, rm, rv, nrm, nrv, mom, eps, OMT_ACT_RELU, nullptr, false,
                         "omt::bn_relu_train (channels last)");
    return {std::get<0>(r), std::get<1>(r), std::get<2>(r), nrm, nrv};
  }
  Tensor x = contig(x_);
  const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
  Tensor y = empty_dev(x.sizes()), sm = empty_dev({c}), si = empty_dev({c}), nrm = empty_dev({c}), nrv = empty_dev({c});
  Tensor ws = workspace(omt_bn_train_workspace(n, c, hw));
  check(omt_bn_train_fwd(n, c, hw, fp(x), fp(w), fp(b), fp(rm), fp(rv), mom, eps, 1, fpm(y), fpm(sm), fpm(si),
                         fpm(nrm), fpm(nrv), wsptr(ws), wsbytes(ws), cur_stream()),
        "omt::bn_relu_train");
  return {y, sm, si, nrm, nrv};
}
// Training BatchNorm with the running statistics updated in place, then the optional residual and ReLU.
static std::tuple<Tensor, Tensor, Tensor, Tensor> bn_train_inplace_dev(const Tensor& x_, const Tensor& w,
                                                                       const Tensor& b, const Tensor& rm,
                                                                       const Tensor& rv, double mom, double eps,
                                                                       int64_t act,
                                                                       const std::optional<Tensor>& res_) {
  cover(act >= OMT_ACT_NONE && act <= OMT_ACT_HARDSWISH, "activation none, ReLU or hardswish");
  cover(f32(x_) && x_.dim() == 4 && whole(w) && whole(b) && whole(rm) && whole(rv),
       "4-D float32 with contiguous parameters");
  cover(!defined(res_) || (f32(*res_) && res_->sizes() == x_.sizes()), "residual of the input's shape");
  if (is_cl(x_))
    return bn_train_cl(x_, w, b, rm, rv, rm, rv, mom, eps, (int)act, defined(res_) ? &*res_ : nullptr,
                       act == OMT_ACT_HARDSWISH, "omt::bn_train_ (channels last)");
  Tensor x = contig(x_);
  Tensor res;
  if (defined(res_)) res = contig(*res_);
  const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
  Tensor y = empty_dev(x.sizes()), sm = empty_dev({c}), si = empty_dev({c});
  Tensor z = act == OMT_ACT_HARDSWISH ? empty_dev(x.sizes()) : Tensor();
  Tensor ws = workspace(omt_bn_train_workspace(n, c, hw));
  check(omt_bn_train_fwd_res(n, c, hw, fp(x), fp(w), fp(b), fp(rm), fp(rv), mom, eps, (int)act,
                             res.defined() ? fp(res) : nullptr, fpm(y), fpm(z), fpm(sm), fpm(si), fpm(rm), fpm(rv),
                             wsptr(ws), wsbytes(ws), cur_stream()),
        "omt::bn_train_");
  return {y, sm, si, z};
}
// The convolution leaves a K split of up to kFoldSlices slices (kFoldSlicesSmall in channels of at most 1024
// elements, which the BatchNorm reads one vector per thread with eight slices' loads in flight) unsummed and the
// BatchNorm sums them as it reads them (in the slice order of the convolution's own slice sum: the convolution output
// and everything after it are bit-identical to convolution + omt::bn_train_), one launch fewer; other plans run the two
// as they are. (Reading 16-32 slices one at a time, a 2x2-plane layer's BatchNorm took longer than the slice-sum
// launch.)
constexpr int kFoldSlices = 4, kFoldSlicesSmall = 16;
// Channels of up to this many elements (n * oh * ow) are normalized by one BatchNorm launch that holds the channel in
// registers (one read of the input already). Larger ones take the statistics from the convolution's epilogue when
// the output has at least kStatsMinBytes: below that the epilogue's sums cost the convolution more than the skipped
// read saves (graph replays, conv + BN + ReLU: [32,64,56^2] 3x3 +5.3 / -1.6 us, [128,32,32^2] +2.6 / -0.6 us;
// [256,64,56^2] 3x3 +12 / -17 us, 1x1 from 256 channels -8 / -22 us).
constexpr int64_t kBnOneLaunchMax = 8192, kStatsMinBytes = 64ll << 20;
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> conv_bn_train_dev(const Tensor& x_, const Tensor& cw_,
                                                                            IntArrayRef stride, IntArrayRef padding,
                                                                            const Tensor& w, const Tensor& b,
                                                                            const Tensor& rm, const Tensor& rv,
                                                                            double mom, double eps, int64_t act,
                                                                            const std::optional<Tensor>& res_) {
  cover(act >= OMT_ACT_NONE && act <= OMT_ACT_HARDSWISH, "activation none, ReLU or hardswish");
  cover(stride.size() == 2 && padding.size() == 2 && stride[0] == stride[1] && padding[0] == padding[1],
        "uniform 2-D stride and padding");
  if (kind_of(x_, cw_, stride, padding, {1, 1}, false, 1) == OMT_CONV_DENSE && channels_last(x_, cw_)) {
    // channels-last: the NHWC convolution, then the NHWC BatchNorm of its output (no partials to fold)
    Tensor conv = conv_forward(x_, cw_, std::nullopt, stride, padding, {1, 1}, false, 1, false);
    auto r = bn_train_inplace_dev(conv, w, b, rm, rv, mom, eps, act, res_);
    return {std::get<0>(r), std::get<1>(r), std::get<2>(r), std::get<3>(r), conv};
  }
  cover(kind_of(x_, cw_, stride, padding, {1, 1}, false, 1) == OMT_CONV_DENSE, "dense convolution");
  cover(whole(w) && whole(b) && whole(rm) && whole(rv), "contiguous float32 BatchNorm parameters");
  Tensor x = contig(x_), cw = contig(cw_);
  omt_conv_geo g = conv_geo(x.size(0), x.size(1), cw.size(0), x.size(2), x.size(3), cw.size(2), stride[0], padding[0]);
  cover(g.oh >= 1 && g.ow >= 1, "empty output");
  Tensor res;
  if (defined(res_)) {
    cover(f32(*res_) && res_->sizes() == IntArrayRef({g.n, g.co, g.oh, g.ow}), "residual of the output's shape");
    res = contig(*res_);
  }
  tune_conv(OMT_DIR_FWD, g);
  Tensor conv = empty_dev({g.n, g.co, g.oh, g.ow});
  Tensor ws = workspace(omt_conv_fwd_workspace(&g));
  const int64_t n = g.n, c = g.co, hw = g.oh * g.ow;
  Tensor y = empty_dev(conv.sizes()), sm = empty_dev({c}), si = empty_dev({c});
  Tensor z = act == OMT_ACT_HARDSWISH ? empty_dev(conv.sizes()) : Tensor();
  const float* r = res.defined() ? fp(res) : nullptr;
  const int relu = (int)act;
  if (n * hw > kBnOneLaunchMax && n * c * hw * 4 >= kStatsMinBytes) {
    // the statistics from the convolution's epilogue, so the BatchNorm reads the convolution output once; a plan
    // that splits K (or a batch run in chunks) is refused before any launch and takes the path below
    Tensor stats = workspace(omt_conv_fwd_stats_bytes(&g));
    int groups = 0;
    const int st = omt_conv_fwd_stats(&g, fp(x), fp(cw), fpm(conv), (double*)wsptr(stats), wsbytes(stats), &groups,
                                      wsptr(ws), wsbytes(ws), cur_stream());
    if (st == OMT_OK) {
      Tensor bws = workspace(omt_bn_train_workspace(n, c, hw));
      check(omt_bn_train_fwd_stats(n, c, hw, fp(conv), (const double*)wsptr(stats), groups, wsbytes(stats), fp(w),
                                   fp(b), fp(rm),
                                   fp(rv), mom, eps, relu, r, fpm(y), fpm(z), fpm(sm), fpm(si), fpm(rm), fpm(rv),
                                   wsptr(bws), wsbytes(bws), cur_stream()),
            "omt::conv_bn_train_ (BatchNorm from the epilogue statistics)");
      return {y, sm, si, z, conv};
    }
    if (st != OMT_UNSUPPORTED) check(st, "omt::conv_bn_train_ (convolution with statistics)");
  }
  const float* parts = nullptr;
  int slices = 1;
  check(omt_conv_fwd_unsummed(&g, fp(x), fp(cw), fpm(conv), wsptr(ws), wsbytes(ws),
                              n * hw <= 1024 ? kFoldSlicesSmall : kFoldSlices, &parts, &slices, cur_stream()),
        "omt::conv_bn_train_ (convolution)");
  Tensor bws = workspace(omt_bn_train_workspace(n, c, hw));
  if (slices > 1)
    check(omt_bn_train_fwd_parts(n, c, hw, parts, slices, fpm(conv), fp(w), fp(b), fp(rm), fp(rv), mom, eps, relu, r,
                                 fpm(y), fpm(z), fpm(sm), fpm(si), fpm(rm), fpm(rv), wsptr(bws), wsbytes(bws),
                                 cur_stream()),
          "omt::conv_bn_train_ (BatchNorm of the partials)");
  else
    check(omt_bn_train_fwd_res(n, c, hw, fp(conv), fp(w), fp(b), fp(rm), fp(rv), mom, eps, relu, r, fpm(y), fpm(z),
                               fpm(sm), fpm(si), fpm(rm), fpm(rv), wsptr(bws), wsbytes(bws), cur_stream()),
          "omt::conv_bn_train_ (BatchNorm)");
  return {y, sm, si, z, conv};
}
static std::tuple<Tensor, Tensor, Tensor> bn_relu_backward_dev(const Tensor& g_, const Tensor& x_, const Tensor& y_,
                                                               const Tensor& w, const Tensor& mean,
                                                               const Tensor& invstd, std::array<bool, 3> mask) {
  cover(f32(g_) && f32(x_) && f32(y_) && x_.dim() == 4 && whole(w) && whole(mean) && whole(invstd), "4-D float32");
  if (is_cl(x_))
    return bn_backward_cl(g_, nullptr, x_, OMT_ACT_RELU, &y_, w, mean, invstd, mask, false,
                          "omt::bn_relu_backward (channels last)");
  Tensor g = contig(g_), x = contig(x_), y = contig(y_);
  const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
  Tensor gx = mask[0] ? empty_dev(x.sizes()) : Tensor();
  Tensor dg = mask[1] ? empty_dev({c}) : Tensor();
  Tensor db = mask[2] ? empty_dev({c}) : Tensor();
  Tensor ws = workspace(omt_bn_bwd_workspace(n, c, hw));
  check(omt_bn_bwd(n, c, hw, fp(g), fp(x), fp(y), fp(mean), fp(invstd), fp(w), fpm(gx), fpm(dg), fpm(db), wsptr(ws),
                   wsbytes(ws), cur_stream()),
        "omt::bn_relu_backward");
  return {gx, dg, db};
}
static std::tuple<Tensor, Tensor, Tensor> bn_act_backward_dev(const Tensor& g_, const Tensor& x_, const Tensor& r_,
                                                              const Tensor& w, const Tensor& mean,
                                                              const Tensor& invstd, int64_t act,
                                                              std::array<bool, 3> mask) {
  cover(act >= OMT_ACT_NONE && act <= OMT_ACT_HARDSWISH, "activation none, ReLU or hardswish");
  cover(f32(g_) && f32(x_) && f32(r_) && x_.dim() == 4 && g_.sizes() == x_.sizes() && r_.sizes() == x_.sizes() &&
            whole(w) && whole(mean) && whole(invstd),
        "4-D float32 operands of one shape");
  if (is_cl(x_))
    return bn_backward_cl(g_, nullptr, x_, (int)act, act == OMT_ACT_NONE ? nullptr : &r_, w, mean, invstd, mask,
                          false, "omt::bn_act_backward (channels last)");
  Tensor g = contig(g_), x = contig(x_), r = contig(r_);
  const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
  Tensor gx = mask[0] ? empty_dev(x.sizes()) : Tensor();
  Tensor dg = mask[1] ? empty_dev({c}) : Tensor();
  Tensor db = mask[2] ? empty_dev({c}) : Tensor();
  Tensor ws = workspace(omt_bn_bwd_workspace(n, c, hw));
  check(omt_bn_bwd_act(n, c, hw, fp(g), fp(x), (int)act, fp(r), fp(mean), fp(invstd), fp(w), fpm(gx), fpm(dg),
                       fpm(db), wsptr(ws), wsbytes(ws), cur_stream()),
        "omt::bn_act_backward");
  return {gx, dg, db};
}
// The backward of BatchNorm -> [+ residual] -> ReLU at a residual block's end, with the incoming gradient the sum of
// the block output's two uses (g + g2): gz = (g + g2) [y > 0] for the residual branch, and BatchNorm's grads of gz.
static std::tuple<Tensor, Tensor, Tensor, Tensor> bn_relu_res_backward_dev(const Tensor& g_,
                                                                           const std::optional<Tensor>& g2_,
                                                                           const Tensor& x_, const Tensor& y_,
                                                                           const Tensor& w, const Tensor& mean,
                                                                           const Tensor& invstd,
                                                                           std::array<bool, 3> mask) {
  cover(f32(g_) && f32(x_) && f32(y_) && x_.dim() == 4 && whole(w) && whole(mean) && whole(invstd) &&
            g_.sizes() == x_.sizes() && y_.sizes() == x_.sizes() &&
            (!defined(g2_) || (f32(*g2_) && g2_->sizes() == x_.sizes())),
        "4-D float32 operands of one shape");
  if (is_cl(x_))
    return bn_backward_cl4(g_, defined(g2_) ? &*g2_ : nullptr, x_, OMT_ACT_RELU, &y_, w, mean, invstd, mask, true,
                           "omt::bn_relu_res_backward (channels last)");
  Tensor g = contig(g_), x = contig(x_), y = contig(y_);
  Tensor g2 = defined(g2_) ? contig(*g2_) : Tensor();
  const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
  Tensor gx = mask[0] ? empty_dev(x.sizes()) : Tensor();
  Tensor dg = mask[1] ? empty_dev({c}) : Tensor();
  Tensor db = mask[2] ? empty_dev({c}) : Tensor();
  Tensor gz = empty_dev(x.sizes());
  Tensor ws = workspace(omt_bn_bwd_workspace(n, c, hw));
  check(omt_bn_bwd_res(n, c, hw, fp(g), g2.defined() ? fp(g2) : nullptr, fp(x), fp(y), fp(mean), fp(invstd), fp(w),
                       fpm(gx), fpm(dg), fpm(db), fpm(gz), wsptr(ws), wsbytes(ws), cur_stream()),
        "omt::bn_relu_res_backward");
  return {gx, dg, db, gz};
}
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> bn_train_pool_dev(const Tensor& x_, const Tensor& w,
                                                                            const Tensor& b, const Tensor& rm,
                                                                            const Tensor& rv, double mom, double eps,
                                                                            int64_t act, IntArrayRef kernel,
                                                                            IntArrayRef stride, IntArrayRef padding) {
  cover(act >= OMT_ACT_NONE && act <= OMT_ACT_HARDSWISH, "activation none, ReLU or hardswish");
  cover(f32(x_) && x_.dim() == 4 && whole(w) && whole(b) && whole(rm) && whole(rv),
        "4-D float32 with contiguous parameters");
  cover(kernel.size() == 2 && stride.size() == 2 && padding.size() == 2, "2-D pooling window");
  if (is_cl(x_)) {  // channels-last: the NHWC BatchNorm, then the NHWC max pool of its output
    auto r = bn_train_cl(x_, w, b, rm, rv, rm, rv, mom, eps, (int)act, nullptr, false,
                         "omt::bn_train_pool_ (channels last)");
    auto mp = max_pool2d_(std::get<0>(r), kernel, stride, padding, {1, 1}, false);
    return {std::get<0>(r), std::get<1>(r), std::get<2>(r), std::get<0>(mp), std::get<1>(mp)};
  }
  Tensor x = contig(x_);
  const int64_t n = x.size(0), c = x.size(1), h = x.size(2), wd = x.size(3);
  const int64_t kh = kernel[0], kw = kernel[1], sh = stride[0], sw = stride[1], ph = padding[0], pw = padding[1];
  cover(kh >= 1 && kw >= 1 && sh >= 1 && sw >= 1 && ph >= 0 && pw >= 0 && 2 * ph <= kh && 2 * pw <= kw &&
            h + 2 * ph >= kh && wd + 2 * pw >= kw,
        "pooling window");
  const int64_t oh = (h + 2 * ph - kh) / sh + 1, ow = (wd + 2 * pw - kw) / sw + 1;
  Tensor y = empty_dev(x.sizes()), sm = empty_dev({c}), si = empty_dev({c});
  Tensor out = empty_dev({n, c, oh, ow}), idx = empty_dev({n, c, oh, ow}, at::kLong);
  Tensor ws = workspace(omt_bn_train_workspace(n, c, h * wd));
  check(omt_bn_train_fwd_pool(n, c, h, wd, fp(x), fp(w), fp(b), fp(rm), fp(rv), mom, eps, (int)act, fpm(y), fpm(sm),
                              fpm(si), fpm(rm), fpm(rv), kh, kw, sh, sw, ph, pw, fpm(out),
                              idx.mutable_data_ptr<int64_t>(), wsptr(ws), wsbytes(ws), cur_stream()),
        "omt::bn_train_pool_");
  return {y, sm, si, out, idx};
}
// The convolution leaves its grad input unsummed (up to kFoldBwdSlices slices, kFoldBwdSlicesSmall for channels of
// at most 1024 elements, which the BatchNorm reads one vector per thread with eight slices' loads in flight) and the
// one-launch BatchNorm backward sums the partials as it reads them, in the convolution's slice order, and runs the
// grad weight's slice sum on extra workgroups: one launch (the convolution's slice sums) fewer, results equal to the
// two ops run apart. Channels of more than kBnOneLaunchMax elements run the two as they are. (Graph replays of
// ResNet-18 at 64x64: a 2x2-plane layer's BatchNorm reading 32 slices took 16.7 us against 4.7 + 7.4 us for the slice
// sum and the BatchNorm apart; with 2-4 slices the BatchNorm took 2-4 us longer and saved a 4.7 us launch.)
constexpr int kFoldBwdSlices = 4, kFoldBwdSlicesSmall = 8;
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> conv_bn_backward_dev(
    const Tensor& gy_, const Tensor& cx_, const Tensor& cw_, IntArrayRef stride, IntArrayRef padding,
    const std::optional<Tensor>& other_, const Tensor& x_, const Tensor& r_, const Tensor& w, const Tensor& mean,
    const Tensor& invstd, int64_t act, bool res, std::array<bool, 3> mask) {
  cover(res ? act == OMT_ACT_RELU : (act >= OMT_ACT_NONE && act <= OMT_ACT_HARDSWISH),
        "activation none, ReLU or hardswish (ReLU with a residual branch)");
  cover(res || !defined(other_), "a second gradient only with a residual branch");
  cover(stride.size() == 2 && padding.size() == 2 && stride[0] == stride[1] && padding[0] == padding[1],
        "uniform 2-D stride and padding");
  if (kind_of(cx_, cw_, stride, padding, {1, 1}, false, 1) == OMT_CONV_DENSE && channels_last(cx_, cw_) &&
      f32(gy_) && gy_.dim() == 4) {
    // channels-last: the NHWC convolution backward, then the NHWC BatchNorm backward of its grad input
    auto cb = convolution_backward_(gy_, cx_, cw_, std::nullopt, stride, padding, {1, 1}, false, {0, 0}, 1,
                                    {true, true, false});
    if (res) {
      auto b = bn_relu_res_backward_dev(std::get<0>(cb), other_, x_, r_, w, mean, invstd, mask);
      return {std::get<1>(cb), std::get<0>(b), std::get<1>(b), std::get<2>(b), std::get<3>(b)};
    }
    auto b = bn_act_backward_dev(std::get<0>(cb), x_, r_, w, mean, invstd, act, mask);
    return {std::get<1>(cb), std::get<0>(b), std::get<1>(b), std::get<2>(b), Tensor()};
  }
  cover(kind_of(cx_, cw_, stride, padding, {1, 1}, false, 1) == OMT_CONV_DENSE && f32(gy_) && gy_.dim() == 4,
        "dense convolution");
  cover(f32(x_) && f32(r_) && x_.dim() == 4 && cx_.sizes() == x_.sizes() && r_.sizes() == x_.sizes() && whole(w) &&
            whole(mean) && whole(invstd) && (!defined(other_) || (f32(*other_) && other_->sizes() == x_.sizes())),
        "4-D float32 BatchNorm operands of the convolution input's shape");
  Tensor gy = contig(gy_), cx = contig(cx_), cw = contig(cw_), x = contig(x_), r = contig(r_);
  Tensor other = defined(other_) ? contig(*other_) : Tensor();
  omt_conv_geo g = conv_geo(cx.size(0), cx.size(1), cw.size(0), cx.size(2), cx.size(3), cw.size(2), stride[0],
                            padding[0]);
  cover(gy.size(0) == g.n && gy.size(1) == g.co && gy.size(2) == g.oh && gy.size(3) == g.ow, "gradient shape");
  const int64_t n = x.size(0), c = x.size(1), hw = x.size(2) * x.size(3);
  Tensor cgx = empty_dev(cx.sizes()), cgw = empty_dev(cw.sizes());
  Tensor gx = mask[0] ? empty_dev(x.sizes()) : Tensor();
  Tensor dg = mask[1] ? empty_dev({c}) : Tensor();
  Tensor db = mask[2] ? empty_dev({c}) : Tensor();
  Tensor gz = res ? empty_dev(x.sizes()) : Tensor();
  const float* o = other.defined() ? fp(other) : nullptr;
  void* s = cur_stream();
  tune_conv_bwd(g);
  Tensor ws = workspace(omt_conv_bwd_workspace(&g));
  if (n * hw <= kBnOneLaunchMax) {
    const float* parts = nullptr;
    int slices = 1;
    omt_slice_sum job{};
    const int fold = n * hw <= 1024 ? kFoldBwdSlicesSmall : kFoldBwdSlices;
    const int st = omt_conv_bwd_parts(&g, fp(cx), fp(gy), fp(cw), fpm(cgx), fpm(cgw), wsptr(ws), wsbytes(ws), fold,
                                      &parts, &slices, &job, s);
    if (st == OMT_OK) {
      check(omt_bn_bwd_parts(n, c, hw, parts ? parts : fp(cgx), slices, o, fp(x), (int)act, fp(r), fp(mean),
                             fp(invstd), fp(w), fpm(gx), fpm(dg), fpm(db), fpm(gz), &job, job.slices > 0 ? 1 : 0, s),
            "omt::conv_bn_backward (BatchNorm over the partials)");
      return {cgw, gx, dg, db, gz};
    }
    if (st != OMT_UNSUPPORTED) check(st, "omt::conv_bn_backward (convolution)");
  }
  check(omt_conv_bwd(&g, fp(cx), fp(gy), fp(cw), fpm(cgx), fpm(cgw), wsptr(ws), wsbytes(ws), s),
        "omt::conv_bn_backward (convolution)");
  Tensor bws = workspace(omt_bn_bwd_workspace(n, c, hw));
  if (res)
    check(omt_bn_bwd_res(n, c, hw, fp(cgx), o, fp(x), fp(r), fp(mean), fp(invstd), fp(w), fpm(gx), fpm(dg), fpm(db),
                         fpm(gz), wsptr(bws), wsbytes(bws), s),
          "omt::conv_bn_backward (BatchNorm)");
  else
    check(omt_bn_bwd_act(n, c, hw, fp(cgx), fp(x), (int)act, fp(r), fp(mean), fp(invstd), fp(w), fpm(gx), fpm(dg),
                         fpm(db), wsptr(bws), wsbytes(bws), s),
          "omt::conv_bn_backward (BatchNorm)");
  return {cgw, gx, dg, db, gz};
}
static Tensor conv_act_dev(const Tensor& x, const Tensor& w, const std::optional<Tensor>& b, IntArrayRef stride,
                           IntArrayRef padding, int64_t act) {
  cover(stride.size() == 2 && padding.size() == 2, "2-D stride and padding");
  return conv_forward(x, w, b, stride, padding, {1, 1}, false, 1, act == 1);
}
static Tensor conv_bn_act_eval_dev(const Tensor& x, const Tensor& cw_, const std::optional<Tensor>& cb_,
                                   const Tensor& w, const Tensor& b, const Tensor& rm, const Tensor& rv, double eps,
                                   IntArrayRef stride, IntArrayRef padding, int64_t act) {
  cover(f32(cw_) && cw_.dim() == 4 && whole(w) && whole(b) && whole(rm) && whole(rv) && (!defined(cb_) || f32(*cb_)),
       "float32 parameters");
  Tensor cw = contig(cw_);
  Tensor cb = defined(cb_) ? contig(*cb_) : Tensor();
  const int64_t co = cw.size(0);
  Tensor fw = empty_dev(cw.sizes()), fb = empty_dev({co});
  check(omt_fold_bn(co, cw.numel() / co, fp(cw), fp(cb), fp(w), fp(b), fp(rm), fp(rv), (float)eps, fpm(fw), fpm(fb),
                    cur_stream()),
        "omt::conv_bn_act_eval (fold)");
  return conv_act_dev(x, fw, fb, stride, padding, act);
}

// device kernels when they cover the call, else the composite reference (whose aten ops reach the device kernels or
// torch's)
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> bn_relu_train_k(const Tensor& x, const Tensor& w,
                                                                        const Tensor& b, const Tensor& rm,
                                                                        const Tensor& rv, double mom, double eps) {
  return dev_or_ref<&bn_relu_train_dev, &bn_relu_train_ref>("omt::bn_relu_train", x, w, b, rm, rv, mom, eps);
}
static std::tuple<Tensor, Tensor, Tensor, Tensor> bn_train_inplace_k(const Tensor& x, const Tensor& w,
                                                                     const Tensor& b, const Tensor& rm,
                                                                     const Tensor& rv, double mom, double eps,
                                                                     int64_t act, const std::optional<Tensor>& res) {
  return dev_or_ref<&bn_train_inplace_dev, &bn_train_inplace_ref>("omt::bn_train_", x, w, b, rm, rv, mom, eps, act,
                                                                  res);
}
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> conv_bn_train_k(const Tensor& x, const Tensor& cw,
                                                                          IntArrayRef s, IntArrayRef p,
                                                                          const Tensor& w, const Tensor& b,
                                                                          const Tensor& rm, const Tensor& rv,
                                                                          double mom, double eps, int64_t act,
                                                                          const std::optional<Tensor>& res) {
  return dev_or_ref<&conv_bn_train_dev, &conv_bn_train_ref>("omt::conv_bn_train_", x, cw, s, p, w, b, rm, rv, mom, eps,
                                                            act, res);
}
static std::tuple<Tensor, Tensor, Tensor> bn_relu_backward_k(const Tensor& g, const Tensor& x, const Tensor& y,
                                                             const Tensor& w, const Tensor& mean,
                                                             const Tensor& invstd, std::array<bool, 3> mask) {
  return dev_or_ref<&bn_relu_backward_dev, &bn_relu_backward_ref>("omt::bn_relu_backward", g, x, y, w, mean, invstd,
                                                                  mask);
}
static std::tuple<Tensor, Tensor, Tensor> bn_act_backward_k(const Tensor& g, const Tensor& x, const Tensor& r,
                                                            const Tensor& w, const Tensor& mean, const Tensor& invstd,
                                                            int64_t act, std::array<bool, 3> mask) {
  return dev_or_ref<&bn_act_backward_dev, &bn_act_backward_ref>("omt::bn_act_backward", g, x, r, w, mean, invstd, act,
                                                                mask);
}
static std::tuple<Tensor, Tensor, Tensor, Tensor> bn_relu_res_backward_k(const Tensor& g,
                                                                         const std::optional<Tensor>& g2,
                                                                         const Tensor& x, const Tensor& y,
                                                                         const Tensor& w, const Tensor& mean,
                                                                         const Tensor& invstd,
                                                                         std::array<bool, 3> mask) {
  return dev_or_ref<&bn_relu_res_backward_dev, &bn_relu_res_backward_ref>("omt::bn_relu_res_backward", g, g2, x, y, w,
                                                                          mean, invstd, mask);
}
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> bn_train_pool_k(const Tensor& x, const Tensor& w,
                                                                          const Tensor& b, const Tensor& rm,
                                                                          const Tensor& rv, double mom, double eps,
                                                                          int64_t act, IntArrayRef k, IntArrayRef s,
                                                                          IntArrayRef p) {
  return dev_or_ref<&bn_train_pool_dev, &bn_train_pool_ref>("omt::bn_train_pool_", x, w, b, rm, rv, mom, eps, act, k,
                                                            s, p);
}
static std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> conv_bn_backward_k(
    const Tensor& gy, const Tensor& cx, const Tensor& cw, IntArrayRef s, IntArrayRef p,
    const std::optional<Tensor>& other, const Tensor& x, const Tensor& r, const Tensor& w, const Tensor& mean,
    const Tensor& invstd, int64_t act, bool res, std::array<bool, 3> mask) {
  return dev_or_ref<&conv_bn_backward_dev, &conv_bn_backward_ref>("omt::conv_bn_backward", gy, cx, cw, s, p, other, x,
                                                                  r, w, mean, invstd, act, res, mask);
}
static Tensor conv_act_k(const Tensor& x, const Tensor& w, const std::optional<Tensor>& b, IntArrayRef s,
                         IntArrayRef p, int64_t act) {
  return dev_or_ref<&conv_act_dev, &conv_act_ref>("omt::conv_act", x, w, b, s, p, act);
}
static Tensor conv_bn_act_eval_k(const Tensor& x, const Tensor& cw, const std::optional<Tensor>& cb, const Tensor& w,
                                 const Tensor& b, const Tensor& rm, const Tensor& rv, double eps, IntArrayRef s,
                                 IntArrayRef p, int64_t act) {
  return dev_or_ref<&conv_bn_act_eval_dev, &conv_bn_act_eval_ref>("omt::conv_bn_act_eval", x, cw, cb, w, b, rm, rv,
                                                                  eps, s, p, act);
}

TORCH_LIBRARY(omt, m) {
  m.def("bn_relu_train(Tensor x, Tensor w, Tensor b, Tensor rm, Tensor rv, float momentum, float eps) -> "
        "(Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("bn_relu_backward(Tensor g, Tensor x, Tensor y, Tensor w, Tensor mean, Tensor invstd, bool[3] mask) -> "
        "(Tensor, Tensor, Tensor)");
  // the backward of a residual block's end: gz = (g + g2) [y > 0], BatchNorm's (gx, dgamma, dbeta) of gz, and gz
  m.def("bn_relu_res_backward(Tensor g, Tensor? g2, Tensor x, Tensor y, Tensor w, Tensor mean, Tensor invstd, "
        "bool[3] mask) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("conv_act(Tensor x, Tensor w, Tensor? b, int[] stride, int[] padding, int act) -> Tensor");
  // training BatchNorm updating the running statistics in place, then + residual and the activation (act 1 ReLU,
  // 2 hardswish): the compile backend's form of BatchNorm -> [add] -> [activation] with the buffer updates kept in the
  // graph. Returns (y, save_mean, save_invstd, z) with z the hardswish's input (act 2; undefined otherwise)
  m.def("bn_train_(Tensor x, Tensor w, Tensor b, Tensor(a!) rm, Tensor(b!) rv, float momentum, float eps, int act, "
        "Tensor? residual) -> (Tensor, Tensor, Tensor, Tensor)");
  // BatchNorm backward through the activation: r is the ReLU's output (act 1) or the hardswish's input (act 2)
  m.def("bn_act_backward(Tensor g, Tensor x, Tensor r, Tensor w, Tensor mean, Tensor invstd, int act, bool[3] mask) "
        "-> (Tensor, Tensor, Tensor)");
  m.def("conv_bn_act_eval(Tensor x, Tensor cw, Tensor? cb, Tensor w, Tensor b, Tensor rm, Tensor rv, float eps, "
        "int[] stride, int[] padding, int act) -> Tensor");
  // convolution (no bias) -> bn_train_: (y, save_mean, save_invstd, z, convolution output)
  m.def("conv_bn_train_(Tensor x, Tensor cw, int[] stride, int[] padding, Tensor w, Tensor b, Tensor(a!) rm, "
        "Tensor(b!) rv, float momentum, float eps, int act, Tensor? residual) -> (Tensor, Tensor, Tensor, Tensor, "
        "Tensor)");
  // bn_train_ (no residual) -> max_pool2d_with_indices (no dilation, floor mode) of its output in one pass:
  // (y, save_mean, save_invstd, pooled, indices)
  m.def("bn_train_pool_(Tensor x, Tensor w, Tensor b, Tensor(a!) rm, Tensor(b!) rv, float momentum, float eps, "
        "int act, int[] kernel, int[] stride, int[] padding) -> (Tensor, Tensor, Tensor, Tensor, Tensor)");
  // a convolution backward feeding its grad input to a BatchNorm backward (res: omt::bn_relu_res_backward with
  // `other` its g2; else omt::bn_act_backward): (convolution grad weight, gx, dgamma, dbeta, gz)
  m.def("conv_bn_backward(Tensor gy, Tensor cx, Tensor cw, int[] stride, int[] padding, Tensor? other, Tensor x, "
        "Tensor r, Tensor w, Tensor mean, Tensor invstd, int act, bool res, bool[3] mask) -> (Tensor, Tensor, Tensor, "
        "Tensor, Tensor)");
}
TORCH_LIBRARY_IMPL(omt, CompositeExplicitAutograd, m) {
  m.impl("bn_relu_train", &bn_relu_train_ref);
  m.impl("bn_train_", &bn_train_inplace_ref);
  m.impl("bn_relu_backward", &bn_relu_backward_ref);
  m.impl("bn_act_backward", &bn_act_backward_ref);
  m.impl("bn_relu_res_backward", &bn_relu_res_backward_ref);
  m.impl("conv_act", &conv_act_ref);
  m.impl("conv_bn_act_eval", &conv_bn_act_eval_ref);
  m.impl("conv_bn_train_", &conv_bn_train_ref);
  m.impl("conv_bn_backward", &conv_bn_backward_ref);
  m.impl("bn_train_pool_", &bn_train_pool_ref);
}
TORCH_LIBRARY_IMPL(omt, PrivateUse1, m) {
  m.impl("bn_relu_train", &bn_relu_train_k);
  m.impl("bn_train_", &bn_train_inplace_k);
  m.impl("bn_relu_backward", &bn_relu_backward_k);
  m.impl("bn_act_backward", &bn_act_backward_k);
  m.impl("bn_relu_res_backward", &bn_relu_res_backward_k);
  m.impl("conv_act", &conv_act_k);
  m.impl("conv_bn_act_eval", &conv_bn_act_eval_k);
  m.impl("conv_bn_train_", &conv_bn_train_k);
  m.impl("conv_bn_backward", &conv_bn_backward_k);
  m.impl("bn_train_pool_", &bn_train_pool_k);
}

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  HotOps(m)
      .on<at::_ops::convolution, &convolution_>()
      .on<at::_ops::convolution_backward, &convolution_backward_>()
      .on<at::_ops::native_batch_norm, &batch_norm_>()
      .on<at::_ops::native_batch_norm_backward, &batch_norm_backward_>()
      .on<at::_ops::_native_batch_norm_legit, &bn_legit>()
      .on<at::_ops::_native_batch_norm_legit_no_training, &bn_legit_no_training>()
      .on<at::_ops::max_pool2d_with_indices, &max_pool2d_>()
      .on<at::_ops::max_pool2d_with_indices_backward, &max_pool2d_backward_>()
      .on<at::_ops::avg_pool2d, &avg_pool2d_>()
      .on<at::_ops::avg_pool2d_backward, &avg_pool2d_backward_>()
      .on<at::_ops::_adaptive_avg_pool2d, &adaptive_avg_pool2d_>()
      .on<at::_ops::_adaptive_avg_pool2d_backward, &adaptive_avg_pool2d_backward_>();
}

}  // namespace omt
