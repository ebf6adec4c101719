// The linear layers' matrix products (aten::mm, aten::addmm) on the dense-convolution GEMMs of libomt_hip.so.
// Reference: csrc/linalg.cpp:25-79 (mm_into / mm_ / addmm_ over its GEMM template, omarchy_mac_torch/gemm.py kind 4).
//
// A matrix product is a 1x1 convolution over 1x1 images, and the three products a linear layer's training step makes
// are exactly the three directions of that convolution (rows of a row-major [M, K] operand are the "images", its
// columns the channels):
//   forward      y[M, N]  = x[M, K] @ W^T          x row-major, W^T = a column-major view of W [N, K]
//                -> omt_conv_fwd (n = M, ci = K, co = N), with the bias in the GEMM epilogue (addmm);
//   grad input   gx[M, N] = gy[M, K] @ W[K, N]     both row-major
//                -> omt_conv_dgrad (n = M, co = K, ci = N);
//   grad weight  gW[M, N] = gy^T[M, K] @ x[K, N]   gy^T a column-major view of gy [K, M], x row-major
//                -> omt_conv_wgrad (n = K, co = M, ci = N).
// PyTorch's autograd of addmm (mm_mat1_backward / mm_mat2_backward) requests the last two in exactly these layouts
// for nn.Linear. The fourth layout (both operands column-major), other strides, other dtypes and a general addmm
// (beta, alpha != 1, a matrix `self`) run on torch's own HIP GEMMs, like every op without a kernel here. Plans come from
// the convolution plan cache and its tuner, keyed by the convolution geometry.
#include "omt_torch.h"

namespace omt {

namespace {

// [rows, cols] with unit column stride: each row one contiguous run (size-1 dims take any stride)
bool row_major(const Tensor& t) {
  return t.dim() == 2 && (t.size(1) == 1 || t.stride(1) == 1) && (t.size(0) == 1 || t.stride(0) == t.size(1));
}
bool col_major(const Tensor& t) {
  return t.dim() == 2 && (t.size(0) == 1 || t.stride(0) == 1) && (t.size(1) == 1 || t.stride(1) == t.size(0));
}
bool operand(const Tensor& t) { return is_dev(t) && f32(t) && t.dim() == 2 && t.numel() > 0; }

enum Form { kFwd, kDgrad, kWgrad };

Form form_of(const Tensor& a, const Tensor& b, bool forward) {
  cover(operand(a) && operand(b) && a.size(1) == b.size(0), "non-empty float32 2-D operands");
  // a single row or column is both row- and column-major: the forward form wins where it is wanted (a bias to add)
  if (row_major(a) && col_major(b) && (forward || !row_major(b))) return kFwd;
  if (row_major(a) && row_major(b)) return kDgrad;
  if (col_major(a) && row_major(b)) return kWgrad;
  throw NotCovered("both operands column-major, or strided rows");
}

// out[M, N] = a[M, K] @ b[K, N] (+ bias[N] in the forward form)
Tensor product(const Tensor& a, const Tensor& b, const Tensor& bias) {
  const Form f = form_of(a, b, bias.defined());
  cover(!bias.defined() || f == kFwd, "bias with a product that is not a linear layer's forward");
  const int64_t M = a.size(0), K = a.size(1), N = b.size(1);
  Tensor out = empty_dev({M, N});
  void* s = cur_stream();
  if (f == kFwd) {  // x = a [M][K] = [n][ci][1][1]; w = b^T [N][K] = [co][ci][1][1]
    omt_conv_geo g = conv_geo(M, K, N, 1, 1, 1, 1, 0);
    tune_conv(OMT_DIR_FWD, g);
    Tensor ws = workspace(omt_conv_fwd_workspace(&g));
    check(omt_conv_fwd(&g, fp(a), fp(b), fp(bias), bias.defined() ? OMT_EPI_BIAS : 0u, nullptr, nullptr, nullptr,
                       nullptr, 1e-5f, fpm(out), wsptr(ws), wsbytes(ws), s),
          "mm (linear forward)");
  } else if (f == kDgrad) {  // gy = a [M][K] = [n][co]; w = b [K][N] = [co][ci]; gx = out [n][ci]
    omt_conv_geo g = conv_geo(M, N, K, 1, 1, 1, 1, 0);
    tune_conv(OMT_DIR_DGRAD, g);
    Tensor ws = workspace(omt_conv_dgrad_workspace(&g));
    check(omt_conv_dgrad(&g, fp(a), fp(b), fpm(out), wsptr(ws), wsbytes(ws), s), "mm (linear grad input)");
  } else {  // gy = a^T [K][M] = [n][co]; x = b [K][N] = [n][ci]; gw = out [co][ci]
    omt_conv_geo g = conv_geo(K, N, M, 1, 1, 1, 1, 0);
    tune_conv(OMT_DIR_WGRAD, g);
    Tensor ws = workspace(omt_conv_wgrad_workspace(&g));
    check(omt_conv_wgrad(&g, fp(b), fp(a), fpm(out), wsptr(ws), wsbytes(ws), s), "mm (linear grad weight)");
  }
  return out;
}

Tensor mm_(const Tensor& a, const Tensor& b) { return product(a, b, Tensor()); }

Tensor addmm_(const Tensor& self, const Tensor& a, const Tensor& b, const at::Scalar& beta, const at::Scalar& alpha) {
  cover(alpha.isFloatingPoint() || alpha.isIntegral(false), "real alpha");
  cover(beta.isFloatingPoint() || beta.isIntegral(false), "real beta");
  cover(alpha.toDouble() == 1.0, "alpha 1");
  if (beta.toDouble() == 0.0) return product(a, b, Tensor());  // self is ignored (NaN included), as in PyTorch
  cover(beta.toDouble() == 1.0, "beta 0 or 1");
  cover(is_dev(self) && f32(self) && self.dim() == 1 && self.is_contiguous() && b.dim() == 2 &&
            self.size(0) == b.size(1),
        "a bias vector (nn.Linear)");
  return product(a, b, self);
}

// The squeeze-excite block's excitation MLP, s = hardsigmoid(a2), a2 = W2 h + b2, h = relu(W1 z + b1) (omt::se_mlp,
// returning s and, for the backward, h and a2), and its backward from ds (omt::se_mlp_backward: dz, dW1, db1, dW2,
// db2). The references are the ops the compile backend replaces; the device runs omt_se_fwd / omt_se_bwd (two
// launches each).
std::tuple<Tensor, Tensor, Tensor> se_mlp_ref(const Tensor& z, const Tensor& w1, const Tensor& b1, const Tensor& w2,
                                              const Tensor& b2) {
  Tensor h = at::relu(at::linear(z, w1, b1));
  Tensor a2 = at::linear(h, w2, b2);
  return {at::hardsigmoid(a2), h, a2};
}
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> se_mlp_backward_ref(const Tensor& gs, const Tensor& z,
                                                                       const Tensor& h, const Tensor& a2,
                                                                       const Tensor& w1, const Tensor& w2) {
  Tensor da2 = at::hardsigmoid_backward(gs, a2);
  Tensor da1 = at::threshold_backward(at::mm(da2, w2), h, 0);
  return {at::mm(da1, w1), at::mm(da1.t(), z), da1.sum(0), at::mm(da2.t(), h), da2.sum(0)};
}

bool se_operand(const Tensor& t, int dim) { return is_dev(t) && f32(t) && t.dim() == dim && t.is_contiguous(); }

void se_check(const Tensor& z, const Tensor& w1, const Tensor& w2) {
  cover(se_operand(z, 2) && se_operand(w1, 2) && se_operand(w2, 2), "contiguous float32 device operands");
  const int64_t c = z.size(1), r = w1.size(0);
  cover(w1.size(1) == c && w2.size(0) == c && w2.size(1) == r, "nn.Linear shapes c -> r -> c");
}
std::tuple<Tensor, Tensor, Tensor> se_mlp_dev(const Tensor& z, const Tensor& w1, const Tensor& b1, const Tensor& w2,
                                              const Tensor& b2) {
  se_check(z, w1, w2);
  const int64_t n = z.size(0), c = z.size(1), r = w1.size(0);
  cover(se_operand(b1, 1) && se_operand(b2, 1) && b1.size(0) == r && b2.size(0) == c, "both biases, contiguous");
  Tensor s = empty_dev(z.sizes()), h = empty_dev({n, r}), a2 = empty_dev(z.sizes());
  const int st =
      omt_se_fwd(n, c, r, fp(z), fp(w1), fp(b1), fp(w2), fp(b2), fpm(s), fpm(h), fpm(a2), cur_stream());
  cover(st != OMT_UNSUPPORTED, "squeeze-excite sizes (c <= 2048, r <= 1024)");
  check(st, "omt::se_mlp");
  return {s, h, a2};
}
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> se_mlp_backward_dev(const Tensor& gs, const Tensor& z,
                                                                       const Tensor& h, const Tensor& a2,
                                                                       const Tensor& w1, const Tensor& w2) {
  se_check(z, w1, w2);
  const int64_t n = z.size(0), c = z.size(1), r = w1.size(0);
  cover(is_dev(gs) && f32(gs) && gs.sizes() == z.sizes(), "gradient of the output's shape");
  cover(se_operand(h, 2) && se_operand(a2, 2) && h.size(0) == n && h.size(1) == r && a2.sizes() == z.sizes(),
        "the forward's saved h and a2");
  Tensor g = gs.is_contiguous() ? gs : gs.contiguous();
  Tensor gz = empty_dev(z.sizes()), gw1 = empty_dev(w1.sizes()), gb1 = empty_dev({r});
  Tensor gw2 = empty_dev(w2.sizes()), gb2 = empty_dev({c});
  Tensor ws = workspace(omt_se_bwd_workspace(n, c, r));
  const int st = omt_se_bwd(n, c, r, fp(g), fp(z), fp(h), fp(a2), fp(w1), fp(w2), fpm(gz), fpm(gw1), fpm(gb1),
                            fpm(gw2), fpm(gb2), wsptr(ws), wsbytes(ws), cur_stream());
  cover(st != OMT_UNSUPPORTED, "squeeze-excite sizes (c <= 2048, r <= 1024)");
  check(st, "omt::se_mlp_backward");
  return {gz, gw1, gb1, gw2, gb2};
}
std::tuple<Tensor, Tensor, Tensor> se_mlp_k(const Tensor& z, const Tensor& w1, const Tensor& b1, const Tensor& w2,
                                            const Tensor& b2) {
  return dev_or_ref<&se_mlp_dev, &se_mlp_ref>("omt::se_mlp", z, w1, b1, w2, b2);
}
std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor> se_mlp_backward_k(const Tensor& gs, const Tensor& z,
                                                                     const Tensor& h, const Tensor& a2,
                                                                     const Tensor& w1, const Tensor& w2) {
  return dev_or_ref<&se_mlp_backward_dev, &se_mlp_backward_ref>("omt::se_mlp_backward", gs, z, h, a2, w1, w2);
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  HotOps(m).aux<at::_ops::mm, &mm_>().aux<at::_ops::addmm, &addmm_>();
}

TORCH_LIBRARY_FRAGMENT(omt, m) {
  // hardsigmoid(linear(relu(linear(z, w1, b1)), w2, b2)) with the hidden layer and the pre-activation kept for the
  // backward (s, h, a2), and its backward (dz, dw1, db1, dw2, db2); the autograd formula joining them is registered
  // from Python (omarchy_mac_torch/compile.py)
  m.def("se_mlp(Tensor z, Tensor w1, Tensor b1, Tensor w2, Tensor b2) -> (Tensor, Tensor, Tensor)");
  m.def("se_mlp_backward(Tensor gs, Tensor z, Tensor h, Tensor a2, Tensor w1, Tensor w2) -> (Tensor, Tensor, Tensor, "
        "Tensor, Tensor)");
}
TORCH_LIBRARY_IMPL(omt, CompositeExplicitAutograd, m) {
  m.impl("se_mlp", &se_mlp_ref);
  m.impl("se_mlp_backward", &se_mlp_backward_ref);
}
TORCH_LIBRARY_IMPL(omt, PrivateUse1, m) {
  m.impl("se_mlp", &se_mlp_k);
  m.impl("se_mlp_backward", &se_mlp_backward_k);
}

}  // namespace omt
