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

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  HotOps(m).aux<at::_ops::mm, &mm_>().aux<at::_ops::addmm, &addmm_>();
}

}  // namespace omt
