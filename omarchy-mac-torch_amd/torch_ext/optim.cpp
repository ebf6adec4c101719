// The fused optimizers on the device: aten _fused_sgd_, _fused_adam_ and _fused_adamw_ (float and tensor learning
// rate) over libomt_hip.so's multi-tensor kernels (omt_fused_sgd, omt_fused_adam). Reference: csrc/optim.cpp:12-67,
// which registers the same three ops for the PrivateUse1 device. Anything the kernels do not cover (other dtypes,
// non-contiguous tensors, host step counts) runs on torch's HIP kernels through the fallback and is recorded.
#include <vector>

#include "omt_torch.h"

namespace omt {
namespace {

// one dense float32 block on the device, NCHW-contiguous or channels-last (a channels-last model's filters, their
// gradients and optimizer states): the kernels run elementwise over the memory, so every tensor of one parameter
// must share the parameter's memory order (ordered_like)
bool dev_f32c(const Tensor& t) { return is_dev(t) && f32(t) && (t.is_contiguous() || is_cl(t)); }
bool ordered_like(const Tensor& t, const Tensor& p) { return dev_f32c(t) && is_cl(t) == is_cl(p); }

// learning rate: a value, or a float on the device (read by the kernel, so a captured graph sees its updates); a
// host tensor is read here
struct Lr {
  float v = 0.f;
  const float* dev = nullptr;
};
Lr lr_of(double lr) { return Lr{(float)lr, nullptr}; }
Lr lr_of(const Tensor& lr) {
  cover(lr.numel() == 1, "a one-element lr tensor");
  if (is_dev(lr)) {
    cover(f32(lr), "a float32 lr tensor");
    return Lr{0.f, fp(lr)};
  }
  cover(lr.device().is_cpu(), "lr on the host or this device");
  return Lr{(float)lr.item<double>(), nullptr};
}
const float* dev_scalar(const std::optional<Tensor>& t, const char* what) {
  if (!defined(t)) return nullptr;
  cover(is_dev(*t) && f32(*t) && t->numel() == 1, what);
  return fp(*t);
}

template <class LR>
void adam_impl(at::TensorList p, at::TensorList g, at::TensorList m, at::TensorList v, at::TensorList vmax,
               at::TensorList steps, LR lr, double beta1, double beta2, double wd, double eps, bool amsgrad,
               bool maximize, bool decoupled, const std::optional<Tensor>& grad_scale,
               const std::optional<Tensor>& found_inf) {
  const size_t n = p.size();
  cover(g.size() == n && m.size() == n && v.size() == n && steps.size() == n && (!amsgrad || vmax.size() == n),
       "tensor lists of one length");
  std::vector<omt_adam_tensor> ts(n);
  for (size_t i = 0; i < n; ++i) {
    cover(dev_f32c(p[i]) && ordered_like(g[i], p[i]) && ordered_like(m[i], p[i]) && ordered_like(v[i], p[i]),
          "contiguous float32 device tensors");
    const int64_t k = p[i].numel();
    cover(g[i].numel() == k && m[i].numel() == k && v[i].numel() == k, "matching tensor sizes");
    cover(is_dev(steps[i]) && f32(steps[i]) && steps[i].numel() == 1, "float32 step counts on the device");
    if (amsgrad) cover(ordered_like(vmax[i], p[i]) && vmax[i].numel() == k, "contiguous float32 max_exp_avg_sqs");
    ts[i] = omt_adam_tensor{fpm(p[i]), fpm(g[i]), fpm(m[i]), fpm(v[i]), amsgrad ? fpm(vmax[i]) : nullptr,
                            fp(steps[i]), k};
  }
  const Lr l = lr_of(lr);
  const omt_adam_params hp{l.v,         l.dev,   (float)beta1,        (float)beta2,
                           (float)wd,   (float)eps, amsgrad ? 1 : 0,  maximize ? 1 : 0,
                           decoupled ? 1 : 0, dev_scalar(grad_scale, "a float32 grad_scale on the device"),
                           dev_scalar(found_inf, "a float32 found_inf on the device")};
  check(omt_fused_adam(&hp, ts.data(), (int)n, cur_stream()), decoupled ? "_fused_adamw_" : "_fused_adam_");
}

template <class LR>
void sgd_impl(at::TensorList p, at::TensorList g, at::TensorList bufs, double wd, double momentum, LR lr,
              double dampening, bool nesterov, bool maximize, bool first_step, const std::optional<Tensor>& grad_scale,
              const std::optional<Tensor>& found_inf) {
  const size_t n = p.size();
  const bool mom = momentum != 0.0;
  cover(g.size() == n && (!mom || bufs.size() == n), "tensor lists of one length");
  std::vector<omt_sgd_tensor> ts(n);
  for (size_t i = 0; i < n; ++i) {
    cover(dev_f32c(p[i]) && ordered_like(g[i], p[i]) && g[i].numel() == p[i].numel(),
          "contiguous float32 device tensors");
    if (mom)
      cover(ordered_like(bufs[i], p[i]) && bufs[i].numel() == p[i].numel(), "contiguous float32 momentum buffers");
    ts[i] = omt_sgd_tensor{fpm(p[i]), fpm(g[i]), mom ? fpm(bufs[i]) : nullptr, p[i].numel()};
  }
  const Lr l = lr_of(lr);
  const omt_sgd_params hp{l.v,
                          l.dev,
                          (float)momentum,
                          (float)dampening,
                          (float)wd,
                          nesterov ? 1 : 0,
                          maximize ? 1 : 0,
                          first_step ? 1 : 0,
                          dev_scalar(grad_scale, "a float32 grad_scale on the device"),
                          dev_scalar(found_inf, "a float32 found_inf on the device")};
  check(omt_fused_sgd(&hp, ts.data(), (int)n, cur_stream()), "_fused_sgd_");
}

#define OMT_ADAM_ARGS                                                                                          \
  at::TensorList p, at::TensorList g, at::TensorList m, at::TensorList v, at::TensorList vmax,                 \
      at::TensorList steps
#define OMT_ADAM_TAIL                                                                                          \
  double beta1, double beta2, double wd, double eps, bool amsgrad, bool maximize,                              \
      const std::optional<Tensor>&grad_scale, const std::optional<Tensor>&found_inf

void fused_adam_(OMT_ADAM_ARGS, double lr, OMT_ADAM_TAIL) {
  adam_impl(p, g, m, v, vmax, steps, lr, beta1, beta2, wd, eps, amsgrad, maximize, false, grad_scale, found_inf);
}
void fused_adam_tlr(OMT_ADAM_ARGS, const Tensor& lr, OMT_ADAM_TAIL) {
  adam_impl(p, g, m, v, vmax, steps, lr, beta1, beta2, wd, eps, amsgrad, maximize, false, grad_scale, found_inf);
}
void fused_adamw_(OMT_ADAM_ARGS, double lr, OMT_ADAM_TAIL) {
  adam_impl(p, g, m, v, vmax, steps, lr, beta1, beta2, wd, eps, amsgrad, maximize, true, grad_scale, found_inf);
}
void fused_adamw_tlr(OMT_ADAM_ARGS, const Tensor& lr, OMT_ADAM_TAIL) {
  adam_impl(p, g, m, v, vmax, steps, lr, beta1, beta2, wd, eps, amsgrad, maximize, true, grad_scale, found_inf);
}
void fused_sgd_(at::TensorList p, at::TensorList g, at::TensorList bufs, double wd, double momentum, double lr,
                double dampening, bool nesterov, bool maximize, bool first_step,
                const std::optional<Tensor>& grad_scale, const std::optional<Tensor>& found_inf) {
  sgd_impl(p, g, bufs, wd, momentum, lr, dampening, nesterov, maximize, first_step, grad_scale, found_inf);
}
void fused_sgd_tlr(at::TensorList p, at::TensorList g, at::TensorList bufs, double wd, double momentum,
                   const Tensor& lr, double dampening, bool nesterov, bool maximize, bool first_step,
                   const std::optional<Tensor>& grad_scale, const std::optional<Tensor>& found_inf) {
  sgd_impl(p, g, bufs, wd, momentum, lr, dampening, nesterov, maximize, first_step, grad_scale, found_inf);
}

}  // namespace

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  HotOps(m)
      .on<at::_ops::_fused_adam_, &fused_adam_>()
      .on<at::_ops::_fused_adam__tensor_lr, &fused_adam_tlr>()
      .on<at::_ops::_fused_adamw_, &fused_adamw_>()
      .on<at::_ops::_fused_adamw__tensor_lr, &fused_adamw_tlr>()
      .on<at::_ops::_fused_sgd_, &fused_sgd_>()
      .on<at::_ops::_fused_sgd__tensor_lr, &fused_sgd_tlr>();
}

}  // namespace omt
