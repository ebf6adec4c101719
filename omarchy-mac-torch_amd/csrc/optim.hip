// Fused SGD and Adam / AdamW over many parameter tensors per launch (torch.optim's fused=True path: aten
// _fused_sgd_, _fused_adam_, _fused_adamw_). Reference: csrc/optim.cpp:12-67 (fused_sgd_, adam_impl), which launches
// one kernel per parameter; here a launch covers up to kOptSlots tensors, cut into chunks of kOptChunk elements, one
// chunk per workgroup, with the tensor table passed by value in the kernel arguments (so a captured graph replays the
// same launch with no host memory behind it). Step counts, a tensor learning rate, the AMP gradient scale and the
// found-inf flag are read from device memory at run time.
//
// Update rules (torch.optim semantics for float32 parameters). With grad_scale, g is divided by it and the unscaled
// gradient is stored back; found_inf == 1 skips the update; maximize negates g after that store.
//   SGD:   g += wd p; with momentum: b = g on the first step, else b = mu b + (1 - dampening) g; g = nesterov ?
//          g + mu b : b; p -= lr g.
//   Adam:  g += wd p (AdamW instead: p -= lr wd p); m = b1 m + (1 - b1) g; v = b2 v + (1 - b2) g^2; (amsgrad:
//          vmax = max(vmax, v), used for v); with bias corrections c1 = 1 - b1^t, c2 = 1 - b2^t (t the step count,
//          already incremented by the caller): p -= (lr / c1) m / (sqrt(v) / sqrt(c2) + eps).
// Memory-bound: 4 (SGD with momentum: 3) float reads and 3 writes per element, float4 where every pointer of a
// tensor is 16-byte aligned.
#include <cmath>

#include "omt_internal.h"

namespace omt {

constexpr int kOptSlots = 32;    // tensors per launch (the table: 2.2 KB of kernel arguments)
constexpr int kOptChunk = 8192;  // elements per workgroup (256 threads x 8 float4)
constexpr int kOptThreads = 256;

struct AdamSlot {
  float *p, *g, *m, *v, *vmax;
  const float* step;
  int64_t n;
  int vec;  // every pointer 16-byte aligned: float4 body
};
struct AdamTable {
  AdamSlot s[kOptSlots];
  int first[kOptSlots + 1];  // first chunk of each slot; first[count] = chunks of the launch
  int count;
};
struct AdamHyper {
  float lr;
  const float* lr_dev;
  float beta1, beta2, wd, eps;
  int amsgrad, maximize, decoupled;
  const float* grad_scale;
  const float* found_inf;
};

struct SgdSlot {
  float *p, *g, *b;
  int64_t n;
  int vec;
};
struct SgdTable {
  SgdSlot s[kOptSlots];
  int first[kOptSlots + 1];
  int count;
};
static_assert(sizeof(AdamTable) + sizeof(SgdTable) < 4096, "the tables travel in the kernel arguments");
struct SgdHyper {
  float lr;
  const float* lr_dev;
  float momentum, dampening, wd;
  int nesterov, maximize, first_step;
  const float* grad_scale;
  const float* found_inf;
};

// slot of workgroup `chunk` (wave-uniform scan over at most kOptSlots entries)
template <class Table>
__device__ __forceinline__ int slot_of(const Table& t, int chunk) {
  int s = 0;
  while (s + 1 < t.count && chunk >= t.first[s + 1]) ++s;
  return s;
}

struct AdamScalars {
  float lr, step_size, c2_sqrt, inv_scale;
};

__device__ __forceinline__ void adam_one(float& p, float& g, float& m, float& v, float& vmax, const AdamHyper& h,
                                         const AdamScalars& k) {
  if (h.grad_scale) g *= k.inv_scale;
  float gg = h.maximize ? -g : g;
  if (h.wd != 0.f) {
    if (h.decoupled)
      p -= k.lr * h.wd * p;
    else
      gg += h.wd * p;
  }
  m = h.beta1 * m + (1.f - h.beta1) * gg;
  v = h.beta2 * v + (1.f - h.beta2) * gg * gg;
  float vd = v;
  if (h.amsgrad) {
    vd = fmaxf(vmax, v);
    vmax = vd;
  }
  p -= k.step_size * m / (sqrtf(vd) / k.c2_sqrt + h.eps);
}

__global__ void __launch_bounds__(kOptThreads) fused_adam_kernel(const AdamTable t, const AdamHyper h) {
  if (h.found_inf && *h.found_inf == 1.f) return;
  const int chunk = (int)blockIdx.x, si = slot_of(t, chunk);
  const AdamSlot& s = t.s[si];
  const int64_t beg = (int64_t)(chunk - t.first[si]) * kOptChunk;
  const int64_t len = s.n - beg < kOptChunk ? s.n - beg : kOptChunk;
  AdamScalars k;
  k.lr = h.lr_dev ? *h.lr_dev : h.lr;
  const double step = (double)*s.step;
  const double c1 = 1.0 - pow((double)h.beta1, step), c2 = 1.0 - pow((double)h.beta2, step);
  k.step_size = (float)((double)k.lr / c1);
  k.c2_sqrt = (float)sqrt(c2);
  k.inv_scale = h.grad_scale ? 1.f / *h.grad_scale : 1.f;
  float *p = s.p + beg, *g = s.g + beg, *m = s.m + beg, *v = s.v + beg, *vm = h.amsgrad ? s.vmax + beg : nullptr;
  int64_t done = 0;
  if (s.vec) {
    const int n4 = (int)(len / 4);
#pragma unroll 4
    for (int i = threadIdx.x; i < n4; i += kOptThreads) {
      float4 P = reinterpret_cast<float4*>(p)[i], G = reinterpret_cast<float4*>(g)[i];
      float4 M = reinterpret_cast<float4*>(m)[i], V = reinterpret_cast<float4*>(v)[i];
      float4 X = vm ? reinterpret_cast<float4*>(vm)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      adam_one(P.x, G.x, M.x, V.x, X.x, h, k);
      adam_one(P.y, G.y, M.y, V.y, X.y, h, k);
      adam_one(P.z, G.z, M.z, V.z, X.z, h, k);
      adam_one(P.w, G.w, M.w, V.w, X.w, h, k);
      reinterpret_cast<float4*>(p)[i] = P;
      reinterpret_cast<float4*>(m)[i] = M;
      reinterpret_cast<float4*>(v)[i] = V;
      if (h.grad_scale) reinterpret_cast<float4*>(g)[i] = G;
      if (vm) reinterpret_cast<float4*>(vm)[i] = X;
    }
    done = (int64_t)n4 * 4;
  }
  for (int64_t i = done + threadIdx.x; i < len; i += kOptThreads) {
    float P = p[i], G = g[i], M = m[i], V = v[i], X = vm ? vm[i] : 0.f;
    adam_one(P, G, M, V, X, h, k);
    p[i] = P;
    m[i] = M;
    v[i] = V;
    if (h.grad_scale) g[i] = G;
    if (vm) vm[i] = X;
  }
}

__device__ __forceinline__ void sgd_one(float& p, float& g, float& b, bool has_b, const SgdHyper& h, float lr,
                                        float inv_scale) {
  if (h.grad_scale) g *= inv_scale;
  float gg = h.maximize ? -g : g;
  if (h.wd != 0.f) gg += h.wd * p;
  if (has_b) {
    b = h.first_step ? gg : h.momentum * b + (1.f - h.dampening) * gg;
    gg = h.nesterov ? gg + h.momentum * b : b;
  }
  p -= lr * gg;
}

__global__ void __launch_bounds__(kOptThreads) fused_sgd_kernel(const SgdTable t, const SgdHyper h) {
  if (h.found_inf && *h.found_inf == 1.f) return;
  const int chunk = (int)blockIdx.x, si = slot_of(t, chunk);
  const SgdSlot& s = t.s[si];
  const int64_t beg = (int64_t)(chunk - t.first[si]) * kOptChunk;
  const int64_t len = s.n - beg < kOptChunk ? s.n - beg : kOptChunk;
  const float lr = h.lr_dev ? *h.lr_dev : h.lr, inv_scale = h.grad_scale ? 1.f / *h.grad_scale : 1.f;
  float *p = s.p + beg, *g = s.g + beg, *b = s.b ? s.b + beg : nullptr;
  int64_t done = 0;
  if (s.vec) {
    const int n4 = (int)(len / 4);
#pragma unroll 4
    for (int i = threadIdx.x; i < n4; i += kOptThreads) {
      float4 P = reinterpret_cast<float4*>(p)[i], G = reinterpret_cast<float4*>(g)[i];
      float4 B = b ? reinterpret_cast<float4*>(b)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      sgd_one(P.x, G.x, B.x, b != nullptr, h, lr, inv_scale);
      sgd_one(P.y, G.y, B.y, b != nullptr, h, lr, inv_scale);
      sgd_one(P.z, G.z, B.z, b != nullptr, h, lr, inv_scale);
      sgd_one(P.w, G.w, B.w, b != nullptr, h, lr, inv_scale);
      reinterpret_cast<float4*>(p)[i] = P;
      if (h.grad_scale) reinterpret_cast<float4*>(g)[i] = G;
      if (b) reinterpret_cast<float4*>(b)[i] = B;
    }
    done = (int64_t)n4 * 4;
  }
  for (int64_t i = done + threadIdx.x; i < len; i += kOptThreads) {
    float P = p[i], G = g[i], B = b ? b[i] : 0.f;
    sgd_one(P, G, B, b != nullptr, h, lr, inv_scale);
    p[i] = P;
    if (h.grad_scale) g[i] = G;
    if (b) b[i] = B;
  }
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Fills tables of up to kOptSlots non-empty tensors and launches each; `fill(slot, i)` sets slot from tensor i and
// returns its element count.
template <class Table, class Fill, class Launch>
static int launch_tables(int n, Fill fill, Launch launch) {
  int i = 0;
  while (i < n) {
    Table t{};
    int64_t chunks = 0;
    while (i < n && t.count < kOptSlots) {
      const int64_t numel = fill(t.s[t.count], i++);
      if (numel <= 0) continue;
      t.first[t.count] = (int)chunks;
      chunks += cdiv(numel, kOptChunk);
      ++t.count;
      if (chunks >= (1ll << 30)) break;
    }
    if (!t.count) break;
    t.first[t.count] = (int)chunks;
    if (int st = launch(t, (unsigned)chunks)) return st;
  }
  return OMT_OK;
}

}  // namespace omt

using namespace omt;

OMT_EXPORT int omt_fused_adam(const omt_adam_params* hp, const omt_adam_tensor* ts, int n, void* stream) {
  if (!hp || (n > 0 && !ts) || n < 0) return fail(OMT_INVALID, "omt_fused_adam: null pointer or negative count");
  for (int i = 0; i < n; ++i) {
    const omt_adam_tensor& t = ts[i];
    if (t.numel < 0 || (t.numel > 0 && (!t.param || !t.grad || !t.exp_avg || !t.exp_avg_sq || !t.step ||
                                        (hp->amsgrad && !t.max_exp_avg_sq))))
      return fail(OMT_INVALID, "omt_fused_adam: tensor %d: null pointer or negative size", i);
  }
  const AdamHyper h{hp->lr,         hp->lr_dev,   hp->beta1,     hp->beta2,      hp->weight_decay, hp->eps,
                    hp->amsgrad,    hp->maximize, hp->decoupled, hp->grad_scale, hp->found_inf};
  hipStream_t s = stream_of(stream);
  return launch_tables<AdamTable>(
      n,
      [&](AdamSlot& a, int i) {
        const omt_adam_tensor& t = ts[i];
        a = AdamSlot{t.param, t.grad, t.exp_avg, t.exp_avg_sq, hp->amsgrad ? t.max_exp_avg_sq : nullptr, t.step,
                     t.numel, 0};
        a.vec = al16(a.p) && al16(a.g) && al16(a.m) && al16(a.v) && (!a.vmax || al16(a.vmax));
        return t.numel;
      },
      [&](const AdamTable& t, unsigned chunks) {
        hipLaunchKernelGGL(fused_adam_kernel, dim3(chunks), dim3(kOptThreads), 0, s, t, h);
        return launch_check("fused_adam_kernel");
      });
}

OMT_EXPORT int omt_fused_sgd(const omt_sgd_params* hp, const omt_sgd_tensor* ts, int n, void* stream) {
  if (!hp || (n > 0 && !ts) || n < 0) return fail(OMT_INVALID, "omt_fused_sgd: null pointer or negative count");
  for (int i = 0; i < n; ++i) {
    const omt_sgd_tensor& t = ts[i];
    if (t.numel < 0 || (t.numel > 0 && (!t.param || !t.grad || (hp->momentum != 0.f && !t.momentum_buffer))))
      return fail(OMT_INVALID, "omt_fused_sgd: tensor %d: null pointer or negative size", i);
  }
  const SgdHyper h{hp->lr,       hp->lr_dev,   hp->momentum,   hp->dampening,  hp->weight_decay,
                   hp->nesterov, hp->maximize, hp->first_step, hp->grad_scale, hp->found_inf};
  hipStream_t s = stream_of(stream);
  return launch_tables<SgdTable>(
      n,
      [&](SgdSlot& a, int i) {
        const omt_sgd_tensor& t = ts[i];
        a = SgdSlot{t.param, t.grad, hp->momentum != 0.f ? t.momentum_buffer : nullptr, t.numel, 0};
        a.vec = al16(a.p) && al16(a.g) && (!a.b || al16(a.b));
        return t.numel;
      },
      [&](const SgdTable& t, unsigned chunks) {
        hipLaunchKernelGGL(fused_sgd_kernel, dim3(chunks), dim3(kOptThreads), 0, s, t, h);
        return launch_check("fused_sgd_kernel");
      });
}
