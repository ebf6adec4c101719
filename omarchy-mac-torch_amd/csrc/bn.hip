// BatchNorm over NCHW float32 (per-channel statistics over n * hw), HBM-bandwidth-bound wave64 kernels.
//
// Training statistics follow the reference's shifted sums (csrc/kernels/bn_stats_part.wgsl:21-31,
// bn_stats_fin.wgsl:11-22): d = x - x[n=0, c, 0], s1 = sum d, s2 = sum d^2, mean = shift + s1/m,
// var = max(s2/m - (s1/m)^2, 0) (biased), with the running-stat update rm += mom*(mean - rm),
// rv += mom*(var*m/(m-1) - rv) (csrc/nn.cpp:41-45). Each workgroup reduces one (channel, slice) of the n*hw
// elements; lanes accumulate in float64 (free on a bandwidth-bound kernel) and the slices are combined in a fixed
// order, so the statistics are deterministic. Reductions are butterfly shuffles within each wave64, then LDS across
// the four waves of a workgroup.
//
// Backward (csrc/nn.cpp:60-78, bnb_reduce.wgsl / bnb_apply.wgsl; ReLU-masked form bn_bwd_part / bn_bwd_fin /
// bn_bwd_apply of csrc/fused.cpp:86-115): gz = g (or g * [y > 0]), xhat = (x - mean) * invstd,
// dgamma = sum gz * xhat, dbeta = sum gz, gx = gamma * invstd / m * (m * gz - dbeta - xhat * dgamma).
#include "omt_internal.h"

namespace omt {

constexpr int kMaxSlices = 64;

struct Split {
  int sn, sh;      // image slices x hw slices
  int hw_chunk;    // elements of one image row handled per hw slice
};

static Split bn_split(int64_t n, int64_t c, int64_t hw) {
  // aim for ~2048 workgroups overall, each streaming at least ~4K elements
  int64_t want = cdiv(2048, c);
  int64_t by_size = (n * hw) / 4096;
  if (want > by_size) want = by_size;
  if (want > kMaxSlices) want = kMaxSlices;
  if (want < 1) want = 1;
  int64_t sn = want < n ? want : n;
  int64_t sh = want / sn;
  if (sh < 1) sh = 1;
  int64_t chunk = cdiv(hw, sh);
  chunk = cdiv(chunk, 4) * 4;
  sh = cdiv(hw, chunk);
  return {(int)sn, (int)sh, (int)chunk};
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Block-wide sum of two doubles over 256 threads; result valid in thread 0.
__device__ __forceinline__ void block_sum2(double& a, double& b) {
  __shared__ double sa[4], sb[4];
  a = wave_sum(a);
  b = wave_sum(b);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sa[wave] = a;
    sb[wave] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    a = sa[0] + sa[1] + sa[2] + sa[3];
    b = sb[0] + sb[1] + sb[2] + sb[3];
  }
}

// grid (c, sn * sh): partial shifted sums of one (channel, slice)
__global__ void __launch_bounds__(256) bn_stats_part_kernel(const float* __restrict__ x, double* __restrict__ part,
                                                            int n, int c, int hw, int sn, int sh, int chunk) {
  const int ch = blockIdx.x, s = blockIdx.y, si = s / sh, sj = s % sh;
  const float shift = x[(int64_t)ch * hw];
  const int e0 = sj * chunk, e1 = min(hw, e0 + chunk);
  double s1 = 0.0, s2 = 0.0;
  for (int nn = si; nn < n; nn += sn) {
    const float* row = x + ((int64_t)nn * c + ch) * hw;
    for (int e = e0 + threadIdx.x; e < e1; e += 256) {
      const double d = (double)(row[e] - shift);
      s1 += d;
      s2 += d * d;
    }
  }
  block_sum2(s1, s2);
  if (threadIdx.x == 0) {
    part[((int64_t)ch * gridDim.y + s) * 2] = s1;
    part[((int64_t)ch * gridDim.y + s) * 2 + 1] = s2;
  }
}

__global__ void bn_stats_fin_kernel(const float* __restrict__ x, const double* __restrict__ part, int c, int hw,
                                    int slices, double m, double momentum, double eps, const float* __restrict__ rm,
                                    const float* __restrict__ rv, float* __restrict__ save_mean,
                                    float* __restrict__ save_invstd, float* __restrict__ new_rm,
                                    float* __restrict__ new_rv) {
  const int ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= c) return;
  double s1 = 0.0, s2 = 0.0;
  for (int s = 0; s < slices; ++s) {
    s1 += part[((int64_t)ch * slices + s) * 2];
    s2 += part[((int64_t)ch * slices + s) * 2 + 1];
  }
  const double shift = (double)x[(int64_t)ch * hw];
  const double a = s1 / m, mean = shift + a;
  double var = s2 / m - a * a;
  if (var < 0.0) var = 0.0;
  save_mean[ch] = (float)mean;
  save_invstd[ch] = (float)(1.0 / sqrt(var + eps));
  if (new_rm && rm) new_rm[ch] = (float)((double)rm[ch] + momentum * (mean - (double)rm[ch]));
  if (new_rv && rv) {
    const double corr = (double)(float)(m / (m > 1.0 ? m - 1.0 : 1.0));
    new_rv[ch] = (float)((double)rv[ch] + momentum * (var * corr - (double)rv[ch]));
  }
}

// y = (x - mean[c]) * invstd[c] * gamma[c] + beta[c], optional ReLU. grid (planes, hw chunks); float4 when hw % 4 == 0.
// Eval mode passes invstd = null and the running variance in var: invstd = 1 / sqrt(var + eps).
template <bool VEC>
__global__ void __launch_bounds__(256) bn_apply_kernel(const float* __restrict__ x, const float* __restrict__ mean,
                                                       const float* __restrict__ invstd, const float* __restrict__ var,
                                                       double eps, const float* __restrict__ gamma,
                                                       const float* __restrict__ beta, float* __restrict__ y, int c,
                                                       int hw, int relu) {
  const int plane = blockIdx.x, ch = plane % c;
  const float inv = invstd ? invstd[ch] : (float)(1.0 / sqrt((double)var[ch] + eps));
  const float sc = inv * gamma[ch];
  const float sh = beta[ch] - mean[ch] * sc;
  const int64_t base = (int64_t)plane * hw;
  if (VEC) {
    const int n4 = hw >> 2;
    const float4* xv = reinterpret_cast<const float4*>(x + base);
    float4* yv = reinterpret_cast<float4*>(y + base);
    for (int e = blockIdx.y * 256 + threadIdx.x; e < n4; e += gridDim.y * 256) {
      float4 v = xv[e];
      v.x = fmaf(v.x, sc, sh);
      v.y = fmaf(v.y, sc, sh);
      v.z = fmaf(v.z, sc, sh);
      v.w = fmaf(v.w, sc, sh);
      if (relu) {
        v.x = fmaxf(v.x, 0.f);
        v.y = fmaxf(v.y, 0.f);
        v.z = fmaxf(v.z, 0.f);
        v.w = fmaxf(v.w, 0.f);
      }
      yv[e] = v;
    }
  } else {
    for (int e = blockIdx.y * 256 + threadIdx.x; e < hw; e += gridDim.y * 256) {
      float v = fmaf(x[base + e], sc, sh);
      if (relu) v = fmaxf(v, 0.f);
      y[base + e] = v;
    }
  }
}

// grid (c, slices): partial sum gz and sum gz * xhat
__global__ void __launch_bounds__(256) bn_bwd_part_kernel(const float* __restrict__ g, const float* __restrict__ x,
                                                          const float* __restrict__ ry, const float* __restrict__ mean,
                                                          const float* __restrict__ invstd, double* __restrict__ part,
                                                          int n, int c, int hw, int sn, int sh, int chunk) {
  const int ch = blockIdx.x, s = blockIdx.y, si = s / sh, sj = s % sh;
  const float mu = mean[ch], inv = invstd[ch];
  const int e0 = sj * chunk, e1 = min(hw, e0 + chunk);
  double s1 = 0.0, s2 = 0.0;
  for (int nn = si; nn < n; nn += sn) {
    const int64_t off = ((int64_t)nn * c + ch) * hw;
    for (int e = e0 + threadIdx.x; e < e1; e += 256) {
      float gz = g[off + e];
      if (ry && !(ry[off + e] > 0.f)) gz = 0.f;
      const float xhat = (x[off + e] - mu) * inv;
      s1 += (double)gz;
      s2 += (double)gz * (double)xhat;
    }
  }
  block_sum2(s1, s2);
  if (threadIdx.x == 0) {
    part[((int64_t)ch * gridDim.y + s) * 2] = s1;
    part[((int64_t)ch * gridDim.y + s) * 2 + 1] = s2;
  }
}

__global__ void bn_bwd_fin_kernel(const double* __restrict__ part, int c, int slices, double* __restrict__ tot,
                                  float* __restrict__ dgamma, float* __restrict__ dbeta) {
  const int ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= c) return;
  double s1 = 0.0, s2 = 0.0;
  for (int s = 0; s < slices; ++s) {
    s1 += part[((int64_t)ch * slices + s) * 2];
    s2 += part[((int64_t)ch * slices + s) * 2 + 1];
  }
  tot[2 * ch] = s1;
  tot[2 * ch + 1] = s2;
  if (dbeta) dbeta[ch] = (float)s1;
  if (dgamma) dgamma[ch] = (float)s2;
}

// gx = gamma * invstd / m * (m * gz - sum_gz - xhat * sum_gz_xhat) = k1 * gz - k2 - k3 * xhat
__global__ void __launch_bounds__(256) bn_bwd_apply_kernel(const float* __restrict__ g, const float* __restrict__ x,
                                                           const float* __restrict__ ry,
                                                           const float* __restrict__ mean,
                                                           const float* __restrict__ invstd,
                                                           const float* __restrict__ gamma,
                                                           const double* __restrict__ tot, float* __restrict__ gx,
                                                           int c, int hw, double m) {
  const int plane = blockIdx.x, ch = plane % c;
  const double gi = (double)gamma[ch] * (double)invstd[ch];
  const float k1 = (float)gi;
  const float k2 = (float)(gi * tot[2 * ch] / m);
  const float k3 = (float)(gi * tot[2 * ch + 1] / m);
  const float mu = mean[ch], inv = invstd[ch];
  const int64_t base = (int64_t)plane * hw;
  for (int e = blockIdx.y * 256 + threadIdx.x; e < hw; e += gridDim.y * 256) {
    float gz = g[base + e];
    if (ry && !(ry[base + e] > 0.f)) gz = 0.f;
    const float xhat = (x[base + e] - mu) * inv;
    gx[base + e] = k1 * gz - k2 - k3 * xhat;
  }
}

// grid x = plane (n * c), grid y = chunks of the plane
static dim3 apply_grid(int64_t planes, int64_t hw, int per_thread) {
  int64_t gy = cdiv(cdiv(hw, per_thread), 256);
  if (gy > 64) gy = 64;
  return dim3((unsigned)planes, (unsigned)(gy < 1 ? 1 : gy));
}

static bool bn_size_ok(int64_t n, int64_t c, int64_t hw) {
  return n >= 1 && c >= 1 && c <= 65535 && hw >= 1 && n * c < ((int64_t)1 << 31) && hw < ((int64_t)1 << 31);
}

}  // namespace omt

using namespace omt;

OMT_EXPORT size_t omt_bn_train_workspace(int64_t n, int64_t c, int64_t hw) {
  (void)n;
  (void)hw;
  return (size_t)(c * kMaxSlices * 2) * sizeof(double);
}

OMT_EXPORT int omt_bn_train_fwd(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma,
                                const float* beta, const float* running_mean, const float* running_var,
                                double momentum, double eps, int relu, float* y, float* save_mean, float* save_invstd,
                                float* new_rm, float* new_rv, void* workspace, size_t workspace_bytes, void* stream) {
  if (!x || !gamma || !beta || !y || !save_mean || !save_invstd) return fail(OMT_INVALID, "omt_bn_train_fwd: null pointer");
  if (!bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_train_fwd: size not covered");
  if (!workspace || workspace_bytes < omt_bn_train_workspace(n, c, hw))
    return fail(OMT_INVALID, "omt_bn_train_fwd: workspace too small");
  hipStream_t s = stream_of(stream);
  Split sp = bn_split(n, c, hw);
  const int slices = sp.sn * sp.sh;
  double* part = (double*)workspace;
  hipLaunchKernelGGL(bn_stats_part_kernel, dim3((unsigned)c, (unsigned)slices), dim3(256), 0, s, x, part, (int)n,
                     (int)c, (int)hw, sp.sn, sp.sh, sp.hw_chunk);
  if (int st = launch_check("bn_stats_part_kernel")) return st;
  const double m = (double)(n * hw);
  hipLaunchKernelGGL(bn_stats_fin_kernel, dim3(grid1d(c, 256)), dim3(256), 0, s, x, (const double*)part, (int)c,
                     (int)hw, slices, m, momentum, eps, running_mean, running_var, save_mean, save_invstd, new_rm,
                     new_rv);
  if (int st = launch_check("bn_stats_fin_kernel")) return st;
  const bool vec = (hw % 4) == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0;
  if (vec)
    hipLaunchKernelGGL(bn_apply_kernel<true>, apply_grid(n * c, hw, 4), dim3(256), 0, s, x, save_mean, save_invstd,
                       nullptr, eps, gamma, beta, y, (int)c, (int)hw, relu);
  else
    hipLaunchKernelGGL(bn_apply_kernel<false>, apply_grid(n * c, hw, 1), dim3(256), 0, s, x, save_mean, save_invstd,
                       nullptr, eps, gamma, beta, y, (int)c, (int)hw, relu);
  return launch_check("bn_apply_kernel");
}

OMT_EXPORT int omt_bn_eval_fwd(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma,
                               const float* beta, const float* running_mean, const float* running_var, double eps,
                               int relu, float* y, void* stream) {
  if (!x || !gamma || !beta || !running_mean || !running_var || !y)
    return fail(OMT_INVALID, "omt_bn_eval_fwd: null pointer");
  if (!bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_eval_fwd: size not covered");
  hipStream_t s = stream_of(stream);
  const bool vec = (hw % 4) == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0;
  if (vec)
    hipLaunchKernelGGL(bn_apply_kernel<true>, apply_grid(n * c, hw, 4), dim3(256), 0, s, x, running_mean, nullptr,
                       running_var, eps, gamma, beta, y, (int)c, (int)hw, relu);
  else
    hipLaunchKernelGGL(bn_apply_kernel<false>, apply_grid(n * c, hw, 1), dim3(256), 0, s, x, running_mean, nullptr,
                       running_var, eps, gamma, beta, y, (int)c, (int)hw, relu);
  return launch_check("bn_apply_kernel");
}

OMT_EXPORT size_t omt_bn_bwd_workspace(int64_t n, int64_t c, int64_t hw) {
  (void)n;
  (void)hw;
  return (size_t)(c * kMaxSlices * 2 + c * 2) * sizeof(double);
}

OMT_EXPORT int omt_bn_bwd(int64_t n, int64_t c, int64_t hw, const float* g, const float* x, const float* relu_y,
                          const float* save_mean, const float* save_invstd, const float* gamma, float* gx,
                          float* dgamma, float* dbeta, void* workspace, size_t workspace_bytes, void* stream) {
  if (!g || !x || !save_mean || !save_invstd || (gx && !gamma)) return fail(OMT_INVALID, "omt_bn_bwd: null pointer");
  if (!bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_bwd: size not covered");
  if (!workspace || workspace_bytes < omt_bn_bwd_workspace(n, c, hw))
    return fail(OMT_INVALID, "omt_bn_bwd: workspace too small");
  hipStream_t s = stream_of(stream);
  Split sp = bn_split(n, c, hw);
  const int slices = sp.sn * sp.sh;
  double* part = (double*)workspace;
  double* tot = part + c * kMaxSlices * 2;
  hipLaunchKernelGGL(bn_bwd_part_kernel, dim3((unsigned)c, (unsigned)slices), dim3(256), 0, s, g, x, relu_y,
                     save_mean, save_invstd, part, (int)n, (int)c, (int)hw, sp.sn, sp.sh, sp.hw_chunk);
  if (int st = launch_check("bn_bwd_part_kernel")) return st;
  hipLaunchKernelGGL(bn_bwd_fin_kernel, dim3(grid1d(c, 256)), dim3(256), 0, s, (const double*)part, (int)c, slices,
                     tot, dgamma, dbeta);
  if (int st = launch_check("bn_bwd_fin_kernel")) return st;
  if (gx) {
    hipLaunchKernelGGL(bn_bwd_apply_kernel, apply_grid(n * c, hw, 1), dim3(256), 0, s, g, x, relu_y, save_mean,
                       save_invstd, gamma, (const double*)tot, gx, (int)c, (int)hw, (double)(n * hw));
    if (int st = launch_check("bn_bwd_apply_kernel")) return st;
  }
  return OMT_OK;
}
