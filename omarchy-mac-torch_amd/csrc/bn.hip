// BatchNorm over NCHW float32 (per-channel statistics over n * hw), HBM-bandwidth-bound wave64 kernels.
//
// Training statistics follow the reference's shifted sums (csrc/kernels/bn_stats_part.wgsl:21-31,
// bn_stats_fin.wgsl:11-22): d = x - x[n=0, c, 0], s1 = sum d, s2 = sum d^2, mean = shift + s1/m,
// var = max(s2/m - (s1/m)^2, 0) (biased), with the running-stat update rm += mom*(mean - rm),
// rv += mom*(var*m/(m-1) - rv) (csrc/nn.cpp:41-45). A channel's n*hw elements are numbered as VEC-wide vectors
// v = (image, position) (float4 when hw % 4 == 0) and cut into contiguous slices; each workgroup reduces one
// (channel, slice) with four vector loads in flight per thread; lanes accumulate in float64 (free on a
// bandwidth-bound kernel) and the slices are combined in a fixed order, so the statistics are deterministic.
// Reductions are butterfly shuffles within each wave64, then LDS across the four waves of a workgroup.
//
// Backward (csrc/nn.cpp:60-78, bnb_reduce.wgsl / bnb_apply.wgsl; ReLU-masked form bn_bwd_part / bn_bwd_fin /
// bn_bwd_apply of csrc/fused.cpp:86-115): gz = g (or g * [y > 0]), xhat = (x - mean) * invstd,
// dgamma = sum gz * xhat, dbeta = sum gz, gx = gamma * invstd / m * (m * gz - dbeta - xhat * dgamma).
#include "omt_internal.h"
#include "slice_sum.h"

namespace omt {

constexpr int kMaxSlices = 64;

// Per-channel vector numbering and slicing of the reductions.
struct Split {
  int vec;        // 4 (float4) when hw % 4 == 0, else 1
  int hwv;        // vectors per image plane
  int nv;         // vectors per channel: n * hwv
  int slices;     // slices per channel
  int per_slice;  // vectors per slice
  FastDiv div_hwv;
};

// ~1024 workgroups overall (four per CU), each at least 1024 vectors (four per thread) unless the channel is smaller.
static Split bn_split(int64_t n, int64_t c, int64_t hw, bool aligned) {
  Split sp;
  sp.vec = (hw % 4 == 0 && aligned) ? 4 : 1;
  sp.hwv = (int)(hw / sp.vec);
  sp.nv = (int)(n * sp.hwv);
  int64_t want = cdiv(1024, c);
  const int64_t by_size = cdiv(sp.nv, 1024);
  if (want > by_size) want = by_size;
  if (want > kMaxSlices) want = kMaxSlices;
  if (want < 1) want = 1;
  sp.per_slice = (int)cdiv(sp.nv, want);
  sp.slices = (int)cdiv(sp.nv, sp.per_slice);
  sp.div_hwv = make_fastdiv((uint32_t)sp.hwv);
  return sp;
}

template <int VEC>
struct VecT;
template <>
struct VecT<4> {
  using T = float4;
};
template <>
struct VecT<1> {
  using T = float;
};
__device__ __forceinline__ float vget(const float4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
__device__ __forceinline__ float vget(const float& v, int) { return v; }
__device__ __forceinline__ void vset(float4& v, int i, float f) {
  if (i == 0) v.x = f; else if (i == 1) v.y = f; else if (i == 2) v.z = f; else v.w = f;
}
__device__ __forceinline__ void vset(float& v, int, float f) { v = f; }
__device__ __forceinline__ void vadd(float4& a, const float4& b) { a.x += b.x, a.y += b.y, a.z += b.z, a.w += b.w; }
__device__ __forceinline__ void vadd(float& a, const float& b) { a += b; }

// Element offset of vector v of channel ch.
__device__ __forceinline__ int64_t voffset(int v, int ch, int c, int hw, int hwv, const FastDiv& div_hwv, int vec) {
  const int nn = (int)fdiv((uint32_t)v, div_hwv), e = v - nn * hwv;
  return ((int64_t)nn * c + ch) * hw + (int64_t)e * vec;
}

// Block-wide sum of two doubles over NT threads (the wave sums added in wave order); result valid in thread 0.
template <int NT = 256>
__device__ __forceinline__ void block_sum2(double& a, double& b) {
  constexpr int NW = NT / 64;
  __shared__ double sa[NW], sb[NW];
  a = wave_sum(a);
  b = wave_sum(b);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sa[wave] = a;
    sb[wave] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    if constexpr (NW == 4) {  // the 256-thread order, kept as it was
      a = sa[0] + sa[1] + sa[2] + sa[3];
      b = sb[0] + sb[1] + sb[2] + sb[3];
    } else {
      a = sa[0], b = sb[0];
      for (int w = 1; w < NW; ++w) a += sa[w], b += sb[w];
    }
  }
}

// grid (c, slices): partial shifted sums of one (channel, slice)
template <int VEC>
__global__ void __launch_bounds__(256) bn_stats_part_kernel(const float* __restrict__ x, double* __restrict__ part,
                                                            int c, int hw, const Split sp) {
  using V = typename VecT<VEC>::T;
  const int ch = blockIdx.x, s = blockIdx.y;
  const float shift = x[(int64_t)ch * hw];
  const int v0 = s * sp.per_slice, v1 = min(sp.nv, v0 + sp.per_slice);
  double s1 = 0.0, s2 = 0.0;
  for (int v = v0 + (int)threadIdx.x; v < v1; v += 4 * 256) {
    V r[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int vv = v + u * 256;
      if (vv < v1) {
        r[u] = *reinterpret_cast<const V*>(x + voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC));
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) vset(r[u], i, shift);  // contributes d = 0
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const double d = (double)(vget(r[u], i) - shift);
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

// A channel's statistics from its shifted sums over m elements: mean, biased variance and invstd; `write` also
// stores save_mean / save_invstd and the running-statistics update (new_rm / new_rv may alias rm / rv).
struct BnStats {
  float mean, invstd;
};
__device__ __forceinline__ BnStats bn_finalize(double s1, double s2, double shift, double m, double momentum,
                                               double eps, const float* rm, const float* rv, float* save_mean,
                                               float* save_invstd, float* new_rm, float* new_rv, int ch, bool write) {
  const double a = s1 / m, mean = shift + a;
  double var = s2 / m - a * a;
  if (var < 0.0) var = 0.0;
  const BnStats st{(float)mean, (float)(1.0 / sqrt(var + eps))};
  if (write) {
    save_mean[ch] = st.mean;
    save_invstd[ch] = st.invstd;
    if (new_rm && rm) new_rm[ch] = (float)((double)rm[ch] + momentum * (mean - (double)rm[ch]));
    if (new_rv && rv) {
      const double corr = (double)(float)(m / (m > 1.0 ? m - 1.0 : 1.0));
      new_rv[ch] = (float)((double)rv[ch] + momentum * (var * corr - (double)rv[ch]));
    }
  }
  return st;
}

__global__ void bn_stats_fin_kernel(const float* __restrict__ x, const double* __restrict__ part, int c, int hw,
                                    int slices, double m, double momentum, double eps, const float* rm,
                                    const float* rv, float* __restrict__ save_mean, float* __restrict__ save_invstd,
                                    float* new_rm, float* new_rv) {
  const int ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= c) return;
  double s1 = 0.0, s2 = 0.0;
  for (int s = 0; s < slices; ++s) {
    s1 += part[((int64_t)ch * slices + s) * 2];
    s2 += part[((int64_t)ch * slices + s) * 2 + 1];
  }
  bn_finalize(s1, s2, (double)x[(int64_t)ch * hw], m, momentum, eps, rm, rv, save_mean, save_invstd, new_rm, new_rv,
              ch, true);
}

// bn_stats_fin_kernel for unshifted partial sums (the epilogue statistics reduced by bn_stats_groups_kernel).
__global__ void bn_stats_shift0_fin_kernel(const double* __restrict__ part, int c, int slices, double m,
                                           double momentum, double eps, const float* rm, const float* rv,
                                           float* __restrict__ save_mean, float* __restrict__ save_invstd,
                                           float* new_rm, float* new_rv) {
  const int ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= c) return;
  double s1 = 0.0, s2 = 0.0;
  for (int s = 0; s < slices; ++s) {
    s1 += part[((int64_t)ch * slices + s) * 2];
    s2 += part[((int64_t)ch * slices + s) * 2 + 1];
  }
  bn_finalize(s1, s2, 0.0, m, momentum, eps, rm, rv, save_mean, save_invstd, new_rm, new_rv, ch, true);
}

// The slices' partial sums of channel ch summed in slice order by thread 0 (every lane of the first wave loads one
// slice's pair first, so the loads overlap). Valid in thread 0 after the call; all threads must call it.
__device__ __forceinline__ void bn_sum_slices(const double* __restrict__ part, int ch, int slices, double& s1,
                                              double& s2) {
  __shared__ double ps[kMaxSlices][2];
  if ((int)threadIdx.x < slices) {
    ps[threadIdx.x][0] = part[((int64_t)ch * slices + threadIdx.x) * 2];
    ps[threadIdx.x][1] = part[((int64_t)ch * slices + threadIdx.x) * 2 + 1];
  }
  __syncthreads();
  s1 = 0.0, s2 = 0.0;
  if (threadIdx.x == 0)
    for (int s = 0; s < slices; ++s) {
      s1 += ps[s][0];
      s2 += ps[s][1];
    }
}

// y = act((x - mean[c]) * invstd[c] * gamma[c] + beta[c] (+ res)) (act: OMT_ACT_*; zo, when set, receives the value
// before the activation). grid (planes, hw chunks); float4 when hw % 4 == 0. Eval mode passes invstd = null and the
// running variance in var: invstd = 1 / sqrt(var + eps).
template <bool VEC>
__global__ void __launch_bounds__(256) bn_apply_kernel(const float* __restrict__ x, const float* __restrict__ mean,
                                                       const float* __restrict__ invstd, const float* __restrict__ var,
                                                       double eps, const float* __restrict__ gamma,
                                                       const float* __restrict__ beta, const float* __restrict__ res,
                                                       float* __restrict__ y, int c, int hw, int relu,
                                                       float* __restrict__ zo = nullptr) {
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
      if (res) {
        const float4 r = reinterpret_cast<const float4*>(res + base)[e];
        v.x += r.x;
        v.y += r.y;
        v.z += r.z;
        v.w += r.w;
      }
      if (zo) reinterpret_cast<float4*>(zo + base)[e] = v;
      if (relu) {
        v.x = bn_act(v.x, relu);
        v.y = bn_act(v.y, relu);
        v.z = bn_act(v.z, relu);
        v.w = bn_act(v.w, relu);
      }
      yv[e] = v;
    }
  } else {
    for (int e = blockIdx.y * 256 + threadIdx.x; e < hw; e += gridDim.y * 256) {
      float v = fmaf(x[base + e], sc, sh);
      if (res) v += res[base + e];
      if (zo) zo[base + e] = v;
      y[base + e] = bn_act(v, relu);
    }
  }
}

// Plane and chunk of a training-apply workgroup (1-D grid). Forward order (rev = 0): planes fastest, then chunks, the
// order of a (planes, chunks) grid, which puts a workgroup on the XCD (workgroup id mod 8) whose L2 holds its plane
// from the reduction pass when the channels are a multiple of 8 (that pass's workgroup (channel, slice) has id
// slice * c + channel): what tensors that fit the L2s want. Reverse order (rev = 1, large tensors): the planes last to
// first, each plane's chunks together; the reduction pass read the planes first to last, so the apply starts on what
// is most likely still in the memory-side cache. Measured (b256 x 64 x 56^2 backward 275 -> 256 us; at 128 x 32 x
// 32^2, 16 MB, the forward order is faster: 10.7 against 12.8 us).
__device__ __forceinline__ int apply_plane(int planes, int chunks, int rev, int& chunk) {
  const int q = (int)blockIdx.x;
  if (rev) {
    const int p = q / chunks;
    chunk = q - p * chunks;
    return planes - 1 - p;
  }
  chunk = q / planes;
  return q - chunk * planes;
}
// Tensors from this size up take the reverse apply order.
constexpr int64_t kRevApplyBytes = (int64_t)64 << 20;

// Training apply with the finalize folded in (one launch fewer): every workgroup derives its channel's mean and
// invstd from the statistics partials with bn_stats_fin_kernel's arithmetic (so all of a channel's workgroups get the
// same values), and the channel's first workgroup (image 0, chunk 0) also writes save_mean / save_invstd and the
// running statistics. A thread's first vector is loaded before the partials are summed. Plane order: apply_plane.
template <bool VEC>
__global__ void __launch_bounds__(256) bn_train_apply_kernel(const float* __restrict__ x, const double* __restrict__ part,
                                                             int slices, double m, double momentum, double eps,
                                                             const float* rm, const float* rv,
                                                             float* __restrict__ save_mean,
                                                             float* __restrict__ save_invstd, float* new_rm,
                                                             float* new_rv, const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             const float* __restrict__ res, float* __restrict__ y,
                                                             int c, int hw, int relu, int planes, int chunks,
                                                             int rev, int shift0 = 0, float* __restrict__ zo = nullptr) {
  __shared__ float coef[2];
  int chunk;
  const int plane = apply_plane(planes, chunks, rev, chunk), ch = plane % c;
  const int64_t base = (int64_t)plane * hw;
  const int nv = VEC ? hw >> 2 : hw, e0 = chunk * 256 + threadIdx.x, stride = chunks * 256;
  float4 first = make_float4(0.f, 0.f, 0.f, 0.f);
  if (e0 < nv) {
    if (VEC) first = reinterpret_cast<const float4*>(x + base)[e0];
    else first.x = x[base + e0];
  }
  double s1, s2;
  bn_sum_slices(part, ch, slices, s1, s2);
  if (threadIdx.x == 0) {
    const BnStats st = bn_finalize(s1, s2, shift0 ? 0.0 : (double)x[(int64_t)ch * hw], m, momentum, eps, rm, rv,
                                   save_mean, save_invstd, new_rm, new_rv, ch, plane < c && chunk == 0);
    const float sc = st.invstd * gamma[ch];
    coef[0] = sc;
    coef[1] = beta[ch] - st.mean * sc;
  }
  __syncthreads();
  const float sc = coef[0], sh = coef[1];
  for (int e = e0; e < nv; e += stride) {
    if (VEC) {
      float4 v = e == e0 ? first : reinterpret_cast<const float4*>(x + base)[e];
      v.x = fmaf(v.x, sc, sh);
      v.y = fmaf(v.y, sc, sh);
      v.z = fmaf(v.z, sc, sh);
      v.w = fmaf(v.w, sc, sh);
      if (res) {
        const float4 r = reinterpret_cast<const float4*>(res + base)[e];
        v.x += r.x;
        v.y += r.y;
        v.z += r.z;
        v.w += r.w;
      }
      if (zo) reinterpret_cast<float4*>(zo + base)[e] = v;
      if (relu) {
        v.x = bn_act(v.x, relu);
        v.y = bn_act(v.y, relu);
        v.z = bn_act(v.z, relu);
        v.w = bn_act(v.w, relu);
      }
      reinterpret_cast<float4*>(y + base)[e] = v;
    } else {
      float v = fmaf(e == e0 ? first.x : x[base + e], sc, sh);
      if (res) v += res[base + e];
      if (zo) zo[base + e] = v;
      y[base + e] = bn_act(v, relu);
    }
  }
}

// Small planes: the same affine map over a flat range of VEC-wide vectors, channel = (vector / hwv) mod c.
template <int VEC>
__global__ void __launch_bounds__(256) bn_apply_flat_kernel(const float* __restrict__ x, const float* __restrict__ mean,
                                                            const float* __restrict__ invstd,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ beta,
                                                            const float* __restrict__ res, float* __restrict__ y,
                                                            int64_t total_v, FastDiv div_hwv, FastDiv div_c, int c,
                                                            int relu, float* __restrict__ zo = nullptr) {
  using V = typename VecT<VEC>::T;
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < total_v; i += (int64_t)gridDim.x * 256) {
    const uint32_t plane = fdiv((uint32_t)i, div_hwv), ch = plane - fdiv(plane, div_c) * (uint32_t)c;
    const float sc = invstd[ch] * gamma[ch];
    const float sh = beta[ch] - mean[ch] * sc;
    V v = reinterpret_cast<const V*>(x)[i];
    V r, z;
    if (res) r = reinterpret_cast<const V*>(res)[i];
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float f = fmaf(vget(v, e), sc, sh);
      if (res) f += vget(r, e);
      vset(z, e, f);
      vset(v, e, bn_act(f, relu));
    }
    if (zo) reinterpret_cast<V*>(zo)[i] = z;
    reinterpret_cast<V*>(y)[i] = v;
  }
}

// grid (c, slices): partial sum gz and sum gz * xhat. RES: the incoming gradient is g + g2 (a residual branch's
// gradient added before the ReLU mask).
template <int VEC, bool RES>
__global__ void __launch_bounds__(256) bn_bwd_part_kernel(const float* __restrict__ g, const float* __restrict__ g2,
                                                          const float* __restrict__ x,
                                                          const float* __restrict__ ry, const float* __restrict__ mean,
                                                          const float* __restrict__ invstd, double* __restrict__ part,
                                                          int c, int hw, const Split sp, int act) {
  using V = typename VecT<VEC>::T;
  const int ch = blockIdx.x, s = blockIdx.y;
  const float mu = mean[ch], inv = invstd[ch];
  const int v0 = s * sp.per_slice, v1 = min(sp.nv, v0 + sp.per_slice);
  double s1 = 0.0, s2 = 0.0;
  for (int v = v0 + (int)threadIdx.x; v < v1; v += 4 * 256) {
    V rg[4], rx[4], rr[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int vv = v + u * 256;
      if (vv < v1) {
        const int64_t off = voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC);
        rg[u] = *reinterpret_cast<const V*>(g + off);
        if (RES && g2) vadd(rg[u], *reinterpret_cast<const V*>(g2 + off));
        rx[u] = *reinterpret_cast<const V*>(x + off);
        if (ry) rr[u] = *reinterpret_cast<const V*>(ry + off);
      } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          vset(rg[u], i, 0.f);  // gz = 0 contributes nothing
          vset(rx[u], i, mu);
          vset(rr[u], i, 1.f);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        float gz = vget(rg[u], i);
        if (ry) gz = bn_act_grad(gz, vget(rr[u], i), act);
        const float xhat = (vget(rx[u], i) - mu) * inv;
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

// The per-channel constants of the input-gradient map from sum gz (s1) and sum gz * xhat (s2):
// k = {gamma * invstd, gamma * invstd * s1 / m, gamma * invstd * s2 / m, mean, invstd}.
__device__ __forceinline__ void bn_bwd_consts(double s1, double s2, double m, float gamma, float mean, float invstd,
                                              float* k) {
  const double gi = (double)gamma * (double)invstd;
  k[0] = (float)gi;
  k[1] = (float)(gi * s1 / m);
  k[2] = (float)(gi * s2 / m);
  k[3] = mean;
  k[4] = invstd;
}

__global__ void bn_bwd_fin_kernel(const double* __restrict__ part, int c, int slices, const float* __restrict__ mean,
                                  const float* __restrict__ invstd, const float* __restrict__ gamma, double m,
                                  float* __restrict__ kc, float* __restrict__ dgamma, float* __restrict__ dbeta) {
  const int ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= c) return;
  double s1 = 0.0, s2 = 0.0;
  for (int s = 0; s < slices; ++s) {
    s1 += part[((int64_t)ch * slices + s) * 2];
    s2 += part[((int64_t)ch * slices + s) * 2 + 1];
  }
  if (dbeta) dbeta[ch] = (float)s1;
  if (dgamma) dgamma[ch] = (float)s2;
  if (gamma) bn_bwd_consts(s1, s2, m, gamma[ch], mean[ch], invstd[ch], kc + ch * 5);
}

// gx = gamma * invstd / m * (m * gz - sum_gz - xhat * sum_gz_xhat) = k1 * gz - k2 - k3 * xhat, with the per-channel
// constants k1..k3 (and mean, invstd) precomputed by bn_bwd_fin_kernel into kc[ch][5].
__device__ __forceinline__ float bwd_elem(float gz, float xv, float r, bool masked, const float* k) {
  if (masked && !(r > 0.f)) gz = 0.f;
  const float xhat = (xv - k[3]) * k[4];
  return k[0] * gz - k[1] - k[2] * xhat;
}

// Vector i of the backward map: gx (and, RES, the masked incoming gradient gz = (g + g2) [y > 0]).
template <int VEC, bool RES>
__device__ __forceinline__ void bwd_vec(const float* __restrict__ g, const float* __restrict__ g2,
                                        const float* __restrict__ x, const float* __restrict__ ry, const float* k,
                                        float* __restrict__ gx, float* __restrict__ gzo, int64_t i, int act) {
  using V = typename VecT<VEC>::T;
  V vg = reinterpret_cast<const V*>(g)[i];
  if (RES && g2) vadd(vg, reinterpret_cast<const V*>(g2)[i]);
  const V vx = reinterpret_cast<const V*>(x)[i];
  V vr = vg;
  if (ry) vr = reinterpret_cast<const V*>(ry)[i];
  V o, z;
#pragma unroll
  for (int e = 0; e < VEC; ++e) {
    float gz = vget(vg, e);
    if (ry) gz = bn_act_grad(gz, vget(vr, e), act);
    vset(z, e, gz);
    vset(o, e, bwd_elem(gz, vget(vx, e), 1.f, false, k));
  }
  if (gx) reinterpret_cast<V*>(gx)[i] = o;
  if (RES) reinterpret_cast<V*>(gzo)[i] = z;
}

// grid x = plane (n * c), grid y = chunks of the plane
template <int VEC, bool RES>
__global__ void __launch_bounds__(256) bn_bwd_apply_kernel(const float* __restrict__ g, const float* __restrict__ g2,
                                                           const float* __restrict__ x,
                                                           const float* __restrict__ ry, const float* __restrict__ kc,
                                                           float* __restrict__ gx, float* __restrict__ gzo, int c,
                                                           int hwv, int act) {
  const int plane = blockIdx.x, ch = plane % c;
  float k[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) k[i] = kc[ch * 5 + i];
  const int64_t base = (int64_t)plane * hwv;
  for (int e = blockIdx.y * 256 + threadIdx.x; e < hwv; e += gridDim.y * 256)
    bwd_vec<VEC, RES>(g, g2, x, ry, k, gx, gzo, base + e, act);
}

// bn_bwd_apply_kernel with the finalize folded in (one launch fewer): every workgroup derives its channel's constants
// from the partials with bn_bwd_fin_kernel's arithmetic, and the channel's first workgroup (image 0, chunk 0) writes
// dgamma / dbeta. Plane order: apply_plane.
template <int VEC, bool RES>
__global__ void __launch_bounds__(256) bn_bwd_train_apply_kernel(const float* __restrict__ g,
                                                                 const float* __restrict__ g2,
                                                                 const float* __restrict__ x,
                                                                 const float* __restrict__ ry,
                                                                 const double* __restrict__ part, int slices, double m,
                                                                 const float* __restrict__ mean,
                                                                 const float* __restrict__ invstd,
                                                                 const float* __restrict__ gamma,
                                                                 float* __restrict__ dgamma, float* __restrict__ dbeta,
                                                                 float* __restrict__ gx, float* __restrict__ gzo, int c,
                                                                 int hwv, int planes, int chunks, int rev, int act) {
  __shared__ float kc[5];
  int chunk;
  const int plane = apply_plane(planes, chunks, rev, chunk), ch = plane % c;
  double s1, s2;
  bn_sum_slices(part, ch, slices, s1, s2);
  if (threadIdx.x == 0) {
    if (plane < c && chunk == 0) {
      if (dbeta) dbeta[ch] = (float)s1;
      if (dgamma) dgamma[ch] = (float)s2;
    }
    bn_bwd_consts(s1, s2, m, gamma[ch], mean[ch], invstd[ch], kc);
  }
  __syncthreads();
  float k[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) k[i] = kc[i];
  const int64_t base = (int64_t)plane * hwv;
  for (int e = chunk * 256 + threadIdx.x; e < hwv; e += chunks * 256)
    bwd_vec<VEC, RES>(g, g2, x, ry, k, gx, gzo, base + e, act);
}

// Small planes: flat over VEC-wide vectors.
template <int VEC, bool RES>
__global__ void __launch_bounds__(256) bn_bwd_apply_flat_kernel(const float* __restrict__ g,
                                                                const float* __restrict__ g2,
                                                                const float* __restrict__ x,
                                                                const float* __restrict__ ry,
                                                                const float* __restrict__ kc, float* __restrict__ gx,
                                                                float* __restrict__ gzo, int64_t total_v,
                                                                FastDiv div_hwv, FastDiv div_c, int c, int act) {
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < total_v; i += (int64_t)gridDim.x * 256) {
    const uint32_t plane = fdiv((uint32_t)i, div_hwv), ch = plane - fdiv(plane, div_c) * (uint32_t)c;
    float k[5];
#pragma unroll
    for (int j = 0; j < 5; ++j) k[j] = kc[ch * 5 + j];
    bwd_vec<VEC, RES>(g, g2, x, ry, k, gx, gzo, i, act);
  }
}

// ---- one launch per call for small channels ---------------------------------------------------------------------
// A channel of at most kFusedMax elements is reduced, finalized and mapped by one workgroup, in one kernel instead of
// three launches. Each thread loads its share of the channel once, every load in flight together, and keeps it in
// registers for the apply pass (at most kFusedMax / 256 floats per operand). The finalize and apply arithmetic is that
// of the split kernels above, so both paths agree to the float64 summation order.
constexpr int64_t kFusedMax = 8192;
// Channels of at most kFusedSmall elements run the same kernels sized for that (MAXE): a quarter of the registers per
// operand, so every channel's workgroup is resident at once (the 8192-element variants hold 2-3 waves per SIMD,
// leaving ResNet-18's 512-channel layers and MobileNet's 576-channel 7x7 layers two rounds of workgroups). Unused
// register slots hold values that add exact zeros, so both sizes give the same results.
constexpr int64_t kFusedSmall = 2048;
// Channels of up to kFusedLarge elements run the same one-launch kernels with 1024 threads (16 waves) per workgroup,
// at most 32 floats per thread (MobileNetV3's 28x28 layers at batch 32, 25088 elements, otherwise two or three
// launches: forward 11.5 against 16 us; backward 9-11 against 14.5 us at 24-40 channels, 19.5-20 against 21 us at
// 88-96, where one CU's bandwidth per channel bounds it). The backward holds three operands: up to kFusedLargeBwd elements, float4
// vectors only (28 floats per operand in the 128 registers a thread of a 1024-thread workgroup has; the scalar form
// would spill). The BatchNorm + max pool keeps its two launches above kFusedMax: the pool pass of one workgroup per
// channel, reading its outputs back, took twice as long as the split apply + pool.
constexpr int64_t kFusedLarge = 32768, kFusedLargeBwd = 28672;
constexpr int kFusedLargeThreads = 1024;
// and channels of kFusedSmall / 2 .. kFusedSmall elements with 16-byte vectors 512-thread ones (one vector each)
constexpr int kFusedSmallThreads = 512;
// Channels of kFusedSmall .. kFusedMax elements with 16-byte vectors take 1024-thread workgroups too (two float4 per
// thread and operand): a workgroup per channel is one load -> reduce -> apply chain, and with a few hundred channels
// there is about one per CU, whose loads in flight the four times more threads multiply.

// PARTS: x holds `slices` convolution partials of pstride elements each; every element is summed over them in slice
// order (the convolution slice sum's order, so xo, written with the sums, equals the summed convolution output).
// Max pooling of a BatchNorm's output inside its apply pass (BatchNorm -> activation -> max pool: the ResNet stem,
// PlainCNN's blocks): window kh x kw, stride (sh, sw), padding (ph, pw), no dilation, over planes of h x w.
struct PoolArgs {
  float* out;
  int64_t* idx;
  int h, w, oh, ow, kh, kw, sh, sw, ph, pw;
};

// The maximum of v(row, col) over pooled output (oy, ox)'s window and its flat in-plane index: the first maximum in
// row-major order wins ties and a NaN replaces the running maximum (omt_maxpool_fwd's rule, so the values and indices
// equal that op's over the same plane).
template <class F>
__device__ __forceinline__ void pool_window(const PoolArgs& pa, int oy, int ox, F v, float& best, int& bi) {
  best = -INFINITY;
  bi = -1;
  for (int ky = 0; ky < pa.kh; ++ky) {
    const int yy = oy * pa.sh - pa.ph + ky;
    if (yy < 0 || yy >= pa.h) continue;
    for (int kx = 0; kx < pa.kw; ++kx) {
      const int xx = ox * pa.sw - pa.pw + kx;
      if (xx < 0 || xx >= pa.w) continue;
      const float f = v(yy, xx);
      if (bi < 0 || f > best || isnan(f)) {
        best = f;
        bi = yy * pa.w + xx;
      }
    }
  }
}

// POOL: the channel's outputs also go to LDS, from which the workgroup max-pools every image of the channel.
template <int VEC, bool PARTS = false, bool POOL = false, int MAXE = (int)kFusedMax, int NT = 256>
__global__ void __launch_bounds__(NT) bn_train_fused_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             const float* rm, const float* rv, double momentum,
                                                             double eps, int relu, const float* __restrict__ res,
                                                             float* __restrict__ y, float* __restrict__ save_mean,
                                                             float* __restrict__ save_invstd, float* new_rm,
                                                             float* new_rv,  // may alias rm / rv
                                                             int c, int hw, const Split sp, int slices = 1,
                                                             int64_t pstride = 0, float* __restrict__ xo = nullptr,
                                                             float* __restrict__ zo = nullptr,
                                                             const PoolArgs pool = PoolArgs{}) {
  using V = typename VecT<VEC>::T;
  __shared__ float coef[2];
  // POOL: the channel's outputs, image by image, in LDS (MAXE <= kFusedMax)
  static_assert(!POOL || MAXE <= (int)kFusedMax, "the pool reads the channel from LDS");
  __shared__ float chan[POOL ? MAXE : 1];
  const int ch = blockIdx.x;
  float shift = x[(int64_t)ch * hw];
  if (PARTS)
    for (int z = 1; z < slices; ++z) shift += x[z * pstride + (int64_t)ch * hw];
  constexpr int NR = MAXE / (NT * VEC);  // vectors per thread
  V r[NR];
#pragma unroll
  for (int u = 0; u < NR; ++u) {
    const int vv = (int)threadIdx.x + u * NT;
    if (vv < sp.nv) {
      r[u] = *reinterpret_cast<const V*>(x + voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC));
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) vset(r[u], i, shift);
    }
  }
  if (PARTS && sp.nv <= NT) {  // one vector per thread: kReduceBatch slices' loads in flight, added in slice order
    const int vv = (int)threadIdx.x;
    if (vv < sp.nv) {
      const int64_t off = voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC);
      for (int z0 = 1; z0 < slices; z0 += kReduceBatch) {
        V t[kReduceBatch];
#pragma unroll
        for (int u = 0; u < kReduceBatch; ++u)
          if (z0 + u < slices) t[u] = *reinterpret_cast<const V*>(x + (z0 + u) * pstride + off);
#pragma unroll
        for (int u = 0; u < kReduceBatch; ++u)
          if (z0 + u < slices) vadd(r[0], t[u]);
      }
    }
  } else if (PARTS) {  // slice by slice, each slice's loads of all NR vectors in flight together
    for (int z = 1; z < slices; ++z) {
      V t[NR];
#pragma unroll
      for (int u = 0; u < NR; ++u) {
        const int vv = (int)threadIdx.x + u * NT;
        if (vv < sp.nv) t[u] = *reinterpret_cast<const V*>(x + z * pstride + voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC));
      }
#pragma unroll
      for (int u = 0; u < NR; ++u)
        if ((int)threadIdx.x + u * NT < sp.nv) vadd(r[u], t[u]);
    }
  }
  if (PARTS) {
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      const int vv = (int)threadIdx.x + u * NT;
      if (vv < sp.nv) *reinterpret_cast<V*>(xo + voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC)) = r[u];
    }
  }
  double s1 = 0.0, s2 = 0.0;
#pragma unroll
  for (int u = 0; u < NR; ++u)
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const double d = (double)(vget(r[u], i) - shift);
      s1 += d;
      s2 += d * d;
    }
  block_sum2<NT>(s1, s2);
  if (threadIdx.x == 0) {
    const BnStats st = bn_finalize(s1, s2, (double)shift, (double)sp.nv * VEC, momentum, eps, rm, rv, save_mean,
                                   save_invstd, new_rm, new_rv, ch, true);
    const float sc = st.invstd * gamma[ch];
    coef[0] = sc;
    coef[1] = beta[ch] - st.mean * sc;
  }
  __syncthreads();
  const float sc = coef[0], sh = coef[1];
#pragma unroll
  for (int u = 0; u < NR; ++u) {
    const int vv = (int)threadIdx.x + u * NT;
    if (vv < sp.nv) {
      const int64_t off = voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC);
      V t = r[u], q, z;
      if (res) q = *reinterpret_cast<const V*>(res + off);
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        float f = fmaf(vget(t, i), sc, sh);
        if (res) f += vget(q, i);
        vset(z, i, f);
        vset(t, i, bn_act(f, relu));
      }
      if (zo) *reinterpret_cast<V*>(zo + off) = z;
      *reinterpret_cast<V*>(y + off) = t;
      if (POOL)  // element vv VEC + i of the channel is image (vv VEC + i) / hw, position (vv VEC + i) % hw
#pragma unroll
        for (int i = 0; i < VEC; ++i) chan[vv * VEC + i] = vget(t, i);
    }
  }
  if constexpr (POOL) {
    __syncthreads();
    const int per = pool.oh * pool.ow, total = sp.nv * VEC / hw * per;
    for (int o = (int)threadIdx.x; o < total; o += NT) {
      const int img = o / per, r = o - img * per, oy = r / pool.ow, ox = r - oy * pool.ow;
      const float* cp = chan + img * hw;
      float best;
      int bi;
      pool_window(pool, oy, ox, [&](int yy, int xx) { return cp[yy * pool.w + xx]; }, best, bi);
      const int64_t oo = ((int64_t)img * c + ch) * per + r;
      pool.out[oo] = best;
      pool.idx[oo] = bi;
    }
  }
}

// The apply pass of a training BatchNorm too large for one launch, with the max pool of its output: workgroup
// (plane, run of pooled rows [r0, r1)) finalizes its channel as bn_train_apply_kernel does (the same sums and
// arithmetic), writes y over the rows the run owns (r0 sh up to r1 sh, the last run to the plane's end) and the
// run's pooled outputs, each window's values recomputed from x the way y's are.
template <bool VEC>
__global__ void __launch_bounds__(256) bn_apply_pool_kernel(const float* __restrict__ x,
                                                            const double* __restrict__ part, int slices, double m,
                                                            double momentum, double eps, const float* rm,
                                                            const float* rv, float* __restrict__ save_mean,
                                                            float* __restrict__ save_invstd, float* new_rm,
                                                            float* new_rv, const float* __restrict__ gamma,
                                                            const float* __restrict__ beta, float* __restrict__ y,
                                                            int c, int act, int planes, int rows_per_run,
                                                            const PoolArgs pa) {
  __shared__ float coef[2];
  const int q = (int)blockIdx.x, run = q / planes, plane = q - run * planes, ch = plane % c;
  const int hw = pa.h * pa.w;
  const int64_t base = (int64_t)plane * hw;
  double s1, s2;
  bn_sum_slices(part, ch, slices, s1, s2);
  if (threadIdx.x == 0) {
    const BnStats st = bn_finalize(s1, s2, (double)x[(int64_t)ch * hw], m, momentum, eps, rm, rv, save_mean,
                                   save_invstd, new_rm, new_rv, ch, plane < c && run == 0);
    const float sc = st.invstd * gamma[ch];
    coef[0] = sc;
    coef[1] = beta[ch] - st.mean * sc;
  }
  __syncthreads();
  const float sc = coef[0], sh = coef[1];
  const int r0 = run * rows_per_run, r1 = min(pa.oh, r0 + rows_per_run);
  const int y0 = r0 * pa.sh, y1 = r1 == pa.oh ? pa.h : min(pa.h, r1 * pa.sh);
  const float* xp = x + base;
  float* yp = y + base;
  if (VEC) {  // w % 4 == 0: whole rows are whole vectors
    for (int e = y0 * pa.w / 4 + (int)threadIdx.x; e < y1 * pa.w / 4; e += 256) {
      float4 v = reinterpret_cast<const float4*>(xp)[e];
      v.x = bn_act(fmaf(v.x, sc, sh), act);
      v.y = bn_act(fmaf(v.y, sc, sh), act);
      v.z = bn_act(fmaf(v.z, sc, sh), act);
      v.w = bn_act(fmaf(v.w, sc, sh), act);
      reinterpret_cast<float4*>(yp)[e] = v;
    }
  } else {
    for (int e = y0 * pa.w + (int)threadIdx.x; e < y1 * pa.w; e += 256) yp[e] = bn_act(fmaf(xp[e], sc, sh), act);
  }
  const int64_t obase = (int64_t)plane * pa.oh * pa.ow;
  for (int o = r0 * pa.ow + (int)threadIdx.x; o < r1 * pa.ow; o += 256) {
    const int oy = o / pa.ow, ox = o - oy * pa.ow;
    float best;
    int bi;
    pool_window(pa, oy, ox, [&](int yy, int xx) { return bn_act(fmaf(xp[yy * pa.w + xx], sc, sh), act); }, best, bi);
    pa.out[obase + o] = best;
    pa.idx[obase + o] = bi;
  }
}

// xo[i] = sum of the slices' element i in slice order (VEC-wide vectors; nv vectors per slice).
template <int VEC>
__global__ void __launch_bounds__(256) bn_sum_parts_kernel(const float* __restrict__ parts, int slices, int64_t nv,
                                                           float* __restrict__ xo) {
  using V = typename VecT<VEC>::T;
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < nv; i += (int64_t)gridDim.x * 256) {
    V v = reinterpret_cast<const V*>(parts)[i];
    for (int z = 1; z < slices; ++z) vadd(v, reinterpret_cast<const V*>(parts)[z * nv + i]);
    reinterpret_cast<V*>(xo)[i] = v;
  }
}

// Slice sums that ride along in another kernel's launch: workgroups past the kernel's own run them, job after job.
constexpr int kMaxSideSums = 2;
struct SideSums {
  SplitSum job[kMaxSideSums];
  int64_t end[kMaxSideSums];  // workgroups of jobs 0..k together
  int count;
};
__device__ __forceinline__ void run_side_sum(const SideSums& ss, int64_t b) {
#pragma unroll
  for (int k = 0; k < kMaxSideSums; ++k) {
    const int64_t start = k ? ss.end[k - 1] : 0;
    if (k < ss.count && b >= start && b < ss.end[k]) {
      if (ss.job[k].vec4)
        split_sum_any<4>(ss.job[k], b - start, ss.end[k] - start);
      else
        split_sum_any<1>(ss.job[k], b - start, ss.end[k] - start);
    }
  }
}

// PARTS: g holds `slices` convolution partials of pstride elements each, summed here in slice order (the convolution
// slice sum's order) before g2 is added; workgroups past the c channels run the side slice sums.
template <int VEC, bool RES, bool PARTS = false, int MAXE = (int)kFusedMax, int NT = 256>
__global__ void __launch_bounds__(NT) bn_bwd_fused_kernel(const float* __restrict__ g, const float* __restrict__ g2,
                                                           const float* __restrict__ x,
                                                           const float* __restrict__ ry,
                                                           const float* __restrict__ mean,
                                                           const float* __restrict__ invstd,
                                                           const float* __restrict__ gamma, float* __restrict__ gx,
                                                           float* __restrict__ dgamma, float* __restrict__ dbeta,
                                                           float* __restrict__ gzo, int c, int hw, const Split sp,
                                                           int act, int slices = 1, int64_t pstride = 0,
                                                           const SideSums side = SideSums{}) {
  using V = typename VecT<VEC>::T;
  __shared__ float kc[5];
  if (PARTS && (int)blockIdx.x >= c) {
    // the slice sums take kSumThreads threads; a larger workgroup's other waves end here, whole waves, and the sums'
    // barriers wait for the waves still running only
    if (NT > kSumThreads && (int)threadIdx.x >= kSumThreads) return;
    run_side_sum(side, (int64_t)blockIdx.x - c);
    return;
  }
  const int ch = blockIdx.x;
  const float mu = mean[ch], inv = invstd[ch];
  constexpr int NR = MAXE / (NT * VEC);  // vectors per thread
  V rg[NR], rx[NR], rr[NR];
#pragma unroll
  for (int u = 0; u < NR; ++u) {
    const int vv = (int)threadIdx.x + u * NT;
    if (vv < sp.nv) {
      const int64_t off = voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC);
      rg[u] = *reinterpret_cast<const V*>(g + off);
      if (RES && !PARTS && g2) vadd(rg[u], *reinterpret_cast<const V*>(g2 + off));
      rx[u] = *reinterpret_cast<const V*>(x + off);
      if (ry) rr[u] = *reinterpret_cast<const V*>(ry + off);
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        vset(rg[u], i, 0.f);
        vset(rx[u], i, mu);
        vset(rr[u], i, 1.f);
      }
    }
  }
  if (PARTS && sp.nv <= NT) {  // one vector per thread: kReduceBatch slices' loads in flight, added in slice order
    const int vv = (int)threadIdx.x;
    if (vv < sp.nv) {
      const int64_t off = voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC);
      for (int z0 = 1; z0 < slices; z0 += kReduceBatch) {
        V t[kReduceBatch];
#pragma unroll
        for (int u = 0; u < kReduceBatch; ++u)
          if (z0 + u < slices) t[u] = *reinterpret_cast<const V*>(g + (z0 + u) * pstride + off);
#pragma unroll
        for (int u = 0; u < kReduceBatch; ++u)
          if (z0 + u < slices) vadd(rg[0], t[u]);
      }
    }
  } else if (PARTS) {  // slice by slice, each slice's loads of all NR vectors in flight together
    for (int z = 1; z < slices; ++z) {
      V t[NR];
#pragma unroll
      for (int u = 0; u < NR; ++u) {
        const int vv = (int)threadIdx.x + u * NT;
        if (vv < sp.nv) t[u] = *reinterpret_cast<const V*>(g + z * pstride + voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC));
      }
#pragma unroll
      for (int u = 0; u < NR; ++u)
        if ((int)threadIdx.x + u * NT < sp.nv) vadd(rg[u], t[u]);
    }
  }
  if (PARTS) {  // then g2
    if (RES && g2) {
#pragma unroll
      for (int u = 0; u < NR; ++u) {
        const int vv = (int)threadIdx.x + u * NT;
        if (vv < sp.nv) vadd(rg[u], *reinterpret_cast<const V*>(g2 + voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC)));
      }
    }
  }
  double s1 = 0.0, s2 = 0.0;
#pragma unroll
  for (int u = 0; u < NR; ++u)
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float gz = vget(rg[u], i);
      if (ry) gz = bn_act_grad(gz, vget(rr[u], i), act);
      const float xhat = (vget(rx[u], i) - mu) * inv;
      s1 += (double)gz;
      s2 += (double)gz * (double)xhat;
    }
  block_sum2<NT>(s1, s2);
  if (threadIdx.x == 0) {
    if (dbeta) dbeta[ch] = (float)s1;
    if (dgamma) dgamma[ch] = (float)s2;
    if (gx) bn_bwd_consts(s1, s2, (double)sp.nv * VEC, gamma[ch], mu, inv, kc);
  }
  if (!gx && !RES) return;
  __syncthreads();
  float k[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) k[i] = kc[i];
#pragma unroll
  for (int u = 0; u < NR; ++u) {
    const int vv = (int)threadIdx.x + u * NT;
    if (vv < sp.nv) {
      V o, z;
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        float gz = vget(rg[u], i);
        if (ry) gz = bn_act_grad(gz, vget(rr[u], i), act);
        vset(z, i, gz);
        vset(o, i, bwd_elem(gz, vget(rx[u], i), 1.f, false, k));
      }
      const int64_t off = voffset(vv, ch, c, hw, sp.hwv, sp.div_hwv, VEC);
      if (gx) *reinterpret_cast<V*>(gx + off) = o;
      if (RES) *reinterpret_cast<V*>(gzo + off) = z;
    }
  }
}

// grid x = plane (n * c), grid y = chunks of the plane
static dim3 apply_grid(int64_t planes, int64_t hw, int per_thread) {
  int64_t gy = cdiv(cdiv(hw, per_thread), 256);
  if (gy > 64) gy = 64;
  return dim3((unsigned)planes, (unsigned)(gy < 1 ? 1 : gy));
}

static bool bn_size_ok(int64_t n, int64_t c, int64_t hw) {
  return n >= 1 && c >= 1 && c <= 65535 && hw >= 1 && n * hw < ((int64_t)1 << 31) && n * c < ((int64_t)1 << 31) &&
         hw < ((int64_t)1 << 31);
}

static bool al16(const void* p) { return p == nullptr || ((uintptr_t)p % 16) == 0; }

// Planes below this many elements use the flat apply kernels (one workgroup per plane would mostly idle).
constexpr int64_t kFlatPlane = 1024;

static int launch_stats(const Split& sp, const float* x, double* part, int64_t c, int64_t hw, hipStream_t s) {
  const dim3 grid((unsigned)c, (unsigned)sp.slices);
  if (sp.vec == 4)
    hipLaunchKernelGGL(bn_stats_part_kernel<4>, grid, dim3(256), 0, s, x, part, (int)c, (int)hw, sp);
  else
    hipLaunchKernelGGL(bn_stats_part_kernel<1>, grid, dim3(256), 0, s, x, part, (int)c, (int)hw, sp);
  return launch_check("bn_stats_part_kernel");
}

// y = x * (invstd * gamma) + (beta - mean * invstd * gamma) [ReLU] with per-channel mean / invstd arrays.
static int launch_apply(int64_t n, int64_t c, int64_t hw, const float* x, const float* mean, const float* invstd,
                        const float* gamma, const float* beta, const float* res, float* y, int relu, hipStream_t s,
                        float* zo = nullptr) {
  const bool vec = hw % 4 == 0 && al16(x) && al16(y) && (!res || al16(res)) && al16(zo);
  const int64_t vw = vec ? 4 : 1, total_v = n * c * hw / vw;
  if (hw < kFlatPlane && total_v < ((int64_t)1 << 31)) {
    const FastDiv dh = make_fastdiv((uint32_t)(hw / vw)), dc = make_fastdiv((uint32_t)c);
    const dim3 grid(grid1d(total_v, 256, 16384));
    if (vec)
      hipLaunchKernelGGL(bn_apply_flat_kernel<4>, grid, dim3(256), 0, s, x, mean, invstd, gamma, beta, res, y, total_v,
                         dh, dc, (int)c, relu, zo);
    else
      hipLaunchKernelGGL(bn_apply_flat_kernel<1>, grid, dim3(256), 0, s, x, mean, invstd, gamma, beta, res, y, total_v,
                         dh, dc, (int)c, relu, zo);
    return launch_check("bn_apply_flat_kernel");
  }
  if (vec)
    hipLaunchKernelGGL(bn_apply_kernel<true>, apply_grid(n * c, hw, 4), dim3(256), 0, s, x, mean, invstd, nullptr,
                       0.0, gamma, beta, res, y, (int)c, (int)hw, relu, zo);
  else
    hipLaunchKernelGGL(bn_apply_kernel<false>, apply_grid(n * c, hw, 1), dim3(256), 0, s, x, mean, invstd, nullptr,
                       0.0, gamma, beta, res, y, (int)c, (int)hw, relu, zo);
  return launch_check("bn_apply_kernel");
}

// Statistics from a convolution's epilogue (omt_conv_fwd_stats): stats[ch][g][2] holds the unshifted double sums of
// x and x^2 over column group g of channel ch. Workgroup (s, ch) reduces slice s of the channel's groups, [s G / S,
// (s + 1) G / S): thread t sums its contiguous run of them in order and block_sum2 adds the 256 run sums in its fixed
// order, into part[ch][s][2] (the layout of bn_stats_part_kernel's partials, with shift 0).
__global__ void __launch_bounds__(256) bn_stats_groups_kernel(const double* __restrict__ stats, int groups,
                                                              double* __restrict__ part) {
  const int s = blockIdx.x, ch = blockIdx.y, S = gridDim.x, t = threadIdx.x;
  const int64_t lo = (int64_t)groups * s / S, hi = (int64_t)groups * (s + 1) / S, len = hi - lo;
  const int64_t g0 = lo + len * t / 256, g1 = lo + len * (t + 1) / 256;
  const double* sp = stats + (int64_t)ch * groups * 2;
  double s1 = 0.0, s2 = 0.0;
  for (int64_t g = g0; g < g1; ++g) {
    s1 += sp[2 * g];
    s2 += sp[2 * g + 1];
  }
  block_sum2(s1, s2);
  if (t == 0) {
    part[((int64_t)ch * S + s) * 2] = s1;
    part[((int64_t)ch * S + s) * 2 + 1] = s2;
  }
}

}  // namespace omt

using namespace omt;

OMT_EXPORT size_t omt_bn_train_workspace(int64_t n, int64_t c, int64_t hw) {
  (void)n;
  (void)hw;
  return (size_t)(c * kMaxSlices * 2) * sizeof(double);
}

OMT_EXPORT int omt_bn_train_fwd_res(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma,
                                    const float* beta, const float* running_mean, const float* running_var,
                                    double momentum, double eps, int relu, const float* residual, float* y, float* z,
                                    float* save_mean, float* save_invstd, float* new_rm, float* new_rv,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  if (!x || !gamma || !beta || !y || !save_mean || !save_invstd) return fail(OMT_INVALID, "omt_bn_train_fwd: null pointer");
  if (relu < OMT_ACT_NONE || relu > OMT_ACT_HARDSWISH) return fail(OMT_INVALID, "omt_bn_train_fwd: activation %d", relu);
  if (!bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_train_fwd: size not covered");
  if (!workspace || workspace_bytes < omt_bn_train_workspace(n, c, hw))
    return fail(OMT_INVALID, "omt_bn_train_fwd: workspace too small");
  hipStream_t s = stream_of(stream);
  const Split sp = bn_split(n, c, hw, al16(x));
  if (n * hw <= kFusedMax) {
    const bool vec = sp.vec == 4 && al16(y) && (!residual || al16(residual)) && al16(z);
    const Split f = vec ? sp : bn_split(n, c, hw, false);
#define OMT_BN_FUSED(V, E)                                                                                      \
  hipLaunchKernelGGL((bn_train_fused_kernel<V, false, false, E>), dim3((unsigned)c), dim3(256), 0, s, x, gamma, beta, \
                     running_mean, running_var, momentum, eps, relu, residual, y, save_mean, save_invstd, new_rm,      \
                     new_rv, (int)c, (int)hw, f, 1, 0, nullptr, z)
    const bool sm = n * hw <= kFusedSmall;
    if (vec) {
      if (sm && n * hw > kFusedSmall / 2)
        hipLaunchKernelGGL((bn_train_fused_kernel<4, false, false, (int)kFusedSmall, kFusedSmallThreads>),
                           dim3((unsigned)c), dim3(kFusedSmallThreads), 0, s, x, gamma, beta, running_mean, running_var,
                           momentum, eps, relu, residual, y, save_mean, save_invstd, new_rm, new_rv, (int)c, (int)hw, f,
                           1, 0, nullptr, z);
      else if (sm)
        OMT_BN_FUSED(4, (int)kFusedSmall);
      else
        hipLaunchKernelGGL((bn_train_fused_kernel<4, false, false, (int)kFusedMax, kFusedLargeThreads>),
                           dim3((unsigned)c), dim3(kFusedLargeThreads), 0, s, x, gamma, beta, running_mean, running_var,
                           momentum, eps, relu, residual, y, save_mean, save_invstd, new_rm, new_rv, (int)c, (int)hw, f,
                           1, 0, nullptr, z);
    } else {
      if (sm) OMT_BN_FUSED(1, (int)kFusedSmall); else OMT_BN_FUSED(1, (int)kFusedMax);
    }
#undef OMT_BN_FUSED
    return launch_check("bn_train_fused_kernel");
  }
  if (n * hw <= kFusedLarge) {
    const bool vec = sp.vec == 4 && al16(y) && (!residual || al16(residual)) && al16(z);
    const Split f = vec ? sp : bn_split(n, c, hw, false);
#define OMT_BN_FUSED_L(V)                                                                                          \
  hipLaunchKernelGGL((bn_train_fused_kernel<V, false, false, (int)kFusedLarge, kFusedLargeThreads>), dim3((unsigned)c), \
                     dim3(kFusedLargeThreads), 0, s, x, gamma, beta, running_mean, running_var, momentum, eps, relu,      \
                     residual, y, save_mean, save_invstd, new_rm, new_rv, (int)c, (int)hw, f, 1, 0, nullptr, z)
    if (vec) OMT_BN_FUSED_L(4); else OMT_BN_FUSED_L(1);
#undef OMT_BN_FUSED_L
    return launch_check("bn_train_fused_kernel");
  }
  double* part = (double*)workspace;
  if (int st = launch_stats(sp, x, part, c, hw, s)) return st;
  const double m = (double)(n * hw);
  const bool vec = hw % 4 == 0 && al16(x) && al16(y) && al16(residual) && al16(z);
  const dim3 ag = apply_grid(n * c, hw, vec ? 4 : 1), grid(ag.x * ag.y);
  if (hw >= kFlatPlane && (int64_t)ag.x * ag.y < ((int64_t)1 << 31)) {  // the apply finalizes its own channel
    const int rev = n * c * hw * 4 >= kRevApplyBytes;
    if (vec)
      hipLaunchKernelGGL(bn_train_apply_kernel<true>, grid, dim3(256), 0, s, x, (const double*)part, sp.slices, m,
                         momentum, eps, running_mean, running_var, save_mean, save_invstd, new_rm, new_rv, gamma, beta,
                         residual, y, (int)c, (int)hw, relu, (int)ag.x, (int)ag.y, rev, 0, z);
    else
      hipLaunchKernelGGL(bn_train_apply_kernel<false>, grid, dim3(256), 0, s, x, (const double*)part, sp.slices, m,
                         momentum, eps, running_mean, running_var, save_mean, save_invstd, new_rm, new_rv, gamma, beta,
                         residual, y, (int)c, (int)hw, relu, (int)ag.x, (int)ag.y, rev, 0, z);
    return launch_check("bn_train_apply_kernel");
  }
  hipLaunchKernelGGL(bn_stats_fin_kernel, dim3(grid1d(c, 256)), dim3(256), 0, s, x, (const double*)part, (int)c,
                     (int)hw, sp.slices, m, momentum, eps, running_mean, running_var, save_mean, save_invstd, new_rm,
                     new_rv);
  if (int st = launch_check("bn_stats_fin_kernel")) return st;
  return launch_apply(n, c, hw, x, save_mean, save_invstd, gamma, beta, residual, y, relu, s, z);
}

OMT_EXPORT int omt_bn_train_fwd_pool(int64_t n, int64_t c, int64_t h, int64_t w, const float* x, const float* gamma,
                                     const float* beta, const float* running_mean, const float* running_var,
                                     double momentum, double eps, int act, float* y, float* save_mean,
                                     float* save_invstd, float* new_rm, float* new_rv, int64_t kh, int64_t kw,
                                     int64_t sh, int64_t sw, int64_t ph, int64_t pw, float* pooled, int64_t* idx,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  if (!x || !gamma || !beta || !y || !save_mean || !save_invstd || !pooled || !idx)
    return fail(OMT_INVALID, "omt_bn_train_fwd_pool: null pointer");
  if (act < OMT_ACT_NONE || act > OMT_ACT_HARDSWISH) return fail(OMT_INVALID, "omt_bn_train_fwd_pool: activation %d", act);
  const int64_t hw = h * w;
  if (h < 1 || w < 1 || !bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_train_fwd_pool: size not covered");
  if (kh < 1 || kw < 1 || sh < 1 || sw < 1 || ph < 0 || pw < 0 || 2 * ph > kh || 2 * pw > kw || h + 2 * ph < kh ||
      w + 2 * pw < kw)
    return fail(OMT_UNSUPPORTED, "omt_bn_train_fwd_pool: pooling window not covered");
  if (!workspace || workspace_bytes < omt_bn_train_workspace(n, c, hw))
    return fail(OMT_INVALID, "omt_bn_train_fwd_pool: workspace too small");
  const int64_t oh = (h + 2 * ph - kh) / sh + 1, ow = (w + 2 * pw - kw) / sw + 1;
  if (n * c * oh * ow >= ((int64_t)1 << 31)) return fail(OMT_UNSUPPORTED, "omt_bn_train_fwd_pool: output too large");
  const PoolArgs pa{pooled, idx, (int)h, (int)w, (int)oh, (int)ow, (int)kh, (int)kw, (int)sh, (int)sw, (int)ph, (int)pw};
  hipStream_t s = stream_of(stream);
  const Split sp = bn_split(n, c, hw, al16(x));
  if (n * hw <= kFusedMax) {  // one launch: statistics, apply and the pool from LDS
    const bool vec = sp.vec == 4 && al16(y);
    const Split f = vec ? sp : bn_split(n, c, hw, false);
#define OMT_BN_POOL(V, E)                                                                                        \
  hipLaunchKernelGGL((bn_train_fused_kernel<V, false, true, E>), dim3((unsigned)c), dim3(256), 0, s, x, gamma, beta,  \
                     running_mean, running_var, momentum, eps, act, nullptr, y, save_mean, save_invstd, new_rm, new_rv, \
                     (int)c, (int)hw, f, 1, 0, nullptr, nullptr, pa)
    const bool sm = n * hw <= kFusedSmall;
    if (vec) {
      if (sm) OMT_BN_POOL(4, (int)kFusedSmall); else OMT_BN_POOL(4, (int)kFusedMax);
    } else {
      if (sm) OMT_BN_POOL(1, (int)kFusedSmall); else OMT_BN_POOL(1, (int)kFusedMax);
    }
#undef OMT_BN_POOL
    return launch_check("bn_train_fused_kernel (pool)");
  }
  double* part = (double*)workspace;
  if (int st = launch_stats(sp, x, part, c, hw, s)) return st;
  // runs of pooled rows owning about 1024 elements of y each
  const int rows = (int)std::max<int64_t>(1, std::min<int64_t>(oh, cdiv(1024, sh * w)));
  const int64_t runs = cdiv(oh, rows), grid = n * c * runs;
  if (grid >= ((int64_t)1 << 31)) return fail(OMT_UNSUPPORTED, "omt_bn_train_fwd_pool: grid too large");
  const bool vec = w % 4 == 0 && al16(x) && al16(y);
  if (vec)
    hipLaunchKernelGGL(bn_apply_pool_kernel<true>, dim3((unsigned)grid), dim3(256), 0, s, x, (const double*)part,
                       sp.slices, (double)(n * hw), momentum, eps, running_mean, running_var, save_mean, save_invstd,
                       new_rm, new_rv, gamma, beta, y, (int)c, act, (int)(n * c), rows, pa);
  else
    hipLaunchKernelGGL(bn_apply_pool_kernel<false>, dim3((unsigned)grid), dim3(256), 0, s, x, (const double*)part,
                       sp.slices, (double)(n * hw), momentum, eps, running_mean, running_var, save_mean, save_invstd,
                       new_rm, new_rv, gamma, beta, y, (int)c, act, (int)(n * c), rows, pa);
  return launch_check("bn_apply_pool_kernel");
}

OMT_EXPORT int omt_bn_train_fwd_parts(int64_t n, int64_t c, int64_t hw, const float* parts, int slices, float* x,
                                      const float* gamma, const float* beta, const float* running_mean,
                                      const float* running_var, double momentum, double eps, int relu,
                                      const float* residual, float* y, float* z, float* save_mean, float* save_invstd,
                                      float* new_rm, float* new_rv, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  if (!parts || !x || !gamma || !beta || !y || !save_mean || !save_invstd)
    return fail(OMT_INVALID, "omt_bn_train_fwd_parts: null pointer");
  if (relu < OMT_ACT_NONE || relu > OMT_ACT_HARDSWISH)
    return fail(OMT_INVALID, "omt_bn_train_fwd_parts: activation %d", relu);
  if (slices < 1) return fail(OMT_INVALID, "omt_bn_train_fwd_parts: %d slices", slices);
  if (!bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_train_fwd_parts: size not covered");
  if (!workspace || workspace_bytes < omt_bn_train_workspace(n, c, hw))
    return fail(OMT_INVALID, "omt_bn_train_fwd_parts: workspace too small");
  hipStream_t s = stream_of(stream);
  const int64_t total = n * c * hw;
  const bool vec = hw % 4 == 0 && al16(parts) && al16(x) && al16(y) && al16(residual) && al16(z);
  if (n * hw <= kFusedMax) {  // one launch: the slice sums, the statistics and the apply
    const Split f = bn_split(n, c, hw, vec);
#define OMT_BN_PARTS(V, E)                                                                                       \
  hipLaunchKernelGGL((bn_train_fused_kernel<V, true, false, E>), dim3((unsigned)c), dim3(256), 0, s, parts, gamma,    \
                     beta, running_mean, running_var, momentum, eps, relu, residual, y, save_mean, save_invstd, new_rm, \
                     new_rv, (int)c, (int)hw, f, slices, total, x, z)
    const bool sm = n * hw <= kFusedSmall;
    if (vec) {
      if (sm && n * hw > kFusedSmall / 2)
        hipLaunchKernelGGL((bn_train_fused_kernel<4, true, false, (int)kFusedSmall, kFusedSmallThreads>),
                           dim3((unsigned)c), dim3(kFusedSmallThreads), 0, s, parts, gamma, beta, running_mean,
                           running_var, momentum, eps, relu, residual, y, save_mean, save_invstd, new_rm, new_rv, (int)c,
                           (int)hw, f, slices, total, x, z);
      else if (sm)
        OMT_BN_PARTS(4, (int)kFusedSmall);
      else
        hipLaunchKernelGGL((bn_train_fused_kernel<4, true, false, (int)kFusedMax, kFusedLargeThreads>),
                           dim3((unsigned)c), dim3(kFusedLargeThreads), 0, s, parts, gamma, beta, running_mean,
                           running_var, momentum, eps, relu, residual, y, save_mean, save_invstd, new_rm, new_rv, (int)c,
                           (int)hw, f, slices, total, x, z);
    } else {
      if (sm) OMT_BN_PARTS(1, (int)kFusedSmall); else OMT_BN_PARTS(1, (int)kFusedMax);
    }
#undef OMT_BN_PARTS
    return launch_check("bn_train_fused_kernel");
  }
  const bool v4 = total % 4 == 0 && al16(parts) && al16(x);
  const int64_t nv = v4 ? total / 4 : total;
  if (v4)
    hipLaunchKernelGGL(bn_sum_parts_kernel<4>, dim3(grid1d(nv, 256, 16384)), dim3(256), 0, s, parts, slices, nv, x);
  else
    hipLaunchKernelGGL(bn_sum_parts_kernel<1>, dim3(grid1d(nv, 256, 16384)), dim3(256), 0, s, parts, slices, nv, x);
  if (int st = launch_check("bn_sum_parts_kernel")) return st;
  return omt_bn_train_fwd_res(n, c, hw, x, gamma, beta, running_mean, running_var, momentum, eps, relu, residual, y,
                              z, save_mean, save_invstd, new_rm, new_rv, workspace, workspace_bytes, stream);
}

OMT_EXPORT int omt_bn_train_fwd_stats(int64_t n, int64_t c, int64_t hw, const float* x, const double* stats,
                                      int groups, size_t stats_bytes, const float* gamma, const float* beta, const float* running_mean,
                                      const float* running_var, double momentum, double eps, int relu,
                                      const float* residual, float* y, float* z, float* save_mean, float* save_invstd,
                                      float* new_rm, float* new_rv, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  if (!x || !stats || !gamma || !beta || !y || !save_mean || !save_invstd)
    return fail(OMT_INVALID, "omt_bn_train_fwd_stats: null pointer");
  if (relu < OMT_ACT_NONE || relu > OMT_ACT_HARDSWISH)
    return fail(OMT_INVALID, "omt_bn_train_fwd_stats: activation %d", relu);
  if (groups < 1) return fail(OMT_INVALID, "omt_bn_train_fwd_stats: %d column groups", groups);
  if (c < 0 || (uint64_t)c * (uint64_t)groups * 2 * sizeof(double) > stats_bytes)
    return fail(OMT_INVALID, "omt_bn_train_fwd_stats: %d groups of %lld channels exceed the %zu-byte stats buffer",
                groups, (long long)c, stats_bytes);
  if (!bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_train_fwd_stats: size not covered");
  if (!workspace || workspace_bytes < omt_bn_train_workspace(n, c, hw))
    return fail(OMT_INVALID, "omt_bn_train_fwd_stats: workspace too small");
  hipStream_t s = stream_of(stream);
  // the groups reduced to S slices per channel (about 1024 workgroups), then the apply that finalizes its channel
  const int S = (int)std::max<int64_t>(1, std::min<int64_t>({(int64_t)kMaxSlices, cdiv(1024, c), (int64_t)groups}));
  double* part = (double*)workspace;
  hipLaunchKernelGGL(bn_stats_groups_kernel, dim3((unsigned)S, (unsigned)c), dim3(256), 0, s, stats, groups, part);
  if (int st = launch_check("bn_stats_groups_kernel")) return st;
  const double m = (double)(n * hw);
  const bool vec = hw % 4 == 0 && al16(x) && al16(y) && al16(residual) && al16(z);
  const dim3 ag = apply_grid(n * c, hw, vec ? 4 : 1), grid(ag.x * ag.y);
  if (hw >= kFlatPlane && (int64_t)ag.x * ag.y < ((int64_t)1 << 31)) {
    const int rev = n * c * hw * 4 >= kRevApplyBytes;
    if (vec)
      hipLaunchKernelGGL(bn_train_apply_kernel<true>, grid, dim3(256), 0, s, x, (const double*)part, S, m, momentum,
                         eps, running_mean, running_var, save_mean, save_invstd, new_rm, new_rv, gamma, beta, residual, y,
                         (int)c, (int)hw, relu, (int)ag.x, (int)ag.y, rev, 1, z);
    else
      hipLaunchKernelGGL(bn_train_apply_kernel<false>, grid, dim3(256), 0, s, x, (const double*)part, S, m, momentum,
                         eps, running_mean, running_var, save_mean, save_invstd, new_rm, new_rv, gamma, beta, residual, y,
                         (int)c, (int)hw, relu, (int)ag.x, (int)ag.y, rev, 1, z);
    return launch_check("bn_train_apply_kernel");
  }
  hipLaunchKernelGGL(bn_stats_shift0_fin_kernel, dim3(grid1d(c, 256)), dim3(256), 0, s, (const double*)part, (int)c, S,
                     m, momentum, eps, running_mean, running_var, save_mean, save_invstd, new_rm, new_rv);
  if (int st = launch_check("bn_stats_shift0_fin_kernel")) return st;
  return launch_apply(n, c, hw, x, save_mean, save_invstd, gamma, beta, residual, y, relu, s, z);
}

OMT_EXPORT int omt_bn_train_fwd(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma,
                                const float* beta, const float* running_mean, const float* running_var,
                                double momentum, double eps, int relu, float* y, float* save_mean, float* save_invstd,
                                float* new_rm, float* new_rv, void* workspace, size_t workspace_bytes, void* stream) {
  return omt_bn_train_fwd_res(n, c, hw, x, gamma, beta, running_mean, running_var, momentum, eps, relu, nullptr, y,
                              nullptr, save_mean, save_invstd, new_rm, new_rv, workspace, workspace_bytes, stream);
}

OMT_EXPORT int omt_bn_eval_fwd(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma,
                               const float* beta, const float* running_mean, const float* running_var, double eps,
                               int relu, float* y, void* stream) {
  if (!x || !gamma || !beta || !running_mean || !running_var || !y)
    return fail(OMT_INVALID, "omt_bn_eval_fwd: null pointer");
  if (relu < OMT_ACT_NONE || relu > OMT_ACT_HARDSWISH) return fail(OMT_INVALID, "omt_bn_eval_fwd: activation %d", relu);
  if (!bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_eval_fwd: size not covered");
  hipStream_t s = stream_of(stream);
  const bool vec = (hw % 4) == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)y % 16) == 0;
  if (vec)
    hipLaunchKernelGGL(bn_apply_kernel<true>, apply_grid(n * c, hw, 4), dim3(256), 0, s, x, running_mean, nullptr,
                       running_var, eps, gamma, beta, nullptr, y, (int)c, (int)hw, relu);
  else
    hipLaunchKernelGGL(bn_apply_kernel<false>, apply_grid(n * c, hw, 1), dim3(256), 0, s, x, running_mean, nullptr,
                       running_var, eps, gamma, beta, nullptr, y, (int)c, (int)hw, relu);
  return launch_check("bn_apply_kernel");
}

// [c][kMaxSlices][2] double partials, then [c][5] float per-channel constants of the input-gradient map
OMT_EXPORT size_t omt_bn_bwd_workspace(int64_t n, int64_t c, int64_t hw) {
  (void)n;
  (void)hw;
  return (size_t)(c * kMaxSlices * 2) * sizeof(double) + (size_t)(c * 5) * sizeof(float);
}

// The backward of every BN entry point: gz = g (+ g2) through the activation's gradient (relu_y: the ReLU's output,
// masked where not > 0, or the hardswish's input: bn_act_grad), or as it is when relu_y is null; RES also writes gz to
// gzo.
template <bool RES>
static int bn_bwd_impl(int64_t n, int64_t c, int64_t hw, const float* g, const float* g2, const float* x,
                       const float* relu_y, const float* save_mean, const float* save_invstd, const float* gamma,
                       float* gx, float* dgamma, float* dbeta, float* gzo, void* workspace, hipStream_t s,
                       int act = OMT_ACT_RELU) {
  const bool aligned = al16(g) && al16(g2) && al16(x) && al16(relu_y) && al16(gx) && al16(gzo);
  const Split sp = bn_split(n, c, hw, aligned);
  if (n * hw <= kFusedMax) {
#define OMT_BN_BWD(V, E)                                                                                        \
  hipLaunchKernelGGL((bn_bwd_fused_kernel<V, RES, false, E>), dim3((unsigned)c), dim3(256), 0, s, g, g2, x, relu_y, \
                     save_mean, save_invstd, gamma, gx, dgamma, dbeta, gzo, (int)c, (int)hw, sp, act)
    const bool sm = n * hw <= kFusedSmall;
    if (sp.vec == 4) {
      if (sm && n * hw > kFusedSmall / 2)
        hipLaunchKernelGGL((bn_bwd_fused_kernel<4, RES, false, (int)kFusedSmall, kFusedSmallThreads>),
                           dim3((unsigned)c), dim3(kFusedSmallThreads), 0, s, g, g2, x, relu_y, save_mean, save_invstd,
                           gamma, gx, dgamma, dbeta, gzo, (int)c, (int)hw, sp, act);
      else if (sm)
        OMT_BN_BWD(4, (int)kFusedSmall);
      else
        hipLaunchKernelGGL((bn_bwd_fused_kernel<4, RES, false, (int)kFusedMax, kFusedLargeThreads>), dim3((unsigned)c),
                           dim3(kFusedLargeThreads), 0, s, g, g2, x, relu_y, save_mean, save_invstd, gamma, gx, dgamma,
                           dbeta, gzo, (int)c, (int)hw, sp, act);
    } else {
      if (sm) OMT_BN_BWD(1, (int)kFusedSmall); else OMT_BN_BWD(1, (int)kFusedMax);
    }
#undef OMT_BN_BWD
    return launch_check("bn_bwd_fused_kernel");
  }
  if (n * hw <= kFusedLargeBwd && sp.vec == 4) {
    hipLaunchKernelGGL((bn_bwd_fused_kernel<4, RES, false, (int)kFusedLargeBwd, kFusedLargeThreads>),
                       dim3((unsigned)c), dim3(kFusedLargeThreads), 0, s, g, g2, x, relu_y, save_mean, save_invstd,
                       gamma, gx, dgamma, dbeta, gzo, (int)c, (int)hw, sp, act);
    return launch_check("bn_bwd_fused_kernel");
  }
  double* part = (double*)workspace;
  float* kc = (float*)(part + c * kMaxSlices * 2);
  const dim3 pgrid((unsigned)c, (unsigned)sp.slices);
  if (sp.vec == 4)
    hipLaunchKernelGGL((bn_bwd_part_kernel<4, RES>), pgrid, dim3(256), 0, s, g, g2, x, relu_y, save_mean, save_invstd,
                       part, (int)c, (int)hw, sp, act);
  else
    hipLaunchKernelGGL((bn_bwd_part_kernel<1, RES>), pgrid, dim3(256), 0, s, g, g2, x, relu_y, save_mean, save_invstd,
                       part, (int)c, (int)hw, sp, act);
  if (int st = launch_check("bn_bwd_part_kernel")) return st;
  const double m = (double)(n * hw);
  const dim3 ag = apply_grid(n * c, hw, sp.vec), grid(ag.x * ag.y);
  if ((gx || RES) && hw >= kFlatPlane && (int64_t)ag.x * ag.y < ((int64_t)1 << 31)) {  // the apply finalizes its channel
    const int rev = n * c * hw * 4 >= kRevApplyBytes;
    if (sp.vec == 4)
      hipLaunchKernelGGL((bn_bwd_train_apply_kernel<4, RES>), grid, dim3(256), 0, s, g, g2, x, relu_y,
                         (const double*)part, sp.slices, m, save_mean, save_invstd, gamma, dgamma, dbeta, gx, gzo,
                         (int)c, (int)(hw / 4), (int)ag.x, (int)ag.y, rev, act);
    else
      hipLaunchKernelGGL((bn_bwd_train_apply_kernel<1, RES>), grid, dim3(256), 0, s, g, g2, x, relu_y,
                         (const double*)part, sp.slices, m, save_mean, save_invstd, gamma, dgamma, dbeta, gx, gzo,
                         (int)c, (int)hw, (int)ag.x, (int)ag.y, rev, act);
    return launch_check("bn_bwd_train_apply_kernel");
  }
  // the apply pass needs the per-channel constants (gamma) whenever it runs: for gx, or for gzo
  hipLaunchKernelGGL(bn_bwd_fin_kernel, dim3(grid1d(c, 256)), dim3(256), 0, s, (const double*)part, (int)c, sp.slices,
                     save_mean, save_invstd, (gx || RES) ? gamma : nullptr, m, kc, dgamma, dbeta);
  if (int st = launch_check("bn_bwd_fin_kernel")) return st;
  if (!gx && !RES) return OMT_OK;
  float* gxo = gx;
  const int64_t total_v = n * c * hw / sp.vec;
  if (hw < kFlatPlane && total_v < ((int64_t)1 << 31)) {
    const FastDiv dh = make_fastdiv((uint32_t)sp.hwv), dc = make_fastdiv((uint32_t)c);
    const dim3 grid(grid1d(total_v, 256, 16384));
    if (sp.vec == 4)
      hipLaunchKernelGGL((bn_bwd_apply_flat_kernel<4, RES>), grid, dim3(256), 0, s, g, g2, x, relu_y, kc, gxo, gzo,
                         total_v, dh, dc, (int)c, act);
    else
      hipLaunchKernelGGL((bn_bwd_apply_flat_kernel<1, RES>), grid, dim3(256), 0, s, g, g2, x, relu_y, kc, gxo, gzo,
                         total_v, dh, dc, (int)c, act);
    return launch_check("bn_bwd_apply_flat_kernel");
  }
  if (sp.vec == 4)
    hipLaunchKernelGGL((bn_bwd_apply_kernel<4, RES>), apply_grid(n * c, hw, 4), dim3(256), 0, s, g, g2, x, relu_y, kc,
                       gxo, gzo, (int)c, (int)(hw / 4), act);
  else
    hipLaunchKernelGGL((bn_bwd_apply_kernel<1, RES>), apply_grid(n * c, hw, 1), dim3(256), 0, s, g, g2, x, relu_y, kc,
                       gxo, gzo, (int)c, (int)hw, act);
  return launch_check("bn_bwd_apply_kernel");
}

OMT_EXPORT int omt_bn_bwd(int64_t n, int64_t c, int64_t hw, const float* g, const float* x, const float* relu_y,
                          const float* save_mean, const float* save_invstd, const float* gamma, float* gx,
                          float* dgamma, float* dbeta, void* workspace, size_t workspace_bytes, void* stream) {
  if (!g || !x || !save_mean || !save_invstd || (gx && !gamma)) return fail(OMT_INVALID, "omt_bn_bwd: null pointer");
  if (!bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_bwd: size not covered");
  if (!workspace || workspace_bytes < omt_bn_bwd_workspace(n, c, hw))
    return fail(OMT_INVALID, "omt_bn_bwd: workspace too small");
  return bn_bwd_impl<false>(n, c, hw, g, nullptr, x, relu_y, save_mean, save_invstd, gamma, gx, dgamma, dbeta, nullptr,
                            workspace, stream_of(stream));
}

OMT_EXPORT int omt_bn_bwd_res(int64_t n, int64_t c, int64_t hw, const float* g, const float* g2, const float* x,
                              const float* relu_y, const float* save_mean, const float* save_invstd,
                              const float* gamma, float* gx, float* dgamma, float* dbeta, float* gz,
                              void* workspace, size_t workspace_bytes, void* stream) {
  if (!g || !x || !save_mean || !save_invstd || !gz || !gamma) return fail(OMT_INVALID, "omt_bn_bwd_res: null pointer");
  if (!bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_bwd_res: size not covered");
  if (!workspace || workspace_bytes < omt_bn_bwd_workspace(n, c, hw))
    return fail(OMT_INVALID, "omt_bn_bwd_res: workspace too small");
  return bn_bwd_impl<true>(n, c, hw, g, g2, x, relu_y, save_mean, save_invstd, gamma, gx, dgamma, dbeta, gz, workspace,
                           stream_of(stream));
}

OMT_EXPORT int omt_bn_bwd_parts(int64_t n, int64_t c, int64_t hw, const float* g_parts, int slices, const float* g2,
                                const float* x, int act, const float* act_in, const float* save_mean,
                                const float* save_invstd, const float* gamma, float* gx, float* dgamma, float* dbeta,
                                float* gz, const omt_slice_sum* sums, int count, void* stream) {
  if (!g_parts || !x || !save_mean || !save_invstd || (gx && !gamma) || (act != OMT_ACT_NONE && !act_in) ||
      (g2 && !gz) || (count > 0 && !sums))
    return fail(OMT_INVALID, "omt_bn_bwd_parts: null pointer");
  if (act < OMT_ACT_NONE || act > OMT_ACT_HARDSWISH) return fail(OMT_INVALID, "omt_bn_bwd_parts: activation %d", act);
  if (slices < 1 || slices > kMaxSlices) return fail(OMT_INVALID, "omt_bn_bwd_parts: %d slices", slices);
  if (count < 0 || count > kMaxSideSums) return fail(OMT_INVALID, "omt_bn_bwd_parts: %d slice sums", count);
  if (!bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_bwd_parts: size not covered");
  if (n * hw > kFusedMax) return fail(OMT_UNSUPPORTED, "omt_bn_bwd_parts: channels above %lld elements",
                                      (long long)kFusedMax);
  SideSums side{};
  int64_t blocks = c;
  for (int k = 0; k < count; ++k) {
    const omt_slice_sum& j = sums[k];
    if (j.slices < 0 || j.n < 0 || (j.slices > 0 && (!j.parts || !j.out)))
      return fail(OMT_INVALID, "omt_bn_bwd_parts: slice sum %d", k);
    if (j.slices == 0 || j.n == 0) continue;
    side.job[side.count] = split_sum_of(j.parts, j.out, j.n, j.slices);
    blocks += side.job[side.count].blocks;
    side.end[side.count++] = blocks - c;
  }
  if (blocks >= ((int64_t)1 << 31)) return fail(OMT_UNSUPPORTED, "omt_bn_bwd_parts: grid too large");
  const bool aligned = al16(g_parts) && al16(g2) && al16(x) && al16(act_in) && al16(gx) && al16(gz);
  const Split sp = bn_split(n, c, hw, aligned);
  const float* ry = act == OMT_ACT_NONE ? nullptr : act_in;
  const int64_t pstride = n * c * hw;
  hipStream_t s = stream_of(stream);
#define OMT_BWD_PARTS(V, R, E)                                                                                   \
  hipLaunchKernelGGL((bn_bwd_fused_kernel<V, R, true, E>), dim3((unsigned)blocks), dim3(256), 0, s, g_parts, g2, x,  \
                     ry, save_mean, save_invstd, gamma, gx, dgamma, dbeta, gz, (int)c, (int)hw, sp, act, slices,        \
                     pstride, side)
#define OMT_BWD_PARTS_E(V, R)                                                        \
  do {                                                                               \
    if (n * hw <= kFusedSmall) OMT_BWD_PARTS(V, R, (int)kFusedSmall);               \
    else OMT_BWD_PARTS(V, R, (int)kFusedMax);                                        \
  } while (0)
#define OMT_BWD_PARTS_MID(R)                                                                                       \
  hipLaunchKernelGGL((bn_bwd_fused_kernel<4, R, true, (int)kFusedMax, kFusedLargeThreads>), dim3((unsigned)blocks), \
                     dim3(kFusedLargeThreads), 0, s, g_parts, g2, x, ry, save_mean, save_invstd, gamma, gx, dgamma,    \
                     dbeta, gz, (int)c, (int)hw, sp, act, slices, pstride, side)
#define OMT_BWD_PARTS_SM(R)                                                                                          \
  hipLaunchKernelGGL((bn_bwd_fused_kernel<4, R, true, (int)kFusedSmall, kFusedSmallThreads>), dim3((unsigned)blocks), \
                     dim3(kFusedSmallThreads), 0, s, g_parts, g2, x, ry, save_mean, save_invstd, gamma, gx, dgamma,     \
                     dbeta, gz, (int)c, (int)hw, sp, act, slices, pstride, side)
  if (sp.vec == 4 && n * hw > kFusedSmall) {  // 1024-thread workgroups for channels of 2K-8K elements
    if (gz) OMT_BWD_PARTS_MID(true); else OMT_BWD_PARTS_MID(false);
  } else if (sp.vec == 4 && n * hw > kFusedSmall / 2) {  // 512-thread ones for 1K-2K
    if (gz) OMT_BWD_PARTS_SM(true); else OMT_BWD_PARTS_SM(false);
  } else if (sp.vec == 4) {
    if (gz) OMT_BWD_PARTS_E(4, true); else OMT_BWD_PARTS_E(4, false);
  } else {
    if (gz) OMT_BWD_PARTS_E(1, true); else OMT_BWD_PARTS_E(1, false);
  }
#undef OMT_BWD_PARTS_SM
#undef OMT_BWD_PARTS_MID
#undef OMT_BWD_PARTS_E
#undef OMT_BWD_PARTS
  return launch_check("bn_bwd_fused_kernel");
}

OMT_EXPORT int omt_bn_bwd_act(int64_t n, int64_t c, int64_t hw, const float* g, const float* x, int act,
                              const float* act_in, const float* save_mean, const float* save_invstd,
                              const float* gamma, float* gx, float* dgamma, float* dbeta, void* workspace,
                              size_t workspace_bytes, void* stream) {
  if (!g || !x || !save_mean || !save_invstd || (gx && !gamma) || (act != OMT_ACT_NONE && !act_in))
    return fail(OMT_INVALID, "omt_bn_bwd_act: null pointer");
  if (act < OMT_ACT_NONE || act > OMT_ACT_HARDSWISH) return fail(OMT_INVALID, "omt_bn_bwd_act: activation %d", act);
  if (!bn_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_bwd_act: size not covered");
  if (!workspace || workspace_bytes < omt_bn_bwd_workspace(n, c, hw))
    return fail(OMT_INVALID, "omt_bn_bwd_act: workspace too small");
  return bn_bwd_impl<false>(n, c, hw, g, nullptr, x, act == OMT_ACT_NONE ? nullptr : act_in, save_mean, save_invstd,
                            gamma, gx, dgamma, dbeta, nullptr, workspace, stream_of(stream), act);
}

namespace omt {

// ---- channels-last (NHWC) BatchNorm -----------------------------------------------------------------------------
// x [rows = n * hw][c], a channel's elements c apart. Workgroup (channel block, row slice): thread t owns channel
// vector j = block * cb + t % cb (VEC channels: float4 when c % 4 == 0 and the operands are 16-byte aligned) and walks
// rows t / cb, + rl, ... of the slice, so a wave reads whole rows (64 vectors of one row, or several rows of a
// narrower tensor) and every thread keeps its channels' sums, coefficients or constants in registers. The statistics
// are the NCHW kernels' shifted float64 sums (shift x[row 0][ch] = x[n=0, ch, 0, 0], the same element) in another
// order: each thread's rows in order, the row lanes added in lane order, the slices by one wave per channel (lane-
// strided, then the DPP wave sum); finalize and apply arithmetic are the NCHW kernels' (bn_finalize, bn_bwd_consts,
// bwd_elem), so y and gx agree with the NCHW path to the float64 rounding of the sums. Three launches each way:
// partial sums, finalize, apply.
constexpr int kNhwcMaxSlices = 256;

__host__ __device__ __forceinline__ int64_t min64(int64_t a, int64_t b) { return a < b ? a : b; }

struct NhwcSplit {
  int vec;          // channels per vector: 4 or 1
  int cv;           // vectors per row: c / vec
  int cb;           // vectors per workgroup row: min(cv, 64)
  int rl;           // row lanes: 256 / cb
  int cblocks;      // workgroups across a row: cv / cb rounded up
  int slices;       // row slices of the reductions
  int64_t rows;     // n * hw
  int64_t per_slice;
  int hw;           // positions per image, and its divider: a row r is image r / hw, position r % hw
  FastDiv div_hw;
};

static NhwcSplit nhwc_split(int64_t n, int64_t c, int64_t hw, bool aligned) {
  NhwcSplit sp;
  sp.vec = (c % 4 == 0 && aligned) ? 4 : 1;
  sp.cv = (int)(c / sp.vec);
  sp.cb = sp.cv < 64 ? sp.cv : 64;
  sp.rl = 256 / sp.cb;
  sp.cblocks = (int)cdiv(sp.cv, sp.cb);
  sp.rows = n * hw;
  int64_t want = cdiv(1024, sp.cblocks);                        // ~1024 workgroups
  const int64_t by_rows = sp.rows / (4 * (int64_t)sp.rl) > 1 ? sp.rows / (4 * (int64_t)sp.rl) : 1;  // at least 4 rows per thread
  want = min64(min64(want, by_rows), kNhwcMaxSlices);
  sp.per_slice = cdiv(sp.rows, want);
  sp.slices = (int)cdiv(sp.rows, sp.per_slice);
  sp.hw = (int)hw;
  sp.div_hw = make_fastdiv((uint32_t)hw);
  return sp;
}

// The incoming gradient's VEC channels j VEC .. of row r, from a channels-last g, or (g_nchw) from an NCHW g: a
// channels-last model's global-average-pool gradient, broadcast over its planes in NCHW order, read in place.
template <int VEC>
__device__ __forceinline__ typename VecT<VEC>::T nhwc_grad(const float* __restrict__ g, int g_nchw, int64_t r, int j,
                                                           int c, const NhwcSplit& sp) {
  using V = typename VecT<VEC>::T;
  if (!g_nchw) return *reinterpret_cast<const V*>(g + r * c + (int64_t)j * VEC);
  const uint32_t img = fdiv((uint32_t)r, sp.div_hw), pos = (uint32_t)r - img * (uint32_t)sp.hw;
  V v;
#pragma unroll
  for (int i = 0; i < VEC; ++i) vset(v, i, g[((int64_t)img * c + j * VEC + i) * sp.hw + pos]);
  return v;
}

// Row lanes' sums of the block's channels added in lane order: thread t < cb * VEC ends with channel vector t / VEC,
// element t % VEC. All threads call it.
template <int VEC>
__device__ __forceinline__ void nhwc_lane_sums(const NhwcSplit& sp, const double* s1, const double* s2, double& o1,
                                               double& o2) {
  __shared__ double r1[256 * VEC], r2[256 * VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    r1[threadIdx.x * VEC + i] = s1[i];
    r2[threadIdx.x * VEC + i] = s2[i];
  }
  __syncthreads();
  o1 = 0.0, o2 = 0.0;
  const int q = threadIdx.x;
  if (q < sp.cb * VEC) {
    const int jl = q / VEC, i = q - jl * VEC;
    for (int r = 0; r < sp.rl; ++r) {
      o1 += r1[(r * sp.cb + jl) * VEC + i];
      o2 += r2[(r * sp.cb + jl) * VEC + i];
    }
  }
}

// grid (cblocks, slices): shifted partial sums per (channel, slice) into part[ch][slices][2]
template <int VEC>
__global__ void __launch_bounds__(256) bn_nhwc_stats_kernel(const float* __restrict__ x, double* __restrict__ part,
                                                            int c, const NhwcSplit sp) {
  using V = typename VecT<VEC>::T;
  const int jl = threadIdx.x % sp.cb, lane = threadIdx.x / sp.cb, j = blockIdx.x * sp.cb + jl;
  const bool on = lane < sp.rl && j < sp.cv;
  double s1[VEC], s2[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) s1[i] = 0.0, s2[i] = 0.0;
  if (on) {
    const V shift = *reinterpret_cast<const V*>(x + (int64_t)j * VEC);
    const int64_t r0 = blockIdx.y * sp.per_slice, r1 = min64(sp.rows, r0 + sp.per_slice);
    const int64_t step = sp.rl;
    for (int64_t r = r0 + lane; r < r1; r += 4 * step) {
      V v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        v[u] = r + u * step < r1 ? *reinterpret_cast<const V*>(x + (r + u * step) * c + (int64_t)j * VEC) : shift;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          const double d = (double)(vget(v[u], i) - vget(shift, i));  // 0 past the slice's end
          s1[i] += d;
          s2[i] += d * d;
        }
    }
  }
  double o1, o2;
  nhwc_lane_sums<VEC>(sp, s1, s2, o1, o2);
  const int q = threadIdx.x;
  if (q < sp.cb * VEC) {
    const int ch = (blockIdx.x * sp.cb + q / VEC) * VEC + q % VEC;
    if (ch < c) {
      part[((int64_t)ch * sp.slices + blockIdx.y) * 2] = o1;
      part[((int64_t)ch * sp.slices + blockIdx.y) * 2 + 1] = o2;
    }
  }
}

// A channel's slices summed by one wave (lane-strided, then the wave sum); valid in every lane. Whole waves call it.
__device__ __forceinline__ void nhwc_wave_slices(const double* __restrict__ part, int ch, int slices, double& s1,
                                                 double& s2) {
  s1 = 0.0, s2 = 0.0;
  for (int s = threadIdx.x & 63; s < slices; s += 64) {
    s1 += part[((int64_t)ch * slices + s) * 2];
    s2 += part[((int64_t)ch * slices + s) * 2 + 1];
  }
  s1 = wave_sum(s1);
  s2 = wave_sum(s2);
}

// one wave per channel: mean, invstd, the running statistics
__global__ void __launch_bounds__(256) bn_nhwc_fin_kernel(const float* __restrict__ x, const double* __restrict__ part,
                                                          int c, int slices, double m, double momentum, double eps,
                                                          const float* rm, const float* rv,
                                                          float* __restrict__ save_mean,
                                                          float* __restrict__ save_invstd, float* new_rm,
                                                          float* new_rv) {
  const int ch = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (ch >= c) return;  // whole waves
  double s1, s2;
  nhwc_wave_slices(part, ch, slices, s1, s2);
  if ((threadIdx.x & 63) == 0)
    bn_finalize(s1, s2, (double)x[ch], m, momentum, eps, rm, rv, save_mean, save_invstd, new_rm, new_rv, ch, true);
}

// grid (cblocks, chunks of rows): y = act(x * sc + sh (+ res)) with sc = invstd * gamma, sh = beta - mean * sc per
// channel (invstd null: eval, 1 / sqrt(var + eps)); zo, when set, receives the activation's input.
template <int VEC>
__global__ void __launch_bounds__(256) bn_nhwc_apply_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ mean,
                                                            const float* __restrict__ invstd,
                                                            const float* __restrict__ var, double eps,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ beta,
                                                            const float* __restrict__ res, float* __restrict__ y,
                                                            float* __restrict__ zo, int c, int act, const NhwcSplit sp,
                                                            int64_t rows_per_chunk) {
  using V = typename VecT<VEC>::T;
  const int jl = threadIdx.x % sp.cb, lane = threadIdx.x / sp.cb, j = blockIdx.x * sp.cb + jl;
  if (lane >= sp.rl || j >= sp.cv) return;
  float sc[VEC], sh[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const int ch = j * VEC + i;
    const float inv = invstd ? invstd[ch] : (float)(1.0 / sqrt((double)var[ch] + eps));
    sc[i] = inv * gamma[ch];
    sh[i] = beta[ch] - mean[ch] * sc[i];
  }
  const int64_t r0 = blockIdx.y * rows_per_chunk, r1 = min64(sp.rows, r0 + rows_per_chunk);
  for (int64_t r = r0 + lane; r < r1; r += sp.rl) {
    const int64_t off = r * c + (int64_t)j * VEC;
    V v = *reinterpret_cast<const V*>(x + off), q, z;
    if (res) q = *reinterpret_cast<const V*>(res + off);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float f = fmaf(vget(v, i), sc[i], sh[i]);
      if (res) f += vget(q, i);
      vset(z, i, f);
      vset(v, i, bn_act(f, act));
    }
    if (zo) *reinterpret_cast<V*>(zo + off) = z;
    *reinterpret_cast<V*>(y + off) = v;
  }
}

// grid (cblocks, slices): per (channel, slice) sum gz and sum gz * xhat, gz = (g + g2) through the activation's
// gradient (ry: the ReLU's output or the hardswish's input; null: none)
template <int VEC>
__global__ void __launch_bounds__(256) bn_nhwc_bwd_part_kernel(const float* __restrict__ g,
                                                               const float* __restrict__ g2,
                                                               const float* __restrict__ x,
                                                               const float* __restrict__ ry,
                                                               const float* __restrict__ mean,
                                                               const float* __restrict__ invstd,
                                                               double* __restrict__ part, int c, int act,
                                                               const NhwcSplit sp, int g_nchw) {
  using V = typename VecT<VEC>::T;
  const int jl = threadIdx.x % sp.cb, lane = threadIdx.x / sp.cb, j = blockIdx.x * sp.cb + jl;
  const bool on = lane < sp.rl && j < sp.cv;
  double s1[VEC], s2[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) s1[i] = 0.0, s2[i] = 0.0;
  if (on) {
    float mu[VEC], inv[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) mu[i] = mean[j * VEC + i], inv[i] = invstd[j * VEC + i];
    const int64_t r0 = blockIdx.y * sp.per_slice, r1 = min64(sp.rows, r0 + sp.per_slice);
    const int64_t step = sp.rl;
    for (int64_t r = r0 + lane; r < r1; r += 4 * step) {
      V vg[4], vx[4], vr[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (r + u * step < r1) {
          const int64_t off = (r + u * step) * c + (int64_t)j * VEC;
          vg[u] = nhwc_grad<VEC>(g, g_nchw, r + u * step, j, c, sp);
          if (g2) vadd(vg[u], *reinterpret_cast<const V*>(g2 + off));
          vx[u] = *reinterpret_cast<const V*>(x + off);
          if (ry) vr[u] = *reinterpret_cast<const V*>(ry + off);
        } else {
#pragma unroll
          for (int i = 0; i < VEC; ++i) {
            vset(vg[u], i, 0.f);  // gz = 0 contributes nothing
            vset(vx[u], i, mu[i]);
            vset(vr[u], i, 1.f);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          float gz = vget(vg[u], i);
          if (ry) gz = bn_act_grad(gz, vget(vr[u], i), act);
          const float xhat = (vget(vx[u], i) - mu[i]) * inv[i];
          s1[i] += (double)gz;
          s2[i] += (double)gz * (double)xhat;
        }
    }
  }
  double o1, o2;
  nhwc_lane_sums<VEC>(sp, s1, s2, o1, o2);
  const int q = threadIdx.x;
  if (q < sp.cb * VEC) {
    const int ch = (blockIdx.x * sp.cb + q / VEC) * VEC + q % VEC;
    if (ch < c) {
      part[((int64_t)ch * sp.slices + blockIdx.y) * 2] = o1;
      part[((int64_t)ch * sp.slices + blockIdx.y) * 2 + 1] = o2;
    }
  }
}

// one wave per channel: dbeta = sum gz, dgamma = sum gz * xhat, and the input-gradient constants kc[ch][5]
__global__ void __launch_bounds__(256) bn_nhwc_bwd_fin_kernel(const double* __restrict__ part, int c, int slices,
                                                              const float* __restrict__ mean,
                                                              const float* __restrict__ invstd,
                                                              const float* __restrict__ gamma, double m,
                                                              float* __restrict__ kc, float* __restrict__ dgamma,
                                                              float* __restrict__ dbeta) {
  const int ch = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (ch >= c) return;  // whole waves
  double s1, s2;
  nhwc_wave_slices(part, ch, slices, s1, s2);
  if ((threadIdx.x & 63) == 0) {
    if (dbeta) dbeta[ch] = (float)s1;
    if (dgamma) dgamma[ch] = (float)s2;
    if (gamma) bn_bwd_consts(s1, s2, m, gamma[ch], mean[ch], invstd[ch], kc + ch * 5);
  }
}

// grid (cblocks, chunks of rows): gx = k1 gz - k2 - k3 xhat per channel; gzo, when set, receives gz
template <int VEC>
__global__ void __launch_bounds__(256) bn_nhwc_bwd_apply_kernel(const float* __restrict__ g,
                                                                const float* __restrict__ g2,
                                                                const float* __restrict__ x,
                                                                const float* __restrict__ ry,
                                                                const float* __restrict__ kc, float* __restrict__ gx,
                                                                float* __restrict__ gzo, int c, int act,
                                                                const NhwcSplit sp, int64_t rows_per_chunk,
                                                                int g_nchw) {
  using V = typename VecT<VEC>::T;
  const int jl = threadIdx.x % sp.cb, lane = threadIdx.x / sp.cb, j = blockIdx.x * sp.cb + jl;
  if (lane >= sp.rl || j >= sp.cv) return;
  float k[VEC][5];
#pragma unroll
  for (int i = 0; i < VEC; ++i)
#pragma unroll
    for (int e = 0; e < 5; ++e) k[i][e] = kc[(j * VEC + i) * 5 + e];
  const int64_t r0 = blockIdx.y * rows_per_chunk, r1 = min64(sp.rows, r0 + rows_per_chunk);
  for (int64_t r = r0 + lane; r < r1; r += sp.rl) {
    const int64_t off = r * c + (int64_t)j * VEC;
    V vg = nhwc_grad<VEC>(g, g_nchw, r, j, c, sp);
    if (g2) vadd(vg, *reinterpret_cast<const V*>(g2 + off));
    const V vx = *reinterpret_cast<const V*>(x + off);
    V vr = vg;
    if (ry) vr = *reinterpret_cast<const V*>(ry + off);
    V o, z;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float gz = vget(vg, i);
      if (ry) gz = bn_act_grad(gz, vget(vr, i), act);
      vset(z, i, gz);
      vset(o, i, bwd_elem(gz, vget(vx, i), 1.f, false, k[i]));
    }
    if (gx) *reinterpret_cast<V*>(gx + off) = o;
    if (gzo) *reinterpret_cast<V*>(gzo + off) = z;
  }
}

// A channels-last BatchNorm of at most kNhwcFusedRows rows runs in one launch instead of three: workgroup j owns
// channel vector j (VEC channels) over every row, thread t rows t, t + blockDim.x, ... (RPT of them, in registers),
// so the sums, the finalize and the apply need no partials. Each lane reads VEC channels of a row, a 16-byte run rows
// apart: one workgroup reads its vector at the rate one CU fetches scattered lines, which the shortest tensors
// (ResNet-18 b32 64²'s last three stages: 2048 rows and fewer) finish sooner than three launches; at 8192 rows (eight
// per thread) the one workgroup per vector is slower than three launches over the whole chip. The backward keeps gz
// (through the activation) and x, not g and ry.
// The sums are the shifted float64 sums of the three-launch path in another order (each thread's rows in order, the
// wave sums in wave order); the finalize and apply arithmetic is the same.
constexpr int64_t kNhwcFusedRows = 2048;
constexpr int kNhwcFusedRpt = 2;

static bool nhwc_fused_ok(const NhwcSplit& sp) { return sp.rows <= kNhwcFusedRows; }
static unsigned nhwc_fused_threads(const NhwcSplit& sp) {
  const int64_t t = cdiv(cdiv(sp.rows, kNhwcFusedRpt), 64) * 64;
  return (unsigned)(t < 64 ? 64 : t);
}

// Block sums of VEC pairs of doubles over blockDim.x threads (whole waves, at most 1024): the wave sums added in
// wave order, pair i valid in thread i.
template <int VEC>
__device__ __forceinline__ void nhwc_block_sums(double* a, double* b) {
  __shared__ double sa[16][VEC], sb[16][VEC];
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    a[i] = wave_sum(a[i]);
    b[i] = wave_sum(b[i]);
    if ((threadIdx.x & 63) == 0) sa[wave][i] = a[i], sb[wave][i] = b[i];
  }
  __syncthreads();
  if ((int)threadIdx.x < VEC) {
    const int i = threadIdx.x;
    double s = sa[0][i], q = sb[0][i];
    for (int w = 1; w < nw; ++w) s += sa[w][i], q += sb[w][i];
    a[0] = s, b[0] = q;
  }
}

// grid cv (channel vectors), blockDim nhwc_fused_threads: the training forward of bn_nhwc_stats_kernel,
// bn_nhwc_fin_kernel and bn_nhwc_apply_kernel in one pass over x
template <int VEC, int RPT>
__global__ void __launch_bounds__(1024) bn_nhwc_fused_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta, const float* rm,
                                                             const float* rv, double momentum, double eps,
                                                             const float* __restrict__ res, float* __restrict__ y,
                                                             float* __restrict__ zo, float* __restrict__ save_mean,
                                                             float* __restrict__ save_invstd, float* new_rm,
                                                             float* new_rv,  // may alias rm / rv
                                                             int c, int act, int64_t rows) {
  using V = typename VecT<VEC>::T;
  __shared__ float coef[2][VEC];
  const int j = blockIdx.x, nt = blockDim.x;
  const V shift = *reinterpret_cast<const V*>(x + (int64_t)j * VEC);
  V r[RPT];
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int64_t row = threadIdx.x + (int64_t)u * nt;
    r[u] = row < rows ? *reinterpret_cast<const V*>(x + row * c + (int64_t)j * VEC) : shift;  // d = 0 past the end
  }
  double s1[VEC], s2[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    s1[i] = 0.0, s2[i] = 0.0;
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
      const double d = (double)(vget(r[u], i) - vget(shift, i));
      s1[i] += d;
      s2[i] += d * d;
    }
  }
  nhwc_block_sums<VEC>(s1, s2);
  if ((int)threadIdx.x < VEC) {
    const int i = threadIdx.x, ch = j * VEC + i;
    const BnStats st = bn_finalize(s1[0], s2[0], (double)x[ch], (double)rows, momentum, eps, rm, rv, save_mean,
                                   save_invstd, new_rm, new_rv, ch, true);
    const float sc = st.invstd * gamma[ch];
    coef[0][i] = sc;
    coef[1][i] = beta[ch] - st.mean * sc;
  }
  __syncthreads();
  float sc[VEC], sh[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) sc[i] = coef[0][i], sh[i] = coef[1][i];
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int64_t row = threadIdx.x + (int64_t)u * nt;
    if (row < rows) {
      const int64_t off = row * c + (int64_t)j * VEC;
      V v = r[u], q, z;
      if (res) q = *reinterpret_cast<const V*>(res + off);
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        float f = fmaf(vget(v, i), sc[i], sh[i]);
        if (res) f += vget(q, i);
        vset(z, i, f);
        vset(v, i, bn_act(f, act));
      }
      if (zo) *reinterpret_cast<V*>(zo + off) = z;
      *reinterpret_cast<V*>(y + off) = v;
    }
  }
}

// grid cv, blockDim nhwc_fused_threads: bn_nhwc_bwd_part_kernel, bn_nhwc_bwd_fin_kernel and bn_nhwc_bwd_apply_kernel
// in one pass over g (+ g2), x and ry
template <int VEC, int RPT>
__global__ void __launch_bounds__(1024) bn_nhwc_bwd_fused_kernel(const float* __restrict__ g,
                                                                 const float* __restrict__ g2,
                                                                 const float* __restrict__ x,
                                                                 const float* __restrict__ ry,
                                                                 const float* __restrict__ mean,
                                                                 const float* __restrict__ invstd,
                                                                 const float* __restrict__ gamma,
                                                                 float* __restrict__ gx, float* __restrict__ dgamma,
                                                                 float* __restrict__ dbeta, float* __restrict__ gzo,
                                                                 int c, int act, const NhwcSplit sp, int g_nchw) {
  using V = typename VecT<VEC>::T;
  __shared__ float kc[VEC][5];
  const int j = blockIdx.x, nt = blockDim.x;
  float mu[VEC], inv[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) mu[i] = mean[j * VEC + i], inv[i] = invstd[j * VEC + i];
  V vg[RPT], vx[RPT];  // vg: gz, the gradient through the activation
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int64_t row = threadIdx.x + (int64_t)u * nt;
    if (row < sp.rows) {
      const int64_t off = row * c + (int64_t)j * VEC;
      vg[u] = nhwc_grad<VEC>(g, g_nchw, row, j, c, sp);
      if (g2) vadd(vg[u], *reinterpret_cast<const V*>(g2 + off));
      vx[u] = *reinterpret_cast<const V*>(x + off);
      if (ry) {
        const V vr = *reinterpret_cast<const V*>(ry + off);
#pragma unroll
        for (int i = 0; i < VEC; ++i) vset(vg[u], i, bn_act_grad(vget(vg[u], i), vget(vr, i), act));
      }
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        vset(vg[u], i, 0.f);  // gz = 0 contributes nothing
        vset(vx[u], i, mu[i]);
      }
    }
  }
  double s1[VEC], s2[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    s1[i] = 0.0, s2[i] = 0.0;
#pragma unroll
    for (int u = 0; u < RPT; ++u) {
      const float gz = vget(vg[u], i);
      const float xhat = (vget(vx[u], i) - mu[i]) * inv[i];
      s1[i] += (double)gz;
      s2[i] += (double)gz * (double)xhat;
    }
  }
  nhwc_block_sums<VEC>(s1, s2);
  if ((int)threadIdx.x < VEC) {
    const int i = threadIdx.x, ch = j * VEC + i;
    if (dbeta) dbeta[ch] = (float)s1[0];
    if (dgamma) dgamma[ch] = (float)s2[0];
    if (gx) bn_bwd_consts(s1[0], s2[0], (double)sp.rows, gamma[ch], mu[i], inv[i], kc[i]);
  }
  if (!gx && !gzo) return;  // uniform
  __syncthreads();
  float k[VEC][5];
#pragma unroll
  for (int i = 0; i < VEC; ++i)
#pragma unroll
    for (int e = 0; e < 5; ++e) k[i][e] = kc[i][e];
#pragma unroll
  for (int u = 0; u < RPT; ++u) {
    const int64_t row = threadIdx.x + (int64_t)u * nt;
    if (row < sp.rows) {
      const int64_t off = row * c + (int64_t)j * VEC;
      V o;
#pragma unroll
      for (int i = 0; i < VEC; ++i) vset(o, i, bwd_elem(vget(vg[u], i), vget(vx[u], i), 1.f, false, k[i]));
      if (gx) *reinterpret_cast<V*>(gx + off) = o;
      if (gzo) *reinterpret_cast<V*>(gzo + off) = vg[u];
    }
  }
}

// apply-pass grid: (cblocks, chunks of about 8 rows per thread)
static dim3 nhwc_apply_grid(const NhwcSplit& sp, int64_t& rows_per_chunk) {
  rows_per_chunk = 8 * (int64_t)sp.rl;
  int64_t chunks = cdiv(sp.rows, rows_per_chunk);
  if (chunks > 65535) {
    chunks = 65535;
    rows_per_chunk = cdiv(sp.rows, chunks);
  }
  return dim3((unsigned)sp.cblocks, (unsigned)chunks);
}

static bool nhwc_size_ok(int64_t n, int64_t c, int64_t hw) {
  return bn_size_ok(n, c, hw) && n * hw * c < ((int64_t)1 << 46);
}

}  // namespace omt

using namespace omt;

// [c][kNhwcMaxSlices][2] double partials, then [c][5] float constants of the input-gradient map
OMT_EXPORT size_t omt_bn_nhwc_workspace(int64_t n, int64_t c, int64_t hw) {
  (void)n;
  (void)hw;
  return (size_t)(c * kNhwcMaxSlices * 2) * sizeof(double) + (size_t)(c * 5) * sizeof(float);
}

OMT_EXPORT int omt_bn_train_fwd_nhwc(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma,
                                     const float* beta, const float* running_mean, const float* running_var,
                                     double momentum, double eps, int act, const float* residual, float* y, float* z,
                                     float* save_mean, float* save_invstd, float* new_rm, float* new_rv,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  if (!x || !gamma || !beta || !y || !save_mean || !save_invstd)
    return fail(OMT_INVALID, "omt_bn_train_fwd_nhwc: null pointer");
  if (act < OMT_ACT_NONE || act > OMT_ACT_HARDSWISH)
    return fail(OMT_INVALID, "omt_bn_train_fwd_nhwc: activation %d", act);
  if (!nhwc_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_train_fwd_nhwc: size not covered");
  if (!workspace || workspace_bytes < omt_bn_nhwc_workspace(n, c, hw))
    return fail(OMT_INVALID, "omt_bn_train_fwd_nhwc: workspace too small");
  hipStream_t s = stream_of(stream);
  const NhwcSplit sp = nhwc_split(n, c, hw, al16(x) && al16(y) && al16(residual) && al16(z));
  if (nhwc_fused_ok(sp)) {
#define OMT_NHWC_FUSED(V, R)                                                                                       \
  hipLaunchKernelGGL((bn_nhwc_fused_kernel<V, R>), dim3((unsigned)sp.cv), dim3(nhwc_fused_threads(sp)), 0, s, x, gamma, \
                     beta, running_mean, running_var, momentum, eps, residual, y, z, save_mean, save_invstd, new_rm,   \
                     new_rv, (int)c, act, sp.rows)
    if (sp.vec == 4)
      OMT_NHWC_FUSED(4, kNhwcFusedRpt);
    else
      OMT_NHWC_FUSED(1, kNhwcFusedRpt);
#undef OMT_NHWC_FUSED
    return launch_check("bn_nhwc_fused_kernel");
  }
  double* part = (double*)workspace;
  const dim3 sg((unsigned)sp.cblocks, (unsigned)sp.slices);
  if (sp.vec == 4)
    hipLaunchKernelGGL(bn_nhwc_stats_kernel<4>, sg, dim3(256), 0, s, x, part, (int)c, sp);
  else
    hipLaunchKernelGGL(bn_nhwc_stats_kernel<1>, sg, dim3(256), 0, s, x, part, (int)c, sp);
  if (int st = launch_check("bn_nhwc_stats_kernel")) return st;
  hipLaunchKernelGGL(bn_nhwc_fin_kernel, dim3((unsigned)cdiv(c, 4)), dim3(256), 0, s, x, (const double*)part, (int)c,
                     sp.slices, (double)(n * hw), momentum, eps, running_mean, running_var, save_mean, save_invstd,
                     new_rm, new_rv);
  if (int st = launch_check("bn_nhwc_fin_kernel")) return st;
  int64_t rpc;
  const dim3 ag = nhwc_apply_grid(sp, rpc);
  if (sp.vec == 4)
    hipLaunchKernelGGL(bn_nhwc_apply_kernel<4>, ag, dim3(256), 0, s, x, save_mean, save_invstd, nullptr, 0.0, gamma,
                       beta, residual, y, z, (int)c, act, sp, rpc);
  else
    hipLaunchKernelGGL(bn_nhwc_apply_kernel<1>, ag, dim3(256), 0, s, x, save_mean, save_invstd, nullptr, 0.0, gamma,
                       beta, residual, y, z, (int)c, act, sp, rpc);
  return launch_check("bn_nhwc_apply_kernel");
}

OMT_EXPORT int omt_bn_eval_fwd_nhwc(int64_t n, int64_t c, int64_t hw, const float* x, const float* gamma,
                                    const float* beta, const float* running_mean, const float* running_var,
                                    double eps, int act, float* y, void* stream) {
  if (!x || !gamma || !beta || !running_mean || !running_var || !y)
    return fail(OMT_INVALID, "omt_bn_eval_fwd_nhwc: null pointer");
  if (act < OMT_ACT_NONE || act > OMT_ACT_HARDSWISH)
    return fail(OMT_INVALID, "omt_bn_eval_fwd_nhwc: activation %d", act);
  if (!nhwc_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_eval_fwd_nhwc: size not covered");
  hipStream_t s = stream_of(stream);
  const NhwcSplit sp = nhwc_split(n, c, hw, al16(x) && al16(y));
  int64_t rpc;
  const dim3 ag = nhwc_apply_grid(sp, rpc);
  if (sp.vec == 4)
    hipLaunchKernelGGL(bn_nhwc_apply_kernel<4>, ag, dim3(256), 0, s, x, running_mean, nullptr, running_var, eps, gamma,
                       beta, nullptr, y, nullptr, (int)c, act, sp, rpc);
  else
    hipLaunchKernelGGL(bn_nhwc_apply_kernel<1>, ag, dim3(256), 0, s, x, running_mean, nullptr, running_var, eps, gamma,
                       beta, nullptr, y, nullptr, (int)c, act, sp, rpc);
  return launch_check("bn_nhwc_apply_kernel");
}

OMT_EXPORT int omt_bn_bwd_nhwc(int64_t n, int64_t c, int64_t hw, const float* g, int g_nchw, const float* g2,
                               const float* x, int act, const float* act_in, const float* save_mean,
                               const float* save_invstd, const float* gamma, float* gx, float* dgamma, float* dbeta,
                               float* gz, void* workspace, size_t workspace_bytes, void* stream) {
  if (!g || !x || !save_mean || !save_invstd || ((gx || gz) && !gamma) || (act != OMT_ACT_NONE && !act_in))
    return fail(OMT_INVALID, "omt_bn_bwd_nhwc: null pointer");
  if (act < OMT_ACT_NONE || act > OMT_ACT_HARDSWISH) return fail(OMT_INVALID, "omt_bn_bwd_nhwc: activation %d", act);
  if (!nhwc_size_ok(n, c, hw)) return fail(OMT_UNSUPPORTED, "omt_bn_bwd_nhwc: size not covered");
  if (!workspace || workspace_bytes < omt_bn_nhwc_workspace(n, c, hw))
    return fail(OMT_INVALID, "omt_bn_bwd_nhwc: workspace too small");
  hipStream_t s = stream_of(stream);
  const float* ry = act == OMT_ACT_NONE ? nullptr : act_in;
  const NhwcSplit sp =
      nhwc_split(n, c, hw, (g_nchw || al16(g)) && al16(g2) && al16(x) && al16(ry) && al16(gx) && al16(gz));
  if (nhwc_fused_ok(sp)) {
    const float* gam = (gx || gz) ? gamma : nullptr;
#define OMT_NHWC_BWD_FUSED(V, R)                                                                                   \
  hipLaunchKernelGGL((bn_nhwc_bwd_fused_kernel<V, R>), dim3((unsigned)sp.cv), dim3(nhwc_fused_threads(sp)), 0, s, g,    \
                     g2, x, ry, save_mean, save_invstd, gam, gx, dgamma, dbeta, gz, (int)c, act, sp, g_nchw ? 1 : 0)
    if (sp.vec == 4)
      OMT_NHWC_BWD_FUSED(4, kNhwcFusedRpt);
    else
      OMT_NHWC_BWD_FUSED(1, kNhwcFusedRpt);
#undef OMT_NHWC_BWD_FUSED
    return launch_check("bn_nhwc_bwd_fused_kernel");
  }
  double* part = (double*)workspace;
  float* kc = (float*)(part + c * kNhwcMaxSlices * 2);
  const dim3 pg((unsigned)sp.cblocks, (unsigned)sp.slices);
  if (sp.vec == 4)
    hipLaunchKernelGGL(bn_nhwc_bwd_part_kernel<4>, pg, dim3(256), 0, s, g, g2, x, ry, save_mean, save_invstd, part,
                       (int)c, act, sp, g_nchw ? 1 : 0);
  else
    hipLaunchKernelGGL(bn_nhwc_bwd_part_kernel<1>, pg, dim3(256), 0, s, g, g2, x, ry, save_mean, save_invstd, part,
                       (int)c, act, sp, g_nchw ? 1 : 0);
  if (int st = launch_check("bn_nhwc_bwd_part_kernel")) return st;
  hipLaunchKernelGGL(bn_nhwc_bwd_fin_kernel, dim3((unsigned)cdiv(c, 4)), dim3(256), 0, s, (const double*)part, (int)c,
                     sp.slices, save_mean, save_invstd, (gx || gz) ? gamma : nullptr, (double)(n * hw), kc, dgamma,
                     dbeta);
  if (int st = launch_check("bn_nhwc_bwd_fin_kernel")) return st;
  if (!gx && !gz) return OMT_OK;
  int64_t rpc;
  const dim3 ag = nhwc_apply_grid(sp, rpc);
  if (sp.vec == 4)
    hipLaunchKernelGGL(bn_nhwc_bwd_apply_kernel<4>, ag, dim3(256), 0, s, g, g2, x, ry, (const float*)kc, gx, gz,
                       (int)c, act, sp, rpc, g_nchw ? 1 : 0);
  else
    hipLaunchKernelGGL(bn_nhwc_bwd_apply_kernel<1>, ag, dim3(256), 0, s, g, g2, x, ry, (const float*)kc, gx, gz,
                       (int)c, act, sp, rpc, g_nchw ? 1 : 0);
  return launch_check("bn_nhwc_bwd_apply_kernel");
}
