// Depthwise convolution (groups = C, one ks x ks filter per channel): any ks <= 11, stride 1..4, 0 <= pad <= ks.
// These are HBM-bandwidth-bound (ks^2 FLOPs per loaded element), so they run as plain wave64 kernels:
//  - forward: one thread per output element, the filter in registers (reference dw_fwd / dwg_fwd / dw_fwd_bn,
//    csrc/conv.cpp:194-198, csrc/plans.cpp:145-158), optional previous-layer eval BN + ReLU on in-bounds taps;
//  - grad input: one thread per input element, keeping the taps that land on the stride grid (dw_gin / dwg_gin);
//  - grad weight: workgroup (channel, slice) accumulates every tap over its share of n * oh * ow, partials summed in
//    slice order (dw_gwt / dwg_gwt).
#include "omt_internal.h"

namespace omt {

struct DwGeo {
  int n, c, ih, iw, oh, ow, ks, s, p;
};

__global__ void __launch_bounds__(256) dw_fwd_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                     const float* __restrict__ bias, const float* __restrict__ bm,
                                                     const float* __restrict__ bv, const float* __restrict__ bg,
                                                     const float* __restrict__ bb, float eps, float* __restrict__ y,
                                                     int64_t total, DwGeo g) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int ox = (int)(i % g.ow), oy = (int)((i / g.ow) % g.oh);
    const int64_t plane = i / ((int64_t)g.ow * g.oh);
    const int ch = (int)(plane % g.c);
    const float* xp = x + plane * g.ih * g.iw;
    const float* wp = w + ch * g.ks * g.ks;
    float sc = 1.f, sh = 0.f;
    if (bm) {
      const float inv = rsqrtf(bv[ch] + eps);
      sc = inv * bg[ch];
      sh = bb[ch] - bm[ch] * sc;
    }
    const int y0 = oy * g.s - g.p, x0 = ox * g.s - g.p;
    float acc = 0.f;
    for (int ky = 0; ky < g.ks; ++ky) {
      const int yy = y0 + ky;
      if ((unsigned)yy >= (unsigned)g.ih) continue;
      for (int kx = 0; kx < g.ks; ++kx) {
        const int xx = x0 + kx;
        if ((unsigned)xx >= (unsigned)g.iw) continue;
        float v = xp[yy * g.iw + xx];
        if (bm) v = fmaxf(fmaf(v, sc, sh), 0.f);
        acc = fmaf(v, wp[ky * g.ks + kx], acc);
      }
    }
    if (bias) acc += bias[ch];
    y[i] = acc;
  }
}

__global__ void __launch_bounds__(256) dw_dgrad_kernel(const float* __restrict__ gy, const float* __restrict__ w,
                                                       float* __restrict__ gx, int64_t total, DwGeo g) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int xx = (int)(i % g.iw), yy = (int)((i / g.iw) % g.ih);
    const int64_t plane = i / ((int64_t)g.iw * g.ih);
    const int ch = (int)(plane % g.c);
    const float* gp = gy + plane * g.oh * g.ow;
    const float* wp = w + ch * g.ks * g.ks;
    float acc = 0.f;
    for (int ky = 0; ky < g.ks; ++ky) {
      const int ty = yy + g.p - ky;
      if (ty < 0 || ty % g.s) continue;
      const int oy = ty / g.s;
      if (oy >= g.oh) continue;
      for (int kx = 0; kx < g.ks; ++kx) {
        const int tx = xx + g.p - kx;
        if (tx < 0 || tx % g.s) continue;
        const int ox = tx / g.s;
        if (ox >= g.ow) continue;
        acc = fmaf(gp[oy * g.ow + ox], wp[ky * g.ks + kx], acc);
      }
    }
    gx[i] = acc;
  }
}

// grid (c, slices). Each thread owns output pixels and accumulates all taps in registers (KS known at compile time
// for the common 3/5/7; 0 = runtime ks, one tap at a time).
template <int KS>
__global__ void __launch_bounds__(256) dw_wgrad_part_kernel(const float* __restrict__ x, const float* __restrict__ gy,
                                                            float* __restrict__ part, DwGeo g, int per_slice) {
  const int ch = blockIdx.x, sl = blockIdx.y;
  const int ks = KS ? KS : g.ks, kk = ks * ks;
  const int ohw = g.oh * g.ow, total = g.n * ohw;
  const int k0 = sl * per_slice, k1 = min(total, k0 + per_slice);
  __shared__ float red[4][121];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (KS) {
    float acc[KS * KS > 0 ? KS * KS : 1];
#pragma unroll
    for (int t = 0; t < KS * KS; ++t) acc[t] = 0.f;
    for (int k = k0 + threadIdx.x; k < k1; k += 256) {
      const int n = k / ohw, r = k % ohw, oy = r / g.ow, ox = r % g.ow;
      const float gv = gy[((int64_t)n * g.c + ch) * ohw + r];
      const float* xp = x + ((int64_t)n * g.c + ch) * g.ih * g.iw;
      const int y0 = oy * g.s - g.p, x0 = ox * g.s - g.p;
#pragma unroll
      for (int ky = 0; ky < KS; ++ky)
#pragma unroll
        for (int kx = 0; kx < KS; ++kx) {
          const int yy = y0 + ky, xx = x0 + kx;
          if ((unsigned)yy < (unsigned)g.ih && (unsigned)xx < (unsigned)g.iw)
            acc[ky * KS + kx] = fmaf(gv, xp[yy * g.iw + xx], acc[ky * KS + kx]);
        }
    }
#pragma unroll
    for (int t = 0; t < KS * KS; ++t) {
      float v = acc[t];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      if (lane == 0) red[wave][t] = v;
    }
  } else {
    for (int t = 0; t < kk; ++t) {
      const int ky = t / ks, kx = t % ks;
      float v = 0.f;
      for (int k = k0 + threadIdx.x; k < k1; k += 256) {
        const int n = k / ohw, r = k % ohw, oy = r / g.ow, ox = r % g.ow;
        const int yy = oy * g.s - g.p + ky, xx = ox * g.s - g.p + kx;
        if ((unsigned)yy < (unsigned)g.ih && (unsigned)xx < (unsigned)g.iw)
          v = fmaf(gy[((int64_t)n * g.c + ch) * ohw + r], x[((int64_t)n * g.c + ch) * g.ih * g.iw + yy * g.iw + xx], v);
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      if (lane == 0) red[wave][t] = v;
    }
  }
  __syncthreads();
  for (int t = threadIdx.x; t < kk; t += 256)
    part[((int64_t)sl * g.c + ch) * kk + t] = red[0][t] + red[1][t] + red[2][t] + red[3][t];
}

__global__ void __launch_bounds__(256) dw_wgrad_reduce_kernel(const float* __restrict__ part, float* __restrict__ gw,
                                                              int n, int slices) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int z = 0; z < slices; ++z) s += part[(int64_t)z * n + i];
    gw[i] = s;
  }
}

static bool dw_ok(const omt_conv_geo* g) {
  const int64_t lim = (int64_t)1 << 31;
  return g->ci == g->co && g->n >= 1 && g->ci >= 1 && g->ks >= 1 && g->ks <= 11 && g->stride >= 1 &&
         g->stride <= 4 && g->pad >= 0 && g->pad <= g->ks && g->oh >= 1 && g->ow >= 1 &&
         g->oh == (g->ih + 2 * g->pad - g->ks) / g->stride + 1 && g->ow == (g->iw + 2 * g->pad - g->ks) / g->stride + 1 &&
         g->n * g->oh * g->ow < lim && g->ih * g->iw < lim && g->n * g->ci * g->ih * g->iw < ((int64_t)1 << 46);
}

static DwGeo dgeo(const omt_conv_geo* g) {
  return DwGeo{(int)g->n, (int)g->ci, (int)g->ih, (int)g->iw, (int)g->oh, (int)g->ow, (int)g->ks, (int)g->stride,
               (int)g->pad};
}

static int64_t dw_slices(const omt_conv_geo* g) {
  int64_t total = g->n * g->oh * g->ow;
  int64_t want = cdiv(1024, g->ci);
  int64_t cap = cdiv(total, 1024);
  if (want > cap) want = cap;
  return want < 1 ? 1 : want;
}

}  // namespace omt

using namespace omt;

OMT_EXPORT int omt_dw_fwd(const omt_conv_geo* g, const float* x, const float* w, const float* bias,
                          const float* bn_mean, const float* bn_var, const float* bn_gamma, const float* bn_beta,
                          float bn_eps, float* y, void* stream) {
  if (!g || !x || !w || !y) return fail(OMT_INVALID, "omt_dw_fwd: null pointer");
  if (!dw_ok(g)) return fail(OMT_UNSUPPORTED, "omt_dw_fwd: geometry not covered");
  const bool bn = bn_mean || bn_var || bn_gamma || bn_beta;
  if (bn && !(bn_mean && bn_var && bn_gamma && bn_beta)) return fail(OMT_INVALID, "omt_dw_fwd: incomplete BN loader");
  const int64_t total = g->n * g->co * g->oh * g->ow;
  hipLaunchKernelGGL(dw_fwd_kernel, dim3(grid1d(total, 256)), dim3(256), 0, stream_of(stream), x, w, bias,
                     bn ? bn_mean : nullptr, bn_var, bn_gamma, bn_beta, bn_eps, y, total, dgeo(g));
  return launch_check("dw_fwd_kernel");
}

OMT_EXPORT int omt_dw_dgrad(const omt_conv_geo* g, const float* gy, const float* w, float* gx, void* stream) {
  if (!g || !gy || !w || !gx) return fail(OMT_INVALID, "omt_dw_dgrad: null pointer");
  if (!dw_ok(g)) return fail(OMT_UNSUPPORTED, "omt_dw_dgrad: geometry not covered");
  const int64_t total = g->n * g->ci * g->ih * g->iw;
  hipLaunchKernelGGL(dw_dgrad_kernel, dim3(grid1d(total, 256)), dim3(256), 0, stream_of(stream), gy, w, gx, total,
                     dgeo(g));
  return launch_check("dw_dgrad_kernel");
}

OMT_EXPORT size_t omt_dw_wgrad_workspace(const omt_conv_geo* g) {
  if (!g || !dw_ok(g)) return 0;
  return (size_t)(dw_slices(g) * g->ci * g->ks * g->ks) * sizeof(float);
}

OMT_EXPORT int omt_dw_wgrad(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (!g || !x || !gy || !gw) return fail(OMT_INVALID, "omt_dw_wgrad: null pointer");
  if (!dw_ok(g)) return fail(OMT_UNSUPPORTED, "omt_dw_wgrad: geometry not covered");
  if (!workspace || workspace_bytes < omt_dw_wgrad_workspace(g))
    return fail(OMT_INVALID, "omt_dw_wgrad: workspace of %zu bytes needed", omt_dw_wgrad_workspace(g));
  hipStream_t s = stream_of(stream);
  const int64_t slices = dw_slices(g);
  const int per_slice = (int)cdiv(g->n * g->oh * g->ow, slices);
  dim3 grid((unsigned)g->ci, (unsigned)slices);
  float* part = (float*)workspace;
  switch (g->ks) {
    case 3: hipLaunchKernelGGL(dw_wgrad_part_kernel<3>, grid, dim3(256), 0, s, x, gy, part, dgeo(g), per_slice); break;
    case 5: hipLaunchKernelGGL(dw_wgrad_part_kernel<5>, grid, dim3(256), 0, s, x, gy, part, dgeo(g), per_slice); break;
    case 7: hipLaunchKernelGGL(dw_wgrad_part_kernel<7>, grid, dim3(256), 0, s, x, gy, part, dgeo(g), per_slice); break;
    default: hipLaunchKernelGGL(dw_wgrad_part_kernel<0>, grid, dim3(256), 0, s, x, gy, part, dgeo(g), per_slice); break;
  }
  if (int st = launch_check("dw_wgrad_part_kernel")) return st;
  const int n = (int)(g->ci * g->ks * g->ks);
  hipLaunchKernelGGL(dw_wgrad_reduce_kernel, dim3(grid1d(n, 256, 4096)), dim3(256), 0, s, (const float*)part, gw, n,
                     (int)slices);
  return launch_check("dw_wgrad_reduce_kernel");
}
