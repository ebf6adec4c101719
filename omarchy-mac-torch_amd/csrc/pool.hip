// Pooling over NCHW float32 planes (planes = n * c): max (any window / stride / padding / dilation, int64 indices),
// average (PyTorch divisor rules) and adaptive average. Backward passes gather rather than scatter: each input
// element sums the gradients of the outputs that selected or covered it, visiting those outputs in row-major order,
// which is the order PyTorch's CPU backward scatters them in, so no atomics are needed and the sums are
// deterministic. One thread per output (forward) or input (backward) element; HBM-bandwidth-bound. Tensors below 2^32
// elements decompose flat indices with 32-bit multiply-high division (the I32 kernels); larger ones with 64-bit
// arithmetic. Global average pooling stages small planes through LDS (one thread per plane, coalesced loads).
// Reference kernels: maxpool_gen_fwd/bwd, avgpool_gen_fwd/bwd, adapool_fwd/bwd (csrc/nn.cpp:157-222).
#include <algorithm>

#include "omt_internal.h"

namespace omt {

struct PoolGeo {
  int ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, dh, dw;
  FastDiv d_ow, d_ohw, d_iw, d_ihw, d_sh, d_sw;
};

struct Pos {
  int64_t plane;
  int y, x;
};
// (plane, row, col) of flat index i over planes of W columns and HW elements
template <bool I32>
__device__ __forceinline__ Pos decompose(int64_t i, int W, int HW, const FastDiv& dw, const FastDiv& dhw) {
  if (I32) {
    const uint32_t u = (uint32_t)i, pl = fdiv(u, dhw), r = u - pl * (uint32_t)HW, y = fdiv(r, dw);
    return {(int64_t)pl, (int)y, (int)(r - y * (uint32_t)W)};
  }
  const int64_t pl = i / HW;
  const int r = (int)(i - pl * HW);
  return {pl, r / W, r % W};
}
// q = t / d when d divides t exactly (t >= 0), else -1
__device__ __forceinline__ int exact_div(int t, int d, const FastDiv& fd) {
  const int q = (int)fdiv((uint32_t)t, fd);
  return q * d == t ? q : -1;
}

template <bool I32>
__global__ void __launch_bounds__(256) maxpool_fwd_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                          int64_t* __restrict__ idx, int64_t total, PoolGeo g) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const Pos o = decompose<I32>(i, g.ow, g.oh * g.ow, g.d_ow, g.d_ohw);
    const int ox = o.x, oy = o.y;
    const int64_t plane = o.plane;
    const float* xp = x + plane * g.ih * g.iw;
    float best = -INFINITY;
    int bi = -1;
    for (int ky = 0; ky < g.kh; ++ky) {
      const int yy = oy * g.sh - g.ph + ky * g.dh;
      if (yy < 0 || yy >= g.ih) continue;
      for (int kx = 0; kx < g.kw; ++kx) {
        const int xx = ox * g.sw - g.pw + kx * g.dw;
        if (xx < 0 || xx >= g.iw) continue;
        const float v = xp[yy * g.iw + xx];
        if (bi < 0 || v > best || isnan(v)) {  // first max wins ties; a NaN replaces the running max
          best = v;
          bi = yy * g.iw + xx;
        }
      }
    }
    y[i] = best;
    idx[i] = bi;
  }
}

// Square undilated K x K windows (K = 2, 3): the window is unrolled, so all of a thread's in-plane taps are loaded
// before the first compare (the loop above waits on one tap at a time); the compares run in the same row-major
// order with the same rule, so values and indices are those of the general kernel.
template <bool I32, int K>
__global__ void __launch_bounds__(256) maxpool_fwd_k_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                            int64_t* __restrict__ idx, int64_t total, PoolGeo g) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const Pos o = decompose<I32>(i, g.ow, g.oh * g.ow, g.d_ow, g.d_ohw);
    const float* xp = x + o.plane * g.ih * g.iw;
    const int y0 = o.y * g.sh - g.ph, x0 = o.x * g.sw - g.pw;
    float v[K * K];
    bool ok[K * K];
#pragma unroll
    for (int ky = 0; ky < K; ++ky)
#pragma unroll
      for (int kx = 0; kx < K; ++kx) {
        const int yy = y0 + ky, xx = x0 + kx, t = ky * K + kx;
        ok[t] = (unsigned)yy < (unsigned)g.ih && (unsigned)xx < (unsigned)g.iw;
        v[t] = ok[t] ? xp[yy * g.iw + xx] : 0.f;
      }
    float best = -INFINITY;
    int bi = -1;
#pragma unroll
    for (int t = 0; t < K * K; ++t)
      if (ok[t] && (bi < 0 || v[t] > best || isnan(v[t]))) {
        best = v[t];
        bi = (y0 + t / K) * g.iw + x0 + t % K;
      }
    y[i] = best;
    idx[i] = bi;
  }
}

// Square undilated K x K windows at stride S, four consecutive outputs of a row per thread (ow % 4 == 0, iw % 4 == 0,
// x below 2 GiB, x / y / idx 16-byte aligned): each input row the four windows cover is loaded as NV aligned float4
// runs starting at a = x0 - OFF (x0 rounded down to a multiple of 4, so OFF = (-pw) mod 4); runs outside the row or
// the plane read 0 through the buffer range check and the same bounds test as the per-output kernel excludes them.
// Each output compares its taps in row-major order with that kernel's rule, so values and indices are identical.
typedef long long omt_i64x2 __attribute__((ext_vector_type(2)));
template <int K, int S, int OFF>
__global__ void __launch_bounds__(256) maxpool_fwd_v4_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                             int64_t* __restrict__ idx, uint32_t total4, PoolGeo g,
                                                             uint32_t xbytes, FastDiv d_ow4, FastDiv d_oh) {
  constexpr int NV = (OFF + 3 * S + K + 3) / 4;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, xbytes);
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total4; i += gridDim.x * blockDim.x) {
    const uint32_t row = fdiv(i, d_ow4), ox = (i - row * (uint32_t)(g.ow >> 2)) * 4u;
    const uint32_t plane = fdiv(row, d_oh), oy = row - plane * (uint32_t)g.oh;
    const int y0 = (int)oy * S - g.ph, x0 = (int)ox * S - g.pw, a = x0 - OFF;
    const uint32_t pbase = plane * (uint32_t)g.ih * (uint32_t)g.iw;
    float v[K][4 * NV];
#pragma unroll
    for (int ky = 0; ky < K; ++ky) {
      const int yy = y0 + ky;
      const bool rin = (unsigned)yy < (unsigned)g.ih;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int c = a + 4 * j;
        const bool in = rin && (unsigned)c < (unsigned)g.iw;
        const float4 q = bload4(xr, in ? (pbase + (uint32_t)(yy * g.iw + c)) * 4u : kOOB, 0);
        v[ky][4 * j] = q.x;
        v[ky][4 * j + 1] = q.y;
        v[ky][4 * j + 2] = q.z;
        v[ky][4 * j + 3] = q.w;
      }
    }
    float best[4];
    int bi[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      best[e] = -INFINITY;
      bi[e] = -1;
#pragma unroll
      for (int ky = 0; ky < K; ++ky)
#pragma unroll
        for (int kx = 0; kx < K; ++kx) {
          const int yy = y0 + ky, xx = x0 + e * S + kx;
          const float val = v[ky][OFF + e * S + kx];
          if ((unsigned)yy < (unsigned)g.ih && (unsigned)xx < (unsigned)g.iw &&
              (bi[e] < 0 || val > best[e] || isnan(val))) {
            best[e] = val;
            bi[e] = yy * g.iw + xx;
          }
        }
    }
    const uint32_t o = row * (uint32_t)g.ow + ox;
    *reinterpret_cast<float4*>(y + o) = make_float4(best[0], best[1], best[2], best[3]);
    omt_i64x2* ip = reinterpret_cast<omt_i64x2*>(idx + o);
    ip[0] = omt_i64x2{bi[0], bi[1]};
    ip[1] = omt_i64x2{bi[2], bi[3]};
  }
}

// Undilated windows: the outputs whose window covers input (y, x) form the range oy in
// [ceil((y + p - k + 1) / s), floor((y + p) / s)] (clipped to the output) per axis, visited in ascending (oy, ox)
// order like the general kernel below, so the sums are bit-identical; no per-tap divisibility tests.
template <bool I32>
__global__ void __launch_bounds__(256) maxpool_bwd_d1_kernel(const float* __restrict__ g,
                                                             const int64_t* __restrict__ idx, float* __restrict__ gx,
                                                             int64_t total, PoolGeo q) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const Pos in = decompose<I32>(i, q.iw, q.ih * q.iw, q.d_iw, q.d_ihw);
    const int ty = in.y + q.ph, tx = in.x + q.pw;
    const int ay = ty - q.kh + 1, ax = tx - q.kw + 1;
    const int oy0 = ay <= 0 ? 0 : (int)fdiv((uint32_t)(ay + q.sh - 1), q.d_sh);
    const int ox0 = ax <= 0 ? 0 : (int)fdiv((uint32_t)(ax + q.sw - 1), q.d_sw);
    const int oy1 = min((int)fdiv((uint32_t)ty, q.d_sh), q.oh - 1);
    const int ox1 = min((int)fdiv((uint32_t)tx, q.d_sw), q.ow - 1);
    const float* gp = g + in.plane * q.oh * q.ow;
    const int64_t* ip = idx + in.plane * q.oh * q.ow;
    const int64_t me = (int64_t)in.y * q.iw + in.x;
    float acc = 0.f;
    for (int oy = oy0; oy <= oy1; ++oy)
      for (int ox = ox0; ox <= ox1; ++ox) {
        const int o = oy * q.ow + ox;
        const float gv = gp[o];  // loaded with the index, not after the compare
        if (ip[o] == me) acc += gv;
      }
    gx[i] = acc;
  }
}

// Undilated windows, four consecutive inputs of a row per thread (iw % 4 == 0, float4 store): the outputs whose
// windows cover any of the four form an NY x NX block (NY, NX at least the largest such block of the geometry, checked
// on the host); all of its gradients and indices are loaded first, then each input sums, in ascending (oy, ox) order,
// the gradients of the block's outputs whose index names it. An output whose index names an input covers that input,
// so each sum visits the same outputs in the same order as the per-input kernel above: the results are identical.
template <int NY, int NX>
__global__ void __launch_bounds__(256) maxpool_bwd_v4_kernel(const float* __restrict__ g,
                                                             const int64_t* __restrict__ idx, float* __restrict__ gx,
                                                             uint32_t total4, PoolGeo q, FastDiv d_iw4, FastDiv d_ih) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total4; i += gridDim.x * blockDim.x) {
    const uint32_t row = fdiv(i, d_iw4), x = (i - row * (uint32_t)(q.iw >> 2)) * 4u;
    const uint32_t plane = fdiv(row, d_ih), yy = row - plane * (uint32_t)q.ih;
    const int ty = (int)yy + q.ph, ay = ty - q.kh + 1;
    const int oy0 = ay <= 0 ? 0 : (int)fdiv((uint32_t)(ay + q.sh - 1), q.d_sh);
    const int oy1 = min((int)fdiv((uint32_t)ty, q.d_sh), q.oh - 1);
    const int ax = (int)x + q.pw - q.kw + 1, tx = (int)x + 3 + q.pw;
    const int ox0 = ax <= 0 ? 0 : (int)fdiv((uint32_t)(ax + q.sw - 1), q.d_sw);
    const int ox1 = min((int)fdiv((uint32_t)tx, q.d_sw), q.ow - 1);
    const int64_t obase = (int64_t)plane * q.oh * q.ow;
    float gv[NY][NX];
    int64_t iv[NY][NX];
#pragma unroll
    for (int jy = 0; jy < NY; ++jy)
#pragma unroll
      for (int jx = 0; jx < NX; ++jx) {
        const bool ok = oy0 + jy <= oy1 && ox0 + jx <= ox1;
        const int64_t o = obase + (int64_t)(oy0 + jy) * q.ow + ox0 + jx;
        gv[jy][jx] = ok ? g[o] : 0.f;
        iv[jy][jx] = ok ? idx[o] : -1;
      }
    const int64_t me = (int64_t)yy * q.iw + x;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int jy = 0; jy < NY; ++jy)
#pragma unroll
      for (int jx = 0; jx < NX; ++jx)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (iv[jy][jx] == me + e) acc[e] += gv[jy][jx];
    *reinterpret_cast<float4*>(gx + (int64_t)row * q.iw + x) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  }
}

// Stride-2 square windows whose covering outputs of every 8 inputs start at a multiple of 4 (K 3 pad 1: five
// outputs from x / 2 across, up to two rows; K 2 pad 0: four across, one row; iw % 8 == 0, ow % 4 == 0, g, idx and gx
// below 2 GiB and 16-byte aligned): eight consecutive inputs of a row per thread. Each covering output row's
// gradients and indices are loaded as aligned runs (float4 + float, two int64 pairs + int64; runs past the row or
// the plane read 0 and are masked out), then each input sums, in ascending (oy, ox) order, the gradients of the
// outputs whose index names it: the same outputs in the same order as the per-input kernel, so identical results.
template <int K, int P>
__global__ void __launch_bounds__(256) maxpool_bwd_s2x8_kernel(const float* __restrict__ g,
                                                               const int64_t* __restrict__ idx,
                                                               float* __restrict__ gx, uint32_t total8, PoolGeo q,
                                                               FastDiv d_iw8, FastDiv d_ih, uint32_t gbytes) {
  constexpr int NX = K == 3 ? 5 : 4, NY = K == 3 ? 2 : 1;
  static_assert((K == 3 && P == 1) || (K == 2 && P == 0), "stride-2 windows 3 x 3 pad 1 or 2 x 2 pad 0");
  const __amdgpu_buffer_rsrc_t gr = make_rsrc(g, gbytes), ir = make_rsrc(idx, gbytes * 2u);
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total8; i += gridDim.x * blockDim.x) {
    const uint32_t row = fdiv(i, d_iw8), x = (i - row * (uint32_t)(q.iw >> 3)) * 8u;
    const uint32_t plane = fdiv(row, d_ih), yy = row - plane * (uint32_t)q.ih;
    const int ty = (int)yy + P, ay = ty - K + 1;
    const int oy0 = ay <= 0 ? 0 : (ay + 1) >> 1, oy1 = min(ty >> 1, q.oh - 1);
    const int ox0 = (int)(x >> 1), nx = min(NX, q.ow - ox0);
    float gv[NY][NX];
    long long iv[NY][NX];
#pragma unroll
    for (int jy = 0; jy < NY; ++jy) {
      const bool rok = oy0 + jy <= oy1;
      const uint32_t o = (plane * (uint32_t)q.oh + (uint32_t)(oy0 + jy)) * (uint32_t)q.ow + (uint32_t)ox0;
      const float4 g4 = bload4(gr, rok ? o * 4u : kOOB, 0);
      const omt_i64x2 i01 = __builtin_bit_cast(omt_i64x2, __builtin_amdgcn_raw_buffer_load_b128(ir, (int)(rok ? o * 8u : kOOB), 0, 0));
      const omt_i64x2 i23 =
          __builtin_bit_cast(omt_i64x2, __builtin_amdgcn_raw_buffer_load_b128(ir, (int)(rok ? o * 8u + 16u : kOOB), 0, 0));
      gv[jy][0] = g4.x;
      gv[jy][1] = g4.y;
      gv[jy][2] = g4.z;
      gv[jy][3] = g4.w;
      iv[jy][0] = i01.x;
      iv[jy][1] = i01.y;
      iv[jy][2] = i23.x;
      iv[jy][3] = i23.y;
      if constexpr (NX == 5) {
        const bool ok4 = rok && nx == 5;
        gv[jy][4] = bload(gr, ok4 ? o * 4u + 16u : kOOB, 0);
        iv[jy][4] = __builtin_bit_cast(long long, __builtin_amdgcn_raw_buffer_load_b64(ir, (int)(ok4 ? o * 8u + 32u : kOOB), 0, 0));
      }
#pragma unroll
      for (int jx = 0; jx < NX; ++jx)
        if (!rok || jx >= nx) iv[jy][jx] = -1;
    }
    const long long me = (long long)yy * q.iw + x;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
    for (int jy = 0; jy < NY; ++jy)
#pragma unroll
      for (int jx = 0; jx < NX; ++jx)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (iv[jy][jx] == me + e) acc[e] += gv[jy][jx];
    float4* out = reinterpret_cast<float4*>(gx + (size_t)row * q.iw + x);
    out[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    out[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

// Output rows oy whose window row ky lands on input row r: oy * s - p + ky * d = r. Visits oy ascending.
template <bool I32>
__global__ void __launch_bounds__(256) maxpool_bwd_kernel(const float* __restrict__ g, const int64_t* __restrict__ idx,
                                                          float* __restrict__ gx, int64_t total, PoolGeo q) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const Pos in = decompose<I32>(i, q.iw, q.ih * q.iw, q.d_iw, q.d_ihw);
    const int xx = in.x, yy = in.y;
    const int64_t plane = in.plane;
    const float* gp = g + plane * q.oh * q.ow;
    const int64_t* ip = idx + plane * q.oh * q.ow;
    const int64_t me = (int64_t)yy * q.iw + xx;
    float acc = 0.f;
    for (int ky = q.kh - 1; ky >= 0; --ky) {
      const int ty = yy + q.ph - ky * q.dh;
      if (ty < 0) continue;
      const int oy = exact_div(ty, q.sh, q.d_sh);
      if (oy < 0 || oy >= q.oh) continue;
      for (int kx = q.kw - 1; kx >= 0; --kx) {
        const int tx = xx + q.pw - kx * q.dw;
        if (tx < 0) continue;
        const int ox = exact_div(tx, q.sw, q.d_sw);
        if (ox < 0 || ox >= q.ow) continue;
        const int o = oy * q.ow + ox;
        if (ip[o] == me) acc += gp[o];
      }
    }
    gx[i] = acc;
  }
}

__device__ __forceinline__ float avg_divisor(int oy, int ox, const PoolGeo& g, int include_pad, int divisor) {
  if (divisor > 0) return (float)divisor;
  int hs = oy * g.sh - g.ph, ws = ox * g.sw - g.pw;
  int he = min(hs + g.kh, g.ih + g.ph), we = min(ws + g.kw, g.iw + g.pw);
  const int pool = (he - hs) * (we - ws);
  if (include_pad) return (float)pool;
  hs = max(hs, 0);
  ws = max(ws, 0);
  he = min(he, g.ih);
  we = min(we, g.iw);
  return (float)((he - hs) * (we - ws));
}

template <bool I32>
__global__ void __launch_bounds__(256) avgpool_fwd_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                          int64_t total, PoolGeo g, int include_pad, int divisor) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const Pos o = decompose<I32>(i, g.ow, g.oh * g.ow, g.d_ow, g.d_ohw);
    const int ox = o.x, oy = o.y;
    const int64_t plane = o.plane;
    const float* xp = x + plane * g.ih * g.iw;
    const int hs = oy * g.sh - g.ph, ws = ox * g.sw - g.pw;
    const int y0 = max(hs, 0), y1 = min(hs + g.kh, g.ih), x0 = max(ws, 0), x1 = min(ws + g.kw, g.iw);
    float acc = 0.f;
    for (int yy = y0; yy < y1; ++yy)
      for (int xx = x0; xx < x1; ++xx) acc += xp[yy * g.iw + xx];
    y[i] = acc / avg_divisor(oy, ox, g, include_pad, divisor);
  }
}

template <bool I32>
__global__ void __launch_bounds__(256) avgpool_bwd_kernel(const float* __restrict__ gy, float* __restrict__ gx,
                                                          int64_t total, PoolGeo q, int include_pad, int divisor) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const Pos in = decompose<I32>(i, q.iw, q.ih * q.iw, q.d_iw, q.d_ihw);
    const int xx = in.x, yy = in.y;
    const int64_t plane = in.plane;
    const float* gp = gy + plane * q.oh * q.ow;
    // windows [oy*s - p, oy*s - p + k) containing yy: oy in [ceil((yy + p - k + 1) / s), floor((yy + p) / s)]
    const int oy0 = max(0, (yy + q.ph - q.kh + q.sh) / q.sh), oy1 = min(q.oh - 1, (yy + q.ph) / q.sh);
    const int ox0 = max(0, (xx + q.pw - q.kw + q.sw) / q.sw), ox1 = min(q.ow - 1, (xx + q.pw) / q.sw);
    float acc = 0.f;
    for (int oy = oy0; oy <= oy1; ++oy) {
      const int hs = oy * q.sh - q.ph;
      if (yy < hs || yy >= hs + q.kh) continue;
      for (int ox = ox0; ox <= ox1; ++ox) {
        const int ws = ox * q.sw - q.pw;
        if (xx < ws || xx >= ws + q.kw) continue;
        acc += gp[oy * q.ow + ox] / avg_divisor(oy, ox, q, include_pad, divisor);
      }
    }
    gx[i] = acc;
  }
}

__device__ __forceinline__ int bin_lo(int o, int in, int out) { return (int)(((int64_t)o * in) / out); }
__device__ __forceinline__ int bin_hi(int o, int in, int out) { return (int)(((int64_t)(o + 1) * in + out - 1) / out); }

__global__ void __launch_bounds__(256) adapool_fwd_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                          int64_t total, int ih, int iw, int oh, int ow) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int ox = (int)(i % ow), oy = (int)((i / ow) % oh);
    const int64_t plane = i / ((int64_t)ow * oh);
    const float* xp = x + plane * ih * iw;
    const int y0 = bin_lo(oy, ih, oh), y1 = bin_hi(oy, ih, oh), x0 = bin_lo(ox, iw, ow), x1 = bin_hi(ox, iw, ow);
    float acc = 0.f;
    for (int yy = y0; yy < y1; ++yy)
      for (int xx = x0; xx < x1; ++xx) acc += xp[yy * iw + xx];
    y[i] = acc / (float)((y1 - y0) * (x1 - x0));
  }
}

// Global average pool of planes of at most 64 elements: a workgroup stages 256 consecutive planes (one contiguous
// segment) through LDS with float4 loads, then each thread sums one plane. hw odd keeps the per-thread LDS rows on
// distinct banks; an even hw costs some bank conflicts, not correctness.
__global__ void __launch_bounds__(256) gap_small_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                        int64_t planes, int hw) {
  __shared__ float tile[256 * 64];
  const int64_t p0 = (int64_t)blockIdx.x * 256;
  const int np = (int)min<int64_t>(256, planes - p0);
  const int n = np * hw;
  const float* src = x + p0 * hw;
  if ((((uintptr_t)src) & 15) == 0) {
    const int n4 = n >> 2;
    for (int e = threadIdx.x; e < n4; e += 256) reinterpret_cast<float4*>(tile)[e] = reinterpret_cast<const float4*>(src)[e];
    for (int e = (n4 << 2) + threadIdx.x; e < n; e += 256) tile[e] = src[e];
  } else {
    for (int e = threadIdx.x; e < n; e += 256) tile[e] = src[e];
  }
  __syncthreads();
  if ((int)threadIdx.x < np) {
    float acc = 0.f;
    for (int e = 0; e < hw; ++e) acc += tile[threadIdx.x * hw + e];
    y[p0 + threadIdx.x] = acc / (float)hw;
  }
}

// Global average pool of larger planes as one wave per plane: coalesced reads and a wave reduction.
__global__ void __launch_bounds__(256) gap_fwd_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                      int64_t planes, int hw) {
  const int64_t plane = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (plane >= planes) return;
  const int lane = threadIdx.x & 63;
  const float* xp = x + plane * hw;
  float acc = 0.f;
  for (int e = lane; e < hw; e += 64) acc += xp[e];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (lane == 0) y[plane] = acc / (float)hw;
}

// Grad of global average pooling: gx[plane][e] = g[plane] / hw.
template <bool I32>
__global__ void __launch_bounds__(256) gap_bwd_kernel(const float* __restrict__ g, float* __restrict__ gx,
                                                      int64_t total, int hw, FastDiv d_hw) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t plane = I32 ? (int64_t)fdiv((uint32_t)i, d_hw) : i / hw;
    gx[i] = g[plane] / (float)hw;
  }
}

__global__ void __launch_bounds__(256) adapool_bwd_kernel(const float* __restrict__ gy, float* __restrict__ gx,
                                                          int64_t total, int ih, int iw, int oh, int ow) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int xx = (int)(i % iw), yy = (int)((i / iw) % ih);
    const int64_t plane = i / ((int64_t)iw * ih);
    const float* gp = gy + plane * oh * ow;
    float acc = 0.f;
    for (int oy = 0; oy < oh; ++oy) {
      const int y0 = bin_lo(oy, ih, oh), y1 = bin_hi(oy, ih, oh);
      if (yy < y0 || yy >= y1) continue;
      for (int ox = 0; ox < ow; ++ox) {
        const int x0 = bin_lo(ox, iw, ow), x1 = bin_hi(ox, iw, ow);
        if (xx < x0 || xx >= x1) continue;
        acc += gp[oy * ow + ox] / (float)((y1 - y0) * (x1 - x0));
      }
    }
    gx[i] = acc;
  }
}

static bool pool_ok(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow) {
  const int64_t lim = (int64_t)1 << 31;
  return planes >= 0 && ih >= 1 && iw >= 1 && oh >= 1 && ow >= 1 && ih * iw < lim && oh * ow < lim &&
         planes * ih * iw < ((int64_t)1 << 46);
}

static PoolGeo pgeo(int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh, int64_t kw, int64_t sh, int64_t sw,
                    int64_t ph, int64_t pw, int64_t dh, int64_t dw) {
  PoolGeo g{(int)ih, (int)iw, (int)oh, (int)ow, (int)kh, (int)kw, (int)sh, (int)sw, (int)ph, (int)pw, (int)dh, (int)dw};
  g.d_ow = make_fastdiv((uint32_t)ow);
  g.d_ohw = make_fastdiv((uint32_t)(oh * ow));
  g.d_iw = make_fastdiv((uint32_t)iw);
  g.d_ihw = make_fastdiv((uint32_t)(ih * iw));
  g.d_sh = make_fastdiv((uint32_t)sh);
  g.d_sw = make_fastdiv((uint32_t)sw);
  return g;
}

static bool idx32(int64_t total) { return total < ((int64_t)1 << 32); }

// Launches K<true> (32-bit indexing) or K<false> over a 1-D grid for `total` elements.
#define OMT_POOL_LAUNCH(K, total, s, ...)                                                      \
  do {                                                                                         \
    if (idx32(total))                                                                          \
      hipLaunchKernelGGL(K<true>, dim3(grid1d(total, 256)), dim3(256), 0, s, __VA_ARGS__);    \
    else                                                                                       \
      hipLaunchKernelGGL(K<false>, dim3(grid1d(total, 256)), dim3(256), 0, s, __VA_ARGS__);   \
  } while (0)
#define OMT_POOL_LAUNCH_K(K, W, total, s, ...)                                                    \
  do {                                                                                           \
    if (idx32(total))                                                                            \
      hipLaunchKernelGGL((K<true, W>), dim3(grid1d(total, 256)), dim3(256), 0, s, __VA_ARGS__);  \
    else                                                                                         \
      hipLaunchKernelGGL((K<false, W>), dim3(grid1d(total, 256)), dim3(256), 0, s, __VA_ARGS__); \
  } while (0)

// Largest number of outputs whose undilated windows (extent k, stride s, padding p, n outputs) cover any of `span`
// consecutive inputs starting at a multiple of `span` (span 1: any single input), over all such runs of a length-`len`
// axis.
static int max_cover(int64_t len, int64_t n, int64_t k, int64_t s, int64_t p, int64_t span) {
  int64_t best = 0;
  for (int64_t a = 0; a < len; a += span) {
    const int64_t lo_t = a + p - k + 1, hi_t = std::min(a + span - 1, len - 1) + p;
    const int64_t lo = lo_t <= 0 ? 0 : (lo_t + s - 1) / s, hi = std::min(hi_t / s, n - 1);
    best = std::max(best, hi - lo + 1);
  }
  return (int)best;
}


// ---- channels-last (NHWC) pools ---------------------------------------------------------------------------------
// x [n][ih][iw][c], outputs [n][oh][ow][c] (indices int64 in the same order); one thread per (pixel, vector of VEC
// channels: float4 when c % 4 == 0 and the operands are 16-byte aligned), so a wave reads whole runs of channels. The
// windows, the visiting orders and the max / NaN / tie rules are the NCHW kernels' above, so values, indices (flat
// in-plane y * iw + x, as PyTorch's channels-last max pool returns them) and sums are the NCHW results transposed,
// bit for bit.
template <int VEC>
struct PoolVec;
template <>
struct PoolVec<4> {
  using T = float4;
  static __device__ __forceinline__ float get(const float4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
  }
  static __device__ __forceinline__ void set(float4& v, int i, float f) {
    if (i == 0) v.x = f; else if (i == 1) v.y = f; else if (i == 2) v.z = f; else v.w = f;
  }
};
template <>
struct PoolVec<1> {
  using T = float;
  static __device__ __forceinline__ float get(const float& v, int) { return v; }
  static __device__ __forceinline__ void set(float& v, int, float f) { v = f; }
};

struct NhwcPool {
  int c, cv;              // channels, channel vectors per pixel
  FastDiv d_cv, d_w, d_h;  // by cv, and the width and height of the plane a thread's pixel lies in
};

// (image, row, column, channel vector) of thread index i over planes of W x H pixels
__device__ __forceinline__ void nhwc_pos(uint32_t i, const NhwcPool& p, int W, int H, int64_t& img, int& y, int& x,
                                         int& j) {
  const uint32_t pix = fdiv(i, p.d_cv), t = fdiv(pix, p.d_w), im = fdiv(t, p.d_h);
  j = (int)(i - pix * (uint32_t)p.cv);
  x = (int)(pix - t * (uint32_t)W);
  y = (int)(t - im * (uint32_t)H);
  img = im;
}

template <int VEC>
__global__ void __launch_bounds__(256) maxpool_fwd_nhwc_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                               int64_t* __restrict__ idx, uint32_t total, PoolGeo g,
                                                               NhwcPool p) {
  using PV = PoolVec<VEC>;
  using V = typename PV::T;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
    int64_t img;
    int oy, ox, j;
    nhwc_pos(i, p, g.ow, g.oh, img, oy, ox, j);
    float best[VEC];
    int bi[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) best[e] = -INFINITY, bi[e] = -1;
    for (int ky = 0; ky < g.kh; ++ky) {
      const int yy = oy * g.sh - g.ph + ky * g.dh;
      if (yy < 0 || yy >= g.ih) continue;
      for (int kx = 0; kx < g.kw; ++kx) {
        const int xx = ox * g.sw - g.pw + kx * g.dw;
        if (xx < 0 || xx >= g.iw) continue;
        const V v = *reinterpret_cast<const V*>(x + ((img * g.ih + yy) * g.iw + xx) * p.c + (int64_t)j * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float f = PV::get(v, e);
          if (bi[e] < 0 || f > best[e] || isnan(f)) {  // first max wins ties; a NaN replaces the running max
            best[e] = f;
            bi[e] = yy * g.iw + xx;
          }
        }
      }
    }
    const int64_t o = ((img * g.oh + oy) * g.ow + ox) * p.c + (int64_t)j * VEC;
    V out;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      PV::set(out, e, best[e]);
      idx[o + e] = bi[e];
    }
    *reinterpret_cast<V*>(y + o) = out;
  }
}

// Gather form of maxpool_bwd_kernel: the outputs whose window holds input (iy, ix), visited oy, ox ascending.
template <int VEC>
__global__ void __launch_bounds__(256) maxpool_bwd_nhwc_kernel(const float* __restrict__ g,
                                                               const int64_t* __restrict__ idx,
                                                               float* __restrict__ gx, uint32_t total, PoolGeo q,
                                                               NhwcPool p) {
  using PV = PoolVec<VEC>;
  using V = typename PV::T;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
    int64_t img;
    int yy, xx, j;
    nhwc_pos(i, p, q.iw, q.ih, img, yy, xx, j);
    const int64_t me = (int64_t)yy * q.iw + xx;
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    for (int ky = q.kh - 1; ky >= 0; --ky) {
      const int ty = yy + q.ph - ky * q.dh;
      if (ty < 0) continue;
      const int oy = exact_div(ty, q.sh, q.d_sh);
      if (oy < 0 || oy >= q.oh) continue;
      for (int kx = q.kw - 1; kx >= 0; --kx) {
        const int tx = xx + q.pw - kx * q.dw;
        if (tx < 0) continue;
        const int ox = exact_div(tx, q.sw, q.d_sw);
        if (ox < 0 || ox >= q.ow) continue;
        const int64_t o = ((img * q.oh + oy) * q.ow + ox) * p.c + (int64_t)j * VEC;
        const V gv = *reinterpret_cast<const V*>(g + o);
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          if (idx[o + e] == me) acc[e] += PV::get(gv, e);
      }
    }
    V out;
#pragma unroll
    for (int e = 0; e < VEC; ++e) PV::set(out, e, acc[e]);
    *reinterpret_cast<V*>(gx + ((img * q.ih + yy) * q.iw + xx) * p.c + (int64_t)j * VEC) = out;
  }
}

template <int VEC>
__global__ void __launch_bounds__(256) avgpool_fwd_nhwc_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                               uint32_t total, PoolGeo g, NhwcPool p,
                                                               int include_pad, int divisor) {
  using PV = PoolVec<VEC>;
  using V = typename PV::T;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
    int64_t img;
    int oy, ox, j;
    nhwc_pos(i, p, g.ow, g.oh, img, oy, ox, j);
    const int hs = oy * g.sh - g.ph, ws = ox * g.sw - g.pw;
    const int y0 = max(hs, 0), y1 = min(hs + g.kh, g.ih), x0 = max(ws, 0), x1 = min(ws + g.kw, g.iw);
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    for (int yy = y0; yy < y1; ++yy)
      for (int xx = x0; xx < x1; ++xx) {
        const V v = *reinterpret_cast<const V*>(x + ((img * g.ih + yy) * g.iw + xx) * p.c + (int64_t)j * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += PV::get(v, e);
      }
    const float d = avg_divisor(oy, ox, g, include_pad, divisor);
    V out;
#pragma unroll
    for (int e = 0; e < VEC; ++e) PV::set(out, e, acc[e] / d);
    *reinterpret_cast<V*>(y + ((img * g.oh + oy) * g.ow + ox) * p.c + (int64_t)j * VEC) = out;
  }
}

template <int VEC>
__global__ void __launch_bounds__(256) avgpool_bwd_nhwc_kernel(const float* __restrict__ gy, float* __restrict__ gx,
                                                               uint32_t total, PoolGeo q, NhwcPool p,
                                                               int include_pad, int divisor) {
  using PV = PoolVec<VEC>;
  using V = typename PV::T;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
    int64_t img;
    int yy, xx, j;
    nhwc_pos(i, p, q.iw, q.ih, img, yy, xx, j);
    const int oy0 = max(0, (yy + q.ph - q.kh + q.sh) / q.sh), oy1 = min(q.oh - 1, (yy + q.ph) / q.sh);
    const int ox0 = max(0, (xx + q.pw - q.kw + q.sw) / q.sw), ox1 = min(q.ow - 1, (xx + q.pw) / q.sw);
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    for (int oy = oy0; oy <= oy1; ++oy) {
      const int hs = oy * q.sh - q.ph;
      if (yy < hs || yy >= hs + q.kh) continue;
      for (int ox = ox0; ox <= ox1; ++ox) {
        const int ws = ox * q.sw - q.pw;
        if (xx < ws || xx >= ws + q.kw) continue;
        const float d = avg_divisor(oy, ox, q, include_pad, divisor);
        const V v = *reinterpret_cast<const V*>(gy + ((img * q.oh + oy) * q.ow + ox) * p.c + (int64_t)j * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += PV::get(v, e) / d;
      }
    }
    V out;
#pragma unroll
    for (int e = 0; e < VEC; ++e) PV::set(out, e, acc[e]);
    *reinterpret_cast<V*>(gx + ((img * q.ih + yy) * q.iw + xx) * p.c + (int64_t)j * VEC) = out;
  }
}

template <int VEC>
__global__ void __launch_bounds__(256) adapool_fwd_nhwc_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                               uint32_t total, int ih, int iw, int oh, int ow,
                                                               NhwcPool p) {
  using PV = PoolVec<VEC>;
  using V = typename PV::T;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
    int64_t img;
    int oy, ox, j;
    nhwc_pos(i, p, ow, oh, img, oy, ox, j);
    const int y0 = bin_lo(oy, ih, oh), y1 = bin_hi(oy, ih, oh), x0 = bin_lo(ox, iw, ow), x1 = bin_hi(ox, iw, ow);
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    for (int yy = y0; yy < y1; ++yy)
      for (int xx = x0; xx < x1; ++xx) {
        const V v = *reinterpret_cast<const V*>(x + ((img * ih + yy) * iw + xx) * p.c + (int64_t)j * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += PV::get(v, e);
      }
    const float d = (float)((y1 - y0) * (x1 - x0));
    V out;
#pragma unroll
    for (int e = 0; e < VEC; ++e) PV::set(out, e, acc[e] / d);
    *reinterpret_cast<V*>(y + ((img * oh + oy) * ow + ox) * p.c + (int64_t)j * VEC) = out;
  }
}

template <int VEC>
__global__ void __launch_bounds__(256) adapool_bwd_nhwc_kernel(const float* __restrict__ gy, float* __restrict__ gx,
                                                               uint32_t total, int ih, int iw, int oh, int ow,
                                                               NhwcPool p) {
  using PV = PoolVec<VEC>;
  using V = typename PV::T;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
    int64_t img;
    int yy, xx, j;
    nhwc_pos(i, p, iw, ih, img, yy, xx, j);
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    for (int oy = 0; oy < oh; ++oy) {
      const int y0 = bin_lo(oy, ih, oh), y1 = bin_hi(oy, ih, oh);
      if (yy < y0 || yy >= y1) continue;
      for (int ox = 0; ox < ow; ++ox) {
        const int x0 = bin_lo(ox, iw, ow), x1 = bin_hi(ox, iw, ow);
        if (xx < x0 || xx >= x1) continue;
        const float d = (float)((y1 - y0) * (x1 - x0));
        const V v = *reinterpret_cast<const V*>(gy + ((img * oh + oy) * ow + ox) * p.c + (int64_t)j * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += PV::get(v, e) / d;
      }
    }
    V out;
#pragma unroll
    for (int e = 0; e < VEC; ++e) PV::set(out, e, acc[e]);
    *reinterpret_cast<V*>(gx + ((img * ih + yy) * iw + xx) * p.c + (int64_t)j * VEC) = out;
  }
}

// VEC 4 when c % 4 == 0 and every pointer is 16-byte aligned; the plane (W x H) the threads decompose
static NhwcPool nhwc_pool(int64_t c, bool aligned, int64_t W, int64_t H) {
  NhwcPool p;
  p.c = (int)c;
  p.cv = (int)((c % 4 == 0 && aligned) ? c / 4 : c);
  p.d_cv = make_fastdiv((uint32_t)p.cv);
  p.d_w = make_fastdiv((uint32_t)W);
  p.d_h = make_fastdiv((uint32_t)H);
  return p;
}
static bool a16(const void* p) { return p == nullptr || (uintptr_t)p % 16 == 0; }
// thread counts (pixels x channel vectors) below 2^31, so a grid-stride step (at most 2^28) never wraps 32 bits
static bool nhwc_pool_ok(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow) {
  return n >= 0 && c >= 1 && c < ((int64_t)1 << 24) && pool_ok(n * c, ih, iw, oh, ow) &&
         n * ih * iw * c < ((int64_t)1 << 31) && n * oh * ow * c < ((int64_t)1 << 31);
}

#define OMT_NHWC_LAUNCH(K, total, s, vec, ...)                                                               \
  do {                                                                                                       \
    if (vec)                                                                                                 \
      hipLaunchKernelGGL(K<4>, dim3(grid1d(total, 256)), dim3(256), 0, s, __VA_ARGS__);                      \
    else                                                                                                     \
      hipLaunchKernelGGL(K<1>, dim3(grid1d(total, 256)), dim3(256), 0, s, __VA_ARGS__);                      \
  } while (0)

}  // namespace omt

using namespace omt;

OMT_EXPORT int omt_maxpool_fwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh,
                               int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                               const float* x, float* y, int64_t* idx, void* stream) {
  if (!x || !y || !idx) return fail(OMT_INVALID, "omt_maxpool_fwd: null pointer");
  if (!pool_ok(planes, ih, iw, oh, ow) || kh < 1 || kw < 1 || sh < 1 || sw < 1 || dh < 1 || dw < 1 || ph < 0 || pw < 0)
    return fail(OMT_UNSUPPORTED, "omt_maxpool_fwd: geometry not covered");
  const int64_t total = planes * oh * ow;
  if (total == 0) return OMT_OK;
  const PoolGeo q = pgeo(ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, dh, dw);
  const int off = (int)((4 - pw % 4) % 4);
  if (kh == kw && sh == sw && dh == 1 && dw == 1 && ow % 4 == 0 && iw % 4 == 0 && planes * ih * iw * 4 < ((int64_t)1 << 31) &&
      (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0 && (uintptr_t)idx % 16 == 0 &&
      ((kh == 2 && sh == 2 && off == 0) || (kh == 3 && sh == 2 && (off == 0 || off == 3)))) {
    const uint32_t total4 = (uint32_t)(total / 4), xbytes = (uint32_t)(planes * ih * iw * 4);
    const FastDiv d_ow4 = make_fastdiv((uint32_t)(ow / 4)), d_oh = make_fastdiv((uint32_t)oh);
#define OMT_MP_F4(K_, S_, OFF_)                                                                                    \
  hipLaunchKernelGGL((maxpool_fwd_v4_kernel<K_, S_, OFF_>), dim3(grid1d(total4, 256)), dim3(256), 0, stream_of(stream), \
                     x, y, idx, total4, q, xbytes, d_ow4, d_oh)
    if (kh == 2) OMT_MP_F4(2, 2, 0);
    else if (off == 0) OMT_MP_F4(3, 2, 0);
    else OMT_MP_F4(3, 2, 3);
#undef OMT_MP_F4
    return launch_check("maxpool_fwd_v4_kernel");
  }
  if (kh == kw && dh == 1 && dw == 1 && (kh == 2 || kh == 3)) {
    if (kh == 2)
      OMT_POOL_LAUNCH_K(maxpool_fwd_k_kernel, 2, total, stream_of(stream), x, y, idx, total, q);
    else
      OMT_POOL_LAUNCH_K(maxpool_fwd_k_kernel, 3, total, stream_of(stream), x, y, idx, total, q);
    return launch_check("maxpool_fwd_k_kernel");
  }
  OMT_POOL_LAUNCH(maxpool_fwd_kernel, total, stream_of(stream), x, y, idx, total, q);
  return launch_check("maxpool_fwd_kernel");
}

OMT_EXPORT int omt_maxpool_bwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh,
                               int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                               const float* g, const int64_t* idx, float* gx, void* stream) {
  if (!g || !idx || !gx) return fail(OMT_INVALID, "omt_maxpool_bwd: null pointer");
  if (!pool_ok(planes, ih, iw, oh, ow) || kh < 1 || kw < 1 || sh < 1 || sw < 1 || dh < 1 || dw < 1 || ph < 0 || pw < 0)
    return fail(OMT_UNSUPPORTED, "omt_maxpool_bwd: geometry not covered");
  const int64_t total = planes * ih * iw;
  if (total == 0) return OMT_OK;
  if (dh == 1 && dw == 1) {
    const PoolGeo q = pgeo(ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, dh, dw);
    const int64_t gbytes = planes * oh * ow * 4;
    if (sh == 2 && sw == 2 && kh == kw && ((kh == 3 && ph == 1 && pw == 1) || (kh == 2 && ph == 0 && pw == 0)) &&
        iw % 8 == 0 && ow % 4 == 0 && 2 * gbytes < ((int64_t)1 << 31) && total * 4 < ((int64_t)1 << 31) &&
        (uintptr_t)gx % 16 == 0 && (uintptr_t)g % 16 == 0 && (uintptr_t)idx % 16 == 0) {
      const uint32_t total8 = (uint32_t)(total / 8);
      const FastDiv d_iw8 = make_fastdiv((uint32_t)(iw / 8)), d_ih = make_fastdiv((uint32_t)ih);
      if (kh == 3)
        hipLaunchKernelGGL((maxpool_bwd_s2x8_kernel<3, 1>), dim3(grid1d(total8, 256)), dim3(256), 0, stream_of(stream),
                           g, idx, gx, total8, q, d_iw8, d_ih, (uint32_t)gbytes);
      else
        hipLaunchKernelGGL((maxpool_bwd_s2x8_kernel<2, 0>), dim3(grid1d(total8, 256)), dim3(256), 0, stream_of(stream),
                           g, idx, gx, total8, q, d_iw8, d_ih, (uint32_t)gbytes);
      return launch_check("maxpool_bwd_s2x8_kernel");
    }
    if (iw % 4 == 0 && total < ((int64_t)1 << 32) && (uintptr_t)gx % 16 == 0) {
      const int ny = max_cover(ih, oh, kh, sh, ph, 1), nx = max_cover(iw, ow, kw, sw, pw, 4);
      const uint32_t total4 = (uint32_t)(total / 4);
      const FastDiv d_iw4 = make_fastdiv((uint32_t)(iw / 4)), d_ih = make_fastdiv((uint32_t)ih);
#define OMT_MP_V4(NY_, NX_)                                                                                  \
  hipLaunchKernelGGL((maxpool_bwd_v4_kernel<NY_, NX_>), dim3(grid1d(total4, 256)), dim3(256), 0, stream_of(stream), \
                     g, idx, gx, total4, q, d_iw4, d_ih)
      bool launched = true;
      if (ny <= 1 && nx <= 2) OMT_MP_V4(1, 2);
      else if (ny <= 2 && nx <= 3) OMT_MP_V4(2, 3);
      else launched = false;
#undef OMT_MP_V4
      if (launched) return launch_check("maxpool_bwd_v4_kernel");
    }
    OMT_POOL_LAUNCH(maxpool_bwd_d1_kernel, total, stream_of(stream), g, idx, gx, total, q);
    return launch_check("maxpool_bwd_d1_kernel");
  }
  OMT_POOL_LAUNCH(maxpool_bwd_kernel, total, stream_of(stream), g, idx, gx, total,
                  pgeo(ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, dh, dw));
  return launch_check("maxpool_bwd_kernel");
}

OMT_EXPORT int omt_avgpool_fwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh,
                               int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int count_include_pad,
                               int64_t divisor_override, const float* x, float* y, void* stream) {
  if (!x || !y) return fail(OMT_INVALID, "omt_avgpool_fwd: null pointer");
  if (!pool_ok(planes, ih, iw, oh, ow) || kh < 1 || kw < 1 || sh < 1 || sw < 1 || ph < 0 || pw < 0)
    return fail(OMT_UNSUPPORTED, "omt_avgpool_fwd: geometry not covered");
  const int64_t total = planes * oh * ow;
  if (total == 0) return OMT_OK;
  OMT_POOL_LAUNCH(avgpool_fwd_kernel, total, stream_of(stream), x, y, total,
                  pgeo(ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, 1, 1), count_include_pad, (int)divisor_override);
  return launch_check("avgpool_fwd_kernel");
}

OMT_EXPORT int omt_avgpool_bwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh,
                               int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int count_include_pad,
                               int64_t divisor_override, const float* g, float* gx, void* stream) {
  if (!g || !gx) return fail(OMT_INVALID, "omt_avgpool_bwd: null pointer");
  if (!pool_ok(planes, ih, iw, oh, ow) || kh < 1 || kw < 1 || sh < 1 || sw < 1 || ph < 0 || pw < 0)
    return fail(OMT_UNSUPPORTED, "omt_avgpool_bwd: geometry not covered");
  const int64_t total = planes * ih * iw;
  if (total == 0) return OMT_OK;
  OMT_POOL_LAUNCH(avgpool_bwd_kernel, total, stream_of(stream), g, gx, total,
                  pgeo(ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, 1, 1), count_include_pad, (int)divisor_override);
  return launch_check("avgpool_bwd_kernel");
}

OMT_EXPORT int omt_adapool_fwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, const float* x,
                               float* y, void* stream) {
  if (!x || !y) return fail(OMT_INVALID, "omt_adapool_fwd: null pointer");
  if (!pool_ok(planes, ih, iw, oh, ow)) return fail(OMT_UNSUPPORTED, "omt_adapool_fwd: geometry not covered");
  if (planes == 0) return OMT_OK;
  hipStream_t s = stream_of(stream);
  if (oh == 1 && ow == 1) {
    if (ih * iw <= 64 && cdiv(planes, 256) < ((int64_t)1 << 31)) {
      hipLaunchKernelGGL(gap_small_kernel, dim3((unsigned)cdiv(planes, 256)), dim3(256), 0, s, x, y, planes,
                         (int)(ih * iw));
      return launch_check("gap_small_kernel");
    }
    hipLaunchKernelGGL(gap_fwd_kernel, dim3((unsigned)cdiv(planes, 4)), dim3(256), 0, s, x, y, planes, (int)(ih * iw));
    return launch_check("gap_fwd_kernel");
  }
  const int64_t total = planes * oh * ow;
  hipLaunchKernelGGL(adapool_fwd_kernel, dim3(grid1d(total, 256)), dim3(256), 0, s, x, y, total, (int)ih, (int)iw,
                     (int)oh, (int)ow);
  return launch_check("adapool_fwd_kernel");
}

OMT_EXPORT int omt_adapool_bwd(int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow, const float* g,
                               float* gx, void* stream) {
  if (!g || !gx) return fail(OMT_INVALID, "omt_adapool_bwd: null pointer");
  if (!pool_ok(planes, ih, iw, oh, ow)) return fail(OMT_UNSUPPORTED, "omt_adapool_bwd: geometry not covered");
  const int64_t total = planes * ih * iw;
  if (total == 0) return OMT_OK;
  if (oh == 1 && ow == 1) {
    const FastDiv d_hw = make_fastdiv((uint32_t)(ih * iw));
    OMT_POOL_LAUNCH(gap_bwd_kernel, total, stream_of(stream), g, gx, total, (int)(ih * iw), d_hw);
    return launch_check("gap_bwd_kernel");
  }
  hipLaunchKernelGGL(adapool_bwd_kernel, dim3(grid1d(total, 256)), dim3(256), 0, stream_of(stream), g, gx, total,
                     (int)ih, (int)iw, (int)oh, (int)ow);
  return launch_check("adapool_bwd_kernel");
}

OMT_EXPORT int omt_maxpool_fwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh,
                                    int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                                    const float* x, float* y, int64_t* idx, void* stream) {
  if (!x || !y || !idx) return fail(OMT_INVALID, "omt_maxpool_fwd_nhwc: null pointer");
  if (!nhwc_pool_ok(n, c, ih, iw, oh, ow) || kh < 1 || kw < 1 || sh < 1 || sw < 1 || dh < 1 || dw < 1 || ph < 0 ||
      pw < 0)
    return fail(OMT_UNSUPPORTED, "omt_maxpool_fwd_nhwc: geometry not covered");
  const bool vec = c % 4 == 0 && a16(x) && a16(y);
  const NhwcPool p = nhwc_pool(c, vec, ow, oh);
  const int64_t total = n * oh * ow * p.cv;
  if (total == 0) return OMT_OK;
  OMT_NHWC_LAUNCH(maxpool_fwd_nhwc_kernel, total, stream_of(stream), vec, x, y, idx, (uint32_t)total,
                  pgeo(ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, dh, dw), p);
  return launch_check("maxpool_fwd_nhwc_kernel");
}

OMT_EXPORT int omt_maxpool_bwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh,
                                    int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t dh, int64_t dw,
                                    const float* g, const int64_t* idx, float* gx, void* stream) {
  if (!g || !idx || !gx) return fail(OMT_INVALID, "omt_maxpool_bwd_nhwc: null pointer");
  if (!nhwc_pool_ok(n, c, ih, iw, oh, ow) || kh < 1 || kw < 1 || sh < 1 || sw < 1 || dh < 1 || dw < 1 || ph < 0 ||
      pw < 0)
    return fail(OMT_UNSUPPORTED, "omt_maxpool_bwd_nhwc: geometry not covered");
  const bool vec = c % 4 == 0 && a16(g) && a16(gx);
  const NhwcPool p = nhwc_pool(c, vec, iw, ih);
  const int64_t total = n * ih * iw * p.cv;
  if (total == 0) return OMT_OK;
  OMT_NHWC_LAUNCH(maxpool_bwd_nhwc_kernel, total, stream_of(stream), vec, g, idx, gx, (uint32_t)total,
                  pgeo(ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, dh, dw), p);
  return launch_check("maxpool_bwd_nhwc_kernel");
}

OMT_EXPORT int omt_avgpool_fwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh,
                                    int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int count_include_pad,
                                    int64_t divisor_override, const float* x, float* y, void* stream) {
  if (!x || !y) return fail(OMT_INVALID, "omt_avgpool_fwd_nhwc: null pointer");
  if (!nhwc_pool_ok(n, c, ih, iw, oh, ow) || kh < 1 || kw < 1 || sh < 1 || sw < 1 || ph < 0 || pw < 0)
    return fail(OMT_UNSUPPORTED, "omt_avgpool_fwd_nhwc: geometry not covered");
  const bool vec = c % 4 == 0 && a16(x) && a16(y);
  const NhwcPool p = nhwc_pool(c, vec, ow, oh);
  const int64_t total = n * oh * ow * p.cv;
  if (total == 0) return OMT_OK;
  OMT_NHWC_LAUNCH(avgpool_fwd_nhwc_kernel, total, stream_of(stream), vec, x, y, (uint32_t)total,
                  pgeo(ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, 1, 1), p, count_include_pad, (int)divisor_override);
  return launch_check("avgpool_fwd_nhwc_kernel");
}

OMT_EXPORT int omt_avgpool_bwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow, int64_t kh,
                                    int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int count_include_pad,
                                    int64_t divisor_override, const float* g, float* gx, void* stream) {
  if (!g || !gx) return fail(OMT_INVALID, "omt_avgpool_bwd_nhwc: null pointer");
  if (!nhwc_pool_ok(n, c, ih, iw, oh, ow) || kh < 1 || kw < 1 || sh < 1 || sw < 1 || ph < 0 || pw < 0)
    return fail(OMT_UNSUPPORTED, "omt_avgpool_bwd_nhwc: geometry not covered");
  const bool vec = c % 4 == 0 && a16(g) && a16(gx);
  const NhwcPool p = nhwc_pool(c, vec, iw, ih);
  const int64_t total = n * ih * iw * p.cv;
  if (total == 0) return OMT_OK;
  OMT_NHWC_LAUNCH(avgpool_bwd_nhwc_kernel, total, stream_of(stream), vec, g, gx, (uint32_t)total,
                  pgeo(ih, iw, oh, ow, kh, kw, sh, sw, ph, pw, 1, 1), p, count_include_pad, (int)divisor_override);
  return launch_check("avgpool_bwd_nhwc_kernel");
}

OMT_EXPORT int omt_adapool_fwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow,
                                    const float* x, float* y, void* stream) {
  if (!x || !y) return fail(OMT_INVALID, "omt_adapool_fwd_nhwc: null pointer");
  if (!nhwc_pool_ok(n, c, ih, iw, oh, ow)) return fail(OMT_UNSUPPORTED, "omt_adapool_fwd_nhwc: geometry not covered");
  const bool vec = c % 4 == 0 && a16(x) && a16(y);
  const NhwcPool p = nhwc_pool(c, vec, ow, oh);
  const int64_t total = n * oh * ow * p.cv;
  if (total == 0) return OMT_OK;
  OMT_NHWC_LAUNCH(adapool_fwd_nhwc_kernel, total, stream_of(stream), vec, x, y, (uint32_t)total, (int)ih, (int)iw,
                  (int)oh, (int)ow, p);
  return launch_check("adapool_fwd_nhwc_kernel");
}

OMT_EXPORT int omt_adapool_bwd_nhwc(int64_t n, int64_t c, int64_t ih, int64_t iw, int64_t oh, int64_t ow,
                                    const float* g, float* gx, void* stream) {
  if (!g || !gx) return fail(OMT_INVALID, "omt_adapool_bwd_nhwc: null pointer");
  if (!nhwc_pool_ok(n, c, ih, iw, oh, ow)) return fail(OMT_UNSUPPORTED, "omt_adapool_bwd_nhwc: geometry not covered");
  const bool vec = c % 4 == 0 && a16(g) && a16(gx);
  const NhwcPool p = nhwc_pool(c, vec, iw, ih);
  const int64_t total = n * ih * iw * p.cv;
  if (total == 0) return OMT_OK;
  OMT_NHWC_LAUNCH(adapool_bwd_nhwc_kernel, total, stream_of(stream), vec, g, gx, (uint32_t)total, (int)ih, (int)iw,
                  (int)oh, (int)ow, p);
  return launch_check("adapool_bwd_nhwc_kernel");
}
