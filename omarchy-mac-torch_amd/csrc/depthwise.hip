// Depthwise convolution (groups = C, one ks x ks filter per channel): any ks <= 11, stride 1..4, 0 <= pad <= ks.
// These are HBM-bandwidth-bound (ks^2 FLOPs per loaded element).
//
// Stride 1 with "same" padding and ks 3, 5 or 7 (every depthwise layer of the benchmark configurations) runs LDS-tiled:
// a workgroup owns a chunk of R output rows of one (image, channel) plane, stages the R + ks - 1 input rows it reads
// (zero outside the plane) in LDS with ks/2 zero columns either side, keeps the plane's filter in registers and writes
// its outputs contiguously. Grad input is the same correlation over gy with the filter flipped (same padding). Grad
// weight stages x the same way per (channel, image slice) and accumulates all ks^2 taps in registers; the slices are
// summed in order. Every other geometry uses plain wave64 kernels:
//  - forward: one thread per output element, the filter in registers (reference dw_fwd / dwg_fwd / dw_fwd_bn,
//    csrc/conv.cpp:194-198, csrc/plans.cpp:145-158), optional previous-layer eval BN + ReLU on in-bounds taps;
//  - grad input: one thread per input element, keeping the taps that land on the stride grid (dw_gin / dwg_gin);
//  - grad weight: workgroup (channel, slice) accumulates every tap over its share of n * oh * ow, partials summed in
//    slice order (dw_gwt / dwg_gwt).
#include <algorithm>

#include "lds_dma.h"
#include "omt_internal.h"
#include "slice_sum.h"

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

// Slice sums in slice order, eight slices' loads in flight at a time (a grid this small waits on memory latency).
__global__ void __launch_bounds__(256) dw_wgrad_reduce_kernel(const float* __restrict__ part, float* __restrict__ gw,
                                                              int n, int slices) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    float s = 0.f;
    int z = 0;
    for (; z + 8 <= slices; z += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = part[(int64_t)(z + u) * n + i];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; z < slices; ++z) s += part[(int64_t)z * n + i];
    gw[i] = s;
  }
}

// ---- stride 1, "same" padding, ks 3 / 5 / 7: LDS-tiled -----------------------------------------------------------

constexpr int kDwOutPerThread = 8;  // output elements per thread of a tiled forward / grad-input work unit
constexpr int kDwWgOut = 16;        // output gradients per thread of a tiled grad-weight batch

struct DwTiling {
  int rows;    // output rows per work unit
  int chunks;  // work units per plane
  int pitch;   // LDS row pitch: W + ks - 1
  FastDiv div_w, div_chunks, div_pitch;
};

// Stages `rows` rows of a plane, from row r0 - pad, with `pad` zero columns either side, as tile[rr * pitch + cc]. The
// tile is walked as a flat range, kStageBatch elements per thread at a time: all of a batch's loads are issued before
// any LDS store, so a workgroup waits about one memory latency per batch rather than one per row.
constexpr int kStageBatch = 16;
template <int NT>
__device__ __forceinline__ void dw_stage_rows(float* __restrict__ tile, const float* __restrict__ src_plane, int r0,
                                              int rows, int H, int W, int pitch, const FastDiv& div_pitch, int pad,
                                              bool bn, float sc, float sh) {
  const int total = rows * pitch;
  for (int e0 = 0; e0 < total; e0 += NT * kStageBatch) {
    float v[kStageBatch];
#pragma unroll
    for (int j = 0; j < kStageBatch; ++j) {
      const int e = e0 + (int)threadIdx.x + j * NT;
      v[j] = 0.f;
      if (e < total) {
        const int rr = (int)fdiv((uint32_t)e, div_pitch), iy = r0 - pad + rr, ix = e - rr * pitch - pad;
        if ((unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W) v[j] = src_plane[(int64_t)iy * W + ix];
      }
    }
#pragma unroll
    for (int j = 0; j < kStageBatch; ++j) {
      const int e = e0 + (int)threadIdx.x + j * NT;
      if (e < total) {
        float t = v[j];
        if (bn) {  // padding stays zero: BN + ReLU of in-bounds taps only
          const int rr = (int)fdiv((uint32_t)e, div_pitch), iy = r0 - pad + rr, ix = e - rr * pitch - pad;
          if ((unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W) t = fmaxf(fmaf(t, sc, sh), 0.f);
        }
        tile[e] = t;
      }
    }
  }
}

// FLIP: grad input (gy in, filter flipped, no bias / BN).
template <int KS, bool FLIP, int NT>
__global__ void __launch_bounds__(NT) dw_s1_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                   const float* __restrict__ bias, const float* __restrict__ bm,
                                                   const float* __restrict__ bv, const float* __restrict__ bg,
                                                   const float* __restrict__ bb, float eps, float* __restrict__ y,
                                                   int C, int H, int W, const DwTiling t) {
  extern __shared__ float tile[];
  constexpr int PAD = KS / 2, KK = KS * KS;
  const int plane = (int)fdiv(blockIdx.x, t.div_chunks), chunk = (int)blockIdx.x - plane * t.chunks;
  const int ch = plane % C;
  const int r0 = chunk * t.rows, R = min(t.rows, H - r0);
  const int64_t pbase = (int64_t)plane * H * W;
  float sc = 1.f, sh = 0.f;
  const bool bn = !FLIP && bm != nullptr;
  if (bn) {
    const float inv = rsqrtf(bv[ch] + eps);
    sc = inv * bg[ch];
    sh = bb[ch] - bm[ch] * sc;
  }
  dw_stage_rows<NT>(tile, x + pbase, r0, R + KS - 1, H, W, t.pitch, t.div_pitch, PAD, bn, sc, sh);
  float wr[KK];
#pragma unroll
  for (int i = 0; i < KK; ++i) wr[i] = w[ch * KK + (FLIP ? KK - 1 - i : i)];
  const float b = (!FLIP && bias) ? bias[ch] : 0.f;
  __syncthreads();
  float* yp = y + pbase + (int64_t)r0 * W;
  const int nout = R * W, pitch = t.pitch;
  for (int o = threadIdx.x; o < nout; o += NT) {
    const int r = (int)fdiv((uint32_t)o, t.div_w), c = o - r * W;
    const float* tp = tile + r * pitch + c;
    float acc = 0.f;
#pragma unroll
    for (int ky = 0; ky < KS; ++ky)
#pragma unroll
      for (int kx = 0; kx < KS; ++kx) acc = fmaf(tp[ky * pitch + kx], wr[ky * KS + kx], acc);
    yp[o] = acc + b;
  }
}

// Whole small planes, several images of one channel per workgroup. A workgroup of this kernel takes images
// n0 .. n0 + nb - 1 (nb <= B) of channel ch: every thread issues the loads of its kDwBatchEPT interior elements of
// the batch first (consecutive threads on consecutive elements of a plane), zeroes the batch's LDS tiles meanwhile
// (one (H + KS - 1) x (W + KS - 1) tile per plane: the zero border is the padding), stores the values into the tiles'
// interiors and computes every output of the batch from LDS with the channel's filter in registers. Several planes
// per workgroup keep kDwBatchEPT loads per thread in flight where a plane alone would give each thread a few.
constexpr int kDwBatchEPT = 16;
struct DwBatch {
  int B, tile, pitch;  // images per workgroup, LDS floats per plane, LDS row pitch W + KS - 1
  FastDiv div_hw, div_w, div_c;
};
template <int KS, bool FLIP, int NT>
__global__ void __launch_bounds__(NT) dw_s1_batch_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                         const float* __restrict__ bias, const float* __restrict__ bm,
                                                         const float* __restrict__ bv, const float* __restrict__ bg,
                                                         const float* __restrict__ bb, float eps,
                                                         float* __restrict__ y, int N, int C, int H, int W,
                                                         const DwBatch d) {
  extern __shared__ float tile[];
  constexpr int PAD = KS / 2, KK = KS * KS, EPT = kDwBatchEPT;
  const int grp = (int)fdiv(blockIdx.x, d.div_c), ch = (int)blockIdx.x - grp * C;
  const int n0 = grp * d.B, nb = min(d.B, N - n0);
  const int HW = H * W, total = nb * HW, pitch = d.pitch;
  const int64_t cstride = (int64_t)C * HW;
  const float* src = x + ((int64_t)n0 * C + ch) * HW;
  float v[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = (int)threadIdx.x + j * NT;
    v[j] = 0.f;
    if (e < total) {
      const int i = (int)fdiv((uint32_t)e, d.div_hw);
      v[j] = src[i * cstride + (e - i * HW)];
    }
  }
  for (int e = threadIdx.x; e < nb * d.tile; e += NT) tile[e] = 0.f;
  float sc = 1.f, sh = 0.f;
  const bool bn = !FLIP && bm != nullptr;
  if (bn) {
    const float inv = rsqrtf(bv[ch] + eps);
    sc = inv * bg[ch];
    sh = bb[ch] - bm[ch] * sc;
  }
  __syncthreads();  // the zero fill is done before the interiors are written
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = (int)threadIdx.x + j * NT;
    if (e < total) {
      const int i = (int)fdiv((uint32_t)e, d.div_hw), rem = e - i * HW;
      const int r = (int)fdiv((uint32_t)rem, d.div_w), c = rem - r * W;
      tile[i * d.tile + (r + PAD) * pitch + c + PAD] = bn ? fmaxf(fmaf(v[j], sc, sh), 0.f) : v[j];
    }
  }
  float wr[KK];
#pragma unroll
  for (int i = 0; i < KK; ++i) wr[i] = w[ch * KK + (FLIP ? KK - 1 - i : i)];
  const float b = (!FLIP && bias) ? bias[ch] : 0.f;
  __syncthreads();
  float* dst = y + ((int64_t)n0 * C + ch) * HW;
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int o = (int)threadIdx.x + j * NT;
    if (o < total) {
      const int i = (int)fdiv((uint32_t)o, d.div_hw), rem = o - i * HW;
      const int r = (int)fdiv((uint32_t)rem, d.div_w), c = rem - r * W;
      const float* tp = tile + i * d.tile + r * pitch + c;
      float acc = 0.f;
#pragma unroll
      for (int ky = 0; ky < KS; ++ky)
#pragma unroll
        for (int kx = 0; kx < KS; ++kx) acc = fmaf(tp[ky * pitch + kx], wr[ky * KS + kx], acc);
      dst[i * cstride + rem] = acc + b;
    }
  }
}

// Rows of a multiple of 4 (every W % 4 == 0 plane, tensors below 2 GiB): no LDS. A thread owns a 4-column x RB-row
// block of one plane's outputs and loads the RB + KS - 1 input rows it reads straight into registers, each row as one
// 16-byte run over the block's columns plus a KS / 2-float run either side (buffer loads: rows and runs outside the
// plane read 0, the zero padding), all before its first FMA, so a thread keeps (RB + KS - 1) * 3 loads in flight
// where the staged kernels wait one memory round trip per stage. Neighbouring threads read overlapping runs; the
// overlap is served by the caches, not HBM. Each output sums its taps in the staged kernels' order (ky, then kx, from
// 0; bias last), so the results are identical to theirs. The filter comes in 16-byte runs too (per lane: a wave can
// span planes of two channels).
struct DwReg {
  uint32_t threads;           // planes * row blocks * W / 4
  uint32_t bytes;             // bytes of x (and y), below 2^31
  FastDiv div_cg, div_rb, div_c;
};
template <int N>
__device__ __forceinline__ void bload_run(__amdgpu_buffer_rsrc_t r, uint32_t off, float* v) {
  if constexpr (N == 1) {
    v[0] = bload(r, off, 0);
  } else if constexpr (N == 2) {
    // whole-vector bit casts: subscripting the builtin's result directly has compiled to two copies of element 0
    const float2 t = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
    v[0] = t.x;
    v[1] = t.y;
  } else {
    static_assert(N == 3, "runs of 1 to 3 floats");
    typedef float f32x3 __attribute__((ext_vector_type(3)));
    const f32x3 t = __builtin_bit_cast(f32x3, __builtin_amdgcn_raw_buffer_load_b96(r, (int)off, 0, 0));
    v[0] = t.x;
    v[1] = t.y;
    v[2] = t.z;
  }
}
// The input window of a 4-column x RB-row output block at (r0, c0) of the plane starting at element pbase:
// v[i][j] = x[r0 - KS / 2 + i][c0 - KS / 2 + j], zero outside the plane.
template <int KS, int RB>
__device__ __forceinline__ void dw_window(__amdgpu_buffer_rsrc_t xr, uint32_t pbase, int r0, int c0, int H, int W,
                                          float (&v)[RB + KS - 1][4 + 2 * (KS / 2)]) {
  constexpr int PAD = KS / 2, NR = RB + KS - 1;
  const bool lok = c0 > 0, rok = c0 + 4 < W;
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int iy = r0 - PAD + i;
    const bool ok = (unsigned)iy < (unsigned)H;
    const uint32_t off = (pbase + (uint32_t)(iy * W + c0)) * 4u;
    const float4 m = bload4(xr, ok ? off : kOOB, 0);
    v[i][PAD] = m.x;
    v[i][PAD + 1] = m.y;
    v[i][PAD + 2] = m.z;
    v[i][PAD + 3] = m.w;
    if constexpr (PAD > 0) {
      bload_run<PAD>(xr, ok & lok ? off - PAD * 4u : kOOB, &v[i][0]);
      bload_run<PAD>(xr, ok & rok ? off + 16u : kOOB, &v[i][PAD + 4]);
    }
  }
}

template <int KS, bool FLIP, int RB>
__global__ void __launch_bounds__(256) dw_s1_reg_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                        const float* __restrict__ bias, const float* __restrict__ bm,
                                                        const float* __restrict__ bv, const float* __restrict__ bg,
                                                        const float* __restrict__ bb, float eps, float* __restrict__ y,
                                                        int C, int H, int W, const DwReg d) {
  constexpr int PAD = KS / 2, KK = KS * KS, NR = RB + KS - 1, NC = 4 + 2 * PAD;
  const uint32_t t = blockIdx.x * 256u + threadIdx.x;
  if (t >= d.threads) return;
  const uint32_t CG = (uint32_t)W >> 2, u = fdiv(t, d.div_cg), cg = t - u * CG;
  const uint32_t nrb = (uint32_t)(H + RB - 1) / RB, plane = fdiv(u, d.div_rb), rb = u - plane * nrb;
  const int ch = (int)(plane - fdiv(plane, d.div_c) * (uint32_t)C);
  const int c0 = (int)cg * 4, r0 = (int)rb * RB;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, d.bytes);
  const uint32_t pbase = plane * (uint32_t)H * (uint32_t)W;  // elements; below 2^29
  const bool lok = c0 > 0, rok = c0 + 4 < W;
  float v[NR][NC];
  dw_window<KS, RB>(xr, pbase, r0, c0, H, W, v);
  // the filter: KK floats of channel ch in 16-byte runs (the last run's floats past KK belong to the next channel or
  // lie past the tensor; a run is loaded whole only when it ends inside the filter)
  float wr[KK];
  {
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(w, (uint32_t)(C * KK * 4));
    const uint32_t wb = (uint32_t)(ch * KK) * 4u;
    float wl[KK];
#pragma unroll
    for (int k = 0; k + 4 <= KK; k += 4) {
      const float4 q = bload4(wrs, wb + k * 4u, 0);
      wl[k] = q.x;
      wl[k + 1] = q.y;
      wl[k + 2] = q.z;
      wl[k + 3] = q.w;
    }
#pragma unroll
    for (int k = KK & ~3; k < KK; ++k) wl[k] = bload(wrs, wb + k * 4u, 0);
#pragma unroll
    for (int k = 0; k < KK; ++k) wr[k] = wl[FLIP ? KK - 1 - k : k];
  }
  const bool bn = !FLIP && bm != nullptr;
  if (bn) {  // previous layer's eval BN + ReLU on in-plane taps; the padding stays zero
    const float inv = rsqrtf(bv[ch] + eps), sc = inv * bg[ch], sh = bb[ch] - bm[ch] * sc;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
      const int iy = r0 - PAD + i;
      const bool ok = (unsigned)iy < (unsigned)H;
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const bool in = ok & (j < PAD ? lok : j >= PAD + 4 ? rok : true);
        if (in) v[i][j] = fmaxf(fmaf(v[i][j], sc, sh), 0.f);
      }
    }
  }
  float acc[RB][4];
#pragma unroll
  for (int o = 0; o < RB; ++o)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[o][e] = 0.f;
#pragma unroll
  for (int i = 0; i < NR; ++i)
#pragma unroll
    for (int ky = KS - 1; ky >= 0; --ky) {  // output row i - ky: taps in ascending ky as i ascends
      const int o = i - ky;
      if (o < 0 || o >= RB) continue;
#pragma unroll
      for (int kx = 0; kx < KS; ++kx)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[o][e] = fmaf(v[i][e + kx], wr[ky * KS + kx], acc[o][e]);
    }
  const float b = (!FLIP && bias) ? bias[ch] : 0.f;
#pragma unroll
  for (int o = 0; o < RB; ++o)
    if (r0 + o < H)
      *reinterpret_cast<float4*>(y + pbase + (uint32_t)((r0 + o) * W + c0)) =
          make_float4(acc[o][0] + b, acc[o][1] + b, acc[o][2] + b, acc[o][3] + b);
}

// Grad weight, rows of a multiple of 4: workgroup (ch, slice) sums every tap over images [slice * ipw, ...) of
// channel ch. Each thread takes 4-column x RB-row blocks of gy in turn (stride NT over the slice's blocks), loads the
// block and the input window it meets (as the forward kernel does: no LDS, zero padding from the buffer range check)
// and accumulates all KS^2 taps in registers; the taps are then summed over the workgroup (wave_sum, then the waves
// in order). One slice writes gw; several write part[slice][ch], summed in slice order by dw_wgrad_reduce_kernel. A
// fixed thread-to-block map and fixed sum orders make the result deterministic.
struct DwRegW {
  int ipw, CG, nrb, slices;  // images per slice, column groups W / 4, row blocks, slices
  int rb, nt;                // rows per block, threads per workgroup
  uint32_t bytes;            // bytes of x (and gy), below 2^31
  FastDiv div_img, div_cg;   // blocks per image (nrb * CG), CG
};
template <int KS, int RB, int NT>
__global__ void __launch_bounds__(NT) dw_wgrad_reg_kernel(const float* __restrict__ x, const float* __restrict__ gy,
                                                           float* __restrict__ gw, float* __restrict__ part, int N,
                                                           int C, int H, int W, const DwRegW d) {
  constexpr int PAD = KS / 2, KK = KS * KS, NR = RB + KS - 1, NC = 4 + 2 * PAD, NW = NT / 64;
  __shared__ float red[NW][KK];
  const int ch = blockIdx.x, sl = blockIdx.y;
  const int n0 = sl * d.ipw, nimg = min(N - n0, d.ipw);
  const uint32_t per_img = (uint32_t)(d.nrb * d.CG), units = (uint32_t)nimg * per_img;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, d.bytes), gr = make_rsrc(gy, d.bytes);
  float acc[KK];
#pragma unroll
  for (int k = 0; k < KK; ++k) acc[k] = 0.f;
  for (uint32_t u = threadIdx.x; u < units; u += NT) {
    const uint32_t i = fdiv(u, d.div_img), rem = u - i * per_img, rb = fdiv(rem, d.div_cg);
    const int c0 = (int)(rem - rb * (uint32_t)d.CG) * 4, r0 = (int)rb * RB;
    const uint32_t pbase = ((uint32_t)(n0 + (int)i) * (uint32_t)C + (uint32_t)ch) * (uint32_t)H * (uint32_t)W;
    float gv[RB][4];
#pragma unroll
    for (int o = 0; o < RB; ++o) {
      const float4 q = bload4(gr, r0 + o < H ? (pbase + (uint32_t)((r0 + o) * W + c0)) * 4u : kOOB, 0);
      gv[o][0] = q.x;
      gv[o][1] = q.y;
      gv[o][2] = q.z;
      gv[o][3] = q.w;
    }
    float v[NR][NC];
    dw_window<KS, RB>(xr, pbase, r0, c0, H, W, v);
#pragma unroll
    for (int o = 0; o < RB; ++o)
#pragma unroll
      for (int ky = 0; ky < KS; ++ky)
#pragma unroll
        for (int kx = 0; kx < KS; ++kx)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[ky * KS + kx] = fmaf(gv[o][e], v[o + ky][e + kx], acc[ky * KS + kx]);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < KK; ++k) {
    const float t = wave_sum(acc[k]);
    if (lane == 0) red[wave][k] = t;
  }
  __syncthreads();
  const int k = threadIdx.x;
  float t = 0.f;
  if (k < KK) {
#pragma unroll
    for (int wv = 0; wv < NW; ++wv) t += red[wv][k];
  }
  if (d.slices == 1) {
    if (k < KK) gw[ch * KK + k] = t;
    return;
  }
  if (k < KK) part[((int64_t)sl * C + ch) * KK + k] = t;
}

// Grad-weight work of one channel: units u = (image u / chunks, row chunk u % chunks), N * chunks of them. A
// workgroup takes `group` consecutive units and stages `batch` of them at a time (several whole planes when a plane
// has few outputs; then chunks == 1): every load of a batch (the output gradients into registers, the input rows
// into LDS) is issued before its one barrier, so a batch costs one memory round trip.
struct DwUnits {
  int units, group, batch, tile;  // tile: LDS floats per staged unit, (rows + ks - 1) * pitch
  int buf;                        // LDS floats per tile buffer: batch * tile in whole rows of 64
  FastDiv div_tile, div_out;      // div_out: outputs per unit when batch > 1 (H * W)
};

// grid (C, groups): workgroup (ch, g) reduces units [g * group, (g + 1) * group) of channel ch into part[g][ch][KK].
// Output gradients are raw buffer loads into registers; the input rows go straight to LDS (each wave moving one row
// of 64 consecutive tile floats per load), so no register holds a staged value and an address takes one register.
// Two tile buffers, each in whole rows of 64 floats (the last row's lanes past a batch write zeros there): the loads
// of batch b + 1 are issued before the FMAs of batch b. The partial sums of each tap go through wave_sum.
template <int KS, int NT>
__global__ void __launch_bounds__(NT) dw_wgrad_s1_kernel(const float* __restrict__ x, const float* __restrict__ gy,
                                                         float* __restrict__ part, int C, int H, int W,
                                                         const DwTiling t, const DwUnits wu) {
  extern __shared__ float tiles[];
  constexpr int PAD = KS / 2, KK = KS * KS, NW = NT / 64;
  __shared__ float red[NW][KK];
  const int ch = blockIdx.x, pitch = t.pitch, HW = H * W;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const uint32_t cstride = (uint32_t)C * (uint32_t)HW;  // elements from one image's plane of ch to the next's
  const int ubeg = (int)blockIdx.y * wu.group, uend = min(wu.units, ubeg + wu.group);
  float* const buf[2] = {tiles, tiles + wu.buf};

  // batch at u0: batch > 1 covers whole planes (chunk 0, rows = H), batch == 1 one chunk of rows
  struct Batch {
    int nb, n0, r0, nout;
  };
  auto batch_at = [&](int u0) {
    Batch b;
    b.nb = min(wu.batch, uend - u0);
    b.n0 = (int)fdiv((uint32_t)u0, t.div_chunks);
    b.r0 = (u0 - b.n0 * t.chunks) * t.rows;
    b.nout = wu.batch > 1 ? b.nb * HW : min(t.rows, H - b.r0) * W;  // at most kDwWgOut * NT (dw_units)
    return b;
  };
  // the loads of a batch: its output gradients into g, its input rows into tile (tile float e: tile i = e / wu.tile,
  // row rr, column cc within it, is input row r0 - PAD + rr, column cc - PAD of unit u0 + i; padding and lanes past
  // the batch load offset kOOB, which reads 0)
  auto issue = [&](const Batch& b, float* tile, float (&g)[kDwWgOut]) {
    const int64_t base = ((int64_t)b.n0 * C + ch) * HW;
    const uint32_t span = ((uint32_t)(b.nb - 1) * cstride + (uint32_t)HW) * 4u;  // < 2^31 (dw_units)
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(gy + base, span);
#pragma unroll
    for (int j = 0; j < kDwWgOut; ++j) {
      const int o = (int)threadIdx.x + j * NT;
      uint32_t off = kOOB;
      if (o < b.nout) {
        const int i = wu.batch > 1 ? (int)fdiv((uint32_t)o, wu.div_out) : 0, pix = o - i * (wu.batch > 1 ? HW : 0);
        off = ((uint32_t)i * cstride + (uint32_t)(b.r0 * W + pix)) * 4u;
      }
      g[j] = bload(gr, off, 0);
    }
    const omt_u32x4 xr = rsrc_words(x + base, span);
    const int total = b.nb * wu.tile;
    for (int e0 = wave * 64; e0 < total; e0 += NT) {
      const int e = e0 + lane;
      uint32_t off = kOOB;
      if (e < total) {
        const int i = (int)fdiv((uint32_t)e, wu.div_tile), rem = e - i * wu.tile;
        const int rr = (int)fdiv((uint32_t)rem, t.div_pitch), iy = b.r0 - PAD + rr, ix = rem - rr * pitch - PAD;
        if ((unsigned)iy < (unsigned)H && (unsigned)ix < (unsigned)W)
          off = ((uint32_t)i * cstride + (uint32_t)(iy * W + ix)) * 4u;
      }
      lds_load_b32(xr, lds_addr(tile + e0), off, 0);
    }
  };
  float acc[KK];
#pragma unroll
  for (int i = 0; i < KK; ++i) acc[i] = 0.f;
  auto fma_batch = [&](const Batch& b, const float* tile, const float (&g)[kDwWgOut]) {
#pragma unroll 2
    for (int j = 0; j < kDwWgOut; ++j) {
      const int o = (int)threadIdx.x + j * NT;
      if (o < b.nout) {
        const int i = wu.batch > 1 ? (int)fdiv((uint32_t)o, wu.div_out) : 0, pix = o - i * (wu.batch > 1 ? HW : 0);
        const int r = (int)fdiv((uint32_t)pix, t.div_w), c = pix - r * W;
        const float* tp = tile + i * wu.tile + r * pitch + c;
        const float gj = g[j];
#pragma unroll
        for (int ky = 0; ky < KS; ++ky)
#pragma unroll
          for (int kx = 0; kx < KS; ++kx) acc[ky * KS + kx] = fmaf(gj, tp[ky * pitch + kx], acc[ky * KS + kx]);
      }
    }
  };
  // every load issued so far has landed (both kinds count in vmcnt), and then every wave's rows are visible and every
  // wave is done with the other buffer
  auto land = [&]() {
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    asm volatile("" ::: "memory");
    __syncthreads();
  };

  float ga[kDwWgOut], gb[kDwWgOut];
  Batch ba = batch_at(ubeg), bb;
  issue(ba, buf[0], ga);
  for (int u0 = ubeg; u0 < uend; u0 += 2 * wu.batch) {
    land();
    const int u1 = u0 + wu.batch;
    if (u1 < uend) {
      bb = batch_at(u1);
      issue(bb, buf[1], gb);
    }
    fma_batch(ba, buf[0], ga);
    if (u1 >= uend) break;
    land();
    const int u2 = u1 + wu.batch;
    if (u2 < uend) {
      ba = batch_at(u2);
      issue(ba, buf[0], ga);
    }
    fma_batch(bb, buf[1], gb);
  }
#pragma unroll
  for (int i = 0; i < KK; ++i) {
    const float v = wave_sum(acc[i]);
    if (lane == 0) red[wave][i] = v;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < KK; i += NT) {
    float v = 0.f;
#pragma unroll
    for (int wv = 0; wv < NW; ++wv) v += red[wv][i];
    part[((int64_t)blockIdx.y * C + ch) * KK + i] = v;
  }
}

constexpr int kDwMaxLds = 64 * 1024;

// ~8 outputs per thread (at most kDwOutPerThread); one wave for planes of up to 128 outputs.
static DwTiling dw_tiling(int H, int W, int ks, int nt) {
  DwTiling t;
  int rows = (nt * kDwOutPerThread) / W;
  rows = rows < 1 ? 1 : rows > H ? H : rows;
  t.rows = rows;
  t.chunks = (int)cdiv(H, rows);
  t.pitch = W + ks - 1;
  t.div_w = make_fastdiv((uint32_t)W);
  t.div_chunks = make_fastdiv((uint32_t)t.chunks);
  t.div_pitch = make_fastdiv((uint32_t)t.pitch);
  return t;
}
static int dw_threads(const omt_conv_geo* g) { return g->ih * g->iw <= 128 ? 64 : 256; }
static size_t dw_lds(const DwTiling& t, int ks) { return (size_t)(t.rows + ks - 1) * t.pitch * sizeof(float); }

static bool dw_s1(const omt_conv_geo* g) {
  if (g->stride != 1 || g->pad != g->ks / 2 || !(g->ks == 3 || g->ks == 5 || g->ks == 7)) return false;
  if (g->n * g->ci >= ((int64_t)1 << 31)) return false;
  // a work unit (at least one row) must fit kDwOutPerThread outputs per thread
  if (g->iw > (int64_t)dw_threads(g) * kDwOutPerThread) return false;
  return dw_lds(dw_tiling((int)g->ih, (int)g->iw, (int)g->ks, dw_threads(g)), (int)g->ks) <= (size_t)kDwMaxLds;
}
// The tiled grad weight reads a plane through one buffer resource (planes below 2 GiB) and holds two tile buffers,
// each in whole rows of 64 floats, in kDwMaxLds of LDS.
static bool dw_s1_wgrad(const omt_conv_geo* g) {
  if (!dw_s1(g) || g->ih * g->iw * 4 > kMaxBufBytes) return false;
  const DwTiling t = dw_tiling((int)g->ih, (int)g->iw, (int)g->ks, dw_threads(g));
  return 2 * cdiv((int64_t)(t.rows + g->ks - 1) * t.pitch, 64) * 64 * 4 <= kDwMaxLds;
}
// Units of the tiled grad weight: whole planes batched while a batch keeps at most kDwWgOut outputs per thread,
// one load per thread and 64-float row (kStageBatch rows per wave) and two buffers in kDwMaxLds of LDS; groups of
// batches sized for about 2048 workgroups.
static DwUnits dw_units(const omt_conv_geo* g) {
  const int nt = dw_threads(g), ks = (int)g->ks;
  const DwTiling t = dw_tiling((int)g->ih, (int)g->iw, ks, nt);
  DwUnits u{};
  u.units = (int)(g->n * t.chunks);
  u.tile = (t.rows + ks - 1) * t.pitch;
  int64_t b = 1;
  if (t.chunks == 1) {
    // the batch's planes span ((b - 1) * C + 1) * H * W floats, read through one buffer resource (< 2 GiB)
    const int64_t span_cap = (kMaxBufBytes / 4 / (g->ih * g->iw) - 1) / g->ci + 1;
    b = std::min<int64_t>({(int64_t)nt * kDwWgOut / (g->ih * g->iw), (int64_t)nt * kStageBatch / u.tile,
                           ((int64_t)kDwMaxLds / 8 - 64) / u.tile, (int64_t)u.units, span_cap});
    b = std::max<int64_t>(b, 1);
  }
  u.batch = (int)b;
  u.buf = (int)(cdiv(b * u.tile, 64) * 64);
  const int64_t batches = cdiv(u.units, b);
  const int64_t groups = std::max<int64_t>(1, std::min<int64_t>(cdiv(2048, g->ci), batches));
  u.group = (int)(cdiv(batches, groups) * b);
  u.div_tile = make_fastdiv((uint32_t)u.tile);
  u.div_out = make_fastdiv((uint32_t)(g->ih * g->iw));
  return u;
}
// The register-blocked kernel: rows of a multiple of 4 floats, the tensor read through one buffer resource.
static int dw_reg_rows(int ks) { return ks == 7 ? 2 : 4; }
static bool dw_reg_ok(const omt_conv_geo* g) {
  return g->iw % 4 == 0 && g->n * g->ci * g->ih * g->iw * 4 <= kMaxBufBytes && g->ci * g->ks * g->ks * 4 <= kMaxBufBytes;
}

// The register-blocked grad weight: slices of images of about kDwRegUnits blocks each (a workgroup per channel
// leaves most CUs idle when there are few channels), at most kDwRegWgs workgroups, summed by a second launch (an
// in-kernel last-arrival sum costs a device-scope release per workgroup, whole-cache write-backs that serialize:
// measured at b32, dw 3x3 over 72 x 56^2 in 2 / 4 slices 21 / 21 us against 20 / 18 us with the second launch).
// Graph replays at b32 (one slice, 1024 threads -> this split, 256 threads): dw 3x3 over 72 x 56^2 17.8 -> 13.8 us,
// 16 x 56^2 14.2 -> 6.4 us, 88 x 28^2 8.3 -> 6.8 us; dw 5x5 over 96 x 28^2 12.1 -> 10.3 us; b128 dw 3x3 over
// 32 x 28^2 16.0 -> 8.7 us. Workgroups of 1024 threads when a slice still has 1024 blocks of 4 rows, or of 2 rows
// (more waves per CU keep more loads in flight); else 256 threads.
constexpr int kDwRegUnits = 196, kDwRegWgs = 1280;
static DwRegW dw_wreg(const omt_conv_geo* g) {
  DwRegW d{};
  const int ks = (int)g->ks;
  d.CG = (int)(g->iw / 4);
  const int64_t per_img = cdiv(g->ih, dw_reg_rows(ks)) * d.CG;
  const int64_t slices = std::max<int64_t>(
      1, std::min<int64_t>({g->n, cdiv(g->n * per_img, kDwRegUnits), kDwRegWgs / g->ci}));
  d.ipw = (int)cdiv(g->n, slices);
  d.slices = (int)cdiv(g->n, d.ipw);
  auto units = [&](int rb) { return (int64_t)d.ipw * cdiv(g->ih, rb) * d.CG; };
  if (ks != 7 && units(4) >= 1024) {
    d.rb = 4, d.nt = 1024;
  } else if (units(2) >= 1024) {
    d.rb = 2, d.nt = 1024;
  } else {
    d.rb = dw_reg_rows(ks), d.nt = 256;
  }
  d.nrb = (int)cdiv(g->ih, d.rb);
  d.bytes = (uint32_t)(g->n * g->ci * g->ih * g->iw * 4);
  d.div_img = make_fastdiv((uint32_t)(d.nrb * d.CG));
  d.div_cg = make_fastdiv((uint32_t)d.CG);
  return d;
}
// partials [slices][C][ks^2] floats; nothing for one slice
static size_t dw_wreg_workspace(const omt_conv_geo* g) {
  const DwRegW d = dw_wreg(g);
  return d.slices == 1 ? 0 : (size_t)(d.slices * g->ci * g->ks * g->ks) * sizeof(float);
}

static int64_t dw_s1_groups(const omt_conv_geo* g) {
  const DwUnits u = dw_units(g);
  return cdiv(u.units, u.group);
}

// The batched small-plane kernel: B images per workgroup with their tiles in kDwMaxLds, for planes of at most
// kDwBatchMaxHW elements. Measured against the row-chunk kernel (graph replays, b32): 7x7 planes 11.9 -> 8.5 us
// (576 channels, 5x5), 14x14 18.5 -> 11.9 us (240 channels, 5x5); from 28x28 up the row-chunk kernel is faster
// (28x28: 12.9 against 16.1 us), so larger planes keep it.
constexpr int kDwBatchNT = 256, kDwBatchMaxHW = 256;
constexpr int64_t kDwBatchMinWgs = 4 * 256;
static DwBatch dw_batch(const omt_conv_geo* g) {
  DwBatch d{};
  const int64_t hw = g->ih * g->iw, tile = (g->ih + g->ks - 1) * (g->iw + g->ks - 1);
  int64_t b = std::min<int64_t>({(int64_t)kDwBatchEPT * kDwBatchNT / hw, g->n, (int64_t)kDwMaxLds / 4 / tile});
  // fewer images per workgroup where a workgroup per channel (and image group) would leave under four per CU: each
  // workgroup is one load -> LDS -> taps -> store chain, and more of them overlap their chains
  b = std::min<int64_t>(b, std::max<int64_t>(1, cdiv(g->n, cdiv(kDwBatchMinWgs, g->ci))));
  d.B = (int)std::max<int64_t>(b, 0);
  d.tile = (int)tile;
  d.pitch = (int)(g->iw + g->ks - 1);
  d.div_hw = make_fastdiv((uint32_t)hw);
  d.div_w = make_fastdiv((uint32_t)g->iw);
  d.div_c = make_fastdiv((uint32_t)g->ci);
  return d;
}

template <bool FLIP>
static int launch_dw_s1(const omt_conv_geo* g, const float* x, const float* w, const float* bias, const float* bm,
                        const float* bv, const float* bg, const float* bb, float eps, float* y, hipStream_t s) {
  if (dw_reg_ok(g) && (uintptr_t)y % 16 == 0) {
    const int ks = (int)g->ks, rb = dw_reg_rows(ks);
    DwReg d{};
    const int64_t nrb = cdiv(g->ih, rb);
    d.threads = (uint32_t)(g->n * g->ci * nrb * (g->iw / 4));
    d.bytes = (uint32_t)(g->n * g->ci * g->ih * g->iw * 4);
    d.div_cg = make_fastdiv((uint32_t)(g->iw / 4));
    d.div_rb = make_fastdiv((uint32_t)nrb);
    d.div_c = make_fastdiv((uint32_t)g->ci);
    const dim3 grid((unsigned)cdiv(d.threads, 256));
    const int C = (int)g->ci, H = (int)g->ih, W = (int)g->iw;
#define OMT_DW_R(KS_, RB_) \
  hipLaunchKernelGGL((dw_s1_reg_kernel<KS_, FLIP, RB_>), grid, dim3(256), 0, s, x, w, bias, bm, bv, bg, bb, eps, y, C, \
                     H, W, d)
    if (ks == 3) OMT_DW_R(3, 4); else if (ks == 5) OMT_DW_R(5, 4); else OMT_DW_R(7, 2);
#undef OMT_DW_R
    return launch_check("dw_s1_reg_kernel");
  }
  const DwBatch d = dw_batch(g);
  if (d.B >= 1 && g->ih * g->iw <= kDwBatchMaxHW && g->n * g->ci * g->ih * g->iw < ((int64_t)1 << 31)) {
    const dim3 grid((unsigned)(cdiv(g->n, d.B) * g->ci));
    const size_t lds = (size_t)d.B * d.tile * sizeof(float);
    const int N = (int)g->n, C = (int)g->ci, H = (int)g->ih, W = (int)g->iw;
#define OMT_DW_B(KS_) \
  hipLaunchKernelGGL((dw_s1_batch_kernel<KS_, FLIP, kDwBatchNT>), grid, dim3(kDwBatchNT), lds, s, x, w, bias, bm, bv, \
                     bg, bb, eps, y, N, C, H, W, d)
    if (g->ks == 3) OMT_DW_B(3); else if (g->ks == 5) OMT_DW_B(5); else OMT_DW_B(7);
#undef OMT_DW_B
    return launch_check("dw_s1_batch_kernel");
  }
  const int nt = dw_threads(g), ks = (int)g->ks;
  const DwTiling t = dw_tiling((int)g->ih, (int)g->iw, ks, nt);
  const dim3 grid((unsigned)(g->n * g->ci * t.chunks));
  const size_t lds = dw_lds(t, ks);
  const int C = (int)g->ci, H = (int)g->ih, W = (int)g->iw;
#define OMT_DW_S1(KS_, NT_) \
  hipLaunchKernelGGL((dw_s1_kernel<KS_, FLIP, NT_>), grid, dim3(NT_), lds, s, x, w, bias, bm, bv, bg, bb, eps, y, C, H, W, t)
  if (nt == 64) {
    if (ks == 3) OMT_DW_S1(3, 64); else if (ks == 5) OMT_DW_S1(5, 64); else OMT_DW_S1(7, 64);
  } else {
    if (ks == 3) OMT_DW_S1(3, 256); else if (ks == 5) OMT_DW_S1(5, 256); else OMT_DW_S1(7, 256);
  }
#undef OMT_DW_S1
  return launch_check("dw_s1_kernel");
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

// ---- channels-last (NHWC) depthwise -----------------------------------------------------------------------------
// x / gx [n][ih][iw][c], y / gy [n][oh][ow][c]; the filter [c][ks][ks] (a channels_last [c][1][ks][ks] filter has
// that memory order too). Forward and grad input: one thread per (pixel, vector of VEC channels: float4 when c % 4 ==
// 0 and the tensors are 16-byte aligned), so a wave reads runs of channels; the taps in the general kernels' order
// with the same fma chain, so each output is the general NCHW kernel's bit for bit. Grad weight: workgroup (channel
// block, filter row ky, pixel slice), thread (channel vector, row lane) accumulating the row's ks taps over its pixels,
// the row lanes added in lane order, the slices summed in order by a second launch.
template <int VEC>
struct DwVec;
template <>
struct DwVec<4> {
  using T = float4;
  static __device__ __forceinline__ float get(const float4& v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
  }
  static __device__ __forceinline__ void set(float4& v, int i, float f) {
    if (i == 0) v.x = f; else if (i == 1) v.y = f; else if (i == 2) v.z = f; else v.w = f;
  }
};
template <>
struct DwVec<1> {
  using T = float;
  static __device__ __forceinline__ float get(const float& v, int) { return v; }
  static __device__ __forceinline__ void set(float& v, int, float f) { v = f; }
};

struct DwNhwc {
  DwGeo g;
  int cv;                 // channel vectors per pixel
  FastDiv d_cv, d_w, d_h;  // by cv, and the width and height of the plane a thread's pixel lies in
};

__device__ __forceinline__ void dw_nhwc_pos(uint32_t i, const DwNhwc& d, int W, int H, int64_t& img, int& y, int& x,
                                            int& j) {
  const uint32_t pix = fdiv(i, d.d_cv), t = fdiv(pix, d.d_w), im = fdiv(t, d.d_h);
  j = (int)(i - pix * (uint32_t)d.cv);
  x = (int)(pix - t * (uint32_t)W);
  y = (int)(t - im * (uint32_t)H);
  img = im;
}

template <int VEC>
__global__ void __launch_bounds__(256) dw_fwd_nhwc_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                          const float* __restrict__ bias, float* __restrict__ y,
                                                          uint32_t total, DwNhwc d) {
  using DV = DwVec<VEC>;
  using V = typename DV::T;
  const DwGeo& g = d.g;
  const int kk = g.ks * g.ks;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
    int64_t img;
    int oy, ox, j;
    dw_nhwc_pos(i, d, g.ow, g.oh, img, oy, ox, j);
    const int y0 = oy * g.s - g.p, x0 = ox * g.s - g.p;
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    for (int ky = 0; ky < g.ks; ++ky) {
      const int yy = y0 + ky;
      if ((unsigned)yy >= (unsigned)g.ih) continue;
      for (int kx = 0; kx < g.ks; ++kx) {
        const int xx = x0 + kx;
        if ((unsigned)xx >= (unsigned)g.iw) continue;
        const V v = *reinterpret_cast<const V*>(x + ((img * g.ih + yy) * g.iw + xx) * g.c + (int64_t)j * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = fmaf(DV::get(v, e), w[(j * VEC + e) * kk + ky * g.ks + kx], acc[e]);
      }
    }
    V out;
#pragma unroll
    for (int e = 0; e < VEC; ++e) DV::set(out, e, bias ? acc[e] + bias[j * VEC + e] : acc[e]);
    *reinterpret_cast<V*>(y + ((img * g.oh + oy) * g.ow + ox) * g.c + (int64_t)j * VEC) = out;
  }
}

template <int VEC>
__global__ void __launch_bounds__(256) dw_dgrad_nhwc_kernel(const float* __restrict__ gy, const float* __restrict__ w,
                                                            float* __restrict__ gx, uint32_t total, DwNhwc d) {
  using DV = DwVec<VEC>;
  using V = typename DV::T;
  const DwGeo& g = d.g;
  const int kk = g.ks * g.ks;
  for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < total; i += gridDim.x * 256u) {
    int64_t img;
    int yy, xx, j;
    dw_nhwc_pos(i, d, g.iw, g.ih, img, yy, xx, j);
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
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
        const V v = *reinterpret_cast<const V*>(gy + ((img * g.oh + oy) * g.ow + ox) * g.c + (int64_t)j * VEC);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = fmaf(DV::get(v, e), w[(j * VEC + e) * kk + ky * g.ks + kx], acc[e]);
      }
    }
    V out;
#pragma unroll
    for (int e = 0; e < VEC; ++e) DV::set(out, e, acc[e]);
    *reinterpret_cast<V*>(gx + ((img * g.ih + yy) * g.iw + xx) * g.c + (int64_t)j * VEC) = out;
  }
}

constexpr int kDwMaxKs = 11, kDwNhwcMaxSlices = 128;

struct DwNhwcW {
  int cb, rl, cblocks, slices;  // channel vectors per workgroup row, row lanes, channel blocks, pixel slices
  int64_t per_slice;            // output pixels per slice
};

// grid (cblocks, ks, slices): part[slice][ch][ky * ks + kx] = the slice's sum of gy[pixel][ch] x[tap (ky, kx)][ch]
template <int VEC>
__global__ void __launch_bounds__(256) dw_wgrad_nhwc_kernel(const float* __restrict__ x, const float* __restrict__ gy,
                                                            float* __restrict__ part, DwGeo g, int cv, DwNhwcW wp,
                                                            FastDiv d_ohw, FastDiv d_ow) {
  using DV = DwVec<VEC>;
  using V = typename DV::T;
  __shared__ float red[256 * VEC];
  const int jl = threadIdx.x % wp.cb, lane = threadIdx.x / wp.cb, j = blockIdx.x * wp.cb + jl;
  const int ky = blockIdx.y, sl = blockIdx.z;
  const bool on = lane < wp.rl && j < cv;
  float acc[kDwMaxKs][VEC];
#pragma unroll
  for (int kx = 0; kx < kDwMaxKs; ++kx)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[kx][e] = 0.f;
  if (on) {
    const int64_t total = (int64_t)g.n * g.oh * g.ow;
    const int64_t k0 = sl * wp.per_slice, k1 = min(total, k0 + wp.per_slice);
    const uint32_t ohw = (uint32_t)(g.oh * g.ow);
    for (int64_t k = k0 + lane; k < k1; k += wp.rl) {
      const uint32_t n = fdiv((uint32_t)k, d_ohw), r = (uint32_t)k - n * ohw;
      const uint32_t oy = fdiv(r, d_ow), ox = r - oy * (uint32_t)g.ow;
      const int yy = (int)oy * g.s - g.p + ky;
      if ((unsigned)yy >= (unsigned)g.ih) continue;
      const V gv = *reinterpret_cast<const V*>(gy + k * g.c + (int64_t)j * VEC);
      const float* xrow = x + (((int64_t)n * g.ih + yy) * g.iw) * g.c + (int64_t)j * VEC;
      const int x0 = (int)ox * g.s - g.p;
#pragma unroll
      for (int kx = 0; kx < kDwMaxKs; ++kx) {
        const int xx = x0 + kx;
        if (kx < g.ks && (unsigned)xx < (unsigned)g.iw) {
          const V xv = *reinterpret_cast<const V*>(xrow + (int64_t)xx * g.c);
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[kx][e] = fmaf(DV::get(gv, e), DV::get(xv, e), acc[kx][e]);
        }
      }
    }
  }
  // the row lanes' sums of each tap, added in lane order
  for (int kx = 0; kx < g.ks; ++kx) {
    float v[VEC];
#pragma unroll
    for (int t = 0; t < kDwMaxKs; ++t)
      if (t == kx)
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = acc[t][e];
#pragma unroll
    for (int e = 0; e < VEC; ++e) red[threadIdx.x * VEC + e] = v[e];
    __syncthreads();
    const int q = threadIdx.x;
    if (q < wp.cb * VEC) {
      const int ql = q / VEC, e = q - ql * VEC, ch = (blockIdx.x * wp.cb + ql) * VEC + e;
      if (ch < g.c) {
        float s = 0.f;
        for (int r = 0; r < wp.rl; ++r) s += red[(r * wp.cb + ql) * VEC + e];
        part[((int64_t)sl * g.c + ch) * g.ks * g.ks + ky * g.ks + kx] = s;
      }
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(256) dw_nhwc_sum_kernel(const SplitSum r) {
  if (r.vec4)
    split_sum_any<4>(r, blockIdx.x, gridDim.x);
  else
    split_sum_any<1>(r, blockIdx.x, gridDim.x);
}

static bool dw_nhwc_vec(const omt_conv_geo* g, std::initializer_list<const void*> ptrs) {
  if (g->ci % 4) return false;
  for (const void* p : ptrs)
    if (p && (uintptr_t)p % 16) return false;
  return true;
}
static DwNhwc dw_nhwc(const omt_conv_geo* g, bool vec, int64_t W, int64_t H) {
  DwNhwc d;
  d.g = DwGeo{(int)g->n, (int)g->ci, (int)g->ih, (int)g->iw, (int)g->oh, (int)g->ow, (int)g->ks, (int)g->stride,
              (int)g->pad};
  d.cv = (int)(vec ? g->ci / 4 : g->ci);
  d.d_cv = make_fastdiv((uint32_t)d.cv);
  d.d_w = make_fastdiv((uint32_t)W);
  d.d_h = make_fastdiv((uint32_t)H);
  return d;
}
static DwNhwcW dw_nhwc_wsplit(const omt_conv_geo* g, bool vec) {
  DwNhwcW wp;
  const int cv = (int)(vec ? g->ci / 4 : g->ci);
  wp.cb = cv < 64 ? cv : 64;
  wp.rl = 256 / wp.cb;
  wp.cblocks = (int)cdiv(cv, wp.cb);
  const int64_t total = g->n * g->oh * g->ow;
  int64_t want = cdiv(1024, (int64_t)wp.cblocks * g->ks);
  const int64_t by_rows = std::max<int64_t>(1, total / (8 * (int64_t)wp.rl));  // at least 8 pixels per thread
  want = std::min<int64_t>(std::min<int64_t>(want, by_rows), kDwNhwcMaxSlices);
  wp.per_slice = cdiv(total, want);
  wp.slices = (int)cdiv(total, wp.per_slice);
  return wp;
}
// pixels x channel vectors below 2^31 (32-bit thread indices whose grid-stride steps never wrap)
static bool dw_nhwc_ok(const omt_conv_geo* g) {
  return dw_ok(g) && g->n * g->ih * g->iw * g->ci < ((int64_t)1 << 31) &&
         g->n * g->oh * g->ow * g->ci < ((int64_t)1 << 31);
}

#define OMT_DW_NHWC(K, vec, total, s, ...)                                                       \
  do {                                                                                           \
    if (vec)                                                                                     \
      hipLaunchKernelGGL(K<4>, dim3(grid1d(total, 256)), dim3(256), 0, s, __VA_ARGS__);          \
    else                                                                                         \
      hipLaunchKernelGGL(K<1>, dim3(grid1d(total, 256)), dim3(256), 0, s, __VA_ARGS__);          \
  } while (0)


}  // namespace omt

using namespace omt;

OMT_EXPORT int omt_dw_fwd(const omt_conv_geo* g, const float* x, const float* w, const float* bias,
                          const float* bn_mean, const float* bn_var, const float* bn_gamma, const float* bn_beta,
                          float bn_eps, float* y, void* stream) {
  if (!g || !x || !w || !y) return fail(OMT_INVALID, "omt_dw_fwd: null pointer");
  if (!dw_ok(g)) return fail(OMT_UNSUPPORTED, "omt_dw_fwd: geometry not covered");
  const bool bn = bn_mean || bn_var || bn_gamma || bn_beta;
  if (bn && !(bn_mean && bn_var && bn_gamma && bn_beta)) return fail(OMT_INVALID, "omt_dw_fwd: incomplete BN loader");
  if (dw_s1(g))
    return launch_dw_s1<false>(g, x, w, bias, bn ? bn_mean : nullptr, bn_var, bn_gamma, bn_beta, bn_eps, y,
                               stream_of(stream));
  const int64_t total = g->n * g->co * g->oh * g->ow;
  hipLaunchKernelGGL(dw_fwd_kernel, dim3(grid1d(total, 256)), dim3(256), 0, stream_of(stream), x, w, bias,
                     bn ? bn_mean : nullptr, bn_var, bn_gamma, bn_beta, bn_eps, y, total, dgeo(g));
  return launch_check("dw_fwd_kernel");
}

OMT_EXPORT int omt_dw_dgrad(const omt_conv_geo* g, const float* gy, const float* w, float* gx, void* stream) {
  if (!g || !gy || !w || !gx) return fail(OMT_INVALID, "omt_dw_dgrad: null pointer");
  if (!dw_ok(g)) return fail(OMT_UNSUPPORTED, "omt_dw_dgrad: geometry not covered");
  if (dw_s1(g))
    return launch_dw_s1<true>(g, gy, w, nullptr, nullptr, nullptr, nullptr, nullptr, 0.f, gx, stream_of(stream));
  const int64_t total = g->n * g->ci * g->ih * g->iw;
  hipLaunchKernelGGL(dw_dgrad_kernel, dim3(grid1d(total, 256)), dim3(256), 0, stream_of(stream), gy, w, gx, total,
                     dgeo(g));
  return launch_check("dw_dgrad_kernel");
}

OMT_EXPORT size_t omt_dw_wgrad_workspace(const omt_conv_geo* g) {
  if (!g || !dw_ok(g)) return 0;
  if (dw_s1(g) && dw_reg_ok(g)) return dw_wreg_workspace(g);
  return (size_t)((dw_s1_wgrad(g) ? dw_s1_groups(g) : dw_slices(g)) * g->ci * g->ks * g->ks) * sizeof(float);
}

OMT_EXPORT int omt_dw_wgrad(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (!g || !x || !gy || !gw) return fail(OMT_INVALID, "omt_dw_wgrad: null pointer");
  if (!dw_ok(g)) return fail(OMT_UNSUPPORTED, "omt_dw_wgrad: geometry not covered");
  const size_t need = omt_dw_wgrad_workspace(g);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(OMT_INVALID, "omt_dw_wgrad: workspace of %zu bytes needed", need);
  hipStream_t s = stream_of(stream);
  if (dw_s1(g) && dw_reg_ok(g)) {
    const DwRegW d = dw_wreg(g);
    const int ks = (int)g->ks;
    const int N = (int)g->n, C = (int)g->ci, H = (int)g->ih, W = (int)g->iw;
    float* part = (float*)workspace;
    const dim3 grid((unsigned)g->ci, (unsigned)d.slices);
#define OMT_DW_WR(KS_, RB_, NT_) \
  hipLaunchKernelGGL((dw_wgrad_reg_kernel<KS_, RB_, NT_>), grid, dim3(NT_), 0, s, x, gy, gw, part, N, C, H, W, d)
#define OMT_DW_WR_KS(KS_)                                   \
  if (d.nt == 256) OMT_DW_WR(KS_, (KS_ == 7 ? 2 : 4), 256); \
  else if (d.rb == 2) OMT_DW_WR(KS_, 2, 1024);              \
  else OMT_DW_WR(KS_, (KS_ == 7 ? 2 : 4), 1024)
    if (ks == 3) {
      OMT_DW_WR_KS(3);
    } else if (ks == 5) {
      OMT_DW_WR_KS(5);
    } else {
      OMT_DW_WR_KS(7);
    }
#undef OMT_DW_WR_KS
#undef OMT_DW_WR
    if (int st = launch_check("dw_wgrad_reg_kernel")) return st;
    if (d.slices == 1) return OMT_OK;
    const int n = (int)(g->ci * ks * ks);
    hipLaunchKernelGGL(dw_wgrad_reduce_kernel, dim3(grid1d(n, 256, 4096)), dim3(256), 0, s, (const float*)part, gw,
                       n, d.slices);
    return launch_check("dw_wgrad_reduce_kernel");
  }
  if (dw_s1_wgrad(g)) {
    const int nt = dw_threads(g), ks = (int)g->ks;
    const DwTiling t = dw_tiling((int)g->ih, (int)g->iw, ks, nt);
    const DwUnits wu = dw_units(g);
    const int64_t slices = cdiv(wu.units, wu.group);
    const dim3 grid((unsigned)g->ci, (unsigned)slices);
    const size_t lds = (size_t)2 * wu.buf * sizeof(float);
    const int C = (int)g->ci, H = (int)g->ih, W = (int)g->iw;
    float* part = (float*)workspace;
#define OMT_DW_WG(KS_, NT_) \
  hipLaunchKernelGGL((dw_wgrad_s1_kernel<KS_, NT_>), grid, dim3(NT_), lds, s, x, gy, part, C, H, W, t, wu)
    if (nt == 64) {
      if (ks == 3) OMT_DW_WG(3, 64); else if (ks == 5) OMT_DW_WG(5, 64); else OMT_DW_WG(7, 64);
    } else {
      if (ks == 3) OMT_DW_WG(3, 256); else if (ks == 5) OMT_DW_WG(5, 256); else OMT_DW_WG(7, 256);
    }
#undef OMT_DW_WG
    if (int st = launch_check("dw_wgrad_s1_kernel")) return st;
    const int n = (int)(g->ci * ks * ks);
    hipLaunchKernelGGL(dw_wgrad_reduce_kernel, dim3(grid1d(n, 256, 4096)), dim3(256), 0, s, (const float*)part, gw,
                       n, (int)slices);
    return launch_check("dw_wgrad_reduce_kernel");
  }
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

OMT_EXPORT int omt_dw_fwd_nhwc(const omt_conv_geo* g, const float* x, const float* w, const float* bias, float* y,
                               void* stream) {
  if (!g || !x || !w || !y) return fail(OMT_INVALID, "omt_dw_fwd_nhwc: null pointer");
  if (!dw_nhwc_ok(g)) return fail(OMT_UNSUPPORTED, "omt_dw_fwd_nhwc: geometry not covered");
  const bool vec = dw_nhwc_vec(g, {x, y});
  const DwNhwc d = dw_nhwc(g, vec, g->ow, g->oh);
  const int64_t total = g->n * g->oh * g->ow * d.cv;
  OMT_DW_NHWC(dw_fwd_nhwc_kernel, vec, total, stream_of(stream), x, w, bias, y, (uint32_t)total, d);
  return launch_check("dw_fwd_nhwc_kernel");
}

OMT_EXPORT int omt_dw_dgrad_nhwc(const omt_conv_geo* g, const float* gy, const float* w, float* gx, void* stream) {
  if (!g || !gy || !w || !gx) return fail(OMT_INVALID, "omt_dw_dgrad_nhwc: null pointer");
  if (!dw_nhwc_ok(g)) return fail(OMT_UNSUPPORTED, "omt_dw_dgrad_nhwc: geometry not covered");
  const bool vec = dw_nhwc_vec(g, {gy, gx});
  const DwNhwc d = dw_nhwc(g, vec, g->iw, g->ih);
  const int64_t total = g->n * g->ih * g->iw * d.cv;
  OMT_DW_NHWC(dw_dgrad_nhwc_kernel, vec, total, stream_of(stream), gy, w, gx, (uint32_t)total, d);
  return launch_check("dw_dgrad_nhwc_kernel");
}

// the slices' partial filter gradients [slices][c][ks][ks] (the float4 split of the aligned case, which has the most)
OMT_EXPORT size_t omt_dw_wgrad_nhwc_workspace(const omt_conv_geo* g) {
  if (!g || !dw_nhwc_ok(g)) return 0;
  const int sl = std::max(dw_nhwc_wsplit(g, g->ci % 4 == 0).slices, dw_nhwc_wsplit(g, false).slices);
  return (size_t)(sl * g->ci * g->ks * g->ks) * sizeof(float);
}

OMT_EXPORT int omt_dw_wgrad_nhwc(const omt_conv_geo* g, const float* x, const float* gy, float* gw, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  if (!g || !x || !gy || !gw) return fail(OMT_INVALID, "omt_dw_wgrad_nhwc: null pointer");
  if (!dw_nhwc_ok(g)) return fail(OMT_UNSUPPORTED, "omt_dw_wgrad_nhwc: geometry not covered");
  const size_t need = omt_dw_wgrad_nhwc_workspace(g);
  if (!workspace || workspace_bytes < need)
    return fail(OMT_INVALID, "omt_dw_wgrad_nhwc: workspace of %zu bytes needed", need);
  hipStream_t s = stream_of(stream);
  const bool vec = dw_nhwc_vec(g, {x, gy});
  const DwNhwcW wp = dw_nhwc_wsplit(g, vec);
  const int cv = (int)(vec ? g->ci / 4 : g->ci);
  float* part = (float*)workspace;
  const dim3 grid((unsigned)wp.cblocks, (unsigned)g->ks, (unsigned)wp.slices);
  const FastDiv d_ohw = make_fastdiv((uint32_t)(g->oh * g->ow)), d_ow = make_fastdiv((uint32_t)g->ow);
  if (vec)
    hipLaunchKernelGGL(dw_wgrad_nhwc_kernel<4>, grid, dim3(256), 0, s, x, gy, part, dgeo(g), cv, wp, d_ohw, d_ow);
  else
    hipLaunchKernelGGL(dw_wgrad_nhwc_kernel<1>, grid, dim3(256), 0, s, x, gy, part, dgeo(g), cv, wp, d_ohw, d_ow);
  if (int st = launch_check("dw_wgrad_nhwc_kernel")) return st;
  const SplitSum r = split_sum_of(part, gw, g->ci * g->ks * g->ks, wp.slices);
  hipLaunchKernelGGL(dw_nhwc_sum_kernel, dim3((unsigned)r.blocks), dim3(256), 0, s, r);
  return launch_check("dw_nhwc_sum_kernel");
}
