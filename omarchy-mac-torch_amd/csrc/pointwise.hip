// The other device ops of the training configurations (outside the convolution path): pointwise activations and their
// gradients, residual add, the squeeze-excite channel scale, plane and row reductions, log-softmax and the NLL loss.
// Reference counterparts: the general elementwise kernel and its op table (csrc/elementwise.cpp:79-112, 702-817;
// csrc/kernels/ew.wgsl), softmax / log-softmax and the NLL loss (csrc/reduce.cpp:128-202; csrc/kernels/softmax.wgsl,
// softmax_bwd.wgsl, nll_fwd.wgsl, nll_bwd.wgsl).
//
// All of them are HBM- or latency-bound. Pointwise ops stream float4 vectors (16-byte aligned operands) through a
// grid-stride loop; the reductions give each output one wave (DPP sums, omt_internal.h) or, for the NLL loss, one
// workgroup summing in a fixed order, so results do not depend on scheduling.
#include <type_traits>

#include "omt_internal.h"

namespace omt {


template <int OP>
__device__ __forceinline__ float pw_apply(float a, float b, float alpha) {
  if constexpr (OP == OMT_PW_ADD) return a + alpha * b;
  if constexpr (OP == OMT_PW_MUL) return a * b;
  if constexpr (OP == OMT_PW_RELU) return a <= 0.f ? 0.f : a;  // NaN compares false and propagates
  if constexpr (OP == OMT_PW_THRESHOLD_BWD) return b <= alpha ? 0.f : a;
  if constexpr (OP == OMT_PW_HARDSWISH) return hardswish_f(a);
  if constexpr (OP == OMT_PW_HARDSWISH_BWD) return hardswish_grad(a, b);
  if constexpr (OP == OMT_PW_HARDSIGMOID) return hardsigmoid_f(a);
  if constexpr (OP == OMT_PW_HARDSIGMOID_BWD) return hardsigmoid_grad(a, b);
  if constexpr (OP == OMT_PW_SCALE) return a * alpha;
  if constexpr (OP == OMT_PW_ADD_SCALAR) return a + alpha;
  return alpha;  // OMT_PW_FILL
}

// out[i] = op(a[i], b[i]) over n elements; VEC 4: every operand 16-byte aligned (the n % 4 tail element by element).
template <int OP, int VEC>
__global__ void __launch_bounds__(256) pointwise_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                        float* __restrict__ out, int64_t n, float alpha) {
  constexpr bool UNARY = OP == OMT_PW_RELU || OP == OMT_PW_HARDSWISH || OP == OMT_PW_HARDSIGMOID ||
                         OP == OMT_PW_SCALE || OP == OMT_PW_ADD_SCALAR;
  constexpr bool NULLARY = OP == OMT_PW_FILL;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x, t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if constexpr (VEC == 4) {
    const int64_t n4 = n >> 2;
    for (int64_t i = t0; i < n4; i += stride) {
      float4 va = NULLARY ? make_float4(0.f, 0.f, 0.f, 0.f) : reinterpret_cast<const float4*>(a)[i];
      float4 vb = (UNARY || NULLARY) ? va : reinterpret_cast<const float4*>(b)[i];
      float4 r;
      r.x = pw_apply<OP>(va.x, vb.x, alpha);
      r.y = pw_apply<OP>(va.y, vb.y, alpha);
      r.z = pw_apply<OP>(va.z, vb.z, alpha);
      r.w = pw_apply<OP>(va.w, vb.w, alpha);
      reinterpret_cast<float4*>(out)[i] = r;
    }
    for (int64_t i = (n4 << 2) + t0; i < n; i += stride)
      out[i] = pw_apply<OP>(NULLARY ? 0.f : a[i], (UNARY || NULLARY) ? 0.f : b[i], alpha);
  } else {
    for (int64_t i = t0; i < n; i += stride)
      out[i] = pw_apply<OP>(NULLARY ? 0.f : a[i], (UNARY || NULLARY) ? 0.f : b[i], alpha);
  }
}

// y[p][i] = x[p][i] * s[p] (squeeze-excite), or with x == nullptr y[p][i] = s[p] * scale (a plane broadcast: the
// gradient of a plane mean). One workgroup row of the grid per group of planes; VEC 4 when hw % 4 == 0 and aligned.
template <int VEC, bool SCALE_X>
__global__ void __launch_bounds__(256) plane_scale_kernel(const float* __restrict__ x, const float* __restrict__ s,
                                                          float* __restrict__ y, int64_t planes, int hw, float scale,
                                                          FastDiv dv) {
  const int hv = hw / VEC;
  const int64_t total = planes * hv;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t p = total < ((int64_t)1 << 32) ? (int64_t)fdiv((uint32_t)i, dv) : i / hv;
    const float m = SCALE_X ? s[p] : s[p] * scale;
    if constexpr (VEC == 4) {
      float4 v = SCALE_X ? reinterpret_cast<const float4*>(x)[i] : make_float4(1.f, 1.f, 1.f, 1.f);
      reinterpret_cast<float4*>(y)[i] = make_float4(v.x * m, v.y * m, v.z * m, v.w * m);
    } else {
      y[i] = SCALE_X ? x[i] * m : m;
    }
  }
}

// A value the compiler must materialize as it stands: a product passed through it is rounded to float before any
// later addition (no multiply-add contraction across it), as when a separate kernel stores it.
__device__ __forceinline__ float rounded(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// The gradient reaching a squeeze-excite block's input through its two uses: y[p][i] = g[p][i] * s[p] + v[p] * scale
// (the scale's gradient through the gate, plus the plane mean's broadcast gradient), the two products rounded and then
// added as the separate multiply, broadcast and add would (no fused multiply-add).
template <int VEC>
__global__ void __launch_bounds__(256) se_gate_bwd_kernel(const float* __restrict__ g, const float* __restrict__ s,
                                                          const float* __restrict__ v, float* __restrict__ y,
                                                          int64_t planes, int hw, float scale, FastDiv dv) {
  const int hv = hw / VEC;
  const int64_t total = planes * hv;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t p = total < ((int64_t)1 << 32) ? (int64_t)fdiv((uint32_t)i, dv) : i / hv;
    const float m = s[p], a = rounded(v[p] * scale);
    if constexpr (VEC == 4) {
      const float4 t = reinterpret_cast<const float4*>(g)[i];
      reinterpret_cast<float4*>(y)[i] =
          make_float4(rounded(t.x * m) + a, rounded(t.y * m) + a, rounded(t.z * m) + a, rounded(t.w * m) + a);
    } else {
      y[i] = rounded(g[i] * m) + a;
    }
  }
}

// y[p] = scale * sum_i x[p][i], one wave per plane, four planes per workgroup. Each lane sums a strided part of the
// plane in order, then the wave adds the 64 lane sums with DPP (a fixed order). DOT: the terms are x[p][i] * b[p][i]
// (rounded products, as a separate multiply would store them), summed in the same order.
template <bool DOT = false>
__global__ void __launch_bounds__(256) plane_sum_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                        int64_t planes, int hw, float scale,
                                                        const float* __restrict__ b = nullptr) {
  const int64_t plane = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (plane >= planes) return;  // whole waves leave together: wave_sum below runs with all 64 lanes
  const int lane = threadIdx.x & 63;
  const float* xp = x + plane * hw;
  const float* bp = DOT ? b + plane * hw : nullptr;
  float acc = 0.f;
  for (int e0 = lane; e0 < hw; e0 += 256) {  // four loads in flight, added in the same order as one at a time
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = e0 + 64 * j < hw ? xp[e0 + 64 * j] : 0.f;
      if (DOT) v[j] = rounded(v[j] * (e0 + 64 * j < hw ? bp[e0 + 64 * j] : 0.f));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (e0 + 64 * j < hw) acc += v[j];
  }
  acc = wave_sum(acc);
  if (lane == 0) y[plane] = acc * scale;
}

// Large planes (kPlaneWG elements and more): one workgroup per plane. Each thread sums its float4 vectors (stride
// 256, four loads in flight), then the wave sums (DPP) are added in wave order.
constexpr int kPlaneWG = 1024;
template <int VEC, bool DOT = false>
__global__ void __launch_bounds__(256) plane_sum_wg_kernel(const float* __restrict__ x, float* __restrict__ y, int hw,
                                                           float scale, const float* __restrict__ b = nullptr) {
  using V = typename std::conditional<VEC == 4, float4, float>::type;
  __shared__ float red[4];
  const int64_t plane = blockIdx.x;
  const V* xp = reinterpret_cast<const V*>(x + plane * hw);
  const V* bp = DOT ? reinterpret_cast<const V*>(b + plane * hw) : nullptr;
  const int nv = hw / VEC;
  float acc = 0.f;
  for (int e0 = threadIdx.x; e0 < nv; e0 += 1024) {
    V v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (e0 + 256 * j < nv) {
        v[j] = xp[e0 + 256 * j];
        if constexpr (DOT) {
          const V w = bp[e0 + 256 * j];
          if constexpr (VEC == 4)
            v[j] = make_float4(rounded(v[j].x * w.x), rounded(v[j].y * w.y), rounded(v[j].z * w.z),
                               rounded(v[j].w * w.w));
          else
            v[j] = rounded(v[j] * w);
        }
      }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (e0 + 256 * j < nv) {
        if constexpr (VEC == 4) acc += (v[j].x + v[j].y) + (v[j].z + v[j].w);
        else acc += v[j];
      }
  }
  acc = wave_sum(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) y[plane] = ((red[0] + red[1]) + (red[2] + red[3])) * scale;
}

// Maximum over the 64 lanes of a wave, in every lane (the DPP pattern of wave_sum). All 64 lanes must be active.
__device__ __forceinline__ float dpp_max(float v, int moved) { return fmaxf(v, __builtin_bit_cast(float, moved)); }
__device__ __forceinline__ float wave_max(float v) {
  int b = __builtin_bit_cast(int, v);
  v = dpp_max(v, __builtin_amdgcn_update_dpp(0, b, 0xB1, 0xF, 0xF, false));
  b = __builtin_bit_cast(int, v);
  v = dpp_max(v, __builtin_amdgcn_update_dpp(0, b, 0x4E, 0xF, 0xF, false));
  b = __builtin_bit_cast(int, v);
  v = dpp_max(v, __builtin_amdgcn_update_dpp(0, b, 0x141, 0xF, 0xF, false));
  b = __builtin_bit_cast(int, v);
  v = dpp_max(v, __builtin_amdgcn_update_dpp(0, b, 0x140, 0xF, 0xF, false));
  b = __builtin_bit_cast(int, v);
  return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))),
               fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48))));
}

// y[r][j] = x[r][j] - (m_r + log sum_j exp(x[r][j] - m_r)), m_r = max_j x[r][j]; one wave per row.
__global__ void __launch_bounds__(256) log_softmax_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                          int64_t rows, int cols) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const float* xr = x + r * cols;
  float m = -INFINITY;
  for (int j = lane; j < cols; j += 64) m = fmaxf(m, xr[j]);
  m = wave_max(m);
  // a NaN in the row (which fmaxf skips) still reaches every output through the sum of exponentials
  float s = 0.f;
  for (int j = lane; j < cols; j += 64) s += expf(xr[j] - m);
  s = wave_sum(s);
  const float lse = m + logf(s);
  float* yr = y + r * cols;
  for (int j = lane; j < cols; j += 64) yr[j] = xr[j] - lse;
}

// gx[r][j] = g[r][j] - exp(y[r][j]) * sum_j g[r][j] (y the log-softmax output); one wave per row.
__global__ void __launch_bounds__(256) log_softmax_bwd_kernel(const float* __restrict__ g, const float* __restrict__ y,
                                                              float* __restrict__ gx, int64_t rows, int cols) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const float *gr = g + r * cols, *yr = y + r * cols;
  float s = 0.f;
  for (int j = lane; j < cols; j += 64) s += gr[j];
  s = wave_sum(s);
  float* o = gx + r * cols;
  for (int j = lane; j < cols; j += 64) o[j] = gr[j] - expf(yr[j]) * s;
}

// The same two maps for rows of at most 64 R columns: a lane loads its R elements of the row at once (all loads in
// flight together, where the loops above wait on the row once per pass) and every pass reads them from registers.
// Each lane visits its columns in the loops' order, so the results are identical.
template <int R>
__global__ void __launch_bounds__(256) log_softmax_reg_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                              int64_t rows, int cols) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const float* xr = x + r * cols;
  float v[R];
#pragma unroll
  for (int i = 0; i < R; ++i) v[i] = lane + 64 * i < cols ? xr[lane + 64 * i] : -INFINITY;
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < R; ++i) m = fmaxf(m, v[i]);
  m = wave_max(m);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < R; ++i)
    if (lane + 64 * i < cols) s += expf(v[i] - m);
  s = wave_sum(s);
  const float lse = m + logf(s);
  float* yr = y + r * cols;
#pragma unroll
  for (int i = 0; i < R; ++i)
    if (lane + 64 * i < cols) yr[lane + 64 * i] = v[i] - lse;
}
template <int R>
__global__ void __launch_bounds__(256) log_softmax_bwd_reg_kernel(const float* __restrict__ g,
                                                                  const float* __restrict__ y, float* __restrict__ gx,
                                                                  int64_t rows, int cols) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int lane = threadIdx.x & 63;
  const float *gr = g + r * cols, *yr = y + r * cols;
  float gv[R], yv[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const bool in = lane + 64 * i < cols;
    gv[i] = in ? gr[lane + 64 * i] : 0.f;
    yv[i] = in ? yr[lane + 64 * i] : 0.f;
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < R; ++i)
    if (lane + 64 * i < cols) s += gv[i];
  s = wave_sum(s);
  float* o = gx + r * cols;
#pragma unroll
  for (int i = 0; i < R; ++i)
    if (lane + 64 * i < cols) o[lane + 64 * i] = gv[i] - expf(yv[i]) * s;
}

// NLL loss forward over log-probabilities logp[rows][cols] and int64 targets. reduction 0 (none): out[r] = -w[t_r]
// logp[r][t_r] (0 for ignore_index); 1 (mean): sum / total weight; 2 (sum). One workgroup: thread t takes rows t,
// t + 256, ... in order, then a fixed tree over the threads' partial sums.
__global__ void __launch_bounds__(256) nll_fwd_kernel(const float* __restrict__ logp, const int64_t* __restrict__ tgt,
                                                      const float* __restrict__ weight, int64_t rows, int cols,
                                                      int64_t ignore, int reduction, float* __restrict__ out,
                                                      float* __restrict__ total_weight) {
  __shared__ float sl[256], sw[256];
  float l = 0.f, wsum = 0.f;
  for (int64_t r = threadIdx.x; r < rows; r += 256) {
    const int64_t t = tgt[r];
    float lr = 0.f, wr = 0.f;
    if (t != ignore && t >= 0 && t < cols) {
      wr = weight ? weight[t] : 1.f;
      lr = -wr * logp[r * cols + t];
    }
    if (reduction == 0) out[r] = lr;
    l += lr;
    wsum += wr;
  }
  sl[threadIdx.x] = l;
  sw[threadIdx.x] = wsum;
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if ((int)threadIdx.x < h) {
      sl[threadIdx.x] += sl[threadIdx.x + h];
      sw[threadIdx.x] += sw[threadIdx.x + h];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    if (reduction == 1) out[0] = sl[0] / sw[0];
    if (reduction == 2) out[0] = sl[0];
    *total_weight = reduction == 0 ? 0.f : sw[0];
  }
}

// NLL loss backward: gx[r][j] = j == t_r ? -w[t_r] * g' : 0 with g' = g[0] / total_weight (mean), g[0] (sum) or g[r]
// (none), and 0 on rows whose target is ignore_index.
__global__ void __launch_bounds__(256) nll_bwd_kernel(const float* __restrict__ g, const int64_t* __restrict__ tgt,
                                                      const float* __restrict__ weight, int64_t rows, int cols,
                                                      int64_t ignore, int reduction,
                                                      const float* __restrict__ total_weight, float* __restrict__ gx) {
  const int64_t n = rows * cols, stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t r = i / cols, j = i - r * cols;
    const int64_t t = tgt[r];
    float v = 0.f;
    if (j == t && t != ignore) {
      const float w = weight ? weight[t] : 1.f;
      const float gr = reduction == 0 ? g[r] : (reduction == 1 ? g[0] / *total_weight : g[0]);
      v = -w * gr;
    }
    gx[i] = v;
  }
}

// t += value over a list of small tensors (step counts, batch counters), one wave per tensor; the table travels in
// the kernel arguments, so a captured graph replays it unchanged.
constexpr int kForeachMax = 64;
struct ForeachTable {
  void* ptr[kForeachMax];
  int64_t numel[kForeachMax];
};
template <class T>
__global__ void __launch_bounds__(64) foreach_add_kernel(ForeachTable tab, T value) {
  T* p = static_cast<T*>(tab.ptr[blockIdx.x]);
  const int64_t n = tab.numel[blockIdx.x];
  for (int64_t i = threadIdx.x; i < n; i += 64) p[i] += value;
}


// ---- operands in different memory orders (NCHW and channels-last NHWC) ----------------------------------------
// out = op(a, b) over [n][c][hw] tensors whose memory orders differ (each flag: 1 = NHWC); one thread per output
// element, in the output's order, reading the operand stored the other way at the transposed index.
template <int OP>
__global__ void __launch_bounds__(256) pointwise_layouts_kernel(const float* __restrict__ a, int a_nhwc,
                                                                const float* __restrict__ b, int b_nhwc,
                                                                float* __restrict__ out, int out_nhwc, int64_t total,
                                                                int64_t c, int64_t hw, float alpha) {
  constexpr bool UNARY = OP == OMT_PW_RELU || OP == OMT_PW_HARDSWISH || OP == OMT_PW_HARDSIGMOID ||
                         OP == OMT_PW_SCALE || OP == OMT_PW_ADD_SCALAR;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    int64_t img, ch, p;
    if (out_nhwc) {
      const int64_t pix = i / c;
      ch = i - pix * c;
      img = pix / hw;
      p = pix - img * hw;
    } else {
      const int64_t pl = i / hw;
      p = i - pl * hw;
      img = pl / c;
      ch = pl - img * c;
    }
    const int64_t nchw = (img * c + ch) * hw + p, nhwc = (img * hw + p) * c + ch;
    const float va = a[a_nhwc ? nhwc : nchw];
    const float vb = UNARY ? 0.f : b[b_nhwc ? nhwc : nchw];
    out[i] = pw_apply<OP>(va, vb, alpha);
  }
}

// y[img][p][ch] = x[img][p][ch] * s[img][ch] over channels-last planes; VEC channels per thread.
template <int VEC>
__global__ void __launch_bounds__(256) channel_scale_nhwc_kernel(const float* __restrict__ x,
                                                                 const float* __restrict__ s, float* __restrict__ y,
                                                                 int64_t total_v, int64_t cv, int64_t hwcv) {
  using V = typename std::conditional<VEC == 4, float4, float>::type;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total_v; i += (int64_t)gridDim.x * 256) {
    const int64_t img = i / hwcv, j = i % cv;
    const V v = reinterpret_cast<const V*>(x)[i];
    const V f = reinterpret_cast<const V*>(s + img * cv * VEC)[j];
    if constexpr (VEC == 4)
      reinterpret_cast<V*>(y)[i] = make_float4(v.x * f.x, v.y * f.y, v.z * f.z, v.w * f.w);
    else
      y[i] = v * f;
  }
}

// omt_se_gate_bwd over channels-last planes: y[img][p][ch] = g[img][p][ch] * s[img][ch] + v[img][ch] * scale.
template <int VEC>
__global__ void __launch_bounds__(256) se_gate_bwd_nhwc_kernel(const float* __restrict__ g, const float* __restrict__ s,
                                                               const float* __restrict__ v, float* __restrict__ y,
                                                               int64_t total_v, int64_t cv, int64_t hwcv, float scale) {
  using V = typename std::conditional<VEC == 4, float4, float>::type;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total_v; i += (int64_t)gridDim.x * 256) {
    const int64_t img = i / hwcv, j = i % cv;
    const V t = reinterpret_cast<const V*>(g)[i];
    const V m = reinterpret_cast<const V*>(s + img * cv * VEC)[j];
    const V w = reinterpret_cast<const V*>(v + img * cv * VEC)[j];
    if constexpr (VEC == 4)
      reinterpret_cast<V*>(y)[i] = make_float4(
          rounded(t.x * m.x) + rounded(w.x * scale), rounded(t.y * m.y) + rounded(w.y * scale),
          rounded(t.z * m.z) + rounded(w.z * scale), rounded(t.w * m.w) + rounded(w.w * scale));
    else
      y[i] = rounded(t * m) + rounded(w * scale);
  }
}

// y[img][ch] = scale * sum over the hw positions of x [n][hw][c] (channels-last planes). Workgroup (channel block,
// image): thread t owns channel j = block * cb + t % cb and sums positions t / cb, + rl, ... (four loads in flight),
// then the row lanes' sums are added in lane order: a fixed order.
__global__ void __launch_bounds__(256) plane_sum_nhwc_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                             int c, int hw, int cb, float scale) {
  __shared__ float red[256];
  const int rl = 256 / cb, jl = threadIdx.x % cb, lane = threadIdx.x / cb, j = blockIdx.x * cb + jl;
  const int64_t img = blockIdx.y;
  float acc = 0.f;
  if (lane < rl && j < c) {
    const float* xp = x + img * hw * (int64_t)c + j;
    for (int p0 = lane; p0 < hw; p0 += 4 * rl) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = p0 + u * rl < hw ? xp[(int64_t)(p0 + u * rl) * c] : 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (p0 + u * rl < hw) acc += v[u];
    }
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  if ((int)threadIdx.x < cb && j < c) {
    float s = 0.f;
    for (int r = 0; r < rl; ++r) s += red[r * cb + jl];
    y[img * c + j] = s * scale;
  }
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <int OP>
static void launch_pw(int64_t n, const float* a, const float* b, float alpha, float* out, hipStream_t s) {
  const bool v4 = al16(out) && (!a || al16(a)) && (!b || al16(b));
  const unsigned grid = grid1d(v4 ? cdiv(n, 4) : n, 256, 8192);
  if (v4)
    hipLaunchKernelGGL((pointwise_kernel<OP, 4>), dim3(grid), dim3(256), 0, s, a, b, out, n, alpha);
  else
    hipLaunchKernelGGL((pointwise_kernel<OP, 1>), dim3(grid), dim3(256), 0, s, a, b, out, n, alpha);
}

}  // namespace omt

using namespace omt;

OMT_EXPORT int omt_pointwise(int op, int64_t n, const float* a, const float* b, float alpha, float* out,
                             void* stream) {
  if (n < 0) return fail(OMT_INVALID, "omt_pointwise: n %lld", (long long)n);
  if (n == 0) return OMT_OK;
  const bool binary = op == OMT_PW_ADD || op == OMT_PW_MUL || op == OMT_PW_THRESHOLD_BWD ||
                      op == OMT_PW_HARDSWISH_BWD || op == OMT_PW_HARDSIGMOID_BWD;
  if (!out || (op != OMT_PW_FILL && !a) || (binary && !b)) return fail(OMT_INVALID, "omt_pointwise: null pointer");
  hipStream_t s = stream_of(stream);
  switch (op) {
    case OMT_PW_ADD: launch_pw<OMT_PW_ADD>(n, a, b, alpha, out, s); break;
    case OMT_PW_MUL: launch_pw<OMT_PW_MUL>(n, a, b, alpha, out, s); break;
    case OMT_PW_RELU: launch_pw<OMT_PW_RELU>(n, a, nullptr, alpha, out, s); break;
    case OMT_PW_THRESHOLD_BWD: launch_pw<OMT_PW_THRESHOLD_BWD>(n, a, b, alpha, out, s); break;
    case OMT_PW_HARDSWISH: launch_pw<OMT_PW_HARDSWISH>(n, a, nullptr, alpha, out, s); break;
    case OMT_PW_HARDSWISH_BWD: launch_pw<OMT_PW_HARDSWISH_BWD>(n, a, b, alpha, out, s); break;
    case OMT_PW_HARDSIGMOID: launch_pw<OMT_PW_HARDSIGMOID>(n, a, nullptr, alpha, out, s); break;
    case OMT_PW_HARDSIGMOID_BWD: launch_pw<OMT_PW_HARDSIGMOID_BWD>(n, a, b, alpha, out, s); break;
    case OMT_PW_SCALE: launch_pw<OMT_PW_SCALE>(n, a, nullptr, alpha, out, s); break;
    case OMT_PW_FILL: launch_pw<OMT_PW_FILL>(n, nullptr, nullptr, alpha, out, s); break;
    case OMT_PW_ADD_SCALAR: launch_pw<OMT_PW_ADD_SCALAR>(n, a, nullptr, alpha, out, s); break;
    default: return fail(OMT_INVALID, "omt_pointwise: op %d", op);
  }
  return launch_check("pointwise_kernel");
}

OMT_EXPORT int omt_foreach_add_scalar(int count, void* const* ptrs, const int64_t* numels, int dtype, int64_t ivalue,
                                      float fvalue, void* stream) {
  if (count < 0 || (count > 0 && (!ptrs || !numels))) return fail(OMT_INVALID, "omt_foreach_add_scalar: arguments");
  if (dtype != OMT_DT_F32 && dtype != OMT_DT_I64) return fail(OMT_INVALID, "omt_foreach_add_scalar: dtype %d", dtype);
  for (int i = 0; i < count; ++i)
    if (numels[i] < 0 || (numels[i] > 0 && !ptrs[i]) || numels[i] > OMT_FOREACH_MAX_NUMEL)
      return fail(OMT_INVALID, "omt_foreach_add_scalar: tensor %d (numel %lld)", i, (long long)numels[i]);
  hipStream_t s = stream_of(stream);
  for (int i0 = 0; i0 < count; i0 += kForeachMax) {
    ForeachTable tab{};
    int k = 0;
    for (int i = i0; i < count && i < i0 + kForeachMax; ++i) {
      if (numels[i] == 0) continue;
      tab.ptr[k] = ptrs[i];
      tab.numel[k++] = numels[i];
    }
    if (k == 0) continue;
    if (dtype == OMT_DT_F32)
      hipLaunchKernelGGL((foreach_add_kernel<float>), dim3(k), dim3(64), 0, s, tab, fvalue);
    else
      hipLaunchKernelGGL((foreach_add_kernel<int64_t>), dim3(k), dim3(64), 0, s, tab, ivalue);
    if (int st = launch_check("foreach_add_kernel")) return st;
  }
  return OMT_OK;
}

static int plane_scale(int64_t planes, int64_t hw, const float* x, const float* sv, float scale, float* y,
                       void* stream, const char* fn) {
  if (!sv || !y) return fail(OMT_INVALID, "%s: null pointer", fn);
  if (planes < 0 || hw < 0 || hw >= ((int64_t)1 << 31)) return fail(OMT_INVALID, "%s: size", fn);
  if (planes == 0 || hw == 0) return OMT_OK;
  const bool v4 = hw % 4 == 0 && al16(y) && (!x || al16(x));
  const int64_t total = planes * (v4 ? hw / 4 : hw);
  const dim3 grid(grid1d(total, 256, 8192));
  const FastDiv dv = make_fastdiv((uint32_t)(v4 ? hw / 4 : hw));
  hipStream_t s = stream_of(stream);
  if (x) {
    if (v4)
      hipLaunchKernelGGL((plane_scale_kernel<4, true>), grid, dim3(256), 0, s, x, sv, y, planes, (int)hw, scale, dv);
    else
      hipLaunchKernelGGL((plane_scale_kernel<1, true>), grid, dim3(256), 0, s, x, sv, y, planes, (int)hw, scale, dv);
  } else {
    if (v4)
      hipLaunchKernelGGL((plane_scale_kernel<4, false>), grid, dim3(256), 0, s, x, sv, y, planes, (int)hw, scale, dv);
    else
      hipLaunchKernelGGL((plane_scale_kernel<1, false>), grid, dim3(256), 0, s, x, sv, y, planes, (int)hw, scale, dv);
  }
  return launch_check("plane_scale_kernel");
}

OMT_EXPORT int omt_channel_scale(int64_t planes, int64_t hw, const float* x, const float* scale, float* y,
                                 void* stream) {
  if (!x) return fail(OMT_INVALID, "omt_channel_scale: null pointer");
  return plane_scale(planes, hw, x, scale, 1.f, y, stream, "omt_channel_scale");
}

OMT_EXPORT int omt_plane_broadcast(int64_t planes, int64_t hw, const float* v, float scale, float* y, void* stream) {
  return plane_scale(planes, hw, nullptr, v, scale, y, stream, "omt_plane_broadcast");
}

OMT_EXPORT int omt_plane_sum(int64_t planes, int64_t hw, const float* x, float scale, float* y, void* stream) {
  if (!x || !y) return fail(OMT_INVALID, "omt_plane_sum: null pointer");
  if (planes < 0 || hw < 0 || hw >= ((int64_t)1 << 31) || cdiv(planes, 4) >= ((int64_t)1 << 31))
    return fail(OMT_INVALID, "omt_plane_sum: size");
  if (planes == 0) return OMT_OK;
  if (hw >= kPlaneWG && planes < ((int64_t)1 << 31)) {
    if (hw % 4 == 0 && ((uintptr_t)x & 15) == 0)
      hipLaunchKernelGGL((plane_sum_wg_kernel<4, false>), dim3((unsigned)planes), dim3(256), 0, stream_of(stream), x, y,
                         (int)hw, scale, nullptr);
    else
      hipLaunchKernelGGL((plane_sum_wg_kernel<1, false>), dim3((unsigned)planes), dim3(256), 0, stream_of(stream), x, y,
                         (int)hw, scale, nullptr);
    return launch_check("plane_sum_wg_kernel");
  }
  hipLaunchKernelGGL(plane_sum_kernel<false>, dim3((unsigned)cdiv(planes, 4)), dim3(256), 0, stream_of(stream), x, y,
                     planes, (int)hw, scale, nullptr);
  return launch_check("plane_sum_kernel");
}

OMT_EXPORT int omt_plane_dot(int64_t planes, int64_t hw, const float* a, const float* b, float scale, float* y,
                             void* stream) {
  if (!a || !b || !y) return fail(OMT_INVALID, "omt_plane_dot: null pointer");
  if (planes < 0 || hw < 0 || hw >= ((int64_t)1 << 31) || cdiv(planes, 4) >= ((int64_t)1 << 31))
    return fail(OMT_INVALID, "omt_plane_dot: size");
  if (planes == 0) return OMT_OK;
  if (hw >= kPlaneWG && planes < ((int64_t)1 << 31)) {
    if (hw % 4 == 0 && ((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0)
      hipLaunchKernelGGL((plane_sum_wg_kernel<4, true>), dim3((unsigned)planes), dim3(256), 0, stream_of(stream), a, y,
                         (int)hw, scale, b);
    else
      hipLaunchKernelGGL((plane_sum_wg_kernel<1, true>), dim3((unsigned)planes), dim3(256), 0, stream_of(stream), a, y,
                         (int)hw, scale, b);
    return launch_check("plane_sum_wg_kernel (dot)");
  }
  hipLaunchKernelGGL(plane_sum_kernel<true>, dim3((unsigned)cdiv(planes, 4)), dim3(256), 0, stream_of(stream), a, y,
                     planes, (int)hw, scale, b);
  return launch_check("plane_sum_kernel (dot)");
}

OMT_EXPORT int omt_se_gate_bwd(int64_t planes, int64_t hw, const float* g, const float* s, const float* v,
                               float scale, float* y, void* stream) {
  if (!g || !s || !v || !y) return fail(OMT_INVALID, "omt_se_gate_bwd: null pointer");
  if (planes < 0 || hw < 0 || hw >= ((int64_t)1 << 31)) return fail(OMT_INVALID, "omt_se_gate_bwd: size");
  if (planes == 0 || hw == 0) return OMT_OK;
  const bool v4 = hw % 4 == 0 && al16(y) && al16(g);
  const int64_t total = planes * (v4 ? hw / 4 : hw);
  const dim3 grid(grid1d(total, 256, 8192));
  const FastDiv dv = make_fastdiv((uint32_t)(v4 ? hw / 4 : hw));
  if (v4)
    hipLaunchKernelGGL(se_gate_bwd_kernel<4>, grid, dim3(256), 0, stream_of(stream), g, s, v, y, planes, (int)hw,
                       scale, dv);
  else
    hipLaunchKernelGGL(se_gate_bwd_kernel<1>, grid, dim3(256), 0, stream_of(stream), g, s, v, y, planes, (int)hw,
                       scale, dv);
  return launch_check("se_gate_bwd_kernel");
}

OMT_EXPORT int omt_log_softmax_fwd(int64_t rows, int64_t cols, const float* x, float* y, void* stream) {
  if (!x || !y) return fail(OMT_INVALID, "omt_log_softmax_fwd: null pointer");
  if (rows < 0 || cols < 1 || cols >= ((int64_t)1 << 31) || cdiv(rows, 4) >= ((int64_t)1 << 31))
    return fail(OMT_INVALID, "omt_log_softmax_fwd: size");
  if (rows == 0) return OMT_OK;
  const dim3 grid((unsigned)cdiv(rows, 4));
  hipStream_t s = stream_of(stream);
  if (cols <= 256) hipLaunchKernelGGL(log_softmax_reg_kernel<4>, grid, dim3(256), 0, s, x, y, rows, (int)cols);
  else if (cols <= 1024) hipLaunchKernelGGL(log_softmax_reg_kernel<16>, grid, dim3(256), 0, s, x, y, rows, (int)cols);
  else if (cols <= 4096) hipLaunchKernelGGL(log_softmax_reg_kernel<64>, grid, dim3(256), 0, s, x, y, rows, (int)cols);
  else hipLaunchKernelGGL(log_softmax_kernel, grid, dim3(256), 0, s, x, y, rows, (int)cols);
  return launch_check("log_softmax_kernel");
}

OMT_EXPORT int omt_log_softmax_bwd(int64_t rows, int64_t cols, const float* g, const float* y, float* gx,
                                   void* stream) {
  if (!g || !y || !gx) return fail(OMT_INVALID, "omt_log_softmax_bwd: null pointer");
  if (rows < 0 || cols < 1 || cols >= ((int64_t)1 << 31) || cdiv(rows, 4) >= ((int64_t)1 << 31))
    return fail(OMT_INVALID, "omt_log_softmax_bwd: size");
  if (rows == 0) return OMT_OK;
  const dim3 grid((unsigned)cdiv(rows, 4));
  hipStream_t s = stream_of(stream);
  if (cols <= 256)
    hipLaunchKernelGGL(log_softmax_bwd_reg_kernel<4>, grid, dim3(256), 0, s, g, y, gx, rows, (int)cols);
  else if (cols <= 1024)
    hipLaunchKernelGGL(log_softmax_bwd_reg_kernel<16>, grid, dim3(256), 0, s, g, y, gx, rows, (int)cols);
  else if (cols <= 4096)
    hipLaunchKernelGGL(log_softmax_bwd_reg_kernel<64>, grid, dim3(256), 0, s, g, y, gx, rows, (int)cols);
  else
    hipLaunchKernelGGL(log_softmax_bwd_kernel, grid, dim3(256), 0, s, g, y, gx, rows, (int)cols);
  return launch_check("log_softmax_bwd_kernel");
}

OMT_EXPORT int omt_nll_loss_fwd(int64_t rows, int64_t cols, const float* logp, const int64_t* target,
                                const float* weight, int64_t ignore_index, int reduction, float* out,
                                float* total_weight, void* stream) {
  if (!logp || !target || !out || !total_weight) return fail(OMT_INVALID, "omt_nll_loss_fwd: null pointer");
  if (rows < 1 || cols < 1 || cols >= ((int64_t)1 << 31) || reduction < 0 || reduction > 2)
    return fail(OMT_INVALID, "omt_nll_loss_fwd: rows %lld, cols %lld, reduction %d", (long long)rows, (long long)cols,
                reduction);
  hipLaunchKernelGGL(nll_fwd_kernel, dim3(1), dim3(256), 0, stream_of(stream), logp, target, weight, rows, (int)cols,
                     ignore_index, reduction, out, total_weight);
  return launch_check("nll_fwd_kernel");
}

OMT_EXPORT int omt_nll_loss_bwd(int64_t rows, int64_t cols, const float* g, const int64_t* target,
                                const float* weight, int64_t ignore_index, int reduction, const float* total_weight,
                                float* gx, void* stream) {
  if (!g || !target || !gx || (reduction == 1 && !total_weight)) return fail(OMT_INVALID, "omt_nll_loss_bwd: null pointer");
  if (rows < 1 || cols < 1 || cols >= ((int64_t)1 << 31) || reduction < 0 || reduction > 2)
    return fail(OMT_INVALID, "omt_nll_loss_bwd: size or reduction");
  hipLaunchKernelGGL(nll_bwd_kernel, dim3(grid1d(rows * cols, 256, 8192)), dim3(256), 0, stream_of(stream), g, target,
                     weight, rows, (int)cols, ignore_index, reduction, total_weight, gx);
  return launch_check("nll_bwd_kernel");
}

OMT_EXPORT int omt_pointwise_layouts(int op, int64_t n, int64_t c, int64_t hw, const float* a, int a_nhwc,
                                     const float* b, int b_nhwc, float alpha, float* out, int out_nhwc, void* stream) {
  if (n < 0 || c < 0 || hw < 0) return fail(OMT_INVALID, "omt_pointwise_layouts: size");
  const int64_t total = n * c * hw;
  if (total == 0) return OMT_OK;
  const bool binary = op == OMT_PW_ADD || op == OMT_PW_MUL || op == OMT_PW_THRESHOLD_BWD ||
                      op == OMT_PW_HARDSWISH_BWD || op == OMT_PW_HARDSIGMOID_BWD;
  const bool unary = op == OMT_PW_RELU || op == OMT_PW_HARDSWISH || op == OMT_PW_HARDSIGMOID || op == OMT_PW_SCALE ||
                     op == OMT_PW_ADD_SCALAR;
  if (!binary && !unary) return fail(OMT_INVALID, "omt_pointwise_layouts: op %d", op);
  if (!out || !a || (binary && !b)) return fail(OMT_INVALID, "omt_pointwise_layouts: null pointer");
  hipStream_t s = stream_of(stream);
  const dim3 grid(grid1d(total, 256, 8192));
#define OMT_PWL(OP_)                                                                                         \
  case OP_:                                                                                                  \
    hipLaunchKernelGGL(pointwise_layouts_kernel<OP_>, grid, dim3(256), 0, s, a, a_nhwc, b, b_nhwc, out,     \
                       out_nhwc, total, c, hw, alpha);                                                       \
    break
  switch (op) {
    OMT_PWL(OMT_PW_ADD);
    OMT_PWL(OMT_PW_MUL);
    OMT_PWL(OMT_PW_RELU);
    OMT_PWL(OMT_PW_THRESHOLD_BWD);
    OMT_PWL(OMT_PW_HARDSWISH);
    OMT_PWL(OMT_PW_HARDSWISH_BWD);
    OMT_PWL(OMT_PW_HARDSIGMOID);
    OMT_PWL(OMT_PW_HARDSIGMOID_BWD);
    OMT_PWL(OMT_PW_SCALE);
    OMT_PWL(OMT_PW_ADD_SCALAR);
    default: break;
  }
#undef OMT_PWL
  return launch_check("pointwise_layouts_kernel");
}

OMT_EXPORT int omt_plane_sum_nhwc(int64_t n, int64_t c, int64_t hw, const float* x, float scale, float* y,
                                  void* stream) {
  if (!x || !y) return fail(OMT_INVALID, "omt_plane_sum_nhwc: null pointer");
  if (n < 0 || c < 1 || hw < 0 || hw >= ((int64_t)1 << 31) || c >= ((int64_t)1 << 31) || n > 65535 ||
      n * c * hw >= ((int64_t)1 << 46))
    return fail(OMT_INVALID, "omt_plane_sum_nhwc: size");
  if (n == 0) return OMT_OK;
  const int cb = (int)(c < 64 ? c : 64);
  const dim3 grid((unsigned)cdiv(c, cb), (unsigned)n);
  hipLaunchKernelGGL(plane_sum_nhwc_kernel, grid, dim3(256), 0, stream_of(stream), x, y, (int)c, (int)hw, cb, scale);
  return launch_check("plane_sum_nhwc_kernel");
}

OMT_EXPORT int omt_channel_scale_nhwc(int64_t n, int64_t c, int64_t hw, const float* x, const float* scale, float* y,
                                      void* stream) {
  if (!x || !scale || !y) return fail(OMT_INVALID, "omt_channel_scale_nhwc: null pointer");
  if (n < 0 || c < 1 || hw < 0 || n * c * hw >= ((int64_t)1 << 46)) return fail(OMT_INVALID, "omt_channel_scale_nhwc: size");
  if (n == 0 || hw == 0) return OMT_OK;
  const bool v4 = c % 4 == 0 && al16(x) && al16(scale) && al16(y);
  const int64_t cv = v4 ? c / 4 : c, total_v = n * hw * cv;
  const dim3 grid(grid1d(total_v, 256, 8192));
  if (v4)
    hipLaunchKernelGGL(channel_scale_nhwc_kernel<4>, grid, dim3(256), 0, stream_of(stream), x, scale, y, total_v, cv,
                       hw * cv);
  else
    hipLaunchKernelGGL(channel_scale_nhwc_kernel<1>, grid, dim3(256), 0, stream_of(stream), x, scale, y, total_v, cv,
                       hw * cv);
  return launch_check("channel_scale_nhwc_kernel");
}

OMT_EXPORT int omt_se_gate_bwd_nhwc(int64_t n, int64_t c, int64_t hw, const float* g, const float* s, const float* v,
                                    float scale, float* y, void* stream) {
  if (!g || !s || !v || !y) return fail(OMT_INVALID, "omt_se_gate_bwd_nhwc: null pointer");
  if (n < 0 || c < 1 || hw < 0 || n * c * hw >= ((int64_t)1 << 46)) return fail(OMT_INVALID, "omt_se_gate_bwd_nhwc: size");
  if (n == 0 || hw == 0) return OMT_OK;
  const bool v4 = c % 4 == 0 && al16(g) && al16(s) && al16(v) && al16(y);
  const int64_t cv = v4 ? c / 4 : c, total_v = n * hw * cv;
  const dim3 grid(grid1d(total_v, 256, 8192));
  if (v4)
    hipLaunchKernelGGL(se_gate_bwd_nhwc_kernel<4>, grid, dim3(256), 0, stream_of(stream), g, s, v, y, total_v, cv,
                       hw * cv, scale);
  else
    hipLaunchKernelGGL(se_gate_bwd_nhwc_kernel<1>, grid, dim3(256), 0, stream_of(stream), g, s, v, y, total_v, cv,
                       hw * cv, scale);
  return launch_check("se_gate_bwd_nhwc_kernel");
}
