// The squeeze-excite block's excitation MLP (MobileNetV3; omarchy_mac_torch.models.SqueezeExcite): per image n,
// a1 = W1 z[n] + b1, h = relu(a1), a2 = W2 h + b2, s[n] = hardsigmoid(a2), over the squeezed channels z [N][C], with
// W1 [R][C], b1 [R], W2 [C][R], b2 [C] (nn.Linear layouts), and its backward. Two launches forward and two backward,
// where the ops it replaces (linear, relu, linear, hardsigmoid and their gradients, with the GEMMs' slice sums and
// bias gradients) take about five and ten. No counterpart in the reference, whose squeeze-excite runs op by op; the
// torch.compile backend fuses the pattern.
//
// Every matrix-vector product runs a workgroup per (image, tile of 16 outputs): 16 groups of 16 threads, each group
// summing one output over a strided share of the reduction with many loads in flight, the 16 partial sums then added
// by DPP within the group (W v: the group's lanes read consecutive elements of the output's row) or through LDS in a
// fixed order (W^T v: the 16 lanes of a group read 16 consecutive outputs' elements of one row). Every sum runs in a
// fixed order: deterministic.
#include <algorithm>

#include "omt_internal.h"

namespace omt {

constexpr int kSeMaxC = 2048, kSeMaxR = 1024, kSeTile = 16;

// Sum over each row of 16 lanes, in every lane of the row (the first four DPP steps of wave_sum). All 64 lanes active.
__device__ __forceinline__ float row16_sum(float v) {
  int b = __builtin_bit_cast(int, v);
  v = dpp_add(v, __builtin_amdgcn_update_dpp(0, b, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
  b = __builtin_bit_cast(int, v);
  v = dpp_add(v, __builtin_amdgcn_update_dpp(0, b, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
  b = __builtin_bit_cast(int, v);
  v = dpp_add(v, __builtin_amdgcn_update_dpp(0, b, 0x141, 0xF, 0xF, false));  // row_half_mirror
  b = __builtin_bit_cast(int, v);
  return dpp_add(v, __builtin_amdgcn_update_dpp(0, b, 0x140, 0xF, 0xF, false));  // row_mirror
}

// sum over i = l + 16 m < cols of row[i] v[i] (row in global memory, v in LDS), eight loads in flight
__device__ __forceinline__ float strided_dot(const float* __restrict__ row, const float* v, int cols, int l) {
  float acc = 0.f;
  int i = l;
  for (; i + 7 * 16 < cols; i += 8 * 16) {
    float w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) w[u] = row[i + 16 * u];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = fmaf(w[u], v[i + 16 * u], acc);
  }
  for (; i < cols; i += 16) acc = fmaf(row[i], v[i], acc);
  return acc;
}

// sum over j = g + 16 m < rows of W[j][col] v[j] (a column of row-major W with `cols` columns; v in LDS), eight
// loads in flight; the 16 threads of a group read 16 consecutive columns of each row
__device__ __forceinline__ float column_dot(const float* __restrict__ W, int cols, int col, const float* v, int rows,
                                            int g) {
  float acc = 0.f;
  int j = g;
  for (; j + 7 * 16 < rows; j += 8 * 16) {
    float w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) w[u] = W[(int64_t)(j + 16 * u) * cols + col];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = fmaf(w[u], v[j + 16 * u], acc);
  }
  for (; j < rows; j += 16) acc = fmaf(W[(int64_t)j * cols + col], v[j], acc);
  return acc;
}

// The 16 groups' partial sums of each of 16 columns (thread g * 16 + l holds group g's sum for column l), added in
// group order; valid in threads l < 16 (group 0). All threads call it.
__device__ __forceinline__ float column_sum(float part) {
  __shared__ float red[kSeTile][kSeTile];
  const int l = threadIdx.x & 15, g = threadIdx.x >> 4;
  red[g][l] = part;
  __syncthreads();
  float s = 0.f;
  if (g == 0)
    for (int k = 0; k < kSeTile; ++k) s += red[k][l];
  return s;
}

__device__ __forceinline__ float se_relu(float a) { return a <= 0.f ? 0.f : a; }  // NaN propagates, as torch.relu

// forward 1: h[n][j] = relu(b1[j] + W1[j] . z[n]), workgroup (n, tile of 16 j): thread (row j, lane l)
__global__ void __launch_bounds__(256) se_hidden_kernel(const float* __restrict__ z, const float* __restrict__ w1,
                                                        const float* __restrict__ b1, float* __restrict__ h, int c,
                                                        int r, int tiles) {
  __shared__ float zs[kSeMaxC];
  const int n = (int)blockIdx.x / tiles, tile = (int)blockIdx.x - n * tiles;
  for (int i = threadIdx.x; i < c; i += 256) zs[i] = z[(int64_t)n * c + i];
  __syncthreads();
  const int j = tile * kSeTile + (int)(threadIdx.x >> 4), l = threadIdx.x & 15;
  const float acc = row16_sum(j < r ? strided_dot(w1 + (int64_t)j * c, zs, c, l) : 0.f);
  if (l == 0 && j < r) h[(int64_t)n * r + j] = se_relu(acc + b1[j]);
}

// forward 2: a2[n][k] = b2[k] + W2[k] . h[n], s = hardsigmoid(a2), workgroup (n, tile of 16 k)
__global__ void __launch_bounds__(256) se_out_kernel(const float* __restrict__ h, const float* __restrict__ w2,
                                                     const float* __restrict__ b2, float* __restrict__ s,
                                                     float* __restrict__ a2, int c, int r, int tiles) {
  __shared__ float hs[kSeMaxR];
  const int n = (int)blockIdx.x / tiles, tile = (int)blockIdx.x - n * tiles;
  for (int j = threadIdx.x; j < r; j += 256) hs[j] = h[(int64_t)n * r + j];
  __syncthreads();
  const int k = tile * kSeTile + (int)(threadIdx.x >> 4), l = threadIdx.x & 15;
  const float acc = row16_sum(k < c ? strided_dot(w2 + (int64_t)k * r, hs, r, l) : 0.f);
  if (l == 0 && k < c) {
    const float a = acc + b2[k];
    a2[(int64_t)n * c + k] = a;
    s[(int64_t)n * c + k] = hardsigmoid_f(a);
  }
}

// backward 1: da2[n][k] = gs hardsigmoid'(a2); da1[n][j] = (W2^T da2[n])[j] where h > 0, workgroup (n, tile of 16 j):
// thread (group g, column j). Tile 0 also stores da2[n] for the weight gradients.
__global__ void __launch_bounds__(256) se_bwd_hidden_kernel(const float* __restrict__ gs, const float* __restrict__ a2,
                                                            const float* __restrict__ h, const float* __restrict__ w2,
                                                            float* __restrict__ da2, float* __restrict__ da1, int c,
                                                            int r, int tiles) {
  __shared__ float d2[kSeMaxC];
  const int n = (int)blockIdx.x / tiles, tile = (int)blockIdx.x - n * tiles;
  for (int k = threadIdx.x; k < c; k += 256) {
    const float d = hardsigmoid_grad(gs[(int64_t)n * c + k], a2[(int64_t)n * c + k]);
    d2[k] = d;
    if (tile == 0) da2[(int64_t)n * c + k] = d;
  }
  __syncthreads();
  const int j = tile * kSeTile + (threadIdx.x & 15), g = threadIdx.x >> 4;
  const float dh = column_sum(j < r ? column_dot(w2, r, j, d2, c, g) : 0.f);
  if (g == 0 && j < r) da1[(int64_t)n * r + j] = h[(int64_t)n * r + j] > 0.f ? dh : 0.f;
}

// backward 2, one launch of two parts. Workgroups [0, n * ctiles): gz[n][i] = (W1^T da1[n])[i], workgroup (n, tile of
// 16 i). The rest: the weight and bias gradients, a thread per element, each a sum over the N images in image order:
// gw1[j][i] = sum_n da1[n][j] z[n][i], gw2[k][j] = sum_n da2[n][k] h[n][j], gb1[j] = sum_n da1[n][j],
// gb2[k] = sum_n da2[n][k].
__global__ void __launch_bounds__(256) se_bwd_input_kernel(const float* __restrict__ z, const float* __restrict__ h,
                                                           const float* __restrict__ w1, const float* __restrict__ da1,
                                                           const float* __restrict__ da2, float* __restrict__ gz,
                                                           float* __restrict__ gw1, float* __restrict__ gb1,
                                                           float* __restrict__ gw2, float* __restrict__ gb2, int nimg,
                                                           int c, int r, int ctiles) {
  const int64_t gzblocks = (int64_t)nimg * ctiles;
  if ((int64_t)blockIdx.x < gzblocks) {
    __shared__ float d1[kSeMaxR];
    const int n = (int)blockIdx.x / ctiles, tile = (int)blockIdx.x - n * ctiles;
    for (int j = threadIdx.x; j < r; j += 256) d1[j] = da1[(int64_t)n * r + j];
    __syncthreads();
    const int i = tile * kSeTile + (threadIdx.x & 15), g = threadIdx.x >> 4;
    const float dz = column_sum(i < c ? column_dot(w1, c, i, d1, r, g) : 0.f);
    if (g == 0 && i < c) gz[(int64_t)n * c + i] = dz;
    return;
  }
  const int64_t rc = (int64_t)r * c;
  const int64_t e = ((int64_t)blockIdx.x - gzblocks) * 256 + threadIdx.x;
  const float* a;  // per image: a[m * as + ai] * b[m * bs + bi], summed over m
  const float* b = nullptr;
  int64_t as, ai, bs = 0, bi = 0;
  float* out;
  if (e < rc) {  // gw1[j][i]
    const int j = (int)(e / c);
    a = da1, as = r, ai = j, b = z, bs = c, bi = e - (int64_t)j * c, out = gw1 + e;
  } else if (e < 2 * rc) {  // gw2[k][j]
    const int64_t f = e - rc;
    const int k = (int)(f / r);
    a = da2, as = c, ai = k, b = h, bs = r, bi = f - (int64_t)k * r, out = gw2 + f;
  } else if (e < 2 * rc + r) {
    a = da1, as = r, ai = e - 2 * rc, out = gb1 + ai;
  } else if (e < 2 * rc + r + c) {
    a = da2, as = c, ai = e - 2 * rc - r, out = gb2 + ai;
  } else {
    return;
  }
  float acc = 0.f;
  int m = 0;
  for (; m + 8 <= nimg; m += 8) {  // eight images' loads in flight, added in image order
    float x[8], y[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      x[u] = a[(int64_t)(m + u) * as + ai];
      y[u] = b ? b[(int64_t)(m + u) * bs + bi] : 1.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = b ? fmaf(x[u], y[u], acc) : acc + x[u];
  }
  for (; m < nimg; ++m) acc = b ? fmaf(a[(int64_t)m * as + ai], b[(int64_t)m * bs + bi], acc) : acc + a[(int64_t)m * as + ai];
  *out = acc;
}

static bool se_sizes_ok(int64_t n, int64_t c, int64_t r) {
  return n >= 1 && c >= 1 && r >= 1 && c <= kSeMaxC && r <= kSeMaxR && n * c < ((int64_t)1 << 31) &&
         2 * r * c + r + c < ((int64_t)1 << 31) && n * cdiv(c, kSeTile) < ((int64_t)1 << 20);
}

OMT_EXPORT size_t omt_se_bwd_workspace(int64_t n, int64_t c, int64_t r) {
  return se_sizes_ok(n, c, r) ? (size_t)(n * (c + r)) * sizeof(float) : 0;
}

OMT_EXPORT int omt_se_fwd(int64_t n, int64_t c, int64_t r, const float* z, const float* w1, const float* b1,
                          const float* w2, const float* b2, float* s, float* h, float* a2, void* stream) {
  if (!z || !w1 || !b1 || !w2 || !b2 || !s || !h || !a2) return fail(OMT_INVALID, "omt_se_fwd: null pointer");
  if (!se_sizes_ok(n, c, r))
    return fail(OMT_UNSUPPORTED, "omt_se_fwd: %lld x %lld channels, %lld hidden not covered", (long long)n,
                (long long)c, (long long)r);
  hipStream_t st = stream_of(stream);
  const int rt = (int)cdiv(r, kSeTile), ct = (int)cdiv(c, kSeTile);
  hipLaunchKernelGGL(se_hidden_kernel, dim3((unsigned)(n * rt)), dim3(256), 0, st, z, w1, b1, h, (int)c, (int)r, rt);
  if (int e = launch_check("se_hidden_kernel")) return e;
  hipLaunchKernelGGL(se_out_kernel, dim3((unsigned)(n * ct)), dim3(256), 0, st, h, w2, b2, s, a2, (int)c, (int)r, ct);
  return launch_check("se_out_kernel");
}

OMT_EXPORT int omt_se_bwd(int64_t n, int64_t c, int64_t r, const float* gs, const float* z, const float* h,
                          const float* a2, const float* w1, const float* w2, float* gz, float* gw1, float* gb1,
                          float* gw2, float* gb2, void* workspace, size_t workspace_bytes, void* stream) {
  if (!gs || !z || !h || !a2 || !w1 || !w2 || !gz || !gw1 || !gb1 || !gw2 || !gb2)
    return fail(OMT_INVALID, "omt_se_bwd: null pointer");
  if (!se_sizes_ok(n, c, r))
    return fail(OMT_UNSUPPORTED, "omt_se_bwd: %lld x %lld channels, %lld hidden not covered", (long long)n,
                (long long)c, (long long)r);
  if (!workspace || workspace_bytes < omt_se_bwd_workspace(n, c, r))
    return fail(OMT_INVALID, "omt_se_bwd: workspace too small");
  hipStream_t st = stream_of(stream);
  float* da2 = (float*)workspace;
  float* da1 = da2 + n * c;
  const int rt = (int)cdiv(r, kSeTile), ct = (int)cdiv(c, kSeTile);
  hipLaunchKernelGGL(se_bwd_hidden_kernel, dim3((unsigned)(n * rt)), dim3(256), 0, st, gs, a2, h, w2, da2, da1, (int)c,
                     (int)r, rt);
  if (int e = launch_check("se_bwd_hidden_kernel")) return e;
  const int64_t blocks = n * ct + cdiv(2 * r * c + r + c, 256);
  hipLaunchKernelGGL(se_bwd_input_kernel, dim3((unsigned)blocks), dim3(256), 0, st, z, h, w1, da1, da2, gz, gw1, gb1,
                     gw2, gb2, (int)n, (int)c, (int)r, ct);
  return launch_check("se_bwd_input_kernel");
}

}  // namespace omt
