// In-order sums of split-K partials, shared by the convolution's slice-sum launches (conv_gemm.hip) and the
// BatchNorm backward that takes a preceding convolution's slice sums into its own launch (bn.hip): the same code, so
// the same order of additions and the same results wherever a sum runs.
#pragma once

#include <algorithm>

#include "omt_internal.h"

namespace omt {

// Slice sums load kReduceBatch slices at a time (the loads in flight together, the additions still in slice order),
// so a launch waits one memory latency per batch rather than per slice.
constexpr int kReduceBatch = 8;

template <int VEC>
struct VecF;
template <>
struct VecF<1> {
  using T = float;
  static __device__ __forceinline__ void add(float* v, T t) { v[0] += t; }
  static __device__ __forceinline__ void set(float* v, T t) { v[0] = t; }
  static __device__ __forceinline__ T pack(const float* v) { return v[0]; }
};
template <>
struct VecF<4> {
  using T = float4;
  static __device__ __forceinline__ void add(float* v, T t) { v[0] += t.x, v[1] += t.y, v[2] += t.z, v[3] += t.w; }
  static __device__ __forceinline__ void set(float* v, T t) { v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w; }
  static __device__ __forceinline__ T pack(const float* v) { return make_float4(v[0], v[1], v[2], v[3]); }
};

// v = sum_z part[z * nv + i] over z in slice order (vectors of VEC floats; nv vectors per slice).
template <int VEC>
__device__ __forceinline__ void sum_slices(const typename VecF<VEC>::T* __restrict__ part, int64_t nv, int64_t i,
                                           int slices, float* v) {
  using T = typename VecF<VEC>::T;
  for (int z0 = 0; z0 < slices; z0 += kReduceBatch) {
    T t[kReduceBatch];
#pragma unroll
    for (int u = 0; u < kReduceBatch; ++u)
      if (z0 + u < slices) t[u] = part[(int64_t)(z0 + u) * nv + i];
#pragma unroll
    for (int u = 0; u < kReduceBatch; ++u)
      if (z0 + u < slices) {
        if (z0 + u == 0)
          VecF<VEC>::set(v, t[u]);
        else
          VecF<VEC>::add(v, t[u]);
      }
  }
}

// The slice sums run on kSumThreads threads of a workgroup (a larger workgroup's other waves end before them).
constexpr int kSumThreads = 256;

// Sums the slices in slice order (deterministic): out[i] = sum_z part[z][i]. VEC 4 needs n % 4 == 0. Workgroups
// b0 .. b0 + nb - 1 of the launch stride over the vectors.
template <int VEC>
__device__ __forceinline__ void split_sum(const float* __restrict__ part, float* __restrict__ out, int64_t n,
                                          int slices, int64_t b0, int64_t nb) {
  using T = typename VecF<VEC>::T;
  const int64_t nv = n / VEC;
  for (int64_t i = b0 * kSumThreads + threadIdx.x; i < nv; i += nb * kSumThreads) {
    float v[VEC];
    sum_slices<VEC>(reinterpret_cast<const T*>(part), nv, i, slices, v);
    reinterpret_cast<T*>(out)[i] = VecF<VEC>::pack(v);
  }
}

// Many slices (kGroupSlices and more): a workgroup takes 16 consecutive vectors, and each of its 16 groups of 16
// threads sums a contiguous range of about slices / 16 slices in slice order (eight loads in flight); the group sums
// are then added in group order. A fixed order, so still deterministic, and a sixteenth of the dependent load batches
// per thread (a grad weight of 16 x 16 outputs over 251 slices waited 32 batches long in the plain order).
constexpr int kGroupSlices = 32;
template <int VEC>
__device__ __forceinline__ void split_sum_grouped(const float* __restrict__ part, float* __restrict__ out, int64_t n,
                                                  int slices, int64_t b0, int64_t nb) {
  using T = typename VecF<VEC>::T;
  __shared__ float red[16][16][VEC];
  const int64_t nv = n / VEC;
  const int tv = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const int per = (slices + 15) / 16, z0 = grp * per, z1 = min(slices, z0 + per);
  const T* p = reinterpret_cast<const T*>(part);
  for (int64_t base = b0 * 16; base < nv; base += nb * 16) {
    const int64_t i = base + tv;
    float v[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] = 0.f;
    if (i < nv) {
      for (int z = z0; z < z1; z += kReduceBatch) {
        T t[kReduceBatch];
#pragma unroll
        for (int u = 0; u < kReduceBatch; ++u)
          if (z + u < z1) t[u] = p[(int64_t)(z + u) * nv + i];
#pragma unroll
        for (int u = 0; u < kReduceBatch; ++u)
          if (z + u < z1) {
            if (z + u == z0)
              VecF<VEC>::set(v, t[u]);
            else
              VecF<VEC>::add(v, t[u]);
          }
      }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) red[grp][tv][e] = v[e];
    __syncthreads();
    if (grp == 0 && i < nv) {
      float sum[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) sum[e] = red[0][tv][e];
      for (int g2 = 1; g2 < 16; ++g2)
#pragma unroll
        for (int e = 0; e < VEC; ++e) sum[e] += red[g2][tv][e];
      reinterpret_cast<T*>(out)[i] = VecF<VEC>::pack(sum);
    }
    __syncthreads();
  }
}

struct SplitSum {
  const float* part;
  float* out;
  int64_t n;
  int slices;
  bool vec4;
  int64_t blocks;
};
template <int VEC>
__device__ __forceinline__ void split_sum_any(const SplitSum& r, int64_t b0, int64_t nb) {
  if (r.slices >= kGroupSlices)
    split_sum_grouped<VEC>(r.part, r.out, r.n, r.slices, b0, nb);
  else
    split_sum<VEC>(r.part, r.out, r.n, r.slices, b0, nb);
}

// The in-order sum of `slices` consecutive arrays of n floats at `part` into `out`.
inline SplitSum split_sum_of(const float* part, float* out, int64_t n, int64_t slices) {
  SplitSum r{};
  r.part = part;
  r.out = out;
  r.n = n;
  r.slices = (int)slices;
  r.vec4 = r.n % 4 == 0 && (uintptr_t)out % 16 == 0 && (uintptr_t)part % 16 == 0;
  const int64_t nv = r.vec4 ? r.n / 4 : r.n;
  r.blocks = r.slices >= kGroupSlices ? std::min<int64_t>(cdiv(nv, 16), 8192) : grid1d(nv, 256, 8192);
  return r;
}

}  // namespace omt
