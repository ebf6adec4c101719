// Internal helpers shared by the libomt_hip.so translation units: status/error plumbing, launch checks, fast
// integer division and the fp32 MFMA vector type.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "omt_hip.h"

namespace omt {

// Sets this thread's last-error message and returns `st`.
int fail(int st, const char* fmt, ...);
// Maps a HIP error to OMT_DEVICE_ERROR (with the runtime's message), or OMT_OK.
int hip_check(hipError_t e, const char* what);
// Checks the last launch on this thread.
int launch_check(const char* kernel);
// The stream a call runs on: the caller's hipStream_t (NULL = the HIP null stream).
hipStream_t stream_of(void* s);

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline unsigned grid1d(int64_t total, int block, int64_t cap = 1 << 20) {
  int64_t g = cdiv(total, block);
  if (g > cap) g = cap;
  return (unsigned)(g < 1 ? 1 : g);
}

// Unsigned 32-bit division by a runtime-invariant divisor as a multiply-high and shifts (Granlund & Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994, fig. 4.1): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, t = umulhi(m, n) gives n / d = (t + ((n - t) >> 1)) >> (l - 1) for d >= 2.
struct FastDiv {
  uint32_t d, mul, shift;
};
inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0, 0};
  if (d <= 1) return f;
  uint32_t l = 0;
  while ((1ull << l) < d) l++;
  // mul = floor(2^32 * (2^l - d) / d) + 1
  f.mul = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
  f.shift = l;
  return f;
}
__host__ __device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  if (f.d == 1) return n;
  uint32_t hi = (uint32_t)(((uint64_t)n * f.mul) >> 32);
  return (hi + ((n - hi) >> 1)) >> (f.shift - 1);
}

// Raw buffer loads: a resource over [base, base + bytes) with the range check on, so a load at a byte offset past
// `bytes` returns 0 without touching memory. Offsets are 32-bit: every buffer read this way is below 2 GiB, and kOOB
// is an offset beyond all of them (padding taps, tails).
constexpr uint32_t kOOB = 0x80000000u;
constexpr int64_t kMaxBufBytes = 0x7fffffffll;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}
// Four consecutive floats (a multi-dword buffer load needs 4-byte alignment only; all four in range or all four out).
__device__ __forceinline__ float4 bload4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0));
}

// Hardswish and its gradient as PyTorch defines them (torch.nn.Hardswish documentation), in the same order of
// operations as its CPU kernels, so that results agree to the last bit in most cases. Shared by the pointwise kernels
// and the BatchNorm kernels that apply it after the normalization.
__device__ __forceinline__ float hardswish_f(float x) { return x * fminf(fmaxf(x + 3.f, 0.f), 6.f) / 6.f; }
__device__ __forceinline__ float hardswish_grad(float g, float x) {
  return x <= -3.f ? 0.f : (x < 3.f ? g * (x / 3.f + 0.5f) : g);
}
// Hardsigmoid as PyTorch defines it (torch.nn.Hardsigmoid documentation), in the same order of operations as its CPU
// kernels, so that results agree to the last bit in most cases.
__device__ __forceinline__ float hardsigmoid_f(float x) { return fminf(fmaxf(x + 3.f, 0.f), 6.f) / 6.f; }
__device__ __forceinline__ float hardsigmoid_grad(float g, float x) {
  return (x > -3.f && x < 3.f) ? g * (1.f / 6.f) : 0.f;
}
// The activation after a BatchNorm: act OMT_ACT_NONE, OMT_ACT_RELU or OMT_ACT_HARDSWISH.
__device__ __forceinline__ float bn_act(float v, int act) {
  return act == OMT_ACT_RELU ? fmaxf(v, 0.f) : (act == OMT_ACT_HARDSWISH ? hardswish_f(v) : v);
}
// The gradient through that activation: r is the ReLU's output (masked where not > 0) or the hardswish's input.
__device__ __forceinline__ float bn_act_grad(float g, float r, int act) {
  return act == OMT_ACT_RELU ? (r > 0.f ? g : 0.f) : (act == OMT_ACT_HARDSWISH ? hardswish_grad(g, r) : g);
}

// Sum over the 64 lanes of a wave, in every lane: four DPP steps within each row of 16 lanes, each adding a disjoint
// partner (quad_perm [1,0,3,2] and [2,3,0,1]: every lane holds its quad's sum; row_half_mirror pairs the two quads
// of each 8-lane half, row_mirror the two halves), then the four row sums read from lanes 0, 16, 32 and 48. All 64
// lanes must be active. VALU work only: a __shfl_xor butterfly takes six LDS-routed permutes per value.
__device__ __forceinline__ float dpp_add(float v, int moved) { return v + __builtin_bit_cast(float, moved); }
__device__ __forceinline__ float wave_sum(float v) {
  int b = __builtin_bit_cast(int, v);
  v = dpp_add(v, __builtin_amdgcn_update_dpp(0, b, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
  b = __builtin_bit_cast(int, v);
  v = dpp_add(v, __builtin_amdgcn_update_dpp(0, b, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
  b = __builtin_bit_cast(int, v);
  v = dpp_add(v, __builtin_amdgcn_update_dpp(0, b, 0x141, 0xF, 0xF, false));  // row_half_mirror
  b = __builtin_bit_cast(int, v);
  v = dpp_add(v, __builtin_amdgcn_update_dpp(0, b, 0x140, 0xF, 0xF, false));  // row_mirror
  b = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
         (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
          __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

// Doubles through the same DPP steps, both 32-bit halves moved with one control. row16_sum: the sum over each row of
// 16 lanes, in every lane of the row (the four steps above); wave_sum: then the four row sums from lanes 0, 16, 32, 48.
// All 64 lanes must be active. VALU work only.
template <int CTRL>
__device__ __forceinline__ double dpp_move(double v) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ double read_lane(double v, int lane) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
  return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double row16_sum(double v) {
  v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_move<0x141>(v);  // row_half_mirror
  v += dpp_move<0x140>(v);  // row_mirror
  return v;
}
__device__ __forceinline__ double wave_sum(double v) {
  v = row16_sum(v);
  return (read_lane(v, 0) + read_lane(v, 16)) + (read_lane(v, 32) + read_lane(v, 48));
}

}  // namespace omt

typedef float omt_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int omt_u32x4 __attribute__((ext_vector_type(4)));

#define OMT_EXPORT extern "C" __attribute__((visibility("default")))

// Runs `expr` (a HIP call) and returns OMT_DEVICE_ERROR from the enclosing function if it fails.
#define OMT_HIP(expr)                                              \
  do {                                                             \
    hipError_t e_ = (expr);                                        \
    if (e_ != hipSuccess) return ::omt::hip_check(e_, #expr);      \
  } while (0)
