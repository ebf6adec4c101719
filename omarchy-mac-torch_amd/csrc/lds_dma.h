// Direct global -> LDS loads (buffer_load ... lds) and the vmcnt waits that order them, shared by the kernels that
// stage operands without passing them through registers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace omt {

// s_waitcnt immediate that waits for at most n outstanding vector memory operations (vmcnt in bits 3:0 and 15:14),
// leaving expcnt (6:4) and lgkmcnt (11:8) at their maxima, i.e. not waited for
constexpr int vmcnt_imm(int n) { return (n & 0xF) | (((n >> 4) & 3) << 14) | 0x70 | 0xF00; }

// The direct-LDS loads are issued as inline assembly. Through the builtin, the compiler tracks them as LDS writes and
// waits for all loads in flight before any LDS read it cannot prove independent of them (in a multi-stage ring, before
// some stages' reads, which collapses the ring). Hidden from it, ordering rests on the kernel's explicit waits (vmcnt counts these loads in issue
// order, so a wait for at most N outstanding covers every load issued before the last N) and barriers, with
// compiler-level memory barriers ("memory" clobbers) keeping the LDS reads after both.
typedef uint32_t omt_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ omt_u32x4 rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  return omt_u32x4{(uint32_t)p, (uint32_t)(p >> 32) & 0xFFFFu, bytes, 0x00020000u};  // stride 0, raw dwords
}
__device__ __forceinline__ uint32_t lds_addr(const float* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float*)p);
}
// lane i's dword at voff + soff lands at LDS byte address m0 + 4 i
__device__ __forceinline__ void lds_load_b32(omt_u32x4 r, uint32_t m0, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(r), "s"(soff)
               : "memory", "m0");
}
// lane i's 16 bytes at voff land at LDS byte address m0 + 16 i
__device__ __forceinline__ void lds_load_b128(omt_u32x4 r, uint32_t m0, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(r)
               : "memory", "m0");
}

}  // namespace omt
