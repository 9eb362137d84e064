// LDS staging helpers shared by the MFMA kernels (gfx950): direct-to-LDS
// loads, 16-bit transpose-read vector types and s_waitcnt immediates.
#pragma once

#include "qh_common.h"

typedef short qh_v4i16 __attribute__((ext_vector_type(4)));
typedef short qh_v8i16 __attribute__((ext_vector_type(8)));

namespace {

// Direct-to-LDS loads, 16 bytes per lane: lane l's bytes land at LDS byte
// address lds_base + 16 * l (lds_base is wave-uniform and travels in M0).
// They are issued as inline asm so the compiler's wait-count pass does not
// track them: it would otherwise have to assume that every later LDS read may
// alias the in-flight load and wait for it at once, serialising the prefetch.
// Callers wait explicitly (s_waitcnt vmcnt(0) + barrier) before reading the
// destination. M0 has no other user in these kernels.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// 64-bit per-lane address.
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds_base) {
  lds_base = (uint32_t)__builtin_amdgcn_readfirstlane(lds_base);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds_base)
               : "memory", "m0");
}
// Wave-uniform 64-bit base (SGPRs) + per-lane 32-bit byte offset. The base is
// uniform by construction; readfirstlane states it for the compiler.
__device__ __forceinline__ void lds_dma16_s(uint32_t voff, const void* base, uint32_t lds_base) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  // readfirstlane returns int: widen through uint32_t (no sign extension)
  const uint64_t ub = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b) |
                      ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32);
  const void* sbase = (const void*)(uintptr_t)ub;
  lds_base = (uint32_t)__builtin_amdgcn_readfirstlane(lds_base);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
               "s"(lds_base)
               : "memory", "m0");
}
// Non-temporal forms (the `nt` cache-policy hint): for data read once and
// streamed past the caches, such as a decode step's KV cache, whose 0.5 GB per
// layer exceeds the last-level cache so keeping it there only evicts other data.
__device__ __forceinline__ void lds_dma16_nt(const void* src, uint32_t lds_base) {
  lds_base = (uint32_t)__builtin_amdgcn_readfirstlane(lds_base);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_dma16_s_nt(uint32_t voff, const void* base, uint32_t lds_base) {
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint64_t ub = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b) |
                      ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32);
  const void* sbase = (const void*)(uintptr_t)ub;
  lds_base = (uint32_t)__builtin_amdgcn_readfirstlane(lds_base);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase),
               "s"(lds_base)
               : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// s_waitcnt immediates (gfx9 encoding: vmcnt in [3:0] and [15:14], expcnt in
// [6:4], lgkmcnt in [11:8]) that wait on one counter only.
constexpr int waitcnt_vm(int n) { return (n & 0xF) | (((n >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8); }
constexpr int kWaitLgkm0 = 0xF | (0x3 << 14) | (0x7 << 4);

}  // namespace
