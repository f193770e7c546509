// Direct global->LDS loads shared by the MFMA GEMM kernels (gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace mtx {

typedef __attribute__((address_space(3))) char lds_char;

// 16-byte direct global->LDS load: lane l writes LDS byte lds_base + 16*l (lds_base is
// wave-uniform).  Issued as inline asm so that the compiler does not serialise the LDS reads
// of other ring stages behind these loads; kernels wait for them with MTX_VMCNT.
__device__ __forceinline__ void gload_lds16(const void* gptr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_base)
               : "memory", "m0");
}

// 4-byte direct global->LDS load: lane l writes LDS byte lds_base + 4*l.
__device__ __forceinline__ void gload_lds4(const void* gptr, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(gptr), "s"(lds_base)
               : "memory", "m0");
}

// The same two loads with a uniform 64-bit base in SGPRs and a per-lane 32-bit byte offset, so
// that advancing the base (a k step, another tile) costs scalar instead of per-lane 64-bit adds.
__device__ __forceinline__ void gload_lds16_s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}
__device__ __forceinline__ void gload_lds4_s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_base)
               : "memory", "m0");
}

// LDS byte address of a __shared__ array (for M0).
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T* p) {
  return (uint32_t)(uintptr_t)(lds_char*)p;
}

}  // namespace mtx

// s_waitcnt immediate (GFX9 encoding) that waits for vmcnt <= N only.
#define MTX_VMCNT(N) ((((N) & 0xF)) | (0x7 << 4) | (0xF << 8) | ((((N) >> 4) & 0x3) << 14))
// s_waitcnt immediate that waits for lgkmcnt == 0 only.
#define MTX_LGKMCNT0 0xC07F
