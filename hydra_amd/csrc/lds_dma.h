// Buffer-descriptor loads straight into LDS (gfx950 "buffer_load ... lds")
// for the MFMA kernels that stage operand tiles this way.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hydra {

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer descriptor (base, stride 0, num_records, untyped access) as four
// wave-uniform words.
__device__ __forceinline__ i32x4_t raw_rsrc(const void* base, int num_records) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4_t r;
  r.x = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(a)));
  r.y = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(a >> 32) & 0xffffu));
  r.z = __builtin_amdgcn_readfirstlane(num_records);
  r.w = 0x00020000;
  return r;
}

// Buffer load of 16 bytes per lane straight into LDS: lane l's bytes land
// at lds + 16*l (lds must be wave-uniform), whatever its global offset; an
// offset at or past num_records writes zeros.  Written as inline assembly
// so that the compiler, which cannot tell which LDS bytes the transfer
// writes, does not make every later LDS read wait for it (a vmcnt(0) at the
// top of each tile, which would expose the prefetch's whole latency): the
// caller waits with vmcnt(0) and a barrier before reading the destination.
// M0 is written here; the compiler itself sets M0 right before each of its
// own instructions that read it, and the kernels that use this helper have
// none (checked in their assembly), so the clobber loses nothing.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void load16_to_lds(i32x4_t rsrc, uint32_t lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(rsrc) : "memory", "m0");
}
#pragma clang diagnostic pop

// LDS byte address of a pointer into shared memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}

}  // namespace hydra
