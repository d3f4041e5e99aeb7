// Direct global->LDS loads for gfx950 kernels that stream tiles through an
// LDS ring (bf16 BSR SpMM, block-sparse attention).
//
// The loads are issued from inline asm so that the compiler does not track
// them: it cannot tell ring stages apart and would otherwise wait for every
// outstanding load before each LDS read. Callers wait for completion
// explicitly (wait_vm) before the barrier that publishes a stage; loads
// retire in issue order, so vmcnt <= N means all but the N most recent are
// done. M0 holds the wave's LDS destination and lane l writes its 16 bytes
// at M0 + 16 l (a contiguous 1 KiB per wave instruction).
//
// M0 is a reserved register, so its clobber is not tracked (hipcc warns);
// nothing the compiler generates for the kernels using these helpers reads
// or writes M0, so no value is lost across them. The build enforces this:
// it emits the gfx950 assembly of every source including this header and
// fails if an instruction outside the asm blocks names m0
// (trnsparse_amd/build_lib.py). The compiler's own builtins for these loads
// (__builtin_amdgcn_global_load_lds, __builtin_amdgcn_raw_ptr_buffer_load_lds)
// manage M0 themselves but make the compiler wait for every outstanding
// LDS load before each LDS read of the ring: measured +31 % on the bf16 BSR
// kernel at cfg3b (46 -> 60 us), +2 % on the fp32 attention forward.
#pragma once

#include "common.h"

namespace tsp {
namespace dma {

typedef int i32x4 __attribute__((ext_vector_type(4)));

// Raw buffer resource over [base, base + bytes): stride 0, 32-bit format;
// loads at offsets >= bytes return zero.
__device__ inline i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return i32x4{(int)(uint32_t)a, (int)(uint32_t)(a >> 32) & 0xFFFF, (int)bytes, 0x00020000};
}

// LDS byte address of a __shared__ object.
template <typename T>
__device__ inline uint32_t lds_addr(T* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)p;
}

// 16 bytes per lane from the global address g.
__device__ inline void global16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}

// 16 bytes per lane at byte offset voff of the buffer (zero when out of range).
__device__ inline void buffer16(i32x4 rsrc, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc),
               "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}

// Low 32 bits of *p, waited for in place (all earlier loads included): the
// compiler does not see this load either, so it never adds a wait for it on
// the streaming path.
__device__ inline int load_lo32_sync(const void* p) {
  int v;
  asm volatile("global_load_dword %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(p) : "memory");
  return v;
}

// s_waitcnt immediate waiting for vmcnt <= N only (gfx9 encoding).
template <int N>
__device__ inline void wait_vm() {
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (((N >> 4) & 3) << 14) | (0x7 << 4) | (0xF << 8));
}

// Workgroup barrier without the vector-memory part of __syncthreads' fence
// (which would wait for every outstanding load): it waits for the wave's own
// LDS (and scalar) operations, so ordinary LDS writes before it are visible
// after it, and the memory clobber keeps LDS accesses on their side. Loads
// into LDS are waited for separately (wait_vm).
__device__ inline void barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

}  // namespace dma
}  // namespace tsp
