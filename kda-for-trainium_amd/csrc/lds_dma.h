// LDS staging helpers shared by the MFMA kernels: direct global->LDS DMA,
// explicit completion waits, and the transposed fragment read of an
// MN-contiguous bf16 tile.
#pragma once

#include "common.h"

namespace kda {

typedef short v4i16 __attribute__((ext_vector_type(4)));
#define KDA_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// One 16-byte-per-lane DMA from global memory into LDS: lane i's 16 bytes at
// `sbase + voff` land at LDS byte `lds + 16*i`.  The leading s_nop covers the
// M0-write hazard.  Inline asm, so that the compiler does not order later LDS
// reads behind it; completion is awaited with wait_vmcnt before the barrier that
// publishes the data.
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  // the base is wave-uniform by construction; readfirstlane makes that visible
  // (readfirstlane returns a signed int: widen through uint32_t, never sign-extend)
  const uint64_t v = reinterpret_cast<uint64_t>(sbase);
  const uint64_t u =
      ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
      (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff),
               "s"(reinterpret_cast<const void*>(u)), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
// A pointer that is the same in every lane, held in scalar registers.
__device__ __forceinline__ const char* uniform_ptr(const void* ptr) {
  const uint64_t v = reinterpret_cast<uint64_t>(ptr);
  return reinterpret_cast<const char*>(
      ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
      (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v));
}
// Same with a per-lane 64-bit address.
__device__ __forceinline__ void dma16_ptr(const void* src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}

// Waits until at most N of this wave's vector-memory operations (DMA included;
// stores count too) are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)KDA_LDS_PTR(p);
}

// Position of 32-byte segment s of k-row k in an MN-contiguous tile of at least
// 8 segments per row (measured conflict-free for the fragment read below).
__host__ __device__ __forceinline__ int mswz(int k) { return (k & 3) | (((k >> 3) & 1) << 2); }

// Reads the MFMA fragment (column `col0 + lane%16`, k = kbase + 8*(lane/16) .. +7)
// of an MN-contiguous [k][COLS] bf16 tile (segment s of row k at s ^ mswz(k));
// col0 is a multiple of 16.  Two ds_read_b64_tr_b16: within a 16-lane group,
// lane 4r+q names 4 elements of k-row r and lane j receives column j.
template <int COLS>
__device__ __forceinline__ bf16x8 read_mn_frag(const uint8_t* tile, int col0, int kbase, int lane) {
  const int g = lane >> 4, jj = lane & 15;
  const int s = col0 >> 4;
  const int k0 = kbase + 8 * g + (jj >> 2);
  const int k1 = k0 + 4;
  const uint8_t* p0 = tile + k0 * (2 * COLS) + ((s ^ mswz(k0)) << 5) + 8 * (jj & 3);
  const uint8_t* p1 = tile + k1 * (2 * COLS) + ((s ^ mswz(k1)) << 5) + 8 * (jj & 3);
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)KDA_LDS_PTR(p0));
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)KDA_LDS_PTR(p1));
  typedef short v8i16 __attribute__((ext_vector_type(8)));
  const v8i16 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

}  // namespace kda
