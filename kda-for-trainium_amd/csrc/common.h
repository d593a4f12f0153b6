// Shared device/host helpers for the gfx950 kernels: vector types, bf16
// conversion, error reporting across the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kda.h"

namespace kda {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Records a failure for kda_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the calling thread's error message; returns KDA_OK.
int clear_error();
// Converts the status of the last launch into a KDA status code.
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Number of compute units on the current device (cached per device).
int device_cu_count();

// Workspace bytes of kda_gqa_fwd_f32 (layout owned by attention_f32.hip).
int64_t gqa_f32_workspace_bytes(int64_t batch, int64_t seq, int64_t hq, int64_t hkv);

// ---- device helpers -------------------------------------------------------

// fp32 -> bf16 bits, round to nearest even; a NaN stays a NaN (sign kept, quiet
// bit set: adding the rounding bias to a NaN could carry it into +0 or infinity).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __builtin_bit_cast(float, b << 16);
}

// Packs two floats into one dword of two bf16 (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

}  // namespace kda
