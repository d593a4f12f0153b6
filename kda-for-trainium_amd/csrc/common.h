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

// ---- streamed output stores ------------------------------------------------
// A window of `bytes` bytes (at most 4 GiB) from `base` for buffer stores with
// 32-bit offsets; a store at or past the end of the window is dropped by the
// buffer range check.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t out_window(void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, 0x00020000);
}
// 16 bytes at byte offset `off` (+ the wave-uniform `soff`) of window `w`, with
// cache policy SC1 + NT (device-scope coherence, streaming) instead of NT alone.
// Measured on MI355X with inputs and outputs rotating through more memory than the
// Infinity Cache holds, SiLU over 64 MiB and 112 MiB arrays: SC1 alone 1.4 % faster
// than NT, SC1 + NT another 1.2-1.7 % on the single-call median (0.5 % back to
// back; SC0 + SC1 + NT the same); plain and SC0 stores were 1-3 % slower than NT.
// Not a general rule: AdamW ran 1-2 % slower with SC1 or SC1 + NT, RoPE no faster,
// and bmm's strided 1 GB output 22 % slower with SC1, so those keep NT stores.
// A buffer store because no global-store builtin takes a cache policy.
constexpr int kCpolNt = 2;
constexpr int kCpolSc1 = 16;
__device__ __forceinline__ void store_sc1_nt(__amdgpu_buffer_rsrc_t w, uint32_t off, const floatx4& v,
                                             uint32_t soff = 0) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), w, (int)off, (int)soff,
                                         kCpolSc1 | kCpolNt);
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Number of compute units on the current device (cached per device).
int device_cu_count();

// ---- workspace size arithmetic (host) ---------------------------------------
// A size term built from caller-supplied sizes: products and sums of terms go
// invalid (-1) on a negative operand or on int64 overflow instead of wrapping,
// so a size query never overflows and never reports a buffer smaller than the
// one the kernels would use.
struct SizeTerm {
  int64_t v;
  constexpr SizeTerm(int64_t x) : v(x < 0 ? -1 : x) {}
  bool ok() const { return v >= 0; }
  friend SizeTerm operator*(SizeTerm a, SizeTerm b) {
    int64_t r;
    return (!a.ok() || !b.ok() || __builtin_mul_overflow(a.v, b.v, &r)) ? SizeTerm(-1) : SizeTerm(r);
  }
  friend SizeTerm operator+(SizeTerm a, SizeTerm b) {
    int64_t r;
    return (!a.ok() || !b.ok() || __builtin_add_overflow(a.v, b.v, &r)) ? SizeTerm(-1) : SizeTerm(r);
  }
};
// ceil(n / d) for n >= 0, d > 0 without forming n + d - 1; -1 for n < 0
inline SizeTerm ceil_div(int64_t n, int64_t d) { return n < 0 ? SizeTerm(-1) : SizeTerm(n / d + (n % d != 0)); }

// Bump allocator over a caller's workspace (256-byte aligned pieces).  With
// base == nullptr it only measures, so the size query and the entry points share
// one layout.  `used` becomes -1, and every later piece null, once a piece's
// size is invalid or the total overflows.
struct Carve {
  uint8_t* base;
  int64_t used = 0;
  template <class T>
  T* take(SizeTerm count) {
    const SizeTerm start = SizeTerm(used) + 255;
    const SizeTerm bytes = count * SizeTerm((int64_t)sizeof(T));
    if (!start.ok() || !bytes.ok()) {
      used = -1;
      return nullptr;
    }
    const int64_t off = start.v & ~int64_t(255);
    used = (SizeTerm(off) + bytes).v;
    return (base && used >= 0) ? reinterpret_cast<T*>(base + off) : nullptr;
  }
};

// Workspace bytes of kda_gqa_fwd_f32 (layout owned by attention_f32.hip).
int64_t gqa_f32_workspace_bytes(int64_t batch, int64_t seq, int64_t hq, int64_t hkv);

// ---- device helpers -------------------------------------------------------

// fp32 -> bf16 bits with gfx950's conversion instruction (v_cvt_pk_bf16_f32):
// round to nearest even, fp32 denormals kept (bf16 shares fp32's exponent
// range), overflow to infinity, and a NaN stays a NaN (quieted, sign kept).
typedef float kda_floatx2 __attribute__((ext_vector_type(2)));
typedef __bf16 kda_bf16x2 __attribute__((ext_vector_type(2)));

// Packs two floats into one dword of two bf16 (lo in bits 0..15).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((kda_floatx2{lo, hi}), kda_bf16x2));
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return pack_bf16x2(f, 0.0f) & 0xffffu;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __builtin_bit_cast(float, b << 16);
}

// Splits two floats into their bf16 (hi, lo) limbs, hi = bf16(x) and
// lo = bf16(x - hi), packed in pairs (a in bits 0..15).
__device__ __forceinline__ void split_bf16x2(float a, float b, uint32_t& hi, uint32_t& lo) {
  hi = pack_bf16x2(a, b);
  lo = pack_bf16x2(a - __builtin_bit_cast(float, hi << 16),
                   b - __builtin_bit_cast(float, hi & 0xffff0000u));
}

}  // namespace kda
