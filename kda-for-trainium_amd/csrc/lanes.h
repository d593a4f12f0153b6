// Cross-lane reductions over the four lanes that share a row of a 16x16 MFMA
// result tile (lanes l, l^16, l^32, l^48), with the gfx950 permlane swaps.
//
// v_permlane32_swap_b32 a, b exchanges lanes 32..63 of a with lanes 0..31 of b;
// v_permlane16_swap_b32 a, b exchanges the odd 16-lane rows of a with the even
// rows of b.  Started from two copies of x, a and b then hold x[l] and x[l^32]
// (x[l^16]) in some order, so max(a, b) / a + b combine the pair on every lane.
//
// The swaps are inline asm: the compiler folds fmaxf(r[0], r[1]) of
// __builtin_amdgcn_permlane32_swap(x, x, ...) into a copy of r[0], which drops
// the exchanged half (seen in the generated code of this ROCm release).  The
// s_nop covers the two wait states a permlane swap needs after a VALU write of
// its operands.
#pragma once

namespace kda {

__device__ __forceinline__ void permlane32_swap(float& a, float& b) {
  asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

__device__ __forceinline__ void permlane16_swap(float& a, float& b) {
  asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

__device__ __forceinline__ float row_max4(float x) {
  float a = x, b = x;
  permlane32_swap(a, b);
  x = fmaxf(a, b);
  a = x, b = x;
  permlane16_swap(a, b);
  return fmaxf(a, b);
}

__device__ __forceinline__ float row_sum4(float x) {
  float a = x, b = x;
  permlane32_swap(a, b);
  x = a + b;
  a = x, b = x;
  permlane16_swap(a, b);
  return a + b;
}

}  // namespace kda
