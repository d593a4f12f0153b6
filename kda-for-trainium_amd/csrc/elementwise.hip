// Streaming (HBM-bound) kernels: SiLU, AdamW, half-split RoPE.
//
// Layout: every tensor is a dense fp32 array.  Each thread owns UNROLL 16-byte
// vectors spaced one block apart, so every load instruction of a wavefront
// covers 1 KiB of contiguous memory; the grid covers the array exactly once
// (no grid-stride loop), so all loads of a thread are independent and in
// flight together.  A scalar tail handles n % 4 and unaligned pointers.
#include "common.h"

namespace kda {
namespace {

// Threads per workgroup.  Measured on MI355X: SiLU (2 streams) runs best with
// 256 (128: 2 % slower); AdamW (7 streams) and RoPE (5 streams) with 128
// (256: 8 % and 6 % slower, 64 no better).
constexpr int kBlock = 256;
constexpr int kAdamBlock = 128;
constexpr int kRopeBlock = 128;
// 16-byte vectors per thread (per stream).  Measured on MI355X (SiLU over
// 2 x 64 MiB, a 7-stream AdamW update over 7 x 512 MiB): one vector per thread
// beats 2 and 4 -- more workgroups in flight per CU hide more latency than
// deeper per-thread unrolling does.
constexpr int kUnroll = 1;
constexpr int kAdamUnroll = 1;
constexpr int kRopeUnroll = 1;

__device__ __forceinline__ float silu1(float x) {
  // x * sigmoid(x) = x / (1 + exp(-x)); exp(-x) -> +inf for x < -88 gives -0.
  return __fdividef(x, 1.0f + __expf(-x));
}

__global__ __launch_bounds__(kBlock) void silu_vec_kernel(const floatx4* __restrict__ x,
                                                          floatx4* __restrict__ y, int64_t n4) {
  const int64_t first = (int64_t)blockIdx.x * (kBlock * kUnroll);
  const int64_t base = first + threadIdx.x;
  const auto yw = out_window(y + first, (uint32_t)(min(n4 - first, (int64_t)kBlock * kUnroll) * 16));
  floatx4 v[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + (int64_t)u * kBlock;
    if (i < n4) v[u] = __builtin_nontemporal_load(x + i);
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = base + (int64_t)u * kBlock;
    if (i < n4) {
      floatx4 r;
      r.x = silu1(v[u].x);
      r.y = silu1(v[u].y);
      r.z = silu1(v[u].z);
      r.w = silu1(v[u].w);
      store_sc1_nt(yw, (uint32_t)((i - first) * 16), r);
    }
  }
}

__global__ __launch_bounds__(kBlock) void silu_scalar_kernel(const float* __restrict__ x,
                                                             float* __restrict__ y, int64_t begin,
                                                             int64_t n) {
  const int64_t i = begin + (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) y[i] = silu1(x[i]);
}

// ---------------------------------------------------------------- AdamW

struct AdamParams {
  float decay;         // 1 - lr * weight_decay
  float beta1, one_minus_beta1;
  float beta2, one_minus_beta2;
  float step_size;     // lr / (1 - beta1^step)
  float bc2_sqrt;      // sqrt(1 - beta2^step)
  float eps;
};

__device__ __forceinline__ void adam1(float& p, float g, float& m, float& v, const AdamParams& a) {
  p = p * a.decay;
  m = a.beta1 * m + a.one_minus_beta1 * g;
  v = a.beta2 * v + a.one_minus_beta2 * (g * g);
  const float denom = sqrtf(v) / a.bc2_sqrt + a.eps;
  p = p - a.step_size * (m / denom);
}

template <bool kWriteMoments>
__global__ __launch_bounds__(kAdamBlock) void adamw_vec_kernel(const floatx4* p_in, const floatx4* g_in,
                                                           const floatx4* m_in, const floatx4* v_in,
                                                           floatx4* p_out, floatx4* m_out,
                                                           floatx4* v_out, int64_t n4,
                                                           AdamParams a) {
  // p_out may alias p_in (and m_out/v_out alias m_in/v_in): every element is
  // loaded by the thread that later stores it, and all loads precede all stores.
  const int64_t base = (int64_t)blockIdx.x * (kAdamBlock * kAdamUnroll) + threadIdx.x;
  floatx4 p[kAdamUnroll], g[kAdamUnroll], m[kAdamUnroll], v[kAdamUnroll];
#pragma unroll
  for (int u = 0; u < kAdamUnroll; ++u) {
    const int64_t i = base + (int64_t)u * kAdamBlock;
    if (i < n4) {
      p[u] = __builtin_nontemporal_load(p_in + i);
      g[u] = __builtin_nontemporal_load(g_in + i);
      m[u] = __builtin_nontemporal_load(m_in + i);
      v[u] = __builtin_nontemporal_load(v_in + i);
    }
  }
#pragma unroll
  for (int u = 0; u < kAdamUnroll; ++u) {
    const int64_t i = base + (int64_t)u * kAdamBlock;
    if (i < n4) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float pj = p[u][j], mj = m[u][j], vj = v[u][j];
        adam1(pj, g[u][j], mj, vj, a);
        p[u][j] = pj;
        m[u][j] = mj;
        v[u][j] = vj;
      }
      __builtin_nontemporal_store(p[u], p_out + i);
      if (kWriteMoments) {
        __builtin_nontemporal_store(m[u], m_out + i);
        __builtin_nontemporal_store(v[u], v_out + i);
      }
    }
  }
}

__global__ __launch_bounds__(kAdamBlock) void adamw_scalar_kernel(const float* p_in, const float* g_in,
                                                              const float* m_in, const float* v_in,
                                                              float* p_out, float* m_out,
                                                              float* v_out, int64_t begin,
                                                              int64_t n, AdamParams a) {
  const int64_t i = begin + (int64_t)blockIdx.x * kAdamBlock + threadIdx.x;
  if (i >= n) return;
  float p = p_in[i], m = m_in[i], v = v_in[i];
  adam1(p, g_in[i], m, v, a);
  p_out[i] = p;
  if (m_out) m_out[i] = m;
  if (v_out) v_out[i] = v;
}

// ---------------------------------------------------------------- RoPE

// The reference rounds each product and then the sum (numpy, no FMA); keep
// that exact order so results are bit-identical.
#pragma clang fp contract(off)
__device__ __forceinline__ void rope1(float x0, float x1, float c, float s, float& o0, float& o1) {
  const float a = x0 * c, b = x1 * s;
  o0 = a - b;
  const float e = x0 * s, f = x1 * c;
  o1 = e + f;
}
#pragma clang fp contract(on)

// grid: (ceil(s4 / (kRopeBlock*kRopeUnroll)), D/2).  Row d of the lower half pairs with row
// d + D/2 of the upper half; cos/sin rows are shared by both outputs.
__global__ __launch_bounds__(kRopeBlock) void rope_vec_kernel(const floatx4* __restrict__ x,
                                                          const floatx4* __restrict__ cs,
                                                          const floatx4* __restrict__ sn,
                                                          floatx4* __restrict__ out,
                                                          int64_t half, int64_t s4) {
  const int64_t d = blockIdx.y;
  const int64_t base = (int64_t)blockIdx.x * (kRopeBlock * kRopeUnroll) + threadIdx.x;
  const floatx4* x0p = x + d * s4;
  const floatx4* x1p = x + (d + half) * s4;
  const floatx4* cp = cs + d * s4;
  const floatx4* sp = sn + d * s4;
  floatx4* o0p = out + d * s4;
  floatx4* o1p = out + (d + half) * s4;
  floatx4 a[kRopeUnroll], b[kRopeUnroll], c[kRopeUnroll], s[kRopeUnroll];
#pragma unroll
  for (int u = 0; u < kRopeUnroll; ++u) {
    const int64_t i = base + (int64_t)u * kRopeBlock;
    if (i < s4) {
      a[u] = __builtin_nontemporal_load(x0p + i);
      b[u] = __builtin_nontemporal_load(x1p + i);
      c[u] = __builtin_nontemporal_load(cp + i);
      s[u] = __builtin_nontemporal_load(sp + i);
    }
  }
#pragma unroll
  for (int u = 0; u < kRopeUnroll; ++u) {
    const int64_t i = base + (int64_t)u * kRopeBlock;
    if (i < s4) {
      floatx4 r0, r1;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float o0, o1;
        rope1(a[u][j], b[u][j], c[u][j], s[u][j], o0, o1);
        r0[j] = o0;
        r1[j] = o1;
      }
      __builtin_nontemporal_store(r0, o0p + i);
      __builtin_nontemporal_store(r1, o1p + i);
    }
  }
}

__global__ __launch_bounds__(kRopeBlock) void rope_scalar_kernel(const float* x, const float* cs,
                                                             const float* sn, float* out,
                                                             int64_t half, int64_t s) {
  const int64_t d = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * kRopeBlock + threadIdx.x;
  if (i >= s) return;
  float o0, o1;
  rope1(x[d * s + i], x[(d + half) * s + i], cs[d * s + i], sn[d * s + i], o0, o1);
  out[d * s + i] = o0;
  out[(d + half) * s + i] = o1;
}

inline unsigned blocks_for(int64_t items, int64_t per_block) {
  return (unsigned)((items + per_block - 1) / per_block);
}

}  // namespace
}  // namespace kda

using namespace kda;

extern "C" int kda_silu_f32(const float* x, float* y, int64_t n, void* stream) {
  clear_error();
  if (n < 0) return set_error(KDA_ERR_INVALID_ARG, "silu: n=%lld < 0", (long long)n);
  if (n == 0) return KDA_OK;
  if (!x || !y) return set_error(KDA_ERR_INVALID_ARG, "silu: null pointer");
  hipStream_t st = as_stream(stream);
  int64_t vec_end = 0;
  if (aligned16(x) && aligned16(y)) {
    const int64_t n4 = n / 4;
    vec_end = n4 * 4;
    if (n4 > 0) {
      const int64_t per_block = (int64_t)kBlock * kUnroll;
      if (blocks_for(n4, per_block) > 0x7fffffffu)
        return set_error(KDA_ERR_UNSUPPORTED, "silu: n=%lld too large", (long long)n);
      hipLaunchKernelGGL(silu_vec_kernel, dim3(blocks_for(n4, per_block)), dim3(kBlock), 0, st,
                         reinterpret_cast<const floatx4*>(x), reinterpret_cast<floatx4*>(y), n4);
    }
  }
  if (vec_end < n)
    hipLaunchKernelGGL(silu_scalar_kernel, dim3(blocks_for(n - vec_end, kBlock)), dim3(kBlock), 0,
                       st, x, y, vec_end, n);
  return check_launch("silu");
}

extern "C" int kda_adamw_f32(const float* param_in, const float* grad, const float* m_in,
                             const float* v_in, float* param_out, float* m_out, float* v_out,
                             int64_t n, float lr, float beta1, float beta2, float eps,
                             float weight_decay, int64_t step, void* stream) {
  clear_error();
  if (n < 0) return set_error(KDA_ERR_INVALID_ARG, "adamw: n=%lld < 0", (long long)n);
  if (step < 1) return set_error(KDA_ERR_INVALID_ARG, "adamw: step=%lld < 1", (long long)step);
  if (!(beta1 >= 0.f && beta1 < 1.f) || !(beta2 >= 0.f && beta2 < 1.f))
    return set_error(KDA_ERR_INVALID_ARG, "adamw: betas must lie in [0, 1)");
  if ((m_out == nullptr) != (v_out == nullptr))
    return set_error(KDA_ERR_INVALID_ARG, "adamw: m_out and v_out must both be set or both NULL");
  if (n == 0) return KDA_OK;
  if (!param_in || !grad || !m_in || !v_in || !param_out)
    return set_error(KDA_ERR_INVALID_ARG, "adamw: null pointer");

  AdamParams a;
  a.decay = 1.0f - lr * weight_decay;
  a.beta1 = beta1;
  a.one_minus_beta1 = 1.0f - beta1;
  a.beta2 = beta2;
  a.one_minus_beta2 = 1.0f - beta2;
  // Bias corrections in double, rounded once, as the host-side scalars of the
  // reference optimizer are python floats.
  const double bc1 = 1.0 - pow((double)beta1, (double)step);
  const double bc2 = 1.0 - pow((double)beta2, (double)step);
  a.step_size = (float)((double)lr / bc1);
  a.bc2_sqrt = (float)sqrt(bc2);
  a.eps = eps;

  hipStream_t st = as_stream(stream);
  const bool moments = m_out != nullptr;
  int64_t vec_end = 0;
  const bool al = aligned16(param_in) && aligned16(grad) && aligned16(m_in) && aligned16(v_in) &&
                  aligned16(param_out) && (!moments || (aligned16(m_out) && aligned16(v_out)));
  if (al) {
    const int64_t n4 = n / 4;
    vec_end = n4 * 4;
    if (n4 > 0) {
      const int64_t per_block = (int64_t)kAdamBlock * kAdamUnroll;
      if (blocks_for(n4, per_block) > 0x7fffffffu)
        return set_error(KDA_ERR_UNSUPPORTED, "adamw: n=%lld too large", (long long)n);
      auto P = [](const float* q) { return reinterpret_cast<const floatx4*>(q); };
      auto Q = [](float* q) { return reinterpret_cast<floatx4*>(q); };
      if (moments)
        hipLaunchKernelGGL(adamw_vec_kernel<true>, dim3(blocks_for(n4, per_block)), dim3(kAdamBlock), 0,
                           st, P(param_in), P(grad), P(m_in), P(v_in), Q(param_out), Q(m_out),
                           Q(v_out), n4, a);
      else
        hipLaunchKernelGGL(adamw_vec_kernel<false>, dim3(blocks_for(n4, per_block)), dim3(kAdamBlock),
                           0, st, P(param_in), P(grad), P(m_in), P(v_in), Q(param_out), nullptr,
                           nullptr, n4, a);
    }
  }
  if (vec_end < n)
    hipLaunchKernelGGL(adamw_scalar_kernel, dim3(blocks_for(n - vec_end, kAdamBlock)), dim3(kAdamBlock), 0,
                       st, param_in, grad, m_in, v_in, param_out, m_out, v_out, vec_end, n, a);
  return check_launch("adamw");
}

extern "C" int kda_rope_f32(const float* x, const float* cos_t, const float* sin_t, float* out,
                            int64_t d, int64_t s, void* stream) {
  clear_error();
  if (d <= 0 || (d & 1) || s < 0)
    return set_error(KDA_ERR_INVALID_ARG, "rope: need even D > 0 and S >= 0 (got D=%lld S=%lld)",
                     (long long)d, (long long)s);
  if (d / 2 > 65535)
    return set_error(KDA_ERR_UNSUPPORTED, "rope: D=%lld too large", (long long)d);
  if (s == 0) return KDA_OK;
  if (!x || !cos_t || !sin_t || !out) return set_error(KDA_ERR_INVALID_ARG, "rope: null pointer");
  hipStream_t st = as_stream(stream);
  const int64_t half = d / 2;
  const bool vec = (s % 4 == 0) && aligned16(x) && aligned16(cos_t) && aligned16(sin_t) &&
                   aligned16(out);
  if (vec) {
    const int64_t s4 = s / 4;
    hipLaunchKernelGGL(rope_vec_kernel, dim3(blocks_for(s4, kRopeBlock * kRopeUnroll), (unsigned)half),
                       dim3(kRopeBlock), 0, st, reinterpret_cast<const floatx4*>(x),
                       reinterpret_cast<const floatx4*>(cos_t),
                       reinterpret_cast<const floatx4*>(sin_t), reinterpret_cast<floatx4*>(out), half,
                       s4);
  } else {
    hipLaunchKernelGGL(rope_scalar_kernel, dim3(blocks_for(s, kRopeBlock), (unsigned)half),
                       dim3(kRopeBlock), 0, st, x, cos_t, sin_t, out, half, s);
  }
  return check_launch("rope");
}
