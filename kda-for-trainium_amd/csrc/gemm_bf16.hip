// bf16 GEMM family on gfx950 MFMA (v_mfma_f32_16x16x32_bf16), fp32 accumulation.
//
//   C[M,N] = A[M,K] @ B[K,N]        A, B, C row-major bf16
//
// Variants (template `Mode`):
//   kPlain    C = A @ B
//   kRmsNorm  C = (A * rsqrt(mean_k(A^2) + eps) * gamma) @ B.  The per-row sum of
//             squares is accumulated from the A tiles as they stream through the
//             workgroup (every workgroup sees its rows' full K), gamma scales the
//             rows of each B tile while it is staged into LDS, and the per-row
//             rsqrt is applied to the fp32 accumulators in the epilogue.  One
//             kernel, no extra HBM traffic.
//   kSwiGLU   H = silu(A @ Bg) * (A @ Bu): two B operands share each A tile; the
//             epilogue applies silu(gate) * up and stores H.
//
// Tiling: one 256-thread workgroup (4 waves, 2x2) per BM x BN output tile; each
// wave owns a (BM/2) x (BN/2) sub-tile held in MFMA accumulators.  K advances in
// BK=64 steps through a double-buffered LDS ring: while the MFMAs consume stage
// s, the next K-step is already in flight from HBM into registers and is
// written to stage s^1 afterwards (one barrier per K-step).
//
// LDS layout: both operands are stored K-contiguous ([row][64] bf16, 128 B per
// row) so one ds_read_b128 yields an MFMA fragment (8 consecutive k).  The 16 B
// chunk index within a row is XOR-swizzled with (row & 7), which makes the
// fragment reads (8 consecutive rows, same chunk) and the staging writes hit
// distinct banks.  A is copied as-is; B arrives N-contiguous from HBM and is
// transposed in registers (4 k-rows x 8 n per thread, v_perm_b32 or, with the
// gamma scale, v_cvt_pk_bf16_f32) before its LDS write.
//
// MFMA operand order: the B fragment is passed as the MFMA "A" operand and the
// A fragment as "B", so each lane's 4 accumulators are 4 consecutive columns of
// one output row -> one 8-byte store per lane per 16x16 sub-tile.
//
// Workgroup -> tile mapping: workgroups are dealt round-robin to the 8 XCDs, so
// consecutive tile ids are remapped to land on the same XCD (sharing its L2),
// then ordered in groups of kGroupM tile-rows so concurrently running tiles
// reuse the same A rows and B columns.
#include "common.h"

namespace kda {
namespace gemm {

enum class Mode { kPlain, kRmsNorm, kSwiGLU };

constexpr int kThreads = 256;
constexpr int BK = 64;        // K per stage (bf16 elements)
constexpr int kGroupM = 8;    // tile-rows per scheduling group
constexpr int kXcds = 8;

struct Args {
  const uint16_t* a;      // [M][K]
  const uint16_t* b;      // [K][N]  (gate weights for SwiGLU)
  const uint16_t* b2;     // [K][N]  up weights (SwiGLU only)
  const uint16_t* gamma;  // [K]     (RmsNorm only)
  uint16_t* c;            // [M][N]
  int m, n, k;
  float eps;
};

__device__ __forceinline__ int swz(int row, int chunk) { return chunk ^ (row & 7); }

// Maps a linear workgroup id to (tile_m, tile_n): XCD-contiguous, grouped by rows.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int pid = blockIdx.x;
  const int full = (total / kXcds) * kXcds;
  if (pid < full) pid = (pid % kXcds) * (full / kXcds) + pid / kXcds;
  const int per_group = kGroupM * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * kGroupM;
  const int gsize = min(tiles_m - first_m, kGroupM);
  const int local = pid - group * per_group;
  tm = first_m + local % gsize;
  tn = local / gsize;
}

__device__ __forceinline__ float silu_f(float x) { return __fdividef(x, 1.0f + __expf(-x)); }

template <int BM, int BN, int NB, Mode MODE, bool CHECK>
__global__ __launch_bounds__(kThreads, 1) void gemm_bf16_kernel(Args p) {
  static_assert(NB == 1 || NB == 2, "one or two B operands");
  static_assert(BM % 32 == 0 && BN % 32 == 0, "tile");
  constexpr int WM = BM / 2, WN = BN / 2;          // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;        // 16x16 sub-tiles per wave
  constexpr int A_PASSES = BM / 32;                // 16B A chunks per thread per stage
  constexpr int B_UNITS = NB * 2 * BN / kThreads;  // (4k x 8n) B units per thread
  static_assert(B_UNITS >= 1 && (NB * 2 * BN) % kThreads == 0, "B unit split");
  constexpr int A_STAGE = BM * BK;                 // bf16 elements
  constexpr int B_STAGE = BN * BK;

  extern __shared__ __align__(16) uint16_t smem[];
  uint16_t* As = smem;                             // [2][BM][BK]
  uint16_t* Bs = smem + 2 * A_STAGE;               // [2][NB][BN][BK]
  __shared__ float s_inv_rms[MODE == Mode::kRmsNorm ? BM : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int tiles_m = (p.m + BM - 1) / BM, tiles_n = (p.n + BN - 1) / BN;
  int tm, tn;
  tile_coords(tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int K = p.k, N = p.n, M = p.m;
  const int ktiles = (K + BK - 1) / BK;

  // ---- per-thread staging assignment
  const int a_chunk = tid & 7;           // 16B chunk (8 k) within the BK row
  const int a_row0 = tid >> 3;           // + 32 * pass
  u32x4 a_reg[A_PASSES];
  u32x4 b_reg[B_UNITS][4];
  float ssq[MODE == Mode::kRmsNorm ? A_PASSES : 1];
  if constexpr (MODE == Mode::kRmsNorm) {
#pragma unroll
    for (int i = 0; i < A_PASSES; ++i) ssq[i] = 0.f;
  }

  auto load_a = [&](int kt) {
    const int kk = kt * BK + a_chunk * 8;
#pragma unroll
    for (int i = 0; i < A_PASSES; ++i) {
      const int row = a_row0 + 32 * i;
      const int gm = m0 + row;
      if (!CHECK || (gm < M && kk < K)) {
        a_reg[i] = *reinterpret_cast<const u32x4*>(p.a + (size_t)gm * K + kk);
      } else {
        a_reg[i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto load_b = [&](int kt) {
#pragma unroll
    for (int u = 0; u < B_UNITS; ++u) {
      const int unit = tid + u * kThreads;
      const int which = unit / (2 * BN);
      const int kq = unit & 15;
      const int nc = (unit % (2 * BN)) >> 4;
      const uint16_t* src = (NB == 2 && which) ? p.b2 : p.b;
      const int gn = n0 + nc * 8;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int gk = kt * BK + kq * 4 + r;
        if (!CHECK || (gk < K && gn < N)) {
          b_reg[u][r] = *reinterpret_cast<const u32x4*>(src + (size_t)gk * N + gn);
        } else {
          b_reg[u][r] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
  };

  auto store_a = [&](int stage) {
    uint16_t* dst = As + stage * A_STAGE;
#pragma unroll
    for (int i = 0; i < A_PASSES; ++i) {
      const int row = a_row0 + 32 * i;
      if constexpr (MODE == Mode::kRmsNorm) {
        // fp32 sum of squares of the 8 bf16 values (exact widening + FMA).
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float lo = __builtin_bit_cast(float, a_reg[i][w] << 16);
          const float hi = __builtin_bit_cast(float, a_reg[i][w] & 0xffff0000u);
          ssq[i] = fmaf(lo, lo, ssq[i]);
          ssq[i] = fmaf(hi, hi, ssq[i]);
        }
      }
      *reinterpret_cast<u32x4*>(dst + row * BK + swz(row, a_chunk) * 8) = a_reg[i];
    }
  };

  auto store_b = [&](int stage, int kt) {
#pragma unroll
    for (int u = 0; u < B_UNITS; ++u) {
      const int unit = tid + u * kThreads;
      const int which = unit / (2 * BN);
      const int kq = unit & 15;
      const int nc = (unit % (2 * BN)) >> 4;
      uint16_t* dst = Bs + (stage * NB + which) * B_STAGE;
      float g[4];
      if constexpr (MODE == Mode::kRmsNorm) {
        const int gk = kt * BK + kq * 4;
        if (!CHECK || gk < K) {
          const u32x2 gb = *reinterpret_cast<const u32x2*>(p.gamma + gk);
          g[0] = __builtin_bit_cast(float, gb[0] << 16);
          g[1] = __builtin_bit_cast(float, gb[0] & 0xffff0000u);
          g[2] = __builtin_bit_cast(float, gb[1] << 16);
          g[3] = __builtin_bit_cast(float, gb[1] & 0xffff0000u);
        } else {
          g[0] = g[1] = g[2] = g[3] = 0.f;
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int n = nc * 8 + j;
        const int w = j >> 1;
        u32x2 out;
        if constexpr (MODE == Mode::kRmsNorm) {
          float f[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t bits = (j & 1) ? (b_reg[u][r][w] & 0xffff0000u) : (b_reg[u][r][w] << 16);
            f[r] = __builtin_bit_cast(float, bits) * g[r];
          }
          typedef float floatx2 __attribute__((ext_vector_type(2)));
          typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
          out[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{f[0], f[1]}), bf16x2));
          out[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{f[2], f[3]}), bf16x2));
        } else {
          const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
          out[0] = __builtin_amdgcn_perm(b_reg[u][1][w], b_reg[u][0][w], sel);
          out[1] = __builtin_amdgcn_perm(b_reg[u][3][w], b_reg[u][2][w], sel);
        }
        *reinterpret_cast<u32x2*>(dst + n * BK + swz(n, kq >> 1) * 8 + (kq & 1) * 4) = out;
      }
    }
  };

  floatx4 acc[NB][TM][TN];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[b][i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // ---- prologue: stage 0
  load_a(0);
  load_b(0);
  store_a(0);
  store_b(0, 0);
  __syncthreads();

  const int frag_row = lane & 15;
  const int frag_chunk = lane >> 4;   // 0..3 within a 32-k half

  for (int kt = 0; kt < ktiles; ++kt) {
    const int stage = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) {
      load_a(kt + 1);
      load_b(kt + 1);
    }
    const uint16_t* as = As + stage * A_STAGE;
    const uint16_t* bs = Bs + stage * NB * B_STAGE;
#pragma unroll
    for (int kh = 0; kh < BK / 32; ++kh) {
      const int chunk = kh * 4 + frag_chunk;
      bf16x8 af[TM];
      bf16x8 bfr[NB][TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int row = wm * WM + i * 16 + frag_row;
        af[i] = *reinterpret_cast<const bf16x8*>(as + row * BK + swz(row, chunk) * 8);
      }
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int row = wn * WN + j * 16 + frag_row;
          bfr[b][j] = *reinterpret_cast<const bf16x8*>(bs + b * B_STAGE + row * BK + swz(row, chunk) * 8);
        }
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[b][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[b][j], af[i], acc[b][i][j], 0, 0, 0);
    }
    if (more) {
      store_a(stage ^ 1);
      store_b(stage ^ 1, kt + 1);
    }
    __syncthreads();
  }

  // ---- RMSNorm: reduce the per-row sums of squares (8 lanes share a row)
  if constexpr (MODE == Mode::kRmsNorm) {
    const float inv_k = 1.0f / (float)K;
#pragma unroll
    for (int i = 0; i < A_PASSES; ++i) {
      float s = ssq[i];
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      s += __shfl_xor(s, 4);
      if (a_chunk == 0) s_inv_rms[a_row0 + 32 * i] = 1.0f / sqrtf(s * inv_k + p.eps);
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds C[row][col..col+3]
  const int col_in = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int row = wm * WM + i * 16 + frag_row;
    const int gm = m0 + row;
    float scale = 1.0f;
    if constexpr (MODE == Mode::kRmsNorm) scale = s_inv_rms[row];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int gn = n0 + wn * WN + j * 16 + col_in;
      if (CHECK && (gm >= M || gn >= N)) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (MODE == Mode::kSwiGLU) {
          v[r] = silu_f(acc[0][i][j][r]) * acc[NB - 1][i][j][r];
        } else {
          v[r] = acc[0][i][j][r] * scale;
        }
      }
      typedef float floatx2 __attribute__((ext_vector_type(2)));
      typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
      u32x2 o;
      o[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{v[0], v[1]}), bf16x2));
      o[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{v[2], v[3]}), bf16x2));
      *reinterpret_cast<u32x2*>(p.c + (size_t)gm * N + gn) = o;
    }
  }
}

template <int BM, int BN, int NB, Mode MODE>
int launch(const Args& a, hipStream_t st, const char* what) {
  const int tiles = ((a.m + BM - 1) / BM) * ((a.n + BN - 1) / BN);
  const size_t lds = (size_t)2 * (BM + NB * BN) * BK * sizeof(uint16_t);
  const bool full = (a.m % BM == 0) && (a.n % BN == 0) && (a.k % BK == 0);
  // Opt in to > 64 KiB of dynamic LDS once per instantiation (process-wide;
  // the attribute is per function, not per device).
  static const bool attr_ok = [&] {
    const hipError_t e1 = hipFuncSetAttribute(
        reinterpret_cast<const void*>(gemm_bf16_kernel<BM, BN, NB, MODE, false>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    const hipError_t e2 = hipFuncSetAttribute(
        reinterpret_cast<const void*>(gemm_bf16_kernel<BM, BN, NB, MODE, true>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    return e1 == hipSuccess && e2 == hipSuccess;
  }();
  if (!attr_ok) return set_error(KDA_ERR_HIP, "%s: cannot reserve %zu bytes of LDS", what, lds);
  if (full)
    hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, NB, MODE, false>), dim3(tiles), dim3(kThreads),
                       lds, st, a);
  else
    hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, NB, MODE, true>), dim3(tiles), dim3(kThreads),
                       lds, st, a);
  return check_launch(what);
}

int validate(const char* what, const void* a, const void* b, const void* c, int64_t m,
             int64_t n, int64_t k) {
  if (m < 0 || n < 0 || k < 0)
    return set_error(KDA_ERR_INVALID_ARG, "%s: negative size (M=%lld N=%lld K=%lld)", what,
                     (long long)m, (long long)n, (long long)k);
  if (m > (1 << 30) || n > (1 << 30) || k > (1 << 30) || (m * k) > (int64_t(1) << 40))
    return set_error(KDA_ERR_UNSUPPORTED, "%s: size too large", what);
  if ((k % 8) || (n % 8))
    return set_error(KDA_ERR_UNSUPPORTED,
                     "%s: K (%lld) and N (%lld) must be multiples of 8 (16-byte rows)", what,
                     (long long)k, (long long)n);
  if (m && n && (!a || !b || !c)) return set_error(KDA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (!aligned16(a) || !aligned16(b) || !aligned16(c))
    return set_error(KDA_ERR_INVALID_ARG, "%s: pointers must be 16-byte aligned", what);
  return KDA_OK;
}

}  // namespace gemm
}  // namespace kda

using namespace kda;
using namespace kda::gemm;

extern "C" int kda_matmul_bf16(const kda_bf16* a, const kda_bf16* b, kda_bf16* c, int64_t m,
                               int64_t k, int64_t n, void* stream) {
  clear_error();
  if (int rc = validate("matmul_bf16", a, b, c, m, n, k)) return rc;
  if (m == 0 || n == 0) return KDA_OK;
  Args p{a, b, nullptr, nullptr, c, (int)m, (int)n, (int)k, 0.f};
  return launch<256, 128, 1, Mode::kPlain>(p, as_stream(stream), "matmul_bf16");
}

extern "C" int kda_rmsnorm_matmul_bf16(const kda_bf16* x, const kda_bf16* gamma, const kda_bf16* w,
                                       kda_bf16* y, int64_t m, int64_t k, int64_t n, float eps,
                                       void* stream) {
  clear_error();
  if (int rc = validate("rmsnorm_matmul_bf16", x, w, y, m, n, k)) return rc;
  if (k == 0) return set_error(KDA_ERR_INVALID_ARG, "rmsnorm_matmul_bf16: K must be > 0");
  if (!gamma || (reinterpret_cast<uintptr_t>(gamma) & 7))
    return set_error(KDA_ERR_INVALID_ARG, "rmsnorm_matmul_bf16: gamma null or not 8-byte aligned");
  if (!(eps >= 0.f)) return set_error(KDA_ERR_INVALID_ARG, "rmsnorm_matmul_bf16: eps must be >= 0");
  if (m == 0 || n == 0) return KDA_OK;
  Args p{x, w, nullptr, gamma, y, (int)m, (int)n, (int)k, eps};
  return launch<256, 128, 1, Mode::kRmsNorm>(p, as_stream(stream), "rmsnorm_matmul_bf16");
}

extern "C" int kda_swiglu_bf16(const kda_bf16* x, const kda_bf16* w_up, const kda_bf16* w_down,
                               const kda_bf16* w_gate, kda_bf16* h, kda_bf16* y, int64_t m,
                               int64_t k, int64_t f, void* stream) {
  clear_error();
  if (int rc = validate("swiglu_bf16(up/gate)", x, w_gate, h, m, f, k)) return rc;
  if (int rc = validate("swiglu_bf16(down)", h, w_down, y, m, k, f)) return rc;
  if (!w_up || !aligned16(w_up))
    return set_error(KDA_ERR_INVALID_ARG, "swiglu_bf16: w_up null or misaligned");
  if (m == 0 || k == 0) return KDA_OK;
  hipStream_t st = as_stream(stream);
  Args up{x, w_gate, w_up, nullptr, h, (int)m, (int)f, (int)k, 0.f};
  if (int rc = launch<256, 64, 2, Mode::kSwiGLU>(up, st, "swiglu_bf16(up/gate)")) return rc;
  Args down{h, w_down, nullptr, nullptr, y, (int)m, (int)k, (int)f, 0.f};
  return launch<256, 128, 1, Mode::kPlain>(down, st, "swiglu_bf16(down)");
}
