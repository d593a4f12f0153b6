// Batched matmul + row softmax, fp32 (NKIBench bmm_softmax):
//
//   out[b, m, :] = softmax_n(lhs[b, m, :] @ rhs[b, :, :])      (max-shifted)
//
// lhs [B, M, K], rhs [B, K, N], out [B, M, N] fp32, K <= 64, N % 64 == 0.
//
// Precision.  The softmax turns absolute errors of the scores into relative
// errors of the output, and the scores are O(sqrt(K)) large, so the scores need
// close to fp32 accuracy.  Both operands are scaled by powers of two (each lhs
// row, each 64-column tile of rhs, so that the largest |value| lies in
// [2^13, 2^14)) and split into two fp16 limbs, x = x0 + x1 (22 significant
// bits; fp16 keeps 11 bits per limb against bf16's 8).  A score takes the three
// products x0*y0 + x0*y1 + x1*y0 on fp16 MFMA with fp32 accumulation; the
// dropped x1*y1 and the residual below x1 are ~2^-22 of each product, and the
// scaling is undone exactly by the power-of-two factor of (row, tile).  On the
// NKIBench inputs this matches fp64 scores to within 2% of the error of the
// fp32 reference itself.
//
// Work decomposition.  One workgroup = 256 rows of one batch (8 waves x 2 x 16
// rows); it streams the N axis in 64-column tiles of rhs^T (two fp16 limb
// planes [N][K] and the tile scales, made by split_transpose_kernel), DMA'd
// global->LDS into a ring of three buffers shared by the 8 waves.  Each 16-row
// group makes two passes over N:
//   pass 0: online row max and sum of 2^(s - max) (flash-softmax statistics);
//   pass 1: recompute the scores and write 2^(s - max) / sum once.
// The two groups of a wave run one pass apart over three sweeps of the tiles
// (group 0's statistics; group 0's stores with group 1's statistics; group 1's
// stores), so that stores are in flight during two of the three sweeps.
// The output (4 bytes per element) is written exactly once; recomputing the
// K = 64 scores is cheaper than a second pass over the output in HBM.  Scores
// are kept in log2 units (lhs is multiplied by log2(e) before the split), so
// each exponential is one v_exp_f32.
//
// Per wave and 64-column tile: the MFMA B operand is a 16-row block of lhs
// (held in registers for the whole kernel, split on load), the MFMA A operand a
// 16-column block of rhs^T read from LDS (ds_read_b128, 128-byte rows, chunk c of
// row r at c ^ (r & 7)); lane l then holds row l % 16, columns 4*(l/16) .. +3 of
// each 16x16 block.
#include <math.h>

#include <type_traits>

#include "common.h"
#include "lanes.h"

namespace kda {
namespace bmmsm {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kGroups = 2;                       // 16-row groups per wave
constexpr int kRows = 16 * kGroups * kWaves;     // 256 rows per workgroup
constexpr int kCols = 64;                        // columns per tile
constexpr int kK = 64;                           // max contraction (two 32-wide MFMA k steps)
constexpr int kLimbs = 2;
constexpr int kXcds = 8;
constexpr int kPlaneBytes = kCols * kK * 2;               // one limb plane of a tile
constexpr int kTileBytes = kLimbs * kPlaneBytes;          // 16 KiB
constexpr int kDmaPerWave = kTileBytes / 1024 / kWaves;   // 2
constexpr int kStages = 3;                                // tile ring depth
constexpr int kStores = 4;                                // store instructions per wave and storing step (one group)
constexpr int kTopExp = 13;                               // largest |scaled value| in [2^13, 2^14)
constexpr float kLog2e = 1.44269504088896341f;
#define KDA_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// 2^e for e in [-126, 127], from the exponent bits.
__device__ __forceinline__ float pow2(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

// Exponent of a non-negative float's leading bit, clamped to [-100, 128] so that
// both 2^(kTopExp - e) and 2^(e - kTopExp) stay normal (0 gives -100; inf and
// NaN give 128 and stay non-finite after scaling).
__device__ __forceinline__ int top_exponent(float mx) {
  return max((int)((__float_as_uint(mx) >> 23) & 0xff) - 127, -100);
}

// Two fp16 limbs of x (|x| < 2^14 + rounding): x0 = fp16(x), x1 = fp16(x - x0);
// x - x0 is exact in fp32.
__device__ __forceinline__ void limbs2(float x, _Float16& h0, _Float16& h1) {
  h0 = (_Float16)x;
  h1 = (_Float16)(x - (float)h0);
}

// rhs [B][K][N] fp32 -> two fp16 limb planes of rhs^T * 2^(kTopExp - e), each
// [B][N][64] (k padded with zeros up to 64), and tile_scale[b][tile] =
// 2^(e - kTopExp), where 2^e is the leading power of two of the tile's largest
// |value|.  One workgroup per (64-column tile, batch): 16-byte loads of the
// tile's k-rows into LDS, then each thread writes 16 consecutive k of one column
// as two 16-byte stores per plane (a wave writes 2 KiB contiguous per plane).
__global__ __launch_bounds__(256) void split_transpose_kernel(const float* __restrict__ rhs,
                                                              _Float16* __restrict__ p0,
                                                              _Float16* __restrict__ p1,
                                                              float* __restrict__ tile_scale, int k,
                                                              int n) {
  __shared__ float tile[kK][kCols + 1];   // [k][column], rows padded: conflict-free column reads
  __shared__ float wave_max[4];
  const int n0 = blockIdx.x * kCols;
  const int64_t b = blockIdx.y;
  const float* src = rhs + b * (int64_t)k * n + n0;
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < kK / 16; ++i) {
    const int r = (threadIdx.x >> 4) + 16 * i, c = 4 * (threadIdx.x & 15);   // 16 lanes per 256-byte row
    const floatx4 v = r < k ? *reinterpret_cast<const floatx4*>(src + (int64_t)r * n + c)
                            : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      tile[r][c + e] = v[e];
      mx = fmaxf(mx, fabsf(v[e]));
    }
  }
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
  const int e = top_exponent(mx);
  const float sc = pow2(kTopExp - e);
  if (threadIdx.x == 0) tile_scale[b * (n / kCols) + blockIdx.x] = pow2(e - kTopExp);
  const int c = threadIdx.x >> 2, q = threadIdx.x & 3;   // column, 16-k chunk
  const int64_t o = (b * n + n0 + c) * kK + 16 * q;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    half8 h0, h1;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      _Float16 a0, a1;
      limbs2(tile[16 * q + 8 * hh + j][c] * sc, a0, a1);
      h0[j] = a0;
      h1[j] = a1;
    }
    *reinterpret_cast<half8*>(p0 + o + 8 * hh) = h0;
    *reinterpret_cast<half8*>(p1 + o + 8 * hh) = h1;
  }
}

__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Scaled scores of one 64-column tile for the wave's kGroups x 16 rows:
// s[g][j] lane l = rows 16g + l%16, columns 16j + 4(l/16) .. +3.  The score in
// log2 units is s * row_scale[g] * tile_scale.
using Scores = floatx4[kGroups][4];

// Orders the MFMAs of the next tile between the VALU / transcendental work of
// the current one (N MFMA slots, V vector instructions after each).
template <int N, int V>
__device__ __forceinline__ void interleave() {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
    __builtin_amdgcn_sched_group_barrier(0x402, V, 0);   // VALU | TRANS
  }
}

__global__ __launch_bounds__(kThreads, 1) void bmm_softmax_kernel(
    const float* __restrict__ lhs, const _Float16* __restrict__ p0, const _Float16* __restrict__ p1,
    const float* __restrict__ tile_scale, float* __restrict__ out, int m, int n, int k) {
  __shared__ __align__(1024) uint8_t lds[kStages][kTileBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Workgroups are dealt round-robin to the 8 XCDs; remap the linear id so each
  // XCD gets a contiguous range of (batch, row block) pairs.  All workgroups of
  // a batch then share one L2, which holds that batch's rhs limb planes
  // (1 MiB at N = 4096) for the two passes of every row block.
  const int row_blocks = (m + kRows - 1) / kRows;
  const int total_wg = row_blocks * (int)gridDim.y;
  int pid = blockIdx.y * row_blocks + blockIdx.x;
  const int full = (total_wg / kXcds) * kXcds;
  if (pid < full) pid = (pid % kXcds) * (full / kXcds) + pid / kXcds;
  const int64_t b = pid / row_blocks;
  const int row0 = (pid % row_blocks) * kRows + wave * (16 * kGroups);
  const int nt = n / kCols;
  const float* tscale = tile_scale + b * nt;
  // Column tiles are visited in a per-workgroup rotated order.  In pass 1 every
  // workgroup writes 256 bytes of each of its rows per tile; with all
  // workgroups on the same column tile the concurrent stores share their low
  // address bits (rows are n*4 bytes apart) and crowd a few HBM channels
  // (measured 20% slower at 16x4096x4096).
  const int rot = (int)((pid * (int64_t)7) % nt);

  // ---- the wave's rows of lhs * log2(e), scaled per row, as MFMA "B" fragments
  // in two fp16 limbs: lane l holds row row0 + 16g + l%16, k = kh*32 + 8*(l/16) .. +7.
  // Rows beyond m are clamped to m-1: those lanes recompute row m-1 bit for bit
  // and store the same values into it, which keeps every store unconditional.
  half8 a[kGroups][2][kLimbs];
  float row_scale[kGroups];
  float* orow[kGroups];
#pragma unroll
  for (int g = 0; g < kGroups; ++g) {
    const int r = min(row0 + 16 * g + (lane & 15), m - 1);
    const float* src = lhs + (b * m + r) * (int64_t)k;
    orow[g] = out + (b * m + r) * (int64_t)n + 4 * (lane >> 4);
    float v[2][8];
    float mx = 0.f;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int kk = kh * 32 + 8 * (lane >> 4) + e;
        v[kh][e] = kk < k ? src[kk] * kLog2e : 0.f;
        mx = fmaxf(mx, fabsf(v[kh][e]));
      }
    const int ex = top_exponent(row_max4(mx));
    const float sc = pow2(kTopExp - ex);
    row_scale[g] = pow2(ex - kTopExp);
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        _Float16 h0, h1;
        limbs2(v[kh][e] * sc, h0, h1);
        a[g][kh][0][e] = h0;
        a[g][kh][1][e] = h1;
      }
  }

  // ---- DMA of column tile c (of the N axis) into buffer `buf`: 16 x 1 KiB
  // instructions, 2 per wave; instruction q fills plane q/8, rows (q%8)*8 ..+7
  // (8 lanes per 128-byte row, chunk c of row r stored at c ^ (r & 7)).
  const _Float16* planes[kLimbs] = {p0, p1};
  const uint32_t lds_base = (uint32_t)(uintptr_t)KDA_LDS_PTR(&lds[0][0]);
  auto issue = [&](int c, int buf) {
    const int c0 = c * kCols;
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) {
      const int q = j * kWaves + wave;
      const int plane = q / 8, qq = q % 8;
      const int r = qq * 8 + lane / 8;
      const int chunk = (lane % 8) ^ (r & 7);
      const _Float16* src = planes[plane] + ((b * n + c0 + r) * kK + chunk * 8);
      dma16(src, lds_base + buf * kTileBytes + plane * kPlaneBytes + qq * 1024);
    }
  };

  // Scores of the tile in buffer `buf`: 2 x 4 independent 16x16 blocks, issued
  // term by term so consecutive MFMAs never depend on each other.
  auto scores = [&](int buf, Scores& s, auto gmask) {
    constexpr int GM = decltype(gmask)::value;   // bit g: compute group g
    const uint8_t* tile = &lds[buf][0];
#pragma unroll
    for (int g = 0; g < kGroups; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (GM & (1 << g)) s[g][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      const int c = kh * 4 + (lane >> 4);
      half8 bt[4][kLimbs];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = j * 16 + (lane & 15);
#pragma unroll
        for (int l = 0; l < kLimbs; ++l)
          bt[j][l] = *reinterpret_cast<const half8*>(tile + l * kPlaneBytes + r * 128 + ((c ^ (r & 7)) << 4));
      }
      // smaller terms first: (1,0) (0,1) (0,0)
      constexpr int kTerm[3][2] = {{0, 1}, {1, 0}, {0, 0}};
#pragma unroll
      for (int t = 0; t < 3; ++t)
#pragma unroll
        for (int g = 0; g < kGroups; ++g)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (GM & (1 << g)) s[g][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bt[j][kTerm[t][0]], a[g][kh][kTerm[t][1]],
                                                             s[g][j], 0, 0, 0);
    }
  };

  // pass 0: online row statistics (max, and sum of 2^(s - max) per lane)
  float m_run[kGroups], l_run[kGroups], inv_l[kGroups];
#pragma unroll
  for (int g = 0; g < kGroups; ++g) m_run[g] = -INFINITY, l_run[g] = 0.f;
  auto stats = [&](const Scores& s, float ts, auto gc) {
    constexpr int g = decltype(gc)::value;
    const float c = row_scale[g] * ts;
    float mx = s[g][0][0];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[g][j][r]);
    const float m_new = fmaxf(m_run[g], row_max4(mx) * c);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) sum += __builtin_amdgcn_exp2f(__builtin_fmaf(s[g][j][r], c, -m_new));
    l_run[g] = l_run[g] * __builtin_amdgcn_exp2f(m_run[g] - m_new) + sum;
    m_run[g] = m_new;
  };
  // pass 1: normalised probabilities of column tile col, stored directly
  auto probs = [&](const Scores& s, float ts, int col, auto gc) {
    constexpr int g = decltype(gc)::value;
    const float c = row_scale[g] * ts;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      floatx4 p;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[g][j][r], c, -m_run[g])) * inv_l[g];
      *reinterpret_cast<floatx4*>(orow[g] + col * kCols + j * 16) = p;
    }
  };

  // The two 16-row groups of every wave run one pass apart, so that the stores of
  // one group overlap the statistics pass of the other instead of every
  // workgroup storing only in its second half:
  //   steps [0, nt):      group 0 pass 0 (statistics)
  //   steps [nt, 2nt):    group 0 pass 1 (probabilities, stored) + group 1 pass 0
  //   steps [2nt, 3nt):   group 1 pass 1
  // (step t = column tile (t + rot) % nt).  Software pipeline over the 3*nt steps,
  // ring of kStages LDS buffers.  Iteration t: wait for this wave's DMA of step
  // t+1, barrier (step t+1 visible everywhere; buffer t % kStages, last read by
  // the MFMAs of step t one iteration ago, is free), issue the DMA of step t+3
  // into it, then the MFMAs of step t+1 (only the groups it needs) interleaved
  // with the softmax work of step t, whose scores the previous iteration
  // produced.  vmcnt counts loads and stores together and retires in issue order:
  // after DMA(t+1) come the stores of iteration t-2, DMA(t+2) and the stores of
  // iteration t-1, which may stay in flight (every step from nt on stores one
  // group: kStores instructions).
  const int total = 3 * nt;
  auto col = [&](int t) { return (t + rot) % nt; };
  auto dma_after = [&](int t) {   // operations allowed in flight at iteration t
    return (t - 2 >= nt ? kStores : 0) + (t + 2 < total ? kDmaPerWave : 0) + (t - 1 >= nt ? kStores : 0);
  };
  auto wait_step = [&](int t) {
    switch (dma_after(t)) {
      case 2 * kStores + kDmaPerWave: wait_vmcnt<2 * kStores + kDmaPerWave>(); break;
      case 2 * kStores: wait_vmcnt<2 * kStores>(); break;
      case kStores + kDmaPerWave: wait_vmcnt<kStores + kDmaPerWave>(); break;
      case kStores: wait_vmcnt<kStores>(); break;
      case kDmaPerWave: wait_vmcnt<kDmaPerWave>(); break;
      default: wait_vmcnt<0>(); break;
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (t + 3 < total) issue(col(t + 3), (t + 3) % kStages);
  };

  using G0 = std::integral_constant<int, 0>;
  using G1 = std::integral_constant<int, 1>;
  using M0 = std::integral_constant<int, 1>;    // group 0 only
  using M1 = std::integral_constant<int, 2>;    // group 1 only
  using M01 = std::integral_constant<int, 3>;   // both groups

  issue(col(0), 0);
  issue(col(1), 1);
  issue(col(2), 2);   // total >= 3
  wait_vmcnt<2 * kDmaPerWave>();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  Scores sa, sb;
  scores(0, sa, M0{});
  float ta = tscale[col(0)], tb;

  // One pipeline iteration of each kind; `cur` / `ts` hold step t, `next` /
  // `ts_next` receive step t+1 (for the groups step t+1 needs: NEXT).
  // The empty asm keeps the statistics in the iteration's block: without a use
  // there LLVM sinks them past the next wait's branches, away from the MFMAs
  // they should overlap.
  // (non-generic: an asm statement naming captured arrays does not compile in a
  // generic lambda)
  auto pin_stats0 = [&]() { asm volatile("" ::"v"(m_run[0]), "v"(l_run[0])); };
  auto pin_stats1 = [&]() { asm volatile("" ::"v"(m_run[1]), "v"(l_run[1])); };
  auto step_a = [&](int t, const Scores& cur, float ts, Scores& next, float& ts_next, auto next_mask) {
    wait_step(t);
    ts_next = tscale[col(t + 1)];
    scores((t + 1) % kStages, next, next_mask);
    stats(cur, ts, G0{});
    interleave<24, 2>();
    pin_stats0();
  };
  auto step_m = [&](int t, const Scores& cur, float ts, Scores& next, float& ts_next, auto next_mask) {
    wait_step(t);
    ts_next = tscale[col(t + 1)];
    scores((t + 1) % kStages, next, next_mask);
    probs(cur, ts, col(t), G0{});
    stats(cur, ts, G1{});
    interleave<48, 2>();
    pin_stats1();
  };
  auto step_c = [&](int t, const Scores& cur, float ts, Scores& next, float& ts_next, auto next_mask) {
    wait_step(t);
    ts_next = tscale[col(t + 1)];
    scores((t + 1) % kStages, next, next_mask);
    probs(cur, ts, col(t), G1{});
    interleave<24, 2>();
  };
  // `count` iterations from step t, alternating the score buffers; the current
  // step's scores are in sa on entry and on exit
  int t = 0;
  auto run = [&](auto&& step, int count, auto next_mask) {
    int i = 0;
    for (; i + 1 < count; i += 2, t += 2) {
      step(t, sa, ta, sb, tb, next_mask);
      step(t + 1, sb, tb, sa, ta, next_mask);
    }
    if (i < count) {
      step(t, sa, ta, sb, tb, next_mask);
      ++t;
#pragma unroll
      for (int g = 0; g < kGroups; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) sa[g][j] = sb[g][j];
      ta = tb;
    }
  };
  run(step_a, nt - 1, M0{});
  run(step_a, 1, M01{});          // step nt (both groups) follows
  inv_l[0] = 1.0f / row_sum4(l_run[0]);
  run(step_m, nt - 1, M01{});
  run(step_m, 1, M1{});           // step 2nt (group 1 only) follows
  inv_l[1] = 1.0f / row_sum4(l_run[1]);
  run(step_c, nt - 1, M1{});
  probs(sa, ta, col(t), G1{});    // step 3nt - 1
}

}  // namespace bmmsm
}  // namespace kda

using namespace kda;
using namespace kda::bmmsm;

extern "C" int kda_bmm_softmax_f32(const float* lhs, const float* rhs, float* out, int64_t batch,
                                   int64_t m, int64_t k, int64_t n, void* workspace,
                                   int64_t ws_bytes, void* stream) {
  clear_error();
  const char* what = "bmm_softmax_f32";
  if (batch < 0 || m < 0 || k < 0 || n < 0)
    return set_error(KDA_ERR_INVALID_ARG, "%s: negative size", what);
  if (k > kK || k == 0)
    return set_error(KDA_ERR_UNSUPPORTED, "%s: K=%lld outside 1..%d", what, (long long)k, kK);
  if (n % kCols || n == 0)
    return set_error(KDA_ERR_UNSUPPORTED, "%s: N=%lld must be a positive multiple of %d", what,
                     (long long)n, kCols);
  if (batch > 65535 || m > (1 << 30) || n > (1 << 30) ||
      (m + kRows - 1) / kRows * batch > (int64_t)1 << 30)
    return set_error(KDA_ERR_UNSUPPORTED, "%s: problem too large", what);
  if (batch == 0 || m == 0) return KDA_OK;
  if (!lhs || !rhs || !out) return set_error(KDA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (!aligned16(out)) return set_error(KDA_ERR_INVALID_ARG, "%s: out must be 16-byte aligned", what);
  const int64_t need = kda_workspace_size(KDA_OP_BMM_SOFTMAX_F32, batch, m, k, n, 0);
  if (need < 0 || !workspace || !aligned16(workspace) || ws_bytes < need)
    return set_error(KDA_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned and >= %lld bytes",
                     what, (long long)need);
  hipStream_t st = as_stream(stream);
  const int64_t plane = batch * n * kK;   // elements per limb plane
  _Float16* q0 = reinterpret_cast<_Float16*>(workspace);
  _Float16* q1 = q0 + plane;
  float* tscale = reinterpret_cast<float*>(q1 + plane);   // [B][N/64]
  hipLaunchKernelGGL(split_transpose_kernel, dim3((unsigned)(n / kCols), (unsigned)batch), dim3(256),
                     0, st, rhs, q0, q1, tscale, (int)k, (int)n);
  if (int rc = check_launch(what)) return rc;
  hipLaunchKernelGGL(bmm_softmax_kernel, dim3((unsigned)((m + kRows - 1) / kRows), (unsigned)batch),
                     dim3(kThreads), 0, st, lhs, q0, q1, tscale, out, (int)m, (int)n, (int)k);
  return check_launch(what);
}
