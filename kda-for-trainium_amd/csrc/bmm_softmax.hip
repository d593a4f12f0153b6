// Batched matmul + row softmax, fp32 (NKIBench bmm_softmax):
//
//   out[b, m, :] = softmax_n(lhs[b, m, :] @ rhs[b, :, :])      (max-shifted)
//
// lhs [B, M, K], rhs [B, K, N], out [B, M, N] fp32, K <= 64, N % 64 == 0.
//
// Precision.  The softmax turns absolute errors of the scores into relative
// errors of the output, and the scores are O(sqrt(K)) large, so the two-limb
// bf16 split used by the fp32 GEMMs (~1e-5 per product) is not enough.  Both
// operands are split into three bf16 limbs (x = x0 + x1 + x2, residual ~2^-24)
// and each score takes the six products x_i * y_j with i + j <= 2 on bf16 MFMA,
// accumulated in fp32.
//
// Work decomposition.  One workgroup = 128 rows of one batch (8 waves x 16 rows);
// it streams the N axis in 64-column tiles of rhs^T (three bf16 limb planes,
// [N][K] after the pre-pass split_transpose_kernel), DMA'd global->LDS into a
// ring of three buffers and shared by the 8 waves.  Two passes over N:
//   pass 0: online row max and sum of exp (flash-softmax statistics);
//   pass 1: recompute the scores and write exp(s - max) / sum once.
// The output (4 bytes per element) is written exactly once; recomputing the
// K = 64 scores is cheaper than a second pass over the output in HBM.
//
// Per wave and 64-column tile: the MFMA B operand is the 16-row block of lhs
// (held in registers for the whole kernel, split on load), the MFMA A operand a
// 16-column block of rhs^T read from LDS (ds_read_b128, 128-byte rows, chunk c of
// row r at c ^ (r & 7)); lane l then holds row l % 16, columns 4*(l/16) .. +3 of
// each 16x16 block.
#include <math.h>

#include "common.h"

namespace kda {
namespace bmmsm {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kRows = 16 * kWaves;   // rows per workgroup
constexpr int kCols = 64;            // columns per tile
constexpr int kK = 64;               // max contraction (two 32-wide MFMA k steps)
constexpr int kLimbs = 3;
constexpr int kXcds = 8;
constexpr int kPlaneBytes = kCols * kK * 2;           // one limb plane of a tile
constexpr int kTileBytes = kLimbs * kPlaneBytes;      // 24 KiB
constexpr int kDmaPerWave = kTileBytes / 1024 / kWaves;   // 3
constexpr int kStages = 3;                               // tile ring depth
constexpr int kStoresPerTile = 4;                        // store instructions per wave
#define KDA_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

__device__ __forceinline__ void limbs3(float x, uint32_t& b0, uint32_t& b1, uint32_t& b2) {
  b0 = f32_to_bf16_bits(x);
  const float r1 = x - bf16_bits_to_f32(b0);
  b1 = f32_to_bf16_bits(r1);
  const float r2 = r1 - bf16_bits_to_f32(b1);
  b2 = f32_to_bf16_bits(r2);
}

// rhs [B][K][N] fp32 -> three bf16 limb planes of rhs^T, each [B][N][64] (k
// padded with zeros up to 64).  One workgroup per (64-column block, batch).
__global__ __launch_bounds__(256) void split_transpose_kernel(const float* __restrict__ rhs,
                                                              uint16_t* __restrict__ p0,
                                                              uint16_t* __restrict__ p1,
                                                              uint16_t* __restrict__ p2, int k,
                                                              int n) {
  __shared__ float tile[kK][kCols + 1];
  const int n0 = blockIdx.x * kCols;
  const int64_t b = blockIdx.y;
  const float* src = rhs + b * (int64_t)k * n;
  for (int idx = threadIdx.x; idx < kK * kCols; idx += 256) {
    const int r = idx / kCols, c = idx % kCols;   // r = k, c = column (coalesced read)
    tile[r][c] = r < k ? src[(int64_t)r * n + n0 + c] : 0.f;
  }
  __syncthreads();
  const int64_t base = (b * n + n0) * kK;
  for (int idx = threadIdx.x; idx < kK * kCols; idx += 256) {
    const int c = idx / kK, r = idx % kK;         // write k-contiguous
    uint32_t h0, h1, h2;
    limbs3(tile[r][c], h0, h1, h2);
    const int64_t o = base + (int64_t)c * kK + r;
    p0[o] = (uint16_t)h0;
    p1[o] = (uint16_t)h1;
    p2[o] = (uint16_t)h2;
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

__global__ __launch_bounds__(kThreads, 2) void bmm_softmax_kernel(
    const float* __restrict__ lhs, const uint16_t* __restrict__ p0, const uint16_t* __restrict__ p1,
    const uint16_t* __restrict__ p2, float* __restrict__ out, int m, int n, int k) {
  __shared__ __align__(1024) uint8_t lds[kStages][kTileBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Workgroups are dealt round-robin to the 8 XCDs; remap the linear id so each
  // XCD gets a contiguous range of (batch, row block) pairs.  All workgroups of
  // a batch then share one L2, which holds that batch's rhs limb planes
  // (1.5 MiB at N = 4096) for the two passes of every row block.
  const int row_blocks = (m + kRows - 1) / kRows;
  const int total_wg = row_blocks * (int)gridDim.y;
  int pid = blockIdx.y * row_blocks + blockIdx.x;
  const int full = (total_wg / kXcds) * kXcds;
  if (pid < full) pid = (pid % kXcds) * (full / kXcds) + pid / kXcds;
  const int64_t b = pid / row_blocks;
  const int row0 = (pid % row_blocks) * kRows + wave * 16;
  const int nt = n / kCols;
  // Column tiles are visited in a per-workgroup rotated order.  In pass 1 every
  // workgroup writes 256 bytes of each of its rows per tile; with all
  // workgroups on the same column tile the concurrent stores share their low
  // address bits (rows are n*4 bytes apart) and crowd a few HBM channels
  // (measured 20% slower at 16x4096x4096).
  const int rot = (int)((pid * (int64_t)7) % nt);

  // ---- this wave's 16 rows of lhs as MFMA "B" fragments, split into 3 limbs:
  // lane l holds row row0 + l%16, k = kh*32 + 8*(l/16) .. +7
  bf16x8 a[2][kLimbs];
  {
    const int r = min(row0 + (lane & 15), m - 1);
    const float* src = lhs + (b * m + r) * (int64_t)k;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      const int kk = kh * 32 + 8 * (lane >> 4);
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (kk + e < k) ? src[kk + e] : 0.f;
      uint32_t w0[4], w1[4], w2[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        uint32_t x0, x1, x2, y0, y1, y2;
        limbs3(v[e], x0, x1, x2);
        limbs3(v[e + 1], y0, y1, y2);
        w0[e / 2] = x0 | (y0 << 16);
        w1[e / 2] = x1 | (y1 << 16);
        w2[e / 2] = x2 | (y2 << 16);
      }
      a[kh][0] = __builtin_bit_cast(bf16x8, (u32x4{w0[0], w0[1], w0[2], w0[3]}));
      a[kh][1] = __builtin_bit_cast(bf16x8, (u32x4{w1[0], w1[1], w1[2], w1[3]}));
      a[kh][2] = __builtin_bit_cast(bf16x8, (u32x4{w2[0], w2[1], w2[2], w2[3]}));
    }
  }

  // ---- DMA of column tile t (of the N axis) into buffer `buf`: 24 x 1 KiB
  // instructions, 3 per wave; instruction q fills plane q/8, rows (q%8)*8 ..+7
  // (8 lanes per 128-byte row, chunk c of row r stored at c ^ (r & 7)).
  const uint16_t* planes[kLimbs] = {p0, p1, p2};
  const uint32_t lds_base = (uint32_t)(uintptr_t)KDA_LDS_PTR(&lds[0][0]);
  auto issue = [&](int t, int buf) {
    const int c0 = t * kCols;
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) {
      const int q = j * kWaves + wave;
      const int plane = q / 8, qq = q % 8;
      const int r = qq * 8 + lane / 8;
      const int chunk = (lane % 8) ^ (r & 7);
      const uint16_t* src = planes[plane] + ((b * n + c0 + r) * kK + chunk * 8);
      dma16(src, lds_base + buf * kTileBytes + plane * kPlaneBytes + qq * 1024);
    }
  };

  // Scores of the 64-column tile in buffer `buf`: 4 independent 16x16 blocks,
  // issued term by term so consecutive MFMAs never depend on each other.
  auto scores = [&](int buf, floatx4 (&s)[4]) {
    const uint8_t* tile = &lds[buf][0];
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      const int c = kh * 4 + (lane >> 4);
      bf16x8 bt[4][kLimbs];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = j * 16 + (lane & 15);
#pragma unroll
        for (int l = 0; l < kLimbs; ++l)
          bt[j][l] = *reinterpret_cast<const bf16x8*>(tile + l * kPlaneBytes + r * 128 + ((c ^ (r & 7)) << 4));
      }
      // smallest terms first: (2,0) (1,1) (0,2) (1,0) (0,1) (0,0)
      constexpr int kTerm[6][2] = {{0, 2}, {1, 1}, {2, 0}, {0, 1}, {1, 0}, {0, 0}};
#pragma unroll
      for (int t = 0; t < 6; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          s[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bt[j][kTerm[t][0]], a[kh][kTerm[t][1]], s[j],
                                                         0, 0, 0);
    }
  };

  // Software pipeline per tile t (ring of kStages LDS buffers):
  //   wait for this wave's DMA of tile t, barrier (tile t visible everywhere,
  //   buffer (t-1) % kStages free), issue the DMA of tile t+2, store the
  //   probabilities of tile t-1, compute tile t.
  // vmcnt counts loads and stores together and retires in issue order, so the
  // wait for DMA(t) lets the operations issued after it stay in flight: the
  // stores of iteration t-2 and the DMA and stores of iteration t-1.  Stores
  // of the output therefore overlap two further tiles of compute.
  const int total = 2 * nt;   // tiles over both passes
  issue(rot, 0);
  if (total > 1) issue((1 + rot) % nt, 1);
  float m_run = -INFINITY, l_run = 0.f, inv_l = 0.f;
  const int grow = row0 + (lane & 15);
  const bool row_ok = grow < m;
  const bool wave_rows = row0 < m;   // wave-uniform: the wave owns a valid row
  float* orow = out + (b * m + min(grow, m - 1)) * (int64_t)n + 4 * (lane >> 4);
  floatx4 pend[4];            // probabilities of the previous tile (pass 1)
  int pend_col = -1;          // its first column, or -1
  // Returns the number of store instructions issued (wave-uniform).
  auto flush = [&]() -> int {
    int issued = 0;
    if (pend_col >= 0 && wave_rows) {
      if (row_ok) {
        // plain stores: each instruction writes 16 rows x 64 bytes; L2 merges
        // the halves of each 128-byte line (non-temporal 64-byte pieces
        // measured at 3.4 TB/s against 5.5 TB/s for plain stores)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<floatx4*>(orow + pend_col + j * 16) = pend[j];
      }
      issued = kStoresPerTile;   // lane 0's row is valid, so the exec mask is non-empty
    }
    pend_col = -1;
    return issued;
  };
  int st_prev2 = 0, st_prev1 = 0;   // stores issued by iterations t-2 and t-1
  for (int t = 0; t < total; ++t) {
    const int buf = t % kStages;
    // in flight after DMA(t): stores(t-2), DMA(t+1), stores(t-1)
    const int after = st_prev2 + (t + 1 < total ? kDmaPerWave : 0) + st_prev1;
    switch (after) {
      case 11: wait_vmcnt<11>(); break;
      case 8: wait_vmcnt<8>(); break;
      case 7: wait_vmcnt<7>(); break;
      case 4: wait_vmcnt<4>(); break;
      case 3: wait_vmcnt<3>(); break;
      default: wait_vmcnt<0>(); break;
    }
    __builtin_amdgcn_s_barrier();   // tile t visible; buffer (t-1) % kStages free
    asm volatile("" ::: "memory");
    if (t + 2 < total) issue((t + 2 + rot) % nt, (t + 2) % kStages);
    st_prev2 = st_prev1;
    st_prev1 = flush();
    floatx4 s[4];
    scores(buf, s);
    if (t < nt) {
      // pass 0: online statistics; the 4 lanes l, l+16, l+32, l+48 share a row
      float mx = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[j][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) sum += __expf(s[j][r] - m_new);
      l_run = l_run * __expf(m_run - m_new) + sum;
      m_run = m_new;
      if (t + 1 == nt) {
        float l = l_run;
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        inv_l = 1.0f / l;
      }
    } else {
      // pass 1: normalised probabilities, written once (next iteration)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) pend[j][r] = __expf(s[j][r] - m_run) * inv_l;
      pend_col = ((t - nt + rot) % nt) * kCols;
    }
  }
  flush();
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
  if (!workspace || !aligned16(workspace) || ws_bytes < need)
    return set_error(KDA_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned and >= %lld bytes",
                     what, (long long)need);
  hipStream_t st = as_stream(stream);
  const int64_t plane = batch * n * kK;   // elements per limb plane
  uint16_t* q0 = reinterpret_cast<uint16_t*>(workspace);
  uint16_t* q1 = q0 + plane;
  uint16_t* q2 = q1 + plane;
  hipLaunchKernelGGL(split_transpose_kernel, dim3((unsigned)(n / kCols), (unsigned)batch), dim3(256),
                     0, st, rhs, q0, q1, q2, (int)k, (int)n);
  if (int rc = check_launch(what)) return rc;
  hipLaunchKernelGGL(bmm_softmax_kernel, dim3((unsigned)((m + kRows - 1) / kRows), (unsigned)batch),
                     dim3(kThreads), 0, st, lhs, q0, q1, q2, out, (int)m, (int)n, (int)k);
  return check_launch(what);
}
