// Grouped-query attention forward for fp32 q/k/v (NKIBench gqa_full) on gfx950
// fp16 MFMA, flash style: scores never leave the chip, fp32 online softmax.
//
//   out[b, h, s, :] = softmax_j(q[b, s, h, :] . k[b, j, h/G, :] * scale) @ v[b, j, h/G, :]
//   (G = Hq / Hkv query heads per kv head; causal: keys j > s masked; output strides free)
//
// Precision.  The fp32 gate (relative L2 <= 1e-5) rules out bf16 operands.  Each
// operand is scaled by a power of two and split into two fp16 limbs,
// x = x0 + x1 (22 significant bits), and every product takes the three terms
// x0*y0 + x0*y1 + x1*y0 with fp32 accumulation; the dropped x1*y1 and the
// residual below x1 are ~2^-22 of each product.  Scales: q per row (its largest
// |value| in [2^13, 2^14)), k per 64-key tile, v per kv head (the PV sum runs
// over all tiles, so its scale must not change between tiles); the
// probabilities p <= 2^kLazy are multiplied by 2^6 before their split.  All
// scales are undone exactly: q's and k's in the per-(row, tile) score factor,
// v's and p's at the end.  On the NKIBench inputs this matches fp64 attention
// as closely as the fp32 reference does (rel-L2 5.6e-7 against 5.4e-7).
//
// Pre-passes (k_split_kernel, v_split_kernel) write the K and V limb planes in
// the input layout [B][S][Hkv][D] plus their scales into the caller's
// workspace; q is split by the attention kernel itself as it loads it (once per
// wave; a q pre-pass cost 11 us of 373 at the NKIBench shape).
//
// Work decomposition: one workgroup = (batch b, kv head, HPW of its query heads,
// block of 256 / HPW queries), HPW the largest power of two up to 8 dividing G;
// its 8 waves are the HPW heads x 8 / HPW blocks of 32 query rows, so each K/V
// tile staged in LDS serves 256 query rows (the NKIBench G = 2: 2 heads x 128
// queries).
// K and V tiles of 64 keys (both limbs, 32 KiB each) go global->LDS by DMA
// through 2-slot rings and are read with the same fragment scheme as the bf16
// kernel: K [key][d] with 16-byte chunk c of row r at c ^ kswz(r), rows read in
// a permuted order so each lane's 8 probabilities per 32-key chunk are 8
// consecutive keys (the B operand of O^T += V^T P^T without an LDS round trip);
// V [key][d] read transposed (ds_read_b64_tr_b16).  Row sums of p are kept in
// fp32 on the VALU.
#include <type_traits>

#include "common.h"
#include "lanes.h"
#include "lds_dma.h"

namespace kda {
namespace attn32 {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;                      // head dim
constexpr int kBN = 64;                      // keys per tile
constexpr int kWaveRows = 32;                // query rows per wave
constexpr int kIT = kWaveRows / 16;
constexpr int kWaves = 8;                    // HPW query heads x (8 / HPW) blocks of 32 rows
constexpr int kThreads = 64 * kWaves;
constexpr int kPlaneBytes = kBN * kD * 2;    // one limb of a K or V tile: 16 KiB
constexpr int kTileBytes = 2 * kPlaneBytes;  // both limbs: 32 KiB
constexpr int kDmaPerWave = kTileBytes / (kWaves * 1024);   // 4 per K or V tile
constexpr int kTopExp = 13;                  // largest |scaled value| in [2^13, 2^14)
constexpr float kLazy = 8.0f;                // running-max slack (log2 units)
constexpr float kPScale = 64.0f;             // p * 2^6 <= 2^(kLazy + 6) = 2^14
constexpr int kSplitThreads = 256;

// 2^e for e in [-126, 127], from the exponent bits.
__device__ __forceinline__ float pow2(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

// Exponent of a non-negative float's leading bit, clamped to [-100, 128] so that
// both 2^(kTopExp - e) and 2^(e - kTopExp) stay normal (0 gives -100; inf and
// NaN give 128 and stay non-finite after scaling).
__device__ __forceinline__ int top_exponent(float mx) {
  return max((int)((__float_as_uint(mx) >> 23) & 0xff) - 127, -100);
}

// Two fp16 limbs of x: x0 = fp16(x), x1 = fp16(x - x0) (x - x0 is exact in fp32).
__device__ __forceinline__ void limbs2(float x, _Float16& h0, _Float16& h1) {
  h0 = (_Float16)x;
  h1 = (_Float16)(x - (float)h0);
}

__device__ __forceinline__ void store_limbs4(const floatx4& x, float sc, _Float16* p0, _Float16* p1) {
  half4 a, b;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    _Float16 h0, h1;
    limbs2(x[e] * sc, h0, h1);
    a[e] = h0;
    b[e] = h1;
  }
  *reinterpret_cast<half4*>(p0) = a;
  *reinterpret_cast<half4*>(p1) = b;
}

// Block-wide max of a non-negative value (256 threads).
__device__ __forceinline__ float block_max(float x, float* red) {
  for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// One workgroup per (64-key tile, batch x kv head): limbs of the K tile scaled
// by its own power of two (kinv[bh][tile]), and the V tile's largest |value|
// (vtmax[bh][tile]) for the per-head V scale.
__global__ __launch_bounds__(kSplitThreads) void k_split_kernel(
    const float* __restrict__ k, const float* __restrict__ v, _Float16* __restrict__ k0,
    _Float16* __restrict__ k1, float* __restrict__ kinv, float* __restrict__ vtmax, int seq, int hkv) {
  __shared__ float red[4];
  const int nt = gridDim.x, tile = blockIdx.x, bh = blockIdx.y;
  const int b = bh / hkv, h = bh % hkv;
  constexpr int kPer = kBN * kD / 4 / kSplitThreads;   // float4 per thread: 8
  floatx4 x[kPer];
  int64_t off[kPer];
  bool ok[kPer];
  float km = 0.f, vm = 0.f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e4 = threadIdx.x + kSplitThreads * i;
    const int r = e4 / (kD / 4), c4 = e4 % (kD / 4);
    const int j = tile * kBN + r;
    ok[i] = j < seq;
    off[i] = (((int64_t)b * seq + j) * hkv + h) * kD + 4 * c4;
    x[i] = ok[i] ? *reinterpret_cast<const floatx4*>(k + off[i]) : floatx4{0.f, 0.f, 0.f, 0.f};
    const floatx4 y = ok[i] ? *reinterpret_cast<const floatx4*>(v + off[i]) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) km = fmaxf(km, fabsf(x[i][e])), vm = fmaxf(vm, fabsf(y[e]));
  }
  km = block_max(km, red);
  vm = block_max(vm, red);
  const int e = top_exponent(km);
  const float sc = pow2(kTopExp - e);
#pragma unroll
  for (int i = 0; i < kPer; ++i)
    if (ok[i]) store_limbs4(x[i], sc, k0 + off[i], k1 + off[i]);
  if (threadIdx.x == 0) {
    kinv[(int64_t)bh * nt + tile] = pow2(e - kTopExp);
    vtmax[(int64_t)bh * nt + tile] = vm;
  }
}

// One workgroup per (64-key tile, batch x kv head): limbs of the V tile scaled by
// the kv head's power of two (from all tile maxima); tile 0 records vinv[bh].
__global__ __launch_bounds__(kSplitThreads) void v_split_kernel(const float* __restrict__ v,
                                                                const float* __restrict__ vtmax,
                                                                _Float16* __restrict__ v0,
                                                                _Float16* __restrict__ v1,
                                                                float* __restrict__ vinv, int seq,
                                                                int hkv) {
  __shared__ float red[4];
  const int nt = gridDim.x, tile = blockIdx.x, bh = blockIdx.y;
  const int b = bh / hkv, h = bh % hkv;
  float vm = 0.f;
  for (int i = threadIdx.x; i < nt; i += kSplitThreads) vm = fmaxf(vm, vtmax[(int64_t)bh * nt + i]);
  vm = block_max(vm, red);
  const int e = top_exponent(vm);
  const float sc = pow2(kTopExp - e);
  if (tile == 0 && threadIdx.x == 0) vinv[bh] = pow2(e - kTopExp);
  constexpr int kPer = kBN * kD / 4 / kSplitThreads;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int e4 = threadIdx.x + kSplitThreads * i;
    const int r = e4 / (kD / 4), c4 = e4 % (kD / 4);
    const int j = tile * kBN + r;
    if (j >= seq) continue;
    const int64_t off = (((int64_t)b * seq + j) * hkv + h) * kD + 4 * c4;
    store_limbs4(*reinterpret_cast<const floatx4*>(v + off), sc, v0 + off, v1 + off);
  }
}

struct Args {
  const float* q;            // [B][S][Hq][D], fp32 (split in the kernel)
  const _Float16 *k0, *k1;   // [B][S][Hkv][D]
  const _Float16 *v0, *v1;
  const float* kinv;         // [B*Hkv][nt]
  const float* vinv;         // [B*Hkv]
  float* out;
  int64_t o_sb, o_ss, o_sh;  // output strides (elements)
  int batch, seq, hq, hkv, nt;
  float scale_log2;          // softmax scale * log2(e)
};

// Swizzle of the 16 16-byte chunks of a K row (as in the bf16 kernel):
// conflict-free for the permuted 16-row fragment read.
__device__ __forceinline__ int kswz(int row) { return (row & 3) | (((row >> 3) & 3) << 2); }

// K fragment t of d-chunk dc (MFMA A operand): row 32(t>>1) + 8(l16>>2) + 4(t&1) + (l16&3).
__device__ __forceinline__ half8 k_frag(const uint8_t* k_lds, int t, int dc, int lane) {
  const int l16 = lane & 15, g = lane >> 4;
  const int krow = 32 * (t >> 1) + 8 * (l16 >> 2) + 4 * (t & 1) + (l16 & 3);
  return *reinterpret_cast<const half8*>(k_lds + krow * (2 * kD) + (((dc * 4 + g) ^ kswz(krow)) << 4));
}

__device__ __forceinline__ half8 v_frag(const uint8_t* v_lds, int dt, int c, int lane) {
  return __builtin_bit_cast(half8, read_mn_frag<kD>(v_lds, dt * 16, 32 * c, lane));
}

__device__ __forceinline__ uint32_t pack_h2(_Float16 lo, _Float16 hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// HPW query heads (of one kv head) per workgroup, HPW in {1, 2, 4, 8}: the
// workgroup covers BM = 32 * 8 / HPW query rows of each of its heads, and a kv
// head's G query heads are spread over G / HPW workgroups.
template <bool CAUSAL, int HPW>
__global__ __launch_bounds__(kThreads, 1) void gqa_f32_kernel(Args p) {
  constexpr int kBM = kWaveRows * kWaves / HPW;
  __shared__ __align__(1024) uint8_t smem[4 * kTileBytes];   // K slots 0,1; V slots 2,3

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int l16 = lane & 15;
  const int g = lane >> 4;

  const int nqb = (p.seq + kBM - 1) / kBM;
  const int group = p.hq / p.hkv;
  const int nsplit = group / HPW;                   // workgroups per kv head
  const int nbh = p.batch * p.hkv * nsplit;
  // longest causal blocks first
  const int qb = CAUSAL ? (nqb - 1 - (int)blockIdx.x / nbh) : ((int)blockIdx.x / nbh);
  const int bh = blockIdx.x % nbh;
  const int b = bh / (p.hkv * nsplit);
  const int kvh = (bh / nsplit) % p.hkv;
  const int h = kvh * group + (bh % nsplit) * HPW + (wave % HPW);
  const int bkv = b * p.hkv + kvh;                  // index of the per-(b, kv head) scales
  const int q0 = qb * kBM;
  const int w0 = q0 + (wave / HPW) * kWaveRows;     // this wave's first query row

  // ---- Q fragments (MFMA B operand, two limbs): row w0 + 16it + l16, d = 32dc + 8g .. +7.
  // Each row is scaled by 2^(kTopExp - e), e the exponent of its largest |value|
  // (the four lanes of a row hold its 128 values), and split into fp16 limbs
  // here: q is read once per wave, so no pre-pass is needed for it.
  // Rows past the sequence read the last row and are never stored.
  half8 qf[kIT][4][2];
  float rowc[kIT];   // scale_log2 * 2^(e - kTopExp)
#pragma unroll
  for (int it = 0; it < kIT; ++it) {
    const int row = min(w0 + it * 16 + l16, p.seq - 1);
    const float* qr = p.q + (((int64_t)b * p.seq + row) * p.hq + h) * kD + g * 8;
    floatx4 x[4][2];
    float mx = 0.f;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        x[dc][hh] = *reinterpret_cast<const floatx4*>(qr + dc * 32 + hh * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) mx = fmaxf(mx, fabsf(x[dc][hh][e]));
      }
    const int ex = top_exponent(row_max4(mx));
    const float sc = pow2(kTopExp - ex);
#pragma unroll
    for (int dc = 0; dc < 4; ++dc)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          _Float16 h0, h1;
          limbs2(x[dc][hh][e] * sc, h0, h1);
          qf[it][dc][0][hh * 4 + e] = h0;
          qf[it][dc][1][hh * 4 + e] = h1;
        }
    rowc[it] = p.scale_log2 * pow2(ex - kTopExp);
  }
  floatx4 o[kIT][8];
  float m[kIT], l[kIT];
#pragma unroll
  for (int it = 0; it < kIT; ++it) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[it][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    m[it] = -INFINITY;
    l[it] = 0.f;
  }

  // ---- DMA geometry: instruction j of this wave fills LDS bytes
  // [(j*kWaves + wave)*1024, +1024) of a tile: limb j/2, rows 4q' .. 4q'+3 with
  // q' = (j&1)*kWaves + wave; lane -> (row, 16-byte chunk).
  const int64_t row_bytes = (int64_t)p.hkv * kD * 2;
  const int64_t head_off = ((int64_t)b * p.seq * p.hkv + kvh) * kD * 2;
  const char* kb[2] = {reinterpret_cast<const char*>(p.k0) + head_off,
                       reinterpret_cast<const char*>(p.k1) + head_off};
  const char* vb[2] = {reinterpret_cast<const char*>(p.v0) + head_off,
                       reinterpret_cast<const char*>(p.v1) + head_off};
  auto k_tile = [&](int kt) { return smem + (kt & 1) * kTileBytes; };
  auto v_tile = [&](int kt) { return smem + (2 + (kt & 1)) * kTileBytes; };
  // Rows past the sequence are clamped to the last key: their scores are masked
  // and their V rows meet p = 0.  (Addresses are recomputed per tile: a few
  // VALU ops, against a dozen registers held across the loop.)
  auto issue = [&](int kt) {
    const int j0 = kt * kBN;
    const int last = p.seq - 1 - j0;
    const uint32_t kl = lds_addr(k_tile(kt)), vl = lds_addr(v_tile(kt));
    const int t = lane & 15;
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) {
      const int r = ((j & 1) * kWaves + wave) * 4 + (lane >> 4);
      const uint32_t roff = (uint32_t)(min(r, last) * row_bytes);
      const uint32_t kcol = (uint32_t)((t ^ kswz(r)) << 4);
      const uint32_t vcol = (uint32_t)((((t >> 1) ^ mswz(r)) << 5) + ((t & 1) << 4));
      const uint32_t dst = (uint32_t)((j * kWaves + wave) * 1024);
      dma16(kb[j >> 1] + j0 * row_bytes, roff + kcol, kl + dst);
      dma16(vb[j >> 1] + j0 * row_bytes, roff + vcol, vl + dst);
    }
  };

  const int nkt_all = (p.seq + kBN - 1) / kBN;
  const int nkt = CAUSAL ? min(nkt_all, (q0 + kBM - 1) / kBN + 1) : nkt_all;
  int nfree = p.seq / kBN;                          // full tiles
  if (CAUSAL) nfree = min(nfree, (q0 + 1) / kBN);   // keys j0+63 <= q0 for every row
  const float* kinv = p.kinv + (int64_t)bkv * p.nt;

  auto tile_step = [&](auto mask_tag, int kt) {
    constexpr bool MASK = decltype(mask_tag)::value;
    const uint8_t* kt_lds = k_tile(kt);
    const uint8_t* vt_lds = v_tile(kt);
    const float ks = kinv[kt];
    // S^T = K Q^T in three fp16 products; s[it][t] lane = query row l16, keys
    // 32(t>>1) + 8g + 4(t&1) + r
    floatx4 s[kIT][4];
#pragma unroll
    for (int it = 0; it < kIT; ++it)
#pragma unroll
      for (int t = 0; t < 4; ++t) s[it][t] = floatx4{0.f, 0.f, 0.f, 0.f};
    constexpr int kTerm[3][2] = {{0, 1}, {1, 0}, {0, 0}};   // (k limb, q limb), small terms first
#pragma unroll
    for (int dc = 0; dc < 4; ++dc)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const half8 kf[2] = {k_frag(kt_lds, t, dc, lane), k_frag(kt_lds + kPlaneBytes, t, dc, lane)};
#pragma unroll
        for (int term = 0; term < 3; ++term)
#pragma unroll
          for (int it = 0; it < kIT; ++it)
            s[it][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kTerm[term][0]], qf[it][dc][kTerm[term][1]],
                                                              s[it][t], 0, 0, 0);
      }
    // ---- online softmax (log2 units: logit = s * c)
    float c[kIT], alpha[kIT], shift[kIT];
    bool grow_any = false;
#pragma unroll
    for (int it = 0; it < kIT; ++it) {
      c[it] = rowc[it] * ks;
      if constexpr (MASK) {
        const int qrow = w0 + it * 16 + l16;
        const int lim = (CAUSAL ? min(qrow, p.seq - 1) : p.seq - 1) - kt * kBN - 8 * g;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (32 * (t >> 1) + 4 * (t & 1) + r > lim) s[it][t][r] = -INFINITY;
      }
      float mx = s[it][0][0];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[it][t][r]);
      const float mt = row_max4(mx) * c[it];
      // lazy: the running max moves only when a tile exceeds it by 2^kLazy
      const bool grow = mt - m[it] > kLazy;
      grow_any |= grow;
      const float m_new = grow ? mt : m[it];
      alpha[it] = (m_new == -INFINITY) ? 1.f : __builtin_amdgcn_exp2f(m[it] - m_new);
      m[it] = m_new;
      shift[it] = (m_new == -INFINITY) ? 0.f : m_new;
    }
    if (__builtin_amdgcn_ballot_w64(grow_any)) {
#pragma unroll
      for (int it = 0; it < kIT; ++it) {
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[it][dt] *= alpha[it];
        l[it] *= alpha[it];
      }
    }
    // probabilities: fp32 row sums, then p * 2^6 in two fp16 limbs packed as the
    // B operand of O^T += V^T P^T (chunk cc: keys 32cc + 8g .. +7)
    half8 pf[kIT][2][2];
#pragma unroll
    for (int it = 0; it < kIT; ++it) {
      float pv[4][4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pv[t][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[it][t][r], c[it], -shift[it]));
          l[it] += pv[t][r];
        }
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        u32x4 w0v, w1v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = 2 * cc + (e >> 1), r = 2 * (e & 1);
          _Float16 a0, a1, b0, b1;
          limbs2(pv[t][r] * kPScale, a0, a1);
          limbs2(pv[t][r + 1] * kPScale, b0, b1);
          w0v[e] = pack_h2(a0, b0);
          w1v[e] = pack_h2(a1, b1);
        }
        pf[it][cc][0] = __builtin_bit_cast(half8, w0v);
        pf[it][cc][1] = __builtin_bit_cast(half8, w1v);
      }
    }
    // O^T += V^T P^T in three fp16 products (V^T fragment: row d = 16dt + l16)
    constexpr int kTermV[3][2] = {{1, 0}, {0, 1}, {0, 0}};   // (v limb, p limb)
#pragma unroll
    for (int cc = 0; cc < 2; ++cc)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const half8 vf0 = v_frag(vt_lds, dt, cc, lane);
        const half8 vf1 = v_frag(vt_lds + kPlaneBytes, dt, cc, lane);
#pragma unroll
        for (int term = 0; term < 3; ++term)
#pragma unroll
          for (int it = 0; it < kIT; ++it)
            o[it][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kTermV[term][0] ? vf1 : vf0,
                                                               pf[it][cc][kTermV[term][1]], o[it][dt], 0, 0, 0);
      }
  };

  // Iteration kt: wait for this wave's DMA of tile kt, barrier (tile kt visible;
  // slot (kt+1)&1, last read in iteration kt-1, is free), issue tile kt+1, compute.
  // Two loops (unmasked tiles, then masked ones), one tile_step instance each:
  // with both instances in one loop body the register allocator spills.
  issue(0);
  int kt = 0;
  for (; kt < nfree; ++kt) {
    wait_vmcnt<0>();
    __syncthreads();
    if (kt + 1 < nkt) issue(kt + 1);
    tile_step(std::false_type(), kt);
  }
  for (; kt < nkt; ++kt) {
    wait_vmcnt<0>();
    __syncthreads();
    if (kt + 1 < nkt) issue(kt + 1);
    tile_step(std::true_type(), kt);
  }

  // ---- normalise and store: lane holds out[row][d = 16dt + 4g .. +3]
  const float vs = p.vinv[bkv] / kPScale;
  float* op = p.out + b * p.o_sb + (int64_t)h * p.o_sh;
#pragma unroll
  for (int it = 0; it < kIT; ++it) {
    const float inv = vs / row_sum4(l[it]);
    const int row = w0 + it * 16 + l16;
    if (row >= p.seq) continue;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
      *reinterpret_cast<floatx4*>(op + row * p.o_ss + dt * 16 + 4 * g) = o[it][dt] * inv;
  }
}

// Workspace layout shared by the size query and the entry point.
struct Plan {
  _Float16 *k0, *k1, *v0, *v1;
  float *kinv, *vtmax, *vinv;
  int64_t bytes;
};
Plan plan(void* ws, int64_t batch, int64_t seq, int64_t hq, int64_t hkv) {
  Plan pl;
  Carve c{reinterpret_cast<uint8_t*>(ws)};
  (void)hq;
  const SizeTerm nk = SizeTerm(batch) * seq * hkv * kD;   // elements per limb plane
  const SizeTerm heads = SizeTerm(batch) * hkv;
  const SizeTerm nt = ceil_div(seq, kBN);
  pl.k0 = c.take<_Float16>(nk);
  pl.k1 = c.take<_Float16>(nk);
  pl.v0 = c.take<_Float16>(nk);
  pl.v1 = c.take<_Float16>(nk);
  pl.kinv = c.take<float>(heads * nt);
  pl.vtmax = c.take<float>(heads * nt);
  pl.vinv = c.take<float>(heads);
  pl.bytes = c.used;   // -1 when the sizes have no representable workspace
  return pl;
}

}  // namespace attn32

int64_t gqa_f32_workspace_bytes(int64_t batch, int64_t seq, int64_t hq, int64_t hkv) {
  return attn32::plan(nullptr, batch, seq, hq, hkv).bytes;
}

}  // namespace kda

using namespace kda;
using namespace kda::attn32;

extern "C" int kda_gqa_fwd_f32(const float* q, const float* k, const float* v, float* out,
                               int64_t batch, int64_t seq, int64_t hq, int64_t hkv,
                               int64_t head_dim, float scale, int causal, int64_t out_stride_b,
                               int64_t out_stride_s, int64_t out_stride_h, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  clear_error();
  const char* what = "gqa_fwd_f32";
  if (batch < 0 || seq < 0 || hq <= 0 || hkv <= 0)
    return set_error(KDA_ERR_INVALID_ARG, "%s: bad sizes B=%lld S=%lld Hq=%lld Hkv=%lld", what,
                     (long long)batch, (long long)seq, (long long)hq, (long long)hkv);
  if (head_dim != kD)
    return set_error(KDA_ERR_UNSUPPORTED, "%s: head_dim %lld unsupported (only %d)", what,
                     (long long)head_dim, kD);
  if (hq % hkv)
    return set_error(KDA_ERR_INVALID_ARG,
                     "%s: Hq=%lld is not a multiple of Hkv=%lld query heads per kv head", what,
                     (long long)hq, (long long)hkv);
  if (!(scale > 0.f)) return set_error(KDA_ERR_INVALID_ARG, "%s: scale must be > 0", what);
  if (batch == 0 || seq == 0) return KDA_OK;
  if (!q || !k || !v || !out) return set_error(KDA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return set_error(KDA_ERR_INVALID_ARG, "%s: q/k/v/out must be 16-byte aligned", what);
  if ((out_stride_s % 4) || (out_stride_h % 4) || (out_stride_b % 4))
    return set_error(KDA_ERR_INVALID_ARG, "%s: output strides must be multiples of 4", what);
  const int64_t nt = (seq + kBN - 1) / kBN;
  // heads per workgroup: the largest power of two up to 8 that divides the group
  const int64_t group = hq / hkv;
  const int hpw = (group % 8 == 0) ? 8 : (group % 4 == 0) ? 4 : (group % 2 == 0) ? 2 : 1;
  const int64_t bm = kWaveRows * kWaves / hpw;
  const int64_t nblocks = ((seq + bm - 1) / bm) * batch * hkv * (group / hpw);
  if (nblocks > 0x7fffffff || seq > (1 << 24) || batch * hkv > 65535 || nt > 0x7fffffff ||
      batch * seq * hq * kD * 2 > ((int64_t)1 << 32))
    return set_error(KDA_ERR_UNSUPPORTED, "%s: problem too large", what);
  const Plan pl = plan(workspace, batch, seq, hq, hkv);
  if (pl.bytes < 0 || !workspace || !aligned16(workspace) || workspace_bytes < pl.bytes)
    return set_error(KDA_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned and >= %lld bytes",
                     what, (long long)pl.bytes);
  hipStream_t st = as_stream(stream);
  const dim3 kv_grid((unsigned)nt, (unsigned)(batch * hkv));
  hipLaunchKernelGGL(k_split_kernel, kv_grid, dim3(kSplitThreads), 0, st, k, v, pl.k0, pl.k1,
                     pl.kinv, pl.vtmax, (int)seq, (int)hkv);
  if (int rc = check_launch(what)) return rc;
  hipLaunchKernelGGL(v_split_kernel, kv_grid, dim3(kSplitThreads), 0, st, v, pl.vtmax, pl.v0, pl.v1,
                     pl.vinv, (int)seq, (int)hkv);
  if (int rc = check_launch(what)) return rc;

  Args a;
  a.q = q;
  a.k0 = pl.k0;
  a.k1 = pl.k1;
  a.v0 = pl.v0;
  a.v1 = pl.v1;
  a.kinv = pl.kinv;
  a.vinv = pl.vinv;
  a.out = out;
  a.o_sb = out_stride_b;
  a.o_ss = out_stride_s;
  a.o_sh = out_stride_h;
  a.batch = (int)batch;
  a.seq = (int)seq;
  a.hq = (int)hq;
  a.hkv = (int)hkv;
  a.nt = (int)nt;
  a.scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid((unsigned)nblocks), block(kThreads);
#define KDA_GQA_LAUNCH(H)                                                         \
  if (causal)                                                                     \
    hipLaunchKernelGGL((gqa_f32_kernel<true, H>), grid, block, 0, st, a);         \
  else                                                                            \
    hipLaunchKernelGGL((gqa_f32_kernel<false, H>), grid, block, 0, st, a);
  switch (hpw) {
    case 8: KDA_GQA_LAUNCH(8) break;
    case 4: KDA_GQA_LAUNCH(4) break;
    case 2: KDA_GQA_LAUNCH(2) break;
    default: KDA_GQA_LAUNCH(1) break;
  }
#undef KDA_GQA_LAUNCH
  return check_launch(what);
}
