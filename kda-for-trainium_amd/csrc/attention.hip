// Grouped-query attention forward (bf16 in, fp32 online softmax, bf16 out) on
// gfx950 MFMA, flash style: scores never leave the chip.
//
//   out[b, s, h, :] = softmax_j(q[b, s, h, :] . k[b, j, h/G, :] * scale) @ v[b, j, h/G, :]
//   (G = Hq / Hkv query heads per kv head; causal: keys j > s masked)
//
// Work decomposition: one workgroup = (batch b, kv head, block of 64 queries);
// its 8 waves are the 4 query heads of that kv head (G == 4) x 2 halves of the
// query block (32 rows each), so each K/V tile staged in LDS is read by the
// whole query-head group.  32 rows per wave keep the O accumulators, scores and
// Q fragments within the 256 VGPRs a wave has at 2 waves per SIMD.  Keys advance in tiles of
// 64 through a double-buffered LDS ring with a register prefetch of the next
// tile (one barrier per tile).  Causal blocks with the most key tiles are
// scheduled first.
//
// Per wave (32 query rows x 64 keys per tile, head dim 128):
//   S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with K as the MFMA A operand: lane l
//   then holds 4 keys of query row (l & 15) per 16x16 tile.  K rows are read in a
//   permuted order so that, per 32-key chunk, each lane's 8 probabilities are 8
//   consecutive keys -> they form the MFMA operand of O^T += V^T P^T directly
//   (no LDS round trip for P).  V is transposed while being staged (LDS holds
//   V^T, key-contiguous) so that one ds_read_b128 yields a V^T fragment.
//   Online softmax in fp32 with exp2 (scale pre-multiplied by log2 e); the row
//   max is reduced across the 4 lanes sharing a row, the row sum stays per-lane
//   and is reduced once at the end.
#include "common.h"

namespace kda {
namespace attn {

constexpr int kD = 128;       // head dim
constexpr int kBM = 64;       // query rows per workgroup (per head)
constexpr int kWaveRows = 32; // query rows per wave
constexpr int kIT = kWaveRows / 16;
constexpr int kBN = 64;       // keys per tile
constexpr int kGroup = 4;     // query heads per kv head
constexpr int kWaves = kGroup * (kBM / kWaveRows);
constexpr int kThreads = 64 * kWaves;
constexpr int kKChunks = kBN * kD / 8 / kThreads;   // 16B K chunks staged per thread
constexpr int kVUnits = (kBN / 2) * (kD / 8) / kThreads;  // (2 key x 8 d) V units per thread
constexpr float kLazy = 8.0f;  // running-max slack (log2 units) before O and l are rescaled

struct Args {
  const uint16_t* q;   // [B][S][Hq][D] (strides below, in elements)
  const uint16_t* k;   // [B][S][Hkv][D]
  const uint16_t* v;
  uint16_t* out;
  int64_t q_sb, q_ss;  // batch / sequence strides of q (head stride is D)
  int64_t k_sb, k_ss;
  int64_t o_sb, o_ss, o_sh;
  int batch, seq, hq, hkv;
  float scale_log2;    // softmax scale * log2(e)
};

// Swizzled 16-byte chunk within a K row (16 chunks of 8 d): conflict-free for the
// permuted 16-row fragment reads below (rows 32c + 8a + r, a, r in 0..3).
__device__ __forceinline__ int k_swz(int row, int chunk) {
  return chunk ^ ((row & 3) | (((row >> 3) & 3) << 2));
}
// Swizzled 16-byte chunk within a V^T row (8 chunks of 8 keys).
__device__ __forceinline__ int v_swz(int row, int chunk) { return chunk ^ (row & 7); }

template <bool CAUSAL>
__global__ __launch_bounds__(kThreads, 1) void gqa_fwd_kernel(Args p) {
  __shared__ __align__(16) uint16_t Ks[2][kBN * kD];   // [key][d]    (swizzled chunks)
  __shared__ __align__(16) uint16_t Vt[2][kD * kBN];   // [d][key]    (swizzled chunks)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int g = lane >> 4;

  const int nqb = (p.seq + kBM - 1) / kBM;
  const int nbh = p.batch * p.hkv;
  // Longest causal blocks first.
  const int qb = CAUSAL ? (nqb - 1 - (int)blockIdx.x / nbh) : ((int)blockIdx.x / nbh);
  const int bh = blockIdx.x % nbh;
  const int b = bh / p.hkv, kvh = bh % p.hkv;
  const int h = kvh * kGroup + (wave % kGroup);
  const int q0 = qb * kBM;
  const int w0 = q0 + (wave / kGroup) * kWaveRows;   // this wave's first query row

  const uint16_t* qp = p.q + b * p.q_sb + (int64_t)h * kD;
  const uint16_t* kp = p.k + b * p.k_sb + (int64_t)kvh * kD;
  const uint16_t* vp = p.v + b * p.k_sb + (int64_t)kvh * kD;

  // ---- Q fragments (MFMA B operand): row q0 + it*16 + l16, d = dc*32 + 8g .. +8
  bf16x8 qf[kIT][4];
#pragma unroll
  for (int it = 0; it < kIT; ++it) {
    const int row = w0 + it * 16 + l16;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) {
      if (row < p.seq)
        qf[it][dc] = *reinterpret_cast<const bf16x8*>(qp + row * p.q_ss + dc * 32 + g * 8);
      else
        qf[it][dc] = bf16x8{};
    }
  }

  // ---- K/V staging: kKChunks x 16B of K and kVUnits x (2 keys x 8 d) of V per thread
  static_assert(kKChunks >= 1 && kVUnits >= 1, "staging split");
  static_assert(kKChunks * kThreads * 8 == kBN * kD && kVUnits * kThreads * 16 == kBN * kD, "exact split");
  u32x4 kreg[kKChunks], vreg[kVUnits][2];
  auto load_kv = [&](int kt) {
    const int j0 = kt * kBN;
#pragma unroll
    for (int i = 0; i < kKChunks; ++i) {
      const int c = tid + kThreads * i;
      const int row = c >> 4, ch = c & 15;
      const int j = j0 + row;
      kreg[i] = (j < p.seq) ? *reinterpret_cast<const u32x4*>(kp + j * p.k_ss + ch * 8)
                            : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kVUnits; ++u) {
      const int unit = tid + kThreads * u;
      const int jp = unit & 31, dc = unit >> 5;   // keys jp*2..+2, d = dc*8..+8
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int j = j0 + jp * 2 + r;
        vreg[u][r] = (j < p.seq) ? *reinterpret_cast<const u32x4*>(vp + j * p.k_ss + dc * 8)
                                 : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto store_kv = [&](int buf) {
#pragma unroll
    for (int i = 0; i < kKChunks; ++i) {
      const int c = tid + kThreads * i;
      const int row = c >> 4, ch = c & 15;
      *reinterpret_cast<u32x4*>(&Ks[buf][row * kD + k_swz(row, ch) * 8]) = kreg[i];
    }
#pragma unroll
    for (int u = 0; u < kVUnits; ++u) {
      const int unit = tid + kThreads * u;
      const int jp = unit & 31, dc = unit >> 5;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = dc * 8 + e;
        const int w = e >> 1;
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t o = __builtin_amdgcn_perm(vreg[u][1][w], vreg[u][0][w], sel);
        // keys jp*2..+2 -> 16B chunk jp/4, dword jp&3 within it
        *reinterpret_cast<uint32_t*>(&Vt[buf][d * kBN + v_swz(d, jp >> 2) * 8 + (jp & 3) * 2]) = o;
      }
    }
  };

  floatx4 o_acc[kIT][8];   // [i-tile][d-tile]: O^T, lane holds row l16, d = dt*16 + 4g + r
#pragma unroll
  for (int it = 0; it < kIT; ++it)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o_acc[it][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run[kIT], l_run[kIT];
#pragma unroll
  for (int it = 0; it < kIT; ++it) {
    m_run[it] = -INFINITY;
    l_run[it] = 0.f;
  }

  const int nkt_all = (p.seq + kBN - 1) / kBN;
  const int nkt = CAUSAL ? min(nkt_all, (q0 + kBM - 1) / kBN + 1) : nkt_all;

  load_kv(0);
  store_kv(0);
  __syncthreads();

  for (int kt = 0; kt < nkt; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < nkt;
    if (more) load_kv(kt + 1);

    // ---- S^T = K Q^T : tiles t = 2c + hh, keys 32c + 8a + 4hh + r for A-row 4a + r
    floatx4 s[kIT][4];   // [i-tile][t]
#pragma unroll
    for (int it = 0; it < kIT; ++it)
#pragma unroll
      for (int t = 0; t < 4; ++t) s[it][t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int c = t >> 1, hh = t & 1;
      const int krow = 32 * c + 8 * (l16 >> 2) + 4 * hh + (l16 & 3);
#pragma unroll
      for (int dc = 0; dc < 4; ++dc) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(
            &Ks[buf][krow * kD + k_swz(krow, dc * 4 + g) * 8]);
#pragma unroll
        for (int it = 0; it < kIT; ++it)
          s[it][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[it][dc], s[it][t], 0, 0, 0);
      }
    }

    // ---- online softmax (rows: it*16 + l16; this lane's keys: 32c + 8g + 4hh + r)
    // Scores stay unscaled; p = exp2(s*scale_log2 - m*scale_log2) is one FMA and
    // one v_exp_f32.  The running max m is raised lazily: only when some row's
    // tile max exceeds it by more than kLazy (in log2 units), so p <= 2^kLazy,
    // which bf16 P and the fp32 row sums carry exactly as well; the final O / l
    // cancels whichever m was used.  O and l are then rescaled for the whole wave
    // (a wave-uniform branch), otherwise not at all.
    const int j_base = kt * kBN;
    if ((CAUSAL && j_base + kBN - 1 > w0) || j_base + kBN > p.seq) {
#pragma unroll
      for (int it = 0; it < kIT; ++it) {
        const int qrow = w0 + it * 16 + l16;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = j_base + 32 * (t >> 1) + 8 * g + 4 * (t & 1) + r;
            if ((CAUSAL && key > qrow) || key >= p.seq) s[it][t][r] = -INFINITY;
          }
      }
    }
    float mx[kIT];
    bool grow = false;
#pragma unroll
    for (int it = 0; it < kIT; ++it) {
      float m = fmaxf(fmaxf(s[it][0][0], s[it][0][1]), fmaxf(s[it][0][2], s[it][0][3]));
#pragma unroll
      for (int t = 1; t < 4; ++t)
        m = fmaxf(m, fmaxf(fmaxf(s[it][t][0], s[it][t][1]), fmaxf(s[it][t][2], s[it][t][3])));
      m = fmaxf(m, __shfl_xor(m, 16));
      m = fmaxf(m, __shfl_xor(m, 32));
      mx[it] = m;
      grow |= (m - m_run[it]) * p.scale_log2 > kLazy;
    }
    if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
      for (int it = 0; it < kIT; ++it) {
        const float m_new = fmaxf(m_run[it], mx[it]);
        // rows with every key so far masked keep m = -inf: alpha = 0 then (O, l are 0)
        const float alpha = (m_new == -INFINITY)
                                ? 1.f
                                : __builtin_amdgcn_exp2f((m_run[it] - m_new) * p.scale_log2);
        m_run[it] = m_new;
        l_run[it] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o_acc[it][dt] *= alpha;
      }
    }
    bf16x8 pf[kIT][2];   // [i-tile][32-key chunk]
#pragma unroll
    for (int it = 0; it < kIT; ++it) {
      const float shift = (m_run[it] == -INFINITY) ? 0.f : m_run[it] * p.scale_log2;
      float rs = 0.f;
      float pv[4][4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          pv[t][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[it][t][r], p.scale_log2, -shift));
          rs += pv[t][r];
        }
      l_run[it] += rs;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        typedef float floatx2 __attribute__((ext_vector_type(2)));
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        u32x4 w;
        w[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{pv[2 * c][0], pv[2 * c][1]}), bf16x2));
        w[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{pv[2 * c][2], pv[2 * c][3]}), bf16x2));
        w[2] = __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{pv[2 * c + 1][0], pv[2 * c + 1][1]}), bf16x2));
        w[3] = __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{pv[2 * c + 1][2], pv[2 * c + 1][3]}), bf16x2));
        pf[it][c] = __builtin_bit_cast(bf16x8, w);
      }
    }

    // ---- O^T += V^T P^T
#pragma unroll
    for (int c = 0; c < 2; ++c) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const int d = dt * 16 + l16;
        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(&Vt[buf][d * kBN + v_swz(d, c * 4 + g) * 8]);
#pragma unroll
        for (int it = 0; it < kIT; ++it)
          o_acc[it][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[it][c], o_acc[it][dt], 0, 0, 0);
      }
    }

    if (more) store_kv(buf ^ 1);
    __syncthreads();
  }

  // ---- normalise and store: lane holds out[row][d = dt*16 + 4g .. +4]
  uint16_t* op = p.out + b * p.o_sb + (int64_t)h * p.o_sh;
#pragma unroll
  for (int it = 0; it < kIT; ++it) {
    float l = l_run[it];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
    const int row = w0 + it * 16 + l16;
    if (row >= p.seq) continue;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      typedef float floatx2 __attribute__((ext_vector_type(2)));
      typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
      const floatx4 o = o_acc[it][dt] * inv;
      u32x2 w;
      w[0] = __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{o[0], o[1]}), bf16x2));
      w[1] = __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{o[2], o[3]}), bf16x2));
      *reinterpret_cast<u32x2*>(op + row * p.o_ss + dt * 16 + 4 * g) = w;
    }
  }
}

}  // namespace attn
}  // namespace kda

using namespace kda;
using namespace kda::attn;

extern "C" int kda_gqa_fwd_bf16(const kda_bf16* q, const kda_bf16* k, const kda_bf16* v,
                                kda_bf16* out, int64_t batch, int64_t seq, int64_t hq,
                                int64_t hkv, int64_t head_dim, float scale, int causal,
                                int64_t out_stride_b, int64_t out_stride_s, int64_t out_stride_h,
                                void* stream) {
  clear_error();
  if (batch < 0 || seq < 0 || hq <= 0 || hkv <= 0)
    return set_error(KDA_ERR_INVALID_ARG, "gqa_fwd_bf16: bad sizes B=%lld S=%lld Hq=%lld Hkv=%lld",
                     (long long)batch, (long long)seq, (long long)hq, (long long)hkv);
  if (head_dim != kD)
    return set_error(KDA_ERR_UNSUPPORTED, "gqa_fwd_bf16: head_dim %lld unsupported (only %d)",
                     (long long)head_dim, kD);
  if (hq % hkv || hq / hkv != kGroup)
    return set_error(KDA_ERR_UNSUPPORTED,
                     "gqa_fwd_bf16: needs Hq/Hkv == %d query heads per kv head (got %lld/%lld)",
                     kGroup, (long long)hq, (long long)hkv);
  if (!(scale > 0.f)) return set_error(KDA_ERR_INVALID_ARG, "gqa_fwd_bf16: scale must be > 0");
  if (batch == 0 || seq == 0) return KDA_OK;
  if (!q || !k || !v || !out) return set_error(KDA_ERR_INVALID_ARG, "gqa_fwd_bf16: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || (reinterpret_cast<uintptr_t>(out) & 7))
    return set_error(KDA_ERR_INVALID_ARG, "gqa_fwd_bf16: q/k/v must be 16-byte, out 8-byte aligned");
  if ((out_stride_s % 4) || (out_stride_h % 4) || (out_stride_b % 4))
    return set_error(KDA_ERR_INVALID_ARG, "gqa_fwd_bf16: output strides must be multiples of 4");
  const int64_t nblocks = ((seq + kBM - 1) / kBM) * batch * hkv;
  if (nblocks > 0x7fffffff || seq > (1 << 30))
    return set_error(KDA_ERR_UNSUPPORTED, "gqa_fwd_bf16: problem too large");

  Args a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.q_ss = hq * kD;
  a.q_sb = seq * a.q_ss;
  a.k_ss = hkv * kD;
  a.k_sb = seq * a.k_ss;
  a.o_sb = out_stride_b;
  a.o_ss = out_stride_s;
  a.o_sh = out_stride_h;
  a.batch = (int)batch;
  a.seq = (int)seq;
  a.hq = (int)hq;
  a.hkv = (int)hkv;
  a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t st = as_stream(stream);
  if (causal)
    hipLaunchKernelGGL(gqa_fwd_kernel<true>, dim3((unsigned)nblocks), dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL(gqa_fwd_kernel<false>, dim3((unsigned)nblocks), dim3(kThreads), 0, st, a);
  return check_launch("gqa_fwd_bf16");
}
