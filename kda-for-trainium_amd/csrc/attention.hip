// Grouped-query attention forward (bf16 in, fp32 online softmax, bf16 out) on
// gfx950 MFMA, flash style: scores never leave the chip.
//
//   out[b, s, h, :] = softmax_j(q[b, s, h, :] . k[b, j, h/G, :] * scale) @ v[b, j, h/G, :]
//   (G = Hq / Hkv query heads per kv head; causal: keys j > s masked)
//
// Work decomposition: one workgroup = (batch b, kv head, HPW of its query heads,
// block of 256 / HPW queries), HPW the largest power of two up to 8 dividing G;
// its 8 waves are the HPW heads x 8 / HPW blocks of 32 query rows, so each K/V
// tile staged in LDS is read by HPW query heads (the graded G = 4: 4 heads x 64
// queries).  Causal blocks with the most key tiles are scheduled first, on a
// persistent grid of one workgroup per CU that runs its blocks in a snake over
// that order (even totals); a block's last iterations prefetch the next block's
// first K/V tiles and its q rows (into LDS, before the block's output stores, so
// that the next block's q wait leaves those stores in flight).
//
// Staging: K and V tiles of 64 keys go straight from global memory into LDS
// (global_load_lds_dwordx4, no register staging), each through a 4-slot ring
// fetched two iterations ahead; the
// LDS swizzle is applied on the global side by choosing which 16-byte chunk each
// lane fetches.  K is stored [key][d] (16-byte chunk c of row r at c ^ kswz(r)); V
// keeps its HBM orientation [key][d] (32-byte segment s of row r at s ^ mswz(r))
// and its fragments are read transposed (ds_read_b64_tr_b16).
//
// Per wave (32 query rows x 64 keys per tile, head dim 128):
//   S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with K as the MFMA A operand: lane l
//   then holds 4 keys of query row (l & 15) per 16x16 tile.  K rows are read in a
//   permuted order so that, per 32-key chunk, each lane's 8 probabilities are 8
//   consecutive keys -> they form the B operand of O^T += V^T P^T directly
//   (no LDS round trip for P).  Row sums of the probabilities are kept per lane
//   in fp32 (16 keys of a row per lane and tile) and reduced across the row's
//   four lanes once, at the end.
//   Online softmax in fp32 on log2-scaled scores: Q is multiplied by
//   scale*log2(e) (and rounded to bf16) once when it is loaded, and each S^T
//   accumulator starts from -m, the running max of its row, so the MFMAs produce
//   s*scale*log2e - m directly and p = exp2(acc) is one v_exp_f32 per score.  The
//   running max is raised lazily (only when a tile's scores exceed it by more
//   than kLazy), so O is rescaled only then.  Masking is applied only on tiles
//   that cross the causal diagonal or the sequence end.
//   Software pipeline, per iteration kt: the MFMAs of O += V(kt-1) P(kt-1) run in
//   one basic block with the row-max test of S(kt); after the (rarely taken)
//   running-max update, the exponentials of S(kt) and the MFMAs of
//   S(kt+1) = K(kt+1) Q^T run in a second block, S(kt+1) accumulating into the
//   registers of S(kt) tile by tile.  The K and V fragments are read kAhead
//   fragments ahead of the MFMAs that use them, pinned in program order, so
//   several LDS reads are in flight per wave; the reads run on across the two
//   blocks (the first block's last slots fetch the second's first K fragments).
//   The second wave of each SIMD
//   runs at a raised issue priority so both reach the per-iteration barrier
//   together.
#include <algorithm>

#include "attention_geom.h"
#include "common.h"
#include "lanes.h"
#include "lds_dma.h"

namespace kda {
namespace attn {

// Sizes, launch arguments and every global address (q loads, K/V tile DMAs,
// output stores) come from attention_geom.h.
constexpr int kIT = kWaveRows / 16;
constexpr int kDT = kD / 16;                                // O^T tiles along d
constexpr float kLazy = 8.0f;  // running-max slack (log2 units) before O is rescaled

typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{lo, hi}), bf16x2));
}

// Per-wave state carried across key tiles.
struct State {
  bf16x8 qf[kIT][4];      // Q * scale*log2e (MFMA B operand): row it*16 + l16, d = dc*32 + 8g .. +8
  floatx4 o[kIT][kDT];    // O^T: lane holds row l16, d = dt*16 + 4g + r
  float l[kIT];           // this lane's part of the row sum of the probabilities
  floatx4 c0[kIT];        // S^T accumulator seed: -m (the row's running max, log2 units)
};

__device__ __forceinline__ bf16x8 k_frag(const uint8_t* kt_lds, int t, int dc, int lane) {
  const int l16 = lane & 15, g = lane >> 4;
  const int krow = 32 * (t >> 1) + 8 * (l16 >> 2) + 4 * (t & 1) + (l16 & 3);
  return *reinterpret_cast<const bf16x8*>(kt_lds + krow * (2 * kD) +
                                          (((dc * 4 + g) ^ kswz(krow)) << 4));
}

// S^T = K Q^T - m: s[it][t], t = 2c + hh covers keys 32c + 8a + 4hh + r for A-row
// 4a + r.  d-chunk outer: the 8 accumulators rotate, consecutive MFMAs are independent.
__device__ __forceinline__ void scores(const State& st, const uint8_t* k_lds, int lane,
                                       floatx4 (&s)[kIT][4]) {
#pragma unroll
  for (int dc = 0; dc < 4; ++dc)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const bf16x8 kf = k_frag(k_lds, t, dc, lane);
#pragma unroll
      for (int it = 0; it < kIT; ++it)
        s[it][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, st.qf[it][dc],
                                                           dc == 0 ? st.c0[it] : s[it][t], 0, 0, 0);
    }
}

// O^T += V^T P^T (V^T fragment: row d = dt*16 + l16, keys 32c + 8g .. +8).
// The 16 V fragments are read kAhead fragments ahead of the MFMAs that use them,
// so several LDS reads are in flight instead of one.  A scheduling barrier that
// only VALU, SALU and transcendental instructions may cross pins each read and
// MFMA at its place in program order (left alone, the scheduler sinks every read
// to just before its first use to save registers, and moves MFMAs above reads).
constexpr int kAhead = 3;
constexpr int kPinReads = 0x0002 | 0x0004 | 0x0400;   // VALU, SALU, TRANS may cross
__device__ __forceinline__ void pin_reads() { __builtin_amdgcn_sched_barrier(kPinReads); }
__device__ __forceinline__ void accumulate_pv(State& st, const uint8_t* v_lds,
                                              const bf16x8 (&pf)[kIT][2], int lane) {
  bf16x8 vf[16];
#pragma unroll
  for (int f = 0; f < kAhead; ++f) vf[f] = read_mn_frag<kD>(v_lds, (f & 7) * 16, 32 * (f >> 3), lane);
  pin_reads();
#pragma unroll
  for (int f = 0; f < 16; ++f) {
    if (f + kAhead < 16)
      vf[f + kAhead] = read_mn_frag<kD>(v_lds, ((f + kAhead) & 7) * 16, 32 * ((f + kAhead) >> 3), lane);
    pin_reads();
    const int c = f >> 3, dt = f & 7;
#pragma unroll
    for (int it = 0; it < kIT; ++it)
      st.o[it][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[f], pf[it][c], st.o[it][dt], 0, 0, 0);
  }
}

// accumulate_pv whose last kAhead read slots fetch the first kAhead K fragments
// of the block B that follows (K(kt+1) has landed since the previous barrier), so
// the read stream runs on across the two blocks (0.5 % same-box).
__device__ __forceinline__ void accumulate_pv_k(State& st, const uint8_t* v_lds,
                                                const bf16x8 (&pf)[kIT][2], int lane,
                                                const uint8_t* k_lds, bf16x8 (&kf0)[kAhead]) {
  bf16x8 vf[16];
#pragma unroll
  for (int f = 0; f < kAhead; ++f) vf[f] = read_mn_frag<kD>(v_lds, (f & 7) * 16, 32 * (f >> 3), lane);
  pin_reads();
#pragma unroll
  for (int f = 0; f < 16; ++f) {
    if (f + kAhead < 16)
      vf[f + kAhead] = read_mn_frag<kD>(v_lds, ((f + kAhead) & 7) * 16, 32 * ((f + kAhead) >> 3), lane);
    else
      kf0[f + kAhead - 16] = k_frag(k_lds, (f + kAhead - 16) >> 2, (f + kAhead - 16) & 3, lane);
    pin_reads();
    const int c = f >> 3, dt = f & 7;
#pragma unroll
    for (int it = 0; it < kIT; ++it)
      st.o[it][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[f], pf[it][c], st.o[it][dt], 0, 0, 0);
  }
}

// Online softmax of S(kt) (accumulators s = t - m in log2 units, t the scaled
// score, m the row's running max), first half: masking and the row-max test.
// Returns whether some row of the wave has a score above m + kLazy.  A row's max
// exceeds kLazy iff one of its four lanes' partial maxima (16 values each, a tree
// of three-input maxima) does, so the test needs no cross-lane reduction: one
// compare per row and a ballot.
template <bool CAUSAL, bool MASK>
__device__ __forceinline__ bool softmax_test(const Args& p, int kt, int w0, int lane,
                                             floatx4 (&s)[kIT][4], float (&x)[kIT]) {
  const int l16 = lane & 15, g = lane >> 4;
  if constexpr (MASK) {
    const int j_base = kt * kBN;
#pragma unroll
    for (int it = 0; it < kIT; ++it) {
      const int qrow = w0 + it * 16 + l16;
      // keys of this lane: j_base + 32(t>>1) + 8g + 4(t&1) + r; masked if > lim
      const int lim = (CAUSAL ? min(qrow, p.seq - 1) : p.seq - 1) - j_base - 8 * g;
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (32 * (t >> 1) + 4 * (t & 1) + r > lim) s[it][t][r] = -INFINITY;
    }
  }
  bool grow_any = false;
#pragma unroll
  for (int it = 0; it < kIT; ++it) {
    const floatx4(&r)[4] = s[it];
    const float a0 = __builtin_fmaxf(__builtin_fmaxf(r[0][0], r[0][1]), r[0][2]);
    const float a1 = __builtin_fmaxf(__builtin_fmaxf(r[0][3], r[1][0]), r[1][1]);
    const float a2 = __builtin_fmaxf(__builtin_fmaxf(r[1][2], r[1][3]), r[2][0]);
    const float a3 = __builtin_fmaxf(__builtin_fmaxf(r[2][1], r[2][2]), r[2][3]);
    const float a4 = __builtin_fmaxf(__builtin_fmaxf(r[3][0], r[3][1]), r[3][2]);
    const float b0 = __builtin_fmaxf(__builtin_fmaxf(a0, a1), a2);
    const float b1 = __builtin_fmaxf(__builtin_fmaxf(a3, a4), r[3][3]);
    x[it] = __builtin_fmaxf(b0, b1);
    grow_any |= x[it] > kLazy;
  }
  return __builtin_amdgcn_ballot_w64(grow_any) != 0;
}

// Second half, taken when the test above fires (or for the first tile, with
// FIRST: m is then set to the tile's row max whatever its value): rows whose max
// grew get m += delta (delta = their max), their accumulators and seed move by
// -delta, and alpha = 2^-delta is the factor their O and row sums must be
// multiplied by; other rows get alpha = 1.  A row whose keys are all masked
// keeps its m.
template <bool FIRST>
__device__ __forceinline__ void softmax_raise(State& st, floatx4 (&s)[kIT][4],
                                              const float (&x)[kIT], float (&alpha)[kIT]) {
#pragma unroll
  for (int it = 0; it < kIT; ++it) {
    const float m = row_max4(x[it]);
    const bool grow = FIRST ? (m != -INFINITY) : (m > kLazy);
    const float delta = grow ? m : 0.f;
    alpha[it] = grow ? __builtin_amdgcn_exp2f(-delta) : 1.f;
    // the row sums so far (tiles up to kt-1) move to the new m now, before this
    // tile's probabilities are added; O (one tile behind) moves in the next
    // iteration.  The first tile has no sums yet.
    if constexpr (!FIRST) st.l[it] *= alpha[it];
    st.c0[it] -= delta;
#pragma unroll
    for (int t = 0; t < 4; ++t) s[it][t] -= delta;
  }
}

// Probabilities p = exp2(acc), packed to bf16 as the B operand of O^T += V^T P^T.
__device__ __forceinline__ void softmax_probs(State& st, const floatx4 (&s)[kIT][4],
                                              bf16x8 (&pf)[kIT][2]) {
#pragma unroll
  for (int it = 0; it < kIT; ++it) {
    float pv[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) pv[t][r] = __builtin_amdgcn_exp2f(s[it][t][r]);
      st.l[it] += (pv[t][0] + pv[t][1]) + (pv[t][2] + pv[t][3]);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      u32x4 w;
      w[0] = pack2(pv[2 * c][0], pv[2 * c][1]);
      w[1] = pack2(pv[2 * c][2], pv[2 * c][3]);
      w[2] = pack2(pv[2 * c + 1][0], pv[2 * c + 1][1]);
      w[3] = pack2(pv[2 * c + 1][2], pv[2 * c + 1][3]);
      pf[it][c] = __builtin_bit_cast(bf16x8, w);
    }
  }
}

// Block B of an iteration: the probabilities of S(kt) (held in s) and
// S(kt+1) = K(kt+1) Q^T - m, key tile by key tile in place: tile t's exps and
// packs read s[.][t] before the MFMAs of S(kt+1) overwrite it, so S(kt+1) needs
// no second set of accumulators.
// PRE: the first kAhead K fragments are already in kf0 (read by accumulate_pv_k).
template <bool PRE>
__device__ __forceinline__ void probs_then_scores(State& st, const uint8_t* k_lds, int lane,
                                                  floatx4 (&s)[kIT][4], bf16x8 (&pf)[kIT][2],
                                                  const bf16x8 (&kf0)[kAhead]) {
  uint32_t w[kIT][2][4];
  // K fragments (t, dc) in order f = 4t + dc, read kAhead ahead of their MFMAs
  bf16x8 kf[16];
#pragma unroll
  for (int f = 0; f < kAhead; ++f) kf[f] = PRE ? kf0[f] : k_frag(k_lds, f >> 2, f & 3, lane);
  pin_reads();
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int it = 0; it < kIT; ++it) {
      const floatx4 e{__builtin_amdgcn_exp2f(s[it][t][0]), __builtin_amdgcn_exp2f(s[it][t][1]),
                      __builtin_amdgcn_exp2f(s[it][t][2]), __builtin_amdgcn_exp2f(s[it][t][3])};
      w[it][t >> 1][2 * (t & 1)] = pack2(e[0], e[1]);
      w[it][t >> 1][2 * (t & 1) + 1] = pack2(e[2], e[3]);
      st.l[it] += (e[0] + e[1]) + (e[2] + e[3]);
    }
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) {
      const int f = 4 * t + dc;
      if (f + kAhead < 16) kf[f + kAhead] = k_frag(k_lds, (f + kAhead) >> 2, (f + kAhead) & 3, lane);
      pin_reads();
#pragma unroll
      for (int it = 0; it < kIT; ++it)
        s[it][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[f], st.qf[it][dc],
                                                           dc == 0 ? st.c0[it] : s[it][t], 0, 0, 0);
    }
  }
#pragma unroll
  for (int it = 0; it < kIT; ++it)
#pragma unroll
    for (int c = 0; c < 2; ++c)
      pf[it][c] = __builtin_bit_cast(bf16x8, u32x4{w[it][c][0], w[it][c][1], w[it][c][2], w[it][c][3]});
}



// HPW query heads (of one kv head) per workgroup, HPW in {1, 2, 4, 8}: the
// workgroup covers BM = 32 * 8 / HPW query rows of each of its heads, and a
// kv head's G query heads are spread over G / HPW workgroups.
template <bool CAUSAL, int HPW>
__global__ __launch_bounds__(kThreads, 1) void gqa_fwd_kernel(Args p) {
  __shared__ __align__(1024) uint8_t smem[kLdsBytes];   // K slots, V slots, q staging area

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l16 = lane & 15;
  const int g = lane >> 4;

  // The instruction arbiter serves the older waves (0-3) of each SIMD first, and
  // they also issue the K/V DMAs; the younger waves get a higher issue priority
  // so both reach the per-iteration barrier together (1.3 % same-box).
  if (__builtin_amdgcn_readfirstlane(wave) >= kDmaWaves) __builtin_amdgcn_s_setprio(1);

  // ---- DMA geometry: instruction j of issuing wave w (< kDmaWaves) fills LDS
  // bytes [(j*kDmaWaves + w)*1024, +1024) of a tile = rows 4q .. 4q+3, lane -> (row, chunk).
  // Per-lane byte offsets within a tile (row * row_bytes + swizzled chunk) are
  // the same for every block; the LDS destination of each instruction is wave-uniform.
  const int64_t row_bytes = p.k_ss * 2;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  uint32_t koff[kDmaPerWave], voff[kDmaPerWave];
#pragma unroll
  for (int j = 0; j < kDmaPerWave; ++j) {
    const int r = dma_row(j, wave, lane);
    koff[j] = dma_lane_offset(row_bytes, r, dma_kcol(r, lane));
    voff[j] = dma_lane_offset(row_bytes, r, dma_vcol(r, lane));
  }
  // Rows past the sequence (only in the last, partial tile) are clamped to the
  // last key: their scores are masked and their V rows meet p = 0.
  auto issue = [&](const char* base, bool is_v, const uint32_t (&off)[kDmaPerWave], int kt,
                   uint32_t lds) {
    if (wave_u >= kDmaWaves) return;
    const int j0 = kt * kBN;
    const char* tb = base + (int64_t)j0 * row_bytes;
    if (j0 + kBN <= p.seq) {
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j)
        dma16(tb, off[j], lds + (uint32_t)((j * kDmaWaves + wave_u) * 1024));
    } else {
      // The last, partial tile (rare): its clamped offsets are computed here, from a
      // tile index the compiler may not treat as a constant, so that it does not
      // precompute them for the whole launch and hold them in registers.
      int ktv = kt;
      asm volatile("" : "+s"(ktv));
#pragma unroll
      for (int j = 0; j < kDmaPerWave; ++j) {
        const int r = dma_row(j, wave, lane);
        dma16(tb, dma_lane_offset(row_bytes, dma_src_row(p, ktv, r), is_v ? dma_vcol(r, lane) : dma_kcol(r, lane)),
              lds + (uint32_t)((j * kDmaWaves + wave_u) * 1024));
      }
    }
  };

  // Causal: persistent, this workgroup's blocks (sched_block), each (batch, kv
  // head, query heads, rows), longest first.  The last iterations of a block
  // prefetch the next block's first K/V tiles into the ring slots that follow its
  // own (ring_slot), so the next block starts without waiting for them.
  // Non-causal blocks are all equally long: one block per workgroup (the loop
  // runs once, and the compiler sees it).
  const int nb_total = total_blocks(p, HPW);
  int slot_base = 0;   // ring position of the current block's first tile
  int prev_nkt = 0;    // tile count of the previous block (0: none)
  int prev_w0 = 0;     // this wave's first query row in the previous block
  for (int kk = 0; CAUSAL || kk == 0; ++kk) {
  const int bid = sched_block(kk, (int)blockIdx.x, (int)gridDim.x);
  if (bid >= nb_total) break;
  const Block blk = block_of(p, CAUSAL, HPW, bid, wave);
  const int bid_next = sched_block(kk + 1, (int)blockIdx.x, (int)gridDim.x);
  const int w0 = __builtin_amdgcn_readfirstlane(blk.w0);   // this wave's first query row

  State st;
  {
    // Q fragments, scaled by scale*log2(e) and rounded to bf16 once: a
    // workgroup's first block loads them from global memory, later blocks read the
    // rows the previous block staged in LDS.  The staging DMAs were issued before
    // the previous block's 16 output stores (8 per 16 rows, issued when any of the
    // 16 rows exists), so waiting for them leaves the stores in flight when row
    // prev_w0 + 16 exists; otherwise wait for all.
    // The two paths are kept apart so the LDS path waits for no global load.
    auto to_frag = [&](const u32x4& raw) {
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = pack2(__builtin_bit_cast(float, raw[e] << 16) * p.scale_log2,
                     __builtin_bit_cast(float, raw[e] & 0xffff0000u) * p.scale_log2);
      return __builtin_bit_cast(bf16x8, w);
    };
    if (CAUSAL && kk > 0) {
      if (prev_w0 + 16 < p.seq) wait_vmcnt<kIT * kDT>();
      else wait_vmcnt<0>();
      const uint8_t* qs = smem + q_stage_offset(slot_base, wave_u);
#pragma unroll
      for (int it = 0; it < kIT; ++it) {
        const bool live = w0 + it * 16 + l16 < p.seq;
#pragma unroll
        for (int dc = 0; dc < 4; ++dc) {
          const u32x4 raw = *reinterpret_cast<const u32x4*>(qs + q_stage_pos(it * 16 + l16, dc * 4 + g));
          st.qf[it][dc] = to_frag(live ? raw : u32x4{0u, 0u, 0u, 0u});
        }
      }
    } else {
      const uint16_t* qp = p.q + q_head(p, blk);
#pragma unroll
      for (int it = 0; it < kIT; ++it) {
        const int row = w0 + it * 16 + l16;
#pragma unroll
        for (int dc = 0; dc < 4; ++dc)
          st.qf[it][dc] = to_frag((row < p.seq) ? *reinterpret_cast<const u32x4*>(qp + q_elem(p, row, dc, g))
                                                : u32x4{0u, 0u, 0u, 0u});
      }
    }
#pragma unroll
    for (int it = 0; it < kIT; ++it) {
#pragma unroll
      for (int dt = 0; dt < kDT; ++dt) st.o[it][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
      st.c0[it] = floatx4{0.f, 0.f, 0.f, 0.f};   // m = 0 until the first tile sets it
      st.l[it] = 0.f;
    }
  }

  const char* kbase = uniform_ptr(p.k + kv_head(p, blk));
  const char* vbase = uniform_ptr(p.v + kv_head(p, blk));
  auto k_tile = [&](int kt) { return smem + ring_slot(slot_base, kt) * kTileBytes; };
  auto v_tile = [&](int kt) { return smem + (kRing + ring_slot(slot_base, kt)) * kTileBytes; };

  const int nkt = blk.nkt;
  const int nfree = blk.nfree;   // tiles [0, nfree) need no mask for any row of this workgroup

  // Iteration kt (after the barrier that ends iteration kt-1) fetches K(kt+3) into
  // the slot of K(kt-1) and V(kt+1) into the slot of V(kt-3) (both last read in
  // iteration kt-2), then computes O += V(kt-1) P(kt-1), S(kt+1) and the softmax of
  // S(kt).  Each DMA has two iterations to land: the barrier that ends iteration
  // kt waits only for the DMAs issued in iteration kt-1 (K(kt+2), V(kt)), which
  // iteration kt+1 reads.  The prologue issues the first tiles the previous block
  // did not prefetch; the wait below covers both.
  // When every prologue tile was prefetched (and landed before the previous
  // block's stores), nothing is awaited here, so those stores stay in flight.
  const bool all_prefetched = prologue_all_prefetched(prev_nkt);
#pragma unroll
  for (int i = 0; i < kPrologueK; ++i)
    if (!prologue_k_prefetched(i, prev_nkt)) issue(kbase, false, koff, prologue_k_tile(i, nkt), lds_addr(k_tile(i)));
  if (!prologue_v_prefetched(prev_nkt)) issue(vbase, true, voff, 0, lds_addr(v_tile(0)));
  if (!all_prefetched) wait_vmcnt<0>();
  __syncthreads();
  floatx4 s[kIT][4];
  bf16x8 pf[kIT][2];
  float alpha[kIT];
  bf16x8 kf0[kAhead];   // first K fragments of the next block B, read at the end of block A
  scores(st, k_tile(0), lane, s);
  __syncthreads();

  // Past the last tile the DMAs fetch the next block's first tiles, or after the
  // last block the last tile again into a slot that is no longer read, so every
  // iteration issues the same number of DMAs and the wait below has a fixed count.
  // (The next block's geometry is worked out only in a block's last iterations.)
  auto fetch = [&](int kt) {
    if (kt + kPrologueK < nkt) {
      issue(kbase, false, koff, kt + kPrologueK, lds_addr(k_tile(kt + kPrologueK)));
      issue(vbase, true, voff, kt + 1, lds_addr(v_tile(kt + 1)));
    } else {
      const bool has_next = CAUSAL && bid_next < nb_total;
      const Block nxt = block_of(p, CAUSAL, HPW, has_next ? bid_next : bid, wave);
      const Fetch kf = k_fetch(kt, nkt, has_next, nxt.nkt);
      const Fetch vf = v_fetch(kt, nkt, has_next);
      const int64_t kvn = kv_head(p, nxt);
      issue(kf.next ? uniform_ptr(p.k + kvn) : kbase, false, koff, kf.tile, lds_addr(k_tile(kt + kPrologueK)));
      issue(vf.next ? uniform_ptr(p.v + kvn) : vbase, true, voff, vf.tile, lds_addr(v_tile(kt + 1)));
    }
  };
  // O moves to the running max set by the previous tile's statistics; done
  // before the next O += V P (and at the top of an iteration, so the branch does
  // not split the iteration's MFMA/softmax block).
  auto rescale = [&](bool any) {
    if (any) {
#pragma unroll
      for (int it = 0; it < kIT; ++it)
#pragma unroll
        for (int dt = 0; dt < kDT; ++dt) st.o[it][dt] *= alpha[it];
    }
  };
  auto finish = [&]() {
    // DMAs still allowed in flight: those issued in this iteration
    wait_vmcnt<2 * kDmaPerWave>();
    __syncthreads();
  };
  // The next block's q rows into LDS, at the start of the last iteration.
  const bool stage_next = CAUSAL && bid_next < nb_total;
  auto stage_q = [&]() {
    const Block nb = block_of(p, CAUSAL, HPW, bid_next, wave);
    const char* qsrc = uniform_ptr(p.q + q_head(p, nb) + (int64_t)q_src_row0(p, nb.w0) * p.q_ss);
    const uint32_t qlds = lds_addr(smem + q_stage_offset(ring_slot(slot_base, nkt), wave_u));
#pragma unroll
    for (int j = 0; j < kQStageDma; ++j)
      dma16(qsrc, q_dma_offset(p, nb.w0, q_dma_row(j, lane), q_dma_chunk(j, lane)), qlds + j * 1024);
  };

  // kt = 0: no O update yet.  The first tile sets every row's m to its max
  // (S(0) was computed with m = 0), before S(1) is computed from the new seed.
  float x[kIT];
  bool any = false;
  {
    fetch(0);
    if (nkt == 1 && stage_next) stage_q();
    if (nfree > 0) softmax_test<CAUSAL, false>(p, 0, w0, lane, s, x);
    else softmax_test<CAUSAL, true>(p, 0, w0, lane, s, x);
    softmax_raise<true>(st, s, x, alpha);
    if (nkt > 1) probs_then_scores<false>(st, k_tile(1), lane, s, pf, kf0);
    else softmax_probs(st, s, pf);
    // iteration 1 reads K(2) and V(0), issued in the prologue (awaited above) or
    // prefetched by the previous block (landed before its stores)
    if (all_prefetched) __syncthreads();
    else finish();
  }
  // Iteration body: block A = O += V(kt-1) P(kt-1) (36 MFMAs) with the row-max
  // test of S(kt); the rare running-max update; block B = the exponentials of
  // S(kt) with S(kt+1) (32 MFMAs).
  int kt = 1;
  const int n_mid_free = min(nfree, nkt - 1);
  for (; kt < n_mid_free; ++kt) {
    fetch(kt);
    rescale(any);
    accumulate_pv_k(st, v_tile(kt - 1), pf, lane, k_tile(kt + 1), kf0);
    any = softmax_test<CAUSAL, false>(p, kt, w0, lane, s, x);
    if (any) softmax_raise<false>(st, s, x, alpha);
    probs_then_scores<true>(st, k_tile(kt + 1), lane, s, pf, kf0);
    finish();
  }
  for (; kt < nkt - 1; ++kt) {
    fetch(kt);
    rescale(any);
    accumulate_pv_k(st, v_tile(kt - 1), pf, lane, k_tile(kt + 1), kf0);
    any = softmax_test<CAUSAL, true>(p, kt, w0, lane, s, x);
    if (any) softmax_raise<false>(st, s, x, alpha);
    probs_then_scores<true>(st, k_tile(kt + 1), lane, s, pf, kf0);
    finish();
  }
  if (kt == nkt - 1 && kt >= 1) {   // last tile: no S(kt+1)
    fetch(kt);
    if (stage_next) stage_q();
    rescale(any);
    accumulate_pv(st, v_tile(kt - 1), pf, lane);
    any = (kt < nfree) ? softmax_test<CAUSAL, false>(p, kt, w0, lane, s, x)
                       : softmax_test<CAUSAL, true>(p, kt, w0, lane, s, x);
    if (any) softmax_raise<false>(st, s, x, alpha);
    softmax_probs(st, s, pf);
    finish();
  }
  rescale(any);
  accumulate_pv(st, v_tile(nkt - 1), pf, lane);
  // The last fetches (the next block's first tiles, or after the last block
  // repeats of the last tile into slots no longer read) must land before the next
  // block reads them, and before the workgroup exits and its LDS is handed on.
  // The next block's staged q rows (the youngest DMAs) may stay in flight.
  if (stage_next) wait_vmcnt<kQStageDma>();
  else wait_vmcnt<0>();

  // ---- normalise and store: lane holds out[row][d = dt*16 + 4g .. +4]; the
  // row sum is the sum of the four lanes' parts
  uint16_t* op = p.out + out_head(p, blk);
#pragma unroll
  for (int it = 0; it < kIT; ++it) {
    const float inv = 1.0f / row_sum4(st.l[it]);
    const int row = w0 + it * 16 + l16;
    if (row >= p.seq) continue;
#pragma unroll
    for (int dt = 0; dt < kDT; ++dt) {
      const floatx4 o = st.o[it][dt] * inv;
      u32x2 w;
      w[0] = pack2(o[0], o[1]);
      w[1] = pack2(o[2], o[3]);
      *reinterpret_cast<u32x2*>(op + out_elem(p, row, dt, g)) = w;
    }
  }
  slot_base = ring_slot(slot_base, nkt);
  prev_nkt = nkt;
  prev_w0 = w0;
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
  if (hq % hkv)
    return set_error(KDA_ERR_INVALID_ARG,
                     "gqa_fwd_bf16: Hq=%lld is not a multiple of Hkv=%lld query heads per kv head",
                     (long long)hq, (long long)hkv);
  if (!(scale > 0.f)) return set_error(KDA_ERR_INVALID_ARG, "gqa_fwd_bf16: scale must be > 0");
  if (batch == 0 || seq == 0) return KDA_OK;
  if (!q || !k || !v || !out) return set_error(KDA_ERR_INVALID_ARG, "gqa_fwd_bf16: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || (reinterpret_cast<uintptr_t>(out) & 7))
    return set_error(KDA_ERR_INVALID_ARG, "gqa_fwd_bf16: q/k/v must be 16-byte, out 8-byte aligned");
  if ((out_stride_s % 4) || (out_stride_h % 4) || (out_stride_b % 4))
    return set_error(KDA_ERR_INVALID_ARG, "gqa_fwd_bf16: output strides must be multiples of 4");
  const int hpw = heads_per_workgroup(hq / hkv);
  const int64_t nblocks = grid_blocks(batch, seq, hq, hkv);
  if (nblocks > 0x7fffffff || seq > (1 << 30) || hq > (1 << 20))
    return set_error(KDA_ERR_UNSUPPORTED, "gqa_fwd_bf16: problem too large");
  // The K/V DMAs address a tile's rows from a scalar base with 32-bit per-lane
  // byte offsets (row * Hkv*D*2 + chunk start; rows 0..63, chunks start at most
  // 2*D - 16 bytes into a row).
  if ((kBN - 1) * (hkv * kD * 2) + (2 * kD - 16) > (int64_t)0xffffffff)
    return set_error(KDA_ERR_UNSUPPORTED,
                     "gqa_fwd_bf16: Hkv=%lld kv heads exceed the 32-bit DMA offsets of a key tile",
                     (long long)hkv);
  // Causal launches stage a wave's next 32 q rows by DMA with 32-bit per-lane
  // offsets (at most 31 * Hq*D*2 + 240 bytes).
  if (causal && hq > kMaxHqStaged)
    return set_error(KDA_ERR_UNSUPPORTED,
                     "gqa_fwd_bf16: Hq=%lld query heads exceed the 32-bit DMA offsets of the staged q rows "
                     "(causal: at most %lld)",
                     (long long)hq, (long long)kMaxHqStaged);

  const Args a = make_args(reinterpret_cast<const uint16_t*>(q), reinterpret_cast<const uint16_t*>(k),
                           reinterpret_cast<const uint16_t*>(v), reinterpret_cast<uint16_t*>(out), batch,
                           seq, hq, hkv, scale, out_stride_b, out_stride_s, out_stride_h);
  hipStream_t st = as_stream(stream);
  // causal: persistent, one workgroup per CU (or per block, if fewer)
  const dim3 grid((unsigned)(causal ? std::min<int64_t>(nblocks, device_cu_count()) : nblocks)), block(kThreads);
#define KDA_GQA_LAUNCH(H)                                                         \
  if (causal)                                                                     \
    hipLaunchKernelGGL((gqa_fwd_kernel<true, H>), grid, block, 0, st, a);         \
  else                                                                            \
    hipLaunchKernelGGL((gqa_fwd_kernel<false, H>), grid, block, 0, st, a);
  switch (hpw) {
    case 8: KDA_GQA_LAUNCH(8) break;
    case 4: KDA_GQA_LAUNCH(4) break;
    case 2: KDA_GQA_LAUNCH(2) break;
    default: KDA_GQA_LAUNCH(1) break;
  }
#undef KDA_GQA_LAUNCH
  return check_launch("gqa_fwd_bf16");
}
