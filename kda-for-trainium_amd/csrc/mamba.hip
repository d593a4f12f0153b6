// Mamba selective scan, fp32 (NKIBench mamba), bit-identical to the numpy
// definition it restates:
//
//   dA[c,s,m]  = exp(delta[c,m] * a[c,s])
//   dBu[c,s,m] = (delta[c,m] * b[s,m]) * u[c,m]
//   h[c,s,m]   = dA[c,s,m] * h[c,s,m-1] + dBu[c,s,m]        (h[c,s,-1] = 0)
//   out[c,m]   = sum_s c[s,m] * h[c,s,m]
//
// delta, u [C, M]; a [C, S]; b, c [S, M]; out [C, M]; 1 <= S <= 16.
//
// Every rounding follows the numpy evaluation: separate multiply and add (no
// contraction), exp evaluated as numpy's float32 SIMD exp evaluates it, and the
// sum over s in numpy's pairwise order.  The recurrence runs sequentially over m
// for each (c, s): any re-association of the scan (a chunked or tree scan) rounds
// differently, and in fp32 those differences accumulate to a few 1e-6 relative
// over a 7168-step sequence.
//
// Mapping: one workgroup per channel, 1 + kT/64 waves, the sequence in blocks of
// kT steps; dA/dBu triple-buffered in LDS, state checkpoints double-buffered.
//   wave 0 (lanes 0..15, one per state) runs the recurrence over block k: two
//     dependent VALU ops per step, operands read four steps at a time
//     (ds_read_b128); it stores h only after every second step (a checkpoint),
//     two ds_write_b128 per 16 steps;
//   waves 1..kT/64 (kT lanes, one step each) meanwhile produce dA and dBu for block
//     k+1 (coalesced loads of delta, u, b; 16 exps per lane) and reduce block k-1:
//     each lane recomputes h of its step from the checkpoint before its step pair
//     with the same multiply and add (bit-identical), then sums h * c over s in
//     numpy's order and stores out (coalesced).
// One barrier per block.  LDS rows are padded to kT+4 floats so the 16 state rows
// read by wave 0 fall on distinct banks.
#include <math.h>
#include <stddef.h>

#include "common.h"
#include "lds_dma.h"

namespace kda {
namespace mamba {

constexpr int kT = 320;            // steps per block (= producer lanes; 192 measured 23 % slower)
constexpr int kRow = kT + 4;       // LDS row stride in floats
constexpr int kCkRow = 4 + kT / 2; // checkpoint row: [3] = h entering the block, [4 + i] = h after pair i
constexpr int kMaxS = 16;
constexpr int kThreads = 64 + kT;  // recurrence wave + producer waves

struct Args {
  const float* delta;  // [C][M]
  const float* u;      // [C][M]
  const float* a;      // [C][S]
  const float* b;      // [S][M]
  const float* c;      // [S][M]
  float* out;          // [C][M]
  int M, S, nb;
};

#pragma clang fp contract(off)

// float32 exp evaluated the way numpy's SIMD loops evaluate np.exp on float32
// (AVX2/FMA3 and AVX-512F share it; numpy/_core/src/umath/
// loops_exponent_log.dispatch.c.src): k = rint(x*log2 e); Cody-Waite reduction
// r = x - k ln2 with ln2 split in two parts (fused multiply-adds);
// exp(r) = P5(r)/Q2(r), a rational minimax approximation evaluated by Horner with
// fused multiply-adds and a correctly rounded division; result scaled by 2^k;
// x >= 88.7228... gives inf, x <= -103.972... gives 0, NaN stays NaN.
// Agrees bit for bit with np.exp on float32 over the sampled range [-104, 89].
//
// The division: r always lies in [-0.35, 0.35], so the numerator lies in
// [0.70, 1.42] and the denominator in [0.90, 1.10].  For such operands the
// general division (v_div_scale / v_div_fmas / v_div_fixup around a reciprocal
// and three Newton/remainder steps) neither scales nor fixes up, so the core
// sequence alone below gives the same correctly rounded quotient.
//
// Evaluates N arguments in place, each step applied to all N before the next
// (N = 1 in the scan: interleaving eight exps by hand was measured 6 % slower
// there than the compiler's own schedule).
template <int N>
__device__ __forceinline__ void np_expf_n(float (&x)[N]) {
  const float kXmax = 0x1.62e43p+6f;    //  88.72283935546875
  const float kXmin = -0x1.9fe36ap+6f;  // -103.97208404541015625
  float k[N], r[N], n[N], d[N], y[N], q[N];
#pragma unroll
  for (int j = 0; j < N; ++j) k[j] = __builtin_rintf(x[j] * 0x1.715476p+0f);  // log2(e); ties to even
#pragma unroll
  for (int j = 0; j < N; ++j) r[j] = __builtin_fmaf(k[j], -0x1.62e4p-1f, x[j]);
#pragma unroll
  for (int j = 0; j < N; ++j) r[j] = __builtin_fmaf(k[j], -0x1.7f7d1cp-20f, r[j]);
#pragma unroll
  for (int j = 0; j < N; ++j) {
    n[j] = __builtin_fmaf(0x1.0a7bbp-11f, r[j], 0x1.bae2b2p-8f);
    d[j] = __builtin_fmaf(0x1.61d064p-6f, r[j], -0x1.18d0aep-2f);
  }
#pragma unroll
  for (int j = 0; j < N; ++j) {
    n[j] = __builtin_fmaf(n[j], r[j], 0x1.a2fb18p-5f);
    d[j] = __builtin_fmaf(d[j], r[j], 1.0f);
  }
#pragma unroll
  for (int j = 0; j < N; ++j) {
    n[j] = __builtin_fmaf(n[j], r[j], 0x1.fa98bp-3f);
    y[j] = __builtin_amdgcn_rcpf(d[j]);
  }
#pragma unroll
  for (int j = 0; j < N; ++j) n[j] = __builtin_fmaf(n[j], r[j], 0x1.7397aap-1f);
#pragma unroll
  for (int j = 0; j < N; ++j) y[j] = __builtin_fmaf(__builtin_fmaf(-d[j], y[j], 1.0f), y[j], y[j]);
#pragma unroll
  for (int j = 0; j < N; ++j) n[j] = __builtin_fmaf(n[j], r[j], 1.0f);
#pragma unroll
  for (int j = 0; j < N; ++j) q[j] = n[j] * y[j];
#pragma unroll
  for (int j = 0; j < N; ++j) q[j] = __builtin_fmaf(__builtin_fmaf(-d[j], q[j], n[j]), y[j], q[j]);
#pragma unroll
  for (int j = 0; j < N; ++j) q[j] = __builtin_fmaf(__builtin_fmaf(-d[j], q[j], n[j]), y[j], q[j]);
#pragma unroll
  for (int j = 0; j < N; ++j) {
    float e = __builtin_ldexpf(q[j], (int)k[j]);
    e = (x[j] >= kXmax) ? __builtin_inff() : e;
    x[j] = (x[j] <= kXmin) ? 0.f : e;
  }
}

// numpy's pairwise summation of n <= 16 contiguous floats (the reduction loop of
// np.add.reduce over a contiguous axis): n < 8 sequentially from 0; otherwise
// eight partial sums (a[j] + a[j+8] when n == 16), combined as a balanced tree,
// then the remaining a[8..n) added in order.
__device__ __forceinline__ float np_pairwise_sum16(const float (&v)[kMaxS], int n) {
  if (n < 8) {
    float o = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      if (s < n) o += v[s];
    return o;
  }
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = (n == 16) ? v[j] + v[j + 8] : v[j];
  float o = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  if (n < 16) {
#pragma unroll
    for (int s = 8; s < 16; ++s)
      if (s < n) o += v[s];
  }
  return o;
}

// dA/dBu of block k live in buffer k % 3 (produced in iteration k-1, consumed by
// the recurrence in iteration k, re-read by the reduction in iteration k+1); the
// checkpoints of block k in buffer k % 2 (written in iteration k, read in k+1).
struct Smem {
  float da[3][kMaxS][kRow];
  float dbu[3][kMaxS][kRow];
  float ck[2][kMaxS][kCkRow];
};

// Per-step inputs of one block, held in registers one block ahead of their use.
struct StepIn {
  float d, u, b[kMaxS];
};

__device__ __forceinline__ void load_step(StepIn& x, const Args& p, int64_t row, int t, int blk) {
  const int m0 = blk * kT;
  if (blk < p.nb && t < p.M - m0) {
    x.d = p.delta[row + m0 + t];
    x.u = p.u[row + m0 + t];
    // rows s >= S repeat row S-1 (no per-state condition, which became 16
    // branches): those states never reach the output
#pragma unroll
    for (int s = 0; s < kMaxS; ++s) x.b[s] = p.b[(int64_t)min(s, p.S - 1) * p.M + m0 + t];
  }
}

__device__ __forceinline__ void load_c(float (&cv)[kMaxS], const Args& p, int t, int blk) {
  const int m0 = blk * kT;
  if (t < p.M - m0) {
#pragma unroll
    for (int s = 0; s < kMaxS; ++s) cv[s] = p.c[(int64_t)min(s, p.S - 1) * p.M + m0 + t];
  }
}

// dA and dBu of step t of block `blk` into buffer `buf`; the padding steps up to
// the next multiple of 16 get dA = 1, dBu = 0 (the recurrence passes h through
// them unchanged).  States s >= S are computed like the others (from a = 0 and
// row S-1 of b): a per-state condition here became 16 branches (2 % slower);
// their h never reaches the output (the reduction masks s >= S).
__device__ __forceinline__ void produce(Smem& sm, const Args& p, const StepIn& x,
                                        const float (&av)[kMaxS], int t, int blk, int buf) {
  const int len = min(kT, p.M - blk * kT);
  if (t < len) {
#pragma unroll
    for (int s = 0; s < kMaxS; ++s) {
      float e[1] = {x.d * av[s]};
      np_expf_n(e);
      sm.da[buf][s][t] = e[0];
      sm.dbu[buf][s][t] = (x.d * x.b[s]) * x.u;
    }
  } else if (t < ((len + 15) & ~15)) {
#pragma unroll
    for (int s = 0; s < kMaxS; ++s) {
      sm.da[buf][s][t] = 1.f;
      sm.dbu[buf][s][t] = 0.f;
    }
  }
}

// out[m0 + t] = sum_s h[s][t] * c[s][m0 + t] for block `blk` (dA/dBu in buffer
// `buf`, checkpoints in `cbuf`).  h[s][t] is recomputed from the checkpoint h
// before the step pair of t over the pair's steps up to t, with the
// recurrence's own multiply and add, so it equals the value the recurrence had.
__device__ __forceinline__ void reduce(const Smem& sm, const Args& p, const float (&cv)[kMaxS],
                                       int64_t row, int t, int blk, int buf, int cbuf) {
  const int m0 = blk * kT;
  if (t >= min(kT, p.M - m0)) return;
  const int q = t & 1, t0 = t - q;
  float v[kMaxS];
  // Eight states at a time: all LDS reads first, then both steps of the pair
  // computed unconditionally (the empty asm keeps the compiler from turning the
  // per-lane choice of step into branches, which serialised the reads state by
  // state) and the step of this lane selected.
#pragma unroll
  for (int s0 = 0; s0 < kMaxS; s0 += 8) {
    float2 a[8], b[8];
    float h0[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a[j] = *reinterpret_cast<const float2*>(&sm.da[buf][s0 + j][t0]);
      b[j] = *reinterpret_cast<const float2*>(&sm.dbu[buf][s0 + j][t0]);
      h0[j] = sm.ck[cbuf][s0 + j][3 + t0 / 2];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float h1 = a[j].x * h0[j] + b[j].x;
      const float h2 = a[j].y * h1 + b[j].y;
      asm volatile("" ::"v"(h1), "v"(h2));
      const float h = q ? h2 : h1;
      v[s0 + j] = (s0 + j < p.S) ? h * cv[s0 + j] : 0.f;
    }
  }
  p.out[row + m0 + t] = np_pairwise_sum16(v, p.S);
}

// The recurrence over `groups` groups of 16 steps of one block, for the state of
// this lane: h = dA * h + dBu per step (separate multiply and add).  `da` is the
// LDS byte address of the lane's dA row (its dBu row follows kDbuOff bytes
// later), `ck` that of its checkpoint row: h entering the block goes to entry 3,
// h after step pair i of the block to entry 4 + i.
//
// Inline asm with fixed registers and explicit LDS waits.  Compiled code was
// measured 13 % slower with per-step h stores: the compiler waited for the whole
// LDS queue once per 16 steps (its wait counts turn conservative across the
// loop) and reused the registers of pending stores for the chain.  Stores are
// what costs here: a ds_write_b128 of h every 4 steps added 7.5 cycles per step
// to the 13.8 of the bare 2-op chain (gfx950), wherever it was placed.  Storing
// h after every second step halves that; the reduction recomputes the step in
// between (checkpoints every 4 steps made the reduction's recomputation the
// bottleneck instead).  In this loop:
//   operands of group g (dA, dBu: v128..v159 or v160..v191, alternately) are
//   read one group ahead with ds_read_b128, four steps per read;
//   each step pair runs its first step into v192 and its second into a
//   checkpoint register (v200..v207 for groups on the first operand set,
//   v208..v215 on the second), which also carries h into the next pair; the
//   eight checkpoints of a group go out in two ds_write_b128 and are not
//   rewritten for another group;
//   each group starts with lgkmcnt(2): all but the previous group's two
//   checkpoint stores (issued after the operand reads) have completed, i.e. this
//   group's operands are in registers.
// The last group also reads the 16 steps after the block (unused): at most
// 16 floats past the end of a row, which stays inside Smem (a row is followed by
// the next row, the dBu array or the checkpoint array).
#define KDA_S(x) #x
#define KDA_RD(lo, hi, off) "ds_read_b128 v[" KDA_S(lo) ":" KDA_S(hi) "], %[da] offset:" KDA_S(off) "\n\t"
#define KDA_STEP(o, a, b, hin) \
  "v_mul_f32 v" KDA_S(o) ", v" KDA_S(a) ", v" KDA_S(hin) "\n\t" \
  "v_add_f32 v" KDA_S(o) ", v" KDA_S(b) ", v" KDA_S(o) "\n\t"
// two steps on dA in a0, a1, dBu in b0, b1, h entering in hin, leaving in ck
#define KDA_PAIR(a0, a1, b0, b1, hin, ck) KDA_STEP(192, a0, b0, hin) KDA_STEP(ck, a1, b1, 192)
// 16 steps on operand set X (dA v128..v143, dBu v144..v159; checkpoints
// v200..v207, h entering in v215) or Y (v160.., v176..; v208..v215, h in v207)
#define KDA_GROUP_X                                                                     \
  KDA_PAIR(128, 129, 144, 145, 215, 200) KDA_PAIR(130, 131, 146, 147, 200, 201)         \
  KDA_PAIR(132, 133, 148, 149, 201, 202) KDA_PAIR(134, 135, 150, 151, 202, 203)         \
  "ds_write_b128 %[ck], v[200:203] offset:16\n\t"                                        \
  KDA_PAIR(136, 137, 152, 153, 203, 204) KDA_PAIR(138, 139, 154, 155, 204, 205)         \
  KDA_PAIR(140, 141, 156, 157, 205, 206) KDA_PAIR(142, 143, 158, 159, 206, 207)         \
  "ds_write_b128 %[ck], v[204:207] offset:32\n\t"
#define KDA_GROUP_Y                                                                     \
  KDA_PAIR(160, 161, 176, 177, 207, 208) KDA_PAIR(162, 163, 178, 179, 208, 209)         \
  KDA_PAIR(164, 165, 180, 181, 209, 210) KDA_PAIR(166, 167, 182, 183, 210, 211)         \
  "ds_write_b128 %[ck], v[208:211] offset:16\n\t"                                        \
  KDA_PAIR(168, 169, 184, 185, 211, 212) KDA_PAIR(170, 171, 186, 187, 212, 213)         \
  KDA_PAIR(172, 173, 188, 189, 213, 214) KDA_PAIR(174, 175, 190, 191, 214, 215)         \
  "ds_write_b128 %[ck], v[212:215] offset:32\n\t"
// a group's operands into set X / Y: dA at the four offsets past %[da], dBu at
// the four offsets after them (kDbuOff further on)
#define KDA_READ_X(off0, off1, off2, off3, boff0, boff1, boff2, boff3)          \
  KDA_RD(128, 131, off0) KDA_RD(132, 135, off1) KDA_RD(136, 139, off2)         \
  KDA_RD(140, 143, off3) KDA_RD(144, 147, boff0) KDA_RD(148, 151, boff1)        \
  KDA_RD(152, 155, boff2) KDA_RD(156, 159, boff3)
#define KDA_READ_Y(off0, off1, off2, off3, boff0, boff1, boff2, boff3)          \
  KDA_RD(160, 163, off0) KDA_RD(164, 167, off1) KDA_RD(168, 171, off2)         \
  KDA_RD(172, 175, off3) KDA_RD(176, 179, boff0) KDA_RD(180, 183, boff1)        \
  KDA_RD(184, 187, boff2) KDA_RD(188, 191, boff3)
#define KDA_ADVANCE "v_add_u32 %[da], 64, %[da]\n\tv_add_u32 %[ck], 32, %[ck]\n\t"

constexpr int kDbuOff = 62208;  // bytes from a dA row to its dBu row (spelled out in the asm)
static_assert(sizeof(Smem::da) == kDbuOff && offsetof(Smem, dbu) == kDbuOff &&
                  offsetof(Smem, ck) == 2 * kDbuOff && kCkRow % 4 == 0,
              "recurrence asm assumes Smem = da, dbu (62208 bytes each), ck");

__device__ __forceinline__ void recurrence(float& h, uint32_t da, uint32_t ck, int groups) {
  int left;
  asm volatile(
      "s_waitcnt lgkmcnt(0)\n\t"
      KDA_READ_X(0, 16, 32, 48, 62208, 62224, 62240, 62256)
      "v_mov_b32 v215, %[h]\n\t"
      "ds_write_b32 %[ck], v215 offset:12\n\t"
      "s_mov_b32 %[left], %[groups]\n\t"
      "s_waitcnt lgkmcnt(0)\n\t"
      "L_mamba_rec_%=:\n\t"
      "s_waitcnt lgkmcnt(2)\n\t"
      KDA_READ_Y(64, 80, 96, 112, 62272, 62288, 62304, 62320)
      KDA_GROUP_X
      KDA_ADVANCE
      "s_sub_u32 %[left], %[left], 1\n\t"
      "s_cmp_eq_u32 %[left], 0\n\t"
      "s_cbranch_scc1 L_mamba_rec_end_x_%=\n\t"
      "s_waitcnt lgkmcnt(2)\n\t"
      KDA_READ_X(64, 80, 96, 112, 62272, 62288, 62304, 62320)
      KDA_GROUP_Y
      KDA_ADVANCE
      "s_sub_u32 %[left], %[left], 1\n\t"
      "s_cmp_eq_u32 %[left], 0\n\t"
      "s_cbranch_scc0 L_mamba_rec_%=\n\t"
      "v_mov_b32 %[h], v215\n\t"
      "s_branch L_mamba_rec_done_%=\n\t"
      "L_mamba_rec_end_x_%=:\n\t"
      "v_mov_b32 %[h], v207\n\t"
      "L_mamba_rec_done_%=:\n\t"
      "s_waitcnt lgkmcnt(0)"
      : [h] "+v"(h), [da] "+v"(da), [ck] "+v"(ck), [left] "=&s"(left)
      : [groups] "s"(groups)
      : "memory", "scc", "v128", "v129", "v130", "v131", "v132", "v133", "v134", "v135", "v136",
        "v137", "v138", "v139", "v140", "v141", "v142", "v143", "v144", "v145", "v146", "v147",
        "v148", "v149", "v150", "v151", "v152", "v153", "v154", "v155", "v156", "v157", "v158",
        "v159", "v160", "v161", "v162", "v163", "v164", "v165", "v166", "v167", "v168", "v169",
        "v170", "v171", "v172", "v173", "v174", "v175", "v176", "v177", "v178", "v179", "v180",
        "v181", "v182", "v183", "v184", "v185", "v186", "v187", "v188", "v189", "v190", "v191",
        "v192", "v200", "v201", "v202", "v203", "v204", "v205", "v206", "v207", "v208", "v209",
        "v210", "v211", "v212", "v213", "v214", "v215");
}
#undef KDA_S
#undef KDA_RD
#undef KDA_STEP
#undef KDA_PAIR
#undef KDA_GROUP_X
#undef KDA_GROUP_Y
#undef KDA_READ_X
#undef KDA_READ_Y
#undef KDA_ADVANCE

__global__ __launch_bounds__(kThreads) void scan_kernel(Args p) {
  __shared__ __align__(16) Smem sm;
  const int64_t row = (int64_t)blockIdx.x * p.M;
  const int tid = threadIdx.x;
  if (tid < 64) {
    // recurrence wave: lane s carries h[c, s] through the whole sequence
    const int s = tid;
    float h = 0.f;
    __syncthreads();  // block 0 produced
    for (int k = 0; k < p.nb; ++k) {
      const int steps = (min(kT, p.M - k * kT) + 15) & ~15;
      if (s < kMaxS)
        recurrence(h, lds_addr(&sm.da[k % 3][s][0]), lds_addr(&sm.ck[k & 1][s][0]), steps / 16);
      __syncthreads();  // block k consumed and its checkpoints written
    }
  } else {
    const int t = tid - 64;
    float av[kMaxS];
#pragma unroll
    for (int s = 0; s < kMaxS; ++s) av[s] = (s < p.S) ? p.a[(int64_t)blockIdx.x * p.S + s] : 0.f;
    // Register prefetch: the inputs of block k+2 and c of block k are loaded in
    // iteration k, one iteration before their use.
    StepIn cur, nxt;
    float c_use[kMaxS], c_nxt[kMaxS];
    load_step(cur, p, row, t, 0);
    load_step(nxt, p, row, t, 1);
    produce(sm, p, cur, av, t, 0, 0);
    __syncthreads();
    for (int k = 0; k < p.nb; ++k) {
      cur = nxt;  // block k+1
      load_step(nxt, p, row, t, k + 2);
#pragma unroll
      for (int s = 0; s < kMaxS; ++s) c_use[s] = c_nxt[s];  // block k-1
      load_c(c_nxt, p, t, k);
      if (k + 1 < p.nb) produce(sm, p, cur, av, t, k + 1, (k + 1) % 3);
      if (k >= 1) reduce(sm, p, c_use, row, t, k - 1, (k - 1) % 3, (k - 1) & 1);
      __syncthreads();  // block k's checkpoints written by the recurrence wave
    }
    reduce(sm, p, c_nxt, row, t, p.nb - 1, (p.nb - 1) % 3, (p.nb - 1) & 1);
  }
}

#pragma clang fp contract(on)

}  // namespace mamba
}  // namespace kda

using namespace kda;
using namespace kda::mamba;

extern "C" int kda_mamba_f32(const float* delta, const float* u, const float* a, const float* b,
                             const float* c, float* out, int64_t channels, int64_t seq,
                             int64_t states, void* stream) {
  clear_error();
  const char* what = "mamba_f32";
  if (channels < 0 || seq < 0 || states < 0)
    return set_error(KDA_ERR_INVALID_ARG, "%s: negative size", what);
  if (states < 1 || states > kMaxS)
    return set_error(KDA_ERR_UNSUPPORTED, "%s: states=%lld outside 1..%d", what, (long long)states,
                     kMaxS);
  if (channels > INT32_MAX || seq > INT32_MAX - kT)
    return set_error(KDA_ERR_UNSUPPORTED, "%s: problem too large", what);
  if (channels == 0 || seq == 0) return KDA_OK;
  if (!delta || !u || !a || !b || !c || !out)
    return set_error(KDA_ERR_INVALID_ARG, "%s: null pointer", what);
  Args p;
  p.delta = delta;
  p.u = u;
  p.a = a;
  p.b = b;
  p.c = c;
  p.out = out;
  p.M = (int)seq;
  p.S = (int)states;
  p.nb = (int)((seq + kT - 1) / kT);
  hipLaunchKernelGGL(scan_kernel, dim3((unsigned)channels), dim3(kThreads), 0, as_stream(stream), p);
  return check_launch(what);
}
