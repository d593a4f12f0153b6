// Mamba selective scan, fp32 (NKIBench mamba), as a chunked parallel scan:
//
//   dA[c,s,m]  = exp(delta[c,m] * a[c,s])
//   dBu[c,s,m] = (delta[c,m] * b[s,m]) * u[c,m]
//   h[c,s,m]   = dA[c,s,m] * h[c,s,m-1] + dBu[c,s,m]        (h[c,s,-1] = 0)
//   out[c,m]   = sum_s c[s,m] * h[c,s,m]                     (s = 0, 1, ..., S-1 in order)
//
// delta, u [C, M]; a [C, S]; b, c [S, M]; out [C, M]; 1 <= S <= 16.
//
// The recurrence h -> dA*h + dBu composes associatively: two steps (A1, H1) then
// (A2, H2) are one step (A1*A2, A2*H1 + H2).  Mapping: one workgroup per channel,
// one wave per state s, the sequence in segments of 512 steps; lane l of a wave
// owns the chunk of 8 steps [512k + 8l, 512k + 8l + 8) of segment k.
//   1. Each lane evaluates dA and dBu of its 8 steps (exp bit-identical to
//      numpy's float32 exp) and folds them into the chunk's (A, H) from h = 0.
//   2. An inclusive scan of the chunk pairs within each 16-lane row (DPP row
//      shifts), the four row totals chained from the segment's entry state (a
//      per-wave carry, updated from lane 63 for the next segment), and each
//      lane's row-exclusive pair give every chunk its entry state.
//   3. Each lane re-runs its 8 steps from that entry state with the dA/dBu kept
//      in registers (mul then add per step, as numpy rounds), forms c*h, and
//      writes the products to LDS; after one barrier, 512 threads sum the S
//      products of each step in state order and store out coalesced.
// Precision: the chunk products A and the scan are in fp64.  A product of fp32
// factors near 1 rounded at every multiply drifts by a few 1e-6 over 7168 steps,
// the same order as the sequential reference's own rounding noise; in fp64 the
// only deviation from the sequential evaluation is where each chunk's entry
// state is rounded to fp32 (measured on the host: 1.8e-6 relative-L2 at
// C=256, M=7168, S=16, the sequential fp32 evaluation itself being 1.7e-6 from
// an fp64 recurrence on the same dA/dBu).
// exp must be numpy's: a correctly rounded or hardware exp differs from it by
// 1-2 ulp in a large fraction of arguments, and over a 7168-step product that
// alone moves the output by ~1e-5 relative.
#include <stdint.h>

#include "common.h"

namespace kda {
namespace mamba {

constexpr int kL = 8;            // steps per lane (one chunk)
constexpr int kSeg = 64 * kL;    // steps per segment (one wave of chunks)
constexpr int kMaxS = 16;        // states = waves per workgroup

struct Args {
  const float* delta;  // [C][M]
  const float* u;      // [C][M]
  const float* a;      // [C][S]
  const float* b;      // [S][M]
  const float* c;      // [S][M]
  float* out;          // [C][M]
  int M, S, nseg;
};

#pragma clang fp contract(off)

// ---- numpy's float32 exp --------------------------------------------------
// numpy evaluates np.exp on float32 (numpy/_core/src/umath/
// loops_exponent_log.dispatch.c.src, AVX2/AVX-512F) as: k = rint(x * log2 e);
// Cody-Waite reduction r = x - k*ln2 with ln2 in two parts (fused multiply-adds);
// exp(r) = P5(r) / Q2(r), a rational minimax approximation evaluated by Horner
// with fused multiply-adds and divided with correct rounding; scaled by 2^k;
// x >= 88.7228... gives inf, x <= -103.972... gives 0.  r lies in [-0.35, 0.35],
// so the numerator lies in [0.70, 1.42] and the denominator in [0.90, 1.10]; the
// reciprocal and three Newton/remainder steps below then give the correctly
// rounded quotient without the scaling and fix-up steps of a general division.

// P5(r) / Q2(r), correctly rounded, for N arguments (each step over all N first).
template <int N>
__device__ __forceinline__ void np_exp_rational(const float (&r)[N], float (&q)[N]) {
  float n[N], d[N], y[N];
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
}

// exp(x) in place, any x.
template <int N>
__device__ __forceinline__ void np_exp(float (&x)[N]) {
  const float kXmax = 0x1.62e43p+6f;    //  88.72283935546875
  const float kXmin = -0x1.9fe36ap+6f;  // -103.97208404541015625
  float k[N], r[N], q[N];
#pragma unroll
  for (int j = 0; j < N; ++j) k[j] = __builtin_rintf(x[j] * 0x1.715476p+0f);  // ties to even
#pragma unroll
  for (int j = 0; j < N; ++j) r[j] = __builtin_fmaf(k[j], -0x1.62e4p-1f, x[j]);
#pragma unroll
  for (int j = 0; j < N; ++j) r[j] = __builtin_fmaf(k[j], -0x1.7f7d1cp-20f, r[j]);
  np_exp_rational<N>(r, q);
#pragma unroll
  for (int j = 0; j < N; ++j) {
    float e = __builtin_ldexpf(q[j], (int)k[j]);
    e = (x[j] >= kXmax) ? __builtin_inff() : e;
    x[j] = (x[j] <= kXmin) ? 0.f : e;
  }
}

// exp(x) in place for |x| < 0.3: then k = rint(x * log2 e) = 0, both reduction
// steps return x exactly (fma(0, c, x) = x) and the scaling by 2^0 and the range
// tests change nothing, so this equals np_exp bit for bit.
template <int N>
__device__ __forceinline__ void np_exp_small(float (&x)[N]) {
  float q[N];
  np_exp_rational<N>(x, q);
#pragma unroll
  for (int j = 0; j < N; ++j) x[j] = q[j];
}

// ---- loads ------------------------------------------------------------------

// v[i] = row[m0 + i] for m0 + i < M, else 0.  FULL: the caller has established
// that the whole segment is inside the row and that rows are 16-byte aligned
// with M % 4 == 0, so a chunk is two float4 loads without tests.
template <bool FULL>
__device__ __forceinline__ void load_chunk(const float* row, int m0, int M, float (&v)[kL]) {
  if (FULL) {
    const floatx4 lo = *reinterpret_cast<const floatx4*>(row + m0);
    const floatx4 hi = *reinterpret_cast<const floatx4*>(row + m0 + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = lo[i];
      v[4 + i] = hi[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < kL; ++i) v[i] = (m0 + i < M) ? row[m0 + i] : 0.f;
  }
}

// The four inputs of segment `seg` for this lane; the in-bounds test is per
// segment (wave-uniform), so only the last segment takes the masked loads.
template <bool VEC>
__device__ __forceinline__ void load_segment(const float* drow, const float* urow,
                                             const float* brow, const float* crow, int seg,
                                             int lane, int M, float (&d)[kL], float (&u)[kL],
                                             float (&b)[kL], float (&c)[kL]) {
  const int m0 = seg * kSeg + lane * kL;
  if (VEC && (seg + 1) * kSeg <= M) {
    load_chunk<true>(drow, m0, M, d);
    load_chunk<true>(urow, m0, M, u);
    load_chunk<true>(brow, m0, M, b);
    load_chunk<true>(crow, m0, M, c);
  } else {
    load_chunk<false>(drow, m0, M, d);
    load_chunk<false>(urow, m0, M, u);
    load_chunk<false>(brow, m0, M, b);
    load_chunk<false>(crow, m0, M, c);
  }
}

// DPP move of an fp64 value (two 32-bit halves); lanes whose source lies outside
// their 16-lane row keep `ident`.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v, double ident) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint64_t o = __builtin_bit_cast(uint64_t, ident);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)o, (int)(uint32_t)u,
                                                            CTRL, 0xf, 0xf, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(
      (int)(uint32_t)(o >> 32), (int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ double readlane_d(double v, int l) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// One Hillis-Steele step of the inclusive scan within a 16-lane row: the pair of
// lane l - D (DPP row_shr:D) is composed before this lane's.  Lanes without a
// source receive the identity (1, 0), which composes exactly, so no lane test.
template <int D>
__device__ __forceinline__ void row_scan_step(double& A, double& H) {
  const double Ap = dpp_d<0x110 + D>(A, 1.0);
  const double Hp = dpp_d<0x110 + D>(H, 0.0);
  H = __builtin_fma(A, Hp, H);
  A = Ap * A;
}

// Buffers of one segment's inputs for one lane.
struct SegIn {
  float d[kL], u[kL], b[kL], c[kL];
};

// ---- kernel -----------------------------------------------------------------

// Segment k: chunk aggregates, entry states, the re-run with c*h into LDS, one
// barrier, then the state sums of the segment's steps.  `nxt` receives the
// inputs of segment k + 1 (issued first, used by the next call).
template <bool VEC>
__device__ __forceinline__ void segment(const Args& p, int k, int lane, int s, const float* drow,
                                        const float* urow, const float* brow, const float* crow,
                                        float a_s, const SegIn& cur, SegIn& nxt, double& hseg,
                                        float (&prod)[2][kMaxS][kSeg]) {
  const int M = p.M;
  if (k + 1 < p.nseg)
    load_segment<VEC>(drow, urow, brow, crow, k + 1, lane, M, nxt.d, nxt.u, nxt.b, nxt.c);
  // dA (in x) and dBu, rounded as numpy rounds them
  float x[kL], bu[kL];
  bool small = true;
#pragma unroll
  for (int i = 0; i < kL; ++i) {
    x[i] = cur.d[i] * a_s;
    bu[i] = (cur.d[i] * cur.b[i]) * cur.u[i];
    small = small && __builtin_fabsf(x[i]) < 0.3f;
  }
  // in two halves of 4: fewer live temporaries
  float(&x0)[4] = *reinterpret_cast<float(*)[4]>(x);
  float(&x1)[4] = *reinterpret_cast<float(*)[4]>(x + 4);
  if (__builtin_amdgcn_ballot_w64(!small) == 0) {
    np_exp_small<4>(x0);
    np_exp_small<4>(x1);
  } else {
    np_exp<4>(x0);
    np_exp<4>(x1);
  }
  if ((k + 1) * kSeg > M) {   // last segment: steps past the sequence are identities
    const int m0 = k * kSeg + lane * kL;
#pragma unroll
    for (int i = 0; i < kL; ++i)
      if (m0 + i >= M) {
        x[i] = 1.f;
        bu[i] = 0.f;
      }
  }
  // 1. chunk aggregate from h = 0
  float hl = bu[0];
  double A = (double)x[0];
#pragma unroll
  for (int i = 1; i < kL; ++i) {
    hl = __builtin_fmaf(x[i], hl, bu[i]);
    A *= (double)x[i];
  }
  double H = (double)hl;
  // 2. entry state of every chunk: inclusive scan within each 16-lane row, the row
  //    totals (lanes 15, 31, 47, 63) chained from the segment's entry state, and
  //    each lane's row-exclusive pair applied to its row's entry state
  row_scan_step<1>(A, H);
  row_scan_step<2>(A, H);
  row_scan_step<4>(A, H);
  row_scan_step<8>(A, H);
  const double Ax = dpp_d<0x111>(A, 1.0);
  const double Hx = dpp_d<0x111>(H, 0.0);
  const double h_r0 = hseg;
  const double h_r1 = __builtin_fma(readlane_d(A, 15), h_r0, readlane_d(H, 15));
  const double h_r2 = __builtin_fma(readlane_d(A, 31), h_r1, readlane_d(H, 31));
  const double h_r3 = __builtin_fma(readlane_d(A, 47), h_r2, readlane_d(H, 47));
  hseg = __builtin_fma(readlane_d(A, 63), h_r3, readlane_d(H, 63));
  const int row = lane >> 4;
  const double h_row = row == 0 ? h_r0 : row == 1 ? h_r1 : row == 2 ? h_r2 : h_r3;
  float h = (float)__builtin_fma(Ax, h_row, Hx);
  // 3. the 8 steps again from the entry state, multiply then add as numpy rounds
  //    (within the first chunk the result is the sequential one bit for bit);
  //    c*h to LDS
  float pr[kL];
#pragma unroll
  for (int i = 0; i < kL; ++i) {
    h = x[i] * h + bu[i];
    pr[i] = cur.c[i] * h;
  }
  float* dst = &prod[k & 1][s][lane * kL];
  *reinterpret_cast<floatx4*>(dst) = floatx4{pr[0], pr[1], pr[2], pr[3]};
  *reinterpret_cast<floatx4*>(dst + 4) = floatx4{pr[4], pr[5], pr[6], pr[7]};
  __syncthreads();
  // out = sum over states in order; the other buffer is free again because every
  // thread finished the previous segment's sums before reaching this barrier
  const int nthreads = 64 * p.S;
  for (int j = threadIdx.x; j < kSeg; j += nthreads) {
    const int m = k * kSeg + j;
    float v[kMaxS];
#pragma unroll
    for (int s2 = 0; s2 < kMaxS; ++s2) v[s2] = (s2 < p.S) ? prod[k & 1][s2][j] : 0.f;
    float acc = v[0];
#pragma unroll
    for (int s2 = 1; s2 < kMaxS; ++s2)
      if (s2 < p.S) acc += v[s2];
    if (m < M) p.out[(int64_t)blockIdx.x * M + m] = acc;
  }
}

template <bool VEC>
__global__ __launch_bounds__(64 * kMaxS) void chunk_scan_kernel(Args p) {
  __shared__ __align__(16) float prod[2][kMaxS][kSeg];   // c*h per state, two segments

  const int lane = threadIdx.x & 63;
  const int s = threadIdx.x >> 6;           // this wave's state
  const int M = p.M;
  const int64_t ch = blockIdx.x;
  const float* drow = p.delta + ch * M;
  const float* urow = p.u + ch * M;
  const float* brow = p.b + (int64_t)s * M;
  const float* crow = p.c + (int64_t)s * M;
  const float a_s = p.a[ch * p.S + s];

  // Inputs are loaded one segment ahead into two buffers used in turn (the loop
  // body covers two segments, so neither buffer is copied).
  SegIn in0, in1;
  load_segment<VEC>(drow, urow, brow, crow, 0, lane, M, in0.d, in0.u, in0.b, in0.c);
  double hseg = 0.0;                   // state entering the segment
  for (int k = 0; k < p.nseg; k += 2) {
    segment<VEC>(p, k, lane, s, drow, urow, brow, crow, a_s, in0, in1, hseg, prod);
    if (k + 1 < p.nseg)
      segment<VEC>(p, k + 1, lane, s, drow, urow, brow, crow, a_s, in1, in0, hseg, prod);
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
  if (channels > INT32_MAX || seq > INT32_MAX - kSeg || channels * seq > ((int64_t)1 << 40))
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
  p.nseg = (int)((seq + kSeg - 1) / kSeg);
  const bool vec = (seq % 4 == 0) && aligned16(delta) && aligned16(u) && aligned16(b) &&
                   aligned16(c);
  const dim3 grid((unsigned)channels), block((unsigned)(64 * states));
  if (vec)
    hipLaunchKernelGGL(chunk_scan_kernel<true>, grid, block, 0, as_stream(stream), p);
  else
    hipLaunchKernelGGL(chunk_scan_kernel<false>, grid, block, 0, as_stream(stream), p);
  return check_launch(what);
}
