// bf16 GEMM family on gfx950 MFMA (v_mfma_f32_16x16x32_bf16), fp32 accumulation.
//
//   C[M,N] = A[M,K] @ B[K,N]      bf16 operands, bf16 (or fp32) output
//
// Data path (per workgroup = one BM x BN output tile, 4 waves in a 2 x 2 grid,
// each wave owning a (BM/2) x (BN/2) accumulator block in AGPR/VGPR):
//
//   HBM --global_load_lds_dwordx4--> LDS (2-stage ring, BK = 64) --ds_read--> MFMA
//
//   * Operands go straight from global memory into LDS (16 bytes per lane, no
//     register staging, no VALU work): each wave instruction fills 1 KiB of
//     LDS lane-linearly, so the LDS swizzle is applied on the global side by
//     choosing which 16-byte chunk each lane fetches.
//   * K-contiguous operands (A row-major) are stored [rows][64 k], 128 B rows,
//     16-byte chunk c of row r at position c ^ kswz(r); one ds_read_b128 gives
//     an MFMA fragment (one row, 8 consecutive k).
//   * MN-contiguous operands (B row-major [K][N], or A stored [K][M]) are kept in
//     their HBM orientation: [64 k][cols], 32-byte segment s of row k at
//     position s ^ mswz(k).  The fragment (one column, 8 consecutive k) is read
//     with two ds_read_b64_tr_b16: within each 16-lane group, lane 4r+q names
//     4 elements of k-row r and lane j receives column j of that 4 x 16 block,
//     i.e. the transpose happens in the LDS read.
//   * Both swizzles keep the fragment reads free of bank conflicts for 16 (or
//     32) lanes serviced together.
//   * Pipeline: the DMA of k-tile kt+1 is issued right after the barrier that
//     publishes k-tile kt, so it overlaps the 2 x TM x TN MFMAs of tile kt.
//     One s_waitcnt vmcnt(0) + s_barrier per k-tile; no fences.
//
// MFMA operand order: the B fragment is the MFMA "A" operand and the A fragment
// the "B" operand, so each lane's 4 accumulators are 4 consecutive columns of
// one output row (8-byte bf16 stores).
//
// Tile order: workgroups are dealt round-robin to the 8 XCDs, so consecutive
// tile ids are remapped onto one XCD (sharing its L2), then walked in groups of
// kGroupM tile-rows so co-resident tiles reuse the same A rows and B columns.
//
// Epilogues: plain store; per-row scale (the RMSNorm 1/rms, whose statistics
// and gamma-scaled bf16 copy of x come from a streaming pre-pass over x, see
// rms_prep_kernel); SwiGLU (two B operands, silu(gate) * up); fp32 store.
#include <type_traits>

#include "common.h"

namespace kda {
namespace gemm {

constexpr int kWavesM = 2, kWavesN = 4;     // wave grid of a workgroup
constexpr int kWaves = kWavesM * kWavesN;     // 8 waves: 2 per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kBK = 32;        // k per LDS slot
constexpr int kStages = 4;     // LDS slots (4 x 32 KiB for a 256x256 tile)
constexpr int kGroupM = 8;
constexpr int kXcds = 8;

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
#define KDA_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// 16 zero bytes: the DMA source for k-chunks past K (so they contribute 0).
__device__ __align__(16) uint32_t g_zero_chunk[4] = {0u, 0u, 0u, 0u};

enum class Epi { kStore, kRowScale, kSwiGLU, kStoreF32 };

struct Params {
  const uint16_t* a;   // A_KMAJ: a[m*lda + k]; else a[k*lda + m]
  const uint16_t* b;   // b[k*ldb + n]            (gate weights for SwiGLU)
  const uint16_t* b2;  // b2[k*ldb + n]           (up weights, SwiGLU only)
  void* c;             // c[m*ldc + n]  (bf16, or fp32 for kStoreF32)
  const float* row_scale;  // [M] (kRowScale)
  int64_t lda, ldb, ldc;
  int64_t batch_a, batch_b, batch_c;   // per-batch strides (elements), batch = blockIdx.y
  int m, n, k;
};

// Position of 16-byte chunk c of row r in a K-contiguous tile of BK-element
// rows: 64-byte rows (BK=32, 4 chunks) or 128-byte rows (BK=64, 8 chunks).
// Both are measured conflict-free for the fragment read (16 consecutive rows,
// one chunk) at the LDS's 256 B/clk ds_read_b128 rate.
template <int BK>
__device__ __forceinline__ int kswz(int r) { return BK == 32 ? ((r >> 1) & 3) : (r & 7); }
// Position of 32-byte segment s of k-row k in an MN-contiguous tile (measured
// conflict-free for the ds_read_b64_tr_b16 fragment read).
__device__ __forceinline__ int mswz(int k) { return (k & 3) | (((k >> 3) & 1) << 2); }

// Maps the linear workgroup id to (tile_m, tile_n): XCD-contiguous, grouped by rows.
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

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{lo, hi}), bf16x2));
}

// One 16-byte-per-lane DMA from global memory into LDS: lane i's 16 bytes at
// `sbase + voff` land at LDS byte `lds + 16*i`.  Issued as inline asm so the
// compiler does not treat it as an LDS store (it would otherwise wait for it
// with vmcnt(0) before every later LDS read, which serialises the prefetch);
// completion is awaited explicitly (s_waitcnt vmcnt) before the barrier that
// publishes the stage.  The leading s_nop covers the M0-write hazard.
__device__ __forceinline__ void dma16(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds)
               : "memory");
}
// Same with a per-lane 64-bit address (used for the K tail, where lanes past K
// read a zero chunk).
__device__ __forceinline__ void dma16_ptr(const void* src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)KDA_LDS_PTR(p);
}

// Reads the MFMA fragment (column `col0 + lane%16`, k = kbase + 8*(lane/16) .. +7) of an
// MN-contiguous [BK][COLS] tile; col0 is a multiple of 16.
template <int COLS>
__device__ __forceinline__ bf16x8 read_mn_frag(const uint8_t* tile, int col0, int kbase, int lane) {
  const int g = lane >> 4, jj = lane & 15;
  const int s = col0 >> 4;
  const int k0 = kbase + 8 * g + (jj >> 2);
  const int k1 = k0 + 4;
  const uint8_t* p0 = tile + k0 * (2 * COLS) + ((s ^ mswz(k0)) << 5) + 8 * (jj & 3);
  const uint8_t* p1 = tile + k1 * (2 * COLS) + ((s ^ mswz(k1)) << 5) + 8 * (jj & 3);
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)KDA_LDS_PTR(p0));
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)KDA_LDS_PTR(p1));
  typedef short v8i16 __attribute__((ext_vector_type(8)));
  const v8i16 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

// Reads the MFMA fragment (row `row`, k = kbase + 8*(lane/16) .. +7) of a
// K-contiguous [ROWS][BK] tile (128-byte rows).
template <int BK>
__device__ __forceinline__ bf16x8 read_k_frag(const uint8_t* tile, int row, int kbase, int lane) {
  const int c = (kbase >> 3) + (lane >> 4);
  return *reinterpret_cast<const bf16x8*>(tile + row * (BK * 2) + ((c ^ kswz<BK>(row)) << 4));
}

// Pipeline: STAGES k-tiles of BK=32 in an LDS ring.  Each wave runs a stream of
// MFMA groups (one A fragment x all its B fragments) in which the fragments of
// the next group are always in flight.  Once per k-tile, in the middle of the
// tile's groups, the wave waits for the DMA of the next k-tile (vmcnt), passes
// the workgroup barrier (which also proves every wave is done with the stage
// consumed two tiles ago) and issues the DMA STAGES-1 tiles ahead into that
// freed stage; the rest of the tile's groups then prefetch the next tile's
// fragments, so tile boundaries expose neither LDS nor DMA latency.
template <int BM, int BN, int NB, bool A_KMAJ, Epi EPI, bool KTAIL, int BK, int STAGES>
__global__ __launch_bounds__(kThreads, 1) void gemm_bf16_kernel(Params p) {
  static_assert(NB == 1 || NB == 2, "one or two B operands");
  static_assert(BM % 128 == 0 && BN % 128 == 0, "tile");
  static_assert(STAGES >= 2, "ring depth");
  constexpr int WM = BM / kWavesM, WN = BN / kWavesN;   // wave tile (per B operand)
  constexpr int TM = WM / 16, TN = WN / 16;   // 16x16 MFMA tiles per wave
  constexpr int NBF = NB * TN;                // B fragments per k-tile per wave
  constexpr int A_BYTES = BM * BK * 2;
  constexpr int B_BYTES = BN * BK * 2;        // per B operand
  constexpr int STAGE = A_BYTES + NB * B_BYTES;
  constexpr int A_INST = A_BYTES / 1024 / kWaves;  // DMA instructions per wave per stage
  constexpr int B_INST = B_BYTES / 1024 / kWaves;  // ... per B operand
  static_assert(A_INST >= 1 && B_INST >= 1, "DMA split");
  constexpr int TILE_INST = A_INST + NB * B_INST;
  constexpr int A_RPI = A_KMAJ ? 1024 / (2 * BK) : 1024 / (2 * BM);  // tile rows per DMA instruction
  constexpr int B_RPI = 1024 / (2 * BN);
  constexpr int A_LPR = 64 / A_RPI;           // lanes per tile row
  constexpr int B_LPR = 64 / B_RPI;
  static_assert(kWaves == 8, "ping-pong needs 8 waves");

  extern __shared__ __align__(1024) uint8_t smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / kWavesN, wn = wave % kWavesN;

  const int tiles_m = (p.m + BM - 1) / BM, tiles_n = (p.n + BN - 1) / BN;
  int tm, tn;
  tile_coords(tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int M = p.m, N = p.n, K = p.k;
  const int nk = (K + BK - 1) / BK;
  const int64_t bz = blockIdx.y;

  // ---- DMA sources.  Lane offsets are 32-bit byte offsets from the operand's
  // (per-batch) base, which advances by a scalar amount per k-tile.  Rows/columns
  // past M/N are clamped to the last valid one (their outputs are never stored).
  const uint8_t* A = reinterpret_cast<const uint8_t*>(p.a + bz * p.batch_a);
  const uint8_t* Bop[NB];
  Bop[0] = reinterpret_cast<const uint8_t*>(p.b + bz * p.batch_b);
  if constexpr (NB == 2) Bop[NB - 1] = reinterpret_cast<const uint8_t*>(p.b2 + bz * p.batch_b);
  uint32_t a_off[A_INST];
  int a_k[A_INST];   // k (within the k-tile) of the lane's data, for the K tail
#pragma unroll
  for (int j = 0; j < A_INST; ++j) {
    const int q = j * kWaves + wave;
    const int r = q * A_RPI + lane / A_LPR;
    const int t = lane % A_LPR;
    if constexpr (A_KMAJ) {
      const int c = t ^ kswz<BK>(r);
      const int gm = min(m0 + r, M - 1);
      a_off[j] = (uint32_t)(((int64_t)gm * p.lda + 8 * c) * 2);
      a_k[j] = 8 * c;
    } else {
      const int s = (t >> 1) ^ mswz(r);
      const int gm = min(m0 + s * 16 + (t & 1) * 8, M - 8);
      a_off[j] = (uint32_t)(((int64_t)r * p.lda + gm) * 2);
      a_k[j] = r;
    }
  }
  uint32_t b_off[B_INST];
  int b_k[B_INST];
#pragma unroll
  for (int j = 0; j < B_INST; ++j) {
    const int q = j * kWaves + wave;
    const int r = q * B_RPI + lane / B_LPR;
    const int t = lane % B_LPR;
    const int s = (t >> 1) ^ mswz(r);
    const int gn = min(n0 + s * 16 + (t & 1) * 8, N - 8);
    b_off[j] = (uint32_t)(((int64_t)r * p.ldb + gn) * 2);
    b_k[j] = r;
  }
  const int64_t a_step = (A_KMAJ ? BK : BK * p.lda) * 2;   // bytes per k-tile
  const int64_t b_step = BK * p.ldb * 2;
  const uint32_t lds0 = lds_addr(smem);

  // DMA of k-tile `kt` into ring slot `slot % STAGES`.
  auto issue = [&](int kt, int slot) {
    const uint32_t base = lds0 + (slot % STAGES) * STAGE;
    const uint8_t* sa = A + kt * a_step;
    const bool tail = KTAIL && (kt + 1) * BK > K;
    if (!tail) {
#pragma unroll
      for (int j = 0; j < A_INST; ++j) dma16(sa, a_off[j], base + (j * kWaves + wave) * 1024);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint8_t* sb = Bop[b] + kt * b_step;
#pragma unroll
        for (int j = 0; j < B_INST; ++j)
          dma16(sb, b_off[j], base + A_BYTES + b * B_BYTES + (j * kWaves + wave) * 1024);
      }
    } else {
      const int kbase = kt * BK;
#pragma unroll
      for (int j = 0; j < A_INST; ++j) {
        const void* src = (kbase + a_k[j] < K) ? (const void*)(sa + a_off[j]) : (const void*)g_zero_chunk;
        dma16_ptr(src, base + (j * kWaves + wave) * 1024);
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint8_t* sb = Bop[b] + kt * b_step;
#pragma unroll
        for (int j = 0; j < B_INST; ++j) {
          const void* src = (kbase + b_k[j] < K) ? (const void*)(sb + b_off[j]) : (const void*)g_zero_chunk;
          dma16_ptr(src, base + A_BYTES + b * B_BYTES + (j * kWaves + wave) * 1024);
        }
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

  auto stage_ptr = [&](int kt) -> const uint8_t* { return smem + (kt % STAGES) * STAGE; };
  auto read_a = [&](int kt, int kh, int i) -> bf16x8 {
    const uint8_t* at = stage_ptr(kt);
    if constexpr (A_KMAJ)
      return read_k_frag<BK>(at, wm * WM + i * 16 + (lane & 15), kh * 32, lane);
    else
      return read_mn_frag<BM>(at, wm * WM + i * 16, kh * 32, lane);
  };
  auto read_b = [&](int kt, int kh, int bj) -> bf16x8 {
    const int b = bj / TN, j = bj % TN;
    return read_mn_frag<BN>(stage_ptr(kt) + A_BYTES + b * B_BYTES, wn * WN + j * 16, kh * 32, lane);
  };

  // ---- ping-pong schedule.  Waves 0-3 (group 0) and 4-7 (group 1) hold one
  // wave per SIMD each and run the same program one phase apart: while one
  // group issues the back-to-back MFMAs of a k-tile (raised priority), the
  // other reads the fragments of its next k-tile from LDS and issues its share
  // of the DMA two k-tiles ahead.  One workgroup barrier per phase:
  //   phase 2t:   group 0 loads tile t     group 1 computes tile t-1
  //   phase 2t+1: group 0 computes tile t  group 1 loads tile t
  // Tile t must be in LDS before phase 2t.  Each wave issues its share while
  // loading tile t-2 (group 0: phase 2t-4, group 1: 2t-3) and awaits it at the
  // end of phase 2t-1, with only its share of tile t+1 allowed in flight.  The
  // DMA of tile t+2 overwrites the slot of tile t+2-STAGES, whose last reader
  // (group 1) finished in phase 2t+5-2*STAGES < 2t.  Tile indices past the last
  // k-tile are clamped: those DMAs re-read valid memory into unused slots.
  // LEAD = how many k-tiles ahead the DMA runs: 2 with >= 3 slots (each wave
  // issues while loading; group 1's share of tile t is awaited at the end of
  // phase 2t-1 with tile t+1 in flight), 1 with 2 slots (every wave issues its
  // share of tile t+1 at the start of phase 2t -- group 0 while loading, group 1
  // while computing -- into the slot of tile t-1, whose last reader finished in
  // phase 2t-1, and awaits it at the end of phase 2t+1).
  constexpr int LEAD = STAGES >= 3 ? 2 : 1;
  constexpr int KH = BK / 32;                   // 32-wide k halves per tile
  const int grp = wave >> 2;
  issue(0, 0);
  if constexpr (LEAD == 2) {
    issue(min(1, nk - 1), 1);
    wait_vmcnt<TILE_INST>();
  } else {
    wait_vmcnt<0>();
  }
  __builtin_amdgcn_s_barrier();
  if (grp == 1) {
    if constexpr (LEAD == 1) issue(min(1, nk - 1), 1);
    __builtin_amdgcn_s_barrier();   // group 1 starts one phase later
  }
  asm volatile("" ::: "memory");

  bf16x8 af[KH][TM], bfr[KH][NBF];
  for (int kt = 0; kt < nk; ++kt) {
    // -- load phase: fragments of tile kt
    if (LEAD == 2 || grp == 0) issue(min(kt + LEAD, nk - 1), kt + LEAD);
#pragma unroll
    for (int kh = 0; kh < KH; ++kh) {
#pragma unroll
      for (int i = 0; i < TM; ++i) af[kh][i] = read_a(kt, kh, i);
#pragma unroll
      for (int bj = 0; bj < NBF; ++bj) bfr[kh][bj] = read_b(kt, kh, bj);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (grp == 1) {
      if constexpr (LEAD == 2) wait_vmcnt<TILE_INST>();
      else wait_vmcnt<0>();
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // -- compute phase
    if (LEAD == 1 && grp == 1 && kt + 2 < nk + 1) issue(min(kt + 2, nk - 1), kt + 2);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kh = 0; kh < KH; ++kh)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[b][i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[kh][b * TN + j], af[kh][i],
                                                                   acc[b][i][j], 0, 0, 0);
    __builtin_amdgcn_s_setprio(0);
    if (grp == 0) {
      if constexpr (LEAD == 2) wait_vmcnt<TILE_INST>();
      else wait_vmcnt<0>();
    }
    if (!(grp == 1 && kt + 1 == nk)) __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  // No DMA may still be writing this workgroup's LDS when it exits.
  wait_vmcnt<0>();

  // ---- epilogue: lane holds C[row][col .. col+3] for each 16x16 tile
  const int col_in = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int gm = m0 + wm * WM + i * 16 + (lane & 15);
    if (gm >= M) continue;
    float scale = 1.0f;
    if constexpr (EPI == Epi::kRowScale) scale = p.row_scale[gm];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int gn = n0 + wn * WN + j * 16 + col_in;
      if (gn >= N) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (EPI == Epi::kSwiGLU)
          v[r] = silu_f(acc[0][i][j][r]) * acc[NB - 1][i][j][r];
        else
          v[r] = acc[0][i][j][r] * scale;
      }
      const int64_t off = bz * p.batch_c + (int64_t)gm * p.ldc + gn;
      if constexpr (EPI == Epi::kStoreF32) {
        *reinterpret_cast<floatx4*>(reinterpret_cast<float*>(p.c) + off) =
            floatx4{v[0], v[1], v[2], v[3]};
      } else {
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.c) + off) =
            u32x2{pack2(v[0], v[1]), pack2(v[2], v[3])};
      }
    }
  }
}

// ---------------------------------------------------------------- RMSNorm pre-pass
// One workgroup per row: inv_rms[m] = 1/sqrt(mean_k x[m,k]^2 + eps) (fp32 sum of
// squares of the bf16 values) and xg[m,k] = bf16(x[m,k] * gamma[k]).  x is read
// once; xg stays in the 256 MB Infinity Cache for the GEMM that follows.
constexpr int kPrepThreads = 256;
constexpr int kPrepVec = 4;   // 16-byte chunks per thread held in registers (K <= 8192)

__global__ __launch_bounds__(kPrepThreads) void rms_prep_kernel(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ gamma,
                                                                uint16_t* __restrict__ xg,
                                                                float* __restrict__ inv_rms, int k,
                                                                float eps) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nchunk = k / 8;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + (int64_t)row * k);
  u32x4 v[kPrepVec];
  float ssq = 0.f;
#pragma unroll
  for (int u = 0; u < kPrepVec; ++u) {
    const int c = tid + u * kPrepThreads;
    v[u] = (c < nchunk) ? __builtin_nontemporal_load(xr + c) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float lo = __builtin_bit_cast(float, v[u][w] << 16);
      const float hi = __builtin_bit_cast(float, v[u][w] & 0xffff0000u);
      ssq = fmaf(lo, lo, ssq);
      ssq = fmaf(hi, hi, ssq);
    }
  }
  // tail chunks beyond the register-held part (K > 8192)
  for (int c = tid + kPrepVec * kPrepThreads; c < nchunk; c += kPrepThreads) {
    const u32x4 t = xr[c];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float lo = __builtin_bit_cast(float, t[w] << 16);
      const float hi = __builtin_bit_cast(float, t[w] & 0xffff0000u);
      ssq = fmaf(lo, lo, ssq);
      ssq = fmaf(hi, hi, ssq);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ssq += __shfl_xor(ssq, off);
  __shared__ float part[kPrepThreads / 64];
  __shared__ float s_inv;
  if ((tid & 63) == 0) part[tid >> 6] = ssq;
  __syncthreads();
  if (tid == 0) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kPrepThreads / 64; ++w) s += part[w];
    const float inv = 1.0f / sqrtf(s / (float)k + eps);
    s_inv = inv;
    inv_rms[row] = inv;
  }
  __syncthreads();
  (void)s_inv;
  const u32x4* gr = reinterpret_cast<const u32x4*>(gamma);
  u32x4* outr = reinterpret_cast<u32x4*>(xg + (int64_t)row * k);
  auto scale_store = [&](const u32x4& t, int c) {
    const u32x4 g = gr[c];
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float x0 = __builtin_bit_cast(float, t[w] << 16);
      const float x1 = __builtin_bit_cast(float, t[w] & 0xffff0000u);
      const float g0 = __builtin_bit_cast(float, g[w] << 16);
      const float g1 = __builtin_bit_cast(float, g[w] & 0xffff0000u);
      o[w] = pack2(x0 * g0, x1 * g1);
    }
    outr[c] = o;
  };
#pragma unroll
  for (int u = 0; u < kPrepVec; ++u) {
    const int c = tid + u * kPrepThreads;
    if (c < nchunk) scale_store(v[u], c);
  }
  for (int c = tid + kPrepVec * kPrepThreads; c < nchunk; c += kPrepThreads) scale_store(xr[c], c);
}

// ---------------------------------------------------------------- launch helpers

template <int BM, int BN, int NB, bool A_KMAJ, Epi EPI, int BK = kBK, int S = kStages>
int launch(const Params& a, int batch, hipStream_t st, const char* what) {
  const int tiles = ((a.m + BM - 1) / BM) * ((a.n + BN - 1) / BN);
  const size_t lds = (size_t)S * (BM + NB * BN) * BK * sizeof(uint16_t);
  static const bool attr_ok = [&] {
    const hipError_t e1 = hipFuncSetAttribute(
        reinterpret_cast<const void*>(gemm_bf16_kernel<BM, BN, NB, A_KMAJ, EPI, false, BK, S>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    const hipError_t e2 = hipFuncSetAttribute(
        reinterpret_cast<const void*>(gemm_bf16_kernel<BM, BN, NB, A_KMAJ, EPI, true, BK, S>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    return e1 == hipSuccess && e2 == hipSuccess;
  }();
  if (!attr_ok) return set_error(KDA_ERR_HIP, "%s: cannot reserve %zu bytes of LDS", what, lds);
  const dim3 grid(tiles, batch);
  if (a.k % BK == 0)
    hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, NB, A_KMAJ, EPI, false, BK, S>), grid, dim3(kThreads),
                       lds, st, a);
  else
    hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, NB, A_KMAJ, EPI, true, BK, S>), grid, dim3(kThreads),
                       lds, st, a);
  return check_launch(what);
}

// Chooses the N tile: 256 when that still gives at least one wave of tiles over
// the device, else 128 (more, smaller tiles for skinny problems).
template <bool A_KMAJ, Epi EPI>
int launch_auto(const Params& a, int batch, hipStream_t st, const char* what) {
  const int64_t tiles256 = (int64_t)((a.m + 255) / 256) * ((a.n + 255) / 256) * batch;
  if (tiles256 >= device_cu_count()) return launch<256, 256, 1, A_KMAJ, EPI>(a, batch, st, what);
  return launch<256, 128, 1, A_KMAJ, EPI>(a, batch, st, what);
}

int validate(const char* what, const void* a, const void* b, const void* c, int64_t m,
             int64_t n, int64_t k) {
  if (m < 0 || n < 0 || k < 0)
    return set_error(KDA_ERR_INVALID_ARG, "%s: negative size (M=%lld N=%lld K=%lld)", what,
                     (long long)m, (long long)n, (long long)k);
  if (m > (1 << 30) || n > (1 << 30) || k > (1 << 30))
    return set_error(KDA_ERR_UNSUPPORTED, "%s: size too large", what);
  // 32-bit byte offsets address each operand (per batch) from a scalar base.
  if (m * k * 2 > (int64_t)0xffffffff || k * n * 2 > (int64_t)0xffffffff)
    return set_error(KDA_ERR_UNSUPPORTED, "%s: an operand exceeds 4 GiB", what);
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
  if (k == 0) return hipMemsetAsync(c, 0, (size_t)m * n * 2, as_stream(stream)) == hipSuccess
                         ? KDA_OK : set_error(KDA_ERR_HIP, "matmul_bf16: memset failed");
  Params p{};
  p.a = a; p.b = b; p.c = c;
  p.lda = k; p.ldb = n; p.ldc = n;
  p.m = (int)m; p.n = (int)n; p.k = (int)k;
  return launch_auto<true, Epi::kStore>(p, 1, as_stream(stream), "matmul_bf16");
}

extern "C" int64_t kda_rmsnorm_matmul_bf16_workspace_size(int64_t m, int64_t k) {
  if (m < 0 || k < 0) return -1;
  return ((m * k * 2 + 255) / 256) * 256 + m * 4;
}

extern "C" int kda_rmsnorm_matmul_bf16(const kda_bf16* x, const kda_bf16* gamma, const kda_bf16* w,
                                       kda_bf16* y, int64_t m, int64_t k, int64_t n, float eps,
                                       void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  if (int rc = validate("rmsnorm_matmul_bf16", x, w, y, m, n, k)) return rc;
  if (k == 0) return set_error(KDA_ERR_INVALID_ARG, "rmsnorm_matmul_bf16: K must be > 0");
  if (!gamma || !aligned16(gamma))
    return set_error(KDA_ERR_INVALID_ARG, "rmsnorm_matmul_bf16: gamma null or not 16-byte aligned");
  if (!(eps >= 0.f)) return set_error(KDA_ERR_INVALID_ARG, "rmsnorm_matmul_bf16: eps must be >= 0");
  if (m == 0 || n == 0) return KDA_OK;
  const int64_t need = kda_rmsnorm_matmul_bf16_workspace_size(m, k);
  if (!workspace || !aligned16(workspace) || workspace_bytes < need)
    return set_error(KDA_ERR_INVALID_ARG,
                     "rmsnorm_matmul_bf16: workspace must be 16-byte aligned and >= %lld bytes",
                     (long long)need);
  hipStream_t st = as_stream(stream);
  uint16_t* xg = reinterpret_cast<uint16_t*>(workspace);
  float* inv = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(workspace) +
                                        ((m * k * 2 + 255) / 256) * 256);
  hipLaunchKernelGGL(rms_prep_kernel, dim3((unsigned)m), dim3(kPrepThreads), 0, st, x, gamma, xg,
                     inv, (int)k, eps);
  if (int rc = check_launch("rmsnorm_matmul_bf16(prep)")) return rc;
  Params p{};
  p.a = xg; p.b = w; p.c = y; p.row_scale = inv;
  p.lda = k; p.ldb = n; p.ldc = n;
  p.m = (int)m; p.n = (int)n; p.k = (int)k;
  return launch_auto<true, Epi::kRowScale>(p, 1, st, "rmsnorm_matmul_bf16");
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
  if (f == 0) return hipMemsetAsync(y, 0, (size_t)m * k * 2, as_stream(stream)) == hipSuccess
                         ? KDA_OK : set_error(KDA_ERR_HIP, "swiglu_bf16: memset failed");
  hipStream_t st = as_stream(stream);
  Params up{};
  up.a = x; up.b = w_gate; up.b2 = w_up; up.c = h;
  up.lda = k; up.ldb = f; up.ldc = f;
  up.m = (int)m; up.n = (int)f; up.k = (int)k;
  if (int rc = launch<256, 128, 2, true, Epi::kSwiGLU>(up, 1, st, "swiglu_bf16(up/gate)")) return rc;
  Params down{};
  down.a = h; down.b = w_down; down.c = y;
  down.lda = f; down.ldb = k; down.ldc = k;
  down.m = (int)m; down.n = (int)k; down.k = (int)f;
  return launch_auto<true, Epi::kStore>(down, 1, st, "swiglu_bf16(down)");
}
