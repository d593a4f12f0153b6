// GEMM family on gfx950 bf16 MFMA (v_mfma_f32_16x16x32_bf16), fp32 accumulation.
//
//   C[M,N] = sum over K-segments s of  A_s[M,K_s] @ B_s[K_s,N]
//
// One kernel template serves every GEMM-shaped operator of the library:
//   * bf16 operands (graded RMSNorm->matmul and SwiGLU configurations, bf16 matmul);
//   * fp32 operands through a three-product bf16 split: x = hi + lo with hi =
//     bf16(x), lo = bf16(x - hi), and A@B ~= Ah@Bh + Ah@Bl + Al@Bh, expressed as
//     three K-segments (Ah,Bh), (Ah,Bl), (Al,Bh) over bf16 planes written by a
//     streaming pre-pass (split_f32_kernel).  The dropped Al@Bl term is ~2^-16
//     relative per product; fp32 accumulation throughout;
//   * LoRA x@w + (x@a)@b as six segments (the split x@w plus the split t@b);
//   * batched products (blockIdx.y = batch, per-batch strides).
//
// Data path (one BM x BN output tile per workgroup, BM = 256, or 128 for the
// SwiGLU tail columns; 8 waves in a 2 x 4 grid, each wave owning a BM/2 x BN/4
// fp32 accumulator block per B operand):
//
//   HBM --global_load_lds_dwordx4--> LDS (4-slot ring of BK=32 k-tiles) --ds_read--> MFMA
//
//   * Operands go straight from global memory into LDS, 16 bytes per lane with
//     no register staging: each wave instruction fills 1 KiB of LDS lane-
//     linearly, so the LDS swizzle is applied on the global side by choosing
//     which 16-byte chunk each lane fetches.  The DMA is inline asm so the
//     compiler does not serialise later LDS reads behind it; completion is
//     awaited explicitly (s_waitcnt vmcnt) before the barrier that publishes a slot.
//   * K-contiguous operands (A row-major) are stored [rows][32 k] (64-byte
//     rows), chunk c of row r at c ^ ((r >> 1) & 3): one ds_read_b128 gives an
//     MFMA fragment (one row, 8 consecutive k).
//   * MN-contiguous operands (B row-major [K][N], or A stored [K][M]) keep their
//     HBM orientation, [32 k][cols], 32-byte segment s of k-row k at s ^ mswz(k).
//     A fragment (one column, 8 consecutive k) is read with two
//     ds_read_b64_tr_b16: within a 16-lane group, lane 4r+q names 4 elements of
//     k-row r and lane j receives column j of that 4 x 16 block.
//   * Both layouts were measured bank-conflict free (256 B/clk) on this LDS.
//   * Ping-pong schedule: waves 0-3 and 4-7 (one wave per SIMD each) run one
//     phase apart, so that while one group issues the back-to-back MFMAs of a
//     k-tile the other reads its next fragments and issues DMA two tiles ahead.
//
// MFMA operand order: the B fragment is the MFMA "A" operand and the A fragment
// the "B" operand, so each lane's 4 accumulators are 4 consecutive columns of
// one output row (8-byte bf16 or 16-byte fp32 stores).
//
// Tile order: workgroups are dealt round-robin to the 8 XCDs, so consecutive
// tile ids are remapped onto one XCD (sharing its L2), then walked in groups of
// group_m tile-rows (chosen per launch) so co-resident tiles reuse the same A
// rows and B columns.
#include <math.h>

#include <mutex>
#include <type_traits>

#include "common.h"
#include "lds_dma.h"

namespace kda {
namespace gemm {

constexpr int kWavesM = 2, kWavesN = 4;     // wave grid of a workgroup
constexpr int kWaves = kWavesM * kWavesN;     // 8 waves: 2 per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kBK = 32;        // k per LDS slot
constexpr int kStages = 4;     // LDS slots (4 x 32 KiB for a 256x256 tile)
constexpr int kXcds = 8;
constexpr int kMaxSeg = 6;

typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// 16 zero bytes: the DMA source for k-chunks past K (so they contribute 0).
__device__ __align__(16) uint32_t g_zero_chunk[4] = {0u, 0u, 0u, 0u};

enum class Epi {
  kStore,          // bf16 C
  kRowScale,       // bf16 C = acc * row_scale[m]
  kSwiGLU,         // bf16 H = silu(acc_gate) * acc_up
  kStoreF32,       // fp32 C
  kSwiGLUSplit,    // h = silu(acc_gate) * acc_up in fp32, stored as its bf16 planes: hi = bf16(h) in C, lo = bf16(h - hi) in C2
  kAddZSsqF32,     // fp32 C = acc + z; part[m][n/64] = sum over the 64 columns of C^2
  kAddZSsqBf16,    // bf16 C = acc + z (bf16 z); part as above, from the fp32 sums
};

// One K-segment: A_s (M x k), B_s (k x N) (and B2_s for two-B kernels).
struct Seg {
  const uint16_t* a;   // A_KMAJ: a[m*lda + k]; else a[k*lda + m]
  const uint16_t* b;   // b[k*ldb + n]
  const uint16_t* b2;  // b2[k*ldb + n]   (second B operand, SwiGLU)
  int64_t lda, ldb;    // < 2^31
  int k;               // k extent; a multiple of kBK unless it is the only segment
};

struct Params {
  Seg seg[kMaxSeg];
  int nseg;
  void* c;                 // c[m*ldc + n]  (bf16, or fp32 for the *F32 epilogues)
  void* c2;                // c2[m*ldc + n] bf16: the low plane (kSwiGLUSplit)
  const float* row_scale;  // [M]                      (kRowScale)
  const void* z;           // z[m*ldc + n], fp32 or bf16 as C   (kAddZSsq*)
  float* part;             // part[m*(N/WN) + n/WN]             (kAddZSsq*)
  int64_t ldc;
  int64_t batch_a, batch_b, batch_c;   // per-batch strides (elements), batch = blockIdx.y
  int m, n, k;             // k = sum of segment extents
  int group_m;             // tile rows per group of the tile order (set at launch)
  int* zero;               // zero_n ints that workgroup (0, 0) clears before its tile: the
  int zero_n;              // flags of a launch that follows on the same stream
};

// Position of 16-byte chunk c of row r in a K-contiguous tile of BK-element
// rows: 64-byte rows (BK=32, 4 chunks) or 128-byte rows (BK=64, 8 chunks).
// Both are measured conflict-free for the fragment read (16 consecutive rows,
// one chunk) at the LDS's 256 B/clk ds_read_b128 rate.
template <int BK>
__device__ __forceinline__ int kswz(int r) { return BK == 32 ? ((r >> 1) & 3) : (r & 7); }

// Maps the linear workgroup id to (tile_m, tile_n): XCD-contiguous, grouped by rows.
__device__ __forceinline__ void tile_coords(int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int pid = blockIdx.x;
  const int full = (total / kXcds) * kXcds;
  if (pid < full) pid = (pid % kXcds) * (full / kXcds) + pid / kXcds;
  const int per_group = group_m * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * group_m;
  const int gsize = min(tiles_m - first_m, group_m);
  const int local = pid - group * per_group;
  tm = first_m + local % gsize;
  tn = local / gsize;
}

__device__ __forceinline__ float silu_f(float x) { return __fdividef(x, 1.0f + __expf(-x)); }

__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2{lo, hi}), bf16x2));
}

// Reads the MFMA fragment (row `row`, k = kbase + 8*(lane/16) .. +7) of a
// K-contiguous [ROWS][BK] tile.
template <int BK>
__device__ __forceinline__ bf16x8 read_k_frag(const uint8_t* tile, int row, int kbase, int lane) {
  const int c = (kbase >> 3) + (lane >> 4);
  return *reinterpret_cast<const bf16x8*>(tile + row * (BK * 2) + ((c ^ kswz<BK>(row)) << 4));
}

// Wave-tile geometry of a BM x BN (x NB B operands) workgroup tile.
template <int BM, int BN>
struct WaveTile {
  static constexpr int WM = BM / kWavesM, WN = BN / kWavesN;   // wave tile (per B operand)
  static constexpr int TM = WM / 16, TN = WN / 16;             // 16x16 MFMA tiles per wave
};

// A dependency of a k-range on other workgroups: before the DMA of k-tile `kt`
// (and every later one) is issued, *flag must reach `target` (a counter that
// producer workgroups raise with release semantics after their stores).  The wait
// is bounded (see wait_flag).  kt < 0: no dependency.
struct KDep {
  int kt = -1;
  const int* flag = nullptr;
  int target = 0;
};

// Spins (lane 0, relaxed agent-scope loads) until *flag >= target, then acquires
// at agent scope so the producers' stores are visible to the loads that follow.
// Producers are workgroups dispatched before the waiter, so the wait ends; the
// spin is still bounded (2^21 polls of a memory round trip each, about a second)
// so that a broken schedule can never hang the device.
__device__ __forceinline__ void wait_flag(const int* flag, int target) {
  if ((threadIdx.x & 63) == 0) {
    for (int i = 0; i < (1 << 21); ++i) {
      if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) break;
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// Raises *flag by one once every store of the workgroup so far is visible at
// agent scope: each wave waits for its own stores to reach the L2, and after the
// barrier one release increment (which writes the L2 back) publishes them all.
__device__ __forceinline__ void publish(int* flag) {
  wait_vmcnt<0>();
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(flag, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// The K loop of one output tile (m0, n0) of batch bz: DMA ring, ping-pong MFMA
// schedule, fp32 accumulators left in acc.  With DEP, wave 0 waits on dep.flag
// before the barrier that precedes the first issue of k-tile dep.kt.
template <int BM, int BN, int NB, bool A_KMAJ, bool KTAIL, int BK, int STAGES, int NSEG, bool DEP = false>
__device__ __forceinline__ void gemm_mainloop(const Params& p, int m0, int n0, int64_t bz, uint8_t* smem,
                                              floatx4 (&acc)[NB][WaveTile<BM, BN>::TM][WaveTile<BM, BN>::TN],
                                              KDep dep = {}) {
  static_assert(NSEG >= 1 && NSEG <= kMaxSeg, "segments");
  static_assert(NB == 1 || NB == 2, "one or two B operands");
  static_assert(BM % 128 == 0 && BN % 128 == 0, "tile");
  static_assert(STAGES >= 2, "ring depth");
  static_assert(kWaves == 8, "ping-pong needs 8 waves");
  constexpr int WM = WaveTile<BM, BN>::WM, WN = WaveTile<BM, BN>::WN;
  constexpr int TM = WaveTile<BM, BN>::TM, TN = WaveTile<BM, BN>::TN;
  constexpr int NBF = NB * TN;                // B fragments per k-tile per wave
  constexpr int A_BYTES = BM * BK * 2;
  constexpr int B_BYTES = BN * BK * 2;        // per B operand
  constexpr int STAGE = A_BYTES + NB * B_BYTES;
  constexpr int A_INST = A_BYTES / 1024 / kWaves;  // DMA instructions per wave per slot
  constexpr int B_INST = B_BYTES / 1024 / kWaves;  // ... per B operand
  static_assert(A_INST >= 1 && B_INST >= 1, "DMA split");
  constexpr int TILE_INST = A_INST + NB * B_INST;
  constexpr int A_RPI = A_KMAJ ? 1024 / (2 * BK) : 1024 / (2 * BM);  // tile rows per DMA instruction
  constexpr int B_RPI = 1024 / (2 * BN);
  constexpr int A_LPR = 64 / A_RPI;           // lanes per tile row
  constexpr int B_LPR = 64 / B_RPI;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int M = p.m, N = p.n, K = p.k;
  const int nk = (K + BK - 1) / BK;

  // ---- DMA sources.  Each lane keeps the (row, column) it fetches; its byte
  // offset from the segment's per-batch base is formed per issue from the
  // segment's leading dimension.  Rows/columns past M/N are clamped to the last
  // valid one (their outputs are never stored).
  int a_row[A_INST], a_col[A_INST], a_k[A_INST];   // a_k: k within the tile (K tail)
#pragma unroll
  for (int j = 0; j < A_INST; ++j) {
    const int q = j * kWaves + wave;
    const int r = q * A_RPI + lane / A_LPR;
    const int t = lane % A_LPR;
    if constexpr (A_KMAJ) {
      const int c = t ^ kswz<BK>(r);
      a_row[j] = min(m0 + r, M - 1);   // m
      a_col[j] = 8 * c;                // k within the tile
      a_k[j] = 8 * c;
    } else {
      const int s = (t >> 1) ^ mswz(r);
      a_row[j] = r;                    // k within the tile
      a_col[j] = min(m0 + s * 16 + (t & 1) * 8, M - 8);   // m
      a_k[j] = r;
    }
  }
  int b_row[B_INST], b_col[B_INST];
#pragma unroll
  for (int j = 0; j < B_INST; ++j) {
    const int q = j * kWaves + wave;
    const int r = q * B_RPI + lane / B_LPR;
    const int t = lane % B_LPR;
    const int s = (t >> 1) ^ mswz(r);
    b_row[j] = r;
    b_col[j] = min(n0 + s * 16 + (t & 1) * 8, N - 8);
  }
  const uint32_t lds0 = lds_addr(smem);

  // Segment table, pinned in scalar registers (readfirstlane keeps the
  // per-k-tile selection below a chain of scalar selects instead of an
  // indexed load from a private copy of the kernel arguments).
  auto rfl64 = [](const void* q) -> uint64_t {
    const uint64_t v = reinterpret_cast<uint64_t>(q);
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
           (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  };
  uint64_t seg_a[NSEG], seg_b[NSEG], seg_b2[NSEG];
  uint32_t seg_lda[NSEG], seg_ldb[NSEG];
  int seg_end[NSEG];   // first k-tile after the segment
  {
    int end = 0;
#pragma unroll
    for (int i = 0; i < NSEG; ++i) {
      seg_a[i] = rfl64(p.seg[i].a);
      seg_b[i] = rfl64(p.seg[i].b);
      seg_b2[i] = NB == 2 ? rfl64(p.seg[i].b2) : 0;
      seg_lda[i] = __builtin_amdgcn_readfirstlane((uint32_t)p.seg[i].lda);
      seg_ldb[i] = __builtin_amdgcn_readfirstlane((uint32_t)p.seg[i].ldb);
      end += (p.seg[i].k + BK - 1) / BK;
      seg_end[i] = __builtin_amdgcn_readfirstlane(end);
    }
  }

  // DMA of k-tile `kt` into ring slot `slot % STAGES`.
  auto issue = [&](int kt, int slot) {
    const uint32_t base = lds0 + (slot % STAGES) * STAGE;
    uint64_t a64 = seg_a[0], b64 = seg_b[0], b264 = seg_b2[0];
    uint32_t lda32 = seg_lda[0], ldb32 = seg_ldb[0];
    int lt = kt;
#pragma unroll
    for (int i = 1; i < NSEG; ++i) {
      const bool in = kt >= seg_end[i - 1];
      a64 = in ? seg_a[i] : a64;
      b64 = in ? seg_b[i] : b64;
      b264 = in ? seg_b2[i] : b264;
      lda32 = in ? seg_lda[i] : lda32;
      ldb32 = in ? seg_ldb[i] : ldb32;
      lt = in ? kt - seg_end[i - 1] : lt;
    }
    const uint16_t* a = reinterpret_cast<const uint16_t*>(a64);
    const uint16_t* b = reinterpret_cast<const uint16_t*>(b64);
    const uint16_t* b2 = reinterpret_cast<const uint16_t*>(b264);
    const int64_t lda = lda32, ldb = ldb32;
    const uint8_t* sa = reinterpret_cast<const uint8_t*>(a + bz * p.batch_a) +
                        (A_KMAJ ? (int64_t)lt * BK * 2 : (int64_t)lt * BK * lda * 2);
    const uint8_t* sb[NB];
    sb[0] = reinterpret_cast<const uint8_t*>(b + bz * p.batch_b) + (int64_t)lt * BK * ldb * 2;
    if constexpr (NB == 2)
      sb[NB - 1] = reinterpret_cast<const uint8_t*>(b2 + bz * p.batch_b) + (int64_t)lt * BK * ldb * 2;
    const bool tail = KTAIL && (kt + 1) * BK > K;
    if (!tail) {
#pragma unroll
      for (int j = 0; j < A_INST; ++j)
        dma16(sa, ((uint32_t)a_row[j] * lda32 + (uint32_t)a_col[j]) * 2u,
              base + (j * kWaves + wave) * 1024);
#pragma unroll
      for (int bb = 0; bb < NB; ++bb)
#pragma unroll
        for (int j = 0; j < B_INST; ++j)
          dma16(sb[bb], ((uint32_t)b_row[j] * ldb32 + (uint32_t)b_col[j]) * 2u,
                base + A_BYTES + bb * B_BYTES + (j * kWaves + wave) * 1024);
    } else {
      const int kbase = kt * BK;
#pragma unroll
      for (int j = 0; j < A_INST; ++j) {
        const void* src = (kbase + a_k[j] < K)
                              ? (const void*)(sa + ((uint32_t)a_row[j] * lda32 + (uint32_t)a_col[j]) * 2u)
                              : (const void*)g_zero_chunk;
        dma16_ptr(src, base + (j * kWaves + wave) * 1024);
      }
#pragma unroll
      for (int bb = 0; bb < NB; ++bb)
#pragma unroll
        for (int j = 0; j < B_INST; ++j) {
          const void* src = (kbase + b_row[j] < K)
                                ? (const void*)(sb[bb] + ((uint32_t)b_row[j] * ldb32 + (uint32_t)b_col[j]) * 2u)
                                : (const void*)g_zero_chunk;
          dma16_ptr(src, base + A_BYTES + bb * B_BYTES + (j * kWaves + wave) * 1024);
        }
    }
  };

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
  // other reads the fragments of its next k-tile from LDS.  One workgroup
  // barrier per phase:
  //   phase 2t:   group 0 loads tile t     group 1 computes tile t-1
  //   phase 2t+1: group 0 computes tile t  group 1 loads tile t
  // Tile t must be in LDS before phase 2t.  LEAD = how many k-tiles ahead the
  // DMA runs:
  //   * 2 (>= 3 slots): each wave issues its share of tile t while loading tile
  //     t-2 (group 0: phase 2t-4, group 1: 2t-3) and awaits it at the end of
  //     phase 2t-1 with only its share of tile t+1 in flight; the DMA of tile
  //     t+2 overwrites the slot of tile t+2-STAGES, whose last reader (group 1)
  //     finished in phase 2t+5-2*STAGES < 2t.
  //   * 1 (2 slots): every wave issues its share of tile t+1 at the start of
  //     phase 2t (group 0 while loading, group 1 while computing) into the slot
  //     of tile t-1, last read in phase 2t-1, and awaits it at the end of 2t+1.
  // Tile indices past the last k-tile are clamped: those DMAs re-read valid
  // memory into slots that are no longer read.
  constexpr int LEAD = STAGES >= 3 ? 2 : 1;
  constexpr int KH = BK / 32;                   // 32-wide k halves per tile
  const int grp = wave >> 2;
  // Dependencies need the 2-tile DMA lead: k-tile kt is then issued by group 0 in
  // the load phase of iteration kt - 2 and by group 1 one phase later.  The
  // prologue issues tiles 0 and 1 and iteration 0 tile 2, so a dependency on one
  // of those is awaited (by every wave) before the prologue.
  static_assert(!DEP || LEAD == 2, "dependencies need a ring of 3 or more slots");
  if constexpr (DEP) {
    if (dep.kt >= 0 && dep.kt <= LEAD) wait_flag(dep.flag, dep.target);
  }
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
    if (LEAD == 1 && grp == 1 && kt + 2 <= nk) issue(min(kt + 2, nk - 1), kt + 2);
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
    // Group 0 issues k-tile kt + 1 + LEAD right after this barrier and group 1
    // one phase later: wave 0 holds both at the barrier until the dependency is met.
    if constexpr (DEP) {
      if (dep.kt > LEAD && kt == dep.kt - LEAD - 1 && wave == 0) wait_flag(dep.flag, dep.target);
    }
    if (!(grp == 1 && kt + 1 == nk)) __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
  // No DMA may still be writing this workgroup's LDS when it exits.
  wait_vmcnt<0>();
}

// Stores the accumulators of tile (m0, n0) of batch bz through epilogue EPI.
// B operand b's accumulators go to columns n0 + b * BOFF + (column within the
// operand's tile): BOFF = 0 for the epilogues that combine the two operands
// (SwiGLU), BN when two B operands are two halves of one 2*BN-wide tile.
template <int BM, int BN, int NB, Epi EPI, int BOFF = 0>
__device__ __forceinline__ void gemm_epilogue(const Params& p, int m0, int n0, int64_t bz,
                                              floatx4 (&acc)[NB][WaveTile<BM, BN>::TM][WaveTile<BM, BN>::TN]) {
  constexpr int WM = WaveTile<BM, BN>::WM, WN = WaveTile<BM, BN>::WN;
  constexpr int TM = WaveTile<BM, BN>::TM, TN = WaveTile<BM, BN>::TN;
  constexpr int NOUT = BOFF ? NB : 1;   // B operands stored separately
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int M = p.m, N = p.n;

  // ---- epilogue: lane holds C[row][col .. col+3] for each 16x16 tile
  const int col_in = (lane >> 4) * 4;
  // The residual epilogues read z.  Loads and stores complete through one
  // in-order counter, so a z load issued after a store of C would also wait for
  // that store: z is loaded ZI tile rows at a time (64 VGPRs) before any of
  // those rows is stored.
  constexpr bool kZ = EPI == Epi::kAddZSsqF32 || EPI == Epi::kAddZSsqBf16;
  static_assert(!(kZ && BOFF), "the residual epilogues store one B operand");
  static_assert(!(BOFF && (EPI == Epi::kSwiGLU || EPI == Epi::kSwiGLUSplit)), "SwiGLU combines the operands");
  constexpr int ZW = EPI == Epi::kAddZSsqF32 ? 4 : 2;   // 32-bit words of z per lane and tile
  constexpr int ZI = !kZ ? 1 : (64 / (TN * ZW) < TM ? 64 / (TN * ZW) : TM);
  static_assert(TM % ZI == 0, "z batches");
#pragma unroll
  for (int i0 = 0; i0 < TM; i0 += ZI) {
    uint32_t zb[ZI][TN][ZW];
    if constexpr (kZ) {
#pragma unroll
      for (int ii = 0; ii < ZI; ++ii) {
        const int gm = m0 + wm * WM + (i0 + ii) * 16 + (lane & 15);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int gn = n0 + wn * WN + j * 16 + col_in;
          const int64_t off = bz * p.batch_c + (int64_t)gm * p.ldc + gn;
          if (gm < M && gn < N) {
            if constexpr (ZW == 4) {
              const u32x4 t = *reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(p.z) + off);
#pragma unroll
              for (int w = 0; w < 4; ++w) zb[ii][j][w] = t[w];
            } else {
              const u32x2 t = *reinterpret_cast<const u32x2*>(reinterpret_cast<const uint16_t*>(p.z) + off);
              zb[ii][j][0] = t[0];
              zb[ii][j][1] = t[1];
            }
          } else {
#pragma unroll
            for (int w = 0; w < ZW; ++w) zb[ii][j][w] = 0u;
          }
        }
      }
    }
#pragma unroll
    for (int ii = 0; ii < ZI; ++ii) {
      const int i = i0 + ii;
      const int gm = m0 + wm * WM + i * 16 + (lane & 15);
      const bool row_ok = gm < M;
      float scale = 1.0f;
      if constexpr (EPI == Epi::kRowScale) scale = row_ok ? p.row_scale[gm] : 0.f;
      float ssq = 0.f;
#pragma unroll
      for (int jj = 0; jj < NOUT * TN; ++jj) {
        const int bo = jj / TN, j = jj % TN;
        const int gn = n0 + bo * BOFF + wn * WN + j * 16 + col_in;
        const bool ok = row_ok && gn < N;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (EPI == Epi::kSwiGLU || EPI == Epi::kSwiGLUSplit)
            v[r] = silu_f(acc[0][i][j][r]) * acc[NB - 1][i][j][r];
          else
            v[r] = acc[bo][i][j][r] * scale;
          if constexpr (EPI == Epi::kAddZSsqF32) v[r] += __builtin_bit_cast(float, zb[ii][j][r]);
          if constexpr (EPI == Epi::kAddZSsqBf16)
            v[r] += bf16_bits_to_f32(r & 1 ? zb[ii][j][r >> 1] >> 16 : zb[ii][j][r >> 1] & 0xffffu);
        }
        if (!ok) continue;
        if constexpr (kZ) {
#pragma unroll
          for (int r = 0; r < 4; ++r) ssq = fmaf(v[r], v[r], ssq);
        }
        const int64_t off = bz * p.batch_c + (int64_t)gm * p.ldc + gn;
        if constexpr (EPI == Epi::kStoreF32 || EPI == Epi::kAddZSsqF32) {
          *reinterpret_cast<floatx4*>(reinterpret_cast<float*>(p.c) + off) =
              floatx4{v[0], v[1], v[2], v[3]};
        } else if constexpr (EPI == Epi::kSwiGLUSplit) {
          uint32_t h0, h1, l0, l1;
          split_bf16x2(v[0], v[1], h0, l0);
          split_bf16x2(v[2], v[3], h1, l1);
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.c) + off) = u32x2{h0, h1};
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.c2) + off) = u32x2{l0, l1};
        } else {
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(p.c) + off) =
              u32x2{pack2(v[0], v[1]), pack2(v[2], v[3])};
        }
      }
      if constexpr (kZ) {
        // the 4 lanes l, l+16, l+32, l+48 hold the wave's WN columns of this row
        ssq += __shfl_xor(ssq, 16);
        ssq += __shfl_xor(ssq, 32);
        const int chunk = (n0 + wn * WN) / WN;
        if (row_ok && lane < 16 && n0 + wn * WN < N)
          p.part[(int64_t)gm * ((N + WN - 1) / WN) + chunk] = ssq;
      }
    }
  }
}

// One BM x BN output tile per workgroup (blockIdx.y = batch), in the
// XCD-aware tile order.
template <int BM, int BN, int NB, bool A_KMAJ, Epi EPI, bool KTAIL, int BK, int STAGES, int NSEG>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(Params p) {
  extern __shared__ __align__(1024) uint8_t smem[];
  if (p.zero_n && blockIdx.x == 0 && blockIdx.y == 0)
    for (int i = threadIdx.x; i < p.zero_n; i += kThreads) p.zero[i] = 0;
  const int tiles_m = (p.m + BM - 1) / BM, tiles_n = (p.n + BN - 1) / BN;
  int tm, tn;
  tile_coords(tiles_m, tiles_n, p.group_m, tm, tn);
  floatx4 acc[NB][WaveTile<BM, BN>::TM][WaveTile<BM, BN>::TN];
  gemm_mainloop<BM, BN, NB, A_KMAJ, KTAIL, BK, STAGES, NSEG>(p, tm * BM, tn * BN, blockIdx.y, smem, acc);
  gemm_epilogue<BM, BN, NB, EPI>(p, tm * BM, tn * BN, blockIdx.y, acc);
}

// ---------------------------------------------------------------- SwiGLU tail + down GEMM
// After the gate/up launch has produced h[:, :f_main] in full rounds, one launch
// of 2T equal-work workgroups finishes the operator (T = tail tiles = down tiles):
//   workgroup i < T:   the gate/up tail tile i (256 x 128, both B operands, full K,
//                      silu(g)*u into h[:, f_main:]), publishing it per row tile;
//                      then the first X columns of h times w_down for down tile i,
//                      whose fp32 accumulators it parks in the workspace.
//   workgroup T + i:   the remaining F - X columns for down tile i, then adds the
//                      parked accumulators and stores y (bf16).
// X balances the two: tail (2*256*128*K flop) + 256*256*X*2 = 256*256*(F - X)*2,
// less 10 k-tiles for the tail workgroups' fixed extra work.
// The second kind reads h's tail columns only in the last f_tail of its K range,
// after waiting for the row tile's tail tiles (long finished by then); it waits
// once more for the parked half.  Producers have the lower workgroup ids, which
// are dispatched first, so no wait can starve them of a CU.  Down tiles are
// 256 x 256, run as two B operands of 128 columns (w_down and w_down + 128).
struct SwigluFused {
  Params tail;       // x @ (w_gate, w_up)[:, f_main:] -> h[:, f_main:]
  Params down_a;     // h[:, :X] @ w_down[:X, :]
  Params down_b;     // h[:, X:] @ w_down[X:, :] -> y
  floatx4* park;     // [T][waves][2 x TM x TN][64]: down_a's accumulators
  int* row_done;     // [tiles_m]: tail tiles published per row tile
  int* park_flag;    // [T]
  int tail_cols;     // tail tiles per row tile (= down tiles per row tile)
  int dep_kt;        // first k-tile of down_b that reads h[:, f_main:]
};

template <int NB, int TM, int TN>
__device__ __forceinline__ void park_acc(floatx4* tile, const floatx4 (&acc)[NB][TM][TN]) {
  floatx4* w = tile + (size_t)(threadIdx.x >> 6) * (NB * TM * TN * 64) + (threadIdx.x & 63);
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) w[((b * TM + i) * TN + j) * 64] = acc[b][i][j];
}

// The parked values are added kParkBatch accumulators at a time: a batch's loads
// are all issued before its adds, so the wave waits kParkBatch times fewer memory
// round trips than with one load per add, and the compiler barrier after each
// batch keeps the next batch's loads from being hoisted ahead of its adds, which
// would hold the whole parked tile and the accumulators (2 x 128 VGPRs) at once
// and spill.
constexpr int kParkBatch = 16;
template <int NB, int TM, int TN>
__device__ __forceinline__ void add_parked(const floatx4* tile, floatx4 (&acc)[NB][TM][TN]) {
  constexpr int kN = NB * TM * TN;
  static_assert(kN % kParkBatch == 0, "parked tile is a whole number of batches");
  const floatx4* w = tile + (size_t)(threadIdx.x >> 6) * (kN * 64) + (threadIdx.x & 63);
  // parked value q is accumulator (b, i, j) with q = (b * TM + i) * TN + j, as park_acc writes them
#pragma unroll
  for (int q0 = 0; q0 < kN; q0 += kParkBatch) {
    floatx4 t[kParkBatch];
#pragma unroll
    for (int u = 0; u < kParkBatch; ++u) t[u] = w[(q0 + u) * 64];
#pragma unroll
    for (int u = 0; u < kParkBatch; ++u) {
      const int q = q0 + u, b = q / (TM * TN), i = (q / TN) % TM, j = q % TN;
      acc[b][i][j] += t[u];
      asm volatile("" : "+v"(acc[b][i][j]) :: "memory");   // the sums exist before the next batch
    }
  }
}

__global__ __launch_bounds__(kThreads, 1) void swiglu_tail_down_kernel(SwigluFused f) {
  constexpr int BM = 256, BN = 128, NB = 2;
  using W = WaveTile<BM, BN>;
  extern __shared__ __align__(1024) uint8_t smem[];
  floatx4 acc[NB][W::TM][W::TN];
  const int tiles_m = (f.tail.m + BM - 1) / BM;
  const int T = tiles_m * f.tail_cols;
  const bool producer = (int)blockIdx.x < T;
  const int i = producer ? (int)blockIdx.x : (int)blockIdx.x - T;
  // tile i: column tile i % tail_cols of row tile i / tail_cols; workgroups i and
  // T + i sit on the same XCD (T is a multiple of 8), each XCD holding two column
  // tiles of every row tile
  const int tm = i / f.tail_cols, tc = i % f.tail_cols;
  constexpr size_t kParkTile = (size_t)kWaves * NB * W::TM * W::TN * 64;   // floatx4 per tile
  if (producer) {
    gemm_mainloop<BM, BN, NB, true, false, kBK, kStages, 1>(f.tail, tm * BM, tc * BN, 0, smem, acc);
    gemm_epilogue<BM, BN, NB, Epi::kSwiGLU>(f.tail, tm * BM, tc * BN, 0, acc);
    publish(&f.row_done[tm]);   // its barrier also ends this workgroup's LDS reads
    gemm_mainloop<BM, BN, NB, true, false, kBK, kStages, 1>(f.down_a, tm * BM, tc * 2 * BN, 0, smem, acc);
    park_acc(f.park + (size_t)i * kParkTile, acc);
    publish(&f.park_flag[i]);
  } else {
    const KDep dep{f.dep_kt, &f.row_done[tm], f.tail_cols};
    gemm_mainloop<BM, BN, NB, true, false, kBK, kStages, 1, true>(f.down_b, tm * BM, tc * 2 * BN, 0, smem,
                                                                 acc, dep);
    if (threadIdx.x < 64) wait_flag(&f.park_flag[i], 1);
    __syncthreads();
    add_parked(f.park + (size_t)i * kParkTile, acc);
    gemm_epilogue<BM, BN, NB, Epi::kStore, BN>(f.down_b, tm * BM, tc * 2 * BN, 0, acc);
  }
}

// ---------------------------------------------------------------- small-K batched GEMM
// bmm with K <= 64 is bound by writing its fp32 output (16 x 4096 x 4096 = 1.07 GB at
// the NKIBench shape): the arithmetic is 2*K flop per 4-byte output.  This kernel
// keeps the output path as the only heavy traffic: no LDS, no split pre-pass, few
// registers, so several waves per SIMD overlap one tile's stores with the next
// tile's loads.  Each wave computes a 64x64 block of C: its A fragments (8
// consecutive k of one row, 32 contiguous bytes) and B fragments (8 consecutive k
// of one column, one coalesced 64-byte row segment per k across 16 lanes) are read
// straight from global memory, split into bf16 (hi, lo) in registers, and
// accumulated as hi*hi + hi*lo + lo*hi per 32-k step (about 2^-16 relative).
constexpr int kSmallKMax = 64;
constexpr int kSkWave = 64;                   // C block per wave (rows and columns)
constexpr int kSkThreads = 256;               // 2 x 2 waves -> 128 x 128 per workgroup
constexpr int kSkTile = 2 * kSkWave;

__device__ __forceinline__ void split8(const float (&x)[8], bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    // one conversion per element keeps this kernel's register count lowest
    const uint32_t h0 = f32_to_bf16_bits(x[2 * e]), h1 = f32_to_bf16_bits(x[2 * e + 1]);
    const float r0 = x[2 * e] - bf16_bits_to_f32(h0), r1 = x[2 * e + 1] - bf16_bits_to_f32(h1);
    h[e] = h0 | (h1 << 16);
    l[e] = pack_bf16x2(r0, r1);
  }
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}

__global__ __launch_bounds__(kSkThreads, 4) void bmm_smallk_kernel(const float* __restrict__ a,
                                                                const float* __restrict__ b,
                                                                float* __restrict__ c, int m,
                                                                int n, int k, int tiles_n) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // scalar
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
  const int64_t bz = blockIdx.y;
  const int m0 = tm * kSkTile + (wave >> 1) * kSkWave;
  const int n0 = tn * kSkTile + (wave & 1) * kSkWave;
  const float* ab = a + bz * (int64_t)m * k;
  const float* bb = b + bz * (int64_t)k * n;
  float* cb = c + bz * (int64_t)m * n;
  const int l16 = lane & 15, g = lane >> 4;
  floatx4 acc[4][4];   // [row tile i][col tile j]: lane holds C[m0+16i+l16][n0+16j+4g .. +3]
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < k; k0 += 32) {
    bf16x8 bh[4], bl[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {   // columns past N read the last column
      const int col = min(n0 + 16 * j + l16, n - 1);
      const float* src = bb + (int64_t)(k0 + 8 * g) * n + col;
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = src[(int64_t)e * n];
      split8(x, bh[j], bl[j]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {   // rows past M read the last row (their outputs are dropped)
      const int row = min(m0 + 16 * i + l16, m - 1);
      const floatx4* src = reinterpret_cast<const floatx4*>(ab + (int64_t)row * k + k0 + 8 * g);
      const floatx4 v0 = src[0], v1 = src[1];
      const float x[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
      bf16x8 ah, al;
      split8(x, ah, al);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh[j], ah, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bl[j], ah, acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh[j], al, acc[i][j], 0, 0, 0);
      }
    }
  }
  // Epilogue through LDS: per 16-row block, the accumulator layout (16 rows x 64 B
  // per store instruction) is transposed so that each non-temporal store writes
  // 4 rows x 256 contiguous bytes (measured 5.9 TB/s against 3.4 TB/s).  Each wave
  // uses its own 16 x 68-float buffer (rows padded by 4 floats: conflict-free for
  // both the writes and the reads); no barrier is needed within a wave.
  // The lane index is derived again from the exec mask (mbcnt) rather than kept
  // in a register across the K loop: at 4 waves per SIMD (128 VGPRs) that one
  // register was spilled, and a kernel with scratch is dispatched more slowly.
  __shared__ __align__(16) float stage[4][16][kSkWave + 4];
  float (*buf)[kSkWave + 4] = stage[wave];
  {
    const int lane_e = (int)__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    const int l16e = lane_e & 15, ge = lane_e >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<floatx4*>(&buf[l16e][16 * j + 4 * ge]) = acc[i][j];
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = 4 * q + ge;              // row within the block
      const floatx4 v = *reinterpret_cast<const floatx4*>(&buf[r][4 * l16e]);
      const int row = m0 + 16 * i + r;
      const int col = n0 + 4 * l16e;
      if (row < m && col < n)
        __builtin_nontemporal_store(v, reinterpret_cast<floatx4*>(cb + (int64_t)row * n + col));
    }
    __builtin_amdgcn_wave_barrier();
  }
  }
}

// Persistent form of the small-K bmm for K = 64 and whole 128 x 128 tiles: two
// workgroups per CU each loop over tiles, and the stores of one tile stay in
// flight while the operands of the next arrive and are multiplied.  vmcnt
// counts loads and stores together and retires them in issue order, so a wave
// issues the operand DMAs of tile t+1 before the 16 stores of tile t, and at the
// top of the next iteration waits with vmcnt(16): the DMAs are done, the stores
// need not be.  The operands go straight from global memory into LDS (no
// registers held across the stores): A as 128 rows x 256 bytes (16-byte chunk c
// of row r at position c ^ (r & 15)), B as 64 k-rows x 512 bytes (chunk c of
// k-row r at position (c - 4 * ((r >> 3) & 3)) mod 32), both conflict-free for
// the fragment reads.  After the MFMAs the 64 KiB is reused to transpose the
// accumulators into 4-row x 256-byte store pieces, as in bmm_smallk_kernel
// (wave w's 64 x 64 block at 16 KiB * w, chunk c of row r at position c ^ (r & 15)).
constexpr int kPkTile = 128;                       // C tile per workgroup
constexpr int kPkK = 64;                           // the only K it takes
constexpr int kPkABytes = kPkTile * kPkK * 4;      // 32 KiB
constexpr int kPkBBytes = kPkK * kPkTile * 4;      // 32 KiB
constexpr int kPkDmaPerWave = (kPkABytes + kPkBBytes) / 1024 / 4;   // 16
constexpr int kPkStores = 16;                      // 64 x 64 fp32 per wave, 1 KiB per store
constexpr int kPkWgPerCu = 2;

// B k-row r's chunk rotation (a multiple of 4 chunks = 16 banks per 8-row group).
__host__ __device__ __forceinline__ int pk_brot(int r) { return 4 * ((r >> 3) & 3); }

// Tile t of the batched grid: (batch, row block, column block), column blocks fastest.
struct PkTile {
  int64_t bz;
  int tm, tn;
};
__host__ __device__ __forceinline__ PkTile pk_tile(int64_t t, int tiles_m, int tiles_n) {
  const int64_t per_b = (int64_t)tiles_m * tiles_n;
  const int r = (int)(t % per_b);
  return PkTile{t / per_b, r / tiles_n, r % tiles_n};
}
// Byte offsets, from the tile's first A row / first B element, of the 16 bytes
// that lane `lane` of DMA instruction `inst` (0..31 for A, 0..31 for B) fetches.
__host__ __device__ __forceinline__ uint32_t pk_a_off(int inst, int lane) {
  const int row = inst * 4 + (lane >> 4);
  return (uint32_t)(row * (kPkK * 4) + (((lane & 15) ^ (row & 15)) << 4));
}
__host__ __device__ __forceinline__ uint32_t pk_b_off(int inst, int lane, int n) {
  const int row = inst * 2 + (lane >> 5);
  return (uint32_t)row * (uint32_t)n * 4u + (uint32_t)((((lane & 31) + pk_brot(row)) & 31) << 4);
}

// split8 with one conversion per pair of hi values: the same limbs, fewer VALU
// instructions (this kernel has the registers for it).
__device__ __forceinline__ void split8_pairs(const float (&x)[8], bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint32_t he, le;
    split_bf16x2(x[2 * e], x[2 * e + 1], he, le);
    h[e] = he;
    l[e] = le;
  }
  hi = __builtin_bit_cast(bf16x8, h);
  lo = __builtin_bit_cast(bf16x8, l);
}

__global__ __launch_bounds__(kSkThreads, kPkWgPerCu) void bmm_smallk_persist_kernel(
    const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ c, int m, int n,
    int tiles_m, int tiles_n, int64_t tiles) {
  __shared__ __align__(1024) uint8_t lds[kPkABytes + kPkBBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15, g = lane >> 4;
  const int wr = 64 * (wave >> 1), wc = 64 * (wave & 1);   // the wave's 64 x 64 block in the tile

  auto issue = [&](int64_t t) {
    const PkTile pt = pk_tile(t, tiles_m, tiles_n);
    const float* as = a + (pt.bz * m + (int64_t)pt.tm * kPkTile) * kPkK;
    const float* bs = b + pt.bz * kPkK * (int64_t)n + (int64_t)pt.tn * kPkTile;
#pragma unroll
    for (int q = 0; q < kPkDmaPerWave / 2; ++q) {
      const int inst = 4 * q + wave;
      dma16(as, pk_a_off(inst, lane), lds_addr(lds + inst * 1024));
    }
#pragma unroll
    for (int q = 0; q < kPkDmaPerWave / 2; ++q) {
      const int inst = 4 * q + wave;
      dma16(bs, pk_b_off(inst, lane, n), lds_addr(lds + kPkABytes + inst * 1024));
    }
  };

  int64_t t = blockIdx.x;
  issue(t);
  wait_vmcnt<0>();
  for (;;) {
    __builtin_amdgcn_s_barrier();   // every wave's DMAs of tile t have landed
    asm volatile("" ::: "memory");
    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 bh[4], bl[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int cb = wc + 16 * j + l16;
        const int pos = ((cb >> 2) - pk_brot(32 * ks + 8 * g)) & 31;
        const uint8_t* src = lds + kPkABytes + (32 * ks + 8 * g) * (kPkTile * 4) + (pos << 4) + 4 * (cb & 3);
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = *reinterpret_cast<const float*>(src + e * (kPkTile * 4));
        split8_pairs(x, bh[j], bl[j]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ra = wr + 16 * i + l16;
        const int pos = (8 * ks + 2 * g) ^ l16;
        const uint8_t* row = lds + ra * (kPkK * 4);
        const floatx4 v0 = *reinterpret_cast<const floatx4*>(row + (pos << 4));
        const floatx4 v1 = *reinterpret_cast<const floatx4*>(row + ((pos ^ 1) << 4));
        const float x[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        bf16x8 ah, al;
        split8_pairs(x, ah, al);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh[j], ah, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bl[j], ah, acc[i][j], 0, 0, 0);
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh[j], al, acc[i][j], 0, 0, 0);
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();   // every wave is done reading the operands
    asm volatile("" ::: "memory");
    uint8_t* stage = lds + wave * 16384;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<floatx4*>(stage + (16 * i + l16) * 256 + (((4 * j + g) ^ l16) << 4)) = acc[i][j];
    __builtin_amdgcn_wave_barrier();
    floatx4 v[kPkStores];
#pragma unroll
    for (int q = 0; q < kPkStores; ++q) {
      const int r = 4 * q + g;   // rows 16i + 4qq + g, q = 4i + qq
      v[q] = *reinterpret_cast<const floatx4*>(stage + r * 256 + ((l16 ^ (r & 15)) << 4));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();   // every wave holds its tile: the LDS is free
    asm volatile("" ::: "memory");
    const PkTile pt = pk_tile(t, tiles_m, tiles_n);
    const int64_t next = t + gridDim.x;
    if (next < tiles) issue(next);
    float* cb = c + (pt.bz * m + (int64_t)pt.tm * kPkTile + wr) * n + (int64_t)pt.tn * kPkTile + wc + 4 * l16;
#pragma unroll
    for (int q = 0; q < kPkStores; ++q)
      __builtin_nontemporal_store(v[q], reinterpret_cast<floatx4*>(cb + (int64_t)(4 * q + g) * n));
    if (next >= tiles) break;
    t = next;
    wait_vmcnt<kPkStores>();   // the DMAs of tile `next`; this tile's stores may stay in flight
  }
}

// ---------------------------------------------------------------- pre-passes

// Up to kMaxSplitJobs fp32 arrays, each split into (hi, lo) bf16 planes in one
// launch: job t covers flat 4-element indices [end[t-1], end[t]).
constexpr int kMaxSplitJobs = 4;
struct SplitJobs {
  const floatx4* x[kMaxSplitJobs];
  u32x2* hi[kMaxSplitJobs];
  u32x2* lo[kMaxSplitJobs];
  int64_t end[kMaxSplitJobs];   // cumulative counts of 4-element groups
  int n;
};

// One 4-element group of job-relative index i into its planes.
__device__ __forceinline__ void split_group(const floatx4* __restrict__ x, u32x2* __restrict__ hi,
                                            u32x2* __restrict__ lo, int64_t i) {
  const floatx4 v = __builtin_nontemporal_load(x + i);
  uint32_t h0, h1, l0, l1;
  split_bf16x2(v[0], v[1], h0, l0);
  split_bf16x2(v[2], v[3], h1, l1);
  hi[i] = u32x2{h0, h1};
  lo[i] = u32x2{l0, l1};
}

// Grid-stride over the groups of all jobs, starting at workgroup `b0` of `nb`.
__device__ __forceinline__ void split_jobs(const SplitJobs& j, int64_t b0, int64_t nb) {
  const int64_t total = j.end[j.n - 1];
  for (int64_t i = b0 * 256 + threadIdx.x; i < total; i += nb * 256) {
    int t = 0;
#pragma unroll
    for (int q = 0; q < kMaxSplitJobs - 1; ++q) t += (q < j.n - 1 && i >= j.end[q]) ? 1 : 0;
    split_group(j.x[t], j.hi[t], j.lo[t], i - (t ? j.end[t - 1] : 0));
  }
}

// fp32 -> (hi, lo) bf16 planes: hi = bf16(x), lo = bf16(x - hi), round to
// nearest even.  Four elements per thread per step, grid-stride over every job.
__global__ __launch_bounds__(256) void split_f32_kernel(SplitJobs j) {
  split_jobs(j, blockIdx.x, gridDim.x);
}

// Sum of S fp32 split-K partial planes [S][n] (in order of the planes), split
// into bf16 (hi, lo) planes like split_f32_kernel.
__global__ __launch_bounds__(256) void sum_split_f32_kernel(const floatx4* __restrict__ part, int parts,
                                                            u32x2* __restrict__ hi, u32x2* __restrict__ lo,
                                                            int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    floatx4 v = __builtin_nontemporal_load(part + i);
    for (int z = 1; z < parts; ++z) v += __builtin_nontemporal_load(part + z * n4 + i);
    uint32_t h0, h1, l0, l1;
    split_bf16x2(v[0], v[1], h0, l0);
    split_bf16x2(v[2], v[3], h1, l1);
    hi[i] = u32x2{h0, h1};
    lo[i] = u32x2{l0, l1};
  }
}

// x [K][M] fp32 -> bf16 hi/lo planes of x^T, [M][K] (K-contiguous, so the GEMM
// reads A with ds_read_b128 fragments instead of transposed LDS reads).  One
// workgroup per 64 x 64 block through LDS; M % 8 == 0, K % 8 == 0.
// Rows of workgroups at blockIdx.y >= kblocks split `w` (the GEMM's B operand)
// meanwhile.
__global__ __launch_bounds__(256) void split_transpose_f32_kernel(const float* __restrict__ x,
                                                                  uint16_t* __restrict__ hi,
                                                                  uint16_t* __restrict__ lo,
                                                                  int64_t k, int64_t m, int kblocks,
                                                                  SplitJobs w) {
  if ((int)blockIdx.y >= kblocks) {
    split_jobs(w, (int64_t)(blockIdx.y - kblocks) * gridDim.x + blockIdx.x,
               (int64_t)(gridDim.y - kblocks) * gridDim.x);
    return;
  }
  __shared__ float tile[64][65];
  const int64_t m0 = (int64_t)blockIdx.x * 64, k0 = (int64_t)blockIdx.y * 64;
  for (int i = threadIdx.x; i < 64 * 16; i += 256) {
    const int r = i / 16, c4 = i % 16;   // r: k within the block, c4: float4 of m
    const int64_t kk = k0 + r, mm = m0 + 4 * c4;
    floatx4 v{0.f, 0.f, 0.f, 0.f};
    if (kk < k && mm < m) v = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(x + kk * m + mm));
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[r][4 * c4 + e] = v[e];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 8; i += 256) {
    const int mr = i / 8, kc = i % 8;    // mr: m within the block, kc: 8-element chunk of k
    const int64_t mm = m0 + mr, kk = k0 + 8 * kc;
    if (mm >= m || kk >= k) continue;
    u32x4 h, l;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      uint32_t he, le;
      split_bf16x2(tile[8 * kc + 2 * e][mr], tile[8 * kc + 2 * e + 1][mr], he, le);
      h[e] = he;
      l[e] = le;
    }
    *reinterpret_cast<u32x4*>(hi + mm * k + kk) = h;
    *reinterpret_cast<u32x4*>(lo + mm * k + kk) = l;
  }
}

// Zeroes n 16-bit words: the output of a product whose inner dimension is 0.
// A kernel rather than a memset, so a caller may capture the call in a graph.
__global__ __launch_bounds__(256) void zero_u16_kernel(uint16_t* __restrict__ y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    y[i] = 0;
}

// Sum of the two fp32 split-K partials [2][n] into bf16 (n % 4 == 0).
__global__ __launch_bounds__(256) void splitk2_bf16_kernel(const floatx4* __restrict__ part,
                                                           u32x2* __restrict__ y, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    const floatx4 a = __builtin_nontemporal_load(part + i);
    const floatx4 b = __builtin_nontemporal_load(part + n4 + i);
    const floatx4 v = a + b;
    y[i] = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  }
}

// Sum of the two fp32 split-K partials [2][n] into fp32 (n % 4 == 0).
__global__ __launch_bounds__(256) void splitk2_f32_kernel(const floatx4* __restrict__ part,
                                                          floatx4* __restrict__ y, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256)
    y[i] = __builtin_nontemporal_load(part + i) + __builtin_nontemporal_load(part + n4 + i);
}

// One workgroup per row of x [M][K] (fp32): y = x (+ z), then
//   t = sum_k (y^2 / K) + eps;  y = y / sqrt(t) (* g)
// in the reference's operation order, and the result is split into (hi, lo)
// bf16 planes for the GEMM.  K % 4 == 0.
constexpr int kRowThreads = 256;
// Workgroups past the last row split `w` (the GEMM's other operand) meanwhile.
static_assert(kRowThreads == 256, "split_jobs assumes 256-thread workgroups");
__global__ __launch_bounds__(kRowThreads) void rms_split_f32_kernel(
    const float* __restrict__ x, const float* __restrict__ z, const float* __restrict__ g,
    uint16_t* __restrict__ hi, uint16_t* __restrict__ lo, int k, float eps, int rows, SplitJobs w) {
  if ((int)blockIdx.x >= rows) {
    split_jobs(w, blockIdx.x - rows, gridDim.x - rows);
    return;
  }
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int k4 = k / 4;
  const floatx4* xr = reinterpret_cast<const floatx4*>(x + (int64_t)row * k);
  const floatx4* zr = z ? reinterpret_cast<const floatx4*>(z + (int64_t)row * k) : nullptr;
  const float inv_k = 1.0f / (float)k;
  float s = 0.f;
  for (int c = tid; c < k4; c += kRowThreads) {
    floatx4 v = xr[c];
    if (zr) v += zr[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) s += (v[e] * v[e]) * inv_k;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  __shared__ float part[kRowThreads / 64];
  if ((tid & 63) == 0) part[tid >> 6] = s;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < kRowThreads / 64; ++i) t += part[i];
  const float rms = sqrtf(t + eps);
  u32x2* hr = reinterpret_cast<u32x2*>(hi + (int64_t)row * k);
  u32x2* lr = reinterpret_cast<u32x2*>(lo + (int64_t)row * k);
  const floatx4* gr = reinterpret_cast<const floatx4*>(g);
  for (int c = tid; c < k4; c += kRowThreads) {
    floatx4 v = xr[c];
    if (zr) v += zr[c];
    const floatx4 gg = g ? gr[c] : floatx4{1.f, 1.f, 1.f, 1.f};
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = (v[e] / rms) * gg[e];
    uint32_t h0, h1, l0, l1;
    split_bf16x2(y[0], y[1], h0, l0);
    split_bf16x2(y[2], y[3], h1, l1);
    hr[c] = u32x2{h0, h1};
    lr[c] = u32x2{l0, l1};
  }
}

// Row normalisation after a GEMM whose epilogue wrote y = x@w + z into `out` and
// per-WN-column sums of y^2 into part[M][nchunk]:
//   out[m, n] = y[m, n] * g[n] / sqrt(sum_n y^2 / N + eps)
// One workgroup per row; both forms stream at the device's copy rate (a variant
// holding the row in registers so that every load precedes the first store
// measured the same).
__device__ __forceinline__ float row_rms(const float* __restrict__ part, int row, int nchunk,
                                         int n, float eps) {
  const int tid = threadIdx.x;
  float s = 0.f;
  for (int c = tid; c < nchunk; c += kRowThreads) s += part[(int64_t)row * nchunk + c];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  __shared__ float wpart[kRowThreads / 64];
  if ((tid & 63) == 0) wpart[tid >> 6] = s;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kRowThreads / 64; ++w) t += wpart[w];
  return sqrtf(t / (float)n + eps);
}

// fp32 rows, N % 4 == 0.
__global__ __launch_bounds__(kRowThreads) void row_rmsnorm_f32_kernel(
    float* __restrict__ out, const float* __restrict__ part, const float* __restrict__ g, int n,
    int nchunk, float eps) {
  const float rms = row_rms(part, blockIdx.x, nchunk, n, eps);
  floatx4* orow = reinterpret_cast<floatx4*>(out + (int64_t)blockIdx.x * n);
  const floatx4* gr = reinterpret_cast<const floatx4*>(g);
  for (int c = threadIdx.x; c < n / 4; c += kRowThreads) {
    floatx4 v = orow[c];
    const floatx4 gg = gr[c];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = v[e] * gg[e] / rms;
    orow[c] = v;
  }
}

// The bf16 form: the GEMM epilogue wrote bf16(y) into `out` and the fp32 sums of
// y^2 into part; out[m, n] = bf16(bf16(y[m, n]) * g[n] / rms), g bf16, N % 8 == 0.
__global__ __launch_bounds__(kRowThreads) void row_rmsnorm_bf16_kernel(
    uint16_t* __restrict__ out, const float* __restrict__ part, const uint16_t* __restrict__ g,
    int n, int nchunk, float eps) {
  const float rms = row_rms(part, blockIdx.x, nchunk, n, eps);
  u32x4* orow = reinterpret_cast<u32x4*>(out + (int64_t)blockIdx.x * n);
  const u32x4* gr = reinterpret_cast<const u32x4*>(g);
  for (int c = threadIdx.x; c < n / 8; c += kRowThreads) {
    const u32x4 v = orow[c], gg = gr[c];
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack_bf16x2(bf16_bits_to_f32(v[e] & 0xffffu) * bf16_bits_to_f32(gg[e] & 0xffffu) / rms,
                         bf16_bits_to_f32(v[e] >> 16) * bf16_bits_to_f32(gg[e] >> 16) / rms);
    orow[c] = o;
  }
}

// ---------------------------------------------------------------- RMSNorm pre-pass
// One workgroup per row: y = x (+ z when ADD, summed in fp32),
// inv_rms[m] = 1/sqrt(mean_k y[m,k]^2 + eps) (fp32 sum of squares) and
// xg[m,k] = bf16(y[m,k] * gamma[k]).  x (and z) are read once; xg stays in the
// 256 MB Infinity Cache for the GEMM that follows.
// 128 threads per row measured 11.6 us against 13.8 with 256 (4096 x 4096; 64: 12.1).
constexpr int kPrepThreads = 128;
constexpr int kPrepVec = 4;   // 16-byte chunks per thread held in registers (K <= 4096)

// The 8 values of a 16-byte bf16 chunk as fp32 (x, plus z when ADD).
template <bool ADD>
__device__ __forceinline__ void prep_values(const u32x4& xv, const u32x4& zv, float (&y)[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    y[2 * w] = bf16_bits_to_f32(xv[w] & 0xffffu);
    y[2 * w + 1] = bf16_bits_to_f32(xv[w] >> 16);
    if constexpr (ADD) {
      y[2 * w] += bf16_bits_to_f32(zv[w] & 0xffffu);
      y[2 * w + 1] += bf16_bits_to_f32(zv[w] >> 16);
    }
  }
}

template <bool ADD>
__global__ __launch_bounds__(kPrepThreads) void rms_prep_kernel(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ z,
                                                                const uint16_t* __restrict__ gamma,
                                                                uint16_t* __restrict__ xg,
                                                                float* __restrict__ inv_rms, int k,
                                                                float eps) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nchunk = k / 8;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + (int64_t)row * k);
  const u32x4* zr = ADD ? reinterpret_cast<const u32x4*>(z + (int64_t)row * k) : nullptr;
  const u32x4 zero{0u, 0u, 0u, 0u};
  u32x4 v[kPrepVec], vz[kPrepVec];
  float ssq = 0.f;
#pragma unroll
  for (int u = 0; u < kPrepVec; ++u) {
    const int c = tid + u * kPrepThreads;
    v[u] = (c < nchunk) ? __builtin_nontemporal_load(xr + c) : zero;
    vz[u] = (ADD && c < nchunk) ? __builtin_nontemporal_load(zr + c) : zero;
    float y[8];
    prep_values<ADD>(v[u], vz[u], y);
#pragma unroll
    for (int e = 0; e < 8; ++e) ssq = fmaf(y[e], y[e], ssq);
  }
  // tail chunks beyond the register-held part (K > 4096)
  for (int c = tid + kPrepVec * kPrepThreads; c < nchunk; c += kPrepThreads) {
    float y[8];
    prep_values<ADD>(xr[c], ADD ? zr[c] : zero, y);
#pragma unroll
    for (int e = 0; e < 8; ++e) ssq = fmaf(y[e], y[e], ssq);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ssq += __shfl_xor(ssq, off);
  __shared__ float part[kPrepThreads / 64];
  if ((tid & 63) == 0) part[tid >> 6] = ssq;
  __syncthreads();
  if (tid == 0) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kPrepThreads / 64; ++w) s += part[w];
    inv_rms[row] = 1.0f / sqrtf(s / (float)k + eps);
  }
  const u32x4* gr = reinterpret_cast<const u32x4*>(gamma);
  u32x4* outr = reinterpret_cast<u32x4*>(xg + (int64_t)row * k);
  auto scale_store = [&](const u32x4& t, const u32x4& tz, int c) {
    const u32x4 g = gr[c];
    float y[8];
    prep_values<ADD>(t, tz, y);
    u32x4 o;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      o[w] = pack2(y[2 * w] * bf16_bits_to_f32(g[w] & 0xffffu),
                   y[2 * w + 1] * bf16_bits_to_f32(g[w] >> 16));
    outr[c] = o;
  };
#pragma unroll
  for (int u = 0; u < kPrepVec; ++u) {
    const int c = tid + u * kPrepThreads;
    if (c < nchunk) scale_store(v[u], vz[u], c);
  }
  for (int c = tid + kPrepVec * kPrepThreads; c < nchunk; c += kPrepThreads)
    scale_store(xr[c], ADD ? zr[c] : zero, c);
}


// ---------------------------------------------------------------- launch helpers

// Tile-row group height of the tile order.  Every tile shape here holds one
// workgroup per CU, so each XCD runs about T tiles at a time: a grid that fits
// the device at once keeps all its batches resident, else the first CU-count
// tiles of batch 0 are.  Per k-step those T tiles fetch g*BM rows of A and
// ceil(T/g)*BN*NB columns of B into the XCD's L2; the g minimizing that sum is
// taken, the larger on a tie.  (Split-K SwiGLU down GEMM, 8x16 tiles of 256x256
// in 2 batches: T = 16, g = 4, measured 4 % faster than g = 8; the 256-tile
// launches with T = 32 tie from g = 4 to 8 and measure alike.)
int pick_group_m(int tiles_m, int tiles_n, int batch, int bm, int bn_all) {
  const int64_t tiles = (int64_t)tiles_m * tiles_n;
  const int64_t cus = device_cu_count();
  const int64_t conc = tiles * batch <= cus ? tiles : std::min(tiles, cus);
  const int t = (int)std::max<int64_t>(1, conc / kXcds);
  int best = 1;
  int64_t best_cost = INT64_MAX;
  for (int g = 1; g <= std::min(tiles_m, t); ++g) {
    const int64_t cost = (int64_t)g * bm + (int64_t)((t + g - 1) / g) * bn_all;
    if (cost <= best_cost) {
      best = g;
      best_cost = cost;
    }
  }
  return best;
}

template <int BM, int BN, int NB, bool A_KMAJ, Epi EPI, int NSEG, int BK = kBK, int S = kStages>
int launch_n(const Params& p, int batch, hipStream_t st, const char* what) {
  Params a = p;
  a.group_m = pick_group_m((a.m + BM - 1) / BM, (a.n + BN - 1) / BN, batch, BM, BN * NB);
  const int tiles = ((a.m + BM - 1) / BM) * ((a.n + BN - 1) / BN);
  const size_t lds = (size_t)S * (BM + NB * BN) * BK * sizeof(uint16_t);
  static const bool attr_ok = [&] {
    const hipError_t e1 = hipFuncSetAttribute(
        reinterpret_cast<const void*>(gemm_kernel<BM, BN, NB, A_KMAJ, EPI, false, BK, S, NSEG>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    const hipError_t e2 = hipFuncSetAttribute(
        reinterpret_cast<const void*>(gemm_kernel<BM, BN, NB, A_KMAJ, EPI, true, BK, S, NSEG>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    return e1 == hipSuccess && e2 == hipSuccess;
  }();
  if (!attr_ok) return set_error(KDA_ERR_HIP, "%s: cannot reserve %zu bytes of LDS", what, lds);
  if (batch > 65535) return set_error(KDA_ERR_UNSUPPORTED, "%s: batch %d too large", what, batch);
  const dim3 grid(tiles, batch);
  if (a.k % BK == 0)
    hipLaunchKernelGGL((gemm_kernel<BM, BN, NB, A_KMAJ, EPI, false, BK, S, NSEG>), grid, dim3(kThreads),
                       lds, st, a);
  else
    hipLaunchKernelGGL((gemm_kernel<BM, BN, NB, A_KMAJ, EPI, true, BK, S, NSEG>), grid, dim3(kThreads),
                       lds, st, a);
  return check_launch(what);
}

// Dispatches on the segment count (1, 3 or 6).
template <int BM, int BN, int NB, bool A_KMAJ, Epi EPI, int BK = kBK, int S = kStages>
int launch(const Params& a, int batch, hipStream_t st, const char* what) {
  switch (a.nseg) {
    case 1: return launch_n<BM, BN, NB, A_KMAJ, EPI, 1, BK, S>(a, batch, st, what);
    case 3: return launch_n<BM, BN, NB, A_KMAJ, EPI, 3, BK, S>(a, batch, st, what);
    case 6: return launch_n<BM, BN, NB, A_KMAJ, EPI, 6, BK, S>(a, batch, st, what);
  }
  return set_error(KDA_ERR_UNSUPPORTED, "%s: %d K-segments", what, a.nseg);
}

// Every segment but a lone one must span whole k-tiles of `bk`.
bool segments_fit(const Params& a, int bk) {
  if (a.nseg == 1) return true;
  for (int i = 0; i < a.nseg; ++i)
    if (a.seg[i].k % bk) return false;
  return true;
}

// Chooses the N tile: 256 when that still gives at least one wave of tiles over
// the device, else 128 (more, smaller tiles for skinny problems).  The 256x128
// tile runs with 64-deep k-tiles in a 2-slot ring where the segments allow:
// measured 5-9 % faster than 32-deep k-tiles in 4 slots (half the barriers per
// k), while the 256x256 tile keeps 32-deep k-tiles (its 64-deep ring fits only 2
// slots and was 12 % slower).
template <bool A_KMAJ, Epi EPI>
int launch_auto(const Params& a, int batch, hipStream_t st, const char* what) {
  const int64_t tiles256 = (int64_t)((a.m + 255) / 256) * ((a.n + 255) / 256) * batch;
  if (tiles256 >= device_cu_count()) return launch<256, 256, 1, A_KMAJ, EPI>(a, batch, st, what);
  if (segments_fit(a, 64)) return launch<256, 128, 1, A_KMAJ, EPI, 64, 2>(a, batch, st, what);
  return launch<256, 128, 1, A_KMAJ, EPI>(a, batch, st, what);
}

Params make_params(int64_t m, int64_t n, void* c, int64_t ldc) {
  Params p{};
  p.m = (int)m;
  p.n = (int)n;
  p.c = c;
  p.ldc = ldc;
  return p;
}

void add_seg(Params& p, const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb, int64_t k,
             const uint16_t* b2 = nullptr) {
  Seg& s = p.seg[p.nseg++];
  s.a = a;
  s.b = b;
  s.b2 = b2;
  s.lda = lda;
  s.ldb = ldb;
  s.k = (int)k;
  p.k += (int)k;
}

// The three K-segments of a split fp32 product A@B ~= Ah@Bh + Ah@Bl + Al@Bh.
void add_split_segs(Params& p, const uint16_t* ah, const uint16_t* al, int64_t lda,
                    const uint16_t* bh, const uint16_t* bl, int64_t ldb, int64_t k,
                    const uint16_t* b2h = nullptr, const uint16_t* b2l = nullptr) {
  add_seg(p, ah, lda, bh, ldb, k, b2h);
  add_seg(p, ah, lda, bl, ldb, k, b2l);
  add_seg(p, al, lda, bh, ldb, k, b2h);
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
  // a and b hold no element when K = 0 (empty tensors may have null data)
  if (m && n && (!c || (k && (!a || !b)))) return set_error(KDA_ERR_INVALID_ARG, "%s: null pointer", what);
  if (!aligned16(a) || !aligned16(b) || !aligned16(c))
    return set_error(KDA_ERR_INVALID_ARG, "%s: pointers must be 16-byte aligned", what);
  return KDA_OK;
}

// `need` is the operator's workspace_bytes(): -1 when its sizes have no
// representable workspace, which is refused like a missing buffer.
int check_ws(const char* what, const void* ws, int64_t ws_bytes, int64_t need) {
  if (need < 0)
    return set_error(KDA_ERR_UNSUPPORTED, "%s: sizes beyond the workspace's addressable range", what);
  if (need > 0 && (!ws || !aligned16(ws) || ws_bytes < need))
    return set_error(KDA_ERR_INVALID_ARG,
                     "%s: workspace must be 16-byte aligned and >= %lld bytes (got %lld)", what,
                     (long long)need, (long long)ws_bytes);
  return KDA_OK;
}

// fp32 arrays to split into bf16 (hi, lo) planes by one launch.
struct SplitBatch {
  SplitJobs j{};
  int add(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, const char* what) {
    if (n % 4)
      return set_error(KDA_ERR_UNSUPPORTED, "%s: element count %lld not a multiple of 4", what, (long long)n);
    if (!aligned16(x)) return set_error(KDA_ERR_INVALID_ARG, "%s: fp32 input must be 16-byte aligned", what);
    if (n == 0) return KDA_OK;
    if (j.n == kMaxSplitJobs) return set_error(KDA_ERR_UNSUPPORTED, "%s: too many split jobs", what);
    j.x[j.n] = reinterpret_cast<const floatx4*>(x);
    j.hi[j.n] = reinterpret_cast<u32x2*>(hi);
    j.lo[j.n] = reinterpret_cast<u32x2*>(lo);
    j.end[j.n] = (j.n ? j.end[j.n - 1] : 0) + n / 4;
    ++j.n;
    return KDA_OK;
  }
  int64_t groups() const { return j.n ? j.end[j.n - 1] : 0; }
  // workgroups of 256 threads for the batch (one group per thread, at most 16 per CU)
  int64_t blocks() const { return std::min<int64_t>((groups() + 255) / 256, (int64_t)device_cu_count() * 16); }
  int launch(hipStream_t st, const char* what) const {
    if (groups() == 0) return KDA_OK;
    hipLaunchKernelGGL(split_f32_kernel, dim3((unsigned)blocks()), dim3(256), 0, st, j);
    return check_launch(what);
  }
};

int split(const float* x, int64_t n, uint16_t* hi, uint16_t* lo, hipStream_t st, const char* what) {
  SplitBatch b;
  if (int rc = b.add(x, n, hi, lo, what)) return rc;
  return b.launch(st, what);
}

// ---- workspace plans (shared by the size query and the entry points)
struct SplitPlan {     // hi/lo planes of A [count_a] and B [count_b]
  uint16_t *ah, *al, *bh, *bl;
};
SplitPlan plan_split(Carve& c, SizeTerm count_a, SizeTerm count_b) {
  SplitPlan s;
  s.ah = c.take<uint16_t>(count_a);
  s.al = c.take<uint16_t>(count_a);
  s.bh = c.take<uint16_t>(count_b);
  s.bl = c.take<uint16_t>(count_b);
  return s;
}
// K-chunks for the small GEMM t = x @ a [M, R]: its 256x128 tiles would occupy few
// CUs (4096 x 128: 16 tiles), so K is split into up to kLoraMaxParts chunks run as
// a batch into fp32 partials (each chunk a whole number of 64-deep k-tiles).  The
// count depends on the device's CU count; the workspace always holds
// kLoraMaxParts partials, so its size does not.
constexpr int kLoraMaxParts = 16;
int lora_t_parts(int64_t m, int64_t k, int64_t r) {
  const SizeTerm tiles = ceil_div(m, 256) * ceil_div(r, 128);
  int parts = 1;
  while (parts < kLoraMaxParts && tiles.ok() && tiles.v * parts * 2 <= device_cu_count() &&
         k % (parts * 2 * 64) == 0)
    parts *= 2;
  return parts;
}
struct LoraPlan {
  SplitPlan xw;        // x [M,K], w [K,N]
  uint16_t *ah, *al;   // a [K,R]
  float* t;            // x@a [M,R], as `parts` split-K partials [parts][M][R]
  int parts;
  uint16_t *th, *tl;   // split t
  uint16_t *bh, *bl;   // b [R,N]
};
LoraPlan plan_lora(Carve& c, int64_t m, int64_t k, int64_t n, int64_t r) {
  LoraPlan p;
  const SizeTerm M(m), K(k), N(n), R(r);
  p.xw = plan_split(c, M * K, K * N);
  p.ah = c.take<uint16_t>(K * R);
  p.al = c.take<uint16_t>(K * R);
  p.parts = r > 0 ? lora_t_parts(m, k, r) : 1;
  p.t = c.take<float>(SizeTerm(kLoraMaxParts) * M * R);
  p.th = c.take<uint16_t>(M * R);
  p.tl = c.take<uint16_t>(M * R);
  p.bh = c.take<uint16_t>(R * N);
  p.bl = c.take<uint16_t>(R * N);
  return p;
}
struct SwigluPlan {
  uint16_t *xh, *xl, *gh, *gl, *uh, *ul;
  uint16_t *hh, *hl, *dh, *dl;
  float* part;
};
SwigluPlan plan_swiglu(Carve& c, int64_t m, int64_t k, int64_t f) {
  SwigluPlan p;
  const SizeTerm M(m), K(k), F(f);
  p.xh = c.take<uint16_t>(M * K);
  p.xl = c.take<uint16_t>(M * K);
  p.gh = c.take<uint16_t>(K * F);
  p.gl = c.take<uint16_t>(K * F);
  p.uh = c.take<uint16_t>(K * F);
  p.ul = c.take<uint16_t>(K * F);
  p.hh = c.take<uint16_t>(M * F);
  p.hl = c.take<uint16_t>(M * F);
  p.dh = c.take<uint16_t>(F * K);
  p.dl = c.take<uint16_t>(F * K);
  p.part = c.take<float>(SizeTerm(2) * M * K);   // split-K partials of the down GEMM
  return p;
}
struct RmsBf16Plan {
  uint16_t* xg;
  float* inv;
};
RmsBf16Plan plan_rms_bf16(Carve& c, int64_t m, int64_t k) {
  RmsBf16Plan p;
  p.xg = c.take<uint16_t>(SizeTerm(m) * k);
  p.inv = c.take<float>(m);
  return p;
}

// SwiGLU gate/up GEMM on 256x128 tiles: when the tile count leaves a last, partly
// idle round over the device and those r tiles are whole tile columns filling at
// most half a round, the last f_tail = (r / tile rows) * 128 columns run on
// 128x128 tiles (2r of them: one round over the device, full K, the same
// silu(g)*u epilogue), and the rest in full rounds of 256x128 tiles.
struct UpSplit {
  int64_t f_main, f_tail;
};
UpSplit plan_up(int64_t m, int64_t f) {
  const int64_t cu = device_cu_count();
  const int64_t tm = (m + 255) / 256, t = tm * ((f + 127) / 128), r = t % cu;
  if (t <= cu || r == 0 || r % tm || 2 * r > cu || f % 128)
    return {f, 0};
  const int64_t ft = (r / tm) * 128;
  return {f - ft, ft};
}

int64_t workspace_bytes(int op, int64_t b, int64_t m, int64_t k, int64_t n, int64_t r) {
  // Every term is checked arithmetic (SizeTerm): sizes whose workspace does not
  // fit in int64 give -1, as do negative sizes and unknown operators.
  if (b < 0 || m < 0 || k < 0 || n < 0 || r < 0) return -1;
  const SizeTerm B(b), M(m), K(k), N(n);
  Carve c{nullptr};
  switch (op) {
    case KDA_OP_MATMUL_F32:
    case KDA_OP_TRANSPOSE_MATMUL_F32:
    case KDA_OP_RMSNORM_MATMUL_F32:
    case KDA_OP_ADD_RMSNORM_MATMUL_F32:
      plan_split(c, M * K, K * N);
      break;
    case KDA_OP_MATMUL_ADD_RMSNORM_F32:
      plan_split(c, M * K, K * N);
      c.take<float>(M * ceil_div(n, 32));
      break;
    case KDA_OP_BMM_F32:
      plan_split(c, B * M * K, B * K * N);
      break;
    case KDA_OP_LORA_F32:
      plan_lora(c, m, k, n, r);
      break;
    case KDA_OP_SWIGLU_F32:
      plan_swiglu(c, m, k, n);
      break;
    case KDA_OP_RMSNORM_MATMUL_BF16:
    case KDA_OP_ADD_RMSNORM_MATMUL_BF16:
      plan_rms_bf16(c, m, k);
      break;
    case KDA_OP_MATMUL_ADD_RMSNORM_BF16:  // row partials of the sum of squares
      c.take<float>(M * ceil_div(n, 32));
      break;
    case KDA_OP_BMM_SOFTMAX_F32:   // two fp16 limb planes of rhs^T [B][N][64], tile scales [B][N/64]
      c.take<uint16_t>(SizeTerm(2) * B * N * 64 + SizeTerm(2) * B * ceil_div(n, 64));
      break;
    case KDA_OP_GQA_F32:           // m = S, k = Hq, n = Hkv
      return gqa_f32_workspace_bytes(b, m, k, n);
    case KDA_OP_SWIGLU_BF16:       // fp32 split-K partials of the down GEMM, [2][M][K]
      c.take<float>(SizeTerm(2) * M * K);
      break;
    default:
      return -1;
  }
  return c.used;
}

int check_split_k(const char* what, int64_t k) {
  if (k % kBK)
    return set_error(KDA_ERR_UNSUPPORTED, "%s: K (%lld) must be a multiple of %d on the fp32 path",
                     what, (long long)k, kBK);
  return KDA_OK;
}

// Zero `bytes` bytes (a multiple of 2) of a kernel output on `st`.
int zero_output(void* y, int64_t bytes, hipStream_t st, const char* what) {
  const int64_t n = bytes / 2;
  const unsigned blocks = (unsigned)(n / 256 + 1 < 2048 ? n / 256 + 1 : 2048);
  hipLaunchKernelGGL(zero_u16_kernel, dim3(blocks), dim3(256), 0, st, reinterpret_cast<uint16_t*>(y), n);
  return check_launch(what);
}

}  // namespace gemm
}  // namespace kda

using namespace kda;
using namespace kda::gemm;

extern "C" int64_t kda_workspace_size(int op, int64_t batch, int64_t m, int64_t k, int64_t n,
                                      int64_t r) {
  if (batch < 0 || m < 0 || k < 0 || n < 0 || r < 0) return -1;
  return workspace_bytes(op, batch, m, k, n, r);
}

// ---------------------------------------------------------------- bf16 entry points

extern "C" int kda_matmul_bf16(const kda_bf16* a, const kda_bf16* b, kda_bf16* c, int64_t m,
                               int64_t k, int64_t n, void* stream) {
  clear_error();
  if (int rc = validate("matmul_bf16", a, b, c, m, n, k)) return rc;
  if (m == 0 || n == 0) return KDA_OK;
  if (k == 0) return zero_output(c, (int64_t)m * n * 2, as_stream(stream), "matmul_bf16");
  Params p = make_params(m, n, c, n);
  add_seg(p, a, k, b, n, k);
  return launch_auto<true, Epi::kStore>(p, 1, as_stream(stream), "matmul_bf16");
}

namespace {
// RMSNorm -> matmul on bf16 operands, with the residual z added first when given:
// a pre-pass writes bf16((x (+ z)) * gamma) and 1/rms per row into the workspace,
// and the GEMM applies 1/rms in its epilogue.
int rms_matmul_bf16(const char* what, int op, const kda_bf16* x, const kda_bf16* z,
                    const kda_bf16* gamma, const kda_bf16* w, kda_bf16* y, int64_t m, int64_t k,
                    int64_t n, float eps, void* workspace, int64_t ws_bytes, void* stream) {
  if (int rc = validate(what, x, w, y, m, n, k)) return rc;
  if (k == 0) return set_error(KDA_ERR_INVALID_ARG, "%s: K must be > 0", what);
  if (!gamma || !aligned16(gamma))
    return set_error(KDA_ERR_INVALID_ARG, "%s: gamma null or not 16-byte aligned", what);
  if (op == KDA_OP_ADD_RMSNORM_MATMUL_BF16 && (!z || !aligned16(z)))
    return set_error(KDA_ERR_INVALID_ARG, "%s: z null or not 16-byte aligned", what);
  if (!(eps >= 0.f)) return set_error(KDA_ERR_INVALID_ARG, "%s: eps must be >= 0", what);
  if (m == 0 || n == 0) return KDA_OK;
  if (int rc = check_ws(what, workspace, ws_bytes, workspace_bytes(op, 1, m, k, n, 0))) return rc;
  Carve cv{reinterpret_cast<uint8_t*>(workspace)};
  const RmsBf16Plan wp = plan_rms_bf16(cv, m, k);
  hipStream_t st = as_stream(stream);
  if (op == KDA_OP_ADD_RMSNORM_MATMUL_BF16)
    hipLaunchKernelGGL(rms_prep_kernel<true>, dim3((unsigned)m), dim3(kPrepThreads), 0, st, x, z,
                       gamma, wp.xg, wp.inv, (int)k, eps);
  else
    hipLaunchKernelGGL(rms_prep_kernel<false>, dim3((unsigned)m), dim3(kPrepThreads), 0, st, x,
                       nullptr, gamma, wp.xg, wp.inv, (int)k, eps);
  if (int rc = check_launch(what)) return rc;
  Params p = make_params(m, n, y, n);
  p.row_scale = wp.inv;
  add_seg(p, wp.xg, k, w, n, k);
  return launch_auto<true, Epi::kRowScale>(p, 1, st, what);
}
}  // namespace

extern "C" int kda_rmsnorm_matmul_bf16(const kda_bf16* x, const kda_bf16* gamma, const kda_bf16* w,
                                       kda_bf16* y, int64_t m, int64_t k, int64_t n, float eps,
                                       void* workspace, int64_t workspace_bytes_, void* stream) {
  clear_error();
  return rms_matmul_bf16("rmsnorm_matmul_bf16", KDA_OP_RMSNORM_MATMUL_BF16, x, nullptr, gamma, w,
                         y, m, k, n, eps, workspace, workspace_bytes_, stream);
}

extern "C" int kda_add_rmsnorm_matmul_bf16(const kda_bf16* x, const kda_bf16* w, float eps,
                                           const kda_bf16* z, const kda_bf16* g, kda_bf16* out,
                                           int64_t m, int64_t k, int64_t n, void* workspace,
                                           int64_t workspace_bytes_, void* stream) {
  clear_error();
  return rms_matmul_bf16("add_rmsnorm_matmul_bf16", KDA_OP_ADD_RMSNORM_MATMUL_BF16, x, z, g, w,
                         out, m, k, n, eps, workspace, workspace_bytes_, stream);
}

extern "C" int kda_matmul_add_rmsnorm_bf16(const kda_bf16* x, const kda_bf16* w, float eps,
                                           const kda_bf16* z, const kda_bf16* g, kda_bf16* out,
                                           int64_t m, int64_t k, int64_t n, void* workspace,
                                           int64_t workspace_bytes_, void* stream) {
  clear_error();
  const char* what = "matmul_add_rmsnorm_bf16";
  if (int rc = validate(what, x, w, out, m, n, k)) return rc;
  if (!z || !g || !aligned16(z) || !aligned16(g))
    return set_error(KDA_ERR_INVALID_ARG, "%s: z and g must be non-null and 16-byte aligned", what);
  if (!(eps >= 0.f)) return set_error(KDA_ERR_INVALID_ARG, "%s: eps must be >= 0", what);
  if (m == 0 || n == 0) return KDA_OK;
  if (k == 0) return set_error(KDA_ERR_INVALID_ARG, "%s: K must be > 0", what);
  if (int rc = check_ws(what, workspace, workspace_bytes_,
                        workspace_bytes(KDA_OP_MATMUL_ADD_RMSNORM_BF16, 1, m, k, n, 0)))
    return rc;
  hipStream_t st = as_stream(stream);
  Carve cv{reinterpret_cast<uint8_t*>(workspace)};
  float* part = cv.take<float>(m * ((n + 31) / 32));
  // The epilogue writes bf16(x@w + z) into out and per-wave-tile sums of the
  // fp32 (x@w + z)^2; the row pass scales out in place.  256-wide N tiles give
  // 64-column partials, 128-wide ones (when 256-wide tiles would leave CUs
  // idle) 32-column partials.
  Params p = make_params(m, n, out, n);
  add_seg(p, x, k, w, n, k);
  p.z = z;
  p.part = part;
  const int64_t tiles256 = ((m + 255) / 256) * ((n + 255) / 256);
  const bool narrow = tiles256 < device_cu_count();
  const int64_t nchunk = narrow ? (n + 31) / 32 : (n + 63) / 64;
  if (int rc = narrow ? launch_n<256, 128, 1, true, Epi::kAddZSsqBf16, 1, 64, 2>(p, 1, st, what)
                      : launch_n<256, 256, 1, true, Epi::kAddZSsqBf16, 1>(p, 1, st, what))
    return rc;
  hipLaunchKernelGGL(row_rmsnorm_bf16_kernel, dim3((unsigned)m), dim3(kRowThreads), 0, st, out,
                     part, g, (int)n, (int)nchunk, eps);
  return check_launch(what);
}

// ---- allocation-free RMSNorm -> matmul -------------------------------------
// A file-scope device buffer stands in for the caller's workspace.  Its name is
// not a device address in host code: the address is resolved once per device with
// hipGetSymbolAddress (the device current at the first call) and cached; only that
// address is ever passed to a kernel.  The prep kernel rewrites every byte of the
// workspace it uses (normalised rows and 1/rms) before the GEMM reads them, so no
// clearing is needed; each device keeps its buffer until the process ends.
namespace {
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[KDA_NOALLOC_SCRATCH_BYTES];
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

int scratch_address(const char* what, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(KDA_ERR_HIP, "%s: no usable current device (%d)", what, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(KDA_ERR_HIP, "%s: hipGetSymbolAddress of the scratch buffer failed: %s",
                       what, hipGetErrorString(e));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return KDA_OK;
}
}  // namespace

extern "C" int kda_rmsnorm_matmul_bf16_noalloc(const kda_bf16* x, const kda_bf16* gamma,
                                               const kda_bf16* w, kda_bf16* y, int64_t m,
                                               int64_t k, int64_t n, float eps, void* stream) {
  clear_error();
  const char* what = "rmsnorm_matmul_bf16_noalloc";
  if (m < 0 || k < 0 || n < 0)
    return set_error(KDA_ERR_INVALID_ARG, "%s: negative size (M=%lld K=%lld N=%lld)", what,
                     (long long)m, (long long)k, (long long)n);
  // The workspace depends on M and K only (bf16 normalised rows and 1/rms per row).
  const int64_t need = workspace_bytes(KDA_OP_RMSNORM_MATMUL_BF16, 1, m, k, n, 0);
  if (need < 0 || need > KDA_NOALLOC_SCRATCH_BYTES)
    return set_error(KDA_ERR_UNSUPPORTED,
                     "%s: M=%lld K=%lld needs %lld bytes of scratch; the static buffer holds %lld "
                     "(2*M*K + 4*M bytes must fit)",
                     what, (long long)m, (long long)k, (long long)need,
                     (long long)KDA_NOALLOC_SCRATCH_BYTES);
  // The scratch address is resolved for every call, so the entry point below never
  // sees a null workspace with a non-zero size.
  void* ws = nullptr;
  if (int rc = scratch_address(what, &ws)) return rc;
  return kda_rmsnorm_matmul_bf16(x, gamma, w, y, m, k, n, eps, ws, KDA_NOALLOC_SCRATCH_BYTES,
                                 stream);
}

extern "C" int kda_swiglu_bf16(const kda_bf16* x, const kda_bf16* w_up, const kda_bf16* w_down,
                               const kda_bf16* w_gate, kda_bf16* h, kda_bf16* y, int64_t m,
                               int64_t k, int64_t f, void* workspace, int64_t workspace_bytes_,
                               void* stream) {
  clear_error();
  if (int rc = validate("swiglu_bf16(up/gate)", x, w_gate, h, m, f, k)) return rc;
  if (int rc = validate("swiglu_bf16(down)", h, w_down, y, m, k, f)) return rc;
  if (!aligned16(w_up) || (k && f && !w_up))
    return set_error(KDA_ERR_INVALID_ARG, "swiglu_bf16: w_up null or misaligned");
  if (m == 0 || k == 0) return KDA_OK;
  if (f == 0) return zero_output(y, (int64_t)m * k * 2, as_stream(stream), "swiglu_bf16");
  hipStream_t st = as_stream(stream);
  const int64_t ws_need = workspace_bytes(KDA_OP_SWIGLU_BF16, 1, m, k, f, 0);
  const bool have_ws = workspace && aligned16(workspace) && ws_need >= 0 && workspace_bytes_ >= ws_need;
  // Gate/up GEMM: the columns that would leave the last round over the device
  // partly idle (2048 x 14336: 896 tiles of 256x128 = 3.5 rounds on 256 CUs)
  // run as one round of 128x128 tiles (measured 618 -> 604 us for the operator,
  // against a split-K pair into fp32 partials plus a streaming silu(g)*u pass).
  const UpSplit us = plan_up(m, f);
  Params up = make_params(m, us.f_main, h, f);
  add_seg(up, x, k, w_gate, f, k, w_up);
  // The gate/up tail and the down GEMM in one launch of equal-work workgroups
  // (swiglu_tail_down_kernel) when the tail's 256x128 tiles pair one to one with
  // the down GEMM's 256x256 tiles and both kinds fit one round over the device
  // (2048 x 4096 -> 14336: 128 + 128 workgroups on 256 CUs).
  {
    const int64_t tiles_m = (m + 255) / 256;
    const int64_t t = tiles_m * (k / 256);
    // Down columns done by the tail workgroups: an even split of the work, less 10
    // k-tiles for the fixed extra work of a tail workgroup (a second K loop's start
    // and drain, the SiLU epilogue, the parked stores), which otherwise keeps the
    // down workgroups waiting for the parked sums (2048 x 4096 -> 14336: 0.7 %
    // faster than the even split; 4, 6, 8, 12 and 16 k-tiles measured too).
    const int64_t x_split = ((f - k) / 2 - 10 * kBK) / kBK * kBK;
    const SizeTerm park_n = SizeTerm(t) * (int64_t)(kWaves * 2 * 8 * 2 * 64);
    Carve cv{reinterpret_cast<uint8_t*>(workspace)};
    floatx4* park = cv.take<floatx4>(park_n);
    int* flags = cv.take<int>(tiles_m + t);
    if (have_ws && us.f_tail > 0 && k % 256 == 0 && us.f_tail == 128 * (k / 256) && t % kXcds == 0 &&
        2 * t <= device_cu_count() && f % kBK == 0 && x_split >= kBK && us.f_main - x_split >= 4 * kBK &&
        cv.used >= 0 && cv.used <= workspace_bytes_) {
      static const bool attr_ok =
          hipFuncSetAttribute(reinterpret_cast<const void*>(swiglu_tail_down_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kStages * 4 * kBK * 128 * 2) ==
          hipSuccess;
      if (!attr_ok) return set_error(KDA_ERR_HIP, "swiglu_bf16: cannot reserve LDS for the tail/down launch");
      up.zero = flags;                  // the flags below start at zero
      up.zero_n = (int)(tiles_m + t);
      if (int rc = launch<256, 128, 2, true, Epi::kSwiGLU>(up, 1, st, "swiglu_bf16(up/gate)")) return rc;
      SwigluFused fz{};
      fz.tail = make_params(m, us.f_tail, h + us.f_main, f);
      add_seg(fz.tail, x, k, w_gate + us.f_main, f, k, w_up + us.f_main);
      fz.down_a = make_params(m, k, y, k);
      add_seg(fz.down_a, h, f, w_down, k, x_split, w_down + 128);
      fz.down_b = make_params(m, k, y, k);
      add_seg(fz.down_b, h + x_split, f, w_down + x_split * k, k, f - x_split, w_down + x_split * k + 128);
      fz.park = park;
      fz.row_done = flags;
      fz.park_flag = flags + tiles_m;
      fz.tail_cols = (int)(k / 256);
      fz.dep_kt = (int)((us.f_main - x_split) / kBK);
      hipLaunchKernelGGL(swiglu_tail_down_kernel, dim3((unsigned)(2 * t)), dim3(kThreads),
                         kStages * 4 * kBK * 128 * 2, st, fz);
      return check_launch("swiglu_bf16(tail + down)");
    }
  }
  if (int rc = launch<256, 128, 2, true, Epi::kSwiGLU>(up, 1, st, "swiglu_bf16(up/gate)")) return rc;
  if (us.f_tail > 0) {
    Params t = make_params(m, us.f_tail, h + us.f_main, f);
    add_seg(t, x, k, w_gate + us.f_main, f, k, w_up + us.f_main);
    // 64-deep k-tiles in 3 slots (144 KiB): half the barriers per k of the 32-deep ring
    // (measured 0.6 % faster for the operator; 2 slots were 2 % slower)
    if (segments_fit(t, 64)) {
      if (int rc = launch<128, 128, 2, true, Epi::kSwiGLU, 64, 3>(t, 1, st, "swiglu_bf16(up/gate tail)"))
        return rc;
    } else if (int rc = launch<128, 128, 2, true, Epi::kSwiGLU>(t, 1, st, "swiglu_bf16(up/gate tail)")) {
      return rc;
    }
  }
  // Down GEMM y[M,K] = h[M,F] @ w_down[F,K].  When its 256x256 tiles fill at most
  // half the device (M = 2048, K = 4096: 128 tiles), F is split in two halves that
  // run as a batch of two into fp32 partials, summed into bf16 by a streaming
  // pass: 256 workgroups of the efficient 256x256 tile instead of 256x128 tiles
  // (measured 174 + 15 us against 241 us at 2048x14336x4096).
  const int64_t tiles256 = ((m + 255) / 256) * ((k + 255) / 256);
  const bool split = have_ws && 2 * tiles256 <= device_cu_count() && f % (2 * kBK) == 0 &&
                     (m * k) % 4 == 0;
  if (split) {
    float* part = reinterpret_cast<float*>(workspace);
    Params d = make_params(m, k, part, k);
    add_seg(d, h, f, w_down, k, f / 2);
    d.batch_a = f / 2;              // second half: columns F/2.. of h
    d.batch_b = (f / 2) * k;        //              rows F/2.. of w_down
    d.batch_c = m * k;              //              second partial
    if (int rc = launch<256, 256, 1, true, Epi::kStoreF32>(d, 2, st, "swiglu_bf16(down, split-K)")) return rc;
    const int64_t n4 = m * k / 4;
    const int64_t blocks = std::min<int64_t>((n4 + 255) / 256, (int64_t)device_cu_count() * 16);
    hipLaunchKernelGGL(splitk2_bf16_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                       reinterpret_cast<const floatx4*>(part), reinterpret_cast<u32x2*>(y), n4);
    return check_launch("swiglu_bf16(split-K sum)");
  }
  Params down = make_params(m, k, y, k);
  add_seg(down, h, f, w_down, k, f);
  return launch_auto<true, Epi::kStore>(down, 1, st, "swiglu_bf16(down)");
}

// ---------------------------------------------------------------- fp32 entry points
// fp32 operands, fp32 output, via the three-product bf16 split (see the header).

extern "C" int kda_matmul_f32(const float* lhs, const float* rhs, float* out, int64_t m, int64_t k,
                              int64_t n, void* workspace, int64_t ws_bytes, void* stream) {
  clear_error();
  const char* what = "matmul_f32";
  if (int rc = validate(what, lhs, rhs, out, m, n, k)) return rc;
  if (int rc = check_split_k(what, k)) return rc;
  if (m == 0 || n == 0) return KDA_OK;
  if (k == 0) return zero_output(out, (int64_t)m * n * 4, as_stream(stream), what);
  if (int rc = check_ws(what, workspace, ws_bytes, workspace_bytes(KDA_OP_MATMUL_F32, 1, m, k, n, 0)))
    return rc;
  hipStream_t st = as_stream(stream);
  Carve cv{reinterpret_cast<uint8_t*>(workspace)};
  const SplitPlan s = plan_split(cv, m * k, k * n);
  {
    SplitBatch sb;
    if (int rc = sb.add(lhs, m * k, s.ah, s.al, what)) return rc;
    if (int rc = sb.add(rhs, k * n, s.bh, s.bl, what)) return rc;
    if (int rc = sb.launch(st, what)) return rc;
  }
  Params p = make_params(m, n, out, n);
  add_split_segs(p, s.ah, s.al, k, s.bh, s.bl, n, k);
  return launch_auto<true, Epi::kStoreF32>(p, 1, st, what);
}

extern "C" int kda_transpose_matmul_f32(const float* lhs, const float* rhs, float* out, int64_t m,
                                        int64_t k, int64_t n, void* workspace, int64_t ws_bytes,
                                        void* stream) {
  clear_error();
  const char* what = "transpose_matmul_f32";
  if (int rc = validate(what, lhs, rhs, out, m, n, k)) return rc;
  if (int rc = check_split_k(what, k)) return rc;
  if (m % 8) return set_error(KDA_ERR_UNSUPPORTED, "%s: M (%lld) must be a multiple of 8", what, (long long)m);
  if (m == 0 || n == 0) return KDA_OK;
  if (k == 0) return zero_output(out, (int64_t)m * n * 4, as_stream(stream), what);
  if (int rc = check_ws(what, workspace, ws_bytes,
                        workspace_bytes(KDA_OP_TRANSPOSE_MATMUL_F32, 1, m, k, n, 0)))
    return rc;
  hipStream_t st = as_stream(stream);
  Carve cv{reinterpret_cast<uint8_t*>(workspace)};
  const SplitPlan s = plan_split(cv, m * k, k * n);
  // lhs [K][M] is split and transposed in one pass, so the GEMM runs on
  // K-contiguous A planes (measured faster than transposed LDS reads of [K][M])
  if (!aligned16(lhs)) return set_error(KDA_ERR_INVALID_ARG, "%s: lhs must be 16-byte aligned", what);
  // one launch: the 64x64 blocks of lhs, then rows of workgroups that split rhs
  SplitBatch wb;
  if (int rc = wb.add(rhs, k * n, s.bh, s.bl, what)) return rc;
  const int64_t mblocks = (m + 63) / 64, kblocks = (k + 63) / 64;
  const int64_t wrows = (wb.blocks() + mblocks - 1) / mblocks;
  if (kblocks + wrows > 65535) return set_error(KDA_ERR_UNSUPPORTED, "%s: K too large", what);
  hipLaunchKernelGGL(split_transpose_f32_kernel, dim3((unsigned)mblocks, (unsigned)(kblocks + wrows)),
                     dim3(256), 0, st, lhs, s.ah, s.al, k, m, (int)kblocks, wb.j);
  if (int rc = check_launch(what)) return rc;
  Params p = make_params(m, n, out, n);
  add_split_segs(p, s.ah, s.al, k, s.bh, s.bl, n, k);   // A planes [M][K]: lda = K
  return launch_auto<true, Epi::kStoreF32>(p, 1, st, what);
}

extern "C" int kda_bmm_f32(const float* lhs, const float* rhs, float* out, int64_t batch, int64_t m,
                           int64_t k, int64_t n, void* workspace, int64_t ws_bytes, void* stream) {
  clear_error();
  const char* what = "bmm_f32";
  if (batch < 0) return set_error(KDA_ERR_INVALID_ARG, "%s: batch < 0", what);
  if (int rc = validate(what, lhs, rhs, out, m, n, k)) return rc;
  if (int rc = check_split_k(what, k)) return rc;
  if (batch == 0 || m == 0 || n == 0) return KDA_OK;
  if (k == 0) return zero_output(out, (int64_t)batch * m * n * 4, as_stream(stream), what);
  hipStream_t st = as_stream(stream);
  if (k <= kSmallKMax) {
    // output-bound: fragments split in registers, no workspace needed
    if (!aligned16(lhs) || !aligned16(out))
      return set_error(KDA_ERR_INVALID_ARG, "%s: lhs/out must be 16-byte aligned", what);
    const int tiles_n = (int)((n + kSkTile - 1) / kSkTile);
    const int64_t tiles = ((m + kSkTile - 1) / kSkTile) * (int64_t)tiles_n;
    if (tiles > 0x7fffffff || batch > 65535)
      return set_error(KDA_ERR_UNSUPPORTED, "%s: problem too large", what);
    if (k == kPkK && m % kPkTile == 0 && n % kPkTile == 0 && n <= (1 << 24) && aligned16(rhs)) {
      // whole tiles: the persistent form (its 32-bit B DMA offsets reach 63 * N * 4 + 512 bytes)
      const int64_t all = tiles * batch;
      const int64_t grid = std::min<int64_t>(all, (int64_t)kPkWgPerCu * device_cu_count());
      hipLaunchKernelGGL(bmm_smallk_persist_kernel, dim3((unsigned)grid), dim3(kSkThreads), 0, st, lhs,
                         rhs, out, (int)m, (int)n, (int)(m / kPkTile), tiles_n, all);
      return check_launch(what);
    }
    hipLaunchKernelGGL(bmm_smallk_kernel, dim3((unsigned)tiles, (unsigned)batch), dim3(kSkThreads),
                       0, st, lhs, rhs, out, (int)m, (int)n, (int)k, tiles_n);
    return check_launch(what);
  }
  if (int rc = check_ws(what, workspace, ws_bytes, workspace_bytes(KDA_OP_BMM_F32, batch, m, k, n, 0)))
    return rc;
  Carve cv{reinterpret_cast<uint8_t*>(workspace)};
  const SplitPlan s = plan_split(cv, batch * m * k, batch * k * n);
  {
    SplitBatch sb;
    if (int rc = sb.add(lhs, batch * m * k, s.ah, s.al, what)) return rc;
    if (int rc = sb.add(rhs, batch * k * n, s.bh, s.bl, what)) return rc;
    if (int rc = sb.launch(st, what)) return rc;
  }
  Params p = make_params(m, n, out, n);
  add_split_segs(p, s.ah, s.al, k, s.bh, s.bl, n, k);
  p.batch_a = m * k;
  p.batch_b = k * n;
  p.batch_c = m * n;
  return launch_auto<true, Epi::kStoreF32>(p, (int)batch, st, what);
}

extern "C" int kda_lora_f32(const float* x, const float* w, const float* a, const float* b,
                            float* out, int64_t m, int64_t k, int64_t n, int64_t r, void* workspace,
                            int64_t ws_bytes, void* stream) {
  clear_error();
  const char* what = "lora_f32";
  if (int rc = validate(what, x, w, out, m, n, k)) return rc;
  if (int rc = validate(what, x, a, out, m, r, k)) return rc;
  if (int rc = check_split_k(what, k)) return rc;
  if (int rc = check_split_k(what, r)) return rc;
  if (!aligned16(b) || (r && n && !b)) return set_error(KDA_ERR_INVALID_ARG, "%s: b null or misaligned", what);
  if (m == 0 || n == 0) return KDA_OK;
  if (k == 0) return zero_output(out, (int64_t)m * n * 4, as_stream(stream), what);   // x@w = x@a = 0
  if (int rc = check_ws(what, workspace, ws_bytes, workspace_bytes(KDA_OP_LORA_F32, 1, m, k, n, r)))
    return rc;
  hipStream_t st = as_stream(stream);
  Carve cv{reinterpret_cast<uint8_t*>(workspace)};
  const LoraPlan lp = plan_lora(cv, m, k, n, r);
  {
    SplitBatch sb;
    if (int rc = sb.add(x, m * k, lp.xw.ah, lp.xw.al, what)) return rc;
    if (int rc = sb.add(w, k * n, lp.xw.bh, lp.xw.bl, what)) return rc;
    if (r > 0) {
      if (int rc = sb.add(a, k * r, lp.ah, lp.al, what)) return rc;
      if (int rc = sb.add(b, r * n, lp.bh, lp.bl, what)) return rc;
    }
    if (int rc = sb.launch(st, what)) return rc;
  }
  if (r > 0) {
    // t = x @ a  [M, R]
    if (lp.parts > 1 && (m * r) % 4 == 0) {
      const int64_t kc = k / lp.parts;
      Params pt = make_params(m, r, lp.t, r);
      add_split_segs(pt, lp.xw.ah, lp.xw.al, k, lp.ah, lp.al, r, kc);
      pt.batch_a = kc;       // chunk z: columns z*kc.. of x
      pt.batch_b = kc * r;   //          rows z*kc.. of a
      pt.batch_c = m * r;    //          partial plane z
      if (int rc = launch<256, 128, 1, true, Epi::kStoreF32, 64, 2>(pt, lp.parts, st, "lora_f32(x@a, split-K)"))
        return rc;
      const int64_t n4 = m * r / 4;
      const int64_t blocks = std::min<int64_t>((n4 + 255) / 256, (int64_t)device_cu_count() * 16);
      hipLaunchKernelGGL(sum_split_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                         reinterpret_cast<const floatx4*>(lp.t), lp.parts, reinterpret_cast<u32x2*>(lp.th),
                         reinterpret_cast<u32x2*>(lp.tl), n4);
      if (int rc = check_launch("lora_f32(t sum)")) return rc;
    } else {
      Params pt = make_params(m, r, lp.t, r);
      add_split_segs(pt, lp.xw.ah, lp.xw.al, k, lp.ah, lp.al, r, k);
      if (int rc = launch_auto<true, Epi::kStoreF32>(pt, 1, st, "lora_f32(x@a)")) return rc;
      if (int rc = split(lp.t, m * r, lp.th, lp.tl, st, what)) return rc;
    }
  }
  // out = x @ w + t @ b in one accumulation
  Params p = make_params(m, n, out, n);
  add_split_segs(p, lp.xw.ah, lp.xw.al, k, lp.xw.bh, lp.xw.bl, n, k);
  if (r > 0) add_split_segs(p, lp.th, lp.tl, r, lp.bh, lp.bl, n, r);
  return launch_auto<true, Epi::kStoreF32>(p, 1, st, what);
}

// Shared body of the NKIBench rmsnorm_matmul / add_rmsnorm_matmul forwards.
static int rms_matmul_f32(const char* what, int op, const float* x, const float* z, const float* g,
                          const float* w, float* out, int64_t m, int64_t k, int64_t n, float eps,
                          void* workspace, int64_t ws_bytes, void* stream) {
  if (int rc = validate(what, x, w, out, m, n, k)) return rc;
  if (int rc = check_split_k(what, k)) return rc;
  if (k == 0) return set_error(KDA_ERR_INVALID_ARG, "%s: K must be > 0", what);
  if ((z && !aligned16(z)) || (g && !aligned16(g)))
    return set_error(KDA_ERR_INVALID_ARG, "%s: z and g must be 16-byte aligned", what);
  if (!(eps >= 0.f)) return set_error(KDA_ERR_INVALID_ARG, "%s: eps must be >= 0", what);
  if (m == 0 || n == 0) return KDA_OK;
  if (int rc = check_ws(what, workspace, ws_bytes, workspace_bytes(op, 1, m, k, n, 0))) return rc;
  hipStream_t st = as_stream(stream);
  Carve cv{reinterpret_cast<uint8_t*>(workspace)};
  const SplitPlan s = plan_split(cv, m * k, k * n);
  // one launch: a workgroup per row of x, then the split of w
  SplitBatch wb;
  if (int rc = wb.add(w, k * n, s.bh, s.bl, what)) return rc;
  hipLaunchKernelGGL(rms_split_f32_kernel, dim3((unsigned)(m + wb.blocks())), dim3(kRowThreads), 0, st,
                     x, z, g, s.ah, s.al, (int)k, eps, (int)m, wb.j);
  if (int rc = check_launch(what)) return rc;
  Params p = make_params(m, n, out, n);
  add_split_segs(p, s.ah, s.al, k, s.bh, s.bl, n, k);
  return launch_auto<true, Epi::kStoreF32>(p, 1, st, what);
}

extern "C" int kda_rmsnorm_matmul_f32(const float* x, const float* w, float* out, int64_t m,
                                      int64_t k, int64_t n, void* workspace, int64_t ws_bytes,
                                      void* stream) {
  clear_error();
  return rms_matmul_f32("rmsnorm_matmul_f32", KDA_OP_RMSNORM_MATMUL_F32, x, nullptr, nullptr, w,
                        out, m, k, n, 0.0f, workspace, ws_bytes, stream);
}

extern "C" int kda_add_rmsnorm_matmul_f32(const float* x, const float* w, float eps, const float* z,
                                          const float* g, float* out, int64_t m, int64_t k,
                                          int64_t n, void* workspace, int64_t ws_bytes,
                                          void* stream) {
  clear_error();
  if (!z || !g) return set_error(KDA_ERR_INVALID_ARG, "add_rmsnorm_matmul_f32: null z or g");
  return rms_matmul_f32("add_rmsnorm_matmul_f32", KDA_OP_ADD_RMSNORM_MATMUL_F32, x, z, g, w, out,
                        m, k, n, eps, workspace, ws_bytes, stream);
}

extern "C" int kda_matmul_add_rmsnorm_f32(const float* x, const float* w, float eps, const float* z,
                                          const float* g, float* out, int64_t m, int64_t k,
                                          int64_t n, void* workspace, int64_t ws_bytes,
                                          void* stream) {
  clear_error();
  const char* what = "matmul_add_rmsnorm_f32";
  if (int rc = validate(what, x, w, out, m, n, k)) return rc;
  if (int rc = check_split_k(what, k)) return rc;
  if (!z || !g || !aligned16(z) || !aligned16(g))
    return set_error(KDA_ERR_INVALID_ARG, "%s: z and g must be non-null and 16-byte aligned", what);
  if (!(eps >= 0.f)) return set_error(KDA_ERR_INVALID_ARG, "%s: eps must be >= 0", what);
  if (m == 0 || n == 0) return KDA_OK;
  if (k == 0) return set_error(KDA_ERR_INVALID_ARG, "%s: K must be > 0", what);
  if (int rc = check_ws(what, workspace, ws_bytes,
                        workspace_bytes(KDA_OP_MATMUL_ADD_RMSNORM_F32, 1, m, k, n, 0)))
    return rc;
  hipStream_t st = as_stream(stream);
  Carve cv{reinterpret_cast<uint8_t*>(workspace)};
  const SplitPlan s = plan_split(cv, m * k, k * n);
  float* part = cv.take<float>(m * ((n + 31) / 32));
  {
    SplitBatch sb;
    if (int rc = sb.add(x, m * k, s.ah, s.al, what)) return rc;
    if (int rc = sb.add(w, k * n, s.bh, s.bl, what)) return rc;
    if (int rc = sb.launch(st, what)) return rc;
  }
  Params p = make_params(m, n, out, n);
  add_split_segs(p, s.ah, s.al, k, s.bh, s.bl, n, k);
  p.z = z;
  p.part = part;
  // Row partials of the sum of squares: one per wave tile width (64 columns for
  // 256-wide N tiles, 32 for 128-wide ones, used when 256-wide tiles would leave
  // CUs idle: 4096x2048 is 128 tiles of 256x256 on 256 CUs).
  const int64_t tiles256 = ((m + 255) / 256) * ((n + 255) / 256);
  const bool narrow = tiles256 < device_cu_count();
  const int64_t nchunk = narrow ? (n + 31) / 32 : (n + 63) / 64;
  if (int rc = narrow ? (segments_fit(p, 64) ? launch<256, 128, 1, true, Epi::kAddZSsqF32, 64, 2>(p, 1, st, what)
                                             : launch<256, 128, 1, true, Epi::kAddZSsqF32>(p, 1, st, what))
                      : launch<256, 256, 1, true, Epi::kAddZSsqF32>(p, 1, st, what))
    return rc;
  hipLaunchKernelGGL(row_rmsnorm_f32_kernel, dim3((unsigned)m), dim3(kRowThreads), 0, st, out,
                     part, g, (int)n, (int)nchunk, eps);
  return check_launch(what);
}

extern "C" int kda_swiglu_f32(const float* x, const float* w_up, const float* w_down,
                              const float* w_gate, float* out, int64_t m, int64_t k, int64_t f,
                              void* workspace, int64_t ws_bytes, void* stream) {
  clear_error();
  const char* what = "swiglu_f32";
  if (int rc = validate(what, x, w_gate, out, m, f, k)) return rc;
  if (int rc = validate(what, x, w_down, out, m, k, f)) return rc;
  if (int rc = check_split_k(what, k)) return rc;
  if (int rc = check_split_k(what, f)) return rc;
  if (!aligned16(w_up) || (k && f && !w_up))
    return set_error(KDA_ERR_INVALID_ARG, "%s: w_up null or misaligned", what);
  if (m == 0 || k == 0) return KDA_OK;
  if (f == 0) return zero_output(out, (int64_t)m * k * 4, as_stream(stream), what);
  if (int rc = check_ws(what, workspace, ws_bytes, workspace_bytes(KDA_OP_SWIGLU_F32, 1, m, k, f, 0)))
    return rc;
  hipStream_t st = as_stream(stream);
  Carve cv{reinterpret_cast<uint8_t*>(workspace)};
  const SwigluPlan sp = plan_swiglu(cv, m, k, f);
  {
    SplitBatch sb;
    if (int rc = sb.add(x, m * k, sp.xh, sp.xl, what)) return rc;
    if (int rc = sb.add(w_gate, k * f, sp.gh, sp.gl, what)) return rc;
    if (int rc = sb.add(w_up, k * f, sp.uh, sp.ul, what)) return rc;
    if (int rc = sb.add(w_down, f * k, sp.dh, sp.dl, what)) return rc;
    if (int rc = sb.launch(st, what)) return rc;
  }
  // Gate/up GEMM: as on the bf16 path, columns that would leave the last round
  // of 256x128 tiles partly idle (4096 x 3072: 384 tiles, 1.5 rounds on 256 CUs)
  // run as one round of 128x128 dual-B tiles.  The epilogue stores h =
  // silu(g) * u (fp32) directly as the bf16 (hi, lo) planes the down GEMM reads.
  const UpSplit us = plan_up(m, f);
  Params up = make_params(m, us.f_main, sp.hh, f);
  up.c2 = sp.hl;
  add_split_segs(up, sp.xh, sp.xl, k, sp.gh, sp.gl, f, k, sp.uh, sp.ul);
  if (int rc = launch<256, 128, 2, true, Epi::kSwiGLUSplit>(up, 1, st, "swiglu_f32(up/gate)")) return rc;
  if (us.f_tail > 0) {
    const int64_t c0 = us.f_main;
    Params t = make_params(m, us.f_tail, sp.hh + c0, f);
    t.c2 = sp.hl + c0;
    add_split_segs(t, sp.xh, sp.xl, k, sp.gh + c0, sp.gl + c0, f, k, sp.uh + c0, sp.ul + c0);
    // 64-deep k-tiles in 3 slots, as the bf16 tail
    if (int rc = segments_fit(t, 64)
                     ? launch_n<128, 128, 2, true, Epi::kSwiGLUSplit, 3, 64, 3>(t, 1, st,
                                                                                "swiglu_f32(up/gate tail)")
                     : launch_n<128, 128, 2, true, Epi::kSwiGLUSplit, 3>(t, 1, st, "swiglu_f32(up/gate tail)"))
      return rc;
  }
  // Down GEMM [M,F]@[F,K]: with fewer 256x128 tiles than half the device
  // (4096x1024: 128 tiles), F splits in two halves of every product segment,
  // run as a batch of two into fp32 partials and summed.
  const int64_t tiles128 = ((m + 255) / 256) * ((k + 127) / 128);
  if (2 * tiles128 <= device_cu_count() && f % 128 == 0 && (m * k) % 4 == 0) {
    Params d = make_params(m, k, sp.part, k);
    add_split_segs(d, sp.hh, sp.hl, f, sp.dh, sp.dl, k, f / 2);
    d.batch_a = f / 2;         // second half: columns F/2.. of the h planes
    d.batch_b = (f / 2) * k;   //              rows F/2.. of the w_down planes
    d.batch_c = m * k;
    if (int rc = launch<256, 128, 1, true, Epi::kStoreF32, 64, 2>(d, 2, st, "swiglu_f32(down, split-K)"))
      return rc;
    const int64_t n4 = m * k / 4;
    const int64_t blocks = std::min<int64_t>((n4 + 255) / 256, (int64_t)device_cu_count() * 16);
    hipLaunchKernelGGL(splitk2_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                       reinterpret_cast<const floatx4*>(sp.part), reinterpret_cast<floatx4*>(out), n4);
    return check_launch("swiglu_f32(split-K sum)");
  }
  Params down = make_params(m, k, out, k);
  add_split_segs(down, sp.hh, sp.hl, f, sp.dh, sp.dl, k, f);
  return launch_auto<true, Epi::kStoreF32>(down, 1, st, "swiglu_f32(down)");
}
