// Address geometry of the bf16 GQA forward kernel (attention.hip): which
// (batch, kv head, query head, rows) a workgroup and wave own, how many key tiles
// a workgroup visits, and the global byte offsets of its q loads, K/V tile DMAs
// and output stores.  The functions are host and device code: the kernel computes
// every global address through them, and a host-side replay (tests/) walks the
// same functions over every workgroup, wave and lane of a launch to check that
// each access stays inside its buffer.
#pragma once

#include <stdint.h>

#include "common.h"
#include "lds_dma.h"

namespace kda {
namespace attn {

constexpr int kD = 128;       // head dim
constexpr int kWaveRows = 32; // query rows per wave
constexpr int kBN = 64;       // keys per tile
constexpr int kWaves = 8;     // per workgroup: HPW query heads x (8 / HPW) blocks of 32 rows
constexpr int kThreads = 64 * kWaves;
constexpr int kTileBytes = kBN * kD * 2;                    // one K or V tile: 16 KiB
// The K/V DMAs are issued by waves 0-3 only: they are served first by the
// instruction arbiter of their SIMDs and otherwise wait at the barrier for the
// second wave of each SIMD, so the issue work moves off the slower waves.
constexpr int kDmaWaves = kWaves / 2;
constexpr int kDmaPerWave = kTileBytes / (kDmaWaves * 1024);   // DMA instructions per issuing wave per tile

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

// The launch's arguments for dense BSHD q/k/v and output strides (elements).
inline Args make_args(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                      int64_t batch, int64_t seq, int64_t hq, int64_t hkv, float scale,
                      int64_t o_sb, int64_t o_ss, int64_t o_sh) {
  Args a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.q_ss = hq * kD;
  a.q_sb = seq * a.q_ss;
  a.k_ss = hkv * kD;
  a.k_sb = seq * a.k_ss;
  a.o_sb = o_sb;
  a.o_ss = o_ss;
  a.o_sh = o_sh;
  a.batch = (int)batch;
  a.seq = (int)seq;
  a.hq = (int)hq;
  a.hkv = (int)hkv;
  a.scale_log2 = scale * 1.4426950408889634f;
  return a;
}

// Heads per workgroup: the largest power of two up to 8 dividing G = Hq / Hkv.
__host__ __device__ __forceinline__ int heads_per_workgroup(int64_t group) {
  return (group % 8 == 0) ? 8 : (group % 4 == 0) ? 4 : (group % 2 == 0) ? 2 : 1;
}
__host__ __device__ __forceinline__ constexpr int block_rows(int hpw) { return kWaveRows * kWaves / hpw; }

__host__ __device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }

// Workgroups of a launch: query blocks x batch x kv heads x workgroups per kv head.
inline int64_t grid_blocks(int64_t batch, int64_t seq, int64_t hq, int64_t hkv) {
  const int hpw = heads_per_workgroup(hq / hkv);
  const int64_t bm = block_rows(hpw);
  return ((seq + bm - 1) / bm) * batch * hkv * (hq / hkv / hpw);
}

// What workgroup `block`, wave `wave` owns.
struct Block {
  int b, kvh, h;   // batch, kv head, this wave's query head
  int q0, w0;      // the workgroup's first query row, this wave's first query row
  int nkt;         // key tiles the workgroup visits (0 .. nkt-1)
  int nfree;       // tiles [0, nfree) need no mask for any row of the workgroup
};

__host__ __device__ __forceinline__ Block block_of(const Args& p, bool causal, int hpw, int block, int wave) {
  const int bm = block_rows(hpw);
  const int nqb = (p.seq + bm - 1) / bm;
  const int group = p.hq / p.hkv;
  const int nsplit = group / hpw;                   // workgroups per kv head
  const int nbh = p.batch * p.hkv * nsplit;
  Block r;
  // Longest causal blocks first.
  const int qb = causal ? (nqb - 1 - block / nbh) : (block / nbh);
  const int bh = block % nbh;
  r.b = bh / (p.hkv * nsplit);
  r.kvh = (bh / nsplit) % p.hkv;
  r.h = r.kvh * group + (bh % nsplit) * hpw + (wave % hpw);
  r.q0 = qb * bm;
  r.w0 = r.q0 + (wave / hpw) * kWaveRows;
  const int nkt_all = (p.seq + kBN - 1) / kBN;
  r.nkt = causal ? imin(nkt_all, (r.q0 + bm - 1) / kBN + 1) : nkt_all;
  int nfree = p.seq / kBN;                            // full tiles
  if (causal) nfree = imin(nfree, (r.q0 + 1) / kBN);  // keys j0+63 <= q0 for every row
  r.nfree = imin(nfree, r.nkt);
  return r;
}

// Element offsets of a workgroup's q head, K/V kv head and output head.
__host__ __device__ __forceinline__ int64_t q_head(const Args& p, const Block& g) {
  return g.b * p.q_sb + (int64_t)g.h * kD;
}
__host__ __device__ __forceinline__ int64_t kv_head(const Args& p, const Block& g) {
  return g.b * p.k_sb + (int64_t)g.kvh * kD;
}
__host__ __device__ __forceinline__ int64_t out_head(const Args& p, const Block& g) {
  return g.b * p.o_sb + (int64_t)g.h * p.o_sh;
}
// Element offset, from q_head, of the 8 q values lane (l16, g) loads for query
// `row` and d chunk dc (d = dc*32 + 8g .. +8); loaded only when row < seq.
__host__ __device__ __forceinline__ int64_t q_elem(const Args& p, int row, int dc, int g) {
  return row * p.q_ss + dc * 32 + g * 8;
}
// Element offset, from out_head, of the 4 outputs lane (l16, g) stores for query
// `row` and d tile dt (d = dt*16 + 4g .. +4); stored only when row < seq.
__host__ __device__ __forceinline__ int64_t out_elem(const Args& p, int row, int dt, int g) {
  return row * p.o_ss + dt * 16 + 4 * g;
}

// ---- K/V tile DMAs: instruction j of issuing wave w (< kDmaWaves) fills LDS
// bytes [(j*kDmaWaves + w)*1024, +1024) of a tile = rows 4q .. 4q+3, 16 bytes per
// lane: lane -> (row, 16-byte chunk position lane & 15).
__host__ __device__ __forceinline__ int dma_row(int j, int wave, int lane) {
  return (j * kDmaWaves + wave % kDmaWaves) * 4 + (lane >> 4);
}
// Swizzle of the 16 16-byte chunks of a K row: conflict-free for the permuted
// 16-row fragment read (rows 32c + 8a + 4hh + r, a, r in 0..3, one chunk).
__host__ __device__ __forceinline__ int kswz(int row) { return (row & 3) | (((row >> 3) & 3) << 2); }
// Byte offset within a source row of the chunk that lane's DMA places at its
// position (the LDS swizzle applied on the global side).
__host__ __device__ __forceinline__ uint32_t dma_kcol(int r, int lane) {
  return (uint32_t)(((lane & 15) ^ kswz(r)) << 4);
}
__host__ __device__ __forceinline__ uint32_t dma_vcol(int r, int lane) {
  const int t = lane & 15;
  return (uint32_t)((((t >> 1) ^ mswz(r)) << 5) + ((t & 1) << 4));   // V keeps mswz segments
}
// Per-lane 32-bit byte offset, from the tile's first key row, of source row `r`
// (the launcher bounds Hkv so that rows 0..63 never wrap it).
__host__ __device__ __forceinline__ uint32_t dma_lane_offset(int64_t row_bytes, int r, uint32_t col) {
  return (uint32_t)(r * row_bytes) + col;
}
// ---- Persistent schedule.  The grid has G = min(blocks, CUs) workgroups;
// workgroup w runs blocks w, 2G-1-w, 2G+w, 4G-1-w, ... of the longest-first
// order (a snake over the sorted block lengths, so the totals come out even).
__host__ __device__ __forceinline__ int sched_block(int k, int w, int grid) {
  return (k & 1) ? (k + 1) * grid - 1 - w : k * grid + w;
}
__host__ __device__ __forceinline__ int total_blocks(const Args& p, int hpw) {
  const int bm = block_rows(hpw);
  return ((p.seq + bm - 1) / bm) * p.batch * p.hkv * (p.hq / p.hkv / hpw);
}

// ---- K/V tile ring.  A workgroup's key tiles, block after block, take the ring
// slots in turn: tile kt of a block whose first tile sits at ring position
// `base` uses slot (base + kt) mod kRing, for K and for V alike.
constexpr int kRing = 4;   // a power of two
__host__ __device__ __forceinline__ int ring_slot(int base, int kt) { return (base + kt) & (kRing - 1); }

// The key tiles a block's DMAs fetch: before its loop K(0), K(1), K(2) and V(0)
// (clamped to its last tile); iteration kt (0 .. nkt-1) fetches K(kt+3) and
// V(kt+1).  Past the block's last tile those DMAs fetch the next block's first
// tiles (its K(0..2) and V(0)), which that block's prologue then does not
// issue; after the workgroup's last block they fetch the last tile again (into
// a slot no longer read).  Every iteration issues the same number of DMAs.
constexpr int kPrologueK = 3;
struct Fetch {
  bool next;   // a tile of the next block
  int tile;    // key tile within its block
};
__host__ __device__ __forceinline__ Fetch k_fetch(int kt, int nkt, bool has_next, int nkt_next) {
  const int j = kt + kPrologueK;
  if (j < nkt) return Fetch{false, j};
  if (has_next) return Fetch{true, imin(j - nkt, nkt_next - 1)};
  return Fetch{false, nkt - 1};
}
__host__ __device__ __forceinline__ Fetch v_fetch(int kt, int nkt, bool has_next) {
  const int j = kt + 1;
  if (j < nkt) return Fetch{false, j};
  if (has_next) return Fetch{true, 0};
  return Fetch{false, nkt - 1};
}
__host__ __device__ __forceinline__ int prologue_k_tile(int i, int nkt) { return imin(i, nkt - 1); }
// Whether prologue tile K(i) was fetched by the previous block's last
// iterations (prev_nkt: that block's tile count, 0 for a workgroup's first block).
__host__ __device__ __forceinline__ bool prologue_k_prefetched(int i, int prev_nkt) {
  return i >= kPrologueK - prev_nkt;
}
// V(0) likewise (fetched by the previous block's last iteration).
__host__ __device__ __forceinline__ bool prologue_v_prefetched(int prev_nkt) { return prev_nkt > 0; }

// Whether all of a block's prologue tiles (K(0..2), V(0)) were prefetched.
__host__ __device__ __forceinline__ bool prologue_all_prefetched(int prev_nkt) {
  return prologue_k_prefetched(0, prev_nkt) && prologue_v_prefetched(prev_nkt);
}

// ---- q rows of the next block, staged in LDS (causal, persistent).  At the start
// of a block's last iteration (after its DMAs) each wave DMAs its 32 q rows of the
// next block into 8 KiB of LDS: waves 0-3 into a 32 KiB area of their own after
// the rings, waves 4-5 into K slot base+3 and waves 6-7 into V slot base+1, base
// being the next block's ring position.  Those two slots held the block's K(nkt-1)
// and V(nkt-3), last read in iteration nkt-2, and no DMA of this block or of the
// next block's prologue targets them.  The DMAs land during the last iteration, the
// final O += V P and the stores; issued before the stores, they are awaited at the
// top of the next block while the stores are still in flight (vmcnt retires in
// issue order).  The next block reads them before its first ring DMA into those
// slots (iteration 0, after two barriers).
constexpr int kQStageBytes = kWaveRows * kD * 2;      // 8 KiB per wave
constexpr int kQStageDma = kQStageBytes / 1024;       // DMA instructions per wave
constexpr int kQStageArea = 4 * kQStageBytes;         // waves 0-3, after the K and V rings
constexpr int kLdsBytes = 2 * kRing * kTileBytes + kQStageArea;   // 160 KiB
// LDS tile (K slots 0 .. kRing-1, then V slots) and byte offset of a wave's rows.
// (-1: the staging area after the rings).
__host__ __device__ __forceinline__ int q_stage_tile(int base, int wave) {
  return wave < 4 ? -1 : wave < 6 ? ring_slot(base, kPrologueK) : kRing + ring_slot(base, 1);
}
__host__ __device__ __forceinline__ int q_stage_offset(int base, int wave) {
  return wave < 4 ? 2 * kRing * kTileBytes + wave * kQStageBytes
                  : q_stage_tile(base, wave) * kTileBytes + (wave & 1) * kQStageBytes;
}
// Within a wave's 8 KiB: row r (0..31) at r * 256 bytes, its 16-byte chunk c (d =
// 8c .. 8c+7) at position c ^ (r & 15), conflict-free for the fragment read (16
// rows, one chunk).  DMA instruction j (0..7) fills rows 4j .. 4j+3: lane ->
// row 4j + (lane >> 4), position lane & 15.
__host__ __device__ __forceinline__ int q_stage_pos(int r, int c) { return r * 256 + ((c ^ (r & 15)) << 4); }
__host__ __device__ __forceinline__ int q_dma_row(int j, int lane) { return 4 * j + (lane >> 4); }
__host__ __device__ __forceinline__ int q_dma_chunk(int j, int lane) { return (lane & 15) ^ (q_dma_row(j, lane) & 15); }
// The wave's DMA source: q rows w0 .. w0+31 of head q_head, rows past the sequence
// clamped to the last one (their results are never stored).  Per-lane 32-bit byte
// offsets from row min(w0, seq-1), at most 31 * Hq*D*2 + 240 (the launcher bounds Hq).
__host__ __device__ __forceinline__ int q_src_row0(const Args& p, int w0) { return imin(w0, p.seq - 1); }
__host__ __device__ __forceinline__ uint32_t q_dma_offset(const Args& p, int w0, int r, int c) {
  const int row = imin(w0 + r, p.seq - 1);
  return (uint32_t)((int64_t)(row - q_src_row0(p, w0)) * p.q_ss * 2 + c * 16);
}
// Largest Hq whose q DMA offsets fit 32 bits.
constexpr int64_t kMaxHqStaged = (0xffffffffLL - 240) / ((kWaveRows - 1) * kD * 2);

// Source row of tile row r in key tile kt: rows past the sequence (only in the
// last, partial tile) are clamped to the last key.
__host__ __device__ __forceinline__ int dma_src_row(const Args& p, int kt, int r) {
  const int j0 = kt * kBN;
  return (j0 + kBN <= p.seq) ? r : imin(r, p.seq - 1 - j0);
}

}  // namespace attn
}  // namespace kda
