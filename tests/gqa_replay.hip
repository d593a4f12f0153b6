// Host replay of the global memory accesses and the K/V ring schedule of the
// bf16 GQA forward kernel (kda_gqa_fwd_bf16, csrc/attention.hip).  It runs no GPU
// code: it walks every workgroup, block, wave and lane of a launch through the
// geometry and schedule functions the kernel computes its addresses with
// (csrc/attention_geom.h), in the kernel's own order, and checks that
//   - every q load (16 bytes) lies inside q, every K/V tile DMA source (16 bytes,
//     after the clamp of rows past the sequence) inside k or v, and every output
//     store (8 bytes) inside out;
//   - no per-lane 32-bit DMA offset wraps (it equals the exact row * row_bytes + chunk);
//   - every DMA lands inside its 16 KiB LDS tile;
//   - every block is run by exactly one workgroup (the persistent schedule), and
//     every output element is stored exactly once;
//   - the K/V ring holds the right tile whenever the kernel reads one: the tile of
//     the right block, fetched at least two iterations earlier or before a full
//     wait (vmcnt(0)), and no DMA overwrites a slot whose content is still read in
//     the same or a later iteration.  This covers the prefetch of a block's first
//     tiles by the previous block's last iterations;
//   - the next block's q rows, staged by DMA in the last iteration (global source
//     inside q, no 32-bit offset wrap, LDS inside the wave's own 8 KiB), sit in ring
//     slots that nothing reads or overwrites until the next block has read them.
// Buffers sit at fake base addresses, so only the arithmetic is exercised.
//
// usage: gqa_replay B S HQ HKV causal(0/1) layout(bshd/bhsd) [grid [mistake]]
//   grid: workgroups of the causal (persistent) launch, default min(blocks, 256)
//   mistake: replay a deliberately wrong schedule, to show the ring checks catch it:
//     1 = a block's prologue assumes all its first K tiles were prefetched,
//     2 = the K DMA of iteration kt targets the slot of tile kt+2 instead of kt+3,
//     3 = a block's prologue waits for nothing (no vmcnt(0) after its own DMAs),
//     4 = the q rows of waves 4-5 are staged in K slot base+2 instead of base+3
// prints "ok ..." and exits 0, or lists the first violations and exits 1.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "attention_geom.h"

using namespace kda::attn;

namespace {

struct Buf {
  const char* name;
  uint64_t base, bytes;
};

long g_bad = 0;

void fail(const char* what, const char* fmt, long long a, long long b, long long c) {
  if (++g_bad <= 10) {
    std::printf("VIOLATION %s: ", what);
    std::printf(fmt, a, b, c);
    std::printf("\n");
  }
}

void check(const Buf& buf, uint64_t addr, uint64_t n, int block, int wave, int lane) {
  if (addr < buf.base || addr + n > buf.base + buf.bytes)
    fail(buf.name, "block %lld wave %lld lane %lld out of bounds", block, wave, lane);
}

// One ring slot of K or V: which tile it holds and when it was fetched / last read.
struct Slot {
  int block = -1, tile = -1;
  long write_step = -1, last_read = -1;
};
constexpr int kQTile = -2;   // a slot holding staged q rows

}  // namespace

int main(int argc, char** argv) {
  if (argc < 7 || argc > 9) {
    std::fprintf(stderr, "usage: %s B S HQ HKV causal layout [grid [mistake]]\n", argv[0]);
    return 2;
  }
  const int64_t B = std::atoll(argv[1]), S = std::atoll(argv[2]), HQ = std::atoll(argv[3]),
                HKV = std::atoll(argv[4]);
  const bool causal = std::atoi(argv[5]) != 0;
  const bool bhsd = std::strcmp(argv[6], "bhsd") == 0;
  const Buf q{"q", 1ull << 44, (uint64_t)(B * S * HQ * kD * 2)};
  const Buf k{"k", 2ull << 44, (uint64_t)(B * S * HKV * kD * 2)};
  const Buf v{"v", 3ull << 44, (uint64_t)(B * S * HKV * kD * 2)};
  const Buf o{"out", 4ull << 44, (uint64_t)(B * S * HQ * kD * 2)};
  // output strides as kda.ops passes them: BSHD [B][S][Hq][D] or BHSD [B][Hq][S][D]
  const int64_t o_sb = S * HQ * kD, o_ss = bhsd ? kD : HQ * kD, o_sh = bhsd ? S * kD : kD;
  const Args p = make_args(reinterpret_cast<const uint16_t*>(q.base), reinterpret_cast<const uint16_t*>(k.base),
                           reinterpret_cast<const uint16_t*>(v.base), reinterpret_cast<uint16_t*>(o.base), B, S,
                           HQ, HKV, 0.088f, o_sb, o_ss, o_sh);
  const int hpw = heads_per_workgroup(HQ / HKV);
  const int64_t nblocks = grid_blocks(B, S, HQ, HKV);
  if (nblocks != total_blocks(p, hpw)) fail("blocks", "grid_blocks %lld != total_blocks %lld%lld", nblocks, total_blocks(p, hpw), 0);
  // the launcher: causal runs min(blocks, CUs) persistent workgroups, non-causal one per block
  int64_t grid = causal ? (nblocks < 256 ? nblocks : 256) : nblocks;
  if (argc >= 8 && causal && std::atoll(argv[7]) > 0) grid = std::atoll(argv[7]);
  const int mistake = argc == 9 ? std::atoi(argv[8]) : 0;
  std::vector<uint8_t> written((size_t)(B * S * HQ * kD / 4), 0);   // per 4-element store
  std::vector<uint8_t> ran((size_t)nblocks, 0);
  const int64_t row_bytes = p.k_ss * 2;
  long long n_q = 0, n_dma = 0, n_st = 0, n_reads = 0, n_qdma = 0;

  // global source checks of one DMA (all lanes of the issuing waves)
  auto dma = [&](int bid, bool is_v, int kt) {
    const Buf& buf = is_v ? v : k;
    for (int wave = 0; wave < kDmaWaves; ++wave) {
      const Block g = block_of(p, causal, hpw, bid, wave);
      if (kt < 0 || kt >= g.nkt) fail("schedule", "tile %lld outside 0..%lld (block %lld)", kt, g.nkt - 1, bid);
      const uint64_t tile_base = buf.base + 2 * (uint64_t)kv_head(p, g) + (uint64_t)kt * kBN * row_bytes;
      for (int j = 0; j < kDmaPerWave; ++j)
        for (int lane = 0; lane < 64; ++lane) {
          const int r = dma_row(j, wave, lane);
          const int src = dma_src_row(p, kt, r);
          const uint32_t col = is_v ? dma_vcol(r, lane) : dma_kcol(r, lane);
          const uint32_t off = dma_lane_offset(row_bytes, src, col);
          if ((int64_t)off != src * row_bytes + col)
            fail("dma offset", "32-bit offset wraps: row %lld row_bytes %lld block %lld", src, row_bytes, bid);
          check(buf, tile_base + off, 16, bid, wave, lane);
          const int64_t lds = (int64_t)(j * kDmaWaves + wave) * 1024 + 16 * lane;
          if (lds < 0 || lds + 16 > kTileBytes) fail("lds", "DMA lands at %lld (wave %lld lane %lld)", lds, wave, lane);
          ++n_dma;
        }
    }
  };

  for (int64_t w = 0; w < grid; ++w) {
    Slot ring[2][kRing];            // [K, V][slot]
    long full_wait = -1;            // step of the last vmcnt(0): every earlier write has landed
    long step = 0;
    int slot_base = 0, prev_nkt = 0;
    auto write = [&](int kind, int slot, int bid, int tile) {
      Slot& s = ring[kind][slot];
      if (s.last_read >= step)
        fail("ring", "slot %lld overwritten in step %lld while read in step %lld", slot, step, s.last_read);
      s = Slot{bid, tile, step, -1};
      dma(bid, kind == 1, tile);
    };
    auto read = [&](int kind, int slot, int bid, int tile) {
      Slot& s = ring[kind][slot];
      if (s.block != bid || s.tile != tile)
        fail("ring", "step %lld reads tile %lld of block %lld but the slot holds another tile", step, tile, bid);
      if (!(s.write_step + 2 <= step || s.write_step <= full_wait))
        fail("ring", "step %lld reads a tile fetched in step %lld (not yet landed, block %lld)", step, s.write_step, bid);
      s.last_read = step;
      ++n_reads;
    };
    // the next block's q rows: DMA sources and LDS ranges of every wave, and the
    // two ring slots they occupy (waves 4-5: K slot base+3, waves 6-7: V slot base+1)
    auto stage = [&](int bid_n, int base_n) {
      for (int wave = 0; wave < kWaves; ++wave) {
        const Block g = block_of(p, causal, hpw, bid_n, wave);
        const uint64_t src0 = q.base + 2 * (uint64_t)(q_head(p, g) + (int64_t)q_src_row0(p, g.w0) * p.q_ss);
        const int off = q_stage_offset(base_n, wave);
        if (off < 0 || off + kQStageBytes > kLdsBytes || (wave < 4) != (q_stage_tile(base_n, wave) < 0))
          fail("q stage", "wave %lld staged at LDS %lld (block %lld)", wave, off, bid_n);
        for (int j = 0; j < kQStageDma; ++j)
          for (int lane = 0; lane < 64; ++lane) {
            const int r = q_dma_row(j, lane), c = q_dma_chunk(j, lane);
            const int row = imin(g.w0 + r, p.seq - 1);
            const int64_t exact = (int64_t)(row - q_src_row0(p, g.w0)) * p.q_ss * 2 + c * 16;
            const uint32_t o32 = q_dma_offset(p, g.w0, r, c);
            if ((int64_t)o32 != exact) fail("q stage", "32-bit offset wraps: wave %lld row %lld block %lld", wave, row, bid_n);
            check(q, src0 + o32, 16, bid_n, wave, lane);
            if (j * 1024 + 16 * lane != q_stage_pos(r, c))   // where the fragment read looks for it
              fail("q stage", "lane %lld lands where the read does not look (wave %lld, block %lld)", lane, wave, bid_n);
            ++n_qdma;
          }
      }
      for (int wave = 4; wave < kWaves; wave += 2) {
        const int t = q_stage_tile(base_n, wave);
        const int kind = t >= kRing;
        const int slot = mistake == 4 && wave < 6 ? ring_slot(base_n, 2) : t % kRing;
        Slot& sl = ring[kind][slot];
        if (sl.last_read >= step)
          fail("q stage", "slot %lld staged in step %lld while read in step %lld", slot, step, sl.last_read);
        sl = Slot{bid_n, kQTile, step, -1};
      }
    };
    for (int kk = 0;; ++kk) {
      if (!causal && kk > 0) break;
      const int bid = causal ? sched_block(kk, (int)w, (int)grid) : (int)w;
      if (bid >= nblocks) break;
      if (ran[bid]++) fail("schedule", "block %lld run twice (workgroup %lld)%lld", bid, w, 0);
      const int bid_next = causal ? sched_block(kk + 1, (int)w, (int)grid) : (int)nblocks;
      const bool has_next = causal && bid_next < nblocks;
      const Block g0 = block_of(p, causal, hpw, bid, 0);
      const Block gn = block_of(p, causal, hpw, has_next ? bid_next : bid, 0);
      const int nkt = g0.nkt;
      // q loads (a workgroup's first block; later ones read q staged in LDS) and
      // output stores of every wave
      for (int wave = 0; wave < kWaves; ++wave) {
        const Block g = block_of(p, causal, hpw, bid, wave);
        for (int lane = 0; lane < 64; ++lane)
          for (int it = 0; it < kWaveRows / 16; ++it) {
            const int row = g.w0 + it * 16 + (lane & 15);
            if (row >= p.seq) continue;
            for (int dc = 0; dc < 4 && (!causal || kk == 0); ++dc) {
              check(q, q.base + 2 * (uint64_t)(q_head(p, g) + q_elem(p, row, dc, lane >> 4)), 16, bid, wave, lane);
              ++n_q;
            }
            for (int dt = 0; dt < kD / 16; ++dt) {
              const int64_t e = out_head(p, g) + out_elem(p, row, dt, lane >> 4);
              check(o, o.base + 2 * (uint64_t)e, 8, bid, wave, lane);
              if (e % 4 == 0 && e >= 0 && e / 4 < (int64_t)written.size()) ++written[(size_t)(e / 4)];
              else fail("store", "element %lld not a 4-aligned output index (block %lld wave %lld)", e, bid, wave);
              ++n_st;
            }
          }
        if (g.nkt != nkt) fail("schedule", "waves of block %lld disagree on its tile count%lld%lld", bid, 0, 0);
      }
      // staged q rows read at the top of every block after a workgroup's first
      if (causal && kk > 0) {
        for (int wave = 4; wave < kWaves; wave += 2) {
          const int t = q_stage_tile(slot_base, wave);
          const int kind = t >= kRing, slot = t % kRing;
          Slot& sl = ring[kind][mistake == 4 && wave < 6 ? ring_slot(slot_base, 2) : slot];
          if (sl.block != bid || sl.tile != kQTile)
            fail("q stage", "block %lld wave %lld reads q rows that are not in slot %lld", bid, wave, slot);
          sl.last_read = step;
        }
      }
      // prologue: the first tiles the previous block did not prefetch, a full
      // wait unless all were prefetched, then S(0) reads K(0)
      for (int i = 0; i < kPrologueK; ++i)
        if (!(prologue_k_prefetched(i, prev_nkt) || (mistake == 1 && prev_nkt > 0)))
          write(0, ring_slot(slot_base, i), bid, prologue_k_tile(i, nkt));
      if (!prologue_v_prefetched(prev_nkt)) write(1, ring_slot(slot_base, 0), bid, 0);
      if (mistake != 3 && !prologue_all_prefetched(prev_nkt)) full_wait = step;
      read(0, ring_slot(slot_base, 0), bid, 0);
      // iterations kt = 0 .. nkt-1 (one step each), then the last O += V P
      for (int kt = 0; kt < nkt; ++kt) {
        ++step;
        const Fetch kf = k_fetch(kt, nkt, has_next, gn.nkt);
        const Fetch vf = v_fetch(kt, nkt, has_next);
        write(0, ring_slot(slot_base, kt + (mistake == 2 ? kPrologueK - 1 : kPrologueK)), kf.next ? bid_next : bid,
              kf.tile);
        write(1, ring_slot(slot_base, kt + 1), vf.next ? bid_next : bid, vf.tile);
        if (kt == nkt - 1 && has_next) stage(bid_next, ring_slot(slot_base, nkt));
        if (kt >= 1) read(1, ring_slot(slot_base, kt - 1), bid, kt - 1);   // O += V(kt-1) P(kt-1)
        if (kt + 1 < nkt) read(0, ring_slot(slot_base, kt + 1), bid, kt + 1);   // S(kt+1)
      }
      ++step;
      read(1, ring_slot(slot_base, nkt - 1), bid, nkt - 1);
      full_wait = step;   // every ring DMA has landed before the stores
      ++step;
      slot_base = ring_slot(slot_base, nkt);
      prev_nkt = nkt;
    }
  }
  for (int64_t b = 0; b < nblocks; ++b)
    if (ran[(size_t)b] != 1) fail("schedule", "block %lld run %lld times%lld", b, ran[(size_t)b], 0);
  long long never = 0, twice = 0;
  for (uint8_t x : written) never += (x == 0), twice += (x > 1);
  if (never || twice) fail("coverage", "%lld output groups never stored, %lld stored more than once (%lld)", never, twice, 0);
  if (g_bad) {
    std::printf("FAIL %ld violations\n", g_bad);
    return 1;
  }
  std::printf("ok blocks=%lld grid=%lld q_loads=%lld q_dmas=%lld dmas=%lld ring_reads=%lld stores=%lld\n",
              (long long)nblocks, (long long)grid, n_q, n_qdma, n_dma, n_reads, n_st);
  return 0;
}
