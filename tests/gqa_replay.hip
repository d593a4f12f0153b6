// Host replay of the global memory accesses of the bf16 GQA forward kernel
// (kda_gqa_fwd_bf16, csrc/attention.hip).  It runs no GPU code: it walks every
// workgroup, wave and lane of a launch through the geometry functions the kernel
// computes its addresses with (csrc/attention_geom.h), in the kernel's own
// schedule, and checks that
//   - every q load (16 bytes) lies inside q, every K/V tile DMA source (16 bytes,
//     after the clamp of rows past the sequence) inside k or v, and every output
//     store (8 bytes) inside out;
//   - no per-lane 32-bit DMA offset wraps (it equals the exact row * row_bytes + chunk);
//   - every DMA lands inside its 16 KiB LDS tile;
//   - every output element is stored exactly once.
// Buffers sit at fake base addresses, so only the arithmetic is exercised.
//
// usage: gqa_replay B S HQ HKV causal(0/1) layout(bshd/bhsd)
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

}  // namespace

int main(int argc, char** argv) {
  if (argc != 7) {
    std::fprintf(stderr, "usage: %s B S HQ HKV causal layout\n", argv[0]);
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
  std::vector<uint8_t> written((size_t)(B * S * HQ * kD / 4), 0);   // per 4-element store
  const int64_t row_bytes = p.k_ss * 2;
  long long n_q = 0, n_dma = 0, n_st = 0;

  for (int blk = 0; blk < nblocks; ++blk) {
    for (int wave = 0; wave < kWaves; ++wave) {
      const Block g = block_of(p, causal, hpw, blk, wave);
      // q fragments: rows w0 + it*16 + l16, d chunks dc, lane group g4 = lane >> 4
      for (int lane = 0; lane < 64; ++lane)
        for (int it = 0; it < kWaveRows / 16; ++it) {
          const int row = g.w0 + it * 16 + (lane & 15);
          if (row >= p.seq) continue;
          for (int dc = 0; dc < 4; ++dc) {
            check(q, q.base + 2 * (uint64_t)(q_head(p, g) + q_elem(p, row, dc, lane >> 4)), 16, blk, wave, lane);
            ++n_q;
          }
        }
      // K/V tile DMAs in the kernel's order (waves below kDmaWaves issue them)
      if (wave < kDmaWaves) {
        std::vector<std::pair<int, bool>> tiles;   // (key tile, is V)
        for (int i = 0; i < kPrologueK; ++i) tiles.push_back({prologue_k_tile(i, g.nkt), false});
        tiles.push_back({0, true});
        for (int kt = 0; kt < g.nkt; ++kt) {
          tiles.push_back({k_fetch_tile(kt, g.nkt), false});
          tiles.push_back({v_fetch_tile(kt, g.nkt), true});
        }
        for (const auto& tv : tiles) {
          const int kt = tv.first;
          const bool is_v = tv.second;
          if (kt < 0 || kt >= g.nkt) fail("schedule", "tile %lld outside 0..%lld (block %lld)", kt, g.nkt - 1, blk);
          const Buf& buf = is_v ? v : k;
          const uint64_t tile_base = buf.base + 2 * (uint64_t)kv_head(p, g) + (uint64_t)kt * kBN * row_bytes;
          for (int j = 0; j < kDmaPerWave; ++j)
            for (int lane = 0; lane < 64; ++lane) {
              const int r = dma_row(j, wave, lane);
              const int src = dma_src_row(p, kt, r);
              const uint32_t col = is_v ? dma_vcol(r, lane) : dma_kcol(r, lane);
              const uint32_t off = dma_lane_offset(row_bytes, src, col);
              if ((int64_t)off != src * row_bytes + col)
                fail("dma offset", "32-bit offset wraps: row %lld row_bytes %lld block %lld", src, row_bytes, blk);
              check(buf, tile_base + off, 16, blk, wave, lane);
              const int64_t lds = (int64_t)(j * kDmaWaves + wave) * 1024 + 16 * lane;
              if (lds < 0 || lds + 16 > kTileBytes) fail("lds", "DMA lands at %lld (wave %lld lane %lld)", lds, wave, lane);
              ++n_dma;
            }
        }
      }
      // output stores: rows w0 + it*16 + l16, d tiles dt
      for (int lane = 0; lane < 64; ++lane)
        for (int it = 0; it < kWaveRows / 16; ++it) {
          const int row = g.w0 + it * 16 + (lane & 15);
          if (row >= p.seq) continue;
          for (int dt = 0; dt < kD / 16; ++dt) {
            const int64_t e = out_head(p, g) + out_elem(p, row, dt, lane >> 4);
            check(o, o.base + 2 * (uint64_t)e, 8, blk, wave, lane);
            if (e % 4 == 0 && e >= 0 && e / 4 < (int64_t)written.size()) ++written[(size_t)(e / 4)];
            else fail("store", "element %lld not a 4-aligned output index (block %lld wave %lld)", e, blk, wave);
            ++n_st;
          }
        }
    }
  }
  long long never = 0, twice = 0;
  for (uint8_t w : written) never += (w == 0), twice += (w > 1);
  if (never || twice) fail("coverage", "%lld output groups never stored, %lld stored more than once (%lld)", never, twice, 0);
  if (g_bad) {
    std::printf("FAIL %ld violations\n", g_bad);
    return 1;
  }
  std::printf("ok blocks=%lld q_loads=%lld dmas=%lld stores=%lld\n", (long long)nblocks, n_q, n_dma, n_st);
  return 0;
}
