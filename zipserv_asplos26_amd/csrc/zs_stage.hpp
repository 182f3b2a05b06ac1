// zs_stage.hpp -- per-wave LDS staging of one median tile (gfx950).
//
// A median tile (16 x 64 elements) is copied from the compressed streams into
// a wave-private LDS stage with exactly two 16-byte loads per lane: its three
// bitmap planes (3 x 128 B), its SM bytes from the 16-byte-aligned start, and
// up to kFullChunks x 8 of its FULL elements from the 8-aligned start.  The
// decode then reads everything from LDS (decode_median_pair in zs_device.hpp).
#pragma once
#include "zs_device.hpp"

namespace zs {

constexpr int kStBm = 0;                     // 3 x 128 B bitmap planes
constexpr int kStSm = 384;                   // SM bytes from the 16-aligned start
constexpr int kStSmBytes = 1056;             // 65 chunks used + read-window slack
constexpr int kStFull = kStSm + kStSmBytes;  // FULL elements from the 8-aligned start
constexpr int kFullChunks = 33;              // staged outliers: up to 264 per median tile
constexpr int kStBytes = kStFull + kFullChunks * 16 + 16;  // + window-read slack

struct StageRegs {
  u32x4 sm;    // SM chunk l (16 bytes) of the median tile
  u32x4 misc;  // lanes 0..23 bitmap chunks, 24..56 FULL chunks, 57 SM chunk 64
};
struct StageMeta {
  int sm_rel;    // first SM byte of the median tile relative to the stage copy
  int full_rel;  // first FULL element relative to the stage copy
  int fa0;       // stream offset of the stage copy's first FULL element
  int full_direct;  // outliers did not fit the stage: read them from global
};

// Stream offsets of one median tile: first SM byte, first FULL element, and
// the first ones after it (the next median tile's start, or the next global
// tile's padded start for the last median tile).
struct TileOff {
  int hf0, f0, hf1, f1;
};

// Vector-loads the offsets of up to 64 median tiles (lane i -> tile i) so the
// pipeline reads them with readlane instead of waiting on scalar loads.
__device__ __forceinline__ TileOff load_tile_offsets(const Streams& s, int g, int m, bool valid) {
  TileOff t{0, 0, 0, 0};
  if (valid) {
    const int t0 = s.tog[2 * g], tf0 = s.tog[2 * g + 1];
    const int mb = 2 * (4 * g + m);
    t.hf0 = t0 + s.tom[mb];
    t.f0 = tf0 + s.tom[mb + 1];
    if (m < 3) {
      t.hf1 = t0 + s.tom[mb + 2];
      t.f1 = tf0 + s.tom[mb + 3];
    } else {
      t.hf1 = s.tog[2 * g + 2];
      t.f1 = s.tog[2 * g + 3];
    }
  }
  return t;
}

__device__ __forceinline__ TileOff tile_off_at(const TileOff& v, int i) {
  TileOff t;
  t.hf0 = __builtin_amdgcn_readlane(v.hf0, i);
  t.f0 = __builtin_amdgcn_readlane(v.f0, i);
  t.hf1 = __builtin_amdgcn_readlane(v.hf1, i);
  t.f1 = __builtin_amdgcn_readlane(v.f1, i);
  return t;
}

// Stream offsets of median tile m of global tile g (both wave-uniform), read
// through the scalar cache: first SM byte and FULL element of the median tile
// and of the one after it (the tables of csrc/L_API.cu:356-357, :505-506 and
// :541-549: TileOffsets_Global holds one more entry than there are tiles).
__device__ __forceinline__ TileOff med_offsets_s(const Streams& s, int g, int m) {
  using ci32 = const __attribute__((address_space(4))) int32_t;
  ci32* tg = (ci32*)(s.tog + 2 * (int64_t)g);
  ci32* tm = (ci32*)(s.tom + 8 * (int64_t)g + 2 * m);
  const int t0 = tg[0], tf0 = tg[1];
  TileOff t;
  t.hf0 = t0 + tm[0];
  t.f0 = tf0 + tm[1];
  if (m < 3) {
    t.hf1 = t0 + tm[2];
    t.f1 = tf0 + tm[3];
  } else {
    t.hf1 = tg[2];
    t.f1 = tg[3];
  }
  return t;
}

// `bm_lane` is this lane's bitmap plane (lanes 0-7: plane 1, 8-15: plane 2,
// 16-23: plane 3), chosen once per kernel.
__device__ __forceinline__ void stage_issue(const Streams& s, const uint8_t* bm_lane, int g, int m,
                                            const TileOff& o, StageRegs& r, StageMeta& mt) {
  const int l = lane_id();
  const int a0 = o.hf0 & ~15;
  const int nch = min((o.hf1 - a0 + 15) >> 4, 65);
  const int fa0 = o.f0 & ~7;
  const int nfc = (o.f1 - fa0 + 7) >> 3;
  mt.sm_rel = o.hf0 - a0;
  mt.full_rel = o.f0 - fa0;
  mt.fa0 = fa0;
  mt.full_direct = nfc > kFullChunks;
  // Every lane issues exactly two 16-byte loads (addresses clamped to valid
  // data when the lane has nothing to fetch) so the number of loads in flight
  // is the same on every path and the waits stay precise.
  // Lane roles: lanes 24..56 take FULL chunk l - 24 when it exists and the
  // outliers fit, lanes 57..63 SM chunk 64 when the median tile has one;
  // every other lane re-reads its bitmap chunk.
  r.sm = *reinterpret_cast<const u32x4*>(s.sm + a0 + (l < nch ? 16 * l : 0));
  const int fi = l - 24;
  const bool full_lane = fi >= 0 && fi < kFullChunks && fi < nfc && nfc <= kFullChunks;
  const bool sm_lane = fi >= kFullChunks && nch > 64;
  const uint8_t* mp = bm_lane + 512 * g + 128 * m + 16 * (l & 7);
  mp = full_lane ? reinterpret_cast<const uint8_t*>(s.full + fa0) + 16 * fi
                 : (sm_lane ? s.sm + a0 + 1024 : mp);
  r.misc = *reinterpret_cast<const u32x4*>(mp);
}

// Every lane writes its misc chunk: lanes 0..23 the bitmap planes, 24..56 the
// FULL chunks, 57..63 the same SM chunk 64 (identical data when it exists;
// otherwise bytes past the median tile's SM bytes, which no decode selects).
// FULL chunks past the tile's outliers hold bitmap bytes, also never selected.
__device__ __forceinline__ void stage_write(uint8_t* st, const StageRegs& r) {
  const int l = lane_id();
  *reinterpret_cast<u32x4*>(st + kStSm + 16 * l) = r.sm;
  const int dst = l < 24 ? kStBm + 16 * l
                         : (l < 24 + kFullChunks ? kStFull + 16 * (l - 24) : kStSm + 1024);
  *reinterpret_cast<u32x4*>(st + dst) = r.misc;
}

}  // namespace zs
