// zs_rdecode.hpp -- decoder of the CDNA4 re-tiled layout (gfx950).
//
// Layout (one record per 16 x 64 tile; record r = band * K/64 + kt):
//   fixed part, 1408 B:
//     [16*l .. 16*l+15]   sign|mantissa bytes of lane l: half 0 elements 0..7,
//                         then half 1 elements 0..7 (every element, outliers too)
//     [1024 + 4*l]        u32  B1(0,l) | B2(0,l) << 8 | B3(0,l) << 16 | B1(1,l) << 24
//     [1280 + 2*l]        u16  B2(1,l) | B3(1,l) << 8
//   Bp(h,l) bit i is bit p-1 of the 3-bit code of element (h, l, i):
//   0 = outlier, c = 1..7 -> exponent (start_exp + c) mod 256.
//   exponent stream: per outlier, in (h, l, i) order, the byte
//   (exponent - start_exp) mod 256, starting at exps[eoff[r]].
// Element (h, l, i) is matrix row 16*band + l%16, column 64*kt + 32*h +
// 8*(l/16) + i: lane l of half h is exactly lane l's A operand of
// v_mfma_f32_16x16x32_bf16 for the 32 columns of that half.
//
// Decode of one half for lane l (8 bf16 in 4 dwords, element 2d in the low
// half of dword d):
//   x   = E1[b1] + E2[b2] + E3[b3]         start + code per halfword (bits 0..9)
//   ep  = v_perm(window, OSEL[ind])        outlier byte k under outlier k, else 0
//   xe  = (x + ep) << 7                    exponent field at bits 7..14 (mod 256:
//                                          higher bits land under the mask below)
//   out = v_bfi(0x807F807F, v_perm(sm, K_d), xe)
// where ind = b1|b2|b3 and the lane's outlier bytes start at a wave prefix sum
// of popcount(~ind) (both halves scanned at once, 16 bits each).
#pragma once
#include "zs_device.hpp"

namespace zs {

constexpr int kRecBytes = 1408;
constexpr int kRecP32 = 1024;
constexpr int kRecP16 = 1280;
constexpr int kExpChunks = 16;                     // staged exponent chunks per record
constexpr int kExpStage = kExpChunks * 16 + 32;    // + window-read slack

struct RTables {
  uint4 e1[256];    // (start + bit) per halfword field, start_exp dependent
  uint4 e2[256];    // bit << 1
  uint4 e3[256];    // bit << 2
  uint4 osel[256];  // v_perm selectors of the outlier bytes (by ind)
};

__device__ __forceinline__ void build_r_e1(uint4* e1, int start_exp, int tid, int nthreads) {
  const uint32_t st = (uint32_t)start_exp & 0xFFu;
  for (int v = tid; v < 256; v += nthreads) {
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; ++d)
      w[d] = (st + ((v >> (2 * d)) & 1)) | ((st + ((v >> (2 * d + 1)) & 1)) << 16);
    e1[v] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

__device__ __forceinline__ void build_r_tables(RTables& T, int start_exp, int tid, int nthreads) {
  build_r_e1(T.e1, start_exp, tid, nthreads);
  for (int v = tid; v < 256; v += nthreads) {
    uint32_t e2[4], e3[4], os[4];
    uint32_t rank[8];
    uint32_t k = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      rank[j] = k;
      k += ((v >> j) & 1) ? 0u : 1u;
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t lo = (v >> (2 * d)) & 1, hi = (v >> (2 * d + 1)) & 1;
      e2[d] = (lo << 1) | (hi << 17);
      e3[d] = (lo << 2) | (hi << 18);
      const uint32_t slo = lo ? 0x0Cu : rank[2 * d], shi = hi ? 0x0Cu : rank[2 * d + 1];
      os[d] = slo | (0x0Cu << 8) | (shi << 16) | (0x0Cu << 24);
    }
    T.e2[v] = make_uint4(e2[0], e2[1], e2[2], e2[3]);
    T.e3[v] = make_uint4(e3[0], e3[1], e3[2], e3[3]);
    T.osel[v] = make_uint4(os[0], os[1], os[2], os[3]);
  }
}

// One record's per-lane inputs (registers).
struct RecRegs {
  u32x4 sm;      // sign|mantissa bytes, half 0 in .x/.y, half 1 in .z/.w
  uint32_t p32;  // plane bytes (see header)
  uint32_t p16;
};

// Byte selectors placing sign|mantissa byte 2d / 2d+1 under both bytes of
// halfword 0 / 1 of dword d.
__device__ __forceinline__ uint32_t sm_sel(int d) {
  return (uint32_t)(2 * d) * 0x0101u + (uint32_t)(2 * d + 1) * 0x01010000u;
}

__device__ __forceinline__ u32x4 r_half(const RTables& T, const uint4* e1, uint32_t b1,
                                        uint32_t b2, uint32_t b3, uint32_t s0, uint32_t s1,
                                        uint32_t w0, uint32_t w1) {
  const uint32_t ind = b1 | b2 | b3;
  const uint4 x1 = e1[b1], x2 = T.e2[b2], x3 = T.e3[b3], os = T.osel[ind];
  const uint32_t msk = 0x807F807Fu;
  u32x4 o;
  o[0] = __builtin_amdgcn_perm(s1, s0, sm_sel(0));
  o[1] = __builtin_amdgcn_perm(s1, s0, sm_sel(1));
  o[2] = __builtin_amdgcn_perm(s1, s0, sm_sel(2));
  o[3] = __builtin_amdgcn_perm(s1, s0, sm_sel(3));
  const uint32_t xe0 = (x1.x + x2.x + x3.x + __builtin_amdgcn_perm(w1, w0, os.x)) << 7;
  const uint32_t xe1 = (x1.y + x2.y + x3.y + __builtin_amdgcn_perm(w1, w0, os.y)) << 7;
  const uint32_t xe2 = (x1.z + x2.z + x3.z + __builtin_amdgcn_perm(w1, w0, os.z)) << 7;
  const uint32_t xe3 = (x1.w + x2.w + x3.w + __builtin_amdgcn_perm(w1, w0, os.w)) << 7;
  o[0] = (o[0] & msk) | (xe0 & ~msk);
  o[1] = (o[1] & msk) | (xe1 & ~msk);
  o[2] = (o[2] & msk) | (xe2 & ~msk);
  o[3] = (o[3] & msk) | (xe3 & ~msk);
  return o;
}

// Per-lane outlier ranks of both halves (wave prefix sums of popcount(~ind)
// packed 16 bits per half).  rank0/rank1 = first outlier byte of the lane's
// half 0 / half 1 relative to the record's first one.
__device__ __forceinline__ void r_ranks(uint32_t p32, uint32_t p16, int& rank0, int& rank1) {
  const uint32_t ind0 = (p32 | (p32 >> 8) | (p32 >> 16)) & 0xFFu;
  const uint32_t ind1 = ((p32 >> 24) | p16 | (p16 >> 8)) & 0xFFu;
  const int n = (8 - __builtin_popcount(ind0)) | ((8 - __builtin_popcount(ind1)) << 16);
  const int incl = wave_inclusive_scan(n);
  const int excl = incl - n;
  const int tot0 = __builtin_amdgcn_readlane(incl, 63) & 0xFFFF;
  rank0 = excl & 0xFFFF;
  rank1 = tot0 + (excl >> 16);
}

// Reads the 8 outlier bytes starting at byte `off` of `base` (3 aligned
// dwords + v_alignbyte).  `base` is LDS or global memory with >= 12 readable
// bytes past off & ~3.
template <typename P>
__device__ __forceinline__ void r_window(P base, int off, uint32_t& w0, uint32_t& w1) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(base + (off & ~3));
  const uint32_t q0 = q[0], q1 = q[1], q2 = q[2];
  const uint32_t sh = (uint32_t)(off & 3);
  w0 = __builtin_amdgcn_alignbyte(q1, q0, sh);
  w1 = __builtin_amdgcn_alignbyte(q2, q1, sh);
}

// Decodes one record into the two MFMA A operands (half 0, half 1).  `exb`
// holds the record's outlier bytes, the first one at byte `rel`.
template <typename P>
__device__ __forceinline__ void r_decode(const RTables& T, const uint4* e1, const RecRegs& r,
                                         P exb, int rel, u32x4& o0, u32x4& o1) {
  int rank0, rank1;
  r_ranks(r.p32, r.p16, rank0, rank1);
  uint32_t a0, a1, c0, c1;
  r_window(exb, rel + rank0, a0, a1);
  r_window(exb, rel + rank1, c0, c1);
  o0 = r_half(T, e1, r.p32 & 0xFFu, (r.p32 >> 8) & 0xFFu, (r.p32 >> 16) & 0xFFu, r.sm[0], r.sm[1],
              a0, a1);
  o1 = r_half(T, e1, r.p32 >> 24, r.p16 & 0xFFu, (r.p16 >> 8) & 0xFFu, r.sm[2], r.sm[3], c0, c1);
}

// ---------------------------------------------------------------------------
// Record fetch: the fixed part straight into registers, the outlier bytes as
// up to kExpWords dwords (lane l: dword l, 4 bytes per lane so the load
// returns 256 B, not 1 KB) bound for a wave-private LDS stage.  A record with
// more outlier bytes than that (over ~24% outliers) is decoded with its
// outlier windows read from global memory.
// ---------------------------------------------------------------------------
constexpr int kExpWords = kExpChunks * 4;

struct RStage {
  RecRegs r;
  uint32_t ex;
};
struct RMeta {
  int e0;   // first outlier byte of the record (stream offset)
  int rel;  // e0 - first staged byte
  int nw;   // staged dwords (> kExpWords: decode from global memory)
};

__device__ __forceinline__ bool r_staged(const RMeta& mt) { return mt.nw <= kExpWords; }

// Fixed part of record `rec` (no dependency on the outlier offsets).
__device__ __forceinline__ void r_issue_fixed(const uint8_t* fixed, int64_t rec, RStage& s) {
  const int l = lane_id();
  const uint8_t* f = fixed + rec * kRecBytes;
  s.r.sm = *reinterpret_cast<const u32x4*>(f + 16 * l);
  s.r.p32 = *reinterpret_cast<const uint32_t*>(f + kRecP32 + 4 * l);
  s.r.p16 = *reinterpret_cast<const uint16_t*>(f + kRecP16 + 2 * l);
}

// Outlier bytes [e0, e1) of a record, as dwords from e0 & ~3.
__device__ __forceinline__ void r_issue_exps(const uint8_t* exps, int e0, int e1, RStage& s,
                                             RMeta& mt) {
  const int l = lane_id();
  const int ea0 = e0 & ~3;
  const int nw = (e1 - ea0 + 3) >> 2;
  mt.e0 = e0;
  mt.rel = e0 - ea0;
  mt.nw = nw;
  s.ex = *reinterpret_cast<const uint32_t*>(exps + ea0 + (l < nw ? 4 * l : 0));
}

__device__ __forceinline__ void r_issue(const uint8_t* fixed, const uint8_t* exps, int64_t rec,
                                        int e0, int e1, RStage& s, RMeta& mt) {
  r_issue_fixed(fixed, rec, s);
  r_issue_exps(exps, e0, e1, s, mt);
}

// Records whose outlier bytes exceed the stage are decoded from global memory
// and are not staged (the stage holds kExpWords dwords).
__device__ __forceinline__ void r_stage(uint8_t* st, const RStage& s, const RMeta& mt) {
  const int l = lane_id();
  if (r_staged(mt) && l < mt.nw) *reinterpret_cast<uint32_t*>(st + 4 * l) = s.ex;
}

__device__ __forceinline__ void r_decode_staged(const RTables& T, const RStage& s,
                                                const RMeta& mt, const uint8_t* st,
                                                const uint8_t* exps, u32x4& o0, u32x4& o1) {
  if (r_staged(mt))
    r_decode(T, T.e1, s.r, st, mt.rel, o0, o1);
  else
    r_decode(T, T.e1, s.r, exps + mt.e0, 0, o0, o1);
}

}  // namespace zs
