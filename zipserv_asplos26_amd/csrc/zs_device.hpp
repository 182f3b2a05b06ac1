// zs_device.hpp -- gfx950 device building blocks shared by the ZipServ kernels.
//
// The canonical TCA-TBE stream order of one half median tile (16 rows x 32
// columns = eight 8x8 small tiles) is: small tile s = 2*colblock + rowblock,
// row-major inside each small tile (csrc/L_API.cu:403-428).  Numbering the 64
// small-tile rows of a half median tile in that order gives, for row index l:
//     matrix row  = l % 16,      columns = 8*(l/16) .. 8*(l/16)+7,
// which is exactly the A-operand lane map of v_mfma_f32_16x16x32_bf16
// (lane l holds row l%16 and eight consecutive k at 8*(l/16)).  So each lane
// of a wave64 decodes "its" small-tile row straight into the four A registers
// of one MFMA: the bitmap bytes of lane l sit at byte l of a 64-byte run of
// each bitmap array, and the lane's SM / FULL stream offsets are a wave
// exclusive prefix sum of the per-row in-window counts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zs {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Histogram slices of the one-pass re-tiled encoder (zs_retiled.hip writes
// them, zs_encode.hip's window check sums them).
constexpr int kVerifySlices = 16;

// LDS lookup tables used by the row decoder.  e1 is indexed by the plane-1
// bitmap byte (8 positions of a small-tile row); each entry is four dwords =
// eight 16-bit lanes, lane j for position j:
//   e1[v] lane j = (start_exp + bit_j(v)) << 7
// e23 covers planes 2 and 3 of four positions at once: indexed by a nibble
// of each, u = n2 | n3 << 4, entry = two dwords, lane j (0..3) =
//   (bit_j(n2) + 2 bit_j(n3)) << 8
// so e1[b1] + (e23[lo(b2) | lo(b3) << 4], e23[hi(b2) | hi(b3) << 4]) =
// (start_exp + code_j) << 7 = the exponent field (two 8-byte reads instead of
// two 16-byte ones, from a 2 KB table).
// Indexed by the in-window mask v = b1|b2|b3:
//   sel[v]  dword d = v_perm selector bytes [r_2d, r_2d, r_2d+1, r_2d+1],
//           r_j = set bits of v below j (rank of position j in the SM window);
//   osel[v] dword d = v_perm selector bytes picking outlier k_j = j - r_j from
//           a 4-value FULL window (bytes 2k, 2k+1), for the outlier lanes;
//   omsk[v] dword d = 0xFFFF in the 16-bit lanes that are outliers.
struct DecodeTables {
  uint4 e1[256];
  uint4 sel[256];
  uint4 osel[256];
  uint4 omsk[256];
  uint2 e23[256];
};

__device__ __forceinline__ void build_decode_tables(DecodeTables& T, int start_exp, int tid,
                                                    int nthreads) {
  for (int v = tid; v < 256; v += nthreads) {
    uint32_t e1[4], s[4], os[4], om[4];
    uint32_t r[8], k[8];
    uint32_t rank = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      r[j] = rank;
      k[j] = j - rank;
      rank += (v >> j) & 1;
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t lo = (v >> (2 * d)) & 1, hi = (v >> (2 * d + 1)) & 1;
      e1[d] = ((uint32_t)(start_exp + lo) << 7) | ((uint32_t)(start_exp + hi) << 23);
      s[d] = r[2 * d] | (r[2 * d] << 8) | (r[2 * d + 1] << 16) | (r[2 * d + 1] << 24);
      const uint32_t klo = k[2 * d] & 3, khi = k[2 * d + 1] & 3;
      os[d] = (2 * klo) | ((2 * klo + 1) << 8) | ((2 * khi) << 16) | ((2 * khi + 1) << 24);
      om[d] = (lo ? 0u : 0xFFFFu) | (hi ? 0u : 0xFFFF0000u);
    }
    T.e1[v] = make_uint4(e1[0], e1[1], e1[2], e1[3]);
    uint32_t c23[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) c23[j] = ((v >> j) & 1) + 2 * ((v >> (4 + j)) & 1);
    T.e23[v] = make_uint2((c23[0] << 8) | (c23[1] << 24), (c23[2] << 8) | (c23[3] << 24));
    T.sel[v] = make_uint4(s[0], s[1], s[2], s[3]);
    T.osel[v] = make_uint4(os[0], os[1], os[2], os[3]);
    T.omsk[v] = make_uint4(om[0], om[1], om[2], om[3]);
  }
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Inclusive prefix sum over the 64 lanes of a wave: Hillis-Steele inside
// each 16-lane DPP row (row_shr 1,2,4,8), then row_bcast:15 adds row 0's
// total into row 1 and row 2's into row 3, and row_bcast:31 adds the total of
// rows 0-1 into rows 2-3.
__device__ __forceinline__ int wave_inclusive_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return x;
}

// float -> bf16 round-to-nearest-even (quiet NaN kept).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// Compressed-stream pointers of one matrix.
struct Streams {
  const uint8_t* sm;        // sign|mantissa bytes
  const uint16_t* full;     // outlier bf16
  const uint8_t* bm1;       // bitmap planes viewed as bytes
  const uint8_t* bm2;
  const uint8_t* bm3;
  const int32_t* tom;       // TileOffsets_Median
  const int32_t* tog;       // TileOffsets_Global
};

// Per-lane state of one small-tile row ready for decoding.
struct RowRef {
  uint32_t b1, b2, b3;  // bitmap bytes of the lane's row
  uint32_t ind;         // in-window mask (b1|b2|b3)
  int64_t sm_off;       // first SM byte of the row
  int64_t full_off;     // first FULL element of the row
};

// Loads the bitmap bytes of one half median tile and computes every lane's
// stream offsets.  bm_byte = byte index of the half median tile's first row
// (= 512*g + 128*m + 64*h); sm_base / full_base = stream offsets of the half
// median tile's first element.  Returns the tile's in-window count through
// `hf_total` (wave-uniform).
__device__ __forceinline__ RowRef load_half_median(const Streams& s, int64_t bm_byte,
                                                   int64_t sm_base, int64_t full_base,
                                                   int& hf_total) {
  const int l = lane_id();
  RowRef r;
  r.b1 = s.bm1[bm_byte + l];
  r.b2 = s.bm2[bm_byte + l];
  r.b3 = s.bm3[bm_byte + l];
  r.ind = r.b1 | r.b2 | r.b3;
  const int n = __builtin_popcount(r.ind);
  const int incl = wave_inclusive_scan(n);
  const int excl = incl - n;
  hf_total = __builtin_amdgcn_readlane(incl, 63);
  r.sm_off = sm_base + excl;
  r.full_off = full_base + 8 * l - excl;
  return r;
}

// In-window part of a row decode: gathers the lane's sign|mantissa bytes from
// a 12-byte SM window (w0..w2, starting `sh` bytes before the row's first
// byte) with v_perm and merges the exponent field from the LDS tables with
// v_bfi.  `e1` is the plane-1 table holding the start_exp bias (T.e1, or a
// second table for a matrix with another window).  Outlier positions hold
// garbage until patched.
__device__ __forceinline__ u32x4 decode_inwindow(const DecodeTables& T, const uint4* e1,
                                                 uint32_t b1, uint32_t b2, uint32_t b3,
                                                 uint32_t ind, uint32_t w0, uint32_t w1,
                                                 uint32_t w2, uint32_t sh) {
  const uint4 x1 = e1[b1];
  const uint2 y0 = T.e23[(b2 & 15u) | ((b3 & 15u) << 4)];
  const uint2 y1 = T.e23[(b2 >> 4) | (b3 & 0xF0u)];
  const uint4 sel = T.sel[ind];
  const uint32_t s0 = __builtin_amdgcn_alignbyte(w1, w0, sh);
  const uint32_t s1 = __builtin_amdgcn_alignbyte(w2, w1, sh);
  const uint32_t msk = 0x807F807Fu;
  u32x4 o;
  o[0] = (__builtin_amdgcn_perm(s1, s0, sel.x) & msk) | ((x1.x + y0.x) & ~msk);
  o[1] = (__builtin_amdgcn_perm(s1, s0, sel.y) & msk) | ((x1.y + y0.y) & ~msk);
  o[2] = (__builtin_amdgcn_perm(s1, s0, sel.z) & msk) | ((x1.z + y1.x) & ~msk);
  o[3] = (__builtin_amdgcn_perm(s1, s0, sel.w) & msk) | ((x1.w + y1.y) & ~msk);
  return o;
}

// Merges the first four outliers of a row into `o` branch-free: g0/g1 hold
// FULL values k = 0,1 / 2,3 of the row; v_perm places value k_j under each
// outlier lane and v_bfi keeps it only there.
__device__ __forceinline__ void merge_outliers4(const DecodeTables& T, uint32_t ind, uint32_t g0,
                                                uint32_t g1, u32x4& o) {
  const uint4 os = T.osel[ind];
  const uint4 om = T.omsk[ind];
  o[0] = (__builtin_amdgcn_perm(g1, g0, os.x) & om.x) | (o[0] & ~om.x);
  o[1] = (__builtin_amdgcn_perm(g1, g0, os.y) & om.y) | (o[1] & ~om.y);
  o[2] = (__builtin_amdgcn_perm(g1, g0, os.z) & om.z) | (o[2] & ~om.z);
  o[3] = (__builtin_amdgcn_perm(g1, g0, os.w) & om.w) | (o[3] & ~om.w);
}

// Writes the k-th outlier value v of the row into position j (0..7).
__device__ __forceinline__ void patch_outlier(u32x4& o, int j, uint32_t v) {
  const uint32_t shj = (j & 1) * 16;
  const uint32_t keep = ~(0xFFFFu << shj);
  const uint32_t ins = v << shj;
  const int d = j >> 1;
  o[0] = d == 0 ? ((o[0] & keep) | ins) : o[0];
  o[1] = d == 1 ? ((o[1] & keep) | ins) : o[1];
  o[2] = d == 2 ? ((o[2] & keep) | ins) : o[2];
  o[3] = d == 3 ? ((o[3] & keep) | ins) : o[3];
}

// Patches the row's outliers (positions = set bits of fm, in order) from a
// FULL window held in registers: q0..q2 are the 3 dwords starting at the
// 4-byte-aligned address at or below the row's first outlier, `odd` says
// whether that outlier is the high half of q0.  Covers up to 5 outliers
// (6 - odd halfwords); returns the bits of fm still unpatched.
__device__ __forceinline__ uint32_t patch_outliers_window(u32x4& o, uint32_t fm, uint32_t q0,
                                                          uint32_t q1, uint32_t q2, int odd) {
  int hw = odd;
  while (fm && hw < 6) {
    const uint32_t d = hw < 2 ? q0 : (hw < 4 ? q1 : q2);
    patch_outlier(o, __builtin_ctz(fm), (d >> ((hw & 1) * 16)) & 0xFFFFu);
    fm &= fm - 1;
    ++hw;
  }
  return fm;
}

// Decodes the lane's 8 elements into 4 dwords (element 2d in the low half of
// dword d) straight from the global streams.  Outliers are patched from the
// FULL stream in position order.
__device__ __forceinline__ u32x4 decode_row(const Streams& s, const DecodeTables& T,
                                            const RowRef& r) {
  const int64_t a = r.sm_off & ~(int64_t)3;
  const uint32_t* w = reinterpret_cast<const uint32_t*>(s.sm + a);
  u32x4 o = decode_inwindow(T, T.e1, r.b1, r.b2, r.b3, r.ind, w[0], w[1], w[2],
                            (uint32_t)(r.sm_off & 3));
  uint32_t fm = (~r.ind) & 0xFFu;
  if (fm) {
    const uint16_t* f = s.full + r.full_off;
    int k = 0;
    while (fm) {
      patch_outlier(o, __builtin_ctz(fm), f[k]);
      fm &= fm - 1;
      ++k;
    }
  }
  return o;
}

// Decodes both half median tiles (16 rows x 32 columns each) of one staged
// median tile with their dependency chains interleaved.
//   bm     : 3 bitmap planes, plane p at bm + p * plane_stride, rows of half h
//            at byte 64 * h (+ lane)
//   smb    : SM bytes, the median tile's first one at offset `msm`
//   fub    : FULL elements, the median tile's first one at element `mf`
//   gfull  : the same FULL stream in global memory, used when `direct`
// Returns the two MFMA A operands.
struct HalfDec {
  uint32_t b1, b2, b3, ind;
  int n, excl;
};

__device__ __forceinline__ void decode_median_pair(const DecodeTables& T, const uint4* e1,
                                                   const uint8_t* bm,
                                                   int plane_stride, const uint8_t* smb, int msm,
                                                   const uint16_t* fub, int mf, bool direct,
                                                   const uint16_t* gfull, u32x4& o0, u32x4& o1) {
  const int l = lane_id();
  HalfDec d[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    d[h].b1 = bm[64 * h + l];
    d[h].b2 = bm[plane_stride + 64 * h + l];
    d[h].b3 = bm[2 * plane_stride + 64 * h + l];
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    d[h].ind = d[h].b1 | d[h].b2 | d[h].b3;
    d[h].n = __builtin_popcount(d[h].ind);
  }
  // Both halves' in-window counts go through one wave scan, 16 bits each (a
  // half holds at most 512 of them).
  const int nn = d[0].n | (d[1].n << 16);
  const int incl = wave_inclusive_scan(nn);
  const int excl = incl - nn;
  const int tot0 = __builtin_amdgcn_readlane(incl, 63) & 0xFFFF;
  d[0].excl = excl & 0xFFFF;
  d[1].excl = excl >> 16;
  u32x4 o[2];
  int fo[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int smo = msm + (h ? tot0 : 0) + d[h].excl;
    fo[h] = mf + (h ? 512 - tot0 : 0) + 8 * l - d[h].excl;
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(smb + (smo & ~3));
    o[h] = decode_inwindow(T, e1, d[h].b1, d[h].b2, d[h].b3, d[h].ind, wp[0], wp[1], wp[2],
                           (uint32_t)(smo & 3));
  }
  if (!direct) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t* fw = reinterpret_cast<const uint32_t*>(
          reinterpret_cast<const uint8_t*>(fub) + ((2 * fo[h]) & ~3));
      const uint32_t fsh = (uint32_t)((2 * fo[h]) & 3);
      const uint32_t q0 = fw[0], q1 = fw[1], q2 = fw[2];
      merge_outliers4(T, d[h].ind, __builtin_amdgcn_alignbyte(q1, q0, fsh),
                      __builtin_amdgcn_alignbyte(q2, q1, fsh), o[h]);
    }
    // Rows with more than four outliers (fewer than four in-window elements;
    // rare) patch the rest one by one; one wave-wide test skips it all.
    if (__builtin_amdgcn_ballot_w64(d[0].n < 4 || d[1].n < 4))
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (d[h].n < 4) {
        uint32_t rest = (~d[h].ind) & 0xFFu;
        rest &= rest - 1;
        rest &= rest - 1;
        rest &= rest - 1;
        rest &= rest - 1;
        int k = 4;
        while (rest) {
          patch_outlier(o[h], __builtin_ctz(rest), fub[fo[h] + k]);
          rest &= rest - 1;
          ++k;
        }
      }
    }
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t fm = (~d[h].ind) & 0xFFu;
      int k = 0;
      while (fm) {
        patch_outlier(o[h], __builtin_ctz(fm), gfull[fo[h] + k]);
        fm &= fm - 1;
        ++k;
      }
    }
  }
  o0 = o[0];
  o1 = o[1];
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

// X tiles staged in LDS by the 64-row ZipGEMM kernels are stored as MFMA B
// fragments, unpadded: for column block nb and K half h (k 32h .. 32h + 31 of
// the tile) a 1 KB block of 64 16-byte slots; lane l's B operand of
// v_mfma_f32_16x16x32_bf16 (batch row 16*nb + r, k 32h + 8*q .. +7 with
// r = l%16, q = l/16) sits in slot 16*q + (r ^ (8*h + 2*q)).  A B-fragment
// read pass (16 lanes: one q, r = 0..15) then covers 16 slots distinct mod
// 16, and so does a write pass of the X loads (16 threads: two rows r, r ^ 1
// times the eight 16-byte columns 4*h + q of a row), so neither conflicts on
// the LDS banks; the loads keep whole 128-byte rows per 8 threads.
constexpr int kXFragBlock = 1024;
__device__ __forceinline__ int xfrag_slot(int nb, int h, int q, int r) {
  return 64 * (2 * nb + h) + 16 * q + (r ^ (8 * h + 2 * q));
}

}  // namespace zs
