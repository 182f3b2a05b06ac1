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

// LDS lookup tables used by the row decoder.  Indexed by one bitmap byte
// (8 positions of a small-tile row); each entry is four dwords = eight 16-bit
// lanes, lane j for position j.
//   e1[v] lane j = (start_exp + bit_j(v)) << 7
//   e2[v] lane j = bit_j(v) << 8
//   e3[v] lane j = bit_j(v) << 9
// so e1[b1] + e2[b2] + e3[b3] = (start_exp + code_j) << 7 = the exponent field.
//   sel[v] dword d = v_perm selector bytes [r_2d, r_2d, r_2d+1, r_2d+1], r_j =
//   number of set bits of v below j (rank of position j in the SM window).
struct DecodeTables {
  uint4 e1[256];
  uint4 e2[256];
  uint4 e3[256];
  uint4 sel[256];
};

__device__ __forceinline__ void build_decode_tables(DecodeTables& T, int start_exp, int tid,
                                                    int nthreads) {
  for (int v = tid; v < 256; v += nthreads) {
    uint32_t e1[4], e2[4], e3[4], s[4];
    uint32_t r[8];
    uint32_t rank = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      r[j] = rank;
      rank += (v >> j) & 1;
    }
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t lo = (v >> (2 * d)) & 1, hi = (v >> (2 * d + 1)) & 1;
      e1[d] = ((uint32_t)(start_exp + lo) << 7) | ((uint32_t)(start_exp + hi) << 23);
      e2[d] = (lo << 8) | (hi << 24);
      e3[d] = (lo << 9) | (hi << 25);
      s[d] = r[2 * d] | (r[2 * d] << 8) | (r[2 * d + 1] << 16) | (r[2 * d + 1] << 24);
    }
    T.e1[v] = make_uint4(e1[0], e1[1], e1[2], e1[3]);
    T.e2[v] = make_uint4(e2[0], e2[1], e2[2], e2[3]);
    T.e3[v] = make_uint4(e3[0], e3[1], e3[2], e3[3]);
    T.sel[v] = make_uint4(s[0], s[1], s[2], s[3]);
  }
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Inclusive prefix sum over the 64 lanes of a wave: Hillis-Steele inside
// each 16-lane DPP row (row_shr 1,2,4,8), then the three row totals are
// folded in with readlane.
__device__ __forceinline__ int wave_inclusive_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  const int t0 = __builtin_amdgcn_readlane(x, 15);
  const int t1 = __builtin_amdgcn_readlane(x, 31);
  const int t2 = __builtin_amdgcn_readlane(x, 47);
  const int row = lane_id() >> 4;
  x += (row > 0 ? t0 : 0) + (row > 1 ? t1 : 0) + (row > 2 ? t2 : 0);
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

// Decodes the lane's 8 elements into 4 dwords (element 2d in the low half of
// dword d).  In-window elements: v_perm gathers sign|mantissa bytes from an
// aligned 12-byte SM window, v_bfi merges the exponent field from the LDS
// tables.  Outliers are patched from the FULL stream in position order.
__device__ __forceinline__ u32x4 decode_row(const Streams& s, const DecodeTables& T,
                                            const RowRef& r) {
  const uint4 x1 = T.e1[r.b1];
  const uint4 x2 = T.e2[r.b2];
  const uint4 x3 = T.e3[r.b3];
  const uint4 sel = T.sel[r.ind];
  const int64_t a = r.sm_off & ~(int64_t)3;
  const uint32_t sh = (uint32_t)(r.sm_off & 3);
  const uint32_t* w = reinterpret_cast<const uint32_t*>(s.sm + a);
  const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
  const uint32_t s0 = __builtin_amdgcn_alignbyte(w1, w0, sh);
  const uint32_t s1 = __builtin_amdgcn_alignbyte(w2, w1, sh);
  u32x4 o;
  o[0] = __builtin_amdgcn_perm(s1, s0, sel.x);
  o[1] = __builtin_amdgcn_perm(s1, s0, sel.y);
  o[2] = __builtin_amdgcn_perm(s1, s0, sel.z);
  o[3] = __builtin_amdgcn_perm(s1, s0, sel.w);
  const uint32_t msk = 0x807F807Fu;
  o[0] = (o[0] & msk) | ((x1.x + x2.x + x3.x) & ~msk);
  o[1] = (o[1] & msk) | ((x1.y + x2.y + x3.y) & ~msk);
  o[2] = (o[2] & msk) | ((x1.z + x2.z + x3.z) & ~msk);
  o[3] = (o[3] & msk) | ((x1.w + x2.w + x3.w) & ~msk);
  uint32_t fm = (~r.ind) & 0xFFu;
  if (fm) {
    const uint16_t* f = s.full + r.full_off;
    int k = 0;
    while (fm) {
      const int j = __builtin_ctz(fm);
      const uint32_t v = f[k];
      const uint32_t shj = (j & 1) * 16;
      const uint32_t keep = ~(0xFFFFu << shj);
      const uint32_t ins = v << shj;
      const int d = j >> 1;
      o[0] = d == 0 ? ((o[0] & keep) | ins) : o[0];
      o[1] = d == 1 ? ((o[1] & keep) | ins) : o[1];
      o[2] = d == 2 ? ((o[2] & keep) | ins) : o[2];
      o[3] = d == 3 ? ((o[3] & keep) | ins) : o[3];
      fm &= fm - 1;
      ++k;
    }
  }
  return o;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  return __builtin_bit_cast(bf16x8, v);
}

}  // namespace zs
