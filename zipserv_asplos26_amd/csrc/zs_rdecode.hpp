// zs_rdecode.hpp -- decoder of the CDNA4 re-tiled layout (gfx950).
//
// Layout (one record per 16 x 64 tile; record r = band * K/64 + kt):
//   fixed part, 1408 B:
//     [16*l .. 16*l+15]   byte i of half h (h*8 + i) of lane l:
//                         (mantissa(h,l,i) << 1) | sign(h,l,i^1)
//                         (every element, outliers too; the sign bit is that
//                         of the element's pair partner, see the decode)
//     [1024 + 4*l]        u32  C(0,l) | C(1,l) << 24
//     [1280 + 2*l]        u16  C(1,l) >> 8
//   C(h,l) = sum_i code(h,l,i) << 3i (24 bits): the 3-bit code of element
//   (h, l, i): 0 = outlier, c = 1..7 -> exponent (start_exp + c) mod 256.
//   exponent stream: per outlier, in (h, l, i) order, its exponent byte,
//   starting at exps[eoff[r]].
// Element (h, l, i) is matrix row 16*band + l%16, column 64*kt + 32*h +
// 8*(l/16) + i: lane l of half h is exactly lane l's A operand of
// v_mfma_f32_16x16x32_bf16 for the 32 columns of that half.
//
// Decode of one group of 4 elements (g = i/4 of half h) for lane l: with the
// 12 code bits q of the group, one 8-byte table entry TB[q] = {codes, sel}
// gives the 4 codes as bytes and the v_perm selectors that pick, per byte,
// either the in-window exponent or the next outlier byte:
//   E   = v_perm(v_perm(EXP_HI, EXP_LO, codes), window, sel)   4 exponent bytes
//   V_d = v_perm(E, SM_g, {0x05010400, 0x07030602}[d])         [sm0 E0 sm1 E1]
//   out = v_alignbit(V_d, V_d, 1)                              two bf16
// where EXP_LO/EXP_HI hold the bytes start_exp + 0..7 and the rotate by one
// bit turns (exponent << 8 | mantissa << 1 | partner sign) pairs into bf16
// pairs.  The lane's outlier bytes start at a wave prefix sum of its outlier
// counts (both halves scanned at once, 16 bits each); the second group of a
// half reads the window shifted past the first group's outliers.
#pragma once
#include "zs_device.hpp"

namespace zs {

constexpr int kRecBytes = 1408;
constexpr int kRecP32 = 1024;
constexpr int kRecP16 = 1280;
constexpr int kExpChunks = 16;                     // staged exponent chunks per record
constexpr int kExpStage = kExpChunks * 16 + 32;    // + window-read slack

// Group table: 4096 entries {codes, sel}, independent of start_exp.
struct RTables {
  uint2 tb[4096];
};

// Table entries are computed from their index, in registers, by each
// workgroup at start-up: for q = 12 code bits, the codes as bytes cb, the
// in-window flags per byte from a carry-free byte add (c + 0x7F sets bit 7
// exactly when c >= 1), the outlier ranks as a byte prefix sum (one multiply:
// the flags are 0 / 1 and the sums at most 3), and the selectors merged
// with one bit-field insert -- 17 VALU per entry.  (A 32 KB image copied
// from global memory instead costs every workgroup 32 KB of L2 -> CU
// traffic while its first records are in flight: 1-6% slower ZipGEMM.)
__device__ __forceinline__ uint2 r_tab_entry(uint32_t q) {
  const uint32_t cb = (q & 7u) | ((q & 0x38u) << 5) | ((q & 0x1C0u) << 10) | ((q & 0xE00u) << 15);
  const uint32_t t = (cb + 0x7F7F7F7Fu) & 0x80808080u;   // bit 7: in window
  const uint32_t rank = ((t ^ 0x80808080u) >> 7) * 0x01010100u;
  const uint32_t m = t | (t - (t >> 7));                 // 0xFF per in-window byte
  return make_uint2(cb, (m & 0x07060504u) | (~m & rank));
}

// The table by `nthreads` threads (tid = this thread's index among them).
__device__ __forceinline__ void build_r_tables(RTables& T, int tid, int nthreads) {
  uint4* dst = reinterpret_cast<uint4*>(T.tb);
  for (int i = tid; i < 2048; i += nthreads) {
    const uint2 a = r_tab_entry(2u * i), b = r_tab_entry(2u * i + 1u);
    dst[i] = make_uint4(a.x, a.y, b.x, b.y);
  }
}

// The same table specialised to one window: entry .x holds the group's four
// in-window exponent bytes (v_perm of EXP_HI:EXP_LO by the codes) instead of
// the codes, which saves that v_perm per group in every decode.
__device__ __forceinline__ void build_r_tables_exp(RTables& T, int tid, int nthreads,
                                                   uint32_t exp_lo, uint32_t exp_hi) {
  uint4* dst = reinterpret_cast<uint4*>(T.tb);
  for (int i = tid; i < 2048; i += nthreads) {
    const uint2 a = r_tab_entry(2u * i), b = r_tab_entry(2u * i + 1u);
    dst[i] = make_uint4(__builtin_amdgcn_perm(exp_hi, exp_lo, a.x), a.y,
                        __builtin_amdgcn_perm(exp_hi, exp_lo, b.x), b.y);
  }
}

// Exponent bytes start_exp + 0..3 and + 4..7 (mod 256).
struct RExp {
  uint32_t lo, hi;
};
__device__ __forceinline__ RExp r_exp(int start_exp) {
  RExp e;
  e.lo = e.hi = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    e.lo |= ((uint32_t)(start_exp + j) & 0xFFu) << (8 * j);
    e.hi |= ((uint32_t)(start_exp + 4 + j) & 0xFFu) << (8 * j);
  }
  return e;
}

// One record's per-lane inputs (registers).
struct RecRegs {
  u32x4 sm;      // sign|mantissa bytes, half 0 in .x/.y, half 1 in .z/.w
  uint32_t p32;  // code bits (see header)
  uint32_t p16;
};

// Outlier count of a group from its selectors (in-window bytes have bit 2 set).
__device__ __forceinline__ uint32_t r_outliers(uint32_t sel) {
  return __builtin_popcount(~sel & 0x04040404u);
}

// Per-lane outlier ranks of both halves (wave prefix sums of the counts
// packed 16 bits per half).  rank0/rank1 = first outlier byte of the lane's
// half 0 / half 1 relative to the record's first one.
__device__ __forceinline__ void r_scan(uint32_t n0, uint32_t n1, int& rank0, int& rank1) {
  const int n = (int)(n0 | (n1 << 16));
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

// Two bf16 pairs (dwords 2g', 2g'+1 of a half) from a group's exponent bytes
// E and sign|mantissa dword sm.
__device__ __forceinline__ void r_pairs(uint32_t E, uint32_t sm, uint32_t& a, uint32_t& b) {
  const uint32_t v0 = __builtin_amdgcn_perm(E, sm, 0x05010400u);
  const uint32_t v1 = __builtin_amdgcn_perm(E, sm, 0x07030602u);
  a = __builtin_amdgcn_alignbit(v0, v0, 1);
  b = __builtin_amdgcn_alignbit(v1, v1, 1);
}

// Decodes one record into the two MFMA A operands (half 0, half 1).  `exb`
// holds the record's outlier bytes, the first one at byte `rel`.
template <bool kExpTab = false, typename P>
__device__ __forceinline__ void r_decode(const RTables& T, RExp ex, const RecRegs& r, P exb,
                                         int rel, u32x4& o0, u32x4& o1) {
  const uint32_t c1 = __builtin_amdgcn_alignbit(r.p16, r.p32, 24);
  const uint2 t0 = T.tb[r.p32 & 0xFFFu], t1 = T.tb[(r.p32 >> 12) & 0xFFFu];
  const uint2 t2 = T.tb[c1 & 0xFFFu], t3 = T.tb[(c1 >> 12) & 0xFFFu];
  const uint32_t n0 = r_outliers(t0.y), n2 = r_outliers(t2.y);
  int rank0, rank1;
  r_scan(n0 + r_outliers(t1.y), n2 + r_outliers(t3.y), rank0, rank1);
  uint32_t a0, a1, b0, b1;
  r_window(exb, rel + rank0, a0, a1);
  r_window(exb, rel + rank1, b0, b1);
  // windows of the second groups: past the first groups' outliers
  const uint32_t a2 = (uint32_t)((((uint64_t)a1 << 32) | a0) >> (8 * n0));
  const uint32_t b2 = (uint32_t)((((uint64_t)b1 << 32) | b0) >> (8 * n2));
  // in-window exponent bytes: straight from a window-specialised table, or
  // the codes mapped through EXP_HI:EXP_LO
  auto inwin = [&](uint32_t x) {
    return kExpTab ? x : __builtin_amdgcn_perm(ex.hi, ex.lo, x);
  };
  const uint32_t e0 = __builtin_amdgcn_perm(inwin(t0.x), a0, t0.y);
  const uint32_t e1 = __builtin_amdgcn_perm(inwin(t1.x), a2, t1.y);
  const uint32_t e2 = __builtin_amdgcn_perm(inwin(t2.x), b0, t2.y);
  const uint32_t e3 = __builtin_amdgcn_perm(inwin(t3.x), b2, t3.y);
  uint32_t d[8];
  r_pairs(e0, r.sm[0], d[0], d[1]);
  r_pairs(e1, r.sm[1], d[2], d[3]);
  r_pairs(e2, r.sm[2], d[4], d[5]);
  r_pairs(e3, r.sm[3], d[6], d[7]);
  o0 = u32x4{d[0], d[1], d[2], d[3]};
  o1 = u32x4{d[4], d[5], d[6], d[7]};
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

// Raw buffer resource over [base, base + bytes): word 3 is the gfx9-family
// value for untyped dword access (data format 32).  Loads through it take a
// wave-uniform base in SGPRs plus a 32-bit lane offset, so they cost no VALU
// address arithmetic, and lanes past `bytes` read zeros.
constexpr int kBufWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t r_buffer(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufWord3);
}

// Range of a buffer resource over `bytes` bytes (> 0), saturated to the
// 32-bit field: every offset a kernel passes through a resource is below
// 2^32, so a saturated range still covers all of them, where a truncated one
// (bytes mod 2^32) would turn in-bounds reads past it into zeros.
__device__ __forceinline__ uint32_t r_range(int64_t bytes) {
  return bytes >= (int64_t)UINT32_MAX ? UINT32_MAX : (uint32_t)bytes;
}

// Cache policy of the record and outlier-byte loads: non-temporal (the
// gfx950 `nt` bit of the buffer instruction).  Every compressed byte is read
// once per launch; a plain streaming read of HBM measured 6.25 TB/s on
// MI355X against 7.0 TB/s with nt, and the re-tiled kernels run 0-7% faster
// with it.  X, the decode table and the offsets keep the default policy
// (they are re-read from L2).
constexpr int kStreamPolicy = 2;

// Fixed part of record `rec` (no dependency on the outlier offsets).
__device__ __forceinline__ void r_issue_fixed(const uint8_t* fixed, int64_t rec, RStage& s) {
  const uint32_t l = (uint32_t)lane_id();
  const __amdgpu_buffer_rsrc_t r = r_buffer(fixed + rec * kRecBytes, kRecBytes);
  s.r.sm = __builtin_amdgcn_raw_buffer_load_b128(r, 16u * l, 0, kStreamPolicy);
  s.r.p32 = __builtin_amdgcn_raw_buffer_load_b32(r, kRecP32 + 4u * l, 0, kStreamPolicy);
  s.r.p16 = __builtin_amdgcn_raw_buffer_load_b16(r, kRecP16 + 2u * l, 0, kStreamPolicy);
}

// Outlier bytes [e0, e1) of a record, as dwords from e0 & ~3 (lane l: dword
// l; lanes past the record's dwords read zeros).
__device__ __forceinline__ void r_issue_exps(const uint8_t* exps, int e0, int e1, RStage& s,
                                             RMeta& mt) {
  const uint32_t l = (uint32_t)lane_id();
  const int ea0 = e0 & ~3;
  const int nw = (e1 - ea0 + 3) >> 2;
  mt.e0 = e0;
  mt.rel = e0 - ea0;
  mt.nw = nw;
  s.ex = __builtin_amdgcn_raw_buffer_load_b32(r_buffer(exps + ea0, 4u * (uint32_t)nw), 4u * l, 0,
                                              kStreamPolicy);
}

__device__ __forceinline__ void r_issue(const uint8_t* fixed, const uint8_t* exps, int64_t rec,
                                        int e0, int e1, RStage& s, RMeta& mt) {
  r_issue_fixed(fixed, rec, s);
  r_issue_exps(exps, e0, e1, s, mt);
}

// The fixed part through a buffer resource built once per band instead of
// per record, so a record costs no 64-bit base arithmetic and no descriptor
// set-up in the scalar unit: `fixed_r` starts at some record r0 and the
// scalar offset `soff` is (record - r0) * kRecBytes (every byte addressed
// belongs to the record).  The outlier bytes keep a per-record resource
// (r_issue_exps): bounded to the record, lanes past it touch no memory --
// a resource over the whole stream, whose lanes read neighbouring bytes,
// measured 1-10% slower.
__device__ __forceinline__ void r_issue_fixed_r(__amdgpu_buffer_rsrc_t fixed_r, uint32_t soff,
                                                RStage& s) {
  const uint32_t l = (uint32_t)lane_id();
  s.r.sm = __builtin_amdgcn_raw_buffer_load_b128(fixed_r, 16u * l, soff, kStreamPolicy);
  s.r.p32 = __builtin_amdgcn_raw_buffer_load_b32(fixed_r, kRecP32 + 4u * l, soff, kStreamPolicy);
  s.r.p16 = __builtin_amdgcn_raw_buffer_load_b16(fixed_r, kRecP16 + 2u * l, soff, kStreamPolicy);
}

// Stages all 64 dwords of a record's outlier fetch (the stage has room for
// them; bytes past the record are never selected by the decode), with no
// per-lane condition.
__device__ __forceinline__ void r_stage_all(uint8_t* st, const RStage& s) {
  *reinterpret_cast<uint32_t*>(st + 4 * lane_id()) = s.ex;
}

// Records whose outlier bytes exceed the stage are decoded from global memory
// and are not staged (the stage holds kExpWords dwords).
__device__ __forceinline__ void r_stage(uint8_t* st, const RStage& s, const RMeta& mt) {
  const int l = lane_id();
  if (r_staged(mt) && l < mt.nw) *reinterpret_cast<uint32_t*>(st + 4 * l) = s.ex;
}

template <bool kExpTab = false>
__device__ __forceinline__ void r_decode_staged(const RTables& T, RExp ex, const RStage& s,
                                                const RMeta& mt, const uint8_t* st,
                                                const uint8_t* exps, u32x4& o0, u32x4& o1) {
  if (r_staged(mt))
    r_decode<kExpTab>(T, ex, s.r, st, mt.rel, o0, o1);
  else
    r_decode<kExpTab>(T, ex, s.r, exps + mt.e0, 0, o0, o1);
}

}  // namespace zs
