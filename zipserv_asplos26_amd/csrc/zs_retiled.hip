// zs_retiled.hip -- the CDNA4 re-tiled layout on gfx950: encoders (from bf16
// and from canonical TCA-TBE streams), decompress and ZipGEMM.
//
// The layout (zs_rdecode.hpp) stores each 16 x 64 tile as one fixed 1408-byte
// record whose bytes each lane loads straight into the registers it decodes
// from (16 B sign|mantissa + 4 B + 2 B bit-planes), plus a per-record run of
// outlier exponent bytes.  A workgroup streams consecutive records of one
// 16-row band, so HBM sees long contiguous runs; only the outlier bytes pass
// through LDS.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>

#include "../../include/zipserv.h"
#include "zs_device.hpp"
#include "zs_rdecode.hpp"
#include "zs_window.hpp"

namespace zs {

// ---------------------------------------------------------------------------
// Encoders.  One wave per record (grid-stride); lane l gathers its 2 x 8
// elements (one 16-byte load per half) from the bf16 matrix.
// ---------------------------------------------------------------------------
__device__ __forceinline__ const uint16_t* rec_src_at(const uint16_t* a, int K, int64_t band,
                                                      int kt, int h) {
  const int l = lane_id();
  return a + (band * 16 + (l & 15)) * (int64_t)K + kt * 64 + 32 * h + 8 * (l >> 4);
}
__device__ __forceinline__ const uint16_t* rec_src(const uint16_t* a, int K, int64_t rec, int h) {
  const int KT = K >> 6;
  const int64_t band = rec / KT;
  return rec_src_at(a, K, band, (int)(rec - band * KT), h);
}

// The records a wave of a grid-stride loop visits -- rec = w, w + nw, ...
// for wave w of nw -- with their (band, K tile) advanced by addition: one
// division per wave instead of a 64-bit division per record, all in
// wave-uniform (scalar) registers.
struct RecWalk {
  int64_t rec, band, step_band;
  int kt, step_kt, KT;
  __device__ __forceinline__ RecWalk(int K, int64_t nw) {
    KT = K >> 6;
    rec = __builtin_amdgcn_readfirstlane((int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6));
    band = rec / KT;
    kt = (int)(rec - band * KT);
    step_band = nw / KT;
    step_kt = (int)(nw - step_band * KT);
  }
  __device__ __forceinline__ void next(int64_t nw) {
    rec += nw;
    band += step_band;
    kt += step_kt;
    if (kt >= KT) {
      kt -= KT;
      ++band;
    }
  }
};

// Plane bytes of 8 elements from their exponents (window start st).
__device__ __forceinline__ void classify8(u32x4 v, uint32_t st, uint32_t& b1, uint32_t& b2,
                                          uint32_t& b3) {
  b1 = b2 = b3 = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t x = (v[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
    const uint32_t d = (((x >> 7) & 0xFFu) - st) & 0xFFu;
    const uint32_t c = (d >= 1 && d <= 7) ? d : 0u;
    b1 |= (c & 1u) << i;
    b2 |= ((c >> 1) & 1u) << i;
    b3 |= ((c >> 2) & 1u) << i;
  }
}

__device__ __forceinline__ int wave_sum(int x) {
  const int incl = wave_inclusive_scan(x);
  return __builtin_amdgcn_readlane(incl, 63);
}

__global__ __launch_bounds__(256) void rcount_kernel(const uint16_t* a, int M, int K,
                                                     const int32_t* top, int32_t* counts) {
  const uint32_t st = (uint32_t)(top[0] - 1) & 0xFFu;
  const int64_t nrec = (int64_t)(M >> 4) * (K >> 6);
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (RecWalk r(K, nw); r.rec < nrec; r.next(nw)) {
    int n = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t b1, b2, b3;
      classify8(*reinterpret_cast<const u32x4*>(rec_src_at(a, K, r.band, r.kt, h)), st, b1, b2,
                b3);
      n += 8 - __builtin_popcount(b1 | b2 | b3);
    }
    n = wave_sum(n);
    if (lane_id() == 0) counts[r.rec] = n;
  }
}

// Same count from canonical bit-planes (record = median tile m of GT g).
__global__ __launch_bounds__(256) void rcount_canon_kernel(Streams s, int M, int K,
                                                           int32_t* counts) {
  const int KT = K >> 6;
  const int64_t nrec = (int64_t)(M >> 4) * KT;
  const int64_t wid = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const int l = lane_id();
  for (int64_t rec = wid; rec < nrec; rec += nw) {
    const int64_t band = rec / KT, kt = rec % KT;
    const int64_t g = (band >> 2) * KT + kt;
    const int64_t bb = 512 * g + 128 * (band & 3) + l;
    int n = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      n += 8 - __builtin_popcount(s.bm1[bb + 64 * h] | s.bm2[bb + 64 * h] | s.bm3[bb + 64 * h]);
    n = wave_sum(n);
    if (l == 0) counts[rec] = n;
  }
}

// Exclusive scan of the per-record counts into eoff (n + 1 entries), in three
// launches over tiles of 1024 records: each tile's sum is parked at
// eoff[tile * 1024], one workgroup turns those into the tiles' exclusive
// offsets (and writes eoff[n] and *total), then each tile scans its own
// counts from its offset.  Coalesced loads; the single-workgroup pass only
// touches n / 1024 values.
constexpr int kScanTile = 1024;

__device__ __forceinline__ int block256_exclusive(int v, int& total) {
  __shared__ int ws[4];
  const int l = lane_id(), w = threadIdx.x >> 6;
  const int incl = wave_inclusive_scan(v);
  if (l == 63) ws[w] = incl;
  __syncthreads();
  int before = 0;
  for (int i = 0; i < w; ++i) before += ws[i];
  total = ws[0] + ws[1] + ws[2] + ws[3];
  __syncthreads();
  return before + incl - v;
}

// Sum of each kScanTile-record tile into eoff[tile * kScanTile].  With
// `arrive` (a counter that is zero on entry), the workgroup that arrives last
// also turns the tile sums into exclusive tile offsets and writes the total
// (the work of rscan_tiles_kernel, one launch fewer), then returns the
// counter to zero; the sums travel between workgroups through device-scope
// stores and loads, as in splitk_finish.
__global__ __launch_bounds__(256) void rscan_reduce_kernel(const int32_t* counts, int64_t n,
                                                           int32_t* eoff, int32_t* arrive,
                                                           int64_t* total_out) {
  const int64_t base = (int64_t)blockIdx.x * kScanTile;
  int s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t i = base + j * 256 + threadIdx.x;
    if (i < n) s += counts[i];
  }
  int total;
  block256_exclusive(s, total);
  if (!arrive) {
    if (threadIdx.x == 0) eoff[base] = total;
    return;
  }
  __shared__ int last;
  if (threadIdx.x == 0) {
    __hip_atomic_store(&eoff[base], total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the store is performed before the arrival counts
    last = __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           (int)gridDim.x - 1;
  }
  __syncthreads();
  if (!last) return;
  const int64_t ntiles = gridDim.x;
  int64_t carry = 0;
  for (int64_t t0 = 0; t0 < ntiles; t0 += 256) {
    const int64_t tile = t0 + threadIdx.x;
    const int v = tile < ntiles ? __hip_atomic_load(&eoff[tile * kScanTile], __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT)
                                : 0;
    int chunk;
    const int ex = block256_exclusive(v, chunk);
    if (tile < ntiles) eoff[tile * kScanTile] = (int32_t)(carry + ex);
    carry += chunk;
  }
  if (threadIdx.x == 0) {
    eoff[n] = (int32_t)carry;
    *total_out = carry;
    __hip_atomic_store(arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ __launch_bounds__(1024) void rscan_tiles_kernel(int32_t* eoff, int64_t n,
                                                           int64_t* total) {
  __shared__ int64_t wsum[16];
  __shared__ int64_t carry_s;
  const int t = threadIdx.x, l = lane_id(), w = t >> 6;
  const int64_t ntiles = (n + kScanTile - 1) / kScanTile;
  if (t == 0) carry_s = 0;
  __syncthreads();
  for (int64_t t0 = 0; t0 < ntiles; t0 += 1024) {
    const int64_t tile = t0 + t;
    const int v = tile < ntiles ? eoff[tile * kScanTile] : 0;
    const int incl = wave_inclusive_scan(v);
    if (l == 63) wsum[w] = incl;
    __syncthreads();
    int64_t before = carry_s;
    for (int i = 0; i < w; ++i) before += wsum[i];
    if (tile < ntiles) eoff[tile * kScanTile] = (int32_t)(before + incl - v);
    __syncthreads();
    if (t == 0) {
      int64_t sum = 0;
      for (int i = 0; i < 16; ++i) sum += wsum[i];
      carry_s += sum;
    }
    __syncthreads();
  }
  if (t == 0) {
    eoff[n] = (int32_t)carry_s;
    *total = carry_s;
  }
}

__global__ __launch_bounds__(256) void rscan_write_kernel(const int32_t* counts, int64_t n,
                                                          int32_t* eoff) {
  const int64_t base = (int64_t)blockIdx.x * kScanTile;
  const int off = eoff[base];  // this tile's exclusive offset (rewritten unchanged below)
  const int64_t i0 = base + 4 * threadIdx.x;
  int c[4], s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    c[j] = i0 + j < n ? counts[i0 + j] : 0;
    s += c[j];
  }
  int total;
  int run = off + block256_exclusive(s, total);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (i0 + j < n) eoff[i0 + j] = run;
    run += c[j];
  }
}

// Exclusive scan of the per-record outlier counts into eoff (n + 1 entries,
// eoff[n] = *total).  `arrive`: a zeroed counter that lets the reduce kernel
// scan the tile sums itself (two launches instead of three).
static void launch_rscan(hipStream_t st, const int32_t* counts, int64_t n, int32_t* eoff,
                         int64_t* total, int32_t* arrive = nullptr) {
  const int64_t tiles = (n + kScanTile - 1) / kScanTile;
  hipLaunchKernelGGL(rscan_reduce_kernel, dim3((unsigned)tiles), dim3(256), 0, st, counts, n, eoff,
                     arrive, total);
  if (!arrive)
    hipLaunchKernelGGL(rscan_tiles_kernel, dim3(1), dim3(1024), 0, st, eoff, n, total);
  hipLaunchKernelGGL(rscan_write_kernel, dim3((unsigned)tiles), dim3(256), 0, st, counts, n, eoff);
}

// The outlier exponent bytes of one record, in (half, lane, element) order,
// from exps[0] on.
__device__ __forceinline__ void emit_exps(uint8_t* exps, const u32x4 v[2], const uint32_t b[2][3]) {
  uint32_t n[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) n[h] = 8 - __builtin_popcount(b[h][0] | b[h][1] | b[h][2]);
  int rank0, rank1;
  r_scan(n[0], n[1], rank0, rank1);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t fm = ~(b[h][0] | b[h][1] | b[h][2]) & 0xFFu;
    int o = h ? rank1 : rank0;
    while (fm) {
      const int i = __builtin_ctz(fm);
      fm &= fm - 1;
      const uint32_t x = (v[h][i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
      exps[o++] = (uint8_t)((x >> 7) & 0xFFu);
    }
  }
}

// Writes one record from the lane's 16 bf16 values and their code bit-planes
// (Bp bit i = bit p-1 of the code of element i): the fixed part, and the
// outlier bytes from exps[ebase] on unless the record has more than `limit`
// of them.  Returns the record's outlier count.
__device__ __forceinline__ int emit_record(uint8_t* fixed, uint8_t* exps, int64_t rec,
                                           int64_t ebase, const u32x4 v[2],
                                           const uint32_t b[2][3], int limit = 1 << 30) {
  const int l = lane_id();
  u32x4 sm;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      uint32_t w = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 4 * q + j;
        const uint32_t x = (v[h][i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
        const uint32_t xp = (v[h][i >> 1] >> (16 * ((i & 1) ^ 1))) & 0xFFFFu;  // partner i^1
        w |= (((x & 0x7Fu) << 1) | (xp >> 15)) << (8 * j);
      }
      sm[2 * h + q] = w;
    }
  uint32_t c[2], n[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    c[h] = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      c[h] |= (((b[h][0] >> i) & 1u) | (((b[h][1] >> i) & 1u) << 1) | (((b[h][2] >> i) & 1u) << 2))
              << (3 * i);
    n[h] = 8 - __builtin_popcount(b[h][0] | b[h][1] | b[h][2]);
  }
  uint8_t* f = fixed + rec * kRecBytes;
  *reinterpret_cast<u32x4*>(f + 16 * l) = sm;
  *reinterpret_cast<uint32_t*>(f + kRecP32 + 4 * l) = c[0] | (c[1] << 24);
  *reinterpret_cast<uint16_t*>(f + kRecP16 + 2 * l) = (uint16_t)(c[1] >> 8);
  int rank0, rank1;
  r_scan(n[0], n[1], rank0, rank1);
  // total = the last lane's inclusive half-1 rank
  const int total = __builtin_amdgcn_readlane(rank1 + (int)n[1], 63);
  if (total <= limit) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t fm = ~(b[h][0] | b[h][1] | b[h][2]) & 0xFFu;
      int64_t o = ebase + (h ? rank1 : rank0);
      while (fm) {
        const int i = __builtin_ctz(fm);
        fm &= fm - 1;
        const uint32_t x = (v[h][i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
        exps[o++] = (uint8_t)((x >> 7) & 0xFFu);
      }
    }
  }
  return total;
}

__global__ __launch_bounds__(256) void remit_kernel(const uint16_t* a, int M, int K,
                                                    const int32_t* top, const int32_t* eoff,
                                                    uint8_t* fixed, uint8_t* exps) {
  const uint32_t st = (uint32_t)(top[0] - 1) & 0xFFu;
  const int64_t nrec = (int64_t)(M >> 4) * (K >> 6);
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (RecWalk r(K, nw); r.rec < nrec; r.next(nw)) {
    u32x4 v[2];
    uint32_t b[2][3];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v[h] = *reinterpret_cast<const u32x4*>(rec_src_at(a, K, r.band, r.kt, h));
      classify8(v[h], st, b[h][0], b[h][1], b[h][2]);
    }
    emit_record(fixed, exps, r.rec, eoff[r.rec], v, b);
  }
}

// Record encoding a dword (two bf16) at a time.  Codes: with e the exponent
// byte of an element in a 16-bit lane, code = (min((e - st - 1) mod 256, 7)
// + 1) mod 8 -- 1..7 in the window, 0 outside -- from packed 16-bit
// subtract / min / add.  C(h, l) (code of element i at bits 3i) joins the
// lane pairs; z(h) has bit 3i set for each outlier.  The sign / mantissa
// byte of an element, (mantissa << 1) | sign of its pair partner, is byte 0
// (low element) or byte 2 (high element) of the dword rotated left by one
// bit, so one rotate per dword and one byte permute per four elements build
// the record's first 16 bytes.  Same bytes as classify8 + emit_record.
typedef unsigned short us2 __attribute__((ext_vector_type(2)));

struct RecCodes {
  uint32_t c24[2];  // C(h, l)
  uint32_t z[2];    // bit 3i: element i of half h is an outlier
};

__device__ __forceinline__ RecCodes rec_codes(const u32x4 v[2], uint32_t st) {
  const unsigned short s1 = (unsigned short)(st + 1);
  const us2 sub = {s1, s1}, seven = {7, 7}, one = {1, 1};
  RecCodes r;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t e = (v[h][j] >> 7) & 0x00FF00FFu;
      const uint32_t dm = __builtin_bit_cast(uint32_t, __builtin_bit_cast(us2, e) - sub) &
                          0x00FF00FFu;
      const uint32_t c2 =
          __builtin_bit_cast(uint32_t,
                             __builtin_elementwise_min(__builtin_bit_cast(us2, dm), seven) + one) &
          0x00070007u;
      c |= ((c2 & 7u) | (c2 >> 13)) << (6 * j);  // codes of elements 2j, 2j + 1
    }
    r.c24[h] = c;
    r.z[h] = ~(c | (c >> 1) | (c >> 2)) & 0x249249u;
  }
  return r;
}

// Element of bit 3i of z (i = 3i / 3 for 3i <= 21).
__device__ __forceinline__ int rec_elem(int bit3) { return (bit3 * 11) >> 5; }

// emit_record from rec_codes: the fixed part, and the outlier bytes from
// exps[ebase] on unless the record has more than `limit` of them.  Returns
// the record's outlier count.
__device__ __forceinline__ int emit_record_c(uint8_t* fixed, uint8_t* exps, int64_t rec,
                                             int64_t ebase, const u32x4 v[2], const RecCodes& rc,
                                             int limit) {
  const int l = lane_id();
  u32x4 sm;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t t[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) t[j] = __builtin_amdgcn_alignbit(v[h][j], v[h][j], 31);
    sm[2 * h] = __builtin_amdgcn_perm(t[1], t[0], 0x06040200u);
    sm[2 * h + 1] = __builtin_amdgcn_perm(t[3], t[2], 0x06040200u);
  }
  uint8_t* f = fixed + rec * kRecBytes;
  *reinterpret_cast<u32x4*>(f + 16 * l) = sm;
  *reinterpret_cast<uint32_t*>(f + kRecP32 + 4 * l) = rc.c24[0] | (rc.c24[1] << 24);
  *reinterpret_cast<uint16_t*>(f + kRecP16 + 2 * l) = (uint16_t)(rc.c24[1] >> 8);
  const uint32_t n0 = __builtin_popcount(rc.z[0]), n1 = __builtin_popcount(rc.z[1]);
  int rank0, rank1;
  r_scan(n0, n1, rank0, rank1);
  const int total = __builtin_amdgcn_readlane(rank1 + (int)n1, 63);
  if (total <= limit) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t z = rc.z[h];
      int64_t o = ebase + (h ? rank1 : rank0);
      while (z) {
        const int i = rec_elem(__builtin_ctz(z));
        z &= z - 1;
        exps[o++] = (uint8_t)((v[h][i >> 1] >> (16 * (i & 1) + 7)) & 0xFFu);
      }
    }
  }
  return total;
}

// Two-pass encoder (the input is read once after the window histogram):
// rfixed_kernel writes every record's fixed part -- which does not depend
// on where the outlier bytes go -- its outlier count, and up to kExpSlot of
// its outlier bytes into a per-record slot of a temporary buffer; after the
// scan of the counts, rcompact_kernel moves each record's slot to its place
// in the exponent stream (a record with more outliers than the slot re-reads
// its 16 x 64 input tile instead).  Same bytes as rcount + remit.
constexpr int kExpSlot = ZS_RETILED_EXP_SLOT_BYTES;

// kHist: also the exponent histogram of the input, added to hist (64-bit
// bins): in-window elements counted per code from the bit-planes, outliers
// from their exponent bytes.  Workgroup b adds its bins to slice b % kHistSlices
// of hist (kHistSlices histograms 256 bins apart), which spreads the
// same-address atomics of the workgroups over more addresses.  redo: a flag;
// when it is zero the launch does nothing (the one-pass encoder's first pass
// already used the right window).
constexpr int kHistSlices = kVerifySlices;

// The one-pass encoder's window check, at the start of its second launch
// (!kHist with `slices` set): every workgroup sums the first pass's
// kHistSlices histogram slices and applies the rule (zs_window.hpp);
// workgroup 0 writes the histogram (`hist`, 256 x u64), the window (`top`)
// and whether it differs from `guess` (*differs); when it does not, every
// workgroup returns, and otherwise they encode again under it.  (One launch
// fewer than a separate selection kernel before the re-encoding launch.)
struct WindowCheck {
  const uint64_t* slices;
  uint64_t* hist;
  int32_t* top;
  const int32_t* guess;
  int32_t* differs;
  int weights_rule;
};

template <bool kHist>
__global__ __launch_bounds__(256) void rfixed_kernel(const uint16_t* a, int M, int K,
                                                     const int32_t* top, uint8_t* fixed,
                                                     int32_t* counts, uint8_t* tmp,
                                                     uint64_t* hist, const int32_t* redo,
                                                     WindowCheck wc) {
  uint32_t st;
  if constexpr (!kHist) {
    if (wc.slices) {
      __shared__ int64_t cnt[256];
      __shared__ int32_t wtop[8];
      __shared__ int32_t wdiff;
      int64_t c = 0;
#pragma unroll
      for (int sl = 0; sl < kHistSlices; ++sl) c += (int64_t)wc.slices[256 * sl + threadIdx.x];
      cnt[threadIdx.x] = c;
      if (blockIdx.x == 0) wc.hist[threadIdx.x] = (uint64_t)c;
      __syncthreads();
      if (threadIdx.x < 64)
        select_window_wave(wc.weights_rule != 0, cnt, threadIdx.x, wtop, wc.guess, &wdiff);
      __syncthreads();
      if (blockIdx.x == 0 && threadIdx.x < 7) wc.top[threadIdx.x] = wtop[threadIdx.x];
      if (blockIdx.x == 0 && threadIdx.x == 0) *wc.differs = wdiff;
      if (!wdiff) return;
      st = (uint32_t)(wtop[0] - 1) & 0xFFu;
    } else {
      if (redo && *redo == 0) return;
      st = (uint32_t)(top[0] - 1) & 0xFFu;
    }
  } else {
    st = (uint32_t)(top[0] - 1) & 0xFFu;
  }
  __shared__ uint32_t lh[kHist ? 256 : 1];
  if constexpr (kHist) {
    lh[threadIdx.x] = 0;
    __syncthreads();
  }
  const int64_t nrec = (int64_t)(M >> 4) * (K >> 6);
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  uint32_t cc[7] = {0, 0, 0, 0, 0, 0, 0};  // this lane's elements with code 1..7
  for (RecWalk r(K, nw); r.rec < nrec; r.next(nw)) {
    const int64_t rec = r.rec;
    u32x4 v[2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
      v[h] = *reinterpret_cast<const u32x4*>(rec_src_at(a, K, r.band, r.kt, h));
    const RecCodes rc = rec_codes(v, st);
    if constexpr (kHist) {
      // code bit p of element i of half h at bit 3i + h of P[p]; a code's
      // elements are one 3-input bit function of the three planes
      uint32_t P[3];
#pragma unroll
      for (int q = 0; q < 3; ++q)
        P[q] = ((rc.c24[0] >> q) & 0x249249u) | (((rc.c24[1] >> q) & 0x249249u) << 1);
#pragma unroll
      for (int c = 1; c <= 7; ++c)
        cc[c - 1] += __builtin_popcount((c & 1 ? P[0] : ~P[0]) & (c & 2 ? P[1] : ~P[1]) &
                                        (c & 4 ? P[2] : ~P[2]) & 0x6DB6DBu);
    }
    const int n = emit_record_c(fixed, tmp + rec * kExpSlot, rec, 0, v, rc, kExpSlot);
    if constexpr (kHist) {
      // outlier exponents into the workgroup's LDS bins
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint32_t z = rc.z[h];
        while (z) {
          const int i = rec_elem(__builtin_ctz(z));
          z &= z - 1;
          atomicAdd(&lh[(v[h][i >> 1] >> (16 * (i & 1) + 7)) & 0xFFu], 1u);
        }
      }
    }
    if (lane_id() == 0) counts[rec] = n;
  }
  if constexpr (kHist) {
#pragma unroll
    for (int c = 0; c < 7; ++c) {
      const int tot = wave_sum((int)cc[c]);
      if (lane_id() == 0 && tot) atomicAdd(&lh[(st + 1 + c) & 0xFFu], (uint32_t)tot);
    }
    __syncthreads();
    if (lh[threadIdx.x])
      atomicAdd(reinterpret_cast<unsigned long long*>(
                    &hist[256 * (blockIdx.x % kHistSlices) + threadIdx.x]),
                (unsigned long long)lh[threadIdx.x]);
  }
}

// Each wave takes kCompactRecs consecutive records: lane j < kCompactRecs
// loads record r0 + j's offsets, the wave loads the slots of all of them at
// once, then writes them one after another, lane l writing destination dword
// d0 + l of the record's byte range [e0, e0 + n) (d0 = e0 / 4): whole dwords
// with one aligned store (assembled from slot dwords l - 1 and l), the partial
// first and last dwords -- shared with the neighbouring records -- byte by
// byte.  Only the slot dwords that hold outlier bytes are read.  A record
// with more outlier bytes than its slot holds is emitted from a re-read of
// its input tile.  With n <= kExpSlot - 4 the lanes that write stay below
// (n + 3 + 3) / 4 <= kExpSlot / 4, so slot dword l (and l - 1) is in range.
// Few records per wave keep each wave's chain of dependent memory operations
// short; the grid, not the wave, supplies the parallelism.
constexpr int kExpFast = kExpSlot - 4;
constexpr int kCompactRecs = 8;

// A group whose records all fit their slots is assembled in a wave-private
// LDS buffer first (the shared edge dwords of neighbouring records merged
// there, byte writes staying in LDS) and stored as whole dwords, with byte
// stores only at the two ends of the group's range; a group with a record
// past its slot writes each record straight to global memory as below.
constexpr int kCompactBuf = kCompactRecs * kExpFast + 16;  // group range + alignment

__global__ __launch_bounds__(256) void rcompact_kernel(const uint16_t* a, int M, int K,
                                                       const int32_t* top, const int32_t* eoff,
                                                       const uint8_t* __restrict__ tmp,
                                                       uint8_t* __restrict__ exps) {
  __shared__ __attribute__((aligned(16))) uint8_t cbuf[4 * kCompactBuf];
  uint8_t* buf = cbuf + (threadIdx.x >> 6) * kCompactBuf;
  const uint32_t st = (uint32_t)(top[0] - 1) & 0xFFu;
  const int64_t nrec = (int64_t)(M >> 4) * (K >> 6);
  // the stream's slack bytes (read past the end, never selected) as zeros
  if (blockIdx.x == 0 && threadIdx.x < ZS_STREAM_SLACK_BYTES)
    exps[(int64_t)eoff[nrec] + threadIdx.x] = 0;
  const uint32_t* tmp32 = reinterpret_cast<const uint32_t*>(tmp);
  const int64_t wid = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const int l = lane_id();
  for (int64_t r0 = wid * kCompactRecs; r0 < nrec; r0 += nw * kCompactRecs) {
    const int cnt = (int)min<int64_t>(kCompactRecs, nrec - r0);
    const int64_t rl = r0 + min(l, cnt - 1);
    const int e0l = eoff[rl], nl = eoff[rl + 1] - e0l;
    uint32_t cur[kCompactRecs], prev[kCompactRecs];
#pragma unroll
    for (int q = 0; q < kCompactRecs; ++q)
      cur[q] = q < cnt && l < kExpSlot / 4 && 4 * l < __builtin_amdgcn_readlane(nl, q) + 4
                   ? tmp32[(r0 + q) * (kExpSlot / 4) + l]
                   : 0u;
#pragma unroll
    for (int q = 0; q < kCompactRecs; ++q) prev[q] = __shfl_up(cur[q], 1);
    if (__builtin_amdgcn_ballot_w64(l < cnt && nl > kExpFast) == 0) {
      const int E0 = __builtin_amdgcn_readlane(e0l, 0);
      const int E1 = __builtin_amdgcn_readlane(e0l + nl, cnt - 1);
      const int base = E0 & ~3;  // buf byte 0 = stream byte base
#pragma unroll
      for (int q = 0; q < kCompactRecs; ++q) {
        const int n = __builtin_amdgcn_readlane(nl, q);
        const int e0 = __builtin_amdgcn_readlane(e0l, q);
        if (q >= cnt || n == 0) continue;
        const int al = e0 & 3;
        const int p0 = (e0 & ~3) + 4 * l;  // stream byte of this dword
        const uint32_t v = al == 0 ? cur[q] : __builtin_amdgcn_alignbyte(cur[q], prev[q], 4 - al);
        if (p0 >= e0 && p0 + 4 <= e0 + n) {
          *reinterpret_cast<uint32_t*>(buf + (p0 - base)) = v;
        } else {
#pragma unroll
          for (int b = 0; b < 4; ++b)
            if (p0 + b >= e0 && p0 + b < e0 + n) buf[p0 - base + b] = (uint8_t)(v >> (8 * b));
        }
      }
      for (int d = base + 4 * l; d < E1; d += 256) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(buf + (d - base));
        if (d >= E0 && d + 4 <= E1) {
          *reinterpret_cast<uint32_t*>(exps + d) = w;
        } else {
#pragma unroll
          for (int b = 0; b < 4; ++b)
            if (d + b >= E0 && d + b < E1) exps[d + b] = (uint8_t)(w >> (8 * b));
        }
      }
      continue;
    }
    uint32_t slow = 0;  // records re-read from the input
#pragma unroll
    for (int q = 0; q < kCompactRecs; ++q) {
      const int n = __builtin_amdgcn_readlane(nl, q);
      const int e0 = __builtin_amdgcn_readlane(e0l, q);
      if (q >= cnt || n == 0) continue;
      if (n > kExpFast) {
        slow |= 1u << q;
        continue;
      }
      const int al = e0 & 3;
      const int64_t p0 = (int64_t)(e0 & ~3) + 4 * l;  // stream byte of this dword
      // slot bytes 4l - al .. 4l - al + 3
      const uint32_t v = al == 0 ? cur[q] : __builtin_amdgcn_alignbyte(cur[q], prev[q], 4 - al);
      if (p0 >= e0 && p0 + 4 <= e0 + n) {
        *reinterpret_cast<uint32_t*>(exps + p0) = v;
      } else {
#pragma unroll
        for (int b = 0; b < 4; ++b)
          if (p0 + b >= e0 && p0 + b < e0 + n) exps[p0 + b] = (uint8_t)(v >> (8 * b));
      }
    }
    while (slow) {
      const int q = __builtin_ctz(slow);
      slow &= slow - 1;
      u32x4 x[2];
      uint32_t bp[2][3];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        x[h] = *reinterpret_cast<const u32x4*>(rec_src(a, K, r0 + q, h));
        classify8(x[h], st, bp[h][0], bp[h][1], bp[h][2]);
      }
      emit_exps(exps + __builtin_amdgcn_readlane(e0l, q), x, bp);
    }
  }
}

// From canonical streams: each median tile is decoded (global-memory decoder,
// bit-exact) and re-packed; its plane bytes are the canonical bitmap bytes.
__global__ __launch_bounds__(256) void remit_canon_kernel(Streams s, int start_exp, int M, int K,
                                                          const int32_t* eoff, uint8_t* fixed,
                                                          uint8_t* exps) {
  __shared__ DecodeTables T;
  build_decode_tables(T, start_exp, threadIdx.x, blockDim.x);
  __syncthreads();
  const int KT = K >> 6;
  const int64_t nrec = (int64_t)(M >> 4) * KT;
  const int64_t wid = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  const int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t rec = wid; rec < nrec; rec += nw) {
    const int64_t band = rec / KT, kt = rec % KT;
    const int64_t g = (band >> 2) * KT + kt;
    const int m = (int)(band & 3);
    int64_t smb = (int64_t)s.tog[2 * g] + s.tom[2 * (4 * g + m)];
    int64_t fb = (int64_t)s.tog[2 * g + 1] + s.tom[2 * (4 * g + m) + 1];
    u32x4 v[2];
    uint32_t b[2][3];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int tot;
      const RowRef r = load_half_median(s, 512 * g + 128 * m + 64 * h, smb, fb, tot);
      v[h] = decode_row(s, T, r);
      b[h][0] = r.b1;
      b[h][1] = r.b2;
      b[h][2] = r.b3;
      smb += tot;
      fb += 512 - tot;
    }
    emit_record(fixed, exps, rec, eoff[rec], v, b);
  }
}

// ---------------------------------------------------------------------------
// Decompress: a bounded grid of 8-wave workgroups (each copies the decode
// table once); wave g of G takes records g, g + G, g + 2G, ... (consecutive
// waves on consecutive records), fetched three ahead into a register ring
// with their outlier offsets loaded 64 at a time, outlier bytes staged one
// step ahead, and writes each decoded 16x64 tile as 16 rows of 128 bytes.
// ---------------------------------------------------------------------------
constexpr int kDecWaves = 8, kDecDepth = 3;
int device_cu_count();  // zs_gemm.hip
// zs_encode.hip: the window guessed from a sample of the input, and the
// window of a full histogram with a flag saying whether it differs.
hipError_t launch_window_sample(hipStream_t st, const uint16_t* in, int64_t numel,
                                bool weights_rule, uint64_t* sample, uint64_t* zero,
                                int32_t* guess, int32_t* zero32);


__global__ __launch_bounds__(kDecWaves * 64) void rdecompress_kernel(const uint8_t* fixed,
                                                                     const uint8_t* exps,
                                                                     const int32_t* eoff,
                                                                     int start_exp, uint16_t* out,
                                                                     int M, int K) {
  __shared__ RTables T;
  __shared__ __attribute__((aligned(16))) uint8_t stg[kDecWaves][kDecDepth][kExpStage];
  const RExp ex = r_exp(start_exp);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  const int KT = K >> 6;
  const int64_t nrec = (int64_t)(M >> 4) * KT;
  const int64_t G = (int64_t)gridDim.x * kDecWaves;
  const int64_t g = (int64_t)blockIdx.x * kDecWaves + w;
  const int64_t cnt64 = g < nrec ? (nrec - g + G - 1) / G : 0;
  const int cnt = (int)cnt64;  // records of this wave (the host keeps it < 2^31)
  // record j of this wave; waves without records read record 0 (in bounds)
  auto rec_of = [&](int j) { return cnt > 0 ? g + (int64_t)j * G : (int64_t)0; };

  RStage R[kDecDepth];
  RMeta MT[kDecDepth];
  int oe0 = 0, oe1 = 0;
  int c0 = 0;
#define RD_OFFSETS(LAST)                                 \
  {                                                      \
    const int64_t ri_ = rec_of(c0 + min(l, (LAST)));     \
    oe0 = eoff[ri_];                                     \
    oe1 = eoff[ri_ + 1];                                 \
  }
#define RD_FIXED(J, RR) r_issue_fixed(fixed, rec_of(c0 + (J)), RR)
#define RD_EXPS(J, RR, MM)                                                        \
  r_issue_exps(exps, __builtin_amdgcn_readlane(oe0, (J)),                       \
                 __builtin_amdgcn_readlane(oe1, (J)), RR, MM)
  // Start-up (branch-free): offsets and the first records' fixed parts
  // together; outlier bytes once the offsets land; the decode table is
  // computed while they are in flight.
  {
    const int last = max(min(cnt, 64) - 1, 0);
    RD_OFFSETS(last);
#pragma unroll
    for (int k = 0; k < kDecDepth; ++k) RD_FIXED(min(k, last), R[k]);
#pragma unroll
    for (int k = 0; k < kDecDepth; ++k) RD_EXPS(min(k, last), R[k], MT[k]);
    build_r_tables_exp(T, threadIdx.x, kDecWaves * 64, ex.lo, ex.hi);
  }
  __syncthreads();

  for (; c0 < cnt; c0 += 64) {
    const int n = min(cnt - c0, 64);
    const int last = n - 1;
    if (c0 > 0) {
      RD_OFFSETS(last);
#pragma unroll
      for (int k = 0; k < kDecDepth; ++k) {
        RD_FIXED(min(k, last), R[k]);
        RD_EXPS(min(k, last), R[k], MT[k]);
      }
    }
    r_stage_all(stg[w][0], R[0]);
    for (int j = 0; j < n; j += kDecDepth) {
#pragma unroll
      for (int k = 0; k < kDecDepth; ++k) {
        const int jj = j + k;
        const int kn = (k + 1) % kDecDepth;
        r_stage_all(stg[w][kn], R[kn]);
        if (jj < n) {
          u32x4 o0, o1;
          r_decode_staged<true>(T, ex, R[k], MT[k], stg[w][k], exps, o0, o1);
          const int64_t rec = rec_of(c0 + jj);
          const int64_t band = rec / KT, kt = rec - band * KT;
          uint16_t* dst = out + (band * 16 + (l & 15)) * (int64_t)K + kt * 64 + 8 * (l >> 4);
          *reinterpret_cast<u32x4*>(dst) = o0;
          *reinterpret_cast<u32x4*>(dst + 32) = o1;
        }
        const int jn = min(jj + kDecDepth, last);
        RD_FIXED(jn, R[k]);
        RD_EXPS(jn, R[k], MT[k]);
      }
    }
  }
#undef RD_EXPS
#undef RD_FIXED
#undef RD_OFFSETS
}

// ---------------------------------------------------------------------------
// In-kernel split-K reduction (zs_retiled_mm_fused).  Each workgroup stores
// its bf16 partial tile into slice `split` of the workspace with
// device-coherent stores (sc1: written through past the XCD's L2), waits
// until they are complete, and counts its arrival in cnt[tile] with an
// atomic add.  The workgroup that arrives last reads the split_k slices of
// the tile with device-coherent loads, adds them in split order in fp32 --
// the order and rounding of rsplitk_reduce_kernel, so the result is the
// same -- writes C and returns the counter to zero for the next call.  No
// workgroup waits for another, and no L2-wide writeback or invalidation
// (an acquire-release count costs both per workgroup: measured 3-4x slower
// on grids of ~1000 workgroups) is needed, because only these stores and
// loads carry data between workgroups.
// ---------------------------------------------------------------------------
struct SplitFix {
  uint16_t* C;   // final output [N][M]
  int32_t* cnt;  // per-tile arrival counters; nullptr: no in-kernel reduction
  int split_k;
};

__device__ __forceinline__ bool splitk_arrive(int32_t* c, int split_k) {
  return __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == split_k - 1;
}

// Four bf16 of a partial tile; device-coherent when the tile is reduced
// inside the kernel.
__device__ __forceinline__ void store4(uint16_t* p, uint32_t lo, uint32_t hi, bool coherent) {
  if (coherent)
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), (uint64_t)lo | ((uint64_t)hi << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else
    *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
}

__device__ __forceinline__ void splitk_reset(int32_t* c) {
  __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until this wave's stores are complete (acknowledged at device
// scope), before the barrier after which one wave counts the arrival.
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(0); }

__device__ __forceinline__ uint64_t load_agent(const uint16_t* p) {
  return __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<uint16_t*>(p)),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// End of a split-K GEMM workgroup whose tile is rows [m0, m0 + ROWS) x
// columns [n0, n0 + COLS) (waves with `wrote` stored their part of it into
// slice blockIdx.y of ws).  Counts the arrival; the last workgroup of the
// tile sums its split_k slices with all NT threads, 4 rows of one column
// per item, every slice of an item loaded before the first add.
template <int ROWS, int COLS, int NT>
__device__ __forceinline__ void splitk_finish(const SplitFix& fx, const uint16_t* ws, int M, int N,
                                              int m0, int n0, bool wrote) {
  __shared__ int last_arrival;
  if (wrote) wait_stores();
  __syncthreads();
  int32_t* c = fx.cnt + blockIdx.z * gridDim.x + blockIdx.x;
  if (threadIdx.x == 0) last_arrival = splitk_arrive(c, fx.split_k);
  __syncthreads();
  if (!last_arrival) return;
  constexpr int kQ = ROWS / 4;                     // items per column
  constexpr int kPer = (kQ * COLS + NT - 1) / NT;  // items per thread
  constexpr int kBatch = 4;                        // slices in flight per item
  const int64_t mn = (int64_t)M * N;
  const int S = fx.split_k;
  int64_t off[kPer];
  bool ok[kPer];
  float a[kPer][4];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int it = threadIdx.x + NT * j;
    const int n = n0 + it / kQ, m = m0 + 4 * (it % kQ);
    ok[j] = it < kQ * COLS && n < N && m < M;
    off[j] = ok[j] ? (int64_t)n * M + m : 0;
    a[j][0] = a[j][1] = a[j][2] = a[j][3] = 0.f;
  }
  for (int k0 = 0; k0 < S; k0 += kBatch) {
    uint64_t v[kPer][kBatch];
#pragma unroll
    for (int j = 0; j < kPer; ++j)
#pragma unroll
      for (int k = 0; k < kBatch; ++k) v[j][k] = load_agent(ws + min(k0 + k, S - 1) * mn + off[j]);
#pragma unroll
    for (int j = 0; j < kPer; ++j)
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (k0 + k < S) {
          const uint32_t lo = (uint32_t)v[j][k], hi = (uint32_t)(v[j][k] >> 32);
          a[j][0] += bf16_bits_to_f32(lo & 0xFFFFu);
          a[j][1] += bf16_bits_to_f32(lo >> 16);
          a[j][2] += bf16_bits_to_f32(hi & 0xFFFFu);
          a[j][3] += bf16_bits_to_f32(hi >> 16);
        }
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j)
    if (ok[j])
      *reinterpret_cast<uint2*>(fx.C + off[j]) =
          make_uint2(f32_to_bf16_bits(a[j][0]) | (f32_to_bf16_bits(a[j][1]) << 16),
                     f32_to_bf16_bits(a[j][2]) | (f32_to_bf16_bits(a[j][3]) << 16));
  if (threadIdx.x == 0) splitk_reset(c);
}

// ---------------------------------------------------------------------------
// ZipGEMM over the re-tiled layout, narrow batches.  Workgroup = WAVES waves
// on F consecutive 16-row bands x one split-K slice x 16*NB columns; wave w
// takes K tiles kb0+w, kb0+w+WAVES, ... of all F bands, so each X fragment
// it loads feeds F records (X bytes per record / F).  Records are fetched D
// tiles ahead into a register ring, their outlier bytes staged one tile
// ahead.
//
// X, two ways (XD):
//  * XD == 0: each lane loads its two 16-byte MFMA B fragments one tile
//    ahead (2 KB returned per tile whatever N is; rows past N read zeros);
//  * XD > 0 (N <= 2 * XD, one column block): the wave loads just the tile's
//    2*XD batch rows (XD dwords per lane, issued with the records of the same
//    tile, D tiles ahead), writes them to its LDS X stage and reads the B
//    fragments from there.  At N = 1 that is 256 bytes through the texture
//    path per tile instead of 2 KB -- the texture address / data units are
//    ~80% busy in this kernel (counters at 28672 x 8192, N = 1) -- and since
//    vector-memory loads complete in issue order, an X load issued with the
//    records no longer makes the MFMA wait for records issued after it.
//    Same operands, same sums: results are bit-identical to XD == 0.
// ---------------------------------------------------------------------------
template <int F, int NB, int WAVES, int D, int XD>
struct RGemmSmem {
  static constexpr int kXPitch = 144;                            // X stage row pitch
  static constexpr int kXRows = 2 * XD;                          // rows one X load covers
  static constexpr int kXStage = XD > 0 ? kXRows * kXPitch : 0;  // bytes per wave
  static constexpr int kXAt = WAVES * D * F * kExpStage;
  static constexpr int kTabAt = (kXAt + WAVES * kXStage + 15) / 16 * 16;
  static constexpr int kMain = kTabAt + (int)sizeof(RTables);
  static constexpr int kRed = (WAVES - 1) * F * NB * 64 * 16;
  static constexpr int kBytes = kMain > kRed ? kMain : kRed;
};

// X tile of the staged-X path: lane l carries XD dwords, bytes 4*XD*l ..
// of the 2*XD x 64 bf16 tile in row-major order.
template <int XD>
struct XFrag {
  uint32_t d[XD > 0 ? XD : 1];
};
template <int XD>
__device__ __forceinline__ void x_load(__amdgpu_buffer_rsrc_t xrs, uint32_t voff, uint32_t soff,
                                       XFrag<XD>& x) {
  if constexpr (XD == 1) {
    x.d[0] = __builtin_amdgcn_raw_buffer_load_b32(xrs, voff, soff, 0);
  } else if constexpr (XD == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(xrs, voff, soff, 0);
    x.d[0] = v[0];
    x.d[1] = v[1];
  } else {
    static_assert(XD % 4 == 0, "X loads of 1, 2 or a multiple of 4 dwords");
#pragma unroll
    for (int q = 0; q < XD / 4; ++q) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xrs, voff + 16u * q, soff, 0);
      x.d[4 * q] = v[0];
      x.d[4 * q + 1] = v[1];
      x.d[4 * q + 2] = v[2];
      x.d[4 * q + 3] = v[3];
    }
  }
}
template <int XD>
__device__ __forceinline__ void x_stage(uint8_t* p, const XFrag<XD>& x) {
  if constexpr (XD == 1) {
    *reinterpret_cast<uint32_t*>(p) = x.d[0];
  } else if constexpr (XD == 2) {
    *reinterpret_cast<uint2*>(p) = make_uint2(x.d[0], x.d[1]);
  } else {
#pragma unroll
    for (int q = 0; q < XD / 4; ++q)
      *reinterpret_cast<u32x4*>(p + 16 * q) =
          u32x4{x.d[4 * q], x.d[4 * q + 1], x.d[4 * q + 2], x.d[4 * q + 3]};
  }
}

// Launch bounds: one band per wave in 8-wave workgroups is held to 80 VGPRs
// (6 waves per SIMD, three workgroups per CU).
template <int F, int NB, int WAVES, int D, int XD>
__global__ __launch_bounds__(WAVES * 64, (WAVES == 8 && F == 1) ? 6 : 1) void rgemm_kernel(const uint8_t* fixed,
                                                           const uint8_t* exps,
                                                           const int32_t* eoff, int start_exp,
                                                           const uint16_t* X, uint16_t* Y, int M,
                                                           int N, int K, int kb_per_split,
                                                           SplitFix fx) {
  // LDS: the waves' outlier stages first, then the decode table.  (With the
  // stages at a small base, a window's dword reads fold their offsets into
  // the instructions; the table reads take the large constant instead.)
  using SM = RGemmSmem<F, NB, WAVES, D, XD>;
  static_assert(XD == 0 || NB == 1, "the staged-X path covers one 16-column block");
  __shared__ __attribute__((aligned(16))) uint8_t smem[SM::kBytes];
  constexpr int kTabAt = SM::kTabAt;
  static_assert(kTabAt % 16 == 0, "table alignment");
  RTables& T = *reinterpret_cast<RTables*>(smem + kTabAt);
  const RExp ex = r_exp(start_exp);

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  // stage s of band f: smem + ((w * D + s) * F + f) * kExpStage
  uint8_t* stg = smem + w * D * F * kExpStage;
  const int bands = M >> 4;
  const int band0 = blockIdx.x * F;
  const int split = blockIdx.y;
  const int n0 = blockIdx.z * NB * 16;
  const int KT = K >> 6;
  const int kb0 = split * kb_per_split;
  const int kb1 = min(kb0 + kb_per_split, KT);
  const int cnt = kb1 - kb0 > w ? (kb1 - kb0 - w + WAVES - 1) / WAVES : 0;
  // Record of this wave's tile 0 per band (past the end: last band), and the
  // K tile of its X fragments.  A wave without tiles points both at tile 0
  // of the band so that its (unused) start-up loads stay in bounds.
  const int xt0 = cnt > 0 ? kb0 + w : 0;
  int64_t rec0[F];
#pragma unroll
  for (int f = 0; f < F; ++f) rec0[f] = (int64_t)min(band0 + f, bands - 1) * KT + xt0;

  // Buffer resources built once: the records of each band from this wave's
  // tile 0 on (tile j at scalar offset j * WAVES * kRecBytes) and X (tile t
  // at scalar offset 128 t), so those loads carry no per-record descriptor
  // or 64-bit base arithmetic.
  __amdgpu_buffer_rsrc_t frs[F];
#pragma unroll
  for (int f = 0; f < F; ++f) frs[f] = r_buffer(fixed + rec0[f] * kRecBytes, (uint32_t)KT * kRecBytes);
  // X fragments: this lane's 32-bit byte offset (row n, 8 columns; N <= 16
  // here: offsets far below 2^31).  Lanes of rows n >= N get the offset
  // 2^31, at or past the resource's range whether or not the scalar offset
  // counts in the range check: they read zeros without touching memory (at
  // N = 1, 1/16 of the bytes a full fragment returns), and their output
  // columns are dropped anyway.
  const __amdgpu_buffer_rsrc_t xrs = r_buffer(X, 0x80000000u);
  uint32_t xoff[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = n0 + nb * 16 + (l & 15);
    xoff[nb] = n < N ? 2u * ((uint32_t)n * (uint32_t)K + 8u * (uint32_t)(l >> 4)) : 0x80000000u;
  }
  // Staged X: this lane loads row xrow, bytes xcol.. of the tile (rows past N
  // read zeros) and writes them to the wave's stage; it reads its B fragment
  // at batch row l % 16, clamped into the stage (output columns past N are
  // dropped).
  const int xrow = (XD * l) >> 5, xcol = (4 * XD * l) & 127;
  const uint32_t xloff = n0 + xrow < N
                             ? 2u * (uint32_t)(n0 + xrow) * (uint32_t)K + (uint32_t)xcol
                             : 0x80000000u;
  uint8_t* xst = smem + SM::kXAt + w * SM::kXStage;
  uint8_t* xst_w = xst + xrow * SM::kXPitch + xcol;
  const uint8_t* xst_r =
      xst + min(l & 15, (XD > 0 ? SM::kXRows : 1) - 1) * SM::kXPitch + 16 * (l >> 4);
  f32x4 acc[F * NB];
#pragma unroll
  for (int i = 0; i < F * NB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Tiles go in chunks of up to 64 per wave (lane i holds the outlier
  // offsets of tile c0 + i, clamped to the chunk, per band).
  RStage R[D][F];
  RMeta MT[D][F];
  bf16x8 xc[2][NB], xn[2][NB];  // XD == 0: B fragments of this tile and the next
  XFrag<XD> xr[D];              // XD > 0: X tiles of the ring's steps
  int oe0[F], oe1[F];
  int c0 = 0;
#define RZ_OFFSETS()                                                        \
  {                                                                         \
    _Pragma("unroll") for (int f_ = 0; f_ < F; ++f_) {                      \
      const int64_t ri_ = rec0[f_] + (int64_t)(c0 + min(l, last)) * WAVES;  \
      oe0[f_] = eoff[ri_];                                                  \
      oe1[f_] = eoff[ri_ + 1];                                              \
    }                                                                       \
  }
#define RZ_LOADX(J, DST)                                                              \
  {                                                                                   \
    const uint32_t xs_ = (uint32_t)(xt0 + (c0 + (J)) * WAVES) * 128u;                 \
    _Pragma("unroll") for (int nb_ = 0; nb_ < NB; ++nb_) {                            \
      DST[0][nb_] = __builtin_bit_cast(                                               \
          bf16x8, __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff[nb_], xs_, 0));     \
      DST[1][nb_] = __builtin_bit_cast(                                               \
          bf16x8, __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff[nb_] + 64u, xs_, 0)); \
    }                                                                                 \
  }
#define RZ_LOADXS(J, DST)                                                             \
  x_load<XD>(xrs, xloff, (uint32_t)(xt0 + (c0 + (J)) * WAVES) * 128u, DST)
#define RZ_ISSUE_FIXED(J, R)                                                              \
  {                                                                                       \
    const uint32_t fs_ = (uint32_t)((c0 + (J)) * WAVES) * (uint32_t)kRecBytes;            \
    _Pragma("unroll") for (int f_ = 0; f_ < F; ++f_) r_issue_fixed_r(frs[f_], fs_, R[f_]); \
  }
#define RZ_ISSUE_EXPS(J, R, MT)                                                    \
  {                                                                                \
    const int j_ = (J);                                                            \
    _Pragma("unroll") for (int f_ = 0; f_ < F; ++f_)                               \
      r_issue_exps(exps, __builtin_amdgcn_readlane(oe0[f_], j_),                  \
                     __builtin_amdgcn_readlane(oe1[f_], j_), R[f_], MT[f_]);       \
  }
#define RZ_ISSUE(J, R, MT) \
  {                        \
    RZ_ISSUE_FIXED(J, R);  \
    RZ_ISSUE_EXPS(J, R, MT); \
  }
#define RZ_STAGE(S, R, MT)                                                                \
  {                                                                                       \
    _Pragma("unroll") for (int f_ = 0; f_ < F; ++f_)                                      \
      r_stage_all(stg + ((S) * F + f_) * kExpStage, R[f_]);                               \
  }
#define RZ_STEP(J, SC, SN, RC, MC, RN, MN)                                                 \
  {                                                                                        \
    if constexpr (XD == 0) {                                                               \
      _Pragma("unroll") for (int nb_ = 0; nb_ < NB; ++nb_) {                               \
        xc[0][nb_] = xn[0][nb_];                                                           \
        xc[1][nb_] = xn[1][nb_];                                                           \
      }                                                                                    \
      RZ_LOADX(min((J) + 1, last), xn);                                                    \
    }                                                                                      \
    RZ_STAGE(SN, RN, MN);                                                                  \
    if constexpr (XD > 0) {                                                                \
      x_stage<XD>(xst_w, xr[SC]);                                                          \
      xc[0][0] = *reinterpret_cast<const bf16x8*>(xst_r);                                  \
      xc[1][0] = *reinterpret_cast<const bf16x8*>(xst_r + 64);                             \
    }                                                                                      \
    if ((J) < n) {                                                                         \
      _Pragma("unroll") for (int f_ = 0; f_ < F; ++f_) {                                   \
        u32x4 a0_, a1_;                                                                    \
        r_decode_staged<true>(T, ex, RC[f_], MC[f_], stg + ((SC) * F + f_) * kExpStage, exps, a0_, \
                        a1_);                                                              \
        _Pragma("unroll") for (int nb_ = 0; nb_ < NB; ++nb_) {                             \
          f32x4& c_ = acc[f_ * NB + nb_];                                                  \
          c_ = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a0_), xc[0][nb_], c_, 0,  \
                                                       0, 0);                              \
          c_ = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a1_), xc[1][nb_], c_, 0,  \
                                                       0, 0);                              \
        }                                                                                  \
      }                                                                                    \
    }                                                                                      \
    RZ_ISSUE(min((J) + D, last), RC, MC);                                                  \
    if constexpr (XD > 0) RZ_LOADXS(min((J) + D, last), xr[SC]);                           \
  }
  // Start-up: chunk 0's outlier offsets, the first records' fixed parts and
  // the first X tile go out together; the records' outlier bytes follow as
  // soon as the offsets are in (loads return in issue order), and the decode
  // table is computed into LDS while they are in flight.  (No branches
  // here: the wait counts the compiler places stay exact.)
  {
    const int last = max(min(cnt, 64) - 1, 0);
    RZ_OFFSETS();
#pragma unroll
    for (int k = 0; k < D; ++k) {
      RZ_ISSUE_FIXED(min(k, last), R[k]);
      if constexpr (XD > 0) RZ_LOADXS(min(k, last), xr[k]);
    }
    if constexpr (XD == 0) RZ_LOADX(0, xn);
#pragma unroll
    for (int k = 0; k < D; ++k) RZ_ISSUE_EXPS(min(k, last), R[k], MT[k]);
    build_r_tables_exp(T, threadIdx.x, WAVES * 64, ex.lo, ex.hi);
  }
  __syncthreads();

  for (; c0 < cnt; c0 += 64) {
    const int n = min(cnt - c0, 64);
    const int last = n - 1;
    if (c0 > 0) {
      RZ_OFFSETS();
#pragma unroll
      for (int k = 0; k < D; ++k) {
        RZ_ISSUE(min(k, last), R[k], MT[k]);
        if constexpr (XD > 0) RZ_LOADXS(min(k, last), xr[k]);
      }
      if constexpr (XD == 0) RZ_LOADX(0, xn);
    }
    RZ_STAGE(0, R[0], MT[0]);
    for (int j = 0; j < n; j += D) {
#pragma unroll
      for (int k = 0; k < D; ++k)
        RZ_STEP(j + k, k, (k + 1) % D, R[k], MT[k], R[(k + 1) % D], MT[(k + 1) % D]);
    }
  }
#undef RZ_STEP
#undef RZ_STAGE
#undef RZ_ISSUE_EXPS
#undef RZ_ISSUE_FIXED
#undef RZ_ISSUE
#undef RZ_LOADXS
#undef RZ_LOADX
#undef RZ_OFFSETS

  // Deterministic reduction of the WAVES partial accumulators: waves 1.. hand
  // theirs to wave 0 through LDS (after the decode, whose table and stages
  // the LDS held), which adds them pairwise -- a[w] += a[w + h] for
  // h = WAVES/2, ..., 1, the canonical kernel's tree order -- so the other
  // waves are done after one exchange.
  __syncthreads();
  f32x4* red = reinterpret_cast<f32x4*>(smem);
  if (w > 0) {
#pragma unroll
    for (int i = 0; i < F * NB; ++i) red[((w - 1) * F * NB + i) * 64 + l] = acc[i];
  }
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int i = 0; i < F * NB; ++i) {
      f32x4 a[WAVES];
      a[0] = acc[i];
#pragma unroll
      for (int v = 1; v < WAVES; ++v) a[v] = red[((v - 1) * F * NB + i) * 64 + l];
#pragma unroll
      for (int h = WAVES / 2; h >= 1; h /= 2)
#pragma unroll
        for (int v = 0; v < h; ++v) a[v] += a[v + h];
      acc[i] = a[0];
    }
  }
  if (w == 0) {
    uint16_t* out = Y + (int64_t)split * M * N;
#pragma unroll
    for (int f = 0; f < F; ++f)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 v = acc[f * NB + nb];
        const int n = n0 + nb * 16 + (l & 15);
        if (n < N && band0 + f < bands) {
          const int mrow = (band0 + f) * 16 + 4 * (l >> 4);
          const uint32_t lo = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
          const uint32_t hi = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
          store4(out + (int64_t)n * M + mrow, lo, hi, fx.cnt != nullptr);
        }
      }
  }
  if (fx.cnt)
    splitk_finish<16 * F, 16 * NB, WAVES * 64>(fx, Y, M, N, band0 * 16, n0, w == 0);
}

// ---------------------------------------------------------------------------
// ZipGEMM over the re-tiled layout, narrow batches (N <= 16), stream-K
// schedule.  The band-per-workgroup grid of rgemm_kernel leaves CUs idle
// whenever the band count is not a multiple of the resident workgroups (640
// bands on 256 CUs x 3 slots: half the CUs hold 3, half 2) and pays a
// workgroup start-up per band.  Here the grid is exactly kSkPerCu
// workgroups per CU, one round, and workgroup g takes the contiguous record
// range [g R / G, (g + 1) R / G) of the R = bands x K/64 records in band-major
// order; its waves take records r_lo + w, r_lo + w + 8, ... (consecutive
// waves read consecutive records), crossing band boundaries on the way, so
// the record ring never drains inside a workgroup.
//
// Partial sums, deterministic and barrier-free:
//  * a wave that moves on to a new band flushes its accumulator for the old
//    one into an LDS slot of that band segment (16 rows x N columns fp32)
//    and counts itself with an LDS atomic; the wave that completes the
//    count (the segment's records are shared by min(8, length) waves) adds
//    the slots in wave order;
//  * a segment that is a whole band is written to Y as bf16; a band split
//    between workgroups (at most the first and the last segment of a range)
//    has each workgroup's fp32 partial stored device-coherently in the
//    workspace (slot 2g for its first band, 2g + 1 for its last), counted
//    with an agent-scope atomic per band, and the last arrival adds the
//    partials in workgroup order, writes Y and returns the counter to zero
//    (the protocol of splitk_finish, with fp32 partials).
// The sums differ from rgemm_kernel's only in fp32 summation order; no
// partial is rounded to bf16.
// ---------------------------------------------------------------------------
constexpr int kSkWaves = 8;
constexpr int kSkPerCu = 3;       // resident 8-wave workgroups per CU (LDS, 80 VGPRs)
constexpr int kSkMaxSegments = 8; // segment slots per workgroup (LDS)
constexpr int64_t kCuLdsBytes = 160 * 1024;  // LDS per CU on gfx950

template <int XD>
struct RSkSmem {
  static constexpr int kStages = 2;  // outlier stages per wave (ping-pong)
  static constexpr int kXPitch = 144;
  static constexpr int kXRows = 2 * XD;
  static constexpr int kXStage = XD > 0 ? kXRows * kXPitch : 0;
  static constexpr int kXAt = kSkWaves * kStages * kExpStage;
  static constexpr int kTabAt = (kXAt + kSkWaves * kXStage + 15) / 16 * 16;
  static constexpr int kSlotsAt = kTabAt + (int)sizeof(RTables);
  // + S segment slots of kSkWaves x 16 rows x N columns fp32, + S counters
  static constexpr int64_t bytes(int S, int N) {
    return (int64_t)kSlotsAt + (int64_t)S * kSkWaves * 64 * N + 4 * S;
  }
};

// workgroup holding record r of R over G workgroups (range starts g R / G)
__device__ __forceinline__ int sk_wg_of(int64_t r, int64_t R, int G) {
  return (int)(((r + 1) * G - 1) / R);
}

// The kernel's state a segment's completion needs (LDS slots, the
// workspace, the band counters, the range of this workgroup).
struct SkCtx {
  float* slots;
  float* ws;
  int32_t* bcnt;
  uint16_t* Y;
  int M, N, KT;
  int64_t R;
  int G, g;
  int64_t r_lo, r_hi;
  int band_lo;
};

// Completion of segment `s` (band band_lo + s of this workgroup's range) by
// the wave that counted last into it: adds the waves' slots in wave order,
// writes Y for a whole band, and otherwise stores the workgroup's fp32
// partial and, as the band's last arrival, adds the partials of its
// workgroups in order and writes Y.  Runs after the record loop.
__device__ __forceinline__ void sk_finish(const SkCtx& c, int s) {
  const int l = lane_id();
  const int col = l & 15;
  const int N = c.N, KT = c.KT;
  const int band = c.band_lo + s;
  const int64_t lo = max(c.r_lo, (int64_t)band * KT), hi = min(c.r_hi, (int64_t)(band + 1) * KT);
  const int64_t len = hi - lo;
  const float* sl = c.slots + (int64_t)s * kSkWaves * 16 * N;
  // wave v holds records of the segment when (v - wave of record lo) mod 8 < len
  const int wb = (int)((lo - c.r_lo) % kSkWaves);
  f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
  if (col < N) {
#pragma unroll
    for (int v = 0; v < kSkWaves; ++v)
      if ((v - wb + kSkWaves) % kSkWaves < len)
        sum += *reinterpret_cast<const f32x4*>(sl + (v * N + col) * 16 + 4 * (l >> 4));
  }
  const int mrow = band * 16 + 4 * (l >> 4);
  if (lo == (int64_t)band * KT && hi == (int64_t)(band + 1) * KT) {
    if (col < N)
      store4(c.Y + (int64_t)col * c.M + mrow,
             f32_to_bf16_bits(sum[0]) | (f32_to_bf16_bits(sum[1]) << 16),
             f32_to_bf16_bits(sum[2]) | (f32_to_bf16_bits(sum[3]) << 16), false);
    return;
  }
  // a band shared with other workgroups
  float* part = c.ws + (int64_t)(band == c.band_lo ? 2 * c.g : 2 * c.g + 1) * 16 * N;
  if (col < N) {
    uint64_t* pp = reinterpret_cast<uint64_t*>(part + col * 16 + 4 * (l >> 4));
    __hip_atomic_store(pp, (uint64_t)__float_as_uint(sum[0]) | ((uint64_t)__float_as_uint(sum[1]) << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(pp + 1, (uint64_t)__float_as_uint(sum[2]) | ((uint64_t)__float_as_uint(sum[3]) << 32),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  wait_stores();
  int prev = 0;
  if (l == 0)
    prev = __hip_atomic_fetch_add(&c.bcnt[band], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  prev = __builtin_amdgcn_readfirstlane(prev);
  const int ga = sk_wg_of((int64_t)band * KT, c.R, c.G);
  const int gb = sk_wg_of((int64_t)(band + 1) * KT - 1, c.R, c.G);
  if (prev != gb - ga) return;
  f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int gg = ga; gg <= gb; ++gg) {
    const int fb = (int)(((int64_t)gg * c.R / c.G) / KT);  // first band of workgroup gg
    const float* pq = c.ws + (int64_t)(fb == band ? 2 * gg : 2 * gg + 1) * 16 * N;
    if (col < N) {
      const uint16_t* q = reinterpret_cast<const uint16_t*>(pq + col * 16 + 4 * (l >> 4));
      const uint64_t x0 = load_agent(q), x1 = load_agent(q + 4);
      tot += f32x4{__uint_as_float((uint32_t)x0), __uint_as_float((uint32_t)(x0 >> 32)),
                   __uint_as_float((uint32_t)x1), __uint_as_float((uint32_t)(x1 >> 32))};
    }
  }
  if (col < N)
    store4(c.Y + (int64_t)col * c.M + mrow,
           f32_to_bf16_bits(tot[0]) | (f32_to_bf16_bits(tot[1]) << 16),
           f32_to_bf16_bits(tot[2]) | (f32_to_bf16_bits(tot[3]) << 16), false);
  if (l == 0) splitk_reset(&c.bcnt[band]);
}

template <int D, int XD>
__global__ __launch_bounds__(kSkWaves * 64, 6) void rgemm_sk_kernel(
    const uint8_t* fixed, const uint8_t* exps, const int32_t* eoff, int start_exp,
    const uint16_t* X, uint16_t* Y, int M, int N, int K, int64_t R, int G, int S, float* ws,
    int32_t* bcnt) {
  using SM = RSkSmem<XD>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  RTables& T = *reinterpret_cast<RTables*>(smem + SM::kTabAt);
  float* slots = reinterpret_cast<float*>(smem + SM::kSlotsAt);
  int32_t* scnt = reinterpret_cast<int32_t*>(smem + SM::kSlotsAt + (int64_t)S * kSkWaves * 64 * N);
  const RExp ex = r_exp(start_exp);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  const int KT = K >> 6;
  const int g = blockIdx.x;
  const int64_t r_lo = (int64_t)g * R / G, r_hi = (int64_t)(g + 1) * R / G;
  const int band_lo = (int)(r_lo / KT);
  // this wave's steps: records r_lo + w + 8 i, i < nw (a wave without one
  // runs the start-up on record r_lo and stops there)
  const int64_t first = r_lo + w < r_hi ? r_lo + w : r_lo;
  const int nw = r_lo + w < r_hi ? (int)((r_hi - r_lo - w + kSkWaves - 1) / kSkWaves) : 0;
  const int lastw = max(nw - 1, 0);
  uint8_t* stg = smem + w * SM::kStages * kExpStage;
  const __amdgpu_buffer_rsrc_t frs =
      r_buffer(fixed + r_lo * kRecBytes, r_range((r_hi - r_lo) * kRecBytes));
  const __amdgpu_buffer_rsrc_t xrs = r_buffer(X, 0x80000000u);
  // X: staged rows (XD > 0) or B fragments straight from memory (XD == 0),
  // as rgemm_kernel
  const int xrow = (XD * l) >> 5, xcol = (4 * XD * l) & 127;
  const uint32_t xloff = xrow < N ? 2u * (uint32_t)xrow * (uint32_t)K + (uint32_t)xcol : 0x80000000u;
  uint8_t* xst = smem + SM::kXAt + w * SM::kXStage;
  uint8_t* xst_w = xst + xrow * SM::kXPitch + xcol;
  const uint8_t* xst_r =
      xst + min(l & 15, (XD > 0 ? SM::kXRows : 1) - 1) * SM::kXPitch + 16 * (l >> 4);
  const uint32_t xoff = (l & 15) < N ? 2u * ((uint32_t)(l & 15) * (uint32_t)K + 8u * (uint32_t)(l >> 4))
                                     : 0x80000000u;

  // Per chunk of up to 64 steps, lane i holds step c0 + i's record (clamped
  // to the chunk): its K tile | (band - band_lo) << 24 (a range meets at
  // most kSkMaxSegments bands, K / 64 < 2^24) and its outlier offsets.
  int c0 = 0;
  int lmeta = 0, oe0 = 0, oe1 = 0;
  auto chunk_meta = [&](int last) {
    const int64_t rec = first + (int64_t)kSkWaves * (c0 + min(l, last));
    const int64_t band = rec / KT;
    lmeta = (int)(rec - band * KT) | ((int)(band - band_lo) << 24);
    oe0 = eoff[rec];
    oe1 = eoff[rec + 1];
  };
  RStage Rg[D];
  RMeta MT[D];
  XFrag<XD> xr[D];
  bf16x8 xc[2], xn[2];
#define SK_FIXED(J, R_)                                                                        \
  r_issue_fixed_r(frs, (uint32_t)(w + kSkWaves * (c0 + (J))) * (uint32_t)kRecBytes, R_)
#define SK_EXPS(J, R_, MT_)                                                                   \
  r_issue_exps(exps, __builtin_amdgcn_readlane(oe0, (J)), __builtin_amdgcn_readlane(oe1, (J)), R_, \
               MT_)
#define SK_XS(J, DST) \
  x_load<XD>(xrs, xloff, ((uint32_t)__builtin_amdgcn_readlane(lmeta, (J)) & 0xFFFFFFu) * 128u, DST)
#define SK_XB(J, DST)                                                                           \
  {                                                                                             \
    const uint32_t xs_ = ((uint32_t)__builtin_amdgcn_readlane(lmeta, (J)) & 0xFFFFFFu) * 128u;  \
    DST[0] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff, xs_, 0)); \
    DST[1] = __builtin_bit_cast(bf16x8,                                                         \
                                __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff + 64u, xs_, 0)); \
  }
  // Start-up (branch-free): chunk 0's metadata, the first D records' fixed
  // parts and X, then their outlier bytes; the decode table and the segment
  // counters are written before the barrier.
  {
    const int last = min(lastw, 63);
    chunk_meta(last);
#pragma unroll
    for (int k = 0; k < D; ++k) {
      SK_FIXED(min(k, last), Rg[k]);
      if constexpr (XD > 0) SK_XS(min(k, last), xr[k]);
    }
    if constexpr (XD == 0) SK_XB(0, xn);
#pragma unroll
    for (int k = 0; k < D; ++k) SK_EXPS(min(k, last), Rg[k], MT[k]);
    build_r_tables_exp(T, threadIdx.x, kSkWaves * 64, ex.lo, ex.hi);
    if ((int)threadIdx.x < S) scnt[threadIdx.x] = 0;
  }
  __syncthreads();

  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  int acc_band = -1;
  uint32_t done = 0;  // segments whose count this wave completed (bit s)
  const int col = l & 15;
  // A wave moving past band `band`: its sum into the segment's slot, then the
  // count; the wave that completes it finishes the segment after the loop.
  auto flush = [&](int band) {
    const int s_ = band - band_lo;
    const int64_t lo = max(r_lo, (int64_t)band * KT), hi = min(r_hi, (int64_t)(band + 1) * KT);
    const int need = (int)min<int64_t>(kSkWaves, hi - lo);
    float* sl = slots + ((int64_t)s_ * kSkWaves + w) * 16 * N;
    if (col < N) *reinterpret_cast<f32x4*>(sl + col * 16 + 4 * (l >> 4)) = acc;
    int prev = 0;
    if (l == 0)
      prev = __hip_atomic_fetch_add(&scnt[s_], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(prev) == need - 1) done |= 1u << s_;
  };

#define SK_STEP(J, SC, SN, RC, MC, RN, MN)                                                     \
  {                                                                                           \
    if constexpr (XD == 0) {                                                                  \
      xc[0] = xn[0];                                                                          \
      xc[1] = xn[1];                                                                          \
      SK_XB(min((J) + 1, last), xn);                                                          \
    }                                                                                         \
    r_stage_all(stg + (SN) * kExpStage, RN);                                                  \
    if constexpr (XD > 0) {                                                                   \
      x_stage<XD>(xst_w, xr[SC]);                                                             \
      xc[0] = *reinterpret_cast<const bf16x8*>(xst_r);                                        \
      xc[1] = *reinterpret_cast<const bf16x8*>(xst_r + 64);                                   \
    }                                                                                         \
    if ((J) < n) {                                                                            \
      const int bj_ = band_lo + (__builtin_amdgcn_readlane(lmeta, (J)) >> 24);                \
      if (bj_ != acc_band) {                                                                  \
        if (acc_band >= 0) flush(acc_band);                                                   \
        acc = f32x4{0.f, 0.f, 0.f, 0.f};                                                      \
        acc_band = bj_;                                                                       \
      }                                                                                       \
      u32x4 a0_, a1_;                                                                         \
      r_decode_staged<true>(T, ex, RC, MC, stg + ((J) & 1) * kExpStage, exps, a0_, a1_);      \
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a0_), xc[0], acc, 0, 0, 0);     \
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a1_), xc[1], acc, 0, 0, 0);     \
    }                                                                                         \
    SK_FIXED(min((J) + D, last), RC);                                                         \
    SK_EXPS(min((J) + D, last), RC, MC);                                                      \
    if constexpr (XD > 0) SK_XS(min((J) + D, last), xr[SC]);                                  \
  }
  for (; c0 < nw; c0 += 64) {
    const int n = min(nw - c0, 64);
    const int last = n - 1;
    if (c0 > 0) {
      chunk_meta(last);
#pragma unroll
      for (int k = 0; k < D; ++k) {
        SK_FIXED(min(k, last), Rg[k]);
        SK_EXPS(min(k, last), Rg[k], MT[k]);
        if constexpr (XD > 0) SK_XS(min(k, last), xr[k]);
      }
      if constexpr (XD == 0) SK_XB(0, xn);
    }
    r_stage_all(stg, Rg[0]);
    for (int j = 0; j < n; j += D) {
#pragma unroll
      for (int k = 0; k < D; ++k)
        SK_STEP(j + k, k, (k + 1) & 1, Rg[k], MT[k], Rg[(k + 1) % D], MT[(k + 1) % D]);
    }
  }
#undef SK_STEP
#undef SK_XB
#undef SK_XS
#undef SK_EXPS
#undef SK_FIXED
  if (acc_band >= 0) flush(acc_band);
  if (done) {
    const SkCtx cx{slots, ws, bcnt, Y, M, N, KT, R, G, g, r_lo, r_hi, band_lo};
    for (int s_ = 0; s_ < kSkMaxSegments; ++s_)
      if (done & (1u << s_)) sk_finish(cx, s_);
  }
}

// ---------------------------------------------------------------------------
// ZipGEMM over the re-tiled layout for wider batches (N > 16, and 4 <= N <= 16
// on grids of at least 7/8 of a workgroup per CU).  Workgroup =
// BANDS*PH waves on one 16*BANDS-row tile x one split-K slice x 16*NB
// columns; wave w decodes band w%BANDS of K tiles kb0 + PH*s + w/BANDS (PH
// interleaved phases).  Each X tile (16*NB x 64) is loaded once per
// workgroup into LDS and read by the BANDS band waves of its phase, so X
// crosses L2 1/BANDS as often as with 16-row workgroups.  Records are fetched
// RD steps ahead into registers and decoded one step before their MFMAs, X
// tiles two steps ahead into registers and one step ahead into a
// double-buffered LDS tile (B-fragment layout: xfrag_slot, zs_device.hpp);
// one barrier per step.
// ---------------------------------------------------------------------------
template <int NB, int BANDS, int PH>
struct RWideSmem {
  static constexpr int kXTile = 2 * NB * kXFragBlock;
  static constexpr int kX = PH * 2 * kXTile;   // [phase][buffer] tiles
  static constexpr int kStages = BANDS * PH * 2 * kExpStage;
  static constexpr int kMain = (int)sizeof(RTables) + kStages + kX;
  static constexpr int kRed = (PH - 1) * BANDS * NB * 64 * 16;
  static constexpr int kBytes = kMain > kRed ? kMain : kRed;
};

template <int NB, int BANDS, int PH, int RD>
__global__ __launch_bounds__(BANDS * PH * 64) void rgemm_wide_kernel(const uint8_t* fixed,
                                                              const uint8_t* exps,
                                                              const int32_t* eoff, int start_exp,
                                                              const uint16_t* X, uint16_t* Y,
                                                              int M, int N, int K,
                                                              int kb_per_split, SplitFix fx) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[RWideSmem<NB, BANDS, PH>::kBytes];
  constexpr int kXTile = RWideSmem<NB, BANDS, PH>::kXTile;
  RTables& T = *reinterpret_cast<RTables*>(smem);
  const RExp ex = r_exp(start_exp);

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  const int q = w % BANDS, p = w / BANDS;
  const int t = threadIdx.x % (BANDS * 64);  // thread index within the phase
  uint8_t* stage0 = smem + sizeof(RTables) + w * 2 * kExpStage;
  uint8_t* stage1 = stage0 + kExpStage;
  uint8_t* xbase =
      smem + sizeof(RTables) + RWideSmem<NB, BANDS, PH>::kStages + p * 2 * kXTile;
  uint8_t* xb0 = xbase;
  uint8_t* xb1 = xbase + kXTile;
  const int band = blockIdx.x * BANDS + q;
  const int split = blockIdx.y;
  const int n0 = blockIdx.z * NB * 16;
  const int KT = K >> 6;
  const int kb0 = split * kb_per_split;
  const int kb1 = min(kb0 + kb_per_split, KT);
  const int span = max(kb1 - kb0, 0);
  const int steps = (span + PH - 1) / PH;         // same for every phase
  const int cnt = (span - p + PH - 1) / PH;       // valid tiles of this phase
  // K tile of step j of this phase, clamped into the slice (clamped steps
  // only repeat an in-bounds load and skip the decode; an empty slice,
  // kb0 >= KT, clamps to the last tile of the row).
  auto tile_of = [&](int j) { return min(kb0 + PH * j + p, kb1 - 1); };
  const int64_t rowrec = (int64_t)band * KT;
  // Buffer resources built once (the band's records, X);
  // per-record and per-tile positions go into the load offsets.
  const __amdgpu_buffer_rsrc_t frs = r_buffer(fixed + rowrec * kRecBytes, (uint32_t)KT * kRecBytes);
  const __amdgpu_buffer_rsrc_t xrs = r_buffer(X, 0x80000000u);

  // X tile loads of this thread: chunk c = t + 64*BANDS*i, row c/8, 16-byte
  // column c%8 (128*NB chunks per tile; threads past them load and drop).
  // Sources are 32-bit byte offsets into X (rows clamped to N - 1), the
  // tile's column goes into the scalar offset (the host keeps N * K * 2
  // below 2^31).
  constexpr int kXC = (2 * NB + BANDS - 1) / BANDS;  // chunks per thread
  uint32_t xsrc[kXC];
  int xdst[kXC];
#pragma unroll
  for (int i = 0; i < kXC; ++i) {
    const int c = t + 64 * BANDS * i;
    const int row = min(c >> 3, 16 * NB - 1), cc = c & 7;
    xsrc[i] = 2u * ((uint32_t)min(n0 + row, N - 1) * (uint32_t)K + 8u * (uint32_t)cc);
    xdst[i] = c < 128 * NB ? 16 * xfrag_slot(row >> 4, cc >> 2, cc & 3, row & 15) : -1;
  }
  f32x4 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  // B fragment byte offsets of this lane in the block of nb = 0, h = 0 / 1
  const int brd = 16 * xfrag_slot(0, 0, l >> 4, l & 15);
  const int brd1 = 16 * xfrag_slot(0, 1, l >> 4, l & 15);

  // Outlier offsets of a tile through the scalar cache (the address is
  // uniform per wave), fetched one step before the record's loads go out.
  // (Vector loads of 64 tiles' offsets, reloaded inside the step loop, made
  // the compiler wait for every outstanding vector load before each step's
  // record loads.)
  using ci32 = const __attribute__((address_space(4))) int32_t;
  ci32* eoffs = (ci32*)(eoff + rowrec);
  int pe0, pe1;
  auto offs = [&](int j) {
    const int ti = tile_of(j);
    pe0 = eoffs[ti];
    pe1 = eoffs[ti + 1];
  };
  auto issue = [&](int j, RStage& R, RMeta& Mt) {
    r_issue_fixed_r(frs, (uint32_t)tile_of(j) * kRecBytes, R);
    r_issue_exps(exps, pe0, pe1, R, Mt);
  };
  auto xload = [&](int j, u32x4 (&XR)[kXC]) {
    const uint32_t xs = (uint32_t)tile_of(j) * 128u;
#pragma unroll
    for (int i = 0; i < kXC; ++i) XR[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xsrc[i], xs, 0);
  };
  auto xwrite = [&](uint8_t* xb, const u32x4 (&XR)[kXC]) {
#pragma unroll
    for (int i = 0; i < kXC; ++i)
      if (2 * NB >= BANDS * (i + 1) || xdst[i] >= 0)
        *reinterpret_cast<u32x4*>(xb + xdst[i]) = XR[i];
  };

  static_assert(RD % 2 == 0, "record ring of an even number of steps");
  RStage R[RD];
  RMeta MT[RD];
  u32x4 XA[kXC], XB[kXC];
  // Start-up, branch-free (an empty slice runs it on clamped tiles and then
  // no steps): the first outlier offsets, the first records' fixed parts and
  // two X tiles go out together; the outlier bytes follow as soon as the
  // offsets land; the decode table is computed meanwhile.
  {
    int se0[RD + 1], se1[RD + 1];
#pragma unroll
    for (int k = 0; k <= RD; ++k) {
      const int ti = tile_of(k);
      se0[k] = eoffs[ti];
      se1[k] = eoffs[ti + 1];
    }
#pragma unroll
    for (int k = 0; k < RD; ++k) r_issue_fixed_r(frs, (uint32_t)tile_of(k) * kRecBytes, R[k]);
    xload(0, XA);
    xload(1, XB);
#pragma unroll
    for (int k = 0; k < RD; ++k) r_issue_exps(exps, se0[k], se1[k], R[k], MT[k]);
    pe0 = se0[RD];
    pe1 = se1[RD];
    build_r_tables_exp(T, threadIdx.x, BANDS * PH * 64, ex.lo, ex.hi);
  }
  r_stage_all(stage0, R[0]);
  xwrite(xb0, XA);
  xload(2, XA);
  __syncthreads();  // decode tables and X tile 0 visible

  // NB = 8: the step's sixteen B fragments are read from LDS before the
  // decode, so their latency hides behind it instead of stalling each MFMA
  // pair, and the first K half of every column block goes to the MFMA unit
  // before the second, so consecutive MFMAs never depend on each other
  // (N = 128: 3-11% faster; at NB = 4 the extra registers cost more than
  // the latency they hide: 1-7% slower, so it keeps one read pair per
  // column block next to its MFMAs).  Not with three K phases: the 12-wave
  // workgroup needs the registers (<= 170 VGPRs for 3 waves per SIMD).
  constexpr bool kEarlyB = NB >= 8 && PH < 3;
  auto b_read = [&](const uint8_t* xcur, bf16x8 (&b0)[NB], bf16x8 (&b1)[NB]) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const uint8_t* bp = xcur + nb * kXFragBlock * 2;
      b0[nb] = *reinterpret_cast<const bf16x8*>(bp + brd);
      b1[nb] = *reinterpret_cast<const bf16x8*>(bp + brd1);
    }
  };
  auto mfma_step = [&](const uint8_t* xcur, const bf16x8 (&b0)[NB], const bf16x8 (&b1)[NB],
                       const u32x4& a0, const u32x4& a1) {
    if constexpr (kEarlyB) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a0), b0[nb], acc[nb], 0, 0, 0);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a1), b1[nb], acc[nb], 0, 0, 0);
    } else {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint8_t* bp = xcur + nb * kXFragBlock * 2;
        const bf16x8 x0 = *reinterpret_cast<const bf16x8*>(bp + brd);
        const bf16x8 x1 = *reinterpret_cast<const bf16x8*>(bp + brd1);
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a0), x0, acc[nb], 0, 0, 0);
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a1), x1, acc[nb], 0, 0, 0);
      }
    }
  };

  // Software pipeline: step s runs the MFMAs of record s (decoded in step
  // s - 1) and decodes record s + 1, so one wave's decode VALU work overlaps
  // its own matrix-core work (N = 128: 3-9% faster than decoding and
  // multiplying the same record in one step).
  u32x4 ac0, ac1;
  if (0 < cnt) r_decode_staged<true>(T, ex, R[0], MT[0], stage0, exps, ac0, ac1);
#define RW_STEP(S, CUR, NXT, XCUR, RC, MC, RN, MN, XRN, XRC)                           \
  {                                                                                  \
    const RStage cn_ = RN;                                                           \
    const RMeta mn_ = MN;                                                            \
    bf16x8 b0_[NB], b1_[NB];                                                         \
    if constexpr (kEarlyB) b_read(XCUR, b0_, b1_);                                   \
    r_stage_all(NXT, cn_);                                                           \
    issue((S) + RD, RC, MC);                                                         \
    offs((S) + RD + 1);                                                              \
    if ((S) < cnt) mfma_step(XCUR, b0_, b1_, ac0, ac1);                              \
    if ((S) + 1 < cnt) r_decode_staged<true>(T, ex, cn_, mn_, NXT, exps, ac0, ac1);  \
    xwrite((XCUR) == xb0 ? xb1 : xb0, XRN);                                          \
    xload((S) + 3, XRC);                                                             \
    __syncthreads();                                                                 \
  }
  // Steps s <= steps - 3 have record s and s + 1 in every phase (cnt >=
  // steps - 1): no step condition, and the decode and MFMAs of a step share
  // one basic block (records with unstaged outlier bytes take a branch).
#define RW_MAIN(S, CUR, NXT, XCUR, RC, MC, RN, MN, XRN, XRC)                           \
  {                                                                                  \
    const RStage cn_ = RN;                                                           \
    const RMeta mn_ = MN;                                                            \
    bf16x8 b0_[NB], b1_[NB];                                                         \
    if constexpr (kEarlyB) b_read(XCUR, b0_, b1_);                                   \
    r_stage_all(NXT, cn_);                                                           \
    issue((S) + RD, RC, MC);                                                         \
    offs((S) + RD + 1);                                                              \
    u32x4 n0_, n1_;                                                                  \
    if (r_staged(mn_)) {                                                             \
      r_decode<true>(T, ex, cn_.r, NXT, mn_.rel, n0_, n1_);                          \
      mfma_step(XCUR, b0_, b1_, ac0, ac1);                                           \
    } else {                                                                         \
      r_decode<true>(T, ex, cn_.r, exps + mn_.e0, 0, n0_, n1_);                      \
      mfma_step(XCUR, b0_, b1_, ac0, ac1);                                           \
    }                                                                                \
    ac0 = n0_;                                                                       \
    ac1 = n1_;                                                                       \
    xwrite((XCUR) == xb0 ? xb1 : xb0, XRN);                                          \
    xload((S) + 3, XRC);                                                             \
    __syncthreads();                                                                 \
  }
  // Step s reads X buffer s%2; X registers: XB holds step s+1, XA step s+2
  // at the start of an even step (roles swap on odd steps).
  // Record ring: record s + 1 sits in R[(s + 1) % RD] during step s; the
  // slot of record s (decoded in step s - 1) is refilled with record s + RD.
  int s = 0;
  for (; s + RD <= steps - 2; s += RD) {
#pragma unroll
    for (int k = 0; k < RD; k += 2) {
      RW_MAIN(s + k, stage0, stage1, xb0, R[k], MT[k], R[k + 1], MT[k + 1], XB, XB);
      RW_MAIN(s + k + 1, stage1, stage0, xb1, R[k + 1], MT[k + 1], R[(k + 2) % RD],
              MT[(k + 2) % RD], XA, XA);
    }
  }
  for (; s < steps; s += RD) {
#pragma unroll
    for (int k = 0; k < RD; k += 2) {
      if (s + k < steps)
        RW_STEP(s + k, stage0, stage1, xb0, R[k], MT[k], R[k + 1], MT[k + 1], XB, XB);
      if (s + k + 1 < steps)
        RW_STEP(s + k + 1, stage1, stage0, xb1, R[k + 1], MT[k + 1], R[(k + 2) % RD],
                MT[(k + 2) % RD], XA, XA);
    }
  }
#undef RW_MAIN
#undef RW_STEP

  // Phases 1..PH-1 hand their sums to phase 0 through LDS (added in phase
  // order, so the result is deterministic); phase 0 writes its band.
  f32x4* red = reinterpret_cast<f32x4*>(smem);
  if (p > 0) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) red[(((p - 1) * BANDS + q) * NB + nb) * 64 + l] = acc[nb];
  }
  __syncthreads();
  if (p == 0) {
    uint16_t* out = Y + (int64_t)split * M * N;
    const int mrow = band * 16 + 4 * (l >> 4);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      f32x4 v = acc[nb];
#pragma unroll
      for (int pp = 1; pp < PH; ++pp) v += red[(((pp - 1) * BANDS + q) * NB + nb) * 64 + l];
      const int n = n0 + nb * 16 + (l & 15);
      if (n < N) {
        const uint32_t lo = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
        const uint32_t hi = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
        store4(out + (int64_t)n * M + mrow, lo, hi, fx.cnt != nullptr);
      }
    }
  }
  if (fx.cnt)
    splitk_finish<16 * BANDS, 16 * NB, BANDS * PH * 64>(fx, Y, M, N, blockIdx.x * BANDS * 16,
                                                          n0, p == 0);
}

__global__ __launch_bounds__(256) void rsplitk_reduce_kernel(uint16_t* C, const uint16_t* WS,
                                                             int64_t mn, int split_k) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= mn) return;
  if (i + 8 <= mn) {
    float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < split_k; ++k) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(WS + k * mn + i);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s[2 * j] += bf16_bits_to_f32(v[j] & 0xFFFFu);
        s[2 * j + 1] += bf16_bits_to_f32(v[j] >> 16);
      }
    }
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = f32_to_bf16_bits(s[2 * j]) | (f32_to_bf16_bits(s[2 * j + 1]) << 16);
    *reinterpret_cast<u32x4*>(C + i) = o;
  } else {
    for (int64_t e = i; e < mn; ++e) {
      float s = 0.f;
      for (int k = 0; k < split_k; ++k) s += bf16_bits_to_f32(WS[k * mn + e]);
      C[e] = (uint16_t)f32_to_bf16_bits(s);
    }
  }
}

static int r_grid(int64_t nrec, int waves_per_block) {
  const int64_t blocks = (nrec + waves_per_block - 1) / waves_per_block;
  return (int)std::max<int64_t>(1, std::min<int64_t>(blocks, 256 * 64));
}

template <int F, int NB, int kWaves, int XD>
static hipError_t launch_rgemm_x(hipStream_t st, const uint8_t* fixed, const uint8_t* exps,
                                 const int32_t* eoff, int start_exp, const uint16_t* X,
                                 uint16_t* Y, int M, int N, int K, int split_k, int kb_per_split,
                                 SplitFix fx) {
  // records in flight per wave: 4 with one band per wave (more bytes in
  // flight at the same occupancy: 1-2.5 us faster on the 14336- to
  // 28672-row shapes), 3 with two (VGPRs)
  constexpr int kDepth = F == 1 ? 4 : 3;
  dim3 grid((M / 16 + F - 1) / F, split_k, (N + NB * 16 - 1) / (NB * 16));
  hipLaunchKernelGGL((rgemm_kernel<F, NB, kWaves, kDepth, XD>), grid, dim3(kWaves * 64), 0, st,
                     fixed, exps, eoff, start_exp, X, Y, M, N, K, kb_per_split, fx);
  return hipGetLastError();
}

// Narrow kernels: X staged through LDS for N <= 8 (one, two or four dwords
// per lane per tile: 2-9% faster than B fragments from memory on the
// Llama-3 / 3.1 shapes), B fragments straight from memory above.
template <int F, int NB, int kWaves>
static hipError_t launch_rgemm(hipStream_t st, const uint8_t* fixed, const uint8_t* exps,
                               const int32_t* eoff, int start_exp, const uint16_t* X,
                               uint16_t* Y, int M, int N, int K, int split_k, int kb_per_split,
                               SplitFix fx) {
  if (NB == 1 && N <= 2)
    return launch_rgemm_x<F, NB, kWaves, 1>(st, fixed, exps, eoff, start_exp, X, Y, M, N, K,
                                            split_k, kb_per_split, fx);
  if (NB == 1 && N <= 4)
    return launch_rgemm_x<F, NB, kWaves, 2>(st, fixed, exps, eoff, start_exp, X, Y, M, N, K,
                                            split_k, kb_per_split, fx);
  if (NB == 1 && N <= 8)
    return launch_rgemm_x<F, NB, kWaves, 4>(st, fixed, exps, eoff, start_exp, X, Y, M, N, K,
                                            split_k, kb_per_split, fx);
  return launch_rgemm_x<F, NB, kWaves, 0>(st, fixed, exps, eoff, start_exp, X, Y, M, N, K,
                                          split_k, kb_per_split, fx);
}

// Stream-K narrow ZipGEMM: grid, segment slots and LDS of one launch.
struct SkPlan {
  int G = 0;          // workgroups (0: not applicable, use the band kernels)
  int S = 0;          // segment slots per workgroup
  int64_t lds = 0;    // dynamic LDS bytes
};

template <int XD>
static SkPlan sk_plan_x(int M, int N, int K) {
  SkPlan p;
  const int KT = K / 64;
  const int64_t R = (int64_t)(M / 16) * KT;
  if (N < 1 || N > 16 || R <= 0) return p;
  // the most workgroups per CU (of kSkPerCu) whose LDS fits one CU together,
  // so that the whole grid is resident in one round
  for (int per = kSkPerCu; per >= 1; --per) {
    const int64_t G = std::min<int64_t>((int64_t)device_cu_count() * per, R);
    // a range of at most L = ceil(R / G) records meets at most
    // ceil((L - 1) / KT) + 1 bands
    const int64_t L = (R + G - 1) / G;
    const int64_t S = (L - 1 + KT - 1) / KT + 1;
    if (S > kSkMaxSegments) continue;
    const int64_t lds = RSkSmem<XD>::bytes((int)S, N);
    if (lds > 65536 || lds * per > kCuLdsBytes) continue;
    p.G = (int)G;
    p.S = (int)S;
    p.lds = lds;
    return p;
  }
  return p;
}

static SkPlan sk_plan(int M, int N, int K) {
  if (N <= 2) return sk_plan_x<1>(M, N, K);
  if (N <= 4) return sk_plan_x<2>(M, N, K);
  if (N <= 8) return sk_plan_x<4>(M, N, K);
  return sk_plan_x<0>(M, N, K);
}

// fp32 partial slots of the stream-K kernel: two per workgroup
static int64_t sk_workspace_bytes(const SkPlan& p, int N) { return (int64_t)2 * p.G * 16 * N * 4; }

template <int XD>
static hipError_t launch_sk_x(hipStream_t st, const SkPlan& p, const uint8_t* fixed,
                              const uint8_t* exps, const int32_t* eoff, int start_exp,
                              const uint16_t* X, uint16_t* Y, int M, int N, int K, float* ws,
                              int32_t* cnt) {
  const int64_t R = (int64_t)(M / 16) * (K / 64);
  hipLaunchKernelGGL((rgemm_sk_kernel<4, XD>), dim3(p.G), dim3(kSkWaves * 64), (size_t)p.lds, st,
                     fixed, exps, eoff, start_exp, X, Y, M, N, K, R, p.G, p.S, ws, cnt);
  return hipGetLastError();
}

constexpr int kWideDepth = 2;  // records in flight per wave (ring of RD steps)

// ---------------------------------------------------------------------------
// Wide batches with two bands per wave: as rgemm_wide_kernel, but each wave
// decodes the records of two bands for the same K tile and feeds every X
// fragment it reads from LDS to both, halving the LDS bytes per record (the
// X reads dominate the LDS traffic at N >= 64).  Workgroup = BANDS bands x PH
// K phases, BANDS/2 waves per phase.
// ---------------------------------------------------------------------------
template <int NB, int BANDS, int PH>
struct RWide2Smem {
  static constexpr int kXTile = 2 * NB * kXFragBlock;
  static constexpr int kWP = BANDS / 2;                  // waves per phase
  static constexpr int kStageBytes = kWP * PH * 2 * 2 * kExpStage;  // [wave][buf][band]
  static constexpr int kX = PH * 2 * kXTile;             // [phase][buffer] tiles
  static constexpr int kMain = kStageBytes + kX + (int)sizeof(RTables);
  static constexpr int kRed = (PH - 1) * kWP * 2 * NB * 64 * 16;
  static constexpr int kBytes = kMain > kRed ? kMain : kRed;
};

template <int NB, int BANDS, int PH>
__global__ __launch_bounds__(BANDS / 2 * PH * 64) void rgemm_wide2_kernel(
    const uint8_t* fixed, const uint8_t* exps, const int32_t* eoff, int start_exp,
    const uint16_t* X, uint16_t* Y, int M, int N, int K, int kb_per_split, SplitFix fx) {
  using S = RWide2Smem<NB, BANDS, PH>;
  constexpr int kXTile = S::kXTile;
  constexpr int WP = S::kWP;
  __shared__ __attribute__((aligned(16))) uint8_t smem[S::kBytes];
  RTables& T = *reinterpret_cast<RTables*>(smem + S::kStageBytes + S::kX);
  const RExp ex = r_exp(start_exp);

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  const int q = w % WP, p = w / WP;
  const int t = threadIdx.x % (WP * 64);  // thread index within the phase
  // stage (buffer b, band f) of this wave
  uint8_t* stg = smem + w * 4 * kExpStage;
  auto stage_of = [&](int b, int f) { return stg + (2 * b + f) * kExpStage; };
  uint8_t* xbase = smem + S::kStageBytes + p * 2 * kXTile;
  uint8_t* xb0 = xbase;
  uint8_t* xb1 = xbase + kXTile;
  const int band0 = blockIdx.x * BANDS + 2 * q;
  const int split = blockIdx.y;
  const int n0 = blockIdx.z * NB * 16;
  const int KT = K >> 6;
  const int kb0 = split * kb_per_split;
  const int kb1 = min(kb0 + kb_per_split, KT);
  const int span = max(kb1 - kb0, 0);
  const int steps = (span + PH - 1) / PH;         // same for every phase
  const int cnt = (span - p + PH - 1) / PH;       // valid tiles of this phase
  auto tile_of = [&](int j) { return min(kb0 + PH * j + p, kb1 - 1); };
  const int64_t rowrec[2] = {(int64_t)band0 * KT, (int64_t)(band0 + 1) * KT};
  // Buffer resources built once (each band's records, X).
  const __amdgpu_buffer_rsrc_t frs[2] = {
      r_buffer(fixed + rowrec[0] * kRecBytes, (uint32_t)KT * kRecBytes),
      r_buffer(fixed + rowrec[1] * kRecBytes, (uint32_t)KT * kRecBytes)};
  const __amdgpu_buffer_rsrc_t xrs = r_buffer(X, 0x80000000u);

  constexpr int kXC = (2 * NB + WP - 1) / WP;  // 16-byte X chunks per thread
  uint32_t xsrc[kXC];
  int xdst[kXC];
#pragma unroll
  for (int i = 0; i < kXC; ++i) {
    const int c = t + 64 * WP * i;
    const int row = min(c >> 3, 16 * NB - 1), cc = c & 7;
    xsrc[i] = 2u * ((uint32_t)min(n0 + row, N - 1) * (uint32_t)K + 8u * (uint32_t)cc);
    xdst[i] = c < 128 * NB ? 16 * xfrag_slot(row >> 4, cc >> 2, cc & 3, row & 15) : -1;
  }
  f32x4 acc[2][NB];
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[f][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int brd = 16 * xfrag_slot(0, 0, l >> 4, l & 15);
  const int brd1 = 16 * xfrag_slot(0, 1, l >> 4, l & 15);
  // NB = 8: all B fragments of a step read before the decodes (see
  // rgemm_wide_kernel); NB = 4 keeps them next to their MFMAs, where the
  // extra registers would cost a wave per SIMD (measured 12-16% slower).
  constexpr bool kEarlyB2 = NB >= 8;

  int oe0[2] = {0, 0}, oe1[2] = {0, 0}, ochunk = -1;
  auto issue = [&](int j, RStage (&R)[2], RMeta (&Mt)[2]) {
    const int c = j & ~63;
    if (c != ochunk) {
      ochunk = c;
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const int64_t ri = rowrec[f] + tile_of(c + l);
        oe0[f] = eoff[ri];
        oe1[f] = eoff[ri + 1];
      }
    }
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      r_issue_fixed_r(frs[f], (uint32_t)tile_of(j) * kRecBytes, R[f]);
      r_issue_exps(exps, __builtin_amdgcn_readlane(oe0[f], j - c),
                     __builtin_amdgcn_readlane(oe1[f], j - c), R[f], Mt[f]);
    }
  };
  auto xload = [&](int j, u32x4 (&XR)[kXC]) {
    const uint32_t xs = (uint32_t)tile_of(j) * 128u;
#pragma unroll
    for (int i = 0; i < kXC; ++i) XR[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, xsrc[i], xs, 0);
  };
  auto xwrite = [&](uint8_t* xb, const u32x4 (&XR)[kXC]) {
#pragma unroll
    for (int i = 0; i < kXC; ++i)
      if (2 * NB >= WP * (i + 1) || xdst[i] >= 0) *reinterpret_cast<u32x4*>(xb + xdst[i]) = XR[i];
  };

  {
    RStage R0[2], R1[2];
    RMeta M0[2], M1[2];
    u32x4 XA[kXC], XB[kXC];
    // Start-up, branch-free (an empty slice, kb0 >= KT, runs it on the
    // clamped last tile and then no steps): offsets, fixed parts and two X
    // tiles in flight together; outlier bytes as soon as the offsets land;
    // the decode table is computed meanwhile.
    {
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const int64_t ri = rowrec[f] + tile_of(l);
        oe0[f] = eoff[ri];
        oe1[f] = eoff[ri + 1];
      }
      ochunk = 0;
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        r_issue_fixed_r(frs[f], (uint32_t)tile_of(0) * kRecBytes, R0[f]);
        r_issue_fixed_r(frs[f], (uint32_t)tile_of(1) * kRecBytes, R1[f]);
      }
      xload(0, XA);
      xload(1, XB);
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        r_issue_exps(exps, __builtin_amdgcn_readlane(oe0[f], 0),
                     __builtin_amdgcn_readlane(oe1[f], 0), R0[f], M0[f]);
        r_issue_exps(exps, __builtin_amdgcn_readlane(oe0[f], 1),
                     __builtin_amdgcn_readlane(oe1[f], 1), R1[f], M1[f]);
      }
      build_r_tables_exp(T, threadIdx.x, BANDS / 2 * PH * 64, ex.lo, ex.hi);
    }
#pragma unroll
    for (int f = 0; f < 2; ++f) r_stage_all(stage_of(0, f), R0[f]);
    xwrite(xb0, XA);
    xload(2, XA);
    __syncthreads();

#define RW2_STEP(S_, BC, XCUR, RC, MC, RN, MN, XRN, XRC)                                  \
  {                                                                                     \
    RStage cs_[2] = {RC[0], RC[1]};                                                     \
    RMeta cm_[2] = {MC[0], MC[1]};                                                      \
    bf16x8 eb0_[NB], eb1_[NB];                                                          \
    if constexpr (kEarlyB2) {                                                           \
      _Pragma("unroll") for (int nb_ = 0; nb_ < NB; ++nb_) {                            \
        const uint8_t* bp_ = XCUR + nb_ * kXFragBlock * 2;                              \
        eb0_[nb_] = *reinterpret_cast<const bf16x8*>(bp_ + brd);                        \
        eb1_[nb_] = *reinterpret_cast<const bf16x8*>(bp_ + brd1);                       \
      }                                                                                 \
    }                                                                                   \
    _Pragma("unroll") for (int f_ = 0; f_ < 2; ++f_)                                    \
      r_stage_all(stage_of((BC) ^ 1, f_), RN[f_]);                                      \
    issue((S_) + 2, RC, MC);                                                            \
    if ((S_) < cnt) {                                                                   \
      u32x4 a0_[2], a1_[2];                                                             \
      _Pragma("unroll") for (int f_ = 0; f_ < 2; ++f_)                                  \
        r_decode_staged<true>(T, ex, cs_[f_], cm_[f_], stage_of(BC, f_), exps, a0_[f_], \
                              a1_[f_]);                                                 \
      if constexpr (kEarlyB2) {                                                         \
        _Pragma("unroll") for (int f_ = 0; f_ < 2; ++f_)                                \
          _Pragma("unroll") for (int nb_ = 0; nb_ < NB; ++nb_)                          \
            acc[f_][nb_] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(                     \
                as_bf16x8(a0_[f_]), eb0_[nb_], acc[f_][nb_], 0, 0, 0);                  \
        _Pragma("unroll") for (int f_ = 0; f_ < 2; ++f_)                                \
          _Pragma("unroll") for (int nb_ = 0; nb_ < NB; ++nb_)                          \
            acc[f_][nb_] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(                     \
                as_bf16x8(a1_[f_]), eb1_[nb_], acc[f_][nb_], 0, 0, 0);                  \
      } else {                                                                          \
        _Pragma("unroll") for (int nb_ = 0; nb_ < NB; ++nb_) {                          \
          const uint8_t* bp_ = XCUR + nb_ * kXFragBlock * 2;                            \
          const bf16x8 b0_ = *reinterpret_cast<const bf16x8*>(bp_ + brd);               \
          const bf16x8 b1_ = *reinterpret_cast<const bf16x8*>(bp_ + brd1);              \
          _Pragma("unroll") for (int f_ = 0; f_ < 2; ++f_) {                            \
            acc[f_][nb_] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(                     \
                as_bf16x8(a0_[f_]), b0_, acc[f_][nb_], 0, 0, 0);                        \
            acc[f_][nb_] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(                     \
                as_bf16x8(a1_[f_]), b1_, acc[f_][nb_], 0, 0, 0);                        \
          }                                                                             \
        }                                                                               \
      }                                                                                 \
    }                                                                                   \
    xwrite((XCUR) == xb0 ? xb1 : xb0, XRN);                                             \
    xload((S_) + 3, XRC);                                                               \
    __syncthreads();                                                                    \
  }
    for (int s2 = 0; s2 < steps; s2 += 2) {
      RW2_STEP(s2, 0, xb0, R0, M0, R1, M1, XB, XB);
      if (s2 + 1 < steps) RW2_STEP(s2 + 1, 1, xb1, R1, M1, R0, M0, XA, XA);
    }
#undef RW2_STEP
  }

  f32x4* red = reinterpret_cast<f32x4*>(smem);
  if (p > 0) {
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        red[((((p - 1) * WP + q) * 2 + f) * NB + nb) * 64 + l] = acc[f][nb];
  }
  __syncthreads();
  if (p == 0) {
    uint16_t* out = Y + (int64_t)split * M * N;
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const int mrow = (band0 + f) * 16 + 4 * (l >> 4);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        f32x4 v = acc[f][nb];
#pragma unroll
        for (int pp = 1; pp < PH; ++pp) v += red[((((pp - 1) * WP + q) * 2 + f) * NB + nb) * 64 + l];
        const int n = n0 + nb * 16 + (l & 15);
        if (n < N) {
          const uint32_t lo = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
          const uint32_t hi = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
          store4(out + (int64_t)n * M + mrow, lo, hi, fx.cnt != nullptr);
        }
      }
    }
  }
  if (fx.cnt)
    splitk_finish<16 * BANDS, 16 * NB, BANDS / 2 * PH * 64>(fx, Y, M, N, blockIdx.x * BANDS * 16,
                                                              n0, p == 0);
}

template <int NB, int BANDS, int PH>
static hipError_t launch_rwide2(hipStream_t st, const uint8_t* fixed, const uint8_t* exps,
                                const int32_t* eoff, int start_exp, const uint16_t* X,
                                uint16_t* Y, int M, int N, int K, int split_k, int kb_per_split,
                                SplitFix fx) {
  dim3 grid(M / (16 * BANDS), split_k, (N + NB * 16 - 1) / (NB * 16));
  hipLaunchKernelGGL((rgemm_wide2_kernel<NB, BANDS, PH>), grid, dim3(BANDS / 2 * PH * 64), 0, st,
                     fixed, exps, eoff, start_exp, X, Y, M, N, K, kb_per_split, fx);
  return hipGetLastError();
}

template <int NB, int BANDS, int PH>
static hipError_t launch_rwide(hipStream_t st, const uint8_t* fixed, const uint8_t* exps,
                               const int32_t* eoff, int start_exp, const uint16_t* X,
                               uint16_t* Y, int M, int N, int K, int split_k, int kb_per_split,
                               SplitFix fx) {
  dim3 grid(M / (16 * BANDS), split_k, (N + NB * 16 - 1) / (NB * 16));
  hipLaunchKernelGGL((rgemm_wide_kernel<NB, BANDS, PH, kWideDepth>), grid, dim3(BANDS * PH * 64), 0, st, fixed,
                     exps, eoff, start_exp, X, Y, M, N, K, kb_per_split, fx);
  return hipGetLastError();
}

static int status_of(hipError_t e) { return e == hipSuccess ? ZS_OK : (int)e; }

static bool shape_ok(int M, int K) { return M > 0 && K > 0 && M % 64 == 0 && K % 64 == 0; }

}  // namespace zs

using namespace zs;

extern "C" int64_t zs_retiled_num_records(int M, int K) {
  if (!shape_ok(M, K)) return ZS_E_INVAL;
  return (int64_t)(M / 16) * (K / 64);
}

extern "C" int64_t zs_retiled_fixed_bytes(int M, int K) {
  if (!shape_ok(M, K)) return ZS_E_INVAL;
  return (int64_t)(M / 16) * (K / 64) * kRecBytes;
}

extern "C" int zs_compress_retiled_count_gpu(void* stream, const uint16_t* d_input, int M, int K,
                                             const int32_t* d_top_exponents, int32_t* d_counts,
                                             int32_t* d_eoff, int64_t* d_total) {
  if (!shape_ok(M, K) || !d_input || !d_top_exponents || !d_counts || !d_eoff || !d_total)
    return ZS_E_INVAL;
  if ((reinterpret_cast<uintptr_t>(d_input) & 15) != 0) return ZS_E_INVAL;
  const int64_t nrec = (int64_t)(M / 16) * (K / 64);
  if (nrec + 1 > INT32_MAX) return ZS_E_OVERFLOW;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(rcount_kernel, dim3(r_grid(nrec, 4)), dim3(256), 0, st, d_input, M, K,
                     d_top_exponents, d_counts);
  launch_rscan(st, d_counts, nrec, d_eoff, d_total);
  return status_of(hipGetLastError());
}

extern "C" int zs_compress_retiled_emit_gpu(void* stream, const uint16_t* d_input, int M, int K,
                                            const int32_t* d_top_exponents, const int32_t* d_eoff,
                                            uint8_t* d_fixed, uint8_t* d_exps) {
  if (!shape_ok(M, K) || !d_input || !d_top_exponents || !d_eoff || !d_fixed || !d_exps)
    return ZS_E_INVAL;
  if ((reinterpret_cast<uintptr_t>(d_input) & 15) || (reinterpret_cast<uintptr_t>(d_fixed) & 15))
    return ZS_E_INVAL;
  const int64_t nrec = (int64_t)(M / 16) * (K / 64);
  hipLaunchKernelGGL(remit_kernel, dim3(r_grid(nrec, 4)), dim3(256), 0, (hipStream_t)stream,
                     d_input, M, K, d_top_exponents, d_eoff, d_fixed, d_exps);
  return status_of(hipGetLastError());
}

extern "C" int zs_compress_retiled_fixed_gpu(void* stream, const uint16_t* d_input, int M, int K,
                                             const int32_t* d_top_exponents, uint8_t* d_fixed,
                                             int32_t* d_counts, int32_t* d_eoff, int64_t* d_total,
                                             uint8_t* d_tmp) {
  if (!shape_ok(M, K) || !d_input || !d_top_exponents || !d_fixed || !d_counts || !d_eoff ||
      !d_total || !d_tmp)
    return ZS_E_INVAL;
  if ((reinterpret_cast<uintptr_t>(d_input) & 15) || (reinterpret_cast<uintptr_t>(d_fixed) & 15))
    return ZS_E_INVAL;
  const int64_t nrec = (int64_t)(M / 16) * (K / 64);
  if (nrec + 1 > INT32_MAX) return ZS_E_OVERFLOW;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(rfixed_kernel<false>, dim3(r_grid(nrec, 4)), dim3(256), 0, st, d_input, M,
                     K, d_top_exponents, d_fixed, d_counts, d_tmp, nullptr, nullptr,
                     WindowCheck{});
  launch_rscan(st, d_counts, nrec, d_eoff, d_total);
  return status_of(hipGetLastError());
}

// d_work: kHistSlices histogram slices of the encoding pass, as many of the
// sample, the guessed window and the flag that says whether the full
// histogram's window differs.
constexpr int kWorkSample = kHistSlices * 256 * 8, kWorkGuess = 2 * kWorkSample,
              kWorkDiffers = kWorkGuess + 32, kWorkArrive = kWorkDiffers + 4;
static_assert(kWorkArrive + 4 <= ZS_RETILED_AUTO_WORK_BYTES, "auto encoder scratch");

__global__ void zero_i32_kernel(int32_t* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

static int retiled_auto(void* stream, const uint16_t* d_input, int M, int K, int rule,
                        const int32_t* d_guess, uint64_t* d_hist, int32_t* d_top, uint8_t* d_work,
                        uint8_t* d_fixed, int32_t* d_counts, int32_t* d_eoff, int64_t* d_total,
                        uint8_t* d_tmp) {
  if (!shape_ok(M, K) || !d_input || !d_hist || !d_top || !d_work || !d_fixed || !d_counts ||
      !d_eoff || !d_total || !d_tmp || (rule != ZS_WINDOW_KV && rule != ZS_WINDOW_WEIGHTS))
    return ZS_E_INVAL;
  if ((reinterpret_cast<uintptr_t>(d_input) & 15) || (reinterpret_cast<uintptr_t>(d_fixed) & 15) ||
      (reinterpret_cast<uintptr_t>(d_hist) & 7) || (reinterpret_cast<uintptr_t>(d_work) & 7))
    return ZS_E_INVAL;
  const int64_t nrec = (int64_t)(M / 16) * (K / 64);
  if (nrec + 1 > INT32_MAX) return ZS_E_OVERFLOW;
  hipStream_t st = (hipStream_t)stream;
  const bool weights = rule == ZS_WINDOW_WEIGHTS;
  uint64_t* slices = reinterpret_cast<uint64_t*>(d_work);
  uint64_t* sample = reinterpret_cast<uint64_t*>(d_work + kWorkSample);
  int32_t* guess = reinterpret_cast<int32_t*>(d_work + kWorkGuess);
  int32_t* differs = reinterpret_cast<int32_t*>(d_work + kWorkDiffers);
  int32_t* arrive = reinterpret_cast<int32_t*>(d_work + kWorkArrive);  // the scan's counter
  if (d_guess) {
    // the caller's window as the guess: only the histogram slices and the
    // scan's counter need clearing (one fill over the start of d_work)
    hipLaunchKernelGGL(zero_i32_kernel, dim3((kWorkArrive / 4 + 1 + 255) / 256), dim3(256), 0, st,
                       reinterpret_cast<int32_t*>(d_work), (int64_t)(kWorkArrive / 4 + 1));
    guess = const_cast<int32_t*>(d_guess);
  } else {
    const hipError_t e = launch_window_sample(st, d_input, (int64_t)M * K, weights, sample, slices,
                                              guess, arrive);
    if (e != hipSuccess) return status_of(e);
  }
  const int hist_grid = r_grid(nrec, 4);
  hipLaunchKernelGGL(rfixed_kernel<true>, dim3(hist_grid), dim3(256), 0, st, d_input, M, K, guess,
                     d_fixed, d_counts, d_tmp, slices, nullptr, WindowCheck{});
  // The window check, and a second encoding only when the window differs
  // from the guess (a small grid keeps the usual no-op launch cheap).
  hipLaunchKernelGGL(rfixed_kernel<false>, dim3(std::min(r_grid(nrec, 4), device_cu_count() * 2)),
                     dim3(256), 0, st, d_input, M, K, d_top, d_fixed, d_counts, d_tmp, nullptr,
                     nullptr, WindowCheck{slices, d_hist, d_top, guess, differs, weights ? 1 : 0});
  launch_rscan(st, d_counts, nrec, d_eoff, d_total, arrive);
  return status_of(hipGetLastError());
}

extern "C" int zs_compress_retiled_auto_gpu(void* stream, const uint16_t* d_input, int M, int K,
                                            int rule, uint64_t* d_hist, int32_t* d_top,
                                            uint8_t* d_work, uint8_t* d_fixed, int32_t* d_counts,
                                            int32_t* d_eoff, int64_t* d_total, uint8_t* d_tmp) {
  return retiled_auto(stream, d_input, M, K, rule, nullptr, d_hist, d_top, d_work, d_fixed,
                      d_counts, d_eoff, d_total, d_tmp);
}

extern "C" int zs_compress_retiled_guess_gpu(void* stream, const uint16_t* d_input, int M, int K,
                                             int rule, const int32_t* d_guess, uint64_t* d_hist,
                                             int32_t* d_top, uint8_t* d_work, uint8_t* d_fixed,
                                             int32_t* d_counts, int32_t* d_eoff, int64_t* d_total,
                                             uint8_t* d_tmp) {
  if (!d_guess || d_guess == d_top) return ZS_E_INVAL;
  return retiled_auto(stream, d_input, M, K, rule, d_guess, d_hist, d_top, d_work, d_fixed,
                      d_counts, d_eoff, d_total, d_tmp);
}

extern "C" int zs_compress_retiled_exps_gpu(void* stream, const uint16_t* d_input, int M, int K,
                                            const int32_t* d_top_exponents, const int32_t* d_eoff,
                                            const uint8_t* d_tmp, uint8_t* d_exps) {
  if (!shape_ok(M, K) || !d_input || !d_top_exponents || !d_eoff || !d_tmp || !d_exps)
    return ZS_E_INVAL;
  if (reinterpret_cast<uintptr_t>(d_input) & 15) return ZS_E_INVAL;
  const int64_t nrec = (int64_t)(M / 16) * (K / 64);
  hipLaunchKernelGGL(rcompact_kernel, dim3(r_grid((nrec + kCompactRecs - 1) / kCompactRecs, 4)), dim3(256), 0,
                     (hipStream_t)stream,
                     d_input, M, K, d_top_exponents, d_eoff, d_tmp, d_exps);
  return status_of(hipGetLastError());
}

static Streams canon_streams(const uint8_t* sm, const uint16_t* full, const uint64_t* b1,
                             const uint64_t* b2, const uint64_t* b3, const int32_t* tom,
                             const int32_t* tog) {
  Streams s;
  s.sm = sm;
  s.full = full;
  s.bm1 = reinterpret_cast<const uint8_t*>(b1);
  s.bm2 = reinterpret_cast<const uint8_t*>(b2);
  s.bm3 = reinterpret_cast<const uint8_t*>(b3);
  s.tom = tom;
  s.tog = tog;
  return s;
}

extern "C" int zs_retile_triple_bitmap_count_gpu(void* stream, const uint8_t* sm,
                                                 const uint16_t* full, const uint64_t* b1,
                                                 const uint64_t* b2, const uint64_t* b3,
                                                 const int32_t* tom, const int32_t* tog, int M,
                                                 int K, int32_t* d_counts, int32_t* d_eoff,
                                                 int64_t* d_total) {
  if (!shape_ok(M, K) || !sm || !full || !b1 || !b2 || !b3 || !tom || !tog || !d_counts ||
      !d_eoff || !d_total)
    return ZS_E_INVAL;
  const int64_t nrec = (int64_t)(M / 16) * (K / 64);
  if (nrec + 1 > INT32_MAX) return ZS_E_OVERFLOW;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(rcount_canon_kernel, dim3(r_grid(nrec, 4)), dim3(256), 0, st,
                     canon_streams(sm, full, b1, b2, b3, tom, tog), M, K, d_counts);
  launch_rscan(st, d_counts, nrec, d_eoff, d_total);
  return status_of(hipGetLastError());
}

extern "C" int zs_retile_triple_bitmap_emit_gpu(void* stream, const uint8_t* sm,
                                                const uint16_t* full, const uint64_t* b1,
                                                const uint64_t* b2, const uint64_t* b3,
                                                const int32_t* tom, const int32_t* tog,
                                                uint8_t start_exp, int M, int K,
                                                const int32_t* d_eoff, uint8_t* d_fixed,
                                                uint8_t* d_exps) {
  if (!shape_ok(M, K) || !sm || !full || !b1 || !b2 || !b3 || !tom || !tog || !d_eoff ||
      !d_fixed || !d_exps)
    return ZS_E_INVAL;
  if (reinterpret_cast<uintptr_t>(d_fixed) & 15) return ZS_E_INVAL;
  const int64_t nrec = (int64_t)(M / 16) * (K / 64);
  hipLaunchKernelGGL(remit_canon_kernel, dim3(r_grid(nrec, 4)), dim3(256), 0,
                     (hipStream_t)stream, canon_streams(sm, full, b1, b2, b3, tom, tog),
                     (int)start_exp, M, K, d_eoff, d_fixed, d_exps);
  return status_of(hipGetLastError());
}

extern "C" int zs_retiled_decompress(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                                     const int32_t* d_eoff, uint8_t start_exp, uint16_t* out,
                                     int M, int K) {
  if (!shape_ok(M, K) || !d_fixed || !d_exps || !d_eoff || !out) return ZS_E_INVAL;
  if ((reinterpret_cast<uintptr_t>(d_fixed) & 15) || (reinterpret_cast<uintptr_t>(d_exps) & 15))
    return ZS_E_INVAL;
  const int64_t nrec = (int64_t)(M / 16) * (K / 64);
  // four workgroups (32 waves) per CU, each wave decoding every G-th record
  const int grid = (int)std::max<int64_t>(1, std::min<int64_t>((nrec + kDecWaves - 1) / kDecWaves,
                                                               (int64_t)device_cu_count() * 4));
  hipLaunchKernelGGL(rdecompress_kernel, dim3(grid), dim3(kDecWaves * 64), 0,
                     (hipStream_t)stream, d_fixed, d_exps, d_eoff, (int)start_exp, out, M, K);
  return status_of(hipGetLastError());
}

// Split-K partial sums go to ws; with `counters` the GEMM kernel itself adds
// them (last workgroup per tile), without it rsplitk_reduce_kernel does.
// Argument checks of retiled_mm that do not depend on the split-K buffers.
static int retiled_mm_args(const uint8_t* d_fixed, const uint8_t* d_exps, const int32_t* d_eoff,
                           const uint16_t* B, const uint16_t* C, int M, int N, int K,
                           int split_k) {
  if (!shape_ok(M, K) || N <= 0 || !d_fixed || !d_exps || !d_eoff || !B || !C) return ZS_E_INVAL;
  if ((reinterpret_cast<uintptr_t>(d_fixed) & 15) || (reinterpret_cast<uintptr_t>(d_exps) & 15) ||
      (reinterpret_cast<uintptr_t>(B) & 15) || (K % 8))
    return ZS_E_INVAL;
  const int KT = K / 64;
  if (split_k < 1 || split_k > KT) return ZS_E_INVAL;
  // a band's records are addressed with 32-bit scalar offsets
  if ((int64_t)KT * kRecBytes > (int64_t)UINT32_MAX) return ZS_E_OVERFLOW;
  if ((int64_t)M * N * split_k > INT32_MAX * 2LL) return ZS_E_OVERFLOW;
  return ZS_OK;
}

static int retiled_mm(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                      const int32_t* d_eoff, uint8_t start_exp, const uint16_t* B, uint16_t* C,
                      int M, int N, int K, uint16_t* ws, int split_k, int32_t* counters) {
  const int chk = retiled_mm_args(d_fixed, d_exps, d_eoff, B, C, M, N, K, split_k);
  if (chk != ZS_OK) return chk;
  if (split_k > 1 && !ws) return ZS_E_INVAL;
  const int KT = K / 64;
  if ((int64_t)N * K * 2 > INT32_MAX) {
    // The kernels address X with 32-bit byte offsets: run row blocks of X
    // and Y that stay below 2^31 bytes, one after another on the stream.
    const int rows = (int)(INT32_MAX / (2LL * K)) / 16 * 16;
    // a row block of fewer than 16 rows would not fit either (K > 2^26)
    if (rows < 16) return ZS_E_OVERFLOW;
    for (int n0 = 0; n0 < N; n0 += rows) {
      const int st_ = retiled_mm(stream, d_fixed, d_exps, d_eoff, start_exp,
                                 B + (int64_t)n0 * K, C + (int64_t)n0 * M, M,
                                 std::min(rows, N - n0), K, ws, split_k, counters);
      if (st_ != ZS_OK) return st_;
    }
    return ZS_OK;
  }
  hipStream_t st = (hipStream_t)stream;
  const int se = (int)start_exp;
  hipError_t e;
  const int kb_per_split = (KT - 1) / split_k + 1;
  uint16_t* out = split_k == 1 ? C : ws;
  const SplitFix fx{C, split_k > 1 ? counters : nullptr, split_k};
  const int nb = (N + 15) / 16;
  // N > 16: 64-row workgroups sharing each X tile through LDS; four K phases
  // per workgroup (16 waves, one workgroup per CU) when the grid fits one
  // round of them, two otherwise (a 320-workgroup grid of 16-wave ones took
  // two rounds: 38 us against 32 us with two phases, 10240x8192 at N = 8); N > 32 on large grids: 128-row workgroups with two
  // bands per wave.  4 <= N <= 16 with at least 7/8 of a workgroup per CU:
  // the same 64-row workgroups over one 16-column block (each X tile crosses
  // L2 once per four bands: 8-24% faster than one band per workgroup at
  // N = 8 / 16 on such grids, even at N = 4).  Otherwise N <= 16:
  // workgroups of 8 K phases over one or two bands.
  const int64_t wide_wgs = (int64_t)(M / 64) * split_k;
  if (nb >= 2 || (N >= 4 && wide_wgs * 8 >= (int64_t)device_cu_count() * 7)) {
    const bool ph4 = wide_wgs <= (int64_t)device_cu_count();
    if (nb <= 1)
      e = ph4 ? launch_rwide<1, 4, 4>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx)
              : launch_rwide<1, 4, 2>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx);
    else if (nb <= 2 && M % 128 == 0 && split_k <= 2 && (int64_t)(M / 128) * split_k >= 160)
      // two bands per wave at 17 <= N <= 32 on large grids of one or two
      // slices (28672 / 14336 rows: 3-5% faster; with four slices, and on
      // 10240 rows, slower than one band per wave)
      e = launch_rwide2<2, 8, 2>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k,
                                 kb_per_split, fx);
    else if (nb <= 2)
      e = ph4 ? launch_rwide<2, 4, 4>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx)
              : launch_rwide<2, 4, 2>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx);
    else if (nb <= 4 && M % 128 == 0 && split_k <= 2 && (int64_t)(M / 128) * split_k >= 160)
      // (with four slices one band per wave is faster: 8192 rows at N = 48 /
      // 64, 83 -> 80 us)
      e = launch_rwide2<4, 8, 2>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k,
                                 kb_per_split, fx);
    else if (nb <= 4)
      e = ph4 ? launch_rwide<4, 4, 4>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx)
              : launch_rwide<4, 4, 2>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx);
    else if (M % 128 == 0 && (int64_t)(M / 128) * split_k * ((N + 127) / 128) >= 160)
      // two bands per wave halve the LDS reads of X per record; they pay
      // once the 128-row grid still has >= 160 workgroups (measured)
      e = launch_rwide2<8, 8, 2>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k,
                                 kb_per_split, fx);
    else if (kb_per_split >= 32)
      // three K phases (12 waves, 3 per SIMD, B fragments read next to
      // their MFMAs) on slices of >= 32 tiles: 2-10% faster than two phases
      // with the early B reads (4096-deep slices of 32 tiles: ~5%); on
      // slices of 16 tiles the uneven phases cost about what they gain
      e = launch_rwide<8, 4, 3>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx);
    else
      e = launch_rwide<8, 4, 2>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx);
  } else {
    // Two bands per wave halve the X bytes per record (the cost that grows
    // with N) but also the grid: for N > 8 once the grid keeps at least
    // 192 workgroups.  Workgroups of 4 waves (16 per CU, twice the K tiles
    // per wave) instead of 8 for N > 1 on grids of >= 640 bands (measured:
    // 1-5 us faster at N = 8 / 16 on 10240, 14336 and 28672 rows, slower on
    // smaller grids) and for N = 1 on grids of >= 896 bands (14336 rows:
    // 21.9 -> 19.6 us; 28672 rows: 0-2% faster; 10240 rows at N = 1 are
    // 0.6 us slower with 4 waves).
    const bool w4 = M / 16 >= (N > 1 ? 640 : 896);
    if (N > 8 && M / 16 >= 384)
      e = w4 ? launch_rgemm<2, 1, 4>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx)
             : launch_rgemm<2, 1, 8>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx);
    else
      e = w4 ? launch_rgemm<1, 1, 4>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx)
             : launch_rgemm<1, 1, 8>(st, d_fixed, d_exps, d_eoff, se, B, out, M, N, K, split_k, kb_per_split, fx);
  }
  if (e != hipSuccess) return (int)e;
  if (split_k > 1 && !counters) {
    const int64_t mn = (int64_t)M * N;
    const int64_t threads = (mn + 7) / 8;
    hipLaunchKernelGGL(rsplitk_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256),
                       0, st, C, ws, mn, split_k);
    e = hipGetLastError();
  }
  return status_of(e);
}

extern "C" int zs_retiled_mm(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                             const int32_t* d_eoff, uint8_t start_exp, const uint16_t* B,
                             uint16_t* C, int M, int N, int K, uint16_t* ws, int split_k) {
  return retiled_mm(stream, d_fixed, d_exps, d_eoff, start_exp, B, C, M, N, K, ws, split_k,
                    nullptr);
}

extern "C" int64_t zs_retiled_mm_counters(int M, int N) {
  if (M <= 0 || N <= 0) return 0;
  return (int64_t)((M + 15) / 16) * ((N + 15) / 16);
}

extern "C" int zs_retiled_mm_fused(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                                   const int32_t* d_eoff, uint8_t start_exp, const uint16_t* B,
                                   uint16_t* C, int M, int N, int K, uint16_t* ws, int split_k,
                                   int32_t* counters) {
  if (split_k > 1 && (!counters || (reinterpret_cast<uintptr_t>(counters) & 3) ||
                      (reinterpret_cast<uintptr_t>(ws) & 7)))
    return ZS_E_INVAL;
  return retiled_mm(stream, d_fixed, d_exps, d_eoff, start_exp, B, C, M, N, K, ws, split_k,
                    counters);
}

// Stream-K schedule (rgemm_sk_kernel) for N <= 16.
extern "C" int64_t zs_retiled_mm_streamk_workspace_bytes(int M, int N, int K) {
  if (!shape_ok(M, K) || N <= 0) return -1;
  const SkPlan p = sk_plan(M, N, K);
  return p.G ? sk_workspace_bytes(p, N) : 0;
}

extern "C" int zs_retiled_mm_streamk(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                                     const int32_t* d_eoff, uint8_t start_exp, const uint16_t* B,
                                     uint16_t* C, int M, int N, int K, void* workspace,
                                     size_t workspace_bytes, int32_t* counters) {
  const int chk = retiled_mm_args(d_fixed, d_exps, d_eoff, B, C, M, N, K, 1);
  if (chk != ZS_OK) return chk;
  if (N > 16) return ZS_E_UNSUPPORTED;
  if ((int64_t)N * K * 2 > INT32_MAX) return ZS_E_OVERFLOW;
  const SkPlan p = sk_plan(M, N, K);
  if (!p.G) return ZS_E_UNSUPPORTED;
  if (!workspace || (int64_t)workspace_bytes < sk_workspace_bytes(p, N) || !counters ||
      (reinterpret_cast<uintptr_t>(workspace) & 15) || (reinterpret_cast<uintptr_t>(counters) & 3))
    return ZS_E_INVAL;
  hipStream_t st = (hipStream_t)stream;
  float* ws = static_cast<float*>(workspace);
  hipError_t e;
  if (N <= 2)
    e = launch_sk_x<1>(st, p, d_fixed, d_exps, d_eoff, start_exp, B, C, M, N, K, ws, counters);
  else if (N <= 4)
    e = launch_sk_x<2>(st, p, d_fixed, d_exps, d_eoff, start_exp, B, C, M, N, K, ws, counters);
  else if (N <= 8)
    e = launch_sk_x<4>(st, p, d_fixed, d_exps, d_eoff, start_exp, B, C, M, N, K, ws, counters);
  else
    e = launch_sk_x<0>(st, p, d_fixed, d_exps, d_eoff, start_exp, B, C, M, N, K, ws, counters);
  return status_of(e);
}

// ---------------------------------------------------------------------------
// zs_retiled_mm_fused without caller buffers: the split-K partial slabs and
// arrival counters live in `scratch`, a file-scope device array (one copy per
// GPU, at its own address, held until the process ends).  Host code reaches
// it only through the address hipGetSymbolAddress returns for the current
// device (the array's name in host code is not a device address).
// ---------------------------------------------------------------------------
namespace zs {
constexpr int64_t kScratchSlabBytes = 32ll << 20;  // bf16 partials [S][N][M]
constexpr int64_t kScratchCounters = 1 << 16;      // int32 arrival counters
constexpr int64_t kScratchBytes = kScratchSlabBytes + 4 * kScratchCounters;
constexpr int kScratchMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kScratchBytes];

// Per-device address of `scratch`, looked up (and its counters cleared on
// `st`) by the first call on that device.  0 / a hipError_t status.
static int scratch_of(hipStream_t st, uint8_t** out) {
  static std::mutex mu;
  static uint8_t* addr[kScratchMaxDevices] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kScratchMaxDevices) return ZS_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    int32_t* cnt = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(p) + kScratchSlabBytes);
    hipLaunchKernelGGL(zero_i32_kernel, dim3((unsigned)(kScratchCounters / 256)), dim3(256), 0,
                       st, cnt, kScratchCounters);
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    addr[dev] = static_cast<uint8_t*>(p);
  }
  *out = addr[dev];
  return ZS_OK;
}
}  // namespace zs

extern "C" int zs_retiled_mm_fused_noalloc(void* stream, const uint8_t* d_fixed,
                                           const uint8_t* d_exps, const int32_t* d_eoff,
                                           uint8_t start_exp, const uint16_t* B, uint16_t* C,
                                           int M, int N, int K, int split_k) {
  const int chk = retiled_mm_args(d_fixed, d_exps, d_eoff, B, C, M, N, K, split_k);
  if (chk != ZS_OK) return chk;
  if (split_k == 1)  // no partial sums: the scratch array is not touched
    return retiled_mm(stream, d_fixed, d_exps, d_eoff, start_exp, B, C, M, N, K, nullptr, 1,
                      nullptr);
  // the partial slabs [split_k][N][M] and the tile counters must fit
  if ((int64_t)split_k * M * N * 2 > kScratchSlabBytes) return ZS_E_OVERFLOW;
  if (zs_retiled_mm_counters(M, N) > kScratchCounters) return ZS_E_OVERFLOW;
  uint8_t* base = nullptr;
  const int st = scratch_of((hipStream_t)stream, &base);
  if (st != ZS_OK) return st;
  return retiled_mm(stream, d_fixed, d_exps, d_eoff, start_exp, B, C, M, N, K,
                    reinterpret_cast<uint16_t*>(base), split_k,
                    reinterpret_cast<int32_t*>(base + kScratchSlabBytes));
}
