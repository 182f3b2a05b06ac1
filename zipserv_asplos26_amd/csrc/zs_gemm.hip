// zs_gemm.hip -- gfx950 TCA-TBE decompress and ZipGEMM (+ split-K reduce).
//
// The kernels decode one half median tile (16 rows x 32 columns) per wave
// step: lane l owns matrix row l%16, columns 8*(l/16)..+7 (see zs_device.hpp).
//   * decompress: every wave walks every G-th median tile through a
//     wave-private LDS stage ring; each lane stores its 8 decoded bf16 of
//     each half as 16 bytes.
//   * ZipGEMM, 16-row workgroups: one workgroup per 16-row band x split-K
//     slice x 16*NB output columns; its waves take interleaved global-tile
//     columns of the slice, stage each median tile through a wave-private
//     LDS buffer ring, and feed the decoded A fragment to
//     v_mfma_f32_16x16x32_bf16 against 16-byte X loads (B operand lane l:
//     column l%16, the same 8 k as A).  The per-wave partial accumulators
//     are tree-summed through LDS.
//   * ZipGEMM, 64-row workgroups (split-K and wide batches on large grids):
//     one global-tile row per workgroup, each X tile staged once in LDS as
//     B fragments for the four median-tile waves of a K phase.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/zipserv.h"
#include "zs_device.hpp"
#include "zs_stage.hpp"

namespace zs {

// ---------------------------------------------------------------------------
// Decompress.  Every wave walks median tiles t = wave, wave + waves, ... of
// the whole matrix (median tile t % 4 of global tile t / 4), copies each into
// a wave-private LDS stage with two 16-byte loads per lane two tiles ahead
// (stage_issue; the stream offsets come through the scalar cache one tile
// before), decodes it from LDS (decode_median_pair) and stores its 16 rows
// of 64 bf16 as two 16-byte stores per lane.  No barrier after the table
// build: the stages are private to their wave.
// ---------------------------------------------------------------------------
constexpr int kDecompWaves = 16;

__global__ __launch_bounds__(kDecompWaves * 64) void decompress_kernel(Streams s, int start_exp,
                                                                       uint16_t* out, int M,
                                                                       int K) {
  __shared__ __attribute__((aligned(16)))
  uint8_t smem[sizeof(DecodeTables) + kDecompWaves * 2 * kStBytes];
  DecodeTables& T = *reinterpret_cast<DecodeTables*>(smem);
  build_decode_tables(T, start_exp, threadIdx.x, kDecompWaves * 64);
  __syncthreads();
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  uint8_t* stage0 = smem + sizeof(DecodeTables) + w * 2 * kStBytes;
  uint8_t* stage1 = stage0 + kStBytes;
  const int KT = K >> 6;
  // median tiles < 2^31 (checked by the host)
  const int ntiles = (M >> 4) * KT;
  const int wid = blockIdx.x * kDecompWaves + w, nw = gridDim.x * kDecompWaves;
  if (wid >= ntiles) return;
  const int cnt = (ntiles - 1 - wid) / nw + 1;
  auto tile_of = [&](int j) { return wid + min(j, cnt - 1) * nw; };  // clamped re-reads
  const uint8_t* bm_lane = l < 8 ? s.bm1 : (l < 16 ? s.bm2 : s.bm3);
  TileOff po;
  auto offs = [&](int j) {
    const int t = tile_of(j);
    po = med_offsets_s(s, t >> 2, t & 3);
  };
  auto issue = [&](int j, StageRegs& R, StageMeta& Mt) {
    const int t = tile_of(j);
    stage_issue(s, bm_lane, t >> 2, t & 3, po, R, Mt);
  };
  StageRegs R0, R1;
  StageMeta M0, M1;
  offs(0);
  issue(0, R0, M0);
  offs(1);
  issue(1, R1, M1);
  offs(2);
  stage_write(stage0, R0);
  // Step j: tile j + 1 to its stage, tile j + 2 issued into the registers
  // tile j used, tile j decoded and stored.
#define DC_STEP(J, CUR, NXT, RC, MC, RN)                                                  \
  {                                                                                      \
    const StageMeta cm_ = MC;                                                            \
    stage_write(NXT, RN);                                                                \
    issue((J) + 2, RC, MC);                                                              \
    offs((J) + 3);                                                                       \
    u32x4 o0_, o1_;                                                                      \
    decode_median_pair(T, T.e1, CUR + kStBm, 128, CUR + kStSm, cm_.sm_rel,               \
                       reinterpret_cast<const uint16_t*>(CUR + kStFull), cm_.full_rel,   \
                       cm_.full_direct, s.full + cm_.fa0, o0_, o1_);                     \
    const int t_ = wid + (J) * nw;                                                       \
    const int g_ = t_ >> 2, m_ = t_ & 3;                                                 \
    const int gm_ = g_ / KT, gk_ = g_ - gm_ * KT;                                        \
    uint16_t* dst_ = out + (int64_t)(gm_ * 64 + m_ * 16 + (l & 15)) * K + gk_ * 64 +     \
                     8 * (l >> 4);                                                       \
    *reinterpret_cast<u32x4*>(dst_) = o0_;                                               \
    *reinterpret_cast<u32x4*>(dst_ + 32) = o1_;                                          \
  }
  int j = 0;
  for (; j + 2 <= cnt; j += 2) {
    DC_STEP(j, stage0, stage1, R0, M0, R1);
    DC_STEP(j + 1, stage1, stage0, R1, M1, R0);
  }
  if (j < cnt) DC_STEP(j, stage0, stage1, R0, M0, R1);
#undef DC_STEP
}

// ---------------------------------------------------------------------------
// ZipGEMM.  A workgroup of WAVES waves owns one 16-row band (one median tile
// row of the global-tile grid) x one split-K slice x 16*NB output columns.
// Wave w streams global-tile columns kb0+w, kb0+w+WAVES, ... of the slice.
// For each one it copies the median tile's bitmap planes (3 x 128 B), its SM
// bytes and its FULL elements with 16-byte loads into a wave-private,
// double-buffered LDS stage -- the load addresses depend only on the tile
// offsets, so the copy of tile j+2 is in flight while tile j is decoded --
// and decodes each half median tile from LDS into one MFMA A operand.
// ---------------------------------------------------------------------------
template <int NB, int WAVES>
struct GemmSmem {
  static constexpr int kMain = (int)sizeof(DecodeTables) + WAVES * 3 * kStBytes;
  static constexpr int kRed = (WAVES / 2) * NB * 64 * 16;
  static constexpr int kBytes = kMain > kRed ? kMain : kRed;
};

template <int NB, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemm_kernel(Streams s, int start_exp,
                                                          const uint16_t* X, uint16_t* Y, int M,
                                                          int N, int K, int kb_per_split) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[GemmSmem<NB, WAVES>::kBytes];
  DecodeTables& T = *reinterpret_cast<DecodeTables*>(smem);
  build_decode_tables(T, start_exp, threadIdx.x, blockDim.x);
  __syncthreads();

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  uint8_t* stage0 = smem + sizeof(DecodeTables) + w * 3 * kStBytes;
  uint8_t* stage1 = stage0 + kStBytes;
  uint8_t* stage2 = stage1 + kStBytes;
  const int band = blockIdx.x;  // 16-row band
  const int gm = band >> 2, m = band & 3;
  const int split = blockIdx.y;
  const int n0 = blockIdx.z * NB * 16;
  const int KT = K >> 6;
  const int kb0 = split * kb_per_split;
  const int kb1 = min(kb0 + kb_per_split, KT);
  const int cnt = kb1 - kb0 > w ? (kb1 - kb0 - w + WAVES - 1) / WAVES : 0;

  const uint16_t* xrow[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = min(n0 + nb * 16 + (l & 15), N - 1);
    xrow[nb] = X + (int64_t)n * K + 8 * (l >> 4);
  }
  f32x4 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Software pipeline over this wave's tiles, in chunks of 64 (one tile's
  // offsets per lane, read back with readlane).  Register sets rotate by
  // unrolling, so every register name is static; every step issues the same
  // loads, and tile indices past the chunk end are clamped to its last tile
  // (a discarded re-read).
  // Lanes 24..63 use plane 3 as their in-bounds default bitmap address.
  const uint8_t* bm_lane = l < 8 ? s.bm1 : (l < 16 ? s.bm2 : s.bm3);
  for (int c0 = 0; c0 < cnt; c0 += 64) {
    const int n = min(cnt - c0, 64);
    const int last = n - 1;
    const TileOff offs = load_tile_offsets(s, gm * KT + kb0 + w + (c0 + l) * WAVES, m, l < n);
    // A tile's compressed data is fetched three tiles ahead (register sets
    // R0..R2); tile j+1 is written to the next LDS stage while tile j is
    // decoded.  X fragments ride in the same ring for narrow batches
    // (kXRing); wider ones fetch X one tile ahead to stay within 256 VGPRs.
    constexpr bool kXRing = NB <= 2;
    StageRegs R0, R1, R2;
    StageMeta M0, M1, M2;
    bf16x8 X0[2][NB], X1[2][NB], X2[2][NB], xc[2][NB], xn[2][NB];
#define ZS_TILE(J) (gm * KT + kb0 + w + (c0 + (J)) * WAVES)
#define ZS_LOADX(J, DST)                                                            \
  {                                                                                 \
    const int kk_ = (kb0 + w + (c0 + (J)) * WAVES) * 64;                            \
    _Pragma("unroll") for (int h_ = 0; h_ < 2; ++h_)                                \
      _Pragma("unroll") for (int nb_ = 0; nb_ < NB; ++nb_)                          \
        DST[h_][nb_] = *reinterpret_cast<const bf16x8*>(xrow[nb_] + kk_ + 32 * h_); \
  }
#define ZS_ISSUE(J, R, MT, XD)                                                      \
  {                                                                                 \
    stage_issue(s, bm_lane, ZS_TILE(J), m, tile_off_at(offs, (J)), R, MT);          \
    if constexpr (kXRing) ZS_LOADX(J, XD);                                          \
  }
#define ZS_STEP(J, CUR, NXT, RC, MC, XC, RN)                                             \
  {                                                                                      \
    const StageMeta cm_ = MC;                                                            \
    _Pragma("unroll") for (int h_ = 0; h_ < 2; ++h_)                                     \
      _Pragma("unroll") for (int nb_ = 0; nb_ < NB; ++nb_)                               \
        xc[h_][nb_] = kXRing ? XC[h_][nb_] : xn[h_][nb_];                                \
    stage_write(NXT, RN);                                                                \
    ZS_ISSUE(min((J) + 3, last), RC, MC, XC);                                            \
    if constexpr (!kXRing) ZS_LOADX(min((J) + 1, last), xn);                             \
    if ((J) < n) {                                                                       \
      u32x4 a0_, a1_;                                                                    \
      decode_median_pair(T, T.e1, CUR + kStBm, 128, CUR + kStSm, cm_.sm_rel,                   \
                         reinterpret_cast<const uint16_t*>(CUR + kStFull), cm_.full_rel, \
                         cm_.full_direct, s.full + cm_.fa0, a0_, a1_);                   \
      _Pragma("unroll") for (int nb_ = 0; nb_ < NB; ++nb_) {                             \
        acc[nb_] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a0_), xc[0][nb_],   \
                                                           acc[nb_], 0, 0, 0);           \
        acc[nb_] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a1_), xc[1][nb_],   \
                                                           acc[nb_], 0, 0, 0);           \
      }                                                                                  \
    }                                                                                    \
  }
    ZS_ISSUE(0, R0, M0, X0);
    ZS_ISSUE(min(1, last), R1, M1, X1);
    ZS_ISSUE(min(2, last), R2, M2, X2);
    if constexpr (!kXRing) ZS_LOADX(0, xn);
    stage_write(stage0, R0);
    // Period-3 body (3 register sets x 3 LDS stages) without early exits:
    // steps past the end only repeat the clamped loads and skip the decode.
    for (int j = 0; j < n; j += 3) {
      ZS_STEP(j, stage0, stage1, R0, M0, X0, R1);
      ZS_STEP(j + 1, stage1, stage2, R1, M1, X1, R2);
      ZS_STEP(j + 2, stage2, stage0, R2, M2, X2, R0);
    }
#undef ZS_STEP
#undef ZS_LOADX
#undef ZS_ISSUE
#undef ZS_TILE
  }

  // Deterministic tree reduction of the WAVES partial accumulators in LDS.
  __syncthreads();
  f32x4* red = reinterpret_cast<f32x4*>(smem);
#pragma unroll
  for (int half = WAVES / 2; half >= 1; half /= 2) {
    if (w >= half && w < 2 * half) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) red[((w - half) * NB + nb) * 64 + l] = acc[nb];
    }
    __syncthreads();
    if (w < half) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[nb] += red[(w * NB + nb) * 64 + l];
    }
    __syncthreads();
  }
  if (w == 0) {
    uint16_t* out = Y + (int64_t)split * M * N;
    const int mrow = band * 16 + 4 * (l >> 4);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const f32x4 v = acc[nb];
      const int n = n0 + nb * 16 + (l & 15);
      if (n < N) {
        const uint32_t lo = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
        const uint32_t hi = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
        *reinterpret_cast<uint2*>(out + (int64_t)n * M + mrow) = make_uint2(lo, hi);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// ZipGEMM, 64-row workgroups for wider batches (N > 16).  A workgroup of
// 4*PH waves owns one global-tile row (64 rows) x one split-K slice x 16*NB
// output columns; wave w stages and decodes median tile w%4 of K tiles
// kb0 + PH*s + w/4 (PH interleaved phases) through two wave-private LDS
// stages, as gemm_kernel does.  The 256 threads of a phase load each X tile
// once into LDS as MFMA B fragments (xfrag_slot) read by its four median
// waves, so X crosses L2 once per 64 rows instead of once per 16 rows --
// the traffic that grows with N and bounds the 16-row kernel from N = 32 on.
// Median tiles are fetched two steps ahead into registers, X tiles two steps
// ahead into registers and one step ahead into a double-buffered LDS tile;
// one barrier per step.  Stream offsets come through the scalar cache (the
// tile index is uniform per wave), one step before the loads that use them.
// ---------------------------------------------------------------------------
template <int NB, int PH>
struct CWideSmem {
  static constexpr int kXTile = 2 * NB * kXFragBlock;
  static constexpr int kX = PH * 2 * kXTile;             // [phase][buffer]
  static constexpr int kStages = 4 * PH * 2 * kStBytes;  // [wave][buffer]
  static constexpr int kMain = (int)sizeof(DecodeTables) + kStages + kX;
  static constexpr int kRed = (PH - 1) * 4 * NB * 64 * 16;
  static constexpr int kBytes = kMain > kRed ? kMain : kRed;
};

template <int NB, int PH, int RD>
__global__ __launch_bounds__(4 * PH * 64) void cgemm_wide_kernel(Streams s, int start_exp,
                                                                 const uint16_t* X, uint16_t* Y,
                                                                 int M, int N, int K,
                                                                 int kb_per_split) {
  using S = CWideSmem<NB, PH>;
  constexpr int kXTile = S::kXTile;
  __shared__ __attribute__((aligned(16))) uint8_t smem[S::kBytes];
  DecodeTables& T = *reinterpret_cast<DecodeTables*>(smem);

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  const int q = w & 3, p = w >> 2;  // median tile, phase
  const int t = threadIdx.x & 255;  // thread index within the phase
  uint8_t* stage0 = smem + sizeof(DecodeTables) + w * 2 * kStBytes;
  uint8_t* stage1 = stage0 + kStBytes;
  uint8_t* xb0 = smem + sizeof(DecodeTables) + S::kStages + p * 2 * kXTile;
  uint8_t* xb1 = xb0 + kXTile;
  const int gm = blockIdx.x;
  const int split = blockIdx.y;
  const int n0 = blockIdx.z * NB * 16;
  const int KT = K >> 6;
  const int kb0 = split * kb_per_split;
  const int kb1 = min(kb0 + kb_per_split, KT);
  const int span = max(kb1 - kb0, 0);
  const int steps = (span + PH - 1) / PH;    // same for every phase
  const int cnt = (span - p + PH - 1) / PH;  // valid tiles of this phase
  // K tile of step j of this phase, clamped into the slice (clamped steps
  // repeat an in-bounds load and skip the decode; an empty slice, kb0 >= KT,
  // clamps to the last tile of the row).
  auto tile_of = [&](int j) { return min(kb0 + PH * j + p, kb1 - 1); };
  const int g0 = gm * KT;

  // X tile loads of this thread: chunk c = t + 256*i, row c/8 (clamped to
  // N - 1), 16-byte column c%8 (128*NB chunks per tile; threads past them
  // load and drop).
  constexpr int kXC = (2 * NB + 3) / 4;
  const uint16_t* xsrc[kXC];
  int xdst[kXC];
#pragma unroll
  for (int i = 0; i < kXC; ++i) {
    const int c = t + 256 * i;
    const int row = min(c >> 3, 16 * NB - 1), cc = c & 7;
    xsrc[i] = X + (int64_t)min(n0 + row, N - 1) * K + 8 * cc;
    xdst[i] = c < 128 * NB ? 16 * xfrag_slot(row >> 4, cc >> 2, cc & 3, row & 15) : -1;
  }
  f32x4 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int brd = 16 * xfrag_slot(0, 0, l >> 4, l & 15);
  const int brd1 = 16 * xfrag_slot(0, 1, l >> 4, l & 15);

  const uint8_t* bm_lane = l < 8 ? s.bm1 : (l < 16 ? s.bm2 : s.bm3);
  TileOff po;  // offsets of the next median tile to issue
  auto offs = [&](int j) { po = med_offsets_s(s, g0 + tile_of(j), q); };
  auto issue = [&](int j, StageRegs& R, StageMeta& Mt) {
    stage_issue(s, bm_lane, g0 + tile_of(j), q, po, R, Mt);
  };
  auto xload = [&](int j, u32x4 (&XR)[kXC]) {
    const int kk = tile_of(j) * 64;
#pragma unroll
    for (int i = 0; i < kXC; ++i) XR[i] = *reinterpret_cast<const u32x4*>(xsrc[i] + kk);
  };
  auto xwrite = [&](uint8_t* xb, const u32x4 (&XR)[kXC]) {
#pragma unroll
    for (int i = 0; i < kXC; ++i)
      if (2 * NB >= 4 * (i + 1) || xdst[i] >= 0) *reinterpret_cast<u32x4*>(xb + xdst[i]) = XR[i];
  };

  static_assert(RD % 2 == 0, "tile ring of an even number of steps");
  StageRegs R[RD];
  StageMeta MT[RD];
  u32x4 XA[kXC], XB[kXC];
  {
    TileOff so[RD + 1];
#pragma unroll
    for (int k = 0; k <= RD; ++k) so[k] = med_offsets_s(s, g0 + tile_of(k), q);
#pragma unroll
    for (int k = 0; k < RD; ++k) {
      po = so[k];
      issue(k, R[k], MT[k]);
    }
    po = so[RD];
  }
  xload(0, XA);
  xload(1, XB);
  build_decode_tables(T, start_exp, threadIdx.x, 4 * PH * 64);
  stage_write(stage0, R[0]);
  xwrite(xb0, XA);
  xload(2, XA);
  __syncthreads();  // decode tables and X tile 0 visible

  // NB = 8: the step's sixteen B fragments are read before the decode, so
  // their LDS latency hides behind it.
  constexpr bool kEarlyB = NB >= 8;
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

  // Step s: median tile s + 1 goes from registers to its stage, tile s + RD
  // is issued into the registers tile s used, tile s is decoded from its stage
  // and multiplied with X tile s (LDS buffer s % 2), X tile s + 1 goes to the
  // other buffer and X tile s + 3 is loaded into the registers it used.
#define CW_STEP(S, CUR, NXT, XCUR, XNXT, RC, MC, RN, XR, GUARD)                          \
  {                                                                                    \
    bf16x8 b0_[NB], b1_[NB];                                                           \
    if constexpr (kEarlyB) b_read(XCUR, b0_, b1_);                                     \
    const StageMeta cm_ = MC;                                                          \
    stage_write(NXT, RN);                                                              \
    issue((S) + RD, RC, MC);                                                           \
    offs((S) + RD + 1);                                                                \
    if (!(GUARD) || (S) < cnt) {                                                       \
      u32x4 a0_, a1_;                                                                  \
      decode_median_pair(T, T.e1, CUR + kStBm, 128, CUR + kStSm, cm_.sm_rel,           \
                         reinterpret_cast<const uint16_t*>(CUR + kStFull), cm_.full_rel, \
                         cm_.full_direct, s.full + cm_.fa0, a0_, a1_);                 \
      mfma_step(XCUR, b0_, b1_, a0_, a1_);                                             \
    }                                                                                  \
    xwrite(XNXT, XR);                                                                  \
    xload((S) + 3, XR);                                                                \
    __syncthreads();                                                                   \
  }
  // Steps s <= steps - 2 have a tile in every phase (cnt >= steps - 1): no
  // step condition there.
  // Tile ring: tile s + 1 sits in R[(s + 1) % RD] during step s.
  int s0 = 0;
  for (; s0 + RD - 1 <= steps - 2; s0 += RD) {
#pragma unroll
    for (int k = 0; k < RD; k += 2) {
      CW_STEP(s0 + k, stage0, stage1, xb0, xb1, R[k], MT[k], R[k + 1], XB, false);
      CW_STEP(s0 + k + 1, stage1, stage0, xb1, xb0, R[k + 1], MT[k + 1], R[(k + 2) % RD], XA,
              false);
    }
  }
  for (; s0 < steps; s0 += RD) {
#pragma unroll
    for (int k = 0; k < RD; k += 2) {
      if (s0 + k < steps)
        CW_STEP(s0 + k, stage0, stage1, xb0, xb1, R[k], MT[k], R[k + 1], XB, true);
      if (s0 + k + 1 < steps)
        CW_STEP(s0 + k + 1, stage1, stage0, xb1, xb0, R[k + 1], MT[k + 1], R[(k + 2) % RD], XA,
                true);
    }
  }
#undef CW_STEP

  // Phases 1..PH-1 hand their sums to phase 0 through LDS (added in phase
  // order, so the result is deterministic); phase 0 writes its median rows.
  f32x4* red = reinterpret_cast<f32x4*>(smem);
  if (p > 0) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) red[(((p - 1) * 4 + q) * NB + nb) * 64 + l] = acc[nb];
  }
  __syncthreads();
  if (p == 0) {
    uint16_t* out = Y + (int64_t)split * M * N;
    const int mrow = gm * 64 + q * 16 + 4 * (l >> 4);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      f32x4 v = acc[nb];
#pragma unroll
      for (int pp = 1; pp < PH; ++pp) v += red[(((pp - 1) * 4 + q) * NB + nb) * 64 + l];
      const int col = n0 + nb * 16 + (l & 15);
      if (col < N) {
        const uint32_t lo = f32_to_bf16_bits(v[0]) | (f32_to_bf16_bits(v[1]) << 16);
        const uint32_t hi = f32_to_bf16_bits(v[2]) | (f32_to_bf16_bits(v[3]) << 16);
        *reinterpret_cast<uint2*>(out + (int64_t)col * M + mrow) = make_uint2(lo, hi);
      }
    }
  }
}

// C[i] = bf16(sum_s float(WS[s][i])) -- csrc/Reduction_Kernel.cuh:15-37.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(uint16_t* C, const uint16_t* WS,
                                                            int64_t mn, int split_k) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i0 >= mn) return;
  if (i0 + 8 <= mn && (mn % 8) == 0) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int sp = 0; sp < split_k; ++sp) {
      const uint4 v = *reinterpret_cast<const uint4*>(WS + sp * mn + i0);
      const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc[2 * j] += bf16_bits_to_f32(d[j] & 0xFFFF);
        acc[2 * j + 1] += bf16_bits_to_f32(d[j] >> 16);
      }
    }
    uint4 o;
    o.x = f32_to_bf16_bits(acc[0]) | (f32_to_bf16_bits(acc[1]) << 16);
    o.y = f32_to_bf16_bits(acc[2]) | (f32_to_bf16_bits(acc[3]) << 16);
    o.z = f32_to_bf16_bits(acc[4]) | (f32_to_bf16_bits(acc[5]) << 16);
    o.w = f32_to_bf16_bits(acc[6]) | (f32_to_bf16_bits(acc[7]) << 16);
    *reinterpret_cast<uint4*>(C + i0) = o;
  } else {
    for (int64_t i = i0; i < std::min<int64_t>(i0 + 8, mn); ++i) {
      float acc = 0.f;
      for (int sp = 0; sp < split_k; ++sp) acc += bf16_bits_to_f32(WS[sp * mn + i]);
      C[i] = (uint16_t)f32_to_bf16_bits(acc);
    }
  }
}

int device_cu_count() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
      cus = prop.multiProcessorCount;
    if (cus <= 0) cus = 256;
  }
  return cus;
}

static int status_of(hipError_t e) { return e == hipSuccess ? ZS_OK : (int)e; }

template <int NB>
static hipError_t launch_gemm(hipStream_t st, const Streams& s, int start_exp, const uint16_t* X,
                              uint16_t* Y, int M, int N, int K, int split_k, int kb_per_split) {
  constexpr int kWaves = NB <= 4 ? 8 : 4;
  dim3 grid(M / 16, split_k, (N + NB * 16 - 1) / (NB * 16));
  hipLaunchKernelGGL((gemm_kernel<NB, kWaves>), grid, dim3(kWaves * 64), 0, st, s, start_exp, X,
                     Y, M, N, K, kb_per_split);
  return hipGetLastError();
}

// Median tiles in flight per wave: 2 (4 measured 10% slower: the kernel is
// bound by the decode's LDS and VALU work, not by load latency).
constexpr int kCWideDepth = 2;

template <int NB, int PH>
static hipError_t launch_cwide(hipStream_t st, const Streams& s, int start_exp,
                               const uint16_t* X, uint16_t* Y, int M, int N, int K, int split_k,
                               int kb_per_split) {
  dim3 grid(M / 64, split_k, (N + NB * 16 - 1) / (NB * 16));
  hipLaunchKernelGGL((cgemm_wide_kernel<NB, PH, kCWideDepth>), grid, dim3(4 * PH * 64), 0, st, s, start_exp,
                     X, Y, M, N, K, kb_per_split);
  return hipGetLastError();
}

}  // namespace zs

using namespace zs;

static bool streams_ok(const uint8_t* sm, const uint16_t* full, const uint64_t* b1,
                       const uint64_t* b2, const uint64_t* b3, const int32_t* tom,
                       const int32_t* tog) {
  return sm && full && b1 && b2 && b3 && tom && tog;
}

static Streams make_streams(const uint8_t* sm, const uint16_t* full, const uint64_t* b1,
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

extern "C" int zs_bf16_triple_bitmap_decompress(void* stream, const uint8_t* sm,
                                                const uint16_t* full, const uint64_t* b1,
                                                const uint64_t* b2, const uint64_t* b3,
                                                const int32_t* tom, const int32_t* tog,
                                                int max_hf, int max_full, uint8_t start_exp,
                                                uint16_t* out, int M, int K) {
  (void)max_hf;
  (void)max_full;  // LDS staging sizes of the reference kernel; not needed here
  if (M <= 0 || K <= 0 || (M % 64) || (K % 64)) return ZS_E_INVAL;
  if (!streams_ok(sm, full, b1, b2, b3, tom, tog) || !out) return ZS_E_INVAL;
  const int64_t ntiles = (int64_t)(M / 16) * (K / 64);
  if (ntiles > INT32_MAX) return ZS_E_OVERFLOW;
  // one 16-wave workgroup per CU (one table build each; two 8-wave ones
  // measured 5-7% slower, two 12-wave ones the same), each wave on every
  // G-th median tile
  const int64_t grid = std::min<int64_t>((ntiles + kDecompWaves - 1) / kDecompWaves,
                                         (int64_t)device_cu_count());
  hipLaunchKernelGGL(decompress_kernel, dim3((unsigned)grid), dim3(kDecompWaves * 64), 0,
                     (hipStream_t)stream, make_streams(sm, full, b1, b2, b3, tom, tog),
                     (int)start_exp, out, M, K);
  return status_of(hipGetLastError());
}

extern "C" int zs_bf16_triple_bitmap_mm(void* stream, const uint8_t* sm, const uint16_t* full,
                                        const uint64_t* b1, const uint64_t* b2,
                                        const uint64_t* b3, const int32_t* tom,
                                        const int32_t* tog, int max_hf, int max_full,
                                        uint8_t start_exp, const uint16_t* B, uint16_t* C,
                                        int M, int N, int K, uint16_t* ws, int split_k) {
  (void)max_hf;
  (void)max_full;
  if (M <= 0 || K <= 0 || N <= 0 || (M % 64) || (K % 64)) return ZS_E_INVAL;
  if (!streams_ok(sm, full, b1, b2, b3, tom, tog) || !B || !C) return ZS_E_INVAL;
  const int KT = K / 64;
  if (split_k < 1 || split_k > KT) return ZS_E_INVAL;
  if (split_k > 1 && !ws) return ZS_E_INVAL;
  if ((int64_t)M * N * split_k > INT32_MAX * 2LL) return ZS_E_OVERFLOW;
  // K partition of csrc/L_Kernel.cuh:316-326: ceil(KT / split_k) tiles per slice.
  const int kb_per_split = (KT - 1) / split_k + 1;
  hipStream_t st = (hipStream_t)stream;
  const Streams s = make_streams(sm, full, b1, b2, b3, tom, tog);
  uint16_t* out = split_k == 1 ? C : ws;
  const int nb = (N + 15) / 16;
  hipError_t e;
  // 64-row workgroups (each X tile staged once in LDS for four median
  // tiles) for every split-K launch, and for one slice at N > 16 when the
  // grid of 64-row workgroups covers >= 5/8 of the CUs (>= 3/8 for N > 112):
  // 1.05-2.6x the 16-row kernel there.  Four K phases per workgroup (16
  // waves, one workgroup per CU) when the grid fits one round of them, two
  // otherwise.
  // Otherwise 16-row workgroups: four times the grid, for small M.
  const int64_t wgs = (int64_t)(M / 64) * split_k;
  const int64_t cus = device_cu_count();
  const bool cwide =
      split_k > 1 || (nb >= 2 && (wgs * 8 >= cus * 5 || (nb >= 8 && wgs * 8 >= cus * 3)));
  const bool ph4 = wgs <= cus;
  if (cwide) {
    if (nb <= 1)
      e = ph4 ? launch_cwide<1, 4>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split)
              : launch_cwide<1, 2>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split);
    else if (nb <= 2)
      e = ph4 ? launch_cwide<2, 4>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split)
              : launch_cwide<2, 2>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split);
    else if (nb <= 4)
      e = ph4 ? launch_cwide<4, 4>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split)
              : launch_cwide<4, 2>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split);
    else
      e = launch_cwide<8, 2>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split);
  } else if (nb <= 1) e = launch_gemm<1>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split);
  else if (nb <= 2) e = launch_gemm<2>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split);
  else if (nb <= 3) e = launch_gemm<3>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split);
  else if (nb <= 4) e = launch_gemm<4>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split);
  else if (nb <= 6) e = launch_gemm<6>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split);
  else if (nb <= 8) e = launch_gemm<8>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split);
  else e = launch_gemm<16>(st, s, start_exp, B, out, M, N, K, split_k, kb_per_split);
  if (e != hipSuccess) return (int)e;
  if (split_k > 1) {
    const int64_t mn = (int64_t)M * N;
    const int64_t threads = (mn + 7) / 8;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256),
                       0, st, C, ws, mn, split_k);
    e = hipGetLastError();
  }
  return status_of(e);
}
