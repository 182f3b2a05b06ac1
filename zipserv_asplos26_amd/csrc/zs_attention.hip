// zs_attention.hip -- single-token (decode) GQA attention over a KV cache held
// in the TCA-TBE format, and the same kernel over a dense bf16 cache (gfx950).
//
// Work unit: one wave per (batch b, KV head h, sequence split).  The wave walks
// its token range 16 tokens (one median-tile row band) at a time in four steps
//   K0: decode K median tile, dims 0..63   -> S^T += K q^T  (2 x mfma 16x16x32)
//   K1: decode K median tile, dims 64..127 -> S^T complete; online softmax
//   V0: decode V median tile, dims 0..63   -> O^T += V^T P^T (4 x mfma 16x16x16)
//   V1: decode V median tile, dims 64..127 -> O^T += V^T P^T (4 x mfma 16x16x16)
// S^T is tokens x heads: the decoded K fragment (lane l: token l%16, dims
// 8*(l/16)..+7) is the A operand as is and q (lane l: head l%16) the B operand.
// Its accumulator layout (lane l: head l%16, tokens 4*(l/16)+r) is exactly the
// B operand P^T of the 16x16x16 product, and the A operand V^T (lane l: dim
// l%16, tokens 4*(l/16)+j) comes from the decoded V tile written row-major to
// LDS and read back with ds_read_b64_tr_b16.  The O^T accumulator keeps head
// l%16 in lane l, the same lanes that hold that head's running max and sum.
//
// The median tiles are prefetched four steps ahead into registers and staged
// through a wave-private LDS double buffer (zs_stage.hpp), as in ZipGEMM.
// Splits write unnormalised partials (O, m, l) that attn_combine_kernel merges.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "../../include/zipserv.h"
#include "zs_device.hpp"
#include "zs_rdecode.hpp"
#include "zs_stage.hpp"

namespace zs {

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 128;
constexpr int kAttnWaves = 4;   // waves per workgroup, one item each
constexpr int kItemWaves = 4;   // waves per workgroup sharing one item (small grids)
constexpr int kVRow = 160;                  // LDS row pitch of the V tile (bytes)
constexpr int kVBytes = 16 * kVRow;         // 16 tokens x 64 dims (+ pad)
constexpr int kModeCanon = 0;    // canonical TCA-TBE streams
constexpr int kModeDense = 1;    // dense bf16 caches
constexpr int kModeRetiled = 2;  // re-tiled records (zs_rdecode.hpp)
constexpr int kModePaged = 3;    // dense bf16 caches in pages through a block table

template <int kMode>
struct AttnLds {
  // per-workgroup decode tables, then per-wave stages and the V tile
  static constexpr int kTables = kMode == kModeCanon ? (int)sizeof(DecodeTables) + 256 * 16
                                 : kMode == kModeRetiled ? (int)sizeof(RTables)
                                                         : 0;
  static constexpr int kWave = (kMode == kModeCanon ? 2 * kStBytes
                                : kMode == kModeRetiled ? 2 * kExpStage : 0) + kVBytes;
  static constexpr int bytes(int waves) { return kTables + waves * kWave; }
};

struct AttnParams {
  Streams k, v;                 // compressed caches (canonical kernel)
  const uint8_t* kfix;          // re-tiled caches: fixed records, outlier bytes, offsets
  const uint8_t* kexp;
  const int32_t* keo;
  const uint8_t* vfix;
  const uint8_t* vexp;
  const int32_t* veo;
  int k_nrec, v_nrec;           // re-tiled records of each cache (bounds start-up loads)
  const uint16_t* kd;           // dense caches [B][cap][Hkv][D] (dense kernel)
  const uint16_t* vd;           //   or pages [blocks][page][Hkv][D] (paged kernel)
  const int32_t* block_table;   // [B][bt_stride] physical page of each logical page
  int bt_stride, page;          // page: tokens per page, a multiple of 16
  int k_start, v_start;         // start_exp of K and V
  int k_bsr, k_hsr, v_bsr, v_hsr;  // batch / head strides in rows (compressed)
  int cap;                      // dense cache capacity (tokens)
  const uint16_t* q;            // [B][H][D]
  uint16_t* out;                // [B][H][D]
  float* lse;                   // [B][H] or null
  float* ws_o;                  // [B][H][splits][D]   (splits > 1)
  float* ws_ml;                 // [B][H][splits][2]
  const int32_t* seqlens;       // [B] or null
  int seqlen_k, batch, heads, heads_k, group, splits, chunk;
  float scale_log2;             // softmax_scale * log2(e)
};

__device__ __forceinline__ void build_e1(uint4* e1, int start_exp, int tid, int nthreads) {
  for (int v = tid; v < 256; v += nthreads) {
    uint32_t w[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t lo = (v >> (2 * d)) & 1, hi = (v >> (2 * d + 1)) & 1;
      w[d] = ((uint32_t)(start_exp + lo) << 7) | ((uint32_t)(start_exp + hi) << 23);
    }
    e1[v] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

__device__ __forceinline__ float wave_max16(float x) {
  // max over lanes l, l^16, l^32, l^48 (the four row groups)
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float wave_sum16(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const __bf16 ha = (__bf16)a, hb = (__bf16)b;
  return (uint32_t)__builtin_bit_cast(unsigned short, ha) |
         ((uint32_t)__builtin_bit_cast(unsigned short, hb) << 16);
}

// Per-wave attention state over one (batch, KV head, token range): the q^T
// fragments (B operand, lane l -> head l%16 of the group, dims 32c +
// 8*(l/16)..+7), the O^T accumulators (lane l: head l%16, dims 16*i +
// 4*(l/16) + r of O[i]), the running max and sum (log2 domain), and the
// current 16 tokens' scores S^T and softmax weights P^T (bf16 pairs).
struct AttnWave {
  bf16x8 Q[4];
  f32x4 O[8];
  float m_run, l_run;
  f32x4 S;
  uint32_t pb0, pb1;
};

// K step TY (0: dims 0..63, 1: dims 64..127) of 16 tokens: S^T += K q^T with
// the K fragment (lane l: token l%16, dims 8*(l/16)..+7 in a0, +32 in a1) as
// the A operand.
__device__ __forceinline__ void attn_k_step(AttnWave& a, int TY, u32x4 a0, u32x4 a1) {
  if (TY == 0) a.S = f32x4{0.f, 0.f, 0.f, 0.f};
  a.S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a0), a.Q[2 * TY], a.S, 0, 0, 0);
  a.S = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a1), a.Q[2 * TY + 1], a.S, 0, 0, 0);
}

// Online softmax over the 16 tokens of S^T (log2 domain): this lane holds
// tokens tb..tb+3 of head l%16; tokens >= t1 are masked.  Rescales O and
// leaves the bf16 weights in pb0 / pb1 (the B operand P^T of the V steps).
__device__ __forceinline__ void attn_softmax(AttnWave& a, int tb, int t1, float scale_log2) {
  float s[4];
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    s[r] = (tb + r < t1) ? a.S[r] * scale_log2 : -INFINITY;
    mx = fmaxf(mx, s[r]);
  }
  mx = wave_max16(mx);
  const float m_new = fmaxf(a.m_run, mx);
  const float m_use = m_new == -INFINITY ? 0.f : m_new;
  const float alpha = __builtin_amdgcn_exp2f(a.m_run - m_use);
  float pr[4], ps = 0.f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    pr[r] = __builtin_amdgcn_exp2f(s[r] - m_use);
    ps += pr[r];
  }
  ps = wave_sum16(ps);
  a.l_run = a.l_run * alpha + ps;
  if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) a.O[i] *= alpha;
  }
  a.m_run = m_new;
  a.pb0 = pack_bf16x2(pr[0], pr[1]);
  a.pb1 = pack_bf16x2(pr[2], pr[3]);
}

// V step TY (2: dims 0..63, 3: dims 64..127): O^T += V^T P^T, the A operand
// V^T read with ds_read_b64_tr_b16 from the 16-token x 64-dim V tile in LDS
// (row pitch kVRow), `vt` = the tile + this lane's transposed-read offset.
__device__ __forceinline__ void attn_v_step(AttnWave& a, int TY, const uint8_t* vt) {
  const v4i16 pbv = __builtin_bit_cast(v4i16, (uint2){a.pb0, a.pb1});
#pragma unroll
  for (int blk = 0; blk < 4; ++blk) {
    const v4i16 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(vt + 32 * blk));
    const int oi = 4 * (TY - 2) + blk;
    a.O[oi] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pbv, a.O[oi], 0, 0, 0);
  }
}

// Median tile `med` (16 tokens) of the wave's range, column tile c, of K or V:
// global tile index in the compressed 2D matrix (2 column tiles of 64).
// (`rowbase`: a multiple of 16; median `med` of the range is the 16-row
// band (rowbase >> 4) + med: global tile row band / 4, median band % 4)
__device__ __forceinline__ int kv_tile(int rowbase, int med, int c) {
  return (((rowbase >> 4) + med) >> 2) * 2 + c;
}
__device__ __forceinline__ int kv_median(int rowbase, int med) {
  return ((rowbase >> 4) + med) & 3;
}

// Combine buffer of kWpi > 1: per wave, 32 O values + m + l per lane.
constexpr int kCombineBytes = kItemWaves * 34 * 64 * 4;

// kWpi = 1: the workgroup's kAttnWaves waves take one (batch, KV head,
// split) item each.  kWpi = kItemWaves: its waves share one item, each a
// contiguous 1/kWpi of the split's tokens, and merge their softmax states in
// LDS at the end (for small grids: kWpi x the waves without the cost of
// kWpi x the global splits).
// The re-tiled mode asks for three waves per SIMD: the compiler then keeps
// the MFMA accumulators in ordinary VGPRs (140 in all, no spills) instead of
// splitting 135 VGPRs + 36 AGPRs, which allowed only two.
template <int kMode, int kWpi>
__global__ __launch_bounds__((kWpi == 1 ? kAttnWaves : kWpi) * 64,
                             kMode == kModeRetiled ? 3 : 1) void attn_kernel(AttnParams p) {
  constexpr bool kDense = kMode == kModeDense || kMode == kModePaged;
  extern __shared__ __attribute__((aligned(16))) uint8_t attn_smem[];
  DecodeTables& T = *reinterpret_cast<DecodeTables*>(attn_smem);
  RTables& RT = *reinterpret_cast<RTables*>(attn_smem);
  uint4* e1v = reinterpret_cast<uint4*>(
      attn_smem + (kMode == kModeRetiled ? sizeof(RTables) : sizeof(DecodeTables)));
  if constexpr (kMode == kModeCanon) {
    build_decode_tables(T, p.k_start, threadIdx.x, blockDim.x);
    build_e1(e1v, p.v_start, threadIdx.x, blockDim.x);
  }
  // (re-tiled: the decode table is copied during the start-up further down)
  const RExp kex = r_exp(p.k_start), vex = r_exp(p.v_start);
  if constexpr (kMode != kModeRetiled) __syncthreads();

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  const int item0 = kWpi == 1 ? blockIdx.x * kAttnWaves + w : blockIdx.x;
  const int nitems = p.batch * p.heads_k * p.splits;
  if constexpr (kMode != kModeRetiled) {
    if (item0 >= nitems) return;  // uniform when kWpi > 1
  }
  // (re-tiled: a wave past the last item runs the start-up on the last item,
  // which every wave of the workgroup must reach, and returns after it)
  const int item = min(item0, nitems - 1);
  const int sp = item % p.splits;
  const int h = (item / p.splits) % p.heads_k;
  const int b = item / (p.splits * p.heads_k);
  int L = p.seqlen_k;
  if (p.seqlens) L = min(L, __builtin_amdgcn_readfirstlane(p.seqlens[b]));
  L = max(L, 0);
  // token range of this wave (multiples of 16 from the split's start)
  const int sub = kWpi == 1 ? p.chunk : ((p.chunk / 16 + kWpi - 1) / kWpi) * 16;
  const int t0 = sp * p.chunk + (kWpi == 1 ? 0 : w * sub);
  const int t1 = min(min(t0 + sub, sp * p.chunk + p.chunk), L);
  const int nmed = t1 > t0 ? (t1 - t0 + 15) >> 4 : 0;

  uint8_t* wl = attn_smem + AttnLds<kMode>::kTables + w * AttnLds<kMode>::kWave;
  constexpr int kStage = kMode == kModeCanon ? kStBytes : kExpStage;
  uint8_t* stage0 = wl;
  uint8_t* stage1 = wl + kStage;
  uint8_t* vbuf = wl + AttnLds<kMode>::kWave - kVBytes;

  // q^T fragments (B operand): lane l -> head l%16 of this KV group, dims
  // 32c + 8*(l/16) .. +7.  Heads past the group read head 0 and are dropped.
  const int g = l & 15;
  const int qh = h * p.group + (g < p.group ? g : 0);
  const uint16_t* qrow = p.q + ((int64_t)b * p.heads + qh) * kHeadDim + 8 * (l >> 4);
  AttnWave A;
#pragma unroll
  for (int c = 0; c < 4; ++c) A.Q[c] = *reinterpret_cast<const bf16x8*>(qrow + 32 * c);
#pragma unroll
  for (int i = 0; i < 8; ++i) A.O[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  A.m_run = -INFINITY;
  A.l_run = 0.f;
  A.S = f32x4{0.f, 0.f, 0.f, 0.f};
  A.pb0 = A.pb1 = 0;

  // tr16 read address of the V tile: token 4*(l/16) + (l%16)/4, dim 4*(l%4)
  // (+16 per 16-dim block) -> lane gets V[4*(l/16)+j][16*blk + l%16], j=0..3.
  const int vtr = (4 * (l >> 4) + ((l & 15) >> 2)) * kVRow + 8 * (l & 3);
  // ds_write of the decoded half h: token l%16, dims 32h + 8*(l/16).
  const int vwr = (l & 15) * kVRow + 16 * (l >> 4);

  const int k_rowbase = kDense ? 0 : b * p.k_bsr + h * p.k_hsr + t0;
  const int v_rowbase = kDense ? 0 : b * p.v_bsr + h * p.v_hsr + t0;
  const uint8_t* bmk = l < 8 ? p.k.bm1 : (l < 16 ? p.k.bm2 : p.k.bm3);
  const uint8_t* bmv = l < 8 ? p.v.bm1 : (l < 16 ? p.v.bm2 : p.v.bm3);

  // Dense rows: token of lane l in median `med`, clamped to the valid range.
  // Paged caches: a median (16 tokens from a multiple of 16) lies in one
  // page; lane i of `pdelta` holds (physical - logical page) * page for
  // median 64 * pchunk + i, loaded once per 64 medians, so the row of token t
  // is t + pdelta[med].
  int pdelta = 0, pchunk = -1;
  auto dense_row = [&](const uint16_t* base, int med) -> const uint16_t* {
    const int t = min(t0 + 16 * med + (l & 15), L - 1);
    if constexpr (kMode == kModePaged) {
      const int ch = med >> 6;
      if (ch != pchunk) {
        const int lp = (t0 + 16 * min(64 * ch + l, nmed - 1)) / p.page;
        pdelta = (p.block_table[(int64_t)b * p.bt_stride + lp] - lp) * p.page;
        pchunk = ch;
      }
      const int64_t row = (int64_t)t + __builtin_amdgcn_readlane(pdelta, med & 63);
      return base + (row * p.heads_k + h) * kHeadDim + 8 * (l >> 4);
    } else {
      return base + (((int64_t)b * p.cap + t) * p.heads_k + h) * kHeadDim + 8 * (l >> 4);
    }
  };

  // One step: consume the fragments (a0, a1) of step type TY (0 = K0, 1 = K1,
  // 2 = V0, 3 = V1) for median `med`.
  auto consume = [&](int TY, int med, u32x4 a0, u32x4 a1) {
    if (TY < 2) {
      attn_k_step(A, TY, a0, a1);
      if (TY == 1) attn_softmax(A, t0 + 16 * med + 4 * (l >> 4), t1, p.scale_log2);
    } else {
      // V^T P^T for the 64 dims of this column tile, via the LDS transpose
      *reinterpret_cast<u32x4*>(vbuf + vwr) = a0;
      *reinterpret_cast<u32x4*>(vbuf + vwr + 64) = a1;
      attn_v_step(A, TY, vbuf + vtr);
    }
  };

  // Re-tiled start-up (branch-free, so the compiler's wait counts stay
  // exact): the first chunk's outlier offsets and the fixed parts of steps
  // 0..3 go out together; the outlier bytes follow as soon as the offsets
  // land, the decode table is computed meanwhile, and the workgroup
  // synchronises.  Waves without tokens fetch clamped, in-bounds records.
  RStage R0, R1, R2, R3;
  RMeta M0, M1, M2, M3;
  int oe0 = 0, oe1 = 0;
  auto rrec = [&](int j) {  // record of step j of the wave's range, clamped
    const int ty = j & 3, med = j >> 2;
    const int64_t r = (int64_t)(((ty < 2 ? k_rowbase : v_rowbase) >> 4) + med) * 2 + (ty & 1);
    return (int64_t)max(min(r, (int64_t)(ty < 2 ? p.k_nrec : p.v_nrec) - 1), (int64_t)0);
  };
  if constexpr (kMode == kModeRetiled) {
    constexpr int kNT = (kWpi == 1 ? kAttnWaves : kWpi) * 64;
    const int lastc = max(min(4 * nmed, 64) - 1, 3);
    {
      const int j = min(l, lastc);
      const int64_t rec = rrec(j);
      const int32_t* eo = (j & 3) < 2 ? p.keo : p.veo;
      oe0 = eo[rec];
      oe1 = eo[rec + 1];
    }
    r_issue_fixed(p.kfix, rrec(0), R0);
    r_issue_fixed(p.kfix, rrec(1), R1);
    r_issue_fixed(p.vfix, rrec(2), R2);
    r_issue_fixed(p.vfix, rrec(3), R3);
    r_issue_exps(p.kexp, __builtin_amdgcn_readlane(oe0, 0), __builtin_amdgcn_readlane(oe1, 0), R0, M0);
    r_issue_exps(p.kexp, __builtin_amdgcn_readlane(oe0, 1), __builtin_amdgcn_readlane(oe1, 1), R1, M1);
    r_issue_exps(p.vexp, __builtin_amdgcn_readlane(oe0, 2), __builtin_amdgcn_readlane(oe1, 2), R2, M2);
    r_issue_exps(p.vexp, __builtin_amdgcn_readlane(oe0, 3), __builtin_amdgcn_readlane(oe1, 3), R3, M3);
    build_r_tables(RT, threadIdx.x, kNT);
    __syncthreads();
    if (item0 >= nitems) return;  // uniform when kWpi > 1
  }

  if (nmed > 0) {
    const int nstep = 4 * nmed;
    const int last = nstep - 1;
    if constexpr (kDense) {
      // Fragments fetched four steps ahead straight into registers.
      u32x4 A0[4], A1[4];
      auto fetch = [&](int j, u32x4& x0, u32x4& x1) {
        const int ty = j & 3, med = j >> 2;
        const uint16_t* r = dense_row(ty < 2 ? p.kd : p.vd, med) + 64 * (ty & 1);
        x0 = *reinterpret_cast<const u32x4*>(r);
        x1 = *reinterpret_cast<const u32x4*>(r + 32);
      };
#pragma unroll
      for (int i = 0; i < 4; ++i) fetch(i, A0[i], A1[i]);  // nstep >= 4
      for (int j = 0; j < nstep; j += 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const u32x4 a0 = A0[i], a1 = A1[i];
          const int jn = j + 4 + i;
          fetch(jn <= last ? jn : ((last & ~3) | i), A0[i], A1[i]);
          consume(i, (j >> 2), a0, a1);
        }
      }
    } else if constexpr (kMode == kModeRetiled) {
      // Records fetched four steps ahead into registers; outlier bytes staged
      // one step ahead.  Steps K0,K1,V0,V1 of median `med` are the records
      // of its band in K (column tiles 0, 1), then in V.  Buffer resources
      // from this wave's first K / V record are built once; a step's record
      // goes into the scalar offset.
      const int64_t kr0 = (int64_t)(k_rowbase >> 4) * 2, vr0 = (int64_t)(v_rowbase >> 4) * 2;
      const __amdgpu_buffer_rsrc_t kfr =
          r_buffer(p.kfix + kr0 * kRecBytes, r_range((p.k_nrec - kr0) * kRecBytes));
      const __amdgpu_buffer_rsrc_t vfr =
          r_buffer(p.vfix + vr0 * kRecBytes, r_range((p.v_nrec - vr0) * kRecBytes));
      for (int c0 = 0; c0 < nstep; c0 += 64) {
        const int n = min(nstep - c0, 64);
        const int lastc = n - 1;
        if (c0 > 0) {
          const int j = c0 + min(l, lastc);
          const int ty = j & 3, med = j >> 2;
          const int64_t rec = (int64_t)(((ty < 2 ? k_rowbase : v_rowbase) >> 4) + med) * 2 + (ty & 1);
          const int32_t* eo = ty < 2 ? p.keo : p.veo;
          oe0 = eo[rec];
          oe1 = eo[rec + 1];
        }
#define ZR_ISSUE(J, I, R, MT)                                                           \
  {                                                                                     \
    const int jj_ = (J);                                                                \
    const int med_ = (c0 + jj_) >> 2;                                                   \
    r_issue_fixed_r((I) < 2 ? kfr : vfr, (uint32_t)(med_ * 2 + ((I) & 1)) * kRecBytes, R); \
    r_issue_exps((I) < 2 ? p.kexp : p.vexp, __builtin_amdgcn_readlane(oe0, jj_),       \
                 __builtin_amdgcn_readlane(oe1, jj_), R, MT);                           \
  }
#define ZR_CLAMP(J, I) ((J) <= lastc ? (J) : ((lastc & ~3) | (I)))
#define ZR_STEP(J, I, CUR, NXT, RC, MC, RN, MN)                                         \
  {                                                                                     \
    const RStage cs_ = RC;                                                              \
    const RMeta cm_ = MC;                                                               \
    r_stage(NXT, RN, MN);                                                               \
    ZR_ISSUE(ZR_CLAMP((J) + 4, I), I, RC, MC);                                          \
    u32x4 a0_, a1_;                                                                     \
    if (r_staged(cm_))                                                                  \
      r_decode(RT, (I) < 2 ? kex : vex, cs_.r, (const uint8_t*)(CUR), cm_.rel, a0_, a1_);   \
    else                                                                                \
      r_decode(RT, (I) < 2 ? kex : vex, cs_.r, ((I) < 2 ? p.kexp : p.vexp) + cm_.e0,    \
               0, a0_, a1_);                                                            \
    consume((I), (c0 + (J)) >> 2, a0_, a1_);                                            \
  }
        if (c0 > 0) {  // chunk 0's first steps were issued at start-up
          ZR_ISSUE(0, 0, R0, M0);  // n >= 4: a chunk holds whole medians
          ZR_ISSUE(1, 1, R1, M1);
          ZR_ISSUE(2, 2, R2, M2);
          ZR_ISSUE(3, 3, R3, M3);
        }
        r_stage(stage0, R0, M0);
        for (int j = 0; j < n; j += 4) {
          ZR_STEP(j, 0, stage0, stage1, R0, M0, R1, M1);
          ZR_STEP(j + 1, 1, stage1, stage0, R1, M1, R2, M2);
          ZR_STEP(j + 2, 2, stage0, stage1, R2, M2, R3, M3);
          ZR_STEP(j + 3, 3, stage1, stage0, R3, M3, R0, M0);
        }
#undef ZR_STEP
#undef ZR_CLAMP
#undef ZR_ISSUE
      }
    } else {
      // Offsets of up to 64 steps at a time (lane i -> step c0 + i).
      for (int c0 = 0; c0 < nstep; c0 += 64) {
        const int n = min(nstep - c0, 64);
        const int lastc = n - 1;
        TileOff offs{0, 0, 0, 0};
        {
          const int j = c0 + min(l, lastc);
          const int ty = j & 3, med = j >> 2;
          const Streams& st = ty < 2 ? p.k : p.v;
          const int rb = ty < 2 ? k_rowbase : v_rowbase;
          offs = load_tile_offsets(st, kv_tile(rb, med, ty & 1), kv_median(rb, med), true);
        }
        StageRegs R0, R1, R2, R3;
        StageMeta M0, M1, M2, M3;
        // step index within the chunk -> (type, median) of the whole range
// Step type I (0..3) is a literal at every use, so the K / V choice is static.
#define ZA_ISSUE(J, I, R, MT)                                                          \
  {                                                                                    \
    const int jj_ = (J);                                                               \
    const int med_ = (c0 + jj_) >> 2;                                                  \
    stage_issue((I) < 2 ? p.k : p.v, (I) < 2 ? bmk : bmv,                              \
                kv_tile((I) < 2 ? k_rowbase : v_rowbase, med_, (I) & 1),               \
                kv_median((I) < 2 ? k_rowbase : v_rowbase, med_),                      \
                tile_off_at(offs, jj_), R, MT);                                        \
  }
        // Clamp keeps the step type of the slot (c0 and n are multiples of 4).
#define ZA_CLAMP(J, I) ((J) <= lastc ? (J) : ((lastc & ~3) | (I)))
#define ZA_STEP(J, I, CUR, NXT, RC, MC, RN)                                            \
  {                                                                                    \
    const StageMeta cm_ = MC;                                                          \
    stage_write(NXT, RN);                                                              \
    ZA_ISSUE(ZA_CLAMP((J) + 4, I), I, RC, MC);                                            \
    const Streams& st_ = (I) < 2 ? p.k : p.v;                                          \
    u32x4 a0_, a1_;                                                                    \
    decode_median_pair(T, (I) < 2 ? T.e1 : e1v, CUR + kStBm, 128, CUR + kStSm,         \
                       cm_.sm_rel, reinterpret_cast<const uint16_t*>(CUR + kStFull),   \
                       cm_.full_rel, cm_.full_direct, st_.full + cm_.fa0, a0_, a1_);   \
    consume((I), (c0 + (J)) >> 2, a0_, a1_);                                           \
  }
        ZA_ISSUE(0, 0, R0, M0);  // n >= 4: a chunk holds whole medians
        ZA_ISSUE(1, 1, R1, M1);
        ZA_ISSUE(2, 2, R2, M2);
        ZA_ISSUE(3, 3, R3, M3);
        stage_write(stage0, R0);
        for (int j = 0; j < n; j += 4) {
          ZA_STEP(j, 0, stage0, stage1, R0, M0, R1);
          ZA_STEP(j + 1, 1, stage1, stage0, R1, M1, R2);
          ZA_STEP(j + 2, 2, stage0, stage1, R2, M2, R3);
          ZA_STEP(j + 3, 3, stage1, stage0, R3, M3, R0);
        }
#undef ZA_STEP
#undef ZA_CLAMP
#undef ZA_ISSUE
      }
    }
  }

  if constexpr (kWpi > 1) {
    // Merge the waves' softmax states (log2 domain) into wave 0; the decode
    // tables are dead by now, their LDS holds the states.
    __syncthreads();
    float* cb = reinterpret_cast<float*>(attn_smem) + w * 34 * 64 + l;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) cb[(4 * i + r) * 64] = A.O[i][r];
    cb[32 * 64] = A.m_run;
    cb[33 * 64] = A.l_run;
    __syncthreads();
    if (w != 0) return;
    const float* c0 = reinterpret_cast<const float*>(attn_smem) + l;
    float m = -INFINITY;
#pragma unroll
    for (int v = 0; v < kWpi; ++v) m = fmaxf(m, c0[(v * 34 + 32) * 64]);
    const float m_use = m == -INFINITY ? 0.f : m;
    float lsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) A.O[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < kWpi; ++v) {
      const float lv = c0[(v * 34 + 33) * 64];
      const float sc = lv > 0.f ? __builtin_amdgcn_exp2f(c0[(v * 34 + 32) * 64] - m_use) : 0.f;
      lsum += lv * sc;
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) A.O[i][r] += c0[(v * 34 + 4 * i + r) * 64] * sc;
    }
    A.m_run = m;
    A.l_run = lsum;
  }

  // Results: lane l holds head g = l%16, dims 16*i + 4*(l/16) + r of A.O[i].
  const int head = h * p.group + g;
  const bool own = g < p.group;
  const int d0 = 4 * (l >> 4);
  if (p.splits == 1) {
    if (own) {
      const float inv = A.l_run > 0.f ? 1.f / A.l_run : 0.f;
      uint16_t* orow = p.out + ((int64_t)b * p.heads + head) * kHeadDim + d0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint2 v;
        v.x = pack_bf16x2(A.O[i][0] * inv, A.O[i][1] * inv);
        v.y = pack_bf16x2(A.O[i][2] * inv, A.O[i][3] * inv);
        *reinterpret_cast<uint2*>(orow + 16 * i) = v;
      }
      if (p.lse && l < 16)
        p.lse[(int64_t)b * p.heads + head] =
            A.l_run > 0.f ? (A.m_run + __log2f(A.l_run)) * 0.6931471805599453f : -INFINITY;
    }
  } else if (own) {
    const int64_t slot = ((int64_t)b * p.heads + head) * p.splits + sp;
    float* wo = p.ws_o + slot * kHeadDim + d0;
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<f32x4*>(wo + 16 * i) = A.O[i];
    if (l < 16) {
      p.ws_ml[2 * slot] = A.m_run;
      p.ws_ml[2 * slot + 1] = A.l_run;
    }
  }
}

// ---------------------------------------------------------------------------
// Fused decode attention over a token-major re-tiled cache with 8 KV heads
// (rows b * batch_stride + t * 8 + h, bench_zipserv_decode_attention.py:
// 337-344): a 16-row record band holds tokens 2j, 2j+1 of all 8 heads, so
// one head's 16 tokens are spread over 8 bands.  A workgroup of 8 waves
// takes one (batch, split) item and walks it 16 tokens (8 bands) at a time
// in four phases (K dims 0..63, K dims 64..127, V dims 0..63, V 64..127):
//   decode: wave w decodes the phase's record of band w -- lane l holds row
//           l%16 = (token 2w + (l%16)/8, head l%8) -- and writes its two
//           16-byte halves into the phase's exchange tile in LDS, laid out
//           per head as 16 tokens x 64 dims (row pitch kVRow);
//   barrier;
//   compute: wave h reads head h's tile -- as the K fragment (A operand of
//           S^T = K q^T) or through ds_read_b64_tr_b16 as V^T -- and runs
//           the head-major kernel's arithmetic on it (attn_k_step,
//           attn_softmax, attn_v_step).
// Every record is decoded once (the reference decodes each token-major tile
// once per KV head and keeps the rows of that head,
// flash_fwd_kernel.h:325-430), and head h's operands are the values the
// dense kernel reads for it, in the same order, so with one wave per (batch,
// head, split) in both the results are the same bit for bit.  With records
// one step (four phases) ahead, phases alternate between two exchange tiles,
// so one barrier per phase orders both the writes before the reads and the
// reads before the next writes to the same tile.  With records two steps
// ahead (grids of at most one workgroup per CU, where LDS does not limit
// occupancy) every phase has its own tile and a wave decodes the K pair,
// then the V pair, of a step before each barrier: two barriers per step
// instead of four, and two independent decodes per wave between them.
// Outlier bytes are staged one phase ahead, as in attn_kernel.
// ---------------------------------------------------------------------------
constexpr int kTmHeads = 8;                      // KV heads of the fused layout
constexpr int kTmWaves = 8;                      // one wave per band / KV head
// one head's 16 x 64 tile, padded by 16 bytes: a decoding wave's lanes 0..7
// write the same row of 8 heads' tiles, which 16 x kVRow bytes apart would
// all start in one LDS bank (640 dwords, a multiple of the 64 banks)
constexpr int kTmTile = 16 * kVRow + 16;
constexpr int kTmPhase = kTmHeads * kTmTile;     // one phase's exchange tile
// Exchange tiles: two (phases alternate) with the one-step ring; four (one
// per phase) with the two-step ring, whose workgroups decode a K or V pair
// before each barrier.
template <int D>
constexpr int tm_lds() {
  return (int)sizeof(RTables) + kTmWaves * 2 * kExpStage + (D == 8 ? 4 : 2) * kTmPhase;
}

template <int D>
__global__ __launch_bounds__(kTmWaves * 64, D == 4 ? 4 : 2) void attn_tm_kernel(AttnParams p) {
  static_assert(D % 4 == 0, "the ring holds whole steps");
  constexpr bool kPair = D == 8;
  __shared__ __attribute__((aligned(16))) uint8_t attn_smem[tm_lds<D>()];
  RTables& RT = *reinterpret_cast<RTables*>(attn_smem);
  const RExp kex = r_exp(p.k_start), vex = r_exp(p.v_start);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  const int item = blockIdx.x;
  const int sp = item % p.splits;
  const int b = item / p.splits;
  int L = p.seqlen_k;
  if (p.seqlens) L = min(L, __builtin_amdgcn_readfirstlane(p.seqlens[b]));
  L = max(L, 0);
  const int t0 = sp * p.chunk;
  const int t1 = min(t0 + p.chunk, L);
  const int nmed = t1 > t0 ? (t1 - t0 + 15) >> 4 : 0;  // uniform over the workgroup

  uint8_t* stage0 = attn_smem + sizeof(RTables) + w * 2 * kExpStage;
  uint8_t* stage1 = stage0 + kExpStage;
  uint8_t* xch = attn_smem + sizeof(RTables) + kTmWaves * 2 * kExpStage;

  // compute role: KV head h = w, query heads h * group + l%16 (past the group:
  // head 0's, dropped)
  const int h = w;
  const int g = l & 15;
  const int qh = h * p.group + (g < p.group ? g : 0);
  const uint16_t* qrow = p.q + ((int64_t)b * p.heads + qh) * kHeadDim + 8 * (l >> 4);
  AttnWave A;
#pragma unroll
  for (int c = 0; c < 4; ++c) A.Q[c] = *reinterpret_cast<const bf16x8*>(qrow + 32 * c);
#pragma unroll
  for (int i = 0; i < 8; ++i) A.O[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  A.m_run = -INFINITY;
  A.l_run = 0.f;
  A.S = f32x4{0.f, 0.f, 0.f, 0.f};
  A.pb0 = A.pb1 = 0;
  // head h's tile: K fragment read (token l%16, dims 8*(l/16), +32 dims at
  // +64 bytes) and V^T transposed read (token 4*(l/16) + (l%16)/4, dim 4*(l%4))
  const int krd = h * kTmTile + (l & 15) * kVRow + 16 * (l >> 4);
  const int vtr = h * kTmTile + (4 * (l >> 4) + ((l & 15) >> 2)) * kVRow + 8 * (l & 3);
  // decode role: row l%16 of band w is (token 2w + (l%16)/8, head l%8)
  const int xwr = (l & 7) * kTmTile + (2 * w + ((l & 15) >> 3)) * kVRow + 16 * (l >> 4);

  // Band of step `med` for this wave (clamped to the cache: a last step past
  // the rows of the last batch reads real, finite records whose tokens are
  // masked), record = band * 2 + column tile.
  const int nbands_k = p.k_nrec >> 1, nbands_v = p.v_nrec >> 1;
  const int kb0 = (int)(((int64_t)b * p.k_bsr) >> 4) + (t0 >> 1);
  const int vb0 = (int)(((int64_t)b * p.v_bsr) >> 4) + (t0 >> 1);
  auto rrec = [&](int j) {  // record of phase j of this wave's sequence
    const int ty = j & 3, med = j >> 2;
    const int band = ty < 2 ? min(kb0 + 8 * med + w, nbands_k - 1)
                            : min(vb0 + 8 * med + w, nbands_v - 1);
    return (int64_t)band * 2 + (ty & 1);
  };
  const int64_t kr0 = (int64_t)min(kb0 + w, nbands_k - 1) * 2;
  const int64_t vr0 = (int64_t)min(vb0 + w, nbands_v - 1) * 2;
  const __amdgpu_buffer_rsrc_t kfr =
      r_buffer(p.kfix + kr0 * kRecBytes, r_range((p.k_nrec - kr0) * kRecBytes));
  const __amdgpu_buffer_rsrc_t vfr =
      r_buffer(p.vfix + vr0 * kRecBytes, r_range((p.v_nrec - vr0) * kRecBytes));

  // Start-up, branch-free: the first chunk's outlier offsets and phases
  // 0..D-1's fixed parts go out together, the outlier bytes once the
  // offsets land; the decode table is computed meanwhile.
  RStage R[D];
  RMeta MT[D];
  int oe0 = 0, oe1 = 0;
  const int nstep = 4 * nmed;
  {
    const int lastc = max(min(nstep, 64) - 1, D - 1);
    const int j = min(l, lastc);
    const int64_t rec = rrec(j);
    const int32_t* eo = (j & 3) < 2 ? p.keo : p.veo;
    oe0 = eo[rec];
    oe1 = eo[rec + 1];
  }
  {
#pragma unroll
    for (int k = 0; k < D; ++k)
      r_issue_fixed_r((k & 3) < 2 ? kfr : vfr,
                      (uint32_t)(rrec(k) - ((k & 3) < 2 ? kr0 : vr0)) * kRecBytes, R[k]);
#pragma unroll
    for (int k = 0; k < D; ++k)
      r_issue_exps((k & 3) < 2 ? p.kexp : p.vexp, __builtin_amdgcn_readlane(oe0, k),
                   __builtin_amdgcn_readlane(oe1, k), R[k], MT[k]);
    build_r_tables(RT, threadIdx.x, kTmWaves * 64);
  }
  __syncthreads();

  for (int c0 = 0; c0 < nstep; c0 += 64) {
    const int n = min(nstep - c0, 64);
    const int lastc = n - 1;
    if (c0 > 0) {
      const int j = c0 + min(l, lastc);
      const int64_t rec = rrec(j);
      const int32_t* eo = (j & 3) < 2 ? p.keo : p.veo;
      oe0 = eo[rec];
      oe1 = eo[rec + 1];
    }
#define ZT_ISSUE(J, I, R, MT)                                                              \
  {                                                                                        \
    const int jj_ = (J);                                                                   \
    const int64_t rec_ = rrec(c0 + jj_);                                                   \
    r_issue_fixed_r((I) < 2 ? kfr : vfr, (uint32_t)(rec_ - ((I) < 2 ? kr0 : vr0)) * kRecBytes, R); \
    r_issue_exps((I) < 2 ? p.kexp : p.vexp, __builtin_amdgcn_readlane(oe0, jj_),          \
                 __builtin_amdgcn_readlane(oe1, jj_), R, MT);                              \
  }
#define ZT_CLAMP(J, I) ((J) <= lastc ? (J) : ((lastc & ~3) | (I)))
    // (a chunk of n phases, n a multiple of 4 but maybe not of D: the issue
    // clamp keeps every fetch in the chunk, and steps past n are skipped)
#define ZT_DEC(J, I, CUR, NXT, RC, MC, RN, MN)                                             \
  {                                                                                        \
    const RStage cs_ = RC;                                                                 \
    const RMeta cm_ = MC;                                                                  \
    r_stage(NXT, RN, MN);                                                                  \
    ZT_ISSUE(ZT_CLAMP((J) + D, I), I, RC, MC);                                             \
    u32x4 a0_, a1_;                                                                        \
    if (r_staged(cm_))                                                                     \
      r_decode(RT, (I) < 2 ? kex : vex, cs_.r, (const uint8_t*)(CUR), cm_.rel, a0_, a1_);  \
    else                                                                                   \
      r_decode(RT, (I) < 2 ? kex : vex, cs_.r, ((I) < 2 ? p.kexp : p.vexp) + cm_.e0, 0,    \
               a0_, a1_);                                                                  \
    uint8_t* xt_ = xch + (I) * kTmPhase;                                                   \
    *reinterpret_cast<u32x4*>(xt_ + xwr) = a0_;                                            \
    *reinterpret_cast<u32x4*>(xt_ + xwr + 64) = a1_;                                       \
  }
#define ZT_KC(J, I)                                                                        \
  {                                                                                        \
    const uint8_t* xt_ = xch + (I) * kTmPhase;                                             \
    const u32x4 k0_ = *reinterpret_cast<const u32x4*>(xt_ + krd);                          \
    const u32x4 k1_ = *reinterpret_cast<const u32x4*>(xt_ + krd + 64);                     \
    attn_k_step(A, (I), k0_, k1_);                                                         \
    if ((I) == 1) attn_softmax(A, t0 + 16 * ((c0 + (J)) >> 2) + 4 * (l >> 4), t1, p.scale_log2); \
  }
#define ZT_STEP(J, I, CUR, NXT, RC, MC, RN, MN)                                            \
  {                                                                                        \
    const RStage cs_ = RC;                                                                 \
    const RMeta cm_ = MC;                                                                  \
    r_stage(NXT, RN, MN);                                                                  \
    ZT_ISSUE(ZT_CLAMP((J) + D, I), I, RC, MC);                                             \
    u32x4 a0_, a1_;                                                                        \
    if (r_staged(cm_))                                                                     \
      r_decode(RT, (I) < 2 ? kex : vex, cs_.r, (const uint8_t*)(CUR), cm_.rel, a0_, a1_);  \
    else                                                                                   \
      r_decode(RT, (I) < 2 ? kex : vex, cs_.r, ((I) < 2 ? p.kexp : p.vexp) + cm_.e0, 0,    \
               a0_, a1_);                                                                  \
    uint8_t* xt_ = xch + ((I) & 1) * kTmPhase;                                             \
    *reinterpret_cast<u32x4*>(xt_ + xwr) = a0_;                                            \
    *reinterpret_cast<u32x4*>(xt_ + xwr + 64) = a1_;                                       \
    __syncthreads();                                                                       \
    if ((I) < 2) {                                                                         \
      const u32x4 k0_ = *reinterpret_cast<const u32x4*>(xt_ + krd);                        \
      const u32x4 k1_ = *reinterpret_cast<const u32x4*>(xt_ + krd + 64);                   \
      attn_k_step(A, (I), k0_, k1_);                                                       \
      if ((I) == 1)                                                                        \
        attn_softmax(A, t0 + 16 * ((c0 + (J)) >> 2) + 4 * (l >> 4), t1, p.scale_log2);    \
    } else {                                                                               \
      attn_v_step(A, (I), xt_ + vtr);                                                      \
    }                                                                                      \
  }
    if (c0 > 0) {  // chunk 0's first phases were issued at start-up
#pragma unroll
      for (int k = 0; k < D; ++k) ZT_ISSUE(min(k, (lastc & ~3) | (k & 3)), k & 3, R[k], MT[k]);
    }
    r_stage(stage0, R[0], MT[0]);
    for (int j = 0; j < n; j += D) {
      if constexpr (kPair) {
        // per step: K pair decoded, barrier, QK^T and softmax; V pair
        // decoded, barrier, PV.  A wave writes a tile again only after the
        // next barrier that every wave reaches after its reads of it.
#pragma unroll
        for (int k = 0; k < D; k += 4) {
          if (k == 0 || j + k < n) {
            ZT_DEC(j + k, 0, stage0, stage1, R[k], MT[k], R[k + 1], MT[k + 1]);
            ZT_DEC(j + k + 1, 1, stage1, stage0, R[k + 1], MT[k + 1], R[k + 2], MT[k + 2]);
            __syncthreads();
            ZT_KC(j + k, 0);
            ZT_KC(j + k + 1, 1);
            ZT_DEC(j + k + 2, 2, stage0, stage1, R[k + 2], MT[k + 2], R[k + 3], MT[k + 3]);
            ZT_DEC(j + k + 3, 3, stage1, stage0, R[k + 3], MT[k + 3], R[(k + 4) % D],
                   MT[(k + 4) % D]);
            __syncthreads();
            attn_v_step(A, 2, xch + 2 * kTmPhase + vtr);
            attn_v_step(A, 3, xch + 3 * kTmPhase + vtr);
          }
        }
      } else {
#pragma unroll
        for (int k = 0; k < D; ++k) {
          if (k < 4 || j + k < n)
            ZT_STEP(j + k, k & 3, (k & 1) ? stage1 : stage0, (k & 1) ? stage0 : stage1, R[k],
                    MT[k], R[(k + 1) % D], MT[(k + 1) % D]);
        }
      }
    }
#undef ZT_KC
#undef ZT_DEC
#undef ZT_STEP
#undef ZT_CLAMP
#undef ZT_ISSUE
  }

  // Results, as attn_kernel: lane l holds head h * group + l%16.
  const int head = h * p.group + g;
  const bool own = g < p.group;
  const int d0 = 4 * (l >> 4);
  if (p.splits == 1) {
    if (own) {
      const float inv = A.l_run > 0.f ? 1.f / A.l_run : 0.f;
      uint16_t* orow = p.out + ((int64_t)b * p.heads + head) * kHeadDim + d0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        uint2 v;
        v.x = pack_bf16x2(A.O[i][0] * inv, A.O[i][1] * inv);
        v.y = pack_bf16x2(A.O[i][2] * inv, A.O[i][3] * inv);
        *reinterpret_cast<uint2*>(orow + 16 * i) = v;
      }
      if (p.lse && l < 16)
        p.lse[(int64_t)b * p.heads + head] =
            A.l_run > 0.f ? (A.m_run + __log2f(A.l_run)) * 0.6931471805599453f : -INFINITY;
    }
  } else if (own) {
    const int64_t slot = ((int64_t)b * p.heads + head) * p.splits + sp;
    float* wo = p.ws_o + slot * kHeadDim + d0;
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<f32x4*>(wo + 16 * i) = A.O[i];
    if (l < 16) {
      p.ws_ml[2 * slot] = A.m_run;
      p.ws_ml[2 * slot + 1] = A.l_run;
    }
  }
}

// Merges the split partials of one (batch, head) with W waves: the split
// weights exp2(m_s - m) are computed once per chunk of splits into LDS, then
// wave w takes splits 8w..8w+7 of every 8W (lane l owns dims 2l, 2l+1), so
// each wave has eight independent partial-output loads in flight and the W
// wave sums meet in LDS.  A wave's first eight partial loads go out before
// the split maximum is known (they do not depend on it), so they overlap
// its reduction.  W = 16 for more than 32 splits (two rounds of loads per
// wave at 256 splits instead of eight with four waves), else 4.
constexpr int kCombineChunk = 512;

template <int W>
__device__ __forceinline__ float block_reduce(float x, bool is_max, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float y = __shfl_xor(x, off);
    x = is_max ? fmaxf(x, y) : x + y;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < W; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
  __syncthreads();
  return r;
}

template <int W>
__global__ __launch_bounds__(W * 64) void attn_combine_kernel(AttnParams p) {
  constexpr int NT = W * 64;
  __shared__ float sc[kCombineChunk];
  __shared__ float red[W];
  __shared__ float2 part[W - 1][64];
  const int bh = blockIdx.x;
  const int t = threadIdx.x, w = t >> 6, l = t & 63;
  const int S = p.splits;
  const float* ml = p.ws_ml + (int64_t)bh * S * 2;
  const float* wo = p.ws_o + (int64_t)bh * S * kHeadDim + 2 * l;
  float2 x[8];
  {
    const int n = min(S, kCombineChunk);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      x[j] = 8 * w + j < n ? *reinterpret_cast<const float2*>(wo + (int64_t)(8 * w + j) * kHeadDim)
                           : float2{0.f, 0.f};
  }
  float m = -INFINITY;
  for (int s = t; s < S; s += NT) m = fmaxf(m, ml[2 * s]);
  m = block_reduce<W>(m, true, red);
  const float m_use = m == -INFINITY ? 0.f : m;
  float lpart = 0.f;
  float2 acc = {0.f, 0.f};
  for (int c0 = 0; c0 < S; c0 += kCombineChunk) {
    const int n = min(S - c0, kCombineChunk);
    for (int i = t; i < n; i += NT) {
      const float2 e = *reinterpret_cast<const float2*>(ml + 2 * (c0 + i));
      const float wgt = e.y > 0.f ? __builtin_amdgcn_exp2f(e.x - m_use) : 0.f;
      sc[i] = wgt;
      lpart += e.y * wgt;
    }
    __syncthreads();
    const float* wc = wo + (int64_t)c0 * kHeadDim;
    for (int i0 = 8 * w; i0 < n; i0 += 8 * W) {
      if (c0 > 0 || i0 > 8 * w) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          x[j] = i0 + j < n ? *reinterpret_cast<const float2*>(wc + (int64_t)(i0 + j) * kHeadDim)
                            : float2{0.f, 0.f};
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float g = i0 + j < n ? sc[i0 + j] : 0.f;
        acc.x += x[j].x * g;
        acc.y += x[j].y * g;
      }
    }
    __syncthreads();
  }
  const float lsum = block_reduce<W>(lpart, false, red);
  if (w > 0) part[w - 1][l] = acc;
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int i = 0; i < W - 1; ++i) {
      acc.x += part[i][l].x;
      acc.y += part[i][l].y;
    }
    const float vx = lsum > 0.f ? acc.x / lsum : 0.f, vy = lsum > 0.f ? acc.y / lsum : 0.f;
    *reinterpret_cast<uint32_t*>(p.out + (int64_t)bh * kHeadDim + 2 * l) =
        f32_to_bf16_bits(vx) | (f32_to_bf16_bits(vy) << 16);
    if (p.lse && l == 0)
      p.lse[bh] = lsum > 0.f ? (m + __log2f(lsum)) * 0.6931471805599453f : -INFINITY;
  }
}

static hipError_t launch_combine(hipStream_t st, const AttnParams& p) {
  if (p.splits > 32)
    hipLaunchKernelGGL(attn_combine_kernel<16>, dim3(p.batch * p.heads), dim3(16 * 64), 0, st, p);
  else
    hipLaunchKernelGGL(attn_combine_kernel<4>, dim3(p.batch * p.heads), dim3(4 * 64), 0, st, p);
  return hipGetLastError();
}

// Workgroups of four waves per item take grids of fewer than this many items.
constexpr int kSharedItemsBelow = 2048;

static int attn_auto_splits(int batch, int heads_k, int seqlen_k, bool compressed) {
  // One wave per item: about 2048 waves, at least 256 tokens per split.
  // Smaller grids run four waves per item (attn_launch).  There the
  // compressed modes, whose record -> exponent-stream loads form a longer
  // latency chain, measure best at about 512 items (2048 waves; B=1 T=32k
  // 43 -> 34 us, B=8 T=4k 43 -> 32 us) and the dense mode at about 256,
  // with splits of at least 128 tokens (32 per wave; B=1 T=4k against
  // 256-token splits: 16.0 -> 12.8 us compressed, 11.7 -> 10.0 us dense).
  const int units = std::max(1, batch * heads_k);
  const int max_splits = std::max(1, (seqlen_k + 255) / 256);
  const int s1 = std::min(max_splits, std::max(1, (2048 + units - 1) / units));
  if ((int64_t)s1 * units >= kSharedItemsBelow) return s1;
  const int max_shared = std::max(1, (seqlen_k + 127) / 128);
  const int items = compressed ? 512 : 256;
  return std::min(max_shared, std::max(1, (items + units - 1) / units));
}

// Tokens per split: a multiple of 16 (one median, one record band), so that
// every wave's range starts on a band of every layout.
static int attn_chunk(int seqlen_k, int splits) {
  const int blocks = (seqlen_k + 15) / 16;
  return ((blocks + splits - 1) / splits) * 16;
}

static size_t attn_ws_bytes(int batch, int heads, int splits) {
  if (splits <= 1) return 0;
  return (size_t)batch * heads * splits * (kHeadDim + 2) * sizeof(float);
}

template <int kMode>
static int attn_launch(hipStream_t st, AttnParams& p, void* workspace, size_t ws_bytes) {
  if (p.splits > 1) {
    if (!workspace || ws_bytes < attn_ws_bytes(p.batch, p.heads, p.splits)) return ZS_E_INVAL;
    p.ws_o = reinterpret_cast<float*>(workspace);
    p.ws_ml = p.ws_o + (size_t)p.batch * p.heads * p.splits * kHeadDim;
  }
  const int items = p.batch * p.heads_k * p.splits;
  if (items < kSharedItemsBelow && p.chunk > 64) {
    // small grid: four waves per item
    const size_t lds = std::max<size_t>(AttnLds<kMode>::bytes(kItemWaves), kCombineBytes);
    hipLaunchKernelGGL((attn_kernel<kMode, kItemWaves>), dim3(items), dim3(kItemWaves * 64), lds,
                       st, p);
  } else {
    const int grid = (items + kAttnWaves - 1) / kAttnWaves;
    const size_t lds = AttnLds<kMode>::bytes(kAttnWaves);
    hipLaunchKernelGGL((attn_kernel<kMode, 1>), dim3(grid), dim3(kAttnWaves * 64), lds, st, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  if (p.splits > 1) {
    e = launch_combine(st, p);
  }
  return e == hipSuccess ? ZS_OK : (int)e;
}

static int attn_common_checks(int batch, int heads, int heads_k, int head_dim, int seqlen_k,
                              int num_splits, const void* q, const void* out) {
  if (!q || !out || batch <= 0 || heads <= 0 || heads_k <= 0 || seqlen_k < 0 || num_splits < 0)
    return ZS_E_INVAL;
  if (heads % heads_k) return ZS_E_INVAL;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out)) & 15)
    return ZS_E_INVAL;  // 16-byte q rows in, 8-byte out stores
  if (head_dim != kHeadDim || heads / heads_k > 16) return ZS_E_UNSUPPORTED;
  return ZS_OK;
}

// Geometry of one compressed cache against the call: head-major rows are
// ((b * Hkv + h) * head_stride + t), token-major rows b * batch_stride +
// t * Hkv + h (bench_zipserv_decode_attention.py:337-354).
static int kv_geometry_ok(int layout, int rows, int cols, int bsr, int hsr, int start_exp,
                          int batch, int heads_k, int seqlen_k) {
  if (layout != ZS_LAYOUT_HEAD_MAJOR && layout != ZS_LAYOUT_TOKEN_MAJOR) return ZS_E_UNSUPPORTED;
  if (cols != kHeadDim || rows <= 0 || (rows % 64)) return ZS_E_INVAL;
  if (hsr <= 0 || bsr != heads_k * hsr || (int64_t)bsr * batch > rows || hsr < seqlen_k)
    return ZS_E_INVAL;
  if (layout == ZS_LAYOUT_HEAD_MAJOR ? (hsr % 64) : (bsr % 64)) return ZS_E_INVAL;
  if (start_exp < 0 || start_exp > 255) return ZS_E_INVAL;
  return ZS_OK;
}

static size_t staging_bytes(int layout, int rows, int cols) {
  if (layout != ZS_LAYOUT_TOKEN_MAJOR) return 0;
  return ((size_t)rows * cols * 2 + 255) / 256 * 256;
}

int device_cu_count();  // zs_gemm.hip

// Fused token-major attention (attn_tm_kernel) takes re-tiled caches with
// kTmHeads KV heads; other token-major caches run staged.
static bool tm_fused(int heads_k, int cols) { return heads_k == kTmHeads && cols == kHeadDim; }

// Splits of the fused token-major kernel: one 8-wave workgroup per (batch,
// split), about kTmItems of them (two per CU), at least kTmMinTokens
// tokens and at most kTmMaxSplits splits per sequence (the combine reads
// every split's partial of every head), or one per CU when two per CU would
// leave chunks under 128 tokens; an explicit count is used as given (at
// most one split per 16 tokens).  The chunk is a multiple of 16 tokens (a
// step).  Measured over B = 1..32, T = 2k..32k, each count timed after a
// warm-up in both orders: within 3% of the best of 8..256 splits.
constexpr int kTmItems = 512;
constexpr int kTmMinTokens = 32;
constexpr int kTmMaxSplits = 256;

static int tm_splits(int batch, int seqlen_k, int num_splits) {
  const int steps = std::max(1, (seqlen_k + 15) / 16);
  if (num_splits > 0) return std::min(num_splits, steps);
  const int max_splits = std::max(1, (seqlen_k + kTmMinTokens - 1) / kTmMinTokens);
  int s = std::min(std::min(max_splits, kTmMaxSplits), std::max(1, (kTmItems + batch - 1) / batch));
  // More than one workgroup per CU with chunks under 128 tokens: one round
  // of them (the two-step ring with phase pairs) is faster (B = 8, T = 2k /
  // 4k: 28.0 -> 24.0 / 35.9 -> 34.2 us; B = 4, T = 4k: 26.0 -> 24.5 us).
  if ((int64_t)batch * s > device_cu_count() && seqlen_k < 128 * s)
    s = std::max(1, (device_cu_count() + batch - 1) / batch);
  return s;
}

static int tm_chunk(int seqlen_k, int splits) {
  const int steps = std::max(1, (seqlen_k + 15) / 16);
  return ((steps + splits - 1) / splits) * 16;
}

static int attn_tm_launch(hipStream_t st, AttnParams& p, void* workspace, size_t ws_bytes) {
  if (p.splits > 1) {
    if (!workspace || ws_bytes < attn_ws_bytes(p.batch, p.heads, p.splits)) return ZS_E_INVAL;
    p.ws_o = reinterpret_cast<float*>(workspace);
    p.ws_ml = p.ws_o + (size_t)p.batch * p.heads * p.splits * kHeadDim;
  }
  // Grids of at most one workgroup per CU take the ring of two steps (eight
  // records per wave in flight; two waves per SIMD leave it the registers)
  // and decode phase pairs between barriers, larger grids the ring of one
  // step at four waves per SIMD.
  const int items = p.batch * p.splits;
  if (items <= device_cu_count())
    hipLaunchKernelGGL(attn_tm_kernel<8>, dim3(items), dim3(kTmWaves * 64), 0, st, p);
  else
    hipLaunchKernelGGL(attn_tm_kernel<4>, dim3(items), dim3(kTmWaves * 64), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  if (p.splits > 1) {
    e = launch_combine(st, p);
  }
  return e == hipSuccess ? ZS_OK : (int)e;
}

// Token-major caches run staged: both caches are decompressed into the
// workspace (dense [B][head_stride][Hkv][D] views of their rows) and the
// attention kernel runs in its dense mode on them.
static int attn_staged(hipStream_t st, AttnParams& p, const uint16_t* kd, const uint16_t* vd,
                       int cap, void* workspace, size_t ws_bytes) {
  p.kd = kd;
  p.vd = vd;
  p.cap = cap;
  return attn_launch<kModeDense>(st, p, workspace, ws_bytes);
}

}  // namespace zs

using namespace zs;

extern "C" int64_t zs_kv_staging_bytes(int layout, int rows, int cols) {
  if (rows <= 0 || cols <= 0) return -1;
  if (layout != ZS_LAYOUT_HEAD_MAJOR && layout != ZS_LAYOUT_TOKEN_MAJOR) return -1;
  return (int64_t)staging_bytes(layout, rows, cols);
}

extern "C" size_t zs_decode_attention_workspace_bytes(int batch, int num_heads, int head_dim,
                                                      int seqlen_k, int num_splits) {
  if (batch <= 0 || num_heads <= 0 || head_dim != kHeadDim || seqlen_k < 0) return 0;
  // num_splits == 0 asks for the automatic choice, which never exceeds
  // min(ceil(T/128), ceil(2048/batch)) splits, or for fused token-major
  // caches min(ceil(T/16), ceil(kTmItems/batch)).
  const int splits =
      num_splits > 0
          ? num_splits
          : std::max(std::min(std::max(1, (seqlen_k + 127) / 128), (2048 + batch - 1) / batch),
                     std::min(std::max(1, (seqlen_k + 15) / 16), (kTmItems + batch - 1) / batch));
  return attn_ws_bytes(batch, num_heads, splits);
}

extern "C" int64_t zs_kv_retiled_staging_bytes(int layout, int rows, int cols, int num_heads_k) {
  if (rows <= 0 || cols <= 0 || num_heads_k <= 0) return -1;
  if (layout != ZS_LAYOUT_HEAD_MAJOR && layout != ZS_LAYOUT_TOKEN_MAJOR) return -1;
  if (layout == ZS_LAYOUT_TOKEN_MAJOR && tm_fused(num_heads_k, cols)) return 0;
  return (int64_t)staging_bytes(layout, rows, cols);
}

extern "C" int zs_decode_attention(void* stream, const uint16_t* q, const zs_kv_compressed_t* k,
                                   const zs_kv_compressed_t* v, const int32_t* cache_seqlens,
                                   int seqlen_k, int batch, int num_heads, int num_heads_k,
                                   int head_dim, float softmax_scale, uint16_t* out,
                                   float* softmax_lse, void* workspace, size_t workspace_bytes,
                                   int num_splits) {
  int stc = attn_common_checks(batch, num_heads, num_heads_k, head_dim, seqlen_k, num_splits, q,
                               out);
  if (stc != ZS_OK) return stc;
  if (!k || !v) return ZS_E_INVAL;
  const zs_kv_compressed_t* kv[2] = {k, v};
  for (const zs_kv_compressed_t* c : kv) {
    if (!c->sign_mantissa || !c->compressed_full || !c->bitmap1 || !c->bitmap2 ||
        !c->bitmap3 || !c->tile_offsets_median || !c->tile_offsets_global)
      return ZS_E_INVAL;
    const int g = kv_geometry_ok(c->layout, c->rows, c->cols, c->batch_stride_rows,
                                 c->head_stride_rows, c->start_exp, batch, num_heads_k, seqlen_k);
    if (g != ZS_OK) return g;
  }
  if (k->layout != v->layout || k->head_stride_rows != v->head_stride_rows)
    return ZS_E_UNSUPPORTED;
  AttnParams p{};
  auto streams = [](const zs_kv_compressed_t* c) {
    Streams s;
    s.sm = c->sign_mantissa;
    s.full = c->compressed_full;
    s.bm1 = reinterpret_cast<const uint8_t*>(c->bitmap1);
    s.bm2 = reinterpret_cast<const uint8_t*>(c->bitmap2);
    s.bm3 = reinterpret_cast<const uint8_t*>(c->bitmap3);
    s.tom = c->tile_offsets_median;
    s.tog = c->tile_offsets_global;
    return s;
  };
  p.k = streams(k);
  p.v = streams(v);
  p.k_start = k->start_exp;
  p.v_start = v->start_exp;
  p.k_bsr = k->batch_stride_rows;
  p.k_hsr = k->head_stride_rows;
  p.v_bsr = v->batch_stride_rows;
  p.v_hsr = v->head_stride_rows;
  p.q = q;
  p.out = out;
  p.lse = softmax_lse;
  p.seqlens = cache_seqlens;
  p.seqlen_k = seqlen_k;
  p.batch = batch;
  p.heads = num_heads;
  p.heads_k = num_heads_k;
  p.group = num_heads / num_heads_k;
  p.splits = num_splits > 0 ? num_splits : attn_auto_splits(batch, num_heads_k, seqlen_k,
                                                                 k->layout != ZS_LAYOUT_TOKEN_MAJOR);
  p.splits = std::max(1, std::min(p.splits, std::max(1, (seqlen_k + 15) / 16)));
  p.chunk = attn_chunk(std::max(seqlen_k, 1), p.splits);
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  if (k->layout == ZS_LAYOUT_TOKEN_MAJOR) {
    const size_t sk = staging_bytes(k->layout, k->rows, k->cols);
    const size_t sv = staging_bytes(v->layout, v->rows, v->cols);
    if (!workspace || workspace_bytes < sk + sv) return ZS_E_INVAL;
    uint16_t* kd = reinterpret_cast<uint16_t*>(workspace);
    uint16_t* vd = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(workspace) + sk);
    const zs_kv_compressed_t* src[2] = {k, v};
    uint16_t* dst[2] = {kd, vd};
    for (int i = 0; i < 2; ++i) {
      const zs_kv_compressed_t* c = src[i];
      const int e = zs_bf16_triple_bitmap_decompress(
          stream, c->sign_mantissa, c->compressed_full, c->bitmap1, c->bitmap2, c->bitmap3,
          c->tile_offsets_median, c->tile_offsets_global, c->max_high_freq_count,
          c->max_full_count, (uint8_t)c->start_exp, dst[i], c->rows, c->cols);
      if (e != ZS_OK) return e;
    }
    return attn_staged((hipStream_t)stream, p, kd, vd, k->head_stride_rows,
                       reinterpret_cast<uint8_t*>(workspace) + sk + sv,
                       workspace_bytes - sk - sv);
  }
  return attn_launch<kModeCanon>((hipStream_t)stream, p, workspace, workspace_bytes);
}

extern "C" int zs_decode_attention_retiled(void* stream, const uint16_t* q,
                                           const zs_kv_retiled_t* k, const zs_kv_retiled_t* v,
                                           const int32_t* cache_seqlens, int seqlen_k,
                                           int batch, int num_heads, int num_heads_k,
                                           int head_dim, float softmax_scale, uint16_t* out,
                                           float* softmax_lse, void* workspace,
                                           size_t workspace_bytes, int num_splits) {
  int stc = attn_common_checks(batch, num_heads, num_heads_k, head_dim, seqlen_k, num_splits, q,
                               out);
  if (stc != ZS_OK) return stc;
  if (!k || !v) return ZS_E_INVAL;
  const zs_kv_retiled_t* kv[2] = {k, v};
  for (const zs_kv_retiled_t* c : kv) {
    if (!c->fixed || !c->exps || !c->eoff) return ZS_E_INVAL;
    if ((reinterpret_cast<uintptr_t>(c->fixed) & 15) || (reinterpret_cast<uintptr_t>(c->exps) & 15))
      return ZS_E_INVAL;
    const int g = kv_geometry_ok(c->layout, c->rows, c->cols, c->batch_stride_rows,
                                 c->head_stride_rows, c->start_exp, batch, num_heads_k, seqlen_k);
    if (g != ZS_OK) return g;
  }
  if (k->layout != v->layout || k->head_stride_rows != v->head_stride_rows)
    return ZS_E_UNSUPPORTED;
  AttnParams p{};
  p.kfix = k->fixed;
  p.kexp = k->exps;
  p.keo = k->eoff;
  p.vfix = v->fixed;
  p.vexp = v->exps;
  p.veo = v->eoff;
  p.k_nrec = k->rows / 16 * (k->cols / 64);
  p.v_nrec = v->rows / 16 * (v->cols / 64);
  p.k_start = k->start_exp;
  p.v_start = v->start_exp;
  p.k_bsr = k->batch_stride_rows;
  p.k_hsr = k->head_stride_rows;
  p.v_bsr = v->batch_stride_rows;
  p.v_hsr = v->head_stride_rows;
  p.q = q;
  p.out = out;
  p.lse = softmax_lse;
  p.seqlens = cache_seqlens;
  p.seqlen_k = seqlen_k;
  p.batch = batch;
  p.heads = num_heads;
  p.heads_k = num_heads_k;
  p.group = num_heads / num_heads_k;
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  if (k->layout == ZS_LAYOUT_TOKEN_MAJOR && tm_fused(num_heads_k, k->cols)) {
    p.splits = tm_splits(batch, seqlen_k, num_splits);
    p.chunk = tm_chunk(seqlen_k, p.splits);
    return attn_tm_launch((hipStream_t)stream, p, workspace, workspace_bytes);
  }
  p.splits = num_splits > 0 ? num_splits : attn_auto_splits(batch, num_heads_k, seqlen_k,
                                                                 k->layout != ZS_LAYOUT_TOKEN_MAJOR);
  p.splits = std::max(1, std::min(p.splits, std::max(1, (seqlen_k + 15) / 16)));
  p.chunk = attn_chunk(std::max(seqlen_k, 1), p.splits);
  if (k->layout == ZS_LAYOUT_TOKEN_MAJOR) {
    const size_t sk = staging_bytes(k->layout, k->rows, k->cols);
    const size_t sv = staging_bytes(v->layout, v->rows, v->cols);
    if (!workspace || workspace_bytes < sk + sv) return ZS_E_INVAL;
    uint16_t* kd = reinterpret_cast<uint16_t*>(workspace);
    uint16_t* vd = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(workspace) + sk);
    const zs_kv_retiled_t* src[2] = {k, v};
    uint16_t* dst[2] = {kd, vd};
    for (int i = 0; i < 2; ++i) {
      const int e = zs_retiled_decompress(stream, src[i]->fixed, src[i]->exps, src[i]->eoff,
                                          (uint8_t)src[i]->start_exp, dst[i], src[i]->rows,
                                          src[i]->cols);
      if (e != ZS_OK) return e;
    }
    return attn_staged((hipStream_t)stream, p, kd, vd, k->head_stride_rows,
                       reinterpret_cast<uint8_t*>(workspace) + sk + sv,
                       workspace_bytes - sk - sv);
  }
  return attn_launch<kModeRetiled>((hipStream_t)stream, p, workspace, workspace_bytes);
}

extern "C" int zs_decode_attention_dense(void* stream, const uint16_t* q, const uint16_t* k_cache,
                                         const uint16_t* v_cache, const int32_t* cache_seqlens,
                                         int seqlen_k, int cache_capacity, int batch,
                                         int num_heads, int num_heads_k, int head_dim,
                                         float softmax_scale, uint16_t* out, float* softmax_lse,
                                         void* workspace, size_t workspace_bytes,
                                         int num_splits) {
  int stc = attn_common_checks(batch, num_heads, num_heads_k, head_dim, seqlen_k, num_splits, q,
                               out);
  if (stc != ZS_OK) return stc;
  if (!k_cache || !v_cache || cache_capacity < seqlen_k) return ZS_E_INVAL;
  AttnParams p{};
  p.kd = k_cache;
  p.vd = v_cache;
  p.cap = cache_capacity;
  p.q = q;
  p.out = out;
  p.lse = softmax_lse;
  p.seqlens = cache_seqlens;
  p.seqlen_k = seqlen_k;
  p.batch = batch;
  p.heads = num_heads;
  p.heads_k = num_heads_k;
  p.group = num_heads / num_heads_k;
  p.splits = num_splits > 0 ? num_splits : attn_auto_splits(batch, num_heads_k, seqlen_k, false);
  p.splits = std::max(1, std::min(p.splits, std::max(1, (seqlen_k + 15) / 16)));
  p.chunk = attn_chunk(std::max(seqlen_k, 1), p.splits);
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  return attn_launch<kModeDense>((hipStream_t)stream, p, workspace, workspace_bytes);
}

extern "C" int zs_decode_attention_dense_paged(
    void* stream, const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
    const int32_t* block_table, int max_blocks_per_seq, int num_blocks, int page_block_size,
    const int32_t* cache_seqlens, int seqlen_k, int batch, int num_heads, int num_heads_k,
    int head_dim, float softmax_scale, uint16_t* out, float* softmax_lse, void* workspace,
    size_t workspace_bytes, int num_splits) {
  int stc = attn_common_checks(batch, num_heads, num_heads_k, head_dim, seqlen_k, num_splits, q,
                               out);
  if (stc != ZS_OK) return stc;
  if (!k_cache || !v_cache || !block_table || num_blocks <= 0 || max_blocks_per_seq <= 0)
    return ZS_E_INVAL;
  if (page_block_size <= 0 || (page_block_size % 16)) return ZS_E_UNSUPPORTED;
  if ((int64_t)max_blocks_per_seq * page_block_size < seqlen_k) return ZS_E_INVAL;
  if ((int64_t)num_blocks * page_block_size > INT32_MAX) return ZS_E_OVERFLOW;
  AttnParams p{};
  p.kd = k_cache;
  p.vd = v_cache;
  p.block_table = block_table;
  p.bt_stride = max_blocks_per_seq;
  p.page = page_block_size;
  p.q = q;
  p.out = out;
  p.lse = softmax_lse;
  p.seqlens = cache_seqlens;
  p.seqlen_k = seqlen_k;
  p.batch = batch;
  p.heads = num_heads;
  p.heads_k = num_heads_k;
  p.group = num_heads / num_heads_k;
  p.splits = num_splits > 0 ? num_splits : attn_auto_splits(batch, num_heads_k, seqlen_k, false);
  p.splits = std::max(1, std::min(p.splits, std::max(1, (seqlen_k + 15) / 16)));
  p.chunk = attn_chunk(std::max(seqlen_k, 1), p.splits);
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
  return attn_launch<kModePaged>((hipStream_t)stream, p, workspace, workspace_bytes);
}
