// zs_encode.hip -- gfx950 TCA-TBE encoder (the KV-cache compressor path).
//
//   analyze:  hist_kernel (per-lane LDS 256-bin histograms, grid-stride 16-byte loads)
//             -> select_kernel (window choice with the semantics of
//             kernel_benchmark/zipserv_decode_attention_ext.cu:65-134).
//   encode:   classify_kernel (bitmaps, small/median tile counts, per-GT
//             padded totals) -> cscan_* (global offsets, max, totals)
//             -> emit_kernel (re-reads the input, packs SM / FULL of a global
//             tile in LDS and writes them with 16-byte stores at the tile's
//             16-byte-aligned global offset).
// A wave handles one median tile; lane l handles small-tile row l of each
// half median tile (matrix row l%16, columns 8*(l/16)..+7), so the bitmap
// bytes it produces land at byte l of a 64-byte run and its SM offset is a
// wave prefix sum -- the mirror image of the decoder.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/zipserv.h"
#include "zs_device.hpp"
#include "zs_window.hpp"

namespace zs {

__global__ void fill_i32_kernel(int32_t* p, int n, int32_t v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// 256-bin exponent histogram.  Weights concentrate in a few exponents, so
// shared bins serialise on conflicting LDS atomics; each lane of a wave owns
// a copy of the bins (a copy per lane id, shared by the workgroup's waves),
// and copies sit kHistPitch = 257 dwords apart so that 64 lanes adding to
// one bin hit 64 different banks.  A workgroup's own bins stay below 2^31
// (the launch gives each at most 2^30 elements); the global bins are int32
// (the reference's) or 64-bit (any numel).
constexpr int kHistThreads = 512, kHistCopies = 64, kHistPitch = 257;

__device__ __forceinline__ void hist_add8(uint32_t* hc, uint4 x) {
  const uint32_t d[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    atomicAdd(&hc[(d[j] >> 7) & 0xFF], 1u);
    atomicAdd(&hc[(d[j] >> 23) & 0xFF], 1u);
  }
}

__device__ __forceinline__ uint4 nt_load16(const uint4* p) {
  const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(x.x, x.y, x.z, x.w);
}

template <typename C>
__global__ __launch_bounds__(kHistThreads) void hist_kernel(const uint16_t* in, int64_t n,
                                                            C* counts) {
  __shared__ uint32_t h[kHistCopies * kHistPitch];
  for (int i = threadIdx.x; i < kHistCopies * kHistPitch; i += kHistThreads) h[i] = 0;
  __syncthreads();
  uint32_t* hc = h + lane_id() * kHistPitch;
  const int64_t tid = (int64_t)blockIdx.x * kHistThreads + threadIdx.x;
  const int64_t nthreads = (int64_t)gridDim.x * kHistThreads;
  const bool aligned = (reinterpret_cast<uintptr_t>(in) & 15) == 0;
  const int64_t nvec = aligned ? n / 8 : 0;
  const uint4* v = reinterpret_cast<const uint4*>(in);
  int64_t i = tid;
  for (; i + 3 * nthreads < nvec; i += 4 * nthreads) {  // four 16-byte loads in flight
    // streamed once: non-temporal loads keep the caches for other data
    const uint4 x0 = nt_load16(v + i), x1 = nt_load16(v + i + nthreads),
                x2 = nt_load16(v + i + 2 * nthreads), x3 = nt_load16(v + i + 3 * nthreads);
    hist_add8(hc, x0);
    hist_add8(hc, x1);
    hist_add8(hc, x2);
    hist_add8(hc, x3);
  }
  for (; i < nvec; i += nthreads) hist_add8(hc, v[i]);
  for (int64_t e = nvec * 8 + tid; e < n; e += nthreads) atomicAdd(&hc[(in[e] >> 7) & 0xFF], 1u);
  __syncthreads();
  if (threadIdx.x < 256) {
    uint32_t c = 0;
    for (int k = 0; k < kHistCopies; ++k) c += h[k * kHistPitch + threadIdx.x];
    if (c) {
      if constexpr (sizeof(C) == 8)
        atomicAdd(reinterpret_cast<unsigned long long*>(&counts[threadIdx.x]),
                  (unsigned long long)c);
      else
        atomicAdd(&counts[threadIdx.x], (C)c);
    }
  }
}

// Histogram of a sample of the input -- every stride-th 4096-byte chunk,
// stride >= 32 and at most kSampleChunks chunks -- for the window guess of
// the one-pass re-tiled encoder.  kSampleGroups workgroups each write their
// own 256 bins (slice blockIdx.x of `slices`, no atomics, so nothing needs
// zeroing first) and clear `zero` (the fused encoding pass's kVerifySlices
// histogram slices, added to with atomics later) and *zero32 (when given:
// the arrival counter of the offset scan).
constexpr int kSampleStrideMin = 32, kSampleChunks = 128, kSampleGroups = 4;

__device__ __forceinline__ int64_t sample_stride(int64_t nchunks) {
  const int64_t s = (nchunks + kSampleChunks - 1) / kSampleChunks;
  return s > kSampleStrideMin ? s : kSampleStrideMin;
}

__global__ __launch_bounds__(kHistThreads) void sample_hist_kernel(const uint16_t* in,
                                                                   int64_t nchunks,
                                                                   uint64_t* slices,
                                                                   uint64_t* zero,
                                                                   int32_t* zero32) {
  __shared__ uint32_t h[kHistCopies * kHistPitch];
  for (int i = threadIdx.x; i < kHistCopies * kHistPitch; i += kHistThreads) h[i] = 0;
  for (int i = blockIdx.x * kHistThreads + threadIdx.x; i < kVerifySlices * 256;
       i += kSampleGroups * kHistThreads)
    zero[i] = 0;
  if (zero32 && blockIdx.x == 0 && threadIdx.x == 0) *zero32 = 0;
  __syncthreads();
  uint32_t* hc = h + lane_id() * kHistPitch;
  const uint4* v = reinterpret_cast<const uint4*>(in);
  const int64_t stride = sample_stride(nchunks);
  const int64_t nvec = (nchunks + stride - 1) / stride * 256;
  const int64_t nthreads = (int64_t)gridDim.x * kHistThreads;
  auto at = [&](int64_t i) { return v + (i >> 8) * (256 * stride) + (i & 255); };
  int64_t i = (int64_t)blockIdx.x * kHistThreads + threadIdx.x;
  for (; i + 7 * nthreads < nvec; i += 8 * nthreads) {  // eight 16-byte loads in flight
    uint4 x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = nt_load16(at(i + j * nthreads));
#pragma unroll
    for (int j = 0; j < 8; ++j) hist_add8(hc, x[j]);
  }
  for (; i < nvec; i += nthreads) hist_add8(hc, nt_load16(at(i)));
  __syncthreads();
  if (threadIdx.x < 256) {
    uint32_t c = 0;
    for (int k = 0; k < kHistCopies; ++k) c += h[k * kHistPitch + threadIdx.x];
    slices[256 * blockIdx.x + threadIdx.x] = c;
  }
}

// Count of exponent e: the sum of nslices histograms 256 bins apart; written
// back to sum_out (when given) as the one histogram.
template <int NS, typename C>
__device__ __forceinline__ int64_t load_count(const C* counts_g, int e, uint64_t* sum_out) {
  int64_t c = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) c += (int64_t)counts_g[256 * s + e];
  if (sum_out) sum_out[e] = (uint64_t)c;
  return c;
}

// The window rules (zs_window.hpp) as one-workgroup kernels over NS
// histogram slices: thread t sums bin t, then one wave selects.
template <typename C, int NS = 1>
__global__ __launch_bounds__(256) void select_kernel(const C* counts_g,
                                                    uint64_t* sum_out, int32_t* top,
                                                    const int32_t* guess, int32_t* differs) {
  if (blockIdx.x != 0) return;
  __shared__ int64_t counts[256];
  counts[threadIdx.x] = load_count<NS>(counts_g, threadIdx.x, sum_out);
  __syncthreads();
  if (threadIdx.x < 64) select_kv_wave(counts, threadIdx.x, top, guess, differs);
}

template <typename C, int NS = 1>
__global__ __launch_bounds__(256) void select_weights_kernel(const C* counts_g,
                                                            uint64_t* sum_out, int32_t* top,
                                                            const int32_t* guess,
                                                            int32_t* differs) {
  if (blockIdx.x != 0) return;
  __shared__ int64_t counts[256];
  counts[threadIdx.x] = load_count<NS>(counts_g, threadIdx.x, sum_out);
  __syncthreads();
  if (threadIdx.x < 64) select_weights_wave(counts, threadIdx.x, top, guess, differs);
}


// Exponent -> code LUT in LDS (code 0 = outlier), as s_exp_lut of
// csrc/L_API.cu:1149-1156.
__device__ __forceinline__ void build_code_lut(uint8_t* lut, const int32_t* top) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x) lut[i] = 0;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 0; i < 7; ++i) {
      const int e = top[i];
      if (e >= 0 && e <= 255) lut[e] = (uint8_t)(i + 1);
    }
  }
  __syncthreads();
}

struct RowCode {
  uint4 raw;      // the 8 bf16 of the row
  uint32_t b1, b2, b3, ind;
};

__device__ __forceinline__ RowCode classify_row(const uint16_t* src, const uint8_t* lut) {
  RowCode r;
  r.raw = *reinterpret_cast<const uint4*>(src);
  const uint32_t d[4] = {r.raw.x, r.raw.y, r.raw.z, r.raw.w};
  uint32_t b1 = 0, b2 = 0, b3 = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t bits = (d[j >> 1] >> ((j & 1) * 16)) & 0xFFFF;
    const uint32_t c = lut[(bits >> 7) & 0xFF];
    b1 |= (c & 1u) << j;
    b2 |= ((c >> 1) & 1u) << j;
    b3 |= ((c >> 2) & 1u) << j;
  }
  r.b1 = b1;
  r.b2 = b2;
  r.b3 = b3;
  r.ind = b1 | b2 | b3;
  return r;
}

__global__ __launch_bounds__(256) void classify_kernel(const uint16_t* in, int M, int K,
                                                       const int32_t* top, uint8_t* bm1,
                                                       uint8_t* bm2, uint8_t* bm3,
                                                       int32_t* tiles, int32_t* tom,
                                                       int32_t* gt_hf, int32_t* gt_full) {
  __shared__ uint8_t lut[256];
  __shared__ int32_t med_hf[4];
  build_code_lut(lut, top);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  const int KT = K >> 6;
  const int64_t ngt = (int64_t)(M >> 6) * KT;
  for (int64_t g = blockIdx.x; g < ngt; g += gridDim.x) {
    const int64_t gm = g / KT, gk = g % KT;
    int hf_m = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t row = gm * 64 + w * 16 + (l & 15);
      const int64_t col = gk * 64 + h * 32 + 8 * (l >> 4);
      const RowCode rc = classify_row(in + row * K + col, lut);
      const int64_t bidx = 512 * g + 128 * w + 64 * h + l;
      bm1[bidx] = (uint8_t)rc.b1;
      bm2[bidx] = (uint8_t)rc.b2;
      bm3[bidx] = (uint8_t)rc.b3;
      int n = __builtin_popcount(rc.ind);
      int t = n;
      t += __shfl_xor(t, 1);
      t += __shfl_xor(t, 2);
      t += __shfl_xor(t, 4);
      if ((l & 7) == 0) {
        const int64_t tile = 64 * g + 16 * w + 8 * h + (l >> 3);
        tiles[2 * tile] = t;
        tiles[2 * tile + 1] = 64 - t;
      }
      hf_m += __builtin_amdgcn_readlane(wave_inclusive_scan(n), 63);
    }
    if (l == 0) med_hf[w] = hf_m;
    __syncthreads();
    if (threadIdx.x < 4) {
      int before = 0;
      for (int i = 0; i < (int)threadIdx.x; ++i) before += med_hf[i];
      tom[2 * (4 * g + threadIdx.x)] = before;
      tom[2 * (4 * g + threadIdx.x) + 1] = 1024 * threadIdx.x - before;
    }
    if (threadIdx.x == 0) {
      const int hf = med_hf[0] + med_hf[1] + med_hf[2] + med_hf[3];
      const int fu = 4096 - hf;
      gt_hf[g] = (hf + 15) & ~15;
      gt_full[g] = (fu + 7) & ~7;
    }
    __syncthreads();
  }
}

// Offsets of the global tiles' padded SM / FULL sizes, in three coalesced
// passes over spans of kSpan global tiles: per-span sums and maxima, one
// workgroup scanning the span sums, then per-span exclusive offsets.  Output
// slot i (i < ngt) is the exclusive offset of global tile i and slot ngt the
// total, in hf_off / full_off and interleaved in tog (the tile_offsets_global
// array of csrc/L_API.cu).  A span's sums and maxima are parked in its first
// output slots between the passes.
constexpr int kSpan = 1024;

struct Pair {
  int a, b;
};

__device__ __forceinline__ Pair block256_exclusive2(Pair v, Pair& total) {
  __shared__ int ws[2][4];
  const int l = lane_id(), w = threadIdx.x >> 6;
  const int ia = wave_inclusive_scan(v.a), ib = wave_inclusive_scan(v.b);
  if (l == 63) {
    ws[0][w] = ia;
    ws[1][w] = ib;
  }
  __syncthreads();
  Pair before = {0, 0};
  for (int i = 0; i < w; ++i) {
    before.a += ws[0][i];
    before.b += ws[1][i];
  }
  total = {ws[0][0] + ws[0][1] + ws[0][2] + ws[0][3], ws[1][0] + ws[1][1] + ws[1][2] + ws[1][3]};
  __syncthreads();
  return {before.a + ia - v.a, before.b + ib - v.b};
}

__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off));
  return v;
}

__global__ __launch_bounds__(256) void cscan_reduce_kernel(const int32_t* gt_hf,
                                                           const int32_t* gt_full, int64_t ngt,
                                                           int32_t* tog, int32_t* hf_off,
                                                           int32_t* full_off) {
  __shared__ int wm[2][4];
  const int64_t base = (int64_t)blockIdx.x * kSpan;
  Pair s = {0, 0};
  int mh = 0, mf = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t i = base + j * 256 + threadIdx.x;
    if (i < ngt) {
      const int h = gt_hf[i], f = gt_full[i];
      s.a += h;
      s.b += f;
      mh = max(mh, h);
      mf = max(mf, f);
    }
  }
  mh = wave_max(mh);
  mf = wave_max(mf);
  if (lane_id() == 0) {
    wm[0][threadIdx.x >> 6] = mh;
    wm[1][threadIdx.x >> 6] = mf;
  }
  Pair total;
  block256_exclusive2(s, total);  // its barrier also publishes wm
  if (threadIdx.x == 0) {
    hf_off[base] = total.a;
    full_off[base] = total.b;
    tog[2 * base] = max(max(wm[0][0], wm[0][1]), max(wm[0][2], wm[0][3]));
    tog[2 * base + 1] = max(max(wm[1][0], wm[1][1]), max(wm[1][2], wm[1][3]));
  }
}

__global__ __launch_bounds__(1024) void cscan_spans_kernel(int64_t ngt, int32_t* tog,
                                                           int32_t* hf_off, int32_t* full_off,
                                                           int32_t* max_hf, int32_t* max_full,
                                                           int32_t* tot_hf, int32_t* tot_full) {
  __shared__ int64_t wsum[2][16];
  __shared__ int32_t wmax[2][16];
  __shared__ int64_t carry[2];
  __shared__ int32_t mx[2];
  const int t = threadIdx.x, l = lane_id(), w = t >> 6;
  const int64_t nspans = (ngt + kSpan - 1) / kSpan;
  if (t == 0) carry[0] = carry[1] = mx[0] = mx[1] = 0;
  __syncthreads();
  for (int64_t s0 = 0; s0 < nspans; s0 += 1024) {
    const int64_t sp = s0 + t;
    const bool in = sp < nspans;
    const int64_t at = sp * kSpan;
    const int va = in ? hf_off[at] : 0, vb = in ? full_off[at] : 0;
    const int ma = wave_max(in ? tog[2 * at] : 0), mb = wave_max(in ? tog[2 * at + 1] : 0);
    const int ia = wave_inclusive_scan(va), ib = wave_inclusive_scan(vb);
    if (l == 63) {
      wsum[0][w] = ia;
      wsum[1][w] = ib;
    }
    if (l == 0) {
      wmax[0][w] = ma;
      wmax[1][w] = mb;
    }
    __syncthreads();
    int64_t ba = carry[0], bb = carry[1];
    for (int i = 0; i < w; ++i) {
      ba += wsum[0][i];
      bb += wsum[1][i];
    }
    if (in) {
      hf_off[at] = (int32_t)(ba + ia - va);
      full_off[at] = (int32_t)(bb + ib - vb);
    }
    __syncthreads();
    if (t == 0) {
      for (int i = 0; i < 16; ++i) {
        carry[0] += wsum[0][i];
        carry[1] += wsum[1][i];
        mx[0] = max(mx[0], wmax[0][i]);
        mx[1] = max(mx[1], wmax[1][i]);
      }
    }
    __syncthreads();
  }
  if (t == 0) {
    const int32_t th = (int32_t)carry[0], tf = (int32_t)carry[1];
    hf_off[ngt] = th;
    full_off[ngt] = tf;
    tog[2 * ngt] = th;
    tog[2 * ngt + 1] = tf;
    *tot_hf = th;
    *tot_full = tf;
    *max_hf = mx[0];
    *max_full = mx[1];
  }
}

__global__ __launch_bounds__(256) void cscan_write_kernel(const int32_t* gt_hf,
                                                          const int32_t* gt_full, int64_t ngt,
                                                          int32_t* tog, int32_t* hf_off,
                                                          int32_t* full_off) {
  const int64_t base = (int64_t)blockIdx.x * kSpan;
  const Pair off = {hf_off[base], full_off[base]};  // rewritten unchanged below
  const int64_t i0 = base + 4 * threadIdx.x;
  int ch[4], cf[4];
  Pair s = {0, 0};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool in = i0 + j < ngt;
    ch[j] = in ? gt_hf[i0 + j] : 0;
    cf[j] = in ? gt_full[i0 + j] : 0;
    s.a += ch[j];
    s.b += cf[j];
  }
  Pair total;
  const Pair ex = block256_exclusive2(s, total);
  int rh = off.a + ex.a, rf = off.b + ex.b;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (i0 + j < ngt) {
      hf_off[i0 + j] = rh;
      full_off[i0 + j] = rf;
      tog[2 * (i0 + j)] = rh;
      tog[2 * (i0 + j) + 1] = rf;
    }
    rh += ch[j];
    rf += cf[j];
  }
}

__global__ __launch_bounds__(256) void emit_kernel(const uint16_t* in, int M, int K,
                                                   const int32_t* top, const int32_t* tog,
                                                   const int32_t* tom, uint8_t* sm_out,
                                                   uint16_t* full_out) {
  __shared__ uint8_t lut[256];
  __shared__ uint4 sm_stage[4096 / 16];
  __shared__ uint4 full_stage[4096 * 2 / 16];
  build_code_lut(lut, top);
  uint8_t* smb = reinterpret_cast<uint8_t*>(sm_stage);
  uint16_t* fub = reinterpret_cast<uint16_t*>(full_stage);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id();
  const int KT = K >> 6;
  const int64_t ngt = (int64_t)(M >> 6) * KT;
  for (int64_t g = blockIdx.x; g < ngt; g += gridDim.x) {
    const int64_t gm = g / KT, gk = g % KT;
    for (int i = threadIdx.x; i < 4096 / 16; i += blockDim.x) sm_stage[i] = make_uint4(0, 0, 0, 0);
    for (int i = threadIdx.x; i < 4096 * 2 / 16; i += blockDim.x)
      full_stage[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();
    int sm_base = tom[2 * (4 * g + w)];
    int fu_base = tom[2 * (4 * g + w) + 1];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t row = gm * 64 + w * 16 + (l & 15);
      const int64_t col = gk * 64 + h * 32 + 8 * (l >> 4);
      const RowCode rc = classify_row(in + row * K + col, lut);
      const int n = __builtin_popcount(rc.ind);
      const int incl = wave_inclusive_scan(n);
      const int excl = incl - n;
      const int tot = __builtin_amdgcn_readlane(incl, 63);
      int so = sm_base + excl;
      int fo = fu_base + 8 * l - excl;
      const uint32_t d[4] = {rc.raw.x, rc.raw.y, rc.raw.z, rc.raw.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t bits = (d[j >> 1] >> ((j & 1) * 16)) & 0xFFFF;
        if ((rc.ind >> j) & 1) {
          smb[so++] = (uint8_t)(((bits >> 8) & 0x80) | (bits & 0x7F));
        } else {
          fub[fo++] = (uint16_t)bits;
        }
      }
      sm_base += tot;
      fu_base += 512 - tot;
    }
    __syncthreads();
    const int64_t so = tog[2 * g], fo = tog[2 * g + 1];
    const int sm_len = (int)(tog[2 * (g + 1)] - so);      // padded, multiple of 16
    const int fu_len = (int)(tog[2 * (g + 1) + 1] - fo);  // padded, multiple of 8
    uint4* smd = reinterpret_cast<uint4*>(sm_out + so);
    uint4* fud = reinterpret_cast<uint4*>(full_out + fo);
    for (int i = threadIdx.x; i < sm_len / 16; i += blockDim.x) smd[i] = sm_stage[i];
    for (int i = threadIdx.x; i < fu_len / 8; i += blockDim.x) fud[i] = full_stage[i];
    __syncthreads();
  }
}

extern int device_cu_count();

}  // namespace zs

using namespace zs;

static int hip_status(hipError_t e) { return e == hipSuccess ? ZS_OK : (int)e; }

template <typename C>
static int analyze(hipStream_t st, const uint16_t* d_input, int64_t numel, C* d_counts,
                   int32_t* d_top, bool weights_rule = false) {
  // Two 512-thread workgroups per CU (their bins fill 2 x 64 KB of LDS),
  // and at most 2^30 elements each.
  const int64_t blocks = std::max<int64_t>(
      std::min<int64_t>((numel + 8 * kHistThreads - 1) / (8 * kHistThreads),
                        (int64_t)device_cu_count() * 2),
      (numel + (1LL << 30) - 1) >> 30);
  if (blocks > INT32_MAX) return ZS_E_OVERFLOW;
  hipLaunchKernelGGL(fill_i32_kernel, dim3(sizeof(C) / 4), dim3(256), 0, st,
                     reinterpret_cast<int32_t*>(d_counts), (int)(256 * sizeof(C) / 4), 0);
  hipLaunchKernelGGL(hist_kernel<C>, dim3((unsigned)blocks), dim3(kHistThreads), 0, st, d_input, numel,
                     d_counts);
  if (weights_rule)
    hipLaunchKernelGGL(select_weights_kernel<C>, dim3(1), dim3(256), 0, st, d_counts, nullptr, d_top,
                       nullptr, nullptr);
  else
    hipLaunchKernelGGL(select_kernel<C>, dim3(1), dim3(256), 0, st, d_counts, nullptr, d_top,
                       nullptr, nullptr);
  return hip_status(hipGetLastError());
}

namespace zs {

// Window guess from a sample of the input (chunks of 2048 elements, at most
// kSampleChunks of them; a partial last chunk, when numel is not a multiple
// of 2048, is not sampled; input 16-byte aligned) into `guess`; the per-workgroup
// sample bins go to `sample` (kSampleGroups x 256), and `zero`
// (kVerifySlices x 256 entries) and *zero32 (when given) are cleared on the way.
hipError_t launch_window_sample(hipStream_t st, const uint16_t* in, int64_t numel,
                                bool weights_rule, uint64_t* sample, uint64_t* zero,
                                int32_t* guess, int32_t* zero32) {
  hipLaunchKernelGGL(sample_hist_kernel, dim3(kSampleGroups), dim3(kHistThreads), 0, st, in,
                     numel / 2048, sample, zero, zero32);
  if (weights_rule)
    hipLaunchKernelGGL((select_weights_kernel<uint64_t, kSampleGroups>), dim3(1), dim3(256), 0, st,
                       sample, nullptr, guess, nullptr, nullptr);
  else
    hipLaunchKernelGGL((select_kernel<uint64_t, kSampleGroups>), dim3(1), dim3(256), 0, st, sample,
                       nullptr, guess, nullptr, nullptr);
  return hipGetLastError();
}

}  // namespace zs

extern "C" int zs_analyze_top_exponents_gpu(void* stream, const uint16_t* d_input, int64_t numel,
                                            int32_t* d_counts, int32_t* d_top,
                                            int32_t* d_done) {
  if (!d_input || numel <= 0 || !d_counts || !d_top) return ZS_E_INVAL;
  if (numel > INT32_MAX) return ZS_E_OVERFLOW;  // int32 bins of the reference
  hipStream_t st = (hipStream_t)stream;
  if (d_done) hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(256), 0, st, d_done, 1, 0);
  return analyze(st, d_input, numel, d_counts, d_top);
}

extern "C" int zs_analyze_top_exponents_u64_gpu(void* stream, const uint16_t* d_input,
                                                int64_t numel, uint64_t* d_counts,
                                                int32_t* d_top) {
  if (!d_input || numel <= 0 || !d_counts || !d_top) return ZS_E_INVAL;
  return analyze((hipStream_t)stream, d_input, numel, d_counts, d_top);
}

extern "C" int zs_analyze_exponents_weights_gpu(void* stream, const uint16_t* d_input,
                                                 int64_t numel, uint64_t* d_counts,
                                                 int32_t* d_top) {
  if (!d_input || numel <= 0 || !d_counts || !d_top) return ZS_E_INVAL;
  return analyze((hipStream_t)stream, d_input, numel, d_counts, d_top, true);
}

extern "C" int zs_init_bf16_matrix_triple_bitmap_gpu(
    void* stream, const uint16_t* d_input, int M, int K, const int32_t* d_top,
    uint8_t* d_sm, uint16_t* d_full, uint64_t* d_b1, uint64_t* d_b2, uint64_t* d_b3,
    int32_t* d_tiles, int32_t* d_tom, int32_t* d_tog, uint8_t* d_temp_sm, uint16_t* d_temp_full,
    int32_t* d_gt_hf, int32_t* d_gt_full, int32_t* d_hf_off, int32_t* d_full_off,
    int32_t* d_max_hf, int32_t* d_max_full, int32_t* d_tot_hf, int32_t* d_tot_full) {
  (void)d_temp_sm;
  (void)d_temp_full;
  if (M <= 0 || K <= 0 || (M % 64) || (K % 64)) return ZS_E_INVAL;
  const int64_t mk = (int64_t)M * K, ngt = mk / 4096;
  if (mk + 16 * ngt > INT32_MAX) return ZS_E_OVERFLOW;
  if (!d_input || !d_top || !d_sm || !d_full || !d_b1 || !d_b2 || !d_b3 || !d_tiles || !d_tom ||
      !d_tog || !d_gt_hf || !d_gt_full || !d_hf_off || !d_full_off || !d_max_hf ||
      !d_max_full || !d_tot_hf || !d_tot_full)
    return ZS_E_INVAL;
  if ((reinterpret_cast<uintptr_t>(d_input) | reinterpret_cast<uintptr_t>(d_sm) |
       reinterpret_cast<uintptr_t>(d_full)) & 15)
    return ZS_E_INVAL;  // 16-byte rows in, 16-byte tile streams out
  hipStream_t st = (hipStream_t)stream;
  const unsigned grid = (unsigned)std::min<int64_t>(ngt, (int64_t)device_cu_count() * 8);
  hipLaunchKernelGGL(classify_kernel, dim3(grid), dim3(256), 0, st, d_input, M, K, d_top,
                     reinterpret_cast<uint8_t*>(d_b1), reinterpret_cast<uint8_t*>(d_b2),
                     reinterpret_cast<uint8_t*>(d_b3), d_tiles, d_tom, d_gt_hf, d_gt_full);
  const unsigned spans = (unsigned)((ngt + kSpan - 1) / kSpan);
  hipLaunchKernelGGL(cscan_reduce_kernel, dim3(spans), dim3(256), 0, st, d_gt_hf, d_gt_full, ngt,
                     d_tog, d_hf_off, d_full_off);
  hipLaunchKernelGGL(cscan_spans_kernel, dim3(1), dim3(1024), 0, st, ngt, d_tog, d_hf_off,
                     d_full_off, d_max_hf, d_max_full, d_tot_hf, d_tot_full);
  hipLaunchKernelGGL(cscan_write_kernel, dim3(spans), dim3(256), 0, st, d_gt_hf, d_gt_full, ngt,
                     d_tog, d_hf_off, d_full_off);
  hipLaunchKernelGGL(emit_kernel, dim3(grid), dim3(256), 0, st, d_input, M, K, d_top, d_tog,
                     d_tom, d_sm, d_full);
  return hip_status(hipGetLastError());
}
