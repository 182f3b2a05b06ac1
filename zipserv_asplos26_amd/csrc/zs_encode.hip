// zs_encode.hip -- gfx950 TCA-TBE encoder (the KV-cache compressor path).
//
//   analyze:  hist_kernel (LDS 256-bin histogram, grid-stride 16-byte loads)
//             -> select_kernel (window choice with the semantics of
//             kernel_benchmark/zipserv_decode_attention_ext.cu:65-134).
//   encode:   classify_kernel (bitmaps, small/median tile counts, per-GT
//             padded totals) -> scan_kernel (global offsets, max, totals)
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

namespace zs {

__global__ void fill_i32_kernel(int32_t* p, int n, int32_t v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ __launch_bounds__(256) void hist_kernel(const uint16_t* in, int64_t n, int32_t* counts) {
  __shared__ int32_t h[256];
  h[threadIdx.x] = 0;
  __syncthreads();
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nthreads = (int64_t)gridDim.x * blockDim.x;
  const bool aligned = (reinterpret_cast<uintptr_t>(in) & 15) == 0;
  const int64_t nvec = aligned ? n / 8 : 0;
  const uint4* v = reinterpret_cast<const uint4*>(in);
  for (int64_t i = tid; i < nvec; i += nthreads) {
    const uint4 x = v[i];
    const uint32_t d[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      atomicAdd(&h[(d[j] >> 7) & 0xFF], 1);
      atomicAdd(&h[(d[j] >> 23) & 0xFF], 1);
    }
  }
  for (int64_t i = nvec * 8 + tid; i < n; i += nthreads) atomicAdd(&h[(in[i] >> 7) & 0xFF], 1);
  __syncthreads();
  const int32_t c = h[threadIdx.x];
  if (c) atomicAdd(&counts[threadIdx.x], c);
}

// Window selection of zipserv_decode_attention_ext.cu:65-134: seven slots
// start at count -1 (so zero counts can be taken); each exponent 0..255
// replaces the first minimum slot on strictly greater count; candidates are
// sorted, the first one starting 7 present exponents wins, else the start of
// the longest consecutive run, clamped to [0, 248].
__global__ void select_kernel(const int32_t* counts, int32_t* top) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int te[7], tc[7];
  for (int i = 0; i < 7; ++i) {
    te[i] = -1;
    tc[i] = -1;
  }
  for (int e = 0; e < 256; ++e) {
    int mi = 0;
    for (int i = 1; i < 7; ++i)
      if (tc[i] < tc[mi]) mi = i;
    if (counts[e] > tc[mi]) {
      tc[mi] = counts[e];
      te[mi] = e;
    }
  }
  int cand[7], n = 0;
  for (int i = 0; i < 7; ++i)
    if (te[i] >= 0) cand[n++] = te[i];
  for (; n < 7; ++n) cand[n] = 127 - n;
  for (int i = 1; i < 7; ++i) {
    const int key = cand[i];
    int j = i - 1;
    while (j >= 0 && cand[j] > key) {
      cand[j + 1] = cand[j];
      --j;
    }
    cand[j + 1] = key;
  }
  for (int c = 0; c < 7; ++c) {
    const int st = cand[c];
    if (st < 0 || st + 6 > 255) continue;
    bool all = true;
    for (int i = 0; i < 7 && all; ++i) all = counts[st + i] > 0;
    if (all) {
      for (int i = 0; i < 7; ++i) top[i] = st + i;
      return;
    }
  }
  int best = cand[0], best_len = 1, run = 1;
  for (int i = 1; i < 7; ++i) {
    run = (cand[i] == cand[i - 1] + 1) ? run + 1 : 1;
    if (run > best_len) {
      best_len = run;
      best = cand[i] - run + 1;
    }
  }
  best = best < 0 ? 0 : (best > 248 ? 248 : best);
  for (int i = 0; i < 7; ++i) top[i] = best + i;
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

// Single-workgroup scan over the per-tile padded counts: each of the 1024
// threads owns a contiguous chunk, chunk sums are scanned in LDS, then every
// thread writes its chunk's cumulative offsets.
__global__ __launch_bounds__(1024) void scan_kernel(const int32_t* gt_hf, const int32_t* gt_full,
                                                    int64_t ngt, int32_t* tog, int32_t* hf_off,
                                                    int32_t* full_off, int32_t* max_hf,
                                                    int32_t* max_full, int32_t* tot_hf,
                                                    int32_t* tot_full) {
  __shared__ int64_t s_hf[1024], s_fu[1024];
  __shared__ int32_t s_mh[1024], s_mf[1024];
  const int t = threadIdx.x;
  const int64_t chunk = (ngt + 1023) / 1024;
  const int64_t b = std::min<int64_t>(ngt, t * chunk), e = std::min<int64_t>(ngt, b + chunk);
  int64_t sh = 0, sf = 0;
  int32_t mh = 0, mf = 0;
  for (int64_t i = b; i < e; ++i) {
    sh += gt_hf[i];
    sf += gt_full[i];
    mh = max(mh, gt_hf[i]);
    mf = max(mf, gt_full[i]);
  }
  s_hf[t] = sh;
  s_fu[t] = sf;
  s_mh[t] = mh;
  s_mf[t] = mf;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    int64_t ah = 0, af = 0;
    if (t >= off) {
      ah = s_hf[t - off];
      af = s_fu[t - off];
    }
    __syncthreads();
    s_hf[t] += ah;
    s_fu[t] += af;
    __syncthreads();
  }
  for (int off = 512; off > 0; off >>= 1) {
    if (t < off) {
      s_mh[t] = max(s_mh[t], s_mh[t + off]);
      s_mf[t] = max(s_mf[t], s_mf[t + off]);
    }
    __syncthreads();
  }
  int64_t run_h = s_hf[t] - sh, run_f = s_fu[t] - sf;
  for (int64_t i = b; i < e; ++i) {
    run_h += gt_hf[i];
    run_f += gt_full[i];
    tog[2 * (i + 1)] = (int32_t)run_h;
    tog[2 * (i + 1) + 1] = (int32_t)run_f;
    hf_off[i + 1] = (int32_t)run_h;
    full_off[i + 1] = (int32_t)run_f;
  }
  if (t == 0) {
    tog[0] = 0;
    tog[1] = 0;
    hf_off[0] = 0;
    full_off[0] = 0;
    *max_hf = s_mh[0];
    *max_full = s_mf[0];
    *tot_hf = (int32_t)s_hf[1023];
    *tot_full = (int32_t)s_fu[1023];
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

extern "C" int zs_analyze_top_exponents_gpu(void* stream, const uint16_t* d_input, int64_t numel,
                                            int32_t* d_counts, int32_t* d_top,
                                            int32_t* d_done) {
  if (!d_input || numel <= 0 || !d_counts || !d_top) return ZS_E_INVAL;
  if (numel > INT32_MAX) return ZS_E_OVERFLOW;  // int32 bins of the reference
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(256), 0, st, d_counts, 256, 0);
  if (d_done) hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, st, d_done, 1, 0);
  const int64_t blocks = std::max<int64_t>(
      1, std::min<int64_t>((numel + 2047) / 2048, (int64_t)device_cu_count() * 4));
  hipLaunchKernelGGL(hist_kernel, dim3((unsigned)blocks), dim3(256), 0, st, d_input, numel,
                     d_counts);
  hipLaunchKernelGGL(select_kernel, dim3(1), dim3(64), 0, st, d_counts, d_top);
  return hip_status(hipGetLastError());
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
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), 0, st, d_gt_hf, d_gt_full, ngt, d_tog,
                     d_hf_off, d_full_off, d_max_hf, d_max_full, d_tot_hf, d_tot_full);
  hipLaunchKernelGGL(emit_kernel, dim3(grid), dim3(256), 0, st, d_input, M, K, d_top, d_tog,
                     d_tom, d_sm, d_full);
  return hip_status(hipGetLastError());
}
