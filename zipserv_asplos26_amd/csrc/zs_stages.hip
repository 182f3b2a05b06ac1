// zs_stages.hip -- stage profiler of the re-tiled record pipeline (gfx950).
//
// The counterpart of kernel_benchmark/zipserv_tile_stage_bench_ext.cu (one
// CTA timing the fused loader's load / decompress stages with clock64
// brackets).  Here one wave runs the steps of consuming one 16x64 record, as
// the ZipGEMM and decode-attention kernels do, with a shader-clock stamp
// (s_memtime, after waiting for every outstanding memory operation) between
// the steps:
//   0 bracket   two stamps back to back (subtracted from the others on the host)
//   1 offsets   eoff[r], eoff[r + 1]                 (global loads)
//   2 fixed     the record's 1408 fixed bytes        (global loads)
//   3 exps      its outlier bytes, one dword a lane  (global load)
//   4 stage     those dwords into LDS                (ds_write)
//   5 decode    tables, outlier scan, windows, bf16 assembly (VALU + LDS)
//   6 mfma      two v_mfma_f32_16x16x32_bf16 on the decoded operands
//   7 record    steps 1-6 back to back without stamps
// Iteration i uses record (record0 + i * stride) mod num_records, so with a
// large stride the loads miss the caches.  Per stage the kernel writes the
// mean cycles over `iters` measured iterations, then the total shader-clock
// cycles and the total s_memrealtime ticks (100 MHz) of the measured loop, so
// the host can convert cycles to time.
#include <hip/hip_runtime.h>

#include "../../include/zipserv.h"
#include "zs_rdecode.hpp"

namespace zs {

constexpr int kStages = 8;

__device__ __forceinline__ uint64_t stamp() {
  uint64_t t;
  asm volatile(
      "s_waitcnt vmcnt(0) lgkmcnt(0)\n\t"
      "s_memtime %0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=s"(t)
      :
      : "memory");
  return t;
}

__device__ __forceinline__ uint64_t realtime() {
  uint64_t t;
  asm volatile(
      "s_memrealtime %0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=s"(t)
      :
      : "memory");
  return t;
}

// Orders a value's computation before the next stamp.
__device__ __forceinline__ void keep(uint32_t v) { asm volatile("" ::"v"(v)); }
__device__ __forceinline__ void keep4(u32x4 v) {
  keep(v[0]);
  keep(v[1]);
  keep(v[2]);
  keep(v[3]);
}

__global__ __launch_bounds__(64) void rstage_kernel(const uint8_t* fixed, const uint8_t* exps,
                                                    const int32_t* eoff, int start_exp,
                                                    int64_t nrec, int64_t rec0, int64_t stride,
                                                    int warmup, int iters, const uint16_t* X,
                                                    int64_t* out, uint16_t* frag) {
  __shared__ RTables T;
  __shared__ __attribute__((aligned(16))) uint8_t stg[kExpStage];
  const RExp ex = r_exp(start_exp);
  build_r_tables_exp(T, threadIdx.x, 64, ex.lo, ex.hi);
  __syncthreads();
  const int l = lane_id();
  // X fragments for the MFMA step: 16 columns x 64 k (lane l: column l%16)
  const bf16x8 x0 = *reinterpret_cast<const bf16x8*>(X + (l & 15) * 64 + 8 * (l >> 4));
  const bf16x8 x1 = *reinterpret_cast<const bf16x8*>(X + (l & 15) * 64 + 32 + 8 * (l >> 4));
  uint64_t acc[kStages];
#pragma unroll
  for (int s = 0; s < kStages; ++s) acc[s] = 0;
  f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 o0 = u32x4{0, 0, 0, 0}, o1 = u32x4{0, 0, 0, 0};
  uint64_t tot0 = 0, rt0 = 0;
  for (int it = 0; it < warmup + iters; ++it) {
    if (it == warmup) {
#pragma unroll
      for (int s = 0; s < kStages; ++s) acc[s] = 0;
      rt0 = realtime();
      tot0 = stamp();
    }
    const int64_t rec = (rec0 + (int64_t)it * stride) % nrec;
    RStage st;
    RMeta mt;
    uint64_t t = stamp(), u;
    u = stamp();
    acc[0] += u - t;
    t = u;
    const int e0 = eoff[rec], e1 = eoff[rec + 1];
    keep((uint32_t)e0);
    keep((uint32_t)e1);
    u = stamp();
    acc[1] += u - t;
    t = u;
    r_issue_fixed(fixed, rec, st);
    keep4(st.r.sm);
    keep(st.r.p32);
    keep(st.r.p16);
    u = stamp();
    acc[2] += u - t;
    t = u;
    r_issue_exps(exps, __builtin_amdgcn_readfirstlane(e0), __builtin_amdgcn_readfirstlane(e1),
                 st, mt);
    keep(st.ex);
    u = stamp();
    acc[3] += u - t;
    t = u;
    r_stage(stg, st, mt);
    u = stamp();
    acc[4] += u - t;
    t = u;
    r_decode_staged<true>(T, ex, st, mt, stg, exps, o0, o1);
    keep4(o0);
    keep4(o1);
    u = stamp();
    acc[5] += u - t;
    t = u;
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(o0), x0, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(o1), x1, c, 0, 0, 0);
    keep(__float_as_uint(c[0]));
    u = stamp();
    acc[6] += u - t;
    t = u;
    {
      // the same record again, steps back to back
      const int f0 = eoff[rec], f1 = eoff[rec + 1];
      RStage s2;
      RMeta m2;
      r_issue(fixed, exps, rec, __builtin_amdgcn_readfirstlane(f0),
              __builtin_amdgcn_readfirstlane(f1), s2, m2);
      r_stage(stg, s2, m2);
      u32x4 p0, p1;
      r_decode_staged<true>(T, ex, s2, m2, stg, exps, p0, p1);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(p0), x0, c, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(p1), x1, c, 0, 0, 0);
      keep(__float_as_uint(c[0]));
    }
    u = stamp();
    acc[7] += u - t;
  }
  const uint64_t tot = stamp() - tot0;
  const uint64_t rt = realtime() - rt0;
  if (l == 0) {
#pragma unroll
    for (int s = 0; s < kStages; ++s) out[s] = (int64_t)(acc[s] / (uint64_t)iters);
    out[kStages] = (int64_t)tot;
    out[kStages + 1] = (int64_t)rt;
    out[kStages + 2] = (int64_t)__float_as_uint(c[0]);  // keeps the products live
  }
  // the last record's decoded operands, in the record's element order
  *reinterpret_cast<u32x4*>(frag + 16 * l) = o0;
  *reinterpret_cast<u32x4*>(frag + 16 * l + 8) = o1;
}

}  // namespace zs

using namespace zs;

extern "C" int zs_measure_record_stages(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                                        const int32_t* d_eoff, uint8_t start_exp, int M, int K,
                                        int64_t record0, int64_t stride, int warmup, int iters,
                                        const uint16_t* d_x, int64_t* d_out, uint16_t* d_frag) {
  if (M <= 0 || K <= 0 || (M % 64) || (K % 64) || !d_fixed || !d_exps || !d_eoff || !d_x ||
      !d_out || !d_frag)
    return ZS_E_INVAL;
  if (warmup < 0 || iters <= 0 || record0 < 0 || stride < 0) return ZS_E_INVAL;
  if ((reinterpret_cast<uintptr_t>(d_fixed) | reinterpret_cast<uintptr_t>(d_exps) |
       reinterpret_cast<uintptr_t>(d_x) | reinterpret_cast<uintptr_t>(d_frag)) & 15)
    return ZS_E_INVAL;
  const int64_t nrec = (int64_t)(M / 16) * (K / 64);
  hipLaunchKernelGGL(rstage_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, d_fixed, d_exps,
                     d_eoff, (int)start_exp, nrec, record0 % nrec, stride % nrec, warmup, iters,
                     d_x, d_out, d_frag);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? ZS_OK : (int)e;
}
