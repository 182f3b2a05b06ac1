/*
 * zs_oracle.h -- CPU restatement of the ZipServ hot path, used ONLY as a test
 * oracle (tests/, __graft_entry__.smoke(), bench.py cpu_baseline leg).
 * Nothing in the product library links or calls this code.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference checkout).  All bf16 values are carried as uint16_t bit
 * patterns.
 */
#ifndef ZS_ORACLE_H
#define ZS_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Geometry of the canonical TCA-TBE format (csrc/L_API.cu:314-557). */
#define ZSO_GT 64          /* global tile edge (64x64)          */
#define ZSO_SMALL_PER_GT 64 /* 8x8 small tiles per global tile  */
#define ZSO_MEDIAN_PER_GT 4 /* 16x64 median tiles per global tile */

/* bf16 <-> float helpers (round-to-nearest-even, NaN kept quiet). */
float    zso_bf16_to_f32(uint16_t b);
uint16_t zso_f32_to_bf16(float f);

/* Byte offset -> (row, col) of small tile `st` (0..63) inside a global tile,
 * enumerated with the reference's loop nest (csrc/L_API.cu:611-631). */
void zso_small_tile_pos(int st, int* row_off, int* col_off);

/* kernel_benchmark/utils.h:189-272  analyzeExponentDistribution_BF16. */
void zso_analyze_cpu(const uint16_t* a, int64_t n, int top[7]);
/* Same selection applied to a prebuilt 256-bin histogram. */
void zso_select_cpu(const int64_t counts[256], int top[7]);
/* kernel_benchmark/zipserv_decode_attention_ext.cu:35-135
 * (AnalyzeTopExponentsFusedKernel selection semantics). */
void zso_analyze_gpu(const uint16_t* a, int64_t n, int top[7]);
void zso_select_gpu(const int64_t counts[256], int top[7]);
void zso_histogram(const uint16_t* a, int64_t n, int64_t counts[256]);

/* Outputs of an encode.  Arrays are caller-allocated with the worst-case
 * sizes from zso_bounds(). */
typedef struct {
    uint8_t*  sign_mantissa;      /* >= M*K + 16 bytes               */
    uint16_t* compressed_full;    /* >= M*K + 8 elements             */
    uint64_t* bitmap1;            /* M*K/64                          */
    uint64_t* bitmap2;
    uint64_t* bitmap3;
    int32_t*  tile_offsets;       /* 2*M*K/64      (small tiles)     */
    int32_t*  tile_offsets_median;/* 2*M*K/1024                      */
    int32_t*  tile_offsets_global;/* 2*(M*K/4096+1)                  */
    int32_t   max_high_freq_count;
    int32_t   max_full_count;
    int64_t   total_high_freq;    /* padded SM bytes                 */
    int64_t   total_full;         /* padded FULL elements            */
} zso_encoded;

/* csrc/L_API.cu:314-557  InitBF16MatrixTripleBitmap (7-way linear search). */
int zso_compress_plain(const uint16_t* a, int M, int K, const int top[7], zso_encoded* out);
/* csrc/L_API.cu:559-771  InitBF16MatrixTripleBitmap_Reuse (LUT, 3 passes). */
int zso_compress_lut(const uint16_t* a, int M, int K, const int top[7], zso_encoded* out);
/* csrc/L_API.cu:773-1053 InitBF16MatrixTripleBitmap_Reuse_SIMD (SSE/SSSE3). */
int zso_compress_sse(const uint16_t* a, int M, int K, const int top[7], zso_encoded* out);
/* The same bytes with the global tiles spread over `threads` OpenMP threads
 * (<= 0: all), the reference benchmarks' multi-threaded compress mode. */
int zso_compress_sse_mt(const uint16_t* a, int M, int K, const int top[7], zso_encoded* out,
                        int threads);

/* kernel_benchmark/bench_kv_cache_zipserv_decompress_token_scaling.cu:2106-2218
 * DecompressZipServChunkCPU.  Returns 0, or -1 on an out-of-range stream read. */
int zso_decompress(const uint8_t* sm, int64_t sm_len, const uint16_t* full, int64_t full_len,
                   const uint64_t* b1, const uint64_t* b2, const uint64_t* b3,
                   const int32_t* tile_offsets_global, int M, int K, int start_exp,
                   uint16_t* out);

/* Y[n][m] = sum_k W[m][k] * X[n][k], fp32 accumulation in ascending k, result
 * kept in fp32 (no rounding) -- the closed form ZipGEMM must match
 * (csrc/L_Kernel.cuh:294-571 computes the same product, output [N][M]). */
/* CPU-baseline variants, same results: decoder parallel over global tiles;
 * GEMM with each W row widened once, parallel over rows (threads <= 0: all
 * cores). */
int zso_decompress_mt(const uint8_t* sm, int64_t sm_len, const uint16_t* full, int64_t full_len,
                      const uint64_t* b1, const uint64_t* b2, const uint64_t* b3,
                      const int32_t* tog, int M, int K, int start_exp, uint16_t* out,
                      int threads);
void zso_gemm_f32_mt(const uint16_t* W, const uint16_t* X, int M, int N, int K, float* Y,
                     int threads);
void zso_gemm_f32(const uint16_t* W, const uint16_t* X, int M, int N, int K, float* Y);
/* Split-K model: csrc/L_Kernel.cuh:316-326 partitions K into ceil(NK/S) GT
 * blocks per split, each split's fp32 sum is rounded to bf16, then
 * csrc/Reduction_Kernel.cuh:15-37 sums the bf16 partials in fp32 and rounds. */
void zso_gemm_splitk_bf16(const uint16_t* W, const uint16_t* X, int M, int N, int K,
                          int split_k, uint16_t* Y);

/* Decode attention for one query token with GQA, computed in fp64:
 * out[b][h][:] = softmax_t(scale * q[b][h].K[b][t][h/G]) V[b][t][h/G]
 * (flash_fwd_kernel.h compute_attn_1rowblock semantics for seqlen_q == 1).
 * q [B][H][D] bf16, k/v [B][T][Hkv][D] bf16, seqlens[b] <= T.
 * out [B][H][D] fp64, lse [B][H] fp64 (natural log). */
void zso_decode_attention_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              int B, int H, int Hkv, int T, int D, const int32_t* seqlens,
                              double scale, double* out, double* lse);
/* The same, plus absv[B][H][D] = sum_t p_t |v_t,d| (NULL: not computed). */
void zso_decode_attention_absv_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                   int B, int H, int Hkv, int T, int D, const int32_t* seqlens,
                                   double scale, double* out, double* lse, double* absv);

#ifdef __cplusplus
}
#endif
#endif

/* ------------------------------------------------------------------------ */
/* CDNA4 re-tiled device layout (this build's own layout; no counterpart in  */
/* the reference).  A lossless rearrangement of the canonical streams:       */
/* record r = band*(K/64) + kt covers rows 16*band..+15, cols 64*kt..+63.    */
/* Element (h, l, i) of a record (half h < 2, lane l < 64, i < 8) is row     */
/* 16*band + l%16, col 64*kt + 32*h + 8*(l/16) + i.  Fixed part, 1408 B per  */
/* record: byte 16*l + 8*h + i = (mantissa(h,l,i) << 1) | sign(h,l,i^1)     */
/* (the sign bit is the pair partner's); bytes 1024 + 4*l.. = u32            */
/* (C(0,l) | C(1,l) << 24); bytes 1280 + 2*l.. = u16 (C(1,l) >> 8), where    */
/* C(h,l) = sum_i code(h,l,i) << 3i and code 0 = outlier, else exponent      */
/* start + code (mod 256).  Exponent stream: for each outlier, in (h, l, i)  */
/* order, its exponent byte, at exps[eoff[r] + k]; eoff has                  */
/* num_records + 1 cumulative entries.                                       */
/* ------------------------------------------------------------------------ */
#define ZSO_REC_BYTES 1408
/* bf16 -> re-tiled layout for window start `start_exp` (in-window iff
 * (exponent - start_exp) mod 256 in 1..7, the canonical rule for the
 * contiguous window top[i] = start_exp + 1 + i). Returns the outlier count. */
int64_t zso_compress_retiled(const uint16_t* a, int M, int K, int start_exp, uint8_t* fixed,
                             uint8_t* exps, int32_t* eoff);
void zso_decompress_retiled(const uint8_t* fixed, const uint8_t* exps, const int32_t* eoff,
                            int start_exp, int M, int K, uint16_t* out);
