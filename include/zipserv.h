/*
 * zipserv.h -- C-ABI of the MI355X (gfx950) ZipServ hot path.
 *
 * Every entry point mirrors one reference interface (cited as
 * file:line relative to the reference checkout) with plain pointers and
 * sizes: bf16 data is passed as uint16_t bit patterns, streams as
 * hipStream_t cast to void*.  All device entry points are stream-ordered and
 * asynchronous; none allocates, synchronises or prints.
 *
 * Status codes: ZS_OK (0); negative ZS_E_* for argument / capability errors
 * detected on the host before any launch; a positive value is a hipError_t
 * reported by the HIP runtime for a launch.
 *
 * Canonical TCA-TBE format (shared by every entry point): M x K bf16 matrix,
 * M and K multiples of 64, cut into 64x64 global tiles (row-major over
 * tiles), each into four 16x64 median tiles, each into sixteen 8x8 small
 * tiles visited as 2x2 groups in column-major order.  Per small tile: three
 * u64 bit-planes of a 3-bit code (0 = outlier, 1..7 = exponent
 * start_exp + code), one sign|mantissa byte per in-window element (SM
 * stream), one raw bf16 per outlier (FULL stream).  Streams are padded to 16
 * bytes / 8 elements per global tile.  TileOffsets_Global holds
 * num_global_tiles + 1 (SM, FULL) cumulative pairs, TileOffsets_Median the
 * 4 per-tile (SM, FULL) starts of each median tile.
 *
 * Device SM and FULL buffers must stay readable for ZS_STREAM_SLACK_BYTES
 * bytes past the end of their streams (the decoder loads aligned 16-byte
 * windows).  Buffers produced by zs_init_bf16_matrix_triple_bitmap_gpu with
 * the worst-case sizes of zs_sign_mantissa_capacity / zs_full_capacity
 * satisfy this.
 */
#ifndef ZIPSERV_H
#define ZIPSERV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZS_OK 0
#define ZS_E_INVAL (-1)       /* bad shape, null pointer, bad tile size     */
#define ZS_E_UNSUPPORTED (-2) /* valid request this build does not handle  */
#define ZS_E_OVERFLOW (-3)    /* offsets would not fit the int32 format    */
#define ZS_E_NOMEM (-4)       /* host allocation failed                    */

#define ZS_STREAM_SLACK_BYTES 64
/* Bytes of d_tmp per 16 x 64 record for zs_compress_retiled_fixed_gpu. */
#define ZS_RETILED_EXP_SLOT_BYTES 256
/* Window rules of zs_compress_retiled_auto_gpu: the KV-cache compressor's
 * (zipserv_decode_attention_ext.cu:65-134) and the weight path's
 * (kernel_benchmark/utils.h:189-272). */
#define ZS_WINDOW_KV 0
#define ZS_WINDOW_WEIGHTS 1
/* Scratch bytes (d_work) of zs_compress_retiled_auto_gpu. */
#define ZS_RETILED_AUTO_WORK_BYTES 65600

/* KV layouts of a compressed cache (flash.h:19-20). */
#define ZS_LAYOUT_HEAD_MAJOR 0 /* rows = ((b * Hkv + h) * rows_per_head + t) */
#define ZS_LAYOUT_TOKEN_MAJOR 1 /* rows = b * batch_stride + t * Hkv + h      */

const char* zs_version(void);
const char* zs_status_string(int status);

/* ---------------------------------------------------------------------- */
/* Size queries (no counterpart function in the reference; they state the  */
/* worst-case allocations of zipserv_decode_attention_ext.cu:177-199 and    */
/* the size formula of bench_zipserv_gemm_sweep.cu:424-429).                */
/* ---------------------------------------------------------------------- */
int64_t zs_num_global_tiles(int M, int K);
int64_t zs_sign_mantissa_capacity(int M, int K); /* bytes, incl. slack      */
int64_t zs_full_capacity(int M, int K);          /* bf16 elements, incl. slack */
/* Compressed size of the GEMM path: SM + 2*FULL + bitmaps + median + global. */
int64_t zs_compressed_bytes(int M, int K, int64_t total_high_freq, int64_t total_full);
/* Bytes of Reduction_Workspace needed by zs_bf16_triple_bitmap_mm. */
int64_t zs_splitk_workspace_bytes(int M, int N, int split_k);

/* ---------------------------------------------------------------------- */
/* Host codec (CPU)                                                         */
/* ---------------------------------------------------------------------- */

/* kernel_benchmark/utils.h:189-272 analyzeExponentDistribution_BF16:
 * window of 7 contiguous exponents; top_exponents[i] = start + i. */
int zs_analyze_exponents_host(const uint16_t* a, int64_t n, int32_t top_exponents[7]);

/* build/L_API.cuh:53-73 InitBF16MatrixTripleBitmap.  Allocates every output
 * (release each with zs_host_free); returns the number of global tiles or a
 * negative status.  Tile sizes must be (8,16,64, 8,64,64). */
int zs_init_bf16_matrix_triple_bitmap(
    const uint16_t* A, int M, int K, int tile_M, int tile_M_median, int tile_M_global, int tile_K,
    int tile_K_median, int tile_K_global, const int32_t* top_exponents, uint8_t** sign_mantissa,
    uint16_t** compressed_full, uint64_t** bitmap1, uint64_t** bitmap2, uint64_t** bitmap3,
    int32_t** tile_offsets, int32_t** tile_offsets_median, int32_t** tile_offsets_global,
    int32_t* max_high_freq_count, int32_t* max_full_count);
void zs_host_free(void* p);

/* build/L_API.cuh:76-107 InitBF16MatrixTripleBitmap_Reuse: caller buffers
 * (SM >= M*K bytes, FULL >= M*K elements, temp_sm num_GT*(4096+15) bytes,
 * temp_full num_GT*(4096+7) elements, gt_* num_GT, *_offsets num_GT+1).
 * Accepts any 7 distinct exponents. */
int zs_init_bf16_matrix_triple_bitmap_reuse(
    const uint16_t* A, int M, int K, int tile_M, int tile_M_median, int tile_M_global, int tile_K,
    int tile_K_median, int tile_K_global, const int32_t* top_exponents, uint8_t* sign_mantissa,
    uint16_t* compressed_full, uint64_t* bitmap1, uint64_t* bitmap2, uint64_t* bitmap3,
    int32_t* tile_offsets, int32_t* tile_offsets_median, int32_t* tile_offsets_global,
    uint8_t* temp_sm, uint16_t* temp_full, int32_t* gt_hf_count, int32_t* gt_full_count,
    int32_t* hf_offsets, int32_t* full_offsets, int32_t* max_high_freq_count,
    int32_t* max_full_count, int32_t* out_total_hf, int32_t* out_total_full);

/* build/L_API.cuh:109-141 InitBF16MatrixTripleBitmap_Reuse_SIMD: same
 * buffers; the window is taken as [top_exponents[0], top_exponents[0]+6]. */
int zs_init_bf16_matrix_triple_bitmap_reuse_simd(
    const uint16_t* A, int M, int K, int tile_M, int tile_M_median, int tile_M_global, int tile_K,
    int tile_K_median, int tile_K_global, const int32_t* top_exponents, uint8_t* sign_mantissa,
    uint16_t* compressed_full, uint64_t* bitmap1, uint64_t* bitmap2, uint64_t* bitmap3,
    int32_t* tile_offsets, int32_t* tile_offsets_median, int32_t* tile_offsets_global,
    uint8_t* temp_sm, uint16_t* temp_full, int32_t* gt_hf_count, int32_t* gt_full_count,
    int32_t* hf_offsets, int32_t* full_offsets, int32_t* max_high_freq_count,
    int32_t* max_full_count, int32_t* out_total_hf, int32_t* out_total_full);

/* ---------------------------------------------------------------------- */
/* Device codec and kernels (gfx950)                                        */
/* ---------------------------------------------------------------------- */

/* build/L_API.cuh:38-52 BF16TripleBitmap_Decompress_API: TCA-TBE -> dense
 * Output[M][K] bf16, bit-exact. */
int zs_bf16_triple_bitmap_decompress(void* stream, const uint8_t* SignMantissa,
                                     const uint16_t* CompressedFull, const uint64_t* Bitmap1,
                                     const uint64_t* Bitmap2, const uint64_t* Bitmap3,
                                     const int32_t* TileOffsets_Median,
                                     const int32_t* TileOffsets_Global, int max_high_freq_count,
                                     int max_full_count, uint8_t start_exp, uint16_t* Output,
                                     int M_Global, int K_Global);

/* build/L_API.cuh:19-37 BF16TripleBitmap_MM_API: C[N][M] = B[N][K] . W[M][K]^T
 * with W in TCA-TBE, fp32 accumulation, bf16 output.  Split_K > 1 writes
 * bf16 partial slabs [Split_K][N][M] into Reduction_Workspace (at least
 * zs_splitk_workspace_bytes) and sums them in fp32 (Reduction_Kernel.cuh). */
int zs_bf16_triple_bitmap_mm(void* stream, const uint8_t* SignMantissa,
                             const uint16_t* CompressedFull, const uint64_t* Bitmap1,
                             const uint64_t* Bitmap2, const uint64_t* Bitmap3,
                             const int32_t* TileOffsets_Median, const int32_t* TileOffsets_Global,
                             int max_high_freq_count, int max_full_count, uint8_t start_exp,
                             const uint16_t* B, uint16_t* C, int M_Global, int N_Global,
                             int K_Global, uint16_t* Reduction_Workspace, int Split_K);

/* kernel_benchmark/zipserv_decode_attention_ext.cu:137-153
 * AnalyzeTopExponentsGPU: 256-bin histogram of d_input (d_exponent_counts,
 * 256 int32) and the GPU window selection (ext.cu:65-134) into
 * d_top_exponents[7].  d_done_counter (1 int32) is cleared and unused. */
int zs_analyze_top_exponents_gpu(void* stream, const uint16_t* d_input, int64_t numel,
                                 int32_t* d_exponent_counts, int32_t* d_top_exponents,
                                 int32_t* d_done_counter);
/* The same histogram and selection with 64-bit bins (d_exponent_counts:
 * 256 uint64), for tensors past the int32 bins above (numel > INT32_MAX,
 * e.g. a 32 x 8 x 128k x 128 KV cache).  No counterpart in the reference,
 * whose int32 counters (ext.cu:35-63) overflow there; the window rule is
 * unchanged, so it returns the same window wherever both apply. */
int zs_analyze_top_exponents_u64_gpu(void* stream, const uint16_t* d_input, int64_t numel,
                                     uint64_t* d_exponent_counts, int32_t* d_top_exponents);
/* kernel_benchmark/utils.h:189-272 analyzeExponentDistribution_BF16 (the
 * weights path's host window rule: seven strict-maximum passes, ties to the
 * lowest exponent, no [0, 248] clamp) on the device, over the same 64-bit
 * histogram as above: the window zs_analyze_exponents_host returns, without
 * copying the matrix to the host.  The reference runs this rule on the CPU
 * only; the two rules differ on sparse histograms (e.g. a single exponent). */
int zs_analyze_exponents_weights_gpu(void* stream, const uint16_t* d_input, int64_t numel,
                                     uint64_t* d_exponent_counts, int32_t* d_top_exponents);

/* build/L_API.cuh:144-165 InitBF16MatrixTripleBitmap_GPU: device encoder
 * producing the canonical streams.  d_temp_sm / d_temp_full are accepted for
 * signature parity and may be NULL (the encoder re-reads d_input instead of
 * staging per-tile streams).  d_hf_offsets / d_full_offsets (num_GT + 1) and
 * the four scalars are written as in the reference. */
int zs_init_bf16_matrix_triple_bitmap_gpu(
    void* stream, const uint16_t* d_input, int M, int K, const int32_t* d_top_exponents,
    uint8_t* d_sign_mantissa, uint16_t* d_compressed_full, uint64_t* d_bitmap1,
    uint64_t* d_bitmap2, uint64_t* d_bitmap3, int32_t* d_tile_offsets,
    int32_t* d_tile_offsets_median, int32_t* d_tile_offsets_global, uint8_t* d_temp_sm,
    uint16_t* d_temp_full, int32_t* d_gt_hf_count, int32_t* d_gt_full_count,
    int32_t* d_hf_offsets, int32_t* d_full_offsets, int32_t* d_max_hf_count,
    int32_t* d_max_full_count, int32_t* d_total_hf, int32_t* d_total_full);

/* ---------------------------------------------------------------------- */
/* CDNA4 re-tiled layout (this library's device layout; no counterpart in   */
/* the reference).  A lossless rearrangement of the canonical streams with  */
/* the same size: one fixed 1408-byte record per 16x64 tile (record r =     */
/* band * K/64 + kt) holding every element's mantissa and sign bits and its */
/* 3-bit exponent code in MFMA-lane order, plus a stream of the outliers'   */
/* exponent bytes with num_records + 1 int32 cumulative offsets (layout in  */
/* csrc/zs_rdecode.hpp).  `fixed` and `exps` must be 16-byte aligned    */
/* and `exps` must keep ZS_STREAM_SLACK_BYTES readable bytes past its end.  */
/* ---------------------------------------------------------------------- */
int64_t zs_retiled_num_records(int M, int K);
int64_t zs_retiled_fixed_bytes(int M, int K);
/* bf16 -> re-tiled, two phases: count + scan (d_counts: num_records int32,
 * d_eoff: num_records + 1, d_total: 1 int64 = number of outlier bytes),
 * then emit once the caller has sized d_exps.  d_top_exponents is the window
 * from zs_analyze_top_exponents_gpu (start_exp = top[0] - 1). */
int zs_compress_retiled_count_gpu(void* stream, const uint16_t* d_input, int M, int K,
                                  const int32_t* d_top_exponents, int32_t* d_counts,
                                  int32_t* d_eoff, int64_t* d_total);
int zs_compress_retiled_emit_gpu(void* stream, const uint16_t* d_input, int M, int K,
                                 const int32_t* d_top_exponents, const int32_t* d_eoff,
                                 uint8_t* d_fixed, uint8_t* d_exps);
/* The same bytes with the input read once after the window histogram (two
 * input passes in all instead of three): zs_compress_retiled_fixed_gpu
 * writes the fixed parts, the per-record outlier counts and their offsets
 * (*d_total as above) and parks up to ZS_RETILED_EXP_SLOT_BYTES outlier bytes
 * per record in d_tmp (num_records * ZS_RETILED_EXP_SLOT_BYTES bytes); once d_exps is allocated (*d_total +
 * ZS_STREAM_SLACK_BYTES), zs_compress_retiled_exps_gpu moves them into the
 * exponent stream (records with more outliers re-read their input tile) and
 * writes the ZS_STREAM_SLACK_BYTES bytes after it as zeros. */
int zs_compress_retiled_fixed_gpu(void* stream, const uint16_t* d_input, int M, int K,
                                  const int32_t* d_top_exponents, uint8_t* d_fixed,
                                  int32_t* d_counts, int32_t* d_eoff, int64_t* d_total,
                                  uint8_t* d_tmp);
/* zs_analyze_* + zs_compress_retiled_fixed_gpu in one input pass (when the
 * guess holds): the window (rule ZS_WINDOW_KV or ZS_WINDOW_WEIGHTS) is
 * guessed from a sample of the input (every 32nd 4096-byte chunk, or sparser
 * so that at most 128 chunks are read; a partial last chunk is not sampled),
 * the fixed parts,
 * counts and slots are written under the guess while the full exponent
 * histogram is counted (d_hist, 256 x uint64, out), the rule picks the window
 * from the full histogram (d_top, out), and only if it differs from the guess
 * are the fixed parts, counts and slots written again under it.  Outputs are
 * those of zs_analyze_* (u64 bins) followed by zs_compress_retiled_fixed_gpu
 * with d_top.  d_work: ZS_RETILED_AUTO_WORK_BYTES of device scratch (8-byte
 * aligned).  No counterpart in the reference, whose compressor reads its
 * input once for the histogram and once more per encoding pass. */
int zs_compress_retiled_auto_gpu(void* stream, const uint16_t* d_input, int M, int K, int rule,
                                 uint64_t* d_hist, int32_t* d_top, uint8_t* d_work,
                                 uint8_t* d_fixed, int32_t* d_counts, int32_t* d_eoff,
                                 int64_t* d_total, uint8_t* d_tmp);
/* zs_compress_retiled_auto_gpu with the guess taken from d_guess (7 int32
 * window exponents in device memory, e.g. d_top of the previous matrix of a
 * model's weights, which share one window) instead of a sample of the input:
 * one small launch instead of the sample and its selection.  The outputs are
 * the same bytes whatever d_guess holds (a wrong guess costs the second
 * encoding).  d_guess must not alias d_top.  No counterpart in the
 * reference (no GPU encoder of weights there). */
int zs_compress_retiled_guess_gpu(void* stream, const uint16_t* d_input, int M, int K, int rule,
                                  const int32_t* d_guess, uint64_t* d_hist, int32_t* d_top,
                                  uint8_t* d_work, uint8_t* d_fixed, int32_t* d_counts,
                                  int32_t* d_eoff, int64_t* d_total, uint8_t* d_tmp);
int zs_compress_retiled_exps_gpu(void* stream, const uint16_t* d_input, int M, int K,
                                 const int32_t* d_top_exponents, const int32_t* d_eoff,
                                 const uint8_t* d_tmp, uint8_t* d_exps);
/* Canonical TCA-TBE streams -> re-tiled, same two phases (window start_exp). */
int zs_retile_triple_bitmap_count_gpu(void* stream, const uint8_t* SignMantissa,
                                      const uint16_t* CompressedFull, const uint64_t* Bitmap1,
                                      const uint64_t* Bitmap2, const uint64_t* Bitmap3,
                                      const int32_t* TileOffsets_Median,
                                      const int32_t* TileOffsets_Global, int M, int K,
                                      int32_t* d_counts, int32_t* d_eoff, int64_t* d_total);
int zs_retile_triple_bitmap_emit_gpu(void* stream, const uint8_t* SignMantissa,
                                     const uint16_t* CompressedFull, const uint64_t* Bitmap1,
                                     const uint64_t* Bitmap2, const uint64_t* Bitmap3,
                                     const int32_t* TileOffsets_Median,
                                     const int32_t* TileOffsets_Global, uint8_t start_exp, int M,
                                     int K, const int32_t* d_eoff, uint8_t* d_fixed,
                                     uint8_t* d_exps);
/* Decompress / ZipGEMM over the re-tiled layout: same results as
 * zs_bf16_triple_bitmap_decompress / zs_bf16_triple_bitmap_mm on the
 * canonical streams it was built from (same split-K semantics). */
int zs_retiled_decompress(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                          const int32_t* d_eoff, uint8_t start_exp, uint16_t* out, int M, int K);
int zs_retiled_mm(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                  const int32_t* d_eoff, uint8_t start_exp, const uint16_t* B, uint16_t* C, int M,
                  int N, int K, uint16_t* Reduction_Workspace, int Split_K);
/* zs_retiled_mm with the split-K reduction inside the GEMM kernel (no
 * counterpart in the reference, whose split-K always runs
 * SplitK_Reduction, build/L_API.cuh:19-37): every workgroup stores its bf16
 * partial tile into the workspace as above, and the last one of each output
 * tile to finish adds the Split_K slices in split order and writes C -- the
 * same sums and rounding as the two-kernel path, one launch instead of two.
 * d_counters: zs_retiled_mm_counters(M, N) int32 arrival counters (4-byte
 * aligned), zero-filled by the caller once, when allocated; every completed
 * call leaves them zero.  Calls that may overlap in time (other streams)
 * must not share counters or workspace.  The workspace must be 8-byte
 * aligned.  With Split_K == 1 the counters are not touched. */
int64_t zs_retiled_mm_counters(int M, int N);
int zs_retiled_mm_fused(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                        const int32_t* d_eoff, uint8_t start_exp, const uint16_t* B, uint16_t* C,
                        int M, int N, int K, uint16_t* Reduction_Workspace, int Split_K,
                        int32_t* d_counters);
/* Stream-K schedule of the re-tiled ZipGEMM for N <= 16 (no counterpart in
 * the reference, whose Split_K cuts every band's K range into equal slices):
 * one round of workgroups, each over an equal contiguous range of the
 * M/16 x K/64 records in band-major order, so no CU idles for a band count
 * that does not divide over the workgroups and no band pays a workgroup
 * start-up; bands shared between workgroups are added from fp32 partials
 * (no bf16 rounding of partials) in a fixed order, so results are
 * deterministic on one device.  `workspace`: workspace_bytes >=
 * zs_retiled_mm_streamk_workspace_bytes(M, N, K) (for the current device),
 * 16-byte aligned; `d_counters`: >= M/16 int32, zero before the first call
 * and left zero by every call (as zs_retiled_mm_fused's).  Returns
 * ZS_E_UNSUPPORTED for N > 16 and for shapes whose ranges would meet more
 * than 8 bands (zs_retiled_mm_streamk_workspace_bytes returns 0 for them). */
int64_t zs_retiled_mm_streamk_workspace_bytes(int M, int N, int K);
int zs_retiled_mm_streamk(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                          const int32_t* d_eoff, uint8_t start_exp, const uint16_t* B, uint16_t* C,
                          int M, int N, int K, void* workspace, size_t workspace_bytes,
                          int32_t* d_counters);
/* zs_retiled_mm_fused that allocates nothing and takes no workspace: no
 * counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The split-K partial slabs and arrival counters live in a
 * static device array of the library, 32 MiB of partials + 64 Ki counters,
 * one copy per GPU held until the process ends: Split_K > 1 requires
 * Split_K * M * N * 2 <= 32 MiB and zs_retiled_mm_counters(M, N) <= 65536,
 * else ZS_E_OVERFLOW before any launch.  Arguments are validated before
 * the array is touched; Split_K == 1 never touches it.  The first Split_K > 1
 * call on a device looks the array up and clears its counters with a fill
 * kernel on `stream` (no memset node, so that call may also be captured);
 * every completed call leaves them zero.  All calls on one GPU share the
 * array: calls that overlap in time on one GPU (other streams, other
 * threads) race and must not be issued. */
int zs_retiled_mm_fused_noalloc(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                                const int32_t* d_eoff, uint8_t start_exp, const uint16_t* B,
                                uint16_t* C, int M, int N, int K, int Split_K);

/* ---------------------------------------------------------------------- */
/* Decode attention over a compressed KV cache                              */
/* ---------------------------------------------------------------------- */

/* One compressed K or V cache (flash.h:51-68 ZipservCompressedKVParams; the
 * 12 fields of flash_attn_interface.py:23-36 plus the strides derived by
 * _normalize_zipserv_kv, flash_attn_interface.py:75-128). */
typedef struct zs_kv_compressed {
  const uint8_t* sign_mantissa;
  const uint16_t* compressed_full;
  const uint64_t* bitmap1;
  const uint64_t* bitmap2;
  const uint64_t* bitmap3;
  const int32_t* tile_offsets_median;
  const int32_t* tile_offsets_global;
  int32_t rows;              /* padded rows of the 2D matrix                 */
  int32_t cols;              /* padded head_dim (multiple of 64)            */
  int32_t batch_stride_rows; /* rows / batch                                */
  int32_t head_stride_rows;  /* batch_stride_rows / num_heads_k             */
  int32_t max_high_freq_count;
  int32_t max_full_count;
  int32_t start_exp;
  int32_t layout; /* ZS_LAYOUT_*                                           */
} zs_kv_compressed_t;

/* flash_attn_interface.py:1572-1706 flash_attn_with_kvcache(...,
 * zipserv_k=, zipserv_v=) -> flash_api.cpp:1346-1520 mha_fwd_kvcache for one
 * query token (decode): out[b][h] = softmax(scale * q[b][h] . K[b][:L_b][h/G])
 * . V[b][:L_b][h/G], G = num_heads / num_heads_k, fp32 online softmax.
 * q, out: [batch][num_heads][head_dim] bf16, 16-byte aligned.  L_b = cache_seqlens[b] (device
 * int32 [batch]) or seqlen_k when cache_seqlens is NULL.  softmax_lse
 * (optional, [batch][num_heads] fp32) is the natural-log normaliser.
 * num_splits = 0 picks a split of the sequence across workgroups; splits > 1
 * need `workspace` of zs_decode_attention_workspace_bytes bytes.
 * Layouts (flash.h:19-20): HEAD_MAJOR caches (row (b*Hkv + h)*head_stride +
 * t) are decoded inside the attention kernel; TOKEN_MAJOR caches (row
 * b*batch_stride + t*Hkv + h) run staged -- both are first decompressed into
 * the front of `workspace`, which then needs zs_kv_staging_bytes(layout,
 * rows, cols) for K and for V in addition (the same result, bit for bit).
 * K and V must share one layout. */
int64_t zs_kv_staging_bytes(int layout, int rows, int cols);
int zs_decode_attention(void* stream, const uint16_t* q, const zs_kv_compressed_t* k,
                        const zs_kv_compressed_t* v, const int32_t* cache_seqlens, int seqlen_k,
                        int batch, int num_heads, int num_heads_k, int head_dim,
                        float softmax_scale, uint16_t* out, float* softmax_lse, void* workspace,
                        size_t workspace_bytes, int num_splits);
size_t zs_decode_attention_workspace_bytes(int batch, int num_heads, int head_dim, int seqlen_k,
                                           int num_splits);

/* The same decode attention over caches held in the re-tiled layout (no
 * counterpart in the reference; its KV caches use the canonical streams).
 * Fields mirror zs_kv_compressed_t with the three re-tiled buffers. */
typedef struct zs_kv_retiled {
  const uint8_t* fixed;      /* num_records * 1408 bytes, 16-byte aligned      */
  const uint8_t* exps;       /* outlier bytes (+ ZS_STREAM_SLACK_BYTES)        */
  const int32_t* eoff;       /* num_records + 1 offsets into exps              */
  int32_t rows;
  int32_t cols;
  int32_t batch_stride_rows;
  int32_t head_stride_rows;
  int32_t start_exp;
  int32_t layout; /* ZS_LAYOUT_*                                           */
} zs_kv_retiled_t;

/* TOKEN_MAJOR re-tiled caches with num_heads_k == 8 and head_dim 128 are
 * decoded inside the attention kernel (flash_fwd_kernel.h:325-430, :449,
 * :522-536 decode token-major tiles in the kernel too): one workgroup per
 * (batch, split) decodes each record once for all 8 heads and exchanges the
 * rows through LDS; same result, bit for bit, as the dense kernel with one
 * wave per (batch, head, split).  Other token-major caches run staged as in
 * zs_decode_attention. */
int zs_decode_attention_retiled(void* stream, const uint16_t* q, const zs_kv_retiled_t* k,
                                const zs_kv_retiled_t* v, const int32_t* cache_seqlens,
                                int seqlen_k, int batch, int num_heads, int num_heads_k,
                                int head_dim, float softmax_scale, uint16_t* out,
                                float* softmax_lse, void* workspace, size_t workspace_bytes,
                                int num_splits);
/* Staging bytes zs_decode_attention_retiled needs for one cache in front of
 * its split workspace: 0 for head-major caches and for fused token-major
 * ones (num_heads_k == 8, cols == 128), zs_kv_staging_bytes otherwise; -1
 * for bad arguments.  No counterpart in the reference. */
int64_t zs_kv_retiled_staging_bytes(int layout, int rows, int cols, int num_heads_k);

/* The uncompressed comparator (bench_zipserv_decode_attention.py:629-631,
 * dense flash_attn_with_kvcache): same kernel with K/V read from dense bf16
 * caches k_cache / v_cache [batch][cache_capacity][num_heads_k][head_dim]. */
int zs_decode_attention_dense(void* stream, const uint16_t* q, const uint16_t* k_cache,
                              const uint16_t* v_cache, const int32_t* cache_seqlens,
                              int seqlen_k, int cache_capacity, int batch, int num_heads,
                              int num_heads_k, int head_dim, float softmax_scale, uint16_t* out,
                              float* softmax_lse, void* workspace, size_t workspace_bytes,
                              int num_splits);

/* The same over a paged dense cache (flash_attn_interface.py:1583-1658
 * flash_attn_with_kvcache(..., block_table=) -> flash_api.cpp mha_fwd_kvcache,
 * flash_fwd_kernel.h:1229-1239,1410-1420): k_cache / v_cache are pages
 * [num_blocks][page_block_size][num_heads_k][head_dim]; token t of sequence
 * b is row t % page_block_size of page block_table[b * max_blocks_per_seq +
 * t / page_block_size].  page_block_size must be a multiple of 16 (the
 * reference's paged FlashInfer runs use 16; its FlashAttention path asks for
 * multiples of 256); block_table entries must lie in [0, num_blocks). */
int zs_decode_attention_dense_paged(void* stream, const uint16_t* q, const uint16_t* k_cache,
                                    const uint16_t* v_cache, const int32_t* block_table,
                                    int max_blocks_per_seq, int num_blocks, int page_block_size,
                                    const int32_t* cache_seqlens, int seqlen_k, int batch,
                                    int num_heads, int num_heads_k, int head_dim,
                                    float softmax_scale, uint16_t* out, float* softmax_lse,
                                    void* workspace, size_t workspace_bytes, int num_splits);

/* Stage profiler of the re-tiled record pipeline
 * (kernel_benchmark/zipserv_tile_stage_bench_ext.cu measure_zipserv_tile_stages):
 * one wave consumes records record0 + i*stride (mod num_records), waiting
 * out every memory operation and reading the shader clock between the steps.
 * d_out (11 int64, device): mean cycles of [bracket, offsets, fixed, exps,
 * stage, decode, mfma, record] over `iters` iterations after `warmup`, then
 * the loop's total shader cycles and its s_memrealtime ticks (100 MHz), then
 * a value that keeps the products live.  d_x: 16 x 64 bf16 MFMA tile;
 * d_frag: 64 x 16 bf16, the last record's decoded operands in lane order. */
int zs_measure_record_stages(void* stream, const uint8_t* d_fixed, const uint8_t* d_exps,
                             const int32_t* d_eoff, uint8_t start_exp, int M, int K,
                             int64_t record0, int64_t stride, int warmup, int iters,
                             const uint16_t* d_x, int64_t* d_out, uint16_t* d_frag);

/* ---------------------------------------------------------------------- */
/* Container: one compressed matrix as a self-checking byte image (no       */
/* counterpart in the reference, which keeps compressed matrices only in    */
/* memory as seven tensors plus the meta tensor of                          */
/* zipserv_decode_attention_ext.cu:250-262).  Host memory only.  Layout:    */
/* a 256-byte header (magic "ZSRVCNTR", version 1, layout, shape, window,   */
/* max counts, name, per-stream sizes and CRC-32C, header CRC-32C) and the  */
/* streams, each zero-padded to 64 bytes (csrc/zs_container.cpp).           */
/* ---------------------------------------------------------------------- */
#define ZS_CONTAINER_CANONICAL 0 /* 7 streams: SM, FULL, bitmap1..3, median, global */
#define ZS_CONTAINER_RETILED 1   /* 3 streams: fixed records, exponents, offsets    */

typedef struct zs_container_desc {
  int32_t layout; /* ZS_CONTAINER_*                                         */
  int32_t rows, cols, logical_rows, logical_cols;
  int32_t start_exp, max_high_freq_count, max_full_count;
  int32_t num_streams;
  int64_t stream_bytes[8];
} zs_container_desc_t;

/* CRC-32C (Castagnoli) of `bytes` bytes continuing from `crc` (0 to start). */
uint32_t zs_crc32c(uint32_t crc, const void* data, int64_t bytes);
/* Bytes of the container for `d`, or a negative ZS_E_* if `d` is invalid
 * (stream sizes the shape fixes, window range, stream counts). */
int64_t zs_container_bytes(const zs_container_desc_t* d);
/* Writes the container into dst (>= zs_container_bytes).  streams[i]: host
 * pointers to the stream bytes in table order.  name: up to 63 bytes. */
int zs_container_write(const zs_container_desc_t* d, const char* name,
                       const void* const* streams, void* dst, int64_t dst_bytes);
/* Validates a container image (magic, version, CRCs, sizes, and every offset
 * against the bit-planes / codes it indexes: canonical global and median
 * tile offsets, re-tiled per-record outlier offsets) and returns its
 * descriptor, name (64 bytes) and each stream's byte offset in src.
 * ZS_E_INVAL for a damaged or inconsistent image (CRC-valid images with bad
 * offsets included), ZS_E_UNSUPPORTED for another version.  zs_container_write
 * applies the same offset check to its input. */
int zs_container_parse(const void* src, int64_t src_bytes, zs_container_desc_t* d,
                       char* name_out, int64_t* stream_offsets);

#ifdef __cplusplus
}
#endif
#endif /* ZIPSERV_H */
