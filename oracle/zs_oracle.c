/*
 * zs_oracle.c -- TEST INFRASTRUCTURE ONLY: a plain-C restatement of the
 * ZipServ hot path, used as the parity checker by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg.  The product
 * library (zipserv_asplos26_amd/) never links, loads or calls it.
 *
 * Parity pins (tests/test_oracle_*.py):
 *   analyze (cpu + gpu selection) : hand-built histograms (ties, zero counts,
 *                                   127-n fill, longest-run fallback, clamp)
 *   compress (plain / lut / sse)  : three independent restatements must emit
 *                                   identical bytes; hand-derived known
 *                                   answers (uniform tiles, single outlier,
 *                                   position-coded tiles); stream invariants
 *   decompress                    : decode(encode(W)) == W bit-for-bit;
 *                                   hand-built stream known answers
 *   gemm / split-k                : numpy float64 matmul, unit-vector
 *                                   column extraction, split-K rounding model
 *   decode attention              : numpy softmax attention, T=1, equal
 *                                   scores, one-hot scores
 */
#include "zs_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>
#include <tmmintrin.h> /* SSSE3 (_mm_shuffle_epi8) for the SIMD restatement */

/* ------------------------------------------------------------------------ */
/* bf16 helpers                                                             */
/* ------------------------------------------------------------------------ */
float zso_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t zso_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40);
    uint32_t rounding = 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)((u + rounding) >> 16);
}

/* ------------------------------------------------------------------------ */
/* Small-tile traversal inside one 64x64 global tile.                       */
/* csrc/L_API.cu:611-631 (tile_pos[] of _Reuse), identical to the nested    */
/* loops of InitBF16MatrixTripleBitmap at L_API.cu:403-428: median tiles    */
/* top to bottom, then 2x2 groups of 8x8 tiles left to right, each group    */
/* visited column-major: (r0,c0) (r1,c0) (r0,c1) (r1,c1).                   */
/* ------------------------------------------------------------------------ */
static int g_pos_row[64], g_pos_col[64], g_pos_ready = 0;

static void init_tile_pos(void) {
    if (g_pos_ready) return;
    const int tile_M = 8, tile_M_median = 16, tile_M_global = 64;
    const int tile_K = 8, tile_K_median = 64, tile_K_global = 64;
    int tp = 0;
    for (int mm = 0; mm < tile_M_global / tile_M_median; ++mm)
        for (int mk = 0; mk < tile_K_global / tile_K_median; ++mk) {
            const int med_row = mm * tile_M_median, med_col = mk * tile_K_median;
            for (int mg = 0; mg < tile_M_median / tile_M; mg += 2)
                for (int kg = 0; kg < tile_K_median / tile_K; kg += 2)
                    for (int j = 0; j < 2; ++j)
                        for (int i = 0; i < 2; ++i) {
                            g_pos_row[tp] = med_row + (mg + i) * tile_M;
                            g_pos_col[tp] = med_col + (kg + j) * tile_K;
                            ++tp;
                        }
        }
    g_pos_ready = 1;
}

void zso_small_tile_pos(int st, int* row_off, int* col_off) {
    init_tile_pos();
    *row_off = g_pos_row[st & 63];
    *col_off = g_pos_col[st & 63];
}

/* ------------------------------------------------------------------------ */
/* Exponent window selection                                                */
/* ------------------------------------------------------------------------ */
void zso_histogram(const uint16_t* a, int64_t n, int64_t counts[256]) {
    memset(counts, 0, 256 * sizeof(int64_t));
    for (int64_t i = 0; i < n; ++i) counts[(a[i] >> 7) & 0xFF]++;
}

static void sort7(int* v) {
    for (int i = 1; i < 7; ++i) {
        int key = v[i], j = i - 1;
        while (j >= 0 && v[j] > key) { v[j + 1] = v[j]; --j; }
        v[j + 1] = key;
    }
}

/* Shared tail of both selections: first contiguous all-present window starting
 * at one of the sorted candidates (utils.h:228-246 / ext.cu:103-115), else the
 * start of the longest run among the candidates (utils.h:249-270 /
 * ext.cu:117-130).  `clamp` applies ext.cu:131-133. */
static void window_from_candidates(const int64_t counts[256], int* cand, int clamp, int top[7]) {
    sort7(cand);
    for (int c = 0; c < 7; ++c) {
        const int start = cand[c];
        if (start < 0 || start + 6 > 255) continue;
        int ok = 1;
        for (int i = 0; i < 7; ++i)
            if (counts[start + i] <= 0) { ok = 0; break; }
        if (!ok) continue;
        for (int i = 0; i < 7; ++i) top[i] = start + i;
        return;
    }
    int best_start = cand[0], max_len = 1, cur = 1;
    for (int i = 1; i < 7; ++i) {
        if (cand[i] == cand[i - 1] + 1) {
            ++cur;
            if (cur > max_len) { max_len = cur; best_start = cand[i] - cur + 1; }
        } else {
            cur = 1;
        }
    }
    if (clamp) {
        if (best_start < 0) best_start = 0;
        if (best_start > 255 - 7) best_start = 255 - 7;
    }
    for (int i = 0; i < 7; ++i) top[i] = best_start + i;
}

/* kernel_benchmark/utils.h:200-225: seven passes picking the strictly largest
 * unused count (ties -> lowest exponent, zero counts never picked), then the
 * 127-n fill for missing candidates. */
void zso_select_cpu(const int64_t counts[256], int top[7]) {
    int cand[7], used[256], n_found = 0;
    memset(used, 0, sizeof(used));
    for (int t = 0; t < 7; ++t) {
        int best = -1;
        int64_t best_count = 0;
        for (int e = 0; e < 256; ++e)
            if (!used[e] && counts[e] > best_count) { best_count = counts[e]; best = e; }
        if (best >= 0) { cand[n_found++] = best; used[best] = 1; }
    }
    while (n_found < 7) { cand[n_found] = 127 - n_found; ++n_found; }
    window_from_candidates(counts, cand, 0, top);
}

/* kernel_benchmark/zipserv_decode_attention_ext.cu:65-91: a 7-slot
 * replace-the-minimum scan over e = 0..255 with slots initialised to count -1
 * (so zero counts can be taken), first minimum slot replaced on strict >. */
void zso_select_gpu(const int64_t counts[256], int top[7]) {
    int top_exp[7];
    int64_t top_cnt[7];
    for (int i = 0; i < 7; ++i) { top_exp[i] = -1; top_cnt[i] = -1; }
    for (int e = 0; e < 256; ++e) {
        int min_idx = 0;
        for (int i = 1; i < 7; ++i)
            if (top_cnt[i] < top_cnt[min_idx]) min_idx = i;
        if (counts[e] > top_cnt[min_idx]) { top_cnt[min_idx] = counts[e]; top_exp[min_idx] = e; }
    }
    int cand[7], n_found = 0;
    for (int i = 0; i < 7; ++i)
        if (top_exp[i] >= 0) cand[n_found++] = top_exp[i];
    while (n_found < 7) { cand[n_found] = 127 - n_found; ++n_found; }
    window_from_candidates(counts, cand, 1, top);
}

void zso_analyze_cpu(const uint16_t* a, int64_t n, int top[7]) {
    int64_t counts[256];
    zso_histogram(a, n, counts);
    zso_select_cpu(counts, top);
}

void zso_analyze_gpu(const uint16_t* a, int64_t n, int top[7]) {
    int64_t counts[256];
    zso_histogram(a, n, counts);
    zso_select_gpu(counts, top);
}

/* ------------------------------------------------------------------------ */
/* Encoders                                                                 */
/* ------------------------------------------------------------------------ */
static int check_dims(int M, int K) {
    return (M > 0 && K > 0 && M % 64 == 0 && K % 64 == 0) ? 0 : -1;
}

/* csrc/L_API.cu:314-557.  Single pass; streams appended in traversal order,
 * each global tile padded to 16 SM bytes / 8 FULL elements (:512-524),
 * cumulative global offsets built after the pass (:541-550). */
int zso_compress_plain(const uint16_t* a, int M, int K, const int top[7], zso_encoded* out) {
    if (check_dims(M, K)) return -1;
    const int gtm = M / 64, gtk = K / 64, ngt = gtm * gtk;
    int64_t* g_hf = (int64_t*)calloc((size_t)ngt + 1, sizeof(int64_t));
    int64_t* g_full = (int64_t*)calloc((size_t)ngt + 1, sizeof(int64_t));
    if (!g_hf || !g_full) { free(g_hf); free(g_full); return -1; }
    int64_t sm_off = 0, full_off = 0;
    int64_t tile_idx = 0, median_idx = 0;
    out->max_high_freq_count = 0;
    out->max_full_count = 0;
    for (int gm = 0; gm < gtm; ++gm) {
        for (int gk = 0; gk < gtk; ++gk) {
            const int grow = gm * 64, gcol = gk * 64;
            int ghf = 0, gfull = 0, mhf = 0, mfull = 0;
            out->tile_offsets_median[median_idx * 2] = 0;
            out->tile_offsets_median[median_idx * 2 + 1] = 0;
            ++median_idx;
            for (int mt = 0; mt < 4; ++mt) {
                const int mrow = grow + mt * 16, mcol = gcol;
                int lhf = 0, lfull = 0;
                for (int mg = 0; mg < 2; mg += 2)
                    for (int kg = 0; kg < 8; kg += 2)
                        for (int j = 0; j < 2; ++j)
                            for (int i = 0; i < 2; ++i) {
                                const int row0 = mrow + (mg + i) * 8, col0 = mcol + (kg + j) * 8;
                                uint64_t t1 = 0, t2 = 0, t3 = 0;
                                int thf = 0, tfull = 0;
                                for (int ro = 0; ro < 8; ++ro)
                                    for (int co = 0; co < 8; ++co) {
                                        const int pos = ro * 8 + co;
                                        const uint16_t bits = a[(int64_t)(row0 + ro) * K + col0 + co];
                                        const int exponent = (bits >> 7) & 0xFF;
                                        int idx = -1;
                                        for (int e = 0; e < 7; ++e)
                                            if (exponent == top[e]) { idx = e; break; }
                                        if (idx >= 0) {
                                            const int code = idx + 1;
                                            if (code & 1) t1 |= 1ULL << pos;
                                            if (code & 2) t2 |= 1ULL << pos;
                                            if (code & 4) t3 |= 1ULL << pos;
                                            out->sign_mantissa[sm_off++] =
                                                (uint8_t)((((bits >> 15) & 1) << 7) | (bits & 0x7F));
                                            ++thf; ++lhf; ++ghf;
                                        } else {
                                            out->compressed_full[full_off++] = bits;
                                            ++tfull; ++lfull; ++gfull;
                                        }
                                    }
                                out->bitmap1[tile_idx] = t1;
                                out->bitmap2[tile_idx] = t2;
                                out->bitmap3[tile_idx] = t3;
                                out->tile_offsets[tile_idx * 2] = thf;
                                out->tile_offsets[tile_idx * 2 + 1] = tfull;
                                ++tile_idx;
                            }
                if (mt < 3) {
                    mhf += lhf;
                    mfull += lfull;
                    out->tile_offsets_median[median_idx * 2] = mhf;
                    out->tile_offsets_median[median_idx * 2 + 1] = mfull;
                    ++median_idx;
                }
            }
            const int hpad = (16 - ghf % 16) % 16;
            for (int p = 0; p < hpad; ++p) out->sign_mantissa[sm_off++] = 0;
            ghf += hpad;
            const int fpad = (8 - gfull % 8) % 8;
            for (int p = 0; p < fpad; ++p) out->compressed_full[full_off++] = 0;
            gfull += fpad;
            g_hf[gm * gtk + gk + 1] = ghf;
            g_full[gm * gtk + gk + 1] = gfull;
            if (ghf > out->max_high_freq_count) out->max_high_freq_count = ghf;
            if (gfull > out->max_full_count) out->max_full_count = gfull;
        }
    }
    out->tile_offsets_global[0] = 0;
    out->tile_offsets_global[1] = 0;
    for (int i = 1; i <= ngt; ++i) {
        g_hf[i] += g_hf[i - 1];
        g_full[i] += g_full[i - 1];
        out->tile_offsets_global[i * 2] = (int32_t)g_hf[i];
        out->tile_offsets_global[i * 2 + 1] = (int32_t)g_full[i];
    }
    out->total_high_freq = sm_off;
    out->total_full = full_off;
    free(g_hf);
    free(g_full);
    return ngt;
}

/* Pass 2 + pass 3 shared by the two three-pass encoders
 * (csrc/L_API.cu:726-768 and :1020-1050). */
static void scan_and_scatter(int ngt, const uint8_t* temp_sm, const uint16_t* temp_full,
                             const int32_t* gt_hf, const int32_t* gt_full, zso_encoded* out) {
    int64_t hf = 0, fl = 0;
    out->max_high_freq_count = 0;
    out->max_full_count = 0;
    out->tile_offsets_global[0] = 0;
    out->tile_offsets_global[1] = 0;
    for (int i = 0; i < ngt; ++i) {
        memcpy(out->sign_mantissa + hf, temp_sm + (size_t)i * (4096 + 15), (size_t)gt_hf[i]);
        memcpy(out->compressed_full + fl, temp_full + (size_t)i * (4096 + 7),
               (size_t)gt_full[i] * sizeof(uint16_t));
        hf += gt_hf[i];
        fl += gt_full[i];
        out->tile_offsets_global[(i + 1) * 2] = (int32_t)hf;
        out->tile_offsets_global[(i + 1) * 2 + 1] = (int32_t)fl;
        if (gt_hf[i] > out->max_high_freq_count) out->max_high_freq_count = gt_hf[i];
        if (gt_full[i] > out->max_full_count) out->max_full_count = gt_full[i];
    }
    out->total_high_freq = hf;
    out->total_full = fl;
}

/* scan_and_scatter with the copies in parallel: the offsets (a serial scan
 * over the global tiles) first, then every tile's streams copied at once. */
static void scan_and_scatter_mt(int ngt, const uint8_t* temp_sm, const uint16_t* temp_full,
                                const int32_t* gt_hf, const int32_t* gt_full, zso_encoded* out,
                                int threads) {
    int64_t hf = 0, fl = 0;
    out->max_high_freq_count = 0;
    out->max_full_count = 0;
    out->tile_offsets_global[0] = 0;
    out->tile_offsets_global[1] = 0;
    for (int i = 0; i < ngt; ++i) {
        hf += gt_hf[i];
        fl += gt_full[i];
        out->tile_offsets_global[(i + 1) * 2] = (int32_t)hf;
        out->tile_offsets_global[(i + 1) * 2 + 1] = (int32_t)fl;
        if (gt_hf[i] > out->max_high_freq_count) out->max_high_freq_count = gt_hf[i];
        if (gt_full[i] > out->max_full_count) out->max_full_count = gt_full[i];
    }
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int i = 0; i < ngt; ++i) {
        memcpy(out->sign_mantissa + out->tile_offsets_global[2 * i],
               temp_sm + (size_t)i * (4096 + 15), (size_t)gt_hf[i]);
        memcpy(out->compressed_full + out->tile_offsets_global[2 * i + 1],
               temp_full + (size_t)i * (4096 + 7), (size_t)gt_full[i] * sizeof(uint16_t));
    }
    out->total_high_freq = hf;
    out->total_full = fl;
}

/* Median-offset bookkeeping of pass 1 (csrc/L_API.cu:692-716): after each
 * 16-small-tile median except the last, record the cumulative counts. */
static void median_step(int st, int thf, int tfull, int* cur_hf, int* cur_full, int* cum_hf,
                        int* cum_full, int32_t* med, int base_med, int* local_idx) {
    *cur_hf += thf;
    *cur_full += tfull;
    if (st % 16 == 15) {
        if (st / 16 < 3) {
            *cum_hf += *cur_hf;
            *cum_full += *cur_full;
            med[(base_med + *local_idx) * 2] = *cum_hf;
            med[(base_med + *local_idx) * 2 + 1] = *cum_full;
            ++*local_idx;
        }
        *cur_hf = 0;
        *cur_full = 0;
    }
}

/* csrc/L_API.cu:559-771: exponent -> index LUT, per-GT temp streams, then a
 * prefix scan and memcpy scatter. */
int zso_compress_lut(const uint16_t* a, int M, int K, const int top[7], zso_encoded* out) {
    if (check_dims(M, K)) return -1;
    init_tile_pos();
    const int gtk = K / 64, ngt = (M / 64) * gtk;
    uint8_t lut[256];
    memset(lut, 0xFF, sizeof(lut));
    for (int e = 0; e < 7; ++e) lut[top[e] & 0xFF] = (uint8_t)e;
    uint8_t* temp_sm = (uint8_t*)malloc((size_t)ngt * (4096 + 15));
    uint16_t* temp_full = (uint16_t*)malloc((size_t)ngt * (4096 + 7) * sizeof(uint16_t));
    int32_t* gt_hf = (int32_t*)malloc((size_t)ngt * sizeof(int32_t));
    int32_t* gt_full = (int32_t*)malloc((size_t)ngt * sizeof(int32_t));
    if (!temp_sm || !temp_full || !gt_hf || !gt_full) {
        free(temp_sm); free(temp_full); free(gt_hf); free(gt_full);
        return -1;
    }
    for (int gt = 0; gt < ngt; ++gt) {
        const int grow = (gt / gtk) * 64, gcol = (gt % gtk) * 64;
        uint8_t* my_sm = temp_sm + (size_t)gt * (4096 + 15);
        uint16_t* my_full = temp_full + (size_t)gt * (4096 + 7);
        int si = 0, fi = 0, cur_hf = 0, cur_full = 0, cum_hf = 0, cum_full = 0, local = 1;
        out->tile_offsets_median[gt * 4 * 2] = 0;
        out->tile_offsets_median[gt * 4 * 2 + 1] = 0;
        for (int st = 0; st < 64; ++st) {
            const int r0 = grow + g_pos_row[st], c0 = gcol + g_pos_col[st];
            uint64_t t1 = 0, t2 = 0, t3 = 0;
            int thf = 0, tfull = 0;
            for (int ro = 0; ro < 8; ++ro) {
                const uint16_t* rp = a + (int64_t)(r0 + ro) * K + c0;
                for (int co = 0; co < 8; ++co) {
                    const int pos = ro * 8 + co;
                    const uint16_t bits = rp[co];
                    const uint8_t idx = lut[(bits >> 7) & 0xFF];
                    if (idx != 0xFF) {
                        const int code = idx + 1;
                        t1 |= (uint64_t)(code & 1) << pos;
                        t2 |= (uint64_t)((code >> 1) & 1) << pos;
                        t3 |= (uint64_t)((code >> 2) & 1) << pos;
                        my_sm[si++] = (uint8_t)(((bits >> 8) & 0x80) | (bits & 0x7F));
                        ++thf;
                    } else {
                        my_full[fi++] = bits;
                        ++tfull;
                    }
                }
            }
            const int tidx = gt * 64 + st;
            out->bitmap1[tidx] = t1;
            out->bitmap2[tidx] = t2;
            out->bitmap3[tidx] = t3;
            out->tile_offsets[tidx * 2] = thf;
            out->tile_offsets[tidx * 2 + 1] = tfull;
            median_step(st, thf, tfull, &cur_hf, &cur_full, &cum_hf, &cum_full,
                        out->tile_offsets_median, gt * 4, &local);
        }
        while (si % 16) my_sm[si++] = 0;
        while (fi % 8) my_full[fi++] = 0;
        gt_hf[gt] = si;
        gt_full[gt] = fi;
    }
    scan_and_scatter(ngt, temp_sm, temp_full, gt_hf, gt_full, out);
    free(temp_sm); free(temp_full); free(gt_hf); free(gt_full);
    return ngt;
}

/* csrc/L_API.cu:773-1053: one 8-element tile row per SSE step.  The window is
 * taken as [top[0], top[0]+6] (:851-852); the hf mask comes from two signed
 * compares, bit-planes from movemask, sign/mantissa bytes are left-packed with
 * a pshufb table built as at :780-795, outliers are scattered in ascending
 * position order. */
static __m128i g_compress_lut[256];
static int g_compress_lut_ready = 0;

static void init_compress_lut(void) {
    if (g_compress_lut_ready) return;
    for (int mask = 0; mask < 256; ++mask) {
        uint8_t idx[16];
        int p = 0;
        for (int b = 0; b < 8; ++b)
            if (mask & (1 << b)) idx[p++] = (uint8_t)b;
        for (int i = p; i < 16; ++i) idx[i] = 0x80;
        g_compress_lut[mask] = _mm_loadu_si128((const __m128i*)idx);
    }
    g_compress_lut_ready = 1;
}

static int compress_sse_impl(const uint16_t* a, int M, int K, const int top[7], zso_encoded* out,
                             int threads);

int zso_compress_sse(const uint16_t* a, int M, int K, const int top[7], zso_encoded* out) {
    return compress_sse_impl(a, M, K, top, out, 1);
}

/* zso_compress_sse with pass 1 (per global tile, independent) and the pass-3
 * copies spread over `threads` OpenMP threads (<= 0: all), as the
 * reference's multi-threaded compress benchmarks parallelise over tiles
 * (kernel_benchmark/README.md:255-257,
 * bench_kv_cache_zipserv_compress_scaling.cu:681).  Same bytes. */
int zso_compress_sse_mt(const uint16_t* a, int M, int K, const int top[7], zso_encoded* out,
                        int threads) {
    return compress_sse_impl(a, M, K, top, out, threads <= 0 ? omp_get_max_threads() : threads);
}

static int compress_sse_impl(const uint16_t* a, int M, int K, const int top[7], zso_encoded* out,
                             int threads) {
    if (check_dims(M, K)) return -1;
    init_tile_pos();
    init_compress_lut();
    const int gtk = K / 64, ngt = (M / 64) * gtk;
    uint8_t* temp_sm = (uint8_t*)malloc((size_t)ngt * (4096 + 15) + 16);
    uint16_t* temp_full = (uint16_t*)malloc((size_t)ngt * (4096 + 7) * sizeof(uint16_t));
    int32_t* gt_hf = (int32_t*)malloc((size_t)ngt * sizeof(int32_t));
    int32_t* gt_full = (int32_t*)malloc((size_t)ngt * sizeof(int32_t));
    if (!temp_sm || !temp_full || !gt_hf || !gt_full) {
        free(temp_sm); free(temp_full); free(gt_hf); free(gt_full);
        return -1;
    }
    const __m128i v_start = _mm_set1_epi16((short)top[0]);
    const __m128i v_seven = _mm_set1_epi16(7), v_neg1 = _mm_set1_epi16(-1);
    const __m128i v_one = _mm_set1_epi16(1), v_ff = _mm_set1_epi16(0xFF);
    const __m128i v_80 = _mm_set1_epi16(0x80), v_7f = _mm_set1_epi16(0x7F);
    const __m128i v_zero = _mm_setzero_si128();
#pragma omp parallel for schedule(static) num_threads(threads) if (threads > 1)
    for (int gt = 0; gt < ngt; ++gt) {
        const int grow = (gt / gtk) * 64, gcol = (gt % gtk) * 64;
        uint8_t* my_sm = temp_sm + (size_t)gt * (4096 + 15);
        uint16_t* my_full = temp_full + (size_t)gt * (4096 + 7);
        int si = 0, fi = 0, cur_hf = 0, cur_full = 0, cum_hf = 0, cum_full = 0, local = 1;
        out->tile_offsets_median[gt * 4 * 2] = 0;
        out->tile_offsets_median[gt * 4 * 2 + 1] = 0;
        for (int st = 0; st < 64; ++st) {
            const int r0 = grow + g_pos_row[st], c0 = gcol + g_pos_col[st];
            uint64_t t1 = 0, t2 = 0, t3 = 0;
            int thf = 0, tfull = 0;
            for (int ro = 0; ro < 8; ++ro) {
                const __m128i bits = _mm_loadu_si128((const __m128i*)(a + (int64_t)(r0 + ro) * K + c0));
                const __m128i ex = _mm_and_si128(_mm_srli_epi16(bits, 7), v_ff);
                const __m128i sub = _mm_sub_epi16(ex, v_start);
                const __m128i is_hf = _mm_and_si128(_mm_cmpgt_epi16(sub, v_neg1), _mm_cmpgt_epi16(v_seven, sub));
                const int hf_mask = _mm_movemask_epi8(_mm_packs_epi16(is_hf, v_zero)) & 0xFF;
                const __m128i code = _mm_and_si128(_mm_add_epi16(sub, v_one), is_hf);
                const int m1 = _mm_movemask_epi8(_mm_packs_epi16(
                                   _mm_cmpeq_epi16(_mm_and_si128(code, v_one), v_one), v_zero)) & 0xFF;
                const int m2 = _mm_movemask_epi8(_mm_packs_epi16(
                                   _mm_cmpeq_epi16(_mm_and_si128(_mm_srli_epi16(code, 1), v_one), v_one),
                                   v_zero)) & 0xFF;
                const int m3 = _mm_movemask_epi8(_mm_packs_epi16(
                                   _mm_cmpeq_epi16(_mm_and_si128(_mm_srli_epi16(code, 2), v_one), v_one),
                                   v_zero)) & 0xFF;
                t1 |= (uint64_t)m1 << (ro * 8);
                t2 |= (uint64_t)m2 << (ro * 8);
                t3 |= (uint64_t)m3 << (ro * 8);
                const __m128i sm16 = _mm_or_si128(_mm_and_si128(_mm_srli_epi16(bits, 8), v_80),
                                                  _mm_and_si128(bits, v_7f));
                const __m128i packed = _mm_shuffle_epi8(_mm_packus_epi16(sm16, v_zero), g_compress_lut[hf_mask]);
                _mm_storel_epi64((__m128i*)(my_sm + si), packed);
                const int n = __builtin_popcount((unsigned)hf_mask);
                si += n;
                thf += n;
                int fm = (~hf_mask) & 0xFF;
                if (fm) {
                    uint16_t rv[8];
                    _mm_storeu_si128((__m128i*)rv, bits);
                    while (fm) {
                        const int b = __builtin_ctz((unsigned)fm);
                        my_full[fi++] = rv[b];
                        ++tfull;
                        fm &= fm - 1;
                    }
                }
            }
            const int tidx = gt * 64 + st;
            out->bitmap1[tidx] = t1;
            out->bitmap2[tidx] = t2;
            out->bitmap3[tidx] = t3;
            out->tile_offsets[tidx * 2] = thf;
            out->tile_offsets[tidx * 2 + 1] = tfull;
            median_step(st, thf, tfull, &cur_hf, &cur_full, &cum_hf, &cum_full,
                        out->tile_offsets_median, gt * 4, &local);
        }
        while (si % 16) my_sm[si++] = 0;
        while (fi % 8) my_full[fi++] = 0;
        gt_hf[gt] = si;
        gt_full[gt] = fi;
    }
    if (threads > 1) {
        scan_and_scatter_mt(ngt, temp_sm, temp_full, gt_hf, gt_full, out, threads);
    } else {
        scan_and_scatter(ngt, temp_sm, temp_full, gt_hf, gt_full, out);
    }
    free(temp_sm); free(temp_full); free(gt_hf); free(gt_full);
    return ngt;
}

/* ------------------------------------------------------------------------ */
/* CPU decoder: bench_kv_cache_zipserv_decompress_token_scaling.cu:2106-2218 */
/* Walks each global tile's streams sequentially from its global offsets;   */
/* the exponent is (start_exp + code) mod 256 (:2193-2194).                 */
/* ------------------------------------------------------------------------ */
int zso_decompress(const uint8_t* sm, int64_t sm_len, const uint16_t* full, int64_t full_len,
                   const uint64_t* b1, const uint64_t* b2, const uint64_t* b3,
                   const int32_t* tog, int M, int K, int start_exp, uint16_t* out) {
    if (check_dims(M, K)) return -1;
    init_tile_pos();
    const int gtk = K / 64, ngt = (M / 64) * gtk;
    for (int g = 0; g < ngt; ++g) {
        int64_t hi = tog[g * 2], fi = tog[g * 2 + 1];
        const int grow = (g / gtk) * 64, gcol = (g % gtk) * 64;
        for (int st = 0; st < 64; ++st) {
            const int64_t t = (int64_t)g * 64 + st;
            const uint64_t w1 = b1[t], w2 = b2[t], w3 = b3[t], ind = w1 | w2 | w3;
            const int r0 = grow + g_pos_row[st], c0 = gcol + g_pos_col[st];
            for (int pos = 0; pos < 64; ++pos) {
                const int64_t o = (int64_t)(r0 + pos / 8) * K + c0 + pos % 8;
                if ((ind >> pos) & 1) {
                    if (hi < 0 || hi >= sm_len) return -1;
                    const uint8_t c = sm[hi++];
                    const int code = (int)(((w3 >> pos) & 1) << 2 | ((w2 >> pos) & 1) << 1 | ((w1 >> pos) & 1));
                    const uint8_t e = (uint8_t)(start_exp + code);
                    out[o] = (uint16_t)(((c >> 7) & 1) << 15 | (uint16_t)e << 7 | (c & 0x7F));
                } else {
                    if (fi < 0 || fi >= full_len) return -1;
                    out[o] = full[fi++];
                }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* GEMM references                                                          */
/* ------------------------------------------------------------------------ */
void zso_gemm_f32(const uint16_t* W, const uint16_t* X, int M, int N, int K, float* Y) {
    float* xr = (float*)malloc((size_t)K * sizeof(float));
    float* wr = (float*)malloc((size_t)K * sizeof(float));
    for (int n = 0; n < N; ++n) {
        for (int k = 0; k < K; ++k) xr[k] = zso_bf16_to_f32(X[(int64_t)n * K + k]);
        for (int m = 0; m < M; ++m) {
            const uint16_t* w = W + (int64_t)m * K;
            for (int k = 0; k < K; ++k) wr[k] = zso_bf16_to_f32(w[k]);
            float acc = 0.f;
            for (int k = 0; k < K; ++k) acc += wr[k] * xr[k];
            Y[(int64_t)n * M + m] = acc;
        }
    }
    free(xr);
    free(wr);
}

/* CPU baseline variants (same arithmetic, same summation order per output):
 * the decoder parallel over global tiles, and a GEMM that widens each W row
 * once and reuses it for all N columns, parallel over rows of W.  `threads`
 * <= 0 uses every core OpenMP sees. */
int zso_decompress_mt(const uint8_t* sm, int64_t sm_len, const uint16_t* full, int64_t full_len,
                      const uint64_t* b1, const uint64_t* b2, const uint64_t* b3,
                      const int32_t* tog, int M, int K, int start_exp, uint16_t* out,
                      int threads) {
    if (check_dims(M, K)) return -1;
    init_tile_pos();
    const int gtk = K / 64, ngt = (M / 64) * gtk;
    int bad = 0;
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for num_threads(threads) schedule(static) reduction(| : bad)
    for (int g = 0; g < ngt; ++g) {
        int64_t hi = tog[g * 2], fi = tog[g * 2 + 1];
        const int grow = (g / gtk) * 64, gcol = (g % gtk) * 64;
        for (int st = 0; st < 64 && !bad; ++st) {
            const int64_t t = (int64_t)g * 64 + st;
            const uint64_t w1 = b1[t], w2 = b2[t], w3 = b3[t], ind = w1 | w2 | w3;
            const int r0 = grow + g_pos_row[st], c0 = gcol + g_pos_col[st];
            for (int pos = 0; pos < 64; ++pos) {
                const int64_t o = (int64_t)(r0 + pos / 8) * K + c0 + pos % 8;
                if ((ind >> pos) & 1) {
                    if (hi < 0 || hi >= sm_len) { bad = 1; break; }
                    const uint8_t c = sm[hi++];
                    const int code = (int)(((w3 >> pos) & 1) << 2 | ((w2 >> pos) & 1) << 1 | ((w1 >> pos) & 1));
                    const uint8_t e = (uint8_t)(start_exp + code);
                    out[o] = (uint16_t)(((c >> 7) & 1) << 15 | (uint16_t)e << 7 | (c & 0x7F));
                } else {
                    if (fi < 0 || fi >= full_len) { bad = 1; break; }
                    out[o] = full[fi++];
                }
            }
        }
    }
    return bad ? -1 : 0;
}

void zso_gemm_f32_mt(const uint16_t* W, const uint16_t* X, int M, int N, int K, float* Y,
                     int threads) {
    float* xf = (float*)malloc((size_t)N * K * sizeof(float));
    for (int64_t i = 0; i < (int64_t)N * K; ++i) xf[i] = zso_bf16_to_f32(X[i]);
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel num_threads(threads)
    {
        float* wr = (float*)malloc((size_t)K * sizeof(float));
#pragma omp for schedule(static)
        for (int m = 0; m < M; ++m) {
            const uint16_t* w = W + (int64_t)m * K;
            for (int k = 0; k < K; ++k) wr[k] = zso_bf16_to_f32(w[k]);
            for (int n = 0; n < N; ++n) {
                const float* xr = xf + (int64_t)n * K;
                float acc = 0.f;
                for (int k = 0; k < K; ++k) acc += wr[k] * xr[k];
                Y[(int64_t)n * M + m] = acc;
            }
        }
        free(wr);
    }
    free(xf);
}

void zso_gemm_splitk_bf16(const uint16_t* W, const uint16_t* X, int M, int N, int K, int S,
                          uint16_t* Y) {
    const int nk = K / 64;
    const int avg = (nk - 1) / S + 1;
    for (int n = 0; n < N; ++n)
        for (int m = 0; m < M; ++m) {
            float total = 0.f;
            for (int s = 0; s < S; ++s) {
                int kb0 = s * avg, kb1 = kb0 + avg;
                if (kb1 > nk) kb1 = nk;
                float part = 0.f;
                for (int k = kb0 * 64; k < kb1 * 64; ++k)
                    part += zso_bf16_to_f32(W[(int64_t)m * K + k]) * zso_bf16_to_f32(X[(int64_t)n * K + k]);
                total += zso_bf16_to_f32(zso_f32_to_bf16(part));
            }
            Y[(int64_t)n * M + m] = zso_f32_to_bf16(total);
        }
}

/* ------------------------------------------------------------------------ */
/* Decode attention, fp64                                                   */
/* ------------------------------------------------------------------------ */
void zso_decode_attention_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, int B, int H,
                              int Hkv, int T, int D, const int32_t* seqlens, double scale,
                              double* out, double* lse) {
    zso_decode_attention_absv_f64(q, k, v, B, H, Hkv, T, D, seqlens, scale, out, lse, NULL);
}

/* As zso_decode_attention_f64, plus absv[b][h][d] = sum_t p_t |v_t,d| with
 * the softmax weights p_t (when absv is not NULL): the scale of the error
 * that rounding the weights to bf16 before the P.V product can cause
 * (|error| <= 2^-8 * absv for bf16's unit roundoff 2^-8). */
void zso_decode_attention_absv_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, int B,
                                   int H, int Hkv, int T, int D, const int32_t* seqlens,
                                   double scale, double* out, double* lse, double* absv) {
    const int G = H / Hkv;
    double* s = (double*)malloc((size_t)(T > 0 ? T : 1) * sizeof(double));
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const int kh = h / G, L = seqlens ? seqlens[b] : T;
            const uint16_t* qp = q + ((int64_t)b * H + h) * D;
            double mx = -INFINITY;
            for (int t = 0; t < L; ++t) {
                const uint16_t* kp = k + (((int64_t)b * T + t) * Hkv + kh) * D;
                double acc = 0.0;
                for (int d = 0; d < D; ++d) acc += (double)zso_bf16_to_f32(qp[d]) * zso_bf16_to_f32(kp[d]);
                s[t] = acc * scale;
                if (s[t] > mx) mx = s[t];
            }
            double* op = out + ((int64_t)b * H + h) * D;
            double* ap = absv ? absv + ((int64_t)b * H + h) * D : NULL;
            for (int d = 0; d < D; ++d) op[d] = 0.0;
            if (ap) for (int d = 0; d < D; ++d) ap[d] = 0.0;
            if (L <= 0) { lse[(int64_t)b * H + h] = -INFINITY; continue; }
            double den = 0.0;
            for (int t = 0; t < L; ++t) {
                const double p = exp(s[t] - mx);
                den += p;
                const uint16_t* vp = v + (((int64_t)b * T + t) * Hkv + kh) * D;
                for (int d = 0; d < D; ++d) op[d] += p * zso_bf16_to_f32(vp[d]);
                if (ap) for (int d = 0; d < D; ++d) ap[d] += p * fabs((double)zso_bf16_to_f32(vp[d]));
            }
            for (int d = 0; d < D; ++d) op[d] /= den;
            if (ap) for (int d = 0; d < D; ++d) ap[d] /= den;
            lse[(int64_t)b * H + h] = mx + log(den);
        }
    free(s);
}

/* ------------------------------------------------------------------------ */
/* Re-tiled device layout (see zs_oracle.h).                                 */
/* ------------------------------------------------------------------------ */
static inline int64_t zso_rec_elem(int M, int K, int64_t r, int h, int l, int i, int* row, int* col) {
    const int KT = K / 64;
    const int64_t band = r / KT, kt = r % KT;
    (void)M;
    *row = (int)(band * 16 + (l & 15));
    *col = (int)(kt * 64 + 32 * h + 8 * (l >> 4) + i);
    return (int64_t)(*row) * K + *col;
}

int64_t zso_compress_retiled(const uint16_t* a, int M, int K, int start_exp, uint8_t* fixed,
                             uint8_t* exps, int32_t* eoff) {
    const int64_t nrec = (int64_t)(M / 16) * (K / 64);
    int64_t nout = 0;
    const unsigned st = (unsigned)start_exp & 0xFFu;
    eoff[0] = 0;
    for (int64_t r = 0; r < nrec; ++r) {
        uint8_t* f = fixed + r * ZSO_REC_BYTES;
        uint32_t C[64][2];
        memset(C, 0, sizeof(C));
        for (int h = 0; h < 2; ++h)          /* outliers in (h, l, i) order */
            for (int l = 0; l < 64; ++l)
                for (int i = 0; i < 8; ++i) {
                    int row, col, prow, pcol;
                    const uint16_t v = a[zso_rec_elem(M, K, r, h, l, i, &row, &col)];
                    const uint16_t vp = a[zso_rec_elem(M, K, r, h, l, i ^ 1, &prow, &pcol)];
                    const unsigned e = (v >> 7) & 0xFFu;
                    const unsigned d = (e - st) & 0xFFu;
                    const unsigned code = (d >= 1 && d <= 7) ? d : 0;
                    /* mantissa << 1 | sign of the pair partner (element i ^ 1) */
                    f[16 * l + 8 * h + i] = (uint8_t)(((v & 0x7Fu) << 1) | ((vp >> 15) & 1u));
                    C[l][h] |= (uint32_t)code << (3 * i);
                    if (code == 0) exps[nout++] = (uint8_t)e;
                }
        for (int l = 0; l < 64; ++l) {
            const uint32_t w32 = C[l][0] | (C[l][1] << 24);
            const uint16_t w16 = (uint16_t)(C[l][1] >> 8);
            memcpy(f + 1024 + 4 * l, &w32, 4);
            memcpy(f + 1280 + 2 * l, &w16, 2);
        }
        eoff[r + 1] = (int32_t)nout;
    }
    return nout;
}

void zso_decompress_retiled(const uint8_t* fixed, const uint8_t* exps, const int32_t* eoff,
                            int start_exp, int M, int K, uint16_t* out) {
    const int64_t nrec = (int64_t)(M / 16) * (K / 64);
    const unsigned st = (unsigned)start_exp & 0xFFu;
    for (int64_t r = 0; r < nrec; ++r) {
        const uint8_t* f = fixed + r * ZSO_REC_BYTES;
        int64_t k = eoff[r];
        for (int h = 0; h < 2; ++h)
            for (int l = 0; l < 64; ++l) {
                uint32_t w32;
                uint16_t w16;
                memcpy(&w32, f + 1024 + 4 * l, 4);
                memcpy(&w16, f + 1280 + 2 * l, 2);
                const uint32_t c = h ? ((w32 >> 24) | ((uint32_t)w16 << 8)) : (w32 & 0xFFFFFFu);
                for (int i = 0; i < 8; ++i) {
                    const unsigned code = (c >> (3 * i)) & 7u;
                    const unsigned e = code ? ((st + code) & 0xFFu) : exps[k++];
                    const unsigned s = f[16 * l + 8 * h + i];            /* own mantissa */
                    const unsigned sp = f[16 * l + 8 * h + (i ^ 1)];     /* holds own sign */
                    int row, col;
                    out[zso_rec_elem(M, K, r, h, l, i, &row, &col)] =
                        (uint16_t)(((sp & 1u) << 15) | (e << 7) | (s >> 1));
                }
            }
    }
}
