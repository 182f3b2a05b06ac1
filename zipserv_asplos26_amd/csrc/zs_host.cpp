// zs_host.cpp -- host side of libzipserv: status strings, size queries,
// exponent-window analysis and the CPU TCA-TBE encoders.
//
// The encoders walk each 64x64 global tile as 8 "half median tiles"
// (16 rows x 32 columns) and, inside each, the 64 small-tile rows in
// canonical stream order (row index l -> matrix row l%16, columns
// 8*(l/16)..+7).  That order is the order in which csrc/L_API.cu:403-428
// appends elements (small tiles 2x2-grouped column-major, rows row-major), so
// the emitted bytes are the canonical format; it is also the lane order the
// gfx950 decoder uses, which keeps the host and device views identical.
#include <immintrin.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "../../include/zipserv.h"

namespace {

constexpr int kSmStride = 4096 + 15;   // per-GT temp SM capacity (L_API.cu:600)
constexpr int kFullStride = 4096 + 7;  // per-GT temp FULL capacity

bool tiles_ok(int tM, int tMm, int tMg, int tK, int tKm, int tKg) {
  return tM == 8 && tMm == 16 && tMg == 64 && tK == 8 && tKm == 64 && tKg == 64;
}

int check_shape(int M, int K) {
  if (M <= 0 || K <= 0 || (M % 64) || (K % 64)) return ZS_E_INVAL;
  const int64_t mk = (int64_t)M * K;
  // Every stream offset must fit the int32 TileOffsets of the format.
  const int64_t ngt = mk / 4096;
  if (mk + 16 * ngt > INT32_MAX) return ZS_E_OVERFLOW;
  return ZS_OK;
}

// Exponent -> code (1..7), 0 = outlier.
struct CodeTable {
  uint8_t code[256];
  // first_match: a repeated exponent keeps its first index, as the linear
  // search of L_API.cu:447-453 does; otherwise the last one wins, as the index
  // LUT of L_API.cu:603-606 does.  Values outside 0..255 never match.
  CodeTable(const int32_t* top, bool first_match) {
    memset(code, 0, sizeof(code));
    for (int k = 0; k < 7; ++k) {
      const int i = first_match ? 6 - k : k;
      if (top[i] >= 0 && top[i] <= 255) code[top[i]] = (uint8_t)(i + 1);
    }
  }
};

// Left-packing shuffles: entry[mask] moves the bytes whose bit is set in
// `mask` to the front (zero elsewhere).
struct PackTable {
  __m128i shuf[256];
  PackTable() {
    for (int m = 0; m < 256; ++m) {
      alignas(16) uint8_t b[16];
      int p = 0;
      for (int j = 0; j < 8; ++j)
        if (m & (1 << j)) b[p++] = (uint8_t)j;
      while (p < 16) b[p++] = 0x80;
      shuf[m] = _mm_load_si128(reinterpret_cast<const __m128i*>(b));
    }
  }
};

const PackTable& pack_table() {
  static const PackTable t;  // thread-safe one-time init (C++11 magic static)
  return t;
}

// Output cursors of one global tile.
struct GtOut {
  uint8_t* sm;     // per-GT SM staging
  uint16_t* full;  // per-GT FULL staging
  uint8_t* bm1;    // bitmap planes as bytes, already offset to this GT
  uint8_t* bm2;
  uint8_t* bm3;
  int32_t* tiles;   // small-tile (hf, full) pairs of this GT (64 pairs)
  int32_t* median;  // 4 median (hf, full) start pairs of this GT
};

// Encodes one 8-element small-tile row.  Returns the number of in-window
// elements; writes the three bitmap bytes.
template <bool kRange>
inline int encode_row(const uint16_t* src, const CodeTable& ct, int start, uint8_t* sm,
                      uint16_t* full, int* nfull, uint8_t* b1, uint8_t* b2, uint8_t* b3) {
  if (kRange) {
    const __m128i v = _mm_loadu_si128(reinterpret_cast<const __m128i*>(src));
    const __m128i ex = _mm_and_si128(_mm_srli_epi16(v, 7), _mm_set1_epi16(0xFF));
    const __m128i c = _mm_add_epi16(_mm_sub_epi16(ex, _mm_set1_epi16((short)start)),
                                    _mm_set1_epi16(1));  // 1..7 in window
    const __m128i inwin = _mm_and_si128(_mm_cmpgt_epi16(c, _mm_setzero_si128()),
                                        _mm_cmplt_epi16(c, _mm_set1_epi16(8)));
    const __m128i code = _mm_and_si128(c, inwin);
    // Bit planes: shift each code bit into the sign bit of its byte.
    const __m128i p1 = _mm_packs_epi16(_mm_slli_epi16(code, 15), _mm_setzero_si128());
    const __m128i p2 = _mm_packs_epi16(_mm_slli_epi16(code, 14), _mm_setzero_si128());
    const __m128i p3 = _mm_packs_epi16(_mm_slli_epi16(code, 13), _mm_setzero_si128());
    *b1 = (uint8_t)_mm_movemask_epi8(p1);
    *b2 = (uint8_t)_mm_movemask_epi8(p2);
    *b3 = (uint8_t)_mm_movemask_epi8(p3);
    const int mask = _mm_movemask_epi8(_mm_packs_epi16(inwin, _mm_setzero_si128())) & 0xFF;
    // sign|mantissa byte = (hi byte & 0x80) | (lo byte & 0x7F)
    const __m128i smw = _mm_or_si128(_mm_and_si128(_mm_srli_epi16(v, 8), _mm_set1_epi16(0x80)),
                                     _mm_and_si128(v, _mm_set1_epi16(0x7F)));
    const __m128i packed =
        _mm_shuffle_epi8(_mm_packus_epi16(smw, _mm_setzero_si128()), pack_table().shuf[mask]);
    _mm_storel_epi64(reinterpret_cast<__m128i*>(sm), packed);
    int om = (~mask) & 0xFF;
    while (om) {
      const int j = __builtin_ctz(om);
      full[(*nfull)++] = src[j];
      om &= om - 1;
    }
    return __builtin_popcount(mask);
  } else {
    uint32_t x1 = 0, x2 = 0, x3 = 0;
    int n = 0;
    for (int j = 0; j < 8; ++j) {
      const uint16_t bits = src[j];
      const uint32_t c = ct.code[(bits >> 7) & 0xFF];
      if (c) {
        x1 |= (c & 1u) << j;
        x2 |= ((c >> 1) & 1u) << j;
        x3 |= ((c >> 2) & 1u) << j;
        sm[n++] = (uint8_t)(((bits >> 8) & 0x80) | (bits & 0x7F));
      } else {
        full[(*nfull)++] = bits;
      }
    }
    *b1 = (uint8_t)x1;
    *b2 = (uint8_t)x2;
    *b3 = (uint8_t)x3;
    return n;
  }
}

// Encodes global tile (gm, gk) into per-GT staging; returns padded counts.
template <bool kRange>
void encode_gt(const uint16_t* A, int K, int gm, int gk, const CodeTable& ct, int start,
               const GtOut& o, int* sm_count, int* full_count) {
  int sm = 0, fu = 0;
  for (int m = 0; m < 4; ++m) {
    o.median[2 * m] = sm;
    o.median[2 * m + 1] = fu;
    for (int h = 0; h < 2; ++h) {
      for (int st = 0; st < 8; ++st) {  // 8 small tiles of the half median tile
        int t_hf = 0, t_full = 0;
        for (int rr = 0; rr < 8; ++rr) {
          const int l = st * 8 + rr;  // stream-order row index
          const int row = gm * 64 + m * 16 + (l & 15);
          const int col = gk * 64 + h * 32 + 8 * (l >> 4);
          const int bidx = m * 128 + h * 64 + l;
          const int before = fu;
          const int n = encode_row<kRange>(A + (int64_t)row * K + col, ct, start, o.sm + sm,
                                           o.full, &fu, o.bm1 + bidx, o.bm2 + bidx, o.bm3 + bidx);
          sm += n;
          t_hf += n;
          t_full += fu - before;
        }
        const int t = m * 16 + h * 8 + st;
        o.tiles[2 * t] = t_hf;
        o.tiles[2 * t + 1] = t_full;
      }
    }
  }
  while (sm % 16) o.sm[sm++] = 0;
  while (fu % 8) o.full[fu++] = 0;
  *sm_count = sm;
  *full_count = fu;
}

struct Outputs {
  uint8_t* sm;
  uint16_t* full;
  uint64_t* b1;
  uint64_t* b2;
  uint64_t* b3;
  int32_t* tiles;
  int32_t* median;
  int32_t* global;
};

struct Temps {
  uint8_t* sm;
  uint16_t* full;
  int32_t* gt_hf;
  int32_t* gt_full;
  int32_t* hf_off;
  int32_t* full_off;
};

// Pass 1 (per-GT staging), pass 2 (scan), pass 3 (scatter).
template <bool kRange>
int encode_matrix(const uint16_t* A, int M, int K, const int32_t* top, bool first_match,
                  const Outputs& out, const Temps& tmp, int32_t* max_hf, int32_t* max_full,
                  int32_t* total_hf, int32_t* total_full) {
  const int gtm = M / 64, gtk = K / 64, ngt = gtm * gtk;
  const CodeTable ct(top, first_match);
  const int start = top[0];
  for (int g = 0; g < ngt; ++g) {
    GtOut o;
    o.sm = tmp.sm + (size_t)g * kSmStride;
    o.full = tmp.full + (size_t)g * kFullStride;
    o.bm1 = reinterpret_cast<uint8_t*>(out.b1 + (size_t)g * 64);
    o.bm2 = reinterpret_cast<uint8_t*>(out.b2 + (size_t)g * 64);
    o.bm3 = reinterpret_cast<uint8_t*>(out.b3 + (size_t)g * 64);
    o.tiles = out.tiles + (size_t)g * 128;
    o.median = out.median + (size_t)g * 8;
    encode_gt<kRange>(A, K, g / gtk, g % gtk, ct, start, o, &tmp.gt_hf[g], &tmp.gt_full[g]);
  }
  int64_t hf = 0, fu = 0;
  int32_t mh = 0, mf = 0;
  tmp.hf_off[0] = 0;
  tmp.full_off[0] = 0;
  out.global[0] = 0;
  out.global[1] = 0;
  for (int g = 0; g < ngt; ++g) {
    memcpy(out.sm + hf, tmp.sm + (size_t)g * kSmStride, (size_t)tmp.gt_hf[g]);
    memcpy(out.full + fu, tmp.full + (size_t)g * kFullStride, (size_t)tmp.gt_full[g] * 2);
    hf += tmp.gt_hf[g];
    fu += tmp.gt_full[g];
    mh = std::max(mh, tmp.gt_hf[g]);
    mf = std::max(mf, tmp.gt_full[g]);
    tmp.hf_off[g + 1] = (int32_t)hf;
    tmp.full_off[g + 1] = (int32_t)fu;
    out.global[2 * (g + 1)] = (int32_t)hf;
    out.global[2 * (g + 1) + 1] = (int32_t)fu;
  }
  if (max_hf) *max_hf = mh;
  if (max_full) *max_full = mf;
  if (total_hf) *total_hf = (int32_t)hf;
  if (total_full) *total_full = (int32_t)fu;
  return ngt;
}

// Window selection of kernel_benchmark/utils.h:189-272: the 7 most frequent
// exponents (count > 0, ties to the lower exponent), missing ones filled with
// 127-n; then the first candidate (ascending) that starts 7 all-present
// exponents, else the start of the longest consecutive candidate run.
void select_window_cpu(const int64_t* counts, int32_t* top) {
  std::vector<int> order;
  for (int e = 0; e < 256; ++e)
    if (counts[e] > 0) order.push_back(e);
  std::stable_sort(order.begin(), order.end(),
                   [&](int a, int b) { return counts[a] > counts[b]; });
  int cand[7];
  int n = 0;
  for (; n < 7 && n < (int)order.size(); ++n) cand[n] = order[n];
  for (; n < 7; ++n) cand[n] = 127 - n;
  std::sort(cand, cand + 7);
  for (int c = 0; c < 7; ++c) {
    const int s = cand[c];
    if (s < 0 || s + 6 > 255) continue;
    bool all = true;
    for (int i = 0; i < 7 && all; ++i) all = counts[s + i] > 0;
    if (all) {
      for (int i = 0; i < 7; ++i) top[i] = s + i;
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
  for (int i = 0; i < 7; ++i) top[i] = best + i;
}

}  // namespace

extern "C" {

const char* zs_version(void) { return "zipserv-mi355x 0.1 (gfx950)"; }

const char* zs_status_string(int s) {
  switch (s) {
    case ZS_OK: return "ok";
    case ZS_E_INVAL: return "invalid argument";
    case ZS_E_UNSUPPORTED: return "unsupported";
    case ZS_E_OVERFLOW: return "offsets overflow int32";
    case ZS_E_NOMEM: return "out of host memory";
    default: return s > 0 ? "hip runtime error" : "unknown status";
  }
}

int64_t zs_num_global_tiles(int M, int K) {
  if (M <= 0 || K <= 0) return 0;
  return (int64_t)(M / 64) * (K / 64);
}

int64_t zs_sign_mantissa_capacity(int M, int K) {
  return (int64_t)M * K + 16 * zs_num_global_tiles(M, K) + ZS_STREAM_SLACK_BYTES;
}

int64_t zs_full_capacity(int M, int K) {
  return (int64_t)M * K + 8 * zs_num_global_tiles(M, K) + ZS_STREAM_SLACK_BYTES / 2;
}

int64_t zs_compressed_bytes(int M, int K, int64_t total_hf, int64_t total_full) {
  const int64_t mk = (int64_t)M * K;
  return total_hf + 2 * total_full + 24 * (mk / 64) + 8 * (mk / 1024) + 8 * (mk / 4096 + 1);
}

int64_t zs_splitk_workspace_bytes(int M, int N, int split_k) {
  if (split_k <= 1) return 0;
  return (int64_t)split_k * M * N * 2;
}

int zs_analyze_exponents_host(const uint16_t* a, int64_t n, int32_t top[7]) {
  if ((!a && n > 0) || n < 0 || !top) return ZS_E_INVAL;
  int64_t counts[256] = {0};
  // Four interleaved histograms keep the increments independent.
  int64_t h[4][256];
  memset(h, 0, sizeof(h));
  int64_t i = 0;
  for (; i + 4 <= n; i += 4) {
    h[0][(a[i] >> 7) & 0xFF]++;
    h[1][(a[i + 1] >> 7) & 0xFF]++;
    h[2][(a[i + 2] >> 7) & 0xFF]++;
    h[3][(a[i + 3] >> 7) & 0xFF]++;
  }
  for (; i < n; ++i) h[0][(a[i] >> 7) & 0xFF]++;
  for (int e = 0; e < 256; ++e) counts[e] = h[0][e] + h[1][e] + h[2][e] + h[3][e];
  select_window_cpu(counts, top);
  return ZS_OK;
}

void zs_host_free(void* p) { free(p); }

static int encode_entry(bool range, const uint16_t* A, int M, int K, int tM, int tMm, int tMg,
                        int tK, int tKm, int tKg, const int32_t* top, const Outputs& out,
                        const Temps& tmp, int32_t* max_hf, int32_t* max_full, int32_t* total_hf,
                        int32_t* total_full) {
  if (!tiles_ok(tM, tMm, tMg, tK, tKm, tKg)) return ZS_E_UNSUPPORTED;
  const int rc = check_shape(M, K);
  if (rc != ZS_OK) return rc;
  if (!A || !top || !out.sm || !out.full || !out.b1 || !out.b2 || !out.b3 || !out.tiles ||
      !out.median || !out.global || !tmp.sm || !tmp.full || !tmp.gt_hf || !tmp.gt_full ||
      !tmp.hf_off || !tmp.full_off)
    return ZS_E_INVAL;
  return range ? encode_matrix<true>(A, M, K, top, false, out, tmp, max_hf, max_full, total_hf,
                                     total_full)
               : encode_matrix<false>(A, M, K, top, false, out, tmp, max_hf, max_full, total_hf,
                                      total_full);
}

int zs_init_bf16_matrix_triple_bitmap_reuse(
    const uint16_t* A, int M, int K, int tM, int tMm, int tMg, int tK, int tKm, int tKg,
    const int32_t* top, uint8_t* sm, uint16_t* full, uint64_t* b1, uint64_t* b2, uint64_t* b3,
    int32_t* tiles, int32_t* median, int32_t* global, uint8_t* temp_sm, uint16_t* temp_full,
    int32_t* gt_hf, int32_t* gt_full, int32_t* hf_off, int32_t* full_off, int32_t* max_hf,
    int32_t* max_full, int32_t* total_hf, int32_t* total_full) {
  return encode_entry(false, A, M, K, tM, tMm, tMg, tK, tKm, tKg, top,
                      Outputs{sm, full, b1, b2, b3, tiles, median, global},
                      Temps{temp_sm, temp_full, gt_hf, gt_full, hf_off, full_off}, max_hf,
                      max_full, total_hf, total_full);
}

int zs_init_bf16_matrix_triple_bitmap_reuse_simd(
    const uint16_t* A, int M, int K, int tM, int tMm, int tMg, int tK, int tKm, int tKg,
    const int32_t* top, uint8_t* sm, uint16_t* full, uint64_t* b1, uint64_t* b2, uint64_t* b3,
    int32_t* tiles, int32_t* median, int32_t* global, uint8_t* temp_sm, uint16_t* temp_full,
    int32_t* gt_hf, int32_t* gt_full, int32_t* hf_off, int32_t* full_off, int32_t* max_hf,
    int32_t* max_full, int32_t* total_hf, int32_t* total_full) {
  return encode_entry(true, A, M, K, tM, tMm, tMg, tK, tKm, tKg, top,
                      Outputs{sm, full, b1, b2, b3, tiles, median, global},
                      Temps{temp_sm, temp_full, gt_hf, gt_full, hf_off, full_off}, max_hf,
                      max_full, total_hf, total_full);
}

int zs_init_bf16_matrix_triple_bitmap(const uint16_t* A, int M, int K, int tM, int tMm, int tMg,
                                      int tK, int tKm, int tKg, const int32_t* top,
                                      uint8_t** sm, uint16_t** full, uint64_t** b1,
                                      uint64_t** b2, uint64_t** b3, int32_t** tiles,
                                      int32_t** median, int32_t** global, int32_t* max_hf,
                                      int32_t* max_full) {
  if (!tiles_ok(tM, tMm, tMg, tK, tKm, tKg)) return ZS_E_UNSUPPORTED;
  int rc = check_shape(M, K);
  if (rc != ZS_OK) return rc;
  if (!A || !top || !sm || !full || !b1 || !b2 || !b3 || !tiles || !median || !global)
    return ZS_E_INVAL;
  const int64_t mk = (int64_t)M * K, ngt = mk / 4096;
  Outputs o{(uint8_t*)malloc((size_t)zs_sign_mantissa_capacity(M, K)),
            (uint16_t*)malloc((size_t)zs_full_capacity(M, K) * 2),
            (uint64_t*)malloc((size_t)(mk / 64) * 8),
            (uint64_t*)malloc((size_t)(mk / 64) * 8),
            (uint64_t*)malloc((size_t)(mk / 64) * 8),
            (int32_t*)malloc((size_t)(mk / 64) * 8),
            (int32_t*)malloc((size_t)(mk / 1024) * 8),
            (int32_t*)malloc((size_t)(ngt + 1) * 8)};
  Temps t{(uint8_t*)malloc((size_t)ngt * kSmStride + 16),
          (uint16_t*)malloc((size_t)ngt * kFullStride * 2),
          (int32_t*)malloc((size_t)ngt * 4),
          (int32_t*)malloc((size_t)ngt * 4),
          (int32_t*)malloc((size_t)(ngt + 1) * 4),
          (int32_t*)malloc((size_t)(ngt + 1) * 4)};
  int32_t th = 0, tf = 0;
  if (!o.sm || !o.full || !o.b1 || !o.b2 || !o.b3 || !o.tiles || !o.median || !o.global ||
      !t.sm || !t.full || !t.gt_hf || !t.gt_full || !t.hf_off || !t.full_off) {
    rc = ZS_E_NOMEM;
  } else {
    rc = encode_matrix<false>(A, M, K, top, true, o, t, max_hf, max_full, &th, &tf);
  }
  free(t.sm); free(t.full); free(t.gt_hf); free(t.gt_full); free(t.hf_off); free(t.full_off);
  if (rc < 0) {
    free(o.sm); free(o.full); free(o.b1); free(o.b2); free(o.b3);
    free(o.tiles); free(o.median); free(o.global);
    return rc;
  }
  // Zero the slack after each stream so device copies of it read zeros.
  memset(o.sm + th, 0, (size_t)(zs_sign_mantissa_capacity(M, K) - th));
  memset(o.full + tf, 0, (size_t)(zs_full_capacity(M, K) - tf) * 2);
  *sm = o.sm; *full = o.full; *b1 = o.b1; *b2 = o.b2; *b3 = o.b3;
  *tiles = o.tiles; *median = o.median; *global = o.global;
  return rc;
}

}  // extern "C"
