// zs_container.cpp -- versioned byte container for one compressed matrix.
//
// The reference keeps compressed matrices only in memory (seven tensors plus
// the 11-int64 meta tensor of zipserv_decode_attention_ext.cu:250-262); this
// container lets a matrix be compressed once and stored or sent.  Layout,
// little-endian:
//
//   [0, 256)  header
//     0   char[8]  magic "ZSRVCNTR"
//     8   u32      version (1)
//     12  u32      header bytes (256)
//     16  u32      layout (ZS_CONTAINER_CANONICAL / ZS_CONTAINER_RETILED)
//     20  u32      number of streams (7 canonical, 3 re-tiled)
//     24  i32 x 7  rows, cols, logical_rows, logical_cols, start_exp,
//                  max_high_freq_count, max_full_count
//     52  u32      CRC-32C of bytes [0, 256) with this field zero
//     56  u64      container bytes (header + padded streams)
//     64  char[64] name, UTF-8, zero padded
//     128 8 x {u64 bytes, u32 CRC-32C of the stream, u32 zero}
//   [256, ...) the streams in table order, each padded with zeros to a
//              multiple of 64 bytes.
//
// Canonical streams: sign_mantissa, compressed_full, bitmap1..3,
// tile_offsets_median, tile_offsets_global (include/zipserv.h); re-tiled:
// fixed records, outlier exponent bytes, record offsets.  The parser checks
// magic, version, header and stream CRCs, every stream size the shape fixes,
// and that the last offsets match the SM / FULL / exponent stream sizes.
// CRC-32C (Castagnoli polynomial, reflected 0x82F63B78) runs on the SSE4.2
// crc32 instruction, eight bytes per step.
#include <nmmintrin.h>

#include <cstdint>
#include <cstring>

#include "../../include/zipserv.h"

namespace {

constexpr char kMagic[8] = {'Z', 'S', 'R', 'V', 'C', 'N', 'T', 'R'};
constexpr uint32_t kVersion = 1;
constexpr int64_t kHeader = 256;
constexpr int64_t kAlign = 64;
constexpr int kMaxStreams = 8;

int64_t pad64(int64_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

uint32_t crc32c_update(uint32_t crc, const uint8_t* p, int64_t n) {
  uint64_t c = ~crc;
  while (n > 0 && (reinterpret_cast<uintptr_t>(p) & 7)) {
    c = _mm_crc32_u8((uint32_t)c, *p++);
    --n;
  }
  while (n >= 8) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    c = _mm_crc32_u64(c, v);
    p += 8;
    n -= 8;
  }
  while (n-- > 0) c = _mm_crc32_u8((uint32_t)c, *p++);
  return ~(uint32_t)c;
}

void put32(uint8_t* h, int off, uint32_t v) { std::memcpy(h + off, &v, 4); }
void put64(uint8_t* h, int off, uint64_t v) { std::memcpy(h + off, &v, 8); }
uint32_t get32(const uint8_t* h, int off) {
  uint32_t v;
  std::memcpy(&v, h + off, 4);
  return v;
}
uint64_t get64(const uint8_t* h, int off) {
  uint64_t v;
  std::memcpy(&v, h + off, 8);
  return v;
}

// Stream sizes the shape fixes (-1: free, set by the totals).
int expected_sizes(const zs_container_desc_t* d, int64_t* sz) {
  const int64_t M = d->rows, K = d->cols;
  if (M <= 0 || K <= 0 || (M % 64) || (K % 64)) return ZS_E_INVAL;
  const int64_t mk = M * K;
  if (d->layout == ZS_CONTAINER_CANONICAL) {
    if (d->num_streams != 7) return ZS_E_INVAL;
    sz[0] = sz[1] = -1;
    sz[2] = sz[3] = sz[4] = mk / 64 * 8;
    sz[5] = mk / 1024 * 2 * 4;
    sz[6] = (mk / 4096 + 1) * 2 * 4;
  } else if (d->layout == ZS_CONTAINER_RETILED) {
    if (d->num_streams != 3) return ZS_E_INVAL;
    const int64_t nrec = mk / 1024;
    sz[0] = nrec * 1408;
    sz[1] = -1;
    sz[2] = (nrec + 1) * 4;
  } else {
    return ZS_E_UNSUPPORTED;
  }
  return ZS_OK;
}

int check_desc(const zs_container_desc_t* d) {
  if (!d) return ZS_E_INVAL;
  int64_t sz[kMaxStreams];
  const int st = expected_sizes(d, sz);
  if (st != ZS_OK) return st;
  if (d->start_exp < 0 || d->start_exp > 255 || d->max_high_freq_count < 0 ||
      d->max_full_count < 0 || d->logical_rows < 0 || d->logical_cols < 0)
    return ZS_E_INVAL;
  for (int i = 0; i < d->num_streams; ++i) {
    if (d->stream_bytes[i] < 0) return ZS_E_INVAL;
    if (sz[i] >= 0 && d->stream_bytes[i] != sz[i]) return ZS_E_INVAL;
  }
  if (d->layout == ZS_CONTAINER_CANONICAL && (d->stream_bytes[1] & 1)) return ZS_E_INVAL;
  return ZS_OK;
}

// Every offset the kernels follow must agree with the bit-planes / codes it
// indexes, or a decoder would read past its streams: the last offsets equal
// the free streams' sizes, and
//  * canonical: tile_offsets_global starts at (0, 0) and steps by each global
//    tile's in-window / outlier counts (from its bitmaps) padded to 16 / 8;
//    tile_offsets_median holds the unpadded counts before each median tile;
//  * re-tiled: eoff starts at 0 and steps by each record's outlier count
//    (the elements whose 3-bit code is 0).
int check_offsets(const zs_container_desc_t* d, const uint8_t* const* s) {
  if (d->layout == ZS_CONTAINER_CANONICAL) {
    const int64_t ngt = (int64_t)d->rows * d->cols / 4096;
    const uint8_t* bm[3] = {s[2], s[3], s[4]};
    int64_t hf_at = 0, fu_at = 0;
    for (int64_t g = 0; g <= ngt; ++g) {
      int32_t tog[2];
      std::memcpy(tog, s[6] + 8 * g, 8);
      if (tog[0] != hf_at || tog[1] != fu_at) return ZS_E_INVAL;
      if (g == ngt) break;
      int32_t before = 0;
      for (int m = 0; m < 4; ++m) {
        int32_t tom[2];
        std::memcpy(tom, s[5] + 8 * (4 * g + m), 8);
        if (tom[0] != before || tom[1] != 1024 * m - before) return ZS_E_INVAL;
        for (int t = 0; t < 16; ++t) {
          const int64_t tile = 64 * g + 16 * m + t;
          uint64_t b[3];
          for (int k = 0; k < 3; ++k) std::memcpy(&b[k], bm[k] + 8 * tile, 8);
          before += __builtin_popcountll(b[0] | b[1] | b[2]);
        }
      }
      hf_at += (before + 15) & ~15;
      fu_at += (4096 - before + 7) & ~7;
      if (hf_at > INT32_MAX || fu_at > INT32_MAX) return ZS_E_INVAL;
    }
    if (hf_at != d->stream_bytes[0] || 2 * fu_at != d->stream_bytes[1]) return ZS_E_INVAL;
  } else {
    const int64_t nrec = (int64_t)d->rows * d->cols / 1024;
    int64_t at = 0;
    for (int64_t r = 0; r <= nrec; ++r) {
      int32_t e;
      std::memcpy(&e, s[2] + 4 * r, 4);
      if (e != at) return ZS_E_INVAL;
      if (r == nrec) break;
      const uint8_t* rec = s[0] + r * 1408;
      int n = 0;
      for (int l = 0; l < 64; ++l) {
        uint32_t p32;
        uint16_t p16;
        std::memcpy(&p32, rec + 1024 + 4 * l, 4);
        std::memcpy(&p16, rec + 1280 + 2 * l, 2);
        const uint64_t codes = (uint64_t)p32 | ((uint64_t)p16 << 32);  // 16 codes x 3 bits
        for (int i = 0; i < 16; ++i) n += ((codes >> (3 * i)) & 7u) == 0;
      }
      at += n;
      if (at > INT32_MAX) return ZS_E_INVAL;
    }
    if (at != d->stream_bytes[1]) return ZS_E_INVAL;
  }
  return ZS_OK;
}

}  // namespace

extern "C" {

uint32_t zs_crc32c(uint32_t crc, const void* data, int64_t bytes) {
  if (!data || bytes <= 0) return crc;
  return crc32c_update(crc, static_cast<const uint8_t*>(data), bytes);
}

int64_t zs_container_bytes(const zs_container_desc_t* d) {
  const int st = check_desc(d);
  if (st != ZS_OK) return st;
  int64_t n = kHeader;
  for (int i = 0; i < d->num_streams; ++i) n += pad64(d->stream_bytes[i]);
  return n;
}

int zs_container_write(const zs_container_desc_t* d, const char* name,
                       const void* const* streams, void* dst, int64_t dst_bytes) {
  const int64_t total = zs_container_bytes(d);
  if (total < 0) return (int)total;
  if (!streams || !dst || dst_bytes < total) return ZS_E_INVAL;
  for (int i = 0; i < d->num_streams; ++i)
    if (!streams[i] && d->stream_bytes[i] > 0) return ZS_E_INVAL;
  const uint8_t* s[kMaxStreams];
  for (int i = 0; i < d->num_streams; ++i) s[i] = static_cast<const uint8_t*>(streams[i]);
  if (check_offsets(d, s) != ZS_OK) return ZS_E_INVAL;
  uint8_t* out = static_cast<uint8_t*>(dst);
  uint8_t* h = out;
  std::memset(h, 0, kHeader);
  std::memcpy(h, kMagic, 8);
  put32(h, 8, kVersion);
  put32(h, 12, (uint32_t)kHeader);
  put32(h, 16, (uint32_t)d->layout);
  put32(h, 20, (uint32_t)d->num_streams);
  const int32_t f[7] = {d->rows, d->cols, d->logical_rows, d->logical_cols, d->start_exp,
                        d->max_high_freq_count, d->max_full_count};
  std::memcpy(h + 24, f, sizeof(f));
  put64(h, 56, (uint64_t)total);
  if (name) {
    const size_t n = strnlen(name, 63);
    std::memcpy(h + 64, name, n);
  }
  int64_t off = kHeader;
  for (int i = 0; i < d->num_streams; ++i) {
    const int64_t n = d->stream_bytes[i];
    put64(h, 128 + 16 * i, (uint64_t)n);
    put32(h, 136 + 16 * i, zs_crc32c(0, s[i], n));
    if (n > 0) std::memcpy(out + off, s[i], (size_t)n);
    std::memset(out + off + n, 0, (size_t)(pad64(n) - n));
    off += pad64(n);
  }
  put32(h, 52, zs_crc32c(0, h, kHeader));
  return ZS_OK;
}

int zs_container_parse(const void* src, int64_t src_bytes, zs_container_desc_t* d,
                       char* name_out, int64_t* stream_offsets) {
  if (!src || !d || src_bytes < kHeader) return ZS_E_INVAL;
  const uint8_t* h = static_cast<const uint8_t*>(src);
  if (std::memcmp(h, kMagic, 8) != 0) return ZS_E_INVAL;
  if (get32(h, 8) != kVersion || get32(h, 12) != (uint32_t)kHeader) return ZS_E_UNSUPPORTED;
  uint8_t hc[kHeader];
  std::memcpy(hc, h, kHeader);
  put32(hc, 52, 0);
  if (zs_crc32c(0, hc, kHeader) != get32(h, 52)) return ZS_E_INVAL;
  zs_container_desc_t t{};
  t.layout = (int32_t)get32(h, 16);
  t.num_streams = (int32_t)get32(h, 20);
  if (t.num_streams < 0 || t.num_streams > kMaxStreams) return ZS_E_INVAL;
  int32_t f[7];
  std::memcpy(f, h + 24, sizeof(f));
  t.rows = f[0];
  t.cols = f[1];
  t.logical_rows = f[2];
  t.logical_cols = f[3];
  t.start_exp = f[4];
  t.max_high_freq_count = f[5];
  t.max_full_count = f[6];
  for (int i = 0; i < t.num_streams; ++i) {
    const uint64_t n = get64(h, 128 + 16 * i);
    if (n > (uint64_t)INT64_MAX / 2) return ZS_E_INVAL;
    t.stream_bytes[i] = (int64_t)n;
  }
  const int st = check_desc(&t);
  if (st != ZS_OK) return st;
  const int64_t total = zs_container_bytes(&t);
  if ((uint64_t)total != get64(h, 56) || total > src_bytes) return ZS_E_INVAL;
  const uint8_t* s[kMaxStreams];
  int64_t off = kHeader;
  for (int i = 0; i < t.num_streams; ++i) {
    s[i] = h + off;
    if (zs_crc32c(0, s[i], t.stream_bytes[i]) != get32(h, 136 + 16 * i)) return ZS_E_INVAL;
    if (stream_offsets) stream_offsets[i] = off;
    off += pad64(t.stream_bytes[i]);
  }
  if (check_offsets(&t, s) != ZS_OK) return ZS_E_INVAL;
  *d = t;
  if (name_out) {
    std::memcpy(name_out, h + 64, 63);
    name_out[63] = 0;
  }
  return ZS_OK;
}

}  // extern "C"
