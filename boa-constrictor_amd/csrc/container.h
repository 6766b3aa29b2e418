// BOA2 container and small host helpers (header-only, host code).
//
// Byte layout (portability_solved_cpp/boa.cpp:538-581 writer, :190-277
// reader; Python twin boa.py:108-189):
//   "BOA2" | u32 version = 1 | u32 flags (bit 0 = warm-start) | u64 total_size
//   | u32 chunk_len | u32 n_chunks | u32 last_chunk_len | u8 fp_len | fp bytes
//   | payload: per-chunk little-endian u32 word streams, back to back
//   | "IDX2" | n first bytes | n x LEB128(stream bytes) | u32 CRC-32 of the
//   index (from "IDX2" up to the CRC).
// The reader finds the index by scanning backwards for the last "IDX2" or
// "IDX1" tag, as the reference does; IDX1 (delta offsets then lengths) is
// accepted for reading.
#pragma once
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

struct Boa2Header {
  uint32_t version = 1;
  uint32_t flags = 0;
  uint64_t total_size = 0;
  uint32_t chunk_len = 0;
  uint32_t n_chunks = 0;
  uint32_t last_chunk_len = 0;
  std::vector<uint8_t> fp;  // fingerprint / warm-start interleave batch
};

struct Boa2Parsed {
  Boa2Header hdr;
  uint32_t interleave_batch = 0;
  size_t payload_off = 0;
  size_t idx_off = 0;
  int idx_version = 0;
  std::vector<uint8_t> first;
  std::vector<uint64_t> offsets, lengths;
};

inline uint32_t boa2_crc32(const uint8_t* data, size_t n) {
  static uint32_t table[256];
  static bool init = false;
  if (!init) {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1) ? (0xEDB88320u ^ (c >> 1)) : (c >> 1);
      table[i] = c;
    }
    init = true;
  }
  uint32_t c = 0xFFFFFFFFu;
  for (size_t i = 0; i < n; ++i) c = table[(c ^ data[i]) & 0xFFu] ^ (c >> 8);
  return c ^ 0xFFFFFFFFu;
}

inline void boa2_uvarint(std::vector<uint8_t>& out, uint64_t x) {
  for (;;) {
    uint8_t b = (uint8_t)(x & 0x7Fu);
    x >>= 7;
    out.push_back((uint8_t)(b | (x ? 0x80u : 0u)));
    if (!x) break;
  }
}

inline bool boa2_read_uvarint(const uint8_t* buf, size_t end, size_t& pos, uint64_t& out) {
  uint64_t x = 0;
  int shift = 0;
  for (;;) {
    if (pos >= end || shift > 63) return false;
    uint8_t b = buf[pos++];
    x |= (uint64_t)(b & 0x7Fu) << shift;
    if (!(b & 0x80u)) break;
    shift += 7;
  }
  out = x;
  return true;
}

template <class T>
inline void boa2_put(std::vector<uint8_t>& out, T v) {
  uint8_t b[sizeof(T)];
  memcpy(b, &v, sizeof(T));
  out.insert(out.end(), b, b + sizeof(T));
}

inline void boa2_write(const Boa2Header& h, const std::vector<uint8_t>& payload,
                       const uint8_t* first, const uint64_t* stream_bytes, size_t n,
                       std::vector<uint8_t>& out) {
  out.clear();
  out.reserve(33 + h.fp.size() + payload.size() + 8 + n * 6);
  out.insert(out.end(), {'B', 'O', 'A', '2'});
  boa2_put<uint32_t>(out, h.version);
  boa2_put<uint32_t>(out, h.flags);
  boa2_put<uint64_t>(out, h.total_size);
  boa2_put<uint32_t>(out, h.chunk_len);
  boa2_put<uint32_t>(out, h.n_chunks);
  boa2_put<uint32_t>(out, h.last_chunk_len);
  out.push_back((uint8_t)h.fp.size());
  out.insert(out.end(), h.fp.begin(), h.fp.end());
  out.insert(out.end(), payload.begin(), payload.end());
  const size_t idx = out.size();
  out.insert(out.end(), {'I', 'D', 'X', '2'});
  out.insert(out.end(), first, first + n);
  for (size_t i = 0; i < n; ++i) boa2_uvarint(out, stream_bytes[i]);
  const uint32_t crc = boa2_crc32(out.data() + idx, out.size() - idx);
  boa2_put<uint32_t>(out, crc);
}

inline bool boa2_parse(const uint8_t* d, size_t n, Boa2Parsed& P, std::string& why) {
  auto rd32 = [&](size_t p) { uint32_t v; memcpy(&v, d + p, 4); return v; };
  if (n < 33) { why = "Invalid BOA2 file"; return false; }
  if (memcmp(d, "BOA2", 4) != 0) { why = "Bad BOA2 magic"; return false; }
  P.hdr.version = rd32(4);
  if (P.hdr.version != 1) { why = "Unsupported BOA2 version"; return false; }
  P.hdr.flags = rd32(8);
  memcpy(&P.hdr.total_size, d + 12, 8);
  P.hdr.chunk_len = rd32(20);
  P.hdr.n_chunks = rd32(24);
  P.hdr.last_chunk_len = rd32(28);
  const uint8_t fp_len = d[32];
  size_t p = 33;
  if (p + fp_len > n) { why = "Invalid BOA2 file"; return false; }
  P.hdr.fp.assign(d + p, d + p + fp_len);
  if ((P.hdr.flags & 1u) && fp_len >= 4) P.interleave_batch = rd32(p);
  p += fp_len;
  P.payload_off = p;
  size_t idx = (size_t)-1;
  int ver = 0;
  for (size_t i = n - 4; i-- > 0;) {
    if (d[i] == 'I' && d[i + 1] == 'D' && d[i + 2] == 'X') {
      if (d[i + 3] == '2') { idx = i; ver = 2; break; }
      if (d[i + 3] == '1') { idx = i; ver = 1; break; }
    }
  }
  if (idx == (size_t)-1) { why = "IDX not found"; return false; }
  if (n < idx + 8 || idx < P.payload_off) { why = "Bad BOA2 IDX"; return false; }
  if (rd32(n - 4) != boa2_crc32(d + idx, n - idx - 4)) { why = "Bad BOA2 CRC"; return false; }
  P.idx_off = idx;
  P.idx_version = ver;
  const size_t nc = P.hdr.n_chunks, end = n - 4;
  size_t q = idx + 4;
  if (q + nc > end) { why = "Bad BOA2 IDX"; return false; }
  P.first.assign(d + q, d + q + nc);
  q += nc;
  P.offsets.assign(nc, 0);
  P.lengths.assign(nc, 0);
  if (ver == 1) {
    uint64_t prev = 0, dl;
    for (size_t i = 0; i < nc; ++i) {
      if (!boa2_read_uvarint(d, end, q, dl)) { why = "Bad BOA2 IDX"; return false; }
      prev += dl;
      P.offsets[i] = prev;
    }
    for (size_t i = 0; i < nc; ++i)
      if (!boa2_read_uvarint(d, end, q, P.lengths[i])) { why = "Bad BOA2 IDX"; return false; }
  } else {
    uint64_t off = 0;
    for (size_t i = 0; i < nc; ++i) {
      if (!boa2_read_uvarint(d, end, q, P.lengths[i])) { why = "Bad BOA2 IDX"; return false; }
      P.offsets[i] = off;
      off += P.lengths[i];
    }
  }
  const uint64_t payload = idx - P.payload_off;
  for (size_t i = 0; i < nc; ++i)
    if (P.offsets[i] + P.lengths[i] > payload || P.offsets[i] + P.lengths[i] < P.offsets[i]) {
      why = "BOA2 payload out of range";
      return false;
    }
  // Header consistency beyond what the reference's reader checks: the
  // lengths a compressor can write (chunks of at most 2^30 bytes, a last
  // chunk of 1 .. chunk_len bytes, total = (n - 1) chunk_len + last), and a
  // warm-start interleave batch in [1, n_chunks].
  if (nc && (P.hdr.chunk_len == 0 || P.hdr.chunk_len > (1u << 30) || P.hdr.last_chunk_len == 0 ||
             P.hdr.last_chunk_len > P.hdr.chunk_len)) {
    why = "Bad BOA2 chunk lengths";
    return false;
  }
  const uint64_t total = nc ? (uint64_t)(nc - 1) * P.hdr.chunk_len + P.hdr.last_chunk_len : 0;
  if (P.hdr.total_size != total) {
    why = "BOA2 total size does not match the chunk lengths";
    return false;
  }
  if ((P.hdr.flags & 1u) && nc && (fp_len < 4 || P.interleave_batch == 0 || P.interleave_batch > nc)) {
    why = "Bad BOA2 warm-start interleave batch";
    return false;
  }
  return true;
}

inline bool boa_read_file(const char* path, std::vector<uint8_t>& out) {
  FILE* f = fopen(path, "rb");
  if (!f) return false;
  if (fseek(f, 0, SEEK_END) != 0) { fclose(f); return false; }
  long n = ftell(f);
  if (n < 0) { fclose(f); return false; }
  fseek(f, 0, SEEK_SET);
  out.resize((size_t)n);
  bool ok = n == 0 || fread(out.data(), 1, (size_t)n, f) == (size_t)n;
  fclose(f);
  return ok;
}

inline bool boa_write_file(const char* path, const uint8_t* data, size_t n) {
  FILE* f = fopen(path, "wb");
  if (!f) return false;
  bool ok = n == 0 || fwrite(data, 1, n, f) == n;
  ok = (fclose(f) == 0) && ok;
  return ok;
}

// IEEE half -> float widening (boa_gpu.hpp:16-43).
inline float boa_host_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t ex = (h >> 10) & 0x1Fu;
  uint32_t mant = h & 0x3FFu;
  uint32_t out;
  if (ex == 0) {
    if (mant == 0) {
      out = sign;
    } else {
      int e = 1;
      while (!(mant & 0x400u)) { mant <<= 1; e--; }
      mant &= 0x3FFu;
      out = sign | ((uint32_t)(127 - 15 + e) << 23) | (mant << 13);
    }
  } else if (ex == 31) {
    out = sign | 0x7F800000u | (mant << 13);
  } else {
    out = sign | ((ex - 15 + 127) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}
