// xksv_encoder.cpp -- host-side block encoder (the compile step that feeds the
// GPU decode path).  Produces bytes identical to the reference codec:
//   xksv_pack / xksv_pack_parallel      src/c_api.cpp:18-28, 44-65
//   Huffman code lengths                 src/codec.cpp:32-53 (tie-break by node id)
//   canonical code assignment            src/codec.cpp:11-29
//   slab rule + raw fallback             src/compile.cpp:449-486, 257-276
// Identity with the reference is pinned by the golden vectors in tests/golden/.
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

#include "xksv_api_internal.hpp"

namespace xksv {
namespace {

constexpr uint64_t kSlabBytes = 1ull << 20;  // src/compile.cpp:38 (chunk)

void put64(uint8_t* p, uint64_t v) {
  for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i));
}

// Row-major matrix -> row-major 16x16 tiles, edge tiles hold only real
// elements (src/layout.cpp:32-50 with tile_rows = tile_cols = 16).
void tile16(const uint8_t* src, uint64_t rows, uint64_t cols, uint16_t* dst) {
  uint64_t packed = 0;
  for (uint64_t r = 0; r < rows; r += 16) {
    const uint64_t nr = std::min<uint64_t>(16, rows - r);
    for (uint64_t c = 0; c < cols; c += 16) {
      const uint64_t nc = std::min<uint64_t>(16, cols - c);
      for (uint64_t i = 0; i < nr; ++i) {
        memcpy(dst + packed, src + ((r + i) * cols + c) * 2, nc * 2);
        packed += nc;
      }
    }
  }
}

struct Encoded {
  uint64_t count = 0, bits = 0;
  uint8_t lengths[256] = {};
  std::vector<uint8_t> sm, codes;
  uint64_t segment_size() const { return 272 + count + codes.size(); }
  void write(uint8_t* p) const {
    put64(p, count);
    put64(p + 8, bits);
    memcpy(p + 16, lengths, 256);
    if (count) memcpy(p + 272, sm.data(), count);
    if (!codes.empty()) memcpy(p + 272 + count, codes.data(), codes.size());
  }
};

// Huffman lengths over the exponent histogram.  Leaves are numbered in
// ascending symbol order, internal nodes in creation order; the two smallest
// (frequency, node id) pairs merge first, the first popped becoming the left
// child.  A single symbol gets length 1.
bool huffman_lengths(const uint64_t freq[256], uint8_t lengths[256]) {
  struct Item {
    uint64_t f;
    int id;
  };
  auto less = [](const Item& a, const Item& b) { return a.f < b.f || (a.f == b.f && a.id < b.id); };
  Item heap[512];
  int hn = 0, nn = 0;
  int sym[511], left[511], right[511];
  auto push = [&](Item v) {
    int i = hn++;
    heap[i] = v;
    while (i > 0) {
      int p = (i - 1) / 2;
      if (!less(heap[i], heap[p])) break;
      std::swap(heap[i], heap[p]);
      i = p;
    }
  };
  auto pop = [&]() {
    Item top = heap[0];
    heap[0] = heap[--hn];
    int i = 0;
    for (;;) {
      int l = 2 * i + 1, r = l + 1, m = i;
      if (l < hn && less(heap[l], heap[m])) m = l;
      if (r < hn && less(heap[r], heap[m])) m = r;
      if (m == i) break;
      std::swap(heap[i], heap[m]);
      i = m;
    }
    return top;
  };
  for (int s = 0; s < 256; ++s)
    if (freq[s]) {
      sym[nn] = s;
      left[nn] = right[nn] = -1;
      push(Item{freq[s], nn++});
    }
  memset(lengths, 0, 256);
  if (!hn) return true;
  while (hn > 1) {
    Item a = pop(), b = pop();
    if (a.f > UINT64_MAX - b.f) return false;
    sym[nn] = -1;
    left[nn] = a.id;
    right[nn] = b.id;
    push(Item{a.f + b.f, nn++});
  }
  int stack[512], depth[512], sp = 0;
  stack[sp] = heap[0].id;
  depth[sp++] = 0;
  while (sp) {
    --sp;
    const int i = stack[sp], d = depth[sp];
    if (sym[i] >= 0) {
      if (d > 255) return false;
      lengths[sym[i]] = (uint8_t)std::max(d, 1);
    } else {
      stack[sp] = left[i];
      depth[sp++] = d + 1;
      stack[sp] = right[i];
      depth[sp++] = d + 1;
    }
  }
  return true;
}

// Canonical codes, left-aligned in 64 bits: the code of symbol s is the sum
// of 2^(64 - l) over all symbols ordered before s by (length, symbol).
// Lengths produced by huffman_lengths satisfy Kraft <= 1 and, for fewer than
// 2^32 elements, are at most 47 bits, so every code fits.
bool canonical64(const uint8_t lengths[256], uint64_t code[256]) {
  uint64_t acc = 0;
  for (int s = 0; s < 256; ++s)
    if (lengths[s] > 63) return false;
  for (int l = 1; l <= 63; ++l)
    for (int s = 0; s < 256; ++s)
      if (lengths[s] == l) {
        code[s] = acc;
        acc += 1ull << (64 - l);
      }
  return true;
}

bool encode_words(const uint16_t* w, uint64_t n, Encoded& out) {
  uint64_t freq[256] = {};
  for (uint64_t i = 0; i < n; ++i) ++freq[(w[i] >> 7) & 255];
  out.count = n;
  if (!huffman_lengths(freq, out.lengths)) return false;
  uint64_t code[256] = {};
  if (!canonical64(out.lengths, code)) return false;
  uint64_t total = 0;
  for (int s = 0; s < 256; ++s) total += freq[s] * out.lengths[s];
  out.bits = total;
  out.sm.resize(n);
  out.codes.assign((size_t)((total + 7) / 8), 0);
  uint8_t* dst = out.codes.data();
  uint64_t acc = 0;  // pending bits, MSB-aligned; `have` of them valid (< 64)
  unsigned have = 0;
  size_t o = 0;
  for (uint64_t i = 0; i < n; ++i) {
    const uint16_t v = w[i];
    out.sm[i] = (uint8_t)(((v >> 8) & 128) | (v & 127));
    const unsigned s = (v >> 7) & 255, l = out.lengths[s];
    const uint64_t c = code[s];
    acc |= c >> have;
    if (have + l >= 64) {
      for (int k = 0; k < 8; ++k) dst[o++] = (uint8_t)(acc >> (56 - 8 * k));
      const unsigned used = 64 - have;  // 1..63 since l <= 63
      acc = c << used;
      have = have + l - 64;
    } else {
      have += l;
    }
  }
  for (unsigned k = 0; 8 * k < have; ++k) dst[o++] = (uint8_t)(acc >> (56 - 8 * k));
  return true;
}

int emit(const std::vector<uint8_t>& v, void** out, size_t* out_size) {
  void* p = malloc(v.empty() ? 1 : v.size());
  if (!p) return -1;
  if (!v.empty()) memcpy(p, v.data(), v.size());
  *out = p;
  *out_size = v.size();
  return 0;
}

}  // namespace

// Serial block bytes for rows x cols BF16 at `data`.  false on invalid input.
bool encode_serial(const uint8_t* data, uint64_t rows, uint64_t cols, std::vector<uint8_t>& v) {
  const uint64_t n = rows * cols;
  std::vector<uint16_t> tiled(n);
  tile16(data, rows, cols, tiled.data());
  Encoded e;
  if (!encode_words(tiled.data(), n, e)) return false;
  v.resize(e.segment_size());
  e.write(v.data());
  return true;
}

// XKSP2 block bytes (rows <= 16).
bool encode_parallel(const uint8_t* data, uint64_t rows, uint64_t cols, std::vector<uint8_t>& v) {
  const uint64_t n = rows * cols;
  std::vector<uint16_t> tiled(n);
  tile16(data, rows, cols, tiled.data());
  const uint64_t chunks = std::min<uint64_t>(32, n);
  Encoded segs[32];
  uint64_t size = 32 + 8 * chunks;
  for (uint64_t i = 0; i < chunks; ++i) {
    const uint64_t a = n * i / chunks, b = n * (i + 1) / chunks;
    if (!encode_words(tiled.data() + a, b - a, segs[i])) return false;
    size += segs[i].segment_size();
  }
  v.assign(size, 0);
  memcpy(v.data(), "XKSP2\0\0\0", 8);
  put64(v.data() + 8, rows);
  put64(v.data() + 16, cols);
  put64(v.data() + 24, chunks);
  uint64_t pos = 32 + 8 * chunks;
  for (uint64_t i = 0; i < chunks; ++i) {
    put64(v.data() + 32 + 8 * i, segs[i].segment_size());
    segs[i].write(v.data() + pos);
    pos += segs[i].segment_size();
  }
  return true;
}

// Slab rule of the reference compiler for one tensor of `nbytes` bytes:
// BF16 2-D tensors with shape[1] <= 512Ki use cols = shape[1], else
// cols = min(4096, remaining / 2); rows = min(16, 1MiB / (2 cols),
// remaining / (2 cols)), falling back to one row of min(4096, remaining/2)
// columns at the tail.  Non-BF16 data is cut into raw 1 MiB blocks.
std::vector<SlabSpec> slab_rule(uint64_t nbytes, bool bf16, uint64_t shape_cols) {
  std::vector<SlabSpec> out;
  uint64_t cols = 0, remaining = nbytes, offset = 0;
  if (bf16) cols = (shape_cols && shape_cols <= kSlabBytes / 2) ? shape_cols : std::min<uint64_t>(4096, remaining / 2);
  while (remaining) {
    uint64_t rows = cols ? std::min({uint64_t(16), kSlabBytes / (cols * 2), remaining / (cols * 2)}) : 0;
    if (cols && !rows) {
      cols = std::min<uint64_t>(4096, remaining / 2);
      rows = 1;
    }
    const uint64_t length = rows ? rows * cols * 2 : std::min(remaining, kSlabBytes);
    out.push_back(SlabSpec{offset, length, rows, rows ? cols : 0});
    offset += length;
    remaining -= length;
  }
  return out;
}

}  // namespace xksv

using namespace xksv;

extern "C" {

// src/c_api.cpp:17
void xksv_free(void* p) { free(p); }

// src/c_api.cpp:18-28
int xksv_pack(const void* data, size_t n, size_t rows, size_t cols, void** out, size_t* out_size) {
  if (!out || !out_size || n % 2 || rows == 0 || cols > SIZE_MAX / rows || rows * cols != n / 2) return -1;
  if (!data && n) return -1;
  try {
    std::vector<uint8_t> v;
    if (!encode_serial(static_cast<const uint8_t*>(data), rows, cols, v)) return -1;
    return emit(v, out, out_size);
  } catch (...) {
    return -1;
  }
}

// src/c_api.cpp:44-65
int xksv_pack_parallel(const void* data, size_t n, size_t rows, size_t cols, void** out, size_t* out_size) {
  if (!out || !out_size || n % 2 || !rows || rows > 16 || !cols || cols > SIZE_MAX / rows || rows * cols != n / 2 ||
      rows * cols > SIZE_MAX / 32 || !data)
    return -1;
  try {
    std::vector<uint8_t> v;
    if (!encode_parallel(static_cast<const uint8_t*>(data), rows, cols, v)) return -1;
    return emit(v, out, out_size);
  } catch (...) {
    return -1;
  }
}

// Encode a whole tensor into blocks with the compiler's slab rule, on
// `threads` host threads (0 = all cores).  codec: 1 serial, 2 parallel32.
// Blocks whose encoding is not smaller than the raw bytes stay raw
// (src/compile.cpp:268-276).  The encoded archive region is written to *out
// (malloc'd, free with xksv_free); *blocks (malloc'd) gets one descriptor per
// block with offsets relative to *out and out_offset = byte offset of the
// block's raw bytes within the tensor.
int xksv_encode_tensor(const void* data, uint64_t nbytes, int bf16, uint64_t shape_cols, uint32_t codec,
                       uint32_t threads, void** out, uint64_t* out_size, xksv_hip_block** blocks,
                       uint64_t* nblocks) {
  // BF16 data is whole 2-byte words (an odd count would leave a 1-byte tail no slab can hold).
  if (!out || !out_size || !blocks || !nblocks || (nbytes && !data) || (codec != 1 && codec != 2) ||
      (bf16 && nbytes % 2))
    return -1;
  try {
    const std::vector<SlabSpec> slabs = slab_rule(nbytes, bf16 != 0, shape_cols);
    std::vector<std::vector<uint8_t>> enc(slabs.size());
    std::vector<uint32_t> kind(slabs.size(), kCodecRaw);
    std::atomic<size_t> next{0};
    std::atomic<bool> failed{false};
    const uint8_t* src = static_cast<const uint8_t*>(data);
    auto worker = [&]() {
      for (;;) {
        const size_t i = next.fetch_add(1);
        if (i >= slabs.size() || failed.load()) return;
        const SlabSpec& s = slabs[i];
        if (s.rows) {
          std::vector<uint8_t> v;
          const bool ok = codec == 1 ? encode_serial(src + s.offset, s.rows, s.cols, v)
                                     : (s.rows <= 16 && encode_parallel(src + s.offset, s.rows, s.cols, v));
          if (!ok) {
            failed = true;
            return;
          }
          if (v.size() < s.length) {
            enc[i] = std::move(v);
            kind[i] = codec;
            continue;
          }
        }
        enc[i].assign(src + s.offset, src + s.offset + s.length);
      }
    };
    unsigned nt = threads ? threads : std::max(1u, std::thread::hardware_concurrency());
    nt = (unsigned)std::min<size_t>(nt, std::max<size_t>(1, slabs.size()));
    std::vector<std::thread> pool;
    for (unsigned t = 1; t < nt; ++t) pool.emplace_back(worker);
    worker();
    for (auto& t : pool) t.join();
    if (failed) return -1;
    uint64_t total = 0;
    for (auto& e : enc) total += e.size();
    uint8_t* o = static_cast<uint8_t*>(malloc(total ? total : 1));
    xksv_hip_block* b = static_cast<xksv_hip_block*>(malloc(sizeof(xksv_hip_block) * (slabs.empty() ? 1 : slabs.size())));
    if (!o || !b) {
      free(o);
      free(b);
      return -1;
    }
    uint64_t pos = 0;
    for (size_t i = 0; i < slabs.size(); ++i) {
      memcpy(o + pos, enc[i].data(), enc[i].size());
      xksv_hip_block& d = b[i];
      d.offset = pos;
      d.size = enc[i].size();
      d.raw_size = slabs[i].length;
      d.out_offset = slabs[i].offset;
      d.rows = kind[i] == kCodecRaw ? 0 : slabs[i].rows;
      d.cols = kind[i] == kCodecRaw ? 0 : slabs[i].cols;
      d.codec = kind[i];
      d.reserved = 0;
      pos += enc[i].size();
    }
    *out = o;
    *out_size = total;
    *blocks = b;
    *nblocks = slabs.size();
    return 0;
  } catch (...) {
    return -1;
  }
}

}  // extern "C"
