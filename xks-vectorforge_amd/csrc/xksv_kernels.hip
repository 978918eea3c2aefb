// xksv_kernels.hip -- gfx950 (MI355X) kernels for the XKSV compressed-weight path.
//
// What runs here (reference behaviour in brackets):
//   * canonical-Huffman decode of BF16 exponent streams, both block codecs:
//     serial "bf16-huffman-tile16" and XKSP2 "bf16-huffman-parallel32"
//     [src/codec.cpp:59-74, src/c_api.cpp:29-40,66-85, cuda/decode.cu:12-27,
//      cuda/parallel.cu:13-31];
//   * recombination with the stored sign/mantissa byte [src/codec.cpp:70];
//   * inverse 16x16 tiling with 16-byte stores [src/layout.cpp:32-53];
//   * fused decode-GEMV / decode-GEMM that never materialise the weights in
//     HBM [cuda/decode.cu:28-45, cuda/parallel.cu:27].
//
// Execution model.  One wavefront (64 lanes, one workgroup) owns one Huffman
// stream at a time: a parallel32 substream, or a whole serial slab.  The
// wave builds the stream's canonical-code lookup tables in LDS, stages the
// code stream in LDS in segments of 64 x 96 bits, and every lane decodes one
// 96-bit chunk speculatively from the chunk's first bit, recording which bit
// positions of the chunk's first 32 bits start a codeword.  Codes are at most
// 32 bits on this path, so the true entry into a chunk lies within those 32
// bits; a lane is synchronised when its true entry is one of its recorded
// starts, otherwise it re-decodes from the true entry.  A wave prefix sum
// places each lane's symbols; the run is compacted in LDS and handed to a
// consumer (BF16 writer, fused GEMV, fused GEMM) a whole 16x16 tile at a time.
// Streams with codes longer than 32 bits take a bit-serial path in the same
// kernel.  Error semantics equal the reference's: a block fails iff the
// reference's unpack fails on it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "xksv_shared.hpp"

namespace xksv {
namespace {

constexpr uint32_t kWave = 64;
constexpr uint32_t kChunk = 96;                     // code bits per lane per segment
constexpr uint32_t kRegion = kChunk + 4;            // lane scratch stride: 25 dwords, odd -> conflict-free
constexpr uint32_t kSegBits = kWave * kChunk;       // 6144 bits per segment
constexpr uint32_t kCarry = 256;                    // room for an unconsumed partial tile
constexpr uint32_t kSymsBytes = kCarry + kWave * kRegion;
constexpr uint32_t kStreamDw = kSegBits / 32 + 2;   // segment dwords plus lookahead
constexpr uint32_t kStreamLanes = (kStreamDw + 3) / 4;
constexpr uint32_t kLutBits = 10;
constexpr uint32_t kMaxLenFast = 32;
constexpr uint32_t kSlowSeg = 4096;                 // symbols per bit-serial segment (multiple of 256)
constexpr uint64_t kMagicXKSP2 = 0x0000003250534B58ull;  // "XKSP2\0\0\0" little-endian

// Per-wave LDS.  The table area is either the fast tables (LUT + per-length
// limits) or the bit-serial tables; rank/compaction scratch lives in `syms`
// before decoding starts.
struct FastTables {
  uint16_t lut[1u << kLutBits];  // (len << 8) | symbol for codes of <= 10 bits; 0 = longer/invalid
  uint64_t lim[40];              // lim[l] = left-aligned 32-bit end of the length-l codes, C(l+1)
  uint64_t slots[40];            // per-length lane masks (rank computation)
  uint32_t cnt[40];              // codes per length
  uint16_t base[40];             // index of the first length-l symbol in `sorted`
  uint16_t l4[16];               // codes of <= 4 bits, indexed by the top 4 bits
};
struct SlowTables {
  uint32_t cnt[256];
  uint16_t base[256];
  uint16_t open[256];            // prefixes of length l that longer codes extend
  uint16_t cursor[256];
};
struct alignas(16) Smem {
  union {
    FastTables f;
    SlowTables s;
  } t;
  uint8_t sorted[256];           // symbols in (length, symbol) order
  uint32_t stream[kStreamLanes * 4 + 4];  // [0] = zero dword before the segment
  uint32_t bcast[4];
  alignas(16) uint8_t syms[kSymsBytes];
};

// ------------------------------------------------------------------ helpers

__device__ __forceinline__ uint32_t lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}
// Number of set bits of `m` below this lane.
__device__ __forceinline__ uint32_t mbcnt(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
__device__ __forceinline__ uint32_t rdlane(uint32_t v, uint32_t l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ uint64_t rdlane64(uint64_t v, uint32_t l) {
  return (uint64_t)rdlane((uint32_t)v, l) | ((uint64_t)rdlane((uint32_t)(v >> 32), l) << 32);
}
template <typename T>
__device__ __forceinline__ T wave_incl(T v, uint32_t lane) {
#pragma unroll
  for (uint32_t d = 1; d < kWave; d <<= 1) {
    T o = __shfl_up(v, d, kWave);
    if (lane >= d) v += o;
  }
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (uint32_t d = kWave / 2; d >= 1; d >>= 1) {
    T o = __shfl_xor(v, d, kWave);
    v = v > o ? v : o;
  }
  return v;
}
__device__ __forceinline__ uint64_t ldg64(const uint8_t* p) {
  uint64_t v;
  __builtin_memcpy(&v, p, 8);
  return v;
}
__device__ __forceinline__ uint32_t ldg32(const uint8_t* p) {
  uint32_t v;
  __builtin_memcpy(&v, p, 4);
  return v;
}
// 16 bytes at p; bytes at or past `end` read as zero and are never fetched.
__device__ __forceinline__ uint4 ldg16_bounded(const uint8_t* p, const uint8_t* end) {
  uint4 v;
  if (p + 16 <= end) {
    __builtin_memcpy(&v, p, 16);
    return v;
  }
  uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (p + i < end) w[i >> 2] |= (uint32_t)p[i] << (8 * (i & 3));
  v.x = w[0]; v.y = w[1]; v.z = w[2]; v.w = w[3];
  return v;
}
__device__ __forceinline__ uint32_t lds32(const uint8_t* p) {
  uint32_t v;
  __builtin_memcpy(&v, p, 4);
  return v;
}
__device__ __forceinline__ void sts32(uint8_t* p, uint32_t v) { __builtin_memcpy(p, &v, 4); }
__device__ __forceinline__ uint32_t bswap32(uint32_t v) { return __builtin_amdgcn_perm(0u, v, 0x00010203u); }

// Eight exponents (E, little-endian byte i = element i) and eight
// sign/mantissa bytes (M) -> eight BF16 words:
//   word = ((sm & 0x80) << 8) | (exp << 7) | (sm & 0x7f)      [src/codec.cpp:70]
// high byte = (sm & 0x80) | (exp >> 1), low byte = (exp << 7) | (sm & 0x7f).
__device__ __forceinline__ uint4 combine8(uint64_t E, uint64_t M) {
  const uint32_t e0 = (uint32_t)E, e1 = (uint32_t)(E >> 32);
  const uint32_t s0 = (uint32_t)M, s1 = (uint32_t)(M >> 32);
  const uint32_t hi0 = (s0 & 0x80808080u) | ((e0 >> 1) & 0x7f7f7f7fu);
  const uint32_t lo0 = ((e0 << 7) & 0x80808080u) | (s0 & 0x7f7f7f7fu);
  const uint32_t hi1 = (s1 & 0x80808080u) | ((e1 >> 1) & 0x7f7f7f7fu);
  const uint32_t lo1 = ((e1 << 7) & 0x80808080u) | (s1 & 0x7f7f7f7fu);
  uint4 w;
  w.x = __builtin_amdgcn_perm(hi0, lo0, 0x05010400u);
  w.y = __builtin_amdgcn_perm(hi0, lo0, 0x07030602u);
  w.z = __builtin_amdgcn_perm(hi1, lo1, 0x05010400u);
  w.w = __builtin_amdgcn_perm(hi1, lo1, 0x07030602u);
  return w;
}
__device__ __forceinline__ float bf_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

// Tiled position q of a rows x cols slab -> (row, col)          [src/layout.cpp:36-48]
__device__ __forceinline__ void tile_to_rc(uint64_t q, uint64_t rows, uint64_t cols, uint64_t& row, uint64_t& col) {
  const uint64_t band = q / (16 * cols);
  const uint64_t nr = (rows - 16 * band) < 16 ? (rows - 16 * band) : 16;
  const uint64_t local = q - band * 16 * cols;
  const uint64_t t = local / (nr * 16);
  const uint64_t lt = local - t * nr * 16;
  const uint64_t width = (cols - 16 * t) < 16 ? (cols - 16 * t) : 16;
  row = 16 * band + lt / width;
  col = 16 * t + lt % width;
}

// ---------------------------------------------------------- block headers

struct Stream {
  const uint8_t* sm;       // sign/mantissa bytes, one per element, tiled order
  const uint8_t* bits;     // MSB-first exponent code stream
  const uint8_t* lengths;  // 256 code lengths
  uint64_t nbits;
  uint32_t count;          // elements in this stream
  uint32_t start;          // tiled position of the stream's first element in its slab
};

// XKSP2 header and substream k                                   [src/c_api.cpp:66-85]
// Returns error bits; `chunks` is set (> 0) once the block-level checks pass.
__device__ uint32_t parse_parallel(const uint8_t* blk, uint64_t size, const DevBlock& d, uint32_t k,
                                   uint32_t lane, Stream& st, uint32_t& chunks) {
  chunks = 0;
  if (size < 32) return kErrHeader;
  const uint64_t hv = lane < 4 ? ldg64(blk + 8 * lane) : 0;
  const uint64_t magic = rdlane64(hv, 0), rows = rdlane64(hv, 1), cols = rdlane64(hv, 2), nch = rdlane64(hv, 3);
  if (magic != kMagicXKSP2 || !rows || rows > 16 || !cols || !nch || nch > 32 || cols > ~0ull / rows)
    return kErrHeader;
  const uint64_t total = rows * cols;
  if (nch > total || total > size || total > ~0ull / 32 || size < 32 + 8 * nch) return kErrHeader;
  if (rows != d.rows || cols != d.cols || total > kMaxBlockElems) return kErrShape;
  const uint64_t len = lane < nch ? ldg64(blk + 32 + 8 * lane) : 0;
  if (__ballot(lane < nch && (len < 272 || len > size))) return kErrHeader;
  const uint64_t incl = wave_incl(len, lane);
  const uint64_t hdr = 32 + 8 * nch;
  if (hdr + rdlane64(incl, (uint32_t)nch - 1) != size) return kErrHeader;
  chunks = (uint32_t)nch;
  if (k >= chunks) return 0;
  const uint64_t slen = rdlane64(len, k);
  const uint64_t off = hdr + rdlane64(incl, k) - slen;
  const uint64_t fv = lane < 2 ? ldg64(blk + off + 8 * lane) : 0;
  const uint64_t cnt = rdlane64(fv, 0), nb = rdlane64(fv, 1);
  const uint64_t s0 = total * k / nch, s1 = total * (k + 1) / nch;
  if (cnt != s1 - s0 || cnt > slen - 272 || nb / 8 + (nb % 8 != 0) != slen - 272 - cnt) return kErrHeader;
  st.lengths = blk + off + 16;
  st.sm = blk + off + 272;
  st.bits = st.sm + cnt;
  st.nbits = nb;
  st.count = (uint32_t)cnt;
  st.start = (uint32_t)s0;
  return 0;
}

// Serial block: [u64 count][u64 bits][256 lengths][count sm][codes] [src/c_api.cpp:29-34, cuda/decode.cu:49-51]
__device__ uint32_t parse_serial(const uint8_t* blk, uint64_t size, const DevBlock& d, uint32_t lane, Stream& st) {
  const uint64_t rows = d.rows, cols = d.cols;
  if (size < 272 || !rows || !cols || cols > ~0ull / rows) return kErrHeader;
  const uint64_t fv = lane < 2 ? ldg64(blk + 8 * lane) : 0;
  const uint64_t cnt = rdlane64(fv, 0), nb = rdlane64(fv, 1);
  if (cnt != rows * cols || cnt > size - 272 || nb / 8 + (nb % 8 != 0) != size - 272 - cnt) return kErrHeader;
  if (cnt > kMaxBlockElems) return kErrShape;
  st.lengths = blk + 16;
  st.sm = blk + 272;
  st.bits = st.sm + cnt;
  st.nbits = nb;
  st.count = (uint32_t)cnt;
  st.start = 0;
  return 0;
}

// ------------------------------------------------------------ code tables

struct Book {
  uint32_t err;
  uint32_t maxlen;
  bool fast;
};

// Canonical codes [src/codec.cpp:11-29] in closed form: with codes
// left-aligned in 32 bits, the code of symbol s is the sum of 2^(32-l) over
// every symbol ordered before s by (length, symbol).  Group sums give
// C(l) = first code of length l; a symbol's code is C(l) + rank * 2^(32-l),
// rank = number of smaller symbols of the same length.  The assignment is
// oversubscribed (the reference throws) iff the Kraft total exceeds 2^32.
__device__ Book build_fast(Smem& S, uint32_t lane, uint32_t L0, uint32_t L1, uint32_t L2, uint32_t L3,
                           uint32_t maxlen) {
  FastTables& F = S.t.f;
  uint16_t* compact = reinterpret_cast<uint16_t*>(S.syms);  // (len << 8) | symbol, symbol order
  uint8_t* rank = S.syms + 512;
  const uint32_t nz = (L0 != 0) + (L1 != 0) + (L2 != 0) + (L3 != 0);
  const uint32_t incl = wave_incl(nz, lane);
  const uint32_t m = rdlane(incl, kWave - 1);
  uint32_t k = incl - nz;
  if (L0) compact[k++] = (uint16_t)((L0 << 8) | (4 * lane));
  if (L1) compact[k++] = (uint16_t)((L1 << 8) | (4 * lane + 1));
  if (L2) compact[k++] = (uint16_t)((L2 << 8) | (4 * lane + 2));
  if (L3) compact[k++] = (uint16_t)((L3 << 8) | (4 * lane + 3));
  if (lane < 40) F.cnt[lane] = 0;
  for (uint32_t s0 = 0; s0 < m; s0 += kWave) {
    const uint32_t t = s0 + lane;
    const bool valid = t < m;
    if (lane < 40) F.slots[lane] = 0;
    __syncthreads();
    const uint32_t ent = valid ? compact[t] : 0u;
    const uint32_t l = ent >> 8;
    if (valid) atomicOr(reinterpret_cast<unsigned long long*>(&F.slots[l]), 1ull << lane);
    __syncthreads();
    const uint64_t mk = valid ? F.slots[l] : 0ull;
    const uint32_t rin = mbcnt(mk);
    const uint32_t r = valid ? rin + F.cnt[l] : 0u;
    __syncthreads();
    if (valid && rin == 0) F.cnt[l] += (uint32_t)__popcll(mk);
    if (valid) rank[t] = (uint8_t)r;
  }
  __syncthreads();
  // Per-length group sums: C(l+1) = sum_{l' <= l} cnt[l'] * 2^(32 - l').
  const uint32_t c = (lane >= 1 && lane <= 32) ? F.cnt[lane] : 0u;
  const uint64_t g = (lane >= 1 && lane <= 32) ? ((uint64_t)c << (32 - lane)) : 0ull;
  const uint64_t cinc = wave_incl(g, lane);
  const uint32_t binc = wave_incl(c, lane);
  const uint64_t total = rdlane64(cinc, 32);
  if (lane <= 32) {
    F.lim[lane] = cinc;
    F.base[lane] = (uint16_t)(binc - c);
  }
  if (lane < 16) F.l4[lane] = 0;
  if (total > (1ull << 32)) return Book{kErrCodebook, maxlen, true};
  __syncthreads();
  for (uint32_t s0 = 0; s0 < m; s0 += kWave) {
    const uint32_t t = s0 + lane;
    if (t < m) {
      const uint32_t ent = compact[t], l = ent >> 8, sym = ent & 255u, r = rank[t];
      const uint64_t code = F.lim[l - 1] + ((uint64_t)r << (32 - l));
      S.sorted[F.base[l] + r] = (uint8_t)sym;
      if (l <= 4) {
        const uint32_t e0 = (uint32_t)(code >> 28), n = 1u << (4 - l);
        for (uint32_t i = 0; i < n; ++i) F.l4[e0 + i] = (uint16_t)((l << 8) | sym);
      }
    }
  }
  __syncthreads();
  {  // codes of <= 4 bits cover whole 64-entry blocks of the 10-bit LUT
    const uint32_t e4 = F.l4[lane >> 2];
    const uint32_t pair = e4 | (e4 << 16);
    const uint4 v = make_uint4(pair, pair, pair, pair);
    *reinterpret_cast<uint4*>(&F.lut[16 * lane]) = v;
    *reinterpret_cast<uint4*>(&F.lut[16 * lane + 8]) = v;
  }
  __syncthreads();
  for (uint32_t s0 = 0; s0 < m; s0 += kWave) {
    const uint32_t t = s0 + lane;
    if (t < m) {
      const uint32_t ent = compact[t], l = ent >> 8, sym = ent & 255u, r = rank[t];
      if (l >= 5 && l <= kLutBits) {
        const uint64_t code = F.lim[l - 1] + ((uint64_t)r << (32 - l));
        const uint32_t e0 = (uint32_t)(code >> (32 - kLutBits)), n = 1u << (kLutBits - l);
        for (uint32_t i = 0; i < n; ++i) F.lut[e0 + i] = (uint16_t)((l << 8) | sym);
      }
    }
  }
  __syncthreads();
  return Book{0, maxlen, true};
}

// Tables for codes longer than 32 bits (bit-serial path).  cnt/base/sorted
// as above; open[l] counts length-l prefixes that longer codes extend, so a
// prefix beyond them is an invalid code [src/codec.cpp:69 "invalid bitstream"].
__device__ Book build_slow(Smem& S, uint32_t lane, const uint8_t* lengths, uint32_t maxlen) {
  SlowTables& T = S.t.s;
  uint8_t* lens = S.syms + 1024;
  reinterpret_cast<uint32_t*>(lens)[lane] = ldg32(lengths + 4 * lane);
  for (uint32_t i = lane; i < 256; i += kWave) T.cnt[i] = 0;
  __syncthreads();
#pragma unroll
  for (uint32_t q = 0; q < 4; ++q) {
    const uint32_t l = lens[4 * lane + q];
    if (l) atomicAdd(&T.cnt[l], 1u);
  }
  __syncthreads();
  if (lane == 0) {
    uint32_t err = 0, free = 2, b = 0;
    for (uint32_t l = 1; l < 256; ++l) {
      const uint32_t c = T.cnt[l];
      if (c > free) err = kErrCodebook;
      T.base[l] = (uint16_t)b;
      T.cursor[l] = (uint16_t)b;
      b += c;
      free = c > free ? 0 : 2 * (free - c);
      if (free > 1024) free = 1024;
    }
    uint32_t op = 0;
    for (uint32_t l = 255; l >= 1; --l) {
      T.open[l] = (uint16_t)op;
      op = (T.cnt[l] + op + 1) >> 1;
    }
    for (uint32_t s = 0; s < 256; ++s) {
      const uint32_t l = lens[s];
      if (l) S.sorted[T.cursor[l]++] = (uint8_t)s;
    }
    S.bcast[0] = err;
  }
  __syncthreads();
  return Book{S.bcast[0], maxlen, false};
}

__device__ Book build_book(Smem& S, uint32_t lane, const uint8_t* lengths) {
  const uint32_t lw = ldg32(lengths + 4 * lane);
  const uint32_t L0 = lw & 255u, L1 = (lw >> 8) & 255u, L2 = (lw >> 16) & 255u, L3 = lw >> 24;
  const uint32_t mx = max(max(L0, L1), max(L2, L3));
  const uint32_t maxlen = wave_max(mx);
  if (maxlen > kMaxLenFast) return build_slow(S, lane, lengths, maxlen);
  return build_fast(S, lane, L0, L1, L2, L3, maxlen);
}

// ---------------------------------------------------------------- decode

// Codes longer than the LUT: find the length group holding window w.
__device__ __forceinline__ uint32_t long_code(const Smem& S, uint32_t w, uint32_t maxlen) {
  const FastTables& F = S.t.f;
  uint32_t l = kLutBits + 1;
  while (l <= maxlen && (uint64_t)w >= F.lim[l]) ++l;
  if (l > maxlen) return 0;
  const uint64_t first = F.lim[l - 1];
  const uint32_t idx = F.base[l] + (uint32_t)(((uint64_t)w - first) >> (32 - l));
  return (l << 8) | S.sorted[idx];
}

// Decode codewords starting in [from, ce) (bits relative to the segment).
// Symbols go to the lane's scratch region; `mask` records codeword starts
// within [cs, cs + 32); `dead` marks a window that matches no code.
__device__ __forceinline__ void run_chunk(const Smem& S, uint32_t from, uint32_t cs, uint32_t ce, uint8_t* region,
                                          uint32_t maxlen, uint32_t& cnt, uint32_t& ex, uint32_t& mask,
                                          uint32_t& dead) {
  uint32_t p = from, c = 0, m = 0, d = 0;
  while (p < ce) {
    const uint32_t i = (p + 31) >> 5;
    const uint32_t w = __builtin_amdgcn_alignbit(S.stream[i], S.stream[i + 1], 0u - p);
    uint32_t e = S.t.f.lut[w >> (32 - kLutBits)];
    if (e == 0) {
      e = long_code(S, w, maxlen);
      if (e == 0) {
        d = 1;
        break;
      }
    }
    const uint32_t rel = p - cs;
    if (rel < 32) m |= 1u << rel;
    region[c++] = (uint8_t)e;
    p += e >> 8;
  }
  cnt = c;
  ex = p;
  mask = m;
  dead = d;
}

// Decode one stream with the fast tables; the consumer receives the
// exponents in stream order.  Returns error bits.
template <class Cons>
__device__ uint32_t decode_fast(Smem& S, uint32_t lane, const Stream& st, uint32_t maxlen, const uint8_t* blk_end,
                                Cons& C) {
  const uint64_t nbits = st.nbits;
  const uint8_t* bend = st.bits + ((nbits + 7) >> 3);
  if (bend > blk_end) bend = blk_end;
  uint8_t* const region = S.syms + kCarry + lane * kRegion;
  uint32_t carry = 0, pos0 = 0, entry = 0, err = 0;
  uint64_t S0 = 0, true_pos = 0;
  if (lane == 0) S.stream[0] = 0;
  while (true_pos < nbits) {
    if (lane < kStreamLanes) {
      const uint4 v = ldg16_bounded(st.bits + (S0 >> 3) + 16 * lane, bend);
      uint32_t* w = &S.stream[1 + 4 * lane];
      w[0] = bswap32(v.x);
      w[1] = bswap32(v.y);
      w[2] = bswap32(v.z);
      w[3] = bswap32(v.w);
    }
    __syncthreads();
    const uint64_t left = nbits - S0;
    const uint32_t lim_bits = left < kSegBits ? (uint32_t)left : kSegBits;
    const uint32_t cs = lane * kChunk;
    const bool active = cs < lim_bits;
    const uint32_t ce = active ? min(cs + kChunk, lim_bits) : cs;
    uint32_t start = cs, cnt = 0, ex = cs, mask = 0, dead = 0;
    if (active) run_chunk(S, cs, cs, ce, region, maxlen, cnt, ex, mask, dead);
    // Resolve: lane i is consistent when its predecessor's exit is a
    // codeword start on lane i's path.  Lanes before the first
    // inconsistent lane are on the true path.
    for (;;) {
      uint32_t pe = __shfl_up(ex, 1, kWave), pd = __shfl_up(dead, 1, kWave);
      if (lane == 0) {
        pe = entry;
        pd = 0;
      }
      const uint32_t off = pe - cs;
      const bool ok = !active || (!pd && (pe == start || (off < 32 && ((mask >> off) & 1u))));
      const uint64_t bad = __ballot(!ok);
      const uint64_t deadm = __ballot(active && dead);
      const uint64_t resolved = bad ? ((1ull << (__ffsll((unsigned long long)bad) - 1)) - 1) : ~0ull;
      if (deadm & resolved) {
        err = kErrStream;
        break;
      }
      if (!bad) break;
      if (!ok && !pd) {
        start = pe;
        run_chunk(S, pe, cs, ce, region, maxlen, cnt, ex, mask, dead);
      }
    }
    if (err) break;
    uint32_t pe = __shfl_up(ex, 1, kWave);
    if (lane == 0) pe = entry;
    const uint32_t off = pe - cs;
    const uint32_t skip = (active && off < 32) ? (uint32_t)__popc(mask & ((1u << off) - 1u)) : 0u;
    const uint32_t t = active ? cnt - skip : 0u;
    const uint32_t tinc = wave_incl(t, lane);
    const uint32_t total = rdlane(tinc, kWave - 1);
    const uint64_t act = __ballot(active);
    const uint32_t last = 63u - (uint32_t)__clzll((long long)act);
    const uint32_t seg_exit = rdlane(ex, last);
    if ((uint64_t)pos0 + carry + total > st.count) {
      err = kErrStream;  // more codewords than elements: trailing bits
      break;
    }
    // Compact the lanes' runs behind the carried partial tile.
    {
      const uint32_t dst = carry + tinc - t;
      const uint32_t nd = (t + 3) >> 2, ndmax = wave_max(nd);
      const uint32_t nfull = t >> 2, tail = t & 3u;
      uint32_t R[kChunk / 4];
#pragma unroll
      for (uint32_t q = 0; q < kChunk / 4; ++q) {
        if (q >= ndmax) break;
        R[q] = q < nd ? lds32(region + skip + 4 * q) : 0u;
      }
      __syncthreads();
#pragma unroll
      for (uint32_t q = 0; q < kChunk / 4; ++q) {
        if (q >= ndmax) break;
        uint8_t* p = S.syms + dst + 4 * q;
        if (q < nfull) {
          sts32(p, R[q]);
        } else if (q == nfull && tail) {
          p[0] = (uint8_t)R[q];
          if (tail > 1) p[1] = (uint8_t)(R[q] >> 8);
          if (tail > 2) p[2] = (uint8_t)(R[q] >> 16);
        }
      }
      __syncthreads();
    }
    const uint32_t avail = carry + total;
    const uint32_t take = C.consume(S, lane, st, pos0, avail, false);
    const uint32_t rem = avail - take;
    if (take && rem) {  // take is a multiple of 256 here, so source and destination do not overlap
      const uint32_t v = 4 * lane < rem ? lds32(S.syms + take + 4 * lane) : 0u;
      __syncthreads();
      if (4 * lane < rem) sts32(S.syms + 4 * lane, v);
    }
    __syncthreads();
    carry = rem;
    pos0 += take;
    true_pos = S0 + seg_exit;
    entry = seg_exit - kSegBits;
    S0 += kSegBits;
  }
  if (!err) {
    if (true_pos != nbits || (uint64_t)pos0 + carry != st.count) err = kErrStream;
    else if (carry) C.consume(S, lane, st, pos0, carry, true);
  }
  return err;
}

// Bit-serial canonical decode for codes longer than 32 bits: lane 0 walks
// the code one bit at a time (d = offset from the first code of the current
// length); the consumer sees the symbols kSlowSeg at a time.
template <class Cons>
__device__ uint32_t decode_slow(Smem& S, uint32_t lane, const Stream& st, Cons& C) {
  const SlowTables& T = S.t.s;
  const uint64_t nbits = st.nbits;
  uint64_t pos = 0;
  uint32_t produced = 0, err = 0;
  while (produced < st.count) {
    const uint32_t nseg = min(kSlowSeg, st.count - produced);
    if (lane == 0) {
      uint32_t e = 0;
      for (uint32_t i = 0; i < nseg && !e; ++i) {
        if (pos >= nbits) { e = kErrStream; break; }
        uint32_t d = (st.bits[pos >> 3] >> (7 - (pos & 7))) & 1u;
        ++pos;
        for (uint32_t l = 1;; ++l) {
          if (d < T.cnt[l]) {
            S.syms[i] = S.sorted[T.base[l] + d];
            break;
          }
          d -= T.cnt[l];
          if (d >= T.open[l] || l >= 255 || pos >= nbits) { e = kErrStream; break; }
          d = 2 * d + ((st.bits[pos >> 3] >> (7 - (pos & 7))) & 1u);
          ++pos;
        }
      }
      S.bcast[0] = e;
    }
    __syncthreads();
    err = S.bcast[0];
    __syncthreads();
    if (err) break;
    C.consume(S, lane, st, produced, nseg, produced + nseg == st.count);
    __syncthreads();
    produced += nseg;
  }
  if (lane == 0) S.bcast[1] = (pos == nbits);
  __syncthreads();
  if (!err && !S.bcast[1]) err = kErrStream;
  __syncthreads();
  return err;
}

template <class Cons>
__device__ uint32_t decode_stream(Smem& S, uint32_t lane, const Stream& st, const uint8_t* blk_end, Cons& C) {
  const Book b = build_book(S, lane, st.lengths);
  if (b.err) return b.err;
  return b.fast ? decode_fast(S, lane, st, b.maxlen, blk_end, C) : decode_slow(S, lane, st, C);
}

// ------------------------------------------------------------- consumers

// Unit = 8 consecutive tiled positions = half a tile row.  A stream is
// "unit-aligned" when its slab has full 16x16 tiles and the stream starts and
// ends on unit boundaries; then unit u holds row (u/2)%16, columns 16*(u/32)+8*(u%2).
__device__ __forceinline__ bool unit_aligned(const Stream& st, uint64_t rows, uint64_t cols) {
  return rows % 16 == 0 && cols % 16 == 0 && st.start % 8 == 0 && st.count % 8 == 0;
}

// BF16 writer, unit-aligned streams: 16-byte stores of whole half tile rows.
struct WriterAligned {
  uint8_t* out;  // slab base
  uint32_t cols, tpb;
  __device__ uint32_t consume(Smem& S, uint32_t lane, const Stream& st, uint32_t pos0, uint32_t avail, bool final) {
    const uint32_t take = final ? avail : (avail & ~255u);
    const uint32_t units = take >> 3;
    const uint32_t U0 = (st.start + pos0) >> 3;
    for (uint32_t u = lane; u < units; u += kWave) {
      uint64_t E;
      __builtin_memcpy(&E, S.syms + 8 * u, 8);
      const uint64_t M = ldg64(st.sm + pos0 + 8 * u);
      const uint4 w = combine8(E, M);
      const uint32_t U = U0 + u, T = U >> 5;
      const uint32_t band = T / tpb;
      const uint64_t row = 16ull * band + ((U >> 1) & 15u);
      const uint64_t col = 16ull * (T - band * tpb) + 8u * (U & 1u);
      __builtin_memcpy(out + (row * cols + col) * 2, &w, 16);
    }
    return take;
  }
};

// BF16 writer, any shape: one element per lane per step.
struct WriterGeneric {
  uint8_t* out;
  uint64_t rows, cols;
  __device__ uint32_t consume(Smem& S, uint32_t lane, const Stream& st, uint32_t pos0, uint32_t avail, bool) {
    for (uint32_t i = lane; i < avail; i += kWave) {
      const uint32_t P = pos0 + i;
      const uint32_t e = S.syms[i], s = st.sm[P];
      const uint16_t w = (uint16_t)(((s & 0x80u) << 8) | (e << 7) | (s & 0x7fu));
      uint64_t row, col;
      tile_to_rc((uint64_t)st.start + P, rows, cols, row, col);
      __builtin_memcpy(out + (row * cols + col) * 2, &w, 2);
    }
    return avail;
  }
};

// Fused GEMM/GEMV over one unit-aligned stream of a 16-row slab, fp32
// activations X[c * ldx + j] (cuda/decode.cu:94 layout, batch columns
// j < nb).  Every lane keeps one row: unit u = lane + 64 i has row
// ((U0 + u) / 2) % 16, which does not depend on i.
template <int NB>
struct GemmF32 {
  const float* x;
  uint64_t ldx;
  uint32_t nb;
  float acc[NB];
  __device__ void init() {
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = 0.f;
  }
  __device__ uint32_t consume(Smem& S, uint32_t lane, const Stream& st, uint32_t pos0, uint32_t avail, bool final) {
    const uint32_t take = final ? avail : (avail & ~255u);
    const uint32_t units = take >> 3;
    const uint32_t U0 = (st.start + pos0) >> 3;
    for (uint32_t u = lane; u < units; u += kWave) {
      uint64_t E;
      __builtin_memcpy(&E, S.syms + 8 * u, 8);
      const uint64_t M = ldg64(st.sm + pos0 + 8 * u);
      const uint4 w = combine8(E, M);
      const uint32_t U = U0 + u;
      const uint64_t col = 16ull * (U >> 5) + 8u * (U & 1u);
      float f[8] = {bf_lo(w.x), bf_hi(w.x), bf_lo(w.y), bf_hi(w.y), bf_lo(w.z), bf_hi(w.z), bf_lo(w.w), bf_hi(w.w)};
      if (NB == 1) {
        float4 xa, xb;
        __builtin_memcpy(&xa, x + col, 16);
        __builtin_memcpy(&xb, x + col + 4, 16);
        acc[0] = fmaf(f[0], xa.x, acc[0]);
        acc[0] = fmaf(f[1], xa.y, acc[0]);
        acc[0] = fmaf(f[2], xa.z, acc[0]);
        acc[0] = fmaf(f[3], xa.w, acc[0]);
        acc[0] = fmaf(f[4], xb.x, acc[0]);
        acc[0] = fmaf(f[5], xb.y, acc[0]);
        acc[0] = fmaf(f[6], xb.z, acc[0]);
        acc[0] = fmaf(f[7], xb.w, acc[0]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float* xr = x + (col + i) * ldx;
#pragma unroll
          for (int j = 0; j < NB; ++j)
            if (j < (int)nb) acc[j] = fmaf(f[i], xr[j], acc[j]);
        }
      }
    }
    return take;
  }
  // Four lanes share each row: with s = (stream start / 8) % 2, lane l and
  // ((l + s) ^ 1) - s (mod 64) hold the two halves of a tile row, and l ^ 32
  // the same row two tiles on.  After the two exchanges all four hold the sum.
  __device__ void reduce(uint32_t lane, uint32_t s) {
    const int partner = (int)((((lane + s) ^ 1u) - s) & 63u);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      acc[j] += __shfl(acc[j], partner, kWave);
      acc[j] += __shfl_xor(acc[j], 32, kWave);
    }
  }
};

// ----------------------------------------------------------------- kernels

__device__ __forceinline__ void set_status(uint32_t* status, uint32_t slot, uint32_t err, uint32_t lane) {
  if (err && lane == 0) atomicOr(status + slot, err);
}

// Decode a list of blocks of one codec into BF16.  Task = (block, substream)
// for parallel blocks, = block for serial blocks.
__global__ void __launch_bounds__(64) k_decode(const DevBlock* __restrict__ blocks, uint32_t nblocks, uint32_t codec,
                                               const uint8_t* __restrict__ arc, uint8_t* __restrict__ out,
                                               uint32_t* __restrict__ status) {
  __shared__ Smem S;
  const uint32_t lane = lane_id();
  const uint32_t per = codec == kCodecParallel ? kMaxChunks : 1u;
  const uint64_t ntasks = (uint64_t)nblocks * per;
  for (uint64_t task = blockIdx.x; task < ntasks; task += gridDim.x) {
    const uint32_t b = (uint32_t)(task / per), k = (uint32_t)(task % per);
    const DevBlock d = blocks[b];
    const uint8_t* blk = arc + d.src;
    Stream st;
    uint32_t err, chunks = 1;
    if (codec == kCodecParallel) err = parse_parallel(blk, d.size, d, k, lane, st, chunks);
    else err = parse_serial(blk, d.size, d, lane, st);
    if (!err && k >= chunks) continue;
    if (!err) {
      if (unit_aligned(st, d.rows, d.cols)) {
        WriterAligned C{out + d.dst, (uint32_t)d.cols, (uint32_t)(d.cols / 16)};
        err = decode_stream(S, lane, st, blk + d.size, C);
      } else {
        WriterGeneric C{out + d.dst, d.rows, d.cols};
        err = decode_stream(S, lane, st, blk + d.size, C);
      }
    }
    set_status(status, d.status_slot, err, lane);
    __syncthreads();
  }
}

// Fused decode-GEMM for unit-aligned 16-row slabs, fp32 activations
// X[c * ldx + j], output Y[(dst + r) * ldy + j].  Parallel blocks combine
// their substreams' partial sums in substream order through `partial`
// (kMaxChunks x 16 x NB floats per block) and a per-block arrival counter
// that the last arriving wave resets, so the result is deterministic.
template <int NB>
__global__ void __launch_bounds__(64) k_gemm_f32(const DevBlock* __restrict__ blocks, uint32_t nblocks,
                                                 uint32_t codec, const uint8_t* __restrict__ arc,
                                                 const float* __restrict__ x, uint64_t ldx, uint32_t nb,
                                                 float* __restrict__ y, uint64_t ldy, uint32_t* __restrict__ status,
                                                 float* __restrict__ partial, uint32_t* __restrict__ counters) {
  __shared__ Smem S;
  const uint32_t lane = lane_id();
  const uint32_t per = codec == kCodecParallel ? kMaxChunks : 1u;
  const uint64_t ntasks = (uint64_t)nblocks * per;
  for (uint64_t task = blockIdx.x; task < ntasks; task += gridDim.x) {
    const uint32_t b = (uint32_t)(task / per), k = (uint32_t)(task % per);
    const DevBlock d = blocks[b];
    const uint8_t* blk = arc + d.src;
    Stream st;
    uint32_t err, chunks = 1;
    if (codec == kCodecParallel) err = parse_parallel(blk, d.size, d, k, lane, st, chunks);
    else err = parse_serial(blk, d.size, d, lane, st);
    if (codec == kCodecParallel && chunks == 0) {  // block-level header failure: no reduction
      set_status(status, d.status_slot, err, lane);
      continue;
    }
    if (k >= chunks) continue;
    GemmF32<NB> C{x, ldx, nb};
    C.init();
    if (!err && (d.rows != 16 || !unit_aligned(st, d.rows, d.cols))) err = kErrShape;
    if (!err) err = decode_stream(S, lane, st, blk + d.size, C);
    const uint32_t su = (st.start >> 3) & 1u;
    C.reduce(lane, su);
    set_status(status, d.status_slot, err, lane);
    // One holder lane per row: lanes < 32 with (lane + su) even hold slab row
    // ((start / 8 + lane) / 2) % 16, sixteen distinct rows.
    const uint32_t row = (((st.start >> 3) + lane) >> 1) & 15u;
    const bool holder = lane < 32 && ((lane + su) & 1u) == 0;
    if (codec != kCodecParallel) {
      if (holder && !err)
#pragma unroll
        for (int j = 0; j < NB; ++j)
          if (j < (int)nb) y[(d.dst + row) * ldy + j] = C.acc[j];
    } else {
      float* mine = partial + ((uint64_t)b * kMaxChunks + k) * 16 * NB;
      if (holder)
#pragma unroll
        for (int j = 0; j < NB; ++j) mine[row * NB + j] = err ? 0.f : C.acc[j];
      uint32_t old = 0;
      if (lane == 0)
        old = __hip_atomic_fetch_add(counters + b, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      old = rdlane(old, 0);
      if (old == chunks - 1) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        for (uint32_t idx = lane; idx < 16u * NB; idx += kWave) {
          const uint32_t r = idx / NB, j = idx % NB;
          float s = 0.f;
          for (uint32_t q = 0; q < chunks; ++q) s += partial[(((uint64_t)b * kMaxChunks + q) * 16 + r) * NB + j];
          if (j < nb) y[(d.dst + r) * ldy + j] = s;
        }
        if (lane == 0) __hip_atomic_store(counters + b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __syncthreads();
  }
}

// Raw blocks: byte copy archive -> output (decode) [src/compile.cpp:466-467].
__global__ void __launch_bounds__(256) k_copy_raw(const DevBlock* __restrict__ blocks, uint32_t nblocks,
                                                  const uint8_t* __restrict__ arc, uint8_t* __restrict__ out) {
  for (uint32_t b = blockIdx.y; b < nblocks; b += gridDim.y) {
    const DevBlock d = blocks[b];
    const uint8_t* src = arc + d.src;
    uint8_t* dst = out + d.dst;
    const uint64_t n16 = d.size / 16;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * blockDim.x) {
      uint4 v;
      __builtin_memcpy(&v, src + 16 * i, 16);
      __builtin_memcpy(dst + 16 * i, &v, 16);
    }
    const uint64_t tail = d.size - 16 * n16;
    if (blockIdx.x == 0 && threadIdx.x < tail) dst[16 * n16 + threadIdx.x] = src[16 * n16 + threadIdx.x];
  }
}

// Plain GEMM over BF16 matrices already in device memory (raw archive blocks,
// or blocks decoded to scratch when they are not unit-aligned):
// Y[(dst + r) * ldy + j] = sum_c W[r, c] X[c * ldx + j].  One wave per row;
// lanes stride the columns in order and reduce in a fixed tree.
__global__ void __launch_bounds__(64) k_gemm_plain(const DevBlock* __restrict__ blocks, uint32_t nblocks,
                                                   const uint8_t* __restrict__ base, const float* __restrict__ x,
                                                   uint64_t ldx, uint32_t nb, float* __restrict__ y, uint64_t ldy) {
  const uint32_t lane = lane_id();
  for (uint32_t b = blockIdx.y; b < nblocks; b += gridDim.y) {
    const DevBlock d = blocks[b];
    for (uint64_t r = blockIdx.x; r < d.rows; r += gridDim.x) {
      const uint8_t* wrow = base + d.src + r * d.cols * 2;
      for (uint32_t j0 = 0; j0 < nb; j0 += 4) {
        float a[4] = {0.f, 0.f, 0.f, 0.f};
        for (uint64_t c = lane; c < d.cols; c += kWave) {
          uint16_t h;
          __builtin_memcpy(&h, wrow + 2 * c, 2);
          const float w = __uint_as_float((uint32_t)h << 16);
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j)
            if (j0 + j < nb) a[j] = fmaf(w, x[c * ldx + j0 + j], a[j]);
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
#pragma unroll
          for (uint32_t dd = kWave / 2; dd >= 1; dd >>= 1) a[j] += __shfl_xor(a[j], dd, kWave);
          if (lane == 0 && j0 + j < nb) y[(d.dst + r) * ldy + j0 + j] = a[j];
        }
      }
    }
  }
}

__global__ void k_fill_u32(uint32_t* p, uint64_t n, uint32_t v) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

}  // namespace

// ----------------------------------------------------------- host launchers

static unsigned grid_for(uint64_t tasks, unsigned cap) {
  return (unsigned)(tasks < cap ? (tasks ? tasks : 1) : cap);
}

hipError_t launch_decode(const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc, uint8_t* out,
                         uint32_t* status, unsigned max_groups, hipStream_t s) {
  if (!nblocks) return hipSuccess;
  const uint64_t tasks = (uint64_t)nblocks * (codec == kCodecParallel ? kMaxChunks : 1u);
  hipLaunchKernelGGL(k_decode, dim3(grid_for(tasks, max_groups)), dim3(64), 0, s, blocks, nblocks, codec, arc, out,
                     status);
  return hipGetLastError();
}

hipError_t launch_gemm_f32(const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc,
                           const float* x, uint64_t ldx, uint32_t nb, float* y, uint64_t ldy, uint32_t* status,
                           float* partial, uint32_t* counters, unsigned max_groups, hipStream_t s) {
  if (!nblocks) return hipSuccess;
  const uint64_t tasks = (uint64_t)nblocks * (codec == kCodecParallel ? kMaxChunks : 1u);
  const dim3 g(grid_for(tasks, max_groups)), blk(64);
  if (nb == 1)
    hipLaunchKernelGGL(k_gemm_f32<1>, g, blk, 0, s, blocks, nblocks, codec, arc, x, ldx, nb, y, ldy, status, partial,
                       counters);
  else if (nb <= 4)
    hipLaunchKernelGGL(k_gemm_f32<4>, g, blk, 0, s, blocks, nblocks, codec, arc, x, ldx, nb, y, ldy, status, partial,
                       counters);
  else if (nb <= 8)
    hipLaunchKernelGGL(k_gemm_f32<8>, g, blk, 0, s, blocks, nblocks, codec, arc, x, ldx, nb, y, ldy, status, partial,
                       counters);
  else
    hipLaunchKernelGGL(k_gemm_f32<16>, g, blk, 0, s, blocks, nblocks, codec, arc, x, ldx, nb, y, ldy, status,
                       partial, counters);
  return hipGetLastError();
}

hipError_t launch_copy_raw(const DevBlock* blocks, uint32_t nblocks, const uint8_t* arc, uint8_t* out, hipStream_t s) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(k_copy_raw, dim3(64, nblocks < 1024 ? nblocks : 1024), dim3(256), 0, s, blocks, nblocks, arc,
                     out);
  return hipGetLastError();
}

hipError_t launch_gemm_plain(const DevBlock* blocks, uint32_t nblocks, const uint8_t* base, const float* x,
                             uint64_t ldx, uint32_t nb, float* y, uint64_t ldy, hipStream_t s) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(k_gemm_plain, dim3(256, nblocks < 256 ? nblocks : 256), dim3(64), 0, s, blocks, nblocks, base, x,
                     ldx, nb, y, ldy);
  return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t* p, uint64_t n, uint32_t v, hipStream_t s) {
  if (!n) return hipSuccess;
  const uint64_t g = (n + 255) / 256;
  hipLaunchKernelGGL(k_fill_u32, dim3(g < 1024 ? (unsigned)g : 1024u), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

}  // namespace xksv
