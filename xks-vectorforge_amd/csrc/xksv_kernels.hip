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
// 96-bit chunk.  Lane 0 starts at the segment's true entry; every other lane
// starts decoding kSync bits before its chunk and drops what precedes the
// chunk: Huffman codes resynchronise within a few codewords, so the lane's
// first codeword start inside its chunk almost always equals the previous
// lane's exit, which proves the lane is on the true path; a lane where it
// does not re-decodes from that exit.  A wave prefix sum places each lane's
// symbols; the run is compacted in LDS and handed to a consumer (BF16 writer,
// fused GEMV, fused GEMM) a whole 16x16 tile at a time.
// With a codeword index (a load-time sidecar of static weights: the bit
// offset of every 32nd codeword), lane l instead starts at the recorded
// offset of symbol 32 l of each 2,048-symbol segment and decodes exactly 32
// symbols into its own slot; the offsets are checked as they are used (every
// lane must end where the next one starts), so an index that does not match
// the stream only sends the segment back to the speculative path.
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
constexpr uint32_t kSync = 24;                      // bits decoded before a chunk to synchronise
constexpr uint32_t kRegion = kChunk + 4;            // lane symbol stride: 25 dwords, odd -> conflict-free
constexpr uint32_t kSegBits = kWave * kChunk;       // 6144 bits per segment
constexpr uint32_t kCarry = 256;                    // room for an unconsumed partial tile
constexpr uint32_t kSymsBytes = kCarry + kWave * kRegion;
constexpr uint32_t kStreamDw = kSegBits / 32 + 2;   // segment dwords plus lookahead
constexpr uint32_t kStreamLanes = (kStreamDw + 3) / 4;
constexpr uint32_t kLutBits = 10;
constexpr uint32_t kLongLen = 127;
constexpr uint32_t kLongMark = kLongLen << 8;
constexpr uint32_t kMaxLenFast = 32;
constexpr uint32_t kSlowSeg = 4096;                 // symbols per bit-serial segment (multiple of 256)
constexpr uint64_t kMagicXKSP2 = 0x0000003250534B58ull;  // "XKSP2\0\0\0" little-endian
constexpr uint32_t kSerialWaves = 12;               // waves per serial block (workgroup-scale decode)
// Longest segment of an indexed item (fused GEMM codeword index), in code
// bits: the segment, its start's bit offset within its first byte, the
// register window's lookahead (96 bits) and a dead path's jump (kLongLen)
// stay inside the 6,272 staged bits.
constexpr uint32_t kIdxMaxSpan = kStreamLanes * 128 - 7 - 96 - kLongLen - 32;

// Every function that takes the LDS block by reference is force-inlined: the
// compiler then addresses it with DS instructions.  Through a call it would
// become a generic pointer and FLAT instructions, which fault on LDS
// addresses that are not naturally aligned (merged narrow stores can be).
//
// Per-wave LDS.  The table area is either the fast tables (LUT + per-length
// limits) or the bit-serial tables; rank/compaction scratch lives in `syms`
// before decoding starts.
// Two-symbol lookup entry for a 10-bit window: bits 0-7 first symbol, 8-14
// bits consumed, 15 second symbol present, 16-23 second symbol, 24-27 length
// of the first code.  The two symbols sit in the bytes a byte store and a
// high-half byte store write.  A window whose first code is longer than 10
// bits (or matches no code) holds kLongMark; the step resolves it on the spot.
struct FastTables {
  uint32_t lut2[1u << kLutBits];
  uint64_t lim[40];              // lim[l] = left-aligned 32-bit end of the length-l codes, C(l+1)
  uint64_t slots[40];            // per-length lane masks (rank computation)
  uint32_t cnt[40];              // codes per length
  uint16_t base[40];             // index of the first length-l symbol in `sorted`
  uint16_t l4[16];               // codes of <= 4 bits, indexed by the top 4 bits
};
// The one-symbol table (1,024 words, lut1_entry per code of at most 10
// bits, kLongMark elsewhere) lives in the symbol buffer while the tables are
// built.
constexpr uint32_t kLut1Off = 1024;
// One-symbol entry: symbol in bits 0-7 and 16-23, length in bits 8-14,
// 24-27 and 28-31 (the last copy is the shift that skips the code).
__host__ __device__ constexpr uint32_t lut1_entry(uint32_t len, uint32_t sym) {
  return sym | (len << 8) | (sym << 16) | (len << 24) | (len << 28);
}
static_assert(kLut1Off + 4 * (1u << kLutBits) <= kSymsBytes, "one-symbol table must fit the symbol buffer");
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
// X columns of one indexed segment, staged for the fused GEMM consumers: in
// the symbol buffer past the lane slots of the segment's symbols.
// Lane slots of the indexed walk: kIdxLaneSyms symbols, then padding (a
// lone symbol's second byte may land in it); 9 dwords, odd, so that lanes
// storing their n-th symbol together hit distinct LDS banks.
constexpr uint32_t kIdxStride = kIdxLaneSyms + 4;
static_assert(kIdxStride % 8 == 4, "indexed lane slots: odd dword stride");
constexpr uint32_t kXOff = kWave * kIdxStride;
constexpr uint32_t kXBytes = 4096;
static_assert(kXOff + kXBytes <= kSymsBytes, "staged X must fit the symbol buffer");
// Index segments (64 u16 entries each) copied to LDS ahead of their use, two
// buffers (segment sg in buffer sg % 2): past the staged X and the tables'
// scratch, so the first lands while the tables are built.
constexpr uint32_t kIxOff = kXOff + kXBytes;
static_assert(kIxOff + 256 <= kSymsBytes && kIxOff >= kLut1Off + 4 * (1u << kLutBits) && kIxOff % 16 == 0,
              "index entries must fit the symbol buffer beside the tables' scratch");

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
// Wave64 scans and reductions with DPP row shifts and row broadcasts
// (6 DPP operations per 32-bit scan).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return __builtin_amdgcn_update_dpp(0u, v, CTRL, ROW_MASK, 0xf, true);
}
__device__ __forceinline__ uint32_t wave_incl(uint32_t v, uint32_t) {
  v += dpp<0x111>(v);
  v += dpp<0x112>(v);
  v += dpp<0x114>(v);
  v += dpp<0x118>(v);
  v += dpp<0x142, 0xa>(v);
  v += dpp<0x143, 0xc>(v);
  return v;
}
__device__ __forceinline__ uint64_t wave_incl(uint64_t v, uint32_t) {
#define XKSV_STEP64(C, RM)                                                               \
  {                                                                                      \
    const uint32_t lo = dpp<C, RM>((uint32_t)v), hi = dpp<C, RM>((uint32_t)(v >> 32)); \
    v += ((uint64_t)hi << 32) | lo;                                                      \
  }
  XKSV_STEP64(0x111, 0xf) XKSV_STEP64(0x112, 0xf) XKSV_STEP64(0x114, 0xf) XKSV_STEP64(0x118, 0xf)
  XKSV_STEP64(0x142, 0xa) XKSV_STEP64(0x143, 0xc)
#undef XKSV_STEP64
  return v;
}
// Maximum over the wave (unsigned), broadcast to every lane.
__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
  v = max(v, dpp<0x111>(v));
  v = max(v, dpp<0x112>(v));
  v = max(v, dpp<0x114>(v));
  v = max(v, dpp<0x118>(v));
  v = max(v, dpp<0x142, 0xa>(v));
  v = max(v, dpp<0x143, 0xc>(v));
  return __builtin_amdgcn_readlane(v, 63);
}
// Value of lane - 1 (0 for lane 0).
__device__ __forceinline__ uint32_t from_prev_lane(uint32_t v) { return dpp<0x138>(v); }
// Orders this wave's LDS accesses across lanes: LDS executes a wave's
// operations in issue order, so a compiler fence is all a wave needs.  The
// per-stream engine synchronises only within its wave (several waves of one
// workgroup run independent streams and reach different numbers of these).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
// 16 bytes at p with the bytes at or past `end` reading as zero, in two
// halves so that issuing the load does not wait for it: fetch16() issues one
// 16-byte load that never crosses `end` (near the end it reads the 16 bytes
// before `end`) and records how many leading bytes to drop; value() shifts
// them out once the data is needed.  Callers guarantee [end - 16, end) is
// inside the same buffer (every segment holds 272 header bytes before its
// code bytes).
struct Fetch16 {
  uint4 v;
  uint32_t drop;  // leading bytes to drop; 16 = none of the bytes are wanted
  __device__ __forceinline__ uint4 value() const {
    // The 16 bytes as a 128-bit little-endian value shifted right by 8 drop bits.
    const uint32_t sh = 8u * drop;
    const uint64_t lo = (uint64_t)v.x | ((uint64_t)v.y << 32), hi = (uint64_t)v.z | ((uint64_t)v.w << 32);
    uint64_t olo, ohi;
    if (sh >= 64) {
      olo = sh >= 128 ? 0ull : hi >> (sh - 64);
      ohi = 0ull;
    } else {
      olo = sh ? (lo >> sh) | (hi << (64 - sh)) : lo;
      ohi = hi >> sh;
    }
    return make_uint4((uint32_t)olo, (uint32_t)(olo >> 32), (uint32_t)ohi, (uint32_t)(ohi >> 32));
  }
};
__device__ __forceinline__ Fetch16 fetch16(const uint8_t* p, const uint8_t* end) {
  Fetch16 f;
  if (p >= end) {
    f.v = make_uint4(0u, 0u, 0u, 0u);
    f.drop = 16;
    return f;
  }
  const uint8_t* q = p + 16 <= end ? p : end - 16;
  __builtin_memcpy(&f.v, q, 16);
  f.drop = (uint32_t)(p - q);
  return f;
}
__device__ __forceinline__ uint32_t lds32(const uint8_t* p) {
  uint32_t v;
  __builtin_memcpy(&v, p, 4);
  return v;
}
__device__ __forceinline__ void sts32(uint8_t* p, uint32_t v) { __builtin_memcpy(p, &v, 4); }
// Byte stores into LDS that the compiler must keep as single-byte DS stores
// (merged neighbours would be misaligned wider stores).  The explicit LDS
// address space keeps them DS instructions: a volatile generic pointer would
// become FLAT.
typedef __attribute__((address_space(3))) volatile uint8_t* lds_bytes;
__device__ __forceinline__ lds_bytes as_lds(uint8_t* p) { return (lds_bytes)p; }
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
// 32-bit arithmetic: rows * cols < 2^31 on the device path.
__device__ __forceinline__ void tile_to_rc(uint32_t q, uint32_t rows, uint32_t cols, uint32_t& row, uint32_t& col) {
  uint32_t band = 0, local = q, nr = rows;
  if (rows > 16) {  // 16 * cols <= rows * cols here
    const uint32_t bsz = 16u * cols;
    band = q / bsz;
    local = q - band * bsz;
    nr = min(16u, rows - 16u * band);
  }
  const uint32_t tsz = nr * 16u;
  const uint32_t t = local / tsz;
  const uint32_t lt = local - t * tsz;
  const uint32_t width = min(16u, cols - 16u * t);
  const uint32_t r = width == 16 ? (lt >> 4) : lt / width;
  row = 16u * band + r;
  col = 16u * t + (lt - r * width);
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
__device__ __forceinline__ Book build_fast(Smem& S, uint32_t lane, uint32_t L0, uint32_t L1, uint32_t L2, uint32_t L3,
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
  // One symbol per lane (m <= 64, the usual case): its entry and rank stay in
  // registers for the passes below.
  uint32_t ent0 = 0, r0 = 0;
  if (m <= kWave) {
    const bool valid = lane < m;
    if (lane < 40) F.slots[lane] = 0;
    wave_sync();
    ent0 = valid ? compact[lane] : 0u;
    const uint32_t l = ent0 >> 8;
    if (valid) atomicOr(reinterpret_cast<unsigned long long*>(&F.slots[l]), 1ull << lane);
    wave_sync();
    const uint64_t mk = valid ? F.slots[l] : 0ull;
    r0 = valid ? mbcnt(mk) : 0u;
    if (valid && r0 == 0) F.cnt[l] = (uint32_t)__popcll(mk);
  } else {
    for (uint32_t s0 = 0; s0 < m; s0 += kWave) {
      const uint32_t t = s0 + lane;
      const bool valid = t < m;
      if (lane < 40) F.slots[lane] = 0;
      wave_sync();
      const uint32_t ent = valid ? compact[t] : 0u;
      const uint32_t l = ent >> 8;
      if (valid) atomicOr(reinterpret_cast<unsigned long long*>(&F.slots[l]), 1ull << lane);
      wave_sync();
      const uint64_t mk = valid ? F.slots[l] : 0ull;
      const uint32_t rin = mbcnt(mk);
      const uint32_t r = valid ? rin + F.cnt[l] : 0u;
      wave_sync();
      if (valid && rin == 0) F.cnt[l] += (uint32_t)__popcll(mk);
      if (valid) rank[t] = (uint8_t)r;
    }
  }
  wave_sync();
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
  wave_sync();
  uint32_t rl = 0, rs = 0, re0 = 0;  // this lane's code of the first round (t = lane): length, symbol, 10-bit start
  for (uint32_t s0 = 0; s0 < m; s0 += kWave) {
    const uint32_t t = s0 + lane;
    if (t < m) {
      const bool one = m <= kWave;
      const uint32_t ent = one ? ent0 : compact[t], l = ent >> 8, sym = ent & 255u, r = one ? r0 : rank[t];
      const uint64_t code = F.lim[l - 1] + ((uint64_t)r << (32 - l));
      if (s0 == 0) {
        rl = l;
        rs = sym;
        re0 = (uint32_t)(code >> (32 - kLutBits));
      }
      S.sorted[F.base[l] + r] = (uint8_t)sym;
      if (l <= 4) {  // 2^(4-l) entries, naturally aligned
        const uint32_t e0 = (uint32_t)(code >> 28), v = (l << 8) | sym, v2 = v | (v << 16);
        if (l == 1) *reinterpret_cast<uint4*>(&F.l4[e0]) = make_uint4(v2, v2, v2, v2);
        else if (l == 2) *reinterpret_cast<uint2*>(&F.l4[e0]) = make_uint2(v2, v2);
        else if (l == 3) *reinterpret_cast<uint32_t*>(&F.l4[e0]) = v2;
        else F.l4[e0] = (uint16_t)v;
      }
    }
  }
  wave_sync();
  uint32_t* lut1 = reinterpret_cast<uint32_t*>(S.syms + kLut1Off);
  {  // codes of <= 4 bits cover whole 64-entry blocks of the 10-bit table
    const uint32_t e4 = F.l4[lane >> 2];
    const uint32_t v = e4 ? lut1_entry(e4 >> 8, e4 & 255u) : kLongMark;
    const uint4 v4 = make_uint4(v, v, v, v);
    uint4* q = reinterpret_cast<uint4*>(&lut1[16 * lane]);
    // Lane l writes its 16 words in an order rotated by l >> 2, so each
    // store of 16 lanes covers all 64 LDS banks once.
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) q[(j + (lane >> 2)) & 3] = v4;
  }
  wave_sync();
  // Codes of 5..10 bits: 2^(10-l) entries from e0, naturally aligned.
  const auto range_fill = [&](uint32_t l, uint32_t sym, uint32_t e0) {
    const uint32_t v = lut1_entry(l, sym);
    const uint4 v4 = make_uint4(v, v, v, v);
    if (l <= 8) {
      uint4* q = reinterpret_cast<uint4*>(&lut1[e0]);
      q[0] = v4;
      if (l <= 7) q[1] = v4;
      if (l <= 6) {
        q[2] = v4;
        q[3] = v4;
      }
      if (l == 5) {
        q[4] = v4;
        q[5] = v4;
        q[6] = v4;
        q[7] = v4;
      }
    } else if (l == 9) {
      *reinterpret_cast<uint2*>(&lut1[e0]) = make_uint2(v, v);
    } else {
      lut1[e0] = v;
    }
  };
  if (m <= kWave) {  // one symbol per lane: its code is still in registers
    if (lane < m && rl >= 5 && rl <= kLutBits) range_fill(rl, rs, re0);
  } else {
    for (uint32_t s0 = 0; s0 < m; s0 += kWave) {
      const uint32_t t = s0 + lane;
      if (t < m) {
        const uint32_t ent = compact[t], l = ent >> 8, sym = ent & 255u, r = rank[t];
        if (l >= 5 && l <= kLutBits)
          range_fill(l, sym, (uint32_t)((F.lim[l - 1] + ((uint64_t)r << (32 - l))) >> (32 - kLutBits)));
      }
    }
  }
  wave_sync();
  const uint32_t* lut1r = lut1;
  const uint32_t lane_hi = lane << 26;
  // Two-symbol table: entry e holds its first code and, when the code after
  // it also ends within the 10-bit window, that one too.  Lane l takes
  // entries l + 64 i (consecutive lanes, consecutive words).  With the
  // one-symbol entries laid out as lut1_entry, an entry is
  //   a = first entry & 0x0F007FFF (symbol, length in bits 8-14 and 24-27)
  //   x = a + (second entry & 0x00FF7F00) (adds the second symbol at bits
  //       16-23 and its length into bits 8-15: at most 127 + 127)
  // and holds two codes iff bits 8-15 of x are at most 10; markers (length
  // 127) never pair.
  //
  // The second entry is read at the window shifted past the first code, whose
  // low l1 bits would be padding zeros.  Any fill of those bits gives the
  // same result: a second code that fits the window lies wholly in the shifted
  // bits, and one that does not fit is rejected whatever the entry read.  The
  // fill is the lane's top bits (lane << l1 >> 6), so that lanes read distinct
  // LDS banks instead of the 2^l1-way conflict of the zero-padded addresses;
  // for a marker (l1 = 0) the fill lands above bit 9 and is masked off.
#pragma unroll
  for (uint32_t g = 0; g < 2; ++g) {  // eight entries at a time: two LDS round trips per group
    uint32_t v[8], b[8];
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) v[i] = lut1r[lane + kWave * (8 * g + i)];
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      const uint32_t l1 = v[i] >> 28;
      const uint32_t fill = __builtin_amdgcn_alignbit(0u, lane_hi, 32u - l1);
      b[i] = lut1r[(((lane + kWave * (8 * g + i)) << l1) | fill) & ((1u << kLutBits) - 1)];
    }
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      const uint32_t a = v[i] & 0x0F007FFFu;
      const uint32_t x = a + (b[i] & 0x00FF7F00u);
      F.lut2[lane + kWave * (8 * g + i)] = (x & 0xFF00u) <= (kLutBits << 8) ? x | 0x8000u : a;
    }
  }
  wave_sync();
  return Book{0, maxlen, true};
}

// Tables for codes longer than 32 bits (bit-serial path).  cnt/base/sorted
// as above; open[l] counts length-l prefixes that longer codes extend, so a
// prefix beyond them is an invalid code [src/codec.cpp:69 "invalid bitstream"].
__device__ __forceinline__ Book build_slow(Smem& S, uint32_t lane, uint32_t lw, uint32_t maxlen) {
  SlowTables& T = S.t.s;
  uint8_t* lens = S.syms + 1024;
  reinterpret_cast<uint32_t*>(lens)[lane] = lw;
  for (uint32_t i = lane; i < 256; i += kWave) T.cnt[i] = 0;
  wave_sync();
#pragma unroll
  for (uint32_t q = 0; q < 4; ++q) {
    const uint32_t l = lens[4 * lane + q];
    if (l) atomicAdd(&T.cnt[l], 1u);
  }
  wave_sync();
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
  wave_sync();
  return Book{S.bcast[0], maxlen, false};
}

// `lw` holds the code lengths of symbols 4 lane .. 4 lane + 3.
__device__ __forceinline__ Book build_book(Smem& S, uint32_t lane, uint32_t lw) {
  const uint32_t L0 = lw & 255u, L1 = (lw >> 8) & 255u, L2 = (lw >> 16) & 255u, L3 = lw >> 24;
  const uint32_t mx = max(max(L0, L1), max(L2, L3));
  const uint32_t maxlen = wave_max(mx);
  if (maxlen > kMaxLenFast) return build_slow(S, lane, lw, maxlen);
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

// A lane's decoded chunk: `f` = its first codeword start at or past the chunk
// start (kNoStart when the path failed before reaching it), `cnt` symbols at
// region[0 ...], `ex` = the first start at or past the chunk end, `dead` = a
// window in the chunk matched no code.
struct Path {
  uint32_t f, cnt, ex, dead;
};
constexpr uint32_t kNoStart = 0xffffffffu;

// The register window: w0, w1, w2 = segment dwords j - 1 .. j + 1 with
// j = ceil(p / 32), and wb = 32 j, the first bit past w0.  Slide it after p
// advanced by at most 32 bits (p > wb: p left w0); the third dword is re-read
// from LDS off the dependency chain.
__device__ __forceinline__ void slide(const Smem& S, uint32_t p, uint32_t& wb, uint32_t& w0, uint32_t& w1,
                                      uint32_t& w2) {
  const bool adv = p > wb;
  wb += adv ? 32u : 0u;
  __builtin_assume((wb & 31u) == 0u);
  w0 = adv ? w1 : w0;
  w1 = adv ? w2 : w1;
  w2 = S.stream[(wb >> 5) + 2];
}

// Up to two codewords at bit p (lut2 entry layout).  A window without a code
// of at most 10 bits is resolved on the spot with the per-length limits
// (long_code): the entry becomes that one code.  That branch is rare (codes
// longer than the table are well under 0.1% of symbols) and, unlike leaving
// the code to a later round, keeps the other lanes of the wave stepping.  A
// window that matches no code sets `dead` and returns kDeadMark, whose
// "consumed" 127 moves p past the caller's end (chunks are at most kChunk
// bits and paths start at most kSync bits before them).  The second codeword
// may start at or past the caller's end; the caller undoes that after its
// last step (end_pair).  Bit positions stay below kSegBits + kLongLen + 32,
// inside the staged segment buffer.
constexpr uint32_t kDeadMark = kLongLen << 8;
static_assert(kChunk + kSync <= kLongLen, "a dead path must leave every chunk");
__device__ __forceinline__ uint32_t step2(const Smem& S, uint32_t& p, uint32_t& wi, uint32_t& w0, uint32_t& w1,
                                          uint32_t& w2, uint32_t maxlen, uint32_t& dead) {
  const uint32_t win = __builtin_amdgcn_alignbit(w0, w1, 0u - p);
  uint32_t e = S.t.f.lut2[win >> (32 - kLutBits)];
  // A wave-uniform test first: the common step then takes no exec-mask
  // save/restore and no taken branch.
  if (__builtin_expect(__ballot(e == kLongMark) != 0, 0)) {
    if (e == kLongMark) {
      const uint32_t lc = long_code(S, win, maxlen);  // (len << 8) | symbol: no second symbol, len1 0
      dead |= lc == 0;
      e = lc ? lc : kDeadMark;
    }
  }
  p += (e >> 8) & 127u;
  slide(S, p, wi, w0, w1, w2);
  return e;
}

// After a loop of step2 calls that stopped at the first p >= end, with `le`
// the last step's entry: when that step was a pair whose second codeword
// starts at or past `end`, that codeword belongs to the next range: step
// back to it.  Returns 1 when a symbol was taken back.
__device__ __forceinline__ uint32_t end_pair(uint32_t le, uint32_t end, uint32_t& p) {
  const uint32_t lp = p - ((le >> 8) & 127u);
  const uint32_t s2 = lp + ((le >> 24) & 15u);
  const bool back = ((le >> 15) & 1u) && s2 >= end;
  p = back ? s2 : p;
  return back;
}

__device__ __forceinline__ void load_window(const Smem& S, uint32_t p, uint32_t& wb, uint32_t& w0, uint32_t& w1,
                                            uint32_t& w2) {
  const uint32_t j = (p + 31) >> 5;
  wb = 32u * j;
  w0 = S.stream[j];
  w1 = S.stream[j + 1];
  w2 = S.stream[j + 2];
}

// Decode the codewords that start in [cs, ce) into region[0 ...], two per
// lookup where the table allows.  When `from` < cs the codewords before cs
// are decoded and dropped: Huffman codes resynchronise within a few
// codewords, so a path started kSync bits early almost always meets the true
// codeword boundaries before cs (the caller verifies it against the previous
// lane's exit).  Symbols are stored a byte at a time (aligned LDS stores).
// A path that meets a window matching no code is dead: it produces no start
// (f = kNoStart) when that happens before cs, and its symbols are never used.
__device__ __forceinline__ void decode_chunk(const Smem& S, uint32_t from, uint32_t cs, uint32_t ce, uint8_t* region,
                                             uint32_t maxlen, Path& P) {
  uint32_t p = from, d = 0, wi, w0, w1, w2, le = 0;
  load_window(S, p, wi, w0, w1, w2);
  if (p < cs) {
    while (p < cs) le = step2(S, p, wi, w0, w1, w2, maxlen, d);
    end_pair(le, cs, p);
    load_window(S, p, wi, w0, w1, w2);
  }
  P.f = d ? kNoStart : p;
  if (d) p = ce;
  lds_bytes const out = as_lds(region);
  lds_bytes o = out;  // next symbol slot
  le = 0;
  {
    while (p < ce) {
      le = step2(S, p, wi, w0, w1, w2, maxlen, d);
      o[0] = (uint8_t)le;
      o[1] = (uint8_t)(le >> 16);
      o += 1 + ((le >> 15) & 1u);
    }
    P.cnt = (uint32_t)(o - out) - end_pair(le, ce, p);
  }
  P.ex = p;
  P.dead = d;
}

// Inputs of a stream's first segment, loaded ahead of use: the stream
// header words (lanes 0, 1), the 256 code lengths (4 per lane) and the first
// 784 code bytes (16 per lane, lanes < kStreamLanes).
struct StreamIn {
  uint64_t hdr;
  uint32_t lens;
  Fetch16 bits;
};
// Sign/mantissa bytes of the first kSmWin * 64 units (3,072 positions) a
// consume call will see: unit lane_unit(lane) + 64 i in v[i] (the consumer's
// own mapping).  A full 6,144-bit segment of codes averaging 2-2.6 bits holds
// 2,400-3,100 symbols; units past the window are loaded inside the call,
// which then waits for the loads (and for any stores issued before them).
constexpr uint32_t kSmWin = 6;
struct SmWin {
  uint64_t v[kSmWin];
};

// `seg` .. `seg_end` is one serial block or XKSP2 segment; `count` is the
// element count the block header implies (checked against the stream header
// when the loads are used).  All loads stay inside [seg, seg_end).
__device__ __forceinline__ void issue_stream(StreamIn& P, const uint8_t* seg, const uint8_t* seg_end, uint32_t count,
                                             uint32_t lane) {
  P.hdr = lane < 2 ? ldg64(seg + 8 * lane) : 0ull;
  P.lens = ldg32(seg + 16 + 4 * lane);
  if (lane < kStreamLanes) {
    P.bits = fetch16(seg + 272 + (uint64_t)count + 16 * lane, seg_end);
  } else {
    P.bits.v = make_uint4(0u, 0u, 0u, 0u);
    P.bits.drop = 16;
  }
}
// N < kSmWin: only the first N window entries are loaded (a consume call
// that sees at most N * 64 units); the rest are constant zeros.
template <uint32_t N = kSmWin>
__device__ __forceinline__ void issue_sm(SmWin& W, const uint8_t* sm, uint32_t pos0, uint32_t count, uint32_t lu) {
#pragma unroll
  for (uint32_t i = 0; i < kSmWin; ++i) {
    const uint32_t p = pos0 + 8 * (lu + kWave * i);
    W.v[i] = i < N && p + 8 <= count ? ldg64(sm + p) : 0ull;
  }
}
// The stream after the current one (seg == nullptr: none); its inputs are
// issued when the current stream starts and land while it decodes.
struct NextStream {
  const uint8_t* seg;
  const uint8_t* end;
  uint32_t count;
  __device__ __forceinline__ void issue(StreamIn& PN, uint32_t lane) const {
    if (seg) issue_stream(PN, seg, end, count, lane);
  }
};

// Wait for every outstanding global load (and store).  Called just before a
// consumer issues its stores, when all that is in flight is prefetches issued
// long before: on this architecture loads and stores share one in-order
// counter, so a later wait for those prefetches would also wait for the
// consumer's fresh stores.
__device__ __forceinline__ void drain_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0) only

// 16 bytes from global memory straight into LDS (global_load_lds_dwordx4):
// lane l writes the 16 bytes at its `src` to dst + 16 l.  `dst` is the same
// on every lane and 16-byte aligned; every lane's src must be readable.  The
// copy is an outstanding load until drain_loads().
__device__ __forceinline__ void copy_to_lds16(const void* src, uint8_t* dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
}
// The 8 exponents of unit u (8 consecutive symbols) of a consume call:
// compacted runs (decode_fast) hold them at byte 8u; the indexed walk's lane
// slots at kIdxStride (u / 4) + 8 (u % 4), dword aligned.
template <bool kIx>
__device__ __forceinline__ uint64_t unit_exps(const uint8_t* syms, uint32_t u) {
  static_assert(kIdxStride == 36, "slot offset below: 36 (u / 4) + 8 (u % 4) = 8 u + 4 (u / 4)");
  const uint32_t off = kIx ? 8u * u + (u & ~3u) : 8u * u;
  const uint32_t* q = reinterpret_cast<const uint32_t*>(syms + off);
  return (uint64_t)q[0] | ((uint64_t)q[1] << 32);
}
// 16 bytes of LDS through an LDS pointer: a read that the compiler could
// otherwise merge with a global read of the other branch into one FLAT load.
__device__ __forceinline__ uint4 lds16(const uint8_t* p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = *(__attribute__((address_space(3))) const u32x4*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void stage_bits(Smem& S, uint32_t lane, uint4 v) {
  if (lane < kStreamLanes) {
    uint32_t* w = &S.stream[1 + 4 * lane];
    w[0] = bswap32(v.x);
    w[1] = bswap32(v.y);
    w[2] = bswap32(v.z);
    w[3] = bswap32(v.w);
  }
}

// Hand a stream's prefetched inputs to LDS: its first 784 code bytes into the
// segment buffer (behind a zero dword), its 256 code lengths into `sorted`
// (read back before the tables are built) and its header words into `bcast`.
// Called where every load is known to have landed -- right after
// drain_loads() -- so the next stream starts without waiting on the memory
// counter, which by then also counts this stream's output stores.
__device__ __forceinline__ void stage_inputs(Smem& S, uint32_t lane, const StreamIn& P) {
  stage_bits(S, lane, P.bits.value());
  if (lane == 0) S.stream[0] = 0;
  reinterpret_cast<uint32_t*>(S.sorted)[lane] = P.lens;
  if (lane < 2) reinterpret_cast<uint64_t*>(S.bcast)[lane] = P.hdr;
  wave_sync();
}

// A sub-range of a stream (workgroup-scale serial decode): the codewords that
// start in [start_bit, end_bit).  With `spec`, start_bit is not known to be a
// codeword boundary: lane 0 walks its first chunk from up to kSync bits
// earlier, like the other lanes, and `first` returns the first codeword start
// at or past start_bit on that path (kNoStart64 when the path died before it).
// `exit` returns the first codeword start at or past end_bit and `count` the
// symbols decoded.  Only a range that ends the stream checks the trailing bits.
constexpr uint64_t kNoStart64 = ~0ull;
struct Range {
  uint64_t end_bit;
  bool spec;
  uint64_t first, exit;
  uint32_t count;
};
// Consumers that do not read the sign/mantissa bytes (SmUse false) get no
// window loads.
template <class C>
struct SmUse {
  static constexpr bool value = true;
};

// Decode one stream with the fast tables; the consumer receives the
// exponents in stream order.  `first` holds the stream's first 784 code
// bytes; later segments are loaded one segment ahead.  Returns error bits.
template <class Cons>
//
// `start_bit` / `start_pos` resume the stream at a codeword boundary already
// known to be true (its symbol index start_pos, a multiple of 256): the
// indexed path hands a stream over here when its index does not chain.  A
// stream decoded from its start has its first bytes staged with its inputs.
__device__ __forceinline__ uint32_t decode_fast(Smem& S, uint32_t lane, const Stream& st, uint32_t maxlen,
                                                const uint8_t* blk_end, Cons& C, const StreamIn& PN, bool next,
                                                uint64_t start_bit = 0, uint32_t start_pos = 0,
                                                Range* R = nullptr) {
  const uint64_t nbits = st.nbits;
  const uint64_t end = R ? R->end_bit : nbits;  // decode the codewords that start before `end`
  bool spec = R && R->spec;
  const uint8_t* bend = st.bits + ((nbits + 7) >> 3);
  if (bend > blk_end) bend = blk_end;
  uint8_t* const region = S.syms + kCarry + lane * kRegion;
  // A speculative start stages from kSync bits earlier, so lane 0 can walk in.
  uint64_t S0 = (spec ? start_bit - (start_bit < kSync ? start_bit : (uint64_t)kSync) : start_bit) & ~7ull, true_pos = start_bit;
  uint32_t carry = 0, pos0 = start_pos, entry = (uint32_t)(start_bit - S0), err = 0;
  // Chunk size: the stream is cut into the fewest segments of at most kSegBits
  // bits, and each segment evenly over the 64 lanes, so that every segment --
  // the last one included -- keeps all lanes busy.  A wave's time per segment
  // follows its longest chunk, so a stream of 1.1 segments at fixed 96-bit
  // chunks would cost two full segments.
  uint32_t chunk = kChunk;
  if (end > S0) {
    const uint64_t nseg = (end - S0 + kSegBits - 1) / kSegBits;
    chunk = (uint32_t)((end - S0 + kWave * nseg - 1) / (kWave * nseg));
  }
  const uint32_t segbits = kWave * chunk;
  Fetch16 cur;
  cur.v = make_uint4(0u, 0u, 0u, 0u);
  cur.drop = 16;
  const bool resume = start_bit != 0 || start_pos != 0 || spec;
  if (resume && lane < kStreamLanes) cur = fetch16(st.bits + (S0 >> 3) + 16 * lane, bend);
  bool stage_top = resume;
  bool staged = false;
  while (true_pos < end) {
    if (stage_top) {  // a stream's first segment was staged with its inputs
      stage_bits(S, lane, cur.value());
      wave_sync();
    }
    stage_top = true;
    // Next segment's code bytes and this segment's sign/mantissa window go
    // out now and land while the segment decodes.
    if (S0 + segbits < end && lane < kStreamLanes)
      cur = fetch16(st.bits + ((S0 + segbits) >> 3) + 16 * lane, bend);
    SmWin W;
    if constexpr (SmUse<Cons>::value) issue_sm(W, st.sm, pos0, st.count, Cons::lane_unit(lane));
    const uint64_t left = end - S0;
    const uint32_t lim_bits = left < segbits ? (uint32_t)left : segbits;
    // The lanes' chunks tile [0, lim_bits); after a speculative start they
    // tile [entry, lim_bits) instead (the bits before the entry belong to the
    // previous range), in chunks no longer than `chunk`.
    const uint32_t g0 = spec ? min(entry, lim_bits) : 0u;
    const uint32_t cw = spec ? max(1u, (lim_bits - g0 + kWave - 1) / kWave) : chunk;
    const uint32_t cs = g0 + lane * cw;
    const bool active = cs < lim_bits;
    const uint32_t ce = active ? min(cs + cw, lim_bits) : cs;
    // Lane 0 starts at the true entry (speculative: at the segment's first
    // staged bit); the others kSync bits before their chunk, or at the entry
    // when that is closer.  An inactive lane's empty range gives f = ex = cs,
    // cnt = 0.
    Path P;
    decode_chunk(S, !active ? cs : lane == 0 ? (spec ? 0u : entry) : cs > entry + kSync ? cs - kSync : entry, cs, ce,
                 region, maxlen, P);
    if (spec) {  // the range's first codeword on lane 0's path: trusted here, checked by the caller
      const uint32_t f0 = rdlane(P.f, 0);
      R->first = f0 == kNoStart ? kNoStart64 : S0 + f0;
      if (f0 == kNoStart) {
        err = kErrStream;
        break;
      }
      entry = f0;
      spec = false;
    }
    // Resolve: lane i is on the true path when its first start equals its
    // predecessor's exit and the predecessor is.  Lanes that fail re-decode
    // from that exit (rare: a path that did not resynchronise within kSync).
    for (;;) {
      uint32_t pe = from_prev_lane(P.ex), pd = from_prev_lane(P.dead);
      if (lane == 0) {
        pe = entry;
        pd = 0;
      }
      const bool ok = !active || (!pd && P.f == pe);
      const uint64_t bad = __ballot(!ok);
      const uint64_t deadm = __ballot(active && P.dead);
      const uint64_t resolved = bad ? ((1ull << (__ffsll((unsigned long long)bad) - 1)) - 1) : ~0ull;
      if (deadm & resolved) {
        err = kErrStream;
        break;
      }
      if (!bad) break;
      const bool redo = !ok && !pd;
      Path Q;
      decode_chunk(S, redo ? pe : ce, redo ? cs : ce, ce, region, maxlen, Q);  // empty range unless redo
      if (redo) P = Q;
    }
    if (err) break;
    const uint32_t t = active ? P.cnt : 0u;
    const uint32_t tinc = wave_incl(t, lane);
    const uint32_t total = rdlane(tinc, kWave - 1);
    const uint64_t act = __ballot(active);
    const uint32_t last = 63u - (uint32_t)__clzll((long long)act);
    const uint32_t seg_exit = rdlane(P.ex, last);
    if ((uint64_t)pos0 + carry + total > st.count) {
      err = kErrStream;  // more codewords than elements: trailing bits
      break;
    }
    // Compact the lanes' runs behind the carried partial tile, with aligned
    // LDS accesses only: a lane reads its run as aligned dwords, realigns
    // them to the destination with byte funnel shifts, stores the whole
    // destination dwords and writes the (at most 3 + 3) bytes it shares with
    // its neighbours one at a time.  All reads precede all writes: a run's
    // destination can overlap other lanes' sources.
    {
      const uint32_t dst = carry + tinc - t;
      const uint32_t dh = dst & 3u, nq = (t + 3) >> 2, nqmax = wave_max(nq);
      const uint32_t* src = reinterpret_cast<const uint32_t*>(region);
      // Four dwords per step under a wave-uniform bound (no register
      // indexing); bytes past a lane's run are read but never stored.
      constexpr uint32_t kQ = kChunk / 4;
      uint32_t R[kQ + 4];
#pragma unroll
      for (uint32_t q0 = 0; q0 < kQ; q0 += 4) {
        if (q0 < nqmax) {
#pragma unroll
          for (uint32_t q = q0; q < q0 + 4; ++q) R[q] = src[q];
        } else {
#pragma unroll
          for (uint32_t q = q0; q < q0 + 4; ++q) R[q] = 0u;
        }
      }
#pragma unroll
      for (uint32_t q = kQ; q < kQ + 4; ++q) R[q] = 0u;
      wave_sync();
      const uint32_t nw = (dh + t) >> 2;  // destination dwords that end inside the run
      // Destination dword k = run bytes [4k - dh, 4k - dh + 4): bytes 4 - dh
      // .. 7 of source dwords k - 1, k (one byte permute).  Whole dwords are written
      // without per-dword predicates: a lane writes dwords 0 .. (its block of
      // nqmax) + 3, highest first.  Past its run they hold garbage, which
      // lands only on later lanes' dwords of lower index k' < k -- written
      // after it in this order -- or past the data.  A lane whose run starts
      // and ends inside one dword (nw == 0) could share its base dword with
      // the next lane, so it writes to kDummy instead.  A run's first dword,
      // when shared with the bytes before it (dh != 0), is left to byte
      // stores; its last dword (bytes 0 .. (dh + t) % 4 - 1 of dword nw) is
      // written whole at step nw and no later store covers those bytes: the
      // next run writes that dword only when it starts aligned, i.e. when no
      // byte of this run is in it.
      constexpr uint32_t kDummy = kSymsBytes - 4 * (kQ + 4);
      static_assert(255 + kSegBits + 4 * (kQ + 4) <= kDummy, "compaction garbage must stay off the dummy run");
      uint32_t* d32 = reinterpret_cast<uint32_t*>(S.syms + (nw ? (dst & ~3u) : kDummy));
      const uint32_t sel = 0x07060504u - 0x01010101u * dh;  // byte selector of (R[k], R[k - 1])
      uint32_t head = 0;
#pragma unroll
      for (int k0 = (int)kQ; k0 >= 0; k0 -= 4) {
        if ((uint32_t)k0 <= nqmax) {
#pragma unroll
          for (int k = k0 + 3; k >= k0; --k) {
            const uint32_t w = __builtin_amdgcn_perm(R[k], k ? R[k - 1] : 0u, sel);
            if (k == 0) head = w;
            if (k > 0 || dh == 0) d32[k] = w;
            wave_sync();  // keeps the stores one dword per instruction, in this order
          }
        }
      }
      // Bytes of the first dword when it is shared (dh != 0) or holds the
      // whole run (nw == 0).
      lds_bytes d8 = as_lds(S.syms + (dst & ~3u));
      const bool first_bytes = dh != 0 || nw == 0;
#pragma unroll
      for (uint32_t b = 0; b < 4; ++b)
        if (first_bytes && b >= dh && b - dh < t) d8[b] = (uint8_t)(head >> (8 * b));
      wave_sync();
    }
    const uint32_t avail = carry + total;
    const bool fin = S0 + seg_exit >= end;  // last segment: hand over everything
    drain_loads();
    if (fin && next) {  // this stream is done with the segment buffer
      stage_inputs(S, lane, PN);
      staged = true;
    }
    const uint32_t take = C.consume(S, lane, st, pos0, avail, fin, W);
    const uint32_t rem = avail - take;
    if (take && rem) {  // take is a multiple of 256 here, so source and destination do not overlap
      const uint32_t v = 4 * lane < rem ? lds32(S.syms + take + 4 * lane) : 0u;
      wave_sync();
      if (4 * lane < rem) sts32(S.syms + 4 * lane, v);
    }
    wave_sync();
    carry = rem;
    pos0 += take;
    true_pos = S0 + seg_exit;
    entry = seg_exit - segbits;
    S0 += segbits;
  }
  if (R) {
    R->exit = true_pos;
    R->count = pos0 + carry;
    if (!err && end == nbits && true_pos != nbits) err = kErrStream;  // trailing bits
  } else if (!err && (true_pos != nbits || (uint64_t)pos0 + carry != st.count)) {
    err = kErrStream;
  }
  wave_sync();
  if (next && !staged) {  // left early (an error): hand the next stream's inputs on anyway
    drain_loads();
    stage_inputs(S, lane, PN);
  }
  return err;
}

// Decode one stream of a fused GEMM item with its codeword index
// (k_index_items): per segment of kIdxSegSyms symbols, lane l starts at the
// recorded bit offset of symbol kIdxLaneSyms * l and decodes exactly
// kIdxLaneSyms symbols into its slot of the symbol buffer, so the segment
// needs no speculative prefix, no path resolution, no prefix sum and no
// compaction.  The offsets are checked, not trusted: every lane must end
// exactly where the next one starts (the last where the segment ends).  Lane
// 0 of segment 0 starts at the stream's first bit, so by induction every
// start is then a true codeword boundary and the symbols are exact.  When a
// segment does not chain (a stale or damaged index, or a damaged stream),
// it returns false with that segment's start in (rbit, rpos): the caller
// continues the stream speculatively from there (decode_fast), which decodes
// it -- or reports its error -- exactly as decode does.  Otherwise it returns
// true with the stream's error bits in `err`.
//
// The entries are read from LDS (kIxOff): segment 0's are copied there by
// the caller while the tables are built, each later segment's one segment
// ahead, so no segment waits on them.
template <class Cons>
__device__ __forceinline__ bool decode_indexed(Smem& S, uint32_t lane, const Stream& st, uint32_t maxlen,
                                               const uint8_t* blk_end, Cons& C, const StreamIn& PN, bool next,
                                               const uint16_t* idx, uint32_t& err, uint64_t& rbit, uint32_t& rpos) {
  const uint64_t nbits = st.nbits;
  const uint8_t* bend = st.bits + ((nbits + 7) >> 3);
  if (bend > blk_end) bend = blk_end;
  uint64_t segbit = 0;  // stream bit where the segment starts: a true codeword boundary
  uint32_t pos0 = 0;
  bool staged = false;
  Fetch16 cur;
  cur.v = make_uint4(0u, 0u, 0u, 0u);
  cur.drop = 16;
  for (uint32_t sg = 0; pos0 < st.count; ++sg) {
    const uint16_t* e = reinterpret_cast<const uint16_t*>(S.syms + kIxOff + 128 * (sg & 1));
    const uint32_t span = e[0];
    const uint32_t rel = lane ? e[lane] : 0u;
    const uint32_t rel_next = lane < 63 ? e[lane + 1] : span;
    const uint32_t n_s = min(kIdxSegSyms, st.count - pos0);
    const uint32_t last = (n_s - 1) / kIdxLaneSyms;  // last lane with symbols
    const uint32_t k = lane < last ? kIdxLaneSyms : lane == last ? n_s - kIdxLaneSyms * last : 0u;
    const uint32_t want = lane == last ? span : rel_next;
    // Entries must lie inside the staged segment, in order, before any is used
    // (lanes past the last one with symbols hold no entry).
    if (__ballot(span > kIdxMaxSpan || (k && (rel > span || want < rel)))) {
      C.xs = false;  // the previous segment's copy has landed (drained before its consume)
      rbit = segbit;
      rpos = pos0;
      return false;
    }
    if (sg) {  // this segment's bytes, prefetched during the previous one
      stage_bits(S, lane, cur.value());
      wave_sync();
    }
    const uint64_t nextbit = segbit + span;
    const bool more = pos0 + n_s < st.count;
    if (more && lane < kStreamLanes) cur = fetch16(st.bits + (nextbit >> 3) + 16 * lane, bend);
    // the next segment's entries (inside the item's allotment: the caller
    // passes an index only for streams it holds whole); landed by the drain
    // before this segment's consume
    if (more && lane < 8) copy_to_lds16(idx + 64 * (sg + 1) + 8 * lane, S.syms + kIxOff + 128 * ((sg + 1) & 1));
    SmWin W;
    issue_sm<kIdxSegSyms / 8 / kWave>(W, st.sm, pos0, st.count, Cons::lane_unit(lane));
    C.stage_x(S, lane, st, pos0, n_s);  // lands in LDS during the walk
    // The staged buffer starts at byte segbit >> 3 (its bit 0 after the zero dword).
    const uint32_t base = (uint32_t)(segbit & 7u), limit = base + want;
    uint32_t p = base + rel, n = 0, d = 0, wi, w0, w1, w2;
    load_window(S, p, wi, w0, w1, w2);
    lds_bytes const o = as_lds(S.syms + kIdxStride * lane);
    // One exit condition: a lane walks exactly k symbols.  A path on wrong
    // offsets (a stale index) advances at most 127 bits per step for at most
    // kIdxLaneSyms steps, which stays inside this wave's LDS block, and fails
    // the check below.
    {
      // Steps that cannot pass k store both bytes (a lone symbol's second
      // byte is rewritten by the next step); a last single symbol takes one
      // more step that keeps only the entry's first code.  Four steps per
      // iteration while eight symbols are left, then two, then one: fewer
      // loop tests (the exit test and exec-mask update of every step cost
      // 2-4 % of the walk).
      while (n + 8 <= k) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t ec = step2(S, p, wi, w0, w1, w2, maxlen, d);
          o[n] = (uint8_t)ec;
          o[n + 1] = (uint8_t)(ec >> 16);
          n += 1 + ((ec >> 15) & 1u);
        }
      }
      while (n + 4 <= k) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const uint32_t ec = step2(S, p, wi, w0, w1, w2, maxlen, d);
          o[n] = (uint8_t)ec;
          o[n + 1] = (uint8_t)(ec >> 16);
          n += 1 + ((ec >> 15) & 1u);
        }
      }
      while (n + 2 <= k) {
        const uint32_t en = step2(S, p, wi, w0, w1, w2, maxlen, d);
        o[n] = (uint8_t)en;
        o[n + 1] = (uint8_t)(en >> 16);
        n += 1 + ((en >> 15) & 1u);
      }
      if (n < k) {
        const uint32_t en = step2(S, p, wi, w0, w1, w2, maxlen, d);
        o[n] = (uint8_t)en;
        if ((en >> 15) & 1u) p -= ((en >> 8) & 127u) - ((en >> 24) & 15u);
        n += 1;
      }
    }
    if (__ballot(k && (d || p != limit))) {
      drain_loads();  // the X copy must land before decode_fast reuses the buffer
      C.xs = false;
      rbit = segbit;
      rpos = pos0;
      return false;
    }
    wave_sync();
    const bool fin = !more;
    drain_loads();
    if (fin && next) {
      stage_inputs(S, lane, PN);
      staged = true;
    }
    C.template consume<true>(S, lane, st, pos0, n_s, fin, W);  // symbols in the lane slots
    wave_sync();
    pos0 += n_s;
    segbit = nextbit;
  }
  // Every codeword is accounted for: the stream must end where its last one does.
  if (next && !staged) {
    drain_loads();
    stage_inputs(S, lane, PN);
  }
  err = segbit == nbits ? 0u : (uint32_t)kErrStream;
  return true;
}

// Bit-serial canonical decode for codes longer than 32 bits: lane 0 walks
// the code one bit at a time (d = offset from the first code of the current
// length); the consumer sees the symbols kSlowSeg at a time.
template <class Cons>
__device__ __forceinline__ uint32_t decode_slow(Smem& S, uint32_t lane, const Stream& st, Cons& C,
                                                const StreamIn& PN, bool next) {
  const SlowTables& T = S.t.s;
  const uint64_t nbits = st.nbits;
  uint64_t pos = 0;
  uint32_t produced = 0, err = 0;
  while (produced < st.count) {
    const uint32_t nseg = min(kSlowSeg, st.count - produced);
    if (lane == 0) {
      uint32_t e = 0;
      for (uint32_t i = 0; i < nseg && !e; ++i) {
        if (pos >= nbits) {
          e = kErrStream;
          break;
        }
        uint32_t d = (st.bits[pos >> 3] >> (7 - (pos & 7))) & 1u;
        ++pos;
        for (uint32_t l = 1;; ++l) {
          if (d < T.cnt[l]) {
            S.syms[i] = S.sorted[T.base[l] + d];
            break;
          }
          d -= T.cnt[l];
          if (d >= T.open[l] || l >= 255 || pos >= nbits) {
            e = kErrStream;
            break;
          }
          d = 2 * d + ((st.bits[pos >> 3] >> (7 - (pos & 7))) & 1u);
          ++pos;
        }
      }
      S.bcast[0] = e;
    }
    wave_sync();
    err = S.bcast[0];
    wave_sync();
    if (err) break;
    SmWin W;
    issue_sm(W, st.sm, produced, st.count, Cons::lane_unit(lane));
    drain_loads();
    C.consume(S, lane, st, produced, nseg, produced + nseg == st.count, W);
    wave_sync();
    produced += nseg;
  }
  if (lane == 0) S.bcast[1] = (pos == nbits);
  wave_sync();
  if (!err && !S.bcast[1]) err = kErrStream;
  wave_sync();
  if (next) {  // after the last use of bcast (this path is rare: codes over 32 bits)
    drain_loads();
    stage_inputs(S, lane, PN);
  }
  return err;
}

// A stream that fails before decoding still hands the next stream's inputs on.
__device__ __forceinline__ uint32_t fail_stream(Smem& S, uint32_t lane, uint32_t err, const NextStream& N,
                                                const StreamIn& PN) {
  if (N.seg) {
    drain_loads();
    stage_inputs(S, lane, PN);
  }
  return err;
}

// Header checks [src/c_api.cpp:29-40, cuda/decode.cu:47-51], tables, decode.
// The next stream's inputs are issued once this stream's header and lengths
// are in use: loads complete in issue order, so a wait for them issued after
// the prefetch would wait for the prefetch too.
template <class Cons>
__device__ __forceinline__ uint32_t stream_body(Smem& S, uint32_t lane, const uint8_t* seg, const uint8_t* seg_end,
                                                uint32_t count, uint32_t start, Cons& C, const NextStream& N,
                                                StreamIn& PN, const uint16_t* idx) {
  const uint64_t len = (uint64_t)(seg_end - seg);
  const uint64_t cnt = reinterpret_cast<const uint64_t*>(S.bcast)[0], nb = reinterpret_cast<const uint64_t*>(S.bcast)[1];
  const uint32_t lw = reinterpret_cast<const uint32_t*>(S.sorted)[lane];
  wave_sync();  // the staged inputs are read before the tables overwrite them
  N.issue(PN, lane);
  if (cnt != count || cnt > len - 272 || nb / 8 + (nb % 8 != 0) != len - 272 - cnt) return fail_stream(S, lane, kErrHeader, N, PN);
  // The index's first segment lands in LDS while the tables are built (no
  // register held across the build); every path below waits for it before
  // the symbol buffer is written past the tables' scratch.
  if (idx && lane < 8) copy_to_lds16(idx + 8 * lane, S.syms + kIxOff);
  Stream st;
  st.lengths = seg + 16;
  st.sm = seg + 272;
  st.bits = st.sm + cnt;
  st.nbits = nb;
  st.count = count;
  st.start = start;
  const Book b = build_book(S, lane, lw);
  if (idx) drain_loads();
  if (b.err) return fail_stream(S, lane, b.err, N, PN);
  if (!b.fast) return decode_slow(S, lane, st, C, PN, N.seg);
  uint64_t rbit = 0;
  uint32_t rpos = 0, err = 0;
  if (idx && reinterpret_cast<const uint16_t*>(S.syms + kIxOff)[0] != kIdxNone &&
      decode_indexed<Cons>(S, lane, st, b.maxlen, seg_end, C, PN, N.seg, idx, err, rbit, rpos))
    return err;
  return decode_fast<Cons>(S, lane, st, b.maxlen, seg_end, C, PN, N.seg, rbit, rpos);
}

// One stream whose inputs were staged in LDS (stage_inputs); the next
// stream's inputs are issued into PN (when N.seg is given) early on, so they
// load while this stream decodes, and staged when it finishes.  A stream that
// fails before its last segment stages them on the way out.  `idx`: the
// stream's codeword index (fused GEMM items), or nullptr.
template <class Cons>
__device__ __forceinline__ uint32_t run_stream(Smem& S, uint32_t lane, const uint8_t* seg, const uint8_t* seg_end,
                                               uint32_t count, uint32_t start, Cons& C, const NextStream& N,
                                               StreamIn& PN, const uint16_t* idx = nullptr) {
  return stream_body<Cons>(S, lane, seg, seg_end, count, start, C, N, PN, idx);
}

// ------------------------------------------------------------- consumers

// Unit = 8 consecutive tiled positions = half a tile row.  A stream is
// "unit-aligned" when its slab has full 16x16 tiles and the stream starts and
// ends on unit boundaries; then unit u holds row (u/2)%16, columns 16*(u/32)+8*(u%2).
__device__ __forceinline__ bool unit_aligned(uint32_t start, uint32_t count, uint64_t rows, uint64_t cols) {
  return rows % 16 == 0 && cols % 16 == 0 && start % 8 == 0 && count % 8 == 0;
}

// BF16 writer: 16-byte stores of half tile rows for unit-aligned streams,
// one element per lane per step otherwise.
struct Writer {
  uint8_t* out;  // slab base
  uint64_t rows, cols;
  uint32_t tpb;  // tiles per 16-row band
  bool aligned;
  bool xs = false;  // no activations
  __device__ __forceinline__ void stage_x(Smem&, uint32_t, const Stream&, uint32_t, uint32_t) {}
  static __device__ __forceinline__ uint32_t lane_unit(uint32_t lane) { return lane; }
  template <bool kIx>
  __device__ __forceinline__ void unit(const Smem& S, const Stream& st, uint32_t pos0, uint32_t u, uint64_t M) const {
    const uint4 w = combine8(unit_exps<kIx>(S.syms, u), M);
    const uint32_t U = ((st.start + pos0) >> 3) + u, T = U >> 5;
    const uint32_t band = rows == 16 ? 0u : T / tpb;
    const uint32_t row = 16u * band + ((U >> 1) & 15u);
    const uint32_t col = 16u * (T - band * tpb) + 8u * (U & 1u);
    __builtin_memcpy(out + 2ull * (row * (uint32_t)cols + col), &w, 16);
  }
  // kIx: the symbols are in the indexed walk's lane slots.
  template <bool kIx = false>
  __device__ __forceinline__ uint32_t consume(Smem& S, uint32_t lane, const Stream& st, uint32_t pos0, uint32_t avail, bool final,
                              const SmWin& W) {
    if (!aligned) {
      for (uint32_t i = lane; i < avail; i += kWave) {
        const uint32_t P = pos0 + i;
        const uint32_t e = S.syms[kIx ? kIdxStride * (i / kIdxLaneSyms) + i % kIdxLaneSyms : i], s = st.sm[P];
        const uint16_t w = (uint16_t)(((s & 0x80u) << 8) | (e << 7) | (s & 0x7fu));
        uint32_t row, col;
        tile_to_rc(st.start + P, (uint32_t)rows, (uint32_t)cols, row, col);
        __builtin_memcpy(out + 2ull * (row * (uint32_t)cols + col), &w, 2);
      }
      return avail;
    }
    const uint32_t take = final ? avail : (avail & ~255u);
    const uint32_t units = take >> 3;
    if (rows == 16) {
      // One band: unit lane + 64 i is two tiles (64 bytes of its row) after
      // unit lane + 64 (i - 1), so one address serves the window.
      const uint32_t U = ((st.start + pos0) >> 3) + lane;
      uint8_t* const p = out + 2ull * (((U >> 1) & 15u) * (uint32_t)cols + 16u * (U >> 5) + 8u * (U & 1u));
#pragma unroll
      for (uint32_t i = 0; i < kSmWin; ++i) {
        if (lane + kWave * i < units) {
          const uint4 w = combine8(unit_exps<kIx>(S.syms, lane + kWave * i), W.v[i]);
          __builtin_memcpy(p + 64 * i, &w, 16);
        }
      }
    } else {
#pragma unroll
      for (uint32_t i = 0; i < kSmWin; ++i) {
        const uint32_t u = lane + kWave * i;
        if (u < units) unit<kIx>(S, st, pos0, u, W.v[i]);
      }
    }
    for (uint32_t u = lane + kSmWin * kWave; u < units; u += kWave)
      unit<kIx>(S, st, pos0, u, ldg64(st.sm + pos0 + 8 * u));
    return take;
  }
};

// Exponents of a sub-range in stream order, as bytes at dst[0 ...] (first
// pass of the workgroup-scale serial decode).  16-byte stores; a call that
// would pass `cap` bytes sets `overflow` and stores nothing.
struct ScratchWriter {
  uint8_t* dst;
  uint32_t cap;
  bool overflow = false;
  bool xs = false;  // no activations
  __device__ __forceinline__ void stage_x(Smem&, uint32_t, const Stream&, uint32_t, uint32_t) {}
  static __device__ __forceinline__ uint32_t lane_unit(uint32_t lane) { return lane; }
  template <bool kIx = false>
  __device__ __forceinline__ uint32_t consume(Smem& S, uint32_t lane, const Stream&, uint32_t pos0, uint32_t avail,
                                              bool final, const SmWin&) {
    const uint32_t take = final ? avail : (avail & ~255u);
    if ((uint64_t)pos0 + take + 16 > cap) {
      overflow = true;
      return take;
    }
    for (uint32_t o = 16 * lane; o < take; o += 16 * kWave) {
      const uint4 v = lds16(S.syms + o);
      __builtin_memcpy(dst + pos0 + o, &v, 16);
    }
    return take;
  }
};
template <>
struct SmUse<ScratchWriter> {
  static constexpr bool value = false;
};

// Second pass of the workgroup-scale serial decode: tiled positions
// [P, P + n) of a slab, whose exponents are the bytes at src (4-byte aligned,
// readable 8 bytes past n), become BF16 outputs.  On unit-aligned slabs the
// units of 8 positions wholly inside go out as 16-byte stores; the partial
// units at either end, and every position of other slabs, one element at a
// time.  A unit's exponents sit at src offset 8U - P, misaligned by the same
// d = (8 u0 - P) % 4 for every unit, and are funnel-shifted out of 3 dwords.
__device__ __forceinline__ void place_range(const uint8_t* src, const Stream& st, uint32_t P, uint32_t n,
                                            uint8_t* out, uint64_t rows, uint64_t cols, bool aligned, uint32_t lane) {
  const uint32_t u0 = aligned ? (P + 7) >> 3 : 0u, u1 = aligned ? (P + n) >> 3 : 0u;
  const bool units = u0 < u1;
  const uint32_t lo_end = units ? 8 * u0 : P + n, hi_beg = units ? 8 * u1 : P + n;
  // element-wise: [P, lo_end) and [hi_beg, P + n)
  const uint32_t n_lo = lo_end - P, n_el = n_lo + (P + n - hi_beg);
  for (uint32_t i = lane; i < n_el; i += kWave) {
    const uint32_t t = i < n_lo ? P + i : hi_beg + (i - n_lo);
    const uint32_t e = src[t - P], sm = st.sm[t];
    const uint16_t w = (uint16_t)(((sm & 0x80u) << 8) | (e << 7) | (sm & 0x7fu));
    uint32_t row, col;
    tile_to_rc(t, (uint32_t)rows, (uint32_t)cols, row, col);
    __builtin_memcpy(out + 2ull * ((uint64_t)row * cols + col), &w, 2);
  }
  if (!units) return;
  const uint32_t d8 = 8u * ((8u * u0 - P) & 3u), tpb = (uint32_t)(cols / 16);
  for (uint32_t U = u0 + lane; U < u1; U += kWave) {
    const uint32_t j = 8u * U - P;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(src + (j & ~3u));
    const uint32_t a = q[0], b = q[1], c = q[2];
    const uint64_t E = (uint64_t)__builtin_amdgcn_alignbit(b, a, d8) |
                       ((uint64_t)__builtin_amdgcn_alignbit(c, b, d8) << 32);
    const uint4 w = combine8(E, ldg64(st.sm + 8ull * U));
    const uint32_t T = U >> 5, band = rows == 16 ? 0u : T / tpb;
    const uint32_t row = 16u * band + ((U >> 1) & 15u);
    const uint32_t col = 16u * (T - band * tpb) + 8u * (U & 1u);
    __builtin_memcpy(out + 2ull * ((uint64_t)row * cols + col), &w, 16);
  }
}

// Fused GEMM consumers.  Each one accumulates one wave's share of a 16-row
// slab's Y = W X and, after every stream, adds it into the wave's LDS slots
// (kOut floats: 16 rows x kCols batch columns); the kernel sums the waves'
// slots in wave order and stores them through store().
struct GemmArgs {
  const void* x;
  uint64_t ldx;  // X row stride in elements
  uint32_t nb;   // batch columns of this launch (<= kCols)
  float* y;
  uint64_t ldy;  // Y row stride in elements
};

// fp32 activations X[c * ldx + j] (cuda/decode.cu:94 layout), Y[(dst + r) *
// ldy + j]; VALU FMAs.  Lane `lane` accumulates unit u = lane + 64 i of every
// consume call; its row is ((start / 8 + lane) / 2) % 16 for the whole stream.
template <int NB>
struct GemmF32 {
  static constexpr int kCols = NB, kOut = 16 * NB;
  const float* x;
  uint64_t ldx;
  uint32_t nb;
  bool xa;          // x is 16-byte aligned
  bool xs = false;  // this segment's x columns are staged in LDS (kXOff)
  float acc[NB];
  __device__ __forceinline__ explicit GemmF32(const GemmArgs& a)
      : x(static_cast<const float*>(a.x)), ldx(a.ldx), nb(a.nb), xa(((uintptr_t)a.x & 15u) == 0) {}
  // One-column x (NB == 1): the segment's tiles t .. t + 8 need x[16 t, 16 t
  // + 144), at most 36 pieces of 16 bytes, one LDS copy.
  __device__ __forceinline__ void stage_x(Smem& S, uint32_t lane, const Stream& st, uint32_t pos0, uint32_t n) {
    xs = NB == 1 && xa;
    if (!xs) return;
    const uint32_t a = st.start + pos0, t = a >> 8, tiles = ((a + n - 1) >> 8) - t + 1;
    copy_to_lds16(lane < 4 * tiles ? x + 16ull * t + 4 * lane : x, S.syms + kXOff);
  }
  static __device__ __forceinline__ uint32_t lane_unit(uint32_t lane) { return lane; }
  static __device__ __forceinline__ bool fits(uint32_t s0, uint32_t count, uint64_t rows, uint64_t cols) {
    return unit_aligned(s0, count, rows, cols);
  }
  static __device__ __forceinline__ void store(const GemmArgs& a, uint64_t dst, uint32_t r, uint32_t j, float v) {
    if (j < a.nb) a.y[(dst + r) * a.ldy + j] = v;
  }
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = 0.f;
  }
  template <bool kIx>
  __device__ __forceinline__ void unit(const Smem& S, const Stream& st, uint32_t pos0, uint32_t u, uint64_t M) {
    const uint64_t E = unit_exps<kIx>(S.syms, u);
    const uint4 w = combine8(E, M);
    const uint32_t U = ((st.start + pos0) >> 3) + u;
    const uint64_t col = 16ull * (U >> 5) + 8u * (U & 1u);
    const float f[8] = {bf_lo(w.x), bf_hi(w.x), bf_lo(w.y), bf_hi(w.y),
                        bf_lo(w.z), bf_hi(w.z), bf_lo(w.w), bf_hi(w.w)};
    if (NB == 1) {
      float4 xa, xb;
      if (xs) {
        const uint32_t o = kXOff + 4u * (uint32_t)(col - 16ull * ((st.start + pos0) >> 8));
        const uint4 va = lds16(S.syms + o), vb = lds16(S.syms + o + 16);
        __builtin_memcpy(&xa, &va, 16);
        __builtin_memcpy(&xb, &vb, 16);
      } else {
        __builtin_memcpy(&xa, x + col, 16);
        __builtin_memcpy(&xb, x + col + 4, 16);
      }
      float a = acc[0];
      a = fmaf(f[0], xa.x, a);
      a = fmaf(f[1], xa.y, a);
      a = fmaf(f[2], xa.z, a);
      a = fmaf(f[3], xa.w, a);
      a = fmaf(f[4], xb.x, a);
      a = fmaf(f[5], xb.y, a);
      a = fmaf(f[6], xb.z, a);
      a = fmaf(f[7], xb.w, a);
      acc[0] = a;
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
  // kIx: the symbols are in the indexed walk's lane slots.
  template <bool kIx = false>
  __device__ __forceinline__ uint32_t consume(Smem& S, uint32_t lane, const Stream& st, uint32_t pos0,
                                              uint32_t avail, bool final, const SmWin& W) {
    const uint32_t take = final ? avail : (avail & ~255u);
    const uint32_t units = take >> 3;
#pragma unroll
    for (uint32_t i = 0; i < kSmWin; ++i) {
      const uint32_t u = lane + kWave * i;
      if (u < units) unit<kIx>(S, st, pos0, u, W.v[i]);
    }
    for (uint32_t u = lane + kSmWin * kWave; u < units; u += kWave)
      unit<kIx>(S, st, pos0, u, ldg64(st.sm + pos0 + 8 * u));
    return take;
  }
  // Four lanes share each row: with s = (stream start / 8) % 2, lane l and
  // ((l + s) ^ 1) - s (mod 64) hold the two halves of a tile row, and l ^ 32
  // the same row two tiles on.  After the two exchanges all four hold the
  // sum; one of them adds it to the slots.
  __device__ __forceinline__ void deposit(float* slots, uint32_t lane, uint32_t s0) {
    const uint32_t su = (s0 >> 3) & 1u;
    const int partner = (int)((((lane + su) ^ 1u) - su) & 63u);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      acc[j] += __shfl(acc[j], partner, kWave);
      acc[j] += __shfl_xor(acc[j], 32, kWave);
    }
    const uint32_t row = (((s0 >> 3) + lane) >> 1) & 15u;
    if (lane < 32 && ((lane + su) & 1u) == 0)
#pragma unroll
      for (int j = 0; j < NB; ++j) slots[row * NB + j] += acc[j];
  }
  // An item's record (row r, column j < nb at r * nb + j): the same two
  // exchanges as deposit, then the one lane per row that deposit would use
  // stores the row's sums; those 16 lanes cover the 16 rows once.
  __device__ __forceinline__ void record(float* part, uint32_t nb, uint32_t lane, uint32_t s0) {
    const uint32_t su = (s0 >> 3) & 1u;
    const int partner = (int)((((lane + su) ^ 1u) - su) & 63u);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      acc[j] += __shfl(acc[j], partner, kWave);
      acc[j] += __shfl_xor(acc[j], 32, kWave);
    }
    const uint32_t row = (((s0 >> 3) + lane) >> 1) & 15u;
    if (lane < 32 && ((lane + su) & 1u) == 0)
#pragma unroll
      for (int j = 0; j < NB; ++j)
        if (j < (int)nb) part[row * nb + j] = acc[j];
  }
};

// bf16 activations in the layout of x @ W.T: X[j * ldx + c] (batch rows),
// Y[j * ldy + dst + r]; fp32 accumulation on the VALU (batch 1, or streams
// that do not cover whole tiles).  A decoded
// unit is already 8 bf16 weights in 4 packed pairs, and 8 columns of an X row
// are 4 pairs too, so each pair of products is one v_dot2c_f32_bf16 (the
// products of bf16 values are exact in fp32).  Same lane mapping as GemmF32.
template <int NB>
struct GemmBf16 {
  static constexpr int kCols = NB, kOut = 16 * NB;
  static constexpr uint32_t kXRow = 18;  // staged 16-byte pieces per x row: 9 tiles
  static constexpr uint32_t kXCopies = NB <= 8 ? (kXRow * NB + 63) / 64 : 0;
  const uint16_t* x;
  uint64_t ldx;
  uint32_t nb;
  bool xa;          // x and its row stride are 16-byte aligned
  bool xs = false;  // this segment's x columns are staged in LDS (kXOff)
  float acc[NB];
  __device__ __forceinline__ explicit GemmBf16(const GemmArgs& a)
      : x(static_cast<const uint16_t*>(a.x)), ldx(a.ldx), nb(a.nb),
        xa(((uintptr_t)a.x & 15u) == 0 && a.ldx % 8 == 0) {}
  // Rows j < nb of the segment's columns [16 t, 16 t + 144): piece q of the
  // copies is row q / kXRow, columns 8 (q % kXRow) on.
  __device__ __forceinline__ void stage_x(Smem& S, uint32_t lane, const Stream& st, uint32_t pos0, uint32_t n) {
    xs = kXCopies && xa;
    if (!xs) return;
    const uint32_t a = st.start + pos0, t = a >> 8, tiles = ((a + n - 1) >> 8) - t + 1;
#pragma unroll
    for (uint32_t i = 0; i < kXCopies; ++i) {
      const uint32_t q = kWave * i + lane, j = q / kXRow, pc = q - kXRow * j;
      copy_to_lds16(j < nb && pc < 2 * tiles ? x + j * ldx + 16ull * t + 8 * pc : x, S.syms + kXOff + 1024 * i);
    }
  }
  static __device__ __forceinline__ uint32_t lane_unit(uint32_t lane) { return lane; }
  static __device__ __forceinline__ bool fits(uint32_t s0, uint32_t count, uint64_t rows, uint64_t cols) {
    return unit_aligned(s0, count, rows, cols);
  }
  static __device__ __forceinline__ void store(const GemmArgs& a, uint64_t dst, uint32_t r, uint32_t j, float v) {
    if (j < a.nb) a.y[j * a.ldy + dst + r] = v;
  }
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = 0.f;
  }
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    bf16x2 va, vb;
    __builtin_memcpy(&va, &a, 4);
    __builtin_memcpy(&vb, &b, 4);
    return __builtin_amdgcn_fdot2_f32_bf16(va, vb, c, false);
  }
  template <bool kIx>
  __device__ __forceinline__ void unit(const Smem& S, const Stream& st, uint32_t pos0, uint32_t u, uint64_t M) {
    const uint64_t E = unit_exps<kIx>(S.syms, u);
    const uint4 w = combine8(E, M);
    const uint32_t U = ((st.start + pos0) >> 3) + u;
    const uint64_t col = 16ull * (U >> 5) + 8u * (U & 1u);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if (j < (int)nb) {
        uint4 xv;
        if (xs)
          xv = lds16(S.syms + kXOff + 16u * (kXRow * j + (uint32_t)(col / 8 - 2ull * ((st.start + pos0) >> 8))));
        else
          __builtin_memcpy(&xv, x + j * ldx + col, 16);
        float a = acc[j];
        a = dot2(w.x, xv.x, a);
        a = dot2(w.y, xv.y, a);
        a = dot2(w.z, xv.z, a);
        a = dot2(w.w, xv.w, a);
        acc[j] = a;
      }
    }
  }
  // kIx: the symbols are in the indexed walk's lane slots.
  template <bool kIx = false>
  __device__ __forceinline__ uint32_t consume(Smem& S, uint32_t lane, const Stream& st, uint32_t pos0,
                                              uint32_t avail, bool final, const SmWin& W) {
    const uint32_t take = final ? avail : (avail & ~255u);
    const uint32_t units = take >> 3;
#pragma unroll
    for (uint32_t i = 0; i < kSmWin; ++i) {
      const uint32_t u = lane + kWave * i;
      if (u < units) unit<kIx>(S, st, pos0, u, W.v[i]);
    }
    for (uint32_t u = lane + kSmWin * kWave; u < units; u += kWave)
      unit<kIx>(S, st, pos0, u, ldg64(st.sm + pos0 + 8 * u));
    return take;
  }
  __device__ __forceinline__ void deposit(float* slots, uint32_t lane, uint32_t s0) {
    const uint32_t su = (s0 >> 3) & 1u;
    const int partner = (int)((((lane + su) ^ 1u) - su) & 63u);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      acc[j] += __shfl(acc[j], partner, kWave);
      acc[j] += __shfl_xor(acc[j], 32, kWave);
    }
    const uint32_t row = (((s0 >> 3) + lane) >> 1) & 15u;
    if (lane < 32 && ((lane + su) & 1u) == 0)
#pragma unroll
      for (int j = 0; j < NB; ++j) slots[row * NB + j] += acc[j];
  }
  // An item's record (row r, column j < nb at r * nb + j): the same two
  // exchanges as deposit, then the one lane per row that deposit would use
  // stores the row's sums; those 16 lanes cover the 16 rows once.
  __device__ __forceinline__ void record(float* part, uint32_t nb, uint32_t lane, uint32_t s0) {
    const uint32_t su = (s0 >> 3) & 1u;
    const int partner = (int)((((lane + su) ^ 1u) - su) & 63u);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      acc[j] += __shfl(acc[j], partner, kWave);
      acc[j] += __shfl_xor(acc[j], 32, kWave);
    }
    const uint32_t row = (((s0 >> 3) + lane) >> 1) & 15u;
    if (lane < 32 && ((lane + su) & 1u) == 0)
#pragma unroll
      for (int j = 0; j < NB; ++j)
        if (j < (int)nb) part[row * nb + j] = acc[j];
  }
};

// bf16 activations (layout of GemmBf16), bf16 MFMA with fp32 accumulation
// (batch 1..16, padded to 16): v_mfma_f32_16x16x32_bf16 multiplies a 16 x 32
// slice of W (two 16x16 tiles side by side) by a 32 x 16 slice of X.  Lane
// l = r + 16 g supplies W row r, columns 8g..8g+7 of the slice -- exactly one
// decoded unit (half a tile row, unit 32 (g / 2) + 2 r + g % 2 of the tile
// pair) -- and X rows (batch) l % 16 of the same 8 columns; it accumulates
// Y rows 4 g .. 4 g + 3 of batch column l % 16.  Streams must cover whole
// tiles.
struct GemmMfma {
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  static constexpr int kCols = 16, kOut = 256;
  const uint16_t* x;
  uint64_t ldx;
  uint32_t nb;
  bool xa;          // x and its row stride are 16-byte aligned
  bool xs = false;  // this segment's x columns are staged in LDS (kXOff)
  f32x4 acc;
  __device__ __forceinline__ explicit GemmMfma(const GemmArgs& a)
      : x(static_cast<const uint16_t*>(a.x)), ldx(a.ldx), nb(a.nb),
        xa(((uintptr_t)a.x & 15u) == 0 && a.ldx % 8 == 0) {}
  // Rows r < nb of the segment's whole tiles t .. t + 7 (16 pieces of 16
  // bytes per row).  Slot q holds row r = q / 16, piece (q % 16) ^ r: the
  // XOR spreads the 16 rows a consume read touches over all LDS banks.
  __device__ __forceinline__ void stage_x(Smem& S, uint32_t lane, const Stream& st, uint32_t pos0, uint32_t n) {
    xs = xa;
    if (!xs) return;
    const uint32_t t = (st.start + pos0) >> 8, tiles = (n + 255) >> 8;
    for (uint32_t i = 0; kWave * i < 16 * nb; ++i) {
      const uint32_t q = kWave * i + lane, r = q >> 4, pc = (q & 15u) ^ r;
      copy_to_lds16(r < nb && pc < 2 * tiles ? x + r * ldx + 16ull * t + 8 * pc : x, S.syms + kXOff + 1024 * i);
    }
  }
  static __device__ __forceinline__ uint32_t lane_unit(uint32_t lane) {
    const uint32_t r = lane & 15u, g = lane >> 4;
    return 32u * (g >> 1) + 2u * r + (g & 1u);
  }
  static __device__ __forceinline__ bool fits(uint32_t s0, uint32_t count, uint64_t rows, uint64_t cols) {
    return rows == 16 && cols % 16 == 0 && s0 % 256 == 0 && count % 256 == 0;
  }
  static __device__ __forceinline__ void store(const GemmArgs& a, uint64_t dst, uint32_t r, uint32_t j, float v) {
    if (j < a.nb) a.y[j * a.ldy + dst + r] = v;
  }
  __device__ __forceinline__ void init() { acc = f32x4{0.f, 0.f, 0.f, 0.f}; }
  // kIx: the symbols are in the indexed walk's lane slots.
  template <bool kIx = false>
  __device__ __forceinline__ uint32_t consume(Smem& S, uint32_t lane, const Stream& st, uint32_t pos0,
                                              uint32_t avail, bool final, const SmWin& W) {
    const uint32_t take = final ? avail : (avail & ~255u);  // whole tiles for fitting streams
    const uint32_t units = take >> 3, lu = lane_unit(lane), g = lane >> 4, n = lane & 15u;
    const uint32_t t0 = (st.start + pos0) >> 8;  // slab tile of the call's first symbol
    const uint16_t* xr = x + n * ldx;
    for (uint32_t b = 0; 64 * b < units; ++b) {
      const uint32_t u = 64 * b + lu;
      const bool valid = u < units;  // an odd tile count leaves the last pair half empty
      uint64_t E = 0, M = 0;
      if (valid) {
        E = unit_exps<kIx>(S.syms, u);
        M = b < kSmWin ? W.v[b] : ldg64(st.sm + pos0 + 8 * u);
      }
      const uint4 w = combine8(E, M);
      uint4 xv = make_uint4(0u, 0u, 0u, 0u);
      if (valid && n < nb) {
        if (xs)
          xv = lds16(S.syms + kXOff + 16u * (16u * n + ((4u * b + 2u * (g >> 1) + (g & 1u)) ^ n)));
        else
          __builtin_memcpy(&xv, xr + 16u * (t0 + 2 * b + (g >> 1)) + 8u * (g & 1u), 16);
      }
      bf16x8 a, bb;
      __builtin_memcpy(&a, &w, 16);
      __builtin_memcpy(&bb, &xv, 16);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bb, acc, 0, 0, 0);
    }
    return take;
  }
  __device__ __forceinline__ void deposit(float* slots, uint32_t lane, uint32_t) {
    const uint32_t r0 = 4u * (lane >> 4), n = lane & 15u;
    slots[(r0 + 0) * 16 + n] += acc[0];
    slots[(r0 + 1) * 16 + n] += acc[1];
    slots[(r0 + 2) * 16 + n] += acc[2];
    slots[(r0 + 3) * 16 + n] += acc[3];
  }
  // An item's record, packed as the slots path packs it (row r, column n < nb
  // at r * nb + n): lane l holds rows 4 (l / 16) .. + 3 of column l % 16.
  __device__ __forceinline__ void record(float* part, uint32_t nb, uint32_t lane, uint32_t) const {
    const uint32_t r0 = 4u * (lane >> 4), n = lane & 15u;
    if (n < nb) {
      part[(r0 + 0) * nb + n] = acc[0];
      part[(r0 + 1) * nb + n] = acc[1];
      part[(r0 + 2) * nb + n] = acc[2];
      part[(r0 + 3) * nb + n] = acc[3];
    }
  }
};

// ----------------------------------------------------------------- kernels

__device__ __forceinline__ void set_status(uint32_t* status, uint32_t slot, uint32_t err, uint32_t lane) {
  if (err && lane == 0) atomicOr(status + slot, err);
}

// Up to 36 leading 64-bit words of a block (XKSP2 header + segment lengths),
// one per lane, never reading past the block.
__device__ __forceinline__ uint64_t issue_head(const uint8_t* blk, uint64_t size, uint32_t lane) {
  if (lane >= 36) return 0ull;
  const uint64_t at = 8ull * lane;
  if (at + 8 <= size) return ldg64(blk + at);
  uint64_t v = 0;
  for (uint64_t i = 0; i < 8; ++i)
    if (at + i < size) v |= (uint64_t)blk[at + i] << (8 * i);
  return v;
}

// XKSP2 block header checks [src/c_api.cpp:66-72, 78, cuda/parallel.cu:132-139]
// on the words from issue_head.  Sets chunks; lane 4 + k holds segment k's length.
__device__ __forceinline__ uint32_t check_head(uint64_t hv, uint64_t size, const DevBlock& d, uint32_t lane,
                                               uint32_t& chunks) {
  chunks = 0;
  if (size < 32) return kErrHeader;
  const uint64_t magic = rdlane64(hv, 0), rows = rdlane64(hv, 1), cols = rdlane64(hv, 2), nch = rdlane64(hv, 3);
  if (magic != kMagicXKSP2 || !rows || rows > 16 || !cols || !nch || nch > 32 || cols > ~0ull / rows)
    return kErrHeader;
  const uint64_t total = rows * cols;
  if (nch > total || total > size || total > ~0ull / 32 || size < 32 + 8 * nch) return kErrHeader;
  if (rows != d.rows || cols != d.cols || total > kMaxBlockElems) return kErrShape;
  const bool mine = lane >= 4 && lane < 4 + nch;
  const uint64_t len = mine ? hv : 0ull;
  if (__ballot(mine && (len < 272 || len > size))) return kErrHeader;
  const uint64_t sum = rdlane64(wave_incl(len, lane), 63);
  if (32 + 8 * nch + sum != size) return kErrHeader;
  chunks = (uint32_t)nch;
  return 0;
}

// Substream starts of a block: lane q (q <= chunks) gets total * q / chunks
// (the reference's split, cuda/parallel.cu:33-51), one division per lane per
// block instead of several per substream.
__device__ __forceinline__ uint32_t substream_starts(uint64_t total, uint32_t chunks, uint32_t lane) {
  return lane <= chunks && chunks ? (uint32_t)(total * lane / chunks) : 0u;
}

// The block this wave decodes after `b`.  With a queue (a counter the host
// zeroes before the launch) the first gridDim.x blocks go one per workgroup and
// each later one to whichever wave asks first, which balances blocks of
// different sizes; without one, a grid stride.
__device__ __forceinline__ uint32_t claim_next(uint32_t* queue, uint32_t b, uint32_t lane) {
  if (!queue) return b + gridDim.x;
  uint32_t t = 0;
  if (lane == 0) t = atomicAdd(queue, 1u);
  return gridDim.x + rdlane(t, 0);
}

// Substream k's codeword index within a per-block index (launch_index_items
// with `ibase`), or nullptr: none given, or more symbols than the block's
// allotment holds (the indexed walk then never reads past the allotment).
__device__ __forceinline__ const uint16_t* stream_index(const uint16_t* index, const uint64_t* ibase, uint32_t b,
                                                        uint32_t k, uint32_t count) {
  if (!index) return nullptr;
  const uint64_t o0 = ibase[b];
  const uint32_t segs = (uint32_t)((ibase[b + 1] - o0) / (64u * kMaxChunks));
  return count <= segs * kIdxSegSyms ? index + o0 + (uint64_t)k * segs * 64 : nullptr;
}

// Decode XKSP2 blocks: one wave per block, its substreams in order, each
// substream's inputs prefetched while the previous one decodes; the next
// block's header is prefetched at the start of each block.  Blocks from
// `split` on (the plan lists its largest blocks first, so these are its
// smallest, one grid's worth) are claimed a quarter at a time -- substreams
// [chunks q / 4, chunks (q + 1) / 4) -- so that the waves drain together:
// a whole small block is ~0.3 ms of one wave's work, a quarter ~75 us.  Each
// claim reports its block's header and stream errors into the block's status
// word (an OR).
constexpr uint32_t kTailSplit = 4;
// kIdx: with a codeword index (a separate instantiation, so that the decode
// without one compiles as if the indexed walk did not exist).
template <bool kIdx>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3)))
k_decode_parallel(const DevBlock* __restrict__ blocks, uint32_t nblocks,
                                                        const uint8_t* __restrict__ arc, uint8_t* __restrict__ out,
                                                        uint32_t* __restrict__ status, uint32_t* queue,
                                                        const uint16_t* __restrict__ index,
                                                        const uint64_t* __restrict__ ibase, uint32_t split) {
  __shared__ Smem S;
  const uint32_t lane = lane_id();
  const uint32_t nclaims = split + (nblocks - split) * kTailSplit;
  const auto block_of = [split](uint32_t c) { return c < split ? c : split + (c - split) / kTailSplit; };
  uint32_t c = blockIdx.x;
  uint64_t hv = c < nclaims ? issue_head(arc + blocks[block_of(c)].src, blocks[block_of(c)].size, lane) : 0ull;
  for (uint32_t cn; c < nclaims; c = cn) {
    const uint32_t b = block_of(c);
    const DevBlock d = blocks[b];
    const uint8_t* blk = arc + d.src;
    uint32_t chunks;
    uint32_t err = check_head(hv, d.size, d, lane, chunks);
    const uint64_t seglen_v = hv;
    cn = claim_next(queue, c, lane);
    if (cn < nclaims) hv = issue_head(arc + blocks[block_of(cn)].src, blocks[block_of(cn)].size, lane);
    if (err) {
      set_status(status, d.status_slot, err, lane);
      continue;
    }
    const uint32_t q = c < split ? 0u : (c - split) % kTailSplit;
    const uint32_t k0 = c < split ? 0u : chunks * q / kTailSplit;
    const uint32_t k1 = c < split ? chunks : chunks * (q + 1) / kTailSplit;
    if (k0 >= k1) continue;  // fewer than kTailSplit substreams: an empty quarter
    const uint64_t total = d.rows * d.cols;
    const bool aligned = d.rows % 16 == 0 && d.cols % 16 == 0;
    Writer C{out + d.dst, d.rows, d.cols, (uint32_t)(d.cols / 16), false};
    // Substream k0's segment follows the header, the length table and the
    // segments before it (lane 4 + j holds segment j's length).
    uint64_t off = 32 + 8ull * chunks;
    if (k0) off += rdlane64(wave_incl((uint64_t)(lane >= 4 && lane < 4 + k0 ? seglen_v : 0ull), lane), 63);
    uint64_t len = rdlane64(seglen_v, 4 + k0);
    const uint32_t starts = substream_starts(total, chunks, lane);
    StreamIn PN;
    issue_stream(PN, blk + off, blk + off + len, rdlane(starts, k0 + 1) - rdlane(starts, k0), lane);
    drain_loads();
    stage_inputs(S, lane, PN);
    for (uint32_t k = k0; k < k1 && !err; ++k) {
      const uint32_t s0 = rdlane(starts, k), s1 = rdlane(starts, k + 1);
      const uint64_t noff = off + len;
      const uint64_t nlen = k + 1 < k1 ? rdlane64(seglen_v, 4 + k + 1) : 0ull;
      const uint32_t ncount = k + 1 < k1 ? rdlane(starts, k + 2) - s1 : 0u;
      C.aligned = aligned && unit_aligned(s0, s1 - s0, d.rows, d.cols);
      err = run_stream(S, lane, blk + off, blk + off + len, s1 - s0, s0, C,
                       NextStream{k + 1 < k1 ? blk + noff : nullptr, blk + noff + nlen, ncount}, PN,
                       kIdx ? stream_index(index, ibase, b, k, s1 - s0) : nullptr);
      off = noff;
      len = nlen;
    }
    set_status(status, d.status_slot, err, lane);
  }
}

// Decode serial blocks: one wave per block (one stream), the next block's
// inputs prefetched while this one decodes.
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3)))
k_decode_serial(const DevBlock* __restrict__ blocks, uint32_t nblocks, const uint8_t* __restrict__ arc,
                uint8_t* __restrict__ out, uint32_t* __restrict__ status, uint32_t* queue) {
  __shared__ Smem S;
  const uint32_t lane = lane_id();
  StreamIn PN;
  uint32_t b = blockIdx.x;
  if (b < nblocks && blocks[b].size >= 272) {
    issue_stream(PN, arc + blocks[b].src, arc + blocks[b].src + blocks[b].size,
                 (uint32_t)(blocks[b].rows * blocks[b].cols), lane);
    drain_loads();
    stage_inputs(S, lane, PN);
  }
  for (uint32_t bn; b < nblocks; b = bn) {
    const DevBlock d = blocks[b];
    bn = claim_next(queue, b, lane);
    const bool has_next = bn < nblocks && blocks[bn].size >= 272;
    const DevBlock dn = has_next ? blocks[bn] : d;
    uint32_t err = 0;
    if (d.size < 272 || !d.rows || !d.cols || d.cols > ~0ull / d.rows) err = kErrHeader;
    else if (d.rows * d.cols > kMaxBlockElems) err = kErrShape;
    if (!err) {
      const uint32_t n = (uint32_t)(d.rows * d.cols);
      Writer C{out + d.dst, d.rows, d.cols, (uint32_t)(d.cols / 16), unit_aligned(0, n, d.rows, d.cols)};
      err = run_stream(S, lane, arc + d.src, arc + d.src + d.size, n, 0, C,
                       NextStream{has_next ? arc + dn.src : nullptr, arc + dn.src + dn.size,
                                  (uint32_t)(dn.rows * dn.cols)},
                       PN);
    } else if (has_next) {
      issue_stream(PN, arc + dn.src, arc + dn.src + dn.size, (uint32_t)(dn.rows * dn.cols), lane);
      drain_loads();
      stage_inputs(S, lane, PN);
    }
    set_status(status, d.status_slot, err, lane);
  }
}

// Serial-codec blocks at workgroup scale: kSerialWaves waves share a block.
// Pass 1: wave w decodes the codewords that start in its share of the code
// bits, [nbits w / W, nbits (w + 1) / W), from a speculative entry (as a lane
// enters its chunk) into its scratch region, and records its first codeword
// start, its exit and its count.  Then, wave by wave, a range whose first
// start is not its predecessor's exit is decoded again from that exit; a
// range in which no codeword starts passes the exit on.  The block then
// follows the reference's serial walk: a range's decode error counts once its
// start is proven, the counts must add up to the element count, and the last
// range must end on the stream's last bit.  Pass 2: each wave places its
// symbols at the sum of the counts before it.  A block whose stream is short,
// invalid, needs the bit-serial path, or overflows a scratch region is
// decoded by wave 0 alone.
struct SerialPart {
  uint64_t first, exit;
  uint32_t count, err;
};
__global__ void __launch_bounds__(64 * kSerialWaves)
k_decode_serial_wg(const DevBlock* __restrict__ blocks, uint32_t nblocks, const uint8_t* __restrict__ arc,
                   uint8_t* __restrict__ out, uint32_t* __restrict__ status, uint8_t* __restrict__ scratch,
                   uint32_t cap) {
  __shared__ Smem SS[kSerialWaves];
  __shared__ SerialPart R[kSerialWaves];
  __shared__ uint32_t over;
  const uint32_t lane = lane_id(), w = threadIdx.x / kWave;
  Smem& S = SS[w];
  uint8_t* const mine = scratch + ((uint64_t)blockIdx.x * kSerialWaves + w) * cap;
  for (uint32_t b = blockIdx.x; b < nblocks; b += gridDim.x) {
    if (threadIdx.x == 0) over = 0;
    __syncthreads();
    const DevBlock d = blocks[b];
    if (d.size < 272 || !d.rows || !d.cols || d.cols > ~0ull / d.rows || d.rows * d.cols > kMaxBlockElems) {
      if (w == 0) set_status(status, d.status_slot, d.size < 272 || !d.rows || !d.cols || d.cols > ~0ull / d.rows
                                                        ? kErrHeader : kErrShape, lane);
      continue;  // the same block, the same verdict in every wave
    }
    const uint32_t n = (uint32_t)(d.rows * d.cols);
    const uint8_t* const seg = arc + d.src;
    const uint8_t* const seg_end = seg + d.size;
    StreamIn PN;
    issue_stream(PN, seg, seg_end, n, lane);
    drain_loads();
    stage_inputs(S, lane, PN);
    const uint64_t cnt = reinterpret_cast<const uint64_t*>(S.bcast)[0], nb = reinterpret_cast<const uint64_t*>(S.bcast)[1];
    const uint32_t lw = reinterpret_cast<const uint32_t*>(S.sorted)[lane];
    wave_sync();
    const bool head_ok = cnt == n && cnt <= d.size - 272 && nb / 8 + (nb % 8 != 0) == d.size - 272 - cnt;
    Book bk{0, 0, false};
    if (head_ok) bk = build_book(S, lane, lw);
    const bool split = head_ok && !bk.err && bk.fast && nb >= 64ull * kSerialWaves;  // workgroup-uniform
    uint32_t errs = 0;
    if (split) {
      Stream st;
      st.lengths = seg + 16;
      st.sm = seg + 272;
      st.bits = st.sm + cnt;
      st.nbits = nb;
      st.count = n;
      st.start = 0;
      const uint64_t b1 = nb * (w + 1) / kSerialWaves;
      // Round 0 decodes every range from its speculative entry; round v >= 1
      // proves range v's start (and decodes it again from its predecessor's
      // exit when it is not that exit).  One decode call site for all rounds.
      uint64_t from = nb * w / kSerialWaves;
      bool spec = w > 0, todo = true;
      for (uint32_t v = 0; v < kSerialWaves; ++v) {
        if (todo) {
          ScratchWriter C{mine, cap};
          Range rg{b1, spec, from, b1, 0u};
          const uint32_t e = decode_fast(S, lane, st, bk.maxlen, seg_end, C, PN, false, from, 0, &rg);
          if (lane == 0) {
            R[w] = SerialPart{rg.first, rg.exit, rg.count, e};
            if (C.overflow) over = 1;
          }
        }
        __syncthreads();
        if (v + 1 == kSerialWaves) break;
        const uint32_t u = v + 1;
        const uint64_t px = R[v].exit, ub1 = nb * (u + 1) / kSerialWaves;
        const bool pass = px >= ub1;  // no codeword starts in range u
        const bool redo = !pass && R[u].first != px;
        __syncthreads();  // every wave has read R before wave u rewrites it
        if (w == u && pass && lane == 0) R[u] = SerialPart{px, px, 0u, 0u};
        todo = w == u && redo;
        from = px;
        spec = false;
      }
      uint32_t tot = 0, pre = 0;
      for (uint32_t v = 0; v < kSerialWaves; ++v) {
        pre += v < w ? R[v].count : 0u;
        tot += R[v].count;
        errs |= R[v].err;
      }
      if (!errs && (tot != n || R[kSerialWaves - 1].exit != nb)) errs = kErrStream;
      if (!over && !errs)
        place_range(mine, st, pre, R[w].count, out + d.dst, d.rows, d.cols, unit_aligned(0, n, d.rows, d.cols),
                    lane);
    }
    if (!split || over) {  // one wave, the single-wave path from the stream's start
      if (w == 0) {
        issue_stream(PN, seg, seg_end, n, lane);
        drain_loads();
        stage_inputs(S, lane, PN);
        Writer C{out + d.dst, d.rows, d.cols, (uint32_t)(d.cols / 16), unit_aligned(0, n, d.rows, d.cols)};
        errs = run_stream(S, lane, seg, seg_end, n, 0, C, NextStream{nullptr, nullptr, 0u}, PN);
      }
    }
    if (w == 0) set_status(status, d.status_slot, errs, lane);
    __syncthreads();  // R, `over` and the scratch regions are reused by the next block
  }
}

// Fused decode-GEMM over 16-row slabs with consumer Acc (GemmF32, GemmBf16,
// GemmMfma).  One workgroup of W waves per block: wave w takes substreams w,
// w + W, ... (prefetching each next one), adds its partial sums into its own
// LDS slots after every substream, and the workgroup sums the W slots in wave
// order.  No atomics, deterministic.
template <int W, class Acc>
__global__ void __launch_bounds__(64 * W) k_gemm(const DevBlock* __restrict__ blocks, uint32_t nblocks,
                                                 uint32_t codec, const uint8_t* __restrict__ arc, GemmArgs ga,
                                                 uint32_t* __restrict__ status) {
  __shared__ Smem SS[W];
  __shared__ float red[W][Acc::kOut];
  __shared__ uint32_t werr[W];
  const uint32_t lane = lane_id(), w = threadIdx.x / 64;
  Smem& S = SS[w];
  for (uint32_t b = blockIdx.x; b < nblocks; b += gridDim.x) {
    const DevBlock d = blocks[b];
    const uint8_t* blk = arc + d.src;
    for (uint32_t i = lane; i < (uint32_t)Acc::kOut; i += kWave) red[w][i] = 0.f;
    uint32_t err = 0, chunks = 1;
    uint64_t hv = 0;
    if (codec == kCodecParallel) {
      hv = issue_head(blk, d.size, lane);
      err = check_head(hv, d.size, d, lane, chunks);
    } else if (d.size < 272 || d.rows != 16 || !d.cols || d.rows * d.cols > kMaxBlockElems) {
      err = kErrHeader;
    }
    if (!err && (d.rows != 16 || d.cols % 16)) err = kErrShape;
    if (!err) {
      const uint64_t total = d.rows * d.cols;
      // segment offsets: walk to this wave's first substream
      uint64_t off = codec == kCodecParallel ? 32 + 8ull * chunks : 0, len = d.size;
      uint32_t k = w;
      if (codec == kCodecParallel) {
        for (uint32_t q = 0; q < k && q < chunks; ++q) off += rdlane64(hv, 4 + q);
        len = k < chunks ? rdlane64(hv, 4 + k) : 0;
      }
      const uint32_t starts = substream_starts(total, chunks, lane);
      StreamIn PN;
      if (k < chunks) {
        issue_stream(PN, blk + off, blk + off + len, rdlane(starts, k + 1) - rdlane(starts, k), lane);
        drain_loads();
        stage_inputs(S, lane, PN);
      }
      for (; k < chunks && !err; k += W) {
        const uint32_t s0 = rdlane(starts, k), s1 = rdlane(starts, k + 1);
        // next substream of this wave
        uint64_t noff = off, nlen = 0;
        const uint32_t kn = k + W;
        if (kn < chunks) {
          for (uint32_t q = k; q < kn; ++q) noff += rdlane64(hv, 4 + q);
          nlen = rdlane64(hv, 4 + kn);
        }
        const uint32_t ncount = kn < chunks ? rdlane(starts, kn + 1) - rdlane(starts, kn) : 0u;
        if (!Acc::fits(s0, s1 - s0, d.rows, d.cols)) {
          err = kErrShape;
          break;
        }
        Acc C(ga);
        C.init();
        err = run_stream(S, lane, blk + off, blk + off + len, s1 - s0, s0, C,
                         NextStream{kn < chunks ? blk + noff : nullptr, blk + noff + nlen, ncount}, PN);
        C.deposit(red[w], lane, s0);
        off = noff;
        len = nlen;
      }
    }
    if (lane == 0) werr[w] = err;
    __syncthreads();
    uint32_t any = 0;
    for (uint32_t q = 0; q < W; ++q) any |= werr[q];
    if (w == 0) {
      set_status(status, d.status_slot, any, lane);
      if (!any)
        for (uint32_t i = lane; i < (uint32_t)Acc::kOut; i += kWave) {
          float sum = 0.f;
#pragma unroll
          for (int q = 0; q < W; ++q) sum += red[q][i];
          Acc::store(ga, d.dst, i / Acc::kCols, i % Acc::kCols, sum);
        }
    }
    __syncthreads();
  }
}

// Where work item i (substream i % kMaxChunks of block i / kMaxChunks) lies,
// from its block's header words (issue_head).  `run` = the item decodes;
// otherwise err says why not (0: the block has fewer substreams).
struct ItemLoc {
  const uint8_t* seg;
  const uint8_t* end;
  uint32_t count, s0, chunks, err;
  bool run;
};
// Substream k of an XKSP2 block from the header words of issue_head: its
// segment, element count and first tiled position (run = false when the
// header fails or the block has no substream k).
__device__ __forceinline__ ItemLoc locate_sub(const DevBlock& d, const uint8_t* blk, uint32_t k, uint64_t hv,
                                              uint32_t lane) {
  ItemLoc L{nullptr, nullptr, 0u, 0u, 0u, 0u, false};
  L.err = check_head(hv, d.size, d, lane, L.chunks);
  if (L.err || k >= L.chunks) return L;
  const uint64_t len = lane >= 4 && lane < 4 + L.chunks ? hv : 0ull;
  const uint64_t incl = wave_incl(len, lane);
  const uint64_t end = 32 + 8ull * L.chunks + rdlane64(incl, 4 + k);
  const uint64_t total = d.rows * d.cols;
  const uint32_t starts = substream_starts(total, L.chunks, lane);
  L.s0 = rdlane(starts, k);
  L.count = rdlane(starts, k + 1) - L.s0;
  L.seg = blk + (end - rdlane64(len, 4 + k));
  L.end = blk + end;
  L.run = true;
  return L;
}
// As locate_sub, for a fused GEMM item: the slab must be 16 full-tile rows and
// the substream fit consumer Acc.
template <class Acc>
__device__ __forceinline__ ItemLoc locate_item(const DevBlock& d, const uint8_t* blk, uint32_t k, uint64_t hv,
                                               uint32_t lane) {
  ItemLoc L = locate_sub(d, blk, k, hv, lane);
  if (!L.err && (d.rows != 16 || d.cols % 16)) L.err = kErrShape;
  if (L.err && L.run) L.run = false;
  if (L.run && !Acc::fits(L.s0, L.count, d.rows, d.cols)) {
    L.err = kErrShape;
    L.run = false;
  }
  return L;
}

// Decode XKSP2 blocks by substream (work item i = substream i % 32 of block
// i / 32; wave w takes items w, w + gridDim.x, ...): for plans with fewer
// blocks than resident waves, where one wave per block would leave the GPU
// idle and run each block's substreams one after another.  The next item's
// inputs and the header of the one after load while an item decodes.
template <bool kIdx>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3)))
k_decode_items(const DevBlock* __restrict__ blocks, uint32_t nblocks, const uint8_t* __restrict__ arc,
               uint8_t* __restrict__ out, uint32_t* __restrict__ status, const uint16_t* __restrict__ index,
               const uint64_t* __restrict__ ibase) {
  __shared__ Smem S;
  const uint32_t lane = lane_id(), stride = gridDim.x;
  const uint32_t nitems = nblocks * kMaxChunks;
  uint32_t i = blockIdx.x;
  if (i >= nitems) return;
  uint64_t hv = issue_head(arc + blocks[i / kMaxChunks].src, blocks[i / kMaxChunks].size, lane);
  uint64_t hvn = i + stride < nitems
                     ? issue_head(arc + blocks[(i + stride) / kMaxChunks].src, blocks[(i + stride) / kMaxChunks].size, lane)
                     : 0ull;
  ItemLoc L = locate_sub(blocks[i / kMaxChunks], arc + blocks[i / kMaxChunks].src, i % kMaxChunks, hv, lane);
  StreamIn PN;
  if (L.run) {
    issue_stream(PN, L.seg, L.end, L.count, lane);
    drain_loads();
    stage_inputs(S, lane, PN);
  }
  for (;;) {
    const uint32_t in = i + stride, inn = in + stride, k = i % kMaxChunks;
    const DevBlock d = blocks[i / kMaxChunks];
    ItemLoc LN{nullptr, nullptr, 0u, 0u, 0u, 0u, false};
    uint64_t hvnn = 0ull;
    if (in < nitems) {
      const DevBlock dn = blocks[in / kMaxChunks];
      LN = locate_sub(dn, arc + dn.src, in % kMaxChunks, hvn, lane);
      if (inn < nitems) hvnn = issue_head(arc + blocks[inn / kMaxChunks].src, blocks[inn / kMaxChunks].size, lane);
    }
    uint32_t err = L.err;  // a header error is reported by the block's item 0
    if (L.run) {
      const bool aligned = d.rows % 16 == 0 && d.cols % 16 == 0 && unit_aligned(L.s0, L.count, d.rows, d.cols);
      Writer C{out + d.dst, d.rows, d.cols, (uint32_t)(d.cols / 16), aligned};
      err = run_stream(S, lane, L.seg, L.end, L.count, L.s0, C,
                       NextStream{LN.run ? LN.seg : nullptr, LN.end, LN.count}, PN,
                       kIdx ? stream_index(index, ibase, i / kMaxChunks, k, L.count) : nullptr);
    } else if (LN.run) {
      issue_stream(PN, LN.seg, LN.end, LN.count, lane);
      drain_loads();
      stage_inputs(S, lane, PN);
    }
    if (k == 0 || L.run) set_status(status, d.status_slot, err, lane);
    if (in >= nitems) break;
    i = in;
    L = LN;
    hvn = hvnn;
  }
}

// Fused decode-GEMM over XKSP2 blocks of 16-row slabs, one substream per work
// item (item i = substream i % 32 of block i / 32): wave w of the grid takes
// items w, w + gridDim.x, ..., so all resident waves share a layer's blocks x
// 32 substreams whatever the block count, and the waves running at any one
// time work on neighbouring items (one compact window of the archive).  Per
// item a wave decodes the substream into consumer Acc and writes a record:
// its partial sums (batch columns < nb) and its error word; item 0 of each
// block records the block's substream count.  k_gemm_finish adds a block's
// records in order and stores its status word, so no status reset precedes
// the launch.  The next item's inputs and the header of the one after load
// while an item decodes.
template <class Acc>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3)))
k_gemm_items(const DevBlock* __restrict__ blocks, uint32_t nblocks, const uint8_t* __restrict__ arc, GemmArgs ga,
             ItemScratch is) {
  __shared__ Smem S;
  const uint32_t lane = lane_id(), stride = gridDim.x;
  const uint32_t nitems = nblocks * kMaxChunks;
  uint32_t i = blockIdx.x;
  if (i >= nitems) return;
  uint64_t hv = issue_head(arc + blocks[i / kMaxChunks].src, blocks[i / kMaxChunks].size, lane);
  uint64_t hvn = i + stride < nitems
                     ? issue_head(arc + blocks[(i + stride) / kMaxChunks].src, blocks[(i + stride) / kMaxChunks].size, lane)
                     : 0ull;
  ItemLoc L = locate_item<Acc>(blocks[i / kMaxChunks], arc + blocks[i / kMaxChunks].src, i % kMaxChunks, hv, lane);
  StreamIn PN;
  if (L.run) {
    issue_stream(PN, L.seg, L.end, L.count, lane);
    drain_loads();
    stage_inputs(S, lane, PN);
  }
  for (;;) {
    const uint32_t in = i + stride, inn = in + stride, b = i / kMaxChunks, k = i % kMaxChunks;
    ItemLoc LN{nullptr, nullptr, 0u, 0u, 0u, 0u, false};
    uint64_t hvnn = 0ull;
    if (in < nitems) {
      const DevBlock dn = blocks[in / kMaxChunks];
      LN = locate_item<Acc>(dn, arc + dn.src, in % kMaxChunks, hvn, lane);
      if (inn < nitems) hvnn = issue_head(arc + blocks[inn / kMaxChunks].src, blocks[inn / kMaxChunks].size, lane);
    }
    if (k == 0 && lane == 0) is.done[b] = L.err ? 0u : L.chunks;
    uint32_t err = L.err;  // a substream past the count carries no error of its own
    if (L.run) {
      Acc C(ga);
      C.init();
      // (an item with more symbols than its allotment holds has no index entry)
      const uint16_t* idx =
          is.index && L.count <= is.index_segs * kIdxSegSyms ? is.index + (uint64_t)i * is.index_segs * 64 : nullptr;
      err = run_stream<Acc>(S, lane, L.seg, L.end, L.count, L.s0, C,
                                 NextStream{LN.run ? LN.seg : nullptr, LN.end, LN.count}, PN, idx);
      // Live batch columns only, packed: row r, column j < nb at r * nb + j;
      // every output of the item sits in one lane, which stores it.
      C.record(is.partial + (uint64_t)i * kMaxItemOut, ga.nb, lane, L.s0);
    } else if (LN.run) {
      issue_stream(PN, LN.seg, LN.end, LN.count, lane);
      drain_loads();
      stage_inputs(S, lane, PN);
    }
    if (lane == 0) is.err[i] = err;
    if (in >= nitems) break;
    i = in;
    L = LN;
    hvn = hvnn;
  }
}

// Y and the status word of every block from its items' records, added in
// substream order (fixed, so the result does not depend on which wave ran
// which item).  The status word is stored, not ORed: the launch needs no
// prior reset.  One wave per block.
template <class Acc>
__global__ void __launch_bounds__(64) k_gemm_finish(const DevBlock* __restrict__ blocks, uint32_t nblocks,
                                                    GemmArgs ga, uint32_t* __restrict__ status, ItemScratch is) {
  const uint32_t lane = lane_id();
  for (uint32_t b = blockIdx.x; b < nblocks; b += gridDim.x) {
    const DevBlock d = blocks[b];
    const uint32_t chunks = is.done[b];
    const uint32_t nrec = chunks ? chunks : 1u;  // a header error is item 0's
    uint32_t err = lane < nrec ? is.err[b * kMaxChunks + lane] : 0u;
#pragma unroll
    for (int m = 1; m < (int)kWave; m <<= 1) err |= __shfl_xor(err, m, kWave);
    if (lane == 0) status[d.status_slot] = err;
    if (err || !chunks) continue;
    const float* part = is.partial + (uint64_t)b * kMaxChunks * kMaxItemOut;
    for (uint32_t o = lane; o < 16 * ga.nb; o += kWave) {  // packed records: row o / nb, column o % nb
      float v[kMaxChunks];
#pragma unroll
      for (uint32_t k = 0; k < kMaxChunks; ++k) v[k] = k < chunks ? part[k * kMaxItemOut + o] : 0.f;
      float sum = 0.f;
#pragma unroll
      for (uint32_t k = 0; k < kMaxChunks; ++k) sum += v[k];
      Acc::store(ga, d.dst, o / ga.nb, o % ga.nb, sum);
    }
  }
}

// ------------------------------------------------------ codeword index

// 8 bytes at p as a big-endian (MSB-first) 64-bit value; bytes at or past
// `end` read as zero.
__device__ __forceinline__ uint64_t load_be64(const uint8_t* p, const uint8_t* end) {
  uint64_t v;
  if (p + 8 <= end) {
    v = ldg64(p);
  } else {
    v = 0;
    for (uint32_t i = 0; i < 8; ++i)
      if (p + i < end) v |= (uint64_t)p[i] << (8 * i);
  }
  return __builtin_bswap64(v);
}

// Codeword index of the fused XKSP2 items (item i = substream i % kMaxChunks
// of block i / kMaxChunks), the load-time sidecar of static weights.  One lane
// per item: the lane checks its block and substream headers as decode does,
// builds the canonical per-length limits of its code lengths in its own LDS
// slice (lim[l] = left-aligned end of the codes of length <= l, the closed
// form of build_fast), and walks the code once, recording the bit offset of
// every kIdxLaneSyms-th codeword and each segment's length.  An item whose
// stream is invalid, has codes longer than 32 bits, or has a segment longer
// than kIdxMaxSpan bits gets kIdxNone: the fused kernels decode it
// speculatively and report its errors exactly as decode does.
struct IdxLane {
  uint64_t lim[34];
};
// `ibase` (optional, nblocks + 1 entries): block b's index starts at entry
// ibase[b] and holds (ibase[b + 1] - ibase[b]) / (64 kMaxChunks) segments per
// item; without it every item holds `segs` segments, item i at i * segs * 64.
__global__ void __launch_bounds__(64) k_index_items(const DevBlock* __restrict__ blocks, uint32_t nblocks,
                                                    const uint8_t* __restrict__ arc, uint16_t* __restrict__ index,
                                                    uint32_t segs, const uint64_t* __restrict__ ibase) {
  __shared__ IdxLane Lanes[64];
  uint64_t* lim = Lanes[threadIdx.x].lim;
  const uint32_t nitems = nblocks * kMaxChunks;
  for (uint32_t i = blockIdx.x * 64 + threadIdx.x; i < nitems; i += gridDim.x * 64) {
    const DevBlock d = blocks[i / kMaxChunks];
    const uint32_t k = i % kMaxChunks;
    if (ibase) segs = (uint32_t)((ibase[i / kMaxChunks + 1] - ibase[i / kMaxChunks]) / (64u * kMaxChunks));
    uint16_t* out = ibase ? index + ibase[i / kMaxChunks] + (uint64_t)k * segs * 64 : index + (uint64_t)i * segs * 64;
    const uint8_t* blk = arc + d.src;
    bool ok = false;
    if (d.size >= 32) {
      const uint64_t magic = ldg64(blk), rows = ldg64(blk + 8), cols = ldg64(blk + 16), chunks = ldg64(blk + 24);
      const bool head = magic == kMagicXKSP2 && rows == d.rows && cols == d.cols && rows && rows <= 16 && cols &&
                        cols <= kMaxBlockElems / rows && chunks && chunks <= kMaxChunks &&
                        chunks <= rows * cols && d.size >= 32 + 8 * chunks && k < chunks;
      uint64_t off = 32 + 8 * chunks, len = 0;
      bool seg_ok = head;
      for (uint32_t q = 0; seg_ok && q <= k; ++q) {
        len = ldg64(blk + 32 + 8 * q);
        if (len < 272 || len > d.size - off) seg_ok = false;
        else if (q < k) off += len;
      }
      const uint64_t total = rows * cols;
      const uint64_t s0 = seg_ok ? total * k / chunks : 0, count = seg_ok ? total * (k + 1) / chunks - s0 : 0;
      const uint8_t* seg = blk + off;
      uint64_t cnt = 0, nb = 0;
      if (seg_ok) {
        cnt = ldg64(seg);
        nb = ldg64(seg + 8);
        seg_ok = cnt == count && cnt <= len - 272 && nb / 8 + (nb % 8 != 0) == len - 272 - cnt &&
                 count <= (uint64_t)segs * kIdxSegSyms && count > 0;
      }
      uint32_t minlen = 64, maxlen = 0;
      if (seg_ok) {
        for (uint32_t l = 0; l < 34; ++l) lim[l] = 0;
        for (uint32_t q = 0; q < 64; ++q) {
          const uint32_t w = ldg32(seg + 16 + 4 * q);
          for (uint32_t j = 0; j < 4; ++j) {
            const uint32_t l = (w >> (8 * j)) & 255u;
            if (l > kMaxLenFast) seg_ok = false;
            else if (l) {
              lim[l] += 1;
              minlen = min(minlen, l);
              maxlen = max(maxlen, l);
            }
          }
        }
        uint64_t acc = 0;
        for (uint32_t l = 1; seg_ok && l <= kMaxLenFast; ++l) {
          acc += lim[l] << (32 - l);
          lim[l] = acc;
        }
        if (acc > (1ull << 32) || !maxlen) seg_ok = false;
      }
      if (seg_ok) {
        const uint8_t* bits = seg + 272 + cnt;
        const uint8_t* bend = bits + (nb + 7) / 8;
        uint64_t p = 0, segstart = 0, cb = 0, cur = load_be64(bits, bend);
        bool walk = true;
        for (uint64_t n = 0; walk && n < count; ++n) {
          if (n % kIdxLaneSyms == 0) {
            const uint64_t sgi = n / kIdxSegSyms, ln = (n / kIdxLaneSyms) % 64;
            if (ln == 0) {
              if (n) {
                if (p - segstart > kIdxMaxSpan) walk = false;
                out[(sgi - 1) * 64] = (uint16_t)(p - segstart);
              }
              segstart = p;
            } else {
              out[sgi * 64 + ln] = (uint16_t)(p - segstart);
            }
          }
          if (p + 32 > 8 * cb + 64) {
            cb = p >> 3;
            cur = load_be64(bits + cb, bend);
          }
          const uint64_t w = (cur << (p - 8 * cb)) >> 32;
          uint32_t l = minlen;
          while (l <= maxlen && w >= lim[l]) ++l;
          if (l > maxlen) walk = false;
          p += l;
          if (p > nb) walk = false;
        }
        if (walk && p == nb && p - segstart <= kIdxMaxSpan) {
          out[((count - 1) / kIdxSegSyms) * 64] = (uint16_t)(p - segstart);
          ok = true;
        }
      }
    }
    if (!ok && segs) out[0] = kIdxNone;
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
          const float wv = __uint_as_float((uint32_t)h << 16);
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j)
            if (j0 + j < nb) a[j] = fmaf(wv, x[c * ldx + j0 + j], a[j]);
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

// The same over bf16 activations in the layout of x @ W.T:
// Y[j * ldy + dst + r] = sum_c W[r, c] X[j * ldx + c].
__global__ void __launch_bounds__(64) k_gemm_plain_bf16(const DevBlock* __restrict__ blocks, uint32_t nblocks,
                                                        const uint8_t* __restrict__ base,
                                                        const uint16_t* __restrict__ x, uint64_t ldx, uint32_t nb,
                                                        float* __restrict__ y, uint64_t ldy) {
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
          const float wv = __uint_as_float((uint32_t)h << 16);
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j)
            if (j0 + j < nb) a[j] = fmaf(wv, __uint_as_float((uint32_t)x[(j0 + j) * ldx + c] << 16), a[j]);
        }
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
#pragma unroll
          for (uint32_t dd = kWave / 2; dd >= 1; dd >>= 1) a[j] += __shfl_xor(a[j], dd, kWave);
          if (lane == 0 && j0 + j < nb) y[(j0 + j) * ldy + d.dst + r] = a[j];
        }
      }
    }
  }
}

// Routing of XKSP2 blocks for the fused GEMM, from each block's header:
// bit 0 = every substream starts and ends on an 8-element boundary (the fused
// VALU consumers apply), bit 1 = on 256-element boundaries (whole 16x16 tiles:
// the MFMA consumer applies).  A header that does not parse, or disagrees with
// the descriptor, gets both bits: the fused kernels then report its error.
__global__ void __launch_bounds__(256) k_route_parallel(const DevBlock* __restrict__ blocks, uint32_t n,
                                                        const uint8_t* __restrict__ arc, uint32_t* __restrict__ flags) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const DevBlock d = blocks[i];
    uint32_t f = 3;
    if (d.size >= 32) {
      const uint8_t* p = arc + d.src;
      const uint64_t magic = ldg64(p), rows = ldg64(p + 8), cols = ldg64(p + 16), chunks = ldg64(p + 24);
      if (magic == kMagicXKSP2 && rows == d.rows && cols == d.cols && rows && rows <= 16 && cols &&
          cols <= kMaxBlockElems / rows && chunks && chunks <= kMaxChunks && chunks <= rows * cols) {
        const uint64_t total = rows * cols;
        for (uint64_t k = 1; k <= chunks; ++k) {
          const uint64_t b = total * k / chunks;
          if (b % 8) f &= ~1u;
          if (b % 256) f &= ~2u;
        }
        if (!(f & 1u)) f = 0;
      }
    }
    flags[i] = f;
  }
}

// OR of n status words into *flags (a sticky device word the caller owns).
__global__ void __launch_bounds__(256) k_or_status(const uint32_t* __restrict__ status, uint32_t n,
                                                   uint32_t* __restrict__ flags) {
  uint32_t v = 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) v |= status[i];
  if (v) atomicOr(flags, v);
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

// Workgroups of `kernel` resident at once on one CU; times the CU count this
// is the persistent grid (a larger grid would run a second, partly idle round).
template <class K>
static unsigned groups_per_cu(K kernel, unsigned threads) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, (int)threads, 0) != hipSuccess || per_cu < 1)
    per_cu = 1;
  return (unsigned)per_cu;
}

hipError_t launch_decode(const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc, uint8_t* out,
                         uint32_t* status, uint32_t* queue, unsigned cus, hipStream_t s, const uint16_t* index,
                         const uint64_t* ibase) {
  if (!nblocks) return hipSuccess;
  const dim3 blk(64);
  if (codec == kCodecParallel) {
    static const unsigned per_cu = groups_per_cu(k_decode_parallel<false>, 64);
    if ((uint64_t)nblocks < 2ull * per_cu * cus) {  // few blocks: by substream (k_decode_items)
      static const unsigned per_cu_i = groups_per_cu(k_decode_items<false>, 64);
      const dim3 grid(grid_for((uint64_t)nblocks * kMaxChunks, per_cu_i * cus));
      if (index)
        hipLaunchKernelGGL(k_decode_items<true>, grid, blk, 0, s, blocks, nblocks, arc, out, status, index, ibase);
      else
        hipLaunchKernelGGL(k_decode_items<false>, grid, blk, 0, s, blocks, nblocks, arc, out, status, index, ibase);
      return hipGetLastError();
    }
    // The last grid's worth of blocks is claimed by quarters (k_decode_parallel).
    const uint32_t g = grid_for(nblocks, per_cu * cus);
    const uint32_t split = nblocks > g ? nblocks - g : 0u;
    if (index)
      hipLaunchKernelGGL(k_decode_parallel<true>, dim3(g), blk, 0, s, blocks, nblocks, arc, out, status, queue, index,
                         ibase, split);
    else
      hipLaunchKernelGGL(k_decode_parallel<false>, dim3(g), blk, 0, s, blocks, nblocks, arc, out, status, queue, index,
                         ibase, split);
  } else {
    static const unsigned per_cu = groups_per_cu(k_decode_serial, 64);
    hipLaunchKernelGGL(k_decode_serial, dim3(grid_for(nblocks, per_cu * cus)), blk, 0, s, blocks, nblocks, arc, out,
                       status, queue);
  }
  return hipGetLastError();
}

uint64_t serial_wg_scratch(uint32_t nblocks, uint64_t max_elems, unsigned cus, uint32_t* grid, uint32_t* cap) {
  static const unsigned per_cu = groups_per_cu(k_decode_serial_wg, 64 * kSerialWaves);
  *grid = grid_for(nblocks, per_cu * cus);
  // A range holds about max_elems / kSerialWaves symbols; twice that, plus
  // room for a consume call's last 16-byte store, before it overflows (then
  // the block is decoded by one wave).
  const uint64_t c = (2 * ((max_elems + kSerialWaves - 1) / kSerialWaves) + 1024 + 255) & ~255ull;
  *cap = (uint32_t)c;
  return (uint64_t)*grid * kSerialWaves * c;
}

hipError_t launch_decode_serial_wg(const DevBlock* blocks, uint32_t nblocks, const uint8_t* arc, uint8_t* out,
                                   uint32_t* status, uint8_t* scratch, uint32_t cap, uint32_t grid, hipStream_t s) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(k_decode_serial_wg, dim3(grid), dim3(64 * kSerialWaves), 0, s, blocks, nblocks, arc, out, status,
                     scratch, cap);
  return hipGetLastError();
}

template <int W, class Acc>
static void gemm_launch(hipStream_t s, const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc,
                        const GemmArgs& ga, uint32_t* status, unsigned cus) {
  static const unsigned per_cu = groups_per_cu(k_gemm<W, Acc>, 64 * W);
  hipLaunchKernelGGL((k_gemm<W, Acc>), dim3(grid_for(nblocks, per_cu * cus)), dim3(64 * W), 0, s, blocks, nblocks,
                     codec, arc, ga, status);
}

// Item-scheduled launch (XKSP2 blocks with item scratch): the item kernel
// over all resident waves, then the in-order reduction.
template <class Acc>
static void items_launch(hipStream_t s, const DevBlock* blocks, uint32_t nblocks, const uint8_t* arc,
                         const GemmArgs& ga, uint32_t* status, const ItemScratch& is, unsigned cus) {
  static const unsigned per_cu = groups_per_cu(k_gemm_items<Acc>, 64);
  hipLaunchKernelGGL((k_gemm_items<Acc>), dim3(grid_for((uint64_t)nblocks * kMaxChunks, per_cu * cus)), dim3(64),
                     0, s, blocks, nblocks, arc, ga, is);
  hipLaunchKernelGGL((k_gemm_finish<Acc>), dim3(grid_for(nblocks, 8 * cus)), dim3(64), 0, s, blocks, nblocks, ga,
                     status, is);
}

// XKSP2 blocks: by substream when item scratch is given, else one workgroup
// of 4 waves per block (substreams split over the waves).  Serial blocks: one
// wave per block.
template <class Acc>
static void gemm_any(hipStream_t s, const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc,
                     const GemmArgs& ga, uint32_t* status, const ItemScratch* is, unsigned cus) {
  if (codec == kCodecParallel && is) items_launch<Acc>(s, blocks, nblocks, arc, ga, status, *is, cus);
  else if (codec == kCodecParallel) gemm_launch<4, Acc>(s, blocks, nblocks, codec, arc, ga, status, cus);
  else gemm_launch<1, Acc>(s, blocks, nblocks, codec, arc, ga, status, cus);
}

template <template <int> class Acc>
static void gemm_valu(hipStream_t s, const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc,
                      const GemmArgs& ga, uint32_t* status, const ItemScratch* is, unsigned cus) {
  if (ga.nb == 1) gemm_any<Acc<1>>(s, blocks, nblocks, codec, arc, ga, status, is, cus);
  else if (ga.nb <= 4) gemm_any<Acc<4>>(s, blocks, nblocks, codec, arc, ga, status, is, cus);
  else if (ga.nb <= 8) gemm_any<Acc<8>>(s, blocks, nblocks, codec, arc, ga, status, is, cus);
  else gemm_any<Acc<16>>(s, blocks, nblocks, codec, arc, ga, status, is, cus);
}

hipError_t launch_gemm_f32(const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc,
                           const float* x, uint64_t ldx, uint32_t nb, float* y, uint64_t ldy, uint32_t* status,
                           const ItemScratch* is, unsigned cus, hipStream_t s) {
  if (!nblocks) return hipSuccess;
  const GemmArgs ga{x, ldx, nb, y, ldy};
  // GemmF32<1> reads x as a contiguous vector; a one-column group of a wider
  // X (the last group of a batch of 16 k + 1) takes the strided consumer.
  if (nb == 1 && ldx != 1) gemm_any<GemmF32<4>>(s, blocks, nblocks, codec, arc, ga, status, is, cus);
  else gemm_valu<GemmF32>(s, blocks, nblocks, codec, arc, ga, status, is, cus);
  return hipGetLastError();
}

hipError_t launch_gemm_bf16(const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc,
                            const uint16_t* x, uint64_t ldx, uint32_t nb, float* y, uint64_t ldy, bool mfma,
                            uint32_t* status, const ItemScratch* is, unsigned cus, hipStream_t s) {
  if (!nblocks) return hipSuccess;
  const GemmArgs ga{x, ldx, nb, y, ldy};
  // MFMA at every batch (batch 1 padded: 2-3 % faster than the VALU consumer at the 70B shapes)
  if (mfma) gemm_any<GemmMfma>(s, blocks, nblocks, codec, arc, ga, status, is, cus);
  else gemm_valu<GemmBf16>(s, blocks, nblocks, codec, arc, ga, status, is, cus);
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

hipError_t launch_gemm_plain_bf16(const DevBlock* blocks, uint32_t nblocks, const uint8_t* base, const uint16_t* x,
                                  uint64_t ldx, uint32_t nb, float* y, uint64_t ldy, hipStream_t s) {
  if (!nblocks) return hipSuccess;
  hipLaunchKernelGGL(k_gemm_plain_bf16, dim3(256, nblocks < 256 ? nblocks : 256), dim3(64), 0, s, blocks, nblocks,
                     base, x, ldx, nb, y, ldy);
  return hipGetLastError();
}

hipError_t launch_route_parallel(const DevBlock* blocks, uint32_t n, const uint8_t* arc, uint32_t* flags,
                                 hipStream_t s) {
  if (!n) return hipSuccess;
  const unsigned g = (n + 255) / 256;
  hipLaunchKernelGGL(k_route_parallel, dim3(g < 1024 ? g : 1024u), dim3(256), 0, s, blocks, n, arc, flags);
  return hipGetLastError();
}

hipError_t launch_or_status(const uint32_t* status, uint32_t n, uint32_t* flags, hipStream_t s) {
  if (!n) return hipSuccess;
  const unsigned g = (n + 255) / 256;
  hipLaunchKernelGGL(k_or_status, dim3(g < 64 ? g : 64u), dim3(256), 0, s, status, n, flags);
  return hipGetLastError();
}

hipError_t launch_index_items(const DevBlock* blocks, uint32_t nblocks, const uint8_t* arc, uint16_t* index,
                              uint32_t segs, hipStream_t s, const uint64_t* ibase) {
  if (!nblocks) return hipSuccess;
  const uint64_t items = (uint64_t)nblocks * kMaxChunks;
  const uint64_t g = (items + 63) / 64;
  hipLaunchKernelGGL(k_index_items, dim3(g < 4096 ? (unsigned)g : 4096u), dim3(64), 0, s, blocks, nblocks, arc, index,
                     segs, ibase);
  return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t* p, uint64_t n, uint32_t v, hipStream_t s) {
  if (!n) return hipSuccess;
  const uint64_t g = (n + 255) / 256;
  hipLaunchKernelGGL(k_fill_u32, dim3(g < 1024 ? (unsigned)g : 1024u), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

}  // namespace xksv
