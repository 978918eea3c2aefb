// Types shared by the host API (xksv_api.cpp) and the gfx950 kernels
// (xksv_kernels.hip).  Plain structs only: no torch types, no STL.
#pragma once
#include <stdint.h>

namespace xksv {

// Block codecs, as named in the archive index (src/compile.cpp:266-268).
enum Codec : uint32_t {
  kCodecRaw = 0,       // "raw": original bytes
  kCodecSerial = 1,    // "bf16-huffman-tile16": one Huffman stream per slab
  kCodecParallel = 2,  // "bf16-huffman-parallel32": XKSP2 block, <= 32 substreams
};

// Per-block error bits written to the status array (0 = block decoded).
enum Err : uint32_t {
  kErrHeader = 1,    // block or substream header fails the reference's validation
  kErrCodebook = 2,  // oversubscribed canonical code lengths
  kErrStream = 4,    // invalid code, truncated stream, trailing bits, or count mismatch
  kErrShape = 8,     // header shape disagrees with the descriptor, or exceeds device limits
  kErrDigest = 16,   // decoded bytes' SHA-256 differs from the index digest (verification)
};

// One encoded block as the kernels see it (device memory).  `src` and `size`
// locate the encoded bytes inside the archive buffer; `dst` is the output byte
// offset (decode) or the first output row (GEMV/GEMM).  `rows`/`cols` are the
// index's slab shape (src/compile.cpp:461-468).
struct DevBlock {
  uint64_t src;
  uint64_t size;
  uint64_t dst;
  uint64_t rows;
  uint64_t cols;
  uint32_t codec;
  uint32_t status_slot;  // index into the status array
};

// One block to hash: its decoded bytes out[dst, dst + n), digest slot.
struct HashItem {
  uint64_t dst;
  uint64_t n;
  uint32_t slot;
  uint32_t reserved;
};

// Device element limit per block: element indices are 32-bit in the kernels.
constexpr uint64_t kMaxBlockElems = (1ull << 31) - 1;
// Most substreams an XKSP2 block may hold (src/c_api.cpp:66-72).
constexpr uint32_t kMaxChunks = 32;
// Largest batch one fused GEMM launch handles in registers; larger batches
// are split into column groups by the host.
constexpr uint32_t kMaxFusedBatch = 16;
// Fused GEMM over XKSP2 blocks by substream ("items"): per block, kMaxChunks
// records (kMaxItemOut partial sums and an error word each) and the block's
// substream count (written by the item kernel; 0 = header error).
constexpr uint32_t kMaxItemOut = 16 * kMaxFusedBatch;
// Codeword index of the fused XKSP2 items (a load-time sidecar of static
// weights): per item, `index_segs` segments of kIdxSegSyms symbols, each 64
// u16 entries: entry 0 = the segment's length in code bits, entry l (l >= 1)
// = the bit offset of symbol kIdxLaneSyms * l from the segment's start.
// Entry 0 of segment 0 holds kIdxNone when the item has no index (its stream
// does not fit the indexed path); the kernels then decode it speculatively.
constexpr uint32_t kIdxLaneSyms = 32;
constexpr uint32_t kIdxSegSyms = 64 * kIdxLaneSyms;
constexpr uint16_t kIdxNone = 0xFFFF;
struct ItemScratch {
  float* partial;         // [blocks][kMaxChunks][kMaxItemOut]
  uint32_t* err;          // [blocks][kMaxChunks]
  uint32_t* done;         // [blocks]
  const uint16_t* index;  // [items][index_segs][64], or nullptr
  uint32_t index_segs;
};
constexpr uint64_t kItemScratchPerBlock = (uint64_t)kMaxChunks * kMaxItemOut * 4 + kMaxChunks * 4 + 4;
// ItemScratch over `base` for `nblocks` blocks (kItemScratchPerBlock bytes each).
inline ItemScratch item_scratch(uint8_t* base, uint64_t nblocks) {
  ItemScratch is{};
  is.partial = reinterpret_cast<float*>(base);
  is.err = reinterpret_cast<uint32_t*>(base + nblocks * kMaxChunks * kMaxItemOut * 4);
  is.done = reinterpret_cast<uint32_t*>(base + nblocks * (kMaxChunks * kMaxItemOut * 4 + kMaxChunks * 4));
  return is;
}

}  // namespace xksv
