// Internal declarations shared by the host translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "../../include/xksv_hip.h"
#include "xksv_shared.hpp"

namespace xksv {

struct SlabSpec {
  uint64_t offset, length, rows, cols;  // rows == 0: raw slab
};

bool encode_serial(const uint8_t* data, uint64_t rows, uint64_t cols, std::vector<uint8_t>& v);
bool encode_parallel(const uint8_t* data, uint64_t rows, uint64_t cols, std::vector<uint8_t>& v);
std::vector<SlabSpec> slab_rule(uint64_t nbytes, bool bf16, uint64_t shape_cols);

// What a block-level call computes.  kDecode: BF16 into `out` (device).
// kGemmF32: fused GEMM with fp32 X [cols, batch] into Y [rows, batch].
// kGemmBf16: fused GEMM with bf16 X [batch, cols] into fp32 Y [batch, rows]
// (bf16 MFMA when every substream covers whole tiles).
enum Mode { kDecode, kGemmF32, kGemmBf16 };
struct Fused {
  bool unit = false;  // every stream unit-aligned: fused consumers apply
  bool tile = false;  // every stream covers whole 16x16 tiles: MFMA applies
};
// Shape fields of an XKSP2 block with the reference's header checks
// (cuda/parallel.cu:132-134); false when they fail.
struct ParallelHeader {
  uint64_t rows, cols, chunks;
};
bool parallel_header(const uint8_t* p, uint64_t n, ParallelHeader& h);
// Which fused consumers apply to an XKSP2 block of this header.
Fused fused_parallel(const ParallelHeader& h);
// Device staging of one block-level call, byte offsets from its base:
// [2 descriptors][status words][encoded block][scratch: item partial sums of
// a fused XKSP2 GEMM, or the decoded slab of a GEMM that is not unit-aligned].
struct BlockLayout {
  uint64_t desc, status, block, scratch, total;
};
BlockLayout block_layout(uint64_t size, uint32_t codec, uint64_t rows, uint64_t cols, Fused fused, Mode mode);
// One block-level call staged at device memory `base` (layout L): copies the
// host block in, launches on the null stream, synchronises, reads the status.
// 0 on success, 1 on any validation, bitstream or HIP error.
int run_block_at(uint8_t* base, const BlockLayout& L, const uint8_t* input, uint64_t size, uint32_t codec,
                 uint64_t rows, uint64_t cols, Fused fused, Mode mode, void* out, const void* x, uint64_t batch,
                 unsigned cus);

// Kernel launchers (xksv_kernels.hip).  `cus` = the device's CU count; each
// launcher sizes its persistent grid to the workgroups resident at once.
// `queue` (optional) is a zeroed counter the decode waves claim blocks from.
// `index`, `ibase` (optional, XKSP2): a codeword index of `blocks` laid out by
// launch_index_items with `ibase`; the decode checks it as it uses it.
hipError_t launch_decode(const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc, uint8_t* out,
                         uint32_t* status, uint32_t* queue, unsigned cus, hipStream_t s,
                         const uint16_t* index = nullptr, const uint64_t* ibase = nullptr);
// Serial blocks decoded by a workgroup each (k_decode_serial_wg): scratch
// bytes for `nblocks` blocks of at most `max_elems` elements; sets the grid
// and the per-wave region size the launch takes.
uint64_t serial_wg_scratch(uint32_t nblocks, uint64_t max_elems, unsigned cus, uint32_t* grid, uint32_t* cap);
hipError_t launch_decode_serial_wg(const DevBlock* blocks, uint32_t nblocks, const uint8_t* arc, uint8_t* out,
                                   uint32_t* status, uint8_t* scratch, uint32_t cap, uint32_t grid, hipStream_t s);
hipError_t launch_gemm_f32(const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc,
                           const float* x, uint64_t ldx, uint32_t nb, float* y, uint64_t ldy, uint32_t* status,
                           const ItemScratch* is, unsigned cus, hipStream_t s);
// bf16 X [batch rows of ldx], Y [batch rows of ldy]; bf16 MFMA when `mfma`
// (every substream covers whole 16x16 tiles), VALU otherwise.
// With `is` (scratch of kItemScratchPerBlock bytes per block, see
// ItemScratch), XKSP2 blocks run by substream over every resident wave.
hipError_t launch_gemm_bf16(const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc,
                            const uint16_t* x, uint64_t ldx, uint32_t nb, float* y, uint64_t ldy, bool mfma,
                            uint32_t* status, const ItemScratch* is, unsigned cus, hipStream_t s);
hipError_t launch_copy_raw(const DevBlock* blocks, uint32_t nblocks, const uint8_t* arc, uint8_t* out, hipStream_t s);
hipError_t launch_gemm_plain(const DevBlock* blocks, uint32_t nblocks, const uint8_t* base, const float* x,
                             uint64_t ldx, uint32_t nb, float* y, uint64_t ldy, hipStream_t s);
hipError_t launch_gemm_plain_bf16(const DevBlock* blocks, uint32_t nblocks, const uint8_t* base, const uint16_t* x,
                                  uint64_t ldx, uint32_t nb, float* y, uint64_t ldy, hipStream_t s);
hipError_t launch_fill_u32(uint32_t* p, uint64_t n, uint32_t v, hipStream_t s);
// Codeword index (ItemScratch::index) of the fused XKSP2 items of `blocks`:
// `segs` segments of 64 u16 entries per item; with `ibase` (nblocks + 1
// entry offsets), block b's items take (ibase[b + 1] - ibase[b]) / 2048
// entries each from ibase[b] on instead.
hipError_t launch_index_items(const DevBlock* blocks, uint32_t nblocks, const uint8_t* arc, uint16_t* index,
                              uint32_t segs, hipStream_t s, const uint64_t* ibase = nullptr);
// *flags |= OR of status[0 .. n) (vector atomic), enqueued on s.
hipError_t launch_or_status(const uint32_t* status, uint32_t n, uint32_t* flags, hipStream_t s);
// flags[i] for XKSP2 block i: bit 0 = substreams on 8-element boundaries
// (fused consumers apply), bit 1 = on whole tiles (MFMA applies); both bits
// for a header that does not parse (the fused kernels report it).
hipError_t launch_route_parallel(const DevBlock* blocks, uint32_t n, const uint8_t* arc, uint32_t* flags,
                                 hipStream_t s);
// SHA-256 of blocks' decoded bytes (xksv_sha256.hip): lane l hashes
// items[first[l] .. first[l + 1]) one after another, item i's bytes
// out[dst, dst + n) into digests[32 * slot].
hipError_t launch_sha256_lanes(const HashItem* items, const uint32_t* first, uint32_t nlanes, const uint8_t* out,
                               uint8_t* digests, hipStream_t s);
// verdicts[i] = status[i] | kErrDigest when digests[32 i ..] != expected[32 i ..].
hipError_t launch_digest_verdicts(const uint8_t* digests, const uint8_t* expected, const uint32_t* status, uint32_t n,
                                  uint32_t* verdicts, hipStream_t s);

}  // namespace xksv
