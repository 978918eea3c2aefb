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

// Kernel launchers (xksv_kernels.hip).  `cus` = the device's CU count; each
// launcher sizes its persistent grid to the workgroups resident at once.
// `queue` (optional) is a zeroed counter the decode waves claim blocks from.
hipError_t launch_decode(const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc, uint8_t* out,
                         uint32_t* status, uint32_t* queue, unsigned cus, hipStream_t s);
hipError_t launch_gemm_f32(const DevBlock* blocks, uint32_t nblocks, uint32_t codec, const uint8_t* arc,
                           const float* x, uint64_t ldx, uint32_t nb, float* y, uint64_t ldy, uint32_t* status,
                           const ItemScratch* is, unsigned cus, hipStream_t s);
// bf16 X [batch rows of ldx], Y [batch rows of ldy]; bf16 MFMA when `mfma`
// (every substream covers whole 16x16 tiles) and nb >= 8, VALU otherwise.
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
// flags[i] for XKSP2 block i: bit 0 = substreams on 8-element boundaries
// (fused consumers apply), bit 1 = on whole tiles (MFMA applies); both bits
// for a header that does not parse (the fused kernels report it).
hipError_t launch_route_parallel(const DevBlock* blocks, uint32_t n, const uint8_t* arc, uint32_t* flags,
                                 hipStream_t s);
// SHA-256 of each block's decoded bytes out[dst, dst + raw bytes) into
// digests[32 * status_slot] (xksv_sha256.hip).
hipError_t launch_sha256_blocks(const DevBlock* blocks, uint32_t nblocks, const uint8_t* out, uint8_t* digests,
                                hipStream_t s);

}  // namespace xksv
