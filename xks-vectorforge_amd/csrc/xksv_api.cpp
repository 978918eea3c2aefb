// xksv_api.cpp -- C ABI of libxksv_hip.so (host side).
//
// Drop-in entry points (reference signatures, synchronous, host block in):
//   xksv_hip_decode / _gemv / _gemm          cuda/decode.cu:47-98
//   xksv_hip_decode_parallel / _gemv_parallel cuda/parallel.cu:33-74
//   xksv_unpack / xksv_unpack_parallel        src/c_api.cpp:29-40, 66-85 (decoded on the GPU)
// and the device-resident plan API used for throughput (one launch per codec
// over a whole archive or weight tensor, archive resident in HBM).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "xksv_api_internal.hpp"

using namespace xksv;

namespace {

constexpr int kMaxDevices = 64;
constexpr uint64_t kAlign = 256;
// Largest substream partial-sum scratch a plan allocates (32 KiB per fused
// XKSP2 block: 32,768 blocks, a 4 GiB BF16 weight set).
constexpr uint64_t kMaxItemMem = 1ull << 30;
constexpr uint64_t kQueues = 4;  // block-queue counters per plan (one per decode launch of a step)

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }
uint64_t get64(const uint8_t* p) {
  uint64_t v = 0;
  for (int i = 0; i < 8; ++i) v |= (uint64_t)p[i] << (8 * i);
  return v;
}

struct DeviceInfo {
  bool init = false, ok = false;
  int cus = 0;
};
std::mutex g_dev_mu;
DeviceInfo g_dev[kMaxDevices];

// Current device and its CU count; nullptr without a device.
const DeviceInfo* current_device(int* id_out) {
  int id = -1;
  if (hipGetDevice(&id) != hipSuccess || id < 0 || id >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lk(g_dev_mu);
  DeviceInfo& d = g_dev[id];
  if (!d.init) {
    d.init = true;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, id) == hipSuccess && cus > 0) {
      d.cus = cus;
      d.ok = true;
    }
  }
  if (id_out) *id_out = id;
  return d.ok ? &d : nullptr;
}

// Device staging buffers for the synchronous host-pointer entry points,
// pooled per device (grow-only, reused across calls and threads).
struct Buf {
  uint8_t* p = nullptr;
  uint64_t cap = 0;
};
std::mutex g_pool_mu;
std::vector<Buf> g_pool[kMaxDevices];

bool acquire(int dev, uint64_t bytes, Buf& b) {
  {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    auto& v = g_pool[dev];
    for (size_t i = 0; i < v.size(); ++i)
      if (v[i].cap >= bytes) {
        b = v[i];
        v.erase(v.begin() + i);
        return true;
      }
    if (!v.empty()) {  // grow the largest free buffer
      b = v.back();
      v.pop_back();
      (void)hipFree(b.p);
      b = Buf{};
    }
  }
  const uint64_t cap = std::max<uint64_t>(align_up(bytes, 1 << 20), 4 << 20);
  if (hipMalloc(reinterpret_cast<void**>(&b.p), cap) != hipSuccess) return false;
  b.cap = cap;
  return true;
}
void release(int dev, Buf b) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  g_pool[dev].push_back(b);
}

// One block through the GPU, staged in a pooled device buffer.
int run_block(const uint8_t* input, uint64_t size, uint32_t codec, uint64_t rows, uint64_t cols, Fused fused,
              Mode mode, void* out, const void* x, uint64_t batch) {
  int dev = -1;
  const DeviceInfo* di = current_device(&dev);
  if (!di) return 1;
  const BlockLayout L = block_layout(size, codec, rows, cols, fused, mode);
  Buf b;
  if (!acquire(dev, L.total, b)) return 1;
  const int rc = run_block_at(b.p, L, input, size, codec, rows, cols, fused, mode, out, x, batch, (unsigned)di->cus);
  release(dev, b);
  return rc;
}

Fused fused_serial(uint64_t rows, uint64_t cols) {
  Fused f;
  f.unit = f.tile = rows == 16 && cols % 16 == 0;
  return f;
}

// Oversubscription of a lengths table, as the reference's canonical()
// detects it (src/codec.cpp:20-22): some length has more codes than free slots.
bool oversubscribed(const uint8_t* lens) {
  uint32_t cnt[256] = {};
  for (int s = 0; s < 256; ++s) ++cnt[lens[s]];
  uint64_t free = 2;
  for (int l = 1; l < 256; ++l) {
    if (cnt[l] > free) return true;
    free = std::min<uint64_t>(2 * (free - cnt[l]), 1024);
  }
  return false;
}

int to_host(const void* dev_src, uint64_t bytes, void** out, size_t* out_size) {
  void* h = malloc(bytes ? bytes : 1);
  if (!h) return -1;
  if (bytes && hipMemcpy(h, dev_src, bytes, hipMemcpyDeviceToHost) != hipSuccess) {
    free(h);
    return -1;
  }
  *out = h;
  *out_size = bytes;
  return 0;
}

// Decode on the GPU into a temporary device buffer, then copy to the host.
int unpack_via_gpu(const uint8_t* p, uint64_t n, uint32_t codec, uint64_t rows, uint64_t cols, void** out,
                   size_t* out_size) {
  int dev = -1;
  if (!current_device(&dev)) return -1;
  const uint64_t bytes = rows * cols * 2;
  Buf b;
  if (!acquire(dev, align_up(bytes, kAlign) + 64, b)) return -1;
  int rc = run_block(p, n, codec, rows, cols, Fused{}, kDecode, b.p, nullptr, 0) ? -1 : to_host(b.p, bytes, out, out_size);
  release(dev, b);
  return rc;
}

}  // namespace

// ------------------------------------------------------------ plan object

namespace xksv {

// Shape fields of an XKSP2 block, with the reference's header checks
// (cuda/parallel.cu:132-134); the kernel repeats them and validates the rest.
bool parallel_header(const uint8_t* p, uint64_t n, ParallelHeader& h) {
  if (!p || n < 32 || memcmp(p, "XKSP2\0\0\0", 8)) return false;
  h.rows = get64(p + 8);
  h.cols = get64(p + 16);
  h.chunks = get64(p + 24);
  if (!h.rows || h.rows > 16 || !h.cols || !h.chunks || h.chunks > 32 || h.cols > UINT64_MAX / h.rows ||
      h.chunks > h.rows * h.cols || h.rows * h.cols > n || h.rows * h.cols > UINT64_MAX / 32 || n < 32 + 8 * h.chunks)
    return false;
  return h.rows * h.cols <= kMaxBlockElems;
}

// Fused kernels need 16-row slabs of whole tiles whose streams start and end
// on 8-element boundaries; the MFMA consumer needs them on tile boundaries.
Fused fused_parallel(const ParallelHeader& h) {
  Fused f;
  if (h.rows != 16 || h.cols % 16) return f;
  const uint64_t total = h.rows * h.cols;
  f.unit = f.tile = true;
  for (uint64_t k = 0; k <= h.chunks; ++k) {
    const uint64_t b = total * k / h.chunks;
    f.unit = f.unit && b % 8 == 0;
    f.tile = f.tile && b % 256 == 0;
  }
  f.tile = f.tile && f.unit;
  return f;
}
BlockLayout block_layout(uint64_t size, uint32_t codec, uint64_t rows, uint64_t cols, Fused fused, Mode mode) {
  const uint64_t n = rows * cols;
  const bool generic_gemm = mode != kDecode && !fused.unit;
  const bool items = mode != kDecode && !generic_gemm && codec == kCodecParallel;
  uint32_t grid = 0, cap = 0;
  const uint64_t serial = mode == kDecode && codec == kCodecSerial ? serial_wg_scratch(1, n, 1, &grid, &cap) : 0;
  const uint64_t scratch_size = generic_gemm ? n * 2 : items ? kItemScratchPerBlock : serial;
  BlockLayout L;
  L.desc = 0;
  L.status = align_up(L.desc + 2 * sizeof(DevBlock), kAlign);
  L.block = L.status + kAlign;
  L.scratch = align_up(L.block + size + 16, kAlign);
  L.total = L.scratch + align_up(scratch_size, kAlign);
  return L;
}

int run_block_at(uint8_t* base, const BlockLayout& L, const uint8_t* input, uint64_t size, uint32_t codec,
                 uint64_t rows, uint64_t cols, Fused fused, Mode mode, void* out, const void* x, uint64_t batch,
                 unsigned cus) {
  const bool generic_gemm = mode != kDecode && !fused.unit;
  // Fused GEMM over an XKSP2 block runs by substream (item scratch).
  const bool items = mode != kDecode && !generic_gemm && codec == kCodecParallel;
  DevBlock d[2];
  d[0] = DevBlock{L.block, size, 0, rows, cols, codec, 0};
  d[1] = DevBlock{L.scratch, 0, 0, rows, cols, kCodecRaw, 0};
  if (hipMemcpy(base + L.desc, d, sizeof d, hipMemcpyHostToDevice) != hipSuccess) return 1;
  if (hipMemcpy(base + L.block, input, size, hipMemcpyHostToDevice) != hipSuccess) return 1;
  uint32_t* status = reinterpret_cast<uint32_t*>(base + L.status);
  if (launch_fill_u32(status, kAlign / 4, 0, nullptr) != hipSuccess) return 1;
  const DevBlock* dd = reinterpret_cast<const DevBlock*>(base + L.desc);
  const ItemScratch is = item_scratch(base + L.scratch, 1);
  float* y = static_cast<float*>(out);
  if (mode == kDecode && codec == kCodecSerial) {  // one workgroup for the block
    uint32_t grid = 0, cap = 0;
    (void)serial_wg_scratch(1, rows * cols, 1, &grid, &cap);
    if (launch_decode_serial_wg(dd, 1, base, static_cast<uint8_t*>(out), status, base + L.scratch, cap, grid,
                                nullptr) != hipSuccess)
      return 1;
  } else if (mode == kDecode) {
    if (launch_decode(dd, 1, codec, base, static_cast<uint8_t*>(out), status, nullptr, cus, nullptr) != hipSuccess)
      return 1;
  } else if (!generic_gemm) {
    for (uint64_t j0 = 0; j0 < batch; j0 += kMaxFusedBatch) {
      const uint32_t nb = (uint32_t)std::min<uint64_t>(kMaxFusedBatch, batch - j0);
      const hipError_t e =
          mode == kGemmF32
              ? launch_gemm_f32(dd, 1, codec, base, static_cast<const float*>(x) + j0, batch, nb, y + j0, batch,
                                status, items ? &is : nullptr, cus, nullptr)
              : launch_gemm_bf16(dd, 1, codec, base, static_cast<const uint16_t*>(x) + j0 * cols, cols, nb,
                                 y + j0 * rows, rows, fused.tile, status, items ? &is : nullptr, cus, nullptr);
      if (e != hipSuccess) return 1;
    }
  } else {
    // Not unit-aligned: decode to scratch, then a plain deterministic GEMM.
    if (launch_decode(dd, 1, codec, base, base + L.scratch, status, nullptr, cus, nullptr) != hipSuccess) return 1;
    const hipError_t e =
        mode == kGemmF32
            ? launch_gemm_plain(dd + 1, 1, base, static_cast<const float*>(x), batch, (uint32_t)batch, y, batch,
                                nullptr)
            : launch_gemm_plain_bf16(dd + 1, 1, base, static_cast<const uint16_t*>(x), cols, (uint32_t)batch, y,
                                     rows, nullptr);
    if (e != hipSuccess) return 1;
  }
  if (hipStreamSynchronize(nullptr) != hipSuccess) return 1;
  uint32_t st = 1;
  if (hipMemcpy(&st, status, 4, hipMemcpyDeviceToHost) != hipSuccess) return 1;
  return st ? 1 : 0;
}

}  // namespace xksv


struct xksv_hip_plan {
  int device = -1;
  uint64_t archive_size = 0;
  std::vector<xksv_hip_block> blocks;
  // decode lists (status slot = block index)
  DevBlock* d_serial = nullptr;
  DevBlock* d_parallel = nullptr;
  DevBlock* d_raw = nullptr;
  uint32_t n_serial = 0, n_parallel = 0, n_raw = 0;
  uint64_t out_extent = 0;  // bytes the decode writes
  uint32_t* status = nullptr;
  // GEMM routing, built on first use
  bool gemm_ready = false, gemm_valid = false;
  uint64_t cols = 0, rows_extent = 0;
  DevBlock *g_fserial = nullptr, *g_fparallel = nullptr, *g_gser = nullptr, *g_gpar = nullptr, *g_gplain = nullptr,
           *g_raw = nullptr;
  uint32_t n_fserial = 0, n_fparallel = 0, n_gser = 0, n_gpar = 0, n_generic = 0, n_graw = 0;
  bool tile_parallel = false;  // parallel32 slabs split into whole-tile substreams (MFMA consumer)
  uint8_t* scratch = nullptr;
  uint8_t* serial_scratch = nullptr;  // workgroup-scale serial decode (k_decode_serial_wg)
  uint32_t serial_grid = 0, serial_cap = 0;
  uint8_t* item_mem = nullptr;  // ItemScratch of the fused XKSP2 list (none: workgroup-per-block kernels)
  uint8_t* digests = nullptr;   // verification: SHA-256 per block, table order (allocated on first use)
  HashItem* hash_items = nullptr;  // blocks in hashing order, and the first item of each hashing lane
  uint32_t* hash_first = nullptr;
  uint32_t n_hash_lanes = 0;
  uint16_t* index = nullptr;    // codeword index of the fused XKSP2 items (ItemScratch::index)
  uint64_t index_bytes = 0;
  uint16_t* dindex = nullptr;   // decode index of d_parallel (xksv_hip_plan_index), per-block offsets dibase
  uint64_t* dibase = nullptr;
  uint64_t dindex_bytes = 0;
  ItemScratch items{};
  std::vector<uint32_t> h_status;
};

namespace {

template <class T>
bool upload(const std::vector<T>& v, T** dst) {
  *dst = nullptr;
  if (v.empty()) return true;
  if (hipMalloc(reinterpret_cast<void**>(dst), v.size() * sizeof(T)) != hipSuccess) return false;
  return hipMemcpy(*dst, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice) == hipSuccess;
}

// Hashing schedule for the per-block SHA-256.  One lane hashes a block from
// start to end, so a launch lasts at least as long as its largest block
// (a 458 KB slab: 18.1 ms alone), and longer when that lane's wave shares a
// SIMD with other waves.  Blocks go out largest first, so the lanes of a wave
// carry about equal work, and a lane takes further blocks (next fit) while its
// byte total stays within 0.6 of the largest block.  Measured on the Llama-3-8B
// archive (8,192 slabs of 458 KB, 85,840 of 131 KB): one block per lane
// 22.6 ms, two 131 KB slabs per lane 21.4 ms (800 waves), three 30.7 ms (576
// waves, the waves then sharing SIMDs more).
void hash_schedule(const std::vector<xksv_hip_block>& blocks, std::vector<HashItem>& items,
                   std::vector<uint32_t>& first) {
  std::vector<uint32_t> order(blocks.size());
  for (uint32_t i = 0; i < order.size(); ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(),
                   [&](uint32_t a, uint32_t b) { return blocks[a].raw_size > blocks[b].raw_size; });
  const uint64_t cap = order.empty() ? 0 : blocks[order[0]].raw_size / 10 * 6;
  items.clear();
  first.assign(1, 0);
  uint64_t load = 0;
  for (uint32_t i : order) {
    const uint64_t n = blocks[i].raw_size;
    if (!items.empty() && load + n > cap) {
      first.push_back((uint32_t)items.size());
      load = 0;
    }
    items.push_back(HashItem{blocks[i].out_offset, n, i, 0});
    load += n;
  }
  if (!items.empty()) first.push_back((uint32_t)items.size());
}

// GEMM routing: fused kernels for 16-row compressed slabs whose streams start
// and end on 8-element boundaries, decode-to-scratch + plain GEMM for other
// compressed slabs, plain GEMM straight from the archive for raw slabs.  For
// XKSP2 slabs the substream boundaries depend on the block's chunk count, so
// a header pre-pass over the archive of the first GEMM call routes them (one
// synchronisation); later calls take archives with the same block headers
// (copies of one archive), and a block whose header no longer fits the fused
// kernels is reported by them as a shape error.
bool prepare_gemm(xksv_hip_plan* P, const uint8_t* arc, hipStream_t s) {
  if (P->gemm_ready) return P->gemm_valid;
  P->gemm_ready = true;
  uint64_t cols = 0;
  for (const auto& b : P->blocks)
    if (b.codec != XKSV_CODEC_RAW) cols = b.cols;
  if (!cols)  // raw blocks only: the row width comes from their cols field (0 in archive indexes)
    for (const auto& b : P->blocks)
      if (b.cols) cols = b.cols;
  if (!cols) return false;
  // XKSP2 candidates for the fused kernels: their header decides.
  std::vector<DevBlock> cand;
  for (size_t i = 0; i < P->blocks.size(); ++i) {
    const auto& b = P->blocks[i];
    if (b.codec == XKSV_CODEC_PARALLEL && b.cols == cols && b.rows == 16 && cols % 16 == 0)
      cand.push_back(DevBlock{b.offset, b.size, b.out_offset, b.rows, cols, b.codec, (uint32_t)i});
  }
  std::vector<uint32_t> route(P->blocks.size(), 3u);
  if (!cand.empty()) {
    DevBlock* d_cand = nullptr;
    uint32_t* d_flags = nullptr;
    std::vector<uint32_t> flags(cand.size());
    bool ok = upload(cand, &d_cand) &&
              hipMalloc(reinterpret_cast<void**>(&d_flags), cand.size() * 4) == hipSuccess &&
              launch_route_parallel(d_cand, (uint32_t)cand.size(), arc, d_flags, s) == hipSuccess &&
              hipStreamSynchronize(s) == hipSuccess &&
              hipMemcpy(flags.data(), d_flags, cand.size() * 4, hipMemcpyDeviceToHost) == hipSuccess;
    if (d_cand) (void)hipFree(d_cand);
    if (d_flags) (void)hipFree(d_flags);
    if (!ok) return false;
    for (size_t j = 0; j < cand.size(); ++j) route[cand[j].status_slot] = flags[j];
  }
  std::vector<DevBlock> fs, fp, gds, gdp, gp, raw;
  uint64_t scratch = 0, rows_extent = 0;
  bool tile = true;
  for (size_t i = 0; i < P->blocks.size(); ++i) {
    const auto& b = P->blocks[i];
    const uint32_t slot = (uint32_t)i;
    uint64_t rows = b.rows;
    if (b.codec == XKSV_CODEC_RAW) {
      if (b.raw_size % (cols * 2)) return false;
      rows = b.raw_size / (cols * 2);
      raw.push_back(DevBlock{b.offset, b.size, b.out_offset, rows, cols, kCodecRaw, slot});
    } else {
      if (b.cols != cols) return false;
      const bool fused = b.rows == 16 && cols % 16 == 0 && (route[i] & 1u);
      if (fused) {
        if (b.codec == XKSV_CODEC_PARALLEL) tile = tile && (route[i] & 2u);
        (b.codec == XKSV_CODEC_SERIAL ? fs : fp).push_back(DevBlock{b.offset, b.size, b.out_offset, b.rows, cols,
                                                                    b.codec, slot});
      } else {
        (b.codec == XKSV_CODEC_SERIAL ? gds : gdp).push_back(DevBlock{b.offset, b.size, scratch, b.rows, cols, b.codec, slot});
        gp.push_back(DevBlock{scratch, 0, b.out_offset, b.rows, cols, kCodecRaw, slot});
        scratch += align_up(b.raw_size, 16);
      }
    }
    rows_extent = std::max(rows_extent, b.out_offset + rows);
  }
  P->cols = cols;
  P->rows_extent = rows_extent;
  if (!upload(fs, &P->g_fserial) || !upload(fp, &P->g_fparallel) || !upload(gds, &P->g_gser) ||
      !upload(gdp, &P->g_gpar) || !upload(gp, &P->g_gplain) || !upload(raw, &P->g_raw))
    return false;
  P->n_fserial = (uint32_t)fs.size();
  P->n_fparallel = (uint32_t)fp.size();
  P->n_gser = (uint32_t)gds.size();
  P->n_gpar = (uint32_t)gdp.size();
  P->n_generic = (uint32_t)gp.size();
  P->n_graw = (uint32_t)raw.size();
  // The MFMA consumer needs every fused XKSP2 substream to cover whole tiles.
  P->tile_parallel = tile;
  if (scratch && hipMalloc(reinterpret_cast<void**>(&P->scratch), scratch) != hipSuccess) return false;
  // Substream partial sums for the fused XKSP2 list: 32 KiB per block, up to
  // kMaxItemMem; larger lists keep the workgroup-per-block kernels.
  const uint64_t item_bytes = (uint64_t)P->n_fparallel * kItemScratchPerBlock;
  if (P->n_fparallel && item_bytes <= kMaxItemMem) {
    if (hipMalloc(reinterpret_cast<void**>(&P->item_mem), item_bytes) != hipSuccess) return false;
    P->items = item_scratch(P->item_mem, P->n_fparallel);
    // Codeword index of the items (weights are static: built once, here, from
    // the archive of the first GEMM call; the kernels check it as they use it).
    // Sized for the slab rule's 32 substreams of 16 * cols / 32 symbols; an
    // item with more symbols is decoded speculatively.
    const uint64_t syms = (16 * cols + kMaxChunks - 1) / kMaxChunks;
    const uint32_t segs = (uint32_t)std::max<uint64_t>(1, (syms + kIdxSegSyms - 1) / kIdxSegSyms);
    P->index_bytes = (uint64_t)P->n_fparallel * kMaxChunks * segs * 64 * sizeof(uint16_t);
    if (hipMalloc(reinterpret_cast<void**>(&P->index), P->index_bytes) != hipSuccess) return false;
    if (launch_index_items(P->g_fparallel, P->n_fparallel, arc, P->index, segs, s) != hipSuccess) return false;
    P->items.index = P->index;
    P->items.index_segs = segs;
  }
  P->gemm_valid = true;
  return true;
}

}  // namespace

extern "C" {

int xksv_hip_version(void) { return 1; }

int xksv_hip_device_cus(void) {
  const DeviceInfo* d = current_device(nullptr);
  return d ? d->cus : 0;
}

// ----------------------------------------------------- drop-in GPU entries

int xksv_hip_decode(const void* input, size_t size, size_t rows, size_t cols, void* output) {
  const uint8_t* p = static_cast<const uint8_t*>(input);
  if (!p || !output || size < 272 || !rows || !cols || cols > SIZE_MAX / rows) return 1;
  if (rows * cols > kMaxBlockElems) return 1;
  return run_block(p, size, kCodecSerial, rows, cols, Fused{}, kDecode, output, nullptr, 0);
}

int xksv_hip_gemm(const void* input, size_t size, size_t rows, size_t cols, size_t batch, const float* x,
                  float* output) {
  const uint8_t* p = static_cast<const uint8_t*>(input);
  if (!x || !p || !output || size < 272 || !rows || !cols || !batch || cols > SIZE_MAX / rows ||
      batch > SIZE_MAX / rows || batch > SIZE_MAX / cols)
    return 1;
  if (rows * cols > kMaxBlockElems) return 1;
  return run_block(p, size, kCodecSerial, rows, cols, fused_serial(rows, cols), kGemmF32, output, x, batch);
}

int xksv_hip_gemv(const void* input, size_t size, size_t rows, size_t cols, const float* x, float* output) {
  return xksv_hip_gemm(input, size, rows, cols, 1, x, output);
}

int xksv_hip_decode_parallel(const void* input, size_t n, void* output) {
  ParallelHeader h;
  if (!output || !parallel_header(static_cast<const uint8_t*>(input), n, h)) return 1;
  return run_block(static_cast<const uint8_t*>(input), n, kCodecParallel, h.rows, h.cols, Fused{}, kDecode, output,
                   nullptr, 0);
}

int xksv_hip_gemm_parallel(const void* input, size_t n, size_t batch, const float* x, float* output) {
  ParallelHeader h;
  if (!x || !output || !batch || !parallel_header(static_cast<const uint8_t*>(input), n, h)) return 1;
  if (batch > SIZE_MAX / h.rows) return 1;
  return run_block(static_cast<const uint8_t*>(input), n, kCodecParallel, h.rows, h.cols, fused_parallel(h), kGemmF32,
                   output, x, batch);
}

int xksv_hip_gemm_parallel_bf16(const void* input, size_t n, size_t batch, const uint16_t* x, float* output) {
  ParallelHeader h;
  if (!x || !output || !batch || !parallel_header(static_cast<const uint8_t*>(input), n, h)) return 1;
  if (batch > SIZE_MAX / h.rows || batch > SIZE_MAX / h.cols) return 1;
  return run_block(static_cast<const uint8_t*>(input), n, kCodecParallel, h.rows, h.cols, fused_parallel(h),
                   kGemmBf16, output, x, batch);
}

int xksv_hip_gemv_parallel(const void* input, size_t n, const float* x, float* output) {
  return xksv_hip_gemm_parallel(input, n, 1, x, output);
}

int xksv_cuda_decode(const void* input, size_t size, size_t rows, size_t cols, void* output) {
  return xksv_hip_decode(input, size, rows, cols, output);
}
int xksv_cuda_gemv(const void* input, size_t size, size_t rows, size_t cols, const float* x, float* output) {
  return xksv_hip_gemv(input, size, rows, cols, x, output);
}
int xksv_cuda_gemm(const void* input, size_t size, size_t rows, size_t cols, size_t batch, const float* x,
                   float* output) {
  return xksv_hip_gemm(input, size, rows, cols, batch, x, output);
}
int xksv_cuda_decode_parallel(const void* input, size_t n, void* output) {
  return xksv_hip_decode_parallel(input, n, output);
}
int xksv_cuda_gemv_parallel(const void* input, size_t n, const float* x, float* output) {
  return xksv_hip_gemv_parallel(input, n, x, output);
}

// --------------------------------------------- CPU codec surface, GPU decode

int xksv_unpack(const void* data, size_t n, size_t rows, size_t cols, void** out, size_t* out_size) {
  const uint8_t* p = static_cast<const uint8_t*>(data);
  if (!p || !out || !out_size || n < 272 || !rows || cols > SIZE_MAX / rows) return -1;
  const uint64_t count = get64(p), bits = get64(p + 8);
  if (count != rows * cols || count > n - 272 || bits / 8 + (bits % 8 != 0) != n - 272 - count) return -1;
  if (count == 0) {  // zero elements: valid iff the codebook is and no bits remain
    if (oversubscribed(p + 16) || bits) return -1;
    return to_host(nullptr, 0, out, out_size);
  }
  if (count > kMaxBlockElems) return -1;
  return unpack_via_gpu(p, n, kCodecSerial, rows, cols, out, out_size);
}

int xksv_unpack_parallel(const void* data, size_t n, void** out, size_t* out_size) {
  ParallelHeader h;
  if (!out || !out_size || !parallel_header(static_cast<const uint8_t*>(data), n, h)) return -1;
  return unpack_via_gpu(static_cast<const uint8_t*>(data), n, kCodecParallel, h.rows, h.cols, out, out_size);
}

// ----------------------------------------------------------------- plans

int xksv_hip_plan_create(const xksv_hip_block* blocks, size_t nblocks, uint64_t archive_size, xksv_hip_plan** plan) {
  if (!plan || (nblocks && !blocks) || nblocks > 0xffffffffull) return 1;
  *plan = nullptr;
  int dev = -1;
  if (!current_device(&dev)) return 1;
  auto* P = new (std::nothrow) xksv_hip_plan();
  if (!P) return 1;
  P->device = dev;
  P->archive_size = archive_size;
  P->blocks.assign(blocks, blocks + nblocks);
  std::vector<DevBlock> ser, par, raw;
  bool ok = true;
  for (size_t i = 0; i < nblocks && ok; ++i) {
    const xksv_hip_block& b = blocks[i];
    if (b.offset > archive_size || b.size > archive_size - b.offset || b.reserved) ok = false;
    else if (b.codec == XKSV_CODEC_RAW) {
      ok = b.size == b.raw_size;
      raw.push_back(DevBlock{b.offset, b.size, b.out_offset, 0, 0, kCodecRaw, (uint32_t)i});
    } else if (b.codec == XKSV_CODEC_SERIAL || b.codec == XKSV_CODEC_PARALLEL) {
      ok = b.rows && b.cols && b.cols <= UINT64_MAX / b.rows / 2 && b.rows * b.cols * 2 == b.raw_size &&
           b.rows * b.cols <= kMaxBlockElems && (b.codec == XKSV_CODEC_SERIAL || b.rows <= 16);
      (b.codec == XKSV_CODEC_SERIAL ? ser : par)
          .push_back(DevBlock{b.offset, b.size, b.out_offset, b.rows, b.cols, b.codec, (uint32_t)i});
    } else {
      ok = false;
    }
    if (ok) P->out_extent = std::max(P->out_extent, b.out_offset + b.raw_size);
  }
  // Waves claim parallel32 blocks in list order, so the largest go first: a
  // block is one wave's work, and a large one claimed last would keep a few
  // waves busy after the rest have drained (the 16x14336 slabs of a model's
  // last layer take ~3.5x a 16x4096 slab).  Status slots keep table order.
  std::stable_sort(par.begin(), par.end(),
                   [](const DevBlock& a, const DevBlock& b) { return a.rows * a.cols > b.rows * b.cols; });
  ok = ok && upload(ser, &P->d_serial) && upload(par, &P->d_parallel) && upload(raw, &P->d_raw);
  if (ok) {
    std::vector<HashItem> items;
    std::vector<uint32_t> first;
    hash_schedule(P->blocks, items, first);
    ok = upload(items, &P->hash_items) && upload(first, &P->hash_first);
    P->n_hash_lanes = (uint32_t)(first.size() - 1);
  }
  P->n_serial = (uint32_t)ser.size();
  if (ok && !ser.empty()) {  // serial blocks decode a workgroup each
    uint64_t max_elems = 0;
    for (const DevBlock& d : ser) max_elems = std::max<uint64_t>(max_elems, d.rows * d.cols);
    const DeviceInfo* di = current_device(nullptr);
    const uint64_t bytes =
        di ? serial_wg_scratch(P->n_serial, max_elems, (unsigned)di->cus, &P->serial_grid, &P->serial_cap) : 0;
    ok = di && hipMalloc(reinterpret_cast<void**>(&P->serial_scratch), bytes) == hipSuccess;
  }
  P->n_parallel = (uint32_t)par.size();
  P->n_raw = (uint32_t)raw.size();
  P->h_status.assign(nblocks ? nblocks : 1, 0);
  // Status words, then the decode launches' block queues (zeroed together).
  ok = ok && hipMalloc(reinterpret_cast<void**>(&P->status), (nblocks + kQueues) * 4) == hipSuccess &&
       launch_fill_u32(P->status, nblocks + kQueues, 0, nullptr) == hipSuccess &&
       hipStreamSynchronize(nullptr) == hipSuccess;
  if (!ok) {
    xksv_hip_plan_destroy(P);
    return 1;
  }
  *plan = P;
  return 0;
}

int xksv_hip_plan_destroy(xksv_hip_plan* P) {
  if (!P) return 0;
  int cur = -1;
  (void)hipGetDevice(&cur);
  if (P->device >= 0 && cur != P->device) (void)hipSetDevice(P->device);
  for (void* p : {(void*)P->d_serial, (void*)P->d_parallel, (void*)P->d_raw, (void*)P->status, (void*)P->g_fserial,
                  (void*)P->g_fparallel, (void*)P->g_gser, (void*)P->g_gpar, (void*)P->g_gplain, (void*)P->g_raw,
                  (void*)P->scratch, (void*)P->item_mem, (void*)P->digests, (void*)P->index, (void*)P->dindex,
                  (void*)P->dibase,
                  (void*)P->serial_scratch, (void*)P->hash_items, (void*)P->hash_first})
    if (p) (void)hipFree(p);
  if (cur >= 0 && cur != P->device) (void)hipSetDevice(cur);
  delete P;
  return 0;
}

int xksv_hip_plan_decode(xksv_hip_plan* P, const void* archive, void* out, uint64_t out_size, void* stream) {
  if (!P || (!archive && P->archive_size) || (!out && P->out_extent) || P->out_extent > out_size) return 1;
  const DeviceInfo* di = current_device(nullptr);
  if (!di) return 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* arc = static_cast<const uint8_t*>(archive);
  uint8_t* o = static_cast<uint8_t*>(out);
  uint32_t* queue = P->status + P->blocks.size();
  if (launch_fill_u32(P->status, P->blocks.size() + kQueues, 0, s) != hipSuccess) return 1;
  if (launch_decode(P->d_parallel, P->n_parallel, kCodecParallel, arc, o, P->status, queue, (unsigned)di->cus, s,
                    P->dindex, P->dibase) != hipSuccess)
    return 1;
  if (launch_decode_serial_wg(P->d_serial, P->n_serial, arc, o, P->status, P->serial_scratch, P->serial_cap,
                              P->serial_grid, s) != hipSuccess)
    return 1;
  if (launch_copy_raw(P->d_raw, P->n_raw, arc, o, s) != hipSuccess) return 1;
  return 0;
}

int xksv_hip_plan_index(xksv_hip_plan* P, const void* archive, void* stream) {
  if (!P || (!archive && P->archive_size)) return 1;
  if (!current_device(nullptr)) return 1;
  if (!P->n_parallel) return 0;
  if (!P->dindex) {
    // Block b's items get segs_b segments of kIdxSegSyms symbols, enough for
    // the 32 substreams the slab rule writes; other items stay unindexed.
    std::vector<DevBlock> par(P->n_parallel);
    if (hipMemcpy(par.data(), P->d_parallel, par.size() * sizeof(DevBlock), hipMemcpyDeviceToHost) != hipSuccess)
      return 1;
    std::vector<uint64_t> base(par.size() + 1, 0);
    for (size_t i = 0; i < par.size(); ++i) {
      const uint64_t syms = (par[i].rows * par[i].cols + kMaxChunks - 1) / kMaxChunks;
      const uint64_t segs = std::max<uint64_t>(1, (syms + kIdxSegSyms - 1) / kIdxSegSyms);
      base[i + 1] = base[i] + segs * kMaxChunks * 64;
    }
    P->dindex_bytes = base.back() * sizeof(uint16_t);
    if (P->dibase) (void)hipFree(P->dibase);  // left by a call whose index allocation failed
    if (!upload(base, &P->dibase)) return 1;
    if (hipMalloc(reinterpret_cast<void**>(&P->dindex), P->dindex_bytes) != hipSuccess) {
      P->dindex = nullptr;
      return 1;
    }
  }
  return launch_index_items(P->d_parallel, P->n_parallel, static_cast<const uint8_t*>(archive), P->dindex, 0,
                            static_cast<hipStream_t>(stream), P->dibase) == hipSuccess
             ? 0
             : 1;
}

// The plan GEMMs: fused kernels over 16-row compressed slabs, decode to
// scratch + plain GEMM for other compressed slabs, plain GEMM straight from
// the archive for raw slabs.  bf16 == false: fp32 X [cols, batch], Y
// [rows, batch]; bf16 == true: bf16 X [batch, cols], fp32 Y [batch, rows].
static int plan_gemm(xksv_hip_plan* P, const void* archive, const void* x, size_t batch, float* y, void* stream,
                     bool bf16) {
  if (!P || !archive || !x || !y || !batch) return 1;
  const DeviceInfo* di = current_device(nullptr);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* arc = static_cast<const uint8_t*>(archive);
  if (!di || !prepare_gemm(P, arc, s)) return 1;
  const unsigned cus = (unsigned)di->cus;
  uint32_t* queue = P->status + P->blocks.size();
  const float* xf = static_cast<const float*>(x);
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const uint64_t M = P->rows_extent, K = P->cols;
  const ItemScratch* items = P->item_mem ? &P->items : nullptr;
  // The substream kernels store their blocks' status words; the other kernels
  // OR errors in (and the decode queues count from zero).
  if ((!items || P->n_fserial || P->n_gser || P->n_gpar) &&
      launch_fill_u32(P->status, P->blocks.size() + kQueues, 0, s) != hipSuccess)
    return 1;
  for (uint64_t j0 = 0; j0 < batch; j0 += kMaxFusedBatch) {
    const uint32_t nb = (uint32_t)std::min<uint64_t>(kMaxFusedBatch, batch - j0);
    hipError_t e1, e2;
    if (!bf16) {
      e1 = launch_gemm_f32(P->g_fparallel, P->n_fparallel, kCodecParallel, arc, xf + j0, batch, nb, y + j0, batch,
                           P->status, items, cus, s);
      e2 = launch_gemm_f32(P->g_fserial, P->n_fserial, kCodecSerial, arc, xf + j0, batch, nb, y + j0, batch,
                           P->status, nullptr, cus, s);
    } else {
      e1 = launch_gemm_bf16(P->g_fparallel, P->n_fparallel, kCodecParallel, arc, xb + j0 * K, K, nb, y + j0 * M, M,
                            P->tile_parallel, P->status, items, cus, s);
      e2 = launch_gemm_bf16(P->g_fserial, P->n_fserial, kCodecSerial, arc, xb + j0 * K, K, nb, y + j0 * M, M, true,
                            P->status, nullptr, cus, s);
    }
    if (e1 != hipSuccess || e2 != hipSuccess) return 1;
  }
  if (launch_decode(P->g_gser, P->n_gser, kCodecSerial, arc, P->scratch, P->status, queue + 2, cus, s) !=
          hipSuccess ||
      launch_decode(P->g_gpar, P->n_gpar, kCodecParallel, arc, P->scratch, P->status, queue + 3, cus, s) !=
          hipSuccess)
    return 1;
  if (!bf16) {
    if (launch_gemm_plain(P->g_gplain, P->n_generic, P->scratch, xf, batch, (uint32_t)batch, y, batch, s) !=
            hipSuccess ||
        launch_gemm_plain(P->g_raw, P->n_graw, arc, xf, batch, (uint32_t)batch, y, batch, s) != hipSuccess)
      return 1;
  } else {
    if (launch_gemm_plain_bf16(P->g_gplain, P->n_generic, P->scratch, xb, K, (uint32_t)batch, y, M, s) !=
            hipSuccess ||
        launch_gemm_plain_bf16(P->g_raw, P->n_graw, arc, xb, K, (uint32_t)batch, y, M, s) != hipSuccess)
      return 1;
  }
  return 0;
}

int xksv_hip_plan_gemm(xksv_hip_plan* P, const void* archive, const float* x, size_t batch, float* y,
                       void* stream) {
  return plan_gemm(P, archive, x, batch, y, stream, false);
}

int xksv_hip_plan_gemm_bf16(xksv_hip_plan* P, const void* archive, const uint16_t* x, size_t batch, float* y,
                            void* stream) {
  return plan_gemm(P, archive, x, batch, y, stream, true);
}

int xksv_hip_plan_digests(xksv_hip_plan* P, const void* out, uint64_t out_size, uint8_t* digests,
                          uint64_t digests_size, void* stream) {
  if (!P || !out || !digests || out_size < P->out_extent || digests_size < 32ull * P->blocks.size()) return 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint8_t* o = static_cast<const uint8_t*>(out);
  return launch_sha256_lanes(P->hash_items, P->hash_first, P->n_hash_lanes, o, digests, s) == hipSuccess ? 0 : 1;
}

int xksv_hip_plan_verify(xksv_hip_plan* P, const void* out, uint64_t out_size, const uint8_t* expected,
                         uint64_t expected_size, uint32_t* verdicts, void* stream) {
  if (!P || !out || !expected || !verdicts || out_size < P->out_extent || expected_size < 32ull * P->blocks.size())
    return 1;
  if (P->blocks.empty()) return 0;
  if (!P->digests && hipMalloc(reinterpret_cast<void**>(&P->digests), 32 * P->blocks.size()) != hipSuccess) return 1;
  if (xksv_hip_plan_digests(P, out, out_size, P->digests, 32 * P->blocks.size(), stream)) return 1;
  return launch_digest_verdicts(P->digests, expected, P->status, (uint32_t)P->blocks.size(), verdicts,
                                static_cast<hipStream_t>(stream)) == hipSuccess
             ? 0
             : 1;
}

int xksv_hip_plan_error_flags(xksv_hip_plan* P, uint32_t* flags, void* stream) {
  if (!P || !flags) return 1;
  return launch_or_status(P->status, (uint32_t)P->blocks.size(), flags, static_cast<hipStream_t>(stream)) ==
                 hipSuccess
             ? 0
             : 1;
}

int64_t xksv_hip_plan_errors(xksv_hip_plan* P, void* stream, int64_t* first_bad, uint32_t* bits) {
  if (first_bad) *first_bad = -1;
  if (bits) *bits = 0;
  if (!P) return -1;
  if (hipStreamSynchronize(static_cast<hipStream_t>(stream)) != hipSuccess) return -1;
  if (P->blocks.empty()) return 0;
  if (hipMemcpy(P->h_status.data(), P->status, P->blocks.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  int64_t bad = 0;
  uint32_t all = 0;
  for (size_t i = 0; i < P->blocks.size(); ++i)
    if (P->h_status[i]) {
      if (first_bad && *first_bad < 0) *first_bad = (int64_t)i;
      all |= P->h_status[i];
      ++bad;
    }
  if (bits) *bits = all;
  return bad;
}

}  // extern "C"
