// xksv_noalloc.hip -- fused decode-GEMM over one XKSP2 block without any
// device allocation, for callers that cannot allocate (tight serving loops,
// harnesses that forbid hipMalloc).
//
// xksv_hip_gemm_parallel stages each call in a pooled device buffer that it
// allocates on demand.  xksv_hip_gemm_parallel_noalloc runs the same kernels
// and staging layout, but its staging -- descriptors, status word, the
// encoded block copied from the host, the substream partial sums, or the
// decoded slab of a block whose substreams are not unit-aligned -- lives in
// one file-scope device array of fixed size.  Each GPU holds its own copy of
// that array (kNoAllocScratch bytes) until the process ends.  Calls on one GPU
// share it: a per-device host lock makes calls from several host threads
// take turns; without the lock, overlapping calls would race on it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "xksv_api_internal.hpp"

namespace {

constexpr int kMaxDevices = 64;
// Room for the largest call the entry accepts: a 2 MiB encoded block plus a
// 2 MiB decoded slab (16 x 65,536 BF16) or the 32 KiB of substream partial
// sums, with the layout's descriptors, status words and alignment padding.
constexpr uint64_t kNoAllocScratch = XKSV_NOALLOC_SCRATCH_BYTES;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratch];

struct Slot {
  std::mutex mu;
  bool init = false;
  uint8_t* ptr = nullptr;  // this device's address of `scratch`
  int cus = 0;
};
Slot g_slot[kMaxDevices];

// The current device's scratch address and CU count, set up once per device
// with that device current.  The array's host-side name is not a device
// address: every use below goes through the address hipGetSymbolAddress gave.
Slot* device_slot() {
  int id = -1;
  if (hipGetDevice(&id) != hipSuccess || id < 0 || id >= kMaxDevices) return nullptr;
  Slot& s = g_slot[id];
  std::lock_guard<std::mutex> lk(s.mu);
  if (!s.init) {
    void* p = nullptr;
    int cus = 0;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, id) != hipSuccess || cus < 1)
      return nullptr;
    s.ptr = static_cast<uint8_t*>(p);
    s.cus = cus;
    s.init = true;
  }
  return &s;
}

}  // namespace

extern "C" int xksv_hip_gemm_parallel_noalloc(const void* input, size_t n, size_t batch, const float* x,
                                              float* output) {
  using namespace xksv;
  ParallelHeader h;
  if (!x || !output || !batch || !parallel_header(static_cast<const uint8_t*>(input), n, h)) return 1;
  if (batch > SIZE_MAX / h.rows) return 1;
  const Fused fused = fused_parallel(h);
  const BlockLayout L = block_layout(n, kCodecParallel, h.rows, h.cols, fused, kGemmF32);
  if (L.total > kNoAllocScratch) return 2;  // larger than the fixed scratch holds
  Slot* s = device_slot();
  if (!s) return 1;
  std::lock_guard<std::mutex> lk(s->mu);
  return run_block_at(s->ptr, L, static_cast<const uint8_t*>(input), n, kCodecParallel, h.rows, h.cols, fused,
                      kGemmF32, output, x, batch, (unsigned)s->cus);
}
