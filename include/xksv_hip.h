/*
 * xksv_hip.h -- C ABI of the MI355X (gfx950) XKSV compressed-weight path.
 *
 * One shared library, libxksv_hip.so, replaces both reference libraries for
 * this path:
 *   libxksv_native.so  (CPU codec, src/c_api.cpp:16-85)
 *   libxksv_cuda.so    (GPU block decode / fused GEMV / GEMM,
 *                       cuda/decode.cu:85-98, cuda/parallel.cu:68-74)
 * Signatures, argument meaning, pointer residency and return conventions are
 * the reference's; the block format (.xksv serial "bf16-huffman-tile16" and
 * XKSP2 "bf16-huffman-parallel32" blocks) is unchanged.  Plain pointers and
 * sizes only.  Decoding always runs on the GPU: without a HIP device every
 * decode entry point fails (returns its error value), xksv_unpack and
 * xksv_unpack_parallel included -- there is no CPU decode in this library, so
 * CPU-only consumers of the codec keep the reference's libxksv_native.so.
 */
#ifndef XKSV_HIP_H
#define XKSV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------
 * CPU-side codec surface.  Host pointers in and out; 0 on success, -1 on any
 * error; *out is malloc'd and released with xksv_free.
 * ---------------------------------------------------------------------- */

/* Replaces src/c_api.cpp:17. */
void xksv_free(void* p);

/* Replaces src/c_api.cpp:18 (xksv_pack).  Serial block of a rows x cols BF16
 * slab (n = 2*rows*cols bytes); bytes identical to the reference encoder. */
int xksv_pack(const void* data, size_t n, size_t rows, size_t cols, void** out, size_t* out_size);

/* Replaces src/c_api.cpp:29 (xksv_unpack).  Same validation and result; the
 * decode itself runs on the current HIP device. */
int xksv_unpack(const void* data, size_t n, size_t rows, size_t cols, void** out, size_t* out_size);

/* Replaces src/c_api.cpp:44 (xksv_pack_parallel).  XKSP2 block, rows <= 16. */
int xksv_pack_parallel(const void* data, size_t n, size_t rows, size_t cols, void** out, size_t* out_size);

/* Replaces src/c_api.cpp:66 (xksv_unpack_parallel); decodes on the GPU. */
int xksv_unpack_parallel(const void* data, size_t n, void** out, size_t* out_size);

/* ------------------------------------------------------------------------
 * GPU block API.  `input` is a host pointer to one encoded block; `output`,
 * `x` are device pointers on the current device.  Synchronous; 0 on success,
 * 1 on any validation, bitstream or HIP error (output may be partially
 * written on error).  The xksv_cuda_* names are exported as aliases so
 * callers binding the reference names (python/runtime.py:40-44,
 * python/tune.py:16-19) load this library unchanged.
 * ---------------------------------------------------------------------- */

/* Replaces cuda/decode.cu:85 (xksv_cuda_decode): serial block -> BF16
 * rows x cols row-major at output. */
int xksv_hip_decode(const void* input, size_t size, size_t rows, size_t cols, void* output);

/* Replaces cuda/decode.cu:89 (xksv_cuda_gemv): output[r] = sum_c W[r,c] x[c],
 * fp32 x[cols], fp32 output[rows] (fully overwritten).  x == NULL -> 1. */
int xksv_hip_gemv(const void* input, size_t size, size_t rows, size_t cols, const float* x, float* output);

/* Replaces cuda/decode.cu:95 (xksv_cuda_gemm): X and output are row-major
 * fp32 [cols, batch] and [rows, batch]. */
int xksv_hip_gemm(const void* input, size_t size, size_t rows, size_t cols, size_t batch, const float* x,
                  float* output);

/* Replaces cuda/parallel.cu:68 (xksv_cuda_decode_parallel): XKSP2 block; the
 * shape comes from the block header. */
int xksv_hip_decode_parallel(const void* input, size_t n, void* output);

/* Replaces cuda/parallel.cu:71 (xksv_cuda_gemv_parallel): output[rows] fp32,
 * fully overwritten; deterministic summation order. */
int xksv_hip_gemv_parallel(const void* input, size_t n, const float* x, float* output);

/* No reference counterpart (the reference has no parallel GEMM): fused GEMM
 * over an XKSP2 block, X [cols, batch] and output [rows, batch] row-major fp32,
 * the layout of xksv_cuda_gemm. */
int xksv_hip_gemm_parallel(const void* input, size_t n, size_t batch, const float* x, float* output);

/* No reference counterpart (the reference's GEMM takes fp32 X only): fused
 * decode-GEMM over an XKSP2 block with bf16 activations in the layout of
 * torch's x @ W.T -- X [batch, cols] bf16 row-major, output [batch, rows] fp32
 * row-major -- accumulated in fp32.  When every substream covers whole 16x16
 * tiles, the products run on bf16 MFMA (v_mfma_f32_16x16x32_bf16);
 * otherwise on the VALU (v_dot2 of bf16 pairs into fp32). */
int xksv_hip_gemm_parallel_bf16(const void* input, size_t n, size_t batch, const uint16_t* x, float* output);

/* No reference counterpart.  For callers that cannot allocate device memory
 * (serving loops, harnesses that forbid hipMalloc): xksv_hip_gemm_parallel
 * with the same arguments, kernels and results, staged in a fixed device array
 * of XKSV_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends) instead
 * of allocated buffers; it calls no hipMalloc/hipFree.  Returns 0 on success,
 * 1 on any validation, bitstream or HIP error, 2 when the call's staging (the
 * encoded block plus its 32 KiB of substream partial sums, or plus its decoded
 * slab when the substreams are not unit-aligned) exceeds the array; every
 * block the archive compiler writes (at most 1 MiB raw) fits.  Calls on one
 * GPU share the array: they take turns under a per-device host lock. */
#define XKSV_NOALLOC_SCRATCH_BYTES ((4u << 20) + (64u << 10))
int xksv_hip_gemm_parallel_noalloc(const void* input, size_t n, size_t batch, const float* x, float* output);

/* Reference names, same functions. */
int xksv_cuda_decode(const void* input, size_t size, size_t rows, size_t cols, void* output);
int xksv_cuda_gemv(const void* input, size_t size, size_t rows, size_t cols, const float* x, float* output);
int xksv_cuda_gemm(const void* input, size_t size, size_t rows, size_t cols, size_t batch, const float* x,
                   float* output);
int xksv_cuda_decode_parallel(const void* input, size_t n, void* output);
int xksv_cuda_gemv_parallel(const void* input, size_t n, const float* x, float* output);

/* ------------------------------------------------------------------------
 * Device-resident batched API (no reference counterpart; it replaces the
 * per-block loops of python/runtime.py:86-99 (GPU load) and :264-284 (fused
 * GEMV) with one stream-ordered launch per codec).  The archive stays
 * resident in HBM; descriptors are uploaded once per plan.
 * ---------------------------------------------------------------------- */

enum { XKSV_CODEC_RAW = 0, XKSV_CODEC_SERIAL = 1, XKSV_CODEC_PARALLEL = 2 };

/* Per-block error bits reported by xksv_hip_plan_errors (1-8) and xksv_hip_plan_verify (all). */
enum { XKSV_ERR_HEADER = 1, XKSV_ERR_CODEBOOK = 2, XKSV_ERR_STREAM = 4, XKSV_ERR_SHAPE = 8, XKSV_ERR_DIGEST = 16 };

/* One block of the archive index (src/compile.cpp:461-468 fields). */
typedef struct xksv_hip_block {
  uint64_t offset;     /* encoded block: byte offset within the device archive buffer */
  uint64_t size;       /* encoded size in bytes */
  uint64_t raw_size;   /* decoded size in bytes */
  uint64_t out_offset; /* decode: output byte offset; gemv/gemm: first output row */
  uint64_t rows, cols; /* slab shape; 0 for raw blocks */
  uint32_t codec;      /* XKSV_CODEC_* */
  uint32_t reserved;   /* must be 0 */
} xksv_hip_block;

typedef struct xksv_hip_plan xksv_hip_plan;

/* Validate descriptors against the index rules (raw: size == raw_size;
 * compressed: raw_size == 2*rows*cols; block inside archive_size) and upload
 * them to the current device.  0 on success, 1 on error. */
int xksv_hip_plan_create(const xksv_hip_block* blocks, size_t nblocks, uint64_t archive_size, xksv_hip_plan** plan);
int xksv_hip_plan_destroy(xksv_hip_plan* plan);

/* Enqueue decode of every block into `out` (device, out_size bytes) on
 * `stream` (a hipStream_t; NULL = null stream).  Asynchronous; errors are
 * collected per block, read them with xksv_hip_plan_errors. */
int xksv_hip_plan_decode(xksv_hip_plan* plan, const void* archive, void* out, uint64_t out_size, void* stream);

/* No reference counterpart (a load-time sidecar for weights that stay
 * resident and are decoded again and again, the GPU-resident path of
 * python/runtime.py:86-99,248-287): build, on `stream`, a codeword index of
 * the plan's parallel32 blocks from `archive` -- the bit offset of every 32nd
 * codeword of every substream, 128 bytes per 2,048 symbols (~4 % of the
 * encoded size) -- which later xksv_hip_plan_decode calls use to start each
 * lane of a wave at a known codeword.  Every entry is checked as it is used,
 * so an index built from another archive only costs speed: a substream whose
 * entries do not chain is decoded without them, with identical results and
 * errors.  A second call rebuilds it.  0 on success, 1 on error. */
int xksv_hip_plan_index(xksv_hip_plan* plan, const void* archive, void* stream);

/* Enqueue fused decode-GEMM, fp32 X [cols, batch] row-major, Y [rows, batch]
 * (block rows start at out_offset).  All blocks must share `cols`; raw blocks
 * (rows = cols = 0 in archive indexes) take it from the compressed ones, and a
 * table of raw blocks only must give it in their cols field.  batch = 1 is the
 * batch-1 GEMV of python/runtime.py:264-284. */
int xksv_hip_plan_gemm(xksv_hip_plan* plan, const void* archive, const float* x, size_t batch, float* y,
                       void* stream);

/* As xksv_hip_plan_gemm with bf16 activations X [batch, cols] row-major and
 * fp32 output Y [batch, M] row-major, M = the plan's row extent (largest
 * out_offset + rows); bf16 MFMA on whole-tile substreams (see xksv_hip_gemm_parallel_bf16). */
int xksv_hip_plan_gemm_bf16(xksv_hip_plan* plan, const void* archive, const uint16_t* x, size_t batch, float* y,
                            void* stream);

/* No reference counterpart as a C entry (the reference hashes on the host,
 * src/verify.cpp:262-273): enqueue SHA-256 of every block's decoded bytes --
 * out[out_offset, out_offset + raw_size), as written by xksv_hip_plan_decode
 * into `out` (device, out_size bytes) on the same stream -- into `digests`
 * (device, digests_size >= 32 bytes per block, in table order: the per-slab
 * digests of src/compile.cpp:255,443,489).  0 on success, 1 on error (null
 * pointers or buffers too small for the plan). */
int xksv_hip_plan_digests(xksv_hip_plan* plan, const void* out, uint64_t out_size, uint8_t* digests,
                          uint64_t digests_size, void* stream);

/* Block verdicts of an archive verification [src/verify.cpp:239-263]: after
 * xksv_hip_plan_decode into `out` on the same stream, hash every block's
 * decoded bytes with SHA-256 on the GPU and compare with `expected` (device,
 * 32 bytes per block in table order: the index's per-block digests).
 * verdicts[i] (device, one uint32 per block) = the block's decode error bits,
 * plus XKSV_ERR_DIGEST when its digest differs; 0 = the block verifies.
 * Enqueued on `stream`; 0 on success, 1 on error (null pointers or buffers
 * too small for the plan).  The first call allocates the plan's digest
 * buffer (32 bytes per block). */
int xksv_hip_plan_verify(xksv_hip_plan* plan, const void* out, uint64_t out_size, const uint8_t* expected,
                         uint64_t expected_size, uint32_t* verdicts, void* stream);

/* No reference counterpart: enqueue on `stream` an OR of every block's error
 * bits from the plan's last decode or GEMM into *flags (a device word the
 * caller owns and clears; the bits accumulate across calls).  No host
 * synchronisation, so a forward pass can record errors under graph capture
 * and check them later.  0 on success, 1 on error. */
int xksv_hip_plan_error_flags(xksv_hip_plan* plan, uint32_t* flags, void* stream);

/* Synchronize `stream`, return the number of failed blocks (or -1 on a HIP
 * error); *first_bad (optional) gets the first failing block index or -1,
 * *bits (optional) the OR of all error bits. */
int64_t xksv_hip_plan_errors(xksv_hip_plan* plan, void* stream, int64_t* first_bad, uint32_t* bits);

/* Encode one tensor with the compiler's slab rule (src/compile.cpp:449-486)
 * on `threads` host threads (0 = all): codec 1 serial, 2 parallel32; blocks
 * that do not shrink stay raw.  *out / *blocks are malloc'd (xksv_free);
 * block offsets are relative to *out, out_offset is the block's byte offset
 * within the tensor. */
int xksv_encode_tensor(const void* data, uint64_t nbytes, int bf16, uint64_t shape_cols, uint32_t codec,
                       uint32_t threads, void** out, uint64_t* out_size, xksv_hip_block** blocks,
                       uint64_t* nblocks);

/* Library / device information: 0 on success.  cus = compute units of the
 * current device (0 without a device). */
int xksv_hip_version(void);
int xksv_hip_device_cus(void);

#ifdef __cplusplus
}
#endif
#endif /* XKSV_HIP_H */
