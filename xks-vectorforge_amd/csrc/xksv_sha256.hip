// SHA-256 (FIPS 180-4) of each block's decoded bytes, on the GPU: the
// per-slab digests an archive index records for the original-order bytes of
// every block [src/compile.cpp:255,443,489], which verification compares
// after decoding [src/verify.cpp:262-273].
//
// SHA-256 is sequential within a message, so one lane hashes a whole block
// and lanes hash independent blocks side by side; the time of a launch is
// that of its longest lane.  The host therefore hands each lane a list of
// blocks (largest first, smaller ones packed up to 0.6 of the largest block's
// size), so that the lanes of a wave carry equal work and the waves are
// fewer.  The 64 rounds are unrolled with the round constants
// as immediates; the message schedule is a rolling 16-word window in
// registers.  A lane reads its block 64 bytes at a time (four 16-byte loads
// when the block is 16-byte aligned, as every slab of a decoded tensor is;
// byte loads otherwise).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "xksv_shared.hpp"

namespace xksv {
namespace {

constexpr uint32_t kSha256K[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
    0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
    0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
    0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
    0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

__device__ __forceinline__ uint32_t rotr(uint32_t x, uint32_t n) { return __builtin_amdgcn_alignbit(x, x, n); }
// Three-input bitwise functions in one v_bitop3_b32 each (the immediate is the
// function's truth table over the inputs 0xf0, 0xcc, 0xaa); both are symmetric
// in their inputs.  The compiler otherwise splits each three-way XOR into two.
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}
__device__ __forceinline__ uint32_t maj3(uint32_t a, uint32_t b, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, b, c, 0xe8);
}
__device__ __forceinline__ uint32_t be32(uint32_t v) { return __builtin_amdgcn_perm(0u, v, 0x00010203u); }

// One 64-byte chunk (16 big-endian words) into the state.
__device__ __forceinline__ void compress(uint32_t (&h)[8], uint32_t (&w)[16]) {
  uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], k = h[7];
#pragma unroll
  for (int t = 0; t < 64; ++t) {
    uint32_t wt;
    if (t < 16) {
      wt = w[t];
    } else {
      const uint32_t w15 = w[(t - 15) & 15], w2 = w[(t - 2) & 15];
      const uint32_t s0 = xor3(rotr(w15, 7), rotr(w15, 18), w15 >> 3);
      const uint32_t s1 = xor3(rotr(w2, 17), rotr(w2, 19), w2 >> 10);
      wt = w[t & 15] + s0 + w[(t - 7) & 15] + s1;
      w[t & 15] = wt;
    }
    const uint32_t S1 = xor3(rotr(e, 6), rotr(e, 11), rotr(e, 25));
    const uint32_t ch = (e & f) ^ (~e & g);
    const uint32_t t1 = k + S1 + ch + kSha256K[t] + wt;
    const uint32_t S0 = xor3(rotr(a, 2), rotr(a, 13), rotr(a, 22));
    const uint32_t mj = maj3(a, b, c);
    k = g;
    g = f;
    f = e;
    e = d + t1;
    d = c;
    c = b;
    b = a;
    a = t1 + S0 + mj;
  }
  h[0] += a;
  h[1] += b;
  h[2] += c;
  h[3] += d;
  h[4] += e;
  h[5] += f;
  h[6] += g;
  h[7] += k;
}

// The SHA-256 digest of the n bytes at p into digest[0, 32).
__device__ void sha256(const uint8_t* __restrict__ p, uint64_t n, uint8_t* __restrict__ digest) {
  uint32_t h[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                   0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
  uint32_t w[16];
  const uint64_t full = n / 64;
  if ((reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
    // The next chunk is in flight while this one is compressed (~1,400 VALU
    // instructions), which hides the memory latency that the one or two
    // waves per SIMD of this launch cannot (-4 % on the Llama-3-8B archive).  The last chunk reloads itself,
    // so the load needs no branch (a conditional load would make the
    // compiler copy the chunk between register sets, waiting on the load).
    const uint4* q4 = reinterpret_cast<const uint4*>(p);
    uint4 nxt[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) nxt[i] = full ? q4[i] : make_uint4(0u, 0u, 0u, 0u);
    for (uint64_t c = 0; c < full; ++c) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        w[4 * i] = be32(nxt[i].x);
        w[4 * i + 1] = be32(nxt[i].y);
        w[4 * i + 2] = be32(nxt[i].z);
        w[4 * i + 3] = be32(nxt[i].w);
      }
      // The empty asm hides the chunk index from the optimiser, which would
      // otherwise see that nxt equals a load at the chunk's own address and
      // re-issue that load where the chunk is used, waiting on it there.
      uint64_t at = 4 * (c + 1 < full ? c + 1 : c);
      asm volatile("" : "+v"(at));
#pragma unroll
      for (int i = 0; i < 4; ++i) nxt[i] = q4[at + i];
      // Keep the loads ahead of the compression: the scheduler would sink
      // them past it (to free their registers), back to where they are used.
      __builtin_amdgcn_sched_barrier(0);
      compress(h, w);
    }
  } else {
    for (uint64_t c = 0; c < full; ++c) {
      const uint8_t* q = p + 64 * c;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        w[i] = ((uint32_t)q[4 * i] << 24) | ((uint32_t)q[4 * i + 1] << 16) | ((uint32_t)q[4 * i + 2] << 8) | q[4 * i + 3];
      compress(h, w);
    }
  }
  // Padding: the r remaining bytes, 0x80, zeros, then the bit length
  // (big-endian 64-bit) in the last 8 bytes; two chunks when r >= 56.
  const uint32_t r = (uint32_t)(n % 64);
  const uint8_t* q = p + 64 * full;
  const uint64_t bits = n * 8;
  for (uint32_t chunk = 0; chunk < (r >= 56 ? 2u : 1u); ++chunk) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t at = 64 * chunk + 4 * i + j;
        const uint32_t byte = at < r ? q[at] : at == r ? 0x80u : 0u;
        word = (word << 8) | byte;
      }
      w[i] = word;
    }
    if (chunk == (r >= 56 ? 1u : 0u)) {
      w[14] = (uint32_t)(bits >> 32);
      w[15] = (uint32_t)bits;
    }
    compress(h, w);
  }
  uint32_t* dg = reinterpret_cast<uint32_t*>(digest);
#pragma unroll
  for (int i = 0; i < 8; ++i) dg[i] = be32(h[i]);
}

// Lane l hashes items[first[l] .. first[l + 1]) in order.
__global__ void __launch_bounds__(256) k_sha256_lanes(const HashItem* __restrict__ items,
                                                      const uint32_t* __restrict__ first, uint32_t nlanes,
                                                      const uint8_t* __restrict__ out, uint8_t* __restrict__ digests) {
  const uint32_t l = blockIdx.x * blockDim.x + threadIdx.x;
  if (l >= nlanes) return;
  for (uint32_t i = first[l], e = first[l + 1]; i < e; ++i) {
    const HashItem it = items[i];
    sha256(out + it.dst, it.n, digests + 32ull * it.slot);
  }
}

// Per-block verdict of a verification pass: the block's decode error bits
// plus kErrDigest when the SHA-256 of its decoded bytes differs from the
// digest the index records for it [src/verify.cpp:262-263].  Digests, the
// expected digests and the status words are indexed by block (table order).
__global__ void __launch_bounds__(256) k_digest_verdicts(const uint8_t* __restrict__ digests,
                                                         const uint8_t* __restrict__ expected,
                                                         const uint32_t* __restrict__ status, uint32_t n,
                                                         uint32_t* __restrict__ verdicts) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    uint32_t diff = 0;
#pragma unroll
    for (int k = 0; k < 32; k += 4) {
      uint32_t a, b;
      __builtin_memcpy(&a, digests + 32ull * i + k, 4);
      __builtin_memcpy(&b, expected + 32ull * i + k, 4);
      diff |= a ^ b;
    }
    verdicts[i] = status[i] | (diff ? (uint32_t)kErrDigest : 0u);
  }
}

}  // namespace

hipError_t launch_digest_verdicts(const uint8_t* digests, const uint8_t* expected, const uint32_t* status, uint32_t n,
                                  uint32_t* verdicts, hipStream_t s) {
  if (!n) return hipSuccess;
  const unsigned g = (n + 255) / 256;
  hipLaunchKernelGGL(k_digest_verdicts, dim3(g < 1024 ? g : 1024u), dim3(256), 0, s, digests, expected, status, n,
                     verdicts);
  return hipGetLastError();
}

hipError_t launch_sha256_lanes(const HashItem* items, const uint32_t* first, uint32_t nlanes, const uint8_t* out,
                               uint8_t* digests, hipStream_t s) {
  if (!nlanes) return hipSuccess;
  hipLaunchKernelGGL(k_sha256_lanes, dim3((nlanes + 255) / 256), dim3(256), 0, s, items, first, nlanes, out, digests);
  return hipGetLastError();
}

}  // namespace xksv
