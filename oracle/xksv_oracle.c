/*
 * xksv_oracle.c -- CPU oracle for the XKSV compressed-weight path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker, never the product: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.  The
 * shipped library (xks-vectorforge_amd/) never links, loads or calls it.
 *
 * A plain-C restatement of the reference's CPU codec, function by function:
 *   oracle_tile / oracle_untile      src/layout.cpp:32-53   (transform, tile, untile)
 *   canonical()                      src/codec.cpp:11-29    (canonical code assignment)
 *   encode_bf16()                    src/codec.cpp:32-58    (Huffman lengths, tie-breaking, bit packing)
 *   decode_bf16()                    src/codec.cpp:59-74    (bit-serial tree walk + error checks)
 *   oracle_pack / oracle_unpack      src/c_api.cpp:18-40    (serial block, 272-byte header)
 *   oracle_pack_parallel /
 *   oracle_unpack_parallel           src/c_api.cpp:44-85    (XKSP2 block, <=32 substreams)
 *   oracle_free                      src/c_api.cpp:17
 *   oracle_gemm_f64                  cuda/decode.cu:28-45 semantics (Y[r,k] = sum_c W[r,c] X[c,k]),
 *                                    accumulated in fp64 as the parity reference for fused GEMV/GEMM.
 *
 * Every function is pinned by tests/test_oracle.py against the golden vectors
 * in tests/golden/ (written by the compiled reference, oracle/_ref) and against
 * closed forms (exhaustive 65,536-pattern round trip, RFC 1951 canonical codes,
 * Kraft equality of Huffman lengths).  Return conventions follow the reference:
 * 0 on success, -1 on any error; outputs are malloc'd and released with
 * oracle_free.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define MAXSZ ((size_t)-1)

/* ORACLE_PLANTED_MISTAKE selects a deliberately wrong variant (1: Huffman
 * tie-break, 2: canonical symbol order) that tests/test_oracle.py builds on the
 * side to show the golden vectors reject it.  The default build plants nothing. */
#ifndef ORACLE_PLANTED_MISTAKE
#define ORACLE_PLANTED_MISTAKE 0
#endif

/* ------------------------------------------------------------------ layout */

/* src/layout.cpp:32-50: row-major matrix <-> row-major tr x tc tiles; edge
 * tiles hold only the real elements. */
static int transform(const uint16_t *in, size_t rows, size_t cols, size_t tr,
                     size_t tc, int inverse, uint16_t *out) {
  if (!tr || !tc || (cols && rows > MAXSZ / cols)) return -1;
  size_t packed = 0;
  for (size_t r = 0; r < rows;) {
    size_t nr = tr < rows - r ? tr : rows - r;
    for (size_t c = 0; c < cols;) {
      size_t nc = tc < cols - c ? tc : cols - c;
      for (size_t i = 0; i < nr; ++i) {
        size_t original = (r + i) * cols + c;
        if (inverse)
          memcpy(out + original, in + packed, nc * 2);
        else
          memcpy(out + packed, in + original, nc * 2);
        packed += nc;
      }
      c += nc;
    }
    r += nr;
  }
  return 0;
}

int oracle_tile(const uint16_t *in, size_t rows, size_t cols, size_t tr,
                size_t tc, uint16_t *out) {
  return transform(in, rows, cols, tr, tc, 0, out);
}

int oracle_untile(const uint16_t *in, size_t rows, size_t cols, size_t tr,
                  size_t tc, uint16_t *out) {
  return transform(in, rows, cols, tr, tc, 1, out);
}

/* --------------------------------------------------------------- canonical */

/* Codes are kept as bit strings, one byte per bit, exactly like the
 * reference's std::string codes. */
typedef struct {
  uint8_t len[256];
  uint8_t bits[256][256];
} codes_t;

/* src/codec.cpp:11-29: visit (length, symbol) in ascending order; the first
 * code is all zeros, each next code is the previous one plus one, then
 * extended with zeros to its length.  Incrementing an all-ones code means the
 * lengths are oversubscribed. */
static int canonical(const uint8_t lengths[256], codes_t *codes) {
  uint8_t code[256];
  int size = 0;
  memset(codes->len, 0, sizeof codes->len);
  for (int length = 1; length < 256; ++length)
    for (int k = 0; k < 256; ++k) {
#if ORACLE_PLANTED_MISTAKE == 2 /* tests only: symbols of one length in descending order */
      int symbol = 255 - k;
#else
      int symbol = k;
#endif
      if (lengths[symbol] != length) continue;
      if (size == 0) {
        memset(code, 0, (size_t)length);
      } else {
        int i = size - 1;
        while (i >= 0 && code[i] == 1) code[i--] = 0;
        if (i < 0) return -1; /* oversubscribed Huffman codebook */
        code[i] = 1;
        memset(code + size, 0, (size_t)(length - size));
      }
      size = length;
      codes->len[symbol] = (uint8_t)length;
      memcpy(codes->bits[symbol], code, (size_t)length);
    }
  return 0;
}

/* ------------------------------------------------------------------ encode */

typedef struct {
  uint64_t count, bit_count;
  uint8_t lengths[256];
  uint8_t *sign_mantissa; /* count bytes */
  uint8_t *exponents;     /* ceil(bit_count / 8) bytes */
  size_t exp_size;
} block_t;

static void block_release(block_t *b) {
  free(b->sign_mantissa);
  free(b->exponents);
  b->sign_mantissa = b->exponents = NULL;
}

typedef struct { uint64_t freq; int id; } item_t;

static int item_less(item_t a, item_t b) {
#if ORACLE_PLANTED_MISTAKE == 1 /* tests only: ties broken by the larger node id */
  return a.freq < b.freq || (a.freq == b.freq && a.id > b.id);
#else
  return a.freq < b.freq || (a.freq == b.freq && a.id < b.id);
#endif
}

/* Binary min-heap over (freq, node id).  Keys are unique (ids are unique), so
 * the pop order is fully determined and equals std::priority_queue with
 * std::greater<pair<uint64_t,int>>. */
static void heap_push(item_t *h, int *n, item_t v) {
  int i = (*n)++;
  h[i] = v;
  while (i > 0) {
    int p = (i - 1) / 2;
    if (!item_less(h[i], h[p])) break;
    item_t t = h[i]; h[i] = h[p]; h[p] = t;
    i = p;
  }
}

static item_t heap_pop(item_t *h, int *n) {
  item_t top = h[0];
  h[0] = h[--(*n)];
  int i = 0;
  for (;;) {
    int l = 2 * i + 1, r = l + 1, m = i;
    if (l < *n && item_less(h[l], h[m])) m = l;
    if (r < *n && item_less(h[r], h[m])) m = r;
    if (m == i) break;
    item_t t = h[i]; h[i] = h[m]; h[m] = t;
    i = m;
  }
  return top;
}

/* src/codec.cpp:32-58.  Exponent symbol = (w >> 7) & 255.  Leaves get node ids
 * 0..k-1 in ascending symbol order; pop a then b, new node {a, b}; depth via
 * DFS, single symbol gets length 1; depth > 255 is an error. */
static int encode_bf16(const uint16_t *words, size_t n, block_t *out) {
  memset(out, 0, sizeof *out);
  out->count = n;
  uint64_t freq[256] = {0};
  for (size_t i = 0; i < n; ++i) ++freq[(words[i] >> 7) & 255];
  int nsym[511], nleft[511], nright[511], nnodes = 0;
  item_t heap[512];
  int hn = 0;
  for (int i = 0; i < 256; ++i)
    if (freq[i]) {
      nsym[nnodes] = i; nleft[nnodes] = nright[nnodes] = -1;
      item_t it = {freq[i], nnodes++};
      heap_push(heap, &hn, it);
    }
  while (hn > 1) {
    item_t a = heap_pop(heap, &hn), b = heap_pop(heap, &hn);
    if (a.freq > UINT64_MAX - b.freq) return -1; /* frequency overflow */
    nsym[nnodes] = -1;
    nleft[nnodes] = a.id; nright[nnodes] = b.id;
    item_t it = {a.freq + b.freq, nnodes++};
    heap_push(heap, &hn, it);
  }
  if (hn) {
    int stack_node[512], stack_depth[512], sp = 0;
    stack_node[sp] = heap[0].id; stack_depth[sp++] = 0;
    while (sp) {
      int i = stack_node[--sp], depth = stack_depth[sp];
      if (nsym[i] >= 0) {
        if (depth > 255) return -1; /* Huffman tree too deep */
        out->lengths[nsym[i]] = (uint8_t)(depth > 1 ? depth : 1);
      } else {
        stack_node[sp] = nleft[i]; stack_depth[sp++] = depth + 1;
        stack_node[sp] = nright[i]; stack_depth[sp++] = depth + 1;
      }
    }
  }
  codes_t *codes = (codes_t *)malloc(sizeof *codes);
  if (!codes) return -1;
  if (canonical(out->lengths, codes)) { free(codes); return -1; }
  uint64_t total_bits = 0;
  for (size_t i = 0; i < n; ++i) total_bits += codes->len[(words[i] >> 7) & 255];
  out->sign_mantissa = (uint8_t *)malloc(n ? n : 1);
  out->exp_size = (size_t)(total_bits / 8 + (total_bits % 8 != 0));
  out->exponents = (uint8_t *)calloc(out->exp_size ? out->exp_size : 1, 1);
  if (!out->sign_mantissa || !out->exponents) { free(codes); block_release(out); return -1; }
  uint64_t pos = 0;
  for (size_t i = 0; i < n; ++i) {
    uint16_t w = words[i];
    out->sign_mantissa[i] = (uint8_t)(((w >> 8) & 128) | (w & 127));
    int s = (w >> 7) & 255;
    for (int k = 0; k < codes->len[s]; ++k, ++pos)
      if (codes->bits[s][k]) out->exponents[pos / 8] |= (uint8_t)(0x80u >> (pos & 7));
  }
  out->bit_count = pos;
  free(codes);
  return 0;
}

/* ------------------------------------------------------------------ decode */

/* src/codec.cpp:59-74: rebuild the binary tree from the canonical codes,
 * then walk it bit by bit.  Errors: length mismatch, invalid prefix code,
 * invalid codebook, truncated bitstream, missing branch, trailing bits. */
static int decode_bf16(const block_t *b, uint16_t *result) {
  if (b->bit_count / 8 + (b->bit_count % 8 != 0) != b->exp_size) return -1;
  codes_t *codes = (codes_t *)malloc(sizeof *codes);
  if (!codes) return -1;
  if (canonical(b->lengths, codes)) { free(codes); return -1; }
  /* at most 1 + 256 * 255 nodes */
  int cap = 1 + 256 * 255;
  int *child0 = (int *)malloc(sizeof(int) * cap), *child1 = (int *)malloc(sizeof(int) * cap);
  int *symbol = (int *)malloc(sizeof(int) * cap);
  int rc = -1, nodes = 1;
  if (!child0 || !child1 || !symbol) goto done;
  child0[0] = child1[0] = symbol[0] = -1;
  for (int s = 0; s < 256; ++s) {
    if (!codes->len[s]) continue;
    int node = 0;
    for (int k = 0; k < codes->len[s]; ++k) {
      if (symbol[node] != -1) goto done; /* invalid prefix code */
      int *slot = codes->bits[s][k] ? &child1[node] : &child0[node];
      if (*slot < 0) {
        *slot = nodes;
        child0[nodes] = child1[nodes] = symbol[nodes] = -1;
        ++nodes;
      }
      node = *slot;
    }
    if (symbol[node] != -1 || child0[node] != -1 || child1[node] != -1) goto done; /* invalid codebook */
    symbol[node] = s;
  }
  {
    uint64_t pos = 0;
    for (uint64_t i = 0; i < b->count; ++i) {
      int node = 0;
      while (symbol[node] < 0) {
        if (pos >= b->bit_count) goto done; /* truncated bitstream */
        int bit = (b->exponents[pos / 8] >> (7 - (pos % 8))) & 1;
        ++pos;
        node = bit ? child1[node] : child0[node];
        if (node < 0) goto done; /* invalid bitstream */
      }
      uint8_t sm = b->sign_mantissa[i];
      result[i] = (uint16_t)(((sm & 128u) << 8) | ((unsigned)symbol[node] << 7) | (sm & 127u));
    }
    if (pos != b->bit_count) goto done; /* trailing exponent bits */
  }
  rc = 0;
done:
  free(child0); free(child1); free(symbol); free(codes);
  return rc;
}

/* ---------------------------------------------------------------- c_api */

static void put64(uint8_t *p, uint64_t v) {
  for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i));
}

static uint64_t get64(const uint8_t *p) {
  uint64_t v = 0;
  for (int i = 0; i < 8; ++i) v |= (uint64_t)p[i] << (8 * i);
  return v;
}

void oracle_free(void *p) { free(p); }

static size_t segment_size(const block_t *b) { return 272 + (size_t)b->count + b->exp_size; }

static void write_segment(uint8_t *p, const block_t *b) {
  put64(p, b->count);
  put64(p + 8, b->bit_count);
  memcpy(p + 16, b->lengths, 256);
  memcpy(p + 272, b->sign_mantissa, (size_t)b->count);
  memcpy(p + 272 + b->count, b->exponents, b->exp_size);
}

static uint16_t *load_words(const void *data, size_t n) {
  const uint8_t *p = (const uint8_t *)data;
  uint16_t *w = (uint16_t *)malloc(n / 2 ? n : 2);
  if (w)
    for (size_t i = 0; i < n / 2; ++i) w[i] = (uint16_t)(p[2 * i] | (p[2 * i + 1] << 8));
  return w;
}

static int emit_words(const uint16_t *w, size_t count, void **out, size_t *out_size) {
  uint8_t *o = (uint8_t *)malloc(count ? count * 2 : 1);
  if (!o) return -1;
  for (size_t i = 0; i < count; ++i) { o[2 * i] = (uint8_t)(w[i] & 255); o[2 * i + 1] = (uint8_t)(w[i] >> 8); }
  *out = o;
  *out_size = count * 2;
  return 0;
}

/* src/c_api.cpp:18-28 */
int oracle_pack(const void *data, size_t n, size_t rows, size_t cols, void **out, size_t *out_size) {
  if (n % 2 || rows == 0 || cols > MAXSZ / rows || rows * cols != n / 2) return -1;
  uint16_t *words = load_words(data, n), *tiled = (uint16_t *)malloc(n ? n : 2);
  block_t b = {0};
  int rc = -1;
  if (!words || !tiled) goto done;
  if (transform(words, rows, cols, 16, 16, 0, tiled)) goto done;
  if (encode_bf16(tiled, n / 2, &b)) goto done;
  {
    size_t size = segment_size(&b);
    uint8_t *v = (uint8_t *)malloc(size ? size : 1);
    if (!v) goto done;
    write_segment(v, &b);
    *out = v;
    *out_size = size;
  }
  rc = 0;
done:
  free(words); free(tiled); block_release(&b);
  return rc;
}

/* src/c_api.cpp:29-40 */
int oracle_unpack(const void *data, size_t n, size_t rows, size_t cols, void **out, size_t *out_size) {
  if (n < 272 || !rows || cols > MAXSZ / rows) return -1;
  const uint8_t *p = (const uint8_t *)data;
  uint64_t count = get64(p), bits = get64(p + 8);
  if (count != rows * cols || count > n - 272 || bits / 8 + (bits % 8 != 0) != n - 272 - count) return -1;
  block_t b = {0};
  b.count = count; b.bit_count = bits;
  memcpy(b.lengths, p + 16, 256);
  b.sign_mantissa = (uint8_t *)(p + 272);
  b.exponents = (uint8_t *)(p + 272 + count);
  b.exp_size = n - 272 - (size_t)count;
  uint16_t *decoded = (uint16_t *)malloc(count ? count * 2 : 2), *words = (uint16_t *)malloc(count ? count * 2 : 2);
  int rc = -1;
  if (!decoded || !words) goto done;
  if (decode_bf16(&b, decoded)) goto done;
  if (transform(decoded, rows, cols, 16, 16, 1, words)) goto done;
  rc = emit_words(words, (size_t)count, out, out_size);
done:
  free(decoded); free(words);
  return rc;
}

/* src/c_api.cpp:44-65 */
int oracle_pack_parallel(const void *data, size_t n, size_t rows, size_t cols, void **out, size_t *out_size) {
  if (n % 2 || !rows || rows > 16 || !cols || cols > MAXSZ / rows || rows * cols != n / 2 ||
      rows * cols > MAXSZ / 32)
    return -1;
  size_t total = n / 2;
  uint16_t *words = load_words(data, n), *packed = (uint16_t *)malloc(n ? n : 2);
  block_t b[32];
  size_t chunks = total < 32 ? total : 32, made = 0;
  int rc = -1;
  memset(b, 0, sizeof b);
  if (!words || !packed) goto done;
  if (transform(words, rows, cols, 16, 16, 0, packed)) goto done;
  for (; made < chunks; ++made) {
    size_t start = total * made / chunks, end = total * (made + 1) / chunks;
    if (encode_bf16(packed + start, end - start, &b[made])) goto done;
  }
  {
    size_t size = 32 + 8 * chunks;
    for (size_t i = 0; i < chunks; ++i) size += segment_size(&b[i]);
    uint8_t *v = (uint8_t *)malloc(size);
    if (!v) goto done;
    memcpy(v, "XKSP2\0\0\0", 8);
    put64(v + 8, rows); put64(v + 16, cols); put64(v + 24, chunks);
    size_t pos = 32 + 8 * chunks;
    for (size_t i = 0; i < chunks; ++i) {
      put64(v + 32 + 8 * i, segment_size(&b[i]));
      write_segment(v + pos, &b[i]);
      pos += segment_size(&b[i]);
    }
    *out = v;
    *out_size = size;
  }
  rc = 0;
done:
  for (size_t i = 0; i < made && i < 32; ++i) block_release(&b[i]);
  free(words); free(packed);
  return rc;
}

/* src/c_api.cpp:66-85 */
int oracle_unpack_parallel(const void *data, size_t n, void **out, size_t *out_size) {
  const uint8_t *p = (const uint8_t *)data;
  if (n < 32 || memcmp(p, "XKSP2\0\0\0", 8)) return -1;
  uint64_t rows = get64(p + 8), cols = get64(p + 16), chunks = get64(p + 24);
  if (!rows || rows > 16 || !cols || !chunks || chunks > 32 || cols > MAXSZ / rows ||
      chunks > rows * cols || rows * cols > n || rows * cols > MAXSZ / 32 || n < 32 + 8 * chunks)
    return -1;
  size_t total = (size_t)(rows * cols), pos = 32 + 8 * (size_t)chunks, filled = 0;
  uint16_t *packed = (uint16_t *)malloc(total * 2), *words = (uint16_t *)malloc(total * 2);
  int rc = -1;
  if (!packed || !words) goto done;
  for (size_t i = 0; i < chunks; ++i) {
    uint64_t length = get64(p + 32 + 8 * i);
    if (length < 272 || length > n - pos) goto done;
    uint64_t count = get64(p + pos), bits = get64(p + pos + 8);
    if (count != (total * (i + 1) / chunks) - (total * i / chunks) || count > length - 272 ||
        bits / 8 + (bits % 8 != 0) != length - 272 - count)
      goto done;
    block_t b = {0};
    b.count = count; b.bit_count = bits;
    memcpy(b.lengths, p + pos + 16, 256);
    b.sign_mantissa = (uint8_t *)(p + pos + 272);
    b.exponents = (uint8_t *)(p + pos + 272 + count);
    b.exp_size = (size_t)(length - 272 - count);
    if (decode_bf16(&b, packed + filled)) goto done;
    filled += (size_t)count;
    pos += (size_t)length;
  }
  if (pos != n) goto done;
  if (transform(packed, (size_t)rows, (size_t)cols, 16, 16, 1, words)) goto done;
  rc = emit_words(words, total, out, out_size);
done:
  free(packed); free(words);
  return rc;
}

/* ---------------------------------------------------------- fp64 reference */

/* Y[r*batch + k] = sum_c bf16(W[r*cols + c]) * X[c*batch + k], accumulated
 * in double.  Layout follows cuda/decode.cu:94 (X [cols, batch], Y
 * [rows, batch], row-major).  bf16 -> value is bits << 16 reinterpreted as
 * fp32 (cuda/decode.cu:42). */
void oracle_gemm_f64(const uint16_t *w, size_t rows, size_t cols, const double *x, size_t batch, double *y) {
  for (size_t r = 0; r < rows; ++r)
    for (size_t k = 0; k < batch; ++k) {
      double acc = 0.0;
      for (size_t c = 0; c < cols; ++c) {
        uint32_t bits = (uint32_t)w[r * cols + c] << 16;
        float f;
        memcpy(&f, &bits, 4);
        acc += (double)f * x[c * batch + k];
      }
      y[r * batch + k] = acc;
    }
}
