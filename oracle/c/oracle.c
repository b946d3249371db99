/*
 * C restatement of the byte/integer parts of the reference decoder-step path -- TEST
 * INFRASTRUCTURE ONLY (loaded by tests/ through oracle/c_oracle.py, never by edgerag_amd).
 *
 * A second, independent restatement next to the torch-CPU oracle: plain loops, no torch
 * semantics borrowed, so the two cross-check each other.
 *   slot scatter      edgerag/cache/paged.py:186-206 (pool[:, table[p//bs], p%bs] = src)
 *   gather            edgerag/cache/paged.py:229-238
 *   quantize          edgerag/core/quant.py:85-95 (fp32 amax/qmax, rint half-even, clamp)
 *   fp32 -> fp16      torch's .half() (round to nearest even), written from the IEEE-754 format
 *   pack/unpack int4  edgerag/core/quant.py:110-138
 * Built with -ffp-contract=off and without fast-math, so every division and rounding is the
 * IEEE-754 default.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* Scatter (1, H, T, D) source rows into a head-major (H, NB, BS, D) pool, byte-wise. */
int oracle_slot_scatter(uint8_t* pool, int elem_bytes, int H, int NB, int BS, int D,
                        const uint8_t* src, int T, const int32_t* blocks, int n_blocks,
                        int start) {
  const size_t row = (size_t)D * elem_bytes;
  for (int t = 0; t < T; ++t) {
    const int pos = start + t;
    const int logical = pos / BS, off = pos % BS;
    if (logical >= n_blocks) return -1;
    const int blk = blocks[logical];
    if (blk < 0 || blk >= NB) return -2;
    for (int h = 0; h < H; ++h) {
      uint8_t* dst = pool + (((size_t)h * NB + blk) * BS + off) * row;
      const uint8_t* s = src + ((size_t)h * T + t) * row;
      memcpy(dst, s, row);
    }
  }
  return 0;
}

/* out (H, L, D) = pool rows of positions [0, L). */
int oracle_gather(const uint8_t* pool, int elem_bytes, int H, int NB, int BS, int D,
                  const int32_t* blocks, int n_blocks, int L, uint8_t* out) {
  const size_t row = (size_t)D * elem_bytes;
  for (int h = 0; h < H; ++h) {
    for (int p = 0; p < L; ++p) {
      const int logical = p / BS;
      if (logical >= n_blocks) return -1;
      const int blk = blocks[logical];
      if (blk < 0 || blk >= NB) return -2;
      memcpy(out + ((size_t)h * L + p) * row, pool + (((size_t)h * NB + blk) * BS + p % BS) * row,
             row);
    }
  }
  return 0;
}

/* IEEE-754 binary32 -> binary16, round to nearest, ties to even. */
uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const int32_t exp = (int32_t)((x >> 23) & 0xff);
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0)); /* inf / nan */
  int32_t e = exp - 127 + 15;
  if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);                      /* overflow -> inf */
  if (e <= 0) {                                                            /* subnormal half */
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const int shift = 14 - e;
    uint32_t half = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1);
    const uint32_t mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1u))) ++half;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) ++half; /* may carry into the exponent */
  return (uint16_t)(sign | half);
}

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ffu;
  float v;
  if (exp == 0) {
    v = ldexpf((float)man, -24);
  } else if (exp == 0x1f) {
    v = man ? NAN : INFINITY;
  } else {
    v = ldexpf((float)(man | 0x400u), (int)exp - 25);
  }
  uint32_t bits;
  memcpy(&bits, &v, 4);
  bits |= sign;
  memcpy(&v, &bits, 4);
  return v;
}

/* Group-wise symmetric quantisation of w (n, k) along k. codes (n, k) int8, scales (n, k/g) as
 * fp16 bit patterns. Returns 0, or -1 for a ragged group. */
int oracle_quantize(const float* w, int n, int k, int g, int bits, int8_t* codes,
                    uint16_t* scales_f16) {
  if (g <= 0 || k % g) return -1;
  const float qmax = bits == 4 ? 7.0f : 127.0f;
  const int groups = k / g;
  for (int r = 0; r < n; ++r) {
    for (int gi = 0; gi < groups; ++gi) {
      const float* src = w + (size_t)r * k + (size_t)gi * g;
      float amax = 0.0f;
      for (int i = 0; i < g; ++i) {
        const float a = fabsf(src[i]);
        if (a > amax) amax = a;
      }
      const float scale = amax > 0.0f ? amax / qmax : 1.0f;
      scales_f16[(size_t)r * groups + gi] = oracle_f32_to_f16(scale);
      for (int i = 0; i < g; ++i) {
        float c = rintf(src[i] / scale); /* default rounding mode: nearest, ties to even */
        if (c > qmax) c = qmax;
        if (c < -qmax) c = -qmax;
        codes[(size_t)r * k + (size_t)gi * g + i] = (int8_t)c;
      }
    }
  }
  return 0;
}

void oracle_pack_int4(const int8_t* codes, int n, int k, uint8_t* out) {
  for (int r = 0; r < n; ++r)
    for (int j = 0; j < k / 2; ++j) {
      int lo = codes[(size_t)r * k + 2 * j] + 8, hi = codes[(size_t)r * k + 2 * j + 1] + 8;
      lo = lo < 0 ? 0 : lo > 15 ? 15 : lo;
      hi = hi < 0 ? 0 : hi > 15 ? 15 : hi;
      out[(size_t)r * (k / 2) + j] = (uint8_t)(lo | (hi << 4));
    }
}

void oracle_unpack_int4(const uint8_t* packed, int n, int k, int8_t* codes) {
  for (int r = 0; r < n; ++r)
    for (int j = 0; j < k / 2; ++j) {
      const uint8_t b = packed[(size_t)r * (k / 2) + j];
      codes[(size_t)r * k + 2 * j] = (int8_t)((b & 15) - 8);
      codes[(size_t)r * k + 2 * j + 1] = (int8_t)((b >> 4) - 8);
    }
}

/* fp16 weight (n, k) bit patterns: fp16(code) * fp16(scale), the product rounded once. */
void oracle_dequantize(const int8_t* codes, const uint16_t* scales_f16, int n, int k, int g,
                       uint16_t* out) {
  const int groups = k / g;
  for (int r = 0; r < n; ++r)
    for (int i = 0; i < k; ++i) {
      const float s = oracle_f16_to_f32(scales_f16[(size_t)r * groups + i / g]);
      out[(size_t)r * k + i] = oracle_f32_to_f16((float)codes[(size_t)r * k + i] * s);
    }
}
