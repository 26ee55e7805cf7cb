/*
 * Test oracle (CPU, plain C): a restatement of the reference NF4 codec, used
 * only by tests/, the smoke check and the benchmark's CPU baseline. Never
 * linked into or called by the product library.
 *
 *   nf4o_decode  restates nf4_dequant_torch (selas/codecs.py:178-199):
 *                out = round(code[nibble] * absmax[block]) in fp32, then one
 *                rounding to the output type, element 2i from the high nibble.
 *   nf4o_encode  restates encode_nf4 (selas/codecs.py:99-119): block absmax,
 *                x / absmax (absmax 0 -> 1), torch.bucketize(x, mids,
 *                right=False) = number of midpoints that are not >= x,
 *                mids = (code[i+1] + code[i]) / 2 in fp32.
 *
 * Output types: 0 = fp32, 1 = fp16 (IEEE round to nearest even), 2 = bf16
 * (round to nearest even; NaN -> 0x7FC0).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

uint16_t nf4o_bf16_bits(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* IEEE binary32 -> binary16, round to nearest even, written from the format
 * definitions: normal numbers keep 10 mantissa bits, numbers below 2^-14 become
 * subnormals (multiples of 2^-24), magnitudes rounding to >= 65520 overflow. */
uint16_t nf4o_f16_bits(float f) {
  uint32_t u = f2u(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x1ffu));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                                    /* below 2^-14: subnormal or zero */
    /* value = a_float; result = round(a_float / 2^-24) as integer, ties to even */
    uint32_t exp = a >> 23;
    if (exp < 102) return sign; /* below 2^-25: rounds to zero (2^-25 itself ties to 0) */
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126 - exp; /* value = mant * 2^(exp-150) -> units of 2^-24: mant >> (126-exp) */
    uint32_t q = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1;
    return (uint16_t)(sign | q);
  }
  /* normal: rebias exponent 127 -> 15, keep 10 of 23 mantissa bits */
  uint32_t r = a - 0x38000000u; /* (exp - 112) << 23 | mant */
  uint32_t q = r >> 13;
  uint32_t rem = r & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1;
  return (uint16_t)(sign | q);
}

void nf4o_decode(const uint8_t *packed, const float *absmax, int64_t n_bytes, int64_t blocksize, const float *code,
                 void *out, int out_dtype) {
  const int64_t bpb = blocksize / 2;
  for (int64_t i = 0; i < n_bytes; ++i) {
    const float a = absmax[i / bpb];
    const float hi = code[packed[i] >> 4] * a;
    const float lo = code[packed[i] & 15] * a;
    if (out_dtype == 0) {
      ((float *)out)[2 * i] = hi;
      ((float *)out)[2 * i + 1] = lo;
    } else if (out_dtype == 1) {
      ((uint16_t *)out)[2 * i] = nf4o_f16_bits(hi);
      ((uint16_t *)out)[2 * i + 1] = nf4o_f16_bits(lo);
    } else {
      ((uint16_t *)out)[2 * i] = nf4o_bf16_bits(hi);
      ((uint16_t *)out)[2 * i + 1] = nf4o_bf16_bits(lo);
    }
  }
}

int nf4o_encode(const float *w, int64_t n, int64_t blocksize, const float *code, uint8_t *packed, float *absmax) {
  if (blocksize <= 0 || blocksize % 2 || n % blocksize) return 1;
  float mids[15];
  for (int i = 0; i < 15; ++i) mids[i] = (code[i + 1] + code[i]) / 2.0f;
  for (int64_t b = 0; b < n / blocksize; ++b) {
    const float *src = w + b * blocksize;
    float m = 0.0f;
    int nan = 0;
    for (int64_t j = 0; j < blocksize; ++j) {
      const float v = fabsf(src[j]);
      if (v != v) nan = 1;
      else if (v > m) m = v;
    }
    if (nan) m = NAN;
    absmax[b] = m;
    const float safe = m > 0.0f ? m : 1.0f;
    for (int64_t j = 0; j < blocksize; j += 2) {
      unsigned idx[2];
      for (int t = 0; t < 2; ++t) {
        const float x = src[j + t] / safe;
        unsigned c = 0;
        for (int q = 0; q < 15; ++q) c += !(mids[q] >= x);
        idx[t] = c;
      }
      packed[(b * blocksize + j) / 2] = (uint8_t)((idx[0] << 4) | idx[1]);
    }
  }
  return 0;
}
