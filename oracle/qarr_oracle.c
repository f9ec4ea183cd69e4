/*
 * C restatement of pratchya's FP8 block quantizer / dequantizer.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ to cross-check the NumPy oracle
 * (oracle/qarr_oracle.py) byte for byte, and by bench.py as the multi-core CPU
 * baseline.  Never linked into or called by the shipped library.
 *
 * Follows pratchya/_qualia/_qarr.py quantize_impl (458-506) and
 * dequantize_impl (541-569):
 *   m  = max|x| per a x b block, G = max m over K consecutive blocks (row-major
 *        block order per [H,W] slice), NaN-propagating;
 *   r  = m / (G == 0 ? 1 : G); e = (bits(r) >> 23) & 0xFF;
 *   S  = max(f32(e << 23) * G, f32(1e-7)) (NaN-propagating);
 *   q  = e4m3fn(bf16(x / S * 128)), both RNE, e4m3fn non-saturating;
 *   y  = (f32(q) * (f32(e << 23) * G)) / 128.
 * Compiled with -ffp-contract=off so every operation rounds separately.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static int64_t gcd64(int64_t a, int64_t b) {
  while (b) { int64_t t = a % b; a = b; b = t; }
  return a;
}

/* f32 -> bf16 bits, RNE; NaN -> 0x7FC0 | sign */
static uint32_t to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) & 0x8000u) | 0x7FC0u;
  uint32_t lsb = (u >> 16) & 1u;
  return (u + 0x7FFFu + lsb) >> 16;
}

/* bf16 bits -> e4m3fn byte, RNE, overflow/inf/NaN -> 0x7F | sign.
 * Written with an explicit exponent/mantissa decomposition (a different
 * formulation from the NumPy oracle's rebias-and-shift). */
static uint32_t bf16_to_e4m3(uint32_t h) {
  uint32_t sign = (h >> 8) & 0x80u;
  uint32_t exp = (h >> 7) & 0xFFu;
  uint32_t man = h & 0x7Fu;
  if (exp == 0xFF) return 0x7Fu | sign;
  if (exp == 0 && man == 0) return sign;
  /* value = 1.man * 2^(exp-127) (or subnormal bf16: 0.man * 2^-126) */
  int e = (int)exp - 127;
  uint32_t sig = exp ? (0x80u | man) : man; /* 8-bit significand, value = sig * 2^(e-7) */
  if (!exp) e = -126;
  /* target quantum: 2^(max(e,-6) - 3) ; value/quantum = sig * 2^(e - 7 - (max(e,-6)-3)) */
  int qe = (e < -6 ? -6 : e) - 3;
  int shift = (qe) - (e - 7); /* >= 4 */
  uint32_t n;
  if (shift >= 32) {
    n = 0;
  } else {
    uint32_t fl = sig >> shift;
    uint32_t rem = sig & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    n = fl + ((rem > half || (rem == half && (fl & 1u))) ? 1u : 0u);
  }
  /* rounded value = n * 2^qe */
  if (qe == -9) {           /* subnormal range: n in 0..8 (8 -> min normal) */
    return sign | n;        /* encoding of n*2^-9 for n<=8 is n */
  }
  /* normal: n in [8, 16]; renormalise */
  int ee = qe + 3;          /* exponent of 1.xxx */
  if (n == 16) { n = 8; ee += 1; }
  int be = ee + 7;
  uint32_t code = ((uint32_t)be << 3) | (n - 8);
  if (be > 15 || code > 0x7Eu) return 0x7Fu | sign;
  return sign | code;
}

static float e4m3_to_f32(uint32_t q) {
  uint32_t s = q & 0x80u, e = (q >> 3) & 0xFu, m = q & 7u;
  float v;
  if ((q & 0x7Fu) == 0x7Fu) v = NAN;
  else if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf(1.0f + (float)m / 8.0f, (int)e - 7);
  return s ? -v : v;
}

static inline float nanmax(float a, float b) {
  if (isnan(a)) return a;
  if (isnan(b)) return b;
  return a > b ? a : b;
}

/* max |x| of block n (row-major over the block grid) of one [H,W] slice */
static float block_max(const float* xs, int64_t W, int64_t a, int64_t b, int64_t nbc, int64_t n) {
  const int64_t bi = n / nbc, bj = n % nbc;
  float m = 0.0f;
  for (int64_t i = 0; i < a; ++i)
    for (int64_t j = 0; j < b; ++j) m = nanmax(m, fabsf(xs[(bi * a + i) * W + bj * b + j]));
  return m;
}

/* Block (bi,bj) of slice s covers rows bi*a.., cols bj*b.. */
int oracle_quantize(const float* x, int64_t S, int64_t H, int64_t W, int64_t a, int64_t b,
                    uint8_t* x8, uint8_t* sc8, float* sc32) {
  if (a < 1 || b < 1 || H % a || W % b) return 1;
  const int64_t nbr = H / a, nbc = W / b, n_blk = nbr * nbc;
  int64_t tK = (a * b) / 16; if (tK < 1) tK = 1;
  const int64_t K = n_blk ? gcd64(tK, n_blk) : tK;
  const int64_t M = n_blk ? n_blk / K : 0;
  const float clamp = 1e-7f;
#pragma omp parallel for schedule(static)
  for (int64_t sg = 0; sg < S * M; ++sg) {
    const int64_t s = sg / M, g = sg % M;
    const float* xs = x + s * H * W;
    uint8_t* qs = x8 + s * H * W;
    float mk[1024];
    float Gm = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      const float m = block_max(xs, W, a, b, nbc, g * K + k);
      if (k < 1024) mk[k] = m;
      Gm = nanmax(Gm, m);
    }
    const float safe = (Gm == 0.0f) ? 1.0f : Gm;
    sc32[s * M + g] = Gm;
    for (int64_t k = 0; k < K; ++k) {
      const int64_t n = g * K + k, bi = n / nbc, bj = n % nbc;
      const float m = k < 1024 ? mk[k] : block_max(xs, W, a, b, nbc, n);
      const float r = m / safe;
      const uint32_t e = (f2u(r) >> 23) & 0xFFu;
      sc8[s * n_blk + n] = (uint8_t)e;
      float Se = u2f(e << 23) * Gm;
      if (!isnan(Se) && !(Se > clamp)) Se = clamp;
      for (int64_t i = 0; i < a; ++i)
        for (int64_t j = 0; j < b; ++j) {
          const int64_t idx = (bi * a + i) * W + bj * b + j;
          const float t1 = xs[idx] / Se;
          const float t2 = t1 * 128.0f;
          qs[idx] = (uint8_t)bf16_to_e4m3(to_bf16(t2));
        }
    }
  }
  return 0;
}

int oracle_dequantize(const uint8_t* x8, const uint8_t* sc8, const float* sc32, int64_t S,
                      int64_t H, int64_t W, int64_t a, int64_t b, float* out) {
  if (a < 1 || b < 1 || H % a || W % b) return 1;
  const int64_t nbc = W / b, n_blk = (H / a) * nbc;
  int64_t tK = (a * b) / 16; if (tK < 1) tK = 1;
  const int64_t K = n_blk ? gcd64(tK, n_blk) : tK;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < S * H; ++r) {
    const int64_t s = r / H, i = r % H;
    for (int64_t c = 0; c < W; ++c) {
      const int64_t n = (i / a) * nbc + c / b;
      const float sc = u2f((uint32_t)sc8[s * n_blk + n] << 23) * sc32[s * (n_blk / K) + n / K];
      const float p = e4m3_to_f32(x8[r * W + c]) * sc;
      out[r * W + c] = p / 128.0f;
    }
  }
  return 0;
}

/* exposed for the exhaustive conversion test */
uint32_t oracle_bf16_to_e4m3(uint32_t h) { return bf16_to_e4m3(h); }
uint32_t oracle_f32_to_bf16(float f) { return to_bf16(f); }
