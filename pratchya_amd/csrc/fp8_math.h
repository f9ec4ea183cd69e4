// Scalar arithmetic of pratchya's FP8 block format, shared by the gfx950
// kernels (host-callable as well, so the same definitions compile on both sides).
//
// Format (pratchya/_qualia/_qarr.py:484-499, quantize_impl):
//   m  = max|x| of an a x b block;  G = max m over K consecutive blocks
//   r  = m / (G == 0 ? 1 : G)                 IEEE f32 division
//   e  = (bits(r) >> 23) & 0xFF               e8m0 byte
//   S  = max(f32(e << 23) * G, f32(1e-7))     NaN-propagating max
//   q  = e4m3fn_RNE(bf16_RNE(x / S * 128))    two roundings, non-saturating
// and the dequantized value (_qarr.py:562-564) is (f32(q) * (f32(e<<23)*G)) / 128.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define PFN __host__ __device__ __forceinline__
#else
#define PFN static inline
#endif

namespace pfp8 {

constexpr float kClamp = 1e-7f;   // f32(1e-7), _qarr.py:497

PFN uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
PFN float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

PFN bool is_nan_bits(uint32_t u) { return (u & 0x7FFFFFFFu) > 0x7F800000u; }
PFN bool is_finite_f(float f) { return (f2u(f) & 0x7F800000u) != 0x7F800000u; }

// IEEE max that returns NaN when either operand is NaN (XLA's max semantics).
PFN float max_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return a > b ? a : b;
}

// |x| bits of a float: for non-negative floats the unsigned bit order is the
// numeric order, and every NaN compares above +inf, so an unsigned max over
// |x| bits is a NaN-propagating max of |x|.
PFN uint32_t abs_bits(float f) { return f2u(f) & 0x7FFFFFFFu; }

// e8m0 decode by the reference's bit trick: e=0 -> +0.0, e=255 -> +inf.
PFN float e8m0_decode(uint32_t e) { return u2f((e & 0xFFu) << 23); }

// e8m0 byte of r = m / G (m = block max bits, G = group max bits as floats).
PFN uint32_t e8m0_of(float m, float G) {
  float safe = (G == 0.0f) ? 1.0f : G;
  float r = m / safe;
  return (f2u(r) >> 23) & 0xFFu;
}

// Effective quantization scale S of a block (_qarr.py:495-497).
PFN float quant_scale(uint32_t e, float G) {
  float s = e8m0_decode(e) * G;
  return (s != s) ? s : (s > kClamp ? s : kClamp);
}

// f32 -> bf16 bits, round to nearest even.  NaN -> quiet NaN with the input's
// sign (0x7FC0 | sign).
PFN uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = f2u(f);
  if (is_nan_bits(u)) return ((u >> 16) & 0x8000u) | 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// f32 -> bf16 bits for values known not to be NaN.
PFN uint32_t f32_to_bf16_rne_nonan(float f) {
  uint32_t u = f2u(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// bf16 bits -> OCP e4m3fn byte, round to nearest even, non-saturating:
// magnitudes rounding above 448, infinities and NaNs give 0x7F | sign.
PFN uint32_t bf16_to_e4m3fn(uint32_t h) {
  uint32_t sign = (h >> 8) & 0x80u;
  uint32_t mag = h & 0x7FFFu;
  uint32_t code;
  if (mag >= 0x3C80u) {                 // |v| >= 2^-6: e4m3 normal range
    code = (mag - (120u << 7) + 7u + ((mag >> 4) & 1u)) >> 4;
    code = code > 0x7Fu ? 0x7Fu : code;
  } else {                              // e4m3 subnormal: multiples of 2^-9
    float v = u2f(mag << 16) * 512.0f;  // exact: < 8 with <= 8 significant bits
    code = (uint32_t)__builtin_rintf(v);
  }
  return code | sign;
}

// Full-IEEE reference composition for one element (used by the exact path
// of the kernels): e4m3fn(bf16(x / S * 128)).
PFN uint32_t quant_elem_exact(float x, float S) {
  float q = (x / S) * 128.0f;
  return bf16_to_e4m3fn(f32_to_bf16_rne(q));
}

// e4m3fn byte -> f32 (exact).  0x7F / 0xFF -> NaN.
PFN float e4m3fn_to_f32(uint32_t q) {
  uint32_t sign = (q & 0x80u) << 24;
  uint32_t e = (q >> 3) & 0xFu;
  uint32_t m = q & 7u;
  uint32_t bits;
  if ((q & 0x7Fu) == 0x7Fu) {
    bits = 0x7FC00000u;
  } else if (e == 0) {
    // m * 2^-9, m in 0..7: exact in f32
    return u2f(sign | f2u((float)m * 0.001953125f));
  } else {
    bits = ((e + 120u) << 23) | (m << 20);
  }
  return u2f(sign | bits);
}

}  // namespace pfp8
