// Device helpers shared by the quantize kernels (element conversions,
// cross-lane maxima, streaming loads and stores).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fp8_math.h"

using namespace pfp8;

// --------------------------------------------------------------------------
// Element conversion helpers (4 values -> 4 packed e4m3fn bytes)
// --------------------------------------------------------------------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef short short2_t __attribute__((ext_vector_type(2)));

// t[i] finite.  Software path: bf16 RNE by integer rounding, then e4m3fn.
__device__ __forceinline__ uint32_t cvt4_sw(float t0, float t1, float t2, float t3) {
  uint32_t c0 = bf16_to_e4m3fn(f32_to_bf16_rne_nonan(t0));
  uint32_t c1 = bf16_to_e4m3fn(f32_to_bf16_rne_nonan(t1));
  uint32_t c2 = bf16_to_e4m3fn(f32_to_bf16_rne_nonan(t2));
  uint32_t c3 = bf16_to_e4m3fn(f32_to_bf16_rne_nonan(t3));
  return c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
}

// t[i] finite.  gfx950 path: v_cvt_pk_bf16_f32 (RNE) then
// v_cvt_scalef32_pk_fp8_bf16 with scale 1.0.
__device__ __forceinline__ uint32_t cvt4_hw(float t0, float t1, float t2, float t3) {
  bf16x2_t lo = {(__bf16)t0, (__bf16)t1};
  bf16x2_t hi = {(__bf16)t2, (__bf16)t3};
  short2_t r = {0, 0};
  r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r, lo, 1.0f, false);
  r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r, hi, 1.0f, true);
  return __builtin_bit_cast(uint32_t, r);
}

template <bool HW>
__device__ __forceinline__ uint32_t cvt4(float t0, float t1, float t2, float t3) {
  if constexpr (HW) return cvt4_hw(t0, t1, t2, t3);
  else return cvt4_sw(t0, t1, t2, t3);
}

// Exact composition for 4 elements (any inputs, NaN/inf/overflow included).
__device__ __forceinline__ uint32_t cvt4_exact(float x0, float x1, float x2, float x3, float S) {
  return quant_elem_exact(x0, S) | (quant_elem_exact(x1, S) << 8) |
         (quant_elem_exact(x2, S) << 16) | (quant_elem_exact(x3, S) << 24);
}

// Distance of the low 16 bits of t from the bf16 rounding midpoint is <= 4.
__device__ __forceinline__ bool near_bf16_midpoint(float t) {
  return ((f2u(t) + 4u - 0x8000u) & 0xFFFFu) <= 8u;
}

__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t umin(uint32_t a, uint32_t b) { return a < b ? a : b; }

__device__ __forceinline__ uint32_t shfl_xor_u32(uint32_t v, int m) {
  return (uint32_t)__shfl_xor((int)v, m, 64);
}

// Widen the i-th element of a 16-byte vector to f32.
template <bool IS_BF16>
__device__ __forceinline__ float elem_f32(const uint4& v, int i) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  if constexpr (IS_BF16) {
    uint32_t word = w[i >> 1];
    return u2f((i & 1) ? (word & 0xFFFF0000u) : (word << 16));
  } else {
    return u2f(w[i]);
  }
}

// max |x| bits (as f32 bits) over the 16 bytes of v.
template <bool IS_BF16>
__device__ __forceinline__ uint32_t vec_absmax_bits(const uint4& v) {
  if constexpr (IS_BF16) {
    uint32_t m01 = umax(v.x & 0x7FFFu, (v.x >> 16) & 0x7FFFu);
    uint32_t m23 = umax(v.y & 0x7FFFu, (v.y >> 16) & 0x7FFFu);
    uint32_t m45 = umax(v.z & 0x7FFFu, (v.z >> 16) & 0x7FFFu);
    uint32_t m67 = umax(v.w & 0x7FFFu, (v.w >> 16) & 0x7FFFu);
    return umax(umax(m01, m23), umax(m45, m67)) << 16;
  } else {
    return umax(umax(v.x & 0x7FFFFFFFu, v.y & 0x7FFFFFFFu),
                umax(v.z & 0x7FFFFFFFu, v.w & 0x7FFFFFFFu));
  }
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v) {
  // bound_ctrl: lanes without a source read 0, the identity of unsigned max,
  // which lets the compiler fuse the move into v_max_u32_dpp.
  return umax(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true));
}

// Max with the lane X = 16 or 32 positions away (lane ^ X), by gfx950's row
// swaps: v_permlane16_swap exchanges the odd 16-lane rows of one register with
// the even rows of the other, v_permlane32_swap the upper half of one with the
// lower half of the other; with the same value in both, the two results hold
// each lane's own value and its partner's, in some order.  VALU operations,
// where a __shfl_xor is an LDS permute with its latency.
template <int X>
__device__ __forceinline__ uint32_t xor_max_u32(uint32_t v) {
  static_assert(X == 16 || X == 32, "row swaps exchange 16 or 32 lanes");
  if constexpr (X == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return umax(p[0], p[1]);
  } else {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return umax(p[0], p[1]);
  }
}

// Max over aligned groups of BL lanes; every lane of the group gets the result.
template <int BL>
__device__ __forceinline__ uint32_t lane_group_max(uint32_t v) {
  if constexpr (BL >= 2) v = dpp_max_u32<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (BL >= 4) v = dpp_max_u32<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (BL >= 8) v = dpp_max_u32<0x141>(v);  // row_half_mirror
  if constexpr (BL >= 16) v = dpp_max_u32<0x140>(v); // row_mirror
  if constexpr (BL >= 32) v = xor_max_u32<16>(v);
  if constexpr (BL >= 64) v = xor_max_u32<32>(v);
  return v;
}

// Max over the 64 / W lanes that share lane % W (W = 4 or 8), for every lane:
// within each 16-lane row by DPP row rotations (by 4 and 8 lanes: together
// they reach the row's lanes of the same residue), across rows by the swaps.
template <int W>
__device__ __forceinline__ uint32_t strided_lane_max(uint32_t v) {
  static_assert(W == 4 || W == 8, "lane stride 4 or 8");
  if constexpr (W == 4) v = dpp_max_u32<0x124>(v);   // row_ror:4
  v = dpp_max_u32<0x128>(v);                          // row_ror:8
  v = xor_max_u32<16>(v);
  return xor_max_u32<32>(v);
}

__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}

// Raw buffer resources for stores issued by every lane of a wave with the
// lanes that should not store given an offset past the end (the range check
// drops them): a store count that does not depend on a branch lets a wait for
// later loads leave the stores in flight.
constexpr int kRawBuffer = 0x00020000;            // raw buffer resource, 32-bit data format
constexpr int kOutOfRange = (int)0xFFFFFFF0u;     // buffer offset past any scale array

// 16-byte streaming load: the input is read exactly once, so it is loaded
// non-temporally (measured ~12% more HBM throughput than a plain load here).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream16(const char* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

#ifndef PRATCHYA_NT_STORE
#define PRATCHYA_NT_STORE 1
#endif
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void store_stream8(uint8_t* p, u32x2_t w) {
  if (PRATCHYA_NT_STORE) __builtin_nontemporal_store(w, reinterpret_cast<u32x2_t*>(p));
  else *reinterpret_cast<u32x2_t*>(p) = w;
}
__device__ __forceinline__ void store_stream16(void* p, u32x4_t w) {
  if (PRATCHYA_NT_STORE) __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
  else *reinterpret_cast<u32x4_t*>(p) = w;
}
__device__ __forceinline__ void store_stream4(uint8_t* p, uint32_t w) {
  if (PRATCHYA_NT_STORE) __builtin_nontemporal_store(w, reinterpret_cast<uint32_t*>(p));
  else *reinterpret_cast<uint32_t*>(p) = w;
}

// Two e4m3fn bytes of a word (bytes 0,1 or 2,3) -> f32, with gfx950's
// v_cvt_scalef32_pk_f32_fp8 at scale 1.0 (OCP e4m3fn; exact for every byte,
// which the tests check byte by byte).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <int HALF>
__device__ __forceinline__ f32x2_t fp8_pair(uint32_t word) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(word, 1.0f, HALF != 0);
}

template <int J>
__device__ __forceinline__ float fp8_elem(uint32_t word) {
  const f32x2_t p = fp8_pair<(J >> 1) & 1>(word);
  return (J & 1) ? p.y : p.x;
}

// Four e4m3fn bytes of a word -> f32, in byte order.
__device__ __forceinline__ void fp8_word(uint32_t word, float& v0, float& v1, float& v2, float& v3) {
  const f32x2_t lo = fp8_pair<0>(word), hi = fp8_pair<1>(word);
  v0 = lo.x; v1 = lo.y; v2 = hi.x; v3 = hi.y;
}

// Two f32 -> packed bf16 bits (v_cvt_pk_bf16_f32, RNE; NaN stays NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const bf16x2_t p = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, p);
}

// max |x| (as f32 bits) of 8 packed bf16 values, on packed 16-bit lanes.
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t absmax8_bf16(const uint4& v) {
  const u16x2_t a = __builtin_bit_cast(u16x2_t, v.x & 0x7FFF7FFFu);
  const u16x2_t b = __builtin_bit_cast(u16x2_t, v.y & 0x7FFF7FFFu);
  const u16x2_t c = __builtin_bit_cast(u16x2_t, v.z & 0x7FFF7FFFu);
  const u16x2_t d = __builtin_bit_cast(u16x2_t, v.w & 0x7FFF7FFFu);
  const u16x2_t m = __builtin_elementwise_max(__builtin_elementwise_max(a, b),
                                              __builtin_elementwise_max(c, d));
  return (uint32_t)(m.x > m.y ? m.x : m.y) << 16;
}

// f32(128 / 1e-7f) rounded to nearest: the y of a clamped block.
#define PRATCHYA_Y_CLAMP 1.28e9f

// Near a bf16 rounding midpoint: the low 16 bits within 8 of 0x8000, i.e.
// (bits + 0x8008) mod 2^16 <= 16.  mid_key moves those 16 bits to the top
// (one add-and-shift), so that t is near iff mid_key(t) <= kMidKey and the
// minimum of several keys tests them all with one compare.
constexpr uint32_t kMidKey = 16u << 16;
__device__ __forceinline__ uint32_t mid_key(float t) { return (f2u(t) + 0x8008u) << 16; }
__device__ __forceinline__ uint32_t mid_key4(float t0, float t1, float t2, float t3) {
  const uint32_t a = mid_key(t0), b = mid_key(t1), c = mid_key(t2), d = mid_key(t3);
  const uint32_t ab = a < b ? a : b, cd = c < d ? c : d;
  return ab < cd ? ab : cd;
}

// Scales of one block for the division-free cast (the arithmetic of
// k_quant_g8's finite-G path): mb = the block's max |x| bits, Gb = the group's
// (finite), rcpG128 = rcp(G / 128).  e: the e8m0 byte (exponent difference,
// exact; e8m0_of where it does not apply: subnormal or zero maxima, r < 2^-126);
// y: 128 / S to within a few ulp (t = x * y then lies within a few ulp of
// RN(x / S) * 128, so a t that is not near a bf16 rounding midpoint rounds as
// the reference's quotient does); clamped: S is the 1e-7 clamp.
struct BlockScale {
  uint32_t e;
  float y;
  bool clamped;
};
__device__ __forceinline__ BlockScale block_scale(uint32_t mb, uint32_t Gb, float rcpG128) {
  const float G = u2f(Gb);
  const uint32_t EG = Gb >> 23, fG = Gb & 0x7FFFFFu;
  const uint32_t Em = mb >> 23, fm = mb & 0x7FFFFFu;
  const int ef = (int)Em - (int)EG + 127 - (fm < fG ? 1 : 0);
  uint32_t er = (uint32_t)ef;
  if (!(EG >= 1u && Em >= 1u && ef >= 1)) er = mb == 0u ? 0u : e8m0_of(u2f(mb), G);
  const float sG = e8m0_decode(er) * G;
  const bool cl = !(sG >= kClamp);
  return {er, cl ? PRATCHYA_Y_CLAMP : u2f((254u - er) << 23) * rcpG128, cl};
}

// Fake quantization of 4 f32 values of one block, quantize_impl then
// dequantize_impl (Q:484-499, Q:562-564): the e4m3fn payload word of
// (x0..x3), dequantized as (f32(q) * dq) / 128 (dq = 2^(e-127) * G, or the
// repaired scale of quantize_impl_bwd).  finite (G finite): the division-free
// cast with y from block_scale, a word with a value near a bf16 rounding
// midpoint (the mid_key test, as one compare of the smallest key)
// redone exactly; otherwise the exact composition.  S = quant_scale(e, G).
// dqx = dq / 128 when one_mul (see dequant_one_mul), else dq.
__device__ __forceinline__ void fake_quant4(float& x0, float& x1, float& x2, float& x3, float y, float S,
                                            bool finite, float dqx, bool one_mul) {
  uint32_t w;
  if (finite) {
    const float t0 = x0 * y, t1 = x1 * y, t2 = x2 * y, t3 = x3 * y;
    w = cvt4_hw(t0, t1, t2, t3);
    if (mid_key4(t0, t1, t2, t3) <= kMidKey) w = cvt4_exact(x0, x1, x2, x3, S);
  } else {
    w = cvt4_exact(x0, x1, x2, x3, S);
  }
  fp8_word(w, x0, x1, x2, x3);
  if (one_mul) {
    x0 *= dqx;
    x1 *= dqx;
    x2 *= dqx;
    x3 *= dqx;
  } else {
    x0 = (x0 * dqx) * 0.0078125f;
    x1 = (x1 * dqx) * 0.0078125f;
    x2 = (x2 * dqx) * 0.0078125f;
    x3 = (x3 * dqx) * 0.0078125f;
  }
}

// Fake quantization of one value with tgrid (1, 1), quantize_impl then
// dequantize_impl (Q:484-499, Q:562-564): the value is its own block and
// group, so G = |c|, r = |c| / G = 1 and e = 127 for a finite nonzero c (0
// for a zero, 255 for NaN / inf: r is NaN).  Where 1e-7 <= |c| < 2^121, S =
// |c|, c / S * 128 = +-128 exactly (payload +-128) and (128 |c|) / 128 = c;
// a zero stays itself (payload +-0, dequant scale 0).  Elsewhere the
// composition's closed forms: NaN / inf (r NaN, so e = 255 and S is NaN or
// inf): the payload and the value are NaN; 2^121 <= |c| < inf: the payload is
// +-128 and 128 |c| overflows, so +-inf; 0 < |c| < 1e-7: S = 1e-7, the payload
// e4m3fn(bf16(c / S * 128)) (IEEE division; the hardware conversions are exact
// for these finite values), dequantized as (f32(q) * |c|) / 128.  Returns the
// dequantized f32 value; e: the e8m0 byte.
constexpr uint32_t kClampBits = __builtin_bit_cast(uint32_t, kClamp);
__device__ __forceinline__ float fake_quant11(float c, uint32_t& e) {
  const uint32_t a = abs_bits(c);
  e = a == 0u ? 0u : 127u;
  if (a - kClampBits < 0x7C000000u - kClampBits || a == 0u) return c;
  if (a >= 0x7F800000u) {
    e = 255u;
    return __builtin_nanf("");
  }
  if (a >= 0x7C000000u) return u2f((f2u(c) & 0x80000000u) | 0x7F800000u);
  const uint32_t w = cvt4_hw((c / kClamp) * 128.0f, 0.0f, 0.0f, 0.0f);
  return (fp8_elem<0>(w) * u2f(a)) * 0.0078125f;
}

// quantize_impl with tgrid (1, 1) for one value (its own block and group, G
// = |c|): the payload byte and the e8m0 byte.  A finite c with |c| >= 1e-7
// quantizes to +-128 (0x70 | sign), a zero to +-0; the 1e-7 clamp, NaN and
// inf take the exact composition.
__device__ __forceinline__ uint32_t quant11(float c, uint32_t& e) {
  const uint32_t a = abs_bits(c);
  const uint32_t sign = (f2u(c) >> 24) & 0x80u;
  e = a == 0u ? 0u : 127u;
  if (a - kClampBits < 0x7F800000u - kClampBits) return 0x70u | sign;
  if (a == 0u) return sign;
  if (a >= 0x7F800000u) e = 255u;
  return quant_elem_exact(c, quant_scale(e, u2f(a)));
}

// (f32(q) * dq) / 128 equals f32(q) * (dq / 128) for every e4m3fn q when
// 2^-110 <= dq < 2^118: dq / 128 is exact, no product of a nonzero q
// (2^-9 <= |q| <= 448) is subnormal or overflows in either order, and scaling
// by 2^-7 commutes with rounding for normal results (NaN and zero q agree).
__device__ __forceinline__ bool dequant_one_mul(float dq) {
  return dq >= 0x1p-110f && dq < 0x1p118f;
}

// --------------------------------------------------------------------------
// Kernels shared by the general (multi-launch) quantize paths: workspace
// fill, and the per-group scales from the block maxima in the workspace
// (f32 bit patterns of max |x|, one per block).  Internal linkage: each
// translation unit that launches them has its own copy.
// --------------------------------------------------------------------------
static __global__ void k_fill_u32(uint32_t* __restrict__ p, int64_t n, uint32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = v;
}

// Group max and e8m0 bytes: one wave per group.
static __global__ __launch_bounds__(256) void k_group_scales(const uint32_t* __restrict__ ws,
                                                             uint8_t* __restrict__ sc8,
                                                             float* __restrict__ sc32, int64_t n_groups,
                                                             int64_t K) {
  const int lane = threadIdx.x & 63;
  const int64_t g = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (g >= n_groups) return;
  const uint32_t* m = ws + g * K;
  uint32_t G = 0;
  for (int64_t k = lane; k < K; k += 64) G = umax(G, m[k]);
  for (int s = 1; s < 64; s <<= 1) G = umax(G, shfl_xor_u32(G, s));
  const float Gf = u2f(G);
  for (int64_t k = lane; k < K; k += 64) sc8[g * K + k] = (uint8_t)e8m0_of(u2f(m[k]), Gf);
  if (lane == 0) sc32[g] = Gf;
}

// Group max and e8m0 bytes: one thread per group (small K).
static __global__ __launch_bounds__(256) void k_group_scales_small(const uint32_t* __restrict__ ws,
                                                                   uint8_t* __restrict__ sc8,
                                                                   float* __restrict__ sc32,
                                                                   int64_t n_groups, int64_t K) {
  const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= n_groups) return;
  const uint32_t* m = ws + g * K;
  uint32_t G = 0;
  for (int64_t k = 0; k < K; ++k) G = umax(G, m[k]);
  const float Gf = u2f(G);
  for (int64_t k = 0; k < K; ++k) sc8[g * K + k] = (uint8_t)e8m0_of(u2f(m[k]), Gf);
  sc32[g] = Gf;
}
