// Fused arithmetic of two quantized arrays for gfx950: both operands are
// dequantized, combined in f32 and the result quantized, in one pass over
// the payloads.  This is QArrayImpl's binary operators
// (pratchya/_qualia/_qarr.py:121-261): make_elementwise_impl (:715-720)
// computes op(dequantize_impl(x, f32), dequantize_impl(y, f32)) and the
// operator wraps the f32 result as QArrayImpl(out, tgrid) (:129-130), i.e.
// quantize_impl (:458-506).  The two f32 operands and the f32 result are
// never stored.
//
// Operators, with jnp's float32 semantics:
//   add, subtract, multiply, divide  IEEE f32, round to nearest even;
//   floor_divide   jnp's float divmod (CPython's float_divmod in f32):
//                  mod = fmod(x, y), div = (x - mod) / y, and when mod != 0
//                  and sign(y) != sign(mod), div -= 1; the result is div
//                  rounded half away from zero (lax.round's default);
//   remainder      r = fmod(x, y), plus y when r != 0 and (r < 0) != (y < 0).
// Dequantization is dequantize_impl's (f32(q) * (2^(e-127) * G)) / 128.
// Products and sums are rounded one at a time (no contraction to FMA).
//
// Two paths, as for the quantizer:
//   * one pass: result grid (1, b) with b a multiple of 16 and groups of at
//     most 1024 contiguous elements.  A wave owns 1024 results (16 per lane):
//     block and group maxima by lane shuffles, e8m0 scales, payload;
//   * general (any grid, four launches): the block maxima of the results into
//     a workspace with atomics, the group scales, then a second pass that
//     recomputes the results and casts them.  The operands are read twice.
// The operands may have block grids of their own (QArrayImpl's operators on
// arrays quantized with different grids dequantize each with its own grid);
// every grid divides the slice shape.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fp8_math.h"
#include "pratchya_fp8.h"
#include "quant_device.h"

int pratchya_set_error(int code, const char* fmt, ...);

#pragma clang fp contract(off)

namespace {

// A quantized operand: payload, e8m0 block scales, f32 group maxima, and its
// block grid (a, b) with K blocks per group.
struct QOperand {
  const uint8_t* q;
  const uint8_t* s8;
  const float* s32;
  int64_t a, b, K;
  int lb, lk;            // log2 b and log2 K when a == 1 and both are powers of two, else -1
  const int64_t* rows;   // OP_GATHER: operand row of each result row (a [rows_h, W] table)
  int64_t rows_h;
};

// Internal operator: the result is the dequantized operand X read through its
// row map (an embedding lookup), Y unused.
constexpr int OP_GATHER = 100;

// Dequantization factor 2^(e-127) * G of the operand's block holding
// element (i, c) of the [rows, W] array (row-major blocks, _qarr.py:562-564).
template <typename I>
__device__ __forceinline__ float operand_scale(const QOperand& o, I i, I c, I W) {
  const I blk = (i / (I)o.a) * (W / (I)o.b) + c / (I)o.b;
  return e8m0_decode(o.s8[blk]) * o.s32[blk / (I)o.K];
}

__device__ __forceinline__ float lax_sign(float v) {
  return v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : v);   // +-0 and NaN map to themselves
}

template <int OP>
__device__ __forceinline__ float ew_apply(float x, float y) {
  if constexpr (OP == OP_GATHER) {
    return x;
  } else if constexpr (OP == PRATCHYA_OP_ADD) {
    return x + y;
  } else if constexpr (OP == PRATCHYA_OP_SUB) {
    return x - y;
  } else if constexpr (OP == PRATCHYA_OP_MUL) {
    return x * y;
  } else if constexpr (OP == PRATCHYA_OP_DIV) {
    return x / y;
  } else if constexpr (OP == PRATCHYA_OP_FLOORDIV) {
    const float mod = fmodf(x, y);
    float div = (x - mod) / y;
    if (mod != 0.0f && lax_sign(y) != lax_sign(mod)) div = div - 1.0f;
    return roundf(div);
  } else {
    const float r = fmodf(x, y);
    return (r != 0.0f && ((r < 0.0f) != (y < 0.0f))) ? r + y : r;
  }
}

// CH consecutive e4m3fn bytes at p as f32 values.  VEC: one aligned load of
// CH bytes (CH = 4, 8 or 16) and the hardware conversion.
// (16-byte chunks are streamed: loaded non-temporally, as each byte is read once.)
template <int CH, bool VEC>
__device__ __forceinline__ void load_fp8(const uint8_t* __restrict__ p, float (&v)[CH]) {
  if constexpr (VEC) {
    static_assert(CH == 4 || CH == 8 || CH == 16, "vector chunks are 4, 8 or 16 bytes");
    uint32_t w[CH / 4];
    if constexpr (CH == 16) {
      const uint4 u = load_stream16(reinterpret_cast<const char*>(p));
      w[0] = u.x; w[1] = u.y; w[2] = u.z; w[3] = u.w;
    } else if constexpr (CH == 8) {
      const uint2 u = *reinterpret_cast<const uint2*>(p);
      w[0] = u.x; w[1] = u.y;
    } else {
      w[0] = *reinterpret_cast<const uint32_t*>(p);
    }
#pragma unroll
    for (int j = 0; j < CH / 4; ++j) fp8_word(w[j], v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
  } else {
#pragma unroll
    for (int k = 0; k < CH; ++k) v[k] = e4m3fn_to_f32(p[k]);
  }
}

// Results of 16 elements from their loaded payload words and block scales.
template <int OP>
__device__ __forceinline__ void ew_words(const uint4& xw, const uint4& yw, float sx, float sy, float (&z)[16]) {
  float xv[16], yv[16];
  const uint32_t xa[4] = {xw.x, xw.y, xw.z, xw.w}, ya[4] = {yw.x, yw.y, yw.z, yw.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    fp8_word(xa[j], xv[4 * j], xv[4 * j + 1], xv[4 * j + 2], xv[4 * j + 3]);
    fp8_word(ya[j], yv[4 * j], yv[4 * j + 1], yv[4 * j + 2], yv[4 * j + 3]);
  }
  // (f32(q) * s) / 128 as one multiply by s / 128 where that is exact for
  // every payload byte (dequant_one_mul), the two-step form otherwise
  if (dequant_one_mul(sx) && dequant_one_mul(sy)) {
    const float sx7 = sx * 0.0078125f, sy7 = sy * 0.0078125f;
#pragma unroll
    for (int k = 0; k < 16; ++k) z[k] = ew_apply<OP>(xv[k] * sx7, yv[k] * sy7);
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) z[k] = ew_apply<OP>((xv[k] * sx) * 0.0078125f, (yv[k] * sy) * 0.0078125f);
  }
}

template <int OP, int CH, bool VEC>
__device__ __forceinline__ void ew_values(const QOperand& X, const QOperand& Y, float sx, float sy, size_t off,
                                          float (&z)[CH]) {
  float xv[CH], yv[CH];
  load_fp8<CH, VEC>(X.q + off, xv);
  load_fp8<CH, VEC>(Y.q + off, yv);
#pragma unroll
  for (int k = 0; k < CH; ++k) z[k] = ew_apply<OP>((xv[k] * sx) * 0.0078125f, (yv[k] * sy) * 0.0078125f);
}

// Results of CH consecutive elements (i, c .. c + CH - 1); CH divides both
// operands' block widths, so each operand has one block scale for them.
template <int OP, int CH, bool VEC, typename I>
__device__ __forceinline__ void ew_chunk(const QOperand& X, const QOperand& Y, I i, I c, I W, float (&z)[CH]) {
  if constexpr (OP == OP_GATHER) {
    // table row idx[i] (negative counts from the end, clamped: jnp's gather)
    int64_t r = X.rows[i];
    if (r < 0) r += X.rows_h;
    r = r < 0 ? 0 : (r >= X.rows_h ? X.rows_h - 1 : r);
    const float sx = operand_scale<int64_t>(X, r, (int64_t)c, (int64_t)W);
    float xv[CH];
    load_fp8<CH, VEC>(X.q + r * (int64_t)W + c, xv);
#pragma unroll
    for (int k = 0; k < CH; ++k) z[k] = (xv[k] * sx) * 0.0078125f;
  } else {
    ew_values<OP, CH, VEC>(X, Y, operand_scale<I>(X, i, c, W), operand_scale<I>(Y, i, c, W), (size_t)(i * W + c), z);
  }
}

// --------------------------------------------------------------------------
// One pass: result grid (1, b), BL = b / 16 lanes per block and GL = K * BL
// lanes per group, both powers of two <= 64.  Blocks and groups are
// contiguous runs of the flattened array (a = 1), so a wave's 1024 elements
// hold whole groups; W is a multiple of 16, so a lane's 16 elements lie in
// one row and in one block of each operand.
// --------------------------------------------------------------------------
// FLAT: both operands have a = 1 and power-of-two b and K (shifts instead of
// divisions).  BLC, GLC: BL and GL fixed at compile time (DPP lane maxima; a
// whole-wave group reads its 64 / BL block maxima with readlane), or 0 for
// the runtime values (shuffles).
template <int OP, bool FLAT, typename I, int BLC, int GLC>
__global__ __launch_bounds__(256) void k_ew_rowgroup(QOperand X, QOperand Y, uint8_t* __restrict__ q,
                                                     uint8_t* __restrict__ sc8, float* __restrict__ sc32,
                                                     int64_t n, int64_t W, int bl_log2, int gl_log2) {
  const int lane = threadIdx.x & 63;
  // Workgroups are dispatched to the 8 XCDs round-robin, and neighbouring
  // waves read and write neighbouring bytes of the same scale lines: in each
  // window of 128 workgroups XCD x takes the 16 consecutive indices
  // 16x .. 16x + 15, so each scale line passes through one L2
  int64_t wb = blockIdx.x;
  if (gridDim.x % 128 == 0) wb = (blockIdx.x & ~127u) + (blockIdx.x % 8) * 16 + (blockIdx.x % 128) / 8;
  const int64_t base = (wb * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 1024;
  if (base >= n) return;
  const int64_t off = base + (int64_t)lane * 16;
  const bool live = off < n;
  const int BL = 1 << bl_log2, GL = 1 << gl_log2;

  float z[16];
  if (live) {
    if constexpr (FLAT) {
      // all six loads in flight before the first use
      const I bx = (I)off >> X.lb, by = (I)off >> Y.lb;
      const uint4 xw = load_stream16(reinterpret_cast<const char*>(X.q + off));
      const uint4 yw = load_stream16(reinterpret_cast<const char*>(Y.q + off));
      const uint32_t ex = X.s8[bx], ey = Y.s8[by];
      const float gx = X.s32[bx >> X.lk], gy = Y.s32[by >> Y.lk];
      __builtin_amdgcn_sched_barrier(0);
      ew_words<OP>(xw, yw, e8m0_decode(ex) * gx, e8m0_decode(ey) * gy, z);
    } else {
      const I i = (I)off / (I)W, c = (I)off - i * (I)W;
      ew_chunk<OP, 16, true, I>(X, Y, i, c, (I)W, z);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) z[k] = 0.0f;
  }

  // block and group maxima (f32 bit patterns of |z|; unsigned max propagates NaN)
  uint32_t m = 0;
#pragma unroll
  for (int k = 0; k < 16; ++k) m = umax(m, abs_bits(z[k]));
  uint32_t g;
  if constexpr (BLC > 0) {
    m = lane_group_max<BLC>(m);
    if constexpr (GLC == 64) {
      g = 0;
#pragma unroll
      for (int k = 0; k < 64; k += BLC) g = umax(g, readlane_u32(m, k));
    } else {
      g = lane_group_max<GLC>(m);
    }
  } else {
    for (int s = 1; s < BL; s <<= 1) m = umax(m, shfl_xor_u32(m, s));
    g = m;
    for (int s = BL; s < GL; s <<= 1) g = umax(g, shfl_xor_u32(g, s));
  }

  const float G = u2f(g);
  const uint32_t e = e8m0_of(u2f(m), G);
  const float sG = e8m0_decode(e) * G;
  const float S = quant_scale(e, G);
  const float yv = 128.0f / S;
  // unclamped and finite: S == sG exactly and every t below is finite
  const bool ok = !live || (sG >= kClamp && sG <= 3.0e38f);

  // t = z * RN(128 / S) is within 2 ulp of RN(z / S) * 128; four elements
  // whose t lies within 8 ulp of a bf16 rounding midpoint (the mid_key test,
  // one compare of the smallest key) are recomputed with the exact division
  // (a few per thousand waves), and a wave with a clamped or non-finite block
  // takes the exact path throughout.
  uint32_t out[4];
  if (__all(ok)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float t0 = z[4 * j] * yv, t1 = z[4 * j + 1] * yv, t2 = z[4 * j + 2] * yv, t3 = z[4 * j + 3] * yv;
      out[j] = cvt4<true>(t0, t1, t2, t3);
      if (mid_key4(t0, t1, t2, t3) <= kMidKey)
        out[j] = cvt4_exact(z[4 * j], z[4 * j + 1], z[4 * j + 2], z[4 * j + 3], S);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = cvt4_exact(z[4 * j], z[4 * j + 1], z[4 * j + 2], z[4 * j + 3], S);
  }
  if (!live) return;
  store_stream16(q + off, u32x4_t{out[0], out[1], out[2], out[3]});
  if ((lane & (BL - 1)) == 0) sc8[off >> (bl_log2 + 4)] = (uint8_t)e;
  if ((lane & (GL - 1)) == 0) sc32[off >> (gl_log2 + 4)] = G;
}

// --------------------------------------------------------------------------
// General path.  Block maxima: thread per chunk of CH consecutive results in
// `rows` consecutive rows of one block row of the result grid (rows | a); the
// lanes of an aligned run of b / CH lanes cover one block's columns and are
// combined by shuffles when that run is a power of two <= 64 (seg_log2 >= 0).
// --------------------------------------------------------------------------
template <int OP, int CH, bool VEC, typename I>
__global__ __launch_bounds__(256) void k_ew_blockmax(QOperand X, QOperand Y, uint32_t* __restrict__ ws,
                                                     int64_t n_threads, int64_t W, int64_t a, int64_t b,
                                                     int seg_log2, int rows) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool live = t < n_threads;
  uint32_t m = 0;
  I blk = 0;
  if (live) {
    const I cpr = (I)W / CH;                      // chunks per row
    const I rg = (I)t / cpr, c = ((I)t - rg * cpr) * CH;
    const I i0 = rg * (I)rows;
    for (int r = 0; r < rows; ++r) {
      float z[CH];
      ew_chunk<OP, CH, VEC, I>(X, Y, i0 + (I)r, c, (I)W, z);
#pragma unroll
      for (int k = 0; k < CH; ++k) m = umax(m, abs_bits(z[k]));
    }
    blk = (i0 / (I)a) * ((I)W / (I)b) + c / (I)b;
  }
  if (seg_log2 >= 0) {
    const int seg = 1 << seg_log2;
    for (int s = 1; s < seg; s <<= 1) m = umax(m, shfl_xor_u32(m, s));
    if (live && ((threadIdx.x & (seg - 1)) == 0)) atomicMax(&ws[blk], m);
  } else if (live) {
    atomicMax(&ws[blk], m);
  }
}

// Cast: thread per chunk of CH results, recomputed, with the scales of its
// result block.
template <int OP, int CH, bool VEC, typename I>
__global__ __launch_bounds__(256) void k_ew_cast(QOperand X, QOperand Y, uint8_t* __restrict__ q,
                                                 const uint8_t* __restrict__ sc8, const float* __restrict__ sc32,
                                                 int64_t n_chunks, int64_t W, int64_t a, int64_t b, int64_t K) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_chunks) return;
  const I off = (I)t * CH;
  const I i = off / (I)W, c = off - i * (I)W;
  const I blk = (i / (I)a) * ((I)W / (I)b) + c / (I)b;
  const uint32_t e = sc8[blk];
  const float G = sc32[blk / (I)K];
  const float sG = e8m0_decode(e) * G;
  const float S = quant_scale(e, G);
  const bool ok = sG >= kClamp && sG <= 3.0e38f;
  const float yv = 128.0f / S;
  float z[CH];
  ew_chunk<OP, CH, VEC, I>(X, Y, i, c, (I)W, z);
  uint32_t code[CH];
  if constexpr (CH % 4 == 0) {
    // 4 values at a time on the hardware conversions, as k_ew_rowgroup casts
#pragma unroll
    for (int j = 0; j < CH / 4; ++j) {
      uint32_t w;
      if (ok) {
        const float t0 = z[4 * j] * yv, t1 = z[4 * j + 1] * yv, t2 = z[4 * j + 2] * yv, t3 = z[4 * j + 3] * yv;
        w = cvt4_hw(t0, t1, t2, t3);
        if (mid_key4(t0, t1, t2, t3) <= kMidKey) w = cvt4_exact(z[4 * j], z[4 * j + 1], z[4 * j + 2], z[4 * j + 3], S);
      } else {
        w = cvt4_exact(z[4 * j], z[4 * j + 1], z[4 * j + 2], z[4 * j + 3], S);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) code[4 * j + i] = (w >> (8 * i)) & 0xFFu;
    }
  } else {
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const float tv = z[k] * yv;
      code[k] = (ok && !near_bf16_midpoint(tv)) ? bf16_to_e4m3fn(f32_to_bf16_rne_nonan(tv))
                                                : quant_elem_exact(z[k], S);
    }
  }
  uint8_t* o = q + off;
  if constexpr (VEC) {
    uint32_t w[CH / 4];
#pragma unroll
    for (int j = 0; j < CH / 4; ++j)
      w[j] = code[4 * j] | (code[4 * j + 1] << 8) | (code[4 * j + 2] << 16) | (code[4 * j + 3] << 24);
    if constexpr (CH == 16) *reinterpret_cast<uint4*>(o) = make_uint4(w[0], w[1], w[2], w[3]);
    else if constexpr (CH == 8) *reinterpret_cast<uint2*>(o) = make_uint2(w[0], w[1]);
    else *reinterpret_cast<uint32_t*>(o) = w[0];
  } else {
#pragma unroll
    for (int k = 0; k < CH; ++k) o[k] = (uint8_t)code[k];
  }
}

// --------------------------------------------------------------------------
// Host side
// --------------------------------------------------------------------------
int64_t gcd_i64(int64_t x, int64_t y) {
  while (y) {
    const int64_t t = x % y;
    x = y;
    y = t;
  }
  return x;
}

bool pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }
int log2_of(int64_t v) {
  int r = 0;
  while ((int64_t(1) << r) < v) ++r;
  return r;
}
bool is_aligned(const void* p, size_t n) { return reinterpret_cast<uintptr_t>(p) % n == 0; }
unsigned blocks_for(int64_t n, int64_t per) { return (unsigned)((n + per - 1) / per > 0 ? (n + per - 1) / per : 1); }

// Blocks per group of a [H, W] slice with grid (a, b), _qarr.py:474-480.
int grid_layout(const char* what, int64_t H, int64_t W, int64_t a, int64_t b, int64_t* n_blk, int64_t* K) {
  if (a < 1 || b < 1 || H % a || W % b)
    return pratchya_set_error(PRATCHYA_EINVAL, "elementwise: %s grid (%lld, %lld) does not divide the slice (%lld, %lld)",
                              what, (long long)a, (long long)b, (long long)H, (long long)W);
  *n_blk = (H / a) * (W / b);
  const int64_t target = (a * b) / 16 > 1 ? (a * b) / 16 : 1;
  *K = *n_blk ? gcd_i64(target, *n_blk) : 1;
  return PRATCHYA_OK;
}

QOperand operand(const uint8_t* q, const uint8_t* s8, const float* s32, int64_t a, int64_t b, int64_t K) {
  const bool flat = a == 1 && pow2(b) && pow2(K);
  return QOperand{q, s8, s32, a, b, K, flat ? log2_of(b) : -1, flat ? log2_of(K) : -1, nullptr, 0};
}

struct EwPlan {
  bool one_pass;
  int bl_log2, gl_log2;                  // one pass
  int ch, rows, seg_log2;                // general
  bool vec;
};

EwPlan plan(const QOperand& X, const QOperand& Y, const uint8_t* q, int64_t W, int64_t a, int64_t b, int64_t K) {
  EwPlan p{};
  const int64_t BL = b / 16, GL = BL * K;
  p.one_pass = a == 1 && b % 16 == 0 && W % 16 == 0 && X.b % 16 == 0 && Y.b % 16 == 0 && pow2(BL) && BL <= 64 &&
               pow2(GL) && GL <= 64 && is_aligned(X.q, 16) && is_aligned(Y.q, 16) && is_aligned(q, 16);
  if (p.one_pass) {
    p.bl_log2 = log2_of(BL);
    p.gl_log2 = log2_of(GL);
    return p;
  }
  const int64_t bb = gcd_i64(gcd_i64(b, X.b), Y.b);
  p.ch = 1;
  while (p.ch < 16 && bb % (p.ch * 2) == 0) p.ch *= 2;
  p.vec = p.ch >= 4 && is_aligned(X.q, p.ch) && is_aligned(Y.q, p.ch) && is_aligned(q, p.ch);
  p.rows = 1;
  while (p.rows < 16 && a % (p.rows * 2) == 0) p.rows *= 2;
  const int64_t seg = b / p.ch;
  p.seg_log2 = (pow2(seg) && seg <= 64) ? log2_of(seg) : -1;
  return p;
}

template <int OP, typename I>
void launch_one_pass(const QOperand& X, const QOperand& Y, uint8_t* q, uint8_t* sc8, float* sc32, int64_t n,
                     int64_t W, const EwPlan& p, hipStream_t st) {
  const dim3 grid(blocks_for(n, 1024));           // one wave per workgroup
  if (X.lb >= 0 && Y.lb >= 0 && p.bl_log2 == 3 && p.gl_log2 == 6)     // (1, 128), K = 8 everywhere
    hipLaunchKernelGGL((k_ew_rowgroup<OP, true, I, 8, 64>), grid, dim3(64), 0, st, X, Y, q, sc8, sc32, n, W,
                       p.bl_log2, p.gl_log2);
  else if (X.lb >= 0 && Y.lb >= 0)
    hipLaunchKernelGGL((k_ew_rowgroup<OP, true, I, 0, 0>), grid, dim3(64), 0, st, X, Y, q, sc8, sc32, n, W,
                       p.bl_log2, p.gl_log2);
  else
    hipLaunchKernelGGL((k_ew_rowgroup<OP, false, I, 0, 0>), grid, dim3(64), 0, st, X, Y, q, sc8, sc32, n, W,
                       p.bl_log2, p.gl_log2);
}

template <int OP, int CH, bool VEC, typename I>
void launch_general_t(const QOperand& X, const QOperand& Y, uint8_t* q, uint8_t* sc8, float* sc32, uint32_t* ws,
                      int64_t n, int64_t W, int64_t a, int64_t b, int64_t K, int64_t n_blk_total,
                      int64_t n_groups, const EwPlan& p, hipStream_t st) {
  const unsigned fill = blocks_for(n_blk_total, 256);
  hipLaunchKernelGGL(k_fill_u32, dim3(fill > 4096 ? 4096 : fill), dim3(256), 0, st, ws, n_blk_total, 0u);
  const int64_t n_chunks = n / CH;
  const int64_t n_bm = n_chunks / p.rows;
  hipLaunchKernelGGL((k_ew_blockmax<OP, CH, VEC, I>), dim3(blocks_for(n_bm, 256)), dim3(256), 0, st, X, Y, ws, n_bm,
                     W, a, b, p.seg_log2, p.rows);
  if (K >= 32)
    hipLaunchKernelGGL(k_group_scales, dim3(blocks_for(n_groups, 4)), dim3(256), 0, st, ws, sc8, sc32, n_groups, K);
  else
    hipLaunchKernelGGL(k_group_scales_small, dim3(blocks_for(n_groups, 256)), dim3(256), 0, st, ws, sc8, sc32,
                       n_groups, K);
  hipLaunchKernelGGL((k_ew_cast<OP, CH, VEC, I>), dim3(blocks_for(n_chunks, 256)), dim3(256), 0, st, X, Y, q, sc8,
                     sc32, n_chunks, W, a, b, K);
}

template <int OP, typename I>
void launch_general(const QOperand& X, const QOperand& Y, uint8_t* q, uint8_t* sc8, float* sc32, uint32_t* ws,
                    int64_t n, int64_t W, int64_t a, int64_t b, int64_t K, int64_t n_blk_total, int64_t n_groups,
                    const EwPlan& p, hipStream_t st) {
#define PRATCHYA_EW(C, V) \
  launch_general_t<OP, C, V, I>(X, Y, q, sc8, sc32, ws, n, W, a, b, K, n_blk_total, n_groups, p, st)
  if (p.vec) {
    switch (p.ch) {
      case 4: PRATCHYA_EW(4, true); break;
      case 8: PRATCHYA_EW(8, true); break;
      default: PRATCHYA_EW(16, true); break;
    }
  } else {
    switch (p.ch) {
      case 1: PRATCHYA_EW(1, false); break;
      case 2: PRATCHYA_EW(2, false); break;
      case 4: PRATCHYA_EW(4, false); break;
      case 8: PRATCHYA_EW(8, false); break;
      default: PRATCHYA_EW(16, false); break;
    }
  }
#undef PRATCHYA_EW
}

template <int OP>
void launch_op(const QOperand& X, const QOperand& Y, uint8_t* q, uint8_t* sc8, float* sc32, uint32_t* ws, int64_t n,
               int64_t W, int64_t a, int64_t b, int64_t K, int64_t n_blk_total, int64_t n_groups, const EwPlan& p,
               hipStream_t st) {
  const bool narrow = n <= 0x7FFFFFFF;
  if (p.one_pass) {
    if (narrow) launch_one_pass<OP, uint32_t>(X, Y, q, sc8, sc32, n, W, p, st);
    else launch_one_pass<OP, int64_t>(X, Y, q, sc8, sc32, n, W, p, st);
  } else if (narrow) {
    launch_general<OP, uint32_t>(X, Y, q, sc8, sc32, ws, n, W, a, b, K, n_blk_total, n_groups, p, st);
  } else {
    launch_general<OP, int64_t>(X, Y, q, sc8, sc32, ws, n, W, a, b, K, n_blk_total, n_groups, p, st);
  }
}

}  // namespace

extern "C" size_t pratchya_elementwise_workspace_bytes(int64_t slices, int64_t H, int64_t W, int64_t xa, int64_t xb,
                                                       int64_t ya, int64_t yb, int64_t a, int64_t b) {
  int64_t n_blk, K, nx, kx, ny, ky;
  if (slices < 0 || H < 0 || W < 0 || grid_layout("result", H, W, a, b, &n_blk, &K) ||
      grid_layout("x", H, W, xa, xb, &nx, &kx) || grid_layout("y", H, W, ya, yb, &ny, &ky))
    return 0;
  // the one-pass kernel (16-byte aligned payloads) needs none
  alignas(16) static const uint8_t probe[16] = {0};
  const QOperand X = operand(probe, nullptr, nullptr, xa, xb, kx), Y = operand(probe, nullptr, nullptr, ya, yb, ky);
  if (plan(X, Y, probe, W, a, b, K).one_pass) return 0;
  return (size_t)(slices * n_blk) * sizeof(uint32_t);
}

extern "C" int pratchya_elementwise(int op, const uint8_t* x_fp8, const uint8_t* x_sc8, const float* x_sc32,
                                    int64_t xa, int64_t xb, const uint8_t* y_fp8, const uint8_t* y_sc8,
                                    const float* y_sc32, int64_t ya, int64_t yb, int64_t slices, int64_t H, int64_t W,
                                    int64_t a, int64_t b, uint8_t* out_fp8, uint8_t* out_sc8, float* out_sc32,
                                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (op < PRATCHYA_OP_ADD || op > PRATCHYA_OP_MOD)
    return pratchya_set_error(PRATCHYA_EINVAL, "elementwise: unknown operator %d", op);
  if (slices < 0 || H < 0 || W < 0)
    return pratchya_set_error(PRATCHYA_EINVAL, "elementwise: negative shape (%lld, %lld, %lld)", (long long)slices,
                              (long long)H, (long long)W);
  int64_t n_blk, K, nx, kx, ny, ky;
  int rc = grid_layout("result", H, W, a, b, &n_blk, &K);
  if (!rc) rc = grid_layout("x", H, W, xa, xb, &nx, &kx);
  if (!rc) rc = grid_layout("y", H, W, ya, yb, &ny, &ky);
  if (rc) return rc;
  const int64_t n = slices * H * W;
  if (n == 0) return pratchya_set_error(PRATCHYA_OK, "");
  if (!x_fp8 || !x_sc8 || !x_sc32 || !y_fp8 || !y_sc8 || !y_sc32 || !out_fp8 || !out_sc8 || !out_sc32)
    return pratchya_set_error(PRATCHYA_EINVAL, "elementwise: null buffer");
  const QOperand X = operand(x_fp8, x_sc8, x_sc32, xa, xb, kx), Y = operand(y_fp8, y_sc8, y_sc32, ya, yb, ky);
  const EwPlan p = plan(X, Y, out_fp8, W, a, b, K);
  const int64_t n_blk_total = slices * n_blk, n_groups = n_blk_total / K;
  uint32_t* ws = static_cast<uint32_t*>(workspace);
  if (!p.one_pass) {
    const size_t need = (size_t)n_blk_total * sizeof(uint32_t);
    if (!workspace || workspace_bytes < need)
      return pratchya_set_error(PRATCHYA_EINVAL, "elementwise: workspace of %zu bytes needed, got %zu", need,
                                workspace_bytes);
  }
  switch (op) {
    case PRATCHYA_OP_ADD:
      launch_op<PRATCHYA_OP_ADD>(X, Y, out_fp8, out_sc8, out_sc32, ws, n, W, a, b, K, n_blk_total, n_groups, p, stream);
      break;
    case PRATCHYA_OP_SUB:
      launch_op<PRATCHYA_OP_SUB>(X, Y, out_fp8, out_sc8, out_sc32, ws, n, W, a, b, K, n_blk_total, n_groups, p, stream);
      break;
    case PRATCHYA_OP_MUL:
      launch_op<PRATCHYA_OP_MUL>(X, Y, out_fp8, out_sc8, out_sc32, ws, n, W, a, b, K, n_blk_total, n_groups, p, stream);
      break;
    case PRATCHYA_OP_DIV:
      launch_op<PRATCHYA_OP_DIV>(X, Y, out_fp8, out_sc8, out_sc32, ws, n, W, a, b, K, n_blk_total, n_groups, p, stream);
      break;
    case PRATCHYA_OP_FLOORDIV:
      launch_op<PRATCHYA_OP_FLOORDIV>(X, Y, out_fp8, out_sc8, out_sc32, ws, n, W, a, b, K, n_blk_total, n_groups, p,
                                      stream);
      break;
    default:
      launch_op<PRATCHYA_OP_MOD>(X, Y, out_fp8, out_sc8, out_sc32, ws, n, W, a, b, K, n_blk_total, n_groups, p, stream);
      break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return pratchya_set_error(PRATCHYA_EHIP, "elementwise: launch failed: %s", hipGetErrorString(e));
  return pratchya_set_error(PRATCHYA_OK, "");
}

extern "C" int pratchya_gather_quantize(const uint8_t* x_fp8, const uint8_t* x_sc8, const float* x_sc32, int64_t H,
                                        int64_t W, int64_t xa, int64_t xb, const int64_t* idx, int64_t slices,
                                        int64_t T, int64_t a, int64_t b, uint8_t* out_fp8, uint8_t* out_sc8,
                                        float* out_sc32, void* workspace, size_t workspace_bytes,
                                        hipStream_t stream) {
  if (H < 0 || W < 0 || slices < 0 || T < 0)
    return pratchya_set_error(PRATCHYA_EINVAL, "gather_quantize: negative shape");
  int64_t tblk, tK, n_blk, K;
  int rc = grid_layout("table", H, W, xa, xb, &tblk, &tK);
  if (!rc) rc = grid_layout("result", T, W, a, b, &n_blk, &K);
  if (rc) return rc;
  const int64_t n = slices * T * W;
  if (n == 0) return pratchya_set_error(PRATCHYA_OK, "");
  if (H == 0) return pratchya_set_error(PRATCHYA_EINVAL, "gather_quantize: index into an empty table");
  if (!x_fp8 || !x_sc8 || !x_sc32 || !idx || !out_fp8 || !out_sc8 || !out_sc32)
    return pratchya_set_error(PRATCHYA_EINVAL, "gather_quantize: null buffer");
  const int64_t n_blk_total = slices * n_blk, n_groups = n_blk_total / K;
  const size_t need = (size_t)n_blk_total * sizeof(uint32_t);
  if (!workspace || workspace_bytes < need)
    return pratchya_set_error(PRATCHYA_EINVAL, "gather_quantize: workspace of %zu bytes needed, got %zu", need,
                              workspace_bytes);
  QOperand X = operand(x_fp8, x_sc8, x_sc32, xa, xb, tK);
  X.rows = idx;
  X.rows_h = H;
  X.lb = X.lk = -1;
  EwPlan p = plan(X, X, out_fp8, W, a, b, K);
  if (p.one_pass) {                      // the row map needs the general path
    p.one_pass = false;
    const int64_t bb = gcd_i64(b, xb);
    p.ch = 1;
    while (p.ch < 16 && bb % (p.ch * 2) == 0) p.ch *= 2;
    p.vec = p.ch >= 4 && is_aligned(x_fp8, p.ch) && is_aligned(out_fp8, p.ch);
    p.rows = 1;
    while (p.rows < 16 && a % (p.rows * 2) == 0) p.rows *= 2;
    const int64_t seg = b / p.ch;
    p.seg_log2 = (pow2(seg) && seg <= 64) ? log2_of(seg) : -1;
  }
  uint32_t* ws = static_cast<uint32_t*>(workspace);
  if (n <= 0x7FFFFFFF)
    launch_general<OP_GATHER, uint32_t>(X, X, out_fp8, out_sc8, out_sc32, ws, n, W, a, b, K, n_blk_total, n_groups,
                                        p, stream);
  else
    launch_general<OP_GATHER, int64_t>(X, X, out_fp8, out_sc8, out_sc32, ws, n, W, a, b, K, n_blk_total, n_groups,
                                       p, stream);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return pratchya_set_error(PRATCHYA_EHIP, "gather_quantize: launch failed: %s", hipGetErrorString(e));
  return pratchya_set_error(PRATCHYA_OK, "");
}
