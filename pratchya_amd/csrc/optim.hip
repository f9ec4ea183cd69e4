// Elementwise kernels of pratchya's quantized-momentum optimizer step
// (Miulion, pratchya/_nnx_impl/_optimizer.py:62-217) for gfx950.
//
// Per parameter leaf the reference computes, in the leaf's arithmetic dtype
// (f32 for a 2-D quantized parameter, :153-199; bf16 per layer of a 3-D
// stacked one, :117-142):
//   m, g     = dequantize(momentum), dequantize(gradient)     (:124-125, :160-161)
//   c        = beta1 * m + (1 - beta1) * g                    (:134, :175)
//   m_new    = beta2 * m + (1 - beta2) * g                    (:135, :176)
//   momentum = QArrayImpl(m_new, tgrid)                       (:145, :187)
//   update   = -(lr * u + lr * wd * p),  u = NS(c) * sqrt(max(N, M))  (Muon, :147-150, :189-193)
//                                        u = sign(c)                   (Lion, :151-153, :194-197)
// k_momentum produces c and m_new in one pass over the quantized momentum
// and gradient (m_new is then quantized by the block quantizer);
// k_update produces the update from u (or c) and the quantized parameter.
// NS (Newton-Schulz) is plain GEMMs and runs on the BLAS library.
//
// Arithmetic follows the reference's operation order with one rounding per
// operation: products and sums are separately rounded (no fused
// multiply-add).  The momentum runs in the leaf's dtype (bf16: every
// intermediate rounded to bf16), with the Python-scalar constants rounded to
// it by the host.  The update runs in f32: the learning rates come from
// schedules of the int32 step count, f32 arrays that promote the bf16
// operands (only u * sqrt(max(N, M)) stays in the leaf's dtype).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <initializer_list>
#include <utility>

#include "fp8_math.h"
#include "pratchya_fp8.h"
#include "quant_device.h"

int pratchya_set_error(int code, const char* fmt, ...);

#pragma clang fp contract(off)

namespace {

using namespace pfp8;

// Round to the arithmetic dtype (identity for f32).
template <bool BF16>
__device__ __forceinline__ float rnd(float x) {
  if constexpr (BF16) return u2f(f32_to_bf16_rne(x) << 16);
  return x;
}

// Round element pairs of v to the arithmetic dtype: bf16 with
// v_cvt_pk_bf16_f32 (RNE, two values per instruction; checked against the
// software rounding on ties and every subnormal pattern by the test suite).
template <bool BF16, int CH>
__device__ __forceinline__ void rnd_all(float (&v)[CH]) {
  if constexpr (BF16) {
    if constexpr (CH % 2 == 0) {
#pragma unroll
      for (int k = 0; k < CH; k += 2) {
        const uint32_t w = pack_bf16x2(v[k], v[k + 1]);
        v[k] = u2f(w << 16);
        v[k + 1] = u2f(w & 0xFFFF0000u);
      }
    } else {
#pragma unroll
      for (int k = 0; k < CH; ++k) v[k] = rnd<true>(v[k]);
    }
  }
}

// Block index of element `off` of a [rows, W] array with tgrid (a, b)
// (32-bit divisions when the array is small enough).
__device__ __forceinline__ int64_t block_of(int64_t off, int64_t W, int64_t a, int64_t b, bool narrow) {
  if (narrow) {
    const uint32_t o = (uint32_t)off, w = (uint32_t)W;
    const uint32_t i = o / w, c = o - i * w;
    return (int64_t)((i / (uint32_t)a) * (w / (uint32_t)b) + c / (uint32_t)b);
  }
  const int64_t i = off / W, c = off - i * W;
  return (i / a) * (W / b) + c / b;
}

// Dequantization scale s * G of a block (K blocks per group, _qarr.py:562-564).
__device__ __forceinline__ float block_scale(const uint8_t* __restrict__ sc8, const float* __restrict__ sc32,
                                             int64_t blk, int64_t K) {
  return e8m0_decode(sc8[blk]) * sc32[blk / K];
}

// CH elements of type T loaded or stored as one unit (16-byte vector
// accesses for 16 or more bytes; the host checks the alignment).
template <typename T, int CH>
struct alignas((sizeof(T) * CH) >= 16 ? 16 : sizeof(T) * CH) Vec {
  T v[CH];
};

// CH consecutive elements from `off` of an operand given as an fp8 payload
// (mode 0, block scale sc), bf16 (1) or f32 (2), in the arithmetic dtype.
template <int MODE, bool BF16, int CH>
__device__ __forceinline__ void load_operand(const void* __restrict__ x, float sc, int64_t off, float (&out)[CH]) {
  if constexpr (MODE == 0) {
    const Vec<uint8_t, CH> w = *reinterpret_cast<const Vec<uint8_t, CH>*>(static_cast<const uint8_t*>(x) + off);
    if constexpr (CH % 4 == 0) {
      // four bytes per word through v_cvt_scalef32_pk_f32_fp8 (exact)
#pragma unroll
      for (int j = 0; j < CH / 4; ++j) {
        const uint32_t word = (uint32_t)w.v[4 * j] | ((uint32_t)w.v[4 * j + 1] << 8) |
                              ((uint32_t)w.v[4 * j + 2] << 16) | ((uint32_t)w.v[4 * j + 3] << 24);
        fp8_word(word, out[4 * j], out[4 * j + 1], out[4 * j + 2], out[4 * j + 3]);
      }
    } else {
#pragma unroll
      for (int k = 0; k < CH; ++k) out[k] = e4m3fn_to_f32(w.v[k]);
    }
#pragma unroll
    for (int k = 0; k < CH; ++k) out[k] = (out[k] * sc) * 0.0078125f;
    rnd_all<BF16, CH>(out);
  } else if constexpr (MODE == 1) {
    const Vec<uint16_t, CH> w = *reinterpret_cast<const Vec<uint16_t, CH>*>(static_cast<const uint16_t*>(x) + off);
#pragma unroll
    for (int k = 0; k < CH; ++k) out[k] = u2f((uint32_t)w.v[k] << 16);
  } else {
    const Vec<float, CH> w = *reinterpret_cast<const Vec<float, CH>*>(static_cast<const float*>(x) + off);
#pragma unroll
    for (int k = 0; k < CH; ++k) out[k] = w.v[k];
    rnd_all<BF16, CH>(out);
  }
}

// HW: round pairs with v_cvt_pk_bf16_f32 (k_update keeps the integer
// rounding: the compiler's selection of the packed conversion fails on its
// negated sums with packed f32 operations disabled).  A 16-byte chunk (8 bf16
// or 4 f32 values, consecutive lanes on consecutive chunks) is stored
// non-temporally: measured on the FFN down-projection's [16384,4096] leaf,
// the momentum kernel 90-97 -> 71-72 us, the update 62 -> 61 us, the
// optimizer step unchanged.
template <bool BF16, int CH, bool HW = false>
__device__ __forceinline__ void store_chunk(void* out, int64_t off, const float (&v)[CH]) {
  if constexpr (BF16 && HW && CH % 2 == 0) {
    Vec<uint32_t, CH / 2> w;
#pragma unroll
    for (int k = 0; k < CH; k += 2) w.v[k / 2] = pack_bf16x2(v[k], v[k + 1]);
    if constexpr (CH == 8) store_stream16(static_cast<uint16_t*>(out) + off, u32x4_t{w.v[0], w.v[1], w.v[2], w.v[3]});
    else *reinterpret_cast<Vec<uint32_t, CH / 2>*>(static_cast<uint16_t*>(out) + off) = w;
  } else if constexpr (BF16) {
    Vec<uint16_t, CH> w;
#pragma unroll
    for (int k = 0; k < CH; ++k) w.v[k] = (uint16_t)f32_to_bf16_rne(v[k]);
    if constexpr (CH == 8)
      store_stream16(static_cast<uint16_t*>(out) + off,
                     u32x4_t{(uint32_t)w.v[0] | ((uint32_t)w.v[1] << 16), (uint32_t)w.v[2] | ((uint32_t)w.v[3] << 16),
                             (uint32_t)w.v[4] | ((uint32_t)w.v[5] << 16), (uint32_t)w.v[6] | ((uint32_t)w.v[7] << 16)});
    else *reinterpret_cast<Vec<uint16_t, CH>*>(static_cast<uint16_t*>(out) + off) = w;
  } else if constexpr (CH == 4) {
    store_stream16(static_cast<float*>(out) + off, u32x4_t{f2u(v[0]), f2u(v[1]), f2u(v[2]), f2u(v[3])});
  } else {
    Vec<float, CH> w;
#pragma unroll
    for (int k = 0; k < CH; ++k) w.v[k] = v[k];
    *reinterpret_cast<Vec<float, CH>*>(static_cast<float*>(out) + off) = w;
  }
}

// c = b1*m + b1c*g and m_new = b2*m + b2c*g for CH consecutive elements per
// thread, CH dividing b (one block per chunk; the momentum shares the
// gradient's layout).
template <int G_MODE, bool BF16, int CH>
__global__ __launch_bounds__(256) void k_momentum(const uint8_t* __restrict__ m8, const uint8_t* __restrict__ m_sc8,
                                                  const float* __restrict__ m_sc32, const void* __restrict__ g,
                                                  const uint8_t* __restrict__ g_sc8, const float* __restrict__ g_sc32,
                                                  int64_t n_chunks, int64_t W, int64_t a, int64_t b, int64_t K,
                                                  float b1, float b1c, float b2, float b2c, void* __restrict__ c_out,
                                                  void* __restrict__ m_new) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_chunks) return;
  const int64_t base = t * CH;
  const int64_t blk = block_of(base, W, a, b, n_chunks * CH <= 0x7FFFFFFF);
  const float msc = block_scale(m_sc8, m_sc32, blk, K);
  const float gsc = G_MODE == 0 ? block_scale(g_sc8, g_sc32, blk, K) : 0.0f;
  float mv[CH], gv[CH], c[CH], nm[CH], t1[CH], t2[CH], t3[CH], t4[CH];
  load_operand<0, BF16, CH>(m8, msc, base, mv);
  load_operand<G_MODE, BF16, CH>(g, gsc, base, gv);
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    t1[k] = b1 * mv[k];
    t2[k] = b1c * gv[k];
    t3[k] = b2 * mv[k];
    t4[k] = b2c * gv[k];
  }
  rnd_all<BF16, CH>(t1);
  rnd_all<BF16, CH>(t2);
  rnd_all<BF16, CH>(t3);
  rnd_all<BF16, CH>(t4);
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    c[k] = t1[k] + t2[k];
    nm[k] = t3[k] + t4[k];
  }
  // the sums are rounded once more by the bf16 store (RNE), as rnd() would
  store_chunk<BF16, CH, true>(c_out, base, c);
  store_chunk<BF16, CH, true>(m_new, base, nm);
}

// One Newton-Schulz combination X <- 1.5 X - 0.5 B (_optimizer.py:26-27,
// B = (X X^T) X from the library GEMMs) in the dtype of X: both products and
// the difference rounded separately (1.5 and 0.5 are exact in bf16).  CH
// elements per thread (16 bytes of X; CH = 1 for any size and alignment).
// `out` may be `x` (no restrict on them).
template <bool BF16, int CH>
__global__ __launch_bounds__(256) void k_ns_combine(const void* x, const void* __restrict__ bm, void* out,
                                                    int64_t n_chunks) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_chunks) return;
  const int64_t base = t * CH;
  constexpr int MODE = BF16 ? 1 : 2;
  float xv[CH], bv[CH], v[CH];
  load_operand<MODE, BF16, CH>(x, 0.0f, base, xv);
  load_operand<MODE, BF16, CH>(bm, 0.0f, base, bv);
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    xv[k] = 1.5f * xv[k];
    bv[k] = 0.5f * bv[k];
  }
  rnd_all<BF16, CH>(xv);
  rnd_all<BF16, CH>(bv);
#pragma unroll
  for (int k = 0; k < CH; ++k) v[k] = xv[k] - bv[k];
  store_chunk<BF16, CH, true>(out, base, v);        // the difference's rounding (RNE)
}

// Frobenius normalization of a bf16 Newton-Schulz input, X = G / (||G||_F +
// 1e-7) (_optimizer.py:17), with the roundings of that bf16 expression: each
// square rounded to bf16, their f32 sum rounded to bf16, the square root and
// the sum with 1e-7 each rounded to bf16, every quotient rounded to bf16.  Two
// passes with a fixed reduction order, so the result is the same on every
// call: per-workgroup sums of the squares, then every workgroup of the second
// pass sums those partials in one order before it scales its elements.
constexpr int kNormBlocks = 1024;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return u2f(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return u2f(w & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_rne(float v) { return bf16_lo(pack_bf16x2(v, 0.0f)); }

// Sum of a wave's 64 values, the same tree on every call.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__global__ __launch_bounds__(256) void k_sumsq_b16(const uint16_t* __restrict__ x, int64_t n,
                                                   float* __restrict__ part) {
  const int64_t n8 = n / 8;
  float s = 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
    const uint4 v = *reinterpret_cast<const uint4*>(x + i * 8);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float lo = bf16_lo(w[k]), hi = bf16_hi(w[k]);
      const uint32_t q = pack_bf16x2(lo * lo, hi * hi);   // each square rounded to bf16
      s += bf16_lo(q);
      s += bf16_hi(q);
    }
  }
  if (blockIdx.x == 0)
    for (int64_t i = n8 * 8 + threadIdx.x; i < n; i += 256) {
      const float f = bf16_lo(x[i]);
      s += bf16_rne(f * f);
    }
  __shared__ float ws[4];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = (ws[0] + ws[1]) + (ws[2] + ws[3]);
}

// (x and y may be the same array: each element is read and written by one
// thread)
__global__ __launch_bounds__(256) void k_ns_scale_b16(const uint16_t* x, int64_t n, const float* __restrict__ part,
                                                      uint16_t* y) {
  __shared__ float sden;
  if (threadIdx.x < 64) {
    float s = 0.0f;
    for (int i = (int)threadIdx.x; i < kNormBlocks; i += 64) s += part[i];
    s = wave_sum(s);
    if (threadIdx.x == 0) {
      const float total = bf16_rne(s);                 // the sum is a bf16 value
      const float norm = bf16_rne(sqrtf(total));
      sden = bf16_rne(norm + 1e-7f);
    }
  }
  __syncthreads();
  const float den = sden;
  const int64_t n8 = n / 8;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
    const uint4 v = *reinterpret_cast<const uint4*>(x + i * 8);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = pack_bf16x2(bf16_lo(w[k]) / den, bf16_hi(w[k]) / den);
    *reinterpret_cast<uint4*>(y + i * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
  if (blockIdx.x == 0)
    for (int64_t i = n8 * 8 + threadIdx.x; i < n; i += 256)
      y[i] = (uint16_t)(pack_bf16x2(bf16_lo(x[i]) / den, 0.0f) & 0xFFFFu);
}

// The f32 normalization (pratchya/_nnx_impl/_optimizer.py:17 on an f32
// leaf): each square rounded to f32 (no contraction into the sum), the sum
// in f32 in the same fixed order as the bf16 pass, sqrt and the sum with
// 1e-7 in f32, IEEE quotients.
__global__ __launch_bounds__(256) void k_sumsq_f32(const float* __restrict__ x, int64_t n,
                                                   float* __restrict__ part) {
  const int64_t n4 = n / 4;
  float s = 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    const float4 v = *reinterpret_cast<const float4*>(x + i * 4);
    s += __fmul_rn(v.x, v.x);
    s += __fmul_rn(v.y, v.y);
    s += __fmul_rn(v.z, v.z);
    s += __fmul_rn(v.w, v.w);
  }
  if (blockIdx.x == 0)
    for (int64_t i = n4 * 4 + threadIdx.x; i < n; i += 256) s += __fmul_rn(x[i], x[i]);
  __shared__ float ws[4];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = (ws[0] + ws[1]) + (ws[2] + ws[3]);
}

__global__ __launch_bounds__(256) void k_ns_scale_f32(const float* x, int64_t n, const float* __restrict__ part,
                                                      float* y) {
  __shared__ float sden;
  if (threadIdx.x < 64) {
    float s = 0.0f;
    for (int i = (int)threadIdx.x; i < kNormBlocks; i += 64) s += part[i];
    s = wave_sum(s);
    if (threadIdx.x == 0) sden = sqrtf(s) + 1e-7f;
  }
  __syncthreads();
  const float den = sden;
  const int64_t n4 = n / 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    const float4 v = *reinterpret_cast<const float4*>(x + i * 4);
    *reinterpret_cast<float4*>(y + i * 4) = make_float4(v.x / den, v.y / den, v.z / den, v.w / den);
  }
  if (blockIdx.x == 0)
    for (int64_t i = n4 * 4 + threadIdx.x; i < n; i += 256) y[i] = x[i] / den;
}

// jnp.sign: +-1 for nonzero, the argument itself for +-0 and NaN.
__device__ __forceinline__ float sign_of(float x) { return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : x); }

// update = -(lr * u' + lr_wd * p) in f32, u' = sign(u) (Lion) or u * scale
// in the leaf's dtype (Muon), p in the leaf's dtype; CH consecutive elements
// per thread as in k_momentum.
template <bool SIGN, int U_MODE, int P_MODE, bool BF16, bool OUT_BF16, int CH>
__global__ __launch_bounds__(256) void k_update(const void* __restrict__ u, const void* __restrict__ p,
                                                const uint8_t* __restrict__ p_sc8, const float* __restrict__ p_sc32,
                                                int64_t n_chunks, int64_t W, int64_t a, int64_t b, int64_t K,
                                                float scale, float lr, float lr_wd, void* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_chunks) return;
  const int64_t base = t * CH;
  const float psc = P_MODE == 0 ? block_scale(p_sc8, p_sc32, block_of(base, W, a, b, n_chunks * CH <= 0x7FFFFFFF), K)
                                : 0.0f;
  float uv[CH], pv[CH], ut[CH], v[CH];
  load_operand<U_MODE, BF16, CH>(u, 0.0f, base, uv);
  load_operand<P_MODE, BF16, CH>(p, psc, base, pv);
#pragma unroll
  for (int k = 0; k < CH; ++k) ut[k] = SIGN ? sign_of(uv[k]) : uv[k] * scale;
  if constexpr (!SIGN) rnd_all<BF16, CH>(ut);
#pragma unroll
  for (int k = 0; k < CH; ++k) v[k] = -((lr * ut[k]) + (lr_wd * pv[k]));
  store_chunk<OUT_BF16, CH>(out, base, v);
}

int64_t gcd64(int64_t x, int64_t y) {
  while (y) {
    const int64_t t = x % y;
    x = y;
    y = t;
  }
  return x;
}

struct Grid {
  int64_t n, W, a, b, K;
};

// Elements per thread: the first of `sizes` that divides b (a chunk then lies
// in one block) with every pointer aligned for the vector accesses, else 1.
int chunk_of(int64_t b, std::initializer_list<std::pair<const void*, int>> ptrs,
             std::initializer_list<int> sizes = {16, 4}) {
  for (int ch : sizes) {
    if (b % ch) continue;
    bool ok = true;
    for (auto [p, esz] : ptrs) {
      const int64_t need = (int64_t)ch * esz >= 16 ? 16 : (int64_t)ch * esz;
      if (p && reinterpret_cast<uintptr_t>(p) % need) ok = false;
    }
    if (ok) return ch;
  }
  return 1;
}

int dtype_size(int d) { return d == PRATCHYA_DT_F32 ? 4 : (d == PRATCHYA_DT_BF16 ? 2 : 1); }

int make_grid(const char* what, int64_t S, int64_t H, int64_t W, int64_t a, int64_t b, Grid* g) {
  if (S < 0 || H < 0 || W < 0 || a < 1 || b < 1 || H % a || W % b)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: tgrid (%lld, %lld) does not fit the slice (%lld, %lld)", what,
                              (long long)a, (long long)b, (long long)H, (long long)W);
  const int64_t n_blk = (H / a) * (W / b);
  const int64_t target = (a * b) / 16 > 1 ? (a * b) / 16 : 1;
  g->n = S * H * W;
  g->W = W;
  g->a = a;
  g->b = b;
  g->K = n_blk ? gcd64(target, n_blk) : 1;
  return PRATCHYA_OK;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return pratchya_set_error(PRATCHYA_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return PRATCHYA_OK;
}

bool is_float_dtype(int d) { return d == PRATCHYA_DT_F32 || d == PRATCHYA_DT_BF16; }

}  // namespace

extern "C" int pratchya_momentum(const uint8_t* m_fp8, const uint8_t* m_sc8, const float* m_sc32, const void* g,
                                 int g_dtype, const uint8_t* g_sc8, const float* g_sc32, int64_t slices, int64_t H,
                                 int64_t W, int64_t a, int64_t b, int arith_dtype, float beta1, float beta1c,
                                 float beta2, float beta2c, void* c_out, void* m_new, hipStream_t stream) {
  Grid L;
  int rc = make_grid("momentum", slices, H, W, a, b, &L);
  if (rc) return rc;
  if (!is_float_dtype(arith_dtype))
    return pratchya_set_error(PRATCHYA_EINVAL, "momentum: arithmetic dtype must be f32 or bf16 (got %d)", arith_dtype);
  if (g_dtype != PRATCHYA_DT_E4M3 && !is_float_dtype(g_dtype))
    return pratchya_set_error(PRATCHYA_EINVAL, "momentum: unsupported gradient dtype %d", g_dtype);
  if (L.n == 0) return PRATCHYA_OK;
  if (!m_fp8 || !m_sc8 || !m_sc32 || !g || !c_out || !m_new || (g_dtype == PRATCHYA_DT_E4M3 && (!g_sc8 || !g_sc32)))
    return pratchya_set_error(PRATCHYA_EINVAL, "momentum: null buffer");
  // chunks of 16 output bytes: one full-width store per lane and output,
  // contiguous across the wave
  const int ch = chunk_of(L.b, {{m_fp8, 1}, {g, dtype_size(g_dtype)}, {c_out, dtype_size(arith_dtype)},
                                {m_new, dtype_size(arith_dtype)}}, {16 / dtype_size(arith_dtype), 4});
  const int64_t chunks = L.n / ch;
  if (chunks / 256 + 1 > 0x7FFFFFFF) return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "momentum: too many elements");
  const dim3 grid((unsigned)((chunks + 255) / 256));
#define PRATCHYA_MOM(GM, BF, C)                                                                               \
  hipLaunchKernelGGL((k_momentum<GM, BF, C>), grid, dim3(256), 0, stream, m_fp8, m_sc8, m_sc32, g, g_sc8, g_sc32, \
                     chunks, L.W, L.a, L.b, L.K, beta1, beta1c, beta2, beta2c, c_out, m_new)
#define PRATCHYA_MOM_G(BF, C)                                 \
  if (g_dtype == PRATCHYA_DT_E4M3) PRATCHYA_MOM(0, BF, C);    \
  else if (g_dtype == PRATCHYA_DT_BF16) PRATCHYA_MOM(1, BF, C); \
  else PRATCHYA_MOM(2, BF, C);
  const bool bf = arith_dtype == PRATCHYA_DT_BF16;
  if (ch == 8) {
    PRATCHYA_MOM_G(true, 8)
  } else if (ch == 4) {
    if (bf) { PRATCHYA_MOM_G(true, 4) } else { PRATCHYA_MOM_G(false, 4) }
  } else {
    if (bf) { PRATCHYA_MOM_G(true, 1) } else { PRATCHYA_MOM_G(false, 1) }
  }
#undef PRATCHYA_MOM_G
#undef PRATCHYA_MOM
  return check_launch("momentum");
}

extern "C" int pratchya_ns_combine(const void* x, const void* b, void* out, int64_t n, int dtype,
                                   hipStream_t stream) {
  if (!is_float_dtype(dtype))
    return pratchya_set_error(PRATCHYA_EINVAL, "ns_combine: dtype must be f32 or bf16 (got %d)", dtype);
  if (n < 0) return pratchya_set_error(PRATCHYA_EINVAL, "ns_combine: negative size");
  if (n == 0) return PRATCHYA_OK;
  if (!x || !b || !out) return pratchya_set_error(PRATCHYA_EINVAL, "ns_combine: null buffer");
  const int esz = dtype_size(dtype), ch = 16 / esz;
  const bool vec = n % ch == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(b) % 16 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0;
  const int64_t chunks = vec ? n / ch : n;
  if (chunks / 256 + 1 > 0x7FFFFFFF) return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "ns_combine: too many elements");
  const dim3 grid((unsigned)((chunks + 255) / 256));
  if (dtype == PRATCHYA_DT_BF16) {
    if (vec) hipLaunchKernelGGL((k_ns_combine<true, 8>), grid, dim3(256), 0, stream, x, b, out, chunks);
    else hipLaunchKernelGGL((k_ns_combine<true, 1>), grid, dim3(256), 0, stream, x, b, out, chunks);
  } else {
    if (vec) hipLaunchKernelGGL((k_ns_combine<false, 4>), grid, dim3(256), 0, stream, x, b, out, chunks);
    else hipLaunchKernelGGL((k_ns_combine<false, 1>), grid, dim3(256), 0, stream, x, b, out, chunks);
  }
  return check_launch("ns_combine");
}

extern "C" int64_t pratchya_ns_normalize_workspace_bytes(void) { return (int64_t)kNormBlocks * 4; }

extern "C" int pratchya_ns_normalize(const void* g, void* x, int64_t n, void* workspace, int64_t workspace_bytes,
                                     hipStream_t stream) {
  if (n < 0) return pratchya_set_error(PRATCHYA_EINVAL, "ns_normalize: negative size");
  if (n == 0) return PRATCHYA_OK;
  if (!g || !x || !workspace) return pratchya_set_error(PRATCHYA_EINVAL, "ns_normalize: null buffer");
  if (workspace_bytes < (int64_t)kNormBlocks * 4 || reinterpret_cast<uintptr_t>(workspace) % 4)
    return pratchya_set_error(PRATCHYA_EINVAL, "ns_normalize: workspace of %lld bytes (need %d, 4-byte aligned)",
                              (long long)workspace_bytes, kNormBlocks * 4);
  if ((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(x)) % 16)
    return pratchya_set_error(PRATCHYA_EINVAL, "ns_normalize: g and x must be 16-byte aligned");
  float* part = static_cast<float*>(workspace);
  hipLaunchKernelGGL(k_sumsq_b16, dim3(kNormBlocks), dim3(256), 0, stream, static_cast<const uint16_t*>(g), n, part);
  int rc = check_launch("ns_normalize");
  if (rc) return rc;
  const int64_t chunks = n / 8;
  const int64_t blocks = chunks / 256 + 1 < 4096 ? chunks / 256 + 1 : 4096;
  hipLaunchKernelGGL(k_ns_scale_b16, dim3((unsigned)blocks), dim3(256), 0, stream, static_cast<const uint16_t*>(g),
                     n, part, static_cast<uint16_t*>(x));
  return check_launch("ns_normalize");
}

extern "C" int pratchya_ns_normalize_f32(const float* g, float* x, int64_t n, void* workspace,
                                         int64_t workspace_bytes, hipStream_t stream) {
  if (n < 0) return pratchya_set_error(PRATCHYA_EINVAL, "ns_normalize_f32: negative size");
  if (n == 0) return PRATCHYA_OK;
  if (!g || !x || !workspace) return pratchya_set_error(PRATCHYA_EINVAL, "ns_normalize_f32: null buffer");
  if (workspace_bytes < (int64_t)kNormBlocks * 4 || reinterpret_cast<uintptr_t>(workspace) % 4)
    return pratchya_set_error(PRATCHYA_EINVAL, "ns_normalize_f32: workspace of %lld bytes (need %d, 4-byte aligned)",
                              (long long)workspace_bytes, kNormBlocks * 4);
  if ((reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(x)) % 16)
    return pratchya_set_error(PRATCHYA_EINVAL, "ns_normalize_f32: g and x must be 16-byte aligned");
  float* part = static_cast<float*>(workspace);
  hipLaunchKernelGGL(k_sumsq_f32, dim3(kNormBlocks), dim3(256), 0, stream, g, n, part);
  int rc = check_launch("ns_normalize_f32");
  if (rc) return rc;
  const int64_t chunks = n / 4;
  const int64_t blocks = chunks / 256 + 1 < 4096 ? chunks / 256 + 1 : 4096;
  hipLaunchKernelGGL(k_ns_scale_f32, dim3((unsigned)blocks), dim3(256), 0, stream, g, n, part, x);
  return check_launch("ns_normalize_f32");
}

extern "C" int pratchya_apply_update(const void* u, int u_dtype, int use_sign, float scale, const void* p,
                                     int p_dtype, const uint8_t* p_sc8, const float* p_sc32, int64_t slices,
                                     int64_t H, int64_t W, int64_t a, int64_t b, int arith_dtype, float lr,
                                     float lr_wd, void* out, int out_dtype, hipStream_t stream) {
  Grid L;
  int rc = make_grid("apply_update", slices, H, W, a, b, &L);
  if (rc) return rc;
  if (!is_float_dtype(arith_dtype) || !is_float_dtype(u_dtype) || !is_float_dtype(out_dtype) ||
      (p_dtype != PRATCHYA_DT_E4M3 && !is_float_dtype(p_dtype)))
    return pratchya_set_error(PRATCHYA_EINVAL, "apply_update: unsupported dtypes (u %d, p %d, arith %d, out %d)",
                              u_dtype, p_dtype, arith_dtype, out_dtype);
  if (u_dtype == PRATCHYA_DT_F32 && arith_dtype == PRATCHYA_DT_BF16 && !use_sign)
    return pratchya_set_error(PRATCHYA_EINVAL, "apply_update: an f32 direction needs f32 arithmetic");
  if (L.n == 0) return PRATCHYA_OK;
  if (!u || !p || !out || (p_dtype == PRATCHYA_DT_E4M3 && (!p_sc8 || !p_sc32)))
    return pratchya_set_error(PRATCHYA_EINVAL, "apply_update: null buffer");
  // chunks of 16 bytes of the widest stream (u or out)
  const int wide = dtype_size(u_dtype) > dtype_size(out_dtype) ? dtype_size(u_dtype) : dtype_size(out_dtype);
  const int ch = chunk_of(L.b, {{u, dtype_size(u_dtype)}, {p, dtype_size(p_dtype)}, {out, dtype_size(out_dtype)}},
                          {16 / wide, 4});
  const int64_t chunks = L.n / ch;
  if (chunks / 256 + 1 > 0x7FFFFFFF) return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "apply_update: too many elements");
  const dim3 grid((unsigned)((chunks + 255) / 256));
  const bool bf = arith_dtype == PRATCHYA_DT_BF16, ob = out_dtype == PRATCHYA_DT_BF16;
  use_sign = use_sign ? 1 : 0;
  const int um = u_dtype == PRATCHYA_DT_BF16 ? 1 : 2;
  const int pm = p_dtype == PRATCHYA_DT_E4M3 ? 0 : (p_dtype == PRATCHYA_DT_BF16 ? 1 : 2);
  // one instantiation per (sign, u, p, arithmetic, output) combination in use
#define PRATCHYA_UPD(SG, UM, PM, BF, OB)                                                                     \
  if (use_sign == SG && um == UM && pm == PM && bf == BF && ob == OB) {                                       \
    if (ch == 8)                                                                                              \
      hipLaunchKernelGGL((k_update<SG, UM, PM, BF, OB, 8>), grid, dim3(256), 0, stream, u, p, p_sc8, p_sc32,   \
                         chunks, L.W, L.a, L.b, L.K, scale, lr, lr_wd, out);                                   \
    else if (ch == 4)                                                                                         \
      hipLaunchKernelGGL((k_update<SG, UM, PM, BF, OB, 4>), grid, dim3(256), 0, stream, u, p, p_sc8, p_sc32,   \
                         chunks, L.W, L.a, L.b, L.K, scale, lr, lr_wd, out);                                   \
    else                                                                                                      \
      hipLaunchKernelGGL((k_update<SG, UM, PM, BF, OB, 1>), grid, dim3(256), 0, stream, u, p, p_sc8, p_sc32,   \
                         chunks, L.W, L.a, L.b, L.K, scale, lr, lr_wd, out);                                   \
    return check_launch("apply_update");                                                                      \
  }
#define PRATCHYA_UPD_P(SG, UM, BF, OB) \
  PRATCHYA_UPD(SG, UM, 0, BF, OB)      \
  PRATCHYA_UPD(SG, UM, 1, BF, OB)      \
  PRATCHYA_UPD(SG, UM, 2, BF, OB)
  PRATCHYA_UPD_P(1, 1, true, true)
  PRATCHYA_UPD_P(1, 1, true, false)
  PRATCHYA_UPD_P(1, 1, false, true)
  PRATCHYA_UPD_P(1, 1, false, false)
  PRATCHYA_UPD_P(1, 2, true, true)
  PRATCHYA_UPD_P(1, 2, true, false)
  PRATCHYA_UPD_P(1, 2, false, true)
  PRATCHYA_UPD_P(1, 2, false, false)
  PRATCHYA_UPD_P(0, 1, true, true)
  PRATCHYA_UPD_P(0, 1, true, false)
  PRATCHYA_UPD_P(0, 1, false, true)
  PRATCHYA_UPD_P(0, 1, false, false)
  PRATCHYA_UPD_P(0, 2, false, true)
  PRATCHYA_UPD_P(0, 2, false, false)
#undef PRATCHYA_UPD_P
#undef PRATCHYA_UPD
  return pratchya_set_error(PRATCHYA_EINVAL, "apply_update: unsupported combination");
}
