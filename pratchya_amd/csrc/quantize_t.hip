// Transposed requantize for tgrid (128, 1): the wgrad operands.
//
// quantize_impl(x, (128, 1)) (pratchya/_qualia/_qarr.py:458-506) on x [T, C]
// (tokens x channels): blocks are 128 tokens of one channel, and with C a
// multiple of 8 a group (K = gcd(8, n_blk) = 8 blocks) is 8 adjacent channels
// of one 128-token block row.  The e8m0 bytes and group maxima are exactly
// quantize_impl's; the payload is written transposed, [C, T] per slice (each
// channel's tokens contiguous), which is the K-contiguous operand layout of
// the GEMM that contracts over tokens (dW = x^T . dY).
//
// The input is bf16 or f32, or an e4m3fn payload quantized with tgrid (1, 128)
// together with its scales; the latter is dequantized in registers exactly as
// dequantize_impl does ((f32(q) * (2^(e-127) * G)) / 128, _qarr.py:562-564),
// which is the requantization of a stored activation along the token axis
// (fp8_matmul's backward, _qarr.py:784-789, quantizes x^T the same way).
//
// One wave per 128-token x (8 * CGW)-channel tile (an fp8 input is staged
// through LDS per 128 x 128 workgroup tile, so that its global loads cover
// whole 128-byte rows).  Lane (rs, cg) holds TOK
// consecutive tokens (16 or 8) of the 8 channels of group cg: channel maxima
// are an in-lane max over TOK tokens plus xor shuffles across rs, the group
// max an in-lane max over 8 channels, and each channel's TOK payload bytes are
// one 16- or 8-byte store into the transposed layout.  The cast
// uses the same division-free scheme as the row-group quantizer (exact for
// bf16 inputs; for f32 / fp8 inputs and clamped blocks every element is
// checked against the bf16 rounding midpoint, and a lane's 16-element chunk
// holding a close one is recast with IEEE division).
//
// pratchya_quantize_t1x128: quantize_impl(x^T, (1, 128)) instead, the same
// blocks grouped 8 along the tokens of one channel (see k_quant_t128's GT
// form and k_quant_t1x128_fp8).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "fp8_math.h"
#include "pratchya_fp8.h"
#include "quant_device.h"

int pratchya_set_error(int code, const char* fmt, ...);

namespace {

// IN_BF16S: a bf16 cotangent g of a (1, 128)-quantized tensor, taken through
// dequantize_impl_bwd with that tensor's scales (bf16((g * 2^(e-127) * G) / 128),
// _qarr.py:575-601) in registers before it is requantized.
enum { IN_F32 = 0, IN_BF16 = 1, IN_FP8 = 2, IN_BF16S = 3 };

// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1 (compile-time
// channel indices, so per-channel helpers can take them as template arguments).
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

template <int IN>
struct InTraits {
  static constexpr int ESZ = IN == IN_F32 ? 4 : ((IN == IN_BF16 || IN == IN_BF16S) ? 2 : 1);
  static constexpr int NW = 2 * ESZ;        // 32-bit words holding 8 channels
};

// 8 channels of one token row at p.
template <int IN>
__device__ __forceinline__ void load_row(const uint8_t* p, uint32_t (&w)[InTraits<IN>::NW]) {
  if constexpr (IN == IN_F32) {
    const uint4 a = load_stream16(reinterpret_cast<const char*>(p));
    const uint4 b = load_stream16(reinterpret_cast<const char*>(p) + 16);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else if constexpr (IN == IN_BF16 || IN == IN_BF16S) {
    const uint4 a = load_stream16(reinterpret_cast<const char*>(p));
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  } else {
    const u32x2_t a = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    w[0] = a.x; w[1] = a.y;
  }
}

// |channel j| of a row as f32 bits, from the raw bits (a different
// expression from row_elem's, so the compiler does not keep 128 widened
// values alive from the maxima to the cast).
template <int IN, int J>
__device__ __forceinline__ uint32_t row_abs_bits(const uint32_t (&w)[InTraits<IN>::NW], float dq) {
  if constexpr (IN == IN_F32) {
    return w[J] & 0x7FFFFFFFu;
  } else if constexpr (IN == IN_BF16) {
    const uint32_t word = w[J >> 1];
    return ((J & 1) ? (word >> 16) : word) << 16 & 0x7FFF0000u;
  } else {
    const float q = fp8_elem<J>(w[J >> 2] & 0x7F7F7F7Fu);   // |q|: sign bits cleared
    return f2u((q * dq) * 0.0078125f) & 0x7FFFFFFFu;
  }
}

// Channel J of a row as f32 (fp8: dequantized with the row's scale dq, in
// dequantize_impl's order: (q * (2^(e-127) * G)) / 128).
template <int IN, int J>
__device__ __forceinline__ float row_elem(const uint32_t (&w)[InTraits<IN>::NW], float dq) {
  if constexpr (IN == IN_F32) {
    return u2f(w[J]);
  } else if constexpr (IN == IN_BF16) {
    const uint32_t word = w[J >> 1];
    return u2f((J & 1) ? (word & 0xFFFF0000u) : (word << 16));
  } else {
    return (fp8_elem<J>(w[J >> 2]) * dq) * 0.0078125f;
  }
}

// TOK consecutive tokens per lane; RS = 128 / TOK lanes cover a 128-token
// block, CGW = 64 / RS groups of 8 channels per wave.
//
// GT: quantize_impl(x^T, (1, 128)) instead (fp8_matmul's quantization of a
// transposed operand, _qarr.py:784-789) of a bf16 or f32 input: the same
// blocks (128 tokens of one channel) grouped 8 along the tokens of one
// channel (T a multiple of 1024).  A workgroup is 8 waves, one per 128-token
// block of a 1024-token group, all over the same 8 * CGW channels (one
// 128-byte line of each row); they exchange their channel maxima through LDS,
// so each channel has its own group max, and wave 0 writes each channel's 8
// e8m0 bytes (one 8-byte store) and group max.
template <int IN, bool HW, int TOK, bool GT = false>
__global__ __launch_bounds__(GT ? 512 : 256) void k_quant_t128(const uint8_t* __restrict__ x,
                                                    const uint8_t* __restrict__ x_sc8,
                                                    const float* __restrict__ x_sc32, int kg_shift,
                                                    int64_t T, int64_t C, uint8_t* __restrict__ qt,
                                                    uint8_t* __restrict__ sc8,
                                                    float* __restrict__ sc32, int tok_major) {
  constexpr int ESZ = InTraits<IN>::ESZ;
  constexpr int NW = InTraits<IN>::NW;
  const int lane = threadIdx.x & 63;
  constexpr int RS = 128 / TOK, CGW = 64 / RS;
  const int cg = lane % CGW, rs = lane / CGW;
  const int wv = (int)(threadIdx.x >> 6);
  // GT: the workgroups of neighbouring channel chunks read neighbouring bytes
  // of the same input scale rows (one byte per token row and 128 channels).
  // Workgroups are dispatched to the 8 XCDs round-robin in linear order; the
  // linear index is remapped so that neighbours run on one XCD (one L2).
  uint32_t bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
  if (!GT && tok_major) {
    // the grid's x axis walks the token blocks of one channel chunk
    bx = blockIdx.y;
    by = blockIdx.x;
  }
  if constexpr (GT) {
    const uint32_t gx = gridDim.x, gy = gridDim.y, n = gx * gy * gridDim.z;
    uint32_t b = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    if (n % 8 == 0) b = (b % 8) * (n / 8) + b / 8;
    bx = b % gx;
    by = (b / gx) % gy;
    bz = b / (gx * gy);
  }
  const int64_t c0 = GT ? (int64_t)bx * (8 * CGW) + cg * 8 : ((int64_t)bx * 4 + wv) * (8 * CGW) + cg * 8;
  // C is a multiple of 8, so a lane owns a whole group or nothing; the xor
  // partners of a lane (same cg) share its fate.  (Inputs with scales: C is a
  // multiple of 128, so a wave is wholly inside or outside; fp8 inputs: every
  // wave of the grid is inside.  Their waves outside return after the
  // workgroup barrier below.)
  constexpr bool SCALED = IN == IN_FP8 || IN == IN_BF16S;
  if constexpr (!SCALED && !GT) {
    if (c0 >= C) return;
  }
  // GT: every wave reaches the maxima exchange; lanes beyond C only skip
  // their loads and stores
  const bool live = c0 < C;
  const int64_t s = bz, tb = GT ? (int64_t)by * 8 + wv : (int64_t)by;
  const int64_t t0 = tb * 128 + rs * TOK;

  // (1, 128) input scales of the workgroup's 128 token rows and NB channel
  // blocks, loaded once per workgroup into LDS: block (t, c / 128) of the
  // slice; a slice holds a whole number of groups (kg | T * C / 128), so the
  // group of a block is its slice-global index >> kg_shift.  32-bit indices:
  // the host checks slices * T * C / 128 < 2^32.
  constexpr int NB = SCALED ? (4 * 8 * CGW) / 128 : 1;
  __shared__ float sdq[GT ? 1 : NB][GT ? 1024 : 128];
  if constexpr (SCALED && GT) {
    // the workgroup's 1024 token rows of its one 128-channel scale block
    const uint32_t nbr = (uint32_t)(C >> 7);
    const uint32_t cb = (uint32_t)(((int64_t)bx * (8 * CGW)) >> 7);
    for (int i = (int)threadIdx.x; i < 1024; i += 512) {
      const uint32_t blk = (uint32_t)(s * T + (int64_t)by * 1024 + i) * nbr + cb;
      sdq[0][i] = e8m0_decode(x_sc8[blk]) * x_sc32[blk >> kg_shift];
    }
  }
  // (not GT) staged after the payload loads are issued, so that the two
  // round trips to memory overlap (for GT, staging the 1024 rows' scales
  // after the loads measured slower: 132 vs 123 us on a scaled [32768, 4096]
  // cotangent)
  auto stage_scales = [&]() {
    if constexpr (SCALED && !GT) {
      const uint32_t nbr = (uint32_t)(C >> 7);
      const uint32_t cb0 = bx * NB;
      for (int i = (int)threadIdx.x; i < NB * 128; i += 256) {
        const uint32_t b = (uint32_t)i >> 7, row = (uint32_t)i & 127u;
        float v = 0.0f;
        if (cb0 + b < nbr) {
          const uint32_t blk = (uint32_t)(s * T + tb * 128 + row) * nbr + cb0 + b;
          v = e8m0_decode(x_sc8[blk]) * x_sc32[blk >> kg_shift];
        }
        sdq[b][row] = v;
      }
    }
  };

  uint32_t w[TOK][NW];
  if constexpr (GT) {
    // direct row loads (the waves of a workgroup cover different tokens of
    // the same channels)
    if (live) {
      const uint8_t* xr = x + ((s * T + t0) * C + c0) * ESZ;
#pragma unroll
      for (int r = 0; r < TOK; ++r) load_row<IN>(xr + (int64_t)r * C * ESZ, w[r]);
    } else {
#pragma unroll
      for (int r = 0; r < TOK; ++r)
#pragma unroll
        for (int k = 0; k < NW; ++k) w[r][k] = 0u;
    }
    if constexpr (SCALED) __syncthreads();   // the staged scales are visible
  } else if constexpr (IN == IN_FP8) {
    // A lane's rows are 8-byte pieces; read from global memory directly, a
    // wave's row segments would be 32 bytes.  The workgroup's 128 tokens x
    // 128 channels are staged through LDS instead, with 16-byte loads that
    // cover whole 128-byte rows (8 lanes per row).
    static_assert(TOK == 8 && CGW == 4, "the fp8 tile is 128 tokens x 4 waves x 32 channels");
    constexpr int kPitch = 136;              // bytes per staged row (8-byte aligned, fewer bank conflicts)
    __shared__ __attribute__((aligned(16))) uint8_t tile[128 * kPitch];
    const int64_t cw = (int64_t)bx * 128;
    const uint8_t* xt = x + (s * T + tb * 128) * C + cw;
    uint4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = i * 256 + (int)threadIdx.x, row = q >> 3, cc = (q & 7) * 16;
      v[i] = load_stream16(reinterpret_cast<const char*>(xt + (int64_t)row * C + cc));
    }
    stage_scales();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = i * 256 + (int)threadIdx.x, row = q >> 3, cc = (q & 7) * 16;
      uint2* d = reinterpret_cast<uint2*>(tile + row * kPitch + cc);
      d[0] = make_uint2(v[i].x, v[i].y);
      d[1] = make_uint2(v[i].z, v[i].w);
    }
    __syncthreads();
    const int lc = (int)(threadIdx.x >> 6) * 32 + cg * 8;   // the lane's first channel in the tile
#pragma unroll
    for (int r = 0; r < TOK; ++r) {
      const uint2 v = *reinterpret_cast<const uint2*>(tile + (rs * TOK + r) * kPitch + lc);
      w[r][0] = v.x;
      w[r][1] = v.y;
    }
  } else {
    if (!SCALED || c0 < C) {
      const uint8_t* xr = x + ((s * T + t0) * C + c0) * ESZ;
#pragma unroll
      for (int r = 0; r < TOK; ++r) load_row<IN>(xr + (int64_t)r * C * ESZ, w[r]);
    }
    if constexpr (SCALED) {
      stage_scales();
      __syncthreads();                       // the staged scales are visible
      if (c0 >= C) return;
    }
  }

  float dq[TOK];
#pragma unroll
  for (int r = 0; r < TOK; ++r) dq[r] = 1.0f;
  if constexpr (SCALED && GT) {
#pragma unroll
    for (int r = 0; r < TOK; ++r) dq[r] = sdq[0][wv * 128 + rs * TOK + r];
  } else if constexpr (SCALED) {
    const int b = (int)((c0 >> 7) - (int64_t)bx * NB);
#pragma unroll
    for (int r = 0; r < TOK; ++r) dq[r] = sdq[b][rs * TOK + r];
  }
  if constexpr (IN == IN_BF16S) {
    // the cotangent's dequantize_impl_bwd, in place: from here on the rows are
    // plain bf16 values
#pragma unroll
    for (int r = 0; r < TOK; ++r)
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const float lo = (u2f(w[r][k] << 16) * dq[r]) * 0.0078125f;
        const float hi = (u2f(w[r][k] & 0xFFFF0000u) * dq[r]) * 0.0078125f;
        w[r][k] = pack_bf16x2(lo, hi);
      }
  }
  constexpr int INC = IN == IN_BF16S ? IN_BF16 : IN;   // element kind after the prologue

  // fp8 input: each element is dequantized once, for its channel's maximum
  // and its cast (the VALU, not memory, bounds this input's kernel); the
  // other inputs recompute the cheap widening instead of holding 64 values
  constexpr bool ONCE = INC == IN_FP8;
  float vv[ONCE ? TOK : 1][ONCE ? 8 : 1];
  if constexpr (ONCE) {
    static_for<8>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
#pragma unroll
      for (int r = 0; r < TOK; ++r) vv[r][j] = row_elem<INC, j>(w[r], dq[r]);
    });
  }
  auto val = [&](auto jc, int r) -> float {
    constexpr int j = decltype(jc)::value;
    if constexpr (ONCE) return vv[r][j];
    else return row_elem<INC, j>(w[r], dq[r]);
  };
  // channel maxima (as |x| bits: unsigned order, NaN above inf) and group max
  uint32_t mx[8];
  static_for<8>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    uint32_t m = 0;
#pragma unroll
    for (int r = 0; r < TOK; ++r) {
      if constexpr (ONCE) m = umax(m, f2u(vv[r][j]) & 0x7FFFFFFFu);
      else m = umax(m, row_abs_bits<INC, j>(w[r], dq[r]));
    }
    m = strided_lane_max<CGW>(m);
    mx[j] = m;
  });
  // group maxima: of the lane's 8 channels (tgrid (128, 1)), or per channel
  // over the workgroup's 8 token blocks (GT)
  float Gc[8];
  constexpr int CPW = 8 * CGW;
  __shared__ uint32_t mxs[GT ? CPW : 1][GT ? 8 : 1];
  if constexpr (GT) {
    if (rs == 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) mxs[cg * 8 + j][wv] = mx[j];
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint4 a = *reinterpret_cast<const uint4*>(&mxs[cg * 8 + j][0]);
      const uint4 b = *reinterpret_cast<const uint4*>(&mxs[cg * 8 + j][4]);
      Gc[j] = u2f(umax(umax(umax(a.x, a.y), umax(a.z, a.w)), umax(umax(b.x, b.y), umax(b.z, b.w))));
    }
  } else {
    uint32_t Gb = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) Gb = umax(Gb, mx[j]);
#pragma unroll
    for (int j = 0; j < 8; ++j) Gc[j] = u2f(Gb);
  }

  // e8m0 bytes and y ~ 128 / S per channel; then the division-free cast,
  // chunk by chunk (channel j, this lane's 16 tokens).  A chunk is recast with
  // IEEE division when its group's G is not finite, or (f32 / fp8 inputs,
  // clamped blocks) one of its elements lands within 8 ulp of a bf16 rounding
  // midpoint after the multiply -- rare, and only that chunk pays for it.
  uint32_t e[8];
  float y[8];
  uint32_t clamped = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    // finite G: the exponent-difference e8m0 of block_scale (exact; its
    // division fallback covers subnormal and zero maxima); a non-finite G
    // takes the exact cast below, and counts as clamped for the check
    const float G = Gc[j];
    const uint32_t Gbj = f2u(G);
    if ((Gbj >> 23) < 255u) {
      const BlockScale bs = block_scale(mx[j], Gbj, __builtin_amdgcn_rcpf(G * 0.0078125f));
      e[j] = bs.e;
      y[j] = bs.y;
      clamped |= bs.clamped ? 1u : 0u;
    } else {
      e[j] = e8m0_of(u2f(mx[j]), G);
      y[j] = PRATCHYA_Y_CLAMP;
      clamped = 1u;
    }
  }
  const bool check = INC != IN_BF16 || __any(clamped);

  uint8_t* qo = qt + (s * C + c0) * T + t0;
  static_for<8>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    uint32_t o[TOK / 4];
    uint32_t key = 0xFFFFFFFFu;                  // smallest midpoint key of the chunk
#pragma unroll
    for (int k = 0; k < TOK / 4; ++k) {
      const float t0v = val(jc, 4 * k + 0) * y[j];
      const float t1v = val(jc, 4 * k + 1) * y[j];
      const float t2v = val(jc, 4 * k + 2) * y[j];
      const float t3v = val(jc, 4 * k + 3) * y[j];
      if (check) key = umin(key, mid_key4(t0v, t1v, t2v, t3v));
      o[k] = cvt4<HW>(t0v, t1v, t2v, t3v);
    }
    if (key <= kMidKey || !((f2u(Gc[j]) >> 23) < 255u)) {
      const float S = quant_scale(e[j], Gc[j]);
#pragma unroll
      for (int k = 0; k < TOK / 4; ++k)
        o[k] = cvt4_exact(val(jc, 4 * k + 0), val(jc, 4 * k + 1), val(jc, 4 * k + 2), val(jc, 4 * k + 3), S);
    }
    if (live) {
      if constexpr (TOK == 16) {
        const u32x4_t v = {o[0], o[1], o[2], o[3]};
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(qo + (int64_t)j * T));
      } else {
        static_assert(TOK == 8, "8 or 16 tokens per lane");
        const u32x2_t v = {o[0], o[1]};
        __builtin_nontemporal_store(v, reinterpret_cast<u32x2_t*>(qo + (int64_t)j * T));
      }
    }
  });
  if constexpr (GT) {
    // quantize_impl(x^T, (1, 128)) on [C, T]: block (c, tb) is c * T/128 + tb;
    // a channel's 8 blocks of this group are consecutive bytes
    if (wv == 0 && rs == 0 && live) {
      const int64_t nbr = T / 128, nb = C * nbr;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const uint32_t eb = e8m0_of(u2f(mxs[cg * 8 + j][b]), Gc[j]);
          if (b < 4) lo |= eb << (8 * b);
          else hi |= eb << (8 * (b - 4));
        }
        const int64_t c = c0 + j;
        *reinterpret_cast<u32x2_t*>(sc8 + s * nb + c * nbr + (int64_t)by * 8) = u32x2_t{lo, hi};
        sc32[s * (nb / 8) + c * (nbr / 8) + by] = Gc[j];
      }
    }
  } else if (rs == 0) {
    // blocks (tb, c0 .. c0 + 7) are consecutive; they form group (tb*C + c0) / 8
    const int64_t nb = (T / 128) * C;
    const int64_t blk = tb * C + c0;
    uint32_t* e8 = reinterpret_cast<uint32_t*>(sc8 + s * nb + blk);
    e8[0] = e[0] | (e[1] << 8) | (e[2] << 16) | (e[3] << 24);
    e8[1] = e[4] | (e[5] << 8) | (e[6] << 16) | (e[7] << 24);
    sc32[s * (nb / 8) + blk / 8] = Gc[0];
  }
}

// quantize_impl(x^T, (1, 128)) of a stored (1, 128) fp8 tensor x [T, C]
// (its dequantize_impl, Q:541-569, requantized, Q:458-506): the wgrad operand
// of the stored activation.  A workgroup takes one 128-channel column (one
// input scale block per token row) of one 1024-token group: 4 waves x 32
// channels, each lane 8 channels x 8 tokens of a 128-token block, as in
// k_quant_t128's fp8 tile.  Two passes over the group's 8 token blocks, each
// block staged through LDS with 16-byte loads of whole 128-byte rows: the
// first pass takes every channel's block maxima, the second (whose loads find
// the group in the caches) casts and stores.  The loads of the next two
// blocks are in flight while a block is processed.
__global__ __launch_bounds__(256) void k_quant_t1x128_fp8(const uint8_t* __restrict__ x,
                                                          const uint8_t* __restrict__ x_sc8,
                                                          const float* __restrict__ x_sc32, int kg_shift,
                                                          int64_t T, int64_t C, uint8_t* __restrict__ qt,
                                                          uint8_t* __restrict__ sc8, float* __restrict__ sc32) {
  constexpr int TOK = 8, CGW = 4, kPitch = 136;
  const int lane = threadIdx.x & 63, wv = (int)(threadIdx.x >> 6);
  const int cg = lane % CGW, rs = lane / CGW;
  // workgroups of neighbouring columns share no lines here, but those of one
  // XCD share its L2 for the second pass: consecutive columns on one XCD
  uint32_t b = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  const uint32_t n = gridDim.x * gridDim.y * gridDim.z;
  if (n % 8 == 0) b = (b % 8) * (n / 8) + b / 8;
  const uint32_t bx = b % gridDim.x, by = (b / gridDim.x) % gridDim.y, bz = b / (gridDim.x * gridDim.y);
  const int lc = wv * 32 + cg * 8;                 // the lane's first channel in the column
  const int64_t s = bz, tg = (int64_t)by * 1024;   // slice, first token of the group
  __shared__ float sdq[1024];                      // input scale of each token row (this column's block)
  __shared__ __attribute__((aligned(16))) uint8_t tile[128 * kPitch];
  __shared__ __attribute__((aligned(16))) uint32_t bm[128][8];   // block maxima, |x| bits
  {
    const uint32_t nbr = (uint32_t)(C >> 7);
    for (int i = (int)threadIdx.x; i < 1024; i += 256) {
      const uint32_t blk = (uint32_t)(s * T + tg + i) * nbr + bx;
      sdq[i] = e8m0_decode(x_sc8[blk]) * x_sc32[blk >> kg_shift];
    }
  }
  const uint8_t* xg = x + (s * T + tg) * C + (int64_t)bx * 128;
  // 16-byte pieces of block tb: thread t loads rows (i * 256 + t) / 8, i < 4;
  // two blocks are in flight ahead of the one processed
  uint4 v[2][4];
  auto load_block = [&](int tb, uint4 (&vv)[4]) {
    const uint8_t* xt = xg + (int64_t)tb * 128 * C;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = i * 256 + (int)threadIdx.x;
      vv[i] = load_stream16(reinterpret_cast<const char*>(xt + (int64_t)(q >> 3) * C + (q & 7) * 16));
    }
  };
  // block tb's tile into LDS (after every wave is done with the previous
  // one), the loads of block `next` into the freed registers, and the lane's
  // 8 tokens x 8 channels with their input scales out of the tile
  uint32_t w[TOK][2];
  float dq[TOK];
  auto stage = [&](int tb, uint4 (&vc)[4], int next) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = i * 256 + (int)threadIdx.x;
      uint2* d = reinterpret_cast<uint2*>(tile + (q >> 3) * kPitch + (q & 7) * 16);
      d[0] = make_uint2(vc[i].x, vc[i].y);
      d[1] = make_uint2(vc[i].z, vc[i].w);
    }
    if (next < 8) load_block(next, vc);
    __syncthreads();
#pragma unroll
    for (int r = 0; r < TOK; ++r) {
      const uint2 t2 = *reinterpret_cast<const uint2*>(tile + (rs * TOK + r) * kPitch + lc);
      w[r][0] = t2.x;
      w[r][1] = t2.y;
      dq[r] = sdq[tb * 128 + rs * TOK + r];
    }
  };
  load_block(0, v[0]);
  load_block(1, v[1]);
  // pass 1: the block maxima of the lane's 8 channels (the last two blocks'
  // loads start the second pass: blocks 0 and 1 again)
#pragma unroll 2
  for (int tb = 0; tb < 8; ++tb) {
    stage(tb, v[tb & 1], tb + 2 < 8 ? tb + 2 : tb - 6);
    static_for<8>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      uint32_t m = 0;
#pragma unroll
      for (int r = 0; r < TOK; ++r) m = umax(m, row_abs_bits<IN_FP8, j>(w[r], dq[r]));
      m = strided_lane_max<CGW>(m);
      if (rs == 0) bm[lc + j][tb] = m;
    });
  }
  __syncthreads();
  // group maxima; the lanes of token sub-block 0 write the scales: a channel's
  // 8 e8m0 bytes of this group are consecutive (block (c, tb) of x^T [C, T]
  // is c * T/128 + tb)
  float Gc[8];
  {
    const int64_t nbr = T / 128, nb = C * nbr;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint4 a = *reinterpret_cast<const uint4*>(&bm[lc + j][0]);
      const uint4 c = *reinterpret_cast<const uint4*>(&bm[lc + j][4]);
      Gc[j] = u2f(umax(umax(umax(a.x, a.y), umax(a.z, a.w)), umax(umax(c.x, c.y), umax(c.z, c.w))));
      if (rs == 0) {
        const uint32_t lo = e8m0_of(u2f(a.x), Gc[j]) | (e8m0_of(u2f(a.y), Gc[j]) << 8) |
                            (e8m0_of(u2f(a.z), Gc[j]) << 16) | (e8m0_of(u2f(a.w), Gc[j]) << 24);
        const uint32_t hi = e8m0_of(u2f(c.x), Gc[j]) | (e8m0_of(u2f(c.y), Gc[j]) << 8) |
                            (e8m0_of(u2f(c.z), Gc[j]) << 16) | (e8m0_of(u2f(c.w), Gc[j]) << 24);
        const int64_t ch = (int64_t)bx * 128 + lc + j;
        *reinterpret_cast<u32x2_t*>(sc8 + s * nb + ch * nbr + (int64_t)by * 8) = u32x2_t{lo, hi};
        sc32[s * (nb / 8) + ch * (nbr / 8) + by] = Gc[j];
      }
    }
  }
  // pass 2: the cast of each block (the arithmetic of k_quant_t128)
  uint8_t* const qo = qt + (s * C + (int64_t)bx * 128 + lc) * T + tg + rs * TOK;
#pragma unroll 2
  for (int tb = 0; tb < 8; ++tb) {
    stage(tb, v[tb & 1], tb + 2);
    static_for<8>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      const float G = Gc[j];
      const uint32_t Gbj = f2u(G), mb = bm[lc + j][tb];
      uint32_t e;
      float y;
      if ((Gbj >> 23) < 255u) {                 // finite: exponent-difference e8m0
        const BlockScale bs = block_scale(mb, Gbj, __builtin_amdgcn_rcpf(G * 0.0078125f));
        e = bs.e;
        y = bs.y;
      } else {                                  // the exact cast below
        e = e8m0_of(u2f(mb), G);
        y = PRATCHYA_Y_CLAMP;
      }
      uint32_t o[TOK / 4];
      uint32_t key = 0xFFFFFFFFu;                // smallest midpoint key of the chunk
#pragma unroll
      for (int k = 0; k < TOK / 4; ++k) {
        const float t0v = row_elem<IN_FP8, j>(w[4 * k + 0], dq[4 * k + 0]) * y;
        const float t1v = row_elem<IN_FP8, j>(w[4 * k + 1], dq[4 * k + 1]) * y;
        const float t2v = row_elem<IN_FP8, j>(w[4 * k + 2], dq[4 * k + 2]) * y;
        const float t3v = row_elem<IN_FP8, j>(w[4 * k + 3], dq[4 * k + 3]) * y;
        key = umin(key, mid_key4(t0v, t1v, t2v, t3v));
        o[k] = cvt4<true>(t0v, t1v, t2v, t3v);
      }
      if (key <= kMidKey || !((f2u(G) >> 23) < 255u)) {
        const float S = quant_scale(e, G);
#pragma unroll
        for (int k = 0; k < TOK / 4; ++k)
          o[k] = cvt4_exact(row_elem<IN_FP8, j>(w[4 * k + 0], dq[4 * k + 0]),
                            row_elem<IN_FP8, j>(w[4 * k + 1], dq[4 * k + 1]),
                            row_elem<IN_FP8, j>(w[4 * k + 2], dq[4 * k + 2]),
                            row_elem<IN_FP8, j>(w[4 * k + 3], dq[4 * k + 3]), S);
      }
      const u32x2_t ov = {o[0], o[1]};
      __builtin_nontemporal_store(ov, reinterpret_cast<u32x2_t*>(qo + (int64_t)j * T + tb * 128));
    });
  }
}

// quantize_impl(x, (128, 1)) with the payload in x's own layout [slices, T,
// C] (the K-major operand of the weight-gradient GEMM): no transposition, so
// each thread owns one group (8 channels) of 8 token rows of a 128-token x
// 128-channel tile, and 16 threads cover a row's 128 channels with
// consecutive pieces (whole 128-byte lines for fp8 payloads and bf16 rows).
// Thread t of the 256: group t % 16, token rows t / 16 + 16 i (i < 8).
// Channel maxima: an in-thread max over the 8 rows, the 4 lanes of a wave
// sharing the group (row swaps), then the 4 waves through LDS.  The cast is
// k_quant_t128's (the same e8m0 bytes, y and midpoint check), row by row.  A
// workgroup walks nblk consecutive token blocks of its column, the next
// block's loads issued after the current block's stores (prefetching the next
// block into registers measured slower: 83 vs 76 us on config 4's dY, the
// extra registers cost a wave per SIMD).
#ifndef PRATCHYA_ROWS_WGS
#define PRATCHYA_ROWS_WGS 2048   // workgroups the token blocks are spread over
#endif
// threads of k_quant_128x1_rows<IN, R>'s workgroup: 32 / R waves
constexpr int rows_threads(int R) { return 2048 / R; }

template <int IN, int R>
__global__ __launch_bounds__(rows_threads(R)) void k_quant_128x1_rows(const uint8_t* __restrict__ x,
                                                          const uint8_t* __restrict__ x_sc8,
                                                          const float* __restrict__ x_sc32, int kg_shift,
                                                          int64_t T, int64_t C, int nblk, uint8_t* __restrict__ q,
                                                          uint8_t* __restrict__ sc8, float* __restrict__ sc32) {
  constexpr int ESZ = InTraits<IN>::ESZ, NW = InTraits<IN>::NW;
  constexpr bool SCALED = IN == IN_FP8 || IN == IN_BF16S;
  constexpr int INC = IN == IN_BF16S ? IN_BF16 : IN;
  // R token rows per thread and block: NWV = 32 / R waves, token rows
  // rr + SR * i with rr < SR = 128 / R
  static_assert(R == 4 || R == 8, "4 or 8 token rows per thread");
  constexpr int NWV = 32 / R, SR = 128 / R;
  static_assert(NWV * 64 == rows_threads(R), "the workgroup is NWV waves");
  const int lane = (int)threadIdx.x & 63, wv = (int)(threadIdx.x >> 6);
  const int grp = lane & 15, rr = wv * 4 + (lane >> 4);
  const int64_t s = blockIdx.z;
  const int64_t c0 = (int64_t)blockIdx.x * 128 + grp * 8;
  const bool live = c0 < C;                   // C is a multiple of 8: whole groups
  const int64_t nbr = T / 128, nb = nbr * C;
  const int64_t tb0 = (int64_t)blockIdx.y * nblk;
  const int64_t tb1 = tb0 + nblk < nbr ? tb0 + nblk : nbr;
  // input scale blocks of a token row: C / 128 (scaled inputs); this
  // workgroup's column is block blockIdx.x of each row.  32-bit indices: the
  // host checks slices * T * C / 128 < 2^32.
  const uint32_t nsr = (uint32_t)(C >> 7);
  __shared__ __attribute__((aligned(16))) uint32_t smx[2][NWV][128];

  uint32_t w[R][NW];
  uint32_t se[R];
  float sg[R];
  auto load_block = [&](int64_t tb, uint32_t (&wd)[R][NW], uint32_t (&sed)[R], float (&sgd)[R]) {
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int64_t t = tb * 128 + rr + SR * i;
      if (live) {
        load_row<IN>(x + ((s * T + t) * C + c0) * ESZ, wd[i]);
      } else {
#pragma unroll
        for (int k = 0; k < NW; ++k) wd[i][k] = 0u;
      }
      if constexpr (SCALED) {
        const uint32_t blk = (uint32_t)(s * T + t) * nsr + blockIdx.x;
        sed[i] = x_sc8[blk];
        sgd[i] = x_sc32[blk >> kg_shift];
      }
    }
  };
  load_block(tb0, w, se, sg);
  int par = 0;
  for (int64_t tb = tb0; tb < tb1; ++tb, par ^= 1) {
    float dq[R];
#pragma unroll
    for (int i = 0; i < R; ++i) dq[i] = SCALED ? e8m0_decode(se[i]) * sg[i] : 1.0f;
    if constexpr (IN == IN_BF16S) {
      // the cotangent's dequantize_impl_bwd, in place (as in k_quant_t128)
#pragma unroll
      for (int i = 0; i < R; ++i)
#pragma unroll
        for (int k = 0; k < NW; ++k) {
          const float lo = (u2f(w[i][k] << 16) * dq[i]) * 0.0078125f;
          const float hi = (u2f(w[i][k] & 0xFFFF0000u) * dq[i]) * 0.0078125f;
          w[i][k] = pack_bf16x2(lo, hi);
        }
    }
    constexpr bool ONCE = INC == IN_FP8;
    float vv[ONCE ? R : 1][ONCE ? 8 : 1];
    if constexpr (ONCE) {
      static_for<8>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
#pragma unroll
        for (int i = 0; i < R; ++i) vv[i][j] = row_elem<INC, j>(w[i], dq[i]);
      });
    }
    auto val = [&](auto jc, int i) -> float {
      constexpr int j = decltype(jc)::value;
      if constexpr (ONCE) return vv[i][j];
      else return row_elem<INC, j>(w[i], dq[i]);
    };
    // channel maxima (|x| bits): 8 rows in-thread, 4 lanes, then 4 waves
    uint32_t mx[8];
    static_for<8>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      uint32_t m = 0;
#pragma unroll
      for (int i = 0; i < R; ++i) {
        if constexpr (ONCE) m = umax(m, f2u(vv[i][j]) & 0x7FFFFFFFu);
        else m = umax(m, row_abs_bits<INC, j>(w[i], dq[i]));
      }
      mx[j] = xor_max_u32<32>(xor_max_u32<16>(m));
    });
    if (lane < 16) {
      uint4* d = reinterpret_cast<uint4*>(&smx[par][wv][grp * 8]);
      d[0] = make_uint4(mx[0], mx[1], mx[2], mx[3]);
      d[1] = make_uint4(mx[4], mx[5], mx[6], mx[7]);
    }
    __syncthreads();
#pragma unroll
    for (int v = 0; v < NWV; ++v) {
      const uint4 a = *reinterpret_cast<const uint4*>(&smx[par][v][grp * 8]);
      const uint4 b = *reinterpret_cast<const uint4*>(&smx[par][v][grp * 8 + 4]);
      mx[0] = umax(mx[0], a.x); mx[1] = umax(mx[1], a.y); mx[2] = umax(mx[2], a.z); mx[3] = umax(mx[3], a.w);
      mx[4] = umax(mx[4], b.x); mx[5] = umax(mx[5], b.y); mx[6] = umax(mx[6], b.z); mx[7] = umax(mx[7], b.w);
    }
    // the group max, e8m0 bytes and y per channel (k_quant_t128's scheme)
    uint32_t Gb = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) Gb = umax(Gb, mx[j]);
    const float G = u2f(Gb);
    const bool fin = (Gb >> 23) < 255u;
    const float rG = __builtin_amdgcn_rcpf(G * 0.0078125f);
    uint32_t e[8];
    float y[8];
    uint32_t clamped = fin ? 0u : 1u;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (fin) {
        const BlockScale bs = block_scale(mx[j], Gb, rG);
        e[j] = bs.e;
        y[j] = bs.y;
        clamped |= bs.clamped ? 1u : 0u;
      } else {
        e[j] = e8m0_of(u2f(mx[j]), G);
        y[j] = PRATCHYA_Y_CLAMP;
      }
    }
    const bool check = INC != IN_BF16 || __any(clamped);
#pragma unroll
    for (int i = 0; i < R; ++i) {
      float t[8];
      static_for<8>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        t[j] = val(jc, i) * y[j];
      });
      uint32_t lo = cvt4<true>(t[0], t[1], t[2], t[3]), hi = cvt4<true>(t[4], t[5], t[6], t[7]);
      const uint32_t key = check ? umin(mid_key4(t[0], t[1], t[2], t[3]), mid_key4(t[4], t[5], t[6], t[7]))
                                 : 0xFFFFFFFFu;
      if (key <= kMidKey || !fin) {
        uint32_t b[8];
        static_for<8>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          b[j] = quant_elem_exact(val(jc, i), quant_scale(e[j], G));
        });
        lo = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
        hi = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
      }
      if (live) store_stream8(q + (s * T + tb * 128 + rr + SR * i) * C + c0, u32x2_t{lo, hi});
    }
    if (wv == 0 && lane < 16 && live) {
      // blocks (tb, c0 .. c0 + 7) are consecutive bytes; they form group (tb*C + c0) / 8
      const int64_t blk = tb * C + c0;
      store_stream8(sc8 + s * nb + blk, u32x2_t{e[0] | (e[1] << 8) | (e[2] << 16) | (e[3] << 24),
                                                e[4] | (e[5] << 8) | (e[6] << 16) | (e[7] << 24)});
      sc32[s * (nb / 8) + blk / 8] = G;
    }
    if (tb + 1 < tb1) load_block(tb + 1, w, se, sg);
  }
}

// The activation quantize and the weight gradient's requantization of it in
// one pass: (q, sc8, sc32) = quantize_impl(x, (1, 128)) (Q:458-506, the
// quantized Linear's input, M:46-50) and (q2, sc8b, sc32b) =
// quantize_impl(dequantize_impl(q, sc8, sc32), (128, 1)) (Q:541-569 then
// Q:458-506: the stored activation requantized along the tokens for the FP8
// weight gradient, fp8_matmul's scheme Q:784-789), q2 in x's own [T, C]
// layout.  Bit-identical to pratchya_quantize followed by
// pratchya_quantize_128x1 of its payload.
//
// A workgroup of 8 waves owns 128 tokens x 1024 channels (one (1, 128) group
// of each of its tokens, 128 (128, 1) groups).  Wave w takes tokens 16w ..
// 16w + 15 and lane l the channels 16l .. 16l + 15 (one 128-channel block per
// 8 lanes) in both phases, so each lane reads back only bytes it wrote.
// Phase 1, token by token (the next two tokens' loads in flight): block
// maxima over 8 lanes, the group max from the 8 block leaders
// (wave-uniform), the cast, the payload row stored (1 KB per wave), the
// block's dequantization factor 2^(e-127) * G to LDS, and a running maximum
// of each channel's dequantized values (dequantize_impl's (f32(q) * dq) /
// 128).  The channel maxima over the 128 tokens meet in LDS by atomic max;
// each lane then forms its two 8-channel groups' maxima, e8m0 bytes and y.
// Phase 2, token by token: the lane reloads its 16 payload bytes (just
// written, from the cache), dequantizes, casts with the division-free scheme
// (every element checked against the bf16 rounding midpoint, a close one
// recast exactly), and stores the second payload.  Nothing but running maxima
// is held between the phases, so several workgroups share a CU and one's
// arithmetic overlaps another's memory traffic.  C must be a multiple of 1024
// and the token count of 128 (slices flatten into tokens).
template <bool IS_BF16>
__global__ __launch_bounds__(512) void k_quant_dual(const void* __restrict__ xv, int64_t C,
                                                    uint8_t* __restrict__ q, uint8_t* __restrict__ sc8,
                                                    float* __restrict__ sc32, uint8_t* __restrict__ q2,
                                                    uint8_t* __restrict__ sc8b, float* __restrict__ sc32b) {
  constexpr int ESZ = IS_BF16 ? 2 : 4;
  constexpr int NV = ESZ;                       // 16-byte loads per token and lane (16 channels)
  constexpr int TK = 16;                        // tokens per wave
  const int lane = (int)threadIdx.x & 63, wv = (int)(threadIdx.x >> 6);
  const int64_t cg = blockIdx.x, tb = blockIdx.y;
  const int64_t c0 = cg * 1024 + lane * 16;     // the lane's first channel
  const int tw = wv * TK;                       // the wave's first token in the tile
  const int64_t t0 = tb * 128 + tw;
  const int64_t ngc = C >> 10;                  // (1, 128) groups per token row
  const char* xb = static_cast<const char*>(xv);
  __shared__ float dqt[128][8];                 // per token and block: 2^(e-127) * G
  __shared__ __attribute__((aligned(16))) uint32_t cmx[1024];       // channel maxima (|x| bits)
  // the (1, 128) scale arrays as raw buffers (byte counts below 2^31, checked
  // on the host): every lane issues the scale stores, lanes other than 0 past
  // the end, so that the loop's wait for the next tokens' loads does not
  // also wait for them
  const int64_t n_groups = (int64_t)gridDim.y * 128 * ngc;
  const __amdgpu_buffer_rsrc_t r8 = __builtin_amdgcn_make_buffer_rsrc(sc8, 0, (int)(n_groups * 8), kRawBuffer);
  const __amdgpu_buffer_rsrc_t r32 = __builtin_amdgcn_make_buffer_rsrc(sc32, 0, (int)(n_groups * 4), kRawBuffer);

  cmx[threadIdx.x] = 0u;
  cmx[threadIdx.x + 512] = 0u;

  // ---- phase 1: quantize_impl(x, (1, 128)) token by token ----
  auto load_tok = [&](int i, uint4 (&v)[NV]) {
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = load_stream16(xb + ((t0 + i) * C + c0) * ESZ + 16 * k);
  };
  uint32_t mx[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) mx[j] = 0u;
  // two token buffers used alternately (no register copy waits for a load in
  // flight); the loads are unconditional, so the count in flight is fixed
  uint4 va[NV], vb[NV];
  load_tok(0, va);
  load_tok(1, vb);
  auto quant_tok = [&](int i, const uint4 (&v)[NV]) {
    uint32_t lm = 0;
#pragma unroll
    for (int k = 0; k < NV; ++k) lm = umax(lm, IS_BF16 ? absmax8_bf16(v[k]) : vec_absmax_bits<false>(v[k]));
    const uint32_t mb = lane_group_max<8>(lm);            // this lane's block max
    uint32_t Gb = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) Gb = umax(Gb, readlane_u32(mb, 8 * k));
    const float G = u2f(Gb);
    float x[16];
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int j = 0; j < 16 / NV; ++j) x[k * (16 / NV) + j] = elem_f32<IS_BF16>(v[k], j);
    uint32_t e, w4[4];
    if ((Gb >> 23) < 255u) {
      const BlockScale bs = block_scale(mb, Gb, __builtin_amdgcn_rcpf(G * 0.0078125f));
      e = bs.e;
      const bool check = !IS_BF16 || __any(bs.clamped ? 1 : 0);
      uint32_t key = 0xFFFFFFFFu;
      float tt[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) tt[k] = x[k] * bs.y;
#pragma unroll
      for (int w = 0; w < 4; ++w) w4[w] = cvt4_hw(tt[4 * w], tt[4 * w + 1], tt[4 * w + 2], tt[4 * w + 3]);
      if (check) {
#pragma unroll
        for (int w = 0; w < 4; ++w) key = umin(key, mid_key4(tt[4 * w], tt[4 * w + 1], tt[4 * w + 2], tt[4 * w + 3]));
      }
      // a product near a bf16 rounding midpoint: the token's cast redone
      // exactly by the whole wave (a wave-uniform branch, skipped as a whole
      // otherwise; the exact cast equals the fast one wherever that is valid)
      if (check && __any(key <= kMidKey ? 1 : 0)) {
        const float S = quant_scale(e, G);
#pragma unroll
        for (int w = 0; w < 4; ++w) w4[w] = cvt4_exact(x[4 * w], x[4 * w + 1], x[4 * w + 2], x[4 * w + 3], S);
      }
    } else {
      e = e8m0_of(u2f(mb), G);
      const float S = quant_scale(e, G);
#pragma unroll
      for (int w = 0; w < 4; ++w) w4[w] = cvt4_exact(x[4 * w], x[4 * w + 1], x[4 * w + 2], x[4 * w + 3], S);
    }
    const int64_t t = t0 + i;
    // an ordinary store: phase 2 reads these bytes back from the cache
    *reinterpret_cast<u32x4_t*>(q + t * C + c0) = u32x4_t{w4[0], w4[1], w4[2], w4[3]};
    const float dqi = e8m0_decode(e) * G;
    if ((lane & 7) == 0) dqt[tw + i][lane >> 3] = dqi;
    // running channel maxima of f32(|q|) * dq (= |f32(q) * dq|, dq >= 0); the
    // dequantized value divides that by 128, which keeps the order (rounding
    // is monotonic), so the maxima are scaled once after the exchange
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      float d[4];
      fp8_word(w4[w] & 0x7F7F7F7Fu, d[0], d[1], d[2], d[3]);
#pragma unroll
      for (int b = 0; b < 4; ++b) mx[4 * w + b] = umax(mx[4 * w + b], f2u(d[b] * dqi));
    }
    // the group's 8 e8m0 bytes (block k: leader lane 8k) and G
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t ek = readlane_u32(e, 8 * k);
      if (k < 4) lo |= ek << (8 * k);
      else hi |= ek << (8 * (k - 4));
    }
    const int gi = (int)(t * ngc + cg);
    __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{lo, hi}, r8, lane == 0 ? gi * 8 : kOutOfRange, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b32(f2u(G), r32, lane == 0 ? gi * 4 : kOutOfRange, 0, 0);
  };
#pragma unroll 1
  for (int i = 0; i < TK; i += 2) {
    quant_tok(i, va);
    load_tok(i + 2 < TK ? i + 2 : TK - 1, va);
    quant_tok(i + 1, vb);
    load_tok(i + 3 < TK ? i + 3 : TK - 1, vb);
  }
  __syncthreads();                              // cmx cleared by every thread
#pragma unroll
  for (int j = 0; j < 16; ++j) atomicMax(&cmx[lane * 16 + j], mx[j]);
  __syncthreads();
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint4 a = *reinterpret_cast<const uint4*>(&cmx[lane * 16 + 4 * w]);
    const uint32_t m4[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int b = 0; b < 4; ++b) mx[4 * w + b] = f2u(u2f(m4[b]) * 0.0078125f) & 0x7FFFFFFFu;
  }

  // ---- phase 2: quantize_impl(dequantize_impl(q), (128, 1)) ----
  // the two 8-channel groups of the lane: group max, e8m0 bytes (packed, 4
  // per word) and y per channel
  uint32_t ew[4] = {0u, 0u, 0u, 0u};
  float y2[16], Gh[2];
  bool finh[2];
#pragma unroll
  for (int gh = 0; gh < 2; ++gh) {
    uint32_t Gb = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) Gb = umax(Gb, mx[8 * gh + j]);
    const float G = u2f(Gb);
    Gh[gh] = G;
    finh[gh] = (Gb >> 23) < 255u;
    const float rG = __builtin_amdgcn_rcpf(G * 0.0078125f);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint32_t ej;
      if (finh[gh]) {
        const BlockScale bs = block_scale(mx[8 * gh + j], Gb, rG);
        ej = bs.e;
        y2[8 * gh + j] = bs.y;
      } else {
        ej = e8m0_of(u2f(mx[8 * gh + j]), G);
        y2[8 * gh + j] = PRATCHYA_Y_CLAMP;
      }
      ew[(8 * gh + j) >> 2] |= ej << (8 * (j & 3));
    }
  }
  // the lane's payload bytes of the next two tokens in flight (alternating
  // buffers, unconditional loads, as in phase 1)
  auto load_q = [&](int i) { return *reinterpret_cast<const u32x4_t*>(q + (t0 + i) * C + c0); };
  u32x4_t pa = load_q(0), pb = load_q(1);
  // ONE: (f32(q) * dq) / 128 as f32(q) * (dq / 128), exact for every q when
  // dequant_one_mul(dq) holds (taken when it does on the whole wave)
  auto requant_body = [&](auto one_c, int i, const u32x4_t wq, float dqi) {
    constexpr bool ONE = decltype(one_c)::value;
    const int64_t t = t0 + i;
    const float dqx = ONE ? dqi * 0.0078125f : dqi;
    const uint32_t qw[4] = {wq.x, wq.y, wq.z, wq.w};
    uint32_t out[4];
#pragma unroll
    for (int gh = 0; gh < 2; ++gh) {
      float d[8], tv[8];
      fp8_word(qw[2 * gh], d[0], d[1], d[2], d[3]);
      fp8_word(qw[2 * gh + 1], d[4], d[5], d[6], d[7]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        d[j] = ONE ? d[j] * dqx : (d[j] * dqx) * 0.0078125f;
        tv[j] = d[j] * y2[8 * gh + j];
      }
      out[2 * gh] = cvt4<true>(tv[0], tv[1], tv[2], tv[3]);
      out[2 * gh + 1] = cvt4<true>(tv[4], tv[5], tv[6], tv[7]);
      const uint32_t key = umin(mid_key4(tv[0], tv[1], tv[2], tv[3]), mid_key4(tv[4], tv[5], tv[6], tv[7]));
      // the exact cast by the whole wave when a lane needs it (a wave-uniform
      // branch; the exact cast equals the fast one wherever that is valid)
      if (__any((key <= kMidKey || !finh[gh]) ? 1 : 0)) {
        const uint32_t elo = ew[2 * gh], ehi = ew[2 * gh + 1];
        uint32_t b[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          b[j] = quant_elem_exact(d[j], quant_scale(((j < 4 ? elo : ehi) >> (8 * (j & 3))) & 0xFFu, Gh[gh]));
        out[2 * gh] = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
        out[2 * gh + 1] = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
      }
    }
    store_stream16(q2 + t * C + c0, u32x4_t{out[0], out[1], out[2], out[3]});
  };
  auto requant_tok = [&](int i, const u32x4_t wq) {
    const float dqi = dqt[tw + i][lane >> 3];
    if (__all(dequant_one_mul(dqi) ? 1 : 0)) requant_body(std::true_type{}, i, wq, dqi);
    else requant_body(std::false_type{}, i, wq, dqi);
  };
#pragma unroll 1
  for (int i = 0; i < TK; i += 2) {
    requant_tok(i, pa);
    pa = load_q(i + 2 < TK ? i + 2 : TK - 1);
    requant_tok(i + 1, pb);
    pb = load_q(i + 3 < TK ? i + 3 : TK - 1);
  }
  if (wv == 0) {
    // blocks (tb, c0 .. c0 + 15) are consecutive bytes: groups (tb * C + c0) / 8 and the next
    const int64_t blk = tb * C + c0;
    store_stream16(sc8b + blk, u32x4_t{ew[0], ew[1], ew[2], ew[3]});
    store_stream8(reinterpret_cast<uint8_t*>(sc32b + blk / 8), u32x2_t{f2u(Gh[0]), f2u(Gh[1])});
  }
}

int64_t gcd64(int64_t a, int64_t b) {
  while (b) {
    const int64_t t = a % b;
    a = b;
    b = t;
  }
  return a;
}

}  // namespace

namespace {

// pratchya_quantize_t128 (rows = false: payload [C, T] per slice) and
// pratchya_quantize_128x1 (rows = true: payload [T, C], x's own layout):
// the same checks and outputs but for the payload's layout.
int quantize_128x1_impl(bool rows, const void* x, int x_dtype, const uint8_t* x_sc8, const float* x_sc32,
                        int64_t slices, int64_t T, int64_t C, uint8_t* xt_fp8, uint8_t* sc_fp8, float* sc_fp32,
                        hipStream_t stream) {
  const char* name = rows ? "quantize_128x1" : "quantize_t128";
  if (slices < 0 || T < 0 || C < 0) return pratchya_set_error(PRATCHYA_EINVAL, "%s: negative size", name);
  if (x_dtype != PRATCHYA_DT_F32 && x_dtype != PRATCHYA_DT_BF16 && x_dtype != PRATCHYA_DT_E4M3)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: unsupported input dtype %d", name, x_dtype);
  if (T % 128)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: tgrid (128, 1) does not divide %lld tokens", name,
                              (long long)T);
  // an fp8 payload, or a bf16 cotangent given with scales: (1, 128) input scales
  const bool scaled = x_dtype == PRATCHYA_DT_E4M3 || (x_dtype == PRATCHYA_DT_BF16 && x_sc8 && x_sc32);
  if (scaled && C % 128)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: tgrid (1, 128) of the input scales does not divide "
                              "%lld channels", name, (long long)C);
  if (slices == 0 || T == 0 || C == 0) return PRATCHYA_OK;
  if (C % 8)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: channels must be a multiple of 8 (got %lld)", name,
                              (long long)C);
  if (!x || !xt_fp8 || !sc_fp8 || !sc_fp32 || (x_dtype == PRATCHYA_DT_E4M3 && (!x_sc8 || !x_sc32)))
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: null buffer", name);
  const uintptr_t xa = reinterpret_cast<uintptr_t>(x);
  if (xa % 16 || reinterpret_cast<uintptr_t>(xt_fp8) % 16 ||
      reinterpret_cast<uintptr_t>(sc_fp8) % (rows ? 8 : 4) || reinterpret_cast<uintptr_t>(sc_fp32) % 4)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: buffers are not aligned", name);
  if (T / 128 > 65535 || slices > 65535)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: too many token blocks or slices", name);
  if (scaled && (slices * T) * (C / 128) >= ((int64_t)1 << 32))
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: input scales beyond 2^32 blocks", name);
  // 16 tokens per lane (64 channels per wave, 128-byte row segments) for bf16
  // inputs; 8 (32 channels per wave, half the registers) for the VALU-heavier
  // f32 and fp8 inputs, where occupancy matters more than segment length
  // (measured on [16384, 2048] and [16384, 8192]: bf16 85 vs 106 us, fp8 44 vs
  // 36 us, f32 57 vs 48 us for 16 vs 8 tokens)
  // bf16 inputs of 8192 channels or more walk the token blocks of one channel
  // chunk along the grid's x axis (measured on [32768, 16384] with scales:
  // 365 -> 291 us; slower for fewer channels and for fp8 inputs)
  const int tok_major = x_dtype == PRATCHYA_DT_BF16 && C >= 8192 && C / 256 <= 65535 ? 1 : 0;
  auto grid_for_tok = [&](int tok) {
    const int cpw = 8 * (64 / (128 / tok));             // channels per wave
    const unsigned nc = (unsigned)((C + 4 * cpw - 1) / (4 * cpw)), nt = (unsigned)(T / 128);
    return tok_major ? dim3(nt, nc, (unsigned)slices) : dim3(nc, nt, (unsigned)slices);
  };
  const uint8_t* xb = static_cast<const uint8_t*>(x);
  // blocks per group of a (1, 128) input: gcd(8, n_blk), a power of two
  const int64_t kg = scaled ? gcd64(8, T * (C / 128)) : 1;
  const int kg_shift = kg == 8 ? 3 : (kg == 4 ? 2 : (kg == 2 ? 1 : 0));
  if (rows) {
    // a workgroup per 128-channel column and nblk token blocks: about 2048
    // workgroups (measured on config 4's dY: 76 us, one block per workgroup
    // 78 us)
    const int64_t ncol = (C + 127) / 128, nbr = T / 128;
    int64_t nblk = (ncol * nbr * slices) / PRATCHYA_ROWS_WGS;
    nblk = nblk < 1 ? 1 : (nblk > 8 ? 8 : nblk);
    const dim3 grid((unsigned)ncol, (unsigned)((nbr + nblk - 1) / nblk), (unsigned)slices);
    const int nb_i = (int)nblk;
    // 8 token rows per thread (4 measured slower at 8 waves per workgroup and
    // 4-5 waves per SIMD: config 4's dY 81 vs 76 us, its fp8 activation 35 vs
    // 32 us)
    constexpr int RF = 8, RB = 8;
    if (x_dtype == PRATCHYA_DT_BF16 && scaled)
      hipLaunchKernelGGL((k_quant_128x1_rows<IN_BF16S, RB>), grid, dim3(rows_threads(RB)), 0, stream, xb, x_sc8, x_sc32, kg_shift, T,
                         C, nb_i, xt_fp8, sc_fp8, sc_fp32);
    else if (x_dtype == PRATCHYA_DT_BF16)
      hipLaunchKernelGGL((k_quant_128x1_rows<IN_BF16, RB>), grid, dim3(rows_threads(RB)), 0, stream, xb, nullptr, nullptr, 0, T, C,
                         nb_i, xt_fp8, sc_fp8, sc_fp32);
    else if (x_dtype == PRATCHYA_DT_F32)
      hipLaunchKernelGGL((k_quant_128x1_rows<IN_F32, RB>), grid, dim3(rows_threads(RB)), 0, stream, xb, nullptr, nullptr, 0, T, C,
                         nb_i, xt_fp8, sc_fp8, sc_fp32);
    else
      hipLaunchKernelGGL((k_quant_128x1_rows<IN_FP8, RF>), grid, dim3(rows_threads(RF)), 0, stream, xb, x_sc8, x_sc32, kg_shift, T,
                         C, nb_i, xt_fp8, sc_fp8, sc_fp32);
  } else if (x_dtype == PRATCHYA_DT_BF16 && scaled) {
    hipLaunchKernelGGL((k_quant_t128<IN_BF16S, true, 16>), grid_for_tok(16), dim3(256), 0, stream, xb, x_sc8, x_sc32, kg_shift,
                       T, C, xt_fp8, sc_fp8, sc_fp32, tok_major);
  } else if (x_dtype == PRATCHYA_DT_BF16) {
    hipLaunchKernelGGL((k_quant_t128<IN_BF16, true, 16>), grid_for_tok(16), dim3(256), 0, stream, xb, nullptr, nullptr, 0,
                       T, C, xt_fp8, sc_fp8, sc_fp32, tok_major);
  } else if (x_dtype == PRATCHYA_DT_F32) {
    hipLaunchKernelGGL((k_quant_t128<IN_F32, true, 8>), grid_for_tok(8), dim3(256), 0, stream, xb, nullptr, nullptr, 0,
                       T, C, xt_fp8, sc_fp8, sc_fp32, tok_major);
  } else {
    hipLaunchKernelGGL((k_quant_t128<IN_FP8, true, 8>), grid_for_tok(8), dim3(256), 0, stream, xb, x_sc8, x_sc32, kg_shift,
                       T, C, xt_fp8, sc_fp8, sc_fp32, tok_major);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return pratchya_set_error(PRATCHYA_EHIP, "%s: launch failed: %s", name, hipGetErrorString(err));
  return PRATCHYA_OK;
}

}  // namespace

extern "C" int pratchya_quantize_t128(const void* x, int x_dtype, const uint8_t* x_sc8,
                                      const float* x_sc32, int64_t slices, int64_t T, int64_t C,
                                      uint8_t* xt_fp8, uint8_t* sc_fp8, float* sc_fp32,
                                      hipStream_t stream) {
  return quantize_128x1_impl(false, x, x_dtype, x_sc8, x_sc32, slices, T, C, xt_fp8, sc_fp8, sc_fp32, stream);
}

extern "C" int pratchya_quantize_128x1(const void* x, int x_dtype, const uint8_t* x_sc8, const float* x_sc32,
                                       int64_t slices, int64_t T, int64_t C, uint8_t* q_fp8, uint8_t* sc_fp8,
                                       float* sc_fp32, hipStream_t stream) {
  return quantize_128x1_impl(true, x, x_dtype, x_sc8, x_sc32, slices, T, C, q_fp8, sc_fp8, sc_fp32, stream);
}

extern "C" int pratchya_quantize_t1x128(const void* x, int x_dtype, const uint8_t* x_sc8, const float* x_sc32,
                                        int64_t slices, int64_t T, int64_t C, uint8_t* xt_fp8, uint8_t* sc_fp8,
                                        float* sc_fp32, hipStream_t stream) {
  if (slices < 0 || T < 0 || C < 0) return pratchya_set_error(PRATCHYA_EINVAL, "quantize_t1x128: negative size");
  if (x_dtype != PRATCHYA_DT_F32 && x_dtype != PRATCHYA_DT_BF16 && x_dtype != PRATCHYA_DT_E4M3)
    return pratchya_set_error(PRATCHYA_EINVAL, "quantize_t1x128: unsupported input dtype %d", x_dtype);
  if (T % 128)
    return pratchya_set_error(PRATCHYA_EINVAL, "quantize_t1x128: tgrid (1, 128) does not divide %lld tokens",
                              (long long)T);
  const bool scaled = x_dtype == PRATCHYA_DT_E4M3 || (x_dtype == PRATCHYA_DT_BF16 && x_sc8 && x_sc32);
  if (scaled && C % 128)
    return pratchya_set_error(PRATCHYA_EINVAL, "quantize_t1x128: tgrid (1, 128) of the input scales does not "
                              "divide %lld channels", (long long)C);
  if (slices == 0 || T == 0 || C == 0) return PRATCHYA_OK;
  if (T % 1024)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "quantize_t1x128: tokens must be a multiple of 1024 (one "
                              "group of 8 blocks per channel; got %lld)", (long long)T);
  if (C % 8)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "quantize_t1x128: channels must be a multiple of 8 (got %lld)",
                              (long long)C);
  if (!x || !xt_fp8 || !sc_fp8 || !sc_fp32 || (x_dtype == PRATCHYA_DT_E4M3 && (!x_sc8 || !x_sc32)))
    return pratchya_set_error(PRATCHYA_EINVAL, "quantize_t1x128: null buffer");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(xt_fp8) % 16 ||
      reinterpret_cast<uintptr_t>(sc_fp8) % 8 || reinterpret_cast<uintptr_t>(sc_fp32) % 4)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "quantize_t1x128: buffers are not aligned");
  if (T / 1024 > 65535 || slices > 65535)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "quantize_t1x128: too many token groups or slices");
  if (scaled && (slices * T) * (C / 128) >= ((int64_t)1 << 32))
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "quantize_t1x128: input scales beyond 2^32 blocks");
  // workgroups of 8 waves: one per 128-token block of a 1024-token group, over
  // 64 (bf16) or 32 (f32, fp8) channels
  auto grid_for_tok = [&](int tok) {
    const int cpw = 8 * (64 / (128 / tok));
    return dim3((unsigned)((C + cpw - 1) / cpw), (unsigned)(T / 1024), (unsigned)slices);
  };
  const uint8_t* xb = static_cast<const uint8_t*>(x);
  const int64_t kg = scaled ? gcd64(8, T * (C / 128)) : 1;
  const int kg_shift = kg == 8 ? 3 : (kg == 4 ? 2 : (kg == 2 ? 1 : 0));
  if (x_dtype == PRATCHYA_DT_BF16 && scaled) {
    hipLaunchKernelGGL((k_quant_t128<IN_BF16S, true, 16, true>), grid_for_tok(16), dim3(512), 0, stream, xb, x_sc8,
                       x_sc32, kg_shift, T, C, xt_fp8, sc_fp8, sc_fp32, 0);
  } else if (x_dtype == PRATCHYA_DT_BF16) {
    hipLaunchKernelGGL((k_quant_t128<IN_BF16, true, 16, true>), grid_for_tok(16), dim3(512), 0, stream, xb, nullptr,
                       nullptr, 0, T, C, xt_fp8, sc_fp8, sc_fp32, 0);
  } else if (x_dtype == PRATCHYA_DT_F32) {
    hipLaunchKernelGGL((k_quant_t128<IN_F32, true, 8, true>), grid_for_tok(8), dim3(512), 0, stream, xb, nullptr,
                       nullptr, 0, T, C, xt_fp8, sc_fp8, sc_fp32, 0);
  } else {
    // one workgroup per 128-channel column and 1024-token group
    hipLaunchKernelGGL(k_quant_t1x128_fp8, dim3((unsigned)(C / 128), (unsigned)(T / 1024), (unsigned)slices),
                       dim3(256), 0, stream, xb, x_sc8, x_sc32, kg_shift, T, C, xt_fp8, sc_fp8, sc_fp32);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return pratchya_set_error(PRATCHYA_EHIP, "quantize_t1x128: launch failed: %s", hipGetErrorString(err));
  return PRATCHYA_OK;
}

extern "C" int pratchya_quantize_dual(const void* x, int x_dtype, int64_t slices, int64_t T, int64_t C,
                                      uint8_t* q_fp8, uint8_t* sc_fp8, float* sc_fp32, uint8_t* t_fp8,
                                      uint8_t* t_sc8, float* t_sc32, hipStream_t stream) {
  if (slices < 0 || T < 0 || C < 0) return pratchya_set_error(PRATCHYA_EINVAL, "quantize_dual: negative size");
  if (x_dtype != PRATCHYA_DT_F32 && x_dtype != PRATCHYA_DT_BF16)
    return pratchya_set_error(PRATCHYA_EINVAL, "quantize_dual: unsupported input dtype %d", x_dtype);
  if (T % 128)
    return pratchya_set_error(PRATCHYA_EINVAL, "quantize_dual: tgrid (128, 1) does not divide %lld tokens",
                              (long long)T);
  if (C % 128)
    return pratchya_set_error(PRATCHYA_EINVAL, "quantize_dual: tgrid (1, 128) does not divide %lld channels",
                              (long long)C);
  if (slices == 0 || T == 0 || C == 0) return PRATCHYA_OK;
  if (C % 1024)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "quantize_dual: channels must be a multiple of 1024 (one "
                              "(1, 128) group per 1024-channel row segment; got %lld)", (long long)C);
  if (!x || !q_fp8 || !sc_fp8 || !sc_fp32 || !t_fp8 || !t_sc8 || !t_sc32)
    return pratchya_set_error(PRATCHYA_EINVAL, "quantize_dual: null buffer");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(q_fp8) | reinterpret_cast<uintptr_t>(t_fp8) |
       reinterpret_cast<uintptr_t>(t_sc8)) % 16 ||
      reinterpret_cast<uintptr_t>(sc_fp8) % 8 || reinterpret_cast<uintptr_t>(t_sc32) % 8 ||
      reinterpret_cast<uintptr_t>(sc_fp32) % 4)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "quantize_dual: buffers are not aligned");
  const int64_t rows = slices * T;
  if (rows / 128 > 65535 || C / 1024 > 65535 || rows * (C / 128) >= ((int64_t)1 << 31))
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "quantize_dual: too many token blocks, channel groups or "
                              "scale bytes (2^31 or more)");
  // slices flatten into tokens: with T a multiple of 128 and C of 1024 neither
  // grid's blocks or groups cross a slice, and the per-slice scale arrays
  // concatenate in token order
  const dim3 grid((unsigned)(C / 1024), (unsigned)(rows / 128));
  if (x_dtype == PRATCHYA_DT_BF16)
    hipLaunchKernelGGL(k_quant_dual<true>, grid, dim3(512), 0, stream, x, C, q_fp8, sc_fp8, sc_fp32, t_fp8, t_sc8,
                       t_sc32);
  else
    hipLaunchKernelGGL(k_quant_dual<false>, grid, dim3(512), 0, stream, x, C, q_fp8, sc_fp8, sc_fp32, t_fp8, t_sc8,
                       t_sc32);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return pratchya_set_error(PRATCHYA_EHIP, "quantize_dual: launch failed: %s", hipGetErrorString(err));
  return PRATCHYA_OK;
}
