// Block-scaled FP8 GEMM for gfx950 (CDNA4) and its C ABI.
//
// Computes C = dequant(A) . dequant(B)^T for e4m3fn payloads A [M, K] and
// B [N, K] (both K-contiguous, "NT"), with pratchya's two-level block scales
// on each operand: the dequantized element is q * 2^(e-127) * G / 128
// (pratchya/_qualia/_qarr.py:562-564), e an e8m0 byte per block and G an f32
// group max.  This is the contraction of matmul_impl (_qarr.py:605-608) and of
// its backward (_qarr.py:621-622) with both operands in FP8 instead of
// dequantized f32.
//
// Structure (one 256x256 output tile per workgroup, 8 waves of 64x128):
//   * 128-wide K tiles staged in LDS by global_load_lds_dwordx4 (DMA straight
//     into LDS, 64 KB per stage, two stages), rows XOR-swizzled in 16-byte
//     chunks so that the MFMA operand reads are bank-conflict free;
//   * v_mfma_scale_f32_32x32x64_f8f6f4: the e8m0 byte of each operand row
//     and 128-K block is applied by the MFMA itself;
//   * the f32 group maxima G are constant over "spans" of K blocks (1024 K for
//     (1,128) activations, the whole K for a single-group weight).  The
//     accumulator holds C / (gA gB) of the current span and is rescaled by
//     (gA_old/gA_new)(gB_old/gB_new) when a span starts, so one accumulator
//     set suffices; the epilogue multiplies by gA gB / 2^14.
//
// Differences from the reference's f32 dequant-then-matmul: summation order,
// and blocks whose e8m0 byte is 0 (block max below 2^-126 of its group max):
// the reference dequantizes them to exactly 0, the MFMA scales them by 2^-127.
// Both are far below the 1e-2 relative Frobenius tolerance of the contract.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pratchya_fp8.h"

int pratchya_set_error(int code, const char* fmt, ...);

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int TILE_BYTES = BM * BK;            // 32 KB per operand per stage
constexpr int NTHREADS = 512;

struct Scales {
  const uint8_t* e8;   // e8m0 bytes
  const float* g32;    // group maxima
  int64_t r_div;       // rows per block along the non-contraction axis
  int64_t s_r;         // block index stride per row block
  int64_t s_k;         // block index stride per 128-K block
  int64_t kg;          // blocks per group
  int64_t bpg;         // group index of (row, kb) = (base(row) / kg) + (kb / bpg) * gstep
  int64_t gstep;
};

__host__ __device__ __forceinline__ int64_t blk_index(const Scales& s, int64_t row, int64_t kb) {
  return (row / s.r_div) * s.s_r + kb * s.s_k;
}

// 16-byte chunk swizzle of LDS row r: conflict free for 8 or 16 consecutive
// rows reading the same logical chunk (32 or 64 LDS banks).
__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

typedef __attribute__((address_space(3))) void lds_void;

// Issue the DMA of one operand's 256 x 128-byte K tile into LDS (4 row groups
// of 8 rows per wave; lane -> row (lane>>3), physical chunk (lane&7)).
__device__ __forceinline__ void dma_tile(const uint8_t* __restrict__ src, int64_t ld, int row0,
                                         int64_t k0, uint8_t* lds_tile, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int g = wave * 4 + i;
    const int r = g * 8 + (lane >> 3);
    const int c = (lane & 7) ^ swz(r);
    const uint8_t* p = src + (int64_t)(row0 + r) * ld + k0 + c * 16;
    __builtin_amdgcn_global_load_lds(p, (lds_void*)(lds_tile + g * 1024), 16, 0, 0);
  }
}

// 32-byte MFMA operand of LDS row r, logical chunks c0, c0+1.
__device__ __forceinline__ v8i read_frag(const uint8_t* lds_tile, int r, int c0) {
  const int s = swz(r);
  const v4i lo = *reinterpret_cast<const v4i*>(lds_tile + r * BK + ((c0 ^ s) << 4));
  const v4i hi = *reinterpret_cast<const v4i*>(lds_tile + r * BK + (((c0 + 1) ^ s) << 4));
  return v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

// One 32x32x64 MFMA of output tile (MI, NI): a-operand = B rows (e8m0 byte NI
// of eB), b-operand = A rows (byte MI of eA); op_sel picks the byte.
template <int MI, int NI>
__device__ __forceinline__ void mfma_tile(v16f (&acc)[2][4], const v8i (&fa)[2], const v8i (&fb)[4],
                                          uint32_t eA, uint32_t eB) {
  acc[MI][NI] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[NI], fa[MI], acc[MI][NI], 0, 0, NI,
                                                               (int)eB, MI, (int)eA);
}

// B-side group maxima held per lane: 4 (one per 32-column MFMA tile) or 16
// (one per 4-column accumulator group, for scale groups narrower than 32 rows).
template <bool FINE_B>
struct BGroups {
  static constexpr int NJ = FINE_B ? 4 : 1;
  float g[4][NJ];
  uint32_t idx0[4][NJ];
};

template <bool OUT_BF16, bool FINE_B>
__global__ __launch_bounds__(NTHREADS, 1) void k_gemm_bs_nt(
    const uint8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    Scales sa, Scales sb, void* __restrict__ C, int64_t ldc, int K, int span, int tiles_n) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds_a0[TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_b0[TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_a1[TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) uint8_t lds_b1[TILE_BYTES];
  constexpr int NJ = BGroups<FINE_B>::NJ;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave & 3, wn = wave >> 2;
  const int tm = blockIdx.x / tiles_n, tn = blockIdx.x % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int nk = K / BK;
  const int l32 = lane & 31, lhi = lane >> 5;

  // Block-index bases (kb = 0) of the rows this lane feeds to the MFMA: A rows
  // (b-operand) and B rows (a-operand).
  uint32_t baseA[2], baseB[4];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) baseA[mi] = (uint32_t)blk_index(sa, m0 + wm * 64 + mi * 32 + l32, 0);
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) baseB[ni] = (uint32_t)blk_index(sb, n0 + wn * 128 + ni * 32 + l32, 0);
  const uint32_t skA = (uint32_t)sa.s_k, skB = (uint32_t)sb.s_k;

  // group-max indices at kb = 0: A per lane row, B per output column group
  uint32_t gidxA[2];
  BGroups<FINE_B> bg;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) gidxA[mi] = baseA[mi] / (uint32_t)sa.kg;
#pragma unroll
  for (int ni = 0; ni < 4; ++ni)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      bg.idx0[ni][j] = (uint32_t)(blk_index(sb, n0 + wn * 128 + ni * 32 + 8 * j + 4 * lhi, 0) / sb.kg);

  v16f acc[2][4];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = v16f{0};

  // Group maxima of the current span.  A zero group max keeps the previous
  // value: an all-zero group has an all-zero payload and adds nothing.
  float gA[2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const float g = sa.g32[gidxA[mi]];
    gA[mi] = g == 0.0f ? 1.0f : g;
  }
#pragma unroll
  for (int ni = 0; ni < 4; ++ni)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float g = sb.g32[bg.idx0[ni][j]];
      bg.g[ni][j] = g == 0.0f ? 1.0f : g;
    }
  float gAn[2], gBn[4][NJ];

  // e8m0 bytes of the current K block, packed: byte mi of eA, byte ni of eB
  uint32_t eA = 0, eB = 0;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) eA |= (uint32_t)sa.e8[baseA[mi]] << (8 * mi);
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) eB |= (uint32_t)sb.e8[baseB[ni]] << (8 * ni);

  dma_tile(A, lda, m0, 0, lds_a0, wave, lane);
  dma_tile(B, ldb, n0, 0, lds_b0, wave, lane);

  for (int kt = 0; kt < nk; ++kt) {
    // the stage of kt has landed for every wave; every wave is done with kt-1
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const bool odd = kt & 1;
    const uint8_t* la = odd ? lds_a1 : lds_a0;
    const uint8_t* lb = odd ? lds_b1 : lds_b0;

    if (kt > 0 && kt % span == 0) {
      // a new span of group maxima starts: move the accumulator into its units
      float rA[2], rB[4][NJ];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const float g = gAn[mi] == 0.0f ? gA[mi] : gAn[mi];
        rA[mi] = gA[mi] / g;
        gA[mi] = g;
      }
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const float g = gBn[ni][j] == 0.0f ? bg.g[ni][j] : gBn[ni][j];
          rB[ni][j] = bg.g[ni][j] / g;
          bg.g[ni][j] = g;
        }
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[mi][ni][v] *= rA[mi] * rB[ni][FINE_B ? (v >> 2) : 0];
    }

    uint32_t eAn = 0, eBn = 0;
    if (kt + 1 < nk) {
      dma_tile(A, lda, m0, (int64_t)(kt + 1) * BK, odd ? lds_a0 : lds_a1, wave, lane);
      dma_tile(B, ldb, n0, (int64_t)(kt + 1) * BK, odd ? lds_b0 : lds_b1, wave, lane);
      const uint32_t kn = (uint32_t)(kt + 1);
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) eAn |= (uint32_t)sa.e8[baseA[mi] + kn * skA] << (8 * mi);
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) eBn |= (uint32_t)sb.e8[baseB[ni] + kn * skB] << (8 * ni);
      if (kn % (uint32_t)span == 0) {
        const uint32_t dA = (kn / (uint32_t)sa.bpg) * (uint32_t)sa.gstep;
        const uint32_t dB = (kn / (uint32_t)sb.bpg) * (uint32_t)sb.gstep;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) gAn[mi] = sa.g32[gidxA[mi] + dA];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
          for (int j = 0; j < NJ; ++j) gBn[ni][j] = sb.g32[bg.idx0[ni][j] + dB];
      }
    }

#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c0 = ks * 4 + lhi * 2;
      v8i fa[2], fb[4];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) fa[mi] = read_frag(la, wm * 64 + mi * 32 + l32, c0);
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) fb[ni] = read_frag(lb, wn * 128 + ni * 32 + l32, c0);
      mfma_tile<0, 0>(acc, fa, fb, eA, eB);
      mfma_tile<0, 1>(acc, fa, fb, eA, eB);
      mfma_tile<0, 2>(acc, fa, fb, eA, eB);
      mfma_tile<0, 3>(acc, fa, fb, eA, eB);
      mfma_tile<1, 0>(acc, fa, fb, eA, eB);
      mfma_tile<1, 1>(acc, fa, fb, eA, eB);
      mfma_tile<1, 2>(acc, fa, fb, eA, eB);
      mfma_tile<1, 3>(acc, fa, fb, eA, eB);
    }
    eA = eAn;
    eB = eBn;
  }

  // epilogue: C[m][n] = acc * gA * gB / 2^14 (the two /128 of the dequant)
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int64_t m = m0 + wm * 64 + mi * 32 + l32;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + wn * 128 + ni * 32 + 8 * j + 4 * lhi;
        const float f = gA[mi] * bg.g[ni][FINE_B ? j : 0] * 6.103515625e-05f;
        const float c0 = acc[mi][ni][4 * j + 0] * f, c1 = acc[mi][ni][4 * j + 1] * f;
        const float c2 = acc[mi][ni][4 * j + 2] * f, c3 = acc[mi][ni][4 * j + 3] * f;
        if constexpr (OUT_BF16) {
          typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
          const bf16x2 p0 = {(__bf16)c0, (__bf16)c1};
          const bf16x2 p1 = {(__bf16)c2, (__bf16)c3};
          uint2 w;
          w.x = __builtin_bit_cast(uint32_t, p0);
          w.y = __builtin_bit_cast(uint32_t, p1);
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(C) + m * ldc + n) = w;
        } else {
          *reinterpret_cast<float4*>(static_cast<float*>(C) + m * ldc + n) = make_float4(c0, c1, c2, c3);
        }
      }
    }
  }
}

// Affine group index of an operand's scale layout: returns false if the
// group of block (rb, kb) = (rb*s_r + kb*s_k) / kg is not of the form
// floor(rb*s_r / kg) + floor(kb / bpg) * gstep for every row block rb and
// every kb < nk.  The closed forms below cover every layout pratchya's
// quantizer produces for 128-wide contraction blocks; anything else is checked
// exhaustively.
bool affine_groups(Scales* s, int64_t rows, int64_t nk) {
  const int64_t nrb = (rows + s->r_div - 1) / s->r_div;
  auto verify = [&](int64_t bpg, int64_t gstep) {
    if (nrb * nk > (int64_t)1 << 22) return false;
    for (int64_t rb = 0; rb < nrb; ++rb)
      for (int64_t kb = 0; kb < nk; ++kb)
        if ((rb * s->s_r + kb * s->s_k) / s->kg != (rb * s->s_r) / s->kg + (kb / bpg) * gstep)
          return false;
    return true;
  };
  int64_t bpg = 0, gstep = 0;
  if (s->s_k == 0) {
    bpg = nk; gstep = 0;                                   // K does not move the index
  } else if (s->s_k == 1 && s->s_r % s->kg == 0) {
    bpg = s->kg; gstep = 1;                                // each row: aligned runs of kg blocks
  } else if (s->s_k == 1 && s->s_r > 0 && s->kg % s->s_r == 0 && nk <= s->s_r) {
    bpg = nk; gstep = 0;                                   // a row's blocks stay in one group
  } else if (s->s_r * (nrb - 1) < s->s_k && s->kg % s->s_k == 0) {
    bpg = s->kg / s->s_k; gstep = 1;                       // rows interleaved inside a K block
  } else if (s->s_k % s->kg == 0 && s->s_r * (nrb - 1) < s->kg &&
             (s->s_r == 0 || s->kg % s->s_r == 0)) {
    bpg = 1; gstep = s->s_k / s->kg;                       // a new group every K block
  } else {
    for (int64_t b = nk; b >= 1 && !bpg; --b)
      for (int64_t g = 0; g <= 1 && !bpg; ++g)
        if (verify(b, g * ((s->s_k * b) / s->kg))) { bpg = b; gstep = g * ((s->s_k * b) / s->kg); }
    if (!bpg) return false;
  }
  if (bpg > nk) bpg = nk;
  if (bpg < 1) bpg = 1;
  s->bpg = bpg;
  s->gstep = gstep;
  return true;
}

}  // namespace

extern "C" int64_t pratchya_gemm_span(int64_t rows, int64_t K, int64_t r_div, int64_t s_r,
                                      int64_t s_k, int64_t kg) {
  if (K % BK || r_div < 1 || kg < 1) return 0;
  Scales s{nullptr, nullptr, r_div, s_r, s_k, kg, 0, 0};
  if (!affine_groups(&s, rows, K / BK)) return 0;
  return s.bpg;
}

extern "C" int pratchya_gemm_bs_nt(const uint8_t* A, int64_t lda, const uint8_t* a_sc8,
                                   const float* a_sc32, int64_t a_rdiv, int64_t a_sr, int64_t a_sk,
                                   int64_t a_kg, const uint8_t* B, int64_t ldb, const uint8_t* b_sc8,
                                   const float* b_sc32, int64_t b_rdiv, int64_t b_sr, int64_t b_sk,
                                   int64_t b_kg, int64_t M, int64_t N, int64_t K, void* C,
                                   int64_t ldc, int c_dtype, hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0) {
    if (M < 0 || N < 0 || K < 0) return pratchya_set_error(PRATCHYA_EINVAL, "gemm: negative size");
    return PRATCHYA_OK;
  }
  if (M % BM || N % BN || K % BK)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED,
                              "gemm: M, N must be multiples of 256 and K of 128 (got %lld, %lld, %lld)",
                              (long long)M, (long long)N, (long long)K);
  if (!A || !B || !a_sc8 || !a_sc32 || !b_sc8 || !b_sc32 || !C)
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm: null buffer");
  if (c_dtype != PRATCHYA_DT_F32 && c_dtype != PRATCHYA_DT_BF16)
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm: unsupported output dtype %d", c_dtype);
  if (lda < K || ldb < K || ldc < N || lda % 16 || ldb % 16 || ldc % 4 ||
      (reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) % 16 ||
      reinterpret_cast<uintptr_t>(C) % 16)
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm: leading dimensions / alignment not supported");
  if (a_rdiv < 1 || b_rdiv < 1 || a_kg < 1 || b_kg < 1)
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm: bad scale layout");
  Scales sa{a_sc8, a_sc32, a_rdiv, a_sr, a_sk, a_kg, 0, 0};
  Scales sb{b_sc8, b_sc32, b_rdiv, b_sr, b_sk, b_kg, 0, 0};
  const int64_t nk = K / BK;
  if (!affine_groups(&sa, M, nk) || !affine_groups(&sb, N, nk))
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm: scale groups are not affine in K");
  if ((M / a_rdiv) * a_sr + nk * a_sk > (int64_t)UINT32_MAX ||
      (N / b_rdiv) * b_sr + nk * b_sk > (int64_t)UINT32_MAX)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm: scale arrays beyond 2^32 blocks");
  // B's group max per lane: one per 32 output columns, or one per 4 columns.
  const bool fine_b = b_rdiv % 32 != 0;
  if (fine_b && !(b_rdiv % 4 == 0 || (b_rdiv == 1 && b_kg % (4 * b_sr) == 0 && b_sk % (4 * b_sr) == 0)))
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm: B scale groups narrower than 4 columns");
  int64_t x = sa.bpg, y = sb.bpg;   // span: both group patterns are constant over it
  while (y) {
    const int64_t t = x % y;
    x = y;
    y = t;
  }
  const int64_t span = x < 1 ? 1 : x;
  const int64_t tiles_n = N / BN;
  const int64_t tiles = (M / BM) * tiles_n;
#define PRATCHYA_GEMM(BF, FB)                                                                   \
  hipLaunchKernelGGL((k_gemm_bs_nt<BF, FB>), dim3((unsigned)tiles), dim3(NTHREADS), 0, stream, A, lda, \
                     B, ldb, sa, sb, C, ldc, (int)K, (int)span, (int)tiles_n)
  const bool bf = c_dtype == PRATCHYA_DT_BF16;
  if (bf && !fine_b) PRATCHYA_GEMM(true, false);
  else if (bf) PRATCHYA_GEMM(true, true);
  else if (!fine_b) PRATCHYA_GEMM(false, false);
  else PRATCHYA_GEMM(false, true);
#undef PRATCHYA_GEMM
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return pratchya_set_error(PRATCHYA_EHIP, "gemm: launch failed: %s", hipGetErrorString(e));
  return PRATCHYA_OK;
}

// --------------------------------------------------------------------------
// Byte transpose [rows, cols] -> [cols, rows] (fp8 payloads: W [K, N] to the
// K-contiguous [N, K] operand layout, token-major payloads to channel-major).
// 64x64 tiles through LDS; 16-byte global loads and stores.
// --------------------------------------------------------------------------
namespace {
__global__ __launch_bounds__(256) void k_transpose_u8(const uint8_t* __restrict__ src, int64_t rows,
                                                      int64_t cols, uint8_t* __restrict__ dst) {
  __shared__ uint32_t tile[64][17];   // 64 rows x 64 bytes (+1 word pad)
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int t = threadIdx.x;
  {
    const int r = t >> 2, q = t & 3;   // row r, 16-byte quarter q
    const int64_t gr = r0 + r, gc = c0 + q * 16;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (gr < rows && gc + 16 <= cols) v = *reinterpret_cast<const uint4*>(src + gr * cols + gc);
    tile[r][q * 4 + 0] = v.x;
    tile[r][q * 4 + 1] = v.y;
    tile[r][q * 4 + 2] = v.z;
    tile[r][q * 4 + 3] = v.w;
  }
  __syncthreads();
  {
    const int c = t >> 2, q = t & 3;   // output row c (= input column), 16 input rows q*16..
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t acc = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int r = q * 16 + i * 4 + b;
        const uint32_t word = tile[r][c >> 2];
        acc |= ((word >> (8 * (c & 3))) & 0xFFu) << (8 * b);
      }
      w[i] = acc;
    }
    const int64_t gr = c0 + c, gc = r0 + q * 16;
    if (gr < cols && gc + 16 <= rows)
      *reinterpret_cast<uint4*>(dst + gr * rows + gc) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}
}  // namespace

extern "C" int pratchya_transpose_u8(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* dst,
                                     hipStream_t stream) {
  if (rows < 0 || cols < 0) return pratchya_set_error(PRATCHYA_EINVAL, "transpose: negative size");
  if (rows == 0 || cols == 0) return PRATCHYA_OK;
  if (rows % 64 || cols % 64 || reinterpret_cast<uintptr_t>(src) % 16 || reinterpret_cast<uintptr_t>(dst) % 16)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "transpose: sizes must be multiples of 64, buffers 16-byte aligned");
  if (!src || !dst) return pratchya_set_error(PRATCHYA_EINVAL, "transpose: null buffer");
  hipLaunchKernelGGL(k_transpose_u8, dim3((unsigned)(cols / 64), (unsigned)(rows / 64)), dim3(256), 0,
                     stream, src, rows, cols, dst);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return pratchya_set_error(PRATCHYA_EHIP, "transpose: %s", hipGetErrorString(e));
  return PRATCHYA_OK;
}
