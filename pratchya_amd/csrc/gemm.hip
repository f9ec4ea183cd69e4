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
// Structure (one 256x256 output tile per workgroup of 8 waves, each wave a
// 64x128 sub-tile, two waves per SIMD):
//   * 128-wide K tiles staged in LDS by global_load_lds_dwordx4 (DMA straight
//     into LDS, two stages), rows XOR-swizzled in 16-byte chunks so that the
//     MFMA operand reads are bank-conflict free;
//   * the e8m0 bytes of the stage's 256 + 256 rows travel through LDS by the
//     same DMA; their f32 group maxima are loaded into registers by the wave
//     that loads the rows, which writes the accumulator units and unit
//     ratios derived from them into the stage (see publish_g);
//   * "ping-pong": the two waves sharing a SIMD belong to two groups whose
//     phases are offset by one workgroup barrier, so while one group runs its
//     MFMA cluster for a 64-wide K slice the other reads its next operands
//     from LDS (and group 0 issues the next stage's DMA);
//   * v_mfma_scale_f32_32x32x64_f8f6f4: the e8m0 byte of each operand row
//     and 128-K block is applied by the MFMA itself;
//   * the f32 group maxima G are constant over "spans" of K blocks (1024 K for
//     (1,128) activations, the whole K for a single-group weight).  The
//     accumulator holds C / (gA gB) of the current span and is rescaled by
//     (gA_old/gA_new)(gB_old/gB_new) when a span starts, so one accumulator
//     set suffices; the epilogue multiplies by gA gB / 2^14;
//   * tiles are numbered so that the workgroups resident on one XCD (the
//     dispatcher deals workgroups round-robin to the 8 XCDs) cover a 4 x 8
//     block of output tiles and share A and B panels in that XCD's L2;
//   * the same pipeline also runs the bf16 products of Newton-Schulz (BF),
//     with its 1.5 X - 0.5 B combination in the epilogue (FQ 3), and the
//     symmetric product A A^T on the upper-triangle tiles only, split by K
//     between workgroups (FQ 4, see FqArgs).
//
// Differences from the reference's f32 dequant-then-matmul: summation order,
// and blocks whose e8m0 byte is 0 (block max below 2^-126 of its group max):
// the reference dequantizes them to exactly 0, the MFMA scales them by 2^-127.
// Both are far below the 1e-2 relative Frobenius tolerance of the contract.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <numeric>
#include <type_traits>

#include "pratchya_fp8.h"
#include "quant_device.h"

int pratchya_set_error(int code, const char* fmt, ...);

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int TILE_BYTES = BM * BK;            // 32 KB per operand per stage
constexpr int NTHREADS = 512;
// LDS stage: A tile | B tile | A e8m0 words | B e8m0 words | A unit ratios |
// B unit ratios.  After the two stages: A units | B units (of the latest span
// start).  The ratio and unit arrays are in the order the MFMA lanes read
// them: A per row as [band wm][l32][mi] (one 8-byte read per lane); B per 32
// rows, per 4 rows as [wn][ni][lhi][j] (one 16-byte read per 32-column tile),
// or per row as [wn][ni][lhi][j][i] (four 16-byte reads), by the B group
// granularity BG (0, 1, 2; see load_units).
constexpr int OFF_B = TILE_BYTES;
constexpr int OFF_EA = 2 * TILE_BYTES;
constexpr int OFF_EB = OFF_EA + 4 * BM;
constexpr int OFF_RA = OFF_EB + 4 * BN;
constexpr int OFF_RB = OFF_RA + 4 * BM;
constexpr int STAGE_BYTES = 69632;             // OFF_RB + 4 * BN
constexpr int OFF_UA = 2 * STAGE_BYTES;
constexpr int OFF_UB = OFF_UA + 4 * BM;
constexpr int LDS_BYTES = OFF_UB + 4 * BN;
static_assert(OFF_RB + 4 * BN <= STAGE_BYTES && LDS_BYTES <= 160 * 1024, "LDS layout");

struct Scales {
  const uint8_t* e8;   // e8m0 bytes
  const float* g32;    // group maxima
  int64_t r_div;       // rows per block along the non-contraction axis
  int64_t s_r;         // block index stride per row block
  int64_t s_k;         // block index stride per 128-K block
  int64_t kg;          // blocks per group: group of block i is i / kg
};

__host__ __device__ __forceinline__ int64_t blk_index(const Scales& s, int64_t row, int64_t kb) {
  return (row / s.r_div) * s.s_r + kb * s.s_k;
}

// 16-byte chunk swizzle of LDS row r: conflict free for 8 or 16 consecutive
// rows reading the same logical chunk (32 or 64 LDS banks).
__device__ __forceinline__ int swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void dma16(const void* g, uint8_t* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_void*)lds, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, uint8_t* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_void*)lds, 4, 0, 0);
}

// 32-byte MFMA operand: two 16-byte LDS reads at a per-lane address plus a
// compile-time offset (row block and operand), folded into ds_read's offset.
template <int OFF>
__device__ __forceinline__ v8i read_frag2(const uint8_t* base_lo, const uint8_t* base_hi) {
  const v4i lo = *reinterpret_cast<const v4i*>(base_lo + OFF);
  const v4i hi = *reinterpret_cast<const v4i*>(base_hi + OFF);
  return v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

// K-major ("TN") bf16 operand of the Gram product: the stage holds 64 K rows
// of 256 operand rows each (512 bytes per K row, the operand's natural
// layout), 16-byte chunks XOR-swizzled by 4 * (k mod 4) so that the
// transposing reads below are bank-conflict free.  ds_read_b64_tr_b16 lets
// each lane of a 16-lane group read 4 bf16 of one K row; lane i then holds
// element i mod 4 of the reads of lanes i / 4 + 4 e (e = 0..3): with lane j of
// the group reading K row k0 + j / 4 at operand row m0 + 4 (j mod 4), lane i
// receives operand row m0 + i and K rows k0 .. k0 + 3, the MFMA's layout.
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;
__device__ __forceinline__ v4i tr_pair(const uint8_t* p0, const uint8_t* p1) {
  const v4s a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p0);
  const v4s b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)p1);
  const v2i x = __builtin_bit_cast(v2i, a), y = __builtin_bit_cast(v2i, b);
  return v4i{x.x, x.y, y.x, y.y};
}
// 32-byte fragment of 32 operand rows at `base` (the lane's row and K-row
// offsets folded in: K rows +0 for lanes 0-31, +16 for lanes 32-63): K rows
// +0..7 for the first MFMA, +8..15 for the second -- the K values the NT
// fragment gives each lane (read_frag2), so K-major and K-contiguous operands
// mix in one product and give the same sums.
template <int OFF>
__device__ __forceinline__ v8i read_frag_tn(const uint8_t* base) {
  const v4i lo = tr_pair(base + OFF, base + OFF + 4 * 512);
  const v4i hi = tr_pair(base + OFF + 8 * 512, base + OFF + 12 * 512);
  return v8i{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

// FP8 K-major operand: the stage holds 128 K rows of 256 operand bytes, 16-byte
// chunks XOR-swizzled by 2 * (k mod 8).  ds_read_b64_tr_b8: in a 16-lane
// group, lane i holds byte i mod 8 of the 8-byte reads of lanes i / 8 + 2 e
// (e = 0..7); with lane j reading K row k0 + j / 2 at operand row m0 + 8 (j mod
// 2), lane i receives operand row m0 + i and K rows k0 .. k0 + 7.  Four reads
// (K rows +0, +8, +16, +24) give the 32 consecutive K values of an FP8 MFMA
// lane, the K-contiguous fragment's (read_frag2) values.
typedef __attribute__((address_space(3))) v2i lds_v2i;
template <int OFF>
__device__ __forceinline__ v8i read_frag_tn8(const uint8_t* base) {
  const v2i a = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(base + OFF));
  const v2i b = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(base + OFF + 8 * 256));
  const v2i c = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(base + OFF + 16 * 256));
  const v2i d = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(base + OFF + 24 * 256));
  return v8i{a.x, a.y, b.x, b.y, c.x, c.y, d.x, d.y};
}

// One 32x32x64 MFMA of output tile (MI, NI): a-operand = B rows (e8m0 byte NI
// of eB), b-operand = A rows (byte MI of eA); op_sel picks the byte.  BF: the
// operands are bf16 (a 32-byte fragment is 16 K values), two 32x32x16 bf16
// MFMAs on the fragments' first and second 16 bytes (A and B present their K
// values in the same order, so the dot product is the same).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
template <int MI, int NI, bool BF = false>
__device__ __forceinline__ void mfma_tile(v16f (&acc)[2][4], const v8i (&fa)[2], const v8i (&fb)[4],
                                          uint32_t eA, uint32_t eB) {
  if constexpr (BF) {
    const v8i a = fb[NI], b = fa[MI];
    const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, v4i{a.s0, a.s1, a.s2, a.s3});
    const bf16x8_t a1 = __builtin_bit_cast(bf16x8_t, v4i{a.s4, a.s5, a.s6, a.s7});
    const bf16x8_t b0 = __builtin_bit_cast(bf16x8_t, v4i{b.s0, b.s1, b.s2, b.s3});
    const bf16x8_t b1 = __builtin_bit_cast(bf16x8_t, v4i{b.s4, b.s5, b.s6, b.s7});
    acc[MI][NI] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[MI][NI], 0, 0, 0);
    acc[MI][NI] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[MI][NI], 0, 0, 0);
  } else {
    acc[MI][NI] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[NI], fa[MI], acc[MI][NI], 0, 0, NI,
                                                                 (int)eB, MI, (int)eA);
  }
}

// One MFMA whose result is pinned right after it: the asm's memory clobber
// keeps the stage DMA issued between MFMAs from being reordered around it.
template <int MI, int NI, bool BF = false>
__device__ __forceinline__ void mfma_pinned(v16f (&acc)[2][4], const v8i (&fa)[2], const v8i (&fb)[4],
                                            uint32_t eA, uint32_t eB) {
  mfma_tile<MI, NI, BF>(acc, fa, fb, eA, eB);
  asm volatile("" : "+v"(acc[MI][NI]) : : "memory");
}

__device__ __forceinline__ void mfma_all(v16f (&acc)[2][4], const v8i (&fa)[2], const v8i (&fb)[4],
                                         uint32_t eA, uint32_t eB) {
  mfma_tile<0, 0>(acc, fa, fb, eA, eB);
  mfma_tile<0, 1>(acc, fa, fb, eA, eB);
  mfma_tile<0, 2>(acc, fa, fb, eA, eB);
  mfma_tile<0, 3>(acc, fa, fb, eA, eB);
  mfma_tile<1, 0>(acc, fa, fb, eA, eB);
  mfma_tile<1, 1>(acc, fa, fb, eA, eB);
  mfma_tile<1, 2>(acc, fa, fb, eA, eB);
  mfma_tile<1, 3>(acc, fa, fb, eA, eB);
}

// Buffer resources of one operand: payload, e8m0 bytes, group maxima.  Raw
// buffer loads are range-checked against num_records, so an offset outside an
// array reads zeros instead of faulting.
struct OperandRsrc {
  __amdgpu_buffer_rsrc_t pay, e8, g32;
};

__device__ __forceinline__ OperandRsrc make_rsrc(const uint8_t* pay, uint32_t pay_bytes,
                                                 const Scales& s, uint32_t e8_bytes,
                                                 uint32_t g32_bytes) {
  constexpr int kFlags = 0x00020000;   // gfx9 raw buffer: 32-bit data format
  OperandRsrc r;
  r.pay = __builtin_amdgcn_make_buffer_rsrc((void*)pay, 0, (int)pay_bytes, kFlags);
  r.e8 = __builtin_amdgcn_make_buffer_rsrc((void*)s.e8, 0, (int)e8_bytes, kFlags);
  r.g32 = __builtin_amdgcn_make_buffer_rsrc((void*)s.g32, 0, (int)g32_bytes, kFlags);
  return r;
}

// Tile DMA: row group g (8 rows) of the 256-row tile goes to LDS bytes
// [g*1024, g*1024+1024): lane -> row g*8 + (lane>>3), physical chunk lane&7,
// logical chunk (lane&7) ^ swz(row) = (lane&7) ^ (lane>>3) ^ (g&1).  The
// address is a wave-uniform soffset plus one of two per-lane offsets.
__device__ __forceinline__ void dma_offsets(int64_t ld, int lane, uint32_t (&off)[2]) {
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int c = (lane & 7) ^ (lane >> 3) ^ par;
    off[par] = (uint32_t)((lane >> 3) * ld + c * 16);
  }
}

// K-major operand: instruction i of a wave loads 1 KB of consecutive K rows
// (bf16: K rows 2i, 2i + 1 of its 16, 512 bytes each; fp8: K rows 4i .. 4i + 3
// of its 32, 256 bytes each): lane -> K row, LDS chunk c of that row, which
// holds the operand's chunk c ^ 4 (k mod 4) (bf16) or c ^ 2 (k mod 8) (fp8).
template <bool BF>
__device__ __forceinline__ void dma_offsets_tn(int64_t ld, int lane, uint32_t (&off)[2]) {
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    if constexpr (BF) {
      const int rp = lane >> 5, c = lane & 31;
      const int sw = ((2 * par + rp) & 3) << 2;
      off[par] = (uint32_t)(rp * ld + ((c ^ sw) << 4));
    } else {
      const int rp = lane >> 4, c = lane & 15;
      const int sw = ((4 * par + rp) & 7) << 1;
      off[par] = (uint32_t)(rp * ld + ((c ^ sw) << 4));
    }
  }
}

// One wave's share of a stage's DMA.  The stage load is split between the
// two ping-pong groups: wave w of group 0 loads A rows [64w, 64w + 64) of the
// tile, their e8m0 words and group maxima; wave w of group 1 the same for B.
// Each is issued inside a compute phase, between MFMAs, so that the load
// issue (throttled by the vector memory address path) runs in the MFMAs'
// shadow instead of lengthening a memory phase.
struct DmaHalf {
  __amdgpu_buffer_rsrc_t pay, e8, g32;
  uint32_t ld;                 // operand row stride in bytes
  uint32_t s_k, kg;            // block index stride per K block, blocks per group
  uint32_t off[2];             // per-lane byte offset inside an 8-row group (even / odd group)
  int lds_pay, lds_e;          // stage offsets of this wave's payload rows, e8m0 words
  int lds_r, lds_u;            // offsets of the operand's unit ratio (in a stage) and unit arrays
  int pub;                     // byte offset of the lane's row in those arrays
  uint32_t krow0;              // TN: the wave's first K row in a stage (16 per wave)
};

// The rows a wave loads for one output tile: the first of its 64 rows (global
// row index) and the e8m0 block index of the lane's row at kb = 0.
struct DmaRows {
  uint32_t row0, e_word;
  int kb;                      // K block of the unit's first step (a Gram segment; else 0)
};

// Row group i (8 rows) of a stage load whose row group 0 starts at byte
// offset soff0 of the operand (row0 * ld + kt * BK) and LDS address lds0:
// one add per row group, so that little scalar work sits between the MFMAs.
// (rows: operand rows per instruction, 8, or K rows of a K-major operand)
__device__ __forceinline__ void dma_rows_at(const DmaHalf& h, uint32_t soff0, uint8_t* lds0, int i, uint32_t rows) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(h.pay, (lds_void*)(lds0 + i * 1024), 16, h.off[i & 1],
                                           soff0 + (uint32_t)i * (rows * h.ld), 0, 0);
}

// K-major: DMA instruction i of this wave's K rows for K block kt (64 bf16 /
// 128 fp8 K rows) of the operand rows starting at r.row0, into stage st.
template <bool BF>
__device__ __forceinline__ void dma_rows_tn(const DmaHalf& h, const DmaRows& r, uint8_t* st, int kt, int i) {
  constexpr uint32_t ESZ = BF ? 2u : 1u, KROWS = BK / ESZ, RPI = 1024 / (256 * ESZ);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(h.pay, (lds_void*)(st + h.lds_pay + i * 1024), 16, h.off[i & 1],
                                           r.row0 * ESZ + ((uint32_t)kt * KROWS + h.krow0 + RPI * (uint32_t)i) * h.ld,
                                           0, 0);
}

// Row group i (8 rows) of this wave's 64 rows for K block kt into stage st.
__device__ __forceinline__ void dma_rows(const DmaHalf& h, const DmaRows& r, uint8_t* st, int kt, int i) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(h.pay, (lds_void*)(st + h.lds_pay + i * 1024), 16, h.off[i & 1],
                                           (r.row0 + (uint32_t)(i * 8)) * h.ld + (uint32_t)kt * BK, 0, 0);
}

// The e8m0 word of each of this wave's 64 rows for K block kt.
__device__ __forceinline__ void dma_scales(const DmaHalf& h, const DmaRows& r, uint8_t* st, int kt) {
  const uint32_t ia = r.e_word + (uint32_t)kt * h.s_k;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(h.e8, (lds_void*)(st + h.lds_e), 4, ia & ~3u, 0, 0, 0);
}

// The group max of the lane's row for K block kt (exact group index block /
// kg), into a register: it is turned into units by publish_g once the stage
// has landed.
__device__ __forceinline__ float load_g(const DmaHalf& h, const DmaRows& r, int kt) {
  const uint32_t ia = r.e_word + (uint32_t)kt * h.s_k;
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(h.g32, (int)((ia / h.kg) * 4u), 0, 0));
}

// The accumulator holds C / (uA uB) in the units u of its operands' rows,
// set at each span start: the group max, or the previous units where the
// group max is 0 (an all-zero group has an all-zero payload and adds
// nothing); a tile's first K block starts from units 1.  The wave that
// loaded a span start's rows writes the factor old / new units into the
// stage and the new units into the unit arrays, once per row instead of once
// per MFMA lane (for the (128,1) operands of a weight gradient the span is
// one K block).
__device__ __forceinline__ void publish_g(const DmaHalf& h, uint8_t* lds, uint8_t* st, float g_ld, bool first,
                                          float& u_prev) {
  const float prev = first ? 1.0f : u_prev;
  const float u = g_ld == 0.0f ? prev : g_ld;
  *reinterpret_cast<float*>(st + h.lds_r + h.pub) = prev * __builtin_amdgcn_rcpf(u);
  *reinterpret_cast<float*>(lds + h.lds_u + h.pub) = u;
  u_prev = u;
}

// Workgroup barrier without the release/acquire fences of __syncthreads():
// those make the compiler wait for every outstanding memory operation,
// including the in-flight stage DMA.  Each use below states the waits it
// needs explicitly; the memory clobber keeps the compiler from moving memory
// accesses across the barrier.
__device__ __forceinline__ void wg_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// s_waitcnt that the scheduler may not move other instructions across.
#define PINNED_WAITCNT(imm)            \
  do {                                 \
    __builtin_amdgcn_sched_barrier(0); \
    __builtin_amdgcn_s_waitcnt(imm);   \
    __builtin_amdgcn_sched_barrier(0); \
  } while (0)

// Empty asm statements that "redefine" values: volatile asm keeps its order
// relative to the barriers, so values passed through one cannot be computed
// on the other side of a barrier (the MFMAs have no memory effects and would
// otherwise be free to drift across phases).
__device__ __forceinline__ void pin_frags(v8i (&fa)[2], v8i (&fb)[4]) {
  asm volatile("" : "+v"(fa[0]), "+v"(fa[1]), "+v"(fb[0]), "+v"(fb[1]), "+v"(fb[2]), "+v"(fb[3]));
}
__device__ __forceinline__ void pin_acc(v16f (&acc)[2][4]) {
  asm volatile("" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[0][2]), "+v"(acc[0][3]));
  asm volatile("" : "+v"(acc[1][0]), "+v"(acc[1][1]), "+v"(acc[1][2]), "+v"(acc[1][3]));
}

__device__ __forceinline__ uint32_t lds_u32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ __forceinline__ float lds_f32(const uint8_t* p) { return *reinterpret_cast<const float*>(p); }

// B group maxima granularity BG: one per 32 B rows (0), per 4 rows (1), or
// per row (2); the lane holds NJ values per 32-column tile ni.
template <int BG>
struct BGran {
  static constexpr int NJ = BG == 0 ? 1 : (BG == 1 ? 4 : 16);
  // index of accumulator element v (B row 8 * (v >> 2) + 4 * lhi + (v & 3))
  static constexpr int j_of(int v) { return BG == 0 ? 0 : (BG == 1 ? (v >> 2) : v); }
};

// The lane's entries of a stage's unit (or unit ratio) arrays: its A rows
// wm*64 + mi*32 + l32 (mi = 0, 1), and its B rows wn*128 + ni*32 + 8j + 4*lhi
// (+ i = 0..3 with BG 2; j = 0..3 with BG 1, 2) or wn*128 + ni*32 (BG 0).
template <int BG>
__device__ __forceinline__ void load_units(const uint8_t* a, const uint8_t* b, int wm, int wn, int lane,
                                           float (&uA)[2], float (&uB)[4][BGran<BG>::NJ]) {
  const int l32 = lane & 31, lhi = lane >> 5;
  const v2f va = *reinterpret_cast<const v2f*>(a + (wm * 64 + l32 * 2) * 4);
  uA[0] = va.x;
  uA[1] = va.y;
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) {
    if constexpr (BG == 2) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4f vb = *reinterpret_cast<const v4f*>(b + (wn * 128 + (ni * 2 + lhi) * 16 + j * 4) * 4);
        uB[ni][4 * j + 0] = vb.x;
        uB[ni][4 * j + 1] = vb.y;
        uB[ni][4 * j + 2] = vb.z;
        uB[ni][4 * j + 3] = vb.w;
      }
    } else if constexpr (BG == 1) {
      const v4f vb = *reinterpret_cast<const v4f*>(b + (wn * 32 + (ni * 2 + lhi) * 4) * 4);
      uB[ni][0] = vb.x;
      uB[ni][1] = vb.y;
      uB[ni][2] = vb.z;
      uB[ni][3] = vb.w;
    } else {
      uB[ni][0] = lds_f32(b + (wn * 32 + ni * 8) * 4);
    }
  }
}

// acc[mi][ni][v] *= uA(row) * uB(column) with the unit (ratio) arrays at a, b.
// Per-row B values (BG 2) are read 4 at a time (one 16-byte read per lane),
// with scheduling barriers between the reads so that the compiler does not
// hold all 64 beside the accumulator (the kernel is at its register limit).
template <int BG>
__device__ __forceinline__ void scale_by_units(v16f (&acc)[2][4], const uint8_t* a, const uint8_t* b, int wm,
                                               int wn, int lane) {
  if constexpr (BG == 2) {
    const int l32 = lane & 31, lhi = lane >> 5;
    const v2f va = *reinterpret_cast<const v2f*>(a + (wm * 64 + l32 * 2) * 4);
    const uint8_t* bl = b + (wn * 128 + lhi * 16) * 4;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        __builtin_amdgcn_sched_barrier(0);
        const v4f vb = *reinterpret_cast<const v4f*>(bl + (ni * 32 + j * 4) * 4);
        const float u[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[0][ni][4 * j + i] *= va.x * u[i];
          acc[1][ni][4 * j + i] *= va.y * u[i];
        }
      }
    __builtin_amdgcn_sched_barrier(0);
  } else {
    float rA[2], rB[4][BGran<BG>::NJ];
    load_units<BG>(a, b, wm, wn, lane, rA, rB);
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[mi][ni][v] *= rA[mi] * rB[ni][BGran<BG>::j_of(v)];
  }
}

// Output tile of workgroup `bid`: XCD-aware numbering (see the file header).
__host__ __device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int* tm, int* tn) {
  const int T = tiles_m * tiles_n;
  int L = bid;
  if (T % 8 == 0) L = (bid % 8) * (T / 8) + bid / 8;
  const int GM = tiles_m < 4 ? tiles_m : 4;
  const int band = L / (GM * tiles_n);
  const int rows_in_band = (tiles_m - band * GM) < GM ? (tiles_m - band * GM) : GM;
  const int w = L - band * GM * tiles_n;
  *tm = band * GM + w % rows_in_band;
  *tn = w / rows_in_band;
}

// Output requantization in the epilogue (pratchya_gemm_bs_nt_fq): the output
// is fake-quantized with tgrid (1, 128), whose groups are 1024 columns of one
// row, i.e. one "strip" of four 256-wide tiles.  The four workgroups of a
// strip run in the same round of the persistent schedule and exchange their
// row maxima through `gmax` (device-scope atomic max of |x| bits) and an
// arrival count per strip; both are zeroed before the launch.
struct FqArgs {
  uint8_t* sc8;        // output e8m0 bytes [M, N / 128]
  float* sc32;         // output group maxima [M, N / 1024]
  uint32_t* gmax;      // per strip: 256 row group maxima (|x| bits)
  uint32_t* arrive;    // per strip: workgroups that published their maxima
  uint32_t* status;    // set to 1 if a strip's partners did not arrive in time
  int xcd;             // strip partners: workgroups b, b+8, b+16, b+24 (1) or b..b+3 (0)
  // Newton-Schulz combination in the epilogue (FQ 3): X [M, N] bf16 (row
  // stride ldx elements), read where the tile's product is stored
  const uint16_t* ns_x;
  int64_t ldx;
  // Symmetric product C = A A^T (FQ == 4, pratchya_gemm_bf16_gram): only the
  // tri * (tri + 1) / 2 tiles (i, j), i <= j, of the tile grid are computed.
  // Their K steps (steps per tile) form one sequence of iters = tiles * steps
  // steps, numbered tile by tile; workgroup r takes the contiguous range
  // [r * iters / G, (r + 1) * iters / G) ("stream-K"), so every workgroup does
  // the same work.  A tile split between ranges is finished by the range that
  // holds its first step (its "head", the last unit of that range): the later
  // ranges that hold the rest of its steps reach them first, store the f32
  // accumulators of each wave in part (slot = range), and raise flags[range *
  // 8 + wave]; the head adds those partials in range order and stores the
  // tile.  A flag not raised in time sets the status word and makes the
  // tile's sums NaN.
  float* part;
  uint32_t* flags;
  // Block maxima of the f32 output (FQ 5, pratchya_gemm_bs_blockmax): for
  // each 128 x 128 block of C, max |c| as f32 bits (the block maxima of
  // quantize_impl with tgrid (128, 128), Q:484-487), block (r, c) at
  // r * bmax_ld + c
  uint32_t* bmax;
  int bmax_ld;
  int64_t iters;
  int steps;
  int tri;
  int order16;          // tiles in kGramOrder16's order (tri 16, 256 ranges, steps % 32 == 0)
};

// Tile order of the 16 x 16 tile grid (M = 4096) on 256 ranges with a
// multiple of 32 steps per tile: range r starts at step 17 r S / 32, so the
// ranges r = m + 32 n (n = 0..7), which run on one XCD, are at the same K
// step at all times, on tiles q0 + 17 n.  The order makes each such set
// {a + 17 n} a block of tiles over 4 to 6 panels (mostly 2 x 4 tiles; one
// set of near-diagonal tiles spans 8), so the 8 workgroups read the same K
// slices of few panels and share them in their XCD's L2.  Entry q is
// 16 i + j of tile (i, j).
__constant__ uint8_t kGramOrder16[136] = {
    2, 6, 10, 36, 40, 44, 70, 74, 104, 108, 138, 172, 0, 68, 136, 204, 35,
    3, 7, 11, 37, 41, 45, 71, 75, 105, 109, 139, 173, 1, 69, 137, 205, 51,
    4, 8, 12, 38, 42, 46, 72, 76, 106, 110, 140, 174, 17, 85, 153, 221, 103,
    5, 9, 13, 39, 43, 47, 73, 77, 107, 111, 141, 175, 14, 78, 142, 206, 119,
    18, 22, 26, 52, 56, 60, 86, 90, 120, 124, 154, 188, 15, 79, 143, 207, 171,
    19, 23, 27, 53, 57, 61, 87, 91, 121, 125, 155, 189, 30, 94, 158, 222, 187,
    20, 24, 28, 54, 58, 62, 88, 92, 122, 126, 156, 190, 31, 95, 159, 223, 239,
    21, 25, 29, 55, 59, 63, 89, 93, 123, 127, 157, 191, 34, 102, 170, 238, 255,
};

// Upper-triangle tile q of a tri x tri tile grid: by kGramOrder16 (order16),
// else numbered row by row.
__device__ __forceinline__ void tri_of(int q, int tri, bool order16, int* ti, int* tj) {
  if (order16) {
    const int v = kGramOrder16[q];
    *ti = v >> 4;
    *tj = v & 15;
    return;
  }
  int i = 0, base = 0;
  while (q >= base + (tri - i)) {
    base += tri - i;
    ++i;
  }
  *ti = i;
  *tj = i + (q - base);
}

// Gram partials: wave `wave` of range r holds its 128 accumulators per lane
// in 32 float4 columns of 64 lanes (1 KB each, coalesced).
//
// The exchange crosses XCDs, whose L2 caches are not coherent with each
// other.  Every partial store and load is issued at device scope (the sc1
// cache policy, which is also how device-scope atomic loads and stores are
// issued): a store is written through to the device's coherence point and is
// counted complete (vmcnt) only once performed there, and a load is served
// from that point, never from a stale line of this XCD's L2.  So the writer
// waits for its stores to complete and then raises the flag (an atomic), and
// a reader that has seen the flag reads the partial directly -- without the
// device-scope release and acquire fences, which write back and invalidate
// the whole L2 (measured: 18% of the kernel's time).
constexpr int kSc1 = 16;           // cache policy bit sc1 of buffer loads and stores
constexpr int kNt = 2;             // cache policy bit nt (non-temporal: data read once)

__device__ __forceinline__ float* gram_slot(const FqArgs& fq, int r, int wave) {
  return fq.part + ((int64_t)r * 8 + wave) * (32 * 256);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gram_rsrc(const FqArgs& fq, int r, int wave) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)gram_slot(fq, r, wave), 0, 32 * 1024, 0x00020000);
}

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void gram_put_partial(const v16f (&acc)[2][4], const FqArgs& fq, int r, int wave,
                                                 int lane) {
  const __amdgpu_buffer_rsrc_t rs = gram_rsrc(fq, r, wave);
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        // (a whole-vector cast: hipcc miscompiles __builtin_bit_cast of a
        // vector element lvalue into a cast of element 0)
        const v4u d = __builtin_bit_cast(
            v4u, v4f{acc[mi][ni][4 * v4], acc[mi][ni][4 * v4 + 1], acc[mi][ni][4 * v4 + 2], acc[mi][ni][4 * v4 + 3]});
        __builtin_amdgcn_raw_buffer_store_b128(d, rs, (((mi * 4 + ni) * 4 + v4) * 256 + lane * 4) * 4, 0, kSc1);
      }
  // vmcnt(0): the partial is performed at device scope before the flag (the
  // memory clobbers keep the compiler from moving either across the wait)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);
  asm volatile("" ::: "memory");
  if (lane == 0) __hip_atomic_fetch_add(fq.flags + r * 8 + wave, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The head of tile q (range r of G) adds the partials of the later ranges
// that hold steps of q, in range order.
__device__ __forceinline__ void gram_add_partials(v16f (&acc)[2][4], const FqArgs& fq, int r, int G, int q,
                                                  int wave, int lane) {
  const int64_t tile_end = (int64_t)(q + 1) * fq.steps;
  for (int r2 = r + 1; r2 < G && (int64_t)r2 * fq.iters / G < tile_end; ++r2) {
    uint32_t ok = 1;
    if (lane == 0) {
      uint32_t* f = fq.flags + r2 * 8 + wave;
      // the later ranges are resident (one workgroup per CU, grid <= CUs) and
      // reach this tile's steps first; the bound only keeps a broken launch
      // from spinning forever.  The flag is read with a returning atomic, as
      // it was raised with one (both performed where atomics on it are
      // serialized).
      for (int it = 0; __hip_atomic_fetch_add(f, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u; ++it) {
        if (it >= (1 << 20)) {
          __hip_atomic_fetch_or(fq.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    if (!__builtin_amdgcn_readfirstlane(ok)) {
#pragma unroll
      for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
          for (int v = 0; v < 16; ++v) acc[mi][ni][v] = __builtin_nanf("");
      continue;
    }
    asm volatile("" ::: "memory");         // the partial's loads stay after the flag was seen
    const __amdgpu_buffer_rsrc_t rs = gram_rsrc(fq, r2, wave);
    // one 16-value accumulator block at a time (the memory clobber keeps the
    // next block's loads after this block's adds: the accumulators leave no
    // room for more loaded values)
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        v4f p[4];
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4)
          p[v4] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                              rs, (((mi * 4 + ni) * 4 + v4) * 256 + lane * 4) * 4, 0, kSc1));
#pragma unroll
        for (int v4 = 0; v4 < 4; ++v4)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[mi][ni][4 * v4 + e] += p[v4][e];
        asm volatile("" ::: "memory");
      }
  }
}

// Output tile of workgroup-tile counter `bid` with output requantization: the
// four tiles of a strip get consecutive numbers L (L % 4 = tile in the strip),
// and L is XCD-aware as in tile_of when `xcd` (the counters b, b+8, b+16, b+24
// of the workgroups on one XCD then hold one strip); bands of up to 4 tile rows
// are walked strip by strip.
__host__ __device__ __forceinline__ void tile_of_fq(int bid, int tiles_m, int tiles_n, bool xcd, int* tm, int* tn) {
  const int T = tiles_m * tiles_n;
  int L = xcd ? (bid % 8) * (T / 8) + bid / 8 : bid;
  const int q = L & 3;
  L >>= 2;
  const int S = tiles_n >> 2;              // strips per tile row
  const int GM = tiles_m < 4 ? tiles_m : 4;
  const int band = L / (GM * S);
  const int rows_in_band = (tiles_m - band * GM) < GM ? (tiles_m - band * GM) : GM;
  const int w = L - band * GM * S;
  *tm = band * GM + w % rows_in_band;
  *tn = (w / rows_in_band) * 4 + q;
}

// First row of tile t along a dimension of n rows: t * 256, except that the
// last tile of a dimension of at least 256 rows that is not a multiple of 256
// is moved back to end at row n: it overlaps the previous tile, whose outputs
// it recomputes with the same values, and every row it reads exists.  (B's
// scale groups stay aligned: an N quantized in blocks of 32 or more rows is a
// multiple of them, and the host requires N % 4 == 0 for finer groups.)  A
// dimension below 256 rows has one tile at 0: its operand buffer holds 256
// readable rows, and outputs beyond n are not stored.
__host__ __device__ __forceinline__ int tile_base(int t, int n) {
  const int b = t * 256;
  return (n >= 256 && b > n - 256) ? n - 256 : b;
}

// Quantize prologue (QA, pratchya_gemm_bs_nt_qa): the A operand is
// quantize_impl(X, (1, 128)) of a bf16 activation X [M, K] (Q:458-506; the
// quantized Linear's QArrayImpl(x, (1, a)) @ kernel, pratchya/_nnx_impl/
// _module.py:46-50), computed inside the GEMM's launch, once per row, and
// written to the caller's payload and scale arrays, which the GEMM then reads
// as its A operand.
//
// Work: the 1024-element groups of X (K / 1024 per row, in row order), cut
// into runs of 32 consecutive groups (one line of group maxima, two lines of
// e8m0 bytes).  Workgroup b quantizes runs b, b + G, b + 2G, ... before its
// first tile, 4 groups per wave and run, three runs' loads (24 KB) in flight
// per wave while one run is quantized; then every workgroup waits
// until all have finished (a grid-wide count: the persistent grid is
// resident as a whole), and the tile loop runs exactly as without the
// prologue.  The prologue is a function of its own, called once, so that its
// registers (all free before the first tile) do not shape the allocation of
// the tile loop, whose scalar registers are all in use.  (Measured and not
// kept: spreading the runs over the tile boundaries, so that the quantization
// overlaps other workgroups' MFMA work, and per-tile waits for the rows a
// tile reads: either made the K loop reload spilled scalar registers.)
//
// Visibility across XCDs: every line of the payload and scale arrays is
// written by the waves of one workgroup (one XCD's L2), with stores issued at
// device scope (sc1: written through to the device's coherence point, counted
// complete by vmcnt only once performed there), and no XCD reads A before
// every store has been performed, so no L2 holds a line of it from before its
// writes (lines cached by earlier launches are not valid across a launch
// boundary).  Each workgroup adds 1 to the count (device-scope atomic) once
// all its waves have passed a vmcnt(0), and waits for G (bounded: a wait that
// runs out sets bit 2 of the status word; the outputs are then not defined).

// Buffer resources of the quantized outputs (range-checked, 32-bit offsets).
struct QaRsrc {
  __amdgpu_buffer_rsrc_t q, e8, g32;
};

struct QaArgs {
  const uint8_t* x;        // X, bf16 [M, K] (row stride ldx bytes)
  uint8_t* q;              // payload [M, K] (the GEMM's A, row stride K)
  uint8_t* sc8;            // e8m0 bytes [M, K / 128]
  float* sc32;             // group maxima [M, K / 1024]
  uint32_t* done;          // workgroups done with the prologue; then the status word
  int64_t ldx;
};
struct QaNone {};

template <typename T>
__device__ __forceinline__ T* qa_rfl(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// One group of 1024 bf16 values quantized by one wave, the arithmetic of
// k_quant_g8's bf16 payload path: v[r] holds the lane's 8 values at elements
// r * 512 + 8 lane.  Block max by DPP within 16-lane rows, group max G by
// readlane, e8m0 and 128 / S by block_scale, the division-free cast where no
// block is clamped (exact for bf16 inputs), else each 4-value word checked
// against the bf16 rounding midpoints and redone exactly near one; a group
// whose G is not finite takes the exact per-element path.  g: the group's
// index (row * K / 1024 + group in the row).
__device__ __forceinline__ void qa_quant_group(const QaRsrc& rs, const uint4 (&v)[2], int lane, int g) {
  uint32_t m[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) m[r] = lane_group_max<16>(absmax8_bf16(v[r]));
  uint32_t Gb = 0;
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int k = 0; k < 4; ++k) Gb = umax(Gb, readlane_u32(m[r], k * 16));
  const float G = u2f(Gb);
  uint32_t e[2], out[2][2];
  if ((Gb >> 23) < 255u) {
    const float rcpG128 = __builtin_amdgcn_rcpf(G * 0.0078125f);
    float y[2];
    uint32_t clamped = 0;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const BlockScale b = block_scale(m[r], Gb, rcpG128);
      e[r] = b.e;
      y[r] = b.y;
      clamped |= b.clamped ? 1u : 0u;
    }
    if (!__any(clamped)) {
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          out[r][j] = cvt4_hw(elem_f32<true>(v[r], 4 * j) * y[r], elem_f32<true>(v[r], 4 * j + 1) * y[r],
                              elem_f32<true>(v[r], 4 * j + 2) * y[r], elem_f32<true>(v[r], 4 * j + 3) * y[r]);
    } else {
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float x0 = elem_f32<true>(v[r], 4 * j), x1 = elem_f32<true>(v[r], 4 * j + 1);
          const float x2 = elem_f32<true>(v[r], 4 * j + 2), x3 = elem_f32<true>(v[r], 4 * j + 3);
          const float t0 = x0 * y[r], t1 = x1 * y[r], t2 = x2 * y[r], t3 = x3 * y[r];
          out[r][j] = cvt4_hw(t0, t1, t2, t3);
          if (mid_key4(t0, t1, t2, t3) <= kMidKey) out[r][j] = cvt4_exact(x0, x1, x2, x3, quant_scale(e[r], G));
        }
    }
  } else {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      e[r] = e8m0_of(u2f(m[r]), G);
      const float S = quant_scale(e[r], G);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        out[r][j] = cvt4_exact(elem_f32<true>(v[r], 4 * j), elem_f32<true>(v[r], 4 * j + 1),
                               elem_f32<true>(v[r], 4 * j + 2), elem_f32<true>(v[r], 4 * j + 3), S);
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r)
    __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{out[r][0], out[r][1]}, rs.q, g * 1024 + r * 512 + lane * 8, 0,
                                          kSc1);
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t ek = readlane_u32(e[k / 4], (k % 4) * 16);
    if (k < 4) lo |= ek << (8 * k);
    else hi |= ek << (8 * (k - 4));
  }
  const bool lead = lane == 0;
  __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{lo, hi}, rs.e8, lead ? g * 8 : kOutOfRange, 0, kSc1);
  __builtin_amdgcn_raw_buffer_store_b32(f2u(G), rs.g32, lead ? g * 4 : kOutOfRange, 0, kSc1);
}

// Groups 4 wave .. 4 wave + 3 of run R: their indices (ngroups marks none:
// past the last group) and their loads, issued for every group (past the
// last, at an offset the range check turns into zeros), so that the number of
// memory operations in flight never depends on a branch and the waits count
// exactly.
__device__ __forceinline__ void qa_load_run(const __amdgpu_buffer_rsrc_t& rx, int64_t ldx, int gpr, int ngroups,
                                            int R, int wave, int lane, int (&g)[4], uint4 (&v)[4][2]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int gg = R * 32 + wave * 4 + j;
    const bool ok = gg < ngroups;
    g[j] = ok ? gg : ngroups;
    const int row = gg / gpr, gi = gg - row * gpr;
    const int off = (int)(row * ldx) + gi * 2048 + lane * 16;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      v[j][h] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? off + h * 1024 : kOutOfRange,
                                                                                 0, kNt));
  }
}

__device__ __forceinline__ void qa_quant_run(const QaRsrc& rs, const uint4 (&v)[4][2], int lane, const int (&g)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) qa_quant_group(rs, v[j], lane, g[j]);
}

// The quantize prologue of one wave (see above), then the grid-wide wait.
__device__ __attribute__((noinline)) void qa_prologue(const uint8_t* x, uint8_t* q, uint8_t* sc8, float* sc32,
                                                      uint32_t* done, int64_t ldx, int M, int K, int wave,
                                                      int lane) {
  x = qa_rfl(x);
  q = qa_rfl(q);
  sc8 = qa_rfl(sc8);
  sc32 = qa_rfl(sc32);
  done = qa_rfl(done);
  ldx = ((int64_t)__builtin_amdgcn_readfirstlane((int)(ldx >> 32)) << 32) |
        (uint32_t)__builtin_amdgcn_readfirstlane((int)ldx);
  M = __builtin_amdgcn_readfirstlane(M);
  K = __builtin_amdgcn_readfirstlane(K);
  wave = __builtin_amdgcn_readfirstlane(wave);
  const int gpr = K >> 10, ngroups = M * gpr, runs = (ngroups + 31) >> 5, G = (int)gridDim.x, b = (int)blockIdx.x;
  // (the host keeps X within 2^31 bytes)
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(x), 0, (int)((M - 1) * ldx + 2 * (int64_t)K), kRawBuffer);
  QaRsrc rs;
  rs.q = __builtin_amdgcn_make_buffer_rsrc(q, 0, (int)((int64_t)M * K), kRawBuffer);
  rs.e8 = __builtin_amdgcn_make_buffer_rsrc(sc8, 0, ngroups * 8, kRawBuffer);
  rs.g32 = __builtin_amdgcn_make_buffer_rsrc(sc32, 0, ngroups * 4, kRawBuffer);
  // four buffers of one run each in rotation: three runs' loads in flight
  // while one is quantized; every load and store is issued on every pass
  uint4 v0[4][2], v1[4][2], v2[4][2], v3[4][2];
  int g0[4], g1[4], g2[4], g3[4];
  qa_load_run(rx, ldx, gpr, ngroups, b, wave, lane, g0, v0);
  qa_load_run(rx, ldx, gpr, ngroups, b + G, wave, lane, g1, v1);
  qa_load_run(rx, ldx, gpr, ngroups, b + 2 * G, wave, lane, g2, v2);
  for (int R = b; R < runs; R += 4 * G) {
    qa_load_run(rx, ldx, gpr, ngroups, R + 3 * G, wave, lane, g3, v3);
    qa_quant_run(rs, v0, lane, g0);
    if (R + G >= runs) break;
    qa_load_run(rx, ldx, gpr, ngroups, R + 4 * G, wave, lane, g0, v0);
    qa_quant_run(rs, v1, lane, g1);
    if (R + 2 * G >= runs) break;
    qa_load_run(rx, ldx, gpr, ngroups, R + 5 * G, wave, lane, g1, v1);
    qa_quant_run(rs, v2, lane, g2);
    if (R + 3 * G >= runs) break;
    qa_load_run(rx, ldx, gpr, ngroups, R + 6 * G, wave, lane, g2, v2);
    qa_quant_run(rs, v3, lane, g3);
  }
  // every wave's stores performed (device scope) before the workgroup is
  // counted: one atomic per workgroup on the shared count, and one poller
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);
  asm volatile("" ::: "memory");
  __syncthreads();
  if (wave == 0 && lane == 0) {
    __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // the grid is resident as a whole (one workgroup per CU, grid <= CUs);
    // the bound only keeps a broken launch from spinning forever
    for (int it = 0; __hip_atomic_fetch_add(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (uint32_t)G;
         ++it) {
      if (it >= (1 << 20)) {
        __hip_atomic_fetch_or(done + 1, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(16);
    }
  }
  asm volatile("" ::: "memory");       // the operand loads stay after the count was seen
  __syncthreads();
}

// Epilogue: C[m][n] = acc * gA * gB / 2^14 (the two /128 of the dequant) for
// this wave's 64 x 128 sub-tile at (row0, col0); with per-row B units (BG 2)
// gB comes from the unit array at ub (the lane's entries, see load_units),
// read 4 columns at a time where they are applied.  The waves stage RP rows x
// 128 columns each at a time in one LDS stage buffer (free once every wave has
// passed the barrier below) and write them back as full 16-byte lane chunks
// covering whole rows, with non-temporal stores (the output is not read again
// by this kernel; streaming it keeps the operand panels in L2).
// BMAX: also returns the lane's max |c| (f32 bits) over the values it wrote.
template <bool OUT_BF16, int BG, bool BMAX = false>
__device__ __forceinline__ uint32_t store_tile(const v16f (&acc)[2][4], const float (&gA)[2],
                                               const float (&gB)[4][BG == 1 ? 4 : 1], const uint8_t* ub,
                                               uint8_t* stage, int wave, int lane, void* C, int64_t ldc, int row0,
                                               int col0, int M, int N) {
  const int l32 = lane & 31, lhi = lane >> 5;
  uint32_t lmax = 0;
  constexpr int ESZ = OUT_BF16 ? 2 : 4;
  constexpr int ROWB = 128 * ESZ;           // bytes of one staged row
  constexpr int PITCH = ROWB + 16;          // padded LDS row pitch
  constexpr int CHUNKS = ROWB / 16;         // 16-byte chunks per row
  constexpr int RP = OUT_BF16 ? 32 : 16;    // rows staged per pass
  static_assert(8 * RP * PITCH <= STAGE_BYTES, "staging must fit one stage buffer");
  uint8_t* stg = stage + wave * (RP * PITCH);
  __syncthreads();                          // every wave is done with the stage buffer
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
    for (int p = 0; p < 32 / RP; ++p) {
      if (RP == 32 || (l32 / RP) == p) {    // lanes whose row is staged in this pass
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int col = ni * 32 + 8 * j + 4 * lhi;
            float f0, f1, f2, f3;
            if constexpr (BG == 2) {
              const v4f u = *reinterpret_cast<const v4f*>(ub + (ni * 32 + j * 4) * 4);
              const float fa = gA[mi] * 6.103515625e-05f;
              f0 = fa * u.x;
              f1 = fa * u.y;
              f2 = fa * u.z;
              f3 = fa * u.w;
            } else {
              f0 = f1 = f2 = f3 = gA[mi] * gB[ni][BG == 1 ? j : 0] * 6.103515625e-05f;
            }
            const float c0 = acc[mi][ni][4 * j + 0] * f0, c1 = acc[mi][ni][4 * j + 1] * f1;
            const float c2 = acc[mi][ni][4 * j + 2] * f2, c3 = acc[mi][ni][4 * j + 3] * f3;
            uint8_t* dst = stg + (l32 % RP) * PITCH + col * ESZ;
            if constexpr (OUT_BF16) {
              typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
              const bf16x2 p0 = {(__bf16)c0, (__bf16)c1};
              const bf16x2 p1 = {(__bf16)c2, (__bf16)c3};
              *reinterpret_cast<uint2*>(dst) =
                  make_uint2(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1));
            } else {
              *reinterpret_cast<float4*>(dst) = make_float4(c0, c1, c2, c3);
              if constexpr (BMAX)
                lmax = umax(umax(lmax, umax(abs_bits(c0), abs_bits(c1))), umax(abs_bits(c2), abs_bits(c3)));
            }
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's staging writes are done
      // rows row0 + mi*32 + p*RP + [0, RP), columns col0 + [0, 128)
      uint8_t* Cb = static_cast<uint8_t*>(C) + ((int64_t)(row0 + mi * 32 + p * RP) * ldc + col0) * ESZ;
#pragma unroll
      for (int it = 0; it < (RP * CHUNKS) / 64; ++it) {
        const int q = it * 64 + lane;
        const int r = q / CHUNKS, c = q % CHUNKS;
        const v4i v = *reinterpret_cast<const v4i*>(stg + r * PITCH + c * 16);
        // rows / columns beyond [M, N] (a dimension below one tile) are not stored
        if (row0 + mi * 32 + p * RP + r < M && col0 + c * (16 / ESZ) < N)
          __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(Cb + (int64_t)r * ldc * ESZ + c * 16));
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);   // staging reads done before the next pass overwrites
    }
  }
  return lmax;
}

// The 128 x 128 block maxima of a tile (FQ 5): each wave's max over its 64 x
// 128 values (lanes by xor shuffles), the two waves of a block row (wm = 2 br,
// 2 br + 1, same wn) combined through LDS, one plain store per block (the
// tiles partition C, so every block is written by one workgroup; an edge tile
// moved back by 128 rows or columns writes its overlap's maxima again, the
// same values; blocks past M or N, of a dimension below one tile, are not
// written).  The barrier waits for LDS only: the output stores stay in flight.
__device__ __forceinline__ void store_block_max(uint32_t lmax, uint32_t* slot, const FqArgs& fq, int wave, int lane,
                                                int row0, int col0, int M, int N) {
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) lmax = umax(lmax, shfl_xor_u32(lmax, s));
  if (lane == 0) slot[wave] = lmax;
  PINNED_WAITCNT(0xC07F);
  wg_barrier();
  if ((wave & 1) == 0 && lane == 0 && row0 < M && col0 < N) {
    const uint32_t m = umax(slot[wave], slot[wave + 1]);
    fq.bmax[(int64_t)(row0 >> 7) * fq.bmax_ld + (col0 >> 7)] = m;
  }
}

// Output requantization with tgrid (1, 1) in the epilogue (FQ 6,
// pratchya_gemm_bs_nt_q11): every element is its own block and group, so no
// workgroup needs another's maxima.  Per element c (the value store_tile
// would write): fake_quant11's dequantized value in the output dtype, its
// e8m0 byte and its group max |c| (the arrays quantize_impl(C, (1, 1))
// returns, both [M, N] in row order, row stride N).  The f32 tile is staged
// through the wave's LDS slice 16 rows at a time, as store_tile stages an f32
// output; the maxima are written from there; each lane then reads 2 x 16
// consecutive values of the staged rows, casts them, and writes the values
// and e8m0 bytes back into the slice in row layout (the f32 values in place,
// the bytes in a pass of their own); every array leaves the slice as whole
// 16-byte chunks, consecutive lanes on consecutive chunks of a row, so that
// each store instruction writes whole lines (non-temporal).  N is a multiple
// of 16, so no chunk straddles the edge of a partial tile.
template <bool OUT_BF16, int BG>
__device__ __forceinline__ void store_tile_q11(const v16f (&acc)[2][4], const float (&gA)[2],
                                               const float (&gB)[4][BG == 1 ? 4 : 1], const uint8_t* ub,
                                               uint8_t* stage, int wave, int lane, void* C, int64_t ldc,
                                               uint8_t* sc8, float* sc32, int row0, int col0, int M, int N) {
  const int l32 = lane & 31, lhi = lane >> 5;
  constexpr int RP = 16;                    // rows staged per pass
  constexpr int PITCH = 512 + 16;           // padded LDS pitch of a row of 128 f32
  static_assert(8 * RP * PITCH <= STAGE_BYTES, "staging must fit one stage buffer");
  constexpr int ESZ = OUT_BF16 ? 2 : 4;
  constexpr int E8_AT = OUT_BF16 ? 256 : 0; // byte of a staged row where its e8m0 bytes go
  uint8_t* stg = stage + wave * (RP * PITCH);
  // the staged rows to dst + row * ld (rowb bytes of a row at byte `at`,
  // colw output columns per chunk), output rows rbase + [0, 16)
  auto copy_out = [&](uint8_t* dst, int64_t ld, int at, int rowb, int colw, int rbase, bool absval) {
    const int chunks = rowb / 16;
#pragma unroll 1
    for (int q = lane; q < RP * chunks; q += 64) {
      const int r = q / chunks, c = q % chunks;
      v4i v = *reinterpret_cast<const v4i*>(stg + r * PITCH + at + c * 16);
      if (absval) v &= 0x7FFFFFFF;
      if (rbase + r < M && col0 + c * colw < N)
        __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(dst + (int64_t)(rbase + r) * ld + c * 16));
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);     // staging reads done before the slice is written again
  };
  __syncthreads();                          // every wave is done with the stage buffer
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if ((l32 >> 4) == p) {                // lanes whose row is staged in this pass
        uint8_t* srow = stg + (l32 % RP) * PITCH;
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float f0, f1, f2, f3;
            if constexpr (BG == 2) {
              const v4f u = *reinterpret_cast<const v4f*>(ub + (ni * 32 + j * 4) * 4);
              const float fa = gA[mi] * 6.103515625e-05f;
              f0 = fa * u.x;
              f1 = fa * u.y;
              f2 = fa * u.z;
              f3 = fa * u.w;
            } else {
              f0 = f1 = f2 = f3 = gA[mi] * gB[ni][BG == 1 ? j : 0] * 6.103515625e-05f;
            }
            *reinterpret_cast<float4*>(srow + (ni * 32 + 8 * j + 4 * lhi) * 4) =
                make_float4(acc[mi][ni][4 * j] * f0, acc[mi][ni][4 * j + 1] * f1, acc[mi][ni][4 * j + 2] * f2,
                            acc[mi][ni][4 * j + 3] * f3);
          }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): this wave's staging writes are done
      const int rbase = row0 + mi * 32 + p * RP;
      // group maxima |c|
      copy_out(reinterpret_cast<uint8_t*>(sc32 + col0), (int64_t)N * 4, 0, 512, 4, rbase, true);
      // the lane's segments: values 16 s + [0, 16) of staged row r, for
      // q = lane + 64 h (r = q / 8, s = q % 8): half h reads rows 8 h + [0, 8)
      // and writes its results back into the same rows once every lane's
      // reads of them are done
      uint32_t ew[2][4] = {};                // f32 output: the bytes kept for their own pass
#pragma unroll 1
      for (int h = 0; h < 2; ++h) {
        uint8_t* row = stg + ((h * 64 + lane) >> 3) * PITCH;
        const int s = lane & 7;
        float v[16];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const v4f xx = *reinterpret_cast<const v4f*>(row + s * 64 + k * 16);
          v[4 * k] = xx.x;
          v[4 * k + 1] = xx.y;
          v[4 * k + 2] = xx.z;
          v[4 * k + 3] = xx.w;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F); // every lane's reads of these rows are done
        uint32_t e[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          uint32_t e0, e1, e2, e3;
          v[4 * k] = fake_quant11(v[4 * k], e0);
          v[4 * k + 1] = fake_quant11(v[4 * k + 1], e1);
          v[4 * k + 2] = fake_quant11(v[4 * k + 2], e2);
          v[4 * k + 3] = fake_quant11(v[4 * k + 3], e3);
          e[k] = e0 | (e1 << 8) | (e2 << 16) | (e3 << 24);
        }
        if constexpr (OUT_BF16) {
#pragma unroll
          for (int k = 0; k < 2; ++k)
            *reinterpret_cast<v4i*>(row + s * 32 + k * 16) =
                v4i{(int)pack_bf16x2(v[8 * k], v[8 * k + 1]), (int)pack_bf16x2(v[8 * k + 2], v[8 * k + 3]),
                    (int)pack_bf16x2(v[8 * k + 4], v[8 * k + 5]), (int)pack_bf16x2(v[8 * k + 6], v[8 * k + 7])};
          *reinterpret_cast<v4i*>(row + E8_AT + s * 16) = v4i{(int)e[0], (int)e[1], (int)e[2], (int)e[3]};
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k)
            *reinterpret_cast<v4f*>(row + s * 64 + k * 16) = v4f{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            ew[0][k] = h == 0 ? e[k] : ew[0][k];
            ew[1][k] = h == 1 ? e[k] : ew[1][k];
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);
      uint8_t* Cb = static_cast<uint8_t*>(C) + (int64_t)col0 * ESZ;
      copy_out(Cb, ldc * ESZ, 0, 128 * ESZ, 16 / ESZ, rbase, false);
      if constexpr (!OUT_BF16) {
        // the f32 values filled the rows: the e8m0 bytes in a pass of their own
#pragma unroll
        for (int h = 0; h < 2; ++h)
          *reinterpret_cast<v4i*>(stg + ((h * 64 + lane) >> 3) * PITCH + E8_AT + (lane & 7) * 16) =
              v4i{(int)ew[h][0], (int)ew[h][1], (int)ew[h][2], (int)ew[h][3]};
        __builtin_amdgcn_s_waitcnt(0xC07F);
      }
      copy_out(sc8 + col0, N, E8_AT, 128, 16, rbase, false);
    }
  }
}

// Epilogue of the Gram product (bf16 output): the tile as store_tile writes
// it and, for a tile off the diagonal (mirror), its transpose at the mirrored
// position: from each pass's 32 staged rows, a lane takes a column pair and
// 8 rows and writes the two transposed 16-byte row chunks.  (A diagonal tile
// is symmetric as computed: its two triangles hold the same products,
// summed in the same order.)
__device__ __forceinline__ void store_tile_gram(const v16f (&acc)[2][4], uint8_t* stage, int wave, int lane,
                                                void* C, int64_t ldc, int row0, int col0, bool mirror) {
  const int l32 = lane & 31, lhi = lane >> 5;
  constexpr int ROWB = 256;                 // 128 bf16 columns
  constexpr int PITCH = ROWB + 16;
  constexpr int CHUNKS = ROWB / 16;
  constexpr int RP = 32;
  uint8_t* stg = stage + wave * (RP * PITCH);
  __syncthreads();                          // every wave is done with the stage buffer
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = ni * 32 + 8 * j + 4 * lhi;
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        const bf16x2 p0 = {(__bf16)acc[mi][ni][4 * j + 0], (__bf16)acc[mi][ni][4 * j + 1]};
        const bf16x2 p1 = {(__bf16)acc[mi][ni][4 * j + 2], (__bf16)acc[mi][ni][4 * j + 3]};
        *reinterpret_cast<uint2*>(stg + l32 * PITCH + col * 2) =
            make_uint2(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1));
      }
    __builtin_amdgcn_s_waitcnt(0xC07F);     // lgkmcnt(0): this wave's staging writes are done
    uint8_t* Cb = static_cast<uint8_t*>(C) + ((int64_t)(row0 + mi * 32) * ldc + col0) * 2;
#pragma unroll
    for (int it = 0; it < (RP * CHUNKS) / 64; ++it) {
      const int q = it * 64 + lane;
      const int r = q / CHUNKS, c = q % CHUNKS;
      const v4i v = *reinterpret_cast<const v4i*>(stg + r * PITCH + c * 16);
      __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(Cb + (int64_t)r * ldc * 2 + c * 16));
    }
    if (mirror) {
      // output rows col0 + [0, 128), columns row0 + mi * 32 + [0, 32)
      uint8_t* Ct = static_cast<uint8_t*>(C) + ((int64_t)col0 * ldc + row0 + mi * 32) * 2;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int q = it * 64 + lane;
        const int cp = q >> 2, k = q & 3;   // columns 2 cp, 2 cp + 1; staged rows 8 k .. 8 k + 7
        uint32_t w[8];
#pragma unroll
        for (int x = 0; x < 8; ++x) w[x] = *reinterpret_cast<const uint32_t*>(stg + (8 * k + x) * PITCH + cp * 4);
        v4i lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[e] = (int)__builtin_amdgcn_perm(w[2 * e + 1], w[2 * e], 0x05040100u);
          hi[e] = (int)__builtin_amdgcn_perm(w[2 * e + 1], w[2 * e], 0x07060302u);
        }
        __builtin_nontemporal_store(lo, reinterpret_cast<v4i*>(Ct + (int64_t)(2 * cp) * ldc * 2 + k * 16));
        __builtin_nontemporal_store(hi, reinterpret_cast<v4i*>(Ct + (int64_t)(2 * cp + 1) * ldc * 2 + k * 16));
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);     // staging reads done before the next pass overwrites
  }
}

// Output requantization, QArrayImpl(C, (1, 128)).astype(dtype) (Q:458-506
// then Q:541-569; with FIXNAN, quantize_impl_bwd's dequantization that reads
// an e8m0 byte 255 as 1.0, Q:521-526), in two steps.
//
// fq_row_scales: the f32 product (acc scaled as the plain epilogue scales
// it), each row's max |x| over this wave's 128 columns (one block; lanes l32
// and l32 + 32 hold row mi * 32 + l32's values, 64 each), the group max over
// the strip's 8 blocks by the exchange described at FqArgs, and the scales of
// row lhi * 32 + l32 into this wave's 64-entry table in LDS (16 bytes per
// row: y, S, the dequantization factor, and flags: G finite, one multiply).  Writes the output scales of rows
// below M.
constexpr int FQ_TABLE_BYTES = 8 * 64 * 16;

template <bool FIXNAN>
__device__ __forceinline__ void fq_row_scales(v16f (&acc)[2][4], const float (&gA)[2], const float (&gB)[4][1],
                                              const FqArgs& fq, uint8_t* table, int strip, int tn, int wm,
                                              int wn, int lane, int row0, int col0, int M, int N) {
  const int l32 = lane & 31, lhi = lane >> 5;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      const float f = gA[mi] * gB[ni][0] * 6.103515625e-05f;
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mi][ni][v] *= f;
    }
  // block maxima as |x| bits (an unsigned max propagates NaN)
  uint32_t m[2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    uint32_t a = 0;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int v = 0; v < 16; ++v) a = umax(a, f2u(acc[mi][ni][v]) & 0x7FFFFFFFu);
    m[mi] = xor_max_u32<32>(a);
  }
  const uint32_t mb = lhi ? m[1] : m[0];      // this lane's row: lhi * 32 + l32
  uint32_t* gm = fq.gmax + (int64_t)strip * 256 + wm * 64 + lhi * 32 + l32;
  // Every access of the exchange is a device-scope read-modify-write atomic:
  // those on one address are serialized where they are performed, and one
  // that returns a value has been performed when the value arrives.  So a
  // workgroup's maxima are performed before its arrival is counted (the
  // returned values are awaited before the barrier), and a partner that has
  // read a count of 4 reads the group maxima after all of them -- with no
  // assumption about the visibility of plain stores or loads across XCDs.
  const uint32_t prev = __hip_atomic_fetch_max(gm, mb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("" ::"v"(prev));             // wait for the returned value
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t* cnt = fq.arrive + strip;
    uint32_t n = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    // the partners run in the same round of the schedule; the bound only keeps
    // a broken launch from spinning forever.  A timeout sets the status word
    // and raises the strip's maxima to a NaN pattern, so the strip's outputs
    // and scales come out NaN instead of quietly using a partial maximum.
    for (int it = 0; n < 4u; ++it) {
      if (it >= (1 << 20)) {
        __hip_atomic_fetch_or(fq.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t* g0 = fq.gmax + (int64_t)strip * 256;
        for (int r = 0; r < 256; ++r)
          __hip_atomic_fetch_max(g0 + r, 0x7FFFFFFFu, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
      n = __hip_atomic_fetch_add(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  const uint32_t Gb = __hip_atomic_fetch_max(gm, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const float G = u2f(Gb);
  const bool fin = (Gb >> 23) < 255u;
  BlockScale bs;
  if (fin) {
    bs = block_scale(mb, Gb, __builtin_amdgcn_rcpf(G * 0.0078125f));
  } else {
    bs.e = e8m0_of(u2f(mb), G);
    bs.y = 0.0f;
    bs.clamped = false;
  }
  const uint32_t ed = (FIXNAN && bs.e == 0xFFu) ? 0x7Fu : bs.e;
  const float dq = e8m0_decode(ed) * G;
  const bool one = dequant_one_mul(dq);
  *reinterpret_cast<v4f*>(table + (lhi * 32 + l32) * 16) =
      v4f{bs.y, quant_scale(bs.e, G), one ? dq * 0.0078125f : dq, u2f((fin ? 1u : 0u) | (one ? 2u : 0u))};
  // scales of the lane's row: its e8m0 byte for this block, and its group
  // max from the strip's first tile, left wave
  const int row = row0 + lhi * 32 + l32;
  if (row < M) {
    fq.sc8[(int64_t)row * (N >> 7) + (col0 >> 7)] = (uint8_t)bs.e;
    if ((tn & 3) == 0 && wn == 0) fq.sc32[(int64_t)row * (N >> 10) + (tn >> 2)] = G;
  }
}

// Epilogue of the output-requantizing GEMM: acc holds the f32 product; the
// waves stage 16 rows x 128 columns at a time (f32) in the free stage buffer,
// each lane takes a 4-column chunk of one row, fake-quantizes it with its row's
// scales from the table (fake_quant4), and stores the dequantized values
// (16 or 8 bytes; a row's 32 lanes write its 128 columns contiguously).
template <bool OUT_BF16>
__device__ __forceinline__ void store_tile_fq(const v16f (&acc)[2][4], uint8_t* stage, const uint8_t* table,
                                              int wave, int lane, void* C, int64_t ldc, int row0, int col0,
                                              int M) {
  const int l32 = lane & 31, lhi = lane >> 5;
  constexpr int OSZ = OUT_BF16 ? 2 : 4;
  constexpr int PITCH = 512 + 16;           // 128 f32 + padding
  constexpr int RP = 16;                    // rows staged per pass
  static_assert(8 * RP * PITCH <= STAGE_BYTES, "staging must fit one stage buffer");
  uint8_t* stg = stage + wave * (RP * PITCH);
  // the wave's output rows start at Cw; a row offset fits 32 bits (64 rows, ldc below 2^23)
  uint8_t* const Cw = static_cast<uint8_t*>(C) + ((int64_t)row0 * ldc + col0) * OSZ;
  __syncthreads();                          // every wave is done with the stage buffer
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if ((l32 >> 4) == p) {
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            *reinterpret_cast<v4f*>(stg + (l32 & 15) * PITCH + (ni * 32 + 8 * j + 4 * lhi) * 4) =
                v4f{acc[mi][ni][4 * j], acc[mi][ni][4 * j + 1], acc[mi][ni][4 * j + 2], acc[mi][ni][4 * j + 3]};
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): staging writes done
#pragma unroll 1
      for (int it = 0; it < 8; ++it) {
        const int r = it * 2 + lhi;         // staged row; chunk l32
        const int rw = mi * 32 + p * 16 + r;   // row within the wave's 64
        v4f x = *reinterpret_cast<const v4f*>(stg + r * PITCH + l32 * 16);
        const v4f sc = *reinterpret_cast<const v4f*>(table + rw * 16);
        const uint32_t flags = f2u(sc.w);
        float x0 = x.x, x1 = x.y, x2 = x.z, x3 = x.w;
        if (__all((flags & 3u) == 3u)) {
          // every row of the wave finite and dequantized with one multiply
          // (the common case): fake_quant4's arithmetic without its per-lane
          // selections of those two paths
          const float t0 = x0 * sc.x, t1 = x1 * sc.x, t2 = x2 * sc.x, t3 = x3 * sc.x;
          uint32_t w = cvt4_hw(t0, t1, t2, t3);
          if (mid_key4(t0, t1, t2, t3) <= kMidKey) w = cvt4_exact(x0, x1, x2, x3, sc.y);
          fp8_word(w, x0, x1, x2, x3);
          x0 *= sc.z;
          x1 *= sc.z;
          x2 *= sc.z;
          x3 *= sc.z;
        } else {
          fake_quant4(x0, x1, x2, x3, sc.x, sc.y, (flags & 1u) != 0u, sc.z, (flags & 2u) != 0u);
        }
        if (row0 + rw < M) {
          uint8_t* dst = Cw + (uint32_t)((rw * (int)ldc + l32 * 4) * OSZ);
          if constexpr (OUT_BF16) {
            __builtin_nontemporal_store(u32x2_t{pack_bf16x2(x0, x1), pack_bf16x2(x2, x3)},
                                        reinterpret_cast<u32x2_t*>(dst));
          } else {
            __builtin_nontemporal_store(u32x4_t{f2u(x0), f2u(x1), f2u(x2), f2u(x3)},
                                        reinterpret_cast<u32x4_t*>(dst));
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);   // staging reads done before the next pass overwrites
    }
  }
}

// Epilogue of the bf16 product fused with the Newton-Schulz combination
// X <- 1.5 X - 0.5 B (pratchya/_nnx_impl/_optimizer.py:26-27): the product B
// is rounded to bf16 as the plain epilogue rounds it, staged through LDS like
// store_tile's bf16 path, and each 16-byte chunk (8 values of one row) is
// combined with the same chunk of X as k_ns_combine does it -- 1.5 x and 0.5 b
// each rounded to bf16, their difference rounded to bf16 -- and stored to C
// (which may be X itself when X is not an operand of the product: each chunk
// is read before it is written, by the same lane).
__device__ __forceinline__ uint32_t ns_combine2(uint32_t xw, uint32_t bw) {
  const float x0 = u2f(xw << 16), x1 = u2f(xw & 0xFFFF0000u);
  const float b0 = u2f(bw << 16), b1 = u2f(bw & 0xFFFF0000u);
  const uint32_t xr = pack_bf16x2(1.5f * x0, 1.5f * x1);
  const uint32_t br = pack_bf16x2(0.5f * b0, 0.5f * b1);
  return pack_bf16x2(u2f(xr << 16) - u2f(br << 16), u2f(xr & 0xFFFF0000u) - u2f(br & 0xFFFF0000u));
}

__device__ __forceinline__ void store_tile_ns(const v16f (&acc)[2][4], uint8_t* stage, int wave, int lane,
                                              void* C, int64_t ldc, const uint16_t* X, int64_t ldx, int row0,
                                              int col0, int M, int N) {
  const int l32 = lane & 31, lhi = lane >> 5;
  constexpr int ROWB = 256;                 // 128 bf16 columns
  constexpr int PITCH = ROWB + 16;
  constexpr int CHUNKS = ROWB / 16;
  constexpr int RP = 32;
  uint8_t* stg = stage + wave * (RP * PITCH);
  __syncthreads();                          // every wave is done with the stage buffer
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    // this pass's chunks of X first (8 per lane), so that their latency
    // overlaps the staging
    v4i xv[(RP * CHUNKS) / 64];
    const uint16_t* Xb = X + (int64_t)(row0 + mi * 32) * ldx + col0;
#pragma unroll
    for (int it = 0; it < (RP * CHUNKS) / 64; ++it) {
      const int q = it * 64 + lane;
      const int r = q / CHUNKS, c = q % CHUNKS;
      xv[it] = v4i{0, 0, 0, 0};
      if (row0 + mi * 32 + r < M && col0 + c * 8 < N)
        xv[it] = *reinterpret_cast<const v4i*>(Xb + (int64_t)r * ldx + c * 8);
    }
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = ni * 32 + 8 * j + 4 * lhi;
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        const bf16x2 p0 = {(__bf16)acc[mi][ni][4 * j + 0], (__bf16)acc[mi][ni][4 * j + 1]};
        const bf16x2 p1 = {(__bf16)acc[mi][ni][4 * j + 2], (__bf16)acc[mi][ni][4 * j + 3]};
        *reinterpret_cast<uint2*>(stg + l32 * PITCH + col * 2) =
            make_uint2(__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1));
      }
    __builtin_amdgcn_s_waitcnt(0xC07F);     // lgkmcnt(0): this wave's staging writes are done
    uint8_t* Cb = static_cast<uint8_t*>(C) + ((int64_t)(row0 + mi * 32) * ldc + col0) * 2;
#pragma unroll
    for (int it = 0; it < (RP * CHUNKS) / 64; ++it) {
      const int q = it * 64 + lane;
      const int r = q / CHUNKS, c = q % CHUNKS;
      const v4i b = *reinterpret_cast<const v4i*>(stg + r * PITCH + c * 16);
      const v4i o = {(int)ns_combine2((uint32_t)xv[it].x, (uint32_t)b.x), (int)ns_combine2((uint32_t)xv[it].y, (uint32_t)b.y),
                     (int)ns_combine2((uint32_t)xv[it].z, (uint32_t)b.z), (int)ns_combine2((uint32_t)xv[it].w, (uint32_t)b.w)};
      if (row0 + mi * 32 + r < M && col0 + c * 8 < N)
        __builtin_nontemporal_store(o, reinterpret_cast<v4i*>(Cb + (int64_t)r * ldc * 2 + c * 16));
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);     // staging reads done before the next pass overwrites
  }
}

template <bool OUT_BF16, int BG, int FQ, bool BF = false, int KM = 0, bool QA = false>
__global__ __launch_bounds__(NTHREADS, 1) void k_gemm_bs_nt(
    const uint8_t* __restrict__ A, int64_t lda, const uint8_t* __restrict__ B, int64_t ldb,
    Scales sa, Scales sb, void* __restrict__ C, int64_t ldc, int K, int span, int tiles_m,
    int tiles_n, uint32_t a_bytes, uint32_t b_bytes, uint32_t ea_bytes, uint32_t eb_bytes,
    uint32_t ga_bytes, uint32_t gb_bytes, int M, int N, FqArgs fq,
    std::conditional_t<QA, QaArgs, QaNone> qa) {
  static_assert(!QA || (!BF && KM == 0 && FQ <= 2), "the quantize prologue feeds an FP8 A operand");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES + ((FQ == 1 || FQ == 2) ? FQ_TABLE_BYTES : 0) +
                                                         (FQ == 5 ? 64 : 0)];
  const OperandRsrc ra = make_rsrc(A, a_bytes, sa, ea_bytes, ga_bytes);
  const OperandRsrc rb = make_rsrc(B, b_bytes, sb, eb_bytes, gb_bytes);

  const int lane = threadIdx.x & 63;
  // wave index, made provably wave-uniform (LDS DMA targets go through M0)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // waves w, w+4 share SIMD w
  const int grp = wave >> 2;              // ping-pong group
  const int wm = wave & 3, wn = grp;      // 64-row band wm, 128-column half wn
  int nk = K / BK;                        // K steps of the current unit
  const int T = tiles_m * tiles_n;
  // the Gram product (upper-triangle tiles by stream-K, FQ 4); operands
  // given K-major (KM bit 0: A, bit 1: B; read through the LDS transposing
  // loads) or K-contiguous
  constexpr bool GRAM = FQ == 4;
  constexpr bool TN_A = (KM & 1) != 0, TN_B = (KM & 2) != 0;
  static_assert(!GRAM || BF, "the Gram product is a bf16 product");
  const bool kmaj = (wave >> 2) == 0 ? TN_A : TN_B;   // K-major layout of this wave's stage loads
  const int l32 = lane & 31, lhi = lane >> 5;

  // this wave's half of every stage load: A rows (group 0) or B rows (group 1)
  const int w4 = wave & 3;
  const Scales& so = grp == 0 ? sa : sb;
  DmaHalf h;
  {
    const OperandRsrc& ro = grp == 0 ? ra : rb;
    h.pay = ro.pay;
    h.e8 = ro.e8;
    h.g32 = ro.g32;
    h.ld = (uint32_t)(grp == 0 ? lda : ldb);
    h.s_k = (uint32_t)so.s_k;
    h.kg = (uint32_t)so.kg;
    if (kmaj) dma_offsets_tn<BF>(grp == 0 ? lda : ldb, lane, h.off);
    else dma_offsets(grp == 0 ? lda : ldb, lane, h.off);
    h.krow0 = (uint32_t)(w4 * (BF ? 16 : 32));   // the wave's K rows of a K-major stage
    h.lds_pay = (grp == 0 ? 0 : OFF_B) + w4 * 8 * 1024;
    h.lds_e = (grp == 0 ? OFF_EA : OFF_EB) + w4 * 256;
    h.lds_r = grp == 0 ? OFF_RA : OFF_RB;
    h.lds_u = grp == 0 ? OFF_UA : OFF_UB;
    if (grp == 0) {
      h.pub = (w4 * 64 + l32 * 2 + lhi) * 4;              // A row w4*64 + lane: band w4, mi = lhi
    } else {
      // B row r: wn = r / 128, ni = c / 32, lhi = (q >> 2) & 1, j = q >> 3, i = q & 3
      const int r = w4 * 64 + lane, c = r & 127, q = c & 31;
      const int e4 = (r >> 7) * 32 + ((c >> 5) * 2 + ((q >> 2) & 1)) * 4 + (q >> 3);
      h.pub = (BG == 2 ? e4 * 4 + (q & 3) : e4) * 4;
    }
  }
  auto rows_of = [&](int tm_, int tn_, int kb_) {
    DmaRows r;
    // K-major: the tile's first operand row (the wave loads K rows of all
    // 256); the e8m0 words and group maxima stay the wave's 64 operand rows
    const int rb0 = grp == 0 ? tile_base(tm_, M) : tile_base(tn_, N);
    r.row0 = (uint32_t)(rb0 + (kmaj ? 0 : w4 * 64));
    r.e_word = (uint32_t)blk_index(so, (int64_t)rb0 + w4 * 64 + lane, 0);
    r.kb = kb_;
    return r;
  };
  // K block of a unit's first step: 0 except for the segments of a Gram range
  auto kb_of = [&](const DmaRows& r) { return GRAM ? r.kb : 0; };
  auto stage_rows = [&](const DmaRows& r, uint8_t* st, int kt, int i) {
    if (kmaj) dma_rows_tn<BF>(h, r, st, kt, i);
    else dma_rows(h, r, st, kt, i);
  };
  const uint32_t skA = (uint32_t)sa.s_k, skB = (uint32_t)sb.s_k;
  // physical 16-byte chunk offsets of this lane's operand halves: K half ks,
  // lo/hi chunk (logical 4*ks + 2*lhi + h, XOR-swizzled by the lane's row)
  int ch[2][2];
  {
    const int sw = swz(l32);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) ch[ks][hh] = ((ks * 4 + lhi * 2 + hh) ^ sw) << 4;
  }
  // TN fragment reads (read_frag_tn): in 16-lane group g, lane j reads K row
  // 16 (g / 2) + j / 4 at operand row 16 (g % 2) + 4 (j % 4) of a 32-row
  // block; tn_kc is that K row's byte offset plus the row's chunk (c = 2 (g %
  // 2) + (j % 4) / 2 inside the block's 4 chunks) and byte ((j % 2) 8)
  // offsets, tn_s the row's swizzle (k mod 4 = j / 4)
  // (fp8: lane j reads K row 32 (g / 2) + j / 2 at operand row 16 (g % 2) +
  // 8 (j % 2), swizzle k mod 8 = j / 2)
  int tn_kc = 0, tn_s = 0;
  if constexpr (TN_A || TN_B) {
    const int g16 = lane >> 4, j16 = lane & 15;
    if constexpr (BF) {
      tn_kc = (16 * (g16 >> 1) + (j16 >> 2)) * 512 + (2 * (g16 & 1) + ((j16 & 3) >> 1)) * 16 + (j16 & 1) * 8;
      tn_s = j16 >> 2;
    } else {
      tn_kc = (32 * (g16 >> 1) + (j16 >> 1)) * 256 + (g16 & 1) * 16 + (j16 & 1) * 8;
      tn_s = j16 >> 1;
    }
  }

  // Persistent: workgroup b computes tiles b, b + G, b + 2G, ... (G = grid
  // size, a multiple of the 8 XCDs, so every tile of a workgroup falls in the
  // L2 band of its XCD).  The stage pipeline runs on across tile boundaries:
  // the next tile's first stage is loaded during the current tile's last K
  // steps into the stage buffer they no longer read, and its latency is
  // covered by the epilogue, which stages the output in the other buffer.
  //
  // Gram (FQ 4): the units are the segments of this workgroup's range of
  // the stream-K step sequence (see FqArgs): a unit is the part of one tile's
  // K steps inside the range, at most two per range.
  int t = blockIdx.x;
  int tm, tn, kb = 0;
  int64_t g = 0, g_end = 0;               // Gram: the range's next and end steps
  auto next_tile = [&](int t_, int* tm_, int* tn_) {
    if constexpr (FQ == 1 || FQ == 2) tile_of_fq(t_, tiles_m, tiles_n, fq.xcd != 0, tm_, tn_);
    else tile_of(t_, tiles_m, tiles_n, tm_, tn_);
  };
  // Gram unit starting at step g_: tile q_, its K blocks [kb_, kb_ + nk_)
  auto gram_unit = [&](int64_t g_, int* q_, int* tm_, int* tn_, int* kb_, int* nk_) {
    const int64_t qq = g_ / fq.steps;
    const int k0 = (int)(g_ - qq * fq.steps);
    const int64_t left = g_end - g_;
    *nk_ = (int)((int64_t)(fq.steps - k0) < left ? (int64_t)(fq.steps - k0) : left);
    *kb_ = k0;
    *q_ = (int)qq;
    tri_of((int)qq, fq.tri, fq.order16 != 0, tm_, tn_);
  };
  if constexpr (GRAM) {
    g = (int64_t)blockIdx.x * fq.iters / gridDim.x;
    g_end = ((int64_t)blockIdx.x + 1) * fq.iters / gridDim.x;
    gram_unit(g, &t, &tm, &tn, &kb, &nk);
  } else {
    next_tile(t, &tm, &tn);
  }

  // quantize prologue: A is written and complete on every XCD before any
  // tile loads it
  if constexpr (QA) qa_prologue(qa.x, qa.q, qa.sc8, qa.sc32, qa.done, qa.ldx, M, K, wave, lane);
  DmaRows cur = rows_of(tm, tn, kb);
  int par = 0;                            // stage buffer of the unit's first K block

  // prologue: both halves of stage 0; group 1 then starts its half of stage 1
  // (it is one stage ahead of group 0 throughout).  The wave's last stage
  // DMA, not yet published: g_pub (a span start), its group max g_ld, its
  // buffer g_st, g_first (a tile's K block 0).
#pragma unroll
  for (int i = 0; i < 8; ++i) stage_rows(cur, lds, kb_of(cur), i);
  float g_ld = 0.0f, u_prev = 1.0f;
  if constexpr (!BF) {
    dma_scales(h, cur, lds, 0);
    g_ld = load_g(h, cur, 0);
  }
  uint8_t* g_st = lds;
  bool g_first = true, g_pub = true;
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (!BF) publish_g(h, lds, g_st, g_ld, g_first, u_prev);
  __syncthreads();

  for (;;) {
    const int m0 = tile_base(tm, M), n0 = tile_base(tn, N);
    int t_next = t + (int)gridDim.x, kb2 = 0, nk2 = nk;
    bool has_next;
    if constexpr (GRAM) has_next = g + nk < g_end;
    else has_next = t_next < T;
    int tm2 = 0, tn2 = 0;
    DmaRows nxt = cur;
    if (has_next) {
      if constexpr (GRAM) gram_unit(g + nk, &t_next, &tm2, &tn2, &kb2, &nk2);
      else next_tile(t_next, &tm2, &tn2);
      nxt = rows_of(tm2, tn2, kb2);
    }
    if (grp == 1) {
      if (1 < nk) {
        uint8_t* s1 = lds + ((1 + par) & 1) * STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < 8; ++i) stage_rows(cur, s1, 1 + kb_of(cur), i);
        if constexpr (!BF) {
          dma_scales(h, cur, s1, 1);
          g_pub = span == 1;
          if (g_pub) g_ld = load_g(h, cur, 1);
        }
        g_st = s1;
        g_first = false;
      }
      wg_barrier();                  // offset group 1 by one phase
    }
    // e8m0 byte position inside the DMA'd word of each compute row at kb = 0,
    // 2 bits per row: A rows i = 0, 1 in bits 2i, B rows i = 0..3 in bits 4 + 2i
    uint32_t epos = 0;
    if constexpr (!BF) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
        epos |= ((uint32_t)blk_index(sa, m0 + wm * 64 + i * 32 + l32, 0) & 3u) << (2 * i);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        epos |= ((uint32_t)blk_index(sb, n0 + wn * 128 + i * 32 + l32, 0) & 3u) << (4 + 2 * i);
    }

    v16f acc[2][4];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = v16f{0};

    uint32_t eA = 0, eB = 0;
    for (int kt = 0; kt < nk; ++kt) {
      const uint8_t* st = lds + ((kt + par) & 1) * STAGE_BYTES;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        // ---- memory phase ----
        if (ks == 0 && !BF) {
          // group 0 publishes its half of stage kt here (it landed at the end
          // of the previous phase); its own waves read only their own rows'
          // ratios, group 1 reads them one phase later
          if (grp == 0 && kt > 0 && g_pub) publish_g(h, lds, g_st, g_ld, g_first, u_prev);
          // e8m0 bytes of this K block for the lane's 2 A rows / 4 B rows
          eA = 0;
          eB = 0;
          const uint8_t* ea = st + OFF_EA + (wm * 64 + l32) * 4;
          const uint8_t* eb = st + OFF_EB + (wn * 128 + l32) * 4;
          const uint32_t tA = (uint32_t)kt * skA, tB = (uint32_t)kt * skB;
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const uint32_t w = lds_u32(ea + i * 128);
            const uint32_t pos = (__builtin_amdgcn_ubfe(epos, 2 * i, 2) + tA) & 3u;
            eA |= __builtin_amdgcn_ubfe(w, pos * 8u, 8) << (8 * i);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t w = lds_u32(eb + i * 128);
            const uint32_t pos = (__builtin_amdgcn_ubfe(epos, 4 + 2 * i, 2) + tB) & 3u;
            eB |= __builtin_amdgcn_ubfe(w, pos * 8u, 8) << (8 * i);
          }
          if (kt > 0 && kt % span == 0) {
            // a new span of group maxima: move the accumulator into its units
            scale_by_units<BG>(acc, st + OFF_RA, st + OFF_RB, wm, wn, lane);
          }
        }
        // rows of this lane: A wm*64 + i*32 + l32, B wn*128 + i*32 + l32; the
        // swizzle of a row depends only on l32, so row blocks i are immediates
        const uint8_t* alo = st + (wm * 64 + l32) * BK + ch[ks][0];
        const uint8_t* ahi = st + (wm * 64 + l32) * BK + ch[ks][1];
        const uint8_t* blo = st + (wn * 128 + l32) * BK + ch[ks][0];
        const uint8_t* bhi = st + (wn * 128 + l32) * BK + ch[ks][1];
        v8i fa[2], fb[4];
        // K-major operands: the lane's 32-row block R (A: 2 wm + mi, B: 4 wn
        // + ni) at K rows tn_kc (+ the K half ks), operand rows from chunk
        // (4 R + c) ^ (4 tn_s) (bf16) or (2 R + c) ^ (2 tn_s) (fp8)
        const uint8_t* kb0 = st + tn_kc + ks * (BF ? 32 * 512 : 64 * 256);
        auto rb = [&](int R) { return kb0 + ((R ^ tn_s) << (BF ? 6 : 5)); };
        auto frag_tn = [&](const uint8_t* base, auto off) {
          if constexpr (BF) return read_frag_tn<decltype(off)::value>(base);
          else return read_frag_tn8<decltype(off)::value>(base);
        };
        using Z = std::integral_constant<int, 0>;
        using OB = std::integral_constant<int, OFF_B>;
        if constexpr (TN_A) {
          fa[0] = frag_tn(rb(2 * wm), Z{});
          fa[1] = frag_tn(rb(2 * wm + 1), Z{});
        } else {
          fa[0] = read_frag2<0>(alo, ahi);
          fa[1] = read_frag2<32 * BK>(alo, ahi);
        }
        if constexpr (TN_B) {
          fb[0] = frag_tn(rb(4 * wn), OB{});
          fb[1] = frag_tn(rb(4 * wn + 1), OB{});
          fb[2] = frag_tn(rb(4 * wn + 2), OB{});
          fb[3] = frag_tn(rb(4 * wn + 3), OB{});
        } else {
          fb[0] = read_frag2<OFF_B>(blo, bhi);
          fb[1] = read_frag2<OFF_B + 32 * BK>(blo, bhi);
          fb[2] = read_frag2<OFF_B + 64 * BK>(blo, bhi);
          fb[3] = read_frag2<OFF_B + 96 * BK>(blo, bhi);
        }
        if (grp == 1 && ks == 1 && kt + 1 < nk) {
          PINNED_WAITCNT(0);        // also group 1's half of stage kt+1 landed
          if (!BF && g_pub) publish_g(h, lds, g_st, g_ld, g_first, u_prev);
        }
        PINNED_WAITCNT(0xC07F);     // lgkmcnt(0): operands in registers, stage reads (and writes) done
        wg_barrier();
        // ---- compute phase ----
        // Group 0 loads its half of stage kt+1 during its first K half, group 1
        // its half of stage kt+2 during its second (both stages are free: every
        // wave finished reading them before the preceding barrier).  Past the
        // tile's last stage the load is the next tile's stage 0; group 1 skips
        // the next tile's stage 1, whose buffer the epilogue stages in.
        bool dma_now;
        int dkt;                       // stage index counted from this tile's K block 0
        if (grp == 0) {
          dma_now = ks == 0 && (kt + 1 < nk || has_next);
          dkt = kt + 1;
        } else {
          dma_now = ks == 1 && (kt + 2 < nk || (has_next && (kt + 2 == nk || nk == 1)));
          dkt = nk == 1 ? kt + 1 : kt + 2;
        }
        const bool to_next = dkt >= nk;
        const DmaRows& dr = to_next ? nxt : cur;
        const int lkt = to_next ? 0 : dkt;            // K block inside the tile loaded
        uint8_t* dst = lds + ((dkt + par) & 1) * STAGE_BYTES;
        constexpr uint32_t KESZ = BF ? 2u : 1u, KROWS = BK / KESZ, KRPI = 1024 / (256 * KESZ);
        const uint32_t soff0 = kmaj ? dr.row0 * KESZ + ((uint32_t)(lkt + kb_of(dr)) * KROWS + h.krow0) * h.ld
                                    : dr.row0 * h.ld + (uint32_t)(lkt + kb_of(dr)) * BK;
        const uint32_t drows = kmaj ? KRPI : 8u;
        uint8_t* const lds0 = dst + h.lds_pay;
        pin_frags(fa, fb);
        mfma_pinned<0, 0, BF>(acc, fa, fb, eA, eB);
        if (dma_now) { dma_rows_at(h, soff0, lds0, 0, drows); dma_rows_at(h, soff0, lds0, 1, drows); }
        mfma_pinned<0, 1, BF>(acc, fa, fb, eA, eB);
        if (dma_now) { dma_rows_at(h, soff0, lds0, 2, drows); dma_rows_at(h, soff0, lds0, 3, drows); }
        mfma_pinned<0, 2, BF>(acc, fa, fb, eA, eB);
        if (dma_now) { dma_rows_at(h, soff0, lds0, 4, drows); dma_rows_at(h, soff0, lds0, 5, drows); }
        mfma_pinned<0, 3, BF>(acc, fa, fb, eA, eB);
        if (dma_now) { dma_rows_at(h, soff0, lds0, 6, drows); dma_rows_at(h, soff0, lds0, 7, drows); }
        mfma_pinned<1, 0, BF>(acc, fa, fb, eA, eB);
        if (dma_now && !BF) {
          dma_scales(h, dr, dst, lkt);
          g_pub = lkt % span == 0;
          if (g_pub) g_ld = load_g(h, dr, lkt);
          g_st = dst;
          g_first = lkt == 0;
        }
        mfma_pinned<1, 1, BF>(acc, fa, fb, eA, eB);
        mfma_pinned<1, 2, BF>(acc, fa, fb, eA, eB);
        mfma_pinned<1, 3, BF>(acc, fa, fb, eA, eB);
        pin_acc(acc);
        if (grp == 0 && ks == 1 && kt + 1 < nk) PINNED_WAITCNT(0);   // group 0's half of stage kt+1 landed
        wg_barrier();
      }
    }
    if (grp == 0) wg_barrier();      // match group 1's extra barrier

    // units of the last span; the last stage's buffer holds no pending load:
    // stage the output there
    float gA[2], gB[4][BG == 1 ? 4 : 1];
    if constexpr (BF) {
      // no scales: gA * gB / 2^14 = 1
#pragma unroll
      for (int i = 0; i < 2; ++i) gA[i] = 128.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < (BG == 1 ? 4 : 1); ++j) gB[i][j] = 128.0f;
    } else if constexpr (BG == 2) {
      // A units here, per-row B units where the store applies them
      const v2f va = *reinterpret_cast<const v2f*>(lds + OFF_UA + (wm * 64 + l32 * 2) * 4);
      gA[0] = va.x;
      gA[1] = va.y;
      gB[0][0] = gB[1][0] = gB[2][0] = gB[3][0] = 1.0f;
    } else {
      load_units<BG>(lds + OFF_UA, lds + OFF_UB, wm, wn, lane, gA, gB);
    }
    // the next tile's stage 0 and group maxima (loaded during the last K steps)
    // land before the epilogue issues its stores, so that the tile end waits
    // for LDS work only
    __builtin_amdgcn_s_waitcnt(0x0F70);      // vmcnt(0)
    asm volatile("" ::"v"(g_ld));
    if constexpr (GRAM) {
      static_assert(BF && OUT_BF16, "the Gram product is a bf16 product");
      if (kb != 0) {
        // the rest of a tile whose head is an earlier range's
        gram_put_partial(acc, fq, (int)blockIdx.x, wave, lane);
      } else {
        gram_add_partials(acc, fq, (int)blockIdx.x, (int)gridDim.x, t, wave, lane);
        store_tile_gram(acc, lds + ((nk - 1 + par) & 1) * STAGE_BYTES, wave, lane, C, ldc, m0 + wm * 64,
                        n0 + wn * 128, tm != tn);
      }
    } else if constexpr (FQ == 3) {
      static_assert(BF && OUT_BF16, "the Newton-Schulz epilogue combines bf16 products");
      store_tile_ns(acc, lds + ((nk - 1 + par) & 1) * STAGE_BYTES, wave, lane, C, ldc, fq.ns_x, fq.ldx,
                    m0 + wm * 64, n0 + wn * 128, M, N);
    } else if constexpr (FQ == 1 || FQ == 2) {
      static_assert(BG == 0, "output requantization takes B scale groups of 32 rows or more");
      uint8_t* table = lds + LDS_BYTES + wave * 64 * 16;
      fq_row_scales<FQ == 2>(acc, gA, gB, fq, table, tm * (tiles_n >> 2) + (tn >> 2), tn, wm, wn, lane,
                             m0 + wm * 64, n0 + wn * 128, M, N);
      store_tile_fq<OUT_BF16>(acc, lds + ((nk - 1 + par) & 1) * STAGE_BYTES, table, wave, lane, C, ldc,
                              m0 + wm * 64, n0 + wn * 128, M);
    } else if constexpr (FQ == 5) {
      static_assert(!OUT_BF16 && !BF, "block maxima of an f32 FP8 product");
      const uint32_t lm = store_tile<false, BG, true>(acc, gA, gB, lds + OFF_UB + (wn * 128 + lhi * 16) * 4,
                                                      lds + ((nk - 1 + par) & 1) * STAGE_BYTES, wave, lane, C, ldc,
                                                      m0 + wm * 64, n0 + wn * 128, M, N);
      store_block_max(lm, reinterpret_cast<uint32_t*>(lds + LDS_BYTES), fq, wave, lane, m0 + wm * 64, n0 + wn * 128,
                      M, N);
    } else if constexpr (FQ == 6) {
      static_assert(!BF, "the (1, 1) requantization of an FP8 product");
      store_tile_q11<OUT_BF16, BG>(acc, gA, gB, lds + OFF_UB + (wn * 128 + lhi * 16) * 4,
                                   lds + ((nk - 1 + par) & 1) * STAGE_BYTES, wave, lane, C, ldc, fq.sc8, fq.sc32,
                                   m0 + wm * 64, n0 + wn * 128, M, N);
    } else {
      store_tile<OUT_BF16, BG>(acc, gA, gB, lds + OFF_UB + (wn * 128 + lhi * 16) * 4, lds + ((nk - 1 + par) & 1) * STAGE_BYTES, wave, lane, C, ldc,
                                   m0 + wm * 64, n0 + wn * 128, M, N);
    }
    if (!has_next) break;
    t = t_next;
    tm = tm2;
    tn = tn2;
    cur = nxt;
    par = (par + nk) & 1;
    if constexpr (GRAM) {
      g += nk;
      kb = kb2;
      nk = nk2;
    }
    // every wave is done with the staging buffer (its LDS reads); the next
    // tile's stage 0 landed before the epilogue, and the output stores are not
    // waited for: they drain while the next tile starts
    PINNED_WAITCNT(0xC07F);
    if constexpr (!BF) publish_g(h, lds, g_st, g_ld, g_first, u_prev);
    PINNED_WAITCNT(0xC07F);
    wg_barrier();
  }
}

// Measurement aid (no counterpart in the reference): the sustained rate of
// the GEMM's own MFMA sequence on given operand bytes, with no memory traffic,
// LDS or barriers in the loop -- the ceiling a GEMM on these operands can
// approach on this part.  Each wave loads two sets of the fragments the GEMM's
// wave would read (its 64 A rows and 128 B rows of the first 256, 32 bytes of
// K per lane, two 64-byte K slices), then issues mfma_all on them
// alternately, `iters` times each; both waves of every SIMD issue, so the
// MFMA pipes never wait on an operand.  The e8m0 bytes are 2^-7 and 2^-8 (as
// in real data, the scale does not change the work).
template <bool BF>
__global__ __launch_bounds__(NTHREADS, 1) void k_mfma_ceiling(const uint8_t* __restrict__ A,
                                                             const uint8_t* __restrict__ B, int64_t ld,
                                                             int iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l32 = lane & 31, lhi = lane >> 5;
  v8i fa[2][2], fb[2][4];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
      fa[s][mi] = *reinterpret_cast<const v8i*>(A + (int64_t)((wave & 3) * 64 + mi * 32 + l32) * ld + s * 64 + lhi * 32);
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
      fb[s][ni] = *reinterpret_cast<const v8i*>(B + (int64_t)((wave >> 2) * 128 + ni * 32 + l32) * ld + s * 64 + lhi * 32);
  }
  v16f acc[2][4];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = v16f{0};
  const uint32_t eA = 0x78787878u, eB = 0x77777777u;
  for (int it = 0; it < iters; ++it) {
    pin_frags(fa[0], fb[0]);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      mfma_tile<0, 0, BF>(acc, fa[s], fb[s], eA, eB);
      mfma_tile<0, 1, BF>(acc, fa[s], fb[s], eA, eB);
      mfma_tile<0, 2, BF>(acc, fa[s], fb[s], eA, eB);
      mfma_tile<0, 3, BF>(acc, fa[s], fb[s], eA, eB);
      mfma_tile<1, 0, BF>(acc, fa[s], fb[s], eA, eB);
      mfma_tile<1, 1, BF>(acc, fa[s], fb[s], eA, eB);
      mfma_tile<1, 2, BF>(acc, fa[s], fb[s], eA, eB);
      mfma_tile<1, 3, BF>(acc, fa[s], fb[s], eA, eB);
    }
  }
  float sum = 0.0f;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int v = 0; v < 16; ++v) sum += acc[mi][ni][v];
  if (sum == 1.2345e-38f) out[0] = sum;    // keeps the loop; never true for these operands in practice
}

// Compute units of the current device (cached per device), rounded down to a
// multiple of 8 so that a persistent workgroup's tiles stay on one XCD's band.
int64_t gemm_num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 8) v = 256;
    cached[dev] = v - v % 8;
  }
  return cached[dev];
}

// Span of an operand's scale layout: the largest P such that every row's
// group index (block / kg) is constant over each aligned run [jP, jP + P) of
// 128-wide K blocks, i.e. the gcd of all K-block positions at which some row's
// group changes (nk if none does).  The kernel reloads group maxima and
// rescales its accumulator at multiples of the span; P = 1 is always valid.
// Row blocks whose base index has the same residue mod kg change groups at the
// same positions, so only one period of residues is walked.
int64_t group_span(const Scales& s, int64_t rows, int64_t nk) {
  if (nk <= 1 || s.s_k == 0) return nk < 1 ? 1 : nk;
  const int64_t nrb = (rows + s.r_div - 1) / s.r_div;
  const int64_t period = s.kg / std::gcd(s.s_r, s.kg);
  const int64_t n_res = nrb < period ? nrb : period;
  int64_t P = 0;
  for (int64_t rb = 0; rb < n_res && P != 1; ++rb) {
    const int64_t r = (rb * s.s_r) % s.kg;
    for (int64_t j = 1; P != 1; ++j) {
      const int64_t kb = (j * s.kg - r + s.s_k - 1) / s.s_k;   // first kb reaching group boundary j
      if (kb >= nk) break;
      P = std::gcd(P, kb);
    }
  }
  return P == 0 ? nk : P;
}

}  // namespace

extern "C" int64_t pratchya_gemm_span(int64_t rows, int64_t K, int64_t r_div, int64_t s_r,
                                      int64_t s_k, int64_t kg) {
  if (K % BK || r_div < 1 || kg < 1 || s_r < 0 || s_k < 0 || rows < 1) return 0;
  Scales s{nullptr, nullptr, r_div, s_r, s_k, kg};
  return group_span(s, rows, K / BK);
}

namespace {

// Validated launch parameters of one GEMM call.
struct GemmPlan {
  Scales sa, sb;
  int64_t span, tiles_m, tiles_n, grid;
  int64_t a_bytes, b_bytes, ea_bytes, eb_bytes, ga_bytes, gb_bytes;
  int bg;              // B group maxima per 32 rows (0), 4 rows (1) or row (2)
};

int gemm_plan(const char* who, const uint8_t* A, int64_t lda, const uint8_t* a_sc8, const float* a_sc32,
              int64_t a_rdiv, int64_t a_sr, int64_t a_sk, int64_t a_kg, const uint8_t* B, int64_t ldb,
              const uint8_t* b_sc8, const float* b_sc32, int64_t b_rdiv, int64_t b_sr, int64_t b_sk,
              int64_t b_kg, int64_t M, int64_t N, int64_t K, const void* C, int64_t ldc, int c_dtype,
              GemmPlan* P) {
  if (K % BK)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: K must be a multiple of 128 (got %lld)", who,
                              (long long)K);
  // outputs are stored in 16-byte chunks: a dimension below one tile must end on a chunk
  if (N < BN && N % (c_dtype == PRATCHYA_DT_BF16 ? 8 : 4))
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: N below 256 must be a multiple of %d (got %lld)", who,
                              c_dtype == PRATCHYA_DT_BF16 ? 8 : 4, (long long)N);
  if (!A || !B || !a_sc8 || !a_sc32 || !b_sc8 || !b_sc32 || !C)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: null buffer", who);
  if (c_dtype != PRATCHYA_DT_F32 && c_dtype != PRATCHYA_DT_BF16)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: unsupported output dtype %d", who, c_dtype);
  if (lda < K || ldb < K || ldc < N || lda % 16 || ldb % 16 || ldc % (c_dtype == PRATCHYA_DT_BF16 ? 8 : 4) ||
      (reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) % 16 ||
      reinterpret_cast<uintptr_t>(C) % 16)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: leading dimensions / alignment not supported", who);
  if (a_rdiv < 1 || b_rdiv < 1 || a_kg < 1 || b_kg < 1 || a_sr < 0 || a_sk < 0 || b_sr < 0 || b_sk < 0)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: bad scale layout", who);
  P->sa = Scales{a_sc8, a_sc32, a_rdiv, a_sr, a_sk, a_kg};
  P->sb = Scales{b_sc8, b_sc32, b_rdiv, b_sr, b_sk, b_kg};
  const int64_t nk = K / BK;
  if ((M / a_rdiv) * a_sr + nk * a_sk > (int64_t)UINT32_MAX ||
      (N / b_rdiv) * b_sr + nk * b_sk > (int64_t)UINT32_MAX)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: scale arrays beyond 2^32 blocks", who);
  // The stage DMA reads each row's e8m0 byte as the aligned 4-byte word that
  // holds it: the e8m0 arrays are read up to the next multiple of 4 bytes
  // (the caller's buffers are readable that far).
  const int64_t last_a = ((M - 1) / a_rdiv) * a_sr + (nk - 1) * a_sk;
  const int64_t last_b = ((N - 1) / b_rdiv) * b_sr + (nk - 1) * b_sk;
  P->ea_bytes = (last_a + 4) & ~(int64_t)3;
  P->eb_bytes = (last_b + 4) & ~(int64_t)3;
  // B's group max per lane: one per 32 output columns where B's block rows
  // are 32 rows or more, one per 4 columns where every 4 consecutive rows
  // (from a multiple of 4, N a multiple of 4) share their groups, else one
  // per column (16 per lane and 32-column tile).
  if (b_rdiv % 32 == 0)
    P->bg = 0;
  else if (N % 4 == 0 && (b_rdiv % 4 == 0 || (b_rdiv == 1 && b_kg % (4 * b_sr) == 0 && b_sk % (4 * b_sr) == 0)))
    P->bg = 1;
  else
    P->bg = 2;
  // span: both operands' group maxima are constant over it
  P->span = std::gcd(group_span(P->sa, M, nk), group_span(P->sb, N, nk));
  // buffer resources address bytes with 32-bit offsets; an operand of fewer
  // than 256 rows is read as 256 (the caller's buffer holds that many)
  const int64_t Ma = M < BM ? BM : M, Na = N < BN ? BN : N;
  P->a_bytes = (Ma - 1) * lda + K;
  P->b_bytes = (Na - 1) * ldb + K;
  P->ga_bytes = (last_a / a_kg + 1) * 4;
  P->gb_bytes = (last_b / b_kg + 1) * 4;
  if (P->a_bytes > (int64_t)INT32_MAX || P->b_bytes > (int64_t)INT32_MAX || last_a + 1 > INT32_MAX ||
      last_b + 1 > INT32_MAX)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: operands beyond 2 GiB", who);
  P->tiles_m = (M + BM - 1) / BM;
  P->tiles_n = (N + BN - 1) / BN;
  if (P->tiles_m * P->tiles_n > INT32_MAX)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: too many output tiles", who);
  // persistent grid: one workgroup per CU (the kernel's LDS allows no more), a
  // multiple of the 8 XCDs
  const int64_t tiles = P->tiles_m * P->tiles_n, cus = gemm_num_cus();
  P->grid = tiles < cus ? tiles : cus;
  return PRATCHYA_OK;
}

template <bool BF, int BG, int FQ, int KM = 0>
void gemm_launch(const GemmPlan& P, const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, void* C,
                 int64_t ldc, int64_t M, int64_t N, int64_t K, const FqArgs& fq, hipStream_t stream) {
  hipLaunchKernelGGL((k_gemm_bs_nt<BF, BG, FQ, false, KM>), dim3((unsigned)P.grid), dim3(NTHREADS), 0, stream, A, lda, B,
                     ldb, P.sa, P.sb, C, ldc, (int)K, (int)P.span, (int)P.tiles_m, (int)P.tiles_n,
                     (uint32_t)P.a_bytes, (uint32_t)P.b_bytes, (uint32_t)P.ea_bytes, (uint32_t)P.eb_bytes,
                     (uint32_t)P.ga_bytes, (uint32_t)P.gb_bytes, (int)M, (int)N, fq, QaNone{});
}

int launch_status(const char* who) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return pratchya_set_error(PRATCHYA_EHIP, "%s: launch failed: %s", who, hipGetErrorString(e));
  return PRATCHYA_OK;
}

// Workspace of the output-requantizing GEMM: per strip (256 rows x 1024
// columns) 256 row maxima and an arrival count, then one status word.
int64_t fq_strips(int64_t M, int64_t N) { return ((M + BM - 1) / BM) * (N / 1024); }
int64_t fq_workspace_words(int64_t M, int64_t N) { return fq_strips(M, N) * 257 + 1; }

}  // namespace

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
  GemmPlan P;
  int rc = gemm_plan("gemm", A, lda, a_sc8, a_sc32, a_rdiv, a_sr, a_sk, a_kg, B, ldb, b_sc8, b_sc32, b_rdiv,
                     b_sr, b_sk, b_kg, M, N, K, C, ldc, c_dtype, &P);
  if (rc) return rc;
  const FqArgs none{};
  const bool bf = c_dtype == PRATCHYA_DT_BF16;
  if (bf) {
    if (P.bg == 0) gemm_launch<true, 0, 0>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
    else if (P.bg == 1) gemm_launch<true, 1, 0>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
    else gemm_launch<true, 2, 0>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
  } else {
    if (P.bg == 0) gemm_launch<false, 0, 0>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
    else if (P.bg == 1) gemm_launch<false, 1, 0>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
    else gemm_launch<false, 2, 0>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
  }
  return launch_status("gemm");
}

extern "C" int pratchya_gemm_bs_nt_q11(const uint8_t* A, int64_t lda, const uint8_t* a_sc8, const float* a_sc32,
                                       int64_t a_rdiv, int64_t a_sr, int64_t a_sk, int64_t a_kg, const uint8_t* B,
                                       int64_t ldb, const uint8_t* b_sc8, const float* b_sc32, int64_t b_rdiv,
                                       int64_t b_sr, int64_t b_sk, int64_t b_kg, int64_t M, int64_t N, int64_t K,
                                       void* C, int64_t ldc, int c_dtype, uint8_t* c_sc8, float* c_sc32,
                                       hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0) {
    if (M < 0 || N < 0 || K < 0) return pratchya_set_error(PRATCHYA_EINVAL, "gemm_q11: negative size");
    return PRATCHYA_OK;
  }
  if (N % 16)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm_q11: N must be a multiple of 16 (got %lld)",
                              (long long)N);
  if (!c_sc8 || !c_sc32 || (reinterpret_cast<uintptr_t>(c_sc8) & 15) || (reinterpret_cast<uintptr_t>(c_sc32) & 15))
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm_q11: the scale arrays must be 16-byte aligned device memory");
  GemmPlan P;
  int rc = gemm_plan("gemm_q11", A, lda, a_sc8, a_sc32, a_rdiv, a_sr, a_sk, a_kg, B, ldb, b_sc8, b_sc32, b_rdiv,
                     b_sr, b_sk, b_kg, M, N, K, C, ldc, c_dtype, &P);
  if (rc) return rc;
  FqArgs fq{};
  fq.sc8 = c_sc8;
  fq.sc32 = c_sc32;
  if (c_dtype == PRATCHYA_DT_BF16) {
    if (P.bg == 0) gemm_launch<true, 0, 6>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
    else if (P.bg == 1) gemm_launch<true, 1, 6>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
    else gemm_launch<true, 2, 6>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
  } else {
    if (P.bg == 0) gemm_launch<false, 0, 6>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
    else if (P.bg == 1) gemm_launch<false, 1, 6>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
    else gemm_launch<false, 2, 6>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
  }
  return launch_status("gemm_q11");
}

extern "C" int pratchya_gemm_bs_kmajor(const uint8_t* A, int64_t lda, const uint8_t* a_sc8, const float* a_sc32,
                                       int64_t a_rdiv, int64_t a_sr, int64_t a_sk, int64_t a_kg, const uint8_t* B,
                                       int64_t ldb, const uint8_t* b_sc8, const float* b_sc32, int64_t b_rdiv,
                                       int64_t b_sr, int64_t b_sk, int64_t b_kg, int64_t M, int64_t N, int64_t K,
                                       void* C, int64_t ldc, int c_dtype, hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0) {
    if (M < 0 || N < 0 || K < 0) return pratchya_set_error(PRATCHYA_EINVAL, "gemm_kmajor: negative size");
    return PRATCHYA_OK;
  }
  GemmPlan P;
  // validated as the plan of the operands' [rows, K] views, then with the
  // operand sizes of the K-major layouts ([K, M] and [K, N], row strides lda,
  // ldb)
  int rc = gemm_plan("gemm_kmajor", A, K, a_sc8, a_sc32, a_rdiv, a_sr, a_sk, a_kg, B, K, b_sc8, b_sc32, b_rdiv,
                     b_sr, b_sk, b_kg, M, N, K, C, ldc, c_dtype, &P);
  if (rc) return rc;
  if (lda < M || ldb < N || lda % 16 || ldb % 16 || M % 16 || N % 16)
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm_kmajor: M, N and the row strides (at least M, N) must be "
                              "multiples of 16");
  P.a_bytes = (K - 1) * lda + M;
  P.b_bytes = (K - 1) * ldb + N;
  if (P.a_bytes > (int64_t)INT32_MAX || P.b_bytes > (int64_t)INT32_MAX)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm_kmajor: operands beyond 2 GiB");
  const FqArgs none{};
  if (c_dtype == PRATCHYA_DT_BF16) {
    if (P.bg == 0) gemm_launch<true, 0, 0, 3>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
    else if (P.bg == 1) gemm_launch<true, 1, 0, 3>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
    else gemm_launch<true, 2, 0, 3>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
  } else {
    if (P.bg == 0) gemm_launch<false, 0, 0, 3>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
    else if (P.bg == 1) gemm_launch<false, 1, 0, 3>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
    else gemm_launch<false, 2, 0, 3>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
  }
  return launch_status("gemm_kmajor");
}

extern "C" int pratchya_gemm_bs_blockmax(const uint8_t* A, int64_t lda, const uint8_t* a_sc8, const float* a_sc32,
                                         int64_t a_rdiv, int64_t a_sr, int64_t a_sk, int64_t a_kg, const uint8_t* B,
                                         int64_t ldb, const uint8_t* b_sc8, const float* b_sc32, int64_t b_rdiv,
                                         int64_t b_sr, int64_t b_sk, int64_t b_kg, int64_t M, int64_t N, int64_t K,
                                         int kmajor, float* C, int64_t ldc, uint32_t* bmax, hipStream_t stream) {
  const char* who = "gemm_blockmax";
  if (M <= 0 || N <= 0 || K <= 0) {
    if (M < 0 || N < 0 || K < 0) return pratchya_set_error(PRATCHYA_EINVAL, "%s: negative size", who);
    return PRATCHYA_OK;
  }
  if (M % 128 || N % 128)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: M and N must be multiples of 128 (got %lld, %lld)", who,
                              (long long)M, (long long)N);
  if (!bmax) return pratchya_set_error(PRATCHYA_EINVAL, "%s: null buffer", who);
  GemmPlan P;
  int rc = gemm_plan(who, A, kmajor ? K : lda, a_sc8, a_sc32, a_rdiv, a_sr, a_sk, a_kg, B, kmajor ? K : ldb, b_sc8,
                     b_sc32, b_rdiv, b_sr, b_sk, b_kg, M, N, K, C, ldc, PRATCHYA_DT_F32, &P);
  if (rc) return rc;
  if (kmajor) {
    if (lda < M || ldb < N || lda % 16 || ldb % 16 || M % 16 || N % 16)
      return pratchya_set_error(PRATCHYA_EINVAL, "%s: M, N and the row strides (at least M, N) must be multiples of 16",
                                who);
    P.a_bytes = (K - 1) * lda + M;
    P.b_bytes = (K - 1) * ldb + N;
    if (P.a_bytes > (int64_t)INT32_MAX || P.b_bytes > (int64_t)INT32_MAX)
      return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: operands beyond 2 GiB", who);
  }
  FqArgs fq{};
  fq.bmax = bmax;
  fq.bmax_ld = (int)(N / 128);
  if (kmajor) {
    if (P.bg == 0) gemm_launch<false, 0, 5, 3>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
    else if (P.bg == 1) gemm_launch<false, 1, 5, 3>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
    else gemm_launch<false, 2, 5, 3>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
  } else {
    if (P.bg == 0) gemm_launch<false, 0, 5>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
    else if (P.bg == 1) gemm_launch<false, 1, 5>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
    else gemm_launch<false, 2, 5>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
  }
  return launch_status(who);
}

extern "C" int64_t pratchya_gemm_bs_nt_fq_workspace_bytes(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0 || N % 1024) return 0;
  return ((fq_workspace_words(M, N) * 4 + 255) / 256) * 256;
}

extern "C" int64_t pratchya_gemm_bs_nt_fq_status_offset(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0 || N % 1024) return -1;
  const int64_t strips = fq_strips(M, N);
  return (strips * 256 + strips) * 4;
}

extern "C" int pratchya_gemm_bs_nt_fq(const uint8_t* A, int64_t lda, const uint8_t* a_sc8,
                                      const float* a_sc32, int64_t a_rdiv, int64_t a_sr, int64_t a_sk,
                                      int64_t a_kg, const uint8_t* B, int64_t ldb, const uint8_t* b_sc8,
                                      const float* b_sc32, int64_t b_rdiv, int64_t b_sr, int64_t b_sk,
                                      int64_t b_kg, int64_t M, int64_t N, int64_t K, void* C, int64_t ldc,
                                      int c_dtype, int fix_nan, uint8_t* c_sc8, float* c_sc32,
                                      void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0) {
    if (M < 0 || N < 0 || K < 0) return pratchya_set_error(PRATCHYA_EINVAL, "gemm_fq: negative size");
    return PRATCHYA_OK;
  }
  if (N % 1024)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm_fq: N must be a multiple of 1024 (one (1, 128) "
                              "group of 8 blocks per row segment; got %lld)", (long long)N);
  GemmPlan P;
  int rc = gemm_plan("gemm_fq", A, lda, a_sc8, a_sc32, a_rdiv, a_sr, a_sk, a_kg, B, ldb, b_sc8, b_sc32, b_rdiv,
                     b_sr, b_sk, b_kg, M, N, K, C, ldc, c_dtype, &P);
  if (rc) return rc;
  if (P.bg != 0)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm_fq: B scale groups narrower than 32 rows");
  if (ldc >= (int64_t)1 << 23)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm_fq: output row stride of 2^23 elements or more");
  if (!c_sc8 || !c_sc32 || !workspace)
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm_fq: null buffer");
  if (workspace_bytes < pratchya_gemm_bs_nt_fq_workspace_bytes(M, N) || reinterpret_cast<uintptr_t>(workspace) % 4)
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm_fq: workspace of %lld bytes (need %lld, 4-byte aligned)",
                              (long long)workspace_bytes, (long long)pratchya_gemm_bs_nt_fq_workspace_bytes(M, N));
  // The four workgroups of a strip work in the same round: XCD-aware partners
  // b, b+8, b+16, b+24 need whole groups of 32 tiles and workgroups, otherwise
  // partners are four consecutive workgroups.
  const int64_t tiles = P.tiles_m * P.tiles_n;
  FqArgs fq{};
  fq.xcd = tiles % 32 == 0 && P.grid >= 32 ? 1 : 0;
  P.grid -= P.grid % (fq.xcd ? 32 : 4);
  uint32_t* ws = static_cast<uint32_t*>(workspace);
  const int64_t strips = fq_strips(M, N);
  fq.sc8 = c_sc8;
  fq.sc32 = c_sc32;
  fq.gmax = ws;
  fq.arrive = ws + strips * 256;
  fq.status = fq.arrive + strips;
  // maxima, arrival counts and status start at zero (a kernel, not a memset:
  // safe under graph capture)
  const int64_t words = fq_workspace_words(M, N);
  const int64_t fill_blocks = (words + 255) / 256 < 1024 ? (words + 255) / 256 : 1024;
  hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)fill_blocks), dim3(256), 0, stream, ws, words, 0u);
  rc = launch_status("gemm_fq");
  if (rc) return rc;
  const bool bf = c_dtype == PRATCHYA_DT_BF16;
  if (bf && fix_nan) gemm_launch<true, 0, 2>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
  else if (bf) gemm_launch<true, 0, 1>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
  else if (fix_nan) gemm_launch<false, 0, 2>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
  else gemm_launch<false, 0, 1>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
  return launch_status("gemm_fq");
}

namespace {


template <bool OB, int FQ>
void gemm_launch_qa(const GemmPlan& P, const uint8_t* A, int64_t lda, const uint8_t* B, int64_t ldb, void* C,
                    int64_t ldc, int64_t M, int64_t N, int64_t K, const FqArgs& fq, const QaArgs& qa,
                    hipStream_t stream) {
  hipLaunchKernelGGL((k_gemm_bs_nt<OB, 0, FQ, false, 0, true>), dim3((unsigned)P.grid), dim3(NTHREADS), 0, stream,
                     A, lda, B, ldb, P.sa, P.sb, C, ldc, (int)K, (int)P.span, (int)P.tiles_m, (int)P.tiles_n,
                     (uint32_t)P.a_bytes, (uint32_t)P.b_bytes, (uint32_t)P.ea_bytes, (uint32_t)P.eb_bytes,
                     (uint32_t)P.ga_bytes, (uint32_t)P.gb_bytes, (int)M, (int)N, fq, qa);
}

}  // namespace

// Workspace of the quantize prologue: the count of waves done with it, the
// status word, then the output requantization's maxima and counts (fq).
extern "C" int64_t pratchya_gemm_bs_nt_qa_workspace_bytes(int64_t M, int64_t N, int fq) {
  if (M < BM || N <= 0 || (fq && N % 1024)) return 0;
  const int64_t words = 2 + (fq ? fq_workspace_words(M, N) : 0);
  return ((words * 4 + 255) / 256) * 256;
}

extern "C" int64_t pratchya_gemm_bs_nt_qa_status_offset(int64_t M, int64_t N, int fq) {
  if (M < BM || N <= 0 || (fq && N % 1024)) return -1;
  return 4;
}

extern "C" int pratchya_gemm_bs_nt_qa(const void* X, int64_t ldx, uint8_t* A, uint8_t* a_sc8, float* a_sc32,
                                      const uint8_t* B, int64_t ldb, const uint8_t* b_sc8, const float* b_sc32,
                                      int64_t b_rdiv, int64_t b_sr, int64_t b_sk, int64_t b_kg, int64_t M,
                                      int64_t N, int64_t K, void* C, int64_t ldc, int c_dtype, int fq,
                                      uint8_t* c_sc8, float* c_sc32, void* workspace, int64_t workspace_bytes,
                                      hipStream_t stream) {
  const char* who = "gemm_qa";
  if (M < 0 || N < 0 || K < 0) return pratchya_set_error(PRATCHYA_EINVAL, "%s: negative size", who);
  if (M == 0 || N == 0 || K == 0) return PRATCHYA_OK;
  if (M < BM)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: M must be at least 256 (got %lld)", who, (long long)M);
  if (K % 1024)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: K must be a multiple of 1024 (got %lld)", who,
                              (long long)K);
  if (fq != 0 && fq != 1) return pratchya_set_error(PRATCHYA_EINVAL, "%s: fq must be 0 or 1", who);
  if (fq && N % 1024)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: N must be a multiple of 1024 with the output "
                              "requantization (got %lld)", who, (long long)N);
  if (!X || !A || !a_sc8 || !a_sc32 || !workspace) return pratchya_set_error(PRATCHYA_EINVAL, "%s: null buffer", who);
  if (ldx < K || ldx % 8 || reinterpret_cast<uintptr_t>(X) % 16)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: X must be 16-byte aligned with a row stride of at least K, a "
                              "multiple of 8", who);
  if ((M - 1) * ldx * 2 + 2 * K > (int64_t)INT32_MAX)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: X beyond 2 GiB", who);
  if ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(a_sc8) | reinterpret_cast<uintptr_t>(a_sc32)) %
      256)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: the quantized outputs must be 256-byte aligned", who);
  GemmPlan P;
  int rc = gemm_plan(who, A, K, a_sc8, a_sc32, 1, K / 128, 1, 8, B, ldb, b_sc8, b_sc32, b_rdiv, b_sr, b_sk, b_kg,
                     M, N, K, C, ldc, c_dtype, &P);
  if (rc) return rc;
  if (P.bg != 0) return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: B scale groups narrower than 32 rows", who);
  if (workspace_bytes < pratchya_gemm_bs_nt_qa_workspace_bytes(M, N, fq) ||
      reinterpret_cast<uintptr_t>(workspace) % 4)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: workspace of %lld bytes (need %lld, 4-byte aligned)", who,
                              (long long)workspace_bytes, (long long)pratchya_gemm_bs_nt_qa_workspace_bytes(M, N, fq));
  uint32_t* ws = static_cast<uint32_t*>(workspace);
  FqArgs fqa{};
  if (fq) {
    if (ldc >= (int64_t)1 << 23)
      return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: output row stride of 2^23 elements or more", who);
    if (!c_sc8 || !c_sc32) return pratchya_set_error(PRATCHYA_EINVAL, "%s: null buffer", who);
    const int64_t tiles = P.tiles_m * P.tiles_n;
    fqa.xcd = tiles % 32 == 0 && P.grid >= 32 ? 1 : 0;
    P.grid -= P.grid % (fqa.xcd ? 32 : 4);
    const int64_t strips = fq_strips(M, N);
    fqa.sc8 = c_sc8;
    fqa.sc32 = c_sc32;
    fqa.gmax = ws + 2;
    fqa.arrive = fqa.gmax + strips * 256;
    fqa.status = ws + 1;
  }
  QaArgs qa;
  qa.x = static_cast<const uint8_t*>(X);
  qa.q = A;
  qa.sc8 = a_sc8;
  qa.sc32 = a_sc32;
  qa.done = ws;                        // the status word follows
  qa.ldx = ldx * 2;
  // count, status (and the output requantization's maxima and counts) start
  // at zero: a kernel, not a memset, so the call can be captured
  const int64_t words = 2 + (fq ? fq_workspace_words(M, N) : 0);
  const int64_t fill_blocks = (words + 255) / 256 < 1024 ? (words + 255) / 256 : 1024;
  hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)fill_blocks), dim3(256), 0, stream, ws, words, 0u);
  rc = launch_status(who);
  if (rc) return rc;
  const bool bf = c_dtype == PRATCHYA_DT_BF16;
  if (fq) {
    if (bf) gemm_launch_qa<true, 1>(P, A, K, B, ldb, C, ldc, M, N, K, fqa, qa, stream);
    else gemm_launch_qa<false, 1>(P, A, K, B, ldb, C, ldc, M, N, K, fqa, qa, stream);
  } else {
    if (bf) gemm_launch_qa<true, 0>(P, A, K, B, ldb, C, ldc, M, N, K, fqa, qa, stream);
    else gemm_launch_qa<false, 0>(P, A, K, B, ldb, C, ldc, M, N, K, fqa, qa, stream);
  }
  return launch_status(who);
}

namespace {

// Validated plan of a bf16 product C [M, N] = A [M, K] . B [N, K]^T (returns
// a status; *empty when there is nothing to compute).
int bf16_plan(const char* who, const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N,
              int64_t K, const void* C, int64_t ldc, bool bf, GemmPlan* P, bool* empty) {
  *empty = false;
  if (M <= 0 || N <= 0 || K <= 0) {
    if (M < 0 || N < 0 || K < 0) return pratchya_set_error(PRATCHYA_EINVAL, "%s: negative size", who);
    *empty = true;
    return PRATCHYA_OK;
  }
  if (K % 64)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: K must be a multiple of 64 (got %lld)", who, (long long)K);
  if (N < BN && N % (bf ? 8 : 4))
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: N below 256 must be a multiple of %d (got %lld)", who,
                              bf ? 8 : 4, (long long)N);
  if (!A || !B || !C) return pratchya_set_error(PRATCHYA_EINVAL, "%s: null buffer", who);
  if (lda < K || ldb < K || ldc < N || lda % 8 || ldb % 8 || ldc % (bf ? 8 : 4) ||
      (reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B) | reinterpret_cast<uintptr_t>(C)) % 16)
    return pratchya_set_error(PRATCHYA_EINVAL, "%s: leading dimensions / alignment not supported", who);
  // the kernel addresses the operands as byte matrices: a 128-byte stage row
  // holds 64 bf16 values of K
  *P = GemmPlan{};
  P->sa = Scales{nullptr, nullptr, 1, 0, 0, 1};
  P->sb = P->sa;
  P->span = 1;
  P->bg = 0;
  const int64_t Ma = M < BM ? BM : M, Na = N < BN ? BN : N;
  P->a_bytes = ((Ma - 1) * lda + K) * 2;
  P->b_bytes = ((Na - 1) * ldb + K) * 2;
  if (P->a_bytes > (int64_t)INT32_MAX || P->b_bytes > (int64_t)INT32_MAX)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: operands beyond 2 GiB", who);
  P->tiles_m = (M + BM - 1) / BM;
  P->tiles_n = (N + BN - 1) / BN;
  if (P->tiles_m * P->tiles_n > INT32_MAX)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "%s: too many output tiles", who);
  const int64_t tiles = P->tiles_m * P->tiles_n, cus = gemm_num_cus();
  P->grid = tiles < cus ? tiles : cus;
  return PRATCHYA_OK;
}

template <bool OB, int FQ, int KM = 0>
void bf16_launch(const GemmPlan& P, const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                 int64_t M, int64_t N, int64_t K, const FqArgs& fq, hipStream_t stream) {
  hipLaunchKernelGGL((k_gemm_bs_nt<OB, 0, FQ, true, KM>), dim3((unsigned)P.grid), dim3(NTHREADS), 0, stream,
                     static_cast<const uint8_t*>(A), lda * 2, static_cast<const uint8_t*>(B), ldb * 2, P.sa, P.sb,
                     C, ldc, (int)(K * 2), 1, (int)P.tiles_m, (int)P.tiles_n, (uint32_t)P.a_bytes,
                     (uint32_t)P.b_bytes, 0u, 0u, 0u, 0u, (int)M, (int)N, fq, QaNone{});
}

}  // namespace

extern "C" int pratchya_gemm_bf16_nt(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N,
                                     int64_t K, void* C, int64_t ldc, int c_dtype, hipStream_t stream) {
  const bool bf = c_dtype == PRATCHYA_DT_BF16;
  if (c_dtype != PRATCHYA_DT_F32 && !bf)
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm_bf16: unsupported output dtype %d", c_dtype);
  GemmPlan P;
  bool empty;
  int rc = bf16_plan("gemm_bf16", A, lda, B, ldb, M, N, K, C, ldc, bf, &P, &empty);
  if (rc || empty) return rc;
  const FqArgs none{};
  if (bf) bf16_launch<true, 0>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
  else bf16_launch<false, 0>(P, A, lda, B, ldb, C, ldc, M, N, K, none, stream);
  return launch_status("gemm_bf16");
}

extern "C" int pratchya_gemm_bf16_nt_ns(const void* A, int64_t lda, const void* B, int64_t ldb, int b_kmajor,
                                        int64_t M, int64_t N, int64_t K, const void* X, int64_t ldx, void* C,
                                        int64_t ldc, hipStream_t stream) {
  GemmPlan P;
  bool empty;
  // a K-major B ([K, N], row stride ldb >= N) is validated as the plan of its
  // [N, K] view, with the operand size of its own layout
  int rc = bf16_plan("gemm_bf16_ns", A, lda, B, b_kmajor ? K : ldb, M, N, K, C, ldc, true, &P, &empty);
  if (rc || empty) return rc;
  if (b_kmajor) {
    if (ldb < N || ldb % 8 || N % 8)
      return pratchya_set_error(PRATCHYA_EINVAL, "gemm_bf16_ns: a K-major B needs N and a row stride of at "
                                "least N that are multiples of 8");
    const int64_t bytes = ((K - 1) * ldb + N) * 2;
    if (bytes > (int64_t)INT32_MAX)
      return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm_bf16_ns: operand beyond 2 GiB");
    P.b_bytes = bytes;
  }
  if (!X || ldx < N || ldx % 8 || reinterpret_cast<uintptr_t>(X) % 16)
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm_bf16_ns: X must be a 16-byte aligned [M, N] bf16 matrix "
                              "with a row stride that is a multiple of 8");
  // C must not overlap X: an edge tile recomputes part of its neighbour, which
  // would then combine an already combined value
  const uintptr_t x0 = reinterpret_cast<uintptr_t>(X), x1 = x0 + (uintptr_t)(((M - 1) * ldx + N) * 2);
  const uintptr_t c0 = reinterpret_cast<uintptr_t>(C), c1 = c0 + (uintptr_t)(((M - 1) * ldc + N) * 2);
  if (c0 < x1 && x0 < c1)
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm_bf16_ns: the output overlaps X");
  FqArgs fq{};
  fq.ns_x = static_cast<const uint16_t*>(X);
  fq.ldx = ldx;
  if (b_kmajor) bf16_launch<true, 3, 2>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
  else bf16_launch<true, 3>(P, A, lda, B, ldb, C, ldc, M, N, K, fq, stream);
  return launch_status("gemm_bf16_ns");
}

// --------------------------------------------------------------------------
// Symmetric product C = A A^T (the Gram matrix of Newton-Schulz's first
// product): the kernel computes the upper-triangle tiles by stream-K (see
// FqArgs) and writes each off-diagonal tile also transposed, so C is exactly
// symmetric.
// --------------------------------------------------------------------------
namespace {

// Workgroups of the Gram product: one range per CU, at most two per tile
// (each range then holds at least half a tile's steps, so a tile has at most
// three contributors) and at most one per step.
int64_t gram_grid(int64_t M, int64_t K) {
  const int64_t tri = M / BM, tiles = tri * (tri + 1) / 2, iters = tiles * (K / 64);
  int64_t g = gemm_num_cus();
  if (g > 2 * tiles) g = 2 * tiles;
  if (g > iters) g = iters;
  return g;
}

}  // namespace

extern "C" int64_t pratchya_gemm_bf16_gram_workspace_bytes(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0 || M % BM || K % 64) return 0;
  const int64_t G = gram_grid(M, K);
  return G * 8 * (32 * 256) * 4 + (G * 8 + 1) * 4;
}

extern "C" int64_t pratchya_gemm_bf16_gram_status_offset(int64_t M, int64_t K) {
  if (M <= 0 || K <= 0 || M % BM || K % 64) return -1;
  const int64_t G = gram_grid(M, K);
  return (G * 8 * (32 * 256) + G * 8) * 4;
}

extern "C" int pratchya_gemm_bf16_gram(const void* A, int64_t lda, int64_t M, int64_t K, int a_kmajor, void* C,
                                       int64_t ldc, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  GemmPlan P;
  bool empty;
  // a K-major A ([K, M], row stride lda >= M) is validated as the plan of its
  // [M, K] view with the operand sizes of its own layout
  int rc = bf16_plan("gemm_bf16_gram", A, a_kmajor ? K : lda, A, a_kmajor ? K : lda, M, M, K, C, ldc, true, &P,
                     &empty);
  if (rc || empty) return rc;
  if (a_kmajor) {
    if (lda < M || lda % 8)
      return pratchya_set_error(PRATCHYA_EINVAL, "gemm_bf16_gram: a K-major A needs a row stride of at least M, "
                                "a multiple of 8");
    const int64_t bytes = ((K - 1) * lda + M) * 2;
    if (bytes > (int64_t)INT32_MAX)
      return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm_bf16_gram: operand beyond 2 GiB");
    P.a_bytes = P.b_bytes = bytes;
  }
  if (M % BM)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm_bf16_gram: M must be a multiple of 256 (got %lld)",
                              (long long)M);
  const int64_t need = pratchya_gemm_bf16_gram_workspace_bytes(M, K);
  if (!workspace || workspace_bytes < need || reinterpret_cast<uintptr_t>(workspace) % 16)
    return pratchya_set_error(PRATCHYA_EINVAL, "gemm_bf16_gram: workspace of %lld bytes (need %lld, 16-byte aligned)",
                              (long long)workspace_bytes, (long long)need);
  const int64_t tri = M / BM, tiles = tri * (tri + 1) / 2, G = gram_grid(M, K);
  if (tiles * (K / 64) > INT32_MAX)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "gemm_bf16_gram: too many K steps");
  FqArgs fq{};
  fq.part = static_cast<float*>(workspace);
  fq.flags = reinterpret_cast<uint32_t*>(fq.part + G * 8 * (32 * 256));
  fq.status = fq.flags + G * 8;
  fq.iters = tiles * (K / 64);
  fq.steps = (int)(K / 64);
  fq.tri = (int)tri;
  fq.order16 = tri == 16 && G == 256 && fq.steps % 32 == 0 ? 1 : 0;
  // flags and status start at zero (a kernel, not a memset: safe under graph
  // capture)
  const int64_t words = G * 8 + 1;
  hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream, fq.flags, words, 0u);
  rc = launch_status("gemm_bf16_gram");
  if (rc) return rc;
  P.grid = G;
  if (a_kmajor) bf16_launch<true, 4, 3>(P, A, lda, A, lda, C, ldc, M, M, K, fq, stream);
  else bf16_launch<true, 4>(P, A, lda, A, lda, C, ldc, M, M, K, fq, stream);
  return launch_status("gemm_bf16_gram");
}

// --------------------------------------------------------------------------
// Byte transpose [rows, cols] -> [cols, rows] (fp8 payloads: W [K, N] to the
// K-contiguous [N, K] operand layout, token-major payloads to channel-major).
// 128x128 (64x64 for small matrices) tiles through LDS; 16-byte global loads
// and stores.
// --------------------------------------------------------------------------
namespace {
// TILE x TILE tiles, TILE / 16 lanes per row: each load and store
// instruction of a wave moves whole TILE-byte row pieces (128: 8 whole
// 128-byte lines per instruction; 64 for small matrices, where 128-wide
// tiles would leave CUs idle).
template <int TILE>
__global__ __launch_bounds__(256) void k_transpose_u8(const uint8_t* __restrict__ src, int64_t rows,
                                                      int64_t cols, uint8_t* __restrict__ dst) {
  constexpr int LPR = TILE / 16, RPP = 256 / LPR, PASSES = TILE / RPP;
  __shared__ uint32_t tile[TILE][TILE / 4 + 1];   // TILE rows x TILE bytes (+1 word pad)
  // one-dimensional grid over the tiles (no 65535 limit on either axis);
  // partial tiles at the edges (sizes are multiples of 16) move only whole
  // 16-byte pieces inside the matrix
  const int64_t tiles_c = (cols + TILE - 1) / TILE;
  const int64_t r0 = ((int64_t)blockIdx.x / tiles_c) * TILE, c0 = ((int64_t)blockIdx.x % tiles_c) * TILE;
  const int t = threadIdx.x;
  const int q = t % LPR;
#pragma unroll
  for (int h = 0; h < PASSES; ++h) {
    const int r = h * RPP + t / LPR;   // row r, 16-byte piece q
    const int64_t gr = r0 + r, gc = c0 + q * 16;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (gr < rows && gc + 16 <= cols) v = *reinterpret_cast<const uint4*>(src + gr * cols + gc);
    tile[r][q * 4 + 0] = v.x;
    tile[r][q * 4 + 1] = v.y;
    tile[r][q * 4 + 2] = v.z;
    tile[r][q * 4 + 3] = v.w;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < PASSES; ++h) {
    const int c = h * RPP + t / LPR;   // output row c (= input column), input rows 16 q ..
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t acc = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t word = tile[q * 16 + i * 4 + b][c >> 2];
        acc |= ((word >> (8 * (c & 3))) & 0xFFu) << (8 * b);
      }
      w[i] = acc;
    }
    const int64_t gr = c0 + c, gc = r0 + q * 16;
    if (gr < cols && gc + 16 <= rows)
      *reinterpret_cast<uint4*>(dst + gr * rows + gc) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// 16-bit transpose [rows, cols] -> [cols, rows] (bf16 matrices: the
// K-contiguous layout of X^T for the Newton-Schulz products).  64x64 tiles
// through LDS (rows padded to 33 words: the column gathers hit 32 banks);
// 16-byte global loads and stores of 8 elements.
__global__ __launch_bounds__(256) void k_transpose_u16(const uint16_t* __restrict__ src, int64_t rows,
                                                       int64_t cols, uint16_t* __restrict__ dst) {
  __shared__ uint32_t tile[64][33];   // 64 rows x 64 elements (+1 word pad)
  const int64_t tiles_c = (cols + 63) / 64;
  const int64_t r0 = ((int64_t)blockIdx.x / tiles_c) * 64, c0 = ((int64_t)blockIdx.x % tiles_c) * 64;
  const int t = threadIdx.x;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int i = t + 256 * h, r = i >> 3, q = i & 7;   // row r, 8-element piece q
    const int64_t gr = r0 + r, gc = c0 + q * 8;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (gr < rows && gc + 8 <= cols) v = *reinterpret_cast<const uint4*>(src + gr * cols + gc);
    tile[r][q * 4 + 0] = v.x;
    tile[r][q * 4 + 1] = v.y;
    tile[r][q * 4 + 2] = v.z;
    tile[r][q * 4 + 3] = v.w;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int i = t + 256 * h, c = i >> 3, q = i & 7;   // output row c (= input column), input rows 8q..8q+7
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t lo = tile[q * 8 + 2 * k][c >> 1], hi = tile[q * 8 + 2 * k + 1][c >> 1];
      const int sh = 16 * (c & 1);
      w[k] = ((lo >> sh) & 0xFFFFu) | (((hi >> sh) & 0xFFFFu) << 16);
    }
    const int64_t gr = c0 + c, gc = r0 + q * 8;
    if (gr < cols && gc + 8 <= rows)
      *reinterpret_cast<uint4*>(dst + gr * rows + gc) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}
}  // namespace

extern "C" int pratchya_transpose_b16(const void* src, int64_t rows, int64_t cols, void* dst, hipStream_t stream) {
  if (rows < 0 || cols < 0) return pratchya_set_error(PRATCHYA_EINVAL, "transpose_b16: negative size");
  if (rows == 0 || cols == 0) return PRATCHYA_OK;
  if (!src || !dst) return pratchya_set_error(PRATCHYA_EINVAL, "transpose_b16: null buffer");
  if (rows % 8 || cols % 8 || reinterpret_cast<uintptr_t>(src) % 16 || reinterpret_cast<uintptr_t>(dst) % 16)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED,
                              "transpose_b16: sizes must be multiples of 8, buffers 16-byte aligned");
  const int64_t tiles = ((rows + 63) / 64) * ((cols + 63) / 64);
  if (tiles > INT32_MAX) return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "transpose_b16: more than 2^31 tiles");
  hipLaunchKernelGGL(k_transpose_u16, dim3((unsigned)tiles), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(src), rows, cols, static_cast<uint16_t*>(dst));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return pratchya_set_error(PRATCHYA_EHIP, "transpose_b16: %s", hipGetErrorString(e));
  return PRATCHYA_OK;
}

// --------------------------------------------------------------------------
// f32 operands for the bf16 GEMM: an f32 value v is the exact sum of three
// bf16 pieces p1 = trunc(v), p2 = trunc(v - p1), p3 = v - p1 - p2 (trunc:
// the top 8 significand bits; each difference is exact in f32, the pieces
// share v's sign and never overflow), and a product of two pieces is exact in
// f32.  A non-finite v is its own first piece (the others are 0), and only the
// (0,0) pair may carry it: plane 3 is piece 0 with non-finite values as 0, for
// the pairs (0,j>0) and (i>0,0), where it would meet the other operand's
// lower pieces (inf * 0 would make a NaN the f32 product does not have).  So
// dot(a, b) over f32 vectors equals the sum of the piece products, and the
// six pairs (1,1) (1,2) (2,1) (1,3) (2,2) (3,1) leave out only terms below
// 2^-24 of the largest product: one bf16 GEMM over the pieces placed side by
// side along K computes an f32 product to f32 accuracy (up to summation
// order).  k_split_pack writes those K-contiguous operands: segment s of each
// output row holds piece plane[s] of a source row (or column, transposed),
// zero-padded to kp values.
// --------------------------------------------------------------------------
namespace {
__device__ __forceinline__ float bf16_trunc(float v) { return pfp8::u2f(pfp8::f2u(v) & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_piece(float v, int p) {
  if (!pfp8::is_finite_f(v)) return p == 0 ? v : 0.0f;
  if (p == 3) p = 0;
  const float p1 = bf16_trunc(v);
  if (p == 0) return p1;
  const float r1 = v - p1;
  const float p2 = bf16_trunc(r1);
  if (p == 1) return p2;
  return r1 - p2;                     // at most 8 significant bits: exact in bf16
}

// src: f32 or bf16 [rows, cols] with row stride lds elements.  Not TRANSPOSED:
// output row r, segment s, column k < cols is piece plane[s] of src[r][k];
// TRANSPOSED: output row c, column k < rows is piece plane[s] of src[k][c].
// One 64 x 64 source tile per workgroup through LDS; columns kp > len of a
// segment are zero.  planes: 2 bits per segment (bits 2s, 2s+1).
template <bool SRC_BF16, bool TRANSPOSED>
__global__ __launch_bounds__(256) void k_split_pack(const void* __restrict__ src, int64_t rows, int64_t cols,
                                                    int64_t lds, int nseg, uint32_t planes, uint16_t* __restrict__ dst,
                                                    int64_t ldd, int64_t kp) {
  __shared__ float tile[64][65];
  const int64_t out_rows = TRANSPOSED ? cols : rows, seg_len = TRANSPOSED ? rows : cols;
  const int64_t tiles_k = (kp + 63) / 64;            // tiles along the (padded) segment
  const int64_t r0 = ((int64_t)blockIdx.x / tiles_k) * 64, k0 = ((int64_t)blockIdx.x % tiles_k) * 64;
  const int t = threadIdx.x;
  // load the source tile: (output row r0 + i, segment column k0 + j)
#pragma unroll
  for (int h = 0; h < 16; ++h) {
    const int e = t + 256 * h, a = e >> 6, b = e & 63;   // source-contiguous index b
    int64_t sr, sc;
    if (TRANSPOSED) { sr = k0 + a; sc = r0 + b; } else { sr = r0 + a; sc = k0 + b; }
    float v = 0.0f;
    if (sr < rows && sc < cols) {
      if constexpr (SRC_BF16) v = (float)static_cast<const __bf16*>(src)[sr * lds + sc];
      else v = static_cast<const float*>(src)[sr * lds + sc];
    }
    if (TRANSPOSED) tile[b][a] = v; else tile[a][b] = v;   // tile[i][j]: output row i, column j
  }
  __syncthreads();
  (void)seg_len;
  // write: in pass h, thread t -> output row i = 32 h + t / 8, the 8 columns
  // (t % 8) * 8 .. +8 of each segment, one 16-byte store, so that every store
  // instruction of a wave writes 8 whole 128-byte row pieces (16 values per
  // thread as two 16-byte halves of a 32-byte piece wrote half of each line
  // per instruction)
  const int j0 = (t & 7) * 8;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int i = 32 * h + (t >> 3);
    if (r0 + i >= out_rows) break;
    for (int s = 0; s < nseg; ++s) {
      const int p = (planes >> (2 * s)) & 3;
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float a = bf16_piece(tile[i][j0 + 2 * q], p), b = bf16_piece(tile[i][j0 + 2 * q + 1], p);
        w[q] = (pfp8::f2u(a) >> 16) | (pfp8::f2u(b) & 0xFFFF0000u);   // pieces are bf16 values
      }
      const int64_t col = (int64_t)s * kp + k0 + j0;   // kp is a multiple of 64: whole 8-value pieces
      *reinterpret_cast<uint4*>(dst + (r0 + i) * ldd + col) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}
}  // namespace

extern "C" int pratchya_split_pack_bf16(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld_src,
                                        int transpose, int nseg, const int* planes, void* dst, int64_t ld_dst,
                                        int64_t kp, hipStream_t stream) {
  if (rows < 0 || cols < 0 || kp < 0) return pratchya_set_error(PRATCHYA_EINVAL, "split_pack: negative size");
  if (src_dtype != PRATCHYA_DT_F32 && src_dtype != PRATCHYA_DT_BF16)
    return pratchya_set_error(PRATCHYA_EINVAL, "split_pack: source dtype must be f32 or bf16 (got %d)", src_dtype);
  if (nseg < 1 || nseg > 16 || !planes) return pratchya_set_error(PRATCHYA_EINVAL, "split_pack: 1 to 16 segments");
  const int64_t out_rows = transpose ? cols : rows, seg_len = transpose ? rows : cols;
  if (kp % 64 || kp < seg_len || ld_dst < nseg * kp || ld_src < cols)
    return pratchya_set_error(PRATCHYA_EINVAL, "split_pack: segment length %lld must be a multiple of 64 covering "
                              "%lld values, ld_dst >= nseg * kp", (long long)kp, (long long)seg_len);
  if (out_rows == 0 || kp == 0) return PRATCHYA_OK;
  if (!src || !dst || reinterpret_cast<uintptr_t>(dst) % 16 || ld_dst % 8)
    return pratchya_set_error(PRATCHYA_EINVAL, "split_pack: null or misaligned buffer");
  uint32_t pl = 0;
  for (int s = 0; s < nseg; ++s) {
    if (planes[s] < 0 || planes[s] > 3) return pratchya_set_error(PRATCHYA_EINVAL, "split_pack: plane must be 0 to 3");
    pl |= (uint32_t)planes[s] << (2 * s);
  }
  const int64_t tiles = ((out_rows + 63) / 64) * (kp / 64);
  if (tiles > INT32_MAX) return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "split_pack: too many tiles");
  const bool bf = src_dtype == PRATCHYA_DT_BF16;
  uint16_t* d = static_cast<uint16_t*>(dst);
#define PRATCHYA_SPLIT(B, T) hipLaunchKernelGGL((k_split_pack<B, T>), dim3((unsigned)tiles), dim3(256), 0, stream, \
                                                src, rows, cols, ld_src, nseg, pl, d, ld_dst, kp)
  if (bf && transpose) PRATCHYA_SPLIT(true, true);
  else if (bf) PRATCHYA_SPLIT(true, false);
  else if (transpose) PRATCHYA_SPLIT(false, true);
  else PRATCHYA_SPLIT(false, false);
#undef PRATCHYA_SPLIT
  return launch_status("split_pack");
}

extern "C" int pratchya_mfma_ceiling(const void* A, const void* B, int64_t ld, int bf16, int64_t iters,
                                     float* out, int64_t* flop, hipStream_t stream) {
  if (!A || !B || !out || !flop) return pratchya_set_error(PRATCHYA_EINVAL, "mfma_ceiling: null pointer");
  if (ld < 128 || ld % 16 || iters < 1 || iters > INT32_MAX ||
      (reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) % 16)
    return pratchya_set_error(PRATCHYA_EINVAL, "mfma_ceiling: ld must be >= 128 and a multiple of 16, buffers "
                              "16-byte aligned, iters in [1, 2^31)");
  const int64_t grid = gemm_num_cus();
  // per wave and iteration: 16 mfma_tile calls, each 32 x 32 x 64 bytes of K
  // (fp8: one 32x32x64 MFMA, 131072 FLOP; bf16: two 32x32x16, 65536 FLOP)
  *flop = grid * (NTHREADS / 64) * iters * 16 * (bf16 ? 65536 : 131072);
  const uint8_t* a8 = static_cast<const uint8_t*>(A);
  const uint8_t* b8 = static_cast<const uint8_t*>(B);
  if (bf16)
    hipLaunchKernelGGL((k_mfma_ceiling<true>), dim3((unsigned)grid), dim3(NTHREADS), 0, stream, a8, b8, ld,
                       (int)iters, out);
  else
    hipLaunchKernelGGL((k_mfma_ceiling<false>), dim3((unsigned)grid), dim3(NTHREADS), 0, stream, a8, b8, ld,
                       (int)iters, out);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return pratchya_set_error(PRATCHYA_EHIP, "mfma_ceiling: launch failed: %s", hipGetErrorString(err));
  return PRATCHYA_OK;
}

extern "C" int pratchya_transpose_u8(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* dst,
                                     hipStream_t stream) {
  if (rows < 0 || cols < 0) return pratchya_set_error(PRATCHYA_EINVAL, "transpose: negative size");
  if (rows == 0 || cols == 0) return PRATCHYA_OK;
  if (rows % 16 || cols % 16 || reinterpret_cast<uintptr_t>(src) % 16 || reinterpret_cast<uintptr_t>(dst) % 16)
    return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "transpose: sizes must be multiples of 16, buffers 16-byte aligned");
  if (!src || !dst) return pratchya_set_error(PRATCHYA_EINVAL, "transpose: null buffer");
  // 128-wide tiles from 2^22 bytes ([4096,16384]: 36 -> 29 us; [400,1040]:
  // 2.3 us with 64-wide tiles, 3.4 with 128)
  // (either side >= 2^22 implies >= 2^22 bytes; below that the product fits)
  const int64_t big_at = (int64_t)1 << 22;
  const bool big = rows >= big_at || cols >= big_at || rows * cols >= big_at;
  const int64_t tw = big ? 128 : 64;
  const int64_t tr = rows / tw + (rows % tw != 0), tc = cols / tw + (cols % tw != 0);
  if (tr > INT32_MAX / tc) return pratchya_set_error(PRATCHYA_EUNSUPPORTED, "transpose: more than 2^31 tiles");
  const int64_t tiles = tr * tc;
  if (big)
    hipLaunchKernelGGL(k_transpose_u8<128>, dim3((unsigned)tiles), dim3(256), 0, stream, src, rows, cols, dst);
  else
    hipLaunchKernelGGL(k_transpose_u8<64>, dim3((unsigned)tiles), dim3(256), 0, stream, src, rows, cols, dst);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return pratchya_set_error(PRATCHYA_EHIP, "transpose: %s", hipGetErrorString(e));
  return PRATCHYA_OK;
}
