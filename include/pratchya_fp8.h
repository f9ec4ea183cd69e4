/*
 * pratchya_fp8.h -- C ABI of the MI355X (gfx950) FP8 block-quantization path.
 *
 * These entry points replace the jnp bodies of pratchya's quantized-array
 * operators in pratchya/_qualia/_qarr.py ("Q" below).  Each is what an XLA FFI
 * handler (or a ctypes / torch host) binds: plain device pointers, sizes and a
 * HIP stream; no framework types.  Every call only enqueues work on `stream`
 * (no host synchronisation, no device allocation); buffers are owned by the
 * caller.  Calls are reentrant and may be issued concurrently on different
 * streams.
 *
 * Tensor model.  A quantized tensor of logical shape [..., H, W] is treated as
 * `slices` independent [H, W] matrices (leading dims flattened; Q:470-482
 * never groups across them).  0-d and 1-d tensors are [1,1] and [1,n]
 * (Q:461-464).  For tgrid (a, b) with a | H and b | W:
 *   n_blk = (H/a)*(W/b) blocks per slice, numbered row-major over the block grid,
 *   K     = gcd(max(1, a*b/16), n_blk) blocks per group,  M = n_blk / K,
 * and the three arrays of Q:506 are
 *   x_fp8  uint8 (OCP e4m3fn) [slices*H*W]  same layout as the input,
 *   sc_fp8 uint8 (e8m0)       [slices*M*K]  one byte per block,
 *   sc_fp32 float             [slices*M]    one group max per group.
 *
 * Return value: PRATCHYA_OK, or an error code with a message available from
 * pratchya_last_error() (thread-local).  PRATCHYA_EINVAL corresponds to the
 * reference's trace-time errors (non-dividing tgrid at Q:470, missing tgrid at
 * Q:27) and maps to XLA FFI InvalidArgument; PRATCHYA_EHIP (launch failure)
 * maps to Internal.  NaN / inf / clamp cases follow the reference and are not
 * errors.
 */
#ifndef PRATCHYA_FP8_H
#define PRATCHYA_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

#define PRATCHYA_OK 0
#define PRATCHYA_EINVAL 1
#define PRATCHYA_EHIP 2
#define PRATCHYA_EUNSUPPORTED 3

/* element types of input buffers */
#define PRATCHYA_DT_F32 0
#define PRATCHYA_DT_BF16 1
#define PRATCHYA_DT_E4M3 2   /* e4m3fn payload + its (1, 128) scales (pratchya_quantize_t128 only) */

/* ABI version of this header (bumped on any signature change). */
int pratchya_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* pratchya_last_error(void);

/* Block layout of one [H, W] slice under tgrid (a, b) (Q:466-480).
 * Writes n_blk, K and M; fails with PRATCHYA_EINVAL if a does not divide H or
 * b does not divide W. */
int pratchya_quant_layout(int64_t H, int64_t W, int64_t a, int64_t b,
                          int64_t* n_blk, int64_t* K, int64_t* M);

/* Device workspace, in bytes, that pratchya_quantize needs for this shape
 * (0 when the single-pass kernel applies). */
size_t pratchya_quantize_workspace_bytes(int x_dtype, int64_t slices, int64_t H, int64_t W,
                                         int64_t a, int64_t b);

/* quantize_impl(x, tgrid) -> (x_fp8, sc_fp8, sc_fp32)     replaces Q:458-506
 * x: `x_dtype` values [slices*H*W].  `workspace` must hold
 * pratchya_quantize_workspace_bytes(...) bytes (may be NULL when that is 0);
 * its contents on entry are irrelevant. */
int pratchya_quantize(const void* x, int x_dtype, int64_t slices, int64_t H, int64_t W,
                      int64_t a, int64_t b, uint8_t* x_fp8, uint8_t* sc_fp8, float* sc_fp32,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Allocation-free pratchya_quantize.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, results and errors as pratchya_quantize without the workspace:
 * layouts that need one use a file-scope device array of
 * pratchya_quantize_noalloc_max_bytes() bytes (16 MiB: 4 Mi blocks; larger
 * layouts fail with PRATCHYA_EUNSUPPORTED), one per device, kept until the
 * process ends.  It allocates nothing and calls no allocating routine.  All
 * calls on one device share that array: calls that overlap on one device
 * (different streams or threads) race. */
int pratchya_quantize_noalloc(const void* x, int x_dtype, int64_t slices, int64_t H, int64_t W,
                              int64_t a, int64_t b, uint8_t* x_fp8, uint8_t* sc_fp8, float* sc_fp32,
                              hipStream_t stream);
size_t pratchya_quantize_noalloc_max_bytes(void);

/* Fake quantization in one pass (no payload is written):
 *   out = dequantize_impl(*quantize_impl(x, tgrid), out_dtype, tgrid)
 * the value of QArrayImpl(x, tgrid).astype(dtype) (Q:339-342 -> Q:458-506,
 * Q:541-569), which is how a quantized Linear emits its output.  With
 * fix_nan != 0 a NaN e8m0 (0xFF) is dequantized as 1.0, the composition
 * quantize_impl -> quantize_impl_bwd (Q:512-526) that a requantized matmul
 * cotangent (Q:637-638) takes back to its f32 input.  sc_fp8 / sc_fp32 receive
 * quantize_impl's scales unrepaired.  out: `out_dtype` values [slices*H*W].
 * `workspace`: pratchya_quantize_dequantize_workspace_bytes(...) bytes (0, and
 * NULL allowed, for tgrid (1, 128) with K = 8 when x and out are 16-byte and
 * sc_fp8 8-byte aligned). */
size_t pratchya_quantize_dequantize_workspace_bytes(int x_dtype, int64_t slices, int64_t H,
                                                    int64_t W, int64_t a, int64_t b);
int pratchya_quantize_dequantize(const void* x, int x_dtype, int64_t slices, int64_t H, int64_t W,
                                 int64_t a, int64_t b, void* out, int out_dtype, int fix_nan,
                                 uint8_t* sc_fp8, float* sc_fp32, void* workspace,
                                 size_t workspace_bytes, hipStream_t stream);

/* pratchya_quantize_dequantize of an f32 x whose block maxima are given:
 * block_max holds, per block of the (a, b) grid (row-major over the block
 * grid, slices stacked), max |x| as f32 bits (what
 * pratchya_gemm_bs_blockmax writes for a = b = 128), so only the group scales
 * and the cast run.  Same outputs and arguments as
 * pratchya_quantize_dequantize otherwise (x_dtype f32, no workspace). */
int pratchya_quantize_dequantize_premax(const float* x, int64_t slices, int64_t H, int64_t W, int64_t a,
                                        int64_t b, const uint32_t* block_max, void* out, int out_dtype,
                                        int fix_nan, uint8_t* sc_fp8, float* sc_fp32, hipStream_t stream);

/* Requantization of a Linear output's cotangent for the FP8 dgrad, tgrid (1, 128):
 *   quantize_impl(dequantize_impl_bwd(g, g_sc8, g_sc32, (1, 128)), (1, 128))
 * i.e. the output quantization's backward (Q:575-601: (g * 2^(e-127) * G) / 128
 * in g's dtype, passed through Q:518-519) followed by the quantization of the
 * cotangent that fp8_matmul's backward contracts (Q:784-789), in one pass (the
 * dequantized cotangent never reaches memory).  g: bf16 / f32 [slices*H*W];
 * g_sc8 / g_sc32: the (1, 128) scales of the tensor g is the cotangent of.
 * Outputs as pratchya_quantize with tgrid (1, 128).  Needs 8 blocks per group
 * (H*W/128 a multiple of 8), 16-byte aligned g, 8-byte aligned e8m0 arrays
 * (PRATCHYA_EUNSUPPORTED otherwise). */
int pratchya_requantize_cotangent(const void* g, int g_dtype, const uint8_t* g_sc8,
                                  const float* g_sc32, int64_t slices, int64_t H, int64_t W,
                                  uint8_t* x_fp8, uint8_t* sc_fp8, float* sc_fp32,
                                  hipStream_t stream);

/* dequantize_impl(x_fp8, sc_fp8, sc_fp32, dtype, tgrid)    replaces Q:541-569
 * out: `out_dtype` values [slices*H*W] = (f32(x8) * (f32(e<<23) * G)) / 128. */
int pratchya_dequantize(const uint8_t* x_fp8, const uint8_t* sc_fp8, const float* sc_fp32,
                        int64_t slices, int64_t H, int64_t W, int64_t a, int64_t b,
                        void* out, int out_dtype, hipStream_t stream);

/* dequantize_impl_bwd: cotangent of the payload          replaces Q:575-601
 * out (same dtype as g) = (g * (f32(e<<23) * G)) / 128, blockwise. */
int pratchya_dequantize_bwd(const void* g, int g_dtype, const uint8_t* sc_fp8,
                            const float* sc_fp32, int64_t slices, int64_t H, int64_t W,
                            int64_t a, int64_t b, void* out, hipStream_t stream);

/* Row gather of a dequantized table: out[i, :] = dequantize_impl(x)[idx[i], :]
 * for a [H, W] table quantized with tgrid (a, b) -- the value of
 * QArrayImpl.__getitem__ with an integer index array (Q:263-284, an embedding
 * lookup, M:32-37) before it is requantized, reading only the rows returned.
 * idx: int64 [n_idx] device array; a negative index counts from the end, and
 * indices are clamped to [0, H - 1] (jnp's out-of-range gather).
 * out: `out_dtype` [n_idx, W]. */
int pratchya_gather_dequantize(const uint8_t* x_fp8, const uint8_t* sc_fp8, const float* sc_fp32,
                               int64_t H, int64_t W, int64_t a, int64_t b, const int64_t* idx,
                               int64_t n_idx, void* out, int out_dtype, hipStream_t stream);

/* Embedding lookup, requantized, in one pass over the indexed rows:   replaces
 *   QArrayImpl(dequantize_impl(x)[idx], (a, b))   (Q:263-284 with an integer
 * index array, then Q:458-506) without the f32 gather in between.
 * x: e4m3fn table [H, W] with its scales, tgrid (xa, xb); idx: int64
 * [slices * T] (negative ids count from the end; clamped to [0, H - 1]); the
 * result [slices, T, W] quantized with tgrid (a, b) into out_fp8 / out_sc8 /
 * out_sc32, exactly the bytes quantize_impl gives for the f32 rows.
 * `workspace`: slices * n_blk * 4 bytes (n_blk of a [T, W] slice under (a, b),
 * pratchya_quant_layout). */
int pratchya_gather_quantize(const uint8_t* x_fp8, const uint8_t* x_sc8, const float* x_sc32, int64_t H, int64_t W,
                             int64_t xa, int64_t xb, const int64_t* idx, int64_t slices, int64_t T, int64_t a,
                             int64_t b, uint8_t* out_fp8, uint8_t* out_sc8, float* out_sc32, void* workspace,
                             size_t workspace_bytes, hipStream_t stream);

/* operators of pratchya_elementwise (jnp's float32 semantics) */
#define PRATCHYA_OP_ADD 0        /* x + y                                                   */
#define PRATCHYA_OP_SUB 1        /* x - y                                                   */
#define PRATCHYA_OP_MUL 2        /* x * y                                                   */
#define PRATCHYA_OP_DIV 3        /* x / y (IEEE)                                            */
#define PRATCHYA_OP_FLOORDIV 4   /* jnp.floor_divide: round(div) of float divmod            */
#define PRATCHYA_OP_MOD 5        /* jnp.remainder: fmod(x, y), + y where the signs differ   */

/* Workspace of pratchya_elementwise for 16-byte aligned payloads (0 when the
 * one-pass kernel applies: result tgrid (1, b), b a multiple of 16 and W of 16,
 * groups of at most 1024 elements, operand grids with b multiples of 16);
 * otherwise slices * n_blk * 4 bytes.  0 for an invalid shape too. */
size_t pratchya_elementwise_workspace_bytes(int64_t slices, int64_t H, int64_t W, int64_t xa, int64_t xb,
                                            int64_t ya, int64_t yb, int64_t a, int64_t b);

/* Quantized arithmetic, one fused pass:                        replaces
 *   QArrayImpl(op(dequantize_impl(x, f32), dequantize_impl(y, f32)), (a, b))
 * -- QArrayImpl's binary operators (Q:121-261; make_elementwise_impl,
 * Q:715-720, then the result's quantize_impl, Q:458-506).  x and y: e4m3fn
 * payloads [slices, H, W] with their scales, quantized with grids (xa, xb) and
 * (ya, yb); op: PRATCHYA_OP_*; out_fp8 / out_sc8 / out_sc32: the result
 * quantized with tgrid (a, b), exactly the bytes quantize_impl gives for the
 * f32 result.  `workspace`: pratchya_elementwise_workspace_bytes(...) bytes
 * (may be NULL when that is 0; unaligned payloads need the general path's
 * workspace, else PRATCHYA_EINVAL). */
int pratchya_elementwise(int op, const uint8_t* x_fp8, const uint8_t* x_sc8, const float* x_sc32, int64_t xa,
                         int64_t xb, const uint8_t* y_fp8, const uint8_t* y_sc8, const float* y_sc32, int64_t ya,
                         int64_t yb, int64_t slices, int64_t H, int64_t W, int64_t a, int64_t b,
                         uint8_t* out_fp8, uint8_t* out_sc8, float* out_sc32, void* workspace,
                         size_t workspace_bytes, hipStream_t stream);

/* Momentum of the quantized Miulion optimizer step, one pass      replaces
 * pratchya/_nnx_impl/_optimizer.py:124-135 (a layer of a 3-D stacked leaf,
 * bf16 arithmetic) and :157-176 (a 2-D leaf, f32 arithmetic):
 *   m = dequantize(momentum) in the arithmetic dtype, g = the gradient in it,
 *   c_out = beta1 * m + beta1c * g,   m_new = beta2 * m + beta2c * g
 * with beta1c = 1 - beta1 and beta2c = 1 - beta2 as the host rounds them.
 * Every product and sum is rounded separately in arith_dtype (PRATCHYA_DT_F32
 * or PRATCHYA_DT_BF16; the constants must already be values of that dtype).
 * momentum: an e4m3fn payload [slices, H, W] with its scales (tgrid (a, b));
 * g: e4m3fn with g_sc8 / g_sc32 in the same layout (a quantized gradient), or
 * bf16 / f32 [slices, H, W].  c_out and m_new: arith_dtype [slices, H, W];
 * m_new is quantized with pratchya_quantize to give the new momentum. */
int pratchya_momentum(const uint8_t* m_fp8, const uint8_t* m_sc8, const float* m_sc32, const void* g,
                      int g_dtype, const uint8_t* g_sc8, const float* g_sc32, int64_t slices, int64_t H,
                      int64_t W, int64_t a, int64_t b, int arith_dtype, float beta1, float beta1c,
                      float beta2, float beta2c, void* c_out, void* m_new, hipStream_t stream);

/* One Newton-Schulz combination                                 replaces
 * pratchya/_nnx_impl/_optimizer.py:26-27 (X = 1.5 * X - 0.5 * B, B = (X X^T) X):
 *   out = rnd(rnd(1.5 * x) - rnd(0.5 * b))
 * elementwise over n elements of `dtype` (PRATCHYA_DT_BF16 or PRATCHYA_DT_F32),
 * every operation rounded to dtype as the reference's jnp arithmetic does.
 * out may be x. */
int pratchya_ns_combine(const void* x, const void* b, void* out, int64_t n, int dtype, hipStream_t stream);

/* Update of the Miulion step                                  replaces
 * pratchya/_nnx_impl/_optimizer.py:147-153 and :189-197:
 *   out = -(lr * u' + lr_wd * p),  u' = sign(u) (use_sign, Lion) or u * scale (Muon:
 *   u = Newton-Schulz(c), scale = sqrt(max(N, M)))
 * The parameter p and u * scale are rounded to the leaf dtype arith_dtype
 * (scale already a value of it); the products and the sum are f32 (lr and
 * lr_wd = lr * wd are f32), rounded once to out_dtype.  u: f32 or bf16
 * [slices, H, W] (an f32 u with bf16 arith_dtype only with use_sign); p: the
 * parameter, e4m3fn with p_sc8 / p_sc32 (tgrid (a, b)), or bf16 / f32; out:
 * out_dtype (f32 or bf16). */
int pratchya_apply_update(const void* u, int u_dtype, int use_sign, float scale, const void* p,
                          int p_dtype, const uint8_t* p_sc8, const float* p_sc32, int64_t slices,
                          int64_t H, int64_t W, int64_t a, int64_t b, int arith_dtype, float lr,
                          float lr_wd, void* out, int out_dtype, hipStream_t stream);

/* Transposed requantize, tgrid (128, 1):     replaces quantize_impl(x, (128, 1)), Q:458-506,
 * with the payload written transposed (the layout fp8_matmul's backward
 * contracts, Q:784-789, and the wgrad GEMM reads).
 * x: [slices, T, C] row-major, x_dtype PRATCHYA_DT_BF16 / PRATCHYA_DT_F32, or
 * PRATCHYA_DT_E4M3: an e4m3fn payload quantized with tgrid (1, 128) whose
 * scales are x_sc8 / x_sc32; it is dequantized to f32 exactly as
 * dequantize_impl (Q:562-564) before requantization.  A bf16 x given with
 * x_sc8 / x_sc32 is the cotangent of a tensor quantized (1, 128) with those
 * scales: dequantize_impl_bwd (Q:575-601, bf16((x * 2^(e-127) * G) / 128)) is
 * applied first, in registers (the wgrad cotangent of the FP8 backward).
 * Outputs: xt_fp8 uint8 [slices, C, T] (payload of quantize_impl transposed per
 * slice), sc_fp8 [slices*M*8] and sc_fp32 [slices*M] exactly as
 * quantize_impl(x, (128, 1)) (M = T*C/1024; a group is 8 adjacent channels of
 * one 128-token block row).  T must be a multiple of 128 (PRATCHYA_EINVAL), C of
 * 8 (PRATCHYA_EUNSUPPORTED) and, with input scales, of 128 (PRATCHYA_EINVAL). */
int pratchya_quantize_t128(const void* x, int x_dtype, const uint8_t* x_sc8, const float* x_sc32,
                           int64_t slices, int64_t T, int64_t C, uint8_t* xt_fp8, uint8_t* sc_fp8,
                           float* sc_fp32, hipStream_t stream);

/* Requantize, tgrid (128, 1), payload in x's layout:
 *                                      replaces quantize_impl(x, (128, 1)), Q:458-506.
 * Arguments, inputs, scales and errors as for pratchya_quantize_t128; the
 * payload q_fp8 is [slices, T, C] (quantize_impl's own output, 16-byte
 * aligned; sc_fp8 8-byte aligned), which the FP8 GEMM reads K-major
 * (pratchya_gemm_bs_kmajor) when it contracts over the tokens (fp8_matmul's
 * weight gradient, Q:784-789). */
int pratchya_quantize_128x1(const void* x, int x_dtype, const uint8_t* x_sc8, const float* x_sc32,
                            int64_t slices, int64_t T, int64_t C, uint8_t* q_fp8, uint8_t* sc_fp8,
                            float* sc_fp32, hipStream_t stream);

/* Quantize (1, 128) and requantize (128, 1) in one pass:
 *       replaces quantize_impl(x, (1, 128)) (Q:458-506, the quantized Linear's
 *       input, pratchya/_nnx_impl/_module.py:46-50) together with
 *       quantize_impl(dequantize_impl(<that>), (128, 1)) (Q:541-569, Q:458-506:
 *       the stored activation requantized along the tokens for the FP8 weight
 *       gradient, fp8_matmul's scheme Q:784-789).
 * x: bf16 or f32 [slices, T, C] (PRATCHYA_DT_*), 16-byte aligned; T a multiple
 * of 128 and C of 128 (PRATCHYA_EINVAL), C of 1024 (PRATCHYA_EUNSUPPORTED).
 * Outputs, per slice exactly quantize_impl's: q_fp8 [slices, T, C], sc_fp8
 * [slices * T * C / 128] (8-byte aligned), sc_fp32 [slices * T * C / 1024]
 * for (1, 128); t_fp8 [slices, T, C] (the (128, 1) payload in x's layout, as
 * pratchya_quantize_128x1 writes it), t_sc8 [slices * T * C / 128] (16-byte
 * aligned), t_sc32 [slices * T * C / 1024] (8-byte aligned) for (128, 1).
 * Bit-identical to pratchya_quantize followed by pratchya_quantize_128x1 of
 * its payload; the input is read once. */
int pratchya_quantize_dual(const void* x, int x_dtype, int64_t slices, int64_t T, int64_t C, uint8_t* q_fp8,
                           uint8_t* sc_fp8, float* sc_fp32, uint8_t* t_fp8, uint8_t* t_sc8, float* t_sc32,
                           hipStream_t stream);

/* Transposed quantize, tgrid (1, 128) of the transposed tensor:
 *                                         replaces quantize_impl(x^T, (1, 128)),
 * Q:458-506, as fp8_matmul's backward quantizes its transposed raw inputs
 * (Q:786-788), without materialising x^T.
 * x: [slices, T, C] as for pratchya_quantize_t128 (bf16, f32, or an e4m3fn
 * payload with its (1, 128) scales; a bf16 x with scales goes through
 * dequantize_impl_bwd first).  Blocks are 128 tokens of one channel, groups 8
 * consecutive blocks of one channel (T a multiple of 1024, else
 * PRATCHYA_EUNSUPPORTED).  Outputs exactly quantize_impl(x^T, (1, 128)) per
 * slice: xt_fp8 [slices, C, T], sc_fp8 [slices * C * T / 128] (8-byte
 * aligned), sc_fp32 [slices * C * T / 1024].  C a multiple of 8 (128 with
 * input scales). */
int pratchya_quantize_t1x128(const void* x, int x_dtype, const uint8_t* x_sc8, const float* x_sc32,
                             int64_t slices, int64_t T, int64_t C, uint8_t* xt_fp8, uint8_t* sc_fp8,
                             float* sc_fp32, hipStream_t stream);

/* Block-scaled FP8 GEMM, "NT" form:                         replaces the f32 dot
 *   C[m, n] = sum_k dequant(A)[m, k] * dequant(B)[n, k]      of matmul_impl
 * (Q:605-608) and of its backward (Q:621-622), with FP8 operands.
 * A: e4m3fn [M, K] (row stride lda bytes), B: e4m3fn [N, K] (ldb); both
 * K-contiguous.  Each operand's scales are the (sc_fp8, sc_fp32) pair of the
 * quantizer, addressed for (row, 128-wide K block kb) as
 *   block = (row / rdiv) * sr + kb * sk,  e8m0 = sc8[block],  G = sc32[block / kg]
 * so that an operand quantized as [rows, K] with tgrid (a, 128) is
 * (rdiv, sr, sk, kg) = (a, K/128, 1, K_group), and one quantized as [K, rows]
 * with tgrid (128, b) and transposed is (b, 1, rows/b, K_group).
 * C: [M, N] with row stride ldc elements (a multiple of 4 for f32, 8 for
 * bf16), c_dtype f32 or bf16; only the M x N outputs are written.
 * K must be a multiple of 128 (PRATCHYA_EUNSUPPORTED otherwise); M and N are
 * any sizes, except that an N below 256 must be a multiple of 4 (f32) or 8
 * (bf16).  An operand of fewer than 256 rows is read as 256 rows: its buffer
 * must be readable that far (the extra rows' contents only reach outputs that
 * are not stored).  The e8m0 arrays are read in aligned 4-byte words: each
 * must be readable up to the next multiple of 4 bytes.  Any group layout is
 * accepted: the kernel reloads group maxima wherever some row's group changes
 * along K (see pratchya_gemm_span). */
int pratchya_gemm_bs_nt(const uint8_t* A, int64_t lda, const uint8_t* a_sc8, const float* a_sc32,
                        int64_t a_rdiv, int64_t a_sr, int64_t a_sk, int64_t a_kg,
                        const uint8_t* B, int64_t ldb, const uint8_t* b_sc8, const float* b_sc32,
                        int64_t b_rdiv, int64_t b_sr, int64_t b_sk, int64_t b_kg,
                        int64_t M, int64_t N, int64_t K, void* C, int64_t ldc, int c_dtype,
                        hipStream_t stream);

/* The GEMM with the product's requantization in its epilogue: replaces
 *   QArrayImpl(matmul_impl(x, y), (1, 128)).astype(dtype)
 * (Q:605-608, then quantize_impl Q:458-506 and dequantize_impl Q:541-569), the
 * quantized Linear's output (pratchya/_nnx_impl/_module.py:46-50); with
 * fix_nan = 1, quantize_impl_bwd's dequantization of a requantized cotangent
 * instead (an e8m0 byte 255 read as 1.0, Q:521-526: the dgrad output).
 * Operands, M, K and ldc as pratchya_gemm_bs_nt (B's scale groups at least 32
 * rows).  N must be a multiple of 1024: a (1, 128) group of the [M, N] output
 * is 8 blocks of one row, and the kernel exchanges block maxima between the
 * four 256-column tiles of a group.  C [M, N] (ldc) receives the dequantized
 * values in c_dtype (f32 or bf16), c_sc8 [M * N / 128] and c_sc32 [M * N / 1024]
 * the scales quantize_impl(C_f32, (1, 128)) returns.  The results equal
 * pratchya_gemm_bs_nt to f32 followed by pratchya_quantize_dequantize bit for
 * bit.  workspace: pratchya_gemm_bs_nt_fq_workspace_bytes(M, N) bytes, 4-byte
 * aligned, cleared by a kernel of this call (calls sharing one workspace must
 * not overlap); the 32-bit word at byte pratchya_gemm_bs_nt_fq_status_offset(M,
 * N) of it is set to 1 if the kernel's bounded wait for a group's four tiles
 * ran out (never expected: that group's outputs are then NaN), else left 0;
 * the caller reads it after the call has completed (-1: unsupported shape). */
int64_t pratchya_gemm_bs_nt_fq_workspace_bytes(int64_t M, int64_t N);
int64_t pratchya_gemm_bs_nt_fq_status_offset(int64_t M, int64_t N);
int pratchya_gemm_bs_nt_fq(const uint8_t* A, int64_t lda, const uint8_t* a_sc8, const float* a_sc32,
                           int64_t a_rdiv, int64_t a_sr, int64_t a_sk, int64_t a_kg,
                           const uint8_t* B, int64_t ldb, const uint8_t* b_sc8, const float* b_sc32,
                           int64_t b_rdiv, int64_t b_sr, int64_t b_sk, int64_t b_kg,
                           int64_t M, int64_t N, int64_t K, void* C, int64_t ldc, int c_dtype, int fix_nan,
                           uint8_t* c_sc8, float* c_sc32, void* workspace, int64_t workspace_bytes,
                           hipStream_t stream);

/* The GEMM with the product's (1, 1) requantization in its epilogue: replaces
 *   QArrayImpl(matmul_impl(x, y), (1, 1)).astype(dtype)
 * (Q:605-608, then quantize_impl Q:458-506 and dequantize_impl Q:541-569), the
 * output of a Linear whose weight grid is (a, 1): lm_head
 * (pratchya/_nnx_impl/_model.py:77) and the LoRA projections
 * (pratchya/_nnx_impl/_module.py:82-84), whose output grid is (x.tgrid[0],
 * W.tgrid[1]) (Q:104-105).  With tgrid (1, 1) each element is its own block
 * and group, so the epilogue needs no exchange between tiles.  Operands, M, K,
 * C, ldc and c_dtype as pratchya_gemm_bs_nt; N a multiple of 16
 * (PRATCHYA_EUNSUPPORTED otherwise).  C [M, N] receives the dequantized values
 * in c_dtype, c_sc8 [M * N] the e8m0 bytes and c_sc32 [M * N] the group maxima
 * (both in row order, 16-byte aligned), the arrays quantize_impl(C_f32, (1, 1))
 * returns.  The results equal pratchya_gemm_bs_nt to f32 followed by
 * pratchya_quantize_dequantize with tgrid (1, 1) bit for bit. */
int pratchya_gemm_bs_nt_q11(const uint8_t* A, int64_t lda, const uint8_t* a_sc8, const float* a_sc32,
                            int64_t a_rdiv, int64_t a_sr, int64_t a_sk, int64_t a_kg,
                            const uint8_t* B, int64_t ldb, const uint8_t* b_sc8, const float* b_sc32,
                            int64_t b_rdiv, int64_t b_sr, int64_t b_sk, int64_t b_kg,
                            int64_t M, int64_t N, int64_t K, void* C, int64_t ldc, int c_dtype,
                            uint8_t* c_sc8, float* c_sc32, hipStream_t stream);

/* The quantize prologue: replaces the quantized Linear's
 *   QArrayImpl(x, (1, 128)) @ kernel            (pratchya/_nnx_impl/_module.py:46-50)
 * i.e. quantize_impl(X, (1, 128)) (Q:458-506) followed by matmul_impl
 * (Q:605-608), in one launch: before their first output tiles, the GEMM's
 * workgroups quantize each 1024-value group of the bf16 activation X [M, K]
 * once (row stride ldx elements, a multiple of 8, 16-byte aligned) and write
 * the payload A [M, K] (row stride K), e8m0 bytes a_sc8 [M * K / 1024, 8] and
 * group maxima a_sc32 [M * K / 1024] (the arrays quantize_impl returns, bit
 * for bit; 256-byte aligned), wait for one another, and read them back as
 * their A operand.  B and its scales, C, ldc, c_dtype as pratchya_gemm_bs_nt
 * (B's scale groups at least 32 rows); fq = 1: the output requantization of
 * pratchya_gemm_bs_nt_fq as well (N a multiple of 1024, c_sc8 / c_sc32 as
 * there; fq = 0: they are unused).  M at least 256, K a multiple of 1024
 * (PRATCHYA_EUNSUPPORTED otherwise).  workspace:
 * pratchya_gemm_bs_nt_qa_workspace_bytes(M, N, fq) bytes, 4-byte aligned,
 * cleared by a kernel of this call (calls sharing one workspace must not
 * overlap); its 32-bit word at byte pratchya_gemm_bs_nt_qa_status_offset(M, N,
 * fq) has bit 1 set if a wait for a group of four output tiles ran out (those
 * outputs are then NaN) and bit 2 if the wait for the prologue's end ran out
 * (the outputs are then not defined); never expected while the call has the
 * device to itself. */
int64_t pratchya_gemm_bs_nt_qa_workspace_bytes(int64_t M, int64_t N, int fq);
int64_t pratchya_gemm_bs_nt_qa_status_offset(int64_t M, int64_t N, int fq);
int pratchya_gemm_bs_nt_qa(const void* X, int64_t ldx, uint8_t* A, uint8_t* a_sc8, float* a_sc32,
                           const uint8_t* B, int64_t ldb, const uint8_t* b_sc8, const float* b_sc32,
                           int64_t b_rdiv, int64_t b_sr, int64_t b_sk, int64_t b_kg, int64_t M, int64_t N,
                           int64_t K, void* C, int64_t ldc, int c_dtype, int fq, uint8_t* c_sc8, float* c_sc32,
                           void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* pratchya_gemm_bs_nt with both operands K-major:  the weight gradient
 * (Q:621-622, matmul_impl's backward, dW = x^T . dY over the tokens) reading
 * x and dY quantized (128, 1) in their own [T, C] layout, through the LDS
 * transposing loads, instead of transposed payloads.  A: e4m3fn [K, M] (row
 * stride lda >= M), B: [K, N] (ldb >= N); M, N, lda, ldb multiples of 16;
 * scales, K and C as pratchya_gemm_bs_nt (the scale layouts address
 * (row, K block) as for the [M, K] / [N, K] views).  Each MFMA lane sums the
 * same K values as with the K-contiguous operands, so the output is
 * bit-identical to pratchya_gemm_bs_nt on the transposed payloads. */
int pratchya_gemm_bs_kmajor(const uint8_t* A, int64_t lda, const uint8_t* a_sc8, const float* a_sc32,
                            int64_t a_rdiv, int64_t a_sr, int64_t a_sk, int64_t a_kg, const uint8_t* B,
                            int64_t ldb, const uint8_t* b_sc8, const float* b_sc32, int64_t b_rdiv,
                            int64_t b_sr, int64_t b_sk, int64_t b_kg, int64_t M, int64_t N, int64_t K,
                            void* C, int64_t ldc, int c_dtype, hipStream_t stream);

/* The weight gradient's GEMM with its requantization's first pass in the
 * epilogue: pratchya_gemm_bs_nt (kmajor = 0) or pratchya_gemm_bs_kmajor
 * (kmajor = 1; lda / ldb as there) to an f32 C [M, N], which also writes, for
 * each 128 x 128 block of C, max |c| as f32 bits into block_max [M / 128, N /
 * 128] -- the block maxima quantize_impl(C, (128, 128)) starts from (Q:484-487),
 * so that the requantization of matmul_impl's weight cotangent (Q:621-622,
 * :637-638) skips its own pass over C (pratchya_quantize_dequantize_premax).
 * M and N multiples of 128 (PRATCHYA_EUNSUPPORTED otherwise); the other
 * arguments and limits as the two GEMMs. */
int pratchya_gemm_bs_blockmax(const uint8_t* A, int64_t lda, const uint8_t* a_sc8, const float* a_sc32,
                              int64_t a_rdiv, int64_t a_sr, int64_t a_sk, int64_t a_kg, const uint8_t* B,
                              int64_t ldb, const uint8_t* b_sc8, const float* b_sc32, int64_t b_rdiv,
                              int64_t b_sr, int64_t b_sk, int64_t b_kg, int64_t M, int64_t N, int64_t K,
                              int kmajor, float* C, int64_t ldc, uint32_t* block_max, hipStream_t stream);

/* bf16 GEMM, "NT" form:                  replaces the bf16 dots of newton_schulz
 *   C[m, n] = sum_k A[m, k] * B[n, k]     (pratchya/_nnx_impl/_optimizer.py:20-22,
 * A @ A.T and (A @ A.T) @ A in the leaf's dtype; jnp's bf16 dot accumulates in f32)
 * with f32 accumulation.  A: bf16 [M, K] (row stride lda elements), B: bf16
 * [N, K] (ldb); lda, ldb multiples of 8, buffers 16-byte aligned.  C: [M, N]
 * (ldc), c_dtype f32 or bf16 (rounded once, RNE).  K a multiple of 64
 * (PRATCHYA_EUNSUPPORTED otherwise); M, N and short operands as
 * pratchya_gemm_bs_nt (an operand of fewer than 256 rows is read as 256). */
int pratchya_gemm_bf16_nt(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M, int64_t N,
                          int64_t K, void* C, int64_t ldc, int c_dtype, hipStream_t stream);

/* Frobenius normalization of newton_schulz's bf16 input (_optimizer.py:17:
 * X = G / (jnp.linalg.norm(G, ord='fro') + 1e-7), replacing its four jnp
 * element passes): each square rounded to bf16, their f32 sum rounded to
 * bf16, the square root and the sum with 1e-7 each rounded to bf16, every
 * quotient rounded to bf16; two passes in a fixed reduction order
 * (deterministic).  g, x: bf16 [n], 16-byte aligned; x may be g.  workspace:
 * device memory of pratchya_ns_normalize_workspace_bytes() bytes (the first
 * pass's partial sums), 4-byte aligned. */
int64_t pratchya_ns_normalize_workspace_bytes(void);
int pratchya_ns_normalize(const void* g, void* x, int64_t n, void* workspace, int64_t workspace_bytes,
                          hipStream_t stream);

/* The same normalization of an f32 input (_optimizer.py:17 on the f32 leaves
 * of 2-D quantized parameters, _optimizer.py:157-163): each square rounded to
 * f32, their f32 sum (the fixed order of pratchya_ns_normalize), sqrt and the
 * sum with 1e-7 in f32, IEEE f32 quotients.  g, x: f32 [n], 16-byte aligned;
 * x may be g; workspace as pratchya_ns_normalize. */
int pratchya_ns_normalize_f32(const float* g, float* x, int64_t n, void* workspace, int64_t workspace_bytes,
                              hipStream_t stream);

/* One Newton-Schulz step on the bf16 MFMA kernel: C = 1.5 X - 0.5 bf16(A . B^T),
 * the product of pratchya_gemm_bf16_nt (_optimizer.py:20-22, rounded once to
 * bf16) combined with X in its epilogue exactly as pratchya_ns_combine
 * (_optimizer.py:26-27: 1.5 x and 0.5 b each rounded to bf16, then their
 * difference), so that B never goes through HBM.  A, B, M, N, K as
 * pratchya_gemm_bf16_nt with a bf16 output; X: bf16 [M, N] (row stride ldx, a
 * multiple of 8; 16-byte aligned); C: bf16 [M, N] (ldc), not overlapping X
 * (PRATCHYA_EINVAL otherwise).  b_kmajor: B is given in its K-major layout,
 * the [K, N] matrix B^T (row stride ldb >= N; N and ldb multiples of 8),
 * read through the LDS transposing loads: with B^T = X (the iterate of a
 * wide or square leaf) the second product needs no transposed copy. */
int pratchya_gemm_bf16_nt_ns(const void* A, int64_t lda, const void* B, int64_t ldb, int b_kmajor, int64_t M,
                             int64_t N, int64_t K, const void* X, int64_t ldx, void* C, int64_t ldc,
                             hipStream_t stream);

/* Symmetric bf16 product C = A . A^T:     replaces the Gram product of newton_schulz
 *   C[m, n] = sum_k A[m, k] * A[n, k]      (pratchya/_nnx_impl/_optimizer.py:20-22,
 * A @ A.T of the wide iterate, and A.T @ A of a tall one, whose transpose is A)
 * with f32 accumulation, rounded once to bf16.  Only the tiles on and above
 * the diagonal are computed (stream-K: every CU takes an equal share of
 * their K steps; a tile split between CUs is summed in f32 by the CU holding
 * its first steps, in a fixed order, so results are deterministic), and the
 * lower triangle is written as the transposed upper one (C == C^T exactly).
 * A: bf16 [M, K] (row stride lda), or with a_kmajor its K-major layout, the
 * [K, M] matrix A^T (row stride lda >= M): the tall iterate itself, read
 * through the LDS transposing loads instead of a transposed copy; lda a
 * multiple of 8, 16-byte aligned; M a multiple of 256 and K of 64
 * (PRATCHYA_EUNSUPPORTED otherwise).  C: bf16 [M, M] (ldc), not overlapping A.  workspace: device memory of
 * pratchya_gemm_bf16_gram_workspace_bytes(M, K) bytes (f32 partial tiles and
 * flags, ~64 MB on a 256-CU device), 16-byte aligned; the 32-bit word at byte
 * pratchya_gemm_bf16_gram_status_offset(M, K) of it is set to 1 if a partial
 * tile did not arrive in time (that tile is then NaN), else left 0; the
 * caller reads it after the call has completed (-1: unsupported shape).
 * Calls that share a workspace must not overlap. */
int64_t pratchya_gemm_bf16_gram_workspace_bytes(int64_t M, int64_t K);
int64_t pratchya_gemm_bf16_gram_status_offset(int64_t M, int64_t K);
int pratchya_gemm_bf16_gram(const void* A, int64_t lda, int64_t M, int64_t K, int a_kmajor, void* C, int64_t ldc,
                            void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* f32 operands of pratchya_gemm_bf16_nt:    for the f32 products of the mixed
 * matmuls (Q:645-712, jnp.matmul of a dequantized array and an f32 array) and
 * of matmul_impl's backward (Q:618-622).  An f32 value v is the exact sum of
 * the bf16 pieces p0 = trunc_bf16(v), p1 = trunc_bf16(v - p0), p2 = v - p0 - p1,
 * and piece products are exact in f32, so an f32 dot product is a bf16 dot
 * product over piece pairs placed side by side along K ((0,0) (0,1) (1,0)
 * (0,2) (1,1) (2,0) drop only terms below 2^-24 of the largest product).
 * src: f32 or bf16 [rows, cols] (row stride ld_src elements).  Writes dst,
 * bf16 [out_rows, ld_dst] (ld_dst a multiple of 8, dst 16-byte aligned), with
 * out_rows = rows (transpose = 0: segments run along src rows) or cols
 * (transpose = 1: along src columns); segment s (nseg <= 16) holds piece
 * planes[s] of its source vector in columns [s*kp, s*kp + len), zeros up to
 * (s+1)*kp; kp a multiple of 64 covering len = cols (or rows).  Planes 0, 1, 2
 * are the pieces (a non-finite value is its own piece 0, its other pieces 0);
 * plane 3 is piece 0 with non-finite values written as 0 (for every pair but
 * (0,0), so that inf meets only the other operand's leading piece). */
int pratchya_split_pack_bf16(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld_src,
                             int transpose, int nseg, const int* planes, void* dst, int64_t ld_dst, int64_t kp,
                             hipStream_t stream);

/* 16-bit transpose: src [rows, cols] -> dst [cols, rows] (bf16 X -> X.T, the
 * K-contiguous operand of the Newton-Schulz product (X X^T) X,
 * _optimizer.py:21).  rows and cols multiples of 8, buffers 16-byte aligned. */
int pratchya_transpose_b16(const void* src, int64_t rows, int64_t cols, void* dst, hipStream_t stream);

/* Span of an operand's scale layout: the largest P such that every row's group
 * index is constant over each aligned run of P 128-wide K blocks (the GEMM
 * reloads group maxima and rescales its accumulator at multiples of it);
 * 0 for invalid arguments.  Host-only query, used by tests. */
int64_t pratchya_gemm_span(int64_t rows, int64_t K, int64_t r_div, int64_t s_r, int64_t s_k,
                           int64_t kg);

/* Byte transpose of an fp8 payload: src [rows, cols] -> dst [cols, rows]
 * (the K-contiguous operand layout the GEMM reads; QArrayImpl.T, Q:349-352,
 * moves the data the same way).  rows and cols multiples of 16. */
int pratchya_transpose_u8(const uint8_t* src, int64_t rows, int64_t cols, uint8_t* dst,
                          hipStream_t stream);

/* Measurement aid, no counterpart in the reference: the GEMM kernel's MFMA
 * sequence (fp8: v_mfma_scale_f32_32x32x64_f8f6f4; bf16 != 0: two
 * v_mfma_f32_32x32x16_bf16 per 64 bytes of K) run back to back on operand
 * bytes from A and B (the first 256 rows, 128 bytes of each; ld the row
 * stride in bytes, >= 128), `iters` times per wave on every compute unit, with
 * no memory traffic in the loop: the sustained MFMA rate on such data, which a
 * power-limited clock sets below the datasheet peak.  *flop receives the FLOP
 * count of the launch (for timing by the caller); out (one float, device) is
 * written only to keep the loop alive. */
int pratchya_mfma_ceiling(const void* A, const void* B, int64_t ld, int bf16, int64_t iters, float* out,
                          int64_t* flop, hipStream_t stream);

/* Test hooks for the element conversions the kernels use (no reference
 * counterpart; they let the tests check the device arithmetic exhaustively).
 *   mode 0: software bit arithmetic, mode 1: gfx950 conversion instructions.
 * pratchya_debug_bf16_to_e4m3:  in uint16 bf16 bits [n] -> out uint8 [n]
 * pratchya_debug_f32_to_bf16:   in float [n]           -> out uint16 [n] */
int pratchya_debug_bf16_to_e4m3(const uint16_t* in, uint8_t* out, int64_t n, int mode,
                                hipStream_t stream);
int pratchya_debug_f32_to_bf16(const float* in, uint16_t* out, int64_t n, int mode,
                               hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PRATCHYA_FP8_H */
