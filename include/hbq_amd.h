/*
 * hbq_amd.h -- C ABI of the MI355X (gfx950) HBQ hot path.
 *
 * Plain pointers and sizes only.  All tensor pointers are device pointers
 * (HIP global memory), row-major and contiguous; `stream` is a hipStream_t
 * (NULL = the legacy default stream).  Every entry point is asynchronous on
 * `stream`, returns 0 on success and a nonzero HBQ_ERR_* code otherwise;
 * hbq_last_error() then returns the message (thread local).
 *
 * dtype codes: 0 = fp16, 1 = bf16, 2 = fp32.  fp16/bf16 tensors are 16-bit
 * patterns, fp32 tensors 32-bit floats.
 *
 * Blocks run along the last dimension: a tensor is passed as [rows, cols]
 * with cols its last dimension; a ragged last block is zero padded, as
 * _reshape_to_blocks does (src/quantizer.py:67-146).
 *
 * Element rounding (`compiled` argument of the quantizer entry points).  The
 * reference's element quantizer exists in two forms that round differently:
 * make_fp_quant's eager op chain (compiled = 0: the Python scalar 0.5004 and the
 * sum |m| + 0.5004 are rounded to T) and the torch.compile'd function that
 * GLOBAL_FP_QUANT_CACHE serves (compiled = 1: one fused fp32 kernel, the sum is
 * not rounded to T), src/quantizer.py:38-63,202-255.  HBQQuantizer selects the
 * compiled form with use_quant_kernel=True (its default, and what PTQ builds),
 * MXFPQuantizer with activate_dynamo=True (src/quantizer.py:464-469,724).  The two
 * differ on a few 16-bit inputs per element format; for fp32 tensors they agree.
 *
 * Element codes (optional output, NULL to skip): sign | 2-bit exponent field
 * | m mantissa bits, exponent field 0 for subnormals, i.e. the OCP encodings
 * of E2M1/E2M2/E2M3/E2M5.  E2M1 codes are packed two per byte (even column
 * in the low nibble, row stride ceil(cols/2) bytes); wider codes take one byte
 * per element (row stride cols).
 */
#ifndef HBQ_AMD_H
#define HBQ_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HBQ_DTYPE_F16 0
#define HBQ_DTYPE_BF16 1
#define HBQ_DTYPE_F32 2

#define HBQ_ERR_INVALID 1
#define HBQ_ERR_UNSUPPORTED 2
#define HBQ_ERR_HIP 3

/* L2 scheme codes, in the order of HBQQuantizer.L2_SCHEME (src/quantizer.py:708) */
#define HBQ_L2_POT 0
#define HBQ_L2_INT 1
#define HBQ_L2_SIG1 2
#define HBQ_L2_FPM1 3
#define HBQ_L2_FP1 4
#define HBQ_L2_FPM10 5
#define HBQ_L2_FPM100 6
#define HBQ_L2_MIX 7

/* Message of the last failing call on this thread ("" after a success). */
const char *hbq_last_error(void);

/* ABI revision of this header (2: the `compiled` element-rounding argument). */
int hbq_abi_version(void);

/* No reference counterpart: a test hook.  on == 1 routes every hbq_hbq_qdq and
 * hbq_mxfp_qdq call to the generic kernels instead of the table-driven ones;
 * on == 2 makes a call that the table-driven kernel declines fail with
 * HBQ_ERR_UNSUPPORTED instead of falling back to the generic one; 0 restores the
 * default.  Returns the old setting. */
int hbq_set_generic_only(int on);

/*
 * MXFP / NVFP quantize-dequantize.
 * Replaces MXFPQuantizer.q (src/quantizer.py:513-539) together with
 * MXFPQuantizer.get_shared_scale (src/quantizer.py:481-511): sc_mbit == 0
 * selects the power-of-two scale (MXFP4/MXFP8), sc_mbit > 0 the FP scale
 * (NVFP4 with E5M3).  y has x's shape and dtype; scales (optional) is
 * [rows, ceil(cols/block_size)] in x's dtype; codes as described above.
 * per_tensor_scale/tensor_scale carry MXFPQuantizer's per-tensor scale,
 * computed by the caller from max|x| (src/quantizer.py:516-524).
 * GPU limits: ebit == 2, mbit in {1,2,3,5}, block_size a power of two 16..1024.
 */
int hbq_mxfp_qdq(const void *x, void *y, void *scales, void *codes, int64_t rows, int64_t cols, int dtype,
                 int block_size, int ebit, int mbit, int sc_ebit, int sc_mbit, int scale_allow_subnormal,
                 int use_round, int use_ceil, int per_tensor_scale, double tensor_scale, int compiled,
                 void *stream);

/*
 * HBQ two-level quantize-dequantize.
 * Replaces HBQQuantizer.q (src/quantizer.py:741-859) with its L1 scale
 * HBQQuantizer.quant_scale (src/quantizer.py:735-739).  Outputs (each
 * optional except y) mirror the keep_l2_scale attributes:
 *   l1_scale [rows, nblk] in x's dtype          -> shared_scale
 *   l2_index [rows, nblk, block/l2_block] uint8 -> l2_scale
 *   scheme   [rows, nblk] uint8                 -> blk_l2_scheme
 * GPU limits: ebit == 2, mbit in {1,2,3}, l2_block_size in {4,8,16,32},
 * l2_sc_bit in 0..3, block_size a power of two 16..1024.
 */
int hbq_hbq_qdq(const void *x, void *y, void *l1_scale, void *l2_index, void *scheme, void *codes, int64_t rows,
                int64_t cols, int dtype, int block_size, int ebit, int mbit, int sc_ebit, int sc_mbit,
                int l2_block_size, int l2_sc_bit, int l2_scheme, int scale_allow_subnormal, int use_ceil,
                int compiled, void *stream);

/* The attention-weight quantizer of the causal manual attention (src/module.py:113-116,
 * HBQQuantizer.q on the softmax output) in place on x [mats, t, t] (fp16 / bf16,
 * t % 128 == 0, block_size 128), with the arguments of hbq_hbq_qdq.  The blocks
 * entirely above the diagonal must hold +0 (the causal softmax gives exactly that);
 * their quantization is +0, so they are left as they are and never read.  Returns
 * HBQ_ERR_UNSUPPORTED for configurations outside the table kernel's (the caller
 * then uses hbq_hbq_qdq). */
int hbq_hbq_qdq_causal(void *x, int64_t mats, int64_t t, int dtype, int block_size, int ebit, int mbit, int sc_ebit,
                       int sc_mbit, int l2_block_size, int l2_sc_bit, int l2_scheme, int scale_allow_subnormal,
                       int use_ceil, int compiled, void *stream);

/*
 * Packed HBQ tensors (no reference counterpart in src/: the bit layout of the
 * HBQ hardware quantizer's outputs, hardware/HBQ_accelerator/hbq_e_quantizer/
 * top.sv:14-45, and of the MAC test vectors, hardware/BQ/MAC_WXAY/tb_WXAY.sv:68-110).
 * For [rows, cols] with cols % block_size == 0, block_size % 8 == 0 and mbit in
 * 1..3, each row packs into four byte strings:
 *   pcodes  cols fields of mbit + 3 bits (the element codes above), element i at
 *           bits [(mbit+3) i, (mbit+3)(i+1)) of the row's little-endian bit string
 *   pl1     one E5M3 byte per block: exponent field (bias 15) << 3 | mantissa,
 *           the bits [14:7] of the scale as fp16; 0xFF for a non-finite scale
 *   pl2     l2_sc_bit bits per sub-block, LSB first (NULL when l2_sc_bit == 0)
 *   pscheme one bit per block, LSB first (Mix only, else NULL)
 * hbq_hbq_packed_strides writes the four row strides in bytes (0 for an absent string).
 */
int hbq_hbq_packed_strides(int64_t cols, int block_size, int mbit, int l2_block_size, int l2_sc_bit,
                           int l2_scheme, int64_t *strides);

/* Packs hbq_hbq_qdq's codes, l1_scale, l2_index and scheme outputs (same
 * geometry and configuration) into the strings above.  Code buffers 8-byte aligned. */
int hbq_hbq_pack(const void *codes, const void *l1_scale, const void *l2_index, const void *scheme, void *pcodes,
                 void *pl1, void *pl2, void *pscheme, int64_t rows, int64_t cols, int dtype, int block_size,
                 int mbit, int l2_block_size, int l2_sc_bit, int l2_scheme, void *stream);

/* Decodes packed strings to y [rows, cols] in dtype: per element
 * R(R(level * l2[j][s]) * l1) with the code's sign, the dequantization of
 * HBQQuantizer.q (src/quantizer.py:790-796), so unpack(pack(q)) equals
 * hbq_hbq_qdq's y bit for bit.  y 16-byte aligned. */
int hbq_hbq_unpack(const void *pcodes, const void *pl1, const void *pl2, const void *pscheme, void *y, int64_t rows,
                   int64_t cols, int dtype, int block_size, int mbit, int l2_block_size, int l2_sc_bit,
                   int l2_scheme, void *stream);

/* Accumulation modes of hbq_gemm_packed_w (the blockquant_ext ops they follow) */
#define HBQ_ACC_FP32 0      /* gemm_fp32_accum */
#define HBQ_ACC_GROUPED 1   /* gemm_fp16_grouped_accum */
#define HBQ_ACC_MXINT8 2    /* gemm_blockquant_mxint8 */
#define HBQ_ACC_MXFP8 3     /* gemm_blockquant_mxfp8 */

/* GEMM on a packed weight for decode-sized M (no counterpart in src/: the
 * low-bit GEMM the packed format feeds).  C[M,N] fp16 = A[M,K] fp16 x W[N,K]^T
 * where W is given by hbq_hbq_pack's strings of an fp16 tensor (E2M1 codes,
 * block 128, l2_block_size 8/16/32, l2_sc_bit <= 2, L2 factors < 4), decoded in
 * registers ahead of MFMA.  Same bits as unpacking W and running the GEMM of
 * acc_mode (the blockquant_ext ops of blockquant_ext.cpp:51-72, in W[N,K]
  * layout).  Limits: 1 <= M <= 32, N % 32 == 0, K % 256 == 0, the group_k /
 * group_n sets of those ops; A 16-byte, pcodes 4-byte, C 8-byte aligned. */
int hbq_gemm_packed_w(const void *A, const void *pcodes, const void *pl1, const void *pl2, const void *pscheme,
                      void *C, int M, int N, int K, int block_size, int mbit, int l2_block_size, int l2_sc_bit,
                      int l2_scheme, int acc_mode, int group_k, int group_n, void *stream);

/*
 * Elementwise E2Mm quantization with subnormals.
 * Replaces the callable returned by make_fp_quant(ebit, mbit) (src/quantizer.py:187-257,
 * compiled = 0) and the compiled one GLOBAL_FP_QUANT_CACHE serves (src/quantizer.py:38-65,
 * compiled = 1).  codes optional, one byte each.
 */
int hbq_elem_quant(const void *x, void *y, void *codes, int64_t n, int dtype, int ebit, int mbit, int compiled,
                   void *stream);

/*
 * Elementwise scale quantization to E(ebit)M(mbit), half-up (use_ceil=0) or
 * ceil rounding.  clip=0 replaces fp_quant (src/quantizer.py:259-328);
 * clip=1 first clips to the format's [min (sub)normal, max normal] range and
 * replaces HBQQuantizer.quant_scale (src/quantizer.py:735-739).
 */
int hbq_scale_quant(const void *x, void *y, int64_t n, int dtype, int ebit, int mbit, int allow_subnormal,
                    int use_ceil, int clip, void *stream);

/*
 * Block-quant GEMMs of blockquant_ext.  A is [M,K] fp16, C is [M,N] fp16 (caller
 * allocated, fully written).  With b_is_nk == 0, B is [K,N] fp16 as the
 * reference ops take it (blockquant_ext.cpp:12-19); with b_is_nk == 1 it is the
 * weight W[N,K] (same arithmetic, no transpose copy needed by the caller).
 * In-group sums use MFMA fp32 accumulation; the cross-group fp16 accumulation
 * and the psum quantization follow the reference step by step.
 */

/* Replaces gemm_fp32_accum -> gemm_fp32_accum_cuda (blockquant_ext.cpp:21-29, gemm.cu:593-616). */
int hbq_gemm_fp32_accum(const void *A, const void *B, void *C, int64_t M, int64_t N, int64_t K, int b_is_nk,
                        void *stream);

/* gemm_fp32_accum with a caller-provided workspace (no reference counterpart: the
 * reference's fp32-accumulation linears run F.linear, whose sum order is the
 * library's).  For long K on grids of at most one round of tiles (the prefill's
 * down projection) it splits K in halves over twice the workgroups, writes their fp32
 * partial sums to ws and adds them in order before the single fp16 rounding; other
 * shapes, or ws_bytes below hbq_gemm_fp32_accum_workspace(), run hbq_gemm_fp32_accum.
 * The result of each half is the group partial hbq_gemm_group_partials gives for
 * group_k = K / 2. */
int64_t hbq_gemm_fp32_accum_workspace(int64_t M, int64_t N, int64_t K, int b_is_nk);
int hbq_gemm_fp32_accum_ws(const void *A, const void *B, void *C, void *ws, int64_t ws_bytes, int64_t M, int64_t N,
                           int64_t K, int b_is_nk, void *stream);

/* No reference counterpart: hbq_gemm_fp32_accum_ws for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * It allocates nothing and takes no workspace: the split-K partials live in a
 * library-owned device buffer of HBQ_NOALLOC_SCRATCH_BYTES (64 MiB: the prefill's
 * down projection, 2 x 2048 x 4096 fp32) on each GPU, held until the process ends.
 * Same results as hbq_gemm_fp32_accum_ws with a sufficient workspace.  Returns
 * HBQ_ERR_INVALID when hbq_gemm_fp32_accum_workspace() of the shape exceeds the buffer.
 * Every call on a GPU shares that GPU's buffer: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialized by the caller. */
#define HBQ_NOALLOC_SCRATCH_BYTES (64ll << 20)
int hbq_gemm_fp32_accum_noalloc(const void *A, const void *B, void *C, int64_t M, int64_t N, int64_t K, int b_is_nk,
                                void *stream);

/* No reference counterpart: `batches` independent fp32-accumulation GEMMs
 * C_z[M,N] = A_z[M,K] W_z[N,K]^T (fp16, z-th problem at element offsets z * stride_*),
 * the same arithmetic as hbq_gemm_fp32_accum with b_is_nk = 1, in one launch.  The
 * decoder's attention products use it: q against k (W = k, no transpose) and the
 * attention weights against the quantized V^T. */
int hbq_gemm_fp32_accum_batched(const void *A, const void *W, void *C, int64_t batches, int64_t M, int64_t N,
                                int64_t K, int64_t stride_a, int64_t stride_w, int64_t stride_c, void *stream);

/* No reference counterpart: hbq_gemm_fp32_accum_batched with problems z of one group of
 * w_group sharing W (W_z at (z / w_group) * stride_w: grouped-query attention, the
 * query heads of one kv head) and C rows ldc elements apart, so that P.V writes the
 * attention output straight into the [tokens, heads, head_dim] layout the o projection
 * reads (C_h at h * head_dim, ldc = heads * head_dim).  The outputs must not overlap:
 * stride_c >= (M - 1) ldc + N, or stride_c >= N with (batches - 1) stride_c + N <= ldc.
 * ldc != N needs K % 64 == 0, N % 8 == 0 and 16-byte aligned rows (else
 * HBQ_ERR_UNSUPPORTED). */
int hbq_gemm_fp32_accum_batched_ex(const void *A, const void *W, void *C, int64_t batches, int64_t M, int64_t N,
                                   int64_t K, int64_t stride_a, int64_t stride_w, int64_t w_group, int64_t stride_c,
                                   int64_t ldc, void *stream);

/* Replaces gemm_fp16_accum -> gemm_fp16_accum_cuda (blockquant_ext.cpp:31-39, gemm.cu:568-591):
 * one fused fp16 multiply-add per k in ascending order (bit-exact for any input). */
int hbq_gemm_fp16_accum(const void *A, const void *B, void *C, int64_t M, int64_t N, int64_t K, int b_is_nk,
                        void *stream);

/* Replaces gemm_fp16_grouped_accum (blockquant_ext.cpp:41-49, gemm.cu:618-667); group_k in {16,32,64,128}. */
int hbq_gemm_fp16_grouped_accum(const void *A, const void *B, void *C, int64_t M, int64_t N, int64_t K,
                                int group_k, int b_is_nk, void *stream);

/* Replaces gemm_blockquant_mxint8 (blockquant_ext.cpp:64-71, gemm.cu:1399-1478);
 * group_k in {64,128,256}, group_n in {4,8,16,32}, K % group_k == 0, N % group_n == 0. */
int hbq_gemm_blockquant_mxint8(const void *A, const void *B, void *C, int64_t M, int64_t N, int64_t K,
                               int group_k, int group_n, int b_is_nk, void *stream);

/* Replaces gemm_blockquant_mxfp8 (blockquant_ext.cpp:55-62, gemm.cu:1040-1135); same limits as mxint8. */
int hbq_gemm_blockquant_mxfp8(const void *A, const void *B, void *C, int64_t M, int64_t N, int64_t K,
                              int group_k, int group_n, int b_is_nk, void *stream);

/* No reference counterpart: writes the fp32 partial sum of every group_k-wide K
 * group, P[ceil(K/group_k), M, N], from the same MFMA accumulation as the GEMMs,
 * so a test can apply the reference epilogue to exactly the kernel's partials.
 * group_k: 16, 32 or a multiple of 64 (a split-K half, for instance). */
int hbq_gemm_group_partials(const void *A, const void *B, void *P, int64_t M, int64_t N, int64_t K, int group_k,
                            int b_is_nk, void *stream);

/* No reference counterpart: the non-finite test of a GEMM output
 * (torch.isfinite(y).all() after the linear, src/module.py:51-66) without a host
 * synchronization.  x is rows x cols elements with row stride ld (elements), as a
 * column slice of a wider output is.  Sets the device int *flag to 1 if any
 * element is NaN or +-inf; leaves it unchanged otherwise.  Writers only ever
 * store 1, so one flag may collect several calls. */
int hbq_flag_nonfinite(const void *x, int64_t rows, int64_t cols, int64_t ld, int dtype, int *flag, void *stream);

/* Causal attention scores, in place: s = R(R(s * scale) + bias), bias 0 on and below
 * the diagonal and -inf above, for mats [t, t] matrices of fp16 / bf16 (t % 8 == 0,
 * s 16-byte aligned).  The two elementwise steps of the reference's manual attention
 * (src/module.py:96-112: attn_weight = q @ k^T * scale_factor; attn_weight +=
 * attn_bias) fused into one pass with the same bits (torch computes each in fp32 and
 * rounds to the dtype; the scalar is converted to fp32). */
int hbq_scale_causal_mask(void *s, int64_t mats, int64_t t, double scale, int dtype, void *stream);

/* Causal attention probabilities from raw scores, in place allowed (no counterpart
 * kernel): the scaling and causal bias of hbq_scale_causal_mask followed by
 * torch.softmax along the rows (src/module.py:96-113), one pass over the scores.  The
 * softmax repeats torch's persistent warp softmax step for step (row max and sum per
 * 64-lane wave in its element order and butterfly order, exp, division), so p has
 * torch's bits.  [mats, t, t] fp16 / bf16 with t a power of two from 64 to 2048,
 * 16-byte aligned. */
int hbq_causal_softmax(const void *s, void *p, int64_t mats, int64_t t, double scale, int dtype, void *stream);

/* Rotary embedding of the decoder's q or k (no counterpart kernel: the elementwise
 * q * cos + rotate_half(q) * sin of the Llama attention the quantization points sit
 * in, apply_rotary_pos_emb at src/module.py:153-158): y[b, h, t, :] = R(R(x * cos[t]) + R(rotate_half(x) * sin[t]))
 * with rotate_half(x) = cat(-x[d/2:], x[:d/2]), each step as torch computes it.  x is
 * read as [b, t, h, d] with element strides (stride_b, stride_t, stride_h, 1), y is
 * written contiguous [b, h, t, d]; cos, sin [t, d] in the same dtype (fp16 / bf16);
 * d % 16 == 0, rows 16-byte aligned. */
int hbq_rope(const void *x, void *y, const void *cos, const void *sin, int64_t b, int64_t h, int64_t t, int64_t d,
             int64_t stride_b, int64_t stride_t, int64_t stride_h, int dtype, void *stream);

/* Decoder plumbing around the quantized linears (no reference kernels: the Hugging Face
 * Llama modules that src/module.py patches, in torch ops).  Each reproduces torch's
 * eager ops bit for bit: every op in fp32 on the fp16 / bf16 values, rounded to the
 * dtype once per op; n and cols multiples of 8, tensors 16-byte aligned.
 *
 * RMSNorm, first half: sum = R(x + res) when res is non-null (the residual add
 * before the norm; sum may alias x), and sq = s * s in fp32 of s = sum or x
 * (h.float().pow(2)).  The row mean of sq is left to torch.mean, whose reduction
 * order it keeps. */
int hbq_rms_prep(const void *x, const void *res, void *sum, float *sq, int64_t n, int dtype, void *stream);

/* RMSNorm, second half: y = R(w * R(R32(x * rs[row]))), the `h * rs`, `.to(dtype)`
 * and `weight *` steps of LlamaRMSNorm with rs = torch.rsqrt(var + eps) [rows] fp32
 * from torch (its rsqrt and this library's can differ in the last bit); w [cols] in
 * the dtype. */
int hbq_rms_apply(const void *x, const float *rs, const void *w, void *y, int64_t rows, int64_t cols, int dtype,
                  void *stream);

/* The gated MLP product y = R(R(silu(g)) * u), silu(g) = g / (1 + exp(-g)) in fp32
 * (torch.nn.functional.silu(gate) * up of QLlamaMLP, src/module.py:547-569, without
 * a quantizer after the activation). */
int hbq_silu_mul(const void *g, const void *u, void *y, int64_t n, int dtype, void *stream);

/* No reference counterpart as kernels: the linears' input quantizer applied to the
 * output of the pass that produces it (src/module.py:45-50, self.aq(x) of
 * _QBaseLinear.forward, on the RMSNorm output that feeds q/k/v and gate/up and on the
 * SiLU product that feeds down, src/module.py:547-569), in one pass whose producer
 * output is never written.  y is bit for bit hbq_hbq_qdq(x = hbq_rms_apply(x, rs, w))
 * and hbq_hbq_qdq(x = hbq_silu_mul(g, u)) with the same quantizer arguments; [rows,
 * cols] row-major, fp16 / bf16.  Returns HBQ_ERR_UNSUPPORTED outside the fused kernels:
 * E2M2 elements (mbit 2), one L2 scheme (not Mix), block_size 128, an E5M3 L1 scale
 * without subnormals, cols % 128 == 0 and 16-byte aligned tensors. */
int hbq_rms_apply_hbq_qdq(const void *x, const float *rs, const void *w, void *y, int64_t rows, int64_t cols,
                          int dtype, int block_size, int ebit, int mbit, int sc_ebit, int sc_mbit, int l2_block_size,
                          int l2_sc_bit, int l2_scheme, int scale_allow_subnormal, int use_ceil, int compiled,
                          void *stream);
int hbq_silu_mul_hbq_qdq(const void *g, const void *u, void *y, int64_t rows, int64_t cols, int dtype,
                         int block_size, int ebit, int mbit, int sc_ebit, int sc_mbit, int l2_block_size,
                         int l2_sc_bit, int l2_scheme, int scale_allow_subnormal, int use_ceil, int compiled,
                         void *stream);

/* No reference counterpart: dst[cols, rows] = src[rows, cols]^T for 16-bit
 * elements.  The blockquant_ext front end uses it to hand a B[K,N] operand to
 * the W[N,K] kernels. */
int hbq_transpose16(const void *src, void *dst, int64_t rows, int64_t cols, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* HBQ_AMD_H */
