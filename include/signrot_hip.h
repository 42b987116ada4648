/* C ABI of the SignRot W4A4 real-quant path for MI355X (gfx950).
 *
 * Library: signrot_amd/_lib/libsignrot_hip.so
 *
 * Every entry point takes raw device pointers, int64 sizes and an explicit
 * hipStream_t (passed as void*; NULL is the default stream), launches
 * asynchronously on that stream, and returns SRQ_OK (0) or a negative
 * SRQ_E* code.  Nothing throws across the ABI; srq_last_error() returns a
 * thread-local message for the last failure on the calling thread.  No entry
 * point synchronises the stream or reads device data on the host, so all of
 * them can be captured into a HIP graph.  Outputs are caller-allocated.
 *
 * Data formats (the reference's interchange formats, kept bit-for-bit):
 *   packed int4  : uint8, two's-complement nibbles, element 2j in the low
 *                  nibble and 2j+1 in the high nibble of byte j
 *                  (signrot/functional/quantization.py:45-52);
 *   KV uint4     : same nibble order, unsigned;
 *   fp16         : IEEE binary16.
 *
 * Each declaration names the reference interface it replaces (file:line in
 * HYU-ARK-Lab/SignRot).
 */
#ifndef SIGNROT_HIP_H
#define SIGNROT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SRQ_OK 0
#define SRQ_EINVAL (-1)      /* bad argument: shape, pointer, alignment   */
#define SRQ_EUNSUPPORTED (-2) /* valid but outside this build's support    */
#define SRQ_ELAUNCH (-3)     /* the HIP launch itself failed              */

/* Thread-local message describing the last error returned on this thread. */
const char *srq_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int srq_abi_version(void);

/* ------------------------------------------------------------------ quant */

/* Per-row symmetric int4 quantization with nibble packing.
 * x f16 [rows, cols] -> q u8 [rows, ceil(cols/2)], scale f16 [rows].
 * scale = fp16(max|x| / 7) (then fp16(scale * clip_ratio) if clip != 1);
 * q = clamp(rne(fp16(x / scale)), -8, 7).
 * Replaces _CUDA.sym_quant_dynamic (signrot/kernels/bindings.cpp:316-335,
 * fused.cu:68-138). */
int srq_sym_quant_dynamic(const void *x, int64_t rows, int64_t cols,
                          float clip_ratio, void *q, void *scale, void *stream);

/* srq_sym_quant_dynamic of gathered rows: output row r (of rows) quantizes
 * row src_row[r] of x f16 [x_rows, cols] (an index outside [0, x_rows)
 * gives scale 0 and zero codes).  cols % 8 == 0, cols <= 32768, x 16-byte
 * aligned.  Bit-identical to srq_sym_quant_dynamic followed by a row gather
 * of its outputs.  Replaces the quantizer + the `x[token]` gather of the
 * MoE block's expert-sorted rows (signrot/nn/moe.py:186-190). */
int srq_sym_quant_dynamic_rows(const void *x, int64_t x_rows, const int32_t *src_row,
                               int64_t rows, int64_t cols, float clip_ratio, void *q, void *scale,
                               void *stream);

/* Symmetric int4 quantization with a given per-row fp16 scale.
 * Replaces _CUDA.sym_quant (bindings.cpp:208-225, quant.cu:13-62). */
int srq_sym_quant(const void *x, const void *scale, int64_t rows, int64_t cols,
                  void *q, void *stream);

/* out f16 [rows, cols] = fp16((float(q) * float(scale_row)) * float(scale_col)).
 * Replaces _CUDA.sym_dequant (bindings.cpp:228-268, quant.cu:66-131). */
int srq_sym_dequant(const int32_t *q, const void *scale_row, const void *scale_col,
                    int64_t rows, int64_t cols, void *out, void *stream);

/* KV-cache asymmetric uint4 quantize + pack over rows of `cols` (even).
 * x f16 [rows, cols] -> q u8 [rows, cols/2], param f16 [rows, 2] = [scale, zero].
 * Replaces _CUDA.kv_quant_pack (bindings.cpp:359-381, fused.cu:213-273). */
int srq_kv_quant_pack(const void *x, int64_t rows, int64_t cols,
                      void *q, void *param, void *stream);

/* ------------------------------------------------------------------- GEMM */

/* C i32 [M, N] = A · Bᵀ over packed int4 A u8 [M, K/2], B u8 [N, K/2].
 * K % 32 == 0, K < 131072 (int32 accumulator bound); A, B 16-byte aligned.
 * Replaces _CUDA.matmul (bindings.cpp:13-29, gemm.cu:7-45). */
int srq_matmul_s4s4(const void *A, const void *B, int64_t M, int64_t N, int64_t K,
                    int32_t *C, void *stream);

/* Fused W4A4 linear: out f16 [M, N] =
 *   fp16((float(A·Bᵀ) * float(a_scale[m])) * float(b_scale[n]))
 * then, if bias != NULL, fp16(out + bias[n]).  Bit-identical to
 * srq_matmul_s4s4 followed by srq_sym_dequant (and the fp16 bias add).
 * Replaces the matmul_si4_si4 + sym_dequant (+ bias) pair of
 * Linear4bit.forward (signrot/nn/linear.py:30-50). */
int srq_w4a4_linear(const void *A, const void *a_scale, const void *B,
                    const void *b_scale, const void *bias, int64_t M, int64_t N,
                    int64_t K, void *out, void *stream);

/* Gate/up projection with the SwiGLU in the epilogue: B u8
 * [N, K/2] holds the gate and up weight rows interleaved in blocks of 8
 * (rows 16 c .. 16 c + 7 = gate rows 8 c .., rows 16 c + 8 .. = up rows
 * 8 c ..), b_scale likewise; out f16 [M, N/2] = swiglu(g, u) element-wise
 * with g, u the srq_w4a4_linear outputs of the paired columns (the
 * fused.cu:367-390 SwiGLU, rounded as srq_swiglu).  Bit-identical to
 * srq_w4a4_linear over the gate and up weights followed by srq_swiglu.
 * Any M (every kernel of srq_w4a4_linear's dispatch ends in the SwiGLU row
 * pass; the skinny and split-K forms are not used); N % 16 == 0 and out
 * 16-byte aligned, else SRQ_EINVAL.  Replaces the gate_proj / up_proj
 * Linear4bit pair and the SwiGLU before the down_proj's online Hadamard
 * (e2e/quantized_llama/modeling_llama.py:125-137). */
int srq_w4a4_linear_swiglu(const void *A, const void *a_scale, const void *B,
                           const void *b_scale, int64_t M, int64_t N, int64_t K, void *out,
                           void *stream);

/* Workspace form of srq_w4a4_linear (and of srq_w4a4_linear_residual
 * below, with residual): bit-identical outputs.  For mid-size M (65 ..
 * 1023) whose output tiles are too few to fill the GPU (under 192 of
 * 128 x 128, or 64 or 128 of 256 x 128 with K chunks of at least 4096
 * codes), the product is split over K into int32 partials in `workspace` (device
 * memory, srq_w4a4_linear_ws_bytes(M, N, K) bytes, 0 when the shape is not
 * split) and summed by a second pass before the epilogue; with a smaller
 * workspace the call runs as srq_w4a4_linear.  No counterpart in the
 * reference (whose GEMM takes no workspace); for callers that can hand
 * over scratch memory, such as the PyTorch layer, which takes it from its
 * caching allocator.  Calls sharing one workspace must not overlap. */
int64_t srq_w4a4_linear_ws_bytes(int64_t M, int64_t N, int64_t K);
int srq_w4a4_linear_ws(const void *A, const void *a_scale, const void *B,
                       const void *b_scale, const void *bias, int64_t M, int64_t N,
                       int64_t K, void *out, void *workspace, int64_t ws_bytes,
                       void *stream);
int srq_w4a4_linear_residual_ws(const void *A, const void *a_scale, const void *B,
                                const void *b_scale, const void *bias, const void *residual,
                                int64_t M, int64_t N, int64_t K, void *out, void *workspace,
                                int64_t ws_bytes, void *stream);

/* int4 GEMM with unsigned A: C i32 [M, N] = A · Bᵀ, A u8 [M, K/2] of uint4
 * codes (0..15, the asymmetric activation quantizer's), B u8 [N, K/2] of
 * two's-complement int4; same shape rules as srq_matmul_s4s4.
 * Replaces _CUDA.matmul_ui4_si4 (signrot/kernels/bindings.cpp:31-47,
 * gemm.cu:47-85). */
int srq_matmul_u4s4(const void *A, const void *B, int64_t M, int64_t N, int64_t K,
                    int32_t *C, void *stream);

/* Fused W4A4 linear for asymmetric activations: v = A · Bᵀ (A uint4 codes)
 * - a_zero[m] * b_sum[n] in int32 (wrapping), then out f16 [M, N] =
 * fp16((float(v) * float(a_scale[m])) * float(b_scale[n])), then (bias !=
 * NULL) fp16(out + bias[n]).  a_zero int8 [M] (the quantizer's zero point
 * cast to int8), b_sum int32 [N] (srq_sum_i4 of B's rows).  Bit-identical to
 * srq_matmul_u4s4, srq_matmul_colrow_i8_i32, the int32 subtraction and
 * srq_sym_dequant (+ bias).  Replaces the zeros_x branch of
 * Linear4bit.forward (signrot/nn/linear.py:35-50). */
int srq_w4a4_linear_asym(const void *A, const void *a_scale, const int8_t *a_zero,
                         const void *B, const void *b_scale, const int32_t *b_sum,
                         const void *bias, int64_t M, int64_t N, int64_t K, void *out,
                         void *stream);

/* srq_w4a4_linear with the decoder's residual add fused into the epilogue:
 * out = fp16(lin + residual[m, n]) after the dequant (and bias), as torch's
 * fp16 `residual + linear(x)` rounds it.  residual f16 [M, N]; out may be the
 * residual buffer itself (each element is read before it is written by the
 * same thread).  Replaces Linear4bit.forward followed by the residual add of
 * the decoder layer (e2e/quantized_llama/modeling_llama.py:19-137, HF
 * LlamaDecoderLayer residual structure). */
int srq_w4a4_linear_residual(const void *A, const void *a_scale, const void *B,
                             const void *b_scale, const void *bias, const void *residual,
                             int64_t M, int64_t N, int64_t K, void *out, void *stream);

/* ------------------------------------------------------------ bf6 GEMM
 * The same int4 x int4 products on gfx950's 6-bit-operand MFMA
 * (v_mfma_scale_f32_32x32x64_f8f6f4, e3m2 operands), twice the int8 MFMA
 * rate and bit-identical: every int4 code is an exact e3m2 value and the fp32
 * accumulator holds the integer sums exactly (|sum| <= 64 K < 2^24).
 * Operands are in the bf6 block layout: for an R x K code matrix (K % 128
 * == 0, rows padded to a multiple of 32 with zero codes), 32 x 128 blocks of
 * 3072 bytes, block (rb, kb) at byte (rb * K / 128 + kb) * 3072; for MFMA
 * k-slice q (0, 1), lane l = r + 32 h of a block carries codes
 * 128 kb + 64 q + 32 h + j (j < 32) of row 32 rb + r as e3m2 bit fields j
 * (bits 6 j .. 6 j + 5) of 192 bits, bytes 0-15 at 1024 q + 16 l and bytes
 * 16-23 at 2048 + 16 l + 8 q.  No reference counterpart: an
 * execution layout for the products of srq_matmul_s4s4 / srq_w4a4_linear
 * (signrot/kernels/gemm.cu:7-45, quant.cu:84-87), e.g. for a weight
 * converted once at load. */

/* Bytes of the bf6 block layout of a [rows, K] code matrix, or -1 if
 * K % 128 != 0 or a size is negative. */
int64_t srq_bf6_bytes(int64_t rows, int64_t K);

/* Packed int4 rows (the reference's layout) src u8 [rows, K/2] -> dst in the
 * bf6 block layout (srq_bf6_bytes(rows, K) bytes).  K % 128 == 0; src and dst
 * 16-byte aligned. */
int srq_i4_to_bf6(const void *src, int64_t rows, int64_t K, void *dst, void *stream);

/* C int32 [M, N] = A @ B^T from bf6-layout A6 (M rows) and B6 (N rows);
 * equal to srq_matmul_s4s4 on the int4 operands.  K % 128 == 0, K < 131072. */
int srq_matmul_bf6(const void *A6, const void *B6, int64_t M, int64_t N, int64_t K,
                   int32_t *C, void *stream);

/* srq_w4a4_linear from bf6-layout operands: out f16 [M, N] =
 * fp16((float(C) * a_scale[m]) * b_scale[n]) (+ bias[n]), bit-identical. */
int srq_w4a4_linear_bf6(const void *A6, const void *a_scale, const void *B6,
                        const void *b_scale, const void *bias, int64_t M, int64_t N,
                        int64_t K, void *out, void *stream);

/* --------------------------------------------------------------- Hadamard */

/* Walsh-Hadamard transform (Sylvester order) over the last dim, times scale.
 * x, out [rows, n], n a power of two, 8 <= n <= 32768; dtype 0 = f16, 1 = f32
 * (in and out share the dtype); accumulation in fp32.  out may equal x.
 * Replaces fast_hadamard_transform.hadamard_transform(x, scale) (called at
 * signrot/functional/hadamard.py:81,85; transformers/kv_cache.py:72). */
int srq_hadamard_transform(const void *x, void *out, int64_t rows, int64_t n,
                           float scale, int dtype, void *stream);

/* Online rotation with a Kronecker factor, in the reference's rounding
 * order: view each row as [K, n/K], y = fp16(FWHT_{n/K}(chunk) * s) with
 * s = fp32(1/sqrt(n)), out = fp16(hadK · y); then, if sign != NULL,
 * out *= sign (int8 ±1, exact).  With fp32_had != 0 the two intermediate
 * fp16 roundings are skipped and the result is rounded once
 * (OnlineHadamard(force_fp32=True)).  hadK: device [K, K] with ±1 entries,
 * f16 (f32 when fp32_had), NULL when K == 1.  x, out f16 [rows, n],
 * n % 8 == 0, n <= 65536 (LDS-resident row).
 * Replaces matmul_hadU_cuda + `x * had_adj_sign` (signrot/functional/
 * hadamard.py:78-87, signrot/nn/hadamard.py:26-42). */
int srq_online_hadamard(const void *x, void *out, int64_t rows, int64_t n, int64_t K,
                        const void *hadK, const int8_t *sign, int fp32_had, void *stream);

/* Fused OnlineHadamard -> (sign) -> Quantizer: the rotation of
 * srq_online_hadamard followed by srq_sym_quant_dynamic on its fp16 result,
 * in one launch; q u8 [rows, n/2], scale f16 [rows].  Bit-identical to the
 * two-step composition.  Replaces Sequential(OnlineHadamard, Quantizer)
 * (e2e/quantized_llama/modeling_llama.py:134-138). */
int srq_had_sign_quant(const void *x, int64_t rows, int64_t n, int64_t K,
                       const void *hadK, const int8_t *sign, int fp32_had,
                       float clip_ratio, void *q, void *scale, void *stream);

/* srq_had_sign_quant writing the codes in the bf6 block layout of
 * srq_i4_to_bf6 (rows of n codes) for srq_w4a4_linear_bf6: q6 u8
 * [srq_bf6_bytes(rows, n)] (the code fields of rows past `rows` in the last
 * 32-row block are left unwritten), scale f16 [rows].  The same codes and
 * scales as srq_had_sign_quant.  Needs the MFMA rotation (K % 4 == 0,
 * n = K * 512 or K * 1024, 9 <= K <= 32), else SRQ_EUNSUPPORTED.  No
 * reference counterpart (an execution layout of OnlineHadamard + Quantizer,
 * signrot/nn/hadamard.py:26-42, nn/quantization.py:11-40). */
int srq_had_sign_quant_bf6(const void *x, int64_t rows, int64_t n, int64_t K,
                           const void *hadK, const int8_t *sign, float clip_ratio,
                           void *q6, void *scale, void *stream);

/* Rotation + sign of srq_had_sign_quant followed by the per-token asymmetric
 * uint4 quantizer of srq_asym_quant_dynamic (row min/max of the rotated,
 * signed fp16 values, scale, zero point, codes): q u8 [rows, n/2], scale
 * and zero f16 [rows].  Bit-identical to srq_online_hadamard followed by
 * srq_asym_quant_dynamic.  Needs K % 4 == 0 and n = K * 512 or K * 1024
 * (9 <= K <= 32), else SRQ_EUNSUPPORTED.  Replaces OnlineHadamard followed
 * by AsymQuantizer (signrot/nn/hadamard.py:26-42, nn/quantization.py:59-67,
 * kernels/fused.cu:143-195); the reference has no fused form. */
int srq_had_sign_asym_quant(const void *x, int64_t rows, int64_t n, int64_t K,
                            const void *hadK, const int8_t *sign, float clip_ratio, void *q,
                            void *scale, void *zero, void *stream);

/* srq_had_sign_quant whose input row is SwiGLU of two strided rows:
 * x[r, i] = fp16(fp16(silu(gate[r*ld + i])) * up[r*ld + i]) (the srq_swiglu
 * arithmetic), then the rotation, sign and quantizer of srq_had_sign_quant.
 * Bit-identical to srq_swiglu followed by srq_had_sign_quant.  gate, up f16
 * with row stride ld >= n (e.g. the two halves of one [rows, 2n] gate/up
 * projection); needs K % 4 == 0 and n = K * 512 (9 <= K <= 32) or n = K *
 * 1024 (9 <= K <= 28), else SRQ_EUNSUPPORTED.
 * Replaces swiglu -> OnlineHadamard -> Quantizer of the decoder MLP
 * (e2e/quantized_llama/modeling_llama.py:125-137; fused.cu:367-390). */
int srq_swiglu_had_sign_quant(const void *gate, const void *up, int64_t ld, int64_t rows,
                              int64_t n, int64_t K, const void *hadK, const int8_t *sign,
                              float clip_ratio, void *q, void *scale, void *stream);

/* srq_swiglu_had_sign_quant for the expert-sorted rows of the MoE down
 * projection: row r's sign is row expert_ids[r] of sign int8 [num_experts, n]
 * (an id outside [0, num_experts) takes sign +1, as srq_sym_quant_dynamic_moe
 * does); sign NULL: no sign.  Bit-identical to srq_swiglu, then the rotation
 * (srq_online_hadamard, no sign), then srq_sym_quant_dynamic_moe.  gate, up
 * f16 with row stride ld >= n; needs n = K * 512 with 9 <= K <= 32, K % 4 ==
 * 0, else SRQ_EUNSUPPORTED.  Replaces swiglu -> matmul_hadU_cuda ->
 * sym_quant_dynamic_moe of SignRotMoEBlock.forward (signrot/nn/moe.py:186-
 * 236, kernels/moe.cu:60-101); the reference has no fused form. */
int srq_swiglu_had_sign_quant_moe(const void *gate, const void *up, int64_t ld, int64_t rows,
                                  int64_t n, int64_t K, const void *hadK, const int8_t *sign,
                                  const int32_t *expert_ids, int64_t num_experts,
                                  float clip_ratio, void *q, void *scale, void *stream);

/* srq_swiglu_had_sign_quant_moe of an input already through the SwiGLU
 * (x f16 [rows, n], e.g. srq_w4a4_linear_moe_swiglu's output): the
 * rotation, the per-expert sign rows and the quantizer in one launch,
 * bit-identical to srq_online_hadamard (no sign) then
 * srq_sym_quant_dynamic_moe.  n = K * 512 or K * 1024 with 9 <= K <= 32,
 * K % 4 == 0, else SRQ_EUNSUPPORTED.  Replaces matmul_hadU_cuda ->
 * sym_quant_dynamic_moe of SignRotMoEBlock.forward (signrot/nn/moe.py:
 * 186-236, kernels/moe.cu:60-101). */
int srq_had_sign_quant_moe(const void *x, int64_t rows, int64_t n, int64_t K, const void *hadK,
                           const int8_t *sign, const int32_t *expert_ids, int64_t num_experts,
                           float clip_ratio, void *q, void *scale, void *stream);

/* ----------------------------------------------------- paged int4 KV cache */
/* Cache layout (signrot/kernels/include/flashinfer/page.cuh:18-112):
 *   kv_data  u8  [pages, num_layers, 2, num_heads, page_size, head_dim/2]
 *   kv_param f16 [pages, num_layers, 2, num_heads, page_size, 2] ([scale, zero])
 * Request b owns pages kv_indices[kv_indptr[b] .. kv_indptr[b+1]) (int32,
 * device); its length is (#pages - 1) * page_size + last_page_offset[b] and
 * already counts the tokens being appended.  head_dim must be 128. */

/* Append one token per request (k, v u8 [batch, num_heads, head_dim/2],
 * k_param, v_param f16 [batch, num_heads, 2]) at position length - 1.
 * Replaces _CUDA.append_kv_i4 (bindings.cpp:606-645, page.cuh:119-164). */
int srq_append_kv_i4(void *kv_data, void *kv_param, const int32_t *kv_indptr,
                     const int32_t *kv_indices, const int32_t *last_page_offset,
                     const void *k, const void *v, const void *k_param, const void *v_param,
                     int64_t batch, int64_t num_layers, int64_t layer_idx, int64_t num_heads,
                     int64_t page_size, int64_t head_dim, void *stream);

/* Prefill: request b's tokens seqlen_indptr[b] .. seqlen_indptr[b+1] of
 * k, v u8 [total_tokens, num_heads, head_dim/2] (and the params) go to the
 * last (seqlen_indptr[b+1] - seqlen_indptr[b]) positions of request b.
 * Replaces _CUDA.init_kv_i4 (bindings.cpp:561-604, page.cuh:166-219). */
int srq_init_kv_i4(void *kv_data, void *kv_param, const int32_t *kv_indptr,
                   const int32_t *kv_indices, const int32_t *last_page_offset, const void *k,
                   const void *v, const void *k_param, const void *v_param,
                   const int32_t *seqlen_indptr, int64_t batch, int64_t total_tokens,
                   int64_t num_layers, int64_t layer_idx, int64_t num_heads, int64_t page_size,
                   int64_t head_dim, void *stream);

/* Single-query decode attention over the int4 cache of one layer:
 * o, q f16 [batch, num_qo_heads, 128]; query head h reads KV head
 * h / (num_qo_heads / num_kv_heads) (1 to 8 query heads per KV head; the
 * reference's kernel is the ratio-1 case).  k̂ = float(c) * scale - zero,
 * logits q·k̂ / sqrt(128), softmax, o = Σ p v̂ / Σ p.  With tmp != NULL and
 * num_chunks > 1 each request is split into num_chunks slices whose partial
 * states (tmp f32 [batch, num_qo_heads, num_chunks, 132]) are merged by a
 * second kernel; o may then be NULL, which leaves the partial states in tmp
 * unmerged (for srq_merge_head_had_quant).  Replaces _CUDA.batch_decode_i4
 * (bindings.cpp:508-559, flashinfer.cu:11-55, decode.cuh:493-751). */
int srq_batch_decode_i4(void *o, const void *q, const void *kv_data, const void *kv_param,
                        const int32_t *kv_indptr, const int32_t *kv_indices,
                        const int32_t *last_page_offset, int64_t batch, int64_t num_qo_heads,
                        int64_t num_kv_heads, int64_t num_layers, int64_t layer_idx,
                        int64_t page_size, int64_t head_dim, float *tmp, int64_t num_chunks,
                        void *stream);

/* srq_batch_decode_i4 with num_chunks split-KV chunks and no workspace
 * argument: the partial states go to a fixed device array of the library
 * (8 MiB per GPU, held until the process ends), so the call allocates
 * nothing.  No counterpart in the reference: for callers that cannot
 * allocate or pass a workspace (code under graph capture, serving loops,
 * hosts that forbid hipMalloc).  Needs batch * num_qo_heads * num_chunks *
 * (head_dim + 4) * 4 <= 8 MiB (else SRQ_EINVAL); the stream must belong to the
 * current device.  Every call on one GPU shares that array, so calls that
 * overlap on one GPU (other streams, other threads) race: serialize them.
 * Same results as srq_batch_decode_i4 with a workspace, bit for bit. */
int srq_batch_decode_i4_noalloc(void *o, const void *q, const void *kv_data,
                                const void *kv_param, const int32_t *kv_indptr,
                                const int32_t *kv_indices, const int32_t *last_page_offset,
                                int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
                                int64_t num_layers, int64_t layer_idx, int64_t page_size,
                                int64_t head_dim, int64_t num_chunks, void *stream);

/* Decode-step q/k/v post-processing in one launch.  qkv f16 [batch,
 * (n_q_heads + 2 n_kv_heads) * head_dim] is the q/k/v projection output of
 * one new token per request (q heads, then k heads, then v heads); cos, sin
 * f16 [cos_batch, head_dim] (cos_batch 1 or batch).  q and k rows get the
 * rotary embedding (srq_rope_qk arithmetic); with rotate != 0 they are then
 * rotated, fp16(FWHT_D(row) * had_scale) (srq_hadamard_transform
 * arithmetic).  q rows go to q_out f16 [batch, n_q_heads, head_dim]; k and v
 * rows are quantized (srq_kv_quant_pack) into the token's cache slot, as
 * srq_append_kv_i4 places it (request b's last position).  head_dim == 128.
 * Bit-identical to rope_qk -> hadamard_transform(k) -> kv_quant_pack(k, v) ->
 * append_kv_i4 -> hadamard_transform(q).  Replaces that chain in the
 * decoder's attention and MultiLayerPagedKVCache4Bit.update / the decode stub
 * (e2e/quantized_llama/modeling_llama.py:62-79; signrot/transformers/
 * kv_cache.py:144-170, 295-415). */
int srq_qkv_rope_had_append(const void *qkv, const void *cos, const void *sin,
                            int64_t cos_batch, int64_t batch, int64_t n_q_heads,
                            int64_t n_kv_heads, int64_t head_dim, float had_scale, int rotate,
                            void *q_out, void *kv_data, void *kv_param,
                            const int32_t *kv_indptr, const int32_t *kv_indices,
                            const int32_t *last_page_offset, int64_t num_layers,
                            int64_t layer_idx, int64_t page_size, void *stream);

/* srq_qkv_rope_had_append followed by srq_batch_decode_i4, in one launch:
 * each decode block (request, KV head, chunk) computes the rotated q rows of
 * its query-head group from qkv and keeps them on chip, and the block whose
 * chunk holds the new token writes that token's k / v codes into the cache
 * and attends over them directly.  Arguments as the two entry points (q
 * comes from qkv, so there is no q_out); with tmp and num_chunks > 1 and
 * o == NULL the partial states stay in tmp for srq_merge_head_had_quant.
 * Cache bytes and o are bit-identical to the two calls.  Replaces the same
 * chain as srq_qkv_rope_had_append plus the decode call of the reference's
 * attention stub (signrot/transformers/kv_cache.py:144-170, 295-415;
 * bindings.cpp:508-559). */
int srq_qkv_decode_i4(void *o, const void *qkv, const void *cos, const void *sin,
                      int64_t cos_batch, float had_scale, int rotate, void *kv_data,
                      void *kv_param, const int32_t *kv_indptr, const int32_t *kv_indices,
                      const int32_t *last_page_offset, int64_t batch, int64_t num_qo_heads,
                      int64_t num_kv_heads, int64_t num_layers, int64_t layer_idx,
                      int64_t page_size, int64_t head_dim, float *tmp, int64_t num_chunks,
                      void *stream);

/* ------------------------------------------------------ decode-layer glue */

/* out f16 [rows, cols] = fp16(x * 1/sqrt(Σ x² / mean_dim + eps)), the sum in
 * fp32 (no gamma: it is folded into the next linear).
 * Replaces _CUDA.rmsnorm (bindings.cpp:423-435, fused.cu:278-309; module
 * signrot/nn/normalization.py:19-30). */
int srq_rmsnorm(const void *x, int64_t rows, int64_t cols, float eps, int64_t mean_dim,
                void *out, void *stream);

/* RMSNorm followed by the per-token symmetric int4 quantizer in one launch:
 * h = srq_rmsnorm(x) (written to out unless out is NULL), then q u8
 * [rows, cols/2], scale f16 [rows] = srq_sym_quant_dynamic(h, clip_ratio).
 * cols % 8 == 0, cols <= 8192.  Bit-identical to the two-step composition.
 * Replaces RMSNorm -> Quantizer at the decoder's q/k/v and gate/up inputs
 * (e2e/quantized_llama/modeling_llama.py; fused.cu:68-138, 278-309). */
int srq_rmsnorm_quant(const void *x, int64_t rows, int64_t cols, float eps, int64_t mean_dim,
                      float clip_ratio, void *out, void *q, void *scale, void *stream);

/* Head-axis Hadamard of the attention output followed by the per-token
 * quantizer (the o_proj input): x f16 [batch, n_heads, head_dim];
 * y[b, h, d] = fp16(FWHT_H(x[b, :, d])[h] * scale) (srq_hadamard_transform
 * arithmetic over the head axis); q u8 [batch, n_heads * head_dim / 2],
 * qscale f16 [batch] = srq_sym_quant_dynamic of row y[b] (element
 * h * head_dim + d).  rot (optional, f16 [batch, n_heads * head_dim])
 * receives y.  n_heads a power of two <= 64, head_dim % 8 == 0, <= 256.
 * Bit-identical to transpose -> hadamard_transform -> transpose ->
 * sym_quant_dynamic.  Replaces that chain before o_proj
 * (e2e/quantized_llama/modeling_llama.py:94, 117). */
int srq_head_had_quant(const void *x, int64_t batch, int64_t n_heads, int64_t head_dim,
                       float scale, float clip_ratio, void *q, void *qscale, void *rot,
                       void *stream);

/* srq_head_had_quant of the attention output that the split-KV partial
 * states tmp (f32 [batch, n_heads, num_chunks, 132], as srq_batch_decode_i4
 * leaves them with o = NULL) merge to: bit-identical to the merge kernel
 * followed by srq_head_had_quant, in one launch.  head_dim must be 128 and
 * n_heads * num_chunks <= 124 (the block's records are staged in 64 KiB of
 * LDS); otherwise SRQ_EINVAL.
 * Replaces the same chain as srq_head_had_quant, with the split-KV merge of
 * the reference's decode (decode.cuh:726-751) folded in. */
int srq_merge_head_had_quant(const float *tmp, int64_t batch, int64_t n_heads, int64_t head_dim,
                             int64_t num_chunks, float scale, float clip_ratio, void *q,
                             void *qscale, void *rot, void *stream);

/* Causal (or full) grouped-query softmax attention over fp16 q
 * [batch, seq_len, n_q_heads, 128] and k, v [batch, seq_len, n_kv_heads, 128]
 * given by element strides per token and per sequence (last two dims dense,
 * so q/k/v may be column slices of a fused projection output); q head h reads
 * kv head h / (n_q_heads / n_kv_heads).  out f16 [batch, seq_len, n_q_heads,
 * 128] dense.  attention_mask int32 [batch, seq_len] or NULL: keys at 0
 * entries are dropped and the output rows at 0 entries are zero (the
 * unpad / varlen / pad round trip of flash-attn).  Logits are
 * q.k * sm_scale for any finite sm_scale (negative or zero included; a
 * non-finite one is SRQ_EINVAL); fp32 softmax, P rounded to fp16 for the PV
 * product.  SRQ_EINVAL also for a launch grid of 2^31 or more query tiles x
 * head groups per sequence (tens of millions of tokens).
 * Replaces the prefill call of transformers' _flash_attention_forward
 * (flash-attn 2) in e2e/quantized_llama/modeling_llama.py:81-90. */
int srq_prefill_attention(const void *q, const void *k, const void *v,
                          const int32_t *attention_mask, int64_t batch, int64_t seq_len,
                          int64_t n_q_heads, int64_t n_kv_heads, int64_t head_dim,
                          int64_t q_tok_stride, int64_t q_seq_stride, int64_t kv_tok_stride,
                          int64_t kv_seq_stride, float sm_scale, int causal, void *out,
                          void *stream);

/* In-place rotary embedding of q f16 [n_seqs, seq_len, n_q_heads, head_dim]
 * and k f16 [n_seqs, seq_len, n_k_heads, head_dim] with cos, sin f16
 * [cos_batch, seq_len, head_dim] (cos_batch 1 or n_seqs); each of the three
 * ops of x * cos + rotate_half(x) * sin rounds to fp16.
 * Replaces _CUDA.rope_qk (bindings.cpp:383-409, fused.cu:316-362). */
int srq_rope_qk(void *q, void *k, const void *cos, const void *sin, int64_t n_seqs,
                int64_t seq_len, int64_t cos_batch, int64_t n_q_heads, int64_t n_k_heads,
                int64_t head_dim, void *stream);

/* out f16 [n] = fp16(fp16(silu(gate)) * up).
 * Replaces _CUDA.swiglu (bindings.cpp:411-421, fused.cu:367-390). */
int srq_swiglu(const void *gate, const void *up, int64_t n, void *out, void *stream);

/* ------------------------------------------------ asymmetric activations */

/* Per-token asymmetric uint4 quantizer: per row of x f16 [rows, cols],
 * hmin/hmax = fp16(min/max) (times clip_ratio, rounded, when clip != 1),
 * scale = fp16(fp16(hmax - hmin) / 15), zero = fp16(rne(fp16(-hmin /
 * scale))), q = clamp(__half2int_rn(fp16(x / scale)) + __half2int_rn(zero),
 * 0, 15); outputs q u8 [rows, ceil(cols/2)] (column 2j in the low nibble),
 * scale f16 [rows], zero f16 [rows].
 * Replaces _CUDA.asym_quant_dynamic (signrot/kernels/bindings.cpp:337-358,
 * fused.cu:143-195). */
int srq_asym_quant_dynamic(const void *x, int64_t rows, int64_t cols, float clip_ratio,
                           void *q, void *scale, void *zero, void *stream);

/* srq_asym_quant_dynamic of expert-sorted rows, row r first multiplied by
 * sign[expert_ids[r]] (int8 [num_experts, cols], exact; NULL: no sign; an id
 * outside [0, num_experts) takes +1).  Replaces _CUDA.asym_quant_dynamic_moe
 * (signrot/kernels/bindings.cpp:134-159, moe.cu:104-152). */
int srq_asym_quant_dynamic_moe(const void *x, const int8_t *sign, const int32_t *expert_ids,
                               int64_t num_experts, int64_t rows, int64_t cols,
                               float clip_ratio, void *q, void *scale, void *zero,
                               void *stream);

/* Asymmetric quantizer with a given per-row scale and zero (f16 [rows]):
 * q = clamp(__half2int_rn(fp16(x / scale)) + __half2int_rn(zero), lo, hi)
 * with [lo, hi] = [0, 15] (is_signed == 0, uint4) or [-8, 7] (two's-
 * complement int4), packed as srq_asym_quant_dynamic.  Replaces
 * _CUDA.asym_quant_f16_ui4 / asym_quant_f16_si4 (signrot/kernels/
 * bindings.cpp:270-312, quant.cu:133-207). */
int srq_asym_quant(const void *x, const void *scale, const void *zero, int64_t rows,
                   int64_t cols, int is_signed, void *q, void *stream);

/* out int32 [rows] = sum over both nibbles of each byte of row r of x u8
 * [rows, packed_cols], sign-extended when is_signed (int32, wrapping).
 * Replaces _CUDA.sum_i4 (signrot/kernels/bindings.cpp:437-451,
 * quant.cu:233-321). */
int srq_sum_i4(const void *x, int64_t rows, int64_t packed_cols, int is_signed, int32_t *out,
               void *stream);

/* out int32 [rows, cols] = int32(a_col[r]) * b_row[c] (wrapping).  Replaces
 * _CUDA.matmul_colrow_i8_i32 (signrot/kernels/bindings.cpp:453-477,
 * quant.cu:341-383). */
int srq_matmul_colrow_i8_i32(const int8_t *a_col, const int32_t *b_row, int64_t rows,
                             int64_t cols, int32_t *out, void *stream);

/* --------------------------------------------------------------- MoE */

/* Grouped int4 x int4 -> int32 GEMM over `problem_count` problems whose
 * descriptors live in device memory (nothing is read on the host, so the call
 * is graph-capturable with data-dependent sizes): problem p has
 * (m, n, k) = problem_sizes[3p .. 3p+2] (int32), A at ptr_A[p] (packed int4,
 * row stride lda[p] codes), B at ptr_B[p] (packed int4 [n, k/2], row stride
 * ldb[p] codes), and writes C_p[i * ldc[p] + j] = sum_k A_p[i,k] B_p[j,k]
 * (int32) at ptr_C[p].  Each k must be a multiple of 32 and < 131072 (not
 * checkable on the host).  signed_a == 0: A holds unsigned asymmetric codes
 * (0..15), as matmul_ui4_si4.  Per element identical to srq_matmul_s4s4
 * (srq_matmul_u4s4) on each problem.
 * Replaces _CUDA.matmul_grouped (signrot/kernels/bindings.cpp:49-91,
 * gemm_grouped.cu:54-107). */
int srq_matmul_grouped(const int32_t *problem_sizes, const int64_t *ptr_A,
                       const int64_t *ptr_B, const int64_t *ptr_C, const int64_t *lda,
                       const int64_t *ldb, const int64_t *ldc, int64_t problem_count,
                       int signed_a, void *stream);

/* Fused grouped W4A4 linear of the MoE block: expert e owns rows
 * expert_offsets[e] .. expert_offsets[e+1] (device int32 [num_experts + 1],
 * non-decreasing, last <= rows) of A u8 [rows, K/2]; B u8 [num_experts, N,
 * K/2]; out f16 [rows, N] = fp16((float(A_e · B_eᵀ) * float(a_scale[row]))
 * * float(b_scale[e, N])).  Rows outside every expert's range are not
 * written.  Bit-identical to srq_matmul_grouped followed by
 * srq_sym_dequant_moe.  Replaces the matmul_grouped + sym_dequant_moe pair
 * of SignRotMoEBlock._gemm_dequant_grouped (signrot/nn/moe.py:126-136). */
int srq_w4a4_linear_moe(const void *A, const void *a_scale, const void *B, const void *b_scale,
                        const int32_t *expert_offsets, int64_t num_experts, int64_t rows,
                        int64_t N, int64_t K, void *out, void *stream);

/* The gate and up projections of the MoE block in one launch: two
 * srq_w4a4_linear_moe calls over the same A rows (expert e's rows
 * expert_offsets[e] .. expert_offsets[e + 1]), B_gate / B_up
 * [num_experts, N, K/2] with scales s_gate / s_up [num_experts, N], into
 * out_gate / out_up [rows, N].  Each output is bit-identical to its
 * srq_w4a4_linear_moe call; the launch interleaves an expert's gate and up
 * tiles so both read its A rows while they are in L2.  Replaces the two
 * _gemm_dequant_grouped calls of SignRotMoEBlock.forward
 * (signrot/nn/moe.py:187-190). */
int srq_w4a4_linear_moe_gate_up(const void *A, const void *a_scale, const void *B_gate,
                                const void *s_gate, const void *B_up, const void *s_up,
                                const int32_t *expert_offsets, int64_t num_experts,
                                int64_t rows, int64_t N, int64_t K, void *out_gate,
                                void *out_up, void *stream);

/* The gate and up projections of the MoE block with the SwiGLU in the
 * epilogue: B [num_experts, N, K/2] holds each expert's gate and up rows
 * interleaved in blocks of 8 (rows 16 c .. 16 c + 7 = gate rows 8 c ..,
 * rows 16 c + 8 .. = up rows 8 c ..), b_scale [num_experts, N] likewise;
 * out f16 [rows, N/2] = swiglu(gate, up) of the paired columns (the
 * srq_swiglu rounding).  Bit-identical to srq_w4a4_linear_moe_gate_up
 * followed by srq_swiglu.  N % 16 == 0; A, B and out 16-byte aligned.
 * Replaces the two _gemm_dequant_grouped calls and the SwiGLU of
 * SignRotMoEBlock.forward (signrot/nn/moe.py:187-192). */
int srq_w4a4_linear_moe_swiglu(const void *A, const void *a_scale, const void *B,
                               const void *b_scale, const int32_t *expert_offsets,
                               int64_t num_experts, int64_t rows, int64_t N, int64_t K,
                               void *out, void *stream);

/* Routing of the MoE block in one launch (signrot/nn/moe.py:168-185 plus
 * the expert sort of 175-180): logits fp16 [tokens, num_experts]
 * (num_experts <= 64, top_k <= 8) -> weights fp16 [tokens, top_k] (fp32
 * softmax, top-k with ties to the lower expert, renormalized when norm,
 * cast to fp16, as torch's softmax / topk / div / to compute them),
 * choice int32 [tokens * top_k] (expert of row t * top_k + j), and the rows
 * stably sorted by expert: order [R] (sorted position -> row), inv [R]
 * (row -> position), expert [R] and token [R] (= order / top_k) per
 * sorted position, counts [num_experts], offsets [num_experts + 1].
 * Replaces the softmax, topk, argsort, index_add_ and cumsum ops there. */
int srq_moe_route(const void *logits, int64_t tokens, int64_t num_experts, int64_t top_k,
                  int norm, void *weights, int32_t *choice, int32_t *order, int32_t *inv,
                  int32_t *expert, int32_t *token, int32_t *counts, int32_t *offsets,
                  void *stream);

/* The MoE block's combine (signrot/nn/moe.py:226-230): out fp16 [tokens,
 * hidden] = sum over j of fp16(y[inv[t * top_k + j]] * weights[t, j]),
 * accumulated in fp32 in order of j and rounded to fp16, y fp16 [tokens *
 * top_k, hidden] in expert order (the un-permute, product and sum of
 * torch's y[inv].view(T, k, H) * w.unsqueeze(-1)).sum(dim=1)).  hidden % 8
 * == 0. */
int srq_moe_combine(const void *y, const int32_t *inv, const void *weights, int64_t tokens,
                    int64_t top_k, int64_t hidden, void *out, void *stream);

/* srq_w4a4_linear_moe for asymmetric activations: A holds uint4 codes, and
 * before the dequant each int32 product becomes v - a_zero[row] *
 * b_sum[e, col] (wrapping), a_zero int8 [rows], b_sum int32 [num_experts, N]
 * (srq_sum_i4 of each expert's weight rows).  Bit-identical to
 * srq_matmul_grouped (signed_a = 0) followed by srq_sym_dequant_moe with
 * zero_row and w_sum.  Replaces that pair in SignRotMoEBlock's asym path
 * (signrot/nn/moe.py:126-134). */
int srq_w4a4_linear_moe_asym(const void *A, const void *a_scale, const int8_t *a_zero,
                             const void *B, const void *b_scale, const int32_t *b_sum,
                             const int32_t *expert_offsets, int64_t num_experts, int64_t rows,
                             int64_t N, int64_t K, void *out, void *stream);

/* Per-row symmetric int4 quantization of expert-sorted rows with the
 * per-expert SignRot sign fused in: row r is multiplied by
 * sign[expert_ids[r]] (int8 ±1 [num_experts, cols], or NULL) and quantized
 * as srq_sym_quant_dynamic.  q u8 [rows, ceil(cols/2)], scale f16 [rows].
 * An expert id outside [0, num_experts) uses sign +1.
 * Replaces _CUDA.sym_quant_dynamic_moe (signrot/kernels/bindings.cpp:108-132,
 * moe.cu:60-101, 181-188). */
int srq_sym_quant_dynamic_moe(const void *x, const int8_t *sign, const int32_t *expert_ids,
                              int64_t num_experts, int64_t rows, int64_t cols, float clip_ratio,
                              void *q, void *scale, void *stream);

/* Expert-indexed dequant: out f16 [rows, cols] = fp16((float(q[r,c] -
 * zero_row[r] * w_sum[e,c]) * float(scale_row[r])) * float(w_scales[e,c])),
 * e = expert_ids[r]; the int32 correction (two's-complement arithmetic) only
 * when zero_row (int8 [rows]) and w_sum (int32 [num_experts, cols]) are both
 * given.  An expert id outside [0, num_experts) reads scale 0.
 * Replaces _CUDA.sym_dequant_moe (signrot/kernels/bindings.cpp:161-206,
 * moe.cu:202-238). */
int srq_sym_dequant_moe(const int32_t *q, const void *scale_row, const void *w_scales,
                        const int32_t *expert_ids, const int8_t *zero_row, const int32_t *w_sum,
                        int64_t num_experts, int64_t rows, int64_t cols, void *out,
                        void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SIGNROT_HIP_H */
