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
 * K % 32 == 0, K <= 131072; A, B 16-byte aligned.
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

/* --------------------------------------------------------------- Hadamard */

/* Walsh-Hadamard transform (Sylvester order) over the last dim, times scale.
 * x, out [rows, n], n a power of two, 2 <= n <= 32768; dtype 0 = f16, 1 = f32
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

#ifdef __cplusplus
}
#endif

#endif /* SIGNROT_HIP_H */
