// Asymmetric-activation side of the W4A4 path for gfx950: the per-token
// uint4 quantizer (dynamic, MoE sign rows, or with a given scale and zero),
// the per-row int4 code sums of the weights and the zero-point outer product
// of the reference's Linear4bit zeros_x branch (signrot/nn/linear.py:35-43).
// The unsigned-A GEMM lives in gemm.hip (srq_matmul_u4s4, and the fused
// srq_w4a4_linear_asym with the zero correction in its epilogue).
//
// Quantizer arithmetic (fused.cu:143-195, quant.cu:133-207, moe.cu:104-152):
// per row vmin / vmax exact, then asym_row_params (common.h), then per
// element q = clamp(__half2int_rn(fp16(x / scale)) + __half2int_rn(zero),
// lo, hi) with [lo, hi] = [0, 15] (uint4) or [-8, 7] (int4, given-parameter
// form only).  One 256-thread block per row, two passes over the row.
#include "common.h"

#include <float.h>

namespace {

constexpr int kT = 256;

SRQ_DEV float block_min(float v, float *red) {
    v = wave_min(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fminf(fminf(red[0], red[1]), fminf(red[2], red[3]));
}

SRQ_DEV float block_max(float v, float *red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

struct AsymArgs {
    const f16 *x;
    int64_t rows, cols, cols_dst;  // cols_dst = ceil(cols / 2) bytes per row
    float clip;
    // dynamic form: scale/zero outputs; given form: scale/zero inputs
    f16 *scale;
    f16 *zero;
    int given;
    int lo, hi;                    // code range
    const int8_t *sign;            // MoE: [n_sign_rows, cols] or null
    const int32_t *sign_row;       // MoE: expert id per row
    int64_t n_sign_rows;
    uint8_t *q;
};

__global__ __launch_bounds__(kT) void asym_quant_kernel(AsymArgs a) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const f16 *xr = a.x + row * a.cols;
    // MoE: x times sign[expert_ids[row]] (exact); an id outside the table
    // takes sign +1, as the symmetric MoE quantizer does
    const int8_t *sr = nullptr;
    if (a.sign) {
        const int64_t e = a.sign_row[row];
        if (e >= 0 && e < a.n_sign_rows) sr = a.sign + e * a.cols;
    }
    auto load = [&](int64_t i) {
        const float v = (float)xr[i];
        return (sr && sr[i] < 0) ? -v : v;
    };
    float s, zf;
    if (a.given) {
        s = (float)a.scale[row];
        zf = (float)a.zero[row];
    } else {
        float vmin = FLT_MAX, vmax = -FLT_MAX;
        for (int64_t i = threadIdx.x; i < a.cols; i += kT) {
            const float v = load(i);
            vmin = fminf(vmin, v);
            vmax = fmaxf(vmax, v);
        }
        vmin = block_min(vmin, red);
        vmax = block_max(vmax, red);
        f16 sh, zh;
        asym_row_params(vmin, vmax, a.clip, sh, zh);
        if (threadIdx.x == 0) {
            a.scale[row] = sh;
            a.zero[row] = zh;
        }
        s = (float)sh;
        zf = (float)zh;
    }
    const int zi = h2i_rn(zf);
    uint8_t *qr = a.q + row * a.cols_dst;
    for (int64_t b = threadIdx.x; b < a.cols_dst; b += kT) {
        const int64_t c0 = 2 * b;
        const int lo = asym_code(load(c0), s, zi, a.lo, a.hi);
        const int hi = c0 + 1 < a.cols ? asym_code(load(c0 + 1), s, zi, a.lo, a.hi) : 0;
        qr[b] = (uint8_t)((lo & 0xF) | ((hi & 0xF) << 4));
    }
}

// Sum of every nibble of a packed row (sign-extended when SIGNED), int32
// with wrapping adds (signrot/kernels/quant.cu:233-321).
template <bool SIGNED>
__global__ __launch_bounds__(kT) void sum_i4_kernel(const uint8_t *__restrict__ x,
                                                    int64_t packed_cols,
                                                    int32_t *__restrict__ out) {
    __shared__ int red[4];
    const int64_t row = blockIdx.x;
    const uint8_t *xr = x + row * packed_cols;
    u32 acc = 0;
    for (int64_t i = threadIdx.x; i < packed_cols; i += kT) {
        const int byte = xr[i];
        int lo = byte & 0xF, hi = byte >> 4;
        if (SIGNED) {
            lo = lo >= 8 ? lo - 16 : lo;
            hi = hi >= 8 ? hi - 16 : hi;
        }
        acc += (u32)(lo + hi);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += (u32)__shfl_xor((int)acc, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = (int)acc;
    __syncthreads();
    if (threadIdx.x == 0)
        out[row] = (int)((u32)red[0] + (u32)red[1] + (u32)red[2] + (u32)red[3]);
}

// out[r, c] = int32(a[r]) * b[c], wrapping (quant.cu:341-383).
__global__ __launch_bounds__(kT) void colrow_kernel(const int8_t *__restrict__ a,
                                                    const int32_t *__restrict__ b,
                                                    int64_t rows, int64_t cols,
                                                    int32_t *__restrict__ out) {
    const int64_t total = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * kT + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * kT) {
        const int64_t r = i / cols, c = i - r * cols;
        out[i] = (int)((u32)(int)a[r] * (u32)b[c]);
    }
}

int launch_asym(const AsymArgs &a, hipStream_t st, const char *name) {
    asym_quant_kernel<<<dim3((unsigned)a.rows), dim3(kT), 0, st>>>(a);
    SRQ_LAUNCH_CHECK(name);
    return SRQ_OK;
}

}  // namespace

extern "C" int srq_asym_quant_dynamic(const void *x, int64_t rows, int64_t cols,
                                      float clip_ratio, void *q, void *scale, void *zero,
                                      void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0, "asym_quant_dynamic: negative shape");
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(rows <= 0x7fffffffLL, "asym_quant_dynamic: rows > 2^31-1");
    SRQ_CHECK_ARG(cols > 0, "asym_quant_dynamic: empty rows");
    SRQ_CHECK_ARG(x && q && scale && zero, "asym_quant_dynamic: null pointer");
    AsymArgs a{};
    a.x = (const f16 *)x;
    a.rows = rows;
    a.cols = cols;
    a.cols_dst = (cols + 1) / 2;
    a.clip = clip_ratio;
    a.scale = (f16 *)scale;
    a.zero = (f16 *)zero;
    a.lo = 0;
    a.hi = 15;
    a.q = (uint8_t *)q;
    return launch_asym(a, (hipStream_t)stream, "asym_quant_dynamic");
}

extern "C" int srq_asym_quant_dynamic_moe(const void *x, const int8_t *sign,
                                          const int32_t *expert_ids, int64_t num_experts,
                                          int64_t rows, int64_t cols, float clip_ratio, void *q,
                                          void *scale, void *zero, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0 && num_experts >= 0,
                  "asym_quant_dynamic_moe: negative shape");
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(rows <= 0x7fffffffLL, "asym_quant_dynamic_moe: rows > 2^31-1");
    SRQ_CHECK_ARG(cols > 0, "asym_quant_dynamic_moe: empty rows");
    SRQ_CHECK_ARG(x && q && scale && zero, "asym_quant_dynamic_moe: null pointer");
    SRQ_CHECK_ARG(!sign || expert_ids, "asym_quant_dynamic_moe: sign needs expert_ids");
    AsymArgs a{};
    a.x = (const f16 *)x;
    a.rows = rows;
    a.cols = cols;
    a.cols_dst = (cols + 1) / 2;
    a.clip = clip_ratio;
    a.scale = (f16 *)scale;
    a.zero = (f16 *)zero;
    a.lo = 0;
    a.hi = 15;
    a.sign = sign;
    a.sign_row = expert_ids;
    a.n_sign_rows = num_experts;
    a.q = (uint8_t *)q;
    return launch_asym(a, (hipStream_t)stream, "asym_quant_dynamic_moe");
}

extern "C" int srq_asym_quant(const void *x, const void *scale, const void *zero, int64_t rows,
                              int64_t cols, int is_signed, void *q, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0, "asym_quant: negative shape");
    if (rows == 0 || cols == 0) return SRQ_OK;
    SRQ_CHECK_ARG(rows <= 0x7fffffffLL, "asym_quant: rows > 2^31-1");
    SRQ_CHECK_ARG(x && q && scale && zero, "asym_quant: null pointer");
    AsymArgs a{};
    a.x = (const f16 *)x;
    a.rows = rows;
    a.cols = cols;
    a.cols_dst = (cols + 1) / 2;
    a.scale = (f16 *)scale;
    a.zero = (f16 *)zero;
    a.given = 1;
    a.lo = is_signed ? -8 : 0;
    a.hi = is_signed ? 7 : 15;
    a.q = (uint8_t *)q;
    return launch_asym(a, (hipStream_t)stream, "asym_quant");
}

extern "C" int srq_sum_i4(const void *x, int64_t rows, int64_t packed_cols, int is_signed,
                          int32_t *out, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && packed_cols >= 0, "sum_i4: negative shape");
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(rows <= 0x7fffffffLL, "sum_i4: rows > 2^31-1");
    SRQ_CHECK_ARG(out && (x || packed_cols == 0), "sum_i4: null pointer");
    hipStream_t st = (hipStream_t)stream;
    if (is_signed)
        sum_i4_kernel<true><<<dim3((unsigned)rows), dim3(kT), 0, st>>>(
            (const uint8_t *)x, packed_cols, out);
    else
        sum_i4_kernel<false><<<dim3((unsigned)rows), dim3(kT), 0, st>>>(
            (const uint8_t *)x, packed_cols, out);
    SRQ_LAUNCH_CHECK("sum_i4");
    return SRQ_OK;
}

extern "C" int srq_matmul_colrow_i8_i32(const int8_t *a_col, const int32_t *b_row, int64_t rows,
                                        int64_t cols, int32_t *out, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0, "matmul_colrow_i8_i32: negative shape");
    if (rows == 0 || cols == 0) return SRQ_OK;
    SRQ_CHECK_ARG(a_col && b_row && out, "matmul_colrow_i8_i32: null pointer");
    const int64_t blocks = std::min<int64_t>(srq_cdiv(rows * cols, kT), 4096);
    colrow_kernel<<<dim3((unsigned)blocks), dim3(kT), 0, (hipStream_t)stream>>>(a_col, b_row, rows,
                                                                              cols, out);
    SRQ_LAUNCH_CHECK("matmul_colrow_i8_i32");
    return SRQ_OK;
}
