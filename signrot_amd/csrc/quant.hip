// Per-token symmetric int4 activation quantization (+ packing), the given-
// scale quantizer, the int32 -> fp16 dequant and the KV-cache uint4
// quantizer, for gfx950.
//
// Semantics follow the reference kernels bit for bit (signrot/kernels/
// fused.cu:68-138, 213-273; quant.cu:13-131).  The layout work is our own:
// rows are read with 16-byte vector loads held in registers (one pass over
// HBM instead of the reference's two), the row max is a wave64 shuffle
// reduction (plus one LDS hop when a row spans several waves), and eight
// codes are packed into one 32-bit store.
#include "common.h"

#include <stdarg.h>
#include <stdio.h>

static thread_local char g_err[512];

void srq_set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

extern "C" const char *srq_last_error(void) { return g_err; }
extern "C" int srq_abi_version(void) { return 2; }

// Reduce `v` over the TPR threads that share a row.  TPR <= 64 stays inside
// one wave; TPR > 64 adds one LDS hop.  Every thread of the block must call
// this (it contains __syncthreads when TPR > 64).
template <int TPR, int OP>
SRQ_DEV float row_reduce(float v, float *lds) {
    if constexpr (TPR <= 64) {
        return OP == 0 ? group_max<TPR>(v) : (OP == 1 ? group_min<TPR>(v) : group_sum<TPR>(v));
    } else {
        v = OP == 0 ? wave_max(v) : (OP == 1 ? wave_min(v) : wave_sum(v));
        constexpr int WPR = TPR / 64;
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) lds[wave] = v;
        __syncthreads();
        const int first = (wave / WPR) * WPR;
        float r = lds[first];
#pragma unroll
        for (int i = 1; i < WPR; ++i) {
            float o = lds[first + i];
            r = OP == 0 ? fmaxf(r, o) : (OP == 1 ? fminf(r, o) : r + o);
        }
        __syncthreads();
        return r;
    }
}

// --------------------------------------------------------------------------
// sym_quant_dynamic: vector path (cols % 8 == 0, 16-byte aligned rows)

// src_row (optional): output row r quantizes input row src_row[r] of the
// x_rows rows of x; an index outside [0, x_rows) reads as a zero row.
template <int TPR, int VPT>
__global__ __launch_bounds__(256) void sym_quant_dynamic_vec_kernel(
    const f16 *__restrict__ x, int64_t rows, int nvec, float clip,
    u32 *__restrict__ q, f16 *__restrict__ scale_out, const int32_t *__restrict__ src_row,
    int64_t x_rows) {
    constexpr int RPB = 256 / TPR;
    __shared__ float lds[4];
    const int lt = threadIdx.x % TPR;
    const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
    const bool valid = row < rows;
    int64_t srow = row;
    bool live = valid;
    if (src_row && valid) {
        srow = src_row[row];
        live = srow >= 0 && srow < x_rows;
    }
    const v8h *xr = reinterpret_cast<const v8h *>(x) + (live ? srow : 0) * nvec;

    v8h v[VPT];
    float amax = 0.f;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = lt + i * TPR;
        if (live && idx < nvec) {
            v[i] = __builtin_nontemporal_load(xr + idx);
        } else {
            v[i] = (v8h){0, 0, 0, 0, 0, 0, 0, 0};
        }
        amax = absmax8_flag(v[i], amax, bad);
    }
    amax = row_reduce<TPR, 0>(amax, lds);
    // non-finite values take the exact per-element path (row-uniform flag)
    const float badf = row_reduce<TPR, 0>(bad ? 1.f : 0.f, lds);
    const f16 s = sym_row_scale(amax, clip);
    if (!valid) return;
    if (lt == 0) scale_out[row] = s;
    const float sf = (float)s;
    u32 *qr = q + row * nvec;
    if (badf != 0.f) {
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int idx = lt + i * TPR;
            if (idx < nvec) qr[idx] = pack8_sym(v[i], sf);
        }
    } else {
        const float rcp = sym_rcp_safe(sf);
        const bool clampit = sym_row_needs_clamp(amax, sf);
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int idx = lt + i * TPR;
            if (idx < nvec)
                qr[idx] = clampit ? pack8_sym_fast<true>(v[i], rcp) : pack8_sym_fast<false>(v[i], rcp);
        }
    }
}

// Generic path: any cols, any alignment.  One 256-thread block per row, two
// passes over the row (the second one hits cache).
__global__ __launch_bounds__(256) void sym_quant_dynamic_generic_kernel(
    const f16 *__restrict__ x, int64_t rows, int64_t cols, float clip,
    const f16 *__restrict__ given_scale, uint8_t *__restrict__ q,
    f16 *__restrict__ scale_out) {
    __shared__ float lds[4];
    const int64_t row = blockIdx.x;
    const f16 *xr = x + row * cols;
    float sf;
    if (given_scale) {
        sf = (float)given_scale[row];
    } else {
        float amax = 0.f;
        for (int64_t i = threadIdx.x; i < cols; i += 256) amax = fmaxf(amax, fabsf((float)xr[i]));
        amax = row_reduce<256, 0>(amax, lds);
        const f16 s = sym_row_scale(amax, clip);
        if (threadIdx.x == 0) scale_out[row] = s;
        sf = (float)s;
    }
    const int64_t cdst = (cols + 1) / 2;
    uint8_t *qr = q + row * cdst;
    for (int64_t j = threadIdx.x; j < cdst; j += 256) {
        const int64_t c = 2 * j;
        u32 b = (u32)(sym_code((float)xr[c], sf) & 0xF);
        if (c + 1 < cols) b |= (u32)(sym_code((float)xr[c + 1], sf) & 0xF) << 4;
        qr[j] = (uint8_t)b;
    }
}

template <int TPR, int VPT>
static void launch_sqd_vec(const void *x, int64_t rows, int nvec, float clip, void *q,
                           void *scale, hipStream_t st, const int32_t *src_row,
                           int64_t x_rows) {
    constexpr int RPB = 256 / TPR;
    const int64_t blocks = srq_cdiv(rows, RPB);
    sym_quant_dynamic_vec_kernel<TPR, VPT><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
        (const f16 *)x, rows, nvec, clip, (u32 *)q, (f16 *)scale, src_row, x_rows);
}

template <int TPR>
static bool dispatch_sqd_vpt(const void *x, int64_t rows, int nvec, float clip, void *q,
                             void *scale, hipStream_t st, const int32_t *src_row = nullptr,
                             int64_t x_rows = 0) {
    const int vpt = (int)srq_cdiv(nvec, TPR);
    if (vpt <= 1) launch_sqd_vec<TPR, 1>(x, rows, nvec, clip, q, scale, st, src_row, x_rows);
    else if (vpt <= 2) launch_sqd_vec<TPR, 2>(x, rows, nvec, clip, q, scale, st, src_row, x_rows);
    else if (vpt <= 4) launch_sqd_vec<TPR, 4>(x, rows, nvec, clip, q, scale, st, src_row, x_rows);
    else if (vpt <= 8) launch_sqd_vec<TPR, 8>(x, rows, nvec, clip, q, scale, st, src_row, x_rows);
    else if (vpt <= 16) launch_sqd_vec<TPR, 16>(x, rows, nvec, clip, q, scale, st, src_row, x_rows);
    else return false;
    return true;
}

extern "C" int srq_sym_quant_dynamic(const void *x, int64_t rows, int64_t cols,
                                     float clip_ratio, void *q, void *scale, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0, "sym_quant_dynamic: negative shape");
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(rows <= 0x7fffffffLL, "sym_quant_dynamic: rows > 2^31-1");
    SRQ_CHECK_ARG(x && q && scale, "sym_quant_dynamic: null pointer");
    hipStream_t st = (hipStream_t)stream;
    const bool vec_ok = cols > 0 && cols % 8 == 0 && srq_aligned(x, 16) && srq_aligned(q, 4);
    bool done = false;
    if (vec_ok) {
        const int nvec = (int)(cols / 8);
        if (nvec <= 64 * 16 && cols <= 4096)
            done = dispatch_sqd_vpt<64>(x, rows, nvec, clip_ratio, q, scale, st);
        else
            done = dispatch_sqd_vpt<256>(x, rows, nvec, clip_ratio, q, scale, st);
    }
    if (!done) {
        sym_quant_dynamic_generic_kernel<<<dim3((unsigned)rows), dim3(256), 0, st>>>(
            (const f16 *)x, rows, cols, clip_ratio, nullptr, (uint8_t *)q, (f16 *)scale);
    }
    SRQ_LAUNCH_CHECK("sym_quant_dynamic");
    return SRQ_OK;
}

extern "C" int srq_sym_quant_dynamic_rows(const void *x, int64_t x_rows, const int32_t *src_row,
                                          int64_t rows, int64_t cols, float clip_ratio, void *q,
                                          void *scale, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && x_rows >= 0 && cols >= 0, "sym_quant_dynamic_rows: bad shape");
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(rows <= 0x7fffffffLL, "sym_quant_dynamic_rows: rows > 2^31-1");
    SRQ_CHECK_ARG(x && src_row && q && scale, "sym_quant_dynamic_rows: null pointer");
    SRQ_CHECK_ARG(cols > 0 && cols % 8 == 0 && cols <= 8 * 256 * 16,
                  "sym_quant_dynamic_rows: cols=%lld must be a positive multiple of 8 <= 32768",
                  (long long)cols);
    SRQ_CHECK_ARG(srq_aligned(x, 16) && srq_aligned(q, 4),
                  "sym_quant_dynamic_rows: x must be 16-byte and q 4-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    const int nvec = (int)(cols / 8);
    if (nvec <= 64 * 16 && cols <= 4096)
        dispatch_sqd_vpt<64>(x, rows, nvec, clip_ratio, q, scale, st, src_row, x_rows);
    else
        dispatch_sqd_vpt<256>(x, rows, nvec, clip_ratio, q, scale, st, src_row, x_rows);
    SRQ_LAUNCH_CHECK("sym_quant_dynamic_rows");
    return SRQ_OK;
}

// --------------------------------------------------------------------------
// sym_quant with a given per-row scale (vector path: 8 values per thread)

__global__ __launch_bounds__(256) void sym_quant_vec_kernel(
    const f16 *__restrict__ x, const f16 *__restrict__ scale, int64_t rows, int64_t nvec,
    u32 *__restrict__ q) {
    const int64_t total = rows * nvec;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        const int64_t row = i / nvec;
        const v8h v = reinterpret_cast<const v8h *>(x)[i];
        q[i] = pack8_sym(v, (float)scale[row]);
    }
}

extern "C" int srq_sym_quant(const void *x, const void *scale, int64_t rows, int64_t cols,
                             void *q, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0, "sym_quant: negative shape");
    if (rows == 0 || cols == 0) return SRQ_OK;
    SRQ_CHECK_ARG(rows <= 0x7fffffffLL, "sym_quant: rows > 2^31-1");
    SRQ_CHECK_ARG(x && q && scale, "sym_quant: null pointer");
    hipStream_t st = (hipStream_t)stream;
    if (cols % 8 == 0 && srq_aligned(x, 16) && srq_aligned(q, 4)) {
        const int64_t nvec = cols / 8;
        const int64_t blocks = std::min<int64_t>(srq_cdiv(rows * nvec, 256), 65536);
        sym_quant_vec_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
            (const f16 *)x, (const f16 *)scale, rows, nvec, (u32 *)q);
    } else {
        sym_quant_dynamic_generic_kernel<<<dim3((unsigned)rows), dim3(256), 0, st>>>(
            (const f16 *)x, rows, cols, 1.f, (const f16 *)scale, (uint8_t *)q, nullptr);
    }
    SRQ_LAUNCH_CHECK("sym_quant");
    return SRQ_OK;
}

// --------------------------------------------------------------------------
// sym_dequant: out = fp16((float(q) * float(sr)) * float(sc)), 4 per thread

__global__ __launch_bounds__(256) void sym_dequant_vec_kernel(
    const v4i *__restrict__ q, const f16 *__restrict__ sr, const f16 *__restrict__ sc,
    int64_t rows, int64_t ncol4, v4h *__restrict__ out) {
    const int64_t total = rows * ncol4;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        const int64_t row = i / ncol4;
        const int64_t c4 = i - row * ncol4;
        const v4i v = __builtin_nontemporal_load(q + i);
        const float r = (float)sr[row];
        v4h o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float a = (float)v[j] * r;
            o[j] = f16_rn(a * (float)sc[c4 * 4 + j]);
        }
        out[i] = o;
    }
}

__global__ __launch_bounds__(256) void sym_dequant_generic_kernel(
    const int32_t *__restrict__ q, const f16 *__restrict__ sr, const f16 *__restrict__ sc,
    int64_t rows, int64_t cols, f16 *__restrict__ out) {
    const int64_t total = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        const int64_t row = i / cols;
        const int64_t col = i - row * cols;
        const float a = (float)q[i] * (float)sr[row];
        out[i] = f16_rn(a * (float)sc[col]);
    }
}

extern "C" int srq_sym_dequant(const int32_t *q, const void *scale_row, const void *scale_col,
                               int64_t rows, int64_t cols, void *out, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0, "sym_dequant: negative shape");
    if (rows == 0 || cols == 0) return SRQ_OK;
    SRQ_CHECK_ARG(q && scale_row && scale_col && out, "sym_dequant: null pointer");
    hipStream_t st = (hipStream_t)stream;
    if (cols % 4 == 0 && srq_aligned(q, 16) && srq_aligned(out, 8)) {
        const int64_t n4 = cols / 4;
        const int64_t blocks = std::min<int64_t>(srq_cdiv(rows * n4, 256), 65536);
        sym_dequant_vec_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
            (const v4i *)q, (const f16 *)scale_row, (const f16 *)scale_col, rows, n4,
            (v4h *)out);
    } else {
        const int64_t blocks = std::min<int64_t>(srq_cdiv(rows * cols, 256), 65536);
        sym_dequant_generic_kernel<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
            q, (const f16 *)scale_row, (const f16 *)scale_col, rows, cols, (f16 *)out);
    }
    SRQ_LAUNCH_CHECK("sym_dequant");
    return SRQ_OK;
}

// --------------------------------------------------------------------------
// kv_quant_pack: one row (a (token, head) pair, D = cols) per TPR lanes,
// 8 values per lane; param[row] = [scale, zero].

template <int TPR>
__global__ __launch_bounds__(256) void kv_quant_pack_vec_kernel(
    const f16 *__restrict__ x, int64_t rows, int nvec, u32 *__restrict__ q,
    f16 *__restrict__ param) {
    constexpr int RPB = 256 / TPR;
    const int lt = threadIdx.x % TPR;
    const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
    const bool valid = row < rows && lt < nvec;
    v8h v = (v8h){0, 0, 0, 0, 0, 0, 0, 0};
    float vmax = -INFINITY, vmin = INFINITY;
    if (valid) {
        v = reinterpret_cast<const v8h *>(x)[row * nvec + lt];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            vmax = fmaxf(vmax, (float)v[i]);
            vmin = fminf(vmin, (float)v[i]);
        }
    }
    vmax = group_max<TPR>(vmax);
    vmin = group_min<TPR>(vmin);
    if (row >= rows) return;
    f16 scale, zero;
    kv_row_params(vmax, vmin, scale, zero);
    if (lt == 0) {
        param[row * 2 + 0] = scale;
        param[row * 2 + 1] = zero;
    }
    if (!valid) return;
    const float fs = (float)scale, fz = (float)zero;
    u32 w = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) w |= (u32)kv_code((float)v[i], fz, fs) << (4 * i);
    q[row * nvec + lt] = w;
}

__global__ __launch_bounds__(64) void kv_quant_pack_generic_kernel(
    const f16 *__restrict__ x, int64_t rows, int64_t cols, uint8_t *__restrict__ q,
    f16 *__restrict__ param) {
    const int64_t row = blockIdx.x;
    const f16 *xr = x + row * cols;
    float vmax = -INFINITY, vmin = INFINITY;
    for (int64_t i = threadIdx.x; i < cols; i += 64) {
        vmax = fmaxf(vmax, (float)xr[i]);
        vmin = fminf(vmin, (float)xr[i]);
    }
    vmax = wave_max(vmax);
    vmin = wave_min(vmin);
    f16 scale, zero;
    kv_row_params(vmax, vmin, scale, zero);
    if (threadIdx.x == 0) {
        param[row * 2 + 0] = scale;
        param[row * 2 + 1] = zero;
    }
    const float fs = (float)scale, fz = (float)zero;
    const int64_t cdst = cols / 2;
    for (int64_t j = threadIdx.x; j < cdst; j += 64) {
        const u32 b = (u32)kv_code((float)xr[2 * j], fz, fs) |
                      ((u32)kv_code((float)xr[2 * j + 1], fz, fs) << 4);
        q[row * cdst + j] = (uint8_t)b;
    }
}

extern "C" int srq_kv_quant_pack(const void *x, int64_t rows, int64_t cols, void *q,
                                 void *param, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0, "kv_quant_pack: negative shape");
    SRQ_CHECK_ARG(cols % 2 == 0, "kv_quant_pack expects an even last dimension");
    if (rows == 0 || cols == 0) return SRQ_OK;
    SRQ_CHECK_ARG(rows <= 0x7fffffffLL, "kv_quant_pack: rows > 2^31-1");
    SRQ_CHECK_ARG(x && q && param, "kv_quant_pack: null pointer");
    hipStream_t st = (hipStream_t)stream;
    const int64_t nvec = cols / 8;
    if (cols % 8 == 0 && nvec <= 64 && srq_aligned(x, 16) && srq_aligned(q, 4)) {
        int tpr = 1;
        while (tpr < nvec) tpr *= 2;
        const int64_t rpb = 256 / tpr;
        const dim3 grid((unsigned)srq_cdiv(rows, rpb));
        switch (tpr) {
#define SRQ_KV_CASE(T)                                                                 \
    case T:                                                                            \
        kv_quant_pack_vec_kernel<T><<<grid, dim3(256), 0, st>>>(                       \
            (const f16 *)x, rows, (int)nvec, (u32 *)q, (f16 *)param);                  \
        break;
            SRQ_KV_CASE(1)
            SRQ_KV_CASE(2)
            SRQ_KV_CASE(4)
            SRQ_KV_CASE(8)
            SRQ_KV_CASE(16)
            SRQ_KV_CASE(32)
            SRQ_KV_CASE(64)
#undef SRQ_KV_CASE
        }
    } else {
        kv_quant_pack_generic_kernel<<<dim3((unsigned)rows), dim3(64), 0, st>>>(
            (const f16 *)x, rows, cols, (uint8_t *)q, (f16 *)param);
    }
    SRQ_LAUNCH_CHECK("kv_quant_pack");
    return SRQ_OK;
}
