// Expert-indexed activation quantizer and dequant of the MoE block
// (signrot/kernels/moe.cu:60-101, 202-238), for gfx950.
//
// sym_quant_dynamic_moe: row r of x (expert-sorted rows) is multiplied by
// sign[expert_ids[r]] (int8 ±1, exact: a flip of the fp16 sign bit) and then
// quantized exactly as sym_quant_dynamic: scale = fp16(max|x| / 7) (then
// fp16(scale * clip)), q = clamp(rne(fp16(x / scale)), -8, 7).  The sign
// does not change max|x|, so the scale is that of the unsigned row.
// sym_dequant_moe: out[r, c] = fp16((float(q[r, c] - zero_row[r] *
// w_sum[e, c]) * float(scale_row[r])) * float(w_scales[e, c])), e =
// expert_ids[r], with the int32 correction only when zero_row is given.
//
// The expert ids are device data: the sign and per-expert tables are read
// through buffer resources sized num_experts rows, so an id outside
// [0, num_experts) reads zeros (sign +1, scale 0) instead of faulting.
#include "common.h"

namespace {

// fp16 sign-bit xor masks of 8 values from their 8 int8 signs (bit 7 of
// each byte): pair i (values 2i, 2i + 1) in one 32-bit word
SRQ_DEV void sign_masks8(uint2 sb, u32 (&m)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32 d = (i < 2 ? sb.x : sb.y) >> (16 * (i % 2));
        m[i] = ((d & 0x80u) << 8) | ((d & 0x8000u) << 16);
    }
}

SRQ_DEV v8h flip8(v8h v, uint2 sb) {
    u32 m[4];
    sign_masks8(sb, m);
    union {
        v8h h;
        u32 w[4];
    } u;
    u.h = v;
#pragma unroll
    for (int i = 0; i < 4; ++i) u.w[i] ^= m[i];
    return u.h;
}

SRQ_DEV u32 pack8_code(const v8h &v, float s) {
    u32 w = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) w |= (u32)(sym_code((float)v[i], s) & 0xF) << (4 * i);
    return w;
}

SRQ_DEV f16 moe_row_scale(float amax, float clip) {
    f16 s = f16_rn(amax / 7.f);
    if (clip != 1.f) s = f16_rn((float)s * clip);
    return s;
}

// TPR threads per row, VPT 8-value vectors per thread (cols % 8 == 0).
template <int TPR, int VPT>
__global__ __launch_bounds__(256) void sym_quant_dynamic_moe_kernel(
    const f16 *__restrict__ x, const int8_t *sign, const int32_t *__restrict__ eids,
    int64_t num_experts, int64_t rows, int nvec, float clip, u32 *__restrict__ q,
    f16 *__restrict__ scale_out) {
    constexpr int RPB = 256 / TPR;
    __shared__ float lds[4];
    const int lt = threadIdx.x % TPR;
    const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
    const bool valid = row < rows;
    const v8h *xr = reinterpret_cast<const v8h *>(x) + row * nvec;
    const int64_t cols = (int64_t)nvec * 8;
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(sign, sign ? num_experts * cols : 0);
    const int64_t e = valid ? eids[row] : 0;
    const bool e_ok = e >= 0 && e < num_experts;

    v8h v[VPT];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = lt + i * TPR;
        if (valid && idx < nvec) {
            v[i] = xr[idx];
            if (sign) {
                const uint32_t off = e_ok ? (uint32_t)(e * cols + (int64_t)idx * 8) : 0xFFFFFFF0u;
                const uint2 sb =
                    __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(sr, off, 0, 0));
                v[i] = flip8(v[i], sb);
            }
        } else {
            v[i] = (v8h){0, 0, 0, 0, 0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf((float)v[i][j]));
    }
    if constexpr (TPR <= 64) {
        amax = group_max<TPR>(amax);
    } else {
        amax = wave_max(amax);
        constexpr int WPR = TPR / 64;
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) lds[wave] = amax;
        __syncthreads();
        const int first = (wave / WPR) * WPR;
        float r = lds[first];
#pragma unroll
        for (int i = 1; i < WPR; ++i) r = fmaxf(r, lds[first + i]);
        amax = r;
    }
    const f16 s = moe_row_scale(amax, clip);
    if (!valid) return;
    if (lt == 0) scale_out[row] = s;
    const float sf = (float)s;
    u32 *qr = q + row * nvec;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = lt + i * TPR;
        if (idx < nvec) qr[idx] = pack8_code(v[i], sf);
    }
}

// Any cols: one 256-thread block per row, two passes (the second from cache).
__global__ __launch_bounds__(256) void sym_quant_dynamic_moe_generic_kernel(
    const f16 *__restrict__ x, const int8_t *sign, const int32_t *__restrict__ eids,
    int64_t num_experts, int64_t rows, int64_t cols, float clip, uint8_t *__restrict__ q,
    f16 *__restrict__ scale_out) {
    __shared__ float lds[4];
    const int64_t row = blockIdx.x;
    const f16 *xr = x + row * cols;
    const int64_t e = eids[row];
    const int8_t *srow = (sign && e >= 0 && e < num_experts) ? sign + e * cols : nullptr;
    auto at = [&](int64_t i) {
        f16 v = xr[i];
        if (srow && srow[i] < 0) v = -v;
        return (float)v;
    };
    float amax = 0.f;
    for (int64_t i = threadIdx.x; i < cols; i += 256) amax = fmaxf(amax, fabsf(at(i)));
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(lds[0], lds[1]), fmaxf(lds[2], lds[3]));
    const f16 s = moe_row_scale(amax, clip);
    if (threadIdx.x == 0) scale_out[row] = s;
    const float sf = (float)s;
    const int64_t cdst = (cols + 1) / 2;
    uint8_t *qr = q + row * cdst;
    for (int64_t j = threadIdx.x; j < cdst; j += 256) {
        const int64_t c = 2 * j;
        u32 b = (u32)(sym_code(at(c), sf) & 0xF);
        if (c + 1 < cols) b |= (u32)(sym_code(at(c + 1), sf) & 0xF) << 4;
        qr[j] = (uint8_t)b;
    }
}

template <int TPR, int VPT>
void launch_moe_q(const void *x, const int8_t *sign, const int32_t *eids, int64_t E,
                  int64_t rows, int nvec, float clip, void *q, void *scale, hipStream_t st) {
    constexpr int RPB = 256 / TPR;
    sym_quant_dynamic_moe_kernel<TPR, VPT>
        <<<dim3((unsigned)srq_cdiv(rows, RPB)), dim3(256), 0, st>>>(
            (const f16 *)x, sign, eids, E, rows, nvec, clip, (u32 *)q, (f16 *)scale);
}

template <int TPR>
bool dispatch_moe_q(const void *x, const int8_t *sign, const int32_t *eids, int64_t E,
                    int64_t rows, int nvec, float clip, void *q, void *scale, hipStream_t st) {
    const int vpt = (int)srq_cdiv(nvec, TPR);
    if (vpt <= 1) launch_moe_q<TPR, 1>(x, sign, eids, E, rows, nvec, clip, q, scale, st);
    else if (vpt <= 2) launch_moe_q<TPR, 2>(x, sign, eids, E, rows, nvec, clip, q, scale, st);
    else if (vpt <= 4) launch_moe_q<TPR, 4>(x, sign, eids, E, rows, nvec, clip, q, scale, st);
    else if (vpt <= 8) launch_moe_q<TPR, 8>(x, sign, eids, E, rows, nvec, clip, q, scale, st);
    else return false;
    return true;
}

// ---------------------------------------------------------------- dequant

__global__ __launch_bounds__(256) void sym_dequant_moe_kernel(
    const int32_t *__restrict__ q, const f16 *__restrict__ sr, const f16 *w_scales,
    const int32_t *__restrict__ eids, const int8_t *__restrict__ zero_row,
    const int32_t *w_sum, int64_t num_experts, int64_t rows, int64_t cols,
    f16 *__restrict__ out) {
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(w_scales, num_experts * cols * 2);
    const __amdgpu_buffer_rsrc_t zr = make_rsrc(w_sum, w_sum ? num_experts * cols * 4 : 0);
    const int64_t total = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        const int64_t row = i / cols;
        const int64_t col = i - row * cols;
        const int64_t e = eids[row];
        const bool e_ok = e >= 0 && e < num_experts;
        const uint32_t ecol = e_ok ? (uint32_t)(e * cols + col) : 0x3FFFFFFCu;
        u32 v = (u32)q[i];
        if (zero_row) {
            // exact int32 correction (two's-complement wrap, as the
            // reference's int32 arithmetic)
            const u32 ws = __builtin_amdgcn_raw_buffer_load_b32(zr, ecol * 4, 0, 0);
            v -= (u32)(int32_t)zero_row[row] * ws;
        }
        const f16 wsc = __builtin_bit_cast(
            f16, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(wr, ecol * 2, 0, 0));
        const float a = (float)(int32_t)v * (float)sr[row];
        out[i] = f16_rn(a * (float)wsc);
    }
}

}  // namespace

extern "C" int srq_sym_quant_dynamic_moe(const void *x, const int8_t *sign,
                                         const int32_t *expert_ids, int64_t num_experts,
                                         int64_t rows, int64_t cols, float clip_ratio, void *q,
                                         void *scale, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0 && num_experts >= 0,
                  "sym_quant_dynamic_moe: negative shape");
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(rows <= 0x7fffffffLL, "sym_quant_dynamic_moe: rows > 2^31-1");
    SRQ_CHECK_ARG(x && expert_ids && q && scale, "sym_quant_dynamic_moe: null pointer");
    if (sign && num_experts * cols >= 0xFFFFFFF0LL) {
        srq_set_error("sym_quant_dynamic_moe: sign table larger than 4 GiB");
        return SRQ_EUNSUPPORTED;
    }
    hipStream_t st = (hipStream_t)stream;
    bool done = false;
    if (cols > 0 && cols % 8 == 0 && srq_aligned(x, 16) && srq_aligned(q, 4) &&
        srq_aligned(sign, 8)) {
        const int nvec = (int)(cols / 8);
        if (cols <= 4096)
            done = dispatch_moe_q<64>(x, sign, expert_ids, num_experts, rows, nvec, clip_ratio,
                                      q, scale, st);
        else
            done = dispatch_moe_q<256>(x, sign, expert_ids, num_experts, rows, nvec, clip_ratio,
                                       q, scale, st);
    }
    if (!done) {
        sym_quant_dynamic_moe_generic_kernel<<<dim3((unsigned)rows), dim3(256), 0, st>>>(
            (const f16 *)x, sign, expert_ids, num_experts, rows, cols, clip_ratio,
            (uint8_t *)q, (f16 *)scale);
    }
    SRQ_LAUNCH_CHECK("sym_quant_dynamic_moe");
    return SRQ_OK;
}

extern "C" int srq_sym_dequant_moe(const int32_t *q, const void *scale_row,
                                   const void *w_scales, const int32_t *expert_ids,
                                   const int8_t *zero_row, const int32_t *w_sum,
                                   int64_t num_experts, int64_t rows, int64_t cols, void *out,
                                   void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0 && num_experts >= 0, "sym_dequant_moe: negative shape");
    SRQ_CHECK_ARG((zero_row == nullptr) == (w_sum == nullptr),
                  "sym_dequant_moe: zero_row and w_sum must be given together");
    if (rows == 0 || cols == 0) return SRQ_OK;
    SRQ_CHECK_ARG(q && scale_row && w_scales && expert_ids && out,
                  "sym_dequant_moe: null pointer");
    if (num_experts * cols * 4 >= 0xFFFFFFF0LL) {
        srq_set_error("sym_dequant_moe: per-expert tables larger than 4 GiB");
        return SRQ_EUNSUPPORTED;
    }
    const int64_t blocks = std::min<int64_t>(srq_cdiv(rows * cols, 256), 65536);
    sym_dequant_moe_kernel<<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(
        q, (const f16 *)scale_row, (const f16 *)w_scales, expert_ids, zero_row, w_sum,
        num_experts, rows, cols, (f16 *)out);
    SRQ_LAUNCH_CHECK("sym_dequant_moe");
    return SRQ_OK;
}
