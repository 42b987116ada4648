// Element-wise and row-wise glue of the decode layer for gfx950: RMSNorm
// without gamma (gamma is folded into the next linear offline), in-place
// rotary embedding of q and k, and SwiGLU.
//
// Semantics follow signrot/kernels/fused.cu:278-390:
//   rmsnorm: out = fp16(x * rsqrt(sum(x^2) / mean_dim + eps)), fp32 sum
//   rope_qk: x' = fp16(fp16(x * cos) + fp16(rotate_half(x) * sin)), per op
//            rounding as the three-op torch expression (HF rotate_half)
//   swiglu : out = fp16(fp16(g / (1 + exp(-g))) * up)
#include "common.h"

#include <type_traits>

namespace {

// ------------------------------------------------------------------ RMSNorm
// One row per 64-lane wave (rows <= 8192 values: 16-byte loads, the row in
// registers, one wave reduction), 4 rows per block.  QUANT additionally
// quantizes the normalized fp16 row (per-token symmetric int4, the
// sym_quant_dynamic arithmetic) while it is still in registers; `out` may
// then be null.
template <int VPT, bool QUANT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const f16 *__restrict__ x, int64_t rows,
                                                      int nvec, float eps, float mean_dim,
                                                      f16 *__restrict__ out, float clip,
                                                      u32 *__restrict__ q,
                                                      f16 *__restrict__ qscale) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const v8h *xr = reinterpret_cast<const v8h *>(x) + row * nvec;
    v8h v[VPT];
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = lane + 64 * i;
        v[i] = idx < nvec ? xr[idx] : (v8h){};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float f = (float)v[i][e];
            acc = __builtin_fmaf(f, f, acc);
        }
    }
    acc = wave_sum(acc);
    const float inv = 1.0f / __builtin_sqrtf(acc / mean_dim + eps);
    float amax = 0.f;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = lane + 64 * i;
        v8h o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = f16_rn((float)v[i][e] * inv);
        v[i] = o;
        if (idx < nvec) {
            if (out) reinterpret_cast<v8h *>(out)[row * nvec + idx] = o;
            if (QUANT) amax = absmax8_flag(o, amax, bad);
        }
    }
    if (QUANT) {
        amax = wave_max(amax);
        const f16 s = sym_row_scale(amax, clip);
        if (lane == 0) qscale[row] = s;
        u32 *qr = q + row * nvec;
        if (__builtin_amdgcn_ballot_w64(bad)) {
            // a non-finite value: the exact per-element quantizer
            const float sf = (float)s;
#pragma unroll
            for (int i = 0; i < VPT; ++i)
                if (lane + 64 * i < nvec) qr[lane + 64 * i] = pack8_sym(v[i], sf);
        } else {
            const float rcp = sym_rcp_safe((float)s);
            const bool clampit = sym_row_needs_clamp(amax, (float)s);
#pragma unroll
            for (int i = 0; i < VPT; ++i)
                if (lane + 64 * i < nvec)
                    qr[lane + 64 * i] = clampit ? pack8_sym_fast<true>(v[i], rcp)
                                                : pack8_sym_fast<false>(v[i], rcp);
        }
    }
}

// Block per row for few rows (decode batches): the 256 threads of a block
// share one row (VPT vectors of 8 each), so a row's VALU work is spread over
// four waves instead of one; the sum and the maximum cross the waves through
// LDS.  The maximum (NaN-skipping fmaxf) and the non-finite flag do not
// depend on the order; the fp32 sum does, within the fp16 ulp the RMSNorm
// is specified to.
template <int VPT, bool QUANT>
__global__ __launch_bounds__(256) void rmsnorm_row_kernel(const f16 *__restrict__ x, int nvec,
                                                          float eps, float mean_dim,
                                                          f16 *__restrict__ out, float clip,
                                                          u32 *__restrict__ q,
                                                          f16 *__restrict__ qscale) {
    __shared__ float s_sum[4], s_max[4];
    __shared__ int s_bad[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = blockIdx.x;
    const v8h *xr = reinterpret_cast<const v8h *>(x) + row * nvec;
    v8h v[VPT];
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = tid + 256 * i;
        v[i] = idx < nvec ? xr[idx] : (v8h){};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float f = (float)v[i][e];
            acc = __builtin_fmaf(f, f, acc);
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) s_sum[wave] = acc;
    __syncthreads();
    acc = (s_sum[0] + s_sum[1]) + (s_sum[2] + s_sum[3]);
    const float inv = 1.0f / __builtin_sqrtf(acc / mean_dim + eps);
    float amax = 0.f;
    bool bad = false;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
        const int idx = tid + 256 * i;
        v8h o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = f16_rn((float)v[i][e] * inv);
        v[i] = o;
        if (idx < nvec) {
            if (out) reinterpret_cast<v8h *>(out)[row * nvec + idx] = o;
            if (QUANT) amax = absmax8_flag(o, amax, bad);
        }
    }
    if (QUANT) {
        amax = wave_max(amax);
        const bool wbad = __builtin_amdgcn_ballot_w64(bad) != 0;
        if (lane == 0) {
            s_max[wave] = amax;
            s_bad[wave] = wbad;
        }
        __syncthreads();
        amax = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
        const bool anybad = (s_bad[0] | s_bad[1] | s_bad[2] | s_bad[3]) != 0;
        const f16 s = sym_row_scale(amax, clip);
        if (tid == 0) qscale[row] = s;
        u32 *qr = q + row * nvec;
        if (anybad) {
            // a non-finite value: the exact per-element quantizer
            const float sf = (float)s;
#pragma unroll
            for (int i = 0; i < VPT; ++i)
                if (tid + 256 * i < nvec) qr[tid + 256 * i] = pack8_sym(v[i], sf);
        } else {
            const float rcp = sym_rcp_safe((float)s);
            const bool clampit = sym_row_needs_clamp(amax, (float)s);
#pragma unroll
            for (int i = 0; i < VPT; ++i)
                if (tid + 256 * i < nvec)
                    qr[tid + 256 * i] = clampit ? pack8_sym_fast<true>(v[i], rcp)
                                                : pack8_sym_fast<false>(v[i], rcp);
        }
    }
}

__global__ __launch_bounds__(256) void rmsnorm_generic_kernel(const f16 *__restrict__ x,
                                                              int64_t rows, int64_t cols,
                                                              float eps, float mean_dim,
                                                              f16 *__restrict__ out) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const f16 *xr = x + row * cols;
    float acc = 0.f;
    for (int64_t i = threadIdx.x; i < cols; i += 256) {
        const float f = (float)xr[i];
        acc = __builtin_fmaf(f, f, acc);
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    acc = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / __builtin_sqrtf(acc / mean_dim + eps);
    for (int64_t i = threadIdx.x; i < cols; i += 256)
        out[row * cols + i] = f16_rn((float)xr[i] * inv);
}

// ------------------------------------------------------------------ RoPE
// One thread per rotate_half pair (i, i + D/2) of one (token, head).
__global__ __launch_bounds__(256) void rope_qk_kernel(f16 *__restrict__ q, f16 *__restrict__ k,
                                                      const f16 *__restrict__ cs,
                                                      const f16 *__restrict__ sn, int64_t tokens,
                                                      int64_t seq_len, int cos_batch, int hq,
                                                      int hk, int half) {
    const int64_t total = tokens * (hq + hk) * half;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * 256) {
        const int i = (int)(idx % half);
        const int64_t th = idx / half;
        const int h = (int)(th % (hq + hk));
        const int64_t tok = th / (hq + hk);
        f16 *base = h < hq ? q + (tok * hq + h) * (2 * half) : k + (tok * hk + (h - hq)) * (2 * half);
        const int64_t ct = cos_batch == 1 ? tok % seq_len : tok;
        const f16 *c = cs + ct * (2 * half);
        const f16 *s = sn + ct * (2 * half);
        const f16 x0 = base[i], x1 = base[i + half];
        base[i] = rope_lo(x0, x1, c[i], s[i]);
        base[i + half] = rope_hi(x0, x1, c[i + half], s[i + half]);
    }
}

// ------------------------------------------------------------------ SwiGLU
__global__ __launch_bounds__(256) void swiglu_kernel(const f16 *__restrict__ g,
                                                     const f16 *__restrict__ u, int64_t n,
                                                     f16 *__restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        out[i] = swiglu1((float)g[i], (float)u[i]);
    }
}

}  // namespace

// Rows below which a block shares each row (rmsnorm_row_kernel); above it
// one wave per row.  srq_rmsnorm and srq_rmsnorm_quant choose by the same
// rule, so the fused and the unfused normalization round alike.
constexpr int64_t kRmsRowSplitRows = 256;

template <bool QUANT>
static void launch_rmsnorm_vec(const void *x, int64_t rows, int64_t nvec, float eps,
                               float mean_dim, void *out, float clip, void *q, void *qs,
                               hipStream_t st) {
    if (rows < kRmsRowSplitRows && nvec <= 1024) {
        auto go_row = [&](auto vt) {
            constexpr int V = decltype(vt)::value;
            rmsnorm_row_kernel<V, QUANT><<<dim3((unsigned)rows), 256, 0, st>>>(
                (const f16 *)x, (int)nvec, eps, mean_dim, (f16 *)out, clip, (u32 *)q, (f16 *)qs);
        };
        if (nvec <= 256) go_row(std::integral_constant<int, 1>{});
        else if (nvec <= 512) go_row(std::integral_constant<int, 2>{});
        else go_row(std::integral_constant<int, 4>{});
        return;
    }
    const dim3 grid((unsigned)srq_cdiv(rows, 4));
    const int vpt = (int)srq_cdiv(nvec, 64);
    auto go = [&](auto vt) {
        constexpr int V = decltype(vt)::value;
        rmsnorm_kernel<V, QUANT><<<grid, 256, 0, st>>>((const f16 *)x, rows, (int)nvec, eps,
                                                       mean_dim, (f16 *)out, clip, (u32 *)q,
                                                       (f16 *)qs);
    };
    if (vpt <= 1) go(std::integral_constant<int, 1>{});
    else if (vpt <= 2) go(std::integral_constant<int, 2>{});
    else if (vpt <= 4) go(std::integral_constant<int, 4>{});
    else if (vpt <= 8) go(std::integral_constant<int, 8>{});
    else go(std::integral_constant<int, 16>{});
}

extern "C" int srq_rmsnorm(const void *x, int64_t rows, int64_t cols, float eps, int64_t mean_dim,
                           void *out, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0 && mean_dim > 0, "rmsnorm: bad shape");
    if (rows == 0 || cols == 0) return SRQ_OK;
    SRQ_CHECK_ARG(x && out, "rmsnorm: null pointer");
    hipStream_t st = (hipStream_t)stream;
    const int64_t nvec = cols / 8;
    if (cols % 8 == 0 && nvec <= 64 * 16 && srq_aligned(x, 16) && srq_aligned(out, 16)) {
        launch_rmsnorm_vec<false>(x, rows, nvec, eps, (float)mean_dim, out, 1.f, nullptr,
                                  nullptr, st);
    } else {
        rmsnorm_generic_kernel<<<dim3((unsigned)rows), 256, 0, st>>>(
            (const f16 *)x, rows, cols, eps, (float)mean_dim, (f16 *)out);
    }
    SRQ_LAUNCH_CHECK("rmsnorm");
    return SRQ_OK;
}

extern "C" int srq_rmsnorm_quant(const void *x, int64_t rows, int64_t cols, float eps,
                                 int64_t mean_dim, float clip_ratio, void *out, void *q,
                                 void *scale, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && cols >= 0 && mean_dim > 0, "rmsnorm_quant: bad shape");
    if (rows == 0 || cols == 0) return SRQ_OK;
    SRQ_CHECK_ARG(x && q && scale, "rmsnorm_quant: null pointer");
    SRQ_CHECK_ARG(cols % 8 == 0 && cols <= 8192,
                  "rmsnorm_quant: cols=%lld must be a multiple of 8 and <= 8192",
                  (long long)cols);
    SRQ_CHECK_ARG(srq_aligned(x, 16) && srq_aligned(q, 4) && (!out || srq_aligned(out, 16)),
                  "rmsnorm_quant: x and out must be 16-byte aligned, q 4-byte aligned");
    launch_rmsnorm_vec<true>(x, rows, cols / 8, eps, (float)mean_dim, out, clip_ratio, q, scale,
                             (hipStream_t)stream);
    SRQ_LAUNCH_CHECK("rmsnorm_quant");
    return SRQ_OK;
}

extern "C" int srq_rope_qk(void *q, void *k, const void *cos, const void *sin, int64_t n_seqs,
                           int64_t seq_len, int64_t cos_batch, int64_t n_q_heads,
                           int64_t n_k_heads, int64_t head_dim, void *stream) {
    SRQ_CHECK_ARG(n_seqs >= 0 && seq_len >= 0 && n_q_heads >= 0 && n_k_heads >= 0,
                  "rope_qk: bad shape");
    SRQ_CHECK_ARG(head_dim > 0 && head_dim % 2 == 0, "rope_qk expects an even head_dim");
    SRQ_CHECK_ARG(cos_batch == 1 || cos_batch == n_seqs, "rope_qk: cos/sin batch must be 1 or B");
    const int64_t tokens = n_seqs * seq_len;
    if (tokens == 0 || n_q_heads + n_k_heads == 0) return SRQ_OK;
    SRQ_CHECK_ARG(q && k && cos && sin, "rope_qk: null pointer");
    const int64_t total = tokens * (n_q_heads + n_k_heads) * (head_dim / 2);
    const int64_t blocks = std::min<int64_t>(srq_cdiv(total, 256), 65536);
    rope_qk_kernel<<<dim3((unsigned)blocks), 256, 0, (hipStream_t)stream>>>(
        (f16 *)q, (f16 *)k, (const f16 *)cos, (const f16 *)sin, tokens, seq_len, (int)cos_batch,
        (int)n_q_heads, (int)n_k_heads, (int)(head_dim / 2));
    SRQ_LAUNCH_CHECK("rope_qk");
    return SRQ_OK;
}

extern "C" int srq_swiglu(const void *gate, const void *up, int64_t n, void *out, void *stream) {
    SRQ_CHECK_ARG(n >= 0, "swiglu: bad size");
    if (n == 0) return SRQ_OK;
    SRQ_CHECK_ARG(gate && up && out, "swiglu: null pointer");
    const int64_t blocks = std::min<int64_t>(srq_cdiv(n, 256), 65536);
    swiglu_kernel<<<dim3((unsigned)blocks), 256, 0, (hipStream_t)stream>>>(
        (const f16 *)gate, (const f16 *)up, n, (f16 *)out);
    SRQ_LAUNCH_CHECK("swiglu");
    return SRQ_OK;
}

