// Online Hadamard rotation for gfx950: Walsh-Hadamard transform of a 2^k
// block (Sylvester order), the Kronecker factor hadK for n = K * 2^k, the
// SignRot ±1 sign, and -- in the fused variant -- the per-token symmetric
// int4 quantizer, all in one pass over HBM.
//
// Reference semantics (signrot/functional/hadamard.py:78-87,
// signrot/nn/hadamard.py:26-42): y = fp16(FWHT_{n/K}(chunk) / sqrt(n)) per
// chunk of the [K, n/K] view, out = fp16(hadK @ y), out *= sign.  With
// fp32_had (OnlineHadamard(force_fp32=True)) both intermediate roundings are
// skipped and the result is rounded to fp16 once at the end.
//
// Design: one block owns whole rows.  The row is staged once in LDS as
// fp32; the FWHT runs as radix-16 passes (16 values per thread in
// registers, 4 butterfly stages per pass, one LDS round trip per pass); the
// first pass reads HBM directly.  The K-mix keeps one column of the [K, n/K]
// view per thread in registers.  The result leaves LDS with coalesced
// vector stores (fp16 out) or goes straight into the quantizer (fused).
#include "common.h"

#include <type_traits>

#include <math.h>

namespace {

constexpr int kThreads = 256;

struct RotArgs {
    const void *x;
    void *out;          // rotation output (mode 0)
    int64_t rows;
    int n;              // row length
    int m;              // FWHT size = n / K
    int K;              // Kronecker factor (1 = none)
    const void *hadK;   // [K, K] f16 (or f32 when fp32_had)
    const int8_t *sign; // [n] or null
    float scale;        // fp32(1/sqrt(n)) or the caller's scale
    int io_f32;         // input/output are fp32 (hadamard_transform dtype 1)
    int fp32_had;       // keep fp32 between the two rotation stages
    float clip;         // quant mode
    uint32_t *q;        // quant mode: packed codes [rows, n/2] as u32 words
    f16 *qscale;        // quant mode: [rows]
    int rpb;            // rows per block
};

// One radix-R pass over `total` LDS floats: butterflies on the index bits
// [log2(s), log2(s) + log2(R)).  Group g covers base + j*s, j < R.
template <int R>
SRQ_DEV void fwht_pass_lds(float *buf, int total, int s_log2) {
    const int s = 1 << s_log2;
    const int groups = total / R;
    for (int g = threadIdx.x; g < groups; g += kThreads) {
        const int lo = g & (s - 1);
        const int hi = g >> s_log2;
        const int base = hi * s * R + lo;
        float v[R];
#pragma unroll
        for (int j = 0; j < R; ++j) v[j] = buf[base + j * s];
        fwht_regs<R>(v);
#pragma unroll
        for (int j = 0; j < R; ++j) buf[base + j * s] = v[j];
    }
    __syncthreads();
}

SRQ_DEV void fwht_pass_dispatch(float *buf, int total, int s_log2, int r_log2) {
    switch (r_log2) {
        case 1: fwht_pass_lds<2>(buf, total, s_log2); break;
        case 2: fwht_pass_lds<4>(buf, total, s_log2); break;
        case 3: fwht_pass_lds<8>(buf, total, s_log2); break;
        default: fwht_pass_lds<16>(buf, total, s_log2); break;
    }
}

// Load `rpb` rows (rpb * n values) into LDS as fp32 and run the first
// radix-16 (or smaller) pass on the way.  Each thread takes R consecutive
// values.  Returns the number of index bits already transformed.
template <int R>
SRQ_DEV void load_first_pass(const RotArgs &a, float *buf, int64_t row0, int nrows) {
    const int total = nrows * a.n;
    const int groups = total / R;
    for (int g = threadIdx.x; g < groups; g += kThreads) {
        const int64_t off = row0 * a.n + (int64_t)g * R;
        float v[R];
        if (a.io_f32) {
            const float *src = reinterpret_cast<const float *>(a.x) + off;
#pragma unroll
            for (int j = 0; j < R; ++j) v[j] = src[j];
        } else {
            const f16 *src = reinterpret_cast<const f16 *>(a.x) + off;
            if constexpr (R >= 8) {
#pragma unroll
                for (int j = 0; j < R; j += 8) {
                    const v8h h = *reinterpret_cast<const v8h *>(src + j);
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[j + i] = (float)h[i];
                }
            } else {
#pragma unroll
                for (int j = 0; j < R; ++j) v[j] = (float)src[j];
            }
        }
        fwht_regs<R>(v);
#pragma unroll
        for (int j = 0; j < R; ++j) buf[g * R + j] = v[j];
    }
    __syncthreads();
}

SRQ_DEV void fwht_rows(const RotArgs &a, float *buf, int64_t row0, int nrows) {
    const int mlog = __builtin_ctz(a.m);
    const int total = nrows * a.n;
    int done;
    if (mlog >= 4) {
        load_first_pass<16>(a, buf, row0, nrows);
        done = 4;
    } else if (mlog == 3) {
        load_first_pass<8>(a, buf, row0, nrows);
        done = 3;
    } else if (mlog == 2) {
        load_first_pass<4>(a, buf, row0, nrows);
        done = 2;
    } else {
        load_first_pass<2>(a, buf, row0, nrows);
        done = 1;
    }
    while (done < mlog) {
        const int r = (mlog - done) >= 4 ? 4 : (mlog - done);
        fwht_pass_dispatch(buf, total, done, r);
        done += r;
    }
}

// K-mix with one column of the [K, m] view per thread, K <= KT in registers.
// Applies the first rounding point (y = fp16(fwht * scale)) on load and the
// second (fp16(hadK @ y)) on store, unless fp32_had.
template <int KT>
SRQ_DEV void kmix_regs(const RotArgs &a, float *buf, const float *hk, int nrows) {
    const int cols = nrows * a.m;
    for (int c = threadIdx.x; c < cols; c += kThreads) {
        const int r = c / a.m;
        const int j = c - r * a.m;
        float *rb = buf + r * a.n + j;
        float y[KT];
#pragma unroll
        for (int k = 0; k < KT; ++k) {
            if (k < a.K) {
                const float v = rb[k * a.m] * a.scale;
                y[k] = a.fp32_had ? v : round16(v);
            }
        }
        // all outputs of the column in registers first: the hadK reads then
        // are not ordered behind stores to the row buffer
        float o[KT];
#pragma unroll
        for (int k = 0; k < KT; ++k) {
            if (k >= a.K) continue;
            const float *h = hk + k * a.K;
            float acc = 0.f;
#pragma unroll
            for (int kk = 0; kk < KT; ++kk) {
                if (kk < a.K) acc = __builtin_fmaf(h[kk], y[kk], acc);
            }
            o[k] = a.fp32_had ? acc : round16(acc);
        }
#pragma unroll
        for (int k = 0; k < KT; ++k)
            if (k < a.K) rb[k * a.m] = o[k];
    }
    __syncthreads();
}

// K-mix for K > 64: out-of-place into `dst`, hadK read from global memory.
SRQ_DEV void kmix_generic(const RotArgs &a, const float *src, float *dst, int nrows) {
    const int cols = nrows * a.m;
    for (int c = threadIdx.x; c < cols; c += kThreads) {
        const int r = c / a.m;
        const int j = c - r * a.m;
        const float *sb = src + r * a.n + j;
        float *db = dst + r * a.n + j;
        for (int k = 0; k < a.K; ++k) {
            float acc = 0.f;
            for (int kk = 0; kk < a.K; ++kk) {
                const float h = a.fp32_had
                                    ? reinterpret_cast<const float *>(a.hadK)[k * a.K + kk]
                                    : (float)reinterpret_cast<const f16 *>(a.hadK)[k * a.K + kk];
                float v = sb[kk * a.m] * a.scale;
                if (!a.fp32_had) v = round16(v);
                acc = __builtin_fmaf(h, v, acc);
            }
            db[k * a.m] = a.fp32_had ? acc : round16(acc);
        }
    }
    __syncthreads();
}

// Final value of element i of a row (after the rotation stages).
SRQ_DEV float finish(const RotArgs &a, const float *rb, int i) {
    float v = rb[i];
    if (a.K == 1) {
        v *= a.scale;
        if (!a.fp32_had && !a.io_f32) v = round16(v);
    }
    if (a.sign) v *= (float)a.sign[i];
    return v;
}

// finish() of the 8 elements 8w .. 8w + 7, the signs read as one 8-byte
// group (n % 8 == 0 on the quantizing paths)
SRQ_DEV void finish8(const RotArgs &a, const float *rb, int w, float (&v)[8]) {
    uint2 sg = make_uint2(0x01010101u, 0x01010101u);
    if (a.sign) {
        const int8_t *sp = a.sign + 8 * w;
        if (reinterpret_cast<uintptr_t>(a.sign) % 8 == 0) {
            sg = *reinterpret_cast<const uint2 *>(sp);
        } else {
            sg.x = (uint8_t)sp[0] | (uint8_t)sp[1] << 8 | (uint8_t)sp[2] << 16 | (u32)(uint8_t)sp[3] << 24;
            sg.y = (uint8_t)sp[4] | (uint8_t)sp[5] << 8 | (uint8_t)sp[6] << 16 | (u32)(uint8_t)sp[7] << 24;
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        float x = rb[8 * w + e];
        if (a.K == 1) {
            x *= a.scale;
            if (!a.fp32_had && !a.io_f32) x = round16(x);
        }
        const int8_t sb = (int8_t)((e < 4 ? sg.x : sg.y) >> (8 * (e & 3)));
        x *= (float)sb;
        v[e] = x;
    }
}

template <int MODE>
__global__ __launch_bounds__(kThreads) void rotate_kernel(RotArgs a) {
    extern __shared__ float lds[];
    const int64_t row0 = (int64_t)blockIdx.x * a.rpb;
    const int nrows = (int)((a.rows - row0) < a.rpb ? (a.rows - row0) : a.rpb);
    float *buf = lds;
    float *buf2 = nullptr;
    float *hk = nullptr;
    const int cap = a.rpb * a.n;
    if (a.K > 64) {
        buf2 = lds + cap;
    } else if (a.K > 1) {
        hk = lds + cap;
        for (int i = threadIdx.x; i < a.K * a.K; i += kThreads)
            hk[i] = a.fp32_had ? reinterpret_cast<const float *>(a.hadK)[i]
                               : (float)reinterpret_cast<const f16 *>(a.hadK)[i];
        // made visible by the barrier at the end of the FWHT passes
    }

    fwht_rows(a, buf, row0, nrows);

    if (a.K > 64) {
        kmix_generic(a, buf, buf2, nrows);
        buf = buf2;
    } else if (a.K > 32) {
        kmix_regs<64>(a, buf, hk, nrows);
    } else if (a.K > 1) {
        kmix_regs<32>(a, buf, hk, nrows);
    }

    if constexpr (MODE == 0) {
        const int total = nrows * a.n;
        if (a.io_f32) {
            float *dst = reinterpret_cast<float *>(a.out) + row0 * a.n;
            for (int i = threadIdx.x; i < total; i += kThreads) {
                const int r = i / a.n;
                dst[i] = finish(a, buf + r * a.n, i - r * a.n);
            }
        } else {
            f16 *dst = reinterpret_cast<f16 *>(a.out) + row0 * a.n;
            for (int i = threadIdx.x * 8; i < total; i += kThreads * 8) {
                const int r = i / a.n;
                const float *rb = buf + r * a.n;
                const int c = i - r * a.n;
                v8h o;
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = f16_rn(finish(a, rb, c + e));
                *reinterpret_cast<v8h *>(dst + i) = o;
            }
        }
    } else {
        // Fused quantizer.  n >= 1024: the whole block shares one row; else
        // wave w quantizes row w of the block.
        __shared__ float red[4];
        const int nw = a.n / 8;
        if (a.rpb == 1) {
            float amax = 0.f;
            for (int w = threadIdx.x; w < nw; w += kThreads) {
                float v[8];
                finish8(a, buf, w, v);
#pragma unroll
                for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(round16(v[e])));
            }
            amax = wave_max(amax);
            if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
            __syncthreads();
            amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
            f16 s = f16_rn(amax / 7.f);
            if (a.clip != 1.f) s = f16_rn((float)s * a.clip);
            if (threadIdx.x == 0) a.qscale[row0] = s;
            const float sf = (float)s;
            uint32_t *qr = a.q + row0 * nw;
            const float rs = sym_recip(sf);
            for (int w = threadIdx.x; w < nw; w += kThreads) {
                float v[8];
                finish8(a, buf, w, v);
                uint32_t word = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    word |= (uint32_t)(sym_code_r(round16(v[e]), rs) & 0xF) << (4 * e);
                qr[w] = word;
            }
        } else {
            const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
            if (wave < nrows) {
                const float *rb = buf + wave * a.n;
                float amax = 0.f;
                for (int w = lane; w < nw; w += 64) {
                    float v[8];
                    finish8(a, rb, w, v);
#pragma unroll
                    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(round16(v[e])));
                }
                amax = wave_max(amax);
                f16 s = f16_rn(amax / 7.f);
                if (a.clip != 1.f) s = f16_rn((float)s * a.clip);
                const int64_t row = row0 + wave;
                if (lane == 0) a.qscale[row] = s;
                const float sf = (float)s;
                uint32_t *qr = a.q + row * nw;
                const float rs = sym_recip(sf);
                for (int w = lane; w < nw; w += 64) {
                    float v[8];
                    finish8(a, rb, w, v);
                    uint32_t word = 0;
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        word |= (uint32_t)(sym_code_r(round16(v[e]), rs) & 0xF) << (4 * e);
                    qr[w] = word;
                }
            }
        }
    }
}

bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int launch_rotate(RotArgs a, int mode, hipStream_t st, const char *name) {
    // rows per block: small rows share a block (<= 4, one wave each when
    // quantizing), large rows get a block each
    int rpb = 1;
    if (a.n < 1024) {
        rpb = 1024 / a.n;
        if (rpb > 4) rpb = 4;
    }
    a.rpb = rpb;
    size_t lds = (size_t)rpb * a.n * sizeof(float);
    if (a.K > 64) lds *= 2;
    else if (a.K > 1) lds += (size_t)a.K * a.K * sizeof(float);
    if (lds > 160 * 1024) {
        srq_set_error("%s: row of %d elements (K=%d) needs %zu bytes of LDS (> 160 KiB)",
                      name, a.n, a.K, lds);
        return SRQ_EUNSUPPORTED;
    }
    const dim3 grid((unsigned)srq_cdiv(a.rows, rpb));
    const void *fn = mode == 0 ? (const void *)rotate_kernel<0> : (const void *)rotate_kernel<1>;
    if (lds > 64 * 1024) {
        hipError_t err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (err != hipSuccess) {
            srq_set_error("%s: cannot reserve %zu bytes of LDS: %s", name, lds,
                          hipGetErrorString(err));
            return SRQ_ELAUNCH;
        }
    }
    if (mode == 0)
        rotate_kernel<0><<<grid, dim3(kThreads), lds, st>>>(a);
    else
        rotate_kernel<1><<<grid, dim3(kThreads), lds, st>>>(a);
    SRQ_LAUNCH_CHECK(name);
    return SRQ_OK;
}

int check_rotation(const char *name, const void *x, int64_t rows, int64_t n, int64_t K,
                   const void *hadK) {
    SRQ_CHECK_ARG(rows >= 0 && n > 0, "%s: bad shape rows=%lld n=%lld", name, (long long)rows,
                  (long long)n);
    SRQ_CHECK_ARG(rows <= 0x7fffffffLL, "%s: rows > 2^31-1", name);
    SRQ_CHECK_ARG(K >= 1 && n % K == 0 && is_pow2(n / K),
                  "%s: n=%lld is not K=%lld times a power of two", name, (long long)n,
                  (long long)K);
    SRQ_CHECK_ARG(n / K >= 2 && n <= 65536, "%s: n=%lld outside [2K, 65536]", name,
                  (long long)n);
    SRQ_CHECK_ARG(n % 8 == 0 || K == 1, "%s: n must be a multiple of 8", name);
    SRQ_CHECK_ARG(K == 1 || hadK != nullptr, "%s: hadK is null with K=%lld", name,
                  (long long)K);
    SRQ_CHECK_ARG(x != nullptr || rows == 0, "%s: null input", name);
    return SRQ_OK;
}

}  // namespace

int srq_had512_mfma(const void *x, int64_t rows, int64_t n, int64_t K, const void *hadK,
                    const int8_t *sign, float clip, void *q, void *qscale, void *out,
                    hipStream_t st, const void *up = nullptr, int64_t ld = 0,
                    const int32_t *sign_row = nullptr, int64_t n_sign_rows = 0,
                    void *qzero = nullptr, int bf6 = 0);

// Rotation + sign + quantizer of rows of n = 256 E (a power of two, K = 1:
// the plain FWHT) for the decode-sized row counts of a q/k/v-shaped
// QLinear: one 256-thread block per row, thread t holding elements
// [E t, E t + E) in registers.  The FWHT stages run in ascending index bit
// as everywhere else, so the fp32 values are those of the LDS kernel:
// bits below log2 E inside the thread, the next 6 bits across the lanes of
// a wave (shuffles), the top 2 bits across the 4 waves (one LDS exchange).
// Then the finish and the quantizer of rotate_kernel (fp16(y * scale) *
// sign, amax, fp16(amax / 7) (* clip), codes), one 4E-byte store per thread.
namespace {

constexpr int kPow2Threads = 256;

// lane i receives lane sel(i)'s value, sel given by the DPP control CTRL
// (all rows and banks, every lane's source in range)
template <int CTRL>
SRQ_DEV float dpp_f32(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

template <int E>
__global__ __launch_bounds__(kPow2Threads) void rot_pow2_quant_kernel(RotArgs a) {
    static_assert(E >= 8 && E <= 32 && (E & (E - 1)) == 0, "E");
    constexpr int n = kPow2Threads * E;
    __shared__ float xch[4][E][64];
    __shared__ float red[4];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // this thread's E signs (the same for every row), loaded once up front
    // so no row waits a memory round trip for them after its transform
    // (the host passes a 16-byte aligned sign vector)
    float sgn[E];
    if (a.sign) {
        const int8_t *sp = a.sign + E * t;
        u32 raw[E / 4];
        if constexpr (E == 8) {
            const uint2 r2 = *reinterpret_cast<const uint2 *>(sp);
            raw[0] = r2.x;
            raw[1] = r2.y;
        } else {
#pragma unroll
            for (int j = 0; j < E / 16; ++j) {
                const uint4 r4 = *reinterpret_cast<const uint4 *>(sp + 16 * j);
                raw[4 * j] = r4.x;
                raw[4 * j + 1] = r4.y;
                raw[4 * j + 2] = r4.z;
                raw[4 * j + 3] = r4.w;
            }
        }
#pragma unroll
        for (int i = 0; i < E; ++i) sgn[i] = (float)(int8_t)(raw[i / 4] >> (8 * (i % 4)));
    }
    for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
        const f16 *xr = reinterpret_cast<const f16 *>(a.x) + row * n + E * t;
        float v[E];
#pragma unroll
        for (int j = 0; j < E; j += 8) {
            const v8h h = *reinterpret_cast<const v8h *>(xr + j);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[j + i] = (float)h[i];
        }
        // bits 0 .. log2 E - 1
#pragma unroll
        for (int h = 1; h < E; h <<= 1)
#pragma unroll
            for (int i = 0; i < E; ++i)
                if ((i & h) == 0) {
                    const float x0 = v[i], x1 = v[i + h];
                    v[i] = x0 + x1;
                    v[i + h] = x0 - x1;
                }
        // the next 6 bits: lane bit s; the lower partner keeps x0 + x1, the
        // upper x0 - x1 (x0 the lower one's value).  The partner's value
        // (lane ^ 2^s) moves by DPP for bits 0, 1 and 3 (quad permutations,
        // a row rotation by 8: no LDS round trip), by ds_bpermute for bits
        // 2, 4 and 5.
        auto stage = [&](auto sb) __attribute__((always_inline)) {
            constexpr int SB = decltype(sb)::value;
            const bool upper = (lane >> SB) & 1;
#pragma unroll
            for (int i = 0; i < E; ++i) {
                float p;
                if constexpr (SB == 0) p = dpp_f32<0xB1>(v[i]);        // quad_perm [1,0,3,2]
                else if constexpr (SB == 1) p = dpp_f32<0x4E>(v[i]);   // quad_perm [2,3,0,1]
                else if constexpr (SB == 3) p = dpp_f32<0x128>(v[i]);  // row_ror:8
                else p = __shfl_xor(v[i], 1 << SB, 64);
                v[i] = upper ? p - v[i] : v[i] + p;
            }
        };
        stage(std::integral_constant<int, 0>{});
        stage(std::integral_constant<int, 1>{});
        stage(std::integral_constant<int, 2>{});
        stage(std::integral_constant<int, 3>{});
        stage(std::integral_constant<int, 4>{});
        stage(std::integral_constant<int, 5>{});
        // the top 2 bits: the 4 waves' values of (lane, i), FWHT_4 in order
#pragma unroll
        for (int i = 0; i < E; ++i) xch[wave][i][lane] = v[i];
        __syncthreads();
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const float x0 = xch[0][i][lane], x1 = xch[1][i][lane];
            const float x2 = xch[2][i][lane], x3 = xch[3][i][lane];
            const float y0 = x0 + x1, y1 = x0 - x1, y2 = x2 + x3, y3 = x2 - x3;
            const float z0 = y0 + y2, z1 = y1 + y3, z2 = y0 - y2, z3 = y1 - y3;
            v[i] = wave == 0 ? z0 : wave == 1 ? z1 : wave == 2 ? z2 : z3;
        }
        // finish: fp16(y * scale), sign; row amax (NaN-ignoring)
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < E; ++i) {
            float x = round16(v[i] * a.scale);
            if (a.sign) x *= sgn[i];
            v[i] = x;
            amax = fmaxf(amax, fabsf(round16(x)));
        }
        amax = wave_max(amax);
        if (lane == 0) red[wave] = amax;
        __syncthreads();
        amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        f16 sc = f16_rn(amax / 7.f);
        if (a.clip != 1.f) sc = f16_rn((float)sc * a.clip);
        if (t == 0) a.qscale[row] = sc;
        const float rs = sym_recip((float)sc);
        u32 w[E / 8];
#pragma unroll
        for (int k = 0; k < E / 8; ++k) {
            w[k] = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e)
                w[k] |= (u32)(sym_code_r(round16(v[8 * k + e]), rs) & 0xF) << (4 * e);
        }
        u32 *qr = a.q + row * (n / 8) + (E / 8) * t;
#pragma unroll
        for (int k = 0; k < E / 8; ++k) qr[k] = w[k];
        __syncthreads();  // xch and red are reused by the next row
    }
}

}  // namespace

extern "C" int srq_hadamard_transform(const void *x, void *out, int64_t rows, int64_t n,
                                      float scale, int dtype, void *stream) {
    SRQ_CHECK_ARG(dtype == 0 || dtype == 1, "hadamard_transform: dtype must be 0 (f16) or 1 (f32)");
    SRQ_CHECK_ARG(is_pow2(n) && n >= 8 && n <= 32768,
                  "hadamard_transform: n=%lld must be a power of two in [8, 32768]", (long long)n);
    int rc = check_rotation("hadamard_transform", x, rows, n, 1, nullptr);
    if (rc) return rc;
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(out != nullptr, "hadamard_transform: null output");
    SRQ_CHECK_ARG(srq_aligned(x, 16) && srq_aligned(out, 16),
                  "hadamard_transform: x and out must be 16-byte aligned");
    RotArgs a{};
    a.x = x;
    a.out = out;
    a.rows = rows;
    a.n = (int)n;
    a.m = (int)n;
    a.K = 1;
    a.scale = scale;
    a.io_f32 = dtype;
    a.fp32_had = dtype;
    return launch_rotate(a, 0, (hipStream_t)stream, "hadamard_transform");
}

extern "C" int srq_online_hadamard(const void *x, void *out, int64_t rows, int64_t n, int64_t K,
                                   const void *hadK, const int8_t *sign, int fp32_had,
                                   void *stream) {
    int rc = check_rotation("online_hadamard", x, rows, n, K, hadK);
    if (rc) return rc;
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(out != nullptr, "online_hadamard: null output");
    SRQ_CHECK_ARG(srq_aligned(x, 16) && srq_aligned(out, 16),
                  "online_hadamard: x and out must be 16-byte aligned");
    SRQ_CHECK_ARG(n % 8 == 0, "online_hadamard: n must be a multiple of 8");
    RotArgs a{};
    a.x = x;
    a.out = out;
    a.rows = rows;
    a.n = (int)n;
    a.K = (int)K;
    a.m = (int)(n / K);
    a.hadK = hadK;
    a.sign = sign;
    a.scale = 1.0f / sqrtf((float)n);
    a.fp32_had = fp32_had ? 1 : 0;
    if (!fp32_had &&
        srq_had512_mfma(x, rows, n, K, hadK, sign, 1.f, nullptr, nullptr, out, (hipStream_t)stream)) {
        SRQ_LAUNCH_CHECK("online_hadamard");
        return SRQ_OK;
    }
    return launch_rotate(a, 0, (hipStream_t)stream, "online_hadamard");
}

extern "C" int srq_had_sign_quant(const void *x, int64_t rows, int64_t n, int64_t K,
                                  const void *hadK, const int8_t *sign, int fp32_had,
                                  float clip_ratio, void *q, void *scale, void *stream) {
    int rc = check_rotation("had_sign_quant", x, rows, n, K, hadK);
    if (rc) return rc;
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(q && scale, "had_sign_quant: null output");
    SRQ_CHECK_ARG(srq_aligned(x, 16) && srq_aligned(q, 4),
                  "had_sign_quant: x must be 16-byte and q 4-byte aligned");
    SRQ_CHECK_ARG(n % 8 == 0, "had_sign_quant: n must be a multiple of 8");
    RotArgs a{};
    a.x = x;
    a.rows = rows;
    a.n = (int)n;
    a.K = (int)K;
    a.m = (int)(n / K);
    a.hadK = hadK;
    a.sign = sign;
    a.scale = 1.0f / sqrtf((float)n);
    a.fp32_had = fp32_had ? 1 : 0;
    a.clip = clip_ratio;
    a.q = (uint32_t *)q;
    a.qscale = (f16 *)scale;
    if (!fp32_had && srq_had512_mfma(x, rows, n, K, hadK, sign, clip_ratio, q, scale, nullptr,
                                     (hipStream_t)stream)) {
        SRQ_LAUNCH_CHECK("had_sign_quant");
        return SRQ_OK;
    }
    if (!fp32_had && K == 1 && (n == 2048 || n == 4096 || n == 8192) &&
        (!sign || srq_aligned(sign, 16))) {
        const dim3 grid((unsigned)std::min<int64_t>(rows, 4096)), block(kPow2Threads);
        if (n == 2048) rot_pow2_quant_kernel<8><<<grid, block, 0, (hipStream_t)stream>>>(a);
        else if (n == 4096) rot_pow2_quant_kernel<16><<<grid, block, 0, (hipStream_t)stream>>>(a);
        else rot_pow2_quant_kernel<32><<<grid, block, 0, (hipStream_t)stream>>>(a);
        SRQ_LAUNCH_CHECK("had_sign_quant");
        return SRQ_OK;
    }
    return launch_rotate(a, 1, (hipStream_t)stream, "had_sign_quant");
}

extern "C" int srq_swiglu_had_sign_quant(const void *gate, const void *up, int64_t ld,
                                         int64_t rows, int64_t n, int64_t K, const void *hadK,
                                         const int8_t *sign, float clip_ratio, void *q,
                                         void *scale, void *stream) {
    int rc = check_rotation("swiglu_had_sign_quant", gate, rows, n, K, hadK);
    if (rc) return rc;
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(up && q && scale, "swiglu_had_sign_quant: null pointer");
    SRQ_CHECK_ARG(ld >= n && ld % 8 == 0, "swiglu_had_sign_quant: ld=%lld must be >= n and a "
                  "multiple of 8", (long long)ld);
    SRQ_CHECK_ARG(srq_aligned(gate, 16) && srq_aligned(up, 16) && srq_aligned(q, 16),
                  "swiglu_had_sign_quant: gate, up and q must be 16-byte aligned");
    if (srq_had512_mfma(gate, rows, n, K, hadK, sign, clip_ratio, q, scale, nullptr,
                        (hipStream_t)stream, up, ld)) {
        SRQ_LAUNCH_CHECK("swiglu_had_sign_quant");
        return SRQ_OK;
    }
    srq_set_error("swiglu_had_sign_quant: needs K %% 4 == 0 and n = K * 512 (9 <= K <= 32) or "
                  "n = K * 1024 (9 <= K <= 28) (n=%lld, K=%lld)", (long long)n, (long long)K);
    return SRQ_EUNSUPPORTED;
}

extern "C" int srq_swiglu_had_sign_quant_moe(const void *gate, const void *up, int64_t ld,
                                             int64_t rows, int64_t n, int64_t K,
                                             const void *hadK, const int8_t *sign,
                                             const int32_t *expert_ids, int64_t num_experts,
                                             float clip_ratio, void *q, void *scale,
                                             void *stream) {
    int rc = check_rotation("swiglu_had_sign_quant_moe", gate, rows, n, K, hadK);
    if (rc) return rc;
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(up && q && scale, "swiglu_had_sign_quant_moe: null pointer");
    SRQ_CHECK_ARG(!sign || (expert_ids && num_experts > 0),
                  "swiglu_had_sign_quant_moe: sign needs expert_ids and num_experts > 0");
    SRQ_CHECK_ARG(ld >= n && ld % 8 == 0, "swiglu_had_sign_quant_moe: ld=%lld must be >= n and "
                  "a multiple of 8", (long long)ld);
    SRQ_CHECK_ARG(srq_aligned(gate, 16) && srq_aligned(up, 16) && srq_aligned(q, 16),
                  "swiglu_had_sign_quant_moe: gate, up and q must be 16-byte aligned");
    if (srq_had512_mfma(gate, rows, n, K, hadK, sign, clip_ratio, q, scale, nullptr,
                        (hipStream_t)stream, up, ld, sign ? expert_ids : nullptr,
                        num_experts)) {
        SRQ_LAUNCH_CHECK("swiglu_had_sign_quant_moe");
        return SRQ_OK;
    }
    srq_set_error("swiglu_had_sign_quant_moe: needs n = K * 512 with 9 <= K <= 32, K %% 4 == 0 "
                  "(n=%lld, K=%lld)", (long long)n, (long long)K);
    return SRQ_EUNSUPPORTED;
}

extern "C" int srq_had_sign_quant_moe(const void *x, int64_t rows, int64_t n, int64_t K,
                                      const void *hadK, const int8_t *sign,
                                      const int32_t *expert_ids, int64_t num_experts,
                                      float clip_ratio, void *q, void *scale, void *stream) {
    int rc = check_rotation("had_sign_quant_moe", x, rows, n, K, hadK);
    if (rc) return rc;
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(q && scale, "had_sign_quant_moe: null pointer");
    SRQ_CHECK_ARG(!sign || (expert_ids && num_experts > 0),
                  "had_sign_quant_moe: sign needs expert_ids and num_experts > 0");
    SRQ_CHECK_ARG(srq_aligned(x, 16) && srq_aligned(q, 16),
                  "had_sign_quant_moe: x and q must be 16-byte aligned");
    if (srq_had512_mfma(x, rows, n, K, hadK, sign, clip_ratio, q, scale, nullptr,
                        (hipStream_t)stream, nullptr, n, sign ? expert_ids : nullptr,
                        num_experts)) {
        SRQ_LAUNCH_CHECK("had_sign_quant_moe");
        return SRQ_OK;
    }
    srq_set_error("had_sign_quant_moe: needs n = K * 512 or K * 1024 with 9 <= K <= 32, "
                  "K %% 4 == 0 (n=%lld, K=%lld)", (long long)n, (long long)K);
    return SRQ_EUNSUPPORTED;
}

extern "C" int srq_had_sign_quant_bf6(const void *x, int64_t rows, int64_t n, int64_t K,
                                      const void *hadK, const int8_t *sign, float clip_ratio,
                                      void *q6, void *scale, void *stream) {
    int rc = check_rotation("had_sign_quant_bf6", x, rows, n, K, hadK);
    if (rc) return rc;
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(q6 && scale, "had_sign_quant_bf6: null output");
    SRQ_CHECK_ARG(srq_aligned(x, 16) && srq_aligned(q6, 16),
                  "had_sign_quant_bf6: x and q6 must be 16-byte aligned");
    if (srq_had512_mfma(x, rows, n, K, hadK, sign, clip_ratio, q6, scale, nullptr,
                        (hipStream_t)stream, nullptr, 0, nullptr, 0, nullptr, 1)) {
        SRQ_LAUNCH_CHECK("had_sign_quant_bf6");
        return SRQ_OK;
    }
    srq_set_error("had_sign_quant_bf6: needs K %% 4 == 0 and n = K * 512 or K * 1024 with "
                  "9 <= K <= 32 (n=%lld, K=%lld)", (long long)n, (long long)K);
    return SRQ_EUNSUPPORTED;
}

extern "C" int srq_had_sign_asym_quant(const void *x, int64_t rows, int64_t n, int64_t K,
                                       const void *hadK, const int8_t *sign, float clip_ratio,
                                       void *q, void *scale, void *zero, void *stream) {
    int rc = check_rotation("had_sign_asym_quant", x, rows, n, K, hadK);
    if (rc) return rc;
    if (rows == 0) return SRQ_OK;
    SRQ_CHECK_ARG(q && scale && zero, "had_sign_asym_quant: null output");
    SRQ_CHECK_ARG(srq_aligned(x, 16) && srq_aligned(q, 16),
                  "had_sign_asym_quant: x and q must be 16-byte aligned");
    if (srq_had512_mfma(x, rows, n, K, hadK, sign, clip_ratio, q, scale, nullptr,
                        (hipStream_t)stream, nullptr, 0, nullptr, 0, zero)) {
        SRQ_LAUNCH_CHECK("had_sign_asym_quant");
        return SRQ_OK;
    }
    srq_set_error("had_sign_asym_quant: needs K %% 4 == 0 and n = K * 512 or K * 1024 with "
                  "9 <= K <= 32 (n=%lld, K=%lld)", (long long)n, (long long)K);
    return SRQ_EUNSUPPORTED;
}
