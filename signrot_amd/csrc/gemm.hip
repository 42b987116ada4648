// int4 x int4 -> int32 GEMM for gfx950 on the int8 MFMA
// (v_mfma_i32_16x16x64_i8), with an optional fused per-token x per-channel
// fp16 dequant epilogue (+ fp16 bias).
//
// C[m, n] = sum_k A[m, k] * B[n, k]; A u8 [M, K/2] and B u8 [N, K/2] are the
// reference's packed int4 layout (signrot/kernels/gemm.cu:7-45: A row-major,
// B "column-major K x N", both K-contiguous).
//
// Unpacking: for a 32-bit word w of eight nibbles,
//   lo(w) = (w << 4) & 0xF0F0F0F0   -> bytes 16 * (low nibbles)
//   hi(w) =  w       & 0xF0F0F0F0   -> bytes 16 * (high nibbles)
// are int8 values equal to 16x the signed codes, with no sign-extension
// work.  The MFMA then accumulates 256 * sum(a*b) exactly (|.| <= 2^14 * K <
// 2^31 for K <= 131072) and the epilogue shifts right by 8.  The lo/hi split
// permutes K inside each 16-element group; A and B go through the same
// permutation, so the integer dot product is unchanged -- bit-exact.
//
// Epilogue (fused): out = fp16((float(acc) * float(sa[m])) * float(sb[n])),
// two separate fp32 multiplies in this order (quant.cu:84-87), then
// fp16(out + bias[n]) as torch's fp16 add (nn/linear.py:47-48).
#include "common.h"

namespace {

SRQ_DEV u32 lo4(u32 w) { return (w << 4) & 0xF0F0F0F0u; }
SRQ_DEV u32 hi4(u32 w) { return w & 0xF0F0F0F0u; }

// 8 packed bytes (16 int4) -> one MFMA operand of 16 int8
SRQ_DEV v4i unpack8(u32 w0, u32 w1) {
    v4i r;
    r[0] = (int)lo4(w0);
    r[1] = (int)hi4(w0);
    r[2] = (int)lo4(w1);
    r[3] = (int)hi4(w1);
    return r;
}

SRQ_DEV v4i mfma16(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

struct Epi {
    int32_t *C;        // int32 output (plain GEMM) or null
    f16 *out;          // fp16 output (fused) or null
    const f16 *sa;     // [M]
    const f16 *sb;     // [N]
    const f16 *bias;   // [N] or null
};

SRQ_DEV void store_one(const Epi &e, int64_t N, int64_t m, int64_t n, int acc256) {
    const int v = acc256 >> 8;
    if (e.C) {
        e.C[m * N + n] = v;
    } else {
        const float a = (float)v * (float)e.sa[m];
        f16 o = f16_rn(a * (float)e.sb[n]);
        if (e.bias) o = f16_rn((float)o + (float)e.bias[n]);
        e.out[m * N + n] = o;
    }
}

// ---------------------------------------------------------------------------
// Tile kernel: BM x BN block per workgroup of 4 waves (2 x 2), each wave
// (BM/2) x (BN/2) made of 16x16 MFMA blocks; BK = 256 int4 (128 bytes) per
// main-loop step.  Global -> registers (prefetch of the next step) ->
// LDS (one buffer, rows padded to 144 bytes so the 16 rows an MFMA fragment
// reads land on distinct banks) -> registers -> MFMA.

constexpr int kBK = 256;             // int4 elements per step
constexpr int kBKB = kBK / 2;        // bytes per row per step
constexpr int kLdsRow = kBKB + 16;   // padded LDS row stride (bytes)

template <int BM, int BN>
__global__ __launch_bounds__(256) void gemm_tile_kernel(const uint8_t *__restrict__ A,
                                                        const uint8_t *__restrict__ B,
                                                        int64_t M, int64_t N, int64_t K,
                                                        Epi e) {
    constexpr int WM = BM / 2, WN = BN / 2;      // per-wave tile
    constexpr int FM = WM / 16, FN = WN / 16;    // MFMA blocks per wave
    constexpr int A_CHUNKS = BM * kBKB / 16 / 256;  // 16-byte chunks per thread
    constexpr int B_CHUNKS = BN * kBKB / 16 / 256;
    __shared__ __attribute__((aligned(16))) uint8_t As[BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint8_t Bs[BN * kLdsRow];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // XCD-aware tile order: consecutive workgroups land on different XCDs
    // (round-robin dispatch), so give each XCD a contiguous range of tiles.
    const int64_t tiles_n = (N + BN - 1) / BN;
    const int64_t tiles = ((M + BM - 1) / BM) * tiles_n;
    int64_t t = blockIdx.x;
    if (tiles % 8 == 0) t = (t % 8) * (tiles / 8) + t / 8;
    const int64_t m0 = (t / tiles_n) * BM;
    const int64_t n0 = (t % tiles_n) * BN;

    const int64_t KB = K / 2;  // bytes per row
    const int steps = (int)((K + kBK - 1) / kBK);

    v4i ra[A_CHUNKS], rb[B_CHUNKS];
    auto gload = [&](int s) {
        const int64_t kb0 = (int64_t)s * kBKB;
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const int c = tid + 256 * i;
            const int r = c / (kBKB / 16), col = (c % (kBKB / 16)) * 16;
            const int64_t gm = m0 + r, gk = kb0 + col;
            if (gm < M && gk < KB)
                ra[i] = *reinterpret_cast<const v4i *>(A + gm * KB + gk);
            else
                ra[i] = (v4i){0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < B_CHUNKS; ++i) {
            const int c = tid + 256 * i;
            const int r = c / (kBKB / 16), col = (c % (kBKB / 16)) * 16;
            const int64_t gn = n0 + r, gk = kb0 + col;
            if (gn < N && gk < KB)
                rb[i] = *reinterpret_cast<const v4i *>(B + gn * KB + gk);
            else
                rb[i] = (v4i){0, 0, 0, 0};
        }
    };
    auto sstore = [&]() {
#pragma unroll
        for (int i = 0; i < A_CHUNKS; ++i) {
            const int c = tid + 256 * i;
            const int r = c / (kBKB / 16), col = (c % (kBKB / 16)) * 16;
            *reinterpret_cast<v4i *>(As + r * kLdsRow + col) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_CHUNKS; ++i) {
            const int c = tid + 256 * i;
            const int r = c / (kBKB / 16), col = (c % (kBKB / 16)) * 16;
            *reinterpret_cast<v4i *>(Bs + r * kLdsRow + col) = rb[i];
        }
    };

    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = (v4i){0, 0, 0, 0};

    const int frow = lane & 15;
    const int fk = (lane >> 4) * 8;  // byte offset of this lane's 16 codes

    gload(0);
    for (int s = 0; s < steps; ++s) {
        __syncthreads();  // previous step's LDS reads are done
        sstore();
        __syncthreads();
        if (s + 1 < steps) gload(s + 1);
#pragma unroll
        for (int kk = 0; kk < kBKB / 32; ++kk) {
            v4i fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const uint8_t *p = As + (wm * WM + i * 16 + frow) * kLdsRow + kk * 32 + fk;
                const uint2 w = *reinterpret_cast<const uint2 *>(p);
                fa[i] = unpack8(w.x, w.y);
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const uint8_t *p = Bs + (wn * WN + j * 16 + frow) * kLdsRow + kk * 32 + fk;
                const uint2 w = *reinterpret_cast<const uint2 *>(p);
                fb[j] = unpack8(w.x, w.y);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = mfma16(fa[i], fb[j], acc[i][j]);
        }
    }

    // 16x16 accumulator layout: lane holds column (lane & 15), rows
    // 4 * (lane >> 4) + r, r = 0..3.
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int64_t gn = n0 + wn * WN + j * 16 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t gm = m0 + wm * WM + i * 16 + 4 * (lane >> 4) + r;
                if (gm < M && gn < N) store_one(e, N, gm, gn, acc[i][j][r]);
            }
        }
}

// ---------------------------------------------------------------------------
// Skinny kernel for small M (decode / short prefill): weight streaming.
// A workgroup of KW waves owns 16 output columns and MB x 16 rows; wave w
// takes the w-th slice of K.  Each lane loads 16 bytes (32 codes) of B per
// 128-code step straight from HBM (no LDS: every byte of B is used by
// exactly one wave), U steps in flight; the slices' int32 partials are
// summed through LDS (exact).

template <int MB, int KW, int U>
__global__ __launch_bounds__(KW * 64) void gemm_skinny_kernel(const uint8_t *__restrict__ A,
                                                             const uint8_t *__restrict__ B,
                                                             int64_t M, int64_t N, int64_t K,
                                                             Epi e) {
    __shared__ v4i part[KW][MB][64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t n0 = (int64_t)blockIdx.x * 16;
    const int64_t m0 = (int64_t)blockIdx.y * (MB * 16);
    const int64_t KB = K / 2;
    const int64_t steps = (K + 127) / 128;            // 64-byte steps per row
    const int64_t per = (steps + KW - 1) / KW;
    const int64_t s0 = wave * per;
    const int64_t s1 = (s0 + per < steps) ? s0 + per : steps;

    const int64_t bn = n0 + (lane & 15);
    const int kb = (lane >> 4) * 16;  // byte offset inside the 64-byte step
    const bool bvalid = bn < N;
    const uint8_t *bp = B + (bvalid ? bn : 0) * KB + kb;
    const uint8_t *ap[MB];
    bool avalid[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int64_t am = m0 + i * 16 + (lane & 15);
        avalid[i] = am < M;
        ap[i] = A + (avalid[i] ? am : 0) * KB + kb;
    }

    v4i acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = (v4i){0, 0, 0, 0};

    for (int64_t s = s0; s < s1; s += U) {
        v4i wb[U], wa[U][MB];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t off = (s + u) * 64;
            const bool ok = (s + u) < s1 && off + kb < KB;
            wb[u] = (ok && bvalid) ? __builtin_nontemporal_load(reinterpret_cast<const v4i *>(bp + off))
                                   : (v4i){0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < MB; ++i)
                wa[u][i] = (ok && avalid[i]) ? *reinterpret_cast<const v4i *>(ap[i] + off)
                                             : (v4i){0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const v4i b0 = unpack8((u32)wb[u][0], (u32)wb[u][1]);
            const v4i b1 = unpack8((u32)wb[u][2], (u32)wb[u][3]);
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const v4i a0 = unpack8((u32)wa[u][i][0], (u32)wa[u][i][1]);
                const v4i a1 = unpack8((u32)wa[u][i][2], (u32)wa[u][i][3]);
                acc[i] = mfma16(a0, b0, acc[i]);
                acc[i] = mfma16(a1, b1, acc[i]);
            }
        }
    }

#pragma unroll
    for (int i = 0; i < MB; ++i) part[wave][i][lane] = acc[i];
    __syncthreads();
    // wave w reduces and stores row block i = w (and w + KW, ...)
    for (int i = wave; i < MB; i += KW) {
        v4i sum = part[0][i][lane];
#pragma unroll
        for (int w = 1; w < KW; ++w) sum += part[w][i][lane];
        const int64_t gn = n0 + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t gm = m0 + i * 16 + 4 * (lane >> 4) + r;
            if (gm < M && gn < N) store_one(e, N, gm, gn, sum[r]);
        }
    }
}

int check_gemm(const char *name, const void *A, const void *B, int64_t M, int64_t N,
               int64_t K) {
    SRQ_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", name);
    SRQ_CHECK_ARG(K % 32 == 0, "%s: K=%lld must be a multiple of 32", name, (long long)K);
    SRQ_CHECK_ARG(K <= 131072, "%s: K=%lld > 131072 (int32 accumulator bound)", name,
                  (long long)K);
    SRQ_CHECK_ARG(M <= 0x7fffffffLL && N <= 0x7fffffffLL, "%s: M or N > 2^31-1", name);
    if (M && N && K) {
        SRQ_CHECK_ARG(A && B, "%s: null operand", name);
        SRQ_CHECK_ARG(srq_aligned(A, 16) && srq_aligned(B, 16),
                      "%s: A and B must be 16-byte aligned", name);
    }
    return SRQ_OK;
}

__global__ void fill_zero_epilogue(int64_t M, int64_t N, Epi e) {
    // K == 0: C = 0; fused output = fp16(0 * sa * sb) (+ bias)
    const int64_t total = M * N;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256)
        store_one(e, N, i / N, i % N, 0);
}

int run_gemm(const char *name, const void *A, const void *B, int64_t M, int64_t N, int64_t K,
             const Epi &e, hipStream_t st) {
    if (M == 0 || N == 0) return SRQ_OK;
    const uint8_t *a = (const uint8_t *)A;
    const uint8_t *b = (const uint8_t *)B;
    if (K == 0) {
        const int64_t blocks = std::min<int64_t>(srq_cdiv(M * N, 256), 4096);
        fill_zero_epilogue<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(M, N, e);
    } else if (M <= 16) {
        gemm_skinny_kernel<1, 8, 4><<<dim3((unsigned)srq_cdiv(N, 16), 1), dim3(512), 0, st>>>(
            a, b, M, N, K, e);
    } else if (M <= 32) {
        gemm_skinny_kernel<2, 8, 4><<<dim3((unsigned)srq_cdiv(N, 16), 1), dim3(512), 0, st>>>(
            a, b, M, N, K, e);
    } else if (M <= 64) {
        gemm_skinny_kernel<4, 8, 2><<<dim3((unsigned)srq_cdiv(N, 16), 1), dim3(512), 0, st>>>(
            a, b, M, N, K, e);
    } else {
        constexpr int BM = 128, BN = 128;
        const int64_t tiles = srq_cdiv(M, BM) * srq_cdiv(N, BN);
        gemm_tile_kernel<BM, BN><<<dim3((unsigned)tiles), dim3(256), 0, st>>>(a, b, M, N, K, e);
    }
    SRQ_LAUNCH_CHECK(name);
    return SRQ_OK;
}

}  // namespace

extern "C" int srq_matmul_s4s4(const void *A, const void *B, int64_t M, int64_t N, int64_t K,
                               int32_t *C, void *stream) {
    int rc = check_gemm("matmul", A, B, M, N, K);
    if (rc) return rc;
    SRQ_CHECK_ARG(C || M == 0 || N == 0, "matmul: null output");
    Epi e{};
    e.C = C;
    return run_gemm("matmul", A, B, M, N, K, e, (hipStream_t)stream);
}

extern "C" int srq_w4a4_linear(const void *A, const void *a_scale, const void *B,
                               const void *b_scale, const void *bias, int64_t M, int64_t N,
                               int64_t K, void *out, void *stream) {
    int rc = check_gemm("w4a4_linear", A, B, M, N, K);
    if (rc) return rc;
    if (M && N) SRQ_CHECK_ARG(out && a_scale && b_scale, "w4a4_linear: null pointer");
    Epi e{};
    e.out = (f16 *)out;
    e.sa = (const f16 *)a_scale;
    e.sb = (const f16 *)b_scale;
    e.bias = (const f16 *)bias;
    return run_gemm("w4a4_linear", A, B, M, N, K, e, (hipStream_t)stream);
}
