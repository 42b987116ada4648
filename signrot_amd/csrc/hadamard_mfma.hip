// MFMA rotation kernel for n = K * 512 (2 <= K <= 32): the rotation of the
// SignRot down_proj input (Llama-3 FFN 14336 = had_28 ⊗ H_512), optionally
// fused with the SignRot sign and the per-token int4 quantizer.
//
// A block of 4 waves owns one token row at a time (persistent over rows):
// the row is staged in LDS by direct global -> LDS loads (the next row's
// transfer overlaps this row's K-mix and quantization), and wave w computes
// output columns i2 in [32 w, 32 w + 32) of every 128-element segment.
//
// Stage A (bits 0-6 of the 512-chunk, H_128): fp16 MFMA 32x32x16 straight
// from the global loads.  A-operand row rr of a tile is the 128-element
// segment (chunk 8T + ct, quarter i1) with i1 = rr & 3 and
// ct = ((rr >> 3) & 3) | (((rr >> 2) & 1) << 2); with the MFMA output layout
// (lane l, register v -> row 8(v/4) + 4(l/32) + v%4, column l%32) this puts
// i1 = v % 4 and chunk 8T + 4(l/32) + v/4 in the registers of the lane that
// owns column i2 = 32 nt + l%32.  B is H_128 = H_4 ⊗ H_32 (two ±1 fragments
// and their negations).
// Stage B (bits 7-8, H_4 over i1): two butterfly stages in registers.
// y = fp16(fp32 FWHT_512 * 1/sqrt(n))        -- first rounding point
// Stage K (hadK over the K chunks): transposed MFMA out^T[i2][c] =
// sum_c' y[c'][i1][i2] hadK[c][c'], the A operand built from the lane's own
// registers (k-slot (g, e) <-> chunk 8(2s + e/4) + 4g + e%4), so lane
// (c = l%32, g) receives runs of 4 consecutive i2 of chunk c.
// out = fp16(fp32 sum)                        -- second rounding point
// Then sign (xor of the fp16 sign bit), row amax (a first pass over the
// K-mix), scale, and the exact quantizer:
//   t = x * r, e = fma(-s, t, x), t' = fma(e, r, t) with r = 1/s.
// For fp16 x and s the exact quotient x/s is either an fp16 rounding
// midpoint never (12 significant bits cannot be a product of 11-bit
// numbers) or at relative distance >= 2^-22 from every midpoint, and t' is
// within 2^-23 of x/s, so fp16(t') == fp16(x/s): the reference's correctly
// rounded __hdiv.  Round half even and clamp to [-8, 7] via + 1536 in fp16.
#include "common.h"

namespace {

typedef _Float16 v2h __attribute__((ext_vector_type(2)));

SRQ_DEV v16f mfma32(v8h a, v8h b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

SRQ_DEV int parity(int v) { return __builtin_popcount(v) & 1; }


typedef __attribute__((address_space(3))) void lds_void;

struct MfmaRotArgs {
    const f16 *x;
    int64_t rows;
    int KC;               // Kronecker factor K (number of 512-chunks)
    const f16 *hadK;      // [KC, KC]
    const int8_t *sign;   // [n] or null
    float scale;          // fp32 1/sqrt(n)
    float clip;
    uint16_t *q;          // quant mode: packed codes, rows of n/2 bytes
    f16 *qscale;          // quant mode: [rows]
    f16 *out;             // rotation mode: fp16 rows of n
};

template <int NT, int MODE>
__global__ __launch_bounds__(256, 2) void had512_mfma_kernel(MfmaRotArgs a) {
    // One block of 4 waves transforms one token row at a time (persistent
    // over rows).  The row is staged in LDS by direct global -> LDS loads in
    // the lane order of the stage-A A operand: slot (T, ks) holds each lane's
    // 16-byte piece at rowbuf[((T * 8 + ks) * 64 + lane) * 4].  Wave w owns
    // output n-tile nt = w (columns i2 = 32 w .. 32 w + 31 of every
    // 128-segment): its stage A, H_4, K-mix and quantization.
    __shared__ __attribute__((aligned(16))) uint32_t rowbuf[NT * 8 * 64 * 4];
    __shared__ float red[2][4];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nt = wave;
    const int g = lane >> 5;
    const int ln = lane & 31;
    const int n = a.KC * 512;

    // ---- constants
    v8h Bk[8];  // H_128 B operand for this n-tile, k-steps 0..7
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
        const bool neg = parity((ks >> 1) & nt);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const bool m = parity((16 * (ks & 1) + 8 * g + e) & ln) ^ neg;
            Bk[ks][e] = m ? (f16)-1 : (f16)1;
        }
    }
    v8h HB[2];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int cp = 8 * (2 * s + e / 4) + 4 * g + (e % 4);
            HB[s][e] = (ln < a.KC && cp < a.KC) ? a.hadK[ln * a.KC + cp] : (f16)0;
        }
    // sign xor masks of this lane's outputs: for each i1, the 16 values
    // v' (i2 = 32 nt + 8 (v'/4) + 4 g + v'%4 of chunk ln) as 8 fp16 pairs
    uint32_t msk[4][8];
#pragma unroll
    for (int i1 = 0; i1 < 4; ++i1)
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            uint32_t m = 0;
            if (a.sign && ln < a.KC) {
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const int vp = 2 * p + b;
                    const int i2 = 32 * nt + 8 * (vp / 4) + 4 * g + (vp % 4);
                    if (a.sign[ln * 512 + i1 * 128 + i2] < 0) m |= 0x8000u << (16 * b);
                }
            }
            msk[i1][p] = m;
        }

    // A-operand row of this lane: segment (chunk 8T + ct, quarter i1a)
    const int i1a = ln & 3;
    const int cta = ((ln >> 3) & 3) | (((ln >> 2) & 1) << 2);
    // wave w issues the loads of slots (T, ks) with (T * 8 + ks) % 4 == w
    auto load_row = [&](int64_t r) {
#pragma unroll
        for (int T = 0; T < NT; ++T) {
            const int c = 8 * T + cta;
#pragma unroll
            for (int ks = wave & 3; ks < 8; ks += 4) {
                if (c < a.KC)
                    __builtin_amdgcn_global_load_lds(
                        (const void *)(a.x + r * n + c * 512 + i1a * 128 + 8 * g + 16 * ks),
                        (lds_void *)(rowbuf + (T * 8 + ks) * 64 * 4), 16, 0, 0);
            }
        }
    };

    int64_t row = blockIdx.x;
    if (row < a.rows) load_row(row);
    for (int it = 0; row < a.rows; row += gridDim.x, ++it) {
        // this wave's transfers have landed; after the barrier, everyone's
        // (a plain s_barrier: __syncthreads' release fence would also wait
        // for the output stores still in flight)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");

        // ---- stage A (H_128 over i2, this wave's 32 output columns) and
        // stage B (H_4 over i1), y = fp16(FWHT * 1/sqrt(n)) into the K-mix
        // A operands ka[s][i1] (k-slot e <-> tile 2s + e/4, chunk 4g + e%4)
        constexpr int NS = (NT + 1) / 2;
        v8h ka[NS][4];
        if (NT % 2) {
#pragma unroll
            for (int i1 = 0; i1 < 4; ++i1) ka[NS - 1][i1] = (v8h){};
        }
#pragma unroll
        for (int T = 0; T < NT; ++T) {
            v16f d = {};
            const bool live = 8 * T + cta < a.KC;
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const v8h xk = live
                    ? *reinterpret_cast<const v8h *>(rowbuf + ((T * 8 + ks) * 64 + lane) * 4)
                    : (v8h){};
                d = mfma32(xk, Bk[ks], d);
            }
#pragma unroll
            for (int v = 0; v < 16; v += 4) {
                const float a0 = d[v], a1 = d[v + 1], a2 = d[v + 2], a3 = d[v + 3];
                const float b0 = a0 + a1, b1 = a0 - a1, b2 = a2 + a3, b3 = a2 - a3;
                d[v] = b0 + b2;
                d[v + 1] = b1 + b3;
                d[v + 2] = b0 - b2;
                d[v + 3] = b1 - b3;
            }
#pragma unroll
            for (int v = 0; v < 16; ++v)
                ka[T / 2][v % 4][4 * (T % 2) + v / 4] = f16_rn(d[v] * a.scale);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();  // every wave is done with rowbuf
        asm volatile("" ::: "memory");
        if (row + gridDim.x < a.rows) load_row(row + gridDim.x);

        // ---- K-mix pass 1: row max of |fp16(out)| = fp16(max |out|)
        float amax = 0.f;
#pragma unroll
        for (int i1 = 0; i1 < 4; ++i1) {
            v16f z = {};
            z = mfma32(ka[0][i1], HB[0], z);
            if (NS > 1) z = mfma32(ka[NS > 1 ? 1 : 0][i1], HB[1], z);
#pragma unroll
            for (int v = 0; v < 16; ++v) amax = fmaxf(amax, fabsf(z[v]));
        }
        amax = wave_max(amax);
        if (lane == 0) red[it & 1][wave] = amax;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        amax = round16(fmaxf(fmaxf(red[it & 1][0], red[it & 1][1]),
                             fmaxf(red[it & 1][2], red[it & 1][3])));

        f16 s16 = f16_rn(amax / 7.f);
        if (a.clip != 1.f) s16 = f16_rn((float)s16 * a.clip);
        // quotient divisor: s itself, or 2^-126 when s == 0 -- then every
        // nonzero x overflows to ±inf and clamps to 7 / -8, and x == 0 gives
        // 0, which is what x / 0 yields after the reference's __half2int_rn
        // (saturation, NaN -> 0)
        const float sq = fmaxf((float)s16, 0x1p-126f);
        const float rcp = 1.0f / sq;
        if (MODE == 1 && threadIdx.x == 0) a.qscale[row] = s16;

        // ---- K-mix pass 2: round, sign, then quantize (or store)
#pragma unroll
        for (int i1 = 0; i1 < 4; ++i1) {
            v16f z = {};
            z = mfma32(ka[0][i1], HB[0], z);
            if (NS > 1) z = mfma32(ka[NS > 1 ? 1 : 0][i1], HB[1], z);
            uint32_t w[8];
#pragma unroll
            for (int p = 0; p < 8; ++p) {
                v2h h2;
                h2[0] = (f16)z[2 * p];
                h2[1] = (f16)z[2 * p + 1];
                w[p] = __builtin_bit_cast(uint32_t, h2) ^ msk[i1][p];
            }
            if (ln >= a.KC) continue;
            const int64_t base = (int64_t)ln * 512 + i1 * 128 + 32 * nt + 4 * g;
            if constexpr (MODE == 0) {
                // rotation output: runs of 4 fp16 (8 bytes) at i2 = 8u + 4g
                f16 *orow = a.out + row * n + base;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    uint2 pk;
                    pk.x = w[2 * u];
                    pk.y = w[2 * u + 1];
                    *reinterpret_cast<uint2 *>(orow + 8 * u) = pk;
                }
            } else {
                uint16_t *qrow = a.q + (row * n + base) / 4;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    uint32_t nib[2];
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const v2h xv = __builtin_bit_cast(v2h, w[2 * u + hh]);
                        v2h qv;
#pragma unroll
                        for (int b = 0; b < 2; ++b) {
                            const float xf = (float)xv[b];
                            const float t = xf * rcp;
                            const float er = __builtin_fmaf(-sq, t, xf);
                            qv[b] = (f16)__builtin_fmaf(er, rcp, t);
                        }
                        // clamp to [-8, 7] then + 1536: round half even to an
                        // integer whose low nibble is the two's-complement code
                        qv = __builtin_elementwise_min(
                            __builtin_elementwise_max(qv, (v2h){-8, -8}), (v2h){7, 7});
                        qv = qv + (v2h){1536, 1536};
                        const uint32_t bits = __builtin_bit_cast(uint32_t, qv) & 0x000F000Fu;
                        nib[hh] = (bits | (bits >> 12)) & 0xFFu;
                    }
                    qrow[2 * u] = (uint16_t)(nib[0] | (nib[1] << 8));
                }
            }
        }
    }
}

}  // namespace

// Fast path dispatcher, used by srq_online_hadamard / srq_had_sign_quant.
// Returns 1 if it launched, 0 if the shape is not covered.
int srq_had512_mfma(const void *x, int64_t rows, int64_t n, int64_t K, const void *hadK,
                    const int8_t *sign, float clip, void *q, void *qscale, void *out,
                    hipStream_t st) {
    if (K < 9 || K > 32 || n != K * 512) return 0;
    if (!srq_aligned(x, 16)) return 0;
    if (q && !srq_aligned(q, 2)) return 0;
    if (out && !srq_aligned(out, 8)) return 0;
    MfmaRotArgs a{};
    a.x = (const f16 *)x;
    a.rows = rows;
    a.KC = (int)K;
    a.hadK = (const f16 *)hadK;
    a.sign = sign;
    a.scale = 1.0f / sqrtf((float)n);
    a.clip = clip;
    a.q = (uint16_t *)q;
    a.qscale = (f16 *)qscale;
    a.out = (f16 *)out;
    // persistent blocks of 4 waves, up to 2 per CU (256 CUs), one row each
    // at a time
    int64_t blocks = rows;
    if (blocks > 256 * 2) blocks = 256 * 2;
    const dim3 grid((unsigned)blocks), block(256);
    const int nt = (int)srq_cdiv(K, 8);
    if (q) {
        if (nt == 2) had512_mfma_kernel<2, 1><<<grid, block, 0, st>>>(a);
        else if (nt == 3) had512_mfma_kernel<3, 1><<<grid, block, 0, st>>>(a);
        else had512_mfma_kernel<4, 1><<<grid, block, 0, st>>>(a);
    } else {
        if (nt == 2) had512_mfma_kernel<2, 0><<<grid, block, 0, st>>>(a);
        else if (nt == 3) had512_mfma_kernel<3, 0><<<grid, block, 0, st>>>(a);
        else had512_mfma_kernel<4, 0><<<grid, block, 0, st>>>(a);
    }
    return 1;
}
