// MFMA rotation kernel for n = K * 512 and n = K * 1024 (9 <= K <= 32, K a
// multiple of 4): the rotation of the SignRot down_proj input (Llama-3-8B
// FFN 14336 = had_28 ⊗ H_512, Llama-3-70B FFN 28672 = had_28 ⊗ H_1024),
// optionally fused with the SignRot sign and the per-token int4 quantizer.
//
// A block of 4 waves owns one token row at a time (persistent over rows),
// with one barrier per row.  Rows are double-buffered in LDS, in the lane
// order of the stage-A A operand: the next row streams from HBM straight
// into the other buffer (buffer loads into LDS) while this one is
// transformed, and the previous row is quantized from its block reduction
// at the start of this row's iteration, so neither the fetch latency nor
// the reduction needs a barrier of its own.  Wave w computes output
// columns i2 in [32 w, 32 w + 32) of every 128-element segment.
//
// Stage A (bits 0-6 of the 512-chunk, H_128): fp16 MFMA 32x32x16.  A-operand
// row rr of a tile is the 128-element segment (chunk 8T + ct, quarter i1)
// with i1 = rr & 3 and ct = ((rr >> 3) & 3) | (((rr >> 2) & 1) << 2); with
// the MFMA output layout (lane l, register v -> row 8(v/4) + 4(l/32) + v%4,
// column l%32) this puts i1 = v % 4 and chunk 8T + 4(l/32) + v/4 in the
// registers of the lane that owns column i2 = 32 nt + l%32.  B is
// H_128 = H_4 ⊗ H_32 (two ±1 fragments and their negations).
// Stage B (bits 7-8, H_4 over i1): two butterfly stages in registers.
// y = fp16(fp32 FWHT_512 * 1/sqrt(n))        -- first rounding point
// Stage K (hadK over the K chunks): transposed MFMA out^T[i2][c] =
// sum_c' y[c'][i1][i2] hadK[c][c'], the A operand built from the lane's own
// registers (k-slot (g, e) <-> chunk 8(2s + e/4) + 4g + e%4), so lane
// (c = l%32, g) receives 16 outputs of chunk c; stage A's output columns
// are permuted (pl below) so that these are the 16 consecutive
// i2 = 32 nt + 16 g .. + 15, stored directly (no staging through LDS).
// out = fp16(fp32 sum)                        -- second rounding point
//
// H_1024 (P = 2): the row is 2K 512-chunks, chunk j = 2c + h for Hadamard
// chunk c and bit 9 h.  Stages A and B run on the 512-chunks unchanged;
// chunks 2c and 2c + 1 land in registers v and v + 4 (v / 4 even) of the
// same lane, so the bit-9 butterfly is one more fp32 stage in registers
// before the first rounding point (ascending bit order, as everywhere).
// The K-mix then runs once per h, k-slot (g, e) of step s <-> chunk
// c' = 16 s + 4 (e / 2) + 2 g + e % 2, i.e. tile 4 s + e / 2, register
// group v / 4 = 2 (e % 2) + h: again the lane's own registers.
// The K-mix result stays in registers as packed fp16 (with the sign applied
// as an xor of the fp16 sign bit) while the block reduces the row max.
//
// Quantizer: s = fp16(amax / 7) (then fp16(s * clip)), r = fl32(1 / s), and
// per element fp16(x * r) by one v_fma_mix*_f16; the SignRot sign is folded
// into the offset add below (codes of -x are the negated codes of x).  For fp16 x and s that is
// the correctly rounded fp16(x / s) of the reference's __hdiv whenever the
// quotient is >= 2^-14, and it yields the same int4 code for every pair
// (exhaustively checked over all fp16 pairs by tests/c/quot_exact.c).
// Round half even to an integer by + 1544 in fp16 (ulp 1 there): the low
// nibble is then code + 8, turned into the two's-complement nibble by an
// xor with 8 after packing.  The clamp to [-8, 7] is skipped for a row whose
// quotients all lie within ±7.25 (amax <= 7.25 s), the usual case for
// clip = 1; otherwise codes are clamped in fp16 first.
#include "common.h"

#include <type_traits>

namespace {

typedef float v2f __attribute__((ext_vector_type(2)));
typedef u32 v2u __attribute__((ext_vector_type(2)));

SRQ_DEV v16f mfma32(v8h a, v8h b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

SRQ_DEV int parity(int v) { return __builtin_popcount(v) & 1; }

// two fp32 -> packed fp16 pair (v_cvt_pk_f16_f32, round to nearest even)
SRQ_DEV u32 pk16(float a, float b) {
    return __builtin_bit_cast(u32, __builtin_convertvector((v2f){a, b}, v2h));
}

// max(m, |a|, |b|): written as a left-leaning chain, which the backend
// turns into one v_max3_f32 with abs modifiers (an inline-asm v_max3 would
// read MFMA results without the hazard wait states the compiler inserts)
SRQ_DEV float absmax3(float m, float a, float b) { return fmaxf(fmaxf(m, fabsf(a)), fabsf(b)); }

constexpr uint32_t kOob = 0xFFFFFFF0u;

struct MfmaRotArgs {
    const f16 *x;
    int64_t rows;
    int KC;               // Kronecker factor K
    const f16 *hadK;      // [KC, KC]
    const int8_t *sign;   // [n] or null
    float scale;          // fp32 1/sqrt(n)
    float clip;
    uint8_t *q;           // quant mode: packed codes, rows of n/2 bytes
    f16 *qscale;          // quant mode: [rows]
    f16 *qzero;           // asymmetric quant mode: zero points [rows]
    f16 *out;             // rotation mode: fp16 rows of n
    const f16 *up;        // SwiGLU input: x is the gate, this the up projection
    int64_t ld;           // row stride of x (and up), elements
    // per-row sign (MoE down-proj input): row r takes row sign_row[r] of the
    // [n_sign_rows, n] sign table (ids outside the table: sign +1)
    const int32_t *sign_row;
    int64_t n_sign_rows;
    // MODE 1: write the codes in the bf6 block layout of srq_i4_to_bf6
    // (rows of n codes, n % 128 == 0) instead of packed int4
    int bf6;
};

// Stores of one lane's results.  After the K-mix a lane (chunk ln, half g)
// holds, for each quarter i1, the 16 consecutive outputs i2 = 32 nt + 16 g
// + 0..15 of chunk ln as 8 packed fp16 pairs w[i1][0..7]: 32 bytes of a
// rotated row, 8 bytes of its codes (qrow: the lane's first code byte of
// quarter 0; quarter i1 is 64 bytes further).

// Symmetric int4 codes with the SignRot sign folded into the offset add:
// sg[i1][p] holds the two elements' signs as fp16 ±1.0, and
// fp16(q * sign + 1544) rounds the signed quotient half to even (ulp 1 in
// [1024, 2048)) with the code + 8 in the low nibble.  The codes of a sign-
// flipped value are the negated codes (round half to even is odd-symmetric),
// so this equals quantizing x * sign.  CLAMP: the signed quotient is clamped
// to [-8, 7] in fp16 first.
template <bool CLAMP>
SRQ_DEV u32 offset_codes_signed(u32 q, u32 sg) {
    v2h h = __builtin_bit_cast(v2h, q);
    const v2h s = __builtin_bit_cast(v2h, sg);
    if (CLAMP) {
        h = h * s;
        h = __builtin_elementwise_min(__builtin_elementwise_max(h, (v2h){-8, -8}), (v2h){7, 7});
        h = h + (v2h){1544, 1544};
    } else {
        h = __builtin_elementwise_fma(h, s, (v2h){1544, 1544});
    }
    return __builtin_bit_cast(u32, h);
}

template <bool CLAMP>
SRQ_DEV void quant_store(const u32 (&w)[4][8], const u32 (&sg)[4][8], float rcp, uint8_t *qrow) {
#pragma unroll
    for (int i1 = 0; i1 < 4; ++i1) {
        u32 c[8];
#pragma unroll
        for (int p = 0; p < 8; ++p) c[p] = offset_codes_signed<CLAMP>(quot2(w[i1][p], rcp), sg[i1][p]);
        const v2u r = {pack8(c[0], c[1], c[2], c[3]), pack8(c[4], c[5], c[6], c[7])};
        // non-temporal (cfg2 M = 2048: 24.9-25.0 -> 23.7 us per launch, and
        // the GEMM reading the codes next no slower; one box, alternating)
        __builtin_nontemporal_store(r, reinterpret_cast<v2u *>(qrow + i1 * 64));
    }
}

// The same codes for a row holding a NaN or inf (after the rotation), by the
// exact per-element arithmetic: the quotient of the packed route is NaN there
// and would not give the reference's code 0.  r = 1 / s is inf for s == 0
// and 0 for s == inf, so x * r behaves as the reference's x / s.
SRQ_DEV void quant_store_exact(const u32 (&w)[4][8], const u32 (&sg)[4][8], float s,
                               uint8_t *qrow) {
    const float r = sym_recip(s);
#pragma unroll
    for (int i1 = 0; i1 < 4; ++i1) {
        u32 c[2] = {0, 0};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const v2h pr = __builtin_bit_cast(v2h, w[i1][e / 2]);
            const v2h sp = __builtin_bit_cast(v2h, sg[i1][e / 2]);
            const float x = (float)pr[e & 1] * (float)sp[e & 1];  // exact sign flip
            c[e / 8] |= (u32)(sym_code_r(x, r) & 0xF) << (4 * (e % 8));
        }
        *reinterpret_cast<uint2 *>(qrow + i1 * 64) = (uint2){c[0], c[1]};
    }
}

// bf6 output (MODE 1 with MfmaRotArgs::bf6): the codes of a lane's 16
// consecutive outputs i2 = 32 nt + 16 g + e of one quarter are fields
// j = 16 g + e of MFMA lane (row % 32) + 32 (nt % 2), k slice nt / 2, of
// the quarter's 32 x 128 block: 96 bits, written as three dwords -- g = 0 to
// bytes 0-11 of the slice's 16-byte run X, g = 1 to bytes 12-15 of X and
// the slice's 8 bytes of the shared run Y.
typedef _Float16 v32h __attribute__((ext_vector_type(32)));
typedef int v6i __attribute__((ext_vector_type(6)));

// Two quarters' codes per conversion: c[0] (quarter i1) and c[1] (i1 + 1),
// 16 each -> 192 bits, the first 96 for quarter i1.
SRQ_DEV void store_bf6_pair(const v2h (&c)[2][8], uint8_t *const *X, uint8_t *const *Y, int g) {
    v32h v;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            v[16 * t + 2 * p] = c[t][p][0];
            v[16 * t + 2 * p + 1] = c[t][p][1];
        }
    const v6i o = __builtin_amdgcn_cvt_scalef32_pk32_bf6_f16(v, 1.0f);  // exact integers
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        u32 *d0 = reinterpret_cast<u32 *>(g ? X[t] + 12 : X[t]);
        u32 *d1 = reinterpret_cast<u32 *>(g ? Y[t] : X[t] + 4);
        u32 *d2 = reinterpret_cast<u32 *>(g ? Y[t] + 4 : X[t] + 8);
        *d0 = (u32)o[3 * t];
        *d1 = (u32)o[3 * t + 1];
        *d2 = (u32)o[3 * t + 2];
    }
}

template <bool CLAMP>
SRQ_DEV void quant_store_bf6(const u32 (&w)[4][8], const u32 (&sg)[4][8], float rcp,
                             uint8_t *const (&X)[4], uint8_t *const (&Y)[4], int g) {
#pragma unroll
    for (int i0 = 0; i0 < 4; i0 += 2) {
        v2h c[2][8];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int p = 0; p < 8; ++p)
                c[t][p] = __builtin_bit_cast(v2h, offset_codes_signed<CLAMP>(
                                                      quot2(w[i0 + t][p], rcp), sg[i0 + t][p])) -
                          (v2h){1544, 1544};  // the signed code, exact
        store_bf6_pair(c, X + i0, Y + i0, g);
    }
}

// the exact per-element codes (rows holding a NaN or inf), bf6 output
SRQ_DEV void quant_store_bf6_exact(const u32 (&w)[4][8], const u32 (&sg)[4][8], float s,
                                   uint8_t *const (&X)[4], uint8_t *const (&Y)[4], int g) {
    const float r = sym_recip(s);
#pragma unroll
    for (int i0 = 0; i0 < 4; i0 += 2) {
        v2h c[2][8];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const v2h pr = __builtin_bit_cast(v2h, w[i0 + t][e / 2]);
                const v2h sp = __builtin_bit_cast(v2h, sg[i0 + t][e / 2]);
                c[t][e / 2][e & 1] =
                    (f16)(float)sym_code_r((float)pr[e & 1] * (float)sp[e & 1], r);
            }
        store_bf6_pair(c, X + i0, Y + i0, g);
    }
}

// Asymmetric uint4 codes of the same values (MODE 2, w already signed):
// FAST, the packed route (finite row, s > 0, |zi| <= 511); otherwise each
// code by the exact per-element arithmetic (asym_code).
template <bool FAST>
SRQ_DEV void quant_store_asym(const u32 (&w)[4][8], float rcp, v2h lo, v2h hi, v2h zo,
                              float s, int zi, uint8_t *qrow) {
#pragma unroll
    for (int i1 = 0; i1 < 4; ++i1) {
        u32 r[2];
#pragma unroll
        for (int hlf = 0; hlf < 2; ++hlf) {
            const int u = 4 * hlf;
            if constexpr (FAST) {
                r[hlf] = pack8_raw(asym_offset_codes(quot2(w[i1][u], rcp), lo, hi, zo),
                                   asym_offset_codes(quot2(w[i1][u + 1], rcp), lo, hi, zo),
                                   asym_offset_codes(quot2(w[i1][u + 2], rcp), lo, hi, zo),
                                   asym_offset_codes(quot2(w[i1][u + 3], rcp), lo, hi, zo));
            } else {
                r[hlf] = 0;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const v2h pr = __builtin_bit_cast(v2h, w[i1][u + e / 2]);
                    r[hlf] |= (u32)(asym_code((float)pr[e & 1], s, zi, 0, 15) & 0xF) << (4 * e);
                }
            }
        }
        *reinterpret_cast<uint2 *>(qrow + i1 * 64) = (uint2){r[0], r[1]};
    }
}

// MODE: 0 rotation (fp16 out), 1 + symmetric int4 quantizer, 2 + asymmetric
// uint4 quantizer (row min/max, scale and zero point).
// SW: the row is swiglu(gate, up) of two strided inputs (one workgroup per
// CU: the up prefetch needs the registers two workgroups would share; with
// H_1024 chunks up to K = 28).
// P: 512-chunks per Hadamard chunk (1: H_512, 2: H_1024; one workgroup per
// CU, which holds twice the row in registers).
template <int NT, int MODE, bool SW, int P>
__global__ __launch_bounds__(256, (SW || P == 2 || MODE == 2) ? 1 : 2) void had512_mfma_kernel(
    MfmaRotArgs a) {
    // The staged rows, double-buffered (row r of the block's sequence in
    // rowbuf[r & 1]): 128-element segment (chunk c, quarter i1) at
    // + 256 (4c + i1) bytes, its 16-byte piece p at position p ^ 2h(c, i1),
    // h = i1 | ((c >> 2) & 1) << 2.  The swizzle makes the stage-A reads
    // (8 lanes: one piece of 8 segments with distinct h) hit distinct LDS
    // banks.  Chunks K .. 8 NT - 1 stay zero.
    __shared__ v4i rowbuf[2][NT * 8 * 64];
    // row reduction, double-buffered by row parity: MODE 1 max |x| and the
    // non-finite flag per wave; MODE 2 min, max and the non-finite flag
    __shared__ float red[2][MODE == 2 ? 12 : 8];
    const int lane = threadIdx.x & 63;
    const int nt = threadIdx.x >> 6;  // the wave
    const int g = lane >> 5;
    const int ln = lane & 31;
    const int nc = a.KC * P;  // 512-chunks in the row
    const int n = nc * 512;

    // ---- constants
    // Output column permutation: MFMA column ln of this n-tile computes i2 =
    // 32 nt + pl, pl = perm(ln) moving bit 2 of ln to bit 4 and bits 3-4 to
    // bits 2-3.  The MFMA output rows a lane holds (8 j + 4 g + r, r < 4) then
    // become the K-mix rows of the 16 consecutive i2 = 32 nt + 16 g + 4 j + r,
    // so each lane ends with 16 adjacent outputs per quarter and stores them
    // directly (32 bytes of fp16, 8 bytes of codes).
    const int pl = (ln & 3) | (((ln >> 3) & 3) << 2) | (((ln >> 2) & 1) << 4);
    // H_128 B operand for this n-tile, k-steps 0..7: entry e of step ks is
    // (-1)^(parity((16 (ks & 1) + 8 g + e) & pl) ^ parity((ks >> 1) & nt)).
    // The low 3 bits of the row index are e alone, so the parity splits into
    // an 8-entry pattern in e (shared by all steps) and one sign per step.
    union BkU {
        v8h h;
        u32 w[4];
    } Bk[8];
    {
        BkU pat;
#pragma unroll
        for (int e = 0; e < 8; ++e) pat.h[e] = parity(e & pl) ? (f16)-1 : (f16)1;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const u32 flip = (parity((16 * (ks & 1) + 8 * g) & pl) ^ parity((ks >> 1) & nt))
                                 ? 0x80008000u : 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i) Bk[ks].w[i] = pat.w[i] ^ flip;
        }
    }
    // hadK B operand (k-slot (g, e) <-> chunk cp = 8 (2s + e/4) + 4g + e%4,
    // column ln) and the sign xor masks of this lane's outputs (for each i1,
    // the 16 values v' at i2 = 32 nt + 8 (v'/4) + 4 g + v'%4 of chunk ln, as
    // 8 fp16 pairs), fetched by independent buffer loads (out-of-range
    // offsets read zeros) so their latencies overlap.  K is a multiple of 4,
    // so each run of 4 cp is wholly inside or outside the table.
    v8h HB[2];
    {
        const __amdgpu_buffer_rsrc_t hr = make_rsrc(a.hadK, (int64_t)a.KC * a.KC * 2);
        if constexpr (P == 1) {
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int cp = 8 * (2 * s + h) + 4 * g;
                    const uint32_t off =
                        (ln < a.KC && cp < a.KC) ? (uint32_t)((ln * a.KC + cp) * 2) : kOob;
                    const v4h v = __builtin_bit_cast(
                        v4h, __builtin_amdgcn_raw_buffer_load_b64(hr, off, 0, 0));
#pragma unroll
                    for (int e = 0; e < 4; ++e) HB[s][4 * h + e] = v[e];
                }
        } else {
            // k-slot pair (2 q, 2 q + 1) <-> chunks cp, cp + 1
#pragma unroll
            for (int s = 0; s < 2; ++s)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int cp = 16 * s + 4 * q + 2 * g;
                    const uint32_t off =
                        (ln < a.KC && cp < a.KC) ? (uint32_t)((ln * a.KC + cp) * 2) : kOob;
                    const v2h v = __builtin_bit_cast(
                        v2h, __builtin_amdgcn_raw_buffer_load_b32(hr, off, 0, 0));
                    HB[s][2 * q] = v[0];
                    HB[s][2 * q + 1] = v[1];
                }
        }
    }
    // msk[h][i1][p]: the signs of this lane's outputs (Hadamard chunk ln,
    // half h, quarter i1, elements 2p and 2p + 1 of its 16): MODE 0 and 2 as
    // fp16 sign-bit xor masks, MODE 1 as fp16 ±1.0 pairs (the quantizer
    // folds them into its offset add)
    constexpr u32 kSignBase = MODE == 1 ? 0x3C003C00u : 0u;
    u32 msk[P][4][8];
#pragma unroll
    for (int h = 0; h < P; ++h)
#pragma unroll
        for (int i1 = 0; i1 < 4; ++i1)
#pragma unroll
            for (int p = 0; p < 8; ++p) msk[h][i1][p] = kSignBase;
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.sign, a.sign_row ? a.n_sign_rows * n : n);
    // the sign masks of row r's sign row (called before the next row's
    // prefetch is issued, so waiting for them leaves the prefetch in flight)
    // The 16 int8 signs of (h, i1) are 16 consecutive bytes of the sign row
    // (i2 = 32 nt + 16 g .. + 15): one 16-byte load each (a lane per 4-byte
    // piece would touch a cache line per lane per piece); dword u holds the
    // signs of elements 4 u .. 4 u + 3, i.e. of pairs 2 u and 2 u + 1.
    auto load_msk = [&](uint32_t base, bool ok) __attribute__((always_inline)) {
#pragma unroll
        for (int h = 0; h < P; ++h)
#pragma unroll
            for (int i1 = 0; i1 < 4; ++i1) {
                const uint32_t off =
                    ok ? base + (uint32_t)(ln * 512 * P + h * 512 + i1 * 128 + 32 * nt + 16 * g)
                       : kOob;
                const v4i s16 = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                                            sr, off, 0, 0));
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const u32 sw = (u32)s16[u];
                    msk[h][i1][2 * u] = kSignBase | ((sw & 0x80u) << 8) | ((sw & 0x8000u) << 16);
                    msk[h][i1][2 * u + 1] =
                        kSignBase | ((sw & 0x800000u) >> 8) | (sw & 0x80000000u);
                }
            }
    };
    auto load_row_msk = [&](int64_t r) __attribute__((always_inline)) {
        const int64_t e = a.sign_row[r];
        const bool ok = e >= 0 && e < a.n_sign_rows && ln < a.KC;
        load_msk(ok ? (uint32_t)(e * n) : 0u, ok);
    };
    if (a.sign && !a.sign_row) load_msk(0u, ln < a.KC);

    // A-operand row of this lane in stage A: segment (chunk 8T + cta,
    // quarter i1a), piece 2 ks + g.
    const int i1a = ln & 3;
    const int cta = ((ln >> 3) & 3) | (((ln >> 2) & 1) << 2);
    const int ha = i1a | (((cta >> 2) & 1) << 2);
    const int rdbase = (cta * 4 + i1a) * 256 + 16 * g;
    // Row fetch: instruction j of wave w moves chunk c = 4j + w whole (1 KB),
    // K / 4 instructions per wave.  Plain rows go straight from HBM to LDS
    // (buffer loads into LDS: lane L = 16 i1 + p' writes LDS piece p' of
    // segment (c, i1) and so reads global piece p' ^ 2h(c, i1)).  SwiGLU rows
    // are loaded to registers (gate and up), combined, and stored.
    const int64_t xbytes = a.rows > 0 ? ((a.rows - 1) * a.ld + n) * 2 : 0;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x, xbytes);
    const __amdgpu_buffer_rsrc_t ur = make_rsrc(SW ? a.up : a.x, xbytes);
    const int cpw = nc / 4;
    const int wi1 = lane >> 4, wp = lane & 15;
    uint32_t dma_off[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) dma_off[b] = wi1 * 256 + 16 * (wp ^ (2 * (wi1 | (b << 2))));
    v4i pre[SW ? NT * 2 : 1];
    v4i preu[SW ? NT * 2 : 1];
    // SwiGLU rows move in halves (PART 0: j < NT, 1: j >= NT) or whole (-1)
    auto in_part = [](int j, auto part) __attribute__((always_inline)) {
        constexpr int PART = decltype(part)::value;
        return PART < 0 || (PART == 0 ? j < NT : j >= NT);
    };
    using Whole = std::integral_constant<int, -1>;
    auto fetch = [&](int64_t r, int buf, auto part) __attribute__((always_inline)) {
        const uint32_t rb = (uint32_t)(r * a.ld * 2);
        if constexpr (!SW) {
            const uint32_t lb = (uint32_t)(uintptr_t)&rowbuf[buf][0];
#pragma unroll
            for (int j = 0; j < NT * 2; ++j)
                if (j < cpw) {
                    const int c = 4 * j + nt;
                    dma16(xr, rb + c * 1024 + dma_off[(c >> 2) & 1], lb + c * 1024);
                }
        } else {
            const uint32_t lr = rb + (uint32_t)(nt * 1024 + lane * 16);
#pragma unroll
            for (int j = 0; j < NT * 2; ++j)
                if (j < cpw && in_part(j, part)) {
                    pre[j] = __builtin_bit_cast(
                        v4i, __builtin_amdgcn_raw_buffer_load_b128(xr, lr + j * 4096, 0, 0));
                    preu[j] = __builtin_bit_cast(
                        v4i, __builtin_amdgcn_raw_buffer_load_b128(ur, lr + j * 4096, 0, 0));
                }
        }
    };
    // SwiGLU rows: combine the fetched gate / up pieces into rowbuf[buf]
    auto sw_store = [&](int buf, auto part) __attribute__((always_inline)) {
        if constexpr (SW) {
#pragma unroll
            for (int j = 0; j < NT * 2; ++j) {
                if (j >= cpw || !in_part(j, part)) continue;
                const int c = 4 * j + nt;
                const int h = wi1 | (((c >> 2) & 1) << 2);
                const v8h g8 = __builtin_bit_cast(v8h, pre[j]);
                const v8h u8 = __builtin_bit_cast(v8h, preu[j]);
                v8h o;
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = swiglu1((float)g8[e], (float)u8[e]);
                rowbuf[buf][(c * 4 + wi1) * 16 + (wp ^ (2 * h))] = __builtin_bit_cast(v4i, o);
            }
        }
    };
    for (int i = threadIdx.x; i < (NT * 8 - nc) * 64; i += 256) {
        rowbuf[0][nc * 64 + i] = (v4i){0, 0, 0, 0};
        rowbuf[1][nc * 64 + i] = (v4i){0, 0, 0, 0};
    }

    // Row loop, one barrier per row: iteration it transforms row `row` (in
    // rowbuf[it & 1], its block reduction into red[it & 1]) and finishes the
    // previous row (quantization from red[(it - 1) & 1]), while the next
    // row streams into rowbuf[(it + 1) & 1].
    const int64_t step = gridDim.x;
    int64_t row = blockIdx.x;
    // SwiGLU rows of H_1024 are fetched and combined in two halves: the
    // gate / up registers of a whole 2K-chunk row would not fit beside the
    // transform's
    auto fetch_sw_now = [&](int64_t r, int buf) __attribute__((always_inline)) {
        using H0 = std::integral_constant<int, 0>;
        using H1 = std::integral_constant<int, 1>;
        fetch(r, buf, H0{});
        sw_store(buf, H0{});
        fetch(r, buf, H1{});
        sw_store(buf, H1{});
    };
    if (row < a.rows) {
        if constexpr (SW && P == 2) {
            fetch_sw_now(row, 0);
        } else {
            fetch(row, 0, Whole{});
            if constexpr (SW) sw_store(0, Whole{});
        }
    }
    // Settle the prologue loads here, after the first row's fetch is issued
    // (their latencies overlap): the empty asm consumes HB and msk, so the
    // wait for their loads is placed once, before the row loop.
    // Otherwise the wait-count pass, unable to prove across the loop's back
    // edge that these loads are done, waits for them inside every row --
    // and, counting in order, for the next row's prefetch as well.
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
        BkU t;
        t.h = HB[s2];
        asm volatile("" : "+v"(t.w[0]), "+v"(t.w[1]), "+v"(t.w[2]), "+v"(t.w[3]));
        HB[s2] = t.h;
    }
#pragma unroll
    for (int h = 0; h < P; ++h)
#pragma unroll
        for (int i1 = 0; i1 < 4; ++i1)
#pragma unroll
            for (int p = 0; p < 8; ++p) asm volatile("" : "+v"(msk[h][i1][p]));

    // SwiGLU rows of H_1024 quantize each row in its own iteration, after a
    // second barrier: holding the previous row's outputs next to the gate /
    // up prefetch of a 2K-chunk row would exceed the register file
    constexpr bool kDefer = !(SW && P == 2);
    u32 wprev[kDefer ? P : 1][4][8];
    int64_t prev = -1;
    // Quantize the previous row r (its K-mix outputs wprev) from its block
    // reduction in red[par] and store its codes: MODE 1 symmetric int4 with
    // the sign folded into the offset add, MODE 2 asymmetric uint4 (wprev is
    // already signed).
    auto finish_row = [&](int64_t r, int par, auto &wq) __attribute__((always_inline)) {
        // this lane's first code byte: chunk ln, i2 = 32 nt + 16 g (quarter 0)
        uint8_t *qlane = a.q + r * (n / 2) + (ln * 512 * P + 32 * nt + 16 * g) / 2;
        const float *rr = red[par];
        if constexpr (MODE == 1) {
            if (a.sign && a.sign_row) load_row_msk(r);
            const float amx = round16(fmaxf(fmaxf(rr[0], rr[1]), fmaxf(rr[2], rr[3])));
            const bool bad =
                __builtin_amdgcn_readfirstlane((rr[4] + rr[5] + rr[6] + rr[7]) != 0.f);
            f16 s16 = f16_rn(amx / 7.f);
            if (a.clip != 1.f) s16 = f16_rn((float)s16 * a.clip);
            // quotient divisor: s itself, or 2^-126 when s == 0 -- then every
            // nonzero x overflows to ±inf and clamps to 7 / -8, and x == 0
            // gives 0, which is what x / 0 yields after the reference's
            // __half2int_rn (saturation, NaN -> 0)
            const float sq = fmaxf((float)s16, 0x1p-126f);
            const float rcp = 1.0f / sq;
            if (threadIdx.x == 0) a.qscale[r] = s16;
            // row-uniform: can any |x / s| round beyond ±7?
            const bool clampit = __builtin_amdgcn_readfirstlane(!(amx <= 7.25f * sq));
            if (ln < a.KC && !a.bf6) {
#pragma unroll
                for (int h = 0; h < P; ++h) {
                    uint8_t *qrow = qlane + h * 256;
                    if (bad) quant_store_exact(wq[h], msk[h], (float)s16, qrow);
                    else if (clampit) quant_store<true>(wq[h], msk[h], rcp, qrow);
                    else quant_store<false>(wq[h], msk[h], rcp, qrow);
                }
            } else if (ln < a.KC) {
                // 32 x 128 block (r / 32, kb) with kb = 4 (P ln + h) + i1
                const int lm = (int)(r & 31) + 32 * (nt & 1);
                uint8_t *rowblk = a.q + (r >> 5) * (int64_t)(n / 128) * 3072;
#pragma unroll
                for (int h = 0; h < P; ++h) {
                    uint8_t *X[4], *Y[4];
#pragma unroll
                    for (int i1 = 0; i1 < 4; ++i1) {
                        uint8_t *blk = rowblk + (int64_t)(4 * (P * ln + h) + i1) * 3072;
                        X[i1] = blk + 1024 * (nt >> 1) + 16 * lm;
                        Y[i1] = blk + 2048 + 16 * lm + 8 * (nt >> 1);
                    }
                    if (bad) quant_store_bf6_exact(wq[h], msk[h], (float)s16, X, Y, g);
                    else if (clampit) quant_store_bf6<true>(wq[h], msk[h], rcp, X, Y, g);
                    else quant_store_bf6<false>(wq[h], msk[h], rcp, X, Y, g);
                }
            }
        } else {
            const float vmin = fminf(fminf(rr[0], rr[1]), fminf(rr[2], rr[3]));
            const float vmax = fmaxf(fmaxf(rr[4], rr[5]), fmaxf(rr[6], rr[7]));
            const bool bad = (rr[8] + rr[9] + rr[10] + rr[11]) != 0.f;
            f16 sh, zh;
            asym_row_params(vmin, vmax, a.clip, sh, zh);
            if (threadIdx.x == 0) {
                a.qscale[r] = sh;
                a.qzero[r] = zh;
            }
            const float sf = (float)sh;
            const int zi = h2i_rn((float)zh);
            const bool fast = __builtin_amdgcn_readfirstlane(!bad && sf > 0.f && zi >= -511 &&
                                                             zi <= 511);
            const float rcp = 1.0f / fmaxf(sf, 0x1p-126f);
            const v2h lo2 = (v2h){(f16)(float)(-zi), (f16)(float)(-zi)};
            const v2h hi2 = (v2h){(f16)(float)(15 - zi), (f16)(float)(15 - zi)};
            const v2h zo2 = (v2h){(f16)(float)zi, (f16)(float)zi};
            if (ln < a.KC) {
#pragma unroll
                for (int h = 0; h < P; ++h) {
                    uint8_t *qrow = qlane + h * 256;
                    if (fast) quant_store_asym<true>(wq[h], rcp, lo2, hi2, zo2, sf, zi, qrow);
                    else quant_store_asym<false>(wq[h], rcp, lo2, hi2, zo2, sf, zi, qrow);
                }
            }
        }
    };
    // Transform row `row` from rowbuf[buf]: stages A and B, the K-mix
    // into w (packed fp16), MODE 0 stores, MODE 1 / 2 partial row
    // reductions into red[par].
    auto transform = [&](int64_t row, int buf, int par, u32 (&w)[P][4][8])
                         __attribute__((always_inline)) {
        const uint8_t *rowb = reinterpret_cast<const uint8_t *>(&rowbuf[buf][0]);
        if (a.sign && a.sign_row && MODE != 1) load_row_msk(row);

        // ---- stage A (H_128 over i2, this wave's 32 output columns) and
        // stage B (H_4 over i1), y = fp16(FWHT * 1/sqrt(n)) into the K-mix
        // A operands ka[s][h][i1] (P = 1: k-slot e <-> tile 2s + e/4, chunk
        // 4g + e%4; P = 2: tile 4s + e/2, register group 2 (e%2) + h)
        constexpr int TPS = 2 * P;  // tiles per K-mix step
        constexpr int NS = (NT + TPS - 1) / TPS;
        union KA {
            v8h h;
            u32 w[4];
        } ka[NS][P][4];
        if (NT % TPS) {
#pragma unroll
            for (int h = 0; h < P; ++h)
#pragma unroll
                for (int i1 = 0; i1 < 4; ++i1) ka[NS - 1][h][i1].h = (v8h){};
        }
        // (slots of chunks >= K hold zeros: their prefetch read zeros).
        // The 8 LDS reads of tile T + 1 are issued before the MFMAs of tile
        // T (left to itself the scheduler puts each read just before its
        // MFMA and exposes every LDS round trip).
        v8h xk[2][8];
        auto rd = [&](int T, int ks) __attribute__((always_inline)) {
            return *reinterpret_cast<const v8h *>(rowb + T * 8192 + rdbase + 32 * (ks ^ ha));
        };
        // Stage B (+ the bit-9 stage for P = 2) and the first rounding
        // point for tile T's accumulators.  P = 1: register v -> ka[T/2][0]
        // [v%4] element 4 (T%2) + v/4, the pairs (v, v + 4) adjacent
        // elements.  P = 2: registers (4h + i1, 4h + i1 + 8) -> ka[T/4][h]
        // [i1] elements 2 (T%4), 2 (T%4) + 1.
        auto finish = [&](v16f d, int T) __attribute__((always_inline)) {
#pragma unroll
            for (int v = 0; v < 16; v += 4) {
                const float a0 = d[v], a1 = d[v + 1], a2 = d[v + 2], a3 = d[v + 3];
                const float b0 = a0 + a1, b1 = a0 - a1, b2 = a2 + a3, b3 = a2 - a3;
                d[v] = b0 + b2;
                d[v + 1] = b1 + b3;
                d[v + 2] = b0 - b2;
                d[v + 3] = b1 - b3;
            }
            if constexpr (P == 1) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    if ((v / 4) % 2) continue;
                    float lo = d[v] * a.scale, hi = d[v + 4] * a.scale;
                    // pin the fp32 products: fp16(fp32(x * s)), two roundings
                    asm volatile("" : "+v"(lo), "+v"(hi));
                    ka[T / 2][0][v % 4].w[2 * (T % 2) + v / 8] = pk16(lo, hi);
                }
            } else {
                // bit 9: chunk 2c (registers v) with chunk 2c + 1 (v + 4)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    if ((v / 4) % 2) continue;
                    const float lo = d[v], hi = d[v + 4];
                    d[v] = lo + hi;
                    d[v + 4] = lo - hi;
                }
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int i1 = 0; i1 < 4; ++i1) {
                        float lo = d[4 * h + i1] * a.scale, hi = d[4 * h + i1 + 8] * a.scale;
                        asm volatile("" : "+v"(lo), "+v"(hi));
                        ka[T / 4][h][i1].w[T % 4] = pk16(lo, hi);
                    }
            }
        };
        // Software pipeline over the tiles: the LDS reads of tile T + 1 and
        // the stage-B VALU work of tile T - 1 are interleaved with the 8
        // MFMAs of tile T, so the matrix and vector pipes overlap.
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) xk[0][ks] = rd(0, ks);
        v16f dprev = {};
#pragma unroll
        for (int T = 0; T < NT; ++T) {
            if (T + 1 < NT) {
#pragma unroll
                for (int ks = 0; ks < 8; ++ks) xk[(T + 1) & 1][ks] = rd(T + 1, ks);
            }
            v16f d = {};
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) d = mfma32(xk[T & 1][ks], Bk[ks].h, d);
            if (T > 0) finish(dprev, T - 1);
            if (T + 1 < NT) __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (T > 0) __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            dprev = d;
        }
        finish(dprev, NT - 1);

        // ---- K-mix: round to fp16 and keep (MODE 0 and 2 apply the sign
        // here; MODE 1 folds it into the quantizer).  MODE 1: NaN-propagating
        // packed max and min of the rounded outputs (v_pk_maximum3 /
        // v_pk_minimum3, four values per instruction); rounding is monotone
        // and odd-symmetric, so max(mx, -mn) is fp16(max |out|) for a row
        // free of NaN, and inf or NaN flags a row holding a NaN or an output
        // that rounds to inf (|out| >= 65520).  A wave holding such a lane
        // recomputes its NaN-ignoring max (the reference's fmaxf) from the
        // kept values.  MODE 2: packed min and max of the signed fp16 values
        // (NaN-ignoring, as fminf / fmaxf) and the packed NaN-propagating max
        // of |x|.  Lanes past the K chunks hold no outputs and stay out of
        // the reductions and flags.
        v2h mn2 = (v2h){(f16)__builtin_inff(), (f16)__builtin_inff()};
        v2h mx2 = -mn2, ab2 = (v2h){0, 0};
#pragma unroll
        for (int h = 0; h < P; ++h)
#pragma unroll
            for (int i1 = 0; i1 < 4; ++i1) {
                v16f z = {};
                z = mfma32(ka[0][h][i1].h, HB[0], z);
                if (NS > 1) z = mfma32(ka[NS > 1 ? 1 : 0][h][i1].h, HB[1], z);
#pragma unroll
                for (int p = 0; p < 8; ++p) {
                    if (MODE == 1) {
                        w[h][i1][p] = pk16(z[2 * p], z[2 * p + 1]);
                        if (p & 1) {
                            const v2h v0 = __builtin_bit_cast(v2h, w[h][i1][p - 1]);
                            const v2h v1 = __builtin_bit_cast(v2h, w[h][i1][p]);
                            mx2 = __builtin_elementwise_maximum(
                                __builtin_elementwise_maximum(mx2, v0), v1);
                            mn2 = __builtin_elementwise_minimum(
                                __builtin_elementwise_minimum(mn2, v0), v1);
                        }
                    } else {
                        w[h][i1][p] = pk16(z[2 * p], z[2 * p + 1]) ^ msk[h][i1][p];
                    }
                    if (MODE == 2 && ln < a.KC) {
                        const v2h v = __builtin_bit_cast(v2h, w[h][i1][p]);
                        mn2 = __builtin_elementwise_min(mn2, v);
                        mx2 = __builtin_elementwise_max(mx2, v);
                        ab2 = __builtin_elementwise_maximum(ab2, __builtin_elementwise_abs(v));
                    }
                }
            }
        if (MODE == 0) {
            if (ln < a.KC) {
#pragma unroll
                for (int h = 0; h < P; ++h)
#pragma unroll
                    for (int i1 = 0; i1 < 4; ++i1) {
                        // 16 fp16 (32 bytes) at i2 = 32 nt + 16 g
                        f16 *orow = a.out + row * n + ln * 512 * P + h * 512 + i1 * 128 +
                                    32 * nt + 16 * g;
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            uint4 pk;
                            pk.x = w[h][i1][4 * hh];
                            pk.y = w[h][i1][4 * hh + 1];
                            pk.z = w[h][i1][4 * hh + 2];
                            pk.w = w[h][i1][4 * hh + 3];
                            *reinterpret_cast<uint4 *>(orow + 8 * hh) = pk;
                        }
                    }
            }
        }
        if constexpr (MODE == 1) {
            // partial row max |x| and non-finite flag of this wave
            float al = __builtin_elementwise_maximum(
                __builtin_elementwise_maximum((float)mx2[0], (float)mx2[1]),
                -__builtin_elementwise_minimum((float)mn2[0], (float)mn2[1]));
            if (ln >= a.KC) al = 0.f;
            const bool badl = !(al <= 65504.f);
            const bool wbad = __builtin_amdgcn_ballot_w64(badl) != 0;
            if (wbad) {
                // NaN-ignoring max |x| of this lane's kept outputs
                al = 0.f;
                if (ln < a.KC) {
#pragma unroll
                    for (int h = 0; h < P; ++h)
#pragma unroll
                        for (int i1 = 0; i1 < 4; ++i1)
#pragma unroll
                            for (int p = 0; p < 8; ++p) {
                                // through an empty asm, so this rare-path
                                // work stays behind the branch
                                u32 t = w[h][i1][p];
                                asm volatile("" : "+v"(t));
                                const v2h v = __builtin_bit_cast(v2h, t);
                                al = absmax3(al, (float)v[0], (float)v[1]);
                            }
                }
            }
            const float amax = wave_max_dpp(al);
            if (lane == 0) {
                red[par][nt] = amax;
                red[par][4 + nt] = wbad ? 1.f : 0.f;
            }
        } else if constexpr (MODE == 2) {
            // partial row min / max and non-finite flag of this wave
            float fmn = fminf((float)mn2[0], (float)mn2[1]);
            float fmx = fmaxf((float)mx2[0], (float)mx2[1]);
            const bool badl = !((float)ab2[0] <= 65504.f) || !((float)ab2[1] <= 65504.f);
            fmn = -wave_max_dpp(-fmn);
            fmx = wave_max_dpp(fmx);
            const bool wbad = __builtin_amdgcn_ballot_w64(badl) != 0;
            if (lane == 0) {
                red[par][nt] = fmn;
                red[par][4 + nt] = fmx;
                red[par][8 + nt] = wbad ? 1.f : 0.f;
            }
        }
    };
    // One row per iteration and one barrier per row: iteration it
    // transforms row `row` (rowbuf[it & 1], reduction into red[it & 1])
    // and finishes the previous row, while the next row streams into
    // rowbuf[(it + 1) & 1].
    for (int it = 0;; ++it) {
        const bool have = row < a.rows;
        // this wave's row fetches (and the previous row's code stores)
        // are done; after the barrier every wave's are, every wave has
        // finished the previous iteration's LDS reads, and
        // red[(it - 1) & 1] is whole
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        const bool more = have && row + step < a.rows;
        if constexpr (SW && P == 2) {
            // the next row, combined now so its gate / up registers are
            // free during this row's transform
            if (more) fetch_sw_now(row + step, (it + 1) & 1);
        } else {
            if (more) fetch(row + step, (it + 1) & 1, Whole{});
        }
        if constexpr (MODE >= 1 && kDefer) {
            if (prev >= 0) finish_row(prev, (it - 1) & 1, wprev);
            prev = -1;
        }
        if (!have) break;
        if constexpr (kDefer) {
            transform(row, it & 1, it & 1, wprev);
            prev = row;
        } else {
            u32 w[P][4][8];
            transform(row, it & 1, it & 1, w);
            if constexpr (MODE >= 1) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                finish_row(row, it & 1, w);
            }
        }
        if constexpr (SW && P == 1) {
            if (more) sw_store((it + 1) & 1, Whole{});
        }
        row += step;
    }
}

}  // namespace

// Fast path dispatcher, used by srq_online_hadamard / srq_had_sign_quant.
// Returns 1 if it launched, 0 if the shape is not covered.
int srq_had512_mfma(const void *x, int64_t rows, int64_t n, int64_t K, const void *hadK,
                    const int8_t *sign, float clip, void *q, void *qscale, void *out,
                    hipStream_t st, const void *up, int64_t ld, const int32_t *sign_row,
                    int64_t n_sign_rows, void *qzero, int bf6) {
    // K % 4 == 0: the row fetch moves 4 chunks per instruction and the hadK
    // loads take runs of 2 or 4 table entries (every Hadamard order above 2
    // is a multiple of 4)
    if (K < 9 || K > 32 || K % 4) return 0;
    int P;
    if (n == K * 512) P = 1;
    else if (n == K * 1024) P = 2;
    else return 0;
    // the SwiGLU form of H_1024 holds gate and up prefetches of a 2K-chunk
    // row: it fits the register file up to K = 28 (K = 32 would spill)
    if (up && P == 2 && K > 28) return 0;
    if (qzero && (up || !q)) return 0;  // asymmetric codes: plain rows only
    if (bf6 && (!q || qzero || n % 128 || !srq_aligned(q, 16))) return 0;
    if (ld < n) ld = n;
    if (rows > 0 && ((rows - 1) * ld + n) * 2 >= (int64_t)kOob) return 0;  // 32-bit offsets
    if (!srq_aligned(x, 16) || (up && !srq_aligned(up, 16)) || ld % 8) return 0;
    if (q && !srq_aligned(q, 8)) return 0;     // 8-byte code stores
    if (out && !srq_aligned(out, 16)) return 0;  // 16-byte fp16 stores
    MfmaRotArgs a{};
    a.x = (const f16 *)x;
    a.rows = rows;
    a.KC = (int)K;
    a.hadK = (const f16 *)hadK;
    a.sign = sign;
    a.scale = 1.0f / sqrtf((float)n);
    a.clip = clip;
    a.q = (uint8_t *)q;
    a.qscale = (f16 *)qscale;
    a.out = (f16 *)out;
    a.up = (const f16 *)up;
    a.ld = ld;
    a.sign_row = sign_row;
    a.n_sign_rows = n_sign_rows;
    a.qzero = (f16 *)qzero;
    a.bf6 = bf6;
    // persistent blocks of 4 waves, up to 2 per CU (256 CUs; 1 with the
    // SwiGLU input, H_1024 chunks or the asymmetric quantizer), one row each
    // at a time
    const int64_t cap = (up || P == 2 || qzero) ? 256 : 256 * 2;
    const int64_t blocks = rows < cap ? rows : cap;
    const dim3 grid((unsigned)blocks), block(256);
    auto go = [&](auto ntc, auto modec, auto swc, auto pc) {
        had512_mfma_kernel<decltype(ntc)::value, decltype(modec)::value, decltype(swc)::value,
                           decltype(pc)::value><<<grid, block, 0, st>>>(a);
    };
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using I4 = std::integral_constant<int, 4>;
    using I7 = std::integral_constant<int, 7>;
    using I8 = std::integral_constant<int, 8>;
    using M0 = std::integral_constant<int, 0>;
    using M1 = std::integral_constant<int, 1>;
    using M2 = std::integral_constant<int, 2>;
    using S0 = std::false_type;
    using S1 = std::true_type;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    auto mode = [&](auto modec) {
        if (P == 1) {
            // tiles of 8 chunks: K = 12, 16 | 20, 24 | 28, 32
            const int nt = (int)srq_cdiv(K, 8);
            if (nt == 2) go(I2{}, modec, S0{}, P1{});
            else if (nt == 3) go(I3{}, modec, S0{}, P1{});
            else go(I4{}, modec, S0{}, P1{});
        } else {
            // 2K chunks; tiles past the row's chunks hold zeros
            if (K <= 16) go(I4{}, modec, S0{}, P2{});
            else if (K <= 28) go(I7{}, modec, S0{}, P2{});
            else go(I8{}, modec, S0{}, P2{});
        }
    };
    if (up) {
        if (!q) return 0;
        if (P == 1) {
            const int nt = (int)srq_cdiv(K, 8);
            if (nt == 2) go(I2{}, M1{}, S1{}, P1{});
            else if (nt == 3) go(I3{}, M1{}, S1{}, P1{});
            else go(I4{}, M1{}, S1{}, P1{});
        } else {
            if (K <= 16) go(I4{}, M1{}, S1{}, P2{});
            else go(I7{}, M1{}, S1{}, P2{});
        }
    } else if (q && qzero) {
        mode(M2{});
    } else if (q) {
        mode(M1{});
    } else {
        mode(M0{});
    }
    return 1;
}
