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
// 2^31 for K < 131072; K = 131072 with every code -8 reaches 2^31 and would
// wrap, so K <= 131040) and the epilogue shifts right by 8.  The lo/hi split
// permutes K inside each 16-element group; A and B go through the same
// permutation, so the integer dot product is unchanged -- bit-exact.
//
// Epilogue (fused): out = fp16((float(acc) * float(sa[m])) * float(sb[n])),
// two separate fp32 multiplies in this order (quant.cu:84-87), then
// fp16(out + bias[n]) as torch's fp16 add (nn/linear.py:47-48).
#include "common.h"

#include <type_traits>

namespace {

SRQ_DEV u32 lo4(u32 w) { return (w << 4) & 0xF0F0F0F0u; }
SRQ_DEV u32 hi4(u32 w) { return w & 0xF0F0F0F0u; }

// 8 packed bytes (16 int4) -> one MFMA operand of 16 int8.  The two low
// nibble words come from one 64-bit shift (the nibble that crosses from w0
// into w1 is masked off).
SRQ_DEV v4i unpack8(u32 w0, u32 w1) {
    const uint64_t sh = ((uint64_t)w1 << 32 | w0) << 4;
    v4i r;
    r[0] = (int)((u32)sh & 0xF0F0F0F0u);
    r[1] = (int)hi4(w0);
    r[2] = (int)((u32)(sh >> 32) & 0xF0F0F0F0u);
    r[3] = (int)hi4(w1);
    return r;
}

// Unsigned A (matmul_ui4_si4): the nibbles u (0..15) stay in the low half of
// each byte, a non-negative int8, in the same element order as unpack8; with
// B unpacked as 16 w the MFMA accumulates 16 * sum(u * w) exactly
// (|.| <= 1920 K < 2^31) and the epilogue shifts right by 4.
SRQ_DEV v4i unpack8u(u32 w0, u32 w1) {
    v4i r;
    r[0] = (int)(w0 & 0x0F0F0F0Fu);
    r[1] = (int)((w0 >> 4) & 0x0F0F0F0Fu);
    r[2] = (int)(w1 & 0x0F0F0F0Fu);
    r[3] = (int)((w1 >> 4) & 0x0F0F0F0Fu);
    return r;
}

// A-operand unpack: signed (UA = false) or unsigned (UA = true) nibbles
template <bool UA>
SRQ_DEV v4i unpack8a(u32 w0, u32 w1) {
    if constexpr (UA) return unpack8u(w0, w1);
    else return unpack8(w0, w1);
}

SRQ_DEV v4i mfma16(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

constexpr uint32_t kOob = 0xFFFFFFF0u;

SRQ_DEV v4i bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// byte offset of 16-byte chunk (row, kbyte) of a [rows, KB] packed matrix,
// or kOob when it lies outside
SRQ_DEV uint32_t chunk_off(int64_t row, int64_t rows, int64_t kb, int64_t KB) {
    return (row < rows && kb < KB) ? (uint32_t)(row * KB + kb) : kOob;
}

struct Epi {
    int32_t *C;        // int32 output (plain GEMM) or null
    f16 *out;          // fp16 output (fused) or null
    const f16 *sa;     // [M]
    const f16 *sb;     // [N]
    const f16 *bias;   // [N] or null
    const f16 *res;    // [M, N] residual added last (may alias out) or null
    int ua;            // A holds unsigned nibbles (accumulator = 16 sum, not 256 sum)
    const int8_t *zr;  // asymmetric activations: zero point per row [M] (with ws) or null
    const int32_t *ws; // sum of each weight row's codes [N]
    // stream kernel only: the N columns are blocks of 8 gate then 8 up
    // columns and out [M, N / 2] receives swiglu(gate, up) of each pair
    // (C, bias, res and zr null)
    int swiglu;
    // swiglu output row stride in elements, 0 for N / 2 (read by the big
    // and grouped kernels' LDS swiglu epilogues only: launch_gemm's column
    // split)
    int64_t ldo;
};

// The int32 product of output (m, n) from the MFMA accumulator: sum(a * w),
// minus zr[m] * ws[n] (int32 arithmetic, wrapping, as the reference's
// matmul_colrow_i8_i32 and `x -= zeros` do) when zero points are given.
SRQ_DEV int epi_val(const Epi &e, int acc, int64_t m, int64_t n) {
    int v = acc >> (e.ua ? 4 : 8);
    if (e.zr) v = (int)((u32)v - (u32)(int)e.zr[m] * (u32)e.ws[n]);
    return v;
}

SRQ_DEV void store_one(const Epi &e, int64_t N, int64_t m, int64_t n, int acc256) {
    const int v = epi_val(e, acc256, m, n);
    if (e.C) {
        e.C[m * N + n] = v;
    } else {
        const float a = (float)v * (float)e.sa[m];
        f16 o = f16_rn(a * (float)e.sb[n]);
        if (e.bias) o = f16_rn((float)o + (float)e.bias[n]);
        if (e.res) o = f16_rn((float)o + (float)e.res[m * N + n]);
        e.out[m * N + n] = o;
    }
}

// Store a wave's FM x FN block of 16x16 accumulators (16x16 layout: lane
// holds column lane & 15, rows 4 * (lane >> 4) + r), loading each row and
// column scale once.
template <int FM, int FN>
SRQ_DEV void store_block(const Epi &e, int64_t M, int64_t N, int64_t mb, int64_t nb,
                         const v4i (&acc)[FM][FN], int lane) {
    float sbv[FN];
    int64_t gnv[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        gnv[j] = nb + j * 16 + (lane & 15);
        sbv[j] = (!e.C && gnv[j] < N) ? (float)e.sb[gnv[j]] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t gm = mb + i * 16 + 4 * (lane >> 4) + r;
            if (gm >= M) continue;
            const float sa = e.C ? 0.f : (float)e.sa[gm];
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if (gnv[j] >= N) continue;
                const int v = epi_val(e, acc[i][j][r], gm, gnv[j]);
                if (e.C) {
                    e.C[gm * N + gnv[j]] = v;
                } else {
                    const float a = (float)v * sa;
                    f16 o = f16_rn(a * sbv[j]);
                    if (e.bias) o = f16_rn((float)o + (float)e.bias[gnv[j]]);
                    if (e.res) o = f16_rn((float)o + (float)e.res[gm * N + gnv[j]]);
                    e.out[gm * N + gnv[j]] = o;
                }
            }
        }
}

// ---------------------------------------------------------------------------
// Large-M kernel: 256 x 128 block per workgroup, split into two kinds of
// waves.  Producer waves (NPROD) only move data: K advances KBB bytes
// (2 KBB codes) per step through an NSTG-stage LDS ring filled by buffer ->
// LDS DMA (buffer_load_dwordx4 ... lds), NSTG - 1 steps in flight, with
// out-of-range chunks (tile edges, K tail) arriving as zeros.  Compute waves
// (WGM x WGN, each FM x FN blocks of v_mfma_i32_32x32x32_i8, the gfx950 int8
// MFMA with the highest sustained rate) only read LDS, unpack nibbles and
// multiply.  Keeping the DMA issue off the compute waves matters: a burst of
// LDS-DMA instructions stalls the issuing wave until the address unit takes
// them, which, on the compute waves, serialised data movement with the
// MFMAs.  One workgroup barrier per step separates "step s landed / step
// s - 1 consumed" from "step s + NSTG - 1 may be issued".  The DMA is issued
// from inline asm and its completion tracked explicitly with vmcnt.
// A stage holds the 256 A rows then the 128 B rows, KBB bytes each,
// with 16-byte chunk j of row r at position j ^ f(r), f(r) = (r / R) % C
// for R = 256 / KBB rows per 256-byte LDS bank cycle and C = KBB / 16
// chunks per row: the 16 rows that a 16-lane group of a fragment read
// touches (rows r .. r+15 of one chunk column) land in 16 distinct 16-byte
// bank groups.  A lane reads 16 bytes (32 codes) per fragment and feeds two
// MFMA K-slices from it (half-wave g takes chunk 2p + g, bytes 0-7 then
// 8-15); A and B use the same K mapping, so the dot products are exact.

SRQ_DEV v16i mfma32i8(v4i a, v4i b, v16i c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

constexpr int kBigBM = 256, kBigBN = 128;
constexpr int kBigRows = kBigBM + kBigBN;

template <int KBB>
SRQ_DEV int swz(int r) {
    return (r / (256 / KBB)) % (KBB / 16);
}

// Store a wave's FM x FN block of 32x32 accumulators (lane holds column
// lane & 31, rows 8 (v / 4) + 4 (lane / 32) + v % 4), each row and column
// scale loaded once.
template <int FM, int FN>
SRQ_DEV void store_block32(const Epi &e, int64_t M, int64_t N, int64_t mb, int64_t nb,
                           const v16i (&acc)[FM][FN], int lane) {
    float sbv[FN];
    int64_t gnv[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        gnv[j] = nb + j * 32 + (lane & 31);
        sbv[j] = (!e.C && gnv[j] < N) ? (float)e.sb[gnv[j]] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t gm = mb + i * 32 + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
            if (gm >= M) continue;
            const float sa = e.C ? 0.f : (float)e.sa[gm];
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if (gnv[j] >= N) continue;
                const int val = epi_val(e, acc[i][j][v], gm, gnv[j]);
                if (e.C) {
                    e.C[gm * N + gnv[j]] = val;
                } else {
                    const float a = (float)val * sa;
                    f16 o = f16_rn(a * sbv[j]);
                    if (e.bias) o = f16_rn((float)o + (float)e.bias[gnv[j]]);
                    if (e.res) o = f16_rn((float)o + (float)e.res[gm * N + gnv[j]]);
                    e.out[gm * N + gnv[j]] = o;
                }
            }
        }
}

// fp16 epilogue through LDS: the wave's (32 FM) x (32 FN) block is
// dequantized (and bias added) into its private LDS area `tile` (row stride
// 32 FN halves), then stored row-wise, each lane 16 bytes (8 outputs), with
// the residual read the same way.  The MFMA layout stores would write 2
// bytes per lane; this cuts the store instructions 8-fold (the epilogue of
// the M = 2048 GEMM took 20 of its 108 us).  Same arithmetic as store_one.
// Row of accumulator element v of a BS x BS MFMA block held by `lane`
// (column lane % BS): 32x32 -> 8 (v / 4) + 4 (lane / 32) + v % 4,
// 16x16 -> 4 (lane / 16) + v.
template <int BS>
SRQ_DEV int frag_row(int v, int lane) {
    if constexpr (BS == 32) return 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
    else return 4 * (lane >> 4) + v;
}

template <int BS, int FM, int FN, bool CHECK, typename AccT>
SRQ_DEV void store_block_lds_impl(const Epi &e, int64_t M, int64_t N, int64_t mb, int64_t nb,
                                  const AccT (&acc)[FM][FN], int lane, f16 *tile) {
    constexpr int NV = BS * BS / 64;  // accumulator elements per lane per block
    constexpr int W = BS * FN;        // tile row stride (halves)
    float sbv[FN], bv[FN];
    int64_t gnv[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        gnv[j] = nb + j * BS + (lane & (BS - 1));
        const bool on = !CHECK || gnv[j] < N;
        sbv[j] = on ? (float)e.sb[gnv[j]] : 0.f;
        bv[j] = on && e.bias ? (float)e.bias[gnv[j]] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        // the block's row scales first, all loads in flight together
        float sav[NV];
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int64_t gm = mb + i * BS + frag_row<BS>(v, lane);
            sav[v] = !CHECK || gm < M ? (float)e.sa[gm] : 0.f;
        }
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int lr = i * BS + frag_row<BS>(v, lane);
            const int64_t gm = mb + lr;
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                int val = acc[i][j][v] >> (e.ua ? 4 : 8);
                if (e.zr) {  // (uniform) asymmetric activations
                    const bool on = !CHECK || (gm < M && gnv[j] < N);
                    val = on ? epi_val(e, acc[i][j][v], gm, gnv[j]) : 0;
                }
                f16 o = f16_rn((float)val * sav[v] * sbv[j]);
                if (e.bias) o = f16_rn((float)o + bv[j]);
                tile[lr * W + j * BS + (lane & (BS - 1))] = o;
            }
        }
    }
    if (e.swiglu) {
        // 16 staged columns per lane (8 gate, 8 up: N % 16 == 0, blocks of
        // 16 aligned) -> 8 swiglu1 outputs of the [M, N/2] output, 16 bytes
        constexpr int LPS = W / 16;
        constexpr int RPS = 64 / LPS;
        static_assert(LPS >= 1 && 64 % LPS == 0, "swiglu row shape");
        const int c16 = (lane % LPS) * 16;
        const int64_t gs0 = nb + c16;
#pragma unroll
        for (int r0 = 0; r0 < BS * FM; r0 += RPS) {
            const int lr = r0 + lane / LPS;
            const int64_t gm = mb + lr;
            if (lr >= BS * FM || (CHECK && (gm >= M || gs0 + 16 > N))) continue;
            const v8h gv = *reinterpret_cast<const v8h *>(tile + lr * W + c16);
            const v8h uv = *reinterpret_cast<const v8h *>(tile + lr * W + c16 + 8);
            v8h o;
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = swiglu1((float)gv[k], (float)uv[k]);
            *reinterpret_cast<v8h *>(e.out + gm * (e.ldo ? e.ldo : N / 2) + gs0 / 2) = o;
        }
        return;
    }
    constexpr int LPR = W / 8;     // lanes per row (16 bytes each)
    constexpr int RPI = 64 / LPR;  // rows per store instruction
    static_assert(LPR >= 1 && 64 % LPR == 0 && (BS * FM) % RPI == 0, "row store shape");
    const int c8 = (lane % LPR) * 8;
    const int64_t gn0 = nb + c8;
    const bool vec = N % 8 == 0 && ((uintptr_t)e.out % 16 == 0) &&
                     (!e.res || (uintptr_t)e.res % 16 == 0);
#pragma unroll
    for (int r0 = 0; r0 < BS * FM; r0 += RPI) {
        const int lr = r0 + lane / LPR;
        const int64_t gm = mb + lr;
        if (CHECK && gm >= M) continue;
        v8h o = *reinterpret_cast<const v8h *>(tile + lr * W + c8);
        if (vec && (!CHECK || gn0 + 8 <= N)) {
            if (e.res) {
                const v8h rv = *reinterpret_cast<const v8h *>(e.res + gm * N + gn0);
#pragma unroll
                for (int k = 0; k < 8; ++k) o[k] = f16_rn((float)o[k] + (float)rv[k]);
            }
            // non-temporal: the output is not read again by this launch
            // (cfg2 M = 2048 / 8192: 96-97.5 -> 94-95 us and 355 -> 344 us
            // per GEMM, one box, the two forms alternating)
            __builtin_nontemporal_store(o, reinterpret_cast<v8h *>(e.out + gm * N + gn0));
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (gn0 + k >= N) break;
                f16 ok = o[k];
                if (e.res) ok = f16_rn((float)ok + (float)e.res[gm * N + gn0 + k]);
                e.out[gm * N + gn0 + k] = ok;
            }
        }
    }
}

// fp16 epilogue through LDS: the wave's (BS FM) x (BS FN) block of BS x BS
// MFMA accumulators is dequantized (and bias added) into its private LDS
// area `tile` (row stride BS FN halves, BS FM rows), then stored row-wise,
// each lane 16 bytes (8 outputs), with the residual read the same way.  The
// MFMA layout stores would write 2 bytes per lane, 8 times the store
// instructions.  Blocks wholly inside the matrix take a branch-free path
// (per-element bounds checks made the unrolled epilogue hundreds of
// divergent branches: 20 of the M = 2048 GEMM's 108 us).  Same arithmetic
// as store_one.  The caller's LDS `tile` must be free of other readers and
// of in-flight DMA.
template <int BS, int FM, int FN, typename AccT>
SRQ_DEV void store_block_lds(const Epi &e, int64_t M, int64_t N, int64_t mb, int64_t nb,
                             const AccT (&acc)[FM][FN], int lane, f16 *tile) {
    if (mb + BS * FM <= M && nb + BS * FN <= N)
        store_block_lds_impl<BS, FM, FN, false>(e, M, N, mb, nb, acc, lane, tile);
    else
        store_block_lds_impl<BS, FM, FN, true>(e, M, N, mb, nb, acc, lane, tile);
}

// fp16 epilogue through an int32 LDS tile, for kernels with little register
// room: the wave's raw accumulators go to its LDS area `tile` first (row
// stride BS FN words; a row pass reads whole 256-byte LDS rows), which
// frees them, then each lane dequantizes 8 consecutive outputs of a row
// (column scales loaded once per lane, one row scale per row) and stores
// them as 16 bytes.  Same arithmetic as store_one; `tile` must be free of
// other readers and of in-flight DMA, 4 BS FN BS FM bytes.
template <int BS, int FM, int FN, typename AccT>
SRQ_DEV void store_block_lds32(const Epi &e, int64_t M, int64_t N, int64_t mb, int64_t nb,
                               const AccT (&acc)[FM][FN], int lane, int32_t *tile) {
    constexpr int NV = BS * BS / 64;
    constexpr int W = BS * FN;   // outputs per row
    constexpr int WS = W;        // row stride (words)
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int lr = i * BS + frag_row<BS>(v, lane);
#pragma unroll
            for (int j = 0; j < FN; ++j) tile[lr * WS + j * BS + (lane & (BS - 1))] = acc[i][j][v];
        }
    constexpr int LPR = W / 8;     // lanes per row
    constexpr int RPI = 64 / LPR;  // rows per pass
    static_assert(LPR >= 1 && 64 % LPR == 0 && (BS * FM) % RPI == 0, "row pass shape");
    const int c8 = (lane % LPR) * 8;
    const int64_t gn0 = nb + c8;
    const bool full_n = gn0 + 8 <= N;
    float sbv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) sbv[k] = gn0 + k < N ? (float)e.sb[gn0 + k] : 0.f;
    const bool vec = full_n && N % 8 == 0 && ((uintptr_t)e.out % 16 == 0) &&
                     (!e.res || (uintptr_t)e.res % 16 == 0);
    for (int r0 = 0; r0 < BS * FM; r0 += RPI) {
        const int lr = r0 + lane / LPR;
        const int64_t gm = mb + lr;
        if (gm >= M || gn0 >= N) continue;
        const v4i a0 = *reinterpret_cast<const v4i *>(tile + lr * WS + c8);
        const v4i a1 = *reinterpret_cast<const v4i *>(tile + lr * WS + c8 + 4);
        const float sa = (float)e.sa[gm];
        v8h o;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int a = k < 4 ? a0[k] : a1[k - 4];
            const int val = epi_val(e, a, gm, gn0 + k < N ? gn0 + k : gn0);
            f16 x = f16_rn((float)val * sa * sbv[k]);
            // bias read per row pass (cached), not held in 8 more registers
            if (e.bias && gn0 + k < N) x = f16_rn((float)x + (float)e.bias[gn0 + k]);
            o[k] = x;
        }
        if (vec) {
            if (e.res) {
                const v8h rv = *reinterpret_cast<const v8h *>(e.res + gm * N + gn0);
#pragma unroll
                for (int k = 0; k < 8; ++k) o[k] = f16_rn((float)o[k] + (float)rv[k]);
            }
            // non-temporal: the output is not read again by this launch
            // (cfg2 M = 2048 / 8192: 96-97.5 -> 94-95 us and 355 -> 344 us
            // per GEMM, one box, the two forms alternating)
            __builtin_nontemporal_store(o, reinterpret_cast<v8h *>(e.out + gm * N + gn0));
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                if (gn0 + k >= N) break;
                f16 ok = o[k];
                if (e.res) ok = f16_rn((float)ok + (float)e.res[gm * N + gn0 + k]);
                e.out[gm * N + gn0 + k] = ok;
            }
        }
    }
}

// store_block_lds32 for an N whose columns are blocks of 8 gate then 8 up
// columns (nb and N multiples of 16): each lane dequantizes the 16 columns
// of one block of a row as store_block_lds32 would (symmetric A, no bias or
// residual) and stores the 8 swiglu1(gate, up) values as 16 bytes into the
// [M, N/2] output.  4 BS FN BS FM bytes of `tile`, as store_block_lds32.
template <int BS, int FM, int FN, typename AccT>
SRQ_DEV void store_block_lds32_swiglu(const Epi &e, int64_t M, int64_t N, int64_t mb,
                                      int64_t nb, const AccT (&acc)[FM][FN], int lane,
                                      int32_t *tile) {
    constexpr int NV = BS * BS / 64;
    constexpr int W = BS * FN;   // columns per row of the block
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            const int lr = i * BS + frag_row<BS>(v, lane);
#pragma unroll
            for (int j = 0; j < FN; ++j) tile[lr * W + j * BS + (lane & (BS - 1))] = acc[i][j][v];
        }
    constexpr int LPR = W / 16;    // lanes per row
    constexpr int RPI = 64 / LPR;  // rows per pass
    static_assert(LPR >= 1 && 64 % LPR == 0 && (BS * FM) % RPI == 0, "row pass shape");
    const int c16 = (lane % LPR) * 16;
    const int64_t gn0 = nb + c16;
    if (gn0 + 16 > N) return;
    float sbg[8], sbu[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        sbg[k] = (float)e.sb[gn0 + k];
        sbu[k] = (float)e.sb[gn0 + 8 + k];
    }
    for (int r0 = 0; r0 < BS * FM; r0 += RPI) {
        const int lr = r0 + lane / LPR;
        const int64_t gm = mb + lr;
        if (gm >= M) continue;
        const int32_t *tr = tile + lr * W + c16;
        const v4i g0 = *reinterpret_cast<const v4i *>(tr);
        const v4i g1 = *reinterpret_cast<const v4i *>(tr + 4);
        const v4i u0 = *reinterpret_cast<const v4i *>(tr + 8);
        const v4i u1 = *reinterpret_cast<const v4i *>(tr + 12);
        const float sa = (float)e.sa[gm];
        v8h o;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int ga = k < 4 ? g0[k] : g1[k - 4];
            const int ua = k < 4 ? u0[k] : u1[k - 4];
            const f16 gh = f16_rn((float)(ga >> 8) * sa * sbg[k]);
            const f16 uh = f16_rn((float)(ua >> 8) * sa * sbu[k]);
            o[k] = swiglu1((float)gh, (float)uh);
        }
        *reinterpret_cast<v8h *>(e.out + gm * (e.ldo ? e.ldo : N / 2) + gn0 / 2) = o;
    }
}

// One K step of a compute wave: the stage holds BM A rows then the B rows.
// XJ >= 0 (the grouped kernel's extra-row tiles): also the XB blocks of 32
// rows at xs (same row layout as the stage) times this wave's B block XJ,
// into xacc[0 .. XB - 1], from the B operands already unpacked for the tile.
template <int FM, int FN, int KBB, int BM = kBigBM, bool UA = false, int XJ = -1, int XB = 1>
SRQ_DEV void big_compute(const uint8_t *stage, int wm, int wn, int lane, v16i (&acc)[FM][FN],
                         const uint8_t *xs = nullptr, v16i *xacc = nullptr) {
    constexpr int NPP = KBB / 32;  // 16-byte fragment fetches per step
    constexpr int NX = XJ >= 0 ? XB : 0;
    static_assert(XJ < FN, "extra block");
    const int rr = lane & 31;
    const int g = lane >> 5;
    v4i fa[2][FM], fb[2][FN], fx[2][XB];
    auto fetch = [&](int pp, int slot) {
        const int j = 2 * pp + g;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int r = wm * (FM * 32) + i * 32 + rr;
            fa[slot][i] = *reinterpret_cast<const v4i *>(stage + r * KBB + ((j ^ swz<KBB>(r)) << 4));
        }
#pragma unroll
        for (int jn = 0; jn < FN; ++jn) {
            const int r = BM + wn * (FN * 32) + jn * 32 + rr;
            fb[slot][jn] = *reinterpret_cast<const v4i *>(stage + r * KBB + ((j ^ swz<KBB>(r)) << 4));
        }
#pragma unroll
        for (int xb = 0; xb < NX; ++xb) {
            const int r = 32 * xb + rr;
            fx[slot][xb] = *reinterpret_cast<const v4i *>(xs + r * KBB + ((j ^ swz<KBB>(r)) << 4));
        }
    };
    // K slice s = 2 pp + h: bytes 8h .. 8h + 7 of the 16-byte fragments of
    // fetch pp.  Software pipeline: the nibble unpacking of slice s + 1 is
    // interleaved with the MFMAs of slice s (one MFMA, then its share of
    // the unpacking VALU work), so the vector and matrix pipes overlap.
    v4i ua[2][FM], ub[2][FN], ux[2][XB];
    auto unpack = [&](int sl, int buf) {
        const int pp = sl >> 1, h = sl & 1;
#pragma unroll
        for (int i = 0; i < FM; ++i)
            ua[buf][i] = unpack8a<UA>((u32)fa[pp & 1][i][2 * h], (u32)fa[pp & 1][i][2 * h + 1]);
#pragma unroll
        for (int jn = 0; jn < FN; ++jn)
            ub[buf][jn] = unpack8((u32)fb[pp & 1][jn][2 * h], (u32)fb[pp & 1][jn][2 * h + 1]);
#pragma unroll
        for (int xb = 0; xb < NX; ++xb)
            ux[buf][xb] = unpack8a<UA>((u32)fx[pp & 1][xb][2 * h], (u32)fx[pp & 1][xb][2 * h + 1]);
    };
    fetch(0, 0);
    unpack(0, 0);
#pragma unroll
    for (int sl = 0; sl < 2 * NPP; ++sl) {
        const int pp = sl >> 1;
        if ((sl & 1) == 0 && pp + 1 < NPP) fetch(pp + 1, (pp + 1) & 1);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int jn = 0; jn < FN; ++jn)
                acc[i][jn] = mfma32i8(ua[sl & 1][i], ub[sl & 1][jn], acc[i][jn]);
#pragma unroll
        for (int xb = 0; xb < NX; ++xb)
            xacc[xb] = mfma32i8(ux[sl & 1][xb], ub[sl & 1][XJ < 0 ? 0 : XJ], xacc[xb]);
        if (sl + 1 < 2 * NPP) unpack(sl + 1, (sl + 1) & 1);
        if ((sl & 1) == 0 && pp + 1 < NPP)
            __builtin_amdgcn_sched_group_barrier(0x100, FM + FN + NX, 0);
        // unpack8 is 6 VALU; spread a slice's (FM + FN) of them over its
        // FM * FN MFMAs
        constexpr int kMf = FM * FN + NX;
        constexpr int kValuPerMfma = (6 * (FM + FN + NX) + kMf - 1) / kMf;
#pragma unroll
        for (int m = 0; m < kMf; ++m) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (sl + 1 < 2 * NPP) __builtin_amdgcn_sched_group_barrier(0x002, kValuPerMfma, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// WGM x WGN compute waves, each FM x FN blocks of 32 x 32 (a (32 FM) x
// (32 FN) wave tile), plus NPROD producer waves; the block tile is always
// kBigBM x kBigBN.  Kc > 0: split-K form, workgroup row blockIdx.y takes
// codes [y Kc, (y + 1) Kc) of K and stores its int32 partials (e.C, shifted
// down like the dense accumulator) at e.C + y M N.
template <int NPROD, int WGM, int WGN, int FM, int FN, int KBB, int NSTG, bool UA>
__global__ __launch_bounds__(64 * (WGM * WGN + NPROD), 1) void gemm_big_kernel(
    const uint8_t *__restrict__ A, const uint8_t *__restrict__ B, int64_t M, int64_t N,
    int64_t K, Epi e, int64_t Kc) {
    static_assert(WGM * FM * 32 == kBigBM && WGN * FN * 32 == kBigBN, "block tile");
    static_assert(NSTG == 3, "the producers' vmcnt waits assume one step in flight beyond the next");
    constexpr int kCompute = WGM * WGN;
    constexpr int kStage = kBigRows * KBB;
    constexpr int kRowsPerDma = 1024 / KBB;               // rows per 1 KiB DMA block
    constexpr int kDma = kBigRows / kRowsPerDma;          // DMA blocks per stage
    constexpr int kDmaPerWave = kDma / NPROD;
    static_assert(kDmaPerWave * NPROD == kDma, "DMA split");
    static_assert(kDmaPerWave <= 31, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NSTG * kStage];

    const int lane = threadIdx.x & 63;
    // wave-uniform: keeps the DMA addressing in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t tiles_n = (N + kBigBN - 1) / kBigBN;
    // XCD-aware tile order: workgroup b runs on XCD b % 8, and XCD x owns
    // one block of the tile grid, so the 32 CUs of an XCD share a few A row
    // panels and B column panels in their L2 instead of each XCD reading all
    // of B (against row-major: 3-12% faster at M = 2048 / 8192, less fabric
    // traffic).  The grid splits into pm row parts x 8 / pm column parts,
    // pm the divisor with the fewest panel rows per XCD: at M = 2048, K =
    // 14336, N = 4096 (8 x 32 tiles) 4 x 8 blocks, 14.3 MB of panels per XCD
    // against 18.4 for 2 x 16 (FETCH_SIZE 72.1 -> 57.7 MiB per launch); at
    // M = 512, N = 57344 (2 x 448) each XCD holds both tile rows of its 56
    // columns, so every B panel is fetched once.  Other grids: row-major.
    const int64_t tiles_m = (M + kBigBM - 1) / kBigBM;
    int64_t m0, n0;
    // the split of the tile grid into pm row parts x 8 / pm column parts
    // with the fewest panel rows per XCD (pm = 0: none divides the grid)
    int pm = 0;
    int64_t best = 0;
#pragma unroll
    for (int c = 1; c <= 8; c *= 2) {
        if (tiles_m % c || tiles_n % (8 / c)) continue;
        const int64_t cost = (tiles_m / c) * kBigBM + (tiles_n / (8 / c)) * kBigBN;
        if (!pm || cost < best) {
            pm = c;
            best = cost;
        }
    }
    if (pm) {
        // XCD x: row part x % pm, column part x / pm, walked row-fastest so
        // the tiles sharing a B panel run in the same round
        const int64_t x = blockIdx.x % 8, i = blockIdx.x / 8;
        const int64_t am = tiles_m / pm, bn = tiles_n / (8 / pm);
        m0 = ((x % pm) * am + i % am) * kBigBM;
        n0 = ((x / pm) * bn + i / am) * kBigBN;
    } else {
        m0 = ((int64_t)blockIdx.x / tiles_n) * kBigBM;
        n0 = ((int64_t)blockIdx.x % tiles_n) * kBigBN;
    }
    const int64_t KB = K / 2;
    // this workgroup's K bytes [kbase, kend) of every row
    const int64_t kbase = Kc ? (int64_t)blockIdx.y * (Kc / 2) : 0;
    const int64_t kend = Kc ? min(kbase + Kc / 2, KB) : KB;
    const int steps = (int)((kend - kbase + KBB - 1) / KBB);
    if (Kc) e.C += (int64_t)blockIdx.y * M * N;

    if (wave >= kCompute) {
        // ---- producer: DMA block i = kDmaPerWave * pw + q covers stage rows
        // R i .. R i + R - 1 (R = kRowsPerDma); lane l fetches chunk
        // (l % C) ^ f(r) of row r = R i + l / C.  Per-lane row offsets are
        // fixed for the whole K loop: rows outside the matrix get kOob (then
        // every chunk reads as zero); a chunk past the K tail is redirected
        // out of range the same way.
        const int pw = wave - kCompute;
        const __amdgpu_buffer_rsrc_t ar = make_rsrc(A, M * KB), br = make_rsrc(B, N * KB);
        const uint32_t lds0 =
            (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)smem;
        constexpr int C = KBB / 16;
        uint32_t roff[kDmaPerWave];
        int jc[kDmaPerWave];
#pragma unroll
        for (int q = 0; q < kDmaPerWave; ++q) {
            const int i = pw * kDmaPerWave + q;
            const int r = kRowsPerDma * i + lane / C;
            jc[q] = ((lane % C) ^ swz<KBB>(r)) * 16;
            const bool isa = kRowsPerDma * i < kBigBM;
            const int64_t row = isa ? m0 + r : n0 + r - kBigBM;
            roff[q] = row < (isa ? M : N) ? (uint32_t)(row * KB) : kOob;
        }
        auto issue = [&](int st, int sl) {
            const int64_t kb0 = kbase + (int64_t)st * KBB;
            const bool tail = kb0 + KBB > kend;
#pragma unroll
            for (int q = 0; q < kDmaPerWave; ++q) {
                const int i = pw * kDmaPerWave + q;
                const uint32_t dst = lds0 + sl * kStage + i * 1024;
                uint32_t off = roff[q] == kOob ? kOob : roff[q] + (uint32_t)kb0 + jc[q];
                if (tail && kb0 + jc[q] >= kend) off = kOob;
                dma16(kRowsPerDma * i < kBigBM ? ar : br, off, dst);
            }
        };
        issue(0, 0);
        if (steps > 1) issue(1, 1);
        int sl = 0;
        for (int s = 0; s < steps; ++s) {
            // this wave's DMA of step s is done (step s + 1's may stay in
            // flight: vmcnt counts this wave's outstanding DMA in issue order)
            if (s + 1 < steps) {
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerWave) : "memory");
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            // every producer's DMA of step s has landed, and every compute
            // wave is done with the stage that step s + 2 now overwrites
            // (read in step s - 1)
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (s + 2 < steps) issue(s + 2, sl == 0 ? 2 : sl - 1);
            sl = sl == 2 ? 0 : sl + 1;
        }
        // the compute waves meet no barrier after their K loop, so the
        // producers end here
        return;
    }

    // ---- compute
    const int wm = wave / WGN, wn = wave % WGN;
    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = (v16i){};
    int sl = 0;
    for (int s = 0; s < steps; ++s) {
        // step s has landed; every wave is done with step s - 1
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        big_compute<FM, FN, KBB, kBigBM, UA>(smem + sl * kStage, wm, wn, lane, acc);
        sl = sl == 2 ? 0 : sl + 1;
    }

    if (e.C) {
        store_block32<FM, FN>(e, M, N, m0 + wm * (FM * 32), n0 + wn * (FN * 32), acc, lane);
    } else {
        // every wave has passed the last step's barrier, so only the stage
        // of step steps - 1 can still be read: the other two hold the
        // waves' output tiles (32 FM x 32 FN halves each)
        constexpr int kTile = 32 * FM * 32 * FN * 2;
        static_assert(kCompute * kTile <= 2 * kStage, "epilogue tiles");
        uint8_t *fr0 = smem + (steps % 3) * kStage, *fr1 = smem + ((steps + 1) % 3) * kStage;
        const int per0 = kStage / kTile;
        uint8_t *t = wave < per0 ? fr0 + wave * kTile : fr1 + (wave - per0) * kTile;
        store_block_lds<32, FM, FN>(e, M, N, m0 + wm * (FM * 32), n0 + wn * (FN * 32), acc, lane,
                                  reinterpret_cast<f16 *>(t));
    }
}

// ---------------------------------------------------------------------------
// Square-tile kernel for large M x N: 256 x 256 block per workgroup of 8
// waves (2 x 4), each a 128 x 64 compute tile of 32x32x32 int8 MFMAs.  The
// accumulators of a 256 x 256 tile fill half the CU's register file, which
// leaves no room for producer waves (VGPRs are allocated per wave at the
// kernel's count), so every wave issues an eighth of the DMA itself: 8
// buffer -> LDS instructions per 128-byte K step, into a 2-stage ring
// (2 x 64 KiB; the next step's DMA lands while this one is multiplied).
// Against the 256 x 128 tile this moves a third fewer operand bytes from L2
// into LDS per MFMA op, the data movement that sets the large-M GEMM's
// power draw (measured 369 vs 459 us at M = 8192, K = 14336, N = 4096; 64-
// byte steps in 2-4 stages: 397-410 us).  Stage layout, swizzle and
// fragment reads are gemm_big_kernel's (big_compute).  (Split-K over two
// workgroups per tile for grids below 256 tiles was measured and dropped:
// at M = 2048, N = 4096 it took 120 us without any partial exchange -- the
// 256 x 128 kernel takes 108-113 -- and 200 us with the device-scope
// fences the exchange needs, which write back and invalidate the XCD's L2
// under the other workgroups' operand panels.)

constexpr int kSqBM = 256, kSqBN = 256;
constexpr int kSqRows = kSqBM + kSqBN;

template <int KBB, int NSTG, bool UA>
__global__ __launch_bounds__(512, 1) void gemm_sq_kernel(const uint8_t *__restrict__ A,
                                                        const uint8_t *__restrict__ B,
                                                        int64_t M, int64_t N, int64_t K, Epi e) {
    constexpr int FM = 4, FN = 2, WGN = 4, kWaves = 8;
    constexpr int kStage = kSqRows * KBB;
    constexpr int kRowsPerDma = 1024 / KBB;               // rows per 1 KiB DMA block
    constexpr int kDma = kSqRows / kRowsPerDma;           // DMA blocks per stage
    constexpr int kDmaPerWave = kDma / kWaves;
    static_assert(kDmaPerWave * kWaves == kDma, "DMA split");
    static_assert(NSTG >= 2 && NSTG <= 4, "vmcnt waits below cover 0 .. 2 steps ahead");
    static_assert(NSTG * kStage <= 160 * 1024, "LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NSTG * kStage];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t tile = blockIdx.x;
    // XCD-aware tile order, as in gemm_big_kernel
    const int64_t tiles_m = (M + kSqBM - 1) / kSqBM;
    const int64_t tiles_n = (N + kSqBN - 1) / kSqBN;
    int64_t m0, n0;
    if (tiles_m % 4 == 0 && tiles_n % 2 == 0) {
        const int64_t x = tile % 8, i = tile / 8;
        const int64_t bm = tiles_m / 4, bn = tiles_n / 2;
        m0 = ((x % 4) * bm + i / bn) * kSqBM;
        n0 = ((x / 4) * bn + i % bn) * kSqBN;
    } else {
        m0 = (tile / tiles_n) * kSqBM;
        n0 = (tile % tiles_n) * kSqBN;
    }
    const int64_t KB = K / 2;
    const int steps = (int)((KB + KBB - 1) / KBB);

    // DMA block i = kDmaPerWave * wave + q covers stage rows R i .. R i + R - 1
    // (R = kRowsPerDma): lane l fetches chunk (l % C) ^ f(r) of row
    // r = R i + l / C; rows outside the matrix and chunks past the K tail
    // read as zeros (offset kOob)
    const __amdgpu_buffer_rsrc_t ar = make_rsrc(A, M * KB), br = make_rsrc(B, N * KB);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)smem;
    constexpr int C = KBB / 16;
    uint32_t roff[kDmaPerWave];
    int jc[kDmaPerWave];
#pragma unroll
    for (int q = 0; q < kDmaPerWave; ++q) {
        const int i = wave * kDmaPerWave + q;
        const int r = kRowsPerDma * i + lane / C;
        jc[q] = ((lane % C) ^ swz<KBB>(r)) * 16;
        const bool isa = kRowsPerDma * i < kSqBM;
        const int64_t row = isa ? m0 + r : n0 + r - kSqBM;
        roff[q] = row < (isa ? M : N) ? (uint32_t)(row * KB) : kOob;
    }
    auto issue = [&](int st) {
        const int64_t kb0 = (int64_t)st * KBB;
        const bool tail = kb0 + KBB > KB;
        const int sl = st % NSTG;
#pragma unroll
        for (int q = 0; q < kDmaPerWave; ++q) {
            const int i = wave * kDmaPerWave + q;
            const uint32_t dst = lds0 + sl * kStage + i * 1024;
            uint32_t off = roff[q] == kOob ? kOob : roff[q] + (uint32_t)kb0 + jc[q];
            if (tail && kb0 + jc[q] >= KB) off = kOob;
            dma16(kRowsPerDma * i < kSqBM ? ar : br, off, dst);
        }
    };
#pragma unroll
    for (int p = 0; p < NSTG - 1; ++p)
        if (p < steps) issue(p);

    const int wm = wave / WGN, wn = wave % WGN;
    v16i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = (v16i){};
    for (int s = 0; s < steps; ++s) {
        // this wave's DMA of step s is done; the steps after it that were
        // issued may stay in flight (vmcnt counts the wave's DMA in order)
        const int ahead = min(NSTG - 2, steps - 1 - s);
        if (ahead >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kDmaPerWave) : "memory");
        else if (ahead == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerWave) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // every wave's DMA of step s has landed, and every wave is done with
        // step s - 1, whose stage step s + NSTG - 1 now overwrites
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + NSTG - 1 < steps) issue(s + NSTG - 1);
        big_compute<FM, FN, KBB, kSqBM, UA>(smem + (s % NSTG) * kStage, wm, wn, lane, acc);
    }
    if (e.C) {
        store_block32<FM, FN>(e, M, N, m0 + wm * (FM * 32), n0 + wn * (FN * 32), acc, lane);
    } else {
        // every wave is past its last step and no DMA is in flight (the
        // last step waited for vmcnt 0): the whole ring is free for the
        // waves' epilogue tiles
        constexpr int kTile = 32 * FM * 32 * FN * 2;
        static_assert(kWaves * kTile <= NSTG * kStage, "epilogue tiles");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        store_block_lds<32, FM, FN>(e, M, N, m0 + wm * (FM * 32), n0 + wn * (FN * 32), acc, lane,
                                    reinterpret_cast<f16 *>(smem + wave * kTile));
    }
}

// ---------------------------------------------------------------------------
// Ring kernel for mid-size M: BM x BN tile per workgroup, 4 compute waves
// (2 x 2) of 16x16x64 int8 MFMA blocks and 2 producer waves moving the
// tile's rows through an NSTG-stage LDS ring (buffer -> LDS DMA, 128 bytes =
// 256 codes per row per step, 8 rows per 1 KiB DMA block).  A small tile
// does little MFMA work per loaded byte, so the kernel is bound by data
// movement; the deep ring keeps NSTG - 1 steps in flight to cover the
// HBM latency of the weight stream.  Stage layout and swizzle are the
// large-M kernel's (16-byte chunk j of row r at j ^ swz(r)); out-of-range
// rows and the K tail read as zeros.

constexpr int kRingKBB = 128;

// this wave's DMA of step s is done while `later` more of its steps (PER
// DMA instructions each) may stay in flight; vmcnt takes an immediate
template <int PER, int MAXL>
SRQ_DEV void ring_wait(int later) {
    if constexpr (MAXL > 0) {
        if (later >= MAXL) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(MAXL * PER) : "memory");
            return;
        }
        ring_wait<PER, MAXL - 1>(later);
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
}

template <int BM, int BN, int NSTG, int NPROD, bool UA>
__global__ __launch_bounds__(64 * (4 + NPROD), 1) void gemm_ring_kernel(const uint8_t *__restrict__ A,
                                                           const uint8_t *__restrict__ B,
                                                           int64_t M, int64_t N, int64_t K,
                                                           Epi e) {
    constexpr int KBB = kRingKBB;
    constexpr int kRows = BM + BN;
    constexpr int kStage = kRows * KBB;
    constexpr int kDma = kRows / 8;  // 1 KiB DMA blocks per stage
    constexpr int kPer = kDma / NPROD;
    static_assert(kPer * NPROD == kDma && kRows % 8 == 0, "DMA split");
    static_assert((NSTG - 2) * kPer <= 63, "vmcnt range");
    static_assert(NSTG * kStage <= 160 * 1024, "LDS ring");
    constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 16, FN = WN / 16;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NSTG * kStage];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // XCD-aware tile order: consecutive workgroups land on different XCDs
    // (round-robin dispatch), so give each XCD a contiguous range of tiles
    const int64_t tiles_n = (N + BN - 1) / BN;
    const int64_t tiles = ((M + BM - 1) / BM) * tiles_n;
    int64_t t = blockIdx.x;
    if (tiles % 8 == 0) t = (t % 8) * (tiles / 8) + t / 8;
    const int64_t m0 = (t / tiles_n) * BM, n0 = (t % tiles_n) * BN;
    const int64_t KB = K / 2;
    const int steps = (int)((KB + KBB - 1) / KBB);

    if (wave >= 4) {
        // ---- producer pw: DMA blocks i = kPer pw + q, stage rows 8 i .. 8 i
        // + 7; lane l fetches chunk (l % 8) ^ swz(r) of row r = 8 i + l / 8
        const int pw = wave - 4;
        const __amdgpu_buffer_rsrc_t ar = make_rsrc(A, M * KB), br = make_rsrc(B, N * KB);
        const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)smem;
        uint32_t roff[kPer];
        int jc[kPer];
#pragma unroll
        for (int q = 0; q < kPer; ++q) {
            const int i = pw * kPer + q;
            const int r = 8 * i + lane / 8;
            jc[q] = ((lane % 8) ^ swz<KBB>(r)) * 16;
            const bool isa = 8 * i < BM;
            const int64_t row = isa ? m0 + r : n0 + r - BM;
            roff[q] = row < (isa ? M : N) ? (uint32_t)(row * KB) : kOob;
        }
        auto issue = [&](int st) __attribute__((always_inline)) {
            const int64_t kb0 = (int64_t)st * KBB;
            const bool tail = kb0 + KBB > KB;
            const uint32_t dst0 = lds0 + (st % NSTG) * kStage;
#pragma unroll
            for (int q = 0; q < kPer; ++q) {
                const int i = pw * kPer + q;
                uint32_t off = roff[q] == kOob ? kOob : roff[q] + (uint32_t)kb0 + jc[q];
                if (tail && kb0 + jc[q] >= KB) off = kOob;
                dma16(8 * i < BM ? ar : br, off, dst0 + i * 1024);
            }
        };
#pragma unroll
        for (int s = 0; s < NSTG - 1; ++s)
            if (s < steps) issue(s);
        for (int s = 0; s < steps; ++s) {
            // this wave's DMA of step s is done; every producer's after the
            // barrier, and every compute wave is done with step s - 1's stage
            const int later = steps - 1 - s < NSTG - 2 ? steps - 1 - s : NSTG - 2;
            ring_wait<kPer, NSTG - 2>(later);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (s + NSTG - 1 < steps) issue(s + NSTG - 1);
        }
        return;  // the compute waves meet no barrier after their K loop
    }

    // ---- compute wave (wm, wn): FM x FN blocks of 16 x 16; lane reads 8
    // bytes (16 codes) of row (lane & 15) at byte 32 kk + 8 (lane >> 4)
    const int wm = wave >> 1, wn = wave & 1;
    v4i acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = (v4i){0, 0, 0, 0};
    const int frow = lane & 15;
    const int fsub = ((lane >> 4) & 1) * 8;  // byte inside the 16-byte chunk
    const int fch = lane >> 5;                // chunk 2 kk + fch
    auto rd = [&](const uint8_t *stage, int r, int kk) __attribute__((always_inline)) {
        return *reinterpret_cast<const uint2 *>(
            stage + r * KBB + (((2 * kk + fch) ^ swz<KBB>(r)) << 4) + fsub);
    };
    for (int s = 0; s < steps; ++s) {
        // step s has landed; every wave is done with step s - 1
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        const uint8_t *stage = smem + (s % NSTG) * kStage;
        uint2 wa[2][FM], wb[2][FN];
        auto fetch = [&](int kk, int slot) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < FM; ++i) wa[slot][i] = rd(stage, wm * WM + i * 16 + frow, kk);
#pragma unroll
            for (int j = 0; j < FN; ++j) wb[slot][j] = rd(stage, BM + wn * WN + j * 16 + frow, kk);
        };
        fetch(0, 0);
#pragma unroll
        for (int kk = 0; kk < KBB / 32; ++kk) {
            if (kk + 1 < KBB / 32) fetch(kk + 1, (kk + 1) & 1);
            v4i fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) fa[i] = unpack8a<UA>(wa[kk & 1][i].x, wa[kk & 1][i].y);
#pragma unroll
            for (int j = 0; j < FN; ++j) fb[j] = unpack8(wb[kk & 1][j].x, wb[kk & 1][j].y);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = mfma16(fa[i], fb[j], acc[i][j]);
        }
    }
    if (e.C) {
        store_block<FM, FN>(e, M, N, m0 + wm * WM, n0 + wn * WN, acc, lane);
    } else {
        // after the barrier of the last step no DMA is in flight and the
        // waves read only that step's stage, (steps - 1) % NSTG; the next
        // one holds the compute waves' epilogue tiles
        constexpr int kTile = WM * WN * 2;
        static_assert(NSTG >= 2 && 4 * kTile <= kStage, "epilogue tiles");
        uint8_t *fr = smem + (steps % NSTG) * kStage;
        store_block_lds<16, FM, FN>(e, M, N, m0 + wm * WM, n0 + wn * WN, acc, lane,
                                    reinterpret_cast<f16 *>(fr + wave * kTile));
    }
}

// ---------------------------------------------------------------------------
// Skinny kernel for small M (decode / short prefill): weight streaming.
// A workgroup of KW waves owns 16 output columns and MB x 16 rows; wave w
// takes the w-th slice of K.  Each lane loads 16 bytes (32 codes) of B per
// 128-code step straight from HBM (no LDS: every byte of B is used by
// exactly one wave), U steps in flight; the slices' int32 partials are
// summed through LDS (exact).

template <int MB, int KW, int U, bool UA>
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
    const __amdgpu_buffer_rsrc_t ar = make_rsrc(A, M * KB), br = make_rsrc(B, N * KB);

    v4i acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = (v4i){0, 0, 0, 0};

    for (int64_t s = s0; s < s1; s += U) {
        v4i wb[U], wa[U][MB];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t kbyte = (s + u < s1) ? (s + u) * 64 + kb : KB;
            wb[u] = bload16(br, chunk_off(bn, N, kbyte, KB));
#pragma unroll
            for (int i = 0; i < MB; ++i)
                wa[u][i] = bload16(ar, chunk_off(m0 + i * 16 + (lane & 15), M, kbyte, KB));
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const v4i b0 = unpack8((u32)wb[u][0], (u32)wb[u][1]);
            const v4i b1 = unpack8((u32)wb[u][2], (u32)wb[u][3]);
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const v4i a0 = unpack8a<UA>((u32)wa[u][i][0], (u32)wa[u][i][1]);
                const v4i a1 = unpack8a<UA>((u32)wa[u][i][2], (u32)wa[u][i][3]);
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


// ---------------------------------------------------------------------------
// Stream kernel for M <= 32 (decode): weight streaming at the HBM roofline's
// access pattern, with the activation loaded once per workgroup.
//
// Persistent grid of G <= 256 workgroups of KW = 8 waves; workgroup b owns
// column blocks (16 output columns each) b, b + G, ...  The K dimension is
// cut into units of 128 bytes (256 codes) per row; wave w owns units
// [w*per, (w+1)*per) of every column block.
//
// * A (M rows x the wave's units) is loaded once into registers in the MFMA
//   operand layout: read line-friendly (8 rows x 128 B per instruction) and
//   transposed through LDS.  Re-reading it per column block from L2 in the
//   operand layout (16 rows x 16 B per quarter-wave) costs more L1 tag
//   lookups than the weight stream itself.
// * B streams through a per-wave ring of S LDS stages of 16 rows x 128 B by
//   direct-to-LDS loads (no VGPR staging), S-1 items in flight.  Each
//   16-lane quarter-wave fetches two whole 128-byte lines; lane p of a row
//   fetches logical 16-byte chunk p ^ (row & 7), which makes the MFMA-layout
//   reads (lane l: row l & 15, chunk 4t + (l >> 4)) bank-conflict-free.
// * Per column block, each wave's partial sums go into that block's LDS
//   int32 buffer with integer atomic adds (exact and order-independent) and
//   the wave moves on: no barrier inside the stream (a barrier per block cost
//   a third of the time at decode shapes).  After the last block, one
//   barrier, then wave w dequantizes and stores blocks w, w + KW, ...
constexpr int kStreamKW = 8;
constexpr int kStreamS = 4;
constexpr int kStreamMaxCb = 16;   // column blocks per workgroup

// MoE rows past an expert's full 128-row tiles: when an expert has more
// than one tile and its last tile would hold 1..64 rows, those rows ride on
// its last full tile instead (the grouped kernel's compute waves multiply
// them with the B operands they unpack for that tile; the producer waves
// stage their codes), so no mostly empty tile streams the expert's weights
// a second time (cfg5: the down launch's 320 tiles for 256 CUs become 256).
constexpr int kMoeTile = 128, kMoeRemMax = 64;
SRQ_DEV int64_t moe_tiled_rows(int64_t r) {
    const int64_t q = r % kMoeTile;
    return (r > kMoeTile && q > 0 && q <= kMoeRemMax) ? r - q : r;
}

template <int MB, int NSUB, bool AUNP, bool UA, bool BATCH = false>
__global__ __launch_bounds__(kStreamKW * 64) void gemm_stream_kernel(
    const uint8_t *__restrict__ A, const uint8_t *__restrict__ B, int64_t M, int64_t N,
    int64_t K, Epi e) {
    constexpr int KW = kStreamKW, S = kStreamS;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[KW * S * 2048];
    __shared__ int sum[kStreamMaxCb][MB * 256];
    __shared__ float sbl[kStreamMaxCb * 16];
    __shared__ float sal[MB * 16];
    // BATCH: the A transposes after the first batch go through this area
    // (the ring then holds weight items in flight)
    __shared__ __attribute__((aligned(16))) uint8_t astage[BATCH ? KW * MB * 2048 : 16];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t KB = K / 2;
    const int units = (int)((KB + 127) / 128);
    const int per = (units + KW - 1) / KW;
    const int u0 = wave * per;
    const int nsub = max(0, min(per, units - u0));
    // BATCH: the wave's units in batches of NSUB (A of one batch in
    // registers at a time); a batch's units past nsub read as zeros
    const int nbat = BATCH ? (per + NSUB - 1) / NSUB : 1;
    const int ncb = (int)((N + 15) / 16);
    const int G = gridDim.x;
    const int ncb_mine = (ncb - (int)blockIdx.x + G - 1) / G;
    const __amdgpu_buffer_rsrc_t ar = make_rsrc(A, M * KB), br = make_rsrc(B, N * KB);

    for (int t = threadIdx.x; t < ncb_mine * MB * 256; t += KW * 64) (&sum[0][0])[t] = 0;
    if (!e.C) {
        for (int t = threadIdx.x; t < MB * 16; t += KW * 64) sal[t] = t < M ? (float)e.sa[t] : 0.f;
        for (int t = threadIdx.x; t < ncb_mine * 16; t += KW * 64) {
            const int64_t n = (int64_t)(blockIdx.x + (t >> 4) * G) * 16 + (t & 15);
            sbl[t] = n < N ? (float)e.sb[n] : 0.f;
        }
    }

    // The residual (and bias) of the first column block this wave stores
    // (j = wave), fetched now so the epilogue after the stream does not wait
    // a memory round trip for them.
    const int rr = lane & 15;
    f16 res0[MB][4], bias0 = (f16)0;
    if (!e.C && wave < ncb_mine) {
        const int64_t gn = (int64_t)(blockIdx.x + wave * G) * 16 + rr;
        if (e.bias && gn < N) bias0 = e.bias[gn];
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = i * 16 + 4 * (lane >> 4) + r;
                res0[i][r] = (e.res && m < M && gn < N) ? e.res[m * N + gn] : (f16)0;
            }
    }

    // A: unit s of the wave's batch bt, row block i, chunk pair t; lane
    // holds row 16 i + (lane & 15), logical chunk 4 t + (lane >> 4) of the
    // unit, read line-friendly and transposed through the wave's staging
    // area tb
    v4i areg[NSUB][MB][2];
    v4i aun[AUNP ? NSUB : 1][MB][2][2];
    auto load_a = [&](int bt, uint8_t *tb) __attribute__((always_inline)) {
        v4i raw[NSUB][MB][2];
#pragma unroll
        for (int s = 0; s < NSUB; ++s)
#pragma unroll
            for (int h = 0; h < 2 * MB; ++h) {
                const int64_t row = 8 * h + (lane >> 3);
                const int su = bt * NSUB + s;
                const int64_t kb = (int64_t)(u0 + su) * 128 + 16 * (lane & 7);
                const bool ok = su < nsub && row < M && kb < KB;
                raw[s][h >> 1][h & 1] = bload16(ar, ok ? (uint32_t)(row * KB + kb) : kOob);
            }
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
#pragma unroll
            for (int h = 0; h < 2 * MB; ++h) {
                const int row = 8 * h + (lane >> 3);
                *(v4i *)(tb + row * 128 + 16 * ((lane & 7) ^ (row & 7))) = raw[s][h >> 1][h & 1];
            }
#pragma unroll
            for (int i = 0; i < MB; ++i)
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int row = 16 * i + (lane & 15);
                    areg[s][i][t] =
                        *(const v4i *)(tb + row * 128 + 16 * ((4 * t + (lane >> 4)) ^ (row & 7)));
                }
            // this wave's reads of unit s land before unit s + 1 overwrites the slot
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        }
#pragma unroll
        for (int s = 0; s < NSUB; ++s)
#pragma unroll
            for (int i = 0; i < MB; ++i)
#pragma unroll
                for (int t = 0; t < 2; ++t) asm volatile("" : "+v"(areg[s][i][t]));
        if (AUNP) {
#pragma unroll
            for (int s = 0; s < (AUNP ? NSUB : 1); ++s)
#pragma unroll
                for (int i = 0; i < MB; ++i)
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        aun[s][i][t][0] = unpack8a<UA>((u32)areg[s][i][t][0], (u32)areg[s][i][t][1]);
                        aun[s][i][t][1] = unpack8a<UA>((u32)areg[s][i][t][2], (u32)areg[s][i][t][3]);
                    }
        }
    };
    load_a(0, ring + wave * (S * 2048));
    __syncthreads();

    // item = (batch, column block j, unit s); DMA instruction h covers rows
    // 8 h + (lane >> 3).  Without batching the items are (j, s < nsub);
    // with it every batch has NSUB units (those past nsub load zeros).
    const uint32_t ring_w = (uint32_t)(uintptr_t)ring + (uint32_t)wave * (S * 2048);
    const int per_bat = BATCH ? ncb_mine * NSUB : ncb_mine * nsub;
    const int total = per_bat * nbat;
    auto issue = [&](int item) {
        const uint32_t lds = ring_w + (item % S) * 2048;
        int64_t nrow0 = 0, kb0 = 0;
        bool live = item < total;
        if (live) {
            int j, su;
            if (BATCH) {
                const int bt = item / per_bat, rem = item - bt * per_bat;
                j = rem / NSUB;
                su = bt * NSUB + (rem - j * NSUB);
                live = su < nsub;
            } else {
                j = item / nsub;
                su = item - j * nsub;
            }
            nrow0 = (int64_t)(blockIdx.x + j * G) * 16;
            kb0 = (int64_t)(u0 + su) * 128;
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int r = 8 * h + (lane >> 3);
            const int64_t row = nrow0 + r;
            const int64_t kb = kb0 + 16 * ((lane & 7) ^ (r & 7));
            const uint32_t off = (live && row < N && kb < KB) ? (uint32_t)(row * KB + kb) : kOob;
            dma16(br, off, __builtin_amdgcn_readfirstlane(lds + h * 1024));
        }
    };

    v4i acc[MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) acc[i] = (v4i){0, 0, 0, 0};
#pragma unroll
    for (int it = 0; it < S - 1; ++it) issue(it);

    for (int bt = 0; bt < nbat; ++bt) {
        // the next batch's A (the items already in flight keep streaming)
        if (BATCH && bt > 0) load_a(bt, astage + wave * (MB * 2048));
        for (int j = 0; j < ncb_mine; ++j) {
#pragma unroll
            for (int s = 0; s < NSUB; ++s) {
                if (!BATCH && s >= nsub) break;
                const int it = bt * per_bat + j * (BATCH ? NSUB : nsub) + s;
                issue(it + S - 1);  // items past the end load zeros into a free stage
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * (S - 1)) : "memory");
                const uint8_t *st = ring + wave * (S * 2048) + (it % S) * 2048 + 128 * rr;
                v4i bw[2];
#pragma unroll
                for (int t = 0; t < 2; ++t)
                    bw[t] = *(const v4i *)(st + 16 * ((4 * t + (lane >> 4)) ^ (rr & 7)));
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const v4i b0 = unpack8((u32)bw[t][0], (u32)bw[t][1]);
                    const v4i b1 = unpack8((u32)bw[t][2], (u32)bw[t][3]);
#pragma unroll
                    for (int i = 0; i < MB; ++i) {
                        v4i a0, a1;
                        if (AUNP) {
                            a0 = aun[AUNP ? s : 0][i][t][0];
                            a1 = aun[AUNP ? s : 0][i][t][1];
                        } else {
                            v4i w = areg[s][i][t];
                            asm volatile("" : "+v"(w));  // unpack per use, not hoisted out of j
                            a0 = unpack8a<UA>((u32)w[0], (u32)w[1]);
                            a1 = unpack8a<UA>((u32)w[2], (u32)w[3]);
                        }
                        acc[i] = mfma16(a0, b0, acc[i]);
                        acc[i] = mfma16(a1, b1, acc[i]);
                    }
                }
            }
            if (nsub > 0) {
                int *sm = sum[j];
#pragma unroll
                for (int i = 0; i < MB; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        __hip_atomic_fetch_add(&sm[i * 256 + (4 * (lane >> 4) + r) * 16 + rr],
                                               acc[i][r], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_WORKGROUP);
            }
#pragma unroll
            for (int i = 0; i < MB; ++i) acc[i] = (v4i){0, 0, 0, 0};
        }
    }
    // the zero-fill DMAs of items past the end land before the block ends
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (e.swiglu) {
        // lane rr < 8: output column 8 c + rr of column block c from gate
        // column 16 c + rr and up column 16 c + rr + 8, each dequantized as
        // the plain fp16 epilogue does, then swiglu1
        for (int j = wave; j < ncb_mine; j += KW) {
            const int *sm = sum[j];
            const int64_t cb = blockIdx.x + (int64_t)j * G;
            const int c = rr & 7;
            const float sbg = sbl[j * 16 + c], sbu = sbl[j * 16 + c + 8];
#pragma unroll
            for (int i = 0; i < MB; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int m = i * 16 + 4 * (lane >> 4) + r;
                    const int base = i * 256 + (4 * (lane >> 4) + r) * 16;
                    if (rr < 8 && m < M && cb * 16 + 16 <= N) {
                        const f16 g = f16_rn(((float)(sm[base + c] >> 8) * sal[m]) * sbg);
                        const f16 u = f16_rn(((float)(sm[base + c + 8] >> 8) * sal[m]) * sbu);
                        e.out[m * (N / 2) + cb * 8 + c] = swiglu1((float)g, (float)u);
                    }
                }
        }
        return;
    }
    for (int j = wave; j < ncb_mine; j += KW) {
        const int *sm = sum[j];
        const int64_t gn = (int64_t)(blockIdx.x + j * G) * 16 + rr;
        const float sbv = e.C ? 0.f : sbl[j * 16 + rr];
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = i * 16 + 4 * (lane >> 4) + r;
                const int raw = sm[i * 256 + (4 * (lane >> 4) + r) * 16 + rr];
                if (m < M && gn < N) {
                    const int v = epi_val(e, raw, m, gn);
                    if (e.C) {
                        e.C[m * N + gn] = v;
                    } else {
                        const bool first = j == wave;
                        f16 o = f16_rn(((float)v * sal[m]) * sbv);
                        if (e.bias) o = f16_rn((float)o + (float)(first ? bias0 : e.bias[gn]));
                        if (e.res)
                            o = f16_rn((float)o + (float)(first ? res0[i][r] : e.res[m * N + gn]));
                        e.out[m * N + gn] = o;
                    }
                }
            }
    }
}

// Launch the stream kernel if the shape fits its register and LDS budget;
// returns false otherwise.
template <bool UA>
bool launch_stream(const uint8_t *a, const uint8_t *b, int64_t M, int64_t N, int64_t K,
                   const Epi &e, hipStream_t st) {
    if (M > 32) return false;
    const int64_t units = (K / 2 + 127) / 128;
    const int64_t per = (units + kStreamKW - 1) / kStreamKW;
    const int64_t ncb = (N + 15) / 16;
    const int64_t cb_per = (ncb + 255) / 256;
    if (cb_per > kStreamMaxCb) return false;
    const dim3 grid((unsigned)((ncb + cb_per - 1) / cb_per)), block(kStreamKW * 64);
#define SRQ_STREAM(MB, NSUB, AUNP, BATCH) \
    gemm_stream_kernel<MB, NSUB, AUNP, UA, BATCH><<<grid, block, 0, st>>>(a, b, M, N, K, e)
    // per > 8 units per wave (K > 16384): A goes through registers in
    // batches of NSUB units (cfg4 down at M = 1 / 32: 54 us on the skinny
    // kernel before)
    if (M <= 16) {
        if (per <= 2) SRQ_STREAM(1, 2, true, false);
        else if (per <= 4) SRQ_STREAM(1, 4, true, false);
        else if (per <= 8) SRQ_STREAM(1, 8, false, false);
        else SRQ_STREAM(1, 8, false, true);
    } else {
        if (per <= 2) SRQ_STREAM(2, 2, true, false);
        else if (per <= 4) SRQ_STREAM(2, 4, false, false);
        else if (per <= 7) SRQ_STREAM(2, 7, false, false);
        else if (per <= 8) SRQ_STREAM(2, 8, false, false);
        else SRQ_STREAM(2, 7, false, true);
    }
#undef SRQ_STREAM
    return true;
}

// ---------------------------------------------------------------------------
// Grouped GEMM (MoE experts): the producer/consumer structure of the large-M
// kernel with 128 x 128 tiles, made persistent.  The problem list lives in
// device memory only, so the launch needs no host read and is
// graph-capturable: every workgroup walks tiles t = blockIdx.x, +gridDim.x,
// ... of the concatenated per-problem tile lists (tiles of problem p follow
// those of p - 1, row-major within a problem), locating each tile's problem
// with a running prefix sum.  Producers and compute waves walk the same
// sequence, so their barrier counts agree: K steps plus one end-of-tile
// barrier per tile (after it the stages are free for the next tile's
// prologue), and one more before the K loop of a tile with extra rows
// (GroupedProb::xrows).  Rows past a problem's m and chunks past its k read
// as zeros.

constexpr int kGrpBM = 128, kGrpBN = 128;
static_assert(kGrpBM == kMoeTile, "the MoE remainder rule assumes the grouped kernel's tile rows");
constexpr int kGrpRows = kGrpBM + kGrpBN;
// 128-byte K steps in a 3-stage ring (4 stages measured the same: the
// kernel is not bound by DMA latency)
constexpr int kGrpKBB = 128, kGrpStages = 3;
// Persistent grid of the grouped kernel: one workgroup per CU (256 CUs).
constexpr int kGroupedGrid = 256;

struct GroupedArgs {
    int P;
    // pointer-array form (srq_matmul_grouped): problem p has sizes
    // (m, n, k) = sizes[3p .. 3p+2], operands at ptr_a[p] / ptr_b[p] with
    // row strides lda[p] / ldb[p] codes, int32 output at ptr_c[p] with row
    // stride ldc[p]
    const int32_t *sizes;
    const int64_t *pa, *pb, *pc, *lda, *ldb, *ldc;
    // expert-offset form (srq_w4a4_linear_moe): expert p owns rows
    // offsets[p] .. offsets[p + 1] of A [R, K/2]; B [P, N, K/2]; fp16 output
    // [R, N] = fp16((float(acc) * float(sa[row])) * float(sb[p, col]))
    const int32_t *offsets;
    const uint8_t *A, *B;
    int64_t N, K;
    // expert-offset forms with symmetric A and at least two K steps: an
    // expert's rows past its full tiles (moe_tiled_rows) ride on its last
    // full tile (GroupedProb::xrows)
    int skip_rem;
    const f16 *sa, *sb;
    f16 *out;
    // asymmetric activations (expert-offset form, unsigned A): zero point per
    // row [R] and per-expert weight row sums [P, N]
    const int8_t *zr;
    const int32_t *ws;
    // paired expert-offset form (srq_w4a4_linear_moe_gate_up): 2 P problems,
    // problem q = expert q / 2 times B (q even) or B2 (q odd), into out /
    // out2 with sb / sb2 (and ws / ws2); both share the expert's A rows
    int pair;
    const uint8_t *B2;
    const f16 *sb2;
    f16 *out2;
    const int32_t *ws2;
    // dense form (the DENSE instantiation): one problem, A [M, K/2] times
    // B [N, K/2], fp16 out [M, N] with the dense epilogue's bias [N] and
    // residual [M, N] (either may be null)
    int64_t M;
    const f16 *bias, *res;
    int swiglu;  // dense form: the columns are blocks of 8 gate, 8 up; out [M, N/2]
    int64_t ldo;  // dense swiglu form: Epi::ldo
    // split-K form (the SPLITK instantiation): problem p is the dense
    // product over K codes [p Kc, min((p + 1) Kc, K)), its int32 partial
    // (shifted down like the dense accumulator) at ws_c + p M N
    int64_t Kc;
    int32_t *ws_c;
};

// kFormSwiglu: the expert-offset form over gate/up rows interleaved in
// blocks of 8, out [R, N/2] = swiglu(gate, up)
constexpr int kFormGeneral = 0, kFormDense = 1, kFormSplitK = 2, kFormSwiglu = 3;

struct GroupedProb {
    const uint8_t *a, *b;
    int32_t *c;
    int64_t m, n, k, lda_b, ldb_b, ldc, row0;
    // rows m .. m + xrows - 1 of the problem (at most kMoeRemMax), computed
    // on its last M tile
    int64_t xrows;
};

SRQ_DEV int64_t uni(int64_t v) {
    return (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(v >> 32)) << 32) |
                     (uint32_t)__builtin_amdgcn_readfirstlane((int)v));
}

template <int FORM>
SRQ_DEV GroupedProb grouped_prob(const GroupedArgs &g, int p) {
    GroupedProb r;
    r.xrows = 0;
    if constexpr (FORM == kFormSplitK) {
        const int64_t kc0 = (int64_t)p * g.Kc;
        r.row0 = 0;
        r.m = g.M;
        r.n = g.N;
        r.k = g.K - kc0 < g.Kc ? g.K - kc0 : g.Kc;
        r.lda_b = r.ldb_b = g.K / 2;
        r.a = g.A + kc0 / 2;
        r.b = g.B + kc0 / 2;
        r.c = g.ws_c + (int64_t)p * g.M * g.N;
        r.ldc = g.N;
        return r;
    }
    if constexpr (FORM == kFormDense) {
        r.row0 = 0;
        r.m = g.M;
        r.n = g.N;
        r.k = g.K;
        r.lda_b = r.ldb_b = g.K / 2;
        r.a = g.A;
        r.b = g.B;
        r.c = nullptr;
        r.ldc = g.N;
        return r;
    }
    if (g.sizes) {
        r.m = uni(g.sizes[3 * p]);
        r.n = uni(g.sizes[3 * p + 1]);
        r.k = uni(g.sizes[3 * p + 2]);
        r.a = (const uint8_t *)uni(g.pa[p]);
        r.b = (const uint8_t *)uni(g.pb[p]);
        r.c = (int32_t *)uni(g.pc[p]);
        r.lda_b = uni(g.lda[p]) / 2;
        r.ldb_b = uni(g.ldb[p]) / 2;
        r.ldc = uni(g.ldc[p]);
        r.row0 = 0;
    } else {
        const int e = g.pair ? p >> 1 : p;
        r.row0 = uni(g.offsets[e]);
        r.m = uni(g.offsets[e + 1]) - r.row0;
        if (g.skip_rem) {
            const int64_t t = moe_tiled_rows(r.m);
            r.xrows = r.m - t;
            r.m = t;
        }
        r.n = g.N;
        r.k = g.K;
        r.lda_b = r.ldb_b = g.K / 2;
        r.a = g.A + r.row0 * r.lda_b;
        r.b = ((g.pair && (p & 1)) ? g.B2 : g.B) + (int64_t)e * g.N * r.ldb_b;
        r.c = nullptr;
        r.ldc = g.N;
    }
    return r;
}

SRQ_DEV int64_t grouped_tiles(const GroupedProb &r) {
    if (r.m <= 0 || r.n <= 0) return 0;
    return ((r.m + kGrpBM - 1) / kGrpBM) * ((r.n + kGrpBN - 1) / kGrpBN);
}

template <int NPROD, bool UA, int FORM = kFormGeneral, int NSTG = kGrpStages>
__global__ __launch_bounds__(64 * (4 + NPROD), 1) void gemm_grouped_kernel(GroupedArgs g) {
    constexpr int WGN = 2, FM = 2, FN = 2, KBB = kGrpKBB;
    static_assert(KBB == 128, "stage layout validated for 128-byte steps only");
    constexpr int kCompute = 4;
    constexpr int kStage = kGrpRows * KBB;
    constexpr int C = KBB / 16;           // 16-byte chunks per row
    constexpr int R = 1024 / KBB;         // rows per 1 KiB DMA block
    constexpr int kDma = kGrpRows / R;
    constexpr int kDmaPerWave = kDma / NPROD;
    static_assert(kDmaPerWave * NPROD == kDma, "DMA split");
    static_assert(NSTG >= 2 && (NSTG - 2) * kDmaPerWave <= 63, "vmcnt range");
    constexpr int kEpiTile = 4 * 32 * FN * 32 * FM;  // a compute wave's int32 block
    static_assert(NSTG * kStage + kCompute * kEpiTile <= 160 * 1024, "LDS ring");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NSTG * kStage];
    __shared__ __attribute__((aligned(16))) uint8_t epi_lds[kCompute * kEpiTile];

    const int lane0 = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool producer = wave >= kCompute;
    const int pw = wave - kCompute;
    const int wm = wave / WGN, wn = wave % WGN;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)smem;

    int p = 0;
    int64_t pstart = 0;
    GroupedProb pr = grouped_prob<FORM>(g, 0);
    int64_t ptiles = grouped_tiles(pr);
    for (int64_t t = blockIdx.x;; t += gridDim.x) {
        while (p < g.P && t >= pstart + ptiles) {
            pstart += ptiles;
            ++p;
            if (p < g.P) {
                pr = grouped_prob<FORM>(g, p);
                ptiles = grouped_tiles(pr);
            }
        }
        if (p >= g.P) break;
        // lane laundered per tile: its derived LDS addresses are recomputed
        // per tile, not held across the tile loop by both wave roles (that
        // left the producers' extra-row code without registers)
        int lane = lane0;
        asm volatile("" : "+v"(lane));
        const int64_t tiles_n = (pr.n + kGrpBN - 1) / kGrpBN;
        const int64_t local = t - pstart;
        const int64_t m0 = (local / tiles_n) * kGrpBM, n0 = (local % tiles_n) * kGrpBN;
        const int64_t KB = pr.k / 2;
        const int steps = (int)((KB + KBB - 1) / KBB);
        // the expert's last full tile, with its extra rows (signed
        // expert-offset forms; the host asks for them only with two or more
        // K steps)
        constexpr bool kExtra = !UA && (FORM == kFormGeneral || FORM == kFormSwiglu);
        const bool xt = kExtra && pr.xrows > 0 && m0 + kGrpBM == pr.m;

        if (producer) {
            // (wave-uniform, stated: the tile loop's divergent epilogues can
            // hide it from the compiler, which then puts them in VGPRs)
            const __amdgpu_buffer_rsrc_t ar =
                make_rsrc((const uint8_t *)uni((int64_t)pr.a), uni(pr.m * pr.lda_b));
            const __amdgpu_buffer_rsrc_t br =
                make_rsrc((const uint8_t *)uni((int64_t)pr.b), uni(pr.n * pr.ldb_b));
            uint32_t roff[kDmaPerWave];
            int jc[kDmaPerWave];
            // 1 KiB block of DMA q of this wave: its A rows then its B rows,
            // 32 pw .. 32 pw + 31 of each, of the stage
            constexpr int kAPer = kGrpBM / R / NPROD, kBPer = kGrpBN / R / NPROD;
            static_assert(kAPer + kBPer == kDmaPerWave && kBPer * R == 32, "DMA blocks");
            auto blk = [&](int q) {
                return q < kAPer ? kAPer * pw + q : kGrpBM / R + kBPer * pw + (q - kAPer);
            };
#pragma unroll
            for (int q = 0; q < kDmaPerWave; ++q) {
                const int i = blk(q);
                const int r = R * i + lane / C;
                jc[q] = ((lane % C) ^ swz<KBB>(r)) * 16;
                const bool isa = q < kAPer;
                const int64_t row = isa ? m0 + r : n0 + r - kGrpBM;
                roff[q] = row < (isa ? pr.m : pr.n)
                              ? (uint32_t)(row * (isa ? pr.lda_b : pr.ldb_b)) : kOob;
            }
            auto issue = [&](int st, int sl) {
                const int64_t kb0 = (int64_t)st * KBB;
                const bool tail = kb0 + KBB > KB;
                auto one = [&](int q, __amdgpu_buffer_rsrc_t rs) __attribute__((always_inline)) {
                    const uint32_t dst = lds0 + sl * kStage + blk(q) * 1024;
                    uint32_t off = roff[q] == kOob ? kOob : roff[q] + (uint32_t)kb0 + jc[q];
                    if (tail && kb0 + jc[q] >= KB) off = kOob;
                    dma16(rs, off, dst);
                };
#pragma unroll
                for (int q = 0; q < kAPer; ++q) one(q, ar);
#pragma unroll
                for (int q = kAPer; q < kDmaPerWave; ++q) one(q, br);
            };
#pragma unroll
            for (int q = 0; q < NSTG - 1; ++q)
                if (q < steps) issue(q, q);
            if (kExtra && xt) {
                // The expert's rows past its full tiles (1..64; at least two K
                // steps): the compute waves multiply them with the B operands
                // they unpack for the tile.  Their codes stream into NSTG
                // 8 KiB slots of the epilogue area (idle during the K loop),
                // two 1 KiB DMAs (8 rows each) per producer per step in the
                // stage layout, waited before barrier s like step s's stage.  The
                // area is free once the compute waves' previous epilogue is
                // done: on such a tile every wave meets one more barrier
                // before the K loop, after which steps 0 and 1's codes load.
                constexpr int kXSlot = kMoeRemMax * KBB;
                constexpr int kXDma = kMoeRemMax / R / NPROD;  // DMAs per producer per step
                static_assert(NSTG == 3 && kXDma * R * NPROD == kMoeRemMax, "extra-row schedule");
                static_assert(NSTG * kXSlot <= kCompute * kEpiTile, "extra-row slots");
                const uint32_t xlds0 =
                    (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)epi_lds;
                const __amdgpu_buffer_rsrc_t xr = make_rsrc(
                    (const uint8_t *)uni((int64_t)(pr.a + pr.m * pr.lda_b)), uni(pr.xrows * pr.lda_b));
                uint32_t xoff[kXDma];
                int xjc[kXDma];
#pragma unroll
                for (int q = 0; q < kXDma; ++q) {
                    const int xrow = R * (kXDma * pw + q) + lane / C;
                    xjc[q] = ((lane % C) ^ swz<KBB>(xrow)) * 16;
                    xoff[q] = xrow < pr.xrows ? (uint32_t)(xrow * pr.lda_b) : kOob;
                }
                auto issue_x = [&](int st) {
                    const int64_t kb0 = (int64_t)st * KBB;
#pragma unroll
                    for (int q = 0; q < kXDma; ++q) {
                        const uint32_t off = (xoff[q] == kOob || kb0 + xjc[q] >= KB)
                                                 ? kOob : xoff[q] + (uint32_t)kb0 + xjc[q];
                        dma16(xr, off, xlds0 + (st % NSTG) * kXSlot + (kXDma * pw + q) * 1024);
                    }
                };
                __builtin_amdgcn_s_barrier();  // the epilogue area is free
                asm volatile("" ::: "memory");
                issue_x(0);
                issue_x(1);
                for (int s = 0; s < steps; ++s) {
                    // this wave's DMA and codes of step s are done, later
                    // ones may fly (step 0: step 1's codes newer; later: step
                    // s + 1's DMA and codes newer, if any)
                    if (s == 0) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kXDma) : "memory");
                    else ring_wait<kDmaPerWave + kXDma, NSTG - 2>(min(NSTG - 2, steps - 1 - s));
                    __builtin_amdgcn_s_barrier();
                    asm volatile("" ::: "memory");
                    if (s + NSTG - 1 < steps) {
                        issue(s + NSTG - 1, (s + NSTG - 1) % NSTG);
                        issue_x(s + NSTG - 1);
                    }
                }
                // end of tile: every compute wave is done with every stage
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                continue;
            }
            for (int s = 0; s < steps; ++s) {
                // this wave's DMA of step s is done (later steps may fly);
                // after the barrier every wave's is, and step s - 1's stage
                // is free for step s + NSTG - 1
                ring_wait<kDmaPerWave, NSTG - 2>(min(NSTG - 2, steps - 1 - s));
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                if (s + NSTG - 1 < steps) issue(s + NSTG - 1, (s + NSTG - 1) % NSTG);
            }
            // end of tile: every compute wave is done with every stage
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            continue;
        }

        v16i acc[FM][FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = (v16i){};
        // extra-row tiles: extra rows 32 xb .. 32 xb + 31 x B block wm
        v16i xacc[2] = {(v16i){}, (v16i){}};
        bool xdone = false;
        if constexpr (kExtra) {
            if (xt) {
                // the extra-row tile's first barrier (see the producers): this
                // wave's epilogue LDS reads are done
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                static_assert(WGN * FN * 32 == kGrpBN && FN == 2 && kCompute / WGN == 2,
                              "wave wm takes B block wm of its columns");
                constexpr int kXSlot = kMoeRemMax * KBB;
                static_assert(kMoeRemMax == 64, "one or two extra blocks");
                auto xloop = [&](auto xj, auto xb) __attribute__((always_inline)) {
                    for (int s = 0; s < steps; ++s) {
                        __builtin_amdgcn_s_barrier();
                        asm volatile("" ::: "memory");
                        big_compute<FM, FN, KBB, kGrpBM, UA, decltype(xj)::value,
                                    decltype(xb)::value>(smem + (s % NSTG) * kStage, wm, wn, lane,
                                                         acc, epi_lds + (s % NSTG) * kXSlot, xacc);
                    }
                };
                using I0 = std::integral_constant<int, 0>;
                using I1 = std::integral_constant<int, 1>;
                using I2 = std::integral_constant<int, 2>;
                if (pr.xrows > 32) {
                    if (wm == 0) xloop(I0{}, I2{});
                    else xloop(I1{}, I2{});
                } else {
                    if (wm == 0) xloop(I0{}, I1{});
                    else xloop(I1{}, I1{});
                }
                xdone = true;
            }
        }
        if (!xdone) {
            for (int s = 0; s < steps; ++s) {
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                big_compute<FM, FN, KBB, kGrpBM, UA>(smem + (s % NSTG) * kStage, wm, wn, lane, acc);
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if constexpr (kExtra) {
            if (xt) {
                // fp16 outputs of the extra rows from the 32x32 accumulator
                // layout (lane: column rr of B block wm of this wave's
                // columns, rows 32 xb + 8 (v / 4) + 4 gx + v % 4; block 1 is
                // zero unless there are more than 32), with the arithmetic of
                // the tile's LDS-staged epilogue
                const int rr = lane & 31, gx = lane >> 5;
                const int64_t ex = p;
                const f16 *sa = g.sa + pr.row0 + pr.m;
                const int64_t col = n0 + wn * (FN * 32) + wm * 32 + rr;
                if constexpr (FORM == kFormSwiglu) {
                    // columns in blocks of 8 gate then 8 up: a gate lane takes
                    // its up value from the lane 8 above
                    const int jj = rr & 15;
                    const int64_t gn0 = col - jj;
                    const bool on = jj < 8 && gn0 + 16 <= pr.n;
                    const float sbg = on ? (float)g.sb[ex * g.N + gn0 + jj] : 0.f;
                    const float sbu = on ? (float)g.sb[ex * g.N + gn0 + 8 + jj] : 0.f;
                    f16 *out = g.out + (pr.row0 + pr.m) * (g.N / 2) + gn0 / 2 + jj;
#pragma unroll
                    for (int xb = 0; xb < 2; ++xb)
#pragma unroll
                        for (int v = 0; v < 16; ++v) {
                            const int ua = __shfl_down(xacc[xb][v], 8, 64);
                            const int m = 32 * xb + 8 * (v / 4) + 4 * gx + v % 4;
                            if (on && m < pr.xrows) {
                                const float sav = (float)sa[m];
                                const f16 gh = f16_rn((float)(xacc[xb][v] >> 8) * sav * sbg);
                                const f16 uh = f16_rn((float)(ua >> 8) * sav * sbu);
                                out[m * (g.N / 2)] = swiglu1((float)gh, (float)uh);
                            }
                        }
                } else {
                    const bool on = col < pr.n;
                    const float sbv = on ? (float)g.sb[ex * g.N + col] : 0.f;
                    f16 *out = g.out + (pr.row0 + pr.m) * g.N + col;
#pragma unroll
                    for (int xb = 0; xb < 2; ++xb)
#pragma unroll
                        for (int v = 0; v < 16; ++v) {
                            const int m = 32 * xb + 8 * (v / 4) + 4 * gx + v % 4;
                            if (on && m < pr.xrows)
                                out[m * g.N] = f16_rn((float)(xacc[xb][v] >> (UA ? 4 : 8)) *
                                                      (float)sa[m] * sbv);
                        }
                }
            }
        }

        if (g.out) {
            // fp16 (expert-offset form): rows row0 + m of the [R, N] output,
            // through the wave's own LDS tile (the ring's stages already
            // take the next tile's DMA); the sym_dequant_moe zero correction
            // is epi_val's
            constexpr bool DENSE = FORM == kFormDense;
            const bool second = !DENSE && g.pair && (p & 1);
            const int64_t ex = DENSE ? 0 : g.pair ? p >> 1 : p;
            Epi e{};
            const bool sw = FORM == kFormSwiglu || (DENSE && g.swiglu);
            e.out = (second ? g.out2 : g.out) + pr.row0 * (sw ? g.N / 2 : g.N);
            e.sa = g.sa + pr.row0;
            e.sb = (second ? g.sb2 : g.sb) + ex * g.N;
            e.ua = UA;
            if (g.zr) {
                e.zr = g.zr + pr.row0;
                e.ws = (second ? g.ws2 : g.ws) + ex * g.N;
            }
            if constexpr (DENSE) {
                e.bias = g.bias;
                e.res = g.res;
                e.ldo = g.ldo;
            }
            if (sw)
                store_block_lds32_swiglu<32, FM, FN>(
                    e, pr.m, pr.n, m0 + wm * (FM * 32), n0 + wn * (FN * 32), acc, lane,
                    reinterpret_cast<int32_t *>(epi_lds + wave * kEpiTile));
            else
                store_block_lds32<32, FM, FN>(e, pr.m, pr.n, m0 + wm * (FM * 32),
                                              n0 + wn * (FN * 32), acc, lane,
                                              reinterpret_cast<int32_t *>(epi_lds + wave * kEpiTile));
            continue;
        }
        // int32 (pointer-array form): 32x32 accumulator layout, lane holds
        // column lane & 31, rows 8 (v / 4) + 4 (lane / 32) + v % 4
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t gm =
                    m0 + wm * (FM * 32) + i * 32 + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
                if (gm >= pr.m) continue;
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int64_t gn = n0 + wn * (FN * 32) + j * 32 + (lane & 31);
                    if (gn < pr.n) pr.c[gm * pr.ldc + gn] = acc[i][j][v] >> (UA ? 4 : 8);
                }
            }
    }
}

int check_gemm(const char *name, const void *A, const void *B, int64_t M, int64_t N,
               int64_t K) {
    SRQ_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", name);
    SRQ_CHECK_ARG(K % 32 == 0, "%s: K=%lld must be a multiple of 32", name, (long long)K);
    SRQ_CHECK_ARG(K < 131072, "%s: K=%lld >= 131072 (int32 accumulator bound)", name,
                  (long long)K);
    SRQ_CHECK_ARG(M <= 0x7fffffffLL && N <= 0x7fffffffLL, "%s: M or N > 2^31-1", name);
    // operands are read through 32-bit-offset buffer resources
    if (M * (K / 2) >= 0xFFFFFFF0LL || N * (K / 2) >= 0xFFFFFFF0LL) {
        srq_set_error("%s: operand larger than 4 GiB", name);
        return SRQ_EUNSUPPORTED;
    }
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

// Split-K epilogue: out (m, n) from the sum of the S int32 partials, each
// shifted down like the dense accumulator (exact: every product is a
// multiple of the shift), scaled back up so store_one's arithmetic is the
// dense path's (|sum a w| <= 64 K: the shifted-up value fits in int32).
// Four consecutive outputs per thread (16-byte partial loads; M N % 4 == 0
// is the caller's condition, else one per thread).
template <int V>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const int32_t *__restrict__ ws,
                                                            int S, int64_t M, int64_t N,
                                                            Epi e) {
    const int64_t MN = M * N;
    const int sh = e.ua ? 4 : 8;
    for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V; i < MN;
         i += (int64_t)gridDim.x * 256 * V) {
        // the S partials, 8 loads in flight at a time (one at a time, each
        // waited before the next, took ~2x as long)
        int acc[V] = {};
        for (int s0 = 0; s0 < S; s0 += 8) {
            if constexpr (V == 4) {
                v4i p[8];
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    p[k] = s0 + k < S ? *reinterpret_cast<const v4i *>(ws + (s0 + k) * MN + i)
                                      : (v4i){};
#pragma unroll
                for (int k = 0; k < 8; ++k)
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[q] += p[k][q];
            } else {
                int p[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) p[k] = s0 + k < S ? ws[(s0 + k) * MN + i] : 0;
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[0] += p[k];
            }
        }
        if (V == 4 && !e.C && N % 4 == 0) {
            // the four outputs share a row: store_one's arithmetic with every
            // operand loaded before the first store (a store may alias them,
            // so store_one per output waited a round trip for each)
            const int64_t m = i / N, n = i - m * N;
            f16 o[V];
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const int v = epi_val(e, (int)((u32)acc[k] << sh), m, n + k);
                const float a = (float)v * (float)e.sa[m];
                f16 x = f16_rn(a * (float)e.sb[n + k]);
                if (e.bias) x = f16_rn((float)x + (float)e.bias[n + k]);
                if (e.res) x = f16_rn((float)x + (float)e.res[m * N + n + k]);
                o[k] = x;
            }
#pragma unroll
            for (int k = 0; k < V; ++k) e.out[m * N + n + k] = o[k];
        } else {
#pragma unroll
            for (int k = 0; k < V; ++k)
                store_one(e, N, (i + k) / N, (i + k) % N, (int)((u32)acc[k] << sh));
        }
    }
}

// Split-K plan for mid-size M whose 128 x 128 tiles cannot fill the CUs:
// S K-chunks of Kc codes (a multiple of 256) so that tiles * S ~ 256, each
// chunk at least 7 K steps and tiles * S >= 128 (shorter chunks or fewer
// workgroups lose to the ring kernel: M = 128, N = 4096, K = 4096 took 19
// us split 4 ways against 10.5 unsplit; K = 14336 split 8 ways: 24 against
// 28).  S = 0: no split.
struct SplitK {
    int S = 0;
    int64_t Kc = 0;
    bool big = false;  // the big kernel's 256 x 128 tiles, grid (tiles, S)
};
SplitK splitk_plan(int64_t M, int64_t N, int64_t K, bool fp16_out) {
    SplitK p;
    if (!fp16_out || M <= 64 || M >= 1024 || K < 2048) return p;
    const int64_t tiles = srq_cdiv(M, kGrpBM) * srq_cdiv(N, kGrpBN);
    const int64_t big = srq_cdiv(M, kBigBM) * srq_cdiv(N, kBigBN);
    if (tiles >= 192 && big >= 64 && big <= 128 && 256 % big == 0 && K / (256 / big) >= 4096) {
        // enough 128 x 128 tiles for the dense grouped form, but 256 / big
        // K-chunks of 256 x 128 tiles cover the CUs exactly, and the bigger
        // tile unpacks fewer nibbles per MFMA (the grouped kernel's compute
        // waves are bound by that issue)
        p.S = (int)(256 / big);
        p.Kc = srq_cdiv(srq_cdiv(K, p.S), 256) * 256;
        p.S = (int)srq_cdiv(K, p.Kc);
        p.big = true;
        if (p.S < 2) p = SplitK{};
        return p;
    }
    if (tiles >= 192 || big >= 512) return p;
    int64_t S = std::min<int64_t>(256 / tiles, K / 1792);
    if (S < 2 || tiles * S < 128) return p;
    const int64_t Kc = srq_cdiv(srq_cdiv(K, S), 256) * 256;
    p.S = (int)srq_cdiv(K, Kc);
    p.Kc = Kc;
    if (p.S < 2) p.S = 0;
    return p;
}
int64_t splitk_bytes(int64_t M, int64_t N, int64_t K, bool fp16_out) {
    const SplitK p = splitk_plan(M, N, K, fp16_out);
    return p.S ? (int64_t)p.S * M * N * 4 : 0;
}

// The S partials at ws summed into e's epilogue.
void splitk_reduce(const void *ws, int S, int64_t M, int64_t N, const Epi &e, hipStream_t st) {
    if ((M * N) % 4 == 0) {
        // up to one pass per thread (cfg4 down_proj at M = 512: 4096 blocks,
        // 12.0 -> 11.3 us against a grid of 2048)
        const int64_t blocks = std::min<int64_t>(srq_cdiv(M * N / 4, 256), 8192);
        splitk_reduce_kernel<4><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
            (const int32_t *)ws, S, M, N, e);
    } else {
        const int64_t blocks = std::min<int64_t>(srq_cdiv(M * N, 256), 2048);
        splitk_reduce_kernel<1><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
            (const int32_t *)ws, S, M, N, e);
    }
}

// Kernel choice by shape; UA: A holds unsigned nibbles (Epi::ua).  With a
// workspace of at least splitk_bytes, mid-size M shapes with few tiles run
// split over K.
template <bool UA>
void launch_gemm(const uint8_t *a, const uint8_t *b, int64_t M, int64_t N, int64_t K,
                 const Epi &e, hipStream_t st, void *ws = nullptr, int64_t ws_bytes = 0) {
    const SplitK sk = ws ? splitk_plan(M, N, K, !e.C) : SplitK{};
    if (K == 0) {
        const int64_t blocks = std::min<int64_t>(srq_cdiv(M * N, 256), 4096);
        fill_zero_epilogue<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(M, N, e);
    } else if (launch_stream<UA>(a, b, M, N, K, e, st)) {
        // M <= 32: persistent weight-streaming kernel
    } else if (M <= 16 && !e.swiglu) {
        gemm_skinny_kernel<1, 8, 4, UA><<<dim3((unsigned)srq_cdiv(N, 16), 1), dim3(512), 0, st>>>(
            a, b, M, N, K, e);
    } else if (M <= 32 && !e.swiglu) {
        gemm_skinny_kernel<2, 8, 4, UA><<<dim3((unsigned)srq_cdiv(N, 16), 1), dim3(512), 0, st>>>(
            a, b, M, N, K, e);
    } else if (M <= 64 && !e.swiglu) {
        gemm_skinny_kernel<4, 8, 2, UA><<<dim3((unsigned)srq_cdiv(N, 16), 1), dim3(512), 0, st>>>(
            a, b, M, N, K, e);
    } else if (M >= 1024 && srq_cdiv(M, kSqBM) * srq_cdiv(N, kSqBN) >= 256) {
        // enough 256 x 256 tiles to cover the 256 CUs
        const int64_t tiles = srq_cdiv(M, kSqBM) * srq_cdiv(N, kSqBN);
        gemm_sq_kernel<128, 2, UA><<<dim3((unsigned)tiles), dim3(512), 0, st>>>(a, b, M, N, K, e);
    } else if (sk.S && sk.big && !e.swiglu && ws_bytes >= (int64_t)sk.S * M * N * 4) {
        // split-K on the big kernel: S rows of workgroups over K-chunks
        // write int32 partials, then one pass sums them and runs the
        // epilogue
        Epi ep{};
        ep.C = (int32_t *)ws;
        ep.ua = e.ua;
        const int64_t tiles = srq_cdiv(M, kBigBM) * srq_cdiv(N, kBigBN);
        gemm_big_kernel<4, 2, 2, 4, 2, 128, 3, UA>
            <<<dim3((unsigned)tiles, (unsigned)sk.S), dim3(512), 0, st>>>(a, b, M, N, K, ep, sk.Kc);
        splitk_reduce(ws, sk.S, M, N, e, st);
    } else if (sk.S && !e.swiglu && ws_bytes >= (int64_t)sk.S * M * N * 4) {
        // split-K: S dense problems over K-chunks write int32 partials,
        // then one pass sums them and runs the epilogue
        GroupedArgs g{};
        g.P = sk.S;
        g.M = M;
        g.A = a;
        g.B = b;
        g.N = N;
        g.K = K;
        g.Kc = sk.Kc;
        g.ws_c = (int32_t *)ws;
        const int64_t tiles = srq_cdiv(M, kGrpBM) * srq_cdiv(N, kGrpBN) * sk.S;
        gemm_grouped_kernel<4, UA, kFormSplitK>
            <<<dim3((unsigned)std::min<int64_t>(tiles, kGroupedGrid)), dim3(512), 0, st>>>(g);
        splitk_reduce(ws, sk.S, M, N, e, st);
    } else if (M < 1024 && !e.C && srq_cdiv(M, kGrpBM) * srq_cdiv(N, kGrpBN) >= 192 &&
               srq_cdiv(M, kBigBM) * srq_cdiv(N, kBigBN) < 512) {
        // mid-size M with enough 128 x 128 tiles to fill the CUs: the grouped
        // kernel's dense form (64 x 64 32x32-MFMA tiles per compute wave,
        // MFMA-bound where the ring kernel's small tiles are bound by the
        // nibble unpacking: 188 -> 113 us at M = 512, N = 8192, K = 28672)
        GroupedArgs g{};
        g.P = 1;
        g.M = M;
        g.A = a;
        g.B = b;
        g.N = N;
        g.K = K;
        g.sa = e.sa;
        g.sb = e.sb;
        g.out = e.out;
        g.bias = e.bias;
        g.res = e.res;
        g.zr = e.zr;
        g.ws = e.ws;
        g.swiglu = e.swiglu;
        g.ldo = e.ldo;
        const int64_t tiles = srq_cdiv(M, kGrpBM) * srq_cdiv(N, kGrpBN);
        gemm_grouped_kernel<4, UA, kFormDense>
            <<<dim3((unsigned)std::min<int64_t>(tiles, kGroupedGrid)), dim3(512), 0, st>>>(g);
    } else if (M >= 1024 || srq_cdiv(M, kBigBM) * srq_cdiv(N, kBigBN) >= 512) {
        const int64_t tm = srq_cdiv(M, kBigBM), tiles = tm * srq_cdiv(N, kBigBN);
        const int64_t rem = tiles % 256;
        // 4 compute waves (128 x 64 each) + 4 producer waves (8 compute
        // waves of 64 x 64, two per SIMD, measured no faster)
        if (e.swiglu && !e.ldo && M < 1024 && rem && rem <= 128 && rem % tm == 0 &&
            srq_cdiv(M, kGrpBM) * (rem / tm) * (kBigBN / kGrpBN) >= 128) {
            // a last round over at most half the CUs: its columns (whole
            // 128-column tiles) take the grouped kernel's dense form, which
            // spreads 128 x 128 tiles over every CU, and the rest runs in
            // whole rounds (cfg4 M = 512 gate/up: 768 + 256 tiles instead of
            // 3.5 rounds of 256); both write the [M, N / 2] output at its
            // own row stride
            const int64_t tail = rem / tm * kBigBN, head = N - tail;
            Epi eh = e;
            eh.ldo = N / 2;
            gemm_big_kernel<4, 2, 2, 4, 2, 128, 3, UA>
                <<<dim3((unsigned)(tiles - rem)), dim3(512), 0, st>>>(a, b, M, head, K, eh, 0);
            Epi et = eh;
            et.out = e.out + head / 2;
            et.sb = e.sb + head;
            launch_gemm<UA>(a, b + head * (K / 2), M, tail, K, et, st);
        } else {
            gemm_big_kernel<4, 2, 2, 4, 2, 128, 3, UA><<<dim3((unsigned)tiles), dim3(512), 0, st>>>(
                a, b, M, N, K, e, 0);
        }
    } else {
        // mid-size M: the tile shrinks with M so the grid still covers the
        // 256 CUs (at N = 4096: 256 workgroups for M = 128, 256, 512); the
        // smaller the tile, the deeper the DMA ring
        auto ring = [&](auto bm, auto bn, auto nstg) {
            constexpr int BM = decltype(bm)::value, BN = decltype(bn)::value;
            constexpr int NP = 4;  // 4 producers: measured 28.5 vs 31.8 us for 2 at M = 128
            const int64_t tiles = srq_cdiv(M, BM) * srq_cdiv(N, BN);
            gemm_ring_kernel<BM, BN, decltype(nstg)::value, NP, UA>
                <<<dim3((unsigned)tiles), dim3(64 * (4 + NP)), 0, st>>>(a, b, M, N, K, e);
        };
        using I32 = std::integral_constant<int, 32>;
        using I64 = std::integral_constant<int, 64>;
        using I128 = std::integral_constant<int, 128>;
        if (M <= 128) ring(I64{}, I32{}, std::integral_constant<int, 12>{});
        else if (M <= 256) ring(I64{}, I64{}, std::integral_constant<int, 9>{});
        else ring(I128{}, I64{}, std::integral_constant<int, 6>{});
    }
}

int run_gemm(const char *name, const void *A, const void *B, int64_t M, int64_t N, int64_t K,
             const Epi &e, hipStream_t st, void *ws = nullptr, int64_t ws_bytes = 0) {
    if (M == 0 || N == 0) return SRQ_OK;
    const uint8_t *a = (const uint8_t *)A;
    const uint8_t *b = (const uint8_t *)B;
    if (e.ua) launch_gemm<true>(a, b, M, N, K, e, st, ws, ws_bytes);
    else launch_gemm<false>(a, b, M, N, K, e, st, ws, ws_bytes);
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

extern "C" int srq_matmul_u4s4(const void *A, const void *B, int64_t M, int64_t N, int64_t K,
                               int32_t *C, void *stream) {
    int rc = check_gemm("matmul_ui4_si4", A, B, M, N, K);
    if (rc) return rc;
    SRQ_CHECK_ARG(C || M == 0 || N == 0, "matmul_ui4_si4: null output");
    Epi e{};
    e.C = C;
    e.ua = 1;
    return run_gemm("matmul_ui4_si4", A, B, M, N, K, e, (hipStream_t)stream);
}

extern "C" int srq_w4a4_linear_asym(const void *A, const void *a_scale, const int8_t *a_zero,
                                    const void *B, const void *b_scale, const int32_t *b_sum,
                                    const void *bias, int64_t M, int64_t N, int64_t K,
                                    void *out, void *stream) {
    int rc = check_gemm("w4a4_linear_asym", A, B, M, N, K);
    if (rc) return rc;
    if (M && N)
        SRQ_CHECK_ARG(out && a_scale && a_zero && b_scale && b_sum,
                      "w4a4_linear_asym: null pointer");
    Epi e{};
    e.out = (f16 *)out;
    e.sa = (const f16 *)a_scale;
    e.sb = (const f16 *)b_scale;
    e.bias = (const f16 *)bias;
    e.ua = 1;
    e.zr = a_zero;
    e.ws = b_sum;
    return run_gemm("w4a4_linear_asym", A, B, M, N, K, e, (hipStream_t)stream);
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

extern "C" int srq_w4a4_linear_swiglu(const void *A, const void *a_scale, const void *B,
                                      const void *b_scale, int64_t M, int64_t N, int64_t K,
                                      void *out, void *stream) {
    int rc = check_gemm("w4a4_linear_swiglu", A, B, M, N, K);
    if (rc) return rc;
    SRQ_CHECK_ARG(N % 16 == 0, "w4a4_linear_swiglu: N=%lld must be a multiple of 16",
                  (long long)N);
    SRQ_CHECK_ARG(K > 0, "w4a4_linear_swiglu: K must be positive");
    if (M == 0 || N == 0) return SRQ_OK;
    SRQ_CHECK_ARG(out && a_scale && b_scale, "w4a4_linear_swiglu: null pointer");
    SRQ_CHECK_ARG(srq_aligned(out, 16), "w4a4_linear_swiglu: out must be 16-byte aligned");
    Epi e{};
    e.out = (f16 *)out;
    e.sa = (const f16 *)a_scale;
    e.sb = (const f16 *)b_scale;
    e.swiglu = 1;
    // every kernel of the dispatch but the skinny and split-K forms (which
    // it then skips) ends in the swiglu row pass
    launch_gemm<false>((const uint8_t *)A, (const uint8_t *)B, M, N, K, e, (hipStream_t)stream);
    SRQ_LAUNCH_CHECK("w4a4_linear_swiglu");
    return SRQ_OK;
}

extern "C" int64_t srq_w4a4_linear_ws_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    return splitk_bytes(M, N, K, true);
}

extern "C" int srq_w4a4_linear_ws(const void *A, const void *a_scale, const void *B,
                                  const void *b_scale, const void *bias, int64_t M, int64_t N,
                                  int64_t K, void *out, void *workspace, int64_t ws_bytes,
                                  void *stream) {
    int rc = check_gemm("w4a4_linear_ws", A, B, M, N, K);
    if (rc) return rc;
    if (M && N) SRQ_CHECK_ARG(out && a_scale && b_scale, "w4a4_linear_ws: null pointer");
    SRQ_CHECK_ARG(ws_bytes >= 0 && (ws_bytes == 0 || workspace),
                  "w4a4_linear_ws: null workspace");
    // the split-K partials are written and read with 16-byte vector accesses
    SRQ_CHECK_ARG(ws_bytes == 0 || srq_aligned(workspace, 16),
                  "w4a4_linear_ws: workspace must be 16-byte aligned");
    Epi e{};
    e.out = (f16 *)out;
    e.sa = (const f16 *)a_scale;
    e.sb = (const f16 *)b_scale;
    e.bias = (const f16 *)bias;
    return run_gemm("w4a4_linear_ws", A, B, M, N, K, e, (hipStream_t)stream, workspace,
                    ws_bytes);
}

extern "C" int srq_w4a4_linear_residual_ws(const void *A, const void *a_scale, const void *B,
                                           const void *b_scale, const void *bias,
                                           const void *residual, int64_t M, int64_t N,
                                           int64_t K, void *out, void *workspace,
                                           int64_t ws_bytes, void *stream) {
    int rc = check_gemm("w4a4_linear_residual_ws", A, B, M, N, K);
    if (rc) return rc;
    if (M && N)
        SRQ_CHECK_ARG(out && a_scale && b_scale && residual,
                      "w4a4_linear_residual_ws: null pointer");
    SRQ_CHECK_ARG(ws_bytes >= 0 && (ws_bytes == 0 || workspace),
                  "w4a4_linear_residual_ws: null workspace");
    // the split-K partials are written and read with 16-byte vector accesses
    SRQ_CHECK_ARG(ws_bytes == 0 || srq_aligned(workspace, 16),
                  "w4a4_linear_residual_ws: workspace must be 16-byte aligned");
    Epi e{};
    e.out = (f16 *)out;
    e.sa = (const f16 *)a_scale;
    e.sb = (const f16 *)b_scale;
    e.bias = (const f16 *)bias;
    e.res = (const f16 *)residual;
    return run_gemm("w4a4_linear_residual_ws", A, B, M, N, K, e, (hipStream_t)stream,
                    workspace, ws_bytes);
}

extern "C" int srq_w4a4_linear_residual(const void *A, const void *a_scale, const void *B,
                                        const void *b_scale, const void *bias,
                                        const void *residual, int64_t M, int64_t N, int64_t K,
                                        void *out, void *stream) {
    int rc = check_gemm("w4a4_linear_residual", A, B, M, N, K);
    if (rc) return rc;
    if (M && N)
        SRQ_CHECK_ARG(out && a_scale && b_scale && residual,
                      "w4a4_linear_residual: null pointer");
    Epi e{};
    e.out = (f16 *)out;
    e.sa = (const f16 *)a_scale;
    e.sb = (const f16 *)b_scale;
    e.bias = (const f16 *)bias;
    e.res = (const f16 *)residual;
    return run_gemm("w4a4_linear_residual", A, B, M, N, K, e, (hipStream_t)stream);
}

extern "C" int srq_matmul_grouped(const int32_t *problem_sizes, const int64_t *ptr_A,
                                  const int64_t *ptr_B, const int64_t *ptr_C,
                                  const int64_t *lda, const int64_t *ldb, const int64_t *ldc,
                                  int64_t problem_count, int signed_a, void *stream) {
    SRQ_CHECK_ARG(problem_count >= 0 && problem_count <= 0x7fffffffLL,
                  "matmul_grouped: bad problem_count");
    if (problem_count == 0) return SRQ_OK;
    SRQ_CHECK_ARG(problem_sizes && ptr_A && ptr_B && ptr_C && lda && ldb && ldc,
                  "matmul_grouped: null pointer");
    GroupedArgs g{};
    g.P = (int)problem_count;
    g.sizes = problem_sizes;
    g.pa = ptr_A;
    g.pb = ptr_B;
    g.pc = ptr_C;
    g.lda = lda;
    g.ldb = ldb;
    g.ldc = ldc;
    if (signed_a)
        gemm_grouped_kernel<4, false><<<dim3(kGroupedGrid), dim3(512), 0, (hipStream_t)stream>>>(g);
    else
        gemm_grouped_kernel<4, true><<<dim3(kGroupedGrid), dim3(512), 0, (hipStream_t)stream>>>(g);
    SRQ_LAUNCH_CHECK("matmul_grouped");
    return SRQ_OK;
}

extern "C" int srq_w4a4_linear_moe(const void *A, const void *a_scale, const void *B,
                                   const void *b_scale, const int32_t *expert_offsets,
                                   int64_t num_experts, int64_t rows, int64_t N, int64_t K,
                                   void *out, void *stream) {
    SRQ_CHECK_ARG(num_experts >= 0 && num_experts <= 0x7fffffffLL && rows >= 0 && N >= 0 &&
                      K >= 0, "w4a4_linear_moe: bad shape");
    SRQ_CHECK_ARG(K % 32 == 0 && K < 131072, "w4a4_linear_moe: K=%lld must be a multiple of "
                  "32 and < 131072", (long long)K);
    if (num_experts == 0 || rows == 0 || N == 0) return SRQ_OK;
    if (rows * (K / 2) >= 0xFFFFFFF0LL || N * (K / 2) >= 0xFFFFFFF0LL) {
        srq_set_error("w4a4_linear_moe: operand larger than 4 GiB");
        return SRQ_EUNSUPPORTED;
    }
    SRQ_CHECK_ARG(A && a_scale && B && b_scale && expert_offsets && out,
                  "w4a4_linear_moe: null pointer");
    SRQ_CHECK_ARG(srq_aligned(A, 16) && srq_aligned(B, 16),
                  "w4a4_linear_moe: A and B must be 16-byte aligned");
    GroupedArgs g{};
    g.P = (int)num_experts;
    g.offsets = expert_offsets;
    g.A = (const uint8_t *)A;
    g.B = (const uint8_t *)B;
    g.N = N;
    g.K = K;
    g.sa = (const f16 *)a_scale;
    g.sb = (const f16 *)b_scale;
    g.out = (f16 *)out;
    g.skip_rem = K > 2 * kGrpKBB;  // at least two K steps (the extra rows' schedule)
    gemm_grouped_kernel<4, false><<<dim3(kGroupedGrid), dim3(512), 0, (hipStream_t)stream>>>(g);
    SRQ_LAUNCH_CHECK("w4a4_linear_moe");
    return SRQ_OK;
}

extern "C" int srq_w4a4_linear_moe_swiglu(const void *A, const void *a_scale, const void *B,
                                          const void *b_scale, const int32_t *expert_offsets,
                                          int64_t num_experts, int64_t rows, int64_t N,
                                          int64_t K, void *out, void *stream) {
    SRQ_CHECK_ARG(num_experts >= 0 && num_experts <= 0x7fffffffLL && rows >= 0 && N >= 0 &&
                      K >= 0, "w4a4_linear_moe_swiglu: bad shape");
    SRQ_CHECK_ARG(K % 32 == 0 && K < 131072, "w4a4_linear_moe_swiglu: K=%lld must be a "
                  "multiple of 32 and < 131072", (long long)K);
    SRQ_CHECK_ARG(N % 16 == 0, "w4a4_linear_moe_swiglu: N=%lld must be a multiple of 16",
                  (long long)N);
    if (num_experts == 0 || rows == 0 || N == 0) return SRQ_OK;
    if (rows * (K / 2) >= 0xFFFFFFF0LL || N * (K / 2) >= 0xFFFFFFF0LL) {
        srq_set_error("w4a4_linear_moe_swiglu: operand larger than 4 GiB");
        return SRQ_EUNSUPPORTED;
    }
    SRQ_CHECK_ARG(A && a_scale && B && b_scale && expert_offsets && out,
                  "w4a4_linear_moe_swiglu: null pointer");
    SRQ_CHECK_ARG(srq_aligned(A, 16) && srq_aligned(B, 16) && srq_aligned(out, 16),
                  "w4a4_linear_moe_swiglu: A, B and out must be 16-byte aligned");
    GroupedArgs g{};
    g.P = (int)num_experts;
    g.offsets = expert_offsets;
    g.A = (const uint8_t *)A;
    g.B = (const uint8_t *)B;
    g.N = N;
    g.K = K;
    g.sa = (const f16 *)a_scale;
    g.sb = (const f16 *)b_scale;
    g.out = (f16 *)out;
    g.skip_rem = K > 2 * kGrpKBB;  // at least two K steps (the extra rows' schedule)
    gemm_grouped_kernel<4, false, kFormSwiglu>
        <<<dim3(kGroupedGrid), dim3(512), 0, (hipStream_t)stream>>>(g);
    SRQ_LAUNCH_CHECK("w4a4_linear_moe_swiglu");
    return SRQ_OK;
}

extern "C" int srq_w4a4_linear_moe_gate_up(const void *A, const void *a_scale,
                                           const void *B_gate, const void *s_gate,
                                           const void *B_up, const void *s_up,
                                           const int32_t *expert_offsets, int64_t num_experts,
                                           int64_t rows, int64_t N, int64_t K, void *out_gate,
                                           void *out_up, void *stream) {
    SRQ_CHECK_ARG(num_experts >= 0 && num_experts <= 0x3fffffffLL && rows >= 0 && N >= 0 &&
                      K >= 0, "w4a4_linear_moe_gate_up: bad shape");
    SRQ_CHECK_ARG(K % 32 == 0 && K < 131072, "w4a4_linear_moe_gate_up: K=%lld must be a "
                  "multiple of 32 and < 131072", (long long)K);
    if (num_experts == 0 || rows == 0 || N == 0) return SRQ_OK;
    if (rows * (K / 2) >= 0xFFFFFFF0LL || N * (K / 2) >= 0xFFFFFFF0LL) {
        srq_set_error("w4a4_linear_moe_gate_up: operand larger than 4 GiB");
        return SRQ_EUNSUPPORTED;
    }
    SRQ_CHECK_ARG(A && a_scale && B_gate && s_gate && B_up && s_up && expert_offsets &&
                      out_gate && out_up, "w4a4_linear_moe_gate_up: null pointer");
    SRQ_CHECK_ARG(srq_aligned(A, 16) && srq_aligned(B_gate, 16) && srq_aligned(B_up, 16),
                  "w4a4_linear_moe_gate_up: A and B must be 16-byte aligned");
    GroupedArgs g{};
    g.P = 2 * (int)num_experts;
    g.pair = 1;
    g.offsets = expert_offsets;
    g.A = (const uint8_t *)A;
    g.B = (const uint8_t *)B_gate;
    g.B2 = (const uint8_t *)B_up;
    g.N = N;
    g.K = K;
    g.sa = (const f16 *)a_scale;
    g.sb = (const f16 *)s_gate;
    g.sb2 = (const f16 *)s_up;
    g.out = (f16 *)out_gate;
    g.out2 = (f16 *)out_up;
    gemm_grouped_kernel<4, false><<<dim3(kGroupedGrid), dim3(512), 0, (hipStream_t)stream>>>(g);
    SRQ_LAUNCH_CHECK("w4a4_linear_moe_gate_up");
    return SRQ_OK;
}

extern "C" int srq_w4a4_linear_moe_asym(const void *A, const void *a_scale, const int8_t *a_zero,
                                        const void *B, const void *b_scale, const int32_t *b_sum,
                                        const int32_t *expert_offsets, int64_t num_experts,
                                        int64_t rows, int64_t N, int64_t K, void *out,
                                        void *stream) {
    SRQ_CHECK_ARG(num_experts >= 0 && num_experts <= 0x7fffffffLL && rows >= 0 && N >= 0 &&
                      K >= 0, "w4a4_linear_moe_asym: bad shape");
    SRQ_CHECK_ARG(K % 32 == 0 && K < 131072, "w4a4_linear_moe_asym: K=%lld must be a multiple of "
                  "32 and < 131072", (long long)K);
    if (num_experts == 0 || rows == 0 || N == 0) return SRQ_OK;
    if (rows * (K / 2) >= 0xFFFFFFF0LL || N * (K / 2) >= 0xFFFFFFF0LL) {
        srq_set_error("w4a4_linear_moe_asym: operand larger than 4 GiB");
        return SRQ_EUNSUPPORTED;
    }
    SRQ_CHECK_ARG(A && a_scale && a_zero && B && b_scale && b_sum && expert_offsets && out,
                  "w4a4_linear_moe_asym: null pointer");
    SRQ_CHECK_ARG(srq_aligned(A, 16) && srq_aligned(B, 16),
                  "w4a4_linear_moe_asym: A and B must be 16-byte aligned");
    GroupedArgs g{};
    g.P = (int)num_experts;
    g.offsets = expert_offsets;
    g.A = (const uint8_t *)A;
    g.B = (const uint8_t *)B;
    g.N = N;
    g.K = K;
    g.sa = (const f16 *)a_scale;
    g.sb = (const f16 *)b_scale;
    g.out = (f16 *)out;
    g.zr = a_zero;
    g.ws = b_sum;
    gemm_grouped_kernel<4, true><<<dim3(kGroupedGrid), dim3(512), 0, (hipStream_t)stream>>>(g);
    SRQ_LAUNCH_CHECK("w4a4_linear_moe_asym");
    return SRQ_OK;
}
