// W4A4 GEMM on gfx950's 6-bit-operand MFMA.
//
// v_mfma_scale_f32_32x32x64_f8f6f4 with e3m2 ("bf6") operands multiplies a
// 32 x 64 by a 64 x 32 block in the issue time of the int8 MFMA's 32x32x32,
// twice the multiply-accumulates per cycle.  Every int4 code -8 .. 7 is an
// exact e3m2 value, every product of two codes is exact, and the fp32
// accumulator holds the integer sum exactly while it stays below 2^24
// (|sum| <= 64 K, K < 262144), so C equals the int32 product bit for bit.
// The scale operands are e8m0 127 (2^0).
//
// The operands must be in the bf6 block layout: srq_i4_to_bf6 converts
// packed int4 rows (the reference's layout, signrot/kernels/gemm.cu:7-45)
// once -- a Linear4bit weight at load time -- and the activation quantizers
// can write it directly.
//
// bf6 block layout of an R x K code matrix (K % 128 == 0; rows padded to a
// multiple of 32 with zero codes): 32 x 128 blocks of 3072 bytes, block
// (rb, kb) at byte (rb * K / 128 + kb) * 3072.  A block holds the operands
// of two MFMA k-slices q = 0, 1 for 64 lanes: lane l = r + 32 h carries, for
// slice q, codes 128 kb + 64 q + 32 h + j (j < 32) of row 32 rb + r as the
// 6-bit fields j of a 192-bit value (field j at bits 6 j .. 6 j + 5); its
// bytes 0-15 lie at 1024 q + 16 l and bytes 16-23 at 2048 + 16 l + 8 q.  A
// wave reads a block's two fragments with three unit-stride 16-byte LDS
// reads (no bank conflicts), and a tile's 32-row block is a contiguous 3 KiB
// run per 128-code K step, which the buffer-to-LDS DMA moves 1 KiB at a time.
#include "common.h"

#include <algorithm>
#include <type_traits>

namespace {

typedef int v6i __attribute__((ext_vector_type(6)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef _Float16 v32h __attribute__((ext_vector_type(32)));

constexpr uint32_t kOob = 0xFFFFFFF0u;
constexpr int kBlk = 3072;  // bytes of one 32 x 128 bf6 block

// e3m2 operands (format 3) on both sides, scales 2^0
SRQ_DEV v16f mfma_bf6(v8i a, v8i b, v16f c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 3, 3, 0, 127, 0, 127);
}

// ------------------------------------------------------------- conversion
// One thread per (block, lane): for each slice q the lane's 32 codes (16
// packed bytes, code 2 i in the low nibble of byte i) to fp16, then one
// v_cvt_scalef32_pk32 (fp16 -> packed e3m2, exact for these integers).
// Rows past `rows` give zero codes.
__global__ __launch_bounds__(256) void i4_to_bf6_kernel(const uint8_t *__restrict__ src,
                                                        int64_t rows, int64_t K,
                                                        uint8_t *__restrict__ dst,
                                                        int64_t nblk) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t blk = t >> 6;
    if (blk >= nblk) return;
    const int l = (int)(t & 63);
    const int64_t kbn = K / 128;
    const int64_t rb = blk / kbn, kb = blk % kbn;
    const int64_t r = rb * 32 + (l & 31);
    uint8_t *b = dst + blk * kBlk;
    u32 y[4];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int64_t k0 = kb * 128 + 64 * q + 32 * (l >> 5);
        v32h v;
        if (r < rows) {
            const v4i w = *reinterpret_cast<const v4i *>(src + r * (K / 2) + k0 / 2);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int byte = ((u32)w[i / 4] >> (8 * (i % 4))) & 0xFF;
                v[2 * i] = (f16)(float)(((byte & 15) ^ 8) - 8);
                v[2 * i + 1] = (f16)(float)(((byte >> 4) ^ 8) - 8);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) v[j] = (f16)0.f;
        }
        const v6i o = __builtin_amdgcn_cvt_scalef32_pk32_bf6_f16(v, 1.0f);
        *reinterpret_cast<v4i *>(b + 1024 * q + 16 * l) = (v4i){o[0], o[1], o[2], o[3]};
        y[2 * q] = (u32)o[4];
        y[2 * q + 1] = (u32)o[5];
    }
    *reinterpret_cast<v4i *>(b + 2048 + 16 * l) = (v4i){(int)y[0], (int)y[1], (int)y[2], (int)y[3]};
}

// ------------------------------------------------------------------- GEMM
struct Bf6Epi {
    int32_t *C;       // int32 output or null
    f16 *out;         // fp16 output (fused dequant) or null
    const f16 *sa;    // [M]
    const f16 *sb;    // [N]
    const f16 *bias;  // [N] or null
};

// Tile origin of workgroup b for TM x TN tiles.  XCD-aware order: workgroup
// b runs on XCD b % 8; XCD x owns one (tiles_m / 2) x (tiles_n / 4) block of
// the tile grid, so an XCD's L2 holds M/2 A rows and N/4 B rows (the fewest
// operand bytes per XCD for 8 XCDs).  Other grids: row-major.
template <int TM, int TN>
SRQ_DEV void bf6_tile(int64_t M, int64_t N, int64_t &m0, int64_t &n0) {
    const int64_t tiles_n = (N + TN - 1) / TN, tiles_m = (M + TM - 1) / TM;
    if (tiles_m % 2 == 0 && tiles_n % 4 == 0) {
        const int64_t x = blockIdx.x % 8, i = blockIdx.x / 8;
        const int64_t bm = tiles_m / 2, bn = tiles_n / 4;
        m0 = ((x % 2) * bm + i / bn) * TM;
        n0 = ((x / 2) * bn + i % bn) * TN;
    } else {
        m0 = ((int64_t)blockIdx.x / tiles_n) * TM;
        n0 = ((int64_t)blockIdx.x % tiles_n) * TN;
    }
}

// Store a wave's FM x FN 32 x 32 accumulator blocks (lane holds column
// lane & 31, rows 8 (v / 4) + 4 (lane / 32) + v % 4 of each): C = the exact
// integer, or out = fp16((float(acc) * sa) * sb) (+ bias), the reference's
// two fp32 multiplies (quant.cu:84-87).
template <int FM, int FN>
SRQ_DEV void bf6_store(const Bf6Epi &e, int64_t M, int64_t N, int64_t mb0, int64_t nb0,
                       const v16f (&acc)[FM][FN], int lane) {
    int64_t gn[FN];
    float sbv[FN], bv[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        gn[j] = nb0 + j * 32 + (lane & 31);
        sbv[j] = (!e.C && gn[j] < N) ? (float)e.sb[gn[j]] : 0.f;
        bv[j] = (e.bias && gn[j] < N) ? (float)e.bias[gn[j]] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        // one 32-row block at a time (keeps the live addresses and scales
        // of the other blocks out of the registers)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int64_t gm = mb0 + i * 32 + 8 * (v / 4) + 4 * (lane >> 5) + (v % 4);
            if (gm >= M) continue;
            const float sa = e.C ? 0.f : (float)e.sa[gm];
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                if (gn[j] >= N) continue;
                const int iv = (int)acc[i][j][v];  // an exact integer
                if (e.C) {
                    e.C[gm * N + gn[j]] = iv;
                } else {
                    f16 o = f16_rn((float)iv * sa * sbv[j]);
                    if (e.bias) o = f16_rn((float)o + bv[j]);
                    e.out[gm * N + gn[j]] = o;
                }
            }
        }
    }
}

// Fragment of k slice q of a bf6 block in LDS: 16 bytes at 1024 q + 16 l,
// then bytes 16-23 from the shared Y run (2048 + 16 l: slice 0's in the low
// half, slice 1's in the high half; `y` holds that 16-byte read).
SRQ_DEV v8i bf6_frag(const uint8_t *blk, int q, int lane, const v4i &y) {
    const v4i x = *reinterpret_cast<const v4i *>(blk + 1024 * q + 16 * lane);
    return q == 0 ? (v8i){x[0], x[1], x[2], x[3], y[0], y[1], 0, 0}
                  : (v8i){x[0], x[1], x[2], x[3], y[2], y[3], 0, 0};
}

// 256 x 128 tile per workgroup: 4 producer waves move the tile's 12 row
// blocks (8 of A, 4 of B) through an NSTG-stage LDS ring, 128 codes (two
// 64-code k blocks, 3 KiB per row block) per step; 4 compute waves (2 x 2),
// each 128 x 64 = 4 x 2 MFMA blocks, only read LDS and multiply.  One
// barrier per step: barrier s certifies that step s + 1 has landed and that
// step s - 1's stage is consumed (the producers then refill it with step
// s + NSTG - 1), so the compute waves read the next step's first k block
// while they multiply this step's second.  Row blocks past the matrix read
// as zeros (out-of-range buffer offsets).
constexpr int kTM = 256, kTN = 128;
constexpr int kRb = (kTM + kTN) / 32;   // row blocks per tile
constexpr int kStage = kRb * kBlk;  // 36 KiB
constexpr int kProd = 4;
constexpr int kDmaPerWave = kRb * 3 / kProd;  // 1 KiB DMA instructions per producer per step

template <int NSTG>
__global__ __launch_bounds__(512, 1) void gemm_bf6_kernel(const uint8_t *__restrict__ A6,
                                                          const uint8_t *__restrict__ B6,
                                                          int64_t M, int64_t N, int64_t K,
                                                          Bf6Epi e) {
    static_assert(NSTG >= 3 && NSTG <= 4 && NSTG * kStage <= 160 * 1024, "LDS ring");
    static_assert((NSTG - 2) * kDmaPerWave <= 63, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[NSTG * kStage];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int64_t m0, n0;
    bf6_tile<kTM, kTN>(M, N, m0, n0);
    const int steps = (int)(K / 128);
    const int64_t rbytes = steps * (int64_t)kBlk;  // bytes per 32-row block

    if (wave >= 4) {
        // ---- producer pw: tile row blocks 3 pw .. 3 pw + 2 (A: 0-7, B: 8-11)
        const int pw = wave - 4;
        const int64_t mb = srq_cdiv(M, 32), nb = srq_cdiv(N, 32);
        const __amdgpu_buffer_rsrc_t ar = make_rsrc(A6, mb * rbytes);
        const __amdgpu_buffer_rsrc_t br = make_rsrc(B6, nb * rbytes);
        const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)smem;
        uint32_t base[3];
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            const int i = 3 * pw + q;
            const bool isa = i < kTM / 32;
            const int64_t rb = isa ? m0 / 32 + i : n0 / 32 + (i - kTM / 32);
            base[q] = rb < (isa ? mb : nb) ? (uint32_t)(rb * rbytes) : kOob;
        }
        auto issue = [&](int st, int sl) __attribute__((always_inline)) {
#pragma unroll
            for (int q = 0; q < 3; ++q) {
                const int i = 3 * pw + q;
#pragma unroll
                for (int t = 0; t < 3; ++t) {
                    const uint32_t off = base[q] == kOob
                                             ? kOob
                                             : base[q] + (uint32_t)st * kBlk + t * 1024 +
                                                   lane * 16;
                    dma16(i < kTM / 32 ? ar : br, off,
                          lds0 + sl * kStage + i * kBlk + t * 1024);
                }
            }
        };
#pragma unroll
        for (int s = 0; s < NSTG - 1; ++s)
            if (s < steps) issue(s, s);
        // wait until this wave's DMA of step t is done, the `later` steps
        // issued after it may stay in flight (vmcnt counts in issue order)
        auto wait_step = [&](int later) __attribute__((always_inline)) {
            if (later >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kDmaPerWave) : "memory");
            else if (later == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerWave) : "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        };
        wait_step(steps - 1 < NSTG - 2 ? steps - 1 : NSTG - 2);  // step 0
        __builtin_amdgcn_s_barrier();
        for (int s = 0; s < steps; ++s) {
            // barrier s certifies step s + 1 (the compute waves read its
            // first k block during step s) ...
            const int later = steps - s - 2 < NSTG - 3 ? steps - s - 2 : NSTG - 3;
            wait_step(later < 0 ? 0 : later);
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            // ... and every read of step s - 1's stage is done: refill it
            if (s + NSTG - 1 < steps) issue(s + NSTG - 1, (s + NSTG - 1) % NSTG);
        }
        return;  // the compute waves meet no barrier after their K loop
    }

    // ---- compute wave (wm, wn): tile rows 128 wm .., columns 64 wn ..
    const int wm = wave >> 1, wn = wave & 1;
    v16f acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (v16f){};
    // Fragments of one step: slice 0 (X_0 and the shared Y, whose upper
    // half is slice 1's) and slice 1 (X_1).
    auto read0 = [&](int s, v8i (&fa)[4], v8i (&fb)[2], uint2 (&ya)[4], uint2 (&yb)[2])
                     __attribute__((always_inline)) {
        const uint8_t *stage = smem + (s % NSTG) * kStage;
        auto one = [&](const uint8_t *blk, v8i &f, uint2 &y1) __attribute__((always_inline)) {
            const v4i x = *reinterpret_cast<const v4i *>(blk + 16 * lane);
            const v4i y = *reinterpret_cast<const v4i *>(blk + 2048 + 16 * lane);
            f = (v8i){x[0], x[1], x[2], x[3], y[0], y[1], 0, 0};
            y1 = (uint2){(u32)y[2], (u32)y[3]};
        };
#pragma unroll
        for (int i = 0; i < 4; ++i) one(stage + (4 * wm + i) * kBlk, fa[i], ya[i]);
#pragma unroll
        for (int j = 0; j < 2; ++j) one(stage + (kTM / 32 + 2 * wn + j) * kBlk, fb[j], yb[j]);
    };
    auto read1 = [&](int s, v8i (&fa)[4], v8i (&fb)[2], const uint2 (&ya)[4],
                     const uint2 (&yb)[2]) __attribute__((always_inline)) {
        const uint8_t *stage = smem + (s % NSTG) * kStage + 1024;
        auto one = [&](const uint8_t *blk, v8i &f, uint2 y1) __attribute__((always_inline)) {
            const v4i x = *reinterpret_cast<const v4i *>(blk + 16 * lane);
            f = (v8i){x[0], x[1], x[2], x[3], (int)y1.x, (int)y1.y, 0, 0};
        };
#pragma unroll
        for (int i = 0; i < 4; ++i) one(stage + (4 * wm + i) * kBlk, fa[i], ya[i]);
#pragma unroll
        for (int j = 0; j < 2; ++j) one(stage + (kTM / 32 + 2 * wn + j) * kBlk, fb[j], yb[j]);
    };
    auto mma = [&](const v8i (&fa)[4], const v8i (&fb)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf6(fa[i], fb[j], acc[i][j]);
    };
    // Software pipeline across steps: the LDS reads of a k slice overlap
    // the MFMAs of the previous one, including the step boundary (the
    // barrier of step s certifies step s + 1).
    v8i fa0[4], fb0[2], fa1[4], fb1[2];
    uint2 ya[4], yb[2];
    __builtin_amdgcn_s_barrier();  // step 0 landed
    asm volatile("" ::: "memory");
    read0(0, fa0, fb0, ya, yb);
    for (int s = 0; s < steps; ++s) {
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        read1(s, fa1, fb1, ya, yb);
        mma(fa0, fb0);
        if (s + 1 < steps) read0(s + 1, fa0, fb0, ya, yb);
        mma(fa1, fb1);
    }

    bf6_store<4, 2>(e, M, N, m0 + wm * 128, n0 + wn * 64, acc, lane);
}

// 256 x 256 tile per workgroup of 4 waves (2 x 2), each 128 x 128 = 4 x 4
// MFMA blocks (the accumulators fill the accumulation registers: one wave per
// SIMD), every wave also moving a quarter of the tile's 16 row blocks (12
// buffer-to-LDS instructions per step) through a 3-stage ring.  Per operand
// byte it does twice the MFMA work of the 256 x 128 tile, which brings the
// bytes a CU loads per step down to its load rate at the bf6 MFMA rate.
constexpr int kSq = 256;
constexpr int kSqRb = 2 * kSq / 32;     // row blocks per tile
constexpr int kSqStage = kSqRb * kBlk;  // 48 KiB

__global__ __launch_bounds__(256, 1) void gemm_bf6_sq_kernel(const uint8_t *__restrict__ A6,
                                                             const uint8_t *__restrict__ B6,
                                                             int64_t M, int64_t N, int64_t K,
                                                             Bf6Epi e) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[3 * kSqStage];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int64_t m0, n0;
    bf6_tile<kSq, kSq>(M, N, m0, n0);
    const int steps = (int)(K / 128);
    const int64_t rbytes = steps * (int64_t)kBlk;
    // DMA: wave w moves tile row blocks 4 w .. 4 w + 3 (A: 0-7, B: 8-15)
    const bool isa = wave < 2;
    const int64_t rows = isa ? M : N, row0 = isa ? m0 : n0;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(isa ? A6 : B6, srq_cdiv(rows, 32) * rbytes);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)smem +
                          4 * wave * kBlk;
    // per-lane byte offset of this wave's row block q at step 0 (kOob past
    // the matrix: the whole block reads as zeros)
    uint32_t base[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t rb = row0 / 32 + 4 * (wave & 1) + q;
        base[q] = rb < srq_cdiv(rows, 32) ? (uint32_t)(rb * rbytes) + lane * 16 : kOob;
    }
    auto issue = [&](int st, int sl) __attribute__((always_inline)) {
        const uint32_t d = (uint32_t)st * kBlk;
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int t = 0; t < 3; ++t)
                dma16(rs, base[q] == kOob ? kOob : base[q] + d + t * 1024,
                      lds0 + sl * kSqStage + q * kBlk + t * 1024);
    };
    const int wm = wave >> 1, wn = wave & 1;
    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (v16f){};
    issue(0, 0);
    if (steps > 1) issue(1, 1);
    for (int s = 0; s < steps; ++s) {
        // this wave's DMA of step s is done (step s + 1's may stay in flight)
        if (s + 1 < steps) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // every wave's DMA of step s has landed and every wave is done with
        // step s - 1's stage, which step s + 2 now refills
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + 2 < steps) issue(s + 2, (s + 2) % 3);
        const uint8_t *stage = smem + (s % 3) * kSqStage;
        v4i ya[4], yb[4];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            v8i fa[4], fb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint8_t *blk = stage + (4 * wm + i) * kBlk;
                if (q == 0) ya[i] = *reinterpret_cast<const v4i *>(blk + 2048 + 16 * lane);
                fa[i] = bf6_frag(blk, q, lane, ya[i]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint8_t *blk = stage + (8 + 4 * wn + j) * kBlk;
                if (q == 0) yb[j] = *reinterpret_cast<const v4i *>(blk + 2048 + 16 * lane);
                fb[j] = bf6_frag(blk, q, lane, yb[j]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma_bf6(fa[i], fb[j], acc[i][j]);
        }
    }
    bf6_store<4, 4>(e, M, N, m0 + wm * 128, n0 + wn * 128, acc, lane);
}

int check_bf6(const char *name, const void *A6, const void *B6, int64_t M, int64_t N,
              int64_t K) {
    SRQ_CHECK_ARG(M >= 0 && N >= 0 && K >= 0, "%s: negative shape", name);
    SRQ_CHECK_ARG(K % 128 == 0, "%s: K=%lld must be a multiple of 128", name, (long long)K);
    // |sum| <= 64 K must stay below 2^24 (exact in the fp32 accumulator) and
    // the int32 epilogue below 2^31
    SRQ_CHECK_ARG(K < 131072, "%s: K=%lld >= 131072", name, (long long)K);
    SRQ_CHECK_ARG(M <= 0x7fffffffLL && N <= 0x7fffffffLL, "%s: M or N > 2^31-1", name);
    if (srq_cdiv(M, 32) * (K / 128) * kBlk >= (int64_t)kOob ||
        srq_cdiv(N, 32) * (K / 128) * kBlk >= (int64_t)kOob) {
        srq_set_error("%s: operand larger than 4 GiB", name);
        return SRQ_EUNSUPPORTED;
    }
    if (M && N && K) {
        SRQ_CHECK_ARG(A6 && B6, "%s: null operand", name);
        SRQ_CHECK_ARG(srq_aligned(A6, 16) && srq_aligned(B6, 16),
                      "%s: A and B must be 16-byte aligned", name);
    }
    return SRQ_OK;
}

__global__ void bf6_zero_k(int64_t M, int64_t N, Bf6Epi e) {
    // K == 0: C = 0; fused output = fp16(0 * sa * sb) (+ bias)
    const int64_t total = M * N;
    for (int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * 256) {
        const int64_t m = t / N, n = t % N;
        if (e.C) {
            e.C[t] = 0;
        } else {
            f16 o = f16_rn(0.f * (float)e.sa[m] * (float)e.sb[n]);
            if (e.bias) o = f16_rn((float)o + (float)e.bias[n]);
            e.out[t] = o;
        }
    }
}

int run_bf6(const char *name, const void *A6, const void *B6, int64_t M, int64_t N, int64_t K,
            const Bf6Epi &e, hipStream_t st) {
    if (M == 0 || N == 0) return SRQ_OK;
    if (K == 0) {
        const int64_t blocks = std::min<int64_t>(srq_cdiv(M * N, 256), 4096);
        bf6_zero_k<<<dim3((unsigned)blocks), dim3(256), 0, st>>>(M, N, e);
    } else {
        // 256 x 256 tiles once they cover the 256 CUs (twice the MFMA work
        // per loaded byte), else 256 x 128 (measured at K = 14336, N = 4096:
        // M = 2048 138 vs 98 us, M = 8192 305 vs 366 us)
        if (srq_cdiv(M, kSq) * srq_cdiv(N, kSq) >= 256) {
            const int64_t tiles = srq_cdiv(M, kSq) * srq_cdiv(N, kSq);
            gemm_bf6_sq_kernel<<<dim3((unsigned)tiles), dim3(256), 0, st>>>(
                (const uint8_t *)A6, (const uint8_t *)B6, M, N, K, e);
        } else {
            const int64_t tiles = srq_cdiv(M, kTM) * srq_cdiv(N, kTN);
            gemm_bf6_kernel<4><<<dim3((unsigned)tiles), dim3(512), 0, st>>>(
                (const uint8_t *)A6, (const uint8_t *)B6, M, N, K, e);
        }
    }
    SRQ_LAUNCH_CHECK(name);
    return SRQ_OK;
}

}  // namespace

extern "C" int64_t srq_bf6_bytes(int64_t rows, int64_t K) {
    if (rows < 0 || K < 0 || K % 128) return -1;
    return srq_cdiv(rows, 32) * (K / 128) * kBlk;
}

extern "C" int srq_i4_to_bf6(const void *src, int64_t rows, int64_t K, void *dst, void *stream) {
    SRQ_CHECK_ARG(rows >= 0 && K >= 0, "i4_to_bf6: negative shape");
    SRQ_CHECK_ARG(K % 128 == 0, "i4_to_bf6: K=%lld must be a multiple of 128", (long long)K);
    const int64_t nblk = srq_cdiv(rows, 32) * (K / 128);
    if (nblk == 0) return SRQ_OK;
    SRQ_CHECK_ARG(src && dst, "i4_to_bf6: null pointer");
    SRQ_CHECK_ARG(srq_aligned(src, 16) && srq_aligned(dst, 16),
                  "i4_to_bf6: src and dst must be 16-byte aligned");
    i4_to_bf6_kernel<<<dim3((unsigned)srq_cdiv(nblk * 64, 256)), dim3(256), 0,
                       (hipStream_t)stream>>>((const uint8_t *)src, rows, K, (uint8_t *)dst,
                                              nblk);
    SRQ_LAUNCH_CHECK("i4_to_bf6");
    return SRQ_OK;
}

extern "C" int srq_matmul_bf6(const void *A6, const void *B6, int64_t M, int64_t N, int64_t K,
                              int32_t *C, void *stream) {
    int rc = check_bf6("matmul_bf6", A6, B6, M, N, K);
    if (rc) return rc;
    SRQ_CHECK_ARG(C || M == 0 || N == 0, "matmul_bf6: null output");
    Bf6Epi e{};
    e.C = C;
    return run_bf6("matmul_bf6", A6, B6, M, N, K, e, (hipStream_t)stream);
}

extern "C" int srq_w4a4_linear_bf6(const void *A6, const void *a_scale, const void *B6,
                                   const void *b_scale, const void *bias, int64_t M, int64_t N,
                                   int64_t K, void *out, void *stream) {
    int rc = check_bf6("w4a4_linear_bf6", A6, B6, M, N, K);
    if (rc) return rc;
    if (M && N) SRQ_CHECK_ARG(out && a_scale && b_scale, "w4a4_linear_bf6: null pointer");
    Bf6Epi e{};
    e.out = (f16 *)out;
    e.sa = (const f16 *)a_scale;
    e.sb = (const f16 *)b_scale;
    e.bias = (const f16 *)bias;
    return run_bf6("w4a4_linear_bf6", A6, B6, M, N, K, e, (hipStream_t)stream);
}
