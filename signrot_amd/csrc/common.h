// Shared helpers for the SignRot gfx950 kernels and the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/signrot_hip.h"

typedef _Float16 f16;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef unsigned int u32;
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

#define SRQ_DEV __device__ __forceinline__

// ----------------------------------------------------------- error reporting
// The entry points never throw: they return an SRQ_E* code and leave a
// message retrievable with srq_last_error() (thread-local).
void srq_set_error(const char *fmt, ...);

#define SRQ_CHECK_ARG(cond, ...)                                   \
    do {                                                           \
        if (!(cond)) {                                             \
            srq_set_error(__VA_ARGS__);                            \
            return SRQ_EINVAL;                                     \
        }                                                          \
    } while (0)

#define SRQ_LAUNCH_CHECK(name)                                     \
    do {                                                           \
        hipError_t _e = hipGetLastError();                         \
        if (_e != hipSuccess) {                                    \
            srq_set_error("%s: launch failed: %s", name,           \
                          hipGetErrorString(_e));                  \
            return SRQ_ELAUNCH;                                    \
        }                                                          \
    } while (0)

static inline bool srq_aligned(const void *p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

__host__ __device__ static inline int64_t srq_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------------------ wave helpers
SRQ_DEV float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

SRQ_DEV float wave_min(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
    return v;
}

SRQ_DEV float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Wave max by DPP moves inside each row of 16 lanes (no LDS round trips),
// then the four row results read back as uniform values.
#define SRQ_DPP(v, ctrl) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), \
                                                           ctrl, 0xF, 0xF, false))
SRQ_DEV float wave_max_dpp(float v) {
    v = fmaxf(v, SRQ_DPP(v, 0xB1));   // quad_perm [1, 0, 3, 2]
    v = fmaxf(v, SRQ_DPP(v, 0x4E));   // quad_perm [2, 3, 0, 1]
    v = fmaxf(v, SRQ_DPP(v, 0x124));  // row_ror:4
    v = fmaxf(v, SRQ_DPP(v, 0x128));  // row_ror:8
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Reduction over a group of G consecutive lanes (G a power of two <= 64).
template <int G>
SRQ_DEV float group_max(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

template <int G>
SRQ_DEV float group_min(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
    return v;
}

template <int G>
SRQ_DEV float group_sum(float v) {
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// ------------------------------------------------------------ buffer memory
// Raw buffer resource over [p, p + bytes): a load at or past the byte size
// returns zeros in hardware, so tile edges need no branches.
SRQ_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void *p, int64_t bytes) {
    const uint32_t n = bytes > 0xFFFFFFF0LL ? 0xFFFFFFF0u : (uint32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, (int)n, 0x00020000);
}

// Direct global -> LDS loads (no VGPR staging).  One instruction per wave:
// lane l's 16 (dma16) or 4 (dma4) bytes from buffer offset voff land at LDS
// byte address lds + 16 l (resp. + 4 l).  They count in vmcnt like any vector
// load; the caller waits with an explicit s_waitcnt before reading the LDS.
// The LDS base goes in M0 as a "{m0}" operand, so the compiler sets M0 itself
// and knows the register is taken (nothing it keeps in M0 is overwritten).
// The leading s_nop 4 supplies the wait states the hardware needs between
// the compiler's writes of the operands and this instruction's reads of
// them, which the compiler's hazard pass cannot see inside the asm: an SALU
// write of M0 before an LDS-DMA read of M0 (1), and a VALU write of an SGPR
// (v_readlane restoring a spilled descriptor or M0 source) before a VMEM read
// of it (5).  Without it the DMA could take the previous M0 and land in the
// wrong LDS stage: a grouped-GEMM build whose scheduler put
// "s_mov_b32 m0, s33" right before the load returned wrong products.
SRQ_DEV void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :: "v"(voff), "s"(r), "{m0}"(lds) : "memory");
}

SRQ_DEV void dma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds) {
    asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, 0 offen lds"
                 :: "v"(voff), "s"(r), "{m0}"(lds) : "memory");
}

// ------------------------------------------------------- fp16 rounding
// Round an fp32 *result* to fp16 in two steps, as the reference does
// (fp32 op, then __float2half).  The empty asm pins the fp32 value in a
// register so the backend cannot fold `fptrunc(fmul/fma(...))` into a
// v_fma_mix* instruction, which would round the exact product to fp16 once
// -- a different value whenever the fp32 rounding moves it across an fp16
// rounding boundary.
SRQ_DEV f16 f16_rn(float v) {
    asm volatile("" : "+v"(v));
    return (f16)v;
}

SRQ_DEV float round16(float v) { return (float)f16_rn(v); }

// ---------------------------------------------------------- int4 semantics
// Symmetric code of one fp16 value given the fp16 scale, as the reference's
// quantizers define it: q = clamp(round_half_even(fp16(x / s)), -8, 7), where
// fp16(x / s) is the correctly rounded quotient (__hdiv), NaN (0/0 on an
// all-zero row) gives 0 and ±inf saturates.
//
// No division per element: with r = fl32(1 / s), fp16(fl32(x * r)) equals
// the correctly rounded fp16(x / s) whenever |x / s| >= 2^-14, and its code
// equals the quotient's code for every fp16 pair (x, s > 0) -- checked
// exhaustively over all fp16 pairs by tests/c/quot_exact.c; negative x
// follow by symmetry of the rounding.  s == 0 gives r = inf: x * inf is
// ±inf (saturates) and 0 * inf is NaN (code 0), as x / 0 and 0 / 0 are.
SRQ_DEV float sym_recip(float s) { return 1.0f / s; }

SRQ_DEV int sym_code_r(float x, float r) {
    float quot = round16(x * r);
    float c = __builtin_rintf(quot);
    if (c != c) return 0;
    c = fminf(fmaxf(c, -8.f), 7.f);
    return (int)c;
}

SRQ_DEV int sym_code(float x, float s) { return sym_code_r(x, sym_recip(s)); }

// Unsigned asymmetric KV code: clamp(round_half_even(fp16(fp16(x + z) / s)),
// 0, 15), the quotient by the same reciprocal identity (here the shifted
// value is >= 0 and s > 0; quotients below 2^-14 give code 0 either way).
SRQ_DEV int kv_code_r(float x, float zero, float rs) {
    float shifted = round16(x + zero);
    float scaled = round16(shifted * rs);
    float c = __builtin_rintf(scaled);
    if (c != c) return 0;
    c = fminf(fmaxf(c, 0.f), 15.f);
    return (int)c;
}

SRQ_DEV int kv_code(float x, float zero, float scale) {
    return kv_code_r(x, zero, sym_recip(scale));
}

// __half2int_rn of an fp16 value held in fp32: round half to even, NaN -> 0,
// values beyond the int32 range (±inf) saturate.
SRQ_DEV int h2i_rn(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.f) return 0x7fffffff;
    if (v <= -2147483648.f) return (int)0x80000000;
    return (int)__builtin_rintf(v);
}

// Per-row parameters of the asymmetric activation quantizer
// (signrot/kernels/fused.cu:166-179) from the row's exact fp32 min and max:
// hmin, hmax in fp16 (each times clip, rounded, when clip != 1);
// diff = fp16(hmax - hmin); scale = fp16(diff / 15);
// ratio = fp16(-hmin / scale); zero = fp16(round_half_even(ratio)).
SRQ_DEV void asym_row_params(float vmin, float vmax, float clip, f16 &scale, f16 &zero) {
    f16 hmin = f16_rn(vmin), hmax = f16_rn(vmax);
    if (clip != 1.f) {
        hmin = f16_rn((float)hmin * clip);
        hmax = f16_rn((float)hmax * clip);
    }
    const f16 diff = f16_rn((float)hmax - (float)hmin);
    scale = f16_rn((float)diff / 15.f);
    const f16 ratio = f16_rn(-(float)hmin / (float)scale);
    zero = f16_rn(__builtin_rintf((float)ratio));
}

// Asymmetric code: clamp(__half2int_rn(fp16(x / s)) + zero_i, lo, hi), the
// quotient correctly rounded (fp32 division, then one fp16 rounding) and the
// int addition wrapping in int32 as the reference's does.
SRQ_DEV int asym_code(float x, float s, int zero_i, int lo, int hi) {
    const float quot = round16(x / s);
    const int c = (int)((u32)h2i_rn(quot) + (u32)zero_i);
    return c < lo ? lo : (c > hi ? hi : c);
}

// Eight symmetric codes packed into one 32-bit word, element i in bits
// 4i .. 4i + 3 (the reference's nibble order).
SRQ_DEV u32 pack8_sym(const v8h &v, float s) {
    const float r = sym_recip(s);
    u32 w = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) w |= (u32)(sym_code_r((float)v[i], r) & 0xF) << (4 * i);
    return w;
}

SRQ_DEV float absmax8(const v8h &v, float m) {
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf((float)v[i]));
    return m;
}

// Row scale from the exact fp32 max (fused.cu:93-95 order: divide, round to
// fp16, then the clip multiply rounds again).
SRQ_DEV f16 sym_row_scale(float amax, float clip) {
    f16 s = f16_rn(amax / 7.f);
    if (clip != 1.f) s = f16_rn((float)s * clip);
    return s;
}

// SwiGLU of one element: fp16(fp16(g / (1 + exp(-g))) * u)
// (signrot/kernels/fused.cu:367-390); every kernel that applies it calls
// this one function, so fused and unfused forms round identically.
SRQ_DEV f16 swiglu1(float g, float u) {
    const f16 sl = f16_rn(g / (1.f + expf(-g)));
    return (f16)((float)sl * u);
}

// In-register Walsh-Hadamard butterflies over R values (Sylvester order),
// stages in ascending index bit: every FWHT kernel here runs its stages in
// this order, so a fused kernel reproduces the unfused fp32 result exactly.
template <int R>
SRQ_DEV void fwht_regs(float (&v)[R]) {
#pragma unroll
    for (int h = 1; h < R; h <<= 1) {
#pragma unroll
        for (int i = 0; i < R; ++i) {
            if (!(i & h)) {
                const float a = v[i], b = v[i + h];
                v[i] = a + b;
                v[i + h] = a - b;
            }
        }
    }
}

// KV-cache row parameters from the exact row max/min (fused.cu:246-252):
// diff rounds to fp16, the clamp(min=1e-5) rounds to fp16, the / 15 rounds
// again; zero = -min exactly.
SRQ_DEV void kv_row_params(float vmax, float vmin, f16 &scale, f16 &zero) {
    f16 diff = f16_rn((float)(f16)vmax - (float)(f16)vmin);
    diff = f16_rn(fmaxf((float)diff, 1e-5f));
    scale = f16_rn((float)diff / 15.f);
    zero = -(f16)vmin;
}

// Rotary embedding of one rotate_half pair (x0 at i, x1 at i + D/2) with
// per-op fp16 rounding, as the three-op torch expression
// x * cos + rotate_half(x) * sin evaluates it in fp16 (fused.cu:316-362).
// Written in fp16 arithmetic: a correctly rounded fp16 product or sum equals
// the fp32 one rounded to fp16 (products of two fp16 values are exact in
// fp32; fp32 has the 2p + 2 bits that make the double rounding of a sum
// innocuous), and it keeps the sign of zero.  The fp32 form let the
// compiler round x1 * s through fma(x1, s, +0), which turns a -0 product
// into +0 and gave rope_lo -0 where the reference gives +0.
SRQ_DEV f16 rope_lo(f16 x0, f16 x1, f16 c, f16 s) {
    const f16 a = x0 * c;
    const f16 b = (-x1) * s;
    return a + b;
}

SRQ_DEV f16 rope_hi(f16 x0, f16 x1, f16 c, f16 s) {
    const f16 a = x1 * c;
    const f16 b = x0 * s;
    return a + b;
}

// ----------------------------------------------- packed-fp16 int4 quantizer
// fp16(x * r) for both fp16 halves of w, each rounded once from the exact
// product: with r = fl32(1 / s) this is the correctly rounded fp16 quotient
// x / s whenever |x / s| >= 2^-14, and it gives the same int4 code for every
// fp16 pair (tests/c/quot_exact.c checks all pairs).
SRQ_DEV u32 quot2(u32 w, float r) {
    u32 q;
    asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=&v"(q)
        : "v"(w), "v"(r));
    return q;
}

// packed fp16 quotients -> fp16 (round_half_even(q) + 1544): low nibble of
// each half = code + 8
template <bool CLAMP>
SRQ_DEV u32 offset_codes(u32 q) {
    v2h h = __builtin_bit_cast(v2h, q);
    if (CLAMP)
        h = __builtin_elementwise_min(__builtin_elementwise_max(h, (v2h){-8, -8}),
                                      (v2h){7, 7});
    h = h + (v2h){1544, 1544};
    return __builtin_bit_cast(u32, h);
}

// eight offset codes (pairs a = (e0, e1), b = (e2, e3), c = (e4, e5),
// d = (e6, e7), nibble in bits 0-3 and 16-19 of each) -> 32 bits of packed
// two's-complement nibbles, e0 in bits 0-3 ... e7 in bits 28-31
SRQ_DEV u32 pack8_raw(u32 a, u32 b, u32 c, u32 d) {
    const u32 x = __builtin_amdgcn_perm(b, a, 0x06020400u);  // e0 e2 e1 e3
    const u32 y = __builtin_amdgcn_perm(d, c, 0x06020400u);  // e4 e6 e5 e7
    const u32 lo = __builtin_amdgcn_perm(y, x, 0x05040100u); // e0 e2 e4 e6
    const u32 hi = __builtin_amdgcn_perm(y, x, 0x07060302u); // e1 e3 e5 e7
    // each selected byte is the low byte of an fp16 in [1536, 1551]: the
    // code itself, high nibble clear
    return lo | (hi << 4);
}

SRQ_DEV u32 pack8(u32 a, u32 b, u32 c, u32 d) { return pack8_raw(a, b, c, d) ^ 0x88888888u; }

// Packed fp16 quotients -> asymmetric uint4 codes in the low nibble of each
// half: clamp to [-zi, 15 - zi] (exact in fp16 for |zi| <= 511), round half
// to even by + 1536 (ulp 1 in [1024, 2048); 1536 is even, so the sum rounds
// as the quotient does), then + zi (exact): clamp(rne(q) + zi, 0, 15),
// which is the reference's clamp(__half2int_rn(q) + zi, 0, 15) for finite q.
SRQ_DEV u32 asym_offset_codes(u32 q, v2h lo, v2h hi, v2h zo) {
    v2h h = __builtin_bit_cast(v2h, q);
    h = __builtin_elementwise_min(__builtin_elementwise_max(h, lo), hi);
    h = h + (v2h){1536, 1536};
    h = h + zo;
    return __builtin_bit_cast(u32, h);
}

// Reciprocal for the packed quantizer: s == 0 (an all-zero row, or a
// clipped scale that underflowed) becomes 2^-126, so x = 0 gives code 0 and
// any other x saturates, which is what x / 0 gives after the reference's
// round-and-clamp.
SRQ_DEV float sym_rcp_safe(float s) { return 1.0f / fmaxf(s, 0x1p-126f); }

// Can a quotient of this row round beyond ±7 (then the codes are clamped in
// fp16 first)?  Never for clip = 1: s = fp16(amax / 7) >= amax / 7.002.
SRQ_DEV bool sym_row_needs_clamp(float amax, float s) {
    return !(amax <= 7.25f * fmaxf(s, 0x1p-126f));
}

// Eight symmetric int4 codes of finite fp16 values by the packed route
// (2-3 VALU per value instead of a division), identical to pack8_sym.
template <bool CLAMP>
SRQ_DEV u32 pack8_sym_fast(const v8h &v, float rcp) {
    const v4i w = __builtin_bit_cast(v4i, v);
    return pack8(offset_codes<CLAMP>(quot2((u32)w[0], rcp)),
                 offset_codes<CLAMP>(quot2((u32)w[1], rcp)),
                 offset_codes<CLAMP>(quot2((u32)w[2], rcp)),
                 offset_codes<CLAMP>(quot2((u32)w[3], rcp)));
}

// absmax8 that also flags a non-finite value (NaN or inf) in `bad`; rows
// with one take the exact pack8_sym path (the reference maps a NaN to code 0).
SRQ_DEV float absmax8_flag(const v8h &v, float m, bool &bad) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float a = fabsf((float)v[i]);
        m = fmaxf(m, a);
        bad |= !(a <= 65504.f);
    }
    return m;
}
