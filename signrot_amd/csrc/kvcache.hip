// Paged int4 KV cache for gfx950: append (decode), bulk fill (prefill) and
// single-query batch decode attention with on-the-fly uint4 dequant and a
// split-KV merge.
//
// Cache layout (the reference's paged_kv_t, signrot/kernels/include/
// flashinfer/page.cuh:18-112):
//   data  u8  [pages, L, 2, H, page_size, D/2]  (K at 0, V at 1; uint4 codes,
//                                               dim 2j in the low nibble)
//   param f16 [pages, L, 2, H, page_size, 2]    ([scale, zero] per token)
// Request b owns pages indices[indptr[b] .. indptr[b+1]); its length is
// (pages - 1) * page_size + last_page_offset[b].
//
// Attention (decode.cuh:493-751 semantics): k̂ = q4 * scale - zero in fp32,
// logit = (q · k̂) / sqrt(D) (in base 2: times log2 e), exp2 online softmax,
// out = sum p v̂ / sum p, fp16.  GQA is native: query head h reads KV head
// h / (Hq / H), so the cache stores each KV head once (the reference stores
// them repeated to Hq heads; the results are the same).
//
// Decode kernel: one block per (request, KV head, split-KV chunk), four
// waves, 32-token tiles.
//   q · K^T on the fp16 MFMA (32x32x16): B operand = the tile's K codes,
//     converted exactly to fp16 with the 0x6400 magic number (1024 + c, then
//     - 1024), A operand = the g query heads of the group (rows >= g zero);
//     dequant folded as scale * (q · c) - zero * sum(q).
//   P · V on VALU with v_dot2_f32_f16 over token pairs: p * v_scale rounded
//     to fp16 times the integer codes (exact in fp16), the zero-point term
//     sum p * v_zero accumulated separately in fp32.
#include "common.h"

#include <atomic>

#include <math.h>

namespace {

typedef _Float16 v2h __attribute__((ext_vector_type(2)));

struct Paged {
    uint8_t *data;
    f16 *param;
    const int32_t *indptr;
    const int32_t *indices;
    const int32_t *last;
    int64_t L, layer, H, page, D;
};

SRQ_DEV int64_t seq_len_of(const Paged &p, int64_t b) {
    const int64_t np = p.indptr[b + 1] - p.indptr[b];
    return np > 0 ? (np - 1) * p.page + p.last[b] : 0;
}

// byte offset of (page, kv, head, entry) code row; param index likewise
SRQ_DEV int64_t row_index(const Paged &p, int64_t page, int kv, int64_t head, int64_t entry) {
    return (((page * p.L + p.layer) * 2 + kv) * p.H + head) * p.page + entry;
}

// --------------------------------------------------------------- append
// Copy `count` tokens per request into the cache at positions
// [len - count, len): one thread per (token, head, 16-byte chunk) for K and
// V codes, plus the [scale, zero] pairs.
__global__ __launch_bounds__(256) void append_kernel(Paged p, const uint8_t *__restrict__ k,
                                                     const uint8_t *__restrict__ v,
                                                     const f16 *__restrict__ kp,
                                                     const f16 *__restrict__ vp,
                                                     const int32_t *__restrict__ src_indptr,
                                                     int64_t B) {
    const int64_t b = blockIdx.y;
    if (b >= B) return;
    const int64_t len = seq_len_of(p, b);
    const int64_t s0 = src_indptr ? src_indptr[b] : b;
    const int64_t cnt = src_indptr ? src_indptr[b + 1] - s0 : 1;
    const int64_t start = len - cnt;
    const int chunks = (int)(p.D / 2 / 16) + 1;  // code chunks + one param slot
    const int64_t per_tok = p.H * chunks;
    for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < cnt * per_tok;
         idx += (int64_t)gridDim.x * 256) {
        const int64_t j = idx / per_tok;
        const int64_t rem = idx - j * per_tok;
        const int64_t h = rem / chunks;
        const int c = (int)(rem - h * chunks);
        const int64_t pos = start + j;
        if (pos < 0) continue;
        const int64_t page = p.indices[p.indptr[b] + pos / p.page];
        const int64_t entry = pos % p.page;
        const int64_t src = (s0 + j) * p.H + h;
        if (c < chunks - 1) {
            const int64_t so = src * (p.D / 2) + 16 * c;
            const int64_t ko = row_index(p, page, 0, h, entry) * (p.D / 2) + 16 * c;
            const int64_t vo = row_index(p, page, 1, h, entry) * (p.D / 2) + 16 * c;
            *reinterpret_cast<v4i *>(p.data + ko) = *reinterpret_cast<const v4i *>(k + so);
            *reinterpret_cast<v4i *>(p.data + vo) = *reinterpret_cast<const v4i *>(v + so);
        } else {
            const uint32_t kv = reinterpret_cast<const uint32_t *>(kp)[src];
            const uint32_t vv = reinterpret_cast<const uint32_t *>(vp)[src];
            reinterpret_cast<uint32_t *>(p.param)[row_index(p, page, 0, h, entry)] = kv;
            reinterpret_cast<uint32_t *>(p.param)[row_index(p, page, 1, h, entry)] = vv;
        }
    }
}

// ------------------------------------------------ fused q/k/v post-GEMM
// The decode-step work between the q/k/v projection and the attention
// kernel, in one launch (modeling_llama.py:62-79 + kv_cache.py:295-415 +
// kv_cache.py:157-158): for request b and the new token,
//   q-head rows: RoPE -> (rotate) FWHT_D * had_scale -> fp16 -> q_out
//   k-head rows: RoPE -> (rotate) FWHT_D * had_scale -> fp16 -> KV int4
//                quantize -> cache slot of the new token
//   v-head rows: KV int4 quantize -> cache slot
// qkv f16 [B, (Hq + 2 Hk) D] is the projection output (q heads, k heads, v
// heads).  Each D = 128 row is held by 16 lanes, 8 consecutive values per
// lane: FWHT index bits 0-2 are butterflies in registers, bits 3-6 across
// lanes (stages in ascending bit, as the FWHT kernel runs them), the RoPE
// partner i +- 64 is lane l ^ 8.  Every per-element operation is the one the
// separate ops apply (rope_lo/rope_hi, fp32 FWHT, f16_rn, kv_row_params,
// kv_code), so the result equals rope_qk -> hadamard_transform ->
// kv_quant_pack -> append_kv_i4 bit for bit.
struct QkvArgs {
    const f16 *qkv;
    const f16 *cs, *sn;  // [cos_batch, D]
    int cos_batch;
    int64_t B;
    int hq, hk;
    float had_scale;
    int rotate;
    f16 *q_out;          // [B, hq, D]
};

SRQ_DEV float xor_lane(float v, int m) { return __shfl_xor(v, m, 64); }

// The per-row arithmetic, shared by qkv_post_kernel and the fused form of
// decode_kernel so that both give the same bits.  Lane l (0..15) of a
// 16-lane group holds dims 8 l .. 8 l + 7 of one D = 128 row in v; kind 0 / 1
// / 2 = q / k / v row.  Every lane of the wave must call these (shuffles).
// RoPE (q, k), then FWHT_D * had_scale rounded to fp16 (q, k, when rotate).
SRQ_DEV void qkv_row_transform(float (&v)[8], int kind, int l, const f16 *cs, const f16 *sn,
                               int64_t ct, float had_scale, int rotate) {
    constexpr int D = 128;
    {
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float o = xor_lane(v[e], 8);
            const int i = 8 * l + e;
            const f16 c = cs[ct * D + i], s = sn[ct * D + i];
            const f16 xe = (f16)v[e], xo = (f16)o;  // exact: both came from fp16
            y[e] = (float)(l < 8 ? rope_lo(xe, xo, c, s) : rope_hi(xo, xe, c, s));
        }
        if (kind != 2) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = y[e];
        }
    }
    if (rotate) {
        float w[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e] = v[e];
        fwht_regs<8>(w);
#pragma unroll
        for (int m = 1; m < 16; m <<= 1) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float o = xor_lane(w[e], m);
                w[e] = (l & m) ? o - w[e] : w[e] + o;
            }
        }
        if (kind != 2) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (float)f16_rn(w[e] * had_scale);
        }
    }
}

// KV int4 quantizer of a transformed row: the row max / min over the 16
// lanes, [scale, zero], and this lane's 8 codes as one word.
SRQ_DEV u32 kv_row_codes(const float (&v)[8], f16 &scale, f16 &zero) {
    float vmax = -INFINITY, vmin = INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        vmax = fmaxf(vmax, v[e]);
        vmin = fminf(vmin, v[e]);
    }
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
        vmax = fmaxf(vmax, xor_lane(vmax, m));
        vmin = fminf(vmin, xor_lane(vmin, m));
    }
    kv_row_params(vmax, vmin, scale, zero);
    const float fs = (float)scale, fz = (float)zero;
    u32 word = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) word |= (u32)kv_code(v[e], fz, fs) << (4 * e);
    return word;
}

SRQ_DEV uint32_t pack_param(f16 scale, f16 zero) {
    const f16 pr[2] = {scale, zero};
    return *reinterpret_cast<const uint32_t *>(pr);
}

__global__ __launch_bounds__(256) void qkv_post_kernel(QkvArgs a, Paged p) {
    constexpr int D = 128;
    const int lane = threadIdx.x & 63;
    const int l = lane & 15;                       // lane within the row group
    const int hs = a.hq + 2 * a.hk;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const bool valid = row < a.B * hs;
    const int64_t b = valid ? row / hs : 0;
    const int slot = valid ? (int)(row - b * hs) : 0;
    const int kind = slot < a.hq ? 0 : (slot < a.hq + a.hk ? 1 : 2);  // q, k, v
    float v[8];
    {
        v8h x = valid ? *reinterpret_cast<const v8h *>(a.qkv + row * D + 8 * l) : (v8h){};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (float)x[e];
    }
    // The new token's cache slot of a k / v row, looked up now: its two
    // dependent page-table reads then overlap the row load and the
    // transform instead of following them.
    int64_t pos = -1, page = 0;
    if (valid && kind != 0) {
        pos = seq_len_of(p, b) - 1;
        if (pos >= 0) page = p.indices[p.indptr[b] + pos / p.page];
    }
    qkv_row_transform(v, kind, l, a.cs, a.sn, a.cos_batch == 1 ? 0 : b, a.had_scale, a.rotate);
    if (kind == 0) {
        if (valid) {
            v8h o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (f16)v[e];
            *reinterpret_cast<v8h *>(a.q_out + (b * a.hq + slot) * D + 8 * l) = o;
        }
    }
    f16 scale, zero;
    const u32 word = kv_row_codes(v, scale, zero);
    if (!valid || kind == 0 || pos < 0) return;
    const int kv = kind - 1;
    const int64_t h = slot - a.hq - (kind == 2 ? a.hk : 0);
    const int64_t entry = pos % p.page;
    const int64_t ri = row_index(p, page, kv, h, entry);
    reinterpret_cast<u32 *>(p.data + ri * (D / 2))[l] = word;
    if (l == 0) reinterpret_cast<uint32_t *>(p.param)[ri] = pack_param(scale, zero);
}

// --------------------------------------------------------------- decode
constexpr int kTile = 32;
constexpr int kD = 128;

SRQ_DEV v16f mfma32h(v8h a, v8h b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// uint4 -> fp16 by masking alone: a nibble in the low mantissa bits of an
// fp16 with a zero exponent is the subnormal c * 2^-24 (bits 0-3, even dims)
// or 16 c * 2^-24 (bits 4-7, odd dims), both exact.  The MFMA and dot2
// products with these are exact in fp32; the 2^24 (even) and 2^20 (odd)
// factors are applied to the fp32 results (on the query side for K: the odd
// dims of q are pre-divided by 16).  The masks live in VGPRs (opaque to the
// compiler) so each pair is one v_and_b32.
struct Nib {
    u32 mlo, mhi;
};

SRQ_DEV Nib make_nib() {
    Nib n{0x000F000Fu, 0x00F000F0u};
    asm volatile("" : "+v"(n.mlo), "+v"(n.mhi));
    return n;
}

// codes of the low (hi = false) or high nibbles of bytes 0 and 2, scaled by
// 2^-24 (low) or 2^-20 (high)
SRQ_DEV v2h nib_lo(const Nib &n, u32 w) { return __builtin_bit_cast(v2h, w & n.mlo); }
SRQ_DEV v2h nib_hi(const Nib &n, u32 w) { return __builtin_bit_cast(v2h, w & n.mhi); }

// 8 uint4 codes (one dword, code 2j in the low nibble of byte j) -> 8 fp16
// values in the order [0, 4, 1, 5, 2, 6, 3, 7]: c * 2^-24 at even dims,
// c * 2^-20 at odd dims
SRQ_DEV v8h codes8(const Nib &n, u32 w) {
    const u32 w8 = w >> 8;
    const v2h p0 = nib_lo(n, w), p1 = nib_hi(n, w), p2 = nib_lo(n, w8), p3 = nib_hi(n, w8);
    return (v8h){p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// dim order of codes8 slot e (within its 8-dim group)
SRQ_DEV int codes8_dim(int e) { return (e >> 1) + 4 * (e & 1); }

template <int CTRL>
SRQ_DEV float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// max over each 32-lane half of the wave: quad permutes, half-row and row
// mirrors (DPP), then a swizzle that swaps the 16-lane halves
SRQ_DEV float max32(float x) {
    x = fmaxf(x, dpp<0xB1>(x));   // quad_perm [1, 0, 3, 2]
    x = fmaxf(x, dpp<0x4E>(x));   // quad_perm [2, 3, 0, 1]
    x = fmaxf(x, dpp<0x141>(x));  // row_half_mirror
    x = fmaxf(x, dpp<0x140>(x));  // row_mirror
    return fmaxf(x, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(
                                                  __builtin_bit_cast(int, x), 0x401F)));
}

struct DecodeArgs {
    Paged p;
    const f16 *q;      // [B, Hq, D] (unfused form)
    // fused form (qkv non-null): the q/k/v projection output of the new
    // token [B, (Hq + 2 H) D]; q and k get RoPE (cos/sin rows [cos_batch, D])
    // and, when rotate, the head-dim Hadamard times had_scale; k and v are
    // quantized into the new token's cache slot (the qkv_post_kernel
    // arithmetic), and q is used without a trip through memory
    const f16 *qkv = nullptr;
    const f16 *cs = nullptr, *sn = nullptr;
    int cos_batch = 1;
    int rotate = 0;
    float had_scale = 1.f;
    f16 *o;            // [B, Hq, D]
    float *tmp;        // [B, Hq, chunks, D + 4] or null
    int64_t B, Hq, G;  // G = Hq / H (query heads per KV head), <= 8
    int chunks;
    float sm_scale_log2;
};

// Row (token) index of the K row of `entry` in page `pg`; the V row is
// H * page rows further.
SRQ_DEV int64_t k_row(const Paged &p, int64_t pg, int64_t head, int64_t entry) {
    return ((pg * p.L + p.layer) * 2 * p.H + head) * p.page + entry;
}

// ---------------------------------------------------------------------------
// One 32-token tile lives in an LDS stage of the wave:
//   [K codes 2 KiB][V codes 2 KiB][K params 128 B][V params 128 B]
// rows of 64 bytes, token t's 16-byte chunk c stored at chunk
// c ^ ((t >> 2) & 3) (conflict-free reads below).
constexpr int kStageBytes = 2 * 2048 + 2 * 128;
// per-wave fp16 weights P[16 heads][32 tokens] (the P.V MFMA's A operand)
constexpr int kPvBytes = 16 * kTile * 2;
// page-table slice of a chunk kept in LDS
constexpr int kMaxChunkPages = 256;

SRQ_DEV int swz(int t, int chunk) { return t * 64 + 16 * (chunk ^ ((t >> 2) & 3)); }

typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i lds_v2i;

// ds_read_b64_tr_b4: within each 16-lane group, lane i receives nibble i of
// the 8-byte chunks addressed by lanes 0..15 of the group (nibble e of the
// result from lane e's chunk).
SRQ_DEV v2i ds_tr4(const uint8_t *p) {
    return __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_v2i *)(p));
}

SRQ_DEV v4f mfma16h(v8h a, v8h b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Online-softmax state of one wave.
template <int GP>
struct DecodeState {
    v8h qa[8];         // Q.K^T A operand (rows = heads of the group)
    float qs[4];       // sm_scale log2(e) * sum of q, heads 4 h2 + r
    float m_run[4], d_part[4], z_part[4];  // S layout: heads 4 h2 + r
    v4f acc[8];        // P.V output, N-block nb: [head 4 g + r][dim 16 nb + i]
};

// Slot of token e (0..7) in its 8-token group of the P operand: the order
// [0, 4, 1, 5, 2, 6, 3, 7] that codes8 produces from a transposed dword.
SRQ_DEV int p_slot(int e) { return 2 * (e & 3) + (e >> 2); }

// lazy running-max slack (log2 units)
constexpr float kLazyMax = 8.f;

// One tile starting at token tb (tokens >= t1 masked), from LDS stage `sg`.
//   Q.K^T: v_mfma_f32_32x32x16_f16, A = q (heads), B = K codes of the lane's
//   token (lane = token tl + 32 h2, dims 64 h2 .. 64 h2 + 63).
//   P.V:   v_mfma_f32_16x16x32_f16 per 16-dim N-block, A = P[head][token],
//   B = V codes transposed by ds_read_b64_tr_b4: lane (i, g) gets dim
//   16 nb + i of tokens 8 g .. 8 g + 7.
template <int GP>
SRQ_DEV void tile_step(DecodeState<GP> &st, const uint8_t *sg, int64_t tb, int64_t t1, int lane,
                       float sm_scale_log2, f16 *pvt, const Nib &nib) {
    const int tl = lane & 31, h2 = lane >> 5;
    // ---------------- scores: lane (token tl, half h2)
    const int sw = (tl >> 2) & 3;
    const v4i c0 = *reinterpret_cast<const v4i *>(sg + tl * 64 + 16 * ((2 * h2) ^ sw));
    const v4i c1 = *reinterpret_cast<const v4i *>(sg + tl * 64 + 16 * ((2 * h2 + 1) ^ sw));
    const v2h kp = *reinterpret_cast<const v2h *>(sg + 4096 + 4 * tl);
    const v2h vp = *reinterpret_cast<const v2h *>(sg + 4096 + 128 + 4 * tl);
    const bool valid = tb + tl < t1;
    // logits in log2 units: sm_scale log2(e) (2^24 scale * sacc - zero * sum q)
    const float ks2 = (float)kp[0] * (16777216.f * sm_scale_log2), kz = (float)kp[1];
    // V scale of the P operand entry: odd tokens meet V codes scaled by 2^-20
    // (high nibbles of the transposed dword), so they are divided by 16
    const float vs = valid ? (float)vp[0] * ((tl & 1) ? 0.0625f : 1.f) : 0.f;
    const float vz = valid ? (float)vp[1] : 0.f;
    v16f sacc = {};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) sacc = mfma32h(st.qa[ks], codes8(nib, (u32)c0[ks]), sacc);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) sacc = mfma32h(st.qa[4 + ks], codes8(nib, (u32)c1[ks]), sacc);
    // lane (tl, h2) holds 2^-24 S[head 4 h2 + r][token tl] in sacc[r]
    float lg[4], mn[4];
    bool grow = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        lg[i] = valid ? __builtin_fmaf(ks2, sacc[i], -kz * st.qs[i]) : -INFINITY;
        // lazy running max: it moves only when a logit exceeds it by more
        // than kLazyMax, so the weights stay below 2^kLazyMax and the
        // accumulators are rarely rescaled
        grow |= lg[i] > st.m_run[i] + kLazyMax;
        mn[i] = st.m_run[i];
    }
    if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float tmax = max32(lg[i]);  // finite: token tb is valid
            mn[i] = tmax > st.m_run[i] + kLazyMax ? tmax : st.m_run[i];
        }
    }
    float pr[4], ph[4];
    bool big = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        pr[i] = __builtin_amdgcn_exp2f(lg[i] - mn[i]);  // 0 for masked tokens
        ph[i] = pr[i] * vs;
        big |= 4 * h2 + i < GP && ph[i] > 32768.f;
    }
    if (__builtin_amdgcn_ballot_w64(big)) {
        // an fp16 weight would overflow: move the max to this tile's
        // (weights <= 1, |p v_scale| <= 4368)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            mn[i] = fmaxf(mn[i], max32(lg[i]));
            pr[i] = __builtin_amdgcn_exp2f(lg[i] - mn[i]);
            ph[i] = pr[i] * vs;
        }
    }
    const int pcol = 8 * (tl >> 3) + p_slot(tl & 7);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (4 * h2 + i < GP) pvt[(4 * h2 + i) * kTile + pcol] = (f16)ph[i];
    // rescale when a real head's max moved (wave-uniform: heads 0-3 as seen
    // by lane 0, heads 4-7 by lane 32)
    bool moved = false;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const bool m0 = r < GP && __builtin_amdgcn_readlane(__builtin_bit_cast(int, mn[r]), 0) !=
                                      __builtin_amdgcn_readlane(__builtin_bit_cast(int, st.m_run[r]), 0);
        const bool m1 = GP > 4 && __builtin_amdgcn_readlane(__builtin_bit_cast(int, mn[r]), 32) !=
                                      __builtin_amdgcn_readlane(__builtin_bit_cast(int, st.m_run[r]), 32);
        moved |= m0 | m1;
    }
    const int g = lane >> 4;
    float al[4] = {1.f, 1.f, 1.f, 1.f};
    if (moved) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float alpha = __builtin_amdgcn_exp2f(st.m_run[i] - mn[i]);
            st.d_part[i] *= alpha;
            st.z_part[i] *= alpha;
            // alpha of the P.V rows of this lane: heads 4 g + r (g = lane >> 4)
            const float a0 = __builtin_bit_cast(
                float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), 0));
            const float a1 = __builtin_bit_cast(
                float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), 32));
            al[i] = g == 1 ? a1 : a0;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        st.m_run[i] = mn[i];
        st.d_part[i] += pr[i];
        st.z_part[i] = __builtin_fmaf(pr[i], vz, st.z_part[i]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---------------- P.V
    if (moved) {
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) st.acc[nb][r] *= al[r];
    }
    const int i = lane & 15;
    const v8h pa = *reinterpret_cast<const v8h *>(pvt + i * kTile + 8 * g);
    // lanes e = 0..7 of group g address token 8 g + e of N-block 2 nb2, lanes
    // 8..15 the same tokens of N-block 2 nb2 + 1
    const int trow = 8 * g + (i & 7);
#pragma unroll
    for (int nb2 = 0; nb2 < 4; ++nb2) {
        const int nbk = 2 * nb2 + (i >> 3);  // 8-byte chunk = 16-dim block
        const v2i w = ds_tr4(sg + 2048 + swz(trow, nbk >> 1) + 8 * (nbk & 1));
        st.acc[2 * nb2] = mfma16h(pa, codes8(nib, (u32)w[0]), st.acc[2 * nb2]);
        st.acc[2 * nb2 + 1] = mfma16h(pa, codes8(nib, (u32)w[1]), st.acc[2 * nb2 + 1]);
    }
    __builtin_amdgcn_wave_barrier();
}

template <int NW, int S>
struct DecodeCfg {
    static constexpr int wave_lds = S * kStageBytes + kPvBytes;
    static constexpr int lds = NW * wave_lds + 4 * kMaxChunkPages;
};

// Start the direct-to-LDS loads of the tile at tb (page % 32 == 0, so the 32
// rows are consecutive entries of physical page pg: 2 KiB of K codes, 2 KiB
// of V codes, 128 B each of K and V params).  Rows past the request end are
// still inside the page and are masked by the consumer.  5 loads per lane.
SRQ_DEV void dma_tile(const Paged &p, int64_t kvh, int64_t tb, int pg, int lane, uint32_t lds) {
    const int64_t krow = k_row(p, pg, kvh, (int)tb % (int)p.page);
    const int64_t vshift = p.H * p.page;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(p.data + krow * (kD / 2), 2048);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(p.data + (krow + vshift) * (kD / 2), 2048);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(p.param + 2 * krow, vshift * 4 + 128);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int slot = 64 * half + lane;           // LDS chunk slot (row slot / 4, slot % 4)
        const int row = slot >> 2, cs = slot & 3;
        const uint32_t off = row * 64 + 16 * (cs ^ ((row >> 2) & 3));
        dma16(rk, off, lds + 1024 * half);
        dma16(rv, off, lds + 2048 + 1024 * half);
    }
    const uint32_t poff = lane < 32 ? 4 * lane : (uint32_t)(vshift * 4) + 4 * (lane - 32);
    dma4(rp, poff, lds + 4096);
}

// The same tile layout filled with ordinary loads and LDS stores (any page
// size); tokens past t1 are clamped to t1 - 1 (masked by the consumer).
SRQ_DEV void stage_tile(const Paged &p, int64_t np0, int64_t kvh, int64_t tb, int64_t t1, int lane,
                        uint8_t *sg) {
    const int lastc = (int)(t1 - 1 - tb);
    const int64_t vshift = p.H * p.page;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int slot = 64 * half + lane;
        const int row = slot >> 2, cs = slot & 3;
        const int64_t t = tb + min(row, lastc);
        const int64_t krow = k_row(p, p.indices[np0 + t / p.page], kvh, t % p.page);
        const v4i kc = *reinterpret_cast<const v4i *>(p.data + krow * (kD / 2) + 16 * cs);
        const v4i vc = *reinterpret_cast<const v4i *>(p.data + (krow + vshift) * (kD / 2) + 16 * cs);
        *reinterpret_cast<v4i *>(sg + swz(row, cs)) = kc;
        *reinterpret_cast<v4i *>(sg + 2048 + swz(row, cs)) = vc;
        if (half == 0 && cs == 0) {
            reinterpret_cast<u32 *>(sg + 4096)[row] = reinterpret_cast<const u32 *>(p.param)[krow];
            reinterpret_cast<u32 *>(sg + 4096 + 128)[row] =
                reinterpret_cast<const u32 *>(p.param)[krow + vshift];
        }
    }
    // rows 16..31 of the params come from the second half's lanes
    {
        const int row = 16 + (lane >> 2);
        if ((lane & 3) == 0) {
            const int64_t t = tb + min(row, lastc);
            const int64_t krow = k_row(p, p.indices[np0 + t / p.page], kvh, t % p.page);
            reinterpret_cast<u32 *>(sg + 4096)[row] = reinterpret_cast<const u32 *>(p.param)[krow];
            reinterpret_cast<u32 *>(sg + 4096 + 128)[row] =
                reinterpret_cast<const u32 *>(p.param)[krow + vshift];
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Decode attention of one (request, KV head, chunk); NW waves take the
// chunk's 32-token tiles round robin.  When the page size is a multiple of 32
// and the chunk's page-table slice fits in LDS, each wave streams its tiles
// through an S-deep direct-to-LDS ring; otherwise each tile is staged with
// ordinary loads.
// The 4-wave form asks for a minimum of 3 blocks per CU, which keeps the
// compiler from parking the P.V accumulators in AGPRs (171 registers, 2
// waves per SIMD without the hint; 148 VGPRs, 3 waves per SIMD with it: 37
// vs 41 us at config 3); the 8-wave form compiles to the same 148 VGPRs
// with a minimum of one block.
template <int GP, int NW, int S>
__global__ __launch_bounds__(NW * 64, NW == 4 ? 3 : 1) void decode_kernel(DecodeArgs a) {
    using Cfg = DecodeCfg<NW, S>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ float m_s[NW][8], d_s[NW][8], z_s[NW][8];

    const Paged &p = a.p;
    const int64_t b = blockIdx.x;
    const int64_t kvh = blockIdx.y;
    const int chunk = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int G = (int)a.G;

    const int64_t len = seq_len_of(p, b);
    const int64_t per = srq_cdiv(srq_cdiv(len, a.chunks), kTile) * kTile;
    const int64_t t0 = per * chunk;
    const int64_t t1 = (t0 + per < len) ? t0 + per : len;
    const int64_t np0 = p.indptr[b];

    // ---- fused form: the q rows of this KV group and the new token's k and
    // v rows, 16 lanes per row (row slot rs: q heads 0 .. G - 1, then k, v).
    // The block whose chunk holds the new token (position len - 1) writes its
    // k / v codes to the cache; every block keeps the rotated q in LDS.
    __shared__ __attribute__((aligned(16))) f16 q_new[GP * kD];
    __shared__ __attribute__((aligned(16))) u32 kv_new[2][20];  // 16 code words + param
    const bool fused = a.qkv != nullptr;
    const int64_t pos_new = len - 1;
    const bool owns_new = fused && pos_new >= t0 && pos_new < t1;
    if (fused) {
        const int rs = threadIdx.x >> 4, l = threadIdx.x & 15;
        const int kind = rs < G ? 0 : (rs == G ? 1 : 2);
        const bool act = rs < G + 2;
        const int64_t hs = a.Hq + 2 * p.H;
        const int64_t qkv_row = kind == 0 ? kvh * G + rs : (kind == 1 ? a.Hq + kvh : a.Hq + p.H + kvh);
        float v[8];
        {
            const v8h x = act ? *reinterpret_cast<const v8h *>(a.qkv + (b * hs + qkv_row) * kD + 8 * l)
                              : (v8h){};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (float)x[e];
        }
        int64_t page_new = 0;
        if (owns_new && act && kind != 0) page_new = p.indices[np0 + pos_new / p.page];
        qkv_row_transform(v, kind, l, a.cs, a.sn, a.cos_batch == 1 ? 0 : b, a.had_scale, a.rotate);
        f16 scale, zero;
        const u32 word = kv_row_codes(v, scale, zero);
        if (act && kind == 0) {
            v8h o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (f16)v[e];
            *reinterpret_cast<v8h *>(q_new + rs * kD + 8 * l) = o;
        } else if (act) {
            const int kv = kind - 1;
            kv_new[kv][l] = word;
            if (l == 0) kv_new[kv][16] = pack_param(scale, zero);
            if (owns_new) {
                const int64_t ri = row_index(p, page_new, kv, kvh, pos_new % p.page);
                reinterpret_cast<u32 *>(p.data + ri * (kD / 2))[l] = word;
                if (l == 0) reinterpret_cast<uint32_t *>(p.param)[ri] = pack_param(scale, zero);
            }
        }
    }

    // page-table slice of the chunk into LDS
    int *pt = reinterpret_cast<int *>(lds + NW * Cfg::wave_lds);
    const int ipage = (int)p.page;
    const int pfirst = t0 < t1 ? (int)(t0 / ipage) : 0;
    const int pcount = t0 < t1 ? (int)((t1 - 1) / ipage) - pfirst + 1 : 0;
    const bool pipe = ipage % kTile == 0 && pcount <= kMaxChunkPages;
    if (pipe)
        for (int i = threadIdx.x; i < pcount; i += NW * 64) pt[i] = p.indices[np0 + pfirst + i];

    DecodeState<GP> st;
    // ---- query operand: row m = head (zero for m >= G); k-step ks, half h2
    // holds dims 64 h2 + 8 ks + [0, 4, 1, 5, 2, 6, 3, 7] (the codes8 order).
    // Unfused: read from q now (the loads overlap the page-table fetch);
    // fused: from q_new after the barrier below.
    const int m = lane & 31, h2 = lane >> 5;
    auto build_q = [&](const f16 *qrow) __attribute__((always_inline)) {
        float qpart = 0.f;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            v8h raw = *reinterpret_cast<const v8h *>(qrow + 8 * ks);
            if (m >= G) raw = (v8h){};
            // odd dims meet K codes scaled by 2^-20: divide them by 16
            const f16 s16 = (f16)0.0625f;
            st.qa[ks] = (v8h){raw[0], raw[4], raw[1] * s16, raw[5] * s16,
                              raw[2], raw[6], raw[3] * s16, raw[7] * s16};
#pragma unroll
            for (int e = 0; e < 8; ++e) qpart += (float)raw[e];
        }
        qpart += __shfl_xor(qpart, 32, 64);
#pragma unroll
        for (int r = 0; r < 4; ++r) st.qs[r] = __shfl(qpart, 4 * h2 + r, 64) * a.sm_scale_log2;
    };
    if (!fused) build_q(a.q + (b * a.Hq + kvh * G + min(m, G - 1)) * kD + 64 * h2);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        st.m_run[r] = -INFINITY;
        st.d_part[r] = 0.f;
        st.z_part[r] = 0.f;
    }
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) st.acc[nb] = (v4f){};

    const Nib nib = make_nib();
    uint8_t *wlds = lds + wave * Cfg::wave_lds;
    f16 *pvt = reinterpret_cast<f16 *>(wlds + S * kStageBytes);
    const uint32_t wlds_addr = (uint32_t)(uintptr_t)wlds;
    const int64_t stride = NW * kTile;  // a wave's tiles are NW tiles apart
    int64_t tb = t0 + (int64_t)wave * kTile;
    __syncthreads();  // page-table slice (and the fused form's q_new, kv_new)
    if (fused) build_q(q_new + min(m, G - 1) * kD + 64 * h2);
    // fused form: the new token's row of the tile staged at sg (its first
    // token tbj) is replaced by the codes computed above, after the tile
    // has landed: whatever the tile's loads read from that cache row (the
    // block's own write may or may not have reached memory) is overwritten.
    auto put_new = [&](uint8_t *sg, int64_t tbj) __attribute__((always_inline)) {
        if (!owns_new || pos_new < tbj || pos_new >= tbj + kTile) return;
        const int r = (int)(pos_new - tbj);
        if (lane < 8) {
            const int kv = lane >> 2, c = lane & 3;
            const v4i w = *reinterpret_cast<const v4i *>(&kv_new[kv][4 * c]);
            *reinterpret_cast<v4i *>(sg + 2048 * kv + swz(r, c)) = w;
        } else if (lane < 10) {
            const int kv = lane - 8;
            reinterpret_cast<u32 *>(sg + 4096 + 128 * kv)[r] = kv_new[kv][16];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };

    if (pipe) {
        // iteration j issues tile j + S - 1 into stage (j + S - 1) % S, then
        // waits until only the S - 1 newest tiles' 5 loads each may be
        // outstanding: tile j has landed
        const int ntiles = tb < t1 ? (int)srq_cdiv(t1 - tb, stride) : 0;
        auto issue = [&](int j) {
            // past the end: the last tile again, so every step issues 5 loads
            const int tj = (int)tb + min(j, ntiles - 1) * (int)stride;
            const int pg = __builtin_amdgcn_readfirstlane(pt[tj / ipage - pfirst]);
            dma_tile(p, kvh, tj, pg, lane, wlds_addr + (j % S) * kStageBytes);
        };
        if (ntiles > 0) {
#pragma unroll
            for (int j = 0; j < S - 1; ++j) issue(j);
            for (int j = 0; j < ntiles; ++j) {
                issue(j + S - 1);
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(5 * (S - 1)) : "memory");
                put_new(wlds + (j % S) * kStageBytes, tb + (int64_t)j * stride);
                tile_step<GP>(st, wlds + (j % S) * kStageBytes, tb + (int64_t)j * stride, t1, lane,
                              a.sm_scale_log2, pvt, nib);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
    } else {
        for (; tb < t1; tb += stride) {
            stage_tile(p, np0, kvh, tb, t1, lane, wlds);
            put_new(wlds, tb);
            tile_step<GP>(st, wlds, tb, t1, lane, a.sm_scale_log2, pvt, nib);
        }
    }

    // ---- reduce d, z within each 32-lane half
#pragma unroll
    for (int off = 1; off < 32; off <<= 1)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            st.d_part[r] += __shfl_xor(st.d_part[r], off, 64);
            st.z_part[r] += __shfl_xor(st.z_part[r], off, 64);
        }
    // the stage buffers are reused for the cross-wave merge
    __syncthreads();
    float(*o_s)[GP][kD] = reinterpret_cast<float(*)[GP][kD]>(lds);
    if (lane == 0 || lane == 32) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            m_s[wave][4 * h2 + r] = st.m_run[r];
            d_s[wave][4 * h2 + r] = st.d_part[r];
            z_s[wave][4 * h2 + r] = st.z_part[r];
        }
    }
    {
        const int g = lane >> 4, i = lane & 15;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (4 * g + r < GP)
#pragma unroll
                for (int nb = 0; nb < 8; ++nb)
                    o_s[wave][4 * g + r][16 * nb + i] = st.acc[nb][r] * 16777216.f;
    }
    __syncthreads();

    // ---- merge the waves: thread (h, d) for h < G, d < 128
    for (int idx = threadIdx.x; idx < G * kD; idx += NW * 64) {
        const int h = idx / kD, d = idx - h * kD;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) mx = fmaxf(mx, m_s[w][h]);
        float ov = 0.f, dv = 0.f, zv = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float sc = m_s[w][h] == -INFINITY ? 0.f : exp2f(m_s[w][h] - mx);
            ov += o_s[w][h][d] * sc;
            dv += d_s[w][h] * sc;
            zv += z_s[w][h] * sc;
        }
        const float num = ov - zv;  // sum p (c s - z), un-normalised
        const int64_t hq = kvh * G + h;
        if (a.chunks == 1) {
            a.o[(b * a.Hq + hq) * kD + d] = (f16)(dv > 0.f ? num / dv : 0.f);
        } else {
            float *rec = a.tmp + ((b * a.Hq + hq) * a.chunks + chunk) * (kD + 4);
            rec[d] = num;
            if (d == 0) {
                rec[kD] = mx;
                rec[kD + 1] = dv;
            }
        }
    }
}

// Merge of the per-chunk (o, m, d) records of one (request, query head) at
// dim d: o = sum_c o_c 2^(m_c - m) / sum_c d_c 2^(m_c - m), m = max_c m_c
// (decode.cuh:726-751), fp16.
SRQ_DEV f16 merge_rec(const float *rec, int chunks, int d) {
    float mx = -INFINITY;
    for (int c = 0; c < chunks; ++c) mx = fmaxf(mx, rec[c * (kD + 4) + kD]);
    float ov = 0.f, dv = 0.f;
    for (int c = 0; c < chunks; ++c) {
        const float mc = rec[c * (kD + 4) + kD];
        const float sc = mc == -INFINITY ? 0.f : exp2f(mc - mx);
        ov += rec[c * (kD + 4) + d] * sc;
        dv += rec[c * (kD + 4) + kD + 1] * sc;
    }
    return (f16)(dv > 0.f ? ov / dv : 0.f);
}

// (head, chunk) records one merge_head_had_quant block stages in LDS (64 KiB)
constexpr int kMergeHhqMaxRecords = 65536 / ((kD + 4) * 4);
static_assert(kMergeHhqMaxRecords * ((kD + 4) / 4) <= 16 * 256, "record copy: 16 float4 / thread");

__global__ __launch_bounds__(128) void merge_kernel(const float *__restrict__ tmp, f16 *__restrict__ o,
                                                    int64_t Hq, int chunks) {
    const int64_t bh = blockIdx.x;
    const int d = threadIdx.x;
    o[bh * kD + d] = merge_rec(tmp + bh * chunks * (kD + 4), chunks, d);
}

// ------------------------------------------------- head Hadamard + quant
// Input of the o_proj of a decode step (modeling_llama.py:94, 117): the
// attention output x [B, H, D] is rotated over the head axis,
//   y[b, h, d] = fp16(FWHT_H(x[b, :, d])[h] * scale),
// and the row y[b] (element h * D + d) is quantized per token (symmetric
// int4, sym_quant_dynamic arithmetic).  One block per b: thread d holds the
// H values of column d in registers (stages in ascending bit, as the FWHT
// kernel), the rotated row is staged in LDS as fp16, then packed eight
// codes per 32-bit word.  MERGE: x is not given; the attention output of
// head h is merged from the split-KV partial states in tmp first (the
// merge_kernel arithmetic, so the same fp16 values), which saves the merge
// launch and its round trip through memory.  The block's records (H chunks
// x 132 floats, contiguous in tmp) are copied to LDS by all threads at once
// first: merging from global memory per thread would chain H x chunks
// dependent round trips.
template <int H, bool MERGE>
__global__ __launch_bounds__(256) void head_had_quant_kernel(const f16 *__restrict__ x, int D,
                                                             float scale, float clip,
                                                             u32 *__restrict__ q,
                                                             f16 *__restrict__ qscale,
                                                             f16 *__restrict__ rot,
                                                             const float *__restrict__ tmp,
                                                             int chunks) {
    __shared__ __attribute__((aligned(16))) f16 buf[H * 256];
    __shared__ float red[4];
    __shared__ int redb[4];
    extern __shared__ __attribute__((aligned(16))) float recs[];  // MERGE: H chunks records
    __shared__ float scs[MERGE ? kMergeHhqMaxRecords : 1];  // MERGE: 2^(m_c - m) per (h, c)
    __shared__ float dvs[MERGE ? H : 1];                     // MERGE: denominators per h
    const int64_t b = blockIdx.x;
    const f16 *xb = MERGE ? nullptr : x + b * H * D;
    if (MERGE) {
        // at most 64 KiB: 16 float4 per thread, all loads issued before the
        // first store (a plain copy loop waits for each load in turn)
        const int n4 = H * chunks * ((kD + 4) / 4);
        const v4f *src = reinterpret_cast<const v4f *>(tmp + b * H * chunks * (kD + 4));
        v4f t[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int i = threadIdx.x + 256 * k;
            t[k] = i < n4 ? src[i] : (v4f){};
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int i = threadIdx.x + 256 * k;
            if (i < n4) reinterpret_cast<v4f *>(recs)[i] = t[k];
        }
        __syncthreads();
        // per head: the chunk weights and the denominator (merge_rec's
        // arithmetic and order)
        if (threadIdx.x < H) {
            const int h = threadIdx.x;
            const float *rh = recs + h * chunks * (kD + 4);
            float mx = -INFINITY;
            for (int c = 0; c < chunks; ++c) mx = fmaxf(mx, rh[c * (kD + 4) + kD]);
            float dv = 0.f;
            for (int c = 0; c < chunks; ++c) {
                const float mc = rh[c * (kD + 4) + kD];
                const float sc = mc == -INFINITY ? 0.f : exp2f(mc - mx);
                scs[h * chunks + c] = sc;
                dv += rh[c * (kD + 4) + kD + 1] * sc;
            }
            dvs[h] = dv;
        }
        __syncthreads();
    }
    float amax = 0.f;
    bool bad = false;
    const int d = threadIdx.x;
    if (d < D) {
        float v[H];
        if constexpr (MERGE) {
            // chunks outer, heads inner: H independent sums, each in chunk order
#pragma unroll
            for (int h = 0; h < H; ++h) v[h] = 0.f;
            for (int c = 0; c < chunks; ++c)
#pragma unroll
                for (int h = 0; h < H; ++h)
                    v[h] += recs[(h * chunks + c) * (kD + 4) + d] * scs[h * chunks + c];
#pragma unroll
            for (int h = 0; h < H; ++h)
                v[h] = (float)(f16)(dvs[h] > 0.f ? v[h] / dvs[h] : 0.f);
        } else {
#pragma unroll
            for (int h = 0; h < H; ++h) v[h] = (float)xb[h * D + d];
        }
        fwht_regs<H>(v);
#pragma unroll
        for (int h = 0; h < H; ++h) {
            const f16 y = f16_rn(v[h] * scale);
            buf[h * D + d] = y;
            const float a = fabsf((float)y);
            amax = fmaxf(amax, a);
            bad |= !(a <= 65504.f);
        }
    }
    amax = wave_max(amax);
    // the ballot runs with the whole wave active (inside the lane-0 branch it
    // would see lane 0's flag only)
    const bool wbad = __builtin_amdgcn_ballot_w64(bad) != 0;
    if ((threadIdx.x & 63) == 0) {
        red[threadIdx.x >> 6] = amax;
        redb[threadIdx.x >> 6] = wbad;
    }
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const bool anybad = (redb[0] | redb[1] | redb[2] | redb[3]) != 0;
    const f16 s = sym_row_scale(amax, clip);
    if (threadIdx.x == 0) qscale[b] = s;
    const float sf = (float)s;
    const float rcp = sym_rcp_safe(sf);
    const bool clampit = sym_row_needs_clamp(amax, sf);
    const int nw = H * D / 8;
    for (int w = threadIdx.x; w < nw; w += 256) {
        const v8h v = *reinterpret_cast<const v8h *>(buf + 8 * w);
        q[b * nw + w] = anybad    ? pack8_sym(v, sf)
                        : clampit ? pack8_sym_fast<true>(v, rcp)
                                  : pack8_sym_fast<false>(v, rcp);
        if (rot) reinterpret_cast<v8h *>(rot)[b * nw + w] = v;
    }
}

int check_paged(const char *name, const void *data, const void *param, const void *indptr,
                const void *indices, const void *last, int64_t L, int64_t layer, int64_t H,
                int64_t page, int64_t D) {
    SRQ_CHECK_ARG(data && param && indptr && indices && last, "%s: null cache pointer", name);
    SRQ_CHECK_ARG(L > 0 && layer >= 0 && layer < L, "%s: layer %lld outside [0, %lld)", name,
                  (long long)layer, (long long)L);
    SRQ_CHECK_ARG(H > 0 && page > 0, "%s: bad heads/page size", name);
    SRQ_CHECK_ARG(D == kD, "%s: head_dim must be 128 (got %lld)", name, (long long)D);
    SRQ_CHECK_ARG(srq_aligned(data, 16) && srq_aligned(param, 4),
                  "%s: cache data must be 16-byte and params 4-byte aligned", name);
    return SRQ_OK;
}

Paged make_paged(void *data, void *param, const int32_t *indptr, const int32_t *indices,
                 const int32_t *last, int64_t L, int64_t layer, int64_t H, int64_t page,
                 int64_t D) {
    Paged p;
    p.data = (uint8_t *)data;
    p.param = (f16 *)param;
    p.indptr = indptr;
    p.indices = indices;
    p.last = last;
    p.L = L;
    p.layer = layer;
    p.H = H;
    p.page = page;
    p.D = D;
    return p;
}

}  // namespace

namespace {

int launch_append(const char *name, void *kv_data, void *kv_param, const int32_t *kv_indptr,
                  const int32_t *kv_indices, const int32_t *last_page_offset, const void *k,
                  const void *v, const void *k_param, const void *v_param,
                  const int32_t *seqlen_indptr, int64_t batch, int64_t tokens, int64_t num_layers,
                  int64_t layer_idx, int64_t num_heads, int64_t page_size, int64_t head_dim,
                  void *stream) {
    int rc = check_paged(name, kv_data, kv_param, kv_indptr, kv_indices, last_page_offset,
                         num_layers, layer_idx, num_heads, page_size, head_dim);
    if (rc) return rc;
    SRQ_CHECK_ARG(batch >= 0 && batch <= 65535 && tokens >= 0, "%s: bad batch (%lld) or tokens",
                  name, (long long)batch);
    if (batch == 0 || tokens == 0) return SRQ_OK;
    SRQ_CHECK_ARG(k && v && k_param && v_param, "%s: null K/V pointer", name);
    SRQ_CHECK_ARG(srq_aligned(k, 16) && srq_aligned(v, 16) && srq_aligned(k_param, 4) &&
                      srq_aligned(v_param, 4),
                  "%s: K/V codes must be 16-byte and params 4-byte aligned", name);
    Paged p = make_paged(kv_data, kv_param, kv_indptr, kv_indices, last_page_offset, num_layers,
                         layer_idx, num_heads, page_size, head_dim);
    // grid-stride over each request's tokens; size x for the average request
    const int64_t work = srq_cdiv(tokens, batch) * num_heads * (head_dim / 32 + 1);
    const dim3 grid((unsigned)std::max<int64_t>(1, std::min<int64_t>(srq_cdiv(work, 256), 1024)),
                    (unsigned)batch);
    append_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(
        p, (const uint8_t *)k, (const uint8_t *)v, (const f16 *)k_param, (const f16 *)v_param,
        seqlen_indptr, batch);
    SRQ_LAUNCH_CHECK(name);
    return SRQ_OK;
}

}  // namespace

extern "C" int srq_append_kv_i4(void *kv_data, void *kv_param, const int32_t *kv_indptr,
                                const int32_t *kv_indices, const int32_t *last_page_offset,
                                const void *k, const void *v, const void *k_param,
                                const void *v_param, int64_t batch, int64_t num_layers,
                                int64_t layer_idx, int64_t num_heads, int64_t page_size,
                                int64_t head_dim, void *stream) {
    return launch_append("append_kv_i4", kv_data, kv_param, kv_indptr, kv_indices,
                         last_page_offset, k, v, k_param, v_param, nullptr, batch, batch,
                         num_layers, layer_idx, num_heads, page_size, head_dim, stream);
}

extern "C" int srq_init_kv_i4(void *kv_data, void *kv_param, const int32_t *kv_indptr,
                              const int32_t *kv_indices, const int32_t *last_page_offset,
                              const void *k, const void *v, const void *k_param,
                              const void *v_param, const int32_t *seqlen_indptr, int64_t batch,
                              int64_t total_tokens, int64_t num_layers, int64_t layer_idx,
                              int64_t num_heads, int64_t page_size, int64_t head_dim,
                              void *stream) {
    SRQ_CHECK_ARG(seqlen_indptr || batch == 0, "init_kv_i4: null seqlen_indptr");
    return launch_append("init_kv_i4", kv_data, kv_param, kv_indptr, kv_indices,
                         last_page_offset, k, v, k_param, v_param, seqlen_indptr, batch,
                         total_tokens, num_layers, layer_idx, num_heads, page_size, head_dim,
                         stream);
}

namespace {

// Waves per block and ring depth of the decode kernel.  Split launches
// (chunks > 1) run 4-wave blocks, two per CU; an unsplit launch runs 8-wave
// blocks, one per CU: the same waves per CU, and when the batch alone fills
// the CUs (B x KV heads >= CUs) no split is needed, so the partial states
// need no merge pass (config 3: 36.3 us unsplit with 8 waves against 37.6
// split in two with 4, and the head-axis quantizer then skips the merge:
// 39.9 against 42.5 us for both launches).
constexpr int kDecodeS = 2;

template <int GP, int NW>
int launch_decode_nw(const DecodeArgs &a, dim3 grid, hipStream_t st) {
    constexpr int S = kDecodeS;
    using Cfg = DecodeCfg<NW, S>;
    auto kern = decode_kernel<GP, NW, S>;
    static_assert(Cfg::lds <= 160 * 1024 - 4096, "decode LDS");
    if (Cfg::lds > 64 * 1024 &&
        hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                            Cfg::lds) != hipSuccess) {
        srq_set_error("batch_decode_i4: cannot reserve %d bytes of LDS", Cfg::lds);
        return SRQ_ELAUNCH;
    }
    kern<<<grid, NW * 64, Cfg::lds, st>>>(a);
    return SRQ_OK;
}

template <int GP>
int launch_decode_g(const DecodeArgs &a, dim3 grid, hipStream_t st) {
    return a.chunks == 1 ? launch_decode_nw<GP, 8>(a, grid, st) : launch_decode_nw<GP, 4>(a, grid, st);
}

int launch_decode(const DecodeArgs &a, dim3 grid, hipStream_t st) {
    if (a.G == 1) return launch_decode_g<1>(a, grid, st);
    if (a.G == 2) return launch_decode_g<2>(a, grid, st);
    if (a.G <= 4) return launch_decode_g<4>(a, grid, st);
    return launch_decode_g<8>(a, grid, st);
}

}  // namespace

extern "C" int srq_batch_decode_i4(void *o, const void *q, const void *kv_data,
                                   const void *kv_param, const int32_t *kv_indptr,
                                   const int32_t *kv_indices, const int32_t *last_page_offset,
                                   int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
                                   int64_t num_layers, int64_t layer_idx, int64_t page_size,
                                   int64_t head_dim, float *tmp, int64_t num_chunks,
                                   void *stream) {
    int rc = check_paged("batch_decode_i4", kv_data, kv_param, kv_indptr, kv_indices,
                         last_page_offset, num_layers, layer_idx, num_kv_heads, page_size,
                         head_dim);
    if (rc) return rc;
    SRQ_CHECK_ARG(batch >= 0 && num_qo_heads > 0 && num_kv_heads <= 65535,
                  "batch_decode_i4: bad batch/heads");
    SRQ_CHECK_ARG(num_qo_heads % num_kv_heads == 0 && num_qo_heads / num_kv_heads <= 8,
                  "batch_decode_i4: query heads (%lld) must be 1..8 times the KV heads (%lld)",
                  (long long)num_qo_heads, (long long)num_kv_heads);
    if (batch == 0) return SRQ_OK;
    if (num_chunks < 1 || tmp == nullptr) num_chunks = 1;
    // o == NULL: the split partial states stay in tmp, unmerged
    SRQ_CHECK_ARG(q && (o || num_chunks > 1), "batch_decode_i4: null q/o");
    SRQ_CHECK_ARG(srq_aligned(q, 16), "batch_decode_i4: q must be 16-byte aligned");
    SRQ_CHECK_ARG(num_chunks <= 1024, "batch_decode_i4: num_chunks > 1024");
    DecodeArgs a;
    a.p = make_paged((void *)kv_data, (void *)kv_param, kv_indptr, kv_indices, last_page_offset,
                     num_layers, layer_idx, num_kv_heads, page_size, head_dim);
    a.q = (const f16 *)q;
    a.o = (f16 *)o;
    a.tmp = tmp;
    a.B = batch;
    a.Hq = num_qo_heads;
    a.G = num_qo_heads / num_kv_heads;
    a.chunks = (int)num_chunks;
    a.sm_scale_log2 = (1.0f / sqrtf((float)head_dim)) * 1.44269504088896340736f;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)batch, (unsigned)num_kv_heads, (unsigned)num_chunks);
    rc = launch_decode(a, grid, st);
    if (rc) return rc;
    SRQ_LAUNCH_CHECK("batch_decode_i4");
    if (num_chunks > 1 && o) {
        merge_kernel<<<dim3((unsigned)(batch * num_qo_heads)), 128, 0, st>>>(tmp, (f16 *)o,
                                                                          num_qo_heads,
                                                                          (int)num_chunks);
        SRQ_LAUNCH_CHECK("batch_decode_i4 (merge)");
    }
    return SRQ_OK;
}

extern "C" int srq_qkv_decode_i4(void *o, const void *qkv, const void *cos, const void *sin,
                                 int64_t cos_batch, float had_scale, int rotate, void *kv_data,
                                 void *kv_param, const int32_t *kv_indptr,
                                 const int32_t *kv_indices, const int32_t *last_page_offset,
                                 int64_t batch, int64_t num_qo_heads, int64_t num_kv_heads,
                                 int64_t num_layers, int64_t layer_idx, int64_t page_size,
                                 int64_t head_dim, float *tmp, int64_t num_chunks, void *stream) {
    const char *name = "qkv_decode_i4";
    int rc = check_paged(name, kv_data, kv_param, kv_indptr, kv_indices, last_page_offset,
                         num_layers, layer_idx, num_kv_heads, page_size, head_dim);
    if (rc) return rc;
    SRQ_CHECK_ARG(batch >= 0 && num_qo_heads > 0 && num_kv_heads <= 65535,
                  "%s: bad batch/heads", name);
    SRQ_CHECK_ARG(num_qo_heads % num_kv_heads == 0 && num_qo_heads / num_kv_heads <= 8,
                  "%s: query heads (%lld) must be 1..8 times the KV heads (%lld)", name,
                  (long long)num_qo_heads, (long long)num_kv_heads);
    SRQ_CHECK_ARG(cos_batch == 1 || cos_batch == batch, "%s: cos/sin batch must be 1 or B",
                  name);
    if (batch == 0) return SRQ_OK;
    if (num_chunks < 1 || tmp == nullptr) num_chunks = 1;
    SRQ_CHECK_ARG(qkv && cos && sin && (o || num_chunks > 1), "%s: null pointer", name);
    SRQ_CHECK_ARG(srq_aligned(qkv, 16), "%s: qkv must be 16-byte aligned", name);
    SRQ_CHECK_ARG(num_chunks <= 1024, "%s: num_chunks > 1024", name);
    DecodeArgs a;
    a.p = make_paged(kv_data, kv_param, kv_indptr, kv_indices, last_page_offset, num_layers,
                     layer_idx, num_kv_heads, page_size, head_dim);
    a.q = nullptr;
    a.qkv = (const f16 *)qkv;
    a.cs = (const f16 *)cos;
    a.sn = (const f16 *)sin;
    a.cos_batch = (int)cos_batch;
    a.rotate = rotate ? 1 : 0;
    a.had_scale = had_scale;
    a.o = (f16 *)o;
    a.tmp = tmp;
    a.B = batch;
    a.Hq = num_qo_heads;
    a.G = num_qo_heads / num_kv_heads;
    a.chunks = (int)num_chunks;
    a.sm_scale_log2 = (1.0f / sqrtf((float)head_dim)) * 1.44269504088896340736f;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)batch, (unsigned)num_kv_heads, (unsigned)num_chunks);
    rc = launch_decode(a, grid, st);
    if (rc) return rc;
    SRQ_LAUNCH_CHECK(name);
    if (num_chunks > 1 && o) {
        merge_kernel<<<dim3((unsigned)(batch * num_qo_heads)), 128, 0, st>>>(tmp, (f16 *)o,
                                                                          num_qo_heads,
                                                                          (int)num_chunks);
        SRQ_LAUNCH_CHECK("qkv_decode_i4 (merge)");
    }
    return SRQ_OK;
}

// ------------------------------------ allocation-free split-KV decode
// The split-KV partial states of srq_batch_decode_i4_noalloc live in this
// file-scope device array instead of a caller workspace.  Each GPU the
// library runs on holds its own copy (kDecodeScratchBytes) until the process
// ends.  On the host `scratch` names a host-side stand-in, not device memory:
// the device address of the current GPU's copy comes from
// hipGetSymbolAddress, once per device, and only that address is passed on.
namespace {
constexpr int64_t kDecodeScratchBytes = 8LL << 20;
constexpr int kMaxDevices = 64;
std::atomic<float *> g_scratch_addr[kMaxDevices];
std::atomic_flag g_scratch_lock = ATOMIC_FLAG_INIT;  // first lookup per device
}  // namespace

static __device__ __align__(256) float scratch[kDecodeScratchBytes / sizeof(float)];

// Device address of the current device's `scratch` (looked up on the first
// call per device, with that device current).
static int decode_scratch(hipStream_t st, float **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        srq_set_error("batch_decode_i4_noalloc: no current HIP device (or index >= %d)",
                      kMaxDevices);
        return SRQ_ELAUNCH;
    }
    if (st) {
        hipDevice_t sdev = -1;
        if (hipStreamGetDevice(st, &sdev) != hipSuccess || sdev != dev) {
            srq_set_error("batch_decode_i4_noalloc: the stream is not on the current device %d",
                          dev);
            return SRQ_EINVAL;
        }
    }
    float *p = g_scratch_addr[dev].load(std::memory_order_acquire);
    if (!p) {
        while (g_scratch_lock.test_and_set(std::memory_order_acquire)) {
        }
        p = g_scratch_addr[dev].load(std::memory_order_relaxed);
        hipError_t e = hipSuccess;
        if (!p) {
            void *addr = nullptr;
            e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
            if (e == hipSuccess && addr) {
                p = static_cast<float *>(addr);
                g_scratch_addr[dev].store(p, std::memory_order_release);
            }
        }
        g_scratch_lock.clear(std::memory_order_release);
        if (!p) {
            srq_set_error("batch_decode_i4_noalloc: hipGetSymbolAddress(scratch) failed on "
                          "device %d: %s", dev, hipGetErrorString(e));
            return SRQ_ELAUNCH;
        }
    }
    *out = p;
    return SRQ_OK;
}

extern "C" int srq_batch_decode_i4_noalloc(void *o, const void *q, const void *kv_data,
                                           const void *kv_param, const int32_t *kv_indptr,
                                           const int32_t *kv_indices,
                                           const int32_t *last_page_offset, int64_t batch,
                                           int64_t num_qo_heads, int64_t num_kv_heads,
                                           int64_t num_layers, int64_t layer_idx,
                                           int64_t page_size, int64_t head_dim,
                                           int64_t num_chunks, void *stream) {
    if (num_chunks <= 1 || batch <= 0)
        return srq_batch_decode_i4(o, q, kv_data, kv_param, kv_indptr, kv_indices,
                                   last_page_offset, batch, num_qo_heads, num_kv_heads,
                                   num_layers, layer_idx, page_size, head_dim, nullptr, 1,
                                   stream);
    // with chunks and no o the workspace form leaves the unmerged partial
    // states in tmp, which here is the library's private scratch: refuse
    SRQ_CHECK_ARG(o, "batch_decode_i4_noalloc: null output (the split-KV partial states "
                     "would stay in the library's private scratch)");
    SRQ_CHECK_ARG(num_qo_heads > 0 && head_dim > 0 && num_chunks <= 1024,
                  "batch_decode_i4_noalloc: bad heads, head_dim or num_chunks");
    const int64_t need = batch * num_qo_heads * num_chunks * (head_dim + 4) * (int64_t)sizeof(float);
    SRQ_CHECK_ARG(need <= kDecodeScratchBytes,
                  "batch_decode_i4_noalloc: batch %lld x %lld heads x %lld chunks needs %lld "
                  "bytes of split-KV state, more than the fixed %lld-byte scratch (use fewer "
                  "chunks or srq_batch_decode_i4 with a workspace)",
                  (long long)batch, (long long)num_qo_heads, (long long)num_chunks,
                  (long long)need, (long long)kDecodeScratchBytes);
    float *tmp = nullptr;
    const int rc = decode_scratch((hipStream_t)stream, &tmp);
    if (rc) return rc;
    return srq_batch_decode_i4(o, q, kv_data, kv_param, kv_indptr, kv_indices, last_page_offset,
                               batch, num_qo_heads, num_kv_heads, num_layers, layer_idx,
                               page_size, head_dim, tmp, num_chunks, stream);
}


extern "C" int srq_qkv_rope_had_append(const void *qkv, const void *cos, const void *sin,
                                       int64_t cos_batch, int64_t batch, int64_t n_q_heads,
                                       int64_t n_kv_heads, int64_t head_dim, float had_scale,
                                       int rotate, void *q_out, void *kv_data, void *kv_param,
                                       const int32_t *kv_indptr, const int32_t *kv_indices,
                                       const int32_t *last_page_offset, int64_t num_layers,
                                       int64_t layer_idx, int64_t page_size, void *stream) {
    const char *name = "qkv_rope_had_append";
    int rc = check_paged(name, kv_data, kv_param, kv_indptr, kv_indices, last_page_offset,
                         num_layers, layer_idx, n_kv_heads, page_size, head_dim);
    if (rc) return rc;
    SRQ_CHECK_ARG(batch >= 0 && n_q_heads > 0 && n_kv_heads > 0 && n_q_heads <= 1024 &&
                      n_kv_heads <= 1024,
                  "%s: bad batch or head counts", name);
    SRQ_CHECK_ARG(cos_batch == 1 || cos_batch == batch, "%s: cos/sin batch must be 1 or B",
                  name);
    if (batch == 0) return SRQ_OK;
    SRQ_CHECK_ARG(qkv && cos && sin && q_out, "%s: null pointer", name);
    SRQ_CHECK_ARG(srq_aligned(qkv, 16) && srq_aligned(q_out, 16),
                  "%s: qkv and q_out must be 16-byte aligned", name);
    QkvArgs a;
    a.qkv = (const f16 *)qkv;
    a.cs = (const f16 *)cos;
    a.sn = (const f16 *)sin;
    a.cos_batch = (int)cos_batch;
    a.B = batch;
    a.hq = (int)n_q_heads;
    a.hk = (int)n_kv_heads;
    a.had_scale = had_scale;
    a.rotate = rotate ? 1 : 0;
    a.q_out = (f16 *)q_out;
    Paged p = make_paged(kv_data, kv_param, kv_indptr, kv_indices, last_page_offset, num_layers,
                         layer_idx, n_kv_heads, page_size, head_dim);
    const int64_t rows = batch * (n_q_heads + 2 * n_kv_heads);
    const int64_t blocks = srq_cdiv(rows, 16);
    SRQ_CHECK_ARG(blocks <= 0x7fffffffLL, "%s: too many rows", name);
    qkv_post_kernel<<<dim3((unsigned)blocks), 256, 0, (hipStream_t)stream>>>(a, p);
    SRQ_LAUNCH_CHECK(name);
    return SRQ_OK;
}

namespace {
template <bool MERGE>
void launch_head_had_quant(const void *x, const float *tmp, int chunks, int64_t batch,
                           int64_t n_heads, int D, float scale, float clip_ratio, void *q,
                           void *qscale, void *rot, hipStream_t st) {
    const dim3 grid((unsigned)batch);
    const size_t dyn = MERGE ? (size_t)n_heads * chunks * (kD + 4) * sizeof(float) : 0;
    switch (n_heads) {
#define SRQ_HHQ(HH)                                                                       \
    case HH:                                                                              \
        head_had_quant_kernel<HH, MERGE><<<grid, 256, dyn, st>>>(                         \
            (const f16 *)x, D, scale, clip_ratio, (u32 *)q, (f16 *)qscale, (f16 *)rot,    \
            tmp, chunks);                                                                 \
        break;
        SRQ_HHQ(1)
        SRQ_HHQ(2)
        SRQ_HHQ(4)
        SRQ_HHQ(8)
        SRQ_HHQ(16)
        SRQ_HHQ(32)
        SRQ_HHQ(64)
#undef SRQ_HHQ
    }
}
}  // namespace

extern "C" int srq_head_had_quant(const void *x, int64_t batch, int64_t n_heads, int64_t head_dim,
                                  float scale, float clip_ratio, void *q, void *qscale, void *rot,
                                  void *stream) {
    SRQ_CHECK_ARG(batch >= 0 && n_heads > 0 && head_dim > 0, "head_had_quant: bad shape");
    SRQ_CHECK_ARG(n_heads <= 64 && (n_heads & (n_heads - 1)) == 0,
                  "head_had_quant: n_heads=%lld must be a power of two <= 64",
                  (long long)n_heads);
    SRQ_CHECK_ARG(head_dim <= 256 && head_dim % 8 == 0,
                  "head_had_quant: head_dim=%lld must be a multiple of 8 and <= 256",
                  (long long)head_dim);
    SRQ_CHECK_ARG(batch <= 0x7fffffffLL, "head_had_quant: batch > 2^31-1");
    if (batch == 0) return SRQ_OK;
    SRQ_CHECK_ARG(x && q && qscale, "head_had_quant: null pointer");
    SRQ_CHECK_ARG(srq_aligned(q, 4) && (!rot || srq_aligned(rot, 16)),
                  "head_had_quant: q must be 4-byte and rot 16-byte aligned");
    launch_head_had_quant<false>(x, nullptr, 1, batch, n_heads, (int)head_dim, scale, clip_ratio,
                                 q, qscale, rot, (hipStream_t)stream);
    SRQ_LAUNCH_CHECK("head_had_quant");
    return SRQ_OK;
}

extern "C" int srq_merge_head_had_quant(const float *tmp, int64_t batch, int64_t n_heads,
                                        int64_t head_dim, int64_t num_chunks, float scale,
                                        float clip_ratio, void *q, void *qscale, void *rot,
                                        void *stream) {
    SRQ_CHECK_ARG(batch >= 0 && n_heads > 0, "merge_head_had_quant: bad shape");
    SRQ_CHECK_ARG(head_dim == kD, "merge_head_had_quant: head_dim must be %d (got %lld)", kD,
                  (long long)head_dim);
    SRQ_CHECK_ARG(n_heads <= 64 && (n_heads & (n_heads - 1)) == 0,
                  "merge_head_had_quant: n_heads=%lld must be a power of two <= 64",
                  (long long)n_heads);
    SRQ_CHECK_ARG(num_chunks >= 1 && n_heads * num_chunks <= kMergeHhqMaxRecords,
                  "merge_head_had_quant: n_heads * num_chunks = %lld outside [1, %d] (the "
                  "records are staged in LDS)", (long long)(n_heads * num_chunks),
                  kMergeHhqMaxRecords);
    SRQ_CHECK_ARG(batch <= 0x7fffffffLL, "merge_head_had_quant: batch > 2^31-1");
    if (batch == 0) return SRQ_OK;
    SRQ_CHECK_ARG(tmp && q && qscale, "merge_head_had_quant: null pointer");
    SRQ_CHECK_ARG(srq_aligned(q, 4) && (!rot || srq_aligned(rot, 16)),
                  "merge_head_had_quant: q must be 4-byte and rot 16-byte aligned");
    launch_head_had_quant<true>(nullptr, tmp, (int)num_chunks, batch, n_heads, kD, scale,
                                clip_ratio, q, qscale, rot, (hipStream_t)stream);
    SRQ_LAUNCH_CHECK("merge_head_had_quant");
    return SRQ_OK;
}

