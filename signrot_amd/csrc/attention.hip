// Prefill attention over fp16 q/k/v: the causal, grouped-query softmax
// attention that the quantized Llama layer runs on the first (prefill) call
// of a layer, where the reference calls flash-attn 2 through transformers'
// _flash_attention_forward (e2e/quantized_llama/modeling_llama.py:81-90).
// Key positions whose attention_mask entry is 0 are dropped and the output
// rows of masked query positions are zero, which is what the unpad ->
// varlen attention -> pad round trip of that call produces.  Masked keys and
// masked query rows are never read (their K, V and q stage as zeros), so
// whatever a padded position holds, NaN or inf included, cannot reach a
// live row -- the unpad step of the reference never reads them either.
//
// One block = NWV waves over QB = 32 NWV / GH query rows of GH q heads of
// one KV head (sequence b): wave w owns rows [32 (w / GH), + 32) of q head
// w % GH of the group, so each K/V tile staged in LDS serves all GH heads
// that share it (GH = the GQA group size up to 8, in 8-wave blocks; a
// 4-wave block of one head otherwise).  Everything is computed transposed
// so that one lane owns one query row (column l % 32 of the MFMA output):
//   S^T[key][q] = K_tile (64 x 128) . Q^T            fp16 MFMA 32x32x16
//   O^T[d][q]  += V^T (128 x 64)  . P^T               fp16 MFMA 32x32x16
// The MFMA output layout (lane l, register v -> row 8(v/4) + 4(l/32) + v%4,
// column l%32) leaves each lane 16 keys of its own row per 32-key block, so
// the running max / sum of the online softmax are in-lane values plus one
// exchange with lane l ^ 32; P^T becomes the B operand of the PV product
// straight from the lane's registers if the 16 k-slots of each PV step are
// assigned to keys in that same order (k-slot j of lane half g <-> key
// 8(j/4) + 4g + j%4 of the 16-key step).  V stays row-major in LDS and its
// V^T operand comes from gfx950's transposing LDS read (ds_read_b64_tr_b16:
// within each 16 lanes, lane 4a + b receives half b of the 8 bytes read by
// lanes a, a + 4, a + 8, a + 12): lanes reading rows k0 + j / 4, columns
// d + 4 (j % 4) (j = lane % 16) hand lane j the 4 keys k0..k0+3 of column
// d + j, one group of 4 k-slots (two reads per operand).
// Logits are q.k * sm_scale * log2(e); probabilities use exp2, P is rounded
// to fp16 for the PV product (as flash-attn does), O and the row sum stay
// fp32, and out = fp16(O / sum).  The scale c = |sm_scale| log2(e) is applied
// inside the exponent, p = exp2(fma(s, c, -m)), with the row max taken over
// the raw s (the sign of sm_scale goes into Q once: -q for a negative scale,
// 0 for a zero one).  The running max m is moved only when a tile's max
// exceeds it by more than 8 (log2 units): P then stays below 2^8, which fp16
// holds at full relative precision, and out = O / sum is the same quotient,
// while the 64-register rescale of O runs on few tiles instead of most.
#include "common.h"

namespace {

constexpr int HD = 128;          // head dim
constexpr int KT = 64;           // keys per tile
constexpr int KS = HD + 8;       // Ks row stride (halves)
// Row-major V row stride (halves): 288 bytes, so the 4 rows x 32 bytes that
// each 16 lanes of a transposing read touch lie on distinct banks (a
// 272-byte stride measured 2-4% slower at T = 2048-8192)
constexpr int VR = HD + 16;
typedef short v4s __attribute__((vector_size(8)));
constexpr float kRescale = 8.f;  // move the running max when it grows by more (log2 units)

struct AttnArgs {
    const f16 *q, *k, *v;
    const int32_t *mask;         // [B, T] or null
    f16 *out;                    // [B, T, Hq, HD]
    int64_t q_tok, q_seq;        // strides (elements) of q: token, sequence
    int64_t kv_tok, kv_seq;      // strides of k and v
    int T, Hq, group;            // group = Hq / Hkv
    float c;                     // |sm_scale| * log2(e), or 1 for a zero scale
    float qmul;                  // sign of sm_scale (1, -1 or 0), applied to q
    int causal;
};

SRQ_DEV v16f mfma32(v8h a, v8h b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// K/V tiles are double-buffered in LDS: the next tile's global loads are
// issued into registers before this tile's MFMAs and written to the other
// buffer after them, so one barrier per tile covers both "tile t + 1 is in
// LDS" and "every wave is done with the buffer tile t + 2 will overwrite",
// and the load latency hides behind the compute.
template <int NWV, int GH>
__global__ void __launch_bounds__(NWV * 64, 8 / NWV) prefill_attn_kernel(AttnArgs a) {
    constexpr int NT = NWV * 64;              // threads
    constexpr int QB = 32 * NWV / GH;         // query rows per block
    static_assert(NWV % GH == 0 && (NT == 256 || NT == 512), "block shape");
    __shared__ __align__(16) f16 Ks_[2][KT * KS];
    __shared__ __align__(16) f16 Vs_[2][KT * VR];
    __shared__ float kbias_[2][KT];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, ln = lane & 31;
    const int rgrp = wave / GH;               // this wave's 32-row group
    // dispatch order: the linear block id runs over the head groups fastest,
    // so under a causal mask the heaviest q tiles of every head group go
    // first and the light ones fill in behind them (with the q tile fastest,
    // the first wave of blocks mixed heavy and light tiles of half the head
    // groups: Llama-70B heads, T = 2048 / 8192: 139 -> 97 / 1299 -> 1225 us)
    // (the host keeps gridDim.x * gridDim.y below 2^31)
    const uint32_t lin = blockIdx.x + gridDim.x * blockIdx.y;
    const int qt_lin = (int)(lin / gridDim.y), hg = (int)(lin % gridDim.y);
    const int qtile = a.causal ? (int)gridDim.x - 1 - qt_lin : qt_lin;
    const int hq = hg * GH + wave % GH, b = blockIdx.z;
    const int hk = hq / a.group;
    const int q0 = qtile * QB;
    const int qrow = q0 + rgrp * 32 + ln;          // this lane's query row
    const int wave_last = q0 + rgrp * 32 + 31;     // last row of this wave

    const f16 *qb = a.q + (int64_t)b * a.q_seq + (int64_t)hq * HD;
    const f16 *kb = a.k + (int64_t)b * a.kv_seq + (int64_t)hk * HD;
    const f16 *vb = a.v + (int64_t)b * a.kv_seq + (int64_t)hk * HD;
    const int32_t *mb = a.mask ? a.mask + (int64_t)b * a.T : nullptr;

    // Q^T as B operand: k-slot j of step kk <-> d = 16 kk + 8 g + j
    v8h qf[HD / 16];
    {
        const bool ok = qrow < a.T && (!mb || mb[qrow] != 0);
        const f16 *qr = qb + (int64_t)(ok ? qrow : 0) * a.q_tok + 8 * g;
        const f16 qm = (f16)a.qmul;
#pragma unroll
        for (int kk = 0; kk < HD / 16; ++kk) {
            v8h t = *reinterpret_cast<const v8h *>(qr + 16 * kk);
            qf[kk] = ok ? t * qm : (v8h)(f16)0;
        }
    }

    v16f o[HD / 32];
#pragma unroll
    for (int i = 0; i < HD / 32; ++i) o[i] = (v16f)0.f;
    float m = -INFINITY, l = 0.f;

    const int kv_end = a.causal ? min(a.T, q0 + QB) : a.T;
    const int ntiles = (kv_end + KT - 1) / KT;

    // staging registers of one tile, NT threads: row tid / KR of K and of V,
    // KH halves from (tid % KR) * KH; key bias tid (< KT) (raw loads; the
    // masking selects run at store time, after the MFMAs, so that no use of a
    // loaded value forces its wait before them)
    constexpr int KR = NT / KT, KH = HD / KR;
    v8h kx[KH / 8], vx[KH / 8];
    bool ok = false;
    float kbv = 0.f;
    auto load_tile = [&](int t) __attribute__((always_inline)) {
        const int r = tid / KR, d0 = (tid % KR) * KH;
        const int key = t * KT + r;
        ok = key < a.T && (!mb || mb[key] != 0);
        const int64_t off = (int64_t)(ok ? key : 0) * a.kv_tok + d0;
#pragma unroll
        for (int i = 0; i < KH / 8; ++i) {
            kx[i] = *reinterpret_cast<const v8h *>(kb + off + 8 * i);
            vx[i] = *reinterpret_cast<const v8h *>(vb + off + 8 * i);
        }
        if (tid < KT) {
            const int kz = t * KT + tid;
            const bool live = kz < a.T && (!mb || mb[kz] != 0);
            kbv = live ? 0.f : -INFINITY;
        }
    };
    // K and V row-major
    auto store_tile = [&](int buf, int t) __attribute__((always_inline)) {
        // a tile with every key live (no mask, inside the sequence; uniform
        // over the block) needs no selects (T = 8192: 1376 -> 1347 us)
        if ((mb || (t + 1) * KT > a.T) && !ok) {
#pragma unroll
            for (int i = 0; i < KH / 8; ++i) kx[i] = vx[i] = (v8h)(f16)0;
        }
        const int r = tid / KR, d0 = (tid % KR) * KH;
#pragma unroll
        for (int i = 0; i < KH / 8; ++i) {
            *reinterpret_cast<v8h *>(&Ks_[buf][r * KS + d0 + 8 * i]) = kx[i];
            *reinterpret_cast<v8h *>(&Vs_[buf][r * VR + d0 + 8 * i]) = vx[i];
        }
        if (tid < KT) kbias_[buf][tid] = kbv;
    };

    if (ntiles > 0) {
        load_tile(0);
        store_tile(0, 0);
    }
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const int k0 = t * KT;
        const int buf = t & 1;
        const f16 *Ks = Ks_[buf];
        const f16 *Vs = Vs_[buf];
        const float *kbias = kbias_[buf];
        if (t + 1 < ntiles) load_tile(t + 1);  // in flight during this tile's MFMAs
        // this tile's compute (returns early when no key is visible)
        [&]() __attribute__((always_inline)) {
            if (a.causal && k0 > wave_last) return;   // no key of this tile is visible

            // S^T, two 32-key blocks
            v16f s[2];
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                s[sb] = (v16f)0.f;
                const f16 *kr = &Ks[(32 * sb + ln) * KS + 8 * g];
#pragma unroll
                for (int kk = 0; kk < HD / 16; ++kk)
                    s[sb] = mfma32(*reinterpret_cast<const v8h *>(kr + 16 * kk), qf[kk], s[sb]);
            }
            // the K operand reads run 4 ahead of the MFMAs that take them
            // (Llama-70B heads, T = 8192: 1397 -> 1367 us)
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);   // 4 LDS reads
#pragma unroll
            for (int i = 0; i < 12; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // an MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // the next read
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            // mask and tile max of the raw logits.  A tile with every key live
            // and visible to every row of the wave (no mask, inside the
            // sequence, below the causal diagonal) skips the per-key tests:
            // the same values.
            float mt = -INFINITY;
            const bool full = !mb && k0 + KT <= a.T && (!a.causal || k0 + KT - 1 <= q0 + rgrp * 32);
            if (full) {
#pragma unroll
                for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                    for (int v = 0; v < 16; ++v) mt = fmaxf(mt, s[sb][v]);
            } else {
#pragma unroll
                for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int kr = 32 * sb + 8 * (v / 4) + 4 * g + (v % 4);
                        const bool vis = kbias[kr] == 0.f && !(a.causal && k0 + kr > qrow);
                        const float x = vis ? s[sb][v] : -INFINITY;
                        s[sb][v] = x;
                        mt = fmaxf(mt, x);
                    }
            }
            mt = fmaxf(mt, __shfl_xor(mt, 32));
            const float mtc = mt * a.c;   // c > 0: the max of the scaled logits
            const bool grow = mtc > m + kRescale;
            if (__builtin_amdgcn_ballot_w64(grow)) {
                const float alpha = grow ? __builtin_amdgcn_exp2f(m - mtc) : 1.f;
                m = grow ? mtc : m;
                l *= alpha;
#pragma unroll
                for (int i = 0; i < HD / 32; ++i) o[i] *= alpha;
            }
            const float nmu = m == -INFINITY ? 0.f : -m;
            float ps0 = 0.f, ps1 = 0.f;
            v8h pb[4];
#pragma unroll
            for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const float p = __builtin_amdgcn_exp2f(fmaf(s[sb][v], a.c, nmu));
                    if (v & 1) ps1 += p; else ps0 += p;
                    pb[2 * sb + v / 8][v % 8] = (f16)p;
                }
            l += ps0 + ps1;
            // O^T += V^T P^T; PV step st covers keys 16 st .. 16 st + 15 of the tile
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int db = 0; db < HD / 32; ++db) {
                    // lane (16-lane group q, j = lane % 16) reads row 4 g + j / 4 (+ 8),
                    // columns 16 (q & 1) + 4 (j % 4) of the block; the transposing read
                    // hands lane l keys 4 g + 0..3 (+ 8) of column l % 32
                    const f16 *vr = &Vs[(16 * st + 4 * g + ((lane & 15) >> 2)) * VR + 32 * db +
                                        16 * ((lane >> 4) & 1) + 4 * (lane & 3)];
                    v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s *)vr);
                    v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (__attribute__((address_space(3))) v4s *)(vr + 8 * VR));
                    v4h l4 = __builtin_bit_cast(v4h, lo), h4 = __builtin_bit_cast(v4h, hi);
                    v8h av = {l4[0], l4[1], l4[2], l4[3], h4[0], h4[1], h4[2], h4[3]};
                    o[db] = mfma32(av, pb[st], o[db]);
                }
        }();
        if (t + 1 < ntiles) store_tile(buf ^ 1, t + 1);
        __syncthreads();
    }

    if (qrow >= a.T) return;
    l += __shfl_xor(l, 32);
    const bool live = (!mb || mb[qrow] != 0) && l > 0.f;
    const float inv = live ? 1.f / l : 0.f;
    f16 *orow = a.out + ((int64_t)b * a.T + qrow) * ((int64_t)a.Hq * HD) + (int64_t)hq * HD;
#pragma unroll
    for (int db = 0; db < HD / 32; ++db)
#pragma unroll
        for (int grp = 0; grp < 4; ++grp) {
            v4h r;
#pragma unroll
            for (int i = 0; i < 4; ++i) r[i] = (f16)(o[db][4 * grp + i] * inv);
            *reinterpret_cast<v4h *>(orow + 32 * db + 8 * grp + 4 * g) = r;
        }
}

}  // namespace

extern "C" int srq_prefill_attention(const void *q, const void *k, const void *v,
                                     const int32_t *attention_mask, int64_t batch,
                                     int64_t seq_len, int64_t n_q_heads, int64_t n_kv_heads,
                                     int64_t head_dim, int64_t q_tok_stride,
                                     int64_t q_seq_stride, int64_t kv_tok_stride,
                                     int64_t kv_seq_stride, float sm_scale, int causal,
                                     void *out, void *stream) {
    SRQ_CHECK_ARG(batch >= 0 && seq_len >= 0 && n_q_heads >= 0 && n_kv_heads > 0,
                  "prefill_attention: bad shape");
    SRQ_CHECK_ARG(head_dim == HD, "prefill_attention: head_dim=%lld, only 128 is supported",
                  (long long)head_dim);
    SRQ_CHECK_ARG(n_q_heads % n_kv_heads == 0,
                  "prefill_attention: n_q_heads=%lld is not a multiple of n_kv_heads=%lld",
                  (long long)n_q_heads, (long long)n_kv_heads);
    SRQ_CHECK_ARG(__builtin_isfinite(sm_scale), "prefill_attention: sm_scale is not finite");
    if (batch == 0 || seq_len == 0 || n_q_heads == 0) return SRQ_OK;
    SRQ_CHECK_ARG(q && k && v && out, "prefill_attention: null pointer");
    SRQ_CHECK_ARG(seq_len <= (1 << 30) && n_q_heads <= 65535 && batch <= 65535,
                  "prefill_attention: shape out of range");
    SRQ_CHECK_ARG(q_tok_stride >= n_q_heads * HD && kv_tok_stride >= n_kv_heads * HD &&
                      q_seq_stride >= seq_len * q_tok_stride &&
                      kv_seq_stride >= seq_len * kv_tok_stride,
                  "prefill_attention: strides smaller than the [B, T, H, 128] extent");
    SRQ_CHECK_ARG(q_tok_stride % 8 == 0 && kv_tok_stride % 8 == 0 && q_seq_stride % 8 == 0 &&
                      kv_seq_stride % 8 == 0,
                  "prefill_attention: strides must be multiples of 8 elements");
    SRQ_CHECK_ARG(srq_aligned(q, 16) && srq_aligned(k, 16) && srq_aligned(v, 16) &&
                      srq_aligned(out, 16),
                  "prefill_attention: q, k, v and out must be 16-byte aligned");
    AttnArgs a;
    a.q = (const f16 *)q;
    a.k = (const f16 *)k;
    a.v = (const f16 *)v;
    a.mask = attention_mask;
    a.out = (f16 *)out;
    a.q_tok = q_tok_stride;
    a.q_seq = q_seq_stride;
    a.kv_tok = kv_tok_stride;
    a.kv_seq = kv_seq_stride;
    a.T = (int)seq_len;
    a.Hq = (int)n_q_heads;
    a.group = (int)(n_q_heads / n_kv_heads);
    a.c = (sm_scale == 0.f ? 1.f : fabsf(sm_scale)) * 1.4426950408889634f;
    a.qmul = sm_scale > 0.f ? 1.f : sm_scale < 0.f ? -1.f : 0.f;
    a.causal = causal ? 1 : 0;
    // GQA groups of 2, 4 or 8 q heads share each staged K/V tile in 8-wave
    // blocks (32 8 / G query rows of the G heads) when that still gives a
    // block per CU (MI355X: 256); otherwise 4-wave blocks of 128 rows of one
    // head (Llama-70B heads, T = 8192: 2012 -> 1528 us; T = 512 stays on
    // the 4-wave form: 25 against 31 us)
    hipStream_t st = (hipStream_t)stream;
    bool fits = true;
    auto go = [&](auto kern, int nwv, int gh) {
        const int qb = 32 * nwv / gh;
        // the kernel's linear block id over (q tile, head group) is 32-bit
        if (srq_cdiv(seq_len, qb) * (n_q_heads / gh) >= (int64_t)1 << 31) {
            fits = false;
            return;
        }
        dim3 grid((unsigned)srq_cdiv(seq_len, qb), (unsigned)(n_q_heads / gh), (unsigned)batch);
        kern<<<grid, nwv * 64, 0, st>>>(a);
    };
    constexpr int64_t kCUs = 256;
    const bool gqa = (a.group == 2 || a.group == 4 || a.group == 8) &&
                     srq_cdiv(seq_len, 256 / a.group) * (n_q_heads / a.group) * batch >= kCUs;
    switch (gqa ? a.group : 1) {
    case 2: go(prefill_attn_kernel<8, 2>, 8, 2); break;
    case 4: go(prefill_attn_kernel<8, 4>, 8, 4); break;
    case 8: go(prefill_attn_kernel<8, 8>, 8, 8); break;
    default: go(prefill_attn_kernel<4, 1>, 4, 1); break;
    }
    SRQ_CHECK_ARG(fits, "prefill_attention: seq_len x n_q_heads too large (q tiles x heads >= 2^31)");
    SRQ_LAUNCH_CHECK("prefill_attention");
    return SRQ_OK;
}
