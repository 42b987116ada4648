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

// --------------------------------------------------------------- decode
constexpr int kTile = 32;
constexpr int kD = 128;

SRQ_DEV v16f mfma32h(v8h a, v8h b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// 8 uint4 codes (one dword, code 2j in the low nibble of byte j) -> 8 exact
// fp16 values in the order [0, 4, 1, 5, 2, 6, 3, 7]
SRQ_DEV v8h codes8(u32 w) {
    const u32 m = 0x000F000Fu, magic = 0x64006400u;
    const v2h off = (v2h){(f16)-1024, (f16)-1024};
    v2h p0 = __builtin_bit_cast(v2h, (w & m) | magic) + off;
    v2h p1 = __builtin_bit_cast(v2h, ((w >> 4) & m) | magic) + off;
    v2h p2 = __builtin_bit_cast(v2h, ((w >> 8) & m) | magic) + off;
    v2h p3 = __builtin_bit_cast(v2h, ((w >> 12) & m) | magic) + off;
    v8h r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

// dim order of codes8 slot e (within its 8-dim group)
SRQ_DEV int codes8_dim(int e) { return (e >> 1) + 4 * (e & 1); }

struct DecodeArgs {
    Paged p;
    const f16 *q;      // [B, Hq, D]
    f16 *o;            // [B, Hq, D]
    float *tmp;        // [B, Hq, chunks, D + 4] or null
    int64_t B, Hq, G;  // G = Hq / H (query heads per KV head), <= 8
    int chunks;
    float sm_scale_log2;
};

template <int GP>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
    // per-wave scratch: p * v_scale (fp16) [tile token][8 heads] and the
    // tile tokens' V code row offsets; cross-wave merge buffers
    __shared__ __attribute__((aligned(16))) f16 pv_s[4][kTile][8];
    __shared__ int64_t voff_s[4][kTile];
    __shared__ float m_s[4][8], d_s[4][8], z_s[4][8];
    __shared__ __attribute__((aligned(16))) float o_s[4][8][kD];

    const Paged &p = a.p;
    const int64_t b = blockIdx.x;
    const int64_t kvh = blockIdx.y;
    const int chunk = blockIdx.z;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int G = (int)a.G;

    const int64_t len = seq_len_of(p, b);
    const int64_t per = srq_cdiv(srq_cdiv(len, a.chunks), kTile) * kTile;
    const int64_t t0 = per * chunk;
    const int64_t t1 = (t0 + per < len) ? t0 + per : len;

    // ---- query operand: rows = heads (row m < G), k-slot (h2, e) of k-step
    // ks = dim 64 h2 + 8 ks + codes8_dim(e)
    const int m = lane & 31, h2 = lane >> 5;
    const int64_t qrow = (b * a.Hq + kvh * G + m) * kD;
    v8h qa[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            qa[ks][e] = m < G ? a.q[qrow + 64 * h2 + 8 * ks + codes8_dim(e)] : (f16)0;
    // sum of q per head, for the zero-point term (heads 4 h2 .. 4 h2 + 3)
    float qsum[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int h = 4 * h2 + r;
        float s = 0.f;
        if (h < G) {
            const f16 *qr = a.q + (b * a.Hq + kvh * G + h) * kD;
            for (int d = 0; d < kD; ++d) s += (float)qr[d];
        }
        qsum[r] = s;
    }

    // running state.  Token lanes (S layout): heads 4 h2 + r, r < 4.
    float m_run[4], d_part[4], z_part[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        m_run[r] = -INFINITY;
        d_part[r] = 0.f;
        z_part[r] = 0.f;
    }
    // PV layout: lane = (tq = lane >> 4, ds = lane & 15): 8 dims 8 ds .. 8 ds + 7
    const int tq = lane >> 4, ds = lane & 15;
    float acc[GP][8];
#pragma unroll
    for (int h = 0; h < GP; ++h)
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[h][d] = 0.f;

    const int64_t np0 = p.indptr[b];
    for (int64_t tb = t0 + (int64_t)wave * kTile; tb < t1; tb += 4 * kTile) {
        // ---------------- S phase: lane (token tl = lane & 31, half h2)
        const int tl = lane & 31;
        const int64_t t = tb + tl;
        const bool valid = t < t1;
        int64_t kro = 0, vro = 0;
        u32 kw[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float ksc = 0.f, kz = 0.f, vsc = 0.f, vz = 0.f;
        if (valid) {
            const int64_t page = p.indices[np0 + t / p.page];
            const int64_t entry = t % p.page;
            kro = row_index(p, page, 0, kvh, entry);
            vro = row_index(p, page, 1, kvh, entry);
            const v4i c0 = *reinterpret_cast<const v4i *>(p.data + kro * (kD / 2) + 32 * h2);
            const v4i c1 = *reinterpret_cast<const v4i *>(p.data + kro * (kD / 2) + 32 * h2 + 16);
            kw[0] = c0[0]; kw[1] = c0[1]; kw[2] = c0[2]; kw[3] = c0[3];
            kw[4] = c1[0]; kw[5] = c1[1]; kw[6] = c1[2]; kw[7] = c1[3];
            const v2h kp = *reinterpret_cast<const v2h *>(p.param + 2 * kro);
            const v2h vp = *reinterpret_cast<const v2h *>(p.param + 2 * vro);
            ksc = (float)kp[0];
            kz = (float)kp[1];
            vsc = (float)vp[0];
            vz = (float)vp[1];
        }
        if (h2 == 0) voff_s[wave][tl] = valid ? vro * (kD / 2) : -1;
        v16f sacc = {};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) sacc = mfma32h(qa[ks], codes8(kw[ks]), sacc);
        // lane (tl, h2) holds S[head 4 h2 + r][token tl] in sacc[r]
        float lg[4], tmax[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float dot = ksc * sacc[r] - kz * qsum[r];
            lg[r] = valid ? dot * a.sm_scale_log2 : -INFINITY;
            tmax[r] = lg[r];
        }
#pragma unroll
        for (int off = 1; off < 32; off <<= 1)
#pragma unroll
            for (int r = 0; r < 4; ++r) tmax[r] = fmaxf(tmax[r], __shfl_xor(tmax[r], off, 64));
        float alpha[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float mn = fmaxf(m_run[r], tmax[r]);
            // mn == -inf only when every token so far is masked
            alpha[r] = mn == -INFINITY ? 1.f : exp2f(m_run[r] - mn);
            const float pr = valid ? exp2f(lg[r] - mn) : 0.f;
            m_run[r] = mn;
            d_part[r] = d_part[r] * alpha[r] + pr;
            z_part[r] = z_part[r] * alpha[r] + pr * vz;
            pv_s[wave][tl][4 * h2 + r] = (f16)(pr * vsc);
        }
        // the PV lanes need alpha of all 8 heads: heads 0-3 from lane 0,
        // heads 4-7 from lane 32 (uniform within each half)
        float al[8];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            al[r] = __shfl(alpha[r], 0, 64);
            al[4 + r] = __shfl(alpha[r], 32, 64);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

        // ---------------- PV phase: lane (tq, ds), tokens 8 tq .. 8 tq + 7
#pragma unroll
        for (int h = 0; h < GP; ++h)
#pragma unroll
            for (int d = 0; d < 8; ++d) acc[h][d] *= al[h];
#pragma unroll
        for (int pr2 = 0; pr2 < 4; ++pr2) {
            const int ta = 8 * tq + 2 * pr2, tb2 = ta + 1;
            const int64_t oa = voff_s[wave][ta], ob = voff_s[wave][tb2];
            const u32 wa = oa >= 0 ? *reinterpret_cast<const u32 *>(p.data + oa + 4 * ds) : 0u;
            const u32 wb = ob >= 0 ? *reinterpret_cast<const u32 *>(p.data + ob + 4 * ds) : 0u;
            // (p_a v_scale_a, p_b v_scale_b) per head as an fp16 pair
            const v8h pa = *reinterpret_cast<const v8h *>(&pv_s[wave][ta][0]);
            const v8h pb = *reinterpret_cast<const v8h *>(&pv_s[wave][tb2][0]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // byte j of both tokens -> (c_a, c_b) for dims 2j (low) and 2j + 1 (high)
                const u32 pj = ((wa >> (8 * j)) & 0xFFu) | (((wb >> (8 * j)) & 0xFFu) << 16);
                const v2h lo = __builtin_bit_cast(v2h, (pj & 0x000F000Fu) | 0x64006400u) +
                               (v2h){(f16)-1024, (f16)-1024};
                const v2h hi = __builtin_bit_cast(v2h, ((pj >> 4) & 0x000F000Fu) | 0x64006400u) +
                               (v2h){(f16)-1024, (f16)-1024};
#pragma unroll
                for (int h = 0; h < GP; ++h) {
                    const v2h ph = (v2h){pa[h], pb[h]};
                    acc[h][2 * j] = __builtin_amdgcn_fdot2(ph, lo, acc[h][2 * j], false);
                    acc[h][2 * j + 1] = __builtin_amdgcn_fdot2(ph, hi, acc[h][2 * j + 1], false);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }

    // ---- reduce within the wave
    // d, z: sum over the 32 token lanes of each half
#pragma unroll
    for (int off = 1; off < 32; off <<= 1)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            d_part[r] += __shfl_xor(d_part[r], off, 64);
            z_part[r] += __shfl_xor(z_part[r], off, 64);
        }
    // o: sum over the 4 token quarters (lanes with equal ds)
#pragma unroll
    for (int h = 0; h < GP; ++h)
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            float v = acc[h][d];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            acc[h][d] = v;
        }
    if (lane == 0 || lane == 32) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            m_s[wave][4 * h2 + r] = m_run[r];
            d_s[wave][4 * h2 + r] = d_part[r];
            z_s[wave][4 * h2 + r] = z_part[r];
        }
    }
    if (tq == 0) {
#pragma unroll
        for (int h = 0; h < GP; ++h)
#pragma unroll
            for (int d = 0; d < 8; ++d) o_s[wave][h][8 * ds + d] = acc[h][d];
    }
    __syncthreads();

    // ---- merge the four waves: thread (h, d) for h < G, d < 128
    for (int idx = threadIdx.x; idx < G * kD; idx += 256) {
        const int h = idx / kD, d = idx - h * kD;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) mx = fmaxf(mx, m_s[w][h]);
        float ov = 0.f, dv = 0.f, zv = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
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

// merge the per-chunk (o, m, d) records of one (request, query head)
__global__ __launch_bounds__(128) void merge_kernel(const float *__restrict__ tmp, f16 *__restrict__ o,
                                                    int64_t Hq, int chunks) {
    const int64_t bh = blockIdx.x;
    const int d = threadIdx.x;
    const float *rec = tmp + bh * chunks * (kD + 4);
    float mx = -INFINITY;
    for (int c = 0; c < chunks; ++c) mx = fmaxf(mx, rec[c * (kD + 4) + kD]);
    float ov = 0.f, dv = 0.f;
    for (int c = 0; c < chunks; ++c) {
        const float mc = rec[c * (kD + 4) + kD];
        const float sc = mc == -INFINITY ? 0.f : exp2f(mc - mx);
        ov += rec[c * (kD + 4) + d] * sc;
        dv += rec[c * (kD + 4) + kD + 1] * sc;
    }
    o[bh * kD + d] = (f16)(dv > 0.f ? ov / dv : 0.f);
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
    SRQ_CHECK_ARG(o && q, "batch_decode_i4: null q/o");
    if (num_chunks < 1 || tmp == nullptr) num_chunks = 1;
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
    if (a.G == 1)
        decode_kernel<1><<<grid, 256, 0, st>>>(a);
    else if (a.G == 2)
        decode_kernel<2><<<grid, 256, 0, st>>>(a);
    else if (a.G <= 4)
        decode_kernel<4><<<grid, 256, 0, st>>>(a);
    else
        decode_kernel<8><<<grid, 256, 0, st>>>(a);
    SRQ_LAUNCH_CHECK("batch_decode_i4");
    if (num_chunks > 1) {
        merge_kernel<<<dim3((unsigned)(batch * num_qo_heads)), 128, 0, st>>>(tmp, (f16 *)o,
                                                                          num_qo_heads,
                                                                          (int)num_chunks);
        SRQ_LAUNCH_CHECK("batch_decode_i4 (merge)");
    }
    return SRQ_OK;
}
