// Routing and combine of the MoE block (signrot/nn/moe.py:168-185 routing,
// 226-230 combine), for gfx950.
//
// moe_route: per token, the fp32 softmax of its E fp16 router logits, the
// top-k experts by probability, the optional renormalization of the k
// probabilities, the weights cast to fp16; then the T * k (token, choice)
// rows ordered by expert, stable in the row index t * k + j.  Arithmetic
// follows torch's ops step by step:
//   * softmax (softmax_warp_forward for E <= 64): x in fp32, m = max x,
//     e_i = exp(x_i - m), the sum of the e_i over E padded with zeros to a
//     power of two P by the shuffle butterfly v_i + v_{i ^ o} for
//     o = P/2, ..., 1, then p_i = e_i / sum;
//   * top-k by value, ties to the lower expert; the k values in descending
//     order;
//   * renormalization: p_j / (p_0 + p_1 + ... ) summed in order;
//   * weights: fp16 round of the fp32 values.
// The sort is a counting sort in one block: thread i owns a contiguous run
// of tokens (so its rows t * k + j are contiguous and increasing), counts
// its rows per expert into an LDS histogram laid out [expert][thread], and
// one exclusive scan of that histogram gives every (expert, thread) its
// first output position -- the expert offsets are the column-0 entries.
// Each thread then places its rows in order: stable, no atomics on global
// memory, deterministic.
//
// moe_combine: out[t, :] = fp16(sum_j fp32(fp16(y[inv[t k + j], :] *
// w[t, j]))), j in order from 0: the fp16 product and the fp32 sum of
// torch's (y[inv].view(T, k, H) * w.unsqueeze(-1)).sum(dim=1).
#include "common.h"

namespace {

constexpr int kRouteMaxE = 64;
constexpr int kRouteMaxK = 8;
constexpr int kRouteHistInts = 16384;  // at most EP * THREADS: 64 KB of LDS

// EP: the expert count rounded up to 8, 16, 32 or 64 (register arrays of
// that size); EP * THREADS <= kRouteHistInts.
template <int EP, int THREADS>
__global__ __launch_bounds__(THREADS) void moe_route_kernel(
    const f16 *__restrict__ logits, int T, int E, int K, int norm, f16 *__restrict__ weights,
    int32_t *__restrict__ choice, int32_t *__restrict__ order, int32_t *__restrict__ inv,
    int32_t *__restrict__ eid, int32_t *__restrict__ tok, int32_t *__restrict__ counts,
    int32_t *__restrict__ offsets) {
    static_assert(EP * THREADS <= kRouteHistInts, "histogram size");
    constexpr int kWaves = THREADS / 64;
    __shared__ int s_hist[EP * THREADS];  // [expert][thread]
    __shared__ int s_wtot[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < EP * THREADS; i += THREADS) s_hist[i] = 0;
    __syncthreads();

    // ---- per token: softmax, top-k, weights; histogram of this thread's rows
    const int per = (T + THREADS - 1) / THREADS;
    const int t0 = min(T, tid * per), t1 = min(T, t0 + per);
    int P = 1;
    while (P < E) P <<= 1;
    for (int t = t0; t < t1; ++t) {
        float v[EP];
        float m = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < EP; ++i) {
            v[i] = i < E ? (float)logits[(int64_t)t * E + i] : -__builtin_inff();
            m = v[i] > m ? v[i] : m;
        }
        float s[EP];
#pragma unroll
        for (int i = 0; i < EP; ++i) {
            v[i] = i < E ? expf(v[i] - m) : 0.f;
            s[i] = v[i];
        }
        // butterfly over the P-padded row: after the level with offset o,
        // s[i] = s[i] + s[i ^ o]; lane 0's value is the sum every lane ends with
#pragma unroll
        for (int o = EP / 2; o > 0; o >>= 1) {
            if (o < P) {
#pragma unroll
                for (int i = 0; i < o; ++i) s[i] = s[i] + s[i + o];
            }
        }
        const float sum = s[0];
#pragma unroll
        for (int i = 0; i < EP; ++i) v[i] = v[i] / sum;  // the softmax output
        float pk[kRouteMaxK];
        int ek[kRouteMaxK];
        uint64_t taken = 0;
#pragma unroll
        for (int j = 0; j < kRouteMaxK; ++j) {
            if (j >= K) break;
            // NaN ranks above every number (torch.topk's order); a row with
            // a NaN or inf logit has all-NaN probabilities, so its k picks
            // are k distinct experts with NaN weights.  Strict comparisons:
            // ties, NaN ones included, keep the lower expert.
            float best = -1.f;
            bool best_nan = false;
            int bi = -1;
#pragma unroll
            for (int i = 0; i < EP; ++i) {
                const bool vn = v[i] != v[i];
                const bool above = vn ? !best_nan : (!best_nan && v[i] > best);
                const bool ok = i < E && !((taken >> i) & 1) && (bi < 0 || above);
                best = ok ? v[i] : best;
                best_nan = ok ? vn : best_nan;
                bi = ok ? i : bi;
            }
            taken |= 1ull << bi;
            pk[j] = best;
            ek[j] = bi;
        }
        float den = 0.f;
        if (norm) {
#pragma unroll
            for (int j = 0; j < kRouteMaxK; ++j)
                if (j < K) den += pk[j];
        }
#pragma unroll
        for (int j = 0; j < kRouteMaxK; ++j) {
            if (j >= K) break;
            const float w = norm ? pk[j] / den : pk[j];
            weights[(int64_t)t * K + j] = (f16)w;
            choice[(int64_t)t * K + j] = ek[j];
            ++s_hist[ek[j] * THREADS + tid];  // this thread's own column
        }
    }
    __syncthreads();

    // ---- exclusive scan of the histogram in [expert][thread] order: each
    // thread scans EP consecutive entries, then the per-thread totals are
    // scanned across the block
    int run = 0;
#pragma unroll
    for (int i = 0; i < EP; ++i) {
        const int c = s_hist[tid * EP + i];
        s_hist[tid * EP + i] = run;
        run += c;
    }
    int incl = run;  // inclusive scan of the thread totals within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(incl, o);
        if (lane >= o) incl += u;
    }
    if (lane == 63) s_wtot[wave] = incl;
    __syncthreads();
    int base = incl - run;
    for (int w = 0; w < wave; ++w) base += s_wtot[w];
#pragma unroll
    for (int i = 0; i < EP; ++i) s_hist[tid * EP + i] += base;
    __syncthreads();
    const int rows = T * K;
    if (tid < E) {
        const int o0 = s_hist[tid * THREADS];
        const int o1 = tid + 1 < E ? s_hist[(tid + 1) * THREADS] : rows;
        offsets[tid] = o0;
        counts[tid] = o1 - o0;
        if (tid == 0) offsets[E] = rows;
    }
    __syncthreads();

    // ---- place this thread's rows, in row order
    for (int f = t0 * K; f < t1 * K; ++f) {
        const int e = choice[f];  // written by this thread above
        const int pos = s_hist[e * THREADS + tid]++;
        order[pos] = f;
        inv[f] = pos;
        eid[pos] = e;
        tok[pos] = f / K;
    }
}

// One thread per 8 consecutive outputs of a token (16-byte loads/stores).
__global__ __launch_bounds__(256) void moe_combine_kernel(const f16 *__restrict__ y,
                                                          const int32_t *__restrict__ inv,
                                                          const f16 *__restrict__ w, int64_t T,
                                                          int K, int64_t H,
                                                          f16 *__restrict__ out) {
    const int64_t per_tok = H / 8;
    const int64_t total = T * per_tok;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * 256) {
        const int64_t t = i / per_tok, h = (i % per_tok) * 8;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int j = 0; j < K; ++j) {
            const int64_t r = inv[t * K + j];
            const float wj = (float)w[t * K + j];
            const v8h yv = *reinterpret_cast<const v8h *>(y + r * H + h);
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[k] += (float)f16_rn((float)yv[k] * wj);
        }
        v8h o;
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = f16_rn(acc[k]);
        *reinterpret_cast<v8h *>(out + t * H + h) = o;
    }
}

}  // namespace

extern "C" int srq_moe_route(const void *logits, int64_t tokens, int64_t num_experts,
                             int64_t top_k, int norm, void *weights, int32_t *choice,
                             int32_t *order, int32_t *inv, int32_t *expert, int32_t *token,
                             int32_t *counts, int32_t *offsets, void *stream) {
    SRQ_CHECK_ARG(num_experts >= 1 && num_experts <= kRouteMaxE,
                  "moe_route: num_experts=%lld must be in [1, %d]", (long long)num_experts,
                  kRouteMaxE);
    SRQ_CHECK_ARG(top_k >= 1 && top_k <= num_experts && top_k <= kRouteMaxK,
                  "moe_route: top_k=%lld must be in [1, min(num_experts, %d)]",
                  (long long)top_k, kRouteMaxK);
    SRQ_CHECK_ARG(tokens >= 0 && tokens * top_k < 0x7fffffffLL, "moe_route: bad token count");
    SRQ_CHECK_ARG(logits || tokens == 0, "moe_route: null logits");
    SRQ_CHECK_ARG(counts && offsets, "moe_route: null counts / offsets");
    SRQ_CHECK_ARG(tokens == 0 || (weights && choice && order && inv && expert && token),
                  "moe_route: null output");
    auto launch = [&](auto kern, int threads) {
        kern<<<dim3(1), dim3(threads), 0, (hipStream_t)stream>>>(
            (const f16 *)logits, (int)tokens, (int)num_experts, (int)top_k, norm,
            (f16 *)weights, choice, order, inv, expert, token, counts, offsets);
    };
    if (num_experts <= 8)
        launch(moe_route_kernel<8, 1024>, 1024);
    else if (num_experts <= 16)
        launch(moe_route_kernel<16, 1024>, 1024);
    else if (num_experts <= 32)
        launch(moe_route_kernel<32, 512>, 512);
    else
        launch(moe_route_kernel<64, 256>, 256);
    SRQ_LAUNCH_CHECK("moe_route");
    return SRQ_OK;
}

extern "C" int srq_moe_combine(const void *y, const int32_t *inv, const void *weights,
                               int64_t tokens, int64_t top_k, int64_t hidden, void *out,
                               void *stream) {
    SRQ_CHECK_ARG(tokens >= 0 && top_k >= 1 && hidden >= 0, "moe_combine: bad shape");
    SRQ_CHECK_ARG(hidden % 8 == 0, "moe_combine: hidden=%lld must be a multiple of 8",
                  (long long)hidden);
    if (tokens == 0 || hidden == 0) return SRQ_OK;
    SRQ_CHECK_ARG(y && inv && weights && out, "moe_combine: null pointer");
    SRQ_CHECK_ARG(srq_aligned(y, 16) && srq_aligned(out, 16),
                  "moe_combine: y and out must be 16-byte aligned");
    const int64_t blocks = std::min<int64_t>(srq_cdiv(tokens * (hidden / 8), 256), 4096);
    moe_combine_kernel<<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(
        (const f16 *)y, inv, (const f16 *)weights, tokens, (int)top_k, hidden, (f16 *)out);
    SRQ_LAUNCH_CHECK("moe_combine");
    return SRQ_OK;
}
