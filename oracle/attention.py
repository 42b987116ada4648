"""Oracle for the paged int4 KV cache and single-query decode attention --
test infrastructure only.

Restates:
  * the page layout of paged_kv_t (signrot/kernels/include/flashinfer/
    page.cuh:18-112): data [pages, L, 2, H, page, D/2] u8, param
    [pages, L, 2, H, page, 2] f16, request b's pages
    indices[indptr[b]:indptr[b+1]], length (#pages - 1) * page + last[b];
  * AppendPagedKVCacheDecodeKernel / ...PrefillKernel (page.cuh:119-219);
  * BatchDecodeWithPagedKVCacheKernel + MergeChunkStatesKernel
    (decode.cuh:493-751): k̂ = float(q) * scale - zero (fp32,
    quantization.cuh:59-84), logits q·k̂ / sqrt(D), softmax, Σ p v̂ / Σ p.
  * The page table of MultiLayerPagedKVCache4Bit (signrot/transformers/
    kv_cache.py:417-433): physical page of (request b, page j) = j * B + b.
Numbers: the dequantized values are fp32 as in the kernel; the softmax and
the weighted sum are float64 (the kernel's exp2/fp32 order is not a fixed
bit pattern), so the kernel is compared with a tolerance.
"""
import math

import numpy as np

F16 = np.float16
F32 = np.float32


def page_table(batch, length, page_size):
    """(indptr, indices, last) of a uniform-length batch in the reference's
    layout (kv_cache.py:417-433 _set_page_cnt, 435-460 refresh_specs)."""
    pages = (length + page_size - 1) // page_size
    indptr = (np.arange(batch + 1) * pages).astype(np.int32)
    indices = (np.arange(pages)[None, :] * batch + np.arange(batch)[:, None]).reshape(-1)
    last = length % page_size
    if length != 0 and last == 0:
        last = page_size
    return indptr, indices.astype(np.int32), np.full(batch, last, np.int32)


def request_len(indptr, last, page_size, b):
    """page.cuh:76-103 / decode.cuh:512-513."""
    n = int(indptr[b + 1]) - int(indptr[b])
    return 0 if n == 0 else (n - 1) * page_size + int(last[b])


def slot(indptr, indices, page_size, b, t):
    """(physical page, entry) of token t of request b."""
    return int(indices[int(indptr[b]) + t // page_size]), t % page_size


def append(data, param, indptr, indices, last, layer, k, v, kp, vp, seqlen_indptr=None):
    """In-place restatement of the two append kernels (page.cuh:119-219).
    Decode form (seqlen_indptr None): k [B, H, D/2] at position len - 1.
    Prefill form: request b's rows seqlen_indptr[b]:seqlen_indptr[b+1] of
    k [T, H, D/2] at the last positions of request b."""
    page_size = data.shape[4]
    B = len(last)
    for b in range(B):
        L = request_len(indptr, last, page_size, b)
        if seqlen_indptr is None:
            src = [b]
        else:
            src = list(range(int(seqlen_indptr[b]), int(seqlen_indptr[b + 1])))
        start = L - len(src)
        for j, s in enumerate(src):
            pg, e = slot(indptr, indices, page_size, b, start + j)
            data[pg, layer, 0, :, e, :] = k[s]
            data[pg, layer, 1, :, e, :] = v[s]
            param[pg, layer, 0, :, e, :] = kp[s]
            param[pg, layer, 1, :, e, :] = vp[s]


def gather(data, param, indptr, indices, last, layer, b):
    """Dequantized K̂, V̂ [T, H, D] (fp32) of request b."""
    from .quant import kv_dequant
    page_size = data.shape[4]
    T = request_len(indptr, last, page_size, b)
    pages = np.asarray(indices[int(indptr[b]):int(indptr[b + 1])], np.int64)
    H, D = data.shape[3], data.shape[5] * 2
    out = []
    for kv in (0, 1):
        codes = data[pages, layer, kv]                       # [np, H, page, D/2]
        prm = param[pages, layer, kv]                        # [np, H, page, 2]
        codes = codes.transpose(0, 2, 1, 3).reshape(-1, H, D // 2)[:T]
        prm = prm.transpose(0, 2, 1, 3).reshape(-1, H, 2)[:T]
        out.append(kv_dequant(codes, prm))
    return out[0], out[1]


def decode(q_f16, data, param, indptr, indices, last, layer):
    """o [B, Hq, D] (float64) of batch_decode_i4; query head h reads KV head
    h // (Hq / H) (the reference's cache stores KV heads repeated Hq / H
    times, kv_cache.py:346-353, which gives the same result).  An empty
    request gives zeros."""
    q = np.asarray(q_f16, F16).astype(np.float64)
    B, Hq, D = q.shape
    H = data.shape[3]
    g = Hq // H
    out = np.zeros((B, Hq, D))
    for b in range(B):
        k, v = gather(data, param, indptr, indices, last, layer, b)
        if k.shape[0] == 0:
            continue
        k = k.astype(np.float64)
        v = v.astype(np.float64)
        for h in range(Hq):
            logits = k[:, h // g, :] @ q[b, h] / math.sqrt(D)
            p = np.exp(logits - logits.max())
            out[b, h] = (p[:, None] * v[:, h // g, :]).sum(0) / p.sum()
    return out


def prefill(q, k, v, mask=None, causal=True, sm_scale=None):
    """Prefill attention (the flash-attn 2 call of e2e/quantized_llama/
    modeling_llama.py:81-90 through transformers==4.57.6
    _flash_attention_forward, a dependency absent from the reference tree).

    q [B, T, Hq, D], k/v [B, T, Hkv, D] (any float dtype, promoted to
    float64); q head h reads kv head h // (Hq // Hkv).  With mask [B, T]
    (the HF attention_mask), the call unpads the valid tokens of each
    sequence, runs varlen attention over them (causal = key position <=
    query position among the valid tokens, since q and k lengths agree), and
    pads the result back with zero rows; for one sequence that is: query i
    (mask 1) attends keys j with mask[j] = 1 and j <= i; query rows with
    mask 0 are zero.  Logits q.k * sm_scale (default 1/sqrt(D)).  Returns
    float64 [B, T, Hq, D]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    group = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    out = np.zeros((B, T, Hq, D))
    allowed = np.ones((T, T), bool)
    if causal:
        allowed = np.tril(allowed)
    for b in range(B):
        keep = np.ones(T, bool) if mask is None else np.asarray(mask[b]) != 0
        ok = allowed & keep[None, :]
        for h in range(Hq):
            s = q[b, :, h] @ k[b, :, h // group].T * scale
            s = np.where(ok, s, -np.inf)
            rows = keep & ok.any(axis=1)
            s = s[rows]
            p = np.exp(s - s.max(axis=1, keepdims=True))
            out[b, rows, h] = (p / p.sum(axis=1, keepdims=True)) @ v[b, :, h // group]
    return out
