"""Paged int4 KV cache and decode attention, with the interface of the
reference's signrot/transformers/kv_cache.py (MultiLayerPagedKVCache4Bit,
update() returning the decode attention of the layer, the spec dict of the
flashinfer-style ops, refresh/freeze of the specs for graph capture).

Design:
  * `pages` u8 [P, L, 2, H, page, D/2] and `scales` f16 [P, L, 2, H, page, 2]
    are the reference's tensors (same names, shapes and content), so code
    that reads or writes them directly keeps working.
  * `_PageTable` owns the three index tensors the HIP ops read (indptr,
    indices, last-page length).  They are allocated once and rewritten in
    place, so a captured HIP graph keeps valid addresses; the physical page
    of (request b, page j) is j * B + b, the reference's assignment
    (kv_cache.py:417-433), which lets the pool grow by appending.
  * `_SplitDecoder` holds the split-KV workspace and the chunk count, and
    `update()` returns a `_LayerAttention` callable bound to one layer.
  * KV heads are stored once.  The reference repeats each KV head
    `group_size` times (kv_cache.py:346-353) because its decode kernel needs
    as many KV heads as query heads; batch_decode_i4 here maps query head h
    to KV head h // group_size itself, so the cache and the decode traffic
    are group_size times smaller.  Results are the same.
  * Only the int4 cache exists: disable_quant=True (fp16 cache) and lac=True
    (learned clipping, unused by the reference itself) raise
    NotImplementedError.
"""
import math
from typing import Any, Dict, Optional

import torch
from transformers.cache_utils import Cache

from .. import _CUDA
from ..functional import kernel as signrot_kernel


def _init_hf_cache(cache):
    """Cache's own initializer: transformers 4.x takes no arguments, 5.x
    wants a (here empty) list of cache layers."""
    try:
        Cache.__init__(cache, layers=[])
    except TypeError:
        Cache.__init__(cache)


def asym_quantize_and_pack_i4(x, clip_factor_a_max=1.0, clip_factor_a_min=1.0, lac=False,
                              quantize=True):
    """The reference's torch KV quantizer (kv_cache.py:12-58), in x's dtype
    (fp16: every op rounds once, as the fused kv_quant_pack kernel does).

    Default (lac=False): per row over the last dim, scale =
    clamp(max - min, 1e-5) / 15, zero = -min, codes clamp(round((x + zero) /
    scale), 0, 15).  lac=True (learned activation clipping): the range is
    widened to include 0 and multiplied by the clip factors, an all-zero
    range becomes [-1, 1], scale = (max - min) / 15, zero = round(-min /
    scale), codes clamp(round(x / scale) + zero, 0, 15).

    quantize=True returns (u8 codes [..., D/2], element 2j in the low
    nibble of byte j; scale [..., 1]; zero [..., 1]).  quantize=False
    returns (scale * (codes - zero), scale, zero) unpacked -- for the
    default branch that is the reference's expression as written, not the
    cache's dequantization codes * scale - zero."""
    maxq = 15
    hi = torch.amax(x, dim=-1, keepdim=True)
    lo = torch.amin(x, dim=-1, keepdim=True)
    if lac:
        hi = torch.clamp(hi, min=0) * clip_factor_a_max
        lo = torch.clamp(lo, max=0) * clip_factor_a_min
        flat = (lo == 0) & (hi == 0)
        lo = torch.where(flat, torch.full_like(lo, -1.0), lo)
        hi = torch.where(flat, torch.full_like(hi, 1.0), hi)
        scale = (hi - lo) / maxq
        zero = torch.round(-lo / scale)
        codes = torch.clamp(torch.round(x / scale) + zero, 0, maxq)
    else:
        scale = torch.clamp(hi - lo, min=1e-5) / maxq
        zero = -lo
        codes = torch.clamp(torch.round((x + zero) / scale), 0, maxq)
    if not quantize:
        return scale * (codes - zero), scale, zero
    u = codes.to(torch.uint8)
    return u[..., 0::2] | (u[..., 1::2] << 4), scale, zero


def unpack_i4_and_asym_dequantize(q, scale, zero, lac: bool = False):
    """uint4 codes (low nibble first) -> q * scale - zero, or
    scale * (q - zero) with lac (kv_cache.py:60-68)."""
    assert q.dtype == torch.uint8
    codes = torch.stack((q & 0x0F, q >> 4), dim=-1).flatten(-2)
    return scale * (codes - zero) if lac else codes * scale - zero


def matmul_had_cuda(X, dtype):
    """Head-dim Walsh-Hadamard transform, scaled by 1/sqrt(n), computed in
    `dtype` and returned in X's dtype (kv_cache.py:70-73)."""
    n = X.shape[-1]
    out = _CUDA.hadamard_transform(X.to(dtype).contiguous(), scale=1 / math.sqrt(n))
    return out.to(X.dtype).view(X.shape)


def init_kv_i4(kv_data, kv_param, kv_indptr, kv_indices, last_page_offset, k, v, k_param,
               v_param, seqlen_indptr, layer_idx):
    return _CUDA.init_kv_i4(kv_data, kv_param, kv_indptr, kv_indices, last_page_offset, k, v,
                            k_param, v_param, seqlen_indptr, layer_idx)


def append_kv_i4(kv_data, kv_param, kv_indptr, kv_indices, last_page_offset, k, v, k_param,
                 v_param, layer_idx):
    return _CUDA.append_kv_i4(kv_data, kv_param, kv_indptr, kv_indices, last_page_offset, k, v,
                              k_param, v_param, layer_idx)


def batch_decode_i4(o, q, kv_data, kv_param, kv_indptr, kv_indices, last_page_offset,
                    layer_idx, tmp=None, num_chunks=1):
    return _CUDA.batch_decode_i4(o, q, kv_data, kv_param, kv_indptr, kv_indices,
                                 last_page_offset, layer_idx, tmp, num_chunks)


def _pages_for(length, page_size):
    return -(-length // page_size)


def _last_page_len(length: int, page_size: int) -> int:
    """Tokens held by the last page of a request of `length` tokens (0 for
    an empty request, a full page when length is a multiple of it)."""
    if length == 0:
        return 0
    return (length - 1) % page_size + 1


class _PageTable:
    """Request -> physical page map of a batch whose requests all hold the
    same number of pages, in three persistent int32 tensors:
      indptr [B + 1]   request b's pages are indices[indptr[b] : indptr[b+1]]
      indices [capacity] physical page of (b, j) = j * B + b
      last [B]         tokens in each request's last page."""

    def __init__(self, batch, capacity, device):
        self.batch = batch
        self.device = device
        self._row = torch.arange(batch + 1, device=device, dtype=torch.int32)
        self.indptr = torch.empty(batch + 1, device=device, dtype=torch.int32)
        self.last = torch.empty(batch, device=device, dtype=torch.int32)
        self.indices = torch.empty(capacity, device=device, dtype=torch.int32)
        self._written_for = -1

    def grow(self, capacity):
        """A larger indices tensor (the pool grew); the caller re-points the
        spec dict at it."""
        self.indices = torch.empty(capacity, device=self.device, dtype=torch.int32)
        self._written_for = -1

    def set_pages(self, per_request: int):
        torch.mul(self._row, per_request, out=self.indptr)
        if per_request != self._written_for:
            j = torch.arange(per_request, device=self.device, dtype=torch.int32)
            b = torch.arange(self.batch, device=self.device, dtype=torch.int32)
            self.indices[: per_request * self.batch].copy_((j * self.batch + b[:, None]).flatten())
            self._written_for = per_request

    def set_uniform(self, length: int, page_size: int):
        self.last.fill_(_last_page_len(length, page_size))
        self.set_pages(_pages_for(length, page_size))

    def set_from_mask(self, attention_mask, page_size: int):
        """Per-request lengths from an HF attention_mask [B, T]; every request
        must need the same number of pages (the shared page count is read on
        the host)."""
        lens = attention_mask.sum(dim=-1, dtype=torch.int32)
        pages = (lens + page_size - 1) // page_size
        lo, hi = int(pages.min()), int(pages.max())
        if lo != hi:
            raise NotImplementedError("Current implementation does not support the case where "
                                      "batches have different number of pages")
        self.last.copy_(torch.where(lens > 0, (lens - 1) % page_size + 1, 0))
        self.set_pages(lo)

    def clone(self):
        t = _PageTable.__new__(_PageTable)
        t.batch, t.device, t._row = self.batch, self.device, self._row
        t.indptr, t.last, t.indices = self.indptr.clone(), self.last.clone(), self.indices.clone()
        t._written_for = self._written_for
        return t


class _SplitDecoder:
    """batch_decode_i4 with a fixed split-KV configuration: `num_chunks`
    chunks per (request, KV head) and their fp32 workspace `tmp`
    [B, Hq, chunks, D + 4] (no workspace for one chunk)."""

    def __init__(self, batch, num_qo_heads, head_dim, chunks, device, hadamard_dtype):
        self.num_chunks = chunks
        self.hadamard_dtype = hadamard_dtype
        self.tmp = (torch.empty((batch, num_qo_heads, chunks, head_dim + 4), dtype=torch.float32,
                                device=device) if chunks > 1 else None)

    def attend(self, q_rot, spec, layer_idx):
        """o [B, Hq, D] for an already rotated q [B, Hq, D]."""
        o = torch.empty_like(q_rot)
        split = self.tmp is not None and self.tmp.shape[1] == q_rot.shape[1]
        batch_decode_i4(o, q_rot, **spec, layer_idx=layer_idx,
                        tmp=self.tmp if split else None,
                        num_chunks=self.num_chunks if split else 1)
        return o

    def attend_head_had_quant(self, q_rot, spec, layer_idx, scale):
        """head_had_quant(attend(q_rot), scale): the o_proj input codes and
        scales.  Split: the partial states are merged inside the head-axis
        kernel (one launch fewer, the same bits)."""
        Hq = q_rot.shape[1]
        if (self.tmp is not None and self.tmp.shape[1] == Hq
                and Hq * self.num_chunks <= _CUDA.MERGE_HHQ_MAX_RECORDS):
            batch_decode_i4(None, q_rot, **spec, layer_idx=layer_idx, tmp=self.tmp,
                            num_chunks=self.num_chunks)
            return _CUDA.merge_head_had_quant(self.tmp, scale)
        return _CUDA.head_had_quant(self.attend(q_rot, spec, layer_idx), scale)


    def qkv_attend(self, qkv, cos, sin, spec, layer_idx, n_q_heads, had_scale, rotate):
        """qkv_decode_i4 with this split: the attention output o [B, Hq, D]
        of the new token (its k / v quantized into the cache on the way)."""
        B, D = qkv.shape[0], 128
        o = torch.empty((B, n_q_heads, D), dtype=torch.float16, device=qkv.device)
        split = self.tmp is not None and self.tmp.shape[1] == n_q_heads
        _CUDA.qkv_decode_i4(o, qkv, cos, sin, **spec, layer_idx=layer_idx, n_q_heads=n_q_heads,
                            had_scale=had_scale, rotate=rotate,
                            tmp=self.tmp if split else None,
                            num_chunks=self.num_chunks if split else 1)
        return o

    def qkv_attend_head_had_quant(self, qkv, cos, sin, spec, layer_idx, n_q_heads, had_scale,
                                  rotate, scale):
        """head_had_quant(qkv_attend(...), scale), the split merged inside the
        head-axis kernel where the records fit (as attend_head_had_quant)."""
        if (self.tmp is not None and self.tmp.shape[1] == n_q_heads
                and n_q_heads * self.num_chunks <= _CUDA.MERGE_HHQ_MAX_RECORDS):
            _CUDA.qkv_decode_i4(None, qkv, cos, sin, **spec, layer_idx=layer_idx,
                                n_q_heads=n_q_heads, had_scale=had_scale, rotate=rotate,
                                tmp=self.tmp, num_chunks=self.num_chunks)
            return _CUDA.merge_head_had_quant(self.tmp, scale)
        return _CUDA.head_had_quant(
            self.qkv_attend(qkv, cos, sin, spec, layer_idx, n_q_heads, had_scale, rotate), scale)


class _LayerAttention:
    """What update() returns after an append: q [B, 1, Hq, D] -> attention
    over this layer's cache, [B, 1, Hq, D] (the reference's
    _AttentionStub.forward bound to one layer, kv_cache.py:144-170).  q is
    rotated by the head-dim Hadamard first, matching the rotated keys."""

    def __init__(self, decoder: _SplitDecoder, spec, layer_idx):
        self.decoder, self.spec, self.layer_idx = decoder, spec, layer_idx

    def __call__(self, q):
        B, T, Hq, D = q.shape
        if T != 1:
            raise ValueError("decode attention takes one query token per request")
        q = q.view(B, Hq, D)
        if self.decoder.hadamard_dtype is not None:
            q = matmul_had_cuda(q, dtype=self.decoder.hadamard_dtype)
        return self.decoder.attend(q, self.spec, self.layer_idx).unsqueeze(1)


class MultiLayerPagedKVCache4Bit(Cache):
    """Paged int4 KV cache for all layers of a model (the reference's
    MultiLayerPagedKVCache4Bit, kv_cache.py:173-498).

    pages  u8  [pages, n_layers, 2, num_heads, page_size, head_dim / 2]
    scales f16 [pages, n_layers, 2, num_heads, page_size, 2]  ([scale, zero])
    `num_heads` is the number of KV heads; `group_size` the number of query
    heads per KV head."""

    # transformers' Cache exposes batch_size as a read-only property of its
    # layer list; this cache keeps its own (a plain class attribute ahead of
    # the property in the lookup lets __init__ set it)
    batch_size = None

    def __init__(self, batch_size, page_size, max_seq_len, device, n_layers, num_heads,
                 head_dim, disable_quant=False, hadamard_dtype=torch.float16, group_size=1,
                 lac=False):
        if disable_quant:
            raise NotImplementedError("the fp16 KV cache (disable_quant=True) is not built")
        if lac:
            raise NotImplementedError("learned activation clipping (lac=True) is not built")
        if head_dim != 128:
            raise ValueError("head_dim must be 128")
        _init_hf_cache(self)
        self.batch_size = batch_size
        self.page_size = page_size
        self.max_seq_len = max_seq_len
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.group_size = group_size
        self.hadamard_dtype = hadamard_dtype
        self.disable_quant = disable_quant
        self.lac = lac
        self.device = device
        self.length = 0
        pool = _pages_for(max_seq_len, page_size) * batch_size
        self.pages = torch.empty((pool, n_layers, 2, num_heads, page_size, head_dim // 2),
                                 dtype=torch.uint8, device=device)
        self.scales = torch.empty((pool, n_layers, 2, num_heads, page_size, 2),
                                  dtype=torch.float16, device=device)
        self._filled = [False] * n_layers          # layer holds its prefill
        self._table = _PageTable(batch_size, pool, device)
        self._frozen = False
        self._spec = {}
        self._point_spec()
        cus = torch.cuda.get_device_properties(device).multi_processor_count
        chunks = self.decode_chunks(batch_size, num_heads, max_seq_len, cus)
        self._decoder = _SplitDecoder(batch_size, num_heads * group_size, head_dim, chunks,
                                      device, hadamard_dtype)

    def _point_spec(self):
        """The keyword arguments of the paged ops, rebuilt whenever a tensor
        is reallocated (the dict object itself stays the same)."""
        self._spec.update(kv_data=self.pages, kv_param=self.scales,
                          kv_indptr=self._table.indptr, kv_indices=self._table.indices,
                          last_page_offset=self._table.last)

    @staticmethod
    def decode_chunks(batch_size, num_kv_heads, max_seq_len, cu_count):
        """Split-KV chunks per (request, KV head).  A batch with at least one
        (request, KV head) per CU is not split (the unsplit launch runs one
        eight-wave block per CU, and its outputs need no merge); otherwise
        enough chunks for about two four-wave blocks per CU (the registers
        leave room for two, so more chunks only queue), at least 128 tokens
        per chunk, at most 1024 chunks."""
        blocks = max(1, batch_size * num_kv_heads)
        if blocks >= cu_count:
            return 1
        want = -(-2 * cu_count // blocks)
        return max(1, min(want, max_seq_len // 128, 1024))

    def page_cnt_from_length(self, length):
        return (length + self.page_size - 1) // self.page_size

    @property
    def seen_tokens(self):
        return self.length

    def _reserve(self, tokens):
        """Make room for `tokens` per request, doubling the pool when it runs
        out (appended pages keep the j * B + b assignment of the old ones)."""
        need = self.page_cnt_from_length(tokens) * self.batch_size
        have = self.pages.shape[0]
        if need <= have:
            return
        total = max(need, 2 * have)
        extra = total - have
        self.pages = torch.cat([self.pages, self.pages.new_empty((extra, *self.pages.shape[1:]))])
        self.scales = torch.cat([self.scales,
                                 self.scales.new_empty((extra, *self.scales.shape[1:]))])
        self._table.grow(total)
        self._point_spec()

    def _quantize(self, key_states, value_states):
        """Head-dim Hadamard of K (as the decode query gets), then the int4
        quantizer of K and V: codes [B, T, H, D/2] and params [B, T, H, 2]."""
        k = key_states
        if self.hadamard_dtype is not None:
            k = matmul_had_cuda(k, dtype=self.hadamard_dtype)
        kq, kp = signrot_kernel.kv_quant_pack(k)
        vq, vp = signrot_kernel.kv_quant_pack(value_states)
        return kq, kp, vq, vp

    def update(self, key_states, value_states, layer_idx,
               cache_kwargs: Optional[Dict[str, Any]] = None):
        """Quantize and store K/V [B, T, H, D] of one layer (the reference's
        update, kv_cache.py:291-415).  The first call for a layer is the
        prefill: the tokens are written in bulk (init_kv_i4; with an
        attention_mask only its 1-positions) and the fp16 inputs are returned
        for the prefill attention.  Later calls append one token per request
        (append_kv_i4) and return the layer's decode attention."""
        B, T, H, D = key_states.shape
        if H != self.num_heads:
            raise ValueError(f"update() takes the {self.num_heads} KV heads, got {H}")
        if B != self.batch_size:
            raise ValueError(f"batch {B} != the cache's {self.batch_size}")
        mask = (cache_kwargs or {}).get("attention_mask")
        kq, kp, vq, vp = self._quantize(key_states, value_states)
        if layer_idx == 0:
            self._reserve(self.length + T)
            self.length += T
        spec = self.get_cache_specs_for_flash_infer(mask)
        if not self._filled[layer_idx]:
            self._filled[layer_idx] = True
            kq, kp = kq.reshape(B * T, H, D // 2), kp.reshape(B * T, H, 2)
            vq, vp = vq.reshape(B * T, H, D // 2), vp.reshape(B * T, H, 2)
            if mask is None:
                starts = torch.arange(B + 1, device=self.device, dtype=torch.int32) * T
            else:
                live = mask.flatten().nonzero().flatten()
                kq, kp, vq, vp = kq[live], kp[live], vq[live], vp[live]
                counts = mask.sum(dim=-1, dtype=torch.int32)
                starts = torch.zeros(B + 1, device=self.device, dtype=torch.int32)
                torch.cumsum(counts, dim=0, out=starts[1:])
            init_kv_i4(**spec, k=kq.contiguous(), v=vq.contiguous(), k_param=kp.contiguous(),
                       v_param=vp.contiguous(), seqlen_indptr=starts, layer_idx=layer_idx)
            return key_states, value_states
        if T != 1:
            raise ValueError("after the prefill, update() appends one token per request")
        append_kv_i4(**spec, k=kq.view(B, H, D // 2), v=vq.view(B, H, D // 2),
                     k_param=kp.view(B, H, 2), v_param=vp.view(B, H, 2), layer_idx=layer_idx)
        return _LayerAttention(self._decoder, spec, layer_idx)

    def update_qkv_fused(self, qkv, cos, sin, layer_idx, num_q_heads, attention_mask=None):
        """Decode-step form of update() plus the decode query's rotation, one
        kernel: qkv f16 [B, (Hq + 2 H) D] is the q/k/v projection output of
        the new token; q and k get RoPE (cos/sin [1 or B, 1, D]) and the
        head-dim Hadamard, k and v are quantized into the cache.  Returns the
        rotated q [B, Hq, D] for decode_rotated.  Bit for bit the same as
        rope_qk + update() + the query rotation.  The layer must hold its
        prefill already.  attention_mask as for update() (the extended HF
        mask after a left-padded prefill) or None."""
        spec = self._qkv_step(qkv, layer_idx, attention_mask, "update_qkv_fused")
        return _CUDA.qkv_rope_had_append(qkv, cos.contiguous(), sin.contiguous(), num_q_heads,
                                         self.num_heads, **spec, layer_idx=layer_idx,
                                         had_scale=1 / math.sqrt(self.head_dim),
                                         rotate=self.hadamard_dtype is not None)

    def _qkv_step(self, qkv, layer_idx, attention_mask, name):
        if not self._filled[layer_idx]:
            raise RuntimeError(f"{name}: the layer has no prefill yet")
        if qkv.shape[0] != self.batch_size:
            raise ValueError(f"batch {qkv.shape[0]} != the cache's {self.batch_size}")
        if layer_idx == 0:
            self._reserve(self.length + 1)
            self.length += 1
        return self.get_cache_specs_for_flash_infer(attention_mask)

    def update_qkv_decode(self, qkv, cos, sin, layer_idx, num_q_heads, attention_mask=None):
        """update_qkv_fused followed by decode_rotated, one kernel: the new
        token's k / v go into the cache and the attention output o [B, Hq, D]
        is returned; bit for bit the two calls."""
        spec = self._qkv_step(qkv, layer_idx, attention_mask, "update_qkv_decode")
        return self._decoder.qkv_attend(qkv, cos.contiguous(), sin.contiguous(), spec, layer_idx,
                                        num_q_heads, 1 / math.sqrt(self.head_dim),
                                        self.hadamard_dtype is not None)

    def update_qkv_decode_quant(self, qkv, cos, sin, layer_idx, num_q_heads, scale,
                                attention_mask=None):
        """update_qkv_fused followed by decode_rotated_quant (the o_proj
        input: codes [B, Hq D / 2], scales [B, 1]) with the q/k/v step and the
        attention in one kernel; bit for bit the two calls."""
        spec = self._qkv_step(qkv, layer_idx, attention_mask, "update_qkv_decode_quant")
        return self._decoder.qkv_attend_head_had_quant(
            qkv, cos.contiguous(), sin.contiguous(), spec, layer_idx, num_q_heads,
            1 / math.sqrt(self.head_dim), self.hadamard_dtype is not None, scale)

    def decode_rotated(self, q_rot, layer_idx):
        """Decode attention of an already rotated q [B, Hq, D] over this
        layer's cache (after update_qkv_fused) -> [B, Hq, D]."""
        return self._decoder.attend(q_rot, self._spec, layer_idx)

    def decode_rotated_quant(self, q_rot, layer_idx, scale):
        """decode_rotated followed by the head-axis Hadamard (times scale)
        and the per-token quantizer: (codes [B, Hq D / 2], scales [B, 1])."""
        return self._decoder.attend_head_had_quant(q_rot, self._spec, layer_idx, scale)

    # ---------------------------------------------------------- index specs
    def specs(self):
        """The op keyword arguments (kv_data, kv_param, kv_indptr, kv_indices,
        last_page_offset) as they stand."""
        return self._spec

    def refresh_specs(self, length: Optional[int] = None):
        """Rewrite the index tensors in place for a batch of `length` tokens
        per request (default: the current length) and return the specs.  A
        graph-captured decode step calls this before each replay, with the
        specs frozen inside the capture (kv_cache.py:435-464)."""
        self._table.set_uniform(self.length if length is None else length, self.page_size)
        return self._spec

    def freeze_specs(self, frozen=True):
        """While frozen, update() uses the index tensors as they are (no
        refresh), so it can be captured in a graph."""
        self._frozen = frozen

    def get_cache_specs_for_flash_infer(self, attention_mask):
        if attention_mask is not None:
            self._table.set_from_mask(attention_mask, self.page_size)
        elif not self._frozen:
            self._table.set_uniform(self.length, self.page_size)
        return self._spec

    def mark_prefilled(self, length: int):
        """Declare that every layer holds `length` tokens per request, written
        into `pages` / `scales` directly (benchmarks and tests with synthetic
        contexts); the next update() of each layer appends."""
        self._reserve(length)
        self.length = length
        self._filled = [True] * len(self._filled)

    def clone(self):
        """An independent copy: own pages, scales and index tensors, same
        state (length, prefilled layers, split-KV configuration)."""
        c = object.__new__(MultiLayerPagedKVCache4Bit)
        c.__dict__.update(self.__dict__)
        c.pages, c.scales = self.pages.clone(), self.scales.clone()
        c._filled = list(self._filled)
        c._table = self._table.clone()
        c._spec = {}
        c._point_spec()
        dec = _SplitDecoder.__new__(_SplitDecoder)
        dec.__dict__.update(self._decoder.__dict__)
        dec.tmp = None if self._decoder.tmp is None else torch.empty_like(self._decoder.tmp)
        c._decoder = dec
        return c

    def reset(self):
        self.length = 0
        self._filled = [False] * len(self._filled)

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        return self.length

    def get_max_length(self) -> Optional[int]:
        return None

    def __len__(self):
        """The number of layers the cache holds (HF Cache's meaning; also
        keeps `bool(cache)` true)."""
        return len(self._filled)

    def get_usable_length(self, new_seq_length: int, layer_idx: Optional[int] = 0) -> int:
        """Cached tokens the new ones can attend to (HF Cache's rule): all of
        them, the cache having no maximum length."""
        prev = self.get_seq_length(layer_idx)
        cap = self.get_max_length()
        if cap is not None and prev + new_seq_length > cap:
            return cap - new_seq_length
        return prev

    def to_legacy_cache(self):
        return self


class HFCacheAdapter(Cache):
    """An HF Cache that forwards to an inner cache object (kv_cache.py:
    501-520): lets a MultiLayerPagedKVCache4Bit, or any object with the same
    methods, stand where transformers expects a Cache."""

    def __init__(self, inner):
        _init_hf_cache(self)
        self.inner = inner

    def get_usable_length(self, kv_seq_len: int, layer_idx: int) -> int:
        return self.inner.get_usable_length(kv_seq_len, layer_idx)

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        return self.inner.get_seq_length()

    def get_max_length(self) -> Optional[int]:
        return self.inner.get_max_length()

    def update(self, key_states, value_states, layer_idx: int, cache_kwargs=None):
        return self.inner.update(key_states, value_states, layer_idx, cache_kwargs)

    def to_legacy_cache(self):
        to_legacy = getattr(self.inner, "to_legacy_cache", None)
        return to_legacy() if to_legacy is not None else self
