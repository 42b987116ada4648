"""Paged int4 KV cache and decode-attention stub, mirroring
signrot/transformers/kv_cache.py:60-498 on the HIP op table.

Differences from the reference, none of which change results:
  * KV heads are stored once.  The reference repeats each KV head
    `group_size` times in the cache (kv_cache.py:346-353) because its decode
    kernel needs as many KV heads as query heads; batch_decode_i4 here maps
    query head h to KV head h // group_size itself, so the cache is
    group_size times smaller and decode reads group_size times fewer bytes.
  * The split-KV chunk count targets two 256-thread blocks per CU (the
    reference targets two blocks of 128 threads, kv_cache.py:236-258).
  * Only the int4 path exists: disable_quant=True (fp16 cache) and lac=True
    (learned clipping, unused by the reference itself) raise
    NotImplementedError.
"""
import functools
import math
from typing import Any, Dict, Optional

import torch

from .. import _CUDA
from ..functional import kernel as signrot_kernel


def unpack_i4_and_asym_dequantize(q, scale, zero, lac: bool = False):
    """uint4 unpack (low nibble first) and q * scale - zero
    (kv_cache.py:60-68)."""
    assert q.dtype == torch.uint8
    q = torch.stack((q & 0x0F, (q >> 4) & 0x0F), dim=-1).view(*q.shape[:-1], q.shape[-1] * 2)
    if lac:
        return scale * (q - zero)
    return q * scale - zero


def matmul_had_cuda(X, dtype):
    """Sylvester WHT over the last dim scaled by 1/sqrt(n) in `dtype`
    (kv_cache.py:70-73)."""
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


class _AttentionStub(object):
    """Decode attention over the cache (kv_cache.py:144-170): q [B, 1, Hq, D]
    is rotated by the head-dim Hadamard (matching the rotated keys), then
    batch_decode_i4; returns [B, 1, Hq, D]."""

    def __init__(self, cache_page_size, device, n_layers, disable_quant, hadamard_dtype):
        self.cache_page_size = cache_page_size
        self.n_layers = n_layers
        self.disable_quant = disable_quant
        self.hadamard_dtype = hadamard_dtype
        self.num_chunks = 1
        self.tmp = None

    def forward(self, q, num_kv_heads, attention_kwargs, layer_idx):
        batch_size, q_len, num_qo_heads, head_dim = q.shape
        assert q_len == 1
        q = q.view(batch_size, num_qo_heads, head_dim)
        if self.hadamard_dtype is not None:
            q = matmul_had_cuda(q, dtype=self.hadamard_dtype)
        return self.attend_rotated(q, attention_kwargs, layer_idx).unsqueeze(1)

    def attend_rotated(self, q, attention_kwargs, layer_idx):
        """batch_decode_i4 of an already rotated q [B, Hq, D] -> [B, Hq, D]."""
        attn_output = torch.empty_like(q)
        tmp = self.tmp
        if tmp is not None and tmp.shape[1] != q.shape[1]:
            tmp = None
        batch_decode_i4(attn_output, q, **attention_kwargs, layer_idx=layer_idx, tmp=tmp,
                        num_chunks=self.num_chunks if tmp is not None else 1)
        return attn_output


class MultiLayerPagedKVCache4Bit(object):
    """Paged int4 KV cache for all layers (kv_cache.py:173-498).

    pages  u8  [pages, n_layers, 2, num_heads, page_size, head_dim / 2]
    scales f16 [pages, n_layers, 2, num_heads, page_size, 2]
    Physical page of (request b, page j) is j * batch_size + b.
    `num_heads` is the number of KV heads; `group_size` is the number of
    query heads per KV head."""

    def __init__(self, batch_size, page_size, max_seq_len, device, n_layers, num_heads,
                 head_dim, disable_quant=False, hadamard_dtype=torch.float16, group_size=1,
                 lac=False):
        if disable_quant:
            raise NotImplementedError("the fp16 KV cache (disable_quant=True) is not built")
        if lac:
            raise NotImplementedError("learned activation clipping (lac=True) is not built")
        if head_dim != 128:
            raise ValueError("head_dim must be 128")
        self.lac = lac
        self.page_size = page_size
        self.batch_size = batch_size
        self.disable_quant = disable_quant
        self.num_heads = num_heads
        self.head_dim = head_dim
        max_page_cnt = self.page_cnt_from_length(max_seq_len)
        self.pages = torch.empty((max_page_cnt * batch_size, n_layers, 2, num_heads, page_size,
                                  head_dim // 2), dtype=torch.uint8, device=device)
        self.scales = torch.empty((max_page_cnt * batch_size, n_layers, 2, num_heads, page_size,
                                   2), dtype=torch.float16, device=device)
        self.max_seq_len = max_seq_len
        self._needs_init = [True] * n_layers
        self.length = 0
        self.device = device
        self.hadamard_dtype = hadamard_dtype
        self.group_size = group_size
        self._stub = _AttentionStub(self.page_size, device, n_layers, disable_quant,
                                    hadamard_dtype)
        # persistent index buffers, refreshed in place (graph-safe addresses)
        self._kv_indices_full = torch.empty(self.pages.shape[0], device=device, dtype=torch.int32)
        self._spec_page_cnt = None
        self._last_page_offset = torch.empty(batch_size, device=device, dtype=torch.int32)
        self._indptr_base = torch.arange(batch_size + 1, device=device, dtype=torch.int32)
        self._kv_indptr_buf = torch.empty(batch_size + 1, device=device, dtype=torch.int32)
        self._specs_frozen = False
        self._spec_cache = {
            "kv_data": self.pages,
            "kv_param": self.scales,
            "kv_indptr": self._kv_indptr_buf,
            "kv_indices": self._kv_indices_full,
            "last_page_offset": self._last_page_offset,
        }
        self._configure_decode_split(batch_size, num_heads * group_size, head_dim,
                                     max_seq_len, device)

    @staticmethod
    def decode_chunks(batch_size, num_kv_heads, max_seq_len, cu_count):
        """Split-KV chunk count: about two blocks per CU (the decode kernel's
        register use leaves room for two four-wave blocks per CU, so further
        chunks only queue), at most one chunk per 128 tokens of context, at
        most 1024."""
        target_blocks = 2 * cu_count
        chunks = max(1, -(-target_blocks // max(1, batch_size * num_kv_heads)))
        return max(1, min(chunks, max_seq_len // 128, 1024))

    def _configure_decode_split(self, batch_size, num_qo_heads, head_dim, max_seq_len, device):
        cus = torch.cuda.get_device_properties(device).multi_processor_count
        chunks = self.decode_chunks(batch_size, self.num_heads, max_seq_len, cus)
        self._stub.num_chunks = chunks
        if chunks > 1:
            self._stub.tmp = torch.empty((batch_size, num_qo_heads, chunks, head_dim + 4),
                                         dtype=torch.float32, device=device)

    def page_cnt_from_length(self, length):
        return (length + self.page_size - 1) // self.page_size

    def _ensure_page_cnt_per_batch(self, expected_page_cnt_per_batch):
        """Grow the page pool by doubling (kv_cache.py:260-289)."""
        expected_total = expected_page_cnt_per_batch * self.batch_size
        current_total = self.pages.shape[0]
        if expected_total <= current_total:
            return
        grow_to_total = max(expected_total, current_total * 2)
        add_total = grow_to_total - current_total
        self.pages = torch.cat([self.pages, self.pages.new_empty((add_total,
                                                                  *self.pages.shape[1:]))])
        self.scales = torch.cat([self.scales, self.scales.new_empty((add_total,
                                                                     *self.scales.shape[1:]))])
        self._kv_indices_full = torch.empty(self.pages.shape[0], device=self.device,
                                            dtype=torch.int32)
        self._spec_page_cnt = None
        self._spec_cache.update(kv_data=self.pages, kv_param=self.scales,
                                kv_indices=self._kv_indices_full)

    @property
    def seen_tokens(self):
        return self.length

    def update(self, key_states, value_states, layer_idx, cache_kwargs: Optional[Dict[str, Any]]
               = None):
        """Quantize and store K/V [B, T, H, D] of one layer (kv_cache.py:291-415).
        The first call per layer fills (init_kv_i4) and returns the inputs;
        later calls (T == 1) append and return the decode stub bound to this
        layer."""
        cache_kwargs = cache_kwargs or {}
        b_sz, added_length, num_heads, head_dim = key_states.shape
        assert num_heads == self.num_heads, "update() takes the KV heads"
        orig_key_states, orig_value_states = key_states, value_states
        if self.hadamard_dtype is not None:
            key_states = matmul_had_cuda(key_states, dtype=self.hadamard_dtype)
        key_states, k_param = signrot_kernel.kv_quant_pack(key_states)
        value_states, v_param = signrot_kernel.kv_quant_pack(value_states)
        k_param = k_param.view(self.batch_size * added_length, num_heads, 2)
        v_param = v_param.view(self.batch_size * added_length, num_heads, 2)
        qhd = self.pages.shape[-1]
        assert b_sz == self.batch_size
        if layer_idx == 0:
            new_length = self.length + added_length
            self._ensure_page_cnt_per_batch(self.page_cnt_from_length(new_length))
            self.length = new_length
        attention_mask = cache_kwargs.get("attention_mask")
        specs = self.get_cache_specs_for_flash_infer(attention_mask)
        if self._needs_init[layer_idx]:
            self._needs_init[layer_idx] = False
            if attention_mask is not None:
                keep = torch.nonzero(attention_mask.flatten(), as_tuple=False).flatten()
                key_states = key_states.reshape(-1, num_heads * qhd)[keep]
                value_states = value_states.reshape(-1, num_heads * qhd)[keep]
                k_param = k_param.reshape(-1, num_heads * 2)[keep]
                v_param = v_param.reshape(-1, num_heads * 2)[keep]
                seqlens = torch.nn.functional.pad(
                    torch.cumsum(attention_mask.sum(dim=-1, dtype=torch.int32), dim=0,
                                 dtype=torch.int32), (1, 0))
            else:
                seqlens = torch.arange(self.batch_size + 1, device=self.device,
                                       dtype=torch.int32) * added_length
            init_kv_i4(**specs,
                       k=key_states.reshape(-1, num_heads, qhd).contiguous(),
                       v=value_states.reshape(-1, num_heads, qhd).contiguous(),
                       k_param=k_param.reshape(-1, num_heads, 2).contiguous(),
                       v_param=v_param.reshape(-1, num_heads, 2).contiguous(),
                       seqlen_indptr=seqlens, layer_idx=layer_idx)
            return orig_key_states, orig_value_states
        assert added_length == 1
        append_kv_i4(**specs,
                     k=key_states.view(self.batch_size, num_heads, qhd),
                     v=value_states.view(self.batch_size, num_heads, qhd),
                     k_param=k_param.view(-1, num_heads, 2),
                     v_param=v_param.view(-1, num_heads, 2),
                     layer_idx=layer_idx)
        return functools.partial(self._stub.forward, num_kv_heads=num_heads,
                                 attention_kwargs=specs, layer_idx=layer_idx)

    def update_qkv_fused(self, qkv, cos, sin, layer_idx, num_q_heads):
        """Decode-step form of update() + the stub's q rotation, one kernel:
        qkv f16 [B, (Hq + 2 H) D] is the q/k/v projection output of the new
        token; q and k get RoPE (cos/sin [1 or B, 1, D]) and the head-dim
        Hadamard, k and v are quantized into the cache.  Returns the rotated
        q [B, Hq, D] for decode_rotated.  Results equal
        rope_qk + update() + the stub's q rotation bit for bit.  The layer
        must already hold its prefill (one new token per request here)."""
        if self._needs_init[layer_idx]:
            raise RuntimeError("update_qkv_fused: the layer has no prefill yet")
        b_sz = qkv.shape[0]
        assert b_sz == self.batch_size
        if layer_idx == 0:
            new_length = self.length + 1
            self._ensure_page_cnt_per_batch(self.page_cnt_from_length(new_length))
            self.length = new_length
        specs = self.get_cache_specs_for_flash_infer(None)
        rotate = self.hadamard_dtype is not None
        return _CUDA.qkv_rope_had_append(qkv, cos.contiguous(), sin.contiguous(), num_q_heads,
                                         self.num_heads, **specs, layer_idx=layer_idx,
                                         had_scale=1 / math.sqrt(self.head_dim), rotate=rotate)

    def decode_rotated(self, q_rot, layer_idx):
        """Decode attention of an already rotated q [B, Hq, D] over this
        layer's cache (after update_qkv_fused) -> [B, Hq, D]."""
        return self._stub.attend_rotated(q_rot, self._spec_cache, layer_idx)

    def _set_page_cnt(self, page_cnt: int):
        """indptr = b * page_cnt; indices[b, j] = j * B + b
        (kv_cache.py:417-433)."""
        torch.mul(self._indptr_base, page_cnt, out=self._kv_indptr_buf)
        if self._spec_page_cnt == page_cnt:
            return
        self._spec_page_cnt = page_cnt
        idx = (torch.arange(page_cnt, device=self.device, dtype=torch.int32) *
               self.batch_size).unsqueeze(0) + torch.arange(
                   self.batch_size, device=self.device, dtype=torch.int32).unsqueeze(1)
        self._kv_indices_full[:page_cnt * self.batch_size].copy_(idx.reshape(-1))

    def refresh_specs(self, length: Optional[int] = None):
        """Index buffers for a uniform-length batch (kv_cache.py:435-456)."""
        if length is None:
            length = self.length
        page_cnt = self.page_cnt_from_length(length)
        page_ptr = length % self.page_size
        if length != 0 and page_ptr == 0:
            page_ptr = self.page_size
        self._last_page_offset.fill_(page_ptr)
        self._set_page_cnt(page_cnt)
        return self._spec_cache

    def freeze_specs(self, frozen=True):
        self._specs_frozen = frozen

    def get_cache_specs_for_flash_infer(self, attention_mask):
        if attention_mask is None:
            return self._spec_cache if self._specs_frozen else self.refresh_specs()
        seqlens = attention_mask.sum(dim=-1, dtype=torch.int32)
        page_cnt = self.page_cnt_from_length(seqlens)
        if (page_cnt[0] != page_cnt).any():
            raise NotImplementedError("Current implementation does not support the case where "
                                      "batches have different number of pages")
        page_cnt = int(page_cnt[0])
        page_ptr = seqlens % self.page_size
        page_ptr = torch.where((seqlens != 0) & (page_ptr == 0), self.page_size, page_ptr)
        self._last_page_offset.copy_(page_ptr)
        self._set_page_cnt(page_cnt)
        return self._spec_cache

    def reset(self):
        self.length = 0
        self._needs_init = [True] * len(self._needs_init)

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        return self.length

    def get_max_length(self) -> Optional[int]:
        return None

    def to_legacy_cache(self):
        return self
