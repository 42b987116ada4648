"""One Llama decoder layer on the W4A4 real-quant path, decode step.

Mirrors the decode forward of the reference's quantized Llama layer
(e2e/quantized_llama/modeling_llama.py:19-137: SignrotFP16LlamaAttention.
forward, SignrotLlamaAttention, SignrotLlamaMLP) inside HF's LlamaDecoderLayer
residual structure, with every op on this package's HIP kernels:

  h -> RMSNorm -> Quantizer -> q/k/v Linear4bit -> RoPE -> cache.update
    (K Hadamard(D), KV int4 quantize, append) -> decode stub (q Hadamard(D),
    batch_decode_i4) -> head-axis OnlineHadamard(num_heads) -> Quantizer ->
    o_proj -> + h -> RMSNorm -> Quantizer -> gate/up Linear4bit -> SwiGLU ->
    OnlineHadamard(ffn) (+ sign) -> Quantizer -> down_proj -> + residual.

q/k/v (and gate/up) share one quantized input, so their weights are stored
concatenated along the output dim and run as one GEMM; the outputs are the
same as the separate Linear4bit modules' (per-row / per-column dequant).
"""

import torch

from .. import _CUDA
from ..functional import kernel
from ..functional.hadamard import _inv_sqrt_f32, get_hadK, matmul_hadU_cuda
from ..functional.quantization import rtn_weight_pack
from ..nn.normalization import RMSNorm


def rope_cos_sin(positions, head_dim, theta, device):
    """HF Llama rotary tables for the given positions: cos/sin fp16
    [1, len(positions), head_dim] (emb = cat(freqs, freqs))."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    freqs = torch.as_tensor(positions, dtype=torch.float32)[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return (emb.cos().half().unsqueeze(0).to(device), emb.sin().half().unsqueeze(0).to(device))


class W4A4LlamaDecodeLayer(torch.nn.Module):
    """Decoder layer for single-token decode over a MultiLayerPagedKVCache4Bit.

    Weights (int4 codes packed two per byte, fp16 per-output-channel scales):
      w_qkv [Hq*D + 2*Hkv*D, hidden/2], w_o [hidden, hidden/2],
      w_gu [2*ffn, hidden/2] (gate rows then up rows), w_down [hidden, ffn/2],
    and down_sign int8 [ffn] (the SignRot ±1 vector of the down-proj
    rotation)."""

    def __init__(self, hidden, n_heads, n_kv_heads, head_dim, ffn, layer_idx=0, eps=1e-5,
                 rope_theta=500000.0):
        super().__init__()
        assert hidden == n_heads * head_dim and n_heads % n_kv_heads == 0
        self.hidden, self.n_heads, self.n_kv = hidden, n_heads, n_kv_heads
        self.head_dim, self.ffn, self.layer_idx = head_dim, ffn, layer_idx
        self.rope_theta = rope_theta
        self.input_layernorm = RMSNorm(hidden, eps)
        self.post_attention_layernorm = RMSNorm(hidden, eps)
        nqkv = (n_heads + 2 * n_kv_heads) * head_dim
        for name, rows, cols in (("qkv", nqkv, hidden), ("o", hidden, hidden),
                                 ("gu", 2 * ffn, hidden), ("down", hidden, ffn)):
            self.register_buffer(f"w_{name}", torch.zeros(rows, cols // 2, dtype=torch.uint8))
            self.register_buffer(f"s_{name}", torch.zeros(rows, dtype=torch.float16))
        self.register_buffer("down_sign", torch.ones(ffn, dtype=torch.int8))
        had, k = get_hadK(ffn)
        self.down_k = k
        self.register_buffer("down_hadk", had.half() if had is not None else None)

    @classmethod
    def random(cls, hidden, n_heads, n_kv_heads, head_dim, ffn, layer_idx=0, seed=0,
               device="cuda", std=0.02, **kw):
        """Random-init layer: weights N(0, std) fp16, RTN per-channel int4 (the
        down-proj weight with a random ±1 sign folded by column, on the
        symmetric grid, as rtn_fwrd does when a sign is present)."""
        layer = cls(hidden, n_heads, n_kv_heads, head_dim, ffn, layer_idx, **kw)
        g = torch.Generator().manual_seed(seed)
        sign = (torch.randint(0, 2, (ffn,), generator=g) * 2 - 1).to(torch.int8)
        layer.down_sign.copy_(sign)
        for name in ("qkv", "o", "gu", "down"):
            w_buf = getattr(layer, f"w_{name}")
            w = (torch.randn(w_buf.shape[0], w_buf.shape[1] * 2, generator=g) * std).half()
            if name == "down":
                w = w * sign.half()
            packed, scale, _ = rtn_weight_pack(w, symmetric_grid=(name == "down"))
            w_buf.copy_(packed)
            getattr(layer, f"s_{name}").copy_(scale)
        return layer.to(device)

    def _gate_up_interleaved(self):
        """w_gu / s_gu in the blocks-of-8 gate/up layout of
        w4a4_linear_swiglu: a derived copy (2 ffn x hidden / 2 bytes), made
        on first use and again whenever w_gu or s_gu changes in place."""
        key = (self.w_gu.data_ptr(), self.w_gu._version, self.s_gu.data_ptr(),
               self.s_gu._version)
        if getattr(self, "_gu_il_key", None) != key:
            self._gu_il = _CUDA.interleave_gate_up(self.w_gu, self.s_gu, self.ffn)
            self._gu_il_key = key
        return self._gu_il

    def _linear(self, xq, name):
        q, s = xq.quantized_x, xq.scales_x
        return _CUDA.w4a4_linear(q.view(-1, q.shape[-1]), s.view(-1), getattr(self, f"w_{name}"),
                                 getattr(self, f"s_{name}"))

    def forward(self, hidden_states, cache, cos, sin, trace=None, fused=True,
                attention_mask=None):
        """hidden_states fp16 [B, 1, hidden]; cos/sin fp16 [1 or B, 1, head_dim]
        for the new position; returns fp16 [B, 1, hidden].  The cache must
        already hold this layer's context (its first update was a prefill).
        attention_mask: after a left-padded prefill, HF's mask extended by a
        1 per decoded token ([B, prompt + steps]; it gives each request's
        length), else None.  With a dict `trace`, the intermediates are
        stored in it (checkers) and the op-by-op path runs; otherwise
        (fused=True) the fused kernels run, with bit-identical results."""
        if fused and trace is None:
            return self._forward_fused(hidden_states, cache, cos, sin, attention_mask)
        return self._forward_ops(hidden_states, cache, cos, sin, trace, attention_mask)

    def _forward_fused(self, hidden_states, cache, cos, sin, attention_mask=None):
        """The decode step in 9 launches: rmsnorm_quant -> q/k/v GEMM ->
        qkv_decode_i4 (RoPE, K/q Hadamard, KV quantize + append, and the
        attention, one kernel) -> head_had_quant (head-axis Hadamard +
        quantizer; merge_head_had_quant with the split-KV merge folded in
        when the batch is split) -> o_proj GEMM + residual -> rmsnorm_quant ->
        gate/up GEMM with the SwiGLU in its epilogue (ffn % 8 == 0; else the
        GEMM and swiglu_had_sign_quant) -> had_sign_quant -> down GEMM +
        residual."""
        B = hidden_states.shape[0]
        x2 = hidden_states.view(B, self.hidden)
        n1, n2 = self.input_layernorm, self.post_attention_layernorm
        q1, s1 = _CUDA.rmsnorm_quant(x2, n1.eps, n1.mean_dim)
        qkv = _CUDA.w4a4_linear(q1, s1.view(-1), self.w_qkv, self.s_qkv)
        qa, sa = cache.update_qkv_decode_quant(qkv, cos, sin, self.layer_idx, self.n_heads,
                                               _inv_sqrt_f32(self.n_heads), attention_mask)
        x2 = _CUDA.w4a4_linear_residual(qa, sa.view(-1), self.w_o, self.s_o, x2)
        q2, s2 = _CUDA.rmsnorm_quant(x2, n2.eps, n2.mean_dim)
        if self.ffn % 8 == 0:
            # SwiGLU in the gate/up GEMM's epilogue, then the plain rotation
            w_il, s_il = self._gate_up_interleaved()
            a = _CUDA.w4a4_linear_swiglu(q2, s2.view(-1), w_il, s_il)
            qd, sd = _CUDA.had_sign_quant(a, self.down_hadk, self.down_k, self.down_sign)
            out = _CUDA.w4a4_linear_residual(qd, sd.view(-1), self.w_down, self.s_down, x2,
                                             out=x2)
            return out.view(B, 1, self.hidden)
        gu = _CUDA.w4a4_linear(q2, s2.view(-1), self.w_gu, self.s_gu)
        if _CUDA.swiglu_had_fusable(self.ffn, self.down_k):
            qd, sd = _CUDA.swiglu_had_sign_quant(gu, self.down_hadk, self.down_k,
                                                 self.down_sign)
        else:  # no fused SwiGLU form of this rotation size
            a = kernel.swiglu(gu[:, : self.ffn], gu[:, self.ffn:])
            qd, sd = _CUDA.had_sign_quant(a, self.down_hadk, self.down_k, self.down_sign)
        out = _CUDA.w4a4_linear_residual(qd, sd.view(-1), self.w_down, self.s_down, x2, out=x2)
        return out.view(B, 1, self.hidden)

    def _forward_ops(self, hidden_states, cache, cos, sin, trace=None, attention_mask=None):
        """Op-by-op decode step (the reference's sequence of ops)."""
        B = hidden_states.shape[0]
        D, Hq, Hk = self.head_dim, self.n_heads, self.n_kv
        x2 = hidden_states.view(B, self.hidden)
        keep = self._keeper(trace)

        # ---- attention
        h = self.input_layernorm(x2)
        qkv = self._linear(kernel.PackedQuantizedTensor(*kernel.sym_quant_dynamic(h)), "qkv")
        keep("norm1", h)
        keep("qkv", qkv)
        q = qkv[:, : Hq * D].contiguous().view(B, 1, Hq, D)
        k = qkv[:, Hq * D: (Hq + Hk) * D].contiguous().view(B, 1, Hk, D)
        v = qkv[:, (Hq + Hk) * D:].contiguous().view(B, 1, Hk, D)
        kernel.rope_qk(q, k, cos, sin)
        keep("q_rope", q)
        keep("k_rope", k)
        attend = cache.update(k, v, self.layer_idx, {"attention_mask": attention_mask})
        attn = attend(q)                                      # [B, 1, Hq, D]
        keep("attn", attn)
        x2 = self._attn_out(attn, x2, keep)
        return self._mlp(x2, keep).view(B, 1, self.hidden)

    def prefill(self, hidden_states, cache, cos, sin, attention_mask=None, trace=None):
        """The layer's first update: T tokens per request
        (modeling_llama.py:26-100 with the cache's first update,
        kv_cache.py:295-395).  hidden_states fp16 [B, T, hidden]; cos/sin
        fp16 [1 or B, T, head_dim] (left-padded rows take the positions of
        their real tokens, as HF's position_ids do); attention_mask int
        [B, T] (1 = token, 0 = left padding) or None.  K/V are quantized into
        the cache (only the mask's 1-positions), the attention runs causal
        over the fp16 q/k/v (the flash-attn 2 call it replaces), then o_proj
        and the MLP as in decode.  Returns fp16 [B, T, hidden]; rows at
        padding positions are computed but carry no meaning."""
        B, T, _ = hidden_states.shape
        D, Hq, Hk = self.head_dim, self.n_heads, self.n_kv
        x2 = hidden_states.reshape(B * T, self.hidden)
        keep = self._keeper(trace)
        h = self.input_layernorm(x2)
        qkv = self._linear(kernel.PackedQuantizedTensor(*kernel.sym_quant_dynamic(h)), "qkv")
        keep("norm1", h)
        keep("qkv", qkv)
        q = qkv[:, : Hq * D].reshape(B, T, Hq, D).contiguous()
        k = qkv[:, Hq * D: (Hq + Hk) * D].reshape(B, T, Hk, D).contiguous()
        v = qkv[:, (Hq + Hk) * D:].reshape(B, T, Hk, D).contiguous()
        kernel.rope_qk(q, k, cos, sin)
        keep("q_rope", q)
        keep("k_rope", k)
        out = cache.update(k, v, self.layer_idx, {"attention_mask": attention_mask})
        if not isinstance(out, tuple):
            raise RuntimeError("prefill: the cache already holds this layer's context")
        k_f, v_f = out
        attn = _CUDA.prefill_attention(q, k_f, v_f, attention_mask, causal=True)
        keep("attn", attn)
        x2 = self._attn_out(attn.reshape(B * T, Hq, D), x2, keep)
        return self._mlp(x2, keep).view(B, T, self.hidden)

    @staticmethod
    def _keeper(trace):
        def keep(name, t):
            if trace is not None:
                trace[name] = t.clone()
        return keep

    def _attn_out(self, attn, x2, keep):
        """x2 + o_proj(head-axis Hadamard(attn)); attn [R, ..., Hq, D] over
        the R rows of x2 [R, hidden] (modeling_llama.py:94-96)."""
        R = x2.shape[0]
        attn = attn.reshape(R, 1, self.n_heads, self.head_dim)
        attn = attn.transpose(-1, -2).contiguous()            # [R, 1, D, Hq]
        attn = matmul_hadU_cuda(attn, None, 1)
        attn = attn.transpose(-1, -2).reshape(R, self.hidden)
        keep("attn_rot", attn)
        o = self._linear(kernel.PackedQuantizedTensor(*kernel.sym_quant_dynamic(attn)), "o")
        x2 = x2 + o
        keep("resid1", x2)
        return x2

    def _mlp(self, x2, keep):
        """x2 + down(OnlineHadamard(SwiGLU(gate/up(RMSNorm(x2)))))
        (modeling_llama.py:119-142)."""
        h = self.post_attention_layernorm(x2)
        gu = self._linear(kernel.PackedQuantizedTensor(*kernel.sym_quant_dynamic(h)), "gu")
        keep("norm2", h)
        keep("gu", gu)
        a = kernel.swiglu(gu[:, : self.ffn], gu[:, self.ffn:])
        keep("act", a)
        q_a, s_a = _CUDA.had_sign_quant(a, self.down_hadk, self.down_k, self.down_sign)
        keep("down_q", q_a)
        keep("down_s", s_a)
        d = _CUDA.w4a4_linear(q_a, s_a.view(-1), self.w_down, self.s_down)
        keep("down", d)
        return x2 + d

    def unpacked(self):
        """Host copies of the weights for checkers: {name: (codes u8, scales
        f16)} plus the down-proj sign and hadK."""
        out = {n: (getattr(self, f"w_{n}").cpu().numpy(), getattr(self, f"s_{n}").cpu().numpy())
               for n in ("qkv", "o", "gu", "down")}
        out["down_sign"] = self.down_sign.cpu().numpy()
        return out
