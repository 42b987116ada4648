"""MoE block over stacked int4 expert weights (signrot/nn/moe.py:28-236).

Same constructor, buffers and forward as the reference's SignRotMoEBlock:

  router -> permute the (token, choice) rows by expert -> quantize each
  token once (its top-k experts and gate/up read the same codes) -> grouped
  gate/up W4A4 linears -> swiglu -> one online Hadamard over all rows (the
  transform is expert-independent) -> per-expert SignRot sign fused into the
  down-proj quantizer -> grouped down W4A4 linear -> weighted un-permute.

Every routing step is a fixed-shape device op (argsort / index_add_ /
cumsum), nothing is read back to the host on the grouped path, so a forward
is graph-capturable.  The grouped path runs each projection as one launch of
the fused grouped GEMM + expert-indexed dequant (srq_w4a4_linear_moe); the
reference runs matmul_grouped then sym_dequant_moe, which is the same
arithmetic.  `use_grouped=False` is the reference's per-expert loop over the
dense kernels (host-synced; the equivalence oracle), bit-identical to the
grouped path.  asym=True quantizes activations to uint4 with per-token zero
points (asym_quant_dynamic / asym_quant_dynamic_moe) and the grouped GEMM
subtracts zero_row * w_sum before the dequant (srq_w4a4_linear_moe_asym),
the reference's matmul_grouped(signed_a=False) + sym_dequant_moe arithmetic.
"""
import torch

from .. import _CUDA
from ..functional import kernel
from ..functional.hadamard import get_hadK, matmul_hadU_cuda


class SignRotMoEBlock(torch.nn.Module):
    def __init__(self, gate, *, top_k, norm_topk_prob,
                 w_gate, s_gate, w_up, s_up, w_down, s_down,
                 sign_down=None, wsum_gate=None, wsum_up=None, wsum_down=None,
                 asym=False, clip_ratio=1.0, fp32_had=False, use_grouped=True):
        super().__init__()
        self.gate = gate  # router linear (16-bit activations), left untouched
        # grouped path: one launch for swiglu + rotation + sign + quantizer
        # of the down-proj input where the rotation has an MFMA form
        self.fuse_down = True
        self.top_k = top_k
        self.norm_topk_prob = norm_topk_prob
        self.asym = asym
        self.clip_ratio = clip_ratio
        self.fp32_had = fp32_had
        self.use_grouped = use_grouped

        self.num_experts, self.intermediate_size = w_gate.shape[0], w_gate.shape[1]
        self.hidden_size = w_gate.shape[2] * 2
        assert w_down.shape == (self.num_experts, self.hidden_size, self.intermediate_size // 2)

        self.register_buffer("w_gate", w_gate, persistent=False)
        self.register_buffer("w_up", w_up, persistent=False)
        self.register_buffer("w_down", w_down, persistent=False)
        self.register_buffer("s_gate", s_gate, persistent=False)
        self.register_buffer("s_up", s_up, persistent=False)
        self.register_buffer("s_down", s_down, persistent=False)
        self.register_buffer("sign_down", sign_down, persistent=False)
        self.register_buffer("wsum_gate", wsum_gate, persistent=False)
        self.register_buffer("wsum_up", wsum_up, persistent=False)
        self.register_buffer("wsum_down", wsum_down, persistent=False)

        had_K, self.K = get_hadK(self.intermediate_size)
        if had_K is not None:
            # on the weights' device, so a forward never uploads it again
            had_K = had_K.to(w_gate.device, torch.float32 if fp32_had else torch.float16)
        self.register_buffer("had_K", had_K, persistent=False)

    @staticmethod
    def stack_experts(linears, need_wsum=False):
        """Stack per-expert Linear4bit weights [E, out, in/2], fp16 scales
        [E, out] and, for the asymmetric path, the int4 row sums [E, out]
        (moe.py:71-78)."""
        w = torch.stack([m.weight for m in linears])
        s = torch.stack([m.weight_scales.view(-1).to(torch.float16) for m in linears])
        wsum = None
        if need_wsum:
            wsum = torch.stack([kernel.sum_i4(m.weight).view(-1) for m in linears])
        return w.contiguous(), s.contiguous(), wsum

    def _ensure_wsum(self):
        """Row sums of every expert's weight codes for the zero correction
        (moe.py:80-86), computed once when the block was built without them."""
        if not self.asym or self.wsum_gate is not None:
            return
        e = self.num_experts
        self.wsum_gate = kernel.sum_i4(self.w_gate).view(e, -1)
        self.wsum_up = kernel.sum_i4(self.w_up).view(e, -1)
        self.wsum_down = kernel.sum_i4(self.w_down).view(e, -1)

    def _quantize(self, x):
        """(codes, scales, zeros int8 or None) (moe.py:88-93)."""
        if self.asym:
            q, s, z = kernel.asym_quant_dynamic(x, self.clip_ratio)
            return q, s, z.to(torch.int8)
        q, s = kernel.sym_quant_dynamic(x, self.clip_ratio)
        return q, s, None

    # ------------------------------------------------------------ projections

    @staticmethod
    def _gemm_dequant_grouped(q, s, z, offsets, w, s_w, wsum):
        if z is None:
            return kernel.w4a4_linear_moe(q, s, w, s_w, offsets)
        return kernel.w4a4_linear_moe_asym(q, s, z, w, s_w, wsum, offsets)

    @staticmethod
    def _gemm_dequant_loop(q, s, z, counts, w, s_w, wsum):
        """Per-expert loop over the dense kernels (moe.py:138-159); host-syncs
        on counts."""
        out = torch.empty(q.shape[0], w.shape[1], dtype=torch.float16, device=q.device)
        row = 0
        for e, m in enumerate(counts.tolist()):
            if m == 0:
                continue
            rows = slice(row, row + m)
            row += m
            if z is not None:
                i32 = kernel.matmul_ui4_si4(q[rows], w[e])
                i32 -= kernel.matmul_colrow_i8_i32(z[rows], wsum[e].view(1, -1))
            else:
                i32 = kernel.matmul_si4_si4(q[rows], w[e])
            out[rows] = kernel.sym_dequant(i32, s[rows], s_w[e].view(-1, 1))
        return out

    # ---------------------------------------------------------------- forward

    def route(self, x):
        """Router logits, top-k weights (in x's dtype) and the expert-sorted
        row order (moe.py:168-185)."""
        router_logits = self.gate(x)
        routing_weights = torch.softmax(router_logits, dim=1, dtype=torch.float)
        routing_weights, selected = torch.topk(routing_weights, self.top_k, dim=-1)
        if self.norm_topk_prob:
            routing_weights /= routing_weights.sum(dim=-1, keepdim=True)
        routing_weights = routing_weights.to(x.dtype)
        flat_e = selected.reshape(-1)
        perm = torch.argsort(flat_e, stable=True)
        counts = torch.zeros(self.num_experts, dtype=torch.int32, device=x.device)
        counts.index_add_(0, flat_e, torch.ones_like(flat_e, dtype=torch.int32))
        return router_logits, routing_weights, perm, counts, flat_e

    def forward(self, hidden_states: torch.Tensor):
        batch_size, seq_len, hidden_dim = hidden_states.shape
        x = hidden_states.view(-1, hidden_dim)
        x_dtype = x.dtype
        self._ensure_wsum()
        router_logits, routing_weights, perm, counts, flat_e = self.route(x)
        tok = perm // self.top_k
        eid = flat_e[perm].to(torch.int32)

        # each token's top-k experts and gate/up projections read the same
        # codes: quantize once per token, then gather rows
        q_tok, s_tok, z_tok = self._quantize(x.to(torch.float16))
        q_a, s_a = q_tok[tok], s_tok[tok]
        z_a = z_tok[tok] if z_tok is not None else None

        if self.use_grouped:
            offsets = torch.zeros(self.num_experts + 1, dtype=torch.int32, device=x.device)
            offsets[1:] = torch.cumsum(counts, 0)
            gate_h = self._gemm_dequant_grouped(q_a, s_a, z_a, offsets, self.w_gate, self.s_gate,
                                                self.wsum_gate)
            up_h = self._gemm_dequant_grouped(q_a, s_a, z_a, offsets, self.w_up, self.s_up,
                                              self.wsum_up)
        else:
            gate_h = self._gemm_dequant_loop(q_a, s_a, z_a, counts, self.w_gate, self.s_gate,
                                             self.wsum_gate)
            up_h = self._gemm_dequant_loop(q_a, s_a, z_a, counts, self.w_up, self.s_up,
                                           self.wsum_up)

        if self.fuse_down and self.use_grouped and not self.asym and not self.fp32_had and \
                _CUDA.swiglu_had_fusable(gate_h.shape[1], self.K) and gate_h.shape[1] == \
                self.K * 512:
            # swiglu, rotation, per-expert sign and quantizer in one launch
            # (bit-identical to the three steps below)
            q_d, s_d = _CUDA.swiglu_had_sign_quant_moe(gate_h, up_h, self.had_K.half(), self.K,
                                                       self.sign_down, eid, self.clip_ratio)
            y = self._gemm_dequant_grouped(q_d, s_d, None, offsets, self.w_down, self.s_down,
                                           None)
        else:
            inter = kernel.swiglu(gate_h, up_h)
            # the Hadamard is identical for every expert; the had_adj sign is
            # per row, from the [E, inter] table
            h = inter.float() if self.fp32_had else inter
            h = matmul_hadU_cuda(h, self.had_K, self.K).to(torch.float16)
            if self.use_grouped:
                if self.asym:
                    q_d, s_d, z_d = kernel.asym_quant_dynamic_moe(h, self.sign_down, eid,
                                                                  self.clip_ratio)
                    z_d = z_d.to(torch.int8)
                else:
                    q_d, s_d = kernel.sym_quant_dynamic_moe(h, self.sign_down, eid,
                                                            self.clip_ratio)
                    z_d = None
                y = self._gemm_dequant_grouped(q_d, s_d, z_d, offsets, self.w_down, self.s_down,
                                               self.wsum_down)
            else:
                if self.sign_down is not None:
                    h = h * self.sign_down[eid.long()]
                q_d, s_d, z_d = self._quantize(h)
                y = self._gemm_dequant_loop(q_d, s_d, z_d, counts, self.w_down, self.s_down,
                                            self.wsum_down)

        # deterministic un-permute + weighted sum (no atomics: a captured
        # graph replays bit-identically)
        inv = torch.argsort(perm)
        y = y.to(x_dtype)[inv].view(-1, self.top_k, hidden_dim)
        out = (y * routing_weights.unsqueeze(-1)).sum(dim=1)
        return out.view(batch_size, seq_len, hidden_dim), router_logits
