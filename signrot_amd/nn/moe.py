"""MoE feed-forward block over stacked int4 expert weights, with the
constructor, buffers and outputs of the reference's SignRotMoEBlock
(signrot/nn/moe.py:28-236).

A forward is four steps over the (token, choice) rows of the batch:

  1. routing: softmax router probabilities (fp32), top-k, optional
     renormalisation, weights cast to the input dtype; the rows are ordered
     by expert (a stable sort), giving per-expert row ranges;
  2. gate/up: every token is quantized once -- its k rows and both
     projections read the same codes -- then one grouped W4A4 GEMM with the
     expert-indexed dequant per projection (srq_w4a4_linear_moe);
  3. down: SwiGLU, the had_K ⊗ H rotation (one transform for all rows: it
     does not depend on the expert), the expert's SignRot sign and the
     quantizer -- one fused launch where the rotation has an MFMA form --
     then the grouped down GEMM;
  4. combine: each row goes back to its (token, choice) slot and the k rows
     of a token are summed with their routing weights.

Nothing is read back to the host on the grouped path, so a forward can be
captured in a HIP graph.  `use_grouped=False` runs the gate/up/down GEMMs as
one dense launch per expert over the same rows (the row counts are read on
the host): the reference's per-expert loop, kept as the equivalence check,
bit-identical to the grouped path.  `asym=True` quantizes activations to
uint4 with per-row zero points and the GEMMs subtract zero_row * w_sum before
the dequant, as the reference's matmul_grouped(signed_a=False) +
sym_dequant_moe do.
"""
from typing import NamedTuple, Optional

import torch

from .. import _CUDA
from ..functional import kernel
from ..functional.hadamard import get_hadK, matmul_hadU_cuda


class MoERouting(NamedTuple):
    """Routing of one batch: `logits` [T, E]; `weights` [T, k] in the input
    dtype; row r of the expert-ordered batch is (token, choice) row
    `order[r]` (= token * k + choice), of token `token[r]`, expert
    `expert[r]` (int32); `inv` maps a (token, choice) row to its position;
    the rows of expert e are `offsets[e] : offsets[e + 1]` (int32 [E + 1]);
    `counts` [E]."""
    logits: torch.Tensor
    weights: torch.Tensor
    order: torch.Tensor
    expert: torch.Tensor
    counts: torch.Tensor
    offsets: torch.Tensor
    inv: torch.Tensor
    token: torch.Tensor


class _Codes(NamedTuple):
    q: torch.Tensor                 # packed u8 [rows, K / 2]
    scale: torch.Tensor             # f16 [rows, 1]
    zero: Optional[torch.Tensor]    # int8 [rows, 1] (asymmetric) or None

    def rows(self, index):
        return _Codes(self.q[index], self.scale[index],
                      None if self.zero is None else self.zero[index])


class SignRotMoEBlock(torch.nn.Module):
    """Buffers (non-persistent, as in the reference): w_gate / w_up u8
    [E, inter, hidden/2], w_down u8 [E, hidden, inter/2], s_* f16 [E, out],
    sign_down int8 [E, inter] or None, wsum_* int32 [E, out] (asym; computed
    on first use when not given), had_K [K, K] on the weights' device."""

    def __init__(self, gate, *, top_k, norm_topk_prob,
                 w_gate, s_gate, w_up, s_up, w_down, s_down,
                 sign_down=None, wsum_gate=None, wsum_up=None, wsum_down=None,
                 asym=False, clip_ratio=1.0, fp32_had=False, use_grouped=True):
        super().__init__()
        experts, inter, half_hidden = w_gate.shape
        if tuple(w_up.shape) != (experts, inter, half_hidden) or \
                tuple(w_down.shape) != (experts, 2 * half_hidden, inter // 2):
            raise ValueError("w_gate / w_up must be [E, inter, hidden/2] and w_down "
                             "[E, hidden, inter/2]")
        self.gate = gate
        self.top_k = top_k
        self.norm_topk_prob = norm_topk_prob
        self.asym = asym
        self.clip_ratio = clip_ratio
        self.fp32_had = fp32_had
        self.use_grouped = use_grouped
        # grouped path: swiglu + rotation + sign + quantizer of the down-proj
        # input in one launch where the rotation has an MFMA form
        self.fuse_down = True
        self.num_experts, self.intermediate_size, self.hidden_size = experts, inter, 2 * half_hidden
        for name, t in (("w_gate", w_gate), ("w_up", w_up), ("w_down", w_down),
                        ("s_gate", s_gate), ("s_up", s_up), ("s_down", s_down),
                        ("sign_down", sign_down), ("wsum_gate", wsum_gate),
                        ("wsum_up", wsum_up), ("wsum_down", wsum_down)):
            self.register_buffer(name, t, persistent=False)
        table, self.K = get_hadK(inter)
        if table is not None:
            table = table.to(w_gate.device, torch.float32 if fp32_had else torch.float16)
        self.register_buffer("had_K", table, persistent=False)

    @staticmethod
    def stack_experts(linears, need_wsum=False):
        """(w u8 [E, out, in/2], s f16 [E, out], wsum int32 [E, out] or None)
        from per-expert Linear4bit modules (moe.py:71-78)."""
        first = linears[0].weight
        w = first.new_empty((len(linears), *first.shape))
        s = torch.empty((len(linears), first.shape[0]), dtype=torch.float16, device=first.device)
        for e, lin in enumerate(linears):
            w[e].copy_(lin.weight)
            s[e].copy_(lin.weight_scales.reshape(-1))
        wsum = None
        if need_wsum:
            wsum = kernel.sum_i4(w.view(-1, w.shape[-1])).view(len(linears), -1)
        return w, s, wsum

    # --------------------------------------------------------------- pieces

    def _weights(self, proj):
        """(codes, scales, row sums or None) of one projection; the row sums
        of the asymmetric path are computed once, for all experts in one
        launch."""
        w = getattr(self, "w_" + proj)
        wsum = None
        if self.asym:
            wsum = getattr(self, "wsum_" + proj)
            if wsum is None:
                wsum = kernel.sum_i4(w.view(-1, w.shape[-1])).view(self.num_experts, -1)
                setattr(self, "wsum_" + proj, wsum)
        return w, getattr(self, "s_" + proj), wsum

    def _quant(self, x) -> _Codes:
        if self.asym:
            q, s, z = kernel.asym_quant_dynamic(x, self.clip_ratio)
            return _Codes(q, s, z.to(torch.int8))
        q, s = kernel.sym_quant_dynamic(x, self.clip_ratio)
        return _Codes(q, s, None)

    def _quant_per_expert(self, h, expert) -> _Codes:
        """Quantizer of the down-proj input with row r flipped by
        sign_down[expert[r]] (fused into the quantizer)."""
        if self.asym:
            q, s, z = kernel.asym_quant_dynamic_moe(h, self.sign_down, expert, self.clip_ratio)
            return _Codes(q, s, z.to(torch.int8))
        q, s = kernel.sym_quant_dynamic_moe(h, self.sign_down, expert, self.clip_ratio)
        return _Codes(q, s, None)

    def _project(self, codes: _Codes, route: MoERouting, proj):
        """Expert-ordered rows times their expert's weights, dequantized to
        fp16 [rows, out]."""
        w, s_w, wsum = self._weights(proj)
        if self.use_grouped:
            if codes.zero is None:
                return kernel.w4a4_linear_moe(codes.q, codes.scale, w, s_w, route.offsets)
            return kernel.w4a4_linear_moe_asym(codes.q, codes.scale, codes.zero, w, s_w, wsum,
                                               route.offsets)
        # one dense launch per expert with rows (host-synced on the counts)
        out = torch.empty((codes.q.shape[0], w.shape[1]), dtype=torch.float16,
                          device=codes.q.device)
        bounds = route.offsets.tolist()
        for e in range(self.num_experts):
            lo, hi = bounds[e], bounds[e + 1]
            if lo == hi:
                continue
            part = codes.rows(slice(lo, hi))
            if part.zero is None:
                acc = kernel.matmul_si4_si4(part.q, w[e])
            else:
                acc = kernel.matmul_ui4_si4(part.q, w[e]) - \
                    kernel.matmul_colrow_i8_i32(part.zero, wsum[e].view(1, -1))
            out[lo:hi] = kernel.sym_dequant(acc, part.scale, s_w[e].view(-1, 1))
        return out

    def _down_input(self, gate_h, up_h, route: MoERouting) -> _Codes:
        """SwiGLU -> rotation -> per-expert sign -> quantizer."""
        inter = gate_h.shape[1]
        if (self.fuse_down and self.use_grouped and not self.asym and not self.fp32_had
                and inter == self.K * 512 and _CUDA.swiglu_had_fusable(inter, self.K)):
            q, s = _CUDA.swiglu_had_sign_quant_moe(gate_h, up_h, self.had_K.half(), self.K,
                                                   self.sign_down, route.expert, self.clip_ratio)
            return _Codes(q, s, None)
        h = kernel.swiglu(gate_h, up_h)
        if self.fp32_had:
            h = h.float()
        h = matmul_hadU_cuda(h, self.had_K, self.K).to(torch.float16)
        if self.use_grouped:
            return self._quant_per_expert(h, route.expert)
        if self.sign_down is not None:
            h = h * self.sign_down[route.expert.long()]
        return self._quant(h)

    # -------------------------------------------------------------- forward

    def route(self, x) -> MoERouting:
        """Router probabilities in fp32, top-k (renormalised when
        norm_topk_prob), weights in x's dtype (moe.py:168-185); rows ordered
        by expert, stable.  fp16 logits of at most 64 experts (top_k <= 8):
        one srq_moe_route launch; otherwise the same steps as torch ops (a
        stable sort and a scatter-add for the counts: no host reads)."""
        logits = self.gate(x)
        if (logits.dtype == torch.float16 and logits.is_cuda and self.num_experts <= 64
                and self.top_k <= 8):
            w, order, inv, expert, token, counts, offsets = _CUDA.moe_route(
                logits.contiguous(), self.top_k, self.norm_topk_prob)
            return MoERouting(logits, w.to(x.dtype), order, expert, counts, offsets, inv,
                              token)
        probs = torch.softmax(logits, dim=1, dtype=torch.float)
        top_p, top_e = torch.topk(probs, self.top_k, dim=-1)
        if self.norm_topk_prob:
            top_p /= top_p.sum(dim=-1, keepdim=True)
        choice = top_e.reshape(-1)
        order = torch.argsort(choice, stable=True)
        counts = torch.zeros(self.num_experts, dtype=torch.int32, device=x.device)
        counts.scatter_add_(0, choice, torch.ones_like(choice, dtype=torch.int32))
        offsets = torch.zeros(self.num_experts + 1, dtype=torch.int32, device=x.device)
        torch.cumsum(counts, 0, out=offsets[1:])
        return MoERouting(logits, top_p.to(x.dtype), order, choice[order].to(torch.int32),
                          counts, offsets, torch.argsort(order), order // self.top_k)

    def forward(self, hidden_states: torch.Tensor):
        shape = hidden_states.shape
        x = hidden_states.reshape(-1, shape[-1])
        route = self.route(x)
        xh = x.to(torch.float16)
        if (not self.asym and xh.shape[1] % 8 == 0 and route.token.dtype == torch.int32
                and xh.is_contiguous()):
            # quantize the expert-sorted rows straight from their tokens
            codes = _Codes(*_CUDA.sym_quant_dynamic_rows(xh, route.token, self.clip_ratio), None)
        else:
            codes = self._quant(xh).rows(route.token)
        if self._swiglu_epilogue(codes):
            # SwiGLU in the gate/up launch's epilogue, then the plain
            # rotation + per-expert sign + quantizer (bit-identical)
            w_il, s_il = self._gate_up_interleaved()
            a = _CUDA.w4a4_linear_moe_swiglu(codes.q, codes.scale, w_il, s_il, route.offsets)
            q, s = _CUDA.had_sign_quant_moe(a, self.had_K, self.K, self.sign_down, route.expert,
                                            self.clip_ratio)
            y = self._project(_Codes(q, s, None), route, "down")
            return self._combine(x, shape, y, route)
        if self.use_grouped and codes.zero is None:
            # both projections in one launch (bit-identical to two)
            gate_h, up_h = _CUDA.w4a4_linear_moe_gate_up(
                codes.q, codes.scale, self.w_gate, self.s_gate, self.w_up, self.s_up,
                route.offsets)
        else:
            gate_h = self._project(codes, route, "gate")
            up_h = self._project(codes, route, "up")
        y = self._project(self._down_input(gate_h, up_h, route), route, "down")
        return self._combine(x, shape, y, route)

    def _swiglu_epilogue(self, codes: _Codes) -> bool:
        """Whether the gate/up launch can end in the SwiGLU: grouped,
        symmetric, fp16 rotation with an MFMA form for this size."""
        inter, K = self.intermediate_size, self.K
        return (self.fuse_down and self.use_grouped and codes.zero is None and not self.fp32_had
                and self.had_K is not None and inter % 8 == 0 and K % 4 == 0 and 9 <= K <= 32
                and inter in (K * 512, K * 1024))

    def _gate_up_interleaved(self):
        """w_gate / w_up (and scales) as one [E, 2 inter, hidden/2] tensor in
        the blocks-of-8 layout of w4a4_linear_moe_swiglu: a derived copy,
        made on first use and again whenever a source buffer changes in
        place."""
        src = (self.w_gate, self.s_gate, self.w_up, self.s_up)
        key = tuple((t.data_ptr(), t._version) for t in src)
        if getattr(self, "_gu_il_key", None) != key:
            self._gu_il = _CUDA.interleave_gate_up_experts(*src)
            self._gu_il_key = key
        return self._gu_il

    def _combine(self, x, shape, y, route: MoERouting):
        """Expert-ordered rows y back to tokens, weighted and summed over
        each token's k choices."""
        if x.dtype == torch.float16 and shape[-1] % 8 == 0:
            # un-permute, weight and sum in one launch (bit-identical)
            out = _CUDA.moe_combine(y, route.inv.to(torch.int32), route.weights)
            return out.view(shape), route.logits
        # back to (token, choice) order by a scatter through the permutation
        # (no atomics: a replayed graph gives the same bits), then the
        # weighted sum over each token's k choices
        slots = torch.empty_like(y, dtype=x.dtype)
        slots[route.order] = y.to(x.dtype)
        slots = slots.view(x.shape[0], self.top_k, shape[-1])
        out = (slots * route.weights.unsqueeze(-1)).sum(dim=1)
        return out.view(shape), route.logits
