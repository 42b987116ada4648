"""W4 linear module (signrot/nn/linear.py:8-73)."""
import torch

from ..functional import quantization as quant_utils
from ..functional import kernel


class Linear4bit(torch.nn.Module):
    """Symmetric 4-bit linear layer.

    Buffers (same names, shapes and dtypes as the reference, so checkpoints
    load unchanged): weight u8 [out, in/2] packed int4, weight_scales
    [out, 1], optional fp16 bias [out].

    forward(PackedQuantizedTensor) runs the fused int4 GEMM + per-token x
    per-channel dequant (+ bias) kernel in one launch; it is bit-identical to
    the reference's matmul_si4_si4 -> sym_dequant (-> + bias) chain.  With
    asymmetric activations (zeros_x set: uint4 codes) the fused kernel also
    subtracts zeros_x ⊗ weight_sum from the int32 product, as the reference's
    matmul_ui4_si4 -> matmul_colrow_i8_i32 -> `x -= zeros` -> sym_dequant
    chain does (linear.py:35-50); weight_sum = sum_i4(weight) is computed on
    the first such call and kept as a non-persistent buffer.
    forward(fp16 tensor) dequantizes the weight and calls F.linear, as the
    reference does (linear.py:31-34).
    """

    weight: torch.Tensor
    weight_scales: torch.Tensor
    bias: torch.Tensor | None

    def __init__(self, in_features, out_features, bias=False, dtype=torch.float16):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer("weight_scales",
                             torch.zeros((self.out_features, 1), requires_grad=False))
        self.register_buffer("weight", torch.ones((self.out_features, self.in_features // 2),
                                                  dtype=torch.uint8, requires_grad=False))
        if bias:
            self.register_buffer("bias", torch.zeros((self.out_features), dtype=dtype))
        else:
            self.bias = None

    def forward(self, x):
        if not isinstance(x, kernel.PackedQuantizedTensor):
            w_deq = quant_utils.sym_dequant(quant_utils.unpack_i4(self.weight), self.weight_scales)
            return torch.nn.functional.linear(x, w_deq, self.bias)
        q, s = x.quantized_x, x.scales_x
        assert q.shape[-1] * 2 % 32 == 0, "K: {} must be a multiple of 32".format(q.shape[-1] * 2)
        if x.zeros_x is not None:
            if not hasattr(self, "weight_sum"):
                self.register_buffer("weight_sum", kernel.sum_i4(self.weight), persistent=False)
            return kernel.w4a4_linear_asym(q, s, x.zeros_x, self.weight, self._scales_f16(),
                                           self.weight_sum, self.bias)
        return kernel.w4a4_linear(q, s, self.weight, self._scales_f16(), self.bias)

    def _scales_f16(self):
        s = self.weight_scales
        if s.dtype != torch.float16:
            s = s.to(torch.float16)
        return s.reshape(-1)

    @staticmethod
    def from_float(module: torch.nn.Linear, weight_scales=None):
        """Build from an fp16 Linear whose weight is already on the int4 grid
        of `weight_scales` (linear.py:52-73): codes = round(W / s) in W's
        dtype, packed."""
        weight_matrix = module.weight.data
        int_module = Linear4bit(module.in_features, module.out_features,
                                bias=module.bias is not None,
                                dtype=weight_matrix.dtype).to(weight_matrix.dtype)
        if weight_scales is not None:
            assert weight_scales.shape == (module.out_features, 1), \
                "weight_scales should have shape (out_features, 1)"
            dev = weight_matrix.device
            int_module.weight_scales.copy_(weight_scales.to(weight_matrix.dtype))
            int_rounded_weight = (weight_matrix / weight_scales.to(dev)).round()
            int_module.weight.copy_(quant_utils.pack_i4(int_rounded_weight.to(torch.int8)).cpu())
            if module.bias is not None:
                int_module.bias.copy_(module.bias)
        return int_module


class AsymSymmLinear4bit(torch.nn.Module):
    """Asymmetric-activation, symmetric-weight 4-bit linear (linear.py:76-135):
    the activation codes are int4 (asym_quant_f16_si4), and forward is
    sym_dequant(matmul_si4_si4(x, W) - zeros_x ⊗ weight_sum) (+ bias), the
    reference's op sequence.  weight_sum is registered as int32 [out, 1]: the
    reference registers it as uint8, which its own matmul_colrow_i8_i32 call
    rejects."""

    weight: torch.Tensor
    weight_scales: torch.Tensor
    weight_sum: torch.Tensor
    bias: torch.Tensor | None

    def __init__(self, in_features, out_features, bias=False, dtype=torch.float16):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer("weight", torch.ones((self.out_features, self.in_features // 2),
                                                  dtype=torch.uint8, requires_grad=False))
        self.register_buffer("weight_scales",
                             torch.zeros((self.out_features, 1), requires_grad=False))
        self.register_buffer("weight_sum", torch.ones((self.out_features, 1), dtype=torch.int32,
                                                      requires_grad=False))
        if bias:
            self.register_buffer("bias", torch.zeros((self.out_features), dtype=dtype))
        else:
            self.bias = None

    def forward(self, x):
        assert isinstance(x, kernel.PackedQuantizedTensor)
        q, scales_x, zeros_x = x.quantized_x, x.scales_x, x.zeros_x
        c = kernel.matmul_si4_si4(q, self.weight)
        zeros = kernel.matmul_colrow_i8_i32(zeros_x, self.weight_sum.mT.contiguous())
        s_w = self.weight_scales
        if s_w.dtype != torch.float16:
            s_w = s_w.to(torch.float16)
        out = kernel.sym_dequant(c - zeros, scales_x, s_w.reshape(-1))
        if self.bias is not None:
            out += self.bias
        return out

    @staticmethod
    def from_float(module: torch.nn.Linear, weight_scales=None):
        """As Linear4bit.from_float, plus weight_sum = sum_i4 of the packed
        codes (linear.py:113-135)."""
        weight_matrix = module.weight.data
        int_module = AsymSymmLinear4bit(module.in_features, module.out_features,
                                        bias=module.bias is not None,
                                        dtype=weight_matrix.dtype).to(weight_matrix.dtype)
        int_module.weight_sum = int_module.weight_sum.to(torch.int32)
        if weight_scales is not None:
            assert weight_scales.shape == (module.out_features, 1), \
                "weight_scales should have shape (out_features, 1)"
            dev = weight_matrix.device
            int_module.weight_scales.copy_(weight_scales.to(weight_matrix.dtype))
            int_rounded_weight = (weight_matrix / weight_scales.to(dev)).round()
            packed = quant_utils.pack_i4(int_rounded_weight.to(torch.int8))
            int_module.weight.copy_(packed.cpu())
            int_module.weight_sum.copy_(kernel.sum_i4(packed.to(dev)).cpu())
            if module.bias is not None:
                int_module.bias.copy_(module.bias)
        return int_module
