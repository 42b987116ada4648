"""RMSNorm without gamma (gamma is folded into the next linear offline),
mirroring signrot/nn/normalization.py:7-30."""
import torch

from ..functional import kernel


class RMSNorm(torch.nn.Module):
    """x * rsqrt(sum(x^2) / mean_dim + eps) over the last dim.

    fp16 input runs the fused HIP kernel (fp32 sum, one launch); other dtypes
    use forward_reference, as the reference module does."""

    def __init__(self, mean_dim: int, eps=1e-5):
        super().__init__()
        self.eps = eps
        self.mean_dim = mean_dim

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype == torch.float16:
            return kernel.rmsnorm(x, self.eps, self.mean_dim)
        return self.forward_reference(x)

    def forward_reference(self, x: torch.Tensor) -> torch.Tensor:
        input_dtype = x.dtype
        if x.dtype == torch.float16:
            x = x.to(torch.float32)
        variance = x.pow(2).sum(-1, keepdim=True) / self.mean_dim
        x = x * torch.rsqrt(variance + self.eps)
        return x.to(input_dtype)
