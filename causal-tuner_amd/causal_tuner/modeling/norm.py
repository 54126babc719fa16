"""The decoder's RMSNorm module (interface of the reference's modeling/model.py:38-64).

Device inputs run `kernels.core_cuda.RMS` (HIP kernels); host inputs the plain formula in
fp32, rounded to the input dtype and multiplied by the weight in that dtype.

`forward(x, reuse_grad=True)` marks a pre-norm whose consumer hands back a private input
gradient, which the backward may then overwrite. With a frozen bf16 weight whose every
magnitude lies in [1/256, 256] the function also saves its output instead of its input and
rebuilds the normalized rows from output / weight in the backward: outside that range the
division would magnify rounding. The range check reads the weight, so its verdict is kept
per (storage, version) of the weight and refreshed when either changes; under graph capture
(where the check's host read is not allowed) an unchecked weight is not reconstructed.
"""

import torch
from torch import nn

_LOW, _HIGH = 1 / 256, 256


class RMSNorm(nn.Module):
    def __init__(self, size, eps, dtype, device):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(size, dtype=dtype, device=device))
        self.eps = eps
        self._checked = (None, False)   # ((data_ptr, version, dtype), verdict)

    def _weight_key(self, dtype):
        return self.weight.data_ptr(), self.weight._version, dtype

    def _can_reconstruct(self, dtype):
        """True when the backward may rebuild its input from the output (see the module
        docstring for the conditions)."""
        frozen = not self.weight.requires_grad and not torch.is_inference(self.weight)
        if dtype != torch.bfloat16 or not frozen:
            return False
        key = self._weight_key(dtype)
        if self._checked[0] == key:
            return self._checked[1]
        if torch.cuda.is_current_stream_capturing():
            return False
        scale = self.weight.detach().to(dtype).abs()
        verdict = bool(torch.logical_and(scale >= _LOW, scale <= _HIGH).all())
        self._checked = (key, verdict)
        return verdict

    def forward(self, x, *, reuse_grad=False):
        if not x.is_cuda:
            wide = x.float()
            rstd = torch.rsqrt(wide.pow(2).mean(dim=-1, keepdim=True) + self.eps)
            return (wide * rstd).to(x.dtype) * self.weight.to(x.dtype)
        from ..kernels.core_cuda import RMS
        reconstruct = bool(reuse_grad and torch.is_grad_enabled() and self._can_reconstruct(x.dtype))
        return RMS.apply(x, self.weight, self.eps, reuse_grad, reconstruct)
