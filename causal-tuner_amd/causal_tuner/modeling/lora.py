"""Independent projections with unit-scale LoRA and optional frozen NF4 (reference modeling/lora.py:9-62).

Module layout, initialisation and error behaviour follow the reference: `weight [out, in]`
in `base_dtype` (frozen when rank > 0), optional frozen `bias [out]`, fp32
`lora_A [rank, in]` ~ U(+-sqrt(6/in)) and `lora_B [out, rank]` = 0, unit scaling.
`install_nf4` replaces `weight` by a `quantized` holder whose `.weight` is the packed
uint8 tensor carrying `.quant_state`, as bitsandbytes' Linear4bit/Params4bit expose it
(the operator layer reads exactly `quantized.weight` and `weight.quant_state`).
"""

import math

import torch
from torch import nn
from torch.nn import functional as F

from ..quant.nf4 import quantize_nf4


class NF4Linear(nn.Module):
    """Frozen NF4 base weight: `weight` (uint8 Parameter) with `weight.quant_state`."""

    def __init__(self, packed, state, compute_dtype):
        super().__init__()
        self.weight = nn.Parameter(packed, requires_grad=False)
        self.weight.quant_state = state
        self.compute_dtype = compute_dtype

    def forward(self, x):
        from ..kernels.linear import materialize
        return F.linear(x, materialize(self.weight, self.weight.quant_state, x.dtype))


class Projection(nn.Module):
    def __init__(self, inputs, outputs, *, bias=False, rank=0, base_dtype=torch.bfloat16,
                 train_dtype=torch.float32, compute_dtype=torch.bfloat16, device=None):
        super().__init__()
        self.compute_dtype, self.rank = compute_dtype, rank
        self.weight = nn.Parameter(torch.empty(outputs, inputs, dtype=base_dtype, device=device),
                                   requires_grad=not rank)
        self.bias = nn.Parameter(torch.zeros(outputs, dtype=base_dtype, device=device),
                                 requires_grad=not rank) if bias else None
        self.quantized = None
        if rank:
            self.lora_A = nn.Parameter(torch.empty(rank, inputs, dtype=train_dtype, device=device))
            self.lora_B = nn.Parameter(torch.zeros(outputs, rank, dtype=train_dtype, device=device))
            nn.init.uniform_(self.lora_A, -math.sqrt(6/inputs), math.sqrt(6/inputs))
        nn.init.normal_(self.weight, std=0.02)

    def forward(self, x):
        from ..kernels.linear import can_fuse, project_group
        if can_fuse(self, x):
            return project_group((self,), x)[0]
        x = x.to(self.compute_dtype)
        if self.quantized is not None:
            output = self.quantized(x)
            if self.bias is not None:
                output = output + self.bias.to(x.dtype)
        else:
            output = F.linear(x, self.weight.to(x.dtype), None if self.bias is None else self.bias.to(x.dtype))
        if self.rank:
            output = output + F.linear(F.linear(x, self.lora_A.to(x.dtype)), self.lora_B.to(x.dtype))
        return output

    def install_nf4(self, weight, device):
        if not self.rank or weight.requires_grad:
            raise ValueError("NF4 is restricted to frozen adapter base projections")
        if torch.device(device).type != "cuda":
            raise ValueError("NF4 requires a CUDA device")
        packed, state = quantize_nf4(weight.detach().to(device), blocksize=64, compress_statistics=True)
        self.quantized = NF4Linear(packed, state, self.compute_dtype)
        self.register_parameter("weight", None)

    def base_weight(self):
        if self.quantized is None:
            return self.weight
        from ..kernels.nf4_cuda import dequantize_nf4
        state = self.quantized.weight.quant_state
        return dequantize_nf4(self.quantized.weight.data, state, state.dtype)

    def merged_weight(self, dtype=None):
        """The tensor the reference's merged export writes for this projection
        (checkpointing/io.py:270-280): the base weight (NF4 decoded by ct_nf4_dequant) plus
        lora_B @ lora_A, summed in fp32 and rounded once to `dtype` (default: the base
        weight's dtype)."""
        with torch.no_grad():
            weight = self.base_weight()
            dtype = dtype or weight.dtype
            if self.rank:
                weight = weight.float() + self.lora_B.float() @ self.lora_A.float()
            return weight.detach().to(dtype).contiguous()
