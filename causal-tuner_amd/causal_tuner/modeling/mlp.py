"""The LoRA MLP block's projections, as the reference's MLP holds them (modeling/model.py:111-139).

`tiled_lora_mlp` (kernels/mlp_cuda.py) reads `gate_proj`, `up_proj`, `down_proj`, `tile`
and `cache_intermediates` from its module; this class carries exactly those, with the
reference's projection shapes (hidden -> intermediate twice, intermediate -> hidden) and
forward dispatch. The reference builds it from its model config and runtime; here the
fields it reads are arguments.
"""

import torch
from torch import nn
from torch.nn import functional as F

from .lora import Projection


class MLP(nn.Module):
    def __init__(self, hidden_size, intermediate_size, *, rank=0, base_dtype=torch.bfloat16,
                 train_dtype=torch.float32, compute_dtype=torch.bfloat16, device=None, tile=None):
        super().__init__()
        self.tile = tile
        self.cache_intermediates = False
        kwargs = dict(rank=rank, base_dtype=base_dtype, train_dtype=train_dtype, compute_dtype=compute_dtype,
                      device=device)
        self.gate_proj = Projection(hidden_size, intermediate_size, **kwargs)
        self.up_proj = Projection(hidden_size, intermediate_size, **kwargs)
        self.down_proj = Projection(intermediate_size, hidden_size, **kwargs)

    def cache_bytes(self, rows):
        """Bytes that cache mode retains for `rows` tokens (gate, up and their xa)."""
        size = torch.empty((), dtype=self.gate_proj.compute_dtype).element_size()
        return rows*size*sum(projection.lora_B.shape[0]+projection.rank
                             for projection in (self.gate_proj, self.up_proj))

    def untiled(self, x):
        if x.is_cuda:
            from ..kernels.mlp_cuda import silu_multiply
            return self.down_proj(silu_multiply(self.gate_proj(x), self.up_proj(x)))
        return self.down_proj(F.silu(self.gate_proj(x))*self.up_proj(x))

    def forward(self, x, *, residual=None, tile=None, cache=None):
        from ..kernels.linear import can_fuse
        if all(can_fuse(module, x) for module in (self.gate_proj, self.up_proj, self.down_proj)):
            from ..kernels.mlp_cuda import tiled_lora_mlp
            return tiled_lora_mlp(self, x, residual, tile=tile, cache=cache)
        output = self.untiled(x)
        return output if residual is None else output+residual
