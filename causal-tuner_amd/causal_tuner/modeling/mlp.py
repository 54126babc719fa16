"""The decoder's SwiGLU MLP block of three LoRA projections.

It carries what `kernels.mlp_cuda.tiled_lora_mlp` reads from the reference's MLP
(modeling/model.py:111-139): `gate_proj` and `up_proj` (hidden -> intermediate),
`down_proj` (intermediate -> hidden), the row `tile` and the `cache_intermediates` flag that
the model's cache planner sets. The reference builds it from a model config and runtime;
here the sizes and the runtime fields are constructor arguments.
"""

import torch
from torch import nn
from torch.nn import functional as F

from .lora import Projection


class MLP(nn.Module):
    def __init__(self, hidden_size, intermediate_size, *, rank=0, base_dtype=torch.bfloat16,
                 train_dtype=torch.float32, compute_dtype=torch.bfloat16, device=None, tile=None):
        super().__init__()
        options = {"rank": rank, "base_dtype": base_dtype, "train_dtype": train_dtype,
                   "compute_dtype": compute_dtype, "device": device}
        self.gate_proj = Projection(hidden_size, intermediate_size, **options)
        self.up_proj = Projection(hidden_size, intermediate_size, **options)
        self.down_proj = Projection(intermediate_size, hidden_size, **options)
        self.tile = tile
        self.cache_intermediates = False

    def _projections(self):
        return self.gate_proj, self.up_proj, self.down_proj

    def cache_bytes(self, rows):
        """Device bytes that cache mode keeps for `rows` tokens: the gate and up outputs and
        their xa = x a^T, all in the compute dtype."""
        element = torch.finfo(self.gate_proj.compute_dtype).bits // 8
        per_row = sum(p.lora_B.shape[0] + p.rank for p in (self.gate_proj, self.up_proj))
        return rows * per_row * element

    def untiled(self, x):
        """The block through the projections' own forwards (any device, no fusion)."""
        gate, up = self.gate_proj(x), self.up_proj(x)
        if x.is_cuda:
            from ..kernels.mlp_cuda import silu_multiply
            return self.down_proj(silu_multiply(gate, up))
        return self.down_proj(F.silu(gate) * up)

    def forward(self, x, *, residual=None, tile=None, cache=None):
        from ..kernels.linear import can_fuse
        if all(can_fuse(p, x) for p in self._projections()):
            from ..kernels.mlp_cuda import tiled_lora_mlp
            return tiled_lora_mlp(self, x, residual, tile=tile, cache=cache)
        result = self.untiled(x)
        return result + residual if residual is not None else result
