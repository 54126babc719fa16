"""The MQA decoder that calls the projection path, as the reference's model lays it out
(modeling/model.py:68-165: Attention, MLP, Layer, Decoder, the causal LM's head), reduced
to what one training step of packed records needs.

Every projection is a `Projection` with a frozen NF4 base and a unit-scale LoRA adapter,
driven through the reference's group operators: q/k/v share their input in
`project_group` with the partial RoPE applied to q and k (`rotary=`), o_proj adds the
residual, the MLP is `tiled_lora_mlp` with the residual; RMSNorm runs the HIP kernels,
and the loss is `projection_loss` over the supervised rows. Attention is PyTorch-ROCm's
scaled-dot-product attention (memory-efficient backend, flash as the deterministic
choice), causal within each packed record, with the
single key/value head broadcast to the query heads. The MLP cache budget
(`mlp_cache_bytes`) is the reference's runtime option: layers from the last one back keep
their gate/up outputs and xa while the budget lasts (modeling/model.py:227-237), so their
backward skips the gate/up recompute. Not here (the reference's other runtime options):
gradient checkpointing, activation offload, the attention cache, trainable embeddings or
head, tied weights.
"""

from dataclasses import dataclass

import torch
from torch import nn
from torch.nn import functional as F

from .lora import Projection
from .mlp import MLP
from .norm import RMSNorm


@dataclass
class DecoderConfig:
    hidden_size: int = 2048
    num_attention_heads: int = 16
    head_dim: int = 128
    intermediate_size: int = 8192
    num_hidden_layers: int = 24
    vocab_size: int = 49152
    rope_theta: float = 10000.0
    partial_rotary_factor: float = 0.5
    rms_norm_eps: float = 1e-6

    @property
    def rotary_dim(self):
        return int(self.head_dim * self.partial_rotary_factor)


def record_positions(records, device):
    """Token positions restarting at every packed record: records are (start, stop) spans
    covering the sequence in order."""
    return torch.cat([torch.arange(stop - start, device=device) for start, stop in records])


def rotary_values(positions, config, dtype):
    """cosine, sine [tokens, rotary_dim / 2] of positions * theta^(-2i / rotary_dim), as the
    reference's rotary_values (modeling/rotary.py:6-13), rounded to the compute dtype."""
    channel = torch.arange(0, config.rotary_dim, 2, device=positions.device, dtype=torch.float32)
    inverse = 1.0 / (config.rope_theta ** (channel / config.rotary_dim))
    angle = positions.float()[..., None] * inverse
    return angle.cos().to(dtype), angle.sin().to(dtype)


# PyTorch-ROCm's SDPA backends to use, first choice first. Measured on MI355X (one record
# of 2665 tokens, 16 query heads, head 128, bf16, forward + backward): memory-efficient
# 0.48 ms, flash 0.70 ms, flash with enable_gqa (no key/value expansion) 2.1 ms. The
# memory-efficient backward does not repeat bit for bit from run to run; flash does, so it
# goes first under torch.use_deterministic_algorithms(True).
ATTENTION_BACKENDS = ("EFFICIENT_ATTENTION", "FLASH_ATTENTION")


def attention_backends():
    names = tuple(ATTENTION_BACKENDS)
    if torch.are_deterministic_algorithms_enabled() and "FLASH_ATTENTION" in names:
        names = ("FLASH_ATTENTION",) + tuple(n for n in names if n != "FLASH_ATTENTION")
    return names


def _attention(q, k, v, records):
    """Causal attention inside each record. q [1, S, H, D]; k, v [1, S, 1, D]."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    heads = q.shape[2]
    sizes = [stop - start for start, stop in records]
    if sum(sizes) != q.shape[1]:
        raise ValueError("records must cover the sequence")
    outputs = []
    # One split per tensor: its backward concatenates the records' gradients in one
    # launch (a slice per record would fill and add a full-size gradient each).
    # Only the fused backends, in attention_backends() order: never the math fallback.
    with sdpa_kernel([getattr(SDPBackend, name) for name in attention_backends()], set_priority=True):
        for qs, ks, vs in zip(q.split(sizes, dim=1), k.split(sizes, dim=1), v.split(sizes, dim=1)):
            qs = qs.transpose(1, 2)
            ks = ks.transpose(1, 2).expand(-1, heads, -1, -1)
            vs = vs.transpose(1, 2).expand(-1, heads, -1, -1)
            outputs.append(F.scaled_dot_product_attention(qs, ks, vs, is_causal=True).transpose(1, 2))
    return torch.cat(outputs, dim=1)


class Attention(nn.Module):
    def __init__(self, config, *, rank, device=None):
        super().__init__()
        self.config = config
        h, d = config.hidden_size, config.head_dim
        self.q_proj = Projection(h, config.num_attention_heads * d, bias=True, rank=rank, device=device)
        self.k_proj = Projection(h, d, bias=True, rank=rank, device=device)
        self.v_proj = Projection(h, d, bias=True, rank=rank, device=device)
        self.o_proj = Projection(config.num_attention_heads * d, h, rank=rank, device=device)

    def forward(self, x, cosine, sine, records, *, residual=None):
        from ..kernels.linear import project_group
        b, s, _ = x.shape
        c = self.config
        q, k, v = project_group((self.q_proj, self.k_proj, self.v_proj), x, rotary=(cosine, sine, c.head_dim))
        q = q.reshape(b, s, c.num_attention_heads, c.head_dim)
        k, v = k.reshape(b, s, 1, c.head_dim), v.reshape(b, s, 1, c.head_dim)
        y = _attention(q, k, v, records).reshape(b, s, -1)
        return project_group((self.o_proj,), y, residual=residual)[0]


class Layer(nn.Module):
    def __init__(self, config, *, rank, device=None):
        super().__init__()
        self.self_attn = Attention(config, rank=rank, device=device)
        self.mlp = MLP(config.hidden_size, config.intermediate_size, rank=rank, device=device)
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps, torch.bfloat16, device)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps, torch.bfloat16, device)
        for norm in (self.input_layernorm, self.post_attention_layernorm):
            norm.weight.requires_grad_(False)

    def forward(self, x, cosine, sine, records):
        from ..kernels.mlp_cuda import tiled_lora_mlp
        x = self.self_attn(self.input_layernorm(x, reuse_grad=True), cosine, sine, records, residual=x)
        return tiled_lora_mlp(self.mlp, self.post_attention_layernorm(x, reuse_grad=True), x)


class Decoder(nn.Module):
    """Embedding, layers, final norm and a frozen head; `loss` returns the weighted CE sum."""

    def __init__(self, config, *, rank, device=None):
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size, dtype=torch.bfloat16, device=device)
        self.layers = nn.ModuleList([Layer(config, rank=rank, device=device)
                                     for _ in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps, torch.bfloat16, device)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False, dtype=torch.bfloat16,
                                 device=device)
        for name, parameter in self.named_parameters():
            parameter.requires_grad_("lora_" in name)

    def install_nf4(self):
        """Quantize every projection's base weight to NF4 on the device (install_nf4)."""
        for module in self.modules():
            if isinstance(module, Projection) and module.weight is not None:
                module.install_nf4(module.weight, module.weight.device)

    def plan_mlp_cache(self, rows, budget):
        """Cache mode per layer, from the last layer back while `budget` bytes last
        (modeling/model.py:227-237); returns the bytes retained."""
        remaining, retained = budget if torch.is_grad_enabled() else 0, 0
        for layer in reversed(self.layers):
            cost = layer.mlp.cache_bytes(rows) if remaining else 0
            layer.mlp.cache_intermediates = bool(cost and cost <= remaining)
            if layer.mlp.cache_intermediates:
                remaining -= cost
                retained += cost
        return retained

    def hidden(self, ids, records, *, mlp_cache_bytes=0, projection_bytes=0):
        """Final hidden states. `projection_bytes` is the per-group projection budget
        (kernels.linear.projection_budget): 0 keeps the reference's 4096-row tiles and
        saved tensors, a budget that covers a group's rows keeps its forward xa."""
        from ..kernels.linear import projection_budget
        positions = record_positions(records, ids.device)
        cosine, sine = rotary_values(positions, self.config, torch.bfloat16)
        x = self.embed_tokens(ids)
        self.plan_mlp_cache(ids.numel() if ids.is_cuda else 0, mlp_cache_bytes)
        with projection_budget(projection_bytes):
            for layer in self.layers:
                x = layer(x, cosine, sine, records)
        return self.norm(x)

    def loss(self, ids, targets, weights, records, *, token_budget=128, mlp_cache_bytes=0, projection_bytes=0):
        from ..kernels.loss import projection_loss
        hidden = self.hidden(ids, records, mlp_cache_bytes=mlp_cache_bytes, projection_bytes=projection_bytes)
        return projection_loss(hidden, self.lm_head.weight, targets, weights, token_budget=token_budget)
