"""The decoder step that drives the projection path (modeling/decoder.py; reference
modeling/model.py:68-165): a two-layer MQA decoder with NF4 bases, rank-8 LoRA on all seven
projections, partial RoPE, three packed records and the projection loss, against the same
model written out in float32 torch on the host (dequantized bases, per-record causal
softmax attention, per-token CE). Loss within 2e-2 relative; every LoRA gradient within
5e-2 in relative Frobenius norm (bf16 activations against fp32); one FusedAdamW step
lowers the loss."""

import math

import pytest
import torch
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

pytestmark = pytest.mark.gpu


def _tiny():
    from causal_tuner.modeling.decoder import Decoder, DecoderConfig
    config = DecoderConfig(hidden_size=128, num_attention_heads=2, head_dim=64, intermediate_size=256,
                           num_hidden_layers=2, vocab_size=300)
    torch.manual_seed(5)
    model = Decoder(config, rank=8, device="cuda")
    for name, p in model.named_parameters():
        if "lora_B" in name:
            torch.nn.init.normal_(p, std=0.1)
    model.install_nf4()
    return model


def _host_loss(model, ids, targets, weights, records, device="cpu", dtype=torch.float32):
    """The model restated in plain torch on `device` (the host by default) with activations
    in `dtype` (float32 by default; the LoRA leaves are float32 masters cast per product);
    returns (loss, {parameter name: leaf clone})."""
    c = model.config
    leaves = {}

    def leaf(name, p):
        leaves[name] = p.detach().float().to(device).requires_grad_(True)
        return leaves[name].to(dtype)

    modules = dict(model.named_modules())

    def project(name, x):
        p = modules[name]
        out = x @ p.base_weight().to(device, dtype).T
        if p.bias is not None:
            out = out + p.bias.to(device, dtype)
        return out + (x @ leaf(name + ".lora_A", p.lora_A).T) @ leaf(name + ".lora_B", p.lora_B).T

    def norm(module, x):
        wide = x.float()
        normed = (wide * torch.rsqrt(wide.square().mean(-1, keepdim=True) + c.rms_norm_eps)).to(dtype)
        return normed * module.weight.to(device, dtype)

    def rope(x, cos, sin):
        half = cos.shape[-1]
        pairs = x[..., :2 * half].unflatten(-1, (-1, 2))
        a, b = pairs[..., 0], pairs[..., 1]
        cs, sn = cos[:, None, :], sin[:, None, :]
        turned = torch.stack((a * cs - b * sn, b * cs + a * sn), -1).flatten(-2)
        return torch.cat((turned, x[..., 2 * half:]), -1)

    def attend(q, k, v):
        parts = []
        for s, e in records:
            # [heads, q, d] @ [d, k] with the single key head shared: plain contiguous products
            query = q[s:e].transpose(0, 1)
            scores = (query @ k[s:e, 0].T.contiguous()).float() / math.sqrt(c.head_dim)
            mask = torch.ones(e - s, e - s, dtype=torch.bool, device=device).tril()
            probs = scores.masked_fill(~mask, float("-inf")).softmax(-1).to(dtype)
            parts.append((probs @ v[s:e, 0]).transpose(0, 1))
        return torch.cat(parts).flatten(-2)

    positions = torch.cat([torch.arange(e - s) for s, e in records]).float().to(device)
    channel = torch.arange(0, c.rotary_dim, 2, dtype=torch.float32, device=device)
    angle = positions[:, None] * (1.0 / (c.rope_theta ** (channel / c.rotary_dim)))
    cos, sin = angle.cos().to(dtype), angle.sin().to(dtype)
    x = model.embed_tokens.weight.detach().to(device, dtype)[ids.to(device)]
    for index, layer in enumerate(model.layers):
        pre = f"layers.{index}."
        h = norm(layer.input_layernorm, x)
        q = rope(project(pre + "self_attn.q_proj", h).unflatten(-1, (c.num_attention_heads, c.head_dim)), cos, sin)
        k = rope(project(pre + "self_attn.k_proj", h).unflatten(-1, (1, c.head_dim)), cos, sin)
        v = project(pre + "self_attn.v_proj", h).unflatten(-1, (1, c.head_dim))
        # recomputed in the backward, so the [heads, len, len] scores of every layer are
        # not all held at once
        y = checkpoint(attend, q, k, v, use_reentrant=False)
        x = x + project(pre + "self_attn.o_proj", y)
        h = norm(layer.post_attention_layernorm, x)
        g = project(pre + "mlp.gate_proj", h)
        u = project(pre + "mlp.up_proj", h)
        x = x + project(pre + "mlp.down_proj", F.silu(g) * u)
    logits = (norm(model.norm, x) @ model.lm_head.weight.to(device, dtype).T).float()
    loss = (F.cross_entropy(logits, targets.to(device), reduction="none") * weights.to(device)).sum()
    return loss, leaves


def _batch(model):
    records = [(0, 13), (13, 29), (29, 40)]
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(model.config.vocab_size, (40,), generator=g)
    targets = torch.roll(ids, -1)
    weights = torch.ones(40)
    for _, stop in records:
        weights[stop - 1] = 0  # the last token of a record predicts nothing
    return ids.cuda(), targets.cuda(), weights.cuda(), records


def test_decoder_loss_and_lora_gradients_against_fp32_host():
    model = _tiny()
    ids, targets, weights, records = _batch(model)
    loss = model.loss(ids[None], targets[None], weights[None], records, token_budget=16)
    loss.backward()
    want, leaves = _host_loss(model, ids, targets, weights, records)
    want.backward()
    assert abs(float(loss.detach()) - float(want.detach())) <= 2e-2 * abs(float(want.detach()))
    for name, p in model.named_parameters():
        if not p.requires_grad:
            assert p.grad is None
            continue
        ref = leaves[name].grad
        err = (p.grad.float().cpu() - ref).norm() / ref.norm()
        assert err <= 5e-2, (name, float(err))


def test_decoder_adamw_step_lowers_the_loss():
    from causal_tuner.optim import FusedAdamW
    model = _tiny()
    ids, targets, weights, records = _batch(model)
    params = [p for p in model.parameters() if p.requires_grad]
    opt = FusedAdamW(params, lr=1e-3, weight_decay=0.0)
    first = None
    for _ in range(3):
        loss = model.loss(ids[None], targets[None], weights[None], records, token_budget=16)
        first = float(loss.detach()) if first is None else first
        loss.backward()
        torch.nn.utils.clip_grad_norm_(params, 1.0, foreach=True)
        opt.step()
        opt.zero_grad(set_to_none=True)
    assert float(model.loss(ids[None], targets[None], weights[None], records).detach()) < first


def test_mlp_cache_budget_gives_identical_loss_and_gradients():
    """With an MLP cache budget (the reference's mlp_cache_budget_bytes, assigned from the
    last layer back: modeling/model.py:227-237) the cached layers' backward reads the
    forward's gate/up and xa instead of recomputing them: the loss and every LoRA gradient
    equal the uncached step bit for bit. A budget for one layer caches only the last."""
    model = _tiny()
    ids, targets, weights, records = _batch(model)
    rows = ids.numel()
    one = model.layers[0].mlp.cache_bytes(rows)
    results = []
    for budget, cached in ((0, [False, False]), (one, [False, True]), (4 * one, [True, True])):
        model.zero_grad(set_to_none=True)
        loss = model.loss(ids[None], targets[None], weights[None], records, token_budget=16, mlp_cache_bytes=budget)
        assert [layer.mlp.cache_intermediates for layer in model.layers] == cached
        loss.backward()
        results.append((loss.detach().clone(), {n: p.grad.clone() for n, p in model.named_parameters()
                                                if p.grad is not None}))
    for loss, grads in results[1:]:
        assert torch.equal(loss, results[0][0])
        assert grads.keys() == results[0][1].keys()
        for name, grad in grads.items():
            assert torch.equal(grad, results[0][1][name]), name
