"""Fused GEMM epilogues (ct_epilogue on ct_forward_linear / ct_input_gradient) against the
same projection followed by the standalone kernels: the residual add (reference
kernels/linear.py:90-91, kernels/mlp_cuda.py:80), SiLU x up and its backward
(kernels/mlp_cuda.py:10-35,131-133) and the partial GPT-J rotation of q/k
(kernels/core_cuda.py:133-200).

Every route of the GEMM is covered -- the few-row kernels (<= 64 rows), the split 256 x 256
runner (65..511 rows with a small output), the 64/128/256 tiles, a row pitch that is not a
multiple of 8, dense and NF4 bases -- and each must give the unfused sequence's values bit
for bit: both apply the same device functions to the same bf16-rounded projection output.
The operator-level tests run the q/k/v group and the MLP with the fusion on and off
(monkeypatched `fusable`) and require identical outputs and gradients."""

import pytest
import torch

pytestmark = pytest.mark.gpu

# (rows, out features, in features): few-row kernels, split runner, 64 tiles, 128 tiles,
# 256 tiles, unaligned output pitch
ROUTES = [(16, 1024, 2048), (48, 512, 1024), (130, 1024, 2048), (300, 4096, 512), (2048, 2048, 1024),
          (4096, 4096, 512), (77, 1004, 256)]


def _base(k, n, r, nf4, seed):
    from causal_tuner.kernels.linear import _Base, projection_parameters
    from causal_tuner.modeling.lora import Projection
    torch.manual_seed(seed)
    module = Projection(k, n, bias=False, rank=r, device="cuda")
    if nf4:
        module.install_nf4(module.weight.detach().clone(), "cuda")
    torch.nn.init.normal_(module.lora_B, std=0.05)
    (weight, a, b, _), state = projection_parameters(module)
    return _Base(weight, state, torch.bfloat16), a.detach().bfloat16(), b.detach().bfloat16()


def _rand(*shape, seed, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(*shape, device="cuda", generator=g) * scale).to(torch.bfloat16)


def _forward(base, x, a, b, epilogue=None):
    from causal_tuner.kernels.linear import _forward
    out = torch.empty(len(x), base.rows, device="cuda", dtype=torch.bfloat16)
    xa = torch.empty(len(x), len(a), device="cuda", dtype=torch.bfloat16)
    weight = base.matrix if base.state is None else base.weight
    _forward(x, weight, base.state, a, b, None, out, xa, False, epilogue(out) if epilogue else None)
    return out, xa


@pytest.mark.parametrize("nf4", [False, True])
@pytest.mark.parametrize("m,n,k", ROUTES)
def test_forward_epilogues_equal_separate_kernels(m, n, k, nf4):
    from causal_tuner.kernels import _native
    from causal_tuner.kernels.core_cuda import _rope
    from causal_tuner.kernels.mlp_cuda import activation
    print(f"forward epilogues m={m} n={n} k={k} nf4={nf4}", flush=True)
    base, a, b = _base(k, n, 16, nf4, seed=m + n)
    x = _rand(m, k, seed=1)
    plain, xa = _forward(base, x, a, b)
    # residual
    residual = _rand(m, n, seed=2)
    got, got_xa = _forward(base, x, a, b, lambda out: _native.epilogue(_native.CT_EPI_RESIDUAL, m, in0=residual))
    assert torch.equal(got_xa, xa)
    assert torch.equal(got, plain + residual)
    # SiLU x up, with and without keeping the raw up
    gate = _rand(m, n, seed=3, scale=3.0)
    want = activation(gate, plain)
    for keep in (None, torch.empty_like(plain)):
        got, _ = _forward(base, x, a, b, lambda out: _native.epilogue(_native.CT_EPI_SILU, m, in0=gate, out0=keep))
        assert torch.equal(got, want)
        if keep is not None:
            assert torch.equal(keep, plain)
    # partial rotation over heads of head_dim (only 2 * half channels rotate)
    head_dim, half = (128, 32) if n % 128 == 0 else (4, 1)
    for trig_dtype in (torch.bfloat16, torch.float32):
        angle = torch.rand(m, half, device="cuda", generator=torch.Generator(device="cuda").manual_seed(4)) * 1e4
        cosine, sine = angle.cos().to(trig_dtype), angle.sin().to(trig_dtype)
        want = _rope(plain.clone(), plain.clone(), cosine, sine, head_dim, inverse=False, rotated_only=False)
        got, _ = _forward(base, x, a, b, lambda out: _native.epilogue(_native.CT_EPI_ROPE, m,
                                                                        rotary=(cosine, sine, head_dim)))
        assert torch.equal(got, want)


@pytest.mark.parametrize("nf4", [False, True])
@pytest.mark.parametrize("m,n,k", ROUTES)
def test_input_gradient_silu_backward_equals_separate_kernel(m, n, k, nf4):
    """dh = dy w_down + low a_down with (gate, up, dh) -> (d gate, d up, h) in its epilogue,
    in place of the gate/up buffers and beside kept ones."""
    from causal_tuner.kernels import _native
    from causal_tuner.kernels.linear import _input_gradient
    from causal_tuner.kernels.mlp_cuda import _silu_kernel
    print(f"input-gradient epilogue m={m} n={n} k={k} nf4={nf4}", flush=True)
    # down: in features k (the MLP width), out features n; dx is [m, k]
    base, a, b = _base(k, n, 16, nf4, seed=m + k)
    weight = base.matrix if base.state is None else base.weight
    dy = _rand(m, n, seed=5)
    gate, up = _rand(m, k, seed=6, scale=3.0), _rand(m, k, seed=7)
    dh = torch.empty(m, k, device="cuda", dtype=torch.bfloat16)
    low = torch.empty(m, 16, device="cuda", dtype=torch.bfloat16)
    _input_gradient(dy, weight, base.state, a, b, dh, low, False)
    want_g, want_u, want_h = torch.empty_like(gate), torch.empty_like(up), dh.clone()
    _silu_kernel(gate, up, want_h, want_g, want_u, backward=True, reconstruct=True)
    # beside kept gate/up
    d_g, d_u, h = torch.empty_like(gate), torch.empty_like(up), torch.empty_like(dh)
    low2 = torch.empty_like(low)
    e = _native.epilogue(_native.CT_EPI_DSILU, m, in0=gate, in1=up, out0=d_g, out1=d_u)
    _input_gradient(dy, weight, base.state, a, b, h, low2, False, e)
    assert torch.equal(low2, low)
    for got, want in ((d_g, want_g), (d_u, want_u), (h, want_h)):
        assert torch.equal(got, want)
    # in place over the gate/up buffers
    g2, u2 = gate.clone(), up.clone()
    e = _native.epilogue(_native.CT_EPI_DSILU, m, in0=g2, in1=u2, out0=g2, out1=u2)
    _input_gradient(dy, weight, base.state, a, b, h, low2, False, e)
    for got, want in ((g2, want_g), (u2, want_u), (h, want_h)):
        assert torch.equal(got, want)


def test_epilogue_rejected_with_accumulation_and_bad_shapes():
    from causal_tuner.kernels import _native
    from causal_tuner.kernels.linear import _forward, _input_gradient
    base, a, b = _base(256, 512, 16, False, seed=0)
    x = _rand(32, 256, seed=1)
    out = torch.empty(32, 512, device="cuda", dtype=torch.bfloat16)
    xa = torch.empty(32, 16, device="cuda", dtype=torch.bfloat16)
    gate = _rand(32, 256, seed=2)
    e = _native.epilogue(_native.CT_EPI_DSILU, 32, in0=gate, in1=gate, out0=gate.clone(), out1=gate.clone())
    with pytest.raises(ValueError):
        _input_gradient(out, base.matrix, None, a, b, torch.empty_like(x), torch.empty_like(xa), True, e)
    bad = _native.epilogue(_native.CT_EPI_ROPE, 32, rotary=(torch.ones(32, 2, device="cuda"),
                                                            torch.ones(32, 2, device="cuda"), 6))
    with pytest.raises(RuntimeError, match="ct_forward_linear failed"):
        _forward(x, base.matrix, None, a, b, None, out, xa, False, bad)
    missing = _native.Epilogue(kind=_native.CT_EPI_RESIDUAL)
    with pytest.raises(RuntimeError):
        _forward(x, base.matrix, None, a, b, None, out, xa, False, missing)


def test_epilogue_rejects_strided_or_mixed_rotary_tables():
    """The fused rotation reads [rows, half] tables with a row pitch of half and one dtype:
    column slices of a wider table, tables of two dtypes or of another row count are
    refused on the host (the separate ct_rope pass validates its own)."""
    from causal_tuner.kernels import _native
    wide = torch.ones(32, 4, device="cuda")
    for cosine, sine in ((wide[:, :2], wide[:, 2:]),
                         (torch.ones(32, 2, device="cuda"), torch.ones(32, 2, device="cuda", dtype=torch.bfloat16)),
                         (torch.ones(31, 2, device="cuda"), torch.ones(31, 2, device="cuda"))):
        with pytest.raises(ValueError, match="rotary tables"):
            _native.epilogue(_native.CT_EPI_ROPE, 32, rotary=(cosine, sine, 8))


def _unfused(monkeypatch):
    from causal_tuner.kernels import linear, mlp_cuda
    monkeypatch.setattr(linear, "fusable", lambda *tensors: False)
    monkeypatch.setattr(mlp_cuda, "fusable", lambda *tensors: False)


def _group_run(x, rotary, residual, nf4):
    from causal_tuner.kernels.linear import project_group
    from causal_tuner.modeling.lora import Projection
    modules = []
    for i, n in enumerate((1024, 256, 256)):
        torch.manual_seed(10 + i)
        module = Projection(x.shape[1], n, bias=False, rank=16, device="cuda")
        if nf4:
            module.install_nf4(module.weight.detach().clone(), "cuda")
        torch.nn.init.normal_(module.lora_B, std=0.05)
        modules.append(module)
    xd = x.clone().requires_grad_(True)
    outs = project_group(modules, xd, rotary=rotary)
    o = modules[0]
    projected = project_group((o,), x, residual=residual)[0]
    signals = [_rand(*t.shape, seed=20 + i) for i, t in enumerate(outs)]
    params = [xd, *(p for m in modules for p in (m.lora_A, m.lora_B))]
    grads = torch.autograd.grad(outs, params, signals)
    return [*outs, projected], grads


@pytest.mark.parametrize("nf4", [False, True])
@pytest.mark.parametrize("tokens", [40, 300, 4100])
def test_qkv_group_and_residual_fused_equal_unfused(tokens, nf4, monkeypatch):
    """The q/k/v group with rotary (q, k rotated in their GEMM epilogues) and an o-style
    projection with the residual fused, against the same calls with the epilogues as
    separate passes: identical outputs and gradients."""
    print(f"qkv group fused vs unfused tokens={tokens} nf4={nf4}", flush=True)
    x = _rand(tokens, 512, seed=30)
    residual = _rand(tokens, 1024, seed=31)
    angle = torch.rand(tokens, 32, device="cuda", generator=torch.Generator(device="cuda").manual_seed(32)) * 1e3
    rotary = (angle.cos().bfloat16(), angle.sin().bfloat16(), 128)
    fused_outs, fused_grads = _group_run(x, rotary, residual, nf4)
    with monkeypatch.context() as patch:
        _unfused(patch)
        outs, grads = _group_run(x, rotary, residual, nf4)
    for got, want in zip(fused_outs, outs):
        assert torch.equal(got, want)
    for got, want in zip(fused_grads, grads):
        assert torch.equal(got, want)


def _mlp_run(module, x, residual, cache):
    from causal_tuner.kernels.mlp_cuda import tiled_lora_mlp
    xd = x.clone().requires_grad_(True)
    out = tiled_lora_mlp(module, xd, residual, cache=cache)
    dy = _rand(*out.shape, seed=40)
    params = [xd, *(p for p in module.parameters() if p.requires_grad)]
    return out, torch.autograd.grad(out, params, dy)


@pytest.mark.parametrize("cache", [False, True])
@pytest.mark.parametrize("nf4", [False, True])
@pytest.mark.parametrize("tokens,tile", [(24, None), (200, 64), (1030, 512)])
def test_mlp_fused_epilogues_equal_unfused(tokens, tile, nf4, cache, monkeypatch):
    """SiLU x up in the up GEMM, the residual in the down GEMM and the SiLU backward in the
    dh GEMM against the separate kernels: identical outputs and gradients, with and without
    the intermediate cache, in one tile and in several."""
    from causal_tuner.modeling.mlp import MLP
    print(f"mlp fused vs unfused tokens={tokens} tile={tile} nf4={nf4} cache={cache}", flush=True)
    torch.manual_seed(50)
    module = MLP(512, 1536, rank=16, device="cuda", tile=tile)
    for projection in (module.gate_proj, module.up_proj, module.down_proj):
        torch.nn.init.normal_(projection.lora_B, std=0.05)
        if nf4:
            projection.install_nf4(projection.weight.detach().clone(), "cuda")
    x = _rand(tokens, 512, seed=51)
    residual = _rand(tokens, 512, seed=52)
    fused = _mlp_run(module, x, residual, cache)
    with monkeypatch.context() as patch:
        _unfused(patch)
        plain = _mlp_run(module, x, residual, cache)
    assert torch.equal(fused[0], plain[0])
    for got, want in zip(fused[1], plain[1]):
        assert torch.equal(got, want)
