"""Fused NF4 operands of the projection GEMMs (forward x w^T and the transposed dx = dy w).

The fused loaders decode the packed weight tile by tile into LDS with the reference's
decoding rule (kernels/nf4_cuda.py:16-29), and from 512 rows on the entry points decode it
once into the workspace instead; either way a projection over the packed weight must be
bit-identical to the same projection over the weight that `materialize` produces
(kernels/linear.py:6-13): both run the same tile shape and summation order. The float64
oracle bounds the result itself."""

import pytest
import torch

from causal_tuner.kernels import _native
from causal_tuner.kernels.linear import _forward, _input_gradient, materialize
from causal_tuner.quant.nf4 import quantize_nf4
from oracle import lora as olora

pytestmark = pytest.mark.gpu

# (m, k, n, r): tails in every dimension, odd ranks, and 256x256-tile shapes; m <= 64 runs
# the few-row kernels (1, 2 and 4 row blocks; 1, 2 and 4 column blocks per workgroup), and
# from m = 512 on the entry points decode the weight into the workspace first (for dx
# transposed when rows % 8 == 0 and cols % 16 == 0, as (600, 1040, 1096) with partial
# tiles; (520, 96, 84) takes the untransposed decode).
SHAPES = [(37, 96, 80, 8), (300, 256, 192, 5), (1, 64, 64, 4), (513, 1024, 1032, 16), (4096, 4096, 4096, 256),
          (448, 4096, 4096, 64), (511, 1024, 2056, 16), (600, 1040, 1096, 24), (520, 96, 84, 8),
          (2048, 4096, 11008, 256), (4096, 11008, 4096, 64), (16, 6144, 24576, 256), (64, 24576, 6144, 256),
          (5, 1024, 512, 8), (29, 2048, 16384, 16), (64, 4096, 8192, 128), (3, 128, 8200, 4)]


def _weight(n, k, blocksize=64, nested=True, dtype=torch.bfloat16, seed=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(dtype)
    return quantize_nf4(w, blocksize=blocksize, compress_statistics=nested)


def _inputs(m, k, n, r, seed=1):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
    a = ((torch.rand(r, k, device="cuda", generator=g) * 2 - 1) * (6 / k) ** 0.5).to(torch.bfloat16)
    b = (torch.randn(n, r, device="cuda", generator=g) * 0.01).to(torch.bfloat16)
    dy = torch.randn(m, n, device="cuda", generator=g).to(torch.bfloat16)
    bias = (torch.randn(n, device="cuda", generator=g) * 0.1).to(torch.bfloat16)
    return x, a, b, dy, bias


@pytest.mark.parametrize("m,k,n,r", SHAPES)
def test_fused_forward_and_input_gradient_equal_materialized(m, k, n, r):
    packed, state = _weight(n, k)
    if m < 512:   # decoded inside the GEMM: the fused loaders must take the layout
        assert _native.library().ct_nf4_fused_supported(_native.nf4_descriptor(packed, state)) == 1
    dense = materialize(packed, state, torch.bfloat16)
    x, a, b, dy, bias = _inputs(m, k, n, r)
    outs = []
    for weight, st in ((packed, state), (dense, None)):
        out = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        xa = torch.empty(m, r, device="cuda", dtype=torch.bfloat16)
        _forward(x, weight, st, a, b, bias, out, xa)
        dx = torch.full((m, k), float("nan"), device="cuda", dtype=torch.bfloat16)
        low = torch.empty(m, r, device="cuda", dtype=torch.bfloat16)
        _input_gradient(dy, weight, st, a, b, dx, low, False)
        acc = dx.clone()
        _input_gradient(dy, weight, st, a, b, acc, low, True)   # grouped accumulation (add=True)
        outs.append((out, xa, dx, low, acc))
    torch.cuda.synchronize()
    for fused, plain, name in zip(outs[0], outs[1], ("out", "xa", "dx", "low", "dx+=")):
        assert torch.equal(fused.view(torch.int16), plain.view(torch.int16)), name
    if m * k * n <= 2 ** 27:   # float64 oracle on the host for the small shapes
        out, xa, dx, low, _ = (t.cpu() for t in outs[0])
        oout, oxa, odx, olow, _, _ = olora.oracle_projection(x.cpu(), dense.cpu(), a.cpu(), b.cpu(), dy.cpu(),
                                                           bias.cpu())
        for got, want, name in ((out, oout, "out"), (dx, odx, "dx")):
            _, norm = olora.relative_error(got, want)
            assert norm <= 1e-3, (name, norm)


@pytest.mark.parametrize("blocksize,nested,dtype", [(64, False, torch.bfloat16), (128, True, torch.float32),
                                                    (32, True, torch.bfloat16), (4096, True, torch.bfloat16)])
def test_fused_state_variants(blocksize, nested, dtype):
    m, k, n, r = 130, 4096, 96, 8
    packed, state = _weight(n, k, blocksize, nested, dtype)
    dense = materialize(packed, state, torch.bfloat16)
    x, a, b, dy, bias = _inputs(m, k, n, r, seed=3)
    results = []
    for weight, st in ((packed, state), (dense, None)):
        out = torch.empty(m, n, device="cuda", dtype=torch.bfloat16)
        xa = torch.empty(m, r, device="cuda", dtype=torch.bfloat16)
        _forward(x, weight, st, a, b, None, out, xa)
        dx = torch.empty(m, k, device="cuda", dtype=torch.bfloat16)
        low = torch.empty(m, r, device="cuda", dtype=torch.bfloat16)
        _input_gradient(dy, weight, st, a, b, dx, low, False)
        results.append((out, dx))
    for fused, plain in zip(*results):
        assert torch.equal(fused.view(torch.int16), plain.view(torch.int16))


def test_unsupported_layouts_are_refused_not_miscomputed():
    packed, state = _weight(64, 48)            # cols % 32 != 0: the fused loaders refuse it
    assert _native.library().ct_nf4_fused_supported(_native.nf4_descriptor(packed, state)) == 0
    x = torch.randn(8, 48, device="cuda").to(torch.bfloat16)
    a = torch.randn(4, 48, device="cuda").to(torch.bfloat16)
    b = torch.randn(64, 4, device="cuda").to(torch.bfloat16)
    out = torch.empty(8, 64, device="cuda", dtype=torch.bfloat16)
    xa = torch.empty(8, 4, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="fused"):
        _forward(x, packed, state, a, b, None, out, xa)


@pytest.mark.parametrize("m,k,n,r", [(4096, 2048, 2048, 256), (1024, 4096, 4096, 64), (4096, 8192, 2048, 256),
                                     (2048, 2048, 640, 16)])
def test_many_rows_with_less_than_one_round_of_large_tiles(m, k, n, r):
    """Many rows whose output gives the 256 x 256 workgroups less than one round (the C4
    shapes q/o/down at 4096 tokens take the 128 x 128 grid): forward and dx (also with
    add=True) against fp32 products of the same bf16 operands rounded once, and a repeated
    forward bit-identical."""
    packed, state = _weight(n, k, seed=3)
    dense = materialize(packed, state, torch.bfloat16)
    x, a, b, dy, bias = _inputs(m, k, n, r, seed=2)
    xf, wf, af, bf, dyf = (t.float() for t in (x, dense, a, b, dy))
    out = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    xa = torch.empty(m, r, device="cuda", dtype=torch.bfloat16)
    _forward(x, packed, state, a, b, bias, out, xa)
    want_xa = xf @ af.T
    want_out = xf @ wf.T + bias.float() + xa.float() @ bf.T
    dx = torch.full((m, k), float("nan"), device="cuda", dtype=torch.bfloat16)
    low = torch.empty(m, r, device="cuda", dtype=torch.bfloat16)
    _input_gradient(dy, packed, state, a, b, dx, low, False)
    want_dx = dyf @ wf + low.float() @ af
    def check(got, want, name, tol=1e-3):   # against the fp32 result rounded once to bf16
        want = want.to(torch.bfloat16).float()
        norm = ((got.float() - want).norm() / want.norm()).item()
        assert norm <= tol, (name, norm)
    for got, want, name in ((xa, want_xa, "xa"), (out, want_out, "out"), (dx, want_dx, "dx")):
        check(got, want, name)
    acc = dx.clone()
    _input_gradient(dy, packed, state, a, b, acc, low, True)
    check(acc, dx.float() + want_dx, "dx+=")
    again = torch.empty_like(out)
    _forward(x, packed, state, a, b, bias, again, torch.empty_like(xa))
    assert torch.equal(again.view(torch.int16), out.view(torch.int16))
