"""Pins oracle/rope.py (the partial-RoPE restatement) without retyping it: closed-form
angles, a float64 rotation, the round trip, untouched channels, the bf16 rounder against
torch's conversion, and the host `rotate` of the package (the reference's torch-op
formula, modeling/rotary.py:16-24) bit for bit."""

import numpy as np
import pytest
import torch

from oracle import rope as orope


def _bf16(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def test_bf16_rounder_matches_torch_conversion():
    rng = np.random.default_rng(0)
    v = np.concatenate([(rng.standard_normal(100000) * 10.0 ** rng.integers(-30, 30, 100000)).astype(np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9], np.float32)])
    got = orope.round_to(v, "bfloat16")
    want = _bf16(v)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.isnan(orope.round_to(np.array([np.nan], np.float32), "bfloat16")).all()


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_zero_and_quarter_turn_are_exact(dtype):
    rng = np.random.default_rng(1)
    x = orope.round_to(rng.standard_normal((5, 24)).astype(np.float32), dtype)
    ones, zeros = np.ones((5, 3), np.float32), np.zeros((5, 3), np.float32)
    assert np.array_equal(orope.rope(x, ones, zeros, 8, dtype), x)          # angle 0: identity
    turned = orope.rope(x, zeros, ones, 8, dtype)                           # angle pi/2: (e, o) -> (-o, e)
    v, t = x.reshape(5, 3, 4, 2), turned.reshape(5, 3, 4, 2)
    assert np.array_equal(t[:, :, :3, 0], -v[:, :, :3, 1])
    assert np.array_equal(t[:, :, :3, 1], v[:, :, :3, 0])
    assert np.array_equal(t[:, :, 3:], v[:, :, 3:])                           # channels past 2*half


def test_against_float64_rotation_and_round_trip():
    rng = np.random.default_rng(2)
    tokens, heads, head_dim, half = 33, 4, 16, 5
    x = _bf16(rng.standard_normal((tokens, heads * head_dim)))
    angle = rng.uniform(-100, 100, (tokens, half))
    c, s = _bf16(np.cos(angle)), _bf16(np.sin(angle))
    got = orope.rope(x, c, s, head_dim, "bfloat16")
    v = x.reshape(tokens, heads, head_dim // 2, 2).astype(np.float64)
    e, o = v[:, :, :half, 0], v[:, :, :half, 1]
    exact = np.stack((e * c[:, None] - o * s[:, None], o * c[:, None] + e * s[:, None]), -1)
    gv = got.reshape(tokens, heads, head_dim // 2, 2)
    # three bf16 roundings (two products, one sum) bound the error by ~3 ulps of the inputs
    assert np.abs(gv[:, :, :half] - exact).max() <= 3 * 2 ** -8 * np.abs(v).max()
    back = orope.rope(got, c, s, head_dim, "bfloat16", inverse=True)
    assert np.abs(back - x).max() <= 8 * 2 ** -8 * np.abs(x).max()  # cos^2 + sin^2 = 1 up to bf16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_matches_package_host_formula_bit_for_bit(dtype):
    from causal_tuner.modeling.rotary import rotate
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 7, 3, 8, generator=g).to(dtype)
    angle = torch.rand(2, 7, 2, generator=g) * 60000
    c, s = angle.cos().to(dtype), angle.sin().to(dtype)
    want = rotate(x, c, s)
    name = str(dtype).split(".")[-1]
    got = orope.rope(x.float().reshape(14, 24).numpy(), c.float().reshape(14, 2).numpy(),
                     s.float().reshape(14, 2).numpy(), 8, name)
    assert np.array_equal(got, want.float().reshape(14, 24).numpy())
