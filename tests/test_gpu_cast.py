"""cast_all / ct_cast_f32_bf16: the group's fp32 LoRA factors rounded to bf16 in one launch
must equal torch's per-tensor .to(torch.bfloat16) bit for bit (the reference casts each
factor, kernels/linear.py:70,108): random values, ties, infinities, NaN, subnormals, the
largest finite values, sizes around the 8-element groups and the per-workgroup span, and
more tensors than one call takes."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _special(n):
    bits = torch.tensor([0x7f800000, 0xff800000, 0x7fc00000, 0x00000001, 0x807fffff, 0x7f7fffff, 0xff7fffff,
                         0x3f808000, 0x3f818000, 0x3f80ffff, 0x00400000, 0x80000000, 0x33800000],
                        dtype=torch.int64).to(torch.int32)
    values = bits.view(torch.float32)
    return values.repeat(n // len(values) + 1)[:n]


@pytest.mark.parametrize("sizes", [[5, 8, 17], [8192 + 3, 1, 7, 4096 * 4 + 8], [(256, 4096), (4096, 256), (128, 256)],
                                   [33] * 20])
def test_cast_all_matches_torch_bitwise(sizes):
    from causal_tuner.kernels.linear import cast_all
    g = torch.Generator(device="cuda").manual_seed(9)
    tensors = []
    for i, size in enumerate(sizes):
        shape = size if isinstance(size, tuple) else (size,)
        t = torch.randn(*shape, device="cuda", generator=g) * (10.0 ** (i % 5 - 2))
        flat = t.view(-1)
        special = _special(min(flat.numel(), 64)).cuda()
        flat[:special.numel()] = special
        tensors.append(t)
    tensors.append(torch.randn(3, device="cuda").to(torch.bfloat16))  # already bf16: passed through .to
    got = cast_all(tensors, torch.bfloat16)
    for t, c in zip(tensors, got):
        want = t.to(torch.bfloat16)
        assert c.shape == t.shape and c.dtype == torch.bfloat16
        assert torch.equal(c.view(torch.int16), want.view(torch.int16))
