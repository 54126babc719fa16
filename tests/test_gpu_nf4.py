"""NF4 decode on the MI355X: bit-exact against the CPU oracle (ct_nf4_dequant).

Mirrors the reference's test_single_pass_nf4_matches_native_dequantization and
test_nf4_odd_tail_groups (tests/test_kernel_workspaces.py:256-266, 422-430), whose oracle
is bitsandbytes' dequantize_4bit; here the oracle is oracle/nf4.py (pinned in
tests/test_oracle.py), compared with rtol = atol = 0.
"""

import ctypes
import glob
import os

import numpy as np
import pytest
import torch

from oracle import nf4 as onf4

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
NAMES = {torch.bfloat16: onf4.BF16, torch.float16: onf4.F16, torch.float32: onf4.F32}
TORCH = {v: k for k, v in NAMES.items()}


def _state_numpy(packed, state):
    s = {"n": state.shape.numel(), "blocksize": state.blocksize, "nested": state.nested,
         "code": state.code.cpu().numpy(), "absmax": state.absmax.cpu().numpy(), "storage": NAMES[state.dtype]}
    if state.nested:
        s.update(code2=state.state2.code.cpu().numpy(), absmax2=state.state2.absmax.cpu().numpy(),
                 offset=np.float32(state.offset.item()), blocksize2=state.state2.blocksize)
    return packed.cpu().numpy().reshape(-1), s


def _as_numpy(t):
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
    return t.cpu().numpy().reshape(-1)


@pytest.mark.parametrize("nested", [False, True])
@pytest.mark.parametrize("source_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("blocksize", [64, 128, 4096])
def test_single_pass_nf4_matches_oracle(nested, source_dtype, blocksize):
    from causal_tuner.kernels.linear import materialize
    from causal_tuner.quant.nf4 import quantize_nf4
    values = torch.randn(71, 96, device="cuda", dtype=source_dtype)
    packed, state = quantize_nf4(values, blocksize=blocksize, compress_statistics=nested)
    p, s = _state_numpy(packed, state)
    for dtype in (torch.bfloat16, torch.float32, torch.float16):
        got = materialize(packed, state, dtype)
        assert got.shape == (71, 96) and got.dtype == dtype
        np.testing.assert_array_equal(_as_numpy(got), onf4.dequantize_state(p, s, NAMES[dtype]).reshape(-1))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_nf4_odd_tail_groups(dtype):
    from causal_tuner.kernels.linear import materialize
    from causal_tuner.quant.nf4 import quantize_nf4
    source = torch.randn(17, 19, device="cuda", dtype=dtype)
    packed, state = quantize_nf4(source, blocksize=64, compress_statistics=True)
    p, s = _state_numpy(packed, state)
    for compute in (torch.bfloat16, torch.float32):
        np.testing.assert_array_equal(_as_numpy(materialize(packed, state, compute)),
                                      onf4.dequantize_state(p, s, NAMES[compute]))


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(HERE, "golden", "dequant_*.npz"))))
def test_dequant_fixtures(path):
    from causal_tuner.kernels.nf4_cuda import dequantize_nf4
    from causal_tuner.quant.nf4 import QuantState
    f = np.load(path)
    rows, cols, bs, nested = (int(v) for v in f["meta"])
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    state2 = QuantState(dev(f["absmax2"]), torch.Size([len(f["absmax"])]), dev(f["code2"]), 256, "dynamic",
                        torch.float32) if nested else None
    state = QuantState(dev(f["absmax"]), torch.Size([rows, cols]), dev(f["code"]), bs, "nf4",
                       TORCH[str(f["storage"])], dev(f["offset"].reshape(1)) if nested else None, state2)
    for out in (torch.bfloat16, torch.float16, torch.float32):
        got = dequantize_nf4(dev(f["packed"]), state, out)
        np.testing.assert_array_equal(_as_numpy(got), f[f"expected_{NAMES[out]}"].reshape(-1))


def test_nested_scale_is_not_fused():
    from causal_tuner.kernels.nf4_cuda import dequantize_nf4
    from causal_tuner.quant.nf4 import QuantState
    c = 1 + 2 ** -12
    n = 128
    packed = torch.full((n // 2, 1), 0xFF, dtype=torch.uint8, device="cuda")   # code[15] = 1.0
    state2 = QuantState(torch.tensor([c], device="cuda"), torch.Size([2]), torch.full((256,), c, device="cuda"),
                        256, "dynamic", torch.float32)
    state = QuantState(torch.zeros(2, dtype=torch.uint8, device="cuda"), torch.Size([2, 64]),
                       torch.tensor(onf4.NF4_CODE, device="cuda"), 64, "nf4", torch.float32,
                       torch.tensor([-1.0], device="cuda"), state2)
    got = dequantize_nf4(packed, state, torch.float32)
    assert torch.all(got == 2 ** -11), got.flatten()[:4]  # an FMA would give 2^-11 + 2^-24


def test_unaligned_and_strided_inputs_take_the_general_path():
    from causal_tuner.kernels.nf4_cuda import dequantize_nf4_into
    from causal_tuner.quant.nf4 import quantize_nf4
    w = torch.randn(64, 96, device="cuda", dtype=torch.bfloat16)
    packed, state = quantize_nf4(w)
    p, s = _state_numpy(packed, state)
    expected = onf4.dequantize_state(p, s, onf4.BF16)
    storage = torch.empty(packed.numel() + 1, dtype=torch.uint8, device="cuda")
    shifted = storage[1:].view(-1, 1)
    shifted.copy_(packed)
    out_storage = torch.empty(w.numel() + 1, dtype=torch.bfloat16, device="cuda")
    out = out_storage[1:]
    dequantize_nf4_into(shifted, state, out)
    np.testing.assert_array_equal(_as_numpy(out), expected)


@pytest.mark.parametrize("shape", [(8192, 8192), (28672, 8192)])
def test_full_size_dequant_matches_plain_c_oracle(shape):
    """The C2 configurations, decoded whole and compared element for element."""
    from causal_tuner.kernels.linear import materialize
    from causal_tuner.quant.nf4 import quantize_nf4
    g = torch.Generator(device="cuda").manual_seed(2)
    w = (torch.randn(shape, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    packed, state = quantize_nf4(w)
    got = materialize(packed, state, torch.bfloat16)
    torch.cuda.synchronize()
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "lib", "libnf4_oracle.so"))
    p, s = _state_numpy(packed, state)
    n = s["n"]
    expected = np.empty(n, np.uint16)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    lib.ct_oracle_nf4_dequant_bf16(ptr(p), ptr(s["absmax"]), ptr(s["code"]), ptr(s["code2"]), ptr(s["absmax2"]),
                                   ctypes.c_float(s["offset"]), ctypes.c_int64(n), ctypes.c_int64(64),
                                   ctypes.c_int64(256), ptr(expected))
    actual = _as_numpy(got)
    mismatches = int((actual != expected).sum())
    assert mismatches == 0, f"{mismatches} of {n} elements differ"
    # the dequantized weight approximates the source within the NF4 grid resolution
    err = (got.float() - w.float()).abs().max().item()
    assert err <= 0.2 * w.float().abs().max().item()


def _oracle_quantize(values, blocksize, nested, offset=None):
    return onf4.quantize(values.float().cpu().numpy(), blocksize=blocksize, nested=nested,
                         storage=NAMES[values.dtype], offset=offset)


@pytest.mark.parametrize("shape,blocksize,nested,dtype", [
    ((71, 96), 64, True, torch.bfloat16), ((17, 19), 64, True, torch.bfloat16), ((300, 1000), 64, True, torch.bfloat16),
    ((64, 64), 32, True, torch.float16), ((128, 96), 128, False, torch.float32), ((40, 100), 4096, True, torch.float32),
    ((3, 5), 2, True, torch.bfloat16), ((1, 1), 64, False, torch.bfloat16)])
def test_device_quantizer_matches_oracle(shape, blocksize, nested, dtype):
    """ct_nf4_quantize (Projection.install_nf4's quantizer on the device) against the CPU
    restatement of bitsandbytes' algorithm (oracle/nf4.py quantize), byte for byte: packed
    codes, first-level absmax (u8 codes or fp32), absmax2 and offset. Odd element counts,
    a 256-block group boundary (300 x 1000 = 4688 blocks), an all-zero block, blocksizes 2
    to 4096 and every source dtype. Parity with bitsandbytes' own bytes stays unpinned
    (bitsandbytes is absent and the reference's tests store no quantized bytes)."""
    from causal_tuner.quant.nf4 import quantize_nf4
    g = torch.Generator().manual_seed(sum(shape) + blocksize)
    values = (torch.randn(*shape, generator=g) * 0.02).to(dtype)
    if values.numel() >= 2 * blocksize:
        values.view(-1)[blocksize:2 * blocksize] = 0   # an all-zero block (absmax 0, NaN codes)
    packed, state = quantize_nf4(values.cuda(), blocksize=blocksize, compress_statistics=nested)
    torch.cuda.synchronize()
    # the offset is torch's fp32 mean of the block absmax (bitsandbytes' absmax.mean()):
    # within float rounding of the exact mean; the oracle reproduces the rest from it
    offset = state.offset.item() if nested else None
    want_packed, want = _oracle_quantize(values, blocksize, nested, offset)
    if nested:
        _, exact = _oracle_quantize(values, blocksize, nested)
        assert abs(offset - float(exact["offset"])) <= 1e-6 * abs(float(exact["offset"]))
    np.testing.assert_array_equal(packed.cpu().numpy().reshape(-1), want_packed)
    np.testing.assert_array_equal(state.absmax.cpu().numpy(), want["absmax"])
    assert state.blocksize == blocksize and state.dtype == dtype and tuple(state.shape) == shape
    if nested:
        assert np.float32(state.offset.item()) == want["offset"]
        np.testing.assert_array_equal(state.state2.absmax.cpu().numpy(), want["absmax2"])
        np.testing.assert_array_equal(state.state2.code.cpu().numpy(), want["code2"])
    # and the host path (torch ops) agrees with the device path (with the host's fp32 mean)
    hp, hs = quantize_nf4(values, blocksize=blocksize, compress_statistics=nested)
    assert torch.equal(hp, packed.cpu())
    if nested:
        _, host_want = _oracle_quantize(values, blocksize, nested, hs.offset.item())
        np.testing.assert_array_equal(hs.absmax.numpy(), host_want["absmax"])
    else:
        assert torch.equal(hs.absmax, state.absmax.cpu())


def test_device_quantizer_round_trip_large():
    """A C5-sized weight (24576 x 6144): quantize on the device, decode with ct_nf4_dequant,
    and every element lands on its block's nearest code (|w - decoded| <= half the largest
    code gap times the block's scale)."""
    from causal_tuner.kernels.linear import materialize
    from causal_tuner.quant.nf4 import quantize_nf4
    g = torch.Generator(device="cuda").manual_seed(11)
    w = (torch.randn(24576, 6144, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    packed, state = quantize_nf4(w)
    back = materialize(packed, state, torch.float32)
    err = (w.float() - back).abs().view(-1, 64).amax(1)
    scale = w.float().abs().view(-1, 64).amax(1)
    gap = float((torch.tensor(onf4.NF4_CODE[1:]) - torch.tensor(onf4.NF4_CODE[:-1])).max())
    # the decoded scale differs from absmax by the 8-bit second level: allow 2% of it
    assert bool((err <= scale * (gap / 2 + 0.02)).all())
