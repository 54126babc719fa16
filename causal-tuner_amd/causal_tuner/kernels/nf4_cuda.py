"""Decode packed NF4 weights and nested scales in one HIP launch.

Drop-in for the reference's `dequantize_nf4` (kernels/nf4_cuda.py:32-43): same arguments,
same output (a new tensor of `state.shape` in `dtype`, decoded values rounded first to
`state.dtype`), bit-exact. The decode runs in `ct_nf4_dequant` (csrc/nf4_dequant.hip) on
the caller's current stream.
"""

import torch

from . import _native


def dequantize_nf4(weight, state, dtype):
    if dtype not in _native.DTYPE_CODES:
        raise ValueError(f"Unsupported output dtype {dtype}")
    if not weight.is_cuda:
        raise RuntimeError("NF4 decoding runs on the HIP device; the packed weight is on the CPU")
    output = torch.empty(state.shape, device=weight.device, dtype=dtype)
    dequantize_nf4_into(weight, state, output)
    return output


def dequantize_nf4_into(weight, state, output):
    """Decode into a caller-owned, contiguous `output` of `state.shape` elements."""
    if weight.dtype != torch.uint8 or not weight.is_contiguous():
        raise ValueError("NF4 packed weights must be a contiguous uint8 tensor")
    if not output.is_contiguous() or output.numel() != state.shape.numel():
        raise ValueError("NF4 output must be contiguous with the state's element count")
    desc = _native.nf4_descriptor(weight, state)
    with _native.device_of(weight):
        status = _native.library().ct_nf4_dequant(desc, _native.ptr(output), _native.dtype_code(output.dtype),
                                                  _native.stream_of(output))
    _native.check(status, "ct_nf4_dequant")
    return output
