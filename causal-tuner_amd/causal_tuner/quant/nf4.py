"""NF4 weight state and quantizer (the state the reference obtains from bitsandbytes).

The reference quantizes its frozen base weights through bitsandbytes>=0.45,<1
(`pyproject.toml:21`) with `Params4bit(..., compress_statistics=True, quant_type="nf4")`
(`modeling/lora.py:50-55`) and reads back the QuantState fields listed in `QuantState`
below (`kernels/nf4_cuda.py:33-41`, `kernels/linear.py:8`). bitsandbytes is not a
dependency here: `quantize_nf4` restates its published blockwise algorithm, on the device
with the HIP kernels of csrc/nf4_quantize.hip and on the host with torch tensor ops:

1. absmax[g] = max |w| over each block of `blocksize` elements (zero-padded tail);
2. x = w * (1 / absmax[g]) in fp32, NF4 code = number of code-book midpoints below x
   (the midpoints are the fp32 roundings of the float64 means of adjacent codes);
3. two codes per byte, element 2j in the high nibble; [ceil(N/2), 1] uint8;
4. compress_statistics: offset = mean(absmax); absmax - offset is block-quantized in
   blocks of 256 against the signed 8-bit dynamic map (`dynamic_map`), with per-block
   absmax2 and the bitsandbytes binary-search nearest rule (`_dynamic_codes`).
The dequantizer consumes the state as given, so decode parity does not depend on how
closely this quantizer follows bitsandbytes' bits.
"""

import math
from dataclasses import dataclass

import torch

# NormalFloat-4 code book (QLoRA): normal quantiles at linspace(0.9677083, 0.5, 9)[:-1] and
# the negated ones at linspace(0.9677083, 0.5, 8)[:-1], plus 0, sorted and scaled by the max.
NF4_CODE = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453, -0.28444138169288635,
    -0.18477343022823334, -0.09105003625154495, 0.0, 0.07958029955625534, 0.16093020141124725,
    0.24611230194568634, 0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
    0.7229568362236023, 1.0,
)


def nf4_code(device=None):
    return torch.tensor(NF4_CODE, dtype=torch.float32, device=device)


def nf4_thresholds(device=None):
    """Decision midpoints between adjacent NF4 codes, float64 means rounded to fp32."""
    code = torch.tensor(NF4_CODE, dtype=torch.float64)
    return ((code[:-1] + code[1:]) / 2).to(torch.float32).to(device)


def dynamic_map(signed=True, max_exponent_bits=7, total_bits=8):
    """bitsandbytes' dynamic 8-bit map (create_dynamic_map): 256 sorted fp32 values."""
    data = []
    non_sign_bits = total_bits - 1
    additional_items = 2 ** (non_sign_bits - max_exponent_bits) - 1
    for i in range(max_exponent_bits):
        items = int(2 ** (i + non_sign_bits - max_exponent_bits) + 1 if signed
                    else 2 ** (i + non_sign_bits - max_exponent_bits + 1) + 1)
        boundaries = torch.linspace(0.1, 1, items, dtype=torch.float32)
        means = (boundaries[:-1] + boundaries[1:]) / 2.0
        data += ((10 ** (-(max_exponent_bits - 1) + i)) * means).tolist()
        if signed:
            data += (-(10 ** (-(max_exponent_bits - 1) + i)) * means).tolist()
    if additional_items > 0:
        boundaries = torch.linspace(0.1, 1, additional_items + 1, dtype=torch.float32)
        means = (boundaries[:-1] + boundaries[1:]) / 2.0
        data += ((10 ** (-(max_exponent_bits - 1) + max_exponent_bits - 1)) * means).tolist()
        if signed:
            data += (-(10 ** (-(max_exponent_bits - 1) + max_exponent_bits - 1)) * means).tolist()
    data.append(0)
    data.append(1.0)
    data += [0] * (2 ** total_bits - len(data))
    data.sort()
    return torch.tensor(data, dtype=torch.float32)


@dataclass
class QuantState:
    """The QuantState fields the reference's NF4 path reads."""

    absmax: torch.Tensor            # uint8 [nb] codes (nested) or float32 [nb] scales
    shape: torch.Size               # dense weight shape, (out, in)
    code: torch.Tensor              # float32 [16] (first level) or [256] (second level)
    blocksize: int
    quant_type: str = "nf4"
    dtype: torch.dtype = torch.bfloat16  # storage dtype of decoded values (source dtype)
    offset: torch.Tensor | None = None   # float32 scalar tensor (nested)
    state2: "QuantState | None" = None   # second-level state (nested)

    @property
    def nested(self):
        return self.state2 is not None

    def to(self, device):
        moved = QuantState(self.absmax.to(device), self.shape, self.code.to(device), self.blocksize,
                           self.quant_type, self.dtype, None if self.offset is None else self.offset.to(device),
                           None if self.state2 is None else self.state2.to(device))
        return moved


def _dynamic_codes(x, code):
    """bitsandbytes' dQuantize binary search: nearest entry of the sorted 256-entry `code`."""
    pivot = torch.full_like(x, 127, dtype=torch.int64)
    upper_pivot = torch.full_like(pivot, 255)
    lower_pivot = torch.zeros_like(pivot)
    lower = torch.full_like(x, -1.0)
    upper = torch.full_like(x, 1.0)
    val = code[pivot]
    step = 64
    while step > 0:
        right = x > val
        lower_pivot = torch.where(right, pivot, lower_pivot)
        lower = torch.where(right, val, lower)
        upper_pivot = torch.where(right, upper_pivot, pivot)
        upper = torch.where(right, upper, val)
        pivot = torch.where(right, pivot + step, pivot - step)
        val = code[pivot]
        step //= 2
    upper = torch.where(upper_pivot == 255, code[255], upper)
    lower = torch.where(lower_pivot == 0, code[0], lower)
    above = x > val
    mid_up = (upper + val) * 0.5
    mid_low = (lower + val) * 0.5
    return torch.where(above, torch.where(x > mid_up, upper_pivot, pivot),
                       torch.where(x < mid_low, lower_pivot, pivot)).to(torch.uint8)


def _block_absmax(flat, blocksize):
    n = flat.numel()
    blocks = math.ceil(n / blocksize)
    padded = torch.zeros(blocks * blocksize, dtype=torch.float32, device=flat.device)
    padded[:n] = flat
    return padded.view(blocks, blocksize), padded.view(blocks, blocksize).abs().amax(1)


def quantize_blockwise(values, code, blocksize=256):
    """8-bit blockwise quantization against `code` (bitsandbytes quantize_blockwise)."""
    blocks, absmax = _block_absmax(values.reshape(-1).float(), blocksize)
    normed = blocks * (1.0 / absmax)[:, None]
    q = _dynamic_codes(normed.reshape(-1), code)[: values.numel()]
    return q, absmax


def quantize_nf4(weight, blocksize=64, compress_statistics=True):
    """Quantize `weight` to NF4 on its device. Returns (packed uint8 [ceil(N/2), 1], QuantState).

    Device tensors run the HIP quantizer (ct_nf4_quantize); host tensors run the same
    algorithm as torch tensor ops (`_quantize_nf4_ops`)."""
    if blocksize < 2 or blocksize & (blocksize - 1):
        raise ValueError("NF4 blocksize must be a power of two >= 2")
    if weight.is_cuda:
        return _quantize_nf4_device(weight, blocksize, compress_statistics)
    return _quantize_nf4_ops(weight, blocksize, compress_statistics)


def _quantize_nf4_device(weight, blocksize, compress_statistics):
    from ..kernels import _native
    source = weight.detach()
    if source.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError(f"NF4 quantization of {source.dtype} weights is not supported")
    flat = source.reshape(-1).contiguous()
    device = flat.device
    n = flat.numel()
    nb = -(-n // blocksize) if n else 0
    packed = torch.empty((n + 1) // 2, 1, dtype=torch.uint8, device=device)
    code = nf4_code(device)
    midpoints = nf4_thresholds(device)
    nested = bool(compress_statistics)
    lib = _native.library()
    # First level (NF4 codes and fp32 block absmax); with double quantization the absmax
    # then goes through bitsandbytes' second level: offset = absmax.mean() (torch's fp32
    # mean, as quantize_4bit computes it) and absmax - offset quantized in blocks of 256.
    first = torch.empty(nb, dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        stream = _native.stream_of(flat)
        status = lib.ct_nf4_quantize(
            _native.ptr(flat), _native.dtype_code(flat.dtype), n, blocksize, 0, _native.ptr(midpoints), None,
            _native.ptr(packed), _native.ptr(first), None, None, None, 0, stream)
        _native.check(status, "ct_nf4_quantize")
        if not nested:
            return packed, QuantState(first, source.shape, code, blocksize, "nf4", source.dtype)
        offset = first.mean()
        code2 = dynamic_map().to(device)
        absmax = torch.empty(nb, dtype=torch.uint8, device=device)
        absmax2 = torch.empty(-(-nb // 256), dtype=torch.float32, device=device)
        status = lib.ct_quantize_blockwise(_native.ptr(first), nb, _native.ptr(offset), _native.ptr(code2),
                                           _native.ptr(absmax), _native.ptr(absmax2), stream)
        _native.check(status, "ct_quantize_blockwise")
    state2 = QuantState(absmax2, torch.Size([nb]), code2, 256, "dynamic", torch.float32)
    return packed, QuantState(absmax, source.shape, code, blocksize, "nf4", source.dtype, offset, state2)


def _quantize_nf4_ops(weight, blocksize=64, compress_statistics=True):
    """The quantizer as torch tensor ops (host tensors)."""
    source = weight.detach()
    device = source.device
    flat = source.reshape(-1).float()
    n = flat.numel()
    blocks, absmax = _block_absmax(flat, blocksize)
    normed = blocks * (1.0 / absmax)[:, None]
    codes = torch.searchsorted(nf4_thresholds(device), normed.reshape(-1).contiguous())[:n].to(torch.uint8)
    if n % 2:  # the last byte's low nibble is padding
        codes = torch.cat((codes, codes.new_zeros(1)))
    pairs = codes.view(-1, 2)
    packed = ((pairs[:, 0] << 4) | pairs[:, 1]).contiguous().view(-1, 1)
    code = nf4_code(device)
    if compress_statistics:
        offset = absmax.mean()   # bitsandbytes: torch's fp32 mean of the block absmax
        code2 = dynamic_map().to(device)
        qabs, absmax2 = quantize_blockwise(absmax - offset, code2, 256)
        state2 = QuantState(absmax2, torch.Size([absmax.numel()]), code2, 256, "dynamic", torch.float32)
        state = QuantState(qabs, source.shape, code, blocksize, "nf4", source.dtype, offset, state2)
    else:
        state = QuantState(absmax, source.shape, code, blocksize, "nf4", source.dtype)
    return packed, state
