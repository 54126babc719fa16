"""numpy restatement of NF4 decoding and of the bitsandbytes quantizer. TEST INFRASTRUCTURE ONLY.

Reference: kernels/nf4_cuda.py:9-43 (decode), modeling/lora.py:41-56 (quantization via
bitsandbytes>=0.45,<1, pyproject.toml:21; call sites lora.py:50-55, linear.py:11-12).
"""

import numpy as np

# QLoRA NormalFloat-4 code book, fp32 (pinned in tests against its quantile construction).
NF4_CODE = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453, -0.28444138169288635,
    -0.18477343022823334, -0.09105003625154495, 0.0, 0.07958029955625534, 0.16093020141124725,
    0.24611230194568634, 0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
    0.7229568362236023, 1.0], dtype=np.float32)

F32, F16, BF16 = "float32", "float16", "bfloat16"


# ----------------------------------------------------------------------------- rounding
def bf16_bits(values):
    """fp32 -> bf16 bit patterns, round to nearest even (NaN -> quiet NaN)."""
    u = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    if nan.any():
        rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_to(values, dtype):
    """Round fp32 values to `dtype` and widen back to fp32 (exact)."""
    values = np.asarray(values, dtype=np.float32)
    if dtype == BF16:
        return bf16_to_f32(bf16_bits(values))
    if dtype == F16:
        return values.astype(np.float16).astype(np.float32)
    return values


def encode(values_f32, dtype):
    """fp32 values that are already representable -> storage array of `dtype`."""
    if dtype == BF16:
        return bf16_bits(values_f32)
    if dtype == F16:
        return values_f32.astype(np.float16)
    return values_f32.astype(np.float32)


# ----------------------------------------------------------------------------- decode
def block_scales(absmax, nested, code2=None, absmax2=None, offset=None, blocksize2=256):
    """s[g] (kernels/nf4_cuda.py:16-20): code2[absmax[g]] * absmax2[g // blocksize2] + offset,
    an fp32 multiply and a separately rounded fp32 add; non-nested: absmax[g]."""
    if not nested:
        return np.asarray(absmax, dtype=np.float32)
    g = np.arange(len(absmax))
    decoded = np.asarray(code2, np.float32)[np.asarray(absmax, np.int64)] * \
        np.asarray(absmax2, np.float32)[g // blocksize2]
    return (decoded + np.float32(offset)).astype(np.float32)


def dequantize(packed, absmax, n, blocksize=64, nested=True, code=NF4_CODE, code2=None, absmax2=None,
               offset=None, blocksize2=256, storage=BF16, out=BF16):
    """Closed form of _decode (kernels/nf4_cuda.py:13-29) for an n-element weight.

    Returns the output as `out` storage (uint16 bf16 bits, float16 or float32)."""
    packed = np.asarray(packed, dtype=np.uint8).reshape(-1)
    code = np.asarray(code, dtype=np.float32)
    scales = block_scales(absmax, nested, code2, absmax2, offset, blocksize2)
    nibbles = np.empty(2 * len(packed), dtype=np.uint8)
    nibbles[0::2] = packed >> 4        # element 2j: high nibble (nf4_cuda.py:24,27)
    nibbles[1::2] = packed & 15        # element 2j+1: low nibble (nf4_cuda.py:25,27)
    nibbles = nibbles[:n]
    g = np.arange(n) // blocksize
    values = code[nibbles] * scales[g]                       # fp32 product (nf4_cuda.py:27)
    stored = round_to(values, storage)                       # STORAGE_DTYPE cast (nf4_cuda.py:29,36)
    return encode(round_to(stored, out), out)


def dequantize_state(packed, state, out=BF16):
    """Decode from a dict of numpy state fields (the QuantState fields the reference reads)."""
    return dequantize(packed, state["absmax"], state["n"], state["blocksize"], state["nested"],
                      state["code"], state.get("code2"), state.get("absmax2"), state.get("offset"),
                      state.get("blocksize2", 256), state["storage"], out)


# ----------------------------------------------------------------------------- quantizer
def nf4_thresholds():
    code = NF4_CODE.astype(np.float64)
    return ((code[:-1] + code[1:]) / 2).astype(np.float32)


def dynamic_map(signed=True, max_exponent_bits=7, total_bits=8):
    """bitsandbytes create_dynamic_map: 256 sorted fp32 values.

    bitsandbytes builds it with torch CPU ops (fp32 linspace, fp32 scaling); torch CPU is
    used here for the same arithmetic."""
    import torch
    data = []
    non_sign_bits = total_bits - 1
    additional = 2 ** (non_sign_bits - max_exponent_bits) - 1
    ranges = [(i, int(2 ** (i + non_sign_bits - max_exponent_bits) + 1 if signed
                      else 2 ** (i + non_sign_bits - max_exponent_bits + 1) + 1)) for i in range(max_exponent_bits)]
    if additional > 0:
        ranges.append((max_exponent_bits - 1, additional + 1))
    for i, items in ranges:
        bounds = torch.linspace(0.1, 1, items, dtype=torch.float32)
        means = (bounds[:-1] + bounds[1:]) / 2.0
        data += ((10 ** (-(max_exponent_bits - 1) + i)) * means).tolist()
        if signed:
            data += (-(10 ** (-(max_exponent_bits - 1) + i)) * means).tolist()
    data += [0.0, 1.0]
    data += [0.0] * (2 ** total_bits - len(data))
    return np.array(sorted(data), dtype=np.float32)


def dynamic_code(x, code):
    """bitsandbytes dQuantize (binary search + midpoint rule) for one fp32 value, pure Python."""
    x = np.float32(x)
    pivot, upper_pivot, lower_pivot = 127, 255, 0
    lower, upper = np.float32(-1.0), np.float32(1.0)
    val = code[pivot]
    step = 64
    while step > 0:
        if x > val:
            lower_pivot, lower, pivot = pivot, val, pivot + step
        else:
            upper_pivot, upper, pivot = pivot, val, pivot - step
        val = code[pivot]
        step //= 2
    if upper_pivot == 255:
        upper = code[255]
    if lower_pivot == 0:
        lower = code[0]
    if x > val:
        return upper_pivot if x > np.float32((upper + val) * np.float32(0.5)) else pivot
    return lower_pivot if x < np.float32((lower + val) * np.float32(0.5)) else pivot


def quantize(weight_f32, blocksize=64, nested=True, storage=BF16, offset=None):
    """bitsandbytes quantize_4bit(quant_type="nf4", compress_statistics=nested), restated.

    `storage` is the source weight's dtype (QuantState.dtype). bitsandbytes' offset is
    torch's fp32 mean of the block absmax (absmax.mean()), whose last bits depend on torch's
    reduction order: pass that value as `offset` to reproduce a state; without it the
    correctly rounded (float64) mean is used. Returns (packed uint8 [ceil(n/2)], state dict)."""
    flat = np.asarray(weight_f32, dtype=np.float32).reshape(-1)
    n = flat.size
    nb = -(-n // blocksize)
    padded = np.zeros(nb * blocksize, dtype=np.float32)
    padded[:n] = flat
    blocks = padded.reshape(nb, blocksize)
    absmax = np.abs(blocks).max(axis=1).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        normed = blocks * (np.float32(1.0) / absmax)[:, None]
    codes = np.searchsorted(nf4_thresholds(), normed.reshape(-1), side="left").astype(np.uint8)[:n]
    if n % 2:
        codes = np.concatenate([codes, np.zeros(1, np.uint8)])
    packed = ((codes[0::2] << 4) | codes[1::2]).astype(np.uint8)
    state = {"n": n, "blocksize": blocksize, "nested": nested, "code": NF4_CODE.copy(), "storage": storage}
    if nested:
        offset = np.float32(absmax.astype(np.float64).mean()) if offset is None else np.float32(offset)
        code2 = dynamic_map()
        centred = (absmax - offset).astype(np.float32)
        nb2 = -(-nb // 256)
        pad2 = np.zeros(nb2 * 256, dtype=np.float32)
        pad2[:nb] = centred
        absmax2 = np.abs(pad2.reshape(nb2, 256)).max(axis=1).astype(np.float32)
        with np.errstate(divide="ignore", invalid="ignore"):
            normed2 = pad2.reshape(nb2, 256) * (np.float32(1.0) / absmax2)[:, None]
        qabs = np.array([dynamic_code(v, code2) for v in normed2.reshape(-1)[:nb]], dtype=np.uint8)
        state.update(absmax=qabs, code2=code2, absmax2=absmax2, offset=offset, blocksize2=256)
    else:
        state["absmax"] = absmax
    return packed, state
