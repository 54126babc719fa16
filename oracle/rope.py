"""Partial GPT-J rotary embedding, CPU restatement. TEST INFRASTRUCTURE ONLY.

Follows the reference's `_rotate_pair` and `_rope` (kernels/core_cuda.py:133-167): over
x [tokens, heads, head_dim] with cosine/sine [tokens, half], channel pairs (2c, 2c+1),
c < half, become
    e' = T(T(e cos) - T(o sin)),   o' = T(T(o cos) + T(e sin))
in float32 arithmetic with T = rounding to the tensor type (round to nearest even), the
sine negated for the inverse; other channels pass through. numpy, vectorised over pairs.
"""

import numpy as np

_ROUNDERS = {}


def _round_bf16(v):
    """float32 -> nearest-even bfloat16, returned as float32 (exact)."""
    bits = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) >> 16 << 16
    nan = np.isnan(v)
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), out)


def round_to(v, dtype):
    v = np.asarray(v, dtype=np.float32)
    if dtype == "bfloat16":
        return _round_bf16(v)
    if dtype == "float16":
        return v.astype(np.float16).astype(np.float32)
    return v


def rope(x, cosine, sine, head_dim, dtype, *, inverse=False):
    """x: float32 array [tokens, width] holding `dtype` values; cosine/sine float32 [tokens,
    half] holding the trig dtype's values. Returns the rotated array (float32 holding
    `dtype` values)."""
    x = np.asarray(x, dtype=np.float32)
    tokens, width = x.shape
    heads = width // head_dim
    half = cosine.shape[-1]
    view = x.reshape(tokens, heads, head_dim // 2, 2)
    e, o = view[:, :, :half, 0], view[:, :, :half, 1]
    c = np.asarray(cosine, dtype=np.float32)[:, None, :]
    s = np.asarray(sine, dtype=np.float32)[:, None, :]
    if inverse:
        s = -s
    ec, os_ = round_to(e * c, dtype), round_to(o * s, dtype)
    oc, es = round_to(o * c, dtype), round_to(e * s, dtype)
    out = view.copy()
    out[:, :, :half, 0] = round_to(ec - os_, dtype)
    out[:, :, :half, 1] = round_to(oc + es, dtype)
    return out.reshape(tokens, width)
