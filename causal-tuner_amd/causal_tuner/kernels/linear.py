"""Shared-input LoRA projections with bounded workspaces and FP32 adapter gradients, on gfx950.

Same operator API as the reference's kernels/linear.py (`materialize` 6-13, `accumulate`
16-24, `forward_linear` 27-33, `input_gradient` 36-39, `parameter_gradients` 42-44,
`projection_parameters` 47-50, `can_fuse` 53-56, `_LoRAGroup` 59-130, `project_group`
133-148). On the device, every contraction runs in the HIP GEMMs of
lib/libcausal_tuner_hip.so:

* forward_linear: `ct_forward_linear`, xa = x a^T then out = [x | xa] [w | b]^T (+ bias):
  the base GEMM and the rank-r epilogue are one MFMA contraction over k + r columns,
  rounded to bf16 once;
* input_gradient: `ct_input_gradient`, low = dy b then dx = [dy | low] [w ; a] (+ dx);
* parameter_gradients / accumulate: `ct_parameter_gradients` / `ct_accumulate`, fp32
  outputs with a fixed-order split reduction over tokens (repeated backward is
  bit-identical; add=False ignores the destination's contents).

The bf16 path is the benchmarked device path; float32 device operands run the fp32 GEMM
(`ct_gemm_f32`, `mm_f32`). CPU tensors keep the reference's torch semantics (its unfused
CPU route); device tensors of another compute dtype raise NotImplementedError, except in
`accumulate`, which casts mixed operands to the output dtype as the reference does
(linear.py:22-23) and then runs the fp32 or bf16 GEMM (a float16 projection loss with a
float32 head accumulates that way).
"""

import contextlib
import contextvars
import ctypes
import functools

import torch

from . import _native


# ----------------------------------------------------------------------------- helpers
_FLOATS = (torch.float16, torch.bfloat16, torch.float32)


def _device_bf16(*tensors):
    return all(t.is_cuda and t.dtype == torch.bfloat16 for t in tensors if t is not None)


def _unsupported(what, *tensors):
    dtypes = sorted({str(t.dtype) for t in tensors if t is not None})
    raise NotImplementedError(f"{what}: the HIP path computes in bfloat16 on the device (got {', '.join(dtypes)})")


def _device_f32(*tensors):
    return all(t.is_cuda and t.dtype == torch.float32 for t in tensors if t is not None)


def _aligned(t):
    return t.data_ptr() % 16 == 0


def _rows(t):
    """(tensor, leading dimension) of a matrix with unit stride along its rows; a view whose
    base is not 16-byte aligned is copied so the kernels can use 16-byte loads."""
    if t.is_contiguous() and t.dim() == 2 and not t.data_ptr() & 15:   # the common case, fewer queries
        ld = t.stride(0)
        if ld >= t.shape[1]:   # (a one-row view may carry any stride along its rows)
            return t, ld
    if t.dim() != 2:
        raise ValueError("expected a matrix")
    if t.stride(1) != 1 or t.stride(0) < t.shape[1]:
        if t.shape[0] <= 1 and t.stride(1) == 1:
            return (t if _aligned(t) else t.clone()), max(t.shape[1], 1)
        t = t.contiguous()
    if not _aligned(t):
        t = t.clone()
    return t, t.stride(0)


def _operand(t):
    """(tensor, ld, transposed) for a bf16 matrix given as a row- or column-major view."""
    if t.stride(1) == 1 and t.stride(0) >= t.shape[1]:
        return t, t.stride(0), 0
    if t.stride(0) == 1 and t.stride(1) >= t.shape[0]:
        return t, t.stride(1), 1
    t = t.contiguous()
    return t, max(t.shape[1], 1), 0


def fusable(*tensors):
    """Whether a fused GEMM epilogue may write/read these and any window of their rows:
    device bf16 matrices with unit stride along their rows, a row pitch of a multiple of 8
    elements and a 16-byte aligned start (None entries are ignored)."""
    return all(t.is_cuda and t.dtype == torch.bfloat16 and t.dim() == 2 and t.stride(1) == 1
               and t.stride(0) >= t.shape[1] and t.stride(0) % 8 == 0 and _aligned(t)
               for t in tensors if t is not None)


@functools.lru_cache(maxsize=4096)
def _query(name, *args):
    """A workspace-size query of the library (pure in its integer arguments), cached."""
    return getattr(_native.library(), name)(*args)


_NO_WORKSPACE = {}


def _workspace(nbytes, device):
    """Caller-owned scratch for split reductions (the kernels never allocate); torch's
    caching allocator makes the per-call allocation cheap. A call that needs none gets one
    empty tensor per device (a null pointer and 0 bytes), with no allocation."""
    if nbytes <= 0:
        empty = _NO_WORKSPACE.get(device)
        if empty is None:
            empty = _NO_WORKSPACE[device] = torch.empty(0, dtype=torch.uint8, device=device)
        return empty
    return torch.empty(int(nbytes), dtype=torch.uint8, device=device)


class _Output:
    """A caller's output view; kernels write a contiguous stand-in when the view is strided."""

    def __init__(self, target):
        self.target = target
        ok = ((target.is_contiguous() and target.dim() == 2 and not target.data_ptr() & 15) or
              (target.dim() == 2 and target.stride(1) == 1 and target.stride(0) >= target.shape[1]
               and _aligned(target)))
        self.buffer = target if ok else torch.empty(target.shape, dtype=target.dtype, device=target.device)
        self.ld = max(self.buffer.stride(0), self.buffer.shape[1], 1)

    def finish(self):
        if self.buffer is not self.target:
            self.target.copy_(self.buffer)


class _Contiguous(_Output):
    def __init__(self, target):
        self.target = target
        self.buffer = target if target.is_contiguous() else torch.empty(target.shape, dtype=target.dtype,
                                                                        device=target.device)
        self.ld = max(target.shape[-1], 1)


def _f32_operand(t):
    """(tensor, ld, transposed) for a float32 matrix view: stored row-major (0) or as the
    row-major transpose (1); anything else is copied."""
    rows, cols = t.shape
    if t.stride(1) == 1 and t.stride(0) >= max(cols, 1):
        return t, max(t.stride(0), 1), 0
    if t.stride(0) == 1 and t.stride(1) >= max(rows, 1):
        return t, max(t.stride(1), 1), 1
    t = t.contiguous()
    return t, max(cols, 1), 0


def mm_f32(left, right, out, *, add=False, bias=None):
    """out (+)= left right (+ bias) in float32 on the device (ct_gemm_f32: fp32 MFMA
    products and sums): the torch.mm / addmm of the reference's float32 compute dtype
    (kernels/linear.py:16-44). `left` [m, k] and `right` [k, n] may be transposed views."""
    m, k = left.shape
    n = right.shape[1]
    if right.shape[0] != k or tuple(out.shape) != (m, n):
        raise ValueError(f"mm_f32: {tuple(left.shape)} x {tuple(right.shape)} -> {tuple(out.shape)}")
    if not _device_f32(left, right, out, bias):
        _unsupported("mm_f32", left, right, out, bias)
    lt, ldl, tl = _f32_operand(left)
    rt, ldr, tr = _f32_operand(right)
    bias = None if bias is None else bias.contiguous()
    direct = out.stride(1) == 1 and out.stride(0) >= max(n, 1)
    target = out if direct else (out.contiguous() if add else torch.empty((m, n), dtype=out.dtype,
                                                                          device=out.device))
    with _native.device_of(out):
        status = _native.library().ct_gemm_f32(
            _native.ptr(lt), ldl, tl, _native.ptr(rt), ldr, tr, _native.ptr(target), max(target.stride(0), 1),
            int(add), _native.ptr(bias), m, n, k, _native.stream_of(out))
    _native.check(status, "ct_gemm_f32")
    if target is not out:
        out.copy_(target)


def _mm_bf16(left, right, out, *, add=False):
    """out = bf16(left right (+ out)) through ct_gemm (fp32 accumulation, one rounding)."""
    m, k = left.shape
    n = right.shape[1]
    lt, ldl, tl = _operand(left)
    rt, ldr, tr = _operand(right)
    target = _Output(out)
    if add and target.buffer is not out:
        target.buffer.copy_(out)
    lib = _native.library()
    ws = _workspace(_query("ct_gemm_workspace", m, n, k, tl, tr, _native.CT_BF16), out.device)
    with _native.device_of(out):
        status = lib.ct_gemm(_native.ptr(lt), ldl, tl, _native.ptr(rt), ldr, tr, _native.ptr(target.buffer),
                             target.ld, _native.CT_BF16, None, int(add), m, n, k, _native.ptr(ws), ws.numel(),
                             _native.stream_of(out))
    _native.check(status, "ct_gemm")
    target.finish()


def product(left, right, out):
    """out = left right in the operands' dtype: ct_gemm for bf16 device operands (fp32
    accumulation, one rounding), torch.mm otherwise (the reference's product)."""
    if _device_bf16(left, right, out):
        _mm_bf16(left, right, out)
    else:
        torch.mm(left, right, out=out)


# ----------------------------------------------------------------------------- operators
def cast_all(tensors, dtype, outputs=None):
    """[t.to(dtype) for t in tensors], with the fp32 device tensors that go to bf16 rounded
    in one launch (ct_cast_f32_bf16) into views of one buffer (or into the given contiguous
    `outputs`, where an entry is not None): the reference casts each LoRA factor separately
    (kernels/linear.py:70,108; kernels/mlp_cuda.py:62,110)."""
    outputs = outputs or [None] * len(tensors)
    out = [None] * len(tensors)
    batch = ([i for i, t in enumerate(tensors) if t.dtype == torch.float32 and t.is_cuda and t.is_contiguous()
              and t.numel()] if dtype == torch.bfloat16 else [])
    if len(batch) > 1 or any(outputs[i] is not None for i in batch):
        first = tensors[batch[0]]
        fresh = []
        for i in batch:
            out[i] = outputs[i]
            if out[i] is None:
                fresh.append(i)
        # fresh outputs are consecutive views of one buffer, so factors cast together can be
        # stacked without a copy (stacked_rows)
        sizes = [tensors[i].numel() for i in fresh]
        buffer = torch.empty(sum((n + 7) // 8 * 8 for n in sizes), dtype=torch.bfloat16, device=first.device)
        offset = 0
        for i, n in zip(fresh, sizes):
            out[i] = buffer[offset:offset + n].view(tensors[i].shape)
            offset += (n + 7) // 8 * 8   # 16-byte aligned views
        lib, stream, limit = _native.library(), _native.stream_of(first), _native.CT_CAST_MAX
        with _native.device_of(first):
            for start in range(0, len(batch), limit):
                part = batch[start:start + limit]
                src = (ctypes.c_void_p * len(part))(*[tensors[i].data_ptr() for i in part])
                dst = (ctypes.c_void_p * len(part))(*[out[i].data_ptr() for i in part])
                counts = (ctypes.c_int64 * len(part))(*[tensors[i].numel() for i in part])
                _native.check(lib.ct_cast_f32_bf16(src, dst, counts, len(part), stream), "ct_cast_f32_bf16")
    result = [t.to(dtype) if o is None else o for t, o in zip(tensors, out)]
    for i, o in enumerate(outputs):
        if o is not None and result[i] is not o:
            o.copy_(result[i])
            result[i] = o
    return result


def group_factors(parameters, count, dtype, x, shared=None):
    """The compute-dtype LoRA factors of `count` projections, cast together, and when the
    first `shared` of them (default all) read the same input on the device with one rank,
    the stacked [a_1; a_2; ...] (shared * r rows) that gives their xa in one GEMM.
    Returns (factors, stacked or None) with factors = [a_1, b_1, a_2, b_2, ...]."""
    shared = count if shared is None else shared
    tensors = [value for i in range(count) for value in parameters[i*4+1:i*4+3]]
    ranks = {tensors[2*i].shape[0] for i in range(shared)}
    if (shared > 1 and x.is_cuda and dtype == torch.bfloat16 and len(ranks) == 1 and ranks != {0}
            and len({tensors[2*i].shape[1] for i in range(shared)}) == 1):
        r = ranks.pop()
        stack = torch.empty((shared * r, tensors[0].shape[1]), dtype=dtype, device=x.device)
        outputs = [stack[i*r:(i+1)*r] if j == 0 and i < shared else None for i in range(count) for j in (0, 1)]
        return cast_all(tensors, dtype, outputs), stack
    return cast_all(tensors, dtype), None


def materialize(weight, state, dtype):
    if state is not None:
        if state.quant_type != "nf4":
            raise ValueError(f"Unsupported quantization type {state.quant_type!r}")
        if not weight.is_cuda:
            raise RuntimeError("NF4 weights decode on the HIP device only")
        from .nf4_cuda import dequantize_nf4
        return dequantize_nf4(weight.contiguous(), state, dtype)
    return weight.to(dtype)


def accumulate(output, left, right, *, add=True):
    beta = 1 if add else 0
    if output.dtype == torch.float32 and left.dtype == torch.bfloat16 and left.is_cuda:
        if right.dtype != torch.bfloat16:
            _unsupported("accumulate", left, right)
        p, j = left.shape
        q = right.shape[1]
        target = _Output(output)
        lt, ldl, tl = _operand(left)
        rt, ldr, tr = _operand(right)
        lib = _native.library()
        ws = _workspace(_query("ct_accumulate_workspace", p, q, j), output.device)
        with _native.device_of(output):
            status = lib.ct_accumulate(_native.ptr(target.buffer), target.ld, _native.ptr(lt), ldl, tl,
                                       _native.ptr(rt), ldr, tr, p, q, j, int(add) if target.buffer is output else
                                       0, _native.ptr(ws), ws.numel(), _native.stream_of(output))
        _native.check(status, "ct_accumulate")
        if target.buffer is not output:
            output.copy_(target.buffer + output if add else target.buffer)
    elif output.is_cuda:
        if output.dtype == torch.float32 and left.dtype in _FLOATS and right.dtype in _FLOATS:
            # the reference casts mixed operands to the output dtype first (linear.py:22-23):
            # fp16 or bf16 operands widen to float32 exactly, then fp32 products and sums
            mm_f32(left.float(), right.float(), output, add=add)
        elif _device_bf16(output, left, right):
            _mm_bf16(left, right, output, add=add)   # bf16 parameters: one rounding of acc (+ out)
        elif output.dtype == torch.bfloat16 and left.dtype in _FLOATS and right.dtype in _FLOATS:
            _mm_bf16(left.to(torch.bfloat16), right.to(torch.bfloat16), output, add=add)
        else:
            _unsupported("accumulate", output, left, right)
    elif output.dtype != left.dtype:
        output.addmm_(left.to(output.dtype), right.to(output.dtype), beta=beta)
    else:
        output.addmm_(left, right, beta=beta)


def forward_linear(x, weight, a, b, *, out, xa, bias=None):
    if isinstance(weight, _Base):  # a frozen base as the GEMMs consume it (packed NF4 or dense)
        weight.forward(x, a, b, bias, out, xa)
        return
    if not x.is_cuda:
        if bias is None:
            torch.mm(x, weight.T, out=out)
        else:
            torch.addmm(bias, x, weight.T, out=out)
        torch.mm(x, a.T, out=xa)
        out.addmm_(xa, b.T)
        return
    if _device_f32(x, weight, a, b, out, xa, bias):
        # the reference's three products in float32 (kernels/linear.py:28-33)
        mm_f32(x, weight.T, out, bias=bias)
        mm_f32(x, a.T, xa)
        mm_f32(xa, b.T, out, add=True)
        return
    if not _device_bf16(x, weight, a, b, out, xa, bias):
        _unsupported("forward_linear", x, weight, a, b, out, xa, bias)
    _forward(x, weight, None, a, b, bias, out, xa)


def _forward(x, weight, state, a, b, bias, out, xa, xa_given=False, epilogue=None, desc=None):
    """ct_forward_linear; with xa_given, xa (a row-major view, e.g. a column slice of a
    group's shared x [a_1; a_2; ...]^T) already holds x a^T and is only read. `epilogue`
    (a _native.Epilogue over `out`'s rows) is applied to the output in the GEMM. `desc` is the
    weight's NF4 descriptor when the caller holds it already."""
    m, k = x.shape
    n, r = out.shape[1], a.shape[0]
    x, ldx = _rows(x)
    w = None if weight is None else weight.contiguous()
    a, b = a.contiguous(), b.contiguous()
    bias = None if bias is None else bias.contiguous()
    target, low = _Output(out), _Output(xa)
    if epilogue is not None and target.buffer is not out:
        raise ValueError("a fused epilogue needs a unit-stride, 16-byte aligned output")
    if xa_given and low.buffer is not xa:
        low.buffer.copy_(xa)
    if state is not None and desc is None:
        desc = _native.nf4_descriptor(w, state)
    lib = _native.library()
    ws = _workspace(_query("ct_forward_linear_workspace", m, n, k, r, _native.nf4_kind(desc)), x.device)
    with _native.device_of(x):
        status = lib.ct_forward_linear(
            _native.ptr(x), ldx, None if desc is not None else _native.ptr(w), desc, _native.ptr(a),
            _native.ptr(b), _native.ptr(bias), _native.ptr(target.buffer), target.ld, _native.ptr(low.buffer),
            low.ld, int(bool(xa_given)), m, n, k, r, None if epilogue is None else ctypes.byref(epilogue),
            _native.ptr(ws), ws.numel(), _native.stream_of(x))
    _native.check(status, "ct_forward_linear")
    target.finish()
    if not xa_given:
        low.finish()


def input_gradient(dy, weight, a, b, dx, low, *, add=False):
    if isinstance(weight, _Base):
        weight.input_gradient(dy, a, b, dx, low, add)
        return
    if not dy.is_cuda:
        torch.mm(dy, b, out=low)
        torch.addmm(dx, dy, weight, beta=1 if add else 0, out=dx)
        dx.addmm_(low, a)
        return
    if _device_f32(dy, weight, a, b, dx, low):
        # kernels/linear.py:36-39 in float32
        mm_f32(dy, b, low)
        mm_f32(dy, weight, dx, add=add)
        mm_f32(low, a, dx, add=True)
        return
    if not _device_bf16(dy, weight, a, b, dx, low):
        _unsupported("input_gradient", dy, weight, a, b, dx, low)
    _input_gradient(dy, weight, None, a, b, dx, low, add)


def _input_gradient(dy, weight, state, a, b, dx, low, add, epilogue=None, desc=None):
    m, n = dy.shape
    k, r = dx.shape[1], a.shape[0]
    dy, lddy = _rows(dy)
    w = None if weight is None else weight.contiguous()
    a, b = a.contiguous(), b.contiguous()
    target, lowc = _Output(dx), _Contiguous(low)
    if epilogue is not None and (target.buffer is not dx or add):
        raise ValueError("a fused epilogue needs add=False and a unit-stride, 16-byte aligned dx")
    if add and target.buffer is not dx:
        target.buffer.copy_(dx)
    if state is not None and desc is None:
        desc = _native.nf4_descriptor(w, state)
    lib = _native.library()
    ws = _workspace(_query("ct_input_gradient_workspace", m, n, k, r, _native.nf4_kind(desc)), dy.device)
    with _native.device_of(dy):
        status = lib.ct_input_gradient(
            _native.ptr(dy), lddy, None if desc is not None else _native.ptr(w), desc, _native.ptr(a),
            _native.ptr(b), _native.ptr(target.buffer), target.ld, _native.ptr(lowc.buffer), m, n, k, r, int(add),
            None if epilogue is None else ctypes.byref(epilogue), _native.ptr(ws), ws.numel(), _native.stream_of(dy))
    _native.check(status, "ct_input_gradient")
    target.finish()
    lowc.finish()


def parameter_gradients(x, dy, da, db, low, xa, *, add):
    if not x.is_cuda:
        accumulate(da, low.T, x, add=add)
        accumulate(db, dy.T, xa, add=add)
        return
    if not (_device_bf16(x, dy, low, xa) and da.dtype == db.dtype == torch.float32):
        accumulate(da, low.T, x, add=add)
        accumulate(db, dy.T, xa, add=add)
        return
    m, k = x.shape
    n, r = dy.shape[1], low.shape[1]
    x, ldx = _rows(x)
    dy, lddy = _rows(dy)
    low, ldlow = _rows(low)
    xa, ldxa = _rows(xa)
    if not (da.is_contiguous() and db.is_contiguous()):
        accumulate(da, low.T, x, add=add)
        accumulate(db, dy.T, xa, add=add)
        return
    lib = _native.library()
    ws = _workspace(_query("ct_parameter_gradients_workspace", m, n, k, r), x.device)
    with _native.device_of(x):
        status = lib.ct_parameter_gradients(_native.ptr(x), ldx, _native.ptr(dy), lddy, _native.ptr(low), ldlow,
                                             _native.ptr(xa), ldxa, _native.ptr(da), _native.ptr(db), m, n, k, r,
                                             int(add), _native.ptr(ws), ws.numel(), _native.stream_of(x))
    _native.check(status, "ct_parameter_gradients")


# From this many rows ct_input_gradient decodes an NF4 weight into its workspace before the
# dense GEMM (the fused transposing loader loses past one 256-row tile); a group's dx then
# runs as one contraction over the weights decoded side by side (ct_group_input_gradient).
GROUP_DX_ROWS = 257


def _transposable(base):
    """Whether ct_group_input_gradient takes this base: a packed NF4 weight its transposed
    decode accepts, or a dense contiguous bf16 matrix."""
    if base.state is None:
        return base.matrix is not None and base.matrix.dtype == torch.bfloat16 and base.matrix.is_contiguous()
    rows, cols = int(base.state.shape[0]), int(base.state.shape[1])
    return cols % 16 == 0 and rows % 8 == 0 and base.state.blocksize >= 16 and base.weight.data_ptr() % 8 == 0


def group_dx_ready(bases, widths, ranks, rows):
    """Whether the projections' input gradients run as one contraction."""
    return (1 < len(bases) <= _native.CT_GROUP_MAX and rows >= GROUP_DX_ROWS and all(r > 0 for r in ranks)
            and all(n % 8 == 0 for n in widths) and all(_transposable(b) for b in bases))


def stacked_rows(tensors):
    """[t_1; t_2; ...] for contiguous matrices of one width: a view when they are consecutive
    rows of one buffer (the stacked factors group_factors casts into), else a copy."""
    first = tensors[0]
    width, offset, storage = first.shape[1], first.data_ptr(), first.untyped_storage().data_ptr()
    for t in tensors:
        if (not t.is_contiguous() or t.shape[1] != width or t.data_ptr() != offset
                or t.untyped_storage().data_ptr() != storage):
            return torch.cat(tensors)
        offset += t.numel() * t.element_size()
    return first.as_strided((sum(t.shape[0] for t in tensors), width), (width, 1))


def group_input_gradient(bases, dy, widths, ranks, a_stack, bs, dx, low, add):
    """low_i = dy_i b_i and dx (+)= sum_i (dy_i w_i + low_i a_i) for projections that read one
    input (the reference's input_gradient per projection with add=index>0, linear.py:107-122),
    as one contraction rounded once: ct_group_input_gradient. dy = [dy_1 | dy_2 | ...] and low
    = [low_1 | low_2 | ...] are column blocks of two matrices."""
    m, k = dx.shape
    count = len(bases)
    dy, lddy = _rows(dy)
    written, ldlow = _rows(low)
    if written.data_ptr() != low.data_ptr():
        raise ValueError("group_input_gradient: low must be a 16-byte aligned matrix with unit row stride")
    target = _Output(dx)
    if add and target.buffer is not dx:
        target.buffer.copy_(dx)
    descs = [base.desc if base.state is not None else None for base in bases]
    dense = (ctypes.c_void_p * count)(*[None if d is not None else base.matrix.data_ptr()
                                        for base, d in zip(bases, descs)])
    packed = (ctypes.POINTER(_native.NF4Weight) * count)(*[None if d is None else ctypes.pointer(d) for d in descs])
    factors = (ctypes.c_void_p * count)(*[b.contiguous().data_ptr() for b in bs])
    n_arr, r_arr = (ctypes.c_int64 * count)(*widths), (ctypes.c_int64 * count)(*ranks)
    lib = _native.library()
    ws = _workspace(lib.ct_group_input_gradient_workspace(m, count, n_arr, r_arr, k), dx.device)
    with _native.device_of(dx):
        status = lib.ct_group_input_gradient(
            _native.ptr(dy), lddy, count, n_arr, r_arr, dense, packed, _native.ptr(a_stack.contiguous()), factors,
            _native.ptr(target.buffer), target.ld, _native.ptr(low), ldlow, m, k, int(add), _native.ptr(ws),
            ws.numel(), _native.stream_of(dx))
    _native.check(status, "ct_group_input_gradient")
    target.finish()


def group_input_gradient_lead(bases, dy0, tail, widths, ranks, a_stack, bs, dx, add):
    """The same dx and low_i for upstream gradients that arrive as separate tensors
    (linear.py:107-122): dy0 is read in place, tail = [dy_2 | ... | low_1 | low_2 | ...]
    holds the later upstream gradients side by side and receives the low-rank products
    after them (ct_group_input_gradient_lead)."""
    m, k = dx.shape
    count = len(bases)
    dy0, lddy0 = _rows(dy0)
    written, ldtail = _rows(tail)
    if written.data_ptr() != tail.data_ptr():
        raise ValueError("group_input_gradient_lead: tail must be a 16-byte aligned matrix with unit row stride")
    target = _Output(dx)
    if add and target.buffer is not dx:
        target.buffer.copy_(dx)
    descs = [base.desc if base.state is not None else None for base in bases]
    dense = (ctypes.c_void_p * count)(*[None if d is not None else base.matrix.data_ptr()
                                        for base, d in zip(bases, descs)])
    packed = (ctypes.POINTER(_native.NF4Weight) * count)(*[None if d is None else ctypes.pointer(d) for d in descs])
    factors = (ctypes.c_void_p * count)(*[b.contiguous().data_ptr() for b in bs])
    n_arr, r_arr = (ctypes.c_int64 * count)(*widths), (ctypes.c_int64 * count)(*ranks)
    lib = _native.library()
    ws = _workspace(lib.ct_group_input_gradient_lead_workspace(m, count, n_arr, r_arr, k), dx.device)
    with _native.device_of(dx):
        status = lib.ct_group_input_gradient_lead(
            _native.ptr(dy0), lddy0, _native.ptr(tail), ldtail, count, n_arr, r_arr, dense, packed,
            _native.ptr(a_stack.contiguous()), factors, _native.ptr(target.buffer), target.ld, m, k, int(add),
            _native.ptr(ws), ws.numel(), _native.stream_of(dx))
    _native.check(status, "ct_group_input_gradient_lead")
    target.finish()


# From this many rows ct_forward_linear decodes an NF4 weight before its dense GEMM; two
# projections that share an input then run their forward as one GEMM (ct_group_forward).
GROUP_FORWARD_ROWS = 512


def group_forward_ready(bases, widths, ranks, rows, k, biases):
    return (len(bases) == 2 and rows >= GROUP_FORWARD_ROWS and ranks[0] == ranks[1] > 0 and widths[0] % 64 == 0
            and k % 8 == 0 and all(b is None or (b.dtype == torch.bfloat16 and b.is_contiguous()) for b in biases)
            and all(base.state is not None or (base.matrix.dtype == torch.bfloat16 and base.matrix.is_contiguous())
                    for base in bases))


def group_forward(bases, x, b_stack, xa, outputs, biases=(None, None)):
    """out_i = x w_i^T (+ bias_i) + xa_i b_i^T for two projections that read x (forward_linear
    with the stacked xa given, linear.py:72-86) as one GEMM over [w_1; w_2]:
    ct_group_forward. xa = [xa_1 | xa_2]; `outputs` are written in place."""
    m, k = x.shape
    x, ldx = _rows(x)
    xa, ldxa = _rows(xa)
    targets = [_Output(out) for out in outputs]
    descs = [base.desc if base.state is not None else None for base in bases]
    dense = (ctypes.c_void_p * 2)(*[None if d is not None else base.matrix.data_ptr() for base, d in zip(bases, descs)])
    packed = (ctypes.POINTER(_native.NF4Weight) * 2)(*[None if d is None else ctypes.pointer(d) for d in descs])
    n_arr = (ctypes.c_int64 * 2)(*[out.shape[1] for out in outputs])
    out_arr = (ctypes.c_void_p * 2)(*[t.buffer.data_ptr() for t in targets])
    ld_arr = (ctypes.c_int64 * 2)(*[t.ld for t in targets])
    bias_arr = None if all(b is None for b in biases) else \
        (ctypes.c_void_p * 2)(*[None if b is None else _native.ptr(b) for b in biases])
    r = b_stack.shape[1]
    lib = _native.library()
    ws = _workspace(lib.ct_group_forward_workspace(m, 2, n_arr, k, r), x.device)
    with _native.device_of(x):
        status = lib.ct_group_forward(_native.ptr(x), ldx, 2, n_arr, dense, packed, _native.ptr(b_stack.contiguous()),
                                      _native.ptr(xa), ldxa, bias_arr, out_arr, ld_arr, m, k, r, _native.ptr(ws),
                                      ws.numel(), _native.stream_of(x))
    _native.check(status, "ct_group_forward")
    for t in targets:
        t.finish()


def projection_parameters(module):
    weight = module.weight if module.quantized is None else module.quantized.weight
    state = None if module.quantized is None else weight.quant_state
    return (weight, module.lora_A, module.lora_B, module.bias), state


def can_fuse(module, x):
    return (x.is_cuda and module.rank and not (module.bias is not None and module.bias.requires_grad)
            and (module.weight is None or not module.weight.requires_grad)
            and module.lora_A.requires_grad and module.lora_B.requires_grad)


# ----------------------------------------------------------------------------- grouped autograd
class _Base:
    """The frozen base weight of one projection as the HIP GEMMs consume it.

    A packed NF4 weight whose layout the fused loaders accept is handed to the entry points
    packed: below 512 rows (257 for dx) every GEMM decodes it tile by tile into LDS, from
    there on the entry point decodes it once into its workspace (both bit-identical to
    `materialize`).
    Anything else is materialised here once, as the reference does (linear.py:70,107).
    """

    def __init__(self, weight, state, dtype):
        self.weight, self.state, self.matrix, self.desc = weight, None, None, None
        if state is not None and weight.is_cuda and dtype == torch.bfloat16 and weight.dtype == torch.uint8 \
                and weight.is_contiguous() and state.quant_type == "nf4":
            self.desc = _native.nf4_fused_descriptor(weight, state)
            if self.desc is not None:
                self.state = state
        if self.state is None:
            self.matrix = materialize(weight, state, dtype)
        self.rows = int(state.shape[0]) if state is not None else weight.shape[0]

    def forward(self, x, a, b, bias, out, xa, xa_given=False, epilogue=None):
        """out = x w^T + (x a^T) b^T (+ bias). Device only: with xa_given, xa holds x a^T
        already; `epilogue` is an elementwise step fused into the output."""
        if xa_given or epilogue is not None:
            _forward(x, self.matrix if self.state is None else self.weight, self.state, a, b, bias, out, xa,
                     xa_given, epilogue, self.desc)
        elif self.state is None:
            forward_linear(x, self.matrix, a, b, bias=bias, out=out, xa=xa)
        else:
            _forward(x, self.weight, self.state, a, b, bias, out, xa, desc=self.desc)

    def input_gradient(self, dy, a, b, dx, low, add, epilogue=None):
        if epilogue is not None:
            _input_gradient(dy, self.matrix if self.state is None else self.weight, self.state, a, b, dx, low, add,
                            epilogue, self.desc)
        elif self.state is None:
            input_gradient(dy, self.matrix, a, b, dx, low, add=add)
        else:
            _input_gradient(dy, self.weight, self.state, a, b, dx, low, add, desc=self.desc)


# Rows per tile of a projection group called without a tile: the reference's bound
# (linear.py:63), which keeps every row-proportional workspace at most [4096, ...] wide.
DEFAULT_TILE = 4096
_KEEP_BUDGET = contextvars.ContextVar("causal_tuner_projection_budget", default=0)


@contextlib.contextmanager
def projection_budget(nbytes):
    """Let projection groups called without a tile inside this block spend up to `nbytes`
    of device memory on row-proportional state: when a group's whole input fits, it runs
    all rows as one tile and keeps each projection's forward xa = x a^T for its backward
    instead of recomputing it, and with it the compute-dtype LoRA factors (a fixed
    rank x (in + out) elements per projection) instead of casting them again. The default
    budget is 0: 4096-row tiles and nothing saved
    but the input and the parameters, as in the reference (linear.py:59-130). The budget
    is read when the forward runs; the backward follows the forward's choice."""
    if nbytes < 0:
        raise ValueError("The projection budget must be non-negative")
    token = _KEEP_BUDGET.set(int(nbytes))
    try:
        yield
    finally:
        _KEEP_BUDGET.reset(token)


def group_row_bytes(parameters, count, element, head_dim):
    """Device bytes per input row that one whole-input tile of a group holds across its
    forward and backward: every kept xa, the backward's [rows, r] gradient product and,
    with rotary outputs, the inverse-rotation scratch of a q or k gradient."""
    ranks = [parameters[4*i+1].shape[0] for i in range(count)]
    widths = [parameters[4*i+2].shape[0] for i in range(min(count, 2))] if head_dim else [0]
    return element * (sum(ranks) + max(ranks, default=0) + max(widths, default=0))


def _plan_rows(rows, tile, budget, row_bytes):
    """(rows per tile, keep xa): an explicit tile is the reference's tiled path; without one
    the whole input is one tile when the budget covers it, else DEFAULT_TILE rows."""
    if tile:
        return tile, False
    if 0 < rows and rows * row_bytes <= budget:
        return rows, True
    return DEFAULT_TILE, False


def param_run(ranks, widths, k):
    """(first, stop) of the projections after the first whose dA/dB go in one call, or None.
    Their dA is [low_i ...]^T x over the stacked ranks; their dB^T = [xa_i ...]^T [dy_i ...]
    also forms the cross products xa_i^T dy_j (i != j), which are dropped, so a run is
    taken when those stay under a tenth of its useful products: narrow outputs such as k and
    v (C3: 2 x 128 columns beside a 4096-long reduction, 3% extra)."""
    count = len(ranks)
    if count < 3 or len(set(ranks[1:])) != 1 or ranks[1] <= 0:
        return None
    members, n_sum = count - 1, sum(widths[1:])
    if 10 * (members - 1) * n_sum > members * k + n_sum:
        return None
    return 1, count


def _adjacent(views):
    """One view over column slices of one matrix that follow each other, or None."""
    first = views[0]
    element, storage = first.element_size(), first.untyped_storage().data_ptr()
    offset = 0
    for view in views:
        if (view.stride() != first.stride() or view.data_ptr() != first.data_ptr() + offset * element
                or view.untyped_storage().data_ptr() != storage):
            return None
        offset += view.shape[1]
    return first.as_strided((first.shape[0], offset), first.stride())


class _LoRAGroup(torch.autograd.Function):
    """Projections sharing one input (linear.py:59-130), in tiles of rows.

    Projections of one rank that read the same input get their xa = x a_i^T from one GEMM
    over the stacked factors per tile (`group_factors`). Under a projection budget that
    covers the whole input (`projection_budget`) the group runs one tile and saves each
    projection's xa for the backward; otherwise it saves only the input and the
    parameters and the backward recomputes xa tile by tile. The backward visits tiles in
    order and, inside a tile, the projections in order, so dx accumulates over the
    projections (add=index>0) and dA/dB over the tiles (add=start>0) in the reference's
    sequence."""

    @staticmethod
    def forward(ctx, x, dtype, tile, states, cosine, sine, head_dim, residual, *parameters):
        count = len(states)
        flat = _matrix_of(x).to(dtype)
        total = flat.shape[0]
        element = dtype.itemsize
        step, keep = _plan_rows(total, tile, _KEEP_BUDGET.get(),
                                group_row_bytes(parameters, count, element, head_dim))
        ctx.dtype, ctx.states, ctx.head_dim, ctx.step = dtype, states, head_dim, step
        factors, stack = group_factors(parameters, count, dtype, x)
        bases = [_Base(parameters[4*i], state, dtype) for i, state in enumerate(states)]
        biases = [None if parameters[4*i+3] is None else parameters[4*i+3].to(dtype) for i in range(count)]
        outputs = [torch.empty((total, base.rows), device=x.device, dtype=dtype) for base in bases]
        ranks = [parameters[4*i+1].shape[0] for i in range(count)]
        span = min(step, total)
        # xa of every projection for the rows of one tile (all rows when kept), as column
        # slices of one buffer so a stacked GEMM fills them together.
        xa = torch.empty((total if keep else span, sum(ranks)), device=x.device, dtype=dtype)
        columns = [xa] if count == 1 else [xa[:, sum(ranks[:i]):sum(ranks[:i+1])] for i in range(count)]
        # The rotation of q/k (core_cuda.py:192-200) and the residual add (linear.py:90-91)
        # run in the GEMM epilogue when the operands allow it, else as separate passes.
        rotated = min(count, 2) if head_dim else 0
        trig = None
        if rotated:
            half = cosine.shape[-1]
            trig = tuple(value.reshape(-1, half) if value.numel() == total * half else None
                         for value in (cosine, sine))
        # the fused step reads [rows, half] tables with a row pitch of half and one dtype;
        # anything else takes the separate pass, which validates the tables itself
        rope_fused = bool(rotated) and trig[0] is not None and trig[1] is not None and \
            trig[0].is_contiguous() and trig[1].is_contiguous() and trig[0].dtype == trig[1].dtype and \
            fusable(*outputs[:rotated]) and all(out.shape[1] % head_dim == 0 for out in outputs[:rotated])
        residual_flat = None if residual is None else residual.reshape(total, -1)
        residual_fused = residual_flat is not None and not rotated and fusable(outputs[0], residual_flat)
        # Two projections of one rank without steps (gate and up) share one grid of output
        # tiles from GROUP_FORWARD_ROWS rows: one partial last round instead of two.
        paired = (stack is not None and not rotated and residual is None and x.is_cuda and dtype == torch.bfloat16
                  and group_forward_ready(bases, [out.shape[1] for out in outputs], ranks, span, flat.shape[1],
                                          biases))
        if paired:
            b_stack = stacked_rows([factors[1], factors[3]])
        # Otherwise the last two of three (k and v beside q), when neither is rotated, share
        # one grid the same way (C3: 2 x 128 columns as one grid of 64 x 64 tiles, 43 us
        # instead of 71 us for two launches, measured on MI355X).
        tail = (not paired and count == 3 and stack is not None and not rotated and x.is_cuda and dtype == torch.bfloat16
                and group_forward_ready(bases[1:], [out.shape[1] for out in outputs[1:]], ranks[1:], span,
                                        flat.shape[1], biases[1:]))
        if tail:
            tail_b = stacked_rows([factors[3], factors[5]])
        whole = step >= total   # one tile over every row: the tensors themselves, no row views
        for start in range(0, total, step):
            part = _cut(flat, slice(start, start+step), whole)
            n_part = part.shape[0]
            rows = slice(start, start+n_part) if keep else slice(0, n_part)
            window = slice(start, start+n_part)
            if stack is not None:
                _low_rank(part, stack, _cut(xa, rows, whole), transpose=True)
            if paired and n_part > 64:
                group_forward(bases, part, b_stack, _cut(xa, rows, whole), [_cut(out, window, whole) for out in outputs],
                              biases)
                continue
            for index, base in enumerate(bases):
                if tail and index == 1 and n_part > 64:
                    group_forward(bases[1:], part, tail_b, xa[rows, ranks[0]:ranks[0] + ranks[1] + ranks[2]],
                                  [_cut(out, window, whole) for out in outputs[1:]], biases[1:])
                    break
                epilogue = None
                if rope_fused and index < rotated:
                    epilogue = _native.epilogue(_native.CT_EPI_ROPE, n_part,
                                                rotary=(trig[0][window], trig[1][window], head_dim))
                elif residual_fused and index == 0:
                    epilogue = _native.epilogue(_native.CT_EPI_RESIDUAL, n_part, in0=residual_flat[window])
                base.forward(part, factors[2*index], factors[2*index+1], biases[index],
                             _cut(outputs[index], window, whole), _cut(columns[index], rows, whole),
                             xa_given=stack is not None, epilogue=epilogue)
        # Under a projection budget the backward also reuses the compute-dtype factors
        # (the reference casts them again, linear.py:108: the same values).
        kept = [*columns, *factors] if keep else []
        ctx.kept = len(kept)
        # bases that hold no decoded copy (packed NF4 for the fused loaders) serve the backward too
        ctx.bases = bases if all(base.matrix is None for base in bases) else None
        ctx.save_for_backward(x, cosine, sine, *parameters, *kept)
        del factors, stack, bases, xa, columns, kept
        if x.dim() != 2:
            outputs = [out.reshape(*x.shape[:-1], out.shape[1]) for out in outputs]
        if rotated and not rope_fused:
            from .core_cuda import rotate_owned_qk
            rotate_owned_qk(outputs[0], outputs[1], cosine, sine, head_dim)
        if residual is not None and not residual_fused:
            outputs[0].add_(residual)
        return tuple(outputs)

    @staticmethod
    def backward(ctx, *grad_outputs):
        x, cosine, sine, *rest = ctx.saved_tensors
        count = len(ctx.states)
        parameters, kept = rest[:4*count], rest[4*count:4*count+count]
        saved_factors = rest[4*count+count:]
        flat = _matrix_of(x).to(ctx.dtype)
        total = flat.shape[0]
        dx = torch.empty_like(flat) if ctx.needs_input_grad[0] else None
        if ctx.head_dim:
            cosine, sine = (value.reshape(-1, value.shape[-1]) for value in (cosine, sine))
        step, span = ctx.step, min(ctx.step, total)
        if saved_factors:
            factors, stack = list(saved_factors), None
        else:
            factors, stack = group_factors(parameters, count, ctx.dtype, x)
        if dx is None:
            bases = [None] * count
        elif ctx.bases is not None:
            bases = ctx.bases
        else:
            bases = [_Base(parameters[4*i], state, ctx.dtype) for i, state in enumerate(ctx.states)]
        ranks = [parameters[4*i+1].shape[0] for i in range(count)]
        signals = [_matrix_of(grad).to(ctx.dtype) for grad in grad_outputs]
        allocate = torch.empty_like if total else torch.zeros_like
        gradients = [(allocate(parameters[4*i+1]), allocate(parameters[4*i+2])) for i in range(count)]
        xa = None if kept else torch.empty((span, sum(ranks)), device=x.device, dtype=ctx.dtype)
        rotated = min(count, 2) if ctx.head_dim else 0
        widths = [signal.shape[1] for signal in signals]
        # From GROUP_DX_ROWS rows the group's input gradient is one contraction
        # (ct_group_input_gradient_lead): the first upstream gradient read in place (or
        # rotated back into a buffer of its own), the later ones side by side ahead of the
        # low-rank products in one tail matrix, so dx is rounded once instead of after every
        # projection and k and v add no pass over dx.
        # The later upstream gradients arrive as separate tensors: the ones not rotated on
        # the way in are copied into the tail, which pays only while the copies move fewer
        # bytes than the dx passes the one contraction saves (one read and write of dx per
        # projection after the first): q/k/v, not two wide projections such as gate and up.
        copied = sum(widths[max(rotated, 1):])
        grouped = (dx is not None and x.is_cuda and ctx.dtype == torch.bfloat16
                   and group_dx_ready(bases, widths, ranks, span) and copied < (count - 1) * flat.shape[1])
        if grouped:
            n_tail = sum(widths[1:])
            tail = torch.empty((span, n_tail + sum(ranks)), device=x.device, dtype=ctx.dtype)
            low = tail[:, n_tail:]
            head = torch.empty((span, widths[0]), device=x.device, dtype=ctx.dtype) if rotated else None
            a_stack = stack if stack is not None else stacked_rows([factors[2*i] for i in range(count)])
            columns = [None] + [slice(sum(widths[1:i]), sum(widths[1:i+1])) for i in range(1, count)]
            low_columns = [slice(sum(ranks[:i]), sum(ranks[:i+1])) for i in range(count)]
        else:
            low = torch.empty((span, max(ranks)), device=x.device, dtype=ctx.dtype)
        scratch = (torch.empty(span * max(signals[i].shape[1] for i in range(rotated)), device=x.device,
                               dtype=ctx.dtype) if rotated and not grouped else None)
        run = param_run(ranks, widths, flat.shape[1]) if grouped and total else None
        if run is not None and kept:
            kept_run = _adjacent(kept[run[0]:run[1]])
            run = None if kept_run is None else run
        if run is not None:
            # the run's dA (row blocks) and dB^T (diagonal blocks) into two buffers, copied
            # out into each projection's gradients after the last tile
            r_lo, r_hi = sum(ranks[:run[0]]), sum(ranks[:run[1]])
            n_lo, n_hi = sum(widths[:run[0]]), sum(widths[:run[1]])
            run_da = torch.empty((r_hi - r_lo, flat.shape[1]), device=x.device, dtype=gradients[0][0].dtype)
            run_db = torch.empty((n_hi - n_lo, r_hi - r_lo), device=x.device, dtype=gradients[0][1].dtype)
        whole = step >= total   # one tile over every row: the tensors themselves, no row views
        for start in range(0, total, step):
            part = _cut(flat, slice(start, start+step), whole)
            n_part = part.shape[0]
            if not kept:
                if stack is not None:
                    _low_rank(part, stack, xa[:n_part], transpose=True)
                else:
                    for index in range(count):
                        columns_xa = slice(sum(ranks[:index]), sum(ranks[:index+1]))
                        _low_rank(part, factors[2*index], xa[:n_part, columns_xa], transpose=True)
            if grouped:
                tile_signals = []
                for index in range(count):
                    signal = signals[index][start:start+n_part]
                    if index == 0:   # read in place unless rotated back into a buffer of its own
                        target = head[:n_part] if rotated else None
                    else:
                        target = tail[:n_part, columns[index]]
                    if index < rotated:
                        from .core_cuda import inverse_rope_tile
                        signal = inverse_rope_tile(signal, cosine[start:start+n_part],
                                                   sine[start:start+n_part], ctx.head_dim, target)
                    elif index > 0:
                        target.copy_(signal)
                        signal = target
                    tile_signals.append(signal)
                group_input_gradient_lead(bases, tile_signals[0], tail[:n_part], widths, ranks, a_stack,
                                          [factors[2*i+1] for i in range(count)], dx[start:start+n_part], False)
                for index in range(count if run is None else run[0]):
                    inputs = (kept[index][start:start+n_part] if kept else
                              xa[:n_part, sum(ranks[:index]):sum(ranks[:index+1])])
                    parameter_gradients(part, tile_signals[index], *gradients[index],
                                        low[:n_part, low_columns[index]], inputs, add=start > 0)
                if run is not None:
                    inputs = kept_run[start:start+n_part] if kept else xa[:n_part, r_lo:r_hi]
                    parameter_gradients(part, tail[:n_part, n_lo - widths[0]:n_hi - widths[0]], run_da, run_db,
                                        low[:n_part, r_lo:r_hi], inputs, add=start > 0)
                continue
            window = slice(start, start+n_part)
            for index in range(count):
                a, b = factors[2*index], factors[2*index+1]
                signal = _cut(signals[index], window, whole)
                if index < rotated:
                    from .core_cuda import inverse_rope_tile
                    target = scratch[:signal.numel()].view_as(signal)
                    signal = inverse_rope_tile(signal, cosine[window], sine[window], ctx.head_dim, target)
                grad_low = low if whole and low.shape[1] == ranks[index] else low[:n_part, :ranks[index]]
                if dx is not None:
                    bases[index].input_gradient(signal, a, b, _cut(dx, window, whole), grad_low, index > 0)
                else:
                    _low_rank(signal, b, grad_low, transpose=False)
                inputs = (_cut(kept[index], window, whole) if kept else
                          xa[:n_part, sum(ranks[:index]):sum(ranks[:index+1])])
                parameter_gradients(part, signal, *gradients[index], grad_low, inputs, add=start > 0)
        if run is not None:
            for index in range(*run):
                cols = slice(sum(widths[:index]) - n_lo, sum(widths[:index+1]) - n_lo)
                rows = slice(sum(ranks[:index]) - r_lo, sum(ranks[:index+1]) - r_lo)
                # dA: consecutive rows of the run's output, handed out as contiguous views
                gradients[index] = (run_da[rows], gradients[index][1])
                gradients[index][1].copy_(run_db[cols, rows])
        del bases, factors, stack
        results = [value for da, db in gradients for value in (None, da, db, None)]
        residual_grad = grad_outputs[0] if ctx.needs_input_grad[7] else None
        if dx is not None and x.dim() != 2:
            dx = dx.reshape_as(x)
        return (None if dx is None else dx.to(x.dtype), None, None, None, None, None, None,
                residual_grad, *results)


def _matrix_of(t):
    """t as [rows, last dimension] (itself when it is a matrix already)."""
    return t if t.dim() == 2 else t.reshape(-1, t.shape[-1])


def _cut(t, rows, whole):
    """t[rows], or t itself when one tile spans all of its rows (saves a view per call)."""
    return t if whole else t[rows]


def _low_rank(x, factor, out, *, transpose):
    """out = x factor^T (transpose) or x factor: the rank-r products torch.mm computes in
    the reference (linear.py:124-125, mlp_cuda.py:134,140)."""
    if not x.is_cuda:
        torch.mm(x, factor.T if transpose else factor, out=out)
        return
    if _device_f32(x, factor, out):
        mm_f32(x, factor.T if transpose else factor, out)
        return
    if not _device_bf16(x, factor, out):
        _unsupported("low-rank product", x, factor, out)
    m, k = x.shape
    r = out.shape[1]
    x, ldx = _rows(x)
    factor = factor.contiguous()
    target = _Output(out)
    lib = _native.library()
    ws = _workspace(_query("ct_gemm_workspace", m, r, k, 0, int(transpose), _native.CT_BF16), x.device)
    with _native.device_of(x):
        status = lib.ct_gemm(_native.ptr(x), ldx, 0, _native.ptr(factor), k if transpose else r, int(transpose),
                             _native.ptr(target.buffer), target.ld, _native.CT_BF16, None, 0, m, r, k,
                             _native.ptr(ws), ws.numel(), _native.stream_of(x))
    _native.check(status, "ct_gemm")
    target.finish()


def project_group(modules, x, tile=0, *, rotary=None, residual=None):
    if residual is not None:
        if len(modules) != 1:
            raise ValueError("Residual fusion requires one output projection")
        shape = (*x.shape[:-1], len(modules[0].lora_B))
        if residual.shape != shape or residual.dtype != modules[0].compute_dtype:
            return (project_group(modules, x, tile, rotary=rotary)[0]+residual,)
    parameters, states = [], []
    for module in modules:
        values, state = projection_parameters(module)
        parameters.extend(values)
        states.append(state)
    cosine, sine, head_dim = (None, None, 0) if rotary is None else rotary
    if rotary is not None:
        cosine, sine = cosine.contiguous(), sine.contiguous()
    return _LoRAGroup.apply(x, modules[0].compute_dtype, tile, tuple(states), cosine, sine, head_dim, residual,
                            *parameters)
