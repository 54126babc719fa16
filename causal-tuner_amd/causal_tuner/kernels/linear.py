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

The bf16 path is the device path. CPU tensors keep the reference's torch semantics (its
unfused CPU route); device tensors of another compute dtype raise NotImplementedError,
except in `accumulate`, which keeps the reference's addmm for operands that are not bf16
(the fp32 projection loss uses it; linear.py:22-24).
"""

import ctypes

import torch

from . import _native


# ----------------------------------------------------------------------------- helpers
def _device_bf16(*tensors):
    return all(t.is_cuda and t.dtype == torch.bfloat16 for t in tensors if t is not None)


def _unsupported(what, *tensors):
    dtypes = sorted({str(t.dtype) for t in tensors if t is not None})
    raise NotImplementedError(f"{what}: the HIP path computes in bfloat16 on the device (got {', '.join(dtypes)})")


def _aligned(t):
    return t.data_ptr() % 16 == 0


def _rows(t):
    """(tensor, leading dimension) of a matrix with unit stride along its rows; a view whose
    base is not 16-byte aligned is copied so the kernels can use 16-byte loads."""
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


def _workspace(nbytes, device):
    """Caller-owned scratch for split reductions (the kernels never allocate); torch's
    caching allocator makes the per-call allocation cheap."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


class _Output:
    """A caller's output view; kernels write a contiguous stand-in when the view is strided."""

    def __init__(self, target):
        self.target = target
        ok = (target.dim() == 2 and target.stride(1) == 1 and target.stride(0) >= target.shape[1]
              and _aligned(target))
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
    ranks = {len(tensors[2*i]) for i in range(shared)}
    if (shared > 1 and x.is_cuda and dtype == torch.bfloat16 and len(ranks) == 1 and ranks != {0}
            and len({tensors[2*i].shape[1] for i in range(shared)}) == 1):
        r = ranks.pop()
        stack = torch.empty((shared * r, tensors[0].shape[1]), dtype=dtype, device=x.device)
        outputs = [stack[i*r:(i+1)*r] if j == 0 and i < shared else None for i in range(count) for j in (0, 1)]
        return cast_all(tensors, dtype, outputs), stack
    return cast_all(tensors, dtype), None


def _shared_xa(flat, stack):
    """x [a_1; a_2; ...]^T for a group: one ct_gemm, column slice i is projection i's xa."""
    xa = torch.empty((len(flat), len(stack)), dtype=flat.dtype, device=flat.device)
    _low_rank(flat, stack, xa, transpose=True)
    return xa


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
        ws = _workspace(lib.ct_accumulate_workspace(p, q, j), output.device)
        with _native.device_of(output):
            status = lib.ct_accumulate(_native.ptr(target.buffer), target.ld, _native.ptr(lt), ldl, tl,
                                       _native.ptr(rt), ldr, tr, p, q, j, int(add) if target.buffer is output else
                                       0, _native.ptr(ws), ws.numel(), _native.stream_of(output))
        _native.check(status, "ct_accumulate")
        if target.buffer is not output:
            output.copy_(target.buffer + output if add else target.buffer)
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
    if not _device_bf16(x, weight, a, b, out, xa, bias):
        _unsupported("forward_linear", x, weight, a, b, out, xa, bias)
    _forward(x, weight, None, a, b, bias, out, xa)


def _forward(x, weight, state, a, b, bias, out, xa, xa_given=False):
    """ct_forward_linear; with xa_given, xa (a row-major view, e.g. a column slice of a
    group's shared x [a_1; a_2; ...]^T) already holds x a^T and is only read."""
    m, k = x.shape
    n, r = out.shape[1], a.shape[0]
    x, ldx = _rows(x)
    w = None if weight is None else weight.contiguous()
    a, b = a.contiguous(), b.contiguous()
    bias = None if bias is None else bias.contiguous()
    target, low = _Output(out), _Output(xa)
    if xa_given and low.buffer is not xa:
        low.buffer.copy_(xa)
    desc = None if state is None else _native.nf4_descriptor(w, state)
    lib = _native.library()
    ws = _workspace(lib.ct_forward_linear_workspace(m, n, k, r, _native.nf4_kind(desc)), x.device)
    with _native.device_of(x):
        status = lib.ct_forward_linear(
            _native.ptr(x), ldx, None if desc is not None else _native.ptr(w), desc, _native.ptr(a),
            _native.ptr(b), _native.ptr(bias), _native.ptr(target.buffer), target.ld, _native.ptr(low.buffer),
            low.ld, int(bool(xa_given)), m, n, k, r, _native.ptr(ws), ws.numel(), _native.stream_of(x))
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
    if not _device_bf16(dy, weight, a, b, dx, low):
        _unsupported("input_gradient", dy, weight, a, b, dx, low)
    _input_gradient(dy, weight, None, a, b, dx, low, add)


def _input_gradient(dy, weight, state, a, b, dx, low, add):
    m, n = dy.shape
    k, r = dx.shape[1], a.shape[0]
    dy, lddy = _rows(dy)
    w = None if weight is None else weight.contiguous()
    a, b = a.contiguous(), b.contiguous()
    target, lowc = _Output(dx), _Contiguous(low)
    if add and target.buffer is not dx:
        target.buffer.copy_(dx)
    desc = None if state is None else _native.nf4_descriptor(w, state)
    lib = _native.library()
    ws = _workspace(lib.ct_input_gradient_workspace(m, n, k, r, _native.nf4_kind(desc)), dy.device)
    with _native.device_of(dy):
        status = lib.ct_input_gradient(
            _native.ptr(dy), lddy, None if desc is not None else _native.ptr(w), desc, _native.ptr(a),
            _native.ptr(b), _native.ptr(target.buffer), target.ld, _native.ptr(lowc.buffer), m, n, k, r, int(add),
            _native.ptr(ws), ws.numel(), _native.stream_of(dy))
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
    ws = _workspace(lib.ct_parameter_gradients_workspace(m, n, k, r), x.device)
    with _native.device_of(x):
        status = lib.ct_parameter_gradients(_native.ptr(x), ldx, _native.ptr(dy), lddy, _native.ptr(low), ldlow,
                                             _native.ptr(xa), ldxa, _native.ptr(da), _native.ptr(db), m, n, k, r,
                                             int(add), _native.ptr(ws), ws.numel(), _native.stream_of(x))
    _native.check(status, "ct_parameter_gradients")


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
    packed: below 512 rows every GEMM decodes it tile by tile into LDS, from 512 rows on the
    entry point decodes it once into its workspace (both bit-identical to `materialize`).
    Anything else is materialised here once, as the reference does (linear.py:70,107).
    """

    def __init__(self, weight, state, dtype):
        self.weight, self.state, self.matrix = weight, None, None
        if state is not None and weight.is_cuda and dtype == torch.bfloat16 and weight.dtype == torch.uint8 \
                and weight.is_contiguous() and state.quant_type == "nf4":
            desc = _native.nf4_descriptor(weight, state)
            if _native.library().ct_nf4_fused_supported(desc) == 1:
                self.state = state
        if self.state is None:
            self.matrix = materialize(weight, state, dtype)
        self.rows = int(state.shape[0]) if state is not None else len(weight)

    def forward(self, x, a, b, bias, out, xa, xa_given=False):
        if xa_given:   # device path only: xa holds x a^T already
            _forward(x, self.matrix if self.state is None else self.weight, self.state, a, b, bias, out, xa, True)
        elif self.state is None:
            forward_linear(x, self.matrix, a, b, bias=bias, out=out, xa=xa)
        else:
            _forward(x, self.weight, self.state, a, b, bias, out, xa)

    def input_gradient(self, dy, a, b, dx, low, add):
        if self.state is None:
            input_gradient(dy, self.matrix, a, b, dx, low, add=add)
        else:
            _input_gradient(dy, self.weight, self.state, a, b, dx, low, add)


class _LoRAGroup(torch.autograd.Function):
    """Projections sharing one input (linear.py:59-130). Saves the input and parameters and,
    when one tile covers all rows, each projection's forward xa = x a^T ([rows, r], 4 MB at
    8192 x 256 in bf16), which the reference recomputes in the backward (linear.py:124-125):
    the backward then reads the same values instead of running the rank-r GEMMs again.

    Without an explicit tile the backward runs each projection over all rows at once (the
    rank-r workspaces are [rows, r]); an explicit tile bounds them as in the reference and
    keeps its recompute."""

    @staticmethod
    def forward(ctx, x, dtype, tile, states, cosine, sine, head_dim, residual, *parameters):
        ctx.dtype, ctx.tile, ctx.states = dtype, tile, states
        ctx.head_dim = head_dim
        flat = x.reshape(-1, x.shape[-1]).to(dtype)
        outputs = []
        step = tile or max(len(flat), 1)
        rows = min(step, len(flat))
        factors, stack = group_factors(parameters, len(states), dtype, x)
        # One tile over all rows: the projections' xa come from one GEMM over the stacked
        # factors (the same products; the fp32 sums may be split differently than in
        # separate launches, so a value can differ by one bf16 rounding).
        shared = _shared_xa(flat, stack) if stack is not None and 0 < len(flat) <= step else None
        kept = []   # each projection's xa over all rows, for the backward
        for index, state in enumerate(states):
            weight, a, b, bias = parameters[index*4:index*4+4]
            base, ac, bc = _Base(weight, state, dtype), factors[2*index], factors[2*index+1]
            bias = None if bias is None else bias.to(dtype)
            out = torch.empty((len(flat), base.rows), device=x.device, dtype=dtype)
            if shared is not None:
                r = len(a)
                kept.append(shared[:, index*r:(index+1)*r])
                base.forward(flat, ac, bc, bias, out, kept[-1], xa_given=True)
            else:
                low = torch.empty((rows, len(a)), device=x.device, dtype=dtype)
                for start in range(0, len(flat), step):
                    part = flat[start:start+step]
                    base.forward(part, ac, bc, bias, out[start:start+step], low[:len(part)])
                kept.append(low)
                del low
            outputs.append(out.reshape(*x.shape[:-1], base.rows))
            del base, ac, bc
        if not 0 < len(flat) <= step:
            kept = []   # tiled (xa of the last tile only) or empty: the backward recomputes
        ctx.kept = len(kept)
        ctx.save_for_backward(x, cosine, sine, *parameters, *kept)
        del factors, stack, shared, kept
        if head_dim:
            from .core_cuda import rotate_owned_qk
            rotate_owned_qk(outputs[0], outputs[1], cosine, sine, head_dim)
        if residual is not None:
            outputs[0].add_(residual)
        return tuple(outputs)

    @staticmethod
    def backward(ctx, *grad_outputs):
        x, cosine, sine, *parameters = ctx.saved_tensors
        kept = parameters[len(parameters)-ctx.kept:] if ctx.kept else None
        parameters = parameters[:len(parameters)-ctx.kept]
        flat = x.reshape(-1, x.shape[-1]).to(ctx.dtype)
        dx = torch.empty_like(flat) if ctx.needs_input_grad[0] else None
        if ctx.head_dim:
            cosine, sine = (value.reshape(-1, value.shape[-1]) for value in (cosine, sine))
        step = ctx.tile or max(len(flat), 1)
        rows = min(step, len(flat))
        rotary = (torch.empty(rows*max(len(b) for b in parameters[2:8:4]), device=x.device, dtype=ctx.dtype)
                  if ctx.head_dim else None)
        results = []
        factors, stack = group_factors(parameters, len(ctx.states), ctx.dtype, x)
        shared = (_shared_xa(flat, stack) if kept is None and stack is not None and 0 < len(flat) <= step
                  else None)
        for index, (state, grad) in enumerate(zip(ctx.states, grad_outputs)):
            weight, a, b, _ = parameters[index*4:index*4+4]
            base = _Base(weight, state, ctx.dtype) if dx is not None else None
            ac, bc = factors[2*index], factors[2*index+1]
            dy = grad.reshape(-1, grad.shape[-1]).to(ctx.dtype)
            allocate = torch.empty_like if len(flat) else torch.zeros_like
            da, db = allocate(a), allocate(b)
            low = torch.empty((rows, len(a)), device=x.device, dtype=ctx.dtype)
            xa = (kept[index] if kept is not None else shared[:, index*len(a):(index+1)*len(a)] if shared is not None
                  else torch.empty((rows, len(a)), device=x.device, dtype=ctx.dtype))
            rotate = ctx.head_dim and index < 2
            for start in range(0, len(flat), step):
                stop = start+step
                signal = dy[start:stop]
                if rotate:
                    from .core_cuda import inverse_rope_tile
                    target = rotary[:signal.numel()].view_as(signal)
                    signal = inverse_rope_tile(signal, cosine[start:stop], sine[start:stop], ctx.head_dim, target)
                part_low, part_xa = low[:len(signal)], xa[:len(signal)]
                if dx is not None:
                    base.input_gradient(signal, ac, bc, dx[start:stop], part_low, index > 0)
                else:
                    _low_rank(signal, bc, part_low, transpose=False)
                if shared is None and kept is None:
                    _low_rank(flat[start:stop], ac, part_xa, transpose=True)
                parameter_gradients(flat[start:stop], signal, da, db, part_low, part_xa, add=start > 0)
            results.extend((None, da, db, None))
            del base, ac, bc, dy
        residual_grad = grad_outputs[0] if ctx.needs_input_grad[7] else None
        return (None if dx is None else dx.reshape_as(x).to(x.dtype), None, None, None, None, None, None,
                residual_grad, *results)


def _low_rank(x, factor, out, *, transpose):
    """out = x factor^T (transpose) or x factor: the rank-r products torch.mm computes in
    the reference (linear.py:124-125, mlp_cuda.py:134,140)."""
    if not x.is_cuda:
        torch.mm(x, factor.T if transpose else factor, out=out)
        return
    if not _device_bf16(x, factor, out):
        _unsupported("low-rank product", x, factor, out)
    m, k = x.shape
    r = out.shape[1]
    x, ldx = _rows(x)
    factor = factor.contiguous()
    target = _Output(out)
    lib = _native.library()
    ws = _workspace(lib.ct_gemm_workspace(m, r, k, 0, int(transpose), _native.CT_BF16), x.device)
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
