"""ctypes binding of the C ABI in include/causal_tuner_hip.h (lib/libcausal_tuner_hip.so).

torch is imported first so that the library's libamdhip64.so.7 dependency resolves to the
HIP runtime torch already mapped; the streams and device pointers passed across the
boundary therefore belong to the same runtime. A missing library raises RuntimeError:
there is no fallback.
"""

import contextlib
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_LIBRARY = os.path.normpath(os.path.join(_HERE, "..", "..", "lib", "libcausal_tuner_hip.so"))

CT_F32, CT_F16, CT_BF16 = 0, 1, 2
CT_CAST_MAX = 16  # tensors per ct_cast_f32_bf16 call (include/causal_tuner_hip.h)
CT_STATIC_SCRATCH_BYTES = 64 << 20  # scratch of ct_forward_linear_static per GPU
CT_GROUP_MAX = 8  # projections per ct_group_input_gradient call
CT_PROF_FWD_GEMM, CT_PROF_DX_GEMM, CT_PROF_DEQUANT, CT_PROF_PARAM, CT_PROF_LOWRANK = 1, 2, 4, 8, 16
DTYPE_CODES = {torch.float32: CT_F32, torch.float16: CT_F16, torch.bfloat16: CT_BF16}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32


class NF4Weight(ctypes.Structure):
    """Mirror of `ct_nf4_weight`: the QuantState fields the decoder reads."""

    _fields_ = [
        ("packed", _P), ("absmax", _P), ("code", _P), ("code2", _P), ("absmax2", _P), ("offset", _P),
        ("rows", _I64), ("cols", _I64), ("blocksize", _I32), ("blocksize2", _I32), ("nested", _I32),
        ("storage_dtype", _I32),
    ]


CT_EPI_NONE, CT_EPI_RESIDUAL, CT_EPI_SILU, CT_EPI_DSILU, CT_EPI_ROPE = 0, 1, 2, 3, 4


class Epilogue(ctypes.Structure):
    """Mirror of `ct_epilogue`: an elementwise step on a projection's bf16 output."""

    _fields_ = [
        ("kind", _I32), ("trig_dtype", _I32), ("in0", _P), ("ld_in0", _I64), ("in1", _P), ("ld_in1", _I64),
        ("out0", _P), ("ld_out0", _I64), ("out1", _P), ("ld_out1", _I64), ("cosine", _P), ("sine", _P),
        ("head_dim", _I64), ("half", _I64),
    ]


_EPI = ctypes.POINTER(Epilogue)

_SIGNATURES = {
    "ct_abi_version": (ctypes.c_int, []),
    "ct_init_device": (ctypes.c_int, []),
    "ct_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "ct_nf4_dequant": (ctypes.c_int, [ctypes.POINTER(NF4Weight), _P, _I32, _P]),
    "ct_nf4_fused_supported": (ctypes.c_int, [ctypes.POINTER(NF4Weight)]),
    "ct_gemm_workspace": (_I64, [_I64, _I64, _I64, _I32, _I32, _I32]),
    "ct_gemm": (ctypes.c_int, [_P, _I64, _I32, _P, _I64, _I32, _P, _I64, _I32, _P, _I32, _I64, _I64, _I64, _P, _I64,
                               _P]),
    "ct_gemm_f32": (ctypes.c_int, [_P, _I64, _I32, _P, _I64, _I32, _P, _I64, _I32, _P, _I64, _I64, _I64, _P]),
    "ct_forward_linear_workspace": (_I64, [_I64, _I64, _I64, _I64, _I32]),
    "ct_forward_linear": (ctypes.c_int, [_P, _I64, _P, ctypes.POINTER(NF4Weight), _P, _P, _P, _P, _I64, _P,
                                         _I64, _I32, _I64, _I64, _I64, _I64, _EPI, _P, _I64, _P]),
    "ct_forward_linear_static": (ctypes.c_int, [_P, _I64, _P, ctypes.POINTER(NF4Weight), _P, _P, _P, _P, _I64,
                                                _P, _I64, _I32, _I64, _I64, _I64, _I64, _EPI, _P]),
    "ct_input_gradient_workspace": (_I64, [_I64, _I64, _I64, _I64, _I32]),
    "ct_input_gradient": (ctypes.c_int, [_P, _I64, _P, ctypes.POINTER(NF4Weight), _P, _P, _P, _I64, _P,
                                         _I64, _I64, _I64, _I64, _I32, _EPI, _P, _I64, _P]),
    "ct_parameter_gradients_workspace": (_I64, [_I64, _I64, _I64, _I64]),
    "ct_parameter_gradients": (ctypes.c_int, [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64,
                                              _I64, _I32, _P, _I64, _P]),
    "ct_accumulate_workspace": (_I64, [_I64, _I64, _I64]),
    "ct_silu_multiply": (ctypes.c_int, [_P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _P]),
    "ct_rope": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _P]),
    "ct_group_forward_workspace": (_I64, [_I64, _I32, _P, _I64, _I64]),
    "ct_group_forward": (ctypes.c_int, [_P, _I64, _I32, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _P,
                                        _I64, _P]),
    "ct_group_input_gradient_workspace": (_I64, [_I64, _I32, _P, _P, _I64]),
    "ct_group_input_gradient": (ctypes.c_int, [_P, _I64, _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _I64,
                                               _I64, _I32, _P, _I64, _P]),
    "ct_group_input_gradient_lead_workspace": (_I64, [_I64, _I32, _P, _P, _I64]),
    "ct_group_input_gradient_lead": (ctypes.c_int, [_P, _I64, _P, _I64, _I32, _P, _P, _P, _P, _P, _P, _P, _I64,
                                                    _I64, _I64, _I32, _P, _I64, _P]),
    "ct_nf4_quantize_workspace": (_I64, [_I64, _I32, _I32]),
    "ct_nf4_quantize": (ctypes.c_int, [_P, _I32, _I64, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "ct_quantize_blockwise": (ctypes.c_int, [_P, _I64, _P, _P, _P, _P, _P]),
    "ct_rms_forward": (ctypes.c_int, [_P, _I32, _P, _I32, _P, _P, _I64, _I64, ctypes.c_float, _P]),
    "ct_rms_backward_workspace": (_I64, [_I64, _I64, _I32]),
    "ct_rms_backward": (ctypes.c_int, [_P, _I32, _P, _I32, _P, _P, _P, _P, _I64, _I64, _I32, _P, _I64, _P]),
    "ct_weighted_ce_workspace": (_I64, [_I64, _I64]),
    "ct_weighted_ce": (ctypes.c_int, [_P, _I32, _I64, _I64, _I64, _P, _P, _P, _I32, _P, _I64, _P]),
    "ct_cast_f32_bf16": (ctypes.c_int, [_P, _P, _P, _I32, _P]),
    "ct_adamw_step": (ctypes.c_int, [_P, _I64, _P, _I64, _I64, _I32, ctypes.c_double, ctypes.c_double,
                                     ctypes.c_double, ctypes.c_double, ctypes.c_double, _I32, _I32, _P]),
    "ct_profile_begin": (ctypes.c_int, [_I32, _I32]),
    "ct_profile_read": (ctypes.c_int, [_I32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I64),
                                       ctypes.POINTER(ctypes.c_double)]),
    "ct_profile_end": (ctypes.c_int, []),
    "ct_accumulate": (ctypes.c_int, [_P, _I64, _P, _I64, _I32, _P, _I64, _I32, _I64, _I64, _I64, _I32, _P, _I64,
                                     _P]),
}

# Every symbol the header declares; tests check the built library exports each one.
EXPORTED = tuple(_SIGNATURES)

_library = None


ABI_VERSION = 13   # ct_abi_version() of the library these signatures describe


def library_path():
    return os.environ.get("CAUSAL_TUNER_HIP_LIBRARY", DEFAULT_LIBRARY)


def library():
    """Load (once) and return the HIP library with its C signatures declared."""
    global _library
    if _library is None:
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(f"The HIP library {path} is not built; run `python causal-tuner_amd/build.py`")
        lib = ctypes.CDLL(path)
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = restype, argtypes
        if lib.ct_abi_version() != ABI_VERSION:
            raise RuntimeError(f"The HIP library {path} has ABI {lib.ct_abi_version()}, this binding needs "
                               f"{ABI_VERSION}; rebuild it with `python causal-tuner_amd/build.py`")
        _library = lib
    return _library


def check(status, what):
    if status != 0:
        message = library().ct_status_string(status).decode()
        raise RuntimeError(f"{what} failed with status {status}: {message}")


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_CURRENT = contextlib.nullcontext()


def stream_of(tensor):
    """The caller's current HIP stream on the tensor's device (kernels never pick their own),
    as the integer handle the `void *` arguments take."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(tensor.device.index)
    return torch.cuda.current_stream(tensor.device).cuda_stream


_READY = set()


def _init_device(index):
    """The library's per-device set-up (ct_init_device), once per GPU with it current."""
    with torch.cuda.device(index):
        check(library().ct_init_device(), "ct_init_device")
    _READY.add(index)


def device_of(tensor):
    """A context making the tensor's device current for a launch: a no-op when it already is
    (the usual single-device case costs one device query instead of two device switches).
    The first launch on a device runs the library's set-up for it."""
    index = tensor.device.index
    if index not in _READY:
        _init_device(index)
    if index == torch.cuda.current_device():
        return _CURRENT
    return torch.cuda.device(index)


def ptr(tensor):
    return None if tensor is None else tensor.data_ptr()


def dtype_code(dtype):
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"Unsupported element type {dtype}") from None


def nf4_kind(desc):
    """The `nf4` argument of the workspace queries: 0 for a bf16 weight, 1 for a
    double-quantized NF4 weight, 2 for NF4 with plain absmax."""
    if desc is None:
        return 0
    return 1 if desc.nested else 2


def _matrix(t, rows):
    """(pointer, row pitch) of a bf16 tensor viewed as [rows, width] with unit stride."""
    view = t.reshape(rows, -1) if t.dim() != 2 else t
    if view.stride(-1) != 1:
        raise ValueError("epilogue tensors need unit stride along a row")
    return view.data_ptr(), max(view.stride(0), view.shape[1])


def epilogue(kind, rows, in0=None, in1=None, out0=None, out1=None, rotary=None):
    """A ct_epilogue for an output of `rows` rows; `rotary` is (cosine, sine, head_dim)
    with cosine/sine [rows, half] contiguous."""
    e = Epilogue(kind=kind)
    for name, t in (("in0", in0), ("in1", in1), ("out0", out0), ("out1", out1)):
        if t is not None:
            if t.dtype != torch.bfloat16:
                raise ValueError("epilogue tensors are bfloat16")
            ptr, ld = _matrix(t, rows)
            setattr(e, name, ptr)
            setattr(e, "ld_" + name, ld)
    if rotary is not None:
        cosine, sine, head_dim = rotary
        if not (cosine.is_contiguous() and sine.is_contiguous() and cosine.dtype == sine.dtype
                and cosine.shape == sine.shape and cosine.shape[0] == rows):
            raise ValueError("rotary tables must be contiguous [rows, half] tensors of one dtype")
        e.cosine, e.sine = cosine.data_ptr(), sine.data_ptr()
        e.trig_dtype = dtype_code(cosine.dtype)
        e.head_dim, e.half = int(head_dim), int(cosine.shape[-1])
    return e


def _nf4_key(weight, state):
    nested = bool(state.nested)
    aux = state.state2 if nested else None
    return (weight.data_ptr(), state.absmax.data_ptr(), state.code.data_ptr(), tuple(state.shape),
            int(state.blocksize), state.dtype, nested,
            (aux.code.data_ptr(), aux.absmax.data_ptr(), state.offset.data_ptr(), int(aux.blocksize)) if nested
            else None)


def nf4_descriptor(weight, state):
    """The ct_nf4_weight view of a packed weight and its QuantState (no copies). Kept on the
    state with the addresses it was built from, and rebuilt when any of them changes."""
    key = _nf4_key(weight, state)
    cached = getattr(state, "_ct_descriptor", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    desc = _build_nf4_descriptor(weight, state)
    try:
        state._ct_descriptor = (key, desc, None)
    except AttributeError:   # a state type without attribute storage: no cache
        pass
    return desc


def nf4_fused_supported(weight, state):
    """ct_nf4_fused_supported of the weight's descriptor, kept beside the descriptor."""
    return nf4_fused_descriptor(weight, state) is not None


def nf4_fused_descriptor(weight, state):
    """The weight's descriptor when the fused loaders take it (ct_nf4_fused_supported, kept
    beside the descriptor), else None."""
    desc = nf4_descriptor(weight, state)
    cached = getattr(state, "_ct_descriptor", None)
    if cached is not None and cached[1] is desc and cached[2] is not None:
        return desc if cached[2] else None
    supported = library().ct_nf4_fused_supported(desc) == 1
    if cached is not None and cached[1] is desc:
        state._ct_descriptor = (cached[0], desc, supported)
    return desc if supported else None


def _build_nf4_descriptor(weight, state):
    nested = bool(state.nested)
    aux = state.state2 if nested else None
    numel = 1
    for size in state.shape:
        numel *= int(size)
    rows = int(state.shape[0]) if len(state.shape) >= 2 else 1
    cols = numel // rows if rows else 0
    desc = NF4Weight(
        packed=weight.data_ptr(), absmax=state.absmax.data_ptr(), code=state.code.data_ptr(),
        code2=aux.code.data_ptr() if nested else None, absmax2=aux.absmax.data_ptr() if nested else None,
        offset=state.offset.data_ptr() if nested else None, rows=rows, cols=cols, blocksize=int(state.blocksize),
        blocksize2=int(aux.blocksize) if nested else 0, nested=int(nested), storage_dtype=dtype_code(state.dtype))
    return desc


class KernelTimer:
    """Time the launches of some kernel families with HIP events (ct_profile_*).

    Used by the benchmark inside its timed region: `read(family)` returns
    (total_ms, launches, algorithmic_work) for the launches made while active."""

    def __init__(self, families, capacity=4096):
        self.families, self.capacity = families, capacity

    def __enter__(self):
        check(library().ct_profile_begin(self.families, self.capacity), "ct_profile_begin")
        return self

    def read(self, family):
        ms, n, work = ctypes.c_double(), _I64(), ctypes.c_double()
        check(library().ct_profile_read(family, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(work)),
              "ct_profile_read")
        return ms.value, n.value, work.value

    def __exit__(self, *exc):
        library().ct_profile_end()
        return False
