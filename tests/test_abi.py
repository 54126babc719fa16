"""The C ABI library loads, exports every declared symbol, and rejects bad arguments on the
host before anything is enqueued (no GPU needed)."""

import ctypes
import os
import re
import subprocess

import pytest
import torch

from causal_tuner.kernels import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "causal_tuner_hip.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char \*)\s*(ct_\w+)\s*\(", text, re.M)))


def test_header_declarations_match_the_binding():
    assert declared_functions() == sorted(_native.EXPORTED)


def test_library_exports_every_declared_symbol():
    lib = _native.library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _native.library_path()], capture_output=True, text=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if line.strip()}
    assert set(declared_functions()) <= exported


def test_library_embeds_gfx950_code_objects():
    out = subprocess.run(["readelf", "-S", _native.library_path()], capture_output=True, text=True)
    assert ".hip_fatbin" in out.stdout
    blob = open(_native.library_path(), "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    assert b"gfx942" not in blob and b"gfx90a" not in blob


def test_status_strings_and_version():
    lib = _native.library()
    assert lib.ct_abi_version() == 13
    assert lib.ct_status_string(0) == b"success"
    assert b"workspace" in lib.ct_status_string(-5)
    assert b"fused" in lib.ct_status_string(-6)


def test_fused_nf4_operand_conditions():
    """The fused loaders take blocksize >= 32, cols % 32 == 0, 16-byte aligned packed bytes
    and a bf16 or f32 storage type; everything else is decoded by ct_nf4_dequant first."""
    lib = _native.library()
    desc = _native.NF4Weight(packed=256, absmax=256, code=256, rows=4, cols=64, blocksize=64, nested=0,
                             storage_dtype=_native.CT_BF16)
    assert lib.ct_nf4_fused_supported(ctypes.byref(desc)) == 1
    for field, value in (("cols", 48), ("blocksize", 16), ("storage_dtype", _native.CT_F16), ("packed", 264)):
        bad = _native.NF4Weight.from_buffer_copy(desc)
        setattr(bad, field, value)
        assert lib.ct_nf4_fused_supported(ctypes.byref(bad)) == 0, field
    desc.storage_dtype = _native.CT_F32
    assert lib.ct_nf4_fused_supported(ctypes.byref(desc)) == 1


def test_host_side_argument_errors_return_negative_status():
    lib = _native.library()
    null = None
    # null descriptor
    assert lib.ct_nf4_dequant(None, null, _native.CT_BF16, null) == -1
    # bad block size
    desc = _native.NF4Weight(packed=16, absmax=16, code=16, rows=2, cols=64, blocksize=48, nested=0,
                             storage_dtype=_native.CT_BF16)
    assert lib.ct_nf4_dequant(ctypes.byref(desc), ctypes.c_void_p(16), _native.CT_BF16, null) == -4
    desc.blocksize = 64
    assert lib.ct_nf4_dequant(ctypes.byref(desc), ctypes.c_void_p(16), 7, null) == -3
    # negative sizes and short leading dimensions
    assert lib.ct_gemm(16, 4, 0, 16, 4, 1, 16, 4, _native.CT_BF16, null, 0, -1, 4, 4, null, 0, null) == -2
    assert lib.ct_gemm(16, 2, 0, 16, 4, 1, 16, 4, _native.CT_BF16, null, 0, 4, 4, 4, null, 0, null) == -2
    assert lib.ct_gemm(16, 4, 0, 16, 4, 1, 16, 4, 9, null, 0, 4, 4, 4, null, 0, null) == -3
    # empty problems are no-ops
    assert lib.ct_gemm(null, 0, 0, null, 0, 1, null, 0, _native.CT_BF16, null, 0, 0, 0, 0, null, 0, null) == 0
    # few-row problems and rank-r products over many rows ask for split workspace; large
    # square ones and fp32 outputs do not
    assert lib.ct_gemm_workspace(16, 256, 6144, 0, 1, _native.CT_BF16) > 0
    assert lib.ct_gemm_workspace(8192, 256, 4096, 0, 1, _native.CT_BF16) == 4 * 8192 * 256 * 4
    assert lib.ct_gemm_workspace(8192, 4096, 4096, 0, 1, _native.CT_BF16) == 0
    assert lib.ct_gemm_workspace(16, 256, 6144, 0, 1, _native.CT_F32) == 0
    assert lib.ct_input_gradient_workspace(16, 24576, 6144, 256, 1) > 0
    assert lib.ct_forward_linear_workspace(8192, 4096, 4096, 256, 0) == 4 * 8192 * 256 * 4
    # many rows: an NF4 weight is materialized as bf16 inside the workspace first
    assert lib.ct_forward_linear_workspace(8192, 4096, 4096, 256, 1) >= 4096 * 4096 * 2
    assert lib.ct_input_gradient_workspace(8192, 11008, 4096, 256, 1) >= 11008 * 4096 * 2
    assert lib.ct_forward_linear_workspace(64, 4096, 4096, 256, 1) < 4096 * 4096 * 2
    # workspace too small for a split reduction
    need = lib.ct_accumulate_workspace(256, 4096, 8192)
    assert need > 0
    assert lib.ct_accumulate(ctypes.c_void_p(16), 4096, ctypes.c_void_p(16), 256, 1, ctypes.c_void_p(16), 4096, 0,
                             256, 4096, 8192, 0, null, 0, null) == -5
    assert lib.ct_parameter_gradients_workspace(8192, 4096, 4096, 256) >= need


def test_nf4_descriptor_reads_state_fields():
    from causal_tuner.quant.nf4 import quantize_nf4
    w = (torch.randn(17, 19) * 0.02).to(torch.bfloat16)
    packed, state = quantize_nf4(w)
    d = _native.nf4_descriptor(packed, state)
    assert (d.rows, d.cols, d.blocksize, d.blocksize2, d.nested) == (17, 19, 64, 256, 1)
    assert d.storage_dtype == _native.CT_BF16 and d.packed == packed.data_ptr()
    assert d.offset == state.offset.data_ptr() and d.absmax2 == state.state2.absmax.data_ptr()
