"""ct_forward_linear_static, the forward projection for callers that cannot allocate: its
scratch is the library's static device array instead of a caller's workspace. Called
through the C ABI and compared with ct_forward_linear given a torch workspace, on two calls
in a row (the second smaller), bit for bit; a problem whose scratch need exceeds the static
maximum is refused on the host."""

import ctypes

import pytest
import torch

from causal_tuner.kernels import _native
from causal_tuner.quant.nf4 import quantize_nf4

pytestmark = pytest.mark.gpu


def _problem(m, k, n, r, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    packed, state = quantize_nf4(w)
    x = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
    a = ((torch.rand(r, k, device="cuda", generator=g) * 2 - 1) * (6 / k) ** 0.5).to(torch.bfloat16)
    b = (torch.randn(n, r, device="cuda", generator=g) * 0.01).to(torch.bfloat16)
    bias = (torch.randn(n, device="cuda", generator=g) * 0.1).to(torch.bfloat16)
    return packed, state, x, a, b, bias


def _run(entry, problem, m, k, n, r):
    packed, state, x, a, b, bias = problem
    lib = _native.library()
    desc = _native.nf4_descriptor(packed, state)
    out = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    xa = torch.full((m, r), float("nan"), device="cuda", dtype=torch.bfloat16)
    common = (x.data_ptr(), k, None, ctypes.byref(desc), a.data_ptr(), b.data_ptr(), bias.data_ptr(),
              out.data_ptr(), n, xa.data_ptr(), r, 0, m, n, k, r)
    stream = _native.stream_of(x)
    if entry == "static":
        assert lib.ct_init_device() == 0   # the library's per-device set-up, before any static call
        status = lib.ct_forward_linear_static(*common, None, stream)
    else:
        need = lib.ct_forward_linear_workspace(m, n, k, r, 1)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
        status = lib.ct_forward_linear(*common, None, ws.data_ptr(), ws.numel(), stream)
    assert status == 0, (entry, status)
    return out, xa


@pytest.mark.parametrize("shapes", [((600, 4096, 4096, 64), (16, 6144, 24576, 256)),
                                    ((300, 4096, 4096, 256), (64, 24576, 6144, 256))])
def test_static_scratch_forward_matches_workspace_forward(shapes):
    for index, (m, k, n, r) in enumerate(shapes):
        print(f"static-scratch forward: call {index}, m={m} k={k} n={n} r={r}", flush=True)
        problem = _problem(m, k, n, r, seed=index + 1)
        got = _run("static", problem, m, k, n, r)
        want = _run("workspace", problem, m, k, n, r)
        torch.cuda.synchronize()
        for name, g, w in zip(("out", "xa"), got, want):
            assert torch.equal(g.view(torch.int16), w.view(torch.int16)), (index, name)
            assert bool(torch.isfinite(g.float()).all()), (index, name)


def test_static_scratch_refuses_problems_beyond_its_maximum():
    lib = _native.library()
    m, k, n, r = 8192, 4096, 11008, 256
    assert lib.ct_forward_linear_workspace(m, n, k, r, 1) > _native.CT_STATIC_SCRATCH_BYTES
    desc = _native.NF4Weight(packed=256, absmax=256, code=256, code2=256, absmax2=256, offset=256, rows=n, cols=k,
                             blocksize=64, blocksize2=256, nested=1, storage_dtype=_native.CT_BF16)
    status = lib.ct_forward_linear_static(16, k, None, ctypes.byref(desc), 16, 16, None, 16, n, 16, r, 0, m, n, k, r,
                                          None, None)
    assert status == -5
