"""The bf16 MFMA GEMM family (ct_gemm / ct_accumulate) against float64 products of the same
bf16 operands. These are the contractions behind torch.mm / torch.addmm in the reference's
operator layer (kernels/linear.py:16-44)."""

import ctypes

import pytest
import torch

from causal_tuner.kernels import _native

pytestmark = pytest.mark.gpu

# The last two reach the 256x256-tile kernels (>= 256 output tiles); 4100 x 4104 also
# exercises their ragged edges and, transposed, the scalar (non-16-byte) loaders.
SHAPES = [(256, 384, 320), (37, 80, 96), (1, 1, 1), (129, 65, 17), (64, 8, 4096), (300, 260, 72),
          (4096, 4096, 192), (4100, 4104, 136)]


def _operand(rows, cols, transposed):
    """A bf16 matrix [rows, cols] stored row-major, or column-major when `transposed`.

    Returns (logical view, storage, ld). Element (i, j) lives at i*ld + j (row-major) or
    j*ld + i (column-major); the storage always covers the largest such offset."""
    if transposed:
        base = torch.randn(cols, rows, device="cuda").to(torch.bfloat16)
        ld = rows
        assert base.numel() >= (cols - 1) * ld + rows
        return base.T, base, ld
    base = torch.randn(rows, cols, device="cuda").to(torch.bfloat16)
    ld = cols
    assert base.numel() >= (rows - 1) * ld + cols
    return base, base, ld


def _err(got, want):
    d = (got.double() - want).abs()
    return float(d.max() / want.abs().max().clamp_min(1e-30)), float((got.double() - want).norm() /
                                                                     want.norm().clamp_min(1e-30))


@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("trans_a", [0, 1])
@pytest.mark.parametrize("trans_b", [0, 1])
@pytest.mark.parametrize("out", [torch.bfloat16, torch.float32])
def test_gemm_layouts_and_tails(m, n, k, trans_a, trans_b, out):
    lib = _native.library()
    # A(m, k) = a[m*lda + k] (trans_a=0, row-major) or a[k*lda + m] (trans_a=1, column-major)
    a, abase, lda = _operand(m, k, bool(trans_a))
    # B(k, n) = b[k*ldb + n] (trans_b=0, row-major) or b[n*ldb + k] (trans_b=1, column-major)
    b, bbase, ldb = _operand(k, n, bool(trans_b))
    bias = (torch.randn(n, device="cuda") * 0.5).to(torch.bfloat16)
    c = torch.full((m, n), float("nan"), device="cuda", dtype=out)
    status = lib.ct_gemm(abase.data_ptr(), lda, trans_a, bbase.data_ptr(), ldb, trans_b, c.data_ptr(), n,
                         _native.dtype_code(out), bias.data_ptr(), 0, m, n, k, None, 0, _native.stream_of(c))
    assert status == 0
    want = a.double() @ b.double() + bias.double()
    worst, norm = _err(c, want)
    tol = 8e-3 if out == torch.bfloat16 else 1e-5
    assert worst <= tol and norm <= tol / 2, (worst, norm)
    # beta accumulation on top of the previous result, no bias
    status = lib.ct_gemm(abase.data_ptr(), lda, trans_a, bbase.data_ptr(), ldb, trans_b, c.data_ptr(), n,
                         _native.dtype_code(out), None, 1, m, n, k, None, 0, _native.stream_of(c))
    assert status == 0
    worst, norm = _err(c, want + a.double() @ b.double())
    assert worst <= 2 * tol and norm <= tol, (worst, norm)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gradient_first_write_ignores_uninitialized_storage(dtype):
    """tests/test_kernel_workspaces.py:269-279 (accumulate with add=False ignores NaN). bf16
    operands run ct_accumulate; fp32 operands keep the reference's addmm (linear.py:22-24)."""
    from causal_tuner.kernels.linear import accumulate
    left = torch.randn(19, 37, device="cuda", dtype=dtype)
    right = torch.randn(37, 23, device="cuda", dtype=dtype)
    output = torch.full((19, 23), float("nan"), device="cuda")
    expected = left.float() @ right.float()
    accumulate(output, left, right, add=False)
    torch.testing.assert_close(output, expected, rtol=1e-5, atol=1e-5)
    accumulate(output, left, right, add=True)
    torch.testing.assert_close(output, expected * 2, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("p,q,j", [(256, 4096, 8192), (4096, 256, 4096), (16, 1024, 512), (11008, 256, 8192)])
def test_split_reduction_is_deterministic_and_exact_enough(p, q, j):
    """dA/dB-shaped reductions over many tokens: fixed-order split sums, repeat bit-identical."""
    from causal_tuner.kernels.linear import accumulate
    low = torch.randn(j, p, device="cuda").to(torch.bfloat16)    # used transposed, like low.T
    x = torch.randn(j, q, device="cuda").to(torch.bfloat16)
    out = torch.full((p, q), float("nan"), device="cuda")
    accumulate(out, low.T, x, add=False)
    first = out.clone()
    accumulate(out, low.T, x, add=False)
    assert torch.equal(out, first)
    want = low.double().T @ x.double()
    worst, norm = _err(first, want)
    assert worst <= 1e-5 and norm <= 1e-6, (worst, norm)
    accumulate(out, low.T, x, add=True)
    worst, _ = _err(out, 2 * want)
    assert worst <= 1e-5


def test_gemm_runs_on_the_callers_stream():
    lib = _native.library()
    a = torch.randn(512, 512, device="cuda").to(torch.bfloat16)
    stream = torch.cuda.Stream()
    c = torch.empty(512, 512, device="cuda", dtype=torch.float32)
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        assert lib.ct_gemm(a.data_ptr(), 512, 0, a.data_ptr(), 512, 1, c.data_ptr(), 512, _native.CT_F32, None, 0,
                           512, 512, 512, None, 0, ctypes.c_void_p(stream.cuda_stream)) == 0
    torch.cuda.current_stream().wait_stream(stream)
    torch.testing.assert_close(c, (a.float() @ a.float().T), rtol=1e-4, atol=1e-3)


@pytest.mark.parametrize("m,n,k,trans_b", [(16, 256, 6144, 1), (7, 256, 24576, 0), (64, 128, 4096, 1),
                                           (33, 512, 2048, 0), (8192, 256, 4096, 1), (8192, 256, 11008, 0),
                                           (4100, 200, 4104, 1)])
def test_few_row_split_reduction_is_deterministic(m, n, k, trans_b):
    """m <= 64, or a rank-r product (n <= 256) over many rows, with a workspace splits the
    reduction across workgroups; the fp32 partials add in split order, so repeated calls
    agree bit for bit, and the result matches a float64 product of the same bf16 operands
    within bf16 rounding (also without a workspace, where the reduction is not split)."""
    lib = _native.library()
    a, abase, lda = _operand(m, k, False)
    b, bbase, ldb = _operand(k, n, bool(trans_b))
    need = lib.ct_gemm_workspace(m, n, k, 0, trans_b, _native.CT_BF16)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    outs = []
    for workspace, size in ((ws.data_ptr(), need), (ws.data_ptr(), need), (None, 0)):
        c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        assert lib.ct_gemm(abase.data_ptr(), lda, 0, bbase.data_ptr(), ldb, trans_b, c.data_ptr(), n,
                           _native.CT_BF16, None, 0, m, n, k, workspace, size, _native.stream_of(c)) == 0
        outs.append(c)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    want = a.double() @ b.double()
    for c in (outs[0], outs[2]):
        worst, norm = _err(c, want)
        assert worst <= 8e-3 and norm <= 4e-3, (worst, norm)


@pytest.mark.parametrize("m,n,k,trans_b", [(128, 2048, 49152, 0), (96, 1000, 13000, 1), (512, 2048, 16384, 1),
                                           (1024, 2048, 12288, 0), (600, 1032, 20000, 0)])
def test_long_reduction_split_is_deterministic(m, n, k, trans_b):
    """An output short of one round of 256 x 256 tiles over a long reduction (the loss's
    d hidden = derivative head, a 49152-long reduction into [tile, 2048]) takes the split
    route, past 511 rows too: the workspace query asks for the partials, repeated calls
    agree bit for bit, and the result matches a float64 product of the same bf16 operands
    within bf16 rounding (also without a workspace, where the reduction is not split)."""
    lib = _native.library()
    a, abase, lda = _operand(m, k, False)
    b, bbase, ldb = _operand(k, n, bool(trans_b))
    need = lib.ct_gemm_workspace(m, n, k, 0, trans_b, _native.CT_BF16)
    assert need >= 2 * m * n * 4
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    outs = []
    for workspace, size in ((ws.data_ptr(), need), (ws.data_ptr(), need), (None, 0)):
        c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        assert lib.ct_gemm(abase.data_ptr(), lda, 0, bbase.data_ptr(), ldb, trans_b, c.data_ptr(), n,
                           _native.CT_BF16, None, 0, m, n, k, workspace, size, _native.stream_of(c)) == 0
        outs.append(c)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    want = a.double() @ b.double()
    for c in (outs[0], outs[2]):
        worst, norm = _err(c, want)
        assert worst <= 8e-3 and norm <= 4e-3, (worst, norm)


@pytest.mark.parametrize("m,n,k", [(200, 512, 4096), (96, 2048, 49152), (600, 1032, 20000)])
def test_split_route_with_bias_and_accumulation(m, n, k):
    """The split route's reduction adds the bias and, with beta, the previous output (bf16)
    after the partials, in split order: against float64 products of the same operands."""
    lib = _native.library()
    a, abase, lda = _operand(m, k, False)
    b, bbase, ldb = _operand(k, n, True)
    bias = (torch.randn(n, device="cuda") * 0.5).to(torch.bfloat16)
    need = lib.ct_gemm_workspace(m, n, k, 0, 1, _native.CT_BF16)
    assert need >= 2 * m * n * 4
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    assert lib.ct_gemm(abase.data_ptr(), lda, 0, bbase.data_ptr(), ldb, 1, c.data_ptr(), n, _native.CT_BF16,
                       bias.data_ptr(), 0, m, n, k, ws.data_ptr(), need, _native.stream_of(c)) == 0
    product = a.double() @ b.double()
    want = product + bias.double()
    worst, norm = _err(c, want)
    assert worst <= 8e-3 and norm <= 4e-3, (worst, norm)
    first = c.clone()
    assert lib.ct_gemm(abase.data_ptr(), lda, 0, bbase.data_ptr(), ldb, 1, c.data_ptr(), n, _native.CT_BF16,
                       None, 1, m, n, k, ws.data_ptr(), need, _native.stream_of(c)) == 0
    worst, norm = _err(c, first.double() + product)
    assert worst <= 8e-3 and norm <= 4e-3, (worst, norm)


@pytest.mark.parametrize("trans_b", [0, 1])
def test_partial_last_round_column_split_matches_row_slices(trans_b):
    """8192 x 11008 on 256 x 256 tiles is 5 whole rounds of the 256 CUs and 96 tiles: the
    first 10240 columns run as the whole rounds and the last 768 as a second launch on
    128 x 128 tiles (C3's dx of down has this output). Every element's sum is the one a
    256-row slice computes alone (on 64 x 64 tiles, one launch), bit for bit, and the
    float64 product of the same operands bounds both."""
    lib = _native.library()
    m, n, k = 8192, 11008, 320
    a, abase, lda = _operand(m, k, False)
    b, bbase, ldb = _operand(k, n, bool(trans_b))
    bias = (torch.randn(n, device="cuda") * 0.5).to(torch.bfloat16)
    c = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    assert lib.ct_gemm(abase.data_ptr(), lda, 0, bbase.data_ptr(), ldb, trans_b, c.data_ptr(), n, _native.CT_BF16,
                       bias.data_ptr(), 0, m, n, k, None, 0, _native.stream_of(c)) == 0
    for start in (0, m - 256):
        part = torch.full((256, n), float("nan"), device="cuda", dtype=torch.bfloat16)
        assert lib.ct_gemm(abase[start:].data_ptr(), lda, 0, bbase.data_ptr(), ldb, trans_b, part.data_ptr(), n,
                           _native.CT_BF16, bias.data_ptr(), 0, 256, n, k, None, 0, _native.stream_of(c)) == 0
        torch.cuda.synchronize()
        assert torch.equal(c[start:start + 256].view(torch.int16), part.view(torch.int16)), start
    want = a.double() @ b.double() + bias.double()
    worst, norm = _err(c, want)
    assert worst <= 8e-3 and norm <= 4e-3, (worst, norm)
    # beta accumulation into a pitched output (row pitch past n), on both launches
    ld = n + 64
    d = torch.full((m, ld), float("nan"), device="cuda", dtype=torch.bfloat16)
    d[:, :n] = c
    assert lib.ct_gemm(abase.data_ptr(), lda, 0, bbase.data_ptr(), ldb, trans_b, d.data_ptr(), ld, _native.CT_BF16,
                       None, 1, m, n, k, None, 0, _native.stream_of(d)) == 0
    worst, norm = _err(d[:, :n], c.double() + a.double() @ b.double())
    assert worst <= 8e-3 and norm <= 4e-3, (worst, norm)
    assert torch.isnan(d[:, n:]).all()


def test_partial_last_round_column_split_in_the_input_gradient():
    """dx = [dy | low] [w ; a] at C3's down shape (8192 x 11008 output, dense weight): the
    column split offsets both segments' B operands; each 256-row slice computed alone gives
    the same bits."""
    lib = _native.library()
    m, n, k, r = 8192, 192, 11008, 32
    g = torch.Generator(device="cuda").manual_seed(3)
    dy = torch.randn(m, n, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    a = (torch.randn(r, k, device="cuda", generator=g) * 0.05).to(torch.bfloat16)
    bf = (torch.randn(n, r, device="cuda", generator=g) * 0.05).to(torch.bfloat16)

    def call(rows, start):
        dx = torch.full((rows, k), float("nan"), device="cuda", dtype=torch.bfloat16)
        low = torch.empty(rows, r, device="cuda", dtype=torch.bfloat16)
        need = lib.ct_input_gradient_workspace(rows, n, k, r, 0)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
        assert lib.ct_input_gradient(dy[start:].data_ptr(), n, w.data_ptr(), None, a.data_ptr(), bf.data_ptr(),
                                     dx.data_ptr(), k, low.data_ptr(), rows, n, k, r, 0, None,
                                     ws.data_ptr() if rows > 256 else None, need if rows > 256 else 0,
                                     _native.stream_of(dx)) == 0
        return dx

    full = call(m, 0)
    for start in (0, m - 256):
        part = call(256, start)
        torch.cuda.synchronize()
        assert torch.equal(full[start:start + 256].view(torch.int16), part.view(torch.int16)), start
    low = (dy.double() @ bf.double()).bfloat16().double()
    want = dy.double() @ w.double() + low @ a.double()
    worst, norm = _err(full, want)
    assert worst <= 8e-3 and norm <= 4e-3, (worst, norm)
