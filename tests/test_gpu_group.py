"""Projections that share an input, through the C ABI.

ct_group_forward (two projections' forward as one GEMM, the reference's forward_linear per
projection in _LoRAGroup.forward, kernels/linear.py:72-86): bit-identical to
ct_forward_linear with the stacked xa given, per projection.

ct_group_input_gradient: the input gradient of projections that share an input as one
contraction (the dx half of the reference's _LoRAGroup.backward, kernels/linear.py:107-122,
and of the MLP's gate/up, kernels/mlp_cuda.py:136-140):

* low_i is bit-identical to ct_input_gradient's low for the same projection (the same
  rank-r product);
* dx is within 1e-3 (relative Frobenius) of the float64 sum of dy_i w_i + low_i a_i (+ the
  previous dx with add) rounded once to bf16, and within 2e-2 (max-abs relative) of the
  reference's sequence of per-projection input gradients, which rounds after each one;
* a repeated call is bit-identical; NF4 and dense weights; invalid descriptions are
  refused on the host.

ct_group_input_gradient_lead: the same dx and low_i with the first upstream gradient read
in place and the later ones in a tail matrix ahead of the low-rank products it receives:
low_i bit-identical to ct_input_gradient's, dx within 1e-3 of the same float64 sum, within
one bf16 rounding step of ct_group_input_gradient's (the fp32 additions run in another
order), bit-identical on a repeated call, with pitched operands."""

import ctypes

import pytest
import torch

from causal_tuner.kernels import _native
from causal_tuner.quant.nf4 import quantize_nf4

pytestmark = pytest.mark.gpu


def _rand(*shape, seed, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(*shape, device="cuda", generator=g) * scale).to(torch.bfloat16)


def _decode(packed, state):
    from causal_tuner.kernels.nf4_cuda import dequantize_nf4
    return dequantize_nf4(packed, state, torch.bfloat16)


def _call(m, k, widths, ranks, weights, dy, a_stack, bs, dx, low, add):
    lib = _native.library()
    count = len(widths)
    n_arr, r_arr = (ctypes.c_int64 * count)(*widths), (ctypes.c_int64 * count)(*ranks)
    dense = (ctypes.c_void_p * count)(*[w.data_ptr() if isinstance(w, torch.Tensor) else None for w in weights])
    descs = [None if isinstance(w, torch.Tensor) else _native.nf4_descriptor(*w) for w in weights]
    packed = (ctypes.POINTER(_native.NF4Weight) * count)(*[None if d is None else ctypes.pointer(d) for d in descs])
    factors = (ctypes.c_void_p * count)(*[b.data_ptr() for b in bs])
    need = lib.ct_group_input_gradient_workspace(m, count, n_arr, r_arr, k)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    return lib.ct_group_input_gradient(dy.data_ptr(), dy.stride(0), count, n_arr, r_arr, dense, packed,
                                       a_stack.data_ptr(), factors, dx.data_ptr(), dx.stride(0), low.data_ptr(),
                                       low.stride(0), m, k, int(add), ws.data_ptr(), ws.numel(),
                                       _native.stream_of(dy))


def _single(dy, weight, a, b, m, n, k, r):
    """ct_input_gradient for one projection: (dx, low)."""
    lib = _native.library()
    dx = torch.empty(m, k, device="cuda", dtype=torch.bfloat16)
    low = torch.empty(m, r, device="cuda", dtype=torch.bfloat16)
    desc = None if isinstance(weight, torch.Tensor) else _native.nf4_descriptor(*weight)
    need = lib.ct_input_gradient_workspace(m, n, k, r, _native.nf4_kind(desc))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    status = lib.ct_input_gradient(dy.data_ptr(), dy.stride(0), weight.data_ptr() if desc is None else None, desc,
                                   a.data_ptr(), b.data_ptr(), dx.data_ptr(), k, low.data_ptr(), m, n, k, r, 0, None,
                                   ws.data_ptr(), ws.numel(), _native.stream_of(dy))
    assert status == 0, status
    return dx, low


CASES = [
    # m, k, widths, ranks, nf4
    (300, 256, (64, 16, 16), (8, 8, 8), True),      # a q/k/v-like group, decode-first row count
    (520, 128, (96, 96), (16, 16), True),           # a gate/up-like pair
    (97, 128, (32, 8, 8), (4, 4, 4), True),         # few rows, odd m
    (260, 64, (48, 24), (8, 16), False),            # dense weights, unequal ranks
]


@pytest.mark.parametrize("m,k,widths,ranks,nf4", CASES)
@pytest.mark.parametrize("add", [False, True])
def test_group_input_gradient_against_float64_and_per_projection(m, k, widths, ranks, nf4, add):
    print(f"group dx: m={m} k={k} widths={widths} ranks={ranks} nf4={nf4} add={add}", flush=True)
    count = len(widths)
    weights, dense = [], []
    for i, n in enumerate(widths):
        w = _rand(n, k, seed=10 + i, scale=0.02)
        if nf4:
            packed, state = quantize_nf4(w)
            weights.append((packed, state))
            dense.append(_decode(packed, state))
        else:
            weights.append(w)
            dense.append(w)
    a_stack = _rand(sum(ranks), k, seed=20, scale=0.05)
    a_list = list(torch.split(a_stack, list(ranks)))
    bs = [_rand(n, r, seed=30 + i, scale=0.05) for i, (n, r) in enumerate(zip(widths, ranks))]
    dy = _rand(m, sum(widths), seed=40)
    prior = _rand(m, k, seed=41)
    dx = prior.clone() if add else torch.full((m, k), float("nan"), device="cuda", dtype=torch.bfloat16)
    low = torch.full((m, sum(ranks)), float("nan"), device="cuda", dtype=torch.bfloat16)
    assert _call(m, k, widths, ranks, weights, dy, a_stack, bs, dx, low, add) == 0
    again_dx, again_low = (prior.clone() if add else torch.empty_like(dx)), torch.empty_like(low)
    assert _call(m, k, widths, ranks, weights, dy, a_stack, bs, again_dx, again_low, add) == 0
    torch.cuda.synchronize()
    assert torch.equal(dx.view(torch.int16), again_dx.view(torch.int16))
    assert torch.equal(low.view(torch.int16), again_low.view(torch.int16))
    cols = [sum(widths[:i]) for i in range(count + 1)]
    rcols = [sum(ranks[:i]) for i in range(count + 1)]
    want = prior.double() if add else torch.zeros(m, k, device="cuda", dtype=torch.float64)
    sequence = prior.float() if add else None
    for i in range(count):
        dyi = dy[:, cols[i]:cols[i + 1]]
        single_dx, single_low = _single(dyi.contiguous(), weights[i], a_list[i].contiguous(), bs[i], m,
                                        widths[i], k, ranks[i])
        got_low = low[:, rcols[i]:rcols[i + 1]]
        assert torch.equal(got_low.view(torch.int16), single_low.view(torch.int16)), i
        want += dyi.double() @ dense[i].double() + got_low.double() @ a_list[i].double()
        sequence = single_dx.float() if sequence is None else (sequence + single_dx.float()).bfloat16().float()
    want = want.to(torch.bfloat16).float()
    diff = (dx.float() - want)
    assert bool(torch.isfinite(dx.float()).all())
    assert (diff.norm() / want.norm()).item() <= 1e-3
    peak = ((dx.float() - sequence).abs().max() / sequence.abs().max()).item()
    assert peak <= 2e-2, peak


def _call_lead(m, k, widths, ranks, weights, dy0, tail, a_stack, bs, dx, add, ws_extra=0):
    lib = _native.library()
    count = len(widths)
    n_arr, r_arr = (ctypes.c_int64 * count)(*widths), (ctypes.c_int64 * count)(*ranks)
    dense = (ctypes.c_void_p * count)(*[w.data_ptr() if isinstance(w, torch.Tensor) else None for w in weights])
    descs = [None if isinstance(w, torch.Tensor) else _native.nf4_descriptor(*w) for w in weights]
    packed = (ctypes.POINTER(_native.NF4Weight) * count)(*[None if d is None else ctypes.pointer(d) for d in descs])
    factors = (ctypes.c_void_p * count)(*[b.data_ptr() for b in bs])
    need = lib.ct_group_input_gradient_lead_workspace(m, count, n_arr, r_arr, k) + ws_extra
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    return lib.ct_group_input_gradient_lead(dy0.data_ptr(), dy0.stride(0), tail.data_ptr(), tail.stride(0), count,
                                            n_arr, r_arr, dense, packed, a_stack.data_ptr(), factors, dx.data_ptr(),
                                            dx.stride(0), m, k, int(add), ws.data_ptr(), need,
                                            _native.stream_of(dx))


@pytest.mark.parametrize("m,k,widths,ranks,nf4", CASES + [(8192, 512, (512, 64, 64), (32, 32, 32), True)])
@pytest.mark.parametrize("add", [False, True])
def test_group_input_gradient_lead_against_float64_and_joined(m, k, widths, ranks, nf4, add):
    print(f"group dx lead: m={m} k={k} widths={widths} ranks={ranks} nf4={nf4} add={add}", flush=True)
    count = len(widths)
    weights, dense = [], []
    for i, n in enumerate(widths):
        w = _rand(n, k, seed=10 + i, scale=0.02)
        if nf4:
            packed, state = quantize_nf4(w)
            weights.append((packed, state))
            dense.append(_decode(packed, state))
        else:
            weights.append(w)
            dense.append(w)
    a_stack = _rand(sum(ranks), k, seed=20, scale=0.05)
    a_list = list(torch.split(a_stack, list(ranks)))
    bs = [_rand(n, r, seed=30 + i, scale=0.05) for i, (n, r) in enumerate(zip(widths, ranks))]
    dy = _rand(m, sum(widths), seed=40)
    prior = _rand(m, k, seed=41)
    n0, ntail, rt = widths[0], sum(widths[1:]), sum(ranks)
    # dy_0 as a column block of a wider matrix, the tail pitched past its n_tail + r_total
    wide = torch.full((m, n0 + 24), float("nan"), device="cuda", dtype=torch.bfloat16)
    wide[:, 8:8 + n0] = dy[:, :n0]
    dy0 = wide[:, 8:8 + n0]
    store = torch.full((m, ntail + rt + 16), float("nan"), device="cuda", dtype=torch.bfloat16)
    tail = store[:, :ntail + rt]
    tail[:, :ntail] = dy[:, n0:]
    dx = prior.clone() if add else torch.full((m, k), float("nan"), device="cuda", dtype=torch.bfloat16)
    assert _call_lead(m, k, widths, ranks, weights, dy0, tail, a_stack, bs, dx, add) == 0
    again_store = store.clone()
    again_store[:, ntail:ntail + rt] = float("nan")
    again_dx = prior.clone() if add else torch.empty_like(dx)
    assert _call_lead(m, k, widths, ranks, weights, dy0, again_store[:, :ntail + rt], a_stack, bs, again_dx,
                      add) == 0
    joined_dx = prior.clone() if add else torch.empty_like(dx)
    joined_low = torch.empty(m, rt, device="cuda", dtype=torch.bfloat16)
    assert _call(m, k, widths, ranks, weights, dy, a_stack, bs, joined_dx, joined_low, add) == 0
    torch.cuda.synchronize()
    assert torch.equal(dx.view(torch.int16), again_dx.view(torch.int16))
    assert torch.equal(store.view(torch.int16), again_store.view(torch.int16))
    low = tail[:, ntail:]
    assert torch.equal(low.view(torch.int16), joined_low.view(torch.int16))   # the same rank-r products
    assert torch.equal(tail[:, :ntail].view(torch.int16), dy[:, n0:].view(torch.int16))   # read only
    cols = [sum(widths[:i]) for i in range(count + 1)]
    rcols = [sum(ranks[:i]) for i in range(count + 1)]
    want = prior.double() if add else torch.zeros(m, k, device="cuda", dtype=torch.float64)
    for i in range(count):
        dyi = dy[:, cols[i]:cols[i + 1]]
        want += dyi.double() @ dense[i].double() + low[:, rcols[i]:rcols[i + 1]].double() @ a_list[i].double()
        if m <= 1024:
            _, single_low = _single(dyi.contiguous(), weights[i], a_list[i].contiguous(), bs[i], m, widths[i], k,
                                    ranks[i])
            assert torch.equal(low[:, rcols[i]:rcols[i + 1]].view(torch.int16), single_low.view(torch.int16)), i
    want = want.to(torch.bfloat16).float()
    assert bool(torch.isfinite(dx.float()).all())
    assert ((dx.float() - want).norm() / want.norm()).item() <= 1e-3
    # both round one fp32 sum once: apart from rounding flips, one step of bf16 (2^-7 relative
    # to the larger magnitude) at most
    step = torch.maximum(dx.float().abs(), joined_dx.float().abs()) * 2.0 ** -7 + 1e-6
    assert bool(((dx.float() - joined_dx.float()).abs() <= step).all())


def test_group_input_gradient_lead_refuses_invalid_descriptions():
    lib = _native.library()
    m, k = 64, 64
    w = _rand(16, k, seed=1)
    dy0 = _rand(m, 16, seed=2)
    tail = _rand(m, 16 + 8, seed=5)
    a = _rand(8, k, seed=3)
    b = _rand(16, 4, seed=4)
    dx = torch.empty(m, k, device="cuda", dtype=torch.bfloat16)
    stream = _native.stream_of(dy0)

    def call(widths, ranks, dense, ldtail=24, tail_ptr=True, ws=None, count=None):
        count = len(widths) if count is None else count
        n_arr = (ctypes.c_int64 * max(len(widths), 1))(*widths)
        r_arr = (ctypes.c_int64 * max(len(ranks), 1))(*ranks)
        wd = (ctypes.c_void_p * max(len(dense), 1))(*dense)
        bb = (ctypes.c_void_p * max(len(widths), 1))(*[b.data_ptr()] * len(widths))
        return lib.ct_group_input_gradient_lead(dy0.data_ptr(), 16, tail.data_ptr() if tail_ptr else None, ldtail,
                                                count, n_arr, r_arr, wd, None, a.data_ptr(), bb, dx.data_ptr(), k,
                                                m, k, 0, None if ws is None else ws.data_ptr(),
                                                0 if ws is None else ws.numel(), stream)
    pair = (w.data_ptr(), w.data_ptr())
    assert call((16, 12), (4, 4), pair) == -_shape()                        # a width not a multiple of 8
    assert call((), (), (), count=0) == -_shape()                           # no projections
    assert call((16, 16), (4, 4), (w.data_ptr(), None)) == -_pointer()      # a weight missing
    assert call((16, 16), (4, 4), pair, tail_ptr=False) == -_pointer()      # no tail
    assert call((16, 16), (4, 4), pair, ldtail=23) == -_shape()             # tail narrower than 16 + 8
    assert call((16, 16), (4, 4), pair) == -_workspace()                    # no workspace for the weights
    small = torch.empty(4096, dtype=torch.uint8, device="cuda")
    assert call((16, 16), (4, 4), pair, ws=small) == -_workspace()          # too small for both


def test_group_input_gradient_refuses_invalid_descriptions():
    lib = _native.library()
    m, k = 64, 64
    w = _rand(16, k, seed=1)
    dy = _rand(m, 32, seed=2)
    a = _rand(8, k, seed=3)
    b = _rand(16, 4, seed=4)
    dx = torch.empty(m, k, device="cuda", dtype=torch.bfloat16)
    low = torch.empty(m, 8, device="cuda", dtype=torch.bfloat16)
    stream = _native.stream_of(dy)

    def call(widths, ranks, dense, count=None):
        count = len(widths) if count is None else count
        n_arr = (ctypes.c_int64 * max(len(widths), 1))(*widths)
        r_arr = (ctypes.c_int64 * max(len(ranks), 1))(*ranks)
        wd = (ctypes.c_void_p * max(len(dense), 1))(*dense)
        bb = (ctypes.c_void_p * max(len(widths), 1))(*[b.data_ptr()] * len(widths))
        return lib.ct_group_input_gradient(dy.data_ptr(), 32, count, n_arr, r_arr, wd, None, a.data_ptr(), bb,
                                           dx.data_ptr(), k, low.data_ptr(), 8, m, k, 0, None, 0, stream)
    assert call((16, 12), (4, 4), (w.data_ptr(), w.data_ptr())) == -_shape()      # a width not a multiple of 8
    assert call((), (), (), count=0) == -_shape()                                  # no projections
    assert call((16, 16), (4, 4), (w.data_ptr(), None)) == -_pointer()             # a weight missing
    assert call((16, 16), (4, 4), (w.data_ptr(), w.data_ptr())) == -_workspace()   # no workspace for w^T


def _shape():
    return 2


def _pointer():
    return 1


def _workspace():
    return 5


def _forward_single(x, weight, a, b, xa, m, n, k, r, bias=None):
    lib = _native.library()
    out = torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16)
    desc = None if isinstance(weight, torch.Tensor) else _native.nf4_descriptor(*weight)
    need = lib.ct_forward_linear_workspace(m, n, k, r, _native.nf4_kind(desc))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    status = lib.ct_forward_linear(x.data_ptr(), x.stride(0), weight.data_ptr() if desc is None else None, desc,
                                   a.data_ptr(), b.data_ptr(), None if bias is None else bias.data_ptr(),
                                   out.data_ptr(), n, xa.data_ptr(), xa.stride(0), 1,
                                   m, n, k, r, None, ws.data_ptr(), ws.numel(), _native.stream_of(x))
    assert status == 0, status
    return out


@pytest.mark.parametrize("m,k,widths,r,nf4,biased", [
    (600, 256, (512, 256), 16, True, (False, False)), (520, 128, (256, 264), 8, False, (False, False)),
    (8192, 512, (1024, 512), 64, True, (True, True)), (64, 128, (256, 256), 8, True, (False, False)),
    # 256 x 256 tiles here and per projection, the first projection with a bias
    (8192, 256, (2048, 2560), 16, True, (True, False)),
    # narrow outputs (k and v beside q): 64 x 64 tiles, the second one with a bias
    (8192, 512, (128, 128), 256, True, (True, True)), (600, 256, (192, 384), 16, True, (False, True)),
    (333, 128, (384, 136), 8, False, (True, True))])
def test_group_forward_matches_per_projection_forward(m, k, widths, r, nf4, biased):
    print(f"group forward: m={m} k={k} widths={widths} r={r} nf4={nf4} biased={biased}", flush=True)
    lib = _native.library()
    x = _rand(m, k, seed=1)
    weights = []
    for i, n in enumerate(widths):
        w = _rand(n, k, seed=2 + i, scale=0.02)
        weights.append(quantize_nf4(w) if nf4 else w)
    a_stack = _rand(2 * r, k, seed=5, scale=0.05)
    b_stack = _rand(sum(widths), r, seed=6, scale=0.05)
    xa = _rand(m, 2 * r, seed=7)
    outs = [torch.full((m, n), float("nan"), device="cuda", dtype=torch.bfloat16) for n in widths]
    biases = [_rand(n, seed=8 + i) if on else None for i, (n, on) in enumerate(zip(widths, biased))]
    bias_arr = (ctypes.c_void_p * 2)(*[None if b is None else b.data_ptr() for b in biases]) if any(biased) else None
    n_arr = (ctypes.c_int64 * 2)(*widths)
    dense = (ctypes.c_void_p * 2)(*[w.data_ptr() if isinstance(w, torch.Tensor) else None for w in weights])
    descs = [None if isinstance(w, torch.Tensor) else _native.nf4_descriptor(*w) for w in weights]
    packed = (ctypes.POINTER(_native.NF4Weight) * 2)(*[None if d is None else ctypes.pointer(d) for d in descs])
    out_arr = (ctypes.c_void_p * 2)(*[o.data_ptr() for o in outs])
    ld_arr = (ctypes.c_int64 * 2)(*widths)
    need = lib.ct_group_forward_workspace(m, 2, n_arr, k, r)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    status = lib.ct_group_forward(x.data_ptr(), k, 2, n_arr, dense, packed, b_stack.data_ptr(), xa.data_ptr(), 2 * r,
                                  bias_arr, out_arr, ld_arr, m, k, r, ws.data_ptr(), ws.numel(), _native.stream_of(x))
    if m <= 64:
        assert status == -2   # few rows: the caller runs the projections one by one
        return
    assert status == 0, status
    b_list = torch.split(b_stack, list(widths))
    for i, n in enumerate(widths):
        want = _forward_single(x, weights[i], a_stack[i * r:(i + 1) * r], b_list[i].contiguous(),
                               xa[:, i * r:(i + 1) * r], m, n, k, r, biases[i])
        torch.cuda.synchronize()
        assert torch.equal(outs[i].view(torch.int16), want.view(torch.int16)), i


def test_group_forward_rejects_invalid_descriptions():
    """ct_group_forward's checks run on the host, before any launch: the first width must
    start a tile (a multiple of 64), xa must hold both ranks, exactly one weight per
    projection, and a few-row call is left to the per-projection path."""
    lib = _native.library()
    k, r = 64, 8
    x = _rand(128, k, seed=1)
    w = _rand(256, k, seed=2)
    b_stack = _rand(256, r, seed=3)
    xa = _rand(128, 2 * r, seed=4)
    outs = [torch.empty(128, 128, device="cuda", dtype=torch.bfloat16) for _ in range(2)]
    stream = _native.stream_of(x)

    def call(widths, m=128, ldxa=2 * r, dense=None):
        n_arr = (ctypes.c_int64 * 2)(*widths)
        wd = (ctypes.c_void_p * 2)(*(dense if dense is not None else (w.data_ptr(), w.data_ptr())))
        out_arr = (ctypes.c_void_p * 2)(*[o.data_ptr() for o in outs])
        ld_arr = (ctypes.c_int64 * 2)(128, 128)
        return lib.ct_group_forward(x.data_ptr(), k, 2, n_arr, wd, None, b_stack.data_ptr(), xa.data_ptr(), ldxa, None,
                                    out_arr, ld_arr, m, k, r, None, 0, stream)
    assert call((96, 128)) == -_shape()                                # 96 columns: not a tile boundary
    assert call((128, 128), ldxa=r) == -_shape()                       # xa narrower than both ranks
    assert call((128, 128), dense=(w.data_ptr(), None)) == -_pointer()  # a weight missing
    assert call((128, 128), m=64) == -_shape()                         # few rows: per projection
    assert call((128, 128)) == -_workspace()                           # no workspace for [w_1; w_2]


@pytest.mark.parametrize("nf4", [False, True])
def test_rotated_group_backward_against_float64(nf4, monkeypatch):
    """q/k/v through project_group with rotary (q and k rotated, v not) at 300 rows, where the
    input gradient is one grouped contraction with q's upstream gradient rotated back into a
    buffer of its own and k's beside v's in the tail: every gradient within 1e-2 (relative
    Frobenius) of float64 autograd through the reference's host rotation
    (modeling/rotary.py's formula, kernels/linear.py:59-130's product sequence) with the
    same bf16 base weights."""
    from causal_tuner.kernels import linear
    from causal_tuner.kernels.linear import project_group
    from causal_tuner.modeling.lora import Projection
    from causal_tuner.modeling.rotary import rotate
    print(f"rotated q/k/v group backward vs float64 nf4={nf4}", flush=True)
    tokens, width, head_dim = 300, 512, 128
    calls = []
    original = linear.group_input_gradient_lead

    def counted(*args, **kwargs):
        calls.append(1)
        return original(*args, **kwargs)
    monkeypatch.setattr(linear, "group_input_gradient_lead", counted)
    modules = []
    for i, n in enumerate((1024, 256, 256)):
        torch.manual_seed(50 + i)
        module = Projection(width, n, bias=True, rank=16, device="cuda")
        if nf4:
            module.install_nf4(module.weight.detach().clone(), "cuda")
        torch.nn.init.normal_(module.lora_B, std=0.05)
        torch.nn.init.normal_(module.bias, std=0.1)
        modules.append(module)
    x = _rand(tokens, width, seed=60)
    angle = torch.rand(tokens, 32, device="cuda", generator=torch.Generator(device="cuda").manual_seed(61)) * 1e3
    cosine, sine = angle.cos().bfloat16(), angle.sin().bfloat16()
    xd = x.clone().requires_grad_(True)
    outs = project_group(modules, xd, rotary=(cosine, sine, head_dim))
    signals = [_rand(*t.shape, seed=70 + i) for i, t in enumerate(outs)]
    params = [xd, *(p for m in modules for p in (m.lora_A, m.lora_B))]
    grads = torch.autograd.grad(outs, params, signals)
    assert calls, "the grouped contraction did not run"

    x64 = x.double().cpu().requires_grad_(True)
    factors = [(m.lora_A.detach().double().cpu().requires_grad_(True),
                m.lora_B.detach().double().cpu().requires_grad_(True)) for m in modules]
    c64, s64 = cosine.double().cpu(), sine.double().cpu()
    outs64 = []
    for i, (m, (a, b)) in enumerate(zip(modules, factors)):
        w = m.base_weight().detach().double().cpu()
        y = x64 @ w.T + (x64 @ a.T) @ b.T + m.bias.detach().double().cpu()
        if i < 2:
            y = rotate(y.reshape(tokens, -1, head_dim), c64, s64).reshape(tokens, -1)
        outs64.append(y)
    want = torch.autograd.grad(outs64, [x64, *(t for pair in factors for t in pair)],
                               [s.double().cpu() for s in signals])
    for index, (got, ref) in enumerate(zip(grads, want)):
        err = ((got.double().cpu() - ref).norm() / ref.norm()).item()
        assert err <= 1e-2, (index, err)
