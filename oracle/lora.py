"""One NF4-LoRA projection on the CPU: the reference's op sequence and a float64 oracle.

TEST INFRASTRUCTURE ONLY (checker and timed CPU baseline; never on the product path).

`reference_forward` / `reference_backward` restate the torch-op sequence the reference's
`_LoRAGroup` runs for a single projection (kernels/linear.py:59-130 with the helpers at
27-44), in bf16 on the CPU with fp32 dA/dB (accumulate's CPU branch, linear.py:20-24).

`oracle_projection` is the float64-accumulated oracle. It keeps the reference's bf16
rounding of its operands and of the rank-r intermediates (A, B cast at linear.py:70,108;
xa at 32/125; low at 37), accumulates everything else exactly and rounds out and dx once.
"""

import torch
from torch.nn import functional as F

BF16 = torch.bfloat16


def reference_forward(x, w, a, b, bias=None, tile=0):
    """out for one projection, as _LoRAGroup.forward computes it (linear.py:66-85)."""
    x = x.to(BF16)
    ac, bc = a.to(BF16), b.to(BF16)
    bias = None if bias is None else bias.to(BF16)
    rows = min(tile or 4096, len(x))
    low = torch.empty((rows, len(a)), dtype=BF16)
    if tile:
        out = torch.empty((len(x), len(w)), dtype=BF16)
        for start in range(0, len(x), tile):
            part = x[start:start+tile]
            # forward_linear (linear.py:27-33)
            if bias is None:
                torch.mm(part, w.T, out=out[start:start+tile])
            else:
                torch.addmm(bias, part, w.T, out=out[start:start+tile])
            torch.mm(part, ac.T, out=low[:len(part)])
            out[start:start+tile].addmm_(low[:len(part)], bc.T)
        return out
    out = F.linear(x, w, bias)                       # untiled base GEMM (linear.py:80)
    for start in range(0, len(x), 4096):             # bounded rank-r epilogues (linear.py:81-84)
        part = x[start:start+4096]
        torch.mm(part, ac.T, out=low[:len(part)])
        out[start:start+4096].addmm_(low[:len(part)], bc.T)
    return out


def reference_backward(x, w, a, b, dy, tile=0, dx=None, add=False):
    """(dx, da, db) for one projection, as _LoRAGroup.backward computes them (linear.py:95-130)."""
    x, dy = x.to(BF16), dy.to(BF16)
    ac, bc = a.to(BF16), b.to(BF16)
    tile = tile or 4096
    rows = min(tile, len(x))
    dx = torch.empty_like(x) if dx is None else dx
    da = torch.zeros_like(a) if len(x) == 0 else torch.empty_like(a)
    db = torch.zeros_like(b) if len(x) == 0 else torch.empty_like(b)
    low = torch.empty((rows, len(a)), dtype=BF16)
    xa = torch.empty((rows, len(a)), dtype=BF16)
    for start in range(0, len(x), tile):
        signal, part = dy[start:start+tile], x[start:start+tile]
        lo, xp = low[:len(signal)], xa[:len(signal)]
        # input_gradient (linear.py:36-39)
        torch.mm(signal, bc, out=lo)
        torch.addmm(dx[start:start+tile], signal, w, beta=1 if add else 0, out=dx[start:start+tile])
        dx[start:start+tile].addmm_(lo, ac)
        torch.mm(part, ac.T, out=xp)                 # xa recompute (linear.py:125)
        # parameter_gradients + accumulate's fp32 CPU branch (linear.py:42-44, 20-22)
        beta = 1 if start > 0 else 0
        da.addmm_(lo.T.float(), part.float(), beta=beta)
        db.addmm_(signal.T.float(), xp.float(), beta=beta)
    return dx, da, db


def oracle_projection(x, w, a, b, dy, bias=None, dx_in=None):
    """float64-accumulated oracle: (out, xa, dx, low, da, db).

    out = bf16(x w^T + bias + xa b^T), xa = bf16(x a^T); dx = bf16(dy w + low a (+ dx_in)),
    low = bf16(dy b); da = low^T x, db = dy^T xa in float64 (compare against fp32)."""
    X, W = x.to(BF16).double(), w.to(BF16).double()
    A, B = a.to(BF16).double(), b.to(BF16).double()
    DY = dy.to(BF16).double()
    xa = (X @ A.T).to(BF16)
    base = X @ W.T + (0 if bias is None else bias.to(BF16).double())
    out = (base + xa.double() @ B.T).to(BF16)
    low = (DY @ B).to(BF16)
    dx = DY @ W + low.double() @ A
    if dx_in is not None:
        dx = dx + dx_in.double()
    dx = dx.to(BF16)
    da = low.double().T @ X
    db = DY.T @ xa.double()
    return out, xa, dx, low, da, db


def projection_flops(m, k, n, r):
    """Algorithmic FLOPs of one projection fwd+bwd: 2M[2KN + 3r(K+N)] (no xa recompute)."""
    return 2 * m * (2 * k * n + 3 * r * (k + n))


def relative_error(actual, expected):
    """(max|a-r| / max|r|, ||a-r|| / ||r||) in float64."""
    a, r = actual.detach().double(), expected.detach().double()
    diff = (a - r).abs()
    scale = r.abs().max().clamp_min(1e-300)
    return float(diff.max() / scale), float((a - r).norm() / r.norm().clamp_min(1e-300))
