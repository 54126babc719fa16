"""The tiled LoRA MLP on the CPU in float64. TEST INFRASTRUCTURE ONLY.

Restates the reference's kernels/mlp_cuda.py: the SiLU-multiply `_activation` (10-35) with
its bf16 rounding points (silu rounded before the product; the backward's grad * up
rounded before the SiLU derivative), and the `_forward_into` / `_TiledLoRAMLP.backward`
sequence (58-143) over the three projections, with each projection's output, xa, low and
dx rounded to bf16 once (oracle/lora.py's convention).
"""

import torch

BF16 = torch.bfloat16


def _round(t):
    return t.to(BF16).double()


def silu_parts(gate):
    sig = torch.sigmoid(gate)
    return sig, _round(gate * sig)


def activation_forward(gate, up):
    """h = bf16(bf16(silu(g)) * u) (mlp_cuda.py:16-17,25), gate/up float64 of bf16 values."""
    _, act = silu_parts(gate)
    return _round(act * up)


def activation_backward(gate, up, grad):
    """(d gate, d up, hidden) of mlp_cuda.py:18-25, each rounded to bf16."""
    sig, act = silu_parts(gate)
    pg = _round(grad * up)
    dgate = pg * (sig * (1 + gate * (1 - sig)))
    return _round(dgate), _round(grad * act), _round(act * up)


def _project(x, w, a, b):
    xa = _round(x @ a.T)
    return _round(x @ w.T + xa @ b.T), xa


def oracle_mlp(x, weights, adapters, dy):
    """x [M, h], weights (Wg [i, h], Wu [i, h], Wd [h, i]), adapters ((A, B) x 3), dy [M, h].

    Returns out, dx and [(dA, dB)] x 3 in float64 (out, dx rounded to bf16)."""
    X, DY = _round(x), _round(dy)
    W = [_round(w) for w in weights]
    AB = [(_round(a), _round(b)) for a, b in adapters]
    gate, xa_g = _project(X, W[0], *AB[0])
    up, xa_u = _project(X, W[1], *AB[1])
    hidden = activation_forward(gate, up)
    out, _ = _project(hidden, W[2], *AB[2])
    # backward (mlp_cuda.py:131-141)
    low_d = _round(DY @ AB[2][1])
    dh = _round(DY @ W[2] + low_d @ AB[2][0])
    dgate, dup, hidden_b = activation_backward(gate, up, dh)
    xa_d = _round(hidden_b @ AB[2][0].T)
    grads = [None, None, (low_d.T @ hidden_b, DY.T @ xa_d)]
    dx = 0
    for index, (signal, xa) in enumerate(((dgate, xa_g), (dup, xa_u))):
        low = _round(signal @ AB[index][1])
        dx = dx + signal @ W[index] + low @ AB[index][0]
        grads[index] = (low.T @ X, signal.T @ xa)
    return out, _round(dx), grads
