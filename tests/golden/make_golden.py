"""Write the NF4 / projection fixtures in tests/golden/ from the CPU oracle.

The reference stores no golden vectors for this path (its NF4 tests draw random data and
compare against bitsandbytes at run time), so these fixtures are produced by the oracle
from seeded inputs and pinned by tests/test_oracle.py; the GPU tests compare the HIP
kernels against them. Regenerate with `python tests/golden/make_golden.py`.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import lora, nf4  # noqa: E402

# (name, shape, blocksize, nested, storage dtype, seed)
DEQUANT_CASES = [
    ("odd_17x19_bs64_nested_bf16", (17, 19), 64, True, nf4.BF16, 11),
    ("r71x96_bs64_nested_bf16", (71, 96), 64, True, nf4.BF16, 12),
    ("r71x96_bs128_plain_f16", (71, 96), 128, False, nf4.F16, 13),
    ("r71x96_bs4096_nested_f32", (71, 96), 4096, True, nf4.F32, 14),
    ("r130x256_bs64_nested_bf16", (130, 256), 64, True, nf4.BF16, 15),
]
TORCH = {nf4.BF16: torch.bfloat16, nf4.F16: torch.float16, nf4.F32: torch.float32}


def dequant_case(shape, blocksize, nested, storage, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(shape, generator=g) * 0.02).to(TORCH[storage]).float().numpy()
    packed, state = nf4.quantize(w, blocksize, nested, storage)
    arrays = {"packed": packed, "absmax": state["absmax"], "code": state["code"]}
    if nested:
        arrays.update(code2=state["code2"], absmax2=state["absmax2"], offset=np.float32(state["offset"]))
    for out in (nf4.BF16, nf4.F16, nf4.F32):
        arrays[f"expected_{out}"] = nf4.dequantize_state(packed, state, out)
    arrays["meta"] = np.array([shape[0], shape[1], blocksize, int(nested)], dtype=np.int64)
    arrays["storage"] = np.array(storage)
    return arrays


def projection_case(m=37, k=96, n=80, r=8, seed=21):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    packed, state = nf4.quantize(w.float().numpy(), 64, True, nf4.BF16)
    wq = torch.from_numpy(nf4.bf16_to_f32(nf4.dequantize_state(packed, state))).reshape(n, k).to(torch.bfloat16)
    a = (torch.rand(r, k, generator=g) * 2 - 1) * (6 / k) ** 0.5
    b = torch.randn(n, r, generator=g) * 0.01
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16)
    dy = torch.randn(m, n, generator=g).to(torch.bfloat16)
    out, xa, dx, low, da, db = lora.oracle_projection(x, wq, a, b, dy, bias)
    bits = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    return {
        "x": bits(x), "packed": packed, "absmax": state["absmax"], "code": state["code"], "code2": state["code2"],
        "absmax2": state["absmax2"], "offset": np.float32(state["offset"]), "a": a.numpy(), "b": b.numpy(),
        "bias": bits(bias), "dy": bits(dy), "expected_w": bits(wq), "expected_out": bits(out),
        "expected_xa": bits(xa), "expected_dx": bits(dx), "expected_low": bits(low),
        "expected_da": da.numpy(), "expected_db": db.numpy(), "meta": np.array([m, k, n, r], dtype=np.int64),
    }


def main():
    for name, shape, blocksize, nested, storage, seed in DEQUANT_CASES:
        np.savez_compressed(os.path.join(HERE, f"dequant_{name}.npz"),
                            **dequant_case(shape, blocksize, nested, storage, seed))
    np.savez_compressed(os.path.join(HERE, "projection_37x96x80_r8.npz"), **projection_case())
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main()
