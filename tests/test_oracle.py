"""Pins the CPU oracle (oracle/) before any GPU result is compared with it.

Each check is independent of the oracle's own formulas: the published construction of the
NF4 code book, torch's bf16 rounding, hand-built byte patterns with known answers,
brute-force nearest-code searches, a second (plain C) restatement, and algebraic
identities of the projection's gradients.
"""

import ctypes
import glob
import os

import numpy as np
import pytest
import torch

from oracle import lora, nf4

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_nf4_code_book_matches_normal_quantile_construction():
    from scipy.stats import norm
    offset = 0.9677083
    positive = norm.ppf(torch.linspace(offset, 0.5, 9)[:-1].numpy()).tolist()
    negative = (-norm.ppf(torch.linspace(offset, 0.5, 8)[:-1].numpy())).tolist()
    values = torch.tensor(positive + [0.0] * 241 + negative).sort().values
    values = values / values.max()
    nonzero = values[values != 0]
    built = torch.cat([nonzero[nonzero < 0], torch.zeros(1), nonzero[nonzero > 0]]).numpy()
    assert built.dtype == np.float32
    np.testing.assert_array_equal(built, nf4.NF4_CODE)


def test_bf16_rounding_matches_torch():
    g = torch.Generator().manual_seed(0)
    values = torch.cat([torch.randn(100000, generator=g) * 10.0 ** torch.randint(-30, 30, (100000,), generator=g),
                        torch.tensor([0.0, -0.0, 1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 3.3895314e38,
                                      1e-40, -1e-41, float("inf"), -float("inf")])])
    expected = values.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(nf4.bf16_bits(values.numpy()), expected)


def test_known_bytes_decode_high_nibble_first():
    packed = np.array([0xF0, 0x7A, 0xD4], dtype=np.uint8)
    out = nf4.dequantize(packed, np.array([2.0], np.float32), 6, blocksize=64, nested=False)
    np.testing.assert_array_equal(out, np.array([0x4000, 0xC000, 0x0000, 0x3EFC, 0x3F90, 0xBF12], np.uint16))


def test_odd_tail_ignores_the_padding_nibble():
    packed = np.array([0xF0, 0x7A, 0xDF], dtype=np.uint8)
    out = nf4.dequantize(packed, np.array([2.0], np.float32), 5, blocksize=64, nested=False)
    assert out.shape == (5,) and out[-1] == 0x3F90


def test_block_and_group_boundaries_select_their_own_scales():
    n, bs = 64 * 257, 64
    packed = np.full(n // 2, 0xFF, dtype=np.uint8)  # every element decodes code[15] = 1.0
    qabs = np.arange(257).astype(np.uint8)           # block g uses code2[g % 256]
    code2 = np.linspace(-1, 1, 256, dtype=np.float32)
    absmax2 = np.array([0.5, 4.0], np.float32)       # blocks 0..255 -> 0.5, block 256 -> 4.0
    offset = np.float32(0.25)
    out = nf4.dequantize(packed, qabs, n, bs, True, nf4.NF4_CODE, code2, absmax2, offset, 256, nf4.F32, nf4.F32)
    expect = np.array([np.float32(code2[g % 256] * absmax2[g // 256]) + offset for g in range(257)], np.float32)
    np.testing.assert_array_equal(out.reshape(257, 64), np.repeat(expect[:, None], 64, axis=1))


def test_nested_scale_is_multiply_then_separately_rounded_add():
    c = np.float32(1 + 2 ** -12)
    scales = nf4.block_scales(np.array([0], np.uint8), True, np.array([c] * 256, np.float32),
                              np.array([c], np.float32), np.float32(-1.0))
    # exact product 1 + 2^-11 + 2^-24 rounds (to even) to 1 + 2^-11 before the add;
    # a fused multiply-add would keep 2^-11 + 2^-24.
    assert scales[0] == np.float32(2 ** -11)


def test_storage_dtype_rounds_before_the_output_dtype():
    packed = np.array([0xC1], np.uint8)  # code[12], code[1]
    scale = np.array([0.0123], np.float32)
    f32 = nf4.dequantize(packed, scale, 2, 64, False, storage=nf4.F32, out=nf4.F32)
    bf16_then_f32 = nf4.dequantize(packed, scale, 2, 64, False, storage=nf4.BF16, out=nf4.F32)
    f16_then_bf16 = nf4.dequantize(packed, scale, 2, 64, False, storage=nf4.F16, out=nf4.BF16)
    np.testing.assert_array_equal(f32, (nf4.NF4_CODE[[12, 1]] * scale[0]).astype(np.float32))
    np.testing.assert_array_equal(bf16_then_f32.view(np.uint32) >> 16, np.array([0x3BB2, 0xBC0C]))
    expected = torch.tensor(f32).to(torch.float16).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(f16_then_bf16, expected)


@pytest.mark.parametrize("shape,blocksize,nested", [((17, 19), 64, True), ((71, 96), 128, False),
                                                    ((300, 129), 64, True), ((8, 4096), 4096, True)])
def test_quantizer_picks_the_nearest_code_and_round_trips(shape, blocksize, nested):
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(shape, generator=g) * 0.02).to(torch.bfloat16).float().numpy().reshape(-1)
    packed, state = nf4.quantize(w, blocksize, nested)
    n = w.size
    nib = np.empty(2 * packed.size, np.uint8)
    nib[0::2], nib[1::2] = packed >> 4, packed & 15
    nib = nib[:n]
    blocks = -(-n // blocksize)
    absmax = np.abs(np.pad(w, (0, blocks * blocksize - n))).reshape(blocks, blocksize).max(1)
    x = w / np.repeat(absmax, blocksize)[:n]
    dist = np.abs(x[:, None] - nf4.NF4_CODE[None, :].astype(np.float64))
    chosen = dist[np.arange(n), nib]
    assert np.all(chosen <= dist.min(1) + 1e-7)  # brute-force nearest code (ties aside)
    deq = nf4.bf16_to_f32(nf4.dequantize_state(packed, state))
    scale = np.repeat(absmax, blocksize)[:n]
    assert np.all(np.abs(deq - w) <= scale * 0.16 + 0.01 * scale + 1e-6)


def test_dynamic_map_and_binary_search_are_nearest():
    code = nf4.dynamic_map()
    assert code.shape == (256,) and np.all(np.diff(code) >= 0) and code[-1] == 1.0 and 0.0 in code
    rng = np.random.default_rng(0)
    for x in rng.uniform(-1, 1, 2000).astype(np.float32):
        q = nf4.dynamic_code(x, code)
        assert abs(float(code[q]) - float(x)) <= np.abs(code.astype(np.float64) - float(x)).min() + 1e-7


def test_dynamic_map_is_the_dynamic_tree_data_type():
    """The second-level code book against the bit-level definition of the dynamic tree data
    type (Dettmers et al., "8-bit Optimizers via Block-wise Quantization", 2022, sec. 2.1):
    after the sign bit, the number E of leading zero bits sets the scale 10^-E, the next 1
    bit is an indicator, and the F = 6 - E remaining bits pick one of 2^F equal bins of
    [0.1, 1], whose centre is the magnitude; the all-zero magnitude is 0, and the code of
    negative zero is used for 1.0. Enumerated over all 256 codes in float64 and compared
    with the linspace construction (fp32) within 2 ulp: any slip in the exponent count, the
    bins per decade, the bin centres or the signs changes a value by far more."""
    tree = []
    for code in range(256):
        negative, magnitude = code >> 7, code & 127
        if magnitude == 0:
            tree.append(1.0 if negative else 0.0)
            continue
        e = 7 - magnitude.bit_length()            # leading zeros of the 7-bit magnitude
        f = 6 - e                                 # fraction bits after the indicator
        fraction = magnitude & ((1 << f) - 1)
        value = 10.0 ** -e * (0.1 + (fraction + 0.5) * 0.9 / (1 << f))
        tree.append(-value if negative else value)
    tree = np.sort(np.array(tree))
    code = nf4.dynamic_map().astype(np.float64)
    assert np.all(np.abs(code - tree) <= 2 * np.spacing(np.abs(tree).astype(np.float32)).astype(np.float64))
    assert np.count_nonzero(code == 0) == 1 and code[-1] == 1.0
    for e in range(7):   # 2^(6-e) magnitudes in each decade, on each side
        inside = (np.abs(code) >= 0.1 * 10.0 ** -e) & (np.abs(code) < 10.0 ** -e)
        assert np.count_nonzero(inside & (code > 0)) == 2 ** (6 - e) == np.count_nonzero(inside & (code < 0))


def test_package_quantizer_matches_the_oracle_bit_for_bit():
    from causal_tuner.quant.nf4 import quantize_nf4, dynamic_map
    np.testing.assert_array_equal(dynamic_map().numpy(), nf4.dynamic_map())
    for shape, bs in (((17, 19), 64), ((130, 256), 64), ((64, 640), 128)):
        w = (torch.randn(shape) * 0.02).to(torch.bfloat16)
        packed, state = quantize_nf4(w, bs)
        p2, s2 = nf4.quantize(w.float().numpy(), bs, True, offset=state.offset.item())
        np.testing.assert_array_equal(packed.numpy().reshape(-1), p2)
        np.testing.assert_array_equal(state.absmax.numpy(), s2["absmax"])
        np.testing.assert_array_equal(state.state2.absmax.numpy(), s2["absmax2"])
        assert state.offset.item() == s2["offset"] and state.dtype == torch.bfloat16


def test_plain_c_restatement_matches_numpy():
    lib = ctypes.CDLL(os.path.join(ROOT, "oracle", "lib", "libnf4_oracle.so"))
    for n in (1, 19 * 17, 64 * 300 + 5, 1 << 16):
        w = (torch.randn(n) * 0.02).to(torch.bfloat16).float().numpy()
        packed, st = nf4.quantize(w, 64, True)
        out = np.empty(n, np.uint16)
        ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
        lib.ct_oracle_nf4_dequant_bf16(ptr(packed), ptr(st["absmax"]), ptr(st["code"]), ptr(st["code2"]),
                                       ptr(st["absmax2"]), ctypes.c_float(st["offset"]), ctypes.c_int64(n),
                                       ctypes.c_int64(64), ctypes.c_int64(256), ptr(out))
        np.testing.assert_array_equal(out, nf4.dequantize_state(packed, st))


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(HERE, "golden", "dequant_*.npz"))))
def test_oracle_reproduces_dequant_fixtures(path):
    f = np.load(path)
    rows, cols, bs, nested = (int(v) for v in f["meta"])
    storage = str(f["storage"])
    for out in (nf4.BF16, nf4.F16, nf4.F32):
        got = nf4.dequantize(f["packed"], f["absmax"], rows * cols, bs, bool(nested), f["code"],
                             f["code2"] if nested else None, f["absmax2"] if nested else None,
                             f["offset"] if nested else None, 256, storage, out)
        np.testing.assert_array_equal(got, f[f"expected_{out}"])


def _bf16(bits):
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)


def test_projection_oracle_against_loops_and_identities():
    g = torch.Generator().manual_seed(5)
    m, k, n, r = 3, 5, 4, 2
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = torch.randn(n, k, generator=g).to(torch.bfloat16)
    a, b = torch.randn(r, k, generator=g), torch.randn(n, r, generator=g)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    dy = torch.randn(m, n, generator=g).to(torch.bfloat16)
    out, xa, dx, low, da, db = lora.oracle_projection(x, w, a, b, dy, bias)
    X, W, DY = x.double().tolist(), w.double().tolist(), dy.double().tolist()
    A, B = a.to(torch.bfloat16).double().tolist(), b.to(torch.bfloat16).double().tolist()
    XA = [[sum(X[i][q] * A[j][q] for q in range(k)) for j in range(r)] for i in range(m)]
    assert torch.equal(xa, torch.tensor(XA, dtype=torch.float64).to(torch.bfloat16))
    XA = xa.double().tolist()
    OUT = [[sum(X[i][q] * W[o][q] for q in range(k)) + float(bias[o]) + sum(XA[i][j] * B[o][j] for j in range(r))
            for o in range(n)] for i in range(m)]
    assert torch.equal(out, torch.tensor(OUT, dtype=torch.float64).to(torch.bfloat16))
    LOW = low.double().tolist()
    DX = [[sum(DY[i][o] * W[o][q] for o in range(n)) + sum(LOW[i][j] * A[j][q] for j in range(r))
           for q in range(k)] for i in range(m)]
    assert torch.equal(dx, torch.tensor(DX, dtype=torch.float64).to(torch.bfloat16))
    DA = [[sum(LOW[i][j] * X[i][q] for i in range(m)) for q in range(k)] for j in range(r)]
    DB = [[sum(DY[i][o] * XA[i][j] for i in range(m)) for j in range(r)] for o in range(n)]
    assert torch.allclose(da, torch.tensor(DA, dtype=torch.float64), rtol=1e-12, atol=1e-12)
    assert torch.allclose(db, torch.tensor(DB, dtype=torch.float64), rtol=1e-12, atol=1e-12)


def test_projection_oracle_adjoint_identities():
    g = torch.Generator().manual_seed(6)
    m, k, n, r = 64, 96, 80, 8
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    a, b = torch.randn(r, k, generator=g) * 0.2, torch.randn(n, r, generator=g) * 0.1
    dy = torch.randn(m, n, generator=g).to(torch.bfloat16)
    out, xa, dx, low, da, db = lora.oracle_projection(x, w, a, b, dy)
    lora_part = xa.double() @ b.to(torch.bfloat16).double().T
    total = (dy.double() * lora_part).sum()
    # <dA, A> = <dB, B> = <dy, xa b^T> up to the bf16 rounding of low and xa
    assert abs(float((da * a.to(torch.bfloat16).double()).sum() - total)) <= 2e-2 * abs(float(total))
    assert abs(float((db * b.to(torch.bfloat16).double()).sum() - total)) <= 1e-9 * abs(float(total)) + 1e-9
    # <dy, x w^T> = <dy w, x> for the base path (b = 0 isolates it)
    _, _, dx0, _, _, _ = lora.oracle_projection(x, w, a, torch.zeros_like(b), dy)
    base = (dy.double() * (x.double() @ w.double().T)).sum()
    assert abs(float((dx0.double() * x.double()).sum() - base)) <= 1e-2 * float(dy.double().abs().sum())


def test_reference_sequence_within_parity_tolerance_of_oracle():
    g = torch.Generator().manual_seed(7)
    m, k, n, r = 512, 1024, 1024, 16
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    a = (torch.rand(r, k, generator=g) * 2 - 1) * (6 / k) ** 0.5
    b = torch.randn(n, r, generator=g) * 0.01
    dy = torch.randn(m, n, generator=g).to(torch.bfloat16)
    out, xa, dx, _, da, db = lora.oracle_projection(x, w, a, b, dy)
    ref_out = lora.reference_forward(x, w, a, b)
    ref_dx, ref_da, ref_db = lora.reference_backward(x, w, a, b, dy)
    for got, want in ((ref_out, out), (ref_dx, dx), (ref_da, da), (ref_db, db)):
        worst, norm = lora.relative_error(got, want)
        assert worst <= 2e-2 and norm <= 1e-2, (worst, norm)
    # the reference test's own dB formula (test_fast_training.py:116) on the oracle's xa bits
    expected_b = dy.float().T @ xa.float()
    torch.testing.assert_close(db.float(), expected_b, rtol=2e-5, atol=2e-5)


def test_oracle_reproduces_projection_fixture():
    f = np.load(os.path.join(HERE, "golden", "projection_37x96x80_r8.npz"))
    w = _bf16(f["expected_w"])
    out, xa, dx, low, da, db = lora.oracle_projection(_bf16(f["x"]), w, torch.from_numpy(f["a"]),
                                                      torch.from_numpy(f["b"]), _bf16(f["dy"]), _bf16(f["bias"]))
    for got, key in ((out, "out"), (xa, "xa"), (dx, "dx"), (low, "low")):
        assert torch.equal(got, _bf16(f[f"expected_{key}"])), key
    np.testing.assert_array_equal(da.numpy(), f["expected_da"])
    np.testing.assert_array_equal(db.numpy(), f["expected_db"])
    packed_state = {"n": w.numel(), "blocksize": 64, "nested": True, "code": f["code"], "absmax": f["absmax"],
                    "code2": f["code2"], "absmax2": f["absmax2"], "offset": f["offset"], "storage": nf4.BF16}
    np.testing.assert_array_equal(nf4.dequantize_state(f["packed"], packed_state), f["expected_w"].reshape(-1))
