"""The library's launch plans, read through its workspace queries (pure host functions, no
GPU needed): the split counts that the GEMM, the few-row kernels and the parameter
gradients choose for the benchmarked shapes. A query returns splits x rows x cols x 4
bytes of fp32 partials when the reduction is split and 0 (or only the decoded weight)
when it is not, so each assertion pins one planning rule."""

import pytest

from causal_tuner.kernels import _native

F32 = 4


def _gemm_ws(m, n, k, trans_b=1):
    return _native.library().ct_gemm_workspace(m, n, k, 0, trans_b, _native.CT_BF16)


@pytest.mark.parametrize("m,n,k,splits", [
    # 65-511 rows: one round of 256 x 256 workgroups, at least 8 k-tiles per split, at most 32
    (128, 2048, 49152, 32),    # the projection loss's d hidden per 128-row tile
    (256, 24576, 6144, 2),     # C5 at 256 rows, 96 output tiles
    (256, 6144, 24576, 10),    # C5 at 256 rows, 24 output tiles
    (384, 2048, 49152, 16),
    # from 512 rows: reductions of at least 8192 into an output short of one round
    (512, 2048, 16384, 16),
    (2048, 2048, 49152, 4),
    (4096, 2048, 8448, 2),     # C4's down forward and gate/up dx
])
def test_split_route_counts(m, n, k, splits):
    assert _gemm_ws(m, n, k) == splits * m * n * F32


@pytest.mark.parametrize("m,n,k", [
    (4096, 2048, 2304),        # C4's q/o projections: the 128 x 128 grid, no partials
    (2048, 2048, 8000),        # a reduction just under 8192
    (8192, 4096, 11264),       # C3: the output fills the 256 x 256 grid
    (16384, 6144, 24832),      # C5 at 16384 rows
])
def test_no_split_where_the_grid_fills_or_the_reduction_is_short(m, n, k):
    assert _gemm_ws(m, n, k) == 0


@pytest.mark.parametrize("m,n,k,splits", [
    (8192, 256, 4096, 4),      # rank-r products over a reduction of at least 4096: 128 x 128 tiles, 4 splits
    (8192, 256, 11008, 4),
    (8192, 768, 4096, 0),      # the stacked q/k/v factors: 384 tiles of 128 fill the GPU unsplit
    (4096, 256, 8192, 4),
    (4096, 256, 2048, 0),      # over 2048 the unsplit 64 x 64 grid
    (4096, 768, 2048, 0),
])
def test_rank_r_product_splits(m, n, k, splits):
    assert _gemm_ws(m, n, k) == splits * m * n * F32


@pytest.mark.parametrize("m,n,k,trans_b,splits", [
    # few rows: the count (up to one round of resident slots) that spreads the workgroups
    # most evenly over the 256 CUs; rows kernel for trans_b=1, columns kernel for 0
    (16, 24576, 6144, 1, 2),
    (16, 6144, 24576, 1, 8),
    (16, 6144, 24576, 0, 16),
    (16, 24576, 6144, 0, 4),
    (64, 24576, 6144, 1, 2),
    (64, 6144, 24576, 1, 8),   # 96 column blocks, 3 resident per CU: 8 x 96 = 768 workgroups, one round
    (64, 6144, 24576, 0, 5),   # 48 column blocks: 5 x 48 = 240, not 6 x 48 = 288
    (64, 24576, 6144, 0, 1),   # 192 column blocks: one round unsplit
])
def test_few_row_split_counts(m, n, k, trans_b, splits):
    assert _gemm_ws(m, n, k, trans_b) == (splits * m * n * F32 if splits > 1 else 0)


@pytest.mark.parametrize("m,n,k,r,tile,splits", [
    (8192, 4096, 4096, 256, 256, 8),     # C3's q and o: 256 x 256 tiles, 8 splits
    (8192, 11008, 4096, 256, 256, 4),    # C3's gate and up
    (8192, 128, 4096, 256, 128, 3),      # C3's k and v: fewer than 32 tiles of 256 -> 128 x 128
    (4096, 2048, 2048, 256, 128, 4),     # C4's q and o
    (4096, 128, 2048, 256, 128, 7),      # C4's k and v
    (4096, 8192, 2048, 256, 256, 6),     # C4's gate and up
])
def test_parameter_gradient_plans(m, n, k, r, tile, splits):
    width = -(-k // tile) * tile + n
    assert _native.library().ct_parameter_gradients_workspace(m, n, k, r) == splits * r * width * F32


@pytest.mark.parametrize("m,n,k,r,tile", [
    (1024, 24576, 6144, 256, 128),   # up to 2048 tokens: unsplit, 128 x 128 tiles
    (16, 24576, 6144, 256, 128),
    (512, 1024, 1024, 16, 128),      # C1: rank 16 over 512 tokens, one direct 128 x 128 grid
    (512, 256, 960, 16, 128),        # ranks up to 64 over at most 512 tokens: 128 x 128
    (513, 256, 960, 16, 64),         # past 512 tokens: 64 x 64 tiles, too short to split
])
def test_parameter_gradients_unsplit(m, n, k, r, tile):
    """One split: the query still sizes one set of partials (the kernel writes dA and dB
    directly when it can, into the workspace otherwise)."""
    width = -(-k // tile) * tile + n
    assert _native.library().ct_parameter_gradients_workspace(m, n, k, r) == r * width * F32


@pytest.mark.parametrize("m,decoded_fwd,decoded_dx", [
    (256, False, False),   # both fused: the packed weight is decoded into LDS tile by tile
    (257, False, True),    # dx decodes w^T first once a second 256-row tile is needed
    (384, False, True),
    (511, False, True),
    (512, True, True),     # the forward from 512
])
def test_nf4_decode_first_thresholds(m, decoded_fwd, decoded_dx):
    """An NF4 weight the entry point decodes first adds its bf16 copy (out x in x 2 bytes)
    to the workspace query; C5's 6144 -> 24576 projection, rank 256."""
    lib = _native.library()
    weight = 24576 * 6144 * 2
    assert (lib.ct_forward_linear_workspace(m, 24576, 6144, 256, 1) >= weight) == decoded_fwd
    assert (lib.ct_input_gradient_workspace(m, 24576, 6144, 256, 1) >= weight) == decoded_dx


def test_parameter_gradient_runs():
    """Projections after the first share one dA/dB call when the cross products of their
    dB^T stay under a tenth of the useful ones: k and v beside q (C3), not gate and up, not
    three wide outputs."""
    from causal_tuner.kernels.linear import param_run
    assert param_run([256, 256, 256], [4096, 128, 128], 4096) == (1, 3)
    assert param_run([256, 256], [11008, 11008], 4096) is None
    assert param_run([256, 256, 256], [4096, 4096, 4096], 4096) is None
    assert param_run([256, 128, 256], [4096, 128, 128], 4096) is None   # ranks differ
    assert param_run([256, 256, 256], [2048, 128, 128], 2048) == (1, 3)   # C4's k and v


def test_stacked_views_need_one_storage():
    """Factors cast into one buffer stack as a view; tensors of different storages are
    copied even when their addresses happen to follow each other."""
    import torch
    from causal_tuner.kernels.linear import _adjacent, stacked_rows
    buffer = torch.arange(48, dtype=torch.float32)
    a, b = buffer[:24].view(4, 6), buffer[24:].view(4, 6)
    stacked = stacked_rows([a, b])
    assert stacked.data_ptr() == a.data_ptr() and torch.equal(stacked, buffer.view(8, 6))
    # a copy of b placed right after a in address terms cannot be emulated on the host, so
    # check the storage test directly: a separate tensor is copied, never viewed
    other = b.clone()
    assert torch.equal(stacked_rows([a, other]), torch.cat([a, other]))
    assert stacked_rows([a, other]).data_ptr() != a.data_ptr()
    matrix = torch.arange(30, dtype=torch.float32).view(5, 6)
    joined = _adjacent([matrix[:, 1:3], matrix[:, 3:6]])
    assert joined is not None and torch.equal(joined, matrix[:, 1:6])
    assert _adjacent([matrix[:, 1:3], matrix.clone()[:, 3:6]]) is None
