"""The skinny bf16 matrix product (wptv_gemm, through wpt_amd.layers.linear)
against a plain PyTorch FP32 product of the same bf16 operands, on the GPU:
within 1e-2 of the largest expected value (bf16 output rounding and the FP32
accumulation order), and the FP32 output exactly the bf16-rounded product's
value as FP32 where the two round alike."""

import pytest
import torch

from tests.formulas import relative_error
from wpt_amd import layers

pytestmark = pytest.mark.gpu


def operands(M, N, K, seed, device):
    generator = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=generator).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=generator) * 0.02).to(torch.bfloat16)
    return x.to(device), w.to(device)


@pytest.mark.parametrize("M, N, K, splits", [
    (160, 2304, 2048, 0),    # the q/k/v projection at batch 32, k+1 = 5
    (160, 2048, 2048, 0),    # the output projection
    (160, 11264, 2048, 0),   # SwiGLU gate and up
    (160, 2048, 5632, 0),    # the down projection
    (320, 2048, 2048, 0),    # batch 64
    (496, 1024, 2048, 0),    # the tree's 16 x 31 rows (lm_head shape, fewer columns)
    (160, 32768, 2048, 0),   # the lm_head at batch 32, k+1 = 5 (128-column tiles)
    (320, 32768, 2048, 0),   # the lm_head at batch 64
    (496, 32768, 2048, 0),   # the tree config's lm_head over 16 x 31 node rows
    (17, 192, 320, 3),       # rows that are not a multiple of 16, an uneven K split
    (64, 128, 64, 1),        # one K chunk
    # the wide 256 x 256 tiles (above 320 rows, N a multiple of 256, K of 32)
    (321, 256, 64, 0),       # the fewest rows they take; two K chunks, fewer than the ring's lead
    (600, 512, 256, 0),      # three row tiles, the last one partial; two column tiles (no XCD grouping)
    (1100, 2048, 2048, 0),   # five row tiles by 8 column tiles (the XCD grouping)
    (512, 768, 32, 0),       # one K chunk
])
def test_linear_matches_the_fp32_product(device, M, N, K, splits):
    x, w = operands(M, N, K, seed=M + N + K, device=device)
    expected = x.float() @ w.float().T
    got = layers.linear(x, w, splits=splits)
    assert got.dtype == torch.bfloat16 and got.shape == (M, N)
    assert relative_error(got.float().cpu(), expected.cpu()) < 1e-2


def test_fp32_output_is_the_bf16_rounded_product(device):
    M, N, K = 160, 4096, 2048
    x, w = operands(M, N, K, seed=5, device=device)
    got = layers.linear(x, w, out_dtype=torch.float32)
    bf16 = layers.linear(x, w)
    assert got.dtype == torch.float32
    # the same FP32 sums rounded once: identical to the bf16 output's values
    assert torch.equal(got, bf16.float())
    assert relative_error(got.cpu(), (x.float() @ w.float().T).cpu()) < 1e-2


def test_wide_fp32_output_is_the_bf16_rounded_product(device):
    # the lm_head's 128-column tiles: the FP32 output holds the bf16 output's values
    M, N, K = 160, 32768, 2048
    x, w = operands(M, N, K, seed=9, device=device)
    got = layers.linear(x, w, out_dtype=torch.float32)
    assert torch.equal(got, layers.linear(x, w).float())


def test_wide_tiles_fp32_output_is_the_bf16_rounded_product(device):
    # the wide tiles' FP32 output holds the bf16 output's values (the
    # reference's .float() of the autocast product), rows past the last whole tile included
    M, N, K = 496, 4096, 2048
    x, w = operands(M, N, K, seed=11, device=device)
    got = layers.linear(x, w, out_dtype=torch.float32)
    assert got.dtype == torch.float32 and got.shape == (M, N)
    assert torch.equal(got, layers.linear(x, w).float())
    assert relative_error(got.cpu(), (x.float() @ w.float().T).cpu()) < 1e-2


def test_wide_tiles_write_no_row_past_the_output(device):
    # a 330-row output inside a larger buffer: the rows after it stay untouched
    M, N, K = 330, 512, 128
    x, w = operands(M, N, K, seed=12, device=device)
    buffer = torch.full((M + 40, N), 7.0, dtype=torch.bfloat16, device=device)
    from wpt_amd import _lib

    check = _lib.check
    library = _lib.lib()
    check(library.wptv_gemm(x.data_ptr(), K, w.data_ptr(), K, M, N, K, buffer.data_ptr(), N,
                            _lib.dtype_code(torch.bfloat16), 0, None, 0, _lib.stream(device)), "gemm")
    torch.cuda.synchronize()
    assert torch.all(buffer[M:] == 7.0)
    assert relative_error(buffer[:M].float().cpu(), (x.float() @ w.float().T).cpu()) < 1e-2


def test_splits_agree(device):
    M, N, K = 160, 512, 2048
    x, w = operands(M, N, K, seed=6, device=device)
    one = layers.linear(x, w, splits=1).float()
    for splits in (2, 5, 32):
        assert (layers.linear(x, w, splits=splits).float() - one).abs().max() <= 2e-2 * one.abs().max()


def test_batched_rows_and_bad_shapes(device):
    x, w = operands(160, 256, 128, seed=7, device=device)
    got = layers.linear(x.reshape(32, 5, 128), w)
    assert got.shape == (32, 5, 256)
    assert relative_error(got.reshape(160, 256).float().cpu(), (x.float() @ w.float().T).cpu()) < 1e-2
    with pytest.raises(NotImplementedError):
        layers.linear(x, w[:100])            # N not a multiple of 64
    with pytest.raises(NotImplementedError):
        # above 512 rows only the wide tiles serve, and they need N a multiple of 256
        layers.linear(torch.zeros(600, 128, dtype=torch.bfloat16, device=device), w[:192])
    with pytest.raises(ValueError):
        layers.linear(x.float(), w)


def test_parts_sum_to_the_product_and_feed_the_norm(device):
    # the down projection's shape: parts summed by add_rms_norm_parts equal
    # the reduced product fed to add_rms_norm
    M, N, K = 160, 2048, 5632
    x, w = operands(M, N, K, seed=8, device=device)
    parts = layers.linear_parts(x, w)
    assert parts.dtype == torch.float32 and parts.shape[1:] == (M, N) and 1 <= parts.shape[0] <= 8
    assert relative_error(parts.sum(0).cpu(), (x.float() @ w.float().T).cpu()) < 1e-3
    generator = torch.Generator().manual_seed(9)
    h0 = torch.randn(M, N, generator=generator).to(torch.bfloat16).to(device)
    weight = (1 + 0.1 * torch.randn(N, generator=generator)).to(device)
    h1, y1 = h0.clone(), torch.empty_like(h0)
    layers.add_rms_norm_parts(h1, parts, weight, y1)
    h2, y2 = h0.clone(), torch.empty_like(h0)
    layers.add_rms_norm(h2, parts.sum(0).to(torch.bfloat16), weight, y2)
    # the same bf16 delta up to the order of the FP32 part sums
    assert (h1.float() - h2.float()).abs().max() <= 2e-2 * h2.float().abs().max()
    assert relative_error(y1.float().cpu(), y2.float().cpu()) < 1e-2


@pytest.mark.parametrize("M", [1, 5, 160, 320, 512])
def test_the_fused_swiglu_product_equals_the_product_then_swiglu(device, M):
    # the epilogue rounds the gate and up halves to bf16 as the product's
    # bf16 output holds them, then silu(g) * u rounded once: bit for bit the
    # product followed by wptv_swiglu
    from wpt_amd import layers

    generator = torch.Generator().manual_seed(M)
    F, K = 512, 256
    x = torch.randn(M, K, generator=generator).to(torch.bfloat16).to(device)
    w = (torch.randn(2 * F, K, generator=generator) * 0.05).to(torch.bfloat16).to(device)
    expected = layers.swiglu(layers.linear(x, w, splits=1))
    got = layers.linear_swiglu(x, layers.interleave_gate_up(w))
    assert got.shape == (M, F) and got.dtype == torch.bfloat16
    assert torch.equal(got, expected)
