"""The fragment-major (fm) products of the verify step and the kernels that
write their operands, on the GPU:

* packing: the library's fm_pack read back by torch reshapes (fm_unpack) is
  the matrix, padding rows zero;
* wptv_gemm_fm_parts: the parts' sum against a plain FP32 product of the
  same bf16 operands, within 1e-5 of the largest value (the FP32
  accumulation order), at the step's shapes and at row counts that are not
  a multiple of 16;
* wptv_gemm_fm_swiglu: silu(g) * u of the bf16-rounded FP32 sums, within one
  bf16 rounding of the same formula on the FP32 product;
* the producers: the residual add + norm, the embedding + norm and the
  verify attention write the same bits in the fm layout as row-major."""

import pytest
import torch

from tests.formulas import relative_error
from wpt_amd import kernels, layers

pytestmark = pytest.mark.gpu


def operands(M, N, K, seed, device):
    generator = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=generator).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=generator) * 0.02).to(torch.bfloat16)
    return x.to(device), w.to(device)


@pytest.mark.parametrize("R, K, blocks", [(160, 2048, None), (37, 96, None), (5, 32, 4), (48, 64, 3)])
def test_fm_pack_reads_back_as_the_matrix(device, R, K, blocks):
    generator = torch.Generator().manual_seed(R + K)
    a = torch.randn(R, K, generator=generator).to(torch.bfloat16).to(device)
    packed = layers.fm_pack(a, blocks)
    rows = 16 * (blocks if blocks is not None else 2 * ((R + 31) // 32))
    assert packed.numel() == rows * K
    full = layers.fm_unpack(packed, rows, K)
    assert torch.equal(full[:R], a)
    assert not full[R:].any()
    # element 8 l + e of block (ks, rb) is row 16 rb + l % 16, column 32 ks + 8 (l // 16) + e
    blocks_ = rows // 16
    r, k = R - 1, K - 3
    l, e = 16 * ((k % 32) // 8) + r % 16, k % 8
    index = (((k // 32) * blocks_ + r // 16) * 64 + l) * 8 + e
    assert packed[index] == a[r, k]


@pytest.mark.parametrize("M, N, K", [
    (160, 2304, 2048),   # the exact layer's q/k/v at batch 32, k+1 = 5
    (160, 2048, 2048),   # the output projection
    (160, 2048, 5632),   # the down projection
    (320, 2304, 2048),   # batch 64: q/k/v in row quarters
    (320, 2048, 5632),   # batch 64: the down projection
    (300, 2048, 2048),   # rows in the last row group only partly real
    (37, 384, 512),      # rows that are not a multiple of 16
    (5, 64, 256),        # one verify step of one row
])
def test_fm_parts_sum_to_the_fp32_product(device, M, N, K):
    x, w = operands(M, N, K, seed=M + N + K, device=device)
    parts = layers.linear_fm_parts(layers.fm_pack(x), M, layers.FmWeight(w))
    assert parts.dtype == torch.float32 and parts.shape[1:] == (M, N) and 1 <= parts.shape[0] <= 8
    expected = x.float() @ w.float().T
    assert relative_error(parts.sum(0).cpu(), expected.cpu()) < 1e-5


def test_fm_parts_take_a_given_part_count(device):
    M, N, K = 160, 2048, 2048
    x, w = operands(M, N, K, seed=3, device=device)
    xf, wf = layers.fm_pack(x), layers.FmWeight(w)
    expected = (x.float() @ w.float().T).cpu()
    for splits in (1, 2, 4, 8):
        parts = layers.linear_fm_parts(xf, M, wf, splits=splits)
        assert parts.shape[0] == splits
        assert relative_error(parts.sum(0).cpu(), expected) < 1e-5
    with pytest.raises(NotImplementedError):
        layers.linear_fm_parts(xf, M, wf, splits=3)  # 16 k-steps a wave do not split in 3


@pytest.mark.parametrize("M, F, K", [(160, 5632, 2048), (320, 5632, 2048), (37, 384, 256), (5, 64, 512)])
def test_fm_swiglu_is_silu_gate_times_up(device, M, F, K):
    x, w = operands(M, 2 * F, K, seed=M + F, device=device)
    tiles = layers.interleave_gate_up(w)
    out = layers.linear_fm_swiglu(layers.fm_pack(x), M, layers.FmWeight(tiles))
    got = layers.fm_unpack(out, M, F).float().cpu()
    product = (x.float() @ w.float().T).cpu()
    g = product[:, :F].to(torch.bfloat16).float()
    u = product[:, F:].to(torch.bfloat16).float()
    expected = (g * torch.sigmoid(g) * u).to(torch.bfloat16).float()
    # the gate and up sums may round to neighbouring bf16 values: within a few bf16 steps of the output
    assert relative_error(got, expected) < 2e-2
    close = (got - expected).abs() <= 2 ** -7 * expected.abs() + 1e-6
    assert close.float().mean() > 0.99


@pytest.mark.parametrize("M", [160, 320])
def test_fm_swiglu_feeds_the_down_product(device, M):
    # the down product reads the SwiGLU output in place: parts of act . down^T
    F, D = 5632, 2048
    x, w = operands(M, 2 * F, D, seed=11, device=device)
    _, down = operands(M, D, F, seed=12, device=device)
    act = layers.linear_fm_swiglu(layers.fm_pack(x), M, layers.FmWeight(layers.interleave_gate_up(w)))
    parts = layers.linear_fm_parts(act, M, layers.FmWeight(down))
    expected = layers.fm_unpack(act, M, F).float() @ down.float().T
    assert relative_error(parts.sum(0).cpu(), expected.cpu()) < 1e-5


def test_rows_without_a_kernel_form_have_no_plan():
    # 161 to 288 rows (11 to 18 row blocks) and above 320: the decoder reads them on the row-major products
    assert layers.fm_plan(200, 2048, 2048) is None and layers.fm_plan(288, 2048, 2048) is None
    assert layers.fm_plan(321, 2048, 2048) is None
    assert layers.fm_plan(289, 2048, 2048) is not None and layers.fm_plan(160, 2048, 2048) is not None


def test_the_norms_write_the_same_bits_in_the_fm_layout(device):
    M, D, S = 160, 2048, 4
    generator = torch.Generator().manual_seed(7)
    h0 = torch.randn(M, D, generator=generator).to(torch.bfloat16).to(device)
    parts = torch.randn(S, M, D, generator=generator).to(device)
    weight = (1 + 0.1 * torch.randn(D, generator=generator)).to(device)
    h1, h2 = h0.clone(), h0.clone()
    y = torch.empty_like(h0)
    layers.add_rms_norm_parts(h1, parts, weight, y)
    yf = layers.fm_empty(M, D, device)
    layers.add_rms_norm_parts(h2, parts, weight, yf, fm=True)
    assert torch.equal(h1, h2)
    assert torch.equal(layers.fm_unpack(yf, M, D), y)

    B, T, V = 32, 5, 1000
    ids = torch.randint(0, V, (B, T), generator=generator).to(device)
    table = torch.randn(V, D, generator=generator).to(torch.bfloat16).to(device)
    lengths = torch.randint(0, 50, (B,), generator=generator).to(device)
    h, x = torch.empty(B, T, D, dtype=torch.bfloat16, device=device), torch.empty(B, T, D, dtype=torch.bfloat16,
                                                                                 device=device)
    positions = torch.empty(B, T, dtype=torch.long, device=device)
    layers.embed_rms_norm(ids, table, weight, h, x, lengths, positions)
    xf = layers.fm_empty(B * T, D, device)
    hf = torch.empty_like(h)
    layers.embed_rms_norm(ids, table, weight, hf, xf, lengths, positions, fm=True)
    assert torch.equal(hf, h)
    assert torch.equal(layers.fm_unpack(xf, B * T, D), x.reshape(B * T, D))


@pytest.mark.parametrize("B, N, splits", [(32, 4096, 0), (3, 200, 1), (5, 1000, 0)])
def test_verify_attention_writes_the_same_bits_in_the_fm_layout(device, B, N, splits):
    T, H, c = 5, 16, 128
    generator = torch.Generator().manual_seed(B + N)
    q = torch.randn(B, T, H, c, generator=generator).to(torch.bfloat16).to(device)
    table = torch.randn(B, N, 2 * c, generator=generator).to(torch.bfloat16).to(device)
    positions = (N - T + torch.arange(T)).expand(B, T).contiguous().to(device)
    k, v = table[..., :c], table[..., c:]
    out = kernels.verify_attention(q, k, v, positions, c ** -0.5, splits=splits)
    out_fm = kernels.verify_attention(q, k, v, positions, c ** -0.5, splits=splits, out_fm=True)
    assert torch.equal(layers.fm_unpack(out_fm, B * T, H * c), out.reshape(B * T, H * c))


@pytest.mark.parametrize("M, N, K", [
    (496, 32768, 2048),   # the tree verification's lm_head (16 x 31 node rows)
    (600, 512, 256),      # three row tiles, the last partial; two column tiles
    (321, 768, 64),       # the fewest rows of the wide tiles; two K chunks
    (1100, 2048, 2048),   # five row tiles by eight column tiles
    (40, 256, 32),        # one row tile, one K chunk, rows not a multiple of 16
])
def test_the_wide_fm_product_is_the_row_major_wide_product(device, M, N, K):
    # the same 256 x 256 tiles and 32x32x16 products on fm operands: the same
    # bits as the row-major form (which runs above 320 rows), within one bf16
    # rounding of an FP32 product
    x, w = operands(M, N, K, seed=M + K, device=device)
    got = layers.linear_fm_wide(layers.fm_pack(x), M, layers.FmWeight(w))
    assert got.shape == (M, N) and got.dtype == torch.bfloat16
    if M >= layers.WIDE_MIN_ROWS:
        assert torch.equal(got, layers.linear(x, w))
    assert relative_error(got.float().cpu(), (x.float() @ w.float().T).cpu()) < 1e-2
    wide32 = layers.linear_fm_wide(layers.fm_pack(x), M, layers.FmWeight(w), out_dtype=torch.float32)
    assert torch.equal(wide32, got.float())


def test_the_wide_fm_product_reads_x_with_more_row_blocks(device):
    # an fm operand holding more row blocks than its rows need (a producer's
    # padding): the rows past M are never read into the output
    M, N, K = 300, 512, 128
    x, w = operands(M, N, K, seed=3, device=device)
    padded = layers.fm_pack(x, 40)  # 640 rows of storage for 300
    assert torch.equal(layers.linear_fm_wide(padded, M, layers.FmWeight(w)),
                       layers.linear_fm_wide(layers.fm_pack(x), M, layers.FmWeight(w)))


def test_the_wide_fm_product_refuses_bad_shapes(device):
    x, w = operands(64, 320, 64, seed=4, device=device)
    with pytest.raises(ValueError):
        layers.linear_fm_wide(layers.fm_pack(x), 64, layers.FmWeight(w))  # N not a multiple of 256
    x2, w2 = operands(64, 256, 64, seed=4, device=device)
    with pytest.raises(ValueError):
        layers.linear_fm_wide(layers.fm_pack(x2)[: 2 * 16 * 64], 64, layers.FmWeight(w2))  # too few row blocks


@pytest.mark.parametrize("M, N, K", [(496, 32768, 2048), (300, 1024, 128), (40, 512, 64)])
def test_the_fused_head_argmax_is_the_argmax_of_the_bf16_logits(device, M, N, K):
    # the first maximal index of each row's bf16 logits, without storing them:
    # ties planted within a column tile (5, 6) and across tiles (N - 100), a
    # row of NaN and a row of infinities and NaN (torch.argmax takes a NaN as
    # the largest value, the first of several)
    generator = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=generator).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=generator) * 0.02).to(torch.bfloat16)
    rows_tied = torch.arange(0, M, 3)
    favourite = torch.full((K,), 0.05).to(torch.bfloat16)
    w[[5, 6, N - 100]] = favourite  # the same column three times (the last in another column tile)
    x[1] = float("nan")
    x[2, 0] = float("inf")  # +inf or -inf by the sign of column 0 of w, NaN where inf meets -inf
    x[2, 1] = float("-inf")
    x, w = x.to(device), w.to(device)
    x[rows_tied] = x[rows_tied].abs() + 0.5  # these rows prefer the planted columns
    x_fm, w_fm = layers.fm_pack(x), layers.FmWeight(w)
    best = layers.head_argmax_fm_wide(x_fm, M, w_fm)
    logits = layers.linear_fm_wide(x_fm, M, w_fm).float()
    expected = logits.argmax(-1).to(torch.int32)
    assert best.dtype == torch.int32 and best.shape == (M,)
    assert torch.equal(best, expected)
    assert best[1] == 0 and torch.isnan(logits[2]).any()
    assert (best[rows_tied[(rows_tied != 1) & (rows_tied != 2)]] == 5).all()
