"""Pins the oracle decoder's autocast mode (CPU), the restatement of the
reference's bf16 GPU pass (model.py:466 runs extend under
torch.autocast(bfloat16)):

* its matrix product is torch's own bf16 product under CPU autocast, within
  one bf16 rounding step (both take bf16 inputs and accumulate in FP32; the
  order of the FP32 sums may differ);
* its norm is the reference's nn.RMSNorm module applied to the bf16 input,
  bit for bit, and returns bf16;
* its window attention is attention.py:74-82 run under CPU autocast on bf16
  tensors, within one bf16 step;
* a decoder of every layer kind scores within bf16 rounding of the FP32
  oracle (close, and not equal: the rounding happens), reading in pieces
  gives the scores of reading whole within the same bound, and its residual
  stream is bf16."""

import pytest
import torch
import torch.nn.functional as F

from oracle import attention, decoder
from tests.test_oracle_cache import C, H, IDS, KINDS, LAYERS, PIECES, V, weights

BF16_STEP = 2.0 ** -7  # the relative spacing of bf16 values


def within_one_bf16_step(got, expected):
    gap = (got.float() - expected.float()).abs()
    return bool((gap <= BF16_STEP * expected.float().abs() + 1e-30).all())


def test_the_product_is_torch_s_autocast_bf16_product():
    generator = torch.Generator().manual_seed(0)
    x = torch.randn(37, 256, generator=generator)
    w = torch.randn(96, 256, generator=generator).to(torch.bfloat16).float()
    got = decoder.bf16_linear(x, w)
    with torch.autocast("cpu", dtype=torch.bfloat16):
        expected = F.linear(x, w)
    assert got.dtype == expected.dtype == torch.bfloat16
    assert within_one_bf16_step(got, expected)


def test_the_norm_is_the_reference_module_on_a_bf16_input():
    generator = torch.Generator().manual_seed(1)
    x = torch.randn(5, 64, generator=generator).to(torch.bfloat16)
    weight = 1 + 0.1 * torch.randn(64, generator=generator)
    module = torch.nn.RMSNorm(64, eps=decoder.EPS)
    with torch.no_grad():
        module.weight.copy_(weight)
        expected = module(x)
    m = decoder.Decoder(weights(), LAYERS, H, C, autocast=True)
    got = m._norm(x, weight)
    assert got.dtype == torch.bfloat16 and torch.equal(got, expected)


def test_window_attention_is_the_reference_form_under_autocast():
    # attention.py:74-82 as the reference writes it, run under CPU autocast
    generator = torch.Generator().manual_seed(2)
    B, T, W, c = 2, 5, 8, 16
    q = torch.randn(B, T, H, c, generator=generator).to(torch.bfloat16)
    table = torch.randn(B, W - 1 + T, 2 * c, generator=generator).to(torch.bfloat16)
    sink = torch.randn(H, generator=generator)
    positions = torch.tensor([[3, 4, 5, 6, 7], [20, 21, 22, 23, 24]])
    visible = attention.window_visible(positions, W, T)
    k, v = table[..., :c], table[..., c:]
    with torch.autocast("cpu", dtype=torch.bfloat16):
        z = torch.einsum("...qhc,...kc->...hqk", q, k).float() * c ** -0.5
        z = z.masked_fill(~visible[..., None, :, :], float("-inf"))
        lse = torch.logaddexp(torch.logsumexp(z, -1), sink.float()[:, None])
        expected = torch.einsum("...hqk,...kc->...qhc", (z - lse[..., None]).exp().to(v.dtype), v)
    got = decoder.bf16_dense_attention(q, k, v, sink, visible, c ** -0.5)
    assert got.dtype == torch.bfloat16
    assert within_one_bf16_step(got, expected)


def pair(kinds):
    common = dict(kinds=kinds, window=8, rope_dims=8, top_k=4)
    return (decoder.Decoder(weights(), LAYERS, H, C, autocast=True, **common),
            decoder.Decoder(weights(), LAYERS, H, C, **common))


@pytest.mark.parametrize("kinds", KINDS, ids=IDS)
def test_the_autocast_decoder_is_the_fp32_decoder_within_bf16_rounding(kinds):
    low, full = pair(kinds)
    ids = torch.randint(V, (2, 60), generator=torch.Generator().manual_seed(3))
    rows = low.new_cache(2)
    scores, hidden = low.extend(ids, rows)
    expected = full.forward(ids)
    gap = float((scores - expected).abs().max() / expected.abs().max())
    assert scores.dtype == torch.float32 and hidden.dtype == torch.bfloat16
    assert 1e-4 < gap < 5e-2


@pytest.mark.parametrize("kinds", KINDS, ids=IDS)
def test_autocast_reading_in_pieces_gives_the_whole_text_s_scores(kinds):
    low, _ = pair(kinds)
    ids = torch.randint(V, (2, sum(PIECES)), generator=torch.Generator().manual_seed(4))
    whole = low.forward(ids)
    rows, got, start = low.new_cache(2), [], 0
    for size in PIECES:
        got.append(low.extend(ids[:, start:start + size], rows)[0])
        start += size
    assert float((torch.cat(got, 1) - whole).abs().max() / whole.abs().max()) < 2e-2
