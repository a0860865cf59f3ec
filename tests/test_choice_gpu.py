"""The HIP choice of rows of exact attention (top_k > 0) against the oracle, on
the GPU through the C ABI.  The criterion is the reference's own kernel test
(test_kernels.py:156-187): each query chooses as many rows as the oracle, and
every row the kernel chose scores within 1e-2 (in log) of the oracle's
top_k-th, since bf16 scores of two implementations may order near ties
another way; in FP32 the chosen sets are equal."""

import pytest
import torch

from oracle import attention as oracle
from tests.formulas import choice_scores, inputs, relative_error
from wpt_amd import kernels

pytestmark = pytest.mark.gpu


def check_choice(rows, expected_rows, score, tolerance):
    """rows, expected_rows (B, T, K) int64 on the CPU; score (B, T, N) the
    FP64 candidates' scores."""
    assert rows.shape == expected_rows.shape
    assert ((rows >= 0).sum(-1) == (expected_rows >= 0).sum(-1)).all()
    # every row named once, -1 only after the rows
    for query in rows.reshape(-1, rows.shape[-1]):
        named = query[query >= 0]
        assert len(set(named.tolist())) == len(named)
        assert (query[len(named):] == -1).all()
    kth = score.gather(-1, expected_rows.clamp(min=0)).masked_fill(expected_rows < 0, float("inf")).amin(-1)
    picked = score.gather(-1, rows.clamp(min=0)).masked_fill(rows < 0, float("inf"))
    assert (picked >= kth[..., None] - tolerance).all()
    assert torch.isfinite(score.gather(-1, rows.clamp(min=0))[rows >= 0]).all()  # candidates only


# (heads, head width, tokens, top k, window): the reference's kernel-test
# shapes (test_kernels.py:139-140), a pass of T queries over a table of T rows
SHAPES = [(2, 128, 700, 64, 128), (4, 128, 300, 16, 32), (12, 128, 300, 16, 32), (8, 128, 700, 64, 128),
          (8, 128, 2000, 1024, 128)]


@pytest.mark.parametrize("heads, width, T, top_k, window", SHAPES)
def test_the_choice_of_bf16_queries_matches_the_oracle(device, heads, width, T, top_k, window):
    q, k, v, _, positions = inputs(B=2, T=T, H=heads, c=width, dtype=torch.bfloat16)
    expected, expected_rows = oracle.exact_attention(q, k, v, positions, width ** -0.5, top_k, window)
    out, rows = kernels.exact_attention(*[x.to(device) for x in (q, k, v, positions)], width ** -0.5, top_k, window)
    assert out.dtype == torch.bfloat16 and relative_error(out.cpu(), expected) < 1e-2
    check_choice(rows.cpu(), expected_rows, choice_scores(q, k, positions, width ** -0.5, window), 1e-2)


def test_the_verify_step_choice_of_a_wpt_exact_layer(device):
    # the exact layer of a WPT model at the verify step: 32 rows of 4096
    # tokens, k + 1 = 5 queries of 16 heads, TOP_K 1024 outside a WINDOW of
    # 128 (attention.py:53-54), keys and values the halves of one table
    B, T, H, c, N, top_k, window = 32, 5, 16, 128, 4096, 1024, 128
    q, _, _, _, positions = inputs(B=B, T=T, H=H, c=c, N=N, dtype=torch.bfloat16)
    table = torch.randn(B, N, 2 * c, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    k, v = table[..., :c], table[..., c:]
    expected, expected_rows = oracle.exact_attention(q, k, v, positions, c ** -0.5, top_k, window)
    td = table.to(device)
    out, rows = kernels.exact_attention(q.to(device), td[..., :c], td[..., c:], positions.to(device), c ** -0.5,
                                        top_k, window)
    assert relative_error(out.cpu(), expected) < 1e-2
    check_choice(rows.cpu(), expected_rows, choice_scores(q, k, positions, c ** -0.5, window), 1e-2)


@pytest.mark.parametrize("B, T, H, c, N, top_k, window", [
    (2, 30, 3, 16, 50, 5, 8),      # the reference's formula test (test_kernels.py:70-79)
    (2, 12, 3, 16, 12, 100, 4),    # fewer candidates than top_k: all of them (test_kernels.py:82-88)
    (1, 5, 4, 64, 300, 40, 16),    # the plumbing decoder's head layout, a verify pass
    (3, 6, 16, 128, 500, 64, 0),   # no window: every row up to the query is a candidate
])
def test_the_fp32_choice_equals_the_oracle(device, B, T, H, c, N, top_k, window):
    q, k, v, _, positions = inputs(B=B, T=T, H=H, c=c, N=N, seed=3)
    expected, expected_rows = oracle.exact_attention(q, k, v, positions, 0.3, top_k, window)
    out, rows = kernels.exact_attention(*[x.to(device) for x in (q, k, v, positions)], 0.3, top_k, window)
    assert (out.cpu() - expected).abs().max() < 1e-5
    rows = rows.cpu()
    assert rows.shape == expected_rows.shape
    assert [[set(r[r >= 0].tolist()) for r in query] for query in rows] == \
        [[set(r[r >= 0].tolist()) for r in query] for query in expected_rows]


def test_padding_queries_choose_among_the_table_rows(device):
    # a generation pass at different places per row, the last row's later
    # queries past the table (test_triton_kernels.py:58-66)
    B, T, H, c, N = 3, 4, 4, 128, 400
    q, k, v, _, _ = inputs(B=B, T=T, H=H, c=c, N=N, seed=4, dtype=torch.bfloat16)
    positions = torch.tensor([[396, 397, 398, 399], [100, 101, 102, 103], [398, 399, 400, 401]])
    expected, expected_rows = oracle.exact_attention(q, k, v, positions, c ** -0.5, 32, 16)
    out, rows = kernels.exact_attention(*[x.to(device) for x in (q, k, v, positions)], c ** -0.5, 32, 16)
    assert relative_error(out.cpu(), expected) < 1e-2
    # a query past the table sees every row and has the candidates up to its
    # own position - window
    check_choice(rows.cpu(), expected_rows, choice_scores(q, k, positions, c ** -0.5, 16), 1e-2)


def test_ties_keep_the_lowest_rows(device):
    # zero keys give every row but one the same score; row 7 scores above
    # them (positive queries against a positive key): the rows above the
    # K-th score come first, then the equal ones from the lowest row up
    B, T, H, c, N, top_k, window = 1, 2, 2, 64, 256, 10, 4
    q, _, v, _, positions = inputs(B=B, T=T, H=H, c=c, N=N, seed=6, dtype=torch.bfloat16)
    q = q.abs()
    k = torch.zeros(B, N, c, dtype=torch.bfloat16)
    k[0, 7] = 1.0
    _, rows = kernels.exact_attention(*[x.to(device) for x in (q, k, v, positions)], c ** -0.5, top_k, window)
    expected_rows = oracle.exact_attention(q, k, v, positions, c ** -0.5, top_k, window)[1]
    check_choice(rows.cpu(), expected_rows, choice_scores(q, k, positions, c ** -0.5, window), 1e-6)
    assert rows.cpu().tolist() == [[[7, 0, 1, 2, 3, 4, 5, 6, 8, 9]] * T]


def test_a_bad_lse_is_a_value_error(device):
    q, k, _, _, positions = inputs(B=1, T=4, H=2, c=64, N=100, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        kernels.choose_rows(q.to(device), k.to(device), positions.to(device), torch.zeros(1, 4, 3, device=device),
                            0.1, 10, 4)
