"""Pins the oracle's attention (CPU): against brute-force formulas, a closed
form, causality and padding queries past the table."""

import math

import pytest
import torch

from oracle import attention as oracle
from tests.formulas import choice_by_formula, exact_by_formula, inputs, sparse_by_formula, tree_by_formula


def test_exact_attention_follows_the_formula_across_block_joins(monkeypatch):
    # small blocks of queries so that the joins are exercised, as the
    # reference's own test does (test_kernels.py:70-79)
    monkeypatch.setattr(oracle, "BLOCK_VALUES", 4 * 3 * 50)
    q, k, v, _, positions = inputs(T=30, N=50)
    out, chosen = oracle.exact_attention(q, k, v, positions, 0.3, 0, 8)
    assert chosen.shape == (2, 30, 0)
    assert torch.allclose(out.double(), exact_by_formula(q, k, v, positions, 0.3), atol=1e-5)


def test_the_choice_picks_the_rows_of_largest_weight_outside_the_window():
    # the reference's choice rule (pytorch_kernels.py:112-117): a query with
    # fewer far rows than top_k chooses them all (test_kernels.py:86-93)
    q, k, v, _, positions = inputs(T=12)
    _, chosen = oracle.exact_attention(q, k, v, positions, 0.25, 100, 4)
    assert chosen.shape == (2, 12, 8)
    for t in range(12):
        assert set(chosen[0, t][chosen[0, t] >= 0].tolist()) == set(range(max(0, t - 3)))


@pytest.mark.parametrize("top_k, window", [(5, 8), (1, 3), (20, 1), (3, 0)])
def test_the_choice_is_the_top_k_by_the_largest_weight_over_the_heads(monkeypatch, top_k, window):
    # the reference's formula test of the choice (test_kernels.py:70-79): the
    # chosen sets equal the brute-force top_k of max-over-heads weights, in
    # blocks of a few queries
    monkeypatch.setattr(oracle, "BLOCK_VALUES", 4 * 3 * 50)
    q, k, v, _, positions = inputs(T=30, N=50)
    _, chosen = oracle.exact_attention(q, k, v, positions, 0.3, top_k, window)
    assert chosen.shape == (2, 30, oracle.chosen_columns(top_k, window, 50))
    expected = choice_by_formula(q, k, positions, 0.3, top_k, window)
    assert [[set(row[row >= 0].tolist()) for row in query] for query in chosen] == expected


def test_padding_queries_past_the_table_read_up_to_its_last_row():
    # the generation pass of the reference's test_triton_kernels.py:51-66:
    # rows at different places, the last one's later queries past the table
    generator = torch.Generator().manual_seed(0)
    B, T, H, c, N = 3, 4, 4, 32, 400
    q = torch.randn(B, T, H, c, generator=generator)
    entries = torch.randn(B, N, 2 * c, generator=generator)
    k, v = entries[..., :c], entries[..., c:]
    positions = torch.tensor([[396, 397, 398, 399], [100, 101, 102, 103], [398, 399, 400, 401]])
    out, _ = oracle.exact_attention(q, k, v, positions, c ** -0.5, 0, 16)
    assert torch.allclose(out.double(), exact_by_formula(q, k, v, positions, c ** -0.5), atol=1e-5)
    # a padding query reads what a query at the table's last row reads
    last, _ = oracle.exact_attention(q[2:, 2:3], k[2:], v[2:], torch.tensor([[N - 1]]), c ** -0.5, 0, 16)
    assert torch.allclose(out[2, 2], last[0, 0])


def test_a_query_that_sees_one_row_returns_its_value():
    # closed form: softmax over a single row is 1, whatever the score
    q, k, v, _, _ = inputs(B=1, T=1, H=2, c=8, N=5)
    out, _ = oracle.exact_attention(q, k, v, torch.tensor([[0]]), 0.5, 0, 4)
    assert torch.allclose(out[0, 0], v[0, 0].expand(2, 8))


def test_later_rows_never_change_earlier_queries():
    # causality (the reference's test_model.py:30-44, for the attention)
    q, k, v, _, positions = inputs(B=1, T=10, H=2, c=8, N=30)
    out, _ = oracle.exact_attention(q, k, v, positions, 0.4, 0, 4)
    k2, v2 = k.clone(), v.clone()
    k2[:, 25:] += 3.0
    v2[:, 25:] -= 2.0
    out2, _ = oracle.exact_attention(q, k2, v2, positions, 0.4, 0, 4)
    first = 25 - (30 - 10)  # queries at positions < 25
    assert torch.equal(out[:, :first], out2[:, :first])
    assert not torch.allclose(out[:, first:], out2[:, first:])


@pytest.mark.parametrize("K", [0, 6])
def test_sparse_attention_follows_the_formula(K):
    q, k, v, sink, positions = inputs(T=30, N=50)
    generator = torch.Generator().manual_seed(2)
    window = 5
    idx = torch.stack([torch.stack([torch.randperm(int(p) - window + 1, generator=generator)[:K]
                                    if int(p) - window + 1 >= K else torch.full((K,), -1) for p in row])
                       for row in positions]) if K else torch.empty(2, 30, 0, dtype=torch.long)
    if K:
        idx[:, ::3, -2:] = -1
    out = oracle.sparse_attention(q, k, v, sink, idx, positions, 0.3, window)
    assert torch.allclose(out.double(), sparse_by_formula(q, k, v, sink, idx, positions, 0.3, window), atol=1e-5)


def test_a_minus_infinite_sink_is_no_sink():
    q, k, v, _, positions = inputs(T=6, N=20)
    none = torch.full((3,), float("-inf"))
    out = oracle.sparse_attention(q, k, v, none, torch.empty(2, 6, 0, dtype=torch.long), positions, 0.3, 20)
    exact, _ = oracle.exact_attention(q, k, v, positions, 0.3, 0, 4)
    assert torch.allclose(out, exact, atol=1e-6)


def test_tree_attention_sees_the_prefix_and_the_ancestors_only():
    parents = oracle.binary_tree_parents(15)
    assert parents[:7] == [-1, 0, 0, 1, 1, 2, 2]
    generator = torch.Generator().manual_seed(4)
    B, M, H, c, prefix = 2, 15, 2, 16, 20
    q = torch.randn(B, M, H, c, generator=generator)
    k = torch.randn(B, prefix + M, c, generator=generator)
    v = torch.randn(B, prefix + M, c, generator=generator)
    prefixes = torch.tensor([prefix, prefix])
    out = oracle.tree_attention(q, k, v, prefixes, parents, 0.3)
    assert torch.allclose(out.double(), tree_by_formula(q, k, v, prefixes, parents, 0.3), atol=1e-5)
    # the root's and a chain's view: the root sees the prefix and itself
    visible = oracle.tree_visible(parents, prefix, prefix + M)
    assert visible[0].sum() == prefix + 1 and visible[14].sum() == prefix + 4  # 14 -> 6 -> 2 -> 0


def test_the_tree_of_a_chain_is_causal_attention():
    # a tree whose every node has the one before it as parent is a chain:
    # its mask is the causal one
    parents = [-1, 0, 1, 2, 3]
    q, k, v, _, positions = inputs(B=2, T=5, H=2, c=8, N=12)
    tree = oracle.tree_attention(q, k, v, torch.tensor([7, 7]), parents, 0.3)
    exact, _ = oracle.exact_attention(q, k, v, positions, 0.3, 0, 4)
    assert torch.allclose(tree, exact, atol=1e-6)


@pytest.mark.parametrize("start, T, window", [(300, 5, 128), (3, 5, 16), (0, 7, 8), (40, 1, 8)])
def test_window_attention_is_sparse_attention_over_the_last_window_rows(start, T, window):
    # the window layer's form (a table of the carried tail, zeros before the
    # text, and the new entries) against the pinned sparse form over the
    # whole text at the same positions, with no chosen rows
    generator = torch.Generator().manual_seed(7)
    B, H, c = 2, 4, 32
    L = start + T
    q = torch.randn(B, T, H, c, generator=generator)
    full = torch.randn(B, L, 2 * c, generator=generator)
    sink = torch.randn(H, generator=generator)
    positions = (start + torch.arange(T)).expand(B, T)
    tail = torch.zeros(B, window - 1, 2 * c)
    before = full[:, max(0, start - window + 1):start]
    if before.shape[1]:
        tail[:, -before.shape[1]:] = before
    table = torch.cat([tail, full[:, start:]], 1)
    got = oracle.window_attention(q, table[..., :c], table[..., c:], sink, positions, c ** -0.5, window)
    expected = oracle.sparse_attention(q, full[..., :c], full[..., c:], sink, torch.empty(B, T, 0, dtype=torch.long),
                                       positions, c ** -0.5, window)
    assert torch.allclose(got, expected, atol=1e-5)
    assert torch.allclose(got.double(), sparse_by_formula(q, full[..., :c], full[..., c:], sink,
                                                          torch.empty(B, T, 0, dtype=torch.long), positions,
                                                          c ** -0.5, window), atol=1e-5)


def test_rotate_turns_pairs_by_the_position_over_the_frequency():
    # RoPE (attention.py:59-71) from what fixes it: position 0 is the
    # identity; the first pair of the turned dimensions turns by p radians
    # (frequency base^0 = 1) and the last by p / base^(62/64); every pair
    # keeps its length; the dimensions before the last 64 are untouched; and
    # a query-key product depends on the positions' difference only
    generator = torch.Generator().manual_seed(8)
    x = torch.randn(1, 3, 2, 128, generator=generator)
    assert torch.equal(oracle.rotate(x, torch.zeros(3, dtype=torch.long)), x)
    unit = torch.zeros(1, 1, 128)
    unit[..., 64] = 1.0
    unit[..., 126] = 1.0
    p = torch.tensor([5])
    turned = oracle.rotate(unit, p)
    assert torch.allclose(turned[0, 0, 64:66], torch.tensor([math.cos(5.0), math.sin(5.0)]), atol=1e-6)
    angle = 5.0 / 10000 ** (62 / 64)
    assert torch.allclose(turned[0, 0, 126:128], torch.tensor([math.cos(angle), math.sin(angle)]), atol=1e-6)
    y = oracle.rotate(x, torch.tensor([7, 100, 12345]))
    assert torch.equal(y[..., :64], x[..., :64])
    pairs = lambda t: t[..., 64:].reshape(*t.shape[:-1], 32, 2).norm(dim=-1)  # noqa: E731
    assert torch.allclose(pairs(y), pairs(x), atol=1e-5)
    qv, kv = torch.randn(2, 1, 1, 128, generator=generator)
    dots = [float((oracle.rotate(qv, torch.tensor([a])) * oracle.rotate(kv, torch.tensor([b]))).sum())
            for a, b in ((10, 3), (57, 50), (1007, 1000))]
    assert max(dots) - min(dots) < 1e-3
