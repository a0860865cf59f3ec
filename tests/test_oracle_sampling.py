"""Pins the oracle's sampling (CPU): the distribution's closed forms and tie
rule, the exponential-race identity of torch's multinomial, the acceptance
rule's invariants (the reference's own statistical and self-drafting tests,
packages/wpt-inference/tests/test_sampling.py:98-137), a lazy run replayed
through a tape, greedy chains and trees by brute force, and the cut."""

import math

import pytest
import torch

from oracle import sampling


def test_probabilities_without_a_cut_are_the_softmax_of_scores_over_temperature():
    scores = torch.tensor([[1.0, 2.0, 3.0, -1.0]])
    p = sampling.probabilities(scores, 0.5, None)
    expected = torch.exp(scores / 0.5) / torch.exp(scores / 0.5).sum()
    assert torch.allclose(p, expected, atol=1e-7)


def test_top_k_keeps_every_score_tied_with_the_kth():
    # ties with the k-th largest stay (scores < v[-1] are masked, not <=)
    scores = torch.tensor([[5.0, 3.0, 3.0, 3.0, 1.0, 0.0]])
    p = sampling.probabilities(scores, 1.0, 2)
    assert (p[0, :4] > 0).all() and (p[0, 4:] == 0).all()
    kept = torch.exp(scores[0, :4])
    assert torch.allclose(p[0, :4], kept / kept.sum(), atol=1e-7)


def test_top_k_one_is_one_hot_at_a_unique_maximum_and_uniform_over_tied_maxima():
    assert sampling.probabilities(torch.tensor([[0.1, 0.9, 0.3]]), 0.8, 1).tolist() == [[0.0, 1.0, 0.0]]
    p = sampling.probabilities(torch.tensor([[0.9, 0.1, 0.9]]), 0.8, 1)
    assert p.tolist() == [[0.5, 0.0, 0.5]]


@pytest.mark.parametrize("V", [50, 8192, 32768])
def test_multinomial_of_one_is_the_exponential_race(V):
    # torch.multinomial(w, 1) draws argmax(w / E), E ~ Exp(1) from the same
    # generator, and leaves the generator where the exponentials left it
    for seed in range(20):
        w = torch.rand(V, generator=torch.Generator().manual_seed(1000 + seed)) ** 4
        a, b = torch.Generator().manual_seed(seed), torch.Generator().manual_seed(seed)
        drawn = int(torch.multinomial(w / w.sum(), 1, generator=a))
        e = torch.empty(V).exponential_(generator=b)
        assert drawn == sampling.multinomial_by_exponential(w / w.sum(), e)
        assert torch.equal(a.get_state(), b.get_state())


def test_scalar_uniforms_are_the_uniform_stream():
    a, b = torch.Generator().manual_seed(3), torch.Generator().manual_seed(3)
    assert [float(torch.rand((), generator=a)) for _ in range(4)] == torch.rand(4, generator=b).tolist()


def model_and_drafts(B, L, V, seed, temperature=1.0, top_k=None, uniform_drafts=True):
    generator = torch.Generator().manual_seed(seed)
    scores = torch.randn(B, L + 1, V, generator=generator) * 2
    if uniform_drafts:
        q = torch.full((B, L, V), 1.0 / V)
        drafts = torch.randint(V, (B, L), generator=generator)
    else:
        q = torch.softmax(torch.randn(B, L, V, generator=generator), -1)
        drafts = torch.multinomial(q.reshape(-1, V), 1, generator=generator).reshape(B, L)
    return scores, q, drafts


def test_uniform_drafts_keep_the_model_s_distribution():
    # the reference's test_sampling.py:98-121: 4000 rows drafting uniformly;
    # the first written token follows the model's own probabilities
    V, rows = 20, 4000
    scores = torch.randn(1, 5, V, generator=torch.Generator().manual_seed(0))
    p = sampling.probabilities(scores[0], 1.0, None)
    generator = torch.Generator().manual_seed(1)
    firsts = []
    for _ in range(rows):
        drafts = torch.randint(V, (4,), generator=generator)
        q = torch.full((4, V), 1.0 / V)
        firsts.append(sampling.accept_row(p, q, drafts, 4, sampling.LazyDraws(generator))[0])
    counts = torch.bincount(torch.tensor(firsts), minlength=V)
    assert (counts / rows - p[0]).abs().sum() / 2 < 0.05


def test_drafts_drawn_from_the_model_itself_are_all_kept():
    # q = p: u q < p for every u < 1 (test_sampling.py:124-137)
    V, L = 30, 4
    scores = torch.randn(L + 1, V, generator=torch.Generator().manual_seed(2))
    p = sampling.probabilities(scores, 0.8, 10)
    generator = torch.Generator().manual_seed(3)
    for _ in range(50):
        drafts = torch.multinomial(p[:L], 1, generator=generator)[:, 0]
        tokens = sampling.accept_row(p, p[:L], drafts, L, sampling.LazyDraws(generator))
        assert tokens[:L] == drafts.tolist() and len(tokens) == L + 1


def test_a_draft_the_model_never_writes_is_always_replaced_from_the_residual():
    V = 8
    p = torch.zeros(2, V)
    p[:, 0], p[:, 1] = 0.75, 0.25
    q = torch.full((1, V), 1.0 / V)
    for seed in range(20):
        tokens = sampling.accept_row(p, q, torch.tensor([5]), 1, sampling.LazyDraws(torch.Generator().manual_seed(seed)))
        # max(0, p - q) is zero but at tokens 0 and 1
        assert len(tokens) == 1 and tokens[0] in (0, 1)


def test_a_lazy_run_replayed_through_its_tape_writes_the_same_tokens():
    B, L, V = 16, 4, 64
    scores, q, drafts = model_and_drafts(B, L, V, seed=5, uniform_drafts=False)
    lengths = [L] * B
    generator = torch.Generator().manual_seed(9)
    lazy = [sampling.LazyDraws(generator) for _ in range(B)]
    written = [sampling.accept(scores[b:b + 1], q[b:b + 1], drafts[b:b + 1], lengths[b:b + 1], 0.8, None,
                               [lazy[b]])[0] for b in range(B)]
    for b in range(B):
        u = torch.zeros(L)
        u[:len(lazy[b].uniforms)] = torch.tensor(lazy[b].uniforms)
        tape = sampling.TapeDraws(u, lazy[b].exponentials[0])
        assert sampling.accept(scores[b:b + 1], q[b:b + 1], drafts[b:b + 1], lengths[b:b + 1], 0.8, None,
                               [tape])[0] == written[b]


def test_greedy_verification_is_top_k_one_sampling_at_unique_maxima():
    B, L, V = 32, 4, 50
    scores, _, _ = model_and_drafts(B, L, V, seed=7)
    best = scores.argmax(-1)
    generator = torch.Generator().manual_seed(8)
    # drafts that follow the argmax for a random number of positions
    drafts = torch.randint(V, (B, L), generator=generator)
    keep = torch.randint(0, L + 1, (B,), generator=generator)
    for b in range(B):
        drafts[b, :keep[b]] = best[b, :keep[b]]
    q = torch.full((B, L, V), 1.0 / V)
    tape = [sampling.TapeDraws(torch.rand(L, generator=generator), torch.empty(V).exponential_(generator=generator))
            for _ in range(B)]
    greedy = sampling.greedy_chain(scores, drafts, [L] * B)
    sampled = sampling.accept(scores, q, drafts, [L] * B, 0.8, 1, tape)
    assert greedy == sampled
    matches = [next((j for j in range(L) if drafts[b, j] != best[b, j]), L) for b in range(B)]
    assert [len(t) - 1 for t in greedy] == matches
    assert all(t[-1] == int(best[b, n]) for b, (t, n) in enumerate(zip(greedy, matches)))


def test_greedy_tree_follows_the_argmax_down_the_tree():
    # brute force, with distinct tokens among siblings: the root-to-node
    # paths whose every step takes the child carrying its parent's argmax
    # form one chain; the accepted path is its deepest end
    parents = [-1, 0, 0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5, 6, 6]
    M, V = len(parents), 4
    generator = torch.Generator().manual_seed(11)
    for _ in range(30):
        scores = torch.randn(1, M, V, generator=generator)
        tokens = torch.randint(V, (1, M), generator=generator)
        for child in range(2, M, 2):  # siblings (child - 1, child) carry distinct tokens
            if tokens[0, child] == tokens[0, child - 1]:
                tokens[0, child] = (tokens[0, child] + 1) % V
        best = scores.argmax(-1)[0]
        (path, written), = sampling.greedy_tree(scores, tokens, parents)
        paths = []
        for node in range(M):
            chain = [node]
            while parents[chain[-1]] >= 0:
                chain.append(parents[chain[-1]])
            chain.reverse()
            if all(int(tokens[0, c]) == int(best[parents[c]]) for c in chain[1:]):
                paths.append(chain)
        assert path == max(paths, key=len)
        assert written == [int(tokens[0, c]) for c in path[1:]] + [int(best[path[-1]])]


def test_greedy_tree_takes_the_lowest_of_equal_children():
    parents = [-1, 0, 0, 1, 2]
    scores = torch.zeros(1, 5, 3)
    scores[0, :, 2] = 1.0  # every node's argmax is token 2
    tokens = torch.tensor([[0, 2, 2, 0, 2]])  # nodes 1 and 2 both carry it; only node 2 continues
    (path, written), = sampling.greedy_tree(scores, tokens, parents)
    assert path == [0, 1] and written == [2, 2]


def test_cut_stops_after_the_first_stop_and_at_the_limit():
    assert sampling.cut([1, 2, 3, 4], {3}, 10) == [1, 2, 3]
    assert sampling.cut([1, 2, 3, 4], set(), 2) == [1, 2]
    assert sampling.cut([5, 3, 3], {3}, 1) == [5]


def test_the_scheduler_s_known_answers():
    # the reference's own known answers (test_sampling.py:230-238): passes
    # cost the same up to 3 tokens per row, then 20 % more
    costs = [1.0, 1.0, 1.0, 1.2, 1.2, 1.2]
    assert sampling.schedule([[0.9, 0.9, 0.9, 0.1, 0.1], [0.5, 0.5, 0.5, 0.5, 0.5]], [5, 1], costs) == [2, 1]
    assert sampling.schedule([[0.99] * 5, [0.99] * 5], [5, 5], costs) == [5, 5]
    assert sampling.schedule([[0.9] * 5], [0], costs) == [0]


def test_the_scheduler_stops_at_the_first_width_that_does_not_pay():
    # brute force over the widths: the admitted width is the longest prefix
    # of widths along which the expected tokens per second rise at every
    # step, never a later better one (the early stop); flat costs admit
    # every draft; caps bound every row
    import random

    rng = random.Random(5)
    for _ in range(300):
        rows, draft = rng.randint(1, 4), rng.randint(0, 5)
        caps = [rng.randint(0, draft) for _ in range(rows)]
        conf = [[rng.random() for _ in range(draft)] for _ in range(rows)]
        costs = sorted(rng.uniform(0.5, 2.0) for _ in range(draft + 1))
        rates = []
        for width in range(max(caps, default=0) + 1):
            tokens = rows + sum(math.prod(conf[r][:j + 1]) for r in range(rows) for j in range(min(width, caps[r])))
            rates.append(tokens / costs[width])
        width = 0
        while width + 1 < len(rates) and rates[width + 1] > rates[width]:
            width += 1
        assert sampling.schedule(conf, caps, costs) == [min(width, cap) for cap in caps]
        assert sampling.schedule(conf, caps, [1.0] * (draft + 1)) == caps or any(
            c == 0.0 for row in conf for c in row)
