"""The HIP acceptance step against the oracle, on the GPU, through the C ABI
(wpt_amd.sampling calls libwptv.so).  Decisions are compared bit-exactly on
identical scores and tapes; a decision whose two sides u*q and p lie within
1e-5 (relative) of each other may differ by the last bits of the softmax, so
such rows are counted and left out (none occur at these seeds)."""

import pytest
import torch

from oracle import sampling as oracle
from wpt_amd import sampling

pytestmark = pytest.mark.gpu

NEAR = 1e-5


def step_inputs(B, L, V, seed, spread=4.0):
    """Peaked scores correlated with the drafts' distributions, so that rows
    keep, reject and resample at every position (also under a top-k cut)."""
    generator = torch.Generator().manual_seed(seed)
    logits = spread * torch.randn(B, L + 1, V, generator=generator)
    q = torch.softmax(logits[:, :L] + torch.randn(B, L, V, generator=generator), -1)
    drafts = torch.multinomial(q.reshape(-1, V), 1, generator=generator).reshape(B, L)
    scores = logits
    u = torch.rand(B, L, generator=generator)
    e = torch.empty(B, V).exponential_(generator=generator)
    return scores, q, drafts, u, e


def compare(got, expected, gaps):
    near = [b for b, gap in enumerate(gaps) if gap < NEAR]
    for b, (g, x) in enumerate(zip(got, expected)):
        if b not in near:
            assert g == x, f"row {b}: {g} != {x}"
    return near


@pytest.mark.parametrize("V, top_k, temperature", [(32768, None, 0.8), (32768, 40, 0.8), (8192, 40, 1.0),
                                                   (1000, 1, 0.8), (50, None, 1.3), (32768, 1024, 0.8),
                                                   (32768, 1500, 0.8), (2000, 1999, 1.0), (65536, 40, 0.8),
                                                   (65536, None, 1.0)])
def test_accept_matches_the_oracle_on_one_tape(device, V, top_k, temperature):
    B, L = 64, 4
    scores, q, drafts, u, e = step_inputs(B, L, V, seed=V + (top_k or 0))
    lengths = [L] * B
    expected = oracle.accept(scores, q, drafts, lengths, temperature, top_k,
                             [oracle.TapeDraws(u[b], e[b]) for b in range(B)])
    tokens, counts = sampling.accept(*(x.to(device) for x in (scores, q, drafts, u, e)), temperature, top_k)
    got = sampling.written(tokens, counts)
    near = compare(got, expected, oracle.margins(scores, q, drafts, lengths, temperature, top_k, u))
    assert not near
    kept = [len(t) - 1 for t in expected]
    assert min(kept) < L and (max(kept) > 0 or top_k == 1)  # rows keep and reject


@pytest.mark.parametrize("V", [32768, 1000])
def test_draft_rows_copied_into_lds_or_read_in_place_decide_alike(device, V):
    # contiguous q rows (16-byte aligned: the kernel copies each into LDS) and
    # the same values as a view whose rows lie V + 1 entries apart (read from
    # memory entry by entry): the same tokens, bit for bit, and the oracle's
    B, L = 32, 4
    scores, q, drafts, u, e = step_inputs(B, L, V, seed=40 + V)
    wide = torch.zeros(B, L, V + 1)
    wide[..., :V] = q
    on = [x.to(device) for x in (scores, drafts, u, e)]
    spread = wide.to(device)[..., :V]
    assert spread.stride(1) == V + 1
    for top_k in (None, 40):
        t1, c1 = sampling.accept(on[0], q.to(device), on[1], on[2], on[3], 0.8, top_k)
        t2, c2 = sampling.accept(on[0], spread, on[1], on[2], on[3], 0.8, top_k)
        assert torch.equal(t1, t2) and torch.equal(c1, c2)
        expected = oracle.accept(scores, q, drafts, [L] * B, 0.8, top_k,
                                 [oracle.TapeDraws(u[b], e[b]) for b in range(B)])
        assert sampling.written(t1, c1) == expected


@pytest.mark.parametrize("top_k", [5, 40, 1500])
def test_a_top_k_cut_through_tied_scores_keeps_every_tie(device, top_k):
    # scores on a few levels, so that the k-th largest ties with dozens to
    # thousands of entries (28 to 5420 kept per position at these seeds),
    # every one of them kept as the reference's `scores < v[..., [-1]]` keeps
    # them
    B, L, V = 32, 4, 32768
    scores, q, drafts, u, e = step_inputs(B, L, V, seed=20 + top_k)
    scores = torch.round(scores / 8)
    lengths = [L] * B
    expected = oracle.accept(scores, q, drafts, lengths, 0.8, top_k, [oracle.TapeDraws(u[b], e[b]) for b in range(B)])
    tokens, counts = sampling.accept(*(x.to(device) for x in (scores, q, drafts, u, e)), 0.8, top_k)
    near = compare(sampling.written(tokens, counts), expected, oracle.margins(scores, q, drafts, lengths, 0.8, top_k, u))
    assert not near


@pytest.mark.parametrize("top_k", [None, 40])
def test_bf16_scores_decide_as_their_fp32_values(device, top_k):
    # the lm_head's bf16 logits read directly are the reference's
    # scores.float(): every token and count equal, bit for bit
    B, L, V = 32, 4, 32768
    scores, q, drafts, u, e = step_inputs(B, L, V, seed=30)
    low = scores.to(torch.bfloat16)
    on = [x.to(device) for x in (q, drafts, u, e)]
    t16, c16 = sampling.accept(low.to(device), *on, 0.8, top_k)
    t32, c32 = sampling.accept(low.float().to(device), *on, 0.8, top_k)
    assert torch.equal(t16, t32) and torch.equal(c16, c32)
    g16 = sampling.greedy_chain(low.to(device), on[1])
    g32 = sampling.greedy_chain(low.float().to(device), on[1])
    assert all(torch.equal(a, b) for a, b in zip(g16, g32))
    parents = [-1, 0, 0, 1, 1]
    nodes = torch.cat([torch.zeros(B, 1, dtype=torch.long), drafts], 1).to(device)
    w16 = sampling.greedy_tree(low.to(device), nodes, parents)
    w32 = sampling.greedy_tree(low.float().to(device), nodes, parents)
    assert all(torch.equal(a, b) for a, b in zip(w16, w32))


def test_per_row_lengths_and_first_positions(device):
    B, L, V = 16, 4, 4096
    scores, q, drafts, u, e = step_inputs(B, L, V, seed=3)
    generator = torch.Generator().manual_seed(4)
    lengths = torch.randint(0, L + 1, (B,), generator=generator)
    firsts = torch.randint(0, 3, (B,), generator=generator)
    # scores with firsts[b] pending positions before the verified ones
    padded = torch.randn(B, L + 3, V, generator=generator)
    for b in range(B):
        padded[b, firsts[b]:firsts[b] + L + 1] = scores[b]
    expected = oracle.accept(scores, q, drafts, lengths.tolist(), 0.8, 40,
                             [oracle.TapeDraws(u[b], e[b]) for b in range(B)])
    tokens, counts = sampling.accept(*(x.to(device) for x in (padded, q, drafts, u, e)), 0.8, 40,
                                     lengths=lengths, firsts=firsts)
    assert sampling.written(tokens, counts) == expected


def test_a_lazy_run_is_replayed_through_its_tape(device):
    # the reference's lazily drawn stream (torch.rand per draft, multinomial
    # per row) recorded on the CPU and handed to the GPU as a tape
    B, L, V = 32, 4, 2048
    scores, q, drafts, _, _ = step_inputs(B, L, V, seed=6)
    generator = torch.Generator().manual_seed(7)
    lazy = [oracle.LazyDraws(generator) for _ in range(B)]
    expected = [oracle.accept(scores[b:b + 1], q[b:b + 1], drafts[b:b + 1], [L], 0.8, 40, [lazy[b]])[0]
                for b in range(B)]
    u = torch.zeros(B, L)
    for b in range(B):
        u[b, :len(lazy[b].uniforms)] = torch.tensor(lazy[b].uniforms)
    e = torch.stack([draws.exponentials[0] for draws in lazy])
    tokens, counts = sampling.accept(*(x.to(device) for x in (scores, q, drafts, u, e)), 0.8, 40)
    assert sampling.written(tokens, counts) == expected


def offset(generator):
    return int(generator.get_state().view(torch.int64)[1])


def race_gap(w, e):
    """The relative gap between the two largest w / e (how far a
    multinomial draw is from another outcome)."""
    top = torch.topk((w.double() / e.double()).reshape(-1), 2).values
    return float((top[0] - top[1]) / top[0])


@pytest.mark.parametrize("V, top_k, temperature, dtype", [(32768, None, 0.8, torch.float32),
                                                          (32768, 40, 0.8, torch.bfloat16),
                                                          (4096, 1024, 1.0, torch.float32),
                                                          (50, None, 1.3, torch.float32)])
def test_in_order_draws_write_the_reference_loop_s_tokens_from_a_gpu_generator(device, V, top_k, temperature,
                                                                               dtype):
    # the reference's loop run on the GPU with its generator there (torch.rand
    # per draft judged, then a multinomial, row after row) against the fused
    # path drawing the same stream from a generator seeded alike: the same
    # tokens, and the two generators end at the same offset
    B, L = 32, 4
    scores, q, drafts, _, _ = step_inputs(B, L, V, seed=100 + V + (top_k or 0))
    scores = scores.to(dtype).float() if dtype == torch.bfloat16 else scores
    lengths = [(b * 7) % (L + 1) for b in range(B)]  # 0 .. L drafts a row
    on = [x.to(device) for x in (scores, q, drafts)]
    reference = torch.Generator(device=device).manual_seed(11)
    lazy = [oracle.LazyDraws(reference) for _ in range(B)]
    expected = [oracle.accept(on[0][b:b + 1], on[1][b:b + 1], on[2][b:b + 1], [lengths[b]], temperature, top_k,
                              [lazy[b]])[0] for b in range(B)]
    # no decision or draw of the reference's within 1e-5 of flipping (a flip moves every later row's draws)
    u = torch.zeros(B, L)
    for b in range(B):
        u[b, :len(lazy[b].uniforms)] = torch.tensor(lazy[b].uniforms)
    assert min(oracle.margins(scores, q, drafts, lengths, temperature, top_k, u)) > NEAR
    for b in range(B):
        n = len(expected[b]) - 1
        p = oracle.probabilities(on[0][b, n], temperature, top_k)
        w = (p - on[1][b, n]).clamp(min=0) if n < lengths[b] else p
        assert race_gap(w / w.sum(), lazy[b].exponentials[0]) > NEAR
    mine = torch.Generator(device=device).manual_seed(11)
    state = sampling.generator_state(mine, device)
    given = on[0].to(dtype) if dtype == torch.bfloat16 else on[0]
    tokens, counts = sampling.accept_in_order(given, on[1], on[2], state, temperature, top_k, lengths=lengths)
    assert sampling.written(tokens, counts) == expected
    sampling.set_offset(mine, state)
    assert offset(mine) == offset(reference) == 4 * sum(min(len(t), lengths[b]) + 1 for b, t in enumerate(expected))
    # the stream goes on where the reference's does
    assert torch.equal(torch.rand(3, generator=mine, device=device), torch.rand(3, generator=reference, device=device))


@pytest.mark.parametrize("B, V, top_k", [(7, 32768, 40), (65, 32768, None)])
def test_a_joint_in_order_draw_is_the_reference_s_sample_of_every_row(device, B, V, top_k):
    # Writer._sample: one torch.multinomial over the (rows, V) distributions;
    # at 65 x 32768 entries torch's draw takes two words of some threads
    generator = torch.Generator().manual_seed(B)
    scores = (3 * torch.randn(B, 1, V, generator=generator)).to(device)
    reference = torch.Generator(device=device).manual_seed(5)
    p = oracle.probabilities(scores[:, 0], 0.9, top_k)
    state_before = reference.get_state()
    e = torch.empty_like(p).exponential_(generator=reference)
    reference.set_state(state_before)
    expected = torch.multinomial(p, 1, generator=reference)[:, 0].tolist()
    assert min(race_gap(p[b], e[b]) for b in range(B)) > NEAR
    mine = torch.Generator(device=device).manual_seed(5)
    state = sampling.generator_state(mine, device)
    tokens, counts = sampling.accept_in_order(scores, None, None, state, 0.9, top_k, joint=True)
    assert [t[0] for t in sampling.written(tokens, counts)] == expected
    sampling.set_offset(mine, state)
    assert offset(mine) == offset(reference)


def test_in_order_draws_with_the_commit_move_the_cache_as_the_tape_path_does(device):
    # the same tokens with or without the commit, and the commit's lengths,
    # feeds and counts as wptv_accept_commit's for those tokens
    B, L, V = 16, 4, 8192
    scores, q, drafts, _, _ = step_inputs(B, L, V, seed=77)
    on = [x.to(device) for x in (scores, q, drafts)]
    state = sampling.generator_state(torch.Generator(device=device).manual_seed(3), device)
    t1, c1 = sampling.accept_in_order(*on, state.clone(), 0.8, 40)
    before = torch.arange(B, dtype=torch.long, device=device) * 10
    lengths = before + L + 1
    feeds = torch.full((B, 1), -5, dtype=torch.long, device=device)
    written = torch.zeros(B, dtype=torch.long, device=device)
    failed = torch.zeros(1, dtype=torch.int32, device=device)
    t2, c2 = sampling.accept_in_order(*on, state, 0.8, 40, commit=(lengths, before, feeds, failed, written))
    assert torch.equal(t1, t2) and torch.equal(c1, c2)
    assert torch.equal(lengths, before + c2.long()) and torch.equal(written, c2.long())
    last = t2.gather(1, (c2.long() - 1)[:, None])[:, 0]
    assert torch.equal(feeds[:, 0], last) and int(failed) == 0


def test_greedy_chain_matches_the_oracle_and_top_k_one(device):
    B, L, V = 64, 4, 32768
    scores, q, drafts, u, e = step_inputs(B, L, V, seed=8)
    best = scores.argmax(-1)
    keep = torch.randint(0, L + 1, (B,), generator=torch.Generator().manual_seed(9))
    for b in range(B):
        drafts[b, :keep[b]] = best[b, :keep[b]]
    expected = oracle.greedy_chain(scores, drafts, [L] * B)
    args = [x.to(device) for x in (scores, q, drafts, u, e)]
    assert sampling.written(*sampling.greedy_chain(args[0], args[2])) == expected
    assert sampling.written(*sampling.accept(*args, 0.8, 1)) == expected


def test_uniform_drafts_keep_the_model_s_distribution(device):
    # the reference's statistical test (test_sampling.py:98-121) at 4000 rows
    # of one model distribution: the first written token follows p
    rows, L, V = 4000, 4, 20
    generator = torch.Generator().manual_seed(10)
    row_scores = torch.randn(1, L + 1, V, generator=generator)
    scores = row_scores.expand(rows, -1, -1).contiguous()
    q = torch.full((rows, L, V), 1.0 / V)
    drafts = torch.randint(V, (rows, L), generator=generator)
    u, e = torch.rand(rows, L, generator=generator), torch.empty(rows, V).exponential_(generator=generator)
    tokens, counts = sampling.accept(*(x.to(device) for x in (scores, q, drafts, u, e)), 1.0, None)
    first = tokens[:, 0].cpu()
    p = oracle.probabilities(row_scores[0, 0], 1.0, None)
    assert (torch.bincount(first, minlength=V) / rows - p).abs().sum() / 2 < 0.05


def test_drafts_from_the_model_itself_are_all_kept(device):
    B, L, V = 64, 4, 4096
    generator = torch.Generator().manual_seed(11)
    scores = torch.randn(B, L + 1, V, generator=generator)
    p = oracle.probabilities(scores, 0.8, 40)
    drafts = torch.multinomial(p[:, :L].reshape(-1, V), 1, generator=generator).reshape(B, L)
    u, e = torch.rand(B, L, generator=generator), torch.empty(B, V).exponential_(generator=generator)
    tokens, counts = sampling.accept(*(x.to(device) for x in (scores, p[:, :L].contiguous(), drafts, u, e)), 0.8, 40)
    assert (counts == L + 1).all()
    assert torch.equal(tokens[:, :L].cpu(), drafts)


def test_greedy_tree_matches_the_oracle(device):
    # the tree workload's acceptance: a binary draft tree of 31 nodes, with
    # node tokens planted on the argmax path to random depths
    B, V = 16, 32768
    parents = [-1] + [(i - 1) // 2 for i in range(1, 31)]
    generator = torch.Generator().manual_seed(12)
    scores = torch.randn(B, 31, V, generator=generator)
    best = scores.argmax(-1)
    tokens = torch.randint(V, (B, 31), generator=generator)
    for b in range(B):
        node = 0
        for _ in range(int(torch.randint(0, 5, (), generator=generator))):
            child = 2 * node + 1 + int(torch.randint(0, 2, (), generator=generator))
            tokens[b, child] = best[b, node]
            node = child
    expected = oracle.greedy_tree(scores, tokens, parents)
    path, written, counts = sampling.greedy_tree(scores.to(device), tokens.to(device), parents)
    for b, (p, w) in enumerate(expected):
        assert int(counts[b]) == len(w)
        assert path[b, :len(p)].tolist() == p and written[b, :len(w)].tolist() == w


def test_the_walk_from_given_argmaxes_is_the_walk_from_the_scores(device):
    B, V = 16, 4096
    parents = [-1] + [(i - 1) // 2 for i in range(1, 31)]
    generator = torch.Generator().manual_seed(14)
    scores = torch.randn(B, 31, V, generator=generator)
    best = scores.argmax(-1)
    tokens = torch.randint(V, (B, 31), generator=generator)
    for b in range(B):
        node = 0
        for _ in range(int(torch.randint(0, 5, (), generator=generator))):
            child = 2 * node + 1 + int(torch.randint(0, 2, (), generator=generator))
            tokens[b, child] = best[b, node]
            node = child
    want = sampling.greedy_tree(scores.to(device), tokens.to(device), parents)
    got = sampling.greedy_tree_from_argmax(best.to(torch.int32).to(device), tokens.to(device), parents)
    for a, b in zip(want, got):
        assert torch.equal(a, b)


def test_a_residual_with_no_mass_raises(device):
    V = 16
    scores = torch.zeros(1, 2, V)
    q = torch.softmax(scores[:, :1], -1)  # q equals p: the residual is zero everywhere
    drafts = torch.tensor([[3]])
    u = torch.tensor([[1.0]])  # u*q < p fails: the draft is rejected
    e = torch.ones(1, V)
    tokens, counts = sampling.accept(*(x.to(device) for x in (scores, q, drafts, u, e)), 1.0, None)
    with pytest.raises(RuntimeError, match="no mass"):
        sampling.written(tokens, counts)


def test_greedy_decisions_take_nan_as_torch_argmax_does(device):
    # torch.argmax (the reference's greedy, evaluation.py:74-81) takes a NaN
    # above every number, the first one among several: a row of NaN decides
    # index 0, a row with a NaN its first NaN, in the chain and in the tree
    B, L, V = 3, 2, 64
    generator = torch.Generator().manual_seed(13)
    scores = torch.randn(B, L + 1, V, generator=generator)
    scores[1] = float("nan")
    scores[2, 1, 40] = scores[2, 1, 9] = float("nan")
    best = scores.to(device).argmax(-1).cpu()
    assert best[1].tolist() == [0, 0, 0] and best[2, 1] == 9
    drafts = best[:, :L].clone()
    drafts[0, 1] = (drafts[0, 1] + 1) % V  # row 0 rejects its second draft
    tokens, counts = sampling.greedy_chain(scores.to(device), drafts.to(device))
    assert counts.tolist() == [2, L + 1, L + 1]
    assert sampling.written(tokens, counts) == [[best[0, 0].item(), best[0, 1].item()], best[1].tolist(),
                                                best[2].tolist()]
    parents = [-1, 0, 0]
    tree_scores = torch.randn(B, 3, V, generator=generator)
    tree_scores[2, 0] = float("nan")
    tree_scores[0, 0, 17] = float("nan")
    node_tokens = torch.tensor([[0, 5, 17], [0, 1, 2], [0, 0, 0]])
    want = sampling.greedy_tree_from_argmax(tree_scores.to(device).argmax(-1).to(torch.int32), node_tokens.to(device),
                                            parents)
    got = sampling.greedy_tree(tree_scores.to(device), node_tokens.to(device), parents)
    for a, b in zip(want, got):
        assert torch.equal(a, b)
    assert got[1][0, 0] == 17 and got[1][2, 0] == 0  # both walks go through a NaN node


def test_bad_shapes_raise_value_error(device):
    scores = torch.zeros(2, 5, 100, device=device)
    q = torch.zeros(2, 4, 100, device=device)
    with pytest.raises(ValueError):
        sampling.accept(scores, q, torch.zeros(2, 5, dtype=torch.long, device=device), torch.zeros(2, 5, device=device),
                        torch.ones(2, 100, device=device))
    with pytest.raises(ValueError):
        sampling.accept(scores, q, torch.zeros(2, 4, dtype=torch.long, device=device), torch.zeros(2, 4, device=device),
                        torch.ones(2, 100, device=device), temperature=0.0)


@pytest.mark.parametrize("greedy, top_k", [(False, None), (False, 40), (True, None)])
def test_the_fused_commit_equals_accept_undo_and_next_feeds(device, greedy, top_k):
    # wptv_accept_commit against wptv_accept, wptv_cache_lengths (undo) and
    # wptv_next_feeds in turn, on the same inputs: every output bit for bit;
    # row 0 has a residual with no mass (count -1: it keeps its pending token,
    # its cache drops the reading and the flag is raised unless greedy)
    from wpt_amd.cache import _lengths
    from wpt_amd.step import next_feeds
    B, L, V = 48, 4, 4096
    scores, q, drafts, u, e = step_inputs(B, L, V, seed=77)
    scores[0] = 0.0
    q[0] = torch.softmax(scores[0, :L], -1)
    u[0] = 1.0
    on = [x.to(device) for x in (scores, q, drafts, u, e)]
    generator = torch.Generator().manual_seed(5)
    before = torch.randint(0, 1000, (B,), generator=generator)
    lengths = before + L + 1
    lengths[1] = before[1] + 2  # a row that read fewer tokens than it may keep
    feeds = torch.randint(0, V, (B, L + 1), generator=generator)
    written = torch.randint(0, 50, (B,), generator=generator)
    state = [x.to(device) for x in (lengths, before, feeds, written)] + [torch.zeros(1, dtype=torch.int32,
                                                                                    device=device)]
    fused = [x.clone() for x in state]
    t1, c1 = sampling.accept(*on, 0.8, top_k, greedy=greedy)
    _lengths(state[0], state[1], c1, undo=True)
    next_feeds(t1, c1, state[2], state[4], state[3])
    t2, c2 = sampling.accept(*on, 0.8, top_k, greedy=greedy,
                             commit=(fused[0], fused[1], fused[2], fused[4], fused[3]))
    assert torch.equal(t1, t2) and torch.equal(c1, c2)
    for a, b in zip(state, fused):
        assert torch.equal(a, b)
    if not greedy:
        assert int(c2[0]) == -1 and int(fused[4]) == 1
        assert int(fused[0][0]) == int(before[0]) and torch.equal(fused[2][0].cpu(), feeds[0])
    assert int(fused[0][1]) <= int(before[1]) + 2
