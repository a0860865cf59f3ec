"""The verify step at the sizes its workloads are measured on, against the
oracle on the CPU.

* The 24-layer bf16 decoder (d_model 2048, 16 query heads and one key/value
  head of 128, SwiGLU 5632, vocab 32768, weights ~ N(0, 0.02) from seed 0) at
  batch 32 with 4096 rows of cache (the headline step) and at batch 64 with
  2048 (the end-to-end stochastic workload): one undoable stochastic step of
  k = 4 drafts at temperature 0.8, eagerly, then
    - layer by layer, for two rows: each of the 24 layers and the head of
      the oracle decoder, run on the residual stream the GPU fed that layer
      (the reference's features, model.py:406-436) and reading the GPU's own
      cache tables, gives the GPU's next stream within 2e-2 of its largest
      value (the bf16 tolerance; a step of one bf16 ulp at the largest value
      is 0.4-0.8e-2 of it), in the oracle's autocast mode (the reference's
      bf16 pass: bf16 products, norms and residual stream) and in FP32; the
      head's scores within 1e-2;
    - the two rows' free-running scores (each pass from its own streams):
      within 5e-2 of both oracles.  bf16 rounding grows through 24 layers:
      the FP32 oracle and the autocast oracle themselves end 3.3e-2 apart
      on this decoder (measured on the CPU), so a bound of 2e-2 would fail
      the reference's own bf16 pass;
    - every row's tokens against the oracle's acceptance rule
      (__init__.py:210-229) on the step's own logits and tape: bit for bit;
    - the two rows' tokens on the scores of the oracle's head over the
      GPU's final stream: equal, a decision that lies within 1 % of flipping
      being left out (on the free-running scores, 3e-2 apart, a top-k cut or
      a residual draw can differ outright, so those tokens are only
      reported);
    - the lengths after the undo: the lengths before plus each row's count.
* Tree verification at batch 16, 8192 prefix rows, a binary tree of 31 nodes:
  the attention against the oracle (1e-2, the reference's bf16 kernel
  tolerance), then greedy acceptance along the tree on the GPU's bf16
  lm_head logits (the build's product) against the oracle's walk, with paths planted to depths
  0-4 (the tree's five levels) and tied children.
* The captured stochastic step of the headline workload: graph replays and
  eager steps that read the replays' tapes write the same tokens, counts,
  lengths and scores."""

import pytest
import torch
from oracle import attention as oracle_attention
from oracle import cache as oracle_cache
from oracle import decoder as oracle_decoder
from oracle import sampling as oracle_sampling
from tests.formulas import relative_error
from wpt_amd import kernels, layers, sampling
from wpt_amd.decoder import LARGE, MQADecoder, random_weights
from wpt_amd.step import VerifyStep, prefill

pytestmark = pytest.mark.gpu

NEAR = 1e-5   # decisions this close (relative) on identical inputs may differ by the softmax's last bits
HEAD_NEAR = 0.01  # decisions this close on the oracle head's scores may move with the head's bf16 rounding
BF16_NEAR = 0.05  # free-running decisions this close are reported as near ties (None)


@pytest.fixture(scope="module")
def large():
    device = torch.device("cuda", 0)
    weights = random_weights(LARGE, seed=0, std=0.02, dtype=torch.bfloat16, device=device)
    model = MQADecoder(LARGE, weights, dtype=torch.bfloat16, device=device)
    cpu = {name: w.float().cpu() for name, w in weights.items()}
    del weights
    full = oracle_decoder.Decoder(cpu, LARGE.layers, LARGE.heads, LARGE.head_dim)
    low = oracle_decoder.Decoder(cpu, LARGE.layers, LARGE.heads, LARGE.head_dim, autocast=True)
    yield model, (full, low)
    del model, full, low
    torch.cuda.empty_cache()


def prepared_step(model, B, KV, k, seed, top_k=None, given_tape=False):
    """A cache of B rows holding KV - 1 random tokens each and a step whose
    pending tokens and drafts (from q = softmax(N(0, 1) logits)) are set."""
    device = model.device
    V = model.config.vocab
    generator = torch.Generator(device=device).manual_seed(seed)
    prompt = torch.randint(V, (B, KV), generator=generator, device=device)
    cache = model.new_cache(B, capacity=KV + 16 * (k + 1))
    prefill(model, cache, prompt[:, :-1], chunk=1024)
    step = VerifyStep(model, cache, k, temperature=0.8, top_k=top_k, given_tape=given_tape)
    step.feeds[:, 0] = prompt[:, -1]
    step.q.copy_(torch.softmax(torch.randn(B, k, V, generator=generator, device=device), -1))
    step.feeds[:, 1:] = torch.multinomial(step.q.reshape(-1, V), 1, generator=generator).reshape(B, k)
    return cache, step


def draw_margin(p, q, drafts, u, e, tokens):
    """How far the row's last token (a draw from the residual or from p) is
    from another: the relative gap between the two largest w / e."""
    n = len(tokens) - 1
    if n < len(drafts):
        w = (p[n] - q[n]).clamp(min=0)
        w = w / w.sum()
    else:
        w = p[n]
    top = (w / e).topk(2).values
    return float((top[0] - top[1]) / top[0])


@pytest.mark.parametrize("B, KV, top_k", [(32, 4096, None), (64, 2048, None), (64, 2048, 40)])
def test_a_step_of_the_24_layer_decoder_matches_the_oracle(large, B, KV, top_k):
    model, (full, low) = large
    k, T = 4, 0.8
    layers, D = LARGE.layers, LARGE.d_model
    cache, step = prepared_step(model, B, KV, k, seed=B + KV, top_k=top_k)
    before = cache.lengths.clone()
    feeds = step.feeds.clone()
    # the streams entering every layer, read first and undone (the step then
    # rewrites the same rows)
    read = model.extend(feeds, cache, undoable=True, features=range(layers + 1), logits=True)
    model.undo(cache, torch.zeros(B, dtype=torch.long, device=model.device))
    tokens, counts = step.run()
    torch.cuda.synchronize()
    assert torch.equal(step.scores, read[0])  # reading the features changed nothing
    logits = step.scores.float().cpu()  # the bf16 logits' exact values, as the sampler read them
    u, e, q = step.u.cpu(), step.e.cpu(), step.q.cpu()
    drafts = feeds[:, 1:].cpu()
    got = sampling.written(tokens, counts)
    step.check()
    assert cache.lengths.cpu().tolist() == (before.cpu() + counts.cpu().long()).tolist()

    # every row, on the step's own logits and tape
    lengths = [k] * B
    expected = oracle_sampling.accept(logits, q, drafts, lengths, T, top_k,
                                      [oracle_sampling.TapeDraws(u[b], e[b]) for b in range(B)])
    gaps = oracle_sampling.margins(logits, q, drafts, lengths, T, top_k, u)
    near = [b for b in range(B) if gaps[b] < NEAR]
    assert all(got[b] == expected[b] for b in range(B) if b not in near)
    assert len(near) == 0
    kept = [len(t) - 1 for t in got]
    assert min(kept) < k  # rows reject
    print(f"B={B} KV={KV} top_k={top_k}: {sum(len(t) for t in got)} tokens written, kept drafts per row {kept}")

    # two rows through the oracle decoder, reading the GPU's cache tables
    rows = [0, B - 1]
    L = int(before[rows].max())
    tables = [t[rows, :L].cpu() for t in cache.tables]
    streams = read[2][rows].cpu().split(D, -1)

    def state(ora):
        rows_ = oracle_cache.Rows(len(rows))
        rows_.lengths = before[rows].cpu()
        rows_.values = {("entries", i): t if ora.autocast else t.float() for i, t in enumerate(tables)}
        return rows_

    def decide(scores, margin):
        """The two rows' tokens on `scores`, None where a decision is within `margin` of flipping."""
        mine = oracle_sampling.accept(scores, q[rows], drafts[rows], [k] * len(rows), T, top_k,
                                      [oracle_sampling.TapeDraws(u[b], e[b]) for b in rows])
        own = oracle_sampling.margins(scores, q[rows], drafts[rows], [k] * len(rows), T, top_k, u[rows])
        out = []
        for i, b in enumerate(rows):
            p = oracle_sampling.probabilities(scores[i], T, top_k)
            out.append(None if min(own[i], draw_margin(p, q[b], drafts[b], u[b], e[b], mine[i])) < margin
                       else mine[i])
        return out

    for ora in (low, full):  # layer by layer, on the GPU's own streams
        outputs, head = ora.forced(streams, state(ora))
        errors = [relative_error(streams[i + 1], outputs[i].float()) for i in range(layers)]
        print(f"{'autocast' if ora.autocast else 'fp32'} oracle, layer by layer: "
              + " ".join(f"{x:.1e}" for x in errors) + f"; head {relative_error(logits[rows], head):.2e}")
        assert max(errors) < 2e-2 and relative_error(logits[rows], head) < 1e-2
        if ora.autocast:
            for i, b in enumerate(rows):
                mine = decide(head, HEAD_NEAR)[i]
                assert mine is None or mine == got[b], f"row {b}: the oracle's head writes {mine}, the GPU {got[b]}"

    free16 = low.extend(feeds[rows].cpu(), state(low), undoable=True)[0]
    free32 = full.extend(feeds[rows].cpu(), state(full), undoable=True)[0]
    error16, error32 = relative_error(logits[rows], free16), relative_error(logits[rows], free32)
    print(f"free-running scores: against the autocast oracle {error16:.2e}, against the FP32 oracle {error32:.2e}")
    assert error16 < 5e-2 and error32 < 5e-2
    free = decide(free16, BF16_NEAR)
    print("free-running tokens: " + "; ".join(f"row {b} oracle {free[i]} GPU {got[b]}" for i, b in enumerate(rows)))


def plant_paths(best, parents, B):
    """Node tokens whose greedy walk goes to depth b % 5 in row b (each step
    to the child whose token is its parent's argmax), other nodes random;
    rows 3 and 9 give both children of the root the root's argmax (the
    lower index wins)."""
    M = len(parents)
    children = [[] for _ in range(M)]
    for i, parent in enumerate(parents):
        if parent >= 0:
            children[parent].append(i)
    generator = torch.Generator().manual_seed(11)
    tokens = torch.randint(best.shape[-1], (B, M), generator=generator)
    for b in range(B):
        node = 0
        for depth in range(b % 5):
            if not children[node]:
                break
            child = children[node][(b + depth) % 2]
            tokens[b, child] = best[b, node]
            other = [c for c in children[node] if c != child][0]
            if tokens[b, other] == best[b, node]:
                tokens[b, other] = (best[b, node] + 1) % best.shape[-1]
            node = child
        if b in (3, 9):
            tokens[b, children[0]] = best[b, 0]
    return tokens


def test_tree_verification_at_its_workload_size(device):
    # batch 16, 8192 prefix rows, a binary draft tree of 31 nodes (depth 5)
    # after them, the ancestor-only mask; the lm_head [2048 x 32768] over
    # N(0, 0.02) weights; per-path greedy acceptance
    B, M, H, c, prefix, V = 16, 31, 16, 128, 8192, 32768
    parents = oracle_attention.binary_tree_parents(M)
    generator = torch.Generator().manual_seed(14)
    q = torch.randn(B, M, H, c, generator=generator).to(torch.bfloat16)
    table = torch.randn(B, prefix + M, 2 * c, generator=generator).to(torch.bfloat16)
    head = (torch.randn(V, H * c, generator=generator) * 0.02).to(torch.bfloat16)
    prefixes = torch.full((B,), prefix)
    expected = oracle_attention.tree_attention(q, table[..., :c], table[..., c:], prefixes, parents, c ** -0.5)
    td = table.to(device)
    o = kernels.tree_attention(q.to(device), td[..., :c], td[..., c:], prefixes.to(device), parents, c ** -0.5)
    assert relative_error(o.cpu(), expected) < 1e-2
    # the benchmark's path: the attention output as the lm_head's fm operand
    # (the same bits), the head on the wide tiles, bf16 logits read by the walk
    o_fm = kernels.tree_attention(q.to(device), td[..., :c], td[..., c:], prefixes.to(device), parents, c ** -0.5,
                                  out_fm=True)
    assert torch.equal(layers.fm_unpack(o_fm, B * M, H * c), o.reshape(B * M, H * c))
    head_d = head.to(device)
    logits = layers.linear_fm_wide(o_fm, B * M, layers.FmWeight(head_d)).view(B, M, V)
    expected_logits = o.reshape(B * M, H * c).float().cpu() @ head.float().T
    assert relative_error(logits.reshape(B * M, V).float().cpu(), expected_logits) < 1e-2
    best = oracle_sampling.first_argmax(logits.float().cpu())
    node_tokens = plant_paths(best, parents, B)
    # the benchmark's walk: each node's argmax from the head's epilogue, no logits stored
    fused = layers.head_argmax_fm_wide(o_fm, B * M, layers.FmWeight(head_d)).view(B, M)
    assert torch.equal(fused.long().cpu(), best)
    path, tokens, counts = sampling.greedy_tree_from_argmax(fused, node_tokens.to(device), parents)
    walks = oracle_sampling.greedy_tree(logits.float().cpu(), node_tokens, parents)
    counts = counts.cpu().tolist()
    for b, (want_path, want_tokens) in enumerate(walks):
        n = counts[b]
        assert path[b, :n].cpu().tolist() == want_path and tokens[b, :n].cpu().tolist() == want_tokens
    assert sorted({len(p) - 1 for p, _ in walks}) == [0, 1, 2, 3, 4]  # every depth of the tree is reached
    assert walks[3][0][1] == 1 and walks[9][0][1] == 1  # tied children: the lower index


def test_a_captured_stochastic_step_replays_as_eager_steps_on_its_tapes(large):
    # the headline workload's step (batch 32, 4096 rows, k = 4, T = 0.8)
    # captured in a HIP graph, which draws its tape inside; eager steps on a
    # copy of the cache read each replay's tape
    model, _ = large
    B, KV, k = 32, 4096, 4
    cache, step = prepared_step(model, B, KV, k, seed=5)
    twin = cache.select(list(range(B)))
    eager = VerifyStep(model, twin, k, temperature=0.8, top_k=None, given_tape=True)
    eager.feeds.copy_(step.feeds)
    eager.q.copy_(step.q)

    def compare(tokens, counts, tokens_e, counts_e, i):
        torch.cuda.synchronize()
        assert torch.equal(tokens, tokens_e) and torch.equal(counts, counts_e), f"step {i}"
        assert torch.equal(cache.lengths, twin.lengths) and torch.equal(step.feeds, eager.feeds)
        assert torch.equal(step.scores, eager.scores)

    # one eager step on each first (the step drawing its tape, the twin reading it)
    tokens, counts = step.run()
    eager.u.copy_(step.u)
    eager.e.copy_(step.e)
    compare(tokens, counts, *eager.run(), "eager")
    step.capture(warmup=0)  # the capture itself runs nothing
    for i in range(4):
        tokens, counts = step.replay()
        torch.zeros(1000, device=model.device).sum()  # eager work between replays
        eager.u.copy_(step.u)
        eager.e.copy_(step.e)
        compare(tokens, counts, *eager.run(), f"replay {i}")
        step.check()
        eager.check()
    assert int(cache.lengths.min()) > KV - 1  # the steps moved on


def test_a_captured_step_drawing_in_the_reference_s_order_replays_as_eager_steps(large):
    # the headline workload's step drawing as the reference's loop does from a
    # generator on the GPU (its state on the device, moved on by each replay)
    # against eager steps on a copy of the cache from a generator seeded alike
    model, _ = large
    B, KV, k = 32, 4096, 4
    cache, step = prepared_step(model, B, KV, k, seed=9)
    mine = torch.Generator(device=model.device).manual_seed(31)
    other = torch.Generator(device=model.device).manual_seed(31)
    captured = VerifyStep(model, cache, k, temperature=0.8, in_order=True, generator=mine)
    captured.feeds.copy_(step.feeds)
    captured.q.copy_(step.q)
    twin = cache.select(list(range(B)))
    eager = VerifyStep(model, twin, k, temperature=0.8, in_order=True, generator=other)
    eager.feeds.copy_(step.feeds)
    eager.q.copy_(step.q)
    captured.capture(warmup=0)
    moved = 0
    for i in range(4):
        tokens, counts = captured.replay()
        torch.zeros(1000, device=model.device).sum()  # eager work between replays
        tokens_e, counts_e = eager.run()
        torch.cuda.synchronize()
        assert torch.equal(tokens, tokens_e) and torch.equal(counts, counts_e), f"replay {i}"
        assert torch.equal(captured.state, eager.state) and torch.equal(cache.lengths, twin.lengths)
        moved += 4 * int((counts.clamp(max=k) + 1).sum())  # each row: its judged drafts' uniforms, one multinomial
        assert int(captured.state[1]) == moved, f"replay {i}"
        captured.check()
    captured.sync_generator()
    eager.sync_generator()
    assert torch.equal(mine.get_state(), other.get_state())
