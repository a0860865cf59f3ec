"""Oracle sampling: the reference's sampling distribution and the acceptance /
rejection rule of its speculative-decoding step, restated on the CPU in FP32
(test infrastructure; see oracle/__init__.py).

    probabilities      Writer._probabilities
                       (packages/wpt-inference/src/wpt_inference/__init__.py:173-179)
    accept_row         the per-row loop of Writer._speculate (:210-222): draft j
                       is kept iff u * q[j, token] < p[j, token]; the first
                       rejected one is replaced by a draw from max(0, p - q),
                       normalized; when every draft is kept one more token is
                       drawn from p at the position after the last draft
    LazyDraws          the reference's draws from a torch generator, in its
                       order: torch.rand(()) per draft considered (:214), then
                       torch.multinomial(w, 1) (:219, :222); on the
                       generator's device (a GPU generator with scores, q and
                       drafts on that GPU runs the reference's loop as it runs
                       there)
    TapeDraws          the same draws read from a tape: u[j] for draft j and
                       one row e of Exp(1) values; multinomial(w, 1) is
                       argmax(w / e) (the exponential-race form torch's
                       multinomial uses for one sample; the tests pin it
                       against torch)
    greedy_chain       greedy verification (top_k = 1 with a unique maximum;
                       the reference's greedy reads the first maximal index,
                       packages/wpt-worker/src/wpt_worker/evaluation.py:74-81)
    greedy_tree        greedy verification of a draft tree: from the root,
                       the child whose token is the argmax (lowest index among
                       equal children), until none is; then the argmax
    cut                _cut (:338-344): up to the first stop, at most limit
    remember           the drafter's context after a read (_remember,
                       :140-152): each row's last `window` feature rows
                       once the model has read the first counts[b] of its
                       new tokens (zeros before the text)
    schedule           DSpark's prefix scheduler (:236-262): pass widths
                       admitted from the narrowest while the expected tokens
                       per second grow, the first that does not stopping it
"""

import torch


def probabilities(scores, temperature, top_k):
    """scores (..., V) -> FP32 probabilities (..., V): scores / temperature,
    every score below the top_k-th largest masked (ties with it kept), softmax."""
    scores = scores.float() / temperature
    if top_k is not None:
        k = min(top_k, scores.size(-1))
        v, _ = torch.topk(scores, k)
        scores = scores.masked_fill(scores < v[..., [-1]], float("-inf"))
    return torch.softmax(scores, dim=-1)


def multinomial_by_exponential(w, e):
    """One draw from the (unnormalized) distribution w given e ~ Exp(1) per
    entry: the first index of the largest w / e."""
    return int(torch.argmax(w / e))


class LazyDraws:
    """The reference's draws, made from `generator` as its loop makes them."""

    def __init__(self, generator):
        self.generator = generator
        self.uniforms, self.exponentials = [], []  # what was drawn, for a tape replay

    def uniform(self, j):
        u = torch.rand((), generator=self.generator, device=self.generator.device)
        self.uniforms.append(float(u))
        return u

    def multinomial(self, w):
        # record the exponentials the draw consumes (the same state advance)
        state = self.generator.get_state()
        self.exponentials.append(torch.empty_like(w).exponential_(generator=self.generator))
        self.generator.set_state(state)
        return int(torch.multinomial(w, 1, generator=self.generator))


class TapeDraws:
    """Draws read from a tape: u (L,) uniforms, e (V,) Exp(1) values."""

    def __init__(self, u, e):
        self.u, self.e = u, e

    def uniform(self, j):
        return self.u[j]

    def multinomial(self, w):
        return multinomial_by_exponential(w, self.e)


def accept_row(p, q, drafts, length, draws):
    """The tokens one row writes: p (>= length + 1, V) the model's
    probabilities at its pending token and at each draft, q (>= length, V)
    the drafts' distributions, drafts (>= length,) the drafted tokens."""
    tokens = []
    for j, token in enumerate(drafts[:length].tolist()):
        u = draws.uniform(j)
        if u * q[j, token] < p[j, token]:  # kept with probability min(1, p / q)
            tokens.append(token)
            continue
        rest = (p[j] - q[j]).clamp(min=0)
        tokens.append(draws.multinomial(rest / rest.sum()))
        break
    else:  # every draft kept: one more token from the model
        tokens.append(draws.multinomial(p[length]))
    return tokens


def accept(scores, q, drafts, lengths, temperature, top_k, draws):
    """Every row's tokens: scores (B, >= L + 1, V), q (B, L, V), drafts
    (B, L), lengths (B,) ints, draws[b] the row's draw source."""
    out = []
    for b in range(scores.shape[0]):
        n = int(lengths[b])
        p = probabilities(scores[b, :n + 1], temperature, top_k)
        out.append(accept_row(p, q[b].float(), drafts[b], n, draws[b]))
    return out


def margins(scores, q, drafts, lengths, temperature, top_k, u):
    """The smallest relative gap |u q - p| / p over the decisions each row
    makes along its tape (how far each decision is from flipping)."""
    gaps = []
    for b in range(scores.shape[0]):
        n = int(lengths[b])
        p = probabilities(scores[b, :n + 1], temperature, top_k)
        gap = float("inf")
        for j, token in enumerate(drafts[b, :n].tolist()):
            left, right = float(u[b, j] * q[b, j, token]), float(p[j, token])
            gap = min(gap, abs(left - right) / max(abs(right), 1e-30))
            if not left < right:
                break
        gaps.append(gap)
    return gaps


def first_argmax(scores):
    """The first index of the largest value along the last dimension."""
    return scores.float().argmax(-1)


def greedy_chain(scores, drafts, lengths):
    """Greedy verification of each row's chain of drafts: the longest prefix
    equal to the argmax at each position, then the argmax after it."""
    out = []
    best = first_argmax(scores)
    for b in range(scores.shape[0]):
        tokens = []
        for j in range(int(lengths[b])):
            if int(drafts[b, j]) != int(best[b, j]):
                break
            tokens.append(int(drafts[b, j]))
        tokens.append(int(best[b, len(tokens)]))
        out.append(tokens)
    return out


def greedy_tree(scores, node_tokens, parents):
    """Greedy verification of a draft tree per row: scores (B, M, V) at the M
    nodes, node_tokens (B, M), parents (M,) with parents[0] = -1 (the root,
    the token already written).  Returns (path of node indices from the
    root, written tokens) per row."""
    best = first_argmax(scores)
    children = [[] for _ in parents]
    for i, parent in enumerate(parents):
        if parent >= 0:
            children[parent].append(i)
    out = []
    for b in range(scores.shape[0]):
        node, path, tokens = 0, [0], []
        while True:
            target = int(best[b, node])
            match = [c for c in children[node] if int(node_tokens[b, c]) == target]
            if not match:
                tokens.append(target)
                break
            node = min(match)
            path.append(node)
            tokens.append(int(node_tokens[b, node]))
        out.append((path, tokens))
    return out


def remember(context, found, counts, window):
    """context (B, window, F) or None, found (B, n, F) the features the read
    gave, counts (B,) ints: the rows that end counts[b] rows into found, for
    each row b, with the earlier context in front."""
    found = found.float()
    if context is None:
        context = found.new_zeros(found.shape[0], window, found.shape[-1])
    joined = torch.cat([context, found], 1)
    return torch.stack([joined[b, int(n):int(n) + window] for b, n in enumerate(counts)])


def cut(tokens, stops, limit):
    """tokens up to the first stop token, at most limit of them."""
    for i, token in enumerate(tokens):
        if token in stops:
            tokens = tokens[:i + 1]
            break
    return tokens[:limit]


def schedule(confidences, caps, costs):
    """How many drafts of each row one pass verifies (:236-262): width w
    costs costs[w] seconds and adds, for every row whose cap reaches it, the
    product of that row's confidences up to draft w - 1 to the expected
    tokens (one per row to start); widths are admitted while tokens / cost
    grows."""
    chances = [1.0] * len(caps)
    expected = float(len(caps))
    best, admitted = expected / costs[0], 0
    for width in range(1, max(caps, default=0) + 1):
        for r, cap in enumerate(caps):
            if width <= cap:
                chances[r] *= confidences[r][width - 1]
                expected += chances[r]
        if not expected / costs[width] > best:
            break
        best, admitted = expected / costs[width], width
    return [min(admitted, cap) for cap in caps]
