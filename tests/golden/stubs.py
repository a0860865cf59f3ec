"""A stub model and drafters for the Writer's golden token streams: small,
deterministic, CPU-only, with the reference's model protocol (new_cache /
extend / undo, model.py:451-483) and drafter protocol
(wpt_inference/__init__.py:17-33).  Shared by make_writer_vectors.py, which
runs the reference's own Writer on them, and by the test that replays the
streams through the oracle."""

from types import SimpleNamespace

import torch


class Rows:
    """A cache of lengths only: the stub model's scores do not depend on the
    text before a token."""

    def __init__(self, rows):
        self.lengths = torch.zeros(rows, dtype=torch.long)
        self.before = None
        self.routes = None

    def select(self, index):
        copy = Rows(len(index))
        copy.lengths = self.lengths[torch.as_tensor(index, dtype=torch.long)]
        return copy


FEATURE_WIDTH = 4  # the stub's d_model: the width of one layer's features


class Bigram:
    """scores of a token = a fixed row of a (V, V) table (times 3, so that
    the distributions are peaked): the next-token scores depend on the last
    token only.  Its "features" (the residual stream entering layer n, as
    the reference's extend returns them for features=(n, ...)) are a fixed
    slice of the token's table row scaled by n + 1."""

    def __init__(self, vocab=50, seed=0):
        generator = torch.Generator().manual_seed(seed)
        self.table = torch.randn(vocab, vocab, generator=generator) * 3
        self.config = SimpleNamespace(d_model=FEATURE_WIDTH, vocab=vocab)

    def features_of(self, ids, number):
        return self.table[ids][..., :FEATURE_WIDTH] * (number + 1) / 3

    def parameters(self):
        return iter([self.table])

    def new_cache(self, rows, routes=False):
        return Rows(rows)

    def extend(self, ids, cache, counts=None, undoable=False, features=()):
        B, n = ids.shape
        counts = torch.full((B,), n) if counts is None else torch.as_tensor(counts)
        if undoable:
            cache.before = cache.lengths.clone()
        cache.lengths = cache.lengths + counts
        scores = self.table[ids].float()
        if features:
            return scores, scores, torch.cat([self.features_of(ids, n) for n in features], -1)
        return scores, scores

    def undo(self, cache, kept):
        cache.lengths = cache.before + torch.as_tensor(kept)
        cache.before = None

    def __call__(self, ids):
        return self.table[ids].float()


class UniformDrafter:
    """Drafts uniform over the vocabulary, drawn from the writer's generator."""
    features, window = (), 0

    def draft(self, model, histories, context, count, probabilities, generator):
        V = model.config.vocab
        tokens = torch.randint(V, (len(histories), count), generator=generator)
        return tokens, torch.full((len(histories), count, V), 1.0 / V), None


class SkewedDrafter:
    """Drafts from the model's own scores plus fixed noise (std 1 against the
    table's 3), at the writer's temperature and top-k, so that drafts are
    kept and rejected in a mix; the draws come from the writer's generator,
    one multinomial per draft."""
    features, window = (), 0

    def __init__(self, vocab=50, seed=1):
        self.noise = torch.randn(vocab, vocab, generator=torch.Generator().manual_seed(seed))

    def draft(self, model, histories, context, count, probabilities, generator):
        tokens, distributions = [], []
        for history in histories:
            last = history[-1]
            row = []
            for _ in range(count):
                q = probabilities(model.table[last] + self.noise[last])
                last = int(torch.multinomial(q, 1, generator=generator))
                row.append(last)
                distributions.append(q)
            tokens.append(row)
        return torch.tensor(tokens), torch.stack(distributions).view(len(histories), count, -1), None


class ContextDrafter:
    """Drafts from the model's own scores shifted by its context (the
    features of each row's last `window` tokens read, and how many tokens
    the row has read), so that a context kept otherwise draws other tokens;
    one multinomial per draft from the writer's generator."""
    features, window = (0, 2), 3

    def draft(self, model, histories, context, count, probabilities, generator):
        found, lengths = context
        V = model.config.vocab
        tokens, distributions = [], []
        for r, history in enumerate(histories):
            shift = found[r].float().sum(0)  # (F,)
            bias = shift.repeat(V // shift.numel() + 1)[:V] + 0.25 * (int(lengths[r]) % 5)
            last, row = history[-1], []
            for _ in range(count):
                q = probabilities(model.table[last] + bias)
                last = int(torch.multinomial(q, 1, generator=generator))
                row.append(last)
                distributions.append(q)
            tokens.append(row)
        return torch.tensor(tokens), torch.stack(distributions).view(len(histories), count, -1), None


def cases():
    """The streams: (name, writer arguments, drafter, calls of write)."""
    return [
        ("uniform_drafts_top_k_40", dict(rows=3, temperature=0.8, top_k=40, draft=4), "uniform",
         [{0: 6, 1: 6, 2: 2}] * 4),
        ("skewed_drafts_no_top_k", dict(rows=3, temperature=1.0, top_k=None, draft=4), "skewed",
         [{0: 6, 1: 3, 2: 6}] * 5),
        ("skewed_drafts_top_k_5_t0.7", dict(rows=2, temperature=0.7, top_k=5, draft=5), "skewed",
         [{0: 7, 1: 7}] * 6),
        ("no_drafter_top_k_10", dict(rows=2, temperature=0.9, top_k=10, draft=4), None, [{0: 1, 1: 1}] * 5),
    ]


def context_cases():
    """Streams of a drafter that reads the model's features: (name, prompt,
    writer arguments, calls of write as (inputs, limits)).  Inputs make rows
    read tokens before drafting (the Writer's catch-up); a one-token prompt
    starts the context at zeros."""
    return [
        ("context_drafter_inputs_no_top_k", [3, 17, 29, 8], dict(rows=3, temperature=0.9, top_k=None, draft=4),
         [({}, {0: 6, 1: 6, 2: 6}), ({1: [7, 11]}, {0: 6, 1: 6, 2: 3}), ({}, {0: 6, 1: 6, 2: 6}),
          ({0: [2], 2: [40, 41, 42]}, {0: 6, 1: 2, 2: 6}), ({}, {0: 6, 1: 6, 2: 6})]),
        ("context_drafter_one_token_prompt_top_k_8", [5], dict(rows=2, temperature=0.8, top_k=8, draft=3),
         [({}, {0: 5, 1: 5}), ({}, {0: 5, 1: 5}), ({1: [9]}, {0: 5, 1: 5}), ({}, {0: 5, 1: 5})]),
    ]


def drafter(kind):
    return {"uniform": UniformDrafter, "skewed": SkewedDrafter, "context": ContextDrafter}[kind]() if kind else None
