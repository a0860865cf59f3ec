"""Replays a golden Writer stream (tests/golden/writer_vectors.json, drawn by
the reference's own Writer) step by step with the oracle's rule and lazy draws,
keeping for each speculative step what the GPU sampler needs to decide it from
a tape: the scores, drafts, distributions, and the uniforms and exponentials
the lazy draws consumed.  A drafter that reads the model's features gets the
context the oracle keeps (oracle.sampling.remember), the rows' pending tokens
read first (the Writer's catch-up, __init__.py:184-194) and the cache's
lengths."""

import json
from pathlib import Path

import torch

from oracle import sampling as oracle
from tests.golden import stubs

VECTORS = Path(__file__).resolve().parent / "golden" / "writer_vectors.json"


def streams():
    return json.loads(VECTORS.read_text())


def _found(model, feeds, features):
    """The stub's features of each row's feed, padded with token 0 to the widest (B, n, F)."""
    width = max(1, max(len(feed) for feed in feeds))
    ids = torch.tensor([feed + [0] * (width - len(feed)) for feed in feeds])
    return torch.cat([model.features_of(ids, n) for n in features], -1)


def replay(case):
    """(the written tokens of every call, counters, the speculative steps)."""
    model = stubs.Bigram()
    drafter = stubs.drafter(case["drafter"])
    generator = torch.Generator().manual_seed(case["seed"])
    rows, draft = case["rows"], case["draft"]
    temperature, top_k = case["temperature"], case["top_k"]
    prompt = case["prompt"]
    histories = [list(prompt) for _ in range(rows)]
    pending = [[prompt[-1]] for _ in range(rows)]
    features = tuple(drafter.features) if drafter is not None else ()
    window = drafter.window if features else 0
    lengths = [len(prompt) - 1] * rows  # the tokens each row's cache holds
    context = None
    if features:
        if len(prompt) > 1:  # the prompt read once, its context copied into every row
            one = oracle.remember(None, _found(model, [prompt[:-1]], features), [len(prompt) - 1], window)
            context = one.expand(rows, -1, -1).clone()
        else:
            context = torch.zeros(rows, window, len(features) * model.config.d_model)

    def probabilities(scores):
        return oracle.probabilities(scores, temperature, top_k)

    out, steps = [], []
    counters = {"rounds": 0, "verified": 0, "accepted": 0}
    inputs = case.get("inputs") or [{} for _ in case["calls"]]
    for given, limits in zip(inputs, case["calls"]):
        for row, tokens in given.items():
            pending[int(row)] += tokens
            histories[int(row)] += tokens
        limits = {int(row): n for row, n in limits.items()}
        rs = sorted(limits)
        if drafter is None:  # the reference's _sample: one multinomial over every row's distribution
            scores = torch.stack([model.table[pending[row][-1]] for row in rs]).float()
            drawn = torch.multinomial(probabilities(scores), 1, generator=generator)[:, 0].tolist()
            written = {row: [token] for row, token in zip(rs, drawn)}
        else:
            if features:  # every pending token but each row's last is read first
                feeds = [pending[row][:-1] if row in rs and len(pending[row]) > 1 else [] for row in range(rows)]
                counts = [len(feed) for feed in feeds]
                if any(counts):
                    context = oracle.remember(context, _found(model, feeds, features), counts, window)
                    for row, n in enumerate(counts):
                        lengths[row] += n
                        if n:
                            pending[row] = pending[row][-1:]
            given_context = (context[rs], torch.tensor(lengths)[rs]) if features else None
            drafted, q, _ = drafter.draft(model, [histories[row] for row in rs], given_context, draft, probabilities,
                                          generator)
            caps = [min(draft, limits[row] - 1) for row in rs]
            step = {"scores": [], "q": q.float(), "drafts": drafted, "lengths": caps, "u": [], "e": [], "tokens": []}
            written, kept, feeds = {}, [0] * rows, [[] for _ in range(rows)]
            for i, row in enumerate(rs):
                feed = pending[row] + drafted[i, :caps[i]].tolist()
                feeds[row] = feed
                scores = model.table[torch.tensor(feed)].float()
                first = len(pending[row]) - 1
                draws = oracle.LazyDraws(generator)
                tokens = oracle.accept_row(probabilities(scores[first:first + caps[i] + 1]), q[i].float(), drafted[i],
                                           caps[i], draws)
                step["scores"].append(scores[first:])
                step["u"].append(draws.uniforms)
                step["e"].append(draws.exponentials[0])
                step["tokens"].append(tokens)
                counters["verified"] += caps[i]
                counters["accepted"] += len(tokens) - 1
                written[row] = oracle.cut(tokens, set(), limits[row])
                kept[row] = first + len(written[row])
            if features:
                context = oracle.remember(context, _found(model, feeds, features), kept, window)
            for row in range(rows):
                lengths[row] += kept[row]
            counters["rounds"] += 1
            steps.append(step)
        for row, tokens in written.items():
            histories[row] += tokens
            pending[row] = [tokens[-1]]
        out.append({str(row): tokens for row, tokens in written.items()})
    return out, counters, steps
