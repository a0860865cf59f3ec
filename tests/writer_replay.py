"""Replays a golden Writer stream (tests/golden/writer_vectors.json, drawn by
the reference's own Writer) step by step with the oracle's rule and lazy draws,
keeping for each speculative step what the GPU sampler needs to decide it from
a tape: the scores, drafts, distributions, and the uniforms and exponentials
the lazy draws consumed."""

import json
from pathlib import Path

import torch

from oracle import sampling as oracle
from tests.golden import stubs

VECTORS = Path(__file__).resolve().parent / "golden" / "writer_vectors.json"


def streams():
    return json.loads(VECTORS.read_text())


def replay(case):
    """(the written tokens of every call, counters, the speculative steps)."""
    model = stubs.Bigram()
    drafter = stubs.drafter(case["drafter"])
    generator = torch.Generator().manual_seed(case["seed"])
    rows, draft = case["rows"], case["draft"]
    temperature, top_k = case["temperature"], case["top_k"]
    histories = [list(case["prompt"]) for _ in range(rows)]
    pending = [[case["prompt"][-1]] for _ in range(rows)]

    def probabilities(scores):
        return oracle.probabilities(scores, temperature, top_k)

    out, steps = [], []
    counters = {"rounds": 0, "verified": 0, "accepted": 0}
    for limits in case["calls"]:
        limits = {int(row): n for row, n in limits.items()}
        rs = sorted(limits)
        if drafter is None:  # the reference's _sample: one multinomial over every row's distribution
            scores = torch.stack([model.table[pending[row][-1]] for row in rs]).float()
            drawn = torch.multinomial(probabilities(scores), 1, generator=generator)[:, 0].tolist()
            written = {row: [token] for row, token in zip(rs, drawn)}
        else:
            drafted, q, _ = drafter.draft(model, [histories[row] for row in rs], None, draft, probabilities, generator)
            caps = [min(draft, limits[row] - 1) for row in rs]
            step = {"scores": [], "q": q.float(), "drafts": drafted, "lengths": caps, "u": [], "e": [], "tokens": []}
            written = {}
            for i, row in enumerate(rs):
                feed = pending[row] + drafted[i, :caps[i]].tolist()
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
            counters["rounds"] += 1
            steps.append(step)
        for row, tokens in written.items():
            histories[row] += tokens
            pending[row] = [tokens[-1]]
        out.append({str(row): tokens for row, tokens in written.items()})
    return out, counters, steps
