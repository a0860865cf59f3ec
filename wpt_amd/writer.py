"""Speculative writing with the verify step on the GPU: the reference's Writer
(packages/wpt-inference/src/wpt_inference/__init__.py:71-233) with the same
signature, protocol and counters, its acceptance loop replaced by the fused
HIP sampler (wpt_amd.sampling).

What differs from the reference, by design:
    the draws    the reference draws lazily from `generator` (torch.rand per
                 draft it looks at, torch.multinomial per row, :214-222);
                 here each step draws one tape up front from the same
                 generator (sampling.draws: u (rows, drafts), e (rows, V)),
                 and every row is decided on the GPU at once.  The tokens
                 follow the same distribution; a tape made from a lazy run's
                 draws replays it exactly.
    host syncs   one per step (the written tokens), instead of one per draft
                 token (:213, :215, :219, :222).
With a drafter that gives confidences and a table of pass times (costs), each
step verifies only the drafts the prefix scheduler admits
(wpt_amd.scheduling.schedule, the reference's :236-262), as the reference does.
A drafter that reads the model's features (drafter.features, the layers whose
hidden states it reads, and drafter.window, how many of the last read tokens'
states) gets the context the reference's Writer keeps (:140-152, 184-200):
each row's last `window` feature rows, updated after every read the model
makes, with a row's pending tokens but its last read first.
"""

import torch
import torch.nn.functional as F

from . import sampling
from .scheduling import schedule

DRAFT = 5  # draft tokens per row and step (the reference's DRAFT, :67)


def cut(tokens, stops, limit):
    """tokens up to the first stop token, at most limit of them (:338-344)."""
    for i, token in enumerate(tokens):
        if token in stops:
            tokens = tokens[:i + 1]
            break
    return tokens[:limit]


class Writer:
    """Writes for `rows` rows that all start from prompt (a list of ints, at
    least one); the arguments are the reference's (:71-116)."""

    def __init__(self, model, prompt, rows=1, *, temperature=0.8, top_k=40, generator=None, stops=(), drafter=None,
                 draft=DRAFT, costs=None, outcomes=None, routes=False):
        if not prompt:
            raise ValueError("a prompt holds at least one token")
        if costs is not None and len(costs) < draft + 1:
            raise ValueError(f"costs gives {len(costs)} pass times; drafting {draft} tokens needs {draft + 1}")
        self.model, self.temperature, self.top_k, self.generator = model, temperature, top_k, generator
        self.stops, self.drafter, self.draft, self.costs = set(stops), drafter, draft, costs
        self.outcomes = outcomes
        self.rounds = self.verified = self.accepted = 0
        self.device = next(model.parameters()).device
        self.histories = [list(prompt) for _ in range(rows)]
        self.pending = [[prompt[-1]] for _ in range(rows)]
        self.features = tuple(drafter.features) if drafter is not None else ()
        self.cache = self.context = None  # context: the drafter's (rows, window, F)
        if hasattr(model, "new_cache"):
            shared = model.new_cache(1, routes=routes)
            if len(prompt) > 1:
                read = model.extend(self._tensor([prompt[:-1]]), shared, features=self.features)
                self._remember(read, [len(prompt) - 1])
            self.cache = shared.select([0] * rows)
            if self.context is not None:  # the prompt's context, in every row
                self.context = self.context.expand(rows, -1, -1).clone()
            elif self.features:  # nothing read yet: zeros before the text
                self.context = torch.zeros(rows, drafter.window, len(self.features) * model.config.d_model,
                                           device=self.device)
        elif drafter is not None or routes:
            raise ValueError("drafting and recording routes need a model with a generation cache")

    @torch.no_grad()
    def write(self, inputs, limits):
        """inputs: {row: tokens it reads before writing}; limits: {row: the
        most tokens it may write now, at least 1}.  Returns {row: the tokens
        it wrote}: at least one, at most its limit, ending at the first stop."""
        rows = sorted(limits)
        for row in rows:
            self.pending[row] += inputs.get(row, [])
            self.histories[row] += inputs.get(row, [])
        if self.drafter is not None:
            written = self._speculate(rows, limits)
        else:
            written = {row: [token] for row, token in zip(rows, self._sample(self._scores(rows)))}
        for row, tokens in written.items():
            self.histories[row] += tokens
            self.pending[row] = [tokens[-1]]
        return written

    def _tensor(self, rows):
        width = max(len(row) for row in rows)
        return torch.tensor([row + [0] * (width - len(row)) for row in rows], dtype=torch.long, device=self.device)

    def _remember(self, read, counts):
        """The drafter's context once the model has read (read: extend's
        result, with features) the first counts[b] of row b's new tokens:
        each row's last `window` feature rows, older ones first."""
        if not self.features:
            return
        found = read[2].float()
        window = self.drafter.window
        if self.context is None:
            self.context = found.new_zeros(found.shape[0], window, found.shape[-1])
        joined = torch.cat([self.context, found], 1)
        starts = torch.as_tensor(counts, dtype=torch.long, device=found.device)
        places = starts[:, None] + torch.arange(window, device=found.device)
        self.context = joined.gather(1, places[..., None].expand(-1, -1, found.shape[-1]))

    def _read(self, rows, extra=None, undoable=False):
        feeds = [[] for _ in self.pending]
        for i, row in enumerate(rows):
            feeds[row] = self.pending[row] + (extra[i] if extra is not None else [])
        read = self.model.extend(self._tensor(feeds), self.cache, [len(feed) for feed in feeds], undoable,
                                 features=self.features)
        return read[0][rows], read

    def _catch_up(self, rows):
        """The model reads each row's pending tokens but its last (a tool
        result, the template's), so that the context reaches its anchor."""
        behind = [row for row in rows if len(self.pending[row]) > 1]
        if not behind:
            return
        feeds = [self.pending[row][:-1] if row in behind else [] for row in range(len(self.pending))]
        counts = [len(feed) for feed in feeds]
        read = self.model.extend(self._tensor(feeds), self.cache, counts, features=self.features)
        self._remember(read, counts)
        for row in behind:
            self.pending[row] = self.pending[row][-1:]

    def _scores(self, rows):
        if self.cache is None:
            return torch.cat([self.model(self._tensor([self.histories[row]]))[:, -1] for row in rows])
        scores, _ = self._read(rows)
        ends = torch.tensor([len(self.pending[row]) - 1 for row in rows], device=self.device)
        return scores[torch.arange(len(rows), device=self.device), ends]

    def _probabilities(self, scores):
        """The reference's sampling distribution (:173-179), for drafters."""
        scores = scores.float() / self.temperature
        if self.top_k is not None:
            k = min(self.top_k, scores.size(-1))
            v, _ = torch.topk(scores, k)
            scores = scores.masked_fill(scores < v[..., [-1]], float("-inf"))
        return F.softmax(scores, dim=-1)

    def _sample(self, scores):
        """One token per row from the distribution of its scores (R, V)."""
        R, V = scores.shape
        u, e = sampling.draws(R, 0, V, self.generator, self.device)
        tokens, counts = sampling.accept(scores[:, None].float(), scores.new_empty(R, 0, V, dtype=torch.float32),
                                         torch.empty(R, 0, dtype=torch.long, device=self.device), u, e,
                                         self.temperature, self.top_k)
        return [row[0] for row in sampling.written(tokens, counts)]

    def _speculate(self, rows, limits):
        """One step of speculative decoding for rows (:196-233)."""
        if self.features:
            self._catch_up(rows)
        context = (self.context[rows], self.cache.lengths[rows]) if self.features else None
        drafted, q, confidences = self.drafter.draft(self.model, [self.histories[row] for row in rows], context,
                                                     self.draft, self._probabilities, self.generator)
        drafted, q = drafted.to(self.device), q.to(self.device).float()
        caps = [min(self.draft, limits[row] - 1) for row in rows]  # a row writes at most its drafts and one more
        scheduled = confidences is not None and self.costs is not None
        lengths = schedule(confidences.tolist(), caps, self.costs) if scheduled else caps
        scores, read = self._read(rows, [drafted[i, :n].tolist() for i, n in enumerate(lengths)], undoable=True)
        firsts = [len(self.pending[row]) - 1 for row in rows]
        L = drafted.shape[1]
        u, e = sampling.draws(len(rows), L, scores.shape[-1], self.generator, self.device)
        tokens, counts = sampling.accept(scores, q, drafted, u, e, self.temperature, self.top_k, lengths=lengths,
                                         firsts=firsts)
        written, kept = {}, [0] * len(self.pending)
        for i, (row, drawn) in enumerate(zip(rows, sampling.written(tokens, counts))):
            self.verified += lengths[i]
            self.accepted += len(drawn) - 1
            if self.outcomes is not None and confidences is not None:
                self.outcomes.append((confidences[i, :lengths[i]].tolist(), min(len(drawn) - 1, lengths[i])))
            drawn = cut(drawn, self.stops, limits[row])
            written[row] = drawn
            kept[row] = firsts[i] + len(drawn)
        self.rounds += 1
        self.model.undo(self.cache, kept)
        self._remember(read, kept)
        return written
