"""Speculative writing around the GPU verify step: the reference's Writer
interface (packages/wpt-inference/src/wpt_inference/__init__.py:71-233:
constructor arguments, `write`, the rounds/verified/accepted counters and the
drafter protocol), built on this package's device-resident pieces.

How a round runs here:
    drafting    the drafter drafts for the rows being written (with the
                features context when it reads the model's features);
    the feed    each row's unread tokens and the drafts it verifies are laid
                into one (rows, width) id tensor on the device -- the drafts
                never travel to the host;
    verify      one undoable `extend` reads every row, the fused sampler
                (wpt_amd.sampling.accept) decides all rows at once on the
                logits as the lm_head wrote them;
    the host    one synchronization brings the written tokens back (plus one
                for the confidences when the prefix scheduler runs); the
                cache then keeps what each row wrote, and the features
                context follows.

The draws are the ones the reference's loop makes from `generator` (a torch
generator on the model's GPU; None: the device's default one), in its order:
the sampler replays the generator's stream on the device
(sampling.accept_in_order) and the generator is then moved past what was
drawn, so a Writer seeded alike writes the reference Writer's tokens.

capture=True (an MQADecoder): a round in which every row verifies the same
number of drafts after its anchor alone (no inputs, no scheduler cut) runs
the verify reading and the acceptance from a HIP graph captured for that
shape, on static copies of the feed and the drafts; the cache's tables are
reserved ahead for the replays.  The same kernels run, so the tokens are the
eager round's.
"""

from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from . import sampling
from .decoder import MQADecoder
from .scheduling import schedule

DRAFT = 5  # draft tokens a row may verify per round (the reference's default, __init__.py:67)


def cut(tokens, stops, limit):
    """The tokens through the first one in `stops`, and no more than `limit`
    of them (the reference's _cut, __init__.py:338-344)."""
    end = next((i + 1 for i, token in enumerate(tokens) if token in stops), len(tokens))
    return tokens[:min(end, limit)]


@dataclass
class _Row:
    """One row being written: its whole text, and the tail of it the model
    has not read yet (at least its last token, which the next draft follows)."""
    text: list
    unread: list = field(default_factory=list)


def sampling_distribution(scores, temperature, top_k):
    """The reference's Writer._probabilities (__init__.py:173-179): FP32
    scores over the temperature, every score below the top_k-th at -inf (ties
    with it kept), softmax.  Handed to drafters as `probabilities`."""
    scaled = scores.float() / temperature
    if top_k is not None:
        kth = torch.topk(scaled, min(top_k, scaled.shape[-1])).values[..., -1:]
        scaled = torch.where(scaled < kth, torch.full_like(scaled, float("-inf")), scaled)
    return F.softmax(scaled, dim=-1)


class Writer:
    """Writes for `rows` rows that all start from `prompt` (a list of ints,
    at least one token).  Arguments as the reference's Writer: temperature,
    top_k (None: the whole vocabulary), generator (on the model's device;
    None: torch's default), stops (tokens after which a row's call returns),
    drafter / draft / costs / outcomes (speculative decoding: the drafts per
    round, the pass-time table the prefix scheduler reads, a list collecting
    (confidences, kept drafts) per verified row), routes (passed to the
    model's cache)."""

    def __init__(self, model, prompt, rows=1, *, temperature=0.8, top_k=40, generator=None, stops=(), drafter=None,
                 draft=DRAFT, costs=None, outcomes=None, routes=False, capture=False):
        if not prompt:
            raise ValueError("a prompt holds at least one token")
        if costs is not None and len(costs) < draft + 1:
            raise ValueError(f"costs gives {len(costs)} pass times; drafting {draft} tokens needs {draft + 1}")
        cached = hasattr(model, "new_cache")
        if not cached and (drafter is not None or routes):
            raise ValueError("drafting and recording routes need a model with a generation cache")
        self.model, self.drafter, self.draft, self.costs, self.outcomes = model, drafter, draft, costs, outcomes
        self.temperature, self.top_k, self.generator, self.stops = temperature, top_k, generator, frozenset(stops)
        self.rounds = self.verified = self.accepted = 0
        self.device = next(model.parameters()).device
        self._rows = [_Row(list(prompt), [prompt[-1]]) for _ in range(rows)]
        self.features = tuple(getattr(drafter, "features", ())) if drafter is not None else ()
        self.cache = None
        self.context = None  # a feature-reading drafter's context: (rows, window, features x d_model)
        self.capture = bool(capture) and isinstance(model, MQADecoder)
        self._reads = {}  # drafts a row -> _CapturedRead
        if not cached:
            return
        # the prompt but its last token is read once, into a one-row cache copied to every row
        one = model.new_cache(1, routes=routes)
        if len(prompt) > 1:
            read = model.extend(torch.tensor([prompt[:-1]], dtype=torch.long, device=self.device), one,
                                features=self.features)
            self._follow(read, [len(prompt) - 1])
        self.cache = one.select([0] * rows)
        if self.features:
            if self.context is None:  # nothing read: the window holds zeros before the text
                self.context = torch.zeros(1, drafter.window, len(self.features) * model.config.d_model,
                                           dtype=getattr(model, "dtype", torch.float32), device=self.device)
            self.context = self.context.expand(rows, -1, -1).clone()

    @property
    def histories(self):
        """Each row's whole text: the prompt, its inputs and what it wrote."""
        return [row.text for row in self._rows]

    @property
    def routes(self):
        """Each row's recorded routes, from the model's cache (None without one)."""
        return self.cache.routes if self.cache is not None else None

    @property
    def pending(self):
        """Each row's tokens the model has not read yet (the last is the anchor)."""
        return [row.unread for row in self._rows]

    def _probabilities(self, scores):
        return sampling_distribution(scores, self.temperature, self.top_k)

    @torch.no_grad()
    def write(self, inputs, limits):
        """inputs: {row: tokens it reads before writing (possibly none)};
        limits: {row: the most tokens it may write now, at least 1}.  Returns
        {row: the tokens it wrote}: at least one, at most its limit, through
        its first stop token."""
        order = sorted(limits)
        for r in order:
            extra = list(inputs.get(r, ()))
            self._rows[r].text.extend(extra)
            self._rows[r].unread.extend(extra)
        if self.drafter is None:
            out = dict(zip(order, ([t] for t in self._plain(order))))
        else:
            out = self._round(order, limits)
        for r, tokens in out.items():
            self._rows[r].text.extend(tokens)
            self._rows[r].unread = [tokens[-1]]
        return out

    # ---- reading ---------------------------------------------------------

    def _ids(self, feeds, spare=0):
        """feeds: a token list per cache row -> (ids (rows, width + spare)
        int64 on the device, zero-padded; the counts); width is the longest
        feed (at least 1)."""
        counts = [len(f) for f in feeds]
        width = max(1, max(counts))
        ids = torch.zeros(len(feeds), width + spare, dtype=torch.long)
        for r, f in enumerate(feeds):
            if f:
                ids[r, :len(f)] = torch.tensor(f, dtype=torch.long)
        return ids.to(self.device, non_blocking=True), counts

    def _follow(self, read, counts):
        """Moves the drafter's features context past the first counts[b] of
        the tokens the model just read (read: extend's result with features):
        each row keeps the features of its last `window` read tokens."""
        if not self.features:
            return
        # the features come as FP32 (the reference's dtype for them); they are the
        # model's residual stream, so its dtype (bf16) holds them exactly and
        # halves the window's traffic
        fresh = read[2].to(getattr(self.model, "dtype", read[2].dtype))
        window = self.drafter.window
        held = self.context if self.context is not None else fresh.new_zeros(fresh.shape[0], window, fresh.shape[-1])
        both = torch.cat([held, fresh], 1)
        take = torch.as_tensor(counts, dtype=torch.long, device=fresh.device)[:, None] + torch.arange(
            window, device=fresh.device)
        self.context = torch.take_along_dim(both, take[..., None], 1)

    def _read_up_to_anchor(self, order):
        """Reads each row's unread tokens but its anchor (inputs given with a
        call), so that the features context ends at the anchor."""
        feeds = [row.unread[:-1] if (r in order and len(row.unread) > 1) else [] for r, row in enumerate(self._rows)]
        if not any(feeds):
            return
        ids, counts = self._ids(feeds)
        self._follow(self.model.extend(ids, self.cache, counts, features=self.features), counts)
        for r, f in enumerate(feeds):
            if f:
                self._rows[r].unread = self._rows[r].unread[-1:]

    # ---- a call without a drafter: one sampled token per row ---------------

    def _plain(self, order):
        if self.cache is None:  # a model without a cache reads each row's whole text
            last = torch.cat([self.model(torch.tensor([self._rows[r].text], dtype=torch.long, device=self.device))[:, -1]
                              for r in order])
        else:
            feeds = [row.unread if r in order else [] for r, row in enumerate(self._rows)]
            ids, counts = self._ids(feeds)
            scores = self.model.extend(ids, self.cache, counts)[0]
            pick = torch.tensor(order, dtype=torch.long, device=self.device)
            at = torch.tensor([counts[r] - 1 for r in order], dtype=torch.long, device=self.device)
            last = scores[pick, at]
        # the reference's _sample: one multinomial over every row's distribution
        scores = last[:, None] if last.dtype in (torch.float32, torch.bfloat16) else last[:, None].float()
        state = sampling.generator_state(self.generator, self.device)
        tokens, counts = sampling.accept_in_order(scores, None, None, state, self.temperature, self.top_k, joint=True)
        drawn = sampling.written(tokens, counts)
        sampling.set_offset(self.generator, state, self.device)
        return [d[0] for d in drawn]

    # ---- a speculative round ------------------------------------------------

    def _round(self, order, limits):
        if self.features:
            self._read_up_to_anchor(order)
        if self.features:  # every row in order (a steady round) takes the context as it stands: no copy
            whole = list(order) == list(range(len(self._rows)))
            context = (self.context, self.cache.lengths) if whole else (self.context[order], self.cache.lengths[order])
        else:
            context = None
        drafts, q, confidence = self.drafter.draft(self.model, [self._rows[r].text for r in order], context,
                                                   self.draft, self._probabilities, self.generator)
        drafts = drafts.to(self.device, torch.long)
        q = q.to(self.device, torch.float32)
        L = drafts.shape[1]
        # a row writes at most its verified drafts and one token more
        caps = [min(self.draft, limits[r] - 1) for r in order]
        if confidence is not None and self.costs is not None:
            verify = schedule(confidence.tolist(), caps, self.costs)
        else:
            verify = caps
        # the feed of row r: its unread tokens, then the first verify[i] drafts;
        # the first token each row writes is scored at its last unread token
        firsts = [len(self._rows[r].unread) - 1 for r in order]
        feeds = [[] for _ in self._rows]
        for i, r in enumerate(order):
            feeds[r] = self._rows[r].unread + [0] * verify[i]
        steady = (self.capture and L > 0 and order == list(range(len(self._rows))) and not any(firsts)
                  and all(v == L for v in verify))
        if steady:
            read, scores, tokens, ncounts = self._captured_round(drafts, q, L)
            return self._finish_round(order, limits, verify, firsts, confidence, read, tokens, ncounts)
        ids, counts = self._ids(feeds, spare=1)
        width = ids.shape[1] - 1
        pick = torch.tensor(order, dtype=torch.long, device=self.device)
        if L:
            # the drafts laid in on the device (no trip to the host): draft j of
            # row order[i] at column firsts[i] + 1 + j when j < verify[i], the
            # others into the spare last column, which is then cut off
            j = torch.arange(L, device=self.device)[None]
            start = torch.tensor(firsts, dtype=torch.long, device=self.device)[:, None] + 1
            wanted = j < torch.tensor(verify, dtype=torch.long, device=self.device)[:, None]
            cols = torch.where(wanted, start + j, torch.full_like(start + j, width))
            ids[pick[:, None].expand(-1, L), cols] = drafts
        ids = ids[:, :width].contiguous()
        if isinstance(self.model, MQADecoder):  # the logits as the head writes them, read by the sampler as FP32
            read = self.model.extend(ids, self.cache, counts, True, features=self.features, logits=True)
        else:
            read = self.model.extend(ids, self.cache, counts, True, features=self.features)
        scores = read[0] if order == list(range(len(self._rows))) else read[0][pick]
        state = sampling.generator_state(self.generator, self.device)
        tokens, ncounts = sampling.accept_in_order(scores, q, drafts, state, self.temperature, self.top_k,
                                                   lengths=verify, firsts=firsts)
        return self._finish_round(order, limits, verify, firsts, confidence, read, tokens, ncounts, state)

    def _finish_round(self, order, limits, verify, firsts, confidence, read, tokens, ncounts, state=None):
        """The round's one synchronization and the host's part: each row's
        written tokens cut at its stops and limit, the counters, the undo of
        what the rows did not keep, the features context."""
        drawn = sampling.written(tokens, ncounts)  # the round's synchronization
        if state is not None:
            sampling.set_offset(self.generator, state, self.device)
        out, keep = {}, [0] * len(self._rows)
        for i, r in enumerate(order):
            self.verified += verify[i]
            self.accepted += len(drawn[i]) - 1
            if self.outcomes is not None and confidence is not None:
                self.outcomes.append((confidence[i, :verify[i]].tolist(), min(len(drawn[i]) - 1, verify[i])))
            out[r] = cut(drawn[i], self.stops, limits[r])
            # the cache keeps the row's unread tokens and what it wrote but the last (the next anchor)
            keep[r] = firsts[i] + len(out[r])
        self.rounds += 1
        self.model.undo(self.cache, keep)
        self._follow(read, keep)
        return out

    def _captured_round(self, drafts, q, L):
        """The verify reading and the acceptance of a steady round from the
        graph of its shape: (read, scores, tokens, counts), the graph's
        tensors.  The generator hands its state over and takes it back."""
        cap = self._reads.get(L)
        width = L + 1
        if cap is None or self.cache.bound + width > cap.limit:
            cap = self._reads[L] = _CapturedRead(self, L)
        anchors = torch.tensor([row.unread[0] for row in self._rows], dtype=torch.long)
        cap.ids[:, 0].copy_(anchors, non_blocking=True)
        cap.ids[:, 1:].copy_(drafts)
        cap.q.copy_(q)
        cap.drafts.copy_(drafts)
        cap.state.copy_(sampling.generator_state(self.generator, self.device))
        cap.graph.replay()
        # what the reading's host side would have recorded (a replay runs no Python)
        self.cache.pending = True
        self.cache.bound += width
        sampling.set_offset(self.generator, cap.state, self.device)  # the round's synchronization
        return cap.read, cap.read[0], cap.tokens, cap.counts


class _CapturedRead:
    """A steady round's verify reading (every row: its anchor, then L drafts)
    and its acceptance, captured in a HIP graph over static inputs; the
    cache's tables are reserved for ROUNDS more such readings first (a
    graph cannot grow them: past that a new one is captured)."""

    ROUNDS = 64

    def __init__(self, writer, L):
        model, cache, device = writer.model, writer.cache, writer.device
        rows, V, width = cache.rows, model.config.vocab, L + 1
        self.ids = torch.zeros(rows, width, dtype=torch.long, device=device)
        self.q = torch.zeros(rows, L, V, device=device)
        self.drafts = torch.zeros(rows, L, dtype=torch.long, device=device)
        self.state = sampling.generator_state(writer.generator, device).clone()
        cache.reserve(cache.bound + width * self.ROUNDS)
        self.limit = cache.capacity
        pending, bound = cache.pending, cache.bound
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):  # records the kernels; runs none
            self.read = model.extend(self.ids, cache, None, True, features=writer.features, logits=True)
            self.tokens, self.counts = sampling.accept_in_order(self.read[0], self.q, self.drafts, self.state,
                                                                writer.temperature, writer.top_k)
        cache.pending, cache.bound = pending, bound
