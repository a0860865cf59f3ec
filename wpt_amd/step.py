"""One speculative-decoding verify step of fixed shape, run eagerly or replayed
from a HIP graph: the model reads each row's pending token and its k drafts
(extend, undoable), every row is accepted or resampled on the GPU
(wpt_amd.sampling), and the cache takes back the rejected drafts (undo), as
the reference's Writer._speculate does (packages/wpt-inference/src/
wpt_inference/__init__.py:196-233) for rows whose only pending token is the
last one written (firsts = 0, kept = tokens written).

The inputs live in static device buffers (`feeds`: the pending token then the
drafts; `q`: the drafts' distributions), so that a captured graph replays on
new values: after each step the token it drew becomes each row's pending
token.  The draws: with `in_order=True` the ones the reference's loop makes
from `generator` (None: the device's default one), in its order, its Philox
stream replayed on the device from a device copy of the generator's state
(`state`, moved on by every step and replay; `sync_generator()` hands the
offset back to the generator); otherwise a tape (u, e) drawn inside the step
from torch's generator of the device, or read from the static buffers `u`,
`e` (`given_tape=True`), which the caller fills before each step.  After a
step, `scores` (and `u` and `e` for a tape) hold what it read.  The cache's tables must hold every row the replays will write
(reserve), since a graph cannot grow them.

A row whose residual max(0, p - q) has no mass cannot draw; the reference's
multinomial raises there (__init__.py:219).  Inside a step (and a graph) the
row writes nothing, keeps its pending token and its cache, and raises a
device flag; `check()` reads the flag (one synchronization) and raises.
"""

import torch

from . import _lib, sampling
from ._lib import check, ptr
from .cache import Cache
from .decoder import MQADecoder


def next_feeds(tokens, counts, feeds, failed=None, written=None):
    """feeds[:, 0] = each row's last written token, tokens[b, counts[b] - 1]
    (tokens (B, L + 1) int64, counts (B,) int32), on the device; a row with
    no token written keeps its feed and sets failed (an int32 device flag,
    when given) to 1.  written (B,) int64, when given: written[b] +=
    counts[b] for each row that wrote."""
    B, width = tokens.shape
    if counts.dtype != torch.int32 or counts.shape != (B,) or feeds.shape[0] != B or feeds.dtype != torch.int64:
        raise ValueError("tokens (B, L + 1) int64, counts (B,) int32 and feeds (B, n) int64")
    if failed is not None and (failed.dtype != torch.int32 or failed.numel() < 1):
        raise ValueError("failed must be an int32 device tensor")
    if written is not None and (written.dtype != torch.int64 or written.shape != (B,) or not written.is_contiguous()):
        raise ValueError("written must be a contiguous (B,) int64 device tensor")
    check(_lib.lib().wptv_next_feeds(ptr(tokens), tokens.stride(0), ptr(counts), ptr(feeds), feeds.stride(0), B, width,
                                     ptr(failed), ptr(written), _lib.stream(tokens.device)), "next_feeds")


class VerifyStep:
    def __init__(self, model, cache, k, temperature=0.8, top_k=None, greedy=False, given_tape=False,
                 in_order=False, generator=None):
        self.model, self.cache, self.k = model, cache, k
        self.temperature, self.top_k, self.greedy = temperature, top_k, greedy
        self.given_tape = given_tape
        B, V = cache.rows, model.config.vocab
        device = model.device
        if in_order and (greedy or given_tape):
            raise ValueError("in-order draws replace the tape; a greedy step draws nothing")
        self.in_order, self.generator = in_order, generator
        self.state = sampling.generator_state(generator, device) if in_order else None
        self.feeds = torch.zeros(B, k + 1, dtype=torch.long, device=device)
        self.q = torch.full((B, k, V), 1.0 / V, device=device)
        self.u = torch.zeros(B, k, device=device) if given_tape else None
        self.e = torch.ones(B, V, device=device) if given_tape else None
        self.failed = torch.zeros(1, dtype=torch.int32, device=device)
        self.written = torch.zeros(B, dtype=torch.long, device=device)  # tokens each row has written, running
        self.graph = None
        self.tokens = self.counts = self.scores = None

    def run(self):
        """One eager step; returns (tokens (B, k + 1), counts (B,)) on the device."""
        scores, _ = self.model.extend(self.feeds, self.cache, undoable=True, logits=True)  # read as they come
        drafts = self.feeds[:, 1:]
        if not (self.greedy or self.given_tape or self.in_order):
            B, V = scores.shape[0], scores.shape[-1]
            self.u, self.e = sampling.draws(B, self.k, V, device=scores.device)
        # the pick's kernel also takes back the rejected drafts (the model's
        # undo, which for this cache is its lengths alone), makes the drawn
        # token each row's next pending token and grows the running counts
        if isinstance(self.cache, Cache) and type(self.model).undo is MQADecoder.undo:
            lengths, before = self.cache.undo_on_device()
            commit = (lengths, before, self.feeds, self.failed, self.written)
        else:
            commit = None
        if self.in_order:
            tokens, counts = sampling.accept_in_order(scores, self.q, drafts, self.state, self.temperature,
                                                      self.top_k, commit=commit)
        else:
            tokens, counts = sampling.accept(scores, self.q, drafts, self.u, self.e, self.temperature, self.top_k,
                                             greedy=self.greedy, commit=commit)
        if commit is None:
            self.model.undo(self.cache, counts)
            next_feeds(tokens, counts, self.feeds, self.failed, self.written)
        self.tokens, self.counts, self.scores = tokens, counts, scores
        return tokens, counts

    def sync_generator(self):
        """Moves the generator past every draw the in-order steps made (one
        synchronization)."""
        sampling.set_offset(self.generator, self.state, self.model.device)

    def check(self):
        """Raises if a step since the last check had a row with nothing to
        draw from (that row wrote nothing and kept its state); clears the flag."""
        if int(self.failed.item()):
            self.failed.zero_()
            raise RuntimeError("a row's residual distribution max(0, p - q) had no mass to draw from: the row "
                               "wrote nothing")

    def capture(self, warmup=2):
        """Captures the step in a HIP graph (after `warmup` eager steps on a
        side stream, as graph capture needs)."""
        stream = torch.cuda.Stream(self.model.device)
        stream.wait_stream(torch.cuda.current_stream(self.model.device))
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                self.run()
        torch.cuda.current_stream(self.model.device).wait_stream(stream)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.run()
        return self

    def replay(self):
        self.graph.replay()
        return self.tokens, self.counts


def prefill(model, cache, ids, chunk=1024):
    """Reads ids (B, n) into the cache in chunks of `chunk` tokens."""
    for start in range(0, ids.shape[1], chunk):
        model.extend(ids[:, start:start + chunk], cache)
