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
token.  The tape (u, e) is drawn inside the step from torch's generator of the
device.  The cache's tables must hold every row the replays will write
(reserve), since a graph cannot grow them.
"""

import torch

from . import _lib, sampling
from ._lib import check, ptr


def next_feeds(tokens, counts, feeds):
    """feeds[:, 0] = each row's last written token, tokens[b, counts[b] - 1]
    (tokens (B, L + 1) int64, counts (B,) int32), on the device."""
    B, width = tokens.shape
    if counts.dtype != torch.int32 or counts.shape != (B,) or feeds.shape[0] != B or feeds.dtype != torch.int64:
        raise ValueError("tokens (B, L + 1) int64, counts (B,) int32 and feeds (B, n) int64")
    check(_lib.lib().wptv_next_feeds(ptr(tokens), tokens.stride(0), ptr(counts), ptr(feeds), feeds.stride(0), B, width,
                                     _lib.stream(tokens.device)), "next_feeds")


class VerifyStep:
    def __init__(self, model, cache, k, temperature=0.8, top_k=None, greedy=False):
        self.model, self.cache, self.k = model, cache, k
        self.temperature, self.top_k, self.greedy = temperature, top_k, greedy
        B, V = cache.rows, model.config.vocab
        device = model.device
        self.feeds = torch.zeros(B, k + 1, dtype=torch.long, device=device)
        self.q = torch.full((B, k, V), 1.0 / V, device=device)
        self.graph = None
        self.tokens = self.counts = None

    def run(self):
        """One eager step; returns (tokens (B, k + 1), counts (B,)) on the device."""
        scores, _ = self.model.extend(self.feeds, self.cache, undoable=True, logits=True)  # read as they come
        drafts = self.feeds[:, 1:]
        if self.greedy:
            tokens, counts = sampling.greedy_chain(scores, drafts)
        else:
            B, V = scores.shape[0], scores.shape[-1]
            u, e = sampling.draws(B, self.k, V, device=scores.device)
            tokens, counts = sampling.accept(scores, self.q, drafts, u, e, self.temperature, self.top_k)
        self.model.undo(self.cache, counts)
        next_feeds(tokens, counts, self.feeds)  # the drawn token is each row's next pending token
        self.tokens, self.counts = tokens, counts
        return tokens, counts

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
