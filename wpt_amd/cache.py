"""The generation cache of the MQA decoder on the GPU: the reference's Rows /
Reading / Cache (packages/wpt-model/src/wpt_model/cache.py:54-174) for exact
layers, whose carried value is every token's key and value side by side
(carry.Entries, carry.py:66-71), and for window layers, whose carried value
is the last window - 1 tokens' (carry.Tail, carry.py:30-63).

A window layer's entries live in a ring of R rows per batch row (R a power
of 2 of at least window - 1 + the widest reading), token p at row p mod R: a
reading writes its tokens over ones more than R - 1 tokens back, which no
query of it or of a later reading sees, so the ring holds the reference's
tail (the window - 1 rows before each row's length, tail(layer) gathers it)
with no copy per step, and undo, which only restores the lengths, cuts it
back as carry.Tail.undo does (rows past a length are written again before
any query reads them).

A sparse layer carries nothing (it reads the exact layer's table before it)
and has no table: its entry in `tables` is None.

Each exact layer's entries live in one (B, capacity, 2c) table, keys first, token p
of row b at row p.  A reading appends each row's own new entries at its own
length (wptv_kv_append) and returns nothing to copy: the attention reads the
table in place up to each query's position.  Undo restores the lengths from
before the undoable reading plus kept; the entries past a row's length are
never read, and are written again when the row reaches them.

The lengths stay on the device; `bound` is a host-side upper bound of every
row's length (raised by each reading's width, never lowered by undo) so that
growing the tables needs no host synchronization.  The tables grow to
max(need, 2 x capacity) as the reference's do, by a copy; a HIP graph of a
step is captured with the capacity reserved beforehand.
"""

import torch

from . import _lib
from ._lib import check, ptr


def _lengths(lengths, before, counts, undo):
    """wptv_cache_lengths on the lengths' device: before = lengths (when
    given), lengths += counts; or, undo, lengths = before + counts."""
    if counts.device != lengths.device or counts.shape != lengths.shape or counts.dtype not in _lib.INDEX_DTYPES:
        raise ValueError(f"counts must be ({lengths.shape[0]},) int64 or int32 on {lengths.device}")
    counts = counts.contiguous()
    check(_lib.lib().wptv_cache_lengths(ptr(lengths), ptr(before), ptr(counts), _lib.INDEX_DTYPES[counts.dtype],
                                        lengths.shape[0], int(undo), _lib.stream(lengths.device)), "cache_lengths")


class Cache:
    """rings: the layers whose table is a ring of ring_rows rows (window
    layers); bare: the layers with no table (sparse layers); every other
    layer's table grows with the text."""

    def __init__(self, rows, layers, width, dtype, device, capacity=256, rings=(), ring_rows=256, bare=()):
        if ring_rows <= 0 or ring_rows & (ring_rows - 1):
            raise ValueError(f"a ring holds a power of 2 of rows, not {ring_rows}")
        self.lengths = torch.zeros(rows, dtype=torch.long, device=device)
        self.before = torch.zeros_like(self.lengths)  # the lengths before the last undoable reading
        self.rings = frozenset(rings)
        self.tables = [None if i in bare else
                       torch.zeros(rows, ring_rows if i in self.rings else capacity, width, dtype=dtype, device=device)
                       for i in range(layers)]
        self.pending = False
        self.bound = 0
        self.routes = None

    @property
    def rows(self):
        return self.lengths.shape[0]

    @property
    def capacity(self):
        grown = [t.shape[1] for i, t in enumerate(self.tables) if t is not None and i not in self.rings]
        return grown[0] if grown else None

    @property
    def ring_rows(self):
        rings = [self.tables[i].shape[1] for i in sorted(self.rings)]
        return rings[0] if rings else None

    def reserve(self, need):
        """Growing tables of at least `need` rows (grown to max(need, 2 x
        capacity)); the rings keep their size."""
        if self.capacity is None or need <= self.capacity:
            return
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"the cache needs {need} rows but holds {self.capacity}: reserve them before "
                               "capturing a step")
        grown = max(need, 2 * self.capacity)
        self.tables = [t if t is None or i in self.rings else torch.cat([t, t.new_zeros(t.shape[0], grown - t.shape[1],
                                                                           t.shape[2])], 1)
                       for i, t in enumerate(self.tables)]

    def tail(self, layer, steps):
        """A window layer's carried tail (B, steps, width): the entries of the
        steps tokens before each row's length, zeros before the text (the
        reference's Reading.before, cache.py:97-108)."""
        if layer not in self.rings:
            raise ValueError(f"layer {layer} keeps every entry, not a tail")
        ring = self.tables[layer]
        R = ring.shape[1]
        if steps > R:
            raise ValueError(f"the ring holds {R} rows, fewer than {steps}")
        positions = self.lengths[:, None] - steps + torch.arange(steps, device=ring.device)
        rows = ring.gather(1, (positions % R)[..., None].expand(-1, -1, ring.shape[2]))
        return rows.masked_fill((positions < 0)[..., None], 0)

    def finish(self, counts, undoable, width):
        """The rows have read their tokens (the reference's Reading.finish).
        The lengths change in place, so that a captured step replays on the
        cache's current state."""
        _lengths(self.lengths, self.before if undoable else None, counts, undo=False)
        self.pending = bool(undoable)
        self.bound += width

    def undo(self, kept):
        """Back to the lengths before the last undoable reading, plus kept."""
        if not self.pending:
            raise ValueError("no undoable extend to undo")
        _lengths(self.lengths, self.before, kept, undo=True)
        self.pending = False

    def undo_on_device(self):
        """The lengths and the lengths before the last undoable reading, for a
        kernel that applies the undo itself (the sampler's commit); the
        reading counts as undone from here on."""
        if not self.pending:
            raise ValueError("no undoable extend to undo")
        self.pending = False
        return self.lengths, self.before

    def select(self, index):
        """A new cache of the rows index names (a row may come several times),
        copied (the reference's Cache.select, cache.py:157-166)."""
        if self.pending:
            raise ValueError("an undoable extend is pending: undo it before copying rows")
        index = torch.as_tensor(index, dtype=torch.long, device=self.lengths.device)
        copy = object.__new__(Cache)
        copy.lengths = self.lengths[index]
        copy.before = torch.zeros_like(copy.lengths)
        copy.tables = [None if t is None else t[index] for t in self.tables]
        copy.rings = self.rings
        copy.pending, copy.bound, copy.routes = False, self.bound, None
        return copy
