"""The generation cache of the MQA decoder on the GPU: the reference's Rows /
Reading / Cache (packages/wpt-model/src/wpt_model/cache.py:54-174) for exact
layers, whose carried value is every token's key and value side by side
(carry.Entries, carry.py:66-71).

Each layer's entries live in one (B, capacity, 2c) table, keys first, token p
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


class Cache:
    def __init__(self, rows, layers, width, dtype, device, capacity=256):
        self.lengths = torch.zeros(rows, dtype=torch.long, device=device)
        self.before = torch.zeros_like(self.lengths)  # the lengths before the last undoable reading
        self.tables = [torch.zeros(rows, capacity, width, dtype=dtype, device=device) for _ in range(layers)]
        self.pending = False
        self.bound = 0
        self.routes = None

    @property
    def rows(self):
        return self.lengths.shape[0]

    @property
    def capacity(self):
        return self.tables[0].shape[1] if self.tables else 0

    def reserve(self, need):
        """Tables of at least `need` rows (grown to max(need, 2 x capacity))."""
        if need <= self.capacity:
            return
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"the cache needs {need} rows but holds {self.capacity}: reserve them before "
                               "capturing a step")
        grown = max(need, 2 * self.capacity)
        self.tables = [torch.cat([t, t.new_zeros(t.shape[0], grown - t.shape[1], t.shape[2])], 1)
                       for t in self.tables]

    def finish(self, counts, undoable, width):
        """The rows have read their tokens (the reference's Reading.finish).
        The lengths change in place, so that a captured step replays on the
        cache's current state."""
        if undoable:
            self.before.copy_(self.lengths)
        self.pending = bool(undoable)
        self.lengths.add_(counts)
        self.bound += width

    def undo(self, kept):
        """Back to the lengths before the last undoable reading, plus kept."""
        if not self.pending:
            raise ValueError("no undoable extend to undo")
        torch.add(self.before, kept, out=self.lengths)
        self.pending = False

    def select(self, index):
        """A new cache of the rows index names (a row may come several times),
        copied (the reference's Cache.select, cache.py:157-166)."""
        if self.pending:
            raise ValueError("an undoable extend is pending: undo it before copying rows")
        index = torch.as_tensor(index, dtype=torch.long, device=self.lengths.device)
        copy = object.__new__(Cache)
        copy.lengths = self.lengths[index]
        copy.before = torch.zeros_like(copy.lengths)
        copy.tables = [t[index] for t in self.tables]
        copy.pending, copy.bound, copy.routes = False, self.bound, None
        return copy
