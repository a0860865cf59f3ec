"""Oracle generation cache: the reference's Rows / Reading for the entries of
exact layers and the tails of window layers, restated on the CPU (test
infrastructure; see oracle/__init__.py).

    Rows.reading / Rows.undo      cache.py:54-77
    Reading.everything            cache.py:110-128: row b's j-th new entry is
                                  written at lengths[b] + j for j < counts[b];
                                  the table grows to max(need, 2 x capacity)
                                  and the call returns its first `need` rows
    Reading.before (tails)        cache.py:97-108 with carry.Tail.undo and
                                  carry.last (carry.py:60-63, 120-124)
    Reading.finish                cache.py:130-134
Undo restores the lengths from before the reading plus kept; entries are left
as they are (one past a row's tokens is never read, and is written again when
the row reaches it: carry.py:66-71); tails are cut back.
"""

import torch


def last(rows, counts, size):
    """rows (B, size + n, ...) -> (B, size, ...): for row b, the size rows
    that end where its first counts[b] rows after the first size end."""
    index = counts[:, None] + torch.arange(size)
    return rows[torch.arange(len(rows))[:, None], index]


class Rows:
    def __init__(self, rows):
        self.lengths = torch.zeros(rows, dtype=torch.long)
        self.values = {}
        self.pending = None

    def reading(self, counts, undoable):
        return Reading(self, torch.as_tensor(counts, dtype=torch.long), undoable)

    def undo(self, kept):
        if self.pending is None:
            raise ValueError("no undoable extend to undo")
        kept = torch.as_tensor(kept, dtype=torch.long)
        lengths, saved = self.pending
        for key, (steps, before, new) in saved.items():
            self.values[key] = last(torch.cat([before, new], 1), kept, steps)
        self.lengths, self.pending = lengths + kept, None

    def select(self, index):
        if self.pending is not None:
            raise ValueError("an undoable extend is pending: undo it before copying rows")
        index = torch.as_tensor(index, dtype=torch.long)
        copy = Rows(len(index))
        copy.lengths = self.lengths[index]
        copy.values = {key: value[index].clone() for key, value in self.values.items()}
        return copy


class Reading:
    def __init__(self, rows, counts, undoable):
        self.rows, self.counts = rows, counts
        self.start = rows.lengths
        self.saved = {} if undoable else None

    def everything(self, key, new):
        first, made = self.start, self.counts
        need = int((first + made).max())
        held = self.rows.values.get(key)
        if held is None:
            held = new.new_zeros(len(first), 0, *new.shape[2:])
        if need > held.shape[1]:
            grown = max(need, 2 * held.shape[1])
            held = torch.cat([held, held.new_zeros(len(first), grown - held.shape[1], *held.shape[2:])], 1)
        row, j = (torch.arange(new.shape[1])[None] < made[:, None]).nonzero(as_tuple=True)
        held = held.to(new.dtype)
        held[row, first[row] + j] = new[row, j]
        self.rows.values[key] = held
        return held[:, :need]

    def before(self, key, steps, x):
        """A tail of `steps` rows: what came before x (zeros before the text);
        what each row's own tokens leave is kept."""
        earlier = self.rows.values.get(key)
        if earlier is None:
            earlier = x.new_zeros(x.shape[0], steps, *x.shape[2:])
        earlier = earlier.to(x.dtype)
        self.rows.values[key] = last(torch.cat([earlier, x], 1), self.counts, steps)
        if self.saved is not None:
            self.saved[key] = (steps, earlier, x)
        return earlier

    def positions(self, T):
        return self.start[:, None] + torch.arange(T)

    def finish(self):
        rows = self.rows
        rows.pending = (rows.lengths, self.saved) if self.saved is not None else None
        rows.lengths = rows.lengths + self.counts
