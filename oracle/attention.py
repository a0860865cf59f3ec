"""Oracle attention: the reference's PyTorch form, restated in FP32 on the
CPU (test infrastructure; see oracle/__init__.py).

    exact_attention   pytorch_kernels.py:98-121 (_Exact.forward) and :142-146;
                      the block loop of :48-63, the scores of :66-70, the
                      choice of :112-117
    sparse_attention  pytorch_kernels.py:149-153 (_window), :156-161
                      (_gather), :171-187 (_Sparse.forward), :213-217
    dense_attention   attention.py:74-82
    window_attention  attention.py:85-107: each query over the last `window`
                      rows of a (B, window - 1 + T) table of the carried tail
                      and the new entries, none before the text, with a sink
    rotate            attention.py:59-71, the window layers' rotary encoding
    tree_visible      the mask "prefix plus ancestors-or-self" of a draft tree

Forward passes only: the verify step runs under no_grad.
"""

import torch

BLOCK_VALUES = 1 << 24  # values per block of queries, as pytorch_kernels.py:45


def _rows(batch, *sizes):
    """Queries per block so that one block's largest tensor holds about
    BLOCK_VALUES values (pytorch_kernels.py:48-53)."""
    values = batch
    for size in sizes:
        values *= max(1, size)
    return max(1, BLOCK_VALUES // values)


def chosen_columns(top_k, window, N):
    """pytorch_kernels.py:73-77."""
    return max(0, min(top_k, N - window))


def exact_attention(q, k, v, positions, scale, top_k, window):
    """(output (B, T, H, c) in q's dtype, chosen (B, T, K) int64).  Query at
    position p reads rows 0 .. min(p, N - 1); FP32 scores and softmax."""
    B, T, H, c = q.shape
    dtype = q.dtype
    q, k, v = q.float(), k.float(), v.float()
    N = k.shape[1]
    out = q.new_empty(B, T, H, c)
    K = chosen_columns(top_k, window, N)
    chosen = torch.full((B, T, K), -1, dtype=torch.long)
    ends = positions.amax(0)
    rows = _rows(B, H, N)
    for start in range(0, T, rows):
        part = slice(start, start + rows)
        seen = min(int(ends[part].max()) + 1, N)
        z = torch.einsum("brhc,bnc->brhn", q[:, part], k[:, :seen]) * scale
        later = torch.arange(seen) > positions[:, part, None]
        z = z.masked_fill(later[:, :, None], float("-inf"))
        lse = torch.logsumexp(z, -1)
        log_p = z - lse[..., None]
        out[:, part] = torch.einsum("brhn,bnc->brhc", log_p.exp(), v[:, :seen])
        if K:
            score = log_p.amax(2)
            near = torch.arange(seen) > positions[:, part, None] - window
            score = score.masked_fill(near, float("-inf"))
            best, index = score.topk(min(K, seen), -1)
            chosen[:, part, :index.shape[-1]] = index.masked_fill(best == float("-inf"), -1)
    return out.to(dtype), chosen


def window_rows(positions, window, N):
    """(B, T, window): each query's last window rows, -1 before the text and
    past the table (pytorch_kernels.py:149-153)."""
    rows = positions[..., None] - window + 1 + torch.arange(window)
    return rows.masked_fill((rows < 0) | (rows >= N), -1)


def _gather(table, idx):
    B, N, c = table.shape
    flat = idx.clamp(min=0) + torch.arange(B)[:, None, None] * N
    return table.reshape(B * N, c)[flat]


def sparse_attention(q, k, v, sink, idx, positions, scale, window):
    """The output over each query's rows idx and its last window rows, the
    sink (H,) in each head's denominator; a row in both lists counts twice."""
    B, T, H, c = q.shape
    dtype = q.dtype
    rows_all = torch.cat([idx, window_rows(positions, window, k.shape[1])], -1)
    q, k, v, sink = q.float(), k.float(), v.float(), sink.float()
    out = q.new_empty(B, T, H, c)
    rows = _rows(B, rows_all.shape[-1], max(c, H))
    for start in range(0, T, rows):
        part = slice(start, start + rows)
        z = torch.einsum("brhc,brkc->brhk", q[:, part], _gather(k, rows_all[:, part])) * scale
        z = z.masked_fill(rows_all[:, part, None, :] < 0, float("-inf"))
        lse = torch.logaddexp(torch.logsumexp(z, -1), sink)
        out[:, part] = torch.einsum("brhk,brkc->brhc", (z - lse[..., None]).exp(), _gather(v, rows_all[:, part]))
    return out.to(dtype)


def dense_attention(q, k, v, sink, visible, scale):
    """Attention of q (..., Q, H, c) over k, v (..., K, c) under the mask
    visible (..., Q, K), sink (H,) in each head's denominator: (..., Q, H, c)
    in FP32 (attention.py:74-82 computes the product with v in v's dtype;
    the oracle keeps FP32 throughout)."""
    z = torch.einsum("...qhc,...kc->...hqk", q.float(), k.float()) * scale
    z = z.masked_fill(~visible[..., None, :, :], float("-inf"))
    lse = torch.logaddexp(torch.logsumexp(z, -1), sink.float()[:, None])
    return torch.einsum("...hqk,...kc->...qhc", (z - lse[..., None]).exp(), v.float())


ROPE_DIMS = 64  # attention.py:55-56
ROPE_BASE = 10000


def rotate(x, positions, dims=ROPE_DIMS, base=ROPE_BASE):
    """Rotary encoding of the last `dims` dimensions of x (B, T, d) or
    (B, T, H, d) at positions (T,) or (B, T): adjacent pairs (2i, 2i + 1)
    turned by the angle p / base^(2i / dims), computed in FP32 from x's values
    and returned in x's dtype, the other dimensions untouched."""
    pairs = torch.arange(dims // 2, dtype=torch.float32)
    angles = positions.float()[..., None] / base ** (2 * pairs / dims)
    cos, sin = angles.cos(), angles.sin()
    if x.ndim == 4:
        cos, sin = cos[..., None, :], sin[..., None, :]
    kept, turning = x[..., :-dims], x[..., -dims:].float()
    even, odd = turning[..., 0::2], turning[..., 1::2]
    turned = torch.stack([even * cos - odd * sin, even * sin + odd * cos], -1).flatten(-2)
    return torch.cat([kept, turned.to(x.dtype)], -1)


def window_visible(positions, window, T):
    """(B, T, window - 1 + T) bool: query t (its own entry at table row
    window - 1 + t) sees the rows window - 1 + t - d for distances
    0 <= d < window with d <= its position (nothing before the text)."""
    rows = torch.arange(window - 1 + T)
    distance = (window - 1 + torch.arange(T))[:, None] - rows  # (T, rows)
    return (distance >= 0) & (distance < window) & (distance <= positions[..., None])


def window_attention(q, k, v, sink, positions, scale, window):
    """q (B, T, H, c) at positions (B, T); k, v (B, window - 1 + T, c): the
    window - 1 rows before the pass's first token, then its own.  Output
    (B, T, H, c) in FP32 (scores and softmax in FP32, the sink (H,) in each
    head's denominator)."""
    B, T = q.shape[:2]
    positions = positions.expand(B, T)
    return dense_attention(q, k, v, sink, window_visible(positions, window, T), scale)


def binary_tree_parents(nodes):
    """A complete binary draft tree in breadth-first order: node i's parent
    is (i - 1) // 2, the root's -1."""
    return [-1] + [(i - 1) // 2 for i in range(1, nodes)]


def tree_visible(parents, prefix, N):
    """(M, N) bool: node i (at row prefix + i) sees rows 0 .. prefix - 1 and
    the rows of its ancestors and itself."""
    M = len(parents)
    visible = torch.zeros(M, N, dtype=torch.bool)
    visible[:, :prefix] = True
    for i in range(M):
        node = i
        while node >= 0:
            visible[i, prefix + node] = True
            node = parents[node]
    return visible


def tree_attention(q, k, v, prefix, parents, scale, sink=None):
    """q (B, M, H, c) of the M tree nodes at rows prefix[b] + i of k, v
    (B, N, c): dense_attention under tree_visible, one batch row at a time.
    Output in q's dtype."""
    B, M, H, c = q.shape
    N = k.shape[1]
    sink = torch.full((H,), float("-inf")) if sink is None else sink
    out = torch.empty(B, M, H, c)
    for b in range(B):
        visible = tree_visible(parents, int(prefix[b]), N)
        out[b] = dense_attention(q[b], k[b], v[b], sink, visible, scale)
    return out.to(q.dtype)
