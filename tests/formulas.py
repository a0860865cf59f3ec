"""Brute-force formulas, one query at a time, that pin the oracle's attention
(the reference states the same two in
packages/wpt-model/tests/test_kernels.py:23-54), and the inputs its kernel
tests draw (test_kernels.py:57-67)."""

import torch


def exact_by_formula(q, k, v, positions, scale):
    """Softmax over rows 0 .. min(p, N - 1) of each query, in FP64."""
    B, T, H, c = q.shape
    N = k.shape[1]
    out = torch.zeros(B, T, H, c, dtype=torch.float64)
    for b in range(B):
        for t in range(T):
            p = min(int(positions[b, t]), N - 1)
            weights = torch.softmax((q[b, t].double() @ k[b, :p + 1].double().T) * scale, -1)
            out[b, t] = weights @ v[b, :p + 1].double()
    return out


def choice_by_formula(q, k, positions, scale, top_k, window):
    """The set of rows each query chooses (the reference's exact_by_formula,
    test_kernels.py:23-40): the top_k rows among 0 .. p - window by their
    largest softmax weight over the heads, in FP64; all of them when fewer."""
    B, T, H, c = q.shape
    N = k.shape[1]
    chosen = [[set() for _ in range(T)] for _ in range(B)]
    for b in range(B):
        for t in range(T):
            p = min(int(positions[b, t]), N - 1)
            weights = torch.softmax((q[b, t].double() @ k[b, :p + 1].double().T) * scale, -1)  # (H, p + 1)
            far = min(int(positions[b, t]) + 1 - window, N)
            if far > 0:
                score = weights[:, :far].amax(0)
                chosen[b][t] = set(score.topk(min(top_k, far)).indices.tolist())
    return chosen


def choice_scores(q, k, positions, scale, window):
    """(B, T, N) FP64: each row's largest log-weight over the heads for each
    query, -inf at rows that are not candidates (n > p - window)."""
    B, T, H, c = q.shape
    N = k.shape[1]
    z = torch.einsum("bthc,bnc->bthn", q.double(), k.double()) * scale
    z = z.masked_fill(torch.arange(N) > positions[..., None, None], float("-inf"))
    score = (z - z.logsumexp(-1, keepdim=True)).amax(2)
    return score.masked_fill(torch.arange(N) > positions[..., None] - window, float("-inf"))


def sparse_by_formula(q, k, v, sink, idx, positions, scale, window):
    """Each query over its rows idx and its last window rows (a set: the
    reference's chosen rows never meet its window), each head's sink in the
    denominator, in FP64."""
    B, T, H, c = q.shape
    N = k.shape[1]
    out = torch.zeros(B, T, H, c, dtype=torch.float64)
    for b in range(B):
        for t in range(T):
            p = int(positions[b, t])
            rows = sorted({int(i) for i in idx[b, t] if i >= 0}
                          | set(range(max(0, p - window + 1), min(p, N - 1) + 1)))
            z = (q[b, t].double() @ k[b, rows].double().T) * scale
            denominator = z.exp().sum(-1) + sink.double().exp()
            out[b, t] = (z.exp() / denominator[:, None]) @ v[b, rows].double()
    return out


def tree_by_formula(q, k, v, prefix, parents, scale):
    """Node i of each row over the prefix rows and the rows of its ancestors
    and itself, found by walking up the parents, in FP64."""
    B, M, H, c = q.shape
    out = torch.zeros(B, M, H, c, dtype=torch.float64)
    for b in range(B):
        for i in range(M):
            rows, node = list(range(int(prefix[b]))), i
            while node >= 0:
                rows.append(int(prefix[b]) + node)
                node = parents[node]
            weights = torch.softmax((q[b, i].double() @ k[b, rows].double().T) * scale, -1)
            out[b, i] = weights @ v[b, rows].double()
    return out


def inputs(B=2, T=40, H=3, c=16, N=None, seed=0, dtype=torch.float32):
    """q (B, T, H, c), k and v (B, N, c), sink (H,) and the positions of a pass
    whose T queries are the table's last ones, drawn on the CPU from one
    seeded generator as the reference's tests draw them."""
    generator = torch.Generator().manual_seed(seed)
    N = N or T

    def rand(*shape):
        return torch.randn(*shape, generator=generator).to(dtype)

    positions = (N - T + torch.arange(T)).expand(B, T).contiguous()
    return rand(B, T, H, c), rand(B, N, c), rand(B, N, c), rand(H), positions


def relative_error(got, expected):
    """The largest difference as a share of the expected values' largest
    magnitude (the reference's measure, test_kernels.py:143-146)."""
    return float((got.double() - expected.double()).abs().max() / expected.double().abs().max())
