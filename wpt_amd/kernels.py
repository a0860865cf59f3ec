"""The HIP form of the attention operations of the verify step, with the
reference's kernel-module contract (NAME, exact_attention, sparse_attention:
packages/wpt-model/src/wpt_model/pytorch_kernels.py:18-26, dispatched by
kernels.py:160-184), plus the tree-masked and general forms the contract has
no name for (verify_attention, tree_attention).

Contract, as the reference states it: q (B, T, H, c) and the table's k and v
(B, N, c) in one dtype, token p at row p, k and v possibly the strided
halves of one (B, N, 2c) entries table; positions (B, T) int64, each query's
position, a padding query past the table reading up to its last row; sink
(H,) FP32; indices (B, T, K) int64, -1 for none.  Outputs are in q's dtype,
scores and softmax in FP32.

These forms are forward-only: the verify step runs under torch.no_grad
(wpt_model.WPT.extend, model.py:456).  Their backward raises
NotImplementedError, which the reference's kernel tests read as "not
written yet" (test_kernels.py:149-154).
A bad shape or dtype is ValueError; a device without the library is
KernelUnavailable, never a fall back to another form.
"""

import torch

from . import _lib
from ._lib import KernelUnavailable, check, ptr

NAME = "HIP (gfx950)"

__all__ = ["NAME", "KernelUnavailable", "chosen_columns", "exact_attention", "choose_rows", "sparse_attention",
           "verify_attention", "window_attention", "ring_attention", "tree_attention", "tree_ancestors", "kv_append"]


def chosen_columns(top_k, window, N):
    """The columns of the chosen rows for a table of N rows: top_k, or the
    rows at least window tokens before the table's last when fewer
    (pytorch_kernels.py:73-77)."""
    return max(0, min(top_k, N - window))


class _ForwardOnly(torch.autograd.Function):
    """Carries a forward result; its backward is not written."""

    @staticmethod
    def forward(ctx, out, *inputs):
        return out

    @staticmethod
    def backward(ctx, grad):
        raise NotImplementedError("the HIP attention forms are forward-only (the verify step runs under no_grad)")


def _forward_only(out, *inputs):
    if torch.is_grad_enabled() and any(x is not None and x.requires_grad for x in inputs):
        return _ForwardOnly.apply(out, *[x for x in inputs if x is not None])
    return out


def _check_inputs(q, k, v, positions):
    if q.dim() != 4 or k.dim() != 3 or v.dim() != 3:
        raise ValueError(f"q must be (B, T, H, c) and k, v (B, N, c); got {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    B, T, H, c = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[2] != c:
        raise ValueError(f"k and v must be (B={B}, N, c={c}); got {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q, k and v must share one dtype; got {q.dtype}, {k.dtype}, {v.dtype}")
    if not (q.device == k.device == v.device) or q.device.type != "cuda":
        raise KernelUnavailable(f"the HIP attention runs on a GPU; q is on {q.device}")
    if k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("each row of k and v must be contiguous")
    if positions is not None and tuple(positions.shape) != (B, T):
        raise ValueError(f"positions must be (B={B}, T={T}); got {tuple(positions.shape)}")
    if k.shape[1] == 0:
        raise ValueError("the table is empty")
    return B, T, H, c, k.shape[1]


def _long(x, device):
    return x.to(device=device, dtype=torch.long).contiguous()


def verify_attention(q, k, v, positions, scale, *, window=0, sink=None, tree=None, lse=False, splits=0,
                     generic=False, from_positions=False, key_split=False, static_scratch=False, out_fm=False,
                     rows32=False):
    """MQA attention of q (B, T, H, c) over k, v (B, N, c): query t of row b
    sees rows max(0, p - window + 1) .. min(p, N - 1), p = positions[b, t]
    (window 0: from row 0), and with tree = (tree_base (B,), ancestors (T,)
    int64 bit masks) a row r >= tree_base[b] only where bit r - tree_base[b]
    of ancestors[t] is set (positions None with a tree: query t is node t, at
    tree_base[b] + t); sink (H,) joins each head's softmax denominator.
    Returns the output (B, T, H, c) in q's dtype, and with lse=True also the
    (B, T, H) FP32 log-sum-exp.  splits: key-range parts per batch row (0:
    the library chooses); generic: the wave-per-query kernel; from_positions:
    read only the rows the positions reach (a cache table with spare rows);
    key_split: where T*H <= 80, the key-parallel MFMA kernel instead of the
    row-block one; rows32: at head width 128, the row-block kernel on 32-row
    blocks (v_mfma_f32_32x32x16_bf16); static_scratch: the allocation-free entry point
    (wptv_verify_attention_static), whose parts live in the library's own
    device array: no workspace is allocated, and calls overlapping on one
    device race."""
    B, T, H, c, N = _check_inputs(q, k, v, positions)
    device = q.device
    library = _lib.lib()
    dtype = _lib.dtype_code(q.dtype)
    q_ = q.contiguous()
    if positions is None and tree is None:
        raise ValueError("positions are needed unless a tree gives them")
    positions_ = None if positions is None else _long(positions, device)
    if out_fm and (static_scratch or q.dtype != torch.bfloat16):
        raise ValueError("the fm output layout takes bf16 queries and the workspace entry point")
    sink_ = None if sink is None else sink.to(device=device, dtype=torch.float32).contiguous()
    if sink_ is not None and sink_.shape != (H,):
        raise ValueError(f"sink must be (H={H},); got {tuple(sink_.shape)}")
    tree_base = ancestors = None
    if tree is not None:
        tree_base, ancestors = (_long(x, device) for x in tree)
        if tree_base.shape != (B,) or ancestors.shape != (T,):
            raise ValueError(f"tree must be (tree_base (B={B},), ancestors (T={T},))")
    flags = ((_lib.FORCE_GENERIC if generic else 0) | (_lib.RANGE_FROM_POSITIONS if from_positions else 0)
             | (_lib.KEY_SPLIT if key_split else 0) | (_lib.OUT_FM if out_fm else 0)
             | (_lib.ROWS32 if rows32 else 0))
    parts = _lib.ctypes.c_int(int(splits))
    size = _lib.ctypes.c_size_t(0)
    check(library.wptv_attention_workspace(B, T, H, c, N, int(window), dtype, flags, _lib.ctypes.byref(parts),
                                           _lib.ctypes.byref(size)), "verify_attention")
    out = torch.empty_like(q_)
    lse_out = torch.empty(B, T, H, dtype=torch.float32, device=device) if lse else None
    if static_scratch:
        check(library.wptv_verify_attention_static(ptr(q_), ptr(k), k.stride(0), k.stride(1), ptr(v), v.stride(0),
                                                   v.stride(1), dtype, ptr(positions_), int(window), ptr(tree_base),
                                                   ptr(ancestors), ptr(sink_), B, T, H, c, N, float(scale),
                                                   int(splits), flags, ptr(out), ptr(lse_out), _lib.stream(device)),
              "verify_attention_static")
        out = _forward_only(out, q, k, v, sink)
        return (out, lse_out) if lse else out
    workspace = torch.empty(max(1, size.value), dtype=torch.uint8, device=device) if size.value else None
    if out_fm:  # [B T, H c] as the output projection's fm operand (layers.fm_unpack reads it back)
        out = torch.empty(_lib.fm_row_blocks(B * T) * 16 * H * c, dtype=q.dtype, device=device)
    check(library.wptv_verify_attention(ptr(q_), ptr(k), k.stride(0), k.stride(1), ptr(v), v.stride(0), v.stride(1),
                                        dtype, ptr(positions_), int(window), ptr(tree_base), ptr(ancestors),
                                        ptr(sink_), B, T, H, c, N, float(scale), parts.value, flags, ptr(out),
                                        ptr(lse_out), ptr(workspace), size.value, _lib.stream(device)),
          "verify_attention")
    if not out_fm:
        out = _forward_only(out, q, k, v, sink)
    return (out, lse_out) if lse else out


def exact_attention(q, k, v, positions, scale, top_k, window):
    """(output (B, T, H, c), the chosen rows (B, T, K)): every query attends
    to every row up to its position, and chooses the top_k rows it weighs
    most among those at least window tokens back, by their largest
    log-weight over the heads (pytorch_kernels.py:98-121,142-146).  K =
    chosen_columns(top_k, window, N); a query with fewer such rows holds all
    of them, then -1.  The rows are in no particular order (here: those above
    the K-th largest score in row order, then those equal to it)."""
    B, T, H, c, N = _check_inputs(q, k, v, positions)
    K = chosen_columns(top_k, window, N)
    if not K:
        out = verify_attention(q, k, v, positions, scale)
        return out, torch.full((B, T, 0), -1, dtype=torch.long, device=q.device)
    out, lse = verify_attention(q, k, v, positions, scale, lse=True)
    return out, choose_rows(q, k, positions, lse, scale, top_k, window)


def choose_rows(q, k, positions, lse, scale, top_k, window):
    """The exact layer's choice (B, T, K) from the forward pass's lse
    (B, T, H): each query's K = chosen_columns(top_k, window, N) rows among
    0 .. p - window with the largest max_h (q_h . k_n * scale - lse_h), -1
    past a query's candidates (pytorch_kernels.py:112-117)."""
    if q.dim() != 4 or k.dim() != 3:
        raise ValueError(f"q must be (B, T, H, c) and k (B, N, c); got {tuple(q.shape)}, {tuple(k.shape)}")
    B, T, H, c = q.shape
    N = k.shape[1]
    if tuple(lse.shape) != (B, T, H) or lse.dtype != torch.float32:
        raise ValueError(f"lse must be FP32 (B={B}, T={T}, H={H}); got {lse.dtype} {tuple(lse.shape)}")
    if k.shape[0] != B or k.shape[2] != c or k.stride(2) != 1 or k.dtype != q.dtype:
        raise ValueError(f"k must be (B={B}, N, c={c}) in q's dtype with contiguous rows")
    K = chosen_columns(top_k, window, N)
    device = q.device
    chosen = torch.empty(B, T, K, dtype=torch.long, device=device)
    if not K:
        return chosen
    library = _lib.lib()
    size = _lib.ctypes.c_size_t(0)
    check(library.wptv_choice_workspace(B, T, N, _lib.ctypes.byref(size)), "choose_rows")
    workspace = torch.empty(size.value, dtype=torch.uint8, device=device)
    q_ = q.contiguous()
    positions_ = _long(positions, device)
    check(library.wptv_exact_choice(ptr(q_), ptr(k), k.stride(0), k.stride(1), _lib.dtype_code(q.dtype),
                                    ptr(positions_), ptr(lse.contiguous()), B, T, H, c, N, float(scale), int(top_k),
                                    int(window), ptr(chosen), ptr(workspace), size.value, _lib.stream(device)),
          "choose_rows")
    return chosen


def sparse_attention(q, k, v, sink, idx, positions, scale, window, *, gate=None, splits=0):
    """The output (B, T, H, c) of attention over each query's rows idx
    (B, T, K) and its last window tokens, with sink (H,) added to each
    head's denominator (pytorch_kernels.py:149-153,171-187,213-217).  A row
    in both lists counts twice, as the reference's concatenation counts it.
    gate (B, T, >= H*c): the sparse layer's output gate, o * sigmoid(gate)
    (attention.py:128-130).  splits: parts of each query's rows (0: the
    library chooses)."""
    B, T, H, c, N = _check_inputs(q, k, v, positions)
    if idx.dim() != 3 or tuple(idx.shape[:2]) != (B, T):
        raise ValueError(f"idx must be (B={B}, T={T}, K); got {tuple(idx.shape)}")
    if window <= 0:
        raise ValueError(f"the sparse form reads a window of at least one row; got {window}")
    device = q.device
    library = _lib.lib()
    dtype = _lib.dtype_code(q.dtype)
    q_ = q.contiguous()
    idx_ = _long(idx, device)
    positions_ = _long(positions, device)
    sink_ = sink.to(device=device, dtype=torch.float32).contiguous()
    if sink_.shape != (H,):
        raise ValueError(f"sink must be (H={H},); got {tuple(sink_.shape)}")
    gate_stride = 0
    if gate is not None:
        if gate.dtype != q.dtype or gate.shape[:2] != (B, T) or gate.stride(-1) != 1 or \
                gate.stride(0) != T * gate.stride(1) or gate.shape[-1] < H * c:
            raise ValueError(f"gate must be (B={B}, T={T}, >= H*c) in q's dtype, rows one after another")
        gate_stride = gate.stride(1)
    K = idx_.shape[2]
    parts = _lib.ctypes.c_int(int(splits))
    size = _lib.ctypes.c_size_t(0)
    check(library.wptv_sparse_attention_workspace(B, T, H, c, K, int(window), N, dtype, _lib.ctypes.byref(parts),
                                                  _lib.ctypes.byref(size)), "sparse_attention")
    workspace = torch.empty(size.value, dtype=torch.uint8, device=device) if size.value else None
    out = torch.empty_like(q_)
    check(library.wptv_sparse_attention(ptr(q_), ptr(k), k.stride(0), k.stride(1), ptr(v), v.stride(0), v.stride(1),
                                        dtype, ptr(idx_), K, ptr(positions_), int(window), ptr(sink_), ptr(gate),
                                        gate_stride, B, T, H, c, N, float(scale), parts.value, ptr(out), None,
                                        ptr(workspace), size.value, _lib.stream(device)), "sparse_attention")
    return _forward_only(out, q, k, v, sink)


def _window_call(q, k, v, sink, positions, scale, window, row_base, ring_rows, gate, splits=0):
    B, T, H, c = q.shape
    device = q.device
    if not (q.dtype == k.dtype == v.dtype) or k.dim() != 3 or k.shape != v.shape or k.shape[0] != B or \
            k.shape[2] != c:
        raise ValueError(f"k and v must be (B={B}, rows, c={c}) in q's dtype; got {tuple(k.shape)}, {tuple(v.shape)}")
    if q.device.type != "cuda" or k.device != device or v.device != device:
        raise KernelUnavailable(f"the HIP window attention runs on a GPU; q is on {q.device}")
    if k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("each row of k and v must be contiguous")
    if sink.shape != (H,):
        raise ValueError(f"sink must be (H={H},); got {tuple(sink.shape)}")
    positions_ = _long(positions.expand(B, T), device)
    sink_ = sink.to(device=device, dtype=torch.float32).contiguous()
    gate_stride = 0
    if gate is not None:
        if gate.dtype != q.dtype or gate.shape[:2] != (B, T) or gate.stride(-1) != 1 or \
                gate.stride(0) != T * gate.stride(1) or gate.shape[-1] < H * c:
            raise ValueError(f"gate must be (B={B}, T={T}, >= H*c) in q's dtype, rows one after another")
        gate_stride = gate.stride(1)
    library = _lib.lib()
    dtype = _lib.dtype_code(q.dtype)
    parts = _lib.ctypes.c_int(int(splits))
    size = _lib.ctypes.c_size_t(0)
    check(library.wptv_window_attention_workspace(B, T, H, c, int(window), dtype, _lib.ctypes.byref(parts),
                                                  _lib.ctypes.byref(size)), "window_attention")
    workspace = torch.empty(size.value, dtype=torch.uint8, device=device) if size.value else None
    q_ = q.contiguous()
    out = torch.empty_like(q_)
    check(library.wptv_window_attention(ptr(q_), ptr(k), k.stride(0), k.stride(1), ptr(v), v.stride(0), v.stride(1),
                                        dtype, ptr(positions_), ptr(row_base), int(ring_rows), int(window), ptr(sink_),
                                        ptr(gate), gate_stride, B, T, H, c, float(scale), parts.value, ptr(out),
                                        ptr(workspace), size.value, _lib.stream(device)), "window_attention")
    return _forward_only(out, q, k, v, sink)


def window_attention(q, k, v, sink, positions, scale, window=128, gate=None):
    """The reference's window_attention (attention.py:85-107): q (B, T, H, c)
    at positions (T,) or (B, T), consecutive within a row; k, v
    (B, window - 1 + T, c), the window - 1 tokens before the pass's first,
    then its own.  Each query reads the last `window` rows, itself included,
    none before the text, the sink (H,) in each head's denominator.  gate
    (B, T, >= H*c): the output times sigmoid(gate) (attention.py:128-130)."""
    B, T = q.shape[:2]
    if k.dim() != 3 or k.shape[1] != window - 1 + T:
        raise ValueError(f"k must hold window - 1 + T = {window - 1 + T} rows; got {tuple(k.shape)}")
    positions = positions.to(q.device).expand(B, T)
    row_base = _long(positions[:, 0] - (window - 1), q.device)
    return _window_call(q, k, v, sink, positions, scale, window, row_base, k.shape[1], gate)


def ring_attention(q, ring, positions, scale, window, sink, gate=None, splits=0):
    """A window layer's attention over its cache ring (B, R, 2c), R a power
    of 2 of at least window - 1 + T, token n at row n mod R (keys then
    values): window_attention's result from the build's ring cache."""
    c = q.shape[-1]
    return _window_call(q, ring[..., :c], ring[..., c:], sink, positions, scale, window, None, ring.shape[1], gate,
                        splits)


def tree_ancestors(parents):
    """The ancestors-or-self bit masks (M,) int64 of a draft tree given each
    node's parent (parents[0] = -1, parents[i] < i), node i's bit i."""
    masks = []
    for i, parent in enumerate(parents):
        if i >= 64:
            raise ValueError("a draft tree holds at most 64 nodes")
        if i == 0 and parent != -1 or i > 0 and not 0 <= parent < i:
            raise ValueError(f"node {i} has parent {parent}: parents must come before their children")
        masks.append((masks[parent] if parent >= 0 else 0) | (1 << i))
    # two's complement: bit 63 is the sign bit of an int64
    return torch.tensor([m - (1 << 64) if m >= 1 << 63 else m for m in masks], dtype=torch.long)


def tree_attention(q, k, v, tree_base, parents, scale, sink=None, out_fm=False):
    """Attention of the M draft-tree nodes (q (B, M, H, c), node i at table
    row tree_base[b] + i) over the prefix rows before tree_base[b] and over
    the node's ancestors and itself: the reference's dense_attention
    (attention.py:74-82) with the mask "prefix plus ancestors-or-self".
    out_fm: the output as a flat fm operand of B M rows x H c (the lm_head's
    X, layers.linear_fm_wide)."""
    base = tree_base.to(device=q.device, dtype=torch.long)
    key = (tuple(int(p) for p in parents), q.device)
    masks = _TREES.get(key)
    if masks is None:  # made once per tree and device, outside any graph capture
        masks = _TREES[key] = tree_ancestors(parents).to(q.device)
    # node i's position, tree_base[b] + i, is formed by the kernel
    return verify_attention(q, k, v, None, scale, sink=sink, tree=(base, masks), out_fm=out_fm)


_TREES = {}  # (parents, device) -> the ancestors-or-self masks on the device


def kv_append(table, new, start, counts):
    """The in-place KV append of the generation cache (the scatter of the
    reference's Reading.everything, cache.py:110-128): table[b, start[b] + j]
    = new[b, j] for j < counts[b].  table (B, capacity, width) and new
    (B, n, width) share a dtype, each row contiguous; start and counts (B,)
    on the device (no host synchronization).  Rows past the capacity are not
    written: the caller keeps the table large enough."""
    if table.dim() != 3 or new.dim() != 3 or table.shape[0] != new.shape[0] or table.shape[2] != new.shape[2]:
        raise ValueError(f"table (B, capacity, width) and new (B, n, width) do not match: {tuple(table.shape)}, "
                         f"{tuple(new.shape)}")
    if table.dtype != new.dtype:
        raise ValueError(f"table and new must share a dtype; got {table.dtype}, {new.dtype}")
    if table.device.type != "cuda" or new.device != table.device:
        raise KernelUnavailable(f"the HIP KV append runs on a GPU; the table is on {table.device}")
    if table.stride(2) != 1 or new.stride(2) != 1:
        raise ValueError("each row of the table and of new must be contiguous")
    B, n, width = new.shape
    start_ = _long(start, table.device)
    counts_ = _long(counts, table.device)
    if start_.shape != (B,) or counts_.shape != (B,):
        raise ValueError(f"start and counts must be (B={B},)")
    check(_lib.lib().wptv_kv_append(ptr(table), table.stride(0), table.stride(1), table.shape[1], ptr(new),
                                    new.stride(0), new.stride(1), ptr(start_), ptr(counts_), B, n, width,
                                    _lib.dtype_code(table.dtype), _lib.stream(table.device)), "kv_append")
    return table
