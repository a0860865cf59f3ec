"""The acceptance step of speculative decoding on the GPU (libwptv's
wptv_accept / wptv_greedy_tree): the reference's sampling distribution
(Writer._probabilities, packages/wpt-inference/src/wpt_inference/__init__.py:
173-179) and keep / reject / resample loop (Writer._speculate, :210-229) for
every row in two kernel launches and no host synchronization.

The reference draws lazily from a torch generator, one uniform per draft it
looks at and one multinomial per row.  `accept_in_order` draws exactly
those, in that order, from a torch generator on the GPU (its Philox stream
replayed on the device: `generator_state` hands the generator over,
`set_offset` moves it past what was drawn), so a seeded generator writes
the reference's tokens.  `accept` reads a tape drawn up front instead,
`draws(B, L, V)`: u (B, L) uniforms, the one for draft j of row b, and e
(B, V) Exp(1) values, the multinomial draw of row b being argmax_v w_v / e_v
(the exponential race torch's multinomial runs for one sample).  A tape
built from what a lazy run drew replays it exactly.
"""

import torch

from . import _lib
from ._lib import KernelUnavailable, check, ptr

__all__ = ["accept", "accept_in_order", "generator_state", "set_offset", "greedy_chain", "greedy_tree",
           "greedy_tree_from_argmax", "draws", "written"]


def _on_gpu(*tensors):
    for x in tensors:
        if x is not None and x.device.type != "cuda":
            raise KernelUnavailable(f"the HIP sampler runs on a GPU; a tensor is on {x.device}")


def _rows_last_contiguous(x, name, dims):
    if x.dim() != dims:
        raise ValueError(f"{name} must have {dims} dimensions; got {tuple(x.shape)}")
    if x.dtype != torch.float32:
        raise ValueError(f"{name} must be float32; got {x.dtype}")
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x


def _scores(x):
    """The scores as the kernels take them: (B, positions, V), FP32 or bf16
    (the lm_head's logits, read as their exact FP32 values), rows contiguous."""
    if x.dim() != 3:
        raise ValueError(f"scores must have 3 dimensions; got {tuple(x.shape)}")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"scores must be float32 or bfloat16; got {x.dtype}")
    if x.stride(-1) != 1:
        x = x.contiguous()
    return x


def _workspace(device, B, L):
    size = _lib.ctypes.c_size_t(0)
    check(_lib.lib().wptv_accept_workspace(B, L, _lib.ctypes.byref(size)), "accept")
    return torch.empty(size.value, dtype=torch.uint8, device=device), size.value


def draws(B, L, V, generator=None, device="cuda"):
    """A tape for one step: (u (B, L) uniforms in [0, 1), e (B, V) Exp(1))."""
    u = torch.rand(B, L, generator=generator, device=device)
    e = torch.empty(B, V, device=device).exponential_(generator=generator)
    return u, e


def _inputs(scores, q, drafts, lengths, firsts, greedy, temperature):
    """The acceptance inputs checked and laid out as the kernels read them:
    (scores, q, drafts, lengths, firsts) and (B, L, V)."""
    scores = _scores(scores)
    B, _, V = scores.shape
    if drafts is None:
        drafts = torch.empty(B, 0, dtype=torch.long, device=scores.device)
    if drafts.dim() != 2 or drafts.shape[0] != B:
        raise ValueError(f"drafts must be (B={B}, L); got {tuple(drafts.shape)}")
    L = drafts.shape[1]
    device = scores.device
    drafts = drafts.to(device=device, dtype=torch.long)
    if drafts.stride(1) != 1:  # rows of drafts are read with their own stride
        drafts = drafts.contiguous()
    if not greedy:
        if L > 0 or q is not None:
            q = _rows_last_contiguous(q, "q", 3)
            if q.shape != (B, L, V):
                raise ValueError(f"q must be (B={B}, L={L}, V={V}); got {tuple(q.shape)}")
        if not temperature > 0:
            raise ValueError(f"the temperature must be positive; got {temperature}")
    else:
        q = None
    lengths_ = None if lengths is None else torch.as_tensor(lengths, dtype=torch.int32, device=device).contiguous()
    firsts_ = None if firsts is None else torch.as_tensor(firsts, dtype=torch.int32, device=device).contiguous()
    host_lengths = torch.full((B,), L) if lengths is None else torch.as_tensor(lengths).cpu().long()
    host_firsts = torch.zeros(B, dtype=torch.long) if firsts is None else torch.as_tensor(firsts).cpu().long()
    if host_lengths.shape != (B,) or host_firsts.shape != (B,):
        raise ValueError(f"lengths and firsts must be (B={B},)")
    if (host_lengths < 0).any() or (host_lengths > L).any() or (host_firsts < 0).any():
        raise ValueError(f"lengths must lie in [0, {L}] and firsts be non-negative")
    need = int((host_firsts + host_lengths).max()) + 1
    if scores.shape[1] < need:
        raise ValueError(f"scores hold {scores.shape[1]} positions per row; {need} are read")
    return (scores, q, drafts, lengths_, firsts_), (B, L, V)


def _commit(commit, B, device):
    """The pointers of a commit (cache_lengths, cache_before, feeds, failed,
    written), checked; five NULLs and a zero stride for none."""
    if commit is None:
        return (None, None, None, 0, None, None)
    cache_lengths, cache_before, feeds, failed, written = commit
    for name, t in (("cache_lengths", cache_lengths), ("cache_before", cache_before)):
        if t.dtype != torch.int64 or t.shape != (B,) or not t.is_contiguous() or t.device != device:
            raise ValueError(f"{name} must be a contiguous ({B},) int64 tensor on {device}")
    if feeds.dtype != torch.int64 or feeds.shape[0] != B or feeds.device != device:
        raise ValueError(f"feeds must be ({B}, n) int64 on {device}")
    if failed is not None and (failed.dtype != torch.int32 or failed.numel() < 1 or failed.device != device):
        raise ValueError("failed must be an int32 device tensor")
    if written is not None and (written.dtype != torch.int64 or written.shape != (B,) or not written.is_contiguous()
                                or written.device != device):
        raise ValueError(f"written must be a contiguous ({B},) int64 tensor on {device}")
    return (ptr(cache_lengths), ptr(cache_before), ptr(feeds), feeds.stride(0), ptr(failed), ptr(written))


def accept(scores, q, drafts, u, e, temperature=0.8, top_k=40, lengths=None, firsts=None, greedy=False,
           commit=None):
    """Each row's written tokens: (tokens (B, L + 1) int64, -1 past a row's
    count; counts (B,) int32 = kept drafts + 1).

    scores (B, >= L + 1, V) FP32 or bf16: row b's position j is scores[b, firsts[b] + j]
    (firsts None: 0); q (B, L, V) FP32 the drafts' distributions; drafts (B, L)
    int64; u, e the tape (draws); lengths (B,) the drafts each row verifies
    (None: L).  greedy: keep the drafts equal to the argmax (q, u, e unused).

    commit (cache_lengths, cache_before, feeds, failed, written): the verify
    step's next moves in the same launch as the pick (wptv_accept_commit):
    cache_lengths = cache_before + counts (the undo), feeds[:, 0] = each
    row's last written token (a row with none keeps it and sets failed),
    written += counts; failed and written may be None."""
    (scores, q, drafts, lengths_, firsts_), (B, L, V) = _inputs(scores, q, drafts, lengths, firsts, greedy,
                                                                 temperature)
    device = scores.device
    if not greedy:
        if q is None:
            q = torch.empty(B, L, V, device=device)
        u = u.to(device=device, dtype=torch.float32).contiguous()
        e = e.to(device=device, dtype=torch.float32).contiguous()
        if u.shape != (B, L) or e.shape != (B, V):
            raise ValueError(f"the tape must be u (B={B}, L={L}) and e (B={B}, V={V}); got {tuple(u.shape)}, "
                             f"{tuple(e.shape)}")
    else:
        u = e = None
    _on_gpu(scores, q, drafts, u, e)
    tokens = torch.empty(B, L + 1, dtype=torch.long, device=device)
    counts = torch.empty(B, dtype=torch.int32, device=device)
    workspace, size = _workspace(device, B, L)
    args = (ptr(scores), scores.stride(0), scores.stride(1), _lib.dtype_code(scores.dtype), ptr(firsts_), ptr(q),
            q.stride(0) if q is not None else 0, q.stride(1) if q is not None else 0, ptr(drafts), drafts.stride(0),
            ptr(lengths_), ptr(u), ptr(e), float(temperature), 0 if top_k is None else int(top_k),
            1 if greedy else 0, B, L, V, ptr(tokens), ptr(counts), ptr(workspace), size)
    if commit is None:
        check(_lib.lib().wptv_accept(*args, _lib.stream(device)), "accept")
        return tokens, counts
    check(_lib.lib().wptv_accept_commit(*args, *_commit(commit, B, device), _lib.stream(device)), "accept_commit")
    return tokens, counts


def accept_in_order(scores, q, drafts, state, temperature=0.8, top_k=40, lengths=None, firsts=None, joint=False,
                    commit=None):
    """accept, drawing what the reference's loop draws from a torch generator
    on the GPU, in its order (wptv_accept_in_order): state is the generator's
    [seed, offset] as generator_state gives it (int64 on the device), its
    offset moved past this call's draws on the device.  joint (no drafts):
    one multinomial over all rows at once, as the reference's Writer._sample
    draws; otherwise one per row."""
    (scores, q, drafts, lengths_, firsts_), (B, L, V) = _inputs(scores, q, drafts, lengths, firsts, False,
                                                                 temperature)
    device = scores.device
    if state.dtype != torch.int64 or state.shape != (2,) or state.device != device or not state.is_contiguous():
        raise ValueError(f"state must be the generator's [seed, offset] as a contiguous (2,) int64 tensor on {device}")
    if joint and L:
        raise ValueError("a joint draw takes no drafts")
    _on_gpu(scores, q, drafts, state)
    tokens = torch.empty(B, L + 1, dtype=torch.long, device=device)
    counts = torch.empty(B, dtype=torch.int32, device=device)
    workspace, size = _workspace(device, B, L)
    check(_lib.lib().wptv_accept_in_order(
        ptr(scores), scores.stride(0), scores.stride(1), _lib.dtype_code(scores.dtype), ptr(firsts_), ptr(q),
        q.stride(0) if q is not None else 0, q.stride(1) if q is not None else 0, ptr(drafts), drafts.stride(0),
        ptr(lengths_), ptr(state), ptr(state[1:]), 1 if joint else 0, float(temperature),
        0 if top_k is None else int(top_k), B, L, V, ptr(tokens), ptr(counts), ptr(workspace), size,
        *_commit(commit, B, device), _lib.stream(device)), "accept_in_order")
    return tokens, counts


def _generator(generator, device):
    if generator is not None:
        return generator
    device = torch.device(device)
    return torch.cuda.default_generators[device.index if device.index is not None else torch.cuda.current_device()]


def generator_state(generator=None, device="cuda"):
    """A torch generator on the GPU (None: the device's default one) as the
    in-order draws take it: its [seed, offset], int64 on its device."""
    generator = _generator(generator, device)
    if generator.device.type != "cuda":
        raise KernelUnavailable(f"the in-order draws replay a generator on the GPU, not on {generator.device}")
    state = generator.get_state().view(torch.int64)  # torch's device generator: seed, then offset
    return state.to(generator.device)


def set_offset(generator, state, device="cuda"):
    """Moves the generator (None: the device's default one) to the offset in
    state[1] (a host synchronization): its stream continues after what the
    in-order draws drew."""
    generator = _generator(generator, device)
    host = generator.get_state().clone()
    host.view(torch.int64)[1] = int(state[1])
    generator.set_state(host)


def greedy_chain(scores, drafts, lengths=None, firsts=None):
    """Greedy verification: (tokens, counts) as accept, each row keeping the
    longest prefix of drafts equal to the argmax, then the argmax."""
    return accept(scores, None, drafts, None, None, lengths=lengths, firsts=firsts, greedy=True)


def greedy_tree(scores, node_tokens, parents):
    """Greedy verification of a draft tree: scores (B, M, V) FP32 or bf16 at the M
    nodes, node_tokens (B, M), parents (M,) (parents[0] = -1, parents[i] < i).
    Returns (path (B, M + 1) node indices from the root, tokens (B, M + 1)
    written, counts (B,)); -1 past each row's count."""
    scores = _scores(scores)
    B, M, V = scores.shape
    device = scores.device
    parents_ = _parents(parents, M, device)
    node_tokens = node_tokens.to(device=device, dtype=torch.long).contiguous()
    if node_tokens.shape != (B, M):
        raise ValueError(f"node_tokens must be (B={B}, M={M}); got {tuple(node_tokens.shape)}")
    _on_gpu(scores, node_tokens)
    path = torch.empty(B, M + 1, dtype=torch.long, device=device)
    tokens = torch.empty(B, M + 1, dtype=torch.long, device=device)
    counts = torch.empty(B, dtype=torch.int32, device=device)
    workspace, size = _workspace(device, B, M - 1)
    check(_lib.lib().wptv_greedy_tree(ptr(scores), scores.stride(0), scores.stride(1),
                                      _lib.dtype_code(scores.dtype), ptr(node_tokens),
                                      ptr(parents_), B, M, V, ptr(path), ptr(tokens), ptr(counts), ptr(workspace),
                                      size, _lib.stream(device)), "greedy_tree")
    return path, tokens, counts


def greedy_tree_from_argmax(best, node_tokens, parents):
    """greedy_tree from each node's argmax already found: best (B, M) int32
    (e.g. layers.head_argmax_fm_wide of the nodes' lm_head rows; a -1 ends
    the walk writing nothing).  Returns (path, tokens, counts) as greedy_tree."""
    B, M = best.shape
    device = best.device
    parents_ = _parents(parents, M, device)
    node_tokens = node_tokens.to(device=device, dtype=torch.long).contiguous()
    if node_tokens.shape != (B, M) or best.dtype != torch.int32:
        raise ValueError(f"best must be (B, M) int32 and node_tokens (B={B}, M={M})")
    _on_gpu(best, node_tokens)
    path = torch.empty(B, M + 1, dtype=torch.long, device=device)
    tokens = torch.empty(B, M + 1, dtype=torch.long, device=device)
    counts = torch.empty(B, dtype=torch.int32, device=device)
    check(_lib.lib().wptv_greedy_tree_best(ptr(best.contiguous()), ptr(node_tokens), ptr(parents_), B, M, ptr(path),
                                           ptr(tokens), ptr(counts), _lib.stream(device)), "greedy_tree_best")
    return path, tokens, counts


def _parents(parents, M, device):
    """The tree's parents on the device, checked (made once per tree and device)."""
    parents = [int(p) for p in parents]
    if len(parents) != M or parents[0] != -1 or any(not 0 <= p < i for i, p in enumerate(parents) if i > 0):
        raise ValueError("parents must be (M,) with parents[0] = -1 and 0 <= parents[i] < i")
    key = (tuple(parents), device)
    found = _PARENTS.get(key)
    if found is None:  # outside any graph capture
        found = _PARENTS[key] = torch.tensor(parents, dtype=torch.int32, device=device)
    return found


_PARENTS = {}  # (parents, device) -> the parents on the device


def written(tokens, counts):
    """The host lists of each row's written tokens (one synchronization);
    a row with no residual mass raises as the reference's multinomial does."""
    counts = counts.tolist()
    rows = tokens.tolist()
    out = []
    for b, n in enumerate(counts):
        if n < 0:
            raise RuntimeError(f"row {b}: no token to write: the residual distribution max(0, p - q) has no mass to "
                               f"draw from")
        out.append(rows[b][:n])
    return out
