"""The HIP verify attention against the oracle, on the GPU, through the C ABI
(wpt_amd.kernels calls libwptv.so): bf16 within 1e-2 of the largest expected
value (the reference's own kernel tolerance, test_kernels.py:173, tighter than
the 2e-2 the verify step allows), fp32 within 1e-5."""

import pytest
import torch

from oracle import attention as oracle
from tests.formulas import relative_error
from wpt_amd import kernels, layers

pytestmark = pytest.mark.gpu


def draw(*shape, seed, dtype=torch.bfloat16):
    generator = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=generator).to(dtype)


def entries_table(B, N, c, seed, dtype=torch.bfloat16):
    """k and v as the strided halves of one (B, N, 2c) entries table."""
    table = draw(B, N, 2 * c, seed=seed, dtype=dtype)
    return table, table[..., :c], table[..., c:]


def on(device, *tensors):
    return [t.to(device) for t in tensors]


# the MFMA kernel forms: 16-row blocks, key-parallel, 32-row blocks
FORMS = {"row-blocks": {}, "key-parallel": {"key_split": True}, "rows32": {"rows32": True}}


@pytest.mark.parametrize("B, T, H, c, N, splits", [
    (32, 5, 16, 128, 4096, 0),   # the verify-attention workload: 16 query heads, 1 KV head, k+1 = 5
    (32, 5, 16, 128, 4096, 1),   # one part per batch row: no combine
    (4, 5, 16, 128, 1000, 3),    # a key range that does not split evenly
    (3, 4, 4, 128, 400, 0),      # the reference's generation-pass shape (test_triton_kernels.py:58)
    (2, 7, 12, 128, 300, 0),     # 84 query rows: five 16-row blocks, the last partly padding
    (2, 5, 16, 64, 777, 0),      # head width 64
    (1, 1, 4, 64, 1, 0),         # a single row
    (64, 5, 16, 128, 2048, 0),   # the end-to-end step's layer shape
])
@pytest.mark.parametrize("form", list(FORMS))
def test_exact_attention_matches_the_oracle(device, B, T, H, c, N, splits, form):
    q = draw(B, T, H, c, seed=1)
    _, k, v = entries_table(B, N, c, seed=2)
    positions = (N - T + torch.arange(T)).clamp(min=0).expand(B, T).contiguous()
    expected, _ = oracle.exact_attention(q, k, v, positions, c ** -0.5, 0, 128)
    qd, kd, vd, pd = on(device, q, k, v, positions)
    # the strided halves of the device table, as the model's cache gives them
    table = torch.cat([kd, vd], -1)
    got = kernels.verify_attention(qd, table[..., :c], table[..., c:], pd, c ** -0.5, splits=splits,
                                   **FORMS[form])
    assert got.dtype == torch.bfloat16 and got.shape == (B, T, H, c)
    assert relative_error(got.cpu(), expected) < 1e-2


def test_padding_queries_past_the_table(device):
    # the reference's generation pass: rows at different places, the last
    # row's later queries past the table read up to its last row
    B, T, H, c, N = 3, 4, 4, 128, 400
    q = draw(B, T, H, c, seed=0)
    table, k, v = entries_table(B, N, c, seed=1)
    positions = torch.tensor([[396, 397, 398, 399], [100, 101, 102, 103], [398, 399, 400, 401]])
    expected, _ = oracle.exact_attention(q, k, v, positions, c ** -0.5, 0, 16)
    qd, td, pd = on(device, q, table, positions)
    out, chosen = kernels.exact_attention(qd, td[..., :c], td[..., c:], pd, c ** -0.5, 0, 16)
    assert chosen.shape == (B, T, 0)
    assert relative_error(out.cpu(), expected) < 1e-2


def test_fp32_attention_is_within_1e_5(device):
    # the fp32 form (the CPU-runnable plumbing decoder's head layout)
    B, T, H, c, N = 1, 5, 4, 64, 69
    q = draw(B, T, H, c, seed=3, dtype=torch.float32)
    _, k, v = entries_table(B, N, c, seed=4, dtype=torch.float32)
    positions = (N - T + torch.arange(T)).expand(B, T).contiguous()
    expected, _ = oracle.exact_attention(q, k, v, positions, c ** -0.5, 0, 128)
    got = kernels.verify_attention(*on(device, q, k, v, positions), c ** -0.5)
    assert (got.cpu() - expected).abs().max() < 1e-5


def test_the_generic_and_mfma_kernels_agree(device):
    B, T, H, c, N = 2, 5, 16, 128, 1500
    q, (_, k, v) = draw(B, T, H, c, seed=5), entries_table(B, N, c, seed=6)
    positions = (N - T + torch.arange(T)).expand(B, T).contiguous()
    args = on(device, q, k, v, positions)
    generic = kernels.verify_attention(*args, c ** -0.5, generic=True).cpu().float()
    for form in FORMS.values():
        mfma = kernels.verify_attention(*args, c ** -0.5, **form)
        assert relative_error(mfma.cpu(), generic) < 1e-2


@pytest.mark.parametrize("form", list(FORMS))
def test_scores_growing_along_the_keys(device, form):
    # every query along one direction u, key n = f_n u with f_n rising over
    # the rows: each row's maximum grows by far more than 2^32 across the
    # tiles, so the running maximum moves and the partial sums are rescaled
    B, T, H, c, N = 2, 5, 16, 128, 2000
    generator = torch.Generator().manual_seed(31)
    u = torch.randn(c, generator=generator)
    u = u / u.norm()
    q = (8 * u).expand(B, T, H, c) * (1 + 0.1 * torch.randn(B, T, H, 1, generator=generator))
    f = torch.linspace(0, 100, N)
    k = f[None, :, None] * u + 0.05 * torch.randn(B, N, c, generator=generator)
    v = torch.randn(B, N, c, generator=generator)
    q, k, v = (x.to(torch.bfloat16) for x in (q, k, v))
    positions = (N - T + torch.arange(T)).expand(B, T).contiguous()
    expected, _ = oracle.exact_attention(q, k, v, positions, c ** -0.5, 0, 128)
    for splits in (1, 0):
        got = kernels.verify_attention(*on(device, q, k, v, positions), c ** -0.5, splits=splits,
                                       **FORMS[form])
        assert relative_error(got.cpu(), expected) < 1e-2


def test_a_small_tree_on_both_mfma_kernels(device):
    # a draft tree of 5 nodes (root, two children, two grandchildren under
    # the first child): 80 query rows
    B, H, c, prefix = 3, 16, 128, 700
    parents = [-1, 0, 0, 1, 1]
    M = len(parents)
    q = draw(B, M, H, c, seed=32)
    _, k, v = entries_table(B, prefix + M, c, seed=33)
    prefixes = torch.tensor([prefix, prefix - 37, prefix - 300])
    expected = oracle.tree_attention(q, k, v, prefixes, parents, c ** -0.5)
    qd, kd, vd, bd = on(device, q, k, v, prefixes)
    got = kernels.tree_attention(qd, kd, vd, bd, parents, c ** -0.5)
    assert relative_error(got.cpu(), expected) < 1e-2
    positions = bd[:, None] + torch.arange(M, device=device)
    masks = kernels.tree_ancestors(parents).to(device)
    got = kernels.verify_attention(qd, kd, vd, positions, c ** -0.5, tree=(bd, masks), key_split=True)
    assert relative_error(got.cpu(), expected) < 1e-2
    # the positions given, or formed by the kernel as tree_base + node: the same bits on every kernel
    for form in ({}, {"key_split": True}, {"rows32": True}, {"generic": True}):
        given = kernels.verify_attention(qd, kd, vd, positions, c ** -0.5, tree=(bd, masks), **form)
        formed = kernels.verify_attention(qd, kd, vd, None, c ** -0.5, tree=(bd, masks), **form)
        assert torch.equal(given, formed)
    with pytest.raises(ValueError):
        kernels.verify_attention(qd, kd, vd, None, c ** -0.5)  # no positions and no tree


@pytest.mark.parametrize("with_sink", [False, True])
def test_sliding_window_verify_matches_the_oracle(device, with_sink):
    # the sliding-window workload: per-row lengths uniform in [N/2, N], window
    # 1024, k+1 = 5 queries at each row's end
    B, T, H, c, N, W = 8, 5, 16, 128, 32768, 1024
    generator = torch.Generator().manual_seed(7)
    lengths = torch.randint(N // 2, N + 1, (B,), generator=generator)
    positions = lengths[:, None] - T + torch.arange(T)
    q = draw(B, T, H, c, seed=8)
    _, k, v = entries_table(B, N, c, seed=9)
    sink = draw(H, seed=10, dtype=torch.float32) if with_sink else torch.full((H,), float("-inf"))
    idx = torch.empty(B, T, 0, dtype=torch.long)
    expected = oracle.sparse_attention(q, k, v, sink, idx, positions, c ** -0.5, W)
    qd, kd, vd, pd, sd, id_ = on(device, q, k, v, positions, sink, idx)
    got = kernels.sparse_attention(qd, kd, vd, sd, id_, pd, c ** -0.5, W)
    assert relative_error(got.cpu(), expected) < 1e-2


def test_chosen_rows_with_a_window_and_sink_match_the_oracle(device):
    # the sparse form with chosen rows (the generic kernel's gather)
    B, T, H, c, N, W, K = 2, 6, 4, 128, 300, 32, 16
    q = draw(B, T, H, c, seed=11)
    _, k, v = entries_table(B, N, c, seed=12)
    sink = draw(H, seed=13, dtype=torch.float32)
    positions = (N - T + torch.arange(T)).expand(B, T).contiguous()
    generator = torch.Generator().manual_seed(14)
    idx = torch.stack([torch.stack([torch.randperm(int(p) - W + 1, generator=generator)[:K] for p in row])
                       for row in positions])
    idx[:, ::2, -3:] = -1
    expected = oracle.sparse_attention(q, k, v, sink, idx, positions, c ** -0.5, W)
    got = kernels.sparse_attention(*on(device, q, k, v, sink, idx, positions), c ** -0.5, W)
    assert relative_error(got.cpu(), expected) < 1e-2


@pytest.mark.parametrize("B, T, H, c, N, W, K, splits", [
    (32, 5, 16, 128, 4096, 128, 1024, 0),   # a WPT sparse layer at the verify step (TOP_K 1024, WINDOW 128)
    (2, 6, 12, 128, 300, 32, 16, 1),        # 12 heads, one part: no combine
    (3, 5, 16, 64, 500, 40, 100, 3),        # head width 64, three parts
    (2, 4, 16, 128, 200, 16, 300, 0),       # more chosen entries than rows: many -1
])
@pytest.mark.parametrize("gated", [False, True], ids=["plain", "gated"])
def test_the_sparse_gather_kernel_matches_the_oracle(device, B, T, H, c, N, W, K, splits, gated):
    # chosen rows outside each query's window, some -1, some named twice and
    # some also in the window (each counts twice, as the reference's
    # concatenation counts it); the last row's queries past the table
    q = draw(B, T, H, c, seed=40)
    _, k, v = entries_table(B, N, c, seed=41)
    sink = draw(H, seed=42, dtype=torch.float32)
    positions = (N - T + torch.arange(T)).expand(B, T).clone()
    positions[-1] += 2
    generator = torch.Generator().manual_seed(43)
    idx = torch.randint(-1, N, (B, T, K), generator=generator)
    idx[:, :, :2] = positions[..., None].clamp(max=N - 1) - torch.tensor([0, 1])  # also in the window
    idx[:, :, 2] = idx[:, :, 3]                                                   # named twice
    gate = draw(B, T, H * c, seed=44) if gated else None
    expected = oracle.sparse_attention(q, k, v, sink, idx, positions, c ** -0.5, W)
    if gated:
        expected = expected * torch.sigmoid(gate.float()).reshape(B, T, H, c)
    qd, kd, vd, sd, id_, pd = on(device, q, k, v, sink, idx, positions)
    got = kernels.sparse_attention(qd, kd, vd, sd, id_, pd, c ** -0.5, W, splits=splits,
                                   gate=None if gate is None else gate.to(device))
    assert relative_error(got.cpu(), expected) < 1e-2


def test_tree_attention_matches_the_oracle(device):
    # the tree workload's shape at a smaller prefix: a binary draft tree of 31
    # nodes (depth 5) after the prefix, ancestor-only mask (496 query rows: the
    # 32-row kernel by default, the key-parallel form below)
    B, M, H, c, prefix = 4, 31, 16, 128, 1000
    parents = oracle.binary_tree_parents(M)
    q = draw(B, M, H, c, seed=15)
    _, k, v = entries_table(B, prefix + M, c, seed=16)
    prefixes = torch.full((B,), prefix)
    expected = oracle.tree_attention(q, k, v, prefixes, parents, c ** -0.5)
    qd, kd, vd, bd = on(device, q, k, v, prefixes)
    got = kernels.tree_attention(qd, kd, vd, bd, parents, c ** -0.5)
    assert relative_error(got.cpu(), expected) < 1e-2
    positions = bd[:, None] + torch.arange(M, device=device)
    masks = kernels.tree_ancestors(parents).to(device)
    got = kernels.verify_attention(qd, kd, vd, positions, c ** -0.5, tree=(bd, masks), key_split=True)
    assert relative_error(got.cpu(), expected) < 1e-2


def test_lse_is_the_log_sum_exp(device):
    B, T, H, c, N = 2, 5, 16, 128, 513
    q, (_, k, v) = draw(B, T, H, c, seed=17), entries_table(B, N, c, seed=18)
    positions = (N - T + torch.arange(T)).expand(B, T).contiguous()
    z = torch.einsum("bthc,bnc->bthn", q.float(), k.float()) * c ** -0.5
    z = z.masked_fill(torch.arange(N) > positions[..., None, None], float("-inf"))
    for splits in (1, 4):
        for form in FORMS.values():
            _, lse = kernels.verify_attention(*on(device, q, k, v, positions), c ** -0.5, lse=True, splits=splits,
                                              **form)
            assert (lse.cpu() - z.logsumexp(-1)).abs().max() < 2e-2


def test_bad_shapes_raise_value_error(device):
    q = torch.zeros(2, 5, 16, 128, dtype=torch.bfloat16, device=device)
    k = torch.zeros(2, 64, 128, dtype=torch.bfloat16, device=device)
    positions = torch.zeros(2, 4, dtype=torch.long, device=device)
    with pytest.raises(ValueError):
        kernels.verify_attention(q, k, k, positions, 0.1)
    with pytest.raises(ValueError):
        kernels.verify_attention(q, k.float(), k.float(), positions[:, :1].expand(2, 5), 0.1)


@pytest.mark.parametrize("rows", [160, 240])
def test_the_32_row_kernel_with_window_sink_gate_and_fm_output(device, rows):
    # more than 128 query rows a batch row (the 32-row kernel's default
    # range): a window, a sink and the output gate against the oracle, the
    # log-sum-exps, and the fm output bit for bit the row-major one
    B, H, c, N, W = 3, 16, 128, 900, 256
    T = rows // H
    q = draw(B, T, H, c, seed=41)
    _, k, v = entries_table(B, N, c, seed=42)
    sink = draw(H, seed=43, dtype=torch.float32)
    gate = draw(B, T, H * c, seed=44)
    positions = torch.stack([torch.arange(N - T, N), torch.arange(300, 300 + T), torch.arange(N - 2 * T, N - T)])
    idx = torch.empty(B, T, 0, dtype=torch.long)
    expected = oracle.sparse_attention(q, k, v, sink, idx, positions, c ** -0.5, W)
    gated = expected.float() * torch.sigmoid(gate.float()).reshape(B, T, H, c)
    qd, kd, vd, pd, sd, gd = on(device, q, k, v, positions, sink, gate)
    for splits in (1, 0):
        got = kernels.verify_attention(qd, kd, vd, pd, c ** -0.5, window=W, sink=sd, splits=splits)
        assert relative_error(got.cpu(), expected) < 1e-2
    got, lse = kernels.verify_attention(qd, kd, vd, pd, c ** -0.5, window=W, lse=True)
    z = torch.einsum("bthc,bnc->bthn", q.float(), k.float()) * c ** -0.5
    n = torch.arange(N)
    seen = (n <= positions[..., None]) & (n > positions[..., None] - W)
    z = z.masked_fill(~seen[:, :, None, :], float("-inf"))
    assert (lse.cpu() - z.logsumexp(-1)).abs().max() < 2e-2
    out = kernels.verify_attention(qd, kd, vd, pd, c ** -0.5, window=W)
    out_fm = kernels.verify_attention(qd, kd, vd, pd, c ** -0.5, window=W, out_fm=True)
    assert torch.equal(layers.fm_unpack(out_fm, B * T, H * c), out.reshape(B * T, H * c))
    # the window-only sparse form runs the same kernel, here with the output gate
    id_ = idx.to(device)
    got = kernels.sparse_attention(qd, kd, vd, sd, id_, pd, c ** -0.5, W, gate=gd)
    assert relative_error(got.cpu().float(), gated) < 2e-2
