"""The allocation-free verify attention (wptv_verify_attention_static, its
parts in the library's static device array) against the workspace entry
point (wptv_verify_attention), through the C ABI: bit for bit, on two calls in
a row, the second smaller (the array keeps the first call's parts), with the
log-sum-exps and with a tree mask; a request beyond the array's 16 MiB is
refused on the host."""

import pytest
import torch

from oracle import attention as oracle
from wpt_amd import kernels

pytestmark = pytest.mark.gpu


def inputs(B, T, H, c, N, seed):
    generator = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, c, generator=generator).to(torch.bfloat16)
    table = torch.randn(B, N, 2 * c, generator=generator).to(torch.bfloat16)
    positions = (N - T + torch.arange(T)).expand(B, T).contiguous()
    return q, table, positions


@pytest.mark.parametrize("lse", [False, True])
def test_the_allocation_free_entry_point_matches_the_workspace_one(device, lse):
    for B, T, H, c, N in ((32, 5, 16, 128, 4096), (3, 5, 16, 128, 700)):  # the second call smaller
        print(f"static scratch: B={B} T={T} H={H} c={c} N={N} lse={lse}", flush=True)
        q, table, positions = (x.to(device) for x in inputs(B, T, H, c, N, seed=B))
        k, v = table[..., :c], table[..., c:]
        expected = kernels.verify_attention(q, k, v, positions, c ** -0.5, lse=lse)
        got = kernels.verify_attention(q, k, v, positions, c ** -0.5, lse=lse, static_scratch=True)
        torch.cuda.synchronize()
        if lse:
            assert torch.equal(got[0], expected[0]) and torch.equal(got[1], expected[1])
        else:
            assert torch.equal(got, expected)


def test_the_allocation_free_entry_point_takes_a_tree(device):
    B, M, H, c, prefix = 4, 31, 16, 128, 1000
    parents = oracle.binary_tree_parents(M)
    q, table, _ = inputs(B, M, H, c, prefix + M, seed=7)
    q, table = q.to(device), table.to(device)
    base = torch.full((B,), prefix, device=device)
    positions = base[:, None] + torch.arange(M, device=device)
    masks = kernels.tree_ancestors(parents).to(device)
    k, v = table[..., :c], table[..., c:]
    expected = kernels.verify_attention(q, k, v, positions, c ** -0.5, tree=(base, masks))
    got = kernels.verify_attention(q, k, v, positions, c ** -0.5, tree=(base, masks), static_scratch=True)
    assert torch.equal(got, expected)


def test_a_request_beyond_the_static_scratch_is_refused(device):
    q, table, positions = (x.to(device) for x in inputs(32, 5, 16, 128, 4096, seed=1))
    with pytest.raises(ValueError, match="static scratch"):
        kernels.verify_attention(q, table[..., :128], table[..., 128:], positions, 128 ** -0.5, splits=64,
                                 static_scratch=True)


def test_the_library_s_own_split_count_steps_down_to_fit(device):
    # 255 batch rows of 128 query rows: the library's choice for the workspace
    # entry point is 2 splits, whose parts (17 MB) do not fit the static array;
    # the allocation-free entry point takes one split instead, the same bits as
    # the workspace entry point asked for one split
    B, T, H, c, N = 255, 8, 16, 128, 300
    print(f"static scratch step-down: B={B} T={T} H={H} c={c} N={N}", flush=True)
    q, table, positions = (x.to(device) for x in inputs(B, T, H, c, N, seed=11))
    k, v = table[..., :c], table[..., c:]
    got = kernels.verify_attention(q, k, v, positions, c ** -0.5, static_scratch=True)
    expected = kernels.verify_attention(q, k, v, positions, c ** -0.5, splits=1)
    torch.cuda.synchronize()
    assert torch.equal(got, expected)
