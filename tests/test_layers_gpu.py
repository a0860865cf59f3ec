"""The decoder-layer kernels (residual add + RMSNorm, q/k norms + KV append,
SwiGLU) and the standalone KV append against torch on the same inputs:
FP32 within 1e-5 of the largest magnitude, bf16 within 1e-2; appended rows
exact, untouched rows untouched."""

import pytest
import torch
import torch.nn.functional as F

from wpt_amd import kernels, layers

pytestmark = pytest.mark.gpu


def close(got, expected, share):
    return float((got.double() - expected.double()).abs().max()) <= share * float(expected.double().abs().max())


@pytest.mark.parametrize("dtype, share", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
@pytest.mark.parametrize("with_delta", [False, True])
def test_add_rms_norm_matches_torch(device, dtype, share, with_delta):
    g = torch.Generator().manual_seed(0)
    h = torch.randn(37, 2048, generator=g).to(dtype)
    delta = torch.randn(37, 2048, generator=g).to(dtype) if with_delta else None
    weight = 1 + 0.1 * torch.randn(2048, generator=g)
    expected_h = (h + delta) if with_delta else h
    expected = F.rms_norm(expected_h.float(), (2048,), weight, 1e-6)
    hd = h.to(device)
    y = torch.empty_like(hd)
    layers.add_rms_norm(hd, None if delta is None else delta.to(device), weight.to(device), y)
    assert torch.equal(hd.cpu(), expected_h)  # the residual stream in its own dtype
    assert close(y.cpu(), expected, share)


@pytest.mark.parametrize("dtype, share", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
def test_qkv_post_norms_queries_and_appends_entries(device, dtype, share):
    B, T, H, c, cap = 3, 5, 16, 128, 40
    g = torch.Generator().manual_seed(1)
    qkv = torch.randn(B, T, (H + 2) * c, generator=g).to(dtype)
    qn, kn = 1 + 0.1 * torch.randn(c, generator=g), 1 + 0.1 * torch.randn(c, generator=g)
    table = torch.randn(B, cap, 2 * c, generator=g).to(dtype)
    start, counts = torch.tensor([0, 10, 34]), torch.tensor([5, 2, 5])  # the last row reaches past the capacity
    q_expected = F.rms_norm(qkv[..., :H * c].reshape(B, T, H, c).float(), (c,), qn, 1e-6)
    k_expected = F.rms_norm(qkv[..., H * c:H * c + c].float(), (c,), kn, 1e-6).to(dtype)
    expected = table.clone()
    for b in range(B):
        for t in range(int(counts[b])):
            if start[b] + t < cap:
                expected[b, start[b] + t, :c] = k_expected[b, t]
                expected[b, start[b] + t, c:] = qkv[b, t, H * c + c:]
    td = table.to(device)
    q = layers.qkv_post(qkv.to(device), qn.to(device), kn.to(device), td, start.to(device), counts.to(device), H)
    assert close(q.cpu(), q_expected, share)
    got = td.cpu()
    written = torch.zeros(B, cap, dtype=torch.bool)
    for b in range(B):
        written[b, start[b]:min(start[b] + counts[b], cap)] = True
    assert torch.equal(got[~written], table[~written])  # every other row untouched
    assert close(got[written], expected[written].float(), share)


@pytest.mark.parametrize("dtype, share", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
def test_swiglu_matches_torch(device, dtype, share):
    gu = torch.randn(7, 2 * 5632, generator=torch.Generator().manual_seed(2)).to(dtype)
    gate, up = gu.float().chunk(2, -1)
    assert close(layers.swiglu(gu.to(device)).cpu(), F.silu(gate) * up, share)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kv_append_writes_each_row_at_its_length(device, dtype):
    # the scatter of Reading.everything (cache.py:110-128)
    B, n, cap, width = 4, 5, 64, 256
    g = torch.Generator().manual_seed(3)
    table = torch.randn(B, cap, width, generator=g).to(dtype)
    new = torch.randn(B, n, width, generator=g).to(dtype)
    start, counts = torch.tensor([0, 7, 60, 30]), torch.tensor([5, 0, 5, 3])
    expected = table.clone()
    for b in range(B):
        for j in range(int(counts[b])):
            if start[b] + j < cap:
                expected[b, start[b] + j] = new[b, j]
    td = table.to(device)
    kernels.kv_append(td, new.to(device), start.to(device), counts.to(device))
    assert torch.equal(td.cpu(), expected)


@pytest.mark.parametrize("splits", [1, 3, 7])
def test_qkv_post_parts_equals_qkv_post_on_the_summed_product(device, splits):
    # the projection as FP32 split-K parts: summed in order and rounded to
    # bf16, then exactly qkv_post's work
    B, T, H, c, cap = 2, 5, 16, 128, 32
    g = torch.Generator().manual_seed(3)
    parts = torch.randn(splits, B * T, (H + 2) * c, generator=g)
    summed = parts[0].clone()
    for z in range(1, splits):
        summed += parts[z]
    qkv = summed.to(torch.bfloat16).reshape(B, T, (H + 2) * c)
    qn, kn = 1 + 0.1 * torch.randn(c, generator=g), 1 + 0.1 * torch.randn(c, generator=g)
    table = torch.randn(B, cap, 2 * c, generator=g).to(torch.bfloat16)
    start, counts = torch.tensor([3, 20]), torch.tensor([5, 4])
    t1, t2 = table.to(device), table.to(device)
    args = (qn.to(device), kn.to(device))
    q1 = layers.qkv_post(qkv.to(device), *args, t1, start.to(device), counts.to(device), H)
    q2 = layers.qkv_post_parts(parts.to(device), *args, t2, start.to(device), counts.to(device), H, T)
    assert torch.equal(q1, q2)
    assert torch.equal(t1, t2)
