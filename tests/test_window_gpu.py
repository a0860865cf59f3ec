"""The window layer on the GPU against the oracle: window attention with its
sink and output gate (the reference's table of the carried tail and the new
entries, and the build's ring cache), the q/k norms with the rotary encoding
and the ring append, and decoders of window and exact layers through the
generation protocol (reading in pieces, undo) with the carried tails equal
to the oracle's.  bf16 within 2e-2 of the largest expected value, FP32
within 1e-5."""

import pytest
import torch

from oracle import attention as oracle
from oracle import decoder as oracle_decoder
from tests.formulas import relative_error
from wpt_amd import kernels, layers
from wpt_amd.decoder import DecoderConfig, MQADecoder, random_weights

pytestmark = pytest.mark.gpu


def draw(*shape, seed, dtype=torch.bfloat16):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).to(dtype)


def tail_table(full, start, window):
    """The reference's (B, window - 1 + T) table of a pass starting at
    `start`: the window - 1 entries before it (zeros before the text), then
    the pass's own."""
    B, L, width = full.shape
    tail = torch.zeros(B, window - 1, width, dtype=full.dtype)
    before = full[:, max(0, start - window + 1):start]
    if before.shape[1]:
        tail[:, window - 1 - before.shape[1]:] = before
    return torch.cat([tail, full[:, start:]], 1)


@pytest.mark.parametrize("dtype, B, T, H, c, window, start", [
    (torch.bfloat16, 32, 5, 16, 128, 128, 4091),   # a WPT window layer at the verify step
    (torch.bfloat16, 4, 5, 16, 128, 128, 60),      # a text shorter than the window
    (torch.bfloat16, 2, 7, 12, 64, 16, 3),         # 84 query rows, head width 64
    (torch.float32, 2, 5, 4, 64, 128, 300),        # the FP32 form
    (torch.float32, 1, 3, 4, 64, 8, 0),            # the first tokens of a text
])
@pytest.mark.parametrize("gated", [False, True], ids=["plain", "gated"])
def test_window_attention_matches_the_oracle(device, dtype, B, T, H, c, window, start, gated):
    q = draw(B, T, H, c, seed=1, dtype=dtype)
    full = draw(B, start + T, 2 * c, seed=2, dtype=dtype)
    sink = draw(H, seed=3, dtype=torch.float32)
    gate = draw(B, T, H * c + 32, seed=4, dtype=dtype) if gated else None  # wider rows: a strided view
    positions = (start + torch.arange(T)).expand(B, T)
    table = tail_table(full, start, window)
    expected = oracle.window_attention(q, table[..., :c], table[..., c:], sink, positions, c ** -0.5, window)
    if gated:
        expected = expected * torch.sigmoid(gate[..., :H * c].float()).reshape(B, T, H, c)
    td = table.to(device)
    got = kernels.window_attention(q.to(device), td[..., :c], td[..., c:], sink.to(device), positions.to(device),
                                   c ** -0.5, window, gate=None if gate is None else gate.to(device)[..., :H * c])
    assert got.dtype == dtype and got.shape == (B, T, H, c)
    if dtype == torch.float32:
        assert (got.cpu() - expected).abs().max() < 1e-5
    else:
        assert relative_error(got.cpu(), expected) < 2e-2


@pytest.mark.parametrize("start", [0, 100, 251, 40000])
def test_ring_attention_reads_the_ring_by_position(device, start):
    # the build's ring cache (token p at row p mod 256) gives the reference
    # table's result, also where the window wraps around the ring
    B, T, H, c, window, R = 3, 5, 16, 128, 128, 256
    q = draw(B, T, H, c, seed=5)
    full = draw(B, start + T, 2 * c, seed=6)
    sink = draw(H, seed=7, dtype=torch.float32)
    positions = (start + torch.arange(T)).expand(B, T)
    ring = torch.zeros(B, R, 2 * c, dtype=torch.bfloat16)
    keep = range(max(0, start + T - R), start + T)
    ring[:, [p % R for p in keep]] = full[:, list(keep)]
    table = tail_table(full, start, window)
    expected = oracle.window_attention(q, table[..., :c], table[..., c:], sink, positions, c ** -0.5, window)
    got = kernels.ring_attention(q.to(device), ring.to(device), positions.to(device), c ** -0.5, window,
                                 sink.to(device))
    assert relative_error(got.cpu(), expected) < 2e-2


@pytest.mark.parametrize("dtype, c, start, share", [
    (torch.float32, 64, 37, 1e-5), (torch.float32, 128, 900, 1e-5), (torch.bfloat16, 128, 20000, 2e-2),
    (torch.bfloat16, 256, 5, 2e-2)])
def test_window_qkv_post_rotates_and_appends_to_the_ring(device, dtype, c, start, share):
    B, T, H, R = 3, 5, 4, 256
    proj = draw(B, T, (2 * H + 2) * c, seed=8, dtype=dtype)  # q, k, v, then a gate the kernel leaves alone
    q_norm, k_norm = 1 + 0.1 * draw(c, seed=9, dtype=torch.float32), 1 + 0.1 * draw(c, seed=10, dtype=torch.float32)
    lengths = torch.tensor([start, start + 3, start + 200])
    counts = torch.tensor([5, 2, 4])
    positions = lengths[:, None] + torch.arange(T)
    norm = lambda x, w: torch.nn.functional.rms_norm(x.float(), (c,), w, 1e-6).to(dtype)  # noqa: E731
    want_q = oracle.rotate(norm(proj[..., :H * c].reshape(B, T, H, c), q_norm), positions)
    want_k = oracle.rotate(norm(proj[..., H * c:(H + 1) * c], k_norm), positions)
    want_v = proj[..., (H + 1) * c:(H + 2) * c]
    ring = torch.full((B, R, 2 * c), 7.0, dtype=dtype, device=device)
    q = layers.window_qkv_post(proj.to(device), q_norm.to(device), k_norm.to(device), ring, lengths.to(device),
                               counts.to(device), H)
    assert relative_error(q.cpu(), want_q) < share
    ring = ring.cpu()
    for b in range(B):
        for t in range(T):
            slot = int(positions[b, t]) % R
            if t < counts[b]:
                assert relative_error(ring[b, slot, :c], want_k[b, t]) < share
                assert torch.equal(ring[b, slot, c:], want_v[b, t])
            else:
                assert (ring[b, slot] == 7.0).all()  # past counts[b]: untouched


@pytest.mark.parametrize("dtype, c, heads, rope_dims, share", [
    (torch.float32, 64, 4, 32, 1e-5), (torch.bfloat16, 128, 16, 64, 2e-2), (torch.bfloat16, 128, 1, 64, 2e-2),
    (torch.bfloat16, 256, 2, 256, 2e-2)])
def test_head_norms_with_the_rotation_match_the_reference_rotate(device, dtype, c, heads, rope_dims, share):
    # the drafter's q and k: rotate(norm(x), positions) per head of a strided
    # projection, positions per row (clamped at 0 as a window before the text)
    B, T = 3, 7
    proj = draw(B, T, heads * c + 96, seed=11, dtype=dtype)  # wider rows: the heads are a strided view
    weight = 1 + 0.1 * draw(c, seed=12, dtype=torch.float32)
    positions = (torch.tensor([[5], [900], [40000]]) - 3 + torch.arange(T)).clamp(min=0)
    norm = lambda x: torch.nn.functional.rms_norm(x.float(), (c,), weight, 1e-6).to(dtype)  # noqa: E731
    want = oracle.rotate(norm(proj[..., :heads * c].reshape(B, T, heads, c)), positions, dims=rope_dims)
    divisors = layers.rope_divisors(rope_dims, device=device)
    got = layers.heads_rms_norm(proj.to(device), weight.to(device), heads, positions=positions.to(device),
                                divisors=divisors)
    assert got.shape == (B, T, heads, c) and got.dtype == dtype
    assert relative_error(got.cpu(), want) < share
    # without positions: the norm alone
    plain = layers.heads_rms_norm(proj.to(device), weight.to(device), heads)
    assert relative_error(plain.cpu(), norm(proj[..., :heads * c].reshape(B, T, heads, c))) < share


# FP32 on the generic kernels; bf16 with 16 heads of width 128 on the
# matrix-core kernels (two layers and small weights, as the exact decoder's
# bf16 tests, so that bf16 rounding stays inside 2e-2)
CONFIG = DecoderConfig(layers=4, d_model=256, heads=4, head_dim=64, ffn=512, vocab=1024,
                       kinds=("window", "exact", "window", "exact"), window=16, rope_dims=32)
CONFIG_BF16 = DecoderConfig(layers=2, d_model=256, heads=16, head_dim=128, ffn=512, vocab=1024,
                            kinds=("window", "exact"), window=16, rope_dims=64)


def models(config, dtype, seed=0):
    std = 0.05 if dtype == torch.float32 else 0.02
    w = random_weights(config, seed=seed, std=std)
    # the oracle holds the weights the GPU model holds (matrices in its dtype)
    held = {name: value if name.endswith("norm") or name.endswith("sink") else value.to(dtype).float()
            for name, value in w.items()}
    return (MQADecoder(config, w, dtype=dtype),
            oracle_decoder.Decoder(held, config.layers, config.heads, config.head_dim, kinds=config.kinds,
                                   window=config.window, rope_dims=config.rope_dims, rope_base=config.rope_base))


def close(got, expected, share):
    return float((got.double() - expected.double()).abs().max()) <= share * float(expected.double().abs().max())


@pytest.mark.parametrize("config, dtype, share", [(CONFIG, torch.float32, 1e-5), (CONFIG_BF16, torch.bfloat16, 2e-2)],
                         ids=["fp32", "bf16"])
def test_a_decoder_with_window_layers_reads_in_pieces_as_the_oracle_reads_whole(device, config, dtype, share):
    gpu, ora = models(config, dtype)
    ids = torch.randint(config.vocab, (2, 90), generator=torch.Generator().manual_seed(1))
    cache = gpu.new_cache(2, capacity=16, widest=16)  # rings of 32 rows: the 40-token piece is read in three
    got = [gpu.extend(ids[:, a:b].to(device), cache)[0].cpu() for a, b in ((0, 40), (40, 41), (41, 70), (70, 90))]
    assert cache.lengths.tolist() == [90, 90] and cache.ring_rows == 32
    assert close(torch.cat(got, 1), ora.forward(ids), share)


@pytest.mark.parametrize("config, dtype, share", [(CONFIG, torch.float32, 1e-5), (CONFIG_BF16, torch.bfloat16, 2e-2)],
                         ids=["fp32", "bf16"])
def test_undo_leaves_the_window_layers_tails_as_the_oracle_s(device, config, dtype, share):
    # the reference's kept patterns (test_cache.py:206-238), rows at
    # different places; after every undo each window layer's tail (the 15
    # entries before each row's length) equals the oracle's carried tail
    gpu, ora = models(config, dtype)
    generator = torch.Generator().manual_seed(3)
    texts = [torch.randint(config.vocab, (200,), generator=generator).tolist() for _ in range(2)]
    cache, rows = gpu.new_cache(2, capacity=64), ora.new_cache(2)
    first = torch.tensor([texts[0][:30], texts[1][:30]])
    gpu.extend(first.to(device), cache, counts=[30, 21])
    ora.extend(first, rows, counts=[30, 21])
    place = [30, 21]
    for kept in ([4, 0], [1, 4], [0, 2], [3, 3], [2, 1], [4, 4], [0, 0], [1, 3]) * 2:
        ids = torch.tensor([texts[row][place[row]:place[row] + 4] for row in range(2)])
        drafts = ids.clone()
        for row in range(2):
            drafts[row, kept[row]:] = (ids[row, kept[row]:] + 1 + row) % config.vocab
        got, _ = gpu.extend(drafts.to(device), cache, undoable=True)
        want, _ = ora.extend(drafts, rows, undoable=True)
        assert close(got.cpu(), want, share)
        gpu.undo(cache, kept)
        ora.undo(rows, kept)
        for row in range(2):
            place[row] += kept[row]
        assert cache.lengths.tolist() == rows.lengths.tolist() == place
        for i in config.windows:
            tail = cache.tail(i, config.window - 1).cpu()
            assert close(tail, rows.values[("window", i)], share)


def test_a_reading_wider_than_the_rings_must_not_be_undoable(device):
    gpu, _ = models(CONFIG, torch.float32)
    cache = gpu.new_cache(1, widest=8)
    with pytest.raises(ValueError):
        gpu.extend(torch.zeros(1, 40, dtype=torch.long, device=device), cache, undoable=True)
