"""The step's bookkeeping kernels against torch: the embedding with the first
norm and the positions (wptv_embed_rms_norm), the cache's lengths after a
reading and after an undo (wptv_cache_lengths, the reference's
Reading.finish and Rows.undo, cache.py:69-77,130-134), and the next pending
token of each row (wptv_next_feeds)."""

import pytest
import torch
import torch.nn.functional as F

from wpt_amd import layers
from wpt_amd.cache import Cache
from wpt_amd.decoder import PLUMBING, MQADecoder, random_weights
from wpt_amd.step import next_feeds

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("D", [256, 2048, 8 * 3])
def test_the_embedding_norm_and_positions(device, dtype, D):
    generator = torch.Generator().manual_seed(D)
    B, T, V = 3, 5, 50
    table = torch.randn(V, D, generator=generator).to(dtype)
    weight = 1 + 0.1 * torch.randn(D, generator=generator)
    ids = torch.randint(V, (B, T), generator=generator)
    lengths = torch.tensor([0, 7, 4096])
    h = torch.empty(B, T, D, dtype=dtype, device=device)
    x = torch.empty_like(h)
    positions = torch.empty(B, T, dtype=torch.long, device=device)
    layers.embed_rms_norm(ids.to(device), table.to(device), weight.to(device), h, x, lengths.to(device), positions)
    want_h = F.embedding(ids, table)
    assert torch.equal(h.cpu(), want_h)
    want_x = F.rms_norm(want_h.float(), (D,), weight, 1e-6)
    share = 1e-6 if dtype == torch.float32 else 1e-2
    assert float((x.cpu().float() - want_x).abs().max()) <= share * float(want_x.abs().max())
    assert torch.equal(positions.cpu(), lengths[:, None] + torch.arange(T))


@pytest.mark.parametrize("index", [torch.int64, torch.int32])
def test_the_lengths_after_a_reading_and_an_undo(device, index):
    cache = Cache(3, 1, 8, torch.float32, device, capacity=64)
    cache.lengths.copy_(torch.tensor([5, 0, 17]))
    cache.finish(torch.tensor([4, 4, 2], dtype=index, device=device), undoable=True, width=4)
    assert cache.lengths.tolist() == [9, 4, 19] and cache.before.tolist() == [5, 0, 17]
    cache.undo(torch.tensor([1, 0, 2], dtype=index, device=device))
    assert cache.lengths.tolist() == [6, 0, 19]
    # a row the sampler could not draw for (-1) keeps nothing, and no row
    # keeps more than it read
    cache.finish(torch.tensor([4, 4, 2], dtype=index, device=device), undoable=True, width=4)
    cache.undo(torch.tensor([-1, 9, 2], dtype=index, device=device))
    assert cache.lengths.tolist() == [6, 4, 21]
    cache.finish(torch.tensor([3, 1, 0], device=device), undoable=False, width=3)
    assert cache.lengths.tolist() == [9, 5, 21] and cache.before.tolist() == [6, 0, 19]
    with pytest.raises(ValueError):
        cache.undo(torch.zeros(3, dtype=torch.long, device=device))


def test_the_next_pending_token_is_the_last_written(device):
    tokens = torch.tensor([[11, 12, 13, 14], [21, -1, -1, -1], [31, 32, -1, -1]], device=device)
    counts = torch.tensor([4, 1, 2], dtype=torch.int32, device=device)
    feeds = torch.zeros(3, 4, dtype=torch.long, device=device)
    failed = torch.zeros(1, dtype=torch.int32, device=device)
    written = torch.tensor([5, 0, 2], device=device)
    next_feeds(tokens, counts, feeds, failed, written)
    assert feeds[:, 0].tolist() == [14, 21, 32] and not feeds[:, 1:].any() and int(failed) == 0
    assert written.tolist() == [9, 1, 4]
    # a row the sampler could not draw for (-1) keeps its pending token and raises the flag
    feeds[:, 0] = torch.tensor([7, 8, 9], device=device)
    next_feeds(tokens, torch.tensor([-1, 1, 0], dtype=torch.int32, device=device), feeds, failed, written)
    assert feeds[:, 0].tolist() == [7, 21, 9] and int(failed) == 1 and written.tolist() == [9, 2, 4]


def test_host_ids_outside_the_vocabulary_raise(device):
    model = MQADecoder(PLUMBING, random_weights(PLUMBING), dtype=torch.float32)
    cache = model.new_cache(1)
    with pytest.raises(IndexError):
        model.extend(torch.tensor([[0, PLUMBING.vocab]]), cache)
    assert cache.lengths.tolist() == [0]
