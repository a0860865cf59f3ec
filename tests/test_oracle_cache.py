"""Pins the oracle's generation cache and decoder (CPU): reading a text in
pieces gives the scores of reading it whole (the reference's
test_cache.py:74-143), rows sharing one prompt go on apart (:173-203), and
undoing rejected drafts leaves the cache as if only the kept tokens had been
read (:206-238); tails cut back as carry.last says.  Each holds for the
exact layers' entries, for the window layers' carried tails (a window of
8 rows, smaller than the pieces, so that the tails matter) and for sparse
layers reading an exact layer's choice of 4 rows outside that window."""

import pytest
import torch

from oracle import cache, decoder

PIECES = [37, 1, 1, 5, 100, 1, 155]
LAYERS, D, H, C, FFN, V = 3, 64, 4, 16, 96, 50


def weights(seed=0):
    generator = torch.Generator().manual_seed(seed)
    w = {"embedding": torch.randn(V, D, generator=generator), "final_norm": 1 + 0.1 * torch.randn(D, generator=generator),
         "head": torch.randn(V, D, generator=generator) * 0.2}
    for i in range(LAYERS):
        w[f"layers.{i}.attn_norm"] = 1 + 0.1 * torch.randn(D, generator=generator)
        w[f"layers.{i}.qkv"] = torch.randn(H * C + 2 * C, D, generator=generator) * 0.2
        w[f"layers.{i}.q_norm"] = 1 + 0.1 * torch.randn(C, generator=generator)
        w[f"layers.{i}.k_norm"] = 1 + 0.1 * torch.randn(C, generator=generator)
        w[f"layers.{i}.out"] = torch.randn(D, H * C, generator=generator) * 0.1
        w[f"layers.{i}.ffn_norm"] = 1 + 0.1 * torch.randn(D, generator=generator)
        w[f"layers.{i}.gate_up"] = torch.randn(2 * FFN, D, generator=generator) * 0.2
        w[f"layers.{i}.down"] = torch.randn(D, FFN, generator=generator) * 0.1
        w[f"layers.{i}.gate"] = torch.randn(H * C, D, generator=generator) * 0.2
        w[f"layers.{i}.sink"] = torch.randn(H, generator=generator)
        w[f"layers.{i}.q"] = torch.randn(H * C, D, generator=generator) * 0.2
    return w


KINDS = [(), ("window", "exact", "exact"), ("window", "exact", "sparse")]
IDS = ["exact", "window+exact", "window+exact+sparse"]


def model(kinds=()):
    return decoder.Decoder(weights(), LAYERS, H, C, kinds=kinds, window=8, rope_dims=8, top_k=4)


def close(got, expected, share=1e-5):
    return (got - expected).abs().max() <= share * expected.abs().max()


@pytest.mark.parametrize("kinds", KINDS, ids=IDS)
def test_reading_in_pieces_gives_the_whole_text_s_scores(kinds):
    m = model(kinds)
    ids = torch.randint(V, (2, sum(PIECES)), generator=torch.Generator().manual_seed(1))
    whole = m.forward(ids)
    rows, got, start = m.new_cache(2), [], 0
    for size in PIECES:
        got.append(m.extend(ids[:, start:start + size], rows)[0])
        start += size
    assert rows.lengths.tolist() == [start, start]
    assert close(torch.cat(got, 1), whole)


@pytest.mark.parametrize("kinds", KINDS, ids=IDS)
def test_a_shared_prompt_and_rows_at_different_places(kinds):
    m = model(kinds)
    generator = torch.Generator().manual_seed(2)
    prompt = torch.randint(V, (40,), generator=generator).tolist()
    texts = [prompt + torch.randint(V, (n,), generator=generator).tolist() for n in (30, 5, 17)]
    shared = m.new_cache(1)
    m.extend(torch.tensor([prompt]), shared)
    rows = shared.select([0, 0, 0])
    got, place = [[] for _ in texts], [len(prompt)] * 3
    for counts in ([1, 1, 1], [10, 0, 7], [3, 4, 1], [16, 0, 8]):
        ids = torch.zeros(3, max(counts), dtype=torch.long)
        for row, count in enumerate(counts):
            ids[row, :count] = torch.tensor(texts[row][place[row]:place[row] + count])
        scores, _ = m.extend(ids, rows, counts)
        for row, count in enumerate(counts):
            got[row].append(scores[row, :count])
            place[row] += count
    assert place == [len(text) for text in texts]
    for row, text in enumerate(texts):
        assert close(torch.cat(got[row]), m.forward(torch.tensor([text]))[0, len(prompt):])
    assert shared.lengths.tolist() == [len(prompt)]


@pytest.mark.parametrize("kinds", KINDS, ids=IDS)
def test_undoing_rejected_drafts_leaves_only_the_kept_tokens(kinds):
    m = model(kinds)
    generator = torch.Generator().manual_seed(3)
    texts = [torch.randint(V, (200,), generator=generator).tolist() for _ in range(2)]
    rows = m.new_cache(2)
    m.extend(torch.tensor([text[:60] for text in texts]), rows)
    place, got = [60, 60], [[], []]
    for kept in ([4, 0], [1, 4], [0, 2], [3, 3], [2, 1], [4, 4], [0, 0], [1, 3]) * 3:
        ids = torch.tensor([texts[row][place[row]:place[row] + 4] for row in range(2)])
        drafts = ids.clone()
        for row in range(2):  # past the kept ones, drafts the text does not hold
            drafts[row, kept[row]:] = (ids[row, kept[row]:] + 1 + row) % V
        scores, _ = m.extend(drafts, rows, undoable=True)
        m.undo(rows, kept)
        for row in range(2):
            got[row].append(scores[row, :kept[row]])
            place[row] += kept[row]
    assert rows.lengths.tolist() == place
    for row in range(2):
        whole = m.forward(torch.tensor([texts[row][:place[row]]]))[0]
        assert close(torch.cat(got[row]), whole[60:])


@pytest.mark.parametrize("kinds", KINDS, ids=IDS)
def test_later_tokens_never_change_earlier_scores(kinds):
    m = model(kinds)
    ids = torch.randint(V, (1, 50), generator=torch.Generator().manual_seed(4))
    changed = ids.clone()
    changed[0, 30] = (changed[0, 30] + 7) % V
    a, b = m.forward(ids), m.forward(changed)
    assert torch.equal(a[:, :30], b[:, :30]) and not torch.allclose(a[:, 30:], b[:, 30:])


def test_undo_without_an_undoable_reading_raises():
    rows = cache.Rows(1)
    try:
        rows.undo([0])
    except ValueError:
        return
    raise AssertionError("undo without a pending reading did not raise")


def test_a_tail_cut_back_keeps_the_steps_before_the_kept_tokens():
    # carry.last: the size rows ending where the first counts[b] new rows end
    before = torch.arange(3.0)[None, :, None].expand(2, 3, 1)
    new = (10 + torch.arange(4.0))[None, :, None].expand(2, 4, 1)
    got = cache.last(torch.cat([before, new], 1), torch.tensor([0, 2]), 3)
    assert got[0, :, 0].tolist() == [0, 1, 2] and got[1, :, 0].tolist() == [2, 10, 11]


@pytest.mark.parametrize("kinds", KINDS, ids=IDS)
@pytest.mark.parametrize("autocast", [False, True], ids=["fp32", "autocast"])
def test_features_are_the_streams_entering_each_layer(kinds, autocast):
    # model.py:406-436: feature n is the residual stream entering layer n,
    # feature `layers` the final hidden states, side by side in the order
    # named; running each layer on those streams (forced) gives the next one
    m = decoder.Decoder(weights(), LAYERS, H, C, kinds=kinds, window=8, rope_dims=8, top_k=4, autocast=autocast)
    ids = torch.randint(V, (2, 40), generator=torch.Generator().manual_seed(11))
    rows = m.new_cache(2)
    m.extend(ids[:, :30], rows)
    copy = rows.select([0, 1])
    scores, hidden, found = m.extend(ids[:, 30:], rows, undoable=True, features=range(LAYERS + 1))
    streams = found.split(D, -1)
    assert found.dtype == torch.float32 and len(streams) == LAYERS + 1
    assert torch.equal(streams[0], m.w["embedding"][ids[:, 30:]].to(hidden.dtype).float())
    assert torch.equal(streams[-1], hidden.float())
    outputs, forced_scores = m.forced(streams, copy)
    assert all(torch.equal(outputs[i].float(), streams[i + 1]) for i in range(LAYERS))
    assert torch.equal(forced_scores, scores)
    again = m.new_cache(2)
    m.extend(ids[:, :30], again)
    _, _, pair = m.extend(ids[:, 30:], again, features=(2, 0))
    assert torch.equal(pair, torch.cat([streams[2], streams[0]], -1))
