"""Sparse layers on the GPU against the oracle: the per-head query norm
(wptv_heads_rms_norm), and decoders whose exact layers choose rows for the
sparse layers after them (attention.py:157-216, model.py:134-135,411-423)
read in pieces, through undone drafts, as the oracle reads them.

The windows (16) and choices (8 rows) are small beside the texts (90 and 200
tokens), so that most queries have more candidates than the choice keeps.
FP32 runs the generic kernels, and its choices are the oracle's; bf16 with
16 heads of width 128 the matrix-core ones, where the two implementations'
scores may order near ties of the choice another way (the reference's kernel
test allows for it, test_kernels.py:156-187): there the oracle's sparse
layers read the GPU's choice, after every chosen row is checked to score
within CHOICE_SLACK (in log) of the oracle's own top_k-th."""

import pytest
import torch

from oracle import decoder as oracle_decoder
from tests.formulas import choice_scores
from tests.test_choice_gpu import check_choice
from wpt_amd import kernels, layers
from wpt_amd.decoder import DecoderConfig, MQADecoder, layer_kinds, random_weights

pytestmark = pytest.mark.gpu


def relative_error(got, want):
    return float((got.double() - want.double()).abs().max() / want.double().abs().max())


@pytest.mark.parametrize("dtype, share", [(torch.float32, 1e-6), (torch.bfloat16, 1e-2)], ids=["fp32", "bf16"])
@pytest.mark.parametrize("c", [64, 128, 256])
def test_heads_rms_norm_is_the_oracle_s_norm_of_each_head(device, dtype, share, c):
    generator = torch.Generator().manual_seed(c)
    B, T, H = 3, 5, 4
    x = torch.randn(B, T, 2 * H * c + 64, generator=generator).to(dtype)  # rows wider than the heads
    weight = 1 + 0.1 * torch.randn(c, generator=generator)
    got = layers.heads_rms_norm(x.to(device), weight.to(device), H)
    want = oracle_decoder.rms_norm(x[..., :H * c].float().reshape(B, T, H, c), weight)
    assert got.shape == (B, T, H, c) and got.dtype == dtype
    assert relative_error(got.cpu(), want) < share


CONFIG = DecoderConfig(layers=4, d_model=256, heads=4, head_dim=64, ffn=512, vocab=1024,
                       kinds=("window", "exact", "sparse", "sparse"), window=16, rope_dims=32, top_k=8)
CONFIG_BF16 = DecoderConfig(layers=3, d_model=256, heads=16, head_dim=128, ffn=512, vocab=1024,
                            kinds=("exact", "sparse", "window"), window=16, rope_dims=64, top_k=8)


def models(config, dtype, seed=0):
    std = 0.05 if dtype == torch.float32 else 0.02
    w = random_weights(config, seed=seed, std=std)
    held = {name: value if name.endswith("norm") or name.endswith("sink") else value.to(dtype).float()
            for name, value in w.items()}
    return (MQADecoder(config, w, dtype=dtype),
            oracle_decoder.Decoder(held, config.layers, config.heads, config.head_dim, kinds=config.kinds,
                                   window=config.window, rope_dims=config.rope_dims, rope_base=config.rope_base,
                                   top_k=config.top_k))


def close(got, expected, share):
    return float((got.double() - expected.double()).abs().max()) <= share * float(expected.double().abs().max())


CASES = [(CONFIG, torch.float32, 1e-5), (CONFIG_BF16, torch.bfloat16, 2e-2)]
CHOICE_SLACK = 5e-2  # bf16 activations through the layers before the choice, beside the oracle's FP32


@pytest.fixture
def recorded(monkeypatch):
    """The rows each call of the product's choice returned, in order."""
    calls = []
    choose = kernels.choose_rows

    def recording(*args, **kwargs):
        rows = choose(*args, **kwargs)
        calls.append(rows.cpu())
        return rows

    monkeypatch.setattr(kernels, "choose_rows", recording)
    return calls


def joined(choices, K):
    """Choices of consecutive readings (B, T_i, K_i) joined along T, padded or
    cut to K columns (the columns cut must be -1)."""
    out = []
    for rows in choices:
        assert (rows[..., K:] == -1).all()
        out.append(torch.cat([rows[..., :K], rows.new_full((*rows.shape[:2], max(0, K - rows.shape[2])), -1)], -1))
    return torch.cat(out, 1)


def read_as_the_gpu_chose(ora, rows, ids, choices, dtype, config, **kwargs):
    """The oracle's extend; in bf16 its sparse layers read the GPU's choice
    (one choosing layer, the first), checked against the oracle's own."""
    layer = next(i for i in range(config.layers) if config.chooses(i))
    if dtype == torch.bfloat16:
        ora.given = {layer: joined(choices, max(rows.shape[-1] for rows in choices))}
    scores, _ = ora.extend(ids, rows, **kwargs)
    own, q, keys, positions = ora.choices[layer]
    gpu = joined(choices, own.shape[-1])  # the GPU's columns past the oracle's are -1
    # padding queries (t >= counts[b]) read what no text holds, in the
    # reference too (its window layers see the padding's own entries, the
    # build's rings never hold them): their choices are not compared
    B, T = ids.shape
    counts = torch.as_tensor(kwargs.get("counts", [T] * B))
    gpu = torch.where((torch.arange(T) < counts[:, None])[..., None], gpu, own)
    check_choice(gpu, own, choice_scores(q, keys, positions, config.head_dim ** -0.5, config.window),
                 CHOICE_SLACK if dtype == torch.bfloat16 else 0.0)
    if dtype == torch.float32:  # the same sets
        assert [[set(r[r >= 0].tolist()) for r in query] for query in gpu] == \
            [[set(r[r >= 0].tolist()) for r in query] for query in own]
    return scores


@pytest.mark.parametrize("config, dtype, share", CASES, ids=["fp32", "bf16"])
def test_a_decoder_with_sparse_layers_reads_in_pieces_as_the_oracle_reads_whole(device, recorded, config, dtype,
                                                                                  share):
    gpu, ora = models(config, dtype)
    ids = torch.randint(config.vocab, (2, 90), generator=torch.Generator().manual_seed(1))
    cache = gpu.new_cache(2, capacity=16, widest=16)  # the tables grow; the 40-token piece is read in three
    assert [t is None for t in cache.tables] == [kind == "sparse" for kind in config.kinds]
    got = [gpu.extend(ids[:, a:b].to(device), cache)[0].cpu() for a, b in ((0, 40), (40, 41), (41, 70), (70, 90))]
    assert cache.lengths.tolist() == [90, 90]
    assert len(recorded) == 8  # pieces wider than the rings' 16 tokens read in readings of 16
    want = read_as_the_gpu_chose(ora, ora.new_cache(2), ids, recorded, dtype, config)
    assert close(torch.cat(got, 1), want, share)


@pytest.mark.parametrize("config, dtype, share", CASES, ids=["fp32", "bf16"])
def test_undone_drafts_leave_the_sparse_decoder_as_the_oracle_s(device, recorded, config, dtype, share):
    gpu, ora = models(config, dtype)
    generator = torch.Generator().manual_seed(3)
    texts = [torch.randint(config.vocab, (200,), generator=generator).tolist() for _ in range(2)]
    cache, rows = gpu.new_cache(2, capacity=64), ora.new_cache(2)
    first = torch.tensor([texts[0][:60], texts[1][:60]])
    gpu.extend(first.to(device), cache, counts=[60, 41])
    read_as_the_gpu_chose(ora, rows, first, recorded[-1:], dtype, config, counts=[60, 41])
    place = [60, 41]
    for kept in ([4, 0], [1, 4], [0, 2], [3, 3], [2, 1], [4, 4], [0, 0], [1, 3]) * 2:
        ids = torch.tensor([texts[row][place[row]:place[row] + 4] for row in range(2)])
        drafts = ids.clone()
        for row in range(2):
            drafts[row, kept[row]:] = (ids[row, kept[row]:] + 1 + row) % config.vocab
        got, _ = gpu.extend(drafts.to(device), cache, undoable=True)
        want = read_as_the_gpu_chose(ora, rows, drafts, recorded[-1:], dtype, config, undoable=True)
        assert close(got.cpu(), want, share)
        gpu.undo(cache, kept)
        ora.undo(rows, kept)
        for row in range(2):
            place[row] += kept[row]
        assert cache.lengths.tolist() == rows.lengths.tolist() == place


def test_the_reference_layout_of_layer_kinds_runs(device):
    # window layers around one exact layer, then two groups of an exact layer
    # and two sparse layers (config.py:17-23)
    kinds = layer_kinds(1, 2, 2)
    config = DecoderConfig(layers=len(kinds), d_model=256, heads=4, head_dim=64, ffn=512, vocab=1024, kinds=kinds,
                           window=16, rope_dims=32, top_k=8)
    gpu, ora = models(config, torch.float32, seed=5)
    ids = torch.randint(config.vocab, (1, 70), generator=torch.Generator().manual_seed(6))
    assert close(gpu(ids.to(device)).cpu(), ora.forward(ids), 1e-5)
