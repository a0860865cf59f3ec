"""The decoder's layer kinds on the CPU: the reference's layout
(config.py:17-23), which exact layers choose rows (model.py:134-135), the
weights each kind holds (attention.py:109-215), and the kinds a sparse layer
may not follow; the oracle's sparse layers read the choice."""

import pytest
import torch

from oracle import decoder as oracle_decoder
from wpt_amd.decoder import DecoderConfig, layer_kinds, random_weights


def test_the_reference_layout():
    assert layer_kinds(2, 0, 3) == ("window", "window", "exact", "window", "window")
    assert layer_kinds(1, 2, 2) == ("window", "exact", "window", "exact", "sparse", "sparse", "exact", "sparse",
                                    "sparse")


def test_an_exact_layer_chooses_only_before_a_sparse_layer():
    kinds = layer_kinds(1, 2, 2)
    config = DecoderConfig(layers=len(kinds), d_model=64, heads=2, head_dim=16, ffn=96, vocab=50, kinds=kinds)
    assert [i for i in range(config.layers) if config.chooses(i)] == [3, 6]
    assert config.sparse == (4, 5, 7, 8) and config.windows == (0, 2)


@pytest.mark.parametrize("kinds, layers", [(("sparse", "exact"), 2), (("exact", "window", "sparse"), 3),
                                           (("exact", "dense"), 2), (("exact",), 2)])
def test_kinds_a_decoder_cannot_have(kinds, layers):
    with pytest.raises(ValueError):
        DecoderConfig(layers=layers, d_model=64, heads=2, head_dim=16, ffn=96, vocab=50, kinds=kinds)


def test_each_kind_holds_its_own_weights():
    config = DecoderConfig(layers=3, d_model=64, heads=2, head_dim=16, ffn=96, vocab=50,
                           kinds=("window", "exact", "sparse"))
    w = random_weights(config)
    assert {"layers.0.qkv", "layers.0.gate", "layers.0.sink", "layers.0.k_norm"} <= set(w)
    assert {"layers.1.qkv", "layers.1.k_norm"} <= set(w) and "layers.1.gate" not in w
    assert {"layers.2.q", "layers.2.gate", "layers.2.sink"} <= set(w)
    assert "layers.2.qkv" not in w and "layers.2.k_norm" not in w
    assert w["layers.2.q"].shape == (2 * 16, 64)


def test_the_oracle_s_sparse_layer_reads_the_choice():
    # a query with at most top_k candidates outside the window reads all of
    # them, whatever top_k; past that, a smaller choice changes the scores
    config = DecoderConfig(layers=2, d_model=64, heads=2, head_dim=16, ffn=96, vocab=50, kinds=("exact", "sparse"))
    w = random_weights(config, std=0.2)
    for name in ("layers.1.sink",):
        w[name] = torch.zeros_like(w[name])
    window, top_k = 8, 4
    ids = torch.randint(50, (1, 40), generator=torch.Generator().manual_seed(0))

    def scores(k):
        return oracle_decoder.Decoder(w, 2, 2, 16, kinds=config.kinds, window=window, top_k=k).forward(ids)[0]

    few, every = scores(top_k), scores(10 ** 6)
    last_whole = window - 1 + top_k  # position p has p - window + 1 candidates
    assert torch.allclose(few[:last_whole + 1], every[:last_whole + 1], rtol=0, atol=1e-5)
    assert (few[last_whole + 1:] - every[last_whole + 1:]).abs().amax(-1).min() > 1e-4
