"""Pins the oracle drafter (CPU) by what the reference's drafter fixes
(packages/wpt-model/src/wpt_model/drafter.py):

* the mask (:173-176) against the rule written out one entry at a time:
  place k sees every place of the block and context entry j iff its position
  lengths - WINDOW + j is >= 0 and within WINDOW tokens before the place;
* the backbone with every sublayer's output projection at zero: the stream
  is the block's input, so U is the head over the final norm of the anchor's
  embedding at place 0 and of the mask vector after it;
* the block reads itself both ways (DFlash's parallel block): place 0's
  scores move with the mask vector the later places hold;
* the Markov head at its initial zero output (:170): q = probabilities(U);
* the confidence head with zero weights: sigmoid(bias / T_k) (:226, STS's T);
* feature_layers' known answers (:80-87, the rule written in its docstring)."""

import torch

from oracle import drafter as oracle_drafter
from wpt_amd import drafter as gpu_drafter
from wpt_amd.decoder import DecoderConfig

CONFIG = DecoderConfig(layers=4, d_model=64, heads=4, head_dim=64, ffn=96, vocab=50)


def pieces(seed=0, layers=2):
    config = gpu_drafter.DrafterConfig.for_model(CONFIG, features=(1, 3), layers=layers)
    w = gpu_drafter.random_drafter_weights(CONFIG, config, seed=seed)
    generator = torch.Generator().manual_seed(seed + 1)
    embedding = torch.randn(CONFIG.vocab, CONFIG.d_model, generator=generator)
    head = torch.randn(CONFIG.vocab, CONFIG.d_model, generator=generator) * 0.2
    return config, w, embedding, head


def oracle(w, embedding, head, layers=2):
    return oracle_drafter.Drafter(w, embedding, head, layers, CONFIG.heads, CONFIG.head_dim, rope_dims=32)


def test_the_mask_is_the_reference_rule_entry_by_entry():
    W = oracle_drafter.WINDOW
    lengths = torch.tensor([0, 3, 127, 128, 300])
    count = 5
    got = oracle_drafter.visible(lengths, count)
    for r, length in enumerate(lengths.tolist()):
        for k in range(count):
            for j in range(count):
                assert got[r, k, j]
            for j in range(W):
                position = length - W + j
                assert bool(got[r, k, count + j]) == (position >= 0 and position > length + k - W), (r, k, j)


def test_zero_sublayers_leave_the_block_input_to_the_head():
    config, w, embedding, head = pieces()
    for i in range(config.layers):
        w[f"layers.{i}.out"].zero_()
        w[f"layers.{i}.down"].zero_()
    d = oracle(w, embedding, head)
    anchors = torch.tensor([4, 9])
    context = torch.randn(2, oracle_drafter.WINDOW, 2 * CONFIG.d_model, generator=torch.Generator().manual_seed(3))
    _, U = d.backbone(context, torch.tensor([10, 200]), anchors, 4)
    final = w["final_norm"]
    first = oracle_drafter.rms_norm(embedding[anchors], final) @ head.T
    later = oracle_drafter.rms_norm(w["mask"], final) @ head.T
    assert torch.allclose(U[:, 0], first, atol=1e-5)
    assert torch.allclose(U[:, 1:], later.expand(2, 3, -1), atol=1e-5)


def test_the_block_reads_itself_both_ways():
    config, w, embedding, head = pieces(seed=4)
    context = torch.randn(1, oracle_drafter.WINDOW, 2 * CONFIG.d_model, generator=torch.Generator().manual_seed(5))
    anchors = torch.tensor([7])
    _, before = oracle(w, embedding, head).backbone(context, torch.tensor([50]), anchors, 3)
    w["mask"] = w["mask"] + 1.0
    _, after = oracle(w, embedding, head).backbone(context, torch.tensor([50]), anchors, 3)
    assert (after[:, 0] - before[:, 0]).abs().max() > 1e-3


def test_the_markov_head_at_its_start_and_the_confidence_closed_form():
    config, w, embedding, head = pieces(seed=6)
    w["confidence"].zero_()
    w["confidence_bias"].fill_(0.7)
    w["temperatures"] = torch.tensor([1.0, 2.0, 0.5, 1.5, 3.0])
    d = oracle(w, embedding, head)
    context = torch.randn(2, oracle_drafter.WINDOW, 2 * CONFIG.d_model, generator=torch.Generator().manual_seed(7))
    lengths, anchors = torch.tensor([5, 140]), torch.tensor([1, 2])
    drawn = torch.tensor([[3, 4, 5], [6, 7, 8]])
    probabilities = lambda s: torch.softmax(s / 0.8, -1)  # noqa: E731
    q, confidences = d.distributions(context, lengths, anchors, drawn, probabilities)
    _, U = d.backbone(context, lengths, anchors, 3)
    assert torch.allclose(q, probabilities(U), atol=1e-7)  # zero Markov output: no bias
    expected = torch.sigmoid(torch.tensor(0.7) / w["temperatures"][:3])
    assert torch.allclose(confidences, expected.expand(2, 3))


def test_feature_layers_known_answers():
    assert gpu_drafter.feature_layers(24) == (2, 7, 12, 17, 22)
    assert gpu_drafter.feature_layers(4) == (2,)
    assert gpu_drafter.feature_layers(12, count=1) == (2,)
    assert gpu_drafter.feature_layers(10, count=3) == (2, 5, 8)
