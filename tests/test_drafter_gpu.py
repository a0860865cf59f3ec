"""The DSpark-shaped drafter on the GPU (wpt_amd.drafter) against the oracle
drafter on the CPU, with the same weights: its attention (the row-block
kernel over [context ; block] at the chosen positions) against the reference
mask's dense attention, bf16 within 1e-2; the backbone's scores within 2e-2;
the drafts' distributions and confidences along the tokens it drew; and the
Writer driving the decoder with it (its features context, the cache holding
each row's text)."""

import pytest
import torch

from oracle import attention as oracle_attention
from oracle import drafter as oracle_drafter
from tests.formulas import relative_error
from wpt_amd import drafter as gpu_drafter
from wpt_amd import kernels
from wpt_amd.decoder import DecoderConfig, MQADecoder, random_weights
from wpt_amd.writer import Writer

pytestmark = pytest.mark.gpu

CONFIG = DecoderConfig(layers=4, d_model=256, heads=16, head_dim=128, ffn=512, vocab=1024)
LENGTHS = [0, 3, 60, 127, 128, 400]


def setup(device, seed=0):
    weights = random_weights(CONFIG, seed=seed, std=0.05)
    model = MQADecoder(CONFIG, weights, dtype=torch.bfloat16, device=device)
    config = gpu_drafter.DrafterConfig.for_model(CONFIG, features=(1, 3), layers=2)
    w = gpu_drafter.random_drafter_weights(CONFIG, config, seed=seed + 1, std=0.05)
    w["markov_out"] = torch.randn(w["markov_out"].shape, generator=torch.Generator().manual_seed(seed + 2)) * 0.05
    gpu = gpu_drafter.Drafter(model, config, w)
    ora = oracle_drafter.Drafter({k: v.to(torch.bfloat16).float() if k not in ("markov_in", "markov_out")
                                  and not k.endswith(("norm", "sink", "bias", "temperatures", "confidence")) else v
                                  for k, v in w.items()},
                                 weights["embedding"].to(torch.bfloat16), weights["head"].to(torch.bfloat16),
                                 config.layers, CONFIG.heads, CONFIG.head_dim)
    return model, config, gpu, ora


def test_the_chosen_positions_read_what_the_reference_mask_shows(device):
    R, count, H, c = len(LENGTHS), 5, 16, 128
    W = oracle_drafter.WINDOW
    generator = torch.Generator().manual_seed(11)
    q = torch.randn(R, count, H, c, generator=generator).to(torch.bfloat16)
    block = torch.randn(R, count, 2 * c, generator=generator).to(torch.bfloat16)
    context = torch.randn(R, W, 2 * c, generator=generator).to(torch.bfloat16)
    sink = torch.randn(H, generator=generator)
    lengths = torch.tensor(LENGTHS)
    table = torch.cat([block, context], 1)  # the reference's order
    expected = oracle_attention.dense_attention(q, table[..., :c], table[..., c:], sink,
                                                oracle_drafter.visible(lengths, count), c ** -0.5)
    flat = torch.cat([context, block], 1).to(device)  # the kernel's order
    places, span = gpu_drafter.visible_positions(lengths.to(device), count)
    got = kernels.verify_attention(q.to(device), flat[..., :c], flat[..., c:], places, c ** -0.5, window=span,
                                   sink=sink.to(device))
    assert relative_error(got.float().cpu(), expected) < 1e-2


def test_the_backbone_matches_the_oracle(device):
    model, config, gpu, ora = setup(device)
    R = len(LENGTHS)
    generator = torch.Generator().manual_seed(12)
    context = torch.randn(R, oracle_drafter.WINDOW, 2 * CONFIG.d_model, generator=generator)
    anchors = torch.randint(CONFIG.vocab, (R,), generator=generator)
    lengths = torch.tensor(LENGTHS)
    for count in (1, 3, 5):
        h, U = gpu.backbone(context.to(device), lengths.to(device), anchors.to(device), count)
        h_o, U_o = ora.backbone(context.to(torch.bfloat16).float(), lengths, anchors, count)
        assert relative_error(U.cpu(), U_o) < 2e-2, count
        assert relative_error(h.cpu(), h_o) < 2e-2, count


def test_drafts_follow_the_oracle_distributions(device):
    model, config, gpu, ora = setup(device, seed=3)
    R, count = len(LENGTHS), 4
    generator = torch.Generator().manual_seed(13)
    context = torch.randn(R, oracle_drafter.WINDOW, 2 * CONFIG.d_model, generator=generator)
    anchors = torch.randint(CONFIG.vocab, (R,), generator=generator).tolist()
    probabilities = lambda s: torch.softmax(s.float() / 0.8, -1)  # noqa: E731
    tokens, q, confidences = gpu.draft(model, [[a] for a in anchors], (context.to(device), torch.tensor(LENGTHS,
                                       device=device)), count, probabilities,
                                       torch.Generator(device=device).manual_seed(14))
    assert tokens.shape == (R, count) and q.shape == (R, count, CONFIG.vocab) and confidences.shape == (R, count)
    expected_q, expected_c = ora.distributions(context.to(torch.bfloat16).float(), torch.tensor(LENGTHS),
                                               torch.tensor(anchors), tokens.cpu(), probabilities)
    assert (q.cpu() - expected_q).abs().max() < 2e-2 * expected_q.max()
    assert (confidences.cpu() - expected_c).abs().max() < 1e-2
    assert torch.allclose(q.sum(-1).cpu(), torch.ones(R, count), atol=1e-4)


def test_the_writer_drafts_with_it(device):
    # the drafter drives the speculative writer: its context from the
    # decoder's features (layers 1 and 3), rows with tool inputs caught up
    model, config, gpu, _ = setup(device, seed=5)
    writer = Writer(model, [3, 5, 7, 9], 3, temperature=1.0, top_k=None, draft=4,
                    generator=torch.Generator(device=device).manual_seed(6), drafter=gpu)
    for inputs in ({}, {1: [11, 12]}, {}, {}):
        out = writer.write(inputs, {0: 5, 1: 5, 2: 5})
        assert all(1 <= len(tokens) <= 5 for tokens in out.values())
    assert writer.rounds == 4 and writer.verified == 4 * 4 * 3
    assert writer.cache.lengths.tolist() == [len(h) - 1 for h in writer.histories]
    assert writer.context.shape == (3, oracle_drafter.WINDOW, 2 * CONFIG.d_model)


def test_captured_writer_rounds_write_what_eager_rounds_write(device):
    # the drafter's backbone and the Writer's steady rounds from HIP graphs
    # (capture=True) against both eager, from generators seeded alike: the
    # same tokens round after round, a round with tool inputs (eager either
    # way) in between, and the same cache lengths and generator state after
    model, config, _, _ = setup(device, seed=5)
    w = gpu_drafter.random_drafter_weights(CONFIG, config, seed=6, std=0.05)
    runs = []
    for capture in (False, True):
        drafter = gpu_drafter.Drafter(model, config, w, capture=capture)
        generator = torch.Generator(device=device).manual_seed(9)
        writer = Writer(model, [3, 5, 7, 9], 4, temperature=1.0, top_k=None, draft=4, generator=generator,
                        drafter=drafter, capture=capture)
        out = [writer.write(inputs, {row: 5 for row in range(4)})
               for inputs in ({}, {}, {2: [11, 12]}, {}, {}, {})]
        runs.append((out, writer.cache.lengths.tolist(), generator.get_state(), writer.context.clone()))
        if capture:
            assert writer._reads and drafter._graphs  # the graphs were captured and replayed
    (eager, lengths_e, state_e, context_e), (captured, lengths_c, state_c, context_c) = runs
    assert captured == eager
    assert lengths_c == lengths_e and torch.equal(state_c, state_e) and torch.equal(context_c, context_e)


def test_a_captured_backbone_replays_the_eager_one(device):
    model, config, gpu, _ = setup(device, seed=3)
    captured = gpu_drafter.Drafter(model, config, {k: v for k, v in gpu.w.items()}, capture=True)
    R, count = len(LENGTHS), 4
    generator = torch.Generator(device=device).manual_seed(1)
    for call in range(3):  # the first call runs eagerly and captures; the others replay
        features = torch.randn(R, gpu_drafter.WINDOW, len(config.features) * CONFIG.d_model, generator=generator,
                               device=device)
        lengths = torch.tensor(LENGTHS, device=device) + call
        anchors = torch.randint(CONFIG.vocab, (R,), generator=generator, device=device)
        h, U = gpu.backbone(features, lengths, anchors, count)
        h2, U2 = captured._replayed(features, lengths, anchors, count)
        assert torch.equal(h, h2) and torch.equal(U, U2), f"call {call}"
