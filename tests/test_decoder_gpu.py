"""The MQA decoder's generation protocol on the GPU (KV append, verify
attention, undo) against the oracle decoder on the CPU, the plumbing
workload's greedy verify step bit-exact, the Writer, and the verify step
replayed from a HIP graph.  Scores: FP32 within 1e-5 of the largest expected
magnitude, bf16 within 2e-2; token decisions exact."""

import pytest
import torch

from oracle import decoder as oracle_decoder
from oracle import sampling as oracle_sampling
from wpt_amd.decoder import PLUMBING, DecoderConfig, MQADecoder, random_weights
from wpt_amd import sampling
from wpt_amd.step import VerifyStep, prefill
from wpt_amd.writer import Writer

pytestmark = pytest.mark.gpu

SMALL_BF16 = DecoderConfig(layers=2, d_model=256, heads=16, head_dim=128, ffn=512, vocab=1024)


def models(config, dtype, seed=0, std=0.02):
    w = random_weights(config, seed=seed, std=std)
    return MQADecoder(config, w, dtype=dtype), oracle_decoder.Decoder(w, config.layers, config.heads, config.head_dim)


def close(got, expected, share):
    return float((got.double() - expected.double()).abs().max()) <= share * float(expected.double().abs().max())


def test_plumbing_scores_read_in_pieces_match_the_oracle_whole_text(device):
    gpu, ora = models(PLUMBING, torch.float32)
    ids = torch.randint(PLUMBING.vocab, (2, 69), generator=torch.Generator().manual_seed(1))
    cache = gpu.new_cache(2, capacity=16)  # grows while reading
    got = [gpu.extend(ids[:, a:b].to(device), cache)[0].cpu() for a, b in ((0, 37), (37, 38), (38, 64), (64, 69))]
    assert cache.lengths.tolist() == [69, 69] and cache.capacity >= 69
    assert close(torch.cat(got, 1), ora.forward(ids), 1e-5)


def greedy_text(ora, prompt, n):
    """The oracle's greedy continuation of prompt, n tokens."""
    text = list(prompt)
    for _ in range(n):
        text.append(int(ora.forward(torch.tensor([text]))[0, -1].argmax()))
    return text[len(prompt):]


@pytest.mark.parametrize("planted", [0, 2, 4])
def test_plumbing_greedy_verify_step_is_bit_exact(device, planted):
    # the CPU-runnable plumbing workload: 4 layers, d_model 256, 4 query
    # heads, 1 KV head, head width 64, vocab 8192, FP32; a prompt of 64
    # tokens; a chain of 4 uniform drafts, the first `planted` of them the
    # model's own greedy choices, verified greedily
    gpu, ora = models(PLUMBING, torch.float32)
    generator = torch.Generator().manual_seed(0)
    prompt = torch.randint(PLUMBING.vocab, (64,), generator=generator).tolist()
    drafts = torch.randint(PLUMBING.vocab, (4,), generator=generator)
    drafts[:planted] = torch.tensor(greedy_text(ora, prompt, 4)[:planted], dtype=torch.long)
    feeds = torch.tensor([[prompt[-1]] + drafts.tolist()])
    # the oracle: read the prompt but its last token, then the step
    rows = ora.new_cache(1)
    ora.extend(torch.tensor([prompt[:-1]]), rows)
    expected_scores, _ = ora.extend(feeds, rows, undoable=True)
    expected = oracle_sampling.greedy_chain(expected_scores, drafts[None], [4])[0]
    ora.undo(rows, [len(expected)])
    # the GPU
    cache = gpu.new_cache(1, capacity=128)
    gpu.extend(torch.tensor([prompt[:-1]], device=device), cache)
    scores, _ = gpu.extend(feeds.to(device), cache, undoable=True)
    tokens, counts = sampling.greedy_chain(scores, drafts[None].to(device))
    got = sampling.written(tokens, counts)[0]
    gpu.undo(cache, counts.long())
    top2 = expected_scores[0].topk(2, -1).values
    assert float((top2[:, 0] - top2[:, 1]).min()) > 1e-4 * float(expected_scores.abs().max())  # no near ties
    assert got == expected and len(got) == planted + 1
    assert cache.lengths.tolist() == rows.lengths.tolist() == [63 + len(expected)]
    assert close(scores.cpu(), expected_scores, 1e-5)


@pytest.mark.parametrize("config, dtype, share", [(PLUMBING, torch.float32, 1e-5), (SMALL_BF16, torch.bfloat16, 2e-2)])
def test_undoing_rejected_drafts_leaves_only_the_kept_tokens(device, config, dtype, share):
    # the reference's undo contract (test_cache.py:206-238): every round
    # reads 4 drafts per row and keeps a pattern of them
    gpu, ora = models(config, dtype)
    generator = torch.Generator().manual_seed(3)
    texts = [torch.randint(config.vocab, (200,), generator=generator).tolist() for _ in range(2)]
    cache = gpu.new_cache(2, capacity=64)
    gpu.extend(torch.tensor([t[:60] for t in texts], device=device), cache)
    place, got = [60, 60], [[], []]
    for kept in ([4, 0], [1, 4], [0, 2], [3, 3], [2, 1], [4, 4], [0, 0], [1, 3]) * 3:
        ids = torch.tensor([texts[row][place[row]:place[row] + 4] for row in range(2)])
        drafts = ids.clone()
        for row in range(2):
            drafts[row, kept[row]:] = (ids[row, kept[row]:] + 1 + row) % config.vocab
        scores, _ = gpu.extend(drafts.to(device), cache, undoable=True)
        gpu.undo(cache, kept)
        for row in range(2):
            got[row].append(scores[row, :kept[row]].cpu())
            place[row] += kept[row]
    assert cache.lengths.tolist() == place
    for row in range(2):
        whole = ora.forward(torch.tensor([texts[row][:place[row]]]))[0]
        assert close(torch.cat(got[row]), whole[60:], share)


def test_bf16_rows_at_different_places_match_the_oracle(device):
    gpu, ora = models(SMALL_BF16, torch.bfloat16)
    generator = torch.Generator().manual_seed(5)
    prompt = torch.randint(SMALL_BF16.vocab, (70,), generator=generator).tolist()
    texts = [prompt + torch.randint(SMALL_BF16.vocab, (n,), generator=generator).tolist() for n in (30, 5, 17)]
    shared = gpu.new_cache(1, capacity=32)
    gpu.extend(torch.tensor([prompt], device=device), shared)
    cache = shared.select([0, 0, 0])
    got, place = [[] for _ in texts], [len(prompt)] * 3
    for counts in ([1, 1, 1], [10, 0, 7], [3, 4, 1], [16, 0, 8]):
        ids = torch.zeros(3, max(counts), dtype=torch.long)
        for row, count in enumerate(counts):
            ids[row, :count] = torch.tensor(texts[row][place[row]:place[row] + count])
        scores, _ = gpu.extend(ids.to(device), cache, counts)
        for row, count in enumerate(counts):
            got[row].append(scores[row, :count].cpu())
            place[row] += count
    for row, text in enumerate(texts):
        assert close(torch.cat(got[row]), ora.forward(torch.tensor([text]))[0, len(prompt):], 2e-2)
    assert shared.lengths.tolist() == [len(prompt)]


class Itself:
    """The model as its own drafter (the reference's test_sampling.py:82-95):
    its drafts are always kept."""
    features, window = (), 0

    def draft(self, model, histories, context, count, probabilities, generator):
        tokens, distributions = [], []
        for history in histories:
            history = list(history)
            for _ in range(count):
                p = probabilities(model(torch.tensor([history]))[0, -1])
                history.append(int(torch.multinomial(p, 1, generator=generator)))
                distributions.append(p)
            tokens.append(history[-count:])
        return torch.tensor(tokens), torch.stack(distributions).view(len(histories), count, -1), None


class Uniform:
    features, window = (), 0

    def draft(self, model, histories, context, count, probabilities, generator):
        V = model.config.vocab
        tokens = torch.randint(V, (len(histories), count), generator=generator, device=generator.device)
        return tokens, torch.full((len(histories), count, V), 1.0 / V, device=generator.device), None


def reference_rounds(model, prompt, rows, calls, temperature, top_k, generator, drafter, draft, inputs=None,
                     stops=()):
    """The reference Writer's speculative rounds (__init__.py:71-233, no
    features or scheduler), restated with the oracle's rule drawing lazily
    from `generator` (oracle.sampling.LazyDraws): the tokens of each call.
    inputs: per call, {row: tokens read before writing} (None: none)."""
    device = generator.device
    one = model.new_cache(1)
    if len(prompt) > 1:
        model.extend(torch.tensor([prompt[:-1]], device=device), one)
    cache = one.select([0] * rows)
    pending, histories = [[prompt[-1]] for _ in range(rows)], [list(prompt) for _ in range(rows)]

    def probabilities(scores):
        return oracle_sampling.probabilities(scores, temperature, top_k)

    out = []
    for call, limits in enumerate(calls):
        rs = sorted(limits)
        for r, tokens in (inputs[call] if inputs else {}).items():
            pending[r] = pending[r] + list(tokens)
            histories[r] = histories[r] + list(tokens)
        drafted, q, _ = drafter.draft(model, [histories[r] for r in rs], None, draft, probabilities, generator)
        drafted, q = drafted.to(device), q.to(device).float()
        caps = [min(draft, limits[r] - 1) for r in rs]
        feeds = [[] for _ in range(rows)]
        for i, r in enumerate(rs):
            feeds[r] = pending[r] + drafted[i, :caps[i]].tolist()
        width = max(len(f) for f in feeds)
        ids = torch.tensor([f + [0] * (width - len(f)) for f in feeds], device=device)
        scores = model.extend(ids, cache, [len(f) for f in feeds], True)[0][rs]
        written, kept = {}, [0] * rows
        for i, r in enumerate(rs):
            first = len(pending[r]) - 1
            p = probabilities(scores[i, first:first + caps[i] + 1])
            tokens = oracle_sampling.accept_row(p, q[i], drafted[i], caps[i], oracle_sampling.LazyDraws(generator))
            written[r] = oracle_sampling.cut(tokens, set(stops), limits[r])
            kept[r] = first + len(written[r])
        model.undo(cache, kept)
        for r, tokens in written.items():
            histories[r] += tokens
            pending[r] = [tokens[-1]]
        out.append(written)
    return out


@pytest.mark.parametrize("top_k", [None, 40])
def test_a_seeded_writer_writes_the_reference_writer_s_tokens(device, top_k):
    # the same model, drafter and seed: the Writer (its draws replayed from the
    # generator's stream on the GPU) and the reference's rounds write the same
    # tokens, and leave their generators at the same offset
    gpu, _ = models(PLUMBING, torch.float32, std=0.05)
    prompt, calls = [0, 5, 7, 9], [{0: 4, 1: 4, 2: 4}, {0: 2, 2: 5}, {0: 4, 1: 1, 2: 4}, {0: 4, 1: 4, 2: 4}]
    reference = torch.Generator(device=device).manual_seed(21)
    expected = reference_rounds(gpu, prompt, 3, calls, 1.0, top_k, reference, Uniform(), 3)
    mine = torch.Generator(device=device).manual_seed(21)
    writer = Writer(gpu, prompt, 3, temperature=1.0, top_k=top_k, generator=mine, drafter=Uniform(), draft=3)
    assert [writer.write({}, limits) for limits in calls] == expected
    assert torch.equal(mine.get_state(), reference.get_state())


def test_a_seeded_writer_with_inputs_limits_and_stops_writes_the_reference_writer_s_tokens(device):
    # rows that read tool inputs first (their first new token scored after
    # them), limits below a full round (fewer drafts verified), a stop token,
    # and a call that leaves a row out: still the reference's tokens and
    # generator state
    gpu, _ = models(PLUMBING, torch.float32, std=0.05)
    prompt = [0, 5, 7, 9]
    calls = [{0: 4, 1: 4, 2: 4}, {0: 2, 2: 5}, {0: 4, 1: 1, 2: 3}, {1: 4, 2: 4}, {0: 4, 1: 4, 2: 4}]
    inputs = [{}, {2: [11, 12, 13]}, {0: [4]}, {1: [21, 22], 2: [8]}, {}]
    reference = torch.Generator(device=device).manual_seed(33)
    expected = reference_rounds(gpu, prompt, 3, calls, 0.9, 40, reference, Uniform(), 3, inputs, stops=(17,))
    mine = torch.Generator(device=device).manual_seed(33)
    writer = Writer(gpu, prompt, 3, temperature=0.9, top_k=40, generator=mine, drafter=Uniform(), draft=3,
                    stops=(17,))
    assert [writer.write(given, limits) for given, limits in zip(inputs, calls)] == expected
    assert torch.equal(mine.get_state(), reference.get_state())


def test_a_seeded_writer_without_drafts_samples_as_the_reference_does(device):
    # Writer._sample (__init__.py:181-182): one multinomial over every row's
    # distribution at its last token
    gpu, _ = models(PLUMBING, torch.float32, std=0.05)
    prompt = [1, 2, 3]
    mine = torch.Generator(device=device).manual_seed(8)
    writer = Writer(gpu, prompt, 4, temperature=0.7, top_k=40, generator=mine)
    got = writer.write({}, {0: 1, 1: 1, 3: 1})
    reference = torch.Generator(device=device).manual_seed(8)
    one = gpu.new_cache(1)  # the reading the Writer makes: the prompt but its last token, then each row's last
    gpu.extend(torch.tensor([prompt[:-1]], device=device), one)
    ids = torch.tensor([[prompt[-1]]] * 4, device=device)
    scores = gpu.extend(ids, one.select([0] * 4), [1, 1, 0, 1])[0][[0, 1, 3], 0]
    p = oracle_sampling.probabilities(scores, 0.7, 40)
    expected = torch.multinomial(p, 1, generator=reference)[:, 0].tolist()
    assert got == {0: [expected[0]], 1: [expected[1]], 3: [expected[2]]}
    assert torch.equal(mine.get_state(), reference.get_state())


def test_the_writer_keeps_every_draft_of_the_model_itself(device):
    gpu, _ = models(PLUMBING, torch.float32, std=0.05)
    writer = Writer(gpu, [0, 5, 7], 2, temperature=1.0, top_k=None,
                    generator=torch.Generator(device=device).manual_seed(0), drafter=Itself())
    written = writer.write({}, {0: 100, 1: 3})
    assert len(written[0]) == 5 + 1 and len(written[1]) == 3
    assert writer.accepted == 5 + 2 and writer.verified == 5 + 2 and writer.rounds == 1
    stop = written[0][1]
    writer = Writer(gpu, [0, 5, 7], 2, temperature=1.0, top_k=None,
                    generator=torch.Generator(device=device).manual_seed(0), drafter=Itself(), stops=[stop])
    assert writer.write({}, {0: 100, 1: 3})[0] == written[0][:written[0].index(stop) + 1]


def test_the_writer_s_cache_holds_each_row_s_text(device):
    # after speculative steps with uniform drafts, each row's cache reads as
    # its whole text does (the reference's test_sampling.py:112-121)
    gpu, _ = models(PLUMBING, torch.float32, std=0.05)
    writer = Writer(gpu, [0, 5, 7, 9], 3, temperature=1.0, top_k=None,
                    generator=torch.Generator(device=device).manual_seed(1), drafter=Uniform())
    for _ in range(4):
        writer.write({1: [11, 12]} if _ == 2 else {}, {row: 5 for row in range(3)})
    for row in range(3):
        history = writer.histories[row]
        assert int(writer.cache.lengths[row]) == len(history) - 1
    ids = torch.tensor([[h[-1]] for h in writer.histories], device=device)
    scores, _ = gpu.extend(ids, writer.cache)
    for row in range(3):
        whole = gpu(torch.tensor([writer.histories[row]], device=device))[0, -1]
        assert close(scores[row, 0].cpu(), whole.cpu(), 1e-5)


class Confident(Uniform):
    """Uniform drafts with given confidences, for the prefix scheduler."""

    def __init__(self, confidences):
        self.confidences = confidences

    def draft(self, model, histories, context, count, probabilities, generator):
        tokens, q, _ = super().draft(model, histories, context, count, probabilities, generator)
        return tokens, q, torch.tensor(self.confidences[:len(histories)], device=q.device)[:, :count]


class Recording(Uniform):
    """Uniform drafts; reads layers 0, 2 and 4 (the final hidden states) of
    the model, keeps every context it is given."""
    features, window = (0, 2, 4), 5

    def __init__(self):
        self.seen = []

    def draft(self, model, histories, context, count, probabilities, generator):
        found, lengths = context
        self.seen.append((found.clone(), lengths.clone(), [list(h) for h in histories]))
        return super().draft(model, histories, context, count, probabilities, generator)


def test_the_writer_gives_a_feature_drafter_the_last_window_of_features(device):
    # the reference's _remember / _catch_up (wpt_inference/__init__.py:140-152,
    # 184-200): before each draft, a row's context is the features of the last
    # `window` tokens its cache holds (zeros before the text), however the
    # tokens were read: the prompt, catch-up reads of tool inputs, verified drafts
    gpu, _ = models(PLUMBING, torch.float32, std=0.05)
    drafter = Recording()
    writer = Writer(gpu, [3, 5, 7], 3, temperature=1.0, top_k=None,
                    generator=torch.Generator(device=device).manual_seed(4), drafter=drafter, draft=3)
    for call, inputs in enumerate(({}, {1: [11, 12, 13]}, {}, {0: [2], 2: [9, 8]}, {}, {})):
        writer.write(inputs, {0: 4, 1: 4, 2: 4})
    assert len(drafter.seen) == 6
    D = PLUMBING.d_model
    for found, lengths, histories in drafter.seen:
        for row, history in enumerate(histories):
            held = int(lengths[row])
            assert held == len(history) - 1  # every token but the anchor has been read
            _, _, whole = gpu.extend(torch.tensor([history[:-1]], device=device), gpu.new_cache(1), features=(0, 2, 4))
            want = torch.zeros(drafter.window, 3 * D, device=device)
            last = whole[0, -drafter.window:]
            want[drafter.window - last.shape[0]:] = last
            assert close(found[row], want, 1e-5), f"row {row} after {held} tokens"
    # a one-token prompt starts from zeros
    first = Recording()
    Writer(gpu, [3], 2, generator=torch.Generator(device=device).manual_seed(5), drafter=first, draft=2).write(
        {}, {0: 3, 1: 3})
    assert not first.seen[0][0].any() and first.seen[0][1].tolist() == [0, 0]


def test_the_writer_verifies_the_drafts_the_scheduler_admits(device):
    # the reference's known answer (test_sampling.py:236): passes cost the
    # same up to 3 tokens per row, then 20 % more; row 0's confident first
    # drafts are verified, its unlikely ones not, row 1 only to its cap
    gpu, _ = models(PLUMBING, torch.float32, std=0.05)
    costs = [1.0, 1.0, 1.0, 1.2, 1.2, 1.2]
    outcomes = []
    writer = Writer(gpu, [0, 5, 7], 2, temperature=1.0, top_k=None, costs=costs, outcomes=outcomes,
                    generator=torch.Generator(device=device).manual_seed(3),
                    drafter=Confident([[0.9, 0.9, 0.9, 0.1, 0.1], [0.5] * 5]))
    written = writer.write({}, {0: 100, 1: 2})
    assert writer.verified == 2 + 1 and [len(c) for c, _ in outcomes] == [2, 1]
    assert 1 <= len(written[0]) <= 3 and 1 <= len(written[1]) <= 2
    assert writer.cache.lengths.tolist() == [len(h) - 1 for h in writer.histories]


def test_measured_pass_times_feed_the_scheduler(device):
    from wpt_amd import scheduling

    gpu, _ = models(PLUMBING, torch.float32)
    costs = scheduling.measure_costs(gpu, rows=2, draft=4, context=32, repeats=2)
    assert len(costs) == 5 and all(0 < t < 1.0 for t in costs)
    setup = scheduling.costs_setup(PLUMBING, 2, 4, device)
    assert scheduling.replayed_costs(scheduling.costs_file(costs, setup), setup) == costs


def test_a_wide_bf16_reading_matches_reading_in_pieces(device):
    # more than 512 rows take the product then SwiGLU of its interleaved
    # halves, fewer the fused product: the same scores either way
    gpu, _ = models(SMALL_BF16, torch.bfloat16)
    ids = torch.randint(SMALL_BF16.vocab, (2, 300), generator=torch.Generator().manual_seed(9)).to(device)
    whole = gpu(ids)  # 600 rows in one reading
    cache = gpu.new_cache(2, capacity=300)
    pieces = torch.cat([gpu.extend(ids[:, a:a + 100], cache)[0] for a in range(0, 300, 100)], 1)  # 200 rows each
    assert close(pieces.cpu(), whole.cpu(), 2e-2)


def test_a_writer_without_drafts_samples_one_token_per_call(device):
    gpu, _ = models(PLUMBING, torch.float32)
    writer = Writer(gpu, [1, 2, 3], 2, generator=torch.Generator(device=device).manual_seed(2))
    for _ in range(3):
        out = writer.write({}, {0: 1, 1: 1})
        assert all(len(tokens) == 1 for tokens in out.values())
    assert [len(h) for h in writer.histories] == [6, 6]
    assert writer.cache.lengths.tolist() == [5, 5]


def test_a_captured_verify_step_replays_as_the_eager_step(device):
    # greedy steps (no random draws): eager steps on one cache, graph replays
    # on another with the same prefill, eager work between the replays
    config = SMALL_BF16
    w = random_weights(config, seed=7, std=0.05)
    B, k = 4, 4
    ids = torch.randint(config.vocab, (B, 90), generator=torch.Generator().manual_seed(8)).to(device)
    runs = []
    for captured in (False, True):
        model = MQADecoder(config, w, dtype=torch.bfloat16)
        cache = model.new_cache(B, capacity=256)
        prefill(model, cache, ids[:, :-1], chunk=40)
        step = VerifyStep(model, cache, k, greedy=True)
        step.feeds[:, 0] = ids[:, -1]
        step.feeds[:, 1:] = torch.randint(config.vocab, (B, k), generator=torch.Generator().manual_seed(9)).to(device)
        out = []
        if captured:
            step.capture(warmup=1)  # one eager step on a side stream, then the capture (which runs nothing)
            for _ in range(5):
                tokens, counts = step.replay()
                out.append((tokens.clone(), counts.clone(), cache.lengths.clone()))
                torch.zeros(1000, device=device).sum()  # eager work between replays
                torch.cuda.synchronize()
        else:
            for _ in range(6):  # the first step is the captured run's warmup
                tokens, counts = step.run()
                out.append((tokens.clone(), counts.clone(), cache.lengths.clone()))
            out = out[1:]
        runs.append(out)
    for (te, ce, le), (tg, cg, lg) in zip(*runs):
        assert torch.equal(te, tg) and torch.equal(ce, cg) and torch.equal(le, lg)


def test_a_row_with_nothing_to_draw_from_writes_nothing_and_is_reported(device):
    # q = 1 for every token (no distribution): every draft is rejected and the
    # residual max(0, p - q) is 0 everywhere, where the reference's
    # multinomial raises; the step leaves the rows as they were and check()
    # raises
    config = SMALL_BF16
    model = MQADecoder(config, random_weights(config, seed=2), dtype=torch.bfloat16)
    B, k = 3, 4
    cache = model.new_cache(B, capacity=128)
    ids = torch.randint(config.vocab, (B, 20), generator=torch.Generator().manual_seed(6)).to(device)
    prefill(model, cache, ids[:, :-1])
    step = VerifyStep(model, cache, k, temperature=1.0)
    step.feeds[:, 0] = ids[:, -1]
    step.feeds[:, 1:] = 7
    step.q.fill_(1.0)
    tokens, counts = step.run()
    assert counts.tolist() == [-1] * B
    assert cache.lengths.tolist() == [19] * B and step.feeds[:, 0].tolist() == ids[:, -1].tolist()
    with pytest.raises(RuntimeError, match="no mass"):
        step.check()
    step.check()  # cleared


def test_a_model_folder_loads_the_decoder_it_saved(device, tmp_path):
    # the reference's model-folder layout (checkpoint.py): the decoder loaded
    # from it scores as the decoder built from the same weights, bit for bit
    from wpt_amd import folder
    from wpt_amd.decoder import layer_kinds

    kinds = layer_kinds(1, 1, 1)
    config = DecoderConfig(layers=len(kinds), d_model=256, heads=16, head_dim=128, ffn=512, vocab=1024, kinds=kinds,
                           window=16, rope_dims=64, top_k=8)
    weights = random_weights(config, seed=3, dtype=torch.bfloat16)
    folder.save_folder(config, weights, tmp_path, b"{}", "test", max_shard_bytes=1 << 20)
    folder.save_drafter_record(tmp_path)
    ids = torch.randint(config.vocab, (2, 40), generator=torch.Generator().manual_seed(4)).to(device)
    loaded = folder.load_decoder(tmp_path, dtype=torch.bfloat16)
    built = MQADecoder(config, weights, dtype=torch.bfloat16)
    assert torch.equal(loaded(ids), built(ids))
