"""Benchmark of the MI355X speculative-decoding verify step (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]

Prints one JSON line.  The headline workload (`value`) is one verify step of
a random-init 24-layer MQA decoder (d_model 2048, 16 query heads, 1 key/value
head, head width 128, SwiGLU 5632, vocab 32768, bf16 weights ~ N(0, 0.02)) at
batch 32 with 4096 tokens of key/value cache per row (a prefill of 4095 random
tokens, untimed) and a chain of k = 4 drafts per row drawn from
q = softmax(N(0, 1) logits), verified by rejection sampling at temperature 0.8
with seeded uniforms: the KV append, the forward pass, the lm_head, the
fused sampler and the undo, replayed from a HIP graph with every input
resident in HBM.  value = accepted tokens per second = the tokens the steps
write (kept drafts + 1 per row) over the timed steps' wall time.

`roofline` is verify attention at that step's attention shape (batch 32,
4096 table rows, k+1 = 5 causal query positions, 16 query heads, head width
128, bf16: 68,420,864 algorithmic bytes per call): both of its kernels (the
split attention and the split combine), timed with HIP events on their stream
over a graph of 24 back-to-back calls that take six tables in turn (403 MB, so
the keys and values come from HBM, not the 256 MB Infinity Cache), against
8 TB/s.  `configs` reports the other
workloads: the FP32 plumbing decoder's greedy step (checked bit-exact against
the oracle), sliding-window and tree verification, the three attention layers
of a WPT model at the verify shape (exact with its top-1024 choice, sparse over
the chosen rows, window over its ring), the step's matrix products (MFMA
TFLOP/s against the bf16 peak), the 24-layer step at batch 64 / KV 2048, and
the step of a decoder in the layout of the reference's largest model recipe
(window, exact and sparse layers), and the Writer's speculative rounds with
the DSpark-shaped drafter (drafting included).  `cpu_baseline` is the oracle (the reference's PyTorch
algorithm restated in FP32 on the CPU) running the headline step for a sample
of rows on this host's cores.
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


def log(message):
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def cpu_name():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def attention_bytes(B, T, H, c, N, elem=2):
    """Algorithmic HBM bytes of one verify-attention call: every key and value
    row once, the queries and outputs once, the positions."""
    return 2 * B * N * c * elem + 2 * B * T * H * c * elem + B * T * 8


def timed(fn, steps, warmup):
    """Average milliseconds of fn() over `steps` calls after `warmup`, timed
    with HIP events on the current stream."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def graphed(fn):
    """fn captured in a HIP graph (after two eager calls); returns replay."""
    import torch

    fn()
    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return graph.replay


# ---------------------------------------------------------------------------
# the verify step of the 24-layer decoder
# ---------------------------------------------------------------------------

def decoder_step(B, kv, k, steps, warmup, temperature=0.8, top_k=None, seed=0, keep=False, config=None,
                 in_order=True):
    """Builds the decoder (the 24-layer one unless config is given), prefills
    kv - 1 tokens per row, captures the step and times it.  Returns a dict of
    figures (and the pieces, with keep).  in_order: the step draws as the
    reference's loop does from a seeded generator on the GPU (its stream
    replayed on the device); otherwise from a tape drawn inside the step."""
    import torch

    from wpt_amd.decoder import LARGE, MQADecoder, random_weights
    from wpt_amd.step import VerifyStep, prefill

    device = torch.device("cuda", 0)
    config = config or LARGE
    weights = random_weights(config, seed=seed, std=0.02, dtype=torch.bfloat16, device=device)
    model = MQADecoder(config, weights, dtype=torch.bfloat16, device=device)
    generator = torch.Generator(device=device).manual_seed(seed + 1)
    prompt = torch.randint(config.vocab, (B, kv), generator=generator, device=device)
    cache = model.new_cache(B, capacity=kv + (steps + warmup + 8) * (k + 1))
    started = time.perf_counter()
    prefill(model, cache, prompt[:, :-1], chunk=1024)
    torch.cuda.synchronize()
    log(f"prefill B={B} x {kv - 1} tokens: {time.perf_counter() - started:.1f} s")
    draws = torch.Generator(device=device).manual_seed(seed + 2)
    step = VerifyStep(model, cache, k, temperature=temperature, top_k=top_k, in_order=in_order, generator=draws)
    step.feeds[:, 0] = prompt[:, -1]
    logits = torch.randn(B, k, config.vocab, generator=generator, device=device)
    step.q.copy_(torch.softmax(logits, -1))
    step.feeds[:, 1:] = torch.multinomial(step.q.reshape(-1, config.vocab), 1, generator=generator).reshape(B, k)
    torch.cuda.manual_seed(seed + 2)  # a tape's draws come from the device's default generator: seeded
    step.capture(warmup=1)
    for _ in range(warmup):
        step.replay()
    torch.cuda.synchronize()
    written = step.written  # the step's own running counts (kept by its next_feeds kernel)
    written.zero_()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step.replay()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    tokens = int(written.sum())
    # the matrices a step reads whole (a window layer's q/k/v and gate as their
    # one fused matrix, a sparse layer's q and gate too)
    fused = {f"layers.{i}.{part}" for i in config.windows for part in ("qkv", "gate")}
    fused |= {f"layers.{i}.{part}" for i in config.sparse for part in ("q", "gate")}
    params = sum(w.numel() for name, w in model.w.items()
                 if not name.endswith("norm") and not name.endswith("sink") and name != "embedding"
                 and name not in fused)
    out = {"ms_per_step": ms, "accepted_tokens": tokens, "tokens_per_s": tokens / (steps * ms * 1e-3),
           "tokens_per_row_step": tokens / (steps * B), "weight_bytes": 2 * params,
           "lengths_after": int(cache.lengths.max())}
    if keep:
        out["_pieces"] = (model, cache, step, weights)
    return out


def wpt_layout_step(B, kv, k, steps, warmup):
    """The verify step of a decoder in the layout of the reference's largest
    model recipe (data/recipes/models/interstitial-pecker.json: window layers
    4, sparse groups 2 of 5 sparse layers, 21 layers; d_model 512, 8 query
    heads of 128), window 128 and a choice of 1024 rows: all three attention
    kinds in one step.  A dense SwiGLU block of 1536 (the shared expert's 512
    plus four routed experts' 256) stands in for the experts; vocab 32768."""
    from wpt_amd.decoder import DecoderConfig, layer_kinds

    kinds = layer_kinds(4, 2, 5)
    config = DecoderConfig(layers=len(kinds), d_model=512, heads=8, head_dim=128, ffn=1536, vocab=32768, kinds=kinds,
                           window=128, top_k=1024)
    out = decoder_step(B, kv, k, steps, warmup, config=config)
    out["layers"] = "".join(kind[0] for kind in kinds)  # w window, e exact, s sparse
    return out


def drafted_writer(model, B, kv, k, rounds=8, warmup=2, seed=0):
    """Speculative rounds of the Writer with the DSpark-shaped drafter over
    `model` (24 layers), its steady rounds and the drafter's backbone replayed
    from HIP graphs (capture=True; the eager rounds are timed too): the drafter reads the
    residual streams of layers 2, 7, 12, 17 and 22 at the last 128 tokens
    read, 3 layers, random-init (so nearly every draft is rejected); each
    round drafts k tokens per row, verifies them in one undoable reading with
    the features, samples on the GPU and takes back the rejected ones.  B rows
    share one prompt of kv - 1 random tokens."""
    import torch

    from wpt_amd import drafter as drafters
    from wpt_amd.writer import Writer

    device = model.device
    config = drafters.DrafterConfig.for_model(model.config)
    weights = drafters.random_drafter_weights(model.config, config, seed=seed, device=device)
    limits = {row: k + 1 for row in range(B)}
    timed_rounds = {}
    for capture in (False, True):
        drafter = drafters.Drafter(model, config, weights, capture=capture)
        generator = torch.Generator(device=device).manual_seed(seed + 2)
        prompt = torch.randint(model.config.vocab, (kv,), generator=generator, device=device).tolist()
        writer = Writer(model, prompt, B, temperature=0.8, top_k=None, draft=k, generator=generator, drafter=drafter,
                        capture=capture)
        for _ in range(warmup):
            writer.write({}, limits)
        torch.cuda.synchronize()
        started, written = time.perf_counter(), 0
        for _ in range(rounds):
            written += sum(len(tokens) for tokens in writer.write({}, limits).values())
        torch.cuda.synchronize()
        timed_rounds[capture] = ((time.perf_counter() - started) / rounds, written)
    seconds, written = timed_rounds[True]
    context = (writer.context, writer.cache.lengths)
    histories = writer.histories
    probabilities = writer._probabilities
    draft_s = []
    for _ in range(3):
        torch.cuda.synchronize()
        t = time.perf_counter()
        drafter.draft(model, histories, context, k, probabilities, generator)
        torch.cuda.synchronize()
        draft_s.append(time.perf_counter() - t)
    return {"ms_per_round": seconds * 1e3, "tokens_per_s": written / rounds / seconds,
            "tokens_per_row_round": written / rounds / B, "draft_ms": min(draft_s) * 1e3,
            "eager_ms_per_round": timed_rounds[False][0] * 1e3,
            "drafter": {"features": list(config.features), "layers": config.layers, "block": config.block,
                        "markov_rank": config.markov_rank},
            "note": "Writer rounds, the reference's protocol: the drafter's backbone and each steady round's verify "
                    "reading and acceptance replayed from HIP graphs, one synchronization per round; "
                    "eager_ms_per_round: the same rounds eager; draft_ms: one draft (its backbone replayed)"}


# ---------------------------------------------------------------------------
# attention-only workloads
# ---------------------------------------------------------------------------

def attention_c2(steps, warmup):
    import torch

    from wpt_amd import kernels

    B, T, H, c, N = 32, 5, 16, 128, 4096
    device = torch.device("cuda", 0)
    generator = torch.Generator().manual_seed(0)
    q = torch.randn(B, T, H, c, generator=generator).to(torch.bfloat16).to(device)
    # six tables (403 MB, more than the 256 MB Infinity Cache) taken in turn,
    # so every call reads its keys and values from HBM, as each layer of the
    # step does
    tables = [torch.randn(B, N, 2 * c, generator=generator).to(torch.bfloat16).to(device) for _ in range(6)]
    positions = (N - T + torch.arange(T)).expand(B, T).contiguous().to(device)
    calls = 24  # back-to-back calls per graph replay: the per-call time is the kernels', not the graph launch's

    def run():
        for i in range(calls):
            table = tables[i % len(tables)]
            kernels.verify_attention(q, table[..., :c], table[..., c:], positions, c ** -0.5)

    replay = graphed(run)
    # at least 100 replays (about 50 ms of back-to-back calls) after 20: the
    # shorter runs read up to 10 % high while the clocks settle
    ms = timed(replay, max(100, steps // 4), max(20, warmup // 4)) / calls
    nbytes = attention_bytes(B, T, H, c, N)
    return {"ms": ms, "bytes": nbytes, "GBps": nbytes / (ms * 1e-3) / 1e9,
            "query_tokens_per_s": B * T / (ms * 1e-3)}


def attention_c3(steps, warmup):
    """Sliding window: batch 8, 32768 allocated rows, per-row lengths uniform
    in [16384, 32768], window 1024, k+1 = 5 queries at each row's end."""
    import torch

    from wpt_amd import kernels

    B, T, H, c, N, W = 8, 5, 16, 128, 32768, 1024
    device = torch.device("cuda", 0)
    generator = torch.Generator().manual_seed(0)
    lengths = torch.randint(N // 2, N + 1, (B,), generator=generator)
    positions = (lengths[:, None] - T + torch.arange(T)).to(device)
    q = torch.randn(B, T, H, c, generator=generator).to(torch.bfloat16).to(device)
    tables = [torch.randn(B, N, 2 * c, generator=generator).to(torch.bfloat16).to(device) for _ in range(3)]
    sink = torch.full((H,), float("-inf"), device=device)
    idx = torch.empty(B, T, 0, dtype=torch.long, device=device)
    calls = 24  # back-to-back calls per graph replay, so that the graph's own launch is not timed

    def run():
        for i in range(calls):
            table = tables[i % len(tables)]
            kernels.sparse_attention(q, table[..., :c], table[..., c:], sink, idx, positions, c ** -0.5, W)

    ms = timed(graphed(run), max(100, steps // 4), max(20, warmup // 4)) / calls  # as attention_c2
    nbytes = B * (W + T - 1) * 2 * c * 2 + 2 * B * T * H * c * 2 + B * T * 8
    GBps = nbytes / (ms * 1e-3) / 1e9
    return {"ms": ms, "bytes": nbytes, "GBps": GBps, "frac_hbm_peak": GBps / HBM_PEAK_GBS,
            "query_tokens_per_s": B * T / (ms * 1e-3),
            "note": "4.5 MB a call: launch-latency-bound; the three tables' windows stay in the Infinity Cache"}




def tree_c4(steps, warmup):
    """Tree verification: batch 16, 8192 prefix rows, a binary draft tree of 31
    nodes (depth 5) after them with the ancestor-only mask, the lm_head
    [2048 x 32768] ~ N(0, 0.02) on each node's attention output, then per-path
    greedy acceptance."""
    import torch

    from wpt_amd import kernels, layers, sampling

    B, M, H, c, prefix, V = 16, 31, 16, 128, 8192, 32768
    device = torch.device("cuda", 0)
    generator = torch.Generator(device=device).manual_seed(0)
    parents = [-1] + [(i - 1) // 2 for i in range(1, M)]
    q = torch.randn(B, M, H, c, generator=generator, device=device).to(torch.bfloat16)
    table = torch.randn(B, prefix + M, 2 * c, generator=generator, device=device).to(torch.bfloat16)
    head = (torch.randn(V, H * c, generator=generator, device=device) * 0.02).to(torch.bfloat16)
    head_fm = layers.FmWeight(head)  # packed once, as a model's weights are
    node_tokens = torch.randint(V, (B, M), generator=generator, device=device)
    base = torch.full((B,), prefix, device=device)
    written = torch.zeros(B, dtype=torch.long, device=device)

    def step(count=False):
        # the nodes' attention output written as the lm_head's fm operand; the
        # head on the 256 x 256 tiles keeps each node's first maximal index of
        # its bf16 logits (the greedy walk's only use of them), then the walk
        o = kernels.tree_attention(q, table[..., :c], table[..., c:], base, parents, c ** -0.5, out_fm=True)
        best = layers.head_argmax_fm_wide(o, B * M, head_fm).view(B, M)
        _, _, counts = sampling.greedy_tree_from_argmax(best, node_tokens, parents)
        if count:  # counted in a graph of its own, outside the timed one
            written.add_(counts.long())

    replay = graphed(step)
    ms = timed(replay, steps, warmup)
    counted = graphed(lambda: step(count=True))
    # eight back-to-back calls per graph replay, so that the graph's own launch is not timed
    attn = graphed(lambda: [kernels.tree_attention(q, table[..., :c], table[..., c:], base, parents, c ** -0.5)
                            for _ in range(8)])
    attn_ms = timed(attn, steps, warmup) / 8
    written.zero_()
    counted()
    torch.cuda.synchronize()
    per_step = int(written.sum())
    attn_flops = 4 * B * M * H * c * (prefix + M)
    return {"ms_per_step": ms, "accepted_tokens_per_step": per_step, "tokens_per_s": per_step / (ms * 1e-3),
            "attention_ms": attn_ms, "attention_TFLOPs": attn_flops / (attn_ms * 1e-3) / 1e12,
            "lm_head_rows": B * M}


def wpt_layers(steps, warmup):
    """The three attention layers of a WPT model at the verify step, at the
    verify-attention shape (batch 32, 4096 table rows, k+1 = 5 queries, 16
    heads of 128, bf16): the exact layer with its choice of TOP_K = 1024 rows
    outside a WINDOW of 128 (attention.py:51-52), the sparse layer over those
    rows plus its window (sink, output gate), the window layer over its ring
    (sink, output gate).  Four tables taken in turn (268 MB, more than the
    Infinity Cache).  Bytes: the exact layer reads every key and value and the
    keys again for the scores; the sparse layer the 1152 gathered rows of each
    query (a row two queries chose counts twice); the window layer its 132
    rows per batch row."""
    import torch

    from wpt_amd import kernels

    B, T, H, c, N, TOPK, W = 32, 5, 16, 128, 4096, 1024, 128
    device = torch.device("cuda", 0)
    generator = torch.Generator(device=device).manual_seed(3)
    q = torch.randn(B, T, H, c, generator=generator, device=device).to(torch.bfloat16)
    tables = [torch.randn(B, N, 2 * c, generator=generator, device=device).to(torch.bfloat16) for _ in range(4)]
    positions = (N - T + torch.arange(T, device=device)).expand(B, T).contiguous()
    sink = torch.randn(H, generator=generator, device=device)
    gate = torch.randn(B, T, H * c, generator=generator, device=device).to(torch.bfloat16)
    rings = [torch.randn(B, 256, 2 * c, generator=generator, device=device).to(torch.bfloat16) for _ in range(4)]
    chosen = [kernels.exact_attention(q, t[..., :c], t[..., c:], positions, c ** -0.5, TOPK, W)[1] for t in tables]
    calls = 8
    io = 2 * B * T * H * c * 2 + B * T * 8

    def per_call(fn):
        replay = graphed(lambda: [fn(i % 4) for i in range(calls)])
        return timed(replay, max(1, steps // 4), max(1, warmup // 4)) / calls

    def entry(ms, nbytes, cpu_s):
        GBps = nbytes / (ms * 1e-3) / 1e9
        return {"us": ms * 1e3, "bytes": nbytes, "GBps": GBps, "frac_hbm_peak": GBps / HBM_PEAK_GBS,
                "cpu_oracle_us": cpu_s * 1e6}

    # the oracle (FP32, this host's cores) on every batch row
    from oracle import attention as oracle_attention

    torch.set_num_threads(host_threads()[0])
    rows = B
    qc, tc = q[:rows].float().cpu(), tables[0][:rows].float().cpu()
    pc, sc, gc = positions[:rows].cpu(), sink.cpu(), gate[:rows].float().cpu()
    ic, rc = chosen[0][:rows].cpu(), rings[0][:rows].float().cpu()
    ring_table = torch.stack([rc[b, [(int(pc[b, 0]) - W + 1 + j) % 256 for j in range(W - 1 + T)]]
                              for b in range(rows)])

    def cpu(fn):
        best = float("inf")
        for _ in range(2):
            start = time.perf_counter()
            fn()
            best = min(best, time.perf_counter() - start)
        return best * B / rows

    out = {}
    ms = per_call(lambda i: kernels.exact_attention(q, tables[i][..., :c], tables[i][..., c:], positions, c ** -0.5,
                                                    TOPK, W))
    nbytes = attention_bytes(B, T, H, c, N) + B * N * c * 2 + 2 * B * T * N * 4 + B * T * TOPK * 8
    out["exact_layer_attention_and_choice_top1024"] = entry(
        ms, nbytes, cpu(lambda: oracle_attention.exact_attention(qc, tc[..., :c], tc[..., c:], pc, c ** -0.5, TOPK, W)))
    ms = per_call(lambda i: kernels.sparse_attention(q, tables[i][..., :c], tables[i][..., c:], sink, chosen[i],
                                                     positions, c ** -0.5, W, gate=gate))
    nbytes = B * T * (TOPK + W) * 2 * c * 2 + io + B * T * TOPK * 8 + B * T * H * c * 2
    out["sparse_layer_1024_chosen_plus_window_128"] = entry(
        ms, nbytes, cpu(lambda: oracle_attention.sparse_attention(qc, tc[..., :c], tc[..., c:], sc, ic, pc, c ** -0.5,
                                                                  W) * torch.sigmoid(gc).view(rows, T, H, c)))
    ms = per_call(lambda i: kernels.ring_attention(q, rings[i], positions, c ** -0.5, W, sink, gate=gate))
    nbytes = B * (W + T - 1) * 2 * c * 2 + io + B * T * H * c * 2
    out["window_layer_ring_window_128"] = entry(
        ms, nbytes, cpu(lambda: oracle_attention.window_attention(qc, ring_table[..., :c], ring_table[..., c:], sc, pc,
                                                                  c ** -0.5, W) * torch.sigmoid(gc).view(rows, T, H, c)))
    out["note"] = ("bytes: algorithmic (the sparse layer counts each query's gathered rows); cpu_oracle_us: the "
                   f"oracle in FP32 on all {B} batch rows, fastest of 2, on {torch.get_num_threads()} host threads")
    return out


def plumbing_c1():
    """The FP32 plumbing decoder: batch 1, a prompt of 64 tokens, 4 uniform
    drafts, greedy verification on the GPU and in the oracle."""
    import torch

    from oracle import decoder as oracle_decoder
    from oracle import sampling as oracle_sampling
    from wpt_amd import sampling
    from wpt_amd.decoder import PLUMBING, MQADecoder, random_weights

    device = torch.device("cuda", 0)
    weights = random_weights(PLUMBING, seed=0)
    gpu = MQADecoder(PLUMBING, weights, dtype=torch.float32, device=device)
    ora = oracle_decoder.Decoder(weights, PLUMBING.layers, PLUMBING.heads, PLUMBING.head_dim)
    generator = torch.Generator().manual_seed(0)
    prompt = torch.randint(PLUMBING.vocab, (64,), generator=generator).tolist()
    drafts = torch.randint(PLUMBING.vocab, (1, 4), generator=generator)
    feeds = torch.tensor([[prompt[-1]] + drafts[0].tolist()])
    rows = ora.new_cache(1)
    ora.extend(torch.tensor([prompt[:-1]]), rows)
    expected_scores, _ = ora.extend(feeds, rows, undoable=True)
    expected = oracle_sampling.greedy_chain(expected_scores, drafts, [4])[0]
    cache = gpu.new_cache(1, capacity=128)
    gpu.extend(torch.tensor([prompt[:-1]], device=device), cache)
    feeds_d, drafts_d = feeds.to(device), drafts.to(device)

    def step():
        scores, _ = gpu.extend(feeds_d, cache, undoable=True)
        tokens, counts = sampling.greedy_chain(scores, drafts_d)
        gpu.undo(cache, torch.zeros_like(counts, dtype=torch.long))  # back to the prompt: the same step again
        return tokens, counts

    tokens, counts = step()
    got = sampling.written(tokens, counts)[0]
    ms = timed(step, 20, 3)
    return {"ms_per_step": ms, "accepted_tokens_per_step": len(got), "tokens_per_s": len(got) / (ms * 1e-3),
            "bit_exact_vs_oracle": got == expected, "tokens": got}


def projections(model, rows, steps, warmup):
    """The step's matrix products at `rows` rows over the decoder's own 24
    layers of weights (each graph replay walks the layers, so every weight is
    cold, as in the step): per product, time per call, TFLOP/s against the bf16
    MFMA peak, and weight GB/s against HBM."""
    import torch

    from wpt_amd import layers

    cfg = model.config
    device = model.device
    generator = torch.Generator(device=device).manual_seed(7)
    out = {}
    fm = model.fm_rows(rows)  # the step's products at these rows: the fm ones, or the row-major split-K ones
    kinds = [("qkv", cfg.d_model, "split-K (parts)"), ("out", cfg.heads * cfg.head_dim, "split-K (parts)"),
             ("gate_up_tiles", cfg.d_model, "SwiGLU in the epilogue"), ("down", cfg.ffn, "split-K (parts)")]
    for name, K, engine in kinds:
        x = torch.randn(rows, K, generator=generator, device=device).to(torch.bfloat16)
        engine = ("build fm, " if fm else "build, ") + engine
        if fm:
            xf = layers.fm_pack(x)
            ws = [model.fm[f"layers.{i}.{name}"] for i in range(cfg.layers)]
            if name == "gate_up_tiles":
                calls = [lambda w=w: layers.linear_fm_swiglu(xf, rows, w) for w in ws]
            else:
                calls = [lambda w=w: layers.linear_fm_parts(xf, rows, w) for w in ws]
        else:
            ws = [model.w[f"layers.{i}.{name}"] for i in range(cfg.layers)]
            if name == "gate_up_tiles":
                calls = [lambda w=w: layers.linear_swiglu(x, w) for w in ws]
            else:
                calls = [lambda w=w: layers.linear_parts(x, w) for w in ws]
        replay = graphed(lambda: [f() for f in calls])
        ms = timed(replay, max(1, steps // 5), max(1, warmup // 5)) / len(ws)
        N = ws[0].shape[0]
        flops, nbytes = 2 * rows * N * K, N * K * 2
        out[name] = {"engine": engine, "N": N, "K": K, "us": ms * 1e3, "TFLOPs": flops / (ms * 1e-3) / 1e12,
                     "frac_bf16_peak": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                     "weight_GBps": nbytes / (ms * 1e-3) / 1e9}
    x = torch.randn(rows, cfg.d_model, generator=generator, device=device).to(torch.bfloat16)
    replay = graphed(lambda: layers.linear(x, model.w["head"]))
    ms = timed(replay, steps, warmup)
    N, K = model.w["head"].shape
    flops = 2 * rows * N * K
    out["lm_head"] = {"engine": "build, 128-column tiles, bf16 logits", "N": N, "K": K, "us": ms * 1e3,
                      "TFLOPs": flops / (ms * 1e-3) / 1e12,
                      "frac_bf16_peak": flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                      "weight_GBps": N * K * 2 / (ms * 1e-3) / 1e9}
    return out


# ---------------------------------------------------------------------------
# the CPU baseline: the oracle running the headline step for sampled rows
# ---------------------------------------------------------------------------

def host_threads():
    """(threads to use, the affinity's CPU count, the cgroup's CPU quota or
    None): the affinity's CPUs, capped by the cgroup quota where one is set
    (more threads than the quota only time-slice)."""
    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        limit, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if limit != "max":
            quota = max(1, int(int(limit) / int(period)))
    except (OSError, ValueError):
        pass
    return (min(affinity, quota) if quota else affinity), affinity, quota


def cpu_baseline(pieces, budget_s=20.0, passes=5):
    """The oracle (FP32, this host's cores) running the headline step for
    every row: the same weights, KV cache, pending tokens, drafts and
    distributions; fastest of up to `passes` passes within the budget, as
    the reference's measure_costs takes the fastest pass."""
    import torch

    from oracle import decoder as oracle_decoder
    from oracle import sampling as oracle_sampling

    model, cache, step, weights = pieces
    threads, affinity, quota = host_threads()
    torch.set_num_threads(threads)
    config = model.config
    rows = cache.rows
    started = time.perf_counter()
    ora = oracle_decoder.Decoder({name: w.float().cpu() for name, w in weights.items()}, config.layers, config.heads,
                                 config.head_dim)
    lengths = cache.lengths.cpu()
    tables = [t[:, :int(lengths.max()) + step.k + 1].float().cpu() for t in cache.tables]
    feeds = step.feeds.cpu()
    q = step.q.cpu()
    log(f"oracle set up in {time.perf_counter() - started:.1f} s ({rows} rows, {threads} threads)")
    generator = torch.Generator().manual_seed(0)
    best, spent, done, written = float("inf"), 0.0, 0, 0
    while done < 1 or (spent < budget_s and done < passes):
        state = oracle_decoder.cache.Rows(rows)
        state.lengths = lengths.clone()
        state.values = {("entries", i): t.clone() for i, t in enumerate(tables)}
        start = time.perf_counter()
        scores, _ = ora.extend(feeds, state, undoable=True)
        draws = [oracle_sampling.LazyDraws(generator) for _ in range(rows)]
        out = oracle_sampling.accept(scores, q, feeds[:, 1:], [step.k] * rows, step.temperature, step.top_k, draws)
        ora.undo(state, [len(t) for t in out])
        elapsed = time.perf_counter() - start
        best, spent, done = min(best, elapsed), spent + elapsed, done + 1
        written = sum(len(t) for t in out)
    return {"value": written / best, "unit": "accepted tokens/s", "cores": threads, "kind": "port",
            "sample": f"the oracle's verify step (24 layers, FP32) for all {rows} rows at the same KV length, "
                      f"drafts and distributions, drawing lazily as the reference does; fastest of {done} passes "
                      f"({best:.2f} s) on {threads} threads ({affinity} CPUs in the affinity, cgroup quota "
                      f"{quota if quota else 'none'}) of {cpu_name()}"}


def cpu_attention_c3():
    """The oracle's sliding-window verify on every row of the C3 workload (FP32, host cores): seconds."""
    import torch

    from oracle import attention as oracle_attention

    torch.set_num_threads(host_threads()[0])
    B, T, H, c, N, W = 8, 5, 16, 128, 32768, 1024
    generator = torch.Generator().manual_seed(0)
    lengths = torch.randint(N // 2, N + 1, (B,), generator=generator)
    positions = lengths[:, None] - T + torch.arange(T)
    q = torch.randn(B, T, H, c, generator=generator).to(torch.bfloat16)
    table = torch.randn(B, N, 2 * c, generator=generator).to(torch.bfloat16)
    sink = torch.full((H,), float("-inf"))
    idx = torch.empty(B, T, 0, dtype=torch.long)
    best = float("inf")
    for _ in range(3):
        start = time.perf_counter()
        oracle_attention.sparse_attention(q, table[..., :c], table[..., c:], sink, idx, positions, c ** -0.5, W)
        best = min(best, time.perf_counter() - start)
    return best


def cpu_tree_c4():
    """The oracle's tree step on every row of the C4 workload (attention, the
    FP32 lm_head over the 496 node rows, greedy tree acceptance; host
    cores): (seconds, tokens written)."""
    import torch

    from oracle import attention as oracle_attention
    from oracle import sampling as oracle_sampling

    torch.set_num_threads(host_threads()[0])
    B, M, H, c, prefix, V = 16, 31, 16, 128, 8192, 32768
    generator = torch.Generator().manual_seed(0)
    parents = oracle_attention.binary_tree_parents(M)
    q = torch.randn(B, M, H, c, generator=generator).to(torch.bfloat16)
    table = torch.randn(B, prefix + M, 2 * c, generator=generator).to(torch.bfloat16)
    head = (torch.randn(V, H * c, generator=generator) * 0.02).to(torch.bfloat16).float()
    node_tokens = torch.randint(V, (B, M), generator=generator)
    prefixes = torch.full((B,), prefix)
    best, written = float("inf"), 0
    for _ in range(2):
        start = time.perf_counter()
        o = oracle_attention.tree_attention(q, table[..., :c], table[..., c:], prefixes, parents, c ** -0.5)
        scores = o.float().reshape(B, M, H * c) @ head.T
        walks = oracle_sampling.greedy_tree(scores, node_tokens, parents)
        best = min(best, time.perf_counter() - start)
        written = sum(len(tokens) for _, tokens in walks)
    return best, written


def pmc_workload():
    import torch

    from wpt_amd import kernels

    B, T, H, c, N = 32, 5, 16, 128, 4096
    device = torch.device("cuda", 0)
    generator = torch.Generator().manual_seed(0)
    q = torch.randn(B, T, H, c, generator=generator).to(torch.bfloat16).to(device)
    tables = [torch.randn(B, N, 2 * c, generator=generator).to(torch.bfloat16).to(device) for _ in range(5)]
    positions = (N - T + torch.arange(T)).expand(B, T).contiguous().to(device)
    for table in tables:  # a table each, read from HBM as in the roofline measurement
        kernels.verify_attention(q, table[..., :c], table[..., c:], positions, c ** -0.5)
    torch.cuda.synchronize()
    src = torch.ones(32 * 1024 * 1024, dtype=torch.bfloat16, device=device)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("pmc workload done")


def pmc_products():
    """For counter passes over the layer products: the verify step's four
    fragment-major products at 160 rows (batch 32, k = 4), each called once
    per layer of the 24-layer decoder's weights (every weight read cold, as in
    the step), eagerly, twice over."""
    import torch

    from wpt_amd import layers
    from wpt_amd.decoder import LARGE, MQADecoder, random_weights

    device = torch.device("cuda", 0)
    weights = random_weights(LARGE, seed=0, std=0.02, dtype=torch.bfloat16, device=device)
    model = MQADecoder(LARGE, weights, dtype=torch.bfloat16, device=device)
    rows = 160
    generator = torch.Generator(device=device).manual_seed(7)
    for _ in range(2):
        for name, K in (("qkv", LARGE.d_model), ("out", LARGE.heads * LARGE.head_dim),
                        ("gate_up_tiles", LARGE.d_model), ("down", LARGE.ffn)):
            xf = layers.fm_pack(torch.randn(rows, K, generator=generator, device=device).to(torch.bfloat16))
            for i in range(LARGE.layers):
                w = model.fm[f"layers.{i}.{name}"]
                if name == "gate_up_tiles":
                    layers.linear_fm_swiglu(xf, rows, w)
                else:
                    layers.linear_fm_parts(xf, rows, w)
            torch.cuda.synchronize()
    log("pmc products done")


COPY_BYTES = 64 * 1024 * 1024  # the plain device copy of --pmc-workload (32 Mi bf16 values), read and written once


def counter_pass(counter, timeout=180):
    """One rocprofv3 --pmc pass of `counter` over this script's
    --pmc-workload, in a child process: {kernel name: [value per dispatch]}."""
    import csv
    import shutil
    import subprocess
    import tempfile

    rocprof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    with tempfile.TemporaryDirectory(prefix="wptv_pmc_", dir="/tmp") as where:
        command = [rocprof, "--pmc", counter, "--output-format", "csv", "-d", where, "-o", "pmc", "--",
                   sys.executable, str(ROOT / "bench.py"), "--pmc-workload"]
        subprocess.run(command, cwd="/tmp", env={**os.environ, "TMPDIR": "/tmp"}, capture_output=True,
                       timeout=timeout, check=True)
        found = {}
        for path in Path(where).rglob("*counter_collection.csv"):
            with open(path, newline="") as f:
                for row in csv.DictReader(f):
                    if row["Counter_Name"] == counter:
                        found.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
        return found


def measured_traffic():
    """HBM bytes per verify-attention call at the roofline shape, measured in
    this run: FETCH_SIZE and WRITE_SIZE passes (KiB per dispatch) over the
    five calls of --pmc-workload, each scaled so that the plain 64 MiB copy
    of the same workload reads (writes) 64 MiB.  (bytes, the two scale
    factors) or (None, the reason)."""
    try:
        per_call = 0.0
        factors = {}
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            found = counter_pass(counter)
            copy = [v for name, values in found.items() if "copy" in name.lower() for v in values[-5:]]
            attention = [sum(values) for name, values in found.items()
                         if "verify_attention" in name or "combine_splits" in name]
            if not copy or not attention:
                return None, f"{counter}: no copy or attention dispatch in the counter output"
            factor = COPY_BYTES / (sorted(copy)[len(copy) // 2] * 1024)  # the workload's last copies
            factors[counter] = factor
            per_call += sum(attention) / 5 * 1024 * factor  # five calls in the workload
        return int(per_call), factors
    except Exception as error:  # the counters are a report, never the run's failure
        return None, f"{type(error).__name__}: {error}"


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--quick", action="store_true",
                        help="the headline step and its roofline only (no other configs, no CPU baseline)")
    parser.add_argument("--wpt-layers", action="store_true",
                        help="only the WPT attention layers at the verify shape (exact + choice, sparse, window); "
                             "prints their JSON")
    parser.add_argument("--tree", action="store_true",
                        help="only the tree workload (batch 16, 8192 prefix rows, 31 nodes, lm_head, greedy walk); "
                             "prints its JSON")
    parser.add_argument("--writer", action="store_true",
                        help="only the drafted Writer rounds over the 24-layer decoder (batch 32, KV 4096, k 4); "
                             "prints their JSON")
    parser.add_argument("--tape-draws", action="store_true",
                        help="the headline step reads a tape drawn inside it instead of drawing in the reference's "
                             "order")
    parser.add_argument("--pmc-products", action="store_true",
                        help="for counter passes: the step's four fragment-major layer products at 160 rows, each "
                             "over the 24 layers' weights, twice; prints no JSON")
    parser.add_argument("--pmc-workload", action="store_true",
                        help="for a counter pass: five verify-attention calls of the roofline shape, then five "
                             "plain 64 MiB device copies (the counters' calibration); prints no JSON")
    args = parser.parse_args()
    if args.pmc_workload:
        pmc_workload()
        return
    if args.pmc_products:
        pmc_products()
        return
    if args.wpt_layers:
        print(json.dumps(wpt_layers(args.steps, args.warmup)), flush=True)
        return
    if args.tree:
        print(json.dumps(tree_c4(args.steps, args.warmup)), flush=True)
        return
    if args.writer:
        model = decoder_step(32, 4096, 4, 2, 1, keep=True)["_pieces"][0]
        print(json.dumps(drafted_writer(model, 32, 4096, 4)), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the verify step here is built and timed on a single MI355X "
              f"(--gpus {args.gpus} is not supported)", file=sys.stderr)
        sys.exit(2)
    import torch

    B, KV, K = 32, 4096, 4
    log("headline step")
    head = decoder_step(B, KV, K, args.steps, args.warmup, keep=True, in_order=not args.tape_draws)
    log(f"headline step: {head['ms_per_step']:.3f} ms, {head['tokens_per_s']:.0f} accepted tok/s")
    attn = attention_c2(args.steps, args.warmup)
    log(f"verify attention: {attn['ms'] * 1e3:.2f} us, {attn['GBps']:.0f} GB/s")
    configs = {}
    if not args.quick:
        configs["plumbing_fp32_greedy_B1"] = plumbing_c1()
        configs["verify_attention_B32_KV4096"] = attn
        configs["sliding_window_B8_KV32768_W1024"] = attention_c3(args.steps, args.warmup)
        seconds = cpu_attention_c3()
        configs["sliding_window_B8_KV32768_W1024"]["cpu_baseline"] = {
            "value": 8 * 5 / seconds, "unit": "query tokens/s", "cores": host_threads()[0], "kind": "port",
            "sample": f"the oracle's sparse_attention (window only), all 8 rows, fastest of 3: {seconds * 1e3:.1f} ms"}
        configs["tree_B16_KV8192_31nodes_lm_head"] = tree_c4(args.steps, args.warmup)
        seconds, tokens = cpu_tree_c4()
        configs["tree_B16_KV8192_31nodes_lm_head"]["cpu_baseline"] = {
            "value": tokens / seconds, "unit": "accepted tokens/s", "cores": host_threads()[0], "kind": "port",
            "sample": f"the oracle's tree attention, FP32 lm_head and greedy walk, all 16 rows, fastest of 2: "
                      f"{seconds * 1e3:.0f} ms"}
        configs["wpt_attention_layers_B32_KV4096"] = wpt_layers(args.steps, args.warmup)
        log("configs c1-c4 and the WPT attention layers done")
    pieces = head.pop("_pieces")
    if not args.quick:
        configs["projections_rows160"] = projections(pieces[0], B * (K + 1), args.steps, args.warmup)
        log("projections done")
        configs["drafted_writer_B32_KV4096_k4"] = drafted_writer(pieces[0], B, KV, K)
        log(f"drafted writer: {configs['drafted_writer_B32_KV4096_k4']['ms_per_round']:.2f} ms a round")
    cpu = None if args.quick else cpu_baseline(pieces)
    del pieces
    torch.cuda.empty_cache()
    if not args.quick:
        for top_k in (None, 40):
            configs[f"decoder_step_B64_KV2048_k4_T0.8_topk{top_k}"] = decoder_step(64, 2048, K, args.steps,
                                                                                  args.warmup, top_k=top_k)
            torch.cuda.empty_cache()
        configs["wpt_layout_step_B32_KV4096_k4"] = wpt_layout_step(B, KV, K, args.steps, args.warmup)
        torch.cuda.empty_cache()
    traffic, traffic_note = (None, "not measured with --quick") if args.quick else measured_traffic()
    if traffic is not None:
        traffic_note = (f"rocprofv3 FETCH_SIZE + WRITE_SIZE passes over --pmc-workload in this run, scaled by "
                        f"{traffic_note['FETCH_SIZE']:.3f} and {traffic_note['WRITE_SIZE']:.3f} (a plain 64 MiB copy "
                        f"reads and writes 64 MiB); algorithmic bytes {attention_bytes(32, 5, 16, 128, 4096)}")
    line = {
        "metric": "accepted tok/s (B=32,KV=4096,k=4 bf16); verify-attn % of HBM roofline",
        "value": head["tokens_per_s"], "unit": "accepted tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "speculative verify step: random-init 24-layer MQA decoder (d_model 2048, 16q/1kv "
                               "heads, head 128, SwiGLU 5632, vocab 32768), batch 32, KV 4096, chain k=4, "
                               "rejection sampling T=0.8, HIP graph", "global_batch": B, "seq_len": KV,
                   "draws": "tape drawn in the step" if args.tape_draws else
                            "the reference's order from a seeded GPU generator",
                   "draft": K, "tokens_per_row_step": head["tokens_per_row_step"]},
        "roofline": {"bound": "hbm", "achieved": attn["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": attn["GBps"] / HBM_PEAK_GBS, "traffic": traffic,
                     "traffic_note": traffic_note,
                     "kernel": "verify attention, batch 32 x 4096 rows x 5 queries x 16 heads x 128, bf16",
                     "ms": attn["ms"]},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
