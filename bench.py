"""Benchmark of the MI355X speculative-decoding verify step (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload attention]

Prints one JSON line.  Workloads:

    attention  verify attention alone: MQA, 16 query heads, 1 key/value head,
               head width 128, bf16, batch 32, 4096 table rows per batch row
               (one contiguous (B, N, 2c) entries table, keys first), k+1 = 5
               query positions at the table's end (causal among the drafts)

A step is one pass of the hot path over one batch, inputs resident in HBM.
The roofline figure is the verify-attention kernel's algorithmic bytes over
its average duration, timed with HIP events on the stream it runs on.  The
CPU baseline is the oracle (the reference's PyTorch algorithm restated in
FP32 on the CPU) timed on this host's cores on the same inputs.
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


def attention_bytes(B, T, H, c, N, elem=2):
    """Algorithmic HBM bytes of one verify-attention call: the key and value
    rows once, the queries and outputs once, the positions."""
    return 2 * B * N * c * elem + 2 * B * T * H * c * elem + B * T * 8


def cpu_name():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def attention_inputs(B, T, H, c, N, seed=0):
    import torch

    generator = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, c, generator=generator).to(torch.bfloat16)
    table = torch.randn(B, N, 2 * c, generator=generator).to(torch.bfloat16)
    positions = (N - T + torch.arange(T)).expand(B, T).contiguous()
    return q, table, positions


def cpu_attention_baseline(q, table, positions, budget_s=15.0):
    """The oracle's exact attention on the host cores: the fastest of as many
    passes as fit the budget (at least two), in query-row tokens per second."""
    import torch

    from oracle import attention as oracle_attention

    threads = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(threads)
    c = q.shape[-1]
    k, v = table[..., :c], table[..., c:]
    best, spent, passes = float("inf"), 0.0, 0
    while passes < 2 or (spent < budget_s and passes < 20):
        start = time.perf_counter()
        oracle_attention.exact_attention(q, k, v, positions, c ** -0.5, 0, 128)
        elapsed = time.perf_counter() - start
        best, spent, passes = min(best, elapsed), spent + elapsed, passes + 1
    return best, threads, passes


def bench_attention(args):
    import torch

    from wpt_amd import kernels

    B, T, H, c, N = 32, 5, 16, 128, 4096
    device = torch.device("cuda", 0)
    q, table, positions = attention_inputs(B, T, H, c, N)
    qd, td, pd = q.to(device), table.to(device), positions.to(device)
    kd, vd = td[..., :c], td[..., c:]
    scale = c ** -0.5
    # One step is one verify-attention call, replayed from a HIP graph so that
    # the host's launch cost stays out of the GPU timeline.
    for _ in range(3):
        kernels.verify_attention(qd, kd, vd, pd, scale)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        kernels.verify_attention(qd, kd, vd, pd, scale)
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    nbytes = attention_bytes(B, T, H, c, N)
    achieved = nbytes / (ms * 1e-3) / 1e9
    cpu_s, threads, passes = cpu_attention_baseline(q, table, positions)
    return {
        "metric": "verify-attention query tokens/s (B=32, KV=4096, k=4, bf16 MQA)",
        "value": B * T / (ms * 1e-3),
        "unit": "query tokens/s",
        "ms_per_step": ms,
        "dtype": "bf16",
        "config": {"workload": "verify attention: MQA 16q/1kv heads, head width 128, batch 32, KV 4096, "
                               "k+1=5 causal query positions, bf16", "global_batch": B, "seq_len": N},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None},
        "cpu_baseline": {"value": B * T / cpu_s, "unit": "query tokens/s", "cores": threads, "kind": "port",
                         "sample": f"the oracle's exact attention on the whole workload, fastest of {passes} passes "
                                   f"on {cpu_name()}"},
    }


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--workload", default="attention", choices=["attention"])
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the verify step here is built and timed on a single MI355X "
              f"(--gpus {args.gpus} is not supported)", file=sys.stderr)
        sys.exit(2)
    result = bench_attention(args)
    line = {"metric": result["metric"], "value": result["value"], "unit": result["unit"], "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": result["ms_per_step"],
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": result["dtype"],
            "data": "synthetic", "config": result["config"], "roofline": result["roofline"],
            "cpu_baseline": result["cpu_baseline"]}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
