"""Writes tests/golden/torch_gpu_draws.json: values a torch generator on the
GPU drew (torch.rand, exponential_, multinomial), with the generator's offset
before and after each call, and the device's multiprocessor figures that
shape the draws.  They pin oracle/philox.py's restatement of that stream
(tests/test_oracle_philox.py), which is what the reference's Writer consumes
when its generator lives on the GPU.

Needs a GPU; run from the repository root:
    python tests/golden/make_torch_gpu_draws.py [output path]
"""

import json
import sys

import numpy as np
import torch

SEED = 1234567


def offset(generator):
    return int(generator.get_state().view(torch.int64)[1])


def bits(x):
    return np.asarray(x, dtype=np.float32).view(np.int32).tolist()


def main(path="tests/golden/torch_gpu_draws.json"):
    device = torch.device("cuda")
    props = torch.cuda.get_device_properties(device)
    g = torch.Generator(device=device).manual_seed(SEED)
    picks = np.random.default_rng(0)
    cases = []

    def record(call, numel, values, before, **extra):
        values = np.asarray(values, dtype=np.float32).reshape(-1)
        if values.size > 64:  # the first and last 16 entries and 32 between
            index = np.unique(np.concatenate([np.arange(16), np.arange(numel - 16, numel),
                                              picks.integers(16, numel - 16, 32)]))
        else:
            index = np.arange(values.size)
        cases.append({"call": call, "numel": numel, "offset_before": before, "offset_after": offset(g),
                      "index": index.tolist(), "bits": bits(values[index]), **extra})

    for _ in range(3):
        before = offset(g)
        record("rand_scalar", 1, [torch.rand((), generator=g, device=device).item()], before)
    for numel in (8, 1_000_000, 3_000_000):
        before = offset(g)
        record("rand", numel, torch.rand(numel, generator=g, device=device).cpu().numpy(), before)
    for numel in (50, 32768):
        before = offset(g)
        record("exponential", numel, torch.empty(numel, device=device).exponential_(generator=g).cpu().numpy(),
               before)
    before = offset(g)
    record("exponential", 17 * 32768, torch.empty(17, 32768, device=device).exponential_(generator=g).cpu().numpy(),
           before)
    for shape in ((50,), (7, 50)):
        p = torch.softmax(3 * torch.randn(shape, generator=g, device=device), -1)
        before = offset(g)
        drawn = torch.multinomial(p, 1, generator=g).reshape(-1)
        cases.append({"call": "multinomial", "numel": p.numel(), "shape": list(shape), "offset_before": before,
                      "offset_after": offset(g), "p_bits": bits(p.cpu().numpy().reshape(-1)),
                      "drawn": drawn.cpu().tolist()})
    out = {"seed": SEED, "cus": props.multi_processor_count,
           "threads_per_cu": props.max_threads_per_multi_processor, "torch": torch.__version__, "cases": cases}
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {path}: {len(cases)} calls")


if __name__ == "__main__":
    main(*sys.argv[1:])
