"""DSpark's prefix scheduler and the table of pass times it reads, for the
speculative writer (the reference's schedule, measure_costs, costs_setup,
costs_file and replayed_costs,
packages/wpt-inference/src/wpt_inference/__init__.py:236-330).

    schedule        how many drafts of each row one verify pass checks: the
                    pass widths are admitted from the narrowest while the
                    expected tokens per second grow (the reference's
                    Algorithm 1 with its early stop, :236-262)
    measure_costs   the seconds of one verify pass reading n tokens per row,
                    n = 1 .. draft + 1, the fastest of `repeats` undone passes
                    (:265-288); on the GPU each pass is timed with HIP events
                    on the model's stream around the pass alone
    costs_setup, costs_file, replayed_costs
                    the scheduler-costs.json record of a table and the check
                    that a replayed table was measured on the same setup
                    (:291-330), the file format kept as the reference writes it

The scheduler runs on the host in float64, on the drafter's confidences, in
the reference's order of additions, so that its admissions are the
reference's bit for bit; it is a few dozen operations per step.
"""

import json
import os
import time
from dataclasses import asdict, is_dataclass

import torch

COSTS_FILE = "scheduler-costs.json"  # the reference's name for a run's measured table (:68)


def schedule(confidences, caps, costs):
    """The drafts of each row to verify.  confidences[r][j]: the chance that
    draft j of row r is kept when every draft before it was; caps[r]: the
    most of row r's drafts that may be verified; costs[n - 1]: the seconds of
    a pass that reads n tokens per row.  A pass reads every row as wide as
    its widest, so width j + 1 adds every row's draft j at once; it is
    admitted while the expected tokens (each row's one token plus the chance
    of each admitted draft, the product of the confidences up to it) per
    second of the pass grow, and the first width that does not stops the
    admission."""
    keep = [1.0] * len(caps)  # the chance that every draft of the row so far is kept
    tokens = float(len(caps))
    rate, width = tokens / costs[0], 0
    for j in range(max(caps, default=0)):
        for r, cap in enumerate(caps):
            if j < cap:
                keep[r] *= confidences[r][j]
                tokens += keep[r]
        wider = tokens / costs[j + 1]
        if wider <= rate:
            break
        rate, width = wider, j + 1
    return [min(width, cap) for cap in caps]


def _synchronize(device):
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def _pass_seconds(run, device):
    """The seconds one call of run() takes: on a GPU, between two HIP events
    recorded on the current stream around it (the device's own clock, the
    launch gaps included); on the CPU, by the host clock."""
    if device.type == "cuda":
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        run()
        end.record()
        end.synchronize()
        return start.elapsed_time(end) * 1e-3
    began = time.perf_counter()
    run()
    return time.perf_counter() - began


@torch.no_grad()
def measure_costs(model, rows=1, draft=5, context=256, repeats=3):
    """The seconds of one pass of `model` (with a generation cache) reading n
    tokens per row through a cache of `rows` rows that have read `context`
    tokens, n = 1 .. draft + 1: for each n the fastest of `repeats` passes,
    each undone before the next."""
    device = next(model.parameters()).device
    cache = model.new_cache(rows)
    model.extend(torch.zeros(rows, context, dtype=torch.long, device=device), cache)
    _synchronize(device)
    table = []
    for width in range(1, draft + 2):
        ids = torch.zeros(rows, width, dtype=torch.long, device=device)
        times = []
        for _ in range(repeats):
            times.append(_pass_seconds(lambda: model.extend(ids, cache, undoable=True), device))
            model.undo(cache, [0] * rows)
        table.append(min(times))
    return table


def processor_name():
    """The host processor's model name as /proc/cpuinfo gives it, else the
    platform's (the reference names a CPU this way, wpt_utils/device.py:105-136)."""
    try:
        with open("/proc/cpuinfo") as info:
            for line in info:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return os.uname().machine


def costs_setup(model_config, rows, draft, device):
    """What a table of pass times was measured on: the model's config (a
    dataclass), the writer's rows, the drafts per step and the device by kind
    and name (the processor's for the CPU, the GPU's otherwise)."""
    device = torch.device(device)
    name = processor_name() if device.type == "cpu" else torch.cuda.get_device_name(device)
    config = asdict(model_config) if is_dataclass(model_config) else dict(model_config)
    return json.loads(json.dumps({"model": config, "rows": rows, "draft": draft, "device": f"{device.type} ({name})"}))


def costs_file(costs, setup):
    """The bytes of COSTS_FILE for a table measured on setup."""
    return (json.dumps({"setup": setup, "seconds": costs}, indent=2) + "\n").encode()


def replayed_costs(data, setup):
    """The seconds of a COSTS_FILE (its bytes) for a writer on setup;
    ValueError naming every difference when it was measured on another."""
    table = json.loads(data)
    if "setup" not in table:
        raise ValueError("the recorded costs name no setup; a replay needs the setup they were measured on")
    recorded = table["setup"]
    differences = []
    for key in setup:
        if key == "model":
            mine, theirs = setup["model"], recorded.get("model") or {}
            differences += [f"model {name} {theirs.get(name)!r}, here {mine.get(name)!r}"
                            for name in sorted(set(mine) | set(theirs)) if mine.get(name) != theirs.get(name)]
        elif recorded.get(key) != setup[key]:
            differences.append(f"{key} {recorded.get(key)!r}, here {setup[key]!r}")
    if differences:
        raise ValueError("the recorded costs were measured on another setup: " + "; ".join(differences))
    return [float(seconds) for seconds in table["seconds"]]
