"""Writes tests/golden/writer_vectors.json: the token streams the reference's
own Writer (packages/wpt-inference/src/wpt_inference/__init__.py:71-233)
draws from a seeded generator, on the stub model and drafters of
tests/golden/stubs.py.  Nothing else pins the order in which the reference
consumes its generator (its tests assert only "same seed, same tokens"), so
these vectors pin the oracle's lazy draws (tests/test_oracle_writer.py).

Needs the reference checkout at /root/reference; run from the repository root:
    python tests/golden/make_writer_vectors.py
"""

import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PACKAGES = Path("/root/reference/packages")
sys.path[:0] = [str(HERE.parents[1]), str(PACKAGES / "wpt-inference" / "src"), str(PACKAGES / "wpt-utils" / "src")]

import torch  # noqa: E402
from wpt_inference import Writer  # noqa: E402

from tests.golden import stubs  # noqa: E402

PROMPT = [3, 17, 29, 8]


def main():
    out = []
    for name, kwargs, kind, calls in stubs.cases():
        model = stubs.Bigram()
        rows = kwargs.pop("rows")
        writer = Writer(model, PROMPT, rows, generator=torch.Generator().manual_seed(1234), drafter=stubs.drafter(kind),
                        **kwargs)
        written = []
        for limits in calls:
            got = writer.write({}, limits)
            written.append({str(row): tokens for row, tokens in got.items()})
        out.append({"name": name, "prompt": PROMPT, "rows": rows, **kwargs, "drafter": kind, "seed": 1234,
                    "calls": [{str(k): v for k, v in limits.items()} for limits in calls], "written": written,
                    "rounds": writer.rounds, "verified": writer.verified, "accepted": writer.accepted})
    for name, prompt, kwargs, calls in stubs.context_cases():
        model = stubs.Bigram()
        rows = kwargs.pop("rows")
        writer = Writer(model, prompt, rows, generator=torch.Generator().manual_seed(1234),
                        drafter=stubs.drafter("context"), **kwargs)
        written = []
        for inputs, limits in calls:
            got = writer.write(inputs, limits)
            written.append({str(row): tokens for row, tokens in got.items()})
        out.append({"name": name, "prompt": prompt, "rows": rows, **kwargs, "drafter": "context", "seed": 1234,
                    "inputs": [{str(k): v for k, v in inputs.items()} for inputs, _ in calls],
                    "calls": [{str(k): v for k, v in limits.items()} for _, limits in calls], "written": written,
                    "rounds": writer.rounds, "verified": writer.verified, "accepted": writer.accepted})
    path = HERE / "writer_vectors.json"
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path} ({len(out)} streams)")


if __name__ == "__main__":
    main()
