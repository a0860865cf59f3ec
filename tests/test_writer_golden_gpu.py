"""The GPU sampler on the reference Writer's own token streams: every
speculative step of the golden streams (tests/golden/writer_vectors.json,
drawn by the reference's Writer), decided by wptv_accept from a tape made of
the draws the reference's lazy order consumed (the oracle replay recovers
them), writes the tokens the reference wrote.  Decisions are exact; a
decision within 1e-5 of flipping would be reported (none at these seeds)."""

import pytest
import torch

from oracle import sampling as oracle
from tests.writer_replay import replay, streams
from wpt_amd import sampling

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", [c for c in streams() if c["drafter"]], ids=lambda case: case["name"])
def test_the_gpu_sampler_writes_the_reference_writer_s_tokens(device, case):
    _, _, steps = replay(case)
    assert steps
    for number, step in enumerate(steps):
        R, L = step["drafts"].shape
        V = step["q"].shape[-1]
        scores = torch.zeros(R, L + 1, V)
        u = torch.full((R, L), 0.5)
        for i in range(R):
            scores[i, :step["scores"][i].shape[0]] = step["scores"][i]
            u[i, :len(step["u"][i])] = torch.tensor(step["u"][i])
        e = torch.stack(step["e"])
        gaps = oracle.margins(scores, step["q"], step["drafts"], step["lengths"], case["temperature"], case["top_k"], u)
        assert min(gaps) > 1e-5, f"step {number}: a decision within 1e-5 of flipping"
        tokens, counts = sampling.accept(scores.to(device), step["q"].to(device), step["drafts"].to(device),
                                         u.to(device), e.to(device), case["temperature"], case["top_k"],
                                         lengths=step["lengths"])
        assert sampling.written(tokens, counts) == step["tokens"], f"step {number}"
