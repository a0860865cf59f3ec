"""Pins the oracle's lazy draws against the reference's own Writer: the token
streams tests/golden/writer_vectors.json holds were drawn by the reference's
Writer (imported by tests/golden/make_writer_vectors.py) from a seeded
generator; the oracle's acceptance rule, drawing lazily from a generator of
the same seed in its order, writes the same tokens, and counts the same
rounds, verified and accepted drafts."""

import pytest

from tests.writer_replay import replay, streams


@pytest.mark.parametrize("case", streams(), ids=lambda case: case["name"])
def test_the_oracle_writes_the_reference_writer_s_tokens(case):
    written, counters, _ = replay(case)
    assert written == case["written"]
    assert counters == {key: case[key] for key in ("rounds", "verified", "accepted")}
