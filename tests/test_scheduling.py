"""The writer's prefix scheduler and its table of pass times (host code, CPU):
the scheduler against the oracle's and the reference's known answers, and the
scheduler-costs.json record round trip with its setup check."""

import random

import pytest

from oracle import sampling as oracle
from wpt_amd import scheduling
from wpt_amd.decoder import PLUMBING


def test_the_scheduler_gives_the_reference_s_known_answers():
    # test_sampling.py:230-238
    costs = [1.0, 1.0, 1.0, 1.2, 1.2, 1.2]
    assert scheduling.schedule([[0.9, 0.9, 0.9, 0.1, 0.1], [0.5] * 5], [5, 1], costs) == [2, 1]
    assert scheduling.schedule([[0.99] * 5, [0.99] * 5], [5, 5], costs) == [5, 5]
    assert scheduling.schedule([[0.9] * 5], [0], costs) == [0]


def test_the_scheduler_equals_the_oracle_s():
    rng = random.Random(11)
    for _ in range(500):
        rows, draft = rng.randint(1, 6), rng.randint(0, 6)
        caps = [rng.randint(0, draft) for _ in range(rows)]
        conf = [[rng.random() for _ in range(draft)] for _ in range(rows)]
        costs = [rng.uniform(0.5, 2.0) for _ in range(draft + 1)]
        assert scheduling.schedule(conf, caps, costs) == oracle.schedule(conf, caps, costs)


def test_a_costs_record_replays_on_its_setup_only():
    setup = scheduling.costs_setup(PLUMBING, rows=4, draft=5, device="cpu")
    assert setup["device"].startswith("cpu (") and setup["model"]["d_model"] == PLUMBING.d_model
    data = scheduling.costs_file([0.1, 0.1, 0.12, 0.13, 0.15, 0.2], setup)
    assert scheduling.replayed_costs(data, setup) == [0.1, 0.1, 0.12, 0.13, 0.15, 0.2]
    other = dict(setup, rows=8)
    with pytest.raises(ValueError, match="rows 4, here 8"):
        scheduling.replayed_costs(data, other)
    with pytest.raises(ValueError, match="no setup"):
        scheduling.replayed_costs(b'{"seconds": [1.0]}', setup)
