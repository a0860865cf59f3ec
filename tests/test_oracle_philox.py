"""oracle/philox.py against values a torch generator on an MI355X drew
(tests/golden/torch_gpu_draws.json): the uniforms bit for bit, the offsets
each call moves the generator by, the exponentials within a few units in the
last place (numpy's log against the device's), and multinomial draws as the
exponential race over those exponentials."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import philox

GOLDEN = json.loads((Path(__file__).parent / "golden" / "torch_gpu_draws.json").read_text())
SEED = GOLDEN["seed"]
DEVICE = {"cus": GOLDEN["cus"], "threads_per_cu": GOLDEN["threads_per_cu"]}


def cases(call):
    return [c for c in GOLDEN["cases"] if c["call"] == call]


def f32(bits):
    return np.asarray(bits, dtype=np.int32).view(np.float32)


def test_the_fixture_covers_every_kind_of_call():
    assert {c["call"] for c in GOLDEN["cases"]} == {"rand_scalar", "rand", "exponential", "multinomial"}
    # a draw large enough that some threads give two words (numel > S)
    assert any(c["numel"] > philox.threads(c["numel"], **DEVICE) for c in GOLDEN["cases"])
    # and one whose threads take a second block (numel > 4 S)
    assert any(c["numel"] > 4 * philox.threads(c["numel"], **DEVICE) for c in GOLDEN["cases"])


def test_every_call_moves_the_offset_by_its_step():
    for c in GOLDEN["cases"]:
        assert c["offset_after"] - c["offset_before"] == philox.step(c["numel"], **DEVICE), c["call"]


def test_scalar_uniforms_are_torch_s():
    for c in cases("rand_scalar"):
        assert philox.rand_scalar(SEED, c["offset_before"]) == f32(c["bits"])[0]


@pytest.mark.parametrize("case", range(3))
def test_uniform_draws_are_torch_s_bit_for_bit(case):
    c = cases("rand")[case]
    u = philox.uniforms(SEED, c["offset_before"], c["numel"], **DEVICE)[c["index"]]
    u = np.where(u == 1, np.float32(0), u)  # torch.rand reads 1 as 0
    assert np.array_equal(u.view(np.int32), np.asarray(c["bits"], dtype=np.int32))


def test_exponentials_are_torch_s_within_four_ulp():
    for c in cases("exponential"):
        e = philox.exponentials(SEED, c["offset_before"], c["numel"], **DEVICE)[c["index"]]
        ulps = np.abs(e.view(np.int32).astype(np.int64) - np.asarray(c["bits"], dtype=np.int64))
        assert ulps.max() <= 4, c["numel"]


def test_a_wrong_subsequence_or_block_order_fails_the_pin():
    # the restatement with its counter halves swapped draws other values
    c = cases("rand")[0]
    words = philox.philox4x32_10(np.arange(c["numel"]), c["offset_before"] // 4, SEED)[:, 0]
    swapped = np.float32(2.0 ** -32) + words.astype(np.float32) * np.float32(2.0 ** -32)
    assert not np.array_equal(swapped.view(np.int32), np.asarray(c["bits"], dtype=np.int32))


def test_multinomial_is_the_race_over_the_call_s_exponentials():
    for c in cases("multinomial"):
        p = f32(c["p_bits"]).reshape(c["shape"]).astype(np.float64)
        e = philox.exponentials(SEED, c["offset_before"], c["numel"], **DEVICE).reshape(c["shape"])
        drawn = np.argmax(p / e, axis=-1).reshape(-1)
        assert drawn.tolist() == c["drawn"]
