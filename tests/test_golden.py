"""The oracle reproduces the committed config-1 fixture (tests/golden/config1.json)."""
import json
import os

from tests.golden import make_golden

HERE = os.path.dirname(os.path.abspath(__file__))


def test_config1_fixture_is_reproduced():
    with open(os.path.join(HERE, "golden", "config1.json")) as fh:
        committed = json.load(fh)
    assert make_golden.summary() == committed


def test_config1_online_attention_matches_double_reference():
    fresh = make_golden.summary()
    for a, b in zip(fresh["attention_first_values"], fresh["attention_reference_first_values"]):
        assert abs(a - b) <= 1e-5 * (1 + abs(b))
