"""The oracle and the seeded input generator reproduce the committed golden
digests (tests/golden/attn_hashes.json, written by tests/golden/make_golden.py)."""

from __future__ import annotations

import json
import pathlib
import sys

import pytest

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "golden"))

import make_golden  # noqa: E402

WANT = json.loads((HERE / "golden" / "attn_hashes.json").read_text())


def test_fixture_covers_every_case():
    assert sorted(WANT) == sorted(make_golden.CASES)


@pytest.mark.parametrize("case", sorted(make_golden.CASES))
def test_oracle_matches_golden(case):
    got = make_golden.compute_case(case)
    assert got == WANT[case]
