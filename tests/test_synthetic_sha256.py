"""The benchmark's synthetic inputs are what the committed digests say: every tensor re-derived
from the seeded generator (tests/golden/synthetic.py, the tags, shapes and distributions bench.py
uses) hashes to tests/golden/synthetic_sha256.json. The two 100M-element config-2 caches and the
front half's weight set are checked by the writer script only (make_synthetic_sha256.py)."""
import json
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import synthetic  # noqa: E402

WANT = json.load(open(os.path.join(HERE, "golden", "synthetic_sha256.json")))


@pytest.mark.parametrize("name", [n for n, (_, fast) in synthetic.ENTRIES.items() if fast])
def test_synthetic_digest(name):
    gen, _ = synthetic.ENTRIES[name]
    assert synthetic.digest(gen()) == WANT[name]


def test_every_entry_has_a_digest():
    assert sorted(WANT) == sorted(synthetic.ENTRIES)
