"""Writes tests/golden/rope_inv_freq.json: the binary32 bits of inv_freq as the
reference computes it (src/pretrain/model/modules/rope.py:21-22, torch binary32
pow and division) for the (head_dim, theta) pairs the configurations use.

    python tests/golden/make_rope_fixture.py          # rewrite the fixture
    python tests/golden/make_rope_fixture.py --check  # compare, exit 1 on a difference

torch's binary32 pow is not correctly rounded, so these bits are what torch
gives; the fixture makes a host whose torch gives other bits (and so other
RoPE'd inputs) fail loudly instead of changing the inputs silently.
"""

from __future__ import annotations

import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
FIXTURE = HERE / "rope_inv_freq.json"
PAIRS = [(64, 10000.0), (128, 10000.0), (128, 500000.0)]


def compute() -> dict:
    sys.path.insert(0, str(ROOT))
    import __graft_entry__

    __graft_entry__.load_package()
    from open_transformers_amd import rope

    return {f"D{D}_theta{int(theta)}": [f"{int(u):08x}" for u in rope.inv_freq(D, theta).view(np.uint32)]
            for D, theta in PAIRS}


if __name__ == "__main__":
    got = compute()
    if "--check" in sys.argv:
        sys.exit(0 if json.loads(FIXTURE.read_text()) == got else 1)
    FIXTURE.write_text(json.dumps(got, indent=1) + "\n")
    print(f"wrote {FIXTURE}")
