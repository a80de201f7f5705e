"""The RoPE tables (open-transformers_amd/rope.py) against the reference's
recipe (src/pretrain/model/modules/rope.py:21-31).

  entries       every cos/sin entry of the tables the configurations use equals
                the binary32 rounding of libquadmath's cosq / sinq of the
                binary32 angle (repop's cos/sin are correctly rounded).
  slow path     the 60-digit evaluation that decides entries the binary64 libm
                value leaves open gives the same bits on random and special
                angles.
  inv_freq      torch binary32 pow and division, the bits of the committed
                fixture (tests/golden/rope_inv_freq.json); 19 of the 64 entries
                at theta 10000, D 128 differ from a binary64 evaluation.
  one table     the input generator and the decoder layer use the same tables.
"""

from __future__ import annotations

import json
import pathlib

import numpy as np
import pytest

from oracle import oracle as orc
from open_transformers_amd import rope, synthetic

HERE = pathlib.Path(__file__).resolve().parent


@pytest.mark.parametrize("S,D,theta", [(8192, 128, 10000.0), (4096, 128, 500000.0), (2048, 64, 10000.0)])
def test_table_entries_are_correctly_rounded(S, D, theta):
    cos, sin = rope.rope_tables(S, D, theta)
    qc, qs = orc.cos_sin_quad(rope.angles(S, D, theta))
    assert np.array_equal(cos.view(np.uint32), qc.view(np.uint32))
    assert np.array_equal(sin.view(np.uint32), qs.view(np.uint32))


def test_high_precision_path_matches_quadmath():
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.uniform(0, 8192, 400).astype(np.float32),
        rng.uniform(-4, 4, 200).astype(np.float32),
        np.array([0.0, -0.0, 1e-30, np.pi, np.float32(np.pi), 3 * np.float32(np.pi) / 2, 4096.0, 8191.0], np.float32),
    ])
    qc, qs = orc.cos_sin_quad(x)
    for xi, c, s in zip(x, qc, qs):
        hc, hs = rope._hp_cos_sin(float(xi))
        assert rope._round_decimal_f32(hc) == c, xi
        assert rope._round_decimal_f32(hs).view(np.uint32) == s.view(np.uint32), xi


def test_checked_rounding_defers_near_boundaries():
    # a binary64 value on a binary32 rounding boundary (tie) must be deferred to the slow path
    lo = np.float32(1.0)
    hi = np.nextafter(lo, np.float32(2.0))
    mid = (np.float64(lo) + np.float64(hi)) / 2
    _, ok = rope._round_checked(np.array([mid, 0.75, 0.0]))
    assert list(ok) == [False, True, True]


def test_inv_freq_is_torch_binary32():
    want = json.loads((HERE / "golden" / "rope_inv_freq.json").read_text())
    for D, theta in [(64, 10000.0), (128, 10000.0), (128, 500000.0)]:
        got = [f"{int(u):08x}" for u in rope.inv_freq(D, theta).view(np.uint32)]
        assert got == want[f"D{D}_theta{int(theta)}"], (D, theta)
    inv = rope.inv_freq(128, 10000.0)
    f64 = (1.0 / (10000.0 ** (np.arange(0, 128, 2) / 128))).astype(np.float32)
    assert int(np.count_nonzero(inv != f64)) == 19
    assert inv[0] == 1.0 and inv.dtype == np.float32


def test_generator_and_layer_share_tables():
    from open_transformers_amd.nn.layer import rope_tables as layer_tables

    c1, s1 = synthetic.rope_tables(256, 128, 10000.0)
    c2, s2 = layer_tables(256, 128, 10000.0)
    assert np.array_equal(c1.view(np.uint32), c2.numpy().view(np.uint32))
    assert np.array_equal(s1.view(np.uint32), s2.numpy().view(np.uint32))
