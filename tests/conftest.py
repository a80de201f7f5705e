"""Test configuration: puts the repository root on sys.path, imports the
package directory ``open-transformers_amd`` as ``open_transformers_amd`` and
registers the markers (``gpu`` = needs an MI355X, run with ``-m gpu``)."""

from __future__ import annotations

import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (run with -m gpu)")
    config.addinivalue_line("markers", "slow: long-running CPU test")
