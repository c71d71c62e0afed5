"""Shared pytest configuration: the ``gpu`` marker and repository import path."""

from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config) -> None:
    config.addinivalue_line("markers", "gpu: needs a real MI355X (gfx950) and the built HIP library")
