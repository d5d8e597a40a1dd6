"""Shared pytest setup: the ``gpu`` marker, import paths and seeded inputs."""

from __future__ import annotations

import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libmt_attn.so")


@pytest.fixture(scope="session")
def mta():
    """The package under test (its directory name carries a hyphen)."""
    return importlib.import_module("mega-trading_amd")
