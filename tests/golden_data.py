"""Loaders for the committed golden fixtures in ``tests/golden/`` (not a test module).

The fixtures are data written by ``tests/golden/make_golden.py`` from the CPU
oracle; they travel with the repository, so GPU tests compare against them
without recomputing the oracle at full size.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def load_npz(name: str) -> dict:
    with np.load(GOLDEN / name, allow_pickle=False) as data:
        return {key: data[key] for key in data.files}


def load_json(name: str) -> dict:
    return json.loads((GOLDEN / name).read_text())
