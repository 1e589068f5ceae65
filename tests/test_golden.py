"""The committed golden fixtures are what the oracle produces today.

``tests/golden/make_golden.py`` is re-run into a temporary directory and every
array (and the config-0 JSON record) must match the committed bytes, so a
change to the oracle or to the seeded draws that would silently move the truth
the GPU tests compare against fails here first.
"""
from __future__ import annotations

import importlib.util
import json

import numpy as np
import pytest

from tests.golden_data import GOLDEN, load_json, load_npz


def _generator():
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


@pytest.mark.parametrize("name,builder,args", [
    ("w3_gptq_64x256.npz", "w3_gptq_case", (64, 256)),
    ("w3_gptq_288x384.npz", "w3_gptq_case", (288, 384)),
    ("norms_config2.npz", "norms_case", ()),
    ("two_base_hybrid_257x384.npz", "hybrid_case", ()),
    ("two_base_rank_one_64x256.npz", "rank_one_case", ()),
])
def test_oracle_regenerates_npz_fixture(tmp_path, name, builder, args):
    module = _generator()
    getattr(module, builder)(*args, tmp_path / name)
    fresh = dict(np.load(tmp_path / name, allow_pickle=False))
    committed = load_npz(name)
    assert sorted(fresh) == sorted(committed)
    for key in committed:
        assert fresh[key].dtype == committed[key].dtype, key
        np.testing.assert_array_equal(fresh[key], committed[key], err_msg=key)


def test_oracle_regenerates_config0_record(tmp_path):
    module = _generator()
    module.config0_case(tmp_path / "c0.json")
    assert json.loads((tmp_path / "c0.json").read_text()) == load_json("w3_q_proj_config0.json")


def test_config0_record_is_consistent():
    record = load_json("w3_q_proj_config0.json")
    y = np.asarray(record["y_exact_sample"])
    assert len(record["sample_rows"]) == 64 == len(set(record["sample_rows"]))
    assert np.all(np.abs(y) <= record["y_exact_abs_max"])
    # bf16 samples are the nearest bf16 values of the exact samples
    assert np.all(np.abs(np.asarray(record["y_bf16_sample"]) - y) <= 2.0 ** -8 * np.abs(y) + 1e-30)
