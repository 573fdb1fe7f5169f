"""The committed golden fixtures (tests/golden/fixtures.json) against this host.

Re-running the oracle on the seeded inputs must reproduce every fixture bit
for bit: the input hashes pin the generator, the output and cache hashes pin
the C restatement (and the host libm it calls for RoPE angles), so a GPU box
whose host computes differently is caught before its parity tests run.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle as o
from tests.golden.cases import CASES, raw_inputs, run_oracle, sample_index, sha

FIXTURES = json.loads((Path(__file__).resolve().parent / "golden" / "fixtures.json").read_text())["cases"]


def test_every_case_has_a_fixture():
    assert sorted(FIXTURES) == sorted(c.name for c in CASES)


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_oracle_reproduces_fixture_bitwise(oracle, case):
    fx = FIXTURES[case.name]
    assert sha(*raw_inputs(case)) == fx["inputs_sha256"], "seeded generator changed"
    out, keys, values = run_oracle(case, o)
    assert sha(out) == fx["out_sha256"]
    assert sha(keys) == fx["cache_keys_sha256"]
    assert sha(values) == fx["cache_values_sha256"]
    idx = np.arange(out.size) if fx["index"] == "all" else sample_index(out.size)
    assert np.array_equal(out[idx].view(np.uint32), np.array(fx["values_f32_bits"], dtype=np.uint32))
    assert float(np.max(np.abs(out))) == fx["out_max_abs"]
