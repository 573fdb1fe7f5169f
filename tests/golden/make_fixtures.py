"""Writes tests/golden/fixtures.json from the CPU oracle (run from the repo root).

    python -m tests.golden.make_fixtures

For every case of cases.py the file records the SHA-256 of the seeded inputs
(pins the generator), of the oracle's output and of the cache after the append
(pins the oracle bit for bit), the output's max |value|, and output values as
float32 bit patterns: all of them for outputs of at most 4096 elements, else a
fixed sample (cases.sample_index). GPU tests compare against these values
without running the oracle.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import oracle as o  # noqa: E402
from tests.golden.cases import CASES, raw_inputs, run_oracle, sample_index, sha  # noqa: E402

OUT = Path(__file__).resolve().parent / "fixtures.json"
FULL_LIMIT = 4096


def fixture(case) -> dict:
    out, keys, values = run_oracle(case, o)
    idx = np.arange(out.size) if out.size <= FULL_LIMIT else sample_index(out.size)
    return {
        "params": {k: getattr(case, k) for k in ("config", "kind", "Hq", "Hkv", "D", "P", "S", "base",
                                                   "divisor", "window", "layer")},
        "inputs_sha256": sha(*raw_inputs(case)),
        "out_sha256": sha(out),
        "cache_keys_sha256": sha(keys),
        "cache_values_sha256": sha(values),
        "out_max_abs": float(np.max(np.abs(out))),
        "index": "all" if out.size <= FULL_LIMIT else "sample",
        "values_f32_bits": out[idx].view(np.uint32).tolist(),
    }


def main() -> None:
    o.build()
    data = {"generator": "tests/golden/make_fixtures.py (oracle/spissa_oracle.c)", "cases": {}}
    for case in CASES:
        data["cases"][case.name] = fixture(case)
        print(case.name, data["cases"][case.name]["out_sha256"][:16], flush=True)
    OUT.write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
