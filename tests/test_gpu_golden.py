"""GPU pipeline of each golden case against the committed fixtures.

The device path runs the whole layer the way a runtime would (device RoPE or
Gemma QK-norm prologue on the resident table, the fused decode step or the
prefill kernel, the in-place append) and is compared with the oracle values
stored in tests/golden/fixtures.json, without running the oracle here:
  output: max |gpu - ref| <= tol * max |ref| (tol 1e-4 for single-token f32
          decode, 1e-2 for the bf16-MFMA prefill / chunk);
  cache after the append: bitwise (RoPE, RMSNorm and append are exact).
"""
import json
from pathlib import Path

import numpy as np
import pytest

from tests.golden.cases import CASES, EPS, raw_inputs, sample_index, sha

pytestmark = pytest.mark.gpu

FIXTURES = json.loads((Path(__file__).resolve().parent / "golden" / "fixtures.json").read_text())["cases"]


def run_device(case):
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session
    from spissa_amd.rotary import KvAttentionConfig

    c = case
    s = Session(0)
    gemma = c.kind == "gemma"
    table = s.rope_table(_ffi.ROPE_GEMMA if gemma else _ffi.ROPE_LLAMA, c.D, c.base, c.divisor,
                         max_positions=c.P + c.S + 8)
    q, k, v, qn, kn = (torch.from_numpy(x).cuda() for x in raw_inputs(c))
    w = c.Hkv * c.D
    kp, kc = k[:c.P * w].contiguous(), k[c.P * w:].contiguous()
    vp, vc = v[:c.P * w].contiguous(), v[c.P * w:].contiguous()
    cache = s.kv_cache(c.Hkv, c.D, c.P + c.S)
    if c.P:
        dummy = torch.zeros(c.P * c.D, device="cuda")
        if gemma:
            s.gemma_qk_prologue(table, dummy, kp, c.P, 1, c.Hkv, c.D, qn, kn, EPS, 0, 1.0)
        else:
            s.rope_apply(table, dummy, kp, c.P, 1, c.Hkv, c.D, 0)
        s.append(cache, kp, vp, c.P)
    cfg = KvAttentionConfig(c.S, c.Hq, c.Hkv, c.D, True, c.window)
    out = torch.empty(c.n_out, device="cuda")
    if gemma:  # QK-norm -> RoPE -> prescale (x1.0), in place
        s.gemma_qk_prologue(table, q, kc, c.S, c.Hq, c.Hkv, c.D, qn, kn, EPS, c.P, 1.0)
    if c.S == 1:  # one fused launch pair: (RoPE +) attention + append
        s.decode_step(None if gemma else table, q, kc, vc, [cache], cfg, out)
    else:
        if not gemma:
            s.rope_apply(table, q, kc, c.S, c.Hq, c.Hkv, c.D, c.P)
        s.attention(q, kc, vc, cache, cfg, out)
        s.append(cache, kc, vc, c.S)
    s.sync()
    return out.cpu().numpy(), cache.keys(), cache.values()


@pytest.mark.parametrize("case", CASES, ids=[c.name for c in CASES])
def test_device_layer_matches_golden_fixture(gpu, case):
    print(f"[case] golden {case.name}", flush=True)
    fx = FIXTURES[case.name]
    got, keys, values = run_device(case)
    idx = np.arange(got.size) if fx["index"] == "all" else sample_index(got.size)
    ref = np.array(fx["values_f32_bits"], dtype=np.uint32).view(np.float32)
    tol = 1e-4 if case.S == 1 else 1e-2
    err = float(np.max(np.abs(got[idx].astype(np.float64) - ref))) / fx["out_max_abs"]
    assert err <= tol, f"{case.name}: {err:.3g} > {tol}"
    assert float(np.max(np.abs(got))) == pytest.approx(fx["out_max_abs"], rel=tol * 10)
    assert sha(keys) == fx["cache_keys_sha256"], "cache keys differ from the oracle's"
    assert sha(values) == fx["cache_values_sha256"], "cache values differ from the oracle's"
