"""Seeded random GEMM shapes against the CPU oracle (ops.rs:62-105 arithmetic).

Above 64 tokens the bf16 projections run the MFMA GEMM in one of two tile
shapes: 128 x 256 tiles, two workgroups per CU, or 256 x 320 tiles, one per
CU, when the small tiles would leave a second round of slots mostly empty.
This sweeps shapes on both sides of that choice, with ragged edges, short and
odd k-tile counts, with and without bias, and checks sampled rows (the first,
the last and rows around tile edges, every output column) against the oracle
at the f32 bar: max |gpu - oracle| <= 1e-4 x max |oracle|.
"""
import numpy as np
import pytest

import oracle as o
import spissa_amd as sa
from spissa_amd.linear import DTYPE_BF16, StreamingLinearConfig
from spissa_amd.synth import normal_f32, seed_for
from tests.helpers import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-4
N_CASES = 16
CUS = 256  # MI355X


def wide_tiles(m: int, n: int, cus: int = CUS) -> bool:
    """The launch's choice (linear.hip, linear_gemm_wide), restated to label the cases."""
    small = -(-m // 128) * -(-n // 256)
    wide = -(-m // 256) * -(-n // 320)
    return 5 * -(-wide // cus) < 4 * -(-small // (2 * cus))


def _cases():
    rng = np.random.RandomState(20261204)
    out = []
    while len(out) < N_CASES:
        want_wide = len(out) % 2 == 0
        if want_wide:
            m = int(rng.randint(2049, 4600))
            n = int(rng.randint(4200, 6200))
        else:
            m = int(rng.randint(65, 3000))
            n = int(rng.randint(1, 4000))
        k = int(32 * rng.randint(1, 7))
        bias = bool(rng.rand() < 0.5)
        if wide_tiles(m, n) != want_wide:
            continue
        out.append((m, n, k, bias))
    return out


CASES = _cases()


@pytest.mark.parametrize("m,n,k,bias", CASES,
                         ids=[f"{c[0]}x{c[1]}x{c[2]}-{'wide' if wide_tiles(c[0], c[1]) else 'small'}-"
                              f"{'bias' if c[3] else 'nobias'}" for c in CASES])
def test_random_gemm_shape(gpu, m, n, k, bias):
    print(f"[case] random gemm {m} x {n} x {k} bias={bias} wide={wide_tiles(m, n)}", flush=True)
    w = normal_f32(seed_for(70, m, n, "q", k), n * k, 0.0, 0.05)
    wb = ((w.view(np.uint32).astype(np.uint64) + 0x7FFF + ((w.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    x = normal_f32(seed_for(70, m, n, "k", k), m * k)
    b = normal_f32(seed_for(70, m, n, "v", k), n) if bias else None
    got = sa.linear(sa.LinearWeight(wb, DTYPE_BF16, n, k), x, b, StreamingLinearConfig(m, k, n))
    assert np.isfinite(got).all()
    rows = {0, 1, 127, 128, 255, 256, m // 2, m - 2, m - 1}
    pick = np.array(sorted(r for r in rows if 0 <= r < m))
    ref = o.linear(x.reshape(m, k)[pick].ravel().copy(), wb, o.DTYPE_BF16, b, len(pick), k, n)
    err = rel_err(got.reshape(m, n)[pick].ravel(), ref)
    print(f"[gemm] {m} x {n} x {k}: rel err {err:.2e}", flush=True)
    assert err <= TOL
