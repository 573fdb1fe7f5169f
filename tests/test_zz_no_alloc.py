"""The allocation-free decode step (spissa_decode_step_device_noalloc) against
the workspace one (spissa_decode_step_device), through the C ABI.

Both run the fused RoPE + single-token attention + append of
rotary.rs:75-125, 335-415 and 226-256 on identical caches and inputs. The bar
is the f32 decode bar, max|a - b| / max|b| <= 1e-4 (the results are identical
when both use the same key splits), and the appended cache rows must be
bitwise equal. Two calls in a row, the second on a smaller input, share the
static scratch array; a third case makes the scratch array coarsen the key
splits; an oversized launch is rejected before anything runs.
"""
import numpy as np
import pytest

from spissa_amd import _ffi
from spissa_amd.synth import normal_f32, seed_for
from tests.helpers import assert_bitwise, rel_err

pytestmark = pytest.mark.gpu

DECODE_TOL = 1e-4


def make_caches(s, Hkv, D, past, cap, seed):
    """Two identical sets of caches holding `past[b]` seeded rows each."""
    a, b = [], []
    for i, P in enumerate(past):
        ca, cb = s.kv_cache(Hkv, D, cap), s.kv_cache(Hkv, D, cap)
        if P:
            k = normal_f32(seed_for(seed, i, 0, "k"), P * Hkv * D)
            v = normal_f32(seed_for(seed, i, 0, "v"), P * Hkv * D)
            ca.append(k, v, P)
            cb.append(k, v, P)
        a.append(ca), b.append(cb)
    return a, b


def step_both(gpu, s, table, Hq, Hkv, D, past, W, seed):
    import torch

    print(f"[case] noalloc decode Hq={Hq} Hkv={Hkv} D={D} B={len(past)} past={past[:4]} W={W}", flush=True)
    B = len(past)
    cap = max(past) + 2
    ca, cb = make_caches(s, Hkv, D, past, cap, seed)
    q = torch.from_numpy(normal_f32(seed_for(seed, 99, 0, "q"), B * Hq * D)).cuda()
    k = torch.from_numpy(normal_f32(seed_for(seed, 99, 0, "k"), B * Hkv * D)).cuda()
    v = torch.from_numpy(normal_f32(seed_for(seed, 99, 0, "v"), B * Hkv * D)).cuda()
    out_a = torch.full((B * Hq * D,), float("nan"), device="cuda")
    out_b = torch.full((B * Hq * D,), float("nan"), device="cuda")
    torch.cuda.synchronize()
    cfg = gpu.KvAttentionConfig(1, Hq, Hkv, D, True, W)
    s.decode_step(table, q, k, v, ca, cfg, out_a)
    s.decode_step_noalloc(table, q, k, v, cb, cfg, out_b)
    s.sync()
    a, b = out_a.cpu().numpy(), out_b.cpu().numpy()
    assert np.all(np.isfinite(b))
    err = rel_err(b, a)
    print(f"[noalloc] rel err vs workspace step {err:.2e}", flush=True)
    assert err <= DECODE_TOL
    for x, y in zip(ca, cb):
        assert x.len() == y.len()
        assert_bitwise(y.keys(), x.keys(), "keys after the append")
        assert_bitwise(y.values(), x.values(), "values after the append")
    return a, b


def test_noalloc_decode_step_two_calls_second_smaller(gpu):
    from spissa_amd.device import Session

    s = Session(0)
    table = s.rope_table(_ffi.ROPE_LLAMA, 128, 500000.0, max_positions=8200)
    # Llama-3.2-3B decode at 8192 cached tokens, batch 2 (same key splits as
    # the workspace path: identical results)
    a, b = step_both(gpu, s, table, 24, 8, 128, [8192, 8000], 0, 31)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # then a smaller launch on the same scratch array: batch 1 at 512 tokens
    a, b = step_both(gpu, s, table, 24, 8, 128, [512], 0, 32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_noalloc_decode_step_coarsens_splits_to_the_scratch_array(gpu):
    from spissa_amd.device import Session, plan_attention

    s = Session(0)
    past = [16384] + [64] * 15
    cfg = gpu.KvAttentionConfig(1, 32, 8, 256, True, 0)
    assert plan_attention(cfg, past)["partial_bytes"] > 8 << 20  # the workspace step splits wider
    step_both(gpu, s, None, 32, 8, 256, past, 0, 33)
    # windowed (Gemma local layer shape), smaller again
    step_both(gpu, s, None, 8, 4, 256, [3000, 100], 1024, 34)


def test_noalloc_decode_step_rejects_partials_beyond_the_array(gpu):
    import torch

    from spissa_amd.device import Session

    s = Session(0)
    Hq, D, B = 512, 256, 16  # 16 x 512 x 258 floats = 8.45 MB > 8 MiB
    caches = [s.kv_cache(Hq, D, 4) for _ in range(B)]
    q = torch.zeros(B * Hq * D, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(gpu.ShapeError):
        s.decode_step_noalloc(None, q, q, q, caches, gpu.KvAttentionConfig(1, Hq, Hq, D, True), out)
    assert all(c.len() == 0 for c in caches)


def test_noalloc_decode_step_under_graph_capture(gpu):
    """The use the entry point is for: one call captured into a HIP graph on a
    fresh session (no call before the capture), then replayed three times
    with eager work and synchronisation between the replays. Every replay
    matches the workspace step on an identical cache (1e-4) and the previous
    replay (bitwise); the appended row is the workspace step's, bitwise."""
    import torch

    from spissa_amd.device import Session

    print("[case] noalloc decode step captured in a graph, 3 replays", flush=True)
    Hq, Hkv, D, P = 24, 8, 128, 8192
    stream = torch.cuda.Stream()
    s = Session(0, stream=stream)
    table = s.rope_table(_ffi.ROPE_LLAMA, D, 500000.0, max_positions=P + 8)
    ca, cb = make_caches(s, Hkv, D, [P], P + 1, 36)
    q = torch.from_numpy(normal_f32(seed_for(36, 99, 0, "q"), Hq * D)).cuda()
    k = torch.from_numpy(normal_f32(seed_for(36, 99, 0, "k"), Hkv * D)).cuda()
    v = torch.from_numpy(normal_f32(seed_for(36, 99, 0, "v"), Hkv * D)).cuda()
    out_g = torch.full((Hq * D,), float("nan"), device="cuda")
    out_w = torch.full((Hq * D,), float("nan"), device="cuda")
    cfg = gpu.KvAttentionConfig(1, Hq, Hkv, D, True, 0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        s.decode_step_noalloc(table, q, k, v, cb, cfg, out_g)
    assert cb[0].len() == P + 1  # the host length advanced at capture
    s.decode_step(table, q, k, v, ca, cfg, out_w)
    s.sync()
    want = out_w.cpu().numpy()
    prev = None
    for r in range(3):
        out_g.fill_(float("nan"))  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        s.sync()
        got = out_g.cpu().numpy()
        assert np.all(np.isfinite(got)), r
        err = rel_err(got, want)
        print(f"[noalloc graph] replay {r}: rel err vs workspace step {err:.2e}", flush=True)
        assert err <= DECODE_TOL, r
        if prev is not None:
            assert np.array_equal(got.view(np.uint32), prev.view(np.uint32)), r
        prev = got
    w = Hkv * D
    assert_bitwise(cb[0].keys()[P * w:], ca[0].keys()[P * w:], "appended key")
    assert_bitwise(cb[0].values()[P * w:], ca[0].values()[P * w:], "appended value")
    del g
