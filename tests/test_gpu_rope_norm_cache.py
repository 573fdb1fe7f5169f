"""GPU parity, bit-exact part: RoPE (three kinds, drop-in and resident-table
paths), RMSNorm / Gemma QK-norm prologue, and KV-cache append / truncate /
clear / clone indexing, all against the CPU oracle on identical seeded inputs."""
import numpy as np
import pytest

import oracle as o
from spissa_amd.synth import normal_f32, seed_for
from tests.helpers import assert_bitwise

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("S,Hq,Hkv,D,rot,base,off", [
    (1, 32, 8, 64, 64, 500000.0, 512),        # config 1 decode position
    (7, 24, 8, 128, 128, 500000.0, 8185),     # config 3 near 8192
    (64, 4, 1, 256, 256, 10000.0, 0),         # gemma-1B local shape as llama
    (3, 2, 1, 6, 4, 10000.0, 5),              # partial rotary, odd-sized head
    (2, 4, 2, 80, 80, 1e6, 32760),
])
def test_llama_rope_bitwise(gpu, S, Hq, Hkv, D, rot, base, off):
    q = normal_f32(seed_for(90, S, 0, "q"), S * Hq * D)
    k = normal_f32(seed_for(90, S, 0, "k"), S * Hkv * D)
    rq, rk = q.copy(), k.copy()
    o.apply_llama_rotary_inplace(rq, rk, Hq, Hkv, S, D, rot, base, off)
    cfg = gpu.RotaryEmbeddingConfig(S, Hq, D, rot, base, off)
    gpu.apply_llama_rotary_inplace(q, k, Hq, Hkv, cfg)
    assert_bitwise(q, rq, "q")
    assert_bitwise(k, rk, "k")


def test_llama_rope_longrope_freq_scale_bitwise(gpu):
    S, Hq, Hkv, D, rot = 5, 4, 2, 96, 64  # Phi-3-like partial rotary with a divisor per pair
    fs = (1.0 + np.arange(rot // 2, dtype=np.float32) * np.float32(0.37)).astype(np.float32)
    q, k = normal_f32(91, S * Hq * D), normal_f32(92, S * Hkv * D)
    rq, rk = q.copy(), k.copy()
    o.apply_llama_rotary_inplace(rq, rk, Hq, Hkv, S, D, rot, 10000.0, 3000, fs)
    gpu.apply_llama_rotary_inplace(q, k, Hq, Hkv, gpu.RotaryEmbeddingConfig(S, Hq, D, rot, 10000.0, 3000), fs)
    assert_bitwise(q, rq, "q")
    assert_bitwise(k, rk, "k")


@pytest.mark.parametrize("base,div,off", [(1e6, 8.0, 32767), (10000.0, 1.0, 4095), (1e6, 1.0, 16383)])
def test_gemma_rope_bitwise(gpu, base, div, off):
    S, Hq, Hkv, D = 3, 8, 4, 256
    q, k = normal_f32(93, S * Hq * D), normal_f32(94, S * Hkv * D)
    rq, rk = q.copy(), k.copy()
    o.apply_gemma_rotary_inplace(rq, rk, Hq, Hkv, S, D, D, base, off, div)
    gpu.apply_gemma_rotary_inplace(q, k, Hq, Hkv, gpu.RotaryEmbeddingConfig(S, Hq, D, D, base, off), div)
    assert_bitwise(q, rq, "q")
    assert_bitwise(k, rk, "k")


def test_gpt_neox_rope_bitwise_and_tail_untouched(gpu):
    S, H, D, rot = 9, 8, 64, 16
    q, k = normal_f32(95, S * H * D), normal_f32(96, S * H * D)
    rq, rk = q.copy(), k.copy()
    o.apply_gpt_neox_rotary_inplace(rq, rk, S, H, D, rot, 10000.0, 100)
    tail = q.reshape(S, H, D)[:, :, rot:].copy()
    gpu.apply_gpt_neox_rotary_inplace(q, k, gpu.RotaryEmbeddingConfig(S, H, D, rot, 10000.0, 100))
    assert_bitwise(q, rq, "q")
    assert_bitwise(k, rk, "k")
    assert_bitwise(q.reshape(S, H, D)[:, :, rot:], tail, "tail")


def test_resident_rope_table_matches_drop_in(gpu):
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session

    s = Session(0)
    S, Hq, Hkv, D = 33, 24, 8, 128
    q, k = normal_f32(97, S * Hq * D), normal_f32(98, S * Hkv * D)
    rq, rk = q.copy(), k.copy()
    o.apply_llama_rotary_inplace(rq, rk, Hq, Hkv, S, D, D, 500000.0, 8000)
    t = s.rope_table(_ffi.ROPE_LLAMA, D, 500000.0, max_positions=8192 + 64)
    dq, dk = torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda()
    s.rope_apply(t, dq, dk, S, Hq, Hkv, D, 8000)
    s.sync()
    assert_bitwise(dq.cpu().numpy(), rq, "q")
    assert_bitwise(dk.cpu().numpy(), rk, "k")
    with pytest.raises(gpu.ShapeError):
        s.rope_apply(t, dq, dk, S, Hq, Hkv, D, 8192 + 64 - S + 1)


@pytest.mark.parametrize("rows,cols", [(4096 * 8, 256), (1, 3072), (16, 1152), (7, 2560), (3, 8192), (2, 9000)])
def test_rms_norm_bitwise(gpu, rows, cols):
    # head rows (one thread per row), model-width rows (a workgroup per row), and
    # rows beyond the staged width (one thread per row again)
    x, w = normal_f32(99, rows * cols), normal_f32(100, cols, 1.0, 0.1)
    assert_bitwise(gpu.rms_norm(x, w, rows, cols, 1e-6), o.rms_norm(x, w, rows, cols, 1e-6), "rms_norm")


@pytest.mark.parametrize("layer,S,Hq,Hkv,D", [
    (0, 17, 8, 4, 256), (5, 17, 8, 4, 256),
    (0, 5, 2, 1, 128),   # 15 rows: the last workgroup has one idle wave
    (5, 9, 4, 1, 64),
])
def test_gemma_qk_prologue_device_bitwise(gpu, layer, S, Hq, Hkv, D):
    """models/gemma/generate.rs:232-278 on the device (one wave per row, lane 0
    summing the staged squares in index order) against the oracle, bitwise."""
    import torch

    from spissa_amd import _ffi
    from spissa_amd.device import Session

    off = 1000
    is_global = gpu.is_global_layer(layer, 6)
    base, div = (1e6, 8.0) if is_global else (10000.0, 1.0)
    q, k = normal_f32(seed_for(5, layer, 0, "q"), S * Hq * D), normal_f32(seed_for(5, layer, 0, "k"), S * Hkv * D)
    qn = normal_f32(seed_for(5, layer, 0, "qnorm"), D, 1.0, 0.1)
    kn = normal_f32(seed_for(5, layer, 0, "knorm"), D, 1.0, 0.1)
    rq, rk = q.copy(), k.copy()
    o.gemma_qk_prologue(rq, rk, S, Hq, Hkv, D, qn, kn, 1e-6, base, div, off, float(D))
    s = Session(0)
    t = s.rope_table(_ffi.ROPE_GEMMA, D, base, div, max_positions=2048)
    dq, dk = torch.from_numpy(q).cuda(), torch.from_numpy(k).cuda()
    prescale = float(np.float32(np.float32(1.0) / np.sqrt(np.float32(D))) * np.sqrt(np.float32(D)))
    s.gemma_qk_prologue(t, dq, dk, S, Hq, Hkv, D, torch.from_numpy(qn).cuda(), torch.from_numpy(kn).cuda(),
                        1e-6, off, prescale)
    s.sync()
    assert_bitwise(dq.cpu().numpy(), rq, "q")
    assert_bitwise(dk.cpu().numpy(), rk, "k")


def test_kv_cache_reference_semantics_on_device(gpu):
    # rotary.rs:772-824 on the device cache, compared to the oracle after every step.
    f = lambda *x: np.array(x, dtype=np.float32)
    c = gpu.KvCache(1, 2, 3)
    c.append(f(1, 2, 3, 4), f(5, 6, 7, 8), 2)
    assert c.len() == 2 and list(c.keys()) == [1, 2, 3, 4] and list(c.values()) == [5, 6, 7, 8]
    with pytest.raises(gpu.ShapeError):
        c.append(f(9, 10, 11, 12), f(13, 14, 15, 16), 2)
    assert c.len() == 2 and list(c.keys()) == [1, 2, 3, 4]
    with pytest.raises(gpu.ShapeError):
        c.append(f(9, 10), f(13, 14), 0)
    with pytest.raises(gpu.ShapeError):
        c.append(f(9, 10, 1), f(13, 14, 1), 1)
    c2 = gpu.KvCache(2, 3, 4)
    c2.append(np.arange(1, 13, dtype=np.float32), np.arange(13, 25, dtype=np.float32), 2)
    c2.truncate(1)
    assert c2.len() == 1 and list(c2.keys()) == [1, 2, 3, 4, 5, 6] and list(c2.values()) == [13, 14, 15, 16, 17, 18]
    assert c2.resident_bytes() == 48
    with pytest.raises(gpu.ShapeError):
        c2.truncate(2)
    assert c2.len() == 1
    c2.clear()
    assert c2.is_empty() and c2.keys().size == 0
    assert (c2.max_seq_len(), c2.num_heads(), c2.head_dim()) == (4, 2, 3)


def test_kv_cache_indexing_bitwise_at_scale(gpu):
    Hkv, D, cap = 8, 128, 8192 + 64
    dev, ref = gpu.KvCache(Hkv, D, cap), o.KvCache(Hkv, D, cap)
    w = Hkv * D
    steps = [4096, 1, 1, 2047, 3, 1]
    for i, n in enumerate(steps):
        k = normal_f32(seed_for(3, i, 0, "k"), n * w)
        v = normal_f32(seed_for(3, i, 0, "v"), n * w)
        dev.append(k, v, n)
        ref.append(k, v, n)
        if i == 3:
            dev.truncate(5000)
            ref.truncate(5000)
    assert dev.len() == ref.len()
    assert_bitwise(dev.keys(), ref.keys(), "keys")
    assert_bitwise(dev.values(), ref.values(), "values")
    cl = dev.clone()
    assert_bitwise(cl.keys(), ref.keys(), "clone keys")
    cl.append(np.ones(w, np.float32), np.ones(w, np.float32), 1)
    assert cl.len() == dev.len() + 1 and dev.len() == ref.len()
    assert dev.resident_bytes() == ref.resident_bytes()
