"""CPU-side checks of the C ABI: the library loads, exports every declared
symbol, and reports the reference's error variants for invalid inputs before
touching the device (validation runs first, as in rotary.rs)."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import spissa_amd as sa
from spissa_amd import _ffi

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(spissa_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = _ffi.load()
    names = declared_symbols()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) <= set(_ffi.SIGNATURES), sorted(set(names) - set(_ffi.SIGNATURES))


def test_library_targets_gfx950_only():
    blob = _ffi.LIB_PATH.read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    assert b"amdgcn-amd-amdhsa--gfx942" not in blob


def f32(*x):
    return np.array(x, dtype=np.float32)


def test_rope_validation_errors_without_device():
    cfg = sa.RotaryEmbeddingConfig(1, 1, 2, 2, 10000.0, 0)
    with pytest.raises(sa.InvalidTensorDataError):  # rotary.rs:148-152
        sa.apply_gemma_rotary_inplace(f32(1, 2), f32(1, 2), 1, 1, cfg, 0.0)
    with pytest.raises(sa.ShapeError):  # rotary.rs:145-147
        sa.apply_gemma_rotary_inplace(f32(1, 2), f32(1, 2), 0, 1, cfg, 1.0)
    with pytest.raises(sa.ShapeError):  # rotary.rs:86-96
        sa.apply_llama_rotary_inplace(f32(1, 2, 3), f32(1, 2), 1, 1, cfg)
    bad = sa.RotaryEmbeddingConfig(1, 1, 4, 3, 10000.0, 0)
    with pytest.raises(sa.ShapeError):  # rotary.rs:436-444 (odd rotary_dim)
        sa.apply_gpt_neox_rotary_inplace(f32(1, 2, 3, 4), f32(1, 2, 3, 4), bad)
    neg = sa.RotaryEmbeddingConfig(1, 1, 2, 2, -1.0, 0)
    with pytest.raises(sa.InvalidTensorDataError):  # rotary.rs:445-450
        sa.apply_gpt_neox_rotary_inplace(f32(1, 2), f32(1, 2), neg)
    assert sa.gpt_neox_rotary_dim(64, 0.25) == 16
    with pytest.raises(sa.InvalidTensorDataError):
        sa.gpt_neox_rotary_dim(64, 1.5)


def test_attention_validation_errors_without_device():
    cfg = sa.KvAttentionConfig(1, 3, 2, 2, True)  # 3 % 2 != 0, rotary.rs:500-505
    with pytest.raises(sa.ShapeError):
        sa.scaled_dot_product_attention_with_cache(f32(*range(6)), f32(1, 2, 3, 4), f32(1, 2, 3, 4), None, cfg)
    cfg = sa.KvAttentionConfig(0, 1, 1, 2, True)  # zero dim, rotary.rs:490-499
    with pytest.raises(sa.ShapeError):
        sa.scaled_dot_product_attention_with_cache(f32(), f32(), f32(), None, cfg)
    cfg = sa.KvAttentionConfig(1, 2, 1, 2, True)  # length mismatch, rotary.rs:516-525
    with pytest.raises(sa.ShapeError):
        sa.scaled_dot_product_attention_with_cache(f32(1, 2), f32(1, 2), f32(1, 2), None, cfg)
    with pytest.raises(sa.ShapeError):  # ops.rs:160-166
        sa.rms_norm(f32(1, 2, 3), f32(1, 1), 1, 2, 1e-6)
    with pytest.raises(sa.ShapeError):  # ops.rs:246-255
        sa.scaled_dot_product_attention(f32(1, 2), f32(1, 2), f32(1), 1, 1, 2, True)
    assert sa.scaled_dot_product_attention(f32(), f32(), f32(), 0, 1, 2, True).size == 0


def test_kv_cache_new_validation_without_device():
    with pytest.raises(sa.ShapeError):  # rotary.rs:207-211
        sa.KvCache(0, 2, 3)
    with pytest.raises(sa.ShapeError):  # rotary.rs:212-215
        sa.KvCache(1 << 40, 1 << 20, 1 << 20)


def test_is_global_layer_schedule():
    assert [i for i in range(26) if sa.is_global_layer(i, 6)] == [5, 11, 17, 23]
    assert sa.is_global_layer(3, 1) and sa.is_global_layer(3, 0)
