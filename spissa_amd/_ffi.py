"""ctypes binding of include/spissa_hip.h (libspissa_hip.so, built in-tree).

Loading fails loudly when the library has not been built: there is no CPU
fallback behind this package.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libspissa_hip.so"

OK = 0
ERR_SHAPE = 1
ERR_INVALID_TENSOR_DATA = 2
ERR_DEVICE = 3
ERR_ARGUMENT = 4

ROPE_LLAMA = 0
ROPE_GEMMA = 1
ROPE_NEOX = 2

PREFILL_BF16 = 0
PREFILL_F32 = 1

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

c_size = C.c_size_t
c_float_p = C.POINTER(C.c_float)
c_void_p = C.c_void_p


class LinearConfigC(C.Structure):
    """spissa_linear_config (streaming/mod.rs:511-516)."""

    _fields_ = [("batch", c_size), ("in_features", c_size), ("out_features", c_size)]


class AttentionLayerC(C.Structure):
    """spissa_attention_layer (models/gemma/generate.rs:178-312)."""

    _fields_ = [
        ("hidden", c_size), ("q_heads", c_size), ("kv_heads", c_size), ("head_dim", c_size),
        ("q_weight", c_void_p), ("k_weight", c_void_p), ("v_weight", c_void_p), ("o_weight", c_void_p),
        ("d_input_norm", c_void_p), ("d_q_norm", c_void_p), ("d_k_norm", c_void_p), ("d_post_norm", c_void_p),
        ("eps", C.c_float), ("rope", c_void_p), ("q_prescale", C.c_float), ("causal", C.c_int),
        ("window", c_size),
    ]


class RotaryConfigC(C.Structure):
    """spissa_rotary_config (rotary.rs:6-14)."""

    _fields_ = [
        ("seq_len", c_size),
        ("num_heads", c_size),
        ("head_dim", c_size),
        ("rotary_dim", c_size),
        ("base", C.c_float),
        ("position_offset", c_size),
    ]


class AttnConfigC(C.Structure):
    """spissa_kv_attention_config (rotary.rs:320-327 + window)."""

    _fields_ = [
        ("query_len", c_size),
        ("num_heads", c_size),
        ("kv_heads", c_size),
        ("head_dim", c_size),
        ("causal", C.c_int),
        ("window", c_size),
    ]


KERNEL_DECODE = 0
KERNEL_PREFILL_BF16 = 1
KERNEL_GENERIC = 2


class AttentionPlanC(C.Structure):
    """spissa_attention_plan: the launch geometry of one attention call."""

    _fields_ = [
        ("path", C.c_int), ("heads_per_block", C.c_int), ("head_blocks", C.c_int),
        ("keys_per_split", C.c_int), ("splits", C.c_int), ("token_split", C.c_int), ("tiles_per_split", C.c_int),
        ("tile_keys", C.c_int), ("workgroup_queries", C.c_int), ("block_waves", C.c_int),
        ("xcd_group", C.c_int), ("max_tiles", C.c_long), ("workgroups", c_size), ("partial_bytes", c_size), ("stage_bytes", c_size),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    "spissa_last_error": (C.c_char_p, []),
    "spissa_version": (C.c_char_p, []),
    "spissa_session_create": (C.c_int, [C.c_int, c_void_p, C.POINTER(c_void_p)]),
    "spissa_session_destroy": (None, [c_void_p]),
    "spissa_default_session": (C.c_int, [C.POINTER(c_void_p)]),
    "spissa_session_sync": (C.c_int, [c_void_p]),
    "spissa_session_stream": (c_void_p, [c_void_p]),
    "spissa_session_device": (C.c_int, [c_void_p]),
    "spissa_session_set_prefill_precision": (C.c_int, [c_void_p, C.c_int]),
    "spissa_kv_cache_new": (C.c_int, [c_size, c_size, c_size, C.POINTER(c_void_p)]),
    "spissa_kv_cache_new_in": (C.c_int, [c_void_p, c_size, c_size, c_size, C.POINTER(c_void_p)]),
    "spissa_kv_cache_free": (None, [c_void_p]),
    "spissa_kv_cache_clone": (C.c_int, [c_void_p, C.POINTER(c_void_p)]),
    "spissa_kv_cache_append": (C.c_int, [c_void_p, c_float_p, c_size, c_float_p, c_size, c_size]),
    "spissa_kv_cache_append_device": (C.c_int, [c_void_p, c_void_p, c_void_p, c_size]),
    "spissa_kv_cache_clear": (None, [c_void_p]),
    "spissa_kv_cache_truncate": (C.c_int, [c_void_p, c_size]),
    "spissa_kv_cache_len": (c_size, [c_void_p]),
    "spissa_kv_cache_is_empty": (C.c_int, [c_void_p]),
    "spissa_kv_cache_max_seq_len": (c_size, [c_void_p]),
    "spissa_kv_cache_num_heads": (c_size, [c_void_p]),
    "spissa_kv_cache_head_dim": (c_size, [c_void_p]),
    "spissa_kv_cache_resident_bytes": (c_size, [c_void_p]),
    "spissa_kv_cache_read_keys": (C.c_int, [c_void_p, c_float_p, c_size]),
    "spissa_kv_cache_read_values": (C.c_int, [c_void_p, c_float_p, c_size]),
    "spissa_kv_cache_device_keys": (c_void_p, [c_void_p]),
    "spissa_kv_cache_device_values": (c_void_p, [c_void_p]),
    "spissa_gpt_neox_rotary_dim": (C.c_int, [c_size, C.c_float, C.POINTER(c_size)]),
    "spissa_apply_gpt_neox_rotary_inplace": (
        C.c_int, [c_float_p, c_size, c_float_p, c_size, C.POINTER(RotaryConfigC)]),
    "spissa_apply_llama_rotary_inplace": (
        C.c_int,
        [c_float_p, c_size, c_float_p, c_size, c_size, c_size, C.POINTER(RotaryConfigC), c_float_p,
         c_size]),
    "spissa_apply_gemma_rotary_inplace": (
        C.c_int,
        [c_float_p, c_size, c_float_p, c_size, c_size, c_size, C.POINTER(RotaryConfigC), C.c_float]),
    "spissa_rope_table_new": (
        C.c_int,
        [c_void_p, C.c_int, c_size, C.c_float, C.c_float, c_float_p, c_size, c_size,
         C.POINTER(c_void_p)]),
    "spissa_rope_table_free": (None, [c_void_p]),
    "spissa_rope_apply_device": (
        C.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_size, c_size, c_size, c_size]),
    "spissa_rms_norm": (
        C.c_int, [c_float_p, c_size, c_float_p, c_size, c_size, c_size, C.c_float, c_float_p, c_size]),
    "spissa_rms_norm_device": (
        C.c_int, [c_void_p, c_void_p, c_void_p, c_size, c_size, C.c_float, c_void_p]),
    "spissa_is_global_layer": (C.c_int, [c_size, c_size]),
    "spissa_gemma_qk_prologue_device": (
        C.c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_size, c_size, c_size, c_void_p, c_void_p,
         C.c_float, c_size, C.c_float]),
    "spissa_scaled_dot_product_attention_with_cache": (
        C.c_int,
        [c_float_p, c_size, c_float_p, c_size, c_float_p, c_size, c_void_p, C.POINTER(AttnConfigC),
         c_float_p, c_size]),
    "spissa_attention_device": (
        C.c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, C.POINTER(AttnConfigC), c_void_p]),
    "spissa_attention_decode_batch_device": (
        C.c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, C.POINTER(c_void_p), c_size,
         C.POINTER(AttnConfigC), c_void_p]),
    "spissa_decode_step_device": (
        C.c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, C.POINTER(c_void_p), c_size,
         C.POINTER(AttnConfigC), c_void_p]),
    "spissa_gemma_decode_step_device": (
        C.c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, C.POINTER(c_void_p), c_size,
         C.POINTER(AttnConfigC), c_void_p, c_void_p, C.c_float, C.c_float, c_void_p]),
    "spissa_decode_step_device_noalloc": (
        C.c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, C.POINTER(c_void_p), c_size,
         C.POINTER(AttnConfigC), c_void_p]),
    "spissa_plan_attention": (
        C.c_int,
        [C.POINTER(AttnConfigC), C.POINTER(c_size), c_size, C.c_int, C.c_int, C.c_int,
         C.POINTER(AttentionPlanC)]),
    "spissa_hbm_read_probe_device": (C.c_int, [c_void_p, c_void_p, c_size, c_void_p]),
    "spissa_mfma_rate_probe_device": (C.c_int, [c_void_p, C.c_int, c_void_p, C.POINTER(C.c_double)]),
    "spissa_gemma_prefill_step_device": (
        C.c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, C.POINTER(AttnConfigC), c_void_p, c_void_p,
         C.c_float, C.c_float, c_void_p]),
    "spissa_prefill_step_device": (
        C.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, C.POINTER(AttnConfigC), c_void_p]),
    "spissa_attention_cached_device": (
        C.c_int, [c_void_p, c_void_p, c_void_p, C.POINTER(AttnConfigC), c_void_p]),
    "spissa_scaled_dot_product_attention": (
        C.c_int,
        [c_float_p, c_size, c_float_p, c_size, c_float_p, c_size, c_size, c_size, c_size, C.c_int,
         c_float_p, c_size]),
    "spissa_linear_weight_new": (
        C.c_int, [c_void_p, C.c_int, c_size, c_size, c_void_p, c_size, C.POINTER(c_void_p)]),
    "spissa_linear_weight_free": (None, [c_void_p]),
    "spissa_linear": (
        C.c_int, [c_void_p, c_float_p, c_size, c_float_p, c_size, C.POINTER(LinearConfigC), c_float_p,
                  c_size]),
    "spissa_linear_device": (C.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_void_p]),
    "spissa_lm_head_logits": (C.c_int, [c_void_p, c_float_p, c_size, c_float_p, c_size]),
    "spissa_sample_argmax": (C.c_int, [c_void_p, c_float_p, c_size, C.c_int64, C.POINTER(c_size)]),
    "spissa_argmax_device": (C.c_int, [c_void_p, c_void_p, c_size, C.c_int64, c_void_p]),
    "spissa_lm_head_device": (C.c_int, [c_void_p, c_void_p, c_void_p, C.c_int64, c_void_p, c_void_p]),
    "spissa_attention_sublayer_device": (
        C.c_int, [c_void_p, C.POINTER(AttentionLayerC), c_void_p, c_size, c_void_p, c_void_p]),
}

_lib = None


def load() -> C.CDLL:
    """Loads libspissa_hip.so; raises ImportError with the build command when absent."""
    global _lib
    if _lib is not None:
        return _lib
    path = Path(os.environ.get("SPISSA_HIP_LIB", LIB_PATH))
    if not path.exists():
        raise ImportError(
            f"{path} is missing: build the HIP extension first (python -m spissa_amd.build); "
            "spissa_amd has no CPU fallback")
    lib = C.CDLL(str(path), mode=C.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().spissa_last_error()
    return msg.decode() if msg else ""
