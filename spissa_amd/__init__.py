"""spissa_amd -- MI355X (gfx950) attention path of the Spissa runtime.

The package mirrors crates/spissa-runtime/src/rotary.rs, the ops the path
uses, the streaming linear projections either side of it and the LM head
with greedy sampling after it, over the C ABI
in include/spissa_hip.h (libspissa_hip.so). There is no
CPU fallback: every call runs the HIP kernels.
"""
from .errors import (ArgumentError, DeviceError, InvalidTensorDataError, ShapeError,  # noqa: F401
                     SpissaError)
from .linear import (LinearModel, LinearWeight, StreamingLinearConfig,  # noqa: F401
                     StreamingTileLinearConfig, linear, streaming_tile_linear_from_model)
from .ops import is_global_layer, rms_norm, scaled_dot_product_attention  # noqa: F401
from .sampling import (lm_head_logits_parallel, lm_head_logits_parallel_bf16,  # noqa: F401
                       sample_argmax, sample_argmax_excluding)
from .rotary import (KvAttentionConfig, KvCache, RotaryEmbeddingConfig,  # noqa: F401
                     apply_gemma_rotary_inplace, apply_gpt_neox_rotary_inplace,
                     apply_llama_rotary_inplace, gpt_neox_rotary_dim,
                     scaled_dot_product_attention_with_cache)

__version__ = "0.1.0"
