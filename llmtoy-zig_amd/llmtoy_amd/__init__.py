"""MI355X (gfx950) decode hot path of llmtoy-zig: GGUF block-quantised matvec
and the MoE layer, behind the C ABI in include/llmtoy_hip.h."""
from . import ggml, gguf, synth  # noqa: F401
from .lib import (ACT_GELU_TANH, ACT_SILU, Context, LtError, Tensor, UnsupportedError,  # noqa: F401
                  load_library, upload_moe)
