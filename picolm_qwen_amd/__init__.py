"""MI355X (gfx950) backend for the attention path of rain1201/picolm_qwen's
C++ forward pass: QK-RMSNorm, RoPE, fp16 KV append and GQA attention over an
HBM-resident KV cache, behind the C ABI in include/pqa.h (libpqa.so)."""
from .attention import (ROPE_LLAMA_INTERLEAVED, ROPE_LLAMA_X86_BLOCK8, ROPE_NEOX_HALF, PicoAttention,
                        rope_table)
from ._lib import EXPORTS, PQAError

__all__ = ["PicoAttention", "rope_table", "PQAError", "EXPORTS", "ROPE_NEOX_HALF", "ROPE_LLAMA_X86_BLOCK8",
           "ROPE_LLAMA_INTERLEAVED"]
