"""ctypes binding of libpqa.so (include/pqa.h). Loading fails loudly: there is
no CPU fallback for any entry point."""
from __future__ import annotations

import ctypes as C
import os

from ._build import LIB, STAMPS_LIB, STEP_STAMPS_LIB

PQA_OK = 0
PQA_ERR_ARG = -1
PQA_ERR_RANGE = -2
PQA_ERR_UNSUPPORTED = -3
PQA_ERR_HIP = -4
PQA_ERR_NOMEM = -5
PQA_ERR_IO = -6
PQA_ERR_FORMAT = -7

GGUF_NONE, GGUF_F32, GGUF_F16, GGUF_Q4_0, GGUF_Q8_0, GGUF_Q4_K, GGUF_Q6_K = 0, 1, 2, 3, 9, 13, 15

EXPORTS = [
    "pqa_create", "pqa_set_qk_norm", "pqa_decode", "pqa_prefill", "pqa_decode_host",
    "pqa_prefill_host", "pqa_kv_upload", "pqa_kv_download", "pqa_kv_cache", "pqa_stream",
    "pqa_sync", "pqa_last_error", "pqa_destroy", "pqa_rope_table", "pqa_fp32_to_fp16",
    "pqa_synth_kv", "pqa_set_decode_split", "pqa_set_prefill_precision", "pqa_set_batch_projection", "pqa_set_token_projection", "pqa_set_out_projection", "pqa_kvc_save", "pqa_kvc_load",
    "pqa_set_qkv_weights", "pqa_qkv_project", "pqa_decode_x", "pqa_set_out_weights", "pqa_out_project",
    "pqa_attention_block", "pqa_qkv_project_batch", "pqa_prefill_x", "pqa_decode_noalloc",
    "pqa_out_project_batch", "pqa_prefill_block", "pqa_attention_block_host", "pqa_prefill_block_host",
]


class PQAError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"pqa error {code}: {msg}")
        self.code = code


_lib = None
_stamped = None
_step_stamped = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is not built; run __graft_entry__.build() (hipcc, gfx950)")
        _lib = _bind(C.CDLL(LIB))
    return _lib


def stamped_lib(step: bool = False) -> C.CDLL:
    """The phase-stamped build of the same sources (measurement only: its
    kernels also write s_memrealtime stamps; pqa_decode_stamps_read /
    pqa_prefill_stamps_read return them, the _clear calls zero them). With
    step: the build that also stamps each step of the prefill tile loop
    (pqa_prefill_step_stamps_read)."""
    global _stamped, _step_stamped
    if (_step_stamped if step else _stamped) is None:
        path = STEP_STAMPS_LIB if step else STAMPS_LIB
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built; run python -m picolm_qwen_amd._build --stamps")
        L = _bind(C.CDLL(path))
        L.pqa_decode_stamps_read.argtypes = [C.c_void_p, C.c_int]
        L.pqa_decode_stamps_read.restype = C.c_int
        L.pqa_decode_stamps_clear.argtypes = []
        L.pqa_decode_stamps_clear.restype = C.c_int
        L.pqa_prefill_stamps_read.argtypes = [C.c_void_p, C.c_int]
        L.pqa_prefill_stamps_read.restype = C.c_int
        L.pqa_prefill_stamps_clear.argtypes = []
        L.pqa_prefill_stamps_clear.restype = C.c_int
        L.pqa_prefill_step_stamps_read.argtypes = [C.c_void_p, C.c_int]
        L.pqa_prefill_step_stamps_read.restype = C.c_int
        if step:
            _step_stamped = L
        else:
            _stamped = L
    return _step_stamped if step else _stamped


def _bind(L: C.CDLL) -> C.CDLL:
    vp, i, f, u64, sz = C.c_void_p, C.c_int, C.c_float, C.c_uint64, C.c_size_t
    fp = C.POINTER(C.c_float)
    L.pqa_create.argtypes = [C.POINTER(vp), i, i, i, i, i, i, vp, vp]
    L.pqa_set_qk_norm.argtypes = [vp, i, vp, vp]
    L.pqa_decode.argtypes = [vp, i, i, vp, vp, vp, vp]
    L.pqa_decode_noalloc.argtypes = [vp, i, i, vp, vp, vp, vp]
    L.pqa_prefill.argtypes = [vp, i, i, i, vp, vp, vp, vp]
    L.pqa_decode_host.argtypes = [vp, i, i, vp, vp, vp, vp]
    L.pqa_prefill_host.argtypes = [vp, i, i, i, vp, vp, vp, vp]
    L.pqa_kv_upload.argtypes = [vp, i, i, i, vp, vp]
    L.pqa_kv_download.argtypes = [vp, i, i, i, vp, vp]
    L.pqa_kv_cache.argtypes = [vp, C.POINTER(vp), C.POINTER(vp)]
    L.pqa_stream.argtypes = [vp]
    L.pqa_stream.restype = vp
    L.pqa_sync.argtypes = [vp]
    L.pqa_last_error.argtypes = [vp]
    L.pqa_last_error.restype = C.c_char_p
    L.pqa_destroy.argtypes = [vp]
    L.pqa_destroy.restype = None
    L.pqa_rope_table.argtypes = [f, i, i, fp, fp]
    L.pqa_rope_table.restype = None
    L.pqa_fp32_to_fp16.argtypes = [vp, vp, vp, sz]
    L.pqa_synth_kv.argtypes = [vp, i, i, i, u64, f]
    L.pqa_set_decode_split.argtypes = [vp, i]
    L.pqa_set_prefill_precision.argtypes = [vp, i]
    L.pqa_set_batch_projection.argtypes = [vp, i]
    L.pqa_set_token_projection.argtypes = [vp, i]
    L.pqa_set_out_projection.argtypes = [vp, i]
    L.pqa_kvc_save.argtypes = [vp, C.c_char_p, i]
    L.pqa_kvc_load.argtypes = [vp, C.c_char_p]
    L.pqa_set_qkv_weights.argtypes = [vp, i, i] + [vp, i, vp, i] * 3
    L.pqa_qkv_project.argtypes = [vp, i, vp, vp, vp, vp]
    L.pqa_decode_x.argtypes = [vp, i, i, vp, vp]
    L.pqa_set_out_weights.argtypes = [vp, i, i, vp, i, vp, i]
    L.pqa_out_project.argtypes = [vp, i, vp, vp]
    L.pqa_attention_block.argtypes = [vp, i, i, vp, vp]
    L.pqa_qkv_project_batch.argtypes = [vp, i, i, vp, vp, vp, vp]
    L.pqa_prefill_x.argtypes = [vp, i, i, i, vp, vp]
    L.pqa_out_project_batch.argtypes = [vp, i, i, vp, vp]
    L.pqa_prefill_block.argtypes = [vp, i, i, i, vp, vp]
    L.pqa_attention_block_host.argtypes = [vp, i, i, vp, vp]
    L.pqa_prefill_block_host.argtypes = [vp, i, i, i, vp, vp]
    for name in EXPORTS:
        if name not in ("pqa_stream", "pqa_last_error", "pqa_destroy", "pqa_rope_table"):
            getattr(L, name).restype = C.c_int
    return L


def check(rc: int, ctx=None) -> None:
    if rc != PQA_OK:
        msg = lib().pqa_last_error(ctx)
        raise PQAError(rc, msg.decode() if msg else "")
