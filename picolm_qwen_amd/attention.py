"""Host-side mirror of the reference's attention block over the HIP backend.

The reference (rain1201/picolm_qwen) runs the block inline in
Model::forward(token, pos) (cpp/model.hpp:288, block :326-418) and
Model::forward_batch(tokens, start_pos) (cpp/model.hpp:462, block :507-593),
with the KV cache and RoPE tables in its RunState (cpp/model.hpp:158-174).
`PicoAttention` owns that state in HBM and exposes the block per layer with the
same argument meaning:

    forward(layer, pos, q, k, v)              decode at pos (append, attend 0..pos)
    forward_batch(layer, start_pos, q, k, v)  prompt rows start_pos.. (token-major)

q/k/v may be torch tensors on the GPU (device path, asynchronous on the
context stream) or host numpy arrays (copy in, run, copy out). Every call
goes through libpqa.so; a missing library raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from ._lib import check, lib

ROPE_NEOX_HALF = 0          # rope_qwen       cpp/tensor.hpp:201-283
ROPE_LLAMA_X86_BLOCK8 = 1   # rope_llama SSE2 cpp/tensor.hpp:290-346 (x86 reference)
ROPE_LLAMA_INTERLEAVED = 2  # rope_llama scalar cpp/tensor.hpp:347-368


def rope_table(rope_base: float, head_dim: int, max_seq_len: int):
    """RoPE table rows [max_seq_len][head_dim/2] as cpp/model.hpp:1008-1017 builds it."""
    half = head_dim // 2
    c = np.empty((max_seq_len, half), dtype=np.float32)
    s = np.empty((max_seq_len, half), dtype=np.float32)
    fp = C.POINTER(C.c_float)
    lib().pqa_rope_table(rope_base, head_dim, max_seq_len, c.ctypes.data_as(fp), s.ctypes.data_as(fp))
    return c, s


def _is_torch(x) -> bool:
    return type(x).__module__.startswith("torch")


def _dev_ptr(t, dtype_name: str, numel: int):
    """Device address of a tensor the library reads or writes numel elements
    of; anything else (another dtype, a strided view, another size, host
    memory) raises before the call, since a kernel would then access memory
    outside the tensor."""
    if not _is_torch(t):
        raise ValueError(f"expected a torch tensor on the GPU, got {type(t).__name__}")
    if str(t.dtype) != "torch." + dtype_name:
        raise ValueError(f"expected {dtype_name}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError("tensors must be contiguous")
    if t.numel() != numel:
        raise ValueError(f"expected {numel} elements, got {t.numel()}")
    if not t.is_cuda:
        raise ValueError("torch tensors must be on the GPU")
    return C.c_void_p(t.data_ptr())


def _host(x, numel: int):
    a = np.ascontiguousarray(x, dtype=np.float32)
    if a.size != numel:
        raise ValueError(f"expected {numel} elements, got {a.size}")
    return a


def _host_inout(x, numel: int):
    """A host array the library reads and updates in place (the residual stream)."""
    if not (isinstance(x, np.ndarray) and x.dtype == np.float32 and x.flags.c_contiguous and x.flags.writeable
            and x.size == numel):
        raise ValueError(f"x must be a writeable C-contiguous float32 array of {numel} elements")
    return x


def _host_out(out, numel: int):
    """A host output array the library may write numel floats into."""
    if out is None:
        return np.empty(numel, dtype=np.float32)
    if not (isinstance(out, np.ndarray) and out.dtype == np.float32 and out.flags.c_contiguous
            and out.flags.writeable and out.size == numel):
        raise ValueError(f"out must be a writeable C-contiguous float32 array of {numel} elements")
    return out


# GGUF block geometry (elements, bytes per block) of the weight types the
# projections take, as the reference's dequantize_row_* reads them
# (cpp/quant.hpp:33-63, :176-281).
_GGUF_BLOCK = {1: (1, 4), 2: (1, 2), 3: (32, 18), 9: (32, 34), 13: (256, 144), 15: (256, 210)}


def _gguf_row_bytes(wtype: int, n: int):
    """Bytes of one GGUF row of n elements, or None for a type the library
    rejects itself (PQA_ERR_UNSUPPORTED) or a width that is not whole blocks."""
    be_bb = _GGUF_BLOCK.get(int(wtype))
    if be_bb is None or n % be_bb[0]:
        return None
    return n // be_bb[0] * be_bb[1]


def _host_rows(a, rows: int, wtype: int, n: int, what: str):
    """A host weight array that holds at least rows GGUF rows of n elements
    (the library copies rows x row bytes from it)."""
    if a is None:
        return None
    a = np.ascontiguousarray(a)
    rb = _gguf_row_bytes(wtype, n)
    if rb is not None and a.nbytes < rows * rb:
        raise ValueError(f"{what}: {a.nbytes} bytes, need {rows} rows x {rb} bytes")
    return a


def _host_bias(b, rows: int, btype: int, what: str):
    if b is None or int(btype) == 0:
        return None
    b = np.ascontiguousarray(b)
    need = rows * (4 if int(btype) == 1 else 2)
    if int(btype) in (1, 2) and b.nbytes < need:
        raise ValueError(f"{what}: {b.nbytes} bytes, need {need}")
    return b


class PicoAttention:
    def __init__(self, n_layers: int, max_seq_len: int, n_heads: int, n_kv_heads: int, head_dim: int,
                 rope_style: int = ROPE_NEOX_HALF, rope_base: float = 10000.0, rope_cos=None, rope_sin=None):
        if rope_cos is None or rope_sin is None:
            rope_cos, rope_sin = rope_table(rope_base, head_dim, max_seq_len)
        rope_cos = np.ascontiguousarray(rope_cos, dtype=np.float32)
        rope_sin = np.ascontiguousarray(rope_sin, dtype=np.float32)
        if rope_cos.size != max_seq_len * (head_dim // 2) or rope_sin.size != rope_cos.size:
            raise ValueError("RoPE tables must be [max_seq_len][head_dim/2]")
        self.n_layers, self.max_seq_len = n_layers, max_seq_len
        self.n_heads, self.n_kv_heads, self.head_dim = n_heads, n_kv_heads, head_dim
        self.q_dim, self.kv_dim = n_heads * head_dim, n_kv_heads * head_dim
        self.rope_style = rope_style
        # per layer: the input width of the q/k/v weights and the row count of
        # attn_output (0 = not set), for the size checks of the device calls
        self._qkv_embd = [0] * n_layers
        self._out_rows = [0] * n_layers
        h = C.c_void_p()
        check(lib().pqa_create(C.byref(h), n_layers, max_seq_len, n_heads, n_kv_heads, head_dim, rope_style,
                               rope_cos.ctypes.data_as(C.c_void_p), rope_sin.ctypes.data_as(C.c_void_p)))
        self._h = h

    # -- lifecycle ---------------------------------------------------------
    @property
    def handle(self) -> C.c_void_p:
        if self._h is None:
            raise RuntimeError("context destroyed")
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            self._ext = None
            lib().pqa_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def stream(self) -> int:
        """The context's hipStream_t as an int (torch.cuda.ExternalStream(stream))."""
        return lib().pqa_stream(self.handle) or 0

    def sync(self) -> None:
        check(lib().pqa_sync(self.handle), self.handle)

    def _ext_stream(self, device):
        import torch
        s = getattr(self, "_ext", None)
        if s is None:
            s = torch.cuda.ExternalStream(self.stream, device=device)
            self._ext = s
        return s

    def _enter(self, device, tensors):
        # The context stream waits for torch's current stream, so the inputs are
        # ready. The tensors are NOT record_stream()ed on the context stream:
        # torch would record events on it when they are freed, possibly after
        # the context (and its stream) is destroyed. _leave() orders torch's
        # stream after the call instead, which also covers the allocator
        # reusing the blocks.
        import torch
        ext = self._ext_stream(device)
        ext.wait_stream(torch.cuda.current_stream(device))
        return ext

    def _leave(self, device, ext):
        import torch
        torch.cuda.current_stream(device).wait_stream(ext)

    def set_decode_split(self, rows_per_split: int) -> None:
        check(lib().pqa_set_decode_split(self.handle, rows_per_split), self.handle)

    def set_prefill_precision(self, split_q: bool) -> None:
        """True (the default): prefill scores from q as fp16 hi + lo; False: one
        fp16 q (faster; its score error grows with |q| |k|)."""
        check(lib().pqa_set_prefill_precision(self.handle, int(bool(split_q))), self.handle)

    def set_batch_projection(self, exact_kv: bool) -> None:
        """True (the default): the batched entry points compute K and V in the
        reference's summation order (bit-exact cache rows) and q on the split
        fp16 GEMM; False: all three on the split GEMM (faster; a K/V element can
        land one fp16 step off)."""
        check(lib().pqa_set_batch_projection(self.handle, int(bool(exact_kv))), self.handle)

    def set_token_projection(self, exact_q: bool) -> None:
        """False (the default): the one-token projections sum the q rows of
        F32, F16 and Q4_K in any order on a bandwidth-bound path (within the
        fp32 reordering bound; q only feeds scores); True: q in the
        reference's order too, bit-identical to matmul_bias. k and v keep the
        reference's order either way."""
        check(lib().pqa_set_token_projection(self.handle, int(bool(exact_q))), self.handle)

    def set_out_projection(self, exact: bool) -> None:
        """True (the default): the one-token attn_output projection in the
        reference's order (bit-identical x); False: its F32, F16 and Q4_K rows
        in any order on the bandwidth-bound path (within the fp32 reordering
        bound)."""
        check(lib().pqa_set_out_projection(self.handle, int(bool(exact))), self.handle)

    # -- the block ----------------------------------------------------------
    def set_qk_norm(self, layer: int, q_norm_w, k_norm_w) -> None:
        """Layer's attn_q_norm / attn_k_norm weights ([head_dim] each); None turns it off."""
        if q_norm_w is None and k_norm_w is None:
            check(lib().pqa_set_qk_norm(self.handle, layer, None, None), self.handle)
            return
        qw = _host(q_norm_w, self.head_dim)
        kw = _host(k_norm_w, self.head_dim)
        check(lib().pqa_set_qk_norm(self.handle, layer, qw.ctypes.data_as(C.c_void_p),
                                    kw.ctypes.data_as(C.c_void_p)), self.handle)

    def forward(self, layer: int, pos: int, q, k, v, out=None):
        """Decode block at `pos` (cpp/model.hpp:326-418); returns xb [n_heads*head_dim]."""
        if _is_torch(q):
            import torch
            if out is None:
                out = torch.empty(self.q_dim, dtype=torch.float32, device=q.device)
            ptrs = (_dev_ptr(q, "float32", self.q_dim), _dev_ptr(k, "float32", self.kv_dim),
                    _dev_ptr(v, "float32", self.kv_dim), _dev_ptr(out, "float32", self.q_dim))
            ext = self._enter(q.device, (q, k, v, out))
            check(lib().pqa_decode(self.handle, layer, pos, *ptrs), self.handle)
            self._leave(q.device, ext)
            return out
        qh, kh, vh = _host(q, self.q_dim), _host(k, self.kv_dim), _host(v, self.kv_dim)
        res = _host_out(out, self.q_dim)
        check(lib().pqa_decode_host(self.handle, layer, pos, qh.ctypes.data_as(C.c_void_p),
                                    kh.ctypes.data_as(C.c_void_p), vh.ctypes.data_as(C.c_void_p),
                                    res.ctypes.data_as(C.c_void_p)), self.handle)
        return res

    def forward_noalloc(self, layer: int, pos: int, q, k, v, out):
        """forward() on device tensors through pqa_decode_noalloc: split
        partials in the library's static per-GPU scratch, nothing allocated
        (out must be given). Calls that overlap on one GPU race."""
        ptrs = (_dev_ptr(q, "float32", self.q_dim), _dev_ptr(k, "float32", self.kv_dim),
                _dev_ptr(v, "float32", self.kv_dim), _dev_ptr(out, "float32", self.q_dim))
        ext = self._enter(q.device, (q, k, v, out))
        check(lib().pqa_decode_noalloc(self.handle, layer, pos, *ptrs), self.handle)
        self._leave(q.device, ext)
        return out

    def forward_batch(self, layer: int, start_pos: int, q, k, v, out=None):
        """Prompt rows start_pos..start_pos+n-1 (cpp/model.hpp:493-593); q [n][q_dim],
        k/v [n][kv_dim]; returns out [n][q_dim]."""
        n_tok = int(q.shape[0])
        if _is_torch(q):
            import torch
            if out is None:
                out = torch.empty((n_tok, self.q_dim), dtype=torch.float32, device=q.device)
            ptrs = (_dev_ptr(q, "float32", n_tok * self.q_dim), _dev_ptr(k, "float32", n_tok * self.kv_dim),
                    _dev_ptr(v, "float32", n_tok * self.kv_dim), _dev_ptr(out, "float32", n_tok * self.q_dim))
            ext = self._enter(q.device, (q, k, v, out))
            check(lib().pqa_prefill(self.handle, layer, start_pos, n_tok, *ptrs), self.handle)
            self._leave(q.device, ext)
            return out
        qh = _host(q, n_tok * self.q_dim)
        kh, vh = _host(k, n_tok * self.kv_dim), _host(v, n_tok * self.kv_dim)
        res = _host_out(out, n_tok * self.q_dim).reshape(n_tok, self.q_dim)
        check(lib().pqa_prefill_host(self.handle, layer, start_pos, n_tok, qh.ctypes.data_as(C.c_void_p),
                                     kh.ctypes.data_as(C.c_void_p), vh.ctypes.data_as(C.c_void_p),
                                     res.ctypes.data_as(C.c_void_p)), self.handle)
        return res

    # -- cache access ---------------------------------------------------------
    def kv_download(self, layer: int, pos0: int, n: int):
        """Rows [pos0, pos0+n) as uint16 [n][kv_dim] (state.key_cache/val_cache bytes)."""
        k = np.empty((n, self.kv_dim), dtype=np.uint16)
        v = np.empty((n, self.kv_dim), dtype=np.uint16)
        check(lib().pqa_kv_download(self.handle, layer, pos0, n, k.ctypes.data_as(C.c_void_p),
                                    v.ctypes.data_as(C.c_void_p)), self.handle)
        return k, v

    def kv_upload(self, layer: int, pos0: int, k_rows, v_rows) -> None:
        k = np.ascontiguousarray(k_rows, dtype=np.uint16)
        v = np.ascontiguousarray(v_rows, dtype=np.uint16)
        n = k.size // self.kv_dim
        if k.size != n * self.kv_dim or v.size != k.size:
            raise ValueError("rows must be [n][kv_dim] uint16")
        check(lib().pqa_kv_upload(self.handle, layer, pos0, n, k.ctypes.data_as(C.c_void_p),
                                  v.ctypes.data_as(C.c_void_p)), self.handle)

    def kv_cache_ptrs(self):
        kp, vp = C.c_void_p(), C.c_void_p()
        check(lib().pqa_kv_cache(self.handle, C.byref(kp), C.byref(vp)), self.handle)
        return kp.value, vp.value

    # -- Q/K/V projections (cpp/model.hpp:320-366) -----------------------------
    def set_qkv_weights(self, layer: int, n_embd: int, wq, wq_type: int, wk, wk_type: int, wv, wv_type: int,
                        bq=None, bq_type: int = 0, bk=None, bk_type: int = 0, bv=None, bv_type: int = 0) -> None:
        """attn_q/k/v GGUF rows (uint8 arrays, [rows][row bytes]) and optional F32/F16 biases."""
        ws = [_host_rows(w, r, t, n_embd, name) for w, r, t, name in
              ((wq, self.q_dim, wq_type, "wq"), (wk, self.kv_dim, wk_type, "wk"), (wv, self.kv_dim, wv_type, "wv"))]
        bs = [_host_bias(b, r, t, name) for b, r, t, name in
              ((bq, self.q_dim, bq_type, "bq"), (bk, self.kv_dim, bk_type, "bk"), (bv, self.kv_dim, bv_type, "bv"))]

        def ptr(a):
            return None if a is None else a.ctypes.data_as(C.c_void_p)
        self._check_layer(layer)
        self._qkv_embd[layer] = 0
        check(lib().pqa_set_qkv_weights(self.handle, layer, n_embd, ptr(ws[0]), wq_type, ptr(bs[0]), bq_type,
                                        ptr(ws[1]), wk_type, ptr(bs[1]), bk_type, ptr(ws[2]), wv_type, ptr(bs[2]),
                                        bv_type), self.handle)
        self._qkv_embd[layer] = int(n_embd)

    def _check_layer(self, layer: int) -> None:
        if not 0 <= layer < self.n_layers:
            raise ValueError(f"layer {layer} outside [0, {self.n_layers})")

    def _embd(self, layer: int) -> int:
        self._check_layer(layer)
        if not self._qkv_embd[layer]:
            raise ValueError(f"layer {layer} has no q/k/v weights")
        return self._qkv_embd[layer]

    def _outr(self, layer: int) -> int:
        self._check_layer(layer)
        if not self._out_rows[layer]:
            raise ValueError(f"layer {layer} has no attn_output weights")
        return self._out_rows[layer]

    @staticmethod
    def _tokens(xb, n_embd: int) -> int:
        """Token count of a [n_tok][n_embd] prompt input."""
        if xb.ndim != 2 or int(xb.shape[1]) != n_embd:
            raise ValueError(f"expected xb of shape [n_tok][{n_embd}], got {tuple(xb.shape)}")
        if int(xb.shape[0]) <= 0:
            raise ValueError("n_tok must be positive")
        return int(xb.shape[0])

    def qkv_project(self, layer: int, xb, q=None, k=None, v=None):
        """q, k, v = matmul_bias(xb) on the GPU (torch tensors on the device)."""
        import torch
        n = self._embd(layer)
        dev = xb.device
        q = torch.empty(self.q_dim, dtype=torch.float32, device=dev) if q is None else q
        k = torch.empty(self.kv_dim, dtype=torch.float32, device=dev) if k is None else k
        v = torch.empty(self.kv_dim, dtype=torch.float32, device=dev) if v is None else v
        ptrs = (_dev_ptr(xb, "float32", n), _dev_ptr(q, "float32", self.q_dim),
                _dev_ptr(k, "float32", self.kv_dim), _dev_ptr(v, "float32", self.kv_dim))
        ext = self._enter(dev, (xb, q, k, v))
        check(lib().pqa_qkv_project(self.handle, layer, *ptrs), self.handle)
        self._leave(dev, ext)
        return q, k, v

    def forward_x(self, layer: int, pos: int, xb, out=None):
        """The attention block from the normed input xb: projections, then decode at pos."""
        import torch
        n = self._embd(layer)
        dev = xb.device
        out = torch.empty(self.q_dim, dtype=torch.float32, device=dev) if out is None else out
        ptrs = (_dev_ptr(xb, "float32", n), _dev_ptr(out, "float32", self.q_dim))
        ext = self._enter(dev, (xb, out))
        check(lib().pqa_decode_x(self.handle, layer, pos, *ptrs), self.handle)
        self._leave(dev, ext)
        return out

    def set_out_weights(self, layer: int, n_embd: int, wo, wo_type: int, bo=None, bo_type: int = 0) -> None:
        """attn_output GGUF rows (uint8 [n_embd][row bytes of q_dim elements]) and an optional bias."""
        wo = _host_rows(wo, n_embd, wo_type, self.q_dim, "wo")
        b = _host_bias(bo, n_embd, bo_type, "bo")
        self._check_layer(layer)
        self._out_rows[layer] = 0
        check(lib().pqa_set_out_weights(self.handle, layer, n_embd, None if wo is None else wo.ctypes.data_as(C.c_void_p),
                                        wo_type, None if b is None else b.ctypes.data_as(C.c_void_p), bo_type),
              self.handle)
        self._out_rows[layer] = int(n_embd)

    def out_project(self, layer: int, attn, x):
        """x += Wo attn + bo (cpp/model.hpp:420-427); torch tensors on the device, x updated in place."""
        rows = self._outr(layer)
        ptrs = (_dev_ptr(attn, "float32", self.q_dim), _dev_ptr(x, "float32", rows))
        ext = self._enter(attn.device, (attn, x))
        check(lib().pqa_out_project(self.handle, layer, *ptrs), self.handle)
        self._leave(attn.device, ext)
        return x

    def attention_block(self, layer: int, pos: int, xb, x):
        """cpp/model.hpp:320-427 from the normed input xb: x += attn_output(attention(q, k, v)).
        torch tensors on the device (x updated in place), or numpy arrays (the host
        entry point; x updated in place)."""
        n, rows = self._embd(layer), self._outr(layer)
        if not _is_torch(xb):
            xh, hx = _host(xb, n), _host_inout(x, rows)
            check(lib().pqa_attention_block_host(self.handle, layer, pos, xh.ctypes.data_as(C.c_void_p),
                                                 hx.ctypes.data_as(C.c_void_p)), self.handle)
            return x
        ptrs = (_dev_ptr(xb, "float32", n), _dev_ptr(x, "float32", rows))
        ext = self._enter(xb.device, (xb, x))
        check(lib().pqa_attention_block(self.handle, layer, pos, *ptrs), self.handle)
        self._leave(xb.device, ext)
        return x

    def qkv_project_batch(self, layer: int, xb):
        """q, k, v [n_tok][...] of a prompt: one GEMM over exactly dequantized
        weights, split into fp16 hi + lo parts with fp32 accumulation (within
        (3 n_embd + 12) 2^-24 sum |w x| of the reference)."""
        import torch
        n = self._embd(layer)
        n_tok = self._tokens(xb, n)
        dev = xb.device
        q = torch.empty((n_tok, self.q_dim), dtype=torch.float32, device=dev)
        k = torch.empty((n_tok, self.kv_dim), dtype=torch.float32, device=dev)
        v = torch.empty((n_tok, self.kv_dim), dtype=torch.float32, device=dev)
        ptrs = (_dev_ptr(xb, "float32", n_tok * n), _dev_ptr(q, "float32", n_tok * self.q_dim),
                _dev_ptr(k, "float32", n_tok * self.kv_dim), _dev_ptr(v, "float32", n_tok * self.kv_dim))
        ext = self._enter(dev, (xb, q, k, v))
        check(lib().pqa_qkv_project_batch(self.handle, layer, n_tok, *ptrs), self.handle)
        self._leave(dev, ext)
        return q, k, v

    def forward_batch_x(self, layer: int, start_pos: int, xb, out=None):
        """The prompt path of a layer from the normed inputs xb [n_tok][n_embd]."""
        import torch
        n = self._embd(layer)
        n_tok = self._tokens(xb, n)
        out = torch.empty((n_tok, self.q_dim), dtype=torch.float32, device=xb.device) if out is None else out
        ptrs = (_dev_ptr(xb, "float32", n_tok * n), _dev_ptr(out, "float32", n_tok * self.q_dim))
        ext = self._enter(xb.device, (xb, out))
        check(lib().pqa_prefill_x(self.handle, layer, start_pos, n_tok, *ptrs), self.handle)
        self._leave(xb.device, ext)
        return out

    def out_project_batch(self, layer: int, attn, x):
        """x[t] += Wo attn[t] + bo for a whole prompt (cpp/model.hpp:595-600), on the
        split fp16 GEMM (within (3 q_dim + 12) 2^-24 sum |w a|); torch tensors on the
        device, x [n_tok][n_embd] updated in place."""
        rows = self._outr(layer)
        n_tok = self._tokens(attn, self.q_dim)
        ptrs = (_dev_ptr(attn, "float32", n_tok * self.q_dim), _dev_ptr(x, "float32", n_tok * rows))
        ext = self._enter(attn.device, (attn, x))
        check(lib().pqa_out_project_batch(self.handle, layer, n_tok, *ptrs), self.handle)
        self._leave(attn.device, ext)
        return x

    def prefill_block(self, layer: int, start_pos: int, xb, x):
        """The attention half of a forward_batch layer (cpp/model.hpp:493-600 without
        the FFN): xb [n_tok][n_embd] (the attention norm's output) to the residual
        stream x [n_tok][n_embd], updated in place. torch tensors on the device, or
        numpy arrays (the host entry point)."""
        n, rows = self._embd(layer), self._outr(layer)
        n_tok = self._tokens(xb, n)
        if not _is_torch(xb):
            xh, hx = _host(xb, n_tok * n), _host_inout(x, n_tok * rows)
            check(lib().pqa_prefill_block_host(self.handle, layer, start_pos, n_tok, xh.ctypes.data_as(C.c_void_p),
                                               hx.ctypes.data_as(C.c_void_p)), self.handle)
            return x
        ptrs = (_dev_ptr(xb, "float32", n_tok * n), _dev_ptr(x, "float32", n_tok * rows))
        ext = self._enter(xb.device, (xb, x))
        check(lib().pqa_prefill_block(self.handle, layer, start_pos, n_tok, *ptrs), self.handle)
        self._leave(xb.device, ext)
        return x

    # -- .kvc persistence (picolm/model.c:870-983) ---------------------------
    def kvc_save(self, path: str, n_pos: int) -> None:
        """kvcache_save: rows [0, n_pos) of every layer to `path`; raises PQAError."""
        check(lib().pqa_kvc_save(self.handle, os.fsencode(path), n_pos), self.handle)

    def kvc_load(self, path: str) -> int:
        """kvcache_load: the file's position count, 0 on failure (reason in last_error())."""
        return lib().pqa_kvc_load(self.handle, os.fsencode(path))

    def last_error(self) -> str:
        msg = lib().pqa_last_error(self.handle)
        return msg.decode() if msg else ""

    def synth_kv(self, layer: int, pos0: int, n: int, seed: int, outlier_prob: float = 0.0) -> None:
        """Seeded synthetic history rows (same generator as the CPU oracle)."""
        check(lib().pqa_synth_kv(self.handle, layer, pos0, n, seed, outlier_prob), self.handle)

    def fp32_to_fp16(self, src, dst) -> None:
        """Device fp32 -> fp16 with the reference rounding (torch tensors on the GPU)."""
        n = src.numel()
        ptrs = (_dev_ptr(src, "float32", n), _dev_ptr(dst, "int16", n))
        ext = self._enter(src.device, (src, dst))
        check(lib().pqa_fp32_to_fp16(self.handle, *ptrs, n), self.handle)
        self._leave(src.device, ext)
